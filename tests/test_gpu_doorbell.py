"""Doorbell kernels on the device, through the reference-named C ABI
(src/doorbell/mod.rs:31-69): the round trips of src/doorbell/tests.rs:316-413
and must-fail arms (a wait whose target never arrives must time out, not hang,
and must copy nothing)."""
import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


class Mapped:
    """A zeroed fine-grained mapped allocation with its host and device views."""

    def __init__(self, nm, nbytes):
        self.L = nm.lib()
        p = C.c_void_p()
        assert self.L.doorbell_alloc_mapped(C.byref(p), nbytes) == 0
        self.host = p.value
        d = C.c_void_p()
        self.L.doorbell_get_device_ptr(self.host, C.byref(d))
        assert d.value
        self.dev = d.value
        self.nbytes = nbytes

    def view(self, dtype, offset=0, count=None):
        dtype = np.dtype(dtype)
        if count is None:
            count = (self.nbytes - offset) // dtype.itemsize
        buf = (C.c_uint8 * (count * dtype.itemsize)).from_address(self.host + offset)
        return np.frombuffer(buf, dtype=dtype)

    def free(self):
        self.L.doorbell_free_host(self.host)


def test_topk_doorbell_round_trips_ids_and_weights(gpu):
    nm = gpu
    L = nm.lib()
    max_n = 8
    m = Mapped(nm, 8 + max_n * 8)  # [seq][pad][ids][weights]
    ids = nm.DeviceBuffer.from_array(np.array([3, 7, 1, 5], np.uint32))
    ws = nm.DeviceBuffer.from_array(np.array([0.5, 0.25, 0.125, 0.0625], np.float32))
    seq0 = L.naiwa_host_load_acquire_u32(m.host)
    L.doorbell_ring(m.dev, m.dev + 8, m.dev + 8 + max_n * 4, ids.ptr, ws.ptr, 4, 0)
    assert L.naiwa_host_wait_ge(m.host, seq0 + 1, 5_000_000, 50) == 0
    assert m.view(np.uint32, 8, 4).tolist() == [3, 7, 1, 5]
    assert m.view(np.float32, 8 + max_n * 4, 4).tolist() == [0.5, 0.25, 0.125, 0.0625]
    nm.synchronize()
    m.free()


def test_activation_doorbell_uses_seq_to_pick_the_ring_slot(gpu):
    nm = gpu
    L = nm.lib()
    depth, max_n = 8, 4
    m = Mapped(nm, 8 + depth * max_n * 4)
    for seq in range(3):
        values = np.array([seq * 10.0 + i for i in range(4)], np.float32)
        src = nm.DeviceBuffer.from_array(values)
        slot_off = 8 + (seq % depth) * max_n * 4
        L.doorbell_copy_f32(m.dev, m.dev + slot_off, src.ptr, 4, 0)
        assert L.naiwa_host_wait_ge(m.host, seq + 1, 5_000_000, 50) == 0
        assert np.array_equal(m.view(np.float32, slot_off, 4), values)
    nm.synchronize()
    m.free()


def test_result_doorbell_copies_host_payload_to_the_device(gpu):
    nm = gpu
    L = nm.lib()
    depth, max_n = 8, 4
    m = Mapped(nm, 8 + depth * max_n * 4)  # [seq][consumed][ring]
    values = np.array([1.0, 2.0, 3.0, 4.0], np.float32)
    seq = 1
    slot = m.view(np.float32, 8 + (seq % depth) * max_n * 4, 4)
    slot[:] = values
    L.naiwa_host_store_release_u32(m.host, seq)
    dst = nm.DeviceBuffer(16)
    dst.zero()
    L.doorbell_wait_copy_f32(m.dev, seq, m.dev + 8 + (seq % depth) * max_n * 4, 0, m.dev + 4,
                             dst.ptr, 4, 0)
    nm.synchronize()
    assert np.array_equal(dst.download(np.float32), values)
    assert L.naiwa_host_load_acquire_u32(m.host + 4) >= 1
    m.free()


def test_device_wait_released_by_a_later_host_publish(gpu):
    """The copy kernel is queued before the host writes: it must spin until the
    seq bump, then copy what the host wrote (not the zeroes it saw first)."""
    nm = gpu
    L = nm.lib()
    m = Mapped(nm, 8 + 64 * 4)
    dst = nm.DeviceBuffer(64 * 4)
    dst.zero()
    s = nm.Stream()
    L.doorbell_wait_copy_f32(m.dev, 1, m.dev + 8, 0, m.dev + 4, dst.ptr, 64, s.handle)
    import time
    time.sleep(0.05)
    values = np.arange(64, dtype=np.float32) + 0.5
    m.view(np.float32, 8, 64)[:] = values
    L.naiwa_host_store_release_u32(m.host, 1)
    s.sync()
    assert np.array_equal(dst.download(np.float32), values)
    assert L.naiwa_host_load_acquire_u32(m.host + 4) == 1
    m.free()


def test_wait_on_a_never_published_seq_times_out(gpu):
    """Must-fail arm: a target the host never publishes ends the kernel by its
    wall-clock bound, copies nothing and counts a timeout."""
    nm = gpu
    L = nm.lib()
    m = Mapped(nm, 8 + 16)
    dst = nm.DeviceBuffer(16)
    dst.upload(np.full(4, -7.0, np.float32))
    m.view(np.float32, 8, 4)[:] = 9.0
    before = C.c_uint32(0)
    assert L.naiwa_doorbell_timeouts(C.byref(before)) == 0
    assert L.naiwa_doorbell_set_wait_limit_us(20_000) == 0
    try:
        L.doorbell_wait_copy_f32(m.dev, 5, m.dev + 8, 0, m.dev + 4, dst.ptr, 4, 0)
        nm.synchronize()
    finally:
        L.naiwa_doorbell_set_wait_limit_us(0)
    after = C.c_uint32(0)
    assert L.naiwa_doorbell_timeouts(C.byref(after)) == 0
    assert after.value == before.value + 1
    assert np.array_equal(dst.download(np.float32), np.full(4, -7.0, np.float32))
    assert L.naiwa_host_load_acquire_u32(m.host + 4) == 0  # consumed not published
    m.free()


def test_stale_seq_is_not_accepted(gpu):
    """Must-fail arm: a counter below the target (a previous lap) does not release the wait."""
    nm = gpu
    L = nm.lib()
    m = Mapped(nm, 8 + 16)
    L.naiwa_host_store_release_u32(m.host, 3)
    dst = nm.DeviceBuffer(16)
    dst.upload(np.zeros(4, np.float32))
    m.view(np.float32, 8, 4)[:] = 1.0
    L.naiwa_doorbell_set_wait_limit_us(20_000)
    try:
        L.doorbell_wait_copy_f32(m.dev, 4, m.dev + 8, 0, m.dev + 4, dst.ptr, 4, 0)
        nm.synchronize()
    finally:
        L.naiwa_doorbell_set_wait_limit_us(0)
    assert not dst.download(np.float32).any()
    m.free()


# ---- the persistent-wave doorbell (doorbell_poll_serve / _wait / _signal) -----------------

def _timeouts(L):
    n = C.c_uint32(0)
    assert L.naiwa_doorbell_timeouts(C.byref(n)) == 0
    return n.value


def test_poll_serve_answers_every_host_ring(gpu):
    """One wave serves 200 host rings in a row: the host raises seq to i, the wave
    release-stores i to ack, and the host sees it before ringing again -- the
    round trip the reference's harness times with a stream sync per ring
    (docs/worklogs/m0.md:43).  No wait runs out."""
    nm = gpu
    L = nm.lib()
    m = Mapped(nm, 256)              # seq at 0, ack at 128 (own cache lines)
    s = nm.Stream()
    before = _timeouts(L)
    L.naiwa_doorbell_set_wait_limit_us(2_000_000)
    try:
        assert L.doorbell_poll_serve(m.dev, m.dev + 128, 1, 200, s.handle) == 0
        for i in range(1, 201):
            L.naiwa_host_store_release_u32(m.host, i)
            assert L.naiwa_host_wait_ge(m.host + 128, i, 2_000_000, 0) == 0, i
        s.sync()
    finally:
        L.naiwa_doorbell_set_wait_limit_us(0)
    assert L.naiwa_host_load_acquire_u32(m.host + 128) == 200
    assert _timeouts(L) == before
    m.free()


def test_poll_signal_then_wait_orders_two_streams(gpu):
    """doorbell_poll_signal on stream A after A's work, doorbell_poll_wait on stream B
    before B's reader: B's copy sees what A wrote last, every epoch, although A starts
    with a long copy and the host never synchronises between them."""
    nm = gpu
    L = nm.lib()
    a, b = nm.Stream(), nm.Stream()
    flag = nm.DeviceBuffer(256)
    big_src, big_dst = nm.DeviceBuffer(64 << 20), nm.DeviceBuffer(64 << 20)
    marker, seen = nm.DeviceBuffer(256), nm.DeviceBuffer(256 * 8)
    assert L.naiwa_memset(flag.ptr, 0, 256, 0) == 0
    assert L.naiwa_memset(seen.ptr, 0, 256 * 8, 0) == 0
    nm.synchronize()
    before = _timeouts(L)
    for epoch in range(1, 9):
        assert L.naiwa_memcpy_d2d(big_dst.ptr, big_src.ptr, 64 << 20, a.handle) == 0   # A is busy
        assert L.naiwa_memset(marker.ptr, 0x10 + epoch, 4, a.handle) == 0             # A's last write
        assert L.doorbell_poll_signal(flag.ptr, epoch, a.handle) == 0
        assert L.doorbell_poll_wait(flag.ptr, epoch, b.handle) == 0
        assert L.naiwa_memcpy_d2d(seen.ptr + 256 * (epoch - 1), marker.ptr, 4, b.handle) == 0
    a.sync()
    b.sync()
    got = seen.download(np.uint8).reshape(8, 256)[:, :4]
    for epoch in range(1, 9):
        assert (got[epoch - 1] == 0x10 + epoch).all(), (epoch, got[epoch - 1])
    assert _timeouts(L) == before


def test_poll_wait_that_is_never_signalled_gives_up_on_its_bound(gpu):
    """Must-fail arm: a flag nobody raises ends doorbell_poll_wait by its wall-clock
    bound (here 2 ms), counts one timeout, and the stream goes on.  The persistent
    server given a ring that never comes does the same."""
    nm = gpu
    L = nm.lib()
    flag = nm.DeviceBuffer(256)
    assert L.naiwa_memset(flag.ptr, 0, 256, 0) == 0
    m = Mapped(nm, 256)
    nm.synchronize()
    before = _timeouts(L)
    L.naiwa_doorbell_set_wait_limit_us(2_000)
    try:
        assert L.doorbell_poll_wait(flag.ptr, 1, 0) == 0
        assert L.doorbell_poll_serve(m.dev, m.dev + 128, 1, 1, 0) == 0
        nm.synchronize()
    finally:
        L.naiwa_doorbell_set_wait_limit_us(0)
    assert _timeouts(L) == before + 2
    assert L.naiwa_host_load_acquire_u32(m.host + 128) == 0   # no ack for a ring never rung
    m.free()
