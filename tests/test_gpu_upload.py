"""GPU tests of the batched host -> device upload (naiwa_copy_batch): the bytes of
every range land exactly, an unmapped or misaligned source is refused before
anything is queued, and the staged uploads of a cached layer use it."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def test_copy_batch_copies_every_range(gpu):
    nm = gpu
    rng = np.random.default_rng(7)
    # a Q4_K projection of the Qwen3 expert shape, a Q8_0 one, small and empty ranges
    sizes = [884736, 2 * 1408 * 2176, 16, 4096 + 16, 0, 1 << 20]
    host = nm.PinnedBuffer(sum(sizes) + 64)
    hv = host.view()
    hv[:] = rng.integers(0, 256, hv.size, dtype=np.uint8)
    devs = [nm.DeviceBuffer(max(s, 16)) for s in sizes]
    items, off = [], 16
    for d, s in zip(devs, sizes):
        items.append((d.ptr, host.ptr + off, s))
        off += s
    print(f"[copy_batch ranges={len(items)} bytes={sum(sizes)}]", flush=True)
    stream = nm.Stream()
    assert nm.copy_batch(items, stream.handle)
    stream.sync()
    off = 16
    for d, s in zip(devs, sizes):
        if s:
            assert np.array_equal(d.download(np.uint8, s), hv[off:off + s]), s
        off += s


def test_copy_batch_refuses_unmapped_or_misaligned(gpu):
    nm = gpu
    d = nm.DeviceBuffer(4096)
    d.zero()
    pageable = np.arange(4096, dtype=np.uint8)
    host = nm.PinnedBuffer(8192)
    host.view()[:] = 7
    # pageable memory is not mapped for the device: refused, nothing queued
    assert not nm.copy_batch([(d.ptr, pageable.ctypes.data, 4096)])
    # misaligned source or size
    assert not nm.copy_batch([(d.ptr, host.ptr + 8, 4096)])
    assert not nm.copy_batch([(d.ptr, host.ptr, 4008)])
    nm.synchronize()
    assert not d.download(np.uint8).any()
    with pytest.raises(ValueError):
        nm.copy_batch([(d.ptr, host.ptr, 16)] * 65)
