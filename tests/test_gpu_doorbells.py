"""Doorbell protocols on the device, as the reference tests them
(src/doorbell/tests.rs:8-105), plus the executor's result channel."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def test_topk_doorbell_round_trips_ids_and_weights(gpu):
    nm = gpu
    bell = nm.doorbells.TopkDoorbell(8)
    ids = nm.DeviceBuffer.from_array(np.array([3, 7, 1, 5], dtype=np.uint32))
    ws = nm.DeviceBuffer.from_array(np.array([0.5, 0.25, 0.125, 0.0625], dtype=np.float32))
    got_ids, got_ws = bell.publish_and_read(ids, ws, 4)
    assert got_ids.tolist() == [3, 7, 1, 5]
    assert got_ws.tolist() == [0.5, 0.25, 0.125, 0.0625]
    # a second publish on the same bell reads the new payload
    ids2 = nm.DeviceBuffer.from_array(np.array([9, 2], dtype=np.uint32))
    ws2 = nm.DeviceBuffer.from_array(np.array([0.75, 0.25], dtype=np.float32))
    got_ids, got_ws = bell.publish_and_read(ids2, ws2, 2)
    assert got_ids.tolist() == [9, 2] and got_ws.tolist() == [0.75, 0.25]


def test_activation_doorbell_uses_seq_to_pick_the_ring_slot(gpu):
    nm = gpu
    bell = nm.doorbells.ActivationDoorbell(4)
    for seq in range(3):
        values = np.array([seq * 10.0 + i for i in range(4)], dtype=np.float32)
        src = nm.DeviceBuffer.from_array(values)
        bell.publish(src, 4, seq)
        got = bell.wait_publish(seq, 4)
        assert got is not None and got.tolist() == values.tolist()


def test_result_doorbell_copies_host_payload_to_the_device(gpu):
    nm = gpu
    bell = nm.doorbells.ResultDoorbell(4)
    dst = nm.DeviceBuffer(16)
    dst.zero()
    values = [1.0, 2.0, 3.0, 4.0]
    assert bell.publish(values, 1), "an empty ring always takes the payload"
    bell.wait_copy(1, 4, dst)
    nm.synchronize()
    assert dst.download(np.float32).tolist() == values
    assert bell.consumed() >= 1


def test_result_doorbell_backpressure_waits_for_consumed_and_then_drops(gpu):
    nm = gpu
    bell = nm.doorbells.ResultDoorbell(4)
    depth = bell.depth
    values = [1.0, 2.0, 3.0, 4.0]
    for seq in range(1, depth + 1):
        assert bell.publish(values, seq), f"seq {seq} is inside the first lap"
    assert not bell.publish(values, depth + 1), "a full ring must refuse the payload"
    dst = nm.DeviceBuffer(16)
    bell.wait_copy(depth + 1, 4, dst)   # the seq bump still happened: the device does not hang
    nm.synchronize()
    assert bell.consumed() >= depth + 1
    assert bell.publish(values, depth + 2)


def test_pass_cell_hands_the_latest_claim_to_the_consumer(gpu):
    nm = gpu
    cs = nm.Stream()
    cell = nm.doorbells.PassCell()
    assert cell.wait_latest() is None, "no claim, no GPU work"
    assert cell.claim(cs.handle) == 1
    nm.synchronize()
    assert cell.wait_latest() == 1
    assert cell.claim(cs.handle) == 2
    assert cell.claimed() == 2
    nm.synchronize()
    assert cell.wait_latest() == 2


def test_executor_results_reach_the_device_in_order(gpu):
    nm = gpu
    ex = nm.doorbells.Executor()
    stream = nm.Stream()
    outs = []
    for j in range(12):   # more jobs than the ring depth: the stream consumes as they come
        p = ex.submit_result(6, lambda j=j: np.arange(6, dtype=np.float32) + 10 * j)
        dst = nm.DeviceBuffer(24)
        ex.upload(p, dst, stream.handle)
        outs.append(dst)
    stream.sync()
    for j, dst in enumerate(outs):
        assert dst.download(np.float32).tolist() == (np.arange(6) + 10 * j).tolist()
    assert ex.stalls() == 0 and ex.take_error() is None
    # a failing task publishes an empty payload (the stream still advances) and reports
    p = ex.submit_result(6, lambda: 1 / 0)
    dst = nm.DeviceBuffer(24)
    ex.upload(p, dst, stream.handle)
    stream.sync()
    ex.wait_idle()
    assert ex.take_error() is not None
    ex.close()
