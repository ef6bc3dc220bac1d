"""The prefill stream's memory plan (include/naiwa_prefill.h) on the reference's
own known answers (src/prefill_stream.rs:1815-1911): the chunk's price is the
measured line, the chunk is as large as free memory allows, the second buffer
is taken only at the same chunk, borrowing pays only the scratch, and nothing
fitting turns the stream off."""
import os

import pytest

from naiwa_moe import prefill as P

MIB, GIB = 1 << 20, 1 << 30
LAYER = 650 * MIB

ENV = ("NAIWA_CHUNK_FIXED_MIB", "NAIWA_CHUNK_PER_ROW_KIB", "NAIWA_PREFILL_SLACK_MIB", "NAIWA_DECODE_RESERVE_MIB",
       "NAIWA_DEPTH_CAP")


@pytest.fixture(autouse=True)
def no_probe_overrides(monkeypatch):
    for name in ENV:
        monkeypatch.delenv(name, raising=False)


def test_the_chunk_line_is_the_two_points_that_were_measured():
    assert P.chunk_scratch(288) >> 20 == 131
    assert P.chunk_scratch(1216) >> 20 == 452
    assert P.chunk_scratch(1216) > P.activation_bytes(1216)
    assert P.chunk_scratch(1216) < 1346 * MIB


def test_plan_spends_memory_on_the_chunk_before_the_second_buffer():
    act = P.activation_bytes
    assert act(8192) - act(P.SUB_ROWS) == (8192 - P.SUB_ROWS) * (24 << 10)
    assert P.plan(12 * GIB, LAYER, 8192, False) == (2, 8192)
    assert P.plan(2049 * MIB, LAYER, 8192, True) == (1, 4864)
    assert P.plan_with_lend(2049 * MIB, LAYER, 8192, True, 0, 1536 * MIB) == (2, 4864)
    assert P.plan_with_lend(12 * GIB, LAYER, 8192, True, 0, 1300 * MIB - 1)[0] == 1
    assert P.plan_with_lend(2049 * MIB, LAYER, 8192, False, 0, 1536 * MIB)[0] == 1
    lent = P.plan(2049 * MIB, LAYER, 8192, True)[1]
    owned = P.plan(2049 * MIB, LAYER, 8192, False)[1]
    assert owned < lent
    assert P.chunk_scratch(lent) + P.CHUNK_HEAD <= 2049 * MIB
    assert P.plan(2049 * MIB, LAYER, 8192, False) == (1, 2304)
    assert P.plan(2400 * MIB, LAYER, 8192, False) == (1, 3328)
    assert P.plan(3034 * MIB, LAYER, 8192, False) == (1, 5120)
    assert P.plan(12 * GIB, LAYER, 512, False)[1] == 512
    assert P.plan(8 * GIB, LAYER, 8192, False) == (2, 8192)
    assert P.plan(LAYER, LAYER, 1024, False) is None


def test_depth_reserve_and_overrides(monkeypatch):
    # deeper buffers when the same chunk affords them, down to 1 (MAX_DEPTH caps the ask)
    assert P.plan_with_lend_depth(64 * GIB, LAYER, 8192, False, 0, 0, 4) == (4, 8192)
    assert P.plan_with_lend_depth(64 * GIB, LAYER, 8192, False, 0, 0, 9) == (4, 8192)
    assert P.plan_with_lend_depth(64 * GIB, LAYER, 8192, False, 0, 0, 1) == (1, 8192)
    # the KV reserve comes off the free bytes first
    assert P.plan_with_reserve(2049 * MIB + 384 * MIB, LAYER, 8192, False, 384 * MIB) == (1, 2304)
    # a 288 GB device: the ceiling and four buffers of a DeepSeek-V2-Lite layer (~406 MiB)
    assert P.plan_with_lend_depth(280 * GIB, 406 * MIB, 8192, False, 0, 0, 4) == (4, 8192)
    # the probes the reference reads
    monkeypatch.setenv("NAIWA_CHUNK_PER_ROW_KIB", "0")
    assert P.chunk_scratch(1216) == 32 * MIB
    monkeypatch.setenv("NAIWA_DEPTH_CAP", "4")
    assert P.plan_with_lend_depth(2049 * MIB, LAYER, 8192, True, 0, 3 * LAYER, 4)[0] == 3
