"""The expert-cache profile reader (include/naiwa_policy.h, naiwa_profile_*),
on the cases of the reference's own tests (src/moe/profile.rs:114-158): the
ranking split per layer in rank order, pairs outside the model dropped and
repeats kept once, and files it cannot read rejected with the reason."""
import struct

import pytest

import naiwa_moe as nm
from naiwa_moe.policy import ExpertProfile, hit_rate, write_profile


def strp(pairs, layers, experts, version=1):
    """The reference test's writer: header (slots = n) and the ranking, no rank table."""
    b = b"STRP" + struct.pack("<5I", version, layers, experts, len(pairs), len(pairs))
    return b + b"".join(struct.pack("<HH", l, e) for l, e in pairs)


def test_reads_the_ranking_per_layer_in_rank_order(tmp_path):
    p = tmp_path / "order.bin"
    p.write_bytes(strp([(1, 5), (0, 9), (1, 2), (0, 7)], 2, 16))
    prof = ExpertProfile(p, 2, 16)
    assert prof.layer(0) == [9, 7] and prof.layer(1) == [5, 2] and prof.pairs == 4
    assert prof.layer(1) == [5, 2]
    assert prof.layer(2) == [] and prof.layer(-1) == []
    assert prof.source.endswith("(2x16, 4 ranked pairs)")


def test_drops_pairs_outside_the_model(tmp_path):
    p = tmp_path / "filter.bin"
    p.write_bytes(strp([(0, 3), (0, 300), (0, 3), (9, 1)], 2, 256))
    prof = ExpertProfile(p, 2, 256)
    assert prof.layer(0) == [3] and prof.layer(1) == [] and prof.pairs == 1


def _rc(path, layers=2, experts=16):
    try:
        ExpertProfile(path, layers, experts)
        return 0
    except nm.NaiwaError as e:
        return e.rc


def test_rejects_what_it_cannot_read(tmp_path):
    p = tmp_path / "bad.bin"
    p.write_bytes(b"NOPE")
    assert _rc(p) == nm.E_FORMAT
    p.write_bytes(strp([(0, 1)], 2, 16)[:26])  # the header says 1 pair, no room for it
    assert _rc(p) == nm.E_FORMAT
    p.write_bytes(strp([(0, 1)], 2, 16)[:20])  # shorter than the header
    assert _rc(p) == nm.E_FORMAT
    p.write_bytes(strp([(0, 1)], 2, 16, version=2))
    assert _rc(p) == nm.E_UNSUPPORTED
    assert _rc(tmp_path / "missing.bin") == nm.E_IO
    p.write_bytes(strp([], 2, 16))  # an empty ranking reads as empty
    prof = ExpertProfile(p, 2, 16)
    assert prof.pairs == 0 and prof.layer(0) == []


def test_written_profile_reads_back_and_the_rank_table_is_ignored(tmp_path):
    pairs = [(l, e) for e in (7, 3, 11, 0) for l in (2, 0, 1)] + [(0, 3)]
    p = tmp_path / "w.bin"
    write_profile(p, pairs, 3, 16, slots=12)
    data = p.read_bytes()
    assert data[:4] == b"STRP" and len(data) == 24 + 4 * len(pairs) + 4 * 3 * 16
    assert struct.unpack_from("<5I", data, 4) == (1, 3, 16, 12, len(pairs))
    prof = ExpertProfile(p, 3, 16)
    assert [prof.layer(l) for l in range(3)] == [[7, 3, 11, 0]] * 3 and prof.pairs == 12
    # bounded by the model the reader is given
    small = ExpertProfile(p, 2, 8)
    assert small.layer(0) == [7, 3, 0] and small.layer(2) == [] and small.pairs == 6


def test_hit_rate():
    assert hit_rate({"hits": 3, "misses": 1}) == 0.75 and hit_rate({"hits": 0, "misses": 0}) == 0.0
