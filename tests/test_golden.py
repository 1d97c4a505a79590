"""The committed golden vectors (tests/golden/golden_small.npz) against the
CPU oracle: every array is recomputed and must match bit for bit, so any change
to the oracle or to the seeded input generators fails here. The reference's
literal known answers inside the fixture are also checked as literals."""
import os
import sys

import numpy as np
import pytest

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
sys.path.insert(0, GOLDEN)

import make_golden  # noqa: E402


@pytest.fixture(scope="module")
def stored():
    with np.load(make_golden.OUT, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


@pytest.fixture(scope="module")
def fresh():
    return make_golden.cases()


def test_fixture_covers_every_case(stored, fresh):
    assert sorted(stored) == sorted(fresh)


def test_oracle_reproduces_every_vector(stored, fresh):
    bad = [k for k in fresh
           if fresh[k].dtype != stored[k].dtype or fresh[k].shape != stored[k].shape
           or fresh[k].tobytes() != stored[k].tobytes()]
    assert not bad, f"oracle output changed for {bad}"


def test_literal_known_answers(stored):
    # src/int8.rs:416-422
    assert stored["igemm_kat.c"].tolist() == [[-4, 7]]
    # src/ternary.rs:427-446: round trips; codes 01 = +1, 10 = -1, 00 = 0, element i at bits 2i
    t = stored["ternary_pack_kat.t"]
    word = int(stored["ternary_pack_kat.packed"][0])
    codes = [(word >> (2 * i)) & 3 for i in range(16)]
    assert codes == [{1: 1, -1: 2, 0: 0}[int(v)] for v in t]
    # src/quant.rs:291-310: 4-bit error below 0.15 x the value range
    x, y = stored["rq_ref.x"], stored["rq_ref.y"]
    assert np.abs(y - x).max() < 0.15 * (x.max() - x.min())
    # src/ternary.rs:412-424: row [10, -10, 0.001, -0.001, ...] -> [+1, -1, 0, 0, ...]
    p = stored["ternary_rows.packed"]
    first = [(int(p[0]) >> (2 * i)) & 3 for i in range(4)]
    assert first == [1, 2, 0, 0]

    # src/quantize.rs:862-872: E2M1 points at scale 1 round-trip exactly
    assert stored["qt_nvfp4.NVFP4.deq"].tolist() == stored["qt_nvfp4.x"].tolist()
    # odd groups: each packed on its own, read through data[i/2] (src/quantize.rs:377-396)
    assert stored["qt_odd.INT4.data"].tolist() == [0x97, 0x01, 0x74, 0x0C]
    assert stored["qt_odd.INT4.deq"].tolist() == [7.0, -7.0, 1.0, 0.0, 4.0, 7.0]
