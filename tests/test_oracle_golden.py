"""The oracle's number formats against the reference's golden vectors.

tests/golden/quant_q8_0_f16_bf16.tsv holds the Q8_0, F16 and BF16 rows of the reference's
tests/core/data/quant.tsv (gguf-py dequantized floats; consumed by Quant.DequantizeMatchesGgufPy,
tests/core/quant_test.cpp:255-268): type, block bytes (hex), expected float32 values (little-endian hex).
"""
from pathlib import Path

import numpy as np
import pytest

import oracle_py as O

GOLDEN = Path(__file__).resolve().parent / "golden" / "quant_q8_0_f16_bf16.tsv"


def rows():
    out = []
    for line in GOLDEN.read_text().splitlines():
        t, blk, vals = line.split("\t")
        out.append((t, np.frombuffer(bytes.fromhex(blk), np.uint8).copy(),
                    np.frombuffer(bytes.fromhex(vals), np.float32).copy()))
    return out


def test_fixture_counts():
    r = rows()
    assert [t for t, _, _ in r].count("Q8_0") == 12
    assert [t for t, _, _ in r].count("F16") == 12
    assert [t for t, _, _ in r].count("BF16") == 12


def _decode(t, blk):
    o = O.oracle()
    if t == "Q8_0":
        out = np.empty(32 * (len(blk) // 34), np.float32)
        o.or_dequant_q8_0(blk, out, out.size)
        return out
    halves = blk.view(np.uint16)
    f = o.or_fp16_to_f32 if t == "F16" else o.or_bf16_to_f32
    return np.array([f(int(h)) for h in halves], np.float32)


@pytest.mark.parametrize("i", range(36))
def test_golden_row_bit_exact(i):
    t, blk, want = rows()[i]
    got = _decode(t, blk)
    assert got.view(np.uint32).tolist() == want.view(np.uint32).tolist()


def test_golden_two_block_rows():
    # Two consecutive blocks of one type decoded as one row (block indexing), as the reference test does.
    r = rows()
    for i in range(len(r) - 1):
        if r[i][0] == r[i + 1][0] == "Q8_0":
            got = _decode("Q8_0", np.concatenate([r[i][1], r[i + 1][1]]))
            want = np.concatenate([r[i][2], r[i + 1][2]])
            assert got.view(np.uint32).tolist() == want.view(np.uint32).tolist()


@pytest.mark.skipif(not O.has_ref(), reason="oracle/_ref not built (reference sources absent)")
def test_reference_build_agrees_on_golden():
    R = O.ref()
    for t, blk, want in rows():
        if t == "Q8_0":
            out = np.empty(32, np.float32)
            R.ref_dequant_q8_0(blk, out, 32)
            assert out.view(np.uint32).tolist() == want.view(np.uint32).tolist()
        elif t == "F16":
            got = np.array([R.ref_fp16_to_f32(int(h)) for h in blk.view(np.uint16)], np.float32)
            assert got.view(np.uint32).tolist() == want.view(np.uint32).tolist()
