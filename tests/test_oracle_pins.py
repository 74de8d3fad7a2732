"""Pins for the CPU oracle (oracle/oracle.c): closed forms, brute force and the reference's own CPU code.

Each check is chosen so that a plausible slip in the oracle (wrong rounding mode, dropped scale, transposed
operand, wrong tie order) fails it. The oracle/_ref checks compare with the reference's cpu_ops.cpp / quant.cpp
compiled from its sources (skipped where the reference tree is absent, e.g. on the GPU box).
"""
import numpy as np
import pytest

import oracle_py as O

needs_ref = pytest.mark.skipif(not O.has_ref(), reason="oracle/_ref not built")


def test_fp16_decode_exhaustive():
    o = O.oracle()
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = np.array([o.or_fp16_to_f32(int(v)) for v in h], np.float32)
    want = h.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_fp16_encode_matches_ieee_rne():
    o = O.oracle()
    rng = np.random.default_rng(1)
    xs = np.concatenate([
        rng.normal(0, 1, 4000).astype(np.float32),
        (rng.normal(0, 1, 4000) * 1e-5).astype(np.float32),  # subnormal halves
        (rng.normal(0, 1, 2000) * 7e4).astype(np.float32),  # overflow
        np.array([0.0, -0.0, 65504.0, 65520.0, 65519.996, 2.0 ** -24, 2.0 ** -25, 3 * 2.0 ** -26], np.float32),
        # exact ties between two halves: 1 + (2k+1) * 2^-11
        (1.0 + (2 * np.arange(50) + 1) * 2.0 ** -11).astype(np.float32),
    ])
    got = np.array([o.or_f32_to_fp16(float(x)) for x in xs], np.uint16)
    want = xs.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)


def test_bf16_round_trip():
    o = O.oracle()
    rng = np.random.default_rng(2)
    xs = rng.normal(0, 3, 2000).astype(np.float32)
    for x in xs:
        b = o.or_f32_to_bf16(float(x))
        y = o.or_bf16_to_f32(b)
        # RNE: the result is the nearer of the two bf16 neighbours.
        u = np.float32(x).view(np.uint32)
        lo = np.uint32(u & 0xFFFF0000).view(np.float32)
        hi = np.uint32((u & 0xFFFF0000) + 0x10000).view(np.float32)
        assert y in (lo, hi)
        assert abs(y - x) <= abs((hi if y == lo else lo) - x)


def _np_quantize(x):
    x = x.reshape(-1, 32).astype(np.float32)
    amax = np.abs(x).max(axis=1)
    scale = (amax / np.float32(127.0)).astype(np.float32)
    with np.errstate(divide="ignore", invalid="ignore"):
        q = np.where(scale[:, None] > 0, np.rint(x / scale[:, None]), 0).astype(np.int8)
    return q.reshape(-1), scale


def test_quantizer_closed_form_random():
    rng = np.random.default_rng(3)
    x = rng.normal(0, 1, 32 * 512).astype(np.float32)
    xq, xs = O.quantize(x)
    q, s = _np_quantize(x)
    assert np.array_equal(xs.view(np.uint32), s.view(np.uint32))
    assert np.array_equal(xq, q)


def test_quantizer_edge_blocks():
    blocks = []
    blocks.append(np.zeros(32, np.float32))  # all zero -> scale 0, q 0
    b = np.zeros(32, np.float32)
    b[0] = 127.0
    b[1:8] = [0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 126.5]  # exact halves: ties to even
    blocks.append(b)
    blocks.append(np.full(32, -3.0, np.float32))  # all -amax -> -127
    tiny = np.zeros(32, np.float32)
    tiny[3] = np.float32(1e-40)  # denormal amax
    tiny[4] = np.float32(-5e-41)
    blocks.append(tiny)
    x = np.concatenate(blocks)
    xq, xs = O.quantize(x)
    q, s = _np_quantize(x)
    assert np.array_equal(xq, q) and np.array_equal(xs.view(np.uint32), s.view(np.uint32))
    assert xs[0] == 0 and not xq[:32].any()
    assert xq[32:40].tolist() == [127, 0, 2, 2, 0, -2, -2, 126]
    assert (xq[64:96] == -127).all()
    assert xq[96 + 3] == 127


def test_block_dots_brute_force():
    rng = np.random.default_rng(4)
    qs = rng.integers(-127, 128, (37, 96), dtype=np.int8)
    xq = rng.integers(-128, 128, 96, dtype=np.int8)
    got = O.block_dots(qs, xq)
    want = (qs.astype(np.int64).reshape(37, 3, 32) * xq.astype(np.int64).reshape(1, 3, 32)).sum(-1)
    assert np.array_equal(got, want)
    # extremes: 32 * (-127 * -128) fits int32
    qs = np.full((1, 32), -127, np.int8)
    xq = np.full(32, -128, np.int8)
    assert O.block_dots(qs, xq)[0, 0] == 32 * 127 * 128


def test_gemv_q8a8_matches_float64_restatement():
    rng = np.random.default_rng(5)
    qs, d = O.synth_q8(rng, 64, 256)
    x = rng.normal(0, 1, 256).astype(np.float32)
    xq, xs = O.quantize(x)
    y, mag = O.gemv_q8a8(qs, d, xq, xs)
    isum = O.block_dots(qs, xq).astype(np.float64)
    dw = d.view(np.float16).astype(np.float64)
    want = (dw * xs.astype(np.float64)[None, :] * isum).sum(1)
    assert np.array_equal(y, want.astype(np.float32))
    assert np.allclose(mag, np.abs(dw * xs[None, :] * isum).sum(1))
    # and it approximates the fp32 product W x to the quantization error
    w = (qs.reshape(64, 8, 32) * dw[:, :, None]).reshape(64, 256)
    assert np.all(np.abs(y - w @ x) <= 0.02 * np.abs(w) @ np.abs(x) + 1e-6)


def test_repack_pack_round_trip():
    rng = np.random.default_rng(6)
    raw = rng.integers(0, 256, 7 * 4 * 34, dtype=np.uint8)
    o = O.oracle()
    qs = np.zeros((7, 144), np.int8)
    d = np.zeros((7, 4), np.uint16)
    o.or_repack_q8_0(raw, qs, d, 7, 128, 144)
    back = np.zeros_like(raw)
    o.or_pack_q8_0(qs, d, back, 7, 128, 144)
    assert np.array_equal(raw, back)
    blk = raw[:34]
    assert int(d[0, 0]) == int(blk[0]) | (int(blk[1]) << 8)
    assert np.array_equal(qs[0, :32], blk[2:].view(np.int8))


def test_route_topk_ties_and_renorm():
    o = O.oracle()
    rng = np.random.default_rng(7)
    # 0.25-grid logits so that ties are exact (reference tests/model/routing_test.cpp:40)
    logits = (rng.integers(-8, 8, 512) * 0.25).astype(np.float32)
    ids = np.zeros(10, np.uint32)
    w = np.zeros(10, np.float32)
    o.or_route_topk(logits, 512, 10, ids, w)
    order = sorted(range(512), key=lambda i: (-logits[i], i))[:10]  # stable: ties -> lower id
    assert ids.tolist() == order
    assert abs(w.sum() - 1.0) < 1e-6
    assert np.all(np.diff(w) <= 0)


@needs_ref
def test_route_topk_matches_reference():
    o, R = O.oracle(), O.ref()
    rng = np.random.default_rng(8)
    for trial in range(50):
        logits = (rng.normal(0, 1, 512) if trial % 2 else rng.integers(-4, 4, 512) * 0.25).astype(np.float32)
        a_i, a_w = np.zeros(10, np.uint32), np.zeros(10, np.float32)
        b_i, b_w = np.zeros(10, np.uint32), np.zeros(10, np.float32)
        o.or_route_topk(logits, 512, 10, a_i, a_w)
        R.ref_route_topk(logits, 512, 10, b_i, b_w)
        assert np.array_equal(a_i, b_i) and np.array_equal(a_w.view(np.uint32), b_w.view(np.uint32))


@needs_ref
def test_matvec_f32x_matches_reference_bitwise():
    o, R = O.oracle(), O.ref()
    rng = np.random.default_rng(9)
    qs, d = O.synth_q8(rng, 300, 512)
    raw = np.zeros(300 * 16 * 34, np.uint8)
    o.or_pack_q8_0(qs, d, raw, 300, 512, 512)
    x = rng.normal(0, 1, 512).astype(np.float32)
    a = np.zeros(300, np.float32)
    b = np.zeros(300, np.float32)
    o.or_matvec_q8_0_f32x(qs, d, 300, 512, 512, x, a, 4)
    R.ref_matvec_q8_0(raw, 300, 512, x, b)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


@needs_ref
@pytest.mark.parametrize("rows,cols", [(512, 2048), (3, 1001), (600, 2048)])
def test_matvec_f32_matches_reference_bitwise(rows, cols):
    """or_matvec_f32 (the router / rowblock checker) against the reference's cpu::MatVec over an F32 tensor
    (cpu_ops.cpp:97-132): double accumulation in column order, bitwise, including the row-split threaded case
    (rows * cols >= 2^20) and ragged shapes."""
    o, R = O.oracle(), O.ref()
    rng = np.random.default_rng(rows + cols)
    w = rng.normal(0, 0.02, (rows, cols)).astype(np.float32)
    x = rng.normal(0, 1, cols).astype(np.float32)
    a, b = np.zeros(rows, np.float32), np.zeros(rows, np.float32)
    o.or_matvec_f32(w, rows, cols, x, a)
    R.ref_matvec_f32(w, rows, cols, x, b)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_matvec_f32_closed_form():
    """One-hot rows select x exactly; a row of ones over exactly representable values sums exactly."""
    o = O.oracle()
    cols = 96
    x = (np.arange(cols, dtype=np.float32) - 40.0) * 0.25
    w = np.zeros((cols + 1, cols), np.float32)
    w[np.arange(cols), (np.arange(cols) * 7) % cols] = 1.0
    w[cols] = 1.0
    y = np.zeros(cols + 1, np.float32)
    o.or_matvec_f32(w, cols + 1, cols, x, y)
    assert np.array_equal(y[:cols], x[(np.arange(cols) * 7) % cols])
    assert y[cols] == np.float32(x.astype(np.float64).sum())


@needs_ref
def test_elementwise_match_reference():
    o, R = O.oracle(), O.ref()
    rng = np.random.default_rng(10)
    for v in rng.normal(0, 8, 300).astype(np.float32):
        assert o.or_silu(float(v)) == R.ref_silu(float(v))
        assert o.or_sigmoid(float(v)) == R.ref_sigmoid(float(v))
        assert o.or_softplus(float(v)) == R.ref_softplus(float(v))
    for fn_o, fn_r in ((o.or_l2norm, R.ref_l2norm),):
        x = rng.normal(0, 1, 128).astype(np.float32)
        a, b = x.copy(), x.copy()
        fn_o(a, 128, 1e-6)
        fn_r(b, 128, 1e-6)
        assert np.array_equal(a, b)
    x = rng.normal(0, 1, 256).astype(np.float32)
    w = rng.normal(1, 0.1, 256).astype(np.float32)
    a, b = x.copy(), x.copy()
    o.or_rmsnorm(a, 256, w.ctypes.data, 1e-6)
    R.ref_rmsnorm(b, 256, w.ctypes.data, 1e-6)
    assert np.array_equal(a, b)
    x = rng.normal(0, 1, 4 * 256).astype(np.float32)
    a, b = x.copy(), x.copy()
    o.or_rope_neox(a, 4, 256, 64, 8191, 1e7)
    R.ref_rope(b, 4, 256, 64, 8191, 1e7)
    assert np.array_equal(a, b)


def test_rope_closed_form():
    # position 0 is the identity; the rotation preserves each pair's norm; pair i turns by pos * theta^(-2i/rot)
    o = O.oracle()
    rng = np.random.default_rng(11)
    x = rng.normal(0, 1, 256).astype(np.float32)
    a = x.copy()
    o.or_rope_neox(a, 1, 256, 256, 0, 1e7)
    assert np.array_equal(a, x)
    a = x.copy()
    o.or_rope_neox(a, 1, 256, 256, 77, 1e7)
    i = np.arange(128)
    ang = 77 * (1e7 ** (-2.0 * i / 256))
    want_lo = x[:128] * np.cos(ang) - x[128:] * np.sin(ang)
    want_hi = x[:128] * np.sin(ang) + x[128:] * np.cos(ang)
    assert np.allclose(a[:128], want_lo, atol=1e-4) and np.allclose(a[128:], want_hi, atol=1e-4)


def _np_gdn_step(S, q, k, v, g, beta):
    S = S * np.exp(g)
    u = S @ k
    delta = (v - u) * beta
    S = S + np.outer(delta, k)
    return S, (S @ q) / np.sqrt(len(q))


def test_gdn_step_invariants():
    o = O.oracle()
    rng = np.random.default_rng(12)
    d = 16
    q = rng.normal(0, 1, d).astype(np.float32)
    k = rng.normal(0, 1, d).astype(np.float32)
    k /= np.linalg.norm(k)
    v = rng.normal(0, 1, d).astype(np.float32)
    # beta = 1, |k| = 1: the delta rule stores v exactly under key k (S_new k = v).
    S = rng.normal(0, 1, (d, d)).astype(np.float32)
    S1 = S.copy()
    out = np.zeros(d, np.float32)
    o.or_gdn_step(S1, d, q, k, v, -0.3, 1.0, out)
    assert np.allclose(S1 @ k, v, atol=1e-5)
    # beta = 0: decay only
    S2 = S.copy()
    o.or_gdn_step(S2, d, q, k, v, -0.7, 0.0, out)
    assert np.allclose(S2, S * np.exp(np.float32(-0.7)), rtol=1e-6)
    # general case against a float64 restatement
    S3 = S.copy()
    o.or_gdn_step(S3, d, q, k, v, -0.2, 0.6, out)
    Sw, ow = _np_gdn_step(S.astype(np.float64), q, k, v, -0.2, 0.6)
    assert np.allclose(S3, Sw, atol=1e-5) and np.allclose(out, ow, atol=1e-5)


def test_gdn_sequence_mag_closed_form_and_bound():
    """The DeltaNet error bar: from a zero state one token gives M = |beta| |v| |k|^T and o_mag = |beta| |v| (|k| .
    |q|) / sqrt(d); with all inputs non-negative and a non-negative state (no cancellation) the bar equals |o| and
    |S| exactly (up to fp32 rounding of the value path); over random signed sequences it bounds |o| and |S|."""
    o = O.oracle()
    rng = np.random.default_rng(21)
    d, T = 16, 9
    q = rng.normal(0, 1, (T, d)).astype(np.float32)
    k = rng.normal(0, 1, (T, d)).astype(np.float32)
    v = rng.normal(0, 1, (T, d)).astype(np.float32)
    g = rng.normal(-0.3, 0.2, T).astype(np.float32)
    b = rng.uniform(0.1, 0.9, T).astype(np.float32)
    M = np.zeros((d, d), np.float64)
    om = np.zeros((T, d), np.float64)
    o.or_gdn_sequence_mag(M.ctypes.data, d, 1, q.ctypes.data, d, k.ctypes.data, d, v.ctypes.data, d, g.ctypes.data,
                          b.ctypes.data, 1, om.ctypes.data, d)
    v64, k64, q64, b64 = (x.astype(np.float64) for x in (v[0], k[0], q[0], b[0]))
    assert np.allclose(M, b64 * np.outer(np.abs(v64), np.abs(k64)), rtol=1e-12)
    assert np.allclose(om[0], b64 * np.abs(v64) * (np.abs(k64) @ np.abs(q64)) / np.sqrt(d), rtol=1e-12)
    # signed sequence: a bound on the values
    S0 = rng.normal(0, 0.5, (d, d)).astype(np.float32)
    S = S0.copy()
    M = np.abs(S0).astype(np.float64)
    out = np.zeros((T, d), np.float32)
    o.or_gdn_sequence(S, d, T, q.ctypes.data, d, k.ctypes.data, d, v.ctypes.data, d, g.ctypes.data, b.ctypes.data, 1,
                      out.ctypes.data, d)
    o.or_gdn_sequence_mag(M.ctypes.data, d, T, q.ctypes.data, d, k.ctypes.data, d, v.ctypes.data, d, g.ctypes.data,
                          b.ctypes.data, 1, om.ctypes.data, d)
    assert np.all(np.abs(out) <= om * (1 + 1e-5)) and np.all(np.abs(S) <= M * (1 + 1e-5))
    # no cancellation (q, k >= 0, v >= 0, S0 >= 0, and decay S k never exceeds v: beta small, state small): equal
    qp, kp, vp = np.abs(q), np.abs(k) * 0.01, np.abs(v) + 5.0
    S = np.zeros((d, d), np.float32)
    M = np.zeros((d, d), np.float64)
    o.or_gdn_sequence(S, d, 1, qp.ctypes.data, d, kp.ctypes.data, d, vp.ctypes.data, d, g.ctypes.data,
                      b.ctypes.data, 1, out.ctypes.data, d)
    o.or_gdn_sequence_mag(M.ctypes.data, d, 1, qp.ctypes.data, d, kp.ctypes.data, d, vp.ctypes.data, d,
                          g.ctypes.data, b.ctypes.data, 1, om.ctypes.data, d)
    assert np.allclose(S, M, rtol=1e-6) and np.allclose(out[0], om[0], rtol=1e-6)


def test_attention_head_closed_forms():
    o = O.oracle()
    rng = np.random.default_rng(13)
    hd = 8
    q = rng.normal(0, 1, hd).astype(np.float32)
    k = rng.normal(0, 1, (5, hd)).astype(np.float32)
    v = rng.normal(0, 1, (5, hd)).astype(np.float32)
    out = np.zeros(hd, np.float32)
    o.or_attention_head(q, k[:1].copy(), v[:1].copy(), 1, hd, hd, out)
    assert np.allclose(out, v[0])  # one position: the value itself
    kk = np.repeat(k[:1], 5, 0)
    o.or_attention_head(q, np.ascontiguousarray(kk), v, 5, hd, hd, out)
    assert np.allclose(out, v.mean(0), atol=1e-6)  # equal keys: the mean of the values
    o.or_attention_head(q, k, v, 5, hd, hd, out)
    s = k @ q / np.sqrt(hd)
    p = np.exp(s - s.max())
    p /= p.sum()
    assert np.allclose(out, p @ v, atol=1e-6)
