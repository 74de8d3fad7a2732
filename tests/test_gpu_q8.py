"""GPU parity: Q8_0 repack, activation quantizer, exact block dots and the GEMV family (configs C0 and C1).

Bars: integer work (repack bytes, quantized activations and scales, int32 half-block dots) bit-exact against the
oracle; fp32 outputs within 1e-5 * sum|term| + 1e-6 of the oracle's double-accumulated sum (the reference's own
tolerance, tests/gpu/quant_gpu_test.cpp:115-122), which is tighter than the benchmark contract's 1e-3 relative; argmax equal.
"""
import numpy as np
import pytest

import halo_amd as H
import oracle_py as O

pytestmark = pytest.mark.gpu
TOL = 1e-5


def _check_y(y, want, mag):
    err = np.abs(y.astype(np.float64) - want.astype(np.float64))
    bound = TOL * mag + 1e-6
    bad = np.nonzero(err > bound)
    assert bad[0].size == 0, f"{bad[0].size} outputs off; worst {np.max(err - bound)} at {bad}"
    assert np.argmax(y.reshape(-1, y.shape[-1]), -1).tolist() == np.argmax(
        want.reshape(-1, want.shape[-1]), -1).tolist()


def _weights(dev, rng, rows, cols):
    qs, d = O.synth_q8(rng, rows, cols)
    return qs, d, H.Q8Weights.from_host(dev, qs, d)


def test_repack_bit_exact(dev):
    rng = np.random.default_rng(100)
    rows, cols = 257, 2048
    raw = rng.integers(0, 256, rows * (cols // 32) * 34, dtype=np.uint8)
    qs = np.zeros((rows, cols), np.int8)
    d = np.zeros((rows, cols // 32), np.uint16)
    O.oracle().or_repack_q8_0(raw, qs, d, rows, cols, cols)
    graw = dev.to_device(raw)
    w = H.Q8Weights(dev, rows, cols)
    dev.op("repack_q8_0", graw.ptr, w.qs.ptr, w.d.ptr, rows, cols, w.qstride)
    gq, gd = w.host()
    assert np.array_equal(gq, qs) and np.array_equal(gd, d)


@pytest.mark.parametrize("tokens,cols", [(1, 4096), (3, 2048), (16, 512), (1, 32)])
def test_quantizer_bit_exact(dev, tokens, cols):
    rng = np.random.default_rng(cols + tokens)
    x = rng.normal(0, 1, (tokens, cols)).astype(np.float32)
    x[0, :32] = 0.0  # zero block
    if cols >= 64:
        x[0, 32:64] = np.array([127.0, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 126.5] + [0.25] * 24, np.float32)
    gx = dev.to_device(x)
    gq = dev.array((tokens, cols), np.int8)
    gs = dev.array((tokens, cols // 32), np.float32)
    dev.op("quantize_q8", gx.ptr, gq.ptr, gs.ptr, tokens, cols)
    xq, xs = O.quantize(x)
    assert np.array_equal(gs.download().view(np.uint32), xs.view(np.uint32))
    assert np.array_equal(gq.download(), xq)


@pytest.mark.parametrize("tokens", [1, 3, 16])
def test_quantizer_pair_bit_exact(dev, tokens):
    """Two inputs of different widths quantized by one launch: both equal the oracle's quantizer bit for bit."""
    rng = np.random.default_rng(100 + tokens)
    x0 = rng.normal(0, 1, (tokens, 2048)).astype(np.float32)
    x1 = rng.normal(0, 3, (tokens, 4096)).astype(np.float32)
    x1[0, :32] = 0.0
    g0, g1 = dev.to_device(x0), dev.to_device(x1)
    q0, s0 = dev.array((tokens, 2048), np.int8), dev.array((tokens, 64), np.float32)
    q1, s1 = dev.array((tokens, 4096), np.int8), dev.array((tokens, 128), np.float32)
    dev.op("quantize_q8_pair", g0.ptr, q0.ptr, s0.ptr, 2048, g1.ptr, q1.ptr, s1.ptr, 4096, tokens)
    for x, q, sc in ((x0, q0, s0), (x1, q1, s1)):
        xq, xs = O.quantize(x)
        assert np.array_equal(q.download(), xq)
        assert np.array_equal(sc.download().view(np.uint32), xs.view(np.uint32))


def _near_tie_rows(rng, tokens, cols):
    """Rows whose 32-value blocks hold an amax and 31 values within a few ulps of (k + 1/2) * scale: quotients at
    half-integers, where any quotient other than the IEEE one (a reciprocal times v) can round the other way."""
    nb = tokens * cols // 32
    amax = (np.abs(rng.normal(0, 1, nb)) * 10.0 ** rng.integers(-6, 6, nb) + 1e-3).astype(np.float32)
    scale = (amax / np.float32(127.0)).astype(np.float32)
    k = rng.integers(-127, 127, (nb, 31)).astype(np.float32)
    v = ((k + np.float32(0.5)) * scale[:, None]).astype(np.float32)
    steps = rng.integers(-3, 4, v.shape)
    for s_ in range(1, 4):
        v = np.where(steps >= s_, np.nextafter(v, np.float32(np.inf)), v)
        v = np.where(steps <= -s_, np.nextafter(v, np.float32(-np.inf)), v)
    v = np.clip(v, -amax[:, None], amax[:, None])
    blocks = np.concatenate([amax[:, None], v], 1).astype(np.float32)
    blocks = np.take_along_axis(blocks, rng.permuted(np.tile(np.arange(32), (nb, 1)), axis=1), 1)
    return blocks.reshape(tokens, cols)


def test_quantizers_near_ties_bit_exact(dev):
    """Every quantizer's codes equal the oracle's IEEE-quotient codes on values placed at half-integer quotients:
    the standalone and pair quantizers (halo::QuantQuad) and a projection prologue's quantized copy of its input
    (halo::QuantRow8)."""
    rng = np.random.default_rng(2024)
    x = _near_tie_rows(rng, 3, 2048)
    xq, xs = O.quantize(x)
    gx = dev.to_device(x)
    gq, gs = dev.array((3, 2048), np.int8), dev.array((3, 64), np.float32)
    dev.op("quantize_q8", gx.ptr, gq.ptr, gs.ptr, 3, 2048)
    assert np.array_equal(gs.download().view(np.uint32), xs.view(np.uint32))
    assert np.array_equal(gq.download(), xq)
    x1 = _near_tie_rows(rng, 3, 4096)
    g1 = dev.to_device(x1)
    q0, s0 = dev.array((3, 2048), np.int8), dev.array((3, 64), np.float32)
    q1, s1 = dev.array((3, 4096), np.int8), dev.array((3, 128), np.float32)
    dev.op("quantize_q8_pair", gx.ptr, q0.ptr, s0.ptr, 2048, g1.ptr, q1.ptr, s1.ptr, 4096, 3)
    assert np.array_equal(q0.download(), xq)
    x1q, x1s = O.quantize(x1)
    assert np.array_equal(q1.download(), x1q)
    assert np.array_equal(s1.download().view(np.uint32), x1s.view(np.uint32))
    for tokens in (1, 3):
        ws = [H.Q8Weights(dev, 64, 2048).synth(dev, seed=3)]
        ys = [dev.array((tokens, 64), np.float32)]
        xo, so = dev.array((tokens, 2048), np.int8), dev.array((tokens, 64), np.float32)
        H.proj_q8(dev, ws, ys, H.ProjInput(x=gx.ptr, xq_out=xo.ptr, xs_out=so.ptr, mode=H.PROJ_F), tokens)
        assert np.array_equal(xo.download(), xq[:tokens])
        assert np.array_equal(so.download().view(np.uint32), xs[:tokens].view(np.uint32))


def test_q8x_cols_two_level_bit_exact(dev):
    rng = np.random.default_rng(7)
    B, cols, xstride = 3, 2048, 2100
    x = rng.normal(0, 1, (B, xstride)).astype(np.float32)
    gx = dev.to_device(x)
    q1, s1 = dev.array((B, cols), np.int8), dev.array((B, cols // 32), np.float32)
    q2, s2 = dev.array((B, cols), np.int8), dev.array((B, cols // 32), np.float32)
    dev.launch("halo_q8x_cols", ((cols + 255) // 256, B), (256,),
               [gx, ("u32", xstride), ("u32", cols), q1, s1, q2, s2])
    xq, xs = O.quantize(x[:, :cols])
    assert np.array_equal(q1.download(), xq) and np.array_equal(s1.download(), xs)
    resid = (x[:, :cols] - xq.astype(np.float32) * np.repeat(xs, 32, 1)).astype(np.float32)
    rq, rs = O.quantize(resid)
    gq2, gs2 = q2.download(), s2.download()
    bad = np.argwhere(gq2 != rq)
    assert bad.size == 0, f"{len(bad)} residual codes differ, first {bad[:4].tolist()}: gpu {gq2[tuple(bad[0])]} " \
        f"want {rq[tuple(bad[0])]}, scales equal {np.array_equal(gs2, rs)}"
    assert np.array_equal(gs2.view(np.uint32), rs.view(np.uint32))


def test_half_block_dots_bit_exact(dev):
    rng = np.random.default_rng(11)
    rows, cols = 512, 4096
    qs, d, w = _weights(dev, rng, rows, cols)
    x = rng.normal(0, 1, cols).astype(np.float32)
    xq, xs = O.quantize(x)
    gx = dev.to_device(xq)
    gi = dev.array((rows, cols // 16), np.int32)
    dev.op("q8_half_dots", C_ref(w), gx.ptr, gi.ptr)
    half = gi.download()
    want_half = (qs.astype(np.int64).reshape(rows, -1, 16) * xq.astype(np.int64).reshape(1, -1, 16)).sum(-1)
    assert np.array_equal(half, want_half)
    assert np.array_equal(half.reshape(rows, -1, 2).sum(-1), O.block_dots(qs, xq))


def C_ref(w):
    import ctypes

    return ctypes.byref(w.desc)


def _gemv_case(dev, rng, rows, cols, m):
    qs, d, w = _weights(dev, rng, rows, cols)
    x = rng.normal(0, 1, (m, cols)).astype(np.float32)
    xq, xs = O.quantize(x)
    want, mag = O.gemv_q8a8(qs, d, xq, xs)
    return w, xq, xs, want, mag


def test_c0_gemv_4096(dev):
    rng = np.random.default_rng(0)
    w, xq, xs, want, mag = _gemv_case(dev, rng, 4096, 4096, 1)
    gq, gs, gy = dev.to_device(xq), dev.to_device(xs), dev.array((1, 4096), np.float32)
    dev.op("matvec_q8a8", C_ref(w), gq.ptr, gs.ptr, gy.ptr, 1, 4096)
    _check_y(gy.download(), want, mag)


@pytest.mark.parametrize("rows,cols", [(4096, 4096), (1001, 4096), (998, 2048)])
def test_gemv_lds_staged_bitwise(dev, rows, cols):
    """halo_gemv_q8a8s_l64_r1_b1 (the activation row staged in LDS by DMA once per block) gives the bits of
    halo_gemv_q8a8_l64_r1_b1 (the same per-wave arithmetic, activations read per wave), and both meet the oracle."""
    rng = np.random.default_rng(rows + cols)
    w, xq, xs, want, mag = _gemv_case(dev, rng, rows, cols, 1)
    gq, gs = dev.to_device(xq), dev.to_device(xs)
    ys = []
    for name in ("halo_gemv_q8a8_l64_r1_b1", "halo_gemv_q8a8s_l64_r1_b1"):
        gy = dev.array(rows, np.float32)
        dev.launch(name, ((rows + 3) // 4,), (256,), [w.qs, w.d, gq, gs, gy, ("u32", rows),
                                                      ("u32", cols), ("u32", w.qstride), ("u32", rows)])
        ys.append(gy.download())
    for y_ in ys[1:]:
        assert np.array_equal(ys[0].view(np.uint32), y_.view(np.uint32))
    _check_y(ys[1][None, :], want, mag)


@pytest.mark.parametrize("rows,cols", [(4096, 2048), (512, 2048), (2048, 4096)])
@pytest.mark.parametrize("m", [1, 2, 3, 4, 8, 16])
def test_c1_projections(dev, rows, cols, m):
    rng = np.random.default_rng(rows * 31 + cols + m)
    w, xq, xs, want, mag = _gemv_case(dev, rng, rows, cols, m)
    gq, gs = dev.to_device(xq), dev.to_device(xs)
    gy = dev.array((m, rows), np.float32)
    dev.op("matvec_q8a8", C_ref(w), gq.ptr, gs.ptr, gy.ptr, m, rows)
    _check_y(gy.download(), want, mag)


@pytest.mark.parametrize("m", [16, 40, 64, 130])
def test_mfma_tiles(dev, m):
    """M >= 16 runs the int8 MFMA tiles (16 rows x 16 or 64 tokens, one MFMA per Q8_0 block); ragged M and rows."""
    rng = np.random.default_rng(m)
    rows, cols = 1000, 2048
    w, xq, xs, want, mag = _gemv_case(dev, rng, rows, cols, m)
    gq, gs = dev.to_device(xq), dev.to_device(xs)
    gy = dev.array((m, rows + 3), np.float32)
    dev.op("matvec_q8a8", C_ref(w), gq.ptr, gs.ptr, gy.ptr, m, rows + 3)
    _check_y(gy.download()[:, :rows], want, mag)


@pytest.mark.parametrize("lpr", [16, 32, 64])
@pytest.mark.parametrize("rpl", [1, 2, 4])
@pytest.mark.parametrize("m", [1, 8])
def test_tilings_agree(dev, lpr, rpl, m):
    rng = np.random.default_rng(lpr * 7 + rpl + m)
    rows, cols = 1000, 1024  # rows not a multiple of any tile
    w, xq, xs, want, mag = _gemv_case(dev, rng, rows, cols, m)
    gq, gs = dev.to_device(xq), dev.to_device(xs)
    for waves in (1, 4):
        gy = dev.array((m, rows), np.float32)
        dev.op("matvec_q8a8_tiled", C_ref(w), gq.ptr, gs.ptr, gy.ptr, m, rows, lpr, rpl, waves)
        _check_y(gy.download(), want, mag)


@pytest.mark.parametrize("nb", [1, 3, 8])
@pytest.mark.parametrize("r", [1, 2, 4])
def test_reference_named_i8_kernels(dev, nb, r):
    """halo_gemv_q8r_i8_r{R}_b{NB} with the reference's grid convention: 8*R rows per 256-thread block, two
    column groups, split-K in two planes (batch_decode.hip:273-298)."""
    rng = np.random.default_rng(nb * 10 + r)
    rows, cols, groups = 300, 2048, 2
    qs, d, w = _weights(dev, rng, rows, cols)
    x = rng.normal(0, 1, (groups * nb, cols)).astype(np.float32)
    xq, xs = O.quantize(x)
    gq, gs = dev.to_device(xq), dev.to_device(xs)
    chunk, parts = 1024, 2
    ystride = parts * rows  # column b holds its split-K planes back to back (batch_decode.cpp:306-311)
    gy = dev.array((groups * nb, ystride), np.float32).fill(0)
    grid = ((rows + 8 * r - 1) // (8 * r) * groups, parts)
    dev.launch(f"halo_gemv_q8r_i8_r{r}_b{nb}", grid, (256,),
               [w.qs, w.d, gq, gs, None, None, gy, ("u32", rows), ("u32", cols), ("u32", w.qstride),
                ("u32", ystride), ("u32", groups), ("u32", chunk)])
    out = gy.download().astype(np.float64)
    y = out[:, :rows] + out[:, rows:]
    want, mag = O.gemv_q8a8(qs, d, xq, xs)
    _check_y(y.astype(np.float32), want, mag)


def test_fp32x_reference_gemv(dev):
    rng = np.random.default_rng(21)
    for rows, cols in ((4096, 2048), (1000, 4096)):
        qs, d, w = _weights(dev, rng, rows, cols)
        x = rng.normal(0, 1, cols).astype(np.float32)
        want = np.zeros(rows, np.float32)
        O.oracle().or_matvec_q8_0_f32x(qs, d, rows, cols, cols, x, want, 1)
        dw = np.repeat(d.view(np.float16).astype(np.float64), 32, 1)
        mag = (np.abs(qs * dw) @ np.abs(x.astype(np.float64)))
        gx, gy = dev.to_device(x), dev.array((1, rows), np.float32)
        dev.op("matvec_q8_f32x", C_ref(w), gx.ptr, gy.ptr)
        _check_y(gy.download(), want[None], mag[None])


def test_synth_distribution(dev):
    w = H.Q8Weights(dev, 256, 4096).synth(dev, seed=1234)
    qs, d = w.host()
    assert qs.min() == -127 and qs.max() == 127
    dd = d.view(np.float16).astype(np.float64) * 127
    assert abs(np.sqrt((dd ** 2).mean()) - 0.02) < 0.001  # |N(0, 0.02)| has rms 0.02
    w2 = H.Q8Weights(dev, 256, 4096).synth(dev, seed=1234)
    assert np.array_equal(w2.host()[0], qs)  # deterministic


@pytest.mark.parametrize("m,rows,cols", [(128, 512, 2048), (300, 1024, 4096), (2048, 256, 2048), (1100, 3840, 1024),
                                         (200, 200, 64), (77, 136, 128), (130, 200, 192), (64, 256, 320)])
def test_mfma_gemm_prefill_tiles(dev, m, rows, cols):
    """Prefill-sized M (>= 64) runs the 128 x 128 LDS-DMA-staged kernel halo_gemm_q8a8_mfma32 (v_mfma_i32_32x32x32_i8,
    one MFMA per Q8_0 block and 32 x 32 tile); dense output, ragged M and rows. cols 64 .. 320 cover one to five
    64-column stages, i.e. the stage loop's tails after whole rounds of three buffers."""
    rng = np.random.default_rng(m + rows)
    w, xq, xs, want, mag = _gemv_case(dev, rng, rows, cols, m)
    gq, gs = dev.to_device(xq), dev.to_device(xs)
    gy = dev.array((m, rows), np.float32)
    dev.op("matvec_q8a8", C_ref(w), gq.ptr, gs.ptr, gy.ptr, m, rows)
    _check_y(gy.download(), want, mag)


@pytest.mark.parametrize("m,rows,cols", [(300, 1024, 4096), (130, 200, 192)])
def test_mfma_gemm_staging_variants_bitwise(dev, m, rows, cols):
    """The LDS-DMA tile (halo_gemm_q8a8_mfma32) and the register-staged one (halo_gemm_q8a8_mfma32_p) do the same
    arithmetic in the same block order: bitwise equal outputs, both within the oracle's bar."""
    rng = np.random.default_rng(m * 7 + cols)
    w, xq, xs, want, mag = _gemv_case(dev, rng, rows, cols, m)
    gq, gs = dev.to_device(xq), dev.to_device(xs)
    outs = []
    for name in ("halo_gemm_q8a8_mfma32", "halo_gemm_q8a8_mfma32_p"):
        gy = dev.array((m, rows), np.float32)
        dev.launch(name, ((rows + 127) // 128, (m + 127) // 128), (512,),
                   [w.qs, w.d, gq, gs, gy, ("u32", rows), ("u32", cols), ("u32", w.qstride), ("u32", m),
                    ("u32", rows)])
        outs.append(gy.download())
    _check_y(outs[0], want, mag)
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))


@pytest.mark.parametrize("nb,r", [(1, 4), (3, 2), (8, 1)])
def test_reference_named_i8_dual_kernels(dev, nb, r):
    """halo_gemv_q8r_i8_dual_r{R}_b{NB}: two matrices (DeltaNet qkv and z) over the same NB columns in one launch,
    row blocks [0, blocks1) on the first, two column groups (batch_decode.hip:310-345)."""
    rng = np.random.default_rng(nb * 100 + r)
    rows1, rows2, cols, groups = 300, 130, 2048, 2
    qs1, d1, w1 = _weights(dev, rng, rows1, cols)
    qs2, d2, w2 = _weights(dev, rng, rows2, cols)
    x = rng.normal(0, 1, (groups * nb, cols)).astype(np.float32)
    xq, xs = O.quantize(x)
    y1, y2 = dev.array((groups * nb, rows1), np.float32), dev.array((groups * nb, rows2), np.float32)
    blocks1 = (rows1 + 8 * r - 1) // (8 * r)
    grid = ((blocks1 + (rows2 + 8 * r - 1) // (8 * r)) * groups,)
    dev.launch(f"halo_gemv_q8r_i8_dual_r{r}_b{nb}", grid, (256,),
               [w1.qs, w1.d, y1, ("u32", rows1), ("u32", w1.qstride), w2.qs, w2.d, y2, ("u32", rows2),
                ("u32", w2.qstride), dev.to_device(xq), dev.to_device(xs), None, None, ("u32", cols),
                ("u32", blocks1), ("u32", rows1), ("u32", rows2), ("u32", groups)])
    for y, qs, d in ((y1, qs1, d1), (y2, qs2, d2)):
        want, mag = O.gemv_q8a8(qs, d, xq, xs)
        _check_y(y.download(), want, mag)


def test_fp32x_reference_gemv_dual(dev):
    """halo_gemv_q8r_dual: two matrices with the same fp32 input, 32 rows per block (core.hip:2960-2985)."""
    rng = np.random.default_rng(23)
    rows1, rows2, cols = 1000, 77, 2048
    qs1, d1, w1 = _weights(dev, rng, rows1, cols)
    qs2, d2, w2 = _weights(dev, rng, rows2, cols)
    x = rng.normal(0, 1, cols).astype(np.float32)
    y1, y2 = dev.array((1, rows1), np.float32), dev.array((1, rows2), np.float32)
    blocks1 = (rows1 + 31) // 32
    dev.launch("halo_gemv_q8r_dual", (blocks1 + (rows2 + 31) // 32,), (256,),
               [w1.qs, w1.d, y1, ("u32", rows1), ("u32", w1.qstride), w2.qs, w2.d, y2, ("u32", rows2),
                ("u32", w2.qstride), dev.to_device(x), ("u32", cols), ("u32", blocks1)])
    for y, qs, d, rows in ((y1, qs1, d1, rows1), (y2, qs2, d2, rows2)):
        want = np.zeros(rows, np.float32)
        O.oracle().or_matvec_q8_0_f32x(qs, d, rows, cols, cols, x, want, 1)
        mag = np.abs(qs * np.repeat(d.view(np.float16).astype(np.float64), 32, 1)) @ np.abs(x.astype(np.float64))
        _check_y(y.download(), want[None], mag[None])
