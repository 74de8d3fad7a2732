"""GPU parity for the grouped projections with a fused activation prologue (halo_op_proj_q8).

Bars: the prologue's quantized activations are bit-exact against the oracle's quantizer (mode F) and against the
standalone residual-add + RMSNorm + quantize kernel (mode N, same canonical row decomposition); the residual written
back is bit-exact; every output row is within 1e-5 * sum|term| + 1e-6 of the oracle's GEMV on those activations
(the reference's tolerance, tests/gpu/quant_gpu_test.cpp:115-122) and the argmax is equal; mode Q on the same
activations gives the same bits as mode F.
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
    assert not np.any(err > bound), f"{np.count_nonzero(err > bound)} outputs off"
    assert np.argmax(y, -1).tolist() == np.argmax(want, -1).tolist()


def _mats(dev, rng, shapes):
    host, dev_w = [], []
    for rows, cols in shapes:
        qs, d = O.synth_q8(rng, rows, cols)
        host.append((qs, d))
        dev_w.append(H.Q8Weights.from_host(dev, qs, d))
    return host, dev_w


@pytest.mark.parametrize("tokens", [1, 2, 3, 4, 8])
@pytest.mark.parametrize("shapes", [
    [(4096, 2048), (512, 2048)],                    # C1 q|gate and kv
    [(2048, 4096)],                                  # C1 o
    [(8192, 2048), (4096, 2048), (64, 2048)],        # DeltaNet q|k|v, z, alpha|beta
    [(300, 512), (17, 512), (1, 512), (64, 512)],    # ragged rows, four matrices, LPR 32
    [(40, 256)],                                     # LPR 16
])
def test_proj_mode_f_and_q(dev, tokens, shapes):
    rng = np.random.default_rng(tokens * 7 + len(shapes))
    cols = shapes[0][1]
    host, ws = _mats(dev, rng, shapes)
    x = rng.normal(0, 1, (tokens, cols)).astype(np.float32)
    x[0, :32] = 0.0
    gx = dev.to_device(x)
    xq_o, xs_o = dev.array((tokens, cols), np.int8), dev.array((tokens, cols // 32), np.float32)
    outs = [dev.array((tokens, r), np.float32) for r, _ in shapes]
    inp = H.ProjInput(x=gx.ptr, xq_out=xq_o.ptr, xs_out=xs_o.ptr, mode=H.PROJ_F)
    H.proj_q8(dev, ws, outs, inp, tokens)
    xq, xs = O.quantize(x)
    assert np.array_equal(xq_o.download(), xq)
    assert np.array_equal(xs_o.download().view(np.uint32), xs.view(np.uint32))
    got_f = [o.download() for o in outs]
    for (qs, d), y in zip(host, got_f):
        want, mag = O.gemv_q8a8(qs, d, xq, xs)
        _check_y(y, want, mag)
    # mode Q on the same activations through the same (v_dot4) kernel: the same bits
    outs_q = [dev.array((tokens, r), np.float32) for r, _ in shapes]
    inq = H.ProjInput(xq=xq_o.ptr, xs=xs_o.ptr, mode=H.PROJ_Q)
    H.proj_q8(dev, ws, outs_q, inq, tokens, 1, 1)
    for a, o in zip(got_f, outs_q):
        assert np.array_equal(a.view(np.uint32), o.download().view(np.uint32))


@pytest.mark.parametrize("tokens", [1, 2, 3, 5, 8, 9, 12, 16])
@pytest.mark.parametrize("shapes", [
    [(4096, 2048), (512, 2048)],                        # C1 q|gate and kv
    [(2048, 4096)],                                      # C1 o
    [(300, 1024), (17, 1024), (1, 1024), (64, 1024)],   # ragged rows (partial 16-row tasks), four matrices
])
def test_proj_mode_q_matrix_cores(dev, tokens, shapes):
    """halo_proj_q8m_c* (int8 MFMA, two Q8_0 blocks per step with separate integer sums; the default for mode Q at
    9-16 tokens, forced here from 1): every output within 1e-5 * sum|term| of the oracle's GEMV on the same codes,
    argmax equal; a zero block and an all-zero token row included; token 0's outputs carry the same bits as at one
    token (each token's products and sums depend on its own row only)."""
    rng = np.random.default_rng(tokens * 11 + len(shapes))
    cols = shapes[0][1]
    host, ws = _mats(dev, rng, shapes)
    x = rng.normal(0, 1, (tokens, cols)).astype(np.float32)
    x[0, 32:64] = 0.0
    x[tokens - 1] = 0.0 if tokens > 2 else x[tokens - 1]
    xq, xs = O.quantize(x)
    gq, gs = dev.to_device(xq), dev.to_device(xs)
    outs = [dev.array((tokens, r), np.float32) for r, _ in shapes]
    H.proj_q8(dev, ws, outs, H.ProjInput(xq=gq.ptr, xs=gs.ptr, mode=H.PROJ_Q), tokens, 2, 2)
    for (qs, d), o in zip(host, outs):
        want, mag = O.gemv_q8a8(qs, d, xq, xs)
        y = o.download()
        err = np.abs(y.astype(np.float64) - want.astype(np.float64))
        assert not np.any(err > TOL * mag + 1e-6), f"{np.count_nonzero(err > TOL * mag + 1e-6)} outputs off"
        live = np.abs(want).max(-1) > 0
        assert np.argmax(y[live], -1).tolist() == np.argmax(want[live], -1).tolist()
        if tokens > 2:
            assert not np.any(y[tokens - 1])
    one = [dev.array((1, r), np.float32) for r, _ in shapes]
    H.proj_q8(dev, ws, one, H.ProjInput(xq=gq.ptr, xs=gs.ptr, mode=H.PROJ_Q), 1, 2, 2)
    for a, b in zip(outs, one):
        assert a.download()[0].tobytes() == b.download()[0].tobytes()


@pytest.mark.parametrize("tokens,cols,with_delta", [(1, 2048, True), (4, 2048, True), (3, 4096, False),
                                                    (8, 2048, True)])
def test_proj_mode_n_matches_norm_kernel(dev, tokens, cols, with_delta):
    rng = np.random.default_rng(tokens + cols)
    shapes = [(1024, cols), (512, cols)]
    host, ws = _mats(dev, rng, shapes)
    res = rng.normal(0, 1, (tokens, cols)).astype(np.float32)
    delta = rng.normal(0, 0.5, (tokens, cols)).astype(np.float32)
    w = (1.0 + 0.1 * rng.normal(0, 1, cols)).astype(np.float32)
    eps = 1e-6
    gres, gdel, gw = dev.to_device(res), dev.to_device(delta), dev.to_device(w)
    rout = dev.array((tokens, cols), np.float32)
    xq_o, xs_o = dev.array((tokens, cols), np.int8), dev.array((tokens, cols // 32), np.float32)
    outs = [dev.array((tokens, r), np.float32) for r, _ in shapes]
    inp = H.ProjInput(x=gres.ptr, delta=gdel.ptr if with_delta else None, norm_w=gw.ptr, res_out=rout.ptr,
                      xq_out=xq_o.ptr, xs_out=xs_o.ptr, eps=eps, mode=H.PROJ_N)
    H.proj_q8(dev, ws, outs, inp, tokens)
    # the standalone norm kernel on a copy of the residual
    r2 = dev.to_device(res)
    xn2 = dev.array((tokens, cols), np.float32)
    xq2, xs2 = dev.array((tokens, cols), np.int8), dev.array((tokens, cols // 32), np.float32)
    dev.launch("halo_add_rmsnorm_q8", (tokens,), (256,),
               [r2, gdel if with_delta else None, gw, xn2, xq2, xs2, ("u32", cols), ("f32", eps)])
    summed = res + delta if with_delta else res
    if with_delta:
        assert np.array_equal(rout.download().view(np.uint32), summed.view(np.uint32))
        assert np.array_equal(r2.download().view(np.uint32), summed.view(np.uint32))
    assert np.array_equal(xq_o.download(), xq2.download())
    assert np.array_equal(xs_o.download().view(np.uint32), xs2.download().view(np.uint32))
    # the norm itself against the oracle's RMSNorm (fp32 sums in another order: 1e-5 relative)
    xn_want = summed.copy()
    for t in range(tokens):
        O.oracle().or_rmsnorm(xn_want[t], cols, w.ctypes.data, eps)
    assert np.allclose(xn2.download(), xn_want, rtol=1e-5, atol=1e-6)
    xq, xs = xq2.download(), xs2.download()
    for (qs, d), y in zip(host, outs):
        want, mag = O.gemv_q8a8(qs, d, xq, xs)
        _check_y(y.download(), want, mag)


@pytest.mark.parametrize("cols,with_delta", [(2048, True), (1024, False)])
def test_proj_mode_n_one_token_every_tiling(dev, cols, with_delta):
    """At one token the RMSNorm prologue runs in one wave (lanes playing the 256-thread layout); every tiling gives
    the norm kernel's residual, codes and scales and the same outputs bit for bit."""
    rng = np.random.default_rng(cols + 7)
    shapes = [(1024, cols), (512, cols), (64, cols)]
    host, ws = _mats(dev, rng, shapes)
    res = rng.normal(0, 1, (1, cols)).astype(np.float32)
    delta = rng.normal(0, 0.5, (1, cols)).astype(np.float32)
    w = (1.0 + 0.1 * rng.normal(0, 1, cols)).astype(np.float32)
    gres, gdel, gw = dev.to_device(res), dev.to_device(delta), dev.to_device(w)
    r2 = dev.to_device(res)
    xn2 = dev.array((1, cols), np.float32)
    xq2, xs2 = dev.array((1, cols), np.int8), dev.array((1, cols // 32), np.float32)
    dev.launch("halo_add_rmsnorm_q8", (1,), (256,),
               [r2, gdel if with_delta else None, gw, xn2, xq2, xs2, ("u32", cols), ("f32", 1e-6)])
    for lpr in (16, 32, 64):
        if cols > 64 * lpr:
            continue
        for tpw in (1, 2, 4):
            rout = dev.array((1, cols), np.float32)
            xq_o, xs_o = dev.array((1, cols), np.int8), dev.array((1, cols // 32), np.float32)
            outs = [dev.array((1, r), np.float32) for r, _ in shapes]
            inp = H.ProjInput(x=gres.ptr, delta=gdel.ptr if with_delta else None, norm_w=gw.ptr, res_out=rout.ptr,
                              xq_out=xq_o.ptr, xs_out=xs_o.ptr, eps=1e-6, mode=H.PROJ_N)
            H.proj_q8(dev, ws, outs, inp, 1, tpw, lpr)
            if with_delta:
                assert np.array_equal(rout.download().view(np.uint32), (res + delta).view(np.uint32))
            assert np.array_equal(xq_o.download(), xq2.download()), (lpr, tpw)
            assert np.array_equal(xs_o.download().view(np.uint32), xs2.download().view(np.uint32)), (lpr, tpw)
            xq, xs = xq2.download(), xs2.download()
            for (qs, d), y in zip(host, outs):
                want, mag = O.gemv_q8a8(qs, d, xq, xs)
                _check_y(y.download(), want, mag)


def test_proj_rejects_bad_shapes(dev):
    rng = np.random.default_rng(5)
    _, ws = _mats(dev, rng, [(64, 2048), (64, 1024)])
    x = dev.array((1, 2048), np.float32)
    outs = [dev.array((1, 64), np.float32) for _ in range(2)]
    with pytest.raises(H.HaloError):
        H.proj_q8(dev, ws, outs, H.ProjInput(x=x.ptr, mode=H.PROJ_F), 1)          # cols differ
    with pytest.raises(H.HaloError):
        H.proj_q8(dev, ws[:1], outs[:1], H.ProjInput(x=x.ptr, mode=H.PROJ_F), 9)  # too many tokens
    with pytest.raises(H.HaloError):
        H.proj_q8(dev, ws[:1], outs[:1], H.ProjInput(x=x.ptr, norm_w=x.ptr, res_out=x.ptr, mode=H.PROJ_N), 1)


@pytest.mark.parametrize("tokens", [1, 4])
def test_proj_mode_g_matches_gated_norm_kernel(dev, tokens):
    """DeltaNet output projection: per-head RMSNorm * w * sigmoid(z) (reference.cpp:359-364) in the prologue."""
    rng = np.random.default_rng(40 + tokens)
    Hv, d = 32, 128
    cols = Hv * d
    host, ws = _mats(dev, rng, [(2048, cols)])
    o = rng.normal(0, 1, (tokens, cols)).astype(np.float32)
    z = rng.normal(0, 1, (tokens, cols)).astype(np.float32)
    w = (1.0 + 0.1 * rng.normal(0, 1, d)).astype(np.float32)
    eps = 1e-6
    go, gz, gw = dev.to_device(o), dev.to_device(z), dev.to_device(w)
    xq_o, xs_o = dev.array((tokens, cols), np.int8), dev.array((tokens, cols // 32), np.float32)
    y = dev.array((tokens, 2048), np.float32)
    inp = H.ProjInput(x=go.ptr, delta=gz.ptr, norm_w=gw.ptr, xq_out=xq_o.ptr, xs_out=xs_o.ptr, eps=eps,
                      mode=H.PROJ_G)
    H.proj_q8(dev, ws, [y], inp, tokens)
    xq2, xs2 = dev.array((tokens, cols), np.int8), dev.array((tokens, cols // 32), np.float32)
    dev.launch("halo_gated_rmsnorm_q8", (tokens,), (256,),
               [go, gz, gw, xq2, xs2, ("u32", Hv), ("u32", d), ("f32", eps)])
    a_s, b_s = xs_o.download(), xs2.download()
    bad = np.nonzero(a_s.view(np.uint32) != b_s.view(np.uint32))
    assert bad[0].size == 0, f"scales differ at {bad}: {a_s[bad][:8]} vs {b_s[bad][:8]}"
    assert np.array_equal(xq_o.download(), xq2.download())
    # the oracle: cpu RmsNorm per head, then sigmoid(z) (reference.cpp:359-364)
    want = o.copy()
    for t in range(tokens):
        for h in range(Hv):
            seg = np.ascontiguousarray(want[t, h * d:(h + 1) * d])
            O.oracle().or_rmsnorm(seg, d, w.ctypes.data, eps)
            want[t, h * d:(h + 1) * d] = seg * np.array([O.oracle().or_sigmoid(float(v)) for v in
                                                         z[t, h * d:(h + 1) * d]], np.float32)
    xq_w, xs_w = O.quantize(want)
    got_q = xq2.download().astype(np.int32)
    diff = got_q - xq_w.astype(np.int32)
    assert np.abs(diff).max() <= 1 and np.count_nonzero(diff) <= max(2, diff.size // 2000)
    assert np.allclose(xs2.download(), xs_w, rtol=1e-5)
    qs, dd = host[0]
    want_y, mag = O.gemv_q8a8(qs, dd, xq2.download(), xs2.download())
    _check_y(y.download(), want_y, mag)


@pytest.mark.parametrize("tokens", [2, 3, 4, 8, 9, 16])
def test_proj_pair_matches_two_launches(dev, tokens):
    """The C1 pass's two projections with their own quantized inputs in one launch (q | gate + kv on x, o on a):
    bit for bit the outputs of the two grouped launches (v_dot4 up to 8 tokens, int8 matrix cores from 9), and
    within the bar of the oracle."""
    rng = np.random.default_rng(300 + tokens)
    host1, ws1 = _mats(dev, rng, [(4096, 2048), (512, 2048)])
    host2, ws2 = _mats(dev, rng, [(2048, 4096)])
    x = rng.normal(0, 1, (tokens, 2048)).astype(np.float32)
    a = rng.normal(0, 1, (tokens, 4096)).astype(np.float32)
    xq, xs = O.quantize(x)
    aq, as_ = O.quantize(a)
    gxq, gxs, gaq, gas = (dev.to_device(v) for v in (xq, xs, aq, as_))
    in1 = H.ProjInput(xq=gxq.ptr, xs=gxs.ptr, mode=H.PROJ_Q)
    in2 = H.ProjInput(xq=gaq.ptr, xs=gas.ptr, mode=H.PROJ_Q)
    sep = [dev.array((tokens, r), np.float32) for r in (4096, 512, 2048)]
    H.proj_q8(dev, ws1, sep[:2], in1, tokens)
    H.proj_q8(dev, ws2, sep[2:], in2, tokens)
    pair = [dev.array((tokens, r), np.float32) for r in (4096, 512, 2048)]
    H.proj_q8_pair(dev, ws1 + ws2, pair, 2, in1, in2, tokens)
    for s_, p_ in zip(sep, pair):
        assert s_.download().tobytes() == p_.download().tobytes()
    for (qs, d), y in zip(host1, pair[:2]):
        want, mag = O.gemv_q8a8(qs, d, xq, xs)
        _check_y(y.download(), want, mag)
    want, mag = O.gemv_q8a8(host2[0][0], host2[0][1], aq, as_)
    _check_y(pair[2].download(), want, mag)


def test_proj_pair_rejects_bad_shapes(dev):
    ws = [H.Q8Weights(dev, 64, 2048), H.Q8Weights(dev, 64, 1024)]
    outs = [dev.array((4, 64), np.float32) for _ in ws]
    q = dev.array((4, 2048), np.int8)
    s = dev.array((4, 64), np.float32)
    inp = H.ProjInput(xq=q.ptr, xs=s.ptr, mode=H.PROJ_Q)
    with pytest.raises(RuntimeError, match="paired kernel"):
        H.proj_q8_pair(dev, ws, outs, 1, inp, inp, 4)
    with pytest.raises(RuntimeError, match="tokens"):
        H.proj_q8_pair(dev, ws[:1] + ws[:1], outs, 1, inp, inp, 1)
