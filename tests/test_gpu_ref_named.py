"""Reference-named decode kernels (ref_named.hip), launched by name with the reference's parameter lists and grids
(src/kernels/core.hip:259-586, 2621-2650, 3003-3063), against the oracle (oracle.c, pinned against the reference's
own CPU functions) or numpy closed forms:
  norms, RoPE, gated norm          -> or_rmsnorm / or_l2norm / or_rope_neox, numpy; 1e-5 relative
  conv step (+ L2)                 -> numpy causal conv + SiLU; state shift exact
  DeltaNet step (two-loop, d128, d128 + norm) -> or_gdn_step (value-major state; the kernels keep it key-major)
  attention decode / chunked prefill          -> or_attention_head, gated by sigmoid
  elementwise                      -> numpy
Bars: fp32 results within 1e-5 of the magnitude of their terms (sum |term|), as the repository's other fp32 kernels.
"""
import numpy as np
import pytest

import halo_amd as H
import oracle_py as O

pytestmark = pytest.mark.gpu


def close(got, want, mag, rel=1e-5):
    err = np.max(np.abs(got.astype(np.float64) - want.astype(np.float64)) / (np.asarray(mag, np.float64) + 1e-30))
    assert err <= rel, f"error {err:.2e} of the terms' magnitude"


def sig(x):
    return 1.0 / (1.0 + np.exp(-x.astype(np.float64)))


def silu(x):
    return x.astype(np.float64) * sig(x)


def test_norms_rope_elementwise(dev):
    rng = np.random.default_rng(1)
    nv, d = 6, 256
    x = rng.normal(0, 1, (nv, d)).astype(np.float32)
    w = rng.normal(1, 0.1, (nv, d)).astype(np.float32)
    gx, gw, gy = dev.to_device(x), dev.to_device(w), dev.array((nv, d), np.float32)
    for stride in (0, d):
        dev.launch("halo_rmsnorm", (nv,), (256,), [gx, gw, gy, ("u32", d), ("f32", 1e-6), ("u32", stride)])
        want = x.copy()
        for b in range(nv):
            O.oracle().or_rmsnorm(want[b], d, w[b if stride else 0].ctypes.data, 1e-6)
        close(gy.download(), want, np.abs(want) + 1e-3)
    gl = dev.to_device(x)
    dev.launch("halo_l2norm", (nv,), (128,), [gl, ("u32", d), ("f32", 1e-6)])
    want = x.copy()
    for b in range(nv):
        O.oracle().or_l2norm(want[b], d, 1e-6)
    close(gl.download(), want, np.abs(want) + 1e-4)
    # RoPE: plain, rows (2 tokens x 3 heads from pos0 = 40), from step params
    heads, hd, rot = 6, 256, 64
    xr = rng.normal(0, 1, (heads, hd)).astype(np.float32)
    for kind in ("plain", "rows", "p"):
        g = dev.to_device(xr)
        if kind == "plain":
            dev.launch("halo_rope_neox", (heads,), (64,), [g, ("u32", hd), ("u32", rot), ("u32", 77), ("f32", 1e7)])
            poss = [77] * heads
        elif kind == "rows":
            dev.launch("halo_rope_neox_rows", (heads,), (64,),
                       [g, ("u32", hd), ("u32", rot), ("u32", 40), ("u32", 3), ("f32", 1e7)])
            poss = [40, 40, 40, 41, 41, 41]
        else:
            prm = dev.to_device(np.array([5, 12, 9], np.uint32))
            dev.launch("halo_rope_neox_p", (heads,), (64,),
                       [g, prm, ("u32", hd), ("u32", rot), ("u32", 1), ("u32", 3), ("f32", 1e7)])
            poss = [36] * heads
        want = xr.copy()
        for h in range(heads):
            O.oracle().or_rope_neox(want[h], 1, hd, rot, poss[h], 1e7)
        close(g.download(), want, np.abs(xr).max(), 2e-5)
    # elementwise (grid-stride with a grid smaller than the data)
    n = 10000
    a, b = rng.normal(0, 1, n).astype(np.float32), rng.normal(0, 1, n).astype(np.float32)
    cases = [("halo_add", lambda: a + b.astype(np.float64)), ("halo_silu_mul", lambda: silu(a) * b),
             ("halo_sigmoid_gate", lambda: a * sig(b))]
    for name, f in cases:
        ga, gb = dev.to_device(a), dev.to_device(b)
        dev.launch(name, (7,), (256,), [ga, gb, ("u32", n)])
        close(ga.download(), f(), np.abs(f()) + np.abs(a) + 1e-6)
    ga, gb = dev.to_device(a), dev.to_device(b)
    dev.launch("halo_axpy", (7,), (256,), [ga, gb, ("f32", 0.5), ("u32", n)])
    close(ga.download(), a + 0.5 * b.astype(np.float64), np.abs(a) + np.abs(b) + 1e-6)
    gd = dev.array(n, np.float32)
    dev.launch("halo_copy", (3,), (256,), [gd, ga, ("u32", n)])
    assert np.array_equal(gd.download(), ga.download())
    cache = dev.array((8, 300), np.float32).fill(0)
    prm = dev.to_device(np.array([0, 5], np.uint32))
    src = dev.to_device(b[:300])
    dev.launch("halo_copy_at", (2,), (64,), [cache, src, prm, ("u32", 1), ("u32", 300), ("u32", 300)])
    got = cache.download()
    assert np.array_equal(got[5], b[:300]) and not got[np.arange(8) != 5].any()
    # split q | gate
    qg = rng.normal(0, 1, (4, 2 * 256)).astype(np.float32)
    gq, g1, g2 = dev.to_device(qg), dev.array((4, 256), np.float32), dev.array((4, 256), np.float32)
    dev.launch("halo_split_qgate", (4,), (256,), [gq, g1, g2, ("u32", 256)])
    assert np.array_equal(g1.download(), qg[:, :256]) and np.array_equal(g2.download(), qg[:, 256:])


def test_conv_steps(dev):
    rng = np.random.default_rng(2)
    C, K, d = 640, 4, 128
    w = rng.normal(0, 0.5, (C, K)).astype(np.float32)
    st = rng.normal(0, 1, (K - 1, C)).astype(np.float32)
    x = rng.normal(0, 1, C).astype(np.float32)
    conv = w[:, K - 1].astype(np.float64) * x + (w[:, :K - 1].T.astype(np.float64) * st).sum(0)
    y = silu(conv.astype(np.float32))
    shifted = np.concatenate([st[1:], x[None]], 0)
    for name in ("halo_conv_step", "halo_conv_l2norm"):
        gst, gw, gx, go = dev.to_device(st), dev.to_device(w), dev.to_device(x), dev.array(C, np.float32)
        if name == "halo_conv_step":
            dev.launch(name, ((C + 255) // 256,), (256,), [gx, gst, gw, go, ("u32", C), ("u32", K)])
            want = y
        else:  # the first 2 heads (q, k) L2-normalised per 128 channels
            dev.launch(name, (C // d,), (d,), [gx, gst, gw, go, ("u32", C), ("u32", K), ("u32", 2 * d), ("f32", 1e-6)])
            want = y.copy()
            for h in range(2):
                seg = want[h * d:(h + 1) * d]
                want[h * d:(h + 1) * d] = seg / np.sqrt((seg * seg).sum() + 1e-6)
        assert np.array_equal(gst.download(), shifted)
        mag = np.abs(w[:, K - 1] * x) + (np.abs(w[:, :K - 1].T * st)).sum(0) + 1e-3
        close(go.download(), want, mag)


def gdn_inputs(rng, Hv, Hk, d):
    q = rng.normal(0, 1, (Hk, d)).astype(np.float32)
    k = rng.normal(0, 1, (Hk, d)).astype(np.float32)
    q /= np.linalg.norm(q, axis=1, keepdims=True)
    k /= np.linalg.norm(k, axis=1, keepdims=True)
    v = rng.normal(0, 1, (Hv, d)).astype(np.float32)
    al, be = rng.normal(0, 1, Hv).astype(np.float32), rng.normal(0, 1, Hv).astype(np.float32)
    a = -np.exp(rng.normal(0, 0.5, Hv)).astype(np.float32)
    dt = rng.normal(0, 0.5, Hv).astype(np.float32)
    S = rng.normal(0, 0.1, (Hv, d, d)).astype(np.float32)  # key-major [h][i][j]
    return q, k, v, al, be, a, dt, S


def gdn_oracle(q, k, v, al, be, a, dt, S, Hk):
    Hv, d = v.shape
    Sn = np.empty_like(S)
    o = np.empty((Hv, d), np.float32)
    L = O.oracle()
    for h in range(Hv):
        Sv = np.ascontiguousarray(S[h].T)  # value-major
        g = float(a[h]) * L.or_softplus(float(al[h] + dt[h]))
        oh = np.empty(d, np.float32)
        L.or_gdn_step(Sv, d, q[h % Hk].copy(), k[h % Hk].copy(), v[h].copy(), g, L.or_sigmoid(float(be[h])), oh)
        Sn[h] = Sv.T
        o[h] = oh
    return Sn, o


@pytest.mark.parametrize("kernel", ["halo_gdn_step", "halo_gdn_step_d128", "halo_gdn_step_d128_norm"])
def test_gdn_steps(dev, kernel):
    rng = np.random.default_rng(3)
    Hv, Hk, d = 8, 4, 128
    q, k, v, al, be, a, dt, S = gdn_inputs(rng, Hv, Hk, d)
    Sn, o = gdn_oracle(q, k, v, al, be, a, dt, S, Hk)
    gs = dev.to_device(S)
    ins = [dev.to_device(t) for t in (q, k, v, al, be, a, dt)]
    go = dev.array((Hv, d), np.float32)
    if kernel == "halo_gdn_step":
        dev.launch(kernel, (Hv,), (d,), ins + [gs, go, ("u32", Hk), ("u32", d)])
    elif kernel == "halo_gdn_step_d128":
        dev.launch(kernel, (Hv,), (128,), ins + [gs, go, ("u32", Hk)])
    else:
        w = rng.normal(1, 0.1, d).astype(np.float32)
        z = rng.normal(0, 1, (Hv, d)).astype(np.float32)
        dev.launch(kernel, (Hv,), (128,), ins + [gs, dev.to_device(w), dev.to_device(z), go, ("u32", Hk),
                                                 ("f32", 1e-6), ("u32", 1)])
        on = o.astype(np.float64)
        on = on / np.sqrt((on * on).mean(1, keepdims=True) + 1e-6) * w * sig(z)
        o = on.astype(np.float32)
    # magnitudes of the terms: S' = decay S + k delta, delta <= |v| + sum_i |S_ij k_i|; o = sum_i S'_ij q_i
    kk = np.abs(k[np.arange(Hv) % Hk]).astype(np.float64)
    qq = np.abs(q[np.arange(Hv) % Hk]).astype(np.float64)
    dmag = np.abs(v) + np.einsum("hij,hi->hj", np.abs(S).astype(np.float64), kk)
    mag_s = np.abs(S) + kk[:, :, None] * dmag[:, None, :]
    close(gs.download(), Sn, mag_s)
    mag_o = np.einsum("hij,hi->hj", mag_s, qq) / np.sqrt(d)
    if kernel == "halo_gdn_step_d128_norm":  # after the norm: relative to the normalized values, 1e-4
        close(go.download(), o, np.abs(o) + 1e-3, 1e-4)
    else:
        close(go.download(), o, mag_o)


@pytest.mark.parametrize("kernel", ["halo_attention_decode", "halo_attention_prefill"])
def test_attention(dev, kernel):
    rng = np.random.default_rng(4)
    Hq, Hkv, hd, n, T = 8, 2, 256, 300, 3
    max_n = 512
    kc = rng.normal(0, 1, (n, Hkv, hd)).astype(np.float32)
    vc = rng.normal(0, 1, (n, Hkv, hd)).astype(np.float32)
    rows = 1 if kernel == "halo_attention_decode" else T
    q = rng.normal(0, 1, (rows, Hq, hd)).astype(np.float32)
    gate = rng.normal(0, 1, (rows, Hq, hd)).astype(np.float32)
    gk, gv, gq, gg = dev.to_device(kc), dev.to_device(vc), dev.to_device(q), dev.to_device(gate)
    go, sc = dev.array((rows, Hq, hd), np.float32), dev.array((rows, Hq, max_n), np.float32)
    if kernel == "halo_attention_decode":
        dev.launch(kernel, (Hq,), (256,), [gq, gk, gv, gg, go, sc, ("u32", Hq), ("u32", Hkv), ("u32", hd), ("u32", n),
                                           ("u32", max_n)])
        lens = [n]
    else:
        pos0 = n - T
        dev.launch(kernel, (Hq, T), (256,), [gq, gk, gv, gg, go, sc, ("u32", Hq), ("u32", Hkv), ("u32", hd),
                                             ("u32", pos0), ("u32", max_n)])
        lens = [pos0 + t + 1 for t in range(T)]
    got = go.download()
    for t, m in enumerate(lens):
        for h in range(Hq):
            kvh = h // (Hq // Hkv)
            want = np.empty(hd, np.float32)
            O.oracle().or_attention_head(q[t, h].copy(), np.ascontiguousarray(kc[:m, kvh]),
                                         np.ascontiguousarray(vc[:m, kvh]), m, hd, hd, want)
            want = want * sig(gate[t, h])
            close(got[t, h], want, np.abs(vc[:m, kvh]).max(0) + 1e-3)


# ---- reference-named MoE / GEMV kernels (src/kernels/core.hip:2183-2211, 2362-2378, 2436-2458, 2988, 3313,
# 9263-9285, 9401, 9642) -> or_matvec_q8_0_f32x, or_matvec_f32, or_quantize_q8_act, or_route_topk, numpy.
# GEMV bars as the other Q8 GEMVs: 1e-5 of sum |term| + 1e-6; quantizer and top-k ids bit-exact, top-k weights
# bit-exact against halo_router_topk (the same results are the kernel's contract).

def _q8_ref(qs, d, x):
    rows, cols = qs.shape
    y = np.zeros(rows, np.float32)
    O.oracle().or_matvec_q8_0_f32x(np.ascontiguousarray(qs), np.ascontiguousarray(d), rows, cols, cols,
                                   np.ascontiguousarray(x), y, 1)
    mag = np.abs(qs * np.repeat(d.view(np.float16).astype(np.float64), 32, 1)) @ np.abs(x.astype(np.float64))
    return y, mag


def _gemv_close(got, want, mag):
    err = np.abs(got.astype(np.float64) - want.astype(np.float64))
    assert np.all(err <= 1e-5 * mag + 1e-6), f"worst {np.max(err - 1e-5 * mag - 1e-6)}"


@pytest.mark.parametrize("name,rpb", [("halo_gemv_q8r_wide", 8), ("halo_gemv_q8r_r4n", 32)])
def test_q8r_wide_r4n(dev, name, rpb):
    rng = np.random.default_rng(41)
    for rows, cols in ((100, 10240), (1037, 2048), (4, 6144)):
        qs, d = O.synth_q8(rng, rows, cols)
        x = rng.normal(0, 1, cols).astype(np.float32)
        gq, gd, gx, gy = dev.to_device(qs), dev.to_device(d), dev.to_device(x), dev.array((rows,), np.float32)
        dev.launch(name, ((rows + rpb - 1) // rpb,), (256,), [gq, gd, gx, gy, ("u32", rows), ("u32", cols),
                                                              ("u32", cols)])
        _gemv_close(gy.download(), *_q8_ref(qs, d, x))


@pytest.mark.parametrize("r", [1, 4])
def test_expert_gemv_and_down(dev, r):
    rng = np.random.default_rng(42 + r)
    E, rows, cols, slots = 9, 520, 1024, 5
    qs, d = O.synth_q8(rng, E * rows, cols)
    qs3, d3 = qs.reshape(E, rows, cols), d.reshape(E, rows, cols // 32)
    ids = np.array([7, 0, 8, 3, 7], np.uint32)
    h = rng.normal(0, 1, (slots, cols)).astype(np.float32)
    gq, gd, gi, gh = dev.to_device(qs), dev.to_device(d), dev.to_device(ids), dev.to_device(h)
    rpb = 8 * r
    grid = (rows + rpb - 1) // rpb
    suffix = "_r4" if r == 4 else ""
    dims = [("u32", rows), ("u32", cols), ("u32", cols)]
    for slot in range(slots):
        gx, gy = dev.to_device(h[slot]), dev.array((rows,), np.float32)
        dev.launch("halo_gemv_q8r_expert" + suffix, (grid,), (256,), [gq, gd, gi, gx, gy, ("u32", slot)] + dims)
        _gemv_close(gy.download(), *_q8_ref(qs3[ids[slot]], d3[ids[slot]], h[slot]))
    part = dev.array((slots, rows), np.float32)
    dev.launch("halo_moe_down_q8r" + suffix, (grid, slots), (256,), [gq, gd, gi, gh, part] + dims)
    got = part.download()
    for slot in range(slots):
        _gemv_close(got[slot], *_q8_ref(qs3[ids[slot]], d3[ids[slot]], h[slot]))


@pytest.mark.parametrize("name", ["halo_moe_combine", "halo_moe_combine_u"])
def test_moe_combine(dev, name):
    rng = np.random.default_rng(43)
    for slots, n in ((8, 2048), (16, 1000), (1, 77)):
        part = rng.normal(0, 1, (slots, n)).astype(np.float32)
        w = rng.random(slots).astype(np.float32)
        gp, gw, go = dev.to_device(part), dev.to_device(w), dev.array((n,), np.float32)
        dev.launch(name, (4,), (256,), [gp, gw, go, ("u32", slots), ("u32", n)])
        want = (w.astype(np.float64)[:, None] * part).sum(0)
        close(go.download(), want, (np.abs(w.astype(np.float64)[:, None] * part)).sum(0) + 1e-6)


@pytest.mark.parametrize("suffix", ["", "_u"])
def test_matvec_rowblock(dev, suffix):
    rng = np.random.default_rng(44)
    for rows, cols in ((512, 2048), (48, 4096), (3, 1001)):
        wa = rng.normal(0, 1, (rows, cols)).astype(np.float32)
        wb = rng.normal(0, 1, (rows, cols)).astype(np.float32)
        x = rng.normal(0, 1, cols).astype(np.float32)
        gwa, gwb, gx = dev.to_device(wa), dev.to_device(wb), dev.to_device(x)
        ya, yb = dev.array((rows,), np.float32), dev.array((rows,), np.float32)
        dev.launch("halo_matvec_f32_rowblock" + suffix, (rows,), (256,), [gwa, gx, ya, ("u32", rows), ("u32", cols)])
        want = np.zeros(rows, np.float32)
        O.oracle().or_matvec_f32(wa, rows, cols, x, want)
        mag = np.abs(wa.astype(np.float64)) @ np.abs(x.astype(np.float64))
        close(ya.download(), want, mag)
        dev.launch("halo_matvec_f32_rowblock2" + suffix, (2 * rows,), (256,),
                   [gwa, gwb, gx, ya, yb, ("u32", rows), ("u32", cols)])
        close(ya.download(), want, mag)
        O.oracle().or_matvec_f32(wb, rows, cols, x, want)
        close(yb.download(), want, np.abs(wb.astype(np.float64)) @ np.abs(x.astype(np.float64)))


def test_quantize_kblocked_bit_exact(dev):
    rng = np.random.default_rng(45)
    T, cols = 5, 2048
    x = rng.normal(0, 1, (T, cols)).astype(np.float32)
    x[1, 64:96] = 0.0  # an all-zero block: scale 0, q 0
    gx, gq, gd = dev.to_device(x), dev.array((cols // 64, T, 64), np.int8), dev.array((cols // 32, T), np.float32)
    dev.launch("halo_quantize_q8_kblocked", (T,), (256,), [gx, gq, gd, ("u32", cols), ("u32", T)])
    wq, wd = np.zeros((T, cols), np.int8), np.zeros((T, cols // 32), np.float32)
    for t in range(T):
        O.oracle().or_quantize_q8_act(x[t], wq[t], wd[t], cols)
    assert np.array_equal(gq.download(), wq.reshape(T, cols // 64, 64).transpose(1, 0, 2))
    assert gd.download().tobytes() == np.ascontiguousarray(wd.T).tobytes()


@pytest.mark.parametrize("T,cols", [(1, 512), (13, 512), (21, 2048), (8, 96)])
def test_quantize_rows8_bit_exact(dev, T, cols):
    """halo_quantize_q8_rows8 (8 rows per block, ragged last block) against the oracle's quantizer and bytewise
    against the one-row halo_quantize_q8_rows."""
    rng = np.random.default_rng(T * cols)
    x = rng.normal(0, 1, (T, cols)).astype(np.float32)
    x[T // 2, :32] = 0.0  # an all-zero block: scale 0, q 0
    gx = dev.to_device(x)
    outs = []
    for name, grid, extra in (("halo_quantize_q8_rows8", ((T + 7) // 8,), [("u32", T)]),
                              ("halo_quantize_q8_rows", (T,), [])):
        gq, gd = dev.array((T, cols), np.int8), dev.array((T, cols // 32), np.float32)
        dev.launch(name, grid, (256,), [gx, gq, gd, ("u32", cols)] + extra)
        outs.append((gq.download(), gd.download()))
    wq, wd = np.zeros((T, cols), np.int8), np.zeros((T, cols // 32), np.float32)
    for t in range(T):
        O.oracle().or_quantize_q8_act(x[t], wq[t], wd[t], cols)
    assert np.array_equal(outs[0][0], wq) and outs[0][1].tobytes() == wd.tobytes()
    assert np.array_equal(outs[0][0], outs[1][0]) and outs[0][1].tobytes() == outs[1][1].tobytes()


def test_router_topk_w(dev):
    rng = np.random.default_rng(46)
    for n, k in ((512, 10), (256, 8), (1024, 16), (64, 1)):
        logits = rng.normal(0, 2, n).astype(np.float32)
        logits[5] = logits[9]  # a tie: the lower index ranks first
        gl = dev.to_device(logits)
        outs = []
        for name, block in (("halo_router_topk_w", 256), ("halo_router_topk", 64)):
            gi, gw = dev.array((k,), np.uint32), dev.array((k,), np.float32)
            dev.launch(name, (1,), (block,), [gl, gi, gw, ("u32", n), ("u32", k)])
            outs.append((gi.download(), gw.download()))
        wi, ww = np.zeros(k, np.uint32), np.zeros(k, np.float32)
        O.oracle().or_route_topk(logits, n, k, wi, ww)
        assert np.array_equal(outs[0][0], wi) and outs[0][1].tobytes() == outs[1][1].tobytes()
        np.testing.assert_allclose(outs[0][1], ww, rtol=1e-5)


# ---- select attention, DeltaNet prefill helpers, shared expert, router with activation record ------------------
# (core.hip:783-918, 3480-3662, 9196-9343, 9418-9446, 9590-9636.) Chunked kernels are checked bit for bit against
# stepping with the decode kernels (the reference's contract for them); the rest against the oracle as above.

@pytest.mark.parametrize("kernel", ["halo_attention_select", "halo_attention_select_b", "halo_attention_select_rows"])
def test_attention_select(dev, kernel):
    rng = np.random.default_rng(47)
    Hq, Hkv, hd, npos, max_n = 8, 2, 256, 400, 256
    kc = rng.normal(0, 1, (npos, Hkv, hd)).astype(np.float32)
    vc = rng.normal(0, 1, (npos, Hkv, hd)).astype(np.float32)
    T = 2 if kernel.endswith("rows") else 1
    ns = [150, 1][:T] if T == 2 else [203]
    vis = np.zeros((T, max_n), np.uint32)
    params = np.zeros((T, 16), np.uint32)
    for t, n in enumerate(ns):
        vis[t, :n] = rng.choice(npos, n, replace=False)
        params[t, 5] = n
    q = rng.normal(0, 1, (T, Hq, hd)).astype(np.float32)
    gate = rng.normal(0, 1, (T, Hq, hd)).astype(np.float32)
    go, sc = dev.array((T, Hq, hd), np.float32), dev.array((T, Hq, max_n), np.float32)
    args = [dev.to_device(q), dev.to_device(kc), dev.to_device(vc), dev.to_device(gate), dev.to_device(vis), go, sc,
            dev.to_device(params), ("u32", Hq), ("u32", Hkv), ("u32", hd), ("u32", max_n)]
    dev.launch(kernel, (Hq, T) if T > 1 else (Hq,), (256,), args)
    got = go.download()
    for t, n in enumerate(ns):
        for h in range(Hq):
            kvh = h // (Hq // Hkv)
            rows = vis[t, :n].astype(np.int64)
            want = np.empty(hd, np.float32)
            O.oracle().or_attention_head(q[t, h].copy(), np.ascontiguousarray(kc[rows, kvh]),
                                         np.ascontiguousarray(vc[rows, kvh]), n, hd, hd, want)
            want = want * sig(gate[t, h])
            close(got[t, h], want, np.abs(vc[rows, kvh]).max(0) + 1e-3)


def test_gdn_step_norm_r_and_prefill_equal_stepping(dev):
    """T single steps of halo_gdn_step_d128_norm against one chunked halo_gdn_prefill_d128_norm launch over padded
    rows (per-head a and dt shared by the chunk), and the _r name against the first step: bit for bit."""
    rng = np.random.default_rng(48)
    Hv, Hk, d, T = 8, 4, 128, 5
    w = rng.normal(1, 0.1, d).astype(np.float32)
    toks = [gdn_inputs(rng, Hv, Hk, d) for _ in range(T)]
    S0, a, dt = toks[0][7], toks[0][5], toks[0][6]
    z = rng.normal(0, 1, (T, Hv, d)).astype(np.float32)
    gw, ga, gdt = dev.to_device(w), dev.to_device(a), dev.to_device(dt)
    tail = lambda t, gs, go: [gs, gw, dev.to_device(z[t]), go, ("u32", Hk), ("f32", 1e-6), ("u32", 0)]
    gs, outs = dev.to_device(S0), []
    for t in range(T):
        ins = [dev.to_device(x) for x in toks[t][:5]] + [ga, gdt]
        if t == 0:
            gs_r, go_r = dev.to_device(S0), dev.array((Hv, d), np.float32)
            dev.launch("halo_gdn_step_d128_norm_r", (Hv,), (128,), ins + tail(t, gs_r, go_r))
        go = dev.array((Hv, d), np.float32)
        dev.launch("halo_gdn_step_d128_norm", (Hv,), (128,), ins + tail(t, gs, go))
        outs.append(go.download())
        if t == 0:
            assert go_r.download().tobytes() == outs[0].tobytes()
            assert gs_r.download().tobytes() == gs.download().tobytes()
    # rows padded: q, k rows Hk d + 64 apart, v rows Hv d + 32, z and out rows Hv d + 128
    qs_, vs_, zs_ = Hk * d + 64, Hv * d + 32, Hv * d + 128
    qb, kb = np.zeros((T, qs_), np.float32), np.zeros((T, qs_), np.float32)
    vb, zb = np.zeros((T, vs_), np.float32), np.zeros((T, zs_), np.float32)
    al, be = np.stack([x[3] for x in toks]), np.stack([x[4] for x in toks])
    for t in range(T):
        qb[t, :Hk * d], kb[t, :Hk * d] = toks[t][0].ravel(), toks[t][1].ravel()
        vb[t, :Hv * d], zb[t, :Hv * d] = toks[t][2].ravel(), z[t].ravel()
    gs2, gout = dev.to_device(S0), dev.array((T, zs_), np.float32)
    dev.launch("halo_gdn_prefill_d128_norm", (Hv,), (128,),
               [dev.to_device(qb), dev.to_device(kb), dev.to_device(vb), dev.to_device(al), dev.to_device(be), ga,
                gdt, gs2, gw, dev.to_device(zb), gout, ("u32", Hk), ("f32", 1e-6), ("u32", 0), ("u32", T),
                ("u32", qs_), ("u32", vs_), ("u32", zs_)])
    got = gout.download()
    for t in range(T):
        assert got[t, :Hv * d].tobytes() == outs[t].ravel().tobytes(), f"token {t}"
    assert gs2.download().tobytes() == gs.download().tobytes()


@pytest.mark.parametrize("T", [6, 2])
def test_conv_prefill_and_state_advance_equal_stepping(dev, T):
    rng = np.random.default_rng(49 + T)
    C, K, d, l2 = 640, 4, 128, 256
    w = rng.normal(0, 0.5, (C, K)).astype(np.float32)
    st = rng.normal(0, 1, (K - 1, C)).astype(np.float32)
    x = rng.normal(0, 1, (T, C)).astype(np.float32)
    gw, gst = dev.to_device(w), dev.to_device(st)
    want = []
    for t in range(T):
        go = dev.array(C, np.float32)
        dev.launch("halo_conv_l2norm", (C // d,), (d,), [dev.to_device(x[t]), gst, gw, go, ("u32", C), ("u32", K),
                                                           ("u32", l2), ("f32", 1e-6)])
        want.append(go.download())
    gst2, gx, gout = dev.to_device(st), dev.to_device(x), dev.array((T, C), np.float32)
    dev.launch("halo_conv_l2norm_prefill", (C // d, T), (d,), [gx, gst2, gw, gout, ("u32", C), ("u32", K),
                                                                ("u32", l2), ("f32", 1e-6)])
    assert gout.download().tobytes() == np.stack(want).tobytes()
    dev.launch("halo_conv_state_advance", ((C + 255) // 256,), (256,), [gx, gst2, ("u32", C), ("u32", K), ("u32", T)])
    assert gst2.download().tobytes() == gst.download().tobytes()


@pytest.mark.parametrize("suffix", ["", "_u"])
def test_shared_expert(dev, suffix):
    rng = np.random.default_rng(50)
    H, F, slots = 2048, 512, 10
    gq, gd = O.synth_q8(rng, F, H)
    uq, ud = O.synth_q8(rng, F, H)
    dq, dd = O.synth_q8(rng, H, F)
    gate_inp = rng.normal(0, 0.02, H).astype(np.float32)
    x = rng.normal(0, 1, H).astype(np.float32)
    h, sg = dev.array((F,), np.float32), dev.array((1,), np.float32)
    dev.launch("halo_shexp_gate_up" + suffix, ((F + 15) // 16,), (256,),
               [dev.to_device(gq), dev.to_device(gd), dev.to_device(uq), dev.to_device(ud), dev.to_device(gate_inp),
                dev.to_device(x), h, sg, ("u32", F), ("u32", H), ("u32", H)])
    g, gm = _q8_ref(gq, gd, x)
    u, um = _q8_ref(uq, ud, x)
    hw = silu(g) * u
    got_h = h.download()
    close(got_h, hw, np.abs(silu(g)) * um + np.abs(u) * gm + 1e-6)
    close(sg.download(), np.array([gate_inp.astype(np.float64) @ x]), np.array([np.abs(gate_inp) @ np.abs(x)]))
    part = rng.normal(0, 1, (slots, H)).astype(np.float32)
    wts = rng.random(slots).astype(np.float32)
    out = dev.array((H,), np.float32)
    dev.launch("halo_shexp_down_combine" + suffix, ((H + 31) // 32,), (256,),
               [dev.to_device(dq), dev.to_device(dd), h, sg, dev.to_device(part), dev.to_device(wts), ("u32", slots),
                out, ("u32", H), ("u32", F), ("u32", F)])
    y, ym = _q8_ref(dq, dd, got_h)
    s = sig(sg.download()[0])
    want = (wts.astype(np.float64)[:, None] * part).sum(0) + s * y
    close(out.download(), want, (np.abs(wts[:, None] * part)).sum(0) + s * ym + 1e-6)


def test_router_rowblock_q8act(dev):
    rng = np.random.default_rng(51)
    E, H = 512, 2048
    w = rng.normal(0, 0.02, (E, H)).astype(np.float32)
    x = rng.normal(0, 1, H).astype(np.float32)
    x[64:96] = 0.0
    y, act = dev.array((E,), np.float32), dev.array((1024 + 256,), np.uint32)
    dev.launch("halo_router_rowblock_q8act", (max(E, H // 32),), (256,),
               [dev.to_device(w), dev.to_device(x), y, ("u32", E), ("u32", H), act])
    want = np.zeros(E, np.float32)
    O.oracle().or_matvec_f32(w, E, H, x, want)
    close(y.download(), want, np.abs(w.astype(np.float64)) @ np.abs(x.astype(np.float64)))
    a = act.download()
    wq, ws = np.zeros(H, np.int8), np.zeros(H // 32, np.float32)
    O.oracle().or_quantize_q8_act(x, wq, ws, H)
    assert np.array_equal(a[:H // 4].view(np.int8), wq)
    assert a[1024:1024 + H // 32].view(np.float32).tobytes() == ws.tobytes()
    sums = a[1152:1152 + H // 32].view(np.float32)
    blocks = x.reshape(-1, 32).astype(np.float64)
    close(sums, blocks.sum(1), np.abs(blocks).sum(1) + 1e-6, 1e-6)


# ---- reference-named prefill int8 GEMMs (core.hip:3103-3153, 3303-3311, 3466-3476) -> or_gemv_q8a8 per token,
# the bar of the other Q8 GEMMs (1e-5 of sum |term| + 1e-6). Shapes with ragged row and token tiles.
@pytest.mark.parametrize("name,block,bm,bn,kblocked", [
    ("halo_gemm_q8r_wmma", 128, 64, 64, False), ("halo_gemm_q8r_wmma_t", 256, 128, 128, False),
    ("halo_gemm_q8a8_128x128", 256, 128, 128, True), ("halo_gemm_q8a8_128x64", 256, 128, 64, True),
    ("halo_gemm_q8a8_320x64", 256, 320, 64, True), ("halo_gemm_q8a8_160x64", 256, 160, 64, True),
    ("halo_gemm_q8a8_256x128", 256, 256, 128, True)])
def test_reference_prefill_gemms(dev, name, block, bm, bn, kblocked):
    rng = np.random.default_rng(52)
    rows, cols, T = 700, 1024, 200
    qs, d = O.synth_q8(rng, rows, cols)
    x = rng.normal(0, 1, (T, cols)).astype(np.float32)
    xq, xs = np.zeros((T, cols), np.int8), np.zeros((T, cols // 32), np.float32)
    for t in range(T):
        O.oracle().or_quantize_q8_act(x[t], xq[t], xs[t], cols)
    want, mag = O.gemv_q8a8(qs, d, xq, xs)
    if kblocked:
        gxq = dev.to_device(np.ascontiguousarray(xq.reshape(T, cols // 64, 64).transpose(1, 0, 2)))
        gxs = dev.to_device(np.ascontiguousarray(xs.T))
    else:
        gxq, gxs = dev.to_device(xq), dev.to_device(xs)
    gy = dev.array((T, rows), np.float32)
    dev.launch(name, ((T + bn - 1) // bn, (rows + bm - 1) // bm), (block,),
               [dev.to_device(qs), dev.to_device(d), gxq, gxs, gy, ("u32", rows), ("u32", cols), ("u32", cols),
                ("u32", T)])
    got = gy.download()
    err = np.abs(got.astype(np.float64) - want.astype(np.float64))
    assert np.all(err <= 1e-5 * mag + 1e-6), f"worst {np.max(err - 1e-5 * mag - 1e-6)}"


@pytest.mark.parametrize("B", [1, 4, 8])
def test_moe_bucket_and_grouped_down(dev, B):
    """halo_moe_bucket_b (distinct experts over B columns' top-k, in first-appearance order, pairs in order; exact)
    and halo_moe_down_q8r_r4_b{B} (every pair's down projection by its expert) against numpy and the oracle GEMV
    (batch_decode.hip:415-446, 646-697)."""
    rng = np.random.default_rng(53 + B)
    E, k, H, F = 24, 10, 512, 256
    ids = np.concatenate([rng.choice(E, k, replace=False) for _ in range(B)]).astype(np.uint32)
    n = B * k
    gids = dev.to_device(ids)
    ucount, uexp = dev.array((1,), np.uint32), dev.array((n,), np.uint32)
    unum, upair = dev.array((n,), np.uint32), dev.array((n * 8,), np.uint32)
    dev.launch("halo_moe_bucket_b", (1,), (128,), [gids, ("u32", n), ucount, uexp, unum, upair])
    order = list(dict.fromkeys(ids.tolist()))
    U = int(ucount.download()[0])
    assert U == len(order)
    assert uexp.download()[:U].tolist() == order
    got_num, got_pair = unum.download(), upair.download()
    for u, e in enumerate(order):
        pairs = [p for p in range(n) if ids[p] == e]
        assert got_num[u] == len(pairs) and got_pair[u * 8:u * 8 + len(pairs)].tolist() == pairs
    qs, d = O.synth_q8(rng, E * H, F)
    h = rng.normal(0, 1, (n, F)).astype(np.float32)
    part = dev.array((n, H), np.float32)
    dev.launch(f"halo_moe_down_q8r_r4_b{B}", ((H + 31) // 32, n), (256,),
               [dev.to_device(qs), dev.to_device(d), ucount, uexp, unum, upair, dev.to_device(h), part, ("u32", H),
                ("u32", F), ("u32", F)])
    got = part.download()
    for p in range(n):
        e = int(ids[p])
        _gemv_close(got[p], *_q8_ref(qs[e * H:(e + 1) * H], d[e * H:(e + 1) * H], h[p]))


@pytest.mark.parametrize("T", [1, 300])
def test_moe_prefill_buckets(dev, T):
    """halo_moe_bucket and the three-pass halo_moe_bucket_count / _scan / _scatter (core.hip:4725-4864): pairs
    grouped by expert in pair order (a stable sort), each pair's position, 64-pair tiles in expert order; exact."""
    rng = np.random.default_rng(54 + T)
    E, k = 512, 10
    ids = np.concatenate([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.uint32)
    P = ids.size
    order = np.argsort(ids, kind="stable").astype(np.uint32)
    pos = np.empty(P, np.uint32)
    pos[order] = np.arange(P, dtype=np.uint32)
    counts = np.bincount(ids, minlength=E)
    want_tiles, off = [], 0
    for e in range(E):
        for i in range(0, counts[e], 64):
            want_tiles.append((e, off + i, min(64, counts[e] - i)))
        off += counts[e]
    gids = dev.to_device(ids)
    maxt = P // 64 + E + 1
    # one block
    s1, p1, t1, n1 = (dev.array((P,), np.uint32), dev.array((P,), np.uint32), dev.array((3 * maxt,), np.uint32),
                      dev.array((1,), np.uint32))
    dev.launch("halo_moe_bucket", (1,), (1024,), [gids, ("u32", P), ("u32", E), s1, p1, t1, n1])
    # three passes
    chunks = (P + 1023) // 1024
    cnt = dev.array((chunks, E), np.uint32)
    s2, p2, t2, n2, base = (dev.array((P,), np.uint32), dev.array((P,), np.uint32),
                            dev.array((3 * maxt,), np.uint32), dev.array((1,), np.uint32), dev.array((E,), np.uint32))
    dev.launch("halo_moe_bucket_count", (chunks,), (1024,), [gids, ("u32", P), ("u32", E), cnt])
    dev.launch("halo_moe_bucket_scan", (1,), (1024,), [cnt, ("u32", chunks), ("u32", E), t2, n2, base])
    dev.launch("halo_moe_bucket_scatter", (chunks,), (1024,), [gids, ("u32", P), ("u32", E), cnt, base, s2, p2])
    for s, p, t, n in ((s1, p1, t1, n1), (s2, p2, t2, n2)):
        assert int(n.download()[0]) == len(want_tiles)
        assert np.array_equal(s.download(), order) and np.array_equal(p.download(), pos)
        assert t.download()[:3 * len(want_tiles)].reshape(-1, 3).tolist() == [list(x) for x in want_tiles]
    assert np.array_equal(base.download(), np.concatenate([[0], np.cumsum(counts)[:-1]]).astype(np.uint32))


def _rms(x, w, eps):
    x64 = x.astype(np.float64)
    return x64 / np.sqrt((x64 * x64).mean(-1, keepdims=True) + eps) * w


def _rope(v, rot, pos, theta):
    """NEOX rotation of the first rot values of each row of v (float64) at positions pos (per row)."""
    out = v.copy()
    half = rot // 2
    i = np.arange(half)
    ang = np.asarray(pos, np.float64)[:, None] * theta ** (-2.0 * i / rot)
    a, b = v[:, :half], v[:, half:rot]
    out[:, :half] = a * np.cos(ang) - b * np.sin(ang)
    out[:, half:rot] = a * np.sin(ang) + b * np.cos(ang)
    return out


def test_norm_rope_and_batched_glue(dev):
    """halo_split_qgate_norm_rope, halo_norm_rope_rows (+ cache row), halo_rope_neox_blocks, halo_rmsnorm_rows and the
    batched-column _y kernels against numpy (core.hip:308-440, 4045; batch_decode.hip:1680-1705); norms at 1e-5 of
    each value, rotations at 5e-5 of the rows' largest value (fp32 angles at positions up to 900)."""
    rng = np.random.default_rng(55)
    T, heads, hd, rot, theta, eps, pos0 = 3, 4, 256, 64, 1e7, 1e-6, 40
    qg = rng.normal(0, 1, (T * heads, 2 * hd)).astype(np.float32)
    w = rng.normal(1, 0.1, hd).astype(np.float32)
    gq, gg = dev.array((T * heads, hd), np.float32), dev.array((T * heads, hd), np.float32)
    dev.launch("halo_split_qgate_norm_rope", (T * heads,), (hd,),
               [dev.to_device(qg), gq, gg, dev.to_device(w), ("f32", eps), ("u32", rot), ("u32", pos0),
                ("u32", heads), ("f32", theta)])
    pos = pos0 + np.arange(T * heads) // heads
    want = _rope(_rms(qg[:, :hd], w, eps), rot, pos, theta)
    close(gq.download(), want, np.abs(want).max(), 5e-5)
    assert np.array_equal(gg.download(), qg[:, hd:])
    # norm + rope rows with the cache copy (d = 256)
    x = rng.normal(0, 1, (T * heads, hd)).astype(np.float32)
    gx, gc = dev.to_device(x), dev.array((T * heads, hd), np.float32)
    dev.launch("halo_norm_rope_rows", (T * heads,), (256,),
               [gx, dev.to_device(w), ("f32", eps), ("u32", hd), ("u32", rot), ("u32", pos0), ("u32", heads),
                ("f32", theta), gc])
    want = _rope(_rms(x, w, eps), rot, pos, theta)
    close(gx.download(), want, np.abs(want).max(), 5e-5)
    assert gc.download().tobytes() == gx.download().tobytes()
    # pooled blocks at (b0 + b) * ratio
    xb = rng.normal(0, 1, (5, hd)).astype(np.float32)
    gb = dev.to_device(xb)
    dev.launch("halo_rope_neox_blocks", (5,), (64,), [gb, ("u32", hd), ("u32", rot), ("u32", 3), ("u32", 16),
                                                      ("f32", theta)])
    want = _rope(xb.astype(np.float64), rot, (3 + np.arange(5)) * 16, theta)
    close(gb.download(), want, np.abs(want).max(), 5e-5)
    # rmsnorm rows with gammas repeating every 2 vectors
    xr = rng.normal(0, 1, (6, 128)).astype(np.float32)
    wr = rng.normal(1, 0.1, (2, 130)).astype(np.float32)
    gy = dev.array((6, 128), np.float32)
    dev.launch("halo_rmsnorm_rows", (6,), (128,), [dev.to_device(xr), dev.to_device(wr), gy, ("u32", 128),
                                                   ("f32", eps), ("u32", 130), ("u32", 2)])
    want = _rms(xr, wr[np.arange(6) % 2, :128], eps)
    close(gy.download(), want, np.abs(want) + 1e-3)
    # batched columns: B = 2 entries, data `stride` floats apart
    B, stride, pstride = 2, heads * 2 * hd + 64, 16
    qgb = rng.normal(0, 1, (B, stride)).astype(np.float32)
    q_stride = heads * hd + 32
    gqb, ggb = dev.array((B, q_stride), np.float32), dev.array((B, q_stride), np.float32)
    dev.launch("halo_split_qgate_y", (heads, B), (256,), [dev.to_device(qgb), gqb, ggb, ("u32", hd), ("u32", stride),
                                                          ("u32", q_stride)])
    for e in range(B):
        v = qgb[e, :heads * 2 * hd].reshape(heads, 2, hd)
        assert np.array_equal(gqb.download()[e, :heads * hd], v[:, 0].ravel())
        assert np.array_equal(ggb.download()[e, :heads * hd], v[:, 1].ravel())
    wn = rng.normal(1, 0.1, (heads, hd)).astype(np.float32)
    xy = rng.normal(0, 1, (B, q_stride)).astype(np.float32)
    gxy = dev.to_device(xy)
    dev.launch("halo_rmsnorm_y", (heads, B), (256,), [gxy, dev.to_device(wn), ("u32", hd), ("f32", eps), ("u32", hd),
                                                      ("u32", q_stride)])
    got = gxy.download()
    for e in range(B):
        want = _rms(xy[e, :heads * hd].reshape(heads, hd), wn, eps)
        close(got[e, :heads * hd].reshape(heads, hd), want, np.abs(want) + 1e-3)
    params = np.zeros((B, pstride), np.uint32)
    params[:, 1] = [17, 900]
    gxr = dev.to_device(xy)
    dev.launch("halo_rope_neox_p_y", (heads, B), (64,), [gxr, dev.to_device(params), ("u32", hd), ("u32", rot),
                                                         ("u32", 1), ("u32", 1), ("f32", theta), ("u32", q_stride),
                                                         ("u32", pstride)])
    got = gxr.download()
    for e in range(B):
        want = _rope(xy[e, :heads * hd].reshape(heads, hd).astype(np.float64), rot, [params[e, 1]] * heads, theta)
        close(got[e, :heads * hd].reshape(heads, hd), want, np.abs(want).max(), 5e-5)
    # copy_at_y: each entry's cache through a pointer table
    caches = [dev.array((50, 300), np.float32).fill(0) for _ in range(B)]
    tab = np.zeros((B, 3), np.uint64)
    for e in range(B):
        tab[e, 2] = caches[e].ptr
    src = rng.normal(0, 1, (B, 320)).astype(np.float32)
    params[:, 2] = [4, 33]
    dev.launch("halo_copy_at_y", (2, B), (256,), [dev.to_device(tab), ("u32", 3), ("u32", 2), dev.to_device(src),
                                                  dev.to_device(params), ("u32", 2), ("u32", 300), ("u32", 300),
                                                  ("u32", 320), ("u32", pstride)])
    for e in range(B):
        c = caches[e].download()
        assert np.array_equal(c[params[e, 2]], src[e, :300]) and np.count_nonzero(c) == np.count_nonzero(src[e, :300])


def test_small_elementwise(dev):
    rng = np.random.default_rng(56)
    n, T = 1000, 3
    y = rng.normal(0, 1, (T, n)).astype(np.float32)
    x = rng.normal(0, 1, (T, n)).astype(np.float32)
    g = rng.normal(0, 1, T).astype(np.float32)
    wts = rng.random(4).astype(np.float32)
    gy = dev.to_device(y[0])
    dev.launch("halo_axpy_slot", (2,), (256,), [gy, dev.to_device(x[0]), dev.to_device(wts), ("u32", 2), ("u32", n)])
    close(gy.download(), y[0] + wts[2].astype(np.float64) * x[0], np.abs(y[0]) + np.abs(x[0]))
    gy = dev.to_device(y[0])
    dev.launch("halo_axpy_sigmoid", (2,), (256,), [gy, dev.to_device(x[0]), dev.to_device(g), ("u32", n)])
    close(gy.download(), y[0] + sig(g[0]) * x[0], np.abs(y[0]) + np.abs(x[0]))
    gy = dev.to_device(y)
    dev.launch("halo_axpy_sigmoid_rows", (4,), (256,), [gy, dev.to_device(x), dev.to_device(g), ("u32", n),
                                                        ("u32", T)])
    close(gy.download(), y + sig(g)[:, None] * x, np.abs(y) + np.abs(x))
    gx = dev.to_device(x[0])
    dev.launch("halo_scale_silu", (2,), (256,), [gx, ("f32", 0.25), ("u32", n)])
    close(gx.download(), silu((x[0] * np.float32(0.25)).astype(np.float32)), np.abs(x[0]) + 1e-3)


@pytest.mark.parametrize("name,cols", [("halo_gemm_f32_tiled", 2048), ("halo_gemm_f32_tiled", 1040),
                                       ("halo_gemm_f32_rows", 2048), ("halo_gemm_f32_narrow", 96),
                                       ("halo_gemm_f32_narrow", 1001), ("halo_gemm_f32_skinny", 2048),
                                       ("halo_gemm_f32_skinny", 1001)])
def test_f32_gemms(dev, name, cols):
    """The fp32 prefill GEMMs (core.hip:3767-3800, 5605-5680, 8975-9000) against a float64 product; 1e-5 of
    sum |term|. Ragged rows and tokens; a trailing half stage for the tiled GEMM (cols % 32 == 16), unaligned rows
    (cols 1001) for the narrow and skinny ones."""
    rng = np.random.default_rng(57)
    T = 70
    rows = 13 if name == "halo_gemm_f32_skinny" else 130
    w = rng.normal(0, 0.02, (rows, cols)).astype(np.float32)
    x = rng.normal(0, 1, (T, cols)).astype(np.float32)
    gy = dev.array((T, rows), np.float32)
    args = [dev.to_device(w), dev.to_device(x), gy, ("u32", rows), ("u32", cols)]
    if name == "halo_gemm_f32_tiled":
        dev.launch(name, ((T + 63) // 64, (rows + 63) // 64), (256,), args + [("u32", T)])
    elif name == "halo_gemm_f32_rows":
        dev.launch(name, ((rows + 7) // 8, T), (256,), args)
    elif name == "halo_gemm_f32_narrow":
        dev.launch(name, ((rows + 255) // 256, T), (256,), args)
    else:
        dev.launch(name, ((T + 7) // 8,), (256,), args + [("u32", T)])
    want = x.astype(np.float64) @ w.astype(np.float64).T
    close(gy.download(), want, np.abs(x.astype(np.float64)) @ np.abs(w.astype(np.float64)).T)


def test_shexp_down_add_and_topk_y(dev):
    rng = np.random.default_rng(58)
    H, F = 2048, 512
    dq, dd = O.synth_q8(rng, H, F)
    h = rng.normal(0, 1, F).astype(np.float32)
    out0 = rng.normal(0, 1, H).astype(np.float32)
    sg = np.array([0.3], np.float32)
    go = dev.to_device(out0)
    dev.launch("halo_shexp_down_add", ((H + 31) // 32,), (256,),
               [dev.to_device(dq), dev.to_device(dd), dev.to_device(h), dev.to_device(sg), go, ("u32", H), ("u32", F),
                ("u32", F)])
    y, ym = _q8_ref(dq, dd, h)
    close(go.download(), out0 + sig(sg[0]) * y, np.abs(out0) + sig(sg[0]) * ym + 1e-6)
    B, n, k, lstride = 3, 512, 10, 600
    logits = rng.normal(0, 2, (B, lstride)).astype(np.float32)
    gi, gw = dev.array((B, k), np.uint32), dev.array((B, k), np.float32)
    dev.launch("halo_router_topk_w_y", (1, B), (256,), [dev.to_device(logits), gi, gw, ("u32", n), ("u32", k),
                                                        ("u32", lstride)])
    for b in range(B):
        wi, ww = np.zeros(k, np.uint32), np.zeros(k, np.float32)
        O.oracle().or_route_topk(np.ascontiguousarray(logits[b, :n]), n, k, wi, ww)
        assert np.array_equal(gi.download()[b], wi)
        np.testing.assert_allclose(gw.download()[b], ww, rtol=1e-5)


def test_batched_select_and_conv_through_tables(dev):
    """halo_attention_select_b_y and halo_conv_l2norm_y (batch_decode.hip:1727-1748): each column through its own
    cache / state pointer equals the single-column kernel on that column, bit for bit."""
    rng = np.random.default_rng(59)
    B, Hq, Hkv, hd, npos, max_n = 2, 8, 2, 256, 120, 128
    qs_ = Hq * hd + 64
    caches = [(dev.to_device(rng.normal(0, 1, (npos, Hkv, hd)).astype(np.float32)),
               dev.to_device(rng.normal(0, 1, (npos, Hkv, hd)).astype(np.float32))) for _ in range(B)]
    tab = np.zeros((B, 4), np.uint64)
    for e in range(B):
        tab[e, 1], tab[e, 2] = caches[e][0].ptr, caches[e][1].ptr
    q = rng.normal(0, 1, (B, qs_)).astype(np.float32)
    gate = rng.normal(0, 1, (B, qs_)).astype(np.float32)
    vis = np.zeros((B, max_n), np.uint32)
    params = np.zeros((B, 16), np.uint32)
    for e, n in enumerate((77, 120)):
        vis[e, :n] = rng.choice(npos, n, replace=False)
        params[e, 5] = n
    out, sc = dev.array((B, qs_), np.float32), dev.array((B, Hq * max_n), np.float32)
    dev.launch("halo_attention_select_b_y", (Hq, B), (256,),
               [dev.to_device(q), dev.to_device(tab), ("u32", 4), ("u32", 1), dev.to_device(gate), dev.to_device(vis),
                out, sc, dev.to_device(params), ("u32", Hq), ("u32", Hkv), ("u32", hd), ("u32", max_n),
                ("u32", qs_), ("u32", max_n), ("u32", Hq * max_n), ("u32", 16)])
    got = out.download()
    for e in range(B):
        o1, s1 = dev.array((Hq, hd), np.float32), dev.array((Hq, max_n), np.float32)
        dev.launch("halo_attention_select_b", (Hq,), (256,),
                   [dev.to_device(q[e, :Hq * hd]), caches[e][0], caches[e][1], dev.to_device(gate[e, :Hq * hd]),
                    dev.to_device(vis[e]), o1, s1, dev.to_device(params[e]), ("u32", Hq), ("u32", Hkv), ("u32", hd),
                    ("u32", max_n)])
        assert got[e, :Hq * hd].tobytes() == o1.download().tobytes()
    C, K, d = 512, 4, 128
    w = rng.normal(0, 0.5, (C, K)).astype(np.float32)
    st = [rng.normal(0, 1, (K - 1, C)).astype(np.float32) for _ in range(B)]
    x = rng.normal(0, 1, (B, C + 32)).astype(np.float32)
    gst = [dev.to_device(s) for s in st]
    tab = np.zeros((B, 2), np.uint64)
    for e in range(B):
        tab[e, 1] = gst[e].ptr
    go = dev.array((B, C + 32), np.float32)
    gw = dev.to_device(w)
    dev.launch("halo_conv_l2norm_y", (C // d, B), (d,), [dev.to_device(x), dev.to_device(tab), ("u32", 2), ("u32", 1),
                                                        gw, go, ("u32", C), ("u32", K), ("u32", 256), ("f32", 1e-6),
                                                        ("u32", C + 32)])
    got = go.download()
    for e in range(B):
        s1, o1 = dev.to_device(st[e]), dev.array((C,), np.float32)
        dev.launch("halo_conv_l2norm", (C // d,), (d,), [dev.to_device(x[e, :C]), s1, gw, o1, ("u32", C), ("u32", K),
                                                         ("u32", 256), ("f32", 1e-6)])
        assert got[e, :C].tobytes() == o1.download().tobytes()
        assert gst[e].download().tobytes() == s1.download().tobytes()


@pytest.mark.parametrize("T,C", [(13, 512), (2, 512), (21, 576)])
def test_conv_prefill8(dev, T, C):
    """halo_conv_l2norm_prefill8 (kern 4, 128 channels x 8 tokens per block; core.hip:3512-3570) against numpy:
    causal conv over the state then the chunk, SiLU, the first two heads L2-normalised; 1e-5 of the terms' magnitude.
    Its bytes equal halo_conv_l2norm_prefill's (the stepping arithmetic) on the same input, including a partial last
    head (C = 576: channels not a multiple of 128) and T % 8 != 0."""
    rng = np.random.default_rng(60 + T)
    K, d, l2 = 4, 128, 256
    w = rng.normal(0, 0.5, (C, K)).astype(np.float32)
    st = rng.normal(0, 1, (K - 1, C)).astype(np.float32)
    x = rng.normal(0, 1, (T, C)).astype(np.float32)
    go = dev.array((T, C), np.float32)
    gx, gst, gw = dev.to_device(x), dev.to_device(st), dev.to_device(w)
    dev.launch("halo_conv_l2norm_prefill8", ((C + d - 1) // d, (T + 7) // 8), (d,),
               [gx, gst, gw, go, ("u32", C), ("u32", T), ("u32", l2), ("f32", 1e-6)])
    seq = np.concatenate([st, x]).astype(np.float64)
    conv = np.stack([(seq[t:t + K] * w.T).sum(0) for t in range(T)])
    y = silu(conv.astype(np.float32))
    for h in range(l2 // d):
        seg = y[:, h * d:(h + 1) * d]
        y[:, h * d:(h + 1) * d] = seg / np.sqrt((seg * seg).sum(1, keepdims=True) + 1e-6)
    mag = np.stack([(np.abs(seq[t:t + K] * w.T)).sum(0) for t in range(T)]) + 1e-3
    got = go.download()
    close(got, y, mag)
    g1 = dev.array((T, C), np.float32)
    dev.launch("halo_conv_l2norm_prefill", ((C + d - 1) // d, T), (d,),
               [gx, gst, gw, g1, ("u32", C), ("u32", K), ("u32", l2), ("f32", 1e-6)])
    assert got.tobytes() == g1.download().tobytes()


# ---- exact batched fp32-x GEMVs (batch_decode.hip:133-190): every column equals the single-column kernel ----------
@pytest.mark.parametrize("R,NB,suf,groups", [(4, 1, "", 1), (4, 3, "_p", 2), (4, 8, "_ps", 1), (2, 2, "", 3),
                                             (2, 5, "_s", 1), (2, 8, "", 2)])
def test_batched_gemv_columns_equal_single(dev, R, NB, suf, groups):
    rng = np.random.default_rng(80 + R * 10 + NB)
    rows, cols, xstride, ystride = 1000, 2048, 2052, 1003  # ragged rows, padded column strides
    qs, d = O.synth_q8(rng, rows, cols)
    ncol = NB * groups
    x = rng.normal(0, 1, (ncol, xstride)).astype(np.float32)
    gq, gd, gx = dev.to_device(qs), dev.to_device(d), dev.to_device(x)
    gy = dev.array((ncol, ystride), np.float32)
    blocks = (rows + 8 * R - 1) // (8 * R)
    dev.launch(f"halo_gemv_q8r_r{R}_b{NB}{suf}", (blocks * groups,), (256,),
               [gq, gd, gx, gy, ("u32", rows), ("u32", cols), ("u32", cols), ("u32", xstride), ("u32", ystride),
                ("u32", groups)])
    got = gy.download()
    one = dev.array(rows, np.float32)
    for b in range(ncol):
        xb = dev.to_device(np.ascontiguousarray(x[b, :cols]))
        dev.launch(f"halo_gemv_q8r_r{R}" if R != 1 else "halo_gemv_q8r", (blocks,), (256,),
                   [gq, gd, xb, one, ("u32", rows), ("u32", cols), ("u32", cols)])
        assert got[b, :rows].tobytes() == one.download().tobytes(), f"column {b}"
    if NB == 1 and groups == 1:  # and the single kernel against the oracle
        want = np.zeros(rows, np.float32)
        O.oracle().or_matvec_q8_0_f32x(qs, d, rows, cols, cols, np.ascontiguousarray(x[0, :cols]), want, 1)
        w = np.abs(qs.astype(np.float64) * np.repeat(d.view(np.float16).astype(np.float64), 32, axis=1))
        close(got[0, :rows], want, w @ np.abs(x[0, :cols].astype(np.float64)))


@pytest.mark.parametrize("NB,suf,groups", [(1, "", 1), (4, "_p", 2), (8, "_ps", 1), (6, "_s", 1)])
def test_batched_dual_gemv_columns_equal_single(dev, NB, suf, groups):
    rng = np.random.default_rng(90 + NB)
    rows1, rows2, cols, xstride = 700, 300, 2048, 2048
    q1, d1 = O.synth_q8(rng, rows1, cols)
    q2, d2 = O.synth_q8(rng, rows2, cols)
    ncol = NB * groups
    x = rng.normal(0, 1, (ncol, xstride)).astype(np.float32)
    g1, e1, g2, e2, gx = (dev.to_device(a) for a in (q1, d1, q2, d2, x))
    y1, y2 = dev.array((ncol, rows1), np.float32), dev.array((ncol, rows2), np.float32)
    b1, b2 = (rows1 + 31) // 32, (rows2 + 31) // 32
    dev.launch(f"halo_gemv_q8r_dual_b{NB}{suf}", ((b1 + b2) * groups,), (256,),
               [g1, e1, y1, ("u32", rows1), ("u32", cols), g2, e2, y2, ("u32", rows2), ("u32", cols), gx,
                ("u32", cols), ("u32", b1), ("u32", xstride), ("u32", rows1), ("u32", rows2), ("u32", groups)])
    a1, a2 = y1.download(), y2.download()
    s1, s2 = dev.array(rows1, np.float32), dev.array(rows2, np.float32)
    for b in range(ncol):
        xb = dev.to_device(np.ascontiguousarray(x[b]))
        dev.launch("halo_gemv_q8r_dual", (b1 + b2,), (256,),
                   [g1, e1, s1, ("u32", rows1), ("u32", cols), g2, e2, s2, ("u32", rows2), ("u32", cols), xb,
                    ("u32", cols), ("u32", b1)])
        assert a1[b].tobytes() == s1.download().tobytes() and a2[b].tobytes() == s2.download().tobytes(), b
