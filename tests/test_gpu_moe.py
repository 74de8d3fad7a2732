"""GPU parity for the MoE decode layer (config C2: 512 experts + shared, hidden 2048, ff 512, top-10).

Checks, per token count T in {1, 4, 16}:
  * router logits within 1e-5 * sum|w x| of a float64 product;
  * top-k ids and renormalized weights equal to the oracle's RouteTopK applied to the GPU logits (bitwise ids,
    weights to 1e-6), and to the oracle's route of its own float64 logits except at measured near-ties;
  * every routed pair's h written (the union of experts is computed inside the gate/up launch: only the first
    token selecting an expert computes it, for all its tokens);
  * quantized activations bit-exact; h codes equal to the oracle's composition (SwiGLU of the exact-integer
    gate/up GEMVs, quantized per 32) except at rounding-boundary flips of +-1;
  * the layer output within 1e-5 * magnitude of the oracle composition fed the GPU's h codes, and within the benchmark contract's
    1e-3 relative of the oracle end to end.
"""
import ctypes

import numpy as np
import pytest

import halo_amd as H
import oracle_py as O

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def layer(dev):
    return H.MoeLayer(dev, seed=42)


@pytest.fixture(scope="module")
def small_layer(dev):
    """The reduced twin's shapes: 16 experts top-4, hidden 1024, ff 256 (lanes past ff idle in the down launch)."""
    return H.MoeLayer(dev, n_experts=16, n_used=4, hidden=1024, ff=256, shared_ff=256, seed=7)


def _view(ws, base, ptr, n, dtype):
    return ws.download_range(ptr - base, n, dtype)


def _gemv(qs, d, xq, xs):
    y, mag = O.gemv_q8a8(qs, d, xq, xs)
    return y.astype(np.float64), mag


@pytest.mark.parametrize("T,shape", [(1, "c2"), (4, "c2"), (16, "c2"), (1, "small"), (3, "small")])
def test_moe_decode_matches_oracle(dev, layer, small_layer, T, shape):
    L = layer if shape == "c2" else small_layer
    rng = np.random.default_rng(T)
    x = rng.normal(0, 1, (T, L.H)).astype(np.float32)
    gx = dev.to_device(x)
    out = dev.array((T, L.H), np.float32)
    ws = L.workspace(T)
    L.forward(gx, out, T, ws)
    got = out.download()
    v = L.views(T, ws)
    base = ws.ptr
    k, E = L.k, L.E
    logits = _view(ws, base, v.logits, T * E, np.float32).reshape(T, E)
    sgl = _view(ws, base, v.shared_logit, T, np.float32)
    ids = _view(ws, base, v.ids, T * k, np.uint32).reshape(T, k)
    wts = _view(ws, base, v.weights, T * k, np.float32).reshape(T, k)
    pof = np.arange(T * k, dtype=np.uint32).reshape(T, k)  # h row of (t, s) is t * k + s
    gxq = _view(ws, base, v.xq, T * L.H, np.int8).reshape(T, L.H)
    gxs = _view(ws, base, v.xs, T * L.H // 32, np.float32).reshape(T, -1)
    hstride = v.hstride
    gh = _view(ws, base, v.h, T * (k + 1) * hstride, np.float32).reshape(T * (k + 1), hstride)
    ghq, ghs = O.quantize(np.ascontiguousarray(gh[:, : L.F]))  # the down launch quantizes h exactly so

    # router
    R = L.router.download().astype(np.float64)
    want_logits = x.astype(np.float64) @ R.T
    mag = np.abs(x.astype(np.float64)) @ np.abs(R.T)
    assert np.all(np.abs(logits - want_logits) <= 1e-5 * mag + 1e-6)
    sg = L.sgate.download().astype(np.float64)
    assert np.all(np.abs(sgl - x.astype(np.float64) @ sg) <= 1e-5 * (np.abs(x) @ np.abs(sg)) + 1e-6)

    # routing: oracle's RouteTopK on the GPU logits
    o = O.oracle()
    for t in range(T):
        oi, ow = np.zeros(k, np.uint32), np.zeros(k, np.float32)
        o.or_route_topk(np.ascontiguousarray(logits[t]), E, k, oi, ow)
        assert ids[t].tolist() == oi.tolist()
        assert np.allclose(wts[t], ow, rtol=1e-6, atol=0)
        # and on float64 logits: the same ids unless the k-th and (k+1)-th logits are a near-tie
        fi, fw = np.zeros(k, np.uint32), np.zeros(k, np.float32)
        o.or_route_topk(want_logits[t].astype(np.float32), E, k, fi, fw)
        if fi.tolist() != oi.tolist():
            srt = np.sort(want_logits[t])[::-1]
            assert np.min(np.abs(np.diff(srt[: k + 1]))) < 1e-5, "routing differs away from a tie"

    # activations
    xq, xs = O.quantize(x)
    assert np.array_equal(gxq, xq) and np.array_equal(gxs.view(np.uint32), xs.view(np.uint32))

    # oracle composition, slot by slot
    F = L.F
    want_h = np.zeros((T * (k + 1), F), np.float32)
    for t in range(T):
        for s in range(k + 1):
            if s < k:
                e = int(ids[t, s])
                gq, gd = L.gate.host_rows(e * F, F)
                uq, ud = L.up.host_rows(e * F, F)
                p = int(pof[t, s])
            else:
                gq, gd = L.sg.host()
                uq, ud = L.su.host()
                p = T * k + t
            g, _ = _gemv(gq, gd, xq[t], xs[t])
            u_, _ = _gemv(uq, ud, xq[t], xs[t])
            h = np.array([o.or_silu(float(a)) for a in g.astype(np.float32)], np.float32) * u_.astype(np.float32)
            want_h[p] = h
    hq_w, hs_w = O.quantize(want_h)
    hmag = np.abs(want_h).max()
    assert np.allclose(gh[:, :F], want_h, rtol=1e-4, atol=1e-5 * hmag)
    diff = ghq.astype(np.int32) - hq_w.astype(np.int32)
    assert np.abs(diff).max() <= 1 and np.count_nonzero(diff) <= max(2, diff.size // 2000)
    assert np.allclose(ghs, hs_w, rtol=1e-5, atol=0)

    # down + combine: teacher-forced on the GPU's h codes (tight) and end to end (the contract's 1e-3)
    for t in range(T):
        acc_tf = np.zeros(L.H, np.float64)
        acc_e2e = np.zeros(L.H, np.float64)
        mag = np.zeros(L.H, np.float64)
        for s in range(k + 1):
            if s < k:
                e = int(ids[t, s])
                dq, dd = L.down.host_rows(e * L.H, L.H)
                p, wgt = int(pof[t, s]), float(wts[t, s])
            else:
                dq, dd = L.sd.host()
                p, wgt = T * k + t, float(o.or_sigmoid(float(sgl[t])))
            y_tf, m_tf = _gemv(dq, dd, np.ascontiguousarray(ghq[p, :F]), np.ascontiguousarray(ghs[p, : F // 32]))
            y_e2e, _ = _gemv(dq, dd, np.ascontiguousarray(hq_w[p]), np.ascontiguousarray(hs_w[p]))
            acc_tf += wgt * y_tf
            acc_e2e += wgt * y_e2e
            mag += abs(wgt) * m_tf
        assert np.all(np.abs(got[t] - acc_tf) <= 1e-5 * mag + 1e-6), f"token {t}: teacher-forced"
        assert np.all(np.abs(got[t] - acc_e2e) <= 1e-3 * mag + 1e-6), f"token {t}: end to end"
        assert int(np.argmax(got[t])) == int(np.argmax(acc_e2e))


def _topk_cases(rng, E):
    """Rows that reach every selection path of the one-wave top-k: exact ties among few values, about 100 equal
    maxima (more candidates than lanes), all equal (more than the candidate scratch: the arg-max fallback), 40 equal
    maxima among distinct values, and plain normal logits."""
    rows = [(rng.integers(-6, 6, E) * 0.25) for _ in range(3)]
    r = rng.normal(0, 1, E) - 10.0
    r[rng.choice(E, 100, replace=False)] = 2.5
    rows += [r, np.full(E, 0.75)]
    r = rng.normal(0, 1, E)
    r[rng.choice(E, 40, replace=False)] = 4.0
    rows += [r, rng.normal(0, 1, E), rng.normal(0, 3, E)]
    # 30 logits a few ulp apart at the top (probabilities that round together); one large logit over 100 near-zero
    # ones that all round to the same l - max (more than 64 candidates, ranked in two passes); a spread so wide that
    # selected probabilities are below 2^-100 or zero
    r = rng.normal(0, 1, E).astype(np.float32)
    r[rng.choice(E, 30, replace=False)] = np.float32(3.0) + rng.integers(0, 6, 30) * np.spacing(np.float32(3.0))
    rows.append(r)
    r = np.full(E, -5.0, np.float32)
    r[rng.choice(E, 100, replace=False)] = (rng.normal(0, 1, 100) * 1e-7).astype(np.float32)
    r[7] = 30.0
    rows.append(r)
    rows.append(rng.normal(0, 1, E) * 300.0)
    return np.stack(rows).astype(np.float32)


@pytest.mark.parametrize("kernel", ["halo_router_topk_rows", "halo_moe_topk_w512", "halo_moe_topk_w1024"])
def test_router_topk_reference_named(dev, kernel):
    """The one-wave top-k kernels (the reference-named rows launch and the decode-batch routing launches) on rows
    that reach every selection path: ids equal to the oracle's RouteTopK, weights to 1e-6."""
    rng = np.random.default_rng(5)
    E, k = 512, 10
    logits = _topk_cases(rng, E)
    T = logits.shape[0]
    gl = dev.to_device(logits)
    gi, gw = dev.array((T, k), np.uint32), dev.array((T, k), np.float32)
    dev.launch(kernel, (T,), (64,), [gl, gi, gw, ("u32", E), ("u32", k)])
    ids, w = gi.download(), gw.download()
    for t in range(T):
        oi, ow = np.zeros(k, np.uint32), np.zeros(k, np.float32)
        O.oracle().or_route_topk(logits[t], E, k, oi, ow)
        assert ids[t].tolist() == oi.tolist()
        assert np.allclose(w[t], ow, rtol=1e-6)


def test_gate_up_topk_one_token_selection_paths(dev, layer):
    """The one-token gate/up launch with its routing folded in (halo_moe_gate_up_topk_q8_s2_e512) on crafted logits
    that reach every selection path: block (0, 0)'s ids / weights equal the oracle's RouteTopK, and every h row
    (the k routed slots and the shared expert) equals the plain gate/up launch given those ids, bitwise."""
    L = layer
    rng = np.random.default_rng(17)
    E, k, F, H_ = L.E, L.k, L.F, L.H
    x = rng.normal(0, 1, H_).astype(np.float32)
    xq, xs = O.quantize(x[None, :])
    gxq, gxs = dev.to_device(xq), dev.to_device(xs)
    for row in _topk_cases(rng, E):
        gl = dev.to_device(row)
        ids, w = dev.array(k, np.uint32), dev.array(k, np.float32)
        h1, h2 = dev.array((k + 1, F), np.float32), dev.array((k + 1, F), np.float32)
        common = [L.gate.qs, L.gate.d, L.up.qs, L.up.d, L.sg.qs, L.sg.d, L.su.qs, L.su.d, gxq, gxs]
        dev.launch("halo_moe_gate_up_topk_q8_s2_e512", (k + 1, F // 4), (256,),
                   common + [gl, ids, w, h1, ("u32", E), ("u32", F), ("u32", F), ("u32", k), ("u32", F)])
        oi, ow = np.zeros(k, np.uint32), np.zeros(k, np.float32)
        O.oracle().or_route_topk(row, E, k, oi, ow)
        assert ids.download().tolist() == oi.tolist()
        assert np.allclose(w.download(), ow, rtol=1e-6, atol=0)
        dev.launch("halo_moe_gate_up_q8_s2", (k + 1, F // 4), (256,),
                   common + [dev.to_device(oi), h2, ("u32", 1), ("u32", F), ("u32", F), ("u32", k), ("u32", F)])
        assert np.array_equal(h1.download().view(np.uint32), h2.download().view(np.uint32))


@pytest.mark.parametrize("T", [1, 2, 4])
def test_moe_decode_norm_equals_norm_then_moe(dev, layer, T):
    """The router launch with the FFN norm in its prologue against halo_add_rmsnorm_q8 followed by the plain
    decode: the residual sum bitwise, the quantized activations bitwise (same canonical norm arithmetic), the logits
    within float reassociation, the routing identical, the output within 1e-5 of its magnitude."""
    L = layer
    rng = np.random.default_rng(100 + T)
    res = rng.normal(0, 1, (T, L.H)).astype(np.float32)
    delta = rng.normal(0, 1, (T, L.H)).astype(np.float32)
    nw = rng.normal(1, 0.1, L.H).astype(np.float32)
    g_res, g_delta, g_nw = dev.to_device(res), dev.to_device(delta), dev.to_device(nw)
    g_out_res = dev.array((T, L.H), np.float32)
    out_n = dev.array((T, L.H), np.float32)
    ws_n = L.workspace(T)
    L.forward_norm(g_res, g_delta, g_nw, g_out_res, out_n, T, ws_n)
    v = L.views(T, ws_n)
    k, E = L.k, L.E
    rd = lambda ws, p, n, dt: ws.download_range(p - ws.ptr, n, dt)
    # reference: the standalone norm (in place on a copy of res), then the plain decode
    r2 = dev.to_device(res)
    xn = dev.array((T, L.H), np.float32)
    xq = dev.array((T, L.H), np.int8)
    xs = dev.array((T, L.H // 32), np.float32)
    dev.launch("halo_add_rmsnorm_q8", (T,), (256,), [r2, g_delta, g_nw, xn, xq, xs, ("u32", L.H), ("f32", 1e-6)])
    out_r = dev.array((T, L.H), np.float32)
    ws_r = L.workspace(T)
    L.forward(xn, out_r, T, ws_r)
    assert np.array_equal(g_out_res.download().view(np.uint32), r2.download().view(np.uint32))
    assert np.array_equal(rd(ws_n, v.xq, T * L.H, np.int8), xq.download().reshape(-1))
    assert np.array_equal(rd(ws_n, v.xs, T * L.H // 32, np.float32).view(np.uint32), xs.download().reshape(-1).view(np.uint32))
    vr = L.views(T, ws_r)
    ln = rd(ws_n, v.logits, T * E, np.float32).reshape(T, E)
    lr = rd(ws_r, vr.logits, T * E, np.float32).reshape(T, E)
    x64 = xn.download().astype(np.float64)
    mag = np.abs(x64) @ np.abs(L.router.download().astype(np.float64).T)
    assert np.all(np.abs(ln - lr) <= 2e-5 * mag + 1e-6)
    ids_n = rd(ws_n, v.ids, T * k, np.uint32).reshape(T, k)
    ids_r = rd(ws_r, vr.ids, T * k, np.uint32).reshape(T, k)
    on, orr = out_n.download(), out_r.download()
    for t in range(T):
        if ids_n[t].tolist() != ids_r[t].tolist():
            srt = np.sort(lr[t].astype(np.float64))[::-1]
            assert np.min(np.abs(np.diff(srt[: k + 1]))) < 1e-5, "routing differs away from a tie"
            continue
        assert np.all(np.abs(on[t] - orr[t]) <= 1e-5 * np.abs(orr[t]).max() + 1e-6)


def test_moe_decode_workspace_reuse_across_token_counts(dev, layer):
    """One workspace for calls with T = 1, 4, 16, 2, 1, 3 in turn (T = 1: the routing inside the gate/up launch; else
    a top-k launch of its own): after every call the ids are the oracle's RouteTopK of the GPU logits and the output
    equals a call on a fresh workspace bitwise."""
    L = layer
    ws = L.workspace(16)
    o = O.oracle()
    for i, T in enumerate((1, 4, 16, 2, 1, 3)):
        rng = np.random.default_rng(100 + i)
        gx = dev.to_device(rng.normal(0, 1, (T, L.H)).astype(np.float32))
        out, out_fresh = dev.array((T, L.H), np.float32), dev.array((T, L.H), np.float32)
        L.forward(gx, out, T, ws)
        L.forward(gx, out_fresh, T, L.workspace(T))
        v = L.views(T, ws)
        logits = _view(ws, ws.ptr, v.logits, T * L.E, np.float32).reshape(T, L.E)
        ids = _view(ws, ws.ptr, v.ids, T * L.k, np.uint32).reshape(T, L.k)
        for t in range(T):
            oi, ow = np.zeros(L.k, np.uint32), np.zeros(L.k, np.float32)
            o.or_route_topk(np.ascontiguousarray(logits[t]), L.E, L.k, oi, ow)
            assert ids[t].tolist() == oi.tolist(), f"call {i} (T={T}) token {t}"
        assert np.array_equal(out.download().view(np.uint32), out_fresh.download().view(np.uint32))
