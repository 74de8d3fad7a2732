"""GPU parity for the batched MoE layer (prefill: config C2's shapes at T = 48 tokens, and the reduced twin's shapes
at T = 1, 200 and 400, the last with 100 pairs per expert, so the grouped GEMMs take 128-pair tiles): fp32 router GEMM, top-k, pairs grouped by expert, grouped int8 MFMA gate/up (SwiGLU) and down,
slot-order combine with the shared expert.

Bars: router logits within 1e-5 * sum|w x| of a float64 product; ids equal to the oracle's RouteTopK on the GPU
logits and weights to 1e-6; the GPU's h codes equal to the host's quantization of the oracle's h except codes at a
rounding boundary, which may differ by one (counted, at most 1 in 10^4), and its h scales within 1e-5; each token's
output within 1e-5 of the terms' magnitude against the oracle's down projection of the GPU's own h codes
(teacher-forced), argmax equal; for T <= 16 the benchmark contract's 1e-3 against the decode path's output.
"""
import numpy as np
import pytest

import halo_amd as H
import oracle_py as O

pytestmark = pytest.mark.gpu


def _down(ws, off, n, dtype):
    return ws.download_range(off, n, dtype)


@pytest.fixture(scope="module")
def c2(dev):
    return H.MoeLayer(dev, seed=42)


@pytest.fixture(scope="module")
def small(dev):
    return H.MoeLayer(dev, n_experts=16, n_used=4, hidden=1024, ff=256, shared_ff=256, seed=7)


@pytest.mark.parametrize("shape,T", [("c2", 48), ("small", 1), ("small", 200), ("small", 400)])
def test_moe_prefill_matches_oracle(dev, c2, small, shape, T):
    L = c2 if shape == "c2" else small
    E, k, Hh, F = L.E, L.k, L.H, L.F
    rng = np.random.default_rng(T + E)
    x = rng.normal(0, 1, (T, Hh)).astype(np.float32)
    gx, out = dev.to_device(x), dev.array((T, Hh), np.float32)
    ws = L.prefill_workspace(T)
    L.forward_prefill(gx, out, T, ws)
    got = out.download()
    o_logits, o_sgl, o_ids, o_w = L.prefill_views(T)
    logits = _down(ws, o_logits, T * E, np.float32).reshape(T, E)
    sgl = _down(ws, o_sgl, T, np.float32)
    ids = _down(ws, o_ids, T * k, np.uint32).reshape(T, k)
    wts = _down(ws, o_w, T * k, np.float32).reshape(T, k)
    R = L.router.download().astype(np.float64)
    sg = L.sgate.download().astype(np.float64)
    want_logits = x.astype(np.float64) @ R.T
    assert np.all(np.abs(logits - want_logits) <= 1e-5 * (np.abs(x) @ np.abs(R.T)) + 1e-6)
    assert np.all(np.abs(sgl - x.astype(np.float64) @ sg) <= 1e-5 * (np.abs(x) @ np.abs(sg)) + 1e-6)
    o = O.oracle()
    gq, gd = L.gate.host()
    uq, ud = L.up.host()
    dq, dd = L.down.host()
    sgw, suw, sdw = L.sg.host(), L.su.host(), L.sd.host()
    xq, xs = O.quantize(x)
    o_pos, o_hq, o_hs = L.prefill_h_views(T)
    P = T * k
    pos = _down(ws, o_pos, P, np.uint32)
    ghq = _down(ws, o_hq, (P + T) * F, np.int8).reshape(P + T, F)
    ghs = _down(ws, o_hs, (P + T) * F // 32, np.float32).reshape(P + T, F // 32)
    flips = 0
    for t in range(T):
        oi, ow = np.zeros(k, np.uint32), np.zeros(k, np.float32)
        o.or_route_topk(np.ascontiguousarray(logits[t]), E, k, oi, ow)
        assert ids[t].tolist() == oi.tolist()
        assert np.allclose(wts[t], ow, rtol=1e-6, atol=0)
        acc = np.zeros(Hh, np.float64)
        mag = np.zeros(Hh, np.float64)
        for s in range(k + 1):
            if s < k:
                e = int(ids[t, s])
                gw, uw = (gq[e * F:(e + 1) * F], gd[e * F:(e + 1) * F]), (uq[e * F:(e + 1) * F], ud[e * F:(e + 1) * F])
                dw = (dq[e * Hh:(e + 1) * Hh], dd[e * Hh:(e + 1) * Hh])
                wgt = float(wts[t, s])
                row = int(pos[t * k + s])
            else:
                gw, uw, dw = sgw, suw, sdw
                wgt = float(o.or_sigmoid(float(sgl[t])))
                row = P + t
            g, _ = O.gemv_q8a8(*gw, xq[t], xs[t])
            u, _ = O.gemv_q8a8(*uw, xq[t], xs[t])
            h = np.array([o.or_silu(float(a)) for a in g], np.float32) * u.astype(np.float32)
            hq, hs = O.quantize(h)
            # the GPU's h codes: equal to the host's except a code at a rounding boundary (the GPU's fp32 h and the
            # host's differ in the last bits), which may differ by one
            dif = np.abs(ghq[row].astype(np.int32) - hq.astype(np.int32))
            assert dif.max() <= 1, f"token {t} slot {s}: h codes differ by {dif.max()}"
            assert np.allclose(ghs[row], hs, rtol=1e-5, atol=0), f"token {t} slot {s}: h scales"
            flips += int(np.count_nonzero(dif))
            # the down projection from the GPU's own codes (teacher-forced: no flip propagates)
            y, m = O.gemv_q8a8(*dw, ghq[row], ghs[row])
            acc += wgt * y
            mag += abs(wgt) * m
        assert np.all(np.abs(got[t] - acc) <= 1e-5 * mag + 1e-6), \
            f"token {t}: worst error / bar {np.max(np.abs(got[t] - acc) / (1e-5 * mag + 1e-6)):.3g}"
        assert int(np.argmax(got[t])) == int(np.argmax(acc)) or np.sort(acc)[-1] - np.sort(acc)[-2] <= 2e-5 * mag.max()
    assert flips <= max(8, (T * (k + 1) * F) // 10000), f"{flips} h-code flips"
    if T <= 16:
        wsd = L.workspace(T)
        outd = dev.array((T, Hh), np.float32)
        L.forward(gx, outd, T, wsd)
        dec = outd.download()
        scale = np.abs(dec).max()
        assert np.all(np.abs(got - dec) <= 1e-3 * scale), "prefill and decode paths disagree"
