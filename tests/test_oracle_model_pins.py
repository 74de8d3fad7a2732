"""Pins of the host layer restatement (tests/layer_ref.py) against the reference's own layer code.

oracle/_ref/libhaloref_model.so compiles the reference's ReferenceModel (src/model/reference.cpp) where it lies and
exposes its LinearAttention (:278-366), Attention (:368-527) and Moe (:530-578) one layer at a time. Each test feeds
the reference layer and the restatement the same weights (raw GGUF Q8_0 blocks) and inputs over several consecutive
tokens, with the projections done by the reference's own cpu::MatVec (fp32 activations, double accumulation), so the
only differences left are the summation orders inside the restated stages. Bars: 1e-5 of each output's terms'
magnitude; routing ids exact; the conv history bitwise. A plausible slip in the restatement (silu for sigmoid on the
output gate, the wrong key head for a value head, a conv tap order reversed, the state transposed, an unrenormalised
routing weight, the shared gate applied to the routed sum) moves the outputs by far more than that.
Skipped where the reference tree is absent (the GPU box).
"""
import numpy as np
import pytest

import oracle_py as O
from layer_ref import attn_heads, attn_qk, deltanet_core, moe_token

pytestmark = pytest.mark.skipif(not O.has_ref_model(), reason="oracle/_ref/libhaloref_model.so not built")


def q8_raw(rng, rows, cols, sigma=0.02):
    qs, d = O.synth_q8(rng, rows, cols, sigma)
    raw = np.zeros(rows * (cols // 32) * 34, np.uint8)
    O.oracle().or_pack_q8_0(qs, d, raw, rows, cols, cols)
    return raw, qs, d


def ref_matvec(raw, rows, cols, x):
    """The reference's cpu::MatVec over a raw Q8_0 matrix (fp32 activations, double accumulation)."""
    y = np.zeros(rows, np.float32)
    O.ref().ref_matvec_q8_0(raw, rows, cols, np.ascontiguousarray(x, np.float32), y)
    return y


def q8_mag(qs, d, x):
    """sum |w x| of each row of a Q8_0 matrix."""
    w = np.abs(qs.astype(np.float64) * np.repeat(d.view(np.float16).astype(np.float64), 32, axis=1))
    return w @ np.abs(np.asarray(x, np.float64))


def close(got, want, mag, rel=1e-5):
    err = np.abs(np.asarray(got, np.float64) - np.asarray(want, np.float64))
    bar = rel * np.asarray(mag, np.float64) + 1e-30
    assert np.all(err <= bar), f"max error / bar {float(np.max(err / bar)):.3g}"


def test_linear_attention_matches_reference_model():
    rng = np.random.default_rng(70)
    H, Hk, Hv, d, K, eps = 256, 2, 4, 128, 4, 1e-6
    C, Dv = (2 * Hk + Hv) * d, Hv * d
    qkv, _, _ = q8_raw(rng, C, H)
    z, _, _ = q8_raw(rng, Dv, H)
    al, _, _ = q8_raw(rng, Hv, H)
    be, _, _ = q8_raw(rng, Hv, H)
    out, oq, od = q8_raw(rng, H, Dv)
    cw = rng.normal(0, 0.5, (C, K)).astype(np.float32)
    a = -np.exp(rng.normal(0, 0.5, Hv)).astype(np.float32)
    dt = rng.normal(0, 0.5, Hv).astype(np.float32)
    nw = rng.normal(1, 0.1, d).astype(np.float32)
    shape_u, shape_f = np.array([H, Hk, Hv, d, K], np.uint32), np.array([eps], np.float32)
    conv_r = np.zeros((K - 1, C), np.float32)
    st_r = np.zeros((Hv, d, d), np.float32)  # S[h][j][i], value-major: the restatement's layout too
    conv_h, st_h = conv_r.copy(), st_r.copy()
    for t in range(6):
        x = rng.normal(0, 1, H).astype(np.float32)
        y_r = np.zeros(H, np.float32)
        O.ref_model().ref_linear_attention(shape_u, shape_f, qkv, z, al, be, out, cw, a, dt, nw, conv_r, st_r, x, y_r)
        p_qkv, p_z = ref_matvec(qkv, C, H, x), ref_matvec(z, Dv, H, x)
        p_ab = np.concatenate([ref_matvec(al, Hv, H, x), ref_matvec(be, Hv, H, x)])
        o = deltanet_core(Hk, Hv, d, eps, cw, a, dt, nw, p_qkv, p_z, p_ab, conv_h, st_h)
        y_h = ref_matvec(out, H, Dv, o)
        assert np.array_equal(conv_h, conv_r), f"token {t}: conv history"
        close(st_h, st_r, np.abs(st_r) + 1e-2 * np.abs(st_r).max())
        close(y_h, y_r, q8_mag(oq, od, o))


def test_attention_matches_reference_model():
    rng = np.random.default_rng(71)
    H, Hq, Hkv, hd, rot, theta, eps = 256, 4, 2, 256, 64, 1e7, 1e-6
    T = 7
    q, _, _ = q8_raw(rng, Hq * 2 * hd, H)
    k, _, _ = q8_raw(rng, Hkv * hd, H)
    v, _, _ = q8_raw(rng, Hkv * hd, H)
    o, oq, od = q8_raw(rng, H, Hq * hd)
    qn = rng.normal(1, 0.1, hd).astype(np.float32)
    kn = rng.normal(1, 0.1, hd).astype(np.float32)
    x = rng.normal(0, 1, (T, H)).astype(np.float32)
    y_r = np.zeros((T, H), np.float32)
    O.ref_model().ref_attention(np.array([H, Hq, Hkv, hd, rot], np.uint32), np.array([eps, theta], np.float32), q, k,
                                v, o, qn, kn, x, y_r, T)
    Kc, Vc = np.zeros((T, Hkv, hd), np.float32), np.zeros((T, Hkv, hd), np.float32)
    for t in range(T):
        qq, gate, kk = attn_qk(Hq, Hkv, hd, rot, theta, eps, ref_matvec(q, Hq * 2 * hd, H, x[t]),
                               ref_matvec(k, Hkv * hd, H, x[t]), qn, kn, t)
        Kc[t], Vc[t] = kk, ref_matvec(v, Hkv * hd, H, x[t]).reshape(Hkv, hd)
        ctx = attn_heads(qq, Kc[:t + 1], Vc[:t + 1], gate)
        close(ref_matvec(o, H, Hq * hd, ctx), y_r[t], q8_mag(oq, od, ctx))


def test_moe_matches_reference_model():
    rng = np.random.default_rng(72)
    H, E, k, F, SF = 256, 16, 4, 64, 64
    router = rng.normal(0, 0.02, (E, H)).astype(np.float32)
    gate, _, _ = q8_raw(rng, E * F, H)
    up, _, _ = q8_raw(rng, E * F, H)
    down, dq, dd = q8_raw(rng, E * H, F)
    sgate_inp = rng.normal(0, 0.02, H).astype(np.float32)
    sg, _, _ = q8_raw(rng, SF, H)
    su, _, _ = q8_raw(rng, SF, H)
    sd, sdq, sdd = q8_raw(rng, H, SF)
    gb, db = F * (H // 32) * 34, H * (F // 32) * 34  # bytes of one expert's gate (up) and down

    def proj(w, xv):
        raw, rows, cols = w
        return ref_matvec(raw, rows, cols, xv)

    def expert(e):
        return ((gate[e * gb:(e + 1) * gb], F, H), (up[e * gb:(e + 1) * gb], F, H), (down[e * db:(e + 1) * db], H, F))

    for t in range(8):
        x = rng.normal(0, 1, H).astype(np.float32)
        y_r = np.zeros(H, np.float32)
        O.ref_model().ref_moe(np.array([H, E, k, F, SF], np.uint32), router, gate, up, down, sgate_inp, sg, su, sd, x,
                              y_r)
        y_h, ids, wts = moe_token(x, router, sgate_inp, k, expert, ((sg, SF, H), (su, SF, H), (sd, H, SF)), proj)
        assert wts.sum() == pytest.approx(1.0, abs=1e-6)
        # magnitude: sum over slots of |weight| * |W_down| |h| (h = SiLU(gate x) * up x of the slot's expert)
        mag = np.zeros(H)
        sw = 1.0 / (1.0 + np.exp(-float(np.dot(sgate_inp.astype(np.float64), x))))
        for s_, (e, wgt) in enumerate(list(zip(ids.tolist(), wts.tolist())) + [(None, sw)]):
            gw, uw, _ = expert(e) if e is not None else ((sg, SF, H), (su, SF, H), None)
            g_, u_ = proj(gw, x), proj(uw, x)
            hv = g_ / (1.0 + np.exp(-g_.astype(np.float64))) * u_
            qd = (dq[e * H:(e + 1) * H], dd[e * H:(e + 1) * H]) if e is not None else (sdq, sdd)
            mag += abs(wgt) * q8_mag(qd[0], qd[1], hv)
        close(y_h, y_r, mag)
