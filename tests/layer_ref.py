"""Host restatement of the synthetic model's layer stages (test infrastructure only).

One function per stage of ReferenceModel's layers, values only, composed from the oracle's pinned primitives (RmsNorm,
L2Norm, Rope, the DeltaNet step, softmax attention, RouteTopK). They are shared by tests/model_ref.py (the whole
decode step), tests/teacher.py (the teacher-forced per-layer checks of the GPU) and tests/test_oracle_model_pins.py,
which pins each composition against the reference's own ReferenceModel::LinearAttention / Attention / Moe compiled
into oracle/_ref (src/model/reference.cpp:278-578). Projections are a parameter (`proj(w, x) -> y`): the engine's
int8-activation GEMV for the model, the reference's fp32 cpu::MatVec for the pins.
"""
from __future__ import annotations

import numpy as np

import oracle_py as O


def f16(d):
    return d.view(np.float16).astype(np.float32)


def sigmoid(x):
    return (1.0 / (1.0 + np.exp(-np.asarray(x, np.float64)))).astype(np.float32)


def silu(x):
    x = np.asarray(x, np.float32)
    return (x.astype(np.float64) * sigmoid(x).astype(np.float64)).astype(np.float32)


def softplus(x):
    x = np.asarray(x, np.float64)
    return np.where(x > 20.0, x, np.log1p(np.exp(x))).astype(np.float32)


def rmsnorm(x, w, eps):
    y = np.ascontiguousarray(x, np.float32).copy()
    O.oracle().or_rmsnorm(y, y.size, np.ascontiguousarray(w, np.float32).ctypes.data, eps)
    return y


def l2norm(x, eps):
    y = np.ascontiguousarray(x, np.float32).copy()
    O.oracle().or_l2norm(y, y.size, eps)
    return y


# ---- Gated DeltaNet (reference.cpp:278-366) ----------------------------------------------------------------------
def conv_silu(cw, window):
    """Causal depthwise conv of one step: taps cw [C][K] against window [K][C] (oldest input first, the current
    projection last), then SiLU (reference.cpp:296-305)."""
    K = cw.shape[1]
    acc = sum(cw[:, j].astype(np.float64) * np.asarray(window[j], np.float64) for j in range(K))
    return silu(acc.astype(np.float32))


def split_qkv(y, Hk, Hv, d, eps):
    """Conv output [2 Hk d + Hv d] -> q, k (each key head L2-normalised) and v (reference.cpp:307-316)."""
    Dk = Hk * d
    q = np.concatenate([l2norm(y[h * d:(h + 1) * d], eps) for h in range(Hk)])
    k = np.concatenate([l2norm(y[Dk + h * d:Dk + (h + 1) * d], eps) for h in range(Hk)])
    return q, k, np.asarray(y[2 * Dk:], np.float32)


def gdn_gates(a, dt, alpha, beta_logit):
    """Per value head: log decay g = a softplus(alpha + dt) and beta = sigmoid(beta logit) (reference.cpp:330-331)."""
    return (a * softplus(np.asarray(alpha, np.float32) + dt)).astype(np.float32), sigmoid(beta_logit)


def gdn_head(S_vm, q, k, v, g, beta):
    """One value head's delta-rule step on its value-major state S[j][i] (in place); returns o = S' q / sqrt(d)
    (reference.cpp:332-358)."""
    d = v.size
    o = np.zeros(d, np.float32)
    O.oracle().or_gdn_step(S_vm, d, np.ascontiguousarray(q, np.float32), np.ascontiguousarray(k, np.float32),
                           np.ascontiguousarray(v, np.float32), float(g), float(beta), o)
    return o


def gated_head_norm(o, norm_w, z, eps):
    """Per-head RMSNorm * w, then the sigmoid output gate (reference.cpp:359-363)."""
    return rmsnorm(o, norm_w, eps) * sigmoid(z)


def deltanet_core(Hk, Hv, d, eps, cw, a, dt, norm_w, qkv, z, ab, hist, S):
    """Everything of LinearAttention between its input projections and its output projection, for one token.
    hist [K-1][C] (oldest first) and S (per value head, value-major [d][d]) are updated in place; returns the gated,
    normalised heads o [Hv d]."""
    K = cw.shape[1]
    window = [hist[j] for j in range(K - 1)] + [qkv]
    y = conv_silu(cw, window)
    if K > 1:
        hist[:-1] = hist[1:].copy()
        hist[K - 2] = qkv
    q, k, v = split_qkv(y, Hk, Hv, d, eps)
    g, beta = gdn_gates(a, dt, ab[:Hv], ab[Hv:])
    o = np.zeros(Hv * d, np.float32)
    for h in range(Hv):
        kh = h % Hk
        oh = gdn_head(S[h], q[kh * d:(kh + 1) * d], k[kh * d:(kh + 1) * d], v[h * d:(h + 1) * d], g[h], beta[h])
        o[h * d:(h + 1) * d] = gated_head_norm(oh, norm_w, z[h * d:(h + 1) * d], eps)
    return o


# ---- gated GQA (reference.cpp:368-416, 492-527) ------------------------------------------------------------------
def attn_qk(Hq, Hkv, hd, rot, theta, eps, qg, k, q_norm, k_norm, pos):
    """q | gate split per head, RMSNorm of q and k heads, NEOX rope at pos: q [Hq][hd], gate [Hq][hd], k [Hkv][hd]."""
    g3 = np.asarray(qg, np.float32).reshape(Hq, 2, hd)
    q = np.ascontiguousarray(np.stack([rmsnorm(g3[h, 0], q_norm, eps) for h in range(Hq)]))
    kk = np.ascontiguousarray(np.stack([rmsnorm(np.asarray(k, np.float32).reshape(Hkv, hd)[h], k_norm, eps)
                                        for h in range(Hkv)]))
    O.oracle().or_rope_neox(q.reshape(-1), Hq, hd, rot, pos, theta)
    O.oracle().or_rope_neox(kk.reshape(-1), Hkv, hd, rot, pos, theta)
    return q, np.ascontiguousarray(g3[:, 1]), kk


def attn_heads(q, K, V, gate):
    """Softmax attention of each query head over positions K, V [n][Hkv][hd] (kv head h / (Hq / Hkv)), gated by
    sigmoid(gate); o [Hq hd]."""
    Hq, hd = q.shape
    n, Hkv = K.shape[0], K.shape[1]
    G = Hq // Hkv
    o = np.zeros((Hq, hd), np.float32)
    for h in range(Hq):
        kvh = h // G
        oh = np.zeros(hd, np.float32)
        O.oracle().or_attention_head(np.ascontiguousarray(q[h]), np.ascontiguousarray(K[:, kvh]),
                                     np.ascontiguousarray(V[:, kvh]), n, hd, hd, oh)
        o[h] = oh * sigmoid(gate[h])
    return o.reshape(-1)


# ---- MoE (reference.cpp:530-578) ---------------------------------------------------------------------------------
def route(router, x, k):
    """fp32 router logits (double accumulation, cpu::MatVec) and RouteTopK: logits, ids, weights."""
    E, H = router.shape
    logits = np.zeros(E, np.float32)
    O.oracle().or_matvec_f32(np.ascontiguousarray(router, np.float32), E, H, np.ascontiguousarray(x, np.float32),
                             logits)
    ids, wts = np.zeros(k, np.uint32), np.zeros(k, np.float32)
    O.oracle().or_route_topk(logits, E, k, ids, wts)
    return logits, ids, wts


def moe_token(x, router, shared_gate, k, expert, shared, proj):
    """out = sum over routed slots (slot order) of w_s down_e(SiLU(gate_e x) * up_e x) + sigmoid(shared_gate . x)
    * shared expert; expert(e) -> (gate, up, down) weights, shared = (gate, up, down), proj(w, v) -> y."""
    _, ids, wts = route(router, x, k)
    out = np.zeros(np.asarray(x).size, np.float32)
    for s in range(k + 1):
        if s < k:
            gw, uw, dw = expert(int(ids[s]))
            wgt = float(wts[s])
        else:
            gw, uw, dw = shared
            wgt = float(sigmoid(np.array([np.dot(np.asarray(shared_gate, np.float64),
                                                 np.asarray(x, np.float64))], np.float32))[0])
        h = (silu(proj(gw, x)) * proj(uw, x)).astype(np.float32)
        out = (out + np.float32(wgt) * proj(dw, h)).astype(np.float32)
    return out, ids, wts
