"""Host restatement of one decode step of the synthetic hybrid model, composed from the oracle's primitives.

TEST INFRASTRUCTURE ONLY: the checker for tests/test_gpu_model_oracle.py. It recomputes, from the model's own
weights (downloaded through halo_model_tensor), what the reference's ReferenceModel does for one token:
  embedding row (dequantized Q8_0)                      reference.cpp Forward, weights.cpp
  per layer: RMSNorm -> Q8 projections                  cpu_ops.cpp:134-145, reference.cpp MatVec
    DeltaNet: causal conv + SiLU, L2 norms, gates,      reference.cpp:278-366
              delta rule, gated RMSNorm, out projection
    GQA: q / gate split, q / k RMSNorm, NEOX rope,      reference.cpp:368-416, 492-527
         softmax attention over the cache, sigmoid gate
  residual, RMSNorm, MoE (router, top-k, experts,        reference.cpp:530-578, cpu_ops.cpp:187-207
  shared expert), residual
  final RMSNorm, LM head, argmax.
Activations entering a Q8_0 projection are quantized per 32 values (amax / 127, round half to even) as the
engine's int8 path does (src/kernels/core.hip:3089-3101). Element-wise functions run in float64 numpy and are
rounded to float32 per the reference's float arithmetic; the step is compared with a tolerance, not bitwise.
"""
from __future__ import annotations

import numpy as np

import oracle_py as O


def _f16(d):
    return d.view(np.float16).astype(np.float32)


def _sigmoid(x):
    return (1.0 / (1.0 + np.exp(-x.astype(np.float64)))).astype(np.float32)


def _silu(x):
    return (x.astype(np.float64) * _sigmoid(x).astype(np.float64)).astype(np.float32)


def _softplus(x):
    x = x.astype(np.float64)
    return np.where(x > 20.0, x, np.log1p(np.exp(x))).astype(np.float32)


def _rmsnorm(x, w, eps):
    y = np.ascontiguousarray(x, np.float32).copy()
    O.oracle().or_rmsnorm(y, y.size, np.ascontiguousarray(w, np.float32).ctypes.data, eps)
    return y


def _l2norm(x, eps):
    y = np.ascontiguousarray(x, np.float32).copy()
    O.oracle().or_l2norm(y, y.size, eps)
    return y


def _gemv(w, x):
    """Q8_0 weights (qs, d) times a float32 row quantized to Q8_0."""
    qs, d = w
    xq, xs = O.quantize(np.ascontiguousarray(x, np.float32))
    y, _ = O.gemv_q8a8(qs, d, xq, xs)
    return y


class RefModel:
    def __init__(self, model, cfg):
        self.c = cfg
        L = cfg.layers
        self.attn = [(l + 1) % cfg.attn_interval == 0 for l in range(L)]
        names_common = ["attn_norm", "ffn_norm", "router", "shared_gate", "gate", "up", "down", "sgate", "sup",
                        "sdown"]
        names_gdn = ["qkv", "z", "ab", "out", "conv_w", "a", "dt", "norm_w"]
        names_attn = ["qg", "k", "v", "o", "q_norm", "k_norm"]
        self.w = []
        for l in range(L):
            names = names_common + (names_attn if self.attn[l] else names_gdn)
            self.w.append({n: model.tensor(l, n) for n in names})
        self.embd = model.tensor(-1, "embd")
        self.head = model.tensor(-1, "head")
        self.out_norm = model.tensor(-1, "out_norm")[0]
        self.reset()

    def reset(self):
        c = self.c
        C = (2 * c.gdn_k_heads + c.gdn_v_heads) * c.gdn_head_dim
        self.pos = 0
        self.S = [np.zeros((c.gdn_v_heads, c.gdn_head_dim, c.gdn_head_dim), np.float32) if not a else None
                  for a in self.attn]
        self.conv = [np.zeros((max(c.conv_kernel - 1, 1), C), np.float32) if not a else None for a in self.attn]
        self.kc = [np.zeros((c.max_context, c.kv_heads, c.head_dim), np.float32) if a else None for a in self.attn]
        self.vc = [np.zeros((c.max_context, c.kv_heads, c.head_dim), np.float32) if a else None for a in self.attn]

    def _deltanet(self, l, xn):
        c, W = self.c, self.w[l]
        Hk, Hv, d, K = c.gdn_k_heads, c.gdn_v_heads, c.gdn_head_dim, c.conv_kernel
        Dk, Dv = Hk * d, Hv * d
        qkv = _gemv(W["qkv"], xn)
        z = _gemv(W["z"], xn)
        ab = _gemv(W["ab"], xn)
        cw = W["conv_w"]
        hist = self.conv[l]
        acc = cw[:, K - 1] * qkv
        for j in range(K - 1):
            acc = (acc + cw[:, j] * hist[j]).astype(np.float32)
        if K > 1:
            hist[:-1] = hist[1:].copy() if K > 2 else hist[:-1]
            hist[K - 2] = qkv
        y = _silu(acc.astype(np.float32))
        q = np.concatenate([_l2norm(y[h * d:(h + 1) * d], c.rms_eps) for h in range(Hk)])
        k = np.concatenate([_l2norm(y[Dk + h * d:Dk + (h + 1) * d], c.rms_eps) for h in range(Hk)])
        v = y[2 * Dk:]
        a, dt = W["a"][0], W["dt"][0]
        g = (a * _softplus((ab[:Hv] + dt).astype(np.float32))).astype(np.float32)
        beta = _sigmoid(ab[Hv:])
        o = np.zeros(Dv, np.float32)
        ora = O.oracle()
        for h in range(Hv):
            kh = h % Hk
            Sh = np.ascontiguousarray(self.S[l][h])
            oh = np.zeros(d, np.float32)
            ora.or_gdn_step(Sh, d, np.ascontiguousarray(q[kh * d:(kh + 1) * d]),
                            np.ascontiguousarray(k[kh * d:(kh + 1) * d]), np.ascontiguousarray(v[h * d:(h + 1) * d]),
                            float(g[h]), float(beta[h]), oh)
            self.S[l][h] = Sh
            on = _rmsnorm(oh, W["norm_w"][0], c.rms_eps)
            o[h * d:(h + 1) * d] = on * _sigmoid(z[h * d:(h + 1) * d])
        return _gemv(W["out"], o)

    def _attention(self, l, xn):
        c, W = self.c, self.w[l]
        Hq, Hkv, hd = c.q_heads, c.kv_heads, c.head_dim
        G = Hq // Hkv
        qg = _gemv(W["qg"], xn).reshape(Hq, 2, hd)
        kk = _gemv(W["k"], xn).reshape(Hkv, hd)
        vv = _gemv(W["v"], xn).reshape(Hkv, hd)
        q = np.stack([_rmsnorm(qg[h, 0], W["q_norm"][0], c.rms_eps) for h in range(Hq)])
        gate = qg[:, 1]
        kn = np.stack([_rmsnorm(kk[h], W["k_norm"][0], c.rms_eps) for h in range(Hkv)])
        q = np.ascontiguousarray(q)
        kn = np.ascontiguousarray(kn)
        O.oracle().or_rope_neox(q.reshape(-1), Hq, hd, c.rotary_dim, self.pos, c.rope_theta)
        O.oracle().or_rope_neox(kn.reshape(-1), Hkv, hd, c.rotary_dim, self.pos, c.rope_theta)
        self.kc[l][self.pos] = kn
        self.vc[l][self.pos] = vv
        n = self.pos + 1
        o = np.zeros((Hq, hd), np.float32)
        for h in range(Hq):
            kvh = h // G
            Kh = np.ascontiguousarray(self.kc[l][:n, kvh])
            Vh = np.ascontiguousarray(self.vc[l][:n, kvh])
            oh = np.zeros(hd, np.float32)
            O.oracle().or_attention_head(np.ascontiguousarray(q[h]), Kh, Vh, n, hd, hd, oh)
            o[h] = oh * _sigmoid(gate[h])
        return _gemv(W["o"], o.reshape(-1))

    def _moe(self, l, xn):
        c, W = self.c, self.w[l]
        E, k, F, SF, H = c.n_experts, c.n_used, c.expert_ff, c.shared_ff, c.hidden
        logits = np.zeros(E, np.float32)
        O.oracle().or_matvec_f32(np.ascontiguousarray(W["router"]), E, H, np.ascontiguousarray(xn), logits)
        ids, wts = np.zeros(k, np.uint32), np.zeros(k, np.float32)
        O.oracle().or_route_topk(logits, E, k, ids, wts)
        srt = np.sort(logits.astype(np.float64))[::-1]
        self.route_gaps.append(float(srt[k - 1] - srt[k]))  # logit gap at the top-k boundary
        out = np.zeros(H, np.float32)
        gq, gd = W["gate"]
        uq, ud = W["up"]
        dq, dd = W["down"]
        for s in range(k + 1):
            if s < k:
                e = int(ids[s])
                gw, uw = (gq[e * F:(e + 1) * F], gd[e * F:(e + 1) * F]), (uq[e * F:(e + 1) * F], ud[e * F:(e + 1) * F])
                dw = (dq[e * H:(e + 1) * H], dd[e * H:(e + 1) * H])
                wgt = float(wts[s])
            else:
                gw, uw, dw = W["sgate"], W["sup"], W["sdown"]
                wgt = float(_sigmoid(np.array([np.dot(W["shared_gate"][0].astype(np.float64),
                                                      xn.astype(np.float64))], np.float32))[0])
            h = (_silu(_gemv(gw, xn)) * _gemv(uw, xn)).astype(np.float32)
            out = (out + np.float32(wgt) * _gemv(dw, h)).astype(np.float32)
        return out, ids

    def step(self, token):
        """Feeds one token at the next position; returns the logits."""
        c = self.c
        qs, d = self.embd
        res = (_f16(d[token]).repeat(32) * qs[token].astype(np.float32)).astype(np.float32)
        self.last_ids = []
        self.route_gaps = []
        for l in range(c.layers):
            W = self.w[l]
            xn = _rmsnorm(res, W["attn_norm"][0], c.rms_eps)
            delta = self._attention(l, xn) if self.attn[l] else self._deltanet(l, xn)
            res = (res + delta).astype(np.float32)
            xn = _rmsnorm(res, W["ffn_norm"][0], c.rms_eps)
            m, ids = self._moe(l, xn)
            self.last_ids.append(ids)
            res = (res + m).astype(np.float32)
        self.pos += 1
        xn = _rmsnorm(res, self.out_norm, c.rms_eps)
        return _gemv(self.head, xn)
