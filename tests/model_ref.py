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
from layer_ref import attn_heads, attn_qk, deltanet_core, f16, moe_token, rmsnorm, route


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
        qkv, z, ab = _gemv(W["qkv"], xn), _gemv(W["z"], xn), _gemv(W["ab"], xn)
        o = deltanet_core(c.gdn_k_heads, c.gdn_v_heads, c.gdn_head_dim, c.rms_eps, W["conv_w"], W["a"][0],
                          W["dt"][0], W["norm_w"][0], qkv, z, ab, self.conv[l], self.S[l])
        return _gemv(W["out"], o)

    def _attention(self, l, xn):
        c, W = self.c, self.w[l]
        q, gate, kn = attn_qk(c.q_heads, c.kv_heads, c.head_dim, c.rotary_dim, c.rope_theta, c.rms_eps,
                              _gemv(W["qg"], xn), _gemv(W["k"], xn), W["q_norm"][0], W["k_norm"][0], self.pos)
        self.kc[l][self.pos] = kn
        self.vc[l][self.pos] = _gemv(W["v"], xn).reshape(c.kv_heads, c.head_dim)
        n = self.pos + 1
        return _gemv(W["o"], attn_heads(q, self.kc[l][:n], self.vc[l][:n], gate))

    def _moe(self, l, xn):
        c, W = self.c, self.w[l]
        F, H = c.expert_ff, c.hidden
        logits, _, _ = route(W["router"], xn, c.n_used)
        srt = np.sort(logits.astype(np.float64))[::-1]
        self.route_gaps.append(float(srt[c.n_used - 1] - srt[c.n_used]))  # logit gap at the top-k boundary
        gq, gd = W["gate"]
        uq, ud = W["up"]
        dq, dd = W["down"]

        def expert(e):
            return ((gq[e * F:(e + 1) * F], gd[e * F:(e + 1) * F]), (uq[e * F:(e + 1) * F], ud[e * F:(e + 1) * F]),
                    (dq[e * H:(e + 1) * H], dd[e * H:(e + 1) * H]))

        out, ids, _ = moe_token(xn, W["router"], W["shared_gate"][0], c.n_used, expert,
                                (W["sgate"], W["sup"], W["sdown"]), _gemv)
        return out, ids

    def step(self, token):
        """Feeds one token at the next position; returns the logits."""
        c = self.c
        qs, d = self.embd
        res = (f16(d[token]).repeat(32) * qs[token].astype(np.float32)).astype(np.float32)
        self.last_ids = []
        self.route_gaps = []
        for l in range(c.layers):
            W = self.w[l]
            xn = rmsnorm(res, W["attn_norm"][0], c.rms_eps)
            delta = self._attention(l, xn) if self.attn[l] else self._deltanet(l, xn)
            res = (res + delta).astype(np.float32)
            xn = rmsnorm(res, W["ffn_norm"][0], c.rms_eps)
            m, ids = self._moe(l, xn)
            self.last_ids.append(ids)
            res = (res + m).astype(np.float32)
        self.pos += 1
        xn = rmsnorm(res, self.out_norm, c.rms_eps)
        return _gemv(self.head, xn)
