"""Teacher-forced per-layer parity of the GPU decode step (test infrastructure only).

Every layer of one traced GPU step (halo_model_step_trace) is recomputed on the host from the GPU's OWN inputs to
that layer, stage by stage, so an error cannot hide behind accumulated drift and a Q8 rounding flip cannot propagate:

  stage                                host input (from the GPU)            host restatement
  norm + quantize (layer input)        res_in                               oracle RmsNorm, then the Q8 quantizer
  projections                          the GPU's codes xq / xs              or_gemv_q8a8 (exact int32 block dots)
  DeltaNet core                        qkv, z, ab, conv ring and state      ReferenceModel::LinearAttention
                                       before the step                      (src/model/reference.cpp:278-366)
  GQA core                             qg, k, v, the KV cache               ReferenceModel::Attention, dense branch
                                                                            (src/model/reference.cpp:368-416, 492-527)
  output projection                    the GPU's codes oq / os              or_gemv_q8a8
  MoE                                  mres, the GPU's codes mxq / mxs,     ReferenceModel::Moe (reference.cpp:530-578)
                                       the GPU's h rows                     with RouteTopK (cpu_ops.cpp:187-207)
  final norm + LM head                 res_in of the head, its codes        RmsNorm, or_gemv_q8a8, argmax

Bars: fp32 outputs within 1e-5 * sum|term| (the reference's own GPU-test bound, tests/gpu/quant_gpu_test.cpp:115-122;
BASELINE's 1e-3 is 100x looser); integer work (codes, routing ids, residual adds) exact; a quantizer's code may
differ by +-1 only where the host's value lies within 2e-3 of a code's rounding boundary (the GPU's fp32 row and the
host's differ in the last bits), and every such flip is counted and reported. The recurrent state after the step is
checked against the host's update of the GPU's state before it.
"""
from __future__ import annotations

import numpy as np

import oracle_py as O
from layer_ref import (attn_heads, attn_qk, conv_silu, f16, gated_head_norm, gdn_gates, gdn_head, l2norm, rmsnorm,
                       sigmoid, silu, softplus, split_qkv)

FLIP_WINDOW = 2e-3  # in units of one code


# the value path of every stage is tests/layer_ref.py's (pinned against the reference's ReferenceModel layers)
_f16, _sigmoid, _silu, _softplus, _rmsnorm, _l2norm = f16, sigmoid, silu, softplus, rmsnorm, l2norm


def rope_mag(x, pos, rot, theta):
    """Term magnitude of NEOX-rotated rows x [heads][hd] (before rotation) at `pos`, for a 1e-5 bar: |a| + |b| of
    each rotated pair, widened by the angle's own fp32 rounding (the reference forms angle = float(pos) * freq in
    fp32, src/model/cpu_ops.cpp:168-185, so one ulp of freq can move the angle by one ulp of the angle, ~angle
    * 2^-23, whichever way a given powf rounds); dims past rot keep |x|."""
    x = np.asarray(x, np.float64)
    mag = np.abs(x).copy()
    half = rot // 2
    for i in range(half):
        ang = pos * theta ** (-2.0 * i / rot)
        widen = 1.0 + 2.0 * ang * 2.0 ** -23 / 1e-5
        ab = (np.abs(x[:, i]) + np.abs(x[:, i + half])) * widen
        mag[:, i] = ab
        mag[:, i + half] = ab
    return mag


class Report:
    """Counts of checks and quantizer flips, and the worst error of each stage relative to its bar."""

    def __init__(self):
        self.flips = 0
        self.loose = 0  # codes of cancellation-dominated values, within their magnitude bar (not flips)
        self.codes = 0
        self.worst = {}

    def close(self, what, got, want, mag, rel=1e-5):
        got = np.asarray(got, np.float64)
        want = np.asarray(want, np.float64)
        bar = rel * np.asarray(mag, np.float64) + 1e-30
        err = np.abs(got - want)
        r = float(np.max(err / bar)) if err.size else 0.0
        self.worst[what.split("@")[0]] = max(self.worst.get(what.split("@")[0], 0.0), r)
        if r > 1.0:
            i = int(np.argmax(err / bar))
            raise AssertionError(f"{what}: element {i} off by {err.flat[i]:.3e}, bar {bar.flat[i]:.3e} "
                                 f"(got {got.flat[i]:.6e}, want {want.flat[i]:.6e})")

    def codes_match(self, what, gq, gs, x_host, xmag=None):
        """GPU Q8 codes / scales of a row vs the host's fp32 value of the same row. xmag (default |x|) is the
        element's term magnitude: the GPU's value may differ from the host's by 1e-5 * xmag, so a block's scale by
        1e-5 * its largest xmag / 127, and a code by one where the host's value lies within FLIP_WINDOW + that
        difference (in codes) of a rounding boundary. Where that difference alone exceeds half a code (a value
        that is mostly cancellation: its terms are >= 5e4 codes' worth larger than the value), the code may lie
        anywhere within it: |code - host value / scale| <= 0.5 + FLIP_WINDOW + the difference; such codes are counted
        apart (`loose`), not as flips."""
        x = np.ascontiguousarray(x_host, np.float32).reshape(-1)
        xm = np.abs(x).astype(np.float64) if xmag is None else np.asarray(xmag, np.float64).reshape(-1)
        gq = np.asarray(gq).reshape(-1)
        gs = np.asarray(gs, np.float32).reshape(-1)
        hq, hs = O.quantize(x)
        bmag = np.maximum(np.abs(hs).astype(np.float64), xm.reshape(-1, 32).max(1) / 127.0)
        self.close(what + " scales", gs, hs, bmag, rel=1e-5)
        gsr = np.repeat(gs.astype(np.float64), 32)
        t = np.where(gsr > 0, x.astype(np.float64) / np.where(gsr > 0, gsr, 1.0), 0.0)
        want = np.rint(t)
        diff = gq.astype(np.int64) - want.astype(np.int64)
        bad = np.nonzero(diff)[0]
        self.codes += x.size
        if bad.size:
            dist = np.abs(np.abs(t[bad] - np.floor(t[bad])) - 0.5)
            allow = 1e-5 * xm[bad] / np.where(gsr[bad] > 0, gsr[bad], 1.0)  # the value bar in codes
            window = FLIP_WINDOW + allow
            flip = (np.abs(diff[bad]) <= 1) & (dist <= window)
            loose = ~flip & (allow > 0.5) & (np.abs(gq[bad].astype(np.float64) - t[bad]) <= 0.5 + window)
            ok = flip | loose
            if not ok.all():
                i = bad[np.argmin(ok)]
                raise AssertionError(f"{what}: code {i} is {gq[i]}, host value {t[i]:.6f} codes "
                                     f"(not a rounding-boundary flip; the bar in codes {allow[np.argmin(ok)]:.4g})")
            self.flips += int(flip.sum())
            self.loose += int(loose.sum())


def gemv(report, what, w, xq, xs, got):
    """A Q8_0 projection of the GPU's codes: exact integer block dots, fp32 within 1e-5 sum|term|."""
    y, mag = O.gemv_q8a8(w[0], w[1], np.ascontiguousarray(xq), np.ascontiguousarray(xs))
    report.close(what, got, y, mag)
    return y


class LayerChecker:
    """Checks every layer of traced steps of a halo_amd.Model against the host restatement."""

    def __init__(self, model, cfg):
        self.m, self.c = model, cfg
        self.attn = [(l + 1) % cfg.attn_interval == 0 for l in range(cfg.layers)]
        self.dense = {}
        self.report = Report()

    def _w(self, l, name):
        key = (l, name)
        if key not in self.dense:
            self.dense[key] = self.m.tensor(l, name)
        return self.dense[key]

    def _expert(self, l, name, e, rows):
        """Rows [e rows, (e + 1) rows) of a stacked expert tensor (small tensors are downloaded whole once)."""
        if self.c.n_experts * rows * self.c.hidden <= (64 << 20):
            qs, d = self._w(l, name)
            return qs[e * rows:(e + 1) * rows], d[e * rows:(e + 1) * rows]
        return self.m.tensor_rows(l, name, e * rows, rows)

    def snapshot(self, S, layers=None):
        """The GPU's recurrent state before a step: per layer DeltaNet state / conv ring, or the KV pools (all layers,
        or those in `layers`)."""
        snap = {"nkv": self.m.raw(-1, "nkv", np.uint32)[0, :S].copy(), "pages": self.m.raw(-1, "pages", np.uint32)}
        for l in range(self.c.layers):
            if layers is not None and l not in layers:
                continue
            if self.attn[l]:
                snap[(l, "k_pool")] = self.m.raw(l, "k_pool")
                snap[(l, "v_pool")] = self.m.raw(l, "v_pool")
            else:
                snap[(l, "state")] = self.m.raw(l, "state")
                snap[(l, "conv_ring")] = self.m.raw(l, "conv_ring")
        return snap

    # ---- stages ----------------------------------------------------------------------------------------------
    def _input(self, l, tr, S, norm_w):
        """The layer's residual input and the GPU's quantized RMSNorm of it (checked against the host's)."""
        c, H = self.c, self.c.hidden
        res = tr[(l, "res_in")].reshape(S, H)
        xq = tr[(l, "xq")].reshape(S, H)
        xs = tr[(l, "xs")].reshape(S, H // 32)
        for s in range(S):
            if self._do(s):
                self.report.codes_match(f"norm codes@L{l}s{s}", xq[s], xs[s], _rmsnorm(res[s], norm_w, c.rms_eps))
        return res, xq, xs

    sample = None  # batch rows whose per-token stages a prefill check covers (None: all)

    def _do(self, t):
        return self.sample is None or t in self.sample

    def _deltanet(self, l, tr, S, snap, after):
        c, r = self.c, self.report
        Hk, Hv, d, K = c.gdn_k_heads, c.gdn_v_heads, c.gdn_head_dim, c.conv_kernel
        Dk, Dv = Hk * d, Hv * d
        C = 2 * Dk + Dv
        _, xq, xs = self._input(l, tr, S, self._w(l, "attn_norm")[0])
        qkv = tr[(l, "qkv")].reshape(S, C)
        z = tr[(l, "z")].reshape(S, Dv)
        ab = tr[(l, "ab")].reshape(S, 2 * Hv)
        for s in range(S):
            gemv(r, f"qkv@L{l}s{s}", self._w(l, "qkv"), xq[s], xs[s], qkv[s])
            gemv(r, f"z@L{l}s{s}", self._w(l, "z"), xq[s], xs[s], z[s])
            gemv(r, f"ab@L{l}s{s}", self._w(l, "ab"), xq[s], xs[s], ab[s])
        cw = self._w(l, "conv_w")
        a, dt, nw = self._w(l, "a")[0], self._w(l, "dt")[0], self._w(l, "norm_w")[0]
        ring0 = snap[(l, "conv_ring")].reshape(c.max_sessions, K, C)
        ring1 = after[(l, "conv_ring")].reshape(c.max_sessions, K, C)
        st0 = snap[(l, "state")].reshape(c.max_sessions, Hv, d, d)
        st1 = after[(l, "state")].reshape(c.max_sessions, Hv, d, d)
        oq = tr[(l, "oq")].reshape(S, Dv)
        os_ = tr[(l, "os")].reshape(S, Dv // 32)
        for s in range(S):
            p = int(snap["nkv"][s]) - 1  # the step's position
            # causal conv: slots (p + 1 + j) % K, oldest first, then this step's projection (reference.cpp:296-305)
            win = [ring0[s, (p + 1 + j) % K] for j in range(K - 1)] + [qkv[s]]
            assert np.array_equal(ring1[s, p % K], qkv[s]), f"conv ring slot of L{l}"
            y = conv_silu(cw, win)
            q, k, v = split_qkv(y, Hk, Hv, d, c.rms_eps)
            # term magnitudes carried into the recurrence: the conv's sum |w x| through SiLU (slope <= 1.1) and,
            # for k, the head's L2 normalisation
            ymag = 1.1 * sum(np.abs(cw[:, j].astype(np.float64) * win[j]) for j in range(K)) + np.abs(y)
            kmag = np.concatenate([ymag[Dk + h * d:Dk + (h + 1) * d] /
                                   np.sqrt(np.sum(y[Dk + h * d:Dk + (h + 1) * d].astype(np.float64) ** 2) + c.rms_eps)
                                   for h in range(Hk)])
            vmag = ymag[2 * Dk:]
            g, beta = gdn_gates(a, dt, ab[s, :Hv], ab[s, Hv:])
            o = np.zeros(Dv, np.float32)
            omag = np.zeros(Dv, np.float64)
            for h in range(Hv):
                kh = h % Hk
                qh, khv, vh = q[kh * d:(kh + 1) * d], k[kh * d:(kh + 1) * d], v[h * d:(h + 1) * d]
                Sv = np.ascontiguousarray(st0[s, h].T)  # value-major for the oracle
                S_old = Sv.astype(np.float64).copy()
                oh = gdn_head(Sv, qh, khv, vh, g[h], beta[h])
                decay = np.exp(np.float64(g[h]))
                km = kmag[kh * d:(kh + 1) * d]
                dmag = vmag[h * d:(h + 1) * d] + np.abs(S_old) @ km
                mag_s = decay * np.abs(S_old) + np.outer(dmag, km)
                r.close(f"state@L{l}s{s}h{h}", st1[s, h].T, Sv, mag_s)
                zg = _sigmoid(z[s, h * d:(h + 1) * d])
                o[h * d:(h + 1) * d] = gated_head_norm(oh, nw, z[s, h * d:(h + 1) * d], c.rms_eps)
                # o = S' q / sqrt(d), normalised: its terms' magnitude scaled like the value
                rms = np.sqrt(np.mean(oh.astype(np.float64) ** 2) + c.rms_eps)
                omag[h * d:(h + 1) * d] = (mag_s @ np.abs(qh)) / np.sqrt(d) / rms * np.abs(nw) * zg
            r.codes_match(f"deltanet out codes@L{l}s{s}", oq[s], os_[s], o, np.maximum(omag, np.abs(o)))
            gemv(r, f"out@L{l}s{s}", self._w(l, "out"), oq[s], os_[s], tr[(l, "delta")].reshape(S, -1)[s])

    def _attention(self, l, tr, S, snap, after):
        c, r = self.c, self.report
        Hq, Hkv, hd = c.q_heads, c.kv_heads, c.head_dim
        G = Hq // Hkv
        _, xq, xs = self._input(l, tr, S, self._w(l, "attn_norm")[0])
        qg = tr[(l, "qg")].reshape(S, Hq * 2 * hd)
        kk = tr[(l, "k")].reshape(S, Hkv * hd)
        vv = tr[(l, "v")].reshape(S, Hkv * hd)
        for s in range(S):
            gemv(r, f"qg@L{l}s{s}", self._w(l, "qg"), xq[s], xs[s], qg[s])
            gemv(r, f"k@L{l}s{s}", self._w(l, "k"), xq[s], xs[s], kk[s])
            gemv(r, f"v@L{l}s{s}", self._w(l, "v"), xq[s], xs[s], vv[s])
        kp = after[(l, "k_pool")].reshape(-1, Hkv, 16, hd)
        vp = after[(l, "v_pool")].reshape(-1, Hkv, 16, hd)
        pages = snap["pages"]
        qn, kn = self._w(l, "q_norm")[0], self._w(l, "k_norm")[0]
        oq = tr[(l, "oq")].reshape(S, Hq * hd)
        os_ = tr[(l, "os")].reshape(S, Hq * hd // 32)
        for s in range(S):
            p = int(snap["nkv"][s]) - 1
            q, gate, k = attn_qk(Hq, Hkv, hd, c.rotary_dim, c.rope_theta, c.rms_eps, qg[s], kk[s], qn, kn, p)
            k_pre = np.stack([_rmsnorm(kk[s].reshape(Hkv, hd)[h], kn, c.rms_eps) for h in range(Hkv)])
            kmag = rope_mag(k_pre, p, c.rotary_dim, c.rope_theta)
            # this step's K / V rows as the GPU appended them
            pg = int(pages[s, p // 16])
            r.close(f"k append@L{l}s{s}", kp[pg, :, p % 16], k, kmag)
            assert np.array_equal(vp[pg, :, p % 16], vv[s].reshape(Hkv, hd)), f"v append L{l}"
            n = p + 1
            rows = np.array([int(pages[s, t // 16]) for t in range(n)])
            Kc = kp[rows, :, np.arange(n) % 16]  # [n][Hkv][hd], the GPU's cache (teacher-forced)
            Vc = vp[rows, :, np.arange(n) % 16]
            o = attn_heads(q, Kc, Vc, gate).reshape(Hq, hd)
            omag = np.zeros((Hq, hd), np.float64)
            for h in range(Hq):
                kvh = h // G
                gh = _sigmoid(gate[h])
                sc = Kc[:, kvh].astype(np.float64) @ q[h].astype(np.float64) / np.sqrt(hd)
                pw = np.exp(sc - sc.max())
                pw /= pw.sum()
                omag[h] = (pw @ np.abs(Vc[:, kvh]).astype(np.float64)) * gh  # sum_p P_p |v_p|, gated
            r.codes_match(f"attention out codes@L{l}s{s}", oq[s], os_[s], o.reshape(-1),
                          np.maximum(omag.reshape(-1), np.abs(o.reshape(-1))))
            gemv(r, f"o@L{l}s{s}", self._w(l, "o"), oq[s], os_[s], tr[(l, "delta")].reshape(S, -1)[s])

    def _moe(self, l, tr, S):
        c, r = self.c, self.report
        E, k, F, SF, H = c.n_experts, c.n_used, c.expert_ff, c.shared_ff, c.hidden
        res_in = tr[(l, "res_in")].reshape(S, H)
        delta = tr[(l, "delta")].reshape(S, H)
        mres = tr[(l, "mres")].reshape(S, H)
        assert np.array_equal(mres, (res_in + delta).astype(np.float32)), f"residual add L{l}"
        fnw = self._w(l, "ffn_norm")[0]
        xq = tr[(l, "mxq")].reshape(S, H)
        xs = tr[(l, "mxs")].reshape(S, H // 32)
        logits = tr[(l, "mlogits")].reshape(S, E)
        ids = tr[(l, "mids")].reshape(S, k)
        wts = tr[(l, "mweights")].reshape(S, k)
        shl = tr[(l, "mshared")].reshape(S)
        hst = tr[(l, "mh")].size // (S * (k + 1))
        hh = tr[(l, "mh")].reshape(S * (k + 1), hst)
        out = tr[(l, "mout")].reshape(S, H)
        R = self._w(l, "router")
        sg = self._w(l, "shared_gate")[0]
        for s in range(S):
            xn = _rmsnorm(mres[s], fnw, c.rms_eps)
            r.codes_match(f"moe input codes@L{l}s{s}", xq[s], xs[s], xn)
            x64 = xn.astype(np.float64)
            r.close(f"router@L{l}s{s}", logits[s], R.astype(np.float64) @ x64, np.abs(R) @ np.abs(x64))
            r.close(f"shared gate@L{l}s{s}", [shl[s]], [sg.astype(np.float64) @ x64], [np.abs(sg) @ np.abs(x64)])
            oi, ow = np.zeros(k, np.uint32), np.zeros(k, np.float32)
            O.oracle().or_route_topk(np.ascontiguousarray(logits[s]), E, k, oi, ow)
            assert ids[s].tolist() == oi.tolist(), f"routing of L{l}: {ids[s]} vs {oi}"
            r.close(f"route weights@L{l}s{s}", wts[s], ow, np.abs(ow), rel=1e-6)
            acc = np.zeros(H, np.float64)
            mag = np.zeros(H, np.float64)
            for slot in range(k + 1):
                if slot < k:
                    e = int(ids[s, slot])
                    gw, uw = self._expert(l, "gate", e, F), self._expert(l, "up", e, F)
                    dw = self._expert(l, "down", e, H)
                    f, wgt, row = F, float(wts[s, slot]), s * k + slot
                else:
                    gw, uw, dw = self._w(l, "sgate"), self._w(l, "sup"), self._w(l, "sdown")
                    f, wgt, row = SF, float(_sigmoid(shl[s])), S * k + s
                gy, gm = O.gemv_q8a8(gw[0], gw[1], xq[s], xs[s])
                uy, um = O.gemv_q8a8(uw[0], uw[1], xq[s], xs[s])
                hw = (_silu(gy) * uy).astype(np.float32)
                hmag = np.abs(_silu(gy)) * um + np.abs(uy) * gm * 1.1
                r.close(f"moe h@L{l}s{s}", hh[row, :f], hw, hmag + 1e-30)
                hq, hs = O.quantize(np.ascontiguousarray(hh[row, :f]))  # the down launch quantizes the GPU's h
                dy, dm = O.gemv_q8a8(dw[0], dw[1], hq, hs)
                acc += np.float64(np.float32(wgt)) * dy
                mag += abs(wgt) * dm
            r.close(f"moe out@L{l}s{s}", out[s], acc, mag)

    def _head(self, tr, S, logits):
        c, r = self.c, self.report
        H = c.hidden
        res = tr[(-1, "res_in")].reshape(S, H)
        lres = tr[(c.layers - 1, "mres")].reshape(S, H) + tr[(c.layers - 1, "mout")].reshape(S, H)
        assert np.array_equal(res, lres.astype(np.float32)), "final residual add"
        xq = tr[(-1, "xq")].reshape(S, H)
        xs = tr[(-1, "xs")].reshape(S, H // 32)
        head = self._w(-1, "head")
        on = self.m.tensor(-1, "out_norm")[0]
        for s in range(S):
            r.codes_match(f"head codes s{s}", xq[s], xs[s], _rmsnorm(res[s], on, c.rms_eps))
            y, mag = O.gemv_q8a8(head[0], head[1], xq[s], xs[s])
            r.close(f"lm head s{s}", logits[s], y, mag)
            top = np.argsort(y)[::-1]
            if int(np.argmax(logits[s])) != int(top[0]):
                assert y[top[0]] - y[top[1]] <= 2e-5 * mag[top[0]], "argmax differs away from a tie"

    def check_step(self, S, tokens, prefix=0):
        """Runs one traced GPU step for sessions 0..S-1 (tokens: the token each session feeds) and checks every
        layer; returns the step's logits [S][vocab]."""
        snap = self.snapshot(S)
        tr = self.m.step_trace(S, prefix)
        after = self.snapshot(S)
        logits = np.stack([self.m.logits(s) for s in range(S)])
        for l in range(self.c.layers):
            if tr[(l, "res_in")].size != S * self.c.hidden:
                raise AssertionError("trace shape")
            if l == 0:
                emb_q, emb_d = self._w(-1, "embd")
                want = np.stack([(_f16(emb_d[t]).repeat(32) * emb_q[t].astype(np.float32)) for t in tokens])
                assert np.array_equal(tr[(0, "res_in")].reshape(S, -1), want.astype(np.float32)), "embedding"
            else:
                prev = tr[(l - 1, "mres")].reshape(S, -1) + tr[(l - 1, "mout")].reshape(S, -1)
                assert np.array_equal(tr[(l, "res_in")].reshape(S, -1), prev.astype(np.float32)), f"residual L{l}"
            if self.attn[l]:
                self._attention(l, tr, S, snap, after)
            else:
                self._deltanet(l, tr, S, snap, after)
            self._moe(l, tr, S)
        self._head(tr, S, logits)
        return logits


class PrefillChecker(LayerChecker):
    """Every layer of one traced batched prefill (halo_model_prefill_trace) against the host restatement, token by
    token, from the GPU's own inputs of each stage. The DeltaNet recurrence is re-run on the host over the batch from
    the GPU's state before it and the GPU's per-token q / k / v / decay / beta (the chunked WY form on the GPU sums in
    another order, so its outputs are held to 1e-5 of the terms' magnitudes carried through the recurrence)."""

    def check_prefill(self, segments, prompts, layers=None, sample=None):
        """segments: (session, start, length) in batch order; prompts[s]: session s's prompt (host tokens).
        layers: the layer indices to trace and check (-1: the final norm and LM head; None: all). sample: the batch
        rows whose per-token stages are checked (None: all); the DeltaNet recurrence still runs over every token (the
        state after the batch is checked whole), and whole-batch checks (pair positions, h codes) cover every row."""
        c = self.c
        S = max(s for s, _, _ in segments) + 1
        self.sample = None if sample is None else set(int(t) for t in sample)
        sel = list(range(c.layers)) + [-1] if layers is None else sorted(set(layers))
        snap = self.snapshot(S, layers=None if layers is None else set(sel))
        tr = self.m.prefill_trace(segments, layers=None if layers is None else sel)
        after = self.snapshot(S, layers=None if layers is None else set(sel))
        self.after = after
        rows = []  # (session, position) of every batch row
        for s, a, n in segments:
            rows += [(s, a + j) for j in range(n)]
        T = len(rows)
        if 0 in sel:
            emb_q, emb_d = self._w(-1, "embd")
            want = np.stack([_f16(emb_d[int(prompts[s][p])]).repeat(32) * emb_q[int(prompts[s][p])].astype(np.float32)
                             for s, p in rows])
            assert np.array_equal(tr[(0, "res_in")].reshape(T, -1), want.astype(np.float32)), "embedding"
        for l in range(c.layers):
            if l not in sel:
                continue
            if l > 0 and l - 1 in sel:
                prev = tr[(l - 1, "mres")].reshape(T, -1) + tr[(l - 1, "mout")].reshape(T, -1)
                assert np.array_equal(tr[(l, "res_in")].reshape(T, -1), prev.astype(np.float32)), f"residual L{l}"
            if self.attn[l]:
                self._attention_prefill(l, tr, T, rows, snap, after)
            else:
                self._deltanet_prefill(l, tr, T, segments, snap, after)
            self._moe_prefill(l, tr, T)
        if -1 not in sel:
            return
        # final norm and the LM head on each segment's last token
        H = c.hidden
        res = tr[(-1, "res_in")].reshape(T, H)
        if c.layers - 1 in sel:
            lres = tr[(c.layers - 1, "mres")].reshape(T, H) + tr[(c.layers - 1, "mout")].reshape(T, H)
            assert np.array_equal(res, lres.astype(np.float32)), "final residual add"
        xq, xs = tr[(-1, "xq")].reshape(T, H), tr[(-1, "xs")].reshape(T, H // 32)
        head = self._w(-1, "head")
        on = self.m.tensor(-1, "out_norm")[0]
        f = 0
        for s, _, n in segments:
            t = f + n - 1
            f += n
            self.report.codes_match(f"head codes s{s}", xq[t], xs[t], _rmsnorm(res[t], on, c.rms_eps))
            y, mag = O.gemv_q8a8(head[0], head[1], xq[t], xs[t])
            got = self.m.logits(s)
            self.report.close(f"lm head s{s}", got, y, mag)
            top = np.argsort(y)[::-1]
            if int(np.argmax(got)) != int(top[0]):
                assert y[top[0]] - y[top[1]] <= 2e-5 * mag[top[0]], "argmax differs away from a tie"

    def _deltanet_prefill(self, l, tr, T, segments, snap, after):
        c, r = self.c, self.report
        Hk, Hv, d, K = c.gdn_k_heads, c.gdn_v_heads, c.gdn_head_dim, c.conv_kernel
        Dk, Dv = Hk * d, Hv * d
        C = 2 * Dk + Dv
        _, xq, xs = self._input(l, tr, T, self._w(l, "attn_norm")[0])
        qkv, z, ab = tr[(l, "qkv")].reshape(T, C), tr[(l, "z")].reshape(T, Dv), tr[(l, "ab")].reshape(T, 2 * Hv)
        for t in range(T):
            if self._do(t):
                gemv(r, f"qkv@L{l}t{t}", self._w(l, "qkv"), xq[t], xs[t], qkv[t])
                gemv(r, f"z@L{l}t{t}", self._w(l, "z"), xq[t], xs[t], z[t])
                gemv(r, f"ab@L{l}t{t}", self._w(l, "ab"), xq[t], xs[t], ab[t])
        gq, gk = tr[(l, "gq")].reshape(T, Dk), tr[(l, "gk")].reshape(T, Dk)
        gv = tr[(l, "gv")].reshape(T, Dv)
        gg, gb = tr[(l, "g")].reshape(T, Hv), tr[(l, "beta")].reshape(T, Hv)
        go = tr[(l, "o")].reshape(T, Dv)
        oq, os_ = tr[(l, "oq")].reshape(T, Dv), tr[(l, "os")].reshape(T, Dv // 32)
        cw = self._w(l, "conv_w")
        a, dt, nw = self._w(l, "a")[0], self._w(l, "dt")[0], self._w(l, "norm_w")[0]
        ring0 = snap[(l, "conv_ring")].reshape(c.max_sessions, K, C)
        ring1 = after[(l, "conv_ring")].reshape(c.max_sessions, K, C)
        st0 = snap[(l, "state")].reshape(c.max_sessions, Hv, d, d)
        st1 = after[(l, "state")].reshape(c.max_sessions, Hv, d, d)
        f = 0
        for s, start, n in segments:
            Sv = [np.ascontiguousarray(st0[s, h].T) for h in range(Hv)]  # value-major
            Sm = [np.abs(x).astype(np.float64) for x in Sv]  # term magnitudes carried by the recurrence
            for j in range(n):
                t, p = f + j, start + j
                win = []
                for jj in range(K):
                    pp = p - (K - 1) + jj
                    if pp >= start:
                        win.append(qkv[f + pp - start])
                    elif pp >= 0:
                        win.append(ring0[s, pp % K])
                    else:
                        win.append(np.zeros(C, np.float32))
                y = conv_silu(cw, win)
                ymag = 1.1 * sum(np.abs(cw[:, jj].astype(np.float64) * win[jj]) for jj in range(K)) + np.abs(y)
                for h in range(Hk):
                    for nm, base, got in (("q", 0, gq), ("k", Dk, gk)):
                        seg = y[base + h * d:base + (h + 1) * d]
                        nrm = np.sqrt(np.sum(seg.astype(np.float64) ** 2) + c.rms_eps)
                        r.close(f"conv {nm}@L{l}t{t}", got[t, h * d:(h + 1) * d], _l2norm(seg, c.rms_eps),
                                ymag[base + h * d:base + (h + 1) * d] / nrm)
                r.close(f"conv v@L{l}t{t}", gv[t], y[2 * Dk:], ymag[2 * Dk:])
                g, beta = gdn_gates(a, dt, ab[t, :Hv], ab[t, Hv:])
                r.close(f"decay@L{l}t{t}", gg[t], g, np.abs(g) + 1e-6)
                r.close(f"beta@L{l}t{t}", gb[t], beta, np.abs(beta))
                # the recurrence from the GPU's inputs (teacher-forced per token)
                kmag = np.concatenate([ymag[Dk + h * d:Dk + (h + 1) * d] /
                                       np.sqrt(np.sum(y[Dk + h * d:Dk + (h + 1) * d].astype(np.float64) ** 2) +
                                               c.rms_eps) for h in range(Hk)])
                for h in range(Hv):
                    kh = h % Hk
                    qh, kv_, vh = gq[t, kh * d:(kh + 1) * d], gk[t, kh * d:(kh + 1) * d], gv[t, h * d:(h + 1) * d]
                    km = np.maximum(kmag[kh * d:(kh + 1) * d], np.abs(kv_))
                    # this token's terms: |v| and |decay S k| (the actual state, so errors carried in from earlier
                    # tokens enter through the contraction decay (I - beta k k^T) rather than a worst-case feedback)
                    decay = np.exp(np.float64(gg[t, h]))
                    dmag = ymag[2 * Dk + h * d:2 * Dk + (h + 1) * d] + decay * (np.abs(Sv[h]).astype(np.float64) @ km)
                    Sm[h] = decay * Sm[h] + np.outer(dmag, km)
                    oh = gdn_head(Sv[h], qh, kv_, vh, gg[t, h], gb[t, h])
                    r.close(f"recurrence o@L{l}t{t}", go[t, h * d:(h + 1) * d], oh,
                            (Sm[h] @ np.abs(qh)) / np.sqrt(d))
                if not self._do(t):
                    continue
                # gated output norm from the GPU's o
                on = np.concatenate([gated_head_norm(go[t, h * d:(h + 1) * d], nw, z[t, h * d:(h + 1) * d],
                                                     c.rms_eps) for h in range(Hv)])
                r.codes_match(f"gated norm codes@L{l}t{t}", oq[t], os_[t], on)
                gemv(r, f"out@L{l}t{t}", self._w(l, "out"), oq[t], os_[t], tr[(l, "delta")].reshape(T, -1)[t])
            for h in range(Hv):
                r.close(f"state@L{l}s{s}h{h}", st1[s, h].T, Sv[h], Sm[h])
            for jj in range(min(K, n)):  # the ring holds the segment's last projections
                p = start + n - 1 - jj
                assert np.array_equal(ring1[s, p % K], qkv[f + n - 1 - jj]), f"conv ring L{l}"
            f += n

    def _attention_prefill(self, l, tr, T, rows, snap, after):
        c, r = self.c, self.report
        Hq, Hkv, hd = c.q_heads, c.kv_heads, c.head_dim
        G = Hq // Hkv
        _, xq, xs = self._input(l, tr, T, self._w(l, "attn_norm")[0])
        qg, kk, vv = (tr[(l, "qg")].reshape(T, Hq * 2 * hd), tr[(l, "k")].reshape(T, Hkv * hd),
                      tr[(l, "v")].reshape(T, Hkv * hd))
        aq = tr[(l, "aq")].reshape(T, Hq, hd)
        oq, os_ = tr[(l, "oq")].reshape(T, Hq * hd), tr[(l, "os")].reshape(T, Hq * hd // 32)
        kp = after[(l, "k_pool")].reshape(-1, Hkv, 16, hd)
        vp = after[(l, "v_pool")].reshape(-1, Hkv, 16, hd)
        pages = snap["pages"]
        qn, kn = self._w(l, "q_norm")[0], self._w(l, "k_norm")[0]
        for t, (s, p) in enumerate(rows):
            if not self._do(t):
                continue
            gemv(r, f"qg@L{l}t{t}", self._w(l, "qg"), xq[t], xs[t], qg[t])
            gemv(r, f"k@L{l}t{t}", self._w(l, "k"), xq[t], xs[t], kk[t])
            gemv(r, f"v@L{l}t{t}", self._w(l, "v"), xq[t], xs[t], vv[t])
            g3 = qg[t].reshape(Hq, 2, hd)
            q_pre = np.stack([_rmsnorm(g3[h, 0], qn, c.rms_eps) for h in range(Hq)])
            k_pre = np.stack([_rmsnorm(kk[t].reshape(Hkv, hd)[h], kn, c.rms_eps) for h in range(Hkv)])
            qmag, kmag = rope_mag(q_pre, p, c.rotary_dim, c.rope_theta), rope_mag(k_pre, p, c.rotary_dim, c.rope_theta)
            q, gate, k = attn_qk(Hq, Hkv, hd, c.rotary_dim, c.rope_theta, c.rms_eps, qg[t], kk[t], qn, kn, p)
            r.close(f"q rope@L{l}t{t}", aq[t], q, qmag)
            pg = int(pages[s, p // 16])
            r.close(f"k append@L{l}t{t}", kp[pg, :, p % 16], k, kmag)
            assert np.array_equal(vp[pg, :, p % 16], vv[t].reshape(Hkv, hd)), f"v append L{l}"
            n = p + 1
            prow = np.array([int(pages[s, u // 16]) for u in range(n)])
            Kc, Vc = kp[prow, :, np.arange(n) % 16], vp[prow, :, np.arange(n) % 16]
            o = attn_heads(aq[t], Kc, Vc, gate).reshape(Hq, hd)  # the GPU's rotated queries (teacher-forced)
            omag = np.zeros((Hq, hd), np.float64)
            for h in range(Hq):
                kvh = h // G
                qh = aq[t, h]
                gh = _sigmoid(gate[h])
                sc = Kc[:, kvh].astype(np.float64) @ qh.astype(np.float64) / np.sqrt(hd)
                pw = np.exp(sc - sc.max())
                pw /= pw.sum()
                omag[h] = (pw @ np.abs(Vc[:, kvh]).astype(np.float64)) * gh
            r.codes_match(f"attention out codes@L{l}t{t}", oq[t], os_[t], o.reshape(-1),
                          np.maximum(omag.reshape(-1), np.abs(o.reshape(-1))))
            gemv(r, f"o@L{l}t{t}", self._w(l, "o"), oq[t], os_[t], tr[(l, "delta")].reshape(T, -1)[t])

    def _moe_prefill(self, l, tr, T):
        c, r = self.c, self.report
        E, k, F, H = c.n_experts, c.n_used, c.expert_ff, c.hidden
        res_in, delta, mres = (tr[(l, "res_in")].reshape(T, H), tr[(l, "delta")].reshape(T, H),
                               tr[(l, "mres")].reshape(T, H))
        assert np.array_equal(mres, (res_in + delta).astype(np.float32)), f"residual add L{l}"
        fnw = self._w(l, "ffn_norm")[0]
        xq, xs = tr[(l, "mxq")].reshape(T, H), tr[(l, "mxs")].reshape(T, H // 32)
        logits, shl = tr[(l, "mlogits")].reshape(T, E), tr[(l, "mshared")].reshape(T)
        ids, wts, pos = tr[(l, "mids")].reshape(T, k), tr[(l, "mweights")].reshape(T, k), tr[(l, "mpos")].reshape(T, k)
        hh, hq, hs = (tr[(l, "mh")].reshape(-1, F), tr[(l, "mhq")].reshape(-1, F), tr[(l, "mhs")].reshape(-1, F // 32))
        out = tr[(l, "mout")].reshape(T, H)
        assert sorted(pos.reshape(-1).tolist()) == list(range(T * k)), "pair positions"
        # h codes: the quantizer on the GPU's own h rows, bit for bit
        wq, wsc = O.quantize(np.ascontiguousarray(hh))
        assert np.array_equal(hq, wq) and hs.tobytes() == wsc.tobytes(), f"h codes L{l}"
        R, sg = self._w(l, "router"), self._w(l, "shared_gate")[0]
        for t in range(T):
            if not self._do(t):
                continue
            xn = _rmsnorm(mres[t], fnw, c.rms_eps)
            r.codes_match(f"moe input codes@L{l}t{t}", xq[t], xs[t], xn)
            x64 = xn.astype(np.float64)
            r.close(f"router@L{l}t{t}", logits[t], R.astype(np.float64) @ x64, np.abs(R) @ np.abs(x64))
            r.close(f"shared gate@L{l}t{t}", [shl[t]], [sg.astype(np.float64) @ x64], [np.abs(sg) @ np.abs(x64)])
            oi, ow = np.zeros(k, np.uint32), np.zeros(k, np.float32)
            O.oracle().or_route_topk(np.ascontiguousarray(logits[t]), E, k, oi, ow)
            assert ids[t].tolist() == oi.tolist(), f"routing of L{l} token {t}"
            r.close(f"route weights@L{l}t{t}", wts[t], ow, np.abs(ow), rel=1e-6)
            acc, mag = np.zeros(H, np.float64), np.zeros(H, np.float64)
            for slot in range(k + 1):
                if slot < k:
                    e = int(ids[t, slot])
                    gw, uw = self._expert(l, "gate", e, F), self._expert(l, "up", e, F)
                    dw = self._expert(l, "down", e, H)
                    wgt, row = float(wts[t, slot]), int(pos[t, slot])
                else:
                    gw, uw, dw = self._w(l, "sgate"), self._w(l, "sup"), self._w(l, "sdown")
                    wgt, row = float(_sigmoid(shl[t])), T * k + t
                gy, gm = O.gemv_q8a8(gw[0], gw[1], xq[t], xs[t])
                uy, um = O.gemv_q8a8(uw[0], uw[1], xq[t], xs[t])
                r.close(f"moe h@L{l}t{t}", hh[row], (_silu(gy) * uy).astype(np.float32),
                        np.abs(_silu(gy)) * um + np.abs(uy) * gm * 1.1 + 1e-30)
                dy, dm = O.gemv_q8a8(dw[0], dw[1], hq[row], hs[row])
                acc += np.float64(np.float32(wgt)) * dy
                mag += abs(wgt) * dm
            r.close(f"moe out@L{l}t{t}", out[t], acc, mag)
