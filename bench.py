#!/usr/bin/env python3
"""Benchmark of the quantized decode hot path on one MI355X.

Headline workload (C0, batch 1): one Q8_0 GEMV, W [4096 x 4096] x Q8_0-quantized x, the
metric's "Q8_0 GEMV achieved HBM GB/s". Weights are seeded on the device and rotated over enough distinct copies
(>= 600 MB) that no launch reads weights from the 256 MB MALL. A step is one GEMV; exactly --steps GEMVs are timed,
after --warmup untimed ones in the same graph, between two device wall-clock stamps.

value    = algorithmic bytes of a GEMV (17,858,560: weights + x + y) / measured time per GEMV, in GB/s.
roofline = the same kernel (halo_gemv_q8a8s_l64_r1_b1) against 8 TB/s, with the calibrated PMC traffic from the
           committed profile; moe.T1.roofline likewise for the MoE layer at one token.
cpu_baseline = the reference's cpu::MatVec (built from its sources into oracle/_ref) on the same GEMV, all hardware
           threads, plus legs: 1 thread, the C1 projections, the C2 MoE layer at T=1 and the C3 recurrence at S=4.
Other sections: c1 (the three projections at M = 1..16), moe (C2), gdn (C3), c4 (the hybrid model), sample.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "halo-flash_amd"))

HBM_PEAK_GBS = 8000.0
C0_BYTES = 4096 * 128 * 34 + 4096 * 4 + 4096 * 4  # 17,858,560
C1_SHAPES = [(4096, 2048), (512, 2048), (2048, 4096)]  # fused q/gate, kv, o
MIN_ROTATION_BYTES = 600 << 20


def q8_bytes(rows, cols):
    return rows * (cols // 32) * 34


def c1_pass_bytes(m: int) -> int:
    """Algorithmic bytes of one C1 pass: every weight byte once, fp32 inputs and outputs per token."""
    w = sum(q8_bytes(r, c) for r, c in C1_SHAPES)
    act = m * (2048 * 4 + 4096 * 4)  # x (read by the quantizer) and a
    out = m * (4096 + 512 + 2048) * 4
    return w + act + out


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def run_gpu(args):
    import halo_amd as H

    dev = H.Device()
    try:
        res = {}
        if args.mode == "c0":
            return run_c0(args, dev, H, res)
        if args.mode == "membw":
            return run_membw(args, dev, H, res)
        if args.mode == "moe":
            return run_moe(args, dev, H, res)
        if args.mode == "gdn":
            return run_gdn(args, dev, H, res)
        if args.mode == "c4":
            return run_c4(args, dev, H, res)
        if args.mode == "pmc":
            return run_pmc(args, dev, H, res)
        if args.mode == "attn":
            return run_attn(args, dev, H, res)
        if args.mode == "proj":
            return run_proj(args, dev, H, res)
        if args.mode == "prefill":
            return run_prefill(args, dev, H, res)
        if args.mode == "pgemm":
            return run_pgemm(args, dev, H, res)
        if args.mode == "sample":
            return run_sample(args, dev, H, res)
        if args.mode == "c1":
            return run_c1(args, dev, H, res)
        if args.mode == "phases":
            return run_phases(args, dev, H, res)
        run_c0(args, dev, H, res)
        if not args.quick:
            roof = res["roofline"]
            run_c1(args, dev, H, res)
            run_moe(args, dev, H, res)
            run_gdn(args, dev, H, res)
            run_c4(args, dev, H, res)
            run_sample(args, dev, H, res)
            res["roofline"] = roof
        return res
    finally:
        dev.close()


def run_c1(args, dev, H, res):
    """C1: one decode pass through the three projections (quantize x -> q|gate + kv, quantize a -> o), fused
    (prologue quantization, grouped matrices) and unfused, at M = 1, 2, 4, 8, 16 tokens."""
    per_copy = sum(q8_bytes(r, c) for r, c in C1_SHAPES)
    copies = max(2, -(-MIN_ROTATION_BYTES // per_copy))
    log(f"[bench] C1: {copies} weight copies ({copies * per_copy / 2**20:.0f} MiB)")
    sets = []
    for i in range(copies):
        sets.append([H.Q8Weights(dev, r, c).synth(dev, seed=1000 * i + j) for j, (r, c) in enumerate(C1_SHAPES)])
    mmax = 16
    x = dev.array((mmax, 2048), np.float32)
    a = dev.array((mmax, 4096), np.float32)
    dev.op("synth_f32", x.ptr, mmax * 2048, 7, 1.0)
    dev.op("synth_f32", a.ptr, mmax * 4096, 8, 1.0)
    xq, xs = dev.array((mmax, 2048), np.int8), dev.array((mmax, 64), np.float32)
    aq, as_ = dev.array((mmax, 4096), np.int8), dev.array((mmax, 128), np.float32)
    yqg, ykv, yo = (dev.array((mmax, 4096), np.float32), dev.array((mmax, 512), np.float32),
                    dev.array((mmax, 2048), np.float32))
    dev.sync()

    in_x = H.ProjInput(x=x.ptr, mode=H.PROJ_F)
    in_a = H.ProjInput(x=a.ptr, mode=H.PROJ_F)

    in_xq = H.ProjInput(xq=xq.ptr, xs=xs.ptr, mode=H.PROJ_Q)
    in_aq = H.ProjInput(xq=aq.ptr, xs=as_.ptr, mode=H.PROJ_Q)

    def c1_pass(ws, m, fused=True, mfma=False, pair=True):
        if fused and (m == 1 or (m == 2 and not pair)):
            # one launch per input row set: quantize prologue + (q|gate, kv), then quantize prologue + o
            H.proj_q8(dev, ws[:2], [yqg, ykv], in_x, m)
            H.proj_q8(dev, ws[2:], [yo], in_a, m)
            return
        if fused:
            # from 2 token rows: both inputs quantized by one launch, then the grouped projections on the quantized
            # rows (v_dot4 up to 8 tokens, int8 matrix cores beyond; `mfma`: the matrix cores at any token count)
            t = (2, 2) if mfma else (0, 0)
            dev.op("quantize_q8_pair", x.ptr, xq.ptr, xs.ptr, 2048, a.ptr, aq.ptr, as_.ptr, 4096, m)
            if pair and (not mfma or m >= 9):  # both projections in one launch (halo_proj_q8q2_* / _q8m2_*)
                H.proj_q8_pair(dev, ws, [yqg, ykv, yo], 2, in_xq, in_aq, m)
                return
            H.proj_q8(dev, ws[:2], [yqg, ykv], in_xq, m, *t)
            H.proj_q8(dev, ws[2:], [yo], in_aq, m, *t)
            return
        dev.op("quantize_q8", x.ptr, xq.ptr, xs.ptr, m, 2048)
        dev.op("matvec_q8a8", ctypes.byref(ws[0].desc), xq.ptr, xs.ptr, yqg.ptr, m, 4096)
        dev.op("matvec_q8a8", ctypes.byref(ws[1].desc), xq.ptr, xs.ptr, ykv.ptr, m, 512)
        dev.op("quantize_q8", a.ptr, aq.ptr, as_.ptr, m, 4096)
        dev.op("matvec_q8a8", ctypes.byref(ws[2].desc), aq.ptr, as_.ptr, yo.ptr, m, 2048)

    # correctness spot check of copy 0 against the oracle before timing anything
    sys.path.insert(0, str(ROOT / "oracle"))
    import oracle_py as O

    c1_pass(sets[0], 1)
    qs, d = sets[0][2].host()
    a_host = a.download()[0]
    aq_h, as_h = O.quantize(a_host)
    want, mag = O.gemv_q8a8(qs, d, aq_h, as_h)
    got = yo.download()[0]
    assert np.all(np.abs(got - want) <= 1e-5 * mag + 1e-6), "bench spot check failed"

    if args.eager:  # kernel durations (and counters) of the M = 1, 4, 8, 16 passes, direct launches
        for m in (1, 4, 8, 16):
            for _ in range(3):
                for ws in sets:
                    c1_pass(ws, m)
            dev.sync()
        res["c1"] = None
        return res

    def graph_for(m, fused=True, mfma=False, pair=True):
        dev.begin_capture()
        for ws in sets:
            c1_pass(ws, m, fused, mfma, pair)
        return dev.end_capture()

    sweep = {}
    g = graph_for(1, fused=False)  # the unfused sequence (2 quantize + 3 GEMV launches), for comparison
    dev.launch_graph(g)
    dev.sync()
    nrep = max(1, -(-1000 // copies))
    dev.timer_start()
    for _ in range(nrep):
        dev.launch_graph(g)
    ms = dev.timer_stop()
    sweep["1_unfused"] = {"us_per_pass": round(ms / (nrep * copies) * 1e3, 3),
                          "GBps": round(c1_pass_bytes(1) / (ms / (nrep * copies) * 1e-3) / 1e9, 1)}
    dev.free_graph(g)
    for m in (1, 2, 3, 4, 8, 16, "2_prologue", "4_two", "8_two", "16_two", "4_mfma", "8_mfma"):
        tag = str(m).split("_")[1] if isinstance(m, str) else ""
        # 2_prologue: both launches quantizing in their prologues; *_two: quantize + two projection launches
        g = graph_for(int(str(m).split("_")[0]), mfma=tag == "mfma", pair=tag not in ("two", "prologue"))
        reps = 1 if m != 1 else max(1, args.warmup // copies)
        for _ in range(reps):
            dev.launch_graph(g)
        dev.sync()
        nrep = max(1, -(-(2000 if m == 1 else 400) // copies))
        dev.timer_start()
        for _ in range(nrep):
            dev.launch_graph(g)
        ms = dev.timer_stop()
        steps = nrep * copies
        mi = int(str(m).split("_")[0])
        sweep[str(m)] = {"us_per_pass": round(ms / steps * 1e3, 3),
                         "GBps": round(c1_pass_bytes(mi) / (ms / steps * 1e-3) / 1e9, 1)}
        dev.free_graph(g)
    res["c1"] = {"workload": "C1 Q8_0 projections 2048->4096, 2048->512, 4096->2048 from fp32 activations: at M = 1 "
                             "quantized in the projections' prologues (2 launches); from M = 2 both inputs quantized "
                             "by one launch, then both projections on the quantized rows in one launch (v_dot4, "
                             "halo_proj_q8q2_*) up to 8 tokens, on int8 matrix cores (halo_proj_q8m2_c2x4) at 16; "
                             "*_two: the two "
                             "projections as two launches; 2_prologue: M = 2 as M = 1 runs; *_mfma: the matrix-core "
                             "kernel at that M", "bytes_per_pass_m1": c1_pass_bytes(1),
                 "GBps_m1": sweep["1"]["GBps"], "sweep": sweep}
    log(f"[bench] C1 sweep {sweep}")
    return res


def moe_bytes(E, H_, F, SF, U, T):
    """Algorithmic bytes of one MoE decode call: router (fp32) + shared gate row + shared expert + U routed
    experts (Q8_0, 34 bytes per 32 weights), fp32 activations in and out."""
    q8 = lambda r, c: r * (c // 32) * 34
    expert = 2 * q8(F, H_) + q8(H_, F)
    shared = 2 * q8(SF, H_) + q8(H_, SF)
    return E * H_ * 4 + H_ * 4 + shared + U * expert + 2 * T * H_ * 4


def run_moe(args, dev, H, res):
    """C2: one MoE layer decode at T tokens. The 512-expert pool (1.7 GB) is shared; router, shared gate and
    shared expert are rotated over copies (> 256 MB), and each call routes a different x, so expert weights come
    from HBM."""
    import ctypes as C

    base = H.MoeLayer(dev, seed=77)
    ncopy = 40
    copies = []
    for i in range(ncopy):
        r = dev.array((base.E, base.H), np.float32)
        dev.op("synth_f32", r.ptr, base.E * base.H, 1000 + i, 0.02)
        sgv = dev.array(base.H, np.float32)
        dev.op("synth_f32", sgv.ptr, base.H, 2000 + i, 0.02)
        sg = H.Q8Weights(dev, base.SF, base.H).synth(dev, 3000 + i)
        su = H.Q8Weights(dev, base.SF, base.H).synth(dev, 4000 + i)
        sd = H.Q8Weights(dev, base.H, base.SF).synth(dev, 5000 + i)
        w = H.MoeWeights()
        C.memmove(C.byref(w), C.byref(base.w), C.sizeof(w))
        w.router, w.shared_gate = r.ptr, sgv.ptr
        w.shared_gate_proj, w.shared_up, w.shared_down = sg.desc, su.desc, sd.desc
        copies.append((w, [r, sgv, sg, su, sd]))
    out = {}
    for T in (1, 4, 16):
        xs = [dev.array((T, base.H), np.float32) for _ in range(ncopy)]
        for i, x in enumerate(xs):
            dev.op("synth_f32", x.ptr, T * base.H, 9000 + 100 * T + i, 1.0)
        y = dev.array((T, base.H), np.float32)
        wsb = H.lib().halo_op_moe_workspace_bytes(C.byref(base.w), T)
        wss = [dev.array(wsb, np.uint8) for _ in range(ncopy)]
        dev.sync()
        if args.eager:  # per-kernel durations under a profiler that cannot trace graph launches
            for _ in range(5):
                for (w, _), x, ws in zip(copies, xs, wss):
                    dev.op("moe_decode", C.byref(w), x.ptr, y.ptr, T, ws.ptr, ws.nbytes)
            dev.sync()
            continue
        dev.begin_capture()
        for (w, _), x, ws in zip(copies, xs, wss):
            dev.op("moe_decode", C.byref(w), x.ptr, y.ptr, T, ws.ptr, ws.nbytes)
        g = dev.end_capture()
        dev.launch_graph(g)
        dev.sync()
        nrep = max(1, 2000 // ncopy // max(1, T // 4))
        dev.timer_start()
        for _ in range(nrep):
            dev.launch_graph(g)
        ms = dev.timer_stop()
        us = ms * 1e3 / (nrep * ncopy)
        dev.free_graph(g)
        Us = []
        for (w, _), ws in zip(copies, wss):
            v = H.MoeViews()
            H._call("halo_op_moe_views", C.byref(w), T, ws.ptr, C.byref(v))
            ids = ws.download_range(v.ids - ws.ptr, T * base.k, np.uint32)
            Us.append(len(set(ids.tolist())))
        nbytes = float(np.mean([moe_bytes(base.E, base.H, base.F, base.SF, u, T) for u in Us]))
        out[f"T{T}"] = {"us_per_layer": round(us, 3), "mean_U": round(float(np.mean(Us)), 2),
                        "GBps": round(nbytes / (us * 1e-6) / 1e9, 1)}
        if T == 1:
            gbps = nbytes / (us * 1e-6) / 1e9
            out["T1"]["roofline"] = {
                "bound": "hbm", "kernel": "MoE decode layer at T=1 (halo_op_moe_decode: router, top-k, gate/up, down)",
                "achieved": round(gbps, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(gbps / HBM_PEAK_GBS, 4),
                "traffic": None, "algorithmic_bytes_per_launch": round(nbytes),
                "timing": "HIP events over graph replays of 40 layers with rotated routers, shared experts and inputs"}
        if T <= 4:
            # the layer as the model runs it: residual + delta -> FFN norm -> MoE, as a norm launch followed by the
            # plain decode, and with the norm in the router launch
            dl = [dev.array((T, base.H), np.float32) for _ in range(ncopy)]
            for i, x in enumerate(dl):
                dev.op("synth_f32", x.ptr, T * base.H, 19000 + 100 * T + i, 1.0)
            nw = dev.array(base.H, np.float32)
            dev.op("synth_f32", nw.ptr, base.H, 777, 1.0)
            r2, xn = dev.array((T, base.H), np.float32), dev.array((T, base.H), np.float32)
            times = {}
            for variant in ("norm_then_moe", "norm_in_router"):
                dev.begin_capture()
                for (w, _), x, d, ws in zip(copies, xs, dl, wss):
                    if variant == "norm_then_moe":
                        dev.launch("halo_add_rmsnorm_q8", (T,), (256,), [("ptr", x.ptr), ("ptr", d.ptr), nw, xn,
                                                                         None, None, ("u32", base.H), ("f32", 1e-6)])
                        dev.op("moe_decode", C.byref(w), xn.ptr, y.ptr, T, ws.ptr, ws.nbytes)
                    else:
                        inp = H.ProjInput(x=x.ptr, delta=d.ptr, norm_w=nw.ptr, res_out=r2.ptr, eps=1e-6,
                                          mode=H.PROJ_N)
                        dev.op("moe_decode_norm", C.byref(w), C.byref(inp), y.ptr, T, ws.ptr, ws.nbytes)
                g = dev.end_capture()
                dev.launch_graph(g)
                dev.sync()
                dev.timer_start()
                for _ in range(nrep):
                    dev.launch_graph(g)
                times[variant] = round(dev.timer_stop() * 1e3 / (nrep * ncopy), 3)
                dev.free_graph(g)
            out[f"T{T}"]["us_with_ffn_norm"] = times
        log(f"[bench] moe T={T}: {out[f'T{T}']}")
    res["moe"] = out
    res["roofline"] = None
    return res


def run_proj(args, dev, H, res):
    """Grouped projections alone, over a grid-size sweep: the C1 pair (q|gate 4096 + kv 512 rows, cols 2048,
    fp32 input quantized in the prologue) and the DeltaNet input group (q|k|v 8192 + z 4096 + alpha|beta 64 rows,
    RMSNorm(res + delta) prologue), at 1 and 4 tokens; weights rotated over > 600 MB."""
    groups = {"c1_pair": ([(4096, 2048), (512, 2048)], H.PROJ_F), "gdn_in": ([(8192, 2048), (4096, 2048), (64, 2048)],
                                                                             H.PROJ_N)}
    out = {}
    for gname, (shapes, mode) in groups.items():
        per = sum(q8_bytes(r, c) for r, c in shapes)
        ncopy = max(2, -(-MIN_ROTATION_BYTES // per))
        sets = [[H.Q8Weights(dev, r, c).synth(dev, seed=500 * i + j) for j, (r, c) in enumerate(shapes)]
                for i in range(ncopy)]
        x = dev.array((8, 2048), np.float32)
        dl = dev.array((8, 2048), np.float32)
        w = dev.array(2048, np.float32)
        r2 = dev.array((8, 2048), np.float32)
        for a, sd in ((x, 1), (dl, 2), (w, 3)):
            dev.op("synth_f32", a.ptr, a.nbytes // 4, sd, 1.0)
        ys = [dev.array((8, r), np.float32) for r, _ in shapes]
        inp = H.ProjInput(x=x.ptr, delta=dl.ptr if mode == H.PROJ_N else None, norm_w=w.ptr, res_out=r2.ptr,
                          eps=1e-6, mode=mode)
        xq = dev.array((8, 2048), np.int8)
        xs = dev.array((8, 64), np.float32)
        dev.op("quantize_q8", x.ptr, xq.ptr, xs.ptr, 8, 2048)
        inq = H.ProjInput(xq=xq.ptr, xs=xs.ptr, mode=H.PROJ_Q)
        for T in (1, 4):
            for pname, pin in (("pro", inp), ("q", inq)):
                for lpr in (64, 32):
                    for blocks in (1, 2, 4):  # tasks per wave
                        dev.begin_capture()
                        for ws in sets:
                            H.proj_q8(dev, ws, ys, pin, T, blocks, lpr)
                        g = dev.end_capture()
                        dev.launch_graph(g)
                        dev.sync()
                        nrep = max(1, -(-2000 // ncopy))
                        dev.timer_start()
                        for _ in range(nrep):
                            dev.launch_graph(g)
                        us = dev.timer_stop() * 1e3 / (nrep * ncopy)
                        dev.free_graph(g)
                        key = f"{gname}_T{T}_{pname}_l{lpr}_t{blocks}"
                        out[key] = {"us": round(us, 2), "GBps": round(per / (us * 1e-6) / 1e9, 1)}
                        log(f"[bench] proj {key}: {us:.2f} us, {per / (us * 1e-6) / 1e9:.0f} GB/s")
        # the same bytes as one stacked matrix through the plain int8 GEMV (activations quantized beforehand)
        rows_all = sum(r for r, _ in shapes)
        big = [H.Q8Weights(dev, rows_all, 2048).synth(dev, seed=900 + i) for i in range(ncopy)]
        yb = dev.array((8, rows_all), np.float32)
        for T in (1, 4):
            dev.begin_capture()
            for wb in big:
                dev.op("matvec_q8a8", ctypes.byref(wb.desc), xq.ptr, xs.ptr, yb.ptr, T, rows_all)
            g = dev.end_capture()
            dev.launch_graph(g)
            dev.sync()
            nrep = max(1, -(-2000 // ncopy))
            dev.timer_start()
            for _ in range(nrep):
                dev.launch_graph(g)
            us = dev.timer_stop() * 1e3 / (nrep * ncopy)
            dev.free_graph(g)
            key = f"{gname}_T{T}_plain_gemv_stacked"
            out[key] = {"us": round(us, 2), "GBps": round(per / (us * 1e-6) / 1e9, 1)}
            log(f"[bench] proj {key}: {us:.2f} us, {per / (us * 1e-6) / 1e9:.0f} GB/s")
        del big
        # the same group with every copy carved out of one pooled allocation (qs and scales contiguous)
        pool_bytes = ncopy * sum(r * c + r * (c // 32) * 2 for r, c in shapes) + 4096 * ncopy * len(shapes) * 2
        pool = dev.array(pool_bytes, np.uint8)
        psets, off = [], 0
        for i in range(ncopy):
            ws_ = []
            for j, (r, c) in enumerate(shapes):
                qs_p = pool.ptr + off
                off += (r * c + 4095) // 4096 * 4096
                d_p = pool.ptr + off
                off += (r * (c // 32) * 2 + 4095) // 4096 * 4096
                dev.op("synth_q8", qs_p, d_p, r, c, c, 700 + 10 * i + j, 0.02)
                ws_.append(H.Q8Matrix(qs_p, d_p, r, c, c, 0))
            psets.append(ws_)
        for T in (1, 4):
            dev.begin_capture()
            for ws_ in psets:
                mats = (H.Q8Matrix * len(ws_))(*ws_)
                ysp = (ctypes.c_void_p * len(ys))(*[o.ptr for o in ys])
                dev.op("proj_q8_grid", mats, ysp, len(ws_), ctypes.byref(inq), T, 1, 32)
            g = dev.end_capture()
            dev.launch_graph(g)
            dev.sync()
            nrep = max(1, -(-2000 // ncopy))
            dev.timer_start()
            for _ in range(nrep):
                dev.launch_graph(g)
            us = dev.timer_stop() * 1e3 / (nrep * ncopy)
            dev.free_graph(g)
            key = f"{gname}_T{T}_q_l32_g1024_pooled"
            out[key] = {"us": round(us, 2), "GBps": round(per / (us * 1e-6) / 1e9, 1)}
            log(f"[bench] proj {key}: {us:.2f} us, {per / (us * 1e-6) / 1e9:.0f} GB/s")
        del pool
        del sets
    res["proj"] = out
    return res


def run_attn(args, dev, H, res):
    """C4's decode attention alone (16 q heads, 2 kv heads, head_dim 256, fp32 paged KV): 1 session at 8576
    visible positions, and 4 sessions sharing an 8192-token prefix with 384 suffix positions each. Eight KV pools
    (> 256 MB) are rotated so K/V come from HBM. Bytes = K/V rows read (the shared prefix once). `S*` times the
    decode from normalized queries, `S*_step` the model's form from the projections (norms, rotation, K / V
    append in the partial launch)."""
    import ctypes as C

    Hq, Hkv, D, PAGE, ncopy = 16, 2, 256, 16, 8
    out = {}
    for S, prefix, suffix in ((1, 0, 8576), (4, 8192, 384)):
        max_context = prefix + suffix
        max_pages = -(-max_context // PAGE)
        total = prefix // PAGE + S * (max_pages - prefix // PAGE)
        pages = np.zeros((S, max_pages), np.uint32)
        nxt = prefix // PAGE
        for s in range(S):
            pages[s, : prefix // PAGE] = np.arange(prefix // PAGE)
            pages[s, prefix // PAGE:] = np.arange(nxt, nxt + max_pages - prefix // PAGE)
            nxt += max_pages - prefix // PAGE
        nkv = np.full(S, max_context, np.uint32)
        gp, gn = dev.to_device(pages), dev.to_device(nkv)
        keep, descs = [gp, gn], []
        for i in range(ncopy):
            k = dev.array((total, Hkv, PAGE, D), np.float32)
            v = dev.array((total, Hkv, PAGE, D), np.float32)
            dev.op("synth_f32", k.ptr, k.nbytes // 4, 100 + i, 1.0)
            dev.op("synth_f32", v.ptr, v.nbytes // 4, 200 + i, 1.0)
            keep += [k, v]
            descs.append(H.PagedKV(k.ptr, v.ptr, gp.ptr, gn.ptr, S, Hkv, D, max_pages, prefix, max_context))
        q = dev.array((S, Hq, D), np.float32)
        gate = dev.array((S, Hq, D), np.float32)
        dev.op("synth_f32", q.ptr, S * Hq * D, 7, 1.0)
        dev.op("synth_f32", gate.ptr, S * Hq * D, 8, 1.0)
        oq, os_ = dev.array((S, Hq * D), np.int8), dev.array((S, Hq * D // 32), np.float32)
        wsb = H.lib().halo_op_attn_decode_workspace_bytes(C.byref(descs[0]), Hq)
        ws = dev.array(wsb, np.uint8)
        call = lambda d: dev.op("attn_decode_q8", C.byref(d), q.ptr, gate.ptr, None, oq.ptr, os_.ptr, Hq, ws.ptr,
                                wsb)
        # the model's form: from the q | gate, k and v projections (norms, rotation and the K / V append inside)
        qg = dev.array((S, Hq, 2 * D), np.float32)
        kin, vin = dev.array((S, Hkv, D), np.float32), dev.array((S, Hkv, D), np.float32)
        wq, wk = dev.array(D, np.float32), dev.array(D, np.float32)
        for a, sd in ((qg, 9), (kin, 10), (vin, 11), (wq, 12), (wk, 13)):
            dev.op("synth_f32", a.ptr, a.nbytes // 4, sd, 1.0)
        step = lambda d: dev.op("attn_decode_step_q8", C.byref(d), qg.ptr, kin.ptr, vin.ptr, wq.ptr, wk.ptr, 64, 1e7,
                                1e-6, None, oq.ptr, os_.ptr, Hq, ws.ptr, wsb)
        dev.sync()
        if args.eager:
            for _ in range(5):
                for d in descs:
                    call(d)
                for d in descs:
                    step(d)
            dev.sync()
            continue
        rows = (prefix + S * suffix) * Hkv
        nbytes = rows * D * 4 * 2
        for key, fn in ((f"S{S}", call), (f"S{S}_step", step)):
            dev.begin_capture()
            for d in descs:
                fn(d)
            g = dev.end_capture()
            dev.launch_graph(g)
            dev.sync()
            nrep = 100
            dev.timer_start()
            for _ in range(nrep):
                dev.launch_graph(g)
            us = dev.timer_stop() * 1e3 / (nrep * ncopy)
            dev.free_graph(g)
            out[key] = {"us_per_layer": round(us, 2), "kv_MB": round(nbytes / 1e6, 1),
                        "GBps": round(nbytes / (us * 1e-6) / 1e9, 1)}
            log(f"[bench] attn {key}: {out[key]}")
        del keep
    res["attn"] = out
    return res


def run_pmc(args, dev, H, res):
    """Eager launches for hardware-counter passes (rocprofv3 --pmc FETCH_SIZE, then WRITE_SIZE): a plain streaming
    read and a copy of C0-sized buffers (the calibration: their algorithmic bytes are known) and the C0 GEMV, each 40
    times over rotated copies (> 600 MB) so that every launch reads HBM."""
    n16 = C0_BYTES // 16
    nbuf = 40
    pool = dev.array(nbuf * n16 * 16, np.uint8)
    dst = dev.array(n16 * 16, np.uint8)
    sink = dev.array(4, np.int32)
    for i in range(nbuf):
        dev.launch("halo_stream_read", (4096,), (256,), [("ptr", pool.ptr + i * n16 * 16), ("u64", n16), sink])
    for i in range(nbuf):
        dev.launch("halo_stream_copy", (4096,), (256,), [("ptr", pool.ptr + i * n16 * 16), dst, ("u64", n16)])
    del pool
    ws0 = _arena_q8(dev, H, nbuf, 4096, 4096, 70000)
    x0 = dev.array(4096, np.float32)
    dev.op("synth_f32", x0.ptr, 4096, 9, 1.0)
    x0q, x0s, y0 = dev.array(4096, np.int8), dev.array(128, np.float32), dev.array(4096, np.float32)
    dev.op("quantize_q8", x0.ptr, x0q.ptr, x0s.ptr, 1, 4096)
    for w in ws0:
        dev.op("matvec_q8a8", ctypes.byref(w.desc), x0q.ptr, x0s.ptr, y0.ptr, 1, 4096)
    dev.sync()
    res["roofline"] = None
    return res


def run_c4(args, dev, H, res):
    """C4: the synthetic hybrid model (48 layers, 36 DeltaNet + 12 GQA, MoE 512 x top-10 + shared, vocab 151936,
    Q8_0 weights seeded on the device). Session 0 prefills the 8192-token shared prefix as one batched prefill
    (timed: prefill tok/s); sessions 1-3 fork its state and share its KV pages. 1 session: session 0 alone, its
    256 suffix tokens prefilled, then 128 greedy decode steps (timed). 4 sessions: the four distinct 256-token
    suffixes prefilled as one ragged batch (timed), then 128 greedy decode steps reading the prefix once per step
    (timed)."""
    P, SUF, DEC = 8192, 256, 128
    t0 = time.perf_counter()
    cfg = H.c4_config(max_sessions=4, prefix_tokens=P, max_context=P + SUF + DEC)
    model = H.Model(dev, cfg, seed=2026)
    dev.sync()
    t_build = time.perf_counter() - t0
    log(f"[bench] c4: weights {model.weight_bytes / 1e9:.1f} GB seeded in {t_build:.1f} s")
    rng = np.random.default_rng(4)
    prefix = rng.integers(0, cfg.vocab, P).astype(np.uint32)
    prompts = [np.concatenate([prefix, rng.integers(0, cfg.vocab, SUF).astype(np.uint32)]) for _ in range(4)]
    try:
        if args.eager:
            # per-kernel timing of eager steps at 1 and 4 sessions (no graph launches, so a kernel tracer can
            # follow it). Only durations matter here: the prefix positions are marked present without running it.
            for s in range(4):
                model.set_session(s, prompts[s], nkv=P + SUF - 1)
            prof = {}
            model.step_eager(1)
            dev.profile_begin()
            for _ in range(10):
                model.step_eager(1)
            prof["S1"] = dev.profile_end()
            model.step_eager(4, P)
            dev.profile_begin()
            for _ in range(10):
                model.step_eager(4, P)
            prof["S4"] = dev.profile_end()
            for k, v in prof.items():
                tot = sum(us for _, us in v.values()) / 10
                log(f"[bench] c4 eager {k}: {tot:.1f} us of kernels per step")
                for name, (n, us) in sorted(v.items(), key=lambda kv: -kv[1][1])[:14]:
                    log(f"    {name:40s} {n // 10:5d}/step {us / 10:9.1f} us/step {us / n:8.2f} us/launch")
            res["c4"] = {"profile": {k: {n: [c, round(u, 1)] for n, (c, u) in v.items()} for k, v in prof.items()}}
            return res
        model.set_session(0, prompts[0])
        dev.sync()
        dev.timer_start()
        model.prefill([(0, 0, P)])
        ms_prefix = dev.timer_stop()
        log(f"[bench] c4: prefix {P} tokens prefilled in {ms_prefix:.1f} ms ({P / (ms_prefix * 1e-3):.0f} tok/s)")
        for s in (1, 2, 3):
            model.fork(0, s)
        # 1 session: its suffix prefilled, then greedy decode
        model.prefill([(0, P, SUF)])
        model.run(1, 1)
        dev.sync()
        dev.timer_start()
        model.run(1, DEC)
        ms1 = dev.timer_stop()
        tok1 = DEC / (ms1 * 1e-3)
        log(f"[bench] c4: 1 session {ms1 / DEC:.3f} ms/token, {tok1:.1f} tok/s")
        # 4 sessions: session 0 back at the end of the prefix (session 1 still holds that state); the four suffixes
        # prefill as one ragged batch reading the shared prefix pages, then greedy decode
        model.fork(1, 0)
        for s in range(4):
            model.set_session(s, prompts[s], nkv=P)
        dev.sync()
        dev.timer_start()
        model.prefill([(s, P, SUF) for s in range(4)])
        ms_suffix = dev.timer_stop()
        log(f"[bench] c4: 4 x {SUF} suffix tokens prefilled in {ms_suffix:.1f} ms "
            f"({4 * SUF / (ms_suffix * 1e-3):.0f} tok/s)")
        model.run(4, 1, prefix=P)
        dev.sync()
        dev.timer_start()
        model.run(4, DEC, prefix=P)
        ms4 = dev.timer_stop()
        tok4 = 4 * DEC / (ms4 * 1e-3)
        log(f"[bench] c4: 4 sessions {ms4 / DEC:.3f} ms/step, {tok4:.1f} tok/s aggregate")
        gen = [model.history(s, P + SUF + DEC)[P + SUF:].tolist()[:8] for s in range(4)]
        res["c4"] = {"decode_tok_s_1_session": round(tok1, 1), "ms_per_token_1_session": round(ms1 / DEC, 3),
                     "decode_tok_s_4_sessions": round(tok4, 1), "ms_per_step_4_sessions": round(ms4 / DEC, 3),
                     "prefix_tokens": P, "suffix_tokens": SUF, "decode_steps": DEC,
                     "prefill_prefix_ms": round(ms_prefix, 1),
                     "prefill_prefix_tok_s": round(P / (ms_prefix * 1e-3), 1),
                     "prefill_4x_suffix_ms": round(ms_suffix, 2),
                     "prefill_4x_suffix_tok_s": round(4 * SUF / (ms_suffix * 1e-3), 1), "weight_GB": round(model.weight_bytes / 1e9, 2),
                     "first_generated": gen}
    finally:
        model.close()
    res["roofline"] = res.get("roofline")
    return res


def run_prefill(args, dev, H, res):
    """C4's ragged prefill without graphs (so a kernel tracer or counter pass follows every launch): session 0
    prefills the 8192-token prefix, sessions 1-3 fork it, then the four 256-token suffixes prefill as one batch.
    Then the prefill-shaped Q8 GEMMs alone (M = 2048 tokens: DeltaNet qkv 2048 -> 8192 and out 4096 -> 2048,
    attention qg 2048 -> 8192), timed with events: achieved int8 TOPS against the 5.0 POPS MFMA peak."""
    import ctypes as C

    P, SUF = 8192, 256
    cfg = H.c4_config(max_sessions=4, prefix_tokens=P, max_context=P + SUF + 8)
    model = H.Model(dev, cfg, seed=2026)
    rng = np.random.default_rng(4)
    prefix = rng.integers(0, cfg.vocab, P).astype(np.uint32)
    prompts = [np.concatenate([prefix, rng.integers(0, cfg.vocab, SUF).astype(np.uint32)]) for _ in range(4)]
    out = {}
    try:
        model.set_session(0, prompts[0])
        dev.sync()
        dev.timer_start()
        model.prefill([(0, 0, P)])
        ms = dev.timer_stop()
        out["prefix_ms"], out["prefix_tok_s"] = round(ms, 1), round(P / (ms * 1e-3), 1)
        for s in (1, 2, 3):
            model.fork(0, s)
        for s in range(4):
            model.set_session(s, prompts[s], nkv=P)
        dev.sync()
        dev.timer_start()
        model.prefill([(s, P, SUF) for s in range(4)])
        ms = dev.timer_stop()
        out["suffix_4x256_ms"], out["suffix_tok_s"] = round(ms, 2), round(4 * SUF / (ms * 1e-3), 1)
    finally:
        model.close()
    log(f"[bench] prefill: {out}")
    out["gemm"] = prefill_gemms(dev, H)
    res["prefill"] = out
    res["roofline"] = None
    return res


def run_pgemm(args, dev, H, res):
    """Only the prefill-shaped Q8 GEMMs of run_prefill (a short program for counter passes)."""
    res["prefill"] = {"gemm": prefill_gemms(dev, H)}
    res["roofline"] = None
    return res


def prefill_gemms(dev, H):
    """The prefill-shaped Q8 GEMMs alone (M = 2048 tokens: DeltaNet qkv 2048 -> 8192 and out 4096 -> 2048, attention
    qg 2048 -> 8192), timed with events: achieved int8 TOPS against the 5.0 POPS MFMA peak."""
    import ctypes as C

    gemms = {}
    M = 2048
    for name, rows, cols in (("gdn_qkv", 8192, 2048), ("gdn_out", 2048, 4096), ("attn_qg", 8192, 2048)):
        w = H.Q8Weights(dev, rows, cols).synth(dev, 31 + rows + cols)
        x = dev.array((M, cols), np.float32)
        dev.op("synth_f32", x.ptr, M * cols, 7, 1.0)
        xq, xs = dev.array((M, cols), np.int8), dev.array((M, cols // 32), np.float32)
        ones = dev.to_device(np.ones(cols, np.float32))  # the norm kernel always reads its weights
        dev.launch("halo_add_rmsnorm_q8", (M,), (256,), [x, None, ones, None, xq, xs, ("u32", cols), ("f32", 1e-6)])
        y = dev.array((M, rows), np.float32)
        for _ in range(3):
            dev.op("matvec_q8a8", C.byref(w.desc), xq.ptr, xs.ptr, y.ptr, M, rows)
        dev.sync()
        n = 20
        dev.timer_start()
        for _ in range(n):
            dev.op("matvec_q8a8", C.byref(w.desc), xq.ptr, xs.ptr, y.ptr, M, rows)
        us = dev.timer_stop() * 1e3 / n
        tops = 2.0 * M * rows * cols / (us * 1e-6) / 1e12
        gemms[name] = {"M": M, "N": rows, "K": cols, "us": round(us, 1), "int8_TOPS": round(tops, 1),
                       "frac_of_5000_TOPS": round(tops / 5000.0, 4)}
        log(f"[bench] prefill gemm {name}: {gemms[name]}")
    return gemms


def run_gdn(args, dev, H, res):
    """C3: Gated DeltaNet decode (S = 4 sessions, states rotated over > 256 MB) and the ragged chunked prefill
    {37, 512, 2048, 8191} tokens (bf16 inputs, fp32 state)."""
    S, Hv, Hk, D = 4, 32, 16, 128
    out = {}
    copies = 40  # 40 x 8 MiB of state
    states = [dev.array((S, Hv, D, D), np.float32) for _ in range(copies)]
    for i, st in enumerate(states):
        dev.op("synth_f32", st.ptr, S * Hv * D * D, 100 + i, 0.05)
    q, k = dev.array((S, Hk, D), np.float32), dev.array((S, Hk, D), np.float32)
    v, o = dev.array((S, Hv, D), np.float32), dev.array((S, Hv, D), np.float32)
    g, b = dev.array((S, Hv), np.float32), dev.array((S, Hv), np.float32)
    for i, a in enumerate((q, k, v)):
        dev.op("synth_f32", a.ptr, a.nbytes // 4, 200 + i, 0.09)
    dev.op("synth_f32", g.ptr, S * Hv, 210, 0.1)
    dev.op("synth_f32", b.ptr, S * Hv, 211, 0.1)
    dev.sync()
    dev.begin_capture()
    for st in states:
        dev.op("gdn_decode", st.ptr, q.ptr, k.ptr, v.ptr, g.ptr, b.ptr, o.ptr, S, Hv, Hk, D)
    gr = dev.end_capture()
    dev.launch_graph(gr)
    dev.sync()
    dev.timer_start()
    for _ in range(25):
        dev.launch_graph(gr)
    ms = dev.timer_stop()
    dev.free_graph(gr)
    us = ms * 1e3 / (25 * copies)
    nbytes = 2 * S * Hv * D * D * 4 + S * (2 * Hk + 2 * Hv) * D * 4 + 2 * S * Hv * 4
    out["decode_S4"] = {"us_per_step": round(us, 3), "GBps": round(nbytes / (us * 1e-6) / 1e9, 1)}
    del states
    # prefill
    seqlens = [37, 512, 2048, 8191]
    T = sum(seqlens)
    L = H.lib()
    sl = np.array(seqlens, np.uint32)
    nch = L.halo_gdn_chunk_table(sl.ctypes.data, len(seqlens), None, None)
    chunks = np.zeros((nch, 3), np.uint32)
    seqs = np.zeros((len(seqlens), 2), np.uint32)
    L.halo_gdn_chunk_table(sl.ctypes.data, len(seqlens), chunks.ctypes.data, seqs.ctypes.data)
    gch, gsq = dev.to_device(chunks), dev.to_device(seqs)
    rng = np.random.default_rng(0)

    def bf16(x):
        u = np.ascontiguousarray(x, np.float32).view(np.uint32)
        return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    qh = rng.normal(0, 1, (T, Hk, D)).astype(np.float32)
    kh = rng.normal(0, 1, (T, Hk, D)).astype(np.float32)
    qh /= np.linalg.norm(qh, axis=-1, keepdims=True)
    kh /= np.linalg.norm(kh, axis=-1, keepdims=True)
    pq, pk = dev.to_device(bf16(qh)), dev.to_device(bf16(kh))
    pv = dev.to_device(bf16(rng.normal(0, 1, (T, Hv, D))))
    pg = dev.to_device((-np.log1p(np.exp(rng.normal(0, 1, (T, Hv))))).astype(np.float32))
    pb = dev.to_device((1 / (1 + np.exp(-rng.normal(0, 1, (T, Hv))))).astype(np.float32))
    pst = dev.array((len(seqlens), Hv, D, D), np.float32)
    po = dev.array((T, Hv, D), np.float32)
    ws = dev.array(L.halo_op_gdn_prefill_workspace_bytes(nch, Hv), np.uint8)

    def prefill():
        dev.op("gdn_prefill", pq.ptr, pk.ptr, pv.ptr, pg.ptr, pb.ptr, gch.ptr, gsq.ptr, nch, len(seqlens), pst.ptr,
               po.ptr, Hv, Hk, D, ws.ptr, ws.nbytes)
    prefill()
    dev.sync()
    reps = 5
    dev.timer_start()
    for _ in range(reps):
        prefill()
    ms = dev.timer_stop() / reps
    # per token and value head: 3 d^2 state products and 3 C d chunk terms, 2 flops each
    flops = T * Hv * (3 * D * D + 3 * 64 * D) * 2
    out["prefill_C3"] = {"tokens": T, "ms": round(ms, 3), "tokens_per_s": round(T / (ms * 1e-3)),
                         "TFLOPs": round(flops / (ms * 1e-3) / 1e12, 2)}
    log(f"[bench] gdn {out}")
    res["gdn"] = out
    res["roofline"] = None
    return res


def run_sample(args, dev, H, res):
    """Device sampling latency over C4's vocabulary (N(0, 3) logits), 1 and 4 rows, the common filter sets."""
    V = H.c4_config().vocab
    rng = np.random.default_rng(0)
    configs = {
        "greedy": dict(temperature=0.0),
        "temperature_1": dict(temperature=1.0),
        "top_k40_top_p0.95_T0.7": dict(temperature=0.7, top_k=40, top_p=0.95),
        "top_p0.9_T0.8": dict(temperature=0.8, top_p=0.9),
        "min_p0.05_T1": dict(temperature=1.0, min_p=0.05),
        "penalties64_top_k40": dict(temperature=0.8, top_k=40, repeat_penalty=1.1, frequency_penalty=0.1),
    }
    out = {}
    for rows in (1, 4):
        x = dev.to_device((rng.standard_normal((rows, V)) * 3).astype(np.float32))
        ws = dev.array(H.lib().halo_op_sample_workspace_bytes(rows, V), np.uint8)
        o = dev.array(rows * 16, np.uint8)
        for name, kw in configs.items():
            prm = (H.SampleParams * rows)()
            pen = np.zeros((rows, 64), H.PENALTY_DTYPE)
            for r in range(rows):
                prm[r] = H.SampleParams(top_p=1.0, repeat_penalty=1.0, vocab=V, rng=12345 + r)
                for k, v in kw.items():
                    setattr(prm[r], k, v)
                if "repeat_penalty" in kw:
                    pen[r]["token"] = np.sort(rng.choice(V, 64, replace=False))
                    pen[r]["generated_count"] = 1
                    pen[r]["repeated"] = 1
                    prm[r].n_penalties = 64
            dp = dev.to_device(np.frombuffer(bytes(prm), np.uint8))
            dq = dev.to_device(pen.view(np.uint8).reshape(-1))
            call = lambda: dev.op("sample", x.ptr, rows, V, V, dp.ptr, dq.ptr, 64, o.ptr, ws.ptr, ws.nbytes)
            call()
            dev.sync()
            if args.eager:  # for profilers (rocprofv3 kernel tracing fails inside graph launches)
                for _ in range(50):
                    call()
                dev.sync()
                dp.free()
                dq.free()
                continue
            # 20 calls per graph so the timing is the kernels', not the host's launch path
            dev.begin_capture()
            for _ in range(20):
                call()
            g = dev.end_capture()
            dev.launch_graph(g)
            dev.sync()
            nrep = 20
            dev.timer_start()
            for _ in range(nrep):
                dev.launch_graph(g)
            us = dev.timer_stop() * 1e3 / (nrep * 20)
            dev.free_graph(g)
            out[f"{name}_rows{rows}"] = round(us, 2)
            log(f"[bench] sample {name} rows={rows}: {us:.2f} us")
            dp.free()
            dq.free()
        for a in (x, ws, o):
            a.free()
    res["sample"] = {"vocab": V, "us_per_launch": out}
    res["roofline"] = None
    return res


def run_membw(args, dev, H, res):
    """Streaming-read yardstick: halo_stream_read, one launch per buffer of the given size (buffers rotate over
    >= 600 MB so reads come from HBM), over launch grids; the best grid per size, and a least-squares fit
    time = intercept + bytes / bandwidth over the sizes."""
    out = {}
    sink = dev.array(4, np.int32)
    sizes = [4 << 20, 8 << 20, 16 << 20, C0_BYTES, 32 << 20, 64 << 20, 128 << 20, 256 << 20, 512 << 20]
    pool = dev.array(2 * (512 << 20) + (64 << 20), np.uint8)  # one allocation, carved by offset
    best = {}
    for size in sizes:
        n16 = size // 16
        nbuf = max(2, -(-MIN_ROTATION_BYTES // size))
        step = (size + 4095) // 4096 * 4096
        nbuf = min(nbuf, pool.nbytes // step)
        ptrs = [pool.ptr + i * step for i in range(nbuf)]
        for grid in (1024, 2048, 4096, 8192, 16384):
            if grid * 256 > n16:
                continue
            if args.eager:  # per-launch durations under a profiler: 50 direct launches per (size, grid)
                for i in range(50):
                    dev.launch("halo_stream_read", (grid,), (256,), [("ptr", ptrs[i % nbuf]), ("u64", n16), sink])
                dev.sync()
                continue
            dev.begin_capture()
            for p_ in ptrs:
                dev.launch("halo_stream_read", (grid,), (256,), [("ptr", p_), ("u64", n16), sink])
            g = dev.end_capture()
            dev.launch_graph(g)
            dev.sync()
            nrep = max(2, 2000 // nbuf)
            dev.timer_start()
            for _ in range(nrep):
                dev.launch_graph(g)
            ms = dev.timer_stop()
            us = ms * 1e3 / (nrep * nbuf)
            out[f"{size}B_grid{grid}"] = {"us": round(us, 3), "GBps": round(size / us / 1e3, 1)}
            if size not in best or us < best[size][0]:
                best[size] = (us, grid)
            dev.free_graph(g)
    if args.eager:
        res["membw"] = None
        res["roofline"] = None
        return res
    # an independent ceiling: the runtime's device-to-device copy (hipMemcpyAsync), rotated over buffers beyond the
    # MALL, HIP events on the device stream
    out["memcpy_d2d"] = _memcpy_d2d(dev, [C0_BYTES, 512 << 20])
    xs = np.array(sizes, np.float64)
    ts = np.array([best[z][0] for z in sizes])
    A = np.stack([np.ones_like(xs), xs], 1)
    (icpt, slope), *_ = np.linalg.lstsq(A, ts, rcond=None)
    out["best"] = {str(z): {"us": round(best[z][0], 3), "grid": best[z][1], "GBps": round(z / best[z][0] / 1e3, 1)}
                   for z in sizes}
    out["fit"] = {"intercept_us": round(float(icpt), 3), "GBps_asymptotic": round(1e-3 / float(slope), 1)}
    log(f"[bench] membw best {out['best']} fit {out['fit']}")
    res["membw"] = out
    res["roofline"] = None
    return res


def _memcpy_d2d(dev, sizes):
    """hipMemcpyAsync device-to-device on the device's stream (the HIP runtime the library links), rotated over
    buffers beyond the MALL, HIP events around the copies."""
    hip = ctypes.CDLL("libamdhip64.so")
    hip.hipMemcpyAsync.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int, ctypes.c_void_p]
    hip.hipMemcpyAsync.restype = ctypes.c_int
    stream = dev.stream()
    out = {}
    for size in sizes:
        nbuf = max(2, -(-MIN_ROTATION_BYTES // size))
        step = (size + 65535) // 65536 * 65536
        pool = dev.array(2 * nbuf * step, np.uint8)
        src = [pool.ptr + i * step for i in range(nbuf)]
        dst = [pool.ptr + (nbuf + i) * step for i in range(nbuf)]
        reps = max(nbuf, min(400, (4 << 30) // size))

        def copy(i):
            rc = hip.hipMemcpyAsync(dst[i % nbuf], src[i % nbuf], size, 3, stream)  # hipMemcpyDeviceToDevice
            assert rc == 0, f"hipMemcpyAsync: {rc}"
        for i in range(nbuf):
            copy(i)
        dev.sync()
        dev.timer_start()
        for i in range(reps):
            copy(i)
        us = dev.timer_stop() * 1e3 / reps
        out[str(size)] = {"us": round(us, 3), "read_GBps": round(size / us / 1e3, 1),
                          "read_plus_write_GBps": round(2 * size / us / 1e3, 1), "buffers": nbuf}
        pool.free()
    log(f"[bench] memcpy d2d {out}")
    return out


def _phases_read(dev, H, kind, nb):
    """Per-block phase stamps of kernel family `kind` (0 DeltaNet step, 1 decode attention, 2 RMSNorm-prologue
    projection, 3 MoE gate/up with routing, 4 MoE router, 5 MoE down) of the last launch, in us from the launch's first
    block start: [nb][8] (nb an int: blocks 0 .. nb - 1; else an index array of linear block ids)."""
    buf = np.zeros((6, 4096, 8), np.uint64)
    err = ctypes.create_string_buffer(256)
    if H.lib().halo_read_global(dev.handle, b"halo_phase_timing", buf.ctypes.data, buf.nbytes, err, 256) != 0:
        raise RuntimeError("phase stamps need the timing build: make -C halo-flash_amd timing, then "
                           "HALO_AMD_LIB=halo-flash_amd/libhalo_flash_amd_timing.so")
    t = buf[kind, :nb].astype(np.int64) if isinstance(nb, int) else buf[kind, nb].astype(np.int64)
    return (t - t[:, 0].min()[None]) * 10 / 1000.0 if len(t) else t


def _phases_summary(samples, names):
    """Median over launches of (min, median, max over blocks) per stamp, and the median per-block phase lengths."""
    out = {}
    for i, nm in enumerate(names):
        col = np.array([[r[:, i].min(), np.median(r[:, i]), r[:, i].max()] for r in samples])
        out[nm] = {"min": round(float(np.median(col[:, 0])), 2), "median": round(float(np.median(col[:, 1])), 2),
                   "max": round(float(np.median(col[:, 2])), 2)}
    lens = {}
    for i in range(1, len(names)):
        d = np.array([np.median(r[:, i] - r[:, i - 1]) for r in samples])
        lens[f"{names[i - 1]} -> {names[i]}"] = round(float(np.median(d)), 2)
    return {"stamps_us": out, "phase_us_median_block": lens}


def run_phases(args, dev, H, res):
    """Phase breakdown of two decode kernels with the timing build (HALO_PHASE stamps, 10 ns resolution): the decode
    attention partials at one session over 8576 positions (`halo_attn_decode_partial`, fp32) and at four sessions
    sharing an 8192-token prefix with 384 positions each (`halo_attn_decode_partial_mma`, split-fp16), KV rotated over
    8 pools; and the DeltaNet step of the C4 model (`halo_gdn_step_q8`, the last DeltaNet layer's launch of eager
    steps at 1 and 4 sessions)."""
    import ctypes as C

    out = {}
    Hq, Hkv, D, PAGE, ncopy = 16, 2, 256, 16, 8
    for S, prefix, suffix in ((1, 0, 8576), (4, 8192, 384)):
        max_context = prefix + suffix
        max_pages = -(-max_context // PAGE)
        total = prefix // PAGE + S * (max_pages - prefix // PAGE)
        pages = np.zeros((S, max_pages), np.uint32)
        nxt = prefix // PAGE
        for s_ in range(S):
            pages[s_, : prefix // PAGE] = np.arange(prefix // PAGE)
            pages[s_, prefix // PAGE:] = np.arange(nxt, nxt + max_pages - prefix // PAGE)
            nxt += max_pages - prefix // PAGE
        gp, gn = dev.to_device(pages), dev.to_device(np.full(S, max_context, np.uint32))
        keep, descs = [gp, gn], []
        for i in range(ncopy):
            k = dev.array((total, Hkv, PAGE, D), np.float32)
            v = dev.array((total, Hkv, PAGE, D), np.float32)
            dev.op("synth_f32", k.ptr, k.nbytes // 4, 100 + i, 1.0)
            dev.op("synth_f32", v.ptr, v.nbytes // 4, 200 + i, 1.0)
            keep += [k, v]
            descs.append(H.PagedKV(k.ptr, v.ptr, gp.ptr, gn.ptr, S, Hkv, D, max_pages, prefix, max_context))
        q, gate = dev.array((S, Hq, D), np.float32), dev.array((S, Hq, D), np.float32)
        dev.op("synth_f32", q.ptr, S * Hq * D, 7, 1.0)
        dev.op("synth_f32", gate.ptr, S * Hq * D, 8, 1.0)
        oq, os_ = dev.array((S, Hq * D), np.int8), dev.array((S, Hq * D // 32), np.float32)
        wsb = H.lib().halo_op_attn_decode_workspace_bytes(C.byref(descs[0]), Hq)
        ws = dev.array(wsb, np.uint8)
        nb = Hkv * (prefix // 32 + S * (-(-suffix // 32)))
        samples = []
        for rep in range(40):
            dev.op("attn_decode_q8", C.byref(descs[rep % ncopy]), q.ptr, gate.ptr, None, oq.ptr, os_.ptr, Hq, ws.ptr,
                   wsb)
            dev.sync()
            if rep >= 8:
                samples.append(_phases_read(dev, H, 1, nb))
        if S == 1:  # halo_attn_decode_partial (fp32 VALU)
            names = ["start", "queries in LDS (K, V arrived)", "scores", "softmax", "end (weighted V stored)"]
            cols = [0, 1, 2, 3, 4]
        else:  # halo_attn_decode_partial_mma (split-fp16 matrix cores)
            names = ["start", "queries in LDS", "K halves in LDS (K arrived)", "scores",
                     "softmax + V halves in LDS", "end (weighted V stored)"]
            cols = [0, 1, 2, 3, 5, 4]
        out[f"attn_partial_S{S}"] = dict(blocks=nb, kernel="halo_attn_decode_partial" + ("" if S == 1 else "_mma"),
                                         **_phases_summary([r_[:, cols] for r_ in samples], names))
        # the model's form: from the q | gate, k and v projections (norms, rotation, K / V append in the prologue)
        qg = dev.array((S, Hq, 2 * D), np.float32)
        kin, vin = dev.array((S, Hkv, D), np.float32), dev.array((S, Hkv, D), np.float32)
        wq, wk = dev.array(D, np.float32), dev.array(D, np.float32)
        for a, sd in ((qg, 9), (kin, 10), (vin, 11), (wq, 12), (wk, 13)):
            dev.op("synth_f32", a.ptr, a.nbytes // 4, sd, 1.0)
        samples = []
        for rep in range(40):
            dev.op("attn_decode_step_q8", C.byref(descs[rep % ncopy]), qg.ptr, kin.ptr, vin.ptr, wq.ptr, wk.ptr, 64,
                   1e7, 1e-6, None, oq.ptr, os_.ptr, Hq, ws.ptr, wsb)
            dev.sync()
            if rep >= 8:
                samples.append(_phases_read(dev, H, 1, nb))
        names[1] = "queries normed in LDS" + (" (K, V arrived)" if S == 1 else "")
        out[f"attn_step_S{S}"] = dict(blocks=nb, kernel="halo_attn_decode_partial_qk" + ("2" if S == 1 else ""),
                                      **_phases_summary([r_[:, cols] for r_ in samples], names))
        del keep, ws
    cfg = H.c4_config(max_sessions=4, prefix_tokens=0, max_context=64)
    model = H.Model(dev, cfg, seed=5)
    try:
        rng = np.random.default_rng(0)
        for S in (1, 4):
            model.reset()
            for s_ in range(S):
                model.set_session(s_, rng.integers(0, cfg.vocab, 16).astype(np.uint32))
            samples, extra = [], {2: [], 3: [], 4: [], 5: []}
            # the last layer (attention: q|gate + k + v = 9216 rows, 64 per block) input projection, and the last
            # MoE layer's router (129 blocks) and gate/up blocks of the 10 routed slots (grid 11 x 128)
            nbs = {2: 144, 3: np.array([x + 11 * y for y in range(128) for x in range(10)]), 4: 129, 5: 256}
            for rep in range(12):
                model.step_eager(S)
                dev.sync()
                if rep >= 2:
                    samples.append(_phases_read(dev, H, 0, S * cfg.gdn_v_heads))
                    if S == 1:
                        for k_ in extra:
                            extra[k_].append(_phases_read(dev, H, k_, nbs[k_]))
            if S == 1:
                out["proj_n_S1"] = dict(kernel="halo_proj_q8w_l32_t4", blocks=144, **_phases_summary(
                    extra[2], ["start", "prologue (x arrived, norm, quantized to LDS)", "barrier (all weights issued)", "task 0 dot "
                               "(its weights arrived)", "end (4 tasks stored)"]))
                out["moe_gate_up_S1"] = dict(kernel="halo_moe_gate_up_topk_q8_s2_e512", blocks=1280, **_phases_summary(
                    [r_[:, [0, 5, 6, 7, 1, 2, 3, 4]] for r_ in extra[3]],
                    ["start", "softmax (logits arrived)", "threshold", "candidates in LDS", "wave 0 ranked the logits",
                     "barrier", "dot (weights arrived)", "end"]))
                out["moe_down_S1"] = dict(kernel="halo_moe_down_q8", blocks=256, **_phases_summary(
                    extra[5], ["start", "h loaded, expert rows issued", "dots (rows arrived)", "barrier",
                               "end (combined rows stored)"]))
                out["moe_router_S1"] = dict(kernel="halo_moe_router_n1_h2048", blocks=129, **_phases_summary(
                    extra[4], ["start", "sums of squares (x and weights arrived)", "x in LDS", "end"]))
            out[f"gdn_step_S{S}"] = dict(blocks=S * cfg.gdn_v_heads, **_phases_summary(
                samples, ["start", "conv + gates (state, prologue arrived)", "q / k norms", "u = S^T k",
                          "delta", "update + o (state stored)", "o norm", "end (codes stored)"]))
    finally:
        model.close()
    for k_, v_ in out.items():
        log(f"[bench] phases {k_}: {json.dumps(v_)}")
    res["phases"] = out
    res["roofline"] = None
    return res


class _ArenaView:
    """A window [off, off + nbytes) of one device allocation, with the DeviceArray calls the bench uses."""

    def __init__(self, arena, off, shape, dtype):
        self.arena, self.off, self.shape, self.dtype = arena, off, shape, np.dtype(dtype)
        self.nbytes = int(np.prod(shape)) * self.dtype.itemsize

    def download(self):
        return self.arena.download_range(self.off, int(np.prod(self.shape)), self.dtype).reshape(self.shape)

    @property
    def ptr(self):
        return self.arena.ptr + self.off

    def download_range(self, offset, count, dtype=None):
        return self.arena.download_range(self.off + offset, count, dtype or self.dtype)


def _arena_q8(dev, H, n, rows, cols, seed0):
    """n seeded Q8_0 copies carved out of one device allocation (as a model's weights sit in large arenas)."""
    qb, db = rows * cols, rows * (cols // 32) * 2
    step = -(-(qb + db) // (1 << 21)) * (1 << 21)
    arena = dev.array(n * step, np.uint8)
    out = []
    for i in range(n):
        w = H.Q8Weights.__new__(H.Q8Weights)
        w.rows, w.cols, w.qstride = rows, cols, cols
        w.qs = _ArenaView(arena, i * step, (rows, cols), np.int8)
        w.d = _ArenaView(arena, i * step + qb, (rows, cols // 32), np.uint16)
        w.desc = H.Q8Matrix(w.qs.ptr, w.d.ptr, rows, cols, cols, 0)
        w._arena = arena
        w.synth(dev, seed=seed0 + i)
        out.append(w)
    return out


def run_c0(args, dev, H, res):
    """C0, the headline: exactly args.steps GEMVs timed (after args.warmup untimed), weights rotated over copies."""
    c0_copies = max(2, -(-MIN_ROTATION_BYTES // q8_bytes(4096, 4096)))
    # the copies sit in one allocation at 2 MB boundaries, as a model's weights sit in large arenas (separately
    # allocated copies measured about 1% slower: their edge pages are not 2 MB translations)
    ws0 = _arena_q8(dev, H, c0_copies, 4096, 4096, 50000)
    x0 = dev.array(4096, np.float32)
    dev.op("synth_f32", x0.ptr, 4096, 9, 1.0)
    x0q, x0s, y0 = dev.array(4096, np.int8), dev.array(128, np.float32), dev.array(4096, np.float32)
    dev.op("quantize_q8", x0.ptr, x0q.ptr, x0s.ptr, 1, 4096)
    dev.sync()
    # correctness spot check of copy 0 against the oracle before timing anything
    sys.path.insert(0, str(ROOT / "oracle"))
    import oracle_py as O

    dev.op("matvec_q8a8", ctypes.byref(ws0[0].desc), x0q.ptr, x0s.ptr, y0.ptr, 1, 4096)
    qs, d = ws0[0].host()
    want, mag = O.gemv_q8a8(qs, d, *O.quantize(x0.download()))
    assert np.all(np.abs(y0.download() - want) <= 1e-5 * mag + 1e-6), "bench spot check failed"

    def gemv(w, t):
        if t == "nt":
            dev.launch("halo_gemv_q8a8nt_l64_r1_b1", (1024,), (256,),
                       [("ptr", w.qs.ptr), ("ptr", w.d.ptr), x0q, x0s, y0, ("u32", 4096), ("u32", 4096),
                        ("u32", w.qstride), ("u32", 4096)])
        elif t is None:
            dev.op("matvec_q8a8", ctypes.byref(w.desc), x0q.ptr, x0s.ptr, y0.ptr, 1, 4096)
        else:
            dev.op("matvec_q8a8_tiled", ctypes.byref(w.desc), x0q.ptr, x0s.ptr, y0.ptr, 1, 4096, *t)

    # Cache flush between the untimed and the timed launches: one streaming read of 512 MB (twice the 256 MB MALL)
    flush = dev.array(512 << 20, np.uint8)
    sink = dev.array(4, np.int32)
    stamps = dev.array(2, np.uint64)
    khz = dev.wall_clock_khz()

    def flush_caches():
        dev.launch("halo_stream_read", (4096,), (256,), [("ptr", flush.ptr), ("u64", flush.nbytes // 16), sink])

    if args.eager:  # kernel durations under a profiler
        for i in range(args.steps):
            gemv(ws0[i % c0_copies], None)
        dev.sync()
        res.update(value=0.0, steps_timed=args.steps, ms_per_step=0.0, roofline=None)
        return res
    # the stamps' own cost (two stamp launches back to back in one graph), subtracted from every timed region
    dev.begin_capture()
    dev.launch("halo_clock_stamp", (1,), (64,), [stamps, ("u32", 0)])
    dev.launch("halo_clock_stamp", (1,), (64,), [stamps, ("u32", 1)])
    g0 = dev.end_capture()
    over = []
    for _ in range(20):
        dev.launch_graph(g0)
        dev.sync()
        st = stamps.download()
        over.append(float(st[1] - st[0]) / khz)
    dev.free_graph(g0)
    stamp_ms = float(np.median(over))
    tilings = [None] + ([(64, 2, 4), (64, 1, 2), (64, 1, 1), (32, 1, 4), "nt"] if args.sweep else [])
    c0 = {}
    for t in tilings:
        steps = args.steps if t is None else 2000
        warm = args.warmup if t is None else 0
        # One graph: the `warm` untimed warm-up GEMVs on copies 0 .. warm - 1, the timer's start mark (a device
        # wall-clock stamp node), exactly `steps` timed GEMVs from copy `warm` on, the stop mark; so the graph
        # launch's own latency and the hand-over from the warm-up are outside the region (warm-up and timed GEMVs
        # as separate graphs put a graph-to-graph transition at the region's start: 4.88-4.92 -> 4.76-4.87 us per
        # GEMV at 20 steps). The graph is launched once untimed first (a first launch pays the upload), then the
        # caches are flushed: every timed GEMV reads weights that no launch touched since the flush (when warm +
        # steps exceeds the copies, the rotation reuses copies only after more than 600 MB of other reads).
        dev.begin_capture()
        for i in range(warm):
            gemv(ws0[i % c0_copies], t)
        dev.launch("halo_clock_stamp", (1,), (64,), [stamps, ("u32", 0)])
        for i in range(steps):
            gemv(ws0[(warm + i) % c0_copies], t)
        dev.launch("halo_clock_stamp", (1,), (64,), [stamps, ("u32", 1)])
        gt = dev.end_capture()
        dev.launch_graph(gt)  # the first launch (upload) before the flush
        dev.sync()
        # cache flush and the graph queued back to back (no host wait between them, so the device does not idle and
        # clock down before the timed region)
        flush_caches()
        dev.launch_graph(gt)
        dev.sync()
        st = stamps.download()
        ms = float(st[1] - st[0]) / khz - stamp_ms
        dev.free_graph(gt)
        us = ms * 1e3 / steps
        c0[str(t)] = {"us_per_gemv": round(us, 4), "GBps": round(C0_BYTES / (us * 1e-6) / 1e9, 1), "steps": steps}
        if t is None:
            res.update(value=C0_BYTES / (us * 1e-6) / 1e9, steps_timed=steps, ms_per_step=us * 1e-3)
    log(f"[bench] C0 {c0}")
    best = c0["None"]
    traffic = None
    prof = ROOT / "profiles" / "gemv_q8a8_c0_4096x4096.md"
    if prof.exists():
        for line in prof.read_text().splitlines():
            if line.startswith("traffic_bytes_per_launch:"):
                traffic = int(line.split(":")[1])
    res["roofline"] = {
        "bound": "hbm",
        "kernel": "halo_gemv_q8a8s_l64_r1_b1 (C0 4096x4096 Q8_0 GEMV)",
        "achieved": best["GBps"],
        "peak": HBM_PEAK_GBS,
        "unit": "GB/s",
        "frac": round(best["GBps"] / HBM_PEAK_GBS, 4),
        "traffic": traffic,
        "traffic_source": "profiles/gemv_q8a8_c0_4096x4096.md (rocprofv3 FETCH_SIZE + WRITE_SIZE, calibrated)",
        "us_per_launch": best["us_per_gemv"],
        "algorithmic_bytes_per_launch": C0_BYTES,
        "timing": ("device wall clock (halo_clock_stamp nodes) around exactly `steps` back-to-back launches, inside "
                   "one graph after the warm-up launches and right after a 512 MB cache flush, less the stamps' own "
                   "time (two stamps back to back, median of 20)"),
        "stamp_overhead_us": round(stamp_ms * 1e3, 3),
    }
    if args.sweep:
        res["c0_tilings"] = c0
    return res


def _median_time(fn, budget_s, min_reps=10, max_reps=2000):
    fn()  # warm-up
    times = []
    t_end = time.perf_counter() + budget_s
    while (time.perf_counter() < t_end or len(times) < min_reps) and len(times) < max_reps:
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return float(np.median(times)), len(times)


def _cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(budget_s: float):
    """The reference's CPU path on the host cores, on bounded samples of the same workloads (median of >= 10 runs
    after a warm-up): the headline C0 GEMV through the reference's cpu::MatVec (built from its sources into
    oracle/_ref; all hardware threads, as MatVec splits rows), and legs: C0 on one thread (the port, bitwise equal to
    cpu::MatVec), the C1 projections, the C2 MoE layer at T=1 (cpu::MatVec router, RouteTopK, 10 routed experts and
    the shared expert through cpu::MatVec) and the C3 DeltaNet recurrence for S=4 sessions (the port's delta rule,
    one thread). GB/s against the same algorithmic bytes as the GPU figures."""
    sys.path.insert(0, str(ROOT / "oracle"))
    import oracle_py as O

    o = O.oracle()
    has_ref = O.has_ref()
    R = O.ref() if has_ref else None
    hw = int(R.ref_hw_threads()) if has_ref else (os.cpu_count() or 1)
    rng = np.random.default_rng(0)

    def raw_q8(r, c, sigma=0.02):
        qs, d = O.synth_q8(rng, r, c, sigma)
        raw = np.zeros(r * (c // 32) * 34, np.uint8)
        o.or_pack_q8_0(qs, d, raw, r, c, c)
        return raw, qs, d

    def matvec(raw, qs, d, r, c, x, y, threads=None):
        if has_ref and threads is None:
            R.ref_matvec_q8_0(raw, r, c, x, y)
        else:
            o.or_matvec_q8_0_f32x(qs, d, r, c, c, x, y, threads or hw)

    legs = {}
    share = budget_s / 5
    # C0, all threads (the headline) and one thread
    raw, qs, d = raw_q8(4096, 4096)
    x = rng.normal(0, 1, 4096).astype(np.float32)
    y = np.empty(4096, np.float32)
    med, n = _median_time(lambda: matvec(raw, qs, d, 4096, 4096, x, y), share)
    head = {"value": round(C0_BYTES / med / 1e9, 2), "unit": "GB/s", "cores": hw,
            "kind": "reference" if has_ref else "port",
            "sample": f"C0 4096x4096 Q8_0 GEMV (fp32 x), median of {n} GEMVs ({med * 1e3:.3f} ms each), {hw} threads"}
    med1, n1 = _median_time(lambda: matvec(raw, qs, d, 4096, 4096, x, y, threads=1), share, max_reps=200)
    legs["c0_1_thread"] = {"GBps": round(C0_BYTES / med1 / 1e9, 2), "ms": round(med1 * 1e3, 3), "cores": 1,
                           "kind": "port (bitwise = cpu::MatVec)", "reps": n1}
    # C1 pass
    mats = [(raw_q8(r, c), r, c) for r, c in C1_SHAPES]
    xs = {2048: rng.normal(0, 1, 2048).astype(np.float32), 4096: rng.normal(0, 1, 4096).astype(np.float32)}

    def c1():
        for (rw, q_, d_), r, c in mats:
            matvec(rw, q_, d_, r, c, xs[c], np.empty(r, np.float32))
    med, n = _median_time(c1, share)
    legs["c1_pass_m1"] = {"GBps": round(c1_pass_bytes(1) / med / 1e9, 2), "ms": round(med * 1e3, 3), "cores": hw,
                          "kind": head["kind"], "reps": n}
    # C2 at T = 1: router + top-10 + 10 routed experts + shared expert (experts built for the ids the token routes
    # to; the timed work is the whole layer)
    E, Hd, F, k = 512, 2048, 512, 10
    router = rng.normal(0, 0.02, (E, Hd)).astype(np.float32)
    sgate = rng.normal(0, 0.02, Hd).astype(np.float32)
    xt = rng.normal(0, 1, Hd).astype(np.float32)
    logits = np.empty(E, np.float32)
    (R.ref_matvec_f32 if has_ref else o.or_matvec_f32)(router, E, Hd, xt, logits)
    ids, wts = np.zeros(k, np.uint32), np.zeros(k, np.float32)
    o.or_route_topk(logits, E, k, ids, wts)
    experts = {int(e): (raw_q8(F, Hd), raw_q8(F, Hd), raw_q8(Hd, F)) for e in ids.tolist() + [-1]}

    def moe():
        lg = np.empty(E, np.float32)
        (R.ref_matvec_f32 if has_ref else o.or_matvec_f32)(router, E, Hd, xt, lg)
        ii, ww = np.zeros(k, np.uint32), np.zeros(k, np.float32)
        (R.ref_route_topk if has_ref else o.or_route_topk)(lg, E, k, ii, ww)
        out = np.zeros(Hd, np.float32)
        for e, wgt in list(zip(ii.tolist(), ww.tolist())) + [(-1, 1.0 / (1.0 + np.exp(-float(sgate @ xt))))]:
            (gr, gq, gd), (ur, uq, ud), (dr, dq, dd) = experts[e]
            g, u, dn = np.empty(F, np.float32), np.empty(F, np.float32), np.empty(Hd, np.float32)
            matvec(gr, gq, gd, F, Hd, xt, g)
            matvec(ur, uq, ud, F, Hd, xt, u)
            h = (g / (1.0 + np.exp(-g)) * u).astype(np.float32)
            matvec(dr, dq, dd, Hd, F, h, dn)
            out += np.float32(wgt) * dn
        return out
    med, n = _median_time(moe, share)
    moe_b = E * Hd * 4 + Hd * 4 + 11 * (2 * q8_bytes(F, Hd) + q8_bytes(Hd, F)) + 2 * Hd * 4
    legs["c2_moe_t1"] = {"GBps": round(moe_b / med / 1e9, 2), "ms": round(med * 1e3, 3), "cores": hw,
                         "kind": head["kind"], "reps": n}
    # C3 recurrence, S = 4 sessions x 32 value heads (16 key heads), d = 128, one thread
    S, Hv, Hk, D = 4, 32, 16, 128
    st = rng.normal(0, 0.05, (S, Hv, D, D)).astype(np.float32)
    q3 = rng.normal(0, 0.09, (S, Hk, D)).astype(np.float32)
    k3 = rng.normal(0, 0.09, (S, Hk, D)).astype(np.float32)
    v3 = rng.normal(0, 1, (S, Hv, D)).astype(np.float32)
    oh = np.empty(D, np.float32)

    def gdn():
        for s_ in range(S):
            for h in range(Hv):
                o.or_gdn_step(st[s_, h], D, q3[s_, h % Hk], k3[s_, h % Hk], v3[s_, h], -0.1, 0.5, oh)
    med, n = _median_time(gdn, share, max_reps=500)
    gdn_b = 2 * S * Hv * D * D * 4 + S * (2 * Hk + 2 * Hv) * D * 4 + 2 * S * Hv * 4
    legs["c3_decode_s4"] = {"GBps": round(gdn_b / med / 1e9, 2), "ms": round(med * 1e3, 3), "cores": 1,
                            "kind": "port (the delta rule of ReferenceModel::LinearAttention)", "reps": n}
    try:
        aff = len(os.sched_getaffinity(0))
    except AttributeError:
        aff = os.cpu_count()
    head["available_cpus"] = aff
    head["nproc"] = os.cpu_count()
    head["cpu_model"] = _cpu_model()
    head["legs"] = legs
    return head


def main():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=2000)
    p.add_argument("--warmup", type=int, default=200)
    p.add_argument("--sweep", action="store_true", help="also time alternative C0 GEMV tilings")
    p.add_argument("--cpu-seconds", type=float, default=20.0)
    p.add_argument("--no-cpu", action="store_true")
    p.add_argument("--quick", action="store_true", help="only the C0 headline and its roofline")
    p.add_argument("--eager", action="store_true", help="launch without graphs (for profiling kernel durations)")
    p.add_argument("--mode", choices=["all", "c0", "c1", "membw", "moe", "gdn", "c4", "pmc", "attn", "proj", "prefill",
                                       "pgemm", "sample", "phases"],
                   default="all",
                   help="c0: only the C0 GEMV loop (for profiling one kernel shape)")
    args = p.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported in this build "
              "(the path runs on one GPU; a sharded version is not built)", file=sys.stderr)
        sys.exit(2)
    res = run_gpu(args)
    if args.mode != "all":
        print(json.dumps({k: res.get(k) for k in ("roofline", "c0_tilings", "c1", "membw", "moe", "gdn", "c4", "attn",
                                                  "proj", "prefill", "sample", "phases")}),
              flush=True)
        return
    line = {
        "metric": "Q8_0 GEMV achieved HBM GB/s; decode tokens/s at 1 and 4 sessions",
        "value": round(res["value"], 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": res["steps_timed"],
        "warmup": args.warmup,
        "ms_per_step": round(res["ms_per_step"], 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (device-seeded Q8_0 weights, N(0,1) activations)",
        "config": {"workload": "C0: one Q8_0 GEMV 4096x4096, x quantized to Q8_0, batch 1 (BASELINE configs[0])",
                   "bytes_per_step": C0_BYTES, "rotated_weight_copies_MiB": 600},
        "roofline": res["roofline"],
    }
    for k in ("c1", "moe", "gdn", "c4", "sample"):
        if k in res:
            line[k] = res[k]
    if "c4" in res:
        line["decode_tok_s"] = {"1_session": res["c4"]["decode_tok_s_1_session"],
                                "4_sessions": res["c4"]["decode_tok_s_4_sessions"]}
    if "c0_tilings" in res:
        line["c0_tilings"] = res["c0_tilings"]
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(args.cpu_seconds)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
