"""GPU parity for causal GQA attention over a ragged batch of prefill tokens (config C4's attention: 16 q heads,
2 kv heads, head_dim 256, 16-token pages, a prefix shared by the sessions).

Each token (session s, position p) is compared with the oracle's dense softmax attention (reference.cpp:492-527)
over its session's K/V rows 0..p, times sigmoid(gate): within 1e-5 relative to sum|p||v| (fp16 matrix-core products of split
hi / lo operands, fp32 accumulation),
and the Q8 output equal to the quantization of the fp32 output it wrote.
"""
import ctypes

import numpy as np
import pytest

import halo_amd as H
import oracle_py as O
from test_gpu_attn import build, gather, outlier_kv, outlier_q

pytestmark = pytest.mark.gpu
D = 256


@pytest.mark.parametrize("S,prefix,segs,max_context", [
    (1, 0, [(0, 0, 100)], 256),
    (4, 512, [(0, 512, 37), (1, 512, 130), (2, 512, 1), (3, 512, 69), (0, 549, 8)], 512 + 256),
    (1, 0, [(0, 0, 64), (0, 64, 33)], 128),
])
def test_attn_prefill(dev, S, prefix, segs, max_context):
    run_case(dev, S, prefix, segs, max_context)


@pytest.mark.parametrize("qk,v", [(0.1, 1e-3), (2.0, 50.0)])
def test_attn_prefill_operand_magnitudes(dev, qk, v):
    """Small and large operands (q and K scaled by qk, V by v): the split-fp16 products keep the 1e-5 bar relative
    to sum |p| |v| with no absolute slack (V of 1e-3 is below the range whose lo halves an unscaled split keeps normal; the
    split paths scale their operands by powers of two, which covers |V| from about 1e-4 to 255)."""
    run_case(dev, 1, 0, [(0, 0, 70)], 128, qk, v, abs_tol=0.0)


def test_attn_prefill_outlier_channels(dev):
    """|q|, |K| and |V| far above 255 in single channels, the V outliers only on the page of positions 32-47 (the
    second 32-key chunk): query rows and K chunks take smaller power-of-two scales, and the V scale drops at that chunk
    (the accumulators of the rows that saw the first chunk are rescaled); same 1e-5 bar, outputs finite."""
    run_case(dev, 1, 0, [(0, 0, 90)], 128, outliers=True)


def run_case(dev, S, prefix, segs, max_context, qk=1.0, v=1.0, abs_tol=1e-6, outliers=False):
    Hq, Hkv = 16, 2
    rng = np.random.default_rng(S + prefix + len(segs))
    tweak = (lambda k_, v_, p_: outlier_kv(k_, v_, v_pages=[int(p_[0, 2])])) if outliers else None
    desc, g, kp, vp, pages, _ = build(dev, rng, S, Hkv, prefix, [max_context - prefix] * S, max_context, qk, v,
                                      tweak=tweak)
    seg_arr = (H.PrefillSegment * len(segs))()
    first = 0
    toks = []
    for i, (s, start, n) in enumerate(segs):
        seg_arr[i] = H.PrefillSegment(s, start, n, first)
        toks += [(s, start + j) for j in range(n)]
        first += n
    T = len(toks)
    q = (qk * rng.normal(0, 1, (T, Hq, D))).astype(np.float32)
    if outliers:
        outlier_q(q)
    gate = rng.normal(0, 1, (T, Hq, D)).astype(np.float32)
    gq, gg = dev.to_device(q), dev.to_device(gate)
    go = dev.array((T, Hq, D), np.float32)
    goq, gos = dev.array((T, Hq * D), np.int8), dev.array((T, Hq * D // 32), np.float32)
    nbytes = H.lib().halo_op_attn_prefill_workspace_bytes(seg_arr, len(segs))
    ws = dev.array(nbytes, np.uint8)
    dev.op("attn_prefill", ctypes.byref(desc),
           seg_arr, len(segs), gq.ptr, gg.ptr, go.ptr, goq.ptr, gos.ptr, Hq, ws.ptr, nbytes)
    got = go.download()
    assert np.isfinite(got).all()
    o = O.oracle()
    G = Hq // Hkv
    for ti, (s, p) in enumerate(toks):
        n = p + 1
        for h in range(Hq):
            K = np.ascontiguousarray(gather(kp, pages[s], n, h // G))
            V = np.ascontiguousarray(gather(vp, pages[s], n, h // G))
            oh = np.zeros(D, np.float32)
            o.or_attention_head(np.ascontiguousarray(q[ti, h]), K, V, n, D, D, oh)
            sg = 1 / (1 + np.exp(-gate[ti, h].astype(np.float64)))
            sc = K.astype(np.float64) @ q[ti, h] / 16.0
            pr = np.exp(sc - sc.max())
            pr /= pr.sum()
            mag = (pr @ np.abs(V)) * sg
            assert np.all(np.abs(got[ti, h] - oh * sg) <= 1e-5 * mag + abs_tol), f"token {ti} (s {s}, p {p}) head {h}"
    xq, xs = O.quantize(got.reshape(T, Hq * D))
    assert np.array_equal(goq.download(), xq)
    assert np.array_equal(gos.download().view(np.uint32), xs.view(np.uint32))
