"""Reference-named fp32 DeltaNet prefill kernels (halo_gdn_prefill_split, halo_gdn_chunk_prep +
halo_gdn_chunk_scan; src/kernels/core.hip:5925, 6053, 6111), launched by name through the C ABI with the
reference's parameter lists, grids and buffer layout (src/engine/prefill_chunk.cpp:604-645: q, k and v are the
conv output [T][2 Dk + Dv] at offsets 0, Dk and 2 Dk, qk_stride = v_stride = channels; alpha, beta [T][heads];
state [heads][128][128] key-major; out [T][heads * 128] ungated), one sequence per launch, against T steps of the
oracle's delta rule (or_gdn_sequence, reference.cpp:329-364). Bar: every output and final-state element within
1e-5 of the magnitude of the terms it sums (or_gdn_sequence_mag).
"""
import numpy as np
import pytest

import halo_amd as H
import oracle_py as O

pytestmark = pytest.mark.gpu
D = 128


def case(rng, T, Hv, Hk, zero_state):
    Dk, Dv = Hk * D, Hv * D
    C = 2 * Dk + Dv
    conv = rng.normal(0, 1, (T, C)).astype(np.float32)
    for part in (0, Dk):  # q and k heads L2-normalised, as the conv + L2 stage leaves them
        x = conv[:, part:part + Dk].reshape(T, Hk, D)
        x /= np.linalg.norm(x, axis=-1, keepdims=True)
    alpha = rng.normal(0, 1, (T, Hv)).astype(np.float32)
    beta = rng.normal(0, 1, (T, Hv)).astype(np.float32)
    a = (-np.exp(rng.normal(0, 0.5, Hv))).astype(np.float32)
    dt = rng.normal(0, 0.5, Hv).astype(np.float32)
    state = np.zeros((Hv, D, D), np.float32) if zero_state else rng.normal(0, 0.05, (Hv, D, D)).astype(np.float32)
    return conv, alpha, beta, a, dt, state


def oracle(conv, alpha, beta, a, dt, state, Hv, Hk):
    o_ = O.oracle()
    T = conv.shape[0]
    Dk = Hk * D
    g = np.array([[a[h] * o_.or_softplus(float(alpha[t, h] + dt[h])) for h in range(Hv)] for t in range(T)],
                 np.float32).reshape(T, Hv)
    b = np.array([[o_.or_sigmoid(float(beta[t, h])) for h in range(Hv)] for t in range(T)],
                 np.float32).reshape(T, Hv)
    out = np.zeros((T, Hv, D), np.float32)
    omag = np.zeros((T, Hv, D), np.float64)
    st = state.copy()
    smag = np.abs(state).astype(np.float64)
    for h in range(Hv):
        kh = h % Hk
        qh = np.ascontiguousarray(conv[:, kh * D:(kh + 1) * D])
        khd = np.ascontiguousarray(conv[:, Dk + kh * D:Dk + (kh + 1) * D])
        vh = np.ascontiguousarray(conv[:, 2 * Dk + h * D:2 * Dk + (h + 1) * D])
        gh, bh = np.ascontiguousarray(g[:, h]), np.ascontiguousarray(b[:, h])
        S = np.ascontiguousarray(state[h].T)  # value-major for the oracle
        M = np.ascontiguousarray(np.abs(state[h].T).astype(np.float64))
        oh = np.zeros((T, D), np.float32)
        mh = np.zeros((T, D), np.float64)
        o_.or_gdn_sequence(S, D, T, qh.ctypes.data, D, khd.ctypes.data, D, vh.ctypes.data, D, gh.ctypes.data,
                           bh.ctypes.data, 1, oh.ctypes.data, D)
        o_.or_gdn_sequence_mag(M.ctypes.data, D, T, qh.ctypes.data, D, khd.ctypes.data, D, vh.ctypes.data, D,
                               gh.ctypes.data, bh.ctypes.data, 1, mh.ctypes.data, D)
        out[:, h], omag[:, h], st[h], smag[h] = oh, mh, S.T, M.T
    return out, omag, st, smag


def check(got, want, mag, what):
    err = np.abs(got.astype(np.float64) - want)
    bad = err > 1e-5 * mag + 1e-30
    assert not bad.any(), f"{what}: {int(bad.sum())} elements off, worst {np.max(err / (mag + 1e-30)):.3g} x 1e-5"


def run(dev, kernel, conv, alpha, beta, a, dt, state, Hv, Hk):
    T, C = conv.shape
    Dk = Hk * D
    g = {n: dev.to_device(np.ascontiguousarray(x)) for n, x in
         dict(conv=conv, alpha=alpha, beta=beta, a=a, dt=dt, state=state).items()}
    out = dev.array((T, Hv * D), np.float32)
    q_, k_, v_ = ("ptr", g["conv"].ptr), ("ptr", g["conv"].ptr + 4 * Dk), ("ptr", g["conv"].ptr + 8 * Dk)
    tail = [("u32", Hk), ("u32", T), ("u32", C)]
    if kernel == "split":
        dev.launch("halo_gdn_prefill_split", (2, Hv), (256,),
                   [q_, k_, v_, g["alpha"], g["beta"], g["a"], g["dt"], g["state"], out] + tail +
                   [("u32", C), ("u32", Hv * D)])
    else:
        nch = (T + 15) // 16
        prep = dev.array(Hv * nch * 576, np.float32)  # the size the reference engine allocates (gdnprep)
        dev.launch("halo_gdn_chunk_prep", (nch, Hv), (256,),
                   [q_, k_, g["alpha"], g["beta"], g["a"], g["dt"], prep] + tail)
        dev.launch("halo_gdn_chunk_scan", (2, Hv), (256,),
                   [q_, k_, v_, prep, g["state"], out] + tail + [("u32", C), ("u32", Hv * D)])
    return out.download().reshape(T, Hv, D), g["state"].download()


@pytest.mark.parametrize("kernel", ["split", "chunked"])
@pytest.mark.parametrize("lengths,zero", [([1, 15, 16, 17], True), ([37, 300], False), ([2048], False)])
def test_gdn_reference_named_prefill_equals_stepping(dev, kernel, lengths, zero):
    """Ragged lengths (one launch per sequence, partial and whole 16-token chunks, one token), C3's heads
    (32 value heads over 16 key heads); zero and random initial states."""
    Hv, Hk = 32, 16
    for i, T in enumerate(lengths):
        rng = np.random.default_rng(100 * T + i)
        conv, alpha, beta, a, dt, state = case(rng, T, Hv, Hk, zero)
        print(f"{kernel}: T={T} zero_state={zero}", flush=True)
        got_o, got_s = run(dev, kernel, conv, alpha, beta, a, dt, state, Hv, Hk)
        want_o, omag, want_s, smag = oracle(conv, alpha, beta, a, dt, state, Hv, Hk)
        check(got_o, want_o, omag, f"{kernel} T={T} outputs")
        check(got_s, want_s, smag, f"{kernel} T={T} final state")


def test_gdn_reference_named_split_equals_chunked(dev):
    """The one-launch form and the prep + scan pair run the same chunk arithmetic: equal bits."""
    Hv, Hk = 32, 16
    rng = np.random.default_rng(5)
    conv, alpha, beta, a, dt, state = case(rng, 133, Hv, Hk, False)
    o1, s1 = run(dev, "split", conv, alpha, beta, a, dt, state, Hv, Hk)
    o2, s2 = run(dev, "chunked", conv, alpha, beta, a, dt, state, Hv, Hk)
    assert o1.tobytes() == o2.tobytes() and s1.tobytes() == s2.tobytes()
