"""GPU parity for the Gated DeltaNet recurrence (config C3: 32 value heads, 16 key heads, d = 128).

Decode: several consecutive steps for S = 4 sessions against the oracle's token step (reference.cpp:329-364, S
value-major there, key-major here), state and output within 1e-5 of the oracle relative to the magnitude of the
terms (sum |S| |k|, the reference's bound style); BASELINE's 1e-3 is looser.
"""
import numpy as np
import pytest

import oracle_py as O

pytestmark = pytest.mark.gpu
D = 128


def inputs(rng, S, Hv, Hk):
    q = rng.normal(0, 1, (S, Hk, D)).astype(np.float32)
    k = rng.normal(0, 1, (S, Hk, D)).astype(np.float32)
    q /= np.linalg.norm(q, axis=-1, keepdims=True)
    k /= np.linalg.norm(k, axis=-1, keepdims=True)
    v = rng.normal(0, 1, (S, Hv, D)).astype(np.float32)
    g = (-np.log1p(np.exp(rng.normal(0, 1, (S, Hv))))).astype(np.float32)
    beta = (1 / (1 + np.exp(-rng.normal(0, 1, (S, Hv))))).astype(np.float32)
    return q, k, v, g, beta


def oracle_step(state, q, k, v, g, beta, Hv, Hk):
    """state [S][Hv][i][j] key-major; the oracle works on S[j][i]."""
    S = state.shape[0]
    out = np.zeros((S, Hv, D), np.float32)
    new = state.copy()
    o = O.oracle()
    for s in range(S):
        for h in range(Hv):
            st = np.ascontiguousarray(state[s, h].T)
            oh = np.zeros(D, np.float32)
            o.or_gdn_step(st, D, np.ascontiguousarray(q[s, h % Hk]), np.ascontiguousarray(k[s, h % Hk]),
                          np.ascontiguousarray(v[s, h]), float(g[s, h]), float(beta[s, h]), oh)
            new[s, h] = st.T
            out[s, h] = oh
    return new, out


@pytest.mark.parametrize("S", [1, 4])
def test_gdn_decode_steps(dev, S):
    Hv, Hk = 32, 16
    rng = np.random.default_rng(S)
    state = rng.normal(0, 0.1, (S, Hv, D, D)).astype(np.float32)
    gs = dev.to_device(state)
    want = state
    for step in range(3):
        q, k, v, g, beta = inputs(rng, S, Hv, Hk)
        bufs = [dev.to_device(a) for a in (q, k, v, g, beta)]
        go = dev.array((S, Hv, D), np.float32)
        dev.op("gdn_decode", gs.ptr, bufs[0].ptr, bufs[1].ptr, bufs[2].ptr, bufs[3].ptr, bufs[4].ptr, go.ptr, S, Hv,
               Hk, D)
        want, wo = oracle_step(want, q, k, v, g, beta, Hv, Hk)
        got_s, got_o = gs.download(), go.download()
        smag = np.abs(want).max()
        assert np.allclose(got_s, want, rtol=1e-5, atol=1e-5 * smag), f"state after step {step}"
        omag = np.abs(wo).max()
        assert np.allclose(got_o, wo, rtol=1e-4, atol=1e-5 * omag), f"output of step {step}"
