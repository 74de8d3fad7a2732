"""Device sampling (halo_op_sample) against the oracle's restatement of SamplerState::Sample (oracle.c
or_sample_state, itself pinned against the reference's SamplerState in test_oracle_sampling.py).

Inputs follow the reference's device test (tests/gpu/sample_gpu_test.cpp:80-186): quantized logit rows with -inf
holes and an occasional clear winner, every filter, penalty lists, random RNG states, vocabularies from 1 to
248,320; its exact-boundary cases; and rows with no finite logit.

Bars: the RNG state after the draw and the nonzero-probability count equal the oracle's in every case. The token
equals the oracle's, except that a row whose kept set reaches past the 4,096 candidates sorted on chip (fixed-point
weights there) may take a different token when a shift of the uniform by 1e-9 makes the oracle take it (a draw on a
CDF boundary, the reference test's own tolerance), in at most 1% of draws. Two launches agree bit for bit.
"""
import numpy as np
import pytest

import halo_amd as H
import oracle_py as O

pytestmark = pytest.mark.gpu

U53 = 2.0 ** -53


def lcg_logits(V, seed, levels, winner):
    """The reference device test's rows (tests/gpu/sample_gpu_test.cpp:92-100): 0.25 steps over `levels` levels,
    one token in 16 at -inf, optionally one clear winner at 9."""
    x = seed
    out = np.empty(V, np.float32)
    xs = np.empty(V, np.uint64)
    for i in range(V):
        x = (x * 1664525 + 1013904223) & 0xFFFFFFFF
        xs[i] = x
    q = ((xs >> np.uint64(8)) % np.uint64(levels)).astype(np.int64) - levels // 2
    out[:] = 0.25 * q
    if V > 1:
        out[(xs >> np.uint64(28)) == 0] = -np.inf
    if winner:
        out[x % V] = 9.0
    return out, x


def make_case(rng, V):
    x_row, x = lcg_logits(V, int(rng.integers(0, 2**32)), int(rng.integers(1, 41)), bool(rng.integers(0, 2)))
    kw = dict(temperature=float(rng.choice([0.0, 0.2, 0.7, 1.0, 1.8])),
              top_k=int(rng.choice([0, 1, 2, 5, 40, 1000])),
              top_p=float(rng.choice([1.0, 0.95, 0.8, 0.5, 0.1, 0.0])),
              min_p=float(rng.choice([0.0, 0.05, 0.3, 1.0])),
              min_keep=int(rng.integers(0, 5)))
    if rng.integers(0, 2):
        kw.update(top_k=0, top_p=1.0, min_keep=min(kw["min_keep"], 1))
    pen = dict(repeat_penalty=float(rng.choice([1.0, 1.3, 0.7])),
               frequency_penalty=float(rng.choice([0.0, 0.4])), presence_penalty=float(rng.choice([0.0, 0.6, -0.3])))
    hist = []
    for _ in range(int(rng.integers(0, 41))):
        x = (x * 1664525 + 1013904223) & 0xFFFFFFFF
        hist.append((x >> 8) % V)
    n_prompt = int(rng.integers(0, len(hist) + 1))
    pens = O.sample_penalties(np.array(hist[:n_prompt], np.uint32), np.array(hist[n_prompt:], np.uint32),
                              repeat_last_n=int(rng.integers(0, 33)), **pen)
    seed = int(rng.integers(0, 2**64, dtype=np.uint64))
    return x_row, kw, pen, pens, seed


def params(kw, pen, seed):
    return H.SampleParams(temperature=kw["temperature"], top_p=kw["top_p"], min_p=kw["min_p"],
                          repeat_penalty=pen.get("repeat_penalty", 1.0),
                          frequency_penalty=pen.get("frequency_penalty", 0.0),
                          presence_penalty=pen.get("presence_penalty", 0.0), top_k=kw["top_k"],
                          min_keep=kw["min_keep"], rng=seed)


def explained(x, seed, pens, kw, pen, token):
    st = np.uint64(seed)
    v = int(st) or 0x9E3779B97F4A7C15
    v ^= v >> 12
    v ^= (v << 25) & 0xFFFFFFFFFFFFFFFF
    v ^= v >> 27
    u = (((v * 0x2545F4914F6CDD1D) & 0xFFFFFFFFFFFFFFFF) >> 11) * U53
    return any(O.sample_state(x, seed, pens, u=min(max(u + du, 0.0), 1 - 1e-12), **kw, **pen)[0] == token
               for du in (-1e-9, 1e-9))


def run_grid(dev, V, n, seed):
    rng = np.random.default_rng(seed)
    cases = [make_case(rng, V) for _ in range(n)]
    logits = np.stack([c[0] for c in cases])
    prm = [params(c[1], c[2], c[4]) for c in cases]
    pl = [c[3] for c in cases]
    got = H.sample_rows(dev, logits, prm, pl)
    again = H.sample_rows(dev, logits, prm, pl)
    assert got.tobytes() == again.tobytes(), "device sampling is not deterministic"
    tolerated = 0
    for r, (x, kw, pen, pens, s) in enumerate(cases):
        wt, wst, wlive = O.sample_state(x, s, pens, with_live=True, **kw, **pen)
        g = got[r]
        what = f"V={V} row {r} {kw} {pen}"
        if wt == H.SAMPLE_NO_FINITE:
            assert int(g["token"]) == wt and int(g["rng"]) == s, what
            continue
        assert int(g["rng"]) == wst, f"RNG diverges: {what}"
        assert int(g["live"]) == wlive, f"live {int(g['live'])} vs {wlive}: {what}"
        if int(g["token"]) != wt:
            assert explained(x, s, pens, kw, pen, int(g["token"])), f"token {int(g['token'])} vs {wt}: {what}"
            tolerated += 1
    return tolerated, n


@pytest.mark.parametrize("V", [1, 2, 3, 7, 64, 1000, 1025, 5000])
def test_draws_match_oracle(dev, V):
    tolerated, n = run_grid(dev, V, 120, 1000 + V)
    print(f"V={V}: {tolerated} of {n} draws on a CDF boundary")
    assert tolerated == 0 if V <= 4096 else tolerated * 100 <= n


def test_draws_match_oracle_large_vocab(dev):
    tolerated, n = run_grid(dev, 248320, 24, 7)
    print(f"V=248320: {tolerated} of {n} draws on a CDF boundary")
    assert tolerated * 100 <= max(n, 100)


BOUNDARIES = [([1, 1], 1.0, 0.5, 0.0, 0), ([1, 1, 1, 1], 1.0, 0.5, 0.0, 0), ([2, 2, 0], 1.0, 0.0, 0.0, 3),
              ([1, 1, 0], 1.0, 1.0, 1.0, 0), ([1, 1, 0, 1], 0.7, 1.0, 1.0, 2), ([3, 3, 3], 1.0, 1.0 / 3, 0.0, 0)]


@pytest.mark.parametrize("logits,T,top_p,min_p,top_k", BOUNDARIES)
def test_exact_boundaries(dev, logits, T, top_p, min_p, top_k):
    x = np.array(logits, np.float32)
    seeds = [1, 2, 0x9E3779B97F4A7C15, 12345]
    kw = dict(temperature=T, top_p=top_p, min_p=min_p, top_k=top_k, min_keep=0)
    got = H.sample_rows(dev, np.stack([x] * 4), [params(kw, {}, s) for s in seeds])
    for g, s in zip(got, seeds):
        assert (int(g["token"]), int(g["rng"])) == O.sample_state(x, s, **kw)


def test_no_finite_and_bad_params(dev):
    V = 300
    rows = [np.full(V, -np.inf, np.float32), np.full(V, np.nan, np.float32), np.zeros(V, np.float32),
            np.zeros(V, np.float32)]
    rows[1][::2] = np.inf
    kw = dict(temperature=1.0, top_p=0.9, min_p=0.0, top_k=0, min_keep=0)
    prm = [params(kw, {}, 5), params(kw, {}, 6), params(dict(kw, top_p=1.5), {}, 7),
           params(kw, {"repeat_penalty": 0.0}, 8)]
    got = H.sample_rows(dev, np.stack(rows), prm)
    assert [int(g["token"]) for g in got] == [H.SAMPLE_NO_FINITE, H.SAMPLE_NO_FINITE, H.SAMPLE_BAD_PARAMS,
                                              H.SAMPLE_BAD_PARAMS]
    assert [int(g["rng"]) for g in got] == [5, 6, 7, 8]


def test_heavy_ties_topk_and_single_token(dev):
    """Rows of one value (the 4096-candidate cut falls inside a tie: exact radix collection), a single finite
    logit (no draw: the RNG stays), and a top-k row where the k-th value is shared by thousands of tokens."""
    V = 100000
    rng = np.random.default_rng(3)
    flat = np.zeros(V, np.float32)
    one = np.full(V, -np.inf, np.float32)
    one[777] = 2.0
    steps = (rng.integers(0, 3, V) * 0.5).astype(np.float32)
    rows, prm, want = [], [], []
    for x, kw in [(flat, dict(temperature=1.0, top_p=1.0, min_p=0.0, top_k=40, min_keep=0)),
                  (flat, dict(temperature=0.7, top_p=0.9, min_p=0.0, top_k=0, min_keep=0)),
                  (one, dict(temperature=1.0, top_p=0.5, min_p=0.0, top_k=0, min_keep=0)),
                  (steps, dict(temperature=1.0, top_p=1.0, min_p=0.0, top_k=5000, min_keep=0)),
                  (steps, dict(temperature=1.3, top_p=0.97, min_p=0.0, top_k=3000, min_keep=2)),
                  (steps, dict(temperature=1.0, top_p=1.0, min_p=0.5, top_k=0, min_keep=3))]:
        s = int(rng.integers(0, 2**63))
        rows.append(x)
        prm.append(params(kw, {}, s))
        want.append(O.sample_state(x, s, with_live=True, **kw))
    got = H.sample_rows(dev, np.stack(rows), prm)
    for i, (g, w) in enumerate(zip(got, want)):
        assert int(g["rng"]) == w[1] and int(g["live"]) == w[2], (i, g, w)
        if i < 3:
            assert int(g["token"]) == w[0], (i, g, w)
        elif int(g["token"]) != w[0]:
            kw = [dict(top_k=5000, temperature=1.0, top_p=1.0, min_p=0.0, min_keep=0),
                  dict(top_k=3000, temperature=1.3, top_p=0.97, min_p=0.0, min_keep=2),
                  dict(top_k=0, temperature=1.0, top_p=1.0, min_p=0.5, min_keep=3)][i - 3]
            assert explained(rows[i], int(prm[i].rng), None, kw, {}, int(g["token"])), (i, g, w)
