"""The sampler restatement (oracle.c or_sample / or_sample_penalties) against the reference's own sampler
(src/core/sampling.cpp BuildDistribution + Sample, compiled into oracle/_ref): the same token and the same RNG state
after the draw, over seeded random rows and every filter (penalties, top-k, temperature, top-p, min-p, min_keep),
plus the edge rows the reference handles (non-finite logits, ties, a single finite logit).

The RNG is pinned on its own against the published xorshift64* recurrence.
"""
import itertools

import numpy as np
import pytest

import oracle_py as O

pytestmark = pytest.mark.skipif(not O.has_ref(), reason="oracle/_ref (the reference's sampler) not built")


def test_xorshift_recurrence():
    import ctypes as C
    st = C.c_uint64(0)
    # state 0 is replaced by the golden-ratio constant before the shifts
    v = 0x9E3779B97F4A7C15
    for _ in range(5):
        v ^= v >> 12
        v ^= (v << 25) & 0xFFFFFFFFFFFFFFFF
        v ^= v >> 27
        out = (v * 0x2545F4914F6CDD1D) & 0xFFFFFFFFFFFFFFFF
        assert O.oracle().or_next_random(C.byref(st)) == out and st.value == v


CONFIGS = list(itertools.product([0.0, 0.7, 1.3], [0, 1, 5, 40], [1.0, 0.9, 0.5], [0.0, 0.05], [0, 3]))


@pytest.mark.parametrize("T,top_k,top_p,min_p,min_keep", CONFIGS)
def test_sampler_matches_reference(T, top_k, top_p, min_p, min_keep):
    rng = np.random.default_rng(int(T * 10) + top_k * 7 + int(top_p * 100) + int(min_p * 1000) + min_keep)
    for case in range(6):
        V = int(rng.integers(50, 3000))
        x = (rng.normal(0, 2.0, V)).astype(np.float32)
        if case % 3 == 1:
            x = np.round(x * 2) / 2  # ties
        prompt = rng.integers(0, V, 20)
        generated = rng.integers(0, V, int(rng.integers(0, 30)))
        pen = dict(repeat_penalty=1.3, repeat_last_n=16, frequency_penalty=0.2, presence_penalty=0.1) if case % 2 else {}
        seed = int(rng.integers(0, 2**63))
        kw = dict(temperature=T, top_k=top_k, top_p=top_p, min_p=min_p, min_keep=min_keep, prompt=prompt,
                  generated=generated, **pen)
        assert O.sample(x, seed, **kw) == O.ref_sample(x, seed, **kw), (case, V, kw)


def test_sampler_edge_rows():
    rng = np.random.default_rng(9)
    for x in (np.full(100, -np.inf, np.float32),
              np.array([np.nan, 1.0, np.inf, -np.inf, 0.5], np.float32),
              np.zeros(64, np.float32),
              np.array([3.0], np.float32)):
        for T in (0.0, 1.0):
            for top_k in (0, 2):
                seed = int(rng.integers(0, 2**63))
                assert O.sample(x, seed, temperature=T, top_k=top_k) == O.ref_sample(x, seed, temperature=T, top_k=top_k)


# ---- SamplerState (the engine's sampler, the device sampler's contract) ----------------------------------------

def lcg_logits(V, seed, levels, winner):
    """The reference device test's logit rows (tests/gpu/sample_gpu_test.cpp:92-100): quantized to 0.25 steps over
    `levels` levels, one in 16 tokens -inf, optionally one clear winner at 9."""
    x = seed
    out = np.empty(V, np.float32)
    for i in range(V):
        x = (x * 1664525 + 1013904223) & 0xFFFFFFFF
        out[i] = -np.inf if (x >> 28) == 0 and V > 1 else 0.25 * (int((x >> 8) % levels) - levels // 2)
    if winner:
        out[x % V] = 9.0
    return out, x


def state_case(rng, V):
    seed = int(rng.integers(0, 2**32))
    x_row, x = lcg_logits(V, seed, int(rng.integers(1, 41)), bool(rng.integers(0, 2)))
    kw = dict(temperature=float(rng.choice([0.0, 0.2, 0.7, 1.0, 1.8])),
              top_k=int(rng.choice([0, 1, 2, 5, 40, 1000])),
              top_p=float(rng.choice([1.0, 0.95, 0.8, 0.5, 0.1, 0.0])),
              min_p=float(rng.choice([0.0, 0.05, 0.3, 1.0])),
              min_keep=int(rng.integers(0, 5)))
    if rng.integers(0, 2):
        kw.update(top_k=0, top_p=1.0, min_keep=min(kw["min_keep"], 1))
    pen = dict(repeat_penalty=float(rng.choice([1.0, 1.3, 0.7])), repeat_last_n=int(rng.integers(0, 33)),
               frequency_penalty=float(rng.choice([0.0, 0.4])), presence_penalty=float(rng.choice([0.0, 0.6, -0.3])))
    hist = []
    for _ in range(int(rng.integers(0, 41))):
        x = (x * 1664525 + 1013904223) & 0xFFFFFFFF
        hist.append((x >> 8) % V)
    n_prompt = int(rng.integers(0, len(hist) + 1))
    return x_row, kw, pen, np.array(hist[:n_prompt], np.uint32), np.array(hist[n_prompt:], np.uint32)


@pytest.mark.parametrize("V", [1, 2, 3, 7, 64, 1000, 1025, 5000])
def test_sampler_state_matches_reference(V):
    rng = np.random.default_rng(V)
    for _ in range(60 if V < 5000 else 25):
        x, kw, pen, prompt, gen = state_case(rng, V)
        seed = int(rng.integers(0, 2**64, dtype=np.uint64))
        t, st, pens = O.ref_sampler_state(x, seed, prompt=prompt, generated=gen, **kw, **pen)
        pen.pop("repeat_last_n")
        assert O.sample_state(x, seed, pens, **kw, **pen) == (t, st), (V, kw, pen)


def test_sampler_state_large_vocab():
    rng = np.random.default_rng(248320)
    for _ in range(4):
        x, kw, pen, prompt, gen = state_case(rng, 248320)
        seed = int(rng.integers(0, 2**64, dtype=np.uint64))
        t, st, pens = O.ref_sampler_state(x, seed, prompt=prompt, generated=gen, **kw, **pen)
        pen.pop("repeat_last_n")
        assert O.sample_state(x, seed, pens, **kw, **pen) == (t, st), kw


# exact boundaries (tests/gpu/sample_gpu_test.cpp:169-176): cumulative mass exactly at top-p, ties at the min-p cut
BOUNDARIES = [([1, 1], 1.0, 0.5, 0.0, 0), ([1, 1, 1, 1], 1.0, 0.5, 0.0, 0), ([2, 2, 0], 1.0, 0.0, 0.0, 3),
              ([1, 1, 0], 1.0, 1.0, 1.0, 0), ([1, 1, 0, 1], 0.7, 1.0, 1.0, 2), ([3, 3, 3], 1.0, 1.0 / 3, 0.0, 0)]


@pytest.mark.parametrize("logits,T,top_p,min_p,top_k", BOUNDARIES)
def test_sampler_state_exact_boundaries(logits, T, top_p, min_p, top_k):
    for seed in (1, 2, 0x9E3779B97F4A7C15, 12345):
        kw = dict(temperature=T, top_p=top_p, min_p=min_p, top_k=top_k)
        t, st, _ = O.ref_sampler_state(np.array(logits, np.float32), seed, **kw)
        assert O.sample_state(np.array(logits, np.float32), seed, **kw) == (t, st)
