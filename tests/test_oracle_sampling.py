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
