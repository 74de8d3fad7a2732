"""Device sampling inside the model's decode step (halo_model_set_sampling): each step's drawn token and the RNG
state carried to the next step equal the oracle's SamplerState draw (oracle.c or_sample_state) on that step's
logits, session by session with different parameters and penalty lists; replaying the recorded graph draws the same
sequence as eager steps; temperature 0 through the sampler gives the argmax decode. Bar as in test_gpu_sample.py:
the RNG state always equal, the token equal unless a 1e-9 shift of the uniform explains it (a CDF boundary)."""
import numpy as np
import pytest

import halo_amd as H
import oracle_py as O
from test_gpu_sample import explained

pytestmark = pytest.mark.gpu


def twin():
    return H.ModelConfig(vocab=2048, hidden=1024, layers=4, attn_interval=4, gdn_k_heads=4, gdn_v_heads=8,
                         gdn_head_dim=128, conv_kernel=4, q_heads=4, kv_heads=2, head_dim=256, rotary_dim=64,
                         n_experts=16, n_used=4, expert_ff=256, shared_ff=256, rope_theta=1e7, rms_eps=1e-6,
                         max_sessions=2, max_context=64, prefix_tokens=0)


SESSIONS = [dict(kw=dict(temperature=0.8, top_k=40, top_p=0.95, min_p=0.0, min_keep=0), pen={}, seed=12345),
            dict(kw=dict(temperature=1.5, top_k=0, top_p=1.0, min_p=0.0, min_keep=0),
                 pen=dict(repeat_penalty=1.3, frequency_penalty=0.2, presence_penalty=0.1), seed=0)]


def setup(model, prompts, penalties):
    model.reset()
    for s, p in enumerate(prompts):
        model.set_session(s, p)
    for s, c in enumerate(SESSIONS):
        prm = H.SampleParams(**dict(dict(repeat_penalty=1.0), **c["kw"], **c["pen"]), rng=c["seed"])
        model.set_sampling(s, prm, penalties[s])


def test_step_draws_follow_the_cpu_sampler(dev):
    cfg = twin()
    model = H.Model(dev, cfg, seed=21)
    try:
        rng = np.random.default_rng(8)
        prompts = [rng.integers(0, cfg.vocab, 4).astype(np.uint32), rng.integers(0, cfg.vocab, 3).astype(np.uint32)]
        penalties = [None, O.sample_penalties(prompts[1], np.array([7, 7, 100], np.uint32), repeat_penalty=1.3,
                                              frequency_penalty=0.2, presence_penalty=0.1)]
        setup(model, prompts, penalties)
        states = [c["seed"] for c in SESSIONS]
        tolerated = 0
        for step in range(12):
            model.step_eager(2)
            for s, c in enumerate(SESSIONS):
                x = model.logits(s)
                want, st = O.sample_state(x, states[s], penalties[s], **c["kw"], **c["pen"])
                got = int(model.history(s, step + 2)[step + 1])
                assert model.sample_state(s).rng == st, f"session {s} step {step}: RNG diverges"
                if got != want:
                    assert explained(x, states[s], penalties[s], c["kw"], c["pen"], got), (s, step, got, want)
                    tolerated += 1
                states[s] = st
        assert tolerated <= 1
        eager = [model.history(s, 13) for s in range(2)]
        # the recorded graph draws the same sequence
        setup(model, prompts, penalties)
        model.run(2, 12)
        assert [model.history(s, 13).tolist() for s in range(2)] == [e.tolist() for e in eager]
        assert [model.sample_state(s).rng for s in range(2)] == states
    finally:
        model.close()


def test_temperature_zero_through_the_sampler_is_argmax(dev):
    cfg = twin()
    model = H.Model(dev, cfg, seed=5)
    try:
        prompt = np.arange(5, dtype=np.uint32)
        model.reset()
        model.set_session(0, prompt)
        model.run(1, 10)
        greedy = model.history(0, 11)
        model.reset()
        model.set_session(0, prompt)
        model.set_sampling(0, H.SampleParams(temperature=0.0, top_p=1.0, repeat_penalty=1.0, rng=99))
        model.run(1, 10)
        assert model.history(0, 11).tolist() == greedy.tolist()
        assert model.sample_state(0).rng == 99
    finally:
        model.close()
