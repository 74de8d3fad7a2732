"""GPU checks of batched prefill (halo_model_prefill) on reduced twins of config C4.

A ragged batch of prompts is prefilled in one call (projections as int8 GEMMs, DeltaNet through the chunked
recurrence, causal attention over the paged cache, grouped MoE) and compared with
  - the host restatement in tests/model_ref.py fed the same tokens one at a time (ReferenceModel's path), and
  - the engine's own token-serial decode steps over the same prompt.
Bars: logits within 3e-2 of max|logits| (the Q8 activation quantizer flip bound of the whole-step parity test; the
prefill path sums the DeltaNet recurrence in chunks rather than token by token), and the produced
token equal unless the reference's top two logits are closer than that.
"""
import numpy as np
import pytest

import halo_amd as H
from model_ref import RefModel

pytestmark = pytest.mark.gpu

BAR = 3e-2


def twin(max_sessions=2, prefix=0, ctx=64):
    """C4's attention grouping (8 query heads per kv head, the shape the prefill attention kernel is built for)."""
    return H.ModelConfig(vocab=2048, hidden=1024, layers=4, attn_interval=4, gdn_k_heads=4, gdn_v_heads=8,
                         gdn_head_dim=128, conv_kernel=4, q_heads=16, kv_heads=2, head_dim=256, rotary_dim=64,
                         n_experts=16, n_used=4, expert_ff=256, shared_ff=256, rope_theta=1e7, rms_eps=1e-6,
                         max_sessions=max_sessions, max_context=ctx, prefix_tokens=prefix)


def rel(got, want):
    return float(np.max(np.abs(got - want))) / float(np.max(np.abs(want)))


def check_token(got, want, what):
    top = np.argsort(want)[::-1]
    if int(np.argmax(got)) != int(top[0]):
        assert want[top[0]] - want[top[1]] <= BAR * np.max(np.abs(want)), f"{what}: argmax differs away from a tie"


def test_ragged_prefill_then_decode_matches_host_reference(dev):
    cfg = twin()
    model = H.Model(dev, cfg, seed=11)
    try:
        rng = np.random.default_rng(4)
        prompts = [rng.integers(0, cfg.vocab, 12).astype(np.uint32), rng.integers(0, cfg.vocab, 9).astype(np.uint32)]
        refs = [RefModel(model, cfg), RefModel(model, cfg)]
        want = []
        for ref, p in zip(refs, prompts):
            for t in p[:-1]:
                w = ref.step(int(t))
            want.append(w)
        model.reset()
        for s, p in enumerate(prompts):
            model.set_session(s, p)
        # every prompt token but the last: the last one is the first decode step's input
        model.prefill([(0, 0, 11), (1, 0, 8)])
        for s in range(2):
            got = model.logits(s)
            err = rel(got, want[s])
            print(f"session {s}: prefill logits error {err:.2e}")
            assert err <= BAR
            check_token(got, want[s], f"session {s} prefill")
        assert model.positions(2).tolist() == [12, 9]
        # decode on from there, both sessions in one batch: the last prompt token, then greedy
        tokens = [int(prompts[0][-1]), int(prompts[1][-1])]
        for i in range(6):
            model.step_eager(2)
            for s in range(2):
                got = model.logits(s)
                w = refs[s].step(tokens[s])
                err = rel(got, w)
                assert err <= BAR, f"session {s} decode step {i}: {err:.2e}"
                check_token(got, w, f"session {s} decode step {i}")
                n = len(prompts[s]) + i
                tokens[s] = int(model.history(s, n + 1)[n])
                assert tokens[s] == int(np.argmax(got))
    finally:
        model.close()


def test_split_prefill_equals_whole_and_token_serial(dev):
    """Prefill in two calls (a chunk boundary inside the DeltaNet scan and the conv taps reaching back into the
    ring) against one call and against decode steps; the conv ring and state carry over between calls."""
    cfg = twin(max_sessions=1, ctx=256)
    model = H.Model(dev, cfg, seed=3)
    try:
        rng = np.random.default_rng(5)
        prompt = rng.integers(0, cfg.vocab, 200).astype(np.uint32)
        n = 150
        model.reset()
        model.set_session(0, prompt)
        for _ in range(n):
            model.step_eager(1)
        serial = model.logits(0)
        model.reset()
        model.set_session(0, prompt)
        model.prefill([(0, 0, n)])
        whole = model.logits(0)
        model.reset()
        model.set_session(0, prompt)
        model.prefill([(0, 0, 66)])
        model.prefill([(0, 66, 1)])
        model.prefill([(0, 67, n - 67)])
        split = model.logits(0)
        e1, e2 = rel(whole, serial), rel(split, whole)
        print(f"whole vs serial {e1:.2e}, split vs whole {e2:.2e}")
        assert e1 <= BAR and e2 <= BAR
        check_token(whole, serial, "whole")
        # the next decode step continues from the prefilled state
        model.step_eager(1)
        after = model.logits(0)
        model.reset()
        model.set_session(0, prompt)
        for _ in range(n + 1):
            model.step_eager(1)
        assert rel(after, model.logits(0)) <= BAR
    finally:
        model.close()


def test_prefill_longer_than_one_batch(dev):
    """2,500 tokens: the call splits into batches of 2,048; the second continues state, ring and cache."""
    cfg = twin(max_sessions=1, ctx=2560)
    model = H.Model(dev, cfg, seed=8)
    try:
        rng = np.random.default_rng(6)
        prompt = rng.integers(0, cfg.vocab, 2510).astype(np.uint32)
        n = 2500
        model.reset()
        model.set_session(0, prompt)
        model.run(1, n)
        serial = model.logits(0)
        model.reset()
        model.set_session(0, prompt)
        model.prefill([(0, 0, n)])
        got = model.logits(0)
        err = rel(got, serial)
        print(f"2500-token prefill vs serial decode {err:.2e}")
        assert err <= BAR
        check_token(got, serial, "long prefill")
        assert model.positions(1).tolist() == [n + 1]
    finally:
        model.close()


def test_prefill_suffixes_after_shared_prefix(dev):
    """Session 0 prefills a 64-token prefix, session 1 forks it, then both suffixes prefill in one ragged batch
    reading the shared prefix pages; against the same procedure done with decode steps."""
    cfg = twin(max_sessions=2, prefix=64, ctx=256)
    model = H.Model(dev, cfg, seed=5)
    try:
        rng = np.random.default_rng(2)
        prefix = rng.integers(0, cfg.vocab, 64).astype(np.uint32)
        a = np.concatenate([prefix, rng.integers(0, cfg.vocab, 40).astype(np.uint32)])
        b = np.concatenate([prefix, rng.integers(0, cfg.vocab, 17).astype(np.uint32)])
        model.reset()
        model.set_session(0, a)
        model.run(1, 64)
        model.fork(0, 1)
        model.set_session(1, b, nkv=64)
        for _ in range(16):
            model.run(2, 1, prefix=64)
        model.run(1, 40 - 17)
        want = [model.logits(0), model.logits(1)]
        model.reset()
        model.set_session(0, a)
        model.prefill([(0, 0, 64)])
        model.fork(0, 1)
        model.set_session(1, b, nkv=64)
        model.prefill([(0, 64, 39), (1, 64, 16)])
        for s in range(2):
            got = model.logits(s)
            err = rel(got, want[s])
            print(f"session {s}: suffix prefill vs decode {err:.2e}")
            assert err <= BAR
            check_token(got, want[s], f"session {s}")
        assert model.positions(2).tolist() == [104, 81]
    finally:
        model.close()
