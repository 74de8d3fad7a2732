"""GPU checks of batched prefill (halo_model_prefill) on reduced twins of config C4, teacher-forced per layer.

A ragged batch of prompts is prefilled in one call (projections as int8 GEMMs, DeltaNet through the chunked
recurrence, causal attention over the paged cache, grouped MoE). halo_model_prefill_trace records every layer's
inputs and outputs for all tokens of the batch, and tests/teacher.py (PrefillChecker) recomputes every stage from the
GPU's own inputs of that stage, token by token: fp32 outputs within 1e-5 of their terms' magnitude (the chunked
DeltaNet recurrence is re-run token-serially on the host from the GPU's state before the batch, the magnitudes carried
through it), integer work exact, quantizer rounding-boundary flips counted. Calls that continue earlier ones (split
prompts, batches of 2,048, suffixes after a shared prefix) are each checked from the state the previous call left,
and the decode steps after a prefill are checked the same way (LayerChecker).
"""
import numpy as np
import pytest

import halo_amd as H
from teacher import LayerChecker, PrefillChecker

pytestmark = pytest.mark.gpu


def twin(max_sessions=2, prefix=0, ctx=64, prefill_batch=0, conv_kernel=4):
    """C4's attention grouping (8 query heads per kv head, the shape the prefill attention kernel is built for)."""
    return H.ModelConfig(vocab=2048, hidden=1024, layers=4, attn_interval=4, gdn_k_heads=4, gdn_v_heads=8,
                         gdn_head_dim=128, conv_kernel=conv_kernel, q_heads=16, kv_heads=2, head_dim=256, rotary_dim=64,
                         n_experts=16, n_used=4, expert_ff=256, shared_ff=256, rope_theta=1e7, rms_eps=1e-6,
                         max_sessions=max_sessions, max_context=ctx, prefix_tokens=prefix,
                         prefill_batch=prefill_batch)


def _flips_ok(rep):
    print(f"{rep.flips} flips and {rep.loose} cancellation-bound codes in {rep.codes} codes; worst error / bar per stage {rep.worst}")
    assert rep.flips <= max(4, rep.codes // 10000)
    assert rep.loose <= max(64, rep.codes // 1000)


@pytest.mark.parametrize("conv_kernel", [4, 3, 6])
def test_ragged_prefill_then_decode(dev, conv_kernel):
    """conv_kernel 4 takes the register-row prologue (halo_gdn_prep_prefill_k4), 3 and 6 the general one (6: the
    decode step with the ring slots read in a loop, halo_gdn_step_q8_kn); the 16-token
    prologue block spans both prompts."""
    cfg = twin(conv_kernel=conv_kernel)
    model = H.Model(dev, cfg, seed=11)
    try:
        rng = np.random.default_rng(4)
        prompts = [rng.integers(0, cfg.vocab, 12).astype(np.uint32), rng.integers(0, cfg.vocab, 9).astype(np.uint32)]
        model.reset()
        for s, p in enumerate(prompts):
            model.set_session(s, p)
        pc = PrefillChecker(model, cfg)
        # every prompt token but the last: the last one is the first decode step's input
        pc.check_prefill([(0, 0, 11), (1, 0, 8)], prompts)
        assert model.positions(2).tolist() == [12, 9]
        for s in range(2):
            assert int(model.history(s, len(prompts[s]))[len(prompts[s]) - 1]) == int(np.argmax(model.logits(s)))
        # decode on from there, both sessions in one batch: the last prompt token, then greedy
        lc = LayerChecker(model, cfg)
        lc.report = pc.report
        tokens = [int(prompts[0][-1]), int(prompts[1][-1])]
        for i in range(6):
            logits = lc.check_step(2, tokens)
            for s in range(2):
                n = len(prompts[s]) + i
                tokens[s] = int(model.history(s, n + 1)[n])
                assert tokens[s] == int(np.argmax(logits[s]))
        _flips_ok(pc.report)
    finally:
        model.close()


def test_split_prefill_calls(dev):
    """Prefill in three calls (a chunk boundary inside the DeltaNet scan, a one-token call, the conv taps reaching
    back into the ring); each call is checked from the state the previous one left. The whole prompt in one call
    gives the same bits as itself run twice (deterministic kernels)."""
    cfg = twin(max_sessions=1, ctx=256)
    model = H.Model(dev, cfg, seed=3)
    try:
        rng = np.random.default_rng(5)
        prompt = rng.integers(0, cfg.vocab, 200).astype(np.uint32)
        n = 150
        pc = PrefillChecker(model, cfg)
        model.reset()
        model.set_session(0, prompt)
        for seg in ((0, 0, 66), (0, 66, 1), (0, 67, n - 67)):
            pc.check_prefill([seg], [prompt])
        assert model.positions(1).tolist() == [n + 1]
        lc = LayerChecker(model, cfg)
        lc.report = pc.report
        lc.check_step(1, [int(prompt[n])])
        whole = []
        for _ in range(2):
            model.reset()
            model.set_session(0, prompt)
            model.prefill([(0, 0, n)])
            whole.append(model.logits(0))
        assert whole[0].tobytes() == whole[1].tobytes()
        _flips_ok(pc.report)
    finally:
        model.close()


@pytest.mark.timeout(600)
def test_prefill_longer_than_one_batch(dev):
    """2,100 tokens with a prefill batch of 2,048: halo_model_prefill splits the call into batches of 2,048 and 52;
    the same two batches, traced, are checked layer by layer (the second from the state, ring and cache the first
    left), and the one-call prefill gives the same logits bit for bit."""
    cfg = twin(max_sessions=1, ctx=2176, prefill_batch=2048)
    model = H.Model(dev, cfg, seed=8)
    try:
        rng = np.random.default_rng(6)
        prompt = rng.integers(0, cfg.vocab, 2110).astype(np.uint32)
        n = 2100
        pc = PrefillChecker(model, cfg)
        model.reset()
        model.set_session(0, prompt)
        pc.check_prefill([(0, 0, 2048)], [prompt])
        pc.check_prefill([(0, 2048, n - 2048)], [prompt])
        traced = model.logits(0)
        model.reset()
        model.set_session(0, prompt)
        model.prefill([(0, 0, n)])
        assert model.logits(0).tobytes() == traced.tobytes()
        assert model.positions(1).tolist() == [n + 1]
        _flips_ok(pc.report)
    finally:
        model.close()


def test_prefill_suffixes_after_shared_prefix(dev):
    """Session 0 prefills a 64-token prefix, session 1 forks it, then both suffixes prefill in one ragged batch
    reading the shared prefix pages; both calls checked layer by layer."""
    cfg = twin(max_sessions=2, prefix=64, ctx=256)
    model = H.Model(dev, cfg, seed=5)
    try:
        rng = np.random.default_rng(2)
        prefix = rng.integers(0, cfg.vocab, 64).astype(np.uint32)
        a = np.concatenate([prefix, rng.integers(0, cfg.vocab, 40).astype(np.uint32)])
        b = np.concatenate([prefix, rng.integers(0, cfg.vocab, 17).astype(np.uint32)])
        pc = PrefillChecker(model, cfg)
        model.reset()
        model.set_session(0, a)
        pc.check_prefill([(0, 0, 64)], [a])
        model.fork(0, 1)
        model.set_session(1, b, nkv=64)
        pc.check_prefill([(0, 64, 39), (1, 64, 16)], [a, b])
        assert model.positions(2).tolist() == [104, 81]
        _flips_ok(pc.report)
    finally:
        model.close()
