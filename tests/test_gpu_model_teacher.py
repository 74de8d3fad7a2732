"""Teacher-forced, per-layer parity of the decode step (tests/teacher.py) on the reduced twin of C4 and on the full C4
model (48 layers: 36 Gated DeltaNet + 12 GQA, hidden 2048, 512 experts top-10 + shared, vocab 151,936).

Each traced step recomputes every stage of every layer on the host from the GPU's own inputs to that stage (the
residual entering the layer, the quantized activations each projection read, the recurrent state / KV cache before
the step, the routed h rows), so the bars stay at 1e-5 * sum|term| for fp32 outputs and exact for integer work at
every step, with quantizer rounding-boundary flips counted rather than absorbed into a loose end-to-end bound. The
GPU's produced token must be its logits' argmax, which the LM-head check ties to the host's argmax except at
measured near-ties.
"""
import numpy as np
import pytest

import halo_amd as H
from teacher import LayerChecker
from test_gpu_model_oracle import twin

pytestmark = pytest.mark.gpu


def _run(model, cfg, prompt, steps, S=1, trace_every=1):
    chk = LayerChecker(model, cfg)
    model.reset()
    for s in range(S):
        model.set_session(s, prompt[s])
    toks = [int(prompt[s][0]) for s in range(S)]
    for i in range(steps):
        if i % trace_every == 0:
            logits = chk.check_step(S, toks)
        else:
            model.step_eager(S)
            logits = np.stack([model.logits(s) for s in range(S)])
        for s in range(S):
            produced = int(model.history(s, i + 2)[i + 1])
            assert produced == int(np.argmax(logits[s])), f"step {i} session {s}"
            toks[s] = int(prompt[s][i + 1]) if i + 1 < len(prompt[s]) else produced
    return chk.report


def test_twin_every_layer_every_step(dev):
    """20 steps of one session (12 prompt tokens, then greedy), every step traced."""
    cfg = twin()
    model = H.Model(dev, cfg, seed=11)
    try:
        rng = np.random.default_rng(3)
        prompt = [rng.integers(0, cfg.vocab, 12).astype(np.uint32)]
        rep = _run(model, cfg, prompt, 20)
        print(f"twin S=1: {rep.flips} flips and {rep.loose} cancellation-bound codes in {rep.codes} codes; worst error / bar per stage {rep.worst}")
        assert rep.flips <= max(4, rep.codes // 10000)
        assert rep.loose <= max(64, rep.codes // 1000)
    finally:
        model.close()


def test_twin_two_sessions(dev):
    """Two sessions per step (the batched path: separate norm launches, sessions as GEMV columns)."""
    cfg = twin()
    model = H.Model(dev, cfg, seed=12)
    try:
        rng = np.random.default_rng(4)
        prompt = [rng.integers(0, cfg.vocab, 6).astype(np.uint32) for _ in range(2)]
        rep = _run(model, cfg, prompt, 8, S=2)
        print(f"twin S=2: {rep.flips} flips and {rep.loose} cancellation-bound codes in {rep.codes} codes; worst {rep.worst}")
        assert rep.flips <= max(4, rep.codes // 10000)
        assert rep.loose <= max(64, rep.codes // 1000)
    finally:
        model.close()


@pytest.mark.timeout(900)
def test_c4_full_shape_every_layer(dev):
    """The full C4 model: 5 steps of one session (4 prompt tokens, then greedy); steps 0, 2 and 4 traced through all
    48 layers and the 151,936-row LM head."""
    cfg = H.c4_config(max_sessions=1, prefix_tokens=0, max_context=64)
    model = H.Model(dev, cfg, seed=5)
    try:
        rng = np.random.default_rng(8)
        prompt = [rng.integers(0, cfg.vocab, 4).astype(np.uint32)]
        rep = _run(model, cfg, prompt, 5, trace_every=2)
        print(f"C4: {rep.flips} flips and {rep.loose} cancellation-bound codes in {rep.codes} codes; worst error / bar per stage {rep.worst}")
        assert rep.flips <= max(8, rep.codes // 10000)
        assert rep.loose <= max(64, rep.codes // 1000)
    finally:
        model.close()


@pytest.mark.timeout(900)
def test_c4_full_shape_prefill_every_layer(dev):
    """The full C4 model's batched prefill: two sessions' prompts (19 and 12 tokens) in one ragged batch, traced through
    all 48 layers (DeltaNet chunked recurrence, split-fp16 causal attention, grouped MoE over 512 experts) and the LM
    head, each stage against the host restatement from the GPU's own inputs."""
    from teacher import PrefillChecker

    cfg = H.c4_config(max_sessions=2, prefix_tokens=0, max_context=64)
    model = H.Model(dev, cfg, seed=6)
    try:
        rng = np.random.default_rng(12)
        prompts = [rng.integers(0, cfg.vocab, 20).astype(np.uint32), rng.integers(0, cfg.vocab, 13).astype(np.uint32)]
        model.reset()
        for s, p in enumerate(prompts):
            model.set_session(s, p)
        pc = PrefillChecker(model, cfg)
        pc.check_prefill([(0, 0, 19), (1, 0, 12)], prompts)
        rep = pc.report
        print(f"C4 prefill: {rep.flips} flips and {rep.loose} cancellation-bound codes in {rep.codes} codes; worst error / bar per stage {rep.worst}")
        assert rep.flips <= max(8, rep.codes // 10000)
        assert rep.loose <= max(64, rep.codes // 1000)
    finally:
        model.close()


@pytest.mark.timeout(1500)
def test_c4_workload_prefix_fork_suffixes_decode(dev):
    """The C4 workload at its real size: session 0 prefills the 8192-token random prefix in one batch (layers 0
    (DeltaNet) and 3 (attention) traced and checked, every 512th token's stages plus the last, the recurrence over
    all 8192 tokens); sessions 1-3 fork its state and share its KV pages; the four distinct 256-token suffixes
    prefill as one ragged batch (layers 0, 3, 46, 47 and the LM head traced: every 16th token's stages, each
    session's last token, the recurrence over every token); then one 4-session decode step reading the prefix once
    (split-fp16 attention partials over 8448 positions) is checked through all 48 layers, every MoE and the LM head,
    from a recurrent state and KV cache that are checked to be the prefill's outputs."""
    from teacher import PrefillChecker

    P, SUF = 8192, 256
    cfg = H.c4_config(max_sessions=4, prefix_tokens=P, max_context=P + SUF + 16)
    model = H.Model(dev, cfg, seed=2026)
    try:
        rng = np.random.default_rng(4)
        prefix = rng.integers(0, cfg.vocab, P).astype(np.uint32)
        prompts = [np.concatenate([prefix, rng.integers(0, cfg.vocab, SUF).astype(np.uint32)]) for _ in range(4)]
        model.reset()
        model.set_session(0, prompts[0])
        pc = PrefillChecker(model, cfg)
        pc.check_prefill([(0, 0, P)], prompts, layers=[0, 3], sample=list(range(0, P, 512)) + [P - 1])
        print(f"C4 prefix prefill: {pc.report.flips} flips, {pc.report.loose} loose in {pc.report.codes} codes; "
              f"worst {pc.report.worst}", flush=True)
        for s in (1, 2, 3):
            model.fork(0, s)
        for s in range(4):
            model.set_session(s, prompts[s], nkv=P)
        # the forks: every session holds session 0's DeltaNet state and conv ring, and the same prefix pages
        pages = model.raw(-1, "pages", np.uint32)
        assert all(np.array_equal(pages[s, :P // 16], pages[0, :P // 16]) for s in range(4)), "prefix pages"
        for l in (0, 1, 46):
            st = model.raw(l, "state").reshape(cfg.max_sessions, -1)
            ring = model.raw(l, "conv_ring").reshape(cfg.max_sessions, -1)
            assert all(np.array_equal(st[s], st[0]) and np.array_equal(ring[s], ring[0]) for s in range(4)), l
        pc2 = PrefillChecker(model, cfg)
        layers = [0, 3, 46, 47, -1]
        rows = list(range(0, 4 * SUF, 16)) + [SUF * (s + 1) - 1 for s in range(4)]
        pc2.check_prefill([(s, P, SUF) for s in range(4)], prompts, layers=layers, sample=rows)
        rep = pc2.report
        print(f"C4 suffix prefill: {rep.flips} flips, {rep.loose} loose in {rep.codes} codes; worst {rep.worst}",
              flush=True)
        # the decode step feeds each session's prefill token (its logits' argmax) at position P + SUF
        toks = [int(model.history(s, P + SUF + 1)[P + SUF]) for s in range(4)]
        for s in range(4):
            assert toks[s] == int(np.argmax(model.logits(s))), f"prefill token of session {s}"
        chk = LayerChecker(model, cfg)
        before = chk.snapshot(4, layers={0, 3, 46, 47})
        for l in (0, 46):
            assert np.array_equal(before[(l, "state")], pc2.after[(l, "state")]), f"state L{l} changed after prefill"
        for l in (3, 47):
            assert np.array_equal(before[(l, "k_pool")], pc2.after[(l, "k_pool")]), f"K cache L{l}"
            assert np.array_equal(before[(l, "v_pool")], pc2.after[(l, "v_pool")]), f"V cache L{l}"
        assert before["nkv"].tolist() == [P + SUF + 1] * 4
        logits = chk.check_step(4, toks, prefix=P)
        for s in range(4):
            produced = int(model.history(s, P + SUF + 2)[P + SUF + 1])
            assert produced == int(np.argmax(logits[s])), f"decode token of session {s}"
        rep = chk.report
        print(f"C4 4-session decode step: {rep.flips} flips, {rep.loose} loose in {rep.codes} codes; "
              f"worst {rep.worst}", flush=True)
        for r_ in (pc.report, pc2.report, chk.report):
            assert r_.flips <= max(8, r_.codes // 10000)
            assert r_.loose <= max(64, r_.codes // 1000)
    finally:
        model.close()
