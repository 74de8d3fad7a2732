"""GPU parity of the whole decode step (config C4's model at reduced depth and width) against the host
restatement in tests/model_ref.py, which composes the oracle's primitives the way ReferenceModel does.

A twin of C4 (4 layers: 3 DeltaNet + 1 GQA, hidden 1024, 16 experts top-4 + shared, vocab 2048) is stepped on the
GPU and on the host from the same state: the first step's logits agree within 1e-5 of max|logits| end to end and the
produced token is the same. Later steps are checked layer by layer, teacher-forced from the GPU's own inputs, in
tests/test_gpu_model_teacher.py (a free-running comparison after the first step would measure Q8 rounding-boundary
flips carried by the recurrent state rather than errors of the step).
"""
import numpy as np
import pytest

import halo_amd as H
from model_ref import RefModel

pytestmark = pytest.mark.gpu


def twin():
    return H.ModelConfig(vocab=2048, hidden=1024, layers=4, attn_interval=4, gdn_k_heads=4, gdn_v_heads=8,
                         gdn_head_dim=128, conv_kernel=4, q_heads=4, kv_heads=2, head_dim=256, rotary_dim=64,
                         n_experts=16, n_used=4, expert_ff=256, shared_ff=256, rope_theta=1e7, rms_eps=1e-6,
                         max_sessions=2, max_context=64, prefix_tokens=0)


def test_first_decode_step_matches_host_reference(dev):
    cfg = twin()
    model = H.Model(dev, cfg, seed=11)
    try:
        ref = RefModel(model, cfg)
        rng = np.random.default_rng(3)
        prompt = rng.integers(0, cfg.vocab, 12).astype(np.uint32)
        model.reset()
        model.set_session(0, prompt)
        model.step_eager(1)
        got = model.logits(0)
        want = ref.step(int(prompt[0]))
        err = float(np.max(np.abs(got - want))) / float(np.max(np.abs(want)))
        assert err <= 1e-5, f"first step: logits off by {err:.2e} of max|logits|"
        assert int(np.argmax(got)) == int(np.argmax(want))
        assert int(model.history(0, 2)[1]) == int(np.argmax(got))
    finally:
        model.close()
