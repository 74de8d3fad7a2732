"""GPU checks of the hybrid decode step (halo_model) on a reduced twin of config C4.

Internal consistency (each operator has its own oracle parity test): a batched step equals single-session steps
token for token; a session forked after a shared prefix equals one that ran the whole prompt alone; graph replay
equals eager launches.
"""
import numpy as np
import pytest

import halo_amd as H

pytestmark = pytest.mark.gpu


def twin(max_sessions=2, prefix=64, ctx=256):
    return H.ModelConfig(vocab=2048, hidden=1024, layers=4, attn_interval=4, gdn_k_heads=4, gdn_v_heads=8,
                         gdn_head_dim=128, conv_kernel=4, q_heads=4, kv_heads=2, head_dim=256, rotary_dim=64,
                         n_experts=16, n_used=4, expert_ff=256, shared_ff=256, rope_theta=1e7, rms_eps=1e-6,
                         max_sessions=max_sessions, max_context=ctx, prefix_tokens=prefix)


@pytest.fixture(scope="module")
def model(dev):
    m = H.Model(dev, twin(), seed=5)
    yield m
    m.close()


def test_graph_equals_eager_and_batch_equals_single(dev, model):
    rng = np.random.default_rng(1)
    prompt = rng.integers(0, 2048, 40).astype(np.uint32)
    n = 60
    model.reset()
    model.set_session(0, prompt)
    for _ in range(n):
        model.step_eager(1)
    eager = model.history(0, n + 1)
    model.reset()
    model.set_session(0, prompt)
    model.run(1, n)
    graph = model.history(0, n + 1)
    assert np.array_equal(eager, graph)
    model.reset()
    model.set_session(0, prompt)
    model.set_session(1, prompt)
    model.run(2, n)
    assert np.array_equal(model.history(0, n + 1), graph) and np.array_equal(model.history(1, n + 1), graph)
    assert model.positions(2).tolist() == [n + 1, n + 1]


def test_fork_after_shared_prefix(dev, model):
    rng = np.random.default_rng(2)
    prefix = rng.integers(0, 2048, 64).astype(np.uint32)
    a = np.concatenate([prefix, rng.integers(0, 2048, 20).astype(np.uint32)])
    b = np.concatenate([prefix, rng.integers(0, 2048, 7).astype(np.uint32)])
    steps = 40
    # reference runs: each session alone from position 0
    model.reset()
    model.set_session(0, a)
    model.run(1, 64 + steps)
    ha = model.history(0, 64 + steps + 1)
    model.reset()
    model.set_session(0, b)
    model.run(1, 64 + steps)
    hb = model.history(0, 64 + steps + 1)
    # shared: session 0 runs the prefix, session 1 forks, then both step together reading the prefix once
    model.reset()
    model.set_session(0, a)
    model.run(1, 64)
    model.fork(0, 1)
    model.set_session(1, b, nkv=64)
    model.run(2, steps, prefix=64)
    assert np.array_equal(model.history(0, 64 + steps + 1)[65:], ha[65:])
    assert np.array_equal(model.history(1, 64 + steps + 1)[65:], hb[65:])
