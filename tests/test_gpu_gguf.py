"""GPU checks of the GGUF load path (halo_gguf_upload_q8_0, halo_model_load_gguf): a checkpoint written from one
seeded model and loaded into a model of another seed reproduces every weight bit for bit (Q8_0 rows repacked on the
device, fp32 tensors copied) and therefore the same logits; a Q8_0 tensor uploaded in row ranges through a staging
buffer smaller than the tensor equals its host layout; a checkpoint of another shape is refused before anything is
copied."""
import ctypes as C

import numpy as np
import pytest

import gguf_io as W
import halo_amd as H

pytestmark = pytest.mark.gpu


def twin(layers=4):
    return H.ModelConfig(vocab=2048, hidden=1024, layers=layers, attn_interval=4, gdn_k_heads=4, gdn_v_heads=8,
                         gdn_head_dim=128, conv_kernel=4, q_heads=4, kv_heads=2, head_dim=256, rotary_dim=64,
                         n_experts=16, n_used=4, expert_ff=256, shared_ff=256, rope_theta=1e7, rms_eps=1e-6,
                         max_sessions=2, max_context=64, prefix_tokens=0)


NAMES_GDN = ["attn_norm", "ffn_norm", "router", "shared_gate", "gate", "up", "down", "sgate", "sup", "sdown", "qkv",
             "z", "ab", "out", "conv_w", "a", "dt", "norm_w"]
NAMES_ATTN = ["attn_norm", "ffn_norm", "router", "shared_gate", "gate", "up", "down", "sgate", "sup", "sdown", "qg",
              "k", "v", "o", "q_norm", "k_norm"]


def equal(a, b):
    if isinstance(a, tuple):
        return all(np.array_equal(x, y) for x, y in zip(a, b))
    return np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_checkpoint_round_trip_reproduces_weights_and_logits(dev, tmp_path):
    cfg = twin()
    a = H.Model(dev, cfg, seed=11)
    b = H.Model(dev, cfg, seed=99)
    try:
        path = tmp_path / "twin.gguf"
        path.write_bytes(W.model_checkpoint(a, cfg))
        g = H.Gguf(path=path)
        c = g.config(H.ModelConfig(max_sessions=2, max_context=64))
        assert (c.layers, c.hidden, c.vocab, c.n_experts, c.gdn_v_heads) == (4, 1024, 2048, 16, 8)
        assert not equal(a.tensor(0, "qkv"), b.tensor(0, "qkv"))
        b.load_gguf(g)
        g.close()
        for name in ("embd", "head", "out_norm"):
            assert equal(a.tensor(-1, name), b.tensor(-1, name)), name
        for l in range(cfg.layers):
            for name in (NAMES_ATTN if (l + 1) % cfg.attn_interval == 0 else NAMES_GDN):
                assert equal(a.tensor(l, name), b.tensor(l, name)), (l, name)
        rng = np.random.default_rng(1)
        prompt = rng.integers(0, cfg.vocab, 6).astype(np.uint32)
        out = []
        for m in (a, b):
            m.reset()
            m.set_session(0, prompt)
            for _ in range(8):
                m.step_eager(1)
            out.append((m.logits(0), m.history(0, 9)))
        assert np.array_equal(out[0][0], out[1][0]) and np.array_equal(out[0][1], out[1][1])
    finally:
        a.close()
        b.close()


def test_q8_upload_in_row_ranges_through_small_staging(dev):
    rng = np.random.default_rng(5)
    rows, cols, qstride = 300, 1024, 1040
    qs = rng.integers(-127, 128, (rows, cols)).astype(np.int8)
    d = rng.integers(0, 0x3C00, (rows, cols // 32)).astype(np.uint16)
    blob = W.write([], [("w", W.GGML_Q8_0, [cols, 3, 100], W.q8_blocks(qs, d))])
    g = H.Gguf(data=blob)
    t = g.tensor("w")
    dq = dev.array(rows * qstride, np.int8)
    dd = dev.array(rows * (cols // 32), np.uint16)
    st = dev.array(7 * (cols // 32) * 34 + 5, np.uint8)  # 7 rows per copy
    try:
        for r0, n in ((0, 100), (100, 1), (101, 199)):
            H._call("halo_gguf_upload_q8_0", dev.eng, C.byref(t), r0, n, dq.ptr + r0 * qstride,
                    dd.ptr + r0 * (cols // 32) * 2, qstride, st.ptr, st.nbytes)
        got_q = dq.download().reshape(rows, qstride)[:, :cols]
        got_d = dd.download().reshape(rows, cols // 32)
        assert np.array_equal(got_q, qs) and np.array_equal(got_d, d)
        with pytest.raises(H.HaloError, match="outside"):
            H._call("halo_gguf_upload_q8_0", dev.eng, C.byref(t), 250, 51, dq.ptr, dd.ptr, qstride, st.ptr, st.nbytes)
    finally:
        for x in (dq, dd, st):
            x.free()
        g.close()


def test_checkpoint_of_another_shape_is_refused(dev, tmp_path):
    small = twin()
    a = H.Model(dev, small, seed=3)
    other = twin()
    other.expert_ff = 512
    b = H.Model(dev, other, seed=4)
    try:
        before = b.tensor(0, "qkv")
        g = H.Gguf(data=W.model_checkpoint(a, small))
        with pytest.raises(H.HaloError, match="ffn_gate_exps"):
            b.load_gguf(g)
        g.close()
        assert equal(before, b.tensor(0, "qkv"))  # nothing copied
    finally:
        a.close()
        b.close()
