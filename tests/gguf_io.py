"""A small GGUF writer for tests: metadata of every value type, tensors of any storage type, explicit alignment,
and the model's checkpoint layout (the tensor names halo_model_load_gguf reads)."""
import struct

import numpy as np

U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_SCALAR = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<B", U64: "<Q",
           I64: "<q", F64: "<d"}
GGML_F32, GGML_Q8_0 = 0, 8


def _str(s) -> bytes:
    b = s.encode() if isinstance(s, str) else bytes(s)
    return struct.pack("<Q", len(b)) + b


def _value(ty, v) -> bytes:
    if ty == STRING:
        return _str(v)
    if ty == ARRAY:
        et, items = v
        body = b"".join(_value(et, x) for x in items)
        return struct.pack("<IQ", et, len(items)) + body
    return struct.pack(_SCALAR[ty], v)


def write(meta, tensors, version=3, alignment=32) -> bytes:
    """meta: [(key, type, value)] (arrays: (elem_type, [items])); tensors: [(name, ggml_type, dims, payload bytes)].
    Tensor payloads are laid out in order, each at an offset aligned to `alignment`."""
    head = b"GGUF" + struct.pack("<IQQ", version, len(tensors), len(meta))
    for k, ty, v in meta:
        head += _str(k) + struct.pack("<I", ty) + _value(ty, v)
    offs, off = [], 0
    for _, _, _, payload in tensors:
        offs.append(off)
        off += len(payload)
        off = (off + alignment - 1) // alignment * alignment
    for (name, ty, dims, _), o in zip(tensors, offs):
        head += _str(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        head += struct.pack("<IQ", ty, o)
    pad = (alignment - len(head) % alignment) % alignment
    data = bytearray(off)
    for (_, _, _, payload), o in zip(tensors, offs):
        data[o:o + len(payload)] = payload
    return head + b"\0" * pad + bytes(data)


def q8_blocks(qs: np.ndarray, d: np.ndarray) -> bytes:
    """GGUF Q8_0 rows (per 32 values: fp16 scale bits, then 32 int8) from qs [rows][cols] and d [rows][cols/32]."""
    rows, cols = qs.shape
    nb = cols // 32
    out = np.empty((rows, nb, 34), np.uint8)
    out[:, :, 0:2] = d.astype("<u2").reshape(rows, nb, 1).view(np.uint8)
    out[:, :, 2:] = qs.reshape(rows, nb, 32).view(np.uint8)
    return out.tobytes()


def model_checkpoint(model, cfg, arch="halo_synth") -> bytes:
    """The model's weights (downloaded) as a GGUF checkpoint under the names halo_model_load_gguf reads."""
    tensors = []

    def q8(name, layer, mname, rows=None):
        qs, d = model.tensor(layer, mname)
        if rows is not None:
            qs, d = qs[rows], d[rows]
        tensors.append((name, GGML_Q8_0, [qs.shape[1], qs.shape[0]], q8_blocks(qs, d)))

    def f32(name, layer, mname, dims):
        tensors.append((name, GGML_F32, dims, np.ascontiguousarray(model.tensor(layer, mname), np.float32).tobytes()))

    H, E, F = cfg.hidden, cfg.n_experts, cfg.expert_ff
    q8("token_embd.weight", -1, "embd")
    q8("output.weight", -1, "head")
    f32("output_norm.weight", -1, "out_norm", [H])
    for l in range(cfg.layers):
        b = f"blk.{l}."
        f32(b + "attn_norm.weight", l, "attn_norm", [H])
        f32(b + "post_attention_norm.weight", l, "ffn_norm", [H])
        f32(b + "ffn_gate_inp.weight", l, "router", [H, E])
        f32(b + "ffn_gate_inp_shexp.weight", l, "shared_gate", [H])
        for nm, mn in (("ffn_gate_exps", "gate"), ("ffn_up_exps", "up")):
            qs, d = model.tensor(l, mn)
            tensors.append((b + nm + ".weight", GGML_Q8_0, [H, F, E], q8_blocks(qs, d)))
        qs, d = model.tensor(l, "down")
        tensors.append((b + "ffn_down_exps.weight", GGML_Q8_0, [F, H, E], q8_blocks(qs, d)))
        q8(b + "ffn_gate_shexp.weight", l, "sgate")
        q8(b + "ffn_up_shexp.weight", l, "sup")
        q8(b + "ffn_down_shexp.weight", l, "sdown")
        if (l + 1) % cfg.attn_interval != 0:
            Hv = cfg.gdn_v_heads
            q8(b + "attn_qkv.weight", l, "qkv")
            q8(b + "attn_gate.weight", l, "z")
            q8(b + "ssm_alpha.weight", l, "ab", slice(0, Hv))
            q8(b + "ssm_beta.weight", l, "ab", slice(Hv, 2 * Hv))
            q8(b + "ssm_out.weight", l, "out")
            w = model.tensor(l, "conv_w")
            tensors.append((b + "ssm_conv1d.weight", GGML_F32, [w.shape[1], w.shape[0]], w.tobytes()))
            f32(b + "ssm_a", l, "a", [Hv])
            f32(b + "ssm_dt.bias", l, "dt", [Hv])
            f32(b + "ssm_norm.weight", l, "norm_w", [cfg.gdn_head_dim])
        else:
            q8(b + "attn_q.weight", l, "qg")
            q8(b + "attn_k.weight", l, "k")
            q8(b + "attn_v.weight", l, "v")
            q8(b + "attn_output.weight", l, "o")
            f32(b + "attn_q_norm.weight", l, "q_norm", [cfg.head_dim])
            f32(b + "attn_k_norm.weight", l, "k_norm", [cfg.head_dim])
    p = arch + "."
    meta = [("general.architecture", STRING, arch),
            (p + "block_count", U32, cfg.layers), (p + "embedding_length", U32, H),
            (p + "full_attention_interval", U32, cfg.attn_interval),
            (p + "attention.head_count", U32, cfg.q_heads), (p + "attention.head_count_kv", U32, cfg.kv_heads),
            (p + "attention.key_length", U32, cfg.head_dim), (p + "rope.dimension_count", U32, cfg.rotary_dim),
            (p + "rope.freq_base", F32, cfg.rope_theta), (p + "attention.layer_norm_rms_epsilon", F32, cfg.rms_eps),
            (p + "ssm.conv_kernel", U32, cfg.conv_kernel), (p + "ssm.state_size", U32, cfg.gdn_head_dim),
            (p + "ssm.group_count", U32, cfg.gdn_k_heads), (p + "ssm.time_step_rank", U32, cfg.gdn_v_heads),
            (p + "expert_count", U32, E), (p + "expert_used_count", U32, cfg.n_used),
            (p + "expert_feed_forward_length", U32, F),
            (p + "expert_shared_feed_forward_length", U32, cfg.shared_ff)]
    return write(meta, tensors)
