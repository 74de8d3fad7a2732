"""The GGUF reader (halo_gguf_*) against the reference's GgufReader (src/core/gguf.cpp, compiled into oracle/_ref):
the same images open and the same are refused; for those that open, the same header, tensor table (names, types,
dimensions, offsets, sizes, data positions), metadata values and quantization label. Inputs: writer round trips
with every metadata type, the boundaries the reference tests probe (tests/core/gguf_test.cpp:139-600: alignment,
counts, extents, duplicates, overflowing element counts), and seeded hostile mutations of a valid image. Also the
storage-type size table against quant::EncodedSizeBytes, split checkpoints, and the model configuration read from
metadata. Host code only: no GPU.

Not pinned: the quantization label when two storage types hold exactly the same element count (the reference takes
the first maximum in its hash map's iteration order, which its library does not define); no image here has such a
tie.
"""
import ctypes as C
import struct

import numpy as np
import pytest

import gguf_io as W
import halo_amd as H
import oracle_py as O

needs_ref = pytest.mark.skipif(not O.has_ref(), reason="oracle/_ref (the reference's reader) not built")


def mine(blob: bytes):
    try:
        g = H.Gguf(data=blob)
    except H.HaloError:
        return None, []
    try:
        base = C.addressof(g._buf)
        tensors = [(n, ty, dims, off, sz, addr - base) for n, ty, dims, off, sz, addr in g.tensors()]
        keys = g.keys()
        meta = {k: g.value_text(k) for k in keys}
        return (g.version, g.alignment, g.metadata_count(), tensors, meta, g.label()), keys
    finally:
        g.close()


def same(blob: bytes):
    got, keys = mine(blob)
    want = O.ref_gguf_summary(blob, keys)
    assert (got is None) == (want is None), f"mine {'refuses' if got is None else 'accepts'}, reference differs"
    if got is not None:
        assert got == want
    return got


def sample_image(alignment=32, version=3):
    rng = np.random.default_rng(1)
    meta = [("general.architecture", W.STRING, "halo_synth"), ("general.alignment", W.U32, alignment),
            ("u8", W.U8, 200), ("i8", W.I8, -5), ("u16", W.U16, 60000), ("i16", W.I16, -30000), ("u32", W.U32, 7),
            ("i32", W.I32, -7), ("f32", W.F32, 0.25), ("b", W.BOOL, 1), ("s", W.STRING, "héllo"),
            ("u64", W.U64, 2**63 + 5), ("i64", W.I64, -(2**62)), ("f64", W.F64, -1.5e300),
            ("au32", W.ARRAY, (W.U32, [1, 2, 3])), ("ai32", W.ARRAY, (W.I32, [-1, 2])),
            ("af32", W.ARRAY, (W.F32, [0.5, -2.0])), ("af64", W.ARRAY, (W.F64, [1e-300])),
            ("ab", W.ARRAY, (W.BOOL, [0, 1, 1])), ("as", W.ARRAY, (W.STRING, ["a", "", "xyz"])),
            ("au64", W.ARRAY, (W.U64, [2**64 - 1])), ("ai64", W.ARRAY, (W.I64, [-3])),
            ("au8", W.ARRAY, (W.U8, [1, 2])), ("ai16", W.ARRAY, (W.I16, [-1, 1, 2]))]
    q = rng.integers(-127, 128, (4, 64)).astype(np.int8)
    d = rng.integers(0, 0x3C00, (4, 2)).astype(np.uint16)
    tensors = [("w.q8", W.GGML_Q8_0, [64, 4], W.q8_blocks(q, d)),
               ("w.f32", W.GGML_F32, [3, 2], np.arange(6, dtype=np.float32).tobytes()),
               ("w.f16", 1, [5], bytes(10)), ("w.q4k", 12, [512], bytes(288))]
    return W.write(meta, tensors, version=version, alignment=alignment)


@needs_ref
def test_encoded_bytes_match_reference():
    L = H.lib()
    for ty in range(0, 40):
        for n in (0, 1, 31, 32, 64, 255, 256, 512, 4096 * 3, 2**62, 2**64 - 1, 2**64 - 256):
            assert L.halo_ggml_encoded_bytes(ty, n) == O.ref().ref_encoded_bytes(ty, n), (ty, n)


@needs_ref
@pytest.mark.parametrize("alignment", [32, 64, 1, 4096])
@pytest.mark.parametrize("version", [2, 3])
def test_round_trip_every_value_type(alignment, version):
    got = same(sample_image(alignment, version))
    assert got is not None
    v, a, nm, tensors, meta, label = got
    assert (v, a, nm, len(tensors)) == (version, alignment, 24, 4)
    assert meta[b"u64"] == f"10|u:{2**63 + 5}" and meta[b"as"] == "9|S:3:61,,78797a,"
    assert meta[b"au8"] == "9|u:0"  # 8-bit arrays are skipped, read as 0 (the reference's behaviour)
    g = H.Gguf(data=sample_image(alignment, version))
    t = g.tensor("w.q8")
    assert t.type == W.GGML_Q8_0 and tuple(t.dims[:2]) == (64, 4) and t.size_bytes == 4 * 2 * 34
    u = C.c_uint32()
    assert H.lib().halo_gguf_get_u32(g.h, b"i32", C.byref(u)) != 0  # negative: not a u32
    assert H.lib().halo_gguf_get_u32(g.h, b"u16", C.byref(u)) == 0 and u.value == 60000
    g.close()


def meta_image(entries, tensors=()):
    return W.write(entries, list(tensors))


@needs_ref
def test_boundaries_match_reference():
    f = ("t", W.GGML_F32, [2], bytes(8))
    cases = [
        W.write([], []),                                                   # header only
        W.write([], [])[:23],                                              # 23 bytes
        b"GGUF" + struct.pack("<IQQ", 1, 0, 0),                            # version 1
        b"GGUF" + struct.pack("<IQQ", 4, 0, 0),                            # version 4
        b"GGUX" + struct.pack("<IQQ", 3, 0, 0),                            # magic
        meta_image([("general.alignment", W.U32, 3)], [f]),                # not a power of two
        meta_image([("general.alignment", W.U64, 2**32)], [f]),            # above 2^32 - 1
        meta_image([("general.alignment", W.U8, 16)], [f]),
        meta_image([("general.alignment", W.I32, 32)], [f]),               # signed: refused
        meta_image([("general.alignment", W.BOOL, 1)], [f]),
        meta_image([("k", W.U32, 1), ("k", W.U32, 2)]),                    # duplicate key
        meta_image([("", W.U32, 1)]),                                      # empty key
        meta_image([("b", W.BOOL, 2)]),                                    # bool 2
        meta_image([("a", W.ARRAY, (W.BOOL, [0, 2]))]),
        meta_image([("a", W.ARRAY, (W.ARRAY, []))]),                       # nested array
        meta_image([], [f, f]),                                            # duplicate tensor
        meta_image([], [("q", W.GGML_Q8_0, [48], bytes(34))]),             # not whole blocks
        meta_image([], [("z", W.GGML_F32, [0], b"")]),                     # zero extent
        meta_image([], [("u", 17, [32], bytes(64))]),                      # unknown type
        meta_image([], [("big", W.GGML_F32, [2**62, 8], bytes(8))]),       # element count overflow
        meta_image([], [("n", W.GGML_F32, [1] * 9, bytes(4))]),            # 9 dims
        meta_image([("split.count", W.U32, 0)]),
        meta_image([("x", W.ARRAY, (W.U8, [1, 2, 3]))]),
    ]
    for i, blob in enumerate(cases):
        same(blob)


@needs_ref
def test_hostile_mutations_match_reference():
    base = sample_image()
    rng = np.random.default_rng(7)
    accepted = 0
    for trial in range(1500):
        b = bytearray(base)
        kind = trial % 5
        if kind == 0:  # flip bits in the header region
            for _ in range(int(rng.integers(1, 4))):
                i = int(rng.integers(0, min(len(b), 900)))
                b[i] ^= 1 << int(rng.integers(0, 8))
        elif kind == 1:  # truncate
            b = b[: int(rng.integers(0, len(b)))]
        elif kind == 2:  # overwrite a random 8-byte word with an extreme value
            i = int(rng.integers(0, min(len(b), 900) - 8))
            b[i:i + 8] = struct.pack("<Q", [0, 1, 2**31, 2**32, 2**63, 2**64 - 1, 13, 255][int(rng.integers(0, 8))])
        elif kind == 3:  # inflate a count
            off = 8 + 8 * int(rng.integers(0, 2))
            b[off:off + 8] = struct.pack("<Q", int(rng.integers(0, 2**40)))
        else:  # random bytes spliced in
            i = int(rng.integers(0, min(len(b), 900)))
            b[i:i] = bytes(rng.integers(0, 256, int(rng.integers(1, 9))).astype(np.uint8))
        if same(bytes(b)) is not None:
            accepted += 1
    print(f"{accepted} of 1500 mutated images accepted by both readers")


@needs_ref
def test_quantization_label_matches_reference():
    def img(spec):
        return W.write([], [(f"t{i}", ty, [n], bytes(int(H.lib().halo_ggml_encoded_bytes(ty, n))))
                            for i, (ty, n) in enumerate(spec)])
    for spec in ([], [(8, 4000 * 32 // 32 * 32), (0, 1000)], [(8, 3968), (0, 1000)], [(0, 10), (8, 32), (0, 30)]):
        got = same(img(spec))
        assert got is not None
    assert same(img([(8, 4000 * 32 // 32 * 32), (0, 1000)]))[5] == "Q8_0"
    assert same(img([(8, 3968), (0, 1000)]))[5] == "Q8_0 mixed"
    assert same(img([(0, 10), (8, 32), (0, 30)]))[5] == "F32 mixed"


def test_split_checkpoint_opens_as_one(tmp_path):
    f = lambda name, v: (name, W.GGML_F32, [2], np.array([v, v], np.float32).tobytes())
    common = lambda no: [("general.architecture", W.STRING, "halo_synth"), ("split.count", W.U16, 3),
                         ("split.no", W.U16, no), ("split.tensors.count", W.U64, 4)]
    (tmp_path / "m-00001-of-00003.gguf").write_bytes(W.write(common(0), [f("a", 1.0)]))
    (tmp_path / "m-00002-of-00003.gguf").write_bytes(W.write(common(1), [f("b", 2.0), f("c", 3.0)]))
    (tmp_path / "m-00003-of-00003.gguf").write_bytes(W.write(common(2), [f("d", 4.0)]))
    g = H.Gguf(path=tmp_path / "m-00002-of-00003.gguf")
    assert [t[0] for t in g.tensors()] == [b"a", b"b", b"c", b"d"]
    t = g.tensor("c")
    assert np.frombuffer(C.string_at(t.data, 8), np.float32).tolist() == [3.0, 3.0]
    g.close()
    # a shard that disagrees, a missing shard, a wrong total
    (tmp_path / "m-00003-of-00003.gguf").write_bytes(W.write(common(1), [f("d", 4.0)]))
    with pytest.raises(H.HaloError, match="inconsistent"):
        H.Gguf(path=tmp_path / "m-00001-of-00003.gguf")
    (tmp_path / "m-00003-of-00003.gguf").unlink()
    with pytest.raises(H.HaloError):
        H.Gguf(path=tmp_path / "m-00001-of-00003.gguf")
    (tmp_path / "x.gguf").write_bytes(W.write(common(0), [f("a", 1.0)]))
    with pytest.raises(H.HaloError, match="file name"):
        H.Gguf(path=tmp_path / "x.gguf")
    with pytest.raises(H.HaloError):
        H.Gguf(path=tmp_path / "missing.gguf")


def test_model_config_from_metadata():
    cfg = H.ModelConfig(vocab=2048, hidden=1024, layers=4, attn_interval=4, gdn_k_heads=4, gdn_v_heads=8,
                        gdn_head_dim=128, conv_kernel=4, q_heads=16, kv_heads=2, head_dim=256, rotary_dim=64,
                        n_experts=16, n_used=4, expert_ff=256, shared_ff=256, rope_theta=1e7, rms_eps=1e-6,
                        max_sessions=2, max_context=64, prefix_tokens=0)

    class Fake:
        def tensor(self, layer, name):
            raise AssertionError

    p = "halo_synth."
    meta = [("general.architecture", W.STRING, "halo_synth"), (p + "block_count", W.U32, 4),
            (p + "embedding_length", W.U32, 1024), (p + "full_attention_interval", W.U32, 4),
            (p + "attention.head_count", W.U32, 16), (p + "attention.head_count_kv", W.U32, 2),
            (p + "attention.key_length", W.U32, 256), (p + "rope.dimension_count", W.U32, 64),
            (p + "rope.freq_base", W.F32, 1e7), (p + "attention.layer_norm_rms_epsilon", W.F32, 1e-6),
            (p + "ssm.conv_kernel", W.U32, 4), (p + "ssm.state_size", W.U32, 128), (p + "ssm.group_count", W.U32, 4),
            (p + "ssm.time_step_rank", W.U32, 8), (p + "expert_count", W.U32, 16), (p + "expert_used_count", W.U32, 4),
            (p + "expert_feed_forward_length", W.U32, 256), (p + "expert_shared_feed_forward_length", W.U32, 256)]
    emb = ("token_embd.weight", W.GGML_Q8_0, [1024, 2048], bytes(2048 * 32 * 34))
    g = H.Gguf(data=W.write(meta, [emb]))
    got = g.config(H.ModelConfig(max_sessions=2, max_context=64))
    for name, _ in H.ModelConfig._fields_:
        assert getattr(got, name) == getattr(cfg, name), name
    g.close()
    g = H.Gguf(data=W.write(meta[:-1], [emb]))
    with pytest.raises(H.HaloError, match="expert_shared_feed_forward_length"):
        g.config()
    g.close()


def test_upload_q8_0_refuses_degenerate_shapes():
    """halo_gguf_upload_q8_0 refuses a tensor with no columns (it would divide by a zero row size) and a destination
    row stride shorter than the row or not 16-byte aligned (the repack would write past the rows), before it touches
    the engine or the device: the engine, staging and destination pointers below are placeholders never used."""
    import ctypes

    L = H.lib()
    err = ctypes.create_string_buffer(256)
    blob = ctypes.create_string_buffer(64)
    fake = ctypes.c_void_p(1 << 40)
    for cols, qstride, msg in ((0, 64, b"columns"), (64, 32, b"qstride"), (64, 72, b"qstride")):
        t = H.GgufTensor()
        t.type = 8  # GGML Q8_0
        t.n_dims = 2
        t.dims[0], t.dims[1] = cols, 4
        t.data = ctypes.cast(blob, ctypes.c_void_p)
        rc = L.halo_gguf_upload_q8_0(fake, ctypes.byref(t), 0, 1, fake, fake, qstride, fake, 1 << 20, err, 256)
        assert rc == -1 and msg in err.value, (cols, qstride, err.value)
