"""ctypes binding of the CPU oracle (oracle/liboracle.so) and of the reference build (oracle/_ref/libhaloref.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg, as the
checker. The product library never loads it.
"""
from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ORACLE_SO = HERE / "liboracle.so"
REF_SO = HERE / "_ref" / "libhaloref.so"
REF_MODEL_SO = HERE / "_ref" / "libhaloref_model.so"

_VP, _SZ, _U32, _U64, _F32 = C.c_void_p, C.c_size_t, C.c_uint32, C.c_uint64, C.c_float
_PF = np.ctypeslib.ndpointer(np.float32, flags="C")
_PD = np.ctypeslib.ndpointer(np.float64, flags="C")
_PI8 = np.ctypeslib.ndpointer(np.int8, flags="C")
_PU8 = np.ctypeslib.ndpointer(np.uint8, flags="C")
_PU16 = np.ctypeslib.ndpointer(np.uint16, flags="C")
_PI32 = np.ctypeslib.ndpointer(np.int32, flags="C")
_PU32 = np.ctypeslib.ndpointer(np.uint32, flags="C")

_ORACLE_SIGS = {
    "or_fp16_to_f32": (_F32, [C.c_uint16]),
    "or_f32_to_fp16": (C.c_uint16, [_F32]),
    "or_bf16_to_f32": (_F32, [C.c_uint16]),
    "or_f32_to_bf16": (C.c_uint16, [_F32]),
    "or_dequant_q8_0": (None, [_PU8, _PF, _SZ]),
    "or_repack_q8_0": (None, [_PU8, _PI8, _PU16, _U32, _U32, _U32]),
    "or_pack_q8_0": (None, [_PI8, _PU16, _PU8, _U32, _U32, _U32]),
    "or_quantize_q8_act": (None, [_PF, _PI8, _PF, _SZ]),
    "or_q8_block_dots": (None, [_PI8, _U32, _U32, _U32, _PI8, _PI32]),
    "or_gemv_q8a8": (None, [_PI8, _PU16, _U32, _U32, _U32, _PI8, _PF, _PF]),
    "or_gemv_q8a8_mag": (None, [_PI8, _PU16, _U32, _U32, _U32, _PI8, _PF, _PD]),
    "or_matvec_q8_0_f32x": (None, [_PI8, _PU16, _U32, _U32, _U32, _PF, _PF, C.c_int]),
    "or_matvec_f32": (None, [_PF, _U32, _U32, _PF, _PF]),
    "or_sigmoid": (_F32, [_F32]),
    "or_silu": (_F32, [_F32]),
    "or_softplus": (_F32, [_F32]),
    "or_rmsnorm": (None, [_PF, _SZ, _VP, _F32]),
    "or_l2norm": (None, [_PF, _SZ, _F32]),
    "or_rope_neox": (None, [_PF, _U32, _U32, _U32, _U32, _F32]),
    "or_route_topk": (None, [_PF, _U32, _U32, _PU32, _PF]),
    "or_gdn_step": (None, [_PF, _U32, _PF, _PF, _PF, _F32, _F32, _PF]),
    "or_gdn_sequence": (None, [_PF, _U32, _U32, _VP, _SZ, _VP, _SZ, _VP, _SZ, _VP, _VP, _SZ, _VP, _SZ]),
    "or_gdn_sequence_mag": (None, [_VP, _U32, _U32, _VP, _SZ, _VP, _SZ, _VP, _SZ, _VP, _VP, _SZ, _VP, _SZ]),
    "or_attention_head": (None, [_PF, _PF, _PF, _U32, _U32, _SZ, _PF]),
    "or_next_random": (_U64, [C.POINTER(C.c_uint64)]),
    "or_sample": (_U32, [_PF, _U32, _F32, C.c_int32, _F32, _F32, _U32, _F32, _F32, _F32, _VP, _VP, _VP, _U32,
                         C.POINTER(C.c_uint64)]),
    "or_sample_state": (_U32, [_PF, _U32, _F32, C.c_int32, _F32, _F32, _U32, _F32, _F32, _F32, _VP, _VP, _VP,
                               _U32, C.POINTER(C.c_uint64)]),
    "or_sample_state_ex": (_U32, [_PF, _U32, _F32, C.c_int32, _F32, _F32, _U32, _F32, _F32, _F32, _VP, _VP, _VP,
                                  _U32, C.POINTER(C.c_uint64), C.POINTER(C.c_double), C.POINTER(C.c_uint32)]),
    "or_sample_penalties": (_U32, [_VP, _U32, _VP, _U32, _F32, _U32, _F32, _F32, _VP, _VP, _VP, _U32]),
}

_REF_SIGS = {
    "ref_fp16_to_f32": (_F32, [C.c_uint16]),
    "ref_dequant_q8_0": (None, [_PU8, _PF, _SZ]),
    "ref_dot_q8_0": (_F32, [_PU8, _PF, _SZ]),
    "ref_matvec_q8_0": (None, [_PU8, _U64, _U64, _PF, _PF]),
    "ref_matvec_f32": (None, [_PF, _U64, _U64, _PF, _PF]),
    "ref_route_topk": (None, [_PF, _U32, _U32, _PU32, _PF]),
    "ref_rmsnorm": (None, [_PF, _SZ, _VP, _F32]),
    "ref_l2norm": (None, [_PF, _SZ, _F32]),
    "ref_rope": (None, [_PF, _U32, _U32, _U32, _U32, _F32]),
    "ref_silu": (_F32, [_F32]),
    "ref_sigmoid": (_F32, [_F32]),
    "ref_softplus": (_F32, [_F32]),
    "ref_hw_threads": (C.c_uint, []),
    "ref_sampler_state": (_U32, [_PF, _U32, _F32, C.c_int32, _F32, _F32, _U32, _F32, _U32, _F32, _F32, _VP, _U32,
                                 _VP, _U32, C.POINTER(C.c_uint64), _VP, _VP, _VP, _U32, C.POINTER(C.c_uint32)]),
    "ref_gguf_open": (_VP, [_VP, C.c_size_t]),
    "ref_gguf_close": (None, [_VP]),
    "ref_gguf_header": (None, [_VP, C.POINTER(C.c_uint32), C.POINTER(C.c_uint64), C.POINTER(C.c_uint64),
                               C.POINTER(C.c_uint64)]),
    "ref_gguf_tensor": (C.c_int, [_VP, C.c_uint64, _VP, C.c_char_p, C.c_size_t, C.POINTER(C.c_uint32),
                                  C.POINTER(C.c_uint64), C.POINTER(C.c_uint32), C.POINTER(C.c_uint64),
                                  C.POINTER(C.c_uint64), C.POINTER(C.c_uint64)]),
    "ref_gguf_meta": (C.c_int, [_VP, C.c_char_p, C.c_char_p, C.c_size_t]),
    "ref_gguf_label": (C.c_uint32, [_VP, C.c_char_p, C.c_size_t]),
    "ref_encoded_bytes": (C.c_uint64, [C.c_uint32, C.c_uint64]),
    "ref_sample": (_U32, [_PF, _U32, _F32, C.c_int32, _F32, _F32, _U32, _F32, _U32, _F32, _F32, _VP, _U32, _VP, _U32,
                          C.POINTER(C.c_uint64)]),
}

# the reference's ReferenceModel layer functions (oracle/ref_model_shim.cpp)
_REF_MODEL_SIGS = {
    "ref_linear_attention": (None, [_PU32, _PF, _PU8, _PU8, _PU8, _PU8, _PU8, _PF, _PF, _PF, _PF, _PF, _PF, _PF,
                                    _PF]),
    "ref_attention": (None, [_PU32, _PF, _PU8, _PU8, _PU8, _PU8, _PF, _PF, _PF, _PF, _U32]),
    "ref_moe": (None, [_PU32, _PF, _PU8, _PU8, _PU8, _PF, _PU8, _PU8, _PU8, _PF, _PF]),
}

_libs: dict[str, C.CDLL] = {}


def _load(path: Path, sigs) -> C.CDLL:
    key = str(path)
    if key not in _libs:
        L = C.CDLL(key)
        for n, (r, a) in sigs.items():
            f = getattr(L, n)
            f.restype, f.argtypes = r, a
        _libs[key] = L
    return _libs[key]


def build():
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)


def oracle() -> C.CDLL:
    if not ORACLE_SO.exists():
        build()
    return _load(ORACLE_SO, _ORACLE_SIGS)


def has_ref() -> bool:
    return REF_SO.exists()


def ref() -> C.CDLL:
    return _load(REF_SO, _REF_SIGS)


def has_ref_model() -> bool:
    return REF_MODEL_SO.exists()


def ref_model() -> C.CDLL:
    return _load(REF_MODEL_SO, _REF_MODEL_SIGS)


# ---- numpy conveniences -------------------------------------------------------------------------------------------

def quantize(x: np.ndarray):
    x = np.ascontiguousarray(x, np.float32)
    xq = np.empty(x.shape, np.int8)
    xs = np.empty(x.shape[:-1] + (x.shape[-1] // 32,), np.float32)
    oracle().or_quantize_q8_act(x.reshape(-1), xq.reshape(-1), xs.reshape(-1), x.size)
    return xq, xs


def gemv_q8a8(qs, d, xq, xs):
    """y[t][r] for t tokens (xq [T][cols] or [cols])."""
    qs = np.ascontiguousarray(qs, np.int8)
    d = np.ascontiguousarray(d, np.uint16)
    rows, cols = qs.shape
    xq2 = np.atleast_2d(xq)
    xs2 = np.atleast_2d(xs)
    y = np.empty((xq2.shape[0], rows), np.float32)
    mag = np.empty((xq2.shape[0], rows), np.float64)
    for t in range(xq2.shape[0]):
        oracle().or_gemv_q8a8(qs, d, rows, cols, cols, np.ascontiguousarray(xq2[t]), np.ascontiguousarray(xs2[t]), y[t])
        oracle().or_gemv_q8a8_mag(qs, d, rows, cols, cols, np.ascontiguousarray(xq2[t]),
                                  np.ascontiguousarray(xs2[t]), mag[t])
    if np.ndim(xq) == 1:
        return y[0], mag[0]
    return y, mag


def block_dots(qs, xq):
    qs = np.ascontiguousarray(qs, np.int8)
    rows, cols = qs.shape
    out = np.empty((rows, cols // 32), np.int32)
    oracle().or_q8_block_dots(qs, rows, cols, cols, np.ascontiguousarray(xq, np.int8), out)
    return out


def synth_q8(rng: np.random.Generator, rows: int, cols: int, sigma: float = 0.02):
    """The benchmark's Q8_0 distribution: q ~ U{-127..127}, d = fp16(|N(0, sigma)| / 127)."""
    qs = rng.integers(-127, 128, size=(rows, cols), dtype=np.int8)
    d = (np.abs(rng.normal(0.0, sigma, size=(rows, cols // 32))) / 127.0).astype(np.float16).view(np.uint16)
    return qs, d


def sample_penalties(prompt, generated, repeat_penalty=1.0, repeat_last_n=64, frequency_penalty=0.0,
                     presence_penalty=0.0, cap=8192):
    """The penalty list {token, generated_count, repeated} (sorted by token) the reference builds from history."""
    p = np.ascontiguousarray(prompt, np.uint32)
    g = np.ascontiguousarray(generated, np.uint32)
    tok, gen, rep = (np.zeros(cap, np.uint32) for _ in range(3))
    n = oracle().or_sample_penalties(p.ctypes.data, len(p), g.ctypes.data, len(g), repeat_penalty, repeat_last_n,
                                     frequency_penalty, presence_penalty, tok.ctypes.data, gen.ctypes.data,
                                     rep.ctypes.data, cap)
    return tok[:n].copy(), gen[:n].copy(), rep[:n].copy()


def sample(logits, rng, temperature=1.0, top_k=0, top_p=1.0, min_p=0.0, min_keep=0, repeat_penalty=1.0,
           repeat_last_n=64, frequency_penalty=0.0, presence_penalty=0.0, prompt=(), generated=()):
    """One draw of the restated sampler; returns (token, rng state after)."""
    x = np.ascontiguousarray(logits, np.float32)
    tok, gen, rep = sample_penalties(prompt, generated, repeat_penalty, repeat_last_n, frequency_penalty,
                                     presence_penalty)
    st = C.c_uint64(rng)
    t = oracle().or_sample(x, len(x), temperature, top_k, top_p, min_p, min_keep, repeat_penalty, frequency_penalty,
                           presence_penalty, tok.ctypes.data, gen.ctypes.data, rep.ctypes.data, len(tok),
                           C.byref(st))
    return int(t), int(st.value)


def ref_sample(logits, rng, temperature=1.0, top_k=0, top_p=1.0, min_p=0.0, min_keep=0, repeat_penalty=1.0,
               repeat_last_n=64, frequency_penalty=0.0, presence_penalty=0.0, prompt=(), generated=()):
    """One draw of the reference's own sampler (oracle/_ref); returns (token, rng state after)."""
    x = np.ascontiguousarray(logits, np.float32)
    p = np.ascontiguousarray(prompt, np.uint32)
    g = np.ascontiguousarray(generated, np.uint32)
    st = C.c_uint64(rng)
    t = ref().ref_sample(x, len(x), temperature, top_k, top_p, min_p, min_keep, repeat_penalty, repeat_last_n,
                         frequency_penalty, presence_penalty, p.ctypes.data, len(p), g.ctypes.data, len(g),
                         C.byref(st))
    return int(t), int(st.value)


def sample_state(logits, rng, penalties=None, temperature=1.0, top_k=0, top_p=1.0, min_p=0.0, min_keep=0,
                 repeat_penalty=1.0, frequency_penalty=0.0, presence_penalty=0.0, u=None, with_live=False):
    """One draw of the restated SamplerState::Sample; penalties = (token, generated_count, repeated) arrays sorted
    by token. Returns (token, rng state after), plus the nonzero-probability count when with_live. With u given,
    that uniform replaces the RNG draw."""
    x = np.ascontiguousarray(logits, np.float32)
    if penalties is None:
        penalties = (np.zeros(0, np.uint32),) * 3
    tok, gen, rep = (np.ascontiguousarray(a, np.uint32) for a in penalties)
    st = C.c_uint64(rng)
    live = C.c_uint32(0)
    uf = C.c_double(u) if u is not None else None
    t = oracle().or_sample_state_ex(x, len(x), temperature, top_k, top_p, min_p, min_keep, repeat_penalty,
                                    frequency_penalty, presence_penalty, tok.ctypes.data, gen.ctypes.data,
                                    rep.ctypes.data, len(tok), C.byref(st), C.byref(uf) if uf is not None else None,
                                    C.byref(live))
    if with_live:
        return int(t), int(st.value), int(live.value)
    return int(t), int(st.value)


def ref_sampler_state(logits, rng, temperature=1.0, top_k=0, top_p=1.0, min_p=0.0, min_keep=0, repeat_penalty=1.0,
                      repeat_last_n=64, frequency_penalty=0.0, presence_penalty=0.0, prompt=(), generated=()):
    """The reference's SamplerState over history prompt + accepted generated tokens (oracle/_ref).
    Returns (token, rng state after, penalties as (token, generated_count, repeated) arrays)."""
    x = np.ascontiguousarray(logits, np.float32)
    p = np.ascontiguousarray(prompt, np.uint32)
    g = np.ascontiguousarray(generated, np.uint32)
    cap = 8192
    tok, gen, rep = (np.zeros(cap, np.uint32) for _ in range(3))
    st = C.c_uint64(rng)
    npen = C.c_uint32(0)
    t = ref().ref_sampler_state(x, len(x), temperature, top_k, top_p, min_p, min_keep, repeat_penalty, repeat_last_n,
                                frequency_penalty, presence_penalty, p.ctypes.data, len(p), g.ctypes.data, len(g),
                                C.byref(st), tok.ctypes.data, gen.ctypes.data, rep.ctypes.data, cap, C.byref(npen))
    k = npen.value
    return int(t), int(st.value), (tok[:k].copy(), gen[:k].copy(), rep[:k].copy())


def ref_gguf_summary(blob: bytes, keys):
    """The reference reader's view of a GGUF image: None when it refuses the bytes, else (version, alignment,
    metadata count, [(name, type, dims, offset, size, data offset)], {key: value text} for `keys`, label)."""
    L = ref()
    buf = C.create_string_buffer(blob, len(blob))
    h = L.ref_gguf_open(buf, len(blob))
    if not h:
        return None
    try:
        v, a, nm, nt = C.c_uint32(), C.c_uint64(), C.c_uint64(), C.c_uint64()
        L.ref_gguf_header(h, C.byref(v), C.byref(a), C.byref(nm), C.byref(nt))
        tensors = []
        for i in range(nt.value):
            name = C.create_string_buffer(70000)
            ty, nd = C.c_uint32(), C.c_uint32()
            dims = (C.c_uint64 * 8)()
            off, sz, doff = C.c_uint64(), C.c_uint64(), C.c_uint64()
            n = L.ref_gguf_tensor(h, i, buf, name, 70000, C.byref(ty), dims, C.byref(nd), C.byref(off), C.byref(sz),
                                  C.byref(doff))
            tensors.append((name.raw[:n], ty.value, tuple(dims[:nd.value]), off.value, sz.value, doff.value))
        meta = {}
        for k in keys:
            out = C.create_string_buffer(1 << 20)
            n = L.ref_gguf_meta(h, k, out, 1 << 20)
            meta[k] = None if n < 0 else out.value.decode()
        lab = C.create_string_buffer(64)
        L.ref_gguf_label(h, lab, 64)
        return (v.value, a.value, nm.value, tensors, meta, lab.value.decode())
    finally:
        L.ref_gguf_close(h)
