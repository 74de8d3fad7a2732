"""ctypes binding of libhalo_flash_amd.so (include/halo_rt.h, include/halo_ops.h).

This is a thin harness for tests and the benchmark: every operation goes through the C ABI into the HIP library.
There is no CPU fallback: if the library is missing, importing the binding raises.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

import numpy as np

PKG_DIR = Path(__file__).resolve().parent.parent  # halo-flash_amd/
# HALO_AMD_LIB selects another build of the library (the diagnostic `make timing` build)
LIB_PATH = Path(os.environ["HALO_AMD_LIB"]) if os.environ.get("HALO_AMD_LIB") else PKG_DIR / "libhalo_flash_amd.so"


class HaloError(RuntimeError):
    pass


class Buffer(C.Structure):
    _fields_ = [("device", C.c_void_p), ("bytes", C.c_size_t), ("handle", C.c_void_p)]


class Arg(C.Structure):
    _fields_ = [
        ("kind", C.c_uint8),
        ("size", C.c_uint8),
        ("pad", C.c_uint8 * 6),
        ("buffer", Buffer),
        ("offset", C.c_size_t),
        ("bytes", C.c_uint8 * 8),
    ]


class Dim3(C.Structure):
    _fields_ = [("x", C.c_uint32), ("y", C.c_uint32), ("z", C.c_uint32)]


class Graph(C.Structure):
    _fields_ = [("exec", C.c_void_p)]


class Q8Matrix(C.Structure):
    _fields_ = [
        ("qs", C.c_void_p),
        ("d", C.c_void_p),
        ("rows", C.c_uint32),
        ("cols", C.c_uint32),
        ("qstride", C.c_uint32),
        ("pad", C.c_uint32),
    ]


class ProjInput(C.Structure):
    """halo_proj_input: the activation source of a grouped projection (modes PROJ_Q / PROJ_F / PROJ_N)."""
    _fields_ = [(n, C.c_void_p) for n in ("x", "delta", "norm_w", "res_out", "xq", "xs", "xq_out", "xs_out")] + [
        ("eps", C.c_float), ("mode", C.c_uint32)]


PROJ_Q, PROJ_F, PROJ_N, PROJ_G = 0, 1, 2, 3


def proj_q8(dev, weights, outs, inp: ProjInput, tokens: int, tasks_per_wave: int = 0, lanes_per_row: int = 0):
    """One grouped projection launch: weights is a list of Q8Weights, outs their [tokens][rows] outputs."""
    mats = (Q8Matrix * len(weights))(*[w.desc for w in weights])
    ys = (C.c_void_p * len(outs))(*[o.ptr for o in outs])
    dev.op("proj_q8_grid", mats, ys, len(weights), C.byref(inp), tokens, tasks_per_wave, lanes_per_row)


def proj_q8_pair(dev, weights, outs, n_first: int, inp: ProjInput, inp2: ProjInput, tokens: int):
    """Two grouped mode-Q projections in one launch: weights[:n_first] read inp, weights[n_first] reads inp2."""
    mats = (Q8Matrix * len(weights))(*[w.desc for w in weights])
    ys = (C.c_void_p * len(outs))(*[o.ptr for o in outs])
    dev.op("proj_q8_pair", mats, ys, n_first, C.byref(inp), C.byref(inp2), tokens)


class MoeWeights(C.Structure):
    _fields_ = [
        ("router", C.c_void_p),
        ("shared_gate", C.c_void_p),
        ("gate", Q8Matrix),
        ("up", Q8Matrix),
        ("down", Q8Matrix),
        ("shared_gate_proj", Q8Matrix),
        ("shared_up", Q8Matrix),
        ("shared_down", Q8Matrix),
        ("n_experts", C.c_uint32),
        ("n_used", C.c_uint32),
        ("hidden", C.c_uint32),
        ("ff", C.c_uint32),
        ("shared_ff", C.c_uint32),
        ("pad", C.c_uint32),
    ]


class MoeViews(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in ("logits", "shared_logit", "xq", "xs", "ids", "weights", "h")] + [
        ("hstride", C.c_uint32), ("pad", C.c_uint32), ("bytes", C.c_size_t)]


class PagedKV(C.Structure):
    _fields_ = [("k_pool", C.c_void_p), ("v_pool", C.c_void_p), ("pages", C.c_void_p), ("nkv", C.c_void_p)] + [
        (n, C.c_uint32) for n in ("sessions", "kv_heads", "head_dim", "max_pages", "prefix", "max_context")]


class PrefillSegment(C.Structure):
    _fields_ = [(n, C.c_uint32) for n in ("session", "start", "length", "first")]


class ModelConfig(C.Structure):
    _fields_ = [(n, C.c_uint32) for n in (
        "vocab", "hidden", "layers", "attn_interval", "gdn_k_heads", "gdn_v_heads", "gdn_head_dim", "conv_kernel",
        "q_heads", "kv_heads", "head_dim", "rotary_dim", "n_experts", "n_used", "expert_ff", "shared_ff")] + [
        ("rope_theta", C.c_float), ("rms_eps", C.c_float)] + [
        (n, C.c_uint32) for n in ("max_sessions", "max_context", "prefix_tokens", "prefill_batch")]


class SampleParams(C.Structure):
    """HaloSampleParams (include/halo_sample.h)."""
    _fields_ = [("temperature", C.c_float), ("top_p", C.c_float), ("min_p", C.c_float),
                ("repeat_penalty", C.c_float), ("frequency_penalty", C.c_float), ("presence_penalty", C.c_float),
                ("top_k", C.c_uint32), ("min_keep", C.c_uint32), ("n_penalties", C.c_uint32),
                ("vocab", C.c_uint32), ("rng", C.c_uint64), ("fallback_only", C.c_uint32), ("pad", C.c_uint32)]


SAMPLE_NO_FINITE = 0xFFFFFFFF
SAMPLE_BAD_PARAMS = 0xFFFFFFFC
PENALTY_DTYPE = np.dtype([("token", np.uint32), ("generated_count", np.uint32), ("repeated", np.uint32),
                          ("pad", np.uint32)])
SAMPLE_OUT_DTYPE = np.dtype([("token", np.uint32), ("live", np.uint32), ("rng", np.uint64)])


def sample_rows(dev, logits, params, penalties=None):
    """Device sampling of each row of `logits` (host [rows][vocab] fp32) with params (a list of SampleParams) and
    penalties (a list of (token, generated_count, repeated) arrays per row, or None). Returns the HaloSampleOut rows
    as a structured array (token, live, rng)."""
    x = np.ascontiguousarray(logits, np.float32)
    rows, V = x.shape
    pen_lists = penalties if penalties is not None else [None] * rows
    stride = max([len(pl[0]) for pl in pen_lists if pl is not None] + [1])
    pen = np.zeros((rows, stride), PENALTY_DTYPE)
    prm = (SampleParams * rows)()
    for r in range(rows):
        prm[r] = params[r]
        prm[r].vocab = V if params[r].vocab == 0 else params[r].vocab
        pl = pen_lists[r]
        n = 0 if pl is None else len(pl[0])
        prm[r].n_penalties = n
        if n:
            pen[r, :n]["token"], pen[r, :n]["generated_count"], pen[r, :n]["repeated"] = pl
    dl = dev.to_device(x)
    dp = dev.to_device(np.frombuffer(bytes(prm), np.uint8))
    dq = dev.to_device(pen.view(np.uint8).reshape(-1))
    do = dev.array(rows * 16, np.uint8)
    ws = dev.array(lib().halo_op_sample_workspace_bytes(rows, V), np.uint8)
    try:
        dev.op("sample", dl.ptr, rows, V, V, dp.ptr, dq.ptr, stride, do.ptr, ws.ptr, ws.nbytes)
        dev.sync()
        return do.download().view(SAMPLE_OUT_DTYPE).copy()
    finally:
        for a in (dl, dp, dq, do, ws):
            a.free()


class GgufTensor(C.Structure):
    """halo_gguf_tensor (include/halo_gguf.h)."""
    _fields_ = [("name", C.c_void_p), ("name_len", C.c_size_t), ("type", C.c_uint32), ("n_dims", C.c_uint32),
                ("dims", C.c_uint64 * 8), ("offset", C.c_uint64), ("data", C.c_void_p), ("size_bytes", C.c_uint64)]


class Gguf:
    """A GGUF checkpoint opened by the library's reader (from a file path or from bytes kept alive here)."""

    def __init__(self, path=None, data: bytes | None = None):
        self._buf = None
        self.h = None
        h = C.c_void_p()
        if path is not None:
            _call("halo_gguf_open_file", str(path).encode(), C.byref(h))
        else:
            self._buf = C.create_string_buffer(data, len(data))
            _call("halo_gguf_open_memory", self._buf, len(data), C.byref(h))
        self.h = h

    def close(self):
        if self.h:
            lib().halo_gguf_close(self.h)
            self.h = None

    def __del__(self):
        self.close()

    @property
    def version(self):
        return lib().halo_gguf_version(self.h)

    @property
    def alignment(self):
        return lib().halo_gguf_alignment(self.h)

    def metadata_count(self):
        return lib().halo_gguf_metadata_count(self.h)

    def tensor(self, i_or_name):
        t = GgufTensor()
        L = lib()
        rc = (L.halo_gguf_find_tensor(self.h, i_or_name.encode(), C.byref(t)) if isinstance(i_or_name, str)
              else L.halo_gguf_tensor_at(self.h, i_or_name, C.byref(t)))
        return t if rc == 0 else None

    def tensors(self):
        """[(name bytes, type, dims, offset, size, data address)] in file order."""
        out = []
        for i in range(lib().halo_gguf_tensor_count(self.h)):
            t = self.tensor(i)
            out.append((C.string_at(t.name, t.name_len), t.type, tuple(t.dims[:t.n_dims]), t.offset, t.size_bytes,
                        t.data))
        return out

    def keys(self):
        L = lib()
        out = []
        for i in range(self.metadata_count()):
            p, n = C.c_void_p(), C.c_size_t()
            L.halo_gguf_metadata_key_at(self.h, i, C.byref(p), C.byref(n))
            out.append(C.string_at(p, n.value))
        return out

    def value_text(self, key: bytes):
        """The value as text (u:/i:/f:/b:/s:/S:/U:/I:/F:, prefixed by the value type), None when absent."""
        L = lib()
        ty = L.halo_gguf_metadata_type(self.h, key)
        if ty < 0:
            return None
        hexd = lambda x: np.float64(x).view(np.uint64).item().to_bytes(8, "big").hex()

        def text(prefix, ptr, n):
            return prefix + C.string_at(ptr, n).hex()
        if ty in (0, 2, 4, 10):
            v = C.c_uint64()
            L.halo_gguf_get_u64(self.h, key, C.byref(v))
            body = f"u:{v.value}"
        elif ty in (1, 3, 5, 11):
            v = C.c_int64()
            L.halo_gguf_get_i64(self.h, key, C.byref(v))
            body = f"i:{v.value}"
        elif ty in (6, 12):
            v = C.c_double()
            L.halo_gguf_get_f64(self.h, key, C.byref(v))
            body = "f:" + hexd(v.value)
        elif ty == 7:
            v = C.c_int()
            L.halo_gguf_get_bool(self.h, key, C.byref(v))
            body = f"b:{v.value}"
        elif ty == 8:
            p, n = C.c_void_p(), C.c_size_t()
            L.halo_gguf_get_string(self.h, key, C.byref(p), C.byref(n))
            body = text("s:", p, n.value)
        else:
            et, n = C.c_uint32(), C.c_uint64()
            L.halo_gguf_get_array_info(self.h, key, C.byref(et), C.byref(n))
            et, n = et.value, n.value
            if et == 8:
                parts = []
                for i in range(n):
                    p, m = C.c_void_p(), C.c_size_t()
                    L.halo_gguf_get_array_string(self.h, key, i, C.byref(p), C.byref(m))
                    parts.append(C.string_at(p, m.value).hex() + ",")
                body = f"S:{n}:" + "".join(parts)
            elif et in (6, 12):
                parts = []
                for i in range(n):
                    v = C.c_double()
                    L.halo_gguf_get_array_f64(self.h, key, i, C.byref(v))
                    parts.append(hexd(v.value) + ",")
                body = "F:" + "".join(parts)
            elif et in (4, 7, 10):
                parts = []
                for i in range(n):
                    v = C.c_uint64()
                    L.halo_gguf_get_array_u64(self.h, key, i, C.byref(v))
                    parts.append(f"{v.value},")
                body = "U:" + "".join(parts)
            elif et in (5, 11):
                parts = []
                for i in range(n):
                    v = C.c_int64()
                    L.halo_gguf_get_array_i64(self.h, key, i, C.byref(v))
                    parts.append(f"{v.value},")
                body = "I:" + "".join(parts)
            else:
                body = "u:0"
        return f"{ty}|{body}"

    def label(self):
        b = C.create_string_buffer(64)
        lib().halo_gguf_quantization_label(self.h, b, 64)
        return b.value.decode()

    def config(self, base: "ModelConfig | None" = None) -> "ModelConfig":
        c = ModelConfig() if base is None else base
        _call("halo_model_config_from_gguf", self.h, C.byref(c))
        return c


class TensorView(C.Structure):
    _fields_ = [("data", C.c_void_p), ("scales", C.c_void_p)] + [(n, C.c_uint32) for n in (
        "kind", "rows", "cols", "qstride")]


class TraceEntry(C.Structure):
    """halo_model_trace_entry (include/halo_model.h)."""
    _fields_ = [("name", C.c_char * 24), ("layer", C.c_uint32), ("dtype", C.c_uint32), ("offset", C.c_uint64),
                ("bytes", C.c_uint64)]


TRACE_DTYPES = {0: np.float32, 1: np.int8, 2: np.uint32}


def c4_config(max_sessions=4, prefix_tokens=8192, max_context=8192 + 256 + 128):
    """Benchmark config C4: 48 layers (3 DeltaNet : 1 GQA), hidden 2048, vocab 151936, MoE as C2."""
    return ModelConfig(vocab=151936, hidden=2048, layers=48, attn_interval=4, gdn_k_heads=16, gdn_v_heads=32,
                       gdn_head_dim=128, conv_kernel=4, q_heads=16, kv_heads=2, head_dim=256, rotary_dim=64,
                       n_experts=512, n_used=10, expert_ff=512, shared_ff=512, rope_theta=1e7, rms_eps=1e-6,
                       max_sessions=max_sessions, max_context=max_context, prefix_tokens=prefix_tokens)


ERRLEN = 1024
_VP, _SZ, _U32, _U64, _F32, _I32 = C.c_void_p, C.c_size_t, C.c_uint32, C.c_uint64, C.c_float, C.c_int32
_ERR = [C.c_char_p, _SZ]

# name -> (restype, argtypes without the trailing err/errlen, has_err)
_SIGS = {
    "halo_device_create": (C.c_int, [C.c_int, C.POINTER(_VP)], True),
    "halo_device_destroy": (None, [_VP], False),
    "halo_device_ordinal": (C.c_int, [_VP], False),
    "halo_alloc": (C.c_int, [_VP, _SZ, C.POINTER(Buffer)], True),
    "halo_free": (None, [_VP, C.POINTER(Buffer)], False),
    "halo_upload": (C.c_int, [_VP, C.POINTER(Buffer), _SZ, _VP, _SZ], True),
    "halo_upload_async": (C.c_int, [_VP, C.POINTER(Buffer), _SZ, _VP, _SZ], True),
    "halo_download": (C.c_int, [_VP, C.POINTER(Buffer), _SZ, _VP, _SZ], True),
    "halo_fill": (C.c_int, [_VP, C.POINTER(Buffer), C.c_uint8], True),
    "halo_alloc_host": (_VP, [_VP, _SZ], True),
    "halo_free_host": (None, [_VP, _VP], False),
    "halo_available_bytes": (_SZ, [_VP], False),
    "halo_core_code_object": (C.POINTER(C.c_uint8), [C.POINTER(_SZ)], False),
    "halo_load_module": (C.c_int, [_VP, _VP, _SZ], True),
    "halo_code_object_mach": (C.c_int, [_VP, _SZ], False),
    "halo_kernel": (_I32, [_VP, C.c_char_p], True),
    "halo_launch": (C.c_int, [_VP, _I32, Dim3, Dim3, C.POINTER(Arg), _SZ], True),
    "halo_synchronize": (C.c_int, [_VP], True),
    "halo_begin_capture": (C.c_int, [_VP], True),
    "halo_end_capture": (C.c_int, [_VP, C.POINTER(Graph)], True),
    "halo_launch_graph": (C.c_int, [_VP, C.POINTER(Graph)], True),
    "halo_free_graph": (None, [_VP, C.POINTER(Graph)], False),
    "halo_timer_start": (C.c_int, [_VP], True),
    "halo_page_bytes": (_SZ, [_VP], False),
    "halo_reserve_range": (C.c_int, [_VP, _SZ, C.POINTER(Buffer)], True),
    "halo_release_range": (None, [_VP, C.POINTER(Buffer)], False),
    "halo_create_page": (C.c_int, [_VP, C.POINTER(_VP)], True),
    "halo_release_page": (None, [_VP, _VP], False),
    "halo_map_page": (C.c_int, [_VP, C.POINTER(Buffer), _SZ, _VP], True),
    "halo_unmap_page": (C.c_int, [_VP, C.POINTER(Buffer), _SZ], True),
    "halo_read_global": (C.c_int, [_VP, C.c_char_p, _VP, _SZ], True),
    "halo_write_global": (C.c_int, [_VP, C.c_char_p, _VP, _SZ], True),
    "halo_timer_stop": (C.c_int, [_VP, C.POINTER(_F32)], True),
    "halo_wall_clock_khz": (C.c_int, [_VP, C.POINTER(C.c_int)], True),
    "halo_device_stream": (_VP, [_VP], False),
    "halo_profile_begin": (C.c_int, [_VP], True),
    "halo_profile_end": (C.c_int, [_VP, _VP, _SZ], True),
    "halo_engine_create": (C.c_int, [_VP, C.POINTER(_VP)], True),
    "halo_engine_destroy": (None, [_VP], False),
    "halo_engine_device": (_VP, [_VP], False),
    "halo_engine_launch": (C.c_int, [_VP, C.c_char_p, Dim3, Dim3, C.POINTER(Arg), _SZ], True),
    "halo_op_repack_q8_0": (C.c_int, [_VP, _VP, _VP, _VP, _U32, _U32, _U32], True),
    "halo_op_quantize_q8": (C.c_int, [_VP, _VP, _VP, _VP, _U32, _U32], True),
    "halo_op_quantize_q8_pair": (C.c_int, [_VP, _VP, _VP, _VP, _U32, _VP, _VP, _VP, _U32, _U32], True),
    "halo_op_moe_prefill_workspace_bytes": (_SZ, [C.POINTER(MoeWeights), _U32], False),
    "halo_op_moe_prefill": (C.c_int, [_VP, C.POINTER(MoeWeights), _VP, _VP, _U32, _VP, _SZ], True),
    "halo_op_attn_prefill_workspace_bytes": (_SZ, [C.POINTER(PrefillSegment), _U32], False),
    "halo_op_attn_prefill": (C.c_int, [_VP, C.POINTER(PagedKV), C.POINTER(PrefillSegment), _U32, _VP, _VP, _VP, _VP,
                                       _VP, _U32, _VP, _SZ], True),
    "halo_op_proj_q8": (C.c_int, [_VP, C.POINTER(Q8Matrix), C.POINTER(C.c_void_p), _U32, C.POINTER(ProjInput), _U32],
                        True),
    "halo_op_proj_q8_grid": (C.c_int, [_VP, C.POINTER(Q8Matrix), C.POINTER(C.c_void_p), _U32, C.POINTER(ProjInput),
                                       _U32, _U32, _U32], True),
    "halo_op_proj_q8_pair": (C.c_int, [_VP, C.POINTER(Q8Matrix), C.POINTER(C.c_void_p), _U32, C.POINTER(ProjInput),
                                       C.POINTER(ProjInput), _U32], True),
    "halo_op_matvec_q8a8": (C.c_int, [_VP, C.POINTER(Q8Matrix), _VP, _VP, _VP, _U32, _U32], True),
    "halo_op_matvec_q8a8_tiled": (
        C.c_int, [_VP, C.POINTER(Q8Matrix), _VP, _VP, _VP, _U32, _U32, _U32, _U32, _U32], True),
    "halo_op_matvec_q8_f32x": (C.c_int, [_VP, C.POINTER(Q8Matrix), _VP, _VP], True),
    "halo_op_q8_half_dots": (C.c_int, [_VP, C.POINTER(Q8Matrix), _VP, _VP], True),
    "halo_op_synth_q8": (C.c_int, [_VP, _VP, _VP, _U32, _U32, _U32, _U64, _F32], True),
    "halo_op_synth_f32": (C.c_int, [_VP, _VP, _U64, _U64, _F32], True),
    "halo_op_gdn_decode": (C.c_int, [_VP] + [_VP] * 7 + [_U32] * 4, True),
    "halo_op_attn_decode_workspace_bytes": (_SZ, [C.POINTER(PagedKV), _U32], False),
    "halo_op_attn_decode": (C.c_int, [_VP, C.POINTER(PagedKV), _VP, _VP, _VP, _U32, _VP, _SZ], True),
    "halo_op_attn_decode_q8": (C.c_int, [_VP, C.POINTER(PagedKV), _VP, _VP, _VP, _VP, _VP, _U32, _VP, _SZ], True),
    "halo_op_attn_decode_step_q8": (C.c_int, [_VP, C.POINTER(PagedKV), _VP, _VP, _VP, _VP, _VP, _U32, C.c_float,
                                              C.c_float, _VP, _VP, _VP, _U32, _VP, _SZ], True),
    "halo_op_kv_append": (C.c_int, [_VP, C.POINTER(PagedKV), _VP, _VP], True),
    "halo_gdn_chunk_table": (_U32, [_VP, _U32, _VP, _VP], False),
    "halo_op_gdn_prefill_workspace_bytes": (_SZ, [_U32, _U32], False),
    "halo_op_gdn_prefill": (C.c_int, [_VP] + [_VP] * 7 + [_U32, _U32, _VP, _VP, _U32, _U32, _U32, _VP, _SZ], True),
    "halo_op_gdn_prefill_f32": (C.c_int, [_VP] + [_VP] * 7 + [_U32, _U32, _VP, _VP, _U32, _U32, _U32, _VP, _SZ],
                                True),
    "halo_model_create": (C.c_int, [_VP, C.POINTER(ModelConfig), _U64, C.POINTER(_VP)], True),
    "halo_model_destroy": (None, [_VP], False),
    "halo_model_weight_bytes": (_U64, [_VP], False),
    "halo_model_device_bytes": (_U64, [_VP], False),
    "halo_model_set_session": (C.c_int, [_VP, _U32, _VP, _U32, _U32], True),
    "halo_model_fork": (C.c_int, [_VP, _U32, _U32], True),
    "halo_model_reset": (C.c_int, [_VP], True),
    "halo_model_run": (C.c_int, [_VP, _U32, _U32, _U32], True),
    "halo_model_step_eager": (C.c_int, [_VP, _U32, _U32], True),
    "halo_model_history": (C.c_int, [_VP, _U32, _VP, _U32], True),
    "halo_model_positions": (C.c_int, [_VP, _VP, _U32], True),
    "halo_model_tensor": (C.c_int, [_VP, _U32, C.c_char_p, C.POINTER(TensorView)], True),
    "halo_model_logits": (C.c_int, [_VP, _U32, _VP], True),
    "halo_model_step_trace": (C.c_int, [_VP, _U32, _U32, _VP, _SZ, C.POINTER(TraceEntry), _U32,
                                        C.POINTER(_U32)], True),
    "halo_model_prefill_trace": (C.c_int, [_VP, C.POINTER(PrefillSegment), _U32, _VP, _SZ, C.POINTER(TraceEntry),
                                           _U32, C.POINTER(_U32)], True),
    "halo_model_prefill_trace_layers": (C.c_int, [_VP, C.POINTER(PrefillSegment), _U32, _U64, _VP, _SZ,
                                                  C.POINTER(TraceEntry), _U32, C.POINTER(_U32)], True),
    "halo_model_prefill": (C.c_int, [_VP, C.POINTER(PrefillSegment), _U32], True),
    "halo_op_moe_workspace_bytes": (_SZ, [C.POINTER(MoeWeights), _U32], False),
    "halo_op_moe_views": (C.c_int, [C.POINTER(MoeWeights), _U32, _VP, C.POINTER(MoeViews)], True),
    "halo_op_moe_decode": (C.c_int, [_VP, C.POINTER(MoeWeights), _VP, _VP, _U32, _VP, _SZ], True),
    "halo_op_moe_decode_noalloc": (C.c_int, [_VP, C.POINTER(MoeWeights), _VP, _VP, _U32], True),
    "halo_gguf_open_file": (C.c_int, [C.c_char_p, C.POINTER(_VP)], True),
    "halo_gguf_open_memory": (C.c_int, [_VP, _SZ, C.POINTER(_VP)], True),
    "halo_gguf_close": (None, [_VP], False),
    "halo_gguf_version": (_U32, [_VP], False),
    "halo_gguf_alignment": (_U64, [_VP], False),
    "halo_gguf_tensor_count": (_U64, [_VP], False),
    "halo_gguf_metadata_count": (_U64, [_VP], False),
    "halo_gguf_tensor_at": (C.c_int, [_VP, _U64, _VP], False),
    "halo_gguf_find_tensor": (C.c_int, [_VP, C.c_char_p, _VP], False),
    "halo_gguf_metadata_type": (C.c_int, [_VP, C.c_char_p], False),
    "halo_gguf_metadata_key_at": (C.c_int, [_VP, _U64, C.POINTER(_VP), C.POINTER(_SZ)], False),
    "halo_gguf_get_u32": (C.c_int, [_VP, C.c_char_p, C.POINTER(_U32)], False),
    "halo_gguf_get_u64": (C.c_int, [_VP, C.c_char_p, C.POINTER(_U64)], False),
    "halo_gguf_get_i64": (C.c_int, [_VP, C.c_char_p, C.POINTER(C.c_int64)], False),
    "halo_gguf_get_f32": (C.c_int, [_VP, C.c_char_p, C.POINTER(_F32)], False),
    "halo_gguf_get_f64": (C.c_int, [_VP, C.c_char_p, C.POINTER(C.c_double)], False),
    "halo_gguf_get_bool": (C.c_int, [_VP, C.c_char_p, C.POINTER(C.c_int)], False),
    "halo_gguf_get_string": (C.c_int, [_VP, C.c_char_p, C.POINTER(_VP), C.POINTER(_SZ)], False),
    "halo_gguf_get_array_info": (C.c_int, [_VP, C.c_char_p, C.POINTER(_U32), C.POINTER(_U64)], False),
    "halo_gguf_get_array_u64": (C.c_int, [_VP, C.c_char_p, _U64, C.POINTER(_U64)], False),
    "halo_gguf_get_array_i64": (C.c_int, [_VP, C.c_char_p, _U64, C.POINTER(C.c_int64)], False),
    "halo_gguf_get_array_f64": (C.c_int, [_VP, C.c_char_p, _U64, C.POINTER(C.c_double)], False),
    "halo_gguf_get_array_string": (C.c_int, [_VP, C.c_char_p, _U64, C.POINTER(_VP), C.POINTER(_SZ)], False),
    "halo_gguf_quantization_label": (_SZ, [_VP, C.c_char_p, _SZ], False),
    "halo_ggml_encoded_bytes": (_U64, [_U32, _U64], False),
    "halo_gguf_upload_q8_0": (C.c_int, [_VP, _VP, _U64, _U32, _VP, _VP, _U32, _VP, _SZ], True),
    "halo_model_config_from_gguf": (C.c_int, [_VP, _VP], True),
    "halo_model_load_gguf": (C.c_int, [_VP, _VP], True),
    "halo_model_set_sampling": (C.c_int, [_VP, _U32, _VP, _VP, _U32], True),
    "halo_model_sample_state": (C.c_int, [_VP, _U32, _VP], True),
    "halo_op_sample_workspace_bytes": (_SZ, [_U32, _U32], False),
    "halo_op_sample": (C.c_int, [_VP, _VP, _U32, _U64, _U32, _VP, _VP, _U32, _VP, _VP, _SZ], True),
    "halo_op_moe_decode_norm": (C.c_int, [_VP, C.POINTER(MoeWeights), C.POINTER(ProjInput), _VP, _U32, _VP, _SZ],
                                True),
}

_lib = None


def declared_symbols() -> list[str]:
    """Every function the public headers declare (parsed from include/*.h)."""
    import re

    names = []
    for h in sorted((PKG_DIR.parent / "include").glob("*.h")):
        text = h.read_text()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        for m in re.finditer(r"^[A-Za-z_][\w\s\*]*?\b(halo_\w+)\s*\(", text, flags=re.M):
            names.append(m.group(1))
    return sorted(set(names))


def lib() -> C.CDLL:
    """Loads the HIP library (raises if it was not built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise HaloError(f"{LIB_PATH} is not built (run __graft_entry__.build())")
    L = C.CDLL(str(LIB_PATH))
    for name, (res, args, has_err) in _SIGS.items():
        f = getattr(L, name)
        f.restype = res
        f.argtypes = args + (_ERR if has_err else [])
    _lib = L
    return L


def _call(name, *args):
    f = getattr(lib(), name)
    err = C.create_string_buffer(ERRLEN)
    rc = f(*args, err, ERRLEN)
    if rc not in (0, None) and not (isinstance(rc, int) and rc >= 0 and name == "halo_kernel"):
        raise HaloError(f"{name}: {err.value.decode(errors='replace')}")
    if name == "halo_kernel" and rc < 0:
        raise HaloError(f"{name}: {err.value.decode(errors='replace')}")
    return rc


def _scalar_arg(v, ctype) -> Arg:
    a = Arg()
    a.kind = 1
    raw = bytes(ctype(v))
    a.size = len(raw)
    for i, b in enumerate(raw):
        a.bytes[i] = b
    return a


class DeviceArray:
    """A device allocation with a numpy dtype/shape for uploads and downloads."""

    def __init__(self, dev: "Device", shape, dtype):
        self.dev = dev
        self.shape = tuple(int(s) for s in (shape if isinstance(shape, (tuple, list)) else (shape,)))
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape, dtype=np.int64)) * self.dtype.itemsize
        self.buf = Buffer()
        _call("halo_alloc", dev.handle, self.nbytes, C.byref(self.buf))

    @property
    def ptr(self) -> int:
        return int(self.buf.device)

    def upload(self, host: np.ndarray):
        host = np.ascontiguousarray(host, dtype=self.dtype)
        if host.nbytes != self.nbytes:
            raise HaloError(f"upload of {host.nbytes} bytes into {self.nbytes}")
        _call("halo_upload", self.dev.handle, C.byref(self.buf), 0, host.ctypes.data, host.nbytes)
        return self

    def download_range(self, offset: int, count: int, dtype=None) -> np.ndarray:
        """Download `count` elements of `dtype` (default: the array's) starting at byte `offset`."""
        dt = np.dtype(dtype or self.dtype)
        out = np.empty(count, dt)
        _call("halo_download", self.dev.handle, C.byref(self.buf), offset, out.ctypes.data, out.nbytes)
        return out

    def download(self) -> np.ndarray:
        out = np.empty(self.shape, self.dtype)
        _call("halo_download", self.dev.handle, C.byref(self.buf), 0, out.ctypes.data, out.nbytes)
        return out

    def fill(self, value: int = 0):
        _call("halo_fill", self.dev.handle, C.byref(self.buf), value)
        return self

    def free(self):
        if self.buf.device:
            lib().halo_free(self.dev.handle, C.byref(self.buf))

    def __del__(self):
        try:
            if self.dev.handle and self.buf.device:
                self.free()
        except Exception:
            pass


class Device:
    """halo_device + halo_engine (one HIP device, one stream, the embedded gfx950 code object)."""

    def __init__(self):
        h = C.c_void_p()
        _call("halo_device_create", 0, C.byref(h))
        self.handle = h
        e = C.c_void_p()
        _call("halo_engine_create", self.handle, C.byref(e))
        self.eng = e

    def close(self):
        if self.eng:
            lib().halo_engine_destroy(self.eng)
            self.eng = None
        if self.handle:
            lib().halo_device_destroy(self.handle)
            self.handle = None

    def array(self, shape, dtype) -> DeviceArray:
        return DeviceArray(self, shape, dtype)

    def to_device(self, host: np.ndarray) -> DeviceArray:
        host = np.ascontiguousarray(host)
        return DeviceArray(self, host.shape, host.dtype).upload(host)

    def sync(self):
        _call("halo_synchronize", self.handle)

    def launch(self, kernel: str, grid, block, args):
        """Launch by name; args are DeviceArray / ('u32', v) / ('u64', v) / ('f32', v) / ('ptr', int)."""
        n = len(args)
        arr = (Arg * n)()
        for i, a in enumerate(args):
            if isinstance(a, DeviceArray):
                arr[i].kind = 0
                arr[i].buffer = a.buf
            elif a is None:
                arr[i].kind = 0
            else:
                kind, v = a
                if kind == "ptr":
                    arr[i].kind = 0
                    arr[i].buffer.device = v
                else:
                    ct = {"u32": C.c_uint32, "i32": C.c_int32, "u64": C.c_uint64, "f32": C.c_float}[kind]
                    arr[i] = _scalar_arg(v, ct)
        g = Dim3(*(tuple(grid) + (1,) * (3 - len(grid))))
        b = Dim3(*(tuple(block) + (1,) * (3 - len(block))))
        _call("halo_engine_launch", self.eng, kernel.encode(), g, b, arr, n)

    def op(self, name: str, *args):
        return _call("halo_op_" + name, self.eng, *args)

    def timer_start(self):
        _call("halo_timer_start", self.handle)

    def timer_stop(self) -> float:
        ms = C.c_float()
        _call("halo_timer_stop", self.handle, C.byref(ms))
        return float(ms.value)

    def stream(self) -> int:
        """The device's HIP stream (hipStream_t) as an integer, for calls into the HIP runtime."""
        return int(lib().halo_device_stream(self.handle) or 0)

    def wall_clock_khz(self) -> int:
        khz = C.c_int()
        _call("halo_wall_clock_khz", self.handle, C.byref(khz))
        return int(khz.value)

    def profile_begin(self):
        _call("halo_profile_begin", self.handle)

    def profile_end(self) -> dict:
        buf = C.create_string_buffer(1 << 16)
        _call("halo_profile_end", self.handle, buf, 1 << 16)
        out = {}
        for line in buf.value.decode().splitlines():
            name, n, us = line.split()
            out[name] = (int(n), float(us))
        return out

    def begin_capture(self):
        _call("halo_begin_capture", self.handle)

    def end_capture(self) -> Graph:
        g = Graph()
        _call("halo_end_capture", self.handle, C.byref(g))
        return g

    def launch_graph(self, g: Graph):
        _call("halo_launch_graph", self.handle, C.byref(g))

    def free_graph(self, g: Graph):
        lib().halo_free_graph(self.handle, C.byref(g))


class Q8Weights:
    """A repacked Q8_0 matrix on the device (qs [rows][qstride] int8 + d [rows][cols/32] fp16 bits)."""

    def __init__(self, dev: Device, rows: int, cols: int, qstride: int | None = None):
        self.rows, self.cols = rows, cols
        self.qstride = qstride or ((cols + 15) // 16 * 16)
        self.qs = dev.array((rows, self.qstride), np.int8)
        self.d = dev.array((rows, cols // 32), np.uint16)
        self.desc = Q8Matrix(self.qs.ptr, self.d.ptr, rows, cols, self.qstride, 0)

    @classmethod
    def from_host(cls, dev: Device, qs: np.ndarray, d: np.ndarray):
        w = cls(dev, qs.shape[0], qs.shape[1])
        q = np.zeros((w.rows, w.qstride), np.int8)
        q[:, : w.cols] = qs
        w.qs.upload(q)
        w.d.upload(d.astype(np.uint16))
        return w

    def synth(self, dev: Device, seed: int, sigma: float = 0.02):
        dev.op("synth_q8", self.qs.ptr, self.d.ptr, self.rows, self.cols, self.qstride, seed, sigma)
        return self

    def host(self):
        return self.qs.download()[:, : self.cols], self.d.download()

    def host_rows(self, r0: int, n: int):
        """Rows [r0, r0 + n) as (qs, d) host arrays."""
        q = self.qs.download_range(r0 * self.qstride, n * self.qstride).reshape(n, self.qstride)[:, : self.cols]
        d = self.d.download_range(r0 * (self.cols // 32) * 2, n * (self.cols // 32)).reshape(n, self.cols // 32)
        return q, d


class Model:
    """halo_model: the synthetic hybrid model on the device (include/halo_model.h)."""

    def __init__(self, dev: Device, cfg: ModelConfig, seed: int = 0):
        self.dev, self.cfg = dev, cfg
        h = C.c_void_p()
        _call("halo_model_create", dev.eng, C.byref(cfg), seed, C.byref(h))
        self.h = h

    def close(self):
        if self.h:
            lib().halo_model_destroy(self.h)
            self.h = None

    def _download(self, ptr: int, nbytes: int, dtype):
        out = np.empty(nbytes // np.dtype(dtype).itemsize, dtype)
        b = Buffer(ptr, nbytes, None)
        _call("halo_download", self.dev.handle, C.byref(b), 0, out.ctypes.data, nbytes)
        return out

    def tensor(self, layer: int, name: str):
        """Host copy of a weight: fp32 [rows][cols], or a Q8_0 pair (qs [rows][cols] int8, d [rows][cols/32])."""
        v = TensorView()
        _call("halo_model_tensor", self.h, 0xFFFFFFFF if layer < 0 else layer, name.encode(), C.byref(v))
        if v.kind == 0:
            return self._download(v.data, v.rows * v.cols * 4, np.float32).reshape(v.rows, v.cols)
        qs = self._download(v.data, v.rows * v.qstride, np.int8).reshape(v.rows, v.qstride)[:, : v.cols]
        d = self._download(v.scales, v.rows * (v.cols // 32) * 2, np.uint16).reshape(v.rows, v.cols // 32)
        return np.ascontiguousarray(qs), d

    def _view(self, layer: int, name: str) -> TensorView:
        v = TensorView()
        _call("halo_model_tensor", self.h, 0xFFFFFFFF if layer < 0 else layer, name.encode(), C.byref(v))
        return v

    def tensor_rows(self, layer: int, name: str, r0: int, n: int):
        """Rows [r0, r0 + n) of a weight, as tensor() returns the whole of it (only those rows cross PCIe)."""
        v = self._view(layer, name)
        if v.kind == 0:
            return self._download(v.data + r0 * v.cols * 4, n * v.cols * 4, np.float32).reshape(n, v.cols)
        qs = self._download(v.data + r0 * v.qstride, n * v.qstride, np.int8).reshape(n, v.qstride)[:, : v.cols]
        nb = v.cols // 32
        d = self._download(v.scales + r0 * nb * 2, n * nb * 2, np.uint16).reshape(n, nb)
        return np.ascontiguousarray(qs), d

    def raw(self, layer: int, name: str, dtype=np.float32):
        """A state tensor (state, conv_ring, k_pool, v_pool, pages, nkv) as [rows][cols] of 4-byte `dtype`."""
        v = self._view(layer, name)
        return self._download(v.data, v.rows * v.cols * 4, dtype).reshape(v.rows, v.cols)

    def step_trace(self, S: int, prefix: int = 0) -> dict:
        """One eager step with the teacher-forcing trace: {(layer, name): host array}; layer -1 is the head."""
        return self._trace("halo_model_step_trace", (S, prefix), S)

    def _trace(self, fn, args, T: int, n_layers=None) -> dict:
        cfg = self.cfg
        per_layer = T * (16 * cfg.hidden + 12 * (2 * cfg.gdn_k_heads + 3 * cfg.gdn_v_heads) * cfg.gdn_head_dim +
                         12 * 2 * cfg.q_heads * cfg.head_dim + 4 * cfg.n_experts +
                         8 * (cfg.n_used + 1) * max(cfg.expert_ff, cfg.shared_ff) + 64 * cfg.n_used + 64) + 40 * 256
        nbytes = ((cfg.layers if n_layers is None else n_layers) + 1) * per_layer
        buf = self.dev.array(nbytes, np.uint8)
        maxe = 40 * (cfg.layers + 1)
        ents = (TraceEntry * maxe)()
        n = C.c_uint32()
        try:
            _call(fn, self.h, *args, buf.ptr, nbytes, ents, maxe, C.byref(n))
            self.dev.sync()
            blob = buf.download()
        finally:
            buf.free()
        out = {}
        for e in ents[: n.value]:
            layer = -1 if e.layer == 0xFFFFFFFF else int(e.layer)
            out[(layer, e.name.decode())] = blob[e.offset: e.offset + e.bytes].view(TRACE_DTYPES[e.dtype]).copy()
        return out

    def prefill_trace(self, segments, layers=None) -> dict:
        """halo_model_prefill of (session, start, length) segments (one batch) with the teacher-forcing trace; with
        `layers` (layer indices, -1 for the final norm) only those layers are traced."""
        arr = (PrefillSegment * len(segments))(*[PrefillSegment(s, a, n, 0) for s, a, n in segments])
        T = sum(n for _, _, n in segments)
        if layers is None:
            return self._trace("halo_model_prefill_trace", (arr, len(segments)), T)
        mask = 0
        for l in layers:
            mask |= 1 << (63 if l < 0 else l)
        return self._trace("halo_model_prefill_trace_layers", (arr, len(segments), mask), T,
                           n_layers=len([l for l in layers if l >= 0]))

    def set_sampling(self, s: int, params: "SampleParams", penalties=None):
        """Device sampling for session s; penalties = (token, generated_count, repeated) arrays sorted by token."""
        n = 0 if penalties is None else len(penalties[0])
        pen = np.zeros(max(n, 1), PENALTY_DTYPE)
        if n:
            pen["token"], pen["generated_count"], pen["repeated"] = penalties
        _call("halo_model_set_sampling", self.h, s, C.byref(params), pen.ctypes.data, n)

    def sample_state(self, s: int) -> "SampleParams":
        p = SampleParams()
        _call("halo_model_sample_state", self.h, s, C.byref(p))
        return p

    def load_gguf(self, g: "Gguf"):
        """Every weight from a GGUF checkpoint (halo_model_load_gguf)."""
        _call("halo_model_load_gguf", self.h, g.h)

    def logits(self, s: int) -> np.ndarray:
        out = np.empty(self.cfg.vocab, np.float32)
        _call("halo_model_logits", self.h, s, out.ctypes.data)
        return out

    @property
    def weight_bytes(self) -> int:
        return int(lib().halo_model_weight_bytes(self.h))

    def set_session(self, s: int, prompt, nkv: int = 0):
        p = np.ascontiguousarray(prompt, np.uint32)
        _call("halo_model_set_session", self.h, s, p.ctypes.data, len(p), nkv)

    def fork(self, src: int, dst: int):
        _call("halo_model_fork", self.h, src, dst)

    def reset(self):
        _call("halo_model_reset", self.h)

    def run(self, S: int, steps: int, prefix: int = 0):
        _call("halo_model_run", self.h, S, prefix, steps)

    def step_eager(self, S: int, prefix: int = 0):
        _call("halo_model_step_eager", self.h, S, prefix)

    def prefill(self, segments):
        """Batched prefill of (session, start, length) segments, sessions consecutive and increasing."""
        arr = (PrefillSegment * len(segments))(*[PrefillSegment(s, a, n, 0) for s, a, n in segments])
        _call("halo_model_prefill", self.h, arr, len(segments))

    def history(self, s: int, n: int) -> np.ndarray:
        out = np.zeros(n, np.uint32)
        _call("halo_model_history", self.h, s, out.ctypes.data, n)
        return out

    def positions(self, S: int) -> np.ndarray:
        out = np.zeros(S, np.uint32)
        _call("halo_model_positions", self.h, out.ctypes.data, S)
        return out


class MoeLayer:
    """Seeded synthetic MoE layer on the device (benchmark config C2 shapes by default)."""

    def __init__(self, dev: Device, n_experts=512, n_used=10, hidden=2048, ff=512, shared_ff=512, seed=0,
                 shared=True):
        self.dev = dev
        self.E, self.k, self.H, self.F, self.SF = n_experts, n_used, hidden, ff, shared_ff
        self.router = dev.array((n_experts, hidden), np.float32)
        dev.op("synth_f32", self.router.ptr, n_experts * hidden, seed + 1, 0.02)
        self.gate = Q8Weights(dev, n_experts * ff, hidden).synth(dev, seed + 2)
        self.up = Q8Weights(dev, n_experts * ff, hidden).synth(dev, seed + 3)
        self.down = Q8Weights(dev, n_experts * hidden, ff).synth(dev, seed + 4)
        w = MoeWeights()
        w.router = self.router.ptr
        w.gate, w.up, w.down = self.gate.desc, self.up.desc, self.down.desc
        w.n_experts, w.n_used, w.hidden, w.ff = n_experts, n_used, hidden, ff
        self.shared = shared
        if shared:
            self.sgate = dev.array(hidden, np.float32)
            dev.op("synth_f32", self.sgate.ptr, hidden, seed + 5, 0.02)
            self.sg = Q8Weights(dev, shared_ff, hidden).synth(dev, seed + 6)
            self.su = Q8Weights(dev, shared_ff, hidden).synth(dev, seed + 7)
            self.sd = Q8Weights(dev, hidden, shared_ff).synth(dev, seed + 8)
            w.shared_gate = self.sgate.ptr
            w.shared_gate_proj, w.shared_up, w.shared_down = self.sg.desc, self.su.desc, self.sd.desc
            w.shared_ff = shared_ff
        self.w = w

    def workspace(self, tokens: int):
        n = lib().halo_op_moe_workspace_bytes(C.byref(self.w), tokens)
        if n == 0:
            raise HaloError("moe: unsupported shape")
        return self.dev.array(n, np.uint8)

    def views(self, tokens: int, ws: DeviceArray) -> MoeViews:
        v = MoeViews()
        _call("halo_op_moe_views", C.byref(self.w), tokens, ws.ptr, C.byref(v))
        return v

    def forward(self, x: DeviceArray, out: DeviceArray, tokens: int, ws: DeviceArray):
        self.dev.op("moe_decode", C.byref(self.w), x.ptr, out.ptr, tokens, ws.ptr, ws.nbytes)

    def forward_norm(self, res: DeviceArray, delta: DeviceArray, norm_w: DeviceArray, res_out: DeviceArray,
                     out: DeviceArray, tokens: int, ws: DeviceArray, eps: float = 1e-6):
        """MoE(RMSNorm(res + delta) * norm_w), the norm in the router launch; res_out receives res + delta."""
        inp = ProjInput(x=res.ptr, delta=delta.ptr, norm_w=norm_w.ptr, res_out=res_out.ptr, eps=eps, mode=PROJ_N)
        self.dev.op("moe_decode_norm", C.byref(self.w), C.byref(inp), out.ptr, tokens, ws.ptr, ws.nbytes)

    def prefill_workspace(self, tokens: int):
        n = lib().halo_op_moe_prefill_workspace_bytes(C.byref(self.w), tokens)
        if n == 0:
            raise HaloError("moe prefill: unsupported shape")
        return self.dev.array(n, np.uint8)

    def prefill_views(self, tokens: int):
        """Byte offsets of the router logits, shared logit and the ids / weights in the prefill workspace."""
        al = lambda b: (b + 255) // 256 * 256
        T, E, H, k = tokens, self.E, self.H, self.k
        o_logits = 0
        o_sgl = o_logits + al(T * E * 4)
        o_ids = o_sgl + al(T * 4) + al(T * H) + al(T * H // 8)
        o_w = o_ids + al(T * k * 4)
        return o_logits, o_sgl, o_ids, o_w

    def prefill_h_views(self, tokens: int):
        """Byte offsets of pos [T k] (each routed pair's row in the grouped order; the shared expert's rows follow at
        T k + t) and of the quantized h rows hq [G][ff] int8 / hs [G][ff / 32] fp32 in the prefill workspace (the
        layout of MoePrefillLayout, csrc/engine/moe.cpp)."""
        al = lambda b: (b + 255) // 256 * 256
        T, E, H, k, F = tokens, self.E, self.H, self.k, self.F
        P = T * k
        G = P + T  # the shared expert is present in every MoeLayer
        tile = 128 if P >= 96 * E else 64
        max_tiles = -(-G // tile) + E + 1
        o = self.prefill_views(T)[3] + al(P * 4)  # past the weights
        o += al(-(-P // 4096) * E * 4)  # count histograms
        o += al((E + 2) * 4)  # start
        o += al(3 * max_tiles * 4) + al(4)  # tiles, ntiles
        o += al(G * 4)  # token
        o_pos = o
        o += al(P * 4)
        o += al(G * F * 4)  # h
        o_hq = o
        o_hs = o + al(G * F)
        return o_pos, o_hq, o_hs

    def forward_prefill(self, x: DeviceArray, out: DeviceArray, tokens: int, ws: DeviceArray):
        self.dev.op("moe_prefill", C.byref(self.w), x.ptr, out.ptr, tokens, ws.ptr, ws.nbytes)
