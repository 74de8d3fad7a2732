"""The C-ABI library loads on the CPU and exports every function the public headers declare; the embedded code
object targets gfx950 and contains every kernel the host layer launches. No compute calls (no GPU here)."""
import re
from pathlib import Path

import pytest

import halo_amd as H

ROOT = Path(__file__).resolve().parent.parent


def test_library_exports_every_declared_symbol():
    L = H.lib()
    names = H.declared_symbols()
    assert len(names) > 30
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, missing


def test_binding_covers_declarations():
    # every declared function has a ctypes signature in the binding (so tests call through the real ABI)
    names = set(H.declared_symbols())
    assert names <= set(H._SIGS), sorted(names - set(H._SIGS))


def _code_object() -> bytes:
    import ctypes

    n = ctypes.c_size_t()
    p = H.lib().halo_core_code_object(ctypes.byref(n))
    return ctypes.string_at(p, n.value)


def test_code_object_is_gfx950_elf():
    co = _code_object()
    assert co[:4] == b"\x7fELF"
    assert b"gfx950" in co


def test_code_object_has_every_listed_kernel():
    co = _code_object()
    text = (ROOT / "include" / "halo_kernels.h").read_text()
    listed = re.findall(r"X\((halo_\w+)\)", text)
    assert listed
    for name in listed:
        assert (name + ".kd").encode() in co, name


def test_errors_are_reported_not_raised_in_c():
    # A null device fails cleanly with a message (no GPU needed).
    import ctypes

    err = ctypes.create_string_buffer(256)
    rc = H.lib().halo_alloc(None, 16, ctypes.byref(H.Buffer()), err, 256)
    assert rc == -1 and b"null" in err.value


def test_ops_refuse_null_required_pointers():
    """Every operator checks its required device pointers before touching the engine or the GPU (a null read faults
    the GPU); the refusal names the argument."""
    import ctypes

    L = H.lib()
    err = ctypes.create_string_buffer(256)
    m = H.Q8Matrix()
    calls = {
        "halo_op_quantize_q8": (None, None, None, None, 1, 64),
        "halo_op_matvec_q8a8": (None, ctypes.byref(m), None, None, None, 1, 64),
        "halo_op_matvec_q8_f32x": (None, ctypes.byref(m), None, None),
        "halo_op_repack_q8_0": (None, None, None, None, 4, 64, 64),
        "halo_op_gdn_decode": (None, None, None, None, None, None, None, None, 1, 32, 16, 128),
        "halo_op_kv_append": (None, None, None, None),
        "halo_op_moe_decode": (None, None, None, None, 1, None, 0),
        "halo_op_synth_f32": (None, None, 16, 1, ctypes.c_float(1.0)),
    }
    for name, args in calls.items():
        rc = getattr(L, name)(*args, err, 256)
        assert rc == -1 and b"is null" in err.value, (name, err.value)


def test_device_layer_refuses_null_handles():
    import ctypes

    L = H.lib()
    err = ctypes.create_string_buffer(256)
    b = H.Buffer()
    assert L.halo_reserve_range(None, 1 << 21, ctypes.byref(b), err, 256) == -1
    assert L.halo_map_page(None, ctypes.byref(b), 0, None, err, 256) == -1
    assert L.halo_read_global(None, b"x", None, 4, err, 256) == -1
    assert L.halo_launch_graph(None, None, err, 256) == -1
    assert L.halo_page_bytes(None) == 0


def test_moe_noalloc_refusals_on_the_host():
    """halo_op_moe_decode_noalloc refuses, before touching any device, a workspace above its fixed scratch and a
    missing engine (whose device selects which GPU's scratch array is used); the device ordinal of a null device is
    -1. Tensor pointers are placeholders that are never dereferenced."""
    import ctypes

    L = H.lib()
    err = ctypes.create_string_buffer(256)
    w = H.MoeWeights()
    E, k, Hd, F = 1024, 15, 4096, 512  # within the decode limits; 16 tokens need more than the 512 KiB scratch
    fake = 1 << 40
    w.router = fake
    for name, rows, cols in (("gate", E * F, Hd), ("up", E * F, Hd), ("down", E * Hd, F)):
        m = getattr(w, name)
        m.qs, m.d, m.rows, m.cols, m.qstride = fake, fake, rows, cols, cols
    w.n_experts, w.n_used, w.hidden, w.ff = E, k, Hd, F
    assert L.halo_op_moe_workspace_bytes(ctypes.byref(w), 16) > (512 << 10)
    rc = L.halo_op_moe_decode_noalloc(None, ctypes.byref(w), fake, fake, 16, err, 256)
    assert rc == -1 and b"fixed scratch" in err.value, err.value
    rc = L.halo_op_moe_decode_noalloc(None, ctypes.byref(w), fake, fake, 1, err, 256)
    assert rc == -1 and b"null engine" in err.value, err.value
    rc = L.halo_op_moe_decode_noalloc(None, ctypes.byref(w), None, fake, 1, err, 256)
    assert rc == -1 and b"null" in err.value, err.value
    assert L.halo_device_ordinal(None) == -1


def test_code_object_mach():
    """The embedded object is recognised as gfx950; another AMDGPU target's ELF header reports its own processor
    (the adapter then loads the embedded object instead); bytes that are no AMDGPU ELF64 give -1."""
    import ctypes

    L = H.lib()
    co = _code_object()
    assert L.halo_code_object_mach(co, len(co)) == 0x4F
    other = bytearray(co[:64])
    other[48] = 0x4A  # another processor's EF_AMDGPU_MACH
    assert L.halo_code_object_mach(bytes(other), 64) == 0x4A
    x86 = bytearray(co[:64])
    x86[18], x86[19] = 62, 0  # EM_X86_64
    assert L.halo_code_object_mach(bytes(x86), 64) == -1
    assert L.halo_code_object_mach(b"not an elf" * 8, 80) == -1
    assert L.halo_code_object_mach(None, 0) == -1
