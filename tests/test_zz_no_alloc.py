"""halo_op_moe_decode_noalloc (the MoE decode layer with its workspace in the library's fixed device scratch) against
halo_op_moe_decode with a caller workspace, through the C ABI: the same kernels on the same inputs, so the outputs
must be equal bit for bit. Two calls in a row, the second with fewer tokens (the scratch keeps the first call's
contents), then the first shape again; a token count whose workspace exceeds the scratch is refused with an error.
"""
import ctypes

import numpy as np
import pytest

import halo_amd as H

pytestmark = pytest.mark.gpu


def test_moe_decode_noalloc_matches_workspace_entry_point(dev):
    layer = H.MoeLayer(dev, seed=42)  # C2 shapes: 512 experts top-10 + shared, hidden 2048, ff 512
    rng = np.random.default_rng(7)
    for T in (16, 3, 16):
        x = dev.to_device(rng.normal(0, 1, (T, layer.H)).astype(np.float32))
        want, got = dev.array((T, layer.H), np.float32), dev.array((T, layer.H), np.float32)
        ws = layer.workspace(T)
        layer.forward(x, want, T, ws)
        dev.op("moe_decode_noalloc", ctypes.byref(layer.w), x.ptr, got.ptr, T)
        a, b = want.download(), got.download()
        assert np.isfinite(a).all()
        assert a.tobytes() == b.tobytes(), f"T={T}: max diff {np.abs(a - b).max()}"


def test_moe_decode_noalloc_refuses_oversized(dev):
    """A layer within the decode limits whose workspace exceeds the 512 KiB scratch (1024 experts top-15, hidden 4096,
    16 tokens) is refused before any launch; its tensor pointers are placeholders that are never dereferenced."""
    w = H.MoeWeights()
    E, k, Hd, F = 1024, 15, 4096, 512
    fake = 1 << 40
    w.router = fake
    for name, rows, cols in (("gate", E * F, Hd), ("up", E * F, Hd), ("down", E * Hd, F)):
        m = getattr(w, name)
        m.qs, m.d, m.rows, m.cols, m.qstride = fake, fake, rows, cols, cols
    w.n_experts, w.n_used, w.hidden, w.ff = E, k, Hd, F
    assert H.lib().halo_op_moe_workspace_bytes(ctypes.byref(w), 16) > (512 << 10)
    x, out = dev.array((16, Hd), np.float32), dev.array((16, Hd), np.float32)
    with pytest.raises(H.HaloError, match="fixed scratch"):
        dev.op("moe_decode_noalloc", ctypes.byref(w), x.ptr, out.ptr, 16)
