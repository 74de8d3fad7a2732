"""GPU checks of the device layer's page mapping and module-variable entry points (include/halo_rt.h; the
reference's rt::Device PageBytes ... UnmapPage and ReadGlobal / WriteGlobal, src/rt/device.hpp:101-126).

One physical page is mapped into two reserved ranges at different offsets; bytes written through either range
(a host upload, a kernel's stores) read back through the other, exactly. A module-scope variable of the code object
reads its initial value, takes a write, and a kernel then sees the written value."""
import ctypes as C

import numpy as np
import pytest

import halo_amd as H

pytestmark = pytest.mark.gpu


def test_one_page_mapped_into_two_ranges(dev):
    L = H.lib()
    pb = int(L.halo_page_bytes(dev.handle))
    if pb == 0:
        pytest.skip("device without virtual memory management")
    assert pb % (2 << 20) == 0
    a, b = H.Buffer(), H.Buffer()
    H._call("halo_reserve_range", dev.handle, 2 * pb, C.byref(a))
    H._call("halo_reserve_range", dev.handle, 2 * pb, C.byref(b))
    page = C.c_void_p()
    H._call("halo_create_page", dev.handle, C.byref(page))
    try:
        H._call("halo_map_page", dev.handle, C.byref(a), 0, page)
        H._call("halo_map_page", dev.handle, C.byref(b), pb, page)
        rng = np.random.default_rng(1)
        # a host upload through range a, read back through range b
        x = rng.integers(0, 2**32, 4096, dtype=np.uint32)
        H._call("halo_upload", dev.handle, C.byref(a), 0, x.ctypes.data, x.nbytes)
        got = np.empty_like(x)
        H._call("halo_download", dev.handle, C.byref(b), pb, got.ctypes.data, got.nbytes)
        assert np.array_equal(got, x)
        # a kernel's stores through range b (past the first 16 KB of the page), read through range a
        y = rng.normal(0, 1, 8192).astype(np.float32)
        src = dev.to_device(y)
        dev.launch("halo_copy", (8,), (256,), [("ptr", b.device + pb + 16384), src, ("u32", y.size)])
        dev.sync()
        got = np.empty_like(y)
        H._call("halo_download", dev.handle, C.byref(a), 16384, got.ctypes.data, got.nbytes)
        assert got.tobytes() == y.tobytes()
        # and a kernel reading through range a what the host wrote through range b
        z = rng.normal(0, 1, 1024).astype(np.float32)
        H._call("halo_upload", dev.handle, C.byref(b), pb + 65536, z.ctypes.data, z.nbytes)
        out = dev.array(1024, np.float32)
        dev.launch("halo_copy", (1,), (256,), [out, ("ptr", a.device + 65536), ("u32", 1024)])
        assert out.download().tobytes() == z.tobytes()
        # offsets that are not pages are refused
        with pytest.raises(H.HaloError):
            H._call("halo_map_page", dev.handle, C.byref(a), pb // 2, page)
        H._call("halo_unmap_page", dev.handle, C.byref(a), 0)
        H._call("halo_unmap_page", dev.handle, C.byref(b), pb)
    finally:
        L.halo_release_page(dev.handle, page)
        L.halo_release_range(dev.handle, C.byref(a))
        L.halo_release_range(dev.handle, C.byref(b))
    assert a.device is None and b.device is None


def test_module_variable_read_write(dev):
    info = np.zeros(4, np.uint32)
    H._call("halo_read_global", dev.handle, b"halo_code_object_info", info.ctypes.data, info.nbytes)
    assert info.tolist() == [1, 64, 950, 0]
    new = np.array([5, 6, 7, 8], np.uint32)
    out = dev.array(4, np.uint32)
    try:
        H._call("halo_write_global", dev.handle, b"halo_code_object_info", new.ctypes.data, new.nbytes)
        dev.launch("halo_code_object_info_copy", (1,), (64,), [out])
        assert out.download().tolist() == [5, 6, 7, 8]
    finally:
        H._call("halo_write_global", dev.handle, b"halo_code_object_info", info.ctypes.data, info.nbytes)
    with pytest.raises(H.HaloError):
        H._call("halo_read_global", dev.handle, b"no_such_variable", info.ctypes.data, 4)
    big = np.zeros(8, np.uint32)
    with pytest.raises(H.HaloError, match="requested"):
        H._call("halo_read_global", dev.handle, b"halo_code_object_info", big.ctypes.data, big.nbytes)
