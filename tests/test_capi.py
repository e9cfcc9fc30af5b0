"""The C-ABI library loads and exports every symbol include/b2c.h and include/b2c_kernels.h declare
(no GPU call is made), and its host-only CameraGPU::from agrees with the float32 restatement."""
import ctypes
import os
import re

import numpy as np

from b2ctrain_amd import _native
from b2ctrain_amd import scenes as S

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    names = set()
    for h in ("b2c.h", "b2c_kernels.h"):
        text = open(os.path.join(ROOT, "include", h)).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names |= set(re.findall(r"\b(b2c_\w+)\s*\(", text))
    return names


def test_library_exports_every_declared_symbol():
    L = _native.lib()
    declared = declared_symbols()
    assert len(declared) >= 40
    missing = [n for n in sorted(declared) if not hasattr(L, n)]
    assert not missing, missing
    assert declared == set(_native.EXPORTS), declared ^ set(_native.EXPORTS)


def test_camera_gpu_from_matches_float32_restatement():
    for sc in (S.config1(), S.fd_scene(7)):
        a = _native.camera_gpu_from(sc.cam)
        b = S.camera_gpu(sc.cam)
        for k in ("R", "t", "pos", "fx", "fy", "cx", "cy", "lim_pos_x", "lim_pos_y", "lim_neg_x", "lim_neg_y"):
            assert np.array_equal(np.asarray(a[k], np.float32), np.asarray(b[k], np.float32)), k
        assert (a["W"], a["H"]) == (b["W"], b["H"])


def test_camera_rescale_to_render_size():
    sc = S.config2(n=10)
    a = _native.camera_gpu_from(sc.cam, 400, 400)
    assert a["W"] == 400 and abs(float(a["fx"]) - sc.cam.fx / 2) < 1e-3


def test_temp_sizes_are_monotone():
    L = _native.lib()
    sizes = [L.b2c_radix_sort_temp_bytes(n) for n in (1, 4096, 4097, 1 << 20, 1 << 24)]
    assert sizes == sorted(sizes) and sizes[0] > 0
    assert L.b2c_scan_temp_bytes(1 << 20) >= 4 * 256


def test_noalloc_loss_rejects_images_beyond_its_scratch():
    """The allocation-free loss checks the image against its fixed partials array before any HIP call."""
    import ctypes as C
    L = _native.lib()
    L.b2c_loss_partials.restype = C.c_size_t
    W = H = 32768
    assert L.b2c_loss_partials(W, H) > (1 << 18)
    args = (C.c_char * 256)()  # a zeroed b2c_loss_args: null pointers, then W and H
    C.memmove(C.addressof(args) + 3 * C.sizeof(C.c_void_p), (C.c_int * 2)(W, H), 8)
    L.b2c_hip_photometric_noalloc.argtypes = [C.c_void_p, C.c_void_p]
    assert L.b2c_hip_photometric_noalloc(C.addressof(args), None) == 1  # hipErrorInvalidValue
