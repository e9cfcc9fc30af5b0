"""The allocation-free loss entry point (b2c_hip_photometric_noalloc, include/b2c_kernels.h) against the
regular one (b2c_hip_photometric with a caller-provided partials workspace), called through the C ABI on
device buffers of the library's own (b2c_device_upload, default stream): two calls in a row, the second on a smaller image, each bit-identical to the
regular entry point in the loss value and every per-pixel gradient, in assign mode (loss stored, running
sum updated) and in add mode (loss added to loss_accum[0]). The regular entry point runs first on
each input, then the allocation-free one, so its fixed scratch holds the previous call's partials (stale
contents must not leak into the result)."""
import ctypes as C

import numpy as np
import pytest

from b2ctrain_amd import _native
from tests.gpu_harness import emit

pytestmark = pytest.mark.gpu


class LossArgs(C.Structure):
    _fields_ = [("pred", C.c_void_p), ("gt", C.c_void_p), ("weights", C.c_void_p), ("W", C.c_int), ("H", C.c_int),
                ("l1_w", C.c_float), ("ssim_w", C.c_float), ("bg", C.c_float * 3), ("composite", C.c_int),
                ("mask", C.c_int), ("alpha_lane", C.c_int), ("match_alpha_weight", C.c_float), ("scale", C.c_float),
                ("grad_scale", C.c_float), ("v_out", C.c_void_p), ("loss_accum", C.c_void_p), ("partials", C.c_void_p),
                ("assign", C.c_int), ("running", C.c_int), ("defer_sum_count", C.c_void_p)]


def _inputs(W, H, seed, weights):
    g = np.random.default_rng(seed)
    P = W * H
    pred = g.random((P, 4), dtype=np.float32)
    gt = g.integers(0, 1 << 32, P, dtype=np.uint64).astype(np.uint32)
    t = dict(pred=_native.DeviceArray(pred), gt=_native.DeviceArray(gt))
    t["w"] = _native.DeviceArray(g.integers(85, 256, P).astype(np.uint8)) if weights else None
    return t


def _call(fn, t, W, H, opts, partials, assign):
    a = LossArgs()
    a.pred, a.gt = t["pred"].ptr, t["gt"].ptr
    a.weights = t["w"].ptr if t["w"] is not None else None
    a.W, a.H = W, H
    a.l1_w, a.ssim_w = 0.8, -0.2
    for k in range(3):
        a.bg[k] = opts["bg"][k]
    a.composite, a.mask, a.alpha_lane = opts["composite"], opts["mask"], opts["alpha_lane"]
    a.match_alpha_weight, a.scale, a.grad_scale = 0.1, opts["scale"], 3.0 * W * H
    v_out = _native.DeviceArray(np.zeros((W * H, 4), np.float32))
    acc = _native.DeviceArray(np.full(16, 0.25, np.float32))  # assign mode overwrites [0..3]; add mode adds to [0]
    try:
        a.v_out, a.loss_accum = v_out.ptr, acc.ptr
        a.partials = partials
        a.assign, a.running = assign, assign
        rc = fn(C.byref(a), None)  # the default stream; the downloads below wait for it
        assert rc == 0, f"launcher returned {rc}"
        return v_out.download(np.float32, (W * H, 4)), acc.download(np.float32, 16)
    finally:
        v_out.free()
        acc.free()


def test_noalloc_loss_matches_workspace_loss_twice():
    L = _native.lib()
    L.b2c_hip_photometric.argtypes = [C.c_void_p, C.c_void_p]
    L.b2c_hip_photometric_noalloc.argtypes = [C.c_void_p, C.c_void_p]
    L.b2c_loss_partials.restype = C.c_size_t
    cases = [(1920, 1080, dict(bg=(0.4, 0.3, 0.2), composite=1, mask=0, alpha_lane=1, scale=1.5), True),
             (640, 360, dict(bg=(0.0, 0.0, 0.0), composite=0, mask=1, alpha_lane=0, scale=1.0), False)]
    for k, (W, H, opts, weights) in enumerate(cases):
        emit(f"no-alloc loss call {k + 1}: {W}x{H}")
        t = _inputs(W, H, 100 + k, weights)
        ws = _native.DeviceArray(np.zeros(int(L.b2c_loss_partials(W, H)), np.float32))
        for assign in (1, 0):
            v_ref, acc_ref = _call(L.b2c_hip_photometric, t, W, H, opts, ws.ptr, assign)
            v_na, acc_na = _call(L.b2c_hip_photometric_noalloc, t, W, H, opts, None, assign)
            assert acc_ref[0] > (0 if assign else 0.25) and acc_ref[3] == (1 if assign else 0.25)
            assert np.array_equal(acc_na[:4], acc_ref[:4]), (assign, acc_na[:4], acc_ref[:4])
            assert np.array_equal(v_na, v_ref), f"assign={assign}: {int((v_na != v_ref).sum())} gradient entries differ"
            assert np.abs(v_ref).max() > 0
