"""TEST INFRASTRUCTURE ONLY: ctypes bindings for the CPU oracle (oracle/liborc.so) and for the
reference's own fp64 CPU loss compiled from /root/reference (oracle/_ref/libb2c_ref.so).

Used by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg only — never by the product.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liborc.so")
REF_PATH = os.path.join(HERE, "_ref", "libb2c_ref.so")

RT_W = 8
GRAD_LANES = 13


class OrcCam(C.Structure):
    _fields_ = [("R", C.c_float * 9), ("t", C.c_float * 3), ("pos", C.c_float * 3), ("fx", C.c_float),
                ("fy", C.c_float), ("cx", C.c_float), ("cy", C.c_float), ("W", C.c_int), ("H", C.c_int),
                ("lim_pos_x", C.c_float), ("lim_pos_y", C.c_float), ("lim_neg_x", C.c_float),
                ("lim_neg_y", C.c_float)]


class OrcModel(C.Structure):
    _fields_ = [("n", C.c_int), ("degree", C.c_int), ("pos_op", C.c_void_p), ("quat", C.c_void_p),
                ("lscale", C.c_void_p), ("sh", C.c_void_p)]


class OrcLoss(C.Structure):
    _fields_ = [("l1_w", C.c_float), ("ssim_w", C.c_float), ("bg", C.c_float * 3), ("composite", C.c_int),
                ("mask", C.c_int), ("alpha_lane", C.c_int), ("match_alpha_weight", C.c_float),
                ("scale", C.c_float), ("grad_scale", C.c_float)]


class OrcExt(C.Structure):
    _fields_ = [("feat", C.c_int), ("proj3", C.c_void_p), ("hollow_z", C.c_void_p), ("hollow_margin", C.c_float),
                ("hollow_lam", C.c_float), ("out_feat", C.c_void_p), ("hollow_pen", C.c_void_p), ("v_feat", C.c_void_p)]


class OrcRefExt(C.Structure):
    _fields_ = [("normals", C.c_int), ("gtn", C.c_void_p), ("normal_scale", C.c_double), ("hollow_z", C.c_void_p),
                ("hollow_lam", C.c_double), ("hollow_margin", C.c_double)]


class OrcAdamStep(C.Structure):
    _fields_ = [("t", C.c_int), ("sparse", C.c_int), ("beta1", C.c_float), ("beta2", C.c_float), ("eps", C.c_float),
                ("bc1", C.c_float), ("bc2", C.c_float), ("ln_beta1", C.c_float), ("ln_beta2", C.c_float),
                ("ratio", C.c_float), ("ln_ratio", C.c_float), ("lr_mean", C.c_float), ("lr_rot", C.c_float),
                ("lr_scale", C.c_float), ("lr_opac", C.c_float), ("lr_dc", C.c_float), ("lr_sh_rest", C.c_float),
                ("noise_weight", C.c_float), ("noise_clamp", C.c_float), ("seed", C.c_uint32), ("step", C.c_uint32)]


class OrcAdamModel(C.Structure):
    _fields_ = [("n", C.c_int), ("degree", C.c_int), ("sh_half", C.c_int)] + [
        (k, C.c_void_p) for k in ("pos_op", "quat", "lscale", "sh", "m_pos_op", "v_pos_op", "m_quat", "v_quat",
                                  "m_lscale", "v_lscale", "m_sh", "v_sh", "last_step")]


_lib = None
_ref = None


def build(with_ref: bool | None = None) -> None:
    """Compile liborc.so (and _ref/ when the reference tree is mounted)."""
    subprocess.check_call(["make", "-s", "-B", "-C", HERE, "all"])
    if with_ref is None:
        with_ref = os.path.isdir("/root/reference/tests")
    if with_ref:
        subprocess.check_call(["make", "-s", "-B", "-C", HERE, "ref"])


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build(with_ref=False)
        _lib = C.CDLL(LIB_PATH)
        f = C.c_float
        p = C.c_void_p
        _lib.orc_expf.restype = f; _lib.orc_expf.argtypes = [f]
        _lib.orc_logf.restype = f; _lib.orc_logf.argtypes = [f]
        _lib.orc_tile_bits.restype = C.c_int; _lib.orc_tile_bits.argtypes = [C.c_int]
        _lib.orc_project.restype = None
        _lib.orc_project.argtypes = [C.POINTER(OrcModel), C.POINTER(OrcCam), C.c_int, C.c_int, C.c_int] + [p] * 6
        _lib.orc_bin.restype = C.c_uint32
        _lib.orc_bin.argtypes = [C.c_int, p, p, p, p, C.c_int, C.c_int, C.c_uint32, p, p, p, p, p]
        _lib.orc_raster_fwd.restype = None
        _lib.orc_last_fwd_contrib.restype = C.c_uint64
        _lib.orc_raster_fwd.argtypes = [C.c_int] * 4 + [p] * 9
        _lib.orc_photometric.restype = C.c_double
        _lib.orc_photometric.argtypes = [C.c_int, C.c_int, p, p, p, C.POINTER(OrcLoss), p]
        _lib.orc_raster_bwd.restype = None
        _lib.orc_raster_bwd.argtypes = [C.c_int] * 4 + [p] * 10 + [f, p, p, p]
        _lib.orc_vjp.restype = None
        _lib.orc_vjp.argtypes = [C.POINTER(OrcModel), C.POINTER(OrcCam), C.c_int, p, p, p, p]
        _lib.orc_sh_basis_f.restype = None
        _lib.orc_sh_basis_f.argtypes = [C.c_int, f, f, f, p]
        _lib.orc_sh_basis_d.restype = None
        _lib.orc_sh_basis_d.argtypes = [C.c_int, C.c_double, C.c_double, C.c_double, p]
        _lib.orc_quat_to_mat.restype = None
        _lib.orc_quat_to_mat.argtypes = [p, p]
        _lib.orc_tile_hit.restype = C.c_int
        _lib.orc_tile_hit.argtypes = [f] * 10
        _lib.orc_ref_loss.restype = C.c_double
        _lib.orc_ref_loss.argtypes = [C.c_int, C.c_int] + [p] * 6 + [C.POINTER(OrcCam), C.c_int, C.c_int, p, p, p,
                                                                    C.c_int, C.c_int, C.c_int] + [C.c_double] * 4 + [
                                                                    C.c_int, p]
        _lib.orc_ref_set_sample.restype = None
        _lib.orc_ref_set_sample.argtypes = [C.c_uint64]
        _lib.orc_ref_composite_seconds.restype = C.c_double
        _lib.orc_frag_sigma.restype = None
        _lib.orc_frag_sigma.argtypes = [C.c_int] + [p] * 8
        _lib.orc_set_threads.restype = None
        _lib.orc_set_threads.argtypes = [C.c_int]
        _lib.orc_max_screen.restype = None
        _lib.orc_max_screen.argtypes = [C.POINTER(OrcModel), C.POINTER(OrcCam), p]
        _lib.orc_project_feat.restype = None
        _lib.orc_project_feat.argtypes = [C.POINTER(OrcModel), C.POINTER(OrcCam), C.c_int, C.c_int, C.c_int] + [p] * 6 + [
            C.c_int, p]
        _lib.orc_raster_fwd_ext.restype = None
        _lib.orc_raster_fwd_ext.argtypes = [C.c_int] * 4 + [p] * 9 + [C.POINTER(OrcExt)]
        _lib.orc_raster_bwd_ext.restype = None
        _lib.orc_raster_bwd_ext.argtypes = [C.c_int] * 4 + [p] * 10 + [f, p, p, p, C.POINTER(OrcExt)]
        _lib.orc_normal_loss.restype = C.c_double
        _lib.orc_normal_loss.argtypes = [C.c_int, C.c_int, p, p, p, f, f, p]
        _lib.orc_hollow_sum.restype = C.c_double
        _lib.orc_hollow_sum.argtypes = [C.c_int, p]
        _lib.orc_eval.restype = None
        _lib.orc_eval.argtypes = [C.c_int, C.c_int, p, p, C.c_int, p, p]
        _lib.orc_evidence_view.argtypes = [C.c_int] * 4 + [p] * 11 + [C.c_int, f, p, p]
        _lib.orc_probe.argtypes = [C.c_int] * 4 + [p] * 4 + [f, f, p, f, p]
        _lib.orc_ref_loss_ext.restype = C.c_double
        _lib.orc_ref_loss_ext.argtypes = [C.c_int, C.c_int] + [p] * 6 + [C.POINTER(OrcCam), C.c_int, C.c_int, p, p, p,
                                                                        C.c_int, C.c_int, C.c_int] + [C.c_double] * 4 + [
                                                                        C.c_int, p, C.POINTER(OrcRefExt)]
        _lib.orc_project_ok.restype = C.c_int
        _lib.orc_project_ok.argtypes = [p, p, p, C.POINTER(OrcCam)]
        _lib.orc_adam_constants.restype = None
        _lib.orc_adam_constants.argtypes = [C.POINTER(OrcAdamStep)]
        _lib.orc_adam_update.restype = None
        _lib.orc_adam_update.argtypes = [C.POINTER(OrcAdamModel), C.POINTER(OrcCam), C.c_int, p, p, p, p,
                                         C.POINTER(OrcAdamStep)]
        u32 = C.c_uint32
        _lib.orc_hash_unit.restype = f; _lib.orc_hash_unit.argtypes = [u32, u32, u32]
        _lib.orc_mix32.restype = u32; _lib.orc_mix32.argtypes = [u32]
        _lib.orc_hash_gauss.restype = f; _lib.orc_hash_gauss.argtypes = [u32, u32, u32]
        _lib.orc_cos_turns.restype = f; _lib.orc_cos_turns.argtypes = [f]
        _lib.orc_f16_bits.restype = C.c_uint16; _lib.orc_f16_bits.argtypes = [f]
        _lib.orc_f16_value.restype = f; _lib.orc_f16_value.argtypes = [C.c_uint16]
        _lib.orc_f16_stochastic.restype = C.c_uint16; _lib.orc_f16_stochastic.argtypes = [f, f]
    return _lib


def frag_sigma(mx, my, c00, c01, c11, pcx, pcy):
    """The raster kernels' fragment sigma of splats (centre mx, my; conic c00, c01, c11) at pixel centres
    (pcx, pcy): the quadratic about the centre of the pixel's 8x8 tile (float32, broadcast to one shape)."""
    vals = (mx, my, c00, c01, c11, pcx, pcy)
    shape = np.broadcast_shapes(*[np.shape(v) for v in vals])
    arrs = [np.ascontiguousarray(np.broadcast_to(np.asarray(v, np.float32), shape)).ravel() for v in vals]
    out = np.empty(arrs[0].size, np.float32)
    lib().orc_frag_sigma(out.size, *[_ptr(a) for a in arrs], _ptr(out))
    return out.reshape(shape)


def set_threads(n: int) -> None:
    """Host threads of the tiled raster passes (1 = fixed summation order, the tests' setting)."""
    lib().orc_set_threads(int(n))


def ref_render_sample_seconds(scene, stride, bg=None) -> float:
    """Time the fp64 brute-force render (the reference's CPU algorithm, one thread) over every stride-th
    pixel: the compositing seconds (projection and depth sort excluded)."""
    L = lib()
    L.orc_ref_set_sample(int(stride))
    try:
        ref_loss(scene, bg=bg)
        return float(L.orc_ref_composite_seconds())
    finally:
        L.orc_ref_set_sample(1)


def ref_available() -> bool:
    return os.path.exists(REF_PATH)


def ref_lib():
    global _ref
    if _ref is None:
        if not ref_available():
            raise FileNotFoundError(REF_PATH)
        _ref = C.CDLL(REF_PATH)
        p = C.c_void_p
        _ref.ref_reference_loss.restype = C.c_double
        _ref.ref_reference_loss.argtypes = [C.c_int, C.c_int] + [p] * 5 + [C.c_int, C.c_int, p, p] + [C.c_float] * 4 + [
            p, p, p, C.c_int, C.c_int, C.c_int] + [C.c_double] * 4
        _ref.ref_reference_loss_ext.restype = C.c_double
        _ref.ref_reference_loss_ext.argtypes = _ref.ref_reference_loss.argtypes + [p, C.c_double, p, C.c_double,
                                                                                   C.c_double]
    return _ref


def _ptr(a):
    if a is None:
        return None
    if not a.flags["C_CONTIGUOUS"]:
        raise ValueError("oracle arrays must be C-contiguous (a strided view would be read as packed)")
    return a.ctypes.data_as(C.c_void_p)


def _in(a, dtype):
    """Contiguous copy (if needed) of an input array."""
    return np.ascontiguousarray(a, dtype)


def make_cam(camd: dict) -> OrcCam:
    c = OrcCam()
    for i in range(9):
        c.R[i] = float(camd["R"][i])
    for i in range(3):
        c.t[i] = float(camd["t"][i])
        c.pos[i] = float(camd["pos"][i])
    for k in ("fx", "fy", "cx", "cy", "lim_pos_x", "lim_pos_y", "lim_neg_x", "lim_neg_y"):
        setattr(c, k, float(camd[k]))
    c.W, c.H = int(camd["W"]), int(camd["H"])
    return c


class _Model:
    def __init__(self, scene):
        self.arrays = [np.ascontiguousarray(a, np.float32) for a in (scene.pos_op, scene.quat, scene.lscale, scene.sh)]
        self.m = OrcModel(scene.n, scene.degree, *[_ptr(a) for a in self.arrays])


def loss_params(scene, grad_scale=1.0, bg=None) -> OrcLoss:
    lp = OrcLoss()
    lp.l1_w, lp.ssim_w = scene.l1_w, scene.ssim_w
    b = scene.bg if bg is None else bg
    for i in range(3):
        lp.bg[i] = float(b[i])
    lp.composite, lp.mask, lp.alpha_lane = int(scene.composite), int(scene.mask), int(scene.alpha_lane)
    lp.match_alpha_weight, lp.scale, lp.grad_scale = scene.match_alpha_weight, scene.scale, grad_scale
    return lp


def expf(x: float) -> float:
    return lib().orc_expf(x)


def logf(x: float) -> float:
    return lib().orc_logf(x)


def tile_geometry(W, H):
    tx, ty = (W + RT_W - 1) // RT_W, (H + RT_W - 1) // RT_W
    return tx, ty, tx * ty, lib().orc_tile_bits(tx * ty)


def project(scene, camd, active_deg=None):
    """Projection with the scene's feature mode (scene.feat_mode / feat_buffer)."""
    n = scene.n
    tx, ty, _, _ = tile_geometry(camd["W"], camd["H"])
    out = dict(proj0=np.zeros((n, 4), np.float32), proj1=np.zeros((n, 4), np.float32),
               proj2=np.zeros((n, 4), np.float32), proj3=np.zeros((n, 2), np.float32),
               tile_count=np.zeros(n, np.uint32), hit_info=np.zeros((n, 2), np.uint32))
    m = _Model(scene)
    cam = make_cam(camd)
    fb = None if scene.feat_buffer is None else _in(scene.feat_buffer, np.float32)
    lib().orc_project_feat(C.byref(m.m), C.byref(cam), scene.degree if active_deg is None else active_deg, tx, ty,
                           *[_ptr(out[k]) for k in ("proj0", "proj1", "proj2", "proj3", "tile_count", "hit_info")],
                           int(scene.feat_mode), _ptr(fb))
    return out


def max_screen(scene, camd, init):
    """The projection's max_screen side output (project.cu:82-83) over a starting array."""
    out = np.array(init, np.float32, copy=True)
    m = _Model(scene)  # holds the arrays the call reads
    cam = make_cam(camd)
    lib().orc_max_screen(C.byref(m.m), C.byref(cam), _ptr(out))
    return out


def refine_stats(v_splat, vis_flag, tile_count, vis_count, refine_norm):
    """The refine statistics optim_kernel updates from a view's gradients before it clears them
    (optim.cu:113,122-124): vis_count += 1 for a splat the backward flagged that has tiles; refine_norm =
    max(refine_norm, lane 9 of v_splat clamped to [0, 1e32], non-finite as 0). Lane 9 is read only for
    flagged splats (the others contribute 0)."""
    vf = np.asarray(vis_flag) != 0
    visible = vf & (np.asarray(tile_count) != 0)
    vc = np.asarray(vis_count, np.float32) + visible.astype(np.float32)
    g9 = np.where(vf, np.asarray(v_splat, np.float32)[:, 9], np.float32(0))
    with np.errstate(invalid="ignore"):
        rn = np.where(np.isfinite(g9), np.minimum(np.maximum(g9, np.float32(0)), np.float32(1e32)), np.float32(0))
    return vc.astype(np.float32), np.maximum(np.asarray(refine_norm, np.float32), rn.astype(np.float32))


def _ext(feat=False, proj3=None, hollow_z=None, margin=0.05, lam=0.0, out_feat=None, hollow_pen=None, v_feat=None):
    e = OrcExt()
    e.feat = int(feat)
    e.proj3 = _ptr(proj3)
    e.hollow_z = _ptr(hollow_z)
    e.hollow_margin, e.hollow_lam = margin, lam
    e.out_feat, e.hollow_pen, e.v_feat = _ptr(out_feat), _ptr(hollow_pen), _ptr(v_feat)
    return e


def _proj3(pr, feat):
    """The feature lanes 1-2 of a projection; only the feature variants read them, and a projection read
    back without them (proj0..2 only) serves every other call."""
    if "proj3" in pr:
        return _in(pr["proj3"], np.float32)
    if feat:
        raise ValueError("feature lanes need the projection's proj3")
    return None


def bin_(pr, W, H):
    n = pr["tile_count"].shape[0]
    tx, ty, T, _ = tile_geometry(W, H)
    M = int(pr["tile_count"].astype(np.uint64).sum())
    out = dict(order=np.zeros(n, np.uint32), tile_off=np.zeros(n, np.uint32), keys_sorted=np.zeros(M, np.uint32),
               vals_sorted=np.zeros(M, np.uint32), tile_ranges=np.zeros((T, 2), np.uint32))
    got = lib().orc_bin(n, _ptr(pr["tile_count"]), _ptr(pr["hit_info"]), _ptr(pr["proj0"]), _ptr(pr["proj1"]), tx, ty,
                        M, *[_ptr(out[k]) for k in ("order", "tile_off", "keys_sorted", "vals_sorted", "tile_ranges")])
    assert got == M
    out["M"] = M
    return out


def raster_fwd(pr, bn, W, H, bg, feat=False, hollow_z=None, hollow_margin=0.05):
    """Forward compositing; with feat also out_feat [P][3], with hollow_z the per-pixel hollow_pen [P]."""
    tx, ty, T, _ = tile_geometry(W, H)
    P = W * H
    ranges = bn["tile_ranges"].copy()
    out = dict(out_rgba=np.zeros((P, 4), np.float32), out_T=np.zeros(P, np.float32), last_idx=np.zeros(P, np.uint32),
               out_feat=np.zeros((P, 3), np.float32), hollow_pen=np.zeros(P, np.float32))
    bgv = np.asarray(bg, np.float32)
    hz = None if hollow_z is None else _in(hollow_z, np.float32)
    ext = _ext(feat, _proj3(pr, feat), hz, hollow_margin, 0.0, out["out_feat"], out["hollow_pen"])
    lib().orc_raster_fwd_ext(W, H, tx, ty, _ptr(bgv), _ptr(ranges), _ptr(bn["vals_sorted"]), _ptr(pr["proj0"]),
                             _ptr(pr["proj1"]), _ptr(pr["proj2"]),
                             *[_ptr(out[k]) for k in ("out_rgba", "out_T", "last_idx")], C.byref(ext))
    out["tile_ranges"] = ranges
    out["f_contrib"] = int(lib().orc_last_fwd_contrib())
    return out


def photometric(scene, pred, grad_scale=1.0, bg=None, want_grad=True):
    lp = loss_params(scene, grad_scale, bg)
    v_out = np.zeros((scene.W * scene.H, 4), np.float32) if want_grad else None
    pred = np.ascontiguousarray(pred, np.float32)
    loss = lib().orc_photometric(scene.W, scene.H, _ptr(pred), _ptr(np.ascontiguousarray(scene.gt, np.uint32)),
                                 _ptr(scene.weights), C.byref(lp), _ptr(v_out))
    return loss, v_out


def raster_bwd(pr, bn, fw, v_out, W, H, bg, n, inv_gscale=1.0, v_feat=None, hollow_z=None, hollow_margin=0.05,
               hollow_lam=0.0):
    """Backward; v_feat [P][4] turns the feature lanes on, hollow_z the hollow term (lam in v_out's units)."""
    tx, ty, T, _ = tile_geometry(W, H)
    v_splat = np.zeros((n, GRAD_LANES), np.float64)
    vis_flag = np.zeros(n, np.uint32)
    vis_weight = np.zeros(n, np.float64)
    bgv = np.asarray(bg, np.float32)
    u32, f32 = np.uint32, np.float32
    vf = None if v_feat is None else _in(v_feat, f32)
    hz = None if hollow_z is None else _in(hollow_z, f32)
    ext = _ext(vf is not None, _proj3(pr, vf is not None), hz, hollow_margin, hollow_lam, v_feat=vf)
    lib().orc_raster_bwd_ext(W, H, tx, ty, _ptr(bgv), _ptr(_in(fw["tile_ranges"], u32)),
                             _ptr(_in(bn["vals_sorted"], u32)), _ptr(_in(pr["proj0"], f32)), _ptr(_in(pr["proj1"], f32)),
                             _ptr(_in(pr["proj2"], f32)), _ptr(_in(fw["out_rgba"], f32)), _ptr(_in(fw["out_T"], f32)),
                             _ptr(_in(fw["last_idx"], u32)), _ptr(_in(v_out, f32)), inv_gscale, _ptr(v_splat),
                             _ptr(vis_flag), _ptr(vis_weight), C.byref(ext))
    return v_splat, vis_flag, vis_weight


def normal_loss(W, H, feat4, normals, weights, scale, grad_scale=1.0):
    """(loss, v_feat [P][4]) of loss.cu:206-238; feat4 is out_feat [P][4] (or [P][3])."""
    f = np.zeros((W * H, 4), np.float32)
    f[:, :3] = np.asarray(feat4, np.float32).reshape(W * H, -1)[:, :3]
    v = np.zeros((W * H, 4), np.float32)
    w = None if weights is None else _in(weights, np.uint8)
    loss = lib().orc_normal_loss(W, H, _ptr(f), _ptr(_in(normals, np.uint32)), _ptr(w), scale, grad_scale, _ptr(v))
    return loss, v


def hollow_sum(pen):
    p = _in(pen, np.float32).reshape(-1)
    return lib().orc_hollow_sum(p.size, _ptr(p))


def eval_metrics(W, H, pred, gt, mask_weighted=False):
    """(sum of squared errors, sum of SSIM) over pixels and channels of loss.cu:240-286."""
    se, ss = C.c_double(0), C.c_double(0)
    lib().orc_eval(W, H, _ptr(_in(pred, np.float32)), _ptr(_in(gt, np.uint32)), int(mask_weighted), C.byref(se),
                   C.byref(ss))
    return se.value, ss.value


LABEL_BINS = 32


def evidence_view(pr, bn, fw, W, H, gt, weights=None, normals=None, labels=None, masked_has_alpha=False,
                  normal_weight=0.0, n=None):
    """One view's evidence sums [n][3] = (w_in, err, w_all) and, with labels, the class votes [n][32], from
    the forward's outputs fw (tile_ranges, out_rgba, last_idx and, with normals, out_feat [P][3])."""
    tx, ty, _, _ = tile_geometry(W, H)
    u32, f32 = np.uint32, np.float32
    n = pr["proj0"].shape[0] if n is None else n
    acc = np.zeros((n, 3), np.float64)
    lab_acc = np.zeros((n, LABEL_BINS), np.float64) if labels is not None else None
    feat = None
    if normals is not None:
        feat = _in(np.asarray(fw["out_feat"])[:, :3], f32)
    lib().orc_evidence_view(W, H, tx, ty, _ptr(_in(fw["tile_ranges"], u32)), _ptr(_in(bn["vals_sorted"], u32)),
                            _ptr(_in(pr["proj0"], f32)), _ptr(_in(pr["proj1"], f32)), _ptr(_in(fw["out_rgba"], f32)),
                            _ptr(feat), _ptr(_in(fw["last_idx"], u32)), _ptr(_in(gt, u32)),
                            _ptr(None if normals is None else _in(normals, u32)),
                            _ptr(None if weights is None else _in(weights, np.uint8)),
                            _ptr(None if labels is None else _in(labels, np.uint8)), int(bool(masked_has_alpha)),
                            float(normal_weight), _ptr(acc), _ptr(lab_acc))
    return acc, lab_acc


def evidence_fold(ev, view_acc, pos, cam_pos):
    """fold_view_kernel (evidence.cu:114-126) in double: ev [n][8] += (w_in, w_all, err, -, w_in dir, w_in^2)."""
    w_in, err, w_all = view_acc[:, 0], view_acc[:, 1], view_acc[:, 2]
    ev[:, 0] += w_in
    ev[:, 1] += w_all
    ev[:, 2] += err
    ev[:, 7] += w_in * w_in
    d = np.asarray(cam_pos, np.float64)[None, :] - np.asarray(pos, np.float64)[:, :3]
    l = np.maximum(np.linalg.norm(d, axis=1), 1e-12)
    ev[:, 4:7] += (w_in / l)[:, None] * d
    return ev


def evidence_export(ev):
    """download_evidence (evidence.cu:236-249): [n][7] with views = (sum w_in)^2 / sum w_in^2."""
    out = np.zeros((ev.shape[0], 7), np.float64)
    out[:, 0:3] = ev[:, 0:3]
    pos = ev[:, 7] > 0
    out[pos, 3] = ev[pos, 0] ** 2 / ev[pos, 7]
    out[:, 4:7] = ev[:, 4:7]
    return out


def label_winners(lab_acc):
    """download_labels (evidence.cu:251-264): [n][2] = (first class with the largest vote, its share)."""
    total = lab_acc.sum(1)
    win = np.argmax(lab_acc, 1)
    out = np.zeros((lab_acc.shape[0], 2), np.float64)
    ok = total > 0
    out[ok, 0] = win[ok]
    out[ok, 1] = lab_acc[ok, win[ok]] / total[ok]
    return out


def probe(pr, bn, W, H, tau, delta, ref_z=None, margin=0.0, tile_ranges=None):
    """probe_kernel (probe.cu:7-45): [P][4] = (A, z_first, deep, behind)."""
    tx, ty, _, _ = tile_geometry(W, H)
    out = np.zeros((W * H, 4), np.float32)
    ranges = bn["tile_ranges"] if tile_ranges is None else tile_ranges
    lib().orc_probe(W, H, tx, ty, _ptr(_in(ranges, np.uint32)), _ptr(_in(bn["vals_sorted"], np.uint32)),
                    _ptr(_in(pr["proj0"], np.float32)), _ptr(_in(pr["proj1"], np.float32)), float(tau), float(delta),
                    _ptr(None if ref_z is None else _in(ref_z, np.float32)), float(margin), _ptr(out))
    return out


def vjp(scene, camd, v_splat, vis_flag, tile_count, active_deg=None):
    m = _Model(scene)
    cam = make_cam(camd)
    per = 11 + 3 * scene.K
    g = np.zeros((scene.n, per), np.float32)
    vs = np.ascontiguousarray(v_splat, np.float32)
    lib().orc_vjp(C.byref(m.m), C.byref(cam), scene.degree if active_deg is None else active_deg, _ptr(vs),
                  _ptr(np.ascontiguousarray(vis_flag, np.uint32)), _ptr(np.ascontiguousarray(tile_count, np.uint32)),
                  _ptr(g))
    return g


def pipeline(scene, camd=None, bg=None, grad_scale=1.0):
    """Full fp32 tiled oracle step: project -> bin -> forward -> loss -> backward -> VJP."""
    from b2ctrain_amd.scenes import camera_gpu
    camd = camera_gpu(scene.cam) if camd is None else camd
    bg = scene.bg if bg is None else bg
    W, H = camd["W"], camd["H"]
    pr = project(scene, camd)
    bn = bin_(pr, W, H)
    feat = scene.feat_mode != 0
    fw = raster_fwd(pr, bn, W, H, bg, feat=feat, hollow_z=scene.hollow_z, hollow_margin=scene.hollow_margin)
    loss, v_out = photometric(scene, fw["out_rgba"], grad_scale=grad_scale, bg=bg)
    v_feat = None
    if feat:
        nloss, v_feat = (0.0, np.zeros((W * H, 4), np.float32))
        if scene.normals is not None and scene.normal_scale > 0:
            nloss, v_feat = normal_loss(W, H, fw["out_feat"], scene.normals, scene.weights, scene.normal_scale,
                                        grad_scale)
        loss += nloss
    if scene.hollow_z is not None:
        loss += scene.hollow_lam * hollow_sum(fw["hollow_pen"])
    v_splat, vis_flag, vis_weight = raster_bwd(pr, bn, fw, v_out, W, H, bg, scene.n, inv_gscale=1.0 / grad_scale,
                                               v_feat=v_feat, hollow_z=scene.hollow_z,
                                               hollow_margin=scene.hollow_margin,
                                               hollow_lam=scene.hollow_lam * grad_scale)
    grads = vjp(scene, camd, v_splat, vis_flag, pr["tile_count"])
    return dict(proj=pr, bin=bn, fwd=fw, loss=loss, v_out=v_out, v_feat=v_feat, v_splat=v_splat, vis_flag=vis_flag,
                vis_weight=vis_weight, grads=grads)


# ---- fp64 brute force -------------------------------------------------------------------------------------

def ref_loss(scene, params=None, camd=None, bg=None, want_img=False, floor=None, float_exp=False):
    """orc_ref_loss on double parameters. ``params`` = dict(pos, log_scale, quat, opacity, sh) in
    SplatCloud layout (float64); defaults to the scene's own values."""
    from b2ctrain_amd.scenes import camera_gpu
    if params is None:
        params = scene_params64(scene)
    camd = camera_gpu(scene.cam) if camd is None else camd
    cam = make_cam(camd)
    bg = np.asarray(scene.bg if bg is None else bg, np.float64)
    img = np.zeros((scene.W * scene.H, 4), np.float64) if want_img else None
    arrs = [np.ascontiguousarray(params[k], np.float64) for k in ("pos", "log_scale", "quat", "opacity", "sh")]
    if floor is None and scene.lscale[:, 3].any():  # the scene's own Mip-Splatting floor
        floor = scene.lscale[:, 3]
    fl = None if floor is None else np.ascontiguousarray(floor, np.float64)
    rx = OrcRefExt()
    gtn = None if scene.normals is None else _in(scene.normals, np.uint32)
    hz = None if scene.hollow_z is None else _in(scene.hollow_z, np.float32)
    rx.normals = int(scene.feat_mode == 1 and gtn is not None)
    rx.gtn, rx.normal_scale = _ptr(gtn), scene.normal_scale
    rx.hollow_z, rx.hollow_lam, rx.hollow_margin = _ptr(hz), scene.hollow_lam, scene.hollow_margin
    loss = lib().orc_ref_loss_ext(scene.n, scene.degree, *[_ptr(a) for a in arrs], _ptr(fl), C.byref(cam), scene.W,
                                  scene.H, _ptr(bg), _ptr(np.ascontiguousarray(scene.gt, np.uint32)),
                                  _ptr(scene.weights), int(scene.composite), int(scene.mask), int(scene.alpha_lane),
                                  scene.l1_w, scene.ssim_w, scene.match_alpha_weight, scene.scale, int(float_exp),
                                  _ptr(img), C.byref(rx))
    return (loss, img) if want_img else loss


def scene_params64(scene):
    return dict(pos=scene.pos_op[:, :3].astype(np.float64).copy(), log_scale=scene.lscale[:, :3].astype(np.float64).copy(),
                quat=scene.quat.astype(np.float64).copy(), opacity=scene.pos_op[:, 3].astype(np.float64).copy(),
                sh=scene.sh.astype(np.float64).reshape(scene.n, -1).copy())


def reference_loss(scene, bg=None):
    """The reference's own tests/reference.cpp:34-143 (compiled from /root/reference), float params."""
    r = ref_lib()
    bgv = np.asarray(scene.bg if bg is None else bg, np.float64)
    cam = scene.cam
    arrs = [np.ascontiguousarray(a, np.float32) for a in (scene.pos_op[:, :3], scene.lscale[:, :3], scene.quat,
                                                          scene.pos_op[:, 3], scene.sh.reshape(scene.n, -1))]
    gtn = _in(scene.normals, np.uint32) if (scene.feat_mode == 1 and scene.normals is not None) else None
    hz = None if scene.hollow_z is None else _in(scene.hollow_z, np.float32)
    return r.ref_reference_loss_ext(scene.n, scene.degree, *[_ptr(a) for a in arrs], scene.W, scene.H,
                                    _ptr(np.ascontiguousarray(cam.R, np.float32)),
                                    _ptr(np.ascontiguousarray(cam.t, np.float32)), cam.fx, cam.fy, cam.cx, cam.cy,
                                    _ptr(bgv), _ptr(np.ascontiguousarray(scene.gt, np.uint32)), _ptr(scene.weights),
                                    int(scene.composite), int(scene.mask), int(scene.alpha_lane), scene.l1_w,
                                    scene.ssim_w, scene.match_alpha_weight, scene.scale, _ptr(gtn), scene.normal_scale,
                                    _ptr(hz), scene.hollow_lam, scene.hollow_margin)


# ---- internal pieces (for the pinning tests) -----------------------------------------------------------

def sh_basis(deg, v, double=False):
    K = (deg + 1) ** 2
    if double:
        out = np.zeros(25, np.float64)
        lib().orc_sh_basis_d(deg, float(v[0]), float(v[1]), float(v[2]), _ptr(out))
    else:
        out = np.zeros(25, np.float32)
        lib().orc_sh_basis_f(deg, float(v[0]), float(v[1]), float(v[2]), _ptr(out))
    return out[:K]


def quat_to_mat(q):
    qa = np.ascontiguousarray(q, np.float32)
    R = np.zeros(9, np.float32)
    lib().orc_quat_to_mat(_ptr(qa), _ptr(R))
    return R.reshape(3, 3)


def tile_hit(rect, mean, conic, power) -> bool:
    return bool(lib().orc_tile_hit(*[float(x) for x in rect], float(mean[0]), float(mean[1]), *[float(c) for c in conic],
                                   float(power)))


# ---- fused optimizer (orc_adam.c: optim.cu:104-148, 298-377) ----

# OptimParams defaults (src/gpu/optim.h:10-20)
ADAM_DEFAULTS = dict(t=1, sparse=0, beta1=0.9, beta2=0.999, eps=1e-15, lr_mean=0.0, lr_rot=2e-3, lr_scale=5e-3,
                     lr_opac=0.012, lr_dc=2e-3, lr_sh_rest=2e-4, noise_weight=0.0, noise_clamp=0.0, seed=42, step=0)
ADAM_STATE_KEYS = ("pos_op", "quat", "lscale", "sh", "m_pos_op", "v_pos_op", "m_quat", "v_quat", "m_lscale",
                   "v_lscale", "m_sh", "v_sh", "last_step")


def adam_step(**kw) -> OrcAdamStep:
    """One step's constants: the defaults, the given fields, then the derived bias corrections and logs."""
    s = OrcAdamStep()
    vals = dict(ADAM_DEFAULTS)
    vals.update(kw)
    for k, v in vals.items():
        setattr(s, k, v)
    lib().orc_adam_constants(C.byref(s))
    return s


def adam_update(state, degree, sh_half, camd, v_splat, vis_flag, tile_count, grads, step: OrcAdamStep,
                active_deg=None):
    """The update of every splat (a new state dict; the input is not modified). state holds the keys of
    ADAM_STATE_KEYS: float4 fields [n][4], sh / m_sh [n][K][3], v_sh [n], last_step [n]."""
    out = {k: np.array(state[k], np.uint32 if k == "last_step" else np.float32, copy=True, order="C")
           for k in ADAM_STATE_KEYS}
    n = out["pos_op"].shape[0]
    m = OrcAdamModel(n, degree, int(sh_half), *[_ptr(out[k]) for k in ADAM_STATE_KEYS])
    cam = make_cam(camd)
    keep = [_in(v_splat, np.float32), _in(vis_flag, np.uint32), _in(tile_count, np.uint32), _in(grads, np.float32)]
    lib().orc_adam_update(C.byref(m), C.byref(cam), degree if active_deg is None else active_deg,
                          *[_ptr(a) for a in keep], C.byref(step))
    return out


def project_ok(po, q, ls, camd) -> bool:
    arrs = [_in(a, np.float32) for a in (po, q, ls)]
    return bool(lib().orc_project_ok(*[_ptr(a) for a in arrs], C.byref(make_cam(camd))))


def hash_unit(a, b, c) -> float:
    return lib().orc_hash_unit(a, b, c)


def mix32(x):
    return lib().orc_mix32(x)


def hash_gauss(a, b, c) -> float:
    return lib().orc_hash_gauss(a, b, c)


def cos_turns(u) -> float:
    return lib().orc_cos_turns(u)


def f16_bits(v) -> int:
    return lib().orc_f16_bits(v)


def f16_value(h) -> float:
    return lib().orc_f16_value(h)


def f16_stochastic(v, u01) -> int:
    return lib().orc_f16_stochastic(v, u01)
