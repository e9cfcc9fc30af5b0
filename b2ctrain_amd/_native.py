"""ctypes binding of libb2c_hip.so (include/b2c.h, include/b2c_kernels.h).

Python is plumbing here: tests and the benchmark drive the C ABI through these wrappers. There is no
fallback: if the HIP library is missing the import of ``lib()`` raises.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
# B2C_HIP_LIB selects another build of the library (for example to compare two builds in one process tree)
LIB_PATH = os.environ.get("B2C_HIP_LIB") or os.path.join(HERE, "lib", "libb2c_hip.so")

GRAD_LANES = 13
RT_W = 8
GRAD_ACCUMULATE, GRAD_SPARSE = 1, 2  # b2c_optimizer_grad / b2c_train_step flags (include/b2c.h)


class Camera(C.Structure):
    _fields_ = [("width", C.c_int), ("height", C.c_int), ("fx", C.c_float), ("fy", C.c_float), ("cx", C.c_float),
                ("cy", C.c_float), ("R", C.c_float * 9), ("t", C.c_float * 3)]


class CameraGPU(C.Structure):
    _fields_ = [("R", C.c_float * 9), ("t", C.c_float * 3), ("pos", C.c_float * 3), ("fx", C.c_float),
                ("fy", C.c_float), ("cx", C.c_float), ("cy", C.c_float), ("W", C.c_int), ("H", C.c_int),
                ("lim_pos_x", C.c_float), ("lim_pos_y", C.c_float), ("lim_neg_x", C.c_float), ("lim_neg_y", C.c_float)]


class RenderOpts(C.Structure):
    _fields_ = [("cam", Camera), ("W", C.c_int), ("H", C.c_int), ("bg", C.c_float * 3), ("sh_degree", C.c_int),
                ("bwd_info", C.c_int), ("feat_mode", C.c_int), ("feat_buffer", C.c_void_p), ("hollow_z", C.c_void_p),
                ("hollow_margin", C.c_float), ("hollow_lam", C.c_float)]


class LossOpts(C.Structure):
    _fields_ = [("l1_w", C.c_float), ("ssim_w", C.c_float), ("bg", C.c_float * 3), ("composite", C.c_int),
                ("mask", C.c_int), ("alpha_lane", C.c_int), ("match_alpha_weight", C.c_float), ("scale", C.c_float),
                ("grad_scale", C.c_float), ("normal_scale", C.c_float)]


class AdamOpts(C.Structure):
    _fields_ = [("t", C.c_int), ("sparse", C.c_int), ("beta1", C.c_float), ("beta2", C.c_float), ("eps", C.c_float),
                ("lr_mean", C.c_float), ("lr_rot", C.c_float), ("lr_scale", C.c_float), ("lr_opac", C.c_float),
                ("lr_dc", C.c_float), ("lr_sh_rest", C.c_float), ("noise_weight", C.c_float),
                ("noise_clamp", C.c_float), ("seed", C.c_uint32), ("step", C.c_uint32)]

    def as_dict(self):
        return {k: getattr(self, k) for k, _ in self._fields_}


def adam_opts(**kw) -> AdamOpts:
    """The reference's OptimParams defaults (b2c_adam_defaults), then any field given by keyword."""
    a = AdamOpts()
    lib().b2c_adam_defaults(C.byref(a))
    for k, v in kw.items():
        if not hasattr(a, k):
            raise KeyError(k)
        setattr(a, k, v)
    return a


class CtxInfo(C.Structure):
    _fields_ = [("W", C.c_int), ("H", C.c_int), ("tiles_x", C.c_int), ("tiles_y", C.c_int), ("n_tiles", C.c_int),
                ("tile_bits", C.c_int), ("num_isect", C.c_uint32), ("isect_cap", C.c_uint64)]


class StepTimes(C.Structure):
    _fields_ = [("project_ms", C.c_float), ("bin_ms", C.c_float), ("forward_ms", C.c_float), ("loss_ms", C.c_float),
                ("backward_ms", C.c_float), ("vjp_ms", C.c_float), ("total_ms", C.c_float),
                ("raster_bwd_ms", C.c_float), ("reduce_ms", C.c_float)]

    def as_dict(self):
        return {k: float(getattr(self, k)) for k, _ in self._fields_}


PLY_FIELDS = ["pos", "log_scale", "quat", "opacity", "sh", "evidence", "labels", "fill", "gate", "gate_s", "open"]
PLY_BLOCKS = {"evidence": 7, "labels": 2, "fill": 1, "gate": 2, "gate_s": 1, "open": 4}


class PlyInfo(C.Structure):
    _fields_ = [("n", C.c_int64), ("sh_degree", C.c_int), ("binary", C.c_int)] + \
               [(f, C.c_int) for f in ("has_scales", "has_evidence", "has_labels", "has_fill", "has_gate",
                                       "has_gate_s", "has_open")]


class DatasetOpts(C.Structure):
    _fields_ = [("source", C.c_char_p), ("max_frames", C.c_int), ("max_resolution", C.c_uint),
                ("eval_split_every", C.c_int), ("subsample_frames", C.c_int), ("alpha_mode", C.c_int)]


class ViewInfo(C.Structure):
    _fields_ = [("w", C.c_int), ("h", C.c_int), ("cam", Camera), ("has_alpha", C.c_int), ("masked", C.c_int),
                ("has_normals", C.c_int), ("has_weights", C.c_int), ("has_labels", C.c_int),
                ("alpha_coverage", C.c_float), ("normal_mask_count", C.c_double), ("name", C.c_char * 256)]


class PlyArrays(C.Structure):
    _fields_ = [(f, C.c_void_p) for f in PLY_FIELDS]


# Every symbol include/b2c.h and include/b2c_kernels.h declare.
EXPORTS = [
    "b2c_last_error", "b2c_get_device_count", "b2c_camera_gpu_from", "b2c_model_create", "b2c_model_destroy",
    "b2c_model_upload", "b2c_model_read", "b2c_model_device_ptr", "b2c_model_sh_view", "b2c_ctx_create",
    "b2c_ctx_destroy", "b2c_ctx_setup", "b2c_ctx_info_get", "b2c_ctx_read", "b2c_ctx_device_ptr", "b2c_ctx_write",
    "b2c_ctx_zero", "b2c_ctx_synchronize", "b2c_ctx_stream", "b2c_view_create",
    "b2c_view_destroy", "b2c_render_forward", "b2c_project_splats", "b2c_bin_and_sort", "b2c_rasterize_forward",
    "b2c_photometric_loss", "b2c_accumulate_loss", "b2c_rasterize_backward", "b2c_optimizer_grad", "b2c_train_step",
    "b2c_model_write", "b2c_model_zero_optimizer", "b2c_model_adam_t", "b2c_adam_defaults", "b2c_optimizer_step",
    "b2c_train_step_adam", "b2c_adam_step_constants", "b2c_view_set_normals", "b2c_device_upload",
    "b2c_device_free", "b2c_normal_loss", "b2c_hollow_loss", "b2c_eval_metrics",
    # launcher layer
    "b2c_hip_project", "b2c_radix_sort_temp_bytes", "b2c_hip_radix_sort_pairs", "b2c_hip_radix_sort_kv2",
    "b2c_hip_depth_keys",
    "b2c_scan_temp_bytes", "b2c_hip_scan_counts", "b2c_hip_scan_counts_host", "b2c_hip_emit", "b2c_hip_tile_ranges", "b2c_hip_raster_fwd",
    "b2c_hip_raster_bwd", "b2c_hip_photometric", "b2c_loss_partials", "b2c_hip_accumulate_loss", "b2c_hip_vjp",
    "b2c_hip_fill_u32", "b2c_hip_model_scatter", "b2c_hip_model_gather", "b2c_hip_planar_regrow",
    "b2c_hip_model_set_floor", "b2c_hip_photometric_noalloc", "b2c_aux_partials", "b2c_hip_normal_loss",
    "b2c_hip_hollow_loss", "b2c_hip_eval_metrics", "b2c_hip_step_loss_sums",
    "b2c_view_set_labels", "b2c_view_set_flags", "b2c_compute_evidence", "b2c_download_evidence",
    "b2c_download_labels", "b2c_probe_depth", "b2c_device_download", "b2c_hip_evidence_view",
    "b2c_hip_evidence_sum", "b2c_hip_probe_depth",
    "b2c_ply_info_get", "b2c_ply_read", "b2c_ply_write", "b2c_ply_is_vertex_only", "b2c_ply_comments",
    "b2c_model_load_ply", "b2c_model_save_ply", "b2c_hip_ply_decode", "b2c_hip_ply_encode",
    "b2c_png_decode", "b2c_image_decode", "b2c_image_resample", "b2c_dataset_load", "b2c_dataset_destroy", "b2c_dataset_count", "b2c_dataset_view_info",
    "b2c_dataset_view_read", "b2c_dataset_view_upload", "b2c_dataset_points", "b2c_dataset_summary",
]

_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"HIP library not built: {LIB_PATH} (run __graft_entry__.build())")
        L = C.CDLL(LIB_PATH)
        p, i, f = C.c_void_p, C.c_int, C.c_float
        L.b2c_last_error.restype = C.c_char_p
        L.b2c_get_device_count.argtypes = [C.POINTER(i)]
        L.b2c_camera_gpu_from.argtypes = [C.POINTER(Camera), i, i, C.POINTER(CameraGPU)]
        L.b2c_model_create.restype = p
        L.b2c_model_destroy.argtypes = [p]
        L.b2c_model_upload.argtypes = [p, i, i, i, p, p, p, p, p, p]
        L.b2c_model_read.argtypes = [p, C.c_char_p, p, C.c_size_t]
        L.b2c_ctx_create.restype = p
        L.b2c_ctx_destroy.argtypes = [p]
        L.b2c_ctx_setup.argtypes = [p, i, i, i]
        L.b2c_ctx_info_get.argtypes = [p, C.POINTER(CtxInfo)]
        L.b2c_ctx_read.argtypes = [p, C.c_char_p, p, C.c_size_t]
        L.b2c_ctx_write.argtypes = [p, C.c_char_p, p, C.c_size_t]
        L.b2c_ctx_zero.argtypes = [p, C.c_char_p]
        L.b2c_ctx_synchronize.argtypes = [p]
        L.b2c_ctx_stream.argtypes = [p]
        L.b2c_ctx_stream.restype = p
        L.b2c_ctx_device_ptr.argtypes = [p, C.c_char_p, C.POINTER(p), C.POINTER(C.c_size_t)]
        L.b2c_model_device_ptr.argtypes = [p, C.c_char_p, C.POINTER(p), C.POINTER(C.c_size_t)]
        L.b2c_view_create.restype = p
        L.b2c_view_create.argtypes = [i, i, p, p]
        L.b2c_view_destroy.argtypes = [p]
        L.b2c_render_forward.argtypes = [p, p, C.POINTER(RenderOpts)]
        L.b2c_project_splats.argtypes = [p, p, C.POINTER(RenderOpts)]
        L.b2c_bin_and_sort.argtypes = [p, p]
        L.b2c_rasterize_forward.argtypes = [p, C.POINTER(RenderOpts)]
        L.b2c_photometric_loss.argtypes = [p, p, C.POINTER(LossOpts)]
        L.b2c_accumulate_loss.argtypes = [p]
        L.b2c_rasterize_backward.argtypes = [p, p, C.POINTER(RenderOpts), i, f]
        L.b2c_optimizer_grad.argtypes = [p, p, C.POINTER(RenderOpts), i, i]
        L.b2c_train_step.argtypes = [p, p, p, C.POINTER(RenderOpts), C.POINTER(LossOpts), i, i, C.POINTER(StepTimes)]
        L.b2c_model_write.argtypes = [p, C.c_char_p, p, C.c_size_t]
        L.b2c_model_zero_optimizer.argtypes = [p]
        L.b2c_model_adam_t.argtypes = [p, C.POINTER(i)]
        L.b2c_adam_defaults.argtypes = [C.POINTER(AdamOpts)]
        L.b2c_adam_defaults.restype = None
        L.b2c_optimizer_step.argtypes = [p, p, C.POINTER(RenderOpts), C.POINTER(AdamOpts)]
        L.b2c_train_step_adam.argtypes = [p, p, p, C.POINTER(RenderOpts), C.POINTER(LossOpts), i, C.POINTER(AdamOpts),
                                          C.POINTER(StepTimes)]
        L.b2c_view_set_normals.argtypes = [p, p]
        L.b2c_device_upload.restype = p
        L.b2c_device_upload.argtypes = [p, C.c_size_t]
        L.b2c_device_free.argtypes = [p]
        L.b2c_device_free.restype = None
        L.b2c_normal_loss.argtypes = [p, p, C.POINTER(LossOpts)]
        L.b2c_hollow_loss.argtypes = [p, f]
        L.b2c_eval_metrics.argtypes = [p, p, i]
        L.b2c_view_set_labels.argtypes = [p, p]
        L.b2c_view_set_flags.argtypes = [p, i, i, f, f]
        L.b2c_compute_evidence.argtypes = [p, p, C.POINTER(p), C.POINTER(Camera), i, f, i]
        L.b2c_download_evidence.argtypes = [p, p]
        L.b2c_download_labels.argtypes = [p, p]
        L.b2c_probe_depth.argtypes = [p, f, f, p, f, p]
        L.b2c_device_download.argtypes = [p, p, C.c_size_t]
        L.b2c_ply_info_get.argtypes = [C.c_char_p, C.POINTER(PlyInfo)]
        L.b2c_ply_read.argtypes = [C.c_char_p, C.POINTER(PlyArrays)]
        L.b2c_ply_write.argtypes = [C.c_char_p, C.POINTER(PlyInfo), C.POINTER(PlyArrays), C.c_char_p]
        L.b2c_ply_is_vertex_only.argtypes = [C.c_char_p]
        L.b2c_ply_comments.argtypes = [C.c_char_p, C.c_char_p, C.c_size_t, C.POINTER(C.c_size_t)]
        L.b2c_model_load_ply.argtypes = [p, C.c_char_p, i, C.POINTER(i)]
        L.b2c_model_save_ply.argtypes = [p, C.c_char_p, C.c_char_p, C.POINTER(PlyInfo), C.POINTER(PlyArrays)]
        L.b2c_png_decode.argtypes = [C.c_char_p, C.POINTER(i), C.POINTER(i), C.POINTER(i), p, C.c_size_t]
        L.b2c_image_decode.argtypes = [C.c_char_p, C.POINTER(i), C.POINTER(i), C.POINTER(i), p, C.c_size_t]
        L.b2c_image_resample.argtypes = [p, i, i, p, i, i, i]
        L.b2c_dataset_load.restype = p
        L.b2c_dataset_load.argtypes = [C.POINTER(DatasetOpts)]
        L.b2c_dataset_destroy.argtypes = [p]
        L.b2c_dataset_destroy.restype = None
        L.b2c_dataset_count.argtypes = [p, i]
        L.b2c_dataset_view_info.argtypes = [p, i, i, C.POINTER(ViewInfo)]
        L.b2c_dataset_view_read.argtypes = [p, i, i, p, p, p, p]
        L.b2c_dataset_view_upload.restype = p
        L.b2c_dataset_view_upload.argtypes = [p, i, i]
        L.b2c_dataset_points.argtypes = [p, p, p, C.POINTER(C.c_int64)]
        L.b2c_dataset_summary.argtypes = [p, C.c_char_p, C.c_size_t, C.POINTER(i)]
        L.b2c_radix_sort_temp_bytes.restype = C.c_size_t
        L.b2c_radix_sort_temp_bytes.argtypes = [C.c_uint32]
        L.b2c_scan_temp_bytes.restype = C.c_size_t
        L.b2c_scan_temp_bytes.argtypes = [C.c_uint32]
        _lib = L
    return _lib


def check(rc: int, what: str = "") -> None:
    if rc != 0:
        raise RuntimeError(f"b2c {what} failed ({rc}): {lib().b2c_last_error().decode()}")


def _ptr(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def camera_struct(cam) -> Camera:
    c = Camera()
    c.width, c.height = int(cam.width), int(cam.height)
    c.fx, c.fy, c.cx, c.cy = float(cam.fx), float(cam.fy), float(cam.cx), float(cam.cy)
    for k in range(9):
        c.R[k] = float(cam.R[k])
    for k in range(3):
        c.t[k] = float(cam.t[k])
    return c


def camera_gpu_from(cam, W=None, H=None) -> dict:
    g = CameraGPU()
    check(lib().b2c_camera_gpu_from(C.byref(camera_struct(cam)), cam.width if W is None else W,
                                    cam.height if H is None else H, C.byref(g)), "camera_gpu_from")
    return dict(R=np.array(g.R[:], np.float32), t=np.array(g.t[:], np.float32), pos=np.array(g.pos[:], np.float32),
                fx=np.float32(g.fx), fy=np.float32(g.fy), cx=np.float32(g.cx), cy=np.float32(g.cy), W=g.W, H=g.H,
                lim_pos_x=np.float32(g.lim_pos_x), lim_pos_y=np.float32(g.lim_pos_y),
                lim_neg_x=np.float32(g.lim_neg_x), lim_neg_y=np.float32(g.lim_neg_y))


def _ply_arrays(arrs):
    pa = PlyArrays()
    for f in PLY_FIELDS:
        a = arrs.get(f)
        setattr(pa, f, None if a is None else a.ctypes.data)
    return pa


def ply_info(path) -> dict:
    """read_ply's view of a file without its rows: n, sh_degree, binary and the has_* flags."""
    info = PlyInfo()
    check(lib().b2c_ply_info_get(os.fsencode(path), C.byref(info)), "ply_info")
    return {f: (int(getattr(info, f)) if f in ("n", "sh_degree") else bool(getattr(info, f))) for f, _ in info._fields_}


def ply_read(path) -> dict:
    """read_ply on the host: a cloud dict (pos, log_scale, quat, opacity, sh [n][K][3], the optional blocks)."""
    info = ply_info(path)
    n, K = info["n"], (info["sh_degree"] + 1) ** 2
    c = dict(n=n, sh_degree=info["sh_degree"], has_scales=info["has_scales"],
             pos=np.zeros((n, 3), np.float32), log_scale=np.zeros((n, 3), np.float32),
             quat=np.zeros((n, 4), np.float32), opacity=np.zeros(n, np.float32), sh=np.zeros((n, K, 3), np.float32))
    for b, w in PLY_BLOCKS.items():
        if info["has_" + b]:
            c[b] = np.zeros((n, w) if w > 1 else n, np.float32)
    check(lib().b2c_ply_read(os.fsencode(path), C.byref(_ply_arrays(c))), "ply_read")
    return c


def _ply_desc(c):
    d = PlyInfo()
    d.n, d.sh_degree, d.binary = int(c["n"]), int(c["sh_degree"]), 1
    for b in PLY_BLOCKS:
        setattr(d, "has_" + b, int(b in c))
    arrs = {f: np.ascontiguousarray(c[f], np.float32) for f in PLY_FIELDS if f in c}
    return d, arrs


def ply_write(path, c, comments=()):
    """write_ply of a cloud dict (see ply_read)."""
    d, arrs = _ply_desc(c)
    cm = "\n".join(comments).encode() if comments else None
    check(lib().b2c_ply_write(os.fsencode(path), C.byref(d), C.byref(_ply_arrays(arrs)), cm), "ply_write")


def ply_is_vertex_only(path) -> bool:
    r = lib().b2c_ply_is_vertex_only(os.fsencode(path))
    if r < 0:
        raise RuntimeError(lib().b2c_last_error().decode())
    return bool(r)


def ply_comments(path) -> list:
    need = C.c_size_t()
    check(lib().b2c_ply_comments(os.fsencode(path), None, 0, C.byref(need)), "ply_comments")
    buf = C.create_string_buffer(need.value)
    check(lib().b2c_ply_comments(os.fsencode(path), buf, need.value, None), "ply_comments")
    text = buf.value.decode("latin-1")
    return text.split("\n") if text else []


def png_decode(path):
    """The loader's PNG decoder: (rgba [h][w][4] uint8, channels in the file)."""
    w, h, ch = C.c_int(), C.c_int(), C.c_int()
    check(lib().b2c_png_decode(os.fsencode(path), C.byref(w), C.byref(h), C.byref(ch), None, 0), "png_decode")
    out = np.zeros((h.value, w.value, 4), np.uint8)
    check(lib().b2c_png_decode(os.fsencode(path), C.byref(w), C.byref(h), C.byref(ch), _ptr(out), out.nbytes),
          "png_decode")
    return out, ch.value


def image_decode(path):
    """The loader's image decoder (PNG or JPEG): (rgba [h][w][4] uint8, channels in the file)."""
    w, h, ch = C.c_int(), C.c_int(), C.c_int()
    check(lib().b2c_image_decode(os.fsencode(path), C.byref(w), C.byref(h), C.byref(ch), None, 0), "image_decode")
    out = np.zeros((h.value, w.value, 4), np.uint8)
    check(lib().b2c_image_decode(os.fsencode(path), C.byref(w), C.byref(h), C.byref(ch), _ptr(out), out.nbytes),
          "image_decode")
    return out, ch.value


RESAMPLE_FILTERS = {"triangle": 0, "mitchell": 1, "point": 2}


def image_resample(rgba, nw, nh, filt):
    """The loader's resize of an RGBA8 image [h][w][4] to [nh][nw][4] (filter: triangle, mitchell, point)."""
    src = np.ascontiguousarray(rgba, np.uint8)
    out = np.zeros((nh, nw, 4), np.uint8)
    check(lib().b2c_image_resample(_ptr(src), src.shape[1], src.shape[0], _ptr(out), nw, nh,
                                   RESAMPLE_FILTERS[filt]), "image_resample")
    return out


class Dataset:
    """load_dataset through the C ABI (b2c_dataset_*): views by split (0 train, 1 eval)."""

    def __init__(self, source, max_frames=None, max_resolution=1920, eval_split_every=None, subsample_frames=None,
                 alpha_mode=None):
        self.L = lib()
        o = DatasetOpts()
        o.source = os.fsencode(source)
        o.max_frames = -1 if max_frames is None else int(max_frames)
        o.max_resolution = int(max_resolution)
        o.eval_split_every = -1 if eval_split_every is None else int(eval_split_every)
        o.subsample_frames = -1 if subsample_frames is None else int(subsample_frames)
        o.alpha_mode = {None: -1, "masked": 0, "transparent": 1}[alpha_mode]
        self.ptr = self.L.b2c_dataset_load(C.byref(o))
        if not self.ptr:
            raise RuntimeError(self.L.b2c_last_error().decode())

    def count(self, split=0):
        return self.L.b2c_dataset_count(self.ptr, split)

    def info(self, split, i):
        v = ViewInfo()
        check(self.L.b2c_dataset_view_info(self.ptr, split, i, C.byref(v)), "dataset_view_info")
        return v

    def planes(self, split, i):
        v = self.info(split, i)
        P = v.w * v.h
        out = dict(rgba=np.zeros(P, np.uint32))
        if v.has_normals:
            out["normals"] = np.zeros(P, np.uint32)
        if v.has_weights:
            out["weights"] = np.zeros(P, np.uint8)
        if v.has_labels:
            out["labels"] = np.zeros(P, np.uint8)
        check(self.L.b2c_dataset_view_read(self.ptr, split, i, *[_ptr(out.get(k)) for k in ("rgba", "normals",
                                                                                          "weights", "labels")]),
              "dataset_view_read")
        return out

    def upload(self, split, i):
        """A device view (b2c_view handle) of a dataset view."""
        h = self.L.b2c_dataset_view_upload(self.ptr, split, i)
        if not h:
            raise RuntimeError(self.L.b2c_last_error().decode())
        return h

    def points(self):
        n = C.c_int64()
        check(self.L.b2c_dataset_points(self.ptr, None, None, C.byref(n)), "dataset_points")
        xyz, rgb = np.zeros((n.value, 3), np.float32), np.zeros((n.value, 3), np.uint8)
        check(self.L.b2c_dataset_points(self.ptr, _ptr(xyz), _ptr(rgb), C.byref(n)), "dataset_points")
        return xyz, rgb

    def summary(self):
        buf = C.create_string_buffer(8192)
        counts = (C.c_int * 5)()
        check(self.L.b2c_dataset_summary(self.ptr, buf, 8192, counts), "dataset_summary")
        root, name, init = buf.value.decode().split("\n")
        return dict(root=root, name=name, init_ply=init, counts=list(counts))

    def close(self):
        if self.ptr:
            self.L.b2c_dataset_destroy(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def device_count() -> int:
    n = C.c_int(0)
    rc = lib().b2c_get_device_count(C.byref(n))
    return n.value if rc == 0 else 0


_FIELD_SPEC = {
    # name: (dtype, per-element shape, size key)  size key: n splats, P pixels, M isects, T tiles (T1: T + 1)
    "proj0": (np.float32, (4,), "n"), "proj1": (np.float32, (4,), "n"), "proj2": (np.float32, (4,), "n"),
    "proj3": (np.float32, (2,), "n"), "raster_rec": (np.float32, (16,), "n"), "tile_count": (np.uint32, (), "n"), "tile_off": (np.uint32, (), "n"),
    "hit_info": (np.uint32, (2,), "n"), "hit_wide": (np.uint32, (2,), "n"), "order": (np.uint32, (), "n"), "depth_keys_sorted": (np.uint32, (), "n"),
    "keys": (np.uint32, (), "M"), "vals": (np.uint32, (), "M"), "keys_sorted": (np.uint32, (), "M"),
    "vals_sorted": (np.uint32, (), "M"), "tile_ranges": (np.uint32, (2,), "T"), "out_rgba": (np.float32, (4,), "P"),
    "out_feat": (np.float32, (4,), "P"), "last_idx": (np.uint32, (), "P"), "v_out": (np.float32, (4,), "P"),
    "v_splat": (np.float32, (GRAD_LANES,), "n"), "vis_flag": (np.uint32, (), "n"), "loss_accum": (np.float32, (16,), "1"),
    "v_feat": (np.float32, (4,), "P"), "hollow_pen": (np.float32, (), "P"),
    "slot_sorted": (np.uint32, (), "M"), "tile_end": (np.uint32, (), "T1"),
    "isect_rows": (np.float32, (12,), "M"),
    "cvals": (np.uint32, (), "M"), "cslots": (np.uint32, (), "M"), "clast": (np.uint32, (), "P"),
    "cend": (np.uint32, (), "T"),
}


class DeviceArray:
    """A device copy of a host array (b2c_device_upload), freed with the object."""

    def __init__(self, arr):
        self.L = lib()
        a = np.ascontiguousarray(arr)
        self.ptr = self.L.b2c_device_upload(_ptr(a), a.nbytes)
        if not self.ptr:
            raise RuntimeError(self.L.b2c_last_error().decode())

    def download(self, dtype, shape):
        """The device bytes as a host array (b2c_device_download: a synchronous copy)."""
        host = np.empty(shape, dtype)
        check(self.L.b2c_device_download(_ptr(host), self.ptr, host.nbytes), "device_download")
        return host

    def free(self):
        if self.ptr:
            self.L.b2c_device_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class View:
    """A target view (b2c_view): packed RGBA8 pixels, optional weight bytes, normal map and label plane, and
    the has_alpha / masked flags."""

    def __init__(self, W, H, gt, weights=None, normals=None, labels=None, has_alpha=False, masked=False):
        self.L = lib()
        self.W, self.H = W, H
        g = np.ascontiguousarray(gt, np.uint32)
        w = None if weights is None else np.ascontiguousarray(weights, np.uint8)
        self.ptr = self.L.b2c_view_create(W, H, _ptr(g), _ptr(w))
        if not self.ptr:
            raise RuntimeError(self.L.b2c_last_error().decode())
        if normals is not None:
            check(self.L.b2c_view_set_normals(self.ptr, _ptr(np.ascontiguousarray(normals, np.uint32))), "view_set_normals")
        if labels is not None:
            check(self.L.b2c_view_set_labels(self.ptr, _ptr(np.ascontiguousarray(labels, np.uint8))), "view_set_labels")
        check(self.L.b2c_view_set_flags(self.ptr, int(has_alpha), int(masked), 1.0, 0.0), "view_set_flags")

    def close(self):
        if self.ptr:
            self.L.b2c_view_destroy(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


_FLOAT4_FIELDS = ("pos_op", "quat", "lscale", "m_pos_op", "v_pos_op", "m_quat", "v_quat", "m_lscale", "v_lscale")


class Renderer:
    """One model + one render context + one view, driven through the C ABI."""

    def __init__(self, scene, W=None, H=None):
        self.L = lib()
        self.scene = scene
        self.W = scene.W if W is None else W
        self.H = scene.H if H is None else H
        self.model = self.L.b2c_model_create()
        self.ctx = self.L.b2c_ctx_create()
        if not self.ctx:
            raise RuntimeError(self.L.b2c_last_error().decode())
        self.view = None
        self.feat_mode = 0        # render options every stage call uses unless given: FeatureMode
        self.feat_buffer = None   # DeviceArray [n][3] for feat_mode 2
        self.hollow = None        # DeviceArray [P] of reference depths, or None
        self.hollow_margin, self.hollow_lam = 0.05, 0.0
        self.normal_scale = 0.0
        self.upload(scene)
        check(self.L.b2c_ctx_setup(self.ctx, self.W, self.H, scene.n), "ctx_setup")
        self.set_target(scene.gt, scene.weights, scene.normals)
        if scene.feat_mode or scene.hollow_z is not None:
            self.set_features(scene.feat_mode, scene.feat_buffer, scene.hollow_z, scene.hollow_margin,
                              scene.hollow_lam, scene.normal_scale)

    def upload(self, scene, floor=None):
        n = scene.n
        arrs = [np.ascontiguousarray(a, np.float32) for a in (scene.pos_op[:, :3], scene.lscale[:, :3], scene.quat,
                                                              scene.pos_op[:, 3], scene.sh.reshape(n, 3 * scene.K))]
        if floor is None and scene.lscale[:, 3].any():  # the scene's own Mip-Splatting floor
            floor = scene.lscale[:, 3]
        fl = None if floor is None else np.ascontiguousarray(floor, np.float32)
        self.sh_fp16 = bool(scene.sh_fp16)
        check(self.L.b2c_model_upload(self.model, n, scene.degree, int(scene.sh_fp16), *[_ptr(a) for a in arrs], _ptr(fl)),
              "model_upload")
        self.n = n
        self.degree = scene.degree

    def set_target(self, gt, weights=None, normals=None):
        if self.view:
            self.L.b2c_view_destroy(self.view)
        g = np.ascontiguousarray(gt, np.uint32)
        w = None if weights is None else np.ascontiguousarray(weights, np.uint8)
        self.view = self.L.b2c_view_create(self.W, self.H, _ptr(g), _ptr(w))
        if not self.view:
            raise RuntimeError(self.L.b2c_last_error().decode())
        if normals is not None:
            nm = np.ascontiguousarray(normals, np.uint32)
            check(self.L.b2c_view_set_normals(self.view, _ptr(nm)), "view_set_normals")

    def set_features(self, mode=0, buffer=None, hollow_z=None, hollow_margin=0.05, hollow_lam=0.0, normal_scale=0.0):
        """Feature lanes (0 none, 1 normals, 2 buffer [n][3]), the hollow loss's reference depths [P] and
        weights, and the normal loss weight, for every following call."""
        self.feat_mode = int(mode)
        self.feat_buffer = None if buffer is None else DeviceArray(np.asarray(buffer, np.float32))
        self.hollow = None if hollow_z is None else DeviceArray(np.asarray(hollow_z, np.float32))
        self.hollow_margin, self.hollow_lam = float(hollow_margin), float(hollow_lam)
        self.normal_scale = float(normal_scale)

    def close(self):
        self.feat_buffer = self.hollow = None
        if self.view:
            self.L.b2c_view_destroy(self.view)
        if self.ctx:
            self.L.b2c_ctx_destroy(self.ctx)
        if self.model:
            self.L.b2c_model_destroy(self.model)
        self.view = self.ctx = self.model = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # -- options
    def render_opts(self, cam=None, bg=None, sh_degree=None, bwd_info=True) -> RenderOpts:
        o = RenderOpts()
        o.cam = camera_struct(self.scene.cam if cam is None else cam)
        o.W, o.H = self.W, self.H
        b = self.scene.bg if bg is None else bg
        for k in range(3):
            o.bg[k] = float(b[k])
        o.sh_degree = self.degree if sh_degree is None else sh_degree
        o.bwd_info = int(bwd_info)
        o.feat_mode = self.feat_mode
        o.feat_buffer = self.feat_buffer.ptr if self.feat_buffer is not None else None
        o.hollow_z = self.hollow.ptr if self.hollow is not None else None
        o.hollow_margin, o.hollow_lam = self.hollow_margin, self.hollow_lam
        return o

    def loss_opts(self, grad_scale=1.0, bg=None) -> LossOpts:
        s = self.scene
        lo = LossOpts()
        lo.l1_w, lo.ssim_w = s.l1_w, s.ssim_w
        b = s.bg if bg is None else bg
        for k in range(3):
            lo.bg[k] = float(b[k])
        lo.composite, lo.mask, lo.alpha_lane = int(s.composite), int(s.mask), int(s.alpha_lane)
        lo.match_alpha_weight, lo.scale, lo.grad_scale = s.match_alpha_weight, s.scale, grad_scale
        lo.normal_scale = self.normal_scale
        return lo

    # -- stages
    def project(self, **kw):
        check(self.L.b2c_project_splats(self.ctx, self.model, C.byref(self.render_opts(**kw))), "project_splats")

    def bin(self):
        check(self.L.b2c_bin_and_sort(self.ctx, self.model), "bin_and_sort")

    def raster_fwd(self, **kw):
        check(self.L.b2c_rasterize_forward(self.ctx, C.byref(self.render_opts(**kw))), "rasterize_forward")

    def forward(self, **kw):
        check(self.L.b2c_render_forward(self.ctx, self.model, C.byref(self.render_opts(**kw))), "render_forward")

    def loss(self, grad_scale=1.0, bg=None, zero=True):
        if zero:
            self.zero("loss_accum")
        check(self.L.b2c_photometric_loss(self.ctx, self.view, C.byref(self.loss_opts(grad_scale, bg))), "photometric_loss")
        return float(self.read("loss_accum")[0])

    def normal_loss(self, grad_scale=1.0):
        check(self.L.b2c_normal_loss(self.ctx, self.view, C.byref(self.loss_opts(grad_scale))), "normal_loss")

    def hollow_loss(self, lam=None):
        check(self.L.b2c_hollow_loss(self.ctx, self.hollow_lam if lam is None else lam), "hollow_loss")

    def eval_metrics(self, mask_weighted=False):
        check(self.L.b2c_eval_metrics(self.ctx, self.view, int(mask_weighted)), "eval_metrics")

    def backward(self, mode=1, grad_scale=1.0, **kw):
        check(self.L.b2c_rasterize_backward(self.ctx, self.model, C.byref(self.render_opts(**kw)), mode, grad_scale),
              "rasterize_backward")

    def vjp(self, accumulate=False, active_deg=None, sparse=False, **kw):
        flags = (GRAD_ACCUMULATE if accumulate else 0) | (GRAD_SPARSE if sparse else 0)
        check(self.L.b2c_optimizer_grad(self.ctx, self.model, C.byref(self.render_opts(**kw)),
                                        self.degree if active_deg is None else active_deg, flags),
              "optimizer_grad")

    def adam(self, opts: AdamOpts | None = None, **kw):
        """optimizer_step without grad_out: the projection VJP fused with the Adam update of the model."""
        a = adam_opts() if opts is None else opts
        check(self.L.b2c_optimizer_step(self.ctx, self.model, C.byref(self.render_opts(**kw)), C.byref(a)),
              "optimizer_step")

    def step_adam(self, opts: AdamOpts | None = None, mode=1, grad_scale=None, timed=False, cam=None, bg=None):
        """One complete training iteration ending in the fused update (b2c_train_step_adam)."""
        gs = 3.0 * self.W * self.H if grad_scale is None else grad_scale
        a = adam_opts() if opts is None else opts
        t = StepTimes() if timed else None
        check(self.L.b2c_train_step_adam(self.ctx, self.model, self.view, C.byref(self.render_opts(cam=cam, bg=bg)),
                                         C.byref(self.loss_opts(gs, bg)), mode, C.byref(a),
                                         C.byref(t) if timed else None), "train_step_adam")
        return t.as_dict() if timed else None

    def adam_t(self) -> int:
        t = C.c_int(0)
        check(self.L.b2c_model_adam_t(self.model, C.byref(t)), "model_adam_t")
        return t.value

    def zero_optimizer(self):
        check(self.L.b2c_model_zero_optimizer(self.model), "model_zero_optimizer")

    def step(self, mode=1, grad_scale=None, accumulate=False, timed=False, cam=None, bg=None):
        gs = 3.0 * self.W * self.H if grad_scale is None else grad_scale
        t = StepTimes() if timed else None
        check(self.L.b2c_train_step(self.ctx, self.model, self.view, C.byref(self.render_opts(cam=cam, bg=bg)),
                                    C.byref(self.loss_opts(gs, bg)), mode, GRAD_ACCUMULATE if accumulate else 0,
                                    C.byref(t) if timed else None), "train_step")
        return t.as_dict() if timed else None

    # -- ply
    def load_ply(self, path, sh_fp16=False):
        """Replace the model by a ply file, decoded on the device (b2c_model_load_ply); sizes the context for
        it. Returns the file's has_scales."""
        hs = C.c_int(0)
        check(self.L.b2c_model_load_ply(self.model, os.fsencode(path), int(sh_fp16), C.byref(hs)), "model_load_ply")
        info = ply_info(path)
        self.n, self.degree, self.sh_fp16 = info["n"], info["sh_degree"], bool(sh_fp16)
        check(self.L.b2c_ctx_setup(self.ctx, self.W, self.H, max(self.n, 1)), "ctx_setup")
        return bool(hs.value)

    def save_ply(self, path, comments=(), extras=None):
        """write_ply of the model, encoded on the device (b2c_model_save_ply); extras: a dict of optional
        blocks (evidence, labels, fill, gate, gate_s, open) with [n] rows."""
        cm = "\n".join(comments).encode() if comments else None
        if extras:
            d, arrs = _ply_desc(dict(extras, n=self.n, sh_degree=self.degree))
            check(self.L.b2c_model_save_ply(self.model, os.fsencode(path), cm, C.byref(d), C.byref(_ply_arrays(arrs))),
                  "model_save_ply")
        else:
            check(self.L.b2c_model_save_ply(self.model, os.fsencode(path), cm, None, None), "model_save_ply")

    # -- tile-list replays
    def compute_evidence(self, views, cams, normal_weight=0.0, export_labels=False, download=True):
        """compute_evidence over View objects and their cameras; returns download_evidence [n][7] (None
        without download)."""
        if len(views) != len(cams):
            raise ValueError("one camera per view")
        vp = (C.c_void_p * len(views))(*[v.ptr for v in views])
        cs = (Camera * len(cams))(*[camera_struct(c) for c in cams])
        check(self.L.b2c_compute_evidence(self.ctx, self.model, vp, cs, len(views), float(normal_weight),
                                          int(export_labels)), "compute_evidence")
        return self.download_evidence() if download else None

    def download_evidence(self):
        out = np.zeros((self.n, 7), np.float32)
        check(self.L.b2c_download_evidence(self.model, _ptr(out)), "download_evidence")
        return out

    def download_labels(self):
        out = np.zeros((self.n, 2), np.float32)
        check(self.L.b2c_download_labels(self.model, _ptr(out)), "download_labels")
        return out

    def probe_depth(self, tau, delta, ref_z=None, margin=0.0):
        """probe_depth on the context's current lists (after forward, or project + bin): [P][4] float32."""
        P = self.W * self.H
        out = DeviceArray(np.zeros((P, 4), np.float32))
        rz = None if ref_z is None else DeviceArray(np.asarray(ref_z, np.float32).reshape(P))
        try:
            check(self.L.b2c_probe_depth(self.ctx, float(tau), float(delta), None if rz is None else rz.ptr,
                                         float(margin), out.ptr), "probe_depth")
            host = np.empty((P, 4), np.float32)
            check(self.L.b2c_device_download(_ptr(host), out.ptr, host.nbytes), "device_download")
            return host
        finally:
            out.free()
            if rz is not None:
                rz.free()

    # -- buffers
    def info(self) -> CtxInfo:
        i = CtxInfo()
        self.L.b2c_ctx_info_get(self.ctx, C.byref(i))
        return i

    def _count(self, key):
        inf = self.info()
        return {"n": self.n, "P": self.W * self.H, "M": inf.num_isect, "T": inf.n_tiles, "T1": inf.n_tiles + 1,
                "1": 1}[key]

    def read(self, field):
        if field == "grads":
            per = 11 + 3 * (self.degree + 1) ** 2
            out = np.empty((self.n, per), np.float32)
        else:
            dt, shape, key = _FIELD_SPEC[field]
            out = np.empty((self._count(key),) + shape, dt)
        check(self.L.b2c_ctx_read(self.ctx, field.encode(), _ptr(out), out.nbytes), f"read {field}")
        return out[0] if field == "loss_accum" else out

    def write(self, field, arr):
        a = np.ascontiguousarray(arr)
        check(self.L.b2c_ctx_write(self.ctx, field.encode(), _ptr(a), a.nbytes), f"write {field}")

    def zero(self, field):
        check(self.L.b2c_ctx_zero(self.ctx, field.encode()), f"zero {field}")

    def read_model(self, field):
        dt = np.uint32 if field == "last_step" else np.float32
        out = np.empty((self.n, 4) if field in _FLOAT4_FIELDS else (self.n,), dt)
        check(self.L.b2c_model_read(self.model, field.encode(), _ptr(out), out.nbytes), f"model_read {field}")
        return out

    def write_model(self, field, arr):
        a = np.ascontiguousarray(arr)
        check(self.L.b2c_model_write(self.model, field.encode(), _ptr(a), a.nbytes), f"model_write {field}")

    def _planar(self, name):
        """A planar [lanes][cap] SH array (parameters or first moments) as [n][lanes] float32."""
        half = name.endswith("_hi")
        _, size = self.device_ptr(name, model=True)
        lanes = 3 if name.endswith("_dc") else 3 * ((self.degree + 1) ** 2 - 1)
        cap = size // (lanes * (2 if half else 4))
        raw = np.empty((lanes, cap), np.uint16 if half else np.float32)
        check(self.L.b2c_model_read(self.model, name.encode(), _ptr(raw), raw.nbytes), f"model_read {name}")
        vals = raw.view(np.float16).astype(np.float32) if half else raw
        return np.ascontiguousarray(vals[:, : self.n].T), cap

    def _write_planar(self, name, vals):
        half = name.endswith("_hi")
        _, size = self.device_ptr(name, model=True)
        lanes = vals.shape[1]
        cap = size // (lanes * (2 if half else 4))
        raw = np.zeros((lanes, cap), np.float32)
        raw[:, : self.n] = vals.T
        raw = raw.astype(np.float16).view(np.uint16) if half else raw
        self.write_model(name, np.ascontiguousarray(raw))

    def _band_names(self, sh_fp16):
        return ("sh_hi", "m_sh_hi") if sh_fp16 else ("sh_hi32", "m_sh_hi32")

    def model_state(self):
        """Parameters and Adam state in host layouts: float4 fields [n][4], SH and their first moments
        coefficient-major [n][K][3] (binary16 bands widened), v_sh [n], last_step [n]."""
        st = {f: self.read_model(f) for f in _FLOAT4_FIELDS}
        st["v_sh"] = self.read_model("v_sh")
        st["last_step"] = self.read_model("last_step")
        K = (self.degree + 1) ** 2
        hi, mhi = self._band_names(self.sh_fp16)
        for key, dc, bands in (("sh", "sh_dc", hi), ("m_sh", "m_sh_dc", mhi)):
            flat = np.zeros((self.n, 3 * K), np.float32)
            flat[:, :3] = self._planar(dc)[0]
            if K > 1:
                flat[:, 3:] = self._planar(bands)[0]
            st[key] = flat.reshape(self.n, K, 3)
        return st

    def set_model_state(self, st):
        """Write back what model_state returns (any subset of its keys)."""
        K = (self.degree + 1) ** 2
        hi, mhi = self._band_names(self.sh_fp16)
        for f, a in st.items():
            if f in ("sh", "m_sh"):
                flat = np.asarray(a, np.float32).reshape(self.n, 3 * K)
                self._write_planar("sh_dc" if f == "sh" else "m_sh_dc", flat[:, :3])
                if K > 1:
                    self._write_planar(hi if f == "sh" else mhi, flat[:, 3:])
            else:
                self.write_model(f, np.asarray(a, np.uint32 if f == "last_step" else np.float32))

    def device_ptr(self, field, model=False):
        """Device address and byte size of a context (or model) buffer."""
        ptr, size = C.c_void_p(), C.c_size_t()
        fn = lib().b2c_model_device_ptr if model else lib().b2c_ctx_device_ptr
        check(fn(self.model if model else self.ctx, field.encode(), C.byref(ptr), C.byref(size)), f"device_ptr {field}")
        return ptr.value, size.value

    def sync(self):
        check(self.L.b2c_ctx_synchronize(self.ctx), "synchronize")
