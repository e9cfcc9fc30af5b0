"""Loads the golden fixtures written by tests/golden/make_golden.py (the reference's own fp64 CPU loss and
its finite differences) back into Scene objects."""
from __future__ import annotations

import glob
import os

import numpy as np

from b2ctrain_amd import scenes as S

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def fixture_paths():
    return sorted(glob.glob(os.path.join(GOLDEN, "ref_*.npz")))


def load(path):
    z = np.load(path, allow_pickle=False)
    n = z["pos"].shape[0]
    deg = int(z["degree"])
    K = (deg + 1) ** 2
    W, H = int(z["W"]), int(z["H"])
    fx, fy, cx, cy = (float(v) for v in z["intr"])
    cam = S.Camera(W, H, fx, fy, cx, cy, z["R"].copy(), z["t"].copy())
    pos_op = np.concatenate([z["pos"], z["opacity"][:, None]], 1).astype(np.float32)
    lscale = np.concatenate([z["log_scale"], np.zeros((n, 1), np.float32)], 1).astype(np.float32)
    w = z["weights"]
    comp, mask, alpha = (bool(v) for v in z["flags"])
    l1, ssim, match, scale = (float(v) for v in z["lossw"])
    sc = S.Scene(str(z["name"]), deg, pos_op, z["quat"].copy(), lscale, z["sh"].reshape(n, K, 3).copy(), cam,
                 z["gt"].copy(), w.copy() if w.size else None, composite=comp, mask=mask, alpha_lane=alpha,
                 match_alpha_weight=match, scale=scale, l1_w=l1, ssim_w=ssim, bg=tuple(float(v) for v in z["bg"]))
    if "normals" in z.files:  # the harness's normal configuration (tests.cpp:386-391)
        sc.feat_mode = 1
        sc.normals = z["normals"].copy()
        sc.normal_scale = float(z["normal_scale"])
    if "hollow_z" in z.files:
        sc.hollow_z = z["hollow_z"].copy()
        sc.hollow_lam, sc.hollow_margin = (float(v) for v in z["hollow"])
    fd = None
    if "fd_index" in z.files:
        fd = dict(index=z["fd_index"], eps=z["fd_eps"], eps4=z["fd_4eps"])
    return sc, float(z["ref_loss"]), fd
