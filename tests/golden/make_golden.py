"""Writes the golden fixtures under tests/golden/ from the reference's own double-precision CPU loss
(tests/reference.cpp:34-143 of Erant/b2ctrain), compiled unmodified from /root/reference into
oracle/_ref/libb2c_ref.so by oracle/Makefile (`make -C oracle ref`).

Run in the build container only (the reference is not present on GPU boxes):

    make -C oracle ref && python tests/golden/make_golden.py

Each fixture is one .npz holding a scene's inputs (SplatCloud layout, float32), the camera, the target,
the loss options, the reference's loss value, and central finite differences of the reference's loss
taken exactly as tests/tests.cpp:413-428 takes them: every 2nd splat, the 11 geometric parameters and
every 5th SH lane, float32 parameter +- float32 eps with eps = 1e-4 and 4e-4 (tests.cpp:104,426-428).
Inputs are stored, not regenerated, so the fixtures do not depend on numpy's generator.
"""
from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from b2ctrain_amd import scenes as S  # noqa: E402
from oracle import oracle as O  # noqa: E402

EPS = np.float32(1e-4)


def scene_list():
    out = []
    # the FD harness's three view modes (tests.cpp:398-401 without normals/hollow), SH degree 2
    out.append(S.fd_scene(1234))
    out.append(S.fd_scene(1235, masked=True))
    s = S.fd_scene(1236)
    s.composite = s.alpha_lane = s.mask = False
    s.name = "fd1236plain"
    out.append(s)
    out.append(S.fd_scene(1237, degree=3))
    s = S.config1()
    s.bg = (0.3, 0.2, 0.1)
    out.append(s)
    # the harness's normal and hollow configurations (tests.cpp:386-391): normals on a transparent view;
    # hollow on the transparent, masked and normals views
    out.append(S.fd_feature_scene(1236, normals=True))
    out.append(S.fd_feature_scene(1234, hollow=True))
    out.append(S.fd_feature_scene(1235, masked=True, hollow=True))
    out.append(S.fd_feature_scene(1236, normals=True, hollow=True))
    return out


def ref_loss(sc, P):
    """reference_loss over float32 parameters P (the SplatCloud holds floats)."""
    sc2 = S.Scene(**{k: getattr(sc, k) for k in sc.__dataclass_fields__})
    sc2.pos_op = np.concatenate([P["pos"], P["opacity"][:, None]], 1).astype(np.float32)
    sc2.lscale = np.concatenate([P["log_scale"], np.zeros((sc.n, 1), np.float32)], 1)
    sc2.quat = P["quat"]
    sc2.sh = P["sh"].reshape(sc.n, sc.K, 3)
    return O.reference_loss(sc2)  # with the scene's normal map and hollow depths


def fd_samples(sc, every=2, sh_every=5):
    """Central differences as tests.cpp:413-428 takes them; with the hollow loss the mean lanes are left out
    (tests.cpp:418-421: the loss's depth dependence is not part of the analytic gradient)."""
    per = 11 + 3 * sc.K
    P0 = dict(pos=sc.pos_op[:, :3].copy(), opacity=sc.pos_op[:, 3].copy(), quat=sc.quat.copy(),
              log_scale=sc.lscale[:, :3].copy(), sh=sc.sh.reshape(sc.n, -1).copy())
    idx, fd1, fd4 = [], [], []
    for i in range(0, sc.n, every):
        for q in range(per):
            if q >= 11 and (q - 11) % sh_every:
                continue
            if sc.hollow_z is not None and q < 3:
                continue
            if q < 3:
                key, j = "pos", (i, q)
            elif q == 3:
                key, j = "opacity", (i,)
            elif q < 8:
                key, j = "quat", (i, q - 4)
            elif q < 11:
                key, j = "log_scale", (i, q - 8)
            else:
                key, j = "sh", (i, q - 11)

            def fd_at(e):
                P = {k: v.copy() for k, v in P0.items()}
                orig = np.float32(P0[key][j])
                P[key][j] = np.float32(orig + e)
                lp = ref_loss(sc, P)
                P[key][j] = np.float32(orig - e)
                lm = ref_loss(sc, P)
                return (lp - lm) / (2.0 * float(e))

            idx.append((i, q))
            fd1.append(fd_at(EPS))
            fd4.append(fd_at(np.float32(4) * EPS))
    return np.array(idx, np.int32), np.array(fd1), np.array(fd4)


def main():
    if not O.ref_available():
        sys.exit("oracle/_ref/libb2c_ref.so is missing: run `make -C oracle ref` (needs /root/reference)")
    for sc in scene_list():
        loss = O.reference_loss(sc)
        with_fd = sc.n <= 64
        rec = dict(
            name=np.array(sc.name), degree=np.int32(sc.degree), W=np.int32(sc.W), H=np.int32(sc.H),
            pos=sc.pos_op[:, :3].copy(), opacity=sc.pos_op[:, 3].copy(), quat=sc.quat.copy(),
            log_scale=sc.lscale[:, :3].copy(), sh=sc.sh.reshape(sc.n, -1).copy(),
            R=np.asarray(sc.cam.R, np.float32), t=np.asarray(sc.cam.t, np.float32),
            intr=np.array([sc.cam.fx, sc.cam.fy, sc.cam.cx, sc.cam.cy], np.float32),
            bg=np.asarray(sc.bg, np.float64), gt=np.asarray(sc.gt, np.uint32),
            weights=np.asarray(sc.weights if sc.weights is not None else np.zeros(0), np.uint8),
            flags=np.array([sc.composite, sc.mask, sc.alpha_lane], np.int32),
            lossw=np.array([sc.l1_w, sc.ssim_w, sc.match_alpha_weight, sc.scale], np.float64),
            ref_loss=np.float64(loss),
        )
        if sc.feat_mode == 1:
            rec["normals"] = np.asarray(sc.normals, np.uint32)
            rec["normal_scale"] = np.float64(sc.normal_scale)
        if sc.hollow_z is not None:
            rec["hollow_z"] = np.asarray(sc.hollow_z, np.float32)
            rec["hollow"] = np.array([sc.hollow_lam, sc.hollow_margin], np.float64)
        if with_fd:
            rec["fd_index"], rec["fd_eps"], rec["fd_4eps"] = fd_samples(sc)
        path = os.path.join(HERE, f"ref_{sc.name}.npz")
        np.savez_compressed(path, **rec)
        print(f"{path}: loss {loss:.9g}" + (f", {len(rec['fd_index'])} FD samples" if with_fd else ""))


if __name__ == "__main__":
    main()
