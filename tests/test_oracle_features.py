"""Pins for the oracle's feature lanes and the losses beside the photometric one (oracle/b2c_oracle.c:
orc_project_feat, orc_normal_loss, orc_hollow_sum, orc_eval) that do not restate them. The fp64 brute force
with normals and the hollow term, and the tiled pipeline's gradients through them, are pinned by the
reference's own numbers (tests/golden/ref_fd*n*.npz, ref_fd*h*.npz, test_oracle_golden.py).

| oracle piece        | reference (file:line)   | pinned by                                                    |
|---------------------|-------------------------|--------------------------------------------------------------|
| orc_project_feat    | project.cu:63-77        | scipy Rotation: the smallest-scale local axis, unit, camera-facing, in camera space |
| orc_normal_loss     | loss.cu:206-238         | closed forms (p = n, p parallel to n) and central differences of its own value |
| orc_eval            | loss.cu:240-286         | scipy.ndimage separable SSIM with zero padding, float64     |
| orc_hollow_sum      | loss.cu:197-204         | numpy sum                                                    |
"""
import numpy as np
from scipy import ndimage
from scipy.spatial.transform import Rotation

from b2ctrain_amd import scenes as S
from oracle import oracle as O


def test_pseudo_normals_are_the_camera_facing_shortest_axis():
    sc = S.fd_scene(41, n=40)
    sc.feat_mode = 1
    camd = S.camera_gpu(sc.cam)
    pr = O.project(sc, camd)
    ok = pr["tile_count"] > 0
    assert ok.sum() > 20
    f = np.concatenate([pr["proj2"][:, 3:4], pr["proj3"]], 1).astype(np.float64)
    R = np.asarray(camd["R"], np.float64).reshape(3, 3)
    q = sc.quat.astype(np.float64)
    rot = Rotation.from_quat(q[:, [1, 2, 3, 0]]).as_matrix()  # scipy takes (x, y, z, w)
    for i in np.flatnonzero(ok):
        ax = int(np.argmin(sc.lscale[i, :3]))
        u = rot[i][:, ax]
        to_splat = sc.pos_op[i, :3].astype(np.float64) - np.asarray(camd["pos"], np.float64)
        want = R @ (u if np.dot(-to_splat, u) >= 0 else -u)
        np.testing.assert_allclose(f[i], want, atol=2e-6)
        assert abs(np.linalg.norm(f[i]) - 1.0) < 2e-6
        assert np.dot(f[i], R @ to_splat) <= 1e-6  # faces the camera


def _normal_map(rng, P, opaque=0.7):
    rgb = (rng.random((P, 3)) * 255).astype(np.uint32)
    a = np.where(rng.random(P) < opaque, 255, 0).astype(np.uint32)
    return (rgb[:, 0] | (rgb[:, 1] << 8) | (rgb[:, 2] << 16) | (a << 24)).astype(np.uint32)


def _decode(nm):
    r, g, b = (nm & 0xFF), ((nm >> 8) & 0xFF), ((nm >> 16) & 0xFF)
    return np.stack([r * (2.0 / 255.0) - 1.0, 1.0 - g * (2.0 / 255.0), 1.0 - b * (2.0 / 255.0)], 1)


def test_normal_loss_closed_forms():
    rng = np.random.default_rng(3)
    W, H = 16, 8
    nm = _normal_map(rng, W * H, opaque=1.0)
    n = _decode(nm)
    w = (64 + rng.random(W * H) * 191).astype(np.uint8)
    # p = n: L1 and 1 - cos both vanish
    loss, v = O.normal_loss(W, H, n.astype(np.float32), nm, w, 0.3)
    assert abs(loss) < 1e-5
    # p = 2 n: cos = 1, so the loss is the weighted L1 distance |n|_1
    loss, _ = O.normal_loss(W, H, (2 * n).astype(np.float32), nm, w, 0.3)
    want = (0.3 * w / 255.0 * np.abs(n).sum(1)).sum()
    assert abs(loss - want) <= 1e-5 * want
    # transparent normal-map pixels contribute nothing
    nm2 = nm & 0x00FFFFFF
    loss, v = O.normal_loss(W, H, rng.normal(0, 1, (W * H, 3)).astype(np.float32), nm2, w, 0.3)
    assert loss == 0.0 and not v.any()


def test_normal_loss_gradient_matches_central_differences():
    rng = np.random.default_rng(4)
    W, H = 12, 10
    P = W * H
    nm = _normal_map(rng, P)
    feat = rng.normal(0, 0.6, (P, 3)).astype(np.float64)
    n = _decode(nm)
    feat[np.abs(feat - n) < 0.05] += 0.1  # keep clear of the L1 kinks
    w = (64 + rng.random(P) * 191).astype(np.uint8)
    _, v = O.normal_loss(W, H, feat.astype(np.float32), nm, w, 0.25, grad_scale=3.0)
    eps = 1e-2
    for pix in rng.choice(P, 40, replace=False):
        for c in range(3):
            fp, fm = feat.copy(), feat.copy()
            fp[pix, c] += eps
            fm[pix, c] -= eps
            lp, _ = O.normal_loss(W, H, fp.astype(np.float32), nm, w, 0.25)
            lm, _ = O.normal_loss(W, H, fm.astype(np.float32), nm, w, 0.25)
            fd = 3.0 * (lp - lm) / (2 * eps)
            assert abs(v[pix, c] - fd) <= 2e-3 * max(abs(fd), 1.0), (pix, c, v[pix, c], fd)


def _ssim_sums(pred, gt, W, H, mask_weighted):
    w = np.exp(-((np.arange(11) - 5.0) ** 2) / 4.5)
    w /= w.sum()

    def blur(a):
        return ndimage.correlate1d(ndimage.correlate1d(a, w, axis=1, mode="constant"), w, axis=0, mode="constant")

    se = ss = 0.0
    g_all = np.stack([(gt >> (8 * c)) & 0xFF for c in range(4)], 1).astype(np.float64) / 255.0
    for c in range(3):
        x = (np.rint(np.clip(pred[:, c].astype(np.float64), 0, 1) * 255) / 255).reshape(H, W)
        y = g_all[:, c].reshape(H, W)
        mu1, mu2 = blur(x), blur(y)
        s1 = np.maximum(0, blur(x * x) - mu1 ** 2)
        s2 = np.maximum(0, blur(y * y) - mu2 ** 2)
        s12 = blur(x * y) - mu1 * mu2
        ssim = np.clip(((2 * mu1 * mu2 + 1e-4) * (2 * s12 + 9e-4)) / ((mu1 ** 2 + mu2 ** 2 + 1e-4) * (s1 + s2 + 9e-4)),
                       -1, 1)
        m = g_all[:, 3].reshape(H, W) if mask_weighted else 1.0
        se += (((x - y) * m) ** 2).sum()
        ss += (ssim * m).sum()
    return se, ss


def test_eval_metrics_match_scipy_ssim():
    rng = np.random.default_rng(5)
    for W, H in ((37, 29), (64, 16)):
        pred = rng.uniform(-0.1, 1.1, (W * H, 4)).astype(np.float32)
        gt = (rng.random((W * H, 4)) * 255).astype(np.uint32)
        gt = gt[:, 0] | (gt[:, 1] << 8) | (gt[:, 2] << 16) | (gt[:, 3] << 24)
        for mw in (False, True):
            se, ss = O.eval_metrics(W, H, pred, gt, mw)
            want_se, want_ss = _ssim_sums(pred, gt, W, H, mw)
            assert abs(se - want_se) <= 1e-5 * want_se
            assert abs(ss - want_ss) <= 1e-5 * abs(want_ss) + 1e-3


def test_hollow_sum_is_the_plain_sum():
    pen = np.random.default_rng(6).random(1000).astype(np.float32)
    assert abs(O.hollow_sum(pen) - pen.astype(np.float64).sum()) < 1e-9
