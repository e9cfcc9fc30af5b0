"""Pins for the oracle's tile-list replays (oracle/b2c_oracle.c: orc_evidence_view, orc_probe; oracle/oracle.py:
evidence_fold, evidence_export, label_winners) that do not restate them.

| oracle piece             | reference (file:line)        | pinned by                                                   |
|--------------------------|------------------------------|-------------------------------------------------------------|
| orc_evidence_view        | evidence.cu:47-112           | conservation (the sums over splats equal the pixel weights times the forward's accumulated alpha) and, splat by splat, a pixel-major fp64 walk over the global depth order with no tiles |
| label vote               | evidence.cu:141-183, 251-264 | the reference's half-frame test (tests/tests.cpp:250-279), class bins summing to w_all, ids >= 32 dropping out |
| evidence_fold / _export  | evidence.cu:114-126, 236-249 | the participation-ratio closed forms the reference states (evidence.cu:8-21) and the camera direction of a splat at a known position |
| orc_probe                | probe.cu:7-45                | accumulated alpha equal to the forward's bit for bit; the limits of tau, delta, ref_z and margin; the mean depth against fp64 |
"""
import numpy as np
import pytest

from b2ctrain_amd import scenes as S
from oracle import oracle as O


def _render(sc, camd=None):
    camd = S.camera_gpu(sc.cam) if camd is None else camd
    pr = O.project(sc, camd)
    bn = O.bin_(pr, sc.W, sc.H)
    fw = O.raster_fwd(pr, bn, sc.W, sc.H, (0.0, 0.0, 0.0))
    return pr, bn, fw


def _chan(gt, c):
    return ((gt >> (8 * c)) & 0xFF).astype(np.float64) / 255.0


def _pixel_terms(sc, fw, masked_has_alpha):
    wp = sc.weights.astype(np.float64) / 255.0 if sc.weights is not None else np.ones(sc.W * sc.H)
    ga = _chan(sc.gt, 3)
    o = fw["out_rgba"].astype(np.float64)
    res = sum(np.abs(o[:, c] - _chan(sc.gt, c)) for c in range(3)) / 3.0
    m = ga * wp
    k = (ga if masked_has_alpha else 1.0) * wp
    return m, m * res, k


@pytest.mark.parametrize("masked_has_alpha", [False, True])
def test_evidence_conserves_the_rendered_alpha(masked_has_alpha):
    """Each pixel hands out exactly its accumulated alpha 1 - T across the splats it composited."""
    sc = S.fd_scene(21, n=80)
    pr, bn, fw = _render(sc)
    acc, _ = O.evidence_view(pr, bn, fw, sc.W, sc.H, sc.gt, sc.weights, masked_has_alpha=masked_has_alpha)
    m, mres, k = _pixel_terms(sc, fw, masked_has_alpha)
    A = fw["out_rgba"][:, 3].astype(np.float64)
    for col, w in ((0, m), (1, mres), (2, k)):
        want = float((w * A).sum())
        assert want > 1.0
        assert abs(acc[:, col].sum() - want) <= 2e-6 * want, (col, acc[:, col].sum(), want)


def _brute_vis(sc, pr):
    """Per pixel, every projected splat in global depth order, fp64 alpha, the forward's termination rule:
    vis [n][P]. No tiles, no lists."""
    n, W, H = sc.n, sc.W, sc.H
    ok = pr["tile_count"] > 0
    p0, p1 = pr["proj0"].astype(np.float64), pr["proj1"].astype(np.float64)
    order = np.flatnonzero(ok)[np.argsort(p1[ok, 2], kind="stable")]
    vis = np.zeros((n, W * H))
    for pix in range(W * H):
        x, y = pix % W + 0.5, pix // W + 0.5
        T = 1.0
        for g in order:
            dx, dy = x - p0[g, 0], y - p0[g, 1]
            sigma = 0.5 * (p0[g, 2] * dx * dx + p1[g, 0] * dy * dy) + p0[g, 3] * dx * dy
            if sigma < 0 or sigma > p1[g, 3]:
                continue
            alpha = min(0.999, p1[g, 1] * np.exp(-sigma))
            if T * (1 - alpha) <= 1e-4:
                break
            vis[g, pix] = alpha * T
            T *= 1 - alpha
    return vis


def test_evidence_per_splat_matches_a_pixel_major_walk():
    sc = S.fd_scene(22, n=40)
    pr, bn, fw = _render(sc)
    acc, _ = O.evidence_view(pr, bn, fw, sc.W, sc.H, sc.gt, sc.weights, masked_has_alpha=True)
    m, mres, k = _pixel_terms(sc, fw, True)
    vis = _brute_vis(sc, pr)
    want = np.stack([vis @ m, vis @ mres, vis @ k], 1)
    scale = np.abs(want).max(0)
    assert (scale > 0).all()
    err = np.abs(acc - want).max(0) / scale
    assert (err <= 1e-4).all(), err
    assert (acc[pr["tile_count"] == 0] == 0).all()


def test_evidence_normal_residual_adds_the_weighted_normal_term():
    sc = S.fd_feature_scene(23, n=60, normals=True)
    camd = S.camera_gpu(sc.cam)
    pr = O.project(sc, camd)
    bn = O.bin_(pr, sc.W, sc.H)
    fw = O.raster_fwd(pr, bn, sc.W, sc.H, (0.0, 0.0, 0.0), feat=True)
    base, _ = O.evidence_view(pr, bn, fw, sc.W, sc.H, sc.gt, sc.weights, normals=sc.normals, normal_weight=0.0)
    withn, _ = O.evidence_view(pr, bn, fw, sc.W, sc.H, sc.gt, sc.weights, normals=sc.normals, normal_weight=0.5)
    np.testing.assert_array_equal(base[:, [0, 2]], withn[:, [0, 2]])  # only the error column moves
    # the extra error mass: sum over supervised pixels of m * 0.5 * (L1 + 1 - cos) * A
    nm = sc.normals
    sup = ((nm >> 24) & 0xFF) > 127
    nvec = np.stack([_chan(nm, 0) * 2 - 1, 1 - _chan(nm, 1) * 2, 1 - _chan(nm, 2) * 2], 1)
    f = fw["out_feat"].astype(np.float64)
    cos = (f * nvec).sum(1) / (np.maximum(np.linalg.norm(f, axis=1), 1e-6) * np.maximum(np.linalg.norm(nvec, axis=1), 1e-6))
    nres = np.abs(f - nvec).sum(1) + 1 - cos
    m, _, _ = _pixel_terms(sc, fw, False)
    want = float((m * 0.5 * nres * fw["out_rgba"][:, 3] * sup).sum())
    got = withn[:, 1].sum() - base[:, 1].sum()
    assert want > 0.1 and abs(got - want) <= 1e-5 * want


def _half_labels(W, H, left=3, right=13):
    x = np.arange(W * H) % W
    return np.where(x < W // 2, left, right).astype(np.uint8)


def test_label_vote_half_frame():
    """tests/tests.cpp:250-279: left half class 3, right half 13; every splat away from the seam and the frame
    edge wins its side at a share above 0.9."""
    sc = S.fd_scene(11, n=60)
    pr, bn, fw = _render(sc)
    labels = _half_labels(sc.W, sc.H)
    acc, lab = O.evidence_view(pr, bn, fw, sc.W, sc.H, sc.gt, None, labels=labels, masked_has_alpha=False)
    win = O.label_winners(lab)
    px = 40.0 * sc.pos_op[:, 0] / sc.pos_op[:, 2] + sc.W / 2.0
    checked = 0
    for i in range(sc.n):
        if abs(px[i] - sc.W / 2.0) < 6 or px[i] < 2 or px[i] > sc.W - 2 or acc[i, 2] == 0:
            continue
        checked += 1
        assert int(win[i, 0]) == (3 if px[i] < sc.W / 2.0 else 13) and win[i, 1] > 0.9, (i, px[i], win[i])
    assert checked > 20
    # without weights and with every id below 32, the class bins of a splat add up to its w_all
    np.testing.assert_allclose(lab.sum(1), acc[:, 2], rtol=1e-12, atol=1e-15)


def test_label_ids_beyond_the_bins_drop_out():
    sc = S.fd_scene(12, n=60)
    pr, bn, fw = _render(sc)
    labels = _half_labels(sc.W, sc.H, left=5, right=40)  # 40 >= 32: ignored
    _, lab = O.evidence_view(pr, bn, fw, sc.W, sc.H, sc.gt, sc.weights, labels=labels)
    # the same replay with the right half's weight zeroed gives the left half's share of w_all
    w_left = sc.weights.copy()
    w_left[(np.arange(sc.W * sc.H) % sc.W) >= sc.W // 2] = 0
    acc_left, _ = O.evidence_view(pr, bn, fw, sc.W, sc.H, sc.gt, w_left)
    np.testing.assert_allclose(lab[:, 5], acc_left[:, 2], rtol=1e-12, atol=1e-15)
    assert lab[:, 6:].sum() == 0 and lab[:, :5].sum() == 0 and lab[:, 5].sum() > 0


def test_effective_view_count_closed_forms():
    """evidence.cu:8-21: 1 for a splat seen in one view whatever its mass, N for one seen equally in N views,
    10 in one view + 0.001 in 99 others -> 1.02."""
    n = 3
    ev = np.zeros((n, 8))
    pos = np.zeros((n, 3))
    views = [np.array([[7.0, 0, 0], [2.0, 0, 0], [10.0, 0, 0]])]
    views += [np.array([[0.0, 0, 0], [2.0, 0, 0], [0.001, 0, 0]]) for _ in range(3)]
    views += [np.array([[0.0, 0, 0], [0.0, 0, 0], [0.001, 0, 0]]) for _ in range(96)]
    for v in views:
        O.evidence_fold(ev, v, pos, (0.0, 0.0, 1.0))
    e = O.evidence_export(ev)
    assert e[0, 3] == pytest.approx(1.0, rel=1e-12)
    assert e[1, 3] == pytest.approx(4.0, rel=1e-12)
    assert e[2, 3] == pytest.approx(1.02, abs=0.005)


def test_fold_direction_is_the_mass_weighted_unit_vector_to_the_camera():
    ev = np.zeros((1, 8))
    pos = np.array([[1.0, 2.0, 3.0]])
    O.evidence_fold(ev, np.array([[2.0, 0.5, 3.0]]), pos, (1.0, 2.0, 7.0))   # straight up z, 4 away
    O.evidence_fold(ev, np.array([[1.0, 0.0, 1.0]]), pos, (4.0, 6.0, 3.0))   # (3, 4, 0) / 5
    O.evidence_fold(ev, np.array([[0.0, 9.0, 9.0]]), pos, (9.0, 9.0, 9.0))   # no in-mask mass: no direction
    np.testing.assert_allclose(ev[0, 4:7], [0.6, 0.8, 2.0], rtol=1e-12)
    np.testing.assert_allclose(ev[0, :3], [3.0, 13.0, 9.5])
    assert ev[0, 7] == 5.0


def test_probe_alpha_is_the_forward_alpha():
    sc = S.fd_scene(31, n=80)
    pr, bn, fw = _render(sc)
    out = O.probe(pr, bn, sc.W, sc.H, tau=0.5, delta=0.1)
    np.testing.assert_array_equal(out[:, 0], fw["out_rgba"][:, 3])
    # the trimmed lists of the forward give the same probe
    np.testing.assert_array_equal(O.probe(pr, bn, sc.W, sc.H, 0.5, 0.1, tile_ranges=fw["tile_ranges"]), out)


def test_probe_limits():
    sc = S.fd_scene(32, n=80)
    pr, bn, fw = _render(sc)
    A = fw["out_rgba"][:, 3]
    vis = _brute_vis(sc, pr)
    z = pr["proj1"][:, 2].astype(np.float64)
    covered = A > 0
    # tau above any alpha: no first surface, nothing deep
    out = O.probe(pr, bn, sc.W, sc.H, tau=2.0, delta=0.0)
    assert np.isinf(out[:, 1]).all() and (out[:, 2] == 0).all()
    # a tiny tau: the first composited fragment's depth
    out = O.probe(pr, bn, sc.W, sc.H, tau=1e-9, delta=np.inf)
    first = np.where(vis > 0, z[:, None], np.inf).min(0)
    np.testing.assert_array_equal(out[covered, 1], first[covered].astype(np.float32))
    assert (out[:, 2] == 0).all()  # delta = inf: nothing is deep
    # behind: ref_z = -inf takes every fragment (behind = A), none without a reference
    ref = np.full(sc.W * sc.H, -np.inf, np.float32)
    out = O.probe(pr, bn, sc.W, sc.H, tau=0.5, delta=0.0, ref_z=ref, margin=0.0)
    np.testing.assert_allclose(out[:, 3], A, atol=2e-6)
    assert (O.probe(pr, bn, sc.W, sc.H, 0.5, 0.0)[:, 3] == 0).all()
    # mean mode: the alpha-weighted mean depth where more than 5% covered
    out = O.probe(pr, bn, sc.W, sc.H, tau=0.0, delta=np.inf)
    tot = vis.sum(0)
    mean = (vis * z[:, None]).sum(0) / np.maximum(tot, 1e-30)
    sel = tot > 0.06
    assert sel.sum() > 100
    np.testing.assert_allclose(out[sel, 1], mean[sel], rtol=1e-5)
    assert np.isinf(out[tot < 0.04, 1]).all()
