"""The tile-list replays on the GPU (b2c_compute_evidence / b2c_download_evidence / b2c_download_labels,
replacing src/train/evidence.cu:47-264, and b2c_probe_depth, replacing src/gpu/probe.cu:7-53) against the CPU
oracle on the same lists.

Bars: per-splat evidence columns within 1e-4 of each column's maximum (the replay's alpha is the hardware
exp2 of the forward, the oracle's expf; the GPU sums with float atomics); the probe's accumulated alpha equal
bit for bit to the forward's own; z_first equal to the oracle's wherever the oracle's crossing is clear of
tau by 1e-4, deep and behind within 1e-4 there; label winners equal wherever the oracle's winning share leads
the runner-up by 1e-3."""
import numpy as np
import pytest

from b2ctrain_amd import _native
from b2ctrain_amd import scenes as S
from oracle import oracle as O
from tests.gpu_harness import emit

pytestmark = pytest.mark.gpu


def _oracle_evidence(sc, cams, views, normal_weight=0.0, fws=None):
    """download_evidence / download_labels of the oracle: per view the oracle's forward (or the GPU's, fws)
    and replay, folded in double."""
    ev = np.zeros((sc.n, 8))
    lab_total = np.zeros((sc.n, O.LABEL_BINS)) if any(v.get("labels") is not None for v in views) else None
    for i, (cam, v) in enumerate(zip(cams, views)):
        camd = S.camera_gpu(cam, sc.W, sc.H)
        nrm = v.get("normals") if normal_weight > 0 else None
        if nrm is not None and sc.feat_mode != 1:
            raise ValueError("the normal residual needs a scene with pseudo-normal features")
        pr = O.project(sc, camd)
        bn = O.bin_(pr, sc.W, sc.H)
        fw = fws[i] if fws is not None else O.raster_fwd(pr, bn, sc.W, sc.H, (0.0, 0.0, 0.0), feat=nrm is not None)
        acc, lab = O.evidence_view(pr, bn, fw, sc.W, sc.H, v["gt"], v.get("weights"), normals=nrm,
                                   labels=v.get("labels"), masked_has_alpha=v.get("masked_has_alpha", False),
                                   normal_weight=normal_weight)
        O.evidence_fold(ev, acc, sc.pos_op, cam.pos)
        if lab is not None:
            lab_total += lab
    return O.evidence_export(ev), lab_total


def _col_err(got, want):
    scale = np.abs(want).max(0) + 1e-30
    return np.abs(got - want).max(0) / scale


def _views(sc, specs):
    return [_native.View(sc.W, sc.H, v["gt"], v.get("weights"), v.get("normals"), v.get("labels"),
                         has_alpha=v.get("has_alpha", True), masked=v.get("masked", False)) for v in specs]


@pytest.mark.parametrize("masked", [False, True])
def test_evidence_one_view_matches_oracle(masked):
    sc = S.config2(n=20_000)
    emit(f"evidence {sc.name} masked={masked}")
    spec = dict(gt=sc.gt, weights=sc.weights, masked=masked, masked_has_alpha=masked)
    r = _native.Renderer(sc)
    vs = _views(sc, [spec])
    try:
        ev = r.compute_evidence(vs, [sc.cam])
        fw = dict(tile_ranges=r.read("tile_ranges"), out_rgba=r.read("out_rgba"), last_idx=r.read("last_idx"))
    finally:
        for v in vs:
            v.close()
        r.close()
    want, _ = _oracle_evidence(sc, [sc.cam], [spec], fws=[fw])
    err = _col_err(ev, want)
    emit(f"    column errors {np.array2string(err, precision=2)}; splats with mass {(want[:, 0] > 0).sum()}")
    assert (want[:, 2] > 0).sum() > 1000
    assert (err <= 1e-4).all()
    assert ((ev[:, 3] == 0) == (want[:, 3] == 0)).all()


def test_evidence_multi_view_with_normals():
    sc = S.fd_feature_scene(51, n=60, normals=True)
    cams = S.multiview_fd_scene(51, views=3).extra_cams
    emit(f"evidence {sc.name} x{len(cams)} views with the normal residual")
    rng = np.random.default_rng(5)
    specs = []
    for v in range(len(cams)):
        g = (rng.random((sc.W * sc.H, 4)) * 255).astype(np.uint32)
        gt = g[:, 0] | (g[:, 1] << 8) | (g[:, 2] << 16) | (g[:, 3] << 24)
        specs.append(dict(gt=gt, weights=(64 + rng.random(sc.W * sc.H) * 191).astype(np.uint8), normals=sc.normals,
                          masked=v == 1, masked_has_alpha=v == 1))
    r = _native.Renderer(sc)
    vs = _views(sc, specs)
    try:
        ev = r.compute_evidence(vs, cams, normal_weight=0.4)
        ev0 = r.compute_evidence(vs, cams, normal_weight=0.0)
    finally:
        for v in vs:
            v.close()
        r.close()
    want, _ = _oracle_evidence(sc, cams, specs, normal_weight=0.4)
    want0, _ = _oracle_evidence(sc, cams, specs, normal_weight=0.0)
    err, err0 = _col_err(ev, want), _col_err(ev0, want0)
    emit(f"    column errors {np.array2string(err, precision=2)} / without normals {np.array2string(err0, precision=2)}")
    assert (err <= 1e-4).all() and (err0 <= 1e-4).all()
    assert ev[:, 2].sum() > ev0[:, 2].sum() * 1.01  # the normal residual raised the error mass
    assert (want[:, 3] > 1.5).sum() > 10  # splats supported by more than one view


def test_label_vote_half_frame_and_oracle():
    """The reference's label test (tests/tests.cpp:250-279) on the GPU, and the votes against the oracle."""
    sc = S.fd_scene(11, n=60)
    emit(f"labels {sc.name}")
    x = np.arange(sc.W * sc.H) % sc.W
    labels = np.where(x < sc.W // 2, 3, 13).astype(np.uint8)
    spec = dict(gt=sc.gt, labels=labels)
    r = _native.Renderer(sc)
    vs = _views(sc, [spec])
    try:
        ev = r.compute_evidence(vs, [sc.cam], export_labels=True)
        lv = r.download_labels()
        fw = dict(tile_ranges=r.read("tile_ranges"), out_rgba=r.read("out_rgba"), last_idx=r.read("last_idx"))
    finally:
        for v in vs:
            v.close()
        r.close()
    px = 40.0 * sc.pos_op[:, 0] / sc.pos_op[:, 2] + sc.W / 2.0
    voted = checked = 0
    for i in range(sc.n):
        voted += lv[i, 1] > 0
        if abs(px[i] - sc.W / 2.0) < 6 or px[i] < 2 or px[i] > sc.W - 2:
            continue
        checked += 1
        assert int(lv[i, 0]) == (3 if px[i] < sc.W / 2.0 else 13) and lv[i, 1] > 0.9, (i, px[i], lv[i])
    emit(f"    {voted}/{sc.n} voted, {checked} checked")
    assert checked > 20
    _, lab = _oracle_evidence(sc, [sc.cam], [spec], fws=[fw])
    win = O.label_winners(lab)
    srt = np.sort(lab, 1)
    clear = (srt[:, -1] - srt[:, -2]) > 1e-3 * np.maximum(srt[:, -1], 1e-30)
    assert (lv[clear, 0] == win[clear, 0]).all()
    np.testing.assert_allclose(lv[:, 1], win[:, 1], atol=1e-4)
    assert ((ev[:, 1] > 0) == (lv[:, 1] > 0)).all()  # unweighted, every id below 32: w_all > 0 <=> a vote


def test_labels_many_classes_config2():
    sc = S.config2(n=20_000)
    emit(f"labels {sc.name}: 8x8-pixel class blocks, ids 0..39")
    bx = (np.arange(sc.W * sc.H) % sc.W) // 8
    by = (np.arange(sc.W * sc.H) // sc.W) // 8
    labels = ((bx * 7 + by * 3) % 40).astype(np.uint8)
    spec = dict(gt=sc.gt, weights=sc.weights, labels=labels)
    r = _native.Renderer(sc)
    vs = _views(sc, [spec])
    try:
        r.compute_evidence(vs, [sc.cam], export_labels=True)
        lv = r.download_labels()
        fw = dict(tile_ranges=r.read("tile_ranges"), out_rgba=r.read("out_rgba"), last_idx=r.read("last_idx"))
    finally:
        for v in vs:
            v.close()
        r.close()
    _, lab = _oracle_evidence(sc, [sc.cam], [spec], fws=[fw])
    win = O.label_winners(lab)
    srt = np.sort(lab, 1)
    clear = (srt[:, -1] - srt[:, -2]) > 1e-3 * np.maximum(srt[:, -1], 1e-30)
    emit(f"    voting splats {(win[:, 1] > 0).sum()}, clear winners {clear.sum()}")
    assert clear.sum() > 1000
    assert (lv[clear, 0] == win[clear, 0]).all()
    np.testing.assert_allclose(lv[:, 1], win[:, 1], atol=1e-4)
    assert (lv[:, 0] < 32).all()


@pytest.mark.parametrize("tau", [0.5, 0.0])
def test_probe_matches_oracle(tau):
    sc = S.config2(n=20_000)
    emit(f"probe {sc.name} tau={tau}")
    y, x = np.mgrid[0:sc.H, 0:sc.W]
    ref_z = (3.5 + 0.5 * np.sin(x * 0.01) * np.cos(y * 0.013)).astype(np.float32).reshape(-1)
    ref_z[::13] = np.inf
    r = _native.Renderer(sc)
    try:
        r.forward(bg=(0.0, 0.0, 0.0))
        A_fwd = r.read("out_rgba")[:, 3].copy()
        ranges = r.read("tile_ranges")
        out = r.probe_depth(tau, 0.2, ref_z, 0.1)
        out_none = r.probe_depth(tau, 0.2, None, 0.1)
    finally:
        r.close()
    np.testing.assert_array_equal(out[:, 0], A_fwd)
    np.testing.assert_array_equal(out_none[:, :3], out[:, :3])
    assert (out_none[:, 3] == 0).all()
    pr = O.project(sc, S.camera_gpu(sc.cam))
    bn = O.bin_(pr, sc.W, sc.H)
    want = O.probe(pr, bn, sc.W, sc.H, tau, 0.2, ref_z, 0.1, tile_ranges=ranges)
    np.testing.assert_allclose(out[:, 0], want[:, 0], atol=1e-5)
    with np.errstate(invalid="ignore"):  # inf - inf where neither has a first surface
        same_z = (out[:, 1] == want[:, 1]) | (np.abs(out[:, 1] - want[:, 1]) <= 1e-5 * np.abs(want[:, 1]))
    frac = 1.0 - same_z.mean()
    emit(f"    z_first differs on {frac:.2e} of pixels; covered {(out[:, 0] > 0.5).mean():.2f}")
    assert frac <= 1e-3
    np.testing.assert_allclose(out[same_z, 2:], want[same_z, 2:], atol=1e-4)
    assert (out[:, 3] > 0).sum() > 100
