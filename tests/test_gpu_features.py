"""Feature lanes, the normal-map loss, the hollow loss and the eval metrics on the GPU (FeatureMode::Normals
and ::Buffer, src/gpu/project.cu:63-77, raster_fwd.cu FEAT/HOLLOW, raster_bwd.cu:84-110,
raster_bwd_tc.cu:126-141, loss.cu:197-293, optim.cu:235-250) against the CPU oracle stage by stage, and the
analytic gradients against finite differences of the double-precision brute force (the reference's FD
harness configurations with normals and the hollow loss, tests/tests.cpp:386-391).

Bars: projection (with the feature lanes) bit-exact; out_feat and hollow_pen within 1e-4 like the colour;
the normal loss's per-pixel gradient bit-exact and its value within 1e-6; the hollow and eval sums within
1e-5; v_splat (lanes 0-12) within 2e-3 of each lane's maximum; parameter gradients within 1e-3 of each
column's maximum; FD relative error 1e-3 (tests/fd_util.py)."""
import numpy as np
import pytest

from b2ctrain_amd import _native
from b2ctrain_amd import scenes as S
from oracle import oracle as O
from tests.fd_util import fd_compare
from tests.gpu_harness import emit, full_check

pytestmark = pytest.mark.gpu

FEATURE_SCENES = {
    "normals": lambda: S.fd_feature_scene(1236, normals=True),
    "hollow": lambda: S.fd_feature_scene(1234, hollow=True),
    "masked_hollow": lambda: S.fd_feature_scene(1235, masked=True, hollow=True),
    "normals_hollow": lambda: S.fd_feature_scene(1236, normals=True, hollow=True),
}


@pytest.mark.parametrize("mode", [0, 1])
@pytest.mark.parametrize("name", list(FEATURE_SCENES))
def test_feature_stages_match_oracle(name, mode):
    sc = FEATURE_SCENES[name]()
    emit(f"features {sc.name} mode {mode}")
    full_check(sc, mode=mode, fp64_rgba=True)


def _config2_with_features(n=20_000, seed=7):
    sc = S.config2(n=n)
    rng = np.random.default_rng(seed)
    P = sc.W * sc.H
    rgb = (rng.random((P, 3)) * 255).astype(np.uint32)
    a = np.where(rng.random(P) > 0.3, 255, 0).astype(np.uint32)
    sc.normals = (rgb[:, 0] | (rgb[:, 1] << 8) | (rgb[:, 2] << 16) | (a << 24)).astype(np.uint32)
    sc.feat_mode = 1
    sc.normal_scale = 0.05 / max(float((a > 0).sum()), 1.0)
    y, x = np.mgrid[0:sc.H, 0:sc.W]
    sc.hollow_z = (4.0 + 0.3 * np.sin(x * 0.02) + 0.2 * np.cos(y * 0.03)).astype(np.float32).reshape(-1)
    sc.hollow_margin, sc.hollow_lam = 0.05, 0.7 / P
    sc.name = f"cfg2/{n}+normals+hollow"
    return sc


@pytest.mark.timeout(300)
@pytest.mark.parametrize("mode", [0, 1])
def test_config2_with_normals_and_hollow(mode):
    sc = _config2_with_features()
    emit(f"features {sc.name} mode {mode}")
    full_check(sc, mode=mode)


def test_feature_buffer_lanes():
    """FeatureMode::Buffer: a caller's per-splat features (non-finite -> 0, clamped to +-100) composited
    and back-propagated like the colour."""
    sc = S.config2(n=20_000)
    rng = np.random.default_rng(3)
    buf = rng.normal(0, 30, (sc.n, 3)).astype(np.float32)
    buf[::97, 0] = np.nan
    buf[1::89, 1] = 1e6
    sc.feat_mode, sc.feat_buffer = 2, buf
    sc.name = "cfg2/20000+buffer"
    emit(f"features {sc.name}")
    full_check(sc, mode=1, loss=False)
    # the backward with a v_feat of the caller's: v_splat lanes 10-12 are the sums of vis * v_feat
    r = _native.Renderer(sc)
    try:
        W, H = sc.W, sc.H
        camd = _native.camera_gpu_from(sc.cam)
        gs = 3.0 * W * H
        r.forward()
        r.loss(grad_scale=gs)
        vfeat = np.zeros((W * H, 4), np.float32)
        vfeat[:, :3] = rng.normal(0, 1, (W * H, 3)) * gs * 1e-7
        r.write("v_feat", vfeat)
        r.zero("v_splat")
        r.zero("vis_flag")
        r.backward(mode=1, grad_scale=gs)
        vs = r.read("v_splat")
        pr = O.project(sc, camd)
        bn = O.bin_(pr, W, H)
        fw = dict(tile_ranges=r.read("tile_ranges"), out_rgba=r.read("out_rgba"), out_T=r.read("out_feat")[:, 3],
                  last_idx=r.read("last_idx"))
        ref, _, _ = O.raster_bwd(pr, bn, fw, r.read("v_out"), W, H, sc.bg, sc.n, inv_gscale=1.0 / gs, v_feat=vfeat)
        scale = np.abs(ref).max(axis=0) + 1e-30
        err = float((np.abs(vs - ref) / scale).max())
        emit(f"    v_splat (buffer features) lane-max err {err:.2e}")
        assert err <= 2e-3
        assert np.abs(ref[:, 10:13]).max() > 0
    finally:
        r.close()


@pytest.mark.parametrize("mask_weighted", [False, True])
def test_eval_metrics(mask_weighted):
    sc = S.config3(n=100_000, masked=True)
    emit(f"eval {sc.name} mask_weighted={mask_weighted}")
    r = _native.Renderer(sc)
    try:
        r.forward(bg=(0.0, 0.0, 0.0))
        r.zero("loss_accum")
        r.eval_metrics(mask_weighted=mask_weighted)
        acc = r.read("loss_accum")
        se, ss = O.eval_metrics(sc.W, sc.H, r.read("out_rgba"), sc.gt, mask_weighted)
        emit(f"    squared error {acc[4]:.6g} (oracle {se:.6g}), SSIM {acc[5]:.6g} (oracle {ss:.6g})")
        assert abs(acc[4] - se) <= 1e-5 * abs(se)
        assert abs(acc[5] - ss) <= 1e-5 * abs(ss)
        assert acc[0] == 0.0 and acc[1] == 0.0  # only [4] and [5] are touched
    finally:
        r.close()


def gpu_gradients(scene, mode=1):
    r = _native.Renderer(scene)
    gs = 3.0 * scene.W * scene.H if mode == 1 else 1.0
    try:
        r.forward()
        r.loss(grad_scale=gs)
        if scene.normals is not None:
            r.normal_loss(grad_scale=gs)
        r.zero("v_splat")
        r.zero("vis_flag")
        r.backward(mode=mode, grad_scale=gs)
        r.vjp()
        return r.read("grads")
    finally:
        r.close()


@pytest.mark.parametrize("mode", [0, 1])
@pytest.mark.parametrize("name", list(FEATURE_SCENES))
def test_fd_feature_scenes(name, mode):
    sc = FEATURE_SCENES[name]()
    emit(f"FD {sc.name} mode {mode}")
    an = gpu_gradients(sc, mode)
    checked, skipped, bad, worst = fd_compare(sc, an)
    emit(f"  checked {checked} skipped {skipped} worst rel {worst:.2e}")
    assert checked > 120
    assert not bad, f"{len(bad)} mismatches, e.g. {bad[:5]}"


def test_train_step_with_normals_and_hollow():
    """b2c_train_step with the normal-map and hollow losses in the trainer's order (trainer.cpp:502-505):
    loss_accum = [photometric + hollow, normal, their sum, 1], and the gradients of the staged calls."""
    sc = S.fd_feature_scene(1236, normals=True, hollow=True)
    emit(f"train step {sc.name}")
    gs = 3.0 * sc.W * sc.H
    r = _native.Renderer(sc)
    try:
        r.step()
        acc = r.read("loss_accum")
        g_step = r.read("grads").copy()
        r.forward()
        photo = r.loss(grad_scale=gs)
        r.normal_loss(grad_scale=gs)
        r.hollow_loss()
        staged = r.read("loss_accum")
        r.zero("v_splat")
        r.zero("vis_flag")
        r.backward(mode=1, grad_scale=gs)
        r.vjp()
        g_staged = r.read("grads")
    finally:
        r.close()
    emit(f"    loss_accum {acc[:4]} (photometric alone {photo:.6g})")
    assert acc[0] == staged[0] and acc[1] == staged[1] and acc[1] > 0
    assert acc[2] == np.float32(acc[0] + acc[1]) and acc[3] == 1.0
    assert acc[0] != np.float32(photo)  # the hollow term is in [0]
    assert np.array_equal(g_step, g_staged)
