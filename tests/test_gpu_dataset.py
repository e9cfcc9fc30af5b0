"""Dataset views on the device (b2c_dataset_view_upload): the ViewGPU built from a loaded COLMAP view feeds the
loss, the normal loss and the evidence label vote exactly as a view built from the same host planes does."""
import numpy as np
import pytest

from b2ctrain_amd import _native as N
from b2ctrain_amd import scenes as S
from tests.gpu_harness import emit
from tests.test_dataset import SCENE

pytestmark = pytest.mark.gpu


def _scene_for(info, planes, seed):
    """Splats in front of the view's camera (placed in camera space, moved to the world by R^T (p - t))."""
    rng = np.random.default_rng(seed)
    n = 40
    R = np.array(info.cam.R, np.float64).reshape(3, 3)
    t = np.array(info.cam.t, np.float64)
    pc = np.stack([rng.uniform(-0.5, 0.5, n), rng.uniform(-0.4, 0.4, n), rng.uniform(1.5, 2.5, n)], 1)
    pw = (pc - t) @ R  # R^T (p - t) row-wise
    cam = S.Camera(info.cam.width, info.cam.height, info.cam.fx, info.cam.fy, info.cam.cx, info.cam.cy,
                   np.array(info.cam.R, np.float32), np.array(info.cam.t, np.float32))
    pos_op = np.concatenate([pw, rng.uniform(-1, 2, (n, 1))], 1).astype(np.float32)
    lscale = np.concatenate([np.log(rng.uniform(0.05, 0.12, (n, 3))), np.zeros((n, 1))], 1).astype(np.float32)
    quat = rng.normal(0, 1, (n, 4)).astype(np.float32)
    sh = rng.normal(0, 0.5, (n, 4, 3)).astype(np.float32)
    sc = S.Scene(f"colmap{seed}", 1, pos_op, quat, lscale, sh, cam, planes["rgba"], planes.get("weights"),
                 composite=not info.masked, mask=bool(info.masked), alpha_lane=not info.masked,
                 match_alpha_weight=0.3, bg=(0.1, 0.2, 0.3))
    if "normals" in planes:
        sc.normals = planes["normals"]
        sc.feat_mode = 1
        sc.normal_scale = 0.05 / max(info.normal_mask_count, 1.0)
    return sc


def test_uploaded_views_feed_the_losses():
    ds = N.Dataset(SCENE, eval_split_every=3)
    try:
        for split in (0, 1):
            for i in range(ds.count(split)):
                info, planes = ds.info(split, i), ds.planes(split, i)
                emit(f"view {info.name.decode()} ({info.w}x{info.h}, masked={info.masked})")
                sc = _scene_for(info, planes, 100 + 10 * split + i)
                r = N.Renderer(sc, W=info.w, H=info.h)
                dev = ds.upload(split, i)
                mine = r.view
                try:
                    r.forward()
                    own = r.loss(grad_scale=3.0 * info.w * info.h)
                    v_own = r.read("v_out").copy()
                    r.view = dev
                    got = r.loss(grad_scale=3.0 * info.w * info.h)
                    assert got == own and np.array_equal(r.read("v_out"), v_own)
                    if "normals" in planes:
                        r.zero("loss_accum")
                        r.normal_loss(grad_scale=1.0)
                        a = r.read("loss_accum")[1]
                        r.view = mine
                        r.zero("loss_accum")
                        r.normal_loss(grad_scale=1.0)
                        assert r.read("loss_accum")[1] == a
                finally:
                    r.view = mine
                    N.lib().b2c_view_destroy(dev)
                    r.close()
    finally:
        ds.close()
