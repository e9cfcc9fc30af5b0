"""Gradients accumulated over several views (8 camera poses rendered forward + backward one
after another, parameter gradients summed). The reference's gradient export overwrites grad_out
(src/gpu/optim.cu:292-296) and consumes v_splat per view (optim.cu:110-121), so a multi-view sum needs this
build's accumulate flag (B2C_GRAD_ACCUMULATE): the projection VJP of each view adds its rows into grads.

* config 4 cut to a quarter of the image in each direction (the same splat sizes, depths, density and so
  the same ~190 composited fragments per pixel, 187,500 splats at 480x270, SH degree 4), all 8 poses:
  - the training step with the accumulate flag over the 8 views equals, bit for bit, the float32
    running sum of the 8 single-view gradients (each view's step is deterministic);
  - the accumulated gradients agree with the sum of the oracle's 8 per-view VJPs, each fed that view's
    GPU v_splat (<= 1e-3 of each column's largest value);
* an FD-harness scene seen from 3 poses: the accumulated analytic gradients against central finite
  differences of the fp64 brute-force loss summed over the 3 views (relative 1e-3)."""
import numpy as np
import pytest

from b2ctrain_amd import _native
from b2ctrain_amd import scenes as S
from oracle import oracle as O
from tests.fd_util import fd_compare
from tests.gpu_harness import emit, rel_percentiles

pytestmark = pytest.mark.gpu


def _scene4():
    sc = S.config4(shrink=4)
    sc.bg = (0.2, 0.25, 0.3)
    return sc


@pytest.mark.timeout(600)
def test_config4_eight_views_accumulate_equals_sum_of_views():
    sc = _scene4()
    cams = sc.extra_cams
    emit(f"config4/4: {sc.n} splats SH4 {sc.W}x{sc.H}, {len(cams)} views")
    r = _native.Renderer(sc)
    try:
        r.step(cam=cams[0])  # allocates the grads buffer
        singles = []
        for v, cam in enumerate(cams):
            r.step(cam=cam)
            singles.append(r.read("grads").copy())
            emit(f"  view {v}: M={r.info().num_isect}")
        r.zero("grads")
        for cam in cams:
            r.step(cam=cam, accumulate=True)
        acc = r.read("grads")
    finally:
        r.close()
    run = np.zeros_like(singles[0])
    for g in singles:
        run = (run + g).astype(np.float32)
    assert np.isfinite(acc).all()
    assert np.array_equal(acc, run), f"{int((acc != run).sum())} entries differ from the float32 running sum"
    touched = (np.abs(np.stack(singles)) > 0).any(2).sum(0)
    emit(f"  splats with gradient in k views: {np.bincount(touched, minlength=9).tolist()}")
    # the views overlap: many rows are sums of several views (only the splats in front of the ~190
    # composited fragments of a pixel receive gradient at all)
    assert (touched >= 2).sum() > 10_000


@pytest.mark.timeout(600)
def test_config4_eight_views_accumulate_vs_oracle_vjps():
    sc = _scene4()
    cams = sc.extra_cams
    gs = 3.0 * sc.W * sc.H
    r = _native.Renderer(sc)
    ref = np.zeros((sc.n, 11 + 3 * sc.K), np.float64)
    try:
        for v, cam in enumerate(cams):
            emit(f"  view {v}")
            r.forward(cam=cam)
            r.loss(grad_scale=gs)
            r.zero("v_splat")
            r.zero("vis_flag")
            r.backward(mode=1, grad_scale=gs, cam=cam)
            vs, vf, tc = r.read("v_splat"), r.read("vis_flag"), r.read("tile_count")
            if v == 0:
                r.vjp(cam=cam)  # overwrite: the first view starts the sum
            else:
                r.vjp(cam=cam, accumulate=True)
            ref += O.vjp(sc.with_camera(cam), S.camera_gpu(cam), vs, vf, tc).astype(np.float64)
        acc = r.read("grads")
    finally:
        r.close()
    col = np.abs(ref).max(axis=0) + 1e-30
    err = float((np.abs(acc - ref) / col).max())
    pc = rel_percentiles(acc, ref)
    emit(f"  column-max err {err:.2e}; per-entry rel p50 {pc['p50']:.1e} p99 {pc['p99']:.1e} over {pc['n']}")
    assert err <= 1e-3
    assert pc["p99"] <= 1e-3


def test_fd_three_views_summed_loss():
    sc = S.multiview_fd_scene(1242, views=3)
    cams = sc.extra_cams
    gs = 3.0 * sc.W * sc.H
    emit(f"FD {sc.name}: gradients of the loss summed over {len(cams)} views")
    r = _native.Renderer(sc)
    try:
        for v, cam in enumerate(cams):
            r.forward(cam=cam)
            r.loss(grad_scale=gs)
            r.backward(mode=1, grad_scale=gs, cam=cam)
            r.vjp(cam=cam, accumulate=v > 0)
        an = r.read("grads")
    finally:
        r.close()
    checked, skipped, bad, worst = fd_compare(sc, an, cams=cams)
    emit(f"  checked {checked} skipped {skipped} worst rel {worst:.2e}")
    assert checked > 150
    assert not bad, f"{len(bad)} mismatches, e.g. {bad[:5]}"
