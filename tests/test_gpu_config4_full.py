"""BASELINE configuration 4 at full size, once: 3M splats at SH degree 4, 1920x1080, 8 camera poses with
gradients accumulated over the views (about 117M intersections a view, a 5.6 GB row buffer; the regime
where 32-bit index and size arithmetic is most exposed).

* view 0: the projection bit-exact against the oracle and the tile key / value lists, depth order, count
  scan and tile ranges bit-exact against orc_bin (binning.cu:109-143);
* the 8-view training step with the accumulate flag equals, bit for bit, the float32 running sum of the
  8 single-view gradients, and every gradient is finite;
* vis_weight (raster_bwd_tc.cu:177-195) over the 8 accumulated views sums to the accumulated alpha
  sum(1 - T_final) of the 8 rendered images, to 1e-4."""
import numpy as np
import pytest

from b2ctrain_amd import _native
from b2ctrain_amd import scenes as S
from tests.gpu_harness import check_binning, check_projection, emit

pytestmark = pytest.mark.gpu


@pytest.mark.timeout(900)
def test_config4_full_size_eight_views():
    sc = S.config4()
    sc.bg = (0.2, 0.25, 0.3)
    cams = sc.extra_cams
    emit(f"config4 full size: {sc.n} splats SH4 {sc.W}x{sc.H}, {len(cams)} views")
    r = _native.Renderer(sc)
    try:
        camd = S.camera_gpu(cams[0])
        r.project(cam=cams[0], bg=sc.bg)
        emit("  view 0: projection")
        pr = check_projection(r, sc, camd)
        r.bin()
        emit(f"  view 0: binning (M={r.info().num_isect})")
        bn = check_binning(r, pr, sc.W, sc.H)
        assert bn["M"] > 100_000_000
        del pr, bn

        r.step(cam=cams[0])  # allocates the grads buffer
        run = None
        for v, cam in enumerate(cams):
            r.step(cam=cam)
            g = r.read("grads")
            assert np.isfinite(g).all(), f"view {v}: non-finite gradients"
            run = g.copy() if run is None else (run + g).astype(np.float32)
            emit(f"  view {v}: M={r.info().num_isect}, {int((g != 0).any(1).sum())} splats with gradient")
            del g
        r.zero("grads")
        r.write_model("vis_weight", np.zeros(sc.n, np.float32))
        alpha = 0.0
        for cam in cams:
            r.step(cam=cam, accumulate=True)
            alpha += float(r.read("out_rgba")[:, 3].astype(np.float64).sum())
        acc = r.read("grads")
        vw = r.read_model("vis_weight")
    finally:
        r.close()
    assert np.array_equal(acc, run), f"{int((acc != run).sum())} entries differ from the float32 running sum"
    total = float(vw.astype(np.float64).sum())
    emit(f"  accumulated = running sum; vis_weight sums to {total:.6g}, the 8 images' alpha to {alpha:.6g}")
    assert alpha > 0.5 * len(cams) * sc.W * sc.H
    assert abs(total - alpha) <= 1e-4 * alpha
