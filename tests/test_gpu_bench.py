"""bench.py's CPU-baseline leg on the GPU context it is meant for: after the benchmark's own training step
(which leaves proj0..3 unwritten) the leg re-projects, reads the GPU's projection, lists and loss gradient,
and its CPU forward over them must composite exactly the fragments the oracle's forward does on the same
scene (the lists are bit-exact)."""
import numpy as np
import pytest

import bench
from b2ctrain_amd import _native
from b2ctrain_amd import scenes as S
from oracle import oracle as O
from tests.gpu_harness import emit

pytestmark = pytest.mark.gpu


def test_cpu_baseline_frame_reads_the_step_frame():
    sc = S.config2(n=20_000)
    bg = (0.3, 0.2, 0.1)
    emit(f"bench CPU-baseline frame, {sc.name}")
    r = _native.Renderer(sc)
    try:
        f_sweep, (f_contrib, tiled, ref) = bench.cpu_baseline_frame(r, sc, 1, bg, sc.cam)
    finally:
        r.close()
    pr = O.project(sc, S.camera_gpu(sc.cam))
    bn = O.bin_(pr, sc.W, sc.H)
    fw = O.raster_fwd(pr, bn, sc.W, sc.H, bg)
    ranges = fw["tile_ranges"].astype(np.int64)
    assert f_sweep == int(64 * (ranges[:, 1] - ranges[:, 0]).clip(min=0).sum())
    assert f_contrib == fw["f_contrib"] > 0
    assert tiled["value"] > 0 and ref["value"] > 0
