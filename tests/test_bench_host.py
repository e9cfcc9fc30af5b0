"""bench.py's host-side legs on the CPU: the CPU-baseline leg (the whole tiled step of the oracle from the scene)
run end to end, and the algorithmic byte formulas."""
import numpy as np

import bench
from b2ctrain_amd import scenes as S
from oracle import oracle as O


class _OracleContext:
    """The reads cpu_baselines makes of a Renderer, served from the oracle: proj0..2 (no feature lanes, as the
    context's read of them), the sorted tile keys and splat ids, and v_out."""

    def __init__(self, sc, bg):
        pr = O.project(sc, S.camera_gpu(sc.cam))
        bn = O.bin_(pr, sc.W, sc.H)
        fw = O.raster_fwd(pr, bn, sc.W, sc.H, bg)
        _, v_out = O.photometric(sc, fw["out_rgba"], grad_scale=3.0 * sc.W * sc.H, bg=bg)
        self.buf = {k: pr[k] for k in ("proj0", "proj1", "proj2")}
        self.buf.update(keys_sorted=bn["keys_sorted"], vals_sorted=bn["vals_sorted"], v_out=v_out)
        self.fw = fw

    def read(self, k):
        return self.buf[k].copy()


def test_cpu_baseline_leg_runs_on_the_oracle():
    sc = S.fd_scene(61, n=50)
    bg = (0.2, 0.1, 0.3)
    ctx = _OracleContext(sc, bg)
    ranges = ctx.fw["tile_ranges"].astype(np.int64)
    f_sweep = int(64 * (ranges[:, 1] - ranges[:, 0]).clip(min=0).sum())
    f_contrib, tiled, ref = bench.cpu_baselines(ctx, sc, bg, f_sweep)
    assert f_contrib == ctx.fw["f_contrib"] > 0
    assert tiled["value"] > 0 and tiled["kind"] == "port" and tiled["cores"] >= 1
    assert set(tiled["stage_seconds"]) == {"project", "bin", "forward", "loss", "backward", "vjp"}
    assert f"F_sweep={f_sweep}," in tiled["sample"]  # the CPU's own lists sweep the GPU's fragment count
    assert ref["value"] > 0 and ref["cores"] == 1


def test_byte_formulas():
    assert bench.projection_bytes(10, 4, 192) == 10 * 52 + 4 * (192 + 72)
    # 4 depth passes (16 B/splat), 2 tile passes at 12 tile bits (16 B/isect), scan 8 B/splat, emit 20 + 8
    assert bench.binning_bytes(100, 1000, 12) == 4 * 16 * 100 + 2 * 16 * 1000 + 8 * 100 + 20 * 100 + 8 * 1000
    assert bench.update_bytes(1, 12) == 68 + 2 * (48 + 96 + 24 + 4) + 64
