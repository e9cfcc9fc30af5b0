"""Benchmark of the MI355X splat rasterizer on BASELINE.json's metric configuration (config 3).

One step = one training step of the hot path on one view, inputs resident in HBM: projection + binning/
sort + forward raster + fused L1/SSIM/alpha loss + MFMA backward + projection VJP (trainer.cpp:487-529
order, grad_out semantics). A new random background is drawn each step (trainer.cpp:470-471).

Prints ONE JSON line. value = Gfrag/s = F_sweep / (t_forward + t_backward) (BASELINE.md's definition:
F_sweep = sum over tiles of 64 x shrunk list length). Stage times come from hipEvents recorded on the
context's stream around each stage; ms_per_step is the wall time of the K timed steps over K, bracketed by
stream synchronisation.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "raster fwd+bwd ms/step @1M splats 1080p; Gfrag/s; % HBM roofline"
HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def projection_bytes(n, n_ok, sh_bytes):
    # all splats: pos_op + quat + lscale (48 B) and tile_count (4 B); splats that pass: SH coefficients,
    # proj0..2 (48 B), proj3 (8 B), hit_info (8 B), max_screen read + write (8 B)
    return n * 52 + n_ok * (sh_bytes + 72)


def cpu_baseline(r, scene, bg):
    """The CPU port (oracle, fp32 tiled restatement, one host core) timed on the same frame: forward raster
    + backward raster over the GPU's own tile lists and per-pixel loss gradient."""
    from oracle import oracle as O

    W, H = scene.W, scene.H
    tx, ty, T, _ = O.tile_geometry(W, H)
    keys = r.read("keys_sorted")
    pr = {k: r.read(k) for k in ("proj0", "proj1", "proj2")}
    tiles = np.arange(T, dtype=np.uint32)
    ranges = np.stack([np.searchsorted(keys, tiles, "left"), np.searchsorted(keys, tiles, "right")], 1).astype(np.uint32)
    ranges[ranges[:, 0] == ranges[:, 1]] = 0
    bn = {"vals_sorted": r.read("vals_sorted"), "tile_ranges": ranges}
    v_out = r.read("v_out")
    t0 = time.perf_counter()
    fw = O.raster_fwd(pr, bn, W, H, bg)
    t1 = time.perf_counter()
    O.raster_bwd(pr, bn, fw, v_out, W, H, bg, scene.n, inv_gscale=1.0 / (3.0 * W * H))
    t2 = time.perf_counter()
    shr = fw["tile_ranges"].astype(np.int64)
    f_sweep = int(64 * (shr[:, 1] - shr[:, 0]).clip(min=0).sum())
    secs = (t1 - t0) + (t2 - t1)
    return {
        "value": f_sweep / secs / 1e9,
        "unit": "Gfrag/s",
        "cores": 1,
        "kind": "port",
        "sample": f"one full config-3 frame (F_sweep={f_sweep}): forward {t1 - t0:.2f} s + backward {t2 - t1:.2f} s "
                  "of the fp32 tiled CPU restatement (oracle/b2c_oracle.c), single thread",
        "cpu_model": _cpu_model(),
        "host_threads_available": os.cpu_count(),
    }


def _cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--splats", type=int, default=1_000_000)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--mode", type=int, default=1, help="backward: 1 = MFMA reduction, 0 = fp32 reduction")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU; --gpus {args.gpus} is not supported (the path would shard "
              "by screen tiles or by views, see DESIGN.md)", file=sys.stderr)
        sys.exit(2)

    from b2ctrain_amd import _native
    from b2ctrain_amd import scenes as S

    log(f"bench: generating config 3 ({args.splats} splats)")
    scene = S.config3(n=args.splats)
    W, H = scene.W, scene.H
    r = _native.Renderer(scene)
    rng = np.random.default_rng(7)
    bgs = [tuple(float(x) for x in rng.random(3)) for _ in range(args.warmup + args.steps)]

    log("bench: warmup")
    for k in range(args.warmup):
        r.step(mode=args.mode, bg=bgs[k], timed=True)
    r.sync()
    log("bench: timed steps")
    stages = []
    t0 = time.perf_counter()
    for k in range(args.steps):
        stages.append(r.step(mode=args.mode, bg=bgs[args.warmup + k], timed=True))
    r.sync()
    wall = time.perf_counter() - t0
    ms_per_step = wall * 1e3 / args.steps
    med = {k: float(np.median([s[k] for s in stages])) for k in stages[0]}
    mean = {k: float(np.mean([s[k] for s in stages])) for k in stages[0]}

    # fragment counts of the last step (deterministic lists)
    ranges = r.read("tile_ranges").astype(np.int64)
    keys = r.read("keys_sorted")
    tiles = np.arange(ranges.shape[0])
    first = np.searchsorted(keys, tiles, "left")
    f_sweep = int(64 * (ranges[:, 1] - first).clip(min=0).sum())
    info = r.info()
    tc = r.read("tile_count")
    n_ok = int((tc > 0).sum())
    t_fb = mean["forward_ms"] + mean["backward_ms"]
    gfrag = f_sweep / (t_fb * 1e-3) / 1e9

    # roofline: projection is the HBM-bound stage the metric prices; the dominant kernel is reported too
    proj_bytes = projection_bytes(scene.n, n_ok, 4 * 3 * scene.K)
    proj_gbs = proj_bytes / (mean["project_ms"] * 1e-3) / 1e9
    dominant = max(("forward_ms", "backward_ms", "loss_ms", "project_ms", "vjp_ms", "bin_ms"), key=lambda k: mean[k])
    roofline = {
        "kernel": "project_kernel + project_big_kernel (projection stage)",
        "bound": "hbm",
        "achieved": round(proj_gbs, 1),
        "peak": HBM_PEAK_GBS,
        "unit": "GB/s",
        "frac": round(proj_gbs / HBM_PEAK_GBS, 4),
        "traffic": None,
        "algorithmic_bytes": proj_bytes,
        "avg_launch_ms": round(mean["project_ms"], 4),
        "dominant_stage": dominant,
    }
    out = {
        "metric": METRIC,
        "value": round(gfrag, 3),
        "unit": "Gfrag/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic",
        "config": {
            "workload": "BASELINE config 3: 1M splats, SH3, 1920x1080, fused L1+SSIM (11-tap) + alpha lane, "
                        "per-pixel weights, elliptic alpha, random per-step background; MFMA backward; projection VJP",
            "splats": scene.n,
            "splats_projected": n_ok,
            "sh_degree": scene.degree,
            "width": W,
            "height": H,
            "isects": int(info.num_isect),
            "F_sweep": f_sweep,
            "backward": "mfma" if args.mode == 1 else "fp32",
            "parallelism": "single GPU",
        },
        "stages_ms_mean": {k: round(v, 4) for k, v in mean.items()},
        "stages_ms_median": {k: round(v, 4) for k, v in med.items()},
        "raster_fwd_bwd_ms": round(t_fb, 4),
        "roofline": roofline,
    }
    if not args.no_cpu_baseline:
        log("bench: CPU baseline (oracle port, one core)")
        r.step(mode=args.mode, bg=bgs[-1])
        r.sync()
        out["cpu_baseline"] = cpu_baseline(r, scene, bgs[-1])
    else:
        out["cpu_baseline"] = None
    r.close()
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
