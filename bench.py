"""Benchmark of the MI355X splat rasterizer on BASELINE.json's metric configuration (config 3).

One step = one training step of the hot path on one view, inputs resident in HBM: projection + binning/
sort + forward raster + fused L1/SSIM/alpha loss + MFMA backward + projection VJP (trainer.cpp:487-529
order, grad_out semantics). A new random background is drawn each step (trainer.cpp:470-471).

Prints ONE JSON line. value = Gfrag/s = F_sweep / (t_forward + t_backward), with F_sweep = the sum over
tiles of 64 x the tile's shrunk list length (the fragments the raster sweeps). Stage times come from hipEvents recorded on the
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


def binning_bytes(n, m, tile_bits):
    """Algorithmic bytes of binning: depth keys (read proj1 z + tile_count, write key/value), 4 depth-sort
    passes (16 B per splat each), the count scan in depth order (12 B per splat), the emit (20 B per splat +
    8 B per intersection), ceil(tile_bits / 8) tile-sort passes (24 B per intersection each: key and two
    values, read and written) and the range pass (4 B per intersection)."""
    tile_passes = (int(tile_bits) + 7) // 8
    return n * (8 + 8) + 4 * 16 * n + 12 * n + 20 * n + 8 * m + tile_passes * 24 * m + 4 * m


def read_traffic(kernel):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 PMC summary (FETCH_SIZE and WRITE_SIZE in
    KiB per dispatch, scaled by the plain-copy calibration recorded in the same file); None if absent."""
    path = os.path.join(ROOT, "profiles", f"{kernel}_cfg3_traffic.txt")
    if not os.path.exists(path):
        return None
    kv = {}
    for line in open(path):
        if ":" in line and not line.startswith("#"):
            k, v = line.split(":", 1)
            kv[k.strip()] = v.strip()
    try:
        fetch = float(kv["fetch_kib_per_dispatch"]) * float(kv["fetch_scale"])
        write = float(kv["write_kib_per_dispatch"]) * float(kv["write_scale"])
    except (KeyError, ValueError):
        return None
    return int((fetch + write) * 1024)


def cpu_baseline(r, scene, bg):
    """The CPU port (oracle, fp32 tiled restatement, one host core) timed on the same frame: forward raster
    + backward raster over the GPU's own tile lists and per-pixel loss gradient. Returns the frame's
    composited-fragment count (F_contrib) and the cpu_baseline record."""
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
    return fw["f_contrib"], {
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
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--splats", type=int, default=1_000_000)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--mode", type=int, default=1, help="backward: 1 = MFMA reduction, 0 = fp32 reduction")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a plain 256 MiB device-to-device copy (three times), the known-size kernel that "
                         "scales rocprofv3's FETCH_SIZE / WRITE_SIZE counters to bytes")
    args = ap.parse_args()
    if args.copy_calibration:
        import torch
        a = torch.ones(64 << 20, dtype=torch.float32, device="cuda")
        b = torch.empty_like(a)
        torch.cuda.synchronize()
        for _ in range(3):
            b.copy_(a)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes": a.numel() * 4, "copies": 3}), flush=True)
        return
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU; --gpus {args.gpus} is not supported (the path would shard "
              "by screen tiles or by views)", file=sys.stderr)
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
    # The timed region runs the steps as a training loop does: no per-stage events (reading them back
    # would drain the stream at the end of every step). The per-stage breakdown comes from a second pass
    # over the same backgrounds with hipEvents recorded on the context's stream.
    log("bench: timed steps")
    t0 = time.perf_counter()
    for k in range(args.steps):
        r.step(mode=args.mode, bg=bgs[args.warmup + k])
    r.sync()
    wall = time.perf_counter() - t0
    ms_per_step = wall * 1e3 / args.steps
    log("bench: per-stage events")
    stages = [r.step(mode=args.mode, bg=bgs[args.warmup + k], timed=True) for k in range(args.steps)]
    r.sync()
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

    # Roofline of the dominant kernel, the MFMA backward raster (raster_bwd_mfma_kernel), timed alone with
    # hipEvents on the context's stream. Algorithmic bytes per launch: per composited-range intersection its
    # list entry, emit position and projected splat (4 + 4 + 48 B) plus its gradient row (48 B, written);
    # per intersection past the shrunk end its zero row (48 B); per pixel out_rgba, out_feat, last_idx and
    # v_out (52 B). MFMA: 8 v_mfma_f32_16x16x32_f16 (16384 flop each) per group of 8 splats.
    m_shrunk = f_sweep // 64
    m_total = int(info.num_isect)
    bwd_bytes = 104 * m_shrunk + 48 * (m_total - m_shrunk) + 52 * W * H
    t_bwd = mean["raster_bwd_ms"] * 1e-3
    bwd_gbs = bwd_bytes / t_bwd / 1e9
    groups = int(np.ceil(m_shrunk / 8.0))
    mfma_tflops = groups * 8 * 16384 / t_bwd / 1e12
    traffic = read_traffic("raster_bwd_mfma_kernel")
    roofline = {
        "kernel": "raster_bwd_mfma_kernel",
        "bound": "hbm",
        "achieved": round(bwd_gbs, 1),
        "peak": HBM_PEAK_GBS,
        "unit": "GB/s",
        "frac": round(bwd_gbs / HBM_PEAK_GBS, 4),
        "traffic": traffic,
        "algorithmic_bytes": bwd_bytes,
        "avg_launch_ms": round(mean["raster_bwd_ms"], 4),
        "mfma": {"achieved": round(mfma_tflops, 1), "peak": MFMA_F16_PEAK_TFLOPS, "unit": "TFLOP/s",
                 "frac": round(mfma_tflops / MFMA_F16_PEAK_TFLOPS, 4)},
        "note": ("VALU-issue bound (per-fragment replay; rocprofv3 SQ_INSTS_VALU gives 91% of the VALU issue "
                 "slots, profiles/raster_step_cfg3_counters.md); HBM and MFMA fractions are low by design"),
    }
    # HBM rooflines of the stages the north star prices: projection, binning/sort, loss
    proj_bytes = projection_bytes(scene.n, n_ok, 4 * 3 * scene.K)
    bin_bytes = binning_bytes(scene.n, m_total, info.tile_bits)
    loss_bytes = 37 * W * H
    stage_rooflines = {}
    for name, nbytes, key in (("projection", proj_bytes, "project_ms"), ("binning_sort", bin_bytes, "bin_ms"),
                              ("loss", loss_bytes, "loss_ms")):
        gbs = nbytes / (mean[key] * 1e-3) / 1e9
        stage_rooflines[name] = {"bound": "hbm", "algorithmic_bytes": int(nbytes), "ms": round(mean[key], 4),
                                 "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                                 "frac": round(gbs / HBM_PEAK_GBS, 4)}
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
        # the step without the projection VJP, the reference's own timed subtotal
        "step_without_vjp_ms": round(mean["total_ms"] - mean["vjp_ms"], 4),
        "roofline": roofline,
        "stage_rooflines": stage_rooflines,
    }
    if not args.no_cpu_baseline:
        log("bench: CPU baseline (oracle port, one core)")
        r.step(mode=args.mode, bg=bgs[-1])
        r.sync()
        f_contrib, out["cpu_baseline"] = cpu_baseline(r, scene, bgs[-1])
        # composited fragments of that frame, counted by the CPU port over the GPU's own lists
        out["config"]["F_contrib"] = f_contrib
        out["gfrag_contrib_per_s"] = round(f_contrib / (t_fb * 1e-3) / 1e9, 3)
    else:
        out["cpu_baseline"] = None
    r.close()
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
