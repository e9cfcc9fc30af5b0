"""Benchmark of the MI355X splat rasterizer on BASELINE.json's metric configuration (config 3 by default).

One step = one training step of the hot path, inputs resident in HBM: projection + binning/sort + forward
raster + fused L1/SSIM/alpha loss + MFMA backward + projection VJP (the order of trainer.cpp:487-529, grad_out
semantics), on every view of the configuration (config 4: 8 camera poses, gradients accumulated over them).
A new random background is drawn each step (trainer.cpp:470-471).

Prints ONE JSON line. value = Gfrag/s = F_sweep / (t_forward + t_backward), with F_sweep = the sum over
tiles of 64 x the tile's shrunk list length (the fragments both raster passes sweep), summed over the views.
Stage times come from hipEvents recorded on the context's stream around each stage; ms_per_step is the wall
time of the K timed steps over K, bracketed by stream synchronisation.

training_iteration reports a complete training iteration besides: the same step ending in the fused Adam /
lazy sparse Adam / MCMC update instead of the gradient export (dense and sparse), with the update kernel's
HBM roofline.

Two CPU baselines are timed on this host (not the optimisation target):
* cpu_baseline: the fp32 tiled CPU restatement (oracle/b2c_oracle.c) of the whole step (projection, binning,
  forward, loss, backward, VJP) on one frame, the raster passes OpenMP over tiles on the host threads this
  process may use;
* cpu_reference_algorithm: the reference's own CPU algorithm (tests/reference.cpp:34-143 restated: fp64,
  every depth-sorted splat tested at every pixel, one thread) on a bounded sample of pixels spread over the
  frame, extrapolated to the whole frame.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "raster fwd+bwd ms/step @1M splats 1080p; Gfrag/s; % HBM roofline"
HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0

WORKLOADS = {
    1: "BASELINE config 1: 1,024 splats, SH0, 64x64, fused L1+SSIM",
    2: "BASELINE config 2: 100k splats, SH3, 800x800, fused L1+SSIM",
    3: "BASELINE config 3: 1M splats, SH3, 1920x1080, fused L1+SSIM (11-tap) + alpha lane, per-pixel weights, "
       "elliptic alpha, random per-step background; MFMA backward; projection VJP",
    4: "BASELINE config 4: 3M splats, SH4, 1920x1080 slab (~190 composited fragments/px), 8 camera poses per step "
       "with gradients accumulated",
    5: "BASELINE config 5: 500k splats, 3840x2160, SH3 with fp16 bands, 5% huge anisotropic splats",
}
DEFAULT_SPLATS = {1: 1024, 2: 100_000, 3: 1_000_000, 4: 3_000_000, 5: 500_000}


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def projection_bytes(n, n_ok, sh_bytes):
    """All splats: pos_op + quat + lscale (48 B) and tile_count (4 B); splats that pass: SH coefficients,
    proj0..2 (48 B), proj3 (8 B), hit_info (8 B), max_screen read + write (8 B)."""
    return n * 52 + n_ok * (sh_bytes + 72)


def binning_bytes(n, m, tile_bits):
    """The survey's algorithmic bytes for the sorts, scan and emit (independent of this design's extra
    passes): 4 depth-sort passes of 16 B per splat, ceil(tile_bits / 8) tile-sort passes of 16 B per
    intersection, the count scan (8 B per splat) and the emit (20 B per splat + 8 B per intersection)."""
    return 4 * 16 * n + ((int(tile_bits) + 7) // 8) * 16 * m + 8 * n + 20 * n + 8 * m


def update_bytes(n, sh_bytes):
    """The fused optimizer's algorithmic bytes over n splats, dense mode: per splat the 13 v_splat lanes,
    vis_flag, tile_count, vis_count and refine_norm are read (68 B); the parameters (48 B), their moments
    (96 B), the SH and their first moments (2 S) and v_sh (4 B) are read and written; v_splat, vis_flag,
    vis_count and refine_norm are written back (64 B). Reads of the SH by the VJP itself are not counted
    again."""
    rw = 48 + 96 + 2 * sh_bytes + 4
    return n * (68 + 2 * rw + 64)


def read_traffic(kernel, config):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 PMC summary (FETCH_SIZE and WRITE_SIZE in
    KiB per dispatch, scaled by the plain-copy calibration recorded in the same file); None if absent."""
    path = os.path.join(ROOT, "profiles", f"{kernel}_cfg{config}_traffic.txt")
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


def cpu_info():
    model, logical = "unknown", os.cpu_count()
    fields = {}
    try:
        for line in open("/proc/cpuinfo"):
            if ":" in line:
                k, v = (x.strip() for x in line.split(":", 1))
                fields.setdefault(k, v)
    except OSError:
        pass
    model = fields.get("model name", model)
    # AMD's family numbers name the core generation where the model string does not (virtual machines
    # often report only "AMD EPYC"): 0x19 Zen 3/4, 0x1A Zen 5
    uarch = {("AuthenticAMD", "25"): "Zen 3 / Zen 4 (family 19h)",
             ("AuthenticAMD", "26"): "Zen 5 (family 1Ah: EPYC 9005)"}.get((fields.get("vendor_id"), fields.get("cpu family")))
    return {"cpu_model": model, "cpu_vendor": fields.get("vendor_id"), "cpu_family": fields.get("cpu family"),
            "cpu_model_id": fields.get("model"), "cpu_microarchitecture": uarch, "host_logical_cpus": logical,
            "host_cpus_usable": len(os.sched_getaffinity(0))}


def host_threads():
    env = os.environ.get("OMP_NUM_THREADS")
    if env and env.isdigit() and int(env) > 0:
        return int(env)
    return len(os.sched_getaffinity(0))


def f_sweep_of(r):
    ranges = r.read("tile_ranges").astype(np.int64)
    return int(64 * (ranges[:, 1] - ranges[:, 0]).clip(min=0).sum())


def kept_of(r):
    """Entries of the forward's compacted lists (the ones some pixel composited), which the MFMA backward
    walks."""
    ranges = r.read("tile_ranges").astype(np.int64)
    return int((r.read("cend").astype(np.int64) - ranges[:, 0]).clip(min=0).sum())


def cpu_baseline_frame(r, scene, mode, bg, cam):
    """Both CPU baselines on one frame of the benchmark's own training step: (F_sweep, cpu_baselines(...))."""
    r.step(mode=mode, bg=bg, cam=cam)
    r.project(cam=cam, bg=bg)  # the step leaves proj0..3 unwritten; the CPU legs read them
    r.sync()
    f_sweep = f_sweep_of(r)
    return f_sweep, cpu_baselines(r, scene.with_camera(cam), bg, f_sweep)


def cpu_baselines(r, scene, bg, f_sweep):
    """Both CPU baselines on the frame the context last rendered (one view, the step's camera and bg)."""
    from b2ctrain_amd.scenes import camera_gpu
    from oracle import oracle as O

    W, H = scene.W, scene.H
    camd = camera_gpu(scene.cam)
    gs = 3.0 * W * H
    threads = host_threads()
    O.set_threads(threads)
    try:  # the whole tiled step of the fp32 CPU restatement, stage by stage, from the scene itself
        t = [time.perf_counter()]
        pr = O.project(scene, camd)
        t.append(time.perf_counter())
        bn = O.bin_(pr, W, H)
        t.append(time.perf_counter())
        fw = O.raster_fwd(pr, bn, W, H, bg)
        t.append(time.perf_counter())
        _, v_out = O.photometric(scene, fw["out_rgba"], grad_scale=gs, bg=bg)
        t.append(time.perf_counter())
        vs, vf, _ = O.raster_bwd(pr, bn, fw, v_out, W, H, bg, scene.n, inv_gscale=1.0 / gs)
        t.append(time.perf_counter())
        O.vjp(scene, camd, vs, vf, pr["tile_count"])
        t.append(time.perf_counter())
    finally:
        O.set_threads(1)
    sec = dict(zip(("project", "bin", "forward", "loss", "backward", "vjp"), np.diff(t)))
    f_sweep_cpu = int(64 * (fw["tile_ranges"][:, 1].astype(np.int64) - fw["tile_ranges"][:, 0]).clip(min=0).sum())
    tiled = {
        "value": round(f_sweep_cpu / (sec["forward"] + sec["backward"]) / 1e9, 4),
        "unit": "Gfrag/s",
        "cores": threads,
        "kind": "port",
        "sample": f"one full frame of the workload (F_sweep={f_sweep_cpu}, the GPU's {f_sweep}): the whole tiled "
                  f"step of the fp32 CPU restatement (oracle/b2c_oracle.c) from the scene: projection, binning "
                  f"and sorts, forward, fused loss, backward, projection VJP; the forward and backward OpenMP over "
                  f"tiles on {threads} host threads, the other stages on one; value = F_sweep / (forward + "
                  f"backward) as the GPU's",
        "stage_seconds": {k: round(v, 3) for k, v in sec.items()},
        "step_seconds": round(sum(sec.values()), 3),
        **cpu_info(),
    }
    # the reference's CPU algorithm: fp64 brute force, one thread, ~400 pixels spread over the frame
    P = W * H
    stride = max(2, P // 400)
    n_sample = (P + stride - 1) // stride
    secs = O.ref_render_sample_seconds(scene, stride, bg=bg)
    frame_s = secs * P / n_sample
    ref = {
        "value": f_sweep / frame_s / 1e9,
        "unit": "Gfrag/s",
        "cores": 1,
        "kind": "port",
        "sample": f"{n_sample} pixels (every {stride}th, row-major) of one frame rendered by the reference's CPU "
                  f"algorithm (tests/reference.cpp:34-143 restated in oracle/b2c_oracle.c: fp64, every depth-sorted "
                  f"splat tested at every pixel) in {secs:.1f} s on one thread; whole frame extrapolated to "
                  f"{frame_s:.0f} s",
        "frame_seconds": round(frame_s, 1),
    }
    return fw["f_contrib"], tiled, ref


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--config", type=int, default=3, choices=sorted(WORKLOADS))
    ap.add_argument("--splats", type=int, default=None)
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

    cfg = args.config
    n = args.splats or DEFAULT_SPLATS[cfg]
    log(f"bench: generating config {cfg} ({n} splats)")
    scene = S.config1() if cfg == 1 else S.CONFIGS[cfg](n=n)
    views = scene.extra_cams or [scene.cam]
    W, H = scene.W, scene.H
    r = _native.Renderer(scene)
    rng = np.random.default_rng(7)
    bgs = [tuple(float(x) for x in rng.random(3)) for _ in range(args.warmup + args.steps)]

    def step(k, timed=False):
        st = None
        for v, cam in enumerate(views):
            t = r.step(mode=args.mode, bg=bgs[k], cam=cam, accumulate=v > 0, timed=timed)
            if timed:
                st = t if st is None else {key: st[key] + t[key] for key in st}
        return st

    log("bench: warmup")
    for k in range(args.warmup):
        step(k, timed=True)
    r.sync()
    # The timed region runs the steps as a training loop does: no per-stage events (reading them back
    # would drain the stream at the end of every view). The per-stage breakdown comes from a second pass
    # over the same backgrounds with hipEvents recorded on the context's stream.
    log("bench: timed steps")
    t0 = time.perf_counter()
    for k in range(args.steps):
        step(args.warmup + k)
    r.sync()
    wall = time.perf_counter() - t0
    ms_per_step = wall * 1e3 / args.steps
    log("bench: per-stage events")
    stages = [step(args.warmup + k, timed=True) for k in range(args.steps)]
    r.sync()
    med = {k: float(np.median([s[k] for s in stages])) for k in stages[0]}
    mean = {k: float(np.mean([s[k] for s in stages])) for k in stages[0]}

    # fragment and intersection counts of one more step, view by view (deterministic lists)
    f_sweep = m_total = n_ok = m_kept = 0
    tile_bits = 0
    for v, cam in enumerate(views):
        r.step(mode=args.mode, bg=bgs[-1], cam=cam, accumulate=v > 0)
        f_sweep += f_sweep_of(r)
        m_kept += kept_of(r)
        info = r.info()
        m_total += int(info.num_isect)
        tile_bits = int(info.tile_bits)
        n_ok += int((r.read("tile_count") > 0).sum())
    t_fb = mean["forward_ms"] + mean["backward_ms"]
    gfrag = f_sweep / (t_fb * 1e-3) / 1e9

    # Roofline of the dominant kernel, the MFMA backward raster (raster_bwd_mfma_kernel), timed alone with
    # hipEvents on the context's stream. It walks the forward's compacted lists (the shrunk-range entries some
    # pixel composited). Algorithmic bytes per launch: per walked entry its splat id, emit position and
    # projected splat (4 + 4 + 48 B) plus its gradient row (48 B, written); per pixel out_rgba, out_feat, its
    # list end and v_out (52 B). MFMA: 8 v_mfma_f32_16x16x32_f16 (16384 flop each) per group of 8 splats.
    m_shrunk = f_sweep // 64
    nv = len(views)
    bwd_bytes = 104 * m_kept + 52 * W * H * nv
    t_bwd = mean["raster_bwd_ms"] * 1e-3
    bwd_gbs = bwd_bytes / t_bwd / 1e9
    mfma_tflops = math.ceil(m_kept / 8.0) * 8 * 16384 / t_bwd / 1e12
    roofline = {
        "kernel": "raster_bwd_mfma_kernel",
        "bound": "valu",
        "achieved": round(bwd_gbs, 1),
        "peak": HBM_PEAK_GBS,
        "unit": "GB/s",
        "frac": round(bwd_gbs / HBM_PEAK_GBS, 4),
        "traffic": read_traffic("raster_bwd_mfma_kernel", cfg),
        "algorithmic_bytes": bwd_bytes,
        "avg_launch_ms": round(mean["raster_bwd_ms"] / nv, 4),
        "mfma": {"achieved": round(mfma_tflops, 1), "peak": MFMA_F16_PEAK_TFLOPS, "unit": "TFLOP/s",
                 "frac": round(mfma_tflops / MFMA_F16_PEAK_TFLOPS, 4)},
        "note": ("the per-fragment replay issues VALU instructions in most cycles (rocprofv3 SQ_INSTS_VALU, "
                 "profiles/raster_step_cfg3_counters.md): the kernel is bound by VALU issue; achieved/peak/frac "
                 "are its algorithmic HBM bytes against 8 TB/s and the mfma entry its matrix-core rate"),
    }
    sh_bytes = 4 * 3 + (2 if scene.sh_fp16 else 4) * 3 * (scene.K - 1)
    stage_rooflines = {}
    for name, nbytes, key in (("projection", projection_bytes(scene.n * nv, n_ok, sh_bytes), "project_ms"),
                              ("binning_sort", binning_bytes(scene.n * nv, m_total, tile_bits), "bin_ms"),
                              ("loss", 37 * W * H * nv, "loss_ms")):
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
            "workload": WORKLOADS[cfg],
            "splats": scene.n,
            "views_per_step": nv,
            "splats_projected": n_ok,
            "sh_degree": scene.degree,
            "width": W,
            "height": H,
            "isects": m_total,
            "F_sweep": f_sweep,
            "bwd_entries": m_kept,
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
        log("bench: CPU baselines (tiled port on all host threads; reference algorithm on a pixel sample)")
        fs0, (f_contrib, out["cpu_baseline"], out["cpu_reference_algorithm"]) = cpu_baseline_frame(
            r, scene, args.mode, bgs[-1], views[0])
        # composited fragments of that frame, counted by the CPU port (its lists equal the GPU's), and the rate
        # of composited fragments through the forward and backward (F_contrib / (t_fwd + t_bwd), one view)
        out["config"]["F_contrib_view0"] = f_contrib
        if nv == 1:
            out["contrib_gfrag_per_s"] = round(f_contrib / (t_fb * 1e-3) / 1e9, 3)
    else:
        out["cpu_baseline"] = None
    # A complete training iteration: the same step ending in the fused Adam / MCMC update instead of the
    # gradient export (b2c_train_step_adam, one update per view as the reference's trainer takes them),
    # with the reference trainer's defaults (lr_mean 2e-5, noise weight lr_mean * 50). Dense, then sparse.
    sh_mom = 4 * 3 + (2 if scene.sh_fp16 else 4) * 3 * (scene.K - 1)
    upd = {}
    for sparse in (False, True):
        opts = _native.adam_opts(t=0, sparse=int(sparse), lr_mean=2e-5, noise_weight=1e-3, noise_clamp=0.01,
                                 seed=7)
        times = []
        log(f"bench: training iterations with the fused update ({'sparse' if sparse else 'dense'})")
        for k in range(args.warmup + min(args.steps, 30)):
            opts.step = k
            for cam in views:
                t = r.step_adam(opts, mode=args.mode, bg=bgs[k % len(bgs)], cam=cam, timed=True)
                if k >= args.warmup:
                    times.append(t)
        um = {key: float(np.mean([t[key] for t in times])) for key in times[0]}
        upd["sparse" if sparse else "dense"] = {"iteration_ms": round(um["total_ms"] * nv, 4),
                                                "vjp_update_ms": round(um["vjp_ms"], 4)}
    ub = update_bytes(scene.n, sh_mom)
    t_upd = upd["dense"]["vjp_update_ms"] * 1e-3
    upd["dense"]["roofline"] = {"kernel": "vjp_kernel (update mode)", "bound": "hbm",
                                "algorithmic_bytes": ub, "achieved": round(ub / t_upd / 1e9, 1),
                                "peak": HBM_PEAK_GBS, "unit": "GB/s",
                                "frac": round(ub / t_upd / 1e9 / HBM_PEAK_GBS, 4)}
    out["training_iteration"] = upd
    # The tile-list replays on the first view: compute_evidence with the label vote (a class plane of
    # 64x64-pixel blocks) and probe_depth, as wall time of the synchronous calls (the evidence call renders
    # the view itself, as the reference's does). Kernel durations are in the rocprofv3 summaries.
    log("bench: evidence and probe replays")
    pix = np.arange(W * H)
    labels = (((pix % W) // 64 + 3 * ((pix // W) // 64)) % 29).astype(np.uint8)
    view = _native.View(W, H, scene.gt, scene.weights, labels=labels, has_alpha=True, masked=False)
    ev_t, pr_t = [], []
    for k in range(8):
        t0 = time.perf_counter()
        r.compute_evidence([view], [views[0]], export_labels=True, download=False)
        ev_t.append(time.perf_counter() - t0)
    r.forward(bg=(0.0, 0.0, 0.0), cam=views[0])
    r.sync()
    for k in range(8):
        t0 = time.perf_counter()
        r.probe_depth(0.5, 0.1)
        pr_t.append(time.perf_counter() - t0)
    view.close()
    out["replays"] = {"evidence_view_ms": round(float(np.median(ev_t[2:])) * 1e3, 4),
                      "probe_ms": round(float(np.median(pr_t[2:])) * 1e3, 4),
                      "note": "median wall time of the synchronous calls; evidence includes rendering the view, "
                              "probe includes allocating and downloading its [P][4] output"}
    r.close()
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
