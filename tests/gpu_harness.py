"""Shared GPU-vs-oracle checks (imported by the gpu tests and by smoke-style scripts).

Each stage of the HIP path is compared with the CPU oracle fed the GPU's own upstream outputs, so a
mismatch names its stage. Tolerances:

* projection outputs, tile counts, hit info, depth order, count scan, tile key/value lists and tile
  ranges: bit-exact (integer / index work and the fp32 projection both sides evaluate identically);
* rendered RGBA: max abs error <= 1e-4 vs the fp32 oracle (the GPU uses the hardware exponential; observed
  ~2e-7 at config 1 and ~1e-5 over the long lists of config 3 at full size) at every pixel whose last
  composited fragment agrees; at most 1e-5 of the pixels may terminate one fragment apart (T (1 - alpha)
  within rounding of the 1e-4 stop: the render's non-smooth points, where the extra fragment's whole
  contribution differs);
* rendered RGBA against the double-precision brute force (the reference's tests/reference.cpp algorithm,
  oracle orc_ref_loss) directly: max abs error <= 1e-4 (check_rgba_fp64);
* loss value: relative 1e-4 (the kernel evaluates SSIM in fp32, where sigma^2 = E[x^2] - mu^2 cancels;
  the oracle in fp64); per-pixel gradient: <= LOSS_GRAD_TOL of the largest |v_out| everywhere except where
  the L1 term's sign flips, i.e. where the prediction equals the effective target to 1e-6 (the fp32 and
  fp64 evaluations of p - g may then round to opposite signs); the count above 1e-4 is reported;
* v_splat: <= 2e-3 of each lane's largest |value| (float atomics sum in arbitrary order; mode 1 reduces
  through fp16 hi/lo MFMA products), and per-entry relative error percentiles over the entries above
  1e-3 of their lane's maximum: 99th percentile <= 1e-3;
* parameter gradients from the GPU's own v_splat: <= 1e-3 of each column's largest |value| (two different
  derivations of the projection VJP, the kernel's from the semi-axis form and the oracle's restating the
  reference's world-covariance chain), and per-entry relative error percentiles as for v_splat;
* the side outputs the reference's refine pass reads (refine.cu:55-95): max_screen after the projection
  (project.cu:82-83) bit-exact, raised from a nonzero starting array; vis_weight after the backward
  (raster_bwd_tc.cu:177-195) at the v_splat bars, and conserved: its sum over splats equals the GPU
  image's accumulated alpha sum(1 - T_final) to 1e-4; vis_count and refine_norm after the VJP
  (optim.cu:113,122-124) bit-exact against the oracle's update of the same starting arrays from the GPU's
  own v_splat and vis_flag.
"""
from __future__ import annotations

import numpy as np

from b2ctrain_amd import _native
from oracle import oracle as O


def emit(msg):
    print(msg, flush=True)


def seed_side_outputs(r, n, seed=7):
    """Nonzero starting values for the per-splat statistics the hot path raises or adds to, so a check
    sees the running maximum / count and not only a first write."""
    rng = np.random.default_rng(seed)
    init = {}
    for k, hi in (("max_screen", 0.01), ("vis_count", 5.0), ("refine_norm", 1e-4)):
        a = rng.uniform(0.0, hi, n).astype(np.float32)
        if k == "vis_count":
            a = np.floor(a)
        a[::5] = 0.0
        r.write_model(k, a)
        init[k] = a
    return init


def check_max_screen(r, scene, camd, init):
    got = r.read_model("max_screen")
    want = O.max_screen(scene, camd, init)
    bad = got.view(np.uint32) != want.view(np.uint32)
    assert not bad.any(), f"max_screen differs for splats {np.flatnonzero(bad)[:10]}"
    raised = int((want > init).sum())
    emit(f"    max_screen bit-exact ({raised} of {scene.n} raised)")
    assert raised > 0 or scene.n == 0


def check_projection(r, scene, camd):
    pr = O.project(scene, camd)
    g = {k: r.read(k) for k in ("proj0", "proj1", "proj2", "proj3", "tile_count", "hit_info")}
    assert np.array_equal(g["tile_count"], pr["tile_count"]), \
        f"tile_count differs at {np.flatnonzero(g['tile_count'] != pr['tile_count'])[:10]}"
    ok = pr["tile_count"] > 0
    for k in ("proj0", "proj1", "proj2", "proj3"):  # proj2.w and proj3: the feature lanes
        a, b = g[k][ok], pr[k][ok]
        bad = ~((a == b) | (np.isnan(a) & np.isnan(b)))
        assert not bad.any(), f"{k} differs for splats {np.flatnonzero(ok)[np.flatnonzero(bad.any(1))[:10]]}"
    assert np.array_equal(g["hit_info"][ok], pr["hit_info"][ok]), "hit_info differs"
    # where the reference's mask word says "recompute", hit_wide holds the 64-bit mask of a bbox of at most 64
    # tiles (as many bits as hits) or (0, 0) beyond 64 tiles; the emitted lists check the bits' positions
    rec = ok & (pr["hit_info"][:, 0] == 0xFFFFFFFF)
    wide = r.read("hit_wide")[rec]
    bits = np.unpackbits(wide.view(np.uint8), axis=1).sum(1)
    none = (wide == 0).all(1)
    assert ((bits == pr["tile_count"][rec]) | none).all(), "hit_wide bit counts differ from tile_count"
    return {**pr, **{k: g[k] for k in g}}


def check_binning(r, pr, W, H):
    bn = O.bin_(pr, W, H)
    info = r.info()
    assert info.num_isect == bn["M"], (info.num_isect, bn["M"])
    for k in ("order", "tile_off", "keys_sorted", "vals_sorted", "tile_ranges"):
        g = r.read(k)
        assert np.array_equal(g, bn[k]), f"{k} differs at {np.flatnonzero((g != bn[k]).reshape(len(g), -1).any(1))[:10]}"
    return bn


def check_forward(r, pr, bn, W, H, bg, tol=1e-4, scene=None):
    feat = scene is not None and scene.feat_mode != 0
    hz = None if scene is None else scene.hollow_z
    fw = O.raster_fwd(pr, bn, W, H, bg, feat=feat, hollow_z=hz,
                      hollow_margin=0.05 if scene is None else scene.hollow_margin)
    rgba = r.read("out_rgba")
    of = r.read("out_feat")
    T = of[:, 3]
    last = r.read("last_idx")
    d = np.abs(rgba - fw["out_rgba"]).max(axis=1) if len(rgba) else np.zeros(0)
    # a termination flip: T (1 - alpha) lands within rounding of the 1e-4 stop on one side only, and one
    # side composites a fragment more (its whole contribution differs: a non-smooth point of the render)
    flip = last != fw["last_idx"]
    err = float(d[~flip].max()) if (~flip).any() else 0.0
    assert err <= tol, f"rgba max abs err {err} outside termination flips"
    assert flip.mean() <= 1e-5, f"last_idx mismatch fraction {flip.mean()}"
    if flip.any():
        emit(f"    {int(flip.sum())} termination flips of {len(last)} pixels (rgba differs by up to {float(d[flip].max()):.2e})")
    ranges = r.read("tile_ranges")
    rm = float((ranges != fw["tile_ranges"]).any(1).mean())
    assert rm <= 1e-3, f"shrunk tile range mismatch fraction {rm}"
    out = dict(out_rgba=rgba, out_T=T, last_idx=last, tile_ranges=ranges, err=err, out_feat4=of)
    if feat:  # the feature lanes composite like the colour (features are unit vectors or clamped to 100)
        fe = np.abs(of[:, :3] - fw["out_feat"]).max(axis=1)
        ferr = float(fe[~flip].max()) if (~flip).any() else 0.0
        emit(f"    out_feat max abs err {ferr:.2e}")
        assert ferr <= tol, f"out_feat max abs err {ferr}"
    if hz is not None:
        pen = r.read("hollow_pen")
        pe = np.abs(pen - fw["hollow_pen"])
        perr = float(pe[~flip].max()) if (~flip).any() else 0.0
        emit(f"    hollow_pen max abs err {perr:.2e}")
        assert perr <= tol, f"hollow_pen max abs err {perr}"
        out["hollow_pen"] = pen
    return out


# Per-entry bound on v_out relative to its largest entry. The fp32 SSIM statistics (sigma^2 = E[x^2] -
# mu^2 over 11x11 windows) cancel in nearly flat windows: observed worst 6.1e-4 at 1080p (135 of 8.3M
# entries above 1e-4).
LOSS_GRAD_TOL = 1e-3


def effective_target(scene, bg):
    """The loss's per-channel target (rgb composited over bg for transparent views, and alpha)."""
    g = np.ascontiguousarray(scene.gt, np.uint32)
    ch = np.stack([(g >> np.uint32(8 * k)) & np.uint32(0xFF) for k in range(4)], 1).astype(np.float32) / np.float32(255)
    if scene.composite:
        ch[:, :3] += (1 - ch[:, 3:4]) * np.asarray(bg, np.float32)[None, :]
    return ch


def rel_percentiles(got, ref, floor_frac=1e-3):
    """Per-entry relative error over the entries whose |ref| exceeds floor_frac of their column's max."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    col = np.abs(ref).max(axis=0, keepdims=True)
    sel = np.abs(ref) > floor_frac * col
    if not sel.any():
        return dict(p50=0.0, p99=0.0, max=0.0, n=0)
    rel = np.abs(got - ref)[sel] / np.abs(ref)[sel]
    return dict(p50=float(np.percentile(rel, 50)), p99=float(np.percentile(rel, 99)), max=float(rel.max()),
                n=int(sel.sum()))


def check_rgba_fp64(rgba, scene, bg, tol=1e-4):
    """GPU image against the double-precision brute-force render (every splat, every pixel, no tiles)."""
    _, img = O.ref_loss(scene, bg=bg, want_img=True)
    err = float(np.abs(np.asarray(rgba, np.float64) - img).max())
    assert err <= tol, f"rgba vs fp64 brute force: max abs err {err:.3e}"
    return err


def check_loss(r, scene, rgba, grad_scale, bg):
    loss = r.loss(grad_scale=grad_scale, bg=bg)
    ref, v_ref = O.photometric(scene, rgba, grad_scale=grad_scale, bg=bg)
    assert abs(loss - ref) <= 1e-4 * abs(ref) + 1e-9, f"loss {loss} vs oracle {ref}"
    v = r.read("v_out")
    scale = float(np.abs(v_ref).max()) + 1e-30
    diff = np.abs(v - v_ref) / scale
    flip = np.abs(np.asarray(rgba, np.float32) - effective_target(scene, bg)) < 1e-6
    worst = float(np.where(flip, 0.0, diff).max()) if diff.size else 0.0
    emit(f"    v_out: worst {worst:.2e} of max outside {int((flip & (diff > LOSS_GRAD_TOL)).sum())} L1 sign flips; "
         f"{int((diff > 1e-4).sum())} of {diff.size} entries above 1e-4")
    assert worst <= LOSS_GRAD_TOL, f"v_out: worst error {worst:.2e} of the largest gradient beyond L1 sign flips"
    return loss, v


def check_aux_losses(r, scene, fw, grad_scale):
    """normal_loss (v_feat bit for bit and the loss against the oracle fed the GPU's out_feat) and
    hollow_loss (lam times the oracle's sum of the GPU's per-pixel penalties). Returns the GPU v_feat."""
    W, H = scene.W, scene.H
    v_feat = None
    if scene.feat_mode == 1 and scene.normals is not None and scene.normal_scale > 0:
        before = float(r.read("loss_accum")[1])
        r.normal_loss(grad_scale=grad_scale)
        got = float(r.read("loss_accum")[1]) - before
        ref, v_ref = O.normal_loss(W, H, fw["out_feat4"], scene.normals, scene.weights, scene.normal_scale, grad_scale)
        v_feat = r.read("v_feat")
        assert abs(got - ref) <= 1e-6 * abs(ref) + 1e-9, f"normal loss {got} vs oracle {ref}"
        assert np.array_equal(v_feat.view(np.uint32), v_ref.view(np.uint32)), \
            f"v_feat differs at {np.flatnonzero((v_feat != v_ref).any(1))[:10]}"
        emit(f"    normal loss {got:.6g} (oracle {ref:.6g}), v_feat bit-exact")
    elif scene.feat_mode:
        v_feat = r.read("v_feat")
    if scene.hollow_z is not None:
        before = float(r.read("loss_accum")[0])
        r.hollow_loss()
        got = float(r.read("loss_accum")[0]) - before
        ref = scene.hollow_lam * O.hollow_sum(fw["hollow_pen"])
        assert abs(got - ref) <= 1e-5 * abs(ref) + 1e-9, f"hollow loss {got} vs oracle {ref}"
        emit(f"    hollow loss {got:.6g} (oracle {ref:.6g})")
    return v_feat


def check_vis_weight(got, ref, out_T):
    """vis_weight against the oracle's at the v_splat bars, and its conservation on the GPU's own image."""
    scale = float(np.abs(ref).max()) + 1e-30
    worst = float((np.abs(got - ref) / scale).max()) if got.size else 0.0
    pc = rel_percentiles(got[:, None], ref[:, None])
    total = float(np.asarray(got, np.float64).sum())
    alpha = float((1.0 - np.asarray(out_T, np.float64)).sum())
    emit(f"    vis_weight max err {worst:.2e} of max; rel p99 {pc['p99']:.1e}; sum {total:.6g} vs image alpha {alpha:.6g}")
    assert worst <= 2e-3, f"vis_weight: worst error {worst:.2e} of the largest"
    assert pc["p99"] <= 1e-3, f"vis_weight per-entry 99th percentile rel err {pc['p99']:.2e}"
    assert abs(total - alpha) <= 1e-4 * alpha + 1e-6, f"vis_weight sums to {total}, the image's alpha to {alpha}"


def check_backward(r, scene, pr, bn, fw, v_out, W, H, bg, mode, grad_scale, v_feat=None):
    r.zero("v_splat")
    r.zero("vis_flag")
    r.write_model("vis_weight", np.zeros(scene.n, np.float32))
    r.backward(mode=mode, grad_scale=grad_scale)
    vs = r.read("v_splat")
    vf = r.read("vis_flag")
    vw = r.read_model("vis_weight")
    inv = 1.0 / grad_scale if mode == 1 else 1.0
    ref_vs, ref_vf, ref_vw = O.raster_bwd(pr, bn, dict(tile_ranges=fw["tile_ranges"], out_rgba=fw["out_rgba"],
                                                  out_T=fw["out_T"], last_idx=fw["last_idx"]), v_out, W, H, bg,
                                     scene.n, inv_gscale=inv, v_feat=v_feat if scene.feat_mode else None,
                                     hollow_z=scene.hollow_z, hollow_margin=scene.hollow_margin,
                                     hollow_lam=scene.hollow_lam * grad_scale)
    assert np.array_equal(vf, ref_vf), f"vis_flag differs for {np.flatnonzero(vf != ref_vf)[:10]}"
    lane_scale = np.abs(ref_vs).max(axis=0) + 1e-30
    err = np.abs(vs - ref_vs) / lane_scale
    worst = float(err.max()) if err.size else 0.0
    assert worst <= 2e-3, f"v_splat mode {mode}: worst lane-relative err {worst:.2e} at lane {int(err.max(0).argmax())}"
    lanes = 13 if scene.feat_mode else 10
    pc = rel_percentiles(vs[:, :lanes], ref_vs[:, :lanes])
    emit(f"    v_splat lane-max err {worst:.2e}; per-entry rel p50 {pc['p50']:.1e} p99 {pc['p99']:.1e} "
         f"max {pc['max']:.1e} over {pc['n']}")
    assert pc["p99"] <= 1e-3, f"v_splat per-entry 99th percentile rel err {pc['p99']:.2e}"
    check_vis_weight(vw, ref_vw, fw["out_T"])
    return vs, vf, worst


def check_vjp(r, scene, camd, vs, vf, tile_count, init=None):
    r.vjp()
    g = r.read("grads")
    if init is not None:  # the refine statistics, from the same v_splat and flags (optim.cu:113,122-124)
        vc, rn = O.refine_stats(vs, vf, tile_count, init["vis_count"], init["refine_norm"])
        for k, want in (("vis_count", vc), ("refine_norm", rn)):
            got = r.read_model(k)
            bad = got.view(np.uint32) != want.view(np.uint32)
            assert not bad.any(), f"{k} differs for splats {np.flatnonzero(bad)[:10]}"
        emit(f"    vis_count / refine_norm bit-exact ({int((vc > init['vis_count']).sum())} splats visible)")
    ref = O.vjp(scene, camd, vs, vf, tile_count)
    col = np.abs(ref).max(axis=0) + 1e-30
    rel = np.abs(g - ref) / col
    err = float(rel.max())
    if err > 1e-3:
        i, k = np.unravel_index(int(rel.argmax()), rel.shape)
        raise AssertionError(f"grads vs oracle VJP (same v_splat): {err:.2e} at splat {i} column {k}: "
                             f"gpu {g[i, k]:.6g} oracle {ref[i, k]:.6g} column max {col[k]:.3g}")
    pc = rel_percentiles(g, ref)
    emit(f"    grads column-max err {err:.2e}; per-entry rel p50 {pc['p50']:.1e} p99 {pc['p99']:.1e} "
         f"max {pc['max']:.1e} over {pc['n']}")
    assert pc["p99"] <= 1e-3, f"grads per-entry 99th percentile rel err {pc['p99']:.2e}"
    assert not r.read("vis_flag").any(), "vis_flag not cleared by the VJP"
    assert not r.read("v_splat").any(), "v_splat not cleared by the VJP"
    return g


def full_check(scene, mode=1, bg=None, loss=True, backward=True, fp64_rgba=False):
    """Run every stage on the GPU and check it; returns a dict of GPU outputs. fp64_rgba also checks the
    image directly against the double-precision brute force (small scenes: it visits every splat per
    pixel)."""
    bg = scene.bg if bg is None else bg
    W, H = scene.W, scene.H
    gs = 3.0 * W * H if mode == 1 else 1.0
    r = _native.Renderer(scene)
    try:
        camd = _native.camera_gpu_from(scene.cam)
        init = seed_side_outputs(r, scene.n)
        emit(f"  [{scene.name}] projection")
        r.project(bg=bg)
        pr = check_projection(r, scene, camd)
        check_max_screen(r, scene, camd, init["max_screen"])
        emit(f"  [{scene.name}] binning")
        r.bin()
        bn = check_binning(r, pr, W, H)
        emit(f"  [{scene.name}] forward (M={bn['M']})")
        r.raster_fwd(bg=bg)
        fw = check_forward(r, pr, bn, W, H, bg, scene=scene)
        out = dict(M=bn["M"], rgba_err=fw["err"])
        if fp64_rgba:
            out["rgba_err64"] = check_rgba_fp64(fw["out_rgba"], scene, bg)
            emit(f"    rgba vs fp64 brute force {out['rgba_err64']:.2e}")
        if loss:
            emit(f"  [{scene.name}] loss")
            out["loss"], v = check_loss(r, scene, fw["out_rgba"], gs, bg)
            v_feat = check_aux_losses(r, scene, fw, gs)
            if backward:
                emit(f"  [{scene.name}] backward mode {mode}")
                vs, vf, out["v_splat_err"] = check_backward(r, scene, pr, bn, fw, v, W, H, bg, mode, gs, v_feat)
                emit(f"  [{scene.name}] vjp")
                out["grads"] = check_vjp(r, scene, camd, vs, vf, pr["tile_count"], init)
        return out
    finally:
        r.close()
