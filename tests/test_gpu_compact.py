"""The forward's compacted lists and the MFMA backward over them. The reference's tensor-core backward walks
every entry of each tile's shrunk range (src/gpu/raster_bwd_tc.cu:29-225); the entries no pixel of the tile
composited have alpha = 0 there and give zero rows. This build's forward also writes each tile's list of the
entries some pixel composited (cvals / cslots / cend) and each pixel's end in it (clast), and the backward walks
that list instead (no reference counterpart; B2C_COMPACT_LISTS=0 turns it off).

* The lists are exactly the composited entries: recomputed here from the GPU's own sorted lists, projection
  and per-pixel ends (last_idx) with the oracle's fragment sigma (the raster kernels' float ops), an entry is
  kept when some pixel inside the image has it before its end with sigma <= power.
* The gradients over the compacted lists equal those over the full ranges: the left-out entries change
  neither a pixel's transmittance nor its running colour sum (alpha = 0), and their zero rows sum to the same
  per-splat totals (compared as values, so a zero's sign may differ).
"""
import numpy as np
import pytest

from b2ctrain_amd import _native
from b2ctrain_amd import scenes as S
from oracle import oracle as O
from tests.gpu_harness import emit

pytestmark = pytest.mark.gpu


def _expected_lists(r, sc):
    W, H = sc.W, sc.H
    tx = (W + 7) // 8
    ranges = r.read("tile_ranges").astype(np.int64)
    keys, vals, slots = r.read("keys_sorted"), r.read("vals_sorted"), r.read("slot_sorted")
    last = r.read("last_idx").astype(np.int64)
    p0, p1 = r.read("proj0"), r.read("proj1")
    M = keys.size
    e = np.arange(M)
    tile = keys.astype(np.int64)
    # entries inside their tile's shrunk range
    inr = (e >= ranges[tile, 0]) & (e < ranges[tile, 1])
    e, tile = e[inr], tile[inr]
    ids = vals[e]
    lx, ly = np.arange(64) % 8, np.arange(64) // 8
    px = (tile % tx)[:, None] * 8 + lx[None, :]
    py = (tile // tx)[:, None] * 8 + ly[None, :]
    inside = (px < W) & (py < H)
    pix = np.where(inside, py * W + px, 0)
    sig = O.frag_sigma(p0[ids, 0][:, None], p0[ids, 1][:, None], p0[ids, 2][:, None], p0[ids, 3][:, None],
                       p1[ids, 0][:, None], (px + 0.5).astype(np.float32), (py + 0.5).astype(np.float32))
    comp = inside & (e[:, None] < last[pix]) & (sig <= p1[ids, 3].astype(np.float32)[:, None])
    kept = comp.any(1)
    return dict(ranges=ranges, e=e[kept], tile=tile[kept], ids=ids[kept], slots=slots[e[kept]], last=last,
                n_entries=int(inr.sum()))


@pytest.mark.parametrize("masked", [False, True])
def test_compacted_lists_hold_the_composited_entries(masked):
    sc = S.config3(n=20_000, masked=masked)
    emit(f"compacted lists, masked={masked}")
    r = _native.Renderer(sc)
    try:
        r.forward()
        want = _expected_lists(r, sc)
        cvals, cslots, clast, cend = (r.read(k) for k in ("cvals", "cslots", "clast", "cend"))
    finally:
        r.close()
    ranges, tile = want["ranges"], want["tile"]
    n_t = ranges.shape[0]
    counts = np.bincount(tile, minlength=n_t)
    assert np.array_equal(cend.astype(np.int64), ranges[:, 0] + counts)
    # kept entries in list order: the k-th kept entry of tile t sits at ranges[t, 0] + k
    order = np.argsort(want["e"], kind="stable")
    t_sorted = tile[order]
    first = np.r_[0, np.cumsum(counts)[:-1]]
    pos = ranges[t_sorted, 0] + (np.arange(order.size) - first[t_sorted])
    assert np.array_equal(cvals[pos], want["ids"][order])
    assert np.array_equal(cslots[pos], want["slots"][order])
    # each pixel's end: its tile's start plus the kept entries before its last_idx
    W, H = sc.W, sc.H
    tx = (W + 7) // 8
    yy, xx = np.mgrid[0:H, 0:W]
    ptile = ((yy // 8) * tx + xx // 8).ravel()
    e_sorted = want["e"][order]
    before = np.searchsorted(e_sorted, want["last"], side="left") - first[ptile]
    before = np.clip(before, 0, None)
    want_clast = ranges[ptile, 0] + np.minimum(before, counts[ptile])
    assert np.array_equal(clast.astype(np.int64), want_clast)
    emit(f"  {want['e'].size} of {want['n_entries']} entries kept ({want['e'].size / want['n_entries']:.3f})")
    assert want["e"].size < want["n_entries"]


@pytest.mark.parametrize("case", ["plain", "masked", "features"])
def test_backward_over_compacted_lists_matches_full_ranges(case, monkeypatch):
    sc = S.config3(n=20_000, masked=case == "masked")
    emit(f"compacted vs full-range backward: {case}")
    got = []
    for env in ("1", "0"):
        monkeypatch.setenv("B2C_COMPACT_LISTS", env)
        r = _native.Renderer(sc)
        try:
            if case == "features":
                r.set_features(mode=1)
            r.step()
            out = {"grads": r.read("grads"), "vis_weight": r.read_model("vis_weight"),
                   "vis_count": r.read_model("vis_count"), "refine_norm": r.read_model("refine_norm")}
            # the staged path: render, loss, MFMA backward into v_splat / vis_flag
            r.forward()
            r.loss(grad_scale=3.0 * sc.W * sc.H)
            r.zero("v_splat")
            r.zero("vis_flag")
            r.backward(mode=1, grad_scale=3.0 * sc.W * sc.H)
            out["v_splat"], out["vis_flag"] = r.read("v_splat"), r.read("vis_flag")
            got.append(out)
        finally:
            r.close()
    on, off = got
    for k in on:
        assert np.array_equal(on[k], off[k]), f"{k}: {int((on[k] != off[k]).sum())} entries differ"
    emit(f"  {int(on['vis_flag'].sum())} splats visible; gradients identical with and without compaction")
