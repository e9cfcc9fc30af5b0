"""The row buffer of the atomic-free backward and of the evidence pass holds rows only for the (tile, splat)
pairs inside the tiles' shrunk ranges. Every row a pass writes carries the pass's tag (a generation, or'd with
the tile id for the backward's rows); the reductions take a row as the pass's own only when its tag matches,
so rows past a shrunk end are neither written nor cleared. The context clears the buffer before a tag could
repeat (at reallocation, when the row layout or the tile bits change, and when the generations run out).

The MFMA backward's reduce either reads every row's tag from the row itself or, with the live-row index
(B2C_ROW_LIVE = 1, the context's choice for long lists), reads a 4-byte tag per row from row_live and only the
rows it marks; the backward tests run both ways. The two modes walk windows of different lengths (256 rows
when every row is read, 1024 through the index), so a splat's run pieces are summed in different groupings
and the two agree to float rounding; within one mode every result is reproducible bit for bit.

Checked here: poisoning the whole row buffer with NaN before a pass leaves v_splat and vis_weight bit-identical
and the evidence finite and equal to rounding (its sums use float atomics), so no row past a shrunk end is
read and every row inside one is written; and passes over changing lists on one context, with the generations
cut to 1 or 2 per epoch (B2C_ROW_GEN_LIMIT) and an evidence pass switching the row layout in between, give
the gradients of a fresh context bit for bit."""
import numpy as np
import pytest

from b2ctrain_amd import _native
from b2ctrain_amd import scenes as S
from tests.gpu_harness import emit

pytestmark = pytest.mark.gpu

live_index = pytest.mark.parametrize("row_live", ["0", "1"], ids=["rows", "live-index"])


def _occluded_scene():
    """Config 4's dense slab cut to an eighth in each image direction (the same depth complexity): most of
    each tile's list lies behind its last contributor."""
    return S.config4(shrink=8)


def _view_grads(r, sc, cam, gs, poison=False):
    r.forward(cam=cam)
    r.loss(grad_scale=gs)
    r.zero("v_splat")
    r.zero("vis_flag")
    r.write_model("vis_weight", np.zeros(sc.n, np.float32))
    if poison:
        r.write("isect_rows", np.full((r.info().num_isect, 12), np.nan, np.float32))
    r.backward(mode=1, grad_scale=gs, cam=cam)
    return r.read("v_splat"), r.read_model("vis_weight"), r.read("vis_flag")


def test_occluded_lists_are_mostly_past_the_shrunk_end():
    sc = _occluded_scene()
    r = _native.Renderer(sc)
    try:
        r.forward()
        ranges, tile_end = r.read("tile_ranges").astype(np.int64), r.read("tile_end").astype(np.int64)
        live = np.clip(ranges[:, 1] - ranges[:, 0], 0, None).sum()
        total = r.info().num_isect
        emit(f"    {sc.name}: {1 - live / total:.0%} of {total} list entries lie past their tile's shrunk end")
        assert live < 0.7 * total and (tile_end[:-1] >= ranges[:, 1]).all()
    finally:
        r.close()


@live_index
@pytest.mark.parametrize("make", [_occluded_scene, lambda: S.config2(n=20_000)], ids=["occluded", "config2"])
def test_backward_reads_no_row_past_the_shrunk_end(make, row_live, monkeypatch):
    monkeypatch.setenv("B2C_ROW_LIVE", row_live)
    sc = make()
    emit(f"poisoned rows, backward {sc.name}")
    r = _native.Renderer(sc)
    gs = 3.0 * sc.W * sc.H
    try:
        clean = _view_grads(r, sc, sc.cam, gs)
        poisoned = _view_grads(r, sc, sc.cam, gs, poison=True)
        for a, b in zip(clean, poisoned):
            assert np.array_equal(a, b)
        assert np.isfinite(poisoned[0]).all() and (poisoned[2] != 0).sum() > 100
    finally:
        r.close()


def test_evidence_reads_no_row_past_the_shrunk_end():
    sc = _occluded_scene()
    emit(f"poisoned rows, evidence {sc.name}")
    r = _native.Renderer(sc)
    v = _native.View(sc.W, sc.H, sc.gt, sc.weights, has_alpha=True)
    try:
        ev = r.compute_evidence([v], [sc.cam])
        r.write("isect_rows", np.full((r.info().num_isect, 12), np.nan, np.float32))
        ev2 = r.compute_evidence([v], [sc.cam])
        # a NaN row read anywhere would make its splat's sums NaN; the sums add run pieces with float
        # atomics in no fixed order, so the two runs agree to rounding, not bit for bit
        assert np.isfinite(ev2).all() and (ev2[:, 2] > 0).sum() > 100
        assert np.allclose(ev2, ev, rtol=1e-5, atol=1e-6 * np.abs(ev).max())
    finally:
        v.close()
        r.close()


@pytest.mark.parametrize("make", [_occluded_scene, lambda: S.config2(n=20_000)], ids=["occluded", "config2"])
def test_live_row_index_gives_the_same_gradients(make, monkeypatch):
    sc = make()
    emit(f"live-row index against full row reads, {sc.name}")
    gs = 3.0 * sc.W * sc.H
    got = {}
    for mode in ("0", "1"):
        monkeypatch.setenv("B2C_ROW_LIVE", mode)
        r = _native.Renderer(sc)
        try:
            got[mode] = _view_grads(r, sc, sc.cam, gs, poison=True)
        finally:
            r.close()
    # v_splat (per gradient lane) and vis_weight: the same sums, grouped differently; vis_flag exactly
    for a, b in zip(got["0"][:2], got["1"][:2]):
        a64, b64 = a.astype(np.float64), b.astype(np.float64)
        scale = np.abs(a64).max(axis=0) + 1e-30
        err = (np.abs(a64 - b64) / scale).max()
        assert err <= 1e-5, err
    assert np.array_equal(got["0"][2], got["1"][2])
    assert (got["1"][2] != 0).sum() > 100


@live_index
@pytest.mark.parametrize("limit", ["1", "2"])
def test_tag_epochs_on_changing_lists(limit, row_live, monkeypatch):
    """With one generation per epoch every pass must clear the buffer first: a pass over another view's
    lists would otherwise read the previous view's rows as its own (they carry the same tag)."""
    monkeypatch.setenv("B2C_ROW_GEN_LIMIT", limit)
    monkeypatch.setenv("B2C_ROW_LIVE", row_live)
    sc = _occluded_scene()
    cams = sc.extra_cams[:3]
    gs = 3.0 * sc.W * sc.H
    emit(f"tag epochs of {limit} generation(s), {sc.name}, {len(cams)} views")
    fresh = []
    for cam in cams:
        r = _native.Renderer(sc)
        try:
            fresh.append(_view_grads(r, sc, cam, gs))
        finally:
            r.close()
    r = _native.Renderer(sc)
    v = _native.View(sc.W, sc.H, sc.gt, sc.weights, has_alpha=True)
    try:
        for rnd in range(2):
            for i, cam in enumerate(cams):
                got = _view_grads(r, sc, cam, gs)
                for a, b in zip(got, fresh[i]):
                    assert np.array_equal(a, b), (rnd, i)
            r.compute_evidence([v], [cams[0]])  # the evidence rows' layout: the next pass starts an epoch
    finally:
        v.close()
        r.close()


@live_index
def test_tag_epochs_across_row_layouts(row_live, monkeypatch):
    """Backward passes with and without feature lanes (16- and 12-float rows) alternate on one context; each
    layout change starts an epoch, and every pass gives the gradients of a fresh context."""
    monkeypatch.setenv("B2C_ROW_GEN_LIMIT", "3")
    monkeypatch.setenv("B2C_ROW_LIVE", row_live)
    sc = _occluded_scene()
    gs = 3.0 * sc.W * sc.H
    emit(f"row layouts, {sc.name}")

    def run(r, feat):
        r.set_features(mode=2 if feat else 0, buffer=np.tile([0.2, -0.4, 0.9], (sc.n, 1)) if feat else None)
        return _view_grads(r, sc, sc.cam, gs)

    fresh = {}
    for feat in (False, True):
        r = _native.Renderer(sc)
        try:
            fresh[feat] = run(r, feat)
        finally:
            r.close()
    r = _native.Renderer(sc)
    try:
        for feat in (False, True, True, False, True, False, False):
            for a, b in zip(run(r, feat), fresh[feat]):
                assert np.array_equal(a, b), feat
    finally:
        r.close()
