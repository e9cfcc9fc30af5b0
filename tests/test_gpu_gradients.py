"""GPU analytic gradients (forward -> fused loss -> MFMA backward -> projection VJP) against central
finite differences of the fp64 brute-force oracle, the reference's own gradient test
(tests/tests.cpp:386-442) with the north-star bar: relative error <= 1e-3. As in the reference, a sample
whose finite differences at eps and 4*eps disagree by more than 10% sits on a non-smooth point (a fragment
crossing the 1/255 cutoff or the transmittance stop) and is skipped; gradients below 1e-9 in absolute
difference are compared absolutely."""
import numpy as np
import pytest

from b2ctrain_amd import _native
from b2ctrain_amd import scenes as S
from oracle import oracle as O
from tests.gpu_harness import emit

pytestmark = pytest.mark.gpu

REL_TOL = 1e-3
ABS_FLOOR = 1e-9


def fd_compare(scene, mode, every=2, sh_every=5, eps=1e-5, max_splats=None):
    r = _native.Renderer(scene)
    gs = 3.0 * scene.W * scene.H if mode == 1 else 1.0
    try:
        r.forward()
        r.loss(grad_scale=gs)
        r.zero("v_splat")
        r.zero("vis_flag")
        r.backward(mode=mode, grad_scale=gs)
        r.vjp()
        an = r.read("grads")
    finally:
        r.close()
    P0 = O.scene_params64(scene)
    per = 11 + 3 * scene.K
    bad, checked, skipped, worst = [], 0, 0, 0.0
    n = scene.n if max_splats is None else min(scene.n, max_splats)
    for i in range(0, n, every):
        for q in range(per):
            if q >= 11 and (q - 11) % sh_every:
                continue

            def at(delta):
                P = {k: v.copy() for k, v in P0.items()}
                if q < 3:
                    P["pos"][i, q] += delta
                elif q == 3:
                    P["opacity"][i] += delta
                elif q < 8:
                    P["quat"][i, q - 4] += delta
                elif q < 11:
                    P["log_scale"][i, q - 8] += delta
                else:
                    P["sh"][i, q - 11] += delta
                return O.ref_loss(scene, params=P)

            fd = (at(eps) - at(-eps)) / (2 * eps)
            fd4 = (at(4 * eps) - at(-4 * eps)) / (8 * eps)
            if abs(fd - fd4) > 0.1 * max(abs(fd), abs(fd4)) + 1e-9:
                skipped += 1
                continue
            a = float(an[i, q])
            d = abs(fd - a)
            den = max(abs(fd), abs(a))
            rel = d / den if den > 0 else 0.0
            checked += 1
            if rel > REL_TOL and d > ABS_FLOOR:
                bad.append((i, q, a, fd, rel))
            if d > ABS_FLOOR:
                worst = max(worst, rel)
    return checked, skipped, bad, worst


@pytest.mark.parametrize("seed,masked,degree", [(1234, False, 2), (1235, True, 2), (1236, False, 3)])
def test_fd_harness_scenes(seed, masked, degree):
    sc = S.fd_scene(seed, masked=masked, degree=degree)
    emit(f"FD {sc.name} deg={degree}")
    checked, skipped, bad, worst = fd_compare(sc, mode=1)
    emit(f"  checked {checked} skipped {skipped} worst rel {worst:.2e}")
    assert checked > 150
    assert not bad, f"{len(bad)} mismatches, e.g. {bad[:5]}"


def test_fd_config1():
    sc = S.config1()
    sc.bg = (0.3, 0.3, 0.3)
    emit("FD config1 (every 128th splat)")
    checked, skipped, bad, worst = fd_compare(sc, mode=1, every=128)
    emit(f"  checked {checked} skipped {skipped} worst rel {worst:.2e}")
    assert checked > 60
    assert not bad, f"{len(bad)} mismatches, e.g. {bad[:5]}"


def test_sparse_gradient_write_leaves_rows_without_gradient():
    """OptimParams::sparse on the gradient-export path (optim.cu:148: the kernel returns before the grad_out
    write when a splat has no gradient this step): rows of such splats keep whatever the buffer held, every
    other row is the dense result. The backward is deterministic, so the same step is run twice."""
    sc = S.config3(n=40_000)
    sc.bg = (0.4, 0.3, 0.2)
    gs = 3.0 * sc.W * sc.H
    r = _native.Renderer(sc)
    try:
        def step_grads(sparse, fill=None):
            r.forward()
            r.loss(grad_scale=gs)
            r.backward(mode=1, grad_scale=gs)
            if fill is not None:
                r.write("grads", fill)
            r.vjp(sparse=sparse)
            return r.read("grads")
        dense = step_grads(False)  # also allocates the buffer
        sentinel = np.full(dense.shape, 12345.0, np.float32)
        sparse = step_grads(True, fill=sentinel)
        dense2 = step_grads(False)
    finally:
        r.close()
    assert np.array_equal(dense, dense2)
    kept = (sparse == sentinel).all(1)
    written = (sparse == dense).all(1)
    assert (kept | written).all(), f"rows neither kept nor written: {np.flatnonzero(~(kept | written))[:10]}"
    assert (dense[kept] == 0).all(), "a kept row had a gradient"
    emit(f"sparse: {int(kept.sum())} rows kept, {int(written.sum())} written of {len(dense)}")
    assert kept.sum() > 1000 and written.sum() > 1000  # both cases exercised
