"""GPU analytic gradients (forward -> fused loss -> MFMA backward -> projection VJP) against central
finite differences of the fp64 brute-force oracle, the reference's own gradient test
(tests/tests.cpp:386-442) with the north-star bar: relative error <= 1e-3. As in the reference, a sample
whose finite differences at eps and 4*eps disagree by more than 10% sits on a non-smooth point (a fragment
crossing the 1/255 cutoff or the transmittance stop) and is skipped (tests/fd_util.py states the absolute
floor). Beyond the reference's scenes (SH degree 2, no floor, no clamped splat) the cases cover SH degrees
3 and 4, the Mip-Splatting floor, splats past the tangent clamp and the fp32 anchor backward."""
import numpy as np
import pytest

from b2ctrain_amd import _native
from b2ctrain_amd import scenes as S
from tests.fd_util import fd_compare
from tests.gpu_harness import emit

pytestmark = pytest.mark.gpu


def gpu_gradients(scene, mode=1):
    r = _native.Renderer(scene)
    gs = 3.0 * scene.W * scene.H if mode == 1 else 1.0
    try:
        r.forward()
        r.loss(grad_scale=gs)
        r.zero("v_splat")
        r.zero("vis_flag")
        r.backward(mode=mode, grad_scale=gs)
        r.vjp()
        return r.read("grads")
    finally:
        r.close()


def run_fd(scene, mode=1, min_checked=150, **kw):
    an = gpu_gradients(scene, mode)
    checked, skipped, bad, worst = fd_compare(scene, an, **kw)
    emit(f"  checked {checked} skipped {skipped} worst rel {worst:.2e}")
    assert checked > min_checked
    assert not bad, f"{len(bad)} mismatches, e.g. {bad[:5]}"


@pytest.mark.parametrize("seed,masked,degree", [(1234, False, 2), (1235, True, 2), (1236, False, 3)])
def test_fd_harness_scenes(seed, masked, degree):
    sc = S.fd_scene(seed, masked=masked, degree=degree)
    emit(f"FD {sc.name} deg={degree}")
    run_fd(sc)


@pytest.mark.parametrize("masked", [False, True])
def test_fd_mip_floor(masked):
    """Every splat has a Mip-Splatting floor (lscale.w > 0): the floor enters the semi-axes and the
    opacity factor of the projection and both VJP terms of the log-scale gradient."""
    sc = S.fd_scene(1238 + 3 * masked, floor=True, masked=masked, degree=3 if masked else 2)
    emit(f"FD {sc.name} floor")
    run_fd(sc)


def test_fd_sh_degree4():
    sc = S.fd_scene(1239, degree=4)
    emit(f"FD {sc.name} SH4")
    run_fd(sc, sh_every=3)


def test_fd_tangent_clamp():
    """Half the splats are centred past the EWA Jacobian's tangent clamp; every parameter of those is
    checked (the clamped branches of the pinhole VJP)."""
    sc = S.clamp_scene(1240)
    emit(f"FD {sc.name}: clamped splats")
    run_fd(sc, every=1, sh_every=7, max_splats=sc.n // 2, min_checked=100)


def test_fd_config1():
    sc = S.config1()
    sc.bg = (0.3, 0.3, 0.3)
    emit("FD config1 (every 128th splat)")
    run_fd(sc, every=128, min_checked=60)


def test_fd_fp32_anchor_backward():
    """The fp32 anchor backward (mode 0) through the same FD bar."""
    sc = S.fd_scene(1236, degree=3)
    emit(f"FD {sc.name} mode 0")
    run_fd(sc, mode=0)


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
