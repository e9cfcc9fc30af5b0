"""The fp32 tiled oracle's analytic gradients (forward -> fused loss -> backward -> projection VJP,
oracle/b2c_oracle.c) against central finite differences of the fp64 brute-force oracle, on the branches
the reference's own FD harness and golden fixtures do not reach (its scenes use SH degree 2, no floor and
no splat past the tangent clamp, tests/tests.cpp:24-59): the Mip-Splatting floor (lscale.w > 0), SH
degree 4, and splats whose EWA Jacobian is clamped. Bar: relative error <= 1e-3 at smooth points."""
import pytest

from b2ctrain_amd import scenes as S
from oracle import oracle as O
from tests.fd_util import fd_compare

CASES = {
    "floor": lambda: S.fd_scene(1238, floor=True),
    "floor_masked_sh3": lambda: S.fd_scene(1241, degree=3, floor=True, masked=True),
    "sh4": lambda: S.fd_scene(1239, degree=4),
    "clamp": lambda: S.clamp_scene(1240),
}


@pytest.mark.parametrize("name", list(CASES))
def test_oracle_gradients_vs_fp64_fd(name):
    sc = CASES[name]()
    grads = O.pipeline(sc)["grads"]
    checked, skipped, bad, worst = fd_compare(sc, grads, every=2, sh_every=3 if sc.degree == 4 else 5)
    assert checked > 150, (checked, skipped)
    assert not bad, f"{len(bad)} mismatches, e.g. {bad[:5]}"


def test_oracle_gradients_clamped_splats_only():
    """Every parameter of the splats centred beyond the clamp (the scene's first half)."""
    sc = S.clamp_scene(1240)
    grads = O.pipeline(sc)["grads"]
    checked, skipped, bad, worst = fd_compare(sc, grads, every=1, sh_every=7, max_splats=sc.n // 2)
    assert checked > 100, (checked, skipped)
    assert not bad, f"{len(bad)} mismatches, e.g. {bad[:5]}"
