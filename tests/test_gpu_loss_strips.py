"""The fused loss at every strip height the launcher can pick (b2ctrain_amd/csrc/kernels/loss.hip,
pick_strip_rows; forced through B2C_LOSS_STRIP_ROWS): loss value and per-pixel gradient against the CPU
oracle (src/gpu/loss.cu:18-195 restated), on a 1920x1080 frame with per-pixel weights and the elliptic
mask, so partial last strips and strip seams are all exercised."""
import pytest

from b2ctrain_amd import _native
from b2ctrain_amd import scenes as S
from tests.gpu_harness import check_loss, emit

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("sh", [35, 46, 57, 79])
def test_loss_each_strip_height(sh, monkeypatch):
    monkeypatch.setenv("B2C_LOSS_STRIP_ROWS", str(sh))
    sc = S.config3(n=20_000, masked=True)
    bg = (0.3, 0.6, 0.2)
    emit(f"loss strip height {sh}")
    r = _native.Renderer(sc)
    try:
        r.project(bg=bg)
        r.bin()
        r.raster_fwd(bg=bg)
        check_loss(r, sc, r.read("out_rgba"), 3.0 * sc.W * sc.H, bg)
    finally:
        r.close()


def test_train_step_keeps_running_loss_sum():
    """The training step keeps the reference's running loss sum (accumulate_kernel, loss.cu:317,324:
    loss_accum[2] += loss_accum[0] + loss_accum[1], loss_accum[3] += 1), applied in the loss's last launch
    instead of a kernel of its own: after two steps [2] is the float32 sum of the two step losses and [3]
    is 2."""
    import numpy as np
    sc = S.config3(n=20_000)
    sc.bg = (0.4, 0.3, 0.2)
    emit("train step running loss sum")
    r = _native.Renderer(sc)
    try:
        r.zero("loss_accum")
        r.step(bg=sc.bg)
        a1 = r.read("loss_accum").copy()
        r.step(bg=sc.bg)
        a2 = r.read("loss_accum").copy()
    finally:
        r.close()
    assert a1[0] > 0 and a1[1] == 0 and a2[1] == 0
    assert a1[3] == 1 and a2[3] == 2
    assert a1[2] == np.float32(0) + (a1[0] + a1[1])
    assert a2[2] == a1[2] + (a2[0] + a2[1])
