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
