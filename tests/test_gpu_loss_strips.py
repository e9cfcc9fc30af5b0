"""The fused loss at strip heights across the range the launcher picks from (b2ctrain_amd/csrc/kernels/loss.hip,
pick_strip_rows; forced through B2C_LOSS_STRIP_ROWS): loss value and per-pixel gradient against the CPU
oracle (src/gpu/loss.cu:18-195 restated), on a 1920x1080 frame with per-pixel weights and the elliptic
mask, so partial last strips, strip seams and walks with and without extra rows before the top halo (the
walk covers whole 11-row rings) are all exercised."""
import pytest

from b2ctrain_amd import _native
from b2ctrain_amd import scenes as S
from tests.gpu_harness import check_loss, emit

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("sh", [35, 39, 46, 60, 79, 128])
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


def test_train_step_loss_accumulators_per_step():
    """What the reference's training step leaves in loss_accum: the trainer clears [0..3] every step
    (src/train/trainer.cpp:491), photometric_loss adds the loss into [0] and accumulate_loss adds [0] + [1]
    into [2] and 1 into [3] (loss.cu:317,324). The fused step stores the same values from the loss's last
    launch: after each of two steps [0] is that step's loss, [1] = 0, [2] = [0] and [3] = 1, whatever the
    buffer held before."""
    import numpy as np
    sc = S.config3(n=20_000)
    sc.bg = (0.4, 0.3, 0.2)
    emit("train step loss accumulators")
    r = _native.Renderer(sc)
    try:
        r.write("loss_accum", np.full(16, 7.0, np.float32))
        r.step(bg=sc.bg)
        a1 = r.read("loss_accum").copy()
        r.step(bg=(0.1, 0.2, 0.3))
        a2 = r.read("loss_accum").copy()
    finally:
        r.close()
    for a in (a1, a2):
        assert a[0] > 0 and a[1] == 0 and a[2] == a[0] and a[3] == 1
    assert a1[0] != a2[0]  # a different background: a different loss


def test_accumulate_loss_entry_points():
    """accumulate_loss (loss.cu:317,324) through both layers of the C ABI: b2c_accumulate_loss on a context
    and b2c_hip_accumulate_loss on a device buffer each do a[2] += a[0] + a[1] and a[3] += 1, leaving the other
    entries, over a running sum of several steps: photometric_loss adds each step's loss into a cleared [0]."""
    import ctypes as C

    import numpy as np
    sc = S.config2(n=5_000)
    emit("accumulate_loss")
    r = _native.Renderer(sc)
    try:
        start = np.arange(16, dtype=np.float32) * 0.5
        start[2], start[3] = 0.0, 0.0
        r.write("loss_accum", start)
        r.forward()
        losses = []
        for step in range(3):
            acc = r.read("loss_accum").copy()
            acc[0], acc[1] = 0.0, 0.25 * step  # the trainer clears [0]; a second loss term in [1]
            r.write("loss_accum", acc)
            check_rc = r.L.b2c_photometric_loss(r.ctx, r.view, C.byref(r.loss_opts(3.0 * sc.W * sc.H, None)))
            assert check_rc == 0
            losses.append(float(r.read("loss_accum")[0]))
            assert r.L.b2c_accumulate_loss(r.ctx) == 0
        a = r.read("loss_accum")
    finally:
        r.close()
    want2 = np.float32(0)
    for step, l in enumerate(losses):
        want2 = np.float32(want2 + np.float32(np.float32(l) + np.float32(0.25 * step)))
    assert a[2] == want2 and a[3] == 3.0, (a[:4], want2)
    assert np.array_equal(a[4:], start[4:])
    # the launcher on a plain device buffer (the library's own allocation, the default stream)
    L = _native.lib()
    L.b2c_hip_accumulate_loss.argtypes = [C.c_void_p, C.c_void_p]
    buf = _native.DeviceArray(np.array([1.5, 2.25, 10.0, 4.0] + [9.0] * 12, np.float32))
    try:
        assert L.b2c_hip_accumulate_loss(C.c_void_p(buf.ptr), None) == 0
        got = buf.download(np.float32, 16)
    finally:
        buf.free()
    assert list(got[:4]) == [1.5, 2.25, 13.75, 5.0] and (got[4:] == 9.0).all()
