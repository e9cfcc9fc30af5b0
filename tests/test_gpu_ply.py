"""The device-direct ply pair (b2c_model_load_ply / b2c_model_save_ply: rows decoded into the model's layout
and encoded from it on the GPU) against the reference's reader and writer (the fixtures under
tests/golden/ply/) and, at a million splats, against the oracle's numpy restatement (oracle/ply.py).

Bars: the loaded model bit-identical to the reference's decoded cloud (SH bands rounded to nearest even when
stored as fp16, as an upload rounds them); saved files byte-identical to the reference writer's."""
import os
import time

import numpy as np
import pytest

from b2ctrain_amd import _native as N
from b2ctrain_amd import scenes as S
from oracle import ply as OP
from tests.gpu_harness import emit
from tests.test_ply import GOOD, WRITTEN, _input_cloud, _path, expected

pytestmark = pytest.mark.gpu


def _holder(n=1, degree=0):
    """A renderer whose model the ply calls replace (an 8x8 view, never rendered)."""
    cam = S.Camera(8, 8, 8.0, 8.0, 4.0, 4.0, np.eye(3, dtype=np.float32).reshape(9), np.zeros(3, np.float32))
    K = (degree + 1) ** 2
    sc = S.Scene("ply", degree, np.zeros((n, 4), np.float32), np.tile(np.float32([1, 0, 0, 0]), (n, 1)),
                 np.zeros((n, 4), np.float32), np.zeros((n, K, 3), np.float32), cam, np.zeros(64, np.uint32), None)
    return N.Renderer(sc)


def _model_cloud(r):
    st = r.model_state()
    return dict(pos=st["pos_op"][:, :3], opacity=st["pos_op"][:, 3], quat=st["quat"], log_scale=st["lscale"][:, :3],
                floor=st["lscale"][:, 3], sh=st["sh"])


def _bits(a):
    return np.ascontiguousarray(a, np.float32).reshape(-1).view(np.uint32)


def _check_model(r, want, sh_fp16, what):
    got = _model_cloud(r)
    assert r.n == want["n"] and r.degree == want["sh_degree"], what
    for f in ("pos", "opacity", "quat", "log_scale"):
        assert np.array_equal(_bits(got[f]), _bits(want[f])), (what, f)
    assert not got["floor"].any(), what
    sh = want["sh"].astype(np.float32).copy()
    if sh_fp16:
        sh[:, 1:, :] = sh[:, 1:, :].astype(np.float16).astype(np.float32)
    assert np.array_equal(_bits(got["sh"]), _bits(sh)), (what, "sh")


@pytest.mark.parametrize("sh_fp16", [False, True])
def test_device_load_matches_the_reference(sh_fp16):
    r = _holder()
    try:
        for case in GOOD:
            want = expected(case)
            emit(f"load {case} (n={want['n']}, sh_fp16={sh_fp16})")
            has_scales = r.load_ply(_path(case), sh_fp16=sh_fp16)
            assert has_scales == want["has_scales"]
            if want["n"]:
                _check_model(r, want, sh_fp16, case)
    finally:
        r.close()


def test_device_save_matches_the_reference(tmp_path):
    for case in WRITTEN:
        c, comments = _input_cloud(case)
        if c["n"] == 0:
            continue
        emit(f"save {case} (n={c['n']})")
        r = _holder(c["n"], c["sh_degree"])
        try:
            sc = r.scene  # the raw (unnormalised) cloud goes in through the model's upload
            sc.pos_op = np.concatenate([c["pos"], c["opacity"][:, None]], 1).astype(np.float32)
            sc.quat = c["quat"].astype(np.float32)
            sc.lscale = np.concatenate([c["log_scale"], np.zeros((c["n"], 1), np.float32)], 1)
            sc.sh = c["sh"].reshape(c["n"], -1, 3).astype(np.float32)
            sc.degree = c["sh_degree"]
            r.upload(sc)
            extras = {b: c[b] for b in N.PLY_BLOCKS if b in c}
            out = tmp_path / f"{case}.ply"
            r.save_ply(str(out), comments, extras or None)
            assert open(out, "rb").read() == open(_path(case), "rb").read(), case
        finally:
            r.close()


def test_million_splats_round_trip(tmp_path):
    """1M splats at SH degree 3 (248 MB of rows): oracle-written file -> device load (bit-exact) -> device save
    (the oracle writer's bytes for the loaded cloud). Prints the end-to-end rates."""
    rng = np.random.default_rng(5)
    n, deg = 1_000_000, 3
    c = dict(n=n, sh_degree=deg, pos=rng.normal(0, 2, (n, 3)).astype(np.float32),
             log_scale=rng.normal(-4, 1, (n, 3)).astype(np.float32), quat=rng.normal(0, 1, (n, 4)).astype(np.float32),
             opacity=rng.normal(0, 2, n).astype(np.float32), sh=rng.normal(0, 0.3, (n, 16, 3)).astype(np.float32),
             evidence=rng.random((n, 7)).astype(np.float32))
    src = str(tmp_path / "big.ply")
    OP.write(src, c, ["SH degree: 3"])
    size = os.path.getsize(src)
    want = OP.read(src)
    r = _holder()
    try:
        t0 = time.perf_counter()
        r.load_ply(src)
        t_load = time.perf_counter() - t0
        _check_model(r, dict(want, n=n, sh_degree=deg), False, "1M load")
        out = str(tmp_path / "big_out.ply")
        t0 = time.perf_counter()
        r.save_ply(out, ["SH degree: 3"], {"evidence": want["evidence"]})
        t_save = time.perf_counter() - t0
        back = dict(want, quat=_model_cloud(r)["quat"])
        ref = str(tmp_path / "big_ref.ply")
        OP.write(ref, back, ["SH degree: 3"])
        assert open(out, "rb").read() == open(ref, "rb").read()
        emit(f"    {size / 1e6:.0f} MB: load {t_load * 1e3:.0f} ms ({size / t_load / 1e9:.2f} GB/s), "
             f"save {t_save * 1e3:.0f} ms ({size / t_save / 1e9:.2f} GB/s)")
    finally:
        r.close()


def test_evidence_export_to_ply(tmp_path):
    """The trainer's export (trainer.cpp:404-410): evidence and labels of the model written beside it."""
    sc = S.fd_scene(11, n=60)
    x = np.arange(sc.W * sc.H) % sc.W
    labels = np.where(x < sc.W // 2, 3, 13).astype(np.uint8)
    r = N.Renderer(sc)
    v = N.View(sc.W, sc.H, sc.gt, labels=labels)
    try:
        ev = r.compute_evidence([v], [sc.cam], export_labels=True)
        lab = r.download_labels()
        out = str(tmp_path / "ev.ply")
        r.save_ply(out, ["SH degree: 2"], {"evidence": ev, "labels": lab})
        back = N.ply_read(out)
        assert np.array_equal(back["evidence"], ev) and np.array_equal(back["labels"], lab)
        assert np.array_equal(back["pos"], sc.pos_op[:, :3])
    finally:
        v.close()
        r.close()
