"""The COLMAP dataset loader on the host (include/b2c.h b2c_dataset_*, replacing src/dataset/views.cpp and
colmap.cpp) against the reference's own loader: tests/golden/colmap/expected.npz holds what the compiled
reference (with the stb_image decoder it vendors) loaded from tests/golden/colmap/scene/
and scene_jpeg/ (tests/golden/make_colmap_golden.py): PNG and JPEG frames, sidecars of other sizes than their
frames, and resolution caps, so every decode and resample path of the loader is compared. The PNG decoder is
also checked against PIL.

Bars: every view's planes, camera, flags, alpha coverage and normal-mask count bit-identical to the
reference's; the same split, counts, points and initial ply."""
import glob
import os

import numpy as np
import pytest
from PIL import Image

from b2ctrain_amd import _native as N

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "colmap")
SCENE = os.path.join(GOLD, "scene")
Z = np.load(os.path.join(GOLD, "expected.npz"), allow_pickle=False)
OPTIONS = {  # name: (scene directory, options) as tests/golden/make_colmap_golden.py loaded them
    "split3": ("scene", dict(eval_split_every=3)),
    "masked_sub2": ("scene", dict(max_frames=5, subsample_frames=2, alpha_mode="masked")),
    "cap16": ("scene", dict(max_resolution=16)),
    "jpeg_split2": ("scene_jpeg", dict(eval_split_every=2)),
    "jpeg_cap32": ("scene_jpeg", dict(max_resolution=32)),
}


@pytest.mark.parametrize("opt", sorted(OPTIONS))
def test_dataset_matches_the_reference(opt):
    scene, kw = OPTIONS[opt]
    ds = N.Dataset(os.path.join(GOLD, scene), **kw)
    try:
        s = ds.summary()
        assert s["counts"] == list(Z[f"{opt}/counts"])
        assert s["name"] == str(Z[f"{opt}/name"])
        init = os.path.relpath(s["init_ply"], s["root"]) if s["init_ply"] else ""
        assert init == str(Z[f"{opt}/init_ply"])
        xyz, rgb = ds.points()
        assert np.array_equal(xyz, Z[f"{opt}/points_xyz"]) and np.array_equal(rgb, Z[f"{opt}/points_rgb"])
        for split in (0, 1):
            assert ds.count(split) == int(Z[f"{opt}/count{split}"])
            for i in range(ds.count(split)):
                key = f"{opt}/{split}/{i}"
                v = ds.info(split, i)
                ints = Z[f"{key}/ints"]
                fl = Z[f"{key}/floats"]
                assert v.name.decode() == str(Z[f"{key}/name"]), key
                assert [v.w, v.h, v.cam.width, v.cam.height, v.has_alpha, v.masked, v.has_normals, v.has_weights,
                        v.has_labels] == list(ints), key
                cam = np.array([v.cam.fx, v.cam.fy, v.cam.cx, v.cam.cy, *v.cam.R, *v.cam.t], np.float32)
                assert np.array_equal(cam.view(np.uint32), fl[:16].view(np.uint32)), key
                assert np.float32(v.alpha_coverage).view(np.uint32) == fl[19].view(np.uint32), key
                assert v.normal_mask_count == float(Z[f"{key}/normal_mask_count"]), key
                planes = ds.planes(split, i)
                for k in ("rgba", "normals", "weights", "labels"):
                    want = Z[f"{key}/{k}"]
                    got = planes.get(k, np.zeros_like(want))
                    assert np.array_equal(got, want), (key, k)
    finally:
        ds.close()


def test_colmap_errors(tmp_path):
    with pytest.raises(RuntimeError, match="no cameras.txt"):
        N.Dataset(str(tmp_path))
    (tmp_path / "cameras.txt").write_text("1 FISHEYE 10 10 1 2 3 4\n")
    (tmp_path / "images.txt").write_text("")
    with pytest.raises(RuntimeError, match="unsupported camera model 'FISHEYE'"):
        N.Dataset(str(tmp_path))
    (tmp_path / "cameras.txt").write_text("1 PINHOLE 10 10 1 2 3\n")
    with pytest.raises(RuntimeError, match="PINHOLE needs 4 params"):
        N.Dataset(str(tmp_path))


@pytest.mark.parametrize("path", sorted(glob.glob(os.path.join(SCENE, "**", "*.png"), recursive=True) +
                                        glob.glob(os.path.join(SCENE, "**", "*.PNG"), recursive=True)))
def test_png_decoder_matches_pil(path):
    got, channels = N.png_decode(path)
    im = Image.open(path)
    mode = im.mode
    if mode in ("I;16", "I;16B", "I"):  # 16-bit grey: the high byte, as the 8-bit loader keeps it
        a = (np.asarray(im, np.uint32) >> 8).astype(np.uint8)
        want = np.stack([a, a, a, np.full_like(a, 255)], -1)
        if "transparency" in im.info:
            want[..., 3][np.asarray(im) == im.info["transparency"]] = 0
    else:  # PIL narrows 16-bit colour to its high byte itself
        want = np.asarray(im.convert("RGBA")).copy()
        depth = open(path, "rb").read()[24]
        if mode == "L" and depth < 8 and "transparency" in im.info:
            # a grey key below 8 bits is compared after scaling to 0..255 (the stb_image rule the reference's
            # loader follows, checked against it by test_dataset_matches_the_reference); PIL leaves it unscaled
            scale = {1: 255, 2: 85, 4: 17}[depth]
            want[..., 3] = np.where(want[..., 0] == im.info["transparency"] * scale, 0, 255)
    assert got.shape == want.shape
    assert np.array_equal(got, want), path
    key = "transparency" in im.info  # a tRNS chunk counts as an alpha channel
    expect_ch = {"L": 1 + key, "LA": 2, "RGB": 3 + key, "RGBA": 4, "I;16": 1 + key, "I;16B": 1 + key, "I": 1 + key,
                 "1": 1 + key, "P": 4 if key else 3}[mode]
    assert channels == expect_ch, (path, mode, channels)
