"""The loader's JPEG decoder and resize (include/b2c.h b2c_image_decode / b2c_image_resample, replacing the
reference's stbi_load and stbir_resize calls in src/dataset/views.cpp:63-78) against the reference's own:
tests/golden/images/expected.npz holds what stb_image v2.30 and stb_image_resize2 v2.18, compiled from the
reference's tree, made of the fixture JPEGs and resize inputs (tests/golden/make_image_golden.py).

Bars: decoded RGBA bytes and channel counts identical; resized bytes identical for the triangle, Mitchell and
point-sample filters over enlarging, shrinking (down to 1/40) and one-axis cases. A PNG read through
b2c_image_decode equals b2c_png_decode."""
import glob
import os

import numpy as np
import pytest

from b2ctrain_amd import _native as N

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "images")
Z = np.load(os.path.join(GOLD, "expected.npz"), allow_pickle=False)
JPEGS = sorted(os.path.basename(p) for p in glob.glob(os.path.join(GOLD, "*.jpg")))
RESIZE = sorted({int(k.split("/")[1]) for k in Z.files if k.startswith("resize/")})


@pytest.mark.parametrize("name", JPEGS)
def test_jpeg_decode_matches_the_reference(name):
    got, channels = N.image_decode(os.path.join(GOLD, name))
    want = Z[f"{name}/rgba"]
    assert got.shape == want.shape
    assert channels == int(Z[f"{name}/channels"])
    diff = np.flatnonzero((got != want).any(-1))
    assert not diff.size, f"{diff.size} pixels differ, first at {np.unravel_index(diff[0], got.shape[:2])}"


@pytest.mark.parametrize("case", RESIZE)
@pytest.mark.parametrize("filt", ["triangle", "mitchell", "point"])
def test_resize_matches_the_reference(case, filt):
    src = Z[f"resize/{case}/in"]
    want = Z[f"resize/{case}/out{N.RESAMPLE_FILTERS[filt]}"]
    got = N.image_resample(src, want.shape[1], want.shape[0], filt)
    assert np.array_equal(got, want), f"{int((got != want).sum())} bytes differ"


def test_resize_identity_and_constant():
    """At the same size the tent and the box return the input (the Mitchell cubic is not interpolating: it
    blurs by [1, 16, 1] / 18); a constant image stays constant under every filter (weights sum to 1)."""
    rng = np.random.default_rng(3)
    img = rng.integers(0, 256, (13, 21, 4), dtype=np.uint8)
    for f in ("triangle", "point"):
        assert np.array_equal(N.image_resample(img, 21, 13, f), img)
    row = np.zeros((1, 9, 4), np.uint8)
    row[0, 4] = 180
    got = N.image_resample(row, 9, 1, "mitchell")[0, :, 0]
    assert list(got[3:6]) == [10, 160, 10] and not got[:3].any() and not got[6:].any()
    for f in N.RESAMPLE_FILTERS:
        flat = np.full((9, 14, 4), 77, np.uint8)
        assert (N.image_resample(flat, 31, 5, f) == 77).all()


def test_png_through_the_generic_decoder():
    png = sorted(glob.glob(os.path.join(GOLD, "..", "colmap", "scene", "images", "*.png")))[0]
    a, ca = N.image_decode(png)
    b, cb = N.png_decode(png)
    assert ca == cb and np.array_equal(a, b)


def test_unknown_and_broken_files_are_rejected(tmp_path):
    (tmp_path / "x.bmp").write_bytes(b"BM" + bytes(60))
    with pytest.raises(RuntimeError, match="unknown image type"):
        N.image_decode(str(tmp_path / "x.bmp"))
    data = open(os.path.join(GOLD, JPEGS[0]), "rb").read()
    (tmp_path / "cut.jpg").write_bytes(data[:40])
    with pytest.raises(RuntimeError, match="failed to decode"):
        N.image_decode(str(tmp_path / "cut.jpg"))
