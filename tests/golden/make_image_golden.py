"""Writes the image fixtures under tests/golden/images/: JPEG files and what the reference's own decoder makes
of them, and resize cases with the reference's own output (stb_image v2.30 and stb_image_resize2 v2.18 as
src/dataset/views.cpp of Erant/b2ctrain compiles them, built unmodified from /root/reference into
oracle/_ref/libb2c_ref.so by oracle/Makefile; ref_image_load / ref_image_resize in oracle/ref_shim.cpp).

Run in the build container only (the reference and PIL's encoder are not needed on GPU boxes):

    make -C oracle ref && python tests/golden/make_image_golden.py

* ``*.jpg``: JPEG files written by PIL (libjpeg) over smooth noisy images: baseline 4:2:0, 4:2:2 and 4:4:4,
  progressive (spectral selection and successive approximation), greyscale, CMYK with an Adobe marker,
  restart intervals, qualities 20-100, sizes from 1x1 to 100x61 and 9x300 (partial MCUs on both edges);
  ``expected.npz`` holds the reference decoder's RGBA bytes and channel count for each;
* ``resize/*``: random RGBA8 inputs, sizes and the three filters the loader uses (triangle, Mitchell, point
  sample), enlarging, shrinking (down to 1/40, where the vertical pass scatters) and one axis only; the
  reference's output for each.
"""
from __future__ import annotations

import ctypes as C
import os
import sys

import numpy as np
from PIL import Image

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
OUT = os.path.join(HERE, "images")


def ref():
    L = C.CDLL(os.path.join(ROOT, "oracle", "_ref", "libb2c_ref.so"))
    L.ref_image_load.argtypes = [C.c_char_p, C.POINTER(C.c_int), C.POINTER(C.c_int), C.POINTER(C.c_int), C.c_void_p,
                                 C.c_size_t, C.c_char_p, C.c_size_t]
    L.ref_image_resize.argtypes = [C.c_void_p, C.c_int, C.c_int, C.c_void_p, C.c_int, C.c_int, C.c_int]
    return L


def ref_decode(L, path):
    w, h, c = C.c_int(), C.c_int(), C.c_int()
    err = C.create_string_buffer(256)
    if L.ref_image_load(path.encode(), w, h, c, None, 0, err, 256):
        raise RuntimeError(err.value.decode())
    buf = np.zeros(w.value * h.value * 4, np.uint8)
    L.ref_image_load(path.encode(), w, h, c, buf.ctypes.data, buf.size, err, 256)
    return buf.reshape(h.value, w.value, 4), c.value


def smooth(rng, h, w, ch):
    y, x = np.mgrid[0:h, 0:w]
    out = np.zeros((h, w, ch))
    for k in range(ch):
        out[..., k] = 128 + 100 * np.sin(x / (3 + k) + y / (5 + 2 * k)) + rng.normal(0, 20, (h, w))
    return np.clip(out, 0, 255).astype(np.uint8)


JPEG_VARIANTS = [
    ("420", "RGB", dict(subsampling=2, quality=85)),
    ("422", "RGB", dict(subsampling=1, quality=75)),
    ("444", "RGB", dict(subsampling=0, quality=90)),
    ("prog", "RGB", dict(progressive=True, quality=80)),
    ("prog444_q100", "RGB", dict(progressive=True, subsampling=0, quality=100, restart_marker_rows=1)),
    ("grey", "L", dict(quality=70)),
    ("grey_prog", "L", dict(progressive=True, quality=60)),
    ("cmyk", "CMYK", dict(quality=80)),
    ("rst_q20", "RGB", dict(quality=20, restart_marker_blocks=3)),
]
JPEG_SIZES = [(1, 1), (17, 9), (37, 23), (100, 61), (9, 300)]


def main():
    L = ref()
    rng = np.random.default_rng(20261203)
    os.makedirs(OUT, exist_ok=True)
    expected = {}
    for w, h in JPEG_SIZES:
        for tag, mode, kw in JPEG_VARIANTS:
            ch = {"RGB": 3, "L": 1, "CMYK": 4}[mode]
            a = smooth(rng, h, w, ch)
            name = f"j_{tag}_{w}x{h}.jpg"
            Image.fromarray(a[..., 0] if ch == 1 else a, mode).save(os.path.join(OUT, name), "JPEG", **kw)
            rgba, channels = ref_decode(L, os.path.join(OUT, name))
            expected[f"{name}/rgba"] = rgba
            expected[f"{name}/channels"] = np.int32(channels)
    cases = [(160, 100, 64, 40), (37, 23, 64, 48), (64, 48, 37, 23), (100, 100, 7, 5), (5, 3, 40, 30),
             (200, 10, 17, 3), (133, 97, 47, 31), (24, 16, 24, 30), (160, 120, 16, 12), (200, 150, 5, 4),
             (2, 2, 1, 1), (1, 5, 3, 9), (97, 61, 1, 61), (61, 97, 61, 5), (48, 32, 36, 24), (128, 72, 96, 54)]
    for k, (w, h, nw, nh) in enumerate(cases):
        img = rng.integers(0, 256, (h, w, 4), dtype=np.uint8)
        if k % 2:  # smooth content: values nearer the rounding midpoints of the blends
            img = np.ascontiguousarray(np.repeat(np.repeat(smooth(rng, h // 4 + 1, w // 4 + 1, 4), 4, 0), 4, 1)[:h, :w])
        expected[f"resize/{k}/in"] = img
        for f in (0, 1, 2):
            out = np.zeros((nh, nw, 4), np.uint8)
            if L.ref_image_resize(img.ctypes.data, w, h, out.ctypes.data, nw, nh, f):
                raise RuntimeError(f"reference resize failed for case {k}")
            expected[f"resize/{k}/out{f}"] = out
    np.savez_compressed(os.path.join(OUT, "expected.npz"), **expected)
    print(f"wrote {len(JPEG_SIZES) * len(JPEG_VARIANTS)} JPEG fixtures and {len(cases)} resize cases")


if __name__ == "__main__":
    sys.exit(main())
