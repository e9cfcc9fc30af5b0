"""Writes the COLMAP dataset fixtures under tests/golden/colmap/ and what the reference's own loader makes of
them (src/dataset/views.cpp and colmap.cpp of Erant/b2ctrain with the stb_image decoder it vendors, compiled
unmodified from /root/reference into oracle/_ref/libb2c_ref.so by oracle/Makefile).

Run in the build container only (the reference is not present on GPU boxes):

    make -C oracle ref && python tests/golden/make_colmap_golden.py

``scene/`` is a small text-model dataset whose frames and sidecars cover the PNG variants a capture can
hold (RGBA, RGB, grey and grey + alpha, palettes with and without tRNS, 16-bit samples, 1/2/4-bit grey,
colour-key tRNS, Adam7 interlacing; the PNG files are written here byte by byte with zlib), masks (with
the .mask suffix and upper-case names), weights (RGB luma and grey), labels and normals sidecars, the three
pinhole camera models, a frame found by a recursive search, a frame whose file is missing, points3D.txt
and splat / mesh plys. ``scene_jpeg/`` holds JPEG frames (baseline 4:2:0 and 4:2:2 with restart markers,
progressive 4:4:4, grey, CMYK) and a PNG frame of mixed sizes, with mask, weight, label and normal sidecars
of other sizes than their frames (JPEG and PNG), the model at the dataset root. ``expected.npz`` holds every
loaded view (planes, camera, flags) for each option set: eval splits, a forced masked alpha mode with frame
subsampling, and resolution caps below the frame sizes (Mitchell-resampled frames; triangle-resampled masks
and weights; point-sampled labels and normals).
"""
from __future__ import annotations

import ctypes as C
import os
import shutil
import struct
import sys
import zlib

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
OUT = os.path.join(HERE, "colmap")
sys.path.insert(0, ROOT)

W, H = 24, 16


def png_bytes(pixels, colour, depth, palette=None, trns=None, interlace=False):
    """A PNG of `pixels` ([H][W][samples] integers at `depth` bits, or palette indices)."""
    h, w = pixels.shape[:2]
    samples = {0: 1, 2: 3, 3: 1, 4: 2, 6: 4}[colour]

    def chunk(tag, body):
        return struct.pack(">I", len(body)) + tag + body + struct.pack(">I", zlib.crc32(tag + body) & 0xFFFFFFFF)

    def rows(px, filt):
        out = bytearray()
        prev = None
        for y in range(px.shape[0]):
            vals = px[y].reshape(-1)
            if depth == 16:
                raw = b"".join(struct.pack(">H", int(v)) for v in vals)
            elif depth == 8:
                raw = bytes(int(v) for v in vals)
            else:
                bits = "".join(format(int(v), f"0{depth}b") for v in vals)
                bits += "0" * (-len(bits) % 8)
                raw = bytes(int(bits[i:i + 8], 2) for i in range(0, len(bits), 8))
            f = filt[y % len(filt)]
            bpp = max(1, samples * depth // 8)
            enc = bytearray(raw)
            for i in range(len(raw)):
                left = raw[i - bpp] if i >= bpp else 0
                up = prev[i] if prev is not None else 0
                ul = prev[i - bpp] if (prev is not None and i >= bpp) else 0
                if f == 1:
                    enc[i] = (raw[i] - left) & 255
                elif f == 2:
                    enc[i] = (raw[i] - up) & 255
                elif f == 3:
                    enc[i] = (raw[i] - ((left + up) >> 1)) & 255
                elif f == 4:
                    p = left + up - ul
                    pa, pb, pc = abs(p - left), abs(p - up), abs(p - ul)
                    pred = left if (pa <= pb and pa <= pc) else (up if pb <= pc else ul)
                    enc[i] = (raw[i] - pred) & 255
            out += bytes([f]) + enc
            prev = raw
        return bytes(out)

    filters = [0, 1, 2, 3, 4]
    if interlace:
        data = b""
        for x0, y0, dx, dy in ((0, 0, 8, 8), (4, 0, 8, 8), (0, 4, 4, 8), (2, 0, 4, 4), (0, 2, 2, 4), (1, 0, 2, 2),
                               (0, 1, 1, 2)):
            sub = pixels[y0::dy, x0::dx]
            if sub.size:
                data += rows(sub, filters)
    else:
        data = rows(pixels, filters)
    ihdr = struct.pack(">IIBBBBB", w, h, depth, colour, 0, 0, 1 if interlace else 0)
    body = chunk(b"IHDR", ihdr)
    if palette is not None:
        body += chunk(b"PLTE", bytes(np.asarray(palette, np.uint8).reshape(-1)))
    if trns is not None:
        body += chunk(b"tRNS", bytes(trns))
    body += chunk(b"tEXt", b"Comment\x00fixture") + chunk(b"IDAT", zlib.compress(data, 9)) + chunk(b"IEND", b"")
    return b"\x89PNG\r\n\x1a\n" + body


def write(path, data):
    os.makedirs(os.path.dirname(path), exist_ok=True)
    with open(path, "wb") as f:
        f.write(data)


def build_scene(rng, root):
    if os.path.exists(root):
        shutil.rmtree(root)
    u8 = lambda *s: rng.integers(0, 256, s)
    frames = {
        "f00_rgba.png": png_bytes(u8(H, W, 4), 6, 8),
        "f01_rgb.png": png_bytes(u8(H, W, 3), 2, 8),
        "f02_grey.png": png_bytes(u8(H, W, 1), 0, 8),
        "f03_palette_trns.png": png_bytes(rng.integers(0, 12, (H, W, 1)), 3, 8, palette=u8(12, 3),
                                          trns=list(rng.integers(0, 256, 9))),
        "f04_grey16_interlaced.png": png_bytes(rng.integers(0, 65536, (H, W, 1)), 0, 16, interlace=True),
        "f05_grey_alpha.png": png_bytes(u8(H, W, 2), 4, 8),
        "f06_rgba16.png": png_bytes(rng.integers(0, 65536, (H, W, 4)), 6, 16),
        "f07_grey4_key.png": png_bytes(rng.integers(0, 16, (H, W, 1)), 0, 4, trns=[0, 7]),
        "f08_rgb_key_interlaced.png": png_bytes(rng.integers(0, 4, (H, W, 3)) * 60, 2, 8, trns=[0, 60, 0, 120, 0, 0],
                                                interlace=True),
        "f09_palette2.png": png_bytes(rng.integers(0, 4, (H, W, 1)), 3, 2, palette=u8(4, 3)),
        "f10_grey1.png": png_bytes(rng.integers(0, 2, (H, W, 1)), 0, 1),
    }
    for name, data in frames.items():
        write(os.path.join(root, "images", name), data)
    # a frame outside images/, found by its path suffix
    write(os.path.join(root, "captures", "sub", "f11_found.png"), png_bytes(u8(H, W, 3), 2, 8))
    # sidecars
    write(os.path.join(root, "masks", "f01_rgb.mask.png"), png_bytes(u8(H, W, 1), 0, 8))
    write(os.path.join(root, "masks", "F02_GREY.PNG"), png_bytes(u8(H, W, 2), 4, 8))  # alpha from its alpha
    write(os.path.join(root, "weights", "f02_grey.png"), png_bytes(u8(H, W, 3), 2, 8))  # luma
    write(os.path.join(root, "weights", "f05_grey_alpha.png"), png_bytes(u8(H, W, 1), 0, 8))  # grey
    write(os.path.join(root, "labels", "f02_grey.png"), png_bytes(rng.integers(0, 29, (H, W, 1)), 0, 8))
    write(os.path.join(root, "labels", "nested", "f06_rgba16.png"), png_bytes(rng.integers(0, 40, (H, W, 3)), 2, 8))
    write(os.path.join(root, "normals", "f02_grey.png"), png_bytes(u8(H, W, 4), 6, 8))
    write(os.path.join(root, "normals", "f00_rgba.png"), png_bytes(u8(H, W, 3), 2, 8))
    # the model under sparse/0: three camera models, unsorted images, one missing frame
    cams = ["# Camera list", "1 PINHOLE 48 32 40.5 41.25 24.0 16.5", "2 SIMPLE_PINHOLE 24 16 20.0 12.0 8.0",
            "3 SIMPLE_RADIAL 96 64 80.0 48.0 32.0 0.01"]
    write(os.path.join(root, "sparse", "0", "cameras.txt"), ("\n".join(cams) + "\n").encode())
    names = sorted(frames) + ["f11_found.png", "missing.png"]
    order = rng.permutation(len(names))
    lines = ["# Image list with two lines of data per image:"]
    for k in order:
        q = rng.normal(0, 1, 4)
        t = rng.normal(0, 1, 3)
        lines.append(f"{k + 1} {q[0]:.9f} {q[1]:.9f} {q[2]:.9f} {q[3]:.9f} {t[0]:.9f} {t[1]:.9f} {t[2]:.9f} "
                     f"{1 + k % 3} {names[k]}")
        lines.append("1.0 2.0 -1" if k % 2 else "")
    write(os.path.join(root, "sparse", "0", "images.txt"), ("\n".join(lines) + "\n").encode())
    pts = ["# 3D point list"] + [f"{k} {x:.6f} {y:.6f} {z:.6f} {r} {g} {b} 0.5 1 2"
                                 for k, (x, y, z, r, g, b) in enumerate(zip(*rng.normal(0, 1, (3, 20)),
                                                                            *rng.integers(0, 256, (3, 20))))]
    write(os.path.join(root, "sparse", "0", "points3D.txt"), ("\n".join(pts) + "\n").encode())
    # plys: a splat cloud named init.ply wins over a later one; a mesh is skipped
    from oracle import ply as OP
    cloud = dict(n=3, sh_degree=0, pos=rng.normal(0, 1, (3, 3)), log_scale=np.zeros((3, 3)),
                 quat=np.tile([1.0, 0, 0, 0], (3, 1)), opacity=np.zeros(3), sh=np.zeros((3, 1, 3)))
    OP.write(os.path.join(root, "init.ply"), cloud)
    OP.write(os.path.join(root, "zz_later.ply"), cloud)
    write(os.path.join(root, "zzz_mesh.ply"), b"ply\nformat ascii 1.0\nelement vertex 3\nproperty float x\n"
                                              b"property float y\nproperty float z\nelement face 1\n"
                                              b"property list uchar int vertex_indices\nend_header\n"
                                              b"0 0 0\n1 0 0\n0 1 0\n3 0 1 2\n")


def ref():
    L = C.CDLL(os.path.join(ROOT, "oracle", "_ref", "libb2c_ref.so"))
    L.ref_dataset_load.argtypes = [C.c_char_p, C.c_int, C.c_uint, C.c_int, C.c_int, C.c_int, C.c_char_p, C.c_size_t]
    L.ref_dataset_count.argtypes = [C.c_int]
    L.ref_dataset_view.argtypes = [C.c_int, C.c_int, C.POINTER(C.c_int), C.POINTER(C.c_float),
                                   C.POINTER(C.c_double), C.c_char_p, C.c_size_t]
    L.ref_dataset_view_arrays.argtypes = [C.c_int, C.c_int] + [C.c_void_p] * 4
    L.ref_dataset_summary.restype = C.c_longlong
    L.ref_dataset_summary.argtypes = [C.POINTER(C.c_int), C.c_char_p, C.c_size_t, C.c_void_p, C.c_void_p]
    return L


OPTION_SETS = {  # name: (scene, max_frames, max_resolution, eval_split_every, subsample_frames, alpha_mode)
    "split3": ("scene", -1, 1920, 3, -1, -1),
    "masked_sub2": ("scene", 5, 1920, -1, 2, 0),
    "cap16": ("scene", -1, 16, -1, -1, -1),  # every frame over the cap: Mitchell, sidecars follow the frame
    "jpeg_split2": ("scene_jpeg", -1, 1920, 2, -1, -1),
    "jpeg_cap32": ("scene_jpeg", -1, 32, -1, -1, -1),
}


def jpeg_bytes(pixels, mode, **kw):
    """A JPEG of `pixels` written by PIL (libjpeg)."""
    import io

    from PIL import Image
    buf = io.BytesIO()
    Image.fromarray(pixels[..., 0] if pixels.shape[-1] == 1 else pixels, mode).save(buf, "JPEG", **kw)
    return buf.getvalue()


def smooth(rng, h, w, ch):
    y, x = np.mgrid[0:h, 0:w]
    out = np.zeros((h, w, ch))
    for k in range(ch):
        out[..., k] = 128 + 100 * np.sin(x / (3 + k) + y / (5 + 2 * k)) + rng.normal(0, 20, (h, w))
    return np.clip(out, 0, 255).astype(np.uint8)


def build_jpeg_scene(rng, root):
    """JPEG frames (baseline 4:2:0 / 4:4:4, progressive, grey, CMYK) of mixed sizes, one PNG frame, and
    sidecars of other sizes than their frames: every decode and resample path of the loader."""
    if os.path.exists(root):
        shutil.rmtree(root)
    frames = {
        "a_420.jpg": (40, 30, jpeg_bytes(smooth(rng, 30, 40, 3), "RGB", subsampling=2, quality=85)),
        "b_444_prog.jpg": (36, 24, jpeg_bytes(smooth(rng, 24, 36, 3), "RGB", subsampling=0, progressive=True)),
        "c_grey.jpg": (32, 20, jpeg_bytes(smooth(rng, 20, 32, 1), "L", quality=70)),
        "d_cmyk.jpg": (30, 20, jpeg_bytes(smooth(rng, 20, 30, 4), "CMYK", quality=80)),
        "e_big_422.jpg": (64, 40, jpeg_bytes(smooth(rng, 40, 64, 3), "RGB", subsampling=1, restart_marker_blocks=2)),
        "f_rgba.png": (24, 16, png_bytes(rng.integers(0, 256, (16, 24, 4)), 6, 8)),
    }
    for name, (_, _, data) in frames.items():
        write(os.path.join(root, "images", name), data)
    # masks: a smaller grey JPEG (triangle enlarge), a larger PNG with alpha (triangle shrink)
    write(os.path.join(root, "masks", "a_420.mask.jpg"), jpeg_bytes(smooth(rng, 15, 20, 1), "L"))
    write(os.path.join(root, "masks", "e_big_422.png"), png_bytes(rng.integers(0, 256, (60, 96, 2)), 4, 8))
    # weights: RGB at another size (luma after a triangle resample), grey JPEG
    write(os.path.join(root, "weights", "b_444_prog.png"), png_bytes(rng.integers(0, 256, (12, 18, 3)), 2, 8))
    write(os.path.join(root, "weights", "e_big_422.jpg"), jpeg_bytes(smooth(rng, 20, 32, 1), "L"))
    # labels and normals: point-sampled from other sizes
    write(os.path.join(root, "labels", "a_420.png"), png_bytes(rng.integers(0, 29, (45, 60, 1)), 0, 8))
    write(os.path.join(root, "labels", "f_rgba.png"), png_bytes(rng.integers(0, 29, (8, 12, 1)), 0, 8))
    write(os.path.join(root, "normals", "e_big_422.png"), png_bytes(rng.integers(0, 256, (20, 32, 4)), 6, 8))
    write(os.path.join(root, "normals", "d_cmyk.jpg"), jpeg_bytes(smooth(rng, 40, 60, 3), "RGB"))
    cams = ["1 PINHOLE 40 30 33.0 34.0 20.0 15.0", "2 SIMPLE_PINHOLE 36 24 30.0 18.0 12.0",
            "3 PINHOLE 32 20 25.0 26.0 16.0 10.0", "4 OPENCV 30 20 24.0 24.5 15.0 10.0 0.1 0.01 0 0",
            "5 PINHOLE 64 40 50.0 51.0 32.0 20.0", "6 PINHOLE 24 16 20.0 20.0 12.0 8.0"]
    write(os.path.join(root, "cameras.txt"), ("\n".join(cams) + "\n").encode())
    lines = []
    for k, name in enumerate(sorted(frames)):
        q = rng.normal(0, 1, 4)
        t = rng.normal(0, 1, 3)
        lines += [f"{k + 1} {q[0]:.9f} {q[1]:.9f} {q[2]:.9f} {q[3]:.9f} {t[0]:.9f} {t[1]:.9f} {t[2]:.9f} {k + 1} {name}",
                  ""]
    write(os.path.join(root, "images.txt"), ("\n".join(lines) + "\n").encode())


def main():
    rng = np.random.default_rng(20261202)
    build_scene(rng, os.path.join(OUT, "scene"))
    build_jpeg_scene(np.random.default_rng(20261203), os.path.join(OUT, "scene_jpeg"))
    L = ref()
    expected = {}
    for opt, (scene_dir, mf, mr, ev, sub, am) in OPTION_SETS.items():
        scene = os.path.join(OUT, scene_dir)
        err = C.create_string_buffer(1024)
        if L.ref_dataset_load(scene.encode(), mf, mr, ev, sub, am, err, 1024):
            raise RuntimeError(err.value.decode())
        counts = (C.c_int * 5)()
        text = C.create_string_buffer(4096)
        npts = L.ref_dataset_summary(counts, text, 4096, None, None)
        xyz, rgb = np.zeros((npts, 3), np.float32), np.zeros((npts, 3), np.uint8)
        L.ref_dataset_summary(counts, text, 4096, xyz.ctypes.data, rgb.ctypes.data)
        root, name, init = text.value.decode().split("\n")
        expected[f"{opt}/counts"] = np.array(list(counts), np.int32)
        expected[f"{opt}/name"] = np.array(name)
        expected[f"{opt}/init_ply"] = np.array(os.path.relpath(init, root) if init else "")
        expected[f"{opt}/points_xyz"], expected[f"{opt}/points_rgb"] = xyz, rgb
        for split in (0, 1):
            n = L.ref_dataset_count(split)
            expected[f"{opt}/count{split}"] = np.int32(n)
            for i in range(n):
                ints, floats, nmc = (C.c_int * 9)(), (C.c_float * 20)(), C.c_double()
                vname = C.create_string_buffer(256)
                L.ref_dataset_view(split, i, ints, floats, C.byref(nmc), vname, 256)
                w, h = ints[0], ints[1]
                planes = dict(rgba=np.zeros(w * h, np.uint32), normals=np.zeros(w * h, np.uint32),
                              weights=np.zeros(w * h, np.uint8), labels=np.zeros(w * h, np.uint8))
                L.ref_dataset_view_arrays(split, i, *[planes[k].ctypes.data for k in ("rgba", "normals", "weights",
                                                                                     "labels")])
                key = f"{opt}/{split}/{i}"
                expected[f"{key}/ints"] = np.array(list(ints), np.int32)
                expected[f"{key}/floats"] = np.array(list(floats), np.float32)
                expected[f"{key}/normal_mask_count"] = np.float64(nmc.value)
                expected[f"{key}/name"] = np.array(vname.value.decode())
                for k, v in planes.items():
                    expected[f"{key}/{k}"] = v
    np.savez_compressed(os.path.join(OUT, "expected.npz"), **expected)
    print("views:", {k: int(v) for k, v in expected.items() if k.endswith("count0") or k.endswith("count1")})


if __name__ == "__main__":
    sys.exit(main())
