"""Writes the ply fixtures under tests/golden/ply/ with the reference's own reader and writer (src/ply.cpp of
Erant/b2ctrain, compiled unmodified from /root/reference into oracle/_ref/libb2c_ref.so by oracle/Makefile).

Run in the build container only (the reference is not present on GPU boxes):

    make -C oracle ref && python tests/golden/make_ply_golden.py

Three kinds of fixture:
* ``written_*.ply``: clouds (inputs stored in expected.npz as ``<case>/in_*``) written by the reference's
  write_ply; this build's writers must produce the same bytes;
* ``input_*.ply``: files in the layouts read_ply accepts (other property types, ascii, colour-only point
  clouds, the optional blocks, comments, an empty non-vertex element), written here byte by byte;
  ``<case>/*`` in expected.npz holds what the reference's read_ply returned;
* ``bad_*.ply``: files read_ply rejects (``<case>/error`` holds the reference's message).
"""
from __future__ import annotations

import ctypes as C
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
OUT = os.path.join(HERE, "ply")
FIELDS = ["pos", "log_scale", "quat", "opacity", "sh", "evidence", "labels", "fill", "gate", "gate_s", "open"]
WIDTH = dict(pos=3, log_scale=3, quat=4, opacity=1, evidence=7, labels=2, fill=1, gate=2, gate_s=1, open=4)
FLAGS = ["has_scales", "has_evidence", "has_labels", "has_fill", "has_gate", "has_gate_s", "has_open"]


def ref():
    L = C.CDLL(os.path.join(ROOT, "oracle", "_ref", "libb2c_ref.so"))
    p = C.c_void_p
    L.ref_ply_info.argtypes = [C.c_char_p, C.POINTER(C.c_longlong), C.POINTER(C.c_int), C.POINTER(C.c_int), C.c_char_p,
                               C.c_size_t]
    L.ref_ply_read.argtypes = [C.c_char_p, C.POINTER(p), C.c_char_p, C.c_size_t]
    L.ref_ply_write.argtypes = [C.c_char_p, C.c_longlong, C.c_int, C.POINTER(C.c_int), C.POINTER(p), C.c_char_p,
                                C.c_char_p, C.c_size_t]
    L.ref_ply_is_vertex_only.argtypes = [C.c_char_p]
    L.ref_ply_comments.argtypes = [C.c_char_p, C.c_char_p, C.c_size_t]
    return L


def ref_read(L, path):
    n, deg, flags = C.c_longlong(), C.c_int(), (C.c_int * 7)()
    err = C.create_string_buffer(1024)
    if L.ref_ply_info(path.encode(), C.byref(n), C.byref(deg), flags, err, 1024):
        return None, err.value.decode()
    n, deg = n.value, deg.value
    K = (deg + 1) ** 2
    f = dict(zip(FLAGS, [bool(x) for x in flags]))
    arrs = {}
    for k in FIELDS:
        w = 3 * K if k == "sh" else WIDTH[k]
        present = k in ("pos", "log_scale", "quat", "opacity", "sh") or f.get("has_" + k, False)
        arrs[k] = np.zeros((n, w), np.float32) if present else None
    ptrs = (C.c_void_p * 11)(*[a.ctypes.data if a is not None else None for a in arrs.values()])
    if L.ref_ply_read(path.encode(), ptrs, err, 1024):
        return None, err.value.decode()
    out = {k: v for k, v in arrs.items() if v is not None}
    out.update(n=np.int64(n), sh_degree=np.int64(deg), **{k: np.bool_(v) for k, v in f.items()})
    return out, None


def ref_write(L, path, c, comments=()):
    n, deg = c["n"], c["sh_degree"]
    flags = (C.c_int * 7)(0, *[int(k in c) for k in ("evidence", "labels", "fill", "gate", "gate_s", "open")])
    keep = [np.ascontiguousarray(c[k], np.float32) if k in c else None for k in FIELDS]
    ptrs = (C.c_void_p * 11)(*[a.ctypes.data if a is not None else None for a in keep])
    err = C.create_string_buffer(1024)
    cm = "\n".join(comments).encode() if comments else None
    if L.ref_ply_write(path.encode(), n, deg, flags, ptrs, cm, err, 1024):
        raise RuntimeError(err.value.decode())


def cloud(rng, n, deg, blocks=()):
    K = (deg + 1) ** 2
    c = dict(n=n, sh_degree=deg, pos=rng.normal(0, 2, (n, 3)), log_scale=rng.normal(-3, 1, (n, 3)),
             quat=rng.normal(0, 1, (n, 4)), opacity=rng.normal(0, 2, n), sh=rng.normal(0, 0.5, (n, K * 3)))
    if n >= 2:
        c["quat"][0] = 0.0  # a zero quaternion: written as the identity
        c["quat"][1] = [1e-20, 0, 0, 0]
    for b in blocks:
        c[b] = rng.normal(0, 1, (n, WIDTH[b]))
    return {k: (v.astype(np.float32) if isinstance(v, np.ndarray) else v) for k, v in c.items()}


def header(props, n, fmt="binary_little_endian", comments=(), extra_elements=()):
    h = f"ply\nformat {fmt} 1.0\n" + "".join(f"comment {c}\n" for c in comments) + f"element vertex {n}\n"
    h += "".join(f"property {t} {nm}\n" for nm, t in props)
    for name, cnt, line in extra_elements:
        h += f"element {name} {cnt}\n{line}\n"
    return (h + "end_header\n").encode()


NP = {"float": "<f4", "double": "<f8", "uchar": "u1", "char": "i1", "ushort": "<u2", "short": "<i2", "uint": "<u4",
      "int": "<i4", "float32": "<f4", "uint8": "u1", "int16": "<i2", "float64": "<f8"}


def binary_file(path, props, cols, **kw):
    n = len(next(iter(cols.values())))
    dt = np.dtype([(nm, NP[t]) for nm, t in props])
    tab = np.zeros(n, dt)
    for nm, _ in props:
        tab[nm] = cols[nm]
    with open(path, "wb") as f:
        f.write(header(props, n, **kw))
        f.write(tab.tobytes())


def main():
    L = ref()
    os.makedirs(OUT, exist_ok=True)
    rng = np.random.default_rng(20260901)
    expected = {}

    # 1. clouds written by the reference's writer
    for name, n, deg, blocks, comments in (
            ("written_deg3", 120, 3, (), ("SH degree: 3", "trained by the reference writer")),
            ("written_deg0_blocks", 80, 0, ("evidence", "labels", "fill", "gate", "gate_s", "open"), ()),
            ("written_deg4_labels", 60, 4, ("labels",), ("labels: 29 classes",)),
            ("written_deg1_gate_s", 40, 1, ("gate_s",), ()),
            ("written_empty", 0, 2, (), ("empty",))):
        c = cloud(rng, n, deg, blocks)
        path = os.path.join(OUT, name + ".ply")
        ref_write(L, path, c, comments)
        for k, v in c.items():
            expected[f"{name}/in_{k}"] = np.asarray(v)
        expected[f"{name}/comments"] = np.array("\n".join(comments))

    # 2. inputs in the other layouts read_ply accepts
    n = 50
    base = {"x": rng.normal(0, 1, n), "y": rng.normal(0, 1, n), "z": rng.normal(3, 1, n)}
    props = [("x", "double"), ("y", "float"), ("z", "double"), ("scale_0", "float"), ("scale_1", "float"),
             ("scale_2", "float"), ("junk", "uchar"), ("rot_0", "float"), ("rot_1", "float"), ("rot_2", "float"),
             ("rot_3", "float"), ("opacity", "short"), ("f_dc_0", "double"), ("f_dc_1", "float32"),
             ("f_dc_2", "float64"), ("idx", "int")] + [(f"f_rest_{j}", "double" if j % 2 else "float") for j in range(9)]
    cols = dict(base)
    for nm, _ in props:
        if nm not in cols:
            cols[nm] = rng.normal(0, 1, n) if nm != "opacity" else rng.integers(-300, 300, n)
    cols["junk"] = rng.integers(0, 255, n)
    cols["idx"] = rng.integers(-2**31, 2**31 - 1, n)
    binary_file(os.path.join(OUT, "input_mixed_types.ply"), props, cols, comments=("mixed", "types"),
                extra_elements=(("face", 0, "property list uchar int vertex_indices"),))
    # a colour-only point cloud (no scales, rotations or opacity), uchar colours
    props = [("x", "float"), ("y", "float"), ("z", "float"), ("red", "uchar"), ("green", "uchar"), ("blue", "uchar")]
    cols = dict(base, red=rng.integers(0, 256, n), green=rng.integers(0, 256, n), blue=rng.integers(0, 256, n))
    binary_file(os.path.join(OUT, "input_points_rgb8.ply"), props, cols)
    # ushort colours named r, g, b, with normals-style extras and int16 / uint8 optional fields
    props = [("x", "float"), ("y", "float"), ("z", "float"), ("nx", "float"), ("r", "ushort"), ("g", "ushort"),
             ("b", "ushort"), ("seg_label", "uchar"), ("cage_fill", "int16"), ("cage_gate_a", "int"),
             ("cage_gate_b", "int"), ("cage_gate_s", "float")]
    cols = dict(base, nx=rng.normal(0, 1, n), r=rng.integers(0, 65536, n), g=rng.integers(0, 65536, n),
                b=rng.integers(0, 65536, n), seg_label=rng.integers(0, 29, n), cage_fill=rng.integers(-5, 5, n),
                cage_gate_a=rng.integers(-1, 1000, n), cage_gate_b=rng.integers(-1, 1000, n),
                cage_gate_s=rng.random(n))
    binary_file(os.path.join(OUT, "input_points_rgb16.ply"), props, cols)
    # float colours: scale 1
    props = [("x", "float"), ("y", "float"), ("z", "float"), ("red", "float"), ("green", "float"), ("blue", "float"),
             ("scale_0", "float"), ("scale_1", "float"), ("scale_2", "float")]
    cols = dict(base, red=rng.random(n), green=rng.random(n), blue=rng.random(n), scale_0=rng.normal(-3, 1, n),
                scale_1=rng.normal(-3, 1, n), scale_2=rng.normal(-3, 1, n))
    binary_file(os.path.join(OUT, "input_rgb_float.ply"), props, cols)
    # ascii, degree 1, labels without a confidence, open block
    props = [("x", "float"), ("y", "float"), ("z", "float"), ("opacity", "float")] + \
            [(f"f_dc_{k}", "float") for k in range(3)] + [(f"f_rest_{j}", "float") for j in range(9)] + \
            [("seg_label", "float"), ("open_r", "float"), ("open_g", "float"), ("open_b", "float"),
             ("open_dopacity", "float")]
    vals = rng.normal(0, 1, (12, len(props)))
    vals[:, 13] = rng.integers(0, 29, 12)
    with open(os.path.join(OUT, "input_ascii.ply"), "wb") as f:
        f.write(header(props, 12, fmt="ascii", comments=("ascii fixture",)))
        for r in vals:
            f.write((" ".join(repr(float(np.float32(v))) if k % 3 else repr(float(v)) for k, v in enumerate(r)) + "\n").encode())
    # CRLF header lines
    props = [("x", "float"), ("y", "float"), ("z", "float"), ("opacity", "float")]
    cols = dict(base, opacity=rng.normal(0, 1, n))
    binary_file(os.path.join(OUT, "input_crlf.ply"), props, cols)
    raw = open(os.path.join(OUT, "input_crlf.ply"), "rb").read()
    head, body = raw.split(b"end_header\n", 1)
    with open(os.path.join(OUT, "input_crlf.ply"), "wb") as f:
        f.write(head.replace(b"\n", b"\r\n") + b"end_header\r\n" + body)

    # 3. files read_ply rejects
    xyz = [("x", "float"), ("y", "float"), ("z", "float")]
    three = dict(base)
    binary_file(os.path.join(OUT, "bad_big_endian.ply"), xyz, three, fmt="binary_big_endian")
    binary_file(os.path.join(OUT, "bad_face.ply"), xyz, three, extra_elements=(("face", 3, "property list uchar int vertex_indices"),))
    binary_file(os.path.join(OUT, "bad_rest_count.ply"), xyz + [(f"f_rest_{j}", "float") for j in range(4)],
                dict(three, **{f"f_rest_{j}": rng.random(n) for j in range(4)}))
    binary_file(os.path.join(OUT, "bad_no_y.ply"), [("x", "float"), ("z", "float")], three)
    with open(os.path.join(OUT, "bad_type.ply"), "wb") as f:
        f.write(header(xyz + [("w", "half")], 1) + np.zeros(14, np.uint8).tobytes())
    with open(os.path.join(OUT, "bad_list.ply"), "wb") as f:
        f.write(b"ply\nformat binary_little_endian 1.0\nelement vertex 1\nproperty list uchar float x\nend_header\n")
    full = open(os.path.join(OUT, "input_points_rgb8.ply"), "rb").read()
    with open(os.path.join(OUT, "bad_truncated.ply"), "wb") as f:
        f.write(full[:-7])
    with open(os.path.join(OUT, "bad_not_ply.ply"), "wb") as f:
        f.write(b"solid mesh\nendsolid\n")

    # a repeated property name: read_ply's name -> column map keeps the last column of that name
    props = [("x", "float"), ("y", "float"), ("z", "float"), ("opacity", "float"), ("junk", "uchar"),
             ("opacity", "short"), ("x", "double")]
    dup = np.zeros(7, np.dtype([(f"p{k}", NP[t]) for k, (_, t) in enumerate(props)]))
    for k, v in enumerate((np.arange(7) * 0.5, np.arange(7) * -1.0, np.arange(7) + 3.0, np.arange(7) * 0.25,
                           np.arange(7) + 100, np.arange(7) * 7 - 20, np.arange(7) * 1.125 - 4)):
        dup[f"p{k}"] = v
    with open(os.path.join(OUT, "input_duplicate_names.ply"), "wb") as f:
        f.write(header(props, 7))
        f.write(dup.tobytes())
    # files without rows whose optional groups are incomplete: read_ply looks the other members of a group up
    # per row, so it accepts them
    with open(os.path.join(OUT, "input_empty_partial_groups.ply"), "wb") as f:
        f.write(header(xyz + [("scale_0", "float"), ("rot_0", "float"), ("rot_1", "float"), ("f_dc_0", "float"),
                              ("ev_w_in", "float"), ("red", "uchar"), ("cage_gate_a", "float")], 0))
    with open(os.path.join(OUT, "input_empty_red_only.ply"), "wb") as f:
        f.write(header(xyz + [("red", "ushort"), ("seg_conf", "float")], 0))

    for fname in sorted(os.listdir(OUT)):
        if not fname.endswith(".ply"):
            continue
        case = fname[:-4]
        path = os.path.join(OUT, fname)
        got, err = ref_read(L, path)
        if err is not None:
            expected[f"{case}/error"] = np.array(err.replace(OUT + os.sep, ""))  # paths relative to the fixtures
        else:
            for k, v in got.items():
                expected[f"{case}/{k}"] = v
        expected[f"{case}/vertex_only"] = np.bool_(L.ref_ply_is_vertex_only(path.encode()))
        buf = C.create_string_buffer(4096)
        L.ref_ply_comments(path.encode(), buf, 4096)
        expected[f"{case}/read_comments"] = np.array(buf.value.decode("latin-1"))
    np.savez_compressed(os.path.join(OUT, "expected.npz"), **expected)
    print(f"wrote {len([f for f in os.listdir(OUT) if f.endswith('.ply')])} ply fixtures and expected.npz")


if __name__ == "__main__":
    sys.exit(main())
