"""TEST INFRASTRUCTURE ONLY: a numpy restatement of the reference's ply reader and writer (src/ply.cpp), the
checker of this build's host and device-direct ply paths. Pinned by the reference's own reader and writer
(tests/golden/ply/, written by tests/golden/make_ply_golden.py from the compiled src/ply.cpp): every fixture
decodes to the reference's arrays bit for bit and every cloud encodes to the reference writer's bytes.

A cloud is a dict: n, sh_degree, pos [n][3], log_scale [n][3], quat [n][4] (w, x, y, z), opacity [n],
sh [n][K][3], has_scales, and for each optional block present its array: evidence [n][7], labels [n][2],
fill [n], gate [n][2], gate_s [n], open [n][4] (float32 throughout)."""
from __future__ import annotations

import math

import numpy as np

SH_C0 = np.float32(0.28209479177387814)
# ply.cpp:27-36
_TYPES = {"float": "<f4", "float32": "<f4", "double": "<f8", "float64": "<f8", "uchar": "u1", "uint8": "u1",
          "char": "i1", "int8": "i1", "ushort": "<u2", "uint16": "<u2", "short": "<i2", "int16": "<i2",
          "uint": "<u4", "uint32": "<u4", "int": "<i4", "int32": "<i4"}
EVIDENCE_FIELDS = ["ev_w_in", "ev_w_all", "ev_err", "ev_views", "ev_dir_0", "ev_dir_1", "ev_dir_2"]
LABEL_FIELDS = ["seg_label", "seg_conf"]
BLOCKS = [("evidence", EVIDENCE_FIELDS), ("labels", LABEL_FIELDS), ("fill", ["cage_fill"]),
          ("gate", ["cage_gate_a", "cage_gate_b"]), ("gate_s", ["cage_gate_s"]),
          ("open", ["open_r", "open_g", "open_b", "open_dopacity"])]


class PlyError(ValueError):
    pass


def parse_header(path):
    """ply.cpp:88-110: format, vertex count, the vertex properties (name, numpy type), data offset."""
    with open(path, "rb") as f:
        first = f.readline()
        if not first.startswith(b"ply"):
            raise PlyError(f"'{path}' is not a ply file")
        binary = big = in_vertex = False
        n, props = 0, []
        while True:
            raw = f.readline()
            if not raw:
                break
            line = raw.rstrip(b"\n").rstrip(b"\r").decode("latin-1")
            tok = line.split()
            if not tok:
                continue
            if tok[0] == "format":
                binary = tok[1] != "ascii"
                big = tok[1] == "binary_big_endian"
            elif tok[0] == "element":
                in_vertex = tok[1] == "vertex"
                cnt = int(tok[2])
                if in_vertex:
                    n = cnt
                elif cnt > 0:
                    raise PlyError(f"ply: unsupported non-vertex element '{tok[1]}'")
            elif tok[0] == "property" and in_vertex:
                if tok[1] == "list":
                    raise PlyError("ply: list properties are not supported on vertices")
                if tok[1] not in _TYPES:
                    raise PlyError(f"ply: unsupported property type '{tok[1]}'")
                props.append((tok[2], _TYPES[tok[1]]))
            elif tok[0] == "end_header":
                break
        offset = f.tell()
    if big:
        raise PlyError("ply: big-endian files are not supported")
    return dict(binary=binary, n=n, props=props, offset=offset)


class _EmptyColumns(dict):
    """Columns of a file with no rows: a name the header lacks reads as an empty column."""

    def __missing__(self, key):
        return np.zeros(0, np.float64)


def read(path):
    h = parse_header(path)
    names = [p[0] for p in h["props"]]
    n = h["n"]
    if h["binary"]:
        dt = np.dtype([(f"p{k}", t) for k, (_, t) in enumerate(h["props"])])
        with open(path, "rb") as f:
            f.seek(h["offset"])
            raw = f.read(n * dt.itemsize)
        if len(raw) < n * dt.itemsize:
            raise PlyError(f"ply: truncated file '{path}'")
        table = np.frombuffer(raw, dt, n)
        # a repeated name resolves to its last column, as read_ply's name -> column map does (ply.cpp:96-97)
        col = {nm: table[f"p{k}"].astype(np.float64) for k, nm in enumerate(names)}
    else:
        with open(path, "rb") as f:
            f.seek(h["offset"])
            vals = f.read().split()
        if len(vals) < n * len(names):
            raise PlyError(f"ply: truncated ascii file '{path}'")
        arr = np.array([float(v) for v in vals[: n * len(names)]], np.float64).reshape(n, len(names))
        col = {nm: arr[:, k] for k, nm in enumerate(names)}
    if n == 0:  # read_ply looks members up per row: a file without rows needs none beyond the flags' first
        col = _EmptyColumns(col)
    has = col.__contains__
    n_rest = 0
    while has(f"f_rest_{n_rest}"):
        n_rest += 1
    K = 1 + n_rest // 3
    deg = int(round(math.sqrt(K))) - 1
    if (deg + 1) ** 2 != K:
        raise PlyError(f"ply: {n_rest} f_rest properties is not a valid SH layout")
    if not (has("x") and has("y") and has("z")):
        raise PlyError("ply: missing x/y/z")

    def f32(a):
        return np.asarray(a, np.float64).astype(np.float32)

    c = dict(n=n, sh_degree=deg)
    c["pos"] = np.stack([f32(col[k]) for k in "xyz"], 1) if n else np.zeros((0, 3), np.float32)
    c["has_scales"] = has("scale_0")
    c["log_scale"] = (np.stack([f32(col[f"scale_{k}"]) for k in range(3)], 1) if c["has_scales"]
                      else np.zeros((n, 3), np.float32))
    c["quat"] = (np.stack([f32(col[f"rot_{k}"]) for k in range(4)], 1) if has("rot_0")
                 else np.tile(np.array([1, 0, 0, 0], np.float32), (n, 1)))
    c["opacity"] = f32(col["opacity"]) if has("opacity") else np.zeros(n, np.float32)
    sh = np.zeros((n, K, 3), np.float32)
    rgb = has("red") or has("r")
    if has("f_dc_0"):
        for ch in range(3):
            sh[:, 0, ch] = f32(col[f"f_dc_{ch}"])
    elif rgb:
        rn = "red" if has("red") else "r"
        t = dict(h["props"])[rn]
        scale = 1.0 / 255.0 if t == "u1" else (1.0 / 65535.0 if t == "<u2" else 1.0)
        for ch, (a, b) in enumerate((("red", "r"), ("green", "g"), ("blue", "b"))):
            sh[:, 0, ch] = f32((col[a if has(a) else b] * scale - 0.5) / np.float64(SH_C0))
    for ch in range(3):
        for k in range(1, K):
            sh[:, k, ch] = f32(col[f"f_rest_{ch * (K - 1) + (k - 1)}"])
    c["sh"] = sh
    if has("ev_w_in"):
        c["evidence"] = np.stack([f32(col[e]) for e in EVIDENCE_FIELDS], 1)
    if has("seg_label"):
        conf = f32(col["seg_conf"]) if has("seg_conf") else np.ones(n, np.float32)
        c["labels"] = np.stack([f32(col["seg_label"]), conf], 1)
    if has("cage_fill"):
        c["fill"] = f32(col["cage_fill"])
    if has("cage_gate_a") and has("cage_gate_b"):
        c["gate"] = np.stack([f32(col["cage_gate_a"]), f32(col["cage_gate_b"])], 1)
        if has("cage_gate_s"):
            c["gate_s"] = f32(col["cage_gate_s"])
    if all(has(k) for k in ("open_r", "open_g", "open_b", "open_dopacity")):
        c["open"] = np.stack([f32(col[k]) for k in ("open_r", "open_g", "open_b", "open_dopacity")], 1)
    return c


def unit_quats(q):
    """write_ply's quaternion (ply.cpp:199-201): q / sqrt(((w^2 + x^2) + y^2) + z^2) in float32, the identity
    when that norm is not above 1e-32."""
    q = np.asarray(q, np.float32)
    w, x, y, z = (q[:, k] for k in range(4))
    qn = np.sqrt(((w * w + x * x) + y * y) + z * z)
    bad = ~(qn > np.float32(1e-32))
    out = q / np.where(bad, np.float32(1), qn)[:, None]
    out[bad] = np.array([1, 0, 0, 0], np.float32)
    return out.astype(np.float32)


def rows(c):
    """The float32 rows write_ply emits (ply.cpp:193-219) and the property names of its header."""
    n, K = c["n"], (c["sh_degree"] + 1) ** 2
    names = ["x", "y", "z", "scale_0", "scale_1", "scale_2", "opacity", "rot_0", "rot_1", "rot_2", "rot_3",
             "f_dc_0", "f_dc_1", "f_dc_2"] + [f"f_rest_{j}" for j in range(3 * (K - 1))]
    sh = np.asarray(c["sh"], np.float32).reshape(n, K, 3)
    parts = [np.asarray(c["pos"], np.float32).reshape(n, 3), np.asarray(c["log_scale"], np.float32).reshape(n, 3),
             np.asarray(c["opacity"], np.float32).reshape(n, 1), unit_quats(np.asarray(c["quat"]).reshape(n, 4)),
             sh[:, 0, :], sh[:, 1:, :].transpose(0, 2, 1).reshape(n, 3 * (K - 1))]
    for key, fields in BLOCKS:
        if key in c:
            names += fields
            parts.append(np.asarray(c[key], np.float32).reshape(n, len(fields)))
    return np.concatenate(parts, 1).astype("<f4"), names


def write(path, c, comments=()):
    table, names = rows(c)
    head = "ply\nformat binary_little_endian 1.0\n" + "".join(f"comment {cm}\n" for cm in comments)
    head += f"element vertex {c['n']}\n" + "".join(f"property float {nm}\n" for nm in names) + "end_header\n"
    with open(path, "wb") as f:
        f.write(head.encode())
        f.write(np.ascontiguousarray(table).tobytes())
