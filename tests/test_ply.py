"""The ply reader and writer on the host (include/b2c.h b2c_ply_*, replacing src/ply.cpp) and the oracle's
numpy restatement (oracle/ply.py), both against the reference's own reader and writer: the fixtures under
tests/golden/ply/ were written and decoded by the compiled src/ply.cpp (tests/golden/make_ply_golden.py).

Bars: every decoded array bit-identical to the reference's; every written file byte-identical to the
reference writer's for the same cloud; the same files rejected with the reference's messages."""
import os

import numpy as np
import pytest

from b2ctrain_amd import _native as N
from oracle import ply as OP

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "ply")
Z = np.load(os.path.join(GOLD, "expected.npz"), allow_pickle=False)
CASES = sorted({k.split("/")[0] for k in Z.files})
GOOD = [c for c in CASES if f"{c}/error" not in Z.files]
BAD = [c for c in CASES if f"{c}/error" in Z.files]
WRITTEN = [c for c in CASES if c.startswith("written_")]
BLOCKS = ["evidence", "labels", "fill", "gate", "gate_s", "open"]


def _path(case):
    return os.path.join(GOLD, case + ".ply")


def expected(case):
    n = int(Z[f"{case}/n"])
    deg = int(Z[f"{case}/sh_degree"])
    K = (deg + 1) ** 2
    e = dict(n=n, sh_degree=deg, has_scales=bool(Z[f"{case}/has_scales"]))
    for f, w in (("pos", 3), ("log_scale", 3), ("quat", 4)):
        e[f] = Z[f"{case}/{f}"].reshape(n, w)
    e["opacity"] = Z[f"{case}/opacity"].reshape(n)
    e["sh"] = Z[f"{case}/sh"].reshape(n, K, 3)
    for b in BLOCKS:
        if bool(Z[f"{case}/has_{b}"]):
            w = N.PLY_BLOCKS[b]
            e[b] = Z[f"{case}/{b}"].reshape((n, w) if w > 1 else n)
    return e


def assert_cloud_equal(got, want, what):
    assert got["n"] == want["n"] and got["sh_degree"] == want["sh_degree"], what
    assert bool(got["has_scales"]) == want["has_scales"], what
    for f in ("pos", "log_scale", "quat", "opacity", "sh") + tuple(BLOCKS):
        assert (f in got) == (f in want), (what, f)
        if f in want:
            a = np.asarray(got[f], np.float32).reshape(-1).view(np.uint32)
            b = np.asarray(want[f], np.float32).reshape(-1).view(np.uint32)
            assert np.array_equal(a, b), (what, f)


@pytest.mark.parametrize("case", GOOD)
def test_reader_matches_the_reference(case):
    want = expected(case)
    assert_cloud_equal(N.ply_read(_path(case)), want, f"library {case}")
    assert_cloud_equal(OP.read(_path(case)), want, f"oracle {case}")
    info = N.ply_info(_path(case))
    assert info["n"] == want["n"] and info["sh_degree"] == want["sh_degree"]


@pytest.mark.parametrize("case", BAD)
def test_rejects_what_the_reference_rejects(case):
    msg = str(Z[f"{case}/error"])
    with pytest.raises(RuntimeError) as e:
        N.ply_read(_path(case))
    assert str(e.value).endswith(msg.replace("'" + case + ".ply'", "'" + _path(case) + "'")), (str(e.value), msg)
    with pytest.raises(OP.PlyError):
        OP.read(_path(case))


@pytest.mark.parametrize("case", CASES)
def test_vertex_only_and_comments(case):
    assert N.ply_is_vertex_only(_path(case)) == bool(Z[f"{case}/vertex_only"])
    want = str(Z[f"{case}/read_comments"])
    assert N.ply_comments(_path(case)) == (want.split("\n") if want else [])


def _input_cloud(case):
    c = {k[len(case) + 4:]: Z[k] for k in Z.files if k.startswith(f"{case}/in_")}
    c["n"], c["sh_degree"] = int(c["n"]), int(c["sh_degree"])
    comments = str(Z[f"{case}/comments"])
    return c, (comments.split("\n") if comments else [])


@pytest.mark.parametrize("case", WRITTEN)
def test_writer_bytes_match_the_reference(case, tmp_path):
    c, comments = _input_cloud(case)
    ref_bytes = open(_path(case), "rb").read()
    N.ply_write(str(tmp_path / "lib.ply"), c, comments)
    assert open(tmp_path / "lib.ply", "rb").read() == ref_bytes
    OP.write(str(tmp_path / "orc.ply"), c, comments)
    assert open(tmp_path / "orc.ply", "rb").read() == ref_bytes


def test_label_round_trip(tmp_path):
    """tests/tests.cpp:281-290: seg_label / seg_conf survive a write and a read."""
    rng = np.random.default_rng(1)
    n = 300
    c = dict(n=n, sh_degree=2, pos=rng.normal(0, 1, (n, 3)), log_scale=rng.normal(-3, 1, (n, 3)),
             quat=rng.normal(0, 1, (n, 4)), opacity=rng.normal(0, 1, n), sh=rng.normal(0, 1, (n, 9, 3)),
             labels=np.stack([rng.integers(0, 29, n), rng.random(n)], 1))
    N.ply_write(str(tmp_path / "l.ply"), c, ["SH degree: 2"])
    back = N.ply_read(str(tmp_path / "l.ply"))
    assert np.array_equal(back["labels"], c["labels"].astype(np.float32))
    assert N.ply_comments(str(tmp_path / "l.ply")) == ["SH degree: 2"]


def test_oracle_writer_quaternions():
    """write_ply's normalisation: unit length within float rounding, the identity for a zero norm."""
    q = np.array([[0, 0, 0, 0], [2, 0, 0, 0], [1, 1, 1, 1], [1e-30, 0, 0, 0], [3, -4, 0, 12]], np.float32)
    u = OP.unit_quats(q)
    assert np.array_equal(u[0], [1, 0, 0, 0]) and np.array_equal(u[1], [1, 0, 0, 0])
    assert np.array_equal(u[2], [0.5, 0.5, 0.5, 0.5]) and np.array_equal(u[3], [1, 0, 0, 0])
    np.testing.assert_allclose(u[4], np.array([3, -4, 0, 12]) / 13.0, rtol=1e-7)
