"""Pins for each piece of the CPU oracle (oracle/b2c_oracle.c) that do not restate it: published
libraries (numpy, scipy), closed forms, invariants and brute force. A plausible slip in the oracle -- a
wrong SH constant or sign, a transposed rotation, a conic off by a factor, a missed tile, an unstable or
mis-ordered list, a wrong SSIM padding -- fails at least one test here.

| oracle function            | reference (file:line)                 | pinned by                                  |
|----------------------------|---------------------------------------|--------------------------------------------|
| orc_expf / orc_logf        | stand-ins for __expf/__logf           | numpy fp64 exp/log, <= 2 ulp               |
| orc_sh_basis_f/_d          | splat_math.cuh:122-145, reference.cpp:16-30 | scipy sph_harm_y (real, 3DGS sign), quadrature orthonormality |
| orc_quat_to_mat            | util.cuh:235-243                      | scipy Rotation, R R^T = I, det = 1         |
| orc_tile_hit               | splat_math.cuh:27-41                  | exact min of the quadratic over the box    |
| orc_project                | project.cu:8-84, splat_math.cuh:224-293 | numpy fp64 EWA with a numerical Jacobian |
| orc_bin                    | binning.cu:10-143                     | sortedness, stability, counts, no missed pixel-centre hit |
| orc_raster_fwd             | raster_fwd.cu:8-71                    | fp64 brute force (pinned to the reference by the golden fixtures), also with splats centred on pixel centres |
| orc_photometric            | loss.cu:18-195, reference.cpp:106-131 | scipy.ndimage separable blur (zero padding); FD of v_out |
| orc_raster_bwd + orc_vjp   | raster_bwd.cu, optim.cu:99-296        | reference FD fixtures (test_oracle_golden.py) |
"""
import math

import numpy as np
import pytest
from scipy import ndimage
from scipy.spatial.transform import Rotation

from b2ctrain_amd import scenes as S
from oracle import oracle as O


# ---------------------------------------------------------------------------------------------- exp / log
def _ulp_err(got, want64):
    want32 = want64.astype(np.float32)
    ulp = np.spacing(np.abs(want32)).astype(np.float64)
    return np.abs(got.astype(np.float64) - want64) / ulp


def test_expf_within_two_ulp():
    x = np.concatenate([np.linspace(-86, 88, 20001), np.random.default_rng(1).uniform(-20, 20, 5000)]).astype(np.float32)
    got = np.array([O.expf(float(v)) for v in x], np.float32)
    err = _ulp_err(got, np.exp(x.astype(np.float64)))
    assert err.max() <= 2.0, float(err.max())
    assert O.expf(-100.0) == 0.0 and math.isinf(O.expf(100.0))


def test_logf_within_two_ulp():
    x = np.exp(np.random.default_rng(2).uniform(-60, 60, 20000)).astype(np.float32)
    x = np.concatenate([x, np.float32([1.0, 255.0, 1.0 / 255.0, 0.7071, 1.4142])])
    got = np.array([O.logf(float(v)) for v in x], np.float32)
    want = np.log(x.astype(np.float64))
    err = np.abs(got - want) / np.maximum(np.spacing(np.abs(want.astype(np.float32))), 1e-45)
    assert err.max() <= 2.0, float(err.max())
    assert O.logf(1.0) == 0.0


# ---------------------------------------------------------------------------------------------- SH basis
def _real_sh_3dgs(l, m, d):
    """Real SH in the 3DGS sign convention from scipy's complex Y_l^m (Condon-Shortley phase):
    m < 0: sqrt2 Im Y_l^|m|, m = 0: Y_l^0, m > 0: sqrt2 Re Y_l^m, evaluated at unit vector d."""
    from scipy.special import sph_harm_y
    theta = math.acos(max(-1.0, min(1.0, d[2])))
    phi = math.atan2(d[1], d[0])
    y = sph_harm_y(l, abs(m), theta, phi)
    if m < 0:
        return math.sqrt(2) * y.imag
    if m == 0:
        return y.real
    return math.sqrt(2) * y.real


@pytest.mark.parametrize("deg", [0, 1, 2, 3, 4])
def test_sh_basis_matches_scipy(deg):
    rng = np.random.default_rng(deg)
    for _ in range(40):
        d = rng.normal(size=3)
        d /= np.linalg.norm(d)
        want = np.array([_real_sh_3dgs(l, m, d) for l in range(deg + 1) for m in range(-l, l + 1)])
        got_f = O.sh_basis(deg, d)
        got_d = O.sh_basis(deg, d, double=True)
        # constants are printed to 7-8 significant digits in the reference
        assert np.allclose(got_f, want, atol=2e-6), (deg, got_f - want)
        assert np.allclose(got_d, want, atol=1e-6), (deg, got_d - want)


def test_sh_basis_orthonormal():
    xg, wg = np.polynomial.legendre.leggauss(24)  # cos(theta) nodes
    nphi = 48
    phis = np.arange(nphi) * 2 * np.pi / nphi
    G = np.zeros((25, 25))
    for ct, w in zip(xg, wg):
        st = math.sqrt(1 - ct * ct)
        for ph in phis:
            b = O.sh_basis(4, (st * math.cos(ph), st * math.sin(ph), ct), double=True)
            G += np.outer(b, b) * w * (2 * np.pi / nphi)
    assert np.abs(G - np.eye(25)).max() < 2e-6, np.abs(G - np.eye(25)).max()


# ---------------------------------------------------------------------------------------------- rotation
def test_quat_to_mat_matches_scipy():
    rng = np.random.default_rng(3)
    for _ in range(200):
        q = rng.normal(size=4)
        q /= np.linalg.norm(q)
        R = O.quat_to_mat(q.astype(np.float32))
        want = Rotation.from_quat([q[1], q[2], q[3], q[0]]).as_matrix()  # scipy is (x, y, z, w)
        assert np.allclose(R, want, atol=2e-6)
        assert np.allclose(R @ R.T, np.eye(3), atol=2e-6) and abs(np.linalg.det(R) - 1) < 2e-6
    # quarter turn about z maps x to y
    c = math.sqrt(0.5)
    assert np.allclose(O.quat_to_mat(np.float32([c, 0, 0, c])) @ [1, 0, 0], [0, 1, 0], atol=1e-6)


# ---------------------------------------------------------------------------------------------- tile hit
def _min_sigma_over_box(x0, y0, x1, y1, mx, my, c00, c01, c11):
    """Exact minimum of 0.5 (c00 dx^2 + c11 dy^2) + c01 dx dy over the box (fp64)."""
    def sig(x, y):
        dx, dy = x - mx, y - my
        return 0.5 * (c00 * dx * dx + c11 * dy * dy) + c01 * dx * dy
    if x0 <= mx <= x1 and y0 <= my <= y1:
        return 0.0
    best = math.inf
    for x in (x0, x1):  # vertical edges: minimise over y
        y = min(max(my - c01 * (x - mx) / c11, y0), y1)
        best = min(best, sig(x, y))
    for y in (y0, y1):
        x = min(max(mx - c01 * (y - my) / c00, x0), x1)
        best = min(best, sig(x, y))
    return best


def test_tile_hit_is_the_exact_box_test():
    rng = np.random.default_rng(4)
    decided = 0
    for _ in range(20000):
        a, b = rng.uniform(0.002, 2.0, 2)
        th = rng.uniform(0, np.pi)
        cth, sth = math.cos(th), math.sin(th)
        c00 = a * cth * cth + b * sth * sth
        c11 = a * sth * sth + b * cth * cth
        c01 = (a - b) * cth * sth
        mx, my = rng.uniform(-40, 56, 2)
        power = rng.uniform(0.01, 5.5)
        x0, y0 = 8.0 * rng.integers(0, 2), 8.0 * rng.integers(0, 2)
        x1, y1 = x0 + 8.0, y0 + 8.0
        m = _min_sigma_over_box(x0, y0, x1, y1, mx, my, c00, c01, c11)
        hit = O.tile_hit((x0, y0, x1, y1), (mx, my), (c00, c01, c11), power)
        if m < power * (1 - 1e-4):
            assert hit, (mx, my, c00, c01, c11, power, m)
            decided += 1
        elif m > power * (1 + 1e-4):
            assert not hit, (mx, my, c00, c01, c11, power, m)
            decided += 1
    assert decided > 19000


# ---------------------------------------------------------------------------------------------- projection
def _ewa_numpy(scene, camd):
    """Independent fp64 EWA projection: per-axis scale sqrt(exp(2 l) + f^2) with the Mip-Splatting floor f
    and the opacity factor sqrt(prod exp(2 l) / prod (exp(2 l) + f^2)) (splat_math.cuh:232-237), cov3d =
    R S S R^T, the Jacobian of the pinhole map by central differences at the centre with its tangent
    clamped to 15% past the frame (render.h:21-22: the clamped Jacobian is the pinhole map's Jacobian at
    the clamped point), cov2d = J W cov3d W^T J^T + 0.3 I."""
    Rv = np.asarray(camd["R"], np.float64).reshape(3, 3)
    t = np.asarray(camd["t"], np.float64)
    fx, fy, cx, cy = (float(camd[k]) for k in ("fx", "fy", "cx", "cy"))
    lim = [float(camd[k]) for k in ("lim_neg_x", "lim_pos_x", "lim_neg_y", "lim_pos_y")]
    out = []
    for i in range(scene.n):
        p = scene.pos_op[i, :3].astype(np.float64)
        mc = Rv @ p + t
        q = scene.quat[i].astype(np.float64)
        Rq = Rotation.from_quat([q[1], q[2], q[3], q[0]]).as_matrix()
        var = np.exp(2.0 * scene.lscale[i, :3].astype(np.float64))
        f2 = float(scene.lscale[i, 3]) ** 2
        cov3 = Rq @ np.diag(var + f2) @ Rq.T
        comp = math.sqrt(np.prod(var) / np.prod(var + f2))
        f = lambda v: np.array([fx * v[0] / v[2] + cx, fy * v[1] / v[2] + cy])
        at = np.array([np.clip(mc[0] / mc[2], lim[0], lim[1]) * mc[2], np.clip(mc[1] / mc[2], lim[2], lim[3]) * mc[2], mc[2]])
        h = 1e-6 * mc[2]
        J = np.stack([(f(at + h * e) - f(at - h * e)) / (2 * h) for e in np.eye(3)], 1)
        cov2 = J @ Rv @ cov3 @ Rv.T @ J.T + 0.3 * np.eye(2)
        conic = np.linalg.inv(cov2)
        op = comp / (1 + math.exp(-float(scene.pos_op[i, 3])))
        d = p - np.asarray(camd["pos"], np.float64)
        d /= np.linalg.norm(d)
        basis = np.array([_real_sh_3dgs(l, m, d) for l in range(scene.degree + 1) for m in range(-l, l + 1)])
        col = np.clip(basis @ scene.sh[i].astype(np.float64) + 0.5, -100, 100)
        out.append((f(mc), conic, op, mc[2], col, mc))
    return out


@pytest.mark.parametrize("make", [lambda: S.config1(), lambda: S.fd_scene(1236, degree=3), lambda: S.config2(n=300),
                                  lambda: S.fd_scene(1238, floor=True), lambda: S.fd_scene(1239, degree=4),
                                  lambda: S.clamp_scene(1240)],
                         ids=["cfg1", "fd1236", "cfg2", "floor", "sh4", "clamp"])
def test_projection_matches_numpy_ewa(make):
    sc = make()
    camd = S.camera_gpu(sc.cam)
    pr = O.project(sc, camd)
    ref = _ewa_numpy(sc, camd)
    checked = clamped = 0
    for i, (m2, conic, op, z, col, mc) in enumerate(ref):
        if pr["tile_count"][i] == 0:
            continue
        rx, ry = mc[0] / mc[2], mc[1] / mc[2]
        clamped += not (camd["lim_neg_x"] < rx < camd["lim_pos_x"] and camd["lim_neg_y"] < ry < camd["lim_pos_y"])
        p0, p1, p2 = pr["proj0"][i], pr["proj1"][i], pr["proj2"][i]
        assert np.allclose(p0[:2], m2, rtol=1e-5, atol=1e-3)
        got = np.array([[p0[2], p0[3]], [p0[3], p1[0]]])
        assert np.allclose(got, conic, rtol=1e-3, atol=1e-6 * np.abs(conic).max()), (i, got, conic)
        assert abs(p1[1] - op) < 1e-6 and abs(p1[2] - z) < 1e-5 * z
        assert abs(p1[3] - math.log(255 * op)) < 1e-5
        assert np.allclose(p2[:3], col, atol=1e-5)
        checked += 1
    assert checked >= 10
    if sc.name.startswith("clamp"):
        assert clamped >= 8  # the clamped Jacobian is what is being checked
    if sc.lscale[:, 3].any():
        assert (pr["proj1"][pr["tile_count"] > 0, 1] < 1 / (1 + np.exp(-sc.pos_op[pr["tile_count"] > 0, 3])) * 0.999).all()


# ---------------------------------------------------------------------------------------------- binning
@pytest.mark.parametrize("make", [lambda: S.config1(), lambda: S.config2(n=3000), lambda: S.config5(n=2000)])
def test_binning_invariants_and_no_missed_hits(make):
    sc = make()
    camd = S.camera_gpu(sc.cam)
    W, H = sc.W, sc.H
    tx, ty, T, bits = O.tile_geometry(W, H)
    pr = O.project(sc, camd)
    bn = O.bin_(pr, W, H)
    keys, vals, M = bn["keys_sorted"], bn["vals_sorted"], bn["M"]
    assert M == int(pr["tile_count"].sum())
    assert np.all(np.diff(keys.astype(np.int64)) >= 0)
    assert keys.max(initial=0) <= T  # T = sentinel for emitted shortfall
    # each splat appears tile_count times, each (tile, splat) once
    assert np.array_equal(np.bincount(vals, minlength=sc.n), pr["tile_count"].astype(np.int64))
    pairs = keys.astype(np.int64) * sc.n + vals
    assert len(np.unique(pairs)) == M
    # within a tile: ordered by (depth bits, splat index) -- the stable two-pass order
    zbits = pr["proj1"][:, 2].copy().view(np.uint32).astype(np.int64)
    k = zbits[vals] * (1 << 32) + vals
    same = keys[1:] == keys[:-1]
    assert np.all(np.diff(k)[same] > 0)
    # ranges cover exactly the tile's entries; absent tiles are (0, 0)
    rng_ = bn["tile_ranges"].astype(np.int64)
    first = np.searchsorted(keys, np.arange(T), "left")
    last = np.searchsorted(keys, np.arange(T), "right")
    present = last > first
    assert np.array_equal(rng_[present, 0], first[present]) and np.array_equal(rng_[present, 1], last[present])
    assert not rng_[~present].any()
    # every pixel centre at sigma <= power (fp64, margin 1e-4) lies in a listed tile of that splat
    listed = set(pairs.tolist())
    rng = np.random.default_rng(5)
    for i in np.flatnonzero(pr["tile_count"]):
        p0, p1 = pr["proj0"][i].astype(np.float64), pr["proj1"][i].astype(np.float64)
        detc = p0[2] * p1[0] - p0[3] ** 2
        ex, ey = math.sqrt(2 * p1[3] * p1[0] / detc) + 2, math.sqrt(2 * p1[3] * p0[2] / detc) + 2
        x0, x1 = max(0, int(p0[0] - ex)), min(W, int(p0[0] + ex) + 1)
        y0, y1 = max(0, int(p0[1] - ey)), min(H, int(p0[1] + ey) + 1)
        if x1 <= x0 or y1 <= y0:
            continue
        if (x1 - x0) * (y1 - y0) <= 200_000:
            py, px = np.mgrid[y0:y1, x0:x1]
            px, py = px.ravel(), py.ravel()
        else:  # huge splats: a random sample of their pixels
            px, py = rng.integers(x0, x1, 200_000), rng.integers(y0, y1, 200_000)
        dx, dy = px + 0.5 - p0[0], py + 0.5 - p0[1]
        sig = 0.5 * (p0[2] * dx * dx + p1[0] * dy * dy) + p0[3] * dx * dy
        hit = sig <= p1[3] * (1 - 1e-4)
        for t in np.unique((py[hit] // 8) * tx + px[hit] // 8):
            assert int(t) * sc.n + int(i) in listed, (i, t)


# ---------------------------------------------------------------------------------------------- forward
@pytest.mark.parametrize("make", [lambda: S.config1(), lambda: S.fd_scene(1235, masked=True)])
def test_forward_fp32_tiled_vs_fp64_brute_force(make):
    sc = make()
    sc.bg = (0.25, 0.5, 0.75)
    out = O.pipeline(sc)
    _, img = O.ref_loss(sc, want_img=True)
    err = np.abs(out["fwd"]["out_rgba"] - img).max()
    assert err <= 1e-4, err


# ---------------------------------------------------------------------------------------------- loss
def _photometric_numpy(sc, pred, bg):
    """Independent fp64 L1 + SSIM + alpha lane: scipy separable 11-tap Gaussian (sigma 1.5), zero padding."""
    W, H = sc.W, sc.H
    g = np.exp(-((np.arange(11) - 5.0) ** 2) / (2 * 1.5 ** 2))
    g /= g.sum()
    blur = lambda a: ndimage.correlate1d(ndimage.correlate1d(a, g, axis=1, mode="constant"), g, axis=0, mode="constant")
    byte = np.stack([(sc.gt >> (8 * c)) & 0xFF for c in range(4)], 1)
    gt = byte.astype(np.float64) / 255.0
    # the kernel decodes the target in fp32 (loss.cu:58, multiply by 1/255) and composites it in fp32
    g32 = byte.astype(np.float32) * np.float32(1.0 / 255.0)
    wp = sc.weights.astype(np.float64) / 255.0 if sc.weights is not None else np.ones(W * H)
    # LossParams holds float32 weights (loss.h:20-30)
    l1_w, ssim_w, match, scale = (float(np.float32(v)) for v in (sc.l1_w, sc.ssim_w, sc.match_alpha_weight, sc.scale))
    loss = 0.0
    for c in range(3):
        X = pred[:, c].astype(np.float64).reshape(H, W)
        Yc = g32[:, c] + (np.float32(1) - g32[:, 3]) * np.float32(bg[c]) if sc.composite else g32[:, c]
        Y = Yc.astype(np.float64).reshape(H, W)
        mu1, mu2 = blur(X), blur(Y)
        s1 = np.maximum(blur(X * X) - mu1 ** 2, 0)
        s2 = np.maximum(blur(Y * Y) - mu2 ** 2, 0)
        s12 = blur(X * Y) - mu1 * mu2
        ssim = np.clip((2 * mu1 * mu2 + 1e-4) * (2 * s12 + 9e-4) / ((mu1 ** 2 + mu2 ** 2 + 1e-4) * (s1 + s2 + 9e-4)), -1, 1)
        M = wp.reshape(H, W) * (gt[:, 3].reshape(H, W) if sc.mask else 1.0) * scale / (3 * W * H)
        loss += (M * (l1_w * np.abs(X - Y) + ssim_w * ssim)).sum()
    if sc.alpha_lane:
        da = (pred[:, 3] - g32[:, 3]).astype(np.float64)  # fp32 difference, as the kernel forms it
        loss += (wp * match * scale / (W * H) * np.abs(da)).sum()
    return loss


@pytest.mark.parametrize("seed,masked", [(1234, False), (1235, True)])
def test_photometric_value_and_gradient(seed, masked):
    sc = S.fd_scene(seed, masked=masked)
    rng = np.random.default_rng(seed)
    pred = rng.uniform(0, 1, (sc.W * sc.H, 4)).astype(np.float32)
    loss, v = O.photometric(sc, pred, grad_scale=1.0)
    want = _photometric_numpy(sc, pred, sc.bg)
    assert abs(loss - want) <= 1e-9 * abs(want), (loss, want)
    # v_out against central differences of the independent loss at random pixels/channels
    for _ in range(40):
        p, c = int(rng.integers(sc.W * sc.H)), int(rng.integers(4))
        if c == 3 and not sc.alpha_lane:
            continue
        h = 1e-4
        a, b = pred.astype(np.float64), pred.astype(np.float64)
        a[p, c] += h
        b[p, c] -= h
        fd = (_photometric_numpy(sc, a, sc.bg) - _photometric_numpy(sc, b, sc.bg)) / (2 * h)
        assert abs(v[p, c] - fd) <= 2e-3 * abs(fd) + 1e-9, (p, c, v[p, c], fd)


@pytest.mark.parametrize("seed", [3, 11])
def test_forward_keeps_fragments_at_the_splat_centre(seed):
    """At a pixel centre on a splat's centre the exact sigma is 0. The tiled raster's sigma (the quadratic
    about the tile centre) rounds there to a small value of either sign (about half of such pixels come out
    below 0): the fragment passes when sigma <= power, as the exact value does, so the render equals the
    fp64 brute force. A rule that also rejected sigma < 0 would drop those centre fragments (alpha 0.5 ..
    0.95 of the pixel's colour)."""
    sc = S.pixel_centred_scene(seed)
    sc.bg = (0.25, 0.5, 0.75)
    out = O.pipeline(sc)
    p0 = out["proj"]["proj0"]
    vis = out["proj"]["tile_count"] > 0
    assert vis.sum() == sc.n
    # the centres really are pixel centres, and the quadratic rounds some of them below 0
    assert np.array_equal(p0[:, 0] - np.floor(p0[:, 0]), np.full(sc.n, 0.5, np.float32))
    assert np.array_equal(p0[:, 1] - np.floor(p0[:, 1]), np.full(sc.n, 0.5, np.float32))
    sig = O.frag_sigma(p0[:, 0], p0[:, 1], p0[:, 2], p0[:, 3], out["proj"]["proj1"][:, 0], p0[:, 0], p0[:, 1])
    assert (sig < 0).any() and (np.abs(sig) < 1e-4).all()
    _, img = O.ref_loss(sc, want_img=True)
    err = np.abs(out["fwd"]["out_rgba"] - img).max()
    assert err <= 1e-4, err
