"""Synthetic scenes for the five BASELINE.json configurations and for the reference's FD-harness scene.

Every scene is a plain bundle of numpy arrays in the layouts the C ABI takes:

* ``pos_op``  [n][4] f32  (x, y, z, opacity logit)              -- Model::pos_op, src/model.h:8-23
* ``quat``    [n][4] f32  (w, x, y, z), unnormalised            -- Model::quat
* ``lscale``  [n][4] f32  (log sx, log sy, log sz, floor f)     -- Model::lscale (floor 0 = none)
* ``sh``      [n][K][3] f32 coefficient-major (SplatCloud order, src/ply.h); when ``sh_fp16`` the bands
  above DC are already rounded to fp16 (round to nearest even), which is what Model::upload stores
  (src/model.cu:66-71).
* ``gt``      [H*W] u32 packed RGBA8 ``r | g<<8 | b<<16 | a<<24`` (premultiplied for transparent views,
  src/dataset/views.cpp:178-183), ``weights`` [H*W] u8 or None.

Random numbers come from numpy's PCG64 generator seeded with ``0xB2C0 + config``. Data is synthetic; no
dataset or checkpoint is read.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np

SH_C0 = 0.28209479177387814


@dataclass
class Camera:
    """Pinhole camera, world->camera R (row major) and t; OpenCV axes (+x right, +y down, +z forward).

    Mirrors b2c::Camera (src/dataset/camera.h:8-36)."""

    width: int
    height: int
    fx: float
    fy: float
    cx: float
    cy: float
    R: np.ndarray  # (9,) f32
    t: np.ndarray  # (3,) f32

    @property
    def pos(self) -> np.ndarray:
        R = self.R.reshape(3, 3).astype(np.float32)
        t = self.t.astype(np.float32)
        # pos = -R^T t, evaluated in float like Camera::update_pos (camera.h:24-29)
        out = np.zeros(3, np.float32)
        for i in range(3):
            out[i] = -(R[0, i] * t[0] + R[1, i] * t[1] + R[2, i] * t[2])
        return out


def camera_gpu(cam: Camera, W: int | None = None, H: int | None = None) -> dict:
    """CameraGPU::from (src/gpu/render.h:15-24) in float32 arithmetic."""
    W = cam.width if W is None else W
    H = cam.height if H is None else H
    f = np.float32
    sx = f(W) / f(cam.width)
    sy = f(H) / f(cam.height)
    fx, fy, cx, cy = f(cam.fx) * sx, f(cam.fy) * sy, f(cam.cx) * sx, f(cam.cy) * sy
    return dict(
        R=cam.R.astype(np.float32).copy(), t=cam.t.astype(np.float32).copy(), pos=cam.pos,
        fx=fx, fy=fy, cx=cx, cy=cy, W=W, H=H,
        lim_pos_x=(f(1.15) * f(W) - cx) / fx, lim_pos_y=(f(1.15) * f(H) - cy) / fy,
        lim_neg_x=(f(-0.15) * f(W) - cx) / fx, lim_neg_y=(f(-0.15) * f(H) - cy) / fy,
    )


@dataclass
class Scene:
    name: str
    degree: int
    pos_op: np.ndarray
    quat: np.ndarray
    lscale: np.ndarray
    sh: np.ndarray
    cam: Camera
    gt: np.ndarray
    weights: np.ndarray | None = None
    sh_fp16: bool = False
    # LossParams (src/gpu/loss.h:20-30)
    l1_w: float = 0.8
    ssim_w: float = -0.2
    composite: bool = False
    mask: bool = False
    alpha_lane: bool = False
    match_alpha_weight: float = 0.1
    scale: float = 1.0
    bg: tuple = (0.0, 0.0, 0.0)
    extra_cams: list = field(default_factory=list)
    # feature lanes and the losses on them (render.h:27-63, loss.h:20-30)
    feat_mode: int = 0                 # 0 none, 1 pseudo-normals, 2 feat_buffer
    feat_buffer: np.ndarray | None = None  # [n][3] float32 with feat_mode 2
    normals: np.ndarray | None = None  # [P] packed RGBA8 normal map (ViewGPU::normals)
    normal_scale: float = 0.0          # normal_loss weight
    hollow_z: np.ndarray | None = None  # [P] float32 reference surface depth (+inf = none)
    hollow_margin: float = 0.05
    hollow_lam: float = 0.0

    @property
    def n(self) -> int:
        return self.pos_op.shape[0]

    @property
    def K(self) -> int:
        return (self.degree + 1) ** 2

    @property
    def W(self) -> int:
        return self.cam.width

    @property
    def H(self) -> int:
        return self.cam.height

    def subset(self, n: int) -> "Scene":
        """First n splats of the scene (same camera, target and loss options)."""
        s = Scene(**{k: getattr(self, k) for k in self.__dataclass_fields__})
        s.pos_op, s.quat, s.lscale, s.sh = (a[:n].copy() for a in (self.pos_op, self.quat, self.lscale, self.sh))
        s.name = f"{self.name}[:{n}]"
        return s

    def with_camera(self, cam: Camera) -> "Scene":
        s = Scene(**{k: getattr(self, k) for k in self.__dataclass_fields__})
        s.cam = cam
        return s


def _rand_quat(rng, n):
    # Shoemake's uniform random rotation (K. Shoemake, "Uniform random rotations", Graphics Gems III)
    u1, u2, u3 = rng.random(n), rng.random(n), rng.random(n)
    a, b = np.sqrt(1 - u1), np.sqrt(u1)
    w = b * np.cos(2 * np.pi * u3)
    x = a * np.sin(2 * np.pi * u2)
    y = a * np.cos(2 * np.pi * u2)
    z = b * np.sin(2 * np.pi * u3)
    return np.stack([w, x, y, z], 1).astype(np.float32)


def look_at(eye, target, down_hint=(0.0, 1.0, 0.0)) -> tuple[np.ndarray, np.ndarray]:
    """World->camera (R, t) for a camera at ``eye`` looking at ``target`` (OpenCV axes, +y down)."""
    eye = np.asarray(eye, np.float64)
    fwd = np.asarray(target, np.float64) - eye
    fwd /= np.linalg.norm(fwd)
    right = np.cross(np.asarray(down_hint, np.float64), fwd)
    right /= np.linalg.norm(right)
    down = np.cross(fwd, right)
    R = np.stack([right, down, fwd], 0)
    t = -R @ eye
    return R.reshape(9).astype(np.float32), t.astype(np.float32)


def _pack_rgba(r, g, b, a):
    q = lambda v: np.clip(np.floor(np.asarray(v) * 255.0 + 0.5), 0, 255).astype(np.uint32)
    return q(r) | (q(g) << 8) | (q(b) << 16) | (q(a) << 24)


def _smooth_target(rng, W, H, n_blobs=32, noise=0.02):
    yy, xx = np.mgrid[0:H, 0:W].astype(np.float32)
    img = np.zeros((H, W, 3), np.float32)
    for _ in range(n_blobs):
        cx, cy = rng.random() * W, rng.random() * H
        s = (0.05 + 0.2 * rng.random()) * min(W, H)
        amp = rng.random(3).astype(np.float32)
        g = np.exp(-((xx - cx) ** 2 + (yy - cy) ** 2) / (2 * s * s))
        img += g[..., None] * amp[None, None, :]
    img /= max(img.max(), 1e-6)
    img += rng.normal(0, noise, img.shape).astype(np.float32)
    return np.clip(img, 0, 1)


def _colour_to_dc(c):
    return ((c - 0.5) / SH_C0).astype(np.float32)


def _fp16_bands(sh):
    out = sh.copy()
    out[:, 1:, :] = out[:, 1:, :].astype(np.float16).astype(np.float32)
    return out


def config1(seed: int | None = None) -> Scene:
    """1,024 splats, SH0, 64x64, fx=fy=64, cx=cy=32; means in a unit cube centred 3 units ahead."""
    rng = np.random.default_rng(0xB2C0 + 1 if seed is None else seed)
    n, W, H = 1024, 64, 64
    pos = rng.random((n, 3)) - 0.5
    pos[:, 2] += 3.0
    op = rng.normal(0, 1, n)
    pos_op = np.concatenate([pos, op[:, None]], 1).astype(np.float32)
    lscale = np.zeros((n, 4), np.float32)
    lscale[:, :3] = rng.normal(-3.0, 0.5, (n, 3))
    sh = _colour_to_dc(rng.random((n, 1, 3)))
    R, t = np.eye(3, dtype=np.float32).reshape(9), np.zeros(3, np.float32)
    cam = Camera(W, H, 64.0, 64.0, 32.0, 32.0, R, t)
    noise = rng.random((H * W, 3))
    gt = _pack_rgba(noise[:, 0], noise[:, 1], noise[:, 2], np.ones(H * W))
    return Scene("cfg1", 0, pos_op, _rand_quat(rng, n), lscale, sh, cam, gt)


def config2(seed: int | None = None, n: int = 100_000) -> Scene:
    """100k splats, SH3 (bands N(0, 0.05)), 800x800, 50 deg FOV; means N(0,1) within r <= 2, 4 units away."""
    rng = np.random.default_rng(0xB2C0 + 2 if seed is None else seed)
    W = H = 800
    pos = rng.normal(0, 1, (n, 3))
    r = np.linalg.norm(pos, axis=1)
    bad = r > 2
    while bad.any():
        pos[bad] = rng.normal(0, 1, (int(bad.sum()), 3))
        bad = np.linalg.norm(pos, axis=1) > 2
    op = rng.normal(-1.0, 1.5, n)
    pos_op = np.concatenate([pos, op[:, None]], 1).astype(np.float32)
    lscale = np.zeros((n, 4), np.float32)
    lscale[:, :3] = rng.normal(-4.5, 0.6, (n, 3))
    sh = np.zeros((n, 16, 3), np.float32)
    sh[:, 0, :] = _colour_to_dc(rng.random((n, 3)))
    sh[:, 1:, :] = rng.normal(0, 0.05, (n, 15, 3))
    f = 400.0 / math.tan(math.radians(25.0))
    R, t = look_at((0.0, 0.0, -4.0), (0.0, 0.0, 0.0))
    cam = Camera(W, H, f, f, 400.0, 400.0, R, t)
    img = _smooth_target(rng, W, H).reshape(-1, 3)
    gt = _pack_rgba(img[:, 0], img[:, 1], img[:, 2], np.ones(H * W))
    return Scene("cfg2", 3, pos_op, _rand_quat(rng, n), lscale, sh, cam, gt)


def _ellipse_alpha(W, H):
    yy, xx = np.mgrid[0:H, 0:W].astype(np.float64)
    # semi-axes a, b with pi*a*b = W*H/2 and a/b = W/H
    b = math.sqrt(W * H / (2 * math.pi) * H / W)
    a = b * W / H
    inside = ((xx + 0.5 - W / 2) / a) ** 2 + ((yy + 0.5 - H / 2) / b) ** 2 <= 1.0
    return inside.reshape(-1)


def config3(seed: int | None = None, n: int = 1_000_000, masked: bool = False) -> Scene:
    """1M splats, SH3, 1920x1080; means uniform in a 6x4x6 box of which ~60% lie in the frustum.

    Fused L1+SSIM with alpha lane, per-pixel weights in [0.5, 1.5] (u8 in [85, 255] with scale 1.5),
    binary elliptic alpha over half the image. ``masked=False`` is the transparent-view mode
    (composite + alpha lane, trainer.cpp:495-497), ``masked=True`` the masked-view mode."""
    rng = np.random.default_rng(0xB2C0 + 3 if seed is None else seed)
    W, H = 1920, 1080
    pos = np.empty((n, 3))
    pos[:, 0] = rng.uniform(-3, 3, n)
    pos[:, 1] = rng.uniform(-2, 2, n)
    pos[:, 2] = rng.uniform(0, 6, n)
    op = rng.normal(-0.5, 2.0, n)
    pos_op = np.concatenate([pos, op[:, None]], 1).astype(np.float32)
    lscale = np.zeros((n, 4), np.float32)
    lscale[:, :3] = rng.normal(-5.0, 0.7, (n, 3))
    sh = np.zeros((n, 16, 3), np.float32)
    sh[:, 0, :] = _colour_to_dc(rng.random((n, 3)))
    sh[:, 1:, :] = rng.normal(0, 0.05, (n, 15, 3))
    f = 1000.0
    # camera just in front of the box's near face, looking down +z through its centre: ~62% of the
    # means project inside the image
    R, t = look_at((0.0, 0.0, -0.05), (0.0, 0.0, 3.0))
    cam = Camera(W, H, f, f, W / 2.0, H / 2.0, R, t)
    img = _smooth_target(rng, W, H).reshape(-1, 3)
    alpha = _ellipse_alpha(W, H).astype(np.float64)
    prem = img * alpha[:, None] if not masked else img
    gt = _pack_rgba(prem[:, 0], prem[:, 1], prem[:, 2], alpha)
    weights = rng.integers(85, 256, W * H).astype(np.uint8)
    return Scene("cfg3" + ("m" if masked else ""), 3, pos_op, _rand_quat(rng, n), lscale, sh, cam, gt, weights,
                 composite=not masked, mask=masked, alpha_lane=not masked, match_alpha_weight=0.1, scale=1.5)


def config4(seed: int | None = None, n: int = 3_000_000, shrink: int = 1) -> Scene:
    """3M splats, SH4, 1920x1080; a slab 0.5 deep facing the camera (high depth complexity); 8 poses
    (``extra_cams``, the first is ``cam``).

    ``shrink`` = k > 1 is the same workload cut to a k-th of the size in each image direction: the slab's
    width and height and the image's divide by k, the splat count by k^2; the focal length, the splat sizes,
    the depths and the density per unit of slab area are unchanged, so every pixel still sees the same
    depth complexity (fragments per pixel) through a narrower field of view."""
    rng = np.random.default_rng(0xB2C0 + 4 if seed is None else seed)
    k = int(shrink)
    n = n if k == 1 else n // (k * k)
    W, H = 1920 // k, 1080 // k
    f = 1000.0
    pos = np.empty((n, 3))
    pos[:, 0] = rng.uniform(-2.2 / k, 2.2 / k, n)
    pos[:, 1] = rng.uniform(-1.25 / k, 1.25 / k, n)
    pos[:, 2] = rng.uniform(-0.25, 0.25, n)
    op = rng.normal(-2.0, 1.0, n)
    pos_op = np.concatenate([pos, op[:, None]], 1).astype(np.float32)
    lscale = np.zeros((n, 4), np.float32)
    lscale[:, :3] = rng.normal(-4.0, 0.5, (n, 3))
    sh = np.zeros((n, 25, 3), np.float32)
    sh[:, 0, :] = _colour_to_dc(rng.random((n, 3)))
    sh[:, 1:, :] = rng.normal(0, 0.05, (n, 24, 3))
    cams = []
    for v in range(8):
        ang = math.radians(-14.0 + 4.0 * v)
        eye = (2.4 * math.sin(ang), 0.15 * math.cos(3 * ang), -2.4 * math.cos(ang))
        R, t = look_at(eye, (0.0, 0.0, 0.0))
        cams.append(Camera(W, H, f, f, W / 2.0, H / 2.0, R, t))
    img = _smooth_target(rng, W, H).reshape(-1, 3)
    gt = _pack_rgba(img[:, 0], img[:, 1], img[:, 2], np.ones(W * H))
    name = "cfg4" if k == 1 else f"cfg4/{k}"
    return Scene(name, 4, pos_op, _rand_quat(rng, n), lscale, sh, cams[0], gt, extra_cams=cams)


def config5(seed: int | None = None, n: int = 500_000) -> Scene:
    """500k splats, 3840x2160, SH3 with fp16 bands; 95% tiny splats, 5% large anisotropic ones."""
    rng = np.random.default_rng(0xB2C0 + 5 if seed is None else seed)
    W, H = 3840, 2160
    f = 2000.0
    pos = np.empty((n, 3))
    pos[:, 0] = rng.uniform(-3, 3, n)
    pos[:, 1] = rng.uniform(-1.8, 1.8, n)
    pos[:, 2] = rng.uniform(1.0, 7.0, n)
    op = rng.normal(0.0, 2.0, n)
    pos_op = np.concatenate([pos, op[:, None]], 1).astype(np.float32)
    lscale = np.zeros((n, 4), np.float32)
    lscale[:, :3] = rng.normal(-7.0, 0.3, (n, 3))
    big = rng.random(n) < 0.05
    lscale[big, :3] = rng.choice(np.array([-1.0, -3.0, -6.0], np.float32), (int(big.sum()), 3))
    sh = np.zeros((n, 16, 3), np.float32)
    sh[:, 0, :] = _colour_to_dc(rng.random((n, 3)))
    sh[:, 1:, :] = rng.normal(0, 0.05, (n, 15, 3))
    R, t = look_at((0.0, 0.0, -1.0), (0.0, 0.0, 4.0))
    cam = Camera(W, H, f, f, W / 2.0, H / 2.0, R, t)
    img = _smooth_target(rng, W, H).reshape(-1, 3)
    gt = _pack_rgba(img[:, 0], img[:, 1], img[:, 2], np.ones(W * H))
    return Scene("cfg5", 3, pos_op, _rand_quat(rng, n), lscale, _fp16_bands(sh), cam, gt, sh_fp16=True)


def pixel_centred_scene(seed: int = 3) -> Scene:
    """Splats whose projections land exactly on pixel centres: camera at the origin looking down +z, fx = fy =
    64, cx = cy = 32, splat means x = (k - 31.5) / 32 at depth z = 2, so 64 x / z + 32 = k + 0.5 in float
    arithmetic. Small, mostly opaque, well separated, so each centre pixel's colour comes from one splat."""
    rng = np.random.default_rng(seed)
    W = H = 64
    ks = rng.permutation(np.arange(2, 62, 5))
    ls = rng.permutation(np.arange(2, 62, 5))
    k, l = np.meshgrid(ks, ls)
    k, l = k.ravel(), l.ravel()
    n = k.size
    pos = np.stack([(k - 31.5) / 32.0, (l - 31.5) / 32.0, np.full(n, 2.0)], 1)
    op = rng.uniform(0.0, 3.0, n)  # opacity sigmoid(op): 0.5 .. 0.95
    pos_op = np.concatenate([pos, op[:, None]], 1).astype(np.float32)
    lscale = np.zeros((n, 4), np.float32)
    lscale[:, :3] = rng.uniform(-4.5, -3.0, (n, 3))  # sigma 0.35 .. 1.6 px at depth 2, f = 64
    sh = _colour_to_dc(rng.random((n, 1, 3)))
    cam = Camera(W, H, 64.0, 64.0, 32.0, 32.0, np.eye(3, dtype=np.float32).reshape(9), np.zeros(3, np.float32))
    gt = _pack_rgba(*rng.random((3, H * W)), np.ones(H * W))
    return Scene("pixel-centred", 0, pos_op, _rand_quat(rng, n), lscale, sh, cam, gt)


def fd_scene(seed: int, n: int = 24, masked: bool = False, degree: int = 2, floor: bool = False) -> Scene:
    """The reference FD harness scene shape (tests/tests.cpp:23-59): 48x40, fx=fy=40, SH degree 2,
    means in [-0.6,0.6]x[-0.5,0.5]x[1.5,2.5], scales 0.05-0.13, jittered quaternions, opacity logits
    in [-2, 2], random RGBA target with u8 weights in [64, 255]. Transparent views use composite +
    alpha lane (match weight 0.3), masked views the mask with scale 1.7 (tests.cpp:67-71).

    ``floor=True`` gives every splat a Mip-Splatting floor f in [0.02, 0.06] (``lscale[:, 3]``), the
    frozen minimum scale of splat_math.cuh:232-237 that the reference's upload leaves at 0."""
    rng = np.random.default_rng(seed)
    W, H = 48, 40
    K = (degree + 1) ** 2
    u = lambda *s: rng.random(s)
    un = lambda *s: rng.random(s) * 2 - 1
    pos = np.stack([un(n) * 0.6, un(n) * 0.5, 2.0 + un(n) * 0.5], 1)
    op = un(n) * 2.0
    pos_op = np.concatenate([pos, op[:, None]], 1).astype(np.float32)
    lscale = np.zeros((n, 4), np.float32)
    lscale[:, :3] = np.log(0.05 + 0.08 * u(n, 3))
    quat = np.stack([1.0 + un(n) * 0.5, un(n) * 0.5, un(n) * 0.5, un(n) * 0.5], 1).astype(np.float32)
    sh = np.zeros((n, K, 3), np.float32)
    sh[:, 0, :] = un(n, 3) * 1.5
    if K > 1:
        sh[:, 1:, :] = un(n, K - 1, 3) * 0.3
    if floor:
        lscale[:, 3] = 0.02 + 0.04 * u(n)
    R, t = np.eye(3, dtype=np.float32).reshape(9), np.zeros(3, np.float32)
    cam = Camera(W, H, 40.0, 40.0, W / 2.0, H / 2.0, R, t)
    rgba = (u(W * H, 4) * 255).astype(np.uint32)
    gt = rgba[:, 0] | (rgba[:, 1] << 8) | (rgba[:, 2] << 16) | (rgba[:, 3] << 24)
    weights = (64 + u(W * H) * 191).astype(np.uint8)
    tag = ("m" if masked else "t") + ("f" if floor else "")
    return Scene(f"fd{seed}{tag}", degree, pos_op, quat, lscale, sh, cam, gt.astype(np.uint32),
                 weights, composite=not masked, mask=masked, alpha_lane=not masked, match_alpha_weight=0.3,
                 scale=1.7 if masked else 1.0, bg=(0.2, 0.1, 0.3))


def fd_feature_scene(seed: int, n: int = 24, masked: bool = False, normals: bool = False, hollow: bool = False,
                     degree: int = 2) -> Scene:
    """The FD harness's normal and hollow configurations (tests/tests.cpp:23-59, 66-76, 386-391) on an
    FD-harness scene: a random normal map opaque on about 70% of the pixels, normal_scale = 0.05 / 100
    (normal_loss_weight over the view's normal count); a reference depth 1.9 + 0.25 sin(0.4 x) +
    0.2 cos(0.3 y) with a 6x6 corner of no surface (+inf), margin 0.05, lam = 0.7 / (W H)."""
    sc = fd_scene(seed, n=n, masked=masked, degree=degree)
    rng = np.random.default_rng(seed + 104729)
    W, H = sc.W, sc.H
    if normals:
        rgb = (rng.random((W * H, 3)) * 255).astype(np.uint32)
        a = np.where(rng.random(W * H) > 0.3, 255, 0).astype(np.uint32)
        sc.normals = (rgb[:, 0] | (rgb[:, 1] << 8) | (rgb[:, 2] << 16) | (a << 24)).astype(np.uint32)
        sc.feat_mode = 1
        sc.normal_scale = 0.05 / 100.0
    if hollow:
        y, x = np.mgrid[0:H, 0:W]
        z = 1.9 + 0.25 * np.sin(x * 0.4) + 0.2 * np.cos(y * 0.3)
        z[(x < 6) & (y < 6)] = np.inf
        sc.hollow_z = z.astype(np.float32).reshape(-1)
        sc.hollow_margin = 0.05
        sc.hollow_lam = 0.7 / (W * H)
    sc.name = sc.name + ("n" if normals else "") + ("h" if hollow else "")
    return sc


def clamp_scene(seed: int, n: int = 24, degree: int = 2) -> Scene:
    """FD-harness camera and target with half the splats centred beyond the EWA Jacobian's tangent clamp
    (x/z or y/z outside 15% past the frame, render.h:21-22): large splats (scales 0.22-0.36 at depth
    ~2) whose centres lie left, right, above or below the frame but whose footprints reach into it, so
    the clamped Jacobian and its VJP branches decide their gradients."""
    sc = fd_scene(seed, n=n, degree=degree)
    rng = np.random.default_rng(seed + 7919)
    m = n // 2
    z = 2.0 + (rng.random(m) * 2 - 1) * 0.3
    side = rng.integers(0, 4, m)
    # the limits are (1.15 W - cx) / fx = 0.78 and (1.15 H - cy) / fy = 0.65 for the 48x40, f = 40 camera
    along = 0.82 + 0.3 * rng.random(m)
    across = (rng.random(m) * 2 - 1) * 0.4
    tx = np.where(side == 0, along, np.where(side == 1, -along, across))
    ty = np.where(side == 2, along * 0.85, np.where(side == 3, -along * 0.85, across * 0.8))
    sc.pos_op[:m, 0] = (tx * z).astype(np.float32)
    sc.pos_op[:m, 1] = (ty * z).astype(np.float32)
    sc.pos_op[:m, 2] = z.astype(np.float32)
    sc.pos_op[:m, 3] = (rng.random(m) * 2.0 + 0.5).astype(np.float32)
    sc.lscale[:m, :3] = np.log(0.22 + 0.14 * rng.random((m, 3))).astype(np.float32)
    sc.name = f"clamp{seed}"
    return sc


def multiview_fd_scene(seed: int, views: int = 3, degree: int = 2) -> Scene:
    """An FD-harness scene seen from ``views`` poses (``extra_cams``): the identity camera and small
    rotations / translations of it, all framing the splats. The target image is shared by the views."""
    sc = fd_scene(seed, degree=degree)
    cams = [sc.cam]
    for v in range(1, views):
        ang = 0.12 * v * (1 if v % 2 else -1)
        eye = (2.0 * math.sin(ang), 0.1 * v, 2.0 - 2.0 * math.cos(ang))
        R, t = look_at(eye, (0.0, 0.0, 2.0))
        cams.append(Camera(sc.W, sc.H, 40.0, 40.0, sc.W / 2.0, sc.H / 2.0, R, t))
    sc.extra_cams = cams
    sc.name = f"mv{seed}x{views}"
    return sc


CONFIGS = {1: config1, 2: config2, 3: config3, 4: config4, 5: config5}
