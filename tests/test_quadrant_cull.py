"""The forward raster's quadrant culling test (quadrant_mask in b2ctrain_amd/csrc/kernels/raster_common.h),
restated in float32 numpy, must be conservative: a quadrant with a pixel centre where the raster kernels'
fp32 sigma (the quadratic about the tile centre of sigma_coefs / poly_sigma, five fused multiply-adds,
evaluated here by the oracle's C restatement; the reference's src/gpu/raster_fwd.cu:44-50 rounds the same
quantity differently) passes sigma <= power must keep its bit. Checked by brute force over all 64 pixel centres on random splats,
including needle-thin ellipses (axis ratio up to 1e5) whose terms cancel, splats centred inside, on the
edges and far outside the tile, and adversarially: power set to the fp32 sigma of one pixel, which puts
that pixel exactly on the cutoff. The GPU parity tests check the device code itself (a wrongly culled
fragment changes the rendered colour by at least alpha = 1/255 of its weight)."""
import numpy as np

from oracle import oracle as O

f32 = np.float32


def edge_lb(ah, b, ch, dx, dy):
    t1 = ah * dx * dx
    t2 = ch * dy * dy
    t3 = b * dx * dy
    return (t1 + t2 + t3) - f32(1e-5) * (np.abs(t1) + np.abs(t2) + np.abs(t3))


def poly_slack_power(mx, my, ah, b, ch, power, x0, y0):
    """power raised by 1e-5 of the magnitude of the tile-centred quadratic's terms over the tile (the
    per-pixel sigma's rounding scale), as quadrant_mask does."""
    mxr, myr, bb = np.abs(mx - (x0 + f32(3.5))), np.abs(my - (y0 + f32(3.5))), np.abs(b)
    scale = (((ah * mxr + bb * myr) * mxr + ch * myr * myr) +
             f32(3.5) * ((f32(2) * ah + bb) * mxr + (bb + f32(2) * ch) * myr) + f32(12.25) * (ah + bb + ch))
    return power + f32(1e-5) * scale


def quadrant_mask(mx, my, ah, b, ch, power, x0, y0):
    """Restates raster_common.h's quadrant_mask: per quadrant, the centre inside the box, or the clamped
    minimum on the (at most one) vertical and (at most one) horizontal edge the centre lies beyond."""
    with np.errstate(all="ignore"):
        power = poly_slack_power(mx, my, ah, b, ch, power, x0, y0)
        ky = -b / (f32(2) * ch)
        kx = -b / (f32(2) * ah)
        ex = [x0 - mx, x0 + f32(3) - mx, x0 + f32(4) - mx, x0 + f32(7) - mx]
        ey = [y0 - my, y0 + f32(3) - my, y0 + f32(4) - my, y0 + f32(7) - my]
        mask = np.zeros(mx.shape, np.uint32)
        for qy in range(2):
            for qx in range(2):
                xlo, xhi, ylo, yhi = ex[2 * qx], ex[2 * qx + 1], ey[2 * qy], ey[2 * qy + 1]
                fv = (xlo > 0) | (xhi < 0)
                fh = (ylo > 0) | (yhi < 0)
                xe = np.where(xlo > 0, xlo, xhi)
                ye = np.where(ylo > 0, ylo, yhi)
                mv = edge_lb(ah, b, ch, xe, np.fmin(np.fmax(ky * xe, ylo), yhi))
                mh = edge_lb(ah, b, ch, np.fmin(np.fmax(kx * ye, xlo), xhi), ye)
                reach = (~fv & ~fh) | (fv & ~(mv > power)) | (fh & ~(mh > power))
                mask |= np.where(reach, np.uint32(1 << (2 * qy + qx)), np.uint32(0))
        keep_all = ~((ah > 0) & (ch > 0)) | ~(mx - mx == 0) | ~(my - my == 0)
        return np.where(keep_all, np.uint32(0xF), mask)


def quadrant_mask_all_edges(mx, my, ah, b, ch, power, x0, y0):
    """The same bound taken over all four edges of each quadrant box (no facing-edge selection)."""
    with np.errstate(all="ignore"):
        power = poly_slack_power(mx, my, ah, b, ch, power, x0, y0)
        ky = -b / (f32(2) * ch)
        kx = -b / (f32(2) * ah)
        ex = [x0 - mx, x0 + f32(3) - mx, x0 + f32(4) - mx, x0 + f32(7) - mx]
        ey = [y0 - my, y0 + f32(3) - my, y0 + f32(4) - my, y0 + f32(7) - my]
        mask = np.zeros(mx.shape, np.uint32)
        for qy in range(2):
            for qx in range(2):
                xlo, xhi, ylo, yhi = ex[2 * qx], ex[2 * qx + 1], ey[2 * qy], ey[2 * qy + 1]
                inside = (xlo <= 0) & (xhi >= 0) & (ylo <= 0) & (yhi >= 0)
                reach = inside.copy()
                for xe in (xlo, xhi):
                    reach |= ~(edge_lb(ah, b, ch, xe, np.fmin(np.fmax(ky * xe, ylo), yhi)) > power)
                for ye in (ylo, yhi):
                    reach |= ~(edge_lb(ah, b, ch, np.fmin(np.fmax(kx * ye, xlo), xhi), ye) > power)
                mask |= np.where(reach, np.uint32(1 << (2 * qy + qx)), np.uint32(0))
        return np.where(~((ah > 0) & (ch > 0)), np.uint32(0xF), mask)


def sigma_at(mx, my, c00, c01, c11, x0, y0, i, j):
    return O.frag_sigma(mx, my, c00, c01, c11, x0 + f32(i), y0 + f32(j))


def pixel_truth(mx, my, c00, c01, c11, power, x0, y0):
    """Per quadrant: does any pixel centre pass the reference's cutoff (fp32, uncontracted)?"""
    truth = np.zeros(mx.shape, np.uint32)
    for j in range(8):
        for i in range(8):
            sig = sigma_at(mx, my, c00, c01, c11, x0, y0, i, j)
            hit = sig <= power
            truth |= np.where(hit, np.uint32(1 << (2 * (j // 4) + i // 4)), np.uint32(0))
    return truth


def _splats(rng, n, spread, log_ratio_max):
    theta = rng.uniform(0, np.pi, n)
    s1 = np.exp(rng.uniform(-1.0, 4.0, n))
    s2 = s1 * np.exp(-rng.uniform(0, log_ratio_max, n))
    c, s = np.cos(theta), np.sin(theta)
    # covariance R diag(s1^2, s2^2) R^T (+0.3 px dilation as the projection adds), conic = inverse
    a = c * c * s1**2 + s * s * s2**2 + 0.3
    bb = c * s * (s1**2 - s2**2)
    d = s * s * s1**2 + c * c * s2**2 + 0.3
    det = a * d - bb * bb
    c00, c01, c11 = (d / det).astype(f32), (-bb / det).astype(f32), (a / det).astype(f32)
    x0, y0 = f32(8 * 37 + 0.5), f32(8 * 11 + 0.5)
    mx = (x0 + 3.5 + rng.normal(0, spread, n)).astype(f32)
    my = (y0 + 3.5 + rng.normal(0, spread, n)).astype(f32)
    power = rng.uniform(0.0, 8.0, n).astype(f32)
    return mx, my, c00, c01, c11, power, x0, y0


def test_quadrant_mask_is_conservative():
    rng = np.random.default_rng(0)
    checked = culled = 0
    for spread, ratio in [(3.0, 2.0), (10.0, 5.0), (40.0, 9.2), (1.0, 9.2)]:
        mx, my, c00, c01, c11, power, x0, y0 = _splats(rng, 200_000, spread, ratio)
        got = quadrant_mask(mx, my, f32(0.5) * c00, c01, f32(0.5) * c11, power, x0, y0)
        truth = pixel_truth(mx, my, c00, c01, c11, power, x0, y0)
        missed = truth & ~got
        assert not missed.any(), f"culled a reachable quadrant: {np.flatnonzero(missed)[:5]}"
        checked += int(np.count_nonzero(truth))
        culled += int(np.count_nonzero(~got & np.uint32(0xF)))
    assert checked > 100_000 and culled > 100_000  # both outcomes well exercised


def test_quadrant_mask_centre_inside_and_degenerate():
    f = lambda *v: [np.array([x], f32) for x in v]
    mx, my, ah, b, ch, p = f(101.0, 101.0, 0.5, 0.0, 0.5, 0.0)
    assert quadrant_mask(mx, my, ah, b, ch, p, f32(96.5), f32(96.5))[0] == 1 << 3  # centre in quadrant (1, 1)
    mx, my, ah, b, ch, p = f(0.0, 0.0, 0.0, 0.0, 0.5, 1.0)
    assert quadrant_mask(mx, my, ah, b, ch, p, f32(96.5), f32(96.5))[0] == 0xF


def test_quadrant_mask_keeps_pixels_exactly_on_the_cutoff():
    rng = np.random.default_rng(7)
    for spread, ratio in [(3.0, 2.0), (1.0, 9.2), (5.0, 11.5), (30.0, 9.2), (100.0, 11.5)]:
        mx, my, c00, c01, c11, _, x0, y0 = _splats(rng, 200_000, spread, ratio)
        i = rng.integers(0, 8, mx.size)
        j = rng.integers(0, 8, mx.size)
        sig = sigma_at(mx, my, c00, c01, c11, x0, y0, i.astype(f32), j.astype(f32))
        power = np.where(sig >= 0, sig, f32(0)).astype(f32)  # pixel (i, j) passes with sigma == power
        on = sig <= power  # every pixel: one rounded below 0 passes against power 0
        qm = quadrant_mask(mx, my, f32(0.5) * c00, c01, f32(0.5) * c11, power, x0, y0)
        qbit = np.uint32(1) << (2 * (j // 4) + i // 4).astype(np.uint32)
        assert not (on & ((qm & qbit) == 0)).any(), "quadrant mask dropped a pixel on the cutoff"


def test_facing_edges_cull_as_much_as_all_edges():
    """The convex minimum over a box lies on an edge the centre is beyond, so testing only those edges keeps
    the same quadrants as testing all four (differences only from rounding at corners, where both edges give
    the same minimum up to the margin)."""
    rng = np.random.default_rng(3)
    diff = total = 0
    for spread, ratio in [(3.0, 2.0), (10.0, 5.0), (40.0, 9.2), (1.0, 9.2)]:
        mx, my, c00, c01, c11, power, x0, y0 = _splats(rng, 200_000, spread, ratio)
        args = (mx, my, f32(0.5) * c00, c01, f32(0.5) * c11, power, x0, y0)
        new, old = quadrant_mask(*args), quadrant_mask_all_edges(*args)
        diff += int(np.count_nonzero(new != old))
        total += mx.size
    assert diff <= total * 1e-5, f"{diff} of {total} masks differ"
