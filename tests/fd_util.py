"""Central finite differences of the fp64 brute-force oracle (orc_ref_loss, the restatement of the
reference's tests/reference.cpp:34-143) over a splat's parameters, taken as the reference's FD harness
takes them (tests/tests.cpp:413-436): every `every`-th splat, all 11 geometric parameters and every
`sh_every`-th SH lane; a sample whose differences at eps and 4 eps disagree by more than 10% sits on a
non-smooth point (a fragment crossing the 1/255 cutoff or the transmittance stop) and is skipped.
Several cameras (``cams``) sum the per-view losses.

A sample fails when its relative error exceeds 1e-3 and its absolute error exceeds both 1e-9 and 1e-6 of
the largest analytic gradient of its column: a gradient that is a float32 sum of many fragment terms of
both signs cannot resolve a value many orders of magnitude below those terms (observed: 4e-7 of the
column maximum on a 5e-8 gradient)."""
from __future__ import annotations

import numpy as np

from oracle import oracle as O

REL_TOL = 1e-3
ABS_FLOOR = 1e-9
COL_FLOOR = 1e-6


def perturbed_loss(scene, P0, i, q, delta, cams=None):
    P = {k: v.copy() for k, v in P0.items()}
    if q < 3:
        P["pos"][i, q] += delta
    elif q == 3:
        P["opacity"][i] += delta
    elif q < 8:
        P["quat"][i, q - 4] += delta
    elif q < 11:
        P["log_scale"][i, q - 8] += delta
    else:
        P["sh"][i, q - 11] += delta
    if not cams:
        return O.ref_loss(scene, params=P)
    return sum(O.ref_loss(scene.with_camera(c), params=P) for c in cams)


def fd_compare(scene, analytic, every=2, sh_every=5, eps=1e-5, max_splats=None, cams=None):
    """Compare analytic gradients [n][11 + 3K] with central differences; returns (checked, skipped,
    mismatches, worst relative error). With the hollow loss the mean lanes are not compared: as in the
    reference (tests.cpp:418-421), its gradient treats a fragment's depth as constant."""
    P0 = O.scene_params64(scene)
    per = 11 + 3 * scene.K
    col_floor = np.maximum(COL_FLOOR * np.abs(np.asarray(analytic, np.float64)).max(axis=0), ABS_FLOOR)
    bad, checked, skipped, worst = [], 0, 0, 0.0
    n = scene.n if max_splats is None else min(scene.n, max_splats)
    for i in range(0, n, every):
        for q in range(per):
            if q >= 11 and (q - 11) % sh_every:
                continue
            if scene.hollow_z is not None and q < 3:
                continue
            at = lambda d: perturbed_loss(scene, P0, i, q, d, cams)
            fd = (at(eps) - at(-eps)) / (2 * eps)
            fd4 = (at(4 * eps) - at(-4 * eps)) / (8 * eps)
            if abs(fd - fd4) > 0.1 * max(abs(fd), abs(fd4)) + 1e-9:
                skipped += 1
                continue
            a = float(analytic[i, q])
            d = abs(fd - a)
            den = max(abs(fd), abs(a))
            rel = d / den if den > 0 else 0.0
            checked += 1
            if rel > REL_TOL and d > col_floor[q]:
                bad.append((i, q, a, fd, rel))
            if d > col_floor[q]:
                worst = max(worst, rel)
    return checked, skipped, bad, worst
