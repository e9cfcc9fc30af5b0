"""Pins for the oracle's fused optimizer (oracle/orc_adam.c, restating src/gpu/optim.cu:104-148 and
298-377 and src/gpu/util.cuh:106-117, 148-162) that do not restate it: closed forms of Adam, the dense
zero-gradient steps that the lazy catch-up summarises, the spherical-harmonic addition theorem, numpy's
binary16 rounding, numpy's cosine and the statistics the random streams must have. A plausible slip -- a
missing bias correction, the wrong learning rate on a lane, a catch-up decaying the wrong moment or by the
wrong power, a biased or one-sided stochastic rounding, a Box-Muller with the wrong constant -- fails at
least one test here.

| oracle piece            | reference (file:line)     | pinned by                                              |
|-------------------------|---------------------------|--------------------------------------------------------|
| orc_f16_bits / _value   | __float2half_rn           | numpy float16 casts (all 65536 patterns, random floats, ties) |
| orc_f16_stochastic      | util.cuh:148-162          | neighbours only, exact P(up) on a uniform grid, mean    |
| orc_cos_turns           | __cosf(2 pi u)            | numpy fp64 cos, <= 3e-7                                |
| orc_hash_unit / _gauss  | util.cuh:106-117          | uniformity (chi^2), lane independence, N(0, 1) moments and KS |
| orc_adam_update: Adam   | optim.cu:84-97, 316-335   | t = 1 and constant-gradient closed forms, per-lane rates |
| lazy catch-up           | optim.cu:142, 298-315     | equal to dense steps with zero gradient over the gap    |
| SH moments              | optim.cu:336-359          | addition theorem sum_m Y_lm^2 = (2l + 1) / 4 pi; the gap |
| MCMC noise              | optim.cu:361-375          | visible-only, N(0, w^2) with w = weight (1 - o)^150, clamp |

The exact bit patterns of the reference's hash stream (util.cuh:106-112) have no vectors in the reference
to check against: that part is pinned only structurally (same mixing function and counters), as stated
in DESIGN.md's pin table.
"""
import math

import numpy as np
import pytest
from scipy import stats

from b2ctrain_amd import scenes as S
from oracle import oracle as O


# ---------------------------------------------------------------------------------------------- binary16
def test_f16_value_matches_numpy_for_every_pattern():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    want = bits.view(np.float16).astype(np.float32)
    got = np.array([O.f16_value(int(b)) for b in bits], np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_f16_round_to_nearest_even_matches_numpy():
    rng = np.random.default_rng(5)
    mags = np.concatenate([rng.uniform(0, 1, 20000), 10.0 ** rng.uniform(-9, 5, 40000)])
    v = (mags * rng.choice([-1, 1], mags.size)).astype(np.float32)
    # exact ties: the midpoints between neighbouring half values (normal and subnormal)
    h = np.arange(0, 0x7bff, 7, dtype=np.uint16)
    lo, hi = h.view(np.float16).astype(np.float64), (h + 1).view(np.float16).astype(np.float64)
    ties = ((lo + hi) / 2).astype(np.float32)
    v = np.concatenate([v, ties, -ties, np.float32([65504, 65519.99, 65520, 7e4, 0, -0.0, np.inf, -np.inf])])
    with np.errstate(over="ignore"):
        want = v.astype(np.float16).view(np.uint16)
    got = np.array([O.f16_bits(float(x)) for x in v], np.uint16)
    assert np.array_equal(got, want)


def test_f16_stochastic_rounds_between_neighbours_with_the_right_odds():
    rng = np.random.default_rng(7)
    grid = (np.arange(4096) / 4096.0).astype(np.float32)  # exact multiples of 2^-12, as hash_unit's values
    for v in np.concatenate([rng.uniform(-3, 3, 40), [1e-6, -3e-7, 0.25 + 1e-5, 64000.3]]).astype(np.float32):
        v = float(v)
        near = np.float16(v)
        lo = float(near) if float(near) <= v else float(np.nextafter(near, np.float16(-np.inf)))
        hi = float(np.nextafter(np.float16(lo), np.float16(np.inf)))
        outs = np.array([O.f16_value(O.f16_stochastic(v, float(u))) for u in grid])
        assert set(np.unique(outs)) <= {lo, hi}
        ups = int((outs == hi).sum())
        frac = (v - lo) / (hi - lo)
        # P(up) = (v - lo) / (hi - lo): the count on the grid is that fraction of 4096, up to rounding
        assert abs(ups - frac * 4096) <= 1.0 + 1e-3 * 4096, (v, ups, frac)
        assert abs(outs.mean() - v) <= 1e-3 * (hi - lo) + 1e-12
    # representable values and the clamp
    assert O.f16_value(O.f16_stochastic(0.5, 0.9)) == 0.5
    # +-1e9 clamp to +-65000, between 64992 and 65024: up with odds 8/32 (24/32 for -65000)
    assert O.f16_value(O.f16_stochastic(1e9, 0.0)) == 65024.0
    assert O.f16_value(O.f16_stochastic(1e9, 0.3)) == 64992.0
    assert O.f16_value(O.f16_stochastic(-1e9, 0.7)) == -64992.0
    assert O.f16_value(O.f16_stochastic(-1e9, 0.8)) == -65024.0


# ---------------------------------------------------------------------------------------------- streams
def test_cos_turns_matches_numpy():
    u = np.concatenate([np.arange(0, 1 << 16) / 65536.0, np.random.default_rng(3).random(20000)]).astype(np.float32)
    got = np.array([O.cos_turns(float(x)) for x in u])
    err = np.abs(got - np.cos(2 * np.pi * u.astype(np.float64)))
    assert err.max() <= 3e-7, float(err.max())


def test_hash_unit_is_uniform_and_lanes_independent():
    n = 60000
    a = np.array([O.hash_unit(12345, i, 0) for i in range(n)])
    b = np.array([O.hash_unit(12345, i, 1) for i in range(n)])
    assert a.min() >= 0.0 and a.max() < 1.0
    assert np.all(np.round(a * 2 ** 24) == a * 2 ** 24)  # multiples of 2^-24
    counts, _ = np.histogram(a, bins=64, range=(0, 1))
    assert stats.chisquare(counts).pvalue > 1e-4
    assert abs(np.corrcoef(a, b)[0, 1]) < 0.02
    c = np.array([O.hash_unit(12346, i, 0) for i in range(n)])  # another seed
    assert abs(np.corrcoef(a, c)[0, 1]) < 0.02


def _lowbias32_inverse(x):
    """The inverse of lowbias32 as C. Wellons publishes it with the hash in hash-prospector (lowbias32_r):
    each xorshift is undone by xoring in the shifted word twice over, each multiply by the inverse of the
    multiplier modulo 2^32."""
    x = x.astype(np.uint32)
    x ^= x >> np.uint32(16)
    x = (x * np.uint32(0x43021123)).astype(np.uint32)
    x ^= (x >> np.uint32(15)) ^ (x >> np.uint32(30))
    x = (x * np.uint32(0x1D69E2A5)).astype(np.uint32)
    x ^= x >> np.uint32(16)
    return x


def test_mix32_is_lowbias32():
    """The finaliser of the random streams (util.cuh:106-110) is lowbias32: the published inverse undoes it
    on every sampled word, and the published inverse multipliers are the modular inverses of the forward
    ones the oracle must then use (checked here from the numbers alone)."""
    assert (0x7FEB352D * 0x1D69E2A5) % 2 ** 32 == 1 and (0x846CA68B * 0x43021123) % 2 ** 32 == 1
    words = np.concatenate([np.random.default_rng(11).integers(0, 2 ** 32, 20000, dtype=np.uint64),
                            np.array([0, 1, 2, 0xFFFFFFFF, 0x80000000, 0x7FFFFFFF], np.uint64)]).astype(np.uint32)
    mixed = np.array([O.mix32(int(w)) for w in words], np.uint32)
    assert np.array_equal(_lowbias32_inverse(mixed), words)
    assert O.mix32(0) == 0 and len(np.unique(mixed)) == len(np.unique(words))


def test_hash_unit_chains_the_xxhash_primes():
    """hash_unit(a, b, c) is the top 24 bits of mix32(a P1 ^ mix32(b P2 ^ mix32(c P3))) over 2^24, with
    P1..P3 xxHash32's PRIME32_1..3 (2654435761, 2246822519, 3266489917 in its specification)."""
    P1, P2, P3 = 2654435761, 2246822519, 3266489917
    m = 2 ** 32
    rng = np.random.default_rng(12)
    for a, b, c in rng.integers(0, 2 ** 32, (3000, 3), dtype=np.uint64).tolist() + [[0, 0, 0], [1, 2, 3]]:
        h = O.mix32((a * P1 % m) ^ O.mix32((b * P2 % m) ^ O.mix32(c * P3 % m)))
        assert O.hash_unit(a, b, c) == (h >> 8) / 2.0 ** 24, (a, b, c)


def test_hash_gauss_is_standard_normal():
    x = np.array([O.hash_gauss(77, i, c) for i in range(20000) for c in range(3)])
    assert abs(x.mean()) < 0.02 and abs(x.std() - 1.0) < 0.02
    assert abs(stats.kurtosis(x)) < 0.1
    assert stats.kstest(x, "norm").statistic < 0.01


# ---------------------------------------------------------------------------------------------- update
def _state(scene):
    n = scene.n
    z4 = np.zeros((n, 4), np.float32)
    return dict(pos_op=scene.pos_op.copy(), quat=scene.quat.copy(), lscale=scene.lscale.copy(), sh=scene.sh.copy(),
                m_pos_op=z4.copy(), v_pos_op=z4.copy(), m_quat=z4.copy(), v_quat=z4.copy(), m_lscale=z4.copy(),
                v_lscale=z4.copy(), m_sh=np.zeros_like(scene.sh), v_sh=np.zeros(n, np.float32),
                last_step=np.zeros(n, np.uint32))


def _visible_scene(seed=11, degree=2, n=24):
    """An FD-harness scene cut to the splats that survive the projection (so the SH term is live)."""
    s = S.fd_scene(seed, n=n, degree=degree)
    camd = S.camera_gpu(s.cam)
    ok = [i for i in range(s.n) if O.project_ok(s.pos_op[i], s.quat[i], s.lscale[i], camd)]
    assert len(ok) >= n // 2
    t = s.subset(s.n)
    t.pos_op, t.quat, t.lscale, t.sh = (a[ok].copy() for a in (s.pos_op, s.quat, s.lscale, s.sh))
    return t, camd


def _moved_by(before, after, want):
    """after = before - want, up to the rounding of the stored float32 values."""
    b = np.asarray(before, np.float64)
    d = b - np.asarray(after, np.float64)
    tol = 2.0 * np.spacing(np.abs(np.asarray(before, np.float32))).astype(np.float64) + 1e-5 * np.abs(want)
    assert np.all(np.abs(d - want) <= tol), float(np.max(np.abs(d - want) - tol))


def _inputs(n, K, rng, visible=True, vc=None):
    """A screen-space gradient row per splat that counts as a gradient (visible, nonzero, finite)."""
    vs = rng.normal(0, 1, (n, 13)).astype(np.float32)
    if vc is not None:
        vs[:, 5:8] = vc
    vis = np.full(n, 1 if visible else 0, np.uint32)
    tc = np.ones(n, np.uint32)
    return vs, vis, tc


def _grads(n, K, rng):
    return rng.normal(0, 1, (n, 11 + 3 * K)).astype(np.float32)


def test_first_step_moves_every_lane_by_its_learning_rate():
    s, camd = _visible_scene()
    rng = np.random.default_rng(1)
    n, K = s.n, s.K
    vs, vis, tc = _inputs(n, K, rng)
    G = _grads(n, K, rng)
    step = O.adam_step(t=1, lr_mean=1e-3)
    out = O.adam_update(_state(s), s.degree, False, camd, vs, vis, tc, G, step)
    st = _state(s)
    # t = 1 from zero moments: m_hat = g, v_hat = g^2, so every parameter moves by lr sign(g)
    _moved_by(st["pos_op"][:, :3], out["pos_op"][:, :3], 1e-3 * np.sign(G[:, :3]))
    _moved_by(st["pos_op"][:, 3], out["pos_op"][:, 3], 0.012 * np.sign(G[:, 3]))
    _moved_by(st["quat"], out["quat"], 2e-3 * np.sign(G[:, 4:8]))
    _moved_by(st["lscale"][:, :3], out["lscale"][:, :3], 5e-3 * np.sign(G[:, 8:11]))
    assert np.array_equal(out["lscale"][:, 3], st["lscale"][:, 3])  # the frozen floor
    assert not out["m_lscale"][:, 3].any() and not out["v_lscale"][:, 3].any()
    b1, b2 = 1.0 - float(np.float32(0.9)), 1.0 - float(np.float32(0.999))  # 1 - beta of the float32 betas
    np.testing.assert_allclose(out["m_pos_op"], b1 * G[:, :4], rtol=1e-6)
    np.testing.assert_allclose(out["v_pos_op"], b2 * G[:, :4] ** 2, rtol=1e-6)
    # SH: the first moment is per lane, the second one per splat, so a lane moves by lr m_hat / sqrt(v_sh_hat)
    vsh = out["v_sh"].astype(np.float64) / (1 - 0.999)
    flat = lambda a: a.reshape(n, 3 * K)
    _moved_by(flat(st["sh"])[:, :3], flat(out["sh"])[:, :3], 2e-3 * G[:, 11:14] / np.sqrt(vsh)[:, None])
    _moved_by(flat(st["sh"])[:, 3:], flat(out["sh"])[:, 3:], 2e-4 * G[:, 14:] / np.sqrt(vsh)[:, None])


def test_sh_second_moment_follows_the_addition_theorem():
    # sum_m Y_lm(d)^2 = (2l + 1) / (4 pi) for every direction, so the lane-mean squared gradient is
    # |vc|^2 (a + 1)^2 / (4 pi) / 3K for active degree a: no dependence on where the splat is
    for degree, active in ((2, 2), (3, 3), (3, 1), (4, 4), (0, 0)):
        s, camd = _visible_scene(seed=20 + degree, degree=degree)
        rng = np.random.default_rng(degree)
        n, K = s.n, s.K
        vc = rng.normal(0, 1, (n, 3)).astype(np.float32)
        vs, vis, tc = _inputs(n, K, rng, vc=vc)
        out = O.adam_update(_state(s), degree, False, camd, vs, vis, tc, _grads(n, K, rng), O.adam_step(t=1),
                            active_deg=active)
        gsq = (vc.astype(np.float64) ** 2).sum(1) * (active + 1) ** 2 / (4 * math.pi) / (3 * K)
        np.testing.assert_allclose(out["v_sh"], (1.0 - float(np.float32(0.999))) * gsq, rtol=2e-6)


def test_constant_gradient_moves_by_lr_per_step():
    s, camd = _visible_scene(seed=12)
    rng = np.random.default_rng(2)
    n, K = s.n, s.K
    vs, vis, tc = _inputs(n, K, rng)
    G = _grads(n, K, rng)
    st = _state(s)
    for t in range(1, 11):
        st = O.adam_update(st, s.degree, False, camd, vs, vis, tc, G, O.adam_step(t=t, lr_mean=1e-3))
    # bias-corrected moments of a constant gradient are exactly g and g^2: ten steps of lr sign(g)
    for before, after, want in ((s.pos_op[:, :3], st["pos_op"][:, :3], 1e-2 * np.sign(G[:, :3])),
                                (s.quat, st["quat"], 2e-2 * np.sign(G[:, 4:8]))):
        d = np.asarray(before, np.float64) - after
        assert np.all(np.abs(d - want) <= 10 * np.spacing(np.abs(before)) + 1e-4 * np.abs(want))


def _run(s, camd, state, t0, gap, G1, G2, sparse, rng_seed=3):
    """Step t0 with G1, `gap` steps in which the splats have no gradient, then step t0 + gap + 1 with G2."""
    rng = np.random.default_rng(rng_seed)
    n, K = s.n, s.K
    vs, vis, tc = _inputs(n, K, rng)
    hidden = np.zeros(n, np.uint32)
    st = O.adam_update(state, s.degree, False, camd, vs, vis, tc, G1, O.adam_step(t=t0, sparse=int(sparse), lr_mean=1e-3))
    after_first = st
    for k in range(gap):
        if sparse:
            break  # a sparse trainer's steps leave these splats alone; nothing to run
        st = O.adam_update(st, s.degree, False, camd, vs, hidden, tc, np.zeros_like(G1),
                           O.adam_step(t=t0 + 1 + k, lr_mean=1e-3))
    before_last = st
    st = O.adam_update(st, s.degree, False, camd, vs, vis, tc, G2,
                       O.adam_step(t=t0 + gap + 1, sparse=int(sparse), lr_mean=1e-3))
    return after_first, before_last, st


@pytest.mark.parametrize("gap", [1, 7, 60])
def test_lazy_catch_up_equals_dense_zero_gradient_steps(gap):
    s, camd = _visible_scene(seed=13)
    rng = np.random.default_rng(4)
    n, K = s.n, s.K
    G1, G2 = _grads(n, K, rng), _grads(n, K, rng)
    t0 = 100000  # bias corrections 1 over the gap, as the catch-up assumes
    first_d, before_d, dense = _run(s, camd, _state(s), t0, gap, G1, G2, sparse=False)
    _, _, lazy = _run(s, camd, _state(s), t0, gap, G1, G2, sparse=True)
    assert np.all(lazy["last_step"] == t0 + gap + 1)
    for key, tol in (("pos_op", 1e-5), ("quat", 1e-5), ("lscale", 1e-5), ("m_pos_op", 1e-5), ("v_pos_op", 1e-5),
                     ("m_quat", 1e-5), ("v_quat", 1e-5), ("m_sh", 1e-5), ("v_sh", 1e-5)):
        d = np.abs(lazy[key].astype(np.float64) - dense[key])
        scale = np.abs(dense[key]).max() + 1e-30
        assert d.max() <= tol * scale, (key, float(d.max() / scale))
    # The SH catch-up divides by the second moment already decayed over the gap (optim.cu:346-347), so its
    # displacement is beta2^(-gap/2) times the dense steps'; the final step is the same in both runs.
    D = before_d["sh"].astype(np.float64) - first_d["sh"]
    want = dense["sh"] + D * (0.999 ** (-gap / 2.0) - 1.0)
    err = np.abs(lazy["sh"] - want)
    assert err.max() <= 1e-5 * np.abs(D).max() + 2e-7 * np.abs(dense["sh"]).max(), float(err.max())


def test_sparse_mode_leaves_splats_without_gradient_untouched():
    s, camd = _visible_scene(seed=14)
    rng = np.random.default_rng(5)
    n, K = s.n, s.K
    st = _state(s)
    st["m_pos_op"] = rng.normal(0, 1e-3, (n, 4)).astype(np.float32)
    st["v_pos_op"] = np.abs(rng.normal(0, 1e-6, (n, 4))).astype(np.float32)
    st["last_step"] = rng.integers(1, 40, n).astype(np.uint32)
    vs, vis, tc = _inputs(n, K, rng)
    vis[::2] = 0          # no gradient: not visible
    vs[1::4, :] = 0.0     # no gradient: visible but all lanes zero
    vs[3::8, 9] = 5.0     # ... the refine lane alone does not count
    G = _grads(n, K, rng)
    out = O.adam_update(st, s.degree, False, camd, vs, vis, tc, G, O.adam_step(t=50, sparse=1, lr_mean=1e-3))
    idle = (vis == 0) | ~np.any(np.delete(vs, 9, axis=1) != 0, axis=1)
    assert idle.any() and (~idle).any()
    for key in O.ADAM_STATE_KEYS:
        assert np.array_equal(out[key][idle], st[key][idle]), key
    for key in ("pos_op", "quat", "m_pos_op", "v_pos_op", "sh", "m_sh", "v_sh"):
        assert np.all(np.any((out[key] != st[key]).reshape(n, -1), axis=1)[~idle]), key
    assert np.all(out["last_step"][~idle] == 50)


def test_noise_moves_visible_low_opacity_means_by_clamped_gaussians():
    s, camd = _visible_scene(seed=15, n=40)
    rng = np.random.default_rng(6)
    n, K = s.n, s.K
    vs, vis, tc = _inputs(n, K, rng)
    tc[::3] = 0  # binned nowhere: not visible, no noise (and no gradient)
    G = np.zeros((n, 11 + 3 * K), np.float32)  # no Adam motion of the means (lr_mean 0 anyway)
    st = _state(s)
    st["pos_op"][:, 3] = -12.0  # opacity ~ 6e-6: weight (1 - o)^150 ~ 1
    st["pos_op"][1::5, 3] = 12.0  # opacity ~ 1: weight ~ 0
    base = O.adam_update(st, s.degree, False, camd, vs, vis, tc, G, O.adam_step(t=1, step=9))
    w = 1e-3
    noisy = O.adam_update(st, s.degree, False, camd, vs, vis, tc, G,
                          O.adam_step(t=1, step=9, noise_weight=w, noise_clamp=1.0))
    d = (noisy["pos_op"][:, :3] - base["pos_op"][:, :3]).astype(np.float64)
    vis_ok = tc != 0
    low = vis_ok & (st["pos_op"][:, 3] < 0)
    assert not d[~vis_ok].any()
    assert np.abs(d[vis_ok & ~low]).max() < 1e-12
    # the displacement is N(0, 1) * w (1 - o)^150; the draws are the seed's Gaussian stream at (splat, axis)
    seed = 42 ^ ((9 * 0x9E3779B9) & 0xFFFFFFFF)
    o = 1.0 / (1.0 + np.exp(-st["pos_op"][:, 3].astype(np.float64)))
    wi = w * (1.0 - o) ** 150
    want = np.array([[O.hash_gauss(seed, i, c) * wi[i] for c in range(3)] for i in range(n)])
    np.testing.assert_allclose(d[low], want[low], rtol=2e-4, atol=3e-7)
    # the clamp
    clamped = O.adam_update(st, s.degree, False, camd, vs, vis, tc, G,
                            O.adam_step(t=1, step=9, noise_weight=w, noise_clamp=2e-4))
    dc = clamped["pos_op"][:, :3].astype(np.float64) - base["pos_op"][:, :3]
    assert np.all(np.abs(dc) <= 2e-4 + 2 * np.spacing(np.abs(base["pos_op"][:, :3])))  # up to the sum's rounding
    np.testing.assert_allclose(dc[low], np.clip(want[low], -2e-4, 2e-4), rtol=2e-4, atol=3e-7)


def test_noise_stream_statistics_over_many_splats():
    x = np.array([[O.hash_gauss(42 ^ ((5 * 0x9E3779B9) & 0xFFFFFFFF), i, c) for c in range(3)] for i in range(20000)])
    assert abs(x.mean()) < 0.02 and abs(x.std() - 1) < 0.02
    assert abs(np.corrcoef(x[:, 0], x[:, 1])[0, 1]) < 0.03


def test_fp16_bands_round_stochastically_and_unbiased():
    s, camd = _visible_scene(seed=16, degree=3, n=64)
    rng = np.random.default_rng(8)
    n, K = s.n, s.K
    st = _state(s)
    # bands at 0.6-0.9 (fp16 spacing 2^-11 ~ 4.9e-4 there) and an update of 2e-4 per step: below half an ulp
    sh = st["sh"]
    sh[:, 1:, :] = rng.uniform(0.6, 0.9, (n, K - 1, 3)).astype(np.float16).astype(np.float32)
    vs, vis, tc = _inputs(n, K, rng, vc=rng.normal(0, 10, (n, 3)).astype(np.float32))  # large v_sh: small steps
    G = np.zeros((n, 11 + 3 * K), np.float32)
    G[:, 14:] = 1.0  # every band lane: gradient +1, so each step subtracts lr_sh_rest m_hat / sqrt(v_sh_hat)
    exact = O.adam_update(st, s.degree, False, camd, vs, vis, tc, G, O.adam_step(t=1))
    half = O.adam_update(st, s.degree, True, camd, vs, vis, tc, G, O.adam_step(t=1))
    e = exact["sh"][:, 1:, :].astype(np.float64)
    h = half["sh"][:, 1:, :].astype(np.float64)
    assert np.array_equal(h.astype(np.float16).astype(np.float64), h)  # stored as binary16 values
    spacing = np.spacing(np.abs(e).astype(np.float16)).astype(np.float64)
    assert np.all(np.abs(h - e) < spacing * (1 + 1e-6))  # one of the two neighbours
    moved = (h != sh[:, 1:, :]).mean()
    assert 0.05 < moved < 0.95  # a sub-half-ulp update still moves a share of the coefficients
    # unbiased: the mean stored change equals the exact change
    assert abs((h - sh[:, 1:, :]).mean() - (e - sh[:, 1:, :]).mean()) < 4 * spacing.mean() / math.sqrt(h.size)
    # the moments are rounded to nearest
    assert np.array_equal(half["m_sh"][:, 1:, :], exact["m_sh"][:, 1:, :].astype(np.float16).astype(np.float32))
