"""The fused optimizer on the GPU (optimizer_step without grad_out: the projection VJP feeding Adam, the lazy
catch-up of sparse Adam, the SH moments with stochastically rounded fp16 bands and the MCMC noise on the
means; src/gpu/optim.cu:99-377) against the CPU restatement (oracle/orc_adam.c), bit for bit.

Each step of each case renders, scores and back-propagates one view on the GPU, keeps the screen-space
gradient (v_splat, vis_flag, tile_count), takes the parameter gradients from the gradient mode of the same
kernel (pinned against the oracle's VJP and finite differences elsewhere), restores the screen-space
gradient and runs the update. Every parameter and every Adam state array must then equal
orc_adam_update applied to the state the GPU held before the step, on the same inputs. Three steps run back
to back per case, from a random optimizer state (moments, second moments, last-update steps including
never-updated splats), with a fresh random background each step.
"""
import numpy as np
import pytest

from b2ctrain_amd import _native
from b2ctrain_amd import scenes as S
from oracle import oracle as O
from tests.gpu_harness import emit

pytestmark = pytest.mark.gpu


def _random_state(r, rng, t):
    st = r.model_state()
    n = r.n
    for k in ("m_pos_op", "m_quat", "m_lscale"):
        st[k] = rng.normal(0, 1e-3, (n, 4)).astype(np.float32)
    for k in ("v_pos_op", "v_quat", "v_lscale"):
        st[k] = np.abs(rng.normal(0, 1e-6, (n, 4))).astype(np.float32)
    st["m_lscale"][:, 3] = 0.0
    st["v_lscale"][:, 3] = 0.0
    st["m_sh"] = rng.normal(0, 1e-3, st["sh"].shape).astype(np.float32)
    st["v_sh"] = np.abs(rng.normal(0, 1e-5, n)).astype(np.float32)
    last = rng.integers(0, t, n).astype(np.uint32)  # 0 = never updated; t - 1 = updated last step
    st["last_step"] = last
    del st["pos_op"], st["quat"], st["lscale"], st["sh"]
    r.set_model_state(st)


def _same(got, want):
    g = np.ascontiguousarray(got)
    w = np.ascontiguousarray(want, g.dtype)
    if g.dtype == np.float32:
        return np.array_equal(g.view(np.uint32), w.view(np.uint32))
    return np.array_equal(g, w)


def _run_case(sc, sparse, noise, t0, steps=3, seed=1, random_state=True):
    rng = np.random.default_rng(seed)
    r = _native.Renderer(sc)
    try:
        if random_state:
            _random_state(r, rng, t0)
        camd = S.camera_gpu(sc.cam)
        gs = 3.0 * sc.W * sc.H
        changed = 0
        for k in range(steps):
            t = t0 + k
            bg = tuple(rng.random(3).astype(np.float32).tolist())
            opts = _native.adam_opts(t=t, sparse=int(sparse), lr_mean=1.6e-4 * 2.0, seed=7, step=100 + k,
                                     noise_weight=(0.02 if noise else 0.0), noise_clamp=0.03)
            emit(f"  step t={t} sparse={sparse} noise={noise}")
            r.forward(bg=bg)
            r.loss(grad_scale=gs, bg=bg)
            r.backward(mode=1, grad_scale=gs, bg=bg)
            v_splat, vis_flag, tile_count = r.read("v_splat"), r.read("vis_flag"), r.read("tile_count")
            r.vjp()
            grads = r.read("grads")
            r.write("v_splat", v_splat)
            r.write("vis_flag", vis_flag)
            before = r.model_state()
            r.adam(opts, bg=bg)
            after = r.model_state()
            step = O.adam_step(**{f: getattr(opts, f) for f, _ in _native.AdamOpts._fields_})
            want = O.adam_update(before, sc.degree, sc.sh_fp16, camd, v_splat, vis_flag, tile_count, grads, step)
            bad = [key for key in O.ADAM_STATE_KEYS if not _same(after[key], want[key])]
            for key in bad:
                d = np.abs(after[key].astype(np.float64) - want[key])
                emit(f"    {key}: {int((d > 0).sum())} entries differ, max {float(d.max()):.3g}")
            assert not bad, bad
            assert not np.any(r.read("v_splat")) and not np.any(r.read("vis_flag"))  # consumed and cleared
            changed += int(np.any(after["pos_op"] != before["pos_op"], axis=1).sum())
            if sparse:
                has = (vis_flag != 0) & (tile_count != 0)
                assert np.all(after["last_step"][~has] == before["last_step"][~has])
        assert changed > 0
    finally:
        r.close()


def _fd(degree=2):
    return S.fd_scene(31, n=24, degree=degree)


CASES = {
    # name: (scene, sparse, noise, first step)
    "fd_sh2_dense_from_zero": (lambda: _fd(), False, False, 1),
    "fd_sh2_sparse_noise": (lambda: _fd(), True, True, 50),
    "cfg1_sh0_dense_noise": (lambda: S.config1(), False, True, 4),
    "cfg2_20k_sh3_dense_noise": (lambda: S.config2(n=20_000), False, True, 7),
    "cfg2_20k_sh3_sparse": (lambda: S.config2(n=20_000), True, False, 300),
    "cfg5_20k_sh3_fp16_sparse_noise": (lambda: S.config5(n=20_000), True, True, 30),
    "cfg5_20k_sh3_fp16_dense": (lambda: S.config5(n=20_000), False, False, 2),
    "cfg4_sh4_sparse_noise": (lambda: S.config4(shrink=8), True, True, 12),
}


@pytest.mark.timeout(300)
@pytest.mark.parametrize("case", list(CASES))
def test_fused_update_matches_oracle(case):
    build, sparse, noise, t0 = CASES[case]
    sc = build()
    emit(f"adam {case}: {sc.n} splats SH{sc.degree}{' fp16' if sc.sh_fp16 else ''} {sc.W}x{sc.H}")
    _run_case(sc, sparse, noise, t0, random_state=t0 > 1)


STATS = ("vis_weight", "vis_count", "refine_norm")


@pytest.mark.timeout(300)
def test_train_step_adam_equals_the_staged_update():
    """b2c_train_step_adam = forward, loss, backward, fused update, with the same visibility statistics (the
    fused step passes visibility to the update in the v_splat rows, the staged calls in vis_flag); and t = 0
    advances the model's counter."""
    sc = S.config2(n=20_000)
    emit(f"adam train_step: {sc.n} splats")
    bg = (0.3, 0.2, 0.1)
    gs = 3.0 * sc.W * sc.H
    opts = _native.adam_opts(t=0, lr_mean=3e-4, noise_weight=40.0, noise_clamp=0.05, step=3)
    states = []
    for staged in (False, True):
        r = _native.Renderer(sc)
        try:
            for _ in range(2):
                if staged:
                    r.forward(bg=bg)
                    r.loss(grad_scale=gs, bg=bg)
                    r.backward(mode=1, grad_scale=gs, bg=bg)
                    r.adam(opts, bg=bg)
                else:
                    r.step_adam(opts, bg=bg)
            assert r.adam_t() == 2
            st = r.model_state()
            st.update({k: r.read_model(k) for k in STATS})
            states.append(st)
        finally:
            r.close()
    for key in O.ADAM_STATE_KEYS + STATS:
        assert _same(states[0][key], states[1][key]), key
