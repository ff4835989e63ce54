"""The UniPC sampler of the "unipc" chunk loop: oracle/unipc.py (the scheduler restated) pinned, and wdl/unipc.py's
linear plan against it.

Pins of the oracle (the scheduler is third-party and absent, so none of them runs it):
- the timesteps of two steps are (999, 833): the reference's first step runs at t = 999
  (scripts/conversion/export_live.py:380) and its second at t_2 = 833 (docs/research/MVP2.md:109);
- two steps are two Euler steps x_{k+1} = x_k - c_k flow_k, the assertion of export_live.py:476-479 (there to 1e-12 in
  float64), with c = (sigma_0 - sigma_1, sigma_1) in closed form;
- zero flows leave x unchanged at every step count (a consistent method; the plan's form rests on it);
- a point-mass data distribution is sampled exactly at every step count (the x0 prediction is constant, and the
  first-order x0-form update is the exact solution then; every correction term is a difference of predictions);
- the last step returns the x0 prediction of the last model input (sigma 0, the lower order at the end);
- third-order convergence of the model inputs on a Gaussian data distribution, whose flow ODE has a closed-form
  solution, over a grid even in lambda: the error ratio from 64 to 128 steps is <= 0.15 (measured 0.124; 1/8 in the
  limit). A dropped or mis-signed corrector, a mis-signed or missing second-order predictor term, or a first-order
  corrector gives 0.21 - 0.53 (checked by planting each in the oracle below).
"""

import math

import numpy as np
import pytest

from oracle import unipc as ou
from wdl import unipc as wu

MU, S = 0.7, 0.5
Z = np.linspace(-2.5, 2.5, 11)


def test_two_step_timesteps_are_the_references():
    for timesteps in (ou.schedule(2)[0], wu.schedule(2)[0]):
        assert timesteps == [999, 833]
    ts, sig = ou.schedule(2)
    assert sig[-1] == 0.0 and all(float(np.float32(s)) == s for s in sig)
    assert wu.schedule(4)[0] == [999, 937, 833, 624]


def test_two_steps_are_euler_steps_with_the_closed_form_coefficients():
    _, sig = ou.schedule(2)
    c = ou.euler_coefficients(2)
    assert abs(c[0] - (sig[0] - sig[1])) < 1e-12 and abs(c[1] - sig[1]) < 1e-12
    rng = np.random.default_rng(3)
    x, f = rng.standard_normal(7), rng.standard_normal((2, 7))
    got = ou.sample(x.copy(), lambda _x, _t, k: f[k], 2)
    assert np.abs(got - (x - c[0] * f[0] - c[1] * f[1])).max() < 1e-12  # export_live.py:476-479
    # not so at three steps: the second-order terms enter
    c3 = ou.euler_coefficients(3)
    f3 = rng.standard_normal((3, 7))
    got3 = ou.sample(x.copy(), lambda _x, _t, k: f3[k], 3)
    assert np.abs(got3 - (x - sum(ck * fk for ck, fk in zip(c3, f3)))).max() > 1e-6


@pytest.mark.parametrize("steps", range(1, 9))
def test_zero_flow_keeps_x_and_a_point_mass_is_exact(steps):
    rng = np.random.default_rng(steps)
    x = rng.standard_normal(9)
    assert np.abs(ou.sample(x.copy(), lambda _x, _t, _k: np.zeros(9), steps) - x).max() < 1e-12
    # data = a point x0*: x_sigma = (1 - sigma) x0* + sigma eps, flow = eps - x0*, the exact flow at (x, sigma)
    target = rng.standard_normal(9)
    _, sig = ou.schedule(steps)
    flow = lambda xk, _t, k: (xk - target) / sig[k]
    x_start = (1 - sig[0]) * target + sig[0] * x
    assert np.abs(ou.sample(x_start, flow, steps) - target).max() < 1e-12


@pytest.mark.parametrize("steps", [1, 2, 3, 5])
def test_the_last_step_returns_the_x0_prediction(steps):
    rng = np.random.default_rng(10 + steps)
    f = rng.standard_normal((steps, 5))
    inputs = []
    final = ou.sample(rng.standard_normal(5), lambda _x, _t, k: f[k], steps, inputs=inputs)
    _, sig = ou.schedule(steps)
    assert np.abs(final - (inputs[-1] - sig[steps - 1] * f[-1])).max() < 1e-12


def gaussian_case(steps, sample=None):
    """The model inputs' error halfway along a lambda-even grid from lambda -2 to 2, data N(MU, S^2): the exact flow
    is E[eps - x0 | x_sigma], the exact path (1 - sigma) MU + sqrt(v(sigma)) z."""
    sample = sample or ou.sample
    v = lambda sg: (1 - sg) ** 2 * S * S + sg * sg
    flow = lambda x, sg: (sg - (1 - sg) * S * S) / v(sg) * (x - (1 - sg) * MU) - MU
    exact = lambda sg: (1 - sg) * MU + math.sqrt(v(sg)) * Z
    sig = list(1 / (1 + np.exp(np.linspace(-2, 2, steps + 1))))
    inputs = []
    sample(exact(sig[0]), lambda x, _t, k: flow(x, sig[k]), steps, inputs=inputs, sigmas=sig)
    return float(np.abs(inputs[steps // 2] - exact(sig[steps // 2])).max())


def test_third_order_convergence_on_gaussian_data():
    ratio = gaussian_case(128) / gaussian_case(64)
    assert ratio <= 0.15, ratio


def _planted(monkeypatch, kind):
    """One plausible mistake in the oracle's update (the check must then fail)."""
    real = ou._update

    def update(x, m0, earlier, sig, s_t, s_0, order, corrector_t=None):
        if kind == "first-order corrector" and corrector_t is not None:
            order = 1
        if kind == "first-order predictor" and corrector_t is None:
            order = 1
        out = real(x, m0, earlier, sig, s_t, s_0, order, corrector_t)
        if kind == "mis-signed predictor term" and corrector_t is None and order == 2:
            return 2 * real(x, m0, earlier, sig, s_t, s_0, 1) - out
        if kind == "mis-signed corrector" and corrector_t is not None:
            return 2 * real(x, m0, earlier, sig, s_t, s_0, order, m0) - out
        return out

    monkeypatch.setattr(ou, "_update", update)


@pytest.mark.parametrize("kind", ["first-order corrector", "first-order predictor", "mis-signed predictor term",
                                  "mis-signed corrector"])
def test_planted_mistakes_fail_the_convergence_pin(monkeypatch, kind):
    _planted(monkeypatch, kind)
    assert gaussian_case(128) / gaussian_case(64) > 0.18


def test_a_dropped_corrector_fails_the_convergence_pin():
    def no_corrector(x, flow, steps, shift=5.0, inputs=None, sigmas=None):
        outputs = []
        for k in range(steps):
            inputs.append(x.copy())
            m = x - sigmas[k] * flow(x, k, k)
            outputs = (outputs + [(k, m)])[-2:]
            x = ou._update(x, m, [o for o in reversed(outputs[:-1])], sigmas, k + 1, k, min(2, steps - k, k + 1))
        return x

    assert gaussian_case(128, no_corrector) / gaussian_case(64, no_corrector) > 0.18


@pytest.mark.parametrize("steps", range(1, 9))
def test_plan_equals_the_oracle_sampler(steps):
    """wdl's linear plan (closed-form orders 1 and 2 on coefficient vectors) against the oracle's loop on latents:
    every model input and the result, to 1e-12."""
    timesteps, C = wu.plan(steps)
    assert timesteps == ou.schedule(steps)[0] and C.shape == (steps + 1, steps)
    assert np.all(C[np.triu_indices(steps + 1, 0, steps)] == 0)  # input k uses flows before k only
    rng = np.random.default_rng(100 + steps)
    x, f = rng.standard_normal(6), rng.standard_normal((steps, 6))
    inputs = []
    final = ou.sample(x.copy(), lambda _x, _t, k: f[k], steps, inputs=inputs)
    for k, want in enumerate(inputs + [final]):
        assert np.abs(x - C[k] @ f - want).max() < 1e-12


def test_plan_of_two_steps_is_the_exported_sampler():
    _, C = wu.plan(2)
    c = ou.euler_coefficients(2)
    assert np.allclose(C, [[0, 0], [c[0], 0], [c[0], c[1]]], atol=1e-15, rtol=0)


def test_chunk_stream_sampler_arguments():
    from wdl import model as wmodel

    with pytest.raises(ValueError):
        wmodel.ChunkStream(None, (1, 1, 2, 2), None, sampler="euler")
    with pytest.raises(ValueError):
        wmodel.ChunkStream(None, (1, 1, 2, 2), None, steps=2)
    s = wmodel.ChunkStream(None, (1, 1, 2, 2), None, sampler="unipc")
    assert s.timesteps == [999, 937, 833, 624] and len(s.plan) == 5
    with pytest.raises(ValueError):
        wu.schedule(0)
