"""The UniPC flow-matching sampler on the CPU — test infrastructure, a restatement of the scheduler the reference's
"unipc" sampler runs (generation/causal.py:620-636; scripts/conversion/export_live.py:452-480 derives its 2-step
coefficients from it). Only tests/ may import it.

The scheduler itself is third-party and absent from the reference tree: LongLive 2.0's wan_5b/utils/
fm_solvers_unipc.py (FlowUniPCMultistepScheduler, Wan 2.1's flow-matching port of diffusers' UniPCMultistepScheduler,
itself the published method of Zhao et al., "UniPC: A Unified Predictor-Corrector Framework for Fast Sampling of
Diffusion Models", NeurIPS 2023). The reference builds it as FlowUniPCMultistepScheduler(num_train_timesteps=1000,
shift=1, use_dynamic_shifting=False) and calls set_timesteps(steps, shift=5); the defaults it keeps are
solver_order 2, predict_x0, solver_type "bh2", lower_order_final, no disabled corrector, final sigma 0. Restated
here in float64 (the scheduler computes its scalars in float32, so its coefficients agree with these to ~1e-6
relative):

  schedule   sigma_max = float32(1 - 1/1000) = 0.999.., sigma_min = 0 (the unshifted training sigmas of __init__);
             sigmas = linspace(sigma_max, 0, steps + 1)[:-1], shifted s -> S s / (1 + (S - 1) s) in float64,
             timesteps = int64(1000 sigma) (truncated), then sigma_steps = 0 appended and all kept as float32.
  step k     m_k = x_k - sigma_k flow_k (the x0 prediction of a flow model);
             for k > 0 the corrector UniC (order p_{k-1}, rho 0.5 at order 1, else solve(R, b)) replaces x_k by
             x^c_k, the model having been evaluated at the uncorrected x_k;
             p_k = min(2, steps - k, k + 1); the predictor UniP of order p_k (rho 0.5 at order 2) from x^c_k gives
             x_{k+1}, both in the x0 form with B(h) = expm1(-h), h = lambda_t - lambda_s, lambda = log(alpha/sigma),
             alpha = 1 - sigma.

Pinned by (tests/test_unipc.py): the reference script's own assertion that 2 steps are two Euler steps x_{k+1} =
x_k - c_k flow_k (export_live.py:476-479), with c = (sigma_0 - sigma_1, sigma_1) the closed form; exactness for a
point-mass data distribution (the x0 prediction constant: every order reproduces the exact flow ODE solution);
consistency (zero flow leaves x unchanged, at every step count); and the convergence order on a Gaussian data
distribution, whose flow ODE has a closed-form solution: the error falls at least as the square of the step
(Euler's falls linearly), which fails if the corrector or the second-order terms are dropped or mis-signed.
"""

from __future__ import annotations

import math

import numpy as np

ORDER = 2  # solver_order


def _f32(v: float) -> float:
    return float(np.float32(v))


def schedule(steps: int, shift: float = 5.0):
    """set_timesteps(steps, shift=shift) of a scheduler built with shift=1: (timesteps [steps] ints, sigmas
    [steps + 1] floats holding float32 values, the last 0)."""
    sigma_max = _f32(1.0 - 1.0 / 1000)  # sigmas[0] of __init__: 1 - alphas, alphas = linspace(1, 1/1000, 1000)[::-1]
    raw = np.linspace(sigma_max, 0.0, steps + 1)[:-1]
    shifted = shift * raw / (1 + (shift - 1) * raw)
    timesteps = [int(t) for t in (shifted * 1000)]
    return timesteps, [_f32(s) for s in shifted] + [0.0]


def _lam(sigma: float) -> float:
    """lambda = log(alpha) - log(sigma), alpha = 1 - sigma; +inf at sigma = 0."""
    return math.inf if sigma == 0 else math.log(1 - sigma) - math.log(sigma)


def _rhs(h: float, order: int, rks: list):
    """The matrix R (rows rks^(i-1)) and vector b of the bh2 update (h phi_k(h) recursion), hh = -h (x0 form)."""
    hh = -h
    h_phi_1 = math.expm1(hh)
    b_h = math.expm1(hh)
    h_phi_k = h_phi_1 / hh - 1
    factorial = 1
    R, b = [], []
    for i in range(1, order + 1):
        R.append([r ** (i - 1) for r in rks])
        b.append(h_phi_k * factorial / b_h)
        factorial *= i + 1
        h_phi_k = h_phi_k / hh - 1 / factorial
    return np.array(R), np.array(b), h_phi_1, b_h


def _update(x, m0, earlier, sig, s_t: int, s_0: int, order: int, corrector_t=None):
    """The x0-form UniP (corrector_t None) or UniC update from x at sigmas[s_0] to sigmas[s_t]: m0 the model output
    at s_0, earlier [(index, model output)] the older ones (nearest first), corrector_t the output at s_t."""
    lam_t, lam_0 = _lam(sig[s_t]), _lam(sig[s_0])
    h = lam_t - lam_0
    rks, d1s = [], []
    for si, mi in earlier[:order - 1]:
        rk = (_lam(sig[si]) - lam_0) / h
        rks.append(rk)
        d1s.append((mi - m0) / rk)
    rks.append(1.0)
    R, b, h_phi_1, b_h = _rhs(h, order, rks)
    alpha_t = 1 - sig[s_t]
    x_t = sig[s_t] / sig[s_0] * x - alpha_t * h_phi_1 * m0
    if corrector_t is None:  # UniP
        if not d1s:
            return x_t
        rhos = [0.5] if order == 2 else np.linalg.solve(R[:-1, :-1], b[:-1])
        return x_t - alpha_t * b_h * sum(r * d for r, d in zip(rhos, d1s))
    rhos = [0.5] if order == 1 else np.linalg.solve(R, b)  # UniC
    res = sum(r * d for r, d in zip(rhos[:-1], d1s)) + rhos[-1] * (corrector_t - m0)
    return x_t - alpha_t * b_h * res


def sample(x, flow, steps: int, shift: float = 5.0, inputs: list | None = None, sigmas: list | None = None):
    """The scheduler's loop (causal.py:632-636): x float64 array, flow(x, t, k) the model's flow at step k (t the
    integer timestep). Returns the final latents; `inputs`, if given, receives each model input x_k. `sigmas`
    ([steps + 1], decreasing) replaces the schedule's noise levels (the timesteps then count the steps)."""
    timesteps, sig = schedule(steps, shift) if sigmas is None else (list(range(steps)), list(sigmas))
    outputs = []  # [(step, m)] newest last
    last = None   # (the corrected sample of the previous step, its order)
    for k, t in enumerate(timesteps):
        if inputs is not None:
            inputs.append(x.copy())
        m = x - sig[k] * flow(x, t, k)
        if last is not None:  # UniC on the previous step, the model output of this one known
            prev, order = last
            x = _update(prev, outputs[-1][1], [(s, o) for s, o in reversed(outputs[:-1])], sig, k, k - 1, order,
                        corrector_t=m)
        outputs = (outputs + [(k, m)])[-ORDER:]
        order = min(ORDER, steps - k, k + 1)
        last = (x, order)
        x = _update(x, m, [(s, o) for s, o in reversed(outputs[:-1])], sig, k + 1, k, order)
    return x


def euler_coefficients(steps: int, shift: float = 5.0) -> list:
    """c_k of x_{k+1} = x_k - c_k flow_k, read off the sampler with unit flows (export_live.py:468-474): minus the
    latents after step k when x_0 = 0 and only flow_k is 1. The form holds for steps <= 2 only."""
    coefficients = []
    for k in range(steps):
        inputs = []
        final = sample(np.zeros(1), lambda x, t, j: np.full(1, float(j == k)), steps, shift, inputs)
        coefficients.append(-float((inputs[1:] + [final])[k][0]))
    return coefficients
