"""The UniPC sampler of the reference's "unipc" chunk loop (generation/causal.py:620-636) as a linear plan.

The reference runs LongLive 2.0's FlowUniPCMultistepScheduler (wan_5b/utils/fm_solvers_unipc.py, Wan 2.1's
flow-matching form of the UniPC method of Zhao et al., NeurIPS 2023) built with num_train_timesteps 1000, shift 1,
no dynamic shifting, then set_timesteps(steps, shift=5): solver order 2, x0 prediction, B(h) = expm1(-h) ("bh2"),
lower order at the last step, the corrector on at every step, final sigma 0.

With its noise levels fixed, every update of that sampler is linear in the chunk's noise x_0 and the model's flows,
and zero flows leave x where it is. So the model input of step k is x_k = x_0 - sum_{j<k} C[k, j] flow_j and the clean
latents are x_0 - sum_j C[steps, j] flow_j; plan() computes C once, in float64 on the host, by running the
predictor / corrector recurrence on the coefficients of (x_0, flow_0, ..) instead of on latents. Two steps reduce to
two Euler steps, x_{k+1} = x_k - c_k flow_k with c = (sigma_0 - sigma_1, sigma_1): the coefficients the reference
exports as the live sampler (scripts/conversion/export_live.py:452-480, which asserts that form).

Updates, from noise level s to t, in the x0 form: lambda = log((1 - sigma) / sigma), h = lambda_t - lambda_s,
g = 1 - exp(-h), m = x - sigma flow the model's x0 prediction;
  predictor, order 1:  x_t = (sigma_t / sigma_s) x + alpha_t g m_s
  predictor, order 2:  ... + alpha_t g rho D1, rho = 1/2, D1 = (m_{s-1} - m_s) / r, r = (lambda_{s-1} - lambda_s) / h
  corrector, order 1:  x_t = (sigma_t / sigma_s) x_s + alpha_t g (m_s + (m_t - m_s) / 2), m_t at the predicted x_t
  corrector, order 2:  ... + alpha_t g (rho_1 D1 + rho_2 (m_t - m_s)), (rho_1, rho_2) solving
                       [[1, 1], [r, 1]] rho = (phi_1 / B, 2 phi_2 / B) of the bh2 recursion.
The model is evaluated at the predicted (uncorrected) sample; the order is min(2, steps - k, k + 1).
"""

from __future__ import annotations

import math

import numpy as np

SHIFT = 5.0
ORDER = 2
TRAIN_STEPS = 1000


def schedule(steps: int, shift: float = SHIFT):
    """set_timesteps(steps, shift): the integer timesteps the model sees and the noise levels [steps + 1] (float32
    values as the scheduler keeps them, the last 0). sigma_max is the largest training sigma, float32(1 - 1/1000);
    the levels are spaced evenly below it, shifted s -> S s / (1 + (S - 1) s), and the timesteps are 1000 s
    truncated: (999, 833) for two steps at shift 5."""
    if not isinstance(steps, int) or steps < 1:
        raise ValueError("steps must be a positive integer")
    sigma_max = float(np.float32(1.0 - 1.0 / TRAIN_STEPS))
    raw = np.linspace(sigma_max, 0.0, steps + 1)[:-1]
    shifted = shift * raw / (1 + (shift - 1) * raw)
    timesteps = [int(t) for t in shifted * TRAIN_STEPS]
    return timesteps, [float(np.float32(s)) for s in shifted] + [0.0]


def _lam(sigma: float) -> float:
    return math.inf if sigma == 0 else math.log((1 - sigma) / sigma)


def _predict(x, m, m_older, sig, k: int, order: int):
    """UniP from level k to k + 1 (x the corrected sample at k, m its model output, m_older the one of k - 1)."""
    s, t = sig[k], sig[k + 1]
    if t == 0:  # h = inf: the x0 prediction itself
        if order != 1:
            raise AssertionError("the last step is first order")
        return m.copy()
    h = _lam(t) - _lam(s)
    g = -math.expm1(-h)
    out = (t / s) * x + (1 - t) * g * m
    if order == 2:
        r = (_lam(sig[k - 1]) - _lam(s)) / h
        out = out + (1 - t) * g * 0.5 * (m_older - m) / r
    return out


def _correct(x, m_s, m_older, m_t, sig, k: int, order: int):
    """UniC of the step from level k - 1 to k: x the corrected sample at k - 1, m_s its model output, m_older the
    one of k - 2, m_t the model output at the predicted sample of level k."""
    s, t = sig[k - 1], sig[k]
    h = _lam(t) - _lam(s)
    g = -math.expm1(-h)
    out = (t / s) * x + (1 - t) * g * m_s
    if order == 1:
        return out + (1 - t) * g * 0.5 * (m_t - m_s)
    r = (_lam(sig[k - 2]) - _lam(s)) / h
    phi1 = g / h - 1                # h phi_1(h) / (-h) - 1 of the bh2 recursion, hh = -h
    phi2 = -phi1 / h - 0.5
    b1, b2 = phi1 / -g, 2 * phi2 / -g
    rho1 = (b1 - b2) / (1 - r)
    rho2 = b1 - rho1
    return out + (1 - t) * g * (rho1 * (m_older - m_s) / r + rho2 * (m_t - m_s))


def plan(steps: int, shift: float = SHIFT):
    """(timesteps [steps], C float64 [steps + 1, steps]): the model input of step k is x_0 - C[k] . flows and the
    clean latents x_0 - C[steps] . flows (row 0 is zero)."""
    timesteps, sig = schedule(steps, shift)
    basis = np.eye(steps + 1)  # coefficients over (x_0, flow_0, .., flow_{steps-1})
    x = basis[0]
    rows = []
    m_older = m_prev = x_prev = None
    order_prev = 0
    for k in range(steps):
        rows.append(x)
        m = x - sig[k] * basis[1 + k]
        if k > 0:
            x = _correct(x_prev, m_prev, m_older, m, sig, k, order_prev)
        order = min(ORDER, steps - k, k + 1)
        x_prev, order_prev = x, order
        x = _predict(x, m, m_prev, sig, k, order)
        m_older, m_prev = m_prev, m
    rows.append(x)
    X = np.stack(rows)
    if np.abs(X[:, 0] - 1).max() > 1e-9:
        raise AssertionError("the sampler moved x with zero flows")
    return timesteps, -X[:, 1:]
