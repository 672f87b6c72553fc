"""CPU restatement (numpy, float64) of one Poisson-loss training step with Adam on the packed
parameter buffer.

TEST INFRASTRUCTURE ONLY: the checker for the fused training step (fhoad_poisson_adam_step).
Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may use it.

What it restates:

* ``adam_update``: Adam (Kingma and Ba, "Adam: A Method for Stochastic Optimization", ICLR
  2015, Algorithm 1) in the form torch.optim.Adam documents (amsgrad = False, maximize = False,
  L2 weight decay added to the gradient), the optimizer of
  /root/reference/benchmarks/benchmark_training.py:41 (``torch.optim.Adam(lr=1e-3)``):
  ``g += wd p; m = b1 m + (1 - b1) g; v = b2 v + (1 - b2) g^2;
  p -= lr (m / (1 - b1^t)) / (sqrt(v / (1 - b2^t)) + eps)``.
* ``poisson_adam_step``: the step of /root/reference/benchmarks/benchmark_training.py:46-60
  and, with boundary points, of /root/reference/benchmarks/train_poisson.py:30-45 (loss of
  src/fused_hoad/training.py:66-88):
  ``loss = mean((lap - f)^2) + w mean(u_b^2)`` from the forward jet (``jet.forward``),
  backward with the upstream gradients autograd forms for that loss (interior:
  grad_u = 0, grad_lap = 2 (lap - f) / B; boundary: grad_u = 2 w u_b / B_b, grad_lap = 0, fed
  to ``jet.backward``), then ``adam_update`` of the packed buffer (Adam is elementwise, so
  running it on the packed 12,737 floats equals running it per parameter tensor).

How it is pinned (tests/test_adam_oracle.py): against torch.optim.Adam itself on the CPU in
float64 (the library routine the reference calls) over several steps with and without
weight decay; against the closed form of the first step from zero state
(``p1 = p0 - lr g / (|g| + eps)``); against planted mistakes (a dropped bias correction, a
swapped beta) that those checks must reject; and, for the loss seed, against torch autograd
of ``(lap - f).pow(2).mean()``; the whole step, boundary term included, against a float64
torch training step with autograd and torch.optim.Adam.
"""

from __future__ import annotations

import numpy as np

from oracle import jet


def adam_update(params, grad, exp_avg, exp_avg_sq, step, *, lr=1e-3, beta1=0.9, beta2=0.999,
                eps=1e-8, weight_decay=0.0):
    """One Adam update. ``step`` is the step count after this update (1 for the first).

    Returns new ``(params, exp_avg, exp_avg_sq)``; the inputs are not modified.
    """
    p = np.asarray(params, dtype=np.float64)
    g = np.asarray(grad, dtype=np.float64)
    if weight_decay:
        g = g + weight_decay * p
    m = beta1 * np.asarray(exp_avg, dtype=np.float64) + (1.0 - beta1) * g
    v = beta2 * np.asarray(exp_avg_sq, dtype=np.float64) + (1.0 - beta2) * g * g
    m_hat = m / (1.0 - beta1**step)
    v_hat = v / (1.0 - beta2**step)
    return p - lr * m_hat / (np.sqrt(v_hat) + eps), m, v


def poisson_seed(lap, source):
    """``(loss, grad_lap)`` of ``mean((lap - f)^2)`` over the batch."""
    r = np.asarray(lap, dtype=np.float64).reshape(-1) - np.asarray(source, dtype=np.float64).reshape(-1)
    return float(np.mean(r * r)), 2.0 * r / r.size


def poisson_adam_step(params, coordinates, source, exp_avg, exp_avg_sq, step, *, boundary=None,
                      boundary_weight=100.0, **adam):
    """One fused step: loss and gradients at ``params``, then Adam.

    ``step`` is the step count after this update. With ``boundary`` points the loss gains
    ``boundary_weight * mean(u(boundary)^2)``. Returns a dict with ``loss``,
    ``grad_parameters``, ``grad_coordinates`` (interior points), ``params``, ``exp_avg``,
    ``exp_avg_sq``.
    """
    p = np.asarray(params, dtype=np.float64)
    x = np.asarray(coordinates, dtype=np.float64)
    _, lap = jet.forward(p, x)
    loss, grad_lap = poisson_seed(lap, source)
    grad_p, grad_x = jet.backward(p, x, np.zeros_like(grad_lap), grad_lap)
    if boundary is not None and len(boundary):
        xb = np.asarray(boundary, dtype=np.float64)
        ub, _ = jet.forward(p, xb)
        loss += boundary_weight * float(np.mean(ub * ub))
        grad_pb, _ = jet.backward(p, xb, 2.0 * boundary_weight * ub / ub.size, np.zeros_like(ub))
        grad_p = grad_p + grad_pb
    new_p, m, v = adam_update(p, grad_p, exp_avg, exp_avg_sq, step, **adam)
    return {
        "loss": loss,
        "grad_parameters": grad_p,
        "grad_coordinates": grad_x,
        "params": new_p,
        "exp_avg": m,
        "exp_avg_sq": v,
    }
