"""CPU oracle for the causal-mean pool with a sigmoid gate -- TEST INFRASTRUCTURE ONLY.

Restates the interference pool of the reference's DWARF block, train/train_2048_condU.py:
289-292:

    counts = arange(1, N + 1).view(1, N, 1)
    pool   = xi.cumsum(dim=1) / counts
    inter  = sigmoid(inter_gate(xi)) * pool

with ``gate_pre`` standing for ``inter_gate(xi)`` (an ordinary Linear the caller applies).
Like the rest of ``oracle/`` it is the checker, never the product: only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline leg use it.

* ``pool_gate_forward`` -- the three lines above, followed literally in torch on the CPU
  (float64 by default), with the sigmoid taken in (and rounded to) gate_pre's dtype as torch
  does for a gate tensor of that dtype.
* ``pool_gate_forward_backward`` -- gradients of the above through torch autograd, the way the
  reference trains through it.
* ``pool_gate_brute_force`` / ``pool_gate_explicit_backward`` -- independent restatements used
  to pin the two: the mean of the first n+1 rows by a Python loop, and the closed-form
  gradients ``dgate = dout * pool * s * (1 - s)``, ``dx[m] = sum_{n>=m} dout[n] s[n] / (n+1)``
  by explicit loops (tests/test_oracle.py).
"""

from __future__ import annotations

import torch


def _sigmoid_in(gate_pre: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """sigmoid taken in gate_pre's own dtype (as the reference's torch.sigmoid(inter_gate(xi))
    is), then widened to the oracle's arithmetic dtype."""
    return torch.sigmoid(gate_pre).to(dtype)


def pool_gate_forward(x: torch.Tensor, gate_pre: torch.Tensor,
                      dtype: torch.dtype = torch.float64) -> torch.Tensor:
    """sigmoid(gate_pre) * x.cumsum(1) / counts; train/train_2048_condU.py:289-292."""
    B, N, C = x.shape
    counts = torch.arange(1, N + 1, dtype=dtype).view(1, N, 1)
    pool = x.to(dtype).cumsum(dim=1) / counts
    return _sigmoid_in(gate_pre, dtype) * pool


def pool_gate_forward_backward(x: torch.Tensor, gate_pre: torch.Tensor, dout: torch.Tensor,
                               dtype: torch.dtype = torch.float64):
    """(out, dx, dgate_pre) in ``dtype`` through torch autograd of the forward above.

    The sigmoid is differentiated in the arithmetic dtype; its value is rounded to gate_pre's
    dtype the same way as in the forward (the rounding passes the gradient straight through).
    """
    xl = x.detach().to(dtype).requires_grad_(True)
    gl = gate_pre.detach().to(dtype).requires_grad_(True)
    B, N, C = x.shape
    counts = torch.arange(1, N + 1, dtype=dtype).view(1, N, 1)
    pool = xl.cumsum(dim=1) / counts
    s = torch.sigmoid(gl)
    if gate_pre.dtype != dtype:  # value rounded to the gate's dtype, gradient unchanged
        s = s + (s.detach().to(gate_pre.dtype).to(dtype) - s.detach())
    out = s * pool
    out.backward(dout.detach().to(dtype))
    return out.detach(), xl.grad, gl.grad


def pool_gate_brute_force(x, gate_pre):
    """out[b,n,c] = sigmoid(g) * mean(x[b,0..n,c]) by explicit loops in float64 (tiny shapes)."""
    B, N, C = x.shape
    xd = x.double()
    s = torch.sigmoid(gate_pre.double())
    out = torch.empty((B, N, C), dtype=torch.float64)
    for b in range(B):
        for n in range(N):
            for c in range(C):
                acc = 0.0
                for m in range(n + 1):
                    acc += float(xd[b, m, c])
                out[b, n, c] = float(s[b, n, c]) * acc / (n + 1)
    return out


def pool_gate_explicit_backward(x, gate_pre, dout):
    """Closed-form gradients by explicit loops in float64 (tiny shapes):
    dgate = dout * pool * s * (1 - s);  dx[m] = sum_{n>=m} dout[n] * s[n] / (n + 1)."""
    B, N, C = x.shape
    xd, dy = x.double(), dout.double()
    s = torch.sigmoid(gate_pre.double())
    dx = torch.zeros((B, N, C), dtype=torch.float64)
    dg = torch.zeros((B, N, C), dtype=torch.float64)
    for b in range(B):
        for c in range(C):
            run = 0.0
            for n in range(N):
                run += float(xd[b, n, c])
                sv = float(s[b, n, c])
                dg[b, n, c] = float(dy[b, n, c]) * (run / (n + 1)) * sv * (1.0 - sv)
            tail = 0.0
            for m in range(N - 1, -1, -1):
                tail += float(dy[b, m, c]) * float(s[b, m, c]) / (m + 1)
                dx[b, m, c] = tail
    return dx, dg
