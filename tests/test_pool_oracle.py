"""Pinning the causal-mean pool oracle (oracle/pool_oracle.py) on the CPU.

The restatement of train/train_2048_condU.py:289-292 is checked against an explicit-loop brute
force (mean of the first n+1 rows), its autograd gradients against the closed forms derived by
hand, torch.autograd.gradcheck in float64, and special cases fixed by the mathematics: constant
input, saturated gate, and a one-hot row (causality: row m only reaches rows n >= m, with
weight 1/(n+1)).  An off-by-one in the counts, an exclusive instead of inclusive sum, or a
prefix instead of a suffix sum in dx fails one of these.
"""

import pytest
import torch

from oracle import (pool_gate_brute_force, pool_gate_explicit_backward, pool_gate_forward,
                    pool_gate_forward_backward)


def _inputs(B, N, C, seed=0, dtype=torch.float64):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn((B, N, C), generator=g, dtype=dtype)
    gp = torch.randn((B, N, C), generator=g, dtype=dtype) * 2
    dy = torch.randn((B, N, C), generator=g, dtype=dtype)
    return x, gp, dy


@pytest.mark.parametrize("shape", [(1, 1, 8), (2, 7, 8), (1, 13, 16)])
def test_pool_forward_matches_brute_force(shape):
    x, gp, _ = _inputs(*shape)
    torch.testing.assert_close(pool_gate_forward(x, gp), pool_gate_brute_force(x, gp),
                               rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("shape", [(1, 1, 8), (2, 9, 8), (1, 17, 16)])
def test_pool_autograd_matches_closed_form(shape):
    x, gp, dy = _inputs(*shape, seed=1)
    out, dx, dg = pool_gate_forward_backward(x, gp, dy)
    ex_dx, ex_dg = pool_gate_explicit_backward(x, gp, dy)
    torch.testing.assert_close(out, pool_gate_brute_force(x, gp), rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(dx, ex_dx, rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(dg, ex_dg, rtol=1e-12, atol=1e-12)


def test_pool_gradcheck_float64():
    x, gp, _ = _inputs(2, 6, 8, seed=2)
    x.requires_grad_(True)
    gp.requires_grad_(True)
    assert torch.autograd.gradcheck(lambda a, b: pool_gate_forward(a, b), (x, gp))


def test_pool_special_cases():
    B, N, C = 2, 11, 8
    # constant input: the causal mean is the constant; a saturated gate passes it through
    x = torch.full((B, N, C), 0.75, dtype=torch.float64)
    big = torch.full((B, N, C), 60.0, dtype=torch.float64)
    torch.testing.assert_close(pool_gate_forward(x, big), x, rtol=0, atol=1e-15)
    # zero gate pre-activation: s = 1/2 exactly
    torch.testing.assert_close(pool_gate_forward(x, torch.zeros_like(x)), x / 2, rtol=0, atol=1e-15)
    # one-hot row m: rows before it see 0, rows n >= m see 1/(n+1)
    m = 4
    x = torch.zeros((B, N, C), dtype=torch.float64)
    x[:, m, :] = 1.0
    out = pool_gate_forward(x, big)
    want = torch.tensor([0.0 if n < m else 1.0 / (n + 1) for n in range(N)], dtype=torch.float64)
    torch.testing.assert_close(out[0, :, 0], want, rtol=0, atol=1e-15)
    # dx for dout = 1 at zero gate: 0.5 * (H_N - H_m), H the harmonic numbers
    x, gp, _ = _inputs(B, N, C, seed=3)
    _, dx, _ = pool_gate_forward_backward(x, torch.zeros_like(gp), torch.ones_like(x))
    H = [sum(1.0 / k for k in range(1, n + 1)) for n in range(N + 1)]
    want = torch.tensor([0.5 * (H[N] - H[m]) for m in range(N)], dtype=torch.float64)
    torch.testing.assert_close(dx[1, :, 3], want, rtol=1e-13, atol=1e-15)


def test_pool_gate_rounding_to_gate_dtype():
    # The sigmoid is taken in the gate's dtype: a float16 gate rounds s to float16 first.
    x, gp, _ = _inputs(1, 5, 8, seed=4)
    g16 = gp.to(torch.float16)
    out = pool_gate_forward(x, g16)
    s16 = torch.sigmoid(g16).double()
    counts = torch.arange(1, 6, dtype=torch.float64).view(1, 5, 1)
    torch.testing.assert_close(out, s16 * x.cumsum(1) / counts, rtol=1e-15, atol=0)
    assert not torch.allclose(out, pool_gate_forward(x, g16.double()), rtol=1e-6, atol=0)
