"""Pins the CPU oracle (oracle/dsqg_oracle.py) before it is trusted as the parity reference.

The reference ships no golden tensors for DSQG (its .gitignore drops *.pt), so the oracle is
pinned by independent restatements and by what the mathematics fixes:
  * float64 brute-force loops (one query, one tap at a time);
  * the shifted-concatenate restatement of train/train_2048_condM_layer_ablation.py:96-136;
  * torch.autograd.gradcheck, and gradients derived by hand (explicit_backward);
  * closed forms and invariants (row 0, constant v, q=0 mean, one-hot bias, shift invariance,
    sum_j dbias = 0, causality, softmax sums to 1, decode ring == full-sequence row).
Each is chosen so that a dropped term, a wrong sign or index, or a transposed operand fails.
"""

import math

import pytest
import torch
import torch.nn.functional as F

from oracle import (OFFSETS_V3, OFFSETS_J46, OFFSETS_J47, brute_force_forward, decode_step,
                    dsqg_forward, dsqg_forward_backward, dsqg_weights, explicit_backward)

f64 = torch.float64


def _inputs(B, H, N, D, J, seed=0, with_se=True, with_g=True, with_a=True):
    g = torch.Generator().manual_seed(seed)
    q, k, v = (torch.randn(B, H, N, D, generator=g, dtype=f64) for _ in range(3))
    pb = torch.randn(J, H, generator=g, dtype=f64)
    se = torch.randn(J, D, generator=g, dtype=f64) * 0.3 if with_se else None
    sg = (torch.rand(H, J, generator=g, dtype=f64) + 0.5) if with_g else None
    a = (torch.rand(H, generator=g, dtype=f64) * 0.4 + 0.8) if with_a else None
    return q, k, v, pb, se, sg, a


@pytest.mark.parametrize("offsets,N", [(OFFSETS_V3, 70), (OFFSETS_J46, 50), ([0, 2, 5, 11], 19)])
@pytest.mark.parametrize("opts", [(False, False, False), (True, False, False), (True, True, True)])
def test_restatement_matches_brute_force(offsets, N, opts):
    q, k, v, pb, se, sg, a = _inputs(1, 2, N, 4, len(offsets), seed=N, with_se=opts[0],
                                     with_g=opts[1], with_a=opts[2])
    out, lse = dsqg_forward(q, k, v, pb, se, offsets, sg, a, return_lse=True)
    bo, bl = brute_force_forward(q, k, v, pb, se, offsets, sg, a)
    assert torch.allclose(out, bo, atol=1e-12, rtol=0)
    assert torch.allclose(lse, bl, atol=1e-12, rtol=0)


def _condm_form(q, k, v, pos_bias, offsets):
    """train/train_2048_condM_layer_ablation.py:96-136: shifted copies stacked over offsets."""
    B, H, N, HD = q.shape
    Ks, Vs = [], []
    for d in offsets:
        if d == 0:
            Ks.append(k); Vs.append(v)
        elif d >= N:
            Ks.append(torch.zeros_like(k)); Vs.append(torch.zeros_like(v))
        else:
            pad = k.new_zeros(B, H, d, HD)
            Ks.append(torch.cat([pad, k[:, :, :N - d]], dim=2))
            Vs.append(torch.cat([pad, v[:, :, :N - d]], dim=2))
    K_all, V_all = torch.stack(Ks, 3), torch.stack(Vs, 3)
    s = (q.unsqueeze(3) * K_all).sum(-1) * HD ** -0.5 + pos_bias.T.unsqueeze(0).unsqueeze(2)
    mask = torch.arange(N).unsqueeze(1) < torch.tensor(offsets).unsqueeze(0)
    s = s.masked_fill(mask, float("-inf"))
    return (F.softmax(s, -1).unsqueeze(-1) * V_all).sum(3)


def test_restatement_matches_condm_form():
    q, k, v, pb, _, _, _ = _inputs(2, 3, 1600, 8, 44, seed=3)
    assert torch.allclose(dsqg_forward(q, k, v, pb), _condm_form(q, k, v, pb, OFFSETS_V3),
                          atol=1e-12, rtol=0)


def test_gradcheck_float64():
    offs = [0, 1, 2, 3, 7, 12]
    q, k, v, pb, se, sg, a = _inputs(1, 2, 16, 3, len(offs), seed=5)
    args = [t.clone().requires_grad_(True) for t in (q, k, v, pb, se, sg, a)]

    def f(q, k, v, pb, se, sg, a):
        return dsqg_forward(q, k, v, pb, se, offs, sg, a)

    assert torch.autograd.gradcheck(f, args, eps=1e-6, atol=1e-7)


@pytest.mark.parametrize("offsets,N", [(OFFSETS_V3, 80), (OFFSETS_J47, 60)])
def test_autograd_matches_hand_derived_gradients(offsets, N):
    q, k, v, pb, se, sg, a = _inputs(2, 2, N, 5, len(offsets), seed=11)
    do = torch.randn(q.shape, dtype=f64, generator=torch.Generator().manual_seed(12))
    r = dsqg_forward_backward(q, k, v, pb, do, se, offsets, sg, a, dtype=f64)
    e = explicit_backward(q, k, v, pb, do, se, offsets, sg, a)
    for key in ("dq", "dk", "dv", "dpos_bias", "dscale_embed", "dscore_gain", "dif_gain"):
        assert torch.allclose(r[key], e[key], atol=1e-10, rtol=0), key


def test_row_zero_is_v0_and_constant_v():
    q, k, v, pb, se, sg, a = _inputs(2, 3, 50, 6, 44, seed=1)
    out = dsqg_forward(q, k, v, pb, se, score_gain=sg, if_gain=a)
    assert torch.allclose(out[:, :, 0], v[:, :, 0] * a.view(1, -1, 1), atol=1e-12)
    vc = torch.full_like(v, 1.75)
    assert torch.allclose(dsqg_forward(q, k, vc, pb, se), torch.full_like(v, 1.75), atol=1e-12)


def test_zero_query_zero_bias_is_mean_of_valid_taps():
    """Masked taps are excluded (not zero-padded with score 0)."""
    _, k, v, _, _, _, _ = _inputs(1, 2, 120, 4, 44, seed=2)
    q = torch.zeros_like(k)
    out = dsqg_forward(q, k, v, torch.zeros(44, 2, dtype=f64))
    for n in (0, 5, 33, 47, 48, 100, 119):
        rows = [n - d for d in OFFSETS_V3 if n - d >= 0]
        assert torch.allclose(out[0, :, n], v[0, :, rows].mean(1), atol=1e-12)


def test_one_hot_bias_selects_tap():
    q, k, v, _, _, _, _ = _inputs(1, 2, 200, 4, 44, seed=4)
    j_star = OFFSETS_V3.index(64)
    pb = torch.zeros(44, 2, dtype=f64)
    pb[j_star] = 1e4
    out = dsqg_forward(q, k, v, pb)
    assert torch.allclose(out[0, :, 64:], v[0, :, :200 - 64], atol=1e-9)


def test_bias_shift_invariance_and_weights_sum_to_one():
    q, k, v, pb, se, _, _ = _inputs(2, 2, 90, 4, 44, seed=6)
    shift = torch.tensor([3.0, -7.5], dtype=f64)
    assert torch.allclose(dsqg_forward(q, k, v, pb, se), dsqg_forward(q, k, v, pb + shift, se),
                          atol=1e-12)
    w = dsqg_weights(q, k, pb, se)
    assert torch.allclose(w.sum(-1), torch.ones(2, 2, 90, dtype=f64), atol=1e-12)
    n = torch.arange(90).view(1, 1, 90, 1)
    assert (w.masked_select(n < torch.tensor(OFFSETS_V3)) == 0).all()


def test_dbias_sums_to_zero_and_dv_formula():
    q, k, v, pb, se, _, _ = _inputs(2, 2, 100, 4, 44, seed=8)
    do = torch.randn(q.shape, dtype=f64, generator=torch.Generator().manual_seed(9))
    r = dsqg_forward_backward(q, k, v, pb, do, se, dtype=f64)
    assert torch.allclose(r["dpos_bias"].sum(0), torch.zeros(2, dtype=f64), atol=1e-10)
    w = dsqg_weights(q, k, pb, se)
    dv = torch.zeros_like(v)
    for j, d in enumerate(OFFSETS_V3):
        if d < 100:
            dv[:, :, :100 - d] += w[:, :, d:, j, None] * do[:, :, d:]
    assert torch.allclose(r["dv"], dv, atol=1e-10)


def test_causality_perturbation():
    """Changing k/v at t changes exactly the rows t + delta_j (train/train_2048_condU.py:490-506)."""
    q, k, v, pb, se, _, _ = _inputs(1, 1, 1700, 4, 44, seed=10)
    base = dsqg_forward(q, k, v, pb, se)
    t = 10
    k2, v2 = k.clone(), v.clone()
    k2[:, :, t] += 1.0
    v2[:, :, t] -= 2.0
    diff = (dsqg_forward(q, k2, v2, pb, se) - base).abs().amax(-1)[0, 0]
    changed = set(torch.nonzero(diff > 0).flatten().tolist())
    assert changed == {t + d for d in OFFSETS_V3 if t + d < 1700}


@pytest.mark.parametrize("p", [5, 40, 1536, 1600, 3100])
def test_decode_step_matches_full_sequence_row(p):
    B, H, D = 2, 3, 8
    g = torch.Generator().manual_seed(p)
    ks = torch.randn(B, H, p + 1, D, generator=g, dtype=f64)
    vs = torch.randn(B, H, p + 1, D, generator=g, dtype=f64)
    qs = torch.randn(B, H, p + 1, D, generator=g, dtype=f64)
    pb = torch.randn(44, H, generator=g, dtype=f64)
    se = torch.randn(44, D, generator=g, dtype=f64) * 0.2
    S = 1537
    k_ring = torch.full((B, H, S, D), float("nan"), dtype=f64)
    v_ring = torch.full((B, H, S, D), float("nan"), dtype=f64)
    for m in range(max(0, p - S + 1), p):           # the ring holds positions < p
        k_ring[:, :, m % S] = ks[:, :, m]
        v_ring[:, :, m % S] = vs[:, :, m]
    pos = torch.full((B,), p, dtype=torch.int64)
    out = decode_step(qs[:, :, p], ks[:, :, p], vs[:, :, p], k_ring, v_ring, pos, pb, se)
    full = dsqg_forward(qs, ks, vs, pb, se)[:, :, p]
    assert torch.allclose(out, full, atol=1e-12)
    assert torch.equal(k_ring[:, :, p % S], ks[:, :, p])
