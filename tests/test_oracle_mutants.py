"""The oracle's pins catch plausible mistakes: each test plants one mistake in a copy of the
oracle's score function (or of the pool restatement), on the CPU, and checks that the pins
used in test_oracle.py / test_pool_oracle.py reject it while the unmodified oracle passes.
Mistakes planted: dropped bias, bias not transposed, wrong scale, gather index off by one,
mask off by one, flipped scale_embed sign, gain applied to the bias, exclusive instead of
inclusive cumsum, counts off by one, prefix instead of suffix sum in dx.
"""

import pytest
import torch
import torch.nn.functional as F

import oracle.dsqg_oracle as O
from oracle import brute_force_forward, pool_gate_brute_force, pool_gate_explicit_backward

f64 = torch.float64


def _scores_variant(mistake):
    """A copy of the oracle's masked-score function with one planted mistake."""
    def scores(q, k, pos_bias, scale_embed, offsets, score_gain):
        B, H, N, HD = q.shape
        sc = HD ** -0.5
        if mistake == "scale":
            sc = 1.0 / HD
        off = torch.tensor(list(offsets), dtype=torch.long)
        maxd = int(off.max())
        kp = F.pad(k, (0, 0, maxd, 0))
        ni = torch.arange(N)
        gi = maxd - off[None, :] + ni[:, None]
        if mistake == "index":
            gi = (gi - 1).clamp(min=0)
        s = (q.unsqueeze(3) * kp[:, :, gi, :]).sum(-1) * sc
        if score_gain is not None and mistake != "gain_on_bias":
            s = s * score_gain[None, :, None, :]
        if mistake == "no_bias":
            pass
        elif mistake == "bias_untransposed":
            s = s + pos_bias.reshape(pos_bias.shape[1], pos_bias.shape[0])[None, :, None, :]
        else:
            s = s + pos_bias.T[None, :, None, :]
        if mistake == "gain_on_bias" and score_gain is not None:
            s = s * score_gain[None, :, None, :]
        if scale_embed is not None:
            t = (q.unsqueeze(3) * scale_embed[None, None, :, :]).sum(-1) * sc
            s = s - t if mistake == "se_sign" else s + t
        cmp = (ni[:, None] <= off[None, :]) if mistake == "mask" else (ni[:, None] < off[None, :])
        s = s.masked_fill(cmp.unsqueeze(0).unsqueeze(0), float("-inf"))
        return s, gi, maxd
    return scores


def _pins_hold():
    """The forward pins of test_oracle.py, on small float64 cases: brute force (with every
    optional term), row 0 = v[0], and q = 0, bias = 0 giving the mean of the valid taps."""
    g = torch.Generator().manual_seed(0)
    offs = [0, 1, 2, 3, 7, 12]
    B, H, N, D, J = 1, 2, 20, 4, len(offs)
    q, k, v = (torch.randn(B, H, N, D, generator=g, dtype=f64) for _ in range(3))
    pb = torch.randn(J, H, generator=g, dtype=f64)
    se = torch.randn(J, D, generator=g, dtype=f64) * 0.3
    sg = torch.rand(H, J, generator=g, dtype=f64) + 0.5
    out = O.dsqg_forward(q, k, v, pb, se, offs, sg)
    if not torch.allclose(out, brute_force_forward(q, k, v, pb, se, offs, sg)[0], atol=1e-10, rtol=0):
        return False
    if not torch.allclose(O.dsqg_forward(q, k, v, pb, None, offs)[:, :, 0], v[:, :, 0], atol=1e-12):
        return False
    zero = O.dsqg_forward(torch.zeros_like(q), k, v, torch.zeros_like(pb), None, offs)
    want = torch.stack([v[:, :, [n - d for d in offs if n - d >= 0]].mean(2) for n in range(N)], 2)
    return torch.allclose(zero, want, atol=1e-12, rtol=0)


def test_unmodified_oracle_passes_the_pins():
    assert _pins_hold()


@pytest.mark.parametrize("mistake", ["no_bias", "bias_untransposed", "scale", "index", "mask",
                                     "se_sign", "gain_on_bias"])
def test_planted_mistake_is_caught(monkeypatch, mistake):
    monkeypatch.setattr(O, "_scores", _scores_variant(mistake))
    assert not _pins_hold(), f"planted mistake '{mistake}' passed the pins"


def _pool_variant(mistake):
    def fwd_bwd(x, g, dy):
        B, N, C = x.shape
        cnt = torch.arange(1, N + 1, dtype=f64).view(1, N, 1)
        if mistake == "counts":
            cnt = cnt + 1
        cs = x.double().cumsum(1)
        if mistake == "exclusive":
            cs = cs - x.double()
        s = torch.sigmoid(g.double())
        pool = cs / cnt
        out = s * pool
        dg = dy * pool * s * (1 - s)
        term = dy * s / cnt
        dx = term.cumsum(1) if mistake == "prefix_dx" else term.flip(1).cumsum(1).flip(1)
        return out, dx, dg
    return fwd_bwd


@pytest.mark.parametrize("mistake", [None, "counts", "exclusive", "prefix_dx"])
def test_pool_pins_catch_planted_mistakes(mistake):
    g = torch.Generator().manual_seed(1)
    x, gp, dy = (torch.randn(1, 9, 8, generator=g, dtype=f64) for _ in range(3))
    out, dx, dg = _pool_variant(mistake)(x, gp, dy)
    ex_dx, ex_dg = pool_gate_explicit_backward(x, gp, dy)
    holds = (torch.allclose(out, pool_gate_brute_force(x, gp), atol=1e-12, rtol=0)
             and torch.allclose(dx, ex_dx, atol=1e-12, rtol=0)
             and torch.allclose(dg, ex_dg, atol=1e-12, rtol=0))
    assert holds == (mistake is None)
