"""CPU oracle for DSQG fixed-offset sparse attention -- TEST INFRASTRUCTURE ONLY.

This module restates the reference's pure-PyTorch DSQG math on the CPU so that the HIP
kernels in ``dwarf_amd`` can be checked against it.  It is the checker, never the product:
only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it, and nothing in ``dwarf_amd`` routes through it.

Functions and what they restate:

* ``OFFSETS_V3`` -- ``kernels/dsqg_attention_v3.py:47-49`` (``ALL_OFFSETS``: range(33) plus
  eleven semi-dyadic taps, 44 entries), identical to ``train/train_2048_condU.py:98-102``.
* ``OFFSETS_J46`` -- V3 plus {2048, 3072}; the 46-offset condU@4096 shape set.
* ``OFFSETS_J47`` -- ``train/train_4096_13m_condU.py:88-93`` (V3 plus {2048, 3072, 4096}).
* ``dsqg_forward`` -- ``kernels/dsqg_attention_v3.py:543-561`` (``_reference_v3``) followed
  literally: pad K/V by max(delta) rows at the front, gather index ``maxd - delta_j + n``,
  content score ``q.k / sqrt(HD)``, ``+ pos_bias.T``, ``+ q.se_j / sqrt(HD)``,
  ``masked_fill(n < delta_j, -inf)``, ``softmax`` over offsets, ``sum_j alpha_j v_j``.
  Two optional terms extend it:

  - ``score_gain[H, J]`` multiplies the content term: ``s_j = g[h,j] * q.k_j / sqrt(HD) + ...``
    (no reference kernel has it; closest form ``verification/src/coherent_scale_retrieval.rs:46-56``).
  - ``if_gain[H]`` multiplies the output per head, as ``train/train_2048_condU.py:187`` does
    after the kernel call.

  Without ``scale_embed`` it is ``_reference`` of ``kernels/dsqg_attention_v2.py:484-498``.
* ``dsqg_forward_backward`` -- backward of the above through torch autograd, the way the
  reference's ``run_tests`` obtains its gradients (``kernels/dsqg_attention_v3.py:593-605``).
* ``decode_step`` -- one ring-buffer decode step.  The reference has no decode kernel; its
  semantics are the circular buffer of ``README.md:175-177``: write (k_t, v_t) at slot
  ``p mod S``, attend slot ``(p - delta_j) mod S`` for every tap, tap masked when p - delta_j < 0.

Pinning (see tests/test_oracle.py): float64 brute-force loops on tiny shapes, a second
restatement in the shifted-concatenate form of ``train/train_2048_condM_layer_ablation.py:96-136``,
``torch.autograd.gradcheck`` in float64, explicit closed-form gradients, and the special cases
(row 0 equals v[0], constant v, mean of valid taps at q=0/b=0, one-hot bias, softmax shift
invariance, sum_j dbias = 0, causality).
"""

from __future__ import annotations

import math
from typing import Sequence

import torch
import torch.nn.functional as F

_SPARSE_V3 = [48, 64, 96, 128, 192, 256, 384, 512, 768, 1024, 1536]
OFFSETS_V3 = list(range(33)) + _SPARSE_V3
OFFSETS_J46 = OFFSETS_V3 + [2048, 3072]
OFFSETS_J47 = OFFSETS_V3 + [2048, 3072, 4096]
assert len(OFFSETS_V3) == 44 and len(OFFSETS_J46) == 46 and len(OFFSETS_J47) == 47


def _scores(q, k, pos_bias, scale_embed, offsets, score_gain):
    """Masked scores [B,H,N,J] and gathered index; kernels/dsqg_attention_v3.py:545-558."""
    B, H, N, HD = q.shape
    sc = HD ** -0.5
    off = torch.tensor(list(offsets), dtype=torch.long)
    maxd = int(off.max())
    kp = F.pad(k, (0, 0, maxd, 0))
    ni = torch.arange(N)
    gi = maxd - off[None, :] + ni[:, None]
    Ka = kp[:, :, gi, :]
    s = (q.unsqueeze(3) * Ka).sum(-1) * sc
    if score_gain is not None:
        s = s * score_gain[None, :, None, :]
    s = s + pos_bias.T[None, :, None, :]
    if scale_embed is not None:
        s = s + (q.unsqueeze(3) * scale_embed[None, None, :, :]).sum(-1) * sc
    mask = (ni[:, None] < off[None, :]).unsqueeze(0).unsqueeze(0)
    s = s.masked_fill(mask, float("-inf"))
    return s, gi, maxd


def dsqg_forward(q, k, v, pos_bias, scale_embed=None, offsets: Sequence[int] = OFFSETS_V3,
                 score_gain=None, if_gain=None, return_lse: bool = False):
    """DSQG forward in the dtype of ``q`` (float32 or float64).

    Inputs are [B,H,N,HD]; pos_bias [J,H]; scale_embed [J,HD]; score_gain [H,J]; if_gain [H].
    Returns out [B,H,N,HD] (and lse [B,H,N] = logsumexp of the masked scores).
    Restates kernels/dsqg_attention_v3.py:543-561 with the two optional gains.
    """
    s, gi, maxd = _scores(q, k, pos_bias, scale_embed, offsets, score_gain)
    vp = F.pad(v, (0, 0, maxd, 0))
    Va = vp[:, :, gi, :]
    a = F.softmax(s, dim=-1)
    out = (a.unsqueeze(-1) * Va).sum(3)
    if if_gain is not None:
        out = out * if_gain.view(1, -1, 1, 1)
    if return_lse:
        return out, torch.logsumexp(s, dim=-1)
    return out


def dsqg_weights(q, k, pos_bias, scale_embed=None, offsets=OFFSETS_V3, score_gain=None):
    """Softmax weights alpha [B,H,N,J] (cf. tools/visualize_attention.py:198-254)."""
    s, _, _ = _scores(q, k, pos_bias, scale_embed, offsets, score_gain)
    return F.softmax(s, dim=-1)


def dsqg_forward_backward(q, k, v, pos_bias, dout, scale_embed=None, offsets=OFFSETS_V3,
                          score_gain=None, if_gain=None, dtype=torch.float32):
    """Forward + autograd backward in ``dtype``.

    Returns a dict with out, lse, dq, dk, dv, dpos_bias and, when the optional tensors are
    given, dscale_embed, dscore_gain, dif_gain.  All inputs are first converted to ``dtype``
    (so bf16-rounded inputs are compared in fp32, the reference's own convention:
    kernels/dsqg_attention_v3.py:548-553 does ``k.float()``).
    """
    def leaf(t):
        return None if t is None else t.detach().to(dtype).clone().requires_grad_(True)

    ql, kl, vl, pbl = leaf(q), leaf(k), leaf(v), leaf(pos_bias)
    sel, gl, al = leaf(scale_embed), leaf(score_gain), leaf(if_gain)
    out, lse = dsqg_forward(ql, kl, vl, pbl, sel, offsets, gl, al, return_lse=True)
    out.backward(dout.detach().to(dtype))
    res = {"out": out.detach(), "lse": lse.detach(), "dq": ql.grad, "dk": kl.grad,
           "dv": vl.grad, "dpos_bias": pbl.grad}
    if sel is not None:
        res["dscale_embed"] = sel.grad
    if gl is not None:
        res["dscore_gain"] = gl.grad
    if al is not None:
        res["dif_gain"] = al.grad
    return res


def decode_step(q, k_new, v_new, k_ring, v_ring, pos, pos_bias, scale_embed=None,
                offsets=OFFSETS_V3, score_gain=None, if_gain=None):
    """One ring-buffer decode step (README.md:175-177 semantics), computed in q's dtype.

    q, k_new, v_new: [B,H,D]; k_ring, v_ring: [B,H,S,D] (modified in place: slot pos mod S
    receives k_new / v_new); pos: [B] int64, the absolute position of the new token.
    Tap j reads slot (pos - delta_j) mod S, or k_new/v_new for delta_j = 0, and is masked when
    pos - delta_j < 0.  Returns out [B,H,D].
    """
    B, H, S, D = k_ring.shape
    off = torch.tensor(list(offsets), dtype=torch.long)
    assert S > int(off.max()), "ring must hold max(delta)+1 slots"
    sc = D ** -0.5
    slot_new = pos % S
    k_ring[torch.arange(B), :, slot_new, :] = k_new.to(k_ring.dtype)
    v_ring[torch.arange(B), :, slot_new, :] = v_new.to(v_ring.dtype)
    p = pos.view(B, 1) - off.view(1, -1)                      # [B,J]
    slots = torch.remainder(p, S)
    bidx = torch.arange(B).view(B, 1).expand_as(slots)
    masked = (p < 0).view(B, 1, -1, 1)                         # taps before position 0
    # A masked tap is never read: its gathered row is zero, as F.pad makes it in the forward.
    Kg = k_ring[bidx, :, slots, :].permute(0, 2, 1, 3).to(q.dtype).masked_fill(masked, 0.0)
    Vg = v_ring[bidx, :, slots, :].permute(0, 2, 1, 3).to(q.dtype).masked_fill(masked, 0.0)
    s = (q.unsqueeze(2) * Kg).sum(-1) * sc                    # [B,H,J]
    if score_gain is not None:
        s = s * score_gain[None].to(q.dtype)
    s = s + pos_bias.T[None].to(q.dtype)
    if scale_embed is not None:
        s = s + (q.unsqueeze(2) * scale_embed[None, None].to(q.dtype)).sum(-1) * sc
    s = s.masked_fill((p < 0).unsqueeze(1), float("-inf"))
    a = F.softmax(s, dim=-1)
    out = (a.unsqueeze(-1) * Vg).sum(2)
    if if_gain is not None:
        out = out * if_gain.view(1, -1, 1).to(q.dtype)
    return out


def brute_force_forward(q, k, v, pos_bias, scale_embed=None, offsets=OFFSETS_V3,
                        score_gain=None, if_gain=None):
    """Pure-Python loop form in float64, for tiny shapes only (independent of _scores)."""
    B, H, N, HD = q.shape
    out = torch.zeros(B, H, N, HD, dtype=torch.float64)
    lse = torch.zeros(B, H, N, dtype=torch.float64)
    c = 1.0 / math.sqrt(HD)
    qd, kd, vd = q.double(), k.double(), v.double()
    for b in range(B):
        for h in range(H):
            for n in range(N):
                sv, rows = [], []
                for j, dlt in enumerate(offsets):
                    m = n - dlt
                    if m < 0:
                        continue
                    g = 1.0 if score_gain is None else float(score_gain[h, j])
                    val = g * c * float(qd[b, h, n] @ kd[b, h, m]) + float(pos_bias[j, h])
                    if scale_embed is not None:
                        val += c * float(qd[b, h, n] @ scale_embed[j].double())
                    sv.append(val)
                    rows.append(m)
                mx = max(sv)
                w = [math.exp(x - mx) for x in sv]
                z = sum(w)
                acc = torch.zeros(HD, dtype=torch.float64)
                for wi, m in zip(w, rows):
                    acc += (wi / z) * vd[b, h, m]
                a = 1.0 if if_gain is None else float(if_gain[h])
                out[b, h, n] = a * acc
                lse[b, h, n] = mx + math.log(z)
    return out, lse


def explicit_backward(q, k, v, pos_bias, dout, scale_embed=None, offsets=OFFSETS_V3,
                      score_gain=None, if_gain=None):
    """Hand-derived DSQG gradients in float64, written without autograd.

    With c = 1/sqrt(HD), u_j = dO.v_j, D = sum_j alpha_j u_j (dO = a_h * dOut):
      dS_j = alpha_j (u_j - D);  dq = c sum_j dS_j (g_j k_j + se_j);
      dk[n-d_j] += c g_j dS_j q[n];  dv[n-d_j] += alpha_j dO[n];  dbias[j,h] = sum dS_j;
      dse_j = c sum dS_j q;  dg[h,j] = c sum dS_j q.k_j;  da_h = sum dOut.o.
    Used to pin the autograd path (a dropped term or wrong index fails the comparison).
    """
    B, H, N, HD = q.shape
    J = len(offsets)
    c = 1.0 / math.sqrt(HD)
    qd, kd, vd, dod = q.double(), k.double(), v.double(), dout.double()
    pb = pos_bias.double()
    se = None if scale_embed is None else scale_embed.double()
    g = None if score_gain is None else score_gain.double()
    a = None if if_gain is None else if_gain.double()
    dq = torch.zeros_like(qd); dk = torch.zeros_like(kd); dv = torch.zeros_like(vd)
    dpb = torch.zeros(J, H, dtype=torch.float64)
    dse = torch.zeros(J, HD, dtype=torch.float64)
    dg = torch.zeros(H, J, dtype=torch.float64)
    da = torch.zeros(H, dtype=torch.float64)
    n_idx = torch.arange(N)
    for h in range(H):
        gh = torch.ones(J, dtype=torch.float64) if g is None else g[h]
        ah = 1.0 if a is None else float(a[h])
        for b in range(B):
            s = torch.full((N, J), float("-inf"), dtype=torch.float64)
            qk = torch.zeros(N, J, dtype=torch.float64)
            u = torch.zeros(N, J, dtype=torch.float64)
            for j, dlt in enumerate(offsets):
                valid = n_idx >= dlt
                m = (n_idx - dlt)[valid]
                qk[valid, j] = (qd[b, h, valid] * kd[b, h, m]).sum(-1)
                val = gh[j] * c * qk[valid, j] + pb[j, h]
                if se is not None:
                    val = val + c * (qd[b, h, valid] @ se[j])
                s[valid, j] = val
                u[valid, j] = (dod[b, h, valid] * vd[b, h, m]).sum(-1)
            alpha = torch.softmax(s, dim=-1)
            Dp = (alpha * u).sum(-1, keepdim=True)          # dOut . o  (pre-gain o)
            da[h] += Dp.sum()
            dS = ah * alpha * (u - Dp)
            dpb[:, h] += dS.sum(0)
            dg[h] += c * (dS * qk).sum(0)
            for j, dlt in enumerate(offsets):
                valid = n_idx >= dlt
                m = (n_idx - dlt)[valid]
                kk = gh[j] * kd[b, h, m]
                if se is not None:
                    kk = kk + se[j]
                dq[b, h, valid] += c * dS[valid, j, None] * kk
                dk[b, h, m] += c * gh[j] * dS[valid, j, None] * qd[b, h, valid]
                dv[b, h, m] += ah * alpha[valid, j, None] * dod[b, h, valid]
                dse[j] += c * (dS[valid, j, None] * qd[b, h, valid]).sum(0)
    res = {"dq": dq, "dk": dk, "dv": dv, "dpos_bias": dpb, "dscale_embed": dse}
    if g is not None:
        res["dscore_gain"] = dg
    if a is not None:
        res["dif_gain"] = da
    return res
