"""Public DSQG entry points with the reference's signatures and dtype rules.

* ``dsqg_attention_v3(q, k, v, pos_bias, scale_embed)`` -- kernels/dsqg_attention_v3.py:445-456.
* ``dsqg_attention_v2(q, k, v, pos_bias)`` -- kernels/dsqg_attention_v2.py:417-428 (V3 with no
  scale_embed term).
* ``dsqg_attention_backend(q, k, v, pos_bias, scale_embed)`` -- the J=47 call of
  train/train_4096_13m_condU.py:104-105 (offset table chosen from pos_bias.shape[0]).
* ``dsqg_attention(...)`` -- the general form: any offset table, optional ``score_gain[H,J]``
  multiplying the content term and ``if_gain[H]`` multiplying the output (what
  train/train_2048_condU.py:187 does after the kernel), fused into the kernels.
* ``dsqg_attention_qkv(qkv, num_heads, ...)`` -- the same on the projection output
  qkv [B,N,3*H*HD] of train/train_2048_condU.py:169-175: the heads are read in place and the
  gradient comes back as one [B,N,3*H*HD] tensor.
* ``causal_mean_pool_gate(x, gate_pre)`` -- the interference pool of a DWARF block,
  train/train_2048_condU.py:289-292: ``sigmoid(gate_pre) * x.cumsum(1) / counts``.

The output [B,H,N,HD] is stored token-major ([B,N,H,HD] memory), so the callers'
``out.permute(0, 2, 1, 3).reshape(B, N, H * HD)`` (train/train_2048_condU.py:186) is a view.

Dtype rules: bf16 in -> bf16 out with fp32 arithmetic; fp32 in -> fp32 out, computed in fp32
(the reference would downcast to bf16, kernels/dsqg_attention_v3.py:452-454); any other
float dtype (fp16 under autocast) is cast to bf16 and the result back, as the reference does.
Shape errors raise AssertionError, as the reference's asserts do (:363-365).
"""

from __future__ import annotations

from typing import Optional, Sequence

import torch
from torch import Tensor

from . import ops
from .offsets import default_offsets, validate


def _check_shapes(q, k, v, pos_bias, scale_embed, score_gain, if_gain, offsets):
    assert q.dim() == 4, f"q must be [B,H,N,HD], got {tuple(q.shape)}"
    B, H, N, HD = q.shape
    assert k.shape == q.shape and v.shape == q.shape, "q, k, v must have the same shape"
    J = len(offsets)
    assert tuple(pos_bias.shape) == (J, H), f"pos_bias must be {(J, H)}, got {tuple(pos_bias.shape)}"
    if scale_embed is not None:
        assert tuple(scale_embed.shape) == (J, HD), \
            f"scale_embed must be {(J, HD)}, got {tuple(scale_embed.shape)}"
    if score_gain is not None:
        assert tuple(score_gain.shape) == (H, J), \
            f"score_gain must be {(H, J)}, got {tuple(score_gain.shape)}"
    if if_gain is not None:
        assert tuple(if_gain.shape) == (H,), f"if_gain must be {(H,)}, got {tuple(if_gain.shape)}"


def _f32(t: Optional[Tensor]) -> Optional[Tensor]:
    return None if t is None else t.float()


def _compute_dtype(q: Tensor, k: Tensor, v: Tensor):
    """q, k, v in the dtype the kernels compute in: q's if float32 or bfloat16, else bfloat16."""
    if q.dtype not in (torch.float32, torch.bfloat16):
        return q.bfloat16(), k.bfloat16(), v.bfloat16()
    return q, k.to(q.dtype), v.to(q.dtype)


def dsqg_attention(q: Tensor, k: Tensor, v: Tensor, pos_bias: Tensor,
                   scale_embed: Optional[Tensor] = None, *,
                   offsets: Optional[Sequence[int]] = None,
                   score_gain: Optional[Tensor] = None,
                   if_gain: Optional[Tensor] = None) -> Tensor:
    """DSQG attention over a fixed offset table (default chosen by pos_bias.shape[0]).

    q, k, v [B,H,N,HD]; pos_bias [J,H]; scale_embed [J,HD]; score_gain [H,J]; if_gain [H].
    Differentiable in q, k, v and every parameter.
    """
    offs = validate(offsets) if offsets is not None else default_offsets(pos_bias.shape[0])
    _check_shapes(q, k, v, pos_bias, scale_embed, score_gain, if_gain, offs)
    orig = q.dtype
    q, k, v = _compute_dtype(q, k, v)
    args = (q, k, v, pos_bias.float(), _f32(scale_embed), _f32(score_gain), _f32(if_gain),
            list(offs))
    out = (ops.dsqg_fwd(*args) if ops.traced(q, k, v) else ops.AttentionFn.apply(*args))[0]
    return out if out.dtype == orig else out.to(orig)


def dsqg_attention_qkv(qkv: Tensor, num_heads: int, pos_bias: Tensor,
                       scale_embed: Optional[Tensor] = None, *,
                       offsets: Optional[Sequence[int]] = None,
                       score_gain: Optional[Tensor] = None,
                       if_gain: Optional[Tensor] = None,
                       kv_inject=None) -> Tensor:
    """dsqg_attention on q, k, v = the head views of qkv [B,N,3*H*HD] (the qkv_proj output).

    Same result as ``dsqg_attention(*split_qkv(qkv, num_heads), ...)``; differentiable in qkv
    and every parameter, with d(qkv) produced as one tensor.  ``kv_inject=(k_delta, v_delta)``
    ([B,H,N,HD] each) attends K + k_delta and V + v_delta (the Huygens injection of
    train/train_2048_condU.py:178-181); the deltas' gradients are the K / V slices of d(qkv).
    """
    assert qkv.dim() == 3, f"qkv must be [B,N,3*H*HD], got {tuple(qkv.shape)}"
    offs = validate(offsets) if offsets is not None else default_offsets(pos_bias.shape[0])
    q, k, v = ops.split_qkv(qkv, num_heads)
    _check_shapes(q, k, v, pos_bias, scale_embed, score_gain, if_gain, offs)
    orig = qkv.dtype
    if orig not in (torch.float32, torch.bfloat16):
        qkv = qkv.bfloat16()
    params = (pos_bias.float(), _f32(scale_embed), _f32(score_gain), _f32(if_gain), list(offs))
    if kv_inject is None:
        args = (qkv, num_heads, *params)
        out = (ops.dsqg_fwd_qkv(*args) if ops.traced(qkv) else ops.AttentionQkvFn.apply(*args))[0]
    else:
        k_delta, v_delta = kv_inject
        assert k_delta.shape == k.shape and v_delta.shape == v.shape, \
            f"kv_inject deltas must be {tuple(k.shape)}"
        args = (qkv, k_delta, v_delta, num_heads, *params)
        fn = ops.dsqg_fwd_qkv_kv if ops.traced(qkv, k_delta, v_delta) else ops.AttentionQkvKvFn.apply
        out = fn(*args)[0]
    return out if out.dtype == orig else out.to(orig)


def dsqg_attention_v3(q: Tensor, k: Tensor, v: Tensor, pos_bias: Tensor,
                      scale_embed: Tensor) -> Tensor:
    """Drop-in for kernels/dsqg_attention_v3.py:445 (44 offsets, Q-weighted scale term)."""
    return dsqg_attention(q, k, v, pos_bias, scale_embed)


def dsqg_attention_v2(q: Tensor, k: Tensor, v: Tensor, pos_bias: Tensor) -> Tensor:
    """Drop-in for kernels/dsqg_attention_v2.py:417 (44 offsets, no scale_embed)."""
    return dsqg_attention(q, k, v, pos_bias)


def dsqg_attention_backend(q: Tensor, k: Tensor, v: Tensor, pos_bias: Tensor,
                           scale_embed: Tensor) -> Tensor:
    """Drop-in for train/train_4096_13m_condU.py:104 (table by pos_bias.shape[0]: 44/46/47)."""
    return dsqg_attention(q, k, v, pos_bias, scale_embed)


def dsqg_attention_with_lse(q, k, v, pos_bias, scale_embed=None, *, offsets=None,
                            score_gain=None, if_gain=None):
    """(out, lse): out in the dtype rules above (differentiable), lse [B,H,N] fp32 (not)."""
    offs = validate(offsets) if offsets is not None else default_offsets(pos_bias.shape[0])
    _check_shapes(q, k, v, pos_bias, scale_embed, score_gain, if_gain, offs)
    orig = q.dtype
    q, k, v = _compute_dtype(q, k, v)
    args = (q, k, v, pos_bias.float(), _f32(scale_embed), _f32(score_gain), _f32(if_gain),
            list(offs))
    out, lse = (ops.dsqg_fwd(*args) if ops.traced(q, k, v) else ops.AttentionFn.apply(*args))[:2]
    return (out if out.dtype == orig else out.to(orig)), lse


def dsqg_decode_step(q: Tensor, k_new: Tensor, v_new: Tensor, k_ring: Tensor, v_ring: Tensor,
                     pos: Tensor, pos_bias: Tensor, scale_embed: Optional[Tensor] = None, *,
                     offsets: Optional[Sequence[int]] = None,
                     score_gain: Optional[Tensor] = None,
                     if_gain: Optional[Tensor] = None) -> Tensor:
    """One decode step: q/k_new/v_new [B,H,D], rings [B,H,S,D] (updated in place), pos [B]."""
    offs = validate(offsets) if offsets is not None else default_offsets(pos_bias.shape[0])

    def f32(t):
        return None if t is None else t.detach().float().contiguous()

    return ops.dsqg_decode(q.contiguous(), k_new.contiguous(), v_new.contiguous(), k_ring,
                           v_ring, pos.to(torch.int64).contiguous(), f32(pos_bias),
                           f32(scale_embed), f32(score_gain), f32(if_gain), list(offs))


def causal_mean_pool_gate(x: Tensor, gate_pre: Tensor) -> Tensor:
    """``sigmoid(gate_pre) * x.cumsum(1) / (n + 1)`` over [B,N,C] (C a multiple of 8), forward
    and backward on the HIP scan kernels: the interference pool of train/train_2048_condU.py:
    289-292 (``pool = xi.cumsum(dim=1) / counts``; ``inter = sigmoid(inter_gate(xi)) * pool``).

    x and gate_pre may be float32, bfloat16 or float16 and may differ (under autocast the
    reference has a float32 LayerNorm output and a float16 gate); the result has their promoted
    dtype, as the reference's product does, and the sigmoid is rounded to gate_pre's dtype first,
    as torch's sigmoid of that tensor is.  Sums are fp32 and deterministic.
    """
    assert x.dim() == 3, f"x must be [B,N,C], got {tuple(x.shape)}"
    assert gate_pre.shape == x.shape, (f"gate_pre must match x {tuple(x.shape)}, "
                                       f"got {tuple(gate_pre.shape)}")
    assert x.shape[2] % 8 == 0, f"channel count {x.shape[2]} must be a multiple of 8"
    if ops.traced(x, gate_pre):
        return ops.pool_gate_fwd(x, gate_pre)
    return ops.PoolGateFn.apply(x, gate_pre)


class DSQGRingCache:
    """Per-layer O(1) decode cache: K/V rings of S = max(offset)+1 slots (README.md:175-179).

    ``prefill(k, v)`` loads the last S positions of a prompt (k, v [B,H,N,D]); ``step(q, k_t,
    v_t)`` runs one decode step at the current position and advances it.
    """

    def __init__(self, B: int, H: int, D: int, offsets: Sequence[int], dtype=torch.bfloat16,
                 device="cuda", slots: Optional[int] = None):
        self.offsets = validate(offsets)
        self.S = int(slots) if slots is not None else self.offsets[-1] + 1
        assert self.S > self.offsets[-1], "ring needs at least max(offset)+1 slots"
        self.k_ring = torch.zeros((B, H, self.S, D), dtype=dtype, device=device)
        self.v_ring = torch.zeros_like(self.k_ring)
        self.pos = torch.zeros((B,), dtype=torch.int64, device=device)

    def prefill(self, k: Tensor, v: Tensor) -> None:
        """Write prompt rows m = N-S..N-1 (those that exist) to slots m mod S; pos becomes N."""
        B, H, N, D = k.shape
        lo = max(0, N - self.S)
        idx = torch.arange(lo, N, device=k.device)
        self.k_ring[:, :, idx % self.S] = k[:, :, lo:N].to(self.k_ring.dtype)
        self.v_ring[:, :, idx % self.S] = v[:, :, lo:N].to(self.v_ring.dtype)
        self.pos.fill_(N)

    def step(self, q: Tensor, k_new: Tensor, v_new: Tensor, pos_bias: Tensor,
             scale_embed: Optional[Tensor] = None, score_gain: Optional[Tensor] = None,
             if_gain: Optional[Tensor] = None) -> Tensor:
        out = dsqg_decode_step(q, k_new, v_new, self.k_ring, self.v_ring, self.pos, pos_bias,
                               scale_embed, offsets=self.offsets, score_gain=score_gain,
                               if_gain=if_gain)
        self.pos += 1
        return out
