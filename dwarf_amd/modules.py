"""Drop-in attention modules: the reference's parameter names, shapes and initialisation, with
the DSQG core on the HIP kernels.

State dicts saved from the reference modules load unchanged (``load_state_dict(strict=True)``):

* ``DSQGAttentionV3``      -- kernels/dsqg_attention_v3.py:463-536 (pos_bias, scale_embed)
* ``DSQGAttentionQW``      -- train/train_2048_condU.py:116-205 (adds if_gain) and, with the
  47-offset table, train/train_4096_13m_condU.py:110-175
* ``DSQGAttentionN_Fused`` -- kernels/dsqg_attention_v2.py:434-471 (pos_bias only, gate bias 2)
* ``DSQGBlock`` / ``FFN``  -- train/train_2048_condU.py:243-297 (pre-norm block around
  DSQGAttentionQW; with ``interference=True`` the causal-mean pool feeds the K/V injection,
  the pool and its gate on the HIP scan kernels)

Forward semantics follow the reference modules: qkv projection, optional Huygens K/V injection
(``kv_inject=(k_delta, v_delta)`` added to K and V only), DSQG attention, per-head IF gain
(QW), ``out_proj(out * sigmoid(gate_proj(x)))`` and dropout.

Incremental decoding (no counterpart in the reference, whose generate() re-runs the whole prefix,
train/train_2048_condU.py:463-487): ``cache = m.new_cache(B)``, ``y = m.prefill(x, cache)``
(the forward on a prompt, which also loads the layer's K/V ring) and ``y_t = m.step(x_t,
cache)`` for each new token, one ring-buffer decode step per layer (README.md:175-179).  Differences that change no
result beyond rounding:

* q, k, v go to the kernels as strided [B,H,N,HD] views of the projection output [B,N,3D]
  (the kernels take row strides), so the three ``permute(...).contiguous()`` copies of the
  reference are gone; without K/V injection the gradient of the projection output comes back
  as one tensor, and the output's head merge is a view (token-major storage);
* the IF gain is applied inside the forward kernel (fp32, before the bf16 rounding of the
  output) and its gradient comes from the backward kernel.
"""

from __future__ import annotations

import math
from typing import Optional, Sequence, Tuple

import torch
import torch.nn.functional as F
from torch import Tensor, nn

from . import ops
from .api import DSQGRingCache, causal_mean_pool_gate, dsqg_attention_qkv
from .offsets import OFFSETS_V3, validate


def _log_linear_bias(offsets: Sequence[int], num_heads: int) -> Tensor:
    """pos_bias[j,h] = -log(1 + delta_j) * linspace(0.2, 2.0, H)[h] (the reference's init)."""
    alphas = torch.linspace(0.2, 2.0, num_heads)
    delta_vals = torch.tensor([math.log(1.0 + d) for d in offsets], dtype=torch.float32)
    return -delta_vals.unsqueeze(1) * alphas.unsqueeze(0)


def _heads(qkv: Tensor, B: int, N: int, H: int, HD: int) -> Tuple[Tensor, Tensor, Tensor]:
    """q, k, v as [B,H,N,HD] views of qkv [B,N,3*H*HD] (row stride 3*H*HD, no copy)."""
    q, k, v = qkv.split(H * HD, dim=-1)
    return tuple(t.view(B, N, H, HD).permute(0, 2, 1, 3) for t in (q, k, v))


class _DSQGBase(nn.Module):
    def __init__(self, embedding_dim: int, num_heads: int, offsets: Sequence[int],
                 dropout: float, gate_bias: float):
        super().__init__()
        assert embedding_dim % num_heads == 0, "embedding_dim must be a multiple of num_heads"
        self.embedding_dim = embedding_dim
        self.num_heads = num_heads
        self.head_dim = embedding_dim // num_heads
        self._offsets = list(offsets)
        self.qkv_proj = nn.Linear(embedding_dim, 3 * embedding_dim, bias=True)
        self.out_proj = nn.Linear(embedding_dim, embedding_dim, bias=True)
        self.gate_proj = nn.Linear(embedding_dim, embedding_dim, bias=True)
        nn.init.constant_(self.gate_proj.bias, gate_bias)
        self.pos_bias = nn.Parameter(_log_linear_bias(self._offsets, num_heads))
        self.dropout = nn.Dropout(dropout)

    def _attend(self, x: Tensor, kv_inject, scale_embed: Optional[Tensor],
                if_gain: Optional[Tensor], cache: Optional[DSQGRingCache] = None) -> Tensor:
        B, N, D = x.shape
        H, HD = self.num_heads, self.head_dim
        qkv = self.qkv_proj(x)
        out = dsqg_attention_qkv(qkv, H, self.pos_bias, scale_embed, offsets=self._offsets,
                                 if_gain=if_gain, kv_inject=kv_inject)
        if cache is not None:
            with torch.no_grad():
                k, v = ops.split_qkv(qkv, H)[1:]
                if kv_inject is not None:
                    k, v = k + kv_inject[0], v + kv_inject[1]
                cache.prefill(k, v)
        out_flat = out.permute(0, 2, 1, 3).reshape(B, N, D)
        gate = torch.sigmoid(self.gate_proj(x))
        return self.dropout(self.out_proj(out_flat * gate))

    @torch.no_grad()
    def _step(self, x_t: Tensor, cache: DSQGRingCache, kv_inject, scale_embed: Optional[Tensor],
              if_gain: Optional[Tensor]) -> Tensor:  # generation: no autograd graph
        B, D = x_t.shape
        H, HD = self.num_heads, self.head_dim
        q, k, v = self.qkv_proj(x_t).view(B, 3, H, HD).unbind(1)
        if kv_inject is not None:
            k_delta, v_delta = kv_inject
            k, v = k + k_delta, v + v_delta
        out = cache.step(q, k, v, self.pos_bias, scale_embed, None, if_gain)
        gate = torch.sigmoid(self.gate_proj(x_t))
        return self.dropout(self.out_proj(out.reshape(B, D) * gate))

    def new_cache(self, batch: int, device=None, dtype=None) -> DSQGRingCache:
        """This layer's K/V ring cache (max offset + 1 slots), in the weights' dtype / device."""
        w = self.qkv_proj.weight
        return DSQGRingCache(batch, self.num_heads, self.head_dim, self._offsets,
                             dtype=dtype or w.dtype, device=device or w.device)

    def _summary(self) -> dict:
        with torch.no_grad():
            pb = self.pos_bias.detach().cpu()
        return {"pos_bias_abs_mean": pb.abs().mean().item(),
                "pos_bias_abs_max": pb.abs().max().item(),
                "pos_bias_mean_per_head": pb.mean(0).tolist()}


class DSQGAttentionV3(_DSQGBase):
    """kernels/dsqg_attention_v3.py:463-536: pos_bias [J,H], scale_embed [J,HD] (zero init),
    gate bias 0; registers the offset table as the buffer ``offsets``."""

    def __init__(self, embedding_dim: int, num_heads: int, seq_len: int = 2048,
                 offsets: Optional[Sequence[int]] = None, dropout: float = 0.1):
        offs = validate(offsets) if offsets is not None else list(OFFSETS_V3)
        super().__init__(embedding_dim, num_heads, offs, dropout, gate_bias=0.0)
        self.register_buffer("offsets", torch.tensor(offs, dtype=torch.long))
        self.n_offsets = len(offs)
        self.scale_embed = nn.Parameter(torch.zeros(len(offs), self.head_dim))

    def forward(self, x: Tensor, kv_inject=None) -> Tensor:
        return self._attend(x, kv_inject, self.scale_embed, None)

    def prefill(self, x: Tensor, cache: DSQGRingCache, kv_inject=None) -> Tensor:
        """forward(x) on a prompt [B,N,E]; loads the prompt's K/V rows into ``cache``."""
        return self._attend(x, kv_inject, self.scale_embed, None, cache)

    def step(self, x_t: Tensor, cache: DSQGRingCache, kv_inject=None) -> Tensor:
        """Output [B,E] for one new token x_t [B,E] at the cache's position (advances it)."""
        return self._step(x_t, cache, kv_inject, self.scale_embed, None)

    def attn_summary(self) -> dict:
        s = self._summary()
        with torch.no_grad():
            se = self.scale_embed.detach().cpu()
        s.update(scale_embed_abs_mean=se.abs().mean().item(), scale_embed_abs_max=se.abs().max().item())
        return s


class DSQGAttentionQW(_DSQGBase):
    """train/train_2048_condU.py:116-205: pos_bias [J,H], scale_embed [J,HD] (zero init),
    if_gain [H] (one init), gate bias 0.  ``offsets`` defaults to the 44-offset table; the
    47-offset table gives the N=4096 trainer's module (train/train_4096_13m_condU.py:110)."""

    def __init__(self, embedding_dim: int, num_heads: int, seq_len: int = 2048,
                 dropout: float = 0.1, offsets: Optional[Sequence[int]] = None):
        offs = validate(offsets) if offsets is not None else list(OFFSETS_V3)
        super().__init__(embedding_dim, num_heads, offs, dropout, gate_bias=0.0)
        self.scale_embed = nn.Parameter(torch.zeros(len(offs), self.head_dim))
        self.if_gain = nn.Parameter(torch.ones(num_heads))

    def forward(self, x: Tensor, kv_inject=None) -> Tensor:
        return self._attend(x, kv_inject, self.scale_embed, self.if_gain)

    def prefill(self, x: Tensor, cache: DSQGRingCache, kv_inject=None) -> Tensor:
        """forward(x) on a prompt [B,N,E]; loads the prompt's K/V rows into ``cache``."""
        return self._attend(x, kv_inject, self.scale_embed, self.if_gain, cache)

    def step(self, x_t: Tensor, cache: DSQGRingCache, kv_inject=None) -> Tensor:
        """Output [B,E] for one new token x_t [B,E] at the cache's position (advances it)."""
        return self._step(x_t, cache, kv_inject, self.scale_embed, self.if_gain)

    def attn_summary(self) -> dict:
        s = self._summary()
        with torch.no_grad():
            se = self.scale_embed.detach().cpu()
            gain = self.if_gain.detach().cpu()
        s.update(scale_embed_abs_mean=se.abs().mean().item(), scale_embed_abs_max=se.abs().max().item(),
                 if_gain=gain.tolist())
        return s


class DSQGAttentionN_Fused(_DSQGBase):
    """kernels/dsqg_attention_v2.py:434-471: pos_bias [J,H] only, gate bias 2; registers the
    offset table as the buffer ``offsets``."""

    def __init__(self, embedding_dim: int, num_heads: int, seq_len: int = 2048,
                 offsets: Optional[Sequence[int]] = None, dropout: float = 0.1):
        offs = validate(offsets) if offsets is not None else list(OFFSETS_V3)
        super().__init__(embedding_dim, num_heads, offs, dropout, gate_bias=2.0)
        self.register_buffer("offsets", torch.tensor(offs, dtype=torch.long))
        self.n_offsets = len(offs)

    def forward(self, x: Tensor) -> Tensor:
        return self._attend(x, None, None, None)

    def prefill(self, x: Tensor, cache: DSQGRingCache) -> Tensor:
        """forward(x) on a prompt [B,N,E]; loads the prompt's K/V rows into ``cache``."""
        return self._attend(x, None, None, None, cache)

    def step(self, x_t: Tensor, cache: DSQGRingCache) -> Tensor:
        """Output [B,E] for one new token x_t [B,E] at the cache's position (advances it)."""
        return self._step(x_t, cache, None, None, None)

    def attn_summary(self) -> dict:
        return self._summary()


class FFN(nn.Module):
    """train/train_2048_condU.py:243-251: fc2(dropout(gelu(fc1(x))))."""

    def __init__(self, embedding_dim: int, ffn_dim: int, dropout: float = 0.1):
        super().__init__()
        self.fc1 = nn.Linear(embedding_dim, ffn_dim)
        self.fc2 = nn.Linear(ffn_dim, embedding_dim)
        self.drop = nn.Dropout(dropout)

    def forward(self, x: Tensor) -> Tensor:
        return self.fc2(self.drop(F.gelu(self.fc1(x))))


class DSQGBlockCache:
    """Decode state of one DSQGBlock: the attention's K/V ring and, with interference, the
    running fp32 sum of the interference-normed inputs (the causal-mean pool's numerator)."""

    def __init__(self, ring: DSQGRingCache, pool_sum: Optional[Tensor]):
        self.ring = ring
        self.pool_sum = pool_sum


class DSQGBlock(nn.Module):
    """train/train_2048_condU.py:260-297: ``x + attn(norm1(x), kv_inject)`` then
    ``x + ffn(norm2(x))``.  With ``interference=True`` the K/V injection is
    ``inter_k_proj(inter)`` / ``inter_v_proj(inter)`` of
    ``inter = sigmoid(inter_gate(xi)) * cumsum(xi) / counts``, ``xi = inter_norm(x)``, the pool
    and gate fused in one HIP scan (``causal_mean_pool_gate``).  Parameter names and shapes are
    the reference's, so its state dicts load with ``strict=True``; ``offsets`` selects the
    attention's table (44 by default).  ``use_checkpoint`` is accepted and, as in the
    reference's condU block, unused."""

    def __init__(self, embedding_dim: int, num_heads: int, ffn_dim: int, seq_len: int = 2048,
                 dropout: float = 0.1, use_checkpoint: bool = False, interference: bool = False,
                 offsets: Optional[Sequence[int]] = None):
        super().__init__()
        self.interference = interference
        self.num_heads = num_heads
        self.head_dim = embedding_dim // num_heads
        self.norm1 = nn.LayerNorm(embedding_dim)
        self.norm2 = nn.LayerNorm(embedding_dim)
        self.attn = DSQGAttentionQW(embedding_dim, num_heads, seq_len=seq_len, dropout=dropout,
                                    offsets=offsets)
        self.ffn = FFN(embedding_dim, ffn_dim, dropout)
        if interference:
            self.inter_norm = nn.LayerNorm(embedding_dim)
            self.inter_gate = nn.Linear(embedding_dim, embedding_dim)
            self.inter_k_proj = nn.Linear(embedding_dim, embedding_dim)
            self.inter_v_proj = nn.Linear(embedding_dim, embedding_dim)

    def _inject(self, inter: Tensor):
        """K/V deltas [B,H,N,HD] (views; the kernels take strides) from inter [B,N,E]."""
        B, N, _ = inter.shape
        H, HD = self.num_heads, self.head_dim
        k_delta = self.inter_k_proj(inter).view(B, N, H, HD).permute(0, 2, 1, 3)
        v_delta = self.inter_v_proj(inter).view(B, N, H, HD).permute(0, 2, 1, 3)
        return k_delta, v_delta

    def _forward(self, x: Tensor, cache: Optional[DSQGBlockCache]) -> Tensor:
        kv_inject = None
        if self.interference:
            xi = self.inter_norm(x)
            kv_inject = self._inject(causal_mean_pool_gate(xi, self.inter_gate(xi)))
            if cache is not None:
                cache.pool_sum = xi.detach().float().sum(dim=1)
        a = self.attn.prefill(self.norm1(x), cache.ring, kv_inject) if cache is not None \
            else self.attn(self.norm1(x), kv_inject=kv_inject)
        x = x + a
        return x + self.ffn(self.norm2(x))

    def forward(self, x: Tensor) -> Tensor:
        return self._forward(x, None)

    def new_cache(self, batch: int, device=None, dtype=None) -> DSQGBlockCache:
        return DSQGBlockCache(self.attn.new_cache(batch, device, dtype), None)

    def prefill(self, x: Tensor, cache: DSQGBlockCache) -> Tensor:
        """forward(x) on a prompt [B,N,E]; loads the K/V ring and the pool's running sum."""
        return self._forward(x, cache)

    @torch.no_grad()
    def step(self, x_t: Tensor, cache: DSQGBlockCache) -> Tensor:
        """Output [B,E] for one new token x_t [B,E] at the cache's position (advances it)."""
        kv_inject = None
        if self.interference:
            B, E = x_t.shape
            xi = self.inter_norm(x_t)
            if cache.pool_sum is None:
                cache.pool_sum = torch.zeros((B, E), dtype=torch.float32, device=x_t.device)
            cache.pool_sum += xi.float()
            count = (cache.ring.pos + 1).to(torch.float32).unsqueeze(1)
            inter = torch.sigmoid(self.inter_gate(xi)) * (cache.pool_sum / count)
            k_delta, v_delta = self._inject(inter.to(xi.dtype).unsqueeze(1))
            kv_inject = (k_delta[:, :, 0], v_delta[:, :, 0])
        x_t = x_t + self.attn.step(self.norm1(x_t), cache.ring, kv_inject)
        return x_t + self.ffn(self.norm2(x_t))
