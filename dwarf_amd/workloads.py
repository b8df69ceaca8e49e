"""The five benchmark/parity workloads and their seeded synthetic inputs.

Inputs are generated on the CPU from seed 1000 + config index with ``torch.Generator`` and then
moved to the device, so a CPU checker and the GPU see identical values.  pos_bias is stored in
the reference's [J,H] layout (kernels/dsqg_attention_v3.py:364), i.e. the transpose of the
``bias[h,i]`` the workload descriptions use.

  0  B1 H8 N2048 D32, fp32, 44 offsets, forward.  bias[h,i] = -linspace(0,2,44)[i]*(h+1)/8.
  1  B8 H8 N2048 D32, bf16, fwd+bwd, bias as 0, dO ~ N(0,1).
  2  B8 H12 N2048 D64, bf16, fwd+bwd, q,k,v ~ N(0,1)/8, bias ~ U(-3,0), dO ~ N(0,1).  Headline.
  3  B4 H8 N4096 D64, bf16, fwd+bwd, 46 offsets, score gain g[h,j] ~ U(0.5,1.5), IF gain
     a[h] ~ U(0.8,1.2), bias as 0 with linspace(0,2,46).
  4  decode: B256 H12 D64, bf16, 44 offsets, rings of 1537 slots, start positions ~ U[1536,8191].

Not a numbered config: ``TRAINER_D96``, the attention call of the 85M condU trainer
(train/train_2048_85m_condU.py:54,60-62: batch 8, d_model 768 over 8 heads, i.e. D = 96, N 2048,
44 offsets), inputs as config 2 with q,k,v ~ N(0,1)/sqrt(96); bench.py's D = 96 leg.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import torch

from .offsets import OFFSETS_J46, OFFSETS_V3


@dataclass(frozen=True)
class Workload:
    index: int
    B: int
    H: int
    N: int
    D: int
    dtype: torch.dtype
    offsets: tuple
    backward: bool
    description: str

    @property
    def J(self) -> int:
        return len(self.offsets)

    @property
    def seed(self) -> int:
        return 1000 + self.index

    def fwd_bytes(self) -> int:
        """Compulsory forward traffic: read q,k,v, write out (+ 4-byte lse per row)."""
        T = self.B * self.H * self.N
        E = torch.finfo(self.dtype).bits // 8
        return 4 * T * self.D * E + 4 * T

    def bwd_bytes(self) -> int:
        """Compulsory backward traffic: read q,k,v,out,dO, write dq,dk,dv (+ lse read)."""
        T = self.B * self.H * self.N
        E = torch.finfo(self.dtype).bits // 8
        return 8 * T * self.D * E + 4 * T


WORKLOADS = {
    0: Workload(0, 1, 8, 2048, 32, torch.float32, OFFSETS_V3, False, "fp32 forward, CPU-runnable"),
    1: Workload(1, 8, 8, 2048, 32, torch.bfloat16, OFFSETS_V3, True, "13M-scale fwd+bwd"),
    2: Workload(2, 8, 12, 2048, 64, torch.bfloat16, OFFSETS_V3, True, "85M-scale fwd+bwd (headline)"),
    3: Workload(3, 4, 8, 4096, 64, torch.bfloat16, OFFSETS_J46, True, "condU N=4096 with gains"),
}

TRAINER_D96 = Workload(5, 8, 8, 2048, 96, torch.bfloat16, OFFSETS_V3, True,
                       "85M condU trainer's attention (D=96)")

DECODE = dict(index=4, B=256, H=12, D=64, dtype=torch.bfloat16, offsets=OFFSETS_V3, S=1537,
              pos_lo=1536, pos_hi=8191, steps=1000)


def decode_bytes_per_step(B: int, H: int, D: int, J: int, elem: int = 2) -> int:
    """Per step: read q, k_new, v_new and (J-1) K + (J-1) V ring rows; write 2 ring rows + out."""
    return B * H * D * elem * (3 + 2 * (J - 1) + 3)


def make_inputs(w: Workload, device="cpu", seed: Optional[int] = None):
    """dict of q, k, v, dout, pos_bias, scale_embed, score_gain, if_gain (None when unused)."""
    g = torch.Generator().manual_seed(w.seed if seed is None else seed)
    shp = (w.B, w.H, w.N, w.D)
    scale = w.D ** -0.5 if w.index in (2, 5) else 1.0
    q = torch.randn(shp, generator=g) * scale
    k = torch.randn(shp, generator=g) * scale
    v = torch.randn(shp, generator=g) * scale
    dout = torch.randn(shp, generator=g)
    J, H = w.J, w.H
    if w.index in (2, 5):
        pos_bias = -3.0 * torch.rand(J, H, generator=g)
    else:
        lin = torch.linspace(0, 2, J)
        pos_bias = -(lin.view(J, 1) * (torch.arange(H, dtype=torch.float32) + 1).view(1, H) / 8)
    score_gain = if_gain = None
    if w.index == 3:
        score_gain = torch.rand(H, J, generator=g) + 0.5
        if_gain = torch.rand(H, generator=g) * 0.4 + 0.8
    out = dict(q=q, k=k, v=v, dout=dout, pos_bias=pos_bias.contiguous(), scale_embed=None,
               score_gain=score_gain, if_gain=if_gain)
    for key in ("q", "k", "v", "dout"):
        out[key] = out[key].to(w.dtype)
    return {k_: (t.to(device) if t is not None else None) for k_, t in out.items()}


def make_decode_inputs(device="cpu", B=None, H=None, D=None, S=None, seed=None):
    """Rings, one step's q/k_new/v_new and start positions for the decode workload."""
    cfg = DECODE
    B = B or cfg["B"]; H = H or cfg["H"]; D = D or cfg["D"]; S = S or cfg["S"]
    g = torch.Generator().manual_seed(1000 + cfg["index"] if seed is None else seed)
    dt = cfg["dtype"]
    k_ring = torch.randn(B, H, S, D, generator=g).to(dt)
    v_ring = torch.randn(B, H, S, D, generator=g).to(dt)
    q = torch.randn(B, H, D, generator=g).to(dt)
    k_new = torch.randn(B, H, D, generator=g).to(dt)
    v_new = torch.randn(B, H, D, generator=g).to(dt)
    pos = torch.randint(cfg["pos_lo"], cfg["pos_hi"] + 1, (B,), generator=g, dtype=torch.int64)
    J = len(cfg["offsets"])
    lin = torch.linspace(0, 2, J)
    pos_bias = -(lin.view(J, 1) * (torch.arange(H, dtype=torch.float32) + 1).view(1, H) / 8)
    res = dict(k_ring=k_ring, v_ring=v_ring, q=q, k_new=k_new, v_new=v_new, pos=pos,
               pos_bias=pos_bias.contiguous())
    return {k_: t.to(device) for k_, t in res.items()}
