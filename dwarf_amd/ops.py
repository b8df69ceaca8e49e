"""torch custom ops over the C ABI: ``dwarf::dsqg_fwd``, ``dwarf::dsqg_fwd_qkv``, ``dwarf::dsqg_bwd``,
``dwarf::dsqg_decode``, and the interference pool ``dwarf::pool_gate_fwd`` / ``_bwd``.

The ops take device tensors, pass raw pointers, element strides and the current HIP stream
to libdsqg_hip.so through ctypes, and allocate their outputs (and the backward workspace) with
torch's caching allocator.  ``dwarf::dsqg_fwd`` carries an autograd formula that calls
``dwarf::dsqg_bwd``, and every op has a fake (meta) implementation so graphs can be traced.

Tensors must live on a ROCm GPU: there is no CPU path, and a missing library raises.

Reference counterparts: _DSQGFnV3.forward / .backward (kernels/dsqg_attention_v3.py:359-442).
"""

from __future__ import annotations

import ctypes
import functools
from typing import List, Optional, Tuple

import torch
from torch import Tensor

from . import _lib
from .offsets import long_range_taps

_DTYPE_CODE = {torch.float32: _lib.DSQG_F32, torch.bfloat16: _lib.DSQG_BF16}


def _ptr(t: Optional[Tensor]):
    return None if t is None or t.numel() == 0 else t.data_ptr()


def _require_gpu(*ts: Optional[Tensor]) -> torch.device:
    dev = None
    for t in ts:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise RuntimeError(
                f"dwarf_amd DSQG ops need tensors on a ROCm GPU, got device {t.device}; "
                "there is no CPU implementation")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise RuntimeError(f"tensors on different devices: {dev} and {t.device}")
    return dev


def _rows_ready(t: Tensor) -> Tensor:
    """Keep t if the kernels can read it in place (unit inner stride, 16-byte aligned rows)."""
    es = t.element_size()
    ok = (t.stride(-1) == 1 and t.data_ptr() % 16 == 0
          and all(s >= 0 and (s * es) % 16 == 0 for s in t.stride()[:-1]))
    return t if ok or t.numel() == 0 else t.contiguous()


def _param(t: Optional[Tensor]) -> Optional[Tensor]:
    # fp32, contiguous and 16-byte aligned (the kernels read scale_embed as 16-byte pieces).
    if t is None or (t.dtype == torch.float32 and t.is_contiguous() and t.data_ptr() % 16 == 0):
        return t  # only its pointer is passed on; the launch keeps a reference
    return t.detach().to(torch.float32).clone(memory_format=torch.contiguous_format)


def _strides(t: Tensor):
    return (ctypes.c_int64 * 4)(*t.stride())


def _stream(dev: torch.device) -> int:
    return torch.cuda.current_stream(dev).cuda_stream


def _token_major(B: int, H: int, N: int, D: int, **kw) -> Tensor:
    """A [B,H,N,D] tensor stored token-major ([B,N,H,D] memory): ``.permute(0, 2, 1, 3)
    .reshape(B, N, H * D)`` of it is a view, so merging the heads costs no copy."""
    return torch.empty((B, N, H, D), **kw).permute(0, 2, 1, 3)


def split_qkv(qkv: Tensor, num_heads: int) -> Tuple[Tensor, Tensor, Tensor]:
    """q, k, v as [B,H,N,HD] views of a projection output qkv [B,N,3*H*HD] (no copy)."""
    B, N, E3 = qkv.shape
    assert E3 % (3 * num_heads) == 0, f"qkv last dim {E3} is not 3 * num_heads * head_dim"
    HD = E3 // (3 * num_heads)
    q, k, v = qkv.split(num_heads * HD, dim=-1)
    return tuple(t.view(B, N, num_heads, HD).permute(0, 2, 1, 3) for t in (q, k, v))


# ------------------------------------------------------------------------------------------
# Forward
# ------------------------------------------------------------------------------------------

class FwdLaunch:
    """Argument block and outputs of one forward call, reusable: ``run()`` relaunches it."""

    def __init__(self, q, k, v, pos_bias, scale_embed, score_gain, if_gain, offsets):
        dev = _require_gpu(q, k, v, pos_bias, scale_embed, score_gain, if_gain)
        self.lib = _lib.load()
        self.device = dev
        B, H, N, D = q.shape
        code = _DTYPE_CODE.get(q.dtype)
        if code is None or k.dtype != q.dtype or v.dtype != q.dtype:
            raise AssertionError(f"q/k/v must share dtype float32 or bfloat16, got "
                                 f"{q.dtype}/{k.dtype}/{v.dtype}")
        q, k, v = _rows_ready(q), _rows_ready(k), _rows_ready(v)
        pb, se, sg, ig = _param(pos_bias), _param(scale_embed), _param(score_gain), _param(if_gain)
        self.out = _token_major(B, H, N, D, dtype=q.dtype, device=dev)
        self.lse = torch.empty((B, H, N), dtype=torch.float32, device=dev)
        # bf16: the long-range taps' weights, saved for the backward (which needs them).
        self.alpha_lr = torch.empty(_alpha_shape(q.dtype, B, H, N, offsets), dtype=torch.float32,
                                    device=dev)
        self._keep = (q, k, v, pb, se, sg, ig)
        a = _lib.FwdArgs()
        a.shape = _lib.make_shape(code, B, H, N, D, offsets)
        a.q, a.q_stride = _ptr(q), _strides(q)
        a.k, a.k_stride = _ptr(k), _strides(k)
        a.v, a.v_stride = _ptr(v), _strides(v)
        a.pos_bias, a.scale_embed, a.score_gain, a.if_gain = _ptr(pb), _ptr(se), _ptr(sg), _ptr(ig)
        a.out, a.out_stride = _ptr(self.out), _strides(self.out)
        a.lse = _ptr(self.lse)
        a.alpha_lr = _ptr(self.alpha_lr)
        self.args = a

    def run(self) -> None:
        _lib.check(self.lib.dsqg_fwd(ctypes.byref(self.args), _stream(self.device)), "dsqg_fwd")


def _alpha_shape(dtype, B: int, H: int, N: int, offsets) -> tuple:
    """Shape of the forward's saved long-range weights: [B,H,NS,N] for bf16, empty for fp32."""
    ns = long_range_taps(offsets)
    return (B, H, ns, N) if dtype == torch.bfloat16 and ns > 0 else (0,)


@torch.library.custom_op("dwarf::dsqg_fwd", mutates_args=())
def dsqg_fwd(q: Tensor, k: Tensor, v: Tensor, pos_bias: Tensor,
             scale_embed: Optional[Tensor], score_gain: Optional[Tensor],
             if_gain: Optional[Tensor], offsets: List[int]) -> Tuple[Tensor, Tensor, Tensor]:
    """out [B,H,N,D] (dtype of q; token-major storage), lse [B,H,N] fp32 and (bf16) the
    long-range taps' weights alpha_lr [B,H,NS,N] fp32 for the backward (empty for fp32)."""
    launch = FwdLaunch(q, k, v, pos_bias, scale_embed, score_gain, if_gain, offsets)
    launch.run()
    return launch.out, launch.lse, launch.alpha_lr


@dsqg_fwd.register_fake
def _(q, k, v, pos_bias, scale_embed, score_gain, if_gain, offsets):
    B, H, N, D = q.shape
    return (q.new_empty((B, N, H, D)).permute(0, 2, 1, 3), q.new_empty((B, H, N), dtype=torch.float32),
            q.new_empty(_alpha_shape(q.dtype, B, H, N, offsets), dtype=torch.float32))


@torch.library.custom_op("dwarf::dsqg_fwd_qkv", mutates_args=())
def dsqg_fwd_qkv(qkv: Tensor, num_heads: int, pos_bias: Tensor, scale_embed: Optional[Tensor],
                 score_gain: Optional[Tensor], if_gain: Optional[Tensor],
                 offsets: List[int]) -> Tuple[Tensor, Tensor, Tensor]:
    """dsqg_fwd on the q, k, v head views of one projection output qkv [B,N,3*H*HD]; its
    gradient is returned as one [B,N,3*H*HD] tensor (no per-head concatenation)."""
    q, k, v = split_qkv(qkv, num_heads)
    launch = FwdLaunch(q, k, v, pos_bias, scale_embed, score_gain, if_gain, offsets)
    launch.run()
    return launch.out, launch.lse, launch.alpha_lr


@dsqg_fwd_qkv.register_fake
def _(qkv, num_heads, pos_bias, scale_embed, score_gain, if_gain, offsets):
    B, N, E3 = qkv.shape
    HD = E3 // (3 * num_heads)
    return (qkv.new_empty((B, N, num_heads, HD)).permute(0, 2, 1, 3),
            qkv.new_empty((B, num_heads, N), dtype=torch.float32),
            qkv.new_empty(_alpha_shape(qkv.dtype, B, num_heads, N, offsets), dtype=torch.float32))


# ------------------------------------------------------------------------------------------
# Backward
# ------------------------------------------------------------------------------------------

class BwdLaunch:
    """Argument block, outputs and workspace of one backward call.

    ``run()`` launches all three phases (dsqg_bwd); ``run("dq")``, ``run("dkdv")`` and
    ``run("params")`` launch one phase each (dsqg_bwd_dq / _dkdv / _params), in that order.
    """

    _ENTRY = {None: "dsqg_bwd", "dq": "dsqg_bwd_dq", "dkdv": "dsqg_bwd_dkdv",
              "params": "dsqg_bwd_params"}

    def __init__(self, q, k, v, dout, lse, pos_bias, scale_embed, score_gain, if_gain, offsets,
                 need_dse, need_dg, need_da, grads=None, alpha_lr=None):
        dev = _require_gpu(q, k, v, dout, lse, pos_bias, scale_embed, score_gain, if_gain)
        self.lib = _lib.load()
        self.device = dev
        B, H, N, D = q.shape
        J = len(offsets)
        code = _DTYPE_CODE.get(q.dtype)
        if code is None or dout.dtype != q.dtype:
            raise AssertionError(f"q and dout must share dtype float32 or bfloat16, got "
                                 f"{q.dtype}/{dout.dtype}")
        q, k, v, dout = _rows_ready(q), _rows_ready(k), _rows_ready(v), _rows_ready(dout)
        lse = lse.contiguous()
        if alpha_lr is not None:  # the forward's long-range weights (bf16), [B,H,NS,N] fp32
            alpha_lr = alpha_lr.contiguous()
        pb, se, sg, ig = _param(pos_bias), _param(scale_embed), _param(score_gain), _param(if_gain)
        if grads is None:  # else (dq, dk, dv) [B,H,N,D] views the caller allocated
            grads = tuple(torch.empty((B, H, N, D), dtype=q.dtype, device=dev) for _ in range(3))
        self.dq, self.dk, self.dv = grads
        f32 = dict(dtype=torch.float32, device=dev)
        self.dpos_bias = torch.empty((J, H), **f32)
        self.dscale_embed = torch.empty((J, D) if need_dse else (0,), **f32)
        self.dscore_gain = torch.empty((H, J) if need_dg else (0,), **f32)
        self.dif_gain = torch.empty((H,) if need_da else (0,), **f32)
        self._keep = (q, k, v, dout, lse, alpha_lr, pb, se, sg, ig)
        a = _lib.BwdArgs()
        a.shape = _lib.make_shape(code, B, H, N, D, offsets)
        a.q, a.q_stride = _ptr(q), _strides(q)
        a.k, a.k_stride = _ptr(k), _strides(k)
        a.v, a.v_stride = _ptr(v), _strides(v)
        a.dout, a.dout_stride = _ptr(dout), _strides(dout)
        a.lse = _ptr(lse)
        a.alpha_lr = _ptr(alpha_lr)
        a.pos_bias, a.scale_embed, a.score_gain, a.if_gain = _ptr(pb), _ptr(se), _ptr(sg), _ptr(ig)
        a.dq, a.dq_stride = _ptr(self.dq), _strides(self.dq)
        a.dk, a.dk_stride = _ptr(self.dk), _strides(self.dk)
        a.dv, a.dv_stride = _ptr(self.dv), _strides(self.dv)
        a.dpos_bias = _ptr(self.dpos_bias)
        a.dscale_embed = _ptr(self.dscale_embed) if need_dse else None
        a.dscore_gain = _ptr(self.dscore_gain) if need_dg else None
        a.dif_gain = _ptr(self.dif_gain) if need_da else None
        nbytes = ctypes.c_size_t(0)
        _lib.check(self.lib.dsqg_bwd_workspace_size(ctypes.byref(a), ctypes.byref(nbytes)),
                   "dsqg_bwd_workspace_size")
        self.workspace = torch.empty((max(int(nbytes.value), 1),), dtype=torch.uint8, device=dev)
        a.workspace, a.workspace_bytes = self.workspace.data_ptr(), int(nbytes.value)
        self.args = a

    def run(self, phase: Optional[str] = None) -> None:
        name = self._ENTRY[phase]
        _lib.check(getattr(self.lib, name)(ctypes.byref(self.args), _stream(self.device)), name)

    def outputs(self):
        return (self.dq, self.dk, self.dv, self.dpos_bias, self.dscale_embed, self.dscore_gain,
                self.dif_gain)


@torch.library.custom_op("dwarf::dsqg_bwd", mutates_args=())
def dsqg_bwd(q: Tensor, k: Tensor, v: Tensor, dout: Tensor, lse: Tensor, alpha_lr: Tensor,
             pos_bias: Tensor, scale_embed: Optional[Tensor], score_gain: Optional[Tensor],
             if_gain: Optional[Tensor], offsets: List[int], need_dse: bool, need_dg: bool,
             need_da: bool) -> Tuple[Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor]:
    """(dq, dk, dv, dpos_bias, dscale_embed, dscore_gain, dif_gain); unrequested ones are empty.
    lse and alpha_lr are the forward's."""
    launch = BwdLaunch(q, k, v, dout, lse, pos_bias, scale_embed, score_gain, if_gain, offsets,
                       need_dse, need_dg, need_da, alpha_lr=alpha_lr)
    launch.run()
    return launch.outputs()


@dsqg_bwd.register_fake
def _(q, k, v, dout, lse, alpha_lr, pos_bias, scale_embed, score_gain, if_gain, offsets, need_dse,
      need_dg, need_da):
    B, H, N, D = q.shape
    J = len(offsets)
    f = dict(dtype=torch.float32)
    return (q.new_empty(q.shape), q.new_empty(q.shape), q.new_empty(q.shape),
            q.new_empty((J, H), **f), q.new_empty((J, D) if need_dse else (0,), **f),
            q.new_empty((H, J) if need_dg else (0,), **f), q.new_empty((H,) if need_da else (0,), **f))


def _setup_context(ctx, inputs, output):
    q, k, v, pos_bias, scale_embed, score_gain, if_gain, offsets = inputs
    _, lse, alpha_lr = output
    ctx.save_for_backward(q, k, v, lse, alpha_lr, pos_bias, scale_embed, score_gain, if_gain)
    ctx.offsets = list(offsets)
    ctx.mark_non_differentiable(lse, alpha_lr)


def _backward(ctx, dout, _dlse, _dalpha, direct: bool = False):
    q, k, v, lse, alpha_lr, pos_bias, scale_embed, score_gain, if_gain = ctx.saved_tensors
    need = ctx.needs_input_grad
    need_dse = bool(need[4]) and scale_embed is not None
    need_dg = bool(need[5]) and score_gain is not None
    need_da = bool(need[6]) and if_gain is not None
    args = (q, k, v, dout.to(q.dtype), lse, alpha_lr, pos_bias, scale_embed, score_gain, if_gain,
            ctx.offsets, need_dse, need_dg, need_da)
    if direct:
        launch = BwdLaunch(*args[:5], *args[6:], alpha_lr=alpha_lr)
        launch.run()
        dq, dk, dv, dpb, dse, dg, da = launch.outputs()
    else:
        dq, dk, dv, dpb, dse, dg, da = dsqg_bwd(*args)
    return (dq, dk, dv, dpb.to(pos_bias.dtype),
            dse.to(scale_embed.dtype) if need_dse else None,
            dg.to(score_gain.dtype) if need_dg else None,
            da.to(if_gain.dtype) if need_da else None, None)


torch.library.register_autograd("dwarf::dsqg_fwd", _backward, setup_context=_setup_context)


def _setup_context_qkv(ctx, inputs, output):
    qkv, num_heads, pos_bias, scale_embed, score_gain, if_gain, offsets = inputs
    _, lse, alpha_lr = output
    ctx.save_for_backward(qkv, lse, alpha_lr, pos_bias, scale_embed, score_gain, if_gain)
    ctx.num_heads = num_heads
    ctx.offsets = list(offsets)
    ctx.mark_non_differentiable(lse, alpha_lr)


def _backward_qkv(ctx, dout, _dlse, _dalpha, direct: bool = False):
    qkv, lse, alpha_lr, pos_bias, scale_embed, score_gain, if_gain = ctx.saved_tensors
    need = ctx.needs_input_grad
    need_dse = bool(need[3]) and scale_embed is not None
    need_dg = bool(need[4]) and score_gain is not None
    need_da = bool(need[5]) and if_gain is not None
    args = (qkv, ctx.num_heads, dout.to(qkv.dtype), lse, alpha_lr, pos_bias, scale_embed,
            score_gain, if_gain, ctx.offsets, need_dse, need_dg, need_da)
    bwd = _bwd_qkv_impl if direct else dsqg_bwd_qkv
    dqkv, dpb, dse, dg, da = bwd(*args)
    return (dqkv, None, dpb.to(pos_bias.dtype),
            dse.to(scale_embed.dtype) if need_dse else None,
            dg.to(score_gain.dtype) if need_dg else None,
            da.to(if_gain.dtype) if need_da else None, None)


@torch.library.custom_op("dwarf::dsqg_bwd_qkv", mutates_args=())
def dsqg_bwd_qkv(qkv: Tensor, num_heads: int, dout: Tensor, lse: Tensor, alpha_lr: Tensor,
                 pos_bias: Tensor, scale_embed: Optional[Tensor], score_gain: Optional[Tensor],
                 if_gain: Optional[Tensor], offsets: List[int], need_dse: bool, need_dg: bool,
                 need_da: bool) -> Tuple[Tensor, Tensor, Tensor, Tensor, Tensor]:
    """(dqkv [B,N,3*H*HD], dpos_bias, dscale_embed, dscore_gain, dif_gain): dq, dk, dv are
    written straight into the head views of one gradient buffer."""
    return _bwd_qkv_impl(qkv, num_heads, dout, lse, alpha_lr, pos_bias, scale_embed, score_gain,
                         if_gain, offsets, need_dse, need_dg, need_da)


def _bwd_qkv_impl(qkv, num_heads, dout, lse, alpha_lr, pos_bias, scale_embed, score_gain, if_gain,
                  offsets, need_dse, need_dg, need_da, k_eff=None, v_eff=None):
    q, k, v = split_qkv(qkv, num_heads)
    if k_eff is not None:  # K/V with the injection added (dsqg_fwd_qkv_kv)
        k, v = k_eff, v_eff
    dqkv = torch.empty_like(qkv, memory_format=torch.contiguous_format)
    launch = BwdLaunch(q, k, v, dout, lse, pos_bias, scale_embed, score_gain, if_gain, offsets,
                       need_dse, need_dg, need_da, grads=split_qkv(dqkv, num_heads),
                       alpha_lr=alpha_lr)
    launch.run()
    _, _, _, dpb, dse, dg, da = launch.outputs()
    return dqkv, dpb, dse, dg, da


@dsqg_bwd_qkv.register_fake
def _(qkv, num_heads, dout, lse, alpha_lr, pos_bias, scale_embed, score_gain, if_gain, offsets,
      need_dse, need_dg, need_da):
    B, N, E3 = qkv.shape
    HD = E3 // (3 * num_heads)
    J = len(offsets)
    f = dict(dtype=torch.float32)
    return (qkv.new_empty(qkv.shape), qkv.new_empty((J, num_heads), **f),
            qkv.new_empty((J, HD) if need_dse else (0,), **f),
            qkv.new_empty((num_heads, J) if need_dg else (0,), **f),
            qkv.new_empty((num_heads,) if need_da else (0,), **f))


torch.library.register_autograd("dwarf::dsqg_fwd_qkv", _backward_qkv,
                                setup_context=_setup_context_qkv)


# K/V injection (train/train_2048_condU.py:178-181: k + k_delta, v + v_delta before the kernel):
# one add per operand in the forward, and a backward that writes dq, dk, dv once into d(qkv),
# whose K and V slices are also the gradients of k_delta and v_delta (the add passes its
# gradient to both summands), so autograd assembles nothing.

def _kv_eff(qkv: Tensor, k_delta: Tensor, v_delta: Tensor, num_heads: int):
    _, k, v = split_qkv(qkv, num_heads)
    return k + k_delta.to(k.dtype), v + v_delta.to(v.dtype)


@torch.library.custom_op("dwarf::dsqg_fwd_qkv_kv", mutates_args=())
def dsqg_fwd_qkv_kv(qkv: Tensor, k_delta: Tensor, v_delta: Tensor, num_heads: int,
                    pos_bias: Tensor, scale_embed: Optional[Tensor], score_gain: Optional[Tensor],
                    if_gain: Optional[Tensor],
                    offsets: List[int]) -> Tuple[Tensor, Tensor, Tensor, Tensor, Tensor]:
    """(out, lse, alpha_lr, k + k_delta, v + v_delta): dsqg_fwd on q = the query view of qkv
    and the injected K/V (returned for the backward)."""
    k_eff, v_eff = _kv_eff(qkv, k_delta, v_delta, num_heads)
    q = split_qkv(qkv, num_heads)[0]
    launch = FwdLaunch(q, k_eff, v_eff, pos_bias, scale_embed, score_gain, if_gain, offsets)
    launch.run()
    return launch.out, launch.lse, launch.alpha_lr, k_eff, v_eff


@dsqg_fwd_qkv_kv.register_fake
def _(qkv, k_delta, v_delta, num_heads, pos_bias, scale_embed, score_gain, if_gain, offsets):
    B, N, E3 = qkv.shape
    HD = E3 // (3 * num_heads)
    return (qkv.new_empty((B, N, num_heads, HD)).permute(0, 2, 1, 3),
            qkv.new_empty((B, num_heads, N), dtype=torch.float32),
            qkv.new_empty(_alpha_shape(qkv.dtype, B, num_heads, N, offsets), dtype=torch.float32),
            qkv.new_empty((B, num_heads, N, HD)), qkv.new_empty((B, num_heads, N, HD)))


@torch.library.custom_op("dwarf::dsqg_bwd_qkv_kv", mutates_args=())
def dsqg_bwd_qkv_kv(qkv: Tensor, k_eff: Tensor, v_eff: Tensor, num_heads: int, dout: Tensor,
                    lse: Tensor, alpha_lr: Tensor, pos_bias: Tensor, scale_embed: Optional[Tensor],
                    score_gain: Optional[Tensor], if_gain: Optional[Tensor], offsets: List[int],
                    need_dse: bool, need_dg: bool,
                    need_da: bool) -> Tuple[Tensor, Tensor, Tensor, Tensor, Tensor]:
    """dsqg_bwd_qkv with the injected K/V: (dqkv, dpos_bias, dscale_embed, dscore_gain, dif_gain)."""
    return _bwd_qkv_impl(qkv, num_heads, dout, lse, alpha_lr, pos_bias, scale_embed, score_gain,
                         if_gain, offsets, need_dse, need_dg, need_da, k_eff, v_eff)


@dsqg_bwd_qkv_kv.register_fake
def _(qkv, k_eff, v_eff, num_heads, dout, lse, alpha_lr, pos_bias, scale_embed, score_gain,
      if_gain, offsets, need_dse, need_dg, need_da):
    B, N, E3 = qkv.shape
    HD = E3 // (3 * num_heads)
    J = len(offsets)
    f = dict(dtype=torch.float32)
    return (qkv.new_empty(qkv.shape), qkv.new_empty((J, num_heads), **f),
            qkv.new_empty((J, HD) if need_dse else (0,), **f),
            qkv.new_empty((num_heads, J) if need_dg else (0,), **f),
            qkv.new_empty((num_heads,) if need_da else (0,), **f))


def _setup_context_qkv_kv(ctx, inputs, output):
    qkv, k_delta, v_delta, num_heads, pos_bias, scale_embed, score_gain, if_gain, offsets = inputs
    _, lse, alpha_lr, k_eff, v_eff = output
    ctx.save_for_backward(qkv, k_eff, v_eff, lse, alpha_lr, pos_bias, scale_embed, score_gain,
                          if_gain)
    ctx.num_heads = num_heads
    ctx.offsets = list(offsets)
    ctx.delta_dtypes = (k_delta.dtype, v_delta.dtype)
    ctx.mark_non_differentiable(lse, alpha_lr, k_eff, v_eff)


def _backward_qkv_kv(ctx, dout, _dlse, _dalpha, _dk_eff, _dv_eff, direct: bool = False):
    qkv, k_eff, v_eff, lse, alpha_lr, pos_bias, scale_embed, score_gain, if_gain = ctx.saved_tensors
    need = ctx.needs_input_grad
    need_dse = bool(need[5]) and scale_embed is not None
    need_dg = bool(need[6]) and score_gain is not None
    need_da = bool(need[7]) and if_gain is not None
    args = (qkv, k_eff, v_eff, ctx.num_heads, dout.to(qkv.dtype), lse, alpha_lr, pos_bias,
            scale_embed, score_gain, if_gain, ctx.offsets, need_dse, need_dg, need_da)
    if direct:
        dqkv, dpb, dse, dg, da = _bwd_qkv_impl(
            qkv, ctx.num_heads, dout.to(qkv.dtype), lse, alpha_lr, pos_bias, scale_embed,
            score_gain, if_gain, ctx.offsets, need_dse, need_dg, need_da, k_eff, v_eff)
    else:
        dqkv, dpb, dse, dg, da = dsqg_bwd_qkv_kv(*args)
    _, dk, dv = split_qkv(dqkv, ctx.num_heads)
    return (dqkv, dk.to(ctx.delta_dtypes[0]), dv.to(ctx.delta_dtypes[1]), None,
            dpb.to(pos_bias.dtype),
            dse.to(scale_embed.dtype) if need_dse else None,
            dg.to(score_gain.dtype) if need_dg else None,
            da.to(if_gain.dtype) if need_da else None, None)


torch.library.register_autograd("dwarf::dsqg_fwd_qkv_kv", _backward_qkv_kv,
                                setup_context=_setup_context_qkv_kv)


# Eager autograd over the same launch objects: the custom ops above are what traced code
# (torch.compile, export, fake tensors) sees; outside tracing the public functions take these
# Functions, which skip the custom-op dispatch (about 100 us of host time per forward +
# backward, measured on the MI355X host, where the kernels themselves take a few tens of us
# at small shapes).  Same kernels, same results.

def traced(*tensors) -> bool:
    """True under torch.compile / export or for fake or meta tensors: use the custom ops."""
    if torch.compiler.is_compiling():
        return True
    from torch._subclasses.fake_tensor import FakeTensor
    return any(isinstance(t, FakeTensor) or (t is not None and t.device.type == "meta")
               for t in tensors)


class AttentionFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, pos_bias, scale_embed, score_gain, if_gain, offsets):
        launch = FwdLaunch(q, k, v, pos_bias, scale_embed, score_gain, if_gain, offsets)
        launch.run()
        outs = (launch.out, launch.lse, launch.alpha_lr)
        _setup_context(ctx, (q, k, v, pos_bias, scale_embed, score_gain, if_gain, offsets), outs)
        return outs

    @staticmethod
    def backward(ctx, dout, dlse, dalpha):
        return _backward(ctx, dout, dlse, dalpha, direct=True)


class AttentionQkvFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, qkv, num_heads, pos_bias, scale_embed, score_gain, if_gain, offsets):
        q, k, v = split_qkv(qkv, num_heads)
        launch = FwdLaunch(q, k, v, pos_bias, scale_embed, score_gain, if_gain, offsets)
        launch.run()
        outs = (launch.out, launch.lse, launch.alpha_lr)
        _setup_context_qkv(ctx, (qkv, num_heads, pos_bias, scale_embed, score_gain, if_gain,
                                 offsets), outs)
        return outs

    @staticmethod
    def backward(ctx, dout, dlse, dalpha):
        return _backward_qkv(ctx, dout, dlse, dalpha, direct=True)


class AttentionQkvKvFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, qkv, k_delta, v_delta, num_heads, pos_bias, scale_embed, score_gain, if_gain,
                offsets):
        k_eff, v_eff = _kv_eff(qkv, k_delta, v_delta, num_heads)
        q = split_qkv(qkv, num_heads)[0]
        launch = FwdLaunch(q, k_eff, v_eff, pos_bias, scale_embed, score_gain, if_gain, offsets)
        launch.run()
        outs = (launch.out, launch.lse, launch.alpha_lr, k_eff, v_eff)
        _setup_context_qkv_kv(ctx, (qkv, k_delta, v_delta, num_heads, pos_bias, scale_embed,
                                    score_gain, if_gain, offsets), outs)
        return outs

    @staticmethod
    def backward(ctx, dout, dlse, dalpha, dk_eff, dv_eff):
        return _backward_qkv_kv(ctx, dout, dlse, dalpha, dk_eff, dv_eff, direct=True)


# ------------------------------------------------------------------------------------------
# Decode step
# ------------------------------------------------------------------------------------------

@torch.library.custom_op("dwarf::dsqg_decode", mutates_args=("k_ring", "v_ring"))
def dsqg_decode(q: Tensor, k_new: Tensor, v_new: Tensor, k_ring: Tensor, v_ring: Tensor,
                pos: Tensor, pos_bias: Tensor, scale_embed: Optional[Tensor],
                score_gain: Optional[Tensor], if_gain: Optional[Tensor],
                offsets: List[int]) -> Tensor:
    """One ring-buffer decode step; writes k_new/v_new into the rings, returns out [B,H,D]."""
    out = torch.empty_like(q)
    decode_step_into(q, k_new, v_new, k_ring, v_ring, pos, pos_bias, scale_embed, score_gain,
                     if_gain, offsets, out, None)
    return out


@dsqg_decode.register_fake
def _(q, k_new, v_new, k_ring, v_ring, pos, pos_bias, scale_embed, score_gain, if_gain, offsets):
    return torch.empty_like(q)


def decode_step_into(q, k_new, v_new, k_ring, v_ring, pos, pos_bias, scale_embed, score_gain,
                     if_gain, offsets, out, pos_next=None) -> None:
    """Decode step writing into a caller-provided ``out`` (and ``pos_next`` = pos + 1 if given).

    Every tensor must already be contiguous on the GPU and parameters fp32, so the call
    allocates nothing and can be captured in a HIP graph.
    """
    dev = _require_gpu(q, k_new, v_new, k_ring, v_ring, pos, pos_bias, out)
    lib = _lib.load()
    B, H, S, D = k_ring.shape
    code = _DTYPE_CODE.get(q.dtype)
    if code is None or any(t.dtype != q.dtype for t in (k_new, v_new, k_ring, v_ring, out)):
        raise AssertionError("q, k_new, v_new, rings and out must share dtype float32 or bfloat16")
    for name, t, shp in (("q", q, (B, H, D)), ("k_new", k_new, (B, H, D)),
                         ("v_new", v_new, (B, H, D)), ("v_ring", v_ring, (B, H, S, D)),
                         ("out", out, (B, H, D))):
        if tuple(t.shape) != shp or not t.is_contiguous():
            raise AssertionError(f"{name} must be a contiguous {shp} tensor, got "
                                 f"{tuple(t.shape)} (contiguous={t.is_contiguous()})")
    if not k_ring.is_contiguous():
        raise AssertionError("k_ring must be contiguous")
    if pos.dtype != torch.int64 or tuple(pos.shape) != (B,) or not pos.is_contiguous():
        raise AssertionError("pos must be a contiguous int64 [B] tensor")
    params = [pos_bias, scale_embed, score_gain, if_gain]
    for t in params:
        if t is not None and (t.dtype != torch.float32 or not t.is_contiguous()):
            raise AssertionError("pos_bias/scale_embed/score_gain/if_gain must be contiguous fp32")
    a = _lib.DecodeArgs()
    a.shape = _lib.make_shape(code, B, H, 0, D, offsets)
    a.S = S
    a.q, a.k_new, a.v_new = _ptr(q), _ptr(k_new), _ptr(v_new)
    a.k_ring, a.v_ring = _ptr(k_ring), _ptr(v_ring)
    a.pos, a.pos_next = _ptr(pos), _ptr(pos_next)
    a.pos_bias, a.scale_embed, a.score_gain, a.if_gain = (_ptr(t) for t in params)
    a.out = _ptr(out)
    _lib.check(lib.dsqg_decode_step(ctypes.byref(a), _stream(dev)), "dsqg_decode_step")


# ------------------------------------------------------------------------------------------
# Causal-mean pool with a sigmoid gate
# ------------------------------------------------------------------------------------------

_POOL_CODE = {torch.float32: _lib.DSQG_F32, torch.bfloat16: _lib.DSQG_BF16,
              torch.float16: _lib.DSQG_F16}


def _pool_ready(t: Tensor, B: int, N: int, C: int, name: str) -> Tensor:
    if tuple(t.shape) != (B, N, C):
        raise AssertionError(f"{name} must be [{B},{N},{C}], got {tuple(t.shape)}")
    if t.dtype not in _POOL_CODE:
        raise AssertionError(f"{name} must be float32, bfloat16 or float16, got {t.dtype}")
    if t.numel() and t.stride(1) < C:  # overlapping rows (e.g. expanded along N): copy
        t = t.contiguous()
    return _rows_ready(t)


def _pool_strides(t: Tensor):
    return (ctypes.c_int64 * 2)(t.stride(0), t.stride(1))


@functools.lru_cache(maxsize=256)
def _pool_workspace_bytes(B: int, N: int, C: int, backward: bool) -> int:
    n = ctypes.c_size_t(0)
    _lib.check(_lib.load().dsqg_pool_gate_workspace_size(B, N, C, int(backward), ctypes.byref(n)),
               "dsqg_pool_gate_workspace_size")
    return int(n.value)


def _pool_workspace(B, N, C, backward: bool, dev) -> Tensor:
    return torch.empty((max(_pool_workspace_bytes(B, N, C, backward), 1),), dtype=torch.uint8,
                       device=dev)


class PoolLaunch:
    """Argument block, outputs and workspace of one pool call, reusable: ``run()`` relaunches it.

    Forward when ``dout`` is None (``out``), else backward (``dx`` / ``dgate``, empty when not
    requested).  Every tensor is [B,N,C]; strided views are read in place when their rows are
    16-byte aligned.
    """

    def __init__(self, x: Tensor, gate_pre: Tensor, dout: Optional[Tensor] = None,
                 need_dx: bool = True, need_dgate: bool = True):
        dev = _require_gpu(x, gate_pre, dout)
        self.lib = _lib.load()
        self.device = dev
        B, N, C = x.shape
        x = _pool_ready(x, B, N, C, "x")
        g = _pool_ready(gate_pre, B, N, C, "gate_pre")
        self.backward = dout is not None
        self.ws = _pool_workspace(B, N, C, self.backward, dev)
        if not self.backward:
            self.out = torch.empty((B, N, C), dtype=torch.promote_types(x.dtype, g.dtype),
                                   device=dev)
            a = _lib.PoolFwdArgs()
            a.out_dtype = _POOL_CODE[self.out.dtype]
            a.out, a.out_stride = _ptr(self.out), _pool_strides(self.out)
            self._keep = (x, g)
        else:
            dy = _pool_ready(dout, B, N, C, "dout")
            self.dx = torch.empty((B, N, C) if need_dx else (0,), dtype=x.dtype, device=dev)
            self.dgate = torch.empty((B, N, C) if need_dgate else (0,), dtype=g.dtype, device=dev)
            a = _lib.PoolBwdArgs()
            a.dout_dtype = _POOL_CODE[dy.dtype]
            a.dout, a.dout_stride = _ptr(dy), _pool_strides(dy)
            if need_dx:
                a.dx, a.dx_stride = _ptr(self.dx), _pool_strides(self.dx)
            if need_dgate:
                a.dgate_pre, a.dgate_stride = _ptr(self.dgate), _pool_strides(self.dgate)
            self._keep = (x, g, dy)
        a.B, a.N, a.C = B, N, C
        a.x_dtype, a.gate_dtype = _POOL_CODE[x.dtype], _POOL_CODE[g.dtype]
        a.x, a.x_stride = _ptr(x), _pool_strides(x)
        a.gate_pre, a.gate_stride = _ptr(g), _pool_strides(g)
        a.workspace, a.workspace_bytes = self.ws.data_ptr(), self.ws.numel()
        self.args = a

    def run(self) -> None:
        name = "dsqg_pool_gate_bwd" if self.backward else "dsqg_pool_gate_fwd"
        _lib.check(getattr(self.lib, name)(ctypes.byref(self.args), _stream(self.device)), name)


@torch.library.custom_op("dwarf::pool_gate_fwd", mutates_args=())
def pool_gate_fwd(x: Tensor, gate_pre: Tensor) -> Tensor:
    """sigmoid(gate_pre) * cumsum(x, 1) / (n + 1) over [B,N,C]; the result has the promoted
    dtype of x and gate_pre, as the reference's ``sigmoid(inter_gate(xi)) * pool`` does."""
    launch = PoolLaunch(x, gate_pre)
    launch.run()
    return launch.out


@pool_gate_fwd.register_fake
def _(x, gate_pre):
    return x.new_empty(x.shape, dtype=torch.promote_types(x.dtype, gate_pre.dtype))


@torch.library.custom_op("dwarf::pool_gate_bwd", mutates_args=())
def pool_gate_bwd(x: Tensor, gate_pre: Tensor, dout: Tensor, need_dx: bool,
                  need_dgate: bool) -> Tuple[Tensor, Tensor]:
    """(dx in x's dtype, dgate_pre in gate_pre's dtype); an unrequested one is empty."""
    launch = PoolLaunch(x, gate_pre, dout, need_dx, need_dgate)
    launch.run()
    return launch.dx, launch.dgate


@pool_gate_bwd.register_fake
def _(x, gate_pre, dout, need_dx, need_dgate):
    return (x.new_empty(x.shape if need_dx else (0,)),
            gate_pre.new_empty(gate_pre.shape if need_dgate else (0,)))


def _pool_setup_context(ctx, inputs, output):
    x, gate_pre = inputs
    ctx.save_for_backward(x, gate_pre)


def _pool_backward(ctx, dout):
    x, gate_pre = ctx.saved_tensors
    need_dx, need_dg = bool(ctx.needs_input_grad[0]), bool(ctx.needs_input_grad[1])
    if not (need_dx or need_dg):
        return None, None
    dx, dg = pool_gate_bwd(x, gate_pre, dout, need_dx, need_dg)
    return (dx if need_dx else None), (dg if need_dg else None)


torch.library.register_autograd("dwarf::pool_gate_fwd", _pool_backward,
                                setup_context=_pool_setup_context)


class PoolGateFn(torch.autograd.Function):
    """Eager autograd of the pool over the launch objects (see AttentionFn)."""

    @staticmethod
    def forward(ctx, x, gate_pre):
        launch = PoolLaunch(x, gate_pre)
        launch.run()
        ctx.save_for_backward(x, gate_pre)
        return launch.out

    @staticmethod
    def backward(ctx, dout):
        x, gate_pre = ctx.saved_tensors
        need_dx, need_dg = bool(ctx.needs_input_grad[0]), bool(ctx.needs_input_grad[1])
        if not (need_dx or need_dg):
            return None, None
        launch = PoolLaunch(x, gate_pre, dout, need_dx, need_dg)
        launch.run()
        return (launch.dx if need_dx else None), (launch.dgate if need_dg else None)
