"""The custom ops' fake (meta) implementations, as torch.compile / export trace them: shapes,
dtypes and output layouts under FakeTensorMode (no kernel runs; the op-level checks need no
GPU), and the autograd formulas that call the backward ops (marked gpu: the autograd engine
initialises the device)."""

import pytest
import torch
from torch._subclasses.fake_tensor import FakeTensorMode

import dwarf_amd
from dwarf_amd import ops
from dwarf_amd.offsets import OFFSETS_V3

B, H, N, D, J = 2, 4, 128, 64, len(OFFSETS_V3)


@pytest.fixture
def fake():
    with FakeTensorMode(allow_non_fake_inputs=False) as mode:
        yield mode


def _t(*shape, dtype=torch.bfloat16, grad=False):
    return torch.empty(*shape, dtype=dtype, device="cuda", requires_grad=grad)


def test_forward_and_backward_ops(fake):
    q = _t(B, H, N, D)
    pb = _t(J, H, dtype=torch.float32)
    out, lse, alr = ops.dsqg_fwd(q, q, q, pb, None, None, None, list(OFFSETS_V3))
    assert out.shape == (B, H, N, D) and out.dtype == torch.bfloat16
    assert out.stride() == (N * H * D, D, H * D, 1)  # token-major storage
    assert lse.shape == (B, H, N) and lse.dtype == torch.float32
    assert alr.shape == (B, H, 11, N) and alr.dtype == torch.float32  # 11 long-range taps
    grads = ops.dsqg_bwd(q, q, q, q, lse, alr, pb, None, None, None, list(OFFSETS_V3), False,
                         False, True)
    assert [tuple(g.shape) for g in grads] == [(B, H, N, D)] * 3 + [(J, H), (0,), (0,), (H,)]
    qkv = _t(B, N, 3 * H * D)
    out, lse, alr = ops.dsqg_fwd_qkv(qkv, H, pb, None, None, None, list(OFFSETS_V3))
    assert out.shape == (B, H, N, D) and lse.shape == (B, H, N) and alr.shape == (B, H, 11, N)
    dqkv, dpb, dse, dg, da = ops.dsqg_bwd_qkv(qkv, H, q, lse, alr, pb, None, None, None,
                                              list(OFFSETS_V3), True, True, False)
    assert dqkv.shape == qkv.shape and dse.shape == (J, D) and dg.shape == (H, J)
    # K/V injection: the injected K/V come back for the backward, which returns one d(qkv).
    out, lse, alr, k_eff, v_eff = ops.dsqg_fwd_qkv_kv(qkv, q, q, H, pb, None, None, None,
                                                      list(OFFSETS_V3))
    assert out.shape == (B, H, N, D) and lse.shape == (B, H, N) and alr.shape == (B, H, 11, N)
    assert k_eff.shape == (B, H, N, D) and v_eff.shape == (B, H, N, D)
    dqkv, dpb, dse, dg, da = ops.dsqg_bwd_qkv_kv(qkv, k_eff, v_eff, H, q, lse, alr, pb, None,
                                                 None, None, list(OFFSETS_V3), False, False, False)
    assert dqkv.shape == qkv.shape and dpb.shape == (J, H) and dse.numel() == 0


def test_decode_and_pool_ops(fake):
    q = _t(B, H, D)
    ring = _t(B, H, 1537, D)
    pos = torch.empty(B, dtype=torch.int64, device="cuda")
    pb = _t(J, H, dtype=torch.float32)
    o = ops.dsqg_decode(q, q, q, ring, ring, pos, pb, None, None, None, list(OFFSETS_V3))
    assert o.shape == (B, H, D) and o.dtype == torch.bfloat16
    x = _t(B, N, 32, dtype=torch.float32)
    g = _t(B, N, 32, dtype=torch.float16)
    y = ops.pool_gate_fwd(x, g)
    assert y.shape == (B, N, 32) and y.dtype == torch.float32  # promoted, as in the reference
    dx, dg = ops.pool_gate_bwd(x, g, y, True, False)
    assert dx.shape == x.shape and dx.dtype == x.dtype and dg.numel() == 0


@pytest.mark.gpu
def test_autograd_through_fake_tensors(gpu_device, fake):
    # The autograd engine sets up the device's streams, so this part needs a visible GPU.
    q, k, v = (_t(B, H, N, D, grad=True) for _ in range(3))
    pb = _t(J, H, dtype=torch.float32, grad=True)
    se = _t(J, D, dtype=torch.float32, grad=True)
    out = dwarf_amd.dsqg_attention_v3(q, k, v, pb, se)
    out.sum().backward()
    assert q.grad.shape == q.shape and pb.grad.shape == pb.shape and se.grad.shape == se.shape
    x = _t(B, N, 64, grad=True)
    g = _t(B, N, 64, grad=True)
    dwarf_amd.causal_mean_pool_gate(x, g).sum().backward()
    assert x.grad.shape == x.shape and g.grad.dtype == g.dtype


@pytest.mark.gpu
def test_compiled_graph_matches_eager(gpu_device):
    """A whole-graph capture (torch.compile, aot_eager backend: no generated kernels) of the
    attention and the pool, forward and backward, gives the eager results bit for bit."""
    g = torch.Generator().manual_seed(3)
    q, k, v = (torch.randn(B, H, N, D, generator=g).to(gpu_device, torch.bfloat16) for _ in range(3))
    pb = torch.randn(J, H, generator=g).to(gpu_device)
    x = torch.randn(B, N, 64, generator=g).to(gpu_device)
    gp = torch.randn(B, N, 64, generator=g).to(gpu_device)

    def fn(q, k, v, pb, x, gp):
        return (dwarf_amd.dsqg_attention_v3(q, k, v, pb, None).float().square().sum()
                + dwarf_amd.causal_mean_pool_gate(x, gp).square().sum())

    def run(f):
        ins = [t.clone().requires_grad_(True) for t in (q, k, v, pb, x, gp)]
        loss = f(*ins)
        loss.backward()
        return [loss.detach()] + [t.grad for t in ins]

    eager = run(fn)
    compiled = run(torch.compile(fn, backend="aot_eager", fullgraph=True))
    for a, b in zip(eager, compiled):
        assert torch.equal(a, b)


@pytest.mark.gpu
def test_compiled_qkv_with_kv_inject_matches_eager(gpu_device):
    """The qkv entry with a K/V injection (custom ops dsqg_fwd_qkv_kv / dsqg_bwd_qkv_kv under
    torch.compile, aot_eager) gives the eager results bit for bit, and its gradients are those
    of the split-head form with the adds written out."""
    g = torch.Generator().manual_seed(4)
    qkv = torch.randn(B, N, 3 * H * D, generator=g).to(gpu_device, torch.bfloat16)
    kd, vd = (torch.randn(B, H, N, D, generator=g).to(gpu_device, torch.bfloat16) for _ in range(2))
    pb = torch.randn(J, H, generator=g).to(gpu_device)
    se = (0.05 * torch.randn(J, D, generator=g)).to(gpu_device)

    def fn(qkv, kd, vd, pb, se):
        out = dwarf_amd.dsqg_attention_qkv(qkv, H, pb, se, kv_inject=(kd, vd))
        return out.float().square().sum()

    def split(qkv, kd, vd, pb, se):
        q, k, v = ops.split_qkv(qkv, H)
        return dwarf_amd.dsqg_attention(q, k + kd, v + vd, pb, se).float().square().sum()

    def run(f):
        ins = [t.clone().requires_grad_(True) for t in (qkv, kd, vd, pb, se)]
        loss = f(*ins)
        loss.backward()
        return [loss.detach()] + [t.grad for t in ins]

    eager = run(fn)
    compiled = run(torch.compile(fn, backend="aot_eager", fullgraph=True))
    for a, b in zip(eager, compiled):
        assert torch.equal(a, b)
    for a, b in zip(eager, run(split)):  # same kernels on the same (bf16-rounded) K/V
        assert torch.equal(a, b)
