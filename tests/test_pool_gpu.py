"""GPU parity of the causal-mean pool with a sigmoid gate (dsqg_pool_gate_fwd / _bwd) against
the CPU oracle (oracle/pool_oracle.py, float64 on the same inputs).

Tolerances, as max|got - ref| over the tensor: fp32 outputs <= 1e-5 * max(1, max|ref|);
float16 outputs <= 2e-3 * max(1, max|ref|); bf16 outputs <= 2e-2 * max(1, max|ref|) (the
rounding of the output dtype, plus fp32 sums in another order than the oracle's).  With a
float16 or bf16 gate, the sigmoid is rounded to the gate's dtype on both sides; the kernel's
fp32 sigmoid and the oracle's differ by a few fp32 ulps, which moves that rounding by one gate
ulp (relative 2^-10 for float16, 2^-7 for bf16) for a few elements in ten thousand.  Those
tests add the resulting bound: u * max|out| for out, u * max|dout * pool| for dgate and
u * max_m sum_{n>=m} |dout| s / (n+1) for dx.
"""

import pytest
import torch

import dwarf_amd
from dwarf_amd import ops
from oracle import pool_gate_forward, pool_gate_forward_backward

pytestmark = pytest.mark.gpu

F32, BF16, F16 = torch.float32, torch.bfloat16, torch.float16
_TOL = {F32: 1e-5, F16: 2e-3, BF16: 2e-2}


def _say(msg):
    print(f"[pool] {msg}", flush=True)


_GATE_ULP = {F32: 0.0, F16: 2.0 ** -10, BF16: 2.0 ** -7}


def _close(got, ref, what, allow=0.0):
    tol = _TOL[got.dtype]
    ref = ref.double()
    scale = max(1.0, ref.abs().max().item()) if ref.numel() else 1.0
    err = (got.detach().cpu().double() - ref).abs().max().item() if ref.numel() else 0.0
    assert err <= tol * scale + allow, (f"{what}: max err {err:.3g} > {tol:.1g} * {scale:.3g}"
                                        f" + {allow:.3g}")


def _gate_allowances(x, gp, dy):
    """Bounds of one gate-dtype ulp of s on (out, dx, dgate); zero for an fp32 gate."""
    u = _GATE_ULP[gp.dtype]
    N = x.shape[1]
    cnt = torch.arange(1, N + 1, dtype=torch.float64).view(1, N, 1)
    pool = x.double().cumsum(1) / cnt
    s = torch.sigmoid(gp.double())
    tail = (dy.double().abs() * s / cnt).flip(1).cumsum(1).flip(1)
    return (u * (s * pool).abs().max().item(), u * tail.max().item(),
            u * (dy.double() * pool).abs().max().item())


def _inputs(B, N, C, xdt, gdt, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn((B, N, C), generator=g).to(xdt)
    gp = (2 * torch.randn((B, N, C), generator=g)).to(gdt)
    dy = torch.randn((B, N, C), generator=g).to(torch.promote_types(xdt, gdt))
    return x, gp, dy


@pytest.mark.parametrize("shape", [(1, 1, 8), (2, 37, 24), (3, 300, 256), (2, 2048, 512),
                                   (1, 5000, 64), (4, 1100, 1032), (4, 4100, 520)])
@pytest.mark.parametrize("xdt,gdt", [(F32, F32), (F32, F16), (BF16, BF16), (F16, F16)])
def test_pool_gate_matches_oracle(gpu_device, shape, xdt, gdt):
    """Forward and both gradients through the autograd op, ragged N and C included ((4, 1100,
    1032): N and C off every power of two, 17 workgroup columns of 64 channels; (4, 4100, 520):
    the forward's 8-rows-per-lane plan, 128-row chunks with a ragged last chunk and a last
    column of 8 channels)."""
    B, N, C = shape
    _say(f"shape={shape} x={xdt} gate={gdt}")
    x, gp, dy = _inputs(B, N, C, xdt, gdt, seed=B * 7919 + N)
    ref_out, ref_dx, ref_dg = pool_gate_forward_backward(x, gp, dy)
    xg = x.to(gpu_device).requires_grad_(True)
    gg = gp.to(gpu_device).requires_grad_(True)
    out = dwarf_amd.causal_mean_pool_gate(xg, gg)
    assert out.dtype == torch.promote_types(xdt, gdt)
    out.backward(dy.to(gpu_device))
    a_out, a_dx, a_dg = _gate_allowances(x, gp, dy)
    _close(out, ref_out, f"{shape} {xdt}/{gdt} out", a_out)
    assert xg.grad.dtype == xdt and gg.grad.dtype == gdt
    _close(xg.grad, ref_dx, f"{shape} {xdt}/{gdt} dx", a_dx)
    _close(gg.grad, ref_dg, f"{shape} {xdt}/{gdt} dgate", a_dg)


def test_pool_gate_strided_views(gpu_device):
    """x a channel slice of a wider tensor and gate_pre a permuted [N,B,C] buffer, read in place
    through their strides; dout expanded along B and N (zero strides, copied by the op)."""
    B, N, C = 3, 333, 64
    _say("strided views")
    g = torch.Generator().manual_seed(3)
    wide = torch.randn((B, N, C + 32), generator=g)
    x = wide[:, :, 16:16 + C]
    gp = torch.randn((N, B, C), generator=g).permute(1, 0, 2)
    row = torch.randn((1, 1, C), generator=g)
    dy = row.expand(B, N, C)
    ref_out, ref_dx, ref_dg = pool_gate_forward_backward(x, gp, dy)
    wg = wide.to(gpu_device)
    xg = wg[:, :, 16:16 + C]
    gg = gp.permute(1, 0, 2).contiguous().to(gpu_device).permute(1, 0, 2)
    assert xg.stride() == (N * (C + 32), C + 32, 1) and gg.stride(0) == C
    out = ops.pool_gate_fwd(xg, gg)
    _close(out, ref_out, "strided out")
    dx, dgate = ops.pool_gate_bwd(xg, gg, row.to(gpu_device).expand(B, N, C), True, True)
    _close(dx, ref_dx, "strided dx")
    _close(dgate, ref_dg, "strided dgate")


def test_pool_gate_single_gradient_and_empty(gpu_device):
    B, N, C = 2, 100, 32
    _say("single gradient / empty")
    x, gp, dy = _inputs(B, N, C, F32, F32, seed=5)
    _, ref_dx, ref_dg = pool_gate_forward_backward(x, gp, dy)
    xg, gg, dyg = x.to(gpu_device), gp.to(gpu_device), dy.to(gpu_device)
    dx, dgate = ops.pool_gate_bwd(xg, gg, dyg, True, False)
    assert dgate.numel() == 0
    _close(dx, ref_dx, "dx only")
    dx, dgate = ops.pool_gate_bwd(xg, gg, dyg, False, True)
    assert dx.numel() == 0
    _close(dgate, ref_dg, "dgate only")
    gx = xg.clone().requires_grad_(True)
    dwarf_amd.causal_mean_pool_gate(gx, gg).backward(dyg)   # gate is not a leaf needing grad
    _close(gx.grad, ref_dx, "autograd dx only")
    for shape in ((0, 5, 16), (2, 0, 16)):
        e = torch.empty(shape, device=gpu_device)
        assert dwarf_amd.causal_mean_pool_gate(e, e).shape == shape
    with pytest.raises(AssertionError):
        dwarf_amd.causal_mean_pool_gate(torch.zeros((1, 4, 12), device=gpu_device),
                                        torch.zeros((1, 4, 12), device=gpu_device))


def test_pool_gate_deterministic(gpu_device):
    x, gp, dy = (t.to(gpu_device) for t in _inputs(4, 1500, 256, BF16, BF16, seed=6))
    _say("determinism")
    a = ops.pool_gate_fwd(x, gp)
    b = ops.pool_gate_fwd(x, gp)
    assert torch.equal(a, b)
    da = ops.pool_gate_bwd(x, gp, dy, True, True)
    db = ops.pool_gate_bwd(x, gp, dy, True, True)
    assert torch.equal(da[0], db[0]) and torch.equal(da[1], db[1])


@pytest.mark.parametrize("shape", [(2, 100_000, 64), (2, 16_384, 2048)])
def test_pool_gate_large_properties(gpu_device, shape):
    """At sizes the float64 oracle would be slow on: constant input gives pool == 1 exactly
    (sums of ones are exact in fp32), so out == sigmoid(gate); the last row times N / s is the
    column total; dx for dout = 1 at gate 0 is 0.5 * (H_N - H_m).  Long columns, then wide
    rows."""
    B, N, C = shape
    _say(f"large shape={shape}")
    ones = torch.ones((B, N, C), device=gpu_device)
    g = torch.Generator(device="cpu").manual_seed(8)
    gp = torch.randn((B, N, C), generator=g).to(gpu_device)
    out = ops.pool_gate_fwd(ones, gp)
    torch.testing.assert_close(out, torch.sigmoid(gp), rtol=2e-6, atol=1e-7)
    x = torch.randn((B, N, C), generator=g).to(gpu_device)
    zero = torch.zeros_like(x)
    out = ops.pool_gate_fwd(x, zero)
    total = x.double().sum(1)
    got = out[:, -1].double() * 2 * N
    assert (got - total).abs().max().item() <= 1e-4 * max(1.0, total.abs().max().item())
    dx, _ = ops.pool_gate_bwd(x, zero, torch.ones_like(x), True, False)
    H = torch.cumsum(1.0 / torch.arange(1, N + 1, dtype=torch.float64), 0)
    Hm = torch.cat([torch.zeros(1, dtype=torch.float64), H[:-1]])
    want = 0.5 * (H[-1] - Hm)
    err = (dx[1, :, 5].double().cpu() - want).abs().max().item()
    assert err <= 1e-5 * want.abs().max().item(), f"harmonic dx err {err:.3g}"


@pytest.mark.parametrize("interference", [False, True])
def test_block_forward_backward_matches_oracle(gpu_device, interference):
    """DSQGBlock (train/train_2048_condU.py:260-297) on the HIP kernels vs the same weights
    through a CPU fp32 restatement with the oracles as the attention and pool cores: output and
    every parameter gradient within 1e-4 of the tensor's max (plus 1e-5)."""
    from oracle import dsqg_forward
    torch.manual_seed(31)
    E, H, F, B, N = 256, 4, 512, 2, 300
    _say(f"block interference={interference}")
    m = dwarf_amd.DSQGBlock(E, H, F, seq_len=N, dropout=0.0, interference=interference)
    with torch.no_grad():
        m.attn.pos_bias.add_(0.3 * torch.randn_like(m.attn.pos_bias))
        m.attn.scale_embed.copy_(0.5 * torch.randn_like(m.attn.scale_embed))
        m.attn.if_gain.copy_(0.8 + 0.4 * torch.rand_like(m.attn.if_gain))
    x = torch.randn(B, N, E)
    dy = torch.randn(B, N, E)
    p = {k: v.detach().clone().requires_grad_(True) for k, v in m.named_parameters()}
    lin = torch.nn.functional.linear
    ln = lambda t, pre: torch.nn.functional.layer_norm(t, (E,), p[pre + ".weight"], p[pre + ".bias"])
    HD = E // H

    def attn(t, kv):
        qkv = lin(t, p["attn.qkv_proj.weight"], p["attn.qkv_proj.bias"])
        q, k, v = (u.reshape(B, N, H, HD).permute(0, 2, 1, 3) for u in qkv.split(E, dim=-1))
        if kv is not None:
            k, v = k + kv[0], v + kv[1]
        o = dsqg_forward(q, k, v, p["attn.pos_bias"], p["attn.scale_embed"],
                         if_gain=p["attn.if_gain"])
        flat = o.permute(0, 2, 1, 3).reshape(B, N, E)
        gate = torch.sigmoid(lin(t, p["attn.gate_proj.weight"], p["attn.gate_proj.bias"]))
        return lin(flat * gate, p["attn.out_proj.weight"], p["attn.out_proj.bias"])

    kv = None
    if interference:
        xi = ln(x, "inter_norm")
        inter = pool_gate_forward(xi, lin(xi, p["inter_gate.weight"], p["inter_gate.bias"]),
                                  dtype=torch.float32)
        kv = tuple(lin(inter, p[f"inter_{n}_proj.weight"], p[f"inter_{n}_proj.bias"])
                   .view(B, N, H, HD).permute(0, 2, 1, 3) for n in ("k", "v"))
    h = x + attn(ln(x, "norm1"), kv)
    f = lin(torch.nn.functional.gelu(lin(ln(h, "norm2"), p["ffn.fc1.weight"], p["ffn.fc1.bias"])),
            p["ffn.fc2.weight"], p["ffn.fc2.bias"])
    ref = h + f
    ref.backward(dy)

    mg = m.to(gpu_device)
    y = mg(x.to(gpu_device))
    y.backward(dy.to(gpu_device))

    def close(a, b, what):
        # 1e-5 absolute floor: the key-projection bias gets no gradient in exact arithmetic
        # (adding a constant to every key of a row shifts the scores by q.c, and the softmax
        # weights' gradients sum to zero), so both sides hold rounding noise of ~1e-7 there.
        err = (a.detach().float().cpu() - b).abs().max().item()
        assert err <= 1e-4 * b.abs().max().item() + 1e-5, f"{what}: err {err:.3g}"

    close(y, ref.detach(), "output")
    for name, prm in mg.named_parameters():
        close(prm.grad, p[name].grad, f"grad {name}")


def test_block_prefill_then_steps_equal_forward(gpu_device):
    """DSQGBlock with interference: prefill on a prompt, then one decode step per token (ring
    step plus the pool's running sum), equals the block's forward row by row (fp32, 1e-4)."""
    torch.manual_seed(41)
    E, H, F, B, N0, T = 256, 4, 512, 2, 90, 5
    _say("block decode")
    m = dwarf_amd.DSQGBlock(E, H, F, dropout=0.0, interference=True).to(gpu_device).eval()
    x = torch.randn(B, N0 + T, E, device=gpu_device)
    with torch.no_grad():
        full = m(x)
        cache = m.new_cache(B)
        pre = m.prefill(x[:, :N0], cache)
        steps = [m.step(x[:, t], cache) for t in range(N0, N0 + T)]
    scale = full.abs().max().item()
    assert (pre - full[:, :N0]).abs().max().item() <= 1e-4 * scale
    got = torch.stack(steps, dim=1)
    err = (got - full[:, N0:]).abs().max().item()
    assert err <= 1e-4 * scale, f"block step err {err:.3g}"
