"""Drop-in modules (dwarf_amd/modules.py): state-dict compatibility with the reference modules
and end-to-end parity of forward + parameter gradients against the oracle.

Reference modules: kernels/dsqg_attention_v3.py:463-536 (DSQGAttentionV3),
train/train_2048_condU.py:116-205 and train/train_4096_13m_condU.py:110-175 (DSQGAttentionQW),
kernels/dsqg_attention_v2.py:434-471 (DSQGAttentionN_Fused).
"""
import io
import math

import pytest
import torch

from dwarf_amd.modules import DSQGAttentionN_Fused, DSQGAttentionQW, DSQGAttentionV3
from dwarf_amd.offsets import OFFSETS_J47, OFFSETS_V3
from oracle import dsqg_forward

# Parameter / buffer names and shapes as the reference constructors create them (E = embedding
# dim, H heads, HD = E / H, J offsets).
def _expected(cls_name, E, H, J):
    HD = E // H
    common = {"qkv_proj.weight": (3 * E, E), "qkv_proj.bias": (3 * E,),
              "out_proj.weight": (E, E), "out_proj.bias": (E,),
              "gate_proj.weight": (E, E), "gate_proj.bias": (E,), "pos_bias": (J, H)}
    if cls_name == "V3":
        return {**common, "offsets": (J,), "scale_embed": (J, HD)}
    if cls_name == "QW":
        return {**common, "scale_embed": (J, HD), "if_gain": (H,)}
    return {**common, "offsets": (J,)}


@pytest.mark.parametrize("name,ctor,J", [
    ("V3", lambda: DSQGAttentionV3(768, 12), 44),
    ("QW", lambda: DSQGAttentionQW(768, 12), 44),
    ("QW", lambda: DSQGAttentionQW(256, 8, seq_len=4096, offsets=OFFSETS_J47), 47),
    ("N", lambda: DSQGAttentionN_Fused(768, 12), 44),
])
def test_state_dict_names_and_shapes(name, ctor, J):
    m = ctor()
    got = {k: tuple(v.shape) for k, v in m.state_dict().items()}
    assert got == _expected(name, m.embedding_dim, m.num_heads, J)


def test_initial_values_match_reference_init():
    H = 12
    for m, gate_bias in ((DSQGAttentionV3(768, H), 0.0), (DSQGAttentionQW(768, H), 0.0),
                         (DSQGAttentionN_Fused(768, H), 2.0)):
        assert torch.all(m.gate_proj.bias == gate_bias)
        # pos_bias[j,h] = -log(1 + delta_j) * (0.2 + 1.8 h / (H - 1)), element by element.
        for j in (0, 1, 32, 33, 43):
            for h in (0, 5, H - 1):
                want = -math.log(1.0 + OFFSETS_V3[j]) * (0.2 + 1.8 * h / (H - 1))
                assert abs(m.pos_bias[j, h].item() - want) < 1e-6
    assert torch.all(DSQGAttentionV3(768, H).scale_embed == 0)
    assert torch.all(DSQGAttentionQW(768, H).if_gain == 1)
    assert DSQGAttentionV3(768, H).offsets.tolist() == list(OFFSETS_V3)


def test_reference_format_checkpoint_loads_strict():
    """A state dict with the reference's keys (as torch.save writes it) loads unchanged."""
    g = torch.Generator().manual_seed(5)
    src = {k: torch.randn(s, generator=g) for k, s in _expected("QW", 256, 8, 44).items()}
    buf = io.BytesIO()
    torch.save(src, buf)
    buf.seek(0)
    sd = torch.load(buf, weights_only=True)
    m = DSQGAttentionQW(256, 8)
    m.load_state_dict(sd, strict=True)
    assert torch.equal(m.if_gain.detach(), src["if_gain"])
    v3 = DSQGAttentionV3(256, 8)
    sd3 = {k: torch.randn(s, generator=g) for k, s in _expected("V3", 256, 8, 44).items()}
    sd3["offsets"] = torch.tensor(OFFSETS_V3, dtype=torch.long)
    v3.load_state_dict(sd3, strict=True)


def _reference_forward(m, x, kv_inject=None):
    """The reference module's forward, fp32 on the CPU, with the oracle as the attention core."""
    B, N, E = x.shape
    H, HD = m.num_heads, m.head_dim
    p = {k: v.detach().float().cpu().requires_grad_(v.requires_grad) for k, v in m.named_parameters()}
    qkv = torch.nn.functional.linear(x, p["qkv_proj.weight"], p["qkv_proj.bias"])
    q, k, v = (t.reshape(B, N, H, HD).permute(0, 2, 1, 3) for t in qkv.split(E, dim=-1))
    if kv_inject is not None:
        k = k + kv_inject[0]
        v = v + kv_inject[1]
    out = dsqg_forward(q, k, v, p["pos_bias"], p.get("scale_embed"), offsets=m._offsets,
                       if_gain=p.get("if_gain"))
    flat = out.permute(0, 2, 1, 3).reshape(B, N, E)
    gate = torch.sigmoid(torch.nn.functional.linear(x, p["gate_proj.weight"], p["gate_proj.bias"]))
    return torch.nn.functional.linear(flat * gate, p["out_proj.weight"], p["out_proj.bias"]), p


@pytest.mark.gpu
@pytest.mark.parametrize("cls", ["V3", "QW", "N"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_module_forward_backward_matches_oracle(gpu_device, cls, dtype):
    """Module on the HIP kernels vs the same weights through the CPU oracle: output and the
    gradients of every parameter.  fp32 tolerance covers GPU-vs-CPU matmul rounding (1e-4 of
    the tensor's max); bf16 runs the module in bf16 (projections and kernels), 3e-2 of max."""
    torch.manual_seed(11)
    E, H, B, N = 256, 4, 2, 320
    m = {"V3": DSQGAttentionV3, "QW": DSQGAttentionQW, "N": DSQGAttentionN_Fused}[cls](E, H, dropout=0.0)
    with torch.no_grad():  # move the zero/one inits so that every parameter matters
        m.pos_bias.add_(0.3 * torch.randn_like(m.pos_bias))
        if hasattr(m, "scale_embed"):
            m.scale_embed.copy_(0.5 * torch.randn_like(m.scale_embed))
        if hasattr(m, "if_gain"):
            m.if_gain.copy_(0.8 + 0.4 * torch.rand_like(m.if_gain))
    x = torch.randn(B, N, E)
    dy = torch.randn(B, N, E)
    ref, p = _reference_forward(m, x)
    ref.backward(dy)

    mg = m.to(gpu_device, dtype)
    xg = x.to(gpu_device, dtype)
    y = mg(xg)
    y.backward(dy.to(gpu_device, dtype))
    tol = 1e-4 if dtype == torch.float32 else 3e-2

    def close(a, b, what):
        a = a.float().cpu()
        scale = max(1.0, b.abs().max().item()) if dtype == torch.bfloat16 else b.abs().max().item()
        err = (a - b).abs().max().item()
        assert err <= tol * scale, f"{cls} {dtype} {what}: max err {err:.3g} vs scale {scale:.3g}"

    close(y.detach(), ref.detach(), "output")
    for name, prm in mg.named_parameters():
        close(prm.grad, p[name].grad, f"grad {name}")


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_module_kv_inject(gpu_device, dtype):
    """Huygens K/V injection (k + k_delta, v + v_delta, q unchanged): output and the gradients
    of x, both deltas and every parameter against the reference forward through the oracle.
    The deltas' gradients come back as the K / V slices of d(qkv).  Tolerance as in
    test_module_forward_backward_matches_oracle."""
    torch.manual_seed(12)
    E, H, B, N = 256, 4, 2, 300
    m = DSQGAttentionQW(E, H, dropout=0.0)
    with torch.no_grad():
        m.pos_bias.add_(0.3 * torch.randn_like(m.pos_bias))
        m.scale_embed.copy_(0.5 * torch.randn_like(m.scale_embed))
        m.if_gain.copy_(0.8 + 0.4 * torch.rand_like(m.if_gain))
    x = torch.randn(B, N, E).to(dtype).float().requires_grad_(True)
    kd = (0.5 * torch.randn(B, H, N, E // H)).to(dtype).float().requires_grad_(True)
    vd = (0.5 * torch.randn(B, H, N, E // H)).to(dtype).float().requires_grad_(True)
    dy = torch.randn(B, N, E).to(dtype).float()
    ref, p = _reference_forward(m, x, (kd, vd))
    ref.backward(dy)

    mg = m.to(gpu_device, dtype)
    xg, kdg, vdg = (t.detach().to(gpu_device, dtype).requires_grad_(True) for t in (x, kd, vd))
    y = mg(xg, kv_inject=(kdg, vdg))
    y.backward(dy.to(gpu_device, dtype))
    tol = 1e-4 if dtype == torch.float32 else 3e-2

    def close(a, b, what):
        a = a.float().cpu()
        scale = max(1.0, b.abs().max().item()) if dtype == torch.bfloat16 else b.abs().max().item()
        err = (a - b).abs().max().item()
        assert err <= tol * scale, f"kv_inject {dtype} {what}: max err {err:.3g} vs scale {scale:.3g}"

    close(y.detach(), ref.detach(), "output")
    close(xg.grad, x.grad, "grad x")
    close(kdg.grad, kd.grad, "grad k_delta")
    close(vdg.grad, vd.grad, "grad v_delta")
    for name, prm in mg.named_parameters():
        close(prm.grad, p[name].grad, f"grad {name}")


@pytest.mark.gpu
@pytest.mark.parametrize("cls,dtype,N0", [("QW", torch.float32, 70), ("QW", torch.bfloat16, 70),
                                          ("V3", torch.bfloat16, 1600), ("N", torch.float32, 40)])
def test_module_prefill_then_steps_equal_forward(gpu_device, cls, dtype, N0):
    """prefill on N0 prompt tokens, then one decode step per token, equals the module's forward
    on the whole sequence, row by row (N0 = 1600 wraps the 1537-slot ring).  QW also checks the
    K/V injection at every step.  Tolerance: fp32 1e-4 of max|y|; bf16 3e-2 * max(1, max|y|)."""
    torch.manual_seed(23)
    E, H, B, T = 256, 4, 2, 4
    m = {"V3": DSQGAttentionV3, "QW": DSQGAttentionQW, "N": DSQGAttentionN_Fused}[cls](E, H, dropout=0.0)
    with torch.no_grad():
        m.pos_bias.add_(0.3 * torch.randn_like(m.pos_bias))
        if hasattr(m, "scale_embed"):
            m.scale_embed.copy_(0.5 * torch.randn_like(m.scale_embed))
        if hasattr(m, "if_gain"):
            m.if_gain.copy_(0.8 + 0.4 * torch.rand_like(m.if_gain))
    m = m.to(gpu_device, dtype).eval()
    x = torch.randn(B, N0 + T, E, device=gpu_device, dtype=dtype)
    inject = cls == "QW"
    kd = (0.5 * torch.randn(B, H, N0 + T, E // H, device=gpu_device)).to(dtype) if inject else None
    vd = (0.5 * torch.randn(B, H, N0 + T, E // H, device=gpu_device)).to(dtype) if inject else None
    with torch.no_grad():
        full = m(x, kv_inject=(kd, vd)) if inject else m(x)
        cache = m.new_cache(B)
        pre = (m.prefill(x[:, :N0], cache, kv_inject=(kd[:, :, :N0], vd[:, :, :N0])) if inject
               else m.prefill(x[:, :N0], cache))
        steps = [m.step(x[:, t], cache, kv_inject=(kd[:, :, t], vd[:, :, t])) if inject
                 else m.step(x[:, t], cache) for t in range(N0, N0 + T)]
    ref = full.float()
    scale = ref.abs().max().item()
    tol = 1e-4 * scale if dtype == torch.float32 else 3e-2 * max(1.0, scale)
    # The prompt part differs from the full forward only by the projections' GEMM shapes.
    err_pre = (pre.float() - ref[:, :N0]).abs().max().item()
    assert err_pre <= tol, f"{cls} {dtype} N0={N0}: prefill err {err_pre:.3g} > {tol:.3g}"
    got = torch.stack(steps, dim=1).float()
    err = (got - ref[:, N0:]).abs().max().item()
    assert err <= tol, f"{cls} {dtype} N0={N0}: step err {err:.3g} > {tol:.3g}"
    assert int(cache.pos[0]) == N0 + T
