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
from tests import tolerance

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


def _reference_forward(m, x, kv_inject=None, rounded=False, keep=None):
    """The reference module's forward, fp32 on the CPU, with the oracle as the attention core.

    With ``rounded`` every tensor the bf16 module stores in bf16 is rounded to bf16 at the same
    point (and autograd rounds the gradients flowing through those points the same way).  With a
    dict ``keep`` the projections' inputs and outputs are left in it (qkv, gate_pre and the
    gated product z retain their gradients)."""
    B, N, E = x.shape
    H, HD = m.num_heads, m.head_dim
    r = (lambda t: t.to(torch.bfloat16).float()) if rounded else (lambda t: t)
    p = {k: v.detach().float().cpu().requires_grad_(v.requires_grad) for k, v in m.named_parameters()}
    qkv = r(torch.nn.functional.linear(x, p["qkv_proj.weight"], p["qkv_proj.bias"]))
    q, k, v = (t.reshape(B, N, H, HD).permute(0, 2, 1, 3) for t in qkv.split(E, dim=-1))
    if kv_inject is not None:
        k = r(k + kv_inject[0])
        v = r(v + kv_inject[1])
    out = r(dsqg_forward(q, k, v, p["pos_bias"], p.get("scale_embed"), offsets=m._offsets,
                         if_gain=p.get("if_gain")))
    flat = out.permute(0, 2, 1, 3).reshape(B, N, E)
    gate_pre = r(torch.nn.functional.linear(x, p["gate_proj.weight"], p["gate_proj.bias"]))
    z = r(flat * r(torch.sigmoid(gate_pre)))
    if keep is not None:
        for t in (qkv, gate_pre, z):
            t.retain_grad()
        keep.update(qkv=qkv, gate_pre=gate_pre, z=z)
    return r(torch.nn.functional.linear(z, p["out_proj.weight"], p["out_proj.bias"])), p


def _reference_run(m, x, dy, kv_inject=None, rounded=False):
    """Output and gradients of the reference forward (see _reference_forward) for upstream dy:
    {"output", "grad <param>", and "grad x" / "grad k_delta" / "grad v_delta" for the inputs
    that require grad}.  With ``rounded`` the parameter gradients are rounded to bf16 too (the
    bf16 module keeps them in its parameters' dtype).  Without it, also the magnitudes of the
    module's projection GEMMs, |A| |B| for each product A B that yields a checked tensor (the
    output, the projections' weight and bias gradients, the input gradient), as a second dict."""
    leaves = [x] + (list(kv_inject) if kv_inject is not None else [])
    leaves = [t.detach().clone().requires_grad_(t.requires_grad) for t in leaves]
    kv = (leaves[1], leaves[2]) if kv_inject is not None else None
    keep = {} if not rounded else None
    y, p = _reference_forward(m, leaves[0], kv, rounded, keep)
    y.backward(dy)
    r = (lambda t: t.to(torch.bfloat16).float()) if rounded else (lambda t: t)
    res = {"output": y.detach()}
    for name, prm in p.items():
        res[f"grad {name}"] = r(prm.grad)
    for name, t in zip(("grad x", "grad k_delta", "grad v_delta"), leaves):
        if t.grad is not None:
            res[name] = r(t.grad)
    if rounded:
        return res
    E = x.shape[-1]
    a = lambda t: t.detach().abs().reshape(-1, t.shape[-1])
    ax, az, ady = a(leaves[0]), a(keep["z"]), a(dy)
    adqkv, adg = a(keep["qkv"].grad), a(keep["gate_pre"].grad)
    mags = {
        "output": (az @ p["out_proj.weight"].detach().abs().t() + p["out_proj.bias"].detach().abs()).reshape(y.shape),
        "grad out_proj.weight": ady.t() @ az, "grad out_proj.bias": ady.sum(0),
        "grad gate_proj.weight": adg.t() @ ax, "grad gate_proj.bias": adg.sum(0),
        "grad qkv_proj.weight": adqkv.t() @ ax, "grad qkv_proj.bias": adqkv.sum(0),
        "grad x": (adqkv @ p["qkv_proj.weight"].detach().abs()
                   + adg @ p["gate_proj.weight"].detach().abs()).reshape(leaves[0].shape),
    }
    assert mags["grad qkv_proj.weight"].shape == (3 * E, E)
    return res, mags


def _bf16_module(m):
    """m with its parameters rounded to bf16 (the values the bf16 module computes with)."""
    return m.to(torch.bfloat16).float()


def _check_module_run(got, ref, ref_rounded, mags, dtype, label):
    """fp32: max|x - ref| <= 1e-4 max|ref| per tensor (GPU vs CPU GEMM accumulation order);
    bf16: the elementwise rule of tests/tolerance.check_module (with the projections' rounding
    term for the tensors a projection GEMM yields)."""
    errs = {}
    for key, want in ref.items():
        have = got[key].float().cpu()
        if dtype == torch.float32:
            err = (have - want).abs().max().item()
            scale = want.abs().max().item()
            assert err <= 1e-4 * scale, f"{label} {key}: max err {err:.3g} vs scale {scale:.3g}"
        else:
            errs[key] = tolerance.check_module(f"{label} {key}", have, want, ref_rounded[key],
                                               mags.get(key),
                                               say=lambda s: print(f"[module] {s}", flush=True))
    if errs:
        worst = max(errs.items(), key=lambda kv: kv[1][1])
        tolerance.SUMMARY.append(f"{label}: worst {worst[0]} {worst[1][0]:.2e}/{worst[1][1]:.2f} "
                                 f"over {len(errs)} tensors")


def _perturb(m):
    """Move the zero/one inits so that every parameter matters."""
    with torch.no_grad():
        m.pos_bias.add_(0.3 * torch.randn_like(m.pos_bias))
        if hasattr(m, "scale_embed"):
            m.scale_embed.copy_(0.5 * torch.randn_like(m.scale_embed))
        if hasattr(m, "if_gain"):
            m.if_gain.copy_(0.8 + 0.4 * torch.rand_like(m.if_gain))


def _module_parity(gpu_device, m, dtype, B, N, label, kv=False):
    E, H = m.embedding_dim, m.num_heads
    if dtype == torch.bfloat16:
        m = _bf16_module(m)
    rnd = (lambda t: t.to(dtype).float())
    x = rnd(torch.randn(B, N, E)).requires_grad_(True)
    dy = rnd(torch.randn(B, N, E))
    inject = None
    if kv:
        inject = tuple(rnd(0.5 * torch.randn(B, H, N, E // H)).requires_grad_(True) for _ in range(2))
    ref, mags = _reference_run(m, x, dy, inject)
    ref_rounded = _reference_run(m, x, dy, inject, rounded=True) if dtype == torch.bfloat16 else None

    mg = m.to(gpu_device, dtype)
    xg = x.detach().to(gpu_device, dtype).requires_grad_(True)
    ig = None
    if kv:
        ig = tuple(t.detach().to(gpu_device, dtype).requires_grad_(True) for t in inject)
    y = mg(xg, kv_inject=ig) if kv else mg(xg)
    y.backward(dy.to(gpu_device, dtype))
    got = {"output": y.detach(), "grad x": xg.grad}
    for name, prm in mg.named_parameters():
        got[f"grad {name}"] = prm.grad
    if kv:
        got["grad k_delta"], got["grad v_delta"] = ig[0].grad, ig[1].grad
    _check_module_run(got, ref, ref_rounded, mags, dtype, label)


@pytest.mark.gpu
@pytest.mark.parametrize("cls", ["V3", "QW", "N"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_module_forward_backward_matches_oracle(gpu_device, cls, dtype):
    """Module on the HIP kernels vs the same (dtype-rounded) weights and input through the CPU
    oracle: the output and the gradients of the input and of every parameter.  fp32: 1e-4 of the
    tensor's max (GPU-vs-CPU GEMM accumulation order); bf16 runs the module in bf16
    (projections and kernels) and is held elementwise to 2e-2 + 2^-9 |ref| plus twice the
    measured effect of the module's bf16 roundings (tests/tolerance.check_module)."""
    torch.manual_seed(11)
    E, H, B, N = 256, 4, 2, 320
    m = {"V3": DSQGAttentionV3, "QW": DSQGAttentionQW, "N": DSQGAttentionN_Fused}[cls](E, H, dropout=0.0)
    _perturb(m)
    _module_parity(gpu_device, m, dtype, B, N, f"module {cls} {str(dtype)[6:]} E{E} H{H} B{B} N{N}")


@pytest.mark.gpu
def test_module_qw_n4096_trainer_shape(gpu_device):
    """The N=4096 13M trainer's attention module in bf16: DSQGAttentionQW(256, 8, seq_len=4096)
    over the 47-offset table (train/train_4096_13m_condU.py:51-54, 89-93, 104-105, 122), so
    HD 32 with 14 long-range taps, at N = 4096 (two sequences), held to the elementwise rule."""
    torch.manual_seed(47)
    m = DSQGAttentionQW(256, 8, seq_len=4096, dropout=0.0, offsets=OFFSETS_J47)
    _perturb(m)
    with torch.no_grad():
        m.scale_embed.mul_(0.1)  # ~0.05 N(0,1), as the reference's tests draw it
    _module_parity(gpu_device, m, torch.bfloat16, 2, 4096, "module QW J47 bf16 E256 H8 B2 N4096")


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_module_kv_inject(gpu_device, dtype):
    """Huygens K/V injection (k + k_delta, v + v_delta, q unchanged): output and the gradients
    of x, both deltas and every parameter against the reference forward through the oracle.
    The deltas' gradients come back as the K / V slices of d(qkv).  Tolerances as in
    test_module_forward_backward_matches_oracle."""
    torch.manual_seed(12)
    E, H, B, N = 256, 4, 2, 300
    m = DSQGAttentionQW(E, H, dropout=0.0)
    _perturb(m)
    _module_parity(gpu_device, m, dtype, B, N, f"module kv_inject {str(dtype)[6:]}", kv=True)


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
