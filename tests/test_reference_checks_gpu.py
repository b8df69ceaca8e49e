"""The reference's own correctness checks, replayed on the HIP path.

* ``run_tests`` of kernels/dsqg_attention_v3.py:568-632: seed 42, q/k/v ~ 0.1 N(0,1) drawn in
  bf16, pos_bias ~ 0.5 N(0,1), scale_embed ~ 0.05 N(0,1), upstream gradient of ``out.sum()``
  (all ones); shapes (1,8,64,32), (2,8,512,32), (4,8,2047,32).  The reference passes at 0.05
  absolute; here the stated elementwise bound (tests/tolerance.py) applies as well.  Inputs are
  drawn on the CPU (the reference draws them on its GPU, whose generator differs).
* ``check_numerical`` of tools/check_kernel.py:346-455: forward max diff < 0.01, backward
  cosine > 0.99 and max diff < 0.05 for every gradient, finite outputs; shapes (1,4,64,32),
  (2,8,128,32).
* ``check_softmax_sanity`` of tools/check_kernel.py:462-526: the weights of every row sum to 1.
  On the kernel this is v = 1 everywhere, so out_n = sum_j alpha_j.
* The causality guard of train/train_2048_condU.py:490-506, at the operator: perturbing k and
  v at row t changes exactly the rows t + delta_j, every other output row is bit-identical;
  perturbing the upstream gradient at row t changes dq only at t and dk/dv only at t - delta_j.
"""

import pytest
import torch

import dwarf_amd
from dwarf_amd import ops
from dwarf_amd.offsets import OFFSETS_J47, OFFSETS_V3
from oracle import dsqg_forward, dsqg_forward_backward
from tests import tolerance

pytestmark = pytest.mark.gpu


def _say(msg):
    print(f"[refcheck] {msg}", flush=True)


def _reference_inputs(B, H, N, D, seed=42):
    """run_tests / check_numerical inputs: bf16 draws scaled by 0.1 in bf16, fp32 parameters."""
    torch.manual_seed(seed)
    q = torch.randn(B, H, N, D, dtype=torch.bfloat16) * 0.1
    k = torch.randn(B, H, N, D, dtype=torch.bfloat16) * 0.1
    v = torch.randn(B, H, N, D, dtype=torch.bfloat16) * 0.1
    pb = torch.randn(44, H, dtype=torch.float32) * 0.5
    se = torch.randn(44, D, dtype=torch.float32) * 0.05
    return q, k, v, pb, se


def _api_grads(q, k, v, pb, se, dev):
    """out and the gradients of out.sum() through the public dsqg_attention_v3."""
    qd, kd, vd, sed = (t.to(dev).requires_grad_(True) for t in (q, k, v, se))
    out = dwarf_amd.dsqg_attention_v3(qd, kd, vd, pb.to(dev), sed)
    out.float().sum().backward()
    torch.cuda.synchronize(dev)
    return {"out": out.detach().cpu(), "dq": qd.grad.cpu(), "dk": kd.grad.cpu(),
            "dv": vd.grad.cpu(), "dscale_embed": sed.grad.cpu()}


@pytest.mark.parametrize("shape", [(1, 8, 64, 32), (2, 8, 512, 32), (4, 8, 2047, 32)])
def test_run_tests_cases(gpu_device, shape):
    B, H, N, D = shape
    q, k, v, pb, se = _reference_inputs(B, H, N, D)
    got = _api_grads(q, k, v, pb, se, gpu_device)
    ref = dsqg_forward_backward(q, k, v, pb, torch.ones(B, H, N, D), se, dtype=torch.float32)
    errs = {}
    for key in got:
        errs[key] = tolerance.check(key, got[key], ref[key], "bf16", say=_say)
    tolerance.record(f"run_tests {shape}", errs)
    # The reference's own criterion (kernels/dsqg_attention_v3.py:607): every max diff < 0.05.
    assert max(e for e, _ in errs.values()) < 0.05


@pytest.mark.parametrize("shape", [(1, 4, 64, 32), (2, 8, 128, 32)])
def test_check_kernel_numerical(gpu_device, shape):
    B, H, N, D = shape
    q, k, v, pb, se = _reference_inputs(B, H, N, D)
    got = _api_grads(q, k, v, pb, se, gpu_device)
    ref = dsqg_forward_backward(q, k, v, pb, torch.ones(B, H, N, D), se, dtype=torch.float32)
    fwd = (got["out"].float() - ref["out"]).abs().max().item()
    assert fwd < 0.01, f"forward max diff {fwd:.4f}"
    for key in ("dq", "dk", "dv", "dscale_embed"):
        a, b = got[key].flatten().double(), ref[key].flatten().double()
        cos = (a @ b / (a.norm() * b.norm() + 1e-12)).item()
        diff = (a - b).abs().max().item()
        _say(f"{shape} {key}: cosine {cos:.6f}, max diff {diff:.3e}")
        assert cos > 0.99 and diff < 0.05, key
        assert torch.isfinite(got[key]).all(), key
    assert torch.isfinite(got["out"]).all()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("offsets", [OFFSETS_V3, OFFSETS_J47])
def test_softmax_weights_sum_to_one(gpu_device, dtype, offsets):
    """tools/check_kernel.py:462-526 on the kernel: with v = 1 the output row is the sum of
    its weights.  Sequence length max(256, max delta + 10), as there."""
    J, maxd = len(offsets), max(offsets)
    B, H, N, D = 1, 4, max(256, maxd + 10), 32
    torch.manual_seed(42)
    q = torch.randn(B, H, N, D) * 0.1
    k = torch.randn(B, H, N, D) * 0.1
    pb = torch.randn(J, H) * 0.5
    se = torch.randn(J, D) * 0.05
    v = torch.ones(B, H, N, D)
    dev = gpu_device
    out, lse, _ = ops.dsqg_fwd(q.to(dtype).to(dev), k.to(dtype).to(dev), v.to(dtype).to(dev),
                               pb.to(dev), se.to(dev), None, None, list(offsets))
    out = out.float().cpu()
    lo, hi = out.min().item(), out.max().item()
    _say(f"{dtype} J={J}: weight sums in [{lo:.6f}, {hi:.6f}]")
    assert lo > 0.99 and hi < 1.01 and torch.isfinite(out).all()
    if dtype == torch.float32:
        assert (out - 1).abs().max().item() <= 1e-6
    _, ref_lse = dsqg_forward(q.to(dtype).double(), k.to(dtype).double(), v.double(), pb.double(),
                              se.double(), offsets, return_lse=True)
    tolerance.check("lse", lse.cpu(), ref_lse, "fp32" if dtype == torch.float32 else "bf16", say=_say)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("t", [10, 700, 1000])
def test_causality_perturbation(gpu_device, dtype, t):
    B, H, N, D = 1, 2, 2600, 64
    g = torch.Generator().manual_seed(t)
    q, k, v, dout = (torch.randn(B, H, N, D, generator=g).to(dtype) for _ in range(4))
    pb = torch.randn(44, H, generator=g) * 0.5
    se = torch.randn(44, D, generator=g) * 0.05
    dev = gpu_device
    d = {n: x.to(dev) for n, x in (("q", q), ("k", k), ("v", v), ("dout", dout), ("pb", pb), ("se", se))}

    def run(kk, vv, dd):
        out, lse, alr = ops.dsqg_fwd(d["q"], kk, vv, d["pb"], d["se"], None, None, list(OFFSETS_V3))
        dq, dk, dv, *_ = ops.dsqg_bwd(d["q"], kk, vv, dd, lse, alr, d["pb"], d["se"], None, None,
                                      list(OFFSETS_V3), True, False, False)
        torch.cuda.synchronize(dev)
        return out.cpu(), dq.cpu(), dk.cpu(), dv.cpu()

    base = run(d["k"], d["v"], d["dout"])
    # Forward: k and v at row t perturbed -> only rows t + delta_j may change.
    k2, v2 = d["k"].clone(), d["v"].clone()
    k2[:, :, t] += 1.0
    v2[:, :, t] -= 1.0
    pert = run(k2, v2, d["dout"])
    hit = sorted({t + dl for dl in OFFSETS_V3 if t + dl < N})
    rows = torch.zeros(N, dtype=torch.bool)
    rows[hit] = True
    diff = (pert[0] != base[0]).any(-1).any(0).any(0)  # [N]: row changed
    assert not diff[~rows].any(), f"rows outside t+delta changed: {torch.nonzero(diff & ~rows)[:5].flatten().tolist()}"
    assert diff[rows].all(), "a row t+delta_j did not change"
    # Backward: the upstream gradient at row t perturbed -> dq changes only at t,
    # dk / dv only at rows t - delta_j.
    d2 = d["dout"].clone()
    d2[:, :, t] += 1.0
    pb_ = run(d["k"], d["v"], d2)
    back = torch.zeros(N, dtype=torch.bool)
    back[[t - dl for dl in OFFSETS_V3 if t - dl >= 0]] = True
    dq_rows = (pb_[1] != base[1]).any(-1).any(0).any(0)
    dk_rows = (pb_[2] != base[2]).any(-1).any(0).any(0)
    dv_rows = (pb_[3] != base[3]).any(-1).any(0).any(0)
    assert dq_rows.nonzero().flatten().tolist() == [t]
    assert not dk_rows[~back].any() and not dv_rows[~back].any()
    assert dv_rows[back].all()
    _say(f"t={t} {dtype}: {len(hit)} forward rows, {int(back.sum())} backward rows, rest bit-identical")
