"""Parity bounds shared by the GPU tests of the DSQG kernels.

* fp32 kernels against the float64 oracle: max|x - ref| <= 1e-5 * max|ref| over the tensor
  (the stated 1e-5 relative tolerance, relative to the tensor's scale).
* bf16 kernels against the fp32 oracle fed the same bf16-rounded inputs, elementwise:
    - tensors the kernels store in bf16 (out, dq, dk, dv, the decode output):
          |x - ref| <= 2e-2 + 2^-9 |ref|
      i.e. the stated 2e-2 absolute tolerance plus half an ulp of the stored bf16 value (the
      rounding of the store itself);
    - tensors the kernels store in fp32 (lse, dpos_bias, dscale_embed, dscore_gain,
      dif_gain): |x - ref| <= 2e-2.

* bf16 module runs (tests/test_modules.py), elementwise: the op-level rule plus the effect of the
  module's own bf16 intermediates (check_module).

``record`` keeps one line per checked case; ``tests/conftest.py`` prints them at the end of the
session, so the per-tensor errors appear in the tail of a ``pytest -q`` run.
"""

from __future__ import annotations

import torch

BF16_STORED = frozenset({"out", "dq", "dk", "dv", "decode"})
ABS_TOL = 2e-2
HALF_ULP = 2.0 ** -9
FP32_REL = 1e-5

SUMMARY: list[str] = []


def _base(name: str) -> str:
    return name.split("(")[0].split(" ")[0]


def elementwise_ratio(name: str, got: torch.Tensor, ref: torch.Tensor):
    """(max abs error, max over elements of error / bound) for a bf16 run."""
    got, ref = got.double(), ref.double()
    if ref.numel() == 0:
        return 0.0, 0.0
    err = (got - ref).abs()
    if _base(name) in BF16_STORED:
        bound = ABS_TOL + HALF_ULP * ref.abs()
    else:
        bound = torch.full_like(ref, ABS_TOL)
    return err.max().item(), (err / bound).max().item()


def check(name: str, got: torch.Tensor, ref: torch.Tensor, mode: str, say=print):
    """Asserts the bound for `mode` ("fp32" or "bf16"); returns (max error, ratio to bound)."""
    assert got.shape == ref.shape, f"{name}: shape {tuple(got.shape)} vs {tuple(ref.shape)}"
    got_d, ref_d = got.double(), ref.double()
    assert torch.isfinite(got_d).all(), f"{name}: non-finite values"
    if mode == "fp32":
        err = (got_d - ref_d).abs().max().item() if ref.numel() else 0.0
        scale = ref_d.abs().max().item() if ref.numel() else 0.0
        bound = FP32_REL * scale
        ratio = err / bound if bound > 0 else (0.0 if err == 0 else float("inf"))
        say(f"{name}: max err {err:.3e} (bound {bound:.3e}, ratio {ratio:.2f})")
        assert err <= bound, f"{name}: max err {err:.3e} > {bound:.3e}"
        return err, ratio
    err, ratio = elementwise_ratio(name, got_d, ref_d)
    kind = "2e-2+2^-9|ref|" if _base(name) in BF16_STORED else "2e-2"
    say(f"{name}: max err {err:.3e} (elementwise bound {kind}, worst ratio {ratio:.2f})")
    assert ratio <= 1.0, f"{name}: error {err:.3e} exceeds the elementwise bound (ratio {ratio:.2f})"
    return err, ratio


def check_module(name: str, got: torch.Tensor, ref: torch.Tensor, ref_rounded: torch.Tensor,
                 mag=None, say=print):
    """Elementwise bound for a tensor of a bf16 module run (every tensor of it is stored in bf16):

        |x - ref| <= 2e-2 + 2^-9 |ref| + 2 |ref_rounded - ref| + 2^-8 mag

    ref is the module's computation in fp32 on the module's own (bf16) parameters and input;
    ref_rounded is the same computation rounded to bf16 at each point where the module stores a
    bf16 tensor (projection outputs, the attention output, the gate, the gated product, the
    output, and the gradients through them).  2 |ref_rounded - ref| is the effect of those
    roundings on this input, doubled because the module's own rounding falls on slightly
    different pre-rounding values.  For a tensor that a projection GEMM A B yields, mag is
    |A| |B| from the fp32 reference, and 2^-8 mag the first-order bound of rounding both of its
    inputs to bf16 (2^-9 relative each): over a sum of many tokens the measured spread of one
    element can fall far below that by chance.  The first two terms are the op-level bf16 rule.
    Returns (max error, worst ratio to the bound)."""
    assert got.shape == ref.shape, f"{name}: shape {tuple(got.shape)} vs {tuple(ref.shape)}"
    got_d, ref_d, rr_d = got.double(), ref.double(), ref_rounded.double()
    assert torch.isfinite(got_d).all(), f"{name}: non-finite values"
    if ref.numel() == 0:
        return 0.0, 0.0
    err = (got_d - ref_d).abs()
    bound = ABS_TOL + HALF_ULP * ref_d.abs() + 2.0 * (rr_d - ref_d).abs()
    if mag is not None:
        bound = bound + 2.0 ** -8 * mag.double()
    e, ratio = err.max().item(), (err / bound).max().item()
    say(f"{name}: max err {e:.3e} (elementwise bound 2e-2+2^-9|ref|+2|rounding spread|, "
        f"worst ratio {ratio:.2f}, largest spread {(rr_d - ref_d).abs().max().item():.2e})")
    assert ratio <= 1.0, f"{name}: error {e:.3e} exceeds the elementwise bound (ratio {ratio:.2f})"
    return e, ratio


def record(case: str, errs: dict):
    """One summary line: case name and each tensor's max error (and ratio to its bound)."""
    parts = [f"{k} {e:.2e}/{r:.2f}" for k, (e, r) in errs.items()]
    SUMMARY.append(f"{case}: " + ", ".join(parts))
