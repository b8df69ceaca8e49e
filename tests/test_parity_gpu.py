"""GPU parity: the HIP kernels (through the C ABI) against the CPU oracle on the same inputs.

Tolerances (tests/tolerance.py, checked per tensor):
  * fp32 kernels vs the float64 oracle:  max|x - ref| <= 1e-5 * max|ref|.
  * bf16 kernels vs the fp32 oracle fed the same bf16-rounded inputs, elementwise:
        tensors stored in bf16 (out, dq, dk, dv):  |x - ref| <= 2e-2 + 2^-9 |ref|
        tensors stored in fp32 (lse and the parameter gradients):  |x - ref| <= 2e-2
    (2e-2 absolute, plus half an ulp of the stored value for the bf16 stores).
Masking (n - delta < 0) is exercised at every N below max(delta) and by rows 0..1535 of the
full-size configs.
"""

import pytest
import torch

import dwarf_amd
from dwarf_amd import ops
from dwarf_amd.offsets import OFFSETS_J46, OFFSETS_J47, OFFSETS_V3
from dwarf_amd.workloads import WORKLOADS, make_inputs
from oracle import dsqg_forward, dsqg_forward_backward
from tests import tolerance

pytestmark = pytest.mark.gpu


def _say(msg):
    print(f"[parity] {msg}", flush=True)


def oracle_chunked(inp, offsets, dtype, backward=True):
    """Oracle over batch chunks (elementwise identical to one call; parameter grads summed)."""
    B = inp["q"].shape[0]
    outs = {}
    for b in range(B):
        sl = {k: (v[b:b + 1] if k in ("q", "k", "v", "dout") else v) for k, v in inp.items()}
        if backward:
            r = dsqg_forward_backward(sl["q"], sl["k"], sl["v"], sl["pos_bias"], sl["dout"],
                                      sl.get("scale_embed"), offsets, sl.get("score_gain"),
                                      sl.get("if_gain"), dtype=dtype)
        else:
            o, l = dsqg_forward(*(None if t is None else t.to(dtype) for t in
                                  (sl["q"], sl["k"], sl["v"], sl["pos_bias"], sl.get("scale_embed"))),
                                offsets=offsets,
                                score_gain=None if sl.get("score_gain") is None else sl["score_gain"].to(dtype),
                                if_gain=None if sl.get("if_gain") is None else sl["if_gain"].to(dtype),
                                return_lse=True)
            r = {"out": o, "lse": l}
        for key, val in r.items():
            if key in ("out", "lse", "dq", "dk", "dv"):
                outs.setdefault(key, []).append(val)
            else:
                outs[key] = outs[key] + val if key in outs else val
    return {k: (torch.cat(v, 0) if isinstance(v, list) else v) for k, v in outs.items()}


def gpu_run(inp, offsets, dev, backward=True):
    d = {k: (None if v is None else v.to(dev)) for k, v in inp.items()}
    out, lse, alr = ops.dsqg_fwd(d["q"], d["k"], d["v"], d["pos_bias"], d.get("scale_embed"),
                                 d.get("score_gain"), d.get("if_gain"), list(offsets))
    res = {"out": out, "lse": lse}
    if backward:
        dq, dk, dv, dpb, dse, dg, da = ops.dsqg_bwd(
            d["q"], d["k"], d["v"], d["dout"], lse, alr, d["pos_bias"], d.get("scale_embed"),
            d.get("score_gain"), d.get("if_gain"), list(offsets),
            d.get("scale_embed") is not None, d.get("score_gain") is not None,
            d.get("if_gain") is not None)
        res.update(dq=dq, dk=dk, dv=dv, dpos_bias=dpb)
        if d.get("scale_embed") is not None:
            res["dscale_embed"] = dse
        if d.get("score_gain") is not None:
            res["dscore_gain"] = dg
        if d.get("if_gain") is not None:
            res["dif_gain"] = da
    torch.cuda.synchronize(dev)
    return {k: v.cpu() for k, v in res.items()}


def check(name, got, ref, mode):
    return tolerance.check(name, got, ref, mode, say=_say)


def compare(got, ref, mode, keys=None, case=None):
    errs = {}
    for key in keys or ref.keys():
        if key in got:
            errs[key] = check(key, got[key], ref[key], mode)
    if case:
        tolerance.record(case, errs)
    return errs


def _rand_inputs(B, H, N, D, offsets, dtype, seed, se=True, gains=True):
    g = torch.Generator().manual_seed(seed)
    J = len(offsets)
    shp = (B, H, N, D)
    inp = dict(q=torch.randn(shp, generator=g), k=torch.randn(shp, generator=g),
               v=torch.randn(shp, generator=g), dout=torch.randn(shp, generator=g),
               pos_bias=torch.randn(J, H, generator=g) * 0.5,
               scale_embed=torch.randn(J, D, generator=g) * 0.1 if se else None,
               score_gain=torch.rand(H, J, generator=g) + 0.5 if gains else None,
               if_gain=torch.rand(H, generator=g) * 0.4 + 0.8 if gains else None)
    for k in ("q", "k", "v", "dout"):
        inp[k] = inp[k].to(dtype)
    return inp


# ---------------------------------------------------------------------------------------------
# Workload configurations
# ---------------------------------------------------------------------------------------------

def test_config0_fp32_forward(gpu_device):
    w = WORKLOADS[0]
    inp = make_inputs(w)
    _say("config 0 fp32 forward B1 H8 N2048 D32")
    got = gpu_run(inp, w.offsets, gpu_device, backward=False)
    ref = oracle_chunked(inp, w.offsets, torch.float64, backward=False)
    compare(got, ref, "fp32")


@pytest.mark.parametrize("D", [32, 64, 80, 96, 128])
def test_fp32_fwd_bwd_all_parameters(gpu_device, D):
    inp = _rand_inputs(2, 3, 1700, D, OFFSETS_V3, torch.float32, seed=100 + D)
    _say(f"fp32 fwd+bwd B2 H3 N1700 D{D} with se, g, a")
    got = gpu_run(inp, OFFSETS_V3, gpu_device)
    ref = oracle_chunked(inp, OFFSETS_V3, torch.float64)
    compare(got, ref, "fp32")


@pytest.mark.parametrize("cfg", [1, 2, 3])
def test_bf16_workload_fwd_bwd(gpu_device, cfg):
    w = WORKLOADS[cfg]
    inp = make_inputs(w)
    _say(f"config {cfg} bf16 fwd+bwd B{w.B} H{w.H} N{w.N} D{w.D} J{w.J}")
    got = gpu_run(inp, w.offsets, gpu_device)
    ref = oracle_chunked(inp, w.offsets, torch.float32)
    compare(got, ref, "bf16", case=f"config {cfg}")
    # sum_j dbias[j,h] = 0 (each row's dS sums to zero over its taps)
    assert got["dpos_bias"].sum(0).abs().max().item() <= 1e-3 * max(1.0, got["dpos_bias"].abs().max().item())


@pytest.mark.parametrize("cfg", [1, 2])
def test_bf16_workload_with_scale_embed(gpu_device, cfg):
    """Configs 1 and 2 at full size with scale_embed ~ 0.05 N(0,1): every reference caller
    passes scale_embed (train/train_2048_condU.py:184), which selects the q.se kernels."""
    w = WORKLOADS[cfg]
    inp = make_inputs(w)
    g = torch.Generator().manual_seed(7000 + cfg)
    inp["scale_embed"] = torch.randn(w.J, w.D, generator=g) * 0.05
    _say(f"config {cfg} + scale_embed bf16 fwd+bwd B{w.B} H{w.H} N{w.N} D{w.D}")
    got = gpu_run(inp, w.offsets, gpu_device)
    ref = oracle_chunked(inp, w.offsets, torch.float32)
    compare(got, ref, "bf16", case=f"config {cfg} + scale_embed")


# ---------------------------------------------------------------------------------------------
# Edge cases
# ---------------------------------------------------------------------------------------------

@pytest.mark.parametrize("N", [1, 2, 31, 33, 47, 49, 65, 129, 257, 1535, 1537, 2047])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_ragged_sequence_lengths(gpu_device, N, dtype):
    inp = _rand_inputs(1, 2, N, 64, OFFSETS_V3, dtype, seed=N)
    _say(f"ragged N={N} {dtype}")
    got = gpu_run(inp, OFFSETS_V3, gpu_device)
    ref = oracle_chunked(inp, OFFSETS_V3, torch.float64 if dtype == torch.float32 else torch.float32)
    compare(got, ref, "fp32" if dtype == torch.float32 else "bf16")


@pytest.mark.parametrize("offsets,N", [(OFFSETS_J47, 4097), (OFFSETS_J46, 3100),
                                       ((0, 1, 2, 5, 9, 100), 300), ((0,), 40),
                                       (tuple(range(48)), 200)])
def test_other_offset_tables(gpu_device, offsets, N):
    inp = _rand_inputs(1, 2, N, 32, offsets, torch.float32, seed=len(offsets))
    _say(f"offsets J={len(offsets)} N={N}")
    got = gpu_run(inp, offsets, gpu_device)
    ref = oracle_chunked(inp, offsets, torch.float64)
    compare(got, ref, "fp32")


@pytest.mark.parametrize("offsets,N", [(OFFSETS_J47, 4097), ((0, 1, 2, 5, 9, 100), 300), ((0,), 40),
                                       ((0, 1, 2) + tuple(range(40, 40 + 16 * 37, 37)), 700)])
def test_other_offset_tables_bf16(gpu_device, offsets, N):
    """bf16 over other tables (the last one has the MFMA kernels' maximum of 16 long-range
    taps, at offsets that are not multiples of 16)."""
    inp = _rand_inputs(1, 3, N, 64, offsets, torch.bfloat16, seed=len(offsets) + 1)
    _say(f"bf16 offsets J={len(offsets)} N={N}")
    got = gpu_run(inp, offsets, gpu_device)
    ref = oracle_chunked(inp, offsets, torch.float32)
    compare(got, ref, "bf16")


@pytest.mark.parametrize("D", [80, 96, 128])
@pytest.mark.parametrize("offsets,N", [(OFFSETS_J47, 2100), (OFFSETS_J46, 1800),
                                       ((0, 1, 2) + tuple(range(40, 40 + 16 * 37, 37)), 700)])
def test_other_offset_tables_wide_heads(gpu_device, D, offsets, N):
    """bf16 with scale_embed, score gain and IF gain over the 47- and 46-offset tables (the
    kernels specialised for 14 and 13 long-range taps) and a 16-tap table (the generic kernels)
    at the head dims above 64, whose forward loads its long-range key rows in three bursts and
    whose kernels keep two long-range taps in flight."""
    inp = _rand_inputs(1, 2, N, D, offsets, torch.bfloat16, seed=len(offsets) + D)
    _say(f"bf16 offsets J={len(offsets)} N={N} D={D} with se, g, a")
    got = gpu_run(inp, offsets, gpu_device)
    ref = oracle_chunked(inp, offsets, torch.float32)
    compare(got, ref, "bf16", case=f"J={len(offsets)} D={D} + se, g, a")


@pytest.mark.parametrize("gains", [True, False])
@pytest.mark.parametrize("D", [32, 64, 80, 96, 128])
@pytest.mark.parametrize("offsets", [OFFSETS_V3, OFFSETS_J47], ids=["J44", "J47"])
def test_heads_without_scale_embed(gpu_device, D, offsets, gains):
    """bf16 without scale_embed at every head dim (the plain kernels, which the headline and the
    D = 96 bench leg run), with the score and IF gains (dq's score-gain gradient forms for 11
    and 14 long-range taps) and without them.  At D = 80 and 96 a row is four lanes of three
    16-byte pieces, so each long-range row sum adds three partials in the lane before the
    lanes'."""
    inp = _rand_inputs(2, 3, 1300, D, offsets, torch.bfloat16, seed=500 + D + len(offsets),
                       se=False, gains=gains)
    _say(f"bf16 B2 H3 N1300 D{D} J{len(offsets)} no se, gains={gains}")
    got = gpu_run(inp, offsets, gpu_device)
    ref = oracle_chunked(inp, offsets, torch.float32)
    compare(got, ref, "bf16", case=f"D={D} J={len(offsets)} no se, gains={gains}")


@pytest.mark.parametrize("D", [32, 64])
@pytest.mark.parametrize("offsets", [OFFSETS_J46, OFFSETS_J47], ids=["J46", "J47"])
def test_score_gain_gradient_with_scale_embed(gpu_device, D, offsets):
    """scale_embed with both gains over the 46- and 47-offset tables at D = 32 and 64: dq's
    score-gain gradient forms with scale_embed for 13 and 14 long-range taps (two batches, so
    a batch group sums two slices)."""
    inp = _rand_inputs(2, 3, 1100, D, offsets, torch.bfloat16, seed=700 + D + len(offsets))
    _say(f"bf16 B2 H3 N1100 D{D} J{len(offsets)} with se, g, a")
    got = gpu_run(inp, offsets, gpu_device)
    ref = oracle_chunked(inp, offsets, torch.float32)
    compare(got, ref, "bf16", case=f"D={D} J={len(offsets)} + se, g, a")


@pytest.mark.parametrize("gains", [True, False])
@pytest.mark.parametrize("B", [3, 5, 6])
def test_scale_embed_batch_groups(gpu_device, B, gains):
    """With scale_embed the dq workgroup takes one head and tile in four batches and sums its
    parameter partials over them; batch counts that leave a short last group (or one group of
    three) against the oracle, with the score gain's gradient (the generic dq) and without it
    (the 11-tap dq of the reference modules' call)."""
    inp = _rand_inputs(B, 3, 700, 64, OFFSETS_V3, torch.bfloat16, seed=300 + B, gains=gains)
    _say(f"bf16 B{B} H3 N700 D64 with se, gains={gains} (batch groups)")
    got = gpu_run(inp, OFFSETS_V3, gpu_device)
    ref = oracle_chunked(inp, OFFSETS_V3, torch.float32)
    compare(got, ref, "bf16", case=f"B={B} batch groups + se, gains={gains}")


def test_long_sequence(gpu_device):
    """A sequence of 100,003 tokens (ragged: the last tile holds 35 rows), bf16 with scale_embed
    and the IF gain: row offsets far beyond the workloads' (N * row bytes = 12.8 MB per slice),
    every tap valid for almost all rows."""
    N = 100_003
    inp = _rand_inputs(1, 2, N, 64, OFFSETS_V3, torch.bfloat16, seed=N, gains=False)
    inp["if_gain"] = torch.tensor([0.9, 1.1])
    _say(f"bf16 long sequence N={N}")
    got = gpu_run(inp, OFFSETS_V3, gpu_device)
    ref = oracle_chunked(inp, OFFSETS_V3, torch.float32)
    compare(got, ref, "bf16", case=f"N={N} + scale_embed")


@pytest.mark.parametrize("offsets,N", [(OFFSETS_J46, 3100), (OFFSETS_J47, 4097)])
def test_long_tables_with_scale_embed(gpu_device, offsets, N):
    """The N=4096 trainers' call (train/train_4096_13m_condU.py:102-105): pos_bias and scale_embed
    over the 46- and 47-offset tables at D=64 with the IF gain and no score gain, which selects
    the scale_embed kernels for 13 and 14 long-range taps."""
    inp = _rand_inputs(1, 2, N, 64, offsets, torch.bfloat16, seed=len(offsets) + 7, gains=False)
    inp["if_gain"] = torch.rand(2, generator=torch.Generator().manual_seed(len(offsets))) * 0.4 + 0.8
    _say(f"bf16 offsets J={len(offsets)} N={N} + scale_embed")
    got = gpu_run(inp, offsets, gpu_device)
    ref = oracle_chunked(inp, offsets, torch.float32)
    compare(got, ref, "bf16", case=f"J={len(offsets)} + scale_embed")


@pytest.mark.parametrize("offsets", [OFFSETS_J47, OFFSETS_J46])
def test_n4096_trainer_shape_d32(gpu_device, offsets):
    """The N=4096 13M trainer's own call at full size: E 256 with H 8 gives HD 32
    (train/train_4096_13m_condU.py:51-54), batch 8 (:45), the 47-offset table (:89-93; the
    46-offset table of BASELINE config 3 alongside), dsqg_attention_backend(q, k, v, pos_bias,
    scale_embed) (:104-105, 157) with the module's IF gain after it.  bf16 B8 H8 N4096 D32
    selects the <32, true, 14> / <32, true, 13> kernels; scale_embed ~ 0.05 N(0,1),
    if_gain ~ U(0.8, 1.2)."""
    J = len(offsets)
    inp = _rand_inputs(8, 8, 4096, 32, offsets, torch.bfloat16, seed=4096 + J, gains=False)
    g = torch.Generator().manual_seed(40 + J)
    inp["scale_embed"] = torch.randn(J, 32, generator=g) * 0.05
    inp["if_gain"] = torch.rand(8, generator=g) * 0.4 + 0.8
    _say(f"N=4096 trainer shape B8 H8 N4096 D32 J{J} + scale_embed + IF gain")
    got = gpu_run(inp, offsets, gpu_device)
    ref = oracle_chunked(inp, offsets, torch.float32)
    compare(got, ref, "bf16", case=f"N=4096 trainer B8 H8 N4096 D32 J{J} + scale_embed + if_gain")


def test_bf16_table_beyond_the_mfma_kernels_is_rejected(gpu_device):
    """bf16 has one implementation: a table with more than 16 taps beyond the dense window
    (here 47) is refused with DSQG_EUNSUPPORTED before any launch; fp32 still takes it."""
    offsets = tuple(range(0, 96, 2))
    inp = _rand_inputs(1, 2, 200, 64, offsets, torch.bfloat16, seed=3)
    d = {k: (None if v is None else v.to(gpu_device)) for k, v in inp.items()}
    with pytest.raises(Exception, match="unsupported"):
        ops.dsqg_fwd(d["q"], d["k"], d["v"], d["pos_bias"], None, None, None, list(offsets))
    lse = torch.zeros(1, 2, 200, device=gpu_device)
    with pytest.raises(Exception, match="unsupported"):
        ops.dsqg_bwd(d["q"], d["k"], d["v"], d["dout"], lse, torch.zeros(1, 2, 15, 200, device=gpu_device),
                     d["pos_bias"], None, None, None,
                     list(offsets), False, False, False)
    f32 = {k: (v.float() if v is not None and v.is_floating_point() else v) for k, v in inp.items()}
    got = gpu_run(f32, offsets, gpu_device)
    ref = oracle_chunked(f32, offsets, torch.float64)
    compare(got, ref, "fp32")


@pytest.mark.parametrize("D", [32, 64, 80, 96, 128])
def test_bf16_head_dims_all_parameters(gpu_device, D):
    inp = _rand_inputs(2, 3, 1700, D, OFFSETS_V3, torch.bfloat16, seed=200 + D)
    _say(f"bf16 fwd+bwd B2 H3 N1700 D{D} with se, g, a")
    got = gpu_run(inp, OFFSETS_V3, gpu_device)
    ref = oracle_chunked(inp, OFFSETS_V3, torch.float32)
    compare(got, ref, "bf16")


def test_85m_condu_trainer_shape_d96(gpu_device):
    """train/train_2048_85m_condU.py:60-62 builds E 768 with H 8 (HD 96) and calls
    dsqg_attention_v3(q, k, v, pos_bias, scale_embed) (:112-115, 169): B8 H8 N2048 D96."""
    inp = _rand_inputs(8, 8, 2048, 96, OFFSETS_V3, torch.bfloat16, seed=96, gains=False)
    inp["scale_embed"] = inp["scale_embed"] * 0.5          # ~0.05 N(0,1), as the reference's tests
    _say("85M condU trainer shape B8 H8 N2048 D96 with scale_embed")
    got = gpu_run(inp, OFFSETS_V3, gpu_device)
    ref = oracle_chunked(inp, OFFSETS_V3, torch.float32)
    compare(got, ref, "bf16", case="85M condU B8 H8 N2048 D96 + scale_embed")


def test_v2_self_test_85m_shape_d80(gpu_device):
    """kernels/dsqg_attention_v2.py:508-513, "85M shape (HD=80)": (4, 8, 2047, 80), seed 42,
    q/k/v ~ 0.1 N(0,1) drawn in bf16, pos_bias ~ 0.5 N(0,1), no scale_embed, gradient of
    out.sum(); the reference passes at 0.05 absolute."""
    B, H, N, D = 4, 8, 2047, 80
    torch.manual_seed(42)
    q = torch.randn(B, H, N, D, dtype=torch.bfloat16) * 0.1
    k = torch.randn(B, H, N, D, dtype=torch.bfloat16) * 0.1
    v = torch.randn(B, H, N, D, dtype=torch.bfloat16) * 0.1
    pb = torch.randn(44, H, dtype=torch.float32) * 0.5
    dev = gpu_device
    qd, kd, vd = (t.to(dev).requires_grad_(True) for t in (q, k, v))
    out = dwarf_amd.dsqg_attention_v2(qd, kd, vd, pb.to(dev))
    out.float().sum().backward()
    torch.cuda.synchronize(dev)
    got = {"out": out.detach().cpu(), "dq": qd.grad.cpu(), "dk": kd.grad.cpu(), "dv": vd.grad.cpu()}
    ref = dsqg_forward_backward(q, k, v, pb, torch.ones(B, H, N, D), None, dtype=torch.float32)
    errs = compare(got, ref, "bf16", keys=("out", "dq", "dk", "dv"), case="V2 self-test (4, 8, 2047, 80)")
    assert max(e for e, _ in errs.values()) < 0.05


def test_empty_inputs(gpu_device):
    for shape in ((0, 2, 16, 64), (1, 2, 0, 64)):
        inp = _rand_inputs(*shape, OFFSETS_V3, torch.bfloat16, seed=1)
        got = gpu_run(inp, OFFSETS_V3, gpu_device)
        assert got["out"].shape == shape and got["dq"].shape == shape
        assert (got["dpos_bias"] == 0).all() and (got["dscale_embed"] == 0).all()


def test_strided_views_match_contiguous(gpu_device):
    """q/k/v as head-split views of one [B,N,3*H*D] projection (no permute copies)."""
    B, H, N, D = 2, 4, 600, 64
    g = torch.Generator().manual_seed(5)
    qkv = torch.randn(B, N, 3 * H * D, generator=g).to(torch.bfloat16).to(gpu_device)
    q, k, v = (t.view(B, N, H, D).permute(0, 2, 1, 3) for t in qkv.split(H * D, dim=-1))
    pb = (torch.randn(44, H, generator=g) * 0.5).to(gpu_device)
    se = (torch.randn(44, D, generator=g) * 0.1).to(gpu_device)
    o1, l1, a1 = ops.dsqg_fwd(q, k, v, pb, se, None, None, list(OFFSETS_V3))
    o2, l2, a2 = ops.dsqg_fwd(q.contiguous(), k.contiguous(), v.contiguous(), pb, se, None, None,
                          list(OFFSETS_V3))
    assert q.stride(2) == 3 * H * D
    assert torch.equal(o1, o2) and torch.equal(l1, l2) and torch.equal(a1, a2)


def test_misaligned_scale_embed_view_matches_aligned(gpu_device):
    """A scale_embed view 4 bytes past a 16-byte boundary is copied to aligned memory by the
    host layer (the kernels read it as 16-byte pieces): results equal the aligned call's."""
    inp = _rand_inputs(2, 4, 600, 64, OFFSETS_V3, torch.bfloat16, seed=13)
    d = {k: (None if v is None else v.to(gpu_device)) for k, v in inp.items()}
    J, D = d["scale_embed"].shape
    buf = torch.zeros(J * D + 1, device=gpu_device)
    se_view = buf[1:].view(J, D)
    se_view.copy_(d["scale_embed"])
    assert se_view.data_ptr() % 16 == 4 and se_view.is_contiguous()
    runs = []
    for se in (d["scale_embed"], se_view):
        out, lse, alr = ops.dsqg_fwd(d["q"], d["k"], d["v"], d["pos_bias"], se, d["score_gain"],
                                     d["if_gain"], list(OFFSETS_V3))
        grads = ops.dsqg_bwd(d["q"], d["k"], d["v"], d["dout"], lse, alr, d["pos_bias"], se,
                             d["score_gain"], d["if_gain"], list(OFFSETS_V3), True, True, True)
        runs.append((out, lse, alr) + tuple(grads))
    for a, b in zip(*runs):
        assert torch.equal(a, b)


@pytest.mark.parametrize("D", [32, 64, 96])
def test_backward_is_deterministic(gpu_device, D):
    """Two runs give the same bits (scale_embed and gains on): every LDS table entry has one
    writer, and the parameter partials are summed in a fixed order."""
    inp = _rand_inputs(4, 8, 2048, D, OFFSETS_V3, torch.bfloat16, seed=9)
    a = gpu_run(inp, OFFSETS_V3, gpu_device)
    b = gpu_run(inp, OFFSETS_V3, gpu_device)
    for key in a:
        assert torch.equal(a[key], b[key]), key


# ---------------------------------------------------------------------------------------------
# Public API (autograd, dtype rules, reference aliases)
# ---------------------------------------------------------------------------------------------

def test_autograd_api_matches_oracle(gpu_device):
    inp = _rand_inputs(2, 4, 700, 32, OFFSETS_V3, torch.bfloat16, seed=21, gains=False)
    d = {k: (None if v is None else v.to(gpu_device)) for k, v in inp.items()}
    q, k, v = (d[n].clone().requires_grad_(True) for n in ("q", "k", "v"))
    pb = d["pos_bias"].clone().requires_grad_(True)
    se = d["scale_embed"].clone().requires_grad_(True)
    out = dwarf_amd.dsqg_attention_v3(q, k, v, pb, se)
    out.backward(d["dout"])
    got = {"out": out.detach().cpu(), "dq": q.grad.cpu(), "dk": k.grad.cpu(), "dv": v.grad.cpu(),
           "dpos_bias": pb.grad.cpu(), "dscale_embed": se.grad.cpu()}
    ref = oracle_chunked(inp, OFFSETS_V3, torch.float32)
    compare(got, ref, "bf16")


def test_fp16_inputs_follow_reference_cast(gpu_device):
    inp = _rand_inputs(1, 2, 300, 64, OFFSETS_V3, torch.float16, seed=3, gains=False)
    d = {k: (None if v is None else v.to(gpu_device)) for k, v in inp.items()}
    out = dwarf_amd.dsqg_attention_v3(d["q"], d["k"], d["v"], d["pos_bias"], d["scale_embed"])
    assert out.dtype == torch.float16
    ref = dsqg_forward(inp["q"].bfloat16().float(), inp["k"].bfloat16().float(),
                       inp["v"].bfloat16().float(), inp["pos_bias"], inp["scale_embed"])
    check("out(fp16 via bf16)", out.float().cpu(), ref, "bf16")


def test_with_lse_follows_the_dtype_rules(gpu_device):
    """dsqg_attention_with_lse: fp16 inputs are computed in bf16 and out comes back as fp16,
    lse [B,H,N] fp32 matches the oracle's logsumexp; out is differentiable."""
    inp = _rand_inputs(1, 2, 300, 64, OFFSETS_V3, torch.float16, seed=5, gains=False)
    d = {k: (None if v is None else v.to(gpu_device)) for k, v in inp.items()}
    q = d["q"].clone().requires_grad_(True)
    out, lse = dwarf_amd.dsqg_attention_with_lse(q, d["k"], d["v"], d["pos_bias"], d["scale_embed"])
    assert out.dtype == torch.float16 and lse.dtype == torch.float32 and tuple(lse.shape) == (1, 2, 300)
    ref, ref_lse = dsqg_forward(inp["q"].bfloat16().float(), inp["k"].bfloat16().float(),
                                inp["v"].bfloat16().float(), inp["pos_bias"], inp["scale_embed"],
                                return_lse=True)
    check("out(with_lse)", out.float().cpu(), ref, "bf16")
    check("lse(with_lse)", lse.cpu(), ref_lse, "bf16")
    out.float().sum().backward()
    assert q.grad is not None and q.grad.dtype == torch.float16


def test_v3_with_zero_scale_embed_equals_v2(gpu_device):
    """kernels/dsqg_attention_v3.py:612-628: V3(SE=0) == V2."""
    inp = _rand_inputs(2, 8, 128, 32, OFFSETS_V3, torch.bfloat16, seed=7, se=False, gains=False)
    d = {k: (None if v is None else v.to(gpu_device)) for k, v in inp.items()}
    o2 = dwarf_amd.dsqg_attention_v2(d["q"], d["k"], d["v"], d["pos_bias"])
    o3 = dwarf_amd.dsqg_attention_v3(d["q"], d["k"], d["v"], d["pos_bias"],
                                     torch.zeros(44, 32, device=gpu_device))
    assert torch.equal(o2, o3)


def test_fp32_path_does_not_downcast(gpu_device):
    inp = _rand_inputs(1, 2, 200, 64, OFFSETS_V3, torch.float32, seed=4, gains=False)
    d = {k: (None if v is None else v.to(gpu_device)) for k, v in inp.items()}
    out = dwarf_amd.dsqg_attention_v3(d["q"], d["k"], d["v"], d["pos_bias"], d["scale_embed"])
    assert out.dtype == torch.float32
    ref = dsqg_forward(*(inp[n].double() for n in ("q", "k", "v", "pos_bias", "scale_embed")))
    check("out fp32", out.cpu(), ref, "fp32")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_qkv_entry_matches_split_heads(gpu_device, dtype):
    """dsqg_attention_qkv on a [B,N,3*H*D] projection output: the same output, and its one
    qkv gradient equals the three head gradients of dsqg_attention on the split views, bit
    for bit (same kernels, same inputs; only the gradient buffer differs)."""
    B, H, N, D = 2, 4, 333, 64
    g = torch.Generator().manual_seed(17)
    qkv0 = torch.randn(B, N, 3 * H * D, generator=g).to(dtype).to(gpu_device)
    pb0 = (torch.randn(44, H, generator=g) * 0.5).to(gpu_device)
    se0 = (torch.randn(44, D, generator=g) * 0.1).to(gpu_device)
    a0 = (0.8 + 0.4 * torch.rand(H, generator=g)).to(gpu_device)
    dy = torch.randn(B, H, N, D, generator=g).to(dtype).to(gpu_device)
    res = []
    for fused in (True, False):
        qkv, pb, se, a = (t.clone().requires_grad_(True) for t in (qkv0, pb0, se0, a0))
        if fused:
            out = dwarf_amd.dsqg_attention_qkv(qkv, H, pb, se, if_gain=a)
        else:
            out = dwarf_amd.dsqg_attention(*ops.split_qkv(qkv, H), pb, se, if_gain=a)
        out.backward(dy)
        res.append((out.detach(), qkv.grad, pb.grad, se.grad, a.grad))
    for name, x, y in zip(("out", "dqkv", "dpos_bias", "dscale_embed", "dif_gain"), *res):
        assert torch.equal(x, y), name
    # The head merge of the output is a view: [B,H,N,D] stored token-major.
    assert res[0][0].permute(0, 2, 1, 3).is_contiguous()


@pytest.mark.parametrize("dtype,D,se", [(torch.bfloat16, 64, False), (torch.bfloat16, 64, True),
                                         (torch.bfloat16, 32, True), (torch.float32, 64, True)])
def test_phase_by_phase_backward_equals_full(gpu_device, dtype, D, se):
    """dsqg_bwd_dq + dsqg_bwd_dkdv + dsqg_bwd_params give bit for bit what dsqg_bwd gives (the
    full backward runs the parameter reduction inside the dk/dv launch)."""
    inp = _rand_inputs(2, 3, 700, D, OFFSETS_V3, dtype, seed=31, se=se)
    d = {k: (None if v is None else v.to(gpu_device)) for k, v in inp.items()}
    fl = ops.FwdLaunch(d["q"], d["k"], d["v"], d["pos_bias"], d.get("scale_embed"),
                       d.get("score_gain"), d.get("if_gain"), list(OFFSETS_V3))
    fl.run()
    res = []
    for phased in (False, True):
        bl = ops.BwdLaunch(d["q"], d["k"], d["v"], d["dout"], fl.lse, d["pos_bias"],
                           d.get("scale_embed"), d.get("score_gain"), d.get("if_gain"),
                           list(OFFSETS_V3), se, True, True, alpha_lr=fl.alpha_lr)
        if phased:
            for phase in ("dq", "dkdv", "params"):
                bl.run(phase)
        else:
            bl.run()
        torch.cuda.synchronize(gpu_device)
        res.append([t.clone() for t in bl.outputs()])
    for name, x, y in zip(("dq", "dk", "dv", "dpos_bias", "dscale_embed", "dscore_gain",
                           "dif_gain"), *res):
        assert torch.equal(x, y), name
