"""GPU parity of the ring-buffer decode step (workload 4) against the CPU oracle.

Tolerance (tests/tolerance.py): bf16 outputs vs the fp32 oracle on the same bf16 inputs,
elementwise |x - ref| <= 2e-2 + 2^-9 |ref| (the output is stored in bf16); fp32 outputs vs the
float64 oracle, max|x - ref| <= 1e-5 * max|ref|.  Ring contents are compared bit for bit (the
step copies rows).
"""

import pytest
import torch

import dwarf_amd
from dwarf_amd import ops
from dwarf_amd.offsets import OFFSETS_J46, OFFSETS_J47, OFFSETS_V3
from dwarf_amd.workloads import DECODE, make_decode_inputs
from oracle import decode_step, dsqg_forward
from tests import tolerance

pytestmark = pytest.mark.gpu


def _say(msg):
    print(f"[decode] {msg}", flush=True)


def _err(got, ref):
    return (got.double() - ref.double()).abs().max().item(), ref.abs().max().item()


def _bf16_ratio(got, ref):
    """Worst ratio of the elementwise error to the bf16-stored bound (<= 1 passes)."""
    return tolerance.elementwise_ratio("decode", got, ref)[1]


def test_decode_workload_1000_steps(gpu_device):
    """Workload 4: B256 H12 D64, 1537-slot rings, positions from [1536, 8191], 1000 steps,
    every step checked against the oracle's gather over its own copy of the rings."""
    cfg = DECODE
    inp = make_decode_inputs()
    d = {k: v.to(gpu_device) for k, v in inp.items()}
    k_ring_ref, v_ring_ref = inp["k_ring"].clone(), inp["v_ring"].clone()
    pos = inp["pos"].clone()
    B, H, D = cfg["B"], cfg["H"], cfg["D"]
    g = torch.Generator().manual_seed(77)
    worst = 0.0
    steps = cfg["steps"]
    for step in range(steps):
        q, kn, vn = (torch.randn(B, H, D, generator=g).to(torch.bfloat16) for _ in range(3))
        out = ops.dsqg_decode(q.to(gpu_device), kn.to(gpu_device), vn.to(gpu_device),
                              d["k_ring"], d["v_ring"], pos.to(gpu_device), d["pos_bias"],
                              None, None, None, list(OFFSETS_V3)).cpu()
        ref = decode_step(q.float(), kn.float(), vn.float(), k_ring_ref, v_ring_ref, pos,
                          inp["pos_bias"])
        err, scale = _err(out, ref)
        ratio = _bf16_ratio(out, ref)
        worst = max(worst, err)
        assert ratio <= 1.0, f"step {step}: err {err:.3e} (ratio {ratio:.2f})"
        pos = pos + 1
        if step % 200 == 0:
            _say(f"step {step} err {err:.3e}")
    _say(f"{steps} steps, worst err {worst:.3e}")
    tolerance.SUMMARY.append(f"decode workload 4, {steps} steps: worst max err {worst:.2e}")
    assert torch.equal(d["k_ring"].cpu(), k_ring_ref)
    assert torch.equal(d["v_ring"].cpu(), v_ring_ref)


@pytest.mark.parametrize("D", [32, 64, 80, 96, 128])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("p", [0, 7, 40, 1535, 1536, 2500])
def test_decode_equals_full_sequence_row(gpu_device, dtype, p, D):
    """After prefilling the ring from a sequence of length p, the step at position p equals
    row p of the full-sequence forward (taps with p - delta < 0 are masked, not wrapped).
    Every head dim: the output's lane layout differs per D."""
    B, H = 3, 2
    g = torch.Generator().manual_seed(1000 + p + D)
    qs, ks, vs = (torch.randn(B, H, p + 1, D, generator=g).to(dtype) for _ in range(3))
    pb = torch.randn(44, H, generator=g) * 0.5
    se = torch.randn(44, D, generator=g) * 0.1
    sg = torch.rand(H, 44, generator=g) + 0.5
    a = torch.rand(H, generator=g) * 0.4 + 0.8
    cache = dwarf_amd.DSQGRingCache(B, H, D, OFFSETS_V3, dtype=dtype, device=gpu_device)
    # Slots no valid tap reads hold NaN: masked taps must not reach the output.
    cache.k_ring.fill_(float("nan"))
    cache.v_ring.fill_(float("nan"))
    if p > 0:
        cache.prefill(ks[:, :, :p].to(gpu_device), vs[:, :, :p].to(gpu_device))
    else:
        cache.pos.zero_()
    dev = {n: t.to(gpu_device) for n, t in (("pb", pb), ("se", se), ("sg", sg), ("a", a))}
    out = cache.step(qs[:, :, p].to(gpu_device), ks[:, :, p].to(gpu_device),
                     vs[:, :, p].to(gpu_device), dev["pb"], dev["se"], dev["sg"], dev["a"]).cpu()
    cd = torch.float64 if dtype == torch.float32 else torch.float32
    ref = dsqg_forward(qs.to(cd), ks.to(cd), vs.to(cd), pb.to(cd), se.to(cd), OFFSETS_V3,
                       sg.to(cd), a.to(cd))[:, :, p]
    err, scale = _err(out, ref)
    assert torch.isfinite(out).all()
    if dtype == torch.float32:
        _say(f"p={p} D={D} {dtype}: err {err:.3e} bound {1e-5 * scale:.3e}")
        assert err <= 1e-5 * scale
    else:
        ratio = _bf16_ratio(out, ref)
        _say(f"p={p} D={D} {dtype}: err {err:.3e} ratio {ratio:.2f}")
        assert ratio <= 1.0
    assert int(cache.pos[0]) == p + 1


def test_decode_pos_next_and_graph_replay(gpu_device):
    """A captured step with pos/pos_next ping-pong replays correctly several times in a row."""
    B, H, D, S = 8, 4, 64, 1537
    inp = make_decode_inputs(B=B, H=H, D=D, S=S, seed=5)
    d = {k: v.to(gpu_device) for k, v in inp.items()}
    k_ref, v_ref = inp["k_ring"].clone(), inp["v_ring"].clone()
    pos_a = d["pos"].clone()
    pos_b = torch.empty_like(pos_a)
    out = torch.empty_like(d["q"])
    offs = list(OFFSETS_V3)
    pb = d["pos_bias"]

    def step(src, dst):
        ops.decode_step_into(d["q"], d["k_new"], d["v_new"], d["k_ring"], d["v_ring"], src, pb,
                             None, None, None, offs, out, dst)

    s = torch.cuda.Stream(gpu_device)
    s.wait_stream(torch.cuda.current_stream(gpu_device))
    with torch.cuda.stream(s):       # warm-up outside the graph (also checks pos_next)
        step(pos_a, pos_b)
    torch.cuda.current_stream(gpu_device).wait_stream(s)
    torch.cuda.synchronize(gpu_device)
    pos = inp["pos"].clone()
    ref = decode_step(inp["q"].float(), inp["k_new"].float(), inp["v_new"].float(), k_ref, v_ref,
                      pos, inp["pos_bias"])
    assert torch.equal(pos_b.cpu(), pos + 1)
    assert _bf16_ratio(out.cpu(), ref) <= 1.0

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        step(pos_b, pos_a)
        step(pos_a, pos_b)
    for rep in range(3):
        graph.replay()
        torch.cuda.synchronize(gpu_device)
        for _ in range(2):
            pos = pos + 1
            ref = decode_step(inp["q"].float(), inp["k_new"].float(), inp["v_new"].float(), k_ref,
                              v_ref, pos, inp["pos_bias"])
        # the graph's second step is the last one; out holds its result
        err, scale = _err(out.cpu(), ref)
        _say(f"replay {rep}: err {err:.3e}")
        assert _bf16_ratio(out.cpu(), ref) <= 1.0
        assert torch.equal(pos_b.cpu(), pos + 1)
    assert torch.equal(d["k_ring"].cpu(), k_ref) and torch.equal(d["v_ring"].cpu(), v_ref)


@pytest.mark.parametrize("offsets,p", [(OFFSETS_J46, 3100), (OFFSETS_J47, 4095),
                                       ((0, 1, 2, 5, 9, 100), 150), ((0,), 3)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_decode_other_offset_tables(gpu_device, offsets, p, dtype):
    """The 46- and 47-offset tables (rings of 3073 and 4097 slots), a short irregular table and
    the lone delta = 0: the step equals row p of the full-sequence forward."""
    B, H, D = 2, 2, 64
    J = len(offsets)
    g = torch.Generator().manual_seed(p + J)
    qs, ks, vs = (torch.randn(B, H, p + 1, D, generator=g).to(dtype) for _ in range(3))
    pb = torch.randn(J, H, generator=g) * 0.5
    cache = dwarf_amd.DSQGRingCache(B, H, D, offsets, dtype=dtype, device=gpu_device)
    cache.k_ring.fill_(float("nan"))
    cache.v_ring.fill_(float("nan"))
    cache.prefill(ks[:, :, :p].to(gpu_device), vs[:, :, :p].to(gpu_device))
    out = cache.step(qs[:, :, p].to(gpu_device), ks[:, :, p].to(gpu_device),
                     vs[:, :, p].to(gpu_device), pb.to(gpu_device)).cpu()
    cd = torch.float64 if dtype == torch.float32 else torch.float32
    ref = dsqg_forward(qs.to(cd), ks.to(cd), vs.to(cd), pb.to(cd), None, list(offsets))[:, :, p]
    err, scale = _err(out, ref)
    _say(f"J={J} p={p} {dtype}: err {err:.3e}")
    assert torch.isfinite(out).all()
    if dtype == torch.float32:
        assert err <= 1e-5 * scale
    else:
        assert _bf16_ratio(out, ref) <= 1.0


def test_decode_positions_beyond_32_bits(gpu_device):
    """Positions at and past 2^31 (the kernel takes p mod S in 64-bit arithmetic there) next to
    an ordinary one: output and ring writes equal the oracle's step, three steps in a row."""
    B, H, D, S = 4, 2, 64, 1537
    inp = make_decode_inputs(B=B, H=H, D=D, S=S, seed=23)
    d = {k: v.to(gpu_device) for k, v in inp.items()}
    k_ref, v_ref = inp["k_ring"].clone(), inp["v_ring"].clone()
    pos = torch.tensor([2 ** 31 - 2, 2 ** 31 + 5, 3_000_000_000_123, 1536], dtype=torch.int64)
    g = torch.Generator().manual_seed(5)
    for step in range(3):
        q, kn, vn = (torch.randn(B, H, D, generator=g).to(torch.bfloat16) for _ in range(3))
        out = ops.dsqg_decode(q.to(gpu_device), kn.to(gpu_device), vn.to(gpu_device),
                              d["k_ring"], d["v_ring"], pos.to(gpu_device), d["pos_bias"],
                              None, None, None, list(OFFSETS_V3)).cpu()
        ref = decode_step(q.float(), kn.float(), vn.float(), k_ref, v_ref, pos, inp["pos_bias"])
        _say(f"step {step} positions {pos.tolist()}: err {_err(out, ref)[0]:.3e}")
        assert _bf16_ratio(out, ref) <= 1.0
        assert torch.equal(d["k_ring"].cpu(), k_ref) and torch.equal(d["v_ring"].cpu(), v_ref)
        pos = pos + 1


def test_decode_negative_position_stays_invalid_over_replays(gpu_device):
    """A negative position gives a NaN output row, leaves that sequence's rings untouched, and
    writes the same negative value to pos_next, so a pos / pos_next ping-pong replay keeps the
    sequence invalid; the other sequences step normally."""
    B, H, D, S = 3, 2, 64, 1537
    inp = make_decode_inputs(B=B, H=H, D=D, S=S, seed=11)
    d = {k: v.to(gpu_device) for k, v in inp.items()}
    k_ref, v_ref = inp["k_ring"].clone(), inp["v_ring"].clone()
    pos0 = inp["pos"].clone()
    pos0[1] = -5
    pos_a = pos0.to(gpu_device)
    pos_b = torch.full_like(pos_a, 12345)
    out = torch.empty_like(d["q"])
    offs = list(OFFSETS_V3)

    def step(src, dst):
        ops.decode_step_into(d["q"], d["k_new"], d["v_new"], d["k_ring"], d["v_ring"], src,
                             d["pos_bias"], None, None, None, offs, out, dst)

    pos = pos0.clone()
    for rep in range(4):
        src, dst = (pos_a, pos_b) if rep % 2 == 0 else (pos_b, pos_a)
        step(src, dst)
        torch.cuda.synchronize(gpu_device)
        valid = torch.tensor([0, 2])
        kv, vv = k_ref[valid].clone(), v_ref[valid].clone()   # the oracle writes its rings
        ref = decode_step(inp["q"][valid].float(), inp["k_new"][valid].float(),
                          inp["v_new"][valid].float(), kv, vv, pos[valid], inp["pos_bias"])
        k_ref[valid], v_ref[valid] = kv, vv
        o = out.cpu()
        assert torch.isnan(o[1]).all()
        assert _bf16_ratio(o[valid], ref) <= 1.0
        nxt = dst.cpu()
        assert int(nxt[1]) == -5, f"replay {rep}: pos_next of the invalid sequence {int(nxt[1])}"
        assert torch.equal(nxt[valid], pos[valid] + 1)
        pos[valid] += 1
    assert torch.equal(d["k_ring"][1].cpu(), inp["k_ring"][1])
    assert torch.equal(d["v_ring"][1].cpu(), inp["v_ring"][1])
