"""A training step (forward + backward through the autograd API) captured in a HIP graph.

The kernels launch no memset and the host layer allocates only through torch's allocator, so
a whole step captures.  Each replay is checked bit for bit against the eager step on the same
inputs: three replays with eager work and synchronisations between them, then a replay after
the static inputs were overwritten with new values (the way a training or serving loop feeds a
captured step).
"""

import pytest
import torch

import dwarf_amd
from dwarf_amd.offsets import OFFSETS_V3

pytestmark = pytest.mark.gpu


def _say(msg):
    print(f"[graph] {msg}", flush=True)


def _inputs(dev, B, H, N, D, seed, se):
    g = torch.Generator().manual_seed(seed)
    q, k, v, dout = (torch.randn(B, H, N, D, generator=g).to(torch.bfloat16).to(dev) for _ in range(4))
    pb = (torch.randn(len(OFFSETS_V3), H, generator=g) * 0.5).to(dev)
    sev = (torch.randn(len(OFFSETS_V3), D, generator=g) * 0.05).to(dev) if se else None
    return q, k, v, pb, sev, dout


def _eager(q, k, v, pb, sev, dout):
    leaves = [t.detach().clone().requires_grad_(True) for t in (q, k, v, pb)]
    if sev is not None:
        leaves.append(sev.detach().clone().requires_grad_(True))
    out = dwarf_amd.dsqg_attention(*leaves[:4], leaves[4] if sev is not None else None)
    out.backward(dout)
    return [out.detach()] + [t.grad for t in leaves]


@pytest.mark.parametrize("se", [False, True])
def test_fwd_bwd_step_replays_equal_eager(gpu_device, se):
    dev = gpu_device
    B, H, N, D = 2, 4, 1024, 64
    _say(f"B{B} H{H} N{N} D{D} se={se}: eager reference")
    q, k, v, pb, sev, dout = _inputs(dev, B, H, N, D, 31, se)
    ref = _eager(q, k, v, pb, sev, dout)
    torch.cuda.synchronize(dev)

    # Static inputs (leaves) and the captured step.
    sq, sk, sv, spb = (t.detach().clone().requires_grad_(True) for t in (q, k, v, pb))
    sse = sev.detach().clone().requires_grad_(True) if se else None
    sdout = dout.clone()
    leaves = [sq, sk, sv, spb] + ([sse] if se else [])

    def step():
        out = dwarf_amd.dsqg_attention(sq, sk, sv, spb, sse)
        out.backward(sdout)
        return out

    side = torch.cuda.Stream(dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side):
        for _ in range(2):
            for t in leaves:
                t.grad = None
            step()
    torch.cuda.current_stream(dev).wait_stream(side)
    torch.cuda.synchronize(dev)
    for t in leaves:
        t.grad = None
    graph = torch.cuda.CUDAGraph()
    _say("capture")
    with torch.cuda.graph(graph):
        sout = step()
    grads = [t.grad for t in leaves]

    scratch = torch.empty(1 << 20, device=dev)
    for rep in range(3):
        _say(f"replay {rep}")
        scratch.normal_()  # eager work between replays
        torch.cuda.synchronize(dev)
        graph.replay()
        torch.cuda.synchronize(dev)
        got = [sout] + grads
        for name, x, y in zip(("out", "dq", "dk", "dv", "dpos_bias", "dscale_embed"), got, ref):
            assert torch.equal(x, y), f"replay {rep}: {name} differs from the eager step"

    _say("replay on new inputs")
    q2, k2, v2, pb2, sev2, dout2 = _inputs(dev, B, H, N, D, 32, se)
    ref2 = _eager(q2, k2, v2, pb2, sev2, dout2)
    with torch.no_grad():
        for dst, src in zip(leaves, (q2, k2, v2, pb2) + ((sev2,) if se else ())):
            dst.copy_(src)
        sdout.copy_(dout2)
    torch.cuda.synchronize(dev)
    graph.replay()
    torch.cuda.synchronize(dev)
    for name, x, y in zip(("out", "dq", "dk", "dv", "dpos_bias", "dscale_embed"), [sout] + grads, ref2):
        assert torch.equal(x, y), f"new inputs: {name} differs from the eager step"
