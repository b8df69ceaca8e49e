"""dsqg_bwd_noalloc: the backward without a workspace argument (static per-device scratch).

It runs the same kernels as dsqg_bwd, so through the C ABI its outputs must equal dsqg_bwd's
bit for bit.  Two calls in a row, the second on a smaller input, show that the scratch the
first call left behind does not leak into the second.  A call whose workspace exceeds the
scratch is refused with DSQG_ETOOLARGE before any HIP call (checked on the CPU as well).
"""

import ctypes

import pytest
import torch

from dwarf_amd import _lib, ops
from dwarf_amd.offsets import OFFSETS_V3


def _big_args():
    """Backward arguments whose workspace exceeds the scratch (pointers are never used)."""
    a = _lib.BwdArgs()
    B, H, N, D = 64, 16, 2048, 64
    a.shape = _lib.make_shape(_lib.DSQG_BF16, B, H, N, D, OFFSETS_V3)
    st = (_lib._i64x4)(H * N * D, N * D, D, 1)
    fake = 0x10000
    for name in ("q", "k", "v", "dout", "dq", "dk", "dv"):
        setattr(a, name, fake)
        setattr(a, name + "_stride", st)
    a.lse = a.alpha_lr = a.pos_bias = a.dpos_bias = a.dscale_embed = fake
    return a


def test_noalloc_refuses_calls_beyond_the_scratch():
    lib = _lib.load()
    a = _big_args()
    need = ctypes.c_size_t(0)
    assert lib.dsqg_bwd_workspace_size(ctypes.byref(a), ctypes.byref(need)) == _lib.DSQG_OK
    assert need.value > _lib.NOALLOC_SCRATCH_BYTES
    assert lib.dsqg_bwd_noalloc(ctypes.byref(a), None) == _lib.DSQG_ETOOLARGE
    assert "static scratch" in _lib.status_string(_lib.DSQG_ETOOLARGE)


def _case(dev, B, H, N, D, se, gains, seed):
    g = torch.Generator().manual_seed(seed)
    shp = (B, H, N, D)
    q, k, v, dout = (torch.randn(shp, generator=g).to(torch.bfloat16).to(dev) for _ in range(4))
    pb = (torch.randn(44, H, generator=g) * 0.5).to(dev)
    sev = (torch.randn(44, D, generator=g) * 0.05).to(dev) if se else None
    sg = (torch.rand(H, 44, generator=g) + 0.5).to(dev) if gains else None
    ig = (torch.rand(H, generator=g) * 0.4 + 0.8).to(dev) if gains else None
    fl = ops.FwdLaunch(q, k, v, pb, sev, sg, ig, list(OFFSETS_V3))
    fl.run()
    return ops.BwdLaunch(q, k, v, dout, fl.lse, pb, sev, sg, ig, list(OFFSETS_V3), se, gains, gains,
                         alpha_lr=fl.alpha_lr)


@pytest.mark.gpu
def test_noalloc_equals_workspace_backward_twice(gpu_device):
    """Two calls in a row (the second smaller), each against dsqg_bwd on the same arguments."""
    lib = _lib.load()
    stream = ops._stream(gpu_device)
    cases = [(4, 12, 2048, 64, True, True, 1), (1, 3, 700, 32, True, False, 2)]
    for B, H, N, D, se, gains, seed in cases:
        print(f"[noalloc] B{B} H{H} N{N} D{D} se={se} gains={gains}", flush=True)
        bl = _case(gpu_device, B, H, N, D, se, gains, seed)
        need = ctypes.c_size_t(0)
        _lib.check(lib.dsqg_bwd_workspace_size(ctypes.byref(bl.args), ctypes.byref(need)), "size")
        assert 0 < need.value <= _lib.NOALLOC_SCRATCH_BYTES
        bl.run()
        torch.cuda.synchronize(gpu_device)
        ref = [t.clone() for t in bl.outputs()]
        for t in bl.outputs():
            if t.numel():
                t.fill_(float("nan"))
        a = bl.args
        a.workspace, a.workspace_bytes = None, 0    # ignored by the allocation-free entry
        _lib.check(lib.dsqg_bwd_noalloc(ctypes.byref(a), stream), "dsqg_bwd_noalloc")
        torch.cuda.synchronize(gpu_device)
        for name, x, y in zip(("dq", "dk", "dv", "dpos_bias", "dscale_embed", "dscore_gain",
                               "dif_gain"), bl.outputs(), ref):
            assert torch.equal(x, y), f"{name} differs from dsqg_bwd (B{B} H{H} N{N} D{D})"


@pytest.mark.gpu
def test_noalloc_under_graph_capture(gpu_device):
    """The case the entry point exists for: dsqg_bwd_noalloc recorded into a HIP graph.  One
    eager call first (the first call on a device takes the scratch address, a query made outside
    capture), then the call is captured with torch.cuda.graph and replayed three times, with
    the outputs poisoned and eager work in between; every replay equals dsqg_bwd bit for bit.
    An eager call leaves the device's free memory and torch's allocation count unchanged."""
    lib = _lib.load()
    bl = _case(gpu_device, 2, 12, 2048, 64, True, True, 3)
    bl.run()
    torch.cuda.synchronize(gpu_device)
    ref = [t.clone() for t in bl.outputs()]
    a = bl.args
    a.workspace, a.workspace_bytes = None, 0
    stream = ops._stream(gpu_device)
    _lib.check(lib.dsqg_bwd_noalloc(ctypes.byref(a), stream), "dsqg_bwd_noalloc (eager)")
    torch.cuda.synchronize(gpu_device)
    free0, alloc0 = torch.cuda.mem_get_info(gpu_device)[0], torch.cuda.memory_allocated(gpu_device)
    _lib.check(lib.dsqg_bwd_noalloc(ctypes.byref(a), stream), "dsqg_bwd_noalloc (eager)")
    torch.cuda.synchronize(gpu_device)
    assert torch.cuda.mem_get_info(gpu_device)[0] == free0
    assert torch.cuda.memory_allocated(gpu_device) == alloc0
    for x, y in zip(bl.outputs(), ref):
        assert torch.equal(x, y)

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        cap = torch.cuda.current_stream().cuda_stream
        _lib.check(lib.dsqg_bwd_noalloc(ctypes.byref(a), ctypes.c_void_p(cap)), "dsqg_bwd_noalloc (capture)")
    for rep in range(3):
        for t in bl.outputs():
            if t.numel():
                t.fill_(float("nan"))
        junk = torch.randn(1 << 20, device=gpu_device).sum()  # eager work between replays
        graph.replay()
        torch.cuda.synchronize(gpu_device)
        assert torch.isfinite(junk)
        for name, x, y in zip(("dq", "dk", "dv", "dpos_bias", "dscale_embed", "dscore_gain",
                               "dif_gain"), bl.outputs(), ref):
            assert torch.equal(x, y), f"{name} differs from dsqg_bwd on replay {rep}"
