"""C-ABI checks that need no GPU: the library loads, exports every symbol include/dsqg.h
declares, the ctypes mirrors match the C layout, and bad arguments are rejected on the host
with the documented status codes before any HIP call."""

import ctypes
import re
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "dsqg.h"


@pytest.fixture(scope="module")
def lib():
    from dwarf_amd import _lib
    if not _lib.LIB_PATH.exists():  # nothing built yet: build once (hipcc cross-compiles here)
        from dwarf_amd.build import build
        build(verbose=False)
    return _lib.load()


def _declared_functions():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:int|const char\*|size_t)\s+(dsqg_\w+)\s*\(", text, re.M)))


def test_exports_every_declared_symbol(lib):
    from dwarf_amd import _lib
    names = _declared_functions()
    assert len(names) >= 7
    for n in names:
        assert hasattr(lib, n), f"{n} declared in dsqg.h but not exported"
        assert n in _lib.SIGNATURES, f"{n} has no ctypes signature"
    assert set(_lib.SIGNATURES) == set(names)
    assert lib.dsqg_abi_version() == _lib.ABI_VERSION


def test_ctypes_layout_matches_c(tmp_path):
    from dwarf_amd import _lib
    probes = {
        "dsqg_shape": (_lib.Shape, ["dtype", "J", "offsets"]),
        "dsqg_fwd_args": (_lib.FwdArgs, ["q", "k_stride", "pos_bias", "if_gain", "out", "lse",
                                         "alpha_lr"]),
        "dsqg_bwd_args": (_lib.BwdArgs, ["dout", "lse", "dq_stride", "dpos_bias", "dif_gain",
                                         "workspace", "workspace_bytes", "alpha_lr"]),
        "dsqg_decode_args": (_lib.DecodeArgs, ["S", "q", "pos", "pos_next", "if_gain", "out"]),
        "dsqg_pool_gate_fwd_args": (_lib.PoolFwdArgs, ["out_dtype", "x", "gate_stride", "out",
                                                       "workspace", "workspace_bytes"]),
        "dsqg_pool_gate_bwd_args": (_lib.PoolBwdArgs, ["dout_dtype", "x", "dout_stride", "dx",
                                                       "dgate_pre", "dgate_stride", "workspace",
                                                       "workspace_bytes"]),
    }
    lines = ['#include <stdio.h>', '#include <stddef.h>', f'#include "{HEADER}"', "int main(void){"]
    for cname, (_, fields) in probes.items():
        lines.append(f'printf("{cname} sizeof %zu\\n", sizeof({cname}));')
        for f in fields:
            lines.append(f'printf("{cname} {f} %zu\\n", offsetof({cname}, {f}));')
    lines.append("return 0;}")
    src = tmp_path / "probe.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "probe"
    subprocess.run(["gcc", "-std=c99", "-Wall", "-Werror", str(src), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout
    for line in out.splitlines():
        cname, what, val = line.split()
        cls = probes[cname][0]
        got = ctypes.sizeof(cls) if what == "sizeof" else getattr(cls, what).offset
        assert got == int(val), f"{cname}.{what}: ctypes {got} vs C {val}"


def _fwd_args(D=64, J=44, dtype=1, offsets=None):
    from dwarf_amd import _lib
    offs = offsets if offsets is not None else list(range(33)) + [48, 64, 96, 128, 192, 256,
                                                                  384, 512, 768, 1024, 1536][:J - 33]
    a = _lib.FwdArgs()
    a.shape = _lib.make_shape(dtype, 2, 3, 128, D, offs) if offs else _lib.Shape()
    fake = 0x10000  # never dereferenced: each case below fails validation first
    st = (ctypes.c_int64 * 4)(3 * 128 * D, 128 * D, D, 1)
    for name in ("q", "k", "v", "out"):
        setattr(a, name, fake)
        setattr(a, name + "_stride", st)
    a.pos_bias = fake
    return a


def _call_fwd(lib, a):
    return lib.dsqg_fwd(ctypes.byref(a), None)


def test_fwd_rejects_bad_arguments(lib):
    from dwarf_amd import _lib
    E, U = _lib.DSQG_EINVAL, _lib.DSQG_EUNSUPPORTED
    assert lib.dsqg_fwd(None, None) == E

    a = _fwd_args(); a.shape.dtype = 7
    assert _call_fwd(lib, a) == E
    a = _fwd_args(D=48)
    assert _call_fwd(lib, a) == U                      # no kernel for D=48
    a = _fwd_args(); a.shape.J = 0
    assert _call_fwd(lib, a) == E
    a = _fwd_args(); a.shape.J = 65
    assert _call_fwd(lib, a) == E
    a = _fwd_args(offsets=list(range(49)))
    assert _call_fwd(lib, a) == U                      # J > 48 taps in registers
    a = _fwd_args(offsets=[1, 2, 3])
    assert _call_fwd(lib, a) == E                      # must start at delta 0
    a = _fwd_args(offsets=[0, 5, 5, 9])
    assert _call_fwd(lib, a) == E                      # strictly increasing
    a = _fwd_args(); a.q_stride[3] = 2
    assert _call_fwd(lib, a) == E                      # unit inner stride
    a = _fwd_args(); a.k_stride[2] = 60
    assert _call_fwd(lib, a) == E                      # rows 16-byte aligned (bf16: 8 elems)
    a = _fwd_args(); a.v = 0x10008
    assert _call_fwd(lib, a) == E                      # misaligned base
    a = _fwd_args(); a.out = None
    assert _call_fwd(lib, a) == E
    a = _fwd_args(); a.pos_bias = None
    assert _call_fwd(lib, a) == E
    a = _fwd_args(); a.scale_embed = 0x10004
    assert _call_fwd(lib, a) == E                      # scale_embed read as 16-byte pieces
    a = _fwd_args(); a.shape.B = -1
    assert _call_fwd(lib, a) == E


def _bwd_args(need_se=True):
    from dwarf_amd import _lib
    f = _fwd_args()
    a = _lib.BwdArgs()
    a.shape = f.shape
    fake = 0x10000
    for name in ("q", "k", "v", "dout", "dq", "dk", "dv"):
        setattr(a, name, fake)
        setattr(a, name + "_stride", f.q_stride)
    a.lse = fake
    a.alpha_lr = fake
    a.pos_bias = fake
    a.dpos_bias = fake
    a.dscale_embed = fake if need_se else None
    return a


def test_bwd_workspace_query_and_errors(lib):
    from dwarf_amd import _lib
    a = _bwd_args(need_se=False)
    n0 = ctypes.c_size_t(0)
    assert lib.dsqg_bwd_workspace_size(ctypes.byref(a), ctypes.byref(n0)) == _lib.DSQG_OK
    assert n0.value >= 4 * 2 * 3 * 128               # at least D' per row
    b = _bwd_args(need_se=True)
    n1 = ctypes.c_size_t(0)
    assert lib.dsqg_bwd_workspace_size(ctypes.byref(b), ctypes.byref(n1)) == _lib.DSQG_OK
    assert n1.value > n0.value                       # dse partials need room
    b.workspace, b.workspace_bytes = 0x100000, n1.value - 1
    assert lib.dsqg_bwd(ctypes.byref(b), None) == _lib.DSQG_EWORKSPACE
    b.workspace, b.workspace_bytes = None, n1.value
    assert lib.dsqg_bwd(ctypes.byref(b), None) == _lib.DSQG_EWORKSPACE
    b.workspace = 0x100010                           # not 256-byte aligned
    assert lib.dsqg_bwd(ctypes.byref(b), None) == _lib.DSQG_EINVAL
    c = _bwd_args(); c.lse = None
    assert lib.dsqg_bwd_workspace_size(ctypes.byref(c), ctypes.byref(n0)) == _lib.DSQG_EINVAL
    c = _bwd_args(); c.dpos_bias = None
    assert lib.dsqg_bwd(ctypes.byref(c), None) == _lib.DSQG_EINVAL
    assert lib.dsqg_bwd_workspace_size(ctypes.byref(c), None) == _lib.DSQG_EINVAL
    c = _bwd_args(); c.scale_embed = 0x10008             # scale_embed not 16-byte aligned
    assert lib.dsqg_bwd_workspace_size(ctypes.byref(c), ctypes.byref(n0)) == _lib.DSQG_EINVAL
    c = _bwd_args(); c.alpha_lr = None                   # bf16 needs the forward's alpha_lr
    assert lib.dsqg_bwd_workspace_size(ctypes.byref(c), ctypes.byref(n0)) == _lib.DSQG_EINVAL
    assert lib.dsqg_bwd(ctypes.byref(c), None) == _lib.DSQG_EINVAL
    c = _bwd_args(); c.alpha_lr = 0x10002                # fp32 elements: 4-byte aligned
    assert lib.dsqg_bwd_workspace_size(ctypes.byref(c), ctypes.byref(n0)) == _lib.DSQG_EINVAL


def test_long_range_taps_and_alpha_size(lib):
    """NS (taps beyond the dense window) of the named tables, and the alpha_lr element count."""
    from dwarf_amd import _lib
    from dwarf_amd.offsets import OFFSETS_J46, OFFSETS_J47, OFFSETS_V3
    for offs, ns in ((OFFSETS_V3, 11), (OFFSETS_J46, 13), (OFFSETS_J47, 14), ((0,), 0),
                     (tuple(range(48)), 15), ((0, 1, 2, 5, 9, 100), 3)):
        assert _lib.long_range_taps(offs) == ns, offs
    arr = (ctypes.c_int32 * 3)(1, 2, 3)
    assert lib.dsqg_long_range_taps(arr, 3) == -_lib.DSQG_EINVAL   # must start at 0
    n = ctypes.c_size_t(0)
    sh = _lib.make_shape(_lib.DSQG_BF16, 2, 3, 100, 64, OFFSETS_V3)
    assert lib.dsqg_alpha_lr_elems(ctypes.byref(sh), ctypes.byref(n)) == _lib.DSQG_OK
    assert n.value == 2 * 3 * 11 * 100
    sh = _lib.make_shape(_lib.DSQG_F32, 2, 3, 100, 64, OFFSETS_V3)
    assert lib.dsqg_alpha_lr_elems(ctypes.byref(sh), ctypes.byref(n)) == _lib.DSQG_OK
    assert n.value == 0


def test_decode_rejects_bad_arguments(lib):
    from dwarf_amd import _lib
    a = _lib.DecodeArgs()
    a.shape = _lib.make_shape(1, 4, 2, 0, 64, list(range(33)) + [48, 64, 1536])
    fake = 0x10000
    for name in ("q", "k_new", "v_new", "k_ring", "v_ring", "out", "pos", "pos_bias"):
        setattr(a, name, fake)
    a.S = 1536                                       # must exceed max offset
    assert lib.dsqg_decode_step(ctypes.byref(a), None) == _lib.DSQG_EINVAL
    a.S = 1537
    a.pos_next = fake                                # must differ from pos
    assert lib.dsqg_decode_step(ctypes.byref(a), None) == _lib.DSQG_EINVAL
    a.pos_next = None
    a.q = 0x10004
    assert lib.dsqg_decode_step(ctypes.byref(a), None) == _lib.DSQG_EINVAL


def test_status_strings_and_head_dims(lib):
    from dwarf_amd import _lib
    for code in range(6):
        assert _lib.status_string(code)
    assert "unknown" in _lib.status_string(99)
    assert sorted(_lib.supported_head_dims()) == [32, 64, 80, 96, 128]


def test_product_refuses_cpu_tensors():
    import torch
    import dwarf_amd
    q = torch.randn(1, 2, 16, 64)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        dwarf_amd.dsqg_attention_v3(q, q, q, torch.zeros(44, 2), torch.zeros(44, 64))
    with pytest.raises(AssertionError):
        dwarf_amd.dsqg_attention_v3(q, q, q, torch.zeros(43, 2), torch.zeros(44, 64))


def _pool_fwd_args(B=2, N=64, C=32, dt=0):
    from dwarf_amd import _lib
    a = _lib.PoolFwdArgs()
    a.B, a.N, a.C = B, N, C
    a.x_dtype = a.gate_dtype = a.out_dtype = dt
    fake = 0x10000  # never dereferenced: each case below fails validation first
    st = (ctypes.c_int64 * 2)(N * C, C)
    for name in ("x", "gate_pre", "out"):
        setattr(a, name, fake)
    a.x_stride, a.gate_stride, a.out_stride = st, st, st
    return a


def test_pool_gate_rejects_bad_arguments(lib):
    from dwarf_amd import _lib
    E, W = _lib.DSQG_EINVAL, _lib.DSQG_EWORKSPACE
    n = ctypes.c_size_t(0)
    assert lib.dsqg_pool_gate_workspace_size(2, 64, 32, 0, ctypes.byref(n)) == _lib.DSQG_OK
    n_fwd = n.value
    assert lib.dsqg_pool_gate_workspace_size(2, 64, 32, 1, ctypes.byref(n)) == _lib.DSQG_OK
    assert n.value > 0 and n_fwd > 0 and n_fwd % 256 == 0 and n.value % 256 == 0
    assert lib.dsqg_pool_gate_workspace_size(2, 64, 30, 0, ctypes.byref(n)) == E   # C % 8
    assert lib.dsqg_pool_gate_workspace_size(-1, 64, 32, 0, ctypes.byref(n)) == E
    assert lib.dsqg_pool_gate_workspace_size(2, 64, 32, 0, None) == E

    call = lambda a: lib.dsqg_pool_gate_fwd(ctypes.byref(a), None)
    assert lib.dsqg_pool_gate_fwd(None, None) == E
    a = _pool_fwd_args(C=12)
    assert call(a) == E                                   # C must be a multiple of 8
    a = _pool_fwd_args(); a.gate_dtype = 5
    assert call(a) == E                                   # unknown element type
    a = _pool_fwd_args(); a.x = 0x10004
    assert call(a) == E                                   # misaligned base
    a = _pool_fwd_args(dt=1); a.gate_stride[1] = 36
    assert call(a) == E                                   # rows 16-byte aligned
    a = _pool_fwd_args(); a.out = None
    assert call(a) == E
    a = _pool_fwd_args(); a.x_stride[1] = 16
    assert call(a) == E                                   # overlapping rows (stride < C)
    a = _pool_fwd_args()                                  # valid, but no workspace
    assert call(a) == W
    a = _pool_fwd_args(N=0)                               # empty: nothing to do, no launch
    assert call(a) == _lib.DSQG_OK

    b = _lib.PoolBwdArgs()
    b.B, b.N, b.C = 2, 64, 32
    st = (ctypes.c_int64 * 2)(64 * 32, 32)
    for name, sname in (("x", "x"), ("gate_pre", "gate"), ("dout", "dout"), ("dx", "dx"),
                        ("dgate_pre", "dgate")):
        setattr(b, name, 0x10000)
        setattr(b, sname + "_stride", st)
    bcall = lambda a: lib.dsqg_pool_gate_bwd(ctypes.byref(a), None)
    assert bcall(b) == W                                  # valid, but no workspace
    b.dout_dtype = 9
    assert bcall(b) == E
    b.dout_dtype = 0; b.dx = 0x10002
    assert bcall(b) == E
    b.dx = None; b.dgate_pre = None                       # nothing requested: no launch
    assert bcall(b) == _lib.DSQG_OK


def test_bf16_row_span_limit(lib):
    """bf16 kernels address each (b,h) slice with 32-bit byte offsets: a call is taken while
    (N + max offset + 64) * (largest row stride) * 2 < 2^31 and refused with DSQG_EUNSUPPORTED
    past it.  At the headline model width (E 768, heads of 64 read as views of a packed qkv
    projection, row stride 3 * 768) that is N <= 464,433 with the 44-offset table; checked here
    through the workspace query and the forward's validation, neither of which launches."""
    from dwarf_amd import _lib
    rs, H, D = 3 * 768, 12, 64
    offs = list(range(33)) + [48, 64, 96, 128, 192, 256, 384, 512, 768, 1024, 1536]
    n_max = (2 ** 31 - 1) // (2 * rs) - 1536 - 64
    assert (n_max + 1600) * rs * 2 < 2 ** 31 <= (n_max + 1601) * rs * 2
    for N, want in ((n_max, _lib.DSQG_OK), (n_max + 1, _lib.DSQG_EUNSUPPORTED)):
        st = (ctypes.c_int64 * 4)(N * rs, D, rs, 1)
        b = _lib.BwdArgs()
        b.shape = _lib.make_shape(_lib.DSQG_BF16, 1, H, N, D, offs)
        for name in ("q", "k", "v", "dout", "dq", "dk", "dv"):
            setattr(b, name, 0x10000)
            setattr(b, name + "_stride", st)
        b.lse = b.alpha_lr = b.pos_bias = b.dpos_bias = 0x10000
        n = ctypes.c_size_t(0)
        assert lib.dsqg_bwd_workspace_size(ctypes.byref(b), ctypes.byref(n)) == want, N
    f = _lib.FwdArgs()
    N = n_max + 1
    f.shape = _lib.make_shape(_lib.DSQG_BF16, 1, H, N, D, offs)
    st = (ctypes.c_int64 * 4)(N * rs, D, rs, 1)
    for name in ("q", "k", "v", "out"):
        setattr(f, name, 0x10000)
        setattr(f, name + "_stride", st)
    f.pos_bias = 0x10000
    assert lib.dsqg_fwd(ctypes.byref(f), None) == _lib.DSQG_EUNSUPPORTED   # refused before a launch
