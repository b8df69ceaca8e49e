"""Benchmark of the DSQG hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config 2] [--no-cpu-baseline]

A step is one DSQG forward + backward over one batch of the headline workload (config 2:
B8 H12 N2048 D64, bf16, 44 offsets, synthetic seeded inputs already resident in HBM).  Three
input sets are rotated so that consecutive steps cannot be served from the 256 MB Infinity Cache.
Prints one JSON line: tok/s (B*N per step), the roofline of the dominant kernel (algorithmic
bytes per launch over its median launch time, HIP events on the launch stream), the
fraction of HBM peak for the whole fwd+bwd step, BASELINE's configs 1 and 3 and the 85M
trainer's D = 96 call under the same protocol, the ring-buffer decode step (workload 4,
1000 steps replayed from a HIP graph), the drop-in DSQGAttentionQW layer fwd+bwd, the DWARF
block's interference pool (causal mean times a sigmoid gate) forward and backward, greedy
generation with the condU 13M model (incremental vs the reference's full recomputation), and
the CPU oracle timed on a bounded sample.
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

HBM_PEAK_GBS = 8000.0


def _events_ms(fn, reps, stream):
    """Median over `reps` calls of fn(i), each bracketed by its own pair of HIP events on
    `stream` (events only, no synchronisation between calls)."""
    import torch
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(reps + 1)]
    torch.cuda.synchronize()
    ev[0].record(stream)
    for i in range(reps):
        fn(i)
        ev[i + 1].record(stream)
    ev[-1].synchronize()
    return statistics.median(ev[i].elapsed_time(ev[i + 1]) for i in range(reps))


def _cpu_identity():
    """os.cpu_count(), torch's thread count and the lscpu model name of this host."""
    import platform
    import subprocess
    import torch
    model = platform.processor() or ""
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            if line.startswith("Model name:"):
                model = line.split(":", 1)[1].strip()
    except (OSError, subprocess.SubprocessError):
        pass
    return {"os_cpu_count": os.cpu_count(), "torch_threads": torch.get_num_threads(),
            "cpu_model": model}


def cpu_baseline(w, inp_cpu, min_seconds=10.0, max_reps=20):
    """CPU oracle (fp32 autograd restatement of the reference) on the whole workload batch.

    One warm-up call, then whole-batch fwd+bwd calls until at least `min_seconds` of CPU work
    (and at least 3 calls) have been timed; value = tokens processed / time.
    """
    import torch
    from oracle import dsqg_forward_backward
    sl = {k: (v.float() if k in ("q", "k", "v", "dout") else v) for k, v in inp_cpu.items()}
    threads = torch.get_num_threads()

    def run():
        dsqg_forward_backward(sl["q"], sl["k"], sl["v"], sl["pos_bias"], sl["dout"],
                              sl["scale_embed"], w.offsets, sl["score_gain"], sl["if_gain"],
                              dtype=torch.float32)

    run()  # warm-up
    times = []
    while len(times) < max_reps and (len(times) < 3 or sum(times) < min_seconds):
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
        print(f"[bench] cpu oracle call {len(times)}: {times[-1]:.2f} s", file=sys.stderr, flush=True)
    total = sum(times)
    tokens = w.B * w.N * len(times)
    return {"value": round(tokens / total, 1), "unit": "tok/s", "cores": threads, "kind": "port",
            "sample": (f"whole config-{w.index} batch (B{w.B} H{w.H} N{w.N} D{w.D} J{w.J}) fwd+bwd, "
                       f"oracle/dsqg_oracle.py fp32 autograd, {len(times)} calls after 1 warm-up, "
                       f"{total:.1f} s timed, torch threads={threads}"),
            "seconds_per_call": round(total / len(times), 3), **_cpu_identity()}


def cpu_baseline_decode(steps=10):
    """CPU oracle decode step (ring restatement, fp32) on the decode workload, `steps` steps."""
    import torch
    from oracle import decode_step
    from dwarf_amd.workloads import DECODE, make_decode_inputs
    d = make_decode_inputs(device="cpu")
    f = {k: (v.float() if v.is_floating_point() else v) for k, v in d.items()}
    pos = f["pos"].clone()
    decode_step(f["q"], f["k_new"], f["v_new"], f["k_ring"], f["v_ring"], pos, f["pos_bias"],
                offsets=DECODE["offsets"])  # warm-up
    t0 = time.perf_counter()
    for _ in range(steps):
        pos += 1
        decode_step(f["q"], f["k_new"], f["v_new"], f["k_ring"], f["v_ring"], pos, f["pos_bias"],
                    offsets=DECODE["offsets"])
    dt = (time.perf_counter() - t0) / steps
    return {"value": round(DECODE["B"] / dt, 1), "unit": "tok/s", "kind": "port",
            "cores": torch.get_num_threads(),
            "sample": (f"decode workload (B{DECODE['B']} H{DECODE['H']} D{DECODE['D']} ring "
                       f"{DECODE['S']}), oracle/dsqg_oracle.py decode_step fp32, {steps} steps "
                       f"after 1 warm-up"),
            "ms_per_step": round(dt * 1e3, 3)}


def bench_decode(dev, steps=1000, layers=8, batch=None):
    """Ring-buffer decode step, workload 4 (B256 H12 D64, 44 offsets, 1537-slot rings; `batch`
    replaces B for the batch sweep).

    Two figures, both from HIP-graph replays timed with HIP events:
    * ``layers`` (the headline): ``layers`` independent ring pairs, as the caches of an
      8-layer model (8 x 1.2 GB), each token stepping every layer once.  A layer's rows come
      back only after the other layers' steps (8 x 36 MB > the 256 MB Infinity Cache), so the
      bytes come from HBM.
    * ``single_ring``: ``steps`` consecutive steps on one ring pair, where a step re-reads the
      dense-window rows the previous step read (cache-assisted; kept for comparison).
    """
    import torch
    from dwarf_amd import ops
    from dwarf_amd.workloads import DECODE, decode_bytes_per_step, make_decode_inputs
    cfg = DECODE
    B, H, D, S = batch or cfg["B"], cfg["H"], cfg["D"], cfg["S"]
    offs = list(cfg["offsets"])
    small = make_decode_inputs(device="cpu", B=B, H=H, D=D, S=2)  # q, k_new, v_new, pos, bias
    gen = torch.Generator(device=dev).manual_seed(4004)
    sets = []
    for _ in range(layers):
        ring = lambda: torch.randn((B, H, S, D), generator=gen, device=dev, dtype=torch.bfloat16)
        rows = lambda: torch.randn((B, H, D), generator=gen, device=dev, dtype=torch.bfloat16)
        pos_a = small["pos"].to(dev)
        sets.append(dict(k_ring=ring(), v_ring=ring(), q=rows(), k_new=rows(), v_new=rows(),
                         pos_a=pos_a, pos_b=torch.empty_like(pos_a),
                         out=torch.empty((B, H, D), device=dev, dtype=torch.bfloat16)))
    pb = small["pos_bias"].to(dev)

    def step(d, flip):
        src, dst = (d["pos_a"], d["pos_b"]) if not flip else (d["pos_b"], d["pos_a"])
        ops.decode_step_into(d["q"], d["k_new"], d["v_new"], d["k_ring"], d["v_ring"], src, pb,
                             None, None, None, offs, d["out"], dst)

    def timed_graph(order):
        s = torch.cuda.Stream(dev)
        s.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(s):
            for i in range(4):
                for li, flip in order[:2 * layers]:
                    step(sets[li], flip)
        torch.cuda.current_stream(dev).wait_stream(s)
        torch.cuda.synchronize(dev)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=s):
            for li, flip in order:
                step(sets[li], flip)
        graph.replay()  # warm-up replay
        torch.cuda.synchronize(dev)
        st = torch.cuda.current_stream(dev)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(st)
        graph.replay()
        e1.record(st)
        e1.synchronize()
        return e0.elapsed_time(e1) * 1000.0 / len(order)

    tokens = max(1, steps // layers)
    # Token t steps layer 0..layers-1, each layer flipping its own pos / pos_next pair.
    us_layers = timed_graph([(li, t % 2 == 1) for t in range(tokens) for li in range(layers)])
    us_single = timed_graph([(0, i % 2 == 1) for i in range(steps)])
    nbytes = decode_bytes_per_step(B, H, D, len(offs))

    def fig(us):
        gbs = nbytes / (us * 1e-6) / 1e9
        return {"us_per_step": round(us, 3), "tok_per_s": round(B / (us * 1e-6), 1),
                "achieved_GBs": round(gbs, 1), "frac_hbm_peak": round(gbs / HBM_PEAK_GBS, 4)}
    res = {"workload": f"decode B{B} H{H} D{D} J{len(offs)} ring {S} (config 4)",
           "algorithmic_bytes_per_step": nbytes,
           **fig(us_layers),
           "layers": {"ring_pairs": layers, "tokens": tokens, "steps": tokens * layers,
                      **fig(us_layers)},
           "single_ring": {"steps": steps, **fig(us_single)},
           "timing": "hipGraph replay, HIP events; headline figures are the layers variant"}
    del sets
    torch.cuda.empty_cache()
    return res


def bench_module(dev, steps=20, warmup=20):
    """DSQGAttentionQW (E768 H12, the config-2 attention layer) fwd+bwd in bf16 on x [8,2048,768]:
    as shipped (q, k, v strided views of the qkv projection), with the reference's
    permute().contiguous() copies put back (train/train_2048_condU.py:173-175), and with a K/V
    injection in the path; plus the injection adds and the gate multiply timed alone (what a fold
    of either into the kernels could save at most)."""
    import torch
    from dwarf_amd import dsqg_attention
    from dwarf_amd.modules import DSQGAttentionQW, _heads
    B, N, E, H = 8, 2048, 768, 12
    torch.manual_seed(3)
    m = DSQGAttentionQW(E, H, dropout=0.0).to(dev, torch.bfloat16)
    x = torch.randn(B, N, E, device=dev, dtype=torch.bfloat16, requires_grad=True)
    dy = torch.randn(B, N, E, device=dev, dtype=torch.bfloat16)

    def contiguous_copy_forward(x):
        q, k, v = (t.contiguous() for t in _heads(m.qkv_proj(x), B, N, H, E // H))
        out = dsqg_attention(q, k, v, m.pos_bias, m.scale_embed, if_gain=m.if_gain)
        flat = out.permute(0, 2, 1, 3).reshape(B, N, E)
        return m.out_proj(flat * torch.sigmoid(m.gate_proj(x)))

    res = {"workload": "DSQGAttentionQW E768 H12, x [8,2048,768] bf16, fwd+bwd incl. projections",
           "steps": steps}
    stream = torch.cuda.current_stream(dev)
    for name, fwd in (("strided_views", m), ("contiguous_copies", contiguous_copy_forward)):
        def step(i):
            fwd(x).backward(dy)
        for i in range(warmup):
            step(i)
        ms = _events_ms(step, steps, stream)
        res[f"ms_per_step_{name}"] = round(ms, 4)
    res["tok_per_s"] = round(B * N / (res["ms_per_step_strided_views"] * 1e-3), 1)

    # The two elementwise steps around the kernels that a fold into the kernels could remove
    # (train/train_2048_condU.py:178-181, 190-191), each timed alone (fwd+bwd, same shapes), and the
    # module with the K/V injection in its path (deltas requiring grad, as the block's are).
    kd, vd = (torch.randn(B, H, N, E // H, device=dev, dtype=torch.bfloat16, requires_grad=True)
              for _ in range(2))
    qkv = torch.randn(B, N, 3 * E, device=dev, dtype=torch.bfloat16, requires_grad=True)
    dk_up = torch.randn(B, H, N, E // H, device=dev, dtype=torch.bfloat16)
    o_flat = torch.randn(B, N, E, device=dev, dtype=torch.bfloat16, requires_grad=True)
    g_pre = torch.randn(B, N, E, device=dev, dtype=torch.bfloat16, requires_grad=True)
    gate = torch.sigmoid(g_pre).detach().requires_grad_(True)

    def inject_step(i):
        _, k, v = _heads(qkv, B, N, H, E // H)
        torch.autograd.backward([k + kd, v + vd], [dk_up, dk_up])

    def gate_step(i):
        (o_flat * gate).backward(dy)

    def module_inject_step(i):
        m(x, kv_inject=(kd, vd)).backward(dy)

    for name, fn in (("kv_inject_adds", inject_step), ("gate_multiply", gate_step),
                     ("module_with_kv_inject", module_inject_step)):
        for i in range(warmup):
            fn(i)
        res[f"ms_{name}"] = round(_events_ms(fn, steps, stream), 4)
    return res


def table_sweep(dev, reps=50):
    """Each attention kernel at the config-2 shape (B8 H12 N2048 D64 bf16) over four offset
    tables: delta = 0 alone (the kernels' fixed structure: window staging, band tiles,
    epilogue), the dense window 0..32, delta = 0 with the eleven long-range taps, and the full
    44-offset table.  Isolated launches (fwd, dq phase, dk/dv phase) timed with HIP events over
    two alternating input sets; medians of `reps`.  Prints one JSON line."""
    import torch
    from dwarf_amd import ops
    from dwarf_amd.offsets import OFFSETS_V3
    B, H, N, D = 8, 12, 2048, 64
    lr = tuple(o for o in OFFSETS_V3 if o > 32)
    tables = [("delta 0", (0,)), ("dense 0..32", tuple(range(33))), ("0 + 11 long-range", (0,) + lr),
              ("V3 (44)", tuple(OFFSETS_V3))]
    stream = torch.cuda.current_stream(dev)
    gen = torch.Generator(device=dev).manual_seed(77)
    rows = []
    for name, offs in tables:
        J = len(offs)
        sets = []
        for _ in range(2):
            q, k, v, do = (torch.randn((B, H, N, D), generator=gen, device=dev).to(torch.bfloat16)
                           for _ in range(4))
            pb = torch.randn((J, H), generator=gen, device=dev) * 0.5
            fl = ops.FwdLaunch(q, k, v, pb, None, None, None, list(offs))
            fl.run()
            bl = ops.BwdLaunch(q, k, v, do, fl.lse, pb, None, None, None, list(offs), False, False, False,
                               alpha_lr=fl.alpha_lr)
            sets.append((fl, bl))
        for i in range(10):
            sets[i % 2][0].run()
            sets[i % 2][1].run()
        times = {"fwd": [], "dq": [], "dkdv": []}
        for i in range(reps):
            fl, bl = sets[i % 2]
            e = [torch.cuda.Event(enable_timing=True) for _ in range(4)]
            e[0].record(stream)
            fl.run()
            e[1].record(stream)
            bl.run("dq")
            e[2].record(stream)
            bl.run("dkdv")
            e[3].record(stream)
            e[3].synchronize()
            for j, key in enumerate(("fwd", "dq", "dkdv")):
                times[key].append(e[j].elapsed_time(e[j + 1]) * 1000.0)
        row = {"table": name, "J": J}
        row.update({f"{key}_us": round(statistics.median(v), 2) for key, v in times.items()})
        rows.append(row)
        print(f"[bench] table {name}: {row}", file=sys.stderr, flush=True)
        del sets
    print(json.dumps({"table_sweep": rows, "shape": f"B{B} H{H} N{N} D{D} bf16"}), flush=True)
    return 0


def decode_sweep(dev, steps):
    """Decode step time against batch size (the fixed per-step latency and the marginal
    bandwidth), next to the per-launch time of a trivial kernel replayed from a hipGraph."""
    import torch
    rows = []
    for B in (32, 64, 128, 256, 512):
        r = bench_decode(dev, steps=steps, batch=B)
        rows.append({"B": B, "us_per_step": r["us_per_step"],
                     "algorithmic_bytes_per_step": r["algorithmic_bytes_per_step"],
                     "frac_hbm_peak": r["frac_hbm_peak"]})
        print(f"[bench] decode B{B}: {r['us_per_step']} us", file=sys.stderr, flush=True)
    x = torch.zeros(64, device=dev)
    s = torch.cuda.Stream(dev)
    s.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(s):
        x.add_(1)
    torch.cuda.current_stream(dev).wait_stream(s)
    torch.cuda.synchronize(dev)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        for _ in range(steps):
            x.add_(1)
    graph.replay()
    torch.cuda.synchronize(dev)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    graph.replay()
    e1.record()
    e1.synchronize()
    trivial = round(e0.elapsed_time(e1) * 1000.0 / steps, 3)
    print(json.dumps({"decode_sweep": rows, "trivial_kernel_us_per_launch": trivial}), flush=True)
    return 0


def bench_pool(dev, steps=200, sets=3):
    """Interference pool of the DWARF block (dsqg_pool_gate_fwd / _bwd: sigmoid(gate) times
    the causal mean, train/train_2048_condU.py:289-292) at the headline layer's width:
    x, gate_pre, dout [8,2048,768] bf16, 3 rotating input sets.  Each direction's `steps`
    calls are captured in one hipGraph and the replay is timed with HIP events, so the figure
    is GPU time (two kernel launches per call).  Algorithmic bytes: forward reads x and
    gate_pre and writes out (3 T C E); backward reads x, gate_pre, dout and writes dx,
    dgate_pre (5 T C E)."""
    import torch
    from dwarf_amd import ops
    B, N, C = 8, 2048, 768
    g = torch.Generator().manual_seed(2024)
    calls = []
    for _ in range(sets):
        x, gp, dy = ((torch.randn((B, N, C), generator=g) * sc).to(dev, torch.bfloat16)
                     for sc in (1.0, 2.0, 1.0))
        calls.append((ops.PoolLaunch(x, gp), ops.PoolLaunch(x, gp, dy)))
    elem = B * N * C * 2
    res = {"workload": f"pool+gate x/gate_pre/dout [{B},{N},{C}] bf16", "steps": steps}
    s = torch.cuda.Stream(dev)
    s.wait_stream(torch.cuda.current_stream(dev))
    for name, idx, nbytes in (("fwd", 0, 3 * elem), ("bwd", 1, 5 * elem)):
        with torch.cuda.stream(s):
            for i in range(2 * sets):
                calls[i % sets][idx].run()
        torch.cuda.current_stream(dev).wait_stream(s)
        torch.cuda.synchronize(dev)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=s):
            for i in range(steps):
                calls[i % sets][idx].run()
        graph.replay()
        torch.cuda.synchronize(dev)
        st = torch.cuda.current_stream(dev)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(st)
        graph.replay()
        e1.record(st)
        e1.synchronize()
        us = e0.elapsed_time(e1) * 1000.0 / steps
        gbs = nbytes / (us * 1e-6) / 1e9
        res[name] = {"us": round(us, 3), "algorithmic_bytes": nbytes, "achieved_GBs": round(gbs, 1),
                     "frac_hbm_peak": round(gbs / HBM_PEAK_GBS, 4)}
    return res


def bench_generation(dev, prompt=1024, new_tokens=64, ref_tokens=16):
    """Greedy generation with the condU 13M model (train/train_2048_condU.py:55-67: vocab 32000,
    E 256, 6 layers, 8 heads, FFN 1024, seq_len 2048; random weights, bf16), one sequence:
    CondMTransformer.generate (prefill once, then one decode step per layer and token) against
    the reference's loop, which runs the whole model on the sequence for every token
    (train/train_2048_condU.py:463-487), timed on `ref_tokens` tokens."""
    import torch
    from dwarf_amd.generation import CondMTransformer
    torch.manual_seed(13)
    m = CondMTransformer(32000, 256, 6, 8, 1024, 2048, dropout=0.0).to(dev, torch.bfloat16).eval()
    ids = torch.randint(0, 32000, (1, prompt), device=dev)

    def timed(fn, reps=3):
        # Both loops are host-bound at batch 1 (the reference's most of all: ~300 launches per
        # token), so the best of a few repetitions is kept against transient host contention.
        best = None
        for _ in range(reps):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            out = fn()
            torch.cuda.synchronize()
            dt = time.perf_counter() - t0
            best = dt if best is None else min(best, dt)
        return out, best

    m.generate(ids[:, :64], 4, temperature=0.0)  # warm-up
    out, t_inc = timed(lambda: m.generate(ids, new_tokens, temperature=0.0))

    def reference_loop():
        x = ids
        with torch.no_grad():
            for _ in range(ref_tokens):
                nxt = m(x[:, -m.seq_len:])[:, -1].argmax(-1, keepdim=True)
                x = torch.cat([x, nxt], dim=1)
        return x

    reference_loop()  # warm-up
    ref, t_ref = timed(reference_loop)
    return {"workload": f"condU 13M (V32000 E256 L6 H8) bf16, prompt {prompt}, greedy, batch 1",
            "new_tokens": new_tokens, "tok_per_s_incremental": round(new_tokens / t_inc, 1),
            "tok_per_s_full_recompute": round(ref_tokens / t_ref, 1),
            "same_tokens": bool(torch.equal(out[:, :prompt + ref_tokens], ref)),
            "timing": "wall clock around the whole loop, synchronised, best of 3"}


TRAFFIC_PROFILE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                               "hbm_traffic_config2.md")


def measured_traffic(kernel):
    """HBM bytes per launch of `kernel` from the committed counter summary, or None.

    The summary holds lines `traffic_bytes_per_launch <kernel> = <bytes>`: FETCH_SIZE plus
    WRITE_SIZE of the kernel (two rocprofv3 --pmc passes of `bench.py --profile-kernel`), each
    scaled by what the same counter reads for a plain device copy of known size.
    """
    try:
        with open(TRAFFIC_PROFILE) as f:
            for line in f:
                parts = line.replace("`", "").split()
                if len(parts) == 4 and parts[0] == "traffic_bytes_per_launch" and parts[1] == kernel:
                    return int(parts[3])
    except OSError:
        pass
    return None


def profile_decode(args, dev):
    """Counter mode for the decode kernel: --profile-reps steps on each of 8 ring pairs in turn
    (as the layers variant of the decode leg), then the plain copy of known size."""
    import torch
    from dwarf_amd import ops
    from dwarf_amd.workloads import DECODE, make_decode_inputs
    B, H, D, S = DECODE["B"], DECODE["H"], DECODE["D"], DECODE["S"]
    small = make_decode_inputs(device="cpu", B=B, H=H, D=D, S=2)
    gen = torch.Generator(device=dev).manual_seed(4004)
    pb = small["pos_bias"].to(dev)
    layers = []
    for _ in range(8):
        r = lambda *shp: torch.randn(shp, generator=gen, device=dev, dtype=torch.bfloat16)
        layers.append((r(B, H, S, D), r(B, H, S, D), r(B, H, D), r(B, H, D), r(B, H, D),
                       small["pos"].to(dev), torch.empty((B, H, D), device=dev, dtype=torch.bfloat16)))
    for rep in range(args.profile_reps):
        for kr, vr, q, kn, vn, pos, out in layers:
            nxt = pos + 1
            ops.decode_step_into(q, kn, vn, kr, vr, pos, pb, None, None, None,
                                 list(DECODE["offsets"]), out, nxt)
            pos.copy_(nxt)
    nbytes = args.copy_mib << 20
    src = torch.ones(nbytes, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    for _ in range(args.profile_reps):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(f"[bench] profile mode: {8 * args.profile_reps} decode steps over 8 ring pairs, "
          f"{args.profile_reps} copies of {nbytes} bytes", file=sys.stderr, flush=True)
    return 0


def profile_mode(args, w, dev):
    """Launches one kernel of the workload a few times and a plain copy of known size.

    With --profile-sets K > 1 the launches rotate over K input sets (each set's inputs, outputs
    and workspace about 250 MB at config 2), so a launch's inputs were last touched K - 1
    launches earlier, with more than the 256 MB Infinity Cache of other data in between: no
    line of them is cached when it starts, and each L2 miss of a line's first touch is an HBM
    read."""
    import torch
    if args.profile_kernel == "decode":
        return profile_decode(args, dev)
    if args.profile_kernel == "pool":
        return profile_pool(args, dev)
    # With --profile-se the scale_embed leg's inputs (scale_embed and if_gain).
    sets = make_sets(w, dev, max(1, args.profile_sets), scale_embed=args.profile_se,
                     if_gain=args.profile_se)
    for _, _, fl, bl in sets:
        fl.run()
        bl.run()
    torch.cuda.synchronize()
    for r in range(args.profile_reps):
        _, _, fl, bl = sets[(r + 1) % len(sets)]
        if args.profile_kernel == "fwd":
            fl.run()
        else:
            bl.run(args.profile_kernel)
    nbytes = args.copy_mib << 20
    src = torch.ones(nbytes, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    for _ in range(args.profile_reps):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(f"[bench] profile mode: {args.profile_reps} launches of {args.profile_kernel}, "
          f"{args.profile_reps} copies of {nbytes} bytes", file=sys.stderr, flush=True)
    return 0


def profile_pool(args, dev):
    """The pool leg's shape (x, gate_pre, dout [8, 2048, 768] bf16): one forward and one
    backward first, then --profile-reps of each (two launches apiece)."""
    import torch
    from dwarf_amd import ops
    B, N, C = 8, 2048, 768
    g = torch.Generator().manual_seed(2024)
    x, gp, dy = ((torch.randn((B, N, C), generator=g) * sc).to(dev, torch.bfloat16)
                 for sc in (1.0, 2.0, 1.0))
    fwd, bwd = ops.PoolLaunch(x, gp), ops.PoolLaunch(x, gp, dy)
    fwd.run()
    bwd.run()
    torch.cuda.synchronize()
    for _ in range(args.profile_reps):
        fwd.run()
        bwd.run()
    torch.cuda.synchronize()
    print(f"[bench] profile mode: {args.profile_reps} pool forward + backward calls", file=sys.stderr,
          flush=True)
    return 0


def make_sets(w, dev, n, scale_embed=False, if_gain=False):
    """`n` input sets of workload w (seeds w.seed + 100 i), each with its launch objects.
    scale_embed / if_gain add the reference module's parameters (se ~ 0.05 N(0,1),
    a ~ U(0.8, 1.2)), the call of train/train_2048_condU.py:184,187."""
    import torch
    from dwarf_amd import ops
    from dwarf_amd.workloads import make_inputs
    sets = []
    for i in range(n):
        inp = make_inputs(w, device="cpu", seed=w.seed + 100 * i)
        g = torch.Generator().manual_seed(w.seed + 100 * i + 7)
        if scale_embed:
            inp["scale_embed"] = torch.randn(w.J, w.D, generator=g) * 0.05
        if if_gain:
            inp["if_gain"] = torch.rand(w.H, generator=g) * 0.4 + 0.8
        d = {k: (None if v is None else v.to(dev)) for k, v in inp.items()}
        fl = ops.FwdLaunch(d["q"], d["k"], d["v"], d["pos_bias"], d["scale_embed"],
                           d["score_gain"], d["if_gain"], list(w.offsets))
        bl = ops.BwdLaunch(d["q"], d["k"], d["v"], d["dout"], fl.lse, d["pos_bias"],
                           d["scale_embed"], d["score_gain"], d["if_gain"], list(w.offsets),
                           d["scale_embed"] is not None, d["score_gain"] is not None,
                           d["if_gain"] is not None, alpha_lr=fl.alpha_lr)
        sets.append((inp if i == 0 else None, d, fl, bl))
    return sets


def run_step(sets, i):
    _, _, fl, bl = sets[i % len(sets)]
    fl.run()
    bl.run()


def ramp(fn, ms):
    """Calls fn(i) until `ms` milliseconds of wall time have passed; returns the call count."""
    import torch
    t0 = time.perf_counter()
    i = 0
    while (time.perf_counter() - t0) * 1000.0 < ms:
        fn(i)
        i += 1
        if i % 16 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()
    return i


def kernel_bytes(w):
    """Algorithmic bytes per launch: forward 4TDE+4T, dq 5TDE+8T, dk/dv 6TDE+8T."""
    T, E = w.B * w.H * w.N, 2
    return {"dsqg_fwd": w.fwd_bytes(), "dsqg_bwd_dq": 5 * T * w.D * E + 8 * T,
            "dsqg_bwd_dkdv": 6 * T * w.D * E + 8 * T, "dsqg_bwd_params": None}


def time_fwd_bwd(sets, steps, warmup, stream):
    """W untimed steps, then K timed steps (median of per-step HIP events); then the per-kernel
    launch durations inside the step's own order (fwd, dq, dk/dv, params, rotating the sets),
    so every kernel meets the caches the step leaves it: a HIP event after each launch, median
    over the steps.  (A full backward runs the parameter reduction inside the dk/dv launch; here
    the phases are launched one by one.)  Returns (ms per step, {kernel: {us}}, wall ms)."""
    import torch
    for i in range(warmup):
        run_step(sets, i)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ms = _events_ms(lambda i: run_step(sets, i), steps, stream)
    wall = (time.perf_counter() - t0) * 1000.0 / steps
    torch.cuda.synchronize()
    names = ("dsqg_fwd", "dsqg_bwd_dq", "dsqg_bwd_dkdv", "dsqg_bwd_params")
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(len(names) + 1)] for _ in range(steps)]
    for i in range(steps):
        _, _, fl, bl = sets[i % len(sets)]
        ev[i][0].record(stream)
        fl.run()
        ev[i][1].record(stream)
        bl.run("dq")
        ev[i][2].record(stream)
        bl.run("dkdv")
        ev[i][3].record(stream)
        bl.run("params")
        ev[i][4].record(stream)
    torch.cuda.synchronize()
    per = {}
    for k, name in enumerate(names):
        us = statistics.median(ev[i][k].elapsed_time(ev[i][k + 1]) for i in range(steps)) * 1000.0
        per[name] = {"us": round(us, 3)}
    return ms, per, wall


def bench_d96(args, dev, stream):
    """The 85M condU trainer's attention call (train/train_2048_85m_condU.py:54,60-62,169): B8
    H8 N2048 D96, 44 offsets, same protocol as the headline step; plain, then with scale_embed
    and IF gain as the trainer's module passes them.  Each with its own fraction of the HBM
    roofline on its own compulsory step bytes, for comparison with the D = 64 step's."""
    from dwarf_amd.workloads import TRAINER_D96 as w
    step_bytes = w.fwd_bytes() + w.bwd_bytes()
    leg = {"workload": f"B{w.B} H{w.H} N{w.N} D{w.D} J{w.J} bf16 fwd+bwd (85M condU trainer)",
           "fwd_bwd_algorithmic_bytes": step_bytes}
    for name, se in (("plain", False), ("scale_embed", True)):
        sets = make_sets(w, dev, args.sets, scale_embed=se, if_gain=se)
        ramp(lambda i: run_step(sets, i), args.ramp_ms / 3)
        ms, per, _ = time_fwd_bwd(sets, args.steps, args.warmup, stream)
        leg[name] = {"ms_per_step": round(ms, 5), "tok_per_s": round(w.B * w.N / (ms * 1e-3), 1),
                     "fwd_bwd_frac_hbm_peak": round(step_bytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                     "kernels": per}
        print(f"[bench] D=96 leg ({name}) {ms:.4f} ms/step, "
              f"{leg[name]['fwd_bwd_frac_hbm_peak']:.3f} of HBM peak", file=sys.stderr, flush=True)
        del sets
    return leg


def bench_configs(args, dev, stream):
    """BASELINE's other training configurations (its parity cases; the metric is quoted on config
    2), same protocol as the headline step, each with its own fraction of the HBM roofline on
    its own compulsory step bytes: config 1 (B8 H8 N2048 D32, the 13M trainers' head dim) and
    config 3 (B4 H8 N4096 D64, 46 offsets, score gain and IF gain, whose gradients the step
    requests)."""
    from dwarf_amd.workloads import WORKLOADS
    legs = {}
    for c in (1, 3):
        w = WORKLOADS[c]
        step_bytes = w.fwd_bytes() + w.bwd_bytes()
        sets = make_sets(w, dev, args.sets)
        ramp(lambda i: run_step(sets, i), args.ramp_ms / 3)
        ms, per, _ = time_fwd_bwd(sets, args.steps, args.warmup, stream)
        legs[f"config_{c}"] = {
            "workload": f"config {c}: B{w.B} H{w.H} N{w.N} D{w.D} J{w.J} bf16 fwd+bwd"
                        + (" with score gain and IF gain" if c == 3 else ""),
            "fwd_bwd_algorithmic_bytes": step_bytes, "ms_per_step": round(ms, 5),
            "tok_per_s": round(w.B * w.N / (ms * 1e-3), 1),
            "fwd_bwd_frac_hbm_peak": round(step_bytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "kernels": per}
        print(f"[bench] config {c} leg {ms:.4f} ms/step, "
              f"{legs[f'config_{c}']['fwd_bwd_frac_hbm_peak']:.3f} of HBM peak",
              file=sys.stderr, flush=True)
        del sets
    return legs


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=200,
                    help="untimed steps first (the GPU clocks ramp during the first ~20 ms of work)")
    ap.add_argument("--config", type=int, default=2, choices=[1, 2, 3])
    ap.add_argument("--sets", type=int, default=3, help="input sets rotated between steps")
    ap.add_argument("--ramp-ms", type=float, default=150.0,
                    help="untimed steps for this long before the warm-up (GPU clock ramp)")
    ap.add_argument("--no-scale-embed-leg", action="store_true",
                    help="skip the leg with scale_embed and IF gain (the reference module's call)")
    ap.add_argument("--decode-steps", type=int, default=1000)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-decode", action="store_true")
    ap.add_argument("--no-d96-leg", action="store_true", help="skip the D = 96 trainer leg")
    ap.add_argument("--no-config-legs", action="store_true",
                    help="skip the config 1 and config 3 legs")
    ap.add_argument("--no-module", action="store_true", help="skip the drop-in module leg")
    ap.add_argument("--no-pool", action="store_true", help="skip the interference-pool leg")
    ap.add_argument("--no-generation", action="store_true", help="skip the generation leg")
    ap.add_argument("--profile-kernel", choices=["fwd", "dq", "dkdv", "decode", "pool"], default=None,
                    help="counter-collection mode: launch only this kernel --profile-reps times, "
                         "plus a plain device copy of --copy-mib MiB (the scale reference for "
                         "FETCH_SIZE / WRITE_SIZE; 'pool': its forward and backward, no copy), "
                         "then exit without a JSON line")
    ap.add_argument("--profile-reps", type=int, default=5)
    ap.add_argument("--profile-sets", type=int, default=1,
                    help="with --profile-kernel: input sets the launches rotate over")
    ap.add_argument("--profile-se", action="store_true",
                    help="with --profile-kernel: the scale_embed leg's inputs (scale_embed, if_gain)")
    ap.add_argument("--copy-mib", type=int, default=256)
    ap.add_argument("--decode-sweep", action="store_true",
                    help="time the decode step (8 ring pairs) at batch 32..512 and a trivial "
                         "graph-replayed kernel, print one JSON line and exit")
    ap.add_argument("--table-sweep", action="store_true",
                    help="time fwd, dq and dk/dv at the config-2 shape over four offset tables "
                         "(delta 0 alone, dense 0..32, delta 0 + 11 long-range, V3), print one "
                         "JSON line and exit")
    args = ap.parse_args(argv)

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py: this build measures one GPU only (--gpus {args.gpus}, WORLD_SIZE "
              f"{world} requested). DSQG shards over (batch, head) with no communication; "
              "multi-GPU runs are not part of this build.", file=sys.stderr)
        return 2

    import torch
    from dwarf_amd import ops
    from dwarf_amd.workloads import WORKLOADS, make_inputs

    if not torch.cuda.is_available():
        print("bench.py: no ROCm GPU visible", file=sys.stderr)
        return 1
    dev = torch.device("cuda:0")
    w = WORKLOADS[args.config]
    print(f"[bench] config {w.index}: B{w.B} H{w.H} N{w.N} D{w.D} J{w.J} {w.dtype}, "
          f"{args.sets} input sets, warmup {args.warmup}, steps {args.steps}", file=sys.stderr, flush=True)

    if args.profile_kernel:
        return profile_mode(args, w, dev)
    if args.decode_sweep:
        return decode_sweep(dev, args.decode_steps)
    if args.table_sweep:
        return table_sweep(dev)

    sets = make_sets(w, dev, args.sets)

    # GPU clock ramp: untimed steps until at least --ramp-ms of wall time have passed (the
    # clocks rise over the first tens of milliseconds of work), then the W warm-up steps.
    stream = torch.cuda.current_stream(dev)
    ramp_steps = ramp(lambda i: run_step(sets, i), args.ramp_ms)
    ms, per, wall = time_fwd_bwd(sets, args.steps, args.warmup, stream)
    print(f"[bench] fwd+bwd {ms:.4f} ms/step (wall {wall:.4f}; clock ramp {ramp_steps} steps)",
          file=sys.stderr, flush=True)
    nbytes_of = kernel_bytes(w)
    for name in per:
        if nbytes_of[name]:
            per[name]["algorithmic_bytes"] = nbytes_of[name]
            per[name]["achieved_GBs"] = round(nbytes_of[name] / (per[name]["us"] * 1e-6) / 1e9, 1)
        print(f"[bench] {name}: {per[name]['us']:.2f} us/launch", file=sys.stderr, flush=True)
    dom = max((k for k in per if "algorithmic_bytes" in per[k]), key=lambda k: per[k]["us"])
    achieved = per[dom]["achieved_GBs"]
    roofline = {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": measured_traffic(dom),
                "kernel": dom, "launch_us": per[dom]["us"],
                "algorithmic_bytes": per[dom]["algorithmic_bytes"]}

    step_bytes = w.fwd_bytes() + w.bwd_bytes()
    tok_s = w.B * w.N / (ms * 1e-3)
    result = {
        "metric": "DSQG fwd+bwd tok/s + % HBM peak (B8 H12 N2048 D64 bf16); decode tok/s",
        "value": round(tok_s, 1), "unit": "tok/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 5), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (seeded N(0,1)-based inputs per workload spec, 3 rotating sets)",
        "config": {"workload": f"config {w.index}: DSQG fwd+bwd B{w.B} H{w.H} N{w.N} D{w.D} "
                               f"J{w.J} bf16", "B": w.B, "H": w.H, "N": w.N, "D": w.D, "J": w.J},
        "fwd_bwd_algorithmic_bytes": step_bytes,
        "fwd_bwd_frac_hbm_peak": round(step_bytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        "roofline": roofline,
        "kernels": per,
    }
    if not args.no_scale_embed_leg:
        # The reference module's call (train/train_2048_condU.py:184,187): config-2 shapes with
        # scale_embed and IF gain, same protocol; its own step fraction of the HBM roofline.
        se_sets = make_sets(w, dev, args.sets, scale_embed=True, if_gain=True)
        ramp(lambda i: run_step(se_sets, i), args.ramp_ms / 3)
        se_ms, se_per, _ = time_fwd_bwd(se_sets, args.steps, args.warmup, stream)
        for name in se_per:
            if nbytes_of[name]:
                se_per[name]["achieved_GBs"] = round(nbytes_of[name] / (se_per[name]["us"] * 1e-6) / 1e9, 1)
        result["scale_embed_leg"] = {
            "workload": f"config {w.index} + scale_embed [J,D] ~ 0.05 N(0,1) + if_gain [H] ~ U(0.8,1.2)",
            "ms_per_step": round(se_ms, 5), "tok_per_s": round(w.B * w.N / (se_ms * 1e-3), 1),
            "fwd_bwd_frac_hbm_peak": round(step_bytes / (se_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "kernels": se_per}
        print(f"[bench] scale_embed leg {se_ms:.4f} ms/step", file=sys.stderr, flush=True)
        del se_sets
    if not args.no_d96_leg:
        result["d96_leg"] = bench_d96(args, dev, stream)
    if not args.no_config_legs and args.config == 2:
        result["config_legs"] = bench_configs(args, dev, stream)
    if not args.no_decode:
        result["decode"] = bench_decode(dev, args.decode_steps)
        print(f"[bench] decode {result['decode']['us_per_step']} us/step over "
              f"{result['decode']['layers']['ring_pairs']} ring pairs "
              f"(single ring {result['decode']['single_ring']['us_per_step']})",
              file=sys.stderr, flush=True)
    if not args.no_module:
        result["module"] = bench_module(dev)
        mres = result["module"]
        print(f"[bench] module QW fwd+bwd {mres['ms_per_step_strided_views']} ms "
              f"(with permute copies {mres['ms_per_step_contiguous_copies']} ms, with K/V "
              f"injection {mres['ms_module_with_kv_inject']} ms; injection adds alone "
              f"{mres['ms_kv_inject_adds']} ms, gate multiply alone {mres['ms_gate_multiply']} ms)",
              file=sys.stderr, flush=True)
    if not args.no_pool:
        result["pool"] = bench_pool(dev)
        print(f"[bench] pool fwd {result['pool']['fwd']['us']} us, bwd "
              f"{result['pool']['bwd']['us']} us", file=sys.stderr, flush=True)
    if not args.no_generation:
        result["generation"] = bench_generation(dev)
        g = result["generation"]
        print(f"[bench] generation {g['tok_per_s_incremental']} tok/s incremental, "
              f"{g['tok_per_s_full_recompute']} tok/s full recompute", file=sys.stderr, flush=True)
    if not args.no_cpu_baseline:
        print("[bench] timing the CPU oracle sample ...", file=sys.stderr, flush=True)
        result["cpu_baseline"] = cpu_baseline(w, sets[0][0])
        if "decode" in result:
            result["decode"]["cpu_baseline"] = cpu_baseline_decode()
    else:
        result["cpu_baseline"] = None
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
