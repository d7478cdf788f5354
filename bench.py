"""Benchmark of the quantized indexed-MoE hot path on one MI355X.

    python bench.py [--gpus 1] [--steps 50] [--warmup 5]

Workload (0-indexed):
  decode  C1: Laguna-shaped MoE layer, batch 1 (H=4096, FF=1536, 256 experts,
          top-10 + shared, gate/up Q4_K, down Q6_K).  One step = one forward
          (router + 10 routed experts + shared expert + combine) of each of
          --layers distinct seeded layers (>= 1 GB of touched weights per step,
          so the 256 MB Infinity Cache cannot serve repeats); the step is
          captured once as a HIP graph and replayed, exactly --steps times.
  prefill C3: the same layer at t = 2048 with a skewed selection bias (grouped
          expert GEMM), reported as TFLOP/s.
`value` is decode HBM throughput: algorithmic bytes (each touched weight byte
once per step, plus router, bias, x and out) / time per step, inputs resident in
HBM.  Weights are synthetic (seeded generator), no checkpoint is loaded.
Progress goes to stderr; stdout carries exactly one JSON line.
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0
METRIC = "batch-1 MoE layer µs + achieved HBM GB/s; prefill-2048 MoE TFLOP/s (1 GPU)"


def measured_traffic():
    """Calibrated HBM bytes per launch of the decode kernels, from the committed
    rocprofv3 PMC summary (FETCH_SIZE / WRITE_SIZE passes); {} when absent."""
    path = ROOT / "profiles" / "decode_c1_hbm_traffic.md"
    try:
        text = path.read_text()
        block = text.split("```json", 1)[1].split("```", 1)[0]
        return json.loads(block)["traffic_bytes"]
    except (OSError, IndexError, KeyError, ValueError):
        return {}


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def layer_bytes(spec, ids_np, t):
    """Algorithmic bytes of one forward: each touched expert once, shared, router, bias, x, out."""
    uniq = len(set(int(e) for e in ids_np.ravel()))
    eb = spec.expert_bytes()
    return (uniq * eb + (eb if spec.shared else 0) + spec.hidden * spec.n_expert * 4 + spec.n_expert * 4
            + 2 * t * spec.hidden * 4), uniq


def layer_flops(spec, t):
    pairs = t * spec.top_k
    per_pair = 2 * (2 * spec.ff * spec.hidden + spec.hidden * spec.ff)
    shared = t * per_pair if spec.shared else 0
    return pairs * per_pair + shared + 2 * t * spec.hidden * spec.n_expert


def profiled(block, x, out, t, n_max=16):
    from maxuna_amd._lib import check, lib
    from maxuna_amd import ops
    import torch
    ws = block.workspace(t, x.device)
    ids = torch.empty((t, block.cfg.n_expert_used), dtype=torch.uint32, device=x.device)
    w = torch.empty((t, block.cfg.n_expert_used), dtype=torch.float32, device=x.device)
    stage = (C.c_float * n_max)()
    n = C.c_int32(0)
    check(lib().mx_moe_forward_profiled(C.byref(block._c), x.data_ptr(), t, None, out.data_ptr(), ids.data_ptr(),
                                        w.data_ptr(), ws.data_ptr(), ws.numel(), ops._stream(), stage, n_max,
                                        C.byref(n)))
    return [stage[i] for i in range(n.value)]


def forward_repeat(block, x, out, stage, times):
    """One layer forward with decode stage `stage` launched `times` times (0: skipped; capturable)."""
    from maxuna_amd._lib import check, lib
    from maxuna_amd import ops
    ws = block.workspace(1, x.device)
    check(lib().mx_moe_forward_repeat(C.byref(block._c), x.data_ptr(), 1, None, out.data_ptr(), None, None,
                                      ws.data_ptr(), ws.numel(), ops._stream(), stage, times))


def read_probe():
    """Plain streaming reads (mx_probe_read) of the C1 expert kernels' byte counts and
    larger ones, each launch on a different region of a 4 GiB pool (no cache
    reuse), 40 launches per captured graph: the achievable HBM read rate."""
    import torch
    from maxuna_amd._lib import check, lib
    from maxuna_amd import ops
    pool = torch.empty(4 << 30, dtype=torch.uint8, device="cuda").fill_(1)
    sink = torch.zeros(1, dtype=torch.int32, device="cuda")
    sizes = {"router (4 MB)": 4 << 20, "C1 down (57 MB)": 56854528, "C1 gate/up (78 MB)": 77873152,
             "C1 layer (135 MB)": 134727680, "512 MiB": 512 << 20}
    for name, n in sizes.items():
        n -= n % 16
        slots = min(40, (4 << 30) // n)

        def launches():
            for r in range(40):
                check(lib().mx_probe_read(pool.data_ptr() + (r % slots) * n, n, sink.data_ptr(), ops._stream()))
        us = graph_us(launches, 3) / 40
        log(f"read probe {name}: {us:.2f} us per read, {n / (us * 1e-6) / 1e9:.0f} GB/s")


def library_gemm():
    """The vendor library's f16 GEMMs (torch.mm -> hipBLASLt) on the C3 prefill's own
    shapes: the per-expert row counts of the C3 layer's routing (routed experts + the
    shared expert's 2048 rows), gate+up [m x 4096] x [4096 x 3072] and down
    [m x 1536] x [1536 x 4096] per expert, plus one GEMM over all 22,528 rows.  Plain
    f16 operands (no dequantisation, no gather): what a library GEMM reaches on this
    work, next to the quantised grouped GEMM's figures."""
    import torch
    from maxuna_amd.synth import CONFIGS, build_layer, make_x
    spec = CONFIGS["C3"]["spec"]
    t = 2048
    layer = build_layer(spec, seed=5151)
    x = torch.from_numpy(make_x(spec, 88, t)).cuda()
    _, ids, _ = layer.block.forward(x, return_routing=True)
    cnt = torch.bincount(ids.view(torch.int32).long().flatten(), minlength=spec.n_expert)
    rows = [int(c) for c in cnt.tolist() if c > 0] + ([t] if spec.shared else [])
    del layer
    h, ff = spec.hidden, spec.ff
    g = torch.Generator(device="cuda").manual_seed(7)
    def rnd(*shape):
        return torch.randn(*shape, device="cuda", dtype=torch.float16, generator=g)
    wgu = [rnd(2 * ff, h) for _ in rows]
    wdn = [rnd(h, ff) for _ in rows]
    agu = [rnd(m, h) for m in rows]
    adn = [rnd(m, ff) for m in rows]
    ogu = [torch.empty(m, 2 * ff, device="cuda", dtype=torch.float16) for m in rows]
    odn = [torch.empty(m, h, device="cuda", dtype=torch.float16) for m in rows]
    big_a = rnd(sum(rows), h)
    big_o = torch.empty(sum(rows), 2 * ff, device="cuda", dtype=torch.float16)

    def timed(fn, reps=10):
        for _ in range(3):
            fn()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        start.record()
        for _ in range(reps):
            fn()
        end.record()
        torch.cuda.synchronize()
        return start.elapsed_time(end) * 1e3 / reps

    n = sum(rows)
    fl_gu, fl_dn = 2 * n * 2 * ff * h, 2 * n * ff * h
    us = timed(lambda: [torch.mm(a, w.t(), out=o) for a, w, o in zip(agu, wgu, ogu)])
    log(f"library f16 GEMM gate+up, {len(rows)} experts (rows {min(rows)}..{max(rows)}, {n} total): "
        f"{us:.0f} us, {fl_gu / us / 1e6:.0f} TFLOP/s")
    us = timed(lambda: [torch.mm(a, w.t(), out=o) for a, w, o in zip(adn, wdn, odn)])
    log(f"library f16 GEMM down, per expert: {us:.0f} us, {fl_dn / us / 1e6:.0f} TFLOP/s")
    us = timed(lambda: torch.mm(big_a, wgu[0].t(), out=big_o))
    log(f"library f16 GEMM gate+up as one [{n} x {h}] x [{h} x {2 * ff}]: {us:.0f} us, "
        f"{fl_gu / us / 1e6:.0f} TFLOP/s")


def graph_us(fn, replays):
    """Average time of one replay of the graph captured from fn(), us."""
    import torch
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    for _ in range(3):
        g.replay()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    for _ in range(replays):
        g.replay()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) * 1e3 / replays


def bench_decode(args):
    import numpy as np
    import torch
    from maxuna_amd.synth import CONFIGS, build_layer, make_x

    spec = CONFIGS["C1"]["spec"]
    L = args.layers
    log(f"decode: building {L} C1 layers ({L * spec.n_expert * spec.expert_bytes() / 1e9:.1f} GB of experts)")
    layers = [build_layer(spec, seed=4242, layer=i) for i in range(L)]
    xs = [torch.from_numpy(make_x(spec, 77, 1, layer=i)).cuda() for i in range(L)]
    outs = [torch.empty_like(x) for x in xs]
    for i in range(max(args.warmup, L)):
        layers[i % L].block.forward(xs[i % L], out=outs[i % L])
    torch.cuda.synchronize()
    # routing of each layer (fixed inputs -> fixed experts)
    tot_bytes = 0
    uniq = []
    for i in range(L):
        _, ids, _ = layers[i].block.forward(xs[i], return_routing=True)
        b, u = layer_bytes(spec, ids.view(torch.int32).cpu().numpy(), 1)
        tot_bytes += b
        uniq.append(u)
    bytes_per_layer = tot_bytes / L
    # capture the rotation once; one step = one replay (one forward of each of the
    # L layers), so K steps time K * L layer forwards
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(L):
            layers[i].block.forward(xs[i], out=outs[i])
    warm = max(args.warmup, -(-30 // L))  # at least 30 layer forwards before timing
    for _ in range(warm):
        g.replay()
    steps = args.steps
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    start.record()
    for _ in range(steps):
        g.replay()
    end.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_step = start.elapsed_time(end) / steps
    ms = ms_step / L
    gbs = bytes_per_layer / (ms * 1e-3) / 1e9
    log(f"decode: {steps} steps x {L} layers, {ms * 1e3:.2f} us/layer, {gbs:.0f} GB/s (wall {wall * 1e3:.1f} ms)")
    replays = max(steps, 8)
    # per-kernel time inside the replayed pipeline: the plain rotation minus the
    # rotation with one stage's kernel left out (HIP events on the stream).  Leaving
    # a launch out, unlike launching it twice, keeps every weight byte an HBM read.
    # (base and skip graphs measured alternately three times, the median of the
    # differences: single pairs moved by 1-2 us from run to run)
    reps = max(32, replays)
    base_fn = lambda: [forward_repeat(layers[i].block, xs[i], outs[i], -1, 1) for i in range(L)]  # noqa: E731
    st = []
    for stage in range(4):
        skip_fn = lambda: [forward_repeat(layers[i].block, xs[i], outs[i], stage, 0) for i in range(L)]  # noqa: E731
        diffs = [graph_us(base_fn, reps) - graph_us(skip_fn, reps) for _ in range(3)]
        st.append(float(np.median(diffs)) / L * 1e-3)  # ms per launch
    # eager per-stage HIP events (include the dispatch gap before each kernel)
    eager = np.array([profiled(layers[r % L].block, xs[r % L], outs[r % L], 1)
                      for r in range(max(1, args.profile_iters))]).mean(0)
    log("decode stage us (graph, differential): " + ", ".join(f"{v * 1e3:.2f}" for v in st)
        + "; eager events: " + ", ".join(f"{v * 1e3:.2f}" for v in eager))
    eb_gu = 2 * spec.ff * (spec.hidden // 256) * 144
    eb_dn = spec.hidden * (spec.ff // 256) * 210
    k = spec.top_k
    gu_bytes = (k + 1) * eb_gu + spec.hidden * 4  # routed + shared gate/up
    dn_bytes = (k + 1) * eb_dn + (k + 1) * spec.ff * 4 + spec.hidden * 4
    kern = {"k_decode_gate_up (routed + shared)": (st[2], gu_bytes), "k_decode_down": (st[3], dn_bytes)}
    dom = max(kern, key=lambda n: kern[n][0])
    dms, dbytes = kern[dom]
    roof = {"bound": "hbm", "kernel": dom, "achieved": round(dbytes / (dms * 1e-3) / 1e9, 1), "peak": HBM_PEAK_GBS,
            "unit": "GB/s", "frac": round(dbytes / (dms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "traffic": measured_traffic().get(dom), "bytes_per_launch": dbytes, "launch_us": round(dms * 1e3, 2)}
    stage_us = {"route_logits": st[0] * 1e3, "topk": st[1] * 1e3, "gate_up": st[2] * 1e3,
                "down": st[3] * 1e3, "eager_events": [round(v * 1e3, 2) for v in eager]}
    return dict(ms_per_layer=ms, ms_per_step=ms_step, steps=steps, warm_layers=warm * L, gbs=gbs,
                bytes_per_layer=bytes_per_layer, bytes_per_step=bytes_per_layer * L, uniq=uniq,
                stage_us=stage_us, roofline=roof, layers=layers)


def bench_prefill(args):
    import numpy as np
    import torch
    from maxuna_amd.synth import CONFIGS, build_layer, make_x

    spec = CONFIGS["C3"]["spec"]
    t = 2048
    log("prefill: building the C3 layer")
    layer = build_layer(spec, seed=5151)
    x = torch.from_numpy(make_x(spec, 88, t)).cuda()
    out = torch.empty_like(x)
    for _ in range(2):
        layer.block.forward(x, out=out)
    _, ids, _ = layer.block.forward(x, return_routing=True)
    torch.cuda.synchronize()
    nbytes, uniq = layer_bytes(spec, ids.view(torch.int32).cpu().numpy(), t)
    flops = layer_flops(spec, t)
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(args.prefill_steps):
        layer.block.forward(x, out=out)
    end.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / args.prefill_steps
    st = np.array([profiled(layer.block, x, out, t) for _ in range(3)]).mean(0)
    names = ["route", "map0", "x_f16", "gate_up_gemm", "act_f16", "down_gemm", "combine"]
    stage_us = {n: round(v * 1e3, 1) for n, v in zip(names, st)}
    log("prefill stage us (eager events): " + ", ".join(f"{n} {v}" for n, v in stage_us.items()))
    kk = spec.top_k + (1 if spec.shared else 0)
    gu_flops = 2 * 2 * t * kk * spec.ff * spec.hidden
    dn_flops = 2 * t * kk * spec.hidden * spec.ff
    gemms = {"k_gemm gate/up (SwiGLU)": (st[3], gu_flops), "k_gemm down": (st[5], dn_flops)}
    dom = max(gemms, key=lambda n: gemms[n][0])
    tf = gemms[dom][1] / (gemms[dom][0] * 1e-3) / 1e12
    log(f"prefill: {ms:.3f} ms/layer, {flops / (ms * 1e-3) / 1e12:.1f} TFLOP/s, {dom} {tf:.1f} TFLOP/s")
    return dict(ms=ms, tflops=flops / (ms * 1e-3) / 1e12, gbs=nbytes / (ms * 1e-3) / 1e9, flops=flops,
                bytes=nbytes, uniq=uniq, stage_us=stage_us,
                gate_gemm={"bound": "mfma", "kernel": dom, "achieved": round(tf, 1), "peak": MFMA_F16_PEAK_TFLOPS,
                           "unit": "TFLOP/s", "frac": round(tf / MFMA_F16_PEAK_TFLOPS, 4),
                           "flops_per_launch": gemms[dom][1], "launch_us": round(gemms[dom][0] * 1e3, 1)},
                tokens_per_s=t / (ms * 1e-3))


def bench_verify(args, dec):
    """C2: the speculative-verify block (t = 16) on the decode layers' rotation.
    Bytes count each expert touched by any of the 16 tokens once."""
    import torch
    from maxuna_amd.synth import CONFIGS, make_x

    spec = CONFIGS["C2"]["spec"]
    t = CONFIGS["C2"]["t"]
    layers = dec["layers"]
    L = len(layers)
    xs = [torch.from_numpy(make_x(spec, 99, t, layer=i)).cuda() for i in range(L)]
    outs = [torch.empty_like(x) for x in xs]
    tot, uniq = 0, []
    for i in range(L):
        _, ids, _ = layers[i].block.forward(xs[i], return_routing=True)
        b, u = layer_bytes(spec, ids.view(torch.int32).cpu().numpy(), t)
        tot += b
        uniq.append(u)
    us = graph_us(lambda: [layers[i].block.forward(xs[i], out=outs[i]) for i in range(L)],
                  max(8, args.steps // 2)) / L
    gbs = tot / L / (us * 1e-6) / 1e9
    log(f"verify C2 (t={t}): {us:.1f} us/block, {gbs:.0f} GB/s, {sum(uniq) / L:.0f} unique experts")
    return {"workload": "C2 verify block, t=16, top-10 of 256 + shared", "us_per_block": round(us, 2),
            "tokens_per_s": round(t / (us * 1e-6), 1), "hbm_gbs": round(gbs, 1),
            "hbm_frac": round(gbs / HBM_PEAK_GBS, 4), "bytes_per_block": int(tot / L),
            "unique_experts": round(sum(uniq) / L, 1)}


def bench_chain(args):
    """C4: one decode step through 48 MoE layers, x <- x + MoE(RMSNorm(x)),
    every layer with its own weights (about 150 GB resident in HBM)."""
    import torch
    from maxuna_amd.synth import CONFIGS, build_layer, make_x

    spec = CONFIGS["C4"]["spec"]
    n = CONFIGS["C4"]["layers"]
    log(f"chain: building {n} C1 layers ({n * spec.n_expert * spec.expert_bytes() / 1e9:.0f} GB of experts)")
    layers = [build_layer(spec, seed=4848, layer=i, rms=True) for i in range(n)]
    x0 = torch.from_numpy(make_x(spec, 48, 1)).cuda()
    x = x0.clone()
    tot = 0
    for lay in layers:  # routing of one pass, for the byte count (RMSNorm weights included)
        xin = x.clone()
        _, ids, _ = lay.block.forward(xin, residual=x, out=x, return_routing=True)
        tot += layer_bytes(spec, ids.view(torch.int32).cpu().numpy(), 1)[0] + spec.hidden * 4
    x.copy_(x0)

    def step():
        for lay in layers:
            lay.block.forward(x, residual=x, out=x)

    us = graph_us(step, max(5, args.steps // 10))
    gbs = tot / (us * 1e-6) / 1e9
    log(f"chain C4: {us / 1e3:.3f} ms/step over {n} layers, {gbs:.0f} GB/s")
    del layers
    torch.cuda.empty_cache()
    return {"workload": "C4 48-layer MoE-only decode step (RMSNorm eps 1e-6, weight 1; residual)",
            "ms_per_step": round(us / 1e3, 4), "tokens_per_s": round(1e6 / us, 1), "hbm_gbs": round(gbs, 1),
            "hbm_frac": round(gbs / HBM_PEAK_GBS, 4), "bytes_per_step": int(tot)}


def bench_lm_head(args):
    """Plain quantised mat-vec at the lm_head shape: Q6_K [100352 x 3072], t = 1,
    over 4 distinct weight copies (1 GB, so the Infinity Cache cannot serve repeats)."""
    import torch
    from maxuna_amd import ops
    from maxuna_amd.gguf import GgmlDType
    from maxuna_amd.synth import synth_stack

    n_out, k, copies = 100352, 3072, 4
    ws = [synth_stack(GgmlDType.Q6_K, 1, n_out, k, key=9000 + i) for i in range(copies)]
    x = torch.randn(1, k, device="cuda")
    us = graph_us(lambda: [ops.mul_mv(w.buffer, GgmlDType.Q6_K, n_out, k, x) for w in ws],
                  max(16, args.steps)) / copies
    nbytes = ws[0].nbytes + k * 4 + n_out * 4
    gbs = nbytes / (us * 1e-6) / 1e9
    log(f"lm_head Q6_K [{n_out} x {k}]: {us:.1f} us, {gbs:.0f} GB/s")
    return {"workload": "plain mat-vec Q6_K [100352 x 3072], t=1 (mul_mv, lm_head shape)", "us": round(us, 2),
            "hbm_gbs": round(gbs, 1), "hbm_frac": round(gbs / HBM_PEAK_GBS, 4), "bytes": int(nbytes)}


def t_sweep(ts, replays=20):
    """C1-shaped layers (C2's routing spread) at other block sizes: 4 distinct
    layers replayed as one graph per t, µs per layer forward.  Which kernels run
    depends on t: the 16-pair MFMA tiles up to 2560 (token, slot) pairs, the
    grouped GEMM beyond."""
    import torch
    from maxuna_amd.synth import CONFIGS, build_layer, make_x

    spec = CONFIGS["C2"]["spec"]
    layers = [build_layer(spec, seed=1002, layer=i) for i in range(4)]
    out = {}
    for t in ts:
        xs = [torch.from_numpy(make_x(spec, 99, t, layer=i)).cuda() for i in range(4)]
        ys = [torch.empty_like(x) for x in xs]
        us = graph_us(lambda: [layers[i].block.forward(xs[i], out=ys[i]) for i in range(4)], replays) / 4
        slots = spec.top_k + 1
        path = "tiles" if t >= 16 and t * slots <= 2560 else ("grouped GEMM" if t >= 32 else "decode")
        log(f"t-sweep t={t}: {us:.1f} us/layer ({path})")
        out[t] = round(us, 1)
    return out


def cpu_model() -> str:
    try:
        for ln in open("/proc/cpuinfo"):
            if ln.startswith("model name"):
                return ln.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(args, dec):
    """The CPU oracle (C restatement of the reference expert path, OpenMP) on a
    bounded sample of the decode workload: C1 layers, t = 1."""
    import numpy as np
    import torch
    from oracle import oracle as orc

    lyr = dec["layers"]
    spec = lyr[0].spec
    H, FF, E = spec.hidden, spec.ff, spec.n_expert
    gdt, ddt = int(spec.gate_dt), int(spec.down_dt)
    from maxuna_amd.synth import make_x
    samples = []
    for li in range(min(2, len(lyr))):
        L = lyr[li]
        x = make_x(spec, 77, 1, layer=li)
        logits = orc.route_logits(x, L.router_t)
        ids, w = orc.route_from_logits(logits, L.bias, spec.top_k, 1.0, True)
        sel = sorted(set(int(e) for e in ids.ravel()))
        g = {e: orc.expert_blocks(gdt, L.keys["gate_exps"], e, FF, H) for e in sel}
        u = {e: orc.expert_blocks(gdt, L.keys["up_exps"], e, FF, H) for e in sel}
        d = {e: orc.expert_blocks(ddt, L.keys["down_exps"], e, H, FF) for e in sel}
        sh = [orc.expert_blocks(gdt, L.keys["gate_shexp"], 0, FF, H), orc.expert_blocks(gdt, L.keys["up_shexp"], 0, FF, H),
              orc.expert_blocks(ddt, L.keys["down_shexp"], 0, H, FF)]
        samples.append((x, L, g, u, d, sh))
    reps, t0 = 0, time.perf_counter()
    while True:
        x, L, g, u, d, sh = samples[reps % len(samples)]
        logits = orc.route_logits(x, L.router_t)
        ids, w = orc.route_from_logits(logits, L.bias, spec.top_k, 1.0, True)
        orc.reference_experts(gdt, g, gdt, u, ddt, d, E, H, FF, x, ids, w)
        orc.swiglu(gdt, sh[0], gdt, sh[1], ddt, sh[2], H, FF, x)
        reps += 1
        el = time.perf_counter() - t0
        if el > args.cpu_seconds or reps >= 200:
            break
    s_per = el / reps
    gbs = dec["bytes_per_layer"] / s_per / 1e9
    log(f"cpu baseline: {reps} layers in {el:.1f} s -> {s_per * 1e3:.1f} ms/layer, {gbs:.2f} GB/s")
    return {"value": round(gbs, 3), "unit": "GB/s", "cores": orc.lib().or_num_threads(), "kind": "port",
            "cpu_model": cpu_model(),
            "sample": f"{reps} C1 decode layers (t=1; routing + 10 routed experts + shared; selected experts "
                      f"pre-generated), {s_per * 1e6:.0f} us/layer",
            "us_per_layer": round(s_per * 1e6, 1)}


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50,
                    help="timed steps; one step = one forward of each of the --layers decode layers")
    ap.add_argument("--warmup", type=int, default=5, help="untimed steps first (at least 30 layer forwards)")
    ap.add_argument("--layers", type=int, default=8, help="distinct decode layers in the rotation")
    ap.add_argument("--prefill-steps", type=int, default=10)
    ap.add_argument("--profile-iters", type=int, default=32)
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--no-decode", action="store_true", help="prefill only (profiling); prints no JSON line")
    ap.add_argument("--no-extra", action="store_true", help="skip the C2 verify, C4 chain and lm_head figures")
    ap.add_argument("--no-chain", action="store_true", help="skip the C4 chain and lm_head figures (keep C2)")
    ap.add_argument("--read-probe", action="store_true",
                    help="only time plain streaming reads of the expert kernels' sizes (achievable HBM read rate)")
    ap.add_argument("--lm-head", action="store_true",
                    help="only time the plain Q6_K mat-vec at the lm_head shape (profiling)")
    ap.add_argument("--library-gemm", action="store_true",
                    help="only time the vendor library's f16 GEMMs on the C3 prefill's per-expert shapes")
    ap.add_argument("--t-sweep", type=str, default="",
                    help="only time C1-shaped layers at these comma-separated block sizes (tokens)")
    ap.add_argument("--copy-probe-mb", type=int, default=0,
                    help="only run N device-to-device copies of this many MB (HBM counter calibration) and exit")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (expert-parallel sharding is "
              "a design note only); run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    import torch
    torch.cuda.set_device(0)
    if args.read_probe:
        read_probe()
        return
    if args.library_gemm:
        library_gemm()
        return
    if args.lm_head:
        bench_lm_head(args)
        return
    if args.t_sweep:
        t_sweep([int(v) for v in args.t_sweep.split(",")])
        return
    if args.copy_probe_mb:
        # a plain copy of known size: FETCH_SIZE / WRITE_SIZE of its dispatches calibrate
        # the counters that give the decode kernels' HBM traffic
        n = args.copy_probe_mb * (1 << 20)
        src = torch.empty(n, dtype=torch.uint8, device="cuda").fill_(1)
        dst = torch.empty_like(src)
        for _ in range(4):
            dst.copy_(src)
        torch.cuda.synchronize()
        log(f"copy probe: 4 x {n} bytes")
        return
    if args.no_decode:
        bench_prefill(args)
        return
    dec = bench_decode(args)
    ver = None if args.no_extra else bench_verify(args, dec)
    pre = None if args.no_prefill else bench_prefill(args)
    cpu = None if args.no_cpu_baseline else cpu_baseline(args, dec)
    extra = {}
    if not args.no_extra and not args.no_chain:
        extra["lm_head"] = bench_lm_head(args)
        del dec["layers"]
        torch.cuda.empty_cache()
        extra["chain"] = bench_chain(args)
    line = {
        "metric": METRIC,
        "value": round(dec["gbs"], 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": dec["steps"],
        "warmup": args.warmup,
        "ms_per_step": round(dec["ms_per_step"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q4_K/q6_K weight blocks; activations on a 24-bit grid per 128-value block (power-of-two "
                 "scale, three int8 digit planes, exact int32 plane sums on v_dot4_i32_i8, Q6_K part sums scaled "
                 "in int32) recombined and scaled in f32, f32 accumulation",
        "data": "synthetic (seeded GGUF blocks generated on device; x, router ~ N(0,1), N(0,0.02))",
        "config": {"workload": f"C1 decode MoE layer, batch 1; one step = one forward of each of {args.layers} "
                               "distinct C1 layers (graph replay)",
                   "hidden": 4096, "expert_ff": 1536,
                   "n_expert": 256, "top_k": 10, "shared_expert": True, "quant": "gate/up Q4_K, down Q6_K",
                   "rotation_layers": args.layers, "graph_replay": True},
        "layer_forwards_timed": dec["steps"] * args.layers,
        "warmup_layer_forwards": dec["warm_layers"],
        "us_per_layer": round(dec["ms_per_layer"] * 1e3, 2),
        "tokens_per_s": round(1e3 / dec["ms_per_layer"], 1),
        "bytes_per_layer": int(dec["bytes_per_layer"]),
        "bytes_per_step": int(dec["bytes_per_step"]),
        "hbm_frac": round(dec["gbs"] / HBM_PEAK_GBS, 4),
        "decode_stage_us": {k: (round(v, 2) if isinstance(v, float) else v) for k, v in dec["stage_us"].items()},
        "roofline": dec["roofline"],
    }
    if pre:
        line["prefill"] = {"workload": "C3 prefill t=2048, skewed bias", "ms_per_layer": round(pre["ms"], 4),
                           "tflops": round(pre["tflops"], 2), "mfma_frac": round(pre["tflops"] / MFMA_F16_PEAK_TFLOPS, 4),
                           "hbm_gbs": round(pre["gbs"], 1), "tokens_per_s": round(pre["tokens_per_s"], 1),
                           "flops": pre["flops"], "bytes": pre["bytes"], "experts_touched": pre["uniq"],
                           "stage_us": pre["stage_us"], "roofline": pre["gate_gemm"]}
    if ver:
        line["verify"] = ver
    line.update(extra)
    if cpu:
        line["cpu_baseline"] = cpu
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
