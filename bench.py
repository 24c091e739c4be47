"""Benchmark: Block-RVQ decode GEMV at Llama-3-8B shapes (configuration c3).

A step is one decode token (M = 1 by default) through every compressed linear
of a 32-layer Llama-3-8B stack: per layer q/k/v/o (4096 or 1024 x 4096),
gate/up (14336 x 4096) and down (4096 x 14336), each a single-stage Block-RVQ
layer with a 4096-entry fp16 codebook, 16-bit indices and an fp16 scale shared
by 128-row groups, bf16 activations.  Weights are seeded random (synthetic,
no checkpoint); all 224 linears live in HBM at once (1.76 GB of indices), so
every step streams cold compressed bytes.  Linears of a layer that read the
same activation run as one launch (q/k/v, gate/up: FusedBlockRVQLinears), the
others one launch each; the drop-in step with one launch per linear is timed
too and reported as config.unfused_tok_s.  Each step is captured in a HIP
graph and replayed; the timed region is exactly --steps replays.

Prints one JSON line (metric, value in tok/s, roofline of the dominant kernel
measured live with HIP events, CPU baseline of the reference's per_group op
sequence timed on this host's cores).

  python bench.py [--gpus 1] [--steps K] [--warmup W] [--config c3] [--m 1]

With --config c4 (M = 2048, two-stage 256-entry codebooks, uint8 indices) the
same stack runs the prefill path instead and the roofline is the bf16 MFMA
one: algorithmic flops (2 M N K per linear) of the dominant launch over its
measured duration, against the 2.5 PFLOP/s dense peak.  Where its cost
model finds it faster (at M = 2048 for every launch) the torch operator runs
a launch as two passes (the dense weight, then torch's GEMM); the roofline
then also carries the fused prefill kernel's own figures (`fused_kernel`,
measured with WAL2026_PREFILL_TWO_PASS=0).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import torch

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

from wal2026_amd import (FusedBlockRVQLinears, PackedGroupedBlockRVQLinear, _lib, fuse_sibling_linears,  # noqa: E402
                         synth, unfuse_sibling_linears)

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E
# linears of a layer that read the same activation, fused into one launch
FUSION_GROUPS = (("qkv", ("q_proj", "k_proj", "v_proj")), ("gate_up", ("gate_proj", "up_proj")))
BF16_PEAK_TFLOPS = 2500.0      # MI355X dense bf16 MFMA


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def build_stack(cfg: synth.Config, dev: torch.device, layers: int):
    gen = synth.generator(0, dev)
    stack = []
    for _ in range(layers):
        layer = {}
        for name, n, k in cfg.shapes():
            enc = synth.make_encoding(n, k, cfg, gen, dev)
            layer[name] = PackedGroupedBlockRVQLinear(enc, matmul_strategy="hip_block_rvq").to(dev)
        stack.append(layer)
    return stack


def linear_bytes(cfg: synth.Config, n: int, k: int) -> int:
    """Algorithmic compressed bytes of one linear: ids + codebooks + scales."""
    B = -(-k // cfg.block_size)
    G = 1 if cfg.group_rows is None else -(-n // cfg.group_rows)
    ib = torch.empty(0, dtype=cfg.ids_dtype()).element_size()
    return cfg.num_stages * n * B * ib + G * cfg.num_stages * cfg.codebook_size * cfg.block_size * 2 + n * 2


def graph_launch_us(fns, reps: int = 5) -> float:
    """Average GPU duration (us) of one launch among `fns` (one per layer, so
    each reads weights the previous one did not): the launches are captured in
    one HIP graph, replayed `reps` times between two HIP events recorded on the
    stream the graph runs on, and the elapsed time is divided by the launches
    run.  Inside a graph the launches follow each other with no host gap and no
    event between them, so this agrees with the profiler's per-dispatch
    durations (an event pair around each eager launch adds the dispatch
    latency of the command processor to every one)."""
    for f in fns:
        f()  # descriptors, codebook images and allocations outside the graph
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for f in fns:
            f()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for f in fns:
            f()
    torch.cuda.synchronize()
    for _ in range(2):
        graph.replay()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record(stream)
    for _ in range(reps):
        graph.replay()
    b.record(stream)
    torch.cuda.synchronize()
    return a.elapsed_time(b) * 1000.0 / (len(fns) * reps)


def traffic_bytes(path: str):
    """HBM bytes per launch of the dominant kernel from a committed rocprofv3
    --pmc summary (FETCH_SIZE + WRITE_SIZE, already scaled by the copy-kernel
    calibration factor the summary states); None when there is none."""
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return int(float(line.split(":", 1)[1]))
    except OSError:
        pass
    return None


def cpu_baseline(cfg: synth.Config, budget_s: float = 20.0) -> dict:
    """The reference's default per_group op sequence (oracle/ref_ops.py) on
    this host's cores, over one layer's linears; tok/s extrapolated to the
    whole stack."""
    from oracle import ref_ops

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    gen = synth.generator(0)
    layer = []
    for name, n, k in cfg.shapes():
        enc = synth.make_encoding(n, k, cfg, gen)
        groups = [dict(stage_ids=list(g.stage_ids), codebooks=list(g.codebooks), row_scale=g.row_scale.to(torch.float16),
                       in_features=k) for g in enc.groups]
        x = synth.make_activation(cfg.m, k, cfg.x_dtype, gen)
        layer.append((groups, enc.row_slices, n, x))

    def one_layer():
        for groups, slices, n, x in layer:
            ref_ops.per_group_forward(x, groups, slices, n)

    one_layer()  # warmup
    reps = 0
    t0 = time.perf_counter()
    while True:
        one_layer()
        reps += 1
        if time.perf_counter() - t0 > budget_s / 2 or reps >= 3:
            break
    per_layer = (time.perf_counter() - t0) / reps
    return {
        "value": round(cfg.m / (per_layer * cfg.layers), 4),
        "unit": "tok/s",
        "cores": cores,
        "kind": "port",
        "sample": f"1 of {cfg.layers} layers ({len(cfg.shapes())} linears, M={cfg.m}), per_group torch op sequence "
                  f"(oracle/ref_ops.py), {reps} reps after 1 warmup; {per_layer * 1e3:.1f} ms/layer, tok/s "
                  f"extrapolated to {cfg.layers} layers",
    }


FP32_PEAK_TFLOPS = 157.3      # MI355X fp32


def bench_encoder(args) -> int:
    """The encoder's assignment step at c3 shapes: every 8-wide block of a
    14336 x 4096 weight (7,340,032 blocks) against a 4096-entry codebook, as
    the reference's encoder assigns all blocks after fitting
    (src/block_vq.py:180-196).  value = blocks per second; the roofline is the
    fp32 one over the distance flops 2 * n * K * d."""
    from wal2026_amd.block_vq import _assign_to_codebook

    dev = torch.device("cuda", 0)
    n, d, k = 14336 * 4096 // 8, 8, 4096
    gen = synth.generator(0, dev)
    blocks = torch.randn(n, d, generator=gen, device=dev) * 0.02
    cb = torch.randn(k, d, generator=gen, device=dev) * 0.02
    for _ in range(args.warmup):
        _assign_to_codebook(blocks, cb)
    stream = torch.cuda.current_stream()
    a = torch.cuda.Event(enable_timing=True)
    b = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    a.record(stream)
    for _ in range(args.steps):
        _assign_to_codebook(blocks, cb)
    b.record(stream)
    torch.cuda.synchronize()
    ms = a.elapsed_time(b) / args.steps
    flops = 2.0 * n * k * d
    # one Lloyd iteration of the codebook fit on the default 131,072-block sample
    from wal2026_amd.block_vq import _fit_kmeans

    sample = blocks[:131_072]
    _fit_kmeans(sample, k, iters=1)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    _fit_kmeans(sample, k, iters=3)
    torch.cuda.synchronize()
    t3 = time.perf_counter() - t0
    t0 = time.perf_counter()
    _fit_kmeans(sample, k, iters=1)
    torch.cuda.synchronize()
    kmeans_ms = (t3 - (time.perf_counter() - t0)) / 2 * 1e3
    out = {
        "metric": "encoder assignment (nearest of 4096 codewords, d=8) blocks/s", "value": round(n / (ms * 1e-3), 1),
        "unit": "blocks/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic (seeded N(0, 0.02) blocks and codebook)",
        "config": {"workload": "c3 gate_proj encode: 7,340,032 blocks of 8 against K=4096", "n_blocks": n, "k": k,
                   "d": d, "kmeans_iteration_ms": round(kmeans_ms, 3),
                   "kmeans_sample": "131,072 blocks, K=4096 (assignment + centroid sums + mean, host-timed)"},
        "roofline": {"bound": "valu", "kernel": "rvq_assign_kernel<8, 4>",
                     "achieved": round(flops / (ms * 1e-3) / 1e12, 2), "peak": FP32_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(flops / (ms * 1e-3) / 1e12 / FP32_PEAK_TFLOPS, 4), "traffic": None},
    }
    if not args.no_cpu_baseline:
        from oracle import c_oracle

        sample = 8192
        hb, hc = blocks[:sample].cpu(), cb.cpu()
        t0 = time.perf_counter()
        c_oracle.assign(hb, hc)
        dt = time.perf_counter() - t0
        out["cpu_baseline"] = {"value": round(sample / dt, 1), "unit": "blocks/s", "cores": 1, "kind": "port",
                               "sample": f"{sample} of the {n} blocks through oracle or_assign (one thread), "
                                         f"{dt:.2f} s"}
    print(json.dumps(out))
    return 0


class Stack:
    """A seeded stack of compressed linears of one config on the GPU, with the
    drop-in (one launch per linear) and fused (linears sharing an input in one
    launch) steps."""

    def __init__(self, cfg: synth.Config, layers: int, dev: torch.device):
        self.cfg, self.layers, self.dev = cfg, layers, dev
        self.stack = build_stack(cfg, dev, layers)
        gen = synth.generator(1, dev)
        self.xs = {k: synth.make_activation(cfg.m, k, cfg.x_dtype, gen, dev) for k in {k for _, _, k in cfg.shapes()}}
        names = [n for n, _, _ in cfg.shapes()]
        self.fuse = [(f, members) for f, members in FUSION_GROUPS if all(m in names for m in members)]
        for layer in self.stack:
            for f, members in self.fuse:
                layer[f] = FusedBlockRVQLinears([layer[m] for m in members])
        self.shape = {n: (o, k) for n, o, k in cfg.shapes()}

    def fused_launches(self):
        """(name, in_features, compressed bytes) of the fused step's launches."""
        cfg, shape = self.cfg, self.shape
        fused_members = {m for _, members in self.fuse for m in members}
        out = [(f, shape[members[0]][1], sum(linear_bytes(cfg, *shape[m]) for m in members)) for f, members in self.fuse]
        out += [(n, k, linear_bytes(cfg, o, k)) for n, o, k in cfg.shapes() if n not in fused_members]
        return out

    def dominant(self):
        return max(self.fused_launches(), key=lambda t: t[2])

    def launch_flops(self, name: str) -> int:
        members = dict(self.fuse).get(name, (name,))
        return sum(2 * self.cfg.m * self.shape[m][0] * self.shape[m][1] for m in members)

    def step_unfused(self):
        """The drop-in step: every linear its own forward (the reference's call pattern)."""
        for layer in self.stack:
            for name, _n, k in self.cfg.shapes():
                layer[name](self.xs[k])

    def step_fused(self):
        for layer in self.stack:
            for name, k, _b in self.fused_launches():
                layer[name](self.xs[k])

    def graph_ms(self, step, steps: int, warmup: int) -> float:
        """ms per replay of one step captured as a HIP graph (steps replays timed)."""
        step()  # builds descriptors and codebook images outside the graph
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            step()
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        with torch.cuda.graph(graph):
            step()
        torch.cuda.synchronize()
        for _ in range(warmup):
            graph.replay()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            graph.replay()
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) * 1000.0 / steps

    def eager_ms(self, step, steps: int, warmup: int) -> tuple[float, float]:
        """(ms per step, host ms per step) of plain eager forwards (no graph):
        what an import swap gives when the host issues every launch; the host
        figure is the time to issue the steps, before waiting for the GPU."""
        for _ in range(max(warmup, 1)):
            step()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            step()
        t_issue = time.perf_counter() - t0
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) * 1000.0 / steps, t_issue * 1000.0 / steps

    def launch_us(self, name: str, reps: int = 5) -> float:
        """Average duration of one `name` launch (graph_launch_us over the layers)."""
        k = next(kk for n, kk, _ in self.fused_launches() if n == name) if name in dict(self.fuse) \
            else self.shape[name][1]
        x = self.xs[k]
        return graph_launch_us([(lambda mod=layer[name]: mod(x)) for layer in self.stack], reps=reps)


def prefill_fused_us(st: Stack, name: str) -> float:
    """Duration of one `name` launch with the fused prefill kernel forced
    (WAL2026_PREFILL_TWO_PASS=0), beside the operator's two-pass choice."""
    old = os.environ.get("WAL2026_PREFILL_TWO_PASS")
    os.environ["WAL2026_PREFILL_TWO_PASS"] = "0"
    try:
        return st.launch_us(name)
    finally:
        if old is None:
            del os.environ["WAL2026_PREFILL_TWO_PASS"]
        else:
            os.environ["WAL2026_PREFILL_TWO_PASS"] = old


def pmc_path(kind: str, config: str, name: str, two_pass: bool = False) -> str:
    return str(ROOT / "profiles" / f"{kind}_{config}_{name}{'_two_pass' if two_pass else ''}_pmc.txt")


def roofline_of(st: Stack, name: str, nbytes: int, us: float, pmc_summary: str | None) -> dict:
    cfg = st.cfg
    # the committed counter summaries are for each config's own M
    own_m = cfg.m == synth.CONFIGS[cfg.name].m
    if cfg.m > 16:
        flops = st.launch_flops(name)
        tflops = flops / (us * 1e-6) / 1e12
        x = st.xs[next(k for n, k, _ in st.fused_launches() if n == name)]
        info = st.stack[0][name].launch_info(x)
        two_pass = info.get("two_pass", False)
        if two_pass:
            kernel = (f"{name} launch, two passes: rvq_dequant8_kernel (the dense weight, bit-exact) + torch's "
                      f"bf16 GEMM (hipBLASLt), {flops} flop")
            pmc_summary = pmc_path("prefill", cfg.name, name, two_pass=True) if own_m else None
        else:
            kernel = (f"rvq_prefill_*_kernel, {info['tile_shape']} tile, {info['k_splits']} k slice(s) "
                      f"({name}, {flops} flop)")
            pmc_summary = pmc_summary if own_m else None
        out = {"bound": "mfma", "kernel": kernel, "two_pass": two_pass,
               "achieved": round(tflops, 1), "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
               "frac": round(tflops / BF16_PEAK_TFLOPS, 4), "avg_launch_us": round(us, 3),
               "algorithmic_flops_per_launch": flops,
               "traffic": traffic_bytes(pmc_summary) if pmc_summary else None}
        if two_pass:
            fus = prefill_fused_us(st, name)
            ftf = flops / (fus * 1e-6) / 1e12
            out["fused_kernel"] = {"kernel": f"rvq_prefill_*_kernel, launcher's choice ({name})",
                                   "avg_launch_us": round(fus, 3), "achieved": round(ftf, 1),
                                   "frac": round(ftf / BF16_PEAK_TFLOPS, 4),
                                   "traffic": traffic_bytes(pmc_path("prefill", cfg.name, name)) if own_m else None}
        return out
    gbs = nbytes / (us * 1e-6) / 1e9
    return {"bound": "hbm", "kernel": f"rvq_decode_kernel ({name}, {nbytes} compressed bytes)",
            "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4),
            "avg_launch_us": round(us, 3), "algorithmic_bytes_per_launch": nbytes,
            "traffic": traffic_bytes(pmc_summary) if pmc_summary else None}


def secondary(name: str, layers: int | None, steps: int, warmup: int, dev: torch.device,
              m: int | None = None) -> dict:
    """One line for another config (optionally at another M): fused-step
    tokens/s over a graph-captured stack and the dominant launch against its
    roofline (HIP events)."""
    cfg = synth.CONFIGS[name]
    if m is not None and m != cfg.m:
        cfg = synth.Config(**{**cfg.__dict__, "m": m})
    layers = layers or cfg.layers
    log(f"secondary {name}: building {layers} layers")
    st = Stack(cfg, layers, dev)
    ms = st.graph_ms(st.step_fused, steps, warmup)
    dom_name, _k, dom_bytes = st.dominant()
    us = st.launch_us(dom_name)
    kind = "prefill" if cfg.m > 16 else "decode"
    us_layer = ms * 1000.0 / layers
    out = {"workload": f"{name}: {kind} M={cfg.m}, S={cfg.num_stages}, K={cfg.codebook_size}, "
                       f"{str(cfg.ids_dtype()).replace('torch.', '')} ids, {layers} of {cfg.layers} layers timed, "
                       f"fused, one HIP graph per step, {steps} steps; tok/s over all {cfg.layers} layers",
           "tok_s": round(cfg.m * 1e6 / (us_layer * cfg.layers), 2), "us_per_layer": round(us_layer, 3),
           "roofline": roofline_of(st, dom_name, dom_bytes, us,
                                   pmc_path(kind, name, dom_name) if m is None else None)}
    if kind == "decode":
        out["step_hbm_fraction"] = round(cfg.compressed_bytes_per_layer() * layers / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
                                         4)
    else:
        out["tflops_per_step"] = round(cfg.flops_per_layer() * layers / (ms * 1e-3) / 1e12, 1)
    del st
    torch.cuda.empty_cache()
    return out


def bench_read_ceiling(args, cfg: synth.Config, layers: int, dev: torch.device) -> int:
    """Time a plain streaming read of the dominant launch's compressed bytes
    (wal_read_probe: the decode kernel's 16-byte streaming buffer loads, no
    compute), one cold buffer per layer as in the decode step, at the decode
    kernel's grid (256 workgroups x 512 threads) and at larger grids, beside the
    dominant launch itself: the read rate HBM gives this byte count per launch
    is the practical ceiling for the decode kernel's roofline fraction."""
    lib = _lib.lib()
    st = Stack(cfg, layers, dev)
    dom_name, dom_k, dom_bytes = st.dominant()
    for layer in st.stack:
        layer[dom_name](st.xs[dom_k])  # descriptors and codebook images built before timing
    torch.cuda.synchronize()
    dom_us = st.launch_us(dom_name)
    nbytes = (dom_bytes + 15) // 16 * 16
    gen = torch.Generator(device=dev).manual_seed(0)
    bufs = [torch.randint(0, 256, (nbytes,), dtype=torch.uint8, device=dev, generator=gen) for _ in range(layers)]
    partial = torch.empty(2**16, dtype=torch.int32, device=dev)
    shapes = [(256, 512), (512, 512), (1024, 512), (2048, 256), (4096, 256)]
    if args.read_grid:
        shapes = [(args.read_grid, 512)]
    rows = []
    for grid, block in shapes:
        def launcher(buf, grid=grid, block=block):
            def run():
                _lib.check(lib.wal_read_probe(buf.data_ptr(), nbytes, partial.data_ptr(), grid, block,
                                              torch.cuda.current_stream().cuda_stream))
            return run
        us = graph_launch_us([launcher(b) for b in bufs], reps=5)
        gbs = nbytes / (us * 1e-6) / 1e9
        rows.append({"grid": grid, "block": block, "us": round(us, 3), "GBps": round(gbs, 1),
                     "frac": round(gbs / HBM_PEAK_GBS, 4)})
        log(f"read probe {grid} x {block}: {us:.2f} us, {gbs:.0f} GB/s")
    best = max(rows, key=lambda r: r["frac"])
    dom_gbs = dom_bytes / (dom_us * 1e-6) / 1e9
    print(json.dumps({
        "mode": "read_ceiling", "config": cfg.name, "launch": dom_name, "bytes_per_launch": nbytes,
        "layers": layers, "read_probe": rows,
        "dominant": {"us": round(dom_us, 3), "GBps": round(dom_gbs, 1), "frac": round(dom_gbs / HBM_PEAK_GBS, 4)},
        "dominant_over_best_read": round(dom_gbs / best["GBps"], 4)}), flush=True)
    return 0


def bench_dense_reference(args, cfg: synth.Config, dev: torch.device) -> int:
    """Time torch's dense bf16 GEMM (hipBLASLt) at each fused launch shape of
    the config, no dequantisation: the library rate the prefill paths are
    compared with.  Two weight layouts: W [out, in] as nn.Linear stores it,
    through F.linear (the two-pass prefill's GEMM), and W^T [in, out]
    contiguous, through x @ W^T.  The natural layout is also timed with
    weights N(0, 0.02) (the scale of this build's synthetic codebooks) and
    with both operands zero: the matrix cores' rate depends on the operands'
    bit activity (the chip lowers its clock under load), so the zero case
    bounds what any data reaches."""
    st_shapes = []
    shape = {name: (n, k) for name, n, k in cfg.shapes()}
    groups = [(f, parts) for f, parts in FUSION_GROUPS if all(p in shape for p in parts)]
    for fused, parts in groups:
        st_shapes.append((fused, sum(shape[p][0] for p in parts), shape[parts[0]][1]))
    fused_parts = {p for _, parts in groups for p in parts}
    for name, n, k in cfg.shapes():
        if name not in fused_parts:
            st_shapes.append((name, n, k))
    def time_us(fn) -> float:
        for _ in range(5):
            fn()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        reps = 20
        a.record()
        for _ in range(reps):
            fn()
        b.record()
        torch.cuda.synchronize()
        return a.elapsed_time(b) * 1000.0 / reps

    rows = {}
    for name, n, k in st_shapes:
        x = torch.randn(cfg.m, k, device=dev, dtype=torch.bfloat16)
        w = torch.randn(n, k, device=dev, dtype=torch.bfloat16)
        wt = w.t().contiguous()
        row = {"m": cfg.m, "n": n, "k": k}
        for lay, fn in (("w_out_in", lambda: torch.nn.functional.linear(x, w)), ("wt_in_out", lambda: x @ wt)):
            us = time_us(fn)
            tf = 2.0 * cfg.m * n * k / (us * 1e-6) / 1e12
            row[lay] = {"us": round(us, 3), "tflops": round(tf, 1), "frac": round(tf / BF16_PEAK_TFLOPS, 4)}
            log(f"dense bf16 {name} {cfg.m}x{n}x{k} ({lay}): {us:.1f} us {tf:.0f} TFLOP/s")
        w_small = (torch.randn(n, k, device=dev) * 0.02).to(torch.bfloat16)
        x0, w0 = torch.zeros_like(x), torch.zeros_like(w)
        for data, fn in (("w_out_in_w002", lambda: torch.nn.functional.linear(x, w_small)),
                         ("w_out_in_zeros", lambda: torch.nn.functional.linear(x0, w0))):
            us = time_us(fn)
            tf = 2.0 * cfg.m * n * k / (us * 1e-6) / 1e12
            row[data] = {"us": round(us, 3), "tflops": round(tf, 1), "frac": round(tf / BF16_PEAK_TFLOPS, 4)}
            log(f"dense bf16 {name} {cfg.m}x{n}x{k} ({data}): {us:.1f} us {tf:.0f} TFLOP/s")
        del w_small, x0, w0
        rows[name] = row
    print(json.dumps({"mode": "dense_reference", "config": cfg.name, "launches": rows}), flush=True)
    return 0


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None,
                    help="timed steps (default 50; 128 for c5, the step count its survey figure is quoted over)")
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", default="c3", choices=["c1", "c2", "c3", "c4", "c5"])
    ap.add_argument("--m", type=int, default=None, help="activation rows (default: the config's, 1 for c3)")
    ap.add_argument("--layers", type=int, default=None)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-secondary", action="store_true",
                    help="skip the c5 decode and c4 prefill lines the default c3 run adds under config.secondary")
    ap.add_argument("--profile-dominant", type=int, default=0, metavar="N",
                    help="only run the dominant launch N times per layer, then one 256 MiB device copy "
                         "(the calibration kernel); for rocprofv3 --pmc runs")
    ap.add_argument("--pmc-summary", default=None,
                    help="rocprofv3 --pmc summary giving the dominant kernel's HBM traffic (default: "
                         "profiles/<decode|prefill>_<config>_<launch>_pmc.txt when it exists)")
    ap.add_argument("--read-ceiling", action="store_true",
                    help="time a plain streaming read of the dominant launch's compressed bytes (wal_read_probe) "
                         "beside the launch itself: the practical HBM ceiling for this byte count per launch")
    ap.add_argument("--read-grid", type=int, default=0,
                    help="with --read-ceiling: only this grid (512 threads per workgroup), for rocprofv3 runs")
    ap.add_argument("--dense-reference", action="store_true",
                    help="time torch's dense bf16 GEMM (hipBLASLt) at the config's launch shapes, no dequantisation")
    ap.add_argument("--encoder", action="store_true",
                    help="time the encoder's assignment step (wal_rvq_assign) on c3's gate_proj blocks instead")
    args = ap.parse_args()
    if args.steps is None:
        args.steps = 128 if args.config == "c5" and not args.encoder else 50
    if args.gpus != 1:
        print("bench.py: this build runs on one GPU only (the path has no multi-GPU code); "
              "run with --gpus 1", file=sys.stderr)
        return 2
    if not torch.cuda.is_available():
        print("bench.py: no ROCm GPU visible", file=sys.stderr)
        return 1

    if args.encoder:
        return bench_encoder(args)

    cfg = synth.CONFIGS[args.config]
    if args.m is not None and args.m != cfg.m:
        cfg = synth.Config(**{**cfg.__dict__, "m": args.m})
    layers = args.layers or cfg.layers
    dev = torch.device("cuda", 0)
    if args.read_ceiling:
        return bench_read_ceiling(args, cfg, layers, dev)
    if args.dense_reference:
        return bench_dense_reference(args, cfg, dev)
    log(f"building {layers} layers of {cfg.name} on {torch.cuda.get_device_name(dev)}")
    st = Stack(cfg, layers, dev)

    if args.profile_dominant:
        dom_name, dom_k, dom_bytes = st.dominant()
        for layer in st.stack:
            layer[dom_name](st.xs[dom_k])  # descriptors and codebook images of the profiled launch only
        torch.cuda.synchronize()
        for _ in range(args.profile_dominant):
            for layer in st.stack:
                layer[dom_name](st.xs[dom_k])
        torch.cuda.synchronize()
        src = torch.empty(64 * 2**20, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        dst.copy_(src)  # 256 MiB read + 256 MiB written: the counters' calibration
        torch.cuda.synchronize()
        print(json.dumps({"profiled": dom_name, "launches": args.profile_dominant * layers,
                          "algorithmic_bytes_per_launch": dom_bytes, "calibration_copy_bytes": 2**28}), flush=True)
        return 0

    log(f"timing {args.steps} graph replays of the drop-in step (one launch per linear)")
    ms_unfused = st.graph_ms(st.step_unfused, args.steps, args.warmup)
    log(f"timing {args.steps} eager drop-in steps (no graph)")
    ms_eager, ms_eager_host = st.eager_ms(st.step_unfused, args.steps, args.warmup)
    # the drop-in step again with each layer's q/k/v and gate/up linked by
    # fuse_sibling_linears: the model's unchanged calls, the fused launches
    log("timing the drop-in step with fuse_sibling_linears (graph, then eager)")
    for layer in st.stack:
        fuse_sibling_linears(torch.nn.ModuleDict({n: layer[n] for n, _, _ in cfg.shapes()}))
    ms_sib = st.graph_ms(st.step_unfused, args.steps, args.warmup)
    ms_sib_eager, _ = st.eager_ms(st.step_unfused, args.steps, args.warmup)
    for layer in st.stack:
        unfuse_sibling_linears(torch.nn.ModuleDict({n: layer[n] for n, _, _ in cfg.shapes()}))
    log(f"timing {args.steps} graph replays of the fused step ({len(st.fused_launches())} launches per layer)")
    ms_per_step = st.graph_ms(st.step_fused, args.steps, args.warmup)
    tok_s = cfg.m * 1000.0 / ms_per_step

    # dominant kernel: the fused step's largest launch, timed per launch
    dom_name, dom_k, dom_bytes = st.dominant()
    log(f"timing the dominant kernel ({dom_name}) per launch")
    dom_us = st.launch_us(dom_name)
    per_launch = {}
    for name, k, nbytes in st.fused_launches():
        us = st.launch_us(name, reps=1)
        per_launch[name] = {"us": round(us, 3), "GBps": round(nbytes / (us * 1e-6) / 1e9, 1)}
    per_linear = {}
    for name, n, k in cfg.shapes():
        us = st.launch_us(name, reps=1)
        per_linear[name] = {"us": round(us, 3), "GBps": round(linear_bytes(cfg, n, k) / (us * 1e-6) / 1e9, 1)}
    layer_bytes = cfg.compressed_bytes_per_layer()
    prefill = cfg.m > 16
    kind = "prefill" if prefill else "decode"
    pmc_summary = args.pmc_summary or pmc_path(kind, cfg.name, dom_name)
    roofline = roofline_of(st, dom_name, dom_bytes, dom_us, pmc_summary)
    n_linears = len(cfg.shapes()) * layers

    result = {
        "metric": "RVQ-GEMV us/layer & %HBM roofline (M=1); decode tok/s at Llama-8B shapes",
        "value": round(tok_s, 3),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded random Block-RVQ encodings and activations)",
        "config": {
            "workload": f"{cfg.name}: Llama-3-8B-shaped {layers}-layer stack of compressed linears, "
                        f"S={cfg.num_stages}, K={cfg.codebook_size}, d={cfg.block_size}, "
                        f"{str(cfg.ids_dtype()).replace('torch.', '')} ids, scale per {cfg.scale_rows} rows, "
                        f"{kind} M={cfg.m}, one HIP graph per step; linears sharing an input fused "
                        f"({', '.join(f for f, _ in st.fuse)})",
            "layers": layers,
            "m": cfg.m,
            "us_per_layer": round(ms_per_step * 1000.0 / layers, 3),
            "compressed_bytes_per_layer": layer_bytes,
            "step_hbm_fraction": round(layer_bytes * layers / (ms_per_step * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "unfused_tok_s": round(cfg.m * 1000.0 / ms_unfused, 3),
            "unfused_us_per_layer": round(ms_unfused * 1000.0 / layers, 3),
            "eager_unfused_tok_s": round(cfg.m * 1000.0 / ms_eager, 3),
            "dropin_sibling_fused_tok_s": round(cfg.m * 1000.0 / ms_sib, 3),
            "eager_dropin_sibling_fused_tok_s": round(cfg.m * 1000.0 / ms_sib_eager, 3),
            "eager_us_per_forward": round(ms_eager * 1000.0 / n_linears, 3),
            "eager_host_issue_us_per_forward": round(ms_eager_host * 1000.0 / n_linears, 3),
            "per_launch": per_launch,
            "per_linear_unfused": per_linear,
        },
        "roofline": roofline,
    }
    if prefill:
        result["config"]["tflops_per_step"] = round(cfg.flops_per_layer() * layers / (ms_per_step * 1e-3) / 1e12, 1)
    del st
    torch.cuda.empty_cache()
    if not args.no_secondary and args.config == "c3" and args.m is None and args.layers is None:
        result["config"]["secondary"] = {
            "c5": secondary("c5", None, 128, args.warmup, dev),
            # (all 32 layers, as `--config c4` times them: a shorter stack
            # weighs the graph launch and the first layer's cold caches more)
            "c4": secondary("c4", None, 10, 2, dev),
            # a batch of 256 prefill rows: the operator picks per launch
            # between the split-K fused kernel and the two passes
            "c4_m256": secondary("c4", None, 10, 2, dev, m=256),
        }
    if not args.no_cpu_baseline:
        log("timing the CPU baseline")
        result["cpu_baseline"] = cpu_baseline(cfg)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
