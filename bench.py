#!/usr/bin/env python3
"""Benchmark of the hip GDN backend on one MI355X.

One step = one fwd+bwd of the gated delta rule through the drop-in API
``cqgdn.gated_delta_net.delta`` (autograd, use_qk_l2norm_in_kernel=True) over
one batch of synthetic inputs already resident in HBM.  The workload is
benchmark config 2: content T=8192 plus 4 read-only CQ query blocks of 256
events at seeded positions (9216 events), H=16, d=128, bf16 q/k/v, fp32 g/beta
and state; timing follows the reference's GDN benchmark (warm-up, then
synchronize around the timed loop, scripts/benchmark_gdn.py:51-56).

The library runs bwd_dkw on a second stream beside the reverse state scan when the
scan's workgroups all fit on the GPU at once (config 2 does): that is the step timed
for ``value``.  bwd_dkw's launch then spans most of the scan, so the per-kernel table
and the roofline come from a second timed pass of K steps with bwd_dkw after the scan
(CQGDN_DKW_BESIDE_SCAN=0), where every launch is the kernel's own time.

Printed: one JSON line with the contract keys, plus
  roofline      the dominant kernel against the roofline that bounds it (HBM below the
                312 FLOP/byte ridge, bf16 MFMA above; HIP events on the stream it runs on,
                recorded inside the timed pass with bwd_dkw after the scan), with the other
                resource's figures beside and its launch time beside the scan
  cpu_baseline  the fp32 chunked torch oracle on this host's cores (a bounded
                sample: one config-2 fwd+bwd; rows: one config-0 forward and the
                config-4 decode step)
  extra         config-1 and config-3 fwd+bwd, config-2 fwd+bwd in the fused mode and
                with fp16 inputs, per-kernel table (MFMA / HBM
                fractions), the whole GatedDelta layer at width 2048 (content 2048 and
                8192 on image-CQ plans, beside the reference's published Ascend 910B
                medians), prefill, and the decode step (B=64, 256 steps, GB/s)

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-extra]
       python bench.py --profile | --profile-layer | --profile-decode   (profiler workloads)
"""

from __future__ import annotations

import argparse
import json
import os
import re
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _p in (ROOT, ROOT / "cq-pretrain_amd", ROOT / "tests"):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

METRIC = "GDN fwd+bwd ms/layer @T=2048/8192 (H=16,d=128); MFMA util %; decode GB/s"
H, D = 16, 128
TRAFFIC_FILE = ROOT / "profiles" / "hbm_traffic_config2.md"


def parse_args():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-extra", action="store_true", help="skip config 1, prefill, decode and the kernel table")
    ap.add_argument("--decode-steps", type=int, default=256)
    ap.add_argument("--profile", action="store_true",
                    help="profiler workload only: config-2 fwd+bwd steps, then a plain copy kernel of "
                         "known size (the scale of the HBM byte counters); prints no JSON")
    ap.add_argument("--config", type=int, default=2, choices=(1, 2, 3),
                    help="with --profile: the benchmark configuration whose fwd+bwd steps are profiled")
    ap.add_argument("--fp16", action="store_true",
                    help="with --profile: fp16 q/k/v and dO (the fp16 kernels, CQGDN_FP16)")
    ap.add_argument("--dkw-after-scan", action="store_true",
                    help="with --profile: bwd_dkw after the reverse scan (CQGDN_DKW_BESIDE_SCAN=0), the "
                         "pass the per-kernel table and the roofline are measured in")
    ap.add_argument("--profile-layer", action="store_true",
                    help="profiler workload only: warmup + steps fused fwd+bwd steps of the width-2048 "
                         "layer at content 2048; prints no JSON")
    ap.add_argument("--profile-decode", action="store_true",
                    help="profiler workload only: the config-4 decode loop (B=64, --decode-steps steps over "
                         "8 rotated layer states), then a plain copy kernel of known size; prints no JSON")
    return ap.parse_args()


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def training_case(gdn, synthetic, torch, config, device, fp16=False):
    T, mask, bounds = synthetic.config_events(config, seed=0)
    xs = [x.to(device) for x in synthetic.make_inputs(T, H, D, seed=config, readonly=mask)]
    gen = torch.Generator().manual_seed(100 + config)
    do = torch.randn(1, T, H, D, generator=gen).bfloat16().to(device)
    if fp16:  # the reference's fp16 training inputs, on the fp16 kernels
        xs = [x.half() if x.dim() == 4 else x for x in xs]
        do = do.half()
    leaves = [x.requires_grad_() for x in xs]
    # packed documents (config 3) go in as cu_seqlens, one state reset per document
    packed = {}
    if len(bounds) > 2:
        packed = dict(cu_seqlens=torch.tensor(bounds, dtype=torch.int64, device=device), cu_seqlens_cpu=list(bounds))

    def step():
        for x in leaves:
            x.grad = None
        y, _ = gdn.delta(*leaves, use_qk_l2norm_in_kernel=True, **packed)
        y.backward(do)

    return T, bounds, step, xs


def time_steps(torch, step, steps, windows=5):
    """Seconds per step of the secondary configurations: the median over `windows` windows of
    `steps` steps each, each window bracketed by synchronizations (the headline value times
    exactly K steps in one window instead)."""
    per = []
    for _ in range(windows):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            step()
        torch.cuda.synchronize()
        per.append((time.perf_counter() - t0) / steps)
    return statistics.median(per)


def kernel_table(torch, _lib, workmodel, step, bounds, reps=5):
    """Average duration of every fwd/bwd kernel (one armed at a time) and its roofline."""
    table = {}
    for name in workmodel.FWD_KERNELS + workmodel.BWD_KERNELS:
        with _lib.KernelTimer(name, reps) as t:
            for _ in range(reps):
                step()
            torch.cuda.synchronize()
        if not t.ms:
            continue
        sec = statistics.mean(t.ms) * 1e-3
        flops, nbytes = workmodel.kernel_work(name, bounds, H)
        table[name] = dict(us=round(sec * 1e6, 2), tflops=round(flops / sec / 1e12, 2),
                           mfma_frac=round(flops / sec / workmodel.PEAK_BF16_FLOPS, 4),
                           gbps=round(nbytes / sec / 1e9, 1),
                           hbm_frac=round(nbytes / sec / workmodel.PEAK_HBM_BYTES, 4))
    return table


def traffic_for(kernel, sha):
    """HBM bytes per launch of ``kernel`` from the committed rocprofv3 counter summary, if it
    was measured on this exact library build; else None."""
    if not TRAFFIC_FILE.exists():
        return None
    for line in TRAFFIC_FILE.read_text().splitlines():
        m = re.match(r"^traffic kernel=(\S+) lib_sha256=(\S+) bytes_per_launch=(\d+)", line.strip())
        if m and m.group(1) == kernel and m.group(2) == sha:
            return int(m.group(3))
    return None


def cpu_baseline(torch, decode_steps=8):
    """The CPU rows of the plan (fp32 torch oracle on this host's cores, one thread per core the
    process may use): config 2 fwd+bwd via autograd (the reported baseline, same unit as
    ``value``), plus the config 0 forward, the config 1 fwd+bwd and the config 4 decode step (``rows``)."""
    from cqgdn import synthetic
    from oracle import gdn_oracle as O

    cores = len(os.sched_getaffinity(0))
    prev = torch.get_num_threads()
    torch.set_num_threads(cores)
    rows = {}
    try:
        T, mask, bounds = synthetic.config_events(2, seed=0)
        xs = [x.float().requires_grad_() for x in synthetic.make_inputs(T, H, D, seed=2, readonly=mask)]
        do = torch.randn(1, T, H, D, generator=torch.Generator().manual_seed(102))
        t0 = time.perf_counter()
        y = O.chunk_delta(*xs, bounds, normalize=True)
        y.backward(do)
        sec = time.perf_counter() - t0
        del xs, y, do
        # config 1: fwd+bwd via autograd, T=2304 (2048 content + 256 read-only)
        T1, mask1, bounds1 = synthetic.config_events(1, seed=0)
        x1 = [x.float().requires_grad_() for x in synthetic.make_inputs(T1, H, D, seed=1, readonly=mask1)]
        do1 = torch.randn(1, T1, H, D, generator=torch.Generator().manual_seed(101))
        t0 = time.perf_counter()
        O.chunk_delta(*x1, bounds1, normalize=True).backward(do1)
        rows["config1_fwd_bwd_ms"] = round((time.perf_counter() - t0) * 1e3, 2)
        del x1, do1
        # config 0: forward only, T=2048, zero initial state, final state returned
        T0, _, b0 = synthetic.config_events(0)
        x0 = [x.float() for x in synthetic.make_inputs(T0, H, D, seed=0)]
        with torch.no_grad():
            O.chunk_delta(*x0, b0, normalize=True, output_final_state=True)  # warm-up
            t0 = time.perf_counter()
            O.chunk_delta(*x0, b0, normalize=True, output_final_state=True)
            rows["config0_fwd_ms"] = round((time.perf_counter() - t0) * 1e3, 2)
        # config 4: the per-step recurrence (models/decoding.py:71-77) at B=64, H=16, fp32 state
        gen = torch.Generator().manual_seed(4)
        n = 64
        state = torch.randn(n, H, D, D, generator=gen) * 0.02
        q = O.l2norm(torch.randn(n, 1, H, D, generator=gen))
        k = O.l2norm(torch.randn(n, 1, H, D, generator=gen))
        v = torch.randn(n, 1, H, D, generator=gen)
        g = -torch.nn.functional.softplus(torch.randn(n, 1, H, generator=gen))
        b = torch.randn(n, 1, H, generator=gen).sigmoid()
        with torch.no_grad():
            O.decode_step(q, k, v, g, b, state)  # warm-up
            t0 = time.perf_counter()
            for _ in range(decode_steps):
                O.decode_step(q, k, v, g, b, state)
            rows["config4_decode_us_per_step"] = round((time.perf_counter() - t0) / decode_steps * 1e6, 1)
    finally:
        torch.set_num_threads(prev)
    return dict(value=round(sec * 1e3, 1), unit="ms/layer", cores=cores, kind="port",
                sample="one fwd+bwd of config 2 (T=9216, H=16, d=128): oracle/gdn_oracle.chunk_delta in fp32 "
                       "(chunk 64) with torch autograd for the backward, "
                       f"torch.set_num_threads({cores}); rows: one config-0 forward (T=2048, final state), one "
                       "config-1 fwd+bwd (T=2304) and "
                       f"the mean of {decode_steps} config-4 decode steps (B=64, H=16, fp32 state, "
                       "oracle/gdn_oracle.decode_step), same threads",
                rows=rows)


def decode_case(gdn, _lib, workmodel, torch, device, steps):
    """Config 4: B=64 sequences, H=16, one event per step, 256 steps over 8 rotated layer states."""
    n, layers = 64, 8
    gen = torch.Generator().manual_seed(4)
    states = [(torch.randn(n, H, D, D, generator=gen) * 0.02).to(device) for _ in range(layers)]
    q = torch.nn.functional.normalize(torch.randn(n, 1, H, D, generator=gen), dim=-1).bfloat16().to(device)
    k = torch.nn.functional.normalize(torch.randn(n, 1, H, D, generator=gen), dim=-1).bfloat16().to(device)
    v = torch.randn(n, 1, H, D, generator=gen).bfloat16().to(device)
    g = (-torch.nn.functional.softplus(torch.randn(n, 1, H, generator=gen))).to(device)
    b = torch.randn(n, 1, H, generator=gen).sigmoid().to(device)
    out = torch.empty_like(q)
    for st in states:
        gdn.recurrent(q, k, v, g, b, st, out)
    # one Python call per step, as a decode loop makes them
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        gdn.recurrent(q, k, v, g, b, states[i % layers], out)
    torch.cuda.synchronize()
    sec = (time.perf_counter() - t0) / steps
    # the kernel's own duration, by events around each launch (a separate pass: the events
    # cost host time of their own)
    with _lib.KernelTimer("recurrent", steps) as t:
        for i in range(steps):
            gdn.recurrent(q, k, v, g, b, states[i % layers], out)
    nbytes = workmodel.decode_bytes(n, H)
    kern = statistics.mean(t.ms) * 1e-3
    # the same loop captured once in a HIP graph and replayed: what a serving loop pays per step
    # without a Python call per launch (the step records no memset)
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for i in range(layers):
            gdn.recurrent(q, k, v, g, b, states[i], out)
    torch.cuda.current_stream().wait_stream(side)
    with torch.cuda.graph(graph):
        for i in range(steps):
            gdn.recurrent(q, k, v, g, b, states[i % layers], out)
    graph.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    graph.replay()
    torch.cuda.synchronize()
    gsec = (time.perf_counter() - t0) / steps
    return dict(us_per_step=round(sec * 1e6, 2), gbps=round(nbytes / sec / 1e9, 1),
                graph_us_per_step=round(gsec * 1e6, 2), graph_gbps=round(nbytes / gsec / 1e9, 1),
                graph_hbm_frac=round(nbytes / gsec / workmodel.PEAK_HBM_BYTES, 4),
                kernel_us=round(kern * 1e6, 2), kernel_gbps=round(nbytes / kern / 1e9, 1),
                kernel_hbm_frac=round(nbytes / kern / workmodel.PEAK_HBM_BYTES, 4),
                bytes_per_step=nbytes, working_set_mb=round(layers * n * H * D * D * 4 / 1e6, 1))


def layer_setup(torch, device, content, queries):
    """Whole GatedDelta layer at width 2048 on an image-CQ plan with the event counts of the
    reference's benchmark rows (scripts/benchmark_gdn.py:34-56).  Returns the plan and
    ``step(fused)``, one fwd+bwd step of the layer (the layer and the plan come from the test
    harness, tests/layer_harness.py)."""
    import layer_harness as layer

    torch.manual_seed(872)
    model = layer.GatedDeltaLayer().to(device, torch.bfloat16)
    model.A_log.data = model.A_log.data.float()
    model.norm_weight.data = model.norm_weight.data.float()
    plan = layer.cq_layer_plan(content, queries).to(device)
    x = torch.randn(plan.hidden_length, 1, 2048, device=device, dtype=torch.bfloat16, requires_grad=True)
    upstream = torch.randn_like(x) / 100

    def step(fused):
        model.zero_grad(set_to_none=True)
        x.grad = None
        y = model(x, plan, fused=fused)
        (y * upstream).sum().backward()
        return y

    def outputs(y):
        """The last step's y, dx and input-projection gradient in fp32 (outside the timed steps,
        as the reference takes them)."""
        return dict(y=y.detach().float(), dx=x.grad.detach().float(),
                    dw=model.in_proj_all.weight.grad.detach().float())

    return plan, step, outputs


def layer_case(torch, device, content, queries, iterations=12):
    """The layer of ``layer_setup`` measured as the reference's layer benchmark does
    (scripts/benchmark_gdn.py:44-64): 3 warm-up steps, peak-memory statistics reset, the median
    of ``iterations`` fwd+bwd steps (each bracketed by synchronize), the peak allocated bytes
    (model, inputs, activations and workspaces of this layer: what the earlier cases of the run
    still hold is subtracted, as the reference measures in a process of its own), and the relative
    RMS of y, dx and the input-projection gradient dw between the two paths."""
    base = torch.cuda.memory_allocated()  # held by the earlier cases: not the layer's
    plan, layer_step, layer_outputs = layer_setup(torch, device, content, queries)

    def timed(fused):
        for _ in range(3):
            layer_step(fused)
        torch.cuda.synchronize()
        torch.cuda.reset_peak_memory_stats()
        durations = []
        for _ in range(iterations):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            y = layer_step(fused)
            torch.cuda.synchronize()
            durations.append((time.perf_counter() - t0) * 1e3)
        peak = torch.cuda.max_memory_allocated() - base
        return round(statistics.median(durations), 4), peak, layer_outputs(y)

    # fused: everything between the projections in the fused kernels (events.layer_core);
    # torch_glue: the reference's torch code around the hip delta, conv and gated norm
    ms_f, peak_f, out_f = timed(True)
    ms_g, peak_g, out_g = timed(False)
    rel = {name: round(float((out_f[name] - out_g[name]).square().mean().sqrt()
                             / out_f[name].square().mean().sqrt().clamp_min(1e-12)), 7) for name in out_f}
    return dict(content_tokens=content, query_tokens=queries, events=len(plan.event_q),
                median_ms=ms_f, torch_glue_median_ms=ms_g, peak_bytes=peak_f, torch_glue_peak_bytes=peak_g,
                relative_rms_fused_vs_torch_glue=rel)


def layer_decode_case(torch, device, N, iterations=200):
    """One decode step of the layer between its projections (events.layer_decode_step:
    conv step, query conv, gates, two-event recurrence, gated norm) for N sequences at H = 16;
    the mean over ``iterations`` back-to-back steps timed with HIP events."""
    from cqgdn import events

    H, K = 16, 4
    S, P = H * 128, 4 * H * 128 + 2 * H
    gen = torch.Generator().manual_seed(70)
    w = (torch.rand(3 * S, K, generator=gen) - 0.5).bfloat16().to(device)
    A_log = torch.rand(H, generator=gen).mul(15.99).add(0.01).log().to(device)
    dt_bias, nw = torch.ones(H, device=device), torch.ones(128, device=device)
    proj = (torch.randn(N, 2, P, generator=gen) * 0.5).bfloat16().to(device)
    cache = {"conv": torch.zeros(N, K - 1, 3 * S, dtype=torch.bfloat16, device=device),
             "state": (torch.randn(N, H, 128, 128, generator=gen) * 0.01).to(device)}
    step = lambda: events.layer_decode_step(proj, w, A_log, dt_bias, nw, cache, heads=H)
    for _ in range(10):
        step()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    for _ in range(iterations):
        step()
    end.record()
    torch.cuda.synchronize()
    us = start.elapsed_time(end) * 1e3 / iterations
    # the same steps captured once in a HIP graph and replayed: the step without a Python call
    # and a ctypes round trip per launch (what a serving loop pays)
    graph_steps = 50
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(graph_steps):
            step()
    graph.replay()
    torch.cuda.synchronize()
    start.record()
    for _ in range(4):
        graph.replay()
    end.record()
    torch.cuda.synchronize()
    gus = start.elapsed_time(end) * 1e3 / (4 * graph_steps)
    state_bytes = 2 * N * H * 128 * 128 * 4
    return dict(sequences=N, us_per_step=round(us, 2), state_gbps=round(state_bytes / us / 1e3, 1),
                graph_us_per_step=round(gus, 2), graph_state_gbps=round(state_bytes / gus / 1e3, 1))


COPY_BYTES = 256 << 20


DKW_ENV = "CQGDN_DKW_BESIDE_SCAN"


class dkw_after_scan:
    """Within the block the library runs bwd_dkw after the reverse scan (the env switch it reads on
    every cqgdn_bwd call)."""

    def __enter__(self):
        self.old = os.environ.get(DKW_ENV)
        os.environ[DKW_ENV] = "0"

    def __exit__(self, *exc):
        if self.old is None:
            os.environ.pop(DKW_ENV, None)
        else:
            os.environ[DKW_ENV] = self.old


def profile_workload(torch, step, steps):
    """Workload run under rocprofv3: ``steps`` fwd+bwd steps, then 3 copies of COPY_BYTES."""
    for i in range(steps):
        step()
        torch.cuda.synchronize()
        log(f"profile step {i} done")
    copy_workload(torch)


def copy_workload(torch):
    """3 plain device copies of COPY_BYTES (read and written): the scale of the byte counters."""
    src = torch.ones(COPY_BYTES // 4, dtype=torch.float32, device="cuda:0")
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    log(f"copy kernel: {COPY_BYTES} bytes read and written per launch; done")


def main():
    args = parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for --gpus {args.gpus}). "
              "Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)
    import torch

    from cqgdn import _lib, gated_delta_net as gdn, synthetic, workmodel

    gdn.initialize()  # raises without a gfx950 GPU or without libcqgdn.so
    device = "cuda:0"
    sha = _lib.sha256()

    if args.profile_decode:
        log("config 4 decode (profile)")
        r = decode_case(gdn, _lib, workmodel, torch, device, args.decode_steps)
        log(f"decode: {r['kernel_us']} us per step by events; copy kernel next")
        copy_workload(torch)
        return
    if args.profile_layer:
        _, layer_step, _ = layer_setup(torch, device, 2048, 1675)
        for i in range(args.warmup + args.steps):
            layer_step(True)
            torch.cuda.synchronize()
            log(f"layer step {i} done")
        return

    if args.profile:
        if args.dkw_after_scan:
            os.environ[DKW_ENV] = "0"
        log(f"config {args.config} fwd+bwd (profile{', bwd_dkw after the scan' if args.dkw_after_scan else ''}"
            f"{', fp16 inputs' if args.fp16 else ''})")
        _, _, step, _ = training_case(gdn, synthetic, torch, args.config, device, fp16=args.fp16)
        for _ in range(args.warmup):
            step()
        torch.cuda.synchronize()
        profile_workload(torch, step, args.steps)
        return
    log("config 2 fwd+bwd")
    T, bounds, step, _ = training_case(gdn, synthetic, torch, 2, device)
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    with dkw_after_scan():
        kernels = {} if args.no_extra else kernel_table(torch, _lib, workmodel, step, bounds)
    dominant = max(kernels, key=lambda k: kernels[k]["us"]) if kernels else "bwd_dkw"

    # timed region (the product path, bwd_dkw beside the reverse scan): K steps with no
    # instrumentation armed, after two untimed steps in this mode
    for _ in range(2):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    ms = elapsed / args.steps * 1e3
    # the same K steps again with the dominant kernel's launches bracketed by HIP events on
    # its stream: its launch span beside the scan
    with _lib.KernelTimer(dominant, args.steps) as timer_beside:
        for _ in range(args.steps):
            step()
        torch.cuda.synchronize()
    # the same K steps with bwd_dkw after the scan: the dominant kernel's own launch time
    with dkw_after_scan():
        for _ in range(2):
            step()
        with _lib.KernelTimer(dominant, args.steps) as timer:
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for _ in range(args.steps):
                step()
            torch.cuda.synchronize()
            ms_after = (time.perf_counter() - t0) / args.steps * 1e3
    launch_s = statistics.mean(timer.ms) * 1e-3
    flops, nbytes = workmodel.kernel_work(dominant, bounds, H)
    # The bound is the resource the roofline model says limits the kernel: its algorithmic FLOPs
    # over its algorithmic bytes (about 75 FLOP/byte for bwd_dkw) against MI355X's ridge, 2.5 PFLOP/s
    # bf16 over 8 TB/s = 312 FLOP/byte.  Below the ridge the attainable rate is bytes-bound, so
    # `achieved` is algorithmic GB/s against 8 TB/s; the bf16 MFMA figures (the north_star's
    # utilization metric) stay beside it.
    intensity = flops / nbytes
    ridge = workmodel.PEAK_BF16_FLOPS / workmodel.PEAK_HBM_BYTES
    mfma = dict(mfma_achieved_tflops=round(flops / launch_s / 1e12, 2),
                mfma_frac=round(flops / launch_s / workmodel.PEAK_BF16_FLOPS, 4))
    hbm = dict(hbm_achieved_gbps=round(nbytes / launch_s / 1e9, 1),
               hbm_frac=round(nbytes / launch_s / workmodel.PEAK_HBM_BYTES, 4))
    if intensity < ridge:
        roof = dict(kernel=dominant, bound="hbm", achieved=hbm["hbm_achieved_gbps"],
                    peak=workmodel.PEAK_HBM_BYTES / 1e9, unit="GB/s", frac=hbm["hbm_frac"])
    else:
        roof = dict(kernel=dominant, bound="mfma", achieved=mfma["mfma_achieved_tflops"],
                    peak=workmodel.PEAK_BF16_FLOPS / 1e12, unit="TFLOP/s", frac=mfma["mfma_frac"])
    roof.update(traffic=traffic_for(dominant, sha), algorithmic_flops=int(flops), algorithmic_bytes=nbytes,
                flop_per_byte=round(intensity, 1), ridge_flop_per_byte=round(ridge, 1), **mfma, **hbm,
                launch_us=round(launch_s * 1e6, 2), launches=len(timer.ms),
                measured_in=f"{args.steps} config-2 steps with bwd_dkw after the reverse scan "
                            f"({DKW_ENV}=0), {ms_after:.4f} ms/step",
                launch_us_beside_scan=round(statistics.mean(timer_beside.ms) * 1e3, 2))
    total_flops = sum(workmodel.kernel_work(k, bounds, H)[0]
                      for k in workmodel.FWD_KERNELS + workmodel.BWD_KERNELS)

    extra = dict(config2_fwd_bwd_ms=round(ms, 4), config2_fwd_bwd_ms_dkw_after_scan=round(ms_after, 4),
                 config2_tflops=round(total_flops / (ms * 1e-3) / 1e12, 2),
                 config2_mfma_frac=round(total_flops / (ms * 1e-3) / workmodel.PEAK_BF16_FLOPS, 4),
                 lib_sha256=sha)
    if kernels:
        par = [k for k in kernels if k not in workmodel.SCAN_KERNELS]
        f = sum(workmodel.kernel_work(k, bounds, H)[0] for k in par)
        t = sum(kernels[k]["us"] for k in par) * 1e-6
        extra["chunk_kernels_mfma_frac"] = round(f / t / workmodel.PEAK_BF16_FLOPS, 4)
        extra["kernels_config2"] = kernels
    if not args.no_extra:
        log("config 1 fwd+bwd")
        T1, bounds1, step1, _ = training_case(gdn, synthetic, torch, 1, device)
        for _ in range(args.warmup):
            step1()
        ms1 = time_steps(torch, step1, args.steps) * 1e3
        f1 = sum(workmodel.kernel_work(k, bounds1, H)[0] for k in workmodel.FWD_KERNELS + workmodel.BWD_KERNELS)
        extra["config1_fwd_bwd_ms"] = round(ms1, 4)
        extra["config1_tflops"] = round(f1 / (ms1 * 1e-3) / 1e12, 2)
        log("config 3 fwd+bwd (packed documents)")
        T3, bounds3, step3, _ = training_case(gdn, synthetic, torch, 3, device)
        for _ in range(args.warmup):
            step3()
        ms3 = time_steps(torch, step3, max(5, args.steps // 2)) * 1e3
        f3 = sum(workmodel.kernel_work(k, bounds3, H)[0] for k in workmodel.FWD_KERNELS + workmodel.BWD_KERNELS)
        extra["config3_fwd_bwd_ms"] = round(ms3, 4)
        extra["config3_tflops"] = round(f3 / (ms3 * 1e-3) / 1e12, 2)
        extra["config3_documents"] = len(bounds3) - 1
        del step3
        log("config 2 fwd+bwd, fused mode (the backward rebuilds the forward workspace)")
        gdn.MODE = "fused"
        try:
            _, _, stepf, _ = training_case(gdn, synthetic, torch, 2, device)
            for _ in range(args.warmup):
                stepf()
            extra["config2_fused_mode_ms"] = round(time_steps(torch, stepf, args.steps) * 1e3, 4)
        finally:
            gdn.MODE = "cached"
        del stepf
        log("config 2 fwd+bwd, fp16 inputs (fp16 kernels)")
        _, _, steph, _ = training_case(gdn, synthetic, torch, 2, device, fp16=True)
        for _ in range(args.warmup):
            steph()
        extra["config2_fwd_bwd_ms_fp16"] = round(time_steps(torch, steph, args.steps) * 1e3, 4)
        del steph
        log("whole GatedDelta layer, width 2048 (content 2048 and 8192, image-CQ plans)")
        log("layer decode step, width 2048 (N = 1 and 64 sequences)")
        extra["layer_decode_w2048"] = [layer_decode_case(torch, device, n) for n in (1, 64)]
        extra["layer_w2048"] = [dict(layer_case(torch, device, c, nq), reference_ascend910b_ms=ref)
                                for c, nq, ref in ((2048, 1675, 10.46), (8192, 7819, 38.60))]
        log("config 2 prefill")
        T2, mask2, b2 = synthetic.config_events(2, seed=0)
        xs = [x.to(device) for x in synthetic.make_inputs(T2, H, D, seed=2, readonly=mask2)]
        for _ in range(args.warmup):
            gdn.prefill(*xs, b2)
        extra["config2_prefill_ms"] = round(time_steps(torch, lambda: gdn.prefill(*xs, b2), args.steps) * 1e3, 4)
        del xs
        log("config 4 decode")
        extra["decode_config4"] = decode_case(gdn, _lib, workmodel, torch, device, args.decode_steps)
    cpu = None
    if not args.no_cpu:
        log("cpu baseline (config 2 fwd+bwd, fp32 oracle)")
        cpu = cpu_baseline(torch)

    print(json.dumps(dict(
        metric=METRIC,
        value=round(ms, 4),
        unit="ms/layer",
        n_gpus=1,
        steps=args.steps,
        warmup=args.warmup,
        ms_per_step=round(ms, 4),
        higher_is_better=False,
        scaling="weak",
        vs_baseline=None,
        dtype="bf16",
        data="synthetic",
        config=dict(workload="config 2: GDN fwd+bwd, content 8192 + 4x256 read-only CQ query events (T=9216), "
                             "H=16, d=128, chunk 64, bf16 q/k/v, fp32 g/beta/state", events=T, heads=H,
                    head_dim=D, chunk=64, documents=len(bounds) - 1),
        roofline=roof,
        cpu_baseline=cpu,
        extra=extra,
    )), flush=True)


if __name__ == "__main__":
    main()
