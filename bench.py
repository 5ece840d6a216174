#!/usr/bin/env python3
"""Decode tokens/s and achieved HBM GB/s of the batched sparse decode step
(score -> top-k -> fused gather+attention) on one MI355X.

Workload: B=16 requests, context lengths
U[512, 2048] in the reference's draw order (mt19937 seed 7 -> 1207 pages),
32 heads x 128 dims, page size 16, top-k 8, FP32 Q/K/V i.i.d. N(0,1).
A step is one pass of the hot path over the batch with its inputs already in
HBM; the timed region is K steps on one HIP stream bracketed by HIP events.

    python bench.py [--steps K] [--warmup W] [--config 1|2|3|4]
    python bench.py --sweep        dense crossover and context-length sweep

Prints one JSON line (the driver contract).  `roofline` is the dominant
kernel (the single-launch step where the step uses it) against 8 TB/s; its
duration is the timed step's when the step is that one launch (HIP events
around the K timed steps on the launch stream), else the attention stage's
over K back-to-back launches; `traffic` is that kernel's HBM bytes per launch from two
rocprofv3 --pmc passes (FETCH_SIZE, WRITE_SIZE) run as child processes of
this bench, scaled by what the counters read for a plain copy of known size.
`roofline_cold` is the same kernel with the steps rotating over disjoint
copies of the batch, so that more than the 256 MB MALL is touched between
reuses of any byte.  `cpu_baseline` times the CPU oracle (a restatement of
the reference's sparse_cpu) on the same inputs, single-threaded, over a
bounded sample.
"""
from __future__ import annotations

import argparse
import ctypes
import csv
import importlib.util
import json
import math
import os
import pathlib
import shutil
import subprocess
import sys
import tempfile
import time

import numpy as np

ROOT = pathlib.Path(__file__).resolve().parent
PKG_DIR = ROOT / "15-618_dynamic_sparse_decode_amd"

METRIC = "decode tokens/s + achieved HBM GB/s (sparse path), B=16 ragged ctx, top-k 8"
HBM_PEAK_GBPS = 8000.0
MALL_BYTES = 256 << 20

# name: (batch, ctx_lo, ctx_hi, heads, head_dim, page_size, top_k, seed)
CONFIGS = {
    1: (1, 1024, 1024, 32, 128, 16, 8, 7),
    2: (16, 512, 2048, 32, 128, 16, 8, 7),
    3: (32, 32768, 32768, 32, 128, 16, 64, 11),
    4: (64, 4096, 16384, 32, 128, 64, 32, 13),
}

# Configs 1 and 2 are generated in the reference's draw order
# (BuildSyntheticBatch, src/synthetic_data.cpp:23-68) with N(0,1) values:
# one std::mt19937(seed); the lengths (uniform_int_distribution); then per
# request its pages' keys, values and its query from
# std::normal_distribution<float> on the same engine.  That is one sequential
# stream (about 10 s at config 2); configs 3 and 4 (8.6G and 5.6G values)
# use one numpy stream per request instead, generated in parallel.
REFERENCE_ORDER_CONFIGS = (1, 2)
DATA_REFERENCE = ("synthetic: N(0,1) fp32 in the reference draw order: std::mt19937(seed), "
                  "context lengths (uniform_int_distribution), then per request its pages' "
                  "keys, values and its query from std::normal_distribution<float> "
                  "(BuildSyntheticBatch's order, src/synthetic_data.cpp:23-68)")
DATA_STREAMS = ("synthetic: N(0,1) fp32, one numpy PCG64 stream per request "
                "(SeedSequence(seed).spawn(B+1)); context lengths in the reference draw "
                "order (mt19937 + uniform_int)")


def data_for(config):
    return DATA_REFERENCE if config in REFERENCE_ORDER_CONFIGS else DATA_STREAMS


def load_package():
    spec = importlib.util.spec_from_file_location(
        "dsd_amd", PKG_DIR / "__init__.py", submodule_search_locations=[str(PKG_DIR)])
    module = importlib.util.module_from_spec(spec)
    sys.modules["dsd_amd"] = module
    spec.loader.exec_module(module)
    return module


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


class Workload:
    """A config's batch uploaded `copies` times into one pool: copy c holds
    the same pages at ids + c * capacity, so steps can rotate over copies that
    share no cache line."""

    def __init__(self, dsd, torch, config, copies, seed=None):
        B, lo, hi, H, D, ps, k, config_seed = CONFIGS[config]
        seed = config_seed if seed is None else seed
        self.B, self.H, self.D, self.ps, self.k, self.seed = B, H, D, ps, k, seed
        self.lo, self.hi = lo, hi
        self.E = H * D
        self.lengths = dsd.reference_context_lengths(B, lo, hi, seed)
        t0 = time.time()
        if config in REFERENCE_ORDER_CONFIGS:
            self.batch = dsd.SyntheticBatch.reference(H, D, ps, B, lo, hi, seed, "normal")
            if self.batch.context_lengths != list(self.lengths):
                raise RuntimeError("the generator's lengths differ from the reference draw")
        else:
            self.batch = dsd.SyntheticBatch(H, D, ps, self.lengths, seed=seed)
        kp = self.batch.key_pool  # generated here
        log(f"config {config}: B={B} pages={self.batch.total_candidates} "
            f"tokens={sum(self.lengths)} generated in {time.time() - t0:.1f}s")
        self.copies = copies
        cap = self.batch.capacity
        self.pool = dsd.DevicePagePool(H, D, ps, cap * copies)
        t0 = time.time()
        ids = self.batch.live_page_ids()
        counts = self.batch.token_counts[ids]
        offs = ids.astype(np.int64) * ps * self.E
        for c in range(copies):
            self.pool.upload_pages(ids + c * cap, counts, offs, kp.reshape(-1),
                                   self.batch.value_pool.reshape(-1))
        log(f"uploaded {copies} x {2 * cap * ps * self.E * 4 / 1e9:.2f} GB in "
            f"{time.time() - t0:.1f}s")
        dev = torch.device("cuda:0")
        self.q = torch.from_numpy(self.batch.queries).to(dev)
        self.offs = torch.from_numpy(self.batch.cand_offsets).to(dev)
        self.ids = [torch.from_numpy((self.batch.cand_ids + c * cap).astype(np.int32)).to(dev)
                    for c in range(copies)]
        self.out = torch.zeros_like(self.q)
        P = self.batch.total_candidates
        self.scores = torch.zeros(max(1, P), dtype=torch.float32, device=dev)
        self.sel = torch.full((B, max(1, k)), -1, dtype=torch.int32, device=dev)
        self.counts = torch.zeros(B, dtype=torch.int32, device=dev)
        self.sel_total = int(sum(min(k, int(n)) for n in np.diff(self.batch.cand_offsets)))
        self.ctx = dsd.SparseContext(self.pool, k, B, P, self.sel_total)

    def step(self, stream, copy=0):
        b = self.batch
        self.ctx.run_batch_device(self.B, b.total_candidates, b.max_candidates,
                                  self.q.data_ptr(), self.offs.data_ptr(),
                                  self.ids[copy].data_ptr(), self.out.data_ptr(),
                                  self.scores.data_ptr(), self.sel.data_ptr(),
                                  self.counts.data_ptr(), stream)

    def close(self):
        self.ctx.close()
        self.pool.close()


GRAPH_STEPS = 10  # steps per captured graph in the graph-replay timing


def timed(torch, stream, fn, steps):
    """Average ms of `steps` back-to-back calls of fn(i) on `stream`,
    bracketed by HIP events and synchronisations."""
    torch.cuda.synchronize()
    a = torch.cuda.Event(enable_timing=True)
    b = torch.cuda.Event(enable_timing=True)
    a.record(stream)
    for i in range(steps):
        fn(i)
    b.record(stream)
    b.synchronize()
    torch.cuda.synchronize()
    return a.elapsed_time(b) / steps


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    # 100 untimed steps: the device's clocks settle after some 10-15 ms of
    # load, and at config 3 (0.36 ms a step) steps timed after only 5
    # warm-up steps ran about 2 % slower (368-370 against 362 us).
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--config", type=int, default=2, choices=sorted(CONFIGS))
    ap.add_argument("--cpu-sample-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-traffic", action="store_true",
                    help="skip the rocprofv3 counter passes (roofline.traffic = null)")
    ap.add_argument("--sweep", action="store_true",
                    help="dense crossover at config 3 and a context-length sweep (B=16, k 8)")
    ap.add_argument("--seeds", default=None, metavar="A-B",
                    help="the config's step over data seeds A..B (one batch each)")
    ap.add_argument("--traffic-probe", action="store_true",
                    help="internal: the launches the counter passes read")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run a plain device-to-device copy of MIB MiB, 5 times")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build runs the decode step on a single "
              "MI355X (--gpus 1); multi-GPU sharding is design-only.", file=sys.stderr)
        return 2

    # torch first: libdsd_hip.so then binds to the HIP runtime torch loaded,
    # so the process holds a single runtime and torch streams are valid.
    import torch

    if args.copy_calibration > 0:
        copy_calibration(torch, args.copy_calibration)
        return 0

    dsd = load_package()
    if not dsd.gpu_available():
        print("no visible gfx950 GPU", file=sys.stderr)
        return 1
    if args.sweep:
        return sweep(dsd, torch, args)
    if args.traffic_probe:
        return traffic_probe(dsd, torch, args)
    if args.seeds:
        return seed_sweep(dsd, torch, args)

    B, lo, hi, H, D, ps, k, seed = CONFIGS[args.config]
    E = H * D
    # Copies for the cold measurement: enough that the other copies' steps
    # touch more than twice the MALL between two uses of one copy.
    lengths = dsd.reference_context_lengths(B, lo, hi, seed)
    est_step = (sum((c + ps - 1) // ps for c in lengths) * E * 4
                + 2 * min(k * ps, max(lengths)) * B * E * 4)
    copies = 1 if est_step >= 2 * MALL_BYTES else min(8, 1 + math.ceil(2 * MALL_BYTES / est_step))
    w = Workload(dsd, torch, args.config, copies)
    batch = w.batch
    stream = torch.cuda.Stream()
    sptr = stream.cuda_stream

    for _ in range(args.warmup):
        w.step(sptr)
    torch.cuda.synchronize()
    w.ctx.exact_rescored_pages(reset=True)
    ms_per_step = timed(torch, stream, lambda i: w.step(sptr), args.steps)
    w.ctx.device_status()
    rescored = w.ctx.exact_rescored_pages(reset=True)
    launch = w.ctx.last_launch()
    log(f"step {ms_per_step * 1e3:.1f} us over {args.steps} steps; "
        f"{rescored} pages rescored exactly; launch {launch}")

    # The step captured into a graph, GRAPH_STEPS steps per graph, replayed
    # back to back (a captured fused step takes its epoch from a device
    # counter that a one-thread kernel in the graph advances).
    graph = torch.cuda.CUDAGraph()
    torch.cuda.synchronize()
    with torch.cuda.graph(graph, stream=stream):
        for _ in range(GRAPH_STEPS):
            w.step(sptr)
    torch.cuda.synchronize()

    def replay(i):
        with torch.cuda.stream(stream):
            graph.replay()

    replay(0)
    graph_ms = timed(torch, stream, replay, max(2, args.steps // GRAPH_STEPS)) / GRAPH_STEPS
    w.ctx.device_status()
    log(f"graph replay ({GRAPH_STEPS} steps per graph): {graph_ms * 1e3:.1f} us per step")

    # One eager step again: a captured step runs in three kernels when the
    # eager one is the wide launch, and the replays below re-run the last
    # step's form.
    w.step(sptr)
    torch.cuda.synchronize()
    w.ctx.device_status()

    # Per-kernel average durations: K back-to-back launches of one kernel on
    # the same stream.  Stages 0-2 are the three-kernel step (score, select,
    # attention); stage 3 is the single-launch fused step.  Every replay block
    # ends with the context's device status (a failure any replay recorded
    # raises here), and the ids / outputs it leaves must be the timed step's.
    sel_ref = w.sel.cpu().numpy().copy()
    cnt_ref = w.counts.cpu().numpy().copy()
    out_ref = w.out.cpu().numpy().copy()

    def check_replay(stage):
        if stage in (1, 3):
            assert np.array_equal(w.counts.cpu().numpy(), cnt_ref), f"stage {stage} counts"
            sel_now = w.sel.cpu().numpy()
            for r in range(B):
                c = int(cnt_ref[r])
                assert np.array_equal(sel_now[r, :c], sel_ref[r, :c]), \
                    f"stage {stage} replays: request {r} ids {sel_now[r, :c]} != {sel_ref[r, :c]}"
        if stage in (2, 3):
            d = float(np.max(np.abs(w.out.cpu().numpy() - out_ref)))
            assert d <= 1e-4, f"stage {stage} replays: outputs differ by {d}"

    def replay_ms(stage):
        w.ctx.replay_stage(stage, sptr)
        ms = timed(torch, stream, lambda i: w.ctx.replay_stage(stage, sptr), args.steps)
        w.ctx.device_status()
        check_replay(stage)
        return ms

    stage_ms = [replay_ms(stage) for stage in range(3)]
    wide = bool(launch.get("wide"))
    fused_ms = replay_ms(3) if launch["fused"] or wide else None
    log("three-kernel stages us: score %.1f select %.1f attention %.1f"
        % tuple(x * 1e3 for x in stage_ms))
    if fused_ms is not None:
        log(f"{'wide' if wide else 'fused'} single-launch step kernel: {fused_ms * 1e3:.1f} us")

    # Algorithmic bytes per launch (fp32), over the timed step's selection.
    sel_h = sel_ref
    cnt_h = cnt_ref
    sel_tokens = int(sum(int(batch.token_counts[sel_h[r, j]])
                         for r in range(B) for j in range(int(cnt_h[r]))))
    P = batch.total_candidates
    score_bytes = B * E * 4 + P * E * 4 + P * 8
    select_bytes = P * 8 + w.sel_total * 4
    attn_bytes = B * E * 4 + sel_tokens * E * 4 * 2 + B * E * 4
    step_bytes = score_bytes + select_bytes + attn_bytes

    # Cold: the same step rotating over the copies (each copy's bytes were
    # last touched `copies` steps earlier), and the attention stage alone
    # over each copy's selected pages (the same kernel through the dense
    # entry point with the selection as its page lists).
    cold_step_ms = timed(torch, stream, lambda i: w.step(sptr, i % copies), args.steps)
    w.ctx.device_status()
    sel_offs = np.zeros(B + 1, np.int32)
    sel_offs[1:] = np.cumsum(cnt_h)
    sel_flat = np.concatenate([sel_h[r, :int(cnt_h[r])] for r in range(B)]).astype(np.int32)
    dev = torch.device("cuda:0")
    sel_offs_d = torch.from_numpy(sel_offs).to(dev)
    sel_ids_d = [torch.from_numpy(sel_flat + c * batch.capacity).to(dev) for c in range(copies)]
    attn_out = torch.zeros_like(w.q)

    def attention(copy):
        dsd.dense_run_batch_device(w.pool, B, w.q.data_ptr(), sel_offs_d.data_ptr(),
                                   sel_ids_d[copy].data_ptr(), attn_out.data_ptr(), sptr)

    attention(0)
    warm_attn_ms = timed(torch, stream, lambda i: attention(0), args.steps)
    cold_attn_ms = timed(torch, stream, lambda i: attention(i % copies), args.steps)
    attn_diff = float(np.max(np.abs(attn_out.cpu().numpy() - w.out.cpu().numpy())))
    assert attn_diff <= 1e-4, f"attention over the selected lists differs by {attn_diff}"
    log(f"cold ({copies} copies): step {cold_step_ms * 1e3:.1f} us, attention "
        f"{cold_attn_ms * 1e3:.1f} us (warm through the same entry {warm_attn_ms * 1e3:.1f})")

    # PCIe-inclusive rate: the host-buffer entry point (queries and CSR in,
    # outputs out through pinned staging), as the reference's RunBatch.
    host_steps = max(20, min(args.steps * 4, 200))
    run_host = lambda timing: w.ctx.run_batch(batch.queries, batch.cand_offsets, batch.cand_ids,
                                              output_mode=dsd.OUTPUT_OUTPUTS,
                                              timing_mode=timing)
    # The C call as a C++ caller makes it (SparseCudaContext::RunBatch's
    # host buffers): arguments built once, one ctypes call per step.
    lib = dsd.load_library()
    hq = np.ascontiguousarray(batch.queries, np.float32)
    hoffs = np.ascontiguousarray(batch.cand_offsets, np.int32)
    hids = np.ascontiguousarray(batch.cand_ids, np.int32)
    hout = np.zeros_like(hq)
    fptr = lambda a: a.ctypes.data_as(ctypes.POINTER(ctypes.c_float))
    iptr = lambda a: a.ctypes.data_as(ctypes.POINTER(ctypes.c_int))
    host_args = (w.ctx.handle, B, fptr(hq), iptr(hoffs), iptr(hids), dsd.OUTPUT_OUTPUTS,
                 dsd.TIMING_NONE, fptr(hout), None, None, None, None)
    for _ in range(5):
        lib.dsd_sparse_run_batch(*host_args)
    t0 = time.perf_counter()
    for _ in range(host_steps):
        lib.dsd_sparse_run_batch(*host_args)
    host_ms = (time.perf_counter() - t0) * 1e3 / host_steps
    host_diff = float(np.max(np.abs(hout - w.out.cpu().numpy())))
    assert host_diff <= 1e-4, f"host-buffer step differs from the device step by {host_diff}"
    log(f"host-buffer step (PCIe-inclusive): {host_ms * 1e3:.1f} us")
    phases = run_host(dsd.TIMING_EVENTS)["timings"]
    log("timed host step phases us: score %.1f select %.1f attention %.1f kernel %.1f"
        % tuple(phases[k] * 1e3 for k in ("score_ms", "topk_ms", "attention_ms", "kernel_ms")))

    stages = {
        "score": {"us": stage_ms[0] * 1e3, "bytes": score_bytes,
                  "GBps": score_bytes / (stage_ms[0] * 1e-3) / 1e9},
        "select": {"us": stage_ms[1] * 1e3, "bytes": select_bytes,
                   "GBps": select_bytes / (stage_ms[1] * 1e-3) / 1e9},
        "attention": {"us": stage_ms[2] * 1e3, "bytes": attn_bytes,
                      "GBps": attn_bytes / (stage_ms[2] * 1e-3) / 1e9},
        "note": "each kernel of the three-kernel step launched alone, back to back; the select "
                "re-runs with its code warm, so it reads low; step_phases_us times the phases "
                "of one real step",
    }
    if fused_ms is not None:
        stages["wide_step" if wide else "fused_step"] = {
            "us": fused_ms * 1e3, "bytes": step_bytes,
            "GBps": step_bytes / (fused_ms * 1e-3) / 1e9}
        if wide:
            roof_kernel = ("WideStepKernel: score slices, certified top-k (by each request's "
                           "last slice) and fused gather/attention in one launch")
        else:
            roof_kernel = ("FusedStepKernel: page scoring + certified top-k + fused gather/"
                           "attention in one launch")
        # The step is this one launch: its duration is the timed step's
        # (events around the K timed steps, launch gaps included).
        roof_name = "WideStepKernel" if wide else "FusedStepKernel"
        roof_bytes, roof_ms = step_bytes, ms_per_step
        cold_ms = cold_step_ms
    else:
        roof_kernel = "AttentionFastKernel<128,16,8,4> (fused gather + online softmax)"
        roof_name, roof_bytes, roof_ms = "AttentionFastKernel", attn_bytes, stage_ms[2]
        cold_ms = cold_attn_ms
    roof_gbps = roof_bytes / (roof_ms * 1e-3) / 1e9
    attn_gbps = attn_bytes / (stage_ms[2] * 1e-3) / 1e9

    traffic = {"bytes": None, "source": "not measured (--no-traffic)"}
    if not args.no_traffic:
        traffic = measure_traffic(args.config, roof_name)
        log(f"traffic: {traffic}")

    # one copy: a step larger than twice the MALL evicts itself
    touched = (copies - 1) * step_bytes if copies > 1 else step_bytes
    result = {
        "metric": METRIC,
        "value": B / (ms_per_step * 1e-3),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": data_for(args.config),
        "config": {
            "workload": f"BASELINE config {args.config}: sparse decode step, B={B}, ctx "
                        f"U[{lo},{hi}] (seed {seed}), {H}x{D}, page {ps}, top-k {k}",
            "batch": B, "pages": P, "selected_tokens": sel_tokens, "context_tokens": sum(lengths),
            "heads": H, "head_dim": D, "page_size": ps, "top_k": k, "seed": seed,
        },
        "launch": launch,
        "step_hbm_GBps": step_bytes / (ms_per_step * 1e-3) / 1e9,
        "selection": {"mode": "certified intervals + exact sequential rescoring",
                      "exact_rescored_pages_per_step": rescored / args.steps},
        "stages": stages,
        "roofline": {"bound": "hbm", "achieved": roof_gbps, "peak": HBM_PEAK_GBPS,
                     "unit": "GB/s", "frac": roof_gbps / HBM_PEAK_GBPS,
                     "traffic": traffic["bytes"], "traffic_source": traffic["source"],
                     "kernel": roof_kernel, "bytes_per_launch": roof_bytes,
                     "us_per_launch": roof_ms * 1e3,
                     "duration_source": ("the timed steps (one launch per step; HIP events "
                                         "around the K steps on the launch stream)"
                                         if fused_ms is not None else
                                         "the attention stage replayed back to back "
                                         "(HIP events on the launch stream)")},
        # The same kernel with every launch on a copy of the batch last
        # touched `copies` launches earlier: its bytes come from HBM, not the
        # MALL that holds a repeated 86 MB step.
        "roofline_cold": {"bound": "hbm", "achieved": roof_bytes / (cold_ms * 1e-3) / 1e9,
                          "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                          "frac": roof_bytes / (cold_ms * 1e-3) / 1e9 / HBM_PEAK_GBPS,
                          "us_per_launch": cold_ms * 1e3, "copies": copies,
                          "bytes_touched_between_reuses": touched,
                          "step_us": cold_step_ms * 1e3},
        # The BASELINE target is phrased for the fused gather + attention
        # stage (>= 60 % of 8 TB/s at config 2): that stage alone, replayed
        # back to back, warm and rotating over the copies.
        "attention_roofline": {"bound": "hbm", "achieved": attn_gbps, "peak": HBM_PEAK_GBPS,
                               "unit": "GB/s", "frac": attn_gbps / HBM_PEAK_GBPS,
                               "target_frac": 0.6, "bytes_per_launch": attn_bytes,
                               "us_per_launch": stage_ms[2] * 1e3,
                               "cold_us_per_launch": cold_attn_ms * 1e3,
                               "cold_frac": attn_bytes / (cold_attn_ms * 1e-3) / 1e9
                               / HBM_PEAK_GBPS},
        "step_phases_us": {k[:-3]: phases[k] * 1e3
                           for k in ("score_ms", "topk_ms", "attention_ms", "kernel_ms")},
        "graph_replay": {"us_per_step": graph_ms * 1e3, "tokens_per_s": B / (graph_ms * 1e-3),
                         "steps_per_graph": GRAPH_STEPS,
                         "note": "the device step captured into a graph (torch.cuda.CUDAGraph), "
                                 "replayed back to back; each captured fused step adds a "
                                 "one-thread epoch kernel; not the headline value"},
        "host_path": {"us_per_step": host_ms * 1e3, "tokens_per_s": B / (host_ms * 1e-3),
                      "steps": host_steps,
                      "note": "dsd_sparse_run_batch with host buffers (queries and CSR in, "
                              "outputs out; PCIe-inclusive), one C call per step; "
                              "not the headline value"},
        "cpu_baseline": None,
    }

    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(batch, k, w.out, args.cpu_sample_seconds)

    w.close()
    print(json.dumps(result), flush=True)
    return 0


def seed_sweep(dsd, torch, args):
    """The config's default step (as the headline line times it) on the
    batches of several data seeds: how the step time depends on the data
    (near ties at the top-k boundary send a request through refined
    intervals or the exact chain)."""
    a, b = (int(x) for x in args.seeds.split("-"))
    points = []
    for seed in range(a, b + 1):
        w = Workload(dsd, torch, args.config, 1, seed=seed)
        stream = torch.cuda.Stream()
        sptr = stream.cuda_stream
        for _ in range(args.warmup):
            w.step(sptr)
        torch.cuda.synchronize()
        w.ctx.exact_rescored_pages(reset=True)
        ms = timed(torch, stream, lambda i: w.step(sptr), args.steps)
        w.ctx.device_status()
        rescored = w.ctx.exact_rescored_pages(reset=True) / args.steps
        points.append({"seed": seed, "step_us": ms * 1e3, "pages": w.batch.total_candidates,
                       "exact_rescored_pages_per_step": rescored})
        log(f"seed {seed}: step {ms * 1e3:.1f} us ({w.batch.total_candidates} pages)")
        w.close()
    us = np.array([p["step_us"] for p in points])
    print(json.dumps({"mode": "seeds", "config": args.config, "steps": args.steps,
                      "points": points, "median_us": float(np.median(us)),
                      "mean_us": float(np.mean(us)), "min_us": float(np.min(us)),
                      "max_us": float(np.max(us))}), flush=True)
    return 0


def copy_calibration(torch, mib):
    n = mib * (1 << 20) // 4
    src = torch.ones(n, dtype=torch.float32, device="cuda:0")
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_bytes": n * 4, "copies": 5}), flush=True)


def traffic_probe(dsd, torch, args):
    """The launches the counter passes read: 5 steps of the config (its
    dominant kernel), then 3 plain device copies of 256 MiB (the known-size
    kernel that scales the counters)."""
    w = Workload(dsd, torch, args.config, 1)
    stream = torch.cuda.Stream()
    for _ in range(5):
        w.step(stream.cuda_stream)
    torch.cuda.synchronize()
    w.close()
    copy_calibration(torch, 256)
    return 0


COPY_BYTES = 256 << 20


def measure_traffic(config, kernel):
    """HBM bytes per launch of `kernel` from two rocprofv3 --pmc child runs of
    this bench's --traffic-probe mode (FETCH_SIZE, then WRITE_SIZE, KiB per
    dispatch), each scaled by what the same counter reads for the probe's
    256 MiB device copy (which reads and writes 256 MiB)."""
    prof = shutil.which("rocprofv3")
    if prof is None:
        return {"bytes": None, "source": "not measured: rocprofv3 not found"}
    values = {}
    for counter in ("FETCH_SIZE", "WRITE_SIZE"):
        out = tempfile.mkdtemp(prefix="dsd_pmc_", dir="/tmp")
        cmd = [prof, "--pmc", counter, "-d", out, "-o", "pmc", "-f", "csv", "--",
               sys.executable, str(ROOT / "bench.py"), "--traffic-probe", "--config", str(config)]
        env = dict(os.environ, TMPDIR="/tmp")
        try:
            proc = subprocess.run(cmd, cwd="/tmp", env=env, capture_output=True, text=True,
                                  timeout=240)
        except subprocess.TimeoutExpired:
            return {"bytes": None, "source": f"not measured: rocprofv3 --pmc {counter} timed out"}
        rows = []
        for f in pathlib.Path(out).rglob("*counter_collection.csv"):
            rows += list(csv.DictReader(open(f)))
        shutil.rmtree(out, ignore_errors=True)
        rows = [r for r in rows if r.get("Counter_Name") == counter]
        order = lambda r: int(r.get("Dispatch_Id", r.get("Dispatch_ID", 0)) or 0)
        rows.sort(key=order)
        kern = [float(r["Counter_Value"]) for r in rows if kernel in r["Kernel_Name"]]
        # the probe's last three copies are the 256 MiB calibration copies
        copy = [float(r["Counter_Value"]) for r in rows if "copyBuffer" in r["Kernel_Name"]][-3:]
        if not kern or not copy:
            return {"bytes": None,
                    "source": f"not measured: rocprofv3 --pmc {counter} exited {proc.returncode} "
                              f"with {len(kern)} kernel and {len(copy)} copy dispatches"}
        # per dispatch, skipping the first (cold code and TLB) when there are more
        k_avg = float(np.mean(kern[1:] if len(kern) > 1 else kern))
        c_avg = float(np.mean(copy))
        values[counter] = (k_avg, c_avg)
    fetch, wcopy = values["FETCH_SIZE"], values["WRITE_SIZE"]
    scale_f = COPY_BYTES / (fetch[1] * 1024.0)
    scale_w = COPY_BYTES / (wcopy[1] * 1024.0)
    total = fetch[0] * 1024.0 * scale_f + wcopy[0] * 1024.0 * scale_w
    return {"bytes": total,
            "source": f"rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE of {kernel} in two child runs "
                      f"of bench.py --traffic-probe: {fetch[0]:.1f} / {wcopy[0]:.1f} KiB per "
                      f"dispatch, scaled x{scale_f:.3f} / x{scale_w:.3f} by a 256 MiB device copy"}


def sweep(dsd, torch, args):
    """The dense crossover on config 3's inputs and a context-length sweep
    (B=16, page 16, top-k 8, every request at the same length, as the
    reference's experiment/01_decode_context_length_sweep.sh): per point the
    sparse step and dense_gpu on the same pages, each with its algorithmic
    bytes and HBM fraction."""
    stream = torch.cuda.Stream()
    sptr = stream.cuda_stream
    points = [(16, c, 16, 8, 7) for c in (512, 1024, 2048, 4096, 8192, 16384, 32768)]
    points.append((32, 32768, 16, 64, 11))
    rows = []
    for B, ctx_len, ps, k, seed in points:
        H, D = 32, 128
        E = H * D
        t0 = time.time()
        batch = dsd.SyntheticBatch(H, D, ps, [ctx_len] * B, seed=seed)
        pool = dsd.DevicePagePool(H, D, ps, batch.capacity)
        ids = batch.live_page_ids()
        import threading
        lock = threading.Lock()

        def upload(r):
            kk, vv = batch.request_pages(r)
            with lock:
                batch.upload_request(pool, r, kk, vv)

        import concurrent.futures as cf
        with cf.ThreadPoolExecutor(max_workers=16) as ex:
            list(ex.map(upload, range(B)))
        dev = torch.device("cuda:0")
        q = torch.from_numpy(batch.queries).to(dev)
        offs = torch.from_numpy(batch.cand_offsets).to(dev)
        idd = torch.from_numpy(batch.cand_ids).to(dev)
        out = torch.zeros_like(q)
        dense_out = torch.zeros_like(q)
        P = batch.total_candidates
        sel_total = int(sum(min(k, int(n)) for n in np.diff(batch.cand_offsets)))
        ctx = dsd.SparseContext(pool, k, B, P, sel_total)
        sel = torch.full((B, k), -1, dtype=torch.int32, device=dev)
        cnt = torch.zeros(B, dtype=torch.int32, device=dev)

        def sparse(i):
            ctx.run_batch_device(B, P, batch.max_candidates, q.data_ptr(), offs.data_ptr(),
                                 idd.data_ptr(), out.data_ptr(), 0, sel.data_ptr(),
                                 cnt.data_ptr(), sptr)

        def dense(i):
            dsd.dense_run_batch_device(pool, B, q.data_ptr(), offs.data_ptr(), idd.data_ptr(),
                                       dense_out.data_ptr(), sptr)

        for _ in range(3):
            sparse(0)
        sparse_ms = timed(torch, stream, sparse, 20)
        ctx.device_status()
        dense(0)
        dense_ms = timed(torch, stream, dense, 5 if ctx_len >= 16384 else 10)
        sel_h, cnt_h = sel.cpu().numpy(), cnt.cpu().numpy()
        sel_tokens = int(sum(int(batch.token_counts[sel_h[r, j]])
                             for r in range(B) for j in range(int(cnt_h[r]))))
        sparse_bytes = (B * E * 4 + P * E * 4 + P * 8 + P * 8 + sel_total * 4
                        + B * E * 4 + sel_tokens * E * 8 + B * E * 4)
        dense_bytes = B * E * 4 * 2 + B * ctx_len * E * 8
        row = {"batch": B, "context": ctx_len, "top_k": k, "pages": P,
               "launch": ctx.last_launch(),
               "sparse_us": sparse_ms * 1e3, "sparse_bytes": sparse_bytes,
               "sparse_frac": sparse_bytes / (sparse_ms * 1e-3) / 1e9 / HBM_PEAK_GBPS,
               "dense_us": dense_ms * 1e3, "dense_bytes": dense_bytes,
               "dense_frac": dense_bytes / (dense_ms * 1e-3) / 1e9 / HBM_PEAK_GBPS,
               "dense_over_sparse": dense_ms / sparse_ms}
        rows.append(row)
        log(f"B={B} ctx={ctx_len} k={k}: sparse {sparse_ms * 1e3:.1f} us "
            f"({row['sparse_frac']:.3f}), dense {dense_ms * 1e3:.1f} us "
            f"({row['dense_frac']:.3f}), dense/sparse {row['dense_over_sparse']:.1f}x "
            f"[{time.time() - t0:.1f}s]")
        ctx.close()
        pool.close()
        del batch
    print(json.dumps({"mode": "sweep", "data": DATA_STREAMS, "points": rows}), flush=True)
    return 0


def cpu_baseline(batch, k, gpu_out, sample_seconds):
    """The CPU oracle (restated sparse_cpu, 1 thread) on the same inputs, timed
    over whole batches until `sample_seconds` have elapsed."""
    sys.path.insert(0, str(ROOT / "tests"))
    import _oracle as orc

    H, D, ps, E = batch.num_heads, batch.head_dim, batch.page_size, batch.elements
    live = batch.live_page_ids()
    summaries = np.zeros((batch.capacity, E), np.float32)
    summaries[live] = orc.pool_summaries(batch.key_pool, batch.token_counts, E, live)
    iters, elapsed = 0, 0.0
    stage = np.zeros(4)
    outs = None
    while elapsed < sample_seconds or iters == 0:
        t0 = time.perf_counter()
        _, _, outs = orc.sparse_batch(batch.queries, batch.key_pool, batch.value_pool,
                                      summaries, batch.token_counts, batch.cand_offsets,
                                      batch.cand_ids, H, D, ps, k, stage_ms=stage)
        elapsed += time.perf_counter() - t0
        iters += 1
    diff = orc.max_abs_diff(gpu_out.cpu().numpy(), outs)
    return {
        "value": batch.batch * iters / elapsed,
        "unit": "tokens/s",
        "cores": 1,
        "kind": "port",
        "sample": f"{iters} full B={batch.batch} sparse_cpu steps ({elapsed:.1f}s) on 1 thread "
                  f"of {os.cpu_count()} host cores ({cpu_model()})",
        "ms_per_step": elapsed / iters * 1e3,
        "stage_ms_per_step": {"score": stage[0] / iters, "topk": stage[1] / iters,
                              "gather_attention": stage[3] / iters},
        "gpu_vs_cpu_max_abs_diff": diff,
    }


if __name__ == "__main__":
    sys.exit(main())
