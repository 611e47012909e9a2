#!/usr/bin/env python3
"""Benchmark of the MI355X sampling step (one JSON line on stdout).

A step is one arbor_sample call over one batch of synthetic logits already resident in
HBM. The workload is BASELINE.json's headline configuration (c3: B=256, V=128256 fp32,
T=0.7, top-k 50 then top-p 0.95, repetition penalty 1.15 over a 1024-token history).
Input sets are rotated so their total exceeds the 256 MB Infinity Cache plus L2, so each
call reads its logits from HBM.

value       rows/s over the timed steps (synchronize on both sides, events on the
            launch stream at both ends)
roofline    algorithmic bytes per call / average launch duration over the timed region
            (back-to-back launches on the launch stream), against 8 TB/s; a second pass
            with an event pair around every launch is reported beside it (those events add
            a gap per launch); copy_gbs = read+write rate of a device copy of one input set
cpu_baseline  the C oracle (a scalar restatement of the step) on this host, 1 thread,
            on a bounded sample of rows of the same workload; `parallel` beside it is the
            same code with rows spread over the host's threads (the CPU share the box
            grants: OMP_NUM_THREADS, else every core)
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
METRIC = "sampled rows/sec at B=256, V=128256 fp32; achieved HBM GB/s vs roofline"


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=1000,
                    help="untimed steps first (the default also lets the GPU clocks settle)")
    ap.add_argument("--config", default="c3", help="c1..c5 (c3 is the headline)")
    ap.add_argument("--cpu-seconds", type=float, default=10.0, help="CPU-baseline budget")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--step", action="store_true",
                    help="time the generation step (arbor_sample_append: sample, then append the ids to the "
                         "row's history ring) instead of arbor_sample; needs a workload with history")
    ap.add_argument("--sets", type=int, default=0, help="input sets rotated (0 = auto)")
    ap.add_argument("--lm-head", action="store_true",
                    help="time the LM head before the sampler (arbor_lm_head: bf16 [B, H] x packed bf16 "
                         "[H, V] weight + bias -> fp32 logits) at B=256, V=128256 and --lm-hidden")
    ap.add_argument("--lm-hidden", type=int, default=4096)
    ap.add_argument("--copy-bytes", type=int, default=0,
                    help="bytes of the device-to-device copy that gives the practical ceiling and "
                         "calibrates the rocprofv3 counters (default: one input set)")
    return ap.parse_args()


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor()


def traffic_from_profiles(cfg: str):
    """HBM bytes per launch measured with rocprofv3 --pmc (FETCH_SIZE + WRITE_SIZE),
    committed under profiles/ as JSON; None if not measured."""
    f = ROOT / "profiles" / f"traffic_{cfg}.json"
    if not f.exists():
        return None
    try:
        return json.loads(f.read_text()).get("bytes_per_launch")
    except (OSError, ValueError):
        return None


def bench_lm_head(args):
    """One JSON line for the LM head: a step is one arbor_lm_head call producing the fp32
    logits of a batch (B=256, H=--lm-hidden, V=128256: c3's batch and vocabulary) from bf16
    hidden states and the packed bf16 weight, bias added. The weight (2·H·V bytes) is read
    once per call, so the roofline is HBM: algorithmic bytes = weight + x + bias + logits."""
    import torch

    from arbornet_amd import sampling as S

    B, H, V = 256, args.lm_hidden, 128256
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(7)
    w = (torch.randn((H, V), device=dev, generator=g) / H ** 0.5).to(torch.bfloat16)  # [hidden, vocab]
    bias = torch.randn(V, device=dev, generator=g) * 0.1
    head = S.LMHead(w, bias, layout="hv")
    x = torch.randn((B, H), device=dev, generator=g).to(torch.bfloat16)
    out = torch.empty((B, V), dtype=torch.float32, device=dev)
    stream = torch.cuda.current_stream(dev)

    def step():
        head(x, out=out)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    wall0 = time.perf_counter()
    e0.record(stream)
    for _ in range(args.steps):
        step()
    e1.record(stream)
    torch.cuda.synchronize()
    wall1 = time.perf_counter()
    ms = e0.elapsed_time(e1) / args.steps
    # practical reference point: torch's bf16 GEMM of the same operands (hipBLASLt; bf16
    # output, no bias), contiguous [B, H] @ [H, V]
    for _ in range(20):
        torch.matmul(x, w)
    torch.cuda.synchronize()
    e0.record(stream)
    for _ in range(args.steps):
        torch.matmul(x, w)
    e1.record(stream)
    torch.cuda.synchronize()
    mm_ms = e0.elapsed_time(e1) / args.steps
    wbytes = int(head.packed.numel())
    nbytes = wbytes + B * H * 2 + V * 4 + B * V * 4
    flops = 2.0 * B * H * V
    gbs = nbytes / (ms / 1e3) / 1e9
    tflops = flops / (ms / 1e3) / 1e12
    cpu = None
    if not args.no_cpu_baseline:
        # numpy fp32 GEMM (threaded BLAS) of the reference's product on a column sample
        cols = 4096
        xh = x.float().cpu().numpy()
        wh = w[:, :cols].float().cpu().numpy()
        bh = bias[:cols].cpu().numpy()
        n, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < max(1.0, args.cpu_seconds / 2):
            _ = xh @ wh + bh
            n += 1
        el = time.perf_counter() - t0
        thr = int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or (os.cpu_count() or 1)
        cpu = {
            "value": round(B * n / el * cols / V, 1), "unit": "rows/s", "cores": thr, "kind": "port",
            "sample": f"numpy fp32 x[{B},{H}] @ W[{H},{cols}] + bias, {n} times in {el:.1f} s, scaled to V={V} "
                      f"({cpu_model()})",
        }
    out_line = {
        "metric": f"LM-head logits rows/sec at B={B}, H={H}, V={V} (bf16 operands, fp32 logits + bias)",
        "value": round(B / (ms / 1e3), 1),
        "unit": "rows/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": f"lm_head: B={B} H={H} V={V}, weight [H, V] bf16 packed, fp32 logits",
                   "wall_s_timed": round(wall1 - wall0, 4)},
        "roofline": {
            "bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None, "algorithmic_bytes": nbytes,
            "mfma_tflops": round(tflops, 1), "mfma_frac": round(tflops / 2500.0, 4),
            "torch_bf16_mm_ms": round(mm_ms, 5),
        },
        "cpu_baseline": cpu,
    }
    print(json.dumps(out_line), flush=True)


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (the sampling step does not shard across GPUs in this "
              f"build); got --gpus {args.gpus}", file=sys.stderr)
        sys.exit(2)

    import torch

    from arbornet_amd import sampling as S
    from arbornet_amd import synthetic as syn

    if not torch.cuda.is_available():
        print("bench.py needs a HIP device", file=sys.stderr)
        sys.exit(1)
    S.library()
    if args.lm_head:
        bench_lm_head(args)
        return
    w = syn.CONFIGS[args.config]
    dev = torch.device("cuda:0")
    inp = syn.generate(w)
    set_bytes = w.algorithmic_bytes()
    nsets = args.sets or max(2, int(np.ceil((288 << 20) * 1.5 / set_bytes)))
    nsets = min(nsets, 16)

    def dev_copy(a):
        if a is None:
            return None
        if a.dtype == np.uint16:
            return torch.from_numpy(a.view(np.int16)).to(dev).view(torch.bfloat16)
        if a.dtype == np.uint32:
            return torch.from_numpy(a.view(np.int32)).to(dev)
        return torch.from_numpy(a).to(dev)

    base = [dev_copy(inp.logits), dev_copy(inp.history), dev_copy(inp.mask), dev_copy(inp.uniforms)]
    sets = [base] + [[None if t is None else t.clone() for t in base] for _ in range(nsets - 1)]
    p = S.params_for(w)
    need = S.workspace_bytes(p)
    ws = torch.zeros(need, dtype=torch.uint8, device=dev)
    ids = [torch.empty(w.batch, dtype=torch.int32, device=dev) for _ in range(nsets)]
    stream = torch.cuda.current_stream(dev)
    sh = stream.cuda_stream

    if args.step and w.hist_len <= 0:
        print(f"--step needs a workload with history; {args.config} has none", file=sys.stderr)
        sys.exit(2)
    positions = [torch.zeros(w.batch, dtype=torch.int32, device=dev) for _ in range(nsets)]

    def step(i):
        x, h, m, u = sets[i % nsets]
        if args.step:  # the history tensor is the ring the sampled ids are appended to
            st = S.sample_append_raw(p, x.data_ptr(), h.data_ptr(), positions[i % nsets].data_ptr(),
                                     None if m is None else m.data_ptr(), u.data_ptr(), ids[i % nsets].data_ptr(),
                                     None, ws.data_ptr(), need, sh)
        else:
            st = S.sample_raw(p, x.data_ptr(), None if h is None else h.data_ptr(),
                              None if m is None else m.data_ptr(), u.data_ptr(), ids[i % nsets].data_ptr(),
                              None, ws.data_ptr(), need, sh)
        if st != 0:
            S.check(st)

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()

    # timed region: K steps bracketed by synchronisation, events on the launch stream
    t_all0 = torch.cuda.Event(enable_timing=True)
    t_all1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    wall0 = time.perf_counter()
    t_all0.record(stream)
    for i in range(args.steps):
        step(i)
    t_all1.record(stream)
    torch.cuda.synchronize()
    wall1 = time.perf_counter()
    total_ms = t_all0.elapsed_time(t_all1)
    ms_per_step = total_ms / args.steps
    rows_per_s = w.batch / (ms_per_step / 1e3)

    # kernel duration: the same K steps again, an event pair around every launch on the
    # launch stream (kept out of the throughput region: each timing event adds a gap
    # between kernels)
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps)]
    torch.cuda.synchronize()
    for i in range(args.steps):
        starts[i].record(stream)
        step(i)
        ends[i].record(stream)
    torch.cuda.synchronize()
    per_launch_ms = np.array([s.elapsed_time(e) for s, e in zip(starts, ends)])
    kernel_ms = float(per_launch_ms.mean())

    # practical ceiling: a device-to-device copy (one input set unless --copy-bytes)
    copy_bytes = args.copy_bytes or int(set_bytes)
    src = torch.empty(copy_bytes, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    dst.copy_(src)
    c0, c1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    c0.record(stream)
    for _ in range(5):
        dst.copy_(src)
    c1.record(stream)
    torch.cuda.synchronize()
    copy_gbs = 2 * copy_bytes * 5 / (c0.elapsed_time(c1) / 1e3) / 1e9
    del src, dst

    # sanity: ids are token ids or sentinels
    got = ids[0].cpu().numpy()
    assert np.all((got >= 0) & (got < w.vocab)), "bench produced out-of-range ids"

    # average launch duration over the timed region (back-to-back launches on one stream;
    # agrees with rocprofv3's kernel-trace average), per-launch event pairs as a cross-check
    achieved_gbs = set_bytes / (ms_per_step / 1e3) / 1e9
    roofline = {
        "bound": "hbm",
        "achieved": round(achieved_gbs, 1),
        "peak": HBM_PEAK_GBS,
        "unit": "GB/s",
        "frac": round(achieved_gbs / HBM_PEAK_GBS, 4),
        "traffic": None if args.step else traffic_from_profiles(args.config),
        "algorithmic_bytes": set_bytes,
        "launch_ms_mean": round(ms_per_step, 5),
        "event_pair_ms_mean": round(kernel_ms, 5),
        "event_pair_ms_median": round(float(np.median(per_launch_ms)), 5),
        "copy_gbs": round(copy_gbs, 1),
    }

    cpu = None
    if not args.no_cpu_baseline:
        from oracle import oracle

        def timed(threads: int, seconds: float):
            # bounded sample: whole batches of the same workload until `seconds` have passed
            n = 0
            t0 = time.perf_counter()
            while True:
                oracle.sample(p, inp.logits, inp.history, inp.mask, inp.uniforms, threads=threads)
                n += w.batch
                if time.perf_counter() - t0 >= seconds:
                    return n, time.perf_counter() - t0

        rows, el = timed(1, args.cpu_seconds)
        nthr = max(1, min(os.cpu_count() or 1, int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or 10**6))
        prows, pel = timed(nthr, max(1.0, args.cpu_seconds / 4))
        cpu = {
            "value": round(rows / el, 1),
            "unit": "rows/s",
            "cores": 1,
            "kind": "port",
            "sample": f"{rows} rows ({rows // w.batch} full {args.config} batches) in {el:.1f} s, "
                      f"1 thread of {os.cpu_count()} ({cpu_model()}), inputs in host memory",
            "parallel": {
                "value": round(prows / pel, 1),
                "threads": nthr,
                "sample": f"{prows} rows in {pel:.1f} s, rows split over {nthr} threads",
            },
        }

    out = {
        "metric": METRIC,
        "value": round(rows_per_s, 1),
        "unit": "rows/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32" if w.dtype == "f32" else "bf16",
        "data": "synthetic",
        "config": {
            "workload": f"{args.config}: B={w.batch} V={w.vocab} {w.dtype} T={w.temperature} top_k={w.top_k} "
                        f"top_p={w.top_p} min_p={w.min_p} rep={w.repetition_penalty} freq={w.frequency_penalty} "
                        f"pres={w.presence_penalty} H={w.hist_len} mask={w.has_mask}"
                        + (" (generation step: sample + history-ring append)" if args.step else ""),
            "batch": w.batch,
            "vocab": w.vocab,
            "input_sets_rotated": nsets,
            "wall_s_timed": round(wall1 - wall0, 4),
        },
        "roofline": roofline,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
