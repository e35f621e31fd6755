"""Handoff map + paged install throughput on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload tp4]

A step is one complete handoff of the workload: every target (layer, KV
head) of the 4096-token history is mapped from its assigned source (layer,
head) and installed into the target's paged pool through the request's block
table (one fused kernel launch). Inputs (source pool, slots, target pool,
block table, packed maps) are resident in HBM before the timed region.

Prints one JSON line. ``value`` is mapped+installed KV tokens/s of the whole
job; ``roofline`` prices the fused kernel's algorithmic HBM bytes (target
writes + distinct source rows read once + fp32-equivalent maps + token index)
per launch against MI355X HBM peak, from HIP events recorded around every
launch on its stream; ``cpu_baseline`` times the CPU oracle on the box's host
cores on the same workload.
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
METRIC = "mapped+installed KV tokens/s at Qwen3-14B→32B shape; 4k-token handoff latency"

WORKLOADS = {
    "tp4": "Qwen3-14B->32B, one TP4 rank: source 40 layers x 2 KV heads -> target 64 layers x 2 "
           "KV heads, head_dim 128, 4096 tokens, bf16, 16 of 40 source layers selected, page 16, "
           "65536-page target pool with a shuffled free list",
    "full": "Qwen3-14B->32B whole model on one GPU: source 40x8 -> target 64x8 KV heads, head_dim "
            "128, 4096 tokens, bf16, page 16, 8192-page target pool",
    "full32k": "Qwen3-14B->32B whole model, long history: source 40x8 -> target 64x8 KV heads, "
               "head_dim 128, 32768 tokens, bf16, page 16, 4096-page target pool",
    "batch": "64 ragged requests (lognormal lengths, median 2048, sigma 0.5, clipped to [256, 16384]; "
             "137,440 tokens) in one launch at the Qwen3-14B->32B TP4 share (40x2 -> 64x2 KV heads, "
             "head_dim 128, bf16) into a shared 0.92 M-slot target pool at 85% occupancy (page 16)",
    "batch_full": "the same 64 ragged requests in one launch at the whole-model geometry (40x8 -> 64x8 "
                  "KV heads, head_dim 128, bf16) into a shared target pool at 50% occupancy (page 16)",
    "gemma": "Gemma-3-style target: source 40x8 -> target 62x16 KV heads (10 global layers keep all "
             "8192 tokens, 52 sliding-window layers keep the last 1023), head map h_src = h // 2, "
             "theta 1e4 local / 1e6 global, head_dim 128, bf16, page 16",
}


def time_handoff(h, steps: int, warmup: int, tokens_per_workgroup: int = 0):
    """Time ``steps`` back-to-back handoffs.

    Returns the wall time of the timed region, the GPU time per launch over
    that region (one HIP event pair on the launch stream around all of its
    launches: nothing else is enqueued between them), and the mean and
    minimum of single-launch latencies from a second, untimed pass that puts
    an event pair around each launch (those events add their own dispatch
    gaps, so they stay out of the timed region).
    """
    import torch

    for _ in range(warmup):
        h.run(tokens_per_workgroup=tokens_per_workgroup)
    stream = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    e0.record(stream)
    for _ in range(steps):
        h.run(tokens_per_workgroup=tokens_per_workgroup)
    e1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    region_ms = e0.elapsed_time(e1) / steps
    n = min(steps, 50)
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(n)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(n)]
    for i in range(n):
        starts[i].record(stream)
        h.run(tokens_per_workgroup=tokens_per_workgroup)
        ends[i].record(stream)
    torch.cuda.synchronize()
    launch_ms = [s.elapsed_time(e) for s, e in zip(starts, ends)]
    if h.mapper.plan.read_errors() != 0:
        raise RuntimeError("kernel flagged out-of-range rows")
    return wall, region_ms, statistics.fmean(launch_ms), min(launch_ms)


def publish_ready_latency(h, block: int = 2048, repeats: int = 10) -> dict:
    """First enqueue -> publish-ready wall time of the unpublished install
    transaction over the workload: ``install_unpublished`` with one fused
    map + install launch per ``block`` tokens on a side stream and that
    stream's fence after each block (the reference's 2048-token blocks)."""
    import torch

    from cachebridge_amd.online.blocks import install_unpublished, map_install_block

    n = h.tokens
    stream = torch.cuda.Stream()
    marks = {}

    def write(value, table, start):
        marks.setdefault("first", time.perf_counter())
        map_install_block(h.mapper, h.source_pool, h.source_slots, h.target_pool, start=start,
                          stop=start + value.shape[0], block_table=table, page_size=h.shape.page_size,
                          prefix_length=n, stream=stream)

    def publish(table):
        marks["publish"] = time.perf_counter()

    def transaction() -> float:
        marks.clear()
        install_unpublished(token_count=n, allocate=lambda k: h.block_table, free=lambda t: None,
                            blocks=((a, min(n, a + block), h.source_slots[a:min(n, a + block)])
                                    for a in range(0, n, block)),
                            write=write, synchronize=stream.synchronize, ready_vote=lambda ok: ok,
                            publish=publish)
        return marks["publish"] - marks["first"]

    transaction()
    times = sorted(transaction() for _ in range(repeats))
    if h.mapper.plan.read_errors() != 0:
        raise RuntimeError("kernel flagged out-of-range rows")
    return {"median_ms": round(1e3 * statistics.median(times), 4), "min_ms": round(1e3 * times[0], 4),
            "blocks": -(-n // block), "block_tokens": block, "transactions": repeats}


def host_cpu() -> dict:
    """Host CPU: the whole /proc/cpuinfo "model name" of the first CPU with its
    family / model / stepping numbers (a virtual machine may report a generic
    name), and the affinity size."""
    fields, sockets = {}, set()
    try:
        for line in open("/proc/cpuinfo"):
            key, _, val = line.partition(":")
            key, val = key.strip(), val.strip()
            if key in ("model name", "cpu family", "model", "stepping") and key not in fields:
                fields[key] = val
            elif key == "physical id":
                sockets.add(val)
    except OSError:
        pass
    model = fields.get("model name", "")
    ids = ", ".join(f"{k} {fields[k]}" for k in ("cpu family", "model", "stepping") if k in fields)
    return {"model": f"{model} ({ids})" if ids else model,
            "affinity_cpus": len(os.sched_getaffinity(0)), "sockets": len(sockets) or None}


def _cpu_batch(workload: str, count: int | None = None):
    """CPU-oracle handoffs of the seeded ragged requests (``count`` first, all 64
    by default), one request after another, as a callable returning the summed
    seconds and the tokens mapped."""
    import torch

    from cachebridge_amd import synthetic
    from oracle import install as oi

    lengths = synthetic.request_lengths()
    lengths = lengths if count is None else lengths[:count]
    sh = synthetic.shape(workload, tokens=max(lengths))
    spec = synthetic.mapper_spec(sh)
    longest = max(lengths)
    values = synthetic.source_values(sh)
    src = oi.RowStorePool(sh.source_layers, longest, sh.source_heads, sh.head_dim, dtype=sh.dtype,
                          fill=values)
    del values
    tgt = oi.RowStorePool(sh.target_layers, longest, sh.target_heads, sh.head_dim, dtype=sh.dtype)
    slots = torch.randperm(longest, generator=torch.Generator().manual_seed(5))

    def once() -> float:
        total = 0.0
        for n in lengths:
            t0 = time.perf_counter()
            oi.map_install_oracle(src, torch.arange(n), tgt, slots[:n], spec, position_start=0,
                                  source_theta=sh.source_theta, target_thetas=sh.target_theta,
                                  windows=sh.windows, prefix_length=n)
            total += time.perf_counter() - t0
        return total

    return once, sum(lengths)


def _cpu_handoff(workload: str, tokens: int):
    """One full CPU-oracle handoff of ``workload`` as a callable returning seconds."""
    import torch

    from cachebridge_amd import synthetic
    from oracle import install as oi

    sh = synthetic.shape(workload, tokens=tokens)
    spec = synthetic.mapper_spec(sh)
    values = synthetic.source_values(sh)
    src = oi.RowStorePool(sh.source_layers, tokens, sh.source_heads, sh.head_dim, dtype=sh.dtype,
                          fill=values)
    del values
    tgt = oi.RowStorePool(sh.target_layers, tokens, sh.target_heads, sh.head_dim, dtype=sh.dtype)
    slots = torch.randperm(tokens, generator=torch.Generator().manual_seed(5))
    thetas = sh.target_theta

    def once() -> float:
        t0 = time.perf_counter()
        oi.map_install_oracle(src, torch.arange(tokens), tgt, slots, spec, position_start=0,
                              source_theta=sh.source_theta, target_thetas=thetas,
                              windows=sh.windows, prefix_length=tokens)
        return time.perf_counter() - t0

    return once


def _timed_cpu(once, threads: int, runs: int, warm: bool = True) -> tuple[float, int]:
    import torch

    prev = torch.get_num_threads()
    try:
        torch.set_num_threads(threads)
        if warm:
            once()
        times = [once() for _ in range(runs)]
    finally:
        torch.set_num_threads(prev)
    return statistics.median(times), len(times)


def cpu_baseline(workload: str, tokens: int, *, runs: int = 5, extra: bool = True) -> dict:
    """CPU oracle (torch fp32, op for op as the reference mapper + row-store install).

    Protocol: all ``sched_getaffinity`` CPUs as torch threads, one warm-up,
    median of ``runs`` full handoffs (weight packing excluded, map and install
    included); the same at 16 threads (the box's nominal CPU share), and the
    better of the two is ``value`` with its thread count in ``cores``. One
    single-thread handoff is timed as well (the reference CI's
    ``OMP_NUM_THREADS=1``). With ``extra``, the other configurations are timed
    at all CPUs (median of 3): the toy fp32 mapper, the Gemma-style target and
    the 64x8 target at T 32768 (at T 4096, labelled, when one run exceeds 60 s).
    """
    host = host_cpu()
    all_cpus = host["affinity_cpus"]
    once = _cpu_handoff(workload, tokens)
    med_all, n_all = _timed_cpu(once, all_cpus, runs)
    med16, n16 = (med_all, n_all) if all_cpus <= 16 else _timed_cpu(once, 16, runs)
    best, cores = (med_all, all_cpus) if med_all <= med16 else (med16, 16)
    single, _ = _timed_cpu(once, 1, 1)
    del once
    out = {"value": round(tokens / best, 1), "unit": "tokens/s", "cores": cores, "kind": "port",
           "sample": f"full {workload} handoff, {tokens} tokens, all target layers/heads; torch fp32 oracle "
                     f"incl. un-RoPE + row-store install; warm-up + median of {n_all}",
           "cpu_model": host["model"], "affinity_cpus": all_cpus,
           "handoff_s_all_cpus": round(med_all, 4), "handoff_s_16_threads": round(med16, 4),
           "single_thread_value": round(tokens / single, 1)}
    if extra:
        configs = {}
        # C4: the 64 seeded ragged requests (137,440 tokens, TP4 share), one
        # CPU handoff per request, summed; one run (about 10 s at 16 threads).
        batch_once, batch_tokens = _cpu_batch("batch")
        batch_s, _ = _timed_cpu(batch_once, all_cpus, 1, warm=False)
        configs["batch"] = {"tokens": batch_tokens, "label": "batch: 64 requests summed, TP4 share",
                            "handoff_s": round(batch_s, 4), "tokens_per_s": round(batch_tokens / batch_s, 1),
                            "runs": 1, "threads": all_cpus}
        del batch_once
        for name, t in (("toy", 256), ("gemma", 8192), ("full32k", 32768)):
            label = name
            probe = _cpu_handoff(name, t)
            first, _ = _timed_cpu(probe, all_cpus, 1, warm=False)  # doubles as the warm-up
            if first > 60.0 and t > 4096:
                del probe
                label = f"{name} at T 4096 (one run at the full T {t} took {first:.1f} s)"
                t = 4096
                probe = _cpu_handoff(name, t)
                _timed_cpu(probe, all_cpus, 1, warm=False)
            med, n = _timed_cpu(probe, all_cpus, 3, warm=False)
            del probe
            configs[name] = {"tokens": t, "label": label, "handoff_s": round(med, 4),
                             "tokens_per_s": round(t / med, 1), "runs": n, "threads": all_cpus}
        # One thread (the reference CI's OMP_NUM_THREADS=1) on a bounded
        # sample of every configuration, a few seconds each.
        single = {}
        for name, t in (("toy", 256), ("full", 1024), ("gemma", 512)):
            probe = _cpu_handoff(name, t)
            sec, _ = _timed_cpu(probe, 1, 1, warm=False)
            del probe
            single[name] = {"tokens": t, "handoff_s": round(sec, 4), "tokens_per_s": round(t / sec, 1)}
        batch_once, batch_tokens = _cpu_batch("batch", count=4)
        sec, _ = _timed_cpu(batch_once, 1, 1, warm=False)
        single["batch"] = {"tokens": batch_tokens, "requests": 4, "handoff_s": round(sec, 4),
                           "tokens_per_s": round(batch_tokens / sec, 1)}
        del batch_once
        out["configs"] = configs
        single["tp4"] = {"tokens": tokens, "handoff_s": round(tokens / out["single_thread_value"], 4),
                         "tokens_per_s": out["single_thread_value"]} if workload == "tp4" else None
        out["single_thread"] = {"threads": 1, "sample": "the first `tokens` tokens of each configuration "
                                "(toy and the TP4 share in full; full stands for full32k too, the same "
                                "40x8 -> 64x8 geometry; batch: its first 4 requests summed)",
                                "configs": single}
    return out


SAMPLE_LAYERS = [0, 1, 17, 31, 32, 47, 62, 63]


def sampled_parity(h, sh, label: str) -> dict:
    """Oracle check of the installed rows of the benchmarked handoff.

    Part of the CPU-baseline leg (the oracle is the checker here, never the
    thing measured): after the timed region, the CPU oracle maps the first,
    middle and last 64 tokens of the history (and both sides of any window
    edge) for 8 target layers, all heads, K and V, from the source rows read
    back from the GPU pool, and the GPU's installed rows at those tokens' slots
    are compared with it to the parity bar of ``oracle.tolerance.check_mapped``
    (1 bf16 ulp, or 2^-14 of the summand magnitude for near-cancelling
    elements; >= 99.9% within 1 ulp; normwise and element-wise relative error
    <= 1e-2).
    """
    import torch

    from cachebridge_amd import synthetic
    from tests import fullsize as fs

    n = sh.tokens
    dev = h.target_pool.k_data.device
    tgt_slots = synthetic.slots_from_pages(h.block_table.cpu(), n, sh.page_size).to(dev)
    first = fs.first_kept(sh.windows, sh.target_layers, prefix=n)
    layers = [l for l in SAMPLE_LAYERS if l < sh.target_layers]
    h.run()
    torch.cuda.synchronize()
    if h.mapper.plan.read_errors() != 0:
        raise RuntimeError("kernel flagged out-of-range rows")
    out = {"workload": label, "sample": f"tokens {fs.token_windows(n, edges=sorted({f for f in first if f}))} "
                                        f"x target layers {layers} x all heads x K/V"}
    try:
        stats = []
        for lo, hi in fs.token_windows(n, edges=sorted({f for f in first if f})):
            stats += fs.oracle_window(h.source_pool, h.source_slots, h.target_pool, tgt_slots, h.spec,
                                      lo=lo, hi=hi, position_start=0, layers=layers,
                                      source_theta=sh.source_theta, target_thetas=sh.target_theta,
                                      first=first)
        summary = fs.summarize(stats)
        out.update(ok=True, elements=summary["elements"], within_1ulp=round(summary["within_1ulp"], 6),
                   beyond_1ulp_fraction=round(summary["beyond_1ulp_fraction"], 6),
                   max_ulp=summary["max_ulp"], max_rel_norm=round(summary["max_rel_norm"], 6),
                   max_rel_elem=round(summary["max_rel_elem"], 6),
                   rel_elem_fraction=round(summary["rel_elem_fraction"], 6),
                   rel_elem_rule="elements with |ref| >= 100 x their near-cancellation allowance")
    except AssertionError as e:
        out.update(ok=False, error=str(e)[:400])
    return out


KERNEL_SOURCE = ROOT / "cachebridge_amd" / "csrc" / "cb_handoff.hip"


def kernel_source_sha16() -> str:
    import hashlib

    return hashlib.sha256(KERNEL_SOURCE.read_bytes()).hexdigest()[:16]


def profiled_traffic(kernel: str, workload: str) -> tuple[int | None, str]:
    """HBM bytes per launch from a committed profiler-counter summary, and where it came from.

    ``profiles/<kernel>_<workload>_traffic.md`` holds ``traffic_bytes_per_launch
    = N`` (from ``rocprofv3 --pmc FETCH_SIZE`` and ``--pmc WRITE_SIZE`` runs of
    this script, each scaled by the same counter's reading for a plain copy of
    known size) and ``kernel_source_sha16 = H``, the first 16 hex digits of the
    SHA-256 of the kernel source it was measured on. The figure is not measured
    in this run: it is returned only while the kernel source still hashes to H,
    and is None otherwise.
    """
    path = ROOT / "profiles" / f"{kernel}_{workload}_traffic.md"
    rel = path.relative_to(ROOT).as_posix()
    if not path.exists():
        return None, "not measured"
    fields = {}
    for line in path.read_text().splitlines():
        if "=" in line and line.split("=", 1)[0].strip() in ("traffic_bytes_per_launch",
                                                              "kernel_source_sha16", "measured"):
            k, v = line.split("=", 1)
            fields[k.strip()] = v.strip()
    now = kernel_source_sha16()
    if fields.get("kernel_source_sha16") != now:
        return None, (f"{rel} was measured on kernel source {fields.get('kernel_source_sha16', '(unrecorded)')}, "
                      f"not the current {now}: not used")
    return int(fields["traffic_bytes_per_launch"]), (
        f"{rel}: rocprofv3 FETCH_SIZE x2 + WRITE_SIZE x1 per dispatch ({fields.get('measured', 'undated')}, "
        f"kernel source {now}); not measured in this run")


def copy_calibration(mib: int = 1024, steps: int = 5) -> None:
    """Plain row copy of ``mib`` MiB (read + write) with the library's copy kernel.

    Used to scale the profiler's FETCH_SIZE / WRITE_SIZE counters: the copy
    moves exactly ``mib`` MiB each way per launch.
    """
    import torch

    from cachebridge_amd.plan import copy_rows, rows_from_page

    rows = mib * 1024 * 1024 // (2 * 256)  # [2, 1, rows, 1, 128] bf16 = mib MiB
    src = torch.randn(2, 1, rows, 1, 128, device="cuda").to(torch.bfloat16)
    dst = torch.empty_like(src)
    for _ in range(steps):
        copy_rows(rows_from_page(src), rows_from_page(dst), num_layers=1, num_tokens=rows,
                  row_elements=128)
    torch.cuda.synchronize()
    assert torch.equal(src, dst)
    print(json.dumps({"copy_calibration_mib": mib, "launches": steps}), flush=True)


FP32_MFMA_PEAK_TFLOPS = 157.3
DELTA_STATE = dict(layers=48, heads=32, dim=128)


def delta_state_bench(steps: int, warmup: int) -> dict:
    """Recurrent-state transform A^T U B of a Qwen3.5-style hybrid model: one
    fp32 [128, 128] state per (linear-attention layer, value head) with its own
    key and value bases, all in one launch of cb_delta_state_transform."""
    import torch

    from cachebridge_amd import architectures

    n = DELTA_STATE["layers"] * DELTA_STATE["heads"]
    d = DELTA_STATE["dim"]
    g = torch.Generator(device="cuda").manual_seed(5)
    u = torch.randn(n, d, d, device="cuda", generator=g)
    a = torch.randn(n, d, d, device="cuda", generator=g) / d ** 0.5
    b = torch.randn(n, d, d, device="cuda", generator=g) / d ** 0.5
    for _ in range(warmup):
        architectures.transform_delta_state(u, a, b)
    stream = torch.cuda.current_stream()
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        starts[i].record(stream)
        architectures.transform_delta_state(u, a, b)
        ends[i].record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    kernel_ms = statistics.fmean(s.elapsed_time(e) for s, e in zip(starts, ends))
    flops = n * 2 * 2 * d ** 3
    bytes_alg = n * 4 * d * d * 4
    tflops = flops / (kernel_ms * 1e-3) / 1e12
    return {
        "metric": "recurrent-state transforms/s (A^T U B, fp32 128x128, Qwen3.5-style 48 layers x 32 heads)",
        "value": round(steps * n / wall, 1), "unit": "matrices/s", "n_gpus": 1, "steps": steps,
        "warmup": warmup, "ms_per_step": round(wall / steps * 1e3, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f32", "data": "synthetic (seeded N(0,1) states, "
        "N(0,1/128) bases)",
        "config": {"workload": f"{n} recurrent states [{d}x{d}] fp32 with per-state bases", **DELTA_STATE},
        "roofline": {"bound": "mfma", "achieved": round(tflops, 2), "peak": FP32_MFMA_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(tflops / FP32_MFMA_PEAK_TFLOPS, 4), "traffic": None,
                     "kernel": "delta_state128_kernel (fp32, 128x128)", "algorithmic_flops_per_launch": flops,
                     "algorithmic_bytes_per_launch": bytes_alg,
                     "hbm_gbs": round(bytes_alg / (kernel_ms * 1e-3) / 1e9, 1),
                     "kernel_ms_mean": round(kernel_ms, 5)},
    }


SPIN_CYCLES = 200_000_000  # GPU spin ahead of short timed launches (tens of ms)


def _delivered_handoff(tokens: int, steps: int, warmup: int, *, two_streams_only: bool = False) -> dict:
    """Block-wise handoff of a TP4-share prefix of ``tokens`` through two
    2048-token receiver slots: delivery then map per block on one stream, the
    same with delivery on its own stream (a block's gather overlaps the map of
    the block before it), and the fused map from the pool. Milliseconds per
    handoff, device time of ``steps`` handoffs back to back."""
    import torch

    from cachebridge_amd import synthetic
    from cachebridge_amd.online.delivery import SelectedBlockDelivery, map_install_delivered

    sh = synthetic.shape("tp4", tokens=tokens)
    h = synthetic.make_handoff(sh, target_pages=max(4096, 4 * ((tokens + 15) // 16)), device_source=True)
    block = 2048
    compute = torch.cuda.current_stream()
    spans = [(a, min(a + block, sh.tokens)) for a in range(0, sh.tokens, block)]
    out = {"tokens": tokens, "blocks": len(spans)}

    def timed(fn) -> float:
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda._sleep(SPIN_CYCLES)  # the host enqueues while the GPU spins
        e0.record(compute)
        for _ in range(steps):
            fn()
        e1.record(compute)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / steps

    for label, stream in (("one_stream_ms", None), ("two_stream_ms", torch.cuda.Stream())):
        d = SelectedBlockDelivery(h.source_pool, h.source_slots, layers=h.mapper.source_layers,
                                  block_tokens=block, stream=stream)

        def handoff():
            if d.stream != compute:  # no delivery runs ahead of the timed region or the last handoff
                d.stream.wait_stream(compute)
            for i, (a, b) in enumerate(spans):
                d.deliver(i % 2, a, b)
                map_install_delivered(h.mapper, d, i % 2, h.target_pool, block_table=h.block_table,
                                      page_size=16, prefix_length=sh.tokens, stream=compute)

        out[label] = round(timed(handoff), 4)
        out["delivery"] = d
    out["fused_ms"] = round(timed(h.run), 4)
    out["shape"] = sh
    return out


def delivery_bench(steps: int, warmup: int) -> dict:
    """Receiver-side delivery of the TP4 share's selected source layers in
    2048-token blocks (two slots), timed per block; and the whole block-wise
    handoff (deliver, then map, per block, on one stream and with delivery on
    a stream of its own) against the fused map from the pool, at 4096 and at
    32768 tokens."""
    import torch

    short = _delivered_handoff(4096, steps, warmup)
    d, sh = short.pop("delivery"), short.pop("shape")
    block = 2048
    # Delivery kernel alone: `steps` blocks back to back on the delivery stream.
    # A block's gather (~20 us) is shorter than the host's deliver() call, so a
    # spin kernel first keeps the GPU busy while the host enqueues them; the
    # events then bracket GPU time only.
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(d.stream):
        torch.cuda._sleep(SPIN_CYCLES)
    e0.record(d.stream)
    for i in range(steps):
        d.deliver(i % 2, 0, block)
        d.release(i % 2, d.stream)
    e1.record(d.stream)
    torch.cuda.synchronize()
    deliver_ms = e0.elapsed_time(e1) / steps
    moved = 2 * 2 * len(d.layers) * block * sh.source_heads * sh.head_dim * 2  # read + write
    long = _delivered_handoff(32768, min(10, steps), min(warmup, 2))
    long.pop("delivery"), long.pop("shape")
    gbs = moved / (deliver_ms * 1e-3) / 1e9
    return {
        "metric": "selected-layer block delivery (receiver slot fill) GB/s, TP4 share, 2048-token blocks",
        "value": round(gbs, 1), "unit": "GB/s", "n_gpus": 1, "steps": steps, "warmup": warmup,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": WORKLOADS["tp4"], "block_tokens": block, "delivered_layers": len(d.layers),
                   "source_layers": sh.source_layers},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None, "kernel": "copy_rows_kernel",
                     "bytes_per_block": moved, "kernel_ms_mean": round(deliver_ms, 5)},
        "delivered_bytes_per_handoff": 2 * len(d.layers) * sh.tokens * sh.source_heads * sh.head_dim * 2,
        "all_layer_bytes_per_handoff": 2 * sh.source_layers * sh.tokens * sh.source_heads * sh.head_dim * 2,
        "delivered_handoff_ms": short["one_stream_ms"], "fused_handoff_ms": short["fused_ms"],
        "block_handoffs": [short, long],
    }


def cohort_bench(steps: int, warmup: int) -> dict:
    """An admitted cohort (the first requests of the seeded 64-request length
    distribution, TP4 share) through the admission state machine: one
    synchronous map+install transaction per request, FIFO, against the whole
    cohort mapped in one launch and then published FIFO. Wall-clock per cohort
    (launches, synchronizations and the out-of-range check per transaction)."""
    import torch

    from cachebridge_amd import synthetic
    from cachebridge_amd.online.admission import MapperRequest, OnlineMapperAdmission
    from cachebridge_amd.online.blocks import map_install_batch, map_install_block

    out = {}
    for size in (4, 16):
        lengths = synthetic.request_lengths()[:size]
        sh = synthetic.shape("batch", tokens=sum(lengths))
        bh = synthetic.make_batch_handoff(sh, lengths)
        ps = sh.page_size
        cohort = [MapperRequest(f"req{i}", n) for i, n in enumerate(lengths)]
        span = {r.request_id: sp for r, sp in zip(cohort, bh.spans)}
        adm = OnlineMapperAdmission(max_cohort_requests=size)
        budget = sum(lengths) + 32 * size

        def transaction(r):
            sp = span[r.request_id]
            e = sp.target_offset // ps
            map_install_block(bh.mapper, bh.source_pool,
                              bh.source_slots[sp.source_offset:sp.source_offset + sp.num_tokens],
                              bh.target_pool, start=0, stop=sp.num_tokens,
                              block_table=bh.block_table[e:e + (sp.num_tokens + ps - 1) // ps], page_size=ps)
            if bh.mapper.plan.read_errors():
                raise RuntimeError("kernel flagged out-of-range rows")

        def map_cohort(rs):
            map_install_batch(bh.mapper, bh.source_pool, bh.source_slots, bh.target_pool,
                              [span[r.request_id] for r in rs], block_table=bh.block_table, page_size=ps)
            if bh.mapper.plan.read_errors():
                raise RuntimeError("kernel flagged out-of-range rows")

        def serial():
            adm.execute_cohort(adm.plan(cohort, available_target_tokens=budget),
                               mapper_transaction=transaction, query_batch=len)

        def batched():
            adm.execute_cohort_batched(adm.plan(cohort, available_target_tokens=budget),
                                       map_cohort=map_cohort, publish=lambda r: None, query_batch=len)

        times = {}
        for name, fn in (("serial", serial), ("batched", batched)):
            for _ in range(warmup):
                fn()
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for _ in range(steps):
                fn()
            times[name] = (time.perf_counter() - t0) / steps * 1e3
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        stream = torch.cuda.current_stream()
        e0.record(stream)
        for _ in range(steps):
            bh.run()
        e1.record(stream)
        torch.cuda.synchronize()
        kernel_ms = e0.elapsed_time(e1) / steps
        out[size] = dict(lengths=lengths, tokens=sum(lengths), serial_ms=times["serial"],
                         batched_ms=times["batched"], kernel_ms=kernel_ms,
                         bytes=synthetic.algorithmic_bytes(sh))
        del bh
        torch.cuda.empty_cache()
    main4 = out[4]
    gbs = main4["bytes"] / (main4["kernel_ms"] * 1e-3) / 1e9
    return {
        "metric": "admitted-cohort handoff, mapped+installed KV tokens/s (4 requests, one launch, FIFO publication)",
        "value": round(main4["tokens"] / (main4["batched_ms"] * 1e-3), 1), "unit": "tokens/s", "n_gpus": 1,
        "steps": steps, "warmup": warmup, "ms_per_step": round(main4["batched_ms"], 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": "the first 4 / 16 requests of " + WORKLOADS["batch"].split(" (")[0]
                   + " lognormal lengths, TP4 share 40x2 -> 64x2 KV heads, head_dim 128, page 16"},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "resolve_batch_kernel + map_install_stream_kernel<128, bf16, per-token positions>",
                     "algorithmic_bytes_per_launch": main4["bytes"], "kernel_ms_mean": round(main4["kernel_ms"], 5)},
        "cohorts": {str(k): {"lengths": v["lengths"], "tokens": v["tokens"],
                             "serial_cohort_ms": round(v["serial_ms"], 4),
                             "batched_cohort_ms": round(v["batched_ms"], 4),
                             "batched_kernel_ms": round(v["kernel_ms"], 4),
                             "serial_over_batched": round(v["serial_ms"] / v["batched_ms"], 2)}
                    for k, v in out.items()},
    }


def support_bench(steps: int, warmup: int, cpu: bool = True) -> dict:
    """The shipped support-8 recipe's structure (every target (layer, head)
    reads 8 source (layer, head) pairs, maps [1024, 128]) at the TP4 share and
    the whole model, 4096 tokens, one fused launch of the support kernel.
    MFMA-bound: algorithmic flops are 2 * 1024 * 128 per token, target head
    and K/V; the split-bf16 products execute 3 (keys) and 2 (values) MFMA
    passes of that."""
    import torch

    from cachebridge_amd import synthetic

    legs = {}
    for name in ("tp4_s8", "full_s8"):
        sh = synthetic.shape(name)
        h = synthetic.make_handoff(sh, device_source=True)
        wall, kernel_ms, launch_ms, launch_min = time_handoff(
            h, steps if name == "tp4_s8" else max(10, steps // 4), warmup)
        flops = synthetic.algorithmic_flops(sh)
        alg = flops / (kernel_ms * 1e-3) / 1e12
        legs[name] = dict(tokens=sh.tokens, target=f"{sh.target_layers}x{sh.target_heads}",
                          source=f"{sh.source_layers}x{sh.source_heads}", support=sh.support,
                          kernel_ms_mean=round(kernel_ms, 5), launch_ms_mean=round(launch_ms, 5),
                          launch_ms_min=round(launch_min, 5),
                          tokens_per_s=round(sh.tokens / (kernel_ms * 1e-3), 1),
                          algorithmic_flops_per_launch=flops, algorithmic_tflops=round(alg, 2),
                          algorithmic_frac=round(alg / BF16_PEAK_TFLOPS, 4),
                          executed_tflops=round(alg * 2.5, 2),
                          executed_frac=round(alg * 2.5 / BF16_PEAK_TFLOPS, 4),
                          hbm_gbs=round(synthetic.algorithmic_bytes(sh) / (kernel_ms * 1e-3) / 1e9, 1),
                          wall_ms_per_step=round(wall / steps * 1e3, 4) if name == "tp4_s8" else None)
        del h
        torch.cuda.empty_cache()
    main = legs["tp4_s8"]
    line = {
        "metric": "support-8 mapped+installed KV tokens/s (TP4 share, 4096-token handoff)",
        "value": main["tokens_per_s"], "unit": "tokens/s", "n_gpus": 1, "steps": steps, "warmup": warmup,
        "ms_per_step": main["wall_ms_per_step"], "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16", "data": "synthetic (seeded N(0,1) x per-channel lognormal "
        "bf16 KV drawn on the device; fp32 maps A~N(0,1/1024), b~N(0,0.01))",
        "config": {"workload": "support-8 maps (8 source (layer, head) pairs per target head, [1024, 128] "
                               "fp32 maps), TP4 share 40x2 -> 64x2 and whole model 40x8 -> 64x8, "
                               "head_dim 128, 4096 tokens, page 16"},
        "roofline": {"bound": "mfma", "achieved": main["algorithmic_tflops"], "peak": BF16_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": main["algorithmic_frac"], "traffic": None,
                     "kernel": "map_install_support_kernel (256-token items, 32x32 split-bf16 MFMA, "
                               "W and source rows staged by LDS DMA)",
                     "executed_frac": main["executed_frac"], "kernel_ms_mean": main["kernel_ms_mean"]},
        "legs": legs,
    }
    if cpu:
        line["cpu_baseline"] = cpu_baseline("tp4_s8", 1024, runs=3, extra=False)
        line["cpu_baseline"]["sample"] += " (1024 of the 4096 tokens)"
    return line


def staged_bench(steps: int, warmup: int, layer_chunk: int = 8) -> dict:
    """Two-stream layer-chunk pipeline (``StagedHandoff``: map chunk i+1 into a
    staging slot on one stream while chunk i is copied into the pool on
    another) against the fused map + install, TP4 share, 4096 tokens. GPU time
    per handoff from events on the caller's stream, after a spin kernel that
    hides the host's enqueue time."""
    import torch

    from cachebridge_amd import synthetic
    from cachebridge_amd.online.pipeline import StagedHandoff
    from cachebridge_amd.pool import pool_rows

    sh = synthetic.shape("tp4")
    h = synthetic.make_handoff(sh)
    n = sh.tokens
    staged = StagedHandoff(h.mapper, layer_chunk=layer_chunk, max_tokens=n)
    src = pool_rows(h.source_pool, index=h.source_slots, tokens=n)
    stream = torch.cuda.current_stream()

    def run_staged():
        staged.run(src, h.target_pool, num_tokens=n, position_start=0, block_table=h.block_table,
                   page_size=sh.page_size, prefix_length=n)

    def gpu_ms(fn) -> float:
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda._sleep(SPIN_CYCLES)
        e0.record(stream)
        for _ in range(steps):
            fn()
        e1.record(stream)
        torch.cuda.synchronize()
        if h.mapper.plan.read_errors() != 0:
            raise RuntimeError("kernel flagged out-of-range rows")
        return e0.elapsed_time(e1) / steps

    fused = gpu_ms(h.run)
    staged_ms = gpu_ms(run_staged)
    return {
        "metric": "staged two-stream handoff vs fused launch, TP4 share, 4096 tokens (ms per handoff)",
        "value": round(staged_ms, 4), "unit": "ms", "n_gpus": 1, "steps": steps, "warmup": warmup,
        "higher_is_better": False, "scaling": "weak", "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": WORKLOADS["tp4"], "layer_chunk": layer_chunk, "chunks": len(staged.chunks),
                   "staging_bytes": staged.staging_bytes},
        "roofline": None,
        "fused_ms": round(fused, 4), "staged_ms": round(staged_ms, 4),
        "staged_over_fused": round(staged_ms / fused, 3),
    }


def overlap_bench(steps: int, warmup: int, reps: int = 6) -> dict:
    """Independent handoffs back to back: ``steps`` (at most 64) requests of one plan
    (same source rows, six disjoint sets of target pages used in turn) on one
    stream, and the same requests spread round-robin over two and three
    streams with no events between them, so that one launch's last
    workgroups and the next launch's start share the CUs. Device time per
    handoff (events on the caller's stream, which waits for every stream at
    the end), median of ``reps`` interleaved repetitions."""
    import statistics

    import torch

    from cachebridge_amd import synthetic
    from cachebridge_amd.online.blocks import map_install_block

    cur = torch.cuda.current_stream()
    streams = [torch.cuda.Stream() for _ in range(3)]
    out = {}
    for name in ("tp4", "full", "gemma"):
        sh = synthetic.shape(name)
        npages = (sh.tokens + sh.page_size - 1) // sh.page_size
        h = synthetic.make_handoff(sh, target_pages=max(sh.target_pages, 6 * npages), device_source=True)
        g = torch.Generator().manual_seed(77)
        free = torch.randperm(h.target_pool.pages, generator=g)[: 6 * npages].to(h.block_table.device)
        tables = [free[i * npages:(i + 1) * npages].to(h.block_table.dtype) for i in range(6)]

        def run(ns: int) -> None:
            ss = [cur] if ns == 1 else streams[:ns]
            for i in range(steps):
                map_install_block(h.mapper, h.source_pool, h.source_slots, h.target_pool, start=0,
                                  stop=sh.tokens, block_table=tables[i % 6], page_size=sh.page_size,
                                  prefix_length=sh.tokens, stream=ss[i % ns])

        def timed(ns: int) -> float:
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            torch.cuda.synchronize()
            torch.cuda._sleep(SPIN_CYCLES)  # the host enqueues while the GPU spins
            e0.record(cur)
            for st in streams[:ns] if ns > 1 else ():
                st.wait_stream(cur)
            run(ns)
            for st in streams[:ns] if ns > 1 else ():
                cur.wait_stream(st)
            e1.record(cur)
            torch.cuda.synchronize()
            return e0.elapsed_time(e1) * 1e3 / steps

        # A plan rotates its launches over 64 work-pool counter pairs, so no
        # more than that many may be in flight at once: synchronize per mode.
        for ns in (1, 2, 3):
            for _ in range(warmup):
                run(ns)
            torch.cuda.synchronize()
        res = {1: [], 2: [], 3: []}
        for _ in range(reps):
            for ns in (1, 2, 3):
                res[ns].append(timed(ns))
        err = h.mapper.plan.read_errors()
        if err != 0:
            raise RuntimeError(f"{name}: kernel error flags {err:#x}")
        out[name] = {f"streams_{ns}_us": round(statistics.median(v), 1) for ns, v in res.items()}
        del h, tables, free
        torch.cuda.empty_cache()
    t1, t2 = out["tp4"]["streams_1_us"], out["tp4"]["streams_2_us"]
    return {
        "metric": "independent TP4-share handoffs back to back, two streams (us per handoff)",
        "value": t2, "unit": "us", "n_gpus": 1, "steps": steps, "warmup": warmup,
        "higher_is_better": False, "scaling": "weak", "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": WORKLOADS["tp4"], "requests_in_turn": 6, "repetitions": reps},
        "roofline": None,
        "one_stream_us": t1, "two_streams_over_one": round(t2 / t1, 3),
        "workloads": out,
    }


def artifacts_bench(layers: int = 64, heads: int = 8, dim: int = 128, support: int = 8) -> dict:
    """Verified mapper load at the shipped recipe's geometry (64 target layers,
    8 KV heads, head_dim 128, 8 selected source layers: 512 MiB of fp32 maps)
    written to a temporary directory: descriptor verification without and with
    the hash record, and the whole verified load into the GPU mapper."""
    import shutil
    import tempfile

    import torch
    from safetensors.torch import save_file

    from cachebridge_amd.artifacts import HashRecord, file_sha256, load_mapper, verify_descriptor
    from cachebridge_amd.mapper import PageMapper

    root = Path(tempfile.mkdtemp(prefix="cb_mapper_"))
    try:
        g = torch.Generator().manual_seed(11)
        selected = torch.tensor([round(x) for x in torch.linspace(0, 39, support).tolist()])
        names, total = {}, 0
        for i in range(layers):
            values = dict(selected=selected, headwise=torch.tensor(True),
                          k_weight=torch.randn(heads, support * dim, dim, generator=g) / dim,
                          v_weight=torch.randn(heads, support * dim, dim, generator=g) / dim,
                          k_bias=torch.randn(heads, dim, generator=g) * 0.1,
                          v_bias=torch.randn(heads, dim, generator=g) * 0.1)
            total += sum(values[k].numel() * 4 for k in ("k_weight", "v_weight", "k_bias", "v_bias"))
            p = root / f"layer_{i:03d}.safetensors"
            save_file(values, str(p))
            names[p.name] = file_sha256(p)
        desc = root / "mapper.json"
        desc.write_text(json.dumps(dict(mapper_id="bench", mapper_dir=".", target_layers=layers, source_layers=40,
                                        kv_heads=heads, head_dim=dim, logical_parameter_bytes=total,
                                        file_hashes=names)))
        kw = dict(source_rope_theta=1e6, target_rope_theta=1e6, dtype=torch.bfloat16, max_positions=8192)

        def timed(fn):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            out = fn()
            torch.cuda.synchronize()
            return (time.perf_counter() - t0) * 1e3, out

        # One untimed construction first: the process's first launches load
        # the library's code objects (about 0.2 s once).
        warm = PageMapper(root, method="cachebridge", **kw)
        torch.cuda.synchronize()
        del warm
        cold_ms, _ = timed(lambda: verify_descriptor(desc))
        record = HashRecord(root / "hashes.json")
        first_ms, _ = timed(lambda: verify_descriptor(desc, hashes=record))
        warm_ms, _ = timed(lambda: verify_descriptor(desc, hashes=HashRecord(root / "hashes.json")))
        shallow_ms, _ = timed(lambda: verify_descriptor(desc, check_tensors=False,
                                                        hashes=HashRecord(root / "hashes.json")))
        load_ms, (mapper, _) = timed(lambda: load_mapper(desc, hashes=HashRecord(root / "hashes.json"), **kw))
        del mapper
        direct_ms, m2 = timed(lambda: PageMapper(root, method="cachebridge", **kw))
        del m2
        torch.cuda.empty_cache()
    finally:
        shutil.rmtree(root, ignore_errors=True)
    return {
        "metric": "verified mapper load, 64 layers x 8 KV heads, head_dim 128, s 8 (512 MiB fp32), ms",
        "value": round(load_ms, 1), "unit": "ms", "n_gpus": 1, "steps": 1, "warmup": 0,
        "higher_is_better": False, "scaling": "strong", "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "config": {"workload": f"{layers} target layers, {heads} KV heads, head_dim {dim}, support {support}, "
                               f"{total} bytes of maps, files in a temporary directory (page cache warm)"},
        "roofline": None,
        "verify_no_record_ms": round(cold_ms, 1), "verify_first_record_ms": round(first_ms, 1),
        "verify_warm_record_ms": round(warm_ms, 1), "verify_warm_record_no_tensor_checks_ms": round(shallow_ms, 1),
        "load_mapper_warm_record_ms": round(load_ms, 1), "page_mapper_unverified_ms": round(direct_ms, 1),
    }


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run a plain MIB-MiB copy (profiler counter calibration)")
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", default="tp4", choices=sorted(WORKLOADS))
    ap.add_argument("--tokens", type=int, default=None,
                    help="history length (default: the workload's own)")
    ap.add_argument("--tokens-per-workgroup", type=int, default=0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-north-star", action="store_true")
    ap.add_argument("--delivery", action="store_true",
                    help="only time the selected-layer block delivery (receiver slots) at the TP4 share")
    ap.add_argument("--artifacts", action="store_true",
                    help="only time a verified mapper load (descriptor checks, hash record, GPU mapper)")
    ap.add_argument("--cohort", action="store_true",
                    help="only time an admitted cohort: per-request transactions vs one batched launch")
    ap.add_argument("--delta-state", action="store_true",
                    help="only time the recurrent-state transform (Qwen3.5-style hybrid model)")
    ap.add_argument("--support", type=int, default=1, choices=(1, 8),
                    help="8: only time the support-8 maps at the TP4 share and the whole model")
    ap.add_argument("--overlap", action="store_true",
                    help="only time independent handoffs back to back on one, two and three streams")
    ap.add_argument("--staged", action="store_true",
                    help="only time the two-stream staged handoff against the fused launch")
    ap.add_argument("--layer-chunk", type=int, default=8, help="target layers per staged chunk")
    args = ap.parse_args()
    if args.copy_calibration:
        copy_calibration(args.copy_calibration)
        return 0
    if args.delta_state:
        print(json.dumps(delta_state_bench(args.steps, args.warmup)), flush=True)
        return 0
    if args.support == 8:
        print(json.dumps(support_bench(args.steps, args.warmup, cpu=not args.no_cpu_baseline)), flush=True)
        return 0
    if args.staged:
        print(json.dumps(staged_bench(args.steps, args.warmup, args.layer_chunk)), flush=True)
        return 0
    if args.delivery:
        print(json.dumps(delivery_bench(args.steps, args.warmup)), flush=True)
        return 0
    if args.overlap:
        print(json.dumps(overlap_bench(min(args.steps, 20), min(args.warmup, 3))), flush=True)
        return 0
    if args.cohort:
        print(json.dumps(cohort_bench(args.steps, args.warmup)), flush=True)
        return 0
    if args.artifacts:
        print(json.dumps(artifacts_bench()), flush=True)
        return 0
    if args.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {args.gpus} is not supported (the handoff "
              "path runs on one GPU's share; multi-GPU sharding is not part of this build)",
              file=sys.stderr)
        return 2

    import torch

    from cachebridge_amd import synthetic

    torch.cuda.set_device(0)
    sh = synthetic.shape(args.workload, tokens=args.tokens)
    if args.workload.startswith("batch"):
        h = synthetic.make_batch_handoff(sh)
    else:
        h = synthetic.make_handoff(sh)
    wall, kernel_ms, launch_ms, launch_min = time_handoff(h, args.steps, args.warmup,
                                                          args.tokens_per_workgroup)
    tokens = sh.tokens
    value = args.steps * tokens / wall
    bytes_alg = synthetic.algorithmic_bytes(sh)
    flops = synthetic.algorithmic_flops(sh)
    achieved = bytes_alg / (kernel_ms * 1e-3) / 1e9
    traffic, traffic_source = profiled_traffic("map_install_stream", args.workload)
    line = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall / args.steps * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) x per-channel lognormal(0,0.5) bf16 KV; fp32 maps "
                "A~N(0,1/128), b~N(0,0.01))",
        "config": {"workload": WORKLOADS[args.workload], "tokens": tokens,
                   "target_layers": sh.target_layers, "target_kv_heads": sh.target_heads,
                   "source_layers": sh.source_layers, "source_kv_heads": sh.source_heads,
                   "head_dim": sh.head_dim, "page_size": sh.page_size},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": traffic, "traffic_source": traffic_source,
                     "kernel": ("resolve_batch_kernel + map_install_stream_kernel<128, bf16, "
                                "per-token positions>" if args.workload.startswith("batch")
                                else "map_install_stream_kernel<128, bf16>"),
                     "algorithmic_bytes_per_launch": bytes_alg,
                     "kernel_ms_mean": round(kernel_ms, 5)},
        "mfma": {"algorithmic_tflops": round(flops / (kernel_ms * 1e-3) / 1e12, 2),
                 "executed_tflops": round(flops * 2.5 / (kernel_ms * 1e-3) / 1e12, 2),
                 "peak_tflops": BF16_PEAK_TFLOPS,
                 "executed_frac": round(flops * 2.5 / (kernel_ms * 1e-3) / 1e12 / BF16_PEAK_TFLOPS, 4)},
        # One handoff on its own: a launch between its own events, mean and
        # best of an untimed pass after the timed region.
        "handoff_latency_ms": round(launch_ms, 4),
        "handoff_latency_min_ms": round(launch_min, 4),
    }
    if not args.workload.startswith("batch"):
        line["publish_ready_ms"] = publish_ready_latency(h)
        if not args.no_cpu_baseline:
            line["parity"] = sampled_parity(h, sh, args.workload)
    del h
    torch.cuda.empty_cache()
    if not args.no_north_star and args.workload == "tp4":
        ns = synthetic.shape("full", tokens=4096)
        hn = synthetic.make_handoff(ns)
        steps_n = max(20, args.steps // 4)
        wall_n, kms_n, lat_n, lat_min_n = time_handoff(hn, steps_n, args.warmup)
        b = synthetic.algorithmic_bytes(ns)
        traffic_n, traffic_src_n = profiled_traffic("map_install_stream", "full")
        gbs_n = b / (kms_n * 1e-3) / 1e9
        line["north_star_64x8"] = {
            "workload": WORKLOADS["full"], "steps": steps_n, "kernel_ms_mean": round(kms_n, 4),
            "handoff_latency_ms": round(lat_n, 4), "handoff_latency_min_ms": round(lat_min_n, 4),
            "tokens_per_s": round(ns.tokens / (kms_n * 1e-3), 1),
            "wall_tokens_per_s": round(steps_n * ns.tokens / wall_n, 1),
            "roofline": {"bound": "hbm", "achieved": round(gbs_n, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(gbs_n / HBM_PEAK_GBS, 4), "traffic": traffic_n,
                         "traffic_source": traffic_src_n, "kernel": "map_install_stream_kernel<128, bf16>",
                         "algorithmic_bytes_per_launch": b, "kernel_ms_mean": round(kms_n, 5)},
            "hbm_frac": round(gbs_n / HBM_PEAK_GBS, 4),
            "algorithmic_bytes_per_launch": b,
            "traffic": traffic_n,
        }
        if not args.no_cpu_baseline:
            line["north_star_64x8"]["parity"] = sampled_parity(hn, ns, "full")
        del hn
        torch.cuda.empty_cache()
        if not args.no_cpu_baseline:
            line["north_star_64x8"]["cpu_baseline"] = cpu_baseline("full", 4096, runs=3, extra=False)
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(args.workload, tokens)
        line["gpu_over_cpu"] = round(value / line["cpu_baseline"]["value"], 1)
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
