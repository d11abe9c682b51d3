#!/usr/bin/env python3
"""MiniMax-M3 three-stage sparse attention on one MI355X.

Headline (BASELINE.json metric): sparse-attention forward+backward effective
TFLOP/s at 32K tokens (config c4: T=32768, Hq=32, G=4, D=Di=128, block 128,
top-16, one local block), plus per-stage milliseconds. A "step" is one
m3_sparse_attention forward + backward (dQ, dK, dV) through the public API on
indices produced by m3_index_score -> m3_topk, with all inputs resident in HBM.

Prints one JSON line on stdout; diagnostics go to stderr.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config c4] [--no-cpu-baseline]
"""

from __future__ import annotations

import argparse
import ctypes
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

MFMA_BF16_PEAK_TFLOPS = 2516.6  # 256 CU x 2.4 GHz x 4096 FLOP/clk (dense bf16)
HBM_PEAK_GBPS = 8000.0

# BASELINE.json configs (c1 is the reference's CPU-runnable case).
CONFIGS = {
    "c1": dict(lengths=[512, 768], hq=8, g=2, d=64, di=64, block=128, topk=4, local=1, jitter=False),
    "c2": dict(lengths=[8192], hq=32, g=4, d=128, di=128, block=128, topk=16, local=1, jitter=False),
    "c3": dict(lengths=[2048, 3072, 5120, 6144], hq=32, g=4, d=128, di=128, block=128, topk=16, local=1,
               jitter=False),
    "c4": dict(lengths=[32768], hq=32, g=4, d=128, di=128, block=128, topk=16, local=1, jitter=True),
    "c5": dict(lengths=[65536], hq=64, g=8, d=128, di=128, block=128, topk=32, local=2, jitter=False),
}


def log(*args):
    print(*args, file=sys.stderr, flush=True)


def make_inputs(cfg, seed=71):
    """Synthetic bf16 inputs in the reference benchmark's draw order (benchmark.py:68-75):
    index_q, index_k, q, k, v, then grad_out; c4 scales index_q per group by U(0.5, 2)
    drawn right after index_q, before rounding to bf16."""
    import torch

    gen = torch.Generator().manual_seed(seed)
    total = sum(cfg["lengths"])
    iq = torch.randn(total, cfg["g"], cfg["di"], generator=gen)
    if cfg["jitter"]:
        iq = iq * (0.5 + 1.5 * torch.rand(cfg["g"], generator=gen))[None, :, None]
    iq = iq.bfloat16()
    ik = torch.randn(total, 1, cfg["di"], generator=gen).bfloat16()
    q = torch.randn(total, cfg["hq"], cfg["d"], generator=gen).bfloat16()
    k = torch.randn(total, cfg["g"], cfg["d"], generator=gen).bfloat16()
    v = torch.randn(total, cfg["g"], cfg["d"], generator=gen).bfloat16()
    dout = torch.randn(total, cfg["hq"], cfg["d"], generator=gen).bfloat16()
    return iq, ik, q, k, v, dout


def visible_keys(cfg):
    """sum over (t, g) of the causally visible keys of the selected blocks, closed form:
    (pos % B + 1) + (min(K, qb + 1) - 1) * B (top-k output: distinct blocks, current block forced)."""
    b, k = cfg["block"], cfg["topk"]
    total = 0
    for n in cfg["lengths"]:
        for pos in range(n):
            qb = pos // b
            total += (pos % b + 1) + (min(k, qb + 1) - 1) * b
    return total * cfg["g"]


def stage_work(cfg):
    """Algorithmic work of the non-attention stages (closed forms of the measurement spec):
    score fwd FLOP, top-k / CSR / score-bwd bytes."""
    b, k, g, di = cfg["block"], cfg["topk"], cfg["g"], cfg["di"]
    T = sum(cfg["lengths"])
    pairs = sum(n * (n + 1) // 2 for n in cfg["lengths"])
    score_flops = 2.0 * di * g * pairs
    causal_blocks = sum(sum(p // b + 1 for p in range(n)) for n in cfg["lengths"])  # valid (t, b) per group
    topk_bytes = causal_blocks * g * 4 + T * g * k * 4
    rows = sum((n + b - 1) // b for n in cfg["lengths"]) * g
    csr_bytes = T * g * k * 4 + (rows + 1) * 4 + 2 * T * g * k * 4 + (len(cfg["lengths"]) + 1) * 4
    # score backward, unavoidable HBM bytes: ds and the tie code of every valid (t, g, b) read,
    # index_q / index_k read once, dq / dk written (the per-entry winner-row gathers, 512 B per
    # valid entry at Di = 128, come from the caches: both inputs total 40 MiB at c4)
    score_bwd_bytes = causal_blocks * g * (4 + 4) + 2 * (T * g * di * 2 + T * di * 2)
    return score_flops, topk_bytes, csr_bytes, score_bwd_bytes


def measured_traffic(config, name, table="kernels"):
    """HBM bytes per call of one kernel (table "kernels": summed over its launches in one
    entry-point call) or one entry point (table "entries") from the committed rocprofv3
    PMC summary (FETCH_SIZE and WRITE_SIZE, calibrated against a copy of known size), if
    present."""
    path = os.path.join(ROOT, "profiles", f"attn_{config}_traffic.json")
    try:
        with open(path) as f:
            data = json.load(f)
        return data[table][name]["bytes_per_call"]
    except (OSError, KeyError, ValueError):
        return None


def cpu_info():
    """Host CPU description for the CPU baseline: logical CPUs, the CPUs this process may
    run on, the model name and torch's intra-op threads."""
    import torch

    model = None
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"nproc": os.cpu_count(), "affinity_cpus": len(os.sched_getaffinity(0)), "cpu_model": model,
            "torch_threads": torch.get_num_threads()}


def _pmc_rows(directory, counter, unit=1024.0):
    """(dispatch id, kernel name, value x unit) of one rocprofv3 counter pass, in dispatch order.
    FETCH_SIZE / WRITE_SIZE are reported in KiB per dispatch (unit 1024: bytes)."""
    import csv
    import glob

    rows = []
    for path in glob.glob(os.path.join(directory, "**", "*counter_collection.csv"), recursive=True):
        with open(path) as f:
            for r in csv.DictReader(f):
                if r["Counter_Name"] == counter:
                    rows.append((int(r["Dispatch_Id"]), r["Kernel_Name"], float(r["Counter_Value"]) * unit))
    rows.sort()
    return rows


def summarize_pmc(config, fetch_dir, write_dir):
    """Per-entry HBM bytes of one msa_attn_fwd and one msa_attn_bwd call from two --pmc-pass runs.
    The calibration copy (the largest copy dispatch) moves COPY bytes each way; each counter is scaled
    so that it reads exactly that. The forward call's dispatches run from its first kv_chunk_bounds up
    to the first backward kernel (kv_bwd_*), the backward call's from there to the end."""
    copy_bytes = 64 << 22  # 256 MiB
    out = {"config": config, "counters": ["FETCH_SIZE", "WRITE_SIZE"],
           "command": [f"rocprofv3 --pmc FETCH_SIZE -d <out> -o f --output-format csv -- python bench.py --config "
                       f"{config} --pmc-pass",
                       f"rocprofv3 --pmc WRITE_SIZE -d <out> -o w --output-format csv -- python bench.py --config "
                       f"{config} --pmc-pass"],
           "calibration": {"copy_bytes": copy_bytes}, "entries": {}}
    per_kernel = {}
    for counter, directory, key in (("FETCH_SIZE", fetch_dir, "read"), ("WRITE_SIZE", write_dir, "write")):
        rows = _pmc_rows(directory, counter)
        calib = max(r[2] for r in rows if "copy" in r[1].lower())
        scale = copy_bytes / calib
        out["calibration"][f"{key}_reported_bytes"] = calib
        out["calibration"][f"{key}_scale"] = round(scale, 4)
        first_bwd = next(i for i, r in enumerate(rows) if "kv_bwd_" in r[1])
        last_bwd = max(i for i, r in enumerate(rows) if "kv_bwd_" in r[1])
        first_fwd = max(i for i, r in enumerate(rows[:first_bwd]) if "kv_chunk_bounds" in r[1])
        for i, (_, name, value) in enumerate(rows):
            if "copy" in name.lower():
                continue
            entry = ("msa_attn_fwd" if first_fwd <= i < first_bwd else
                     "msa_attn_bwd" if first_bwd <= i <= last_bwd else "stages")
            short = name.split("(")[0].replace("void ", "").replace("msa::", "")
            d = per_kernel.setdefault((entry, short), {"dispatches": 0, "read": 0.0, "write": 0.0})
            if key == "read":
                d["dispatches"] += 1
            d[key] += value * scale
            if entry != "stages":
                e = out["entries"].setdefault(entry, {"read_bytes": 0.0, "write_bytes": 0.0})
                e[f"{key}_bytes"] += value * scale
    for e in out["entries"].values():
        e["read_bytes"] = int(e["read_bytes"])
        e["write_bytes"] = int(e["write_bytes"])
        e["bytes_per_call"] = e["read_bytes"] + e["write_bytes"]
    out["kernels"] = {}
    for (entry, name), d in per_kernel.items():
        base = name.split("<")[0]
        if entry == "stages" and base.startswith("kv_"):  # the indexer KL's work plans
            base = "kl_" + base
        k = out["kernels"].setdefault(base, {"entry": entry, "dispatches": 0, "read_bytes": 0, "write_bytes": 0})
        k["dispatches"] += d["dispatches"]
        k["read_bytes"] += int(d["read"])
        k["write_bytes"] += int(d["write"])
    for k in out["kernels"].values():
        k["bytes_per_call"] = k["read_bytes"] + k["write_bytes"]
    path = os.path.join(ROOT, "profiles", f"attn_{config}_traffic.json")
    with open(path, "w") as f:
        json.dump(out, f, indent=1)
    gib = float(1 << 30)
    print("| entry | kernel | dispatches | read GiB | write GiB |")
    print("|---|---|---:|---:|---:|")
    for (entry, name), d in per_kernel.items():
        print(f"| {entry} | `{name}` | {d['dispatches']} | {d['read'] / gib:.3f} | {d['write'] / gib:.3f} |")
    print()
    print("| entry | read GiB / call | write GiB / call | total GB / call | at 8 TB/s |")
    print("|---|---:|---:|---:|---:|")
    for entry, e in out["entries"].items():
        tot = e["bytes_per_call"]
        print(f"| {entry} | {e['read_bytes'] / gib:.2f} | {e['write_bytes'] / gib:.2f} | {tot / 1e9:.2f} | "
              f"{tot / 8e12 * 1e3:.2f} ms |")
    print(f"wrote {path}", file=sys.stderr)


SQ_COUNTERS = ("SQ_INSTS_VALU", "SQ_INSTS_MFMA", "SQ_INSTS_VALU_MFMA_MOPS_BF16", "SQ_VALU_MFMA_BUSY_CYCLES",
               "SQ_BUSY_CYCLES", "SQ_INSTS_LDS", "SQ_LDS_BANK_CONFLICT", "SQ_WAVES")
SHADER_ENGINES = 32    # MI355X: 8 XCDs x 4 shader engines; SQ_BUSY_CYCLES is summed over them
SIMDS = 1024           # 256 CUs x 4 SIMDs; SQ_VALU_MFMA_BUSY_CYCLES is summed over them


def summarize_sq(config, directory, stats_csv=None):
    """Per-kernel instruction and MFMA counters of one --pmc-pass run (one call of every
    stage) as a markdown table: VALU, MFMA and LDS instructions; bf16 MFMA FLOPs
    (SQ_INSTS_VALU_MFMA_MOPS_BF16 x 512); MFMA busy = SQ_VALU_MFMA_BUSY_CYCLES / (SIMDS x
    SQ_BUSY_CYCLES / SHADER_ENGINES), the share of the kernel's cycles the SIMDs' matrix
    cores were busy; LDS bank-conflict cycles per LDS instruction; LDS bytes per workgroup
    and scratch bytes per lane of the dispatch. With a rocprofv3 kernel-stats CSV, also the
    counted bf16 FLOPs over the traced average duration against the 2.4 GHz peak."""
    import csv
    import glob

    per, res, dispatches = {}, {}, {}
    for path in glob.glob(os.path.join(directory, "**", "*counter_collection.csv"), recursive=True):
        with open(path) as f:
            for r in csv.DictReader(f):
                if r["Counter_Name"] not in SQ_COUNTERS:
                    continue
                short = r["Kernel_Name"].split("(")[0].replace("void ", "").replace("msa::", "")
                d = per.setdefault(short, {})
                d[r["Counter_Name"]] = d.get(r["Counter_Name"], 0.0) + float(r["Counter_Value"])
                res[short] = (r.get("LDS_Block_Size"), r.get("Scratch_Size"))
                dispatches.setdefault(short, set()).add(r["Dispatch_Id"])
    durations = {}
    if stats_csv:
        with open(stats_csv) as f:
            for r in csv.DictReader(f):
                short = r["Name"].split("(")[0].replace("void ", "").replace("msa::", "")
                durations[short] = float(r["AverageNs"]) * 1e-9
    print(f"Counters of one --pmc-pass run (config {config}; sums over a kernel's dispatches in one call).")
    print()
    print("| kernel | dispatches | VALU insts | MFMA insts | VALU:MFMA | bf16 MFMA TFLOP | MFMA busy | "
          "MFMA FLOP rate / peak | LDS insts | LDS conflict cycles / inst | LDS B | scratch B |")
    print("|---|---:|---:|---:|---:|---:|---:|---:|---:|---:|---:|---:|")
    for name, d in per.items():
        valu, mfma = d.get("SQ_INSTS_VALU", 0.0), d.get("SQ_INSTS_MFMA", 0.0)
        if valu == 0 and mfma == 0 or name.startswith("at::") or name.startswith("__amd"):
            continue
        flops = d.get("SQ_INSTS_VALU_MFMA_MOPS_BF16", 0.0) * 512
        busy = d.get("SQ_BUSY_CYCLES", 0.0) / SHADER_ENGINES
        mbusy = d.get("SQ_VALU_MFMA_BUSY_CYCLES", 0.0)
        lds = d.get("SQ_INSTS_LDS", 0.0)
        conf = d.get("SQ_LDS_BANK_CONFLICT", 0.0)
        ratio = f"{valu / mfma:.1f}" if mfma else "-"
        disp = len(dispatches[name])
        rate = "-"
        if flops and name in durations:
            rate = f"{flops / (durations[name] * disp) / (MFMA_BF16_PEAK_TFLOPS * 1e12):.1%}"
        ldsb, scr = res.get(name, (None, None))
        print(f"| `{name}` | {disp} | {valu:.3g} | {mfma:.3g} | {ratio} | {flops / 1e12:.3f} | "
              f"{(mbusy / (SIMDS * busy) if busy and mfma else 0):.1%} | {rate} | {lds:.3g} | "
              f"{(conf / lds if lds else 0):.2f} | {ldsb} | {scr} |")


def summarize_trace(stats_csv):
    """Per-kernel rows of a rocprofv3 --kernel-trace --stats run (its kernel_stats.csv) as a
    markdown table, heaviest total first: calls, average / min / max duration and total."""
    import csv

    with open(stats_csv) as f:
        rows = list(csv.DictReader(f))
    rows.sort(key=lambda r: -float(r["TotalDurationNs"]))
    print("| kernel | calls | avg ms | min ms | max ms | total ms | share |")
    print("|---|---:|---:|---:|---:|---:|---:|")
    for r in rows:
        short = r["Name"].split("(")[0].replace("void ", "").replace("msa::", "")
        print(f"| `{short}` | {r['Calls']} | {float(r['AverageNs']) * 1e-6:.4f} | {float(r['MinNs']) * 1e-6:.4f} | "
              f"{float(r['MaxNs']) * 1e-6:.4f} | {float(r['TotalDurationNs']) * 1e-6:.3f} | "
              f"{float(r['Percentage']):.2f} % |")


class Harness:
    """Direct C-ABI launches on preallocated buffers, for per-kernel timing."""

    def __init__(self, cfg, tensors, ids, cu, device):
        import torch

        from msa_triton_amd import _lib
        from msa_triton_amd.k2q import build_k2q_csr
        from msa_triton_amd.layout import sequence_meta

        self.torch = torch
        self.lib = _lib.lib()
        self.cfg = cfg
        iq, ik, q, k, v, dout = tensors
        self.q, self.k, self.v, self.dout = q, k, v, dout
        self.dtype_code = _lib.DTYPE_CODE[q.dtype]
        self.ids, self.cu = ids, cu
        bounds = [0]
        for n in cfg["lengths"]:
            bounds.append(bounds[-1] + n)
        self.meta = sequence_meta(bounds, cfg["block"])
        self.T = bounds[-1]
        self.scale = cfg["d"] ** -0.5
        self.out = torch.empty_like(q)
        self.lse = torch.empty(q.shape[:2], dtype=torch.float32, device=device)
        self.rs = torch.empty((*q.shape[:2], 4), dtype=torch.float64, device=device)
        # the forward's fp32 output, which lets the backward skip its statistics pass
        self.o32 = torch.empty(q.shape, dtype=torch.float32, device=device)
        self.use_f32 = True
        self.dq = torch.empty_like(q)
        self.dk = torch.empty_like(k)
        self.dv = torch.empty_like(v)
        self.csr = build_k2q_csr(ids, cu, block_size=cfg["block"])
        self.fws_bytes = self.lib.msa_attn_fwd_workspace_bytes(self.dtype_code, self.T, cfg["hq"], cfg["g"], cfg["d"],
                                                               cfg["topk"], self.meta.total_blocks, cfg["block"])
        self.fws = torch.empty(max(1, self.fws_bytes), dtype=torch.uint8, device=device)
        self.ws_bytes = self.lib.msa_attn_bwd_workspace_bytes(self.dtype_code, self.T, cfg["hq"], cfg["g"], cfg["d"],
                                                              cfg["topk"], self.meta.total_blocks, cfg["block"])
        self.ws = torch.empty(max(1, self.ws_bytes), dtype=torch.uint8, device=device)
        self.stream = torch.cuda.current_stream(device).cuda_stream

    def fwd(self):
        c = self.cfg
        csr = self.csr
        st = self.lib.msa_attn_fwd(self.q.data_ptr(), self.k.data_ptr(), self.v.data_ptr(), self.dtype_code,
                                   self.ids.data_ptr(), self.cu.data_ptr(), self.meta.num_seqs, self.T, c["hq"], c["g"], c["d"], c["topk"],
                                   c["block"], self.scale, csr.cu_block_lens.data_ptr(), self.meta.total_blocks,
                                   csr.row_ptr.data_ptr(), csr.query_indices.data_ptr(), csr.slot_indices.data_ptr(),
                                   self.fws.data_ptr(), self.fws_bytes, self.out.data_ptr(), self.lse.data_ptr(),
                                   self.rs.data_ptr(), self.o32.data_ptr(), self.stream)
        assert st == 0

    def bwd(self):
        c = self.cfg
        csr = self.csr
        st = self.lib.msa_attn_bwd(self.q.data_ptr(), self.k.data_ptr(), self.v.data_ptr(), self.dtype_code,
                                   self.out.data_ptr(), self.dout.data_ptr(), self.rs.data_ptr(),
                                   self.o32.data_ptr() if self.use_f32 else None, self.ids.data_ptr(), self.cu.data_ptr(),
                                   self.meta.num_seqs, self.T, c["hq"], c["g"], c["d"], c["topk"], c["block"],
                                   self.scale, csr.cu_block_lens.data_ptr(), self.meta.total_blocks,
                                   csr.row_ptr.data_ptr(), csr.query_indices.data_ptr(), csr.slot_indices.data_ptr(),
                                   self.dq.data_ptr(), self.dk.data_ptr(), self.dv.data_ptr(), self.ws.data_ptr(),
                                   self.ws_bytes, self.stream)
        assert st == 0


def time_loop(fn, steps, warmup=2):
    """Milliseconds per call over `steps` back-to-back calls (one event pair, no
    synchronisation in between), like the headline step timing."""
    import torch

    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        fn()
    stop.record()
    torch.cuda.synchronize()
    return start.elapsed_time(stop) / steps


def time_events(fn, repeats, warmup=1):
    """Median / min / p90 milliseconds per call, HIP events on the current stream."""
    import torch

    for _ in range(warmup):
        fn()
    samples = []
    for _ in range(repeats):
        start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        fn()
        stop.record()
        stop.synchronize()
        samples.append(start.elapsed_time(stop))
    samples.sort()
    return {"median": statistics.median(samples), "min": samples[0],
            "p90": samples[min(len(samples) - 1, int(0.9 * len(samples)))]}


def peak_bytes(fn):
    """Device memory one call of fn allocates at its peak above what was allocated before
    it (torch caching-allocator statistics, reset before the call)."""
    import torch

    torch.cuda.synchronize()
    base = torch.cuda.memory_allocated()
    torch.cuda.reset_peak_memory_stats()
    fn()
    torch.cuda.synchronize()
    return torch.cuda.max_memory_allocated() - base


def cpu_baseline(cfg, tensors, ids_cpu, budget_s):
    """Eager CPU restatement (oracle/eager_baseline.py) on the last query rows of the
    first sequence, row-chunked, until ~budget_s seconds of CPU work; returns the
    effective fwd+bwd TFLOP/s of the sample. Also times the eager score (fp32 Q.K^T over
    the dense key range + block amax) on the last query rows for ~budget_s / 3 seconds
    and the eager top-k selection on every row of the first sequence."""
    import torch

    from oracle.eager_baseline import eager_rows_fwd_bwd, eager_score_rows, eager_topk

    iq, ik, q, k, v, dout = tensors
    n0 = cfg["lengths"][0]
    b, kk, hq, d, g = cfg["block"], cfg["topk"], cfg["hq"], cfg["d"], cfg["g"]
    chunk = 64
    flops = 0.0
    rows_done = 0
    t0 = time.perf_counter()
    r1 = n0
    while r1 > 0:
        r0 = max(0, r1 - chunk)
        eager_rows_fwd_bwd(q[:n0], k[:n0], v[:n0], ids_cpu[:n0], (r0, r1), block_size=b, scale=d ** -0.5,
                           dout=dout[:n0])
        for pos in range(r0, r1):
            qb = pos // b
            keys = (pos % b + 1) + (min(kk, qb + 1) - 1) * b
            flops += 3.5 * 4 * d * hq * keys
        rows_done += r1 - r0
        r1 = r0
        if time.perf_counter() - t0 > budget_s:
            break
    elapsed = time.perf_counter() - t0

    # eager score on the last query rows (causal pairs counted, like the GPU stage figure)
    score_flops, score_rows = 0.0, 0
    ts = time.perf_counter()
    r1 = n0
    with torch.no_grad():
        while r1 > 0:
            r0 = max(0, r1 - 256)
            eager_score_rows(iq[:n0], ik[:n0], (r0, r1), block_size=b)
            score_flops += 2.0 * cfg["di"] * g * sum(p + 1 for p in range(r0, r1))
            score_rows += r1 - r0
            r1 = r0
            if time.perf_counter() - ts > budget_s / 3:
                break
    score_s = time.perf_counter() - ts

    # eager top-k over every row of the first sequence
    nb = (max(cfg["lengths"]) + b - 1) // b
    gen = torch.Generator().manual_seed(5)
    scores = torch.randn(n0, g, nb, generator=gen)
    positions = torch.arange(n0)
    tt = time.perf_counter()
    eager_topk(scores, positions, block_size=b, topk_blocks=kk, local_blocks=cfg["local"])
    topk_s = time.perf_counter() - tt
    topk_bytes = sum(p // b + 1 for p in range(n0)) * g * 4 + n0 * g * kk * 4

    info = cpu_info()
    return {
        "value": flops / elapsed / 1e12,
        "unit": "TFLOP/s",
        "cores": info["torch_threads"],
        "kind": "port",
        "sample": (f"eager bf16 restatement (eager/ops.py:153-180 math, dense masked rows, torch CPU autograd) "
                   f"fwd+bwd of the last {rows_done} query rows of the {n0}-token sequence in {chunk}-row chunks, "
                   f"{elapsed:.1f} s; effective FLOPs counted like the GPU value"),
        "host": info,
        "stages": {
            "score_fwd": {"value": round(score_flops / score_s / 1e12, 6), "unit": "TFLOP/s",
                          "sample": f"eager fp32 score (eager/ops.py:45-67) of the last {score_rows} query rows over "
                                    f"the dense {n0}-key range, {score_s:.1f} s; causal pairs counted",
                          "full_config_ms_extrapolated": round(score_s * 1e3 * (2.0 * cfg['di'] * g * sum(
                              n * (n + 1) // 2 for n in cfg["lengths"])) / max(score_flops, 1.0), 1)},
            "topk": {"value": round(topk_bytes / topk_s / 1e9, 3), "unit": "GB/s", "ms": round(topk_s * 1e3, 2),
                     "sample": f"eager masked_fill + torch.topk (eager/ops.py:112-129) over all {n0} rows x {g} "
                               f"groups x {nb} blocks of random fp32 scores; causal bytes counted"},
        },
    }


def main():
    parser = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=10)
    parser.add_argument("--warmup", type=int, default=3)
    parser.add_argument("--config", default="c4", choices=sorted(CONFIGS))
    parser.add_argument("--repeats", type=int, default=10, help="repeats for per-stage timings")
    parser.add_argument("--no-cpu-baseline", action="store_true")
    parser.add_argument("--cpu-seconds", type=float, default=15.0)
    parser.add_argument("--no-stages", action="store_true")
    parser.add_argument("--pmc-pass", action="store_true",
                        help="for rocprofv3 --pmc: a 256 MiB calibration copy, one attention forward and one "
                             "backward call (direct C ABI), then one call of each other stage (score forward with "
                             "its backward state, score backward, top-k, k2q CSR, indexer KL) and exit")
    parser.add_argument("--pmc-summarize", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"),
                        help="read the counter CSVs of two --pmc-pass runs (FETCH_SIZE, WRITE_SIZE), write "
                             "profiles/attn_<config>_traffic.json and print a markdown table; no GPU needed")
    parser.add_argument("--sq-summarize", metavar="SQ_DIR",
                        help="read the counter CSVs of a --pmc-pass run with the SQ_COUNTERS and print a "
                             "per-kernel markdown table; no GPU needed")
    parser.add_argument("--trace-summarize", metavar="STATS_CSV",
                        help="print the per-kernel table of a rocprofv3 --kernel-trace --stats run "
                             "(its kernel_stats.csv); no GPU needed")
    args = parser.parse_args()
    if args.pmc_summarize:
        summarize_pmc(args.config, *args.pmc_summarize)
        return
    if args.sq_summarize:
        summarize_sq(args.config, args.sq_summarize)
        return
    if args.trace_summarize:
        summarize_trace(args.trace_summarize)
        return
    if args.gpus != 1:
        print(f"bench.py measures one MI355X: --gpus {args.gpus} is not supported (this path runs on one GPU "
              "and does not shard across GPUs).", file=sys.stderr)
        sys.exit(2)

    import torch

    import msa_triton_amd as msa
    from msa_triton_amd import _lib
    from msa_triton_amd.k2q import build_k2q_csr

    device = torch.device("cuda:0")
    torch.cuda.set_device(device)
    cfg = CONFIGS[args.config]
    log(f"config {args.config}: {cfg}")
    tensors_cpu = make_inputs(cfg)
    iq, ik, q, k, v, dout = (x.to(device) for x in tensors_cpu)
    total = sum(cfg["lengths"])
    cu_list = [0]
    for n in cfg["lengths"]:
        cu_list.append(cu_list[-1] + n)
    cu = torch.tensor(cu_list, dtype=torch.int32, device=device)
    max_len = max(cfg["lengths"])
    block, topk, local = cfg["block"], cfg["topk"], cfg["local"]

    with torch.no_grad():
        scores = msa.m3_index_score(iq, ik, cu, max_len, block_size=block)
        ids = msa.m3_topk(scores, cu, block_size=block, topk_blocks=topk, local_blocks=local)
    torch.cuda.synchronize()
    keys = visible_keys(cfg)
    # check the closed form against the actual selection (distinct, in-range blocks)
    valid = (ids >= 0)
    assert int(valid.sum()) == sum(min(topk, p // block + 1) for n in cfg["lengths"] for p in range(n)) * cfg["g"]
    fwd_flops = 4.0 * cfg["d"] * (cfg["hq"] // cfg["g"]) * keys
    step_flops = 3.5 * fwd_flops

    if args.pmc_pass:
        src = torch.ones(64 << 20, dtype=torch.float32, device=device)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)  # 256 MiB read + 256 MiB written: calibrates FETCH_SIZE / WRITE_SIZE
        torch.cuda.synchronize()
        h = Harness(cfg, (iq, ik, q, k, v, dout), ids, cu, device)
        torch.cuda.synchronize()
        h.fwd()
        torch.cuda.synchronize()
        h.bwd()
        torch.cuda.synchronize()
        iqg, ikg = iq.detach().clone().requires_grad_(), ik.detach().clone().requires_grad_()
        s = msa.m3_index_score(iqg, ikg, cu, max_len, block_size=block)
        torch.cuda.synchronize()
        s.backward(torch.ones_like(s))
        torch.cuda.synchronize()
        msa.m3_topk(s.detach(), cu, block_size=block, topk_blocks=topk, local_blocks=local)
        torch.cuda.synchronize()
        build_k2q_csr(ids, cu, block_size=block)
        torch.cuda.synchronize()
        iqk, ikk = iq.detach().clone().requires_grad_(), ik.detach().clone().requires_grad_()
        msa.m3_indexer_kl(iqk, ikk, q, k, ids, cu, max_len, block_size=block).backward()
        torch.cuda.synchronize()
        log("pmc pass done")
        return

    qg, kg, vg = (x.detach().clone().requires_grad_() for x in (q, k, v))

    def step():
        qg.grad = kg.grad = vg.grad = None
        out = msa.m3_sparse_attention(qg, kg, vg, ids, cu, max_len, block_size=block)
        out.backward(dout)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    ev0.record()
    for _ in range(args.steps):
        step()
    ev1.record()
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3 / args.steps
    ms = ev0.elapsed_time(ev1) / args.steps
    log(f"attention fwd+bwd: {ms:.3f} ms/step (events), {wall_ms:.3f} ms/step (wall)")
    # the same step timed one at a time: median / min / p90
    step_stats = time_events(step, args.steps, warmup=0)
    log(f"per-step: median {step_stats['median']:.3f} min {step_stats['min']:.3f} p90 {step_stats['p90']:.3f} ms")

    # ---- per-kernel timings: direct C-ABI launches, each kernel bracketed by HIP events on
    # its launch stream (the library's profiling hook), summed per kernel kind per call
    h = Harness(cfg, (iq, ik, q, k, v, dout), ids, cu, device)
    h.fwd()
    kt = {"attn_fwd": time_events(h.fwd, args.repeats), "attn_bwd": time_events(h.bwd, args.repeats)}
    torch.cuda.synchronize()
    with _lib.kernel_timer() as timer:
        for _ in range(args.repeats):
            h.fwd()
            h.bwd()
    kernel_ms = {name: round(v / args.repeats, 4) for name, v in timer.ms.items() if timer.launches[name]}
    kernel_launches = {name: timer.launches[name] // args.repeats for name in kernel_ms}
    for name in kernel_ms:
        log(f"  {name}: {kernel_ms[name]:.3f} ms per call ({kernel_launches[name]} launches)")
    bwd_flops = 2.5 * fwd_flops
    dom = "kv_bwd_main_kernel"
    dom_ms = kernel_ms[dom]
    achieved = bwd_flops / (dom_ms * 1e-3) / 1e12
    entry_achieved = bwd_flops / (kt["attn_bwd"]["median"] * 1e-3) / 1e12
    log(f"attn_fwd: {kt['attn_fwd']['median']:.3f} ms, attn_bwd: {kt['attn_bwd']['median']:.3f} ms; "
        f"{dom}: {dom_ms:.3f} ms per backward = {achieved:.1f} TFLOP/s algorithmic")

    stages = {}
    peak_mem = {}
    if not args.no_stages:
        def score_fwd():
            with torch.no_grad():
                msa.m3_index_score(iq, ik, cu, max_len, block_size=block)

        def sel():
            msa.m3_topk(scores, cu, block_size=block, topk_blocks=topk, local_blocks=local)

        def csr():
            build_k2q_csr(ids, cu, block_size=block)

        # the same two stages with prepared sequence metadata: no host read of cu_seqlens
        # and no host-to-device metadata copies, i.e. the kernels' own time
        seqs_stage = msa.prepare_sequences(cu, block_size=block)

        def sel_prepared():
            msa.m3_topk(scores, seqs_stage, block_size=block, topk_blocks=topk, local_blocks=local)

        def csr_prepared():
            build_k2q_csr(ids, seqs_stage, block_size=block)

        def attn_fwd():
            with torch.no_grad():
                msa.m3_sparse_attention(q, k, v, ids, cu, max_len, block_size=block)

        def pipeline_fwd():
            with torch.no_grad():
                s = msa.m3_index_score(iq, ik, cu, max_len, block_size=block)
                i2 = msa.m3_topk(s, cu, block_size=block, topk_blocks=topk, local_blocks=local)
                msa.m3_sparse_attention(q, k, v, i2, cu, max_len, block_size=block)

        def score_topk_fused():
            with torch.no_grad():
                msa.m3_index_score_topk(iq, ik, cu, max_len, block_size=block, topk_blocks=topk, local_blocks=local)

        def pipeline_fwd_fused():
            with torch.no_grad():
                _, i2 = msa.m3_index_score_topk(iq, ik, cu, max_len, block_size=block, topk_blocks=topk,
                                                local_blocks=local)
                msa.m3_sparse_attention(q, k, v, i2, cu, max_len, block_size=block)

        iqg, ikg = iq.detach().clone().requires_grad_(), ik.detach().clone().requires_grad_()
        ones = torch.ones_like(scores)

        def score_fwd_bwd():
            iqg.grad = ikg.grad = None
            msa.m3_index_score(iqg, ikg, cu, max_len, block_size=block).backward(ones)

        # the score backward alone (dq and dk of the same gradient, through a retained graph)
        iqs_, iks_ = iq.detach().clone().requires_grad_(), ik.detach().clone().requires_grad_()
        s_kept = msa.m3_index_score(iqs_, iks_, cu, max_len, block_size=block)

        def score_bwd():
            iqs_.grad = iks_.grad = None
            s_kept.backward(ones, retain_graph=True)

        # the whole layer: score -> top-k -> attention forward, then the attention backward
        # (dQ, dK, dV) and the score backward (an N(0,1) gradient on the valid scores)
        iqp, ikp = iq.detach().clone().requires_grad_(), ik.detach().clone().requires_grad_()
        qp, kp, vp = (x.detach().clone().requires_grad_() for x in (q, k, v))
        dscore = torch.randn(scores.shape, generator=torch.Generator().manual_seed(9)).to(device)
        dscore = dscore.masked_fill(torch.isinf(scores), 0)

        def pipeline_fwd_bwd():
            iqp.grad = ikp.grad = qp.grad = kp.grad = vp.grad = None
            s = msa.m3_index_score(iqp, ikp, cu, max_len, block_size=block)
            i2 = msa.m3_topk(s.detach(), cu, block_size=block, topk_blocks=topk, local_blocks=local)
            msa.m3_sparse_attention(qp, kp, vp, i2, cu, max_len, block_size=block).backward(dout)
            s.backward(dscore)

        iqk, ikk = iq.detach().clone().requires_grad_(), ik.detach().clone().requires_grad_()

        def indexer_kl():
            # the KL training branch: loss with index_q / index_k gradients (teacher from q, k)
            iqk.grad = ikk.grad = None
            msa.m3_indexer_kl(iqk, ikk, q, k, ids, cu, max_len, block_size=block).backward()

        with torch.no_grad():
            _, attn_lse = msa.m3_sparse_attention(q, k, v, ids, cu, max_len, block_size=block, return_lse=True)

        def indexer_kl_lse():
            # the same, with the teacher normalisers taken from the attention forward's lse
            iqk.grad = ikk.grad = None
            msa.m3_indexer_kl(iqk, ikk, q, k, ids, cu, max_len, block_size=block, teacher_lse=attn_lse).backward()

        reps = max(3, args.repeats // 2)
        for name, fn in (("score_fwd_ms", score_fwd), ("topk_ms", sel), ("k2q_csr_ms", csr),
                         ("topk_prepared_ms", sel_prepared), ("k2q_csr_prepared_ms", csr_prepared),
                         ("attention_fwd_ms", attn_fwd), ("pipeline_fwd_ms", pipeline_fwd),
                         ("score_fwd_bwd_ms", score_fwd_bwd), ("score_bwd_ms", score_bwd),
                         ("score_topk_fused_ms", score_topk_fused),
                         ("pipeline_fwd_fused_ms", pipeline_fwd_fused), ("pipeline_fwd_bwd_ms", pipeline_fwd_bwd),
                         ("indexer_kl_fwd_bwd_ms", indexer_kl), ("indexer_kl_teacher_lse_fwd_bwd_ms", indexer_kl_lse)):
            stages[name] = round(time_events(fn, reps)["median"], 4)
            peak_mem[name.replace("_ms", "")] = round(peak_bytes(fn) / 2**20, 1)
            log(f"{name}: {stages[name]:.3f} (peak {peak_mem[name.replace('_ms', '')]:.0f} MiB)")
        stages["attention_fwd_bwd_ms"] = round(ms, 4)
        peak_mem["attention_fwd_bwd"] = round(peak_bytes(step) / 2**20, 1)

        # fp16 inputs on the MFMA kernels (fp16 products; P and dS split into fp16 terms under
        # power-of-two scales, dQ's dS planes in bf16 against K as two bf16 terms): the same step
        # on this config's inputs and selection, converted to fp16, one step at a time
        h16 = [x.detach().half().requires_grad_() for x in (q, k, v)]
        dout16 = dout.half()

        def step_fp16():
            for x in h16:
                x.grad = None
            msa.m3_sparse_attention(*h16, ids, cu, max_len, block_size=block).backward(dout16)

        stages["attention_fwd_bwd_fp16_ms"] = round(time_events(step_fp16, 3)["median"], 4)
        peak_mem["attention_fwd_bwd_fp16"] = round(peak_bytes(step_fp16) / 2**20, 1)
        log(f"attention_fwd_bwd_fp16_ms: {stages['attention_fwd_bwd_fp16_ms']:.3f} "
            f"({step_flops / stages['attention_fwd_bwd_fp16_ms'] / 1e9:.1f} TFLOP/s)")
        del h16, dout16
        # head dim 256 on the MFMA kernels: this config's tokens, heads and selection with
        # bf16 q / k / v / dO of 256 dims (seeded N(0, 1)); twice the FLOPs of D = 128
        g256 = torch.Generator().manual_seed(256)
        d256 = [torch.randn(x.shape[0], x.shape[1], 256, generator=g256).to(torch.bfloat16).to(device)
                for x in (q, k, v, dout)]
        for x in d256[:3]:
            x.requires_grad_()

        def step_d256():
            for x in d256[:3]:
                x.grad = None
            msa.m3_sparse_attention(*d256[:3], ids, cu, max_len, block_size=block).backward(d256[3])

        stages["attention_fwd_bwd_d256_ms"] = round(time_events(step_d256, 3)["median"], 4)
        peak_mem["attention_fwd_bwd_d256"] = round(peak_bytes(step_d256) / 2**20, 1)
        d256_flops = step_flops * 256 / cfg["d"]
        log(f"attention_fwd_bwd_d256_ms: {stages['attention_fwd_bwd_d256_ms']:.3f} "
            f"({d256_flops / stages['attention_fwd_bwd_d256_ms'] / 1e9:.1f} TFLOP/s)")
        del d256
        # one rank's share under group (head) parallelism over the config's G groups: group
        # 0's query heads, K / V and selection (G = 1, Hq / G heads), i.e. the kernels a rank
        # runs when the G groups are spread over G GPUs (no exchange inside the operators)
        rheads = cfg["hq"] // cfg["g"]
        share = [x.detach()[:, :rheads if x.shape[1] == cfg["hq"] else 1].contiguous() for x in (q, k, v, dout)]
        for x in share[:3]:
            x.requires_grad_()
        ids_share = ids[:, :1].contiguous()

        def step_share():
            for x in share[:3]:
                x.grad = None
            msa.m3_sparse_attention(*share[:3], ids_share, cu, max_len, block_size=block).backward(share[3])

        stages["attention_fwd_bwd_rank_share_ms"] = round(time_events(step_share, 5)["median"], 4)
        log(f"attention_fwd_bwd_rank_share_ms (G = 1, Hq = {rheads}): {stages['attention_fwd_bwd_rank_share_ms']:.3f} "
            f"({step_flops / cfg['g'] / stages['attention_fwd_bwd_rank_share_ms'] / 1e9:.1f} TFLOP/s)")
        del share, ids_share
        # the same autograd step with prepared sequence metadata (no host reads of
        # cu_seqlens), eager and replayed from a HIP graph capture
        seqs = msa.prepare_sequences(cu, block_size=block)

        def step_prepared():
            qg.grad = kg.grad = vg.grad = None
            msa.m3_sparse_attention(qg, kg, vg, ids, seqs, max_len, block_size=block).backward(dout)

        stages["attention_fwd_bwd_prepared_ms"] = round(time_loop(step_prepared, args.steps), 4)
        log(f"attention_fwd_bwd_prepared_ms: {stages['attention_fwd_bwd_prepared_ms']:.3f}")
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(2):
                step_prepared()
        torch.cuda.current_stream().wait_stream(side)
        qg.grad = kg.grad = vg.grad = None
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            msa.m3_sparse_attention(qg, kg, vg, ids, seqs, max_len, block_size=block).backward(dout)
        stages["attention_fwd_bwd_graph_ms"] = round(time_loop(graph.replay, args.steps), 4)
        log(f"attention_fwd_bwd_graph_ms: {stages['attention_fwd_bwd_graph_ms']:.3f}")
        del graph
        stages["attention_bwd_kernel_ms"] = round(kt["attn_bwd"]["median"], 4)
        stages["attention_fwd_kernel_ms"] = round(kt["attn_fwd"]["median"], 4)
        # backward sub-stages (HIP events around each kernel): prep = centre + work plans +
        # statistics pass of the peaked rows; main = the S / dP / dV / dK / dQ products;
        # dkdv = item partials into dK / dV; dq = slot-order dQ merge
        km = kernel_ms.get
        stages["attention_bwd_prep_ms"] = round(km("kv_bwd_center", 0) + km("bwd_plan", 0) +
                                                km("kv_bwd_stats_kernel", 0) + km("kv_bwd_stats_combine", 0), 4)
        stages["attention_bwd_main_ms"] = km(dom, 0)
        stages["attention_bwd_dkdv_ms"] = km("kv_bwd_accumulate", 0)
        stages["attention_bwd_dq_ms"] = km("kv_bwd_dq_combine", 0)
        stages["attention_fwd_partial_ms"] = km("attn_fwd_partial_kernel", 0)
        stages["attention_fwd_combine_ms"] = km("attn_fwd_combine", 0)
        stages["kernel_ms_per_call"] = kernel_ms
        stages["kernel_launches_per_call"] = kernel_launches
        stages["peak_mem_mib"] = peak_mem
        score_flops, topk_bytes, csr_bytes, score_bwd_bytes = stage_work(cfg)
        score_bwd_ms = stages["score_bwd_ms"]

        def frac(work, ms_, peak, scale):
            achieved_ = work / (ms_ * 1e-3) / scale
            return {"achieved": round(achieved_, 2), "peak": peak, "frac": round(achieved_ / peak, 4)}

        stages["roofline"] = {
            "score_fwd": {"bound": "mfma", "unit": "TFLOP/s", **frac(score_flops, stages["score_fwd_ms"],
                                                                      MFMA_BF16_PEAK_TFLOPS, 1e12)},
            # score backward on its unavoidable HBM bytes (ds and tie codes read, the rows of
            # index_q / index_k read once, dq / dk written); its row gathers hit the caches
            "score_bwd": {"bound": "hbm", "unit": "GB/s", **frac(score_bwd_bytes, score_bwd_ms, HBM_PEAK_GBPS, 1e9)},
            # top-k and CSR on their prepared-metadata timings (the plain stage times add host reads)
            "topk": {"bound": "hbm", "unit": "GB/s", **frac(topk_bytes, stages["topk_prepared_ms"], HBM_PEAK_GBPS, 1e9)},
            "k2q_csr": {"bound": "hbm", "unit": "GB/s",
                        **frac(csr_bytes, stages["k2q_csr_prepared_ms"], HBM_PEAK_GBPS, 1e9)},
            "attention_fwd": {"bound": "mfma", "unit": "TFLOP/s",
                              **frac(fwd_flops, stages["attention_fwd_kernel_ms"], MFMA_BF16_PEAK_TFLOPS, 1e12)},
            "attention_fwd_partial_kernel": {"bound": "mfma", "unit": "TFLOP/s",
                                             **frac(fwd_flops, stages["attention_fwd_partial_ms"],
                                                    MFMA_BF16_PEAK_TFLOPS, 1e12)},
            "attention_bwd": {"bound": "mfma", "unit": "TFLOP/s",
                              **frac(bwd_flops, stages["attention_bwd_kernel_ms"], MFMA_BF16_PEAK_TFLOPS, 1e12)},
            "kv_bwd_main_kernel": {"bound": "mfma", "unit": "TFLOP/s",
                                   **frac(bwd_flops, dom_ms, MFMA_BF16_PEAK_TFLOPS, 1e12)},
            "attention_fwd_bwd": {"bound": "mfma", "unit": "TFLOP/s",
                                  **frac(step_flops, ms, MFMA_BF16_PEAK_TFLOPS, 1e12)},
            # per visible (token, group, key): teacher logits 2 D R, student logits 2 Di,
            # d_iq and d_ik 2 Di each
            "indexer_kl": {"bound": "mfma", "unit": "TFLOP/s",
                           **frac(keys * (2.0 * cfg["d"] * (cfg["hq"] // cfg["g"]) + 6.0 * cfg["di"]),
                                  stages["indexer_kl_fwd_bwd_ms"], MFMA_BF16_PEAK_TFLOPS, 1e12)},
            # fp16 on the MFMA kernels, against the dense fp16 MFMA peak (the bf16 figure)
            "attention_fwd_bwd_fp16": {"bound": "mfma", "unit": "TFLOP/s",
                                       **frac(step_flops, stages["attention_fwd_bwd_fp16_ms"], MFMA_BF16_PEAK_TFLOPS,
                                              1e12)},
            # one rank's share under G-way group parallelism: 1 / G of the step's FLOPs
            "attention_fwd_bwd_rank_share": {"bound": "mfma", "unit": "TFLOP/s",
                                             **frac(step_flops / cfg["g"], stages["attention_fwd_bwd_rank_share_ms"],
                                                    MFMA_BF16_PEAK_TFLOPS, 1e12)},
            # head dim 256 (bf16): the step's FLOPs scaled by 256 / D
            "attention_fwd_bwd_d256": {"bound": "mfma", "unit": "TFLOP/s",
                                       **frac(step_flops * 256 / cfg["d"], stages["attention_fwd_bwd_d256_ms"],
                                              MFMA_BF16_PEAK_TFLOPS, 1e12)},
        }

    baseline = None
    if not args.no_cpu_baseline:
        log("cpu baseline ...")
        baseline = cpu_baseline(cfg, tensors_cpu, ids.cpu(), args.cpu_seconds)
        log(f"cpu baseline: {baseline['value']:.4f} TFLOP/s on {baseline['cores']} threads ({baseline['host']})")

    result = {
        "metric": "sparse-attn fwd+bwd TFLOP/s and per-stage ms @32K tokens on 1xMI355X",
        "value": round(step_flops / (ms * 1e-3) / 1e12, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "step_ms": {k_: round(v_, 4) for k_, v_ in step_stats.items()},
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) bf16, reference benchmark draw order)",
        "config": {"workload": f"{args.config}: T={total} lengths={cfg['lengths']} Hq={cfg['hq']} G={cfg['g']} "
                               f"D={cfg['d']} Di={cfg['di']} block={block} topk={topk} local={local}; "
                               "step = m3_sparse_attention fwd+bwd (dQ,dK,dV)",
                   "effective_tflop_per_step": round(step_flops / 1e12, 4)},
        # the dominant kernel: the backward's main KV pass, which performs the whole
        # algorithmic backward (2.5 x forward FLOPs) in kernel_launches launches per call
        "roofline": {"bound": "mfma", "kernel": dom, "achieved": round(achieved, 2),
                     "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(achieved / MFMA_BF16_PEAK_TFLOPS, 4),
                     "traffic": measured_traffic(args.config, dom),
                     "kernel_ms_per_call": dom_ms, "kernel_launches": kernel_launches[dom],
                     "entry": {"name": "msa_attn_bwd", "ms": round(kt["attn_bwd"]["median"], 4),
                               "achieved": round(entry_achieved, 2),
                               "frac": round(entry_achieved / MFMA_BF16_PEAK_TFLOPS, 4),
                               "traffic": measured_traffic(args.config, "msa_attn_bwd", "entries")}},
        "cpu_baseline": baseline,
        "stages": stages,
    }
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
