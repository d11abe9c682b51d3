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
ENTRY_NAMES = {"attn_fwd": "msa_attn_fwd", "attn_bwd": "msa_attn_bwd"}

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
    # score backward: read ds and the tie codes of every valid (t, g, b), gather one index_k row
    # (dq) and one index_q row (dk) per valid entry, write dq and dk
    score_bwd_bytes = causal_blocks * g * (4 + 4 + 2 * di * 2) + T * g * di * 2 + T * di * 2
    return score_flops, topk_bytes, csr_bytes, score_bwd_bytes


def measured_traffic(config, entry):
    """HBM bytes per call of a C-ABI entry point from the committed rocprofv3 PMC summary
    (FETCH_SIZE and WRITE_SIZE, calibrated against a copy of known size), if present."""
    path = os.path.join(ROOT, "profiles", f"attn_{config}_traffic.json")
    try:
        with open(path) as f:
            data = json.load(f)
        return data["entries"][entry]["bytes_per_call"]
    except (OSError, KeyError, ValueError):
        return None


def _pmc_rows(directory, counter):
    """(dispatch id, kernel name, value in bytes) of one rocprofv3 counter pass, in dispatch order.
    FETCH_SIZE / WRITE_SIZE are reported in KiB per dispatch."""
    import csv
    import glob

    rows = []
    for path in glob.glob(os.path.join(directory, "**", "*counter_collection.csv"), recursive=True):
        with open(path) as f:
            for r in csv.DictReader(f):
                if r["Counter_Name"] == counter:
                    rows.append((int(r["Dispatch_Id"]), r["Kernel_Name"], float(r["Counter_Value"]) * 1024.0))
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
        first_fwd = max(i for i, r in enumerate(rows[:first_bwd]) if "kv_chunk_bounds" in r[1])
        for i, (_, name, value) in enumerate(rows[first_fwd:], start=first_fwd):
            entry = "msa_attn_fwd" if i < first_bwd else "msa_attn_bwd"
            short = name.split("(")[0].replace("void ", "").replace("msa::", "")
            d = per_kernel.setdefault((entry, short), {"dispatches": 0, "read": 0.0, "write": 0.0})
            if key == "read":
                d["dispatches"] += 1
            d[key] += value * scale
            e = out["entries"].setdefault(entry, {"read_bytes": 0.0, "write_bytes": 0.0})
            e[f"{key}_bytes"] += value * scale
    for e in out["entries"].values():
        e["read_bytes"] = int(e["read_bytes"])
        e["write_bytes"] = int(e["write_bytes"])
        e["bytes_per_call"] = e["read_bytes"] + e["write_bytes"]
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
        self.fws_bytes = self.lib.msa_attn_fwd_workspace_bytes(2, self.T, cfg["hq"], cfg["g"], cfg["d"], cfg["topk"],
                                                               self.meta.total_blocks, cfg["block"])
        self.fws = torch.empty(max(1, self.fws_bytes), dtype=torch.uint8, device=device)
        self.ws_bytes = self.lib.msa_attn_bwd_workspace_bytes(2, self.T, cfg["hq"], cfg["g"], cfg["d"], cfg["topk"],
                                                              self.meta.total_blocks, cfg["block"])
        self.ws = torch.empty(max(1, self.ws_bytes), dtype=torch.uint8, device=device)
        self.stream = torch.cuda.current_stream(device).cuda_stream

    def fwd(self):
        c = self.cfg
        csr = self.csr
        st = self.lib.msa_attn_fwd(self.q.data_ptr(), self.k.data_ptr(), self.v.data_ptr(), 2, self.ids.data_ptr(),
                                   self.cu.data_ptr(), self.meta.num_seqs, self.T, c["hq"], c["g"], c["d"], c["topk"],
                                   c["block"], self.scale, csr.cu_block_lens.data_ptr(), self.meta.total_blocks,
                                   csr.row_ptr.data_ptr(), csr.query_indices.data_ptr(), csr.slot_indices.data_ptr(),
                                   self.fws.data_ptr(), self.fws_bytes, self.out.data_ptr(), self.lse.data_ptr(),
                                   self.rs.data_ptr(), self.o32.data_ptr(), self.stream)
        assert st == 0

    def bwd(self):
        c = self.cfg
        csr = self.csr
        st = self.lib.msa_attn_bwd(self.q.data_ptr(), self.k.data_ptr(), self.v.data_ptr(), 2, self.out.data_ptr(),
                                   self.dout.data_ptr(), self.rs.data_ptr(),
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


def cpu_baseline(cfg, tensors, ids_cpu, budget_s):
    """Eager CPU restatement (oracle/eager_baseline.py) on the last query rows of the
    first sequence, row-chunked, until ~budget_s seconds of CPU work; returns the
    effective fwd+bwd TFLOP/s of the sample."""
    import torch

    from oracle.eager_baseline import eager_rows_fwd_bwd

    iq, ik, q, k, v, dout = tensors
    n0 = cfg["lengths"][0]
    b, kk, hq, d = cfg["block"], cfg["topk"], cfg["hq"], cfg["d"]
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
    return {
        "value": flops / elapsed / 1e12,
        "unit": "TFLOP/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": (f"eager bf16 restatement (eager/ops.py:153-180 math, dense masked rows, torch CPU autograd) "
                   f"fwd+bwd of the last {rows_done} query rows of the {n0}-token sequence in {chunk}-row chunks, "
                   f"{elapsed:.1f} s; effective FLOPs counted like the GPU value"),
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
                        help="for rocprofv3 --pmc: a 256 MiB calibration copy, then one attention forward and one "
                             "backward call (direct C ABI) and exit")
    parser.add_argument("--pmc-summarize", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"),
                        help="read the counter CSVs of two --pmc-pass runs (FETCH_SIZE, WRITE_SIZE), write "
                             "profiles/attn_<config>_traffic.json and print a markdown table; no GPU needed")
    args = parser.parse_args()
    if args.pmc_summarize:
        summarize_pmc(args.config, *args.pmc_summarize)
        return
    if args.gpus != 1:
        print(f"bench.py measures one MI355X: --gpus {args.gpus} is not supported (this path does not shard "
              "across GPUs; see DESIGN.md for how it would).", file=sys.stderr)
        sys.exit(2)

    import torch

    import msa_triton_amd as msa
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

    # ---- per-kernel timings (direct C-ABI launches, HIP events on the launch stream)
    h = Harness(cfg, (iq, ik, q, k, v, dout), ids, cu, device)
    kern = {
        "attn_fwd": (h.fwd, fwd_flops),
        "attn_bwd": (h.bwd, 2.5 * fwd_flops),
    }
    h.fwd()
    kt = {name: time_events(fn, args.repeats) for name, (fn, _) in kern.items()}
    dom = max(kt, key=lambda n: kt[n]["median"])
    achieved = kern[dom][1] / (kt[dom]["median"] * 1e-3) / 1e12
    for name in kern:
        log(f"{name}: {kt[name]['median']:.3f} ms, {kern[name][1] / (kt[name]['median'] * 1e-3) / 1e12:.1f} "
            "TFLOP/s algorithmic")

    stages = {}
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
                         ("score_fwd_bwd_ms", score_fwd_bwd), ("score_topk_fused_ms", score_topk_fused),
                         ("pipeline_fwd_fused_ms", pipeline_fwd_fused), ("indexer_kl_fwd_bwd_ms", indexer_kl),
                         ("indexer_kl_teacher_lse_fwd_bwd_ms", indexer_kl_lse)):
            stages[name] = round(time_events(fn, reps)["median"], 4)
            log(f"{name}: {stages[name]:.3f}")
        stages["attention_fwd_bwd_ms"] = round(ms, 4)
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
        score_flops, topk_bytes, csr_bytes, score_bwd_bytes = stage_work(cfg)
        score_bwd_ms = max(stages["score_fwd_bwd_ms"] - stages["score_fwd_ms"], 1e-6)

        def frac(work, ms_, peak, scale):
            achieved_ = work / (ms_ * 1e-3) / scale
            return {"achieved": round(achieved_, 2), "peak": peak, "frac": round(achieved_ / peak, 4)}

        stages["roofline"] = {
            "score_fwd": {"bound": "mfma", "unit": "TFLOP/s", **frac(score_flops, stages["score_fwd_ms"],
                                                                      MFMA_BF16_PEAK_TFLOPS, 1e12)},
            "score_bwd": {"bound": "hbm", "unit": "GB/s", **frac(score_bwd_bytes, score_bwd_ms, HBM_PEAK_GBPS, 1e9)},
            # top-k and CSR on their prepared-metadata timings (the plain stage times add host reads)
            "topk": {"bound": "hbm", "unit": "GB/s", **frac(topk_bytes, stages["topk_prepared_ms"], HBM_PEAK_GBPS, 1e9)},
            "k2q_csr": {"bound": "hbm", "unit": "GB/s",
                        **frac(csr_bytes, stages["k2q_csr_prepared_ms"], HBM_PEAK_GBPS, 1e9)},
            "attention_fwd": {"bound": "mfma", "unit": "TFLOP/s",
                              **frac(fwd_flops, stages["attention_fwd_kernel_ms"], MFMA_BF16_PEAK_TFLOPS, 1e12)},
            "attention_bwd": {"bound": "mfma", "unit": "TFLOP/s",
                              **frac(2.5 * fwd_flops, stages["attention_bwd_kernel_ms"], MFMA_BF16_PEAK_TFLOPS,
                                     1e12)},
            # per visible (token, group, key): teacher logits 2 D R, student logits 2 Di,
            # d_iq and d_ik 2 Di each
            "indexer_kl": {"bound": "mfma", "unit": "TFLOP/s",
                           **frac(keys * (2.0 * cfg["d"] * (cfg["hq"] // cfg["g"]) + 6.0 * cfg["di"]),
                                  stages["indexer_kl_fwd_bwd_ms"], MFMA_BF16_PEAK_TFLOPS, 1e12)},
        }

    baseline = None
    if not args.no_cpu_baseline:
        log("cpu baseline ...")
        baseline = cpu_baseline(cfg, tensors_cpu, ids.cpu(), args.cpu_seconds)
        log(f"cpu baseline: {baseline['value']:.4f} TFLOP/s on {baseline['cores']} threads")

    result = {
        "metric": "sparse-attn fwd+bwd TFLOP/s and per-stage ms @32K tokens on 1xMI355X",
        "value": round(step_flops / (ms * 1e-3) / 1e12, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) bf16, reference benchmark draw order)",
        "config": {"workload": f"{args.config}: T={total} lengths={cfg['lengths']} Hq={cfg['hq']} G={cfg['g']} "
                               f"D={cfg['d']} Di={cfg['di']} block={block} topk={topk} local={local}; "
                               "step = m3_sparse_attention fwd+bwd (dQ,dK,dV)",
                   "effective_tflop_per_step": round(step_flops / 1e12, 4)},
        "roofline": {"bound": "mfma", "kernel": ENTRY_NAMES[dom], "achieved": round(achieved, 2),
                     "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(achieved / MFMA_BF16_PEAK_TFLOPS, 4),
                     "traffic": measured_traffic(args.config, ENTRY_NAMES[dom]),
                     "kernel_ms": round(kt[dom]["median"], 4)},
        "cpu_baseline": baseline,
        "stages": stages,
    }
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
