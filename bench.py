"""Benchmark of the LLAISYS KV-cache hot path on one MI355X.

Default workload: batched paged decode attention, B=64,
context lengths U[512, 8192] (seeded), 16-token pages over a randomly permuted
pool, GQA 12 query heads : 2 KV heads, head_dim 128, bf16 Q/K/V, fp32
accumulation, split-KV flash-decoding with the log-sum-exp combine.

One step = one llaisysPagedAttention call over the whole batch (one kernel
launch). Inputs are resident in HBM before timing. Two independent copies of
the inputs (pools, tables, queries) alternate between steps so that no step
finds the previous step's KV in the 256 MB MALL.

Printed (rank 0, one JSON line): the metric of BASELINE.json = achieved HBM
GB/s of the attention kernel (algorithmic bytes / average kernel time from HIP
events on the stream the kernel runs on), with the roofline fraction against
8 TB/s, a CPU baseline (the C oracle on host cores, a bounded sample of the
same workload) and, as "decode_tokens_per_s", the other half of the metric:
greedy decode of the whole random-init Qwen2-1.5B-shape model (config 5,
batch 128 x 2048-token paged contexts; --no-model skips it).

Other workloads (parity configs, for measurement): --workload append_gather
(config 2), mixed (config 4), qwen2 (config 5 alone: value = tokens/s), copy
(plain device copy, for rocprof counter calibration).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
SCALE = 1.0 / 128 ** 0.5


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=None, help="timed steps (default: 200; qwen2: 64)")
    p.add_argument("--warmup", type=int, default=None, help="untimed steps (default: 20; qwen2: 4)")
    p.add_argument("--workload", default="decode", choices=["decode", "mixed", "append_gather", "copy", "qwen2", "serve", "linear"])
    p.add_argument("--ag-fused-only", action="store_true",
                   help="--workload append_gather: time only the fused entry point (profiling runs)")
    p.add_argument("--cpu-seconds", type=float, default=10.0, help="budget of the CPU baseline sample")
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    p.add_argument("--no-model", action="store_true",
                   help="decode workload only: skip the Qwen2 config-5 tokens/s measurement")
    p.add_argument("--seed", type=int, default=0)
    p.add_argument("--copy-mib", type=float, default=512.0, help="--workload copy: bytes copied per launch, MiB")
    p.add_argument("--summarize", nargs=6, metavar=("STATS", "FETCH", "WRITE", "COPY_FETCH", "COPY_WRITE", "TAG"),
                   help="summarise rocprofv3 output directories into profiles/TAG.md and profiles/TAG_traffic.json")
    p.add_argument("--profiles-dir", default=str(ROOT / "profiles"), help="where the --summarize* outputs go")
    p.add_argument("--summarize-step", nargs=2, metavar=("TRACE_DIR", "TAG"),
                   help="per-step kernel table of a --workload qwen2 kernel trace into profiles/TAG.md")
    p.add_argument("--step-pmc", nargs=4, metavar=("FETCH", "WRITE", "COPY_FETCH", "COPY_WRITE"),
                   help="with --summarize-step: FETCH_SIZE / WRITE_SIZE runs of the same workload and of "
                        "--workload copy, for per-kernel HBM bytes per step")
    p.add_argument("--summarize-mfma", nargs="+", metavar="DIR",
                   help="STATS_DIR UTIL_DIR MOPS_DIR [INSTS_DIR] TAG: per-kernel MFMA use from a kernel trace and "
                        "two (three) counter runs into profiles/TAG.md")
    p.add_argument("--summarize-linear", nargs=3, metavar=("TRACE_DIR", "BENCH_LINE", "TAG"),
                   help="kernel table of a --workload linear kernel trace (and the JSON line that run printed) "
                        "into profiles/TAG.md")
    p.add_argument("--summarize-ag-modes", nargs=3, metavar=("TRACE_DIR", "BENCH_LINE", "TAG"),
                   help="appendGatherKernel durations by timing mode from a kernel trace of --workload "
                        "append_gather --ag-fused-only (and the JSON line that run printed) into profiles/TAG.md")
    p.add_argument("--profiled-args", default="--no-cpu --no-model --steps 200",
                   help="bench arguments of the kernel-trace run")
    p.add_argument("--pmc-args", default="--no-cpu --no-model --steps 20 --warmup 5",
                   help="bench arguments of the PMC runs")
    return p.parse_args()


# ----------------------------------------------------------------- inputs


def seeded_ints(seed, n, lo, hi):
    import oracle  # seeded generator only (same draws as the parity tests)

    return oracle.randint(seed, n, lo, hi).astype("int32")


class Instance:
    """One resident copy of a paged-attention problem (pools, table, lengths, q)."""

    def __init__(self, ctx, lq, seed, dev_torch):
        import numpy as np
        import torch

        import llaisys_amd as L

        self.ctx = np.asarray(ctx, np.int32)
        self.lq = np.asarray(lq, np.int32)
        pages = (self.ctx + 15) // 16
        self.maxp = int(pages.max())
        self.nb = int(pages.sum())
        g = torch.Generator(device=dev_torch).manual_seed(seed)
        perm = torch.randperm(self.nb, generator=g, device=dev_torch).to(torch.int32).cpu().numpy()
        table = np.full((len(self.ctx), self.maxp), -1, np.int32)
        used = 0
        for b, p in enumerate(pages):
            table[b, :p] = perm[used:used + p]
            used += p
        self.table_np = table
        self.T = int(self.lq.sum())

        def resident(t):
            """Move a torch tensor into a llaisys tensor and drop the torch copy."""
            lt = L.Tensor(tuple(t.shape), dtype={torch.bfloat16: L.DataType.BF16, torch.int32: L.DataType.I32,
                                                  torch.float32: L.DataType.F32}[t.dtype], device=L.DeviceType.AMD)
            L.RuntimeAPI(L.DeviceType.AMD).memcpy_sync(lt.data_ptr(), t.data_ptr(), t.numel() * t.element_size(),
                                                       L.MemcpyKind.D2D)
            return lt

        shape = (self.nb, 2, 16, 128)
        # i.i.d. N(0,1) values: any permutation inside a page is the same distribution.
        self.k_pool = resident(torch.randn(shape, generator=g, device=dev_torch, dtype=torch.float32).to(torch.bfloat16))
        self.v_pool = resident(torch.randn(shape, generator=g, device=dev_torch, dtype=torch.float32).to(torch.bfloat16))
        self.q = resident(torch.randn((self.T, 12, 128), generator=g, device=dev_torch).to(torch.bfloat16))
        self.out = resident(torch.zeros((self.T, 12, 128), device=dev_torch, dtype=torch.bfloat16))
        self.table = resident(torch.from_numpy(table).to(dev_torch))
        self.ctx_t = resident(torch.from_numpy(self.ctx).to(dev_torch))
        cu = np.concatenate([[0], np.cumsum(self.lq)]).astype(np.int32)
        self.cu_np = cu
        self.cu_q = resident(torch.from_numpy(cu).to(dev_torch))
        torch.cuda.synchronize()

    def algorithmic_bytes(self):
        """KV read once per (token, kv head) + q + out + table + lengths (bf16 KV = 1024 B/token)."""
        kv = int(self.ctx.sum()) * 2 * 2 * 128 * 2
        qo = 2 * self.T * 12 * 128 * 2
        meta = int(((self.ctx + 15) // 16).sum()) * 4 + len(self.ctx) * 4
        return kv + qo + meta

    def decode(self, L):
        L.Ops.paged_attention(self.out, self.q, self.k_pool, self.v_pool, self.table, self.ctx_t, SCALE)

    def mixed(self, L):
        L.Ops.paged_attention_varlen(self.out, self.q, self.k_pool, self.v_pool, self.table, self.cu_q, self.ctx_t,
                                     SCALE)


# ----------------------------------------------------------------- timing


def time_steps(step, stream, steps, warmup):
    """HIP events on the library's stream around exactly `steps` launches,
    bracketed by device synchronisation; returns (avg kernel ms, wall ms/step)."""
    import torch

    for i in range(warmup):
        step(i)
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record(stream)
    for i in range(steps):
        step(i)
    end.record(stream)
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) * 1e3 / steps
    return start.elapsed_time(end) / steps, wall


def time_steps_flushed(step, stream, steps, warmup, flush_mib=512):
    """Like time_steps, but before every step an untimed read (a sum) of a
    flush_mib MiB buffer on the same stream evicts L2 and the 256 MB MALL, so
    each step reads its inputs from HBM. A read leaves the caches clean: no
    write-back of the flush lands inside the timed step. HIP events bracket
    each step alone. Returns (avg kernel ms, wall ms/step including the flush)."""
    import torch

    a = torch.zeros((flush_mib << 20) // 4, dtype=torch.float32, device="cuda")
    for i in range(warmup):
        step(i)
    torch.cuda.synchronize()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    t0 = time.perf_counter()
    for i in range(steps):
        with torch.cuda.stream(stream):
            a.sum()
        ev[i][0].record(stream)
        step(i)
        ev[i][1].record(stream)
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) * 1e3 / steps
    return sum(s.elapsed_time(e) for s, e in ev) / steps, wall


def host_cpus():
    """(threads the CPU legs use, CPUs this process may run on, os.cpu_count()).
    The legs use every CPU of the process's affinity set up to 16, the CPU
    share of a one-GPU box here (the machine's other cores serve other GPUs)."""
    try:
        allowed = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        allowed = os.cpu_count() or 1
    return max(1, min(allowed, 16)), allowed, os.cpu_count()


def _timed(fn, budget_s, min_reps=1):
    """Repeat fn until budget_s has passed (at least min_reps times); seconds per call."""
    reps, total = 0, 0.0
    while total < budget_s or reps < min_reps:
        t0 = time.perf_counter()
        fn()
        total += time.perf_counter() - t0
        reps += 1
    return total / reps, reps, total


def host_tensor(t, ldtype):
    """A LLAISYS_DEVICE_CPU tensor holding a copy of torch tensor t (any device)."""
    import llaisys_amd as L

    t = t.detach().contiguous().cpu()
    lt = L.Tensor(tuple(t.shape), dtype=ldtype, device=L.DeviceType.CPU)
    if t.numel():
        L.RuntimeAPI(L.DeviceType.CPU).memcpy_sync(lt.data_ptr(), t.data_ptr(), t.numel() * t.element_size(),
                                                   L.MemcpyKind.H2H)
    return lt


def host_copy_of(lt):
    """A LLAISYS_DEVICE_CPU tensor with the contents of device tensor lt."""
    import llaisys_amd as L

    h = L.Tensor(lt.shape(), dtype=lt.dtype(), device=L.DeviceType.CPU)
    n = 1
    for d in lt.shape():
        n *= d
    esz = {L.DataType.BF16: 2, L.DataType.F16: 2, L.DataType.F32: 4, L.DataType.I32: 4, L.DataType.I64: 8}[lt.dtype()]
    if n:
        L.RuntimeAPI(L.DeviceType.AMD).memcpy_sync(h.data_ptr(), lt.data_ptr(), n * esz, L.MemcpyKind.D2H)
    return h


def time_host(fn, budget_s=2.0, warmup=10, repeat=100):
    """The reference harness's pattern (test/test_utils.py:163-183): warm-up
    calls, then up to `repeat` timed calls (fewer if budget_s runs out);
    seconds per call."""
    for _ in range(warmup):
        fn()
    n, t0 = 0, time.perf_counter()
    while n < repeat and (n == 0 or time.perf_counter() - t0 < budget_s):
        fn()
        n += 1
    return (time.perf_counter() - t0) / n, n


def cpu_baseline_decode(inst, budget_s):
    """CPU legs of the config-3 workload, on a prefix of its batch sized so one
    pass takes >= 1 s: the C oracle (oracle/oracle.c, the restatement of the
    reference's fp32 algorithm; kind "port") on all the legs' threads, and on
    one thread; the library's own host path (llaisysPagedAttention on CPU
    tensors, the same page-format pools) beside it. GB/s over the same
    per-token byte count as the GPU figure. Plus config 1 (the reference's own
    op, self_attention at L=1, S=513) on the GPU, the library's host path and
    the oracle."""
    import numpy as np
    import torch

    import oracle
    import llaisys_amd as L
    from llaisys_amd import MemcpyKind, RuntimeAPI, DeviceType

    threads, allowed, ncpu = host_cpus()
    api = RuntimeAPI(DeviceType.AMD)
    capi = RuntimeAPI(DeviceType.CPU)

    def host_copy(lt, dtype, shape):
        t = torch.empty(shape, dtype=dtype)
        api.memcpy_sync(t.data_ptr(), lt.data_ptr(), t.numel() * t.element_size(), MemcpyKind.D2H)
        return t

    def cpu_tensor(t, ldtype):
        t = t.contiguous()
        lt = L.Tensor(tuple(t.shape), dtype=ldtype, device=DeviceType.CPU)
        capi.memcpy_sync(lt.data_ptr(), t.data_ptr(), t.numel() * t.element_size(), MemcpyKind.H2H)
        return lt

    kdev_t = host_copy(inst.k_pool, torch.int16, (inst.nb, 2, 16, 128))
    vdev_t = host_copy(inst.v_pool, torch.int16, (inst.nb, 2, 16, 128))
    kdev, vdev = kdev_t.numpy().view(np.uint16), vdev_t.numpy().view(np.uint16)
    k_log = oracle.unpack_pages_np(kdev, False)
    v_log = oracle.unpack_pages_np(vdev, True)
    q_t = host_copy(inst.q, torch.int16, (inst.T, 12, 128))
    q = q_t.numpy().view(np.uint16)

    def oracle_pass(n, nt):
        return oracle.paged_attention(q[:n], k_log, v_log, inst.table_np[:n], inst.ctx[:n], SCALE, nthreads=nt)

    nseq = 4
    while True:
        t0 = time.perf_counter()
        oracle_pass(nseq, threads)
        if time.perf_counter() - t0 >= 1.0 or nseq >= len(inst.ctx):
            break
        nseq = min(len(inst.ctx), nseq * 2)
    per, reps, total = _timed(lambda: oracle_pass(nseq, threads), budget_s)
    ref = oracle_pass(nseq, threads)
    sample_bytes = int(inst.ctx[:nseq].sum()) * 1024 + 2 * nseq * 12 * 128 * 2
    n1 = min(4, len(inst.ctx))
    per1, reps1, total1 = _timed(lambda: oracle_pass(n1, 1), budget_s / 4)
    bytes1 = int(inst.ctx[:n1].sum()) * 1024 + 2 * n1 * 12 * 128 * 2

    # The library's host path on the same sample (device page format as is).
    kp = cpu_tensor(kdev_t.view(torch.bfloat16), L.DataType.BF16)
    vp = cpu_tensor(vdev_t.view(torch.bfloat16), L.DataType.BF16)
    qc = cpu_tensor(q_t[:nseq].view(torch.bfloat16), L.DataType.BF16)
    tab = cpu_tensor(torch.from_numpy(np.ascontiguousarray(inst.table_np[:nseq])), L.DataType.I32)
    cl = cpu_tensor(torch.from_numpy(np.ascontiguousarray(inst.ctx[:nseq])), L.DataType.I32)
    oc = L.Tensor((nseq, 12, 128), dtype=L.DataType.F32, device=DeviceType.CPU)
    perl, repsl, totall = _timed(lambda: L.Ops.paged_attention(oc, qc, kp, vp, tab, cl, SCALE), budget_s / 2)
    lib_out = torch.empty((nseq, 12, 128), dtype=torch.float32)
    capi.memcpy_sync(lib_out.data_ptr(), oc.data_ptr(), lib_out.numel() * 4, MemcpyKind.H2H)
    lib_rel = float(np.max(np.abs(lib_out.numpy() - ref)) / np.max(np.abs(ref)))
    assert L.device_error_flags() == 0

    # Config 1: the reference's own op at L=1, S=513, 12:2, d=128, fp32.
    qn, kn, vn = oracle.randn(1, (1, 12, 128)), oracle.randn(2, (513, 2, 128)), oracle.randn(3, (513, 2, 128))
    c1_bytes = (qn.size + kn.size + vn.size + qn.size) * 4
    c1_ref = oracle.self_attention(qn, kn, vn, SCALE)
    cq, ck, cv = (cpu_tensor(torch.from_numpy(x), L.DataType.F32) for x in (qn, kn, vn))
    co = L.Tensor((1, 12, 128), dtype=L.DataType.F32, device=DeviceType.CPU)
    c1_lib, c1_lib_reps, _ = _timed(lambda: L.Ops.self_attention(co, cq, ck, cv, SCALE), 1.0, 10)
    c1_got = torch.empty((1, 12, 128))
    capi.memcpy_sync(c1_got.data_ptr(), co.data_ptr(), c1_got.numel() * 4, MemcpyKind.H2H)
    c1_orc, c1_orc_reps, _ = _timed(lambda: oracle.self_attention(qn, kn, vn, SCALE), 1.0, 10)
    gq, gk, gv = (torch.from_numpy(x).cuda() for x in (qn, kn, vn))
    go = torch.zeros((1, 12, 128), device="cuda")

    def as_ll(t):
        lt = L.Tensor(tuple(t.shape), dtype=L.DataType.F32, device=DeviceType.AMD)
        api.memcpy_sync(lt.data_ptr(), t.data_ptr(), t.numel() * 4, MemcpyKind.D2D)
        return lt

    lq, lk, lv, lo = as_ll(gq), as_ll(gk), as_ll(gv), as_ll(go)
    stream = torch.cuda.ExternalStream(L.context_stream())
    c1_gpu_ms, _ = time_steps(lambda i: L.Ops.self_attention(lo, lq, lk, lv, SCALE), stream, 200, 20)
    c1_gpu_out = torch.empty((1, 12, 128))
    api.memcpy_sync(c1_gpu_out.data_ptr(), lo.data_ptr(), c1_gpu_out.numel() * 4, MemcpyKind.D2H)

    def rel(x):
        return float(np.max(np.abs(x.numpy() - c1_ref)) / np.max(np.abs(c1_ref)))

    got = host_copy(inst.out, torch.bfloat16, (inst.T, 12, 128))[:nseq].float().numpy()
    max_err = float(np.max(np.abs(got - ref)))
    return {
        "value": round(sample_bytes / per / 1e9, 3),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": f"oracle/oracle.c paged attention (fp32, OpenMP over sequences, {threads} threads of the "
                  f"{allowed} CPUs this process may use, capped at 16 = a one-GPU box's CPU share; "
                  f"os.cpu_count() = {ncpu}) on the first {nseq} of "
                  f"{len(inst.ctx)} sequences ({int(inst.ctx[:nseq].sum())} tokens), {reps} reps in "
                  f"{total:.1f} s; GPU bf16 vs CPU max|err| {max_err:.2e}",
        "host_cpus": {"used": threads, "affinity": allowed, "os_cpu_count": ncpu, "cap": 16},
        "single_thread": {
            "value": round(bytes1 / per1 / 1e9, 3), "unit": "GB/s", "cores": 1,
            "sample": f"the same code with one thread on the first {n1} sequences "
                      f"({int(inst.ctx[:n1].sum())} tokens), {reps1} reps in {total1:.1f} s",
        },
        "library_host_path": {
            "value": round(sample_bytes / perl / 1e9, 3), "unit": "GB/s", "cores": threads,
            "sample": f"llaisysPagedAttention on LLAISYS_DEVICE_CPU tensors (fp32 output), the same {nseq} "
                      f"sequences, {repsl} reps in {totall:.1f} s; max|err| / max|oracle| {lib_rel:.1e}",
        },
        "config1_self_attention": {
            "shape": "L=1, S=513, 12 q heads / 2 kv heads, d=128, fp32, causal",
            "bytes_per_call": c1_bytes,
            "gpu_us": round(c1_gpu_ms * 1e3, 2),
            "library_host_path_us": round(c1_lib * 1e6, 1),
            "oracle_one_thread_us": round(c1_orc * 1e6, 1),
            "host_path_threads": threads,
            "rel_err_vs_oracle": {"gpu": rel(c1_gpu_out), "library_host_path": rel(c1_got)},
        },
    }


# ----------------------------------------------------------------- workloads


def run_decode(args):
    import numpy as np
    import torch

    import llaisys_amd as L

    B = 64
    ctx = seeded_ints(args.seed, B, 512, 8192)
    insts = [Instance(ctx, np.ones(B, np.int32), args.seed + 1 + i, "cuda") for i in range(2)]
    stream = torch.cuda.ExternalStream(L.context_stream())
    kern_ms, wall_ms = time_steps(lambda i: insts[i % 2].decode(L), stream, args.steps, args.warmup)
    assert L.device_error_flags() == 0
    nbytes = insts[0].algorithmic_bytes()
    gbs = nbytes / (kern_ms * 1e-3) / 1e9
    line = {
        "metric": "paged decode attention achieved HBM GB/s (% of peak) + decode tokens/s, 1 GPU",
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall_ms, 5),
        "kernel_ms": round(kern_ms, 5),
        "pct_of_peak": round(100 * gbs / HBM_PEAK_GBS, 2),
        "decode_tokens_per_s_one_attention_layer": round(B / (kern_ms * 1e-3), 1),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) bf16 Q/K/V, seeded context lengths and block permutation)",
        "config": {
            "workload": "batched paged decode attention (BASELINE config 3)",
            "batch": B, "ctx_range": [512, 8192], "ctx_total": int(ctx.sum()), "block_size": 16,
            "q_heads": 12, "kv_heads": 2, "head_dim": 128, "accumulate": "fp32",
            "split": "stream-K over page pairs, log-sum-exp combine kernel",
            # the kernel's grid: 1.75 waves per CU, or more when the longest
            # context needs them (a wave's slice is at most 64 page pairs)
            "waves": max(int(os.environ.get("LLAISYS_DECODE_WAVES",
                                            torch.cuda.get_device_properties(0).multi_processor_count * 7 // 4)),
                         -(-B * 2 * ((insts[0].maxp + 1) // 2) // 64)),
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(gbs, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(gbs / HBM_PEAK_GBS, 4),
            "traffic": traffic_from_profiles("paged_decode_attention_b64"),
            "algorithmic_bytes_per_launch": nbytes,
        },
    }
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline_decode(insts[0], args.cpu_seconds)
    if not args.no_model:
        # The "+ decode tokens/s" half of the metric: config 5 on the same GPU.
        del insts
        torch.cuda.empty_cache()
        margs = argparse.Namespace(**vars(args))
        margs.steps, margs.warmup = 64, 4
        m = run_qwen2(margs)
        line["decode_tokens_per_s"] = m["value"]
        line["model"] = {"workload": m["config"]["workload"], "tokens_per_s": m["value"],
                         "ms_per_step": m["ms_per_step"], "steps": m["steps"], "warmup": m["warmup"],
                         "single_step_call_ms": m["config"]["single_step_call_ms"],
                         "batch": m["config"]["batch"], "context_at_start": m["config"]["context_at_start"],
                         "prefill_tokens_per_s": m["config"]["prefill_tokens_per_s"], "roofline": m["roofline"]}
        # The other measured rows of the path, for the record (their own
        # --workload runs give the full lines).
        torch.cuda.empty_cache()
        oargs = argparse.Namespace(**vars(args))
        oargs.steps, oargs.warmup = 100, 10
        ag = run_append_gather(oargs)
        torch.cuda.empty_cache()
        mx = run_mixed(oargs)
        torch.cuda.empty_cache()
        line["other_configs"] = {
            "config2_append_gather": {"GB/s": ag["value"], "frac_of_hbm_peak": ag["roofline"]["frac"],
                                      "kernel_ms": ag["kernel_ms"], "entry_point": ag["config"]["entry_point"],
                                      "same_bytes_device_copy_ms": ag["same_bytes_device_copy"]["kernel_ms"],
                                      "cpu_host_path_ms": (ag["cpu_host_path"] or {}).get("ms"),
                                      "two_calls_kernel_ms": (ag["two_calls"] or {}).get("kernel_ms")},
            "config4_mixed_prefill_decode": {"TFLOP/s": mx["value"], "kernel_ms": mx["kernel_ms"],
                                             "frac_of_mfma_peak": mx["roofline"]["frac"],
                                             "cpu_host_path_ms": (mx["cpu_host_path"] or {}).get("ms")},
        }
    return line


def run_mixed(args):
    import numpy as np
    import torch

    import llaisys_amd as L

    priors = np.array([0, 1024, 2048, 4096], np.int32)
    dec = seeded_ints(args.seed + 60, 60, 256, 4096)
    ctx = np.concatenate([priors + 512, dec]).astype(np.int32)
    lq = np.concatenate([np.full(4, 512), np.ones(60)]).astype(np.int32)
    insts = [Instance(ctx, lq, args.seed + 1 + i, "cuda") for i in range(2)]
    stream = torch.cuda.ExternalStream(L.context_stream())
    kern_ms, wall_ms = time_steps(lambda i: insts[i % 2].mixed(L), stream, args.steps, args.warmup)
    assert L.device_error_flags() == 0
    # Causal (query, key) pairs: prefill chunk queries see prior + i + 1 keys; decode queries see ctx keys.
    pairs = sum(int(p) * 512 + 512 * 513 // 2 for p in priors) + int(dec.sum())
    flops = pairs * 12 * 128 * 4
    host = None
    if not getattr(args, "no_cpu", False):
        i0 = insts[0]
        hq, hk, hv, ho, ht, hc, hcu = (host_copy_of(t) for t in (i0.q, i0.k_pool, i0.v_pool, i0.out, i0.table,
                                                                  i0.ctx_t, i0.cu_q))
        per, reps = time_host(lambda: L.Ops.paged_attention_varlen(ho, hq, hk, hv, ht, hcu, hc, SCALE),
                              budget_s=5.0, warmup=1, repeat=10)
        host = {"ms": round(per * 1e3, 2), "GFLOP/s": round(flops / per / 1e9, 1), "threads": host_cpus()[0],
                "reps": reps, "what": "llaisysPagedAttentionVarlen on LLAISYS_DEVICE_CPU tensors, same inputs"}
    return {
        "metric": "mixed chunked-prefill + decode paged attention TFLOP/s, 1 GPU",
        "value": round(flops / (kern_ms * 1e-3) / 1e12, 3), "unit": "TFLOP/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(wall_ms, 5),
        "kernel_ms": round(kern_ms, 5), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16", "data": "synthetic",
        "config": {"workload": "BASELINE config 4: 4x512 prefill chunks over priors {0,1024,2048,4096} + 60 decode"},
        "cpu_host_path": host,
        "roofline": {"bound": "mfma", "achieved": round(flops / (kern_ms * 1e-3) / 1e12, 3), "peak": 2500.0,
                     "unit": "TFLOP/s", "frac": round(flops / (kern_ms * 1e-3) / 1e12 / 2500.0, 4), "traffic": None},
    }


# The Qwen2-1.5B projections of prefill and mixed serving steps (M token rows):
# qkv, o, gate-up, down.
LINEAR_SHAPES = [(m, n, k) for m in (2048, 8192) for n, k in ((2048, 1536), (1536, 1536), (17920, 1536), (1536, 8960))]


def run_linear(args):
    """llaisysLinear (the hand-written MFMA GEMM) on the model's prefill and
    serving projection shapes, bf16, against torch.matmul (hipBLASLt) on the
    same inputs and stream."""
    import torch

    import llaisys_amd as L

    sys.path.insert(0, str(ROOT / "tests"))
    from utils import to_llaisys

    stream = torch.cuda.ExternalStream(L.context_stream())
    rows, tot_flops, tot_ours, tot_torch = [], 0.0, 0.0, 0.0
    steps, warmup = min(args.steps, 50), min(args.warmup, 5)
    for m, n, k in LINEAR_SHAPES:
        g = torch.Generator(device="cuda").manual_seed(args.seed + m + n + k)
        x = (torch.randn(m, k, device="cuda", generator=g) * 0.5).to(torch.bfloat16)
        w = (torch.randn(n, k, device="cuda", generator=g) * 0.05).to(torch.bfloat16)
        xl, wl = to_llaisys(x), to_llaisys(w)
        out = to_llaisys(torch.zeros(m, n, dtype=torch.bfloat16, device="cuda"))
        ours, _ = time_steps(lambda i: L.Ops.linear(out, xl, wl, None), stream, steps, warmup)
        y = torch.empty(m, n, dtype=torch.bfloat16, device="cuda")
        with torch.cuda.stream(stream):
            theirs, _ = time_steps(lambda i: torch.matmul(x, w.T, out=y), stream, steps, warmup)
        flops = 2.0 * m * n * k
        tot_flops, tot_ours, tot_torch = tot_flops + flops, tot_ours + ours, tot_torch + theirs
        rows.append({"M": m, "N": n, "K": k, "us": round(ours * 1e3, 2), "TFLOP/s": round(flops / ours / 1e9, 1),
                     "torch_us": round(theirs * 1e3, 2)})
    assert L.device_error_flags() == 0
    tf = tot_flops / (tot_ours * 1e-3) / 1e12
    return {
        "metric": "llaisysLinear bf16 TFLOP/s over the Qwen2-1.5B prefill/serving projection shapes, 1 GPU",
        "value": round(tf, 1), "unit": "TFLOP/s", "n_gpus": 1, "steps": steps, "warmup": warmup,
        "ms_per_step": round(tot_ours, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16", "data": "synthetic (seeded N(0,1) activations, N(0,0.05) weights)",
        "config": {"workload": "llaisysLinear on M in {2048, 8192} x (qkv, o, gate-up, down) of Qwen2-1.5B"},
        "torch_matmul_TFLOP/s": round(tot_flops / (tot_torch * 1e-3) / 1e12, 1),
        "shapes": rows,
        "roofline": {"bound": "mfma", "achieved": round(tf, 1), "peak": 2500.0, "unit": "TFLOP/s",
                     "frac": round(tf / 2500.0, 4), "traffic": None},
    }


QWEN2_1_5B = dict(nlayer=28, hs=1536, nh=12, nkvh=2, di=8960, voc=151936, epsilon=1e-6, theta=10000.0)


def qwen2_step_bytes(meta, ctx_total, B):
    """Algorithmic HBM bytes of one batched decode step: every weight once
    (the input embedding only for the B rows looked up), each layer's K/V of
    every context token once, the new K/V written once; activations are
    O(B * hidden) and left out."""
    hs, q, kv, di, voc = meta.hs, meta.nh * meta.dh, meta.nkvh * meta.dh, meta.di, meta.voc
    per_layer = 2 * ((q + 2 * kv) * hs + (q + 2 * kv) + hs * q + 2 * di * hs + hs * di + 2 * hs)
    weights = meta.nlayer * per_layer + 2 * voc * hs + 2 * hs + 2 * B * hs
    kv_bytes = meta.nlayer * 2 * kv * 2 * (ctx_total + B)
    return weights + kv_bytes, weights, kv_bytes


def run_qwen2(args):
    """random-init Qwen2-1.5B shape, 128 sequences with a
    2048-token paged context each (built by batched prefill steps through the
    model), then greedy decode steps of the whole batch. One step = one decode
    step of all 128 sequences (all 28 layers, LM head, argmax); the K timed
    steps are one llaisysQwen2ModelDecode call, which feeds each step's tokens
    back on the device. The same K steps as single llaisysQwen2ModelStep calls
    (next tokens back on the host each time) are reported beside it."""
    import numpy as np
    import torch

    from llaisys_amd.models import Qwen2, Qwen2Meta

    B, ctx0 = 128, 2048
    meta = Qwen2Meta(**QWEN2_1_5B, maxseq=ctx0 + 2 * (args.warmup + args.steps) + 16)
    blocks = B * ((meta.maxseq + 15) // 16) + 16
    t0 = time.perf_counter()
    model = Qwen2.random(meta, seed=args.seed, std=0.02, num_blocks=blocks)
    ids = np.array([model.create_sequence()[0] for _ in range(B)], np.int64)
    prompts = np.random.default_rng(args.seed).integers(0, meta.voc, (B, ctx0), dtype=np.int64)
    nxt = np.zeros(B, np.int64)
    torch.cuda.synchronize()
    t_init = time.perf_counter() - t0
    chunk = 16  # sequences per prefill step: 32768 tokens
    t0 = time.perf_counter()
    for c in range(0, B, chunk):
        out = np.zeros(chunk, np.int64)
        model.step_arrays(ids[c:c + chunk], np.ascontiguousarray(prompts[c:c + chunk].reshape(-1)),
                          np.full(chunk, ctx0, np.uint64), out)
        nxt[c:c + chunk] = out
    t_prefill = time.perf_counter() - t0
    ones = np.ones(B, np.uint64)
    cur = nxt.copy()

    # Warm-up: single steps (capture the one-step graph) and one multi-step call.
    def step(_):
        model.step_arrays(ids, cur, ones, nxt)
        cur[:] = nxt

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    # For reference: K single-step calls (next tokens back on the host each time).
    t0 = time.perf_counter()
    for i in range(args.steps):
        step(i)
    torch.cuda.synchronize()
    single_ms = (time.perf_counter() - t0) * 1e3 / args.steps
    cur[:] = model.decode(ids, cur, args.warmup)[-1]
    torch.cuda.synchronize()
    ctx_start = int(sum(model.length(int(i)) for i in ids))
    # Timed: exactly K decode steps of the batch in one multi-step call (tokens
    # fed back on the device), bracketed by device synchronisation.
    t0 = time.perf_counter()
    toks = model.decode(ids, cur, args.steps)
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / args.steps
    cur[:] = toks[-1]
    # mean context over the timed steps (it grows by one token per step)
    ctx_mean_total = ctx_start + B * (args.steps - 1) / 2
    nbytes, wbytes, kvbytes = qwen2_step_bytes(meta, ctx_mean_total, B)
    gbs = nbytes / (ms * 1e-3) / 1e9
    return {
        "metric": "paged decode attention achieved HBM GB/s (% of peak) + decode tokens/s, 1 GPU",
        "value": round(B / (ms * 1e-3), 1),
        "unit": "tokens/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (random-init bf16 weights ~ N(0,0.02), seeded random prompts)",
        "config": {"workload": "BASELINE config 5: Qwen2-1.5B-shape greedy decode step", "batch": B,
                   "context_at_start": ctx0, **QWEN2_1_5B, "head_dim": 128, "block_size": 16,
                   "timed_call": f"llaisysQwen2ModelDecode, {args.steps} steps",
                   "single_step_call_ms": round(single_ms, 4),
                   "prefill_tokens_per_s": round(B * ctx0 / t_prefill, 1), "setup_s": round(t_init, 2)},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4),
                     "traffic": traffic_from_profiles("qwen2_1.5b_decode_step_b128"),
                     "algorithmic_bytes_per_step": int(nbytes), "weight_bytes": int(wbytes),
                     "kv_bytes": int(kvbytes)},
    }


def run_serve(args):
    """Continuous batching on the Qwen2-1.5B shape (random-init weights): R
    requests with seeded prompt lengths U[128, 1024] and 128 greedy tokens
    each go through the scheduler (128 sequences at once, 2048 tokens per step,
    prefill chunks of 512); every scheduler step is one mixed varlen model
    step. Model.warm_up() first tunes the GEMM kernel of every decode-sized
    token-count bucket, and a pass of short requests captures the decode
    graphs of the batch sizes. Timed: from the first step to the last request finishing, with
    the device synchronised at both ends. --steps sets R (default 256)."""
    import numpy as np
    import torch

    from llaisys_amd import Scheduler
    from llaisys_amd.models import Qwen2, Qwen2Meta

    R = args.steps if args.steps != 64 else 256
    max_seqs, budget, chunk, new = 128, 2048, 512, 128
    meta = Qwen2Meta(**QWEN2_1_5B, maxseq=1024 + new + 16)
    blocks = max_seqs * ((meta.maxseq + 15) // 16) + 64
    model = Qwen2.random(meta, seed=args.seed, std=0.02, num_blocks=blocks)
    rng = np.random.default_rng(args.seed)

    def serve(n, lo, hi, new_tokens):
        sched = Scheduler(model, max_seqs=max_seqs, max_step_tokens=budget, prefill_chunk=chunk)
        lens = rng.integers(lo, hi + 1, n)
        rids = [sched.add(rng.integers(0, meta.voc, int(m)).tolist(), max_new_tokens=new_tokens) for m in lens]
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        steps = sched.run()
        torch.cuda.synchronize()
        dt = time.perf_counter() - t0
        gen = sum(len(sched.tokens(r)) for r in rids)
        return dt, steps, gen, int(lens.sum()), sched.stats()

    model.warm_up(256)  # tunes every decode-sized step shape bucket
    serve(max(args.warmup, 1) * 64, 1, 300, 24)  # warm-up: graphs of the batch sizes
    dt, steps, gen, prompt_tokens, st = serve(R, 128, 1024, new)
    return {
        "metric": "continuous-batching greedy generation tokens/s (Qwen2-1.5B shape), 1 GPU",
        "value": round(gen / dt, 1), "unit": "tokens/s",
        "n_gpus": 1, "steps": steps, "warmup": args.warmup, "ms_per_step": round(dt * 1e3 / steps, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (random-init bf16 weights ~ N(0,0.02), seeded random prompts)",
        "config": {"workload": "continuous batching through llaisysQwen2Scheduler*", "requests": R,
                   "prompt_len": [128, 1024], "new_tokens": new, "max_seqs": max_seqs,
                   "max_step_tokens": budget, "prefill_chunk": chunk, **QWEN2_1_5B,
                   "prompt_tokens": prompt_tokens, "generated_tokens": gen,
                   "prompt_plus_generated_tokens_per_s": round((prompt_tokens + gen) / dt, 1),
                   "seconds": round(dt, 3), "scheduler": st},
    }


def run_append_gather(args):
    import numpy as np
    import torch

    import llaisys_amd as L

    B, nb = 32, 4096
    seed = args.seed
    while True:
        lens = seeded_ints(seed, B, 1, 2048)
        if ((lens + 16) // 16).sum() <= nb:
            break
        seed += 1
    need = (lens + 16) // 16
    maxp = int(need.max())
    g = torch.Generator(device="cuda").manual_seed(args.seed)
    perm = torch.randperm(nb, generator=g, device="cuda").to(torch.int32).cpu().numpy()
    table = np.full((B, maxp), -1, np.int32)
    used = 0
    for b, p in enumerate(need):
        table[b, :p] = perm[used:used + p]
        used += p
    pool_k = torch.randn((nb, 2, 16, 128), device="cuda").to(torch.bfloat16)
    pool_v = torch.randn((nb, 2, 16, 128), device="cuda").to(torch.bfloat16)
    sys.path.insert(0, str(ROOT / "tests"))
    from utils import to_llaisys

    kp, vp = to_llaisys(pool_k), to_llaisys(pool_v)
    kn_t = torch.randn((B, 2, 128), device="cuda").to(torch.bfloat16)
    vn_t = torch.randn((B, 2, 128), device="cuda").to(torch.bfloat16)
    kn, vn = to_llaisys(kn_t), to_llaisys(vn_t)
    tab = to_llaisys(torch.from_numpy(table))
    ctx = to_llaisys(torch.from_numpy(lens))
    cu = np.concatenate([[0], np.cumsum(lens + 1)]).astype(np.int32)
    T = int(cu[-1])
    ko = to_llaisys(torch.zeros((T, 2, 128), dtype=torch.bfloat16, device="cuda"))
    vo = to_llaisys(torch.zeros((T, 2, 128), dtype=torch.bfloat16, device="cuda"))
    cut = to_llaisys(torch.from_numpy(cu))
    stream = torch.cuda.ExternalStream(L.context_stream())

    def step(i):  # one launch: the append fused into the gather
        L.Ops.paged_kv_append_gather(ko, vo, kp, vp, kn, vn, tab, ctx, cut)

    # Back-to-back launches over enough copies of the pools and outputs that
    # each call's bytes left the 256 MB MALL since their last use: the per-call
    # time is the kernel's cold-cache duration plus the dispatch gap, the
    # figure rocprofv3's average kernel duration reports for the same calls.
    per_copy = 2 * pool_k.numel() * 2 + 2 * T * 256 * 2
    copies = max(2, -(-(640 << 20) // per_copy))
    rot = [(to_llaisys(pool_k), to_llaisys(pool_v),
            to_llaisys(torch.zeros((T, 2, 128), dtype=torch.bfloat16, device="cuda")),
            to_llaisys(torch.zeros((T, 2, 128), dtype=torch.bfloat16, device="cuda"))) for _ in range(copies)]

    def step_rot(i):
        k_, v_, ko_, vo_ = rot[i % copies]
        L.Ops.paged_kv_append_gather(ko_, vo_, k_, v_, kn, vn, tab, ctx, cut)

    def step_two_calls(i):
        L.Ops.paged_kv_append(kp, vp, kn, vn, tab, ctx)
        L.Ops.paged_kv_gather(ko, vo, kp, vp, tab, cut)

    # The pool (64 MiB) and the output fit in the MALL: time each step after a
    # flush so the inputs come from HBM, and report the cache-warm rate beside it.
    kern_ms, wall_ms = time_steps(step_rot, stream, args.steps, args.warmup)
    single_ms, _ = time_steps_flushed(step, stream, args.steps, args.warmup)
    warm_ms, _ = time_steps(step, stream, args.steps, args.warmup)
    two_ms = two_warm_ms = None
    if not getattr(args, "ag_fused_only", False):
        two_ms, _ = time_steps_flushed(step_two_calls, stream, args.steps, args.warmup)
        two_warm_ms, _ = time_steps(step_two_calls, stream, args.steps, args.warmup)
    nbytes = 2 * T * 1024 + 2 * B * 1024
    gbs = nbytes / (kern_ms * 1e-3) / 1e9
    host = None
    if not getattr(args, "no_cpu", False):
        # The library's host path on the same data (CPU tensors, page format).
        hk, hv = host_tensor(pool_k, L.DataType.BF16), host_tensor(pool_v, L.DataType.BF16)
        hargs = [host_tensor(torch.zeros((T, 2, 128), dtype=torch.bfloat16), L.DataType.BF16) for _ in range(2)]
        hkn, hvn = host_tensor(kn_t, L.DataType.BF16), host_tensor(vn_t, L.DataType.BF16)
        htab, hctx = host_tensor(torch.from_numpy(table), L.DataType.I32), host_tensor(torch.from_numpy(lens), L.DataType.I32)
        hcu = host_tensor(torch.from_numpy(cu), L.DataType.I32)
        per, reps = time_host(lambda: L.Ops.paged_kv_append_gather(hargs[0], hargs[1], hk, hv, hkn, hvn, htab, hctx, hcu))
        host = {"ms": round(per * 1e3, 4), "GB/s": round((2 * T * 1024 + 2 * B * 1024) / per / 1e9, 2),
                "threads": host_cpus()[0], "reps": reps,
                "what": "llaisysPagedKVAppendGather on LLAISYS_DEVICE_CPU tensors, same inputs"}
    # The practical ceiling at this size: torch's contiguous device copy of the
    # same bytes (half read, half written), timed the same two ways.
    pairs = [(torch.empty(nbytes // 2, dtype=torch.uint8, device="cuda"),
              torch.empty(nbytes // 2, dtype=torch.uint8, device="cuda")) for _ in range(copies)]
    cstream = torch.cuda.current_stream()
    copy_ms, _ = time_steps(lambda i: pairs[i % copies][1].copy_(pairs[i % copies][0]), cstream, args.steps,
                            args.warmup)
    copy_warm_ms, _ = time_steps(lambda i: pairs[0][1].copy_(pairs[0][0]), cstream, args.steps, args.warmup)
    del pairs, rot
    return {
        "metric": "paged KV append+gather achieved HBM GB/s, 1 GPU", "value": round(gbs, 2), "unit": "GB/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(wall_ms, 5),
        "kernel_ms": round(kern_ms, 5), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16", "data": "synthetic",
        "config": {"workload": "BASELINE config 2: 32 seqs len U[1,2048], 4096-block pool, append 1 + gather",
                   "entry_point": "llaisysPagedKVAppendGather (append fused into the gather, one launch)",
                   "timing": f"HIP events around {args.steps} back-to-back calls rotating over {copies} copies of "
                             "the pools and outputs (each call's bytes cold in the MALL)"},
        "single_call_flushed": {"kernel_ms": round(single_ms, 5),
                                "GB/s": round(nbytes / (single_ms * 1e-3) / 1e9, 2),
                                "timing": "HIP events around one call after an untimed 512 MiB read (the launch "
                                          "and the event gaps are inside)"},
        "mall_resident": {"kernel_ms": round(warm_ms, 5), "GB/s": round(nbytes / (warm_ms * 1e-3) / 1e9, 2),
                          "timing": "back-to-back steps, inputs left in the MALL"},
        "two_calls": None if two_ms is None else {
            "entry_points": "llaisysPagedKVAppend then llaisysPagedKVGather",
            "kernel_ms": round(two_ms, 5), "GB/s": round(nbytes / (two_ms * 1e-3) / 1e9, 2),
            "mall_resident_kernel_ms": round(two_warm_ms, 5)},
        "cpu_host_path": host,
        "same_bytes_device_copy": {
            "what": "torch copy_ of nbytes/2 contiguous bytes (reads + writes = the step's bytes), timed as the "
                    "step: back-to-back over the same number of rotating copies",
            "kernel_ms": round(copy_ms, 5), "mall_resident_kernel_ms": round(copy_warm_ms, 5),
            "step_time_over_copy_time": round(kern_ms / copy_ms, 3)},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4),
                     "traffic": traffic_from_profiles("paged_kv_append_gather_config2"),
                     "algorithmic_bytes_per_launch": nbytes},
    }


def run_copy(args):
    """A plain device copy (512 MiB unless --copy-mib), to calibrate rocprof
    FETCH_SIZE/WRITE_SIZE and to time a copy of a workload's byte count."""
    import torch

    n = int(args.copy_mib * (1 << 20))
    a = torch.empty(n, dtype=torch.uint8, device="cuda")
    b = torch.empty_like(a)
    stream = torch.cuda.current_stream()
    kern_ms, wall_ms = time_steps(lambda i: b.copy_(a), stream, args.steps, args.warmup)
    flushed_ms, _ = time_steps_flushed(lambda i: b.copy_(a), stream, args.steps, args.warmup)
    return {"metric": "device copy GB/s (read+write)", "value": round(2 * n / (kern_ms * 1e-3) / 1e9, 2),
            "unit": "GB/s", "bytes_per_launch_read": n, "bytes_per_launch_written": n, "kernel_ms": kern_ms,
            "from_hbm": {"kernel_ms": flushed_ms, "GB/s": round(2 * n / (flushed_ms * 1e-3) / 1e9, 2),
                         "timing": "L2/MALL flushed by an untimed 512 MiB read before each step"}}


def _csvs(d, suffix):
    import glob

    return glob.glob(os.path.join(d, "**", "*" + suffix), recursive=True)


def _counter_means(d, last_steps=None):
    """Mean counter value per kernel name over a --pmc run's dispatches; with
    last_steps, over the dispatches of the run's last `last_steps` decode steps
    only (a step ends with the argmax finish kernel)."""
    import csv
    from collections import defaultdict

    rows = []
    for f in _csvs(d, "counter_collection.csv"):
        rows += [(int(r["Dispatch_Id"]), r["Kernel_Name"], float(r["Counter_Value"])) for r in csv.DictReader(open(f))]
    rows.sort()
    if last_steps:
        ends = [i for i, r in enumerate(rows) if "argmaxFinish" in r[1]]
        rows = rows[ends[-last_steps - 1] + 1: ends[-1] + 1]
    acc = defaultdict(list)
    for _, name, v in rows:
        acc[name].append(v)
    return {k: sum(v) / len(v) for k, v in acc.items()}


def _counter_scale(copy_dir, copy_bytes=512 << 20):
    """Bytes per counter unit (KiB) from a run of --workload copy over copy_bytes."""
    return copy_bytes / 1024 / max(v for k, v in _counter_means(copy_dir).items() if "copy" in k.lower())


def summarize(args):
    """Markdown + JSON summary of rocprofv3 output directories.

    --summarize STATS_DIR FETCH_DIR WRITE_DIR COPY_FETCH_DIR COPY_WRITE_DIR TAG
    STATS_DIR holds a --kernel-trace --stats run; the PMC dirs hold one-counter
    runs of the same workload (FETCH_SIZE, WRITE_SIZE, KiB per dispatch) and of
    --workload copy, whose known byte counts give the scale of each counter.
    """
    import csv
    import glob
    from collections import defaultdict

    stats_dir, fetch_dir, write_dir, cfetch_dir, cwrite_dir, tag = args.summarize

    def csvs(d, suffix):
        return glob.glob(os.path.join(d, "**", "*" + suffix), recursive=True)

    def counter_means(d):
        acc = defaultdict(list)
        for f in csvs(d, "counter_collection.csv"):
            for r in csv.DictReader(open(f)):
                acc[r["Kernel_Name"]].append(float(r["Counter_Value"]))
        return {k: sum(v) / len(v) for k, v in acc.items()}

    copy_bytes = 512 << 20
    fetch_scale = copy_bytes / 1024 / max(v for k, v in counter_means(cfetch_dir).items() if "copy" in k.lower())
    write_scale = copy_bytes / 1024 / max(v for k, v in counter_means(cwrite_dir).items() if "copy" in k.lower())
    fetch, write = counter_means(fetch_dir), counter_means(write_dir)
    def short(name):
        name = name.replace("(anonymous namespace)::", "").replace("void ", "")
        return name.split("(")[0]

    stats = []
    for f in csvs(stats_dir, "kernel_stats.csv"):
        stats += [r for r in csv.DictReader(open(f)) if "llaisys" in r["Name"]]
    lines = [f"# {tag}: rocprofv3 summary", "", "Commands (from the repo root, on the MI355X box):", "", "```"]
    lines += [f"rocprofv3 --kernel-trace --stats --output-format csv -d {stats_dir} -o run -- python3 bench.py {args.profiled_args}"]
    for c, d in (("FETCH_SIZE", fetch_dir), ("WRITE_SIZE", write_dir)):
        lines += [f"rocprofv3 --pmc {c} --output-format csv -d {d} -o run -- python3 bench.py {args.pmc_args}"]
    for c, d in (("FETCH_SIZE", cfetch_dir), ("WRITE_SIZE", cwrite_dir)):
        lines += [f"rocprofv3 --pmc {c} --output-format csv -d {d} -o run -- python3 bench.py --workload copy --steps 5 --warmup 2"]
    lines += [f"python3 bench.py --summarize {' '.join(args.summarize)} --profiled-args '{args.profiled_args}' "
              f"--pmc-args '{args.pmc_args}'", "```", ""]
    lines += ["## Kernel time (kernel trace)", "", "| kernel | calls | avg us | min us | max us |", "|---|---|---|---|---|"]
    total_us = 0.0
    for r in stats:
        name = short(r["Name"])
        avg = float(r["AverageNs"]) / 1e3
        total_us += avg
        lines.append(f"| `{name}` | {r['Calls']} | {avg:.2f} | {float(r['MinNs'])/1e3:.2f} | {float(r['MaxNs'])/1e3:.2f} |")
    lines += ["", f"Sum of the averages (one op call): {total_us:.2f} us", ""]
    lines += ["## HBM traffic per dispatch (PMC, scaled)", "",
              f"Counter scale from a plain {copy_bytes >> 20} MiB device copy: FETCH_SIZE x{fetch_scale:.3f}, "
              f"WRITE_SIZE x{write_scale:.3f} (copy reads and writes exactly {copy_bytes} bytes).", "",
              "| kernel | FETCH raw KiB | WRITE raw KiB | read MB | written MB |", "|---|---|---|---|---|"]
    total_bytes = 0.0
    for k in sorted(set(fetch) | set(write)):
        if "llaisys" not in k:
            continue
        fr, wr = fetch.get(k, 0.0), write.get(k, 0.0)
        rb, wb = fr * 1024 * fetch_scale, wr * 1024 * write_scale
        total_bytes += rb + wb
        lines.append(f"| `{short(k)}` | {fr:.1f} | {wr:.1f} | {rb/1e6:.2f} | {wb/1e6:.2f} |")
    lines += ["", f"HBM bytes per op call (all llaisys kernels): {total_bytes/1e6:.2f} MB", ""]
    print("\n".join(lines))
    out = {"tag": tag, "hbm_bytes_per_launch": int(total_bytes), "op_time_us_rocprof": round(total_us, 3),
           "fetch_scale": round(fetch_scale, 4), "write_scale": round(write_scale, 4)}
    outdir = Path(args.profiles_dir)
    outdir.mkdir(parents=True, exist_ok=True)
    (outdir / f"{tag}_traffic.json").write_text(json.dumps(out, indent=1) + "\n")
    (outdir / f"{tag}.md").write_text("\n".join(lines) + "\n")


def summarize_step(args):
    """Per-step kernel table of a --workload qwen2 kernel trace.

    --summarize-step TRACE_DIR TAG: reads the *kernel_trace.csv of
    `rocprofv3 --kernel-trace --output-format csv`, takes the dispatches of the
    last --steps decode steps (a step ends with the argmax finish kernel) and
    writes profiles/TAG.md: per kernel (name and grid), dispatches and time per
    step, and the step's span on the GPU clock.
    """
    import csv
    import glob
    from collections import defaultdict

    trace_dir, tag = args.summarize_step
    rows = []
    for f in glob.glob(os.path.join(trace_dir, "**", "*kernel_trace.csv"), recursive=True):
        for r in csv.DictReader(open(f)):
            grid = r.get("Grid_Size_X") or r.get("Grid_Size") or "?"
            rows.append((int(r["Start_Timestamp"]), int(r["End_Timestamp"]), r["Kernel_Name"], grid))
    rows.sort()
    ends = [i for i, r in enumerate(rows) if "argmaxFinish" in r[2]]
    k = args.steps
    sel = rows[ends[-k - 1] + 1: ends[-1] + 1]
    span_us = (sel[-1][1] - sel[0][0]) / 1e3 / k

    def short(name):
        import re

        if name.startswith("Cijk_"):  # library GEMM (Tensile kernels of hipBLASLt): keep the macro tile
            tile = re.search(r"MT\d+x\d+x\d+", name)
            return "hipBLASLt GEMM " + (tile.group(0) if tile else name[:40])
        name = name.replace("(anonymous namespace)::", "").replace("void ", "").replace("llaisys::kernels::", "")
        return name.split("(")[0]

    agg = defaultdict(lambda: [0, 0.0])
    for st, en, name, grid in sel:
        key = (short(name), grid)
        agg[key][0] += 1
        agg[key][1] += (en - st) / 1e3
    busy = sum(v[1] for v in agg.values()) / k
    pmc = args.step_pmc
    fetch = write = None
    if pmc:
        fs, ws = _counter_scale(pmc[2]), _counter_scale(pmc[3])
        fetch = {short(n): v * 1024 * fs for n, v in _counter_means(pmc[0], last_steps=2).items()}
        write = {short(n): v * 1024 * ws for n, v in _counter_means(pmc[1], last_steps=2).items()}
    cmds = [f"rocprofv3 --kernel-trace --output-format csv -d {trace_dir} -o run -- python3 bench.py --workload qwen2 "
            f"--steps {k} --warmup 2 --no-cpu"]
    if pmc:
        for c, d in (("FETCH_SIZE", pmc[0]), ("WRITE_SIZE", pmc[1])):
            cmds.append(f"rocprofv3 --pmc {c} --output-format csv -d {d} -o run -- python3 bench.py --workload qwen2 "
                        f"--steps 2 --warmup 1 --no-cpu")
        for c, d in (("FETCH_SIZE", pmc[2]), ("WRITE_SIZE", pmc[3])):
            cmds.append(f"rocprofv3 --pmc {c} --output-format csv -d {d} -o run -- python3 bench.py --workload copy "
                        f"--steps 5 --warmup 2")
    cmds.append(f"python3 bench.py --summarize-step {trace_dir} {tag} --steps {k}"
                + (f" --step-pmc {' '.join(pmc)}" if pmc else ""))
    lines = [f"# {tag}: one decode step of the Qwen2-1.5B-shape model (rocprofv3 kernel trace)", "",
             "Commands (from the repo root, on the MI355X box):", "", "```", *cmds, "```", "",
             f"Last {k} steps: GPU span {span_us:.1f} us per step, kernels busy {busy:.1f} us per step "
             f"({len(sel) / k:.0f} dispatches per step).", ""]
    if pmc:
        lines += [f"HBM bytes per dispatch: FETCH_SIZE / WRITE_SIZE (KiB) scaled by a plain 512 MiB device copy "
                  f"(x{fs:.3f} / x{ws:.3f}), averaged over the kernel's dispatches in the last two decode steps "
                  f"of the PMC runs.", "",
                  "| kernel | grid (work-items) | per step | us per step | avg us | read MB | written MB | TB/s |",
                  "|---|---|---|---|---|---|---|---|"]
    else:
        lines += ["| kernel | grid (work-items) | per step | us per step | avg us |", "|---|---|---|---|---|"]
    step_bytes = 0.0
    for (name, grid), (n, t) in sorted(agg.items(), key=lambda kv: -kv[1][1]):
        row = f"| `{name}` | {grid} | {n / k:.0f} | {t / k:.1f} | {t / n:.2f} |"
        if pmc:
            rb, wb = fetch.get(name, 0.0), write.get(name, 0.0)
            step_bytes += (rb + wb) * n / k
            row += f" {rb / 1e6:.2f} | {wb / 1e6:.2f} | {(rb + wb) / (t / n * 1e-6) / 1e12:.2f} |"
        lines.append(row)
    if pmc:
        lines += ["", f"HBM bytes per step (every kernel's per-dispatch bytes x its dispatches per step): "
                  f"{step_bytes / 1e9:.3f} GB"]
    print("\n".join(lines))
    outdir = Path(args.profiles_dir)
    outdir.mkdir(parents=True, exist_ok=True)
    (outdir / f"{tag}.md").write_text("\n".join(lines) + "\n")
    if pmc:
        (outdir / f"{tag}_traffic.json").write_text(json.dumps(
            {"tag": tag, "hbm_bytes_per_launch": int(step_bytes), "unit": "bytes per decode step",
             "step_span_us": round(span_us, 1)}, indent=1) + "\n")


def summarize_mfma(args):
    """MFMA use per kernel of a workload from three rocprofv3 runs.

    --summarize-mfma STATS_DIR UTIL_DIR MOPS_DIR [INSTS_DIR] TAG: STATS_DIR
    holds a --kernel-trace --stats run (average duration per kernel), UTIL_DIR
    a `--pmc MfmaUtil` run (SQ_VALU_MFMA_BUSY_CYCLES over GRBM_GUI_ACTIVE x
    SIMDs, percent), MOPS_DIR a `--pmc SQ_INSTS_VALU_MFMA_MOPS_BF16` run (bf16
    MFMA math ops / 512 per dispatch), INSTS_DIR (optional) a `--pmc
    SQ_INSTS_VALU SQ_INSTS_MFMA SQ_INSTS_VALU_TRANS_F32` run (instructions per
    dispatch; MFMA instructions are VALU instructions, so the non-MFMA VALU
    count is their difference). Writes profiles/TAG.md with, per kernel, the
    MFMA-busy percentage, the bf16 MFMA FLOP per dispatch and FLOP/s over the
    average duration against the 2.5 PFLOP/s dense bf16 peak, and the
    instruction mix.
    """
    import csv
    import glob
    from collections import defaultdict

    if len(args.summarize_mfma) not in (4, 5):
        raise SystemExit("--summarize-mfma takes STATS_DIR UTIL_DIR MOPS_DIR [INSTS_DIR] TAG")
    stats_dir, util_dir, mops_dir = args.summarize_mfma[:3]
    insts_dir = args.summarize_mfma[3] if len(args.summarize_mfma) == 5 else None
    tag = args.summarize_mfma[-1]

    def counters(d):
        acc = defaultdict(list)
        for f in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True):
            for r in csv.DictReader(open(f)):
                acc[(r["Kernel_Name"], r["Counter_Name"])].append(float(r["Counter_Value"]))
        return {k: sum(v) / len(v) for k, v in acc.items()}

    def short(name):
        return name.replace("(anonymous namespace)::", "").replace("void ", "").split("(")[0]

    durations = {}
    for f in glob.glob(os.path.join(stats_dir, "**", "*kernel_stats.csv"), recursive=True):
        for r in csv.DictReader(open(f)):
            durations[r["Name"]] = float(r["AverageNs"])
    util, mops = counters(util_dir), counters(mops_dir)
    insts = counters(insts_dir) if insts_dir else {}
    cmd = f"python3 bench.py {args.profiled_args}"
    lines = [f"# {tag}: MFMA use (rocprofv3 counters)", "", "Commands (from the repo root, on the MI355X box):", "",
             "```",
             f"rocprofv3 --kernel-trace --stats --output-format csv -d {stats_dir} -o run -- {cmd}",
             f"rocprofv3 --pmc MfmaUtil --output-format csv -d {util_dir} -o run -- {cmd}",
             f"rocprofv3 --pmc SQ_INSTS_VALU_MFMA_MOPS_BF16 --output-format csv -d {mops_dir} -o run -- {cmd}"]
    if insts_dir:
        lines.append(f"rocprofv3 --pmc SQ_INSTS_VALU SQ_INSTS_MFMA SQ_INSTS_VALU_TRANS_F32 --output-format csv "
                     f"-d {insts_dir} -o run -- {cmd}")
    lines += [f"python3 bench.py --summarize-mfma {' '.join(args.summarize_mfma)} --profiled-args '{args.profiled_args}'",
              "```", "",
              "| kernel | avg us | MFMA busy % | bf16 MFMA GFLOP / dispatch | TFLOP/s | % of 2.5 PFLOP/s |"
              + (" VALU instr. | MFMA instr. | non-MFMA VALU per MFMA | transcendental per MFMA |" if insts_dir else ""),
              "|---|---|---|---|---|---|" + ("---|---|---|---|" if insts_dir else "")]
    for name, ns in sorted(durations.items(), key=lambda kv: -kv[1]):
        if "llaisys" not in name:
            continue
        u = util.get((name, "MfmaUtil"))
        m = mops.get((name, "SQ_INSTS_VALU_MFMA_MOPS_BF16"))
        flop = m * 512 if m is not None else None
        tf = flop / ns / 1e3 if flop else None
        row = (f"| `{short(name)}` | {ns / 1e3:.2f} | {'' if u is None else f'{u:.1f}'} | "
               f"{'' if flop is None else f'{flop / 1e9:.2f}'} | {'' if tf is None else f'{tf:.1f}'} | "
               f"{'' if tf is None else f'{100 * tf / 2500:.1f}'} |")
        if insts_dir:
            v, mf, tr = (insts.get((name, c)) for c in ("SQ_INSTS_VALU", "SQ_INSTS_MFMA", "SQ_INSTS_VALU_TRANS_F32"))
            ratio = (v - mf) / mf if v is not None and mf else None
            trr = tr / mf if tr is not None and mf else None
            row += (f" {'' if v is None else f'{v:.0f}'} | {'' if mf is None else f'{mf:.0f}'} | "
                    f"{'' if ratio is None else f'{ratio:.2f}'} | {'' if trr is None else f'{trr:.2f}'} |")
        lines.append(row)
    print("\n".join(lines))
    outdir = Path(args.profiles_dir)
    outdir.mkdir(parents=True, exist_ok=True)
    (outdir / f"{tag}.md").write_text("\n".join(lines) + "\n")


def summarize_linear(args):
    """profiles/TAG.md from a kernel trace of `bench.py --workload linear`
    (llaisysLinear's kernels and torch.matmul's hipBLASLt kernels) and the
    JSON line the traced run printed."""
    import csv
    import re

    trace_dir, line_file, tag = args.summarize_linear
    stats = next(p for p in _csvs(trace_dir, "_kernel_stats.csv"))
    rows = list(csv.DictReader(open(stats)))
    line = next(json.loads(l) for l in open(line_file) if l.startswith('{"metric"'))
    out = [f"# {tag}: llaisysLinear (hand-written MFMA GEMM) vs torch.matmul (rocprofv3 kernel trace)", "",
           "Commands (from the repo root, on the MI355X box):", "", "```",
           f"rocprofv3 --kernel-trace --stats --output-format csv -d {trace_dir} -o run -- python3 bench.py "
           f"--workload linear > {line_file}",
           f"python3 bench.py --summarize-linear {trace_dir} {line_file} {tag}", "```", "",
           "`bench.py --workload linear` times `llaisysLinear` and then `torch.matmul` (hipBLASLt) on the same bf16",
           "inputs for M in {2048, 8192} x the four Qwen2-1.5B projections (qkv 2048x1536, o 1536x1536, gate-up",
           "17920x1536, down 1536x8960), 55 calls per shape each (5 warm-up + 50 timed).", "",
           "## Kernel time (kernel trace, all shapes together)", "",
           "| kernel | calls | avg us | share of trace |", "|---|---|---|---|"]
    for r in rows:
        name = r["Name"]
        if "gemmKernel" in name:
            short = "gemmKernel<bf16, " + name.split("ElemType)2, ")[1].split(">(")[0] + "> (this library)"
        elif "gemmReduceKernel" in name:
            short = "gemmReduceKernel (this library, split-K sum)"
        elif "Cijk" in name:
            mt = re.search(r"MT\d+x\d+x\d+", name)
            short = "hipBLASLt " + (mt.group(0) if mt else name[:30]) + " (torch)"
        else:
            short = name.split("(")[0][:70]
        out.append(f"| `{short}` | {r['Calls']} | {float(r['AverageNs']) / 1e3:.2f} | {float(r['Percentage']):.1f} % |")
    out += ["", "## The bench line of the traced run (HIP events)", "",
            f"Aggregate over the eight shapes: **{line['value']} TFLOP/s** for llaisysLinear, "
            f"{line['torch_matmul_TFLOP/s']} TFLOP/s for torch.matmul "
            f"({line['value'] / line['torch_matmul_TFLOP/s'] * 100:.0f} %); roofline frac {line['roofline']['frac']} "
            "of 2.5 PFLOP/s dense bf16. (The profiler slows the short torch calls more than ours.)", "",
            "| M x N x K | llaisysLinear us | TFLOP/s | torch us |", "|---|---|---|---|"]
    for r in line["shapes"]:
        out.append(f"| {r['M']} x {r['N']} x {r['K']} | {r['us']} | {r['TFLOP/s']} | {r['torch_us']} |")
    path = Path(args.profiles_dir) / f"{tag}.md"
    path.write_text("\n".join(out) + "\n")
    print(f"wrote {path}")


def summarize_ag_modes(args):
    """profiles/TAG.md: appendGatherKernel's dispatches of one `bench.py
    --workload append_gather --ag-fused-only` run, split by the bench's three
    timing modes (they run in this order, warm-up + timed calls each)."""
    import csv

    trace_dir, line_file, tag = args.summarize_ag_modes
    line = next(json.loads(l) for l in open(line_file) if l.startswith('{"metric"'))
    steps, warmup = line["steps"], line["warmup"]
    trace = next(p for p in _csvs(trace_dir, "_kernel_trace.csv"))
    ev = sorted((int(r["Start_Timestamp"]), int(r["End_Timestamp"])) for r in csv.DictReader(open(trace))
                if "appendGatherKernel" in r["Kernel_Name"])
    assert len(ev) == 3 * (steps + warmup), f"expected {3 * (steps + warmup)} dispatches, found {len(ev)}"
    modes = [f"back-to-back, rotating over copies of pools and outputs (the bench line's kernel_ms: "
             f"{line['kernel_ms'] * 1e3:.2f} us)",
             f"one call after an untimed 512 MiB read (single_call_flushed: "
             f"{line['single_call_flushed']['kernel_ms'] * 1e3:.2f} us by HIP events)",
             f"back-to-back on one copy, inputs MALL-resident (mall_resident: "
             f"{line['mall_resident']['kernel_ms'] * 1e3:.2f} us by HIP events)"]
    out = [f"# {tag}: kernel durations by timing mode (rocprofv3 kernel trace)", "",
           "Commands (from the repo root, on the MI355X box):", "", "```",
           f"rocprofv3 --kernel-trace --stats --output-format csv -d {trace_dir} -o run -- python3 bench.py "
           f"--workload append_gather --no-cpu --ag-fused-only > {line_file}",
           f"python3 bench.py --summarize-ag-modes {trace_dir} {line_file} {tag}", "```", "",
           f"`bench.py --workload append_gather --ag-fused-only` times `appendGatherKernel` three ways, {warmup} warm-up "
           f"+ {steps} calls each, in this order; the table splits the trace's {len(ev)} dispatches accordingly "
           "(warm-up calls left out).", "", "| timing mode | calls | avg us | min us | max us |", "|---|---|---|---|---|"]
    for i, mode in enumerate(modes):
        d = [(e - s) / 1e3 for s, e in ev[i * (steps + warmup) + warmup:(i + 1) * (steps + warmup)]]
        out.append(f"| {mode} | {len(d)} | {sum(d) / len(d):.2f} | {min(d):.2f} | {max(d):.2f} |")
    out += ["", f"Algorithmic bytes per call: {line['roofline']['algorithmic_bytes_per_launch'] / 1e6:.2f} MB. The rotated "
            "calls are the line's value: a steady state in which no copy's data is still in the MALL when it is "
            "reused. The flushed single call's HIP events also hold its launch and the event overhead."]
    path = Path(args.profiles_dir) / f"{tag}.md"
    path.write_text("\n".join(out) + "\n")
    print(f"wrote {path}")


def traffic_from_profiles(kernel_tag):
    """HBM bytes per launch measured by rocprofv3 PMC, if a summary is committed under profiles/."""
    f = ROOT / "profiles" / f"{kernel_tag}_traffic.json"
    if f.is_file():
        try:
            return json.loads(f.read_text()).get("hbm_bytes_per_launch")
        except Exception:
            return None
    return None


def main():
    args = parse()
    small = args.workload in ("qwen2", "serve")
    args.steps = args.steps if args.steps is not None else (64 if small else 200)
    args.warmup = args.warmup if args.warmup is not None else (4 if small else 20)
    if args.summarize:
        summarize(args)
        return
    if args.summarize_step:
        summarize_step(args)
        return
    if args.summarize_mfma:
        summarize_mfma(args)
        return
    if args.summarize_linear:
        summarize_linear(args)
        return
    if args.summarize_ag_modes:
        summarize_ag_modes(args)
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {args.gpus} is not supported: the KV-cache path "
              "is built and measured on a single MI355X", file=sys.stderr)
        sys.exit(2)
    # The library's host ops use this many threads (read once, at their first use).
    os.environ.setdefault("LLAISYS_CPU_THREADS", str(host_cpus()[0]))
    import torch

    assert torch.cuda.is_available(), "bench.py needs the MI355X"
    line = {"decode": run_decode, "mixed": run_mixed, "append_gather": run_append_gather, "copy": run_copy,
            "qwen2": run_qwen2, "serve": run_serve, "linear": run_linear}[args.workload](args)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
