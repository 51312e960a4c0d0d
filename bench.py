"""Benchmark of the MI355X FP8 paged-attention decode (one JSON line).

Metric: KV-read HBM GB/s (and % of the 8 TB/s MI355X peak) plus us per
decode step, on the Llama-3-8B-shaped configuration (batch 64, 32 query / 8
KV heads, head 128, 16-token pages, every context 4096, per-tensor fp8
scales) unless ``--config`` names another.

A step is one ``pa_decode_ps_launch`` call as the reference harness makes
it (recommended split count; the window route with preallocated partials;
the persistent route with the work list planned once):
one launch when workgroups own whole (sequence, kv head) pairs, else the
partition pass plus the LSE reduce.  Inputs are resident in HBM; the timed steps
rotate over several independent KV-cache copies whose total exceeds twice
the 256 MB Infinity Cache, so no step reads KV that the previous step left
in the cache.  ``value`` = attended K+V bytes / step time.

``roofline`` is measured live: the decode kernel (partition pass with the
in-kernel log-sum-exp merge, the only kernel of a step) is launched K times
through the C ABI with pre-marshalled arguments between HIP events on the
stream it runs on; algorithmic bytes per launch / average duration is
``achieved``.
``traffic`` (HBM bytes per launch from rocprofv3 FETCH_SIZE + WRITE_SIZE,
scaled by a copy-kernel calibration) is read from profiles/ when present.

``cpu_baseline``: the CPU oracle (restated torch reference, float32, per
sequence as tests/kernels/test_pa.py:302-330) timed on this host over a
bounded sample of the same workload's sequences.
"""

from __future__ import annotations

import argparse
import ctypes
import json
import math
import os
import platform
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

PEAK_HBM_GBPS = 8000.0
MALL_BYTES = 256 * 1024 * 1024
WARMUP_SECONDS = 0.2  # minimum untimed warm-up before each timed loop


def warm_up(run, min_steps: int) -> int:
    """Untimed run(i) calls: at least min_steps of them and at least
    WARMUP_SECONDS of GPU work (the clocks take a few milliseconds of load to
    settle, longer than a few short steps).  Returns the number of calls."""
    import torch

    i, t0 = 0, time.perf_counter()
    while i < min_steps or time.perf_counter() - t0 < WARMUP_SECONDS:
        run(i)
        i += 1
        if i % 8 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()
    return i


def parse_args():
    p = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=100)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--config", default="c2_llama8b",
                   help="c1_tiny|c2_llama8b|c3_ragged|c4_window|c5_mtp|all (decode), c3_ragged_p1024|c5_mtp_p1024 "
                        "(work-list route), c2_d64|c2_d256 (head sizes 64 and 256), "
                        "rope_decode_llama8b|rope_prefill_llama8b (KV-cache writer), "
                        "qknr_prefill_v4|qknr_decode_v4 (fused RMSNorm + GPT-J RoPE + fp8 quant), "
                        "mla_b32_c8192|mla_b128_c8192 (MLA fp8 decode)")
    p.add_argument("--seed", type=int, default=7)
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--cpu-seconds", type=float, default=10.0, help="CPU baseline sample budget")
    p.add_argument("--copies", type=int, default=0, help="KV-cache copies to rotate (0 = auto)")
    p.add_argument("--partitions", type=int, default=0, help="override max_context_partition_num (0 = heuristic)")
    p.add_argument("--no-metadata", action="store_true",
                   help="flat-page workloads: call pa_decode_ps_launch without the get_pa_metadata work list "
                        "(the launcher's balanced split)")
    p.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                   help="instead of decoding, run a plain device copy of MIB MiB (--steps times): the "
                        "reference point that scales rocprofv3 FETCH_SIZE / WRITE_SIZE to bytes")
    return p.parse_args()


def copy_calibration(mib: int, steps: int) -> None:
    import torch

    n = mib * 1024 * 1024
    src = torch.randint(0, 255, (n,), dtype=torch.uint8, device="cuda:0")
    dst = torch.empty_like(src)
    for _ in range(steps):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_bytes_read_per_launch": n, "bytes_written_per_launch": n, "launches": steps}))


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor()


def median_of_runs(items, run, budget_s: float, repeats: int = 3):
    """CPU baseline timing (median of ``repeats`` runs after one warm-up).

    The warm-up pass runs ``run(item)`` over ``items`` in order until a
    quarter of the budget is spent; the items it reached are the sample,
    which is then timed ``repeats`` more times.  Returns (sample, median
    seconds, every timed run's seconds)."""
    import statistics

    sample, spent = [], 0.0
    for it in items:
        t0 = time.perf_counter()
        run(it)
        spent += time.perf_counter() - t0
        sample.append(it)
        if spent >= budget_s / (repeats + 1):
            break
    runs = []
    for _ in range(repeats):
        t0 = time.perf_counter()
        for it in sample:
            run(it)
        runs.append(time.perf_counter() - t0)
    return sample, statistics.median(runs), runs


def host_desc() -> str:
    return (f"host {cpu_model()}, affinity {len(os.sched_getaffinity(0))} cpus, "
            f"os.cpu_count {os.cpu_count()}")


def cpu_baseline(case_gpu, cfg, budget_s: float) -> dict:
    """Time the CPU oracle on a bounded sample of the same workload's
    sequences (median of 3 runs after a warm-up); KV GB/s of the sample."""
    import torch

    from flydsl_amd import workloads
    from oracle import torch_ref

    ctx_all = case_gpu["context_lengths"].cpu().tolist()
    bs = cfg.block_size
    hkv = cfg.num_kv_heads
    ql = cfg.query_length
    kc = case_gpu["key_cache"]
    vc = case_gpu["value_cache"]
    per_token = case_gpu["key_scale"].dim() > 1

    def prepare(b):
        # compact copy of this sequence's pages (the oracle's input), not timed
        n = math.ceil(ctx_all[b] / bs)
        pages = case_gpu["block_tables"][b, :n].long()
        k = kc.index_select(0, pages).cpu()
        v = vc.index_select(0, pages).cpu()
        nbp = k.shape[0]
        if per_token:
            ks = case_gpu["key_scale"].index_select(0, pages).cpu().reshape(nbp, hkv, bs).permute(1, 0, 2).reshape(hkv, -1)
            vs = case_gpu["value_scale"].index_select(0, pages).cpu().reshape(nbp, hkv, bs).permute(1, 0, 2).reshape(hkv, -1)
        else:
            ks = case_gpu["key_scale"].cpu().expand(hkv, nbp * bs)
            vs = case_gpu["value_scale"].cpu().expand(hkv, nbp * bs)
        q = case_gpu["query"][b * ql : (b + 1) * ql].cpu()
        bt = torch.arange(nbp, dtype=torch.int32).reshape(1, -1)
        cl = torch.tensor([ctx_all[b]], dtype=torch.int32)
        ind = torch.tensor([0, ql], dtype=torch.int32)
        return b, (q, k, v, bt, cl, ind, ks, vs)

    def run(item):
        torch_ref.torch_mha_extend(*item[1], sliding_window=cfg.sliding_window,
                                   softmax_scale=case_gpu["softmax_scale"])

    sample, med, runs = median_of_runs((prepare(b) for b in range(cfg.batch)), run, budget_s)
    done_bytes = workloads.kv_bytes(cfg, [ctx_all[b] for b, _ in sample])
    return {
        "value": round(done_bytes / med / 1e9, 4),
        "unit": "GB/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": f"{len(sample)} of {cfg.batch} sequences of {cfg.name} through the float32 torch oracle "
        f"(oracle/torch_ref.py torch_mha_extend): median of {len(runs)} runs after a warm-up, "
        f"{med:.2f} s (runs {', '.join(f'{r:.2f}' for r in runs)}); {host_desc()}",
    }


def load_traffic(name: str):
    path = os.path.join(ROOT, "profiles", f"traffic_{name}.json")
    if not os.path.exists(path):
        return None
    try:
        with open(path) as f:
            return json.load(f).get("hbm_bytes_per_launch")
    except (OSError, ValueError):
        return None


KERNEL_OF_ENTRY = {
    "pa_fp8_decode_partition": "pa_fp8_partition_kernel",
    "pa_fp8_decode_balanced": "pa_fp8_stream_kernel (balanced split)",
    "pa_fp8_decode_worklist": "pa_fp8_bin_kernel (work list, one workgroup per bin)",
}


def flat_page_list(block_tables, ctx, block_size):
    """kv_page_indices / kv_indptr of the flat-page routes from a block
    table (each sequence's first ceil(ctx / bs) pages)."""
    import torch

    rows = [block_tables[b, : math.ceil(c / block_size)] for b, c in enumerate(ctx)]
    pages = torch.cat(rows).to(torch.int32).contiguous()
    counts = torch.tensor([0] + [r.numel() for r in rows], dtype=torch.int64)
    indptr = torch.cumsum(counts, 0).to(torch.int32).to(block_tables.device)
    return pages, indptr


def run_config(name: str, args) -> dict:
    import torch

    from flydsl_amd import get_pa_metadata, get_recommended_splits, pa_decode_ps_launch, prepare_pa_decode, workloads

    cfg = workloads.CONFIGS[name]
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    case = workloads.build_inputs(cfg, device=dev, seed=args.seed)
    ctx = case["context_lengths"].cpu().tolist()
    kv = workloads.kv_bytes(cfg, ctx)
    kv_sc = workloads.kv_bytes(cfg, ctx, include_scales=True)
    cache_bytes = case["key_cache"].numel() + case["value_cache"].numel()
    copies = args.copies or max(3, math.ceil(2 * MALL_BYTES / max(cache_bytes, 1)) + 1)
    caches = [(case["key_cache"], case["value_cache"], case["key_scale"], case["value_scale"])]
    for _ in range(copies - 1):
        caches.append(tuple(t.clone() for t in caches[0]))

    B, hkv, ql = cfg.batch, cfg.num_kv_heads, cfg.query_length
    eq = ql * cfg.gqa
    if cfg.sliding_window:
        P = get_recommended_splits(B, hkv, sliding_window=cfg.sliding_window, query_length=ql)
    else:
        P = get_recommended_splits(B, hkv, split_kv_blocks=max(1, 256 // cfg.block_size))
    if args.partitions:
        P = args.partitions
    es = torch.empty((B, hkv, P, eq), device=dev)
    ml = torch.empty_like(es)
    tmp = torch.empty((B, hkv, P, eq, cfg.head_size), device=dev, dtype=torch.bfloat16)
    out = torch.empty(case["query"].shape, device=dev, dtype=torch.bfloat16)

    # The call the reference's own harness makes for this route
    # (tests/kernels/test_pa.py:849-900): recommended split count, no
    # caller-side scratch (the window route preallocates its partials).
    sw_scratch = dict(exp_sums=es, max_logits=ml, temporary_output=tmp) if cfg.sliding_window else {}
    # Pages other than 16 / 64 tokens: the persistent route, with the work
    # list planned once for the batch (get_pa_metadata, as the harness calls
    # it before the timed launches, tests/kernels/test_pa.py:834-843).
    flat = cfg.block_size not in (16, 64)
    page_idx = indptr = None
    md = None
    if flat:
        page_idx, indptr = flat_page_list(case["block_tables"], ctx, cfg.block_size)
        if not args.no_metadata:
            md = get_pa_metadata(case["query"], case["key_cache"], case["context_lengths"], indptr,
                                 cfg.num_query_heads, hkv)
            sw_scratch = dict(metadata=md)
    bt_arg = None if flat else case["block_tables"]

    def step(i):
        k, v, ks, vs = caches[i % copies]
        return pa_decode_ps_launch(out, case["query"], k, v, case["context_lengths"], page_idx, indptr,
                                   case["softmax_scale"], ks, vs, sliding_window=cfg.sliding_window,
                                   block_tables=bt_arg, max_context_partition_num=P, **sw_scratch)

    route = step(0)
    warm = 1 + warm_up(step, args.warmup)
    stream = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record(stream)
    for i in range(args.steps):
        step(i)
    e1.record(stream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / args.steps

    # Live timing of the step's decode kernel (the dominant one; with the
    # in-kernel slot merge the only one), launched alone through its C-ABI
    # entry point with pre-marshalled arguments on this same stream.
    calls = []
    for k, v, ks, vs in caches:
        calls.append(prepare_pa_decode(out, case["query"], k, v, case["context_lengths"], page_idx, indptr,
                                       case["softmax_scale"], ks, vs, sliding_window=cfg.sliding_window,
                                       block_tables=bt_arg, max_context_partition_num=P, **sw_scratch))
    kernel_name, _ = calls[0].kernels()[0]
    decode = [c.kernels()[0][1] for c in calls]
    warm_up(lambda i: calls[i % copies].launch(), max(3, args.warmup))
    k0, k1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    k0.record(stream)
    for i in range(args.steps):
        rc = decode[i % copies]()
        if rc != 0:
            raise RuntimeError(f"{kernel_name} failed: {rc}")
    k1.record(stream)
    torch.cuda.synchronize()
    kern_ms = k0.elapsed_time(k1) / args.steps
    kernels_per_step = len(calls[0].kernels())

    achieved = kv / (kern_ms * 1e-3) / 1e9
    value = kv / (ms * 1e-3) / 1e9
    line = {
        "metric": "KV-read HBM GB/s (% of peak) + us/decode step, 8B-shaped fp8 paged decode",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": warm,
        "ms_per_step": round(ms, 5),
        "us_per_step": round(ms * 1e3, 2),
        "pct_of_peak": round(100.0 * value / PEAK_HBM_GBPS, 2),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp8",
        "data": "synthetic (seeded N(0,1) K/V quantised to fp8 e4m3fn, bf16 queries, permuted pages)",
        "config": {
            "workload": name,
            "batch": B,
            "query_length": ql,
            "num_query_heads": cfg.num_query_heads,
            "num_kv_heads": hkv,
            "head_size": cfg.head_size,
            "block_size": cfg.block_size,
            "sliding_window": cfg.sliding_window,
            "kv_scales": "per_token" if cfg.per_token else "per_tensor",
            "context": cfg.ctx,
            "sum_context": int(sum(ctx)),
            "num_partitions": P,
            "route": route,
            "work_list_bins": md["num_sm"] if md is not None else None,
            "kv_bytes_per_step": kv,
            "kv_plus_scale_bytes_per_step": kv_sc,
            "kv_copies_rotated": copies,
        },
        "roofline": {
            "bound": "hbm",
            "kernel": KERNEL_OF_ENTRY[kernel_name],
            "kernels_per_step": kernels_per_step,
            "achieved": round(achieved, 2),
            "peak": PEAK_HBM_GBPS,
            "unit": "GB/s",
            "frac": round(achieved / PEAK_HBM_GBPS, 4),
            "traffic": load_traffic(name),
            "kernel_us": round(kern_ms * 1e3, 2),
            "algorithmic_bytes": kv,
        },
    }
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(
            {k2: case[k2] for k2 in ("context_lengths", "block_tables", "key_cache", "value_cache", "key_scale",
                                     "value_scale", "query", "softmax_scale")}, cfg, args.cpu_seconds)
    del caches
    return line


def rope_cpu_baseline(case_gpu, cfg, budget_s: float) -> dict:
    """Time the writer's CPU oracle on a bounded sample of the workload's
    tokens (slices of growing size; median of 3 runs after a warm-up); GB/s
    of algorithmic bytes."""
    import torch

    from flydsl_amd import workloads
    from oracle import rope_cache as rc

    per_tok = workloads.rope_bytes(cfg) / cfg.num_tokens
    c = {k: (v.cpu() if isinstance(v, torch.Tensor) else v) for k, v in case_gpu.items()}
    kc = c["key_cache"].view(torch.uint8)
    vc = c["value_cache"].view(torch.uint8)

    def slices():
        done, n = 0, 8
        while done < cfg.num_tokens:
            m = min(n, cfg.num_tokens - done)
            yield slice(done, done + m)
            done += m
            n *= 2

    def run(sl):
        rc.rope_cache_ref(c["q"][sl], c["k"][sl], c["v"][sl], c["positions"][sl], c["cos"], c["sin"],
                          c["slot_mapping"][sl], kc, vc, block_size=cfg.block_size, layout=rc.ATOM_TRANS_V,
                          apply_scale=True, k_scale=float(c["k_scale"][0]), v_scale=float(c["v_scale"][0]),
                          inplace=True)

    sample, med, runs = median_of_runs(slices(), run, budget_s)
    done = sum(sl.stop - sl.start for sl in sample)
    return {
        "value": round(done * per_tok / med / 1e9, 4),
        "unit": "GB/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": f"{done} of {cfg.num_tokens} tokens of {cfg.name} through the torch oracle "
        f"(oracle/rope_cache.py rope_cache_ref, caches written in place): median of {len(runs)} runs after a "
        f"warm-up, {med:.2f} s (runs {', '.join(f'{r:.2f}' for r in runs)}); {host_desc()}",
    }


def run_rope_config(name: str, args) -> dict:
    """One KV-cache writer call per step (prepared, as a serving loop makes
    it); inputs rotate over copies so no step reads what the last one left
    in the Infinity Cache."""
    import torch

    from flydsl_amd import build_fused_rope_cache_module, workloads

    cfg = workloads.ROPE_CONFIGS[name]
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    case = workloads.build_rope_inputs(cfg, device=dev, seed=args.seed)
    algo = workloads.rope_bytes(cfg)
    in_bytes = sum(case[k].numel() * case[k].element_size() for k in ("q", "k", "v"))
    if args.copies:
        copies = args.copies
    elif in_bytes > 64 << 20:
        copies = max(2, math.ceil(2 * MALL_BYTES / in_bytes) + 1)
    else:
        copies = 1  # a decode batch's few MB stay cache-resident whatever the rotation
    ins = [(case["q"], case["k"], case["v"])]
    for _ in range(copies - 1):
        ins.append(tuple(t.clone() for t in ins[0]))
    q_out = torch.empty_like(case["q"])
    k_out = torch.empty_like(case["k"])
    launch = build_fused_rope_cache_module(head_dim=cfg.head_size, num_q_heads=cfg.num_q_heads,
                                           num_kv_heads=cfg.num_kv_heads, block_size=cfg.block_size,
                                           flash_layout=False, dtype_str="bf16", apply_scale=True)
    calls = [launch.prepare(q, k, v, case["positions"], case["cos"], case["sin"], case["slot_mapping"],
                            case["key_cache"], case["value_cache"], q_out, k_out, cfg.num_tokens, case["k_scale"],
                            case["v_scale"]) for q, k, v in ins]
    warm = warm_up(lambda i: calls[i % copies].launch(), max(3, args.warmup))
    stream = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record(stream)
    for i in range(args.steps):
        calls[i % copies].launch()
    e1.record(stream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / args.steps
    value = algo / (ms * 1e-3) / 1e9
    line = {
        "metric": "KV-cache writer HBM GB/s (% of peak) + us/call, NeoX RoPE + fp8 paged K/V write",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": warm,
        "ms_per_step": round(ms, 5),
        "us_per_step": round(ms * 1e3, 2),
        "pct_of_peak": round(100.0 * value / PEAK_HBM_GBPS, 2),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) bf16 Q/K/V, 10000-base rotary tables, permuted cache pages)",
        "config": {
            "workload": name,
            "num_tokens": cfg.num_tokens,
            "tokens_per_sequence": cfg.tokens_per_seq,
            "num_query_heads": cfg.num_q_heads,
            "num_kv_heads": cfg.num_kv_heads,
            "head_size": cfg.head_size,
            "block_size": cfg.block_size,
            "cache": "fp8 e4m3fn, K [NB, KH, D/16, bs, 16], V [NB, KH, bs/16, D, 16], per-tensor scales",
            "algorithmic_bytes_per_call": algo,
            "input_copies_rotated": copies,
        },
        "roofline": {
            "bound": "hbm",
            "kernel": "pa_rope_cache_kernel",
            "kernels_per_step": 1,
            "achieved": round(value, 2),
            "peak": PEAK_HBM_GBPS,
            "unit": "GB/s",
            "frac": round(value / PEAK_HBM_GBPS, 4),
            "traffic": load_traffic(name),
            "kernel_us": round(ms * 1e3, 2),
            "algorithmic_bytes": algo,
        },
    }
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = rope_cpu_baseline(case, cfg, args.cpu_seconds)
    return line


def qknr_cpu_baseline(case_gpu, cfg, budget_s: float) -> dict:
    """Time the fused RMSNorm + RoPE CPU oracle on a bounded sample of the
    workload's tokens (slices of growing size; median of 3 runs after a
    warm-up); GB/s of algorithmic bytes."""
    import torch

    from flydsl_amd import workloads
    from oracle import qk_norm_rope as qnr

    per_tok = workloads.qknr_bytes(cfg) / cfg.num_tokens
    c = {k: (v.cpu() if isinstance(v, torch.Tensor) else v) for k, v in case_gpu.items()}

    def slices():
        done, n = 0, 8
        while done < cfg.num_tokens:
            m = min(n, cfg.num_tokens - done)
            yield slice(done, done + m)
            done += m
            n *= 2

    def run(sl):
        qnr.qk_norm_rope_quant(c["q"][sl], c["kv"][sl], c["kv_weight"], c["cos_cache"], c["sin_cache"],
                               c["positions"][sl], num_q_heads=cfg.num_q_heads, head_dim=cfg.head_dim,
                               rope_head_dim=cfg.rope_head_dim, quant=cfg.quant, quant_group_size=cfg.group_size,
                               scale_dtype=cfg.scale_dtype)

    sample, med, runs = median_of_runs(slices(), run, budget_s)
    done = sum(sl.stop - sl.start for sl in sample)
    return {
        "value": round(done * per_tok / med / 1e9, 4),
        "unit": "GB/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": f"{done} of {cfg.num_tokens} tokens of {cfg.name} through the NumPy oracle "
        f"(oracle/qk_norm_rope.py qk_norm_rope_quant): median of {len(runs)} runs after a warm-up, "
        f"{med:.2f} s (runs {', '.join(f'{r:.2f}' for r in runs)}); {host_desc()}",
    }


def run_qknr_config(name: str, args) -> dict:
    """One fused RMSNorm + RoPE (+ fp8) call per step, prepared as a serving
    loop makes it; inputs rotate over copies so no step reads what the last
    one left in the Infinity Cache."""
    import torch

    from flydsl_amd import workloads
    from flydsl_amd.qk_norm_rope import FP8_DTYPE, compile_flydsl_qk_norm_rope_quant

    cfg = workloads.QKNR_CONFIGS[name]
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    case = workloads.build_qknr_inputs(cfg, device=dev, seed=args.seed)
    algo = workloads.qknr_bytes(cfg)
    T, H, D = cfg.num_tokens, cfg.num_q_heads, cfg.head_dim
    in_bytes = sum(case[k].numel() * case[k].element_size() for k in ("q", "kv"))
    if args.copies:
        copies = args.copies
    elif in_bytes > 64 << 20:
        copies = max(2, math.ceil(2 * MALL_BYTES / in_bytes) + 1)
    else:
        copies = 1
    ins = [(case["q"], case["kv"])]
    for _ in range(copies - 1):
        ins.append(tuple(t.clone() for t in ins[0]))
    odt = FP8_DTYPE if cfg.quant else torch.bfloat16
    q_out = torch.empty((T, H, D), dtype=odt, device=dev)
    kv_out = torch.empty((T, D), dtype=odt, device=dev)
    ng = D // cfg.group_size
    sdt = torch.float32 if cfg.scale_dtype == "fp32" else torch.uint8
    q_scale = torch.empty((T, H, ng), dtype=sdt, device=dev)
    kv_scale = torch.empty((T, ng), dtype=sdt, device=dev)
    launcher = compile_flydsl_qk_norm_rope_quant(num_q_heads=H, head_dim=D, rope_head_dim=cfg.rope_head_dim,
                                                 quant=cfg.quant, group_size=cfg.group_size,
                                                 scale_dtype=cfg.scale_dtype, q_weighted=False)
    calls = [launcher.prepare(q.view(T, H, D), kv, case["kv_weight"], case["kv_weight"], case["cos_cache"],
                              case["sin_cache"], case["positions"], q_out, kv_out, q_scale, kv_scale, kv.stride(0), T)
             for q, kv in ins]
    warm = warm_up(lambda i: calls[i % copies].launch(), max(3, args.warmup))
    stream = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record(stream)
    for i in range(args.steps):
        calls[i % copies].launch()
    e1.record(stream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / args.steps
    value = algo / (ms * 1e-3) / 1e9
    line = {
        "metric": "fused RMSNorm + GPT-J RoPE + fp8 quant HBM GB/s (% of peak) + us/call",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": warm,
        "ms_per_step": round(ms, 5),
        "us_per_step": round(ms * 1e3, 2),
        "pct_of_peak": round(100.0 * value / PEAK_HBM_GBPS, 2),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) bf16 Q/KV, 10000-base GPT-J rotary tables, random positions)",
        "config": {
            "workload": name,
            "num_tokens": T,
            "num_query_heads": H,
            "head_dim": D,
            "rope_head_dim": cfg.rope_head_dim,
            "quant": f"fp8 e4m3fn, {cfg.scale_dtype} scale per {cfg.group_size}" if cfg.quant else "bf16",
            "q_weighted": False,
            "algorithmic_bytes_per_call": algo,
            "input_copies_rotated": copies,
        },
        "roofline": {
            "bound": "hbm",
            "kernel": "pa_qk_norm_rope_kernel",
            "kernels_per_step": 1,
            "achieved": round(value, 2),
            "peak": PEAK_HBM_GBPS,
            "unit": "GB/s",
            "frac": round(value / PEAK_HBM_GBPS, 4),
            "traffic": load_traffic(name),
            "kernel_us": round(ms * 1e3, 2),
            "algorithmic_bytes": algo,
        },
    }
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = qknr_cpu_baseline(case, cfg, args.cpu_seconds)
    return line


def mla_cpu_baseline(case_gpu, cfg, budget_s: float) -> dict:
    """Time the MLA CPU oracle (float64 NumPy attention) on a bounded sample
    of the workload's sequences (median of 3 runs after a warm-up); GB/s of
    algorithmic bytes."""
    import torch

    from flydsl_amd import workloads
    from oracle import mla as om

    per_seq = workloads.mla_bytes(cfg) / cfg.batch
    q = om.fp8_to_f64(case_gpu["q"])
    idx = case_gpu["kv_indices"].cpu().numpy()

    def prepare(s):
        rows = idx[s * cfg.context:(s + 1) * cfg.context]
        kv = om.fp8_to_f64(case_gpu["kvs"][0][torch.from_numpy(rows).long().to(case_gpu["q"].device)].view(-1, 576))
        return s, kv

    def run(item):
        s, kv = item
        om.attend(q[s:s + 1], kv, 1.0 / 24.0)

    sample, med, runs = median_of_runs((prepare(s) for s in range(cfg.batch)), run, budget_s)
    return {
        "value": round(len(sample) * per_seq / med / 1e9, 4),
        "unit": "GB/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": f"{len(sample)} of {cfg.batch} sequences of {cfg.name} through the float64 NumPy oracle "
        f"(oracle/mla.py attend): median of {len(runs)} runs after a warm-up, {med:.2f} s "
        f"(runs {', '.join(f'{r:.2f}' for r in runs)}); {host_desc()}",
    }


def run_mla_config(name: str, args) -> dict:
    """One MLA decode step = the decode launch + the log-sum-exp reduce of the
    rows it cut, on a work list planned once (as a serving loop plans it per
    batch shape).  KV buffers rotate over copies so no step reads what the
    last one left in the Infinity Cache."""
    import torch

    from flydsl_amd import workloads
    from flydsl_amd.mla_decode import (flydsl_mla_fwd_decode, get_mla_metadata_info_v1, get_mla_metadata_v1,
                                       mla_reduce_v1)

    cfg = workloads.MLA_CONFIGS[name]
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    kv_bytes = cfg.batch * cfg.context * 576
    copies = args.copies or (max(2, math.ceil(2 * MALL_BYTES / kv_bytes) + 1) if kv_bytes > 64 << 20 else 1)
    case = workloads.build_mla_inputs(cfg, dev, seed=args.seed, copies=copies)
    fp8 = torch.float8_e4m3fn
    sizes = get_mla_metadata_info_v1(cfg.batch, 1, 128, fp8, fp8)
    meta, wp, wi, ri, rf, rp = [torch.empty(sz, dtype=t, device=dev) for sz, t in sizes]
    get_mla_metadata_v1(case["qo_indptr"].to(dev), case["kv_indptr"].to(dev), case["kv_last_page_lens"].to(dev),
                        128, 1, False, meta, wi, wp, ri, rf, rp)
    out = torch.empty(cfg.batch, 128, 512, dtype=torch.bfloat16, device=dev)
    so = torch.empty(rp.size(0), 1, 128, 512, dtype=torch.float32, device=dev)
    sl = torch.empty(rp.size(0), 1, 128, 1, dtype=torch.float32, device=dev)
    sm = 1.0 / math.sqrt(576.0)

    def decode(i):
        flydsl_mla_fwd_decode(case["q"], case["kvs"][i % copies], case["kv_indices"], wp, wi, out, so, sl, sm)

    def step(i):
        decode(i)
        mla_reduce_v1(so, sl, ri, rf, rp, 1, out)

    warm = warm_up(step, max(3, args.warmup))
    stream = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record(stream)
    for i in range(args.steps):
        step(i)
    e1.record(stream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / args.steps
    # the decode kernel alone, same stream, same rotation
    e0.record(stream)
    for i in range(args.steps):
        decode(i)
    e1.record(stream)
    torch.cuda.synchronize()
    kms = e0.elapsed_time(e1) / args.steps
    algo = workloads.mla_bytes(cfg)
    flops = workloads.mla_flops(cfg)
    value = algo / (ms * 1e-3) / 1e9
    kval = algo / (kms * 1e-3) / 1e9
    mh = meta.cpu().tolist()
    line = {
        "metric": "MLA fp8 decode HBM GB/s (KV + Q + out bytes per step) + us/step",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": warm,
        "ms_per_step": round(ms, 5),
        "us_per_step": round(ms * 1e3, 2),
        "pct_of_peak": round(100.0 * value / PEAK_HBM_GBPS, 2),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp8 e4m3fn (q, kv), f32 accumulate, bf16 out",
        "data": "synthetic (seeded N(0,1) q and latent KV rows cast to fp8, pages in random order)",
        "config": {
            "workload": name,
            "batch": cfg.batch,
            "context": cfg.context,
            "num_heads": 128,
            "qk_head_dim": 576,
            "v_head_dim": 512,
            "page_size": 1,
            "works": mh[0], "cut_rows": mh[1], "partial_rows": mh[2], "workers": mh[3],
            "algorithmic_bytes_per_step": algo,
            "algorithmic_flops_per_step": flops,
            "decode_tflops": round(flops / (kms * 1e-3) / 1e12, 1),
            "kv_copies_rotated": copies,
        },
        "roofline": {
            "bound": "hbm",
            "kernel": "mla_fp8_decode_kernel",
            "kernels_per_step": 2,
            "achieved": round(kval, 2),
            "peak": PEAK_HBM_GBPS,
            "unit": "GB/s",
            "frac": round(kval / PEAK_HBM_GBPS, 4),
            "traffic": load_traffic(name),
            "kernel_us": round(kms * 1e3, 2),
            "algorithmic_bytes": algo,
            "mfma_frac_fp8": round(flops / (kms * 1e-3) / 5.0e15, 4),
        },
    }
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = mla_cpu_baseline(case, cfg, args.cpu_seconds)
    return line


def main():
    args = parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print(json.dumps({"error": "this build runs on one GPU; --gpus N > 1 is not supported "
                                   "(the decode path shards by sequence / kv head with no communication)"}))
        sys.exit(2)
    if args.copy_calibration:
        copy_calibration(args.copy_calibration, args.steps)
        return
    names = ["c2_llama8b", "c3_ragged", "c4_window", "c5_mtp"] if args.config == "all" else [args.config]
    for n in names:
        if n.startswith("rope_"):
            line = run_rope_config(n, args)
        elif n.startswith("qknr_"):
            line = run_qknr_config(n, args)
        elif n.startswith("mla_"):
            line = run_mla_config(n, args)
        else:
            line = run_config(n, args)
        print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
