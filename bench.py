#!/usr/bin/env python3
"""Decode microbenchmark of the KV path on one MI355X.

Workload: batch 32, 16 query / 4 KV heads, head_dim 128, bf16; per-row cache lengths drawn
uniformly from [512, 8192] (seed 0); K/V cache, q and new k/v are N(0, 1). One step appends one
token per row at its own position and runs single-token attention over the whole cache
(``flash_attn_with_kvcache``), then advances the positions (``KVCache.advance``; folded into the
operator's last kernel with ``advance=1`` unless --separate-advance). Inputs are resident in HBM
before timing starts; the K timed steps run as one HIP graph replay.

Prints one JSON line: tokens/s (32 tokens per step), the roofline of the decode attention
(algorithmic bytes over its event-timed duration against 8 TB/s), and the reference's CPU
fallback timed on this host's cores on the same workload. Unless --decode-only, the line also
carries a `subsystems` object with the other workloads of the path, each with its own roofline
and CPU baseline: the chunked prefill (attention MFMA utilisation and append GB/s), the
mixed-window stack's decode step and the replication of a prompt cache into 64 rows (the same
measurements as --workload prefill / mixed / replicate, with fixed step counts).

    python bench.py [--gpus 1] [--steps 200] [--warmup 20] [--no-cpu-baseline] [--decode-only]

The roofline figure times the decode call alone, ROOF_LAUNCHES launches at the drawn lengths
(seed 0), whatever --steps and --warmup are, so that its bytes -- and the HBM traffic the
committed counter profile measured for the same launches -- do not depend on them. Two modes
turn rocprofv3 output into the committed summaries (no GPU needed):

    python bench.py --summarize-traffic FETCH.csv WRITE.csv COPY_FETCH.csv COPY_WRITE.csv
    python bench.py --summarize-trace KERNEL_TRACE.csv [--launches N]
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

METRIC = "decode tok/s at B=32 ctx 8k GQA16/4 hd128; KV path HBM GB/s as % of peak"
B, H, H_KV, D = 32, 16, 4, 128
L_MIN, L_MAX = 512, 8192
COPY_BYTES = 1 << 30
TRAFFIC_FILE = "profiles/decode_b32_gqa16x4_hd128_ctx8k_traffic.md"
ROOF_LAUNCHES = 200  # decode calls in the roofline loop
ROOF_WARMUP_S = 0.1  # seconds of untimed calls before them
DECODE_KERNELS = ("decode_fused_kernel", "decode_merge_kernel")


def peaks():
    """(HBM bytes/s, dense bf16 FLOP/s, how they were found) of GPU 0: the reference's MI355
    denominators (modelcore/runtime.py:162, :200), found by device name or gfx950 architecture."""
    from modelcore_amd import runtime
    bw, fl, how = runtime.device_peaks(0)
    if bw == float("inf"):
        raise RuntimeError(f"no peak figures for this GPU ({how}): the roofline needs them")
    return bw, fl, how


def host_cores():
    """Every core this process may run on (the CPU baseline's thread count, reported with it)."""
    return len(os.sched_getaffinity(0))


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def parse_args():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--decode-only", action="store_true",
                    help="default workload: time the decode microbench only, without the "
                         "prefill, mixed-window and replication objects")
    ap.add_argument("--eager", action="store_true",
                    help="decode and mixed workloads: time eager launches instead of a graph "
                         "(the counter runs)")
    ap.add_argument("--library-gemm", action="store_true",
                    help="sample workload: run the decode projections through F.linear (the "
                         "library GEMM) instead of mcamd_linear_bf16")
    ap.add_argument("--separate-residual", action="store_true",
                    help="sample workload: run each residual add and RMS-norm as torch's separate "
                         "ops instead of one mcamd_residual_rmsnorm launch")
    ap.add_argument("--workload", choices=("decode", "prefill", "replicate", "mixed", "sample"),
                    default="decode",
                    help="decode: the decode microbench (default, the headline metric); prefill: "
                         "chunked prefill of 8 x 16384 tokens in chunks of 512, 32q/8kv heads; "
                         "replicate: one 2048-token, 32-layer prompt cache copied into 64 rows; "
                         "mixed: the KV path of one decode step of a 24-layer mixed-window, "
                         "KV-sharing stack at B=16, context 4096; sample: a 32-layer 4096-wide "
                         "model prefills one 2048-token prompt, replicates it to 64 rows and "
                         "samples 512 tokens per row at temperature 1")
    ap.add_argument("--separate-advance", action="store_true",
                    help="decode and mixed workloads: advance the positions with KVCache.advance "
                         "after the step's last operator call (one more launch) instead of inside "
                         "that call (flash_attn_with_kvcache(..., advance=1))")
    ap.add_argument("--no-shared-prefix", action="store_true",
                    help="sample workload: let every row's attention read its own copy of the "
                         "replicated prompt's K/V instead of row 0's (KVCache.shared_prefix = 0)")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="run only a plain device copy of COPY_BYTES, ten times (the known-size "
                         "kernel that scales the FETCH_SIZE / WRITE_SIZE counters)")
    ap.add_argument("--summarize-traffic", nargs=4, metavar="CSV",
                    help="print the traffic summary of the decode call from rocprofv3 --pmc "
                         "FETCH_SIZE and WRITE_SIZE runs of `bench.py --eager --no-cpu-baseline` and "
                         "of `bench.py --calibrate-copy` (counter_collection.csv files)")
    ap.add_argument("--summarize-counters", nargs=7,
                    metavar=("WORKLOAD", "FETCH", "WRITE", "COPY_FETCH", "COPY_WRITE", "UNITS",
                             "ALGO_BYTES"),
                    help="print the traffic summary of workload prefill, mixed or replicate from "
                         "rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE runs of it (its last UNITS "
                         "passes, steps or launches, ALGO_BYTES algorithmic bytes each) and of "
                         "bench.py --calibrate-copy")
    ap.add_argument("--summarize-pmc", nargs="+", metavar="CSV",
                    help="print per-dispatch counter means from rocprofv3 --pmc CSVs over the "
                         "last --launches dispatches of the kernel named by --kernel")
    ap.add_argument("--kernel", default="prefill_mfma_kernel",
                    help="kernel name (substring) for --summarize-pmc")
    ap.add_argument("--summarize-trace", metavar="CSV",
                    help="print the mean duration of the decode call's kernels over the last "
                         "--launches dispatches of a rocprofv3 kernel_trace.csv")
    ap.add_argument("--launches", type=int, default=ROOF_LAUNCHES)
    return ap.parse_args()


def drawn_lengths(seed=0):
    """The decode microbench's per-row cache lengths: U[512, 8192], drawn first from the seeded
    CPU generator (the bench draws its caches and tokens from the same generator after them)."""
    import torch
    g = torch.Generator().manual_seed(seed)
    return torch.randint(L_MIN, L_MAX + 1, (B,), generator=g, dtype=torch.int32)


def roofline_bytes(seed=0):
    """Algorithmic bytes of one decode call of the roofline loop (append + attention of every row
    at its drawn length)."""
    from modelcore_amd import stats
    return stats.decode_step_bytes(drawn_lengths(seed).tolist(), H, H_KV, D, 2, append=True)


def measured_traffic(bytes_now):
    """(HBM bytes per launch of the decode call, where the figure comes from) from the committed
    counter profile: its own figure when it was measured for launches of these algorithmic bytes,
    else its traffic/bytes ratio applied to these bytes (said so); (None, reason) without one."""
    import re
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), TRAFFIC_FILE)
    try:
        with open(path) as f:
            text = f.read()
    except OSError:
        return None, f"{TRAFFIC_FILE} missing"
    t = re.search(r"^traffic_bytes_per_launch:\s*(\d+)", text, re.M)
    a = re.search(r"^algorithmic_bytes_per_launch:\s*(\d+)", text, re.M)
    if not (t and a):
        return None, f"{TRAFFIC_FILE} holds no per-launch figures"
    traffic, algo = int(t.group(1)), int(a.group(1))
    how = (f"{TRAFFIC_FILE}: rocprofv3 FETCH_SIZE x2.0 + WRITE_SIZE (copy-calibrated), mean over the "
           f"{ROOF_LAUNCHES} launches of this loop")
    if algo == bytes_now:
        return traffic, how + ", same positions"
    return round(traffic / algo * bytes_now), how + (f", measured at {algo} algorithmic bytes and "
                                                     f"scaled by its ratio {traffic / algo:.4f}")


APPEND_TRAFFIC_FILE = "profiles/kv_append_b8_c512_hkv8_hd128_traffic.md"


def append_traffic(bytes_now):
    """(HBM bytes per append launch, where the figure comes from) from the committed counter
    profile of the prefill workload's append, when it was measured for launches of these
    algorithmic bytes; (None, reason) otherwise."""
    import re
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), APPEND_TRAFFIC_FILE)
    try:
        with open(path) as f:
            text = f.read()
    except OSError:
        return None, f"{APPEND_TRAFFIC_FILE} missing"
    t = re.search(r"^append_traffic_bytes_per_launch:\s*(\d+)", text, re.M)
    a = re.search(r"^append_algorithmic_bytes_per_launch:\s*(\d+)", text, re.M)
    if not (t and a) or int(a.group(1)) != bytes_now:
        return None, f"{APPEND_TRAFFIC_FILE} holds no figure for launches of {bytes_now} bytes"
    return int(t.group(1)), (f"{APPEND_TRAFFIC_FILE}: rocprofv3 FETCH_SIZE x2.0 + WRITE_SIZE "
                             f"(copy-calibrated), mean over 128 launches of this workload")


def _counter_rows(path):
    import csv
    with open(path) as f:
        return list(csv.DictReader(f))


def summarize_traffic(fetch_csv, write_csv, copy_fetch_csv, copy_write_csv):
    """Markdown summary of the decode call's HBM traffic (the roofline loop's launches)."""
    import statistics as st

    def per_kernel(rows, counter, names, last):
        out = {}
        for name in names:
            vals = [float(r["Counter_Value"]) for r in rows
                    if r["Counter_Name"] == counter and name in r["Kernel_Name"]]
            out[name] = vals[-last:]
        return out

    def copy_scale(rows, counter):
        vals = [float(r["Counter_Value"]) for r in rows
                if r["Counter_Name"] == counter and "copyBuffer" in r["Kernel_Name"]]
        kib = st.median(vals)
        return kib, COPY_BYTES / 1024 / kib

    cf_kib, cf_scale = copy_scale(_counter_rows(copy_fetch_csv), "FETCH_SIZE")
    cw_kib, cw_scale = copy_scale(_counter_rows(copy_write_csv), "WRITE_SIZE")
    fetch = per_kernel(_counter_rows(fetch_csv), "FETCH_SIZE", DECODE_KERNELS, ROOF_LAUNCHES)
    write = per_kernel(_counter_rows(write_csv), "WRITE_SIZE", DECODE_KERNELS, ROOF_LAUNCHES)
    algo = roofline_bytes()
    lines = ["| kernel | launches | FETCH_SIZE (KiB, mean) | x scale | WRITE_SIZE (KiB, mean) | x scale |",
             "|---|---|---|---|---|---|"]
    total = 0.0
    for name in DECODE_KERNELS:
        fk, wk = st.mean(fetch[name]), st.mean(write[name])
        total += fk * cf_scale * 1024 + wk * cw_scale * 1024
        lines.append(f"| {name} | {len(fetch[name])} | {fk:.2f} | {fk * cf_scale:.2f} | {wk:.2f} | "
                     f"{wk * cw_scale:.2f} |")
    print(f"Calibration (plain device copy of {COPY_BYTES >> 20} MiB, `__amd_rocclr_copyBuffer`): "
          f"FETCH_SIZE reads {cf_kib:.1f} KiB per launch (scale {cf_scale:.3f}), WRITE_SIZE "
          f"{cw_kib:.1f} KiB (scale {cw_scale:.3f}).\n")
    print("\n".join(lines))
    print(f"\nPer launch of the decode call: {round(total)} bytes of HBM traffic against {algo} "
          f"algorithmic bytes: {total / algo:.3f}x.\n")
    print(f"traffic_bytes_per_launch: {round(total)}")
    print(f"algorithmic_bytes_per_launch: {algo}")


def summarize_trace(trace_csv, launches):
    """Mean durations (us) of the decode call's kernels over their last `launches` dispatches."""
    import statistics as st
    rows = _counter_rows(trace_csv)
    rows.sort(key=lambda r: int(r["Start_Timestamp"]))
    total = 0.0
    for name in DECODE_KERNELS:
        d = [(int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3 for r in rows
             if name in r["Kernel_Name"]][-launches:]
        total += st.mean(d)
        print(f"| {name} | {len(d)} | {st.mean(d):.2f} | {st.median(d):.2f} | {min(d):.2f} | "
              f"{max(d):.2f} |")
    algo = roofline_bytes()
    print(f"\nsum of means: {total:.2f} us per call; {algo} algorithmic bytes -> "
          f"{algo / total / 1e3:.1f} GB/s")


def calibrate_copy():
    """A plain device-to-device copy of COPY_BYTES, ten times: what FETCH_SIZE and WRITE_SIZE
    read for a kernel that moves a known number of bytes."""
    import torch
    dev = torch.device("cuda", 0)
    src = torch.ones(COPY_BYTES // 2, dtype=torch.bfloat16, device=dev)
    dst = torch.empty_like(src)
    for _ in range(10):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"calibration": "device copy", "bytes_read": COPY_BYTES,
                      "bytes_written": COPY_BYTES, "launches": 10}), flush=True)


PF_B, PF_T, PF_C, PF_H, PF_HKV = 8, 16384, 512, 32, 8

# Committed counter summaries of the other workloads: kernels summed, the unit the traffic is
# given per, and how many of those units the counter run's last dispatches cover.
TRAFFIC_PROFILES = {
    "prefill": dict(file="profiles/prefill_b8_t16384_c512_gqa32x8_hd128_traffic.md",
                    kernels=("prefill_mfma_kernel",), unit="pass", dispatches_per_unit=32),
    "mixed": dict(file="profiles/mixed_l24_b16_ctx4096_gqa12x4_hd128_traffic.md",
                  kernels=("decode_fused_kernel", "decode_merge_kernel"), unit="step",
                  dispatches_per_unit=48),
    "replicate": dict(file="profiles/replicate_s32_p2048_r64_hkv8_hd128_traffic.md",
                      kernels=("kv_replicate_kernel",), unit="launch", dispatches_per_unit=1),
}


def profile_traffic(name, bytes_now):
    """(HBM bytes per unit of workload `name`, where the figure comes from) from its committed
    counter summary, scaled by the summary's traffic/bytes ratio when it was measured at other
    algorithmic bytes (said so); (None, reason) without one."""
    import re
    spec = TRAFFIC_PROFILES[name]
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), spec["file"])
    try:
        with open(path) as f:
            text = f.read()
    except OSError:
        return None, f"{spec['file']} missing"
    t = re.search(r"^traffic_bytes_per_unit:\s*(\d+)", text, re.M)
    a = re.search(r"^algorithmic_bytes_per_unit:\s*(\d+)", text, re.M)
    if not (t and a):
        return None, f"{spec['file']} holds no per-{spec['unit']} figures"
    traffic, algo = int(t.group(1)), int(a.group(1))
    how = (f"{spec['file']}: rocprofv3 FETCH_SIZE x2.0 + WRITE_SIZE (copy-calibrated) of "
           f"{' + '.join(spec['kernels'])}, per {spec['unit']}")
    if algo == bytes_now:
        return traffic, how
    return round(traffic / algo * bytes_now), how + (f", measured at {algo} algorithmic bytes and "
                                                     f"scaled by its ratio {traffic / algo:.4f}")


def summarize_counters(name, fetch_csv, write_csv, copy_fetch_csv, copy_write_csv, units,
                       algo_bytes):
    """Markdown traffic summary of workload `name` from rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE
    runs (the last `units` units' dispatches of its kernels) and of the plain copy; ends with the
    two lines profile_traffic reads."""
    import statistics as st
    spec = TRAFFIC_PROFILES[name]

    def copy_scale(rows, counter):
        vals = [float(r["Counter_Value"]) for r in rows
                if r["Counter_Name"] == counter and "copyBuffer" in r["Kernel_Name"]]
        kib = st.median(vals)
        return kib, COPY_BYTES / 1024 / kib

    def kernel_sum(rows, counter):
        vals = [(int(r["Dispatch_Id"]), float(r["Counter_Value"])) for r in rows
                if r["Counter_Name"] == counter and
                any(k in r["Kernel_Name"] for k in spec["kernels"])]
        vals.sort()
        last = vals[-units * spec["dispatches_per_unit"]:]
        return sum(v for _, v in last), len(last)

    cf_kib, cf_scale = copy_scale(_counter_rows(copy_fetch_csv), "FETCH_SIZE")
    cw_kib, cw_scale = copy_scale(_counter_rows(copy_write_csv), "WRITE_SIZE")
    fk, n_f = kernel_sum(_counter_rows(fetch_csv), "FETCH_SIZE")
    wk, n_w = kernel_sum(_counter_rows(write_csv), "WRITE_SIZE")
    per_unit = (fk * cf_scale + wk * cw_scale) * 1024 / units
    print(f"Calibration (plain device copy of {COPY_BYTES >> 20} MiB): FETCH_SIZE reads "
          f"{cf_kib:.1f} KiB per launch (scale {cf_scale:.3f}), WRITE_SIZE {cw_kib:.1f} KiB "
          f"(scale {cw_scale:.3f}).\n")
    plural = {"pass": "passes", "launch": "launches", "step": "steps"}[spec["unit"]]
    print(f"{' + '.join(spec['kernels'])}: the last {units} {plural} ({n_f} / {n_w} "
          f"dispatches): FETCH_SIZE {fk / units:.1f} KiB, WRITE_SIZE {wk / units:.1f} KiB per "
          f"{spec['unit']}, scaled: {per_unit:.0f} bytes against {algo_bytes} algorithmic "
          f"bytes ({per_unit / algo_bytes:.3f}x).\n")
    print(f"traffic_bytes_per_unit: {round(per_unit)}")
    print(f"algorithmic_bytes_per_unit: {algo_bytes}")


def summarize_pmc(csvs, kernel, last):
    """Per-dispatch means of every counter in rocprofv3 --pmc runs (one CSV per pass) over the
    last `last` dispatches of the kernels whose name contains `kernel`."""
    import collections
    per = collections.defaultdict(dict)  # counter -> dispatch -> value
    for path in csvs:
        for r in _counter_rows(path):
            if kernel in r["Kernel_Name"]:
                per[r["Counter_Name"]][int(r["Dispatch_Id"])] = float(r["Counter_Value"])
    print(f"| counter | mean per dispatch (last {last} of `{kernel}`) |\n|---|---|")
    for name in sorted(per):
        vals = [per[name][d] for d in sorted(per[name])][-last:]
        print(f"| {name} | {sum(vals) / len(vals):.6g} |")


def prefill_pass_bytes():
    """Bytes one attention pass of the chunked prefill must move at least: each chunk reads its
    row's K/V prefix (chunk included) once per KV head and the chunk's q, and writes its out."""
    total = 0
    for c in range(PF_T // PF_C):
        keys = (c + 1) * PF_C
        total += PF_B * keys * PF_HKV * D * 2 * 2 + 2 * PF_B * PF_C * PF_H * D * 2
    return total


def mixed_step_bytes(first, steps):
    """Mean algorithmic bytes of `steps` mixed-stack steps from position 4096 + first."""
    from modelcore_amd import stats
    windows = [-1 if i % 4 == 3 else MX_WIN for i in range(MX_LAYERS)]
    total = 0
    for s in range(steps):
        pos = [MX_P + first + s] * MX_B
        for w in windows:
            total += stats.decode_step_bytes(pos, MX_H, MX_HKV, D, 2, window=w)
    return total // steps


def bench_prefill(args):
    """Chunked prefill: 8 rows x 16384 tokens fed in 32 chunks of 512; each chunk appends its K/V
    at its offset and attends causally to the cache prefix (32 q / 8 kv heads, head_dim 128, bf16,
    N(0, 1) values). One pass = the whole prompt; --steps passes are timed after --warmup."""
    import torch
    from modelcore_amd import _ext, stats
    from modelcore_amd.cache import KVCache
    from modelcore_amd.kernels.flash_attn import flash_attn

    W, K = min(args.warmup, 2), max(1, min(args.steps, 5))
    dev = torch.device("cuda", 0)
    g = torch.Generator(device=dev).manual_seed(args.seed)
    log(f"generating prefill inputs on the GPU: B={PF_B} T={PF_T} H={PF_H} H_kv={PF_HKV} D={D}")
    q = torch.randn(PF_B, PF_T, PF_H, D, generator=g, device=dev).to(torch.bfloat16)
    k = torch.randn(PF_B, PF_T, PF_HKV, D, generator=g, device=dev).to(torch.bfloat16)
    v = torch.randn(PF_B, PF_T, PF_HKV, D, generator=g, device=dev).to(torch.bfloat16)
    cache = KVCache(PF_B, PF_HKV, PF_T, D, 1, dev, torch.bfloat16)
    kc, vc = cache.get_slot_cache(0)
    n_chunks = PF_T // PF_C
    # Each chunk's q/k/v as its own contiguous (B, C, heads, D) tensor, as an attention layer's
    # projections hand them to the operator (slices of the whole-prompt tensors would make the
    # operator copy them first).
    chunks = [tuple(t[:, c * PF_C:(c + 1) * PF_C].contiguous() for t in (q, k, v))
              for c in range(n_chunks)]

    def one_pass():
        cache.reset()
        for qc, kc_new, vc_new in chunks:
            flash_attn.flash_attn_with_kvcache(qc, kc, vc, k=kc_new, v=vc_new,
                                               cache_seqlens=cache.cache_seqlens,
                                               causal=True, window_size=(-1, 0))
            cache.advance(PF_C)

    for _ in range(W):
        one_pass()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(K):
        one_pass()
    end.record()
    torch.cuda.synchronize()
    ms_pass = start.elapsed_time(end) / K

    # Dominant kernel: the attention of each chunk alone (prefill_mfma_kernel), through the C ABI
    # on the stream it runs on, against the cache the passes filled.
    lib = _ext.lib()
    out = torch.empty(PF_B, PF_C, PF_H, D, dtype=torch.bfloat16, device=dev)
    offs = [torch.full((PF_B,), c * PF_C, dtype=torch.int32, device=dev) for c in range(n_chunks)]
    qs = [qc for qc, _, _ in chunks]
    stream = _ext.stream_handle(dev)

    def attn_pass():
        for c in range(n_chunks):
            lib.mcamd_prefill_attention(qs[c].data_ptr(), kc.data_ptr(), vc.data_ptr(),
                                        offs[c].data_ptr(), out.data_ptr(), PF_B, PF_C, PF_H,
                                        PF_HKV, D, PF_T, kc.stride(0), -1, _ext.BF16, stream)

    attn_pass()
    torch.cuda.synchronize()
    start.record()
    for _ in range(K):
        attn_pass()
    end.record()
    torch.cuda.synchronize()
    attn_ms = start.elapsed_time(end) / K
    flops = sum(stats.prefill_flops([c * PF_C] * PF_B, PF_C, PF_H, D) for c in range(n_chunks))
    achieved = flops / (attn_ms * 1e-3)
    bw_peak, flops_peak, peak_src = peaks()

    # The append alone (kv_append_kernel), the same 32 chunk copies through the C ABI: each moves
    # its K and V rows in (B, C, H_kv, D) to their cache positions, algorithmic bytes = read +
    # write of 2 * B * C * H_kv * D bf16 values. A copy takes about as long as one launch through
    # ctypes, so the 32 launches are captured once as a HIP graph and the replays are timed: the
    # kernels then run back to back instead of waiting on the host.
    ks = [kc_new for _, kc_new, _ in chunks]
    vs = [vc_new for _, _, vc_new in chunks]

    def append_pass(strm):
        for c in range(n_chunks):
            _ext.check(lib.mcamd_kv_append(ks[c].data_ptr(), vs[c].data_ptr(), kc.data_ptr(),
                                           vc.data_ptr(), offs[c].data_ptr(), PF_B, PF_C, PF_HKV,
                                           D, PF_T, kc.stride(0), _ext.BF16, strm), "append")

    append_pass(stream)
    torch.cuda.synchronize()
    append_graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(append_graph):
        append_pass(_ext.stream_handle(dev))
    append_graph.replay()
    torch.cuda.synchronize()
    start.record()
    for _ in range(K):
        append_graph.replay()
    end.record()
    torch.cuda.synchronize()
    append_ms = start.elapsed_time(end) / K
    append_bytes = n_chunks * 2 * 2 * PF_B * PF_C * PF_HKV * D * 2
    append_bw = append_bytes / (append_ms * 1e-3)
    append_traffic_launch, append_traffic_src = append_traffic(append_bytes // n_chunks)
    result = {
        "metric": "chunked prefill tok/s at B=8, 16384 tokens in chunks of 512, GQA 32/8 hd128; "
                  "attention MFMA utilisation",
        "value": round(PF_B * PF_T / (ms_pass * 1e-3), 1),
        "unit": "tok/s",
        "n_gpus": 1, "steps": K, "warmup": W, "ms_per_step": round(ms_pass, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "chunked prefill: 8 rows x 16384 tokens, 32 chunks of 512, each "
                               "appended then attended causally against the cache prefix",
                   "batch": PF_B, "tokens": PF_T, "chunk": PF_C, "n_head": PF_H,
                   "n_kv_head": PF_HKV, "head_dim": D},
        "roofline": {"kernel": "prefill_mfma_kernel (attention of the 32 chunks)", "bound": "mfma",
                     "achieved": round(achieved / 1e12, 1), "peak": flops_peak / 1e12,
                     "peak_source": peak_src,
                     "unit": "TFLOP/s", "frac": round(achieved / flops_peak, 4),
                     "ms_per_pass": round(attn_ms, 4), "flops_per_pass": flops},
        "append": {"kernel": "kv_append_kernel (K/V copy of the 32 chunks)", "bound": "hbm",
                   "achieved": round(append_bw / 1e9, 1), "peak": bw_peak / 1e9, "unit": "GB/s",
                   "frac": round(append_bw / bw_peak, 4), "ms_per_pass": round(append_ms, 4),
                   "bytes_per_pass": append_bytes, "traffic": append_traffic_launch,
                   "traffic_source": append_traffic_src,
                   "bytes_per_launch": append_bytes // n_chunks},
    }
    # Traffic of the attention pass: K/V of each chunk's prefix, q and out (the algorithmic
    # bytes a pass must move at least: every key read once per (row, KV head), not once per query
    # tile), against what the counters measured.
    pf_bytes = prefill_pass_bytes()
    t, t_src = profile_traffic("prefill", pf_bytes)
    result["roofline"].update({"traffic": t, "traffic_unit": "bytes per pass",
                               "traffic_min_bytes": pf_bytes, "traffic_source": t_src})
    if not args.no_cpu_baseline:
        log("CPU baseline: the whole chunked prefill on host cores")
        result["cpu_baseline"] = cpu_prefill_baseline(q, k, v)
    return result


def cpu_prefill_baseline(q, k, v):
    """The restated reference fallback (append + masked SDPA with GQA, torch CPU) on the whole
    workload: the same 32 chunks of all 8 rows, appended and attended in order, timed once
    (about 15 s on 16 cores)."""
    import torch
    from oracle import sdpa_fallback

    cores = host_cores()
    torch.set_num_threads(cores)
    qc, kn, vn = q.cpu(), k.cpu(), v.cpu()
    kc = torch.zeros(PF_B, PF_T, PF_HKV, D, dtype=torch.bfloat16)
    vc = torch.zeros_like(kc)
    t0 = time.perf_counter()
    for c in range(PF_T // PF_C):
        a, e = c * PF_C, (c + 1) * PF_C
        pos = torch.full((PF_B,), a, dtype=torch.int32)
        sdpa_fallback.flash_attn_with_kvcache(qc[:, a:e], kc, vc, kn[:, a:e], vn[:, a:e], pos,
                                              (-1, 0))
    dt = time.perf_counter() - t0
    return {"value": round(PF_B * PF_T / dt, 1), "unit": "tok/s", "cores": cores, "kind": "port",
            "sample": f"the whole workload (8 rows x 16384 tokens, 32 chunks of 512, append + "
                      f"attention per chunk), one pass of {dt:.1f} s; torch CPU SDPA restatement "
                      f"of the reference fallback"}


RP_SLOTS, RP_P, RP_ROWS, RP_T, RP_HKV = 32, 2048, 64, 2560, 8


def bench_replicate(args):
    """KVCache.prefill: a batch-1 cache holding a 2048-token prompt in 32 slots (8 KV heads,
    head_dim 128, bf16) replicated into the first 2048 positions of a 64-row cache of 2560
    positions. One step = one prefill() call."""
    import torch
    from modelcore_amd import stats
    from modelcore_amd.cache import KVCache

    W, K = min(args.warmup, 3), max(1, min(args.steps, 20))
    dev = torch.device("cuda", 0)
    g = torch.Generator(device=dev).manual_seed(args.seed)
    log(f"replication: {RP_SLOTS} slots x {RP_P} tokens x {RP_HKV} heads -> {RP_ROWS} rows")
    src = KVCache(1, RP_HKV, RP_P, D, RP_SLOTS, dev, torch.bfloat16)
    src.k_cache.copy_(torch.randn(src.k_cache.shape, generator=g, device=dev))
    src.v_cache.copy_(torch.randn(src.v_cache.shape, generator=g, device=dev))
    src.advance(RP_P)
    dst = KVCache(RP_ROWS, RP_HKV, RP_T, D, RP_SLOTS, dev, torch.bfloat16)

    def step():
        dst.reset()
        dst.prefill(src)

    for _ in range(W):
        step()
    torch.cuda.synchronize()
    assert torch.equal(dst.k_cache[:, RP_ROWS - 1, :RP_P], src.k_cache[:, 0])
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(K):
        step()
    end.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / K
    nbytes = stats.replicate_bytes(RP_SLOTS, RP_ROWS, RP_P, RP_HKV, D, 2)
    gbps = nbytes / (ms * 1e-3) / 1e9
    hbm_peak, _, peak_src = peaks()
    result = {
        "metric": "KV replication GB/s: 2048-token prompt cache, 32 layers x 8 kv heads x hd128, "
                  "into 64 rows; % of HBM peak",
        "value": round(gbps, 1), "unit": "GB/s", "n_gpus": 1, "steps": K, "warmup": W,
        "ms_per_step": round(ms, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": "KVCache.prefill of a batch-1, 2048-token, 32-slot cache into 64 "
                               "rows of a 2560-position cache",
                   "slots": RP_SLOTS, "prompt": RP_P, "rows": RP_ROWS, "n_kv_head": RP_HKV,
                   "head_dim": D},
        "roofline": {"kernel": "kv_replicate_kernel", "bound": "hbm", "achieved": round(gbps, 1),
                     "peak": hbm_peak / 1e9, "peak_source": peak_src, "unit": "GB/s",
                     "frac": round(gbps * 1e9 / hbm_peak, 4), "bytes_per_launch": nbytes},
    }
    t, t_src = profile_traffic("replicate", nbytes)
    result["roofline"].update({"traffic": t, "traffic_unit": "bytes per launch",
                               "traffic_source": t_src})
    if not args.no_cpu_baseline:
        log("CPU baseline: the replication's broadcast copy on host cores")
        result["cpu_baseline"] = cpu_replicate_baseline(src)
    return result


def cpu_replicate_baseline(src, budget_s=10.0):
    """The reference's broadcast copy (oracle.sdpa_fallback.replicate: slice assignment of the
    batch-1 source over all rows) on the host, for 2 of the 32 slots."""
    import torch
    from modelcore_amd import stats
    from oracle import sdpa_fallback

    cores = host_cores()
    torch.set_num_threads(cores)
    n_slots = 2
    sk, sv = src.k_cache[:n_slots].cpu(), src.v_cache[:n_slots].cpu()
    dk = torch.zeros(n_slots, RP_ROWS, RP_T, RP_HKV, D, dtype=torch.bfloat16)
    dv = torch.zeros_like(dk)
    times = []
    t_end = time.perf_counter() + budget_s
    while len(times) < 3 or (time.perf_counter() < t_end and len(times) < 20):
        t0 = time.perf_counter()
        sdpa_fallback.replicate(dk, dv, sk, sv, RP_P)
        times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    nbytes = stats.replicate_bytes(n_slots, RP_ROWS, RP_P, RP_HKV, D, 2)
    return {"value": round(nbytes / med / 1e9, 2), "unit": "GB/s", "cores": cores, "kind": "port",
            "sample": f"{n_slots} of the {RP_SLOTS} slots, median of {len(times)} runs; torch CPU "
                      f"slice-assignment broadcast (the reference's KVCache.prefill copy)"}


MX_LAYERS, MX_B, MX_H, MX_HKV, MX_P, MX_WIN = 24, 16, 12, 4, 4096, 1024


def bench_mixed(args):
    """The KV path of a 24-layer stack per decode step: layer i has window -1 if i % 4 == 3 else
    1024; even layers produce K/V into slot i // 2, odd layers read slot (i - 1) // 2 (and
    rewrite the producer's token there, as the reference's consumer call does). B = 16 rows at
    position 4096 + step, H = 12, H_kv = 4, head_dim 128, bf16. One step = 24 operator calls plus
    the cache advance (inside the last call unless --separate-advance), replayed from a HIP
    graph."""
    import torch
    from modelcore_amd import stats
    from modelcore_amd.cache import KVCache
    from modelcore_amd.kernels.flash_attn import flash_attn

    W, K = args.warmup, args.steps
    dev = torch.device("cuda", 0)
    g = torch.Generator(device=dev).manual_seed(args.seed)
    n_slots = MX_LAYERS // 2
    T = MX_P + W + K + 1
    log(f"mixed-window stack: {MX_LAYERS} layers, {n_slots} slots, B={MX_B}, T={T}")
    cache = KVCache(MX_B, MX_HKV, T, D, n_slots, dev, torch.bfloat16)
    cache.k_cache.copy_(torch.randn(cache.k_cache.shape, generator=g, device=dev))
    cache.v_cache.copy_(torch.randn(cache.v_cache.shape, generator=g, device=dev))
    cache.advance(MX_P)
    n = W + K
    qs = torch.randn(n, MX_LAYERS, MX_B, 1, MX_H, D, generator=g, device=dev).to(torch.bfloat16)
    ks = torch.randn(n, n_slots, MX_B, 1, MX_HKV, D, generator=g, device=dev).to(torch.bfloat16)
    vs = torch.randn(n, n_slots, MX_B, 1, MX_HKV, D, generator=g, device=dev).to(torch.bfloat16)
    windows = [-1 if i % 4 == 3 else MX_WIN for i in range(MX_LAYERS)]

    fold = not args.separate_advance

    def step(s):
        for i in range(MX_LAYERS):
            slot = i // 2
            kc, vc = cache.get_slot_cache(slot)
            last = i == MX_LAYERS - 1
            flash_attn.flash_attn_with_kvcache(qs[s, i], kc, vc, k=ks[s, slot], v=vs[s, slot],
                                               cache_seqlens=cache.cache_seqlens, causal=True,
                                               window_size=(windows[i], 0),
                                               advance=1 if fold and last else 0)
        if fold:
            cache.note_device_advance(1)
        else:
            cache.advance(1)

    for s in range(W):
        step(s)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    if args.eager:  # (the counter runs: one dispatch per kernel, in program order)
        start.record()
        for s in range(K):
            step(W + s)
        end.record()
    else:
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for s in range(K):
                step(W + s)
        # One untimed replay (a graph's first launch also uploads it), then the positions set
        # back: the timed replay rewrites the same new tokens at the same positions.
        graph.replay()
        torch.cuda.synchronize()
        cache.cache_seqlens.fill_(MX_P + W)
        start.record()
        graph.replay()
        end.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / K
    step_bytes = mixed_step_bytes(W, K)
    gbps = step_bytes / (ms * 1e-3) / 1e9
    hbm_peak, _, peak_src = peaks()
    result = {
        "metric": "mixed-window stack decode: KV-path GB/s per step, 24 layers (3:1 local 1024 / "
                  "global), KV sharing, B=16, ctx 4096, GQA 12/4 hd128",
        "value": round(MX_B / (ms * 1e-3), 1), "unit": "tok/s", "n_gpus": 1, "steps": K,
        "warmup": W, "ms_per_step": round(ms, 5), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": "KV path of one decode step of a 24-layer stack (18 layers window "
                               "1024, 6 global; odd layers share the previous layer's slot), B=16, "
                               "positions 4096+", "layers": MX_LAYERS, "batch": MX_B,
                   "n_head": MX_H, "n_kv_head": MX_HKV, "head_dim": D,
                   "timing": "eager" if args.eager else "hip_graph",
                   "advance": "in the last call's merge pass (advance=1)" if fold
                              else "KVCache.advance launch"},
        "roofline": {"kernel": "decode_fused_kernel + decode_merge_kernel (24 calls per step)",
                     "bound": "hbm", "achieved": round(gbps, 1), "peak": hbm_peak / 1e9,
                     "peak_source": peak_src, "unit": "GB/s",
                     "frac": round(gbps * 1e9 / hbm_peak, 4),
                     "bytes_per_step": int(step_bytes)},
    }
    t, t_src = profile_traffic("mixed", int(step_bytes))
    result["roofline"].update({"traffic": t, "traffic_unit": "bytes per step",
                               "traffic_source": t_src})
    if not args.no_cpu_baseline:
        log("CPU baseline: whole steps of the stack (24 calls) on host cores")
        result["cpu_baseline"] = cpu_mixed_baseline(cache, qs, ks, vs, windows, W)
    return result


def cpu_mixed_baseline(cache, qs, ks, vs, windows, first, budget_s=12.0):
    """The restated reference fallback (append + masked SDPA with GQA, torch CPU) on whole steps
    of the stack: the 24 calls of a step in order, each on its layer's slot and window, with the
    same new tokens the GPU steps append, then the positions advance; median over a bounded run
    of consecutive steps from position 4096 + `first`."""
    import torch
    from oracle import sdpa_fallback

    cores = host_cores()
    torch.set_num_threads(cores)
    T = MX_P + first + qs.shape[0] + 1
    kc, vc = cache.k_cache[:, :, :T].cpu(), cache.v_cache[:, :, :T].cpu()
    qc, kn, vn = qs.cpu(), ks.cpu(), vs.cpu()

    def step(s, p):
        pos = torch.full((MX_B,), p, dtype=torch.int32)
        for i in range(MX_LAYERS):
            slot = i // 2
            sdpa_fallback.flash_attn_with_kvcache(qc[s, i], kc[slot], vc[slot], kn[s, slot],
                                                  vn[s, slot], pos, (windows[i], 0))

    times = []
    t_end = time.perf_counter() + budget_s
    step(first, MX_P + first)  # warm-up
    s = first
    while s + 1 < qs.shape[0] and (len(times) < 3 or (time.perf_counter() < t_end and
                                                       len(times) < 20)):
        s += 1
        t0 = time.perf_counter()
        step(s, MX_P + s)
        times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    return {"value": round(MX_B / med, 1), "unit": "tok/s", "cores": cores, "kind": "port",
            "sample": f"whole steps (24 calls: {sum(w >= 0 for w in windows)} window-{MX_WIN}, "
                      f"{sum(w < 0 for w in windows)} global, KV sharing) at B={MX_B}, positions "
                      f"{MX_P + first + 1}+, median of {len(times)}; torch CPU SDPA restatement "
                      f"of the reference fallback"}


SM_LAYERS, SM_D, SM_H, SM_HKV, SM_HID, SM_V = 32, 4096, 32, 8, 14336, 32768
SM_PROMPT, SM_ROWS, SM_NEW = 2048, 64, 512


def sample_config(n_layers):
    """The large-batch sampling model: n_layers llama-style blocks, d_model 4096, 32 q / 8 kv
    heads of 128, gated SiLU MLP 14336, vocab 32768, lm_head softcap 15."""
    from modelcore_amd.model import ComponentSpec, ModelConfig
    blocks = [ComponentSpec("block", {
        "layer_idx": i, "features": [],
        "mixer": ComponentSpec("attention", {"n_head": SM_H, "n_kv_head": SM_HKV, "head_dim": D,
                                             "window": -1, "kv_slot": None, "produces_kv": True,
                                             "features": []}),
        "ffn": ComponentSpec("gated_mlp", {"activation": "silu", "hidden_dim": SM_HID})})
        for i in range(n_layers)]
    return ModelConfig(sequence_len=SM_PROMPT + SM_NEW, vocab_size=SM_V, n_embd=SM_D,
                       shared={"rope": ComponentSpec("rotary", {"head_dim": D, "over_compute": 2}),
                               "norm": ComponentSpec("rms_norm", {"eps": None})},
                       input=ComponentSpec("token_embedding", {"smear": False}),
                       body=ComponentSpec("stack", {"blocks": blocks, "features": []}),
                       output=ComponentSpec("lm_head", {"softcap": 15}))


def cpu_sample_baseline(budget_s=20.0):
    """The reference's decode step on the host, restated: the same model on the CPU in fp32 (the
    reference's CPU compute dtype, modelcore/runtime.py:23-42) with the restated SDPA fallback as
    its operator, 64 rows at position 2048 of a 2560-position cache. One layer is built (seed 0)
    and its step timed with and without the layer's work, and the 32-layer step priced as
    32 layers + embedding and lm_head."""
    import torch
    from modelcore_amd.model import ModelManager
    from modelcore_amd.runtime import Runtime
    from oracle import sdpa_fallback

    cores = host_cores()
    torch.set_num_threads(cores)
    mgr = ModelManager(Runtime(torch.float32), attention=sdpa_fallback.flash_attn)
    model = mgr.create_model(sample_config(1), device=torch.device("cpu"), seed=0)
    cache = mgr.new_kv_cache(model, batch_size=SM_ROWS, seq_len=SM_PROMPT + SM_NEW)
    g = torch.Generator().manual_seed(0)
    cache.k_cache[:, :, :SM_PROMPT].copy_(torch.randn(cache.k_cache[:, :, :SM_PROMPT].shape,
                                                      generator=g))
    cache.v_cache[:, :, :SM_PROMPT].copy_(torch.randn(cache.v_cache[:, :, :SM_PROMPT].shape,
                                                      generator=g))
    tokens = torch.randint(0, SM_V, (SM_ROWS, 1), generator=g)

    def timed(fn, n_min=3, n_max=20, until=None):
        times = []
        fn()  # warm-up
        while len(times) < n_min or (time.perf_counter() < until and len(times) < n_max):
            t0 = time.perf_counter()
            fn()
            times.append(time.perf_counter() - t0)
        return statistics.median(times), len(times)

    def step():
        cache.cache_seqlens.fill_(SM_PROMPT)
        cache._pos_uniform = SM_PROMPT
        model(tokens, kv_cache=cache)

    x = model.embedding(tokens)
    t_end = time.perf_counter() + budget_s
    with torch.no_grad():
        t_step, n_step = timed(step, until=t_end - budget_s / 3)
        t_head, n_head = timed(lambda: model.unembedding(x), until=t_end)
    t_layer = max(t_step - t_head, 0.0)
    step_32 = SM_LAYERS * t_layer + t_head
    return {"value": round(SM_ROWS / step_32, 2), "unit": "tok/s", "cores": cores,
            "kind": "extrapolated",
            "sample": f"one decode step of a 1-layer copy of the model (fp32, oracle operator: the "
                      f"restated reference fallback), 64 rows at position {SM_PROMPT}, median of "
                      f"{n_step}; lm_head alone median of {n_head}; step = {SM_LAYERS} x "
                      f"({t_layer * 1e3:.1f} ms per layer) + {t_head * 1e3:.1f} ms head"}


def sample_weight_bytes():
    """Bytes of the bf16 weights a sampling decode step reads: per layer the stacked QKV
    (6144 x 4096), c_proj (4096 x 4096), the gate/up stack and down_proj (3 x 14336 x 4096), then
    the lm_head (32768 x 4096)."""
    qkv = (SM_H + 2 * SM_HKV) * D * SM_D
    per_layer = qkv + SM_D * SM_D + 3 * SM_HID * SM_D
    return 2 * (SM_LAYERS * per_layer + SM_V * SM_D)


def sample_step_bytes(first, steps, shared=SM_PROMPT):
    """Mean bytes a sampling decode step must read at least, over `steps` steps from decode step
    `first`: the weights, and per layer with the prompt shared (shared > 0) its K/V once plus each
    row's own keys past it, else every row's K/V (the reference's byte model)."""
    from modelcore_amd import stats
    if shared:
        kv = (sum(stats.decode_step_bytes([SM_PROMPT + first + i - shared] * SM_ROWS, SM_H,
                                          SM_HKV, D, 2) for i in range(steps)) / steps
              + 2 * shared * SM_HKV * D * 2) * SM_LAYERS
    else:
        kv = sum(stats.decode_step_bytes([SM_PROMPT + first + i] * SM_ROWS, SM_H, SM_HKV, D, 2)
                 for i in range(steps)) / steps * SM_LAYERS
    return sample_weight_bytes() + kv


def bench_sample(args):
    """Large-batch sampling end to end: a 32-layer model (d_model 4096, 32 q / 8 kv heads of 128,
    gated SiLU MLP 14336, vocab 32768, softcap 15, bf16, random init with seed 0) prefills one
    2048-token prompt (uniform random tokens, seed 0) at batch 1, replicates its cache into 64
    rows (KVCache.prefill), then decodes 512 tokens per row, each drawn on the device at
    temperature 1.0 from a per-row Philox stream (row r seeded r). The first --warmup steps are
    untimed; the value is rows x timed steps / time. The decode attention takes the replicated
    prompt's K/V from row 0 for all rows (KVCache.shared_prefix: that part of the attention runs
    on the matrix cores) unless --no-shared-prefix."""
    import torch
    from modelcore_amd import stats
    from modelcore_amd.model import ModelManager
    from modelcore_amd.runtime import Runtime
    from modelcore_amd.sampling import PhiloxSampler

    dev = torch.device("cuda", 0)
    W = min(args.warmup, SM_NEW - 1)
    K = SM_NEW - W
    cfg = sample_config(SM_LAYERS)
    mgr = ModelManager(Runtime(torch.bfloat16))
    log(f"building the {SM_LAYERS}-layer model on the GPU (seed 0)")
    model = mgr.create_model(cfg, device=dev, seed=0)
    model.cache_inference_weights()
    model.use_skinny_gemm(not args.library_gemm)
    model.set_fused_residual(not args.separate_residual)
    prompt = torch.randint(0, SM_V, (SM_PROMPT,), generator=torch.Generator().manual_seed(0))
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    dec = mgr.new_decoder(model, prompt.tolist(), num_samples=SM_ROWS, max_tokens=SM_NEW)
    end.record()
    torch.cuda.synchronize()
    prefill_ms = start.elapsed_time(end)
    assert dec.kv_cache.shared_prefix == SM_PROMPT, "KVCache.prefill records the shared prompt"
    if args.no_shared_prefix:
        dec.kv_cache.shared_prefix = 0
    sampler = PhiloxSampler(SM_ROWS, dev, base_seed=0)
    graph = not args.eager
    if graph and W == 0:  # capturing runs one real step first
        W, K = 1, SM_NEW - 1
    log(f"prefill + replicate {prefill_ms:.1f} ms; decoding {W} + {K} steps "
        f"({'one captured graph per step' if graph else 'eager'})")
    with torch.inference_mode():
        if graph:
            step = dec.capture(sampler, 1.0)  # includes the first warm-up step
            for _ in range(W - 1):
                step()
        else:
            step = lambda: dec.step(sampler(dec.logits, 1.0).view(-1))  # noqa: E731
            for _ in range(W):
                step()
        torch.cuda.synchronize()
        start.record()
        for _ in range(K):
            step()
        end.record()
        torch.cuda.synchronize()
    ms = start.elapsed_time(end) / K
    assert dec.kv_cache.get_pos() == SM_PROMPT + SM_NEW
    # Weights a step reads: every cached Linear copy (QKV copies are views of their stack), and
    # the interleaved gate/up stacks, whose rows have no per-Linear view.
    weight_bytes = sum(m._cast.numel() * m._cast.element_size() for m in model.modules()
                       if getattr(m, "_cast", None) is not None)
    weight_bytes += sum(m._gate_up.numel() * m._gate_up.element_size() for m in model.modules()
                        if getattr(m, "_gate_up_blocked", False))
    kv = sum(stats.decode_step_bytes([SM_PROMPT + W + i] * SM_ROWS, SM_H, SM_HKV, D, 2)
             for i in range(K)) / K * SM_LAYERS
    shared = dec.kv_cache.shared_prefix
    # Bytes a step must read at least: with the prompt shared, its K/V once per layer and each
    # row's own keys past it; otherwise every row's K/V (the reference's byte model).
    kv_hbm = kv if not shared else (sum(
        stats.decode_step_bytes([SM_PROMPT + W + i - shared] * SM_ROWS, SM_H, SM_HKV, D, 2)
        for i in range(K)) / K + 2 * shared * SM_HKV * D * 2) * SM_LAYERS
    step_bytes = weight_bytes + kv_hbm
    assert abs(step_bytes - sample_step_bytes(W, K, shared)) < 1.0, \
        "the model's cached weight copies differ from the closed-form byte count"
    gbps = step_bytes / (ms * 1e-3) / 1e9
    hbm_peak, _, peak_src = peaks()
    result = {
        "metric": "large-batch sampling tok/s: 32-layer 4096-wide model, one 2048-token prompt "
                  "replicated to 64 rows, 512 tokens per row at temperature 1",
        "value": round(SM_ROWS / (ms * 1e-3), 1), "unit": "tok/s", "n_gpus": 1, "steps": K,
        "warmup": W, "ms_per_step": round(ms, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": "batch-1 prefill of 2048 tokens, KVCache.prefill to 64 rows, "
                               "then one model forward + device sampling per step"
                               + (" (the step captured once as a HIP graph)" if graph else ""),
                   "layers": SM_LAYERS, "d_model": SM_D, "n_head": SM_H, "n_kv_head": SM_HKV,
                   "head_dim": D, "mlp_hidden": SM_HID, "vocab": SM_V, "rows": SM_ROWS,
                   "prompt": SM_PROMPT, "new_tokens": SM_NEW,
                   "decode_gemm": "F.linear" if args.library_gemm else "mcamd_linear_bf16",
                   "residual_step": "torch add + F.rms_norm" if args.separate_residual
                   else "mcamd_residual_rmsnorm",
                   "prefill_and_replicate_ms": round(prefill_ms, 2),
                   "shared_prefix": dec.kv_cache.shared_prefix},
        "roofline": {"kernel": "whole decode step (bf16 weight GEMMs + cached attention of 32 "
                               "layers + sampling)", "bound": "hbm", "achieved": round(gbps, 1),
                     "peak": hbm_peak / 1e9, "peak_source": peak_src, "unit": "GB/s",
                     "frac": round(gbps * 1e9 / hbm_peak, 4), "traffic": None,
                     "traffic_source": "not measured: rocprofv3 --pmc stops with a host "
                                       "segmentation fault at the first launch of "
                                       "decode_fused_prefix_kernel in this workload",
                     "bytes_per_step": int(step_bytes), "weight_bytes": int(weight_bytes),
                     "kv_bytes_per_step": int(kv_hbm),
                     "kv_note": "with shared_prefix > 0 the prompt's K/V count once per layer "
                                "(taken from row 0 for all rows, that part of the attention on "
                                "the matrix cores) plus each row's own keys; the reference's byte "
                                "model counts every row's K/V: reference_model_bytes_per_step",
                     "reference_model_bytes_per_step": int(weight_bytes + kv),
                     "reference_model_gbps": round((weight_bytes + kv) / (ms * 1e-3) / 1e9, 1)},
    }
    if not args.no_cpu_baseline:
        log("CPU baseline: one decode step of a 1-layer copy of the model on host cores")
        result["cpu_baseline"] = cpu_sample_baseline()
    return result


# The other workloads the default run measures beside the headline: (passes or steps timed,
# untimed warm-up) each, fixed so that the run's length does not depend on --steps.
SUBSYSTEM_STEPS = {"prefill": (3, 1), "mixed": (64, 8), "replicate": (10, 2), "sample": (492, 20)}
SUBSYSTEM_KEEP = ("metric", "value", "unit", "ms_per_step", "steps", "warmup", "config",
                  "roofline", "append", "cpu_baseline")


def subsystems(args):
    """The chunked prefill (attention MFMA utilisation and append GB/s), the mixed-window stack's
    decode step, the replication of a prompt cache and the large-batch sampling decode, each as
    its own object with its roofline and a CPU baseline (timed on the same work; the sampling
    one on a 1-layer copy of its model, labelled extrapolated)."""
    import torch
    out = {}
    for name, fn in (("prefill", bench_prefill), ("mixed", bench_mixed),
                     ("replicate", bench_replicate), ("sample", bench_sample)):
        steps, warmup = SUBSYSTEM_STEPS[name]
        sub = argparse.Namespace(**{**vars(args), "steps": steps, "warmup": warmup,
                                    "workload": name})
        log(f"subsystem {name}: {steps} timed after {warmup} warm-up")
        r = fn(sub)
        out[name] = {k: r[k] for k in SUBSYSTEM_KEEP if k in r}
        torch.cuda.synchronize()
        torch.cuda.empty_cache()
    return out


def cpu_baseline(kc, vc, q, k, v, seqlens, budget_s=12.0):
    """The reference's CPU fallback (oracle.sdpa_fallback: append + masked SDPA with GQA) on the
    full decode workload, on this host's cores: median seconds per step over a bounded run."""
    import torch
    from oracle import sdpa_fallback

    cores = host_cores()
    torch.set_num_threads(cores)
    kc, vc = kc.clone(), vc.clone()
    times = []
    t_end = time.perf_counter() + budget_s
    sdpa_fallback.flash_attn_with_kvcache(q, kc, vc, k, v, seqlens, (-1, 0))  # warm-up
    while (len(times) < 20 or time.perf_counter() < t_end) and len(times) < 400:
        t0 = time.perf_counter()
        sdpa_fallback.flash_attn_with_kvcache(q, kc, vc, k, v, seqlens, (-1, 0))
        times.append(time.perf_counter() - t0)
    return statistics.median(times), cores, len(times)


def main():
    args = parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); the KV path runs per GPU "
              f"with no cross-GPU exchange, so run it with --gpus 1", file=sys.stderr)
        sys.exit(2)

    if args.summarize_traffic:
        summarize_traffic(*args.summarize_traffic)
        return
    if args.summarize_trace:
        summarize_trace(args.summarize_trace, args.launches)
        return
    if args.summarize_pmc:
        summarize_pmc(args.summarize_pmc, args.kernel, args.launches)
        return
    if args.summarize_counters:
        name, f, w, cf, cw, units, algo = args.summarize_counters
        summarize_counters(name, f, w, cf, cw, int(units), int(algo))
        return
    if args.calibrate_copy:
        calibrate_copy()
        return
    workloads = {"prefill": bench_prefill, "replicate": bench_replicate, "mixed": bench_mixed,
                 "sample": bench_sample}
    if args.workload in workloads:
        print(json.dumps(workloads[args.workload](args)), flush=True)
        return

    import torch
    from modelcore_amd import _ext, stats
    from modelcore_amd.cache import KVCache
    from modelcore_amd.kernels.flash_attn import flash_attn

    W, K = args.warmup, args.steps
    dev = torch.device("cuda", 0)
    t_alloc = L_MAX + W + K + 1  # room for every step, and for one more query position
    log(f"generating inputs: B={B} H={H} H_kv={H_KV} D={D} T_alloc={t_alloc} steps={W}+{K}")
    g = torch.Generator().manual_seed(args.seed)
    seqlens = torch.randint(L_MIN, L_MAX + 1, (B,), generator=g, dtype=torch.int32)
    assert torch.equal(seqlens, drawn_lengths(args.seed))
    kc = torch.randn(B, t_alloc, H_KV, D, generator=g).to(torch.bfloat16)
    vc = torch.randn(B, t_alloc, H_KV, D, generator=g).to(torch.bfloat16)
    qs = torch.randn(W + K, B, 1, H, D, generator=g).to(torch.bfloat16)
    ks = torch.randn(W + K, B, 1, H_KV, D, generator=g).to(torch.bfloat16)
    vs = torch.randn(W + K, B, 1, H_KV, D, generator=g).to(torch.bfloat16)

    cache = KVCache(B, H_KV, t_alloc, D, 1, dev, torch.bfloat16)
    cache.k_cache[0].copy_(kc)
    cache.v_cache[0].copy_(vc)
    cache.cache_seqlens.copy_(seqlens)
    cache._pos_uniform = None  # right-ragged rows
    qd, kd, vd = qs.to(dev), ks.to(dev), vs.to(dev)
    k_slot, v_slot = cache.get_slot_cache(0)

    def step(i):
        y = flash_attn.flash_attn_with_kvcache(qd[i], k_slot, v_slot, k=kd[i], v=vd[i],
                                               cache_seqlens=cache.cache_seqlens, causal=True,
                                               window_size=(-1, 0),
                                               advance=0 if args.separate_advance else 1)
        if args.separate_advance:
            cache.advance(1)
        else:
            cache.note_device_advance(1)
        return y

    log("warm-up")
    for i in range(W):
        y = step(i)
    torch.cuda.synchronize()
    assert torch.isfinite(y.float()).all()

    if args.eager:
        run = lambda: [step(W + i) for i in range(K)]  # noqa: E731
    else:
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for i in range(K):
                step(W + i)
        run = graph.replay
        # One untimed replay: a graph's first launch also uploads it (~2 us per step more than
        # later replays, measured). The positions are then set back; the timed replay rewrites the
        # same new tokens at the same positions, so it computes exactly what it would have.
        graph.replay()
        torch.cuda.synchronize()
        cache.cache_seqlens.copy_((seqlens + W).to(dev))

    log(f"timing {K} steps ({'eager' if args.eager else 'one graph replay'})")
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    run()
    end.record()
    torch.cuda.synchronize()
    ms_per_step = start.elapsed_time(end) / K
    final = cache.cache_seqlens.cpu()
    assert torch.equal(final, seqlens + W + K), "positions did not advance once per step"

    # Algorithmic bytes of the timed steps (positions grow by one per step).
    base = seqlens.tolist()
    step_bytes = [stats.decode_step_bytes([L + W + i for L in base], H, H_KV, D, 2)
                  for i in range(K)]
    mean_step_bytes = sum(step_bytes) / K
    step_gbps = mean_step_bytes / (ms_per_step * 1e-3) / 1e9

    # Dominant kernels: the decode call of one step as the step issues it -- append of the new
    # token fused into the split-K streaming pass (decode_fused_kernel), then the merge pass
    # (decode_merge_kernel) -- launched back to back through the C ABI on the stream they run on
    # and timed with HIP events around ROOF_LAUNCHES launches. Every launch puts each row's query
    # at its drawn length (whatever --steps and --warmup are) and appends there, so every launch
    # reads the same keys. Launches alternate between this cache and a second one of the same
    # shape (as consecutive layers of a model would), so no launch finds the previous launch's
    # keys in the 256 MB memory-side cache.
    lib = _ext.lib()
    pos = seqlens.to(dev)
    out = torch.empty(B, 1, H, D, dtype=torch.bfloat16, device=dev)
    ws_bytes = lib.mcamd_attn_workspace_bytes(B, 1, H, H_KV, D, t_alloc, -1)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    stream = _ext.stream_handle(dev)
    q1, k1, v1 = qd[0], kd[0], vd[0]
    other = torch.randn(2, *k_slot.shape, device=dev,
                        generator=torch.Generator(device=dev).manual_seed(1)).to(torch.bfloat16)
    slots = [(k_slot, v_slot), (other[0], other[1])]

    def decode_call(i=0):
        kc_i, vc_i = slots[i % 2]
        return lib.mcamd_flash_attn_with_kvcache(
            q1.data_ptr(), k1.data_ptr(), v1.data_ptr(), kc_i.data_ptr(), vc_i.data_ptr(),
            pos.data_ptr(), out.data_ptr(), B, 1, H, H_KV, D, t_alloc, kc_i.stride(0), -1, 1,
            _ext.BF16, ws.data_ptr(), ws_bytes, stream)

    # Warm-up: the first launches over the freshly allocated second cache run ~2 us slower per
    # call (measured on MI355X: 52.6 us in the first block of 200, 50.6 us after), and a run that
    # reaches this loop after only a few steps another ~1 us: the timed launches follow
    # ROOF_WARMUP_S seconds of the same launches, so they are the steady state.
    for i in range(6):
        _ext.check(decode_call(i), "flash_attn_with_kvcache")
    t_warm = time.perf_counter() + ROOF_WARMUP_S
    i = 0
    while time.perf_counter() < t_warm:
        for _ in range(20):
            decode_call(i)
            i += 1
        torch.cuda.synchronize()
    torch.cuda.synchronize()
    start.record()
    for i in range(ROOF_LAUNCHES):
        decode_call(i)
    end.record()
    torch.cuda.synchronize()
    attn_us = start.elapsed_time(end) / ROOF_LAUNCHES * 1e3
    attn_bytes = stats.decode_step_bytes(base, H, H_KV, D, 2, append=True)
    assert attn_bytes == roofline_bytes(args.seed)
    attn_gbps = attn_bytes / (attn_us * 1e-6) / 1e9
    traffic, traffic_src = measured_traffic(attn_bytes) if args.seed == 0 else (None, "seed != 0")
    hbm_peak, _, peak_src = peaks()

    result = {
        "metric": METRIC,
        "value": round(B / (ms_per_step * 1e-3), 1),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": W,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": "decode microbench: append 1 token per row + single-token attention over "
                        "the KV cache + position advance, B=32, GQA 16q/4kv, head_dim 128, "
                        "lengths U[512,8192] seed 0",
            "batch": B, "n_head": H, "n_kv_head": H_KV, "head_dim": D,
            "max_cache_len": t_alloc, "mean_len": round(sum(base) / B + W + K / 2, 1),
            "timing": "eager" if args.eager else "hip_graph",
            "advance": "KVCache.advance launch" if args.separate_advance
                       else "in the operator's merge pass (advance=1)",
        },
        "kv_path_gbps": round(step_gbps, 1),
        "kv_path_pct_peak": round(100 * step_gbps * 1e9 / hbm_peak, 2),
        "roofline": {
            "kernel": "decode_fused_kernel + decode_merge_kernel (append + attention)",
            "bound": "hbm",
            "achieved": round(attn_gbps, 1),
            "peak": hbm_peak / 1e9,
            "peak_source": peak_src,
            "unit": "GB/s",
            "frac": round(attn_gbps * 1e9 / hbm_peak, 4),
            "traffic": traffic,
            "traffic_source": traffic_src,
            "us_per_launch": round(attn_us, 2),
            "bytes_per_launch": attn_bytes,
            "launches": ROOF_LAUNCHES,
            "positions": "the drawn lengths (seed 0), the same for every launch",
        },
    }

    if not args.decode_only:
        result["subsystems"] = subsystems(args)

    if not args.no_cpu_baseline:
        log("CPU baseline: reference fallback (append + masked SDPA) on host cores")
        med, cores, n = cpu_baseline(kc, vc, qs[0], ks[0], vs[0], seqlens)
        result["cpu_baseline"] = {
            "value": round(B / med, 1),
            "unit": "tok/s",
            "cores": cores,
            "kind": "port",
            "sample": f"full decode workload (B=32, lengths U[512,8192]), one step, median of {n} "
                      f"runs; torch CPU SDPA restatement of the reference fallback",
        }
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
