"""Benchmark: fwd+bwd attention TFLOPS and % of MI355X MFMA peak.

Workload (the north-star configuration): bf16 causal
GQA, B=2 Hq=32 Hkv=8 D=128 S=4096, synthetic N(0,1) inputs already resident
in HBM.  One step = forward (O, LSE) + backward (Delta, dQ, dK/dV), exactly
what npu_flash_attention_forward + npu_flash_attention_backward launch
(for head_dim 128 fp16/bf16 the backward stages dS through a workspace:
Delta pass, dK/dV writing dS, dQ = dS K).

FLOP convention: fwd = 4*D*N_pairs*B*Hq over attended (i, j) pairs only,
bwd = 2.5 * fwd (recomputation not counted).  Peak = 2516.6 TFLOP/s
(256 CU x 2.4 GHz x 4096 dense bf16 FLOP/clk/CU).

Prints ONE JSON line.  Per-kernel times come from HIP events recorded on the
stream the kernels are launched on (torch's current stream).  The roofline
"traffic" field (HBM bytes per launch of the dominant kernel) cannot be read
from inside the process: it is the figure recorded by the two rocprofv3
counter passes (FETCH_SIZE, WRITE_SIZE, calibrated on a plain device copy)
over this same command, kept in profiles/hbm_traffic_<config>.md, and null
when no such record exists for the workload.
"""
import argparse
import json
import math
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "npu-flex-att_amd"))

PEAK_TFLOPS = 2516.6  # dense bf16/fp16 MFMA
PEAK_BY_DTYPE = {"bf16": PEAK_TFLOPS, "fp16": PEAK_TFLOPS, "fp32": 157.3}  # dense MFMA per input dtype
TORCH_DTYPE = {"bf16": "bfloat16", "fp16": "float16", "fp32": "float32"}

CONFIGS = {
    # name: (B, Hq, Hkv, Sq, Skv, D, dtype, causal, window, soft_cap, alibi, scale, input_scale)
    "gqa_llama3_8b": (2, 32, 8, 4096, 4096, 128, "bf16", True, 0, 0.0, False, None, 1.0),
    # the same shape on the fp32 path (fp32 matrix cores; peak 157.3 TFLOP/s)
    "gqa_llama3_8b_fp32": (2, 32, 8, 4096, 4096, 128, "fp32", True, 0, 0.0, False, None, 1.0),
    "gemma2_d256": (1, 16, 8, 8192, 8192, 256, "bf16", True, 4096, 50.0, False, 1.0 / 16, 2.0),
    "all_primitives_d64": (1, 28, 4, 16384, 16383, 64, "fp16", True, 2048, 30.0, True, 0.05, 1.0),
    # the reference's own perf-table shapes (RESULT.md:163-167)
    "mha_d64_s128": (1, 2, 2, 128, 128, 64, "fp16", True, 0, 0.0, False, None, 1.0),
    "mha_d64_s512": (1, 2, 2, 512, 512, 64, "fp16", True, 0, 0.0, False, None, 1.0),
    "mha_d64_s1024": (1, 2, 2, 1024, 1024, 64, "fp16", True, 0, 0.0, False, None, 1.0),
    "mha_d64_s2048": (1, 2, 2, 2048, 2048, 64, "fp16", True, 0, 0.0, False, None, 1.0),
}
# Decoding workloads (forward only, split-KV kernels): one new token per
# sequence against a KV cache; HBM-bound, reported in GB/s of K + V read.
DECODE_CONFIGS = {
    "decode_llama3_8b_32k": (8, 32, 8, 1, 32768, 128, "bf16", False, 0, 0.0, False, None, 1.0),
    "decode_gqa_d64_16k": (4, 28, 4, 4, 16384, 64, "fp16", False, 0, 0.0, False, None, 1.0),
}
HBM_PEAK_GBS = 8000.0


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    # 10 warm-up steps, then 100 timed: the first steps of a fresh process run a
    # few percent slower, so short runs understate the steady rate
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--config", default="gqa_llama3_8b", choices=sorted(CONFIGS) + sorted(DECODE_CONFIGS))
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=15.0, help="bounded CPU baseline sample budget")
    ap.add_argument("--layout", default="bnsd", choices=("bnsd", "bsnd"),
                    help="storage of Q/K/V/dO (and so O, dQ, dK, dV): [B,H,S,D], or [B,S,H,D] passed as strided views")
    ap.add_argument("--no-gemm-peak", action="store_true", help="skip the plain GEMM reference rate")
    ap.add_argument("--recompute-dq", action="store_true",
                    help="backward without dS staging: the dQ kernel recomputes S and dP (flexatt_bwd)")
    ap.add_argument("--block-sparsity", type=float, default=0.0,
                    help="also pass a block-sparse map (128 x 128 blocks, shared by all heads) with this fraction "
                         "of the off-diagonal blocks removed; FLOPs count the remaining pairs")
    ap.add_argument("--graph", action="store_true",
                    help="time replays of the step captured once as a HIP graph (torch.cuda.graph) instead of "
                         "eager API calls")
    ap.add_argument("--copy-probe", action="store_true",
                    help="also run one 256 MiB device copy (calibrates FETCH_SIZE/WRITE_SIZE counters)")
    return ap.parse_args()


def metric_name(dts, Hq, Hkv, Sq, Skv, D, causal, window, cap, alibi, scale):
    """The metric label of a workload; for the north-star workload
    exactly BASELINE.json's metric."""
    parts = [dts]
    if causal:
        parts.append("causal")
    if window:
        parts.append(f"window={window}")
    if cap:
        parts.append(f"soft_cap={cap:g}")
    if alibi:
        parts.append("ALiBi")
    if scale is not None:
        parts.append(f"scale={scale:g}")
    parts.append("GQA" if Hq != Hkv else "MHA")
    if Hq != Hkv and Hq // Hkv != 4:
        parts.append(f"G={Hq // Hkv}")
    parts.append(f"D={D}")
    parts.append(f"S={Sq}" if Sq == Skv else f"Sq={Sq} Skv={Skv}")
    return "fwd+bwd attention TFLOPS & % MFMA peak, " + " ".join(parts)


def recorded_traffic(config, kernel):
    """HBM bytes per dispatch of `kernel` from profiles/hbm_traffic_<config>.md."""
    path = os.path.join(ROOT, "profiles", f"hbm_traffic_{config}.md")
    try:
        lines = open(path).read().splitlines()
    except OSError:
        return None
    header = None
    for line in lines:
        cells = [c.strip() for c in line.strip().strip("|").split("|")]
        if header is None and "HBM bytes" in cells:
            header = cells
            continue
        if header and cells and cells[0] == kernel:
            try:
                return int(cells[header.index("HBM bytes")])
            except (ValueError, IndexError):
                return None
    return None


def pairs(sq, skv, causal, window):
    total = 0
    for i in range(sq):
        hi = min(skv - 1, i) if causal else skv - 1
        lo = max(0, i - window) if window > 0 else 0
        total += max(0, hi - lo + 1)
    return total


def main():
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path "
              "(attention over (batch, KV-head) groups shards with no communication). "
              "Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import torch

    import flexatt_lib as L
    import npu_flash_attention as nfa

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)
    dev = torch.device("cuda:0")
    if args.config in DECODE_CONFIGS:
        return decode_main(args, dev)
    nfa.ds_staging_enabled = not args.recompute_dq
    B, Hq, Hkv, Sq, Skv, D, dts, causal, window, cap, alibi, scale, insc = CONFIGS[args.config]
    dtype = getattr(torch, TORCH_DTYPE[dts])
    peak = PEAK_BY_DTYPE[dts]
    g = torch.Generator().manual_seed(42)
    q = (torch.randn(B, Hq, Sq, D, generator=g) * insc).to(dtype).to(dev)
    k = (torch.randn(B, Hkv, Skv, D, generator=g) * insc).to(dtype).to(dev)
    v = (torch.randn(B, Hkv, Skv, D, generator=g) * insc).to(dtype).to(dev)
    do = torch.randn(B, Hq, Sq, D, generator=g).to(dtype).to(dev)
    if args.layout == "bsnd":  # same values, [B, S, H, D] storage, viewed as [B, H, S, D]
        q, k, v, do = (t.transpose(1, 2).contiguous().transpose(1, 2) for t in (q, k, v, do))
    slopes = None
    if alibi:
        slopes = torch.tensor([2.0 ** (-8.0 * (h + 1) / Hq) for h in range(Hq)], dtype=torch.float32, device=dev)
    kw = dict(causal=causal, sliding_window=window, soft_cap=cap, scale=scale, alibi_slope=slopes)
    masks = None
    if args.block_sparsity > 0:
        nqb, nkb = -(-Sq // 128), -(-Skv // 128)
        gb = torch.Generator().manual_seed(7)
        keep = torch.rand(nqb, nkb, generator=gb) >= args.block_sparsity
        keep |= torch.eye(nqb, nkb, dtype=torch.bool)  # every row keeps its diagonal block
        kw["block_mask"] = keep.to(torch.uint8).view(1, 1, nqb, nkb).to(dev)
        masks = nfa._masks(causal, None, None, kw["block_mask"], B, Hq, Sq, Skv, dev)

    if args.copy_probe:
        src = torch.empty(256 << 20, dtype=torch.uint8, device=dev).fill_(1)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    npairs = pairs(Sq, Skv, causal, window)
    if masks is not None:  # pairs of the kept blocks only
        i = torch.arange(Sq).view(-1, 1)
        j = torch.arange(Skv).view(1, -1)
        ok = torch.ones(Sq, Skv, dtype=torch.bool)
        if causal:
            ok &= j <= i
        if window > 0:
            ok &= i - j <= window
        ok &= keep.repeat_interleave(128, 0).repeat_interleave(128, 1)[:Sq, :Skv]
        npairs = int(ok.sum())
    fwd_flop = 4.0 * D * npairs * B * Hq
    bwd_flop = 2.5 * fwd_flop

    def step():
        o, lse = nfa.npu_flash_attention_forward(q, k, v, return_lse=True, **kw)
        nfa.npu_flash_attention_backward(q, k, v, o, lse, do, **kw)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    run = step
    if args.graph:
        # the whole step (forward + backward, its allocations from the graph's
        # pool) captured once; each timed step is one replay
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            step()
        torch.cuda.synchronize()
        run = graph.replay
        for _ in range(args.warmup):
            run()
        torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        run()
    torch.cuda.synchronize()
    ms_step = (time.perf_counter() - t0) * 1e3 / args.steps

    # Per-kernel durations through the C ABI, HIP events on the launch stream,
    # of the launches the backward makes.  With dS staging (head_dim 128
    # fp16/bf16): the Delta pass, dK/dV (which also writes dS) and dQ = dS K.
    # Otherwise: "dq" is flexatt_bwd_dq_delta (the Delta pass, then the dQ
    # kernel that recomputes S and dP) and "dkdv" the dK/dV kernel.
    lib = L.load()
    o, lse = nfa.npu_flash_attention_forward(q, k, v, return_lse=True, **kw)
    delta = torch.empty(B, Hq, Sq, dtype=torch.float32, device=dev)
    dq = torch.empty_like(q)
    dk = torch.empty_like(k)
    dv = torch.empty_like(v)
    p = nfa._problem(q, k, scale if scale is not None else 1.0 / math.sqrt(D), causal, window, cap, slopes, masks)
    st = torch.cuda.current_stream(dev)
    sh = st.cuda_stream
    T = L.tensor
    # the workspace the API itself sizes (npu_flash_attention's workspace budget)
    ws_bytes = nfa._staged_workspace_bytes(lib, p, dev)
    calls = {"fwd": lambda: lib.flexatt_fwd(p, T(q), T(k), T(v), T(o), lse.data_ptr(), sh)}
    if ws_bytes and ws_bytes < lib.flexatt_bwd_workspace(p):
        # the band exceeds the budget: the staged backward runs in passes over
        # chunks of (batch, KV-head) groups, timed as one call
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
        calls["bwd_passes"] = lambda: lib.flexatt_bwd_ws(p, T(q), T(k), T(v), T(o), T(do), lse.data_ptr(),
                                                         delta.data_ptr(), T(dq), T(dk), T(dv), ws.data_ptr(),
                                                         ws_bytes, sh)
    elif ws_bytes:
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
        calls["delta"] = lambda: lib.flexatt_bwd_delta(p, T(o), T(do), delta.data_ptr(), sh)
        calls["dkdv"] = lambda: lib.flexatt_bwd_dkdv_ds(p, T(q), T(k), T(v), T(do), lse.data_ptr(),
                                                        delta.data_ptr(), T(dk), T(dv), ws.data_ptr(), ws_bytes, sh)
        calls["dq"] = lambda: lib.flexatt_bwd_dq_ds(p, T(k), ws.data_ptr(), ws_bytes, T(dq), sh)
    else:
        calls["dq"] = lambda: lib.flexatt_bwd_dq_delta(p, T(q), T(k), T(v), T(o), T(do), lse.data_ptr(),
                                                       delta.data_ptr(), T(dq), sh)
        calls["dkdv"] = lambda: lib.flexatt_bwd_dkdv(p, T(q), T(k), T(v), T(do), lse.data_ptr(), delta.data_ptr(),
                                                     T(dk), T(dv), sh)
    reps = max(args.steps, 10)
    kernel_ms = {}
    for name, fn in calls.items():
        for _ in range(3):
            L.check(fn(), name)
        evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(reps)]
        for a, b in evs:
            a.record(st)
            L.check(fn(), name)
            b.record(st)
        torch.cuda.synchronize()
        kernel_ms[name] = statistics.median(a.elapsed_time(b) for a, b in evs)

    fwd_ms = kernel_ms["fwd"]
    bwd_ms = sum(v_ for k_, v_ in kernel_ms.items() if k_ != "fwd")
    fwd_tf = fwd_flop / fwd_ms / 1e9
    bwd_tf = bwd_flop / bwd_ms / 1e9
    total_tf = (fwd_flop + bwd_flop) / ms_step / 1e9
    # Roofline of the dominant (longest) kernel, with its share of the
    # algorithmic FLOPs per launch: fwd 4*D*pairs*B*Hq; dK/dV 8*D*... (S, dP,
    # P^T dO, dS^T Q: four of the five backward GEMMs); dQ 2*D*... (dS K).  The
    # shares of the backward kernels add up to the 10*D convention; a dQ
    # kernel that recomputes S and dP executes 6*D but is credited 2*D.
    per_kernel_flop = {"fwd": fwd_flop, "dq": 2.0 * D * npairs * B * Hq, "dkdv": 8.0 * D * npairs * B * Hq,
                       "bwd_passes": bwd_flop}
    dom = max(kernel_ms, key=lambda n: kernel_ms[n])
    achieved = per_kernel_flop[dom] / kernel_ms[dom] / 1e9

    gemm = None if args.no_gemm_peak else gemm_peak(dev, dtype, dts)

    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(q, k, v, do, kw, slopes, args.cpu_seconds, Hq // Hkv, causal, window, D, Sq, Skv)

    out = {
        "metric": metric_name(dts, Hq, Hkv, Sq, Skv, D, causal, window, cap, alibi, scale),
        "value": round(total_tf, 2),
        "unit": "TFLOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": dts,
        "data": "synthetic N(0,1), seed 42, resident in HBM",
        "step_launch": "hip graph replay" if args.graph else "eager API calls",
        "config": {
            "workload": f"{args.config}: {dts} B={B} Hq={Hq} Hkv={Hkv} Sq={Sq} Skv={Skv} D={D} causal={causal} "
                        f"window={window} soft_cap={cap} alibi={alibi} scale={scale}"
                        + (f" block_sparsity={args.block_sparsity}" if masks is not None else "") + "; step = fwd + bwd",
            "batch": B, "heads_q": Hq, "heads_kv": Hkv, "seqlen_q": Sq, "seqlen_kv": Skv, "head_dim": D,
            "parallelism": "single GPU", "layout": args.layout,
        },
        "fwd_ms": round(fwd_ms, 4),
        "bwd_ms": round(bwd_ms, 4),
        "kernel_ms": {k_: round(v_, 4) for k_, v_ in kernel_ms.items()},
        "fwd_tflops": round(fwd_tf, 1),
        "bwd_tflops": round(bwd_tf, 1),
        "fwd_frac_peak": round(fwd_tf / peak, 4),
        "bwd_frac_peak": round(bwd_tf / peak, 4),
        "frac_peak": round(total_tf / peak, 4),
        "roofline": {
            "kernel": dom,
            "bound": "mfma",
            "achieved": round(achieved, 1),
            "peak": peak,
            "unit": "TFLOP/s",
            "frac": round(achieved / peak, 4),
            "traffic": recorded_traffic(args.config, dom) if masks is None else None,
        },
        "cpu_baseline": cpu,
    }
    if gemm is not None:
        # secondary denominator: what a plain library bf16 GEMM reaches on this GPU
        out["gemm_peak"] = gemm
        out["frac_gemm_peak"] = round(total_tf / gemm["tflops"], 4)
    print(json.dumps(out), flush=True)


def decode_main(args, dev):
    """Decoding step (forward only) through the drop-in forward, which takes
    the split-KV kernels for this shape; value = K + V bytes / step time."""
    import torch

    import flexatt_lib as L
    import npu_flash_attention as nfa

    B, Hq, Hkv, Sq, Skv, D, dts, causal, window, cap, alibi, scale, insc = DECODE_CONFIGS[args.config]
    dtype = {"bf16": torch.bfloat16, "fp16": torch.float16}[dts]
    g = torch.Generator().manual_seed(42)
    q = torch.randn(B, Hq, Sq, D, generator=g).to(dtype).to(dev)
    k = torch.randn(B, Hkv, Skv, D, generator=g).to(dtype).to(dev)
    v = torch.randn(B, Hkv, Skv, D, generator=g).to(dtype).to(dev)
    kw = dict(causal=causal, sliding_window=window, soft_cap=cap, scale=scale)
    p = nfa._problem(q, k, scale if scale is not None else 1.0 / math.sqrt(D), causal, window, cap, None)
    assert L.load().flexatt_fwd_decode_workspace(p) > 0, "workload outside the decode kernels' range"
    st = torch.cuda.current_stream(dev)

    def timed(n):
        evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(n)]
        for e0, e1 in evs:
            e0.record(st)
            nfa.npu_flash_attention_forward(q, k, v, return_lse=True, **kw)
            e1.record(st)
        torch.cuda.synchronize()
        return statistics.median(e0.elapsed_time(e1) for e0, e1 in evs)

    for _ in range(args.warmup):
        nfa.npu_flash_attention_forward(q, k, v, return_lse=True, **kw)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        nfa.npu_flash_attention_forward(q, k, v, return_lse=True, **kw)
    torch.cuda.synchronize()
    ms_step = (time.perf_counter() - t0) * 1e3 / args.steps
    ms_ev = timed(max(args.steps, 10))
    nfa.decode_enabled = False  # the regular forward kernel on the same step, for reference
    try:
        for _ in range(3):
            nfa.npu_flash_attention_forward(q, k, v, return_lse=True, **kw)
        ms_regular = timed(max(args.steps, 10))
    finally:
        nfa.decode_enabled = True
    es = q.element_size()
    kv_bytes = 2 * B * Hkv * Skv * D * es
    io_bytes = kv_bytes + 2 * B * Hq * Sq * D * es + B * Hq * Sq * 4
    gbs = kv_bytes / ms_step / 1e6
    achieved = io_bytes / ms_ev / 1e6
    cpu = None
    if not args.no_cpu_baseline:
        from oracle import attention_oracle as orc

        torch.set_num_threads(os.cpu_count() or 1)
        G = Hq // Hkv
        qc, kc, vc = (t.float().cpu() for t in (q, k, v))
        done, t1 = 0, time.perf_counter()
        for b in range(B):
            for h in range(Hkv):
                orc.forward(qc[b:b + 1, h * G:(h + 1) * G], kc[b:b + 1, h:h + 1], vc[b:b + 1, h:h + 1], causal,
                            window, None, kw["scale"], cap, torch.float32)
                done += 1
            if time.perf_counter() - t1 > args.cpu_seconds:
                break
        secs = time.perf_counter() - t1
        cpu = {"value": round(2 * done * Skv * D * es / secs / 1e9, 3), "unit": "GB/s", "cores": torch.get_num_threads(),
               "kind": "port", "sample": f"{done} of {B * Hkv} (batch, KV-head) groups, fp32 eager oracle forward, "
                                         f"{secs:.1f} s"}
    out = {
        "metric": "decode attention K+V HBM throughput (split-KV forward)",
        "value": round(gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": dts,
        "data": "synthetic N(0,1), seed 42, resident in HBM",
        "config": {"workload": f"{args.config}: {dts} B={B} Hq={Hq} Hkv={Hkv} Sq={Sq} Skv={Skv} D={D} "
                               f"causal={causal}; step = one forward (O, LSE)",
                   "batch": B, "heads_q": Hq, "heads_kv": Hkv, "seqlen_q": Sq, "seqlen_kv": Skv, "head_dim": D,
                   "parallelism": "single GPU"},
        "kernel_ms": {"decode_and_merge": round(ms_ev, 4), "regular_forward": round(ms_regular, 4)},
        "roofline": {"kernel": "decode", "bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None},
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)


def gemm_peak(dev, dtype, name):
    """Plain GEMM rate in the workload's dtype (torch.matmul, i.e. hipBLASLt): 8192^3, median of 20."""
    import torch

    n = 8192
    a = torch.randn(n, n, device=dev).to(dtype)
    b = torch.randn(n, n, device=dev).to(dtype)
    for _ in range(3):
        torch.matmul(a, b)
    st = torch.cuda.current_stream(dev)
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(20)]
    for e0, e1 in evs:
        e0.record(st)
        torch.matmul(a, b)
        e1.record(st)
    torch.cuda.synchronize()
    ms = statistics.median(e0.elapsed_time(e1) for e0, e1 in evs)
    return {"tflops": round(2.0 * n ** 3 / ms / 1e9, 1), "shape": f"{n}x{n}x{n} {name} torch.matmul"}


def cpu_baseline(q, k, v, do, kw, slopes, budget_s, G, causal, window, D, Sq, Skv):
    """The fp32 eager math path (the oracle) on the host cores, over as many
    (batch, KV-head) groups of the same workload as fit the time budget."""
    import torch

    from oracle import attention_oracle as orc

    torch.set_num_threads(os.cpu_count() or 1)
    qc, kc, vc, dc = (t.float().cpu() for t in (q, k, v, do))
    sl = None if slopes is None else slopes.cpu()
    B, Hkv = kc.shape[0], kc.shape[1]
    done = 0
    t0 = time.perf_counter()
    for b in range(B):
        for h in range(Hkv):
            hs = slice(h * G, (h + 1) * G)
            o, lse = orc.forward(qc[b:b + 1, hs], kc[b:b + 1, h:h + 1], vc[b:b + 1, h:h + 1], causal, window,
                                 None if sl is None else sl[hs], kw["scale"], kw["soft_cap"], torch.float32)
            orc.backward(qc[b:b + 1, hs], kc[b:b + 1, h:h + 1], vc[b:b + 1, h:h + 1], dc[b:b + 1, hs], causal,
                         window, None if sl is None else sl[hs], kw["scale"], kw["soft_cap"], torch.float32, o=o)
            done += 1
            if time.perf_counter() - t0 > budget_s:
                break
        else:
            continue
        break
    secs = time.perf_counter() - t0
    flop = 3.5 * 4.0 * D * pairs(Sq, Skv, causal, window) * G * done
    cpu_model = ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    cpu_model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {
        "value": round(flop / secs / 1e12, 4),
        "unit": "TFLOPS",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": f"{done} of {B * Hkv} (batch, KV-head) groups ({done * G} query heads), fwd+bwd fp32 eager "
                  f"oracle, {secs:.1f} s on {cpu_model or 'host CPU'}",
    }


if __name__ == "__main__":
    main()
