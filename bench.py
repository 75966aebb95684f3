"""Benchmark of the quantized attention path on one MI355X.

Workload: Wan2.1-1.3B 480p x 81-frame DiT self-attention, B=1, L=32760, H=12,
D=128, bf16 q/k after RMSNorm + 3-D RoPE, non-causal.  One step = one attention layer call through
the drop-in entry: K mean, fused Q/K per-block INT8 quantization, V per-channel FP8 quantization and
the INT8-QK / FP8-PV attention kernel.  Each step uses its own seeded inputs (30 layers = 30
independent calls), all resident in HBM before timing starts.

Prints ONE JSON line (rank 0).  value = TOPS of the whole call (4*B*H*Lq*Lk*D ops / ms_per_step).
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)


def _cpu_info() -> dict:
    """Host CPU facts for the CPU-baseline report: model, usable cores (affinity) and OpenMP settings."""
    model = "?"
    try:
        with open("/proc/cpuinfo") as f:
            for ln in f:
                if ln.startswith("model name"):
                    model = ln.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"model": model, "affinity_cpus": len(os.sched_getaffinity(0)), "os_cpu_count": os.cpu_count(),
            "OMP_NUM_THREADS": os.environ.get("OMP_NUM_THREADS")}


def _cpu_baseline(cfg, budget_s: float = 12.0) -> dict:
    """Time the CPU restatement of the reference math (oracle/, gcc -O3, OpenMP) on a bounded sample of the
    workload's first head: one fixed single-thread slice (attention only: 128 queries x all keys) for a
    per-thread rate, then the whole call path (K mean + quantizers + attention) on all threads, growing
    the query rows until one pass takes about budget_s / 2.  Reports the threads that actually ran."""
    import numpy as np
    import torch

    from oracle import oracle
    from telefuser_amd.workloads import make_inputs

    oracle.build()
    q, k, v, _ = make_inputs(cfg, "cpu", call=0)
    qb = q[:, :, :1].contiguous().view(torch.int16).numpy().view(np.uint16)
    kb = k[:, :, :1].contiguous().view(torch.int16).numpy().view(np.uint16)
    vb = v[:, :, :1].contiguous().view(torch.int16).numpy().view(np.uint16)
    sm = cfg.D ** -0.5
    km = oracle.k_mean_bits(kb)
    k8, ks = oracle.quant_per_block_int8(kb, km_bits=km, blk=64)
    v8, vs = oracle.per_channel_fp8(vb)
    q8, qs = oracle.quant_per_block_int8(np.ascontiguousarray(qb[:, :128]), sm_scale=sm * oracle.LOG2E, blk=128)
    threads_all = oracle.num_threads()
    oracle.set_threads(1)
    try:
        one = oracle.parallel_threads()
        t0 = time.perf_counter()
        oracle.qattn_fwd(q8, qs, k8, ks, v8, vs)
        dt1 = time.perf_counter() - t0
    finally:
        oracle.set_threads(threads_all)
    ns_pair_1t = dt1 / (128 * cfg.Lk) * 1e9
    observed = oracle.parallel_threads()

    def whole(rows):
        qh = np.ascontiguousarray(qb[:, :rows])
        t0 = time.perf_counter()
        kmh = oracle.k_mean_bits(kb)
        q8h, qsh = oracle.quant_per_block_int8(qh, sm_scale=sm * oracle.LOG2E, blk=128)
        k8h, ksh = oracle.quant_per_block_int8(kb, km_bits=kmh, blk=64)
        v8h, vsh = oracle.per_channel_fp8(vb)
        oracle.qattn_fwd(q8h, qsh, k8h, ksh, v8h, vsh)
        return time.perf_counter() - t0

    rows = 128 * observed
    dt = whole(rows)
    while dt * 2 < budget_s and rows < cfg.Lq:
        rows = min(cfg.Lq, rows * 2 if dt * 4 < budget_s else int(rows * budget_s / 2 / dt))
        dt = whole(rows)
    pairs = rows * cfg.Lk
    ops = 4.0 * pairs * cfg.D

    # the reference's own CPU-runnable case (config 1: B=1, H=2, L=1024) timed in full on all threads
    from telefuser_amd.workloads import CONFIGS
    c1 = CONFIGS["c1"]
    q1, k1, v1, _ = make_inputs(c1, "cpu", call=0)
    bits = lambda t: t.contiguous().view(torch.int16).numpy().view(np.uint16)
    q1b, k1b, v1b = bits(q1), bits(k1), bits(v1)
    t0 = time.perf_counter()
    km1 = oracle.k_mean_bits(k1b)
    q18, q1s = oracle.quant_per_block_int8(q1b, sm_scale=c1.D ** -0.5 * oracle.LOG2E, blk=128)
    k18, k1s = oracle.quant_per_block_int8(k1b, km_bits=km1, blk=64)
    v18, v1s = oracle.per_channel_fp8(v1b)
    oracle.qattn_fwd(q18, q1s, k18, k1s, v18, v1s)
    dt_c1 = time.perf_counter() - t0
    return {
        "value": round(ops / dt / 1e12, 6),
        "unit": "TOPS",
        "cores": observed,
        "kind": "port",
        "sample": f"head 0 of {cfg.Hq}, first {rows} of {cfg.Lq} queries x all {cfg.Lk} keys (K mean + Q/K/V "
                  f"quantizers + attention) on {observed} threads in {dt:.2f} s",
        "ns_per_query_key_pair_per_thread": round(dt / pairs * 1e9 * observed, 2),
        "single_thread": {"sample": f"attention only, 128 queries x {cfg.Lk} keys", "s": round(dt1, 3),
                          "ns_per_query_key_pair": round(ns_pair_1t, 2), "threads_observed": one},
        "host": dict(_cpu_info(), omp_max_threads=threads_all, omp_threads_observed=observed),
        "c1_full": {"workload": c1.name, "s": round(dt_c1, 4), "TOPS": round(c1.ops() / dt_c1 / 1e12, 6),
                    "threads": observed},
    }


def _stream_bench(steps: int = 20, warmup: int = 3) -> dict:
    """Steady-state streaming step at the C5 shape (4680-token chunk vs a full 32760-slot rolling cache):
    the reference call site (bf16 dict cache, roll + attention() re-quantizing the window) against
    QuantizedKVCache (ring, incremental quantization)."""
    import torch

    from telefuser_amd.attention import AttentionConfig, AttnImplType
    from telefuser_amd.kv_cache import QuantizedKVCache, streaming_self_attention
    from telefuser_amd.workloads import CONFIGS

    cfg = CONFIGS["c5"]
    dev = torch.device("cuda:0")
    n, size, H, D = cfg.Lq, cfg.Lk, cfg.Hq, cfg.D
    g = torch.Generator(device=dev).manual_seed(5)
    chunks = [tuple(torch.randn((1, n, H, D), generator=g, device=dev).to(torch.bfloat16) for _ in range(3))
              for _ in range(4)]
    frames = size // n  # local_attn_size in chunks; every step after the first `frames` evicts one chunk
    cfg_sage = AttentionConfig(attn_impl=AttnImplType.SAGE_ATTN_2_8_8)
    ref = {"k": torch.zeros((1, size, H, D), dtype=torch.bfloat16, device=dev),
           "v": torch.zeros((1, size, H, D), dtype=torch.bfloat16, device=dev),
           "global_end_index": 0, "local_end_index": 0}
    cache = QuantizedKVCache(1, size, H, D, device=dev)
    out = {}
    for name, target in (("reference_dict", ref), ("quantized_ring", cache)):
        for i in range(frames + warmup):
            q, k, v = chunks[i % 4]
            streaming_self_attention(q, k, v, target, i * n, local_attn_size=frames, attention_config=cfg_sage)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for i in range(frames + warmup, frames + warmup + steps):
            q, k, v = chunks[i % 4]
            streaming_self_attention(q, k, v, target, i * n, local_attn_size=frames, attention_config=cfg_sage)
        torch.cuda.synchronize()
        out[name] = (time.perf_counter() - t0) * 1e3 / steps
    return {"workload": cfg.name + " (steady state, cache full, one chunk evicted per step)",
            "ms_per_step_reference_path": round(out["reference_dict"], 4),
            "ms_per_step_quantized_cache": round(out["quantized_ring"], 4),
            "speedup": round(out["reference_dict"] / out["quantized_ring"], 3)}


def _prologue_bench(reps: int = 10) -> dict:
    """C2 shape, Q and K from the linear outputs to INT8: the reference's sequence (RMSNorm kernel, RoPE
    kernel, then K mean + per-block quantization of the materialised bf16 Q/K; norm and rope as torch
    fp32 ops here) against the fused prologue (row statistics, rotated-K mean, one quantizer launch)."""
    import torch

    from telefuser_amd import sageattn2 as sa
    from telefuser_amd.prologue import norm_rope_quant_qk

    B, L, H, D = 1, 32760, 12, 128
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(7)
    xq, xk = (torch.randn((B, L, H * D), generator=g, device=dev).to(torch.bfloat16) for _ in range(2))
    wq = wk = torch.ones(H * D, dtype=torch.bfloat16, device=dev)
    ang = torch.rand((L, 1, D // 2), generator=g, device=dev, dtype=torch.float64) * 6.3
    fc, fs = ang.cos(), ang.sin()
    cs, sn = fc.reshape(1, L, 1, -1).float(), fs.reshape(1, L, 1, -1).float()

    def unfused():
        out = []
        for x, w in ((xq, wq), (xk, wk)):
            xf = x.float()
            y = ((xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + 1e-6)) * w.float()).to(torch.bfloat16)
            y = y.float().reshape(B, L, H, D // 2, 2)
            o = torch.stack([y[..., 0] * cs - y[..., 1] * sn, y[..., 0] * sn + y[..., 1] * cs], -1)
            out.append(o.reshape(B, L, H, D).to(torch.bfloat16))
        km = sa.k_mean(out[1], "NHD")
        return sa.per_block_int8(out[0], out[1], km, sm_scale=D ** -0.5, tensor_layout="NHD")

    def fused():
        return norm_rope_quant_qk(xq, xk, wq, wk, fc, fs, H)

    res = {}
    for name, f in (("unfused_ms", unfused), ("fused_ms", fused)):
        for _ in range(2):
            f()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(reps):
            f()
        b.record()
        torch.cuda.synchronize()
        res[name] = round(a.elapsed_time(b) / reps, 4)
    bytes_min = 2 * B * L * H * D * 2 + 2 * B * L * H * D  # read bf16 Q and K once, write int8 Q and K
    res["fused_GB/s_vs_single_pass_bytes"] = round(bytes_min / (res["fused_ms"] * 1e-3) / 1e9, 1)
    res["workload"] = "wan2.1-1.3b_480p Q/K prologue (B=1, L=32760, H=12, D=128)"
    return res


def _config_bench(name: str, calls: int = 5, warmup: int = 2) -> dict:
    """One BASELINE config through the same drop-in sequence as the headline step (the fused prologue:
    K mean, per-block K (and Q) quantizer, V fp8; then the attention, which quantizes Q itself where
    qattn_fwd_q16 covers the launch), inputs resident in HBM: ms per call, the attention launch alone (HIP
    events on the launch stream) and its roofline fraction.  C4's attention launch is bounded by HBM
    (int8 Q + K + e4m3 V read once, bf16 O written), the others by the dense INT8/FP8 MFMA peak."""
    import torch

    from telefuser_amd import _lib
    from telefuser_amd import sageattn2 as sa
    from telefuser_amd.workloads import CONFIGS, make_inputs, peak_ops

    cfg = CONFIGS[name]
    dev = torch.device("cuda:0")
    q, k, v, kvv = make_inputs(cfg, dev, call=0)
    sm = cfg.D ** -0.5
    L = _lib.load()
    t_attn = []

    q16 = sa.q16_supported(cfg.B, cfg.Lq, cfg.Lk, cfg.Hq, cfg.D, "per_block")

    def call(record):
        q8, qs, k8, ks, _, v8, vs, _ = sa.sage_quant(q, k, v, tensor_layout="NHD", sm_scale=sm, quantize_q=not q16)
        s = torch.cuda.current_stream()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(s)
        if q16:
            o = sa.qattn_fwd_q16(q, k8, ks, v8, vs, tensor_layout="NHD", qk_mult=sm * sa.LOG2E, kv_valid_len=kvv,
                                 qk_quant_gran="per_block")
        else:
            o = sa.qattn_fwd(q8, qs, k8, ks, v8, vs, tensor_layout="NHD", out_dtype=q.dtype, kv_valid_len=kvv)
        e1.record(s)
        if record:
            t_attn.append((e0, e1))
        return o

    for _ in range(warmup):
        call(False)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(calls):
        call(True)
    torch.cuda.synchronize()
    ms_call = (time.perf_counter() - t0) * 1e3 / calls
    # the label comes from the rule the launch used (FP8 V, per-block scales, non-causal, automatic splits),
    # and must agree with the kernel the last launch reports
    splits = L.qattn_fwd_ex_num_splits(cfg.B, cfg.Lq, cfg.Lk, cfg.Hq, _lib.QATTN_V_FP8, _lib.QATTN_GRAN_BLOCK)
    kernel_id = L.qattn_fwd_ex_kernel(cfg.B, cfg.Lq, cfg.Lk, cfg.Hq, _lib.QATTN_V_FP8, _lib.QATTN_GRAN_BLOCK, 0, 0)
    assert kernel_id == L.qattn_last_kernel(), (kernel_id, L.qattn_last_kernel())
    kernel = _lib.KERNEL_NAMES.get(kernel_id, "?")
    ms_attn = sum(a.elapsed_time(b) for a, b in t_attn) / len(t_attn)
    ops = cfg.ops()
    res = {"workload": cfg.name, "calls": calls, "ms_per_call": round(ms_call, 4), "attn_ms": round(ms_attn, 4),
           "q_quantized_in_attention": q16,
           "attn_kernel": kernel + (f" + qattn_combine_kernel ({splits} KV splits)" if splits > 1 else ""),
           "attn_TOPS": round(ops / (ms_attn * 1e-3) / 1e12, 2),
           "call_TOPS": round(ops / (ms_call * 1e-3) / 1e12, 2),
           "mfma_frac": round(ops / (ms_attn * 1e-3) / peak_ops("fp8"), 4)}
    if name == "c4":
        # algorithmic HBM bytes of the attention launch: Q (int8, or bf16 when the kernel quantizes it) + int8 K
        # + e4m3 V read once, bf16 O written
        byts = cfg.B * cfg.Hq * cfg.Lq * cfg.D * ((2 if q16 else 1) + 2) + 2 * cfg.B * cfg.Hkv * cfg.Lk * cfg.D
        res["bound"] = "hbm"
        res["attn_GB/s"] = round(byts / (ms_attn * 1e-3) / 1e9, 1)
        res["hbm_frac"] = round(byts / (ms_attn * 1e-3) / 8e12, 4)
        res["algorithmic_bytes_per_launch"] = byts
    else:
        res["bound"] = "mfma"
    # the same config through the entry TeleFuser's attention() calls for SAGE_ATTN_2_8_8 (per-thread scales,
    # "fp32+fp32"; attention_impl.py:249-258): for key ranges of at most 512 it quantizes Q inside the
    # resident kernel (qattn_fwd_q16)
    def tf_call():
        return sa.sageattn_qk_int8_pv_fp8_cuda(q, k, v, tensor_layout="NHD", qk_quant_gran="per_thread",
                                               pv_accum_dtype="fp32+fp32", kv_valid_len=kvv)

    for _ in range(warmup):
        tf_call()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(calls):
        tf_call()
    torch.cuda.synchronize()
    ms_tf = (time.perf_counter() - t0) * 1e3 / calls
    res["telefuser_path"] = {"entry": "sageattn_qk_int8_pv_fp8_cuda(per_thread, fp32+fp32)",
                             "ms_per_call": round(ms_tf, 4), "call_TOPS": round(ops / (ms_tf * 1e-3) / 1e12, 2),
                             "q_quantized_in_attention": sa.q16_supported(cfg.B, cfg.Lq, cfg.Lk, cfg.Hq, cfg.D,
                                                                          "per_thread")}
    del q, k, v
    torch.cuda.empty_cache()
    return res


def _telefuser_call_path(steps: int = 10, warmup: int = 3) -> dict:
    """C2 through the entry TeleFuser's attention() actually calls for SAGE_ATTN_2_8_8
    (attention_impl.py:249-258): sageattn_qk_int8_pv_fp8_cuda with qk_quant_gran="per_thread" and
    pv_accum_dtype="fp32+fp32", bf16 NHD in and out, 30-layer inputs resident in HBM."""
    import torch

    from telefuser_amd import _lib
    from telefuser_amd import sageattn2 as sa
    from telefuser_amd.workloads import CONFIGS, make_inputs

    cfg = CONFIGS["c2"]
    dev = torch.device("cuda:0")
    q, k, v, _ = make_inputs(cfg, dev, call=0)
    kw = dict(tensor_layout="NHD", is_causal=False, qk_quant_gran="per_thread", pv_accum_dtype="fp32+fp32")
    for _ in range(warmup):
        sa.sageattn_qk_int8_pv_fp8_cuda(q, k, v, **kw)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        sa.sageattn_qk_int8_pv_fp8_cuda(q, k, v, **kw)
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / steps
    return {"entry": "sageattn_qk_int8_pv_fp8_cuda(qk_quant_gran='per_thread', pv_accum_dtype='fp32+fp32')",
            "workload": cfg.name, "ms_per_call": round(ms, 4), "TOPS": round(cfg.ops() / (ms * 1e-3) / 1e12, 2),
            "attn_kernel": _lib.KERNEL_NAMES.get(_lib.load().qattn_last_kernel(), "?")}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=30)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--config", default="c2")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-sdpa", action="store_true")
    ap.add_argument("--no-stream", action="store_true", help="skip the streaming KV-cache comparison")
    ap.add_argument("--no-prologue", action="store_true", help="skip the fused-prologue comparison")
    ap.add_argument("--no-configs", action="store_true", help="skip the C3 / C4 / C5 and per-thread call-path legs")
    ap.add_argument("--profile", action="store_true",
                    help="headline C2 steps only (no SDPA, streaming, prologue, config or CPU legs): for rocprofv3")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run a plain 1 GiB device copy (HBM counter calibration for rocprofv3 --pmc)")
    args = ap.parse_args()
    if args.profile:
        args.no_sdpa = args.no_stream = args.no_prologue = args.no_configs = args.no_cpu_baseline = True
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (--gpus {args.gpus} requested); the path shards "
              "per head across GPUs with no collectives inside the op", file=sys.stderr)
        return 2

    import torch

    from telefuser_amd import _lib
    from telefuser_amd import sageattn2 as sa
    from telefuser_amd.workloads import CONFIGS, make_inputs, peak_ops

    if args.calibrate_copy:
        src = torch.ones(1 << 28, dtype=torch.float32, device="cuda:0")  # 1 GiB
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"calibration": "copy", "bytes_read_per_launch": src.numel() * 4,
                          "bytes_written_per_launch": dst.numel() * 4}))
        return 0
    _lib.load()
    cfg = CONFIGS[args.config]
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    n_inputs = min(args.steps, 30)
    print(f"[bench] generating {n_inputs} input sets for {cfg.name}", file=sys.stderr, flush=True)
    inputs = [make_inputs(cfg, dev, call=i) for i in range(n_inputs)]
    torch.cuda.synchronize()
    sm_scale = cfg.D ** -0.5
    layout = "NHD"

    ev = {n: [] for n in ("attn", "quant")}
    # the drop-in's route for per-block scales: Q quantized inside the attention kernel where qattn_fwd_q16
    # covers the launch (the prologue then quantizes K and V only)
    q16 = sa.q16_supported(cfg.B, cfg.Lq, cfg.Lk, cfg.Hq, cfg.D, "per_block")

    def step(i: int, record: bool):
        q, k, v, kvv = inputs[i % n_inputs]
        if record:
            e0 = torch.cuda.Event(enable_timing=True)
            e0.record()
        q8, qs, k8, ks, _, v8, vs, _ = sa.sage_quant(q, k, v, tensor_layout=layout, sm_scale=sm_scale,
                                                     quantize_q=not q16)
        if record:
            e1 = torch.cuda.Event(enable_timing=True)
            e1.record()
            e2 = e1
        if q16:
            o = sa.qattn_fwd_q16(q, k8, ks, v8, vs, tensor_layout=layout, qk_mult=sm_scale * sa.LOG2E,
                                 kv_valid_len=kvv, qk_quant_gran="per_block")
        else:
            o = sa.qattn_fwd(q8, qs, k8, ks, v8, vs, tensor_layout=layout, out_dtype=q.dtype, kv_valid_len=kvv)
        if record:
            e3 = torch.cuda.Event(enable_timing=True)
            e3.record()
            ev["quant"].append((e0, e1))
            ev["attn"].append((e2, e3))
        return o

    for i in range(args.warmup):
        step(i, False)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        step(i, True)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    kernel_ran = _lib.KERNEL_NAMES.get(_lib.load().qattn_last_kernel(), "?")
    ms_per_step = elapsed * 1e3 / args.steps
    attn_ms = sum(a.elapsed_time(b) for a, b in ev["attn"]) / len(ev["attn"])
    quant_ms = sum(a.elapsed_time(b) for a, b in ev["quant"]) / len(ev["quant"])

    ops = cfg.ops()
    value = ops / (ms_per_step * 1e-3) / 1e12
    peak = peak_ops("fp8") / 1e12
    attn_tops = ops / (attn_ms * 1e-3) / 1e12
    q_elems = cfg.B * cfg.Lq * cfg.Hq * cfg.D
    k_elems = cfg.B * cfg.Lk * cfg.Hkv * cfg.D
    # single-pass bytes of the prologue: bf16 K, V (and Q, unless the attention kernel quantizes it) read
    # once, int8 K (Q) and e4m3 V written once
    quant_bytes = 3 * ((0 if q16 else q_elems) + 2 * k_elems)

    sdpa_ms = None
    if not args.no_sdpa:
        q, k, v, _ = inputs[0]
        qt, kt, vt = (t.transpose(1, 2).contiguous() for t in (q, k, v))
        for _ in range(2):
            torch.nn.functional.scaled_dot_product_attention(qt, kt, vt)
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(5):
            torch.nn.functional.scaled_dot_product_attention(qt, kt, vt)
        b.record()
        torch.cuda.synchronize()
        sdpa_ms = a.elapsed_time(b) / 5

    # HBM bytes per launch come from two rocprofv3 --pmc runs (FETCH_SIZE, WRITE_SIZE) of this file with
    # --profile, committed as a summary: reported with the commit and kernel they were measured on
    traffic, traffic_src = None, None
    tpath = os.path.join(ROOT, "profiles", f"attn_{args.config}_traffic.txt")
    if os.path.exists(tpath):
        with open(tpath) as f:
            tj = json.load(f)
        if tj.get("kernel") == kernel_ran:
            traffic = tj.get("hbm_bytes_per_launch")
            traffic_src = f"profiles/{tj.get('source', os.path.basename(tpath))} (measured at {tj.get('commit', '?')})"

    line = {
        "metric": "quant-attn TOPS & % MFMA peak; ms/call at Wan2.1 480p shape",
        "value": round(value, 2),
        "unit": "TOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8+fp8",
        "data": "synthetic (seeded randn bf16, RMSNorm + 3-D RoPE on q/k)",
        "config": {"workload": cfg.name, "B": cfg.B, "Lq": cfg.Lq, "Lk": cfg.Lk, "H": cfg.Hq, "D": cfg.D,
                   "causal": False, "calls": args.steps, "parallelism": "single GPU"},
        "pct_mfma_peak": round(100 * value / peak, 2),
        "roofline": {"bound": "mfma", "achieved": round(attn_tops, 2), "peak": peak, "unit": "TFLOP/s",
                     "frac": round(attn_tops / peak, 4), "traffic": traffic, "traffic_source": traffic_src,
                     "kernel": kernel_ran, "kernel_ms": round(attn_ms, 4),
                     "algorithmic_ops_per_launch": ops},
        "pre_attention": {"entry": ("qattn_sage_quant (K mean, K INT8 per block, V FP8; Q quantized inside the "
                                    "attention kernel, qattn_fwd_q16)") if q16 else
                                   "qattn_sage_quant (K mean, Q/K INT8 per block, V FP8)",
                          "kernels": "prep_col_kernel, prep_finalize_kernel, v_fp8_kernel, quant_per_block_kernel",
                          "ms": round(quant_ms, 4), "single_pass_bytes": quant_bytes,
                          "GB/s_vs_single_pass": round(quant_bytes / (quant_ms * 1e-3) / 1e9, 1), "peak_GB/s": 8000},
        "sdpa_bf16_ms": None if sdpa_ms is None else round(sdpa_ms, 4),
        "speedup_vs_sdpa": None if sdpa_ms is None else round(sdpa_ms / ms_per_step, 3),
    }
    if not args.no_configs:
        del inputs
        torch.cuda.empty_cache()
        print("[bench] TeleFuser call path (per-thread scales)", file=sys.stderr, flush=True)
        line["telefuser_call_path"] = _telefuser_call_path()
        line["configs"] = {}
        # (sub-millisecond calls get enough warm-up for the card's clock to settle: ~30 ms of work)
        for name, calls, warm in (("c3", 3, 2), ("c4", 20, 40), ("c5", 20, 40)):
            print(f"[bench] config {name}", file=sys.stderr, flush=True)
            line["configs"][name] = _config_bench(name, calls=calls, warmup=warm)
    if not args.no_stream:
        print("[bench] streaming KV-cache comparison", file=sys.stderr, flush=True)
        line["streaming_kv_cache"] = _stream_bench()
    if not args.no_prologue:
        print("[bench] fused prologue comparison", file=sys.stderr, flush=True)
        line["prologue"] = _prologue_bench()
    if not args.no_cpu_baseline:
        print("[bench] timing the CPU baseline", file=sys.stderr, flush=True)
        line["cpu_baseline"] = _cpu_baseline(cfg)
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
