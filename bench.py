#!/usr/bin/env python3
"""Benchmark of the MI355X attention hot path (one GPU).

Prints ONE JSON line.  The headline workload is BASELINE.json configs[3], the
largest single-GPU configuration and the north-star prefill: causal GQA
prefill, batch 1, S=8192, 32 query / 8 KV heads, head_dim 128, with Qwen3's
per-head QK-RMSNorm (eps 1e-6, gamma ~ U(0.9, 1.1)) and RoPE (theta 1e6,
positions 0..8191) fused in front; bf16 ~ N(0,1) seeded; metric TFLOP/s with
the causal FLOP count 4*S^2*Hq*D/2 (attention only; the K pre-pass time is
inside the step).  A step is one toyinfer_prefill_qknorm_rope_attention_bf16
call over that input.  The step first runs untimed for --settle seconds (the
GPU's power controller cuts the clock for ~10-15 ms after an idle-to-MFMA
load step), then W untimed steps, then exactly K timed steps between two
device synchronisations, timed with HIP events recorded on the stream the
kernels run on.

The same line carries, under "components", the other hot-path workloads,
each with its own roofline block:
  * prefill_s1371: configs[1], S=1371, 16/8 (toyinfer_flash_attention_v1_bf16), after
    0.1 s of the same call untimed;
  * decode_b8_l4096: configs[2], split-K decode over 128 MiB of KV, HBM-bound;
  * decode_b1_l32768: the north-star 32k-token decode, 128 MiB of KV;
  * decode_step / decode_contract: the decode-step pre-pass and the
    reference-contract graph decode at the engine's cache size;
  * proj_gemv / proj_gemm: the projections either side of attention (lm-head
    GEMV, HBM-bound; a 4096-token prefill projection, MFMA-bound);
  * sample: the device top-k/top-p pick over a 151936-entry vocabulary;
  * qwen3_e2e: configs[4], random-init Qwen3-0.6B, TTFT of a 1371-token
    prompt and greedy decode tokens/s from a captured hipGraph (and the
    same with the reference's default sampling settings).
Decode steps rotate over 4 independent KV sets (512 MiB) so every step reads
KV that is not resident in the 256 MB Infinity Cache.

cpu_baseline: the CPU oracle (oracle/, the restated host reference of the
reference's tests) timed on this host's cores on a bounded, stated row
subset of the headline workload (all cores, and one core on a smaller
subset), plus the config-3 decode on the CPU; the same oracle output checks
the GPU output of those rows.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "prefill attn TFLOP/s + decode attn HBM GB/s (% MI355X roofline), Qwen3 GQA"
PEAK_BF16_TFLOPS = 2500.0   # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E
SEED = 2026
# Untimed run of the headline step before its warm-up steps, in seconds (see
# settle()): long enough for the power controller's transient to pass.
SETTLE_S = 0.3
# HBM bytes per launch of each workload's dominant kernel: rocprofv3 --pmc
# FETCH_SIZE and WRITE_SIZE passes (KiB per dispatch) over
# `bench.py --workload <name>`, scaled by what the same counters read for a
# 256 MiB device-to-device copy (reads x2.0, writes x1.0); the summaries are
# under profiles/.  (read KiB, write KiB) as the counters report them.
PMC_KIB = {"prefill": (5566.0, 5484.0),            # prefill_splitkv_pair_kernel<128,false>
           "prefill_fused": (83509.4, 65536.0),    # prefill_kernel<128,true,true>
           "decode_b8_l4096": (65844.9, 1632.0),   # decode_split_kernel<128>
           "decode_b1_l32768": (65621.3, 1632.0),  # decode_split_kernel<128>
           "proj_gemv": (607798.8, 593.5),         # gemv_kernel<8,8,1,float>
           "proj_gemm": (98404.0, 32768.0)}        # gemm_kernel<GmCfg<256,256,2,4,1,64>>
FETCH_SCALE, WRITE_SCALE = 2.0, 1.0


def traffic_bytes(workload):
    r, w = PMC_KIB[workload]
    return int(round((r * FETCH_SCALE + w * WRITE_SCALE) * 1024))
WORKLOADS = ("all", "prefill", "prefill_fused", "decode_b8_l4096", "decode_b1_l32768",
             "stream_128mib",
             "decode_step", "decode_contract", "decode_engine_lean", "proj_gemv", "proj_gemm", "qwen3_e2e",
             "sample", "copy_calibration", "torch_sdpa")


def causal_flops(s, hq, d):
    return 4.0 * s * s * hq * d / 2.0


def parse():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-components", action="store_true",
                    help="only the headline workload")
    ap.add_argument("--no-cpu", action="store_true", help="skip the cpu_baseline leg")
    ap.add_argument("--settle", type=float, default=SETTLE_S,
                    help="seconds the headline step runs untimed before its warm-up steps "
                         "(0: none)")
    ap.add_argument("--cpu-seconds", type=float, default=12.0,
                    help="target CPU time of the cpu_baseline sample")
    ap.add_argument("--workload", default="all", choices=WORKLOADS,
                    help="profiling aid: run one workload alone and print its own JSON "
                         "(the default 'all' prints the benchmark line)")
    return ap.parse_args()


def to_dev(bits, dev):
    import numpy as np
    import torch

    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16).to(dev)


def to_host(t):
    import numpy as np
    import torch

    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def settle(fn, stream, seconds):
    """Run `fn(i)` untimed for `seconds` of wall time, in bursts of 16 launches
    each followed by a device synchronisation; returns the launch count.

    After an idle-to-MFMA load step the GPU's power controller cuts the clock
    for about 10-15 ms (per-launch kernel traces of the headline show the
    prefill kernel at a constant ~7.5 M GRBM_GUI_ACTIVE cycles while its
    duration climbs from 520 to 670 us and back), so MFMA-bound steps timed
    straight after a short warm-up measure that transient, not the kernel."""
    import torch

    n, t0 = 0, time.perf_counter()
    with torch.cuda.stream(stream):
        while time.perf_counter() - t0 < seconds:
            for _ in range(16):
                fn(n)
                n += 1
            torch.cuda.synchronize()
    return n


def time_steps(fn, steps, warmup, stream):
    """Mean ms per step of `fn(i)` over `steps` launches, HIP events on `stream`."""
    import torch

    with torch.cuda.stream(stream):
        for i in range(warmup):
            fn(i)
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record(stream)
    with torch.cuda.stream(stream):
        for i in range(steps):
            fn(i)
    end.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps


def roofline(bound, achieved, peak, unit, traffic=None):
    return {"bound": bound, "achieved": round(achieved, 3), "peak": peak, "unit": unit,
            "frac": round(achieved / peak, 4), "traffic": traffic}


# ------------------------------------------------------------------ prefill

def prefill_inputs(s, hq, hkv, d, dev, seed=SEED):
    from toyinfer_amd import synth

    qb = synth.normal_bf16(seed, "q", (s, hq, d))
    kb = synth.normal_bf16(seed, "k", (s, hkv, d))
    vb = synth.normal_bf16(seed, "v", (s, hkv, d))
    return (qb, kb, vb), (to_dev(qb, dev), to_dev(kb, dev), to_dev(vb, dev))


def bench_prefill(dev, stream, steps, warmup, s=1371, hq=16, hkv=8, d=128, settle_s=0.1):
    """causal GQA prefill through toyinfer_flash_attention_v1_bf16.
    The call first runs untimed for `settle_s` seconds (see settle()): the
    component follows host-side input generation that leaves the GPU idle,
    and its 100 timed launches (about 2 ms) would otherwise fall inside the
    power controller's transient."""
    import torch

    from toyinfer_amd import attn

    _, (q, k, v) = prefill_inputs(s, hq, hkv, d, dev)
    o = torch.empty((s, hq, d), dtype=torch.bfloat16, device=dev)
    fn = lambda i: attn.flash_attention_v1_bf16(q, k, v, o, hq, hkv, d, s, stream)
    n_settle = settle(fn, stream, settle_s) if settle_s > 0 else 0
    ms = time_steps(fn, steps, warmup, stream)
    tflops = causal_flops(s, hq, d) / (ms * 1e-3) / 1e12
    return {"workload": f"prefill_causal_gqa_s{s}_hq{hq}_hkv{hkv}_d{d}",
            "entry": "toyinfer_flash_attention_v1_bf16", "steps": steps,
            "settle_s": settle_s, "settle_launches": n_settle,
            "ms_per_step": round(ms, 5), "value": round(tflops, 2), "unit": "TFLOP/s",
            "roofline": roofline("mfma", tflops, PEAK_BF16_TFLOPS, "TFLOP/s",
                                 traffic_bytes("prefill"))}


def bench_torch_sdpa(dev, stream, steps, warmup):
    """For scale, not a measurement of this library: PyTorch's own attention
    on this GPU (torch.nn.functional.scaled_dot_product_attention, is_causal,
    enable_gqa; its ROCm flash kernel) on the attention of configs[3]
    (S=8192, 32/8 heads, no QK-norm/RoPE) and configs[1] (S=1371, 16/8), with
    this library's prefill on the same inputs beside it, and on the decode
    shapes of configs[2] and the north-star decode."""
    import torch
    import torch.nn.functional as F

    from toyinfer_amd import attn

    out = {"workload": "torch_sdpa_causal_gqa_d128",
           "entry": "torch.nn.functional.scaled_dot_product_attention (for scale)"}
    for (s, hq, hkv) in ((8192, 32, 8), (1371, 16, 8)):
        _, (q, k, v) = prefill_inputs(s, hq, hkv, 128, dev)
        qt, kt, vt = (x.permute(1, 0, 2).unsqueeze(0).contiguous() for x in (q, k, v))
        ms_t = time_steps(lambda i: F.scaled_dot_product_attention(qt, kt, vt, is_causal=True,
                                                                   enable_gqa=True),
                          steps, warmup, stream)
        o = torch.empty((s, hq, 128), dtype=torch.bfloat16, device=dev)
        ms_o = time_steps(lambda i: attn.flash_attention_v1_bf16(q, k, v, o, hq, hkv, 128, s, stream),
                          steps, warmup, stream)
        fl = causal_flops(s, hq, 128)
        out[f"s{s}_hq{hq}_hkv{hkv}"] = {
            "torch_sdpa_us": round(ms_t * 1e3, 2), "torch_sdpa_tflops": round(fl / (ms_t * 1e-3) / 1e12, 1),
            "this_library_us": round(ms_o * 1e3, 2),
            "this_library_tflops": round(fl / (ms_o * 1e-3) / 1e12, 1)}
    # Decode shapes (one query row per sequence; the same KV set every call,
    # so the Infinity Cache may hold it, unlike the decode components above).
    for (b, L) in ((8, 4096), (1, 32768)):
        g = torch.Generator(device=dev).manual_seed(SEED + 61)
        qd = torch.randn((b, 32, 1, 128), generator=g, device=dev).to(torch.bfloat16)
        kd = torch.randn((b, 8, L, 128), generator=g, device=dev).to(torch.bfloat16)
        vd = torch.randn((b, 8, L, 128), generator=g, device=dev).to(torch.bfloat16)
        ms_t = time_steps(lambda i: F.scaled_dot_product_attention(qd, kd, vd, enable_gqa=True),
                          steps, warmup, stream)
        out[f"decode_b{b}_l{L}_hq32_hkv8"] = {
            "torch_sdpa_us": round(ms_t * 1e3, 2),
            "torch_sdpa_gbps": round(2.0 * b * L * 8 * 128 * 2 / (ms_t * 1e-3) / 1e9, 1)}
        del qd, kd, vd
    out["value"] = out["s8192_hq32_hkv8"]["torch_sdpa_tflops"]
    out["unit"] = "TFLOP/s"
    return out


FUSED = dict(s=8192, hq=32, hkv=8, d=128, eps=1e-6, theta=1e6)


def fused_inputs(dev, s, hq, hkv, d, theta):
    """configs[3] inputs: raw Q/K/V projections, gamma_q/gamma_k ~ U(0.9, 1.1),
    and the rotary table the model builds once (as the reference keeps
    inv_freq): host bf16 bits and device tensors."""
    import torch

    from toyinfer_amd import attn, synth

    host, (q, k, v) = prefill_inputs(s, hq, hkv, d, dev, seed=SEED + 4)
    gqb = synth.uniform_bf16(SEED + 4, "gamma_q", (d,), 0.9, 1.1)
    gkb = synth.uniform_bf16(SEED + 4, "gamma_k", (d,), 0.9, 1.1)
    f = torch.empty(d // 2, dtype=torch.float32, device=dev)
    attn.precompute_freq_f32(f, d, theta)
    table = torch.empty((s, d // 2, 2), dtype=torch.float32, device=dev)
    attn.rope_cos_sin_f32(table, f, s, d)
    torch.cuda.synchronize()
    return host + (gqb, gkb), (q, k, v, to_dev(gqb, dev), to_dev(gkb, dev), table)


def bench_prefill_fused(dev, stream, steps, warmup, settle_s=SETTLE_S):
    """the headline step (K norm+RoPE pre-pass, then attention
    with Q normalised and rotated on load).  The step first runs untimed for
    `settle_s` seconds (see settle()), then `warmup` untimed and `steps` timed
    steps.  Returns (ms, TFLOP/s, settle launches, host inputs, output bits)."""
    import torch

    from toyinfer_amd import attn

    s, hq, hkv, d = FUSED["s"], FUSED["hq"], FUSED["hkv"], FUSED["d"]
    host, (q, k, v, gq, gk, table) = fused_inputs(dev, s, hq, hkv, d, FUSED["theta"])
    o = torch.empty((s, hq, d), dtype=torch.bfloat16, device=dev)
    k_out = torch.empty_like(k)

    def step(i):
        attn.prefill_qknorm_rope_attention_bf16(q, k, v, o, k_out, gq, gk, table, FUSED["eps"],
                                                hq, hkv, d, s, stream)

    n_settle = settle(step, stream, settle_s) if settle_s > 0 else 0
    ms = time_steps(step, steps, warmup, stream)
    tflops = causal_flops(s, hq, d) / (ms * 1e-3) / 1e12
    return ms, tflops, n_settle, host, to_host(o)


# ------------------------------------------------------------------- decode

def bench_decode(dev, stream, steps, warmup, b, L, hq=32, hkv=8, d=128, sets=4):
    import torch

    from toyinfer_amd import attn, synth

    kv = []
    for r in range(sets):
        kb = synth.normal_bf16(SEED + 10 + r, "k", (b, L, hkv, d))
        vb = synth.normal_bf16(SEED + 10 + r, "v", (b, L, hkv, d))
        kv.append((to_dev(kb, dev), to_dev(vb, dev)))
    q = to_dev(synth.normal_bf16(SEED + 10, "q", (b, hq, d)), dev)
    o = torch.empty((b, hq, d), dtype=torch.bfloat16, device=dev)
    splits = attn.decode_default_splits(b, hq, hkv, d, L)
    ws = attn.decode_workspace(b, hq, d, splits, dev)

    def step(i):
        kc, vc = kv[i % sets]
        attn.decode_attention_bf16(q, kc, vc, o, b, hq, hkv, d, None, L, L * hkv * d, splits, ws,
                                   stream)

    ms = time_steps(step, steps, warmup, stream)
    kv_bytes = 2.0 * b * L * hkv * d * 2
    gbs = kv_bytes / (ms * 1e-3) / 1e9
    return {"workload": f"decode_b{b}_l{L}_hq{hq}_hkv{hkv}_d{d}",
            "entry": "toyinfer_decode_attention_bf16", "splits": splits, "steps": steps,
            "ms_per_step": round(ms, 5), "value": round(gbs, 1), "unit": "GB/s",
            "note": "KV bytes read per step / step time (split + combine kernels); "
                    f"{sets} rotating KV sets defeat the Infinity Cache",
            "roofline": roofline("hbm", gbs, PEAK_HBM_GBS, "GB/s",
                                 traffic_bytes(f"decode_b{b}_l{L}"))}


def bench_decode_step(dev, stream, steps, warmup, hq=32, hkv=8, d=128, msl=40960, pos=4095):
    """Decode-step pre-pass for one token (Qwen3-8B geometry): the fused
    norm + RoPE + cache-write pass against the six drop-in ops of
    src/transformer.cpp:535-552 on the same stream.  Both are launch-latency
    bound (a few KiB move); the figure of merit is time per step."""
    import torch

    from toyinfer_amd import attn, synth

    q = to_dev(synth.normal_bf16(SEED + 20, "q", (hq, d)), dev)
    k = to_dev(synth.normal_bf16(SEED + 20, "k", (hkv, d)), dev)
    v = to_dev(synth.normal_bf16(SEED + 20, "v", (hkv, d)), dev)
    gq = to_dev(synth.uniform_bf16(SEED + 20, "gq", (d,), 0.9, 1.1), dev)
    gk = to_dev(synth.uniform_bf16(SEED + 20, "gk", (d,), 0.9, 1.1), dev)
    inv = torch.empty(d // 2, dtype=torch.float32, device=dev)
    attn.precompute_freq_f32(inv, d, 1e6)
    kc = torch.zeros((msl, hkv, d), dtype=torch.bfloat16, device=dev)
    vc = torch.zeros_like(kc)
    pos_d = torch.tensor([pos], dtype=torch.int32, device=dev)
    qo = torch.empty_like(q)

    def fused(i):
        attn.decode_qkv_prologue_bf16(q, k, v, gq, gk, inv, pos_d, msl, 1e-6, qo, kc, vc, hq, hkv, d,
                                      stream)

    def six(i):
        attn.multi_rmsnorm_bf16(q, gq, qo, 1e-6, hq, d, stream)
        attn.multi_rmsnorm_bf16(k, gk, k, 1e-6, hkv, d, stream)
        attn.rope_bf16_graph(qo, inv, pos_d, hq, d, stream)
        attn.rope_bf16_graph(k, inv, pos_d, hkv, d, stream)
        attn.write_kv_cache_bf16(k, kc, pos_d, hkv * d, stream)
        attn.write_kv_cache_bf16(v, vc, pos_d, hkv * d, stream)

    ms_f = time_steps(fused, steps, warmup, stream)
    ms_6 = time_steps(six, steps, warmup, stream)
    moved = (2 * hq * d + 2 * hkv * d * 2) * 2 + d * 2 * 2 + d * 2
    return {"workload": f"decode_step_prologue_hq{hq}_hkv{hkv}_d{d}",
            "entry": "toyinfer_decode_qkv_prologue_bf16", "steps": steps,
            "ms_per_step": round(ms_f, 5), "value": round(ms_f * 1e3, 2), "unit": "us/step",
            "higher_is_better": False, "six_op_sequence_us": round(ms_6 * 1e3, 2),
            "note": f"one token: {moved} bytes move, so both paths are launch-latency bound; "
                    "six_op_sequence_us = the reference's six launches through this library"}


def bench_decode_contract(dev, stream, steps, warmup, hq=32, hkv=8, d=128, msl=40960, pos=32767,
                          per_graph=12, lean=False):
    """The reference-contract decode the engine calls (attention_bf16_graph:
    device position, score/O_buffer/O outputs, captured in a graph) at a 32k
    position of a 40960-row cache; each replay runs `per_graph` calls.  With
    lean=True the same call site through attention_bf16_graph_lean (score as
    scratch, no probabilities)."""
    import torch

    from toyinfer_amd import attn, synth

    sets = 4  # rotating caches (4 x 168 MB) so no call finds its cache in the Infinity Cache
    kv = [(to_dev(synth.normal_bf16(SEED + 30 + r, "k", (msl, hkv, d)), dev),
           to_dev(synth.normal_bf16(SEED + 30 + r, "v", (msl, hkv, d)), dev)) for r in range(sets)]
    q = to_dev(synth.normal_bf16(SEED + 30, "q", (hq, d)), dev)
    score = torch.empty((hq, msl), dtype=torch.float32, device=dev)
    ob = torch.empty((hq, d), dtype=torch.float32, device=dev)
    o = torch.empty((hq, d), dtype=torch.bfloat16, device=dev)
    pos_d = torch.tensor([pos], dtype=torch.int32, device=dev)
    call = attn.attention_bf16_graph_lean if lean else attn.attention_bf16_graph
    with torch.cuda.stream(stream):
        call(q, kv[0][0], kv[0][1], score, ob, o, hq, hkv, d, pos_d, msl, stream)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        for c in range(per_graph):
            kc, vc = kv[c % sets]
            call(q, kc, vc, score, ob, o, hq, hkv, d, pos_d, msl, stream)
    ms = time_steps(lambda i: graph.replay(), max(5, steps // per_graph), warmup, stream) / per_graph
    kv_bytes = 2.0 * (pos + 1) * hkv * d * 2
    gbs = kv_bytes / (ms * 1e-3) / 1e9
    if lean:
        return {"workload": f"decode_engine_lean_graph_msl{msl}_pos{pos}_hq{hq}_hkv{hkv}_d{d}",
                "entry": "toyinfer_attention_bf16_graph_lean", "steps": steps,
                "ms_per_step": round(ms, 5), "value": round(gbs, 1), "unit": "GB/s",
                "note": "KV bytes attended per call / call time; O and O_buffer written, "
                        "score used as scratch (the engine never reads it)",
                "roofline": roofline("hbm", gbs, PEAK_HBM_GBS, "GB/s")}
    return {"workload": f"decode_contract_graph_msl{msl}_pos{pos}_hq{hq}_hkv{hkv}_d{d}",
            "entry": "toyinfer_attention_bf16_graph", "steps": steps,
            "ms_per_step": round(ms, 5), "value": round(gbs, 1), "unit": "GB/s",
            "note": "KV bytes attended per call / call time; the call also writes the "
                    f"{hq}x{msl} fp32 probability rows the contract requires (from raw "
                    "scores the split pass stores when the rows past pos hold its partials, "
                    "else re-reading K), O_buffer and O",
            "roofline": roofline("hbm", gbs, PEAK_HBM_GBS, "GB/s")}


def bench_proj_gemv(dev, stream, steps, warmup, M=151936, N=4096):
    """The lm-head projection of one decoded token (gemv_proj_bf162float,
    src/transformer.cpp:630) at Qwen3-8B's vocabulary x hidden size: 1.16 GiB
    of bf16 weights streamed once per call, HBM-bound."""
    import torch

    from toyinfer_amd import attn

    g = torch.Generator(device=dev).manual_seed(SEED + 40)
    w = torch.randn((M, N), generator=g, device=dev).to(torch.bfloat16)
    x = torch.randn((N,), generator=g, device=dev).to(torch.bfloat16)
    y = torch.empty((M,), dtype=torch.float32, device=dev)
    ms = time_steps(lambda i: attn.gemv_proj_bf162float(w, x, y, M, N, stream), steps, warmup,
                    stream)
    nbytes = 2.0 * M * N + 2.0 * N + 4.0 * M
    gbs = nbytes / (ms * 1e-3) / 1e9
    return {"workload": f"proj_gemv_lmhead_m{M}_n{N}", "entry": "toyinfer_gemv_proj_bf162float",
            "steps": steps, "ms_per_step": round(ms, 5), "value": round(gbs, 1), "unit": "GB/s",
            "note": "weights + x read, fp32 y written, per call / call time",
            "roofline": roofline("hbm", gbs, PEAK_HBM_GBS, "GB/s", traffic_bytes("proj_gemv"))}


def bench_stream_128mib(dev, stream, steps, warmup, sets=4, M=16384, N=4096):
    """For scale beside the decode workloads: this library's most efficient
    streaming kernel, the lm-head GEMV (gemv_proj_bf162float), over exactly
    the decode step's 128 MiB (M x N bf16 weights, as many bytes as the K/V
    of configs[2]), rotating `sets` weight sets as the decode bench rotates
    its K/V sets.  It reads the same bytes and does almost nothing else, so
    its step time bounds what a one-pass decode over 128 MiB can reach on
    this GPU."""
    import torch

    from toyinfer_amd import attn

    g = torch.Generator(device=dev).manual_seed(SEED + 41)
    ws = [torch.randn((M, N), generator=g, device=dev).to(torch.bfloat16) for _ in range(sets)]
    x = torch.randn((N,), generator=g, device=dev).to(torch.bfloat16)
    y = torch.empty((M,), dtype=torch.float32, device=dev)
    ms = time_steps(lambda i: attn.gemv_proj_bf162float(ws[i % sets], x, y, M, N, stream), steps,
                    warmup, stream)
    nbytes = 2.0 * M * N
    gbs = nbytes / (ms * 1e-3) / 1e9
    return {"workload": f"stream_128MiB_gemv_m{M}_n{N}", "entry": "toyinfer_gemv_proj_bf162float",
            "steps": steps, "ms_per_step": round(ms, 5), "value": round(gbs, 1), "unit": "GB/s",
            "note": "for scale: 128 MiB of weights streamed once per call (the decode step's K/V "
                    f"bytes), {sets} rotating sets; weight bytes / call time",
            "roofline": roofline("hbm", gbs, PEAK_HBM_GBS, "GB/s")}


def bench_proj_gemm(dev, stream, steps, warmup, T=4096, M=4096, N=4096):
    """A prefill projection (batch_gemv_proj_bf16, src/transformer.cpp:370-378)
    over 4096 tokens of Qwen3-8B's hidden size: the MFMA GEMM.  The note
    carries torch.matmul (hipBLASLt) on the same operands for scale."""
    import torch

    from toyinfer_amd import attn

    g = torch.Generator(device=dev).manual_seed(SEED + 41)
    w = torch.randn((M, N), generator=g, device=dev).to(torch.bfloat16)
    x = torch.randn((T, N), generator=g, device=dev).to(torch.bfloat16)
    y = torch.empty((T, M), dtype=torch.bfloat16, device=dev)
    ms = time_steps(lambda i: attn.batch_gemv_proj_bf16(w, x, y, T, M, N, stream), steps, warmup,
                    stream)
    ms_lib = time_steps(lambda i: torch.matmul(x, w.t()), steps, warmup, stream)
    tf = 2.0 * T * M * N / (ms * 1e-3) / 1e12
    return {"workload": f"proj_gemm_t{T}_m{M}_n{N}", "entry": "toyinfer_batch_gemv_proj_bf16",
            "steps": steps, "ms_per_step": round(ms, 5), "value": round(tf, 1),
            "unit": "TFLOP/s", "torch_matmul_tflops": round(2.0 * T * M * N / (ms_lib * 1e-3) / 1e12, 1),
            "roofline": roofline("mfma", tf, PEAK_BF16_TFLOPS, "TFLOP/s", traffic_bytes("proj_gemm"))}


def bench_qwen3_e2e(dev, prompt_len=1371, decode_steps=256, reps=3):
    """Configuration 5: random-init Qwen3-0.6B (28 layers, hidden 1024, 16/8
    heads, D=128, SwiGLU 3072, vocab 151936, tied embeddings; bf16 weights
    N(0, 0.02) seeded, norms 1), prefill of `prompt_len` random token ids, then
    `decode_steps` greedy steps replayed from one captured hipGraph.  TTFT =
    prefill through the lm-head and the greedy pick of the first token; both
    timed with HIP events on the model's stream (best of `reps`)."""
    import torch

    from toyinfer_amd import qwen3

    cfg = dict(num_layers=28, hidden_size=1024, num_q_heads=16, num_kv_heads=8, head_dim=128,
               intermediate_size=3072, vocab_size=151936,
               max_seq_len=prompt_len + decode_steps + 8, max_prefill_tokens=prompt_len,
               rms_norm_eps=1e-6, rope_theta=1e6)
    g = torch.Generator(device=dev).manual_seed(SEED + 50)

    def rnd(shape):
        return (torch.randn(shape, generator=g, device=dev) * 0.02).to(torch.bfloat16)

    shapes = qwen3.layer_shapes(qwen3.Config(**cfg))
    w = {"layers": [{n: (torch.ones(shp, dtype=torch.bfloat16, device=dev) if len(shp) == 1
                         else rnd(shp)) for n, shp in shapes.items()}
                    for _ in range(cfg["num_layers"])]}
    w["embed_tokens"] = rnd((cfg["vocab_size"], cfg["hidden_size"]))
    w["lm_head"] = w["embed_tokens"]
    w["norm"] = torch.ones(cfg["hidden_size"], dtype=torch.bfloat16, device=dev)
    ids = torch.randint(0, cfg["vocab_size"], (prompt_len,), generator=g, device=dev,
                        dtype=torch.int32)
    m = qwen3.Qwen3(qwen3.Config(**cfg), w)
    torch.cuda.synchronize()
    ms_stream = torch.cuda.ExternalStream(m.stream_ptr, device=dev)
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(4)]
    ttft, dec = [], []
    for _ in range(reps):
        ev[0].record(ms_stream)
        m.prefill(ids, prompt_len)
        ev[1].record(ms_stream)
        m.decode(decode_steps, True)
        ev[2].record(ms_stream)
        m.synchronize()
        ttft.append(ev[0].elapsed_time(ev[1]))
        dec.append(ev[1].elapsed_time(ev[2]))
    direct = []
    m.prefill(ids, prompt_len)
    ev[0].record(ms_stream)
    m.decode(32, False)
    ev[1].record(ms_stream)
    m.synchronize()
    direct.append(ev[0].elapsed_time(ev[1]) / 32)
    # The reference's default sampler settings, sampled on the device in the graph.
    m.set_sampling(0.6, 20, 0.95, SEED)
    sampled = []
    for _ in range(reps):
        m.prefill(ids, prompt_len)
        ev[0].record(ms_stream)
        m.decode(decode_steps, True)
        ev[1].record(ms_stream)
        m.synchronize()
        sampled.append(ev[0].elapsed_time(ev[1]) / decode_steps)
    m.close()
    ms_tok = min(dec) / decode_steps
    return {"workload": f"qwen3_0.6b_e2e_prompt{prompt_len}_decode{decode_steps}",
            "entry": "toyinfer_qwen3_prefill / toyinfer_qwen3_decode (hipGraph)",
            "ttft_ms": round(min(ttft), 3), "decode_ms_per_token": round(ms_tok, 4),
            "value": round(1e3 / ms_tok, 1), "unit": "decode tokens/s",
            "direct_launch_ms_per_token": round(direct[0], 4),
            "sampled_decode_ms_per_token": round(min(sampled), 4),
            "note": "random-init weights N(0, 0.02) bf16 (synthetic), tied embeddings; "
                    "TTFT includes the lm-head and the device greedy pick"}


def bench_sample(dev, stream, steps, warmup, V=151936, T=0.6, top_k=20, top_p=0.95):
    """The token pick after the lm-head with the reference's default sampler
    settings (src/options.cpp:32-34): top-k/top-p sampling on the device
    (toyinfer_sample_topk_topp_f32) over fp32 logits N(0, 3^2) of Qwen3's
    vocabulary; the greedy pick (toyinfer_argmax_f32's wide form, same entry
    at temperature 0) timed beside it.  Launch-latency bound: the roofline
    prices the 0.6 MB logits read."""
    import torch

    from toyinfer_amd import attn

    g = torch.Generator(device=dev).manual_seed(SEED + 60)
    logits = torch.randn((V,), generator=g, device=dev) * 3.0
    coin = torch.full((1,), 0.37, dtype=torch.float32, device=dev)
    out = torch.zeros(1, dtype=torch.int32, device=dev)
    ws = torch.zeros(attn.sample_workspace_bytes(), dtype=torch.uint8, device=dev)
    torch.cuda.synchronize()
    ms = time_steps(lambda i: attn.sample_topk_topp_f32(logits, V, T, top_k, top_p, coin, out, ws,
                                                        stream), steps, warmup, stream)
    ms_greedy = time_steps(lambda i: attn.sample_topk_topp_f32(logits, V, 0.0, top_k, top_p, coin,
                                                               out, ws, stream), steps, warmup,
                           stream)
    gbs = 4.0 * V / (ms * 1e-3) / 1e9
    return {"workload": f"sample_topk{top_k}_topp{top_p}_t{T}_v{V}",
            "entry": "toyinfer_sample_topk_topp_f32", "steps": steps,
            "us_per_call": round(ms * 1e3, 2), "greedy_us_per_call": round(ms_greedy * 1e3, 2),
            "value": round(gbs, 1), "unit": "GB/s",
            "note": "logits read per call / call time; launch-latency bound at this size",
            "roofline": roofline("hbm", gbs, PEAK_HBM_GBS, "GB/s")}


def bench_copy(dev, stream, steps, warmup, mib=256):
    """Device-to-device copy of `mib` MiB: a kernel with known HBM traffic (mib
    read + mib written per launch), the scale for the FETCH_SIZE / WRITE_SIZE
    counters of the attention kernels."""
    import torch

    x = torch.ones(mib << 18, dtype=torch.float32, device=dev)
    y = torch.empty_like(x)
    ms = time_steps(lambda i: y.copy_(x), steps, warmup, stream)
    nbytes = 2.0 * (mib << 20)
    return {"workload": f"copy_{mib}MiB", "steps": steps, "ms_per_step": round(ms, 5),
            "value": round(nbytes / (ms * 1e-3) / 1e9, 1), "unit": "GB/s",
            "note": "read + write bytes / step time"}


# ------------------------------------------------------------- CPU baseline

def _subset_rows(s, stride):
    """First and last 64 rows plus every `stride`-th row (deterministic)."""
    return sorted(set(range(min(64, s))) | set(range(max(0, s - 64), s)) | set(range(0, s, stride)))


def _cpu_fused_rows(host, rows, threads):
    """The oracle's config-3 path on `rows`: K norm -> bf16 -> RoPE -> bf16 on
    every row (each query row reads all earlier keys), the same on Q for the
    listed rows only (their own positions), then causal attention for those
    rows (fp64 scores and softmax, fp32 P.V).  Returns float32 [S][Hq][D]
    with the listed rows filled."""
    import numpy as np

    import oracle

    qb, kb, vb, gqb, gkb = host
    s, hq, d = qb.shape
    eps, theta = FUSED["eps"], FUSED["theta"]
    inv = oracle.inv_freq(d, theta)
    gq, gk = oracle.bf16_to_f32(gqb), oracle.bf16_to_f32(gkb)
    kr = oracle.qk_norm_rope(oracle.bf16_to_f32(kb), gk, inv, eps)
    qr = np.zeros((s, hq, d), np.float32)
    qf = oracle.bf16_to_f32(qb[rows])
    for j, r in enumerate(rows):
        qr[r] = oracle.rope(oracle.multi_rmsnorm(qf[j], gq, d, eps), inv, 1, hq, d, pos0=r)
    return oracle.flash_reference(qr, kr, oracle.bf16_to_f32(vb), rows=rows, nthreads=threads)


def cpu_baseline(host, gpu_out, budget_s):
    """The oracle on this host's cores: the headline workload on a row
    subset, all cores (repeated to ~budget_s/2) and one core (a sparser
    subset), plus config 3's decode; the all-core output checks the GPU's
    rows."""
    import numpy as np

    import oracle

    threads = len(os.sched_getaffinity(0))
    s, hq, d = FUSED["s"], FUSED["hq"], FUSED["d"]

    def flops(rows):
        return sum(4.0 * (r + 1) * d * hq for r in rows)

    rows = _subset_rows(s, 61)
    t0 = time.perf_counter()
    ref = _cpu_fused_rows(host, rows, threads)
    reps, el = 1, time.perf_counter() - t0
    while el < budget_s / 2 and reps < 16:
        _cpu_fused_rows(host, rows, threads)
        reps += 1
        el = time.perf_counter() - t0
    tf_all = flops(rows) * reps / el / 1e12
    got = (gpu_out[rows].astype(np.uint32) << 16).view(np.float32)
    diff = np.abs(got - oracle.round_bf16(ref[rows]))

    rows1 = list(range(0, s, 122))
    t0 = time.perf_counter()
    _cpu_fused_rows(host, rows1, 1)
    el1 = time.perf_counter() - t0
    tf_one = flops(rows1) / el1 / 1e12

    # configs[2] decode (B=8, L=4096, 32/8), the full workload.
    from toyinfer_amd import synth

    b, L, dhq, dhkv = 8, 4096, 32, 8
    qb = synth.normal_bf16(SEED + 10, "q", (b, dhq, d))
    kb = synth.normal_bf16(SEED + 10, "k", (b, L, dhkv, d))
    vb = synth.normal_bf16(SEED + 10, "v", (b, L, dhkv, d))
    kv_bytes = 2.0 * b * L * dhkv * d * 2
    dec = {}
    for n in (threads, 1):
        t0 = time.perf_counter()
        oracle.decode_batched(qb, kb, vb, [L] * b, nthreads=n)
        reps_d, eld = 1, time.perf_counter() - t0
        while eld < 1.0 and reps_d < 32:
            oracle.decode_batched(qb, kb, vb, [L] * b, nthreads=n)
            reps_d += 1
            eld = time.perf_counter() - t0
        dec[n] = kv_bytes * reps_d / eld / 1e9
    return {"value": round(tf_all, 6), "unit": "TFLOP/s", "cores": threads, "kind": "port",
            "sample": f"headline workload (S={s}, {hq}/8 heads, D={d}, QK-norm + RoPE) on "
                      f"{len(rows)} query rows (first and last 64 plus every 61st) of all "
                      f"heads, x {reps} runs, {el:.1f} s, {threads} OpenMP threads; the oracle: "
                      "K norm/RoPE on all rows, Q's on those rows, fp64 scores and softmax, fp32 "
                      "P.V; FLOPs = 4*(i+1)*D*Hq summed over those rows",
            "single_core": {"value": round(tf_one, 6), "unit": "TFLOP/s", "cores": 1,
                            "sample": f"{len(rows1)} query rows (every 122nd), {el1:.1f} s"},
            "decode_b8_l4096": {"unit": "GB/s", "value": round(dec[threads], 2),
                                "cores": threads, "single_core_value": round(dec[1], 2),
                                "sample": "configs[2] full workload (KV bytes / time), fp32 "
                                          "scores, softmax and P.V"},
            "parity_vs_gpu": {"rows": len(rows), "max_abs": float(diff.max()),
                              "mean_abs": float(diff.mean())}}


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only: bench.py --gpus 1 "
                                   "(sharding across GPUs is designed, not implemented)"}))
        sys.exit(2)
    import torch

    from toyinfer_amd import attn  # noqa: F401  (fails loudly if the HIP library is missing)

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    stream = torch.cuda.Stream(device=dev)
    comp = {
        "prefill": lambda: bench_prefill(dev, stream, max(50, args.steps * 5), 20),
        "decode_b8_l4096": lambda: bench_decode(dev, stream, max(50, args.steps * 2), 10,
                                                b=8, L=4096),
        "decode_b1_l32768": lambda: bench_decode(dev, stream, max(50, args.steps * 2), 10,
                                                 b=1, L=32768),
        "decode_step": lambda: bench_decode_step(dev, stream, max(50, args.steps * 2), 10),
        "decode_contract": lambda: bench_decode_contract(dev, stream, max(50, args.steps * 2), 2),
        "decode_engine_lean": lambda: bench_decode_contract(dev, stream, max(50, args.steps * 2),
                                                            2, lean=True),
        "proj_gemv": lambda: bench_proj_gemv(dev, stream, max(50, args.steps), 10),
        "proj_gemm": lambda: bench_proj_gemm(dev, stream, max(200, args.steps), 50),
        "stream_128mib": lambda: bench_stream_128mib(dev, stream, max(50, args.steps * 2), 10),
        "sample": lambda: bench_sample(dev, stream, max(200, args.steps), 50),
        "qwen3_e2e": lambda: bench_qwen3_e2e(dev),
        "torch_sdpa": lambda: bench_torch_sdpa(dev, stream, 20, 3),
        "copy_calibration": lambda: bench_copy(dev, stream, args.steps, args.warmup),
    }
    if args.workload != "all":
        if args.workload == "prefill_fused":
            ms, tf, n_settle, _, _ = bench_prefill_fused(dev, stream, args.steps, args.warmup,
                                                         args.settle)
            out = {"workload": "prefill_fused_qknorm_rope_s8192_hq32_hkv8_d128",
                   "ms_per_step": round(ms, 5), "value": round(tf, 2), "unit": "TFLOP/s",
                   "settle_launches": n_settle}
        else:
            out = comp[args.workload]()
        print(json.dumps(out), flush=True)
        return

    s, hq, hkv, d = FUSED["s"], FUSED["hq"], FUSED["hkv"], FUSED["d"]
    ms, tflops, n_settle, host, gpu_out = bench_prefill_fused(dev, stream, args.steps,
                                                              args.warmup, args.settle)
    line = {
        "metric": METRIC, "value": round(tflops, 2), "unit": "TFLOP/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic: bf16 N(0,1) from seed 2030 (SplitMix64 + Box-Muller), "
                "gamma ~ U(0.9, 1.1)",
        "config": {"workload": "prefill_fused_qknorm_rope_s8192_hq32_hkv8_d128", "batch": 1,
                   "seq_len": s, "num_q_heads": hq, "num_kv_heads": hkv, "head_dim": d,
                   "qk_norm_eps": FUSED["eps"], "rope_theta": FUSED["theta"],
                   "flops_per_step": causal_flops(s, hq, d), "accumulate": "fp32",
                   "entry": "toyinfer_prefill_qknorm_rope_attention_bf16",
                   "note": "step = K norm+RoPE pre-pass + attention; FLOPs count attention only; "
                           f"before the {args.warmup} warm-up and {args.steps} timed steps the "
                           f"same step ran untimed for {args.settle:g} s ({n_settle} launches, "
                           "the GPU's power-controller transient after an idle-to-MFMA load "
                           "step); nothing else ran before it",
                   "parallelism": "single GPU"},
        "roofline": roofline("mfma", tflops, PEAK_BF16_TFLOPS, "TFLOP/s",
                             traffic_bytes("prefill_fused")),
    }
    if not args.no_components:
        line["components"] = [comp[n]() for n in
                              ("prefill", "decode_b8_l4096", "decode_b1_l32768", "stream_128mib",
                               "decode_step",
                               "decode_contract", "decode_engine_lean", "proj_gemv",
                               "proj_gemm", "sample",
                               "qwen3_e2e", "torch_sdpa")]
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(host, gpu_out, args.cpu_seconds)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
