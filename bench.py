"""Benchmark of the Q4_K_M x Q8 projection path on one MI355X.

Headline (BASELINE.json metric): Q4_K x Q8 decode GEMV GB/s at M=1 on config
2 (fused gate+up, N=2x17408=34816, K=5120), as a fraction of 8 TB/s HBM; the
same JSON line carries the MMQ int8-equivalent TOPS at M=512 (config 4,
Q4_K N=34816), the other decode M values, and the config-5 full-model weight
pass (64 synthetic layers, one decode step and one 512-token prefill chunk).

A "step" is one projection launch over one weight copy with the Q8
activations resident in HBM. Weight copies rotate (>= 1.2 GB in total) so
MI355X's 256 MB Infinity Cache cannot serve repeats. Weights are seeded fp32
~N(0, 0.02) quantized ON THE GPU by the library's Q4_K fitter (bit-exact with
the reference's pinned llama.cpp fitter); activations ~N(0,1) with 1% of the
channels x20, rounded to BF16 and Q8-packed by the library.

The cpu_baseline leg times the oracle's C restatement of the same contraction
(test infrastructure, OpenMP) on the host cores for a bounded sample.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
INT8_PEAK_TOPS = 5000.0   # MI355X dense int8 MFMA (AMD published)
FP16_PEAK_TFLOPS = 2500.0  # MI355X dense fp16 MFMA (AMD published)
METRIC = "Q4_K×Q8 GEMV GB/s (% of 8 TB/s) at M=1; MMQ int8 TOPS (% peak) at M=512"
# rocprofv3 --pmc summaries of the config-2 M=1 decode kernel, per weight layout:
# (file under profiles/, kernel-name prefix of the M=1 instantiation)
TRAFFIC_PROFILES = {
    0x020D: ("gemv_stream_config2_m1_traffic.txt", r"gemv_stream_kernel"),
    0x0240: ("gemv_w64_config2_m1_traffic.txt", r"gemv_w64_kernel<1,"),
}


def measured_traffic(layout):
    """HBM bytes per launch of the config-2 M=1 GEMV from the committed
    rocprofv3 --pmc summary for this layout: FETCH_SIZE and WRITE_SIZE (KiB
    per dispatch), each scaled by what the same counter reads for a device
    copy of exactly 1 GiB read + 1 GiB written. None when the summary is absent."""
    import re
    if layout not in TRAFFIC_PROFILES:
        return None
    name, kernel = TRAFFIC_PROFILES[layout]
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", name)
    try:
        text = open(path).read()
    except OSError:
        return None
    vals = {}
    for counter in ("FETCH_SIZE", "WRITE_SIZE"):
        g = re.search(kernel + r"[^\n]*\(dispatches=\d+\): " + counter + r"=([\d.e+]+)", text)
        c = re.search(r"__amd_rocclr_copyBuffer \(dispatches=\d+\): " + counter + r"=([\d.e+]+)", text)
        if not g or not c:
            return None
        scale = (1 << 20) / float(c.group(1))  # KiB the counter should read for 1 GiB
        vals[counter] = float(g.group(1)) * scale * 1024
    return {"bytes": vals["FETCH_SIZE"] + vals["WRITE_SIZE"], "read": vals["FETCH_SIZE"],
            "written": vals["WRITE_SIZE"], "source": "profiles/" + name}


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def q4k_bytes(n, k):
    return n * k // 256 * 144


def make_weight(torch, ops, n, k, seed, layout):
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    x = torch.randn(n, k, generator=g, device="cuda", dtype=torch.float32) * 0.02
    fail = torch.zeros(1, dtype=torch.int32, device="cuda")
    blocks = ops.quantize_q4k_blocks(x, n, k, fail)
    del x
    w = ops.upload_q4k_blocks(blocks, n, k, layout=layout)
    torch.cuda.synchronize()
    assert int(fail.item()) == 0
    return w, blocks


def clone_weight(ops, w):
    return ops.PrefillWeight(w.codes.clone(), w.scales.clone(), w.layout, w.quantizer, w.n, w.k,
                             w.padded_n, w.padded_k)


def make_q8(torch, ops, m, k, seed, outliers=True):
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    x = torch.randn(m, k, generator=g, device="cuda", dtype=torch.float32)
    if outliers:
        ch = torch.randperm(k, generator=g, device="cuda")[: max(1, round(0.01 * k))]
        x[:, ch] *= 20.0
    bf = x.to(torch.bfloat16).view(torch.int16).contiguous()
    q = ops.Q8Input.empty(m, k)
    fail = torch.zeros(1, dtype=torch.int32, device="cuda")
    ops.pack_q8(bf, q, fail)
    torch.cuda.synchronize()
    assert int(fail.item()) == 0
    return q, bf


def time_launches(torch, fn, copies, steps, warmup, use_graph=True):
    """Runs `steps` launches rotating over `copies`; returns (ms_per_step, mode)."""
    stream = torch.cuda.current_stream()
    for i in range(warmup):
        fn(i % copies)
    torch.cuda.synchronize()
    mode = "eager"
    graph = None
    if use_graph:
        try:
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, capture_error_mode="thread_local"):
                for i in range(copies):
                    fn(i)
            graph.replay()
            torch.cuda.synchronize()
            mode = "hipgraph"
        except Exception as e:  # fall back to eager launches
            log(f"graph capture unavailable ({e}); timing eager launches")
            graph = None
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    reps = max(1, steps // copies) if graph is not None else steps
    torch.cuda.synchronize()
    start.record(stream)
    if graph is not None:
        for _ in range(reps):
            graph.replay()
        n = reps * copies
    else:
        for i in range(steps):
            fn(i % copies)
        n = steps
    end.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(end) / n, n, mode


def bench_decode(torch, ops, n, k, ms, steps, warmup, layout, seed=11):
    wbytes = q4k_bytes(n, k)
    copies = max(2, math.ceil(1.2e9 / wbytes))
    base, _ = make_weight(torch, ops, n, k, seed, layout)
    ws = [base] + [clone_weight(ops, base) for _ in range(copies - 1)]
    res = {}
    for m in ms:
        q, _ = make_q8(torch, ops, m, k, seed + 100 + m)
        outs = [torch.empty(m, n, device="cuda") for _ in range(copies)]
        ms_step, nsteps, mode = time_launches(
            torch, lambda i: ops.q4k_q8_project(ws[i], q, outs[i]), copies, steps, warmup)
        algo = wbytes + m * k * 1.25 + m * n * 4  # weights + Q8 (1.25 B/elem) + fp32 out
        res[m] = {"ms": ms_step, "gbs": algo / (ms_step * 1e-3) / 1e9, "bytes": algo,
                  "steps": nsteps, "mode": mode}
        log(f"decode N={n} K={k} M={m}: {ms_step*1e3:.2f} us/launch, "
            f"{res[m]['gbs']:.0f} GB/s ({mode})")
    return res, base


def bench_decode_q6(torch, ops, n, k, ms, steps, warmup, seed=61):
    """Config 3: Q6_K down-projection decode (layout 0x0241) at each M in ms,
    rotating weight copies so every launch streams its weights from HBM."""
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    x = torch.randn(n, k, generator=g, device="cuda") * 0.02
    base = ops.upload_q6k_blocks(ops.quantize_q6k_blocks(x, n, k), n, k)
    del x
    wbytes = weight_bytes("q6k", n, k)
    copies = max(2, math.ceil(1.2e9 / wbytes))
    ws = [base] + [clone_weight(ops, base) for _ in range(copies - 1)]
    res = {}
    for m in ms:
        q, _ = make_q8(torch, ops, m, k, seed + 100 + m, outliers=False)
        outs = [torch.empty(m, n, device="cuda") for _ in range(copies)]
        ms_step, nsteps, mode = time_launches(
            torch, lambda i: ops.q4k_q8_project(ws[i], q, outs[i]), copies, steps, warmup)
        algo = wbytes + m * k * 1.25 + m * n * 4
        res[str(m)] = {"us": round(ms_step * 1e3, 3), "gbs": round(algo / (ms_step * 1e-3) / 1e9, 1),
                       "frac_hbm": round(algo / (ms_step * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                       "mode": mode}
        log(f"decode Q6_K N={n} K={k} M={m}: {ms_step*1e3:.2f} us/launch, "
            f"{res[str(m)]['gbs']:.0f} GB/s ({mode})")
    del ws
    return res


def bench_decode_bf16(torch, ops, n, k, steps, warmup, seed=31):
    """BF16-activation decode_mmv (Q4_K 0x020D, M=1, StoreFp32) on the config-2
    shape, rotating weight copies like the Q8 decode."""
    wbytes = q4k_bytes(n, k)
    copies = max(2, math.ceil(1.2e9 / wbytes))
    base, _ = make_weight(torch, ops, n, k, seed, 0x020D)
    ws = [base] + [clone_weight(ops, base) for _ in range(copies - 1)]
    g = torch.Generator(device="cuda")
    g.manual_seed(seed + 1)
    x = torch.randn(k, generator=g, device="cuda").to(torch.bfloat16).view(torch.int16)
    outs = [torch.empty(n, device="cuda") for _ in range(copies)]
    descs = [ops.decode_desc(ws[i], x, outs[i], ops.DECODE_STORE_FP32) for i in range(copies)]
    ms_step, nsteps, mode = time_launches(torch, lambda i: ops.decode_mmv(descs[i]), copies,
                                          steps, warmup)
    algo = wbytes + k * 2 + n * 4
    gbs = algo / (ms_step * 1e-3) / 1e9
    log(f"decode_bf16 N={n} K={k}: {ms_step*1e3:.2f} us/launch, {gbs:.0f} GB/s ({mode})")
    return {"us": round(ms_step * 1e3, 3), "gbs": round(gbs, 1),
            "frac_hbm": round(gbs / HBM_PEAK_GBS, 4), "layout": "0x020d", "steps": nsteps}


def bench_prefill_bf16(torch, ops, n, k, m, steps, warmup, seed=41):
    """BF16 PrefillEngine::project (Q4_K 0x020D operands rebuilt as BF16,
    BF16 MFMA) on the config-4 shape."""
    w, _ = make_weight(torch, ops, n, k, seed, 0x020D)
    g = torch.Generator(device="cuda")
    g.manual_seed(seed + 1)
    x = torch.randn(m, k, generator=g, device="cuda").to(torch.bfloat16).view(torch.int16)
    out = torch.empty(m, n, device="cuda")
    ms_step, nsteps, mode = time_launches(
        torch, lambda i: ops.prefill_project(w, x, m, out, ops.DECODE_STORE_FP32), 1, steps, warmup)
    tf = 2.0 * m * n * k / (ms_step * 1e-3) / 1e12
    log(f"prefill_bf16 N={n} K={k} M={m}: {ms_step*1e3:.1f} us/launch, {tf:.1f} TFLOP/s ({mode})")
    return {"us": round(ms_step * 1e3, 2), "tflops": round(tf, 1),
            "frac_bf16_mfma_peak": round(tf / FP16_PEAK_TFLOPS, 4), "m": m, "n": n, "k": k}


def bench_mmq(torch, ops, n, k, m, steps, warmup, layout, seed=21):
    w, _ = make_weight(torch, ops, n, k, seed, layout)
    q, _ = make_q8(torch, ops, m, k, seed + 1)
    out = torch.empty(m, n, device="cuda")
    ms_step, nsteps, mode = time_launches(
        torch, lambda i: ops.q4k_q8_project(w, q, out), 1, steps, warmup)
    ops_count = 2.0 * m * n * k
    tops = ops_count / (ms_step * 1e-3) / 1e12
    log(f"mmq N={n} K={k} M={m}: {ms_step*1e3:.1f} us/launch, {tops:.1f} TOPS ({mode})")
    return {"ms": ms_step, "tops": tops, "frac_int8_peak": tops / INT8_PEAK_TOPS,
            "frac_fp16_mfma_peak": tops / FP16_PEAK_TFLOPS, "steps": nsteps, "mode": mode,
            "m": m, "n": n, "k": k}


# Config 5: one layer of the synthetic 27B-class stack (out rows, in columns, format)
MODEL_LAYER = (("qkv_gate", 12288, 5120, "q4k"), ("out", 5120, 6144, "q4k"),
               ("gate_up", 34816, 5120, "q4k"), ("down", 5120, 17408, "q6k"))


def weight_bytes(fmt, n, k):
    return n * k // 256 * (144 if fmt == "q4k" else 210)


def bench_model(torch, ops, layers, q4_layout, prefill_m, reps, seed=1000):
    """Config 5: a full weight pass over `layers` synthetic layers (about
    14.5 GB of quantized weights resident in HBM at 64 layers): one decode step
    (M=1, every projection of every layer once) and one prefill chunk
    (M=prefill_m). Each (layer, projection) has its own seeded ~N(0, 0.02)
    weights, quantized on the GPU, and its own fresh seeded ~N(0,1) Q8
    activation rows. Both passes are captured in one hipGraph each and timed
    with events; the aggregate rate covers every byte / op of the pass."""
    t0 = time.perf_counter()
    g = torch.Generator(device="cuda")
    fail = torch.zeros(1, dtype=torch.int32, device="cuda")
    ws = []
    for l in range(layers):
        row = []
        for j, (name, n, k, fmt) in enumerate(MODEL_LAYER):
            g.manual_seed(seed + 16 * l + j)
            x = torch.randn(n, k, generator=g, device="cuda", dtype=torch.float32) * 0.02
            if fmt == "q4k":
                blocks = ops.quantize_q4k_blocks(x, n, k, fail)
                w = ops.upload_q4k_blocks(blocks, n, k, layout=q4_layout)
            else:
                blocks = ops.quantize_q6k_blocks(x, n, k)
                w = ops.upload_q6k_blocks(blocks, n, k)
            del x, blocks
            row.append(w)
        ws.append(row)
    torch.cuda.synchronize()
    assert int(fail.item()) == 0
    t_gen = time.perf_counter() - t0
    res = {"layers": layers, "q4k_layout": f"{q4_layout:#06x}", "q6k_layout": "0x0241",
           "weight_bytes": layers * sum(weight_bytes(f, n, k) for _, n, k, f in MODEL_LAYER),
           "setup_s": round(t_gen, 1)}
    for m in (1, prefill_m):
        qs = [[make_q8(torch, ops, m, k, seed + 7919 + 16 * l + j, outliers=False)[0]
               for j, (_, n, k, _) in enumerate(MODEL_LAYER)] for l in range(layers)]
        outs = [torch.empty(m, n, device="cuda") for _, n, _, _ in MODEL_LAYER]

        def run_pass(_i):
            for l in range(layers):
                for j in range(len(MODEL_LAYER)):
                    ops.q4k_q8_project(ws[l][j], qs[l][j], outs[j])

        ms_pass, npass, mode = time_launches(torch, run_pass, 1, reps, 1)
        nbytes = layers * sum(weight_bytes(f, n, k) + m * k * 1.25 + m * n * 4
                              for _, n, k, f in MODEL_LAYER)
        nops = layers * sum(2.0 * m * n * k for _, n, k, _ in MODEL_LAYER)
        gbs = nbytes / (ms_pass * 1e-3) / 1e9
        tops = nops / (ms_pass * 1e-3) / 1e12
        key = "decode_m1" if m == 1 else f"prefill_m{m}"
        res[key] = {"ms": round(ms_pass, 4), "gbs": round(gbs, 1),
                    "frac_hbm": round(gbs / HBM_PEAK_GBS, 4), "tops": round(tops, 2),
                    "frac_int8_peak": round(tops / INT8_PEAK_TOPS, 4),
                    "launches": layers * len(MODEL_LAYER), "passes": npass, "mode": mode}
        log(f"model pass M={m} ({layers} layers, {res['weight_bytes']/1e9:.2f} GB): "
            f"{ms_pass:.3f} ms, {gbs:.0f} GB/s, {tops:.1f} TOPS ({mode})")
        del qs, outs
    del ws
    torch.cuda.empty_cache()
    return res


def cpu_baseline(torch, blocks, n, k, m, budget_s):
    """Oracle (C restatement, OpenMP) on the host cores: same contraction."""
    import numpy as np

    import oracle
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    w = oracle.Q4K.from_ggml(blocks.cpu().numpy(), n, k)
    rng = np.random.Generator(np.random.PCG64(5))
    x = oracle.fp32_to_bf16(rng.standard_normal((m, k), dtype=np.float32))
    q = oracle.pack_q8(x, m, k)
    reps, t0 = 0, time.perf_counter()
    while True:
        oracle.q4k_q8_contract(w, q, threads=threads)
        reps += 1
        el = time.perf_counter() - t0
        if el >= budget_s:
            break
    per = el / reps
    algo = q4k_bytes(n, k) + m * k * 1.25 + m * n * 4
    return {"value": algo / per / 1e9, "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"{reps} full passes of the N={n} K={k} M={m} Q4_K x Q8 contraction "
                      f"(oracle/oracle.c, exact int32 K32 dots + affine), {el:.1f} s"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=240)
    ap.add_argument("--warmup", type=int, default=24)
    ap.add_argument("--layout", default="0x020D", help="decode weight layout")
    ap.add_argument("--mmq-layout", default="0x0240", help="MMQ weight layout")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-mmq", action="store_true")
    ap.add_argument("--no-bf16", action="store_true", help="skip the BF16-activation decode_mmv")
    ap.add_argument("--decode-m", default="1,2,4,8", help="decode token counts to time")
    ap.add_argument("--no-model", action="store_true", help="skip the config-5 model pass")
    ap.add_argument("--no-q6", action="store_true", help="skip the config-3 Q6_K decode leg")
    ap.add_argument("--model-layers", type=int, default=64)
    ap.add_argument("--model-layout", default="0x020D", help="Q4_K layout of the model pass")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a plain 1 GiB device copy (counter scale for rocprof --pmc)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only: this build has no multi-GPU path "
              f"(--gpus {args.gpus} requested); see DESIGN.md for how it would shard.",
              file=sys.stderr)
        sys.exit(2)

    import torch

    import qw38_amd.ops as ops
    torch.cuda.set_device(0)
    if args.copy_calibration:
        src = torch.empty(1 << 28, dtype=torch.float32, device="cuda").fill_(1.0)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        log("copy calibration: 5 x 1 GiB device-to-device copies done")
        return
    layout = int(args.layout, 16)
    n, k = 34816, 5120
    ms_list = [int(v) for v in args.decode_m.split(",")]
    if 1 not in ms_list:
        ms_list = [1] + ms_list
    dec, base = bench_decode(torch, ops, n, k, ms_list, args.steps, args.warmup, layout)
    head = dec[1]
    mmq_layout = int(args.mmq_layout, 16)
    mmq = None if args.no_mmq else bench_mmq(torch, ops, n, k, 512, max(20, args.steps // 8),
                                              max(3, args.warmup // 4), mmq_layout)
    q6 = None if args.no_q6 else bench_decode_q6(torch, ops, 5120, 17408, [1, 8], args.steps,
                                                 args.warmup)
    dbf16 = None if args.no_bf16 else bench_decode_bf16(torch, ops, n, k, args.steps, args.warmup)
    pbf16 = None if (args.no_bf16 or args.no_mmq) else bench_prefill_bf16(
        torch, ops, n, k, 512, max(20, args.steps // 8), max(3, args.warmup // 4))
    model = None if args.no_model else bench_model(
        torch, ops, args.model_layers, int(args.model_layout, 16), 512, 3)
    cpu = None
    if not args.no_cpu:
        _, blocks = make_weight(torch, ops, n, k, 11, layout)
        cpu = cpu_baseline(torch, blocks, n, k, 1, args.cpu_seconds)
    traffic = measured_traffic(layout)
    line = {
        "metric": METRIC,
        "value": round(head["gbs"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": head["steps"],
        "warmup": args.warmup,
        "ms_per_step": head["ms"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (seeded fp32 ~N(0,0.02) weights quantized to Q4_K on the GPU; "
                "~N(0,1) activations with 1% channels x20 -> BF16 -> Q8)",
        "config": {"workload": "config 2: fused gate+up Q4_K x Q8 decode GEMV, N=34816, "
                               "K=5120, M=1", "layout": f"{layout:#06x}",
                   "mmq_layout": f"{mmq_layout:#06x}",
                   "weight_copies_rotated": max(2, math.ceil(1.2e9 / q4k_bytes(n, k))),
                   "timing": head["mode"]},
        "roofline": {"bound": "hbm", "achieved": round(head["gbs"], 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(head["gbs"] / HBM_PEAK_GBS, 4),
                     "traffic": traffic["bytes"] if traffic else None,
                     "traffic_unit": "HBM bytes per launch (rocprofv3 FETCH_SIZE + WRITE_SIZE, "
                                     "copy-calibrated)",
                     "algorithmic_bytes": q4k_bytes(n, k) + k * 5 // 4 + n * 4},
        "decode_m": {str(m): {"gbs": round(v["gbs"], 1), "us": round(v["ms"] * 1e3, 3),
                              "frac_hbm": round(v["gbs"] / HBM_PEAK_GBS, 4)}
                     for m, v in dec.items()},
        "config3_q6k_decode": q6,
        "mmq_m512": mmq,
        "decode_bf16_m1": dbf16,
        "prefill_bf16_m512": pbf16,
        "config5_model_pass": model,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
