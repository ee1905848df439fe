"""Benchmark of the Q4_K_M x Q8 projection path on one MI355X.

Headline (BASELINE.json metric): Q4_K x Q8 decode GEMV GB/s at M=1 on config
2 (fused gate+up, N=2x17408=34816, K=5120), as a fraction of 8 TB/s HBM; the
same JSON line carries the MMQ int8-equivalent TOPS at M=512 (config 4,
Q4_K N=34816), the other decode M values, and the config-5 full-model weight
pass (64 synthetic layers, one decode step and one 512-token prefill chunk).

A "step" is one rotation over the rotated weight copies of the headline
shape: one projection launch per copy (12 launches over 1.2 GB for config 2),
with the Q8 activations resident in HBM. Copies rotate (>= 1.2 GB in total) so
MI355X's 256 MB Infinity Cache cannot serve repeats; every leg times at least
100 launches. Weights are seeded fp32
~N(0, 0.02) quantized ON THE GPU by the library's Q4_K fitter (bit-exact with
the reference's pinned llama.cpp fitter); activations ~N(0,1) with 1% of the
channels x20, rounded to BF16 and Q8-packed by the library.

The cpu_baseline leg compiles oracle/cpu_baseline.c (the reference's closed-form
contraction as an FP32 CPU kernel over the packed GGML blocks, test
infrastructure) with -O3 -march=native -fopenmp on the host that runs the
bench and times it on the host cores for a bounded sample.
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
    # sections start at their "command:" line; the kernel's value comes from the
    # section that profiled the decode leg, the copy's from --copy-calibration
    sections = re.split(r"(?m)^(?=command:)", text)
    vals = {}
    for counter in ("FETCH_SIZE", "WRITE_SIZE"):
        g = c = None
        for sec in sections:
            head = sec.split("\n", 1)[0]
            if not head.startswith("command:") or ("--pmc " + counter) not in head:
                continue
            if "--copy-calibration" in head:
                c = c or re.search(r"__amd_rocclr_copyBuffer[^\n]*\(dispatches=\d+\):[^\n]*\b" + counter +
                                   r"=([\d.e+]+)", sec)
            else:
                g = g or re.search(kernel + r"[^\n]*\(dispatches=\d+\):[^\n]*\b" + counter + r"=([\d.e+]+)", sec)
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


def time_launches(torch, fn, copies, steps, warmup, use_graph=True, min_launches=100):
    """Times launches of fn(i) rotating over `copies` inputs.

    One rotation (fn(0) .. fn(copies-1), one launch per weight copy) is
    captured in a hipGraph. `warmup` untimed replays, then the timed region
    replays the rotation `steps` times, or more when needed to reach
    `min_launches` launches (rounded up to whole rotations), bracketed by HIP
    events recorded on the launch stream. Returns (ms per launch, launches
    timed, rotations timed, mode)."""
    stream = torch.cuda.current_stream()
    mode = "eager"
    graph = None
    for i in range(copies):  # first calls outside capture (lazy set-up)
        fn(i)
    torch.cuda.synchronize()
    if use_graph:
        try:
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, capture_error_mode="thread_local"):
                for i in range(copies):
                    fn(i)
            torch.cuda.synchronize()
            mode = "hipgraph"
        except Exception as e:  # fall back to eager launches
            log(f"graph capture unavailable ({e}); timing eager launches")
            graph = None
    rot = max(steps, -(-min_launches // copies))
    for _ in range(max(1, warmup)):
        if graph is not None:
            graph.replay()
        else:
            for i in range(copies):
                fn(i)
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record(stream)
    for _ in range(rot):
        if graph is not None:
            graph.replay()
        else:
            for i in range(copies):
                fn(i)
    end.record(stream)
    torch.cuda.synchronize()
    n = rot * copies
    return start.elapsed_time(end) / n, n, rot, mode


def time_both(torch, fn, copies, steps, warmup, min_launches=100):
    """Times the same launch rotation twice: replayed from a hipGraph
    (time_launches) and as eager stream launches (the same number of launches,
    bracketed by events on the launch stream). Graph replay adds a gap of
    about 2 us between kernel nodes on this ROCm, and eager launches are
    host-bound when a call's host cost exceeds its kernel time, so the lower
    of the two device times is reported, with both recorded. Returns
    (ms per launch, launches, rotations, mode, {graph_us, eager_us})."""
    g_ms, n, rot, g_mode = time_launches(torch, fn, copies, steps, warmup, min_launches=min_launches)
    stream = torch.cuda.current_stream()
    for _ in range(max(1, warmup)):
        for i in range(copies):
            fn(i)
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record(stream)
    for _ in range(rot):
        for i in range(copies):
            fn(i)
    end.record(stream)
    torch.cuda.synchronize()
    e_ms = start.elapsed_time(end) / n
    extra = {"graph_us": round(g_ms * 1e3, 3), "eager_us": round(e_ms * 1e3, 3)}
    if e_ms < g_ms:
        return e_ms, n, rot, "eager", extra
    return g_ms, n, rot, g_mode, extra


def time_eager(torch, fn, copies, launches):
    """Eager (no graph) launches rotating over copies: device time per launch
    from events on the launch stream, and host wall time per call."""
    stream = torch.cuda.current_stream()
    for i in range(copies):
        fn(i)
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record(stream)
    t0 = time.perf_counter()
    for i in range(launches):
        fn(i % copies)
    host = (time.perf_counter() - t0) / launches
    end.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(end) / launches, host * 1e3


def hbm_roofline(nbytes, ms, **extra):
    gbs = nbytes / (ms * 1e-3) / 1e9
    return {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(gbs / HBM_PEAK_GBS, 4), "us": round(ms * 1e3, 3),
            "algorithmic_bytes": int(nbytes), **extra}


def mfma_roofline(nops, ms, peak_sclk=None, **extra):
    tops = nops / (ms * 1e-3) / 1e12
    r = {"bound": "mfma", "achieved": round(tops, 1), "peak": INT8_PEAK_TOPS, "unit": "TOPS",
         "frac": round(tops / INT8_PEAK_TOPS, 4), "us": round(ms * 1e3, 2),
         "ops": int(nops), "frac_fp16_mfma_peak": round(tops / FP16_PEAK_TFLOPS, 4), **extra}
    if peak_sclk:
        r["peak_at_measured_sclk"] = round(peak_sclk, 1)
        r["frac_at_measured_sclk"] = round(tops / peak_sclk, 4)
    return r


def weight_bytes(fmt, n, k):
    return n * k // 256 * (144 if fmt == "q4k" else 210)


def make_any_weight(torch, ops, fmt, n, k, seed, layout):
    if fmt == "q4k":
        return make_weight(torch, ops, n, k, seed, layout)
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    x = torch.randn(n, k, generator=g, device="cuda") * 0.02
    blocks = ops.quantize_q6k_blocks(x, n, k)
    del x
    w = ops.upload_q6k_blocks(blocks, n, k)
    torch.cuda.synchronize()
    return w, blocks


def bench_decode(torch, ops, fmt, n, k, ms, steps, warmup, layout, seed, outliers=True,
                 eager_m1=False):
    """Decode GEMV at each M in ms, rotating >= 1.2 GB of weight copies so every
    launch streams its weights from HBM. Returns {M: hbm roofline entry}."""
    wbytes = weight_bytes(fmt, n, k)
    copies = max(2, math.ceil(1.2e9 / wbytes))
    base, _ = make_any_weight(torch, ops, fmt, n, k, seed, layout)
    ws = [base] + [clone_weight(ops, base) for _ in range(copies - 1)]
    res = {}
    for m in ms:
        q, _ = make_q8(torch, ops, m, k, seed + 100 + m, outliers=outliers)
        outs = [torch.empty(m, n, device="cuda") for _ in range(copies)]
        fn = lambda i: ops.q4k_q8_project(ws[i], q, outs[i])  # noqa: E731
        ms_launch, launches, rot, mode, both = time_both(torch, fn, copies, steps, warmup)
        algo = wbytes + m * k * 1.25 + m * n * 4  # weights + Q8 (1.25 B/elem) + fp32 out
        res[m] = hbm_roofline(algo, ms_launch, launches=launches, rotations=rot, copies=copies,
                              timing=mode, **both)
        if eager_m1 and m == 1:
            dev_ms, host_ms = time_eager(torch, fn, copies, 600)
            res[m]["eager_us_per_launch"] = round(dev_ms * 1e3, 3)
            res[m]["eager_host_us_per_call"] = round(host_ms * 1e3, 3)
        log(f"decode {fmt} N={n} K={k} M={m}: {ms_launch*1e3:.2f} us/launch, "
            f"{res[m]['achieved']:.0f} GB/s ({mode}, {launches} launches)")
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
    ms_launch, launches, _, mode = time_launches(torch, lambda i: ops.decode_mmv(descs[i]), copies,
                                                 steps, warmup)
    r = hbm_roofline(wbytes + k * 2 + n * 4, ms_launch, launches=launches, layout="0x020d",
                     timing=mode)
    log(f"decode_bf16 N={n} K={k}: {ms_launch*1e3:.2f} us/launch, {r['achieved']:.0f} GB/s ({mode})")
    del ws
    return r


def bench_decode_head(torch, ops, steps, warmup, seed=51):
    """decode_mmv on the reference's vocabulary head geometry (Q8G32 dense
    tiles 0x0202, N=248320, K=5120, M=1, BF16 input, StoreFp32;
    cuda/decode_mmv.cu:548-553): 1.35 GB of seeded random codes and small
    positive fp16 group scales, larger than the Infinity Cache, so one copy
    streams from HBM on every launch. Timing only; the head's parity is a GPU
    test at N=65536."""
    n, k = 248320, 5120
    pn, pk = ops.pad_n(n), ops.pad_k(k)
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    codes = torch.randint(0, 256, (pn * pk,), generator=g, dtype=torch.uint8, device="cuda")
    scales = (torch.rand(pn * pk // 32, generator=g, device="cuda") * 1e-3 + 1e-4).to(torch.float16)
    w = ops.dense_weight(0x0202, codes, scales.view(torch.uint8), n, k)
    x = torch.randn(k, generator=g, device="cuda").to(torch.bfloat16).view(torch.int16)
    y = torch.empty(n, device="cuda")
    d = ops.decode_desc(w, x, y, ops.DECODE_STORE_FP32)
    ms_launch, launches, _, mode, both = time_both(torch, lambda i: ops.decode_mmv(d), 1, steps, warmup)
    nbytes = codes.numel() + scales.numel() * 2 + k * 2 + n * 4
    r = hbm_roofline(nbytes, ms_launch, launches=launches, layout="0x0202", timing=mode, **both)
    log(f"decode head Q8G32 N={n} K={k}: {ms_launch*1e3:.2f} us/launch, {r['achieved']:.0f} GB/s ({mode})")
    del codes, scales, w
    return r


def bench_prefill_bf16(torch, ops, n, k, m, steps, warmup, seed=41):
    """BF16 PrefillEngine::project (Q4_K 0x020D operands rebuilt as BF16,
    BF16 MFMA) on the config-4 shape."""
    w, _ = make_weight(torch, ops, n, k, seed, 0x020D)
    g = torch.Generator(device="cuda")
    g.manual_seed(seed + 1)
    x = torch.randn(m, k, generator=g, device="cuda").to(torch.bfloat16).view(torch.int16)
    out = torch.empty(m, n, device="cuda")
    ms_launch, launches, _, mode = time_launches(
        torch, lambda i: ops.prefill_project(w, x, m, out, ops.DECODE_STORE_FP32), 1, steps, warmup)
    tf = 2.0 * m * n * k / (ms_launch * 1e-3) / 1e12
    log(f"prefill_bf16 N={n} K={k} M={m}: {ms_launch*1e3:.1f} us/launch, {tf:.1f} TFLOP/s ({mode})")
    return {"bound": "mfma", "achieved": round(tf, 1), "peak": FP16_PEAK_TFLOPS, "unit": "TFLOP/s",
            "frac": round(tf / FP16_PEAK_TFLOPS, 4), "us": round(ms_launch * 1e3, 2),
            "launches": launches, "m": m, "n": n, "k": k}


def bench_mmq(torch, ops, shapes, steps, warmup, layout, peak_sclk, seed=21):
    """Config 4: MMQ at each (format, N, K, M); weights resident (the MMQ is
    MFMA-bound: 2*M*N*K ops against the int8 dense peak)."""
    res = {}
    for fmt, n, k, mlist in shapes:
        w, _ = make_any_weight(torch, ops, fmt, n, k, seed + n, layout)
        for m in mlist:
            q, _ = make_q8(torch, ops, m, k, seed + 1 + m, outliers=(fmt == "q4k"))
            out = torch.empty(m, n, device="cuda")
            ms_launch, launches, _, mode = time_launches(
                torch, lambda i: ops.q4k_q8_project(w, q, out), 1, steps, warmup)
            key = f"{fmt}_n{n}_k{k}_m{m}"
            res[key] = mfma_roofline(2.0 * m * n * k, ms_launch, peak_sclk, launches=launches,
                                     layout=f"{w.layout:#06x}", timing=mode)
            log(f"mmq {key}: {ms_launch*1e3:.1f} us/launch, {res[key]['achieved']:.1f} TOPS ({mode})")
            del q, out
        del w
    return res


def bench_mlp(torch, ops, layouts, steps, warmup, peak_sclk, seed=500):
    """The whole Q8 MLP (q4k_q8_mlp: RMS->Q8, gate+up, SwiGLU->Q8, down +
    residual; Q4_K gate/up 17408x5120, Q6_K down 5120x17408) at M=1 on the
    decode layout and M=512 on the MMQ layout, timed replayed from a hipGraph
    (with the device failure flag, as a captured decode token runs it) and as
    eager launches (time_both). Beside it
    the unfused chain of the same stages as separate launches (two FP32
    [m][17408] slabs and a standalone SwiGLU->Q8 pack); both end in the same
    bits."""
    res = {}
    for m, layout in ((1, layouts[0]), (512, layouts[1])):
        gate, _ = make_any_weight(torch, ops, "q4k", 17408, 5120, seed, layout)
        up, _ = make_any_weight(torch, ops, "q4k", 17408, 5120, seed + 1, layout)
        down, _ = make_any_weight(torch, ops, "q6k", 5120, 17408, seed + 2, 0x0241)
        g = torch.Generator(device="cuda")
        g.manual_seed(seed + 3)
        resid = torch.randn(m, 5120, generator=g, device="cuda")
        gamma = (0.1 * torch.randn(5120, generator=g, device="cuda")).to(torch.bfloat16).view(torch.int16)
        ws = torch.zeros(ops.q8_mlp_workspace_bytes(m), dtype=torch.uint8, device="cuda")
        flag = torch.zeros(1, dtype=torch.int32, device="cuda")
        out = torch.empty(m, 5120, device="cuda")
        ms_f, launches, _, mode, both = time_both(
            torch, lambda i: ops.q4k_q8_mlp(gate, up, down, resid, gamma, 1e-6, out, m, ws,
                                            pending_failure=flag), 1, steps, warmup)
        fused_out = out.clone()
        qx = ops.Q8Input.empty(m, 5120)
        qh = ops.Q8Input.empty(m, 17408)
        gs = torch.empty(m, 17408, device="cuda")
        us = torch.empty(m, 17408, device="cuda")
        out2 = torch.empty(m, 5120, device="cuda")

        def chain(_i):
            ops.hidden_rms_q8(resid, gamma, 1e-6, m, qx, flag)
            ops.q4k_q8_project(gate, qx, gs)
            ops.q4k_q8_project(up, qx, us)
            ops.swiglu_q8(gs, us, m, 17408, qh, flag)
            ops.q4k_q8_project(down, qh, out2, residual=resid)

        ms_c, _, _, _, _ = time_both(torch, chain, 1, steps, warmup)
        torch.cuda.synchronize()
        same = bool(torch.equal(fused_out, out2))
        nops = 2.0 * m * 5120 * (3 * 17408)
        nbytes = 2 * q4k_bytes(17408, 5120) + weight_bytes("q6k", 5120, 17408)
        key = f"mlp_m{m}"
        res[key] = {"us": round(ms_f * 1e3, 2), "unfused_chain_us": round(ms_c * 1e3, 2),
                    "layout": f"{layout:#06x}", "down": "q6k 0x0241", "launches": launches,
                    "timing": mode, **both, "equals_unfused": same}
        if m == 1:
            res[key]["weight_gbs"] = round(nbytes / (ms_f * 1e-3) / 1e9, 1)
        else:
            res[key]["tops"] = round(nops / (ms_f * 1e-3) / 1e12, 1)
            res[key]["frac_int8_peak_at_sclk"] = round(nops / (ms_f * 1e-3) / 1e12 / peak_sclk, 4)
        log(f"mlp m={m}: {ms_f*1e3:.1f} us (unfused chain {ms_c*1e3:.1f} us), equal {same} ({mode})")
        del gate, up, down, ws, gs, us
    return res


# Config 5: one layer of the synthetic 27B-class stack (out rows, in columns, format)
MODEL_LAYER = (("qkv_gate", 12288, 5120, "q4k"), ("out", 5120, 6144, "q4k"),
               ("gate_up", 34816, 5120, "q4k"), ("down", 5120, 17408, "q6k"))


def bench_model(torch, ops, layers, q4_layout, prefill_m, reps, peak_sclk, seed=1000):
    """Config 5: a full weight pass over `layers` synthetic layers (about
    14.5 GB of quantized weights resident in HBM at 64 layers): one decode step
    (M=1, every projection of every layer once) and one prefill chunk
    (M=prefill_m). Each (layer, projection) has its own seeded ~N(0, 0.02)
    weights, quantized on the GPU, and its own fresh seeded ~N(0,1) Q8
    activation rows. Each pass is timed with events both replayed from one
    hipGraph and as eager launches (time_both). After timing, the last layer's four projections are re-run eagerly
    and must equal the graph-replay outputs bitwise (the oracle parity of the
    same pass is a GPU test)."""
    t0 = time.perf_counter()
    ws = []
    for l in range(layers):
        row = []
        for j, (name, n, k, fmt) in enumerate(MODEL_LAYER):
            w, blocks = make_any_weight(torch, ops, fmt, n, k, seed + 16 * l + j, q4_layout)
            del blocks
            row.append(w)
        ws.append(row)
    torch.cuda.synchronize()
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

        ms_pass, npass, _, mode, both = time_both(torch, run_pass, 1, reps, 1, min_launches=1)
        same = True
        for j, (_, n, _, _) in enumerate(MODEL_LAYER):
            again = torch.empty(m, n, device="cuda")
            ops.q4k_q8_project(ws[-1][j], qs[-1][j], again)
            torch.cuda.synchronize()
            same = same and bool(torch.equal(again, outs[j]))
        nbytes = layers * sum(weight_bytes(f, n, k) + m * k * 1.25 + m * n * 4
                              for _, n, k, f in MODEL_LAYER)
        nops = layers * sum(2.0 * m * n * k for _, n, k, _ in MODEL_LAYER)
        key = "decode_m1" if m == 1 else f"prefill_m{m}"
        entry = (hbm_roofline(nbytes, ms_pass) if m == 1 else mfma_roofline(nops, ms_pass, peak_sclk))
        entry.update({"ms": round(ms_pass, 4), "launches": layers * len(MODEL_LAYER),
                      "passes": npass, "timing": mode, "replay_equals_eager": same,
                      "graph_ms": round(both["graph_us"] / 1e3, 4), "eager_ms": round(both["eager_us"] / 1e3, 4)})
        res[key] = entry
        log(f"model pass M={m} ({layers} layers, {res['weight_bytes']/1e9:.2f} GB): "
            f"{ms_pass:.3f} ms, {entry['achieved']} {entry['unit']} ({mode}), replay==eager {same}")
        del qs, outs
    del ws
    torch.cuda.empty_cache()
    return res


def read_probe(torch, nbytes, copies, steps, warmup, points=None):
    """Pure-read ceiling (qw38_read_probe) for a launch that reads `nbytes`:
    grid-stride and per-wave contiguous ranges (8 or 16 loads in flight), each
    at 2 / 4 / 8 blocks of 256 threads per CU, rotating over `copies` buffers
    (beyond the Infinity Cache) like the decode legs; >= 100 launches per
    point, timed like the decode legs (the lower of hipGraph replay and eager
    launches). Returns the best GB/s and every point."""
    from qw38_amd._lib import lib
    nb = nbytes // 1024 * 1024
    buf = torch.empty(copies, nb, dtype=torch.uint8, device="cuda")
    buf.random_(0, 256)
    sink = torch.zeros(8 * 1024, dtype=torch.int32, device="cuda")
    pts = {}
    for mode, name in ((0, "grid_stride"), (1, "wave_ranges"), (2, "wave_ranges16"), (3, "wave_ranges_nt")):
        for bpc in (2, 4, 8):
            if points is not None and (mode, bpc) not in points:
                continue
            def fn(i, mode=mode, bpc=bpc):  # on the current stream (the capture stream inside a graph)
                st = lib().qw38_read_probe(buf[i].data_ptr(), nb, mode, bpc, sink.data_ptr(), sink.numel(),
                                           torch.cuda.current_stream().cuda_stream)
                assert st == 0
            ms, n, _, how, extra = time_both(torch, fn, copies, steps, warmup)
            pts[f"{name}_{bpc}"] = {"us": round(ms * 1e3, 3), "GBps": round(nb / (ms * 1e-3) / 1e9, 1),
                                    "launches": n, "timing": how, **extra}
    best = max(pts, key=lambda k: pts[k]["GBps"])
    del buf
    torch.cuda.empty_cache()
    r = {"bytes": nb, "copies": copies, "best": best, "best_GBps": pts[best]["GBps"],
         "best_frac_of_8TBps": round(pts[best]["GBps"] / HBM_PEAK_GBS, 4), "points": pts}
    log(f"read probe: {r}")
    return r


def clock_probe(torch, ops):
    """Shader clock under a full int8 MFMA load (qw38_mfma_clock_probe) and the
    int8 dense peak at that clock: CUs x 8192 ops/cycle x sclk."""
    import ctypes as C

    from qw38_amd._lib import lib
    ticks = torch.zeros(4, dtype=torch.int64, device="cuda")
    blocks = C.c_uint32(0)
    iters = 40000
    stream = torch.cuda.current_stream()
    for _ in range(2):
        st = lib().qw38_mfma_clock_probe(iters, ticks.data_ptr(), C.byref(blocks), stream.cuda_stream)
        assert st == 0
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record(stream)
    lib().qw38_mfma_clock_probe(iters, ticks.data_ptr(), C.byref(blocks), stream.cuda_stream)
    end.record(stream)
    torch.cuda.synchronize()
    ms = start.elapsed_time(end)
    cyc, rt = (int(v) for v in ticks[:2].cpu())
    sclk = cyc / (rt / 100e6) if rt else float("nan")
    cus = blocks.value
    loop_ops = cus * 4 * iters * 4 * 32 * 32 * 32 * 2.0
    r = {"sclk_mhz": round(sclk / 1e6, 1), "cus": cus,
         "int8_peak_tops_at_sclk": round(cus * 8192 * sclk / 1e12, 1),
         "pure_mfma_loop_tops": round(loop_ops / (ms * 1e-3) / 1e12, 1)}
    log(f"clock probe: {r}")
    return r


def issue_probe(torch):
    """VALU / matrix-core overlap on one SIMD (qw38_issue_probe, two waves per
    SIMD), timed with events: nanoseconds per loop iteration of 32 FP16
    16x16x32 MFMAs alone, 128 FP32 FMAs alone, both interleaved 1:4, 16
    MFMAs with 128 FMAs interleaved 1:8, and one MFMA-only wave (16) beside
    one FMA-only wave (64) per SIMD; and 32 int8 16x16x32 / 16x16x64 MFMAs
    alone; 'overlap' is the fraction of the
    shorter unit's time hidden under the other's (1 = fully hidden, 0 =
    serialized)."""
    from qw38_amd._lib import lib
    ticks = torch.zeros(2, dtype=torch.int64, device="cuda")
    sink = torch.zeros(1, dtype=torch.float32, device="cuda")
    iters = 20000
    ns = {}
    stream = torch.cuda.current_stream()
    for mode in range(7):
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        for rep in range(2):  # the second launch is the one timed
            if rep:
                start.record(stream)
            st = lib().qw38_issue_probe(mode, iters, ticks.data_ptr(), sink.data_ptr(), stream.cuda_stream)
            assert st == 0
        end.record(stream)
        torch.cuda.synchronize()
        ns[mode] = start.elapsed_time(end) * 1e6 / iters
    mf, va = ns[0], ns[1]  # 32 MFMAs, 128 FMAs per SIMD and iteration

    def ov(t, m, v):
        return round((m + v - t) / min(m, v), 3)
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    r = {"ns_per_iter": {"mfma32": round(mf, 1), "fma128": round(va, 1), "mix_1to4": round(ns[2], 1),
                         "mix_1to8_16mfma": round(ns[3], 1), "split_waves_16mfma_64fma": round(ns[4], 1),
                         "i8_16x16x32_32": round(ns[5], 1), "i8_16x16x64_32": round(ns[6], 1)},
         "overlap_1to4": ov(ns[2], mf, va), "overlap_1to8": ov(ns[3], mf / 2, va),
         "overlap_split_waves": ov(ns[4], mf / 2, va / 2),
         "mfma_only_fp16_tflops": round(cus * 4 * 32 * 16384 / mf / 1e3, 1)}
    log(f"issue probe: {r}")
    return r


def cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(torch, blocks, n, k, m, budget_s):
    """oracle/cpu_baseline.c compiled here with -O3 -march=native -fopenmp
    (FP32 closed-form contraction straight from the packed GGML blocks, rows
    in parallel) on the config-2 M=1 workload: median of >= 5 full passes."""
    import ctypes as C
    import subprocess
    import tempfile

    import numpy as np

    import oracle
    src = os.path.join(ROOT, "oracle", "cpu_baseline.c")
    so = os.path.join(tempfile.mkdtemp(prefix="qw38_cpub_"), "libcpu_baseline.so")
    cmd = ["gcc", "-O3", "-march=native", "-fopenmp", "-fPIC", "-shared", "-o", so, src]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        log(f"cpu baseline build failed: {r.stderr[-400:]}")
        return None
    L = C.CDLL(so)
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    gb = np.ascontiguousarray(blocks.cpu().numpy(), np.uint8)
    rng = np.random.Generator(np.random.PCG64(5))
    x = rng.standard_normal((m, k), dtype=np.float32)
    x[:, rng.choice(k, k // 100, replace=False)] *= 20
    q = oracle.pack_q8(oracle.fp32_to_bf16(x), m, k)
    out = np.zeros((m, n), np.float32)
    P = lambda a: a.ctypes.data_as(C.c_void_p)  # noqa: E731
    args = (P(gb), n, k, P(q.codes), P(q.scales), P(q.sums), m, P(out), threads)
    L.cpub_q4k.argtypes = [C.c_void_p, C.c_uint32, C.c_uint32, C.c_void_p, C.c_void_p, C.c_void_p,
                           C.c_uint32, C.c_void_p, C.c_int]
    times, t_all = [], time.perf_counter()
    while len(times) < 5 or time.perf_counter() - t_all < budget_s:
        t0 = time.perf_counter()
        assert L.cpub_q4k(*args) == 0
        times.append(time.perf_counter() - t0)
    med = float(np.median(times))
    algo = q4k_bytes(n, k) + m * k * 1.25 + m * n * 4
    return {"value": round(algo / med / 1e9, 2), "unit": "GB/s", "cores": threads, "kind": "port",
            "cpu_model": cpu_model(), "nproc": os.cpu_count(),
            "omp_num_threads": os.environ.get("OMP_NUM_THREADS"),
            "build": "gcc -O3 -march=native -fopenmp oracle/cpu_baseline.c",
            "sample": f"median of {len(times)} full passes ({time.perf_counter() - t_all:.1f} s) of "
                      f"the config-2 workload N={n} K={k} M={m}: FP32 closed-form contraction "
                      "over the packed Q4_K blocks, exact int32 K32 dots, rows in parallel"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20, help="timed rotations of the headline leg")
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--layout", default="0x020D", help="decode weight layout")
    ap.add_argument("--mmq-layout", default="0x020D", help="MMQ weight layout")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-mmq", action="store_true")
    ap.add_argument("--no-bf16", action="store_true", help="skip the BF16-activation decode_mmv")
    ap.add_argument("--decode-m", default="1,2,4,8", help="decode token counts to time")
    ap.add_argument("--no-model", action="store_true", help="skip the config-5 model pass")
    ap.add_argument("--no-mlp", action="store_true", help="skip the whole-MLP leg")
    ap.add_argument("--no-q6", action="store_true", help="skip the config-3 Q6_K decode leg")
    ap.add_argument("--q6-decode-m", default="1,8", help="config-3 token counts to time")
    ap.add_argument("--no-config1", action="store_true")
    ap.add_argument("--mmq-shapes", default="all", help="'all' (config 4) or 'headline'")
    ap.add_argument("--model-layers", type=int, default=64)
    ap.add_argument("--model-layout", default="0x020D", help="Q4_K layout of the model pass")
    ap.add_argument("--eager-leg", default=None, metavar="FMT:N:K:M:CALLS",
                    help="only run CALLS eager projections of one shape (q4k on --layout, q6k on "
                         "0x0241, over 12 rotated weight copies; bf16: the BF16 prefill projection "
                         "over Q4_K 0x020D), for rocprofv3 traces and counters")
    ap.add_argument("--mlp-leg", default=None, metavar="M:CALLS",
                    help="only run CALLS eager whole-MLP calls at M tokens (Q4_K gate/up on --layout "
                         "for M <= 8, else --mmq-layout; Q6_K down), for rocprofv3 traces")
    ap.add_argument("--no-read-probe", action="store_true", help="skip the pure-read ceiling leg")
    ap.add_argument("--issue-probe-only", action="store_true",
                    help="only the VALU / matrix-core overlap probe")
    ap.add_argument("--read-probe-only", action="store_true",
                    help="only run the pure-read ceiling leg (for rocprofv3 traces)")
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
    mmq_layout = int(args.mmq_layout, 16)
    if args.eager_leg:
        fmt, n_, k_, m_, calls = args.eager_leg.split(":")
        n_, k_, m_, calls = int(n_), int(k_), int(m_), int(calls)
        if fmt == "bf16":  # BF16 PrefillEngine projection over Q4_K 0x020D
            w, _ = make_weight(torch, ops, n_, k_, 11, 0x020D)
            x = torch.randn(m_, k_, device="cuda").to(torch.bfloat16).view(torch.int16)
            out = torch.empty(m_, n_, device="cuda")
            for i in range(calls):
                ops.prefill_project(w, x, m_, out, ops.DECODE_STORE_FP32)
            torch.cuda.synchronize()
            log(f"eager leg {args.eager_leg}: done")
            return
        w, _ = make_any_weight(torch, ops, fmt, n_, k_, 11, layout if fmt == "q4k" else 0x0241)
        ws = [w] + [clone_weight(ops, w) for _ in range(11)]
        q, _ = make_q8(torch, ops, m_, k_, 5, outliers=(fmt == "q4k"))
        out = torch.empty(m_, n_, device="cuda")
        for i in range(calls):
            ops.q4k_q8_project(ws[i % len(ws)], q, out)
        torch.cuda.synchronize()
        log(f"eager leg {args.eager_leg}: done")
        return
    if args.mlp_leg:
        m_, calls = (int(v) for v in args.mlp_leg.split(":"))
        lay = layout if m_ <= 8 else mmq_layout
        gate, _ = make_any_weight(torch, ops, "q4k", 17408, 5120, 500, lay)
        up, _ = make_any_weight(torch, ops, "q4k", 17408, 5120, 501, lay)
        down, _ = make_any_weight(torch, ops, "q6k", 5120, 17408, 502, 0x0241)
        resid = torch.randn(m_, 5120, device="cuda")
        gamma = torch.zeros(5120, dtype=torch.int16, device="cuda")
        ws = torch.zeros(ops.q8_mlp_workspace_bytes(m_), dtype=torch.uint8, device="cuda")
        out = torch.empty(m_, 5120, device="cuda")
        for _ in range(calls):
            ops.q4k_q8_mlp(gate, up, down, resid, gamma, 1e-6, out, m_, ws)
        torch.cuda.synchronize()
        log(f"mlp leg {args.mlp_leg}: done")
        return
    n, k = 34816, 5120
    ms_list = sorted({1, *[int(v) for v in args.decode_m.split(",")]})
    clock = clock_probe(torch, ops)
    peak_sclk = clock["int8_peak_tops_at_sclk"]
    if args.read_probe_only:
        read_probe(torch, 100_270_080, 12, args.steps, args.warmup)
        return
    issue = issue_probe(torch)
    if args.issue_probe_only:
        return
    probe = None if args.no_read_probe else read_probe(torch, 100_270_080, 12, args.steps, args.warmup)
    if probe:  # the same ceiling at the config-1 and config-3 weight sizes
        few = {(0, 4), (1, 8), (2, 8)}
        probe["config1_weights"] = read_probe(torch, 14_745_600, 82, args.steps, args.warmup, few)
        probe["config3_weights"] = read_probe(torch, 73_113_600, 17, args.steps, args.warmup, few)
    rooflines = {}
    dec = bench_decode(torch, ops, "q4k", n, k, ms_list, args.steps, args.warmup, layout, 11,
                       eager_m1=True)
    head = dec[1]
    for m, v in dec.items():
        rooflines[f"config2_m{m}"] = v
    if not args.no_config1:
        c1 = bench_decode(torch, ops, "q4k", 5120, 5120, [1], args.steps, args.warmup, layout, 71,
                          outliers=False)
        rooflines["config1_m1"] = c1[1]
    if not args.no_q6:
        c3 = bench_decode(torch, ops, "q6k", 5120, 17408, [int(v) for v in args.q6_decode_m.split(",")],
                          args.steps, args.warmup, 0x0241, 61, outliers=False)
        for m, v in c3.items():
            rooflines[f"config3_m{m}"] = v
    if not args.no_mmq:
        shapes = ([("q4k", 34816, 5120, [512])] if args.mmq_shapes == "headline" else
                  [("q4k", 12288, 5120, [128, 512, 2048]), ("q4k", 34816, 5120, [128, 512, 2048]),
                   ("q6k", 5120, 17408, [128, 512, 2048])])
        mmq = bench_mmq(torch, ops, shapes, args.steps, args.warmup, mmq_layout, peak_sclk)
        for key, v in mmq.items():
            rooflines["config4_" + key] = v
    if not args.no_bf16:
        rooflines["decode_bf16_config2_m1"] = bench_decode_bf16(torch, ops, n, k, args.steps,
                                                                args.warmup)
        rooflines["decode_q8g32_head_m1"] = bench_decode_head(torch, ops, args.steps, args.warmup)
        if not args.no_mmq:
            rooflines["prefill_bf16_config4_m512"] = bench_prefill_bf16(
                torch, ops, n, k, 512, args.steps, args.warmup)
    mlp = None if args.no_mlp else bench_mlp(torch, ops, (layout, mmq_layout), args.steps,
                                             args.warmup, peak_sclk)
    model = None if args.no_model else bench_model(
        torch, ops, args.model_layers, int(args.model_layout, 16), 512, 3, peak_sclk)
    if model:
        rooflines["config5_decode_m1"] = model["decode_m1"]
        rooflines["config5_prefill_m512"] = model["prefill_m512"]
    cpu = None
    if not args.no_cpu:
        _, blocks = make_weight(torch, ops, n, k, 11, layout)
        cpu = cpu_baseline(torch, blocks, n, k, 1, args.cpu_seconds)
    traffic = measured_traffic(layout)
    rot_bytes = head["algorithmic_bytes"] * head["copies"]
    line = {
        "metric": METRIC,
        "value": head["achieved"],
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": head["rotations"],
        "warmup": args.warmup,
        "ms_per_step": round(rot_bytes / (head["achieved"] * 1e9) * 1e3, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (seeded fp32 ~N(0,0.02) weights quantized to Q4_K on the GPU; "
                "~N(0,1) activations with 1% channels x20 -> BF16 -> Q8)",
        "config": {"workload": "config 2: fused gate+up Q4_K x Q8 decode GEMV, N=34816, "
                               "K=5120, M=1; one step = one launch on each of "
                               f"{head['copies']} rotated weight copies",
                   "layout": f"{layout:#06x}", "mmq_layout": f"{mmq_layout:#06x}",
                   "weight_copies_rotated": head["copies"], "launches_timed": head["launches"],
                   "us_per_launch": head["us"], "timing": head["timing"]},
        "roofline": {"bound": "hbm", "achieved": head["achieved"], "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": head["frac"],
                     "traffic": traffic["bytes"] if traffic else None,
                     "traffic_unit": "HBM bytes per launch (rocprofv3 FETCH_SIZE + WRITE_SIZE, "
                                     "copy-calibrated)",
                     "algorithmic_bytes": head["algorithmic_bytes"],
                     "read_ceiling_GBps": probe["best_GBps"] if probe else None,
                     "frac_of_read_ceiling": round(head["achieved"] / probe["best_GBps"], 4) if probe else None},
        "read_probe": probe,
        "rooflines": rooflines,
        "mfma_clock": clock,
        "issue_probe": issue,
        "config5_model_pass": model,
        "mlp": mlp,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
