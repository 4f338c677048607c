#!/usr/bin/env python3
"""bf16 GEMM throughput on one MI355X through libt0g's C ABI.

One step = one C = A*B GEMM (bf16 in, fp32 accumulate, bf16 out, row-major NN)
at configs[1] of BASELINE.json, M = N = K = 4096, inputs N(0,1)*0.02 resident in HBM.
Prints ONE JSON line.  Besides `value` (TFLOPS of the timed steps) the line
carries the dominant kernel's roofline (HIP events on the stream the kernels
run on), the other benchmark configurations under "extra", and the CPU oracle timed on
this host under "cpu_baseline".
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "t0-gpu_amd"))

METRIC = "bf16 GEMM TFLOPS at 4096³ and 8192³ on 1 MI355X; % of dense bf16 MFMA peak"
PEAK_TFLOPS = 2500.0    # MI355X dense bf16 MFMA
PEAK_GBS = 8000.0       # MI355X HBM3E
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "traffic.json")


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def make_inputs(torch, m, n, k, layout, seed, dist="normal"):
    """A and B as stored for `layout`: N(0,1)*0.02 (the square configs) or, with
    dist="uniform", U(-0.5, 0.5) (the thin configs), rounded to bf16."""
    g = torch.Generator(device="cuda").manual_seed(seed)
    a_shape = (m, k) if layout in ("NT", "NN") else (k, m)
    b_shape = (n, k) if layout in ("NT", "TT") else (k, n)
    if dist == "uniform":
        a = (torch.rand(a_shape, generator=g, device="cuda") - 0.5).to(torch.bfloat16)
        b = (torch.rand(b_shape, generator=g, device="cuda") - 0.5).to(torch.bfloat16)
    else:
        a = (torch.randn(a_shape, generator=g, device="cuda") * 0.02).to(torch.bfloat16)
        b = (torch.randn(b_shape, generator=g, device="cuda") * 0.02).to(torch.bfloat16)
    return a, b


WARM_MIN_MS = 200.0


def _warm(torch, launch, count, min_ms=WARM_MIN_MS):
    """`count` untimed launches, then more until at least min_ms of load has run: the
    shader clock of a power-limited MI355X keeps rising for ~0.2 s under load (4096^3
    NN: 101.6 us per launch after 20 ms of warm-up, 99.8 us after 0.2 s and after 1 s),
    so a line timed earlier reads a few percent below the steady state a training loop
    runs at.  The timed region is still exactly the requested launches."""
    t0 = time.perf_counter()
    for _ in range(count):
        launch()
    torch.cuda.synchronize()
    while (time.perf_counter() - t0) * 1e3 < min_ms:
        for _ in range(8):
            launch()
        torch.cuda.synchronize()


def time_gemm(t0g, torch, rt, stream, m, n, k, layout, steps, warmup, seed=2, out=None, epilogue_ops=None,
              config=None, dist="normal"):
    a, b = make_inputs(torch, m, n, k, layout, seed, dist)
    c = torch.empty((m, n), dtype=torch.bfloat16, device="cuda")
    bias = torch.linspace(-1.0, 1.0, n, device="cuda", dtype=torch.float32)
    desc = t0g.gemm_desc(a.data_ptr(), b.data_ptr(), c.data_ptr(), m, n, k, transpose=layout, out_dtype=t0g.BF16,
                         epilogue_ops=epilogue_ops, bias=bias.data_ptr() if epilogue_ops else 0, config=config)
    kname = t0g.gemm_kernel_name(desc)
    _warm(torch, lambda: rt.gemm_desc(desc), warmup)
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    t_start = time.perf_counter()
    e0.record(stream)
    for _ in range(steps):
        rt.gemm_desc(desc)
    e1.record(stream)
    torch.cuda.synchronize()
    wall_s = time.perf_counter() - t_start
    ev_ms = e0.elapsed_time(e1)
    res = {"kernel": kname, "wall_ms_per_step": wall_s * 1e3 / steps, "event_ms_per_launch": ev_ms / steps,
           "flop": 2.0 * m * n * k, "bytes_min": 2.0 * (m * k + k * n) + 2.0 * m * n, "desc": desc,
           "tensors": (a, b, c, bias)}
    if out is not None:
        out["tensors"] = (a, b, c)
    return res


def c1_latency(t0g, torch, rt, stream, steps, warmup):
    """256^3 NT, the reference's plumbing config: device time per launch (HIP events
    around back-to-back launches), host time per asynchronous t0g_gemm call and per
    call followed by t0g_wait_idle, both through this Python ctypes binding (the
    reference quotes ~2.3 us per asynchronous and ~15 us per synchronous dispatch,
    README.md:34, from Rust)."""
    r = time_gemm(t0g, torch, rt, stream, 256, 256, 256, "NT", steps, warmup, seed=11)
    desc = r["desc"]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        rt.gemm_desc(desc)
    t_async = (time.perf_counter() - t0) / steps
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        rt.gemm_desc(desc)
        rt.wait_idle()
    t_sync = (time.perf_counter() - t0) / steps
    sec = r["event_ms_per_launch"] * 1e-3
    return {"device_us_per_launch": round(sec * 1e6, 2), "tflops": round(r["flop"] / sec / 1e12, 2),
            "host_us_per_async_call": round(t_async * 1e6, 2), "host_us_per_sync_call": round(t_sync * 1e6, 2),
            "kernel": r["kernel"], "host_path": "Python ctypes -> t0g_gemm"}


MLP_SHAPES = [("NN", 1024, 11008, 4096), ("NN", 1024, 4096, 11008), ("NT", 1024, 11008, 4096),
              ("NT", 1024, 4096, 11008), ("TN", 11008, 4096, 1024), ("TN", 4096, 11008, 1024)]


def mlp_step(t0g, torch, rt, stream, steps, warmup, configs=None, grouped=False, clock=False):
    """Benchmark config 5: forward H = X W1, Y = H W2 (NN) and backward dH = dY W2^T,
    dX = dH W1^T (NT), dW2 = H^T dY, dW1 = X^T dH (TN); bf16 in/out.  configs: one
    GemmConfig per GEMM (in MLP_SHAPES order) instead of auto_select's.  grouped: the
    GEMMs that do not depend on each other go through t0g_gemm_group: H, then
    {Y, dH, dW2}, then {dX, dW1}.  clock: also sample the shader clock while steps
    run back to back."""
    bsz, d_in, d_hid = 1024, 4096, 11008
    g = torch.Generator(device="cuda").manual_seed(7)
    x = torch.randn((bsz, d_in), generator=g, device="cuda").to(torch.bfloat16)
    w1 = ((torch.rand((d_in, d_hid), generator=g, device="cuda") - 1.0) * (2.0 / d_in) ** 0.5).to(torch.bfloat16)
    w2 = ((torch.rand((d_hid, d_in), generator=g, device="cuda") - 1.0) * (2.0 / d_hid) ** 0.5).to(torch.bfloat16)
    dy = (torch.randn((bsz, d_in), generator=g, device="cuda") * 0.02).to(torch.bfloat16)
    h = torch.empty((bsz, d_hid), dtype=torch.bfloat16, device="cuda")
    y = torch.empty((bsz, d_in), dtype=torch.bfloat16, device="cuda")
    dh = torch.empty_like(h)
    dx = torch.empty_like(x)
    dw1 = torch.empty_like(w1)
    dw2 = torch.empty_like(w2)
    p = lambda t: t.data_ptr()
    cf = configs or [None] * 6
    descs = [
        t0g.gemm_desc(p(x), p(w1), p(h), bsz, d_hid, d_in, transpose="NN", out_dtype=t0g.BF16, config=cf[0]),
        t0g.gemm_desc(p(h), p(w2), p(y), bsz, d_in, d_hid, transpose="NN", out_dtype=t0g.BF16, config=cf[1]),
        t0g.gemm_desc(p(dy), p(w2), p(dh), bsz, d_hid, d_in, transpose="NT", out_dtype=t0g.BF16, config=cf[2]),
        t0g.gemm_desc(p(dh), p(w1), p(dx), bsz, d_in, d_hid, transpose="NT", out_dtype=t0g.BF16, config=cf[3]),
        t0g.gemm_desc(p(h), p(dy), p(dw2), d_hid, d_in, bsz, transpose="TN", out_dtype=t0g.BF16, config=cf[4]),
        t0g.gemm_desc(p(x), p(dh), p(dw1), d_in, d_hid, bsz, transpose="TN", out_dtype=t0g.BF16, config=cf[5]),
    ]
    def step():
        if grouped:
            rt.gemm_desc(descs[0])
            rt.gemm_group([descs[1], descs[2], descs[4]])
            rt.gemm_group([descs[3], descs[5]])
        else:
            for d in descs:
                rt.gemm_desc(d)

    _warm(torch, step, warmup)
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(steps):
        step()
    e1.record(stream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    flop = 6 * 2.0 * bsz * d_in * d_hid
    out = {"ms_per_step": ms, "tflops": flop / (ms * 1e-3) / 1e12,
           "frac_of_peak": flop / (ms * 1e-3) / 1e12 / PEAK_TFLOPS,
           "kernels": [t0g.gemm_kernel_name(d) for d in descs]}
    if clock:
        clk = sustained_clock(torch, step, 3.0)
        out["clock"] = clk if clk is not None else {"sclk_mhz_median": None}
        out["clock"].update(_mfma_util(out["tflops"], out["clock"].get("sclk_mhz_median")))
    return out


def _event_ms(torch, stream, fn, steps, warmup):
    _warm(torch, fn, warmup)
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(steps):
        fn()
    e1.record(stream)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps


def ignis_linear(torch, rt, stream, steps, warmup):
    """The Ignis caller path on f32 device tensors (src/ignis/ops/bf16_matmul.rs): the
    f32 -> bf16 conversion kernel alone (HBM-bound: 4 B read + 2 B written per element),
    then a Linear layer of the MLP step (X [1024][4096] * W [4096][11008]) through
    matmul (both operands converted on the GPU), matmul_with_wt_bf16 (weight kept
    as bf16, only X converted) and matmul with W's bf16 copy from the weight cache;
    f32 output."""
    n_conv = 64 << 20
    src = torch.randn(n_conv, device="cuda")
    dst = torch.empty(n_conv, dtype=torch.bfloat16, device="cuda")
    ms_conv = _event_ms(torch, stream, lambda: rt.f32_to_bf16(src.data_ptr(), dst.data_ptr(), n_conv), steps, warmup)
    conv_gbs = 6.0 * n_conv / (ms_conv * 1e-3) / 1e9
    del src, dst
    m, k, n = 1024, 4096, 11008
    g = torch.Generator(device="cuda").manual_seed(11)
    x = torch.randn((m, k), generator=g, device="cuda")
    w = torch.randn((k, n), generator=g, device="cuda") * (2.0 / k) ** 0.5
    wt16 = w.t().contiguous().to(torch.bfloat16)
    y = torch.empty((m, n), device="cuda")
    p = lambda t: t.data_ptr()
    ms_mm = _event_ms(torch, stream, lambda: rt.matmul_f32(p(x), p(w), p(y), m, k, n), steps, warmup)
    ms_wt = _event_ms(torch, stream, lambda: rt.matmul_wt_bf16_f32(p(x), p(wt16), p(y), m, k, n), steps, warmup)
    # W's bf16 copy from the GpuRuntime weight cache (gpu_context.rs:385-433): converted on
    # the first call only, so each timed call converts X alone, as matmul_with_wt_bf16 does
    wid = 0x7E57
    rt.invalidate_bf16(wid)
    ms_ca = _event_ms(torch, stream, lambda: rt.matmul_f32_cached(p(x), p(w), wid, p(y), m, k, n), steps, warmup)
    rt.invalidate_bf16(wid)
    flop = 2.0 * m * n * k
    return {"f32_to_bf16_64Mi": {"ms": round(ms_conv, 4), "gbs": round(conv_gbs, 1),
                                 "frac_of_hbm": round(conv_gbs / PEAK_GBS, 4)},
            "matmul_f32_1024x4096x11008": {"ms": round(ms_mm, 4), "tflops": round(flop / (ms_mm * 1e-3) / 1e12, 2)},
            "matmul_wt_bf16_f32_1024x4096x11008": {"ms": round(ms_wt, 4),
                                                   "tflops": round(flop / (ms_wt * 1e-3) / 1e12, 2)},
            "matmul_f32_cached_w_1024x4096x11008": {"ms": round(ms_ca, 4),
                                                    "tflops": round(flop / (ms_ca * 1e-3) / 1e12, 2)}}


def tuner_extra(t0g, torch, rt, stream, steps, warmup):
    """GemmTuner (src/t0/auto_gemm.rs) on the benchmark shapes, from an empty cache: the
    tuning time, a cache hit's time, and each shape's GEMM with auto_select's config
    and with the tuned one (same harness as the other lines); then the MLP step with
    the tuned configs."""
    import tempfile
    shapes = [("NT", 128, 4096, 4096), ("NT", 256, 256, 32768), ("NN", 4096, 4096, 4096)] + MLP_SHAPES
    out = {}
    tuned = {}
    with tempfile.TemporaryDirectory() as d, t0g.GemmTuner.with_cache_dir(d) as tuner:
        rt.set_stream(None)   # the tuner synchronises the library's own stream
        t_tune = 0.0
        for lay, m, n, k in shapes:
            t0 = time.perf_counter()
            cfg = tuner.tune(rt, m, n, k, transpose=lay, out_dtype=t0g.BF16)
            t_tune += time.perf_counter() - t0
            tuned[(lay, m, n, k)] = cfg
        t0 = time.perf_counter()
        for lay, m, n, k in shapes:
            tuner.tune(rt, m, n, k, transpose=lay, out_dtype=t0g.BF16)
        t_hit = (time.perf_counter() - t0) / len(shapes)
        rt.set_stream(stream.cuda_stream)
        out["tuning_s_total"] = round(t_tune, 3)
        out["cache_hit_us"] = round(t_hit * 1e6, 2)
        for lay, m, n, k in shapes:
            cfg = tuned[(lay, m, n, k)]
            auto = t0g.auto_select(m, k, n)
            ra = time_gemm(t0g, torch, rt, stream, m, n, k, lay, steps, warmup, seed=13)
            rtu = time_gemm(t0g, torch, rt, stream, m, n, k, lay, steps, warmup, seed=13, config=cfg)
            out[f"{lay.lower()}_{m}x{n}x{k}"] = {
                "auto_select": auto.name(), "auto_us": round(ra["event_ms_per_launch"] * 1e3, 2),
                "tuned": cfg.name(), "tuned_us": round(rtu["event_ms_per_launch"] * 1e3, 2),
                "tuned_tflops": round(rtu["flop"] / (rtu["event_ms_per_launch"] * 1e-3) / 1e12, 1)}
    out["mlp_step_tuned"] = mlp_step(t0g, torch, rt, stream, max(3, steps // 5), max(2, warmup // 10),
                                     configs=[tuned[s] for s in MLP_SHAPES])
    return out


def stream_k_extra(t0g, torch, rt, stream, steps, warmup):
    """The stream-K schedule against the data-parallel / split-K ones: a tile count
    just past 256 (272 tiles, where auto_select takes stream-K) and the MLP forward
    shape (172 tiles, where it does not)."""
    p256 = t0g.GemmConfig.preset("gfx950_256x256_k64")
    sk = p256.copy(split_k=t0g.STREAM_K)
    out = {}
    for lay, m, n, k, others in [("NN", 4352, 4096, 8192, {"dp": p256, "split2": p256.copy(split_k=2)}),
                                 ("NN", 1024, 11008, 4096, {"dp": p256})]:
        line = {"auto_select": t0g.auto_select(m, k, n).name()}
        r = time_gemm(t0g, torch, rt, stream, m, n, k, lay, steps, warmup, seed=17, config=sk)
        line["stream_k_us"] = round(r["event_ms_per_launch"] * 1e3, 2)
        line["stream_k_tflops"] = round(r["flop"] / (r["event_ms_per_launch"] * 1e-3) / 1e12, 1)
        for name, cfg in others.items():
            r = time_gemm(t0g, torch, rt, stream, m, n, k, lay, steps, warmup, seed=17, config=cfg)
            line[f"{name}_us"] = round(r["event_ms_per_launch"] * 1e3, 2)
        out[f"{lay.lower()}_{m}x{n}x{k}"] = line
    out["ready_flag_timeouts"] = rt.stream_k_timeouts()
    return out


def _amd_smi_sample():
    """One reading of the GFX clocks (MHz, one per XCD) and the socket power (W) from
    amd-smi, run as a child process (it reads the driver's metrics; it does not touch
    this process's GPU context).  Returns (clocks, power, raw text) or None."""
    import re
    import subprocess
    try:
        out = subprocess.run(["amd-smi", "metric", "-g", "0", "-c", "-p", "--json"], capture_output=True,
                             text=True, timeout=10)
    except (OSError, subprocess.TimeoutExpired):
        return None
    if out.returncode != 0:
        return None
    try:
        js = json.loads(out.stdout)
    except ValueError:
        return None
    clocks, power = [], []

    def num(v):
        if isinstance(v, dict):
            v = v.get("value")
        return float(v) if isinstance(v, (int, float)) else None

    def walk(node, parent=""):
        if isinstance(node, dict):
            for key, val in node.items():
                kl = str(key).lower()
                if re.fullmatch(r"gfx_?\d*", kl) and isinstance(val, dict) and "clk" in val:
                    v = num(val["clk"])
                    if v is not None and v > 0:
                        clocks.append(v)
                elif kl in ("socket_power", "current_socket_power", "average_socket_power"):
                    v = num(val)
                    if v is not None and v > 0:
                        power.append(v)
                else:
                    walk(val, kl)
        elif isinstance(node, list):
            for val in node:
                walk(val, parent)

    walk(js)
    return clocks, (power[0] if power else None), out.stdout[:2000]


def sustained_clock(torch, launch, seconds=2.0):
    """Run `launch` back to back for `seconds` while a thread samples amd-smi; the
    samples of the first 0.4 s (the clock's ramp under load) are dropped.  Returns the
    median GFX clock over XCDs and samples, the median socket power, the sample count."""
    import threading
    samples, stop = [], threading.Event()

    def sampler():
        t0 = time.perf_counter()
        while not stop.is_set():
            s = _amd_smi_sample()
            if s is None:
                return
            # readings under the 500 MHz DPM floor are deep-sleep samples of an idle XCD
            clocks = [c for c in s[0] if c >= 500.0]
            if time.perf_counter() - t0 > 0.4 and clocks:
                samples.append((clocks, s[1], s[2]))
            time.sleep(0.05)

    th = threading.Thread(target=sampler, daemon=True)
    th.start()
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        for _ in range(16):
            launch()
        torch.cuda.synchronize()
    stop.set()
    th.join(timeout=15)
    if not samples:
        return None
    clocks = sorted(c for s in samples for c in s[0])
    powers = sorted(s[1] for s in samples if s[1] is not None)
    return {"sclk_mhz_median": clocks[len(clocks) // 2], "sclk_mhz_min": clocks[0], "sclk_mhz_max": clocks[-1],
            "socket_power_w_median": powers[len(powers) // 2] if powers else None, "samples": len(samples),
            "source": "amd-smi metric -c -p (child process) while the GEMM ran back to back"}


def clock_line(torch, rt, desc, flop, seconds=2.0):
    """Measured shader clock next to a result, and the MFMA utilisation it implies: the
    kernel's FLOP rate under the same sustained load over the dense bf16 rate at that
    clock (256 CUs x 4096 FLOP per clock; every MFMA is useful work, checked with the
    SQ_INSTS_VALU_MFMA_MOPS_BF16 counter)."""
    clk = sustained_clock(torch, lambda: rt.gemm_desc(desc), seconds)
    if clk is None:
        return {"sclk_mhz_median": None, "note": "amd-smi gave no clock reading on this host"}
    return clk


def _mfma_util(tflops, sclk_mhz):
    """The FLOP rate over the dense bf16 rate at the measured clock (256 CUs x 4096
    FLOP/clk): the fraction of cycles the MFMA pipes are busy with this GEMM."""
    if not sclk_mhz:
        return {"mfma_util": None}
    at_clock = 256 * 4096 * sclk_mhz * 1e6 / 1e12
    return {"dense_peak_at_sclk_tflops": round(at_clock, 1), "mfma_util": round(tflops / at_clock, 4)}


def cold_gemm(t0g, torch, rt, stream, m, n, k, layout, trials):
    """One GEMM per trial after a 512 MB device copy that evicts the GEMM's operands from
    the 256 MB Infinity Cache and the L2s; each launch timed alone by HIP events; median."""
    a, b = make_inputs(torch, m, n, k, layout, 2)
    c = torch.empty((m, n), dtype=torch.bfloat16, device="cuda")
    flush_src = torch.ones(64 << 20, dtype=torch.float32, device="cuda")
    flush_dst = torch.empty_like(flush_src)
    desc = t0g.gemm_desc(a.data_ptr(), b.data_ptr(), c.data_ptr(), m, n, k, transpose=layout, out_dtype=t0g.BF16)
    for _ in range(3):
        rt.gemm_desc(desc)
    times = []
    for _ in range(trials):
        flush_dst.copy_(flush_src)
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        rt.gemm_desc(desc)
        e1.record(stream)
        torch.cuda.synchronize()
        times.append(e0.elapsed_time(e1))
    times.sort()
    ms = times[len(times) // 2]
    return {"us_median": round(ms * 1e3, 2), "tflops": round(2.0 * m * n * k / (ms * 1e-3) / 1e12, 1),
            "frac_of_peak": round(2.0 * m * n * k / (ms * 1e-3) / 1e12 / PEAK_TFLOPS, 4),
            "us_min": round(times[0] * 1e3, 2), "trials": trials, "kernel": t0g.gemm_kernel_name(desc)}


def cpu_baseline(torch, tensors, m, n, k, min_seconds):
    """The CPU oracle (oracle/ref_gemm.c, a bit-exact restatement of the reference's
    CPU GEMM) on this host: the whole 4096^3 product, repeated to ~min_seconds."""
    import numpy as np
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle
    a, b, _ = tensors
    a_np = a.cpu().view(torch.int16).numpy().view(np.uint16)
    b_np = b.cpu().view(torch.int16).numpy().view(np.uint16)
    threads = oracle.num_threads()
    reps, t_total = 0, 0.0
    while t_total < min_seconds and reps < 20:
        t0 = time.perf_counter()
        oracle.gemm("NN", a_np, b_np, m, n, k, threads=threads)
        t_total += time.perf_counter() - t0
        reps += 1
    fast = 2.0 * m * n * k * reps / t_total / 1e12
    rows = 16
    t0 = time.perf_counter()
    oracle.gemm_nt_naive(a_np, np.ascontiguousarray(b_np.T), m, k, n, rows=(0, rows))
    t_naive = time.perf_counter() - t0
    naive = 2.0 * rows * n * k / t_naive / 1e12
    cpu_model = None
    try:
        import subprocess
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        cpu_model = next((ln.split(":", 1)[1].strip() for ln in out.splitlines() if ln.startswith("Model name")), None)
    except (OSError, ValueError):
        pass
    if not cpu_model:
        try:
            with open("/proc/cpuinfo") as f:
                cpu_model = next((ln.split(":", 1)[1].strip() for ln in f if ln.startswith("model name")), None)
        except OSError:
            pass
    nproc = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
    return {"value": fast, "unit": "TFLOPS", "cores": threads, "kind": "port", "cpu_model": cpu_model,
            "nproc": nproc, "host_cpus": os.cpu_count(),
            "sample": f"full {m}x{n}x{k} NN product x{reps} ({t_total:.1f} s, vectorised + OpenMP, "
                      f"bit-identical to the reference loop)",
            "naive_single_thread": {"value": naive, "unit": "TFLOPS", "cores": 1,
                                    "sample": f"{rows} output rows of {m}x{n}x{k}, reference loop order"}}


def timeline_summary(t0g, torch, rt, desc, k):
    """One launch's per-workgroup timeline (t0g_set_timeline), recorded as the last
    of 20 back-to-back launches (steady clock, a queue of work ahead of it), in
    microseconds from the first workgroup's entry: the launch's span, and per XCD
    the mean K-loop time (entry to the end of the K loop, first DMA wait
    included), the mean epilogue time (stores completed) and the last
    workgroup's end."""
    import numpy as np
    rt.timeline_clear()
    t0g.set_timeline(True)
    try:
        for _ in range(20):
            rt.gemm_desc(desc)
        torch.cuda.synchronize()
        tl = rt.timeline_read()
    finally:
        t0g.set_timeline(False)
    rows = tl[tl[:, 0] != 0].astype(np.float64)
    if len(rows) == 0:
        return {"workgroups": 0, "note": "the kernel records no timeline"}
    us = t0g.TIMELINE_TICK_NS / 1e3
    t0 = rows[:, 0].min()
    entry, kend, end = (rows[:, 0] - t0) * us, (rows[:, 1] - t0) * us, (rows[:, 2] - t0) * us
    xcc = (tl[tl[:, 0] != 0][:, 3] >> np.uint64(32)).astype(np.int64) & 15
    kl, ep = kend - entry, end - kend
    per_xcd = {}
    for x in sorted(set(xcc.tolist())):
        sel = xcc == x
        per_xcd[str(x)] = {"workgroups": int(sel.sum()), "kloop_us_mean": round(float(kl[sel].mean()), 2),
                           "epilogue_us_mean": round(float(ep[sel].mean()), 2),
                           "last_end_us": round(float(end[sel].max()), 2)}
    return {"workgroups": int(len(rows)), "span_us": round(float(end.max()), 2),
            "kloop_us": {"min": round(float(kl.min()), 2), "median": round(float(np.median(kl)), 2),
                         "max": round(float(kl.max()), 2)},
            "epilogue_us": {"min": round(float(ep.min()), 2), "median": round(float(np.median(ep)), 2),
                            "max": round(float(ep.max()), 2)},
            "last_entry_us": round(float(entry.max()), 2), "per_xcd": per_xcd,
            "clock": "s_memrealtime, 100 MHz"}


def main():
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=200,
                    help="untimed launches first (each line also warms for at least 0.2 s of load, the "
                         "time the shader clock takes to reach its steady state)")
    ap.add_argument("--no-extra", action="store_true", help="skip the other benchmark configurations")
    ap.add_argument("--no-clock", action="store_true", help="skip the shader-clock sampling (amd-smi) lines")
    ap.add_argument("--cpu-seconds", type=float, default=10.0, help="CPU baseline budget (0 = skip)")
    ap.add_argument("--clock", action="store_true",
                    help="with --only LAYOUT:M:N:K or MLP: also sample the shader clock and socket power (amd-smi) "
                         "while that GEMM (or step) runs back to back, and the MFMA utilisation they imply")
    ap.add_argument("--timeline", action="store_true",
                    help="with --only LAYOUT:M:N:K: also record one launch's per-workgroup timeline (entry, end "
                         "of the K loop, stores done; t0g_set_timeline) and print its per-XCD summary")
    ap.add_argument("--only", metavar="LAYOUT:M:N:K",
                    help="time just this GEMM (bf16 out) and print its own JSON line; for profiling runs. "
                         "COPY:MiB instead times a plain device-to-device copy of that size, the "
                         "calibration kernel for the FETCH_SIZE / WRITE_SIZE counters; MLP or "
                         "MLP_GROUPED times benchmark config 5's step (six GEMMs); TORCH:LAYOUT:M:N:K "
                         "times torch.mm (hipBLASLt) on the same inputs, for comparison runs")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: --gpus {args.gpus}: this build measures the GEMM on one GPU only "
              f"(no multi-GPU path); run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    import torch
    import t0g

    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        sys.exit(1)
    rt = t0g.GpuRuntime.new(0)
    stream = torch.cuda.Stream()
    rt.set_stream(stream.cuda_stream)
    torch.cuda.set_stream(stream)

    if args.only and args.only.upper().startswith("COPY:"):
        nbytes = int(float(args.only.split(":")[1]) * (1 << 20)) // 16 * 16
        src = torch.randint(0, 1 << 30, (nbytes // 4,), dtype=torch.int32, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(args.warmup):
            dst.copy_(src)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(args.steps):
            dst.copy_(src)
        e1.record(stream)
        torch.cuda.synchronize()
        sec = e0.elapsed_time(e1) * 1e-3 / args.steps
        print(json.dumps({"only": args.only, "bytes_read": nbytes, "bytes_written": nbytes,
                          "us_per_copy": round(sec * 1e6, 2), "gbs": round(2 * nbytes / sec / 1e9, 1)}), flush=True)
        rt.set_stream(None)
        rt.close()
        return

    if args.only and args.only.upper().startswith("CONVERT:"):
        n_el = int(float(args.only.split(":")[1]) * (1 << 20)) // 8 * 8
        src = torch.randn(n_el, device="cuda")
        dst = torch.empty(n_el, dtype=torch.bfloat16, device="cuda")
        ms = _event_ms(torch, stream, lambda: rt.f32_to_bf16(src.data_ptr(), dst.data_ptr(), n_el), args.steps,
                       args.warmup)
        print(json.dumps({"only": args.only, "kernel": "t0g_f32_to_bf16_rne", "elements": n_el,
                          "us_per_launch": round(ms * 1e3, 2), "gbs": round(6.0 * n_el / (ms * 1e-3) / 1e9, 1)}),
              flush=True)
        rt.set_stream(None)
        rt.close()
        return

    if args.only and args.only.upper().startswith("TORCH:"):
        lay, m, n, k = args.only.split(":")[1:5]
        lay, m, n, k = lay.upper(), int(m), int(n), int(k)
        if lay not in ("NN", "NT"):
            raise SystemExit("TORCH: NN or NT only")
        a, b = make_inputs(torch, m, n, k, lay, 2)
        bb = b.t() if lay == "NT" else b   # 2-D mm with a transposed view: hipBLASLt's transB
        c = torch.empty((m, n), dtype=torch.bfloat16, device="cuda")
        ms = _event_ms(torch, stream, lambda: torch.mm(a, bb, out=c), args.steps, args.warmup)
        flop = 2.0 * m * n * k
        print(json.dumps({"only": args.only, "library": "torch.mm (hipBLASLt)", "us_per_launch": round(ms * 1e3, 2),
                          "tflops": round(flop / (ms * 1e-3) / 1e12, 2),
                          "frac_of_peak": round(flop / (ms * 1e-3) / 1e12 / PEAK_TFLOPS, 4)}), flush=True)
        rt.set_stream(None)
        rt.close()
        return

    if args.only and args.only.upper() in ("MLP", "MLP_GROUPED"):
        r = mlp_step(t0g, torch, rt, stream, args.steps, args.warmup, grouped=args.only.upper() == "MLP_GROUPED",
                     clock=args.clock)
        line = {"only": args.only, "ms_per_step": round(r["ms_per_step"], 5), "tflops": round(r["tflops"], 2),
                "frac_of_peak": round(r["frac_of_peak"], 4), "kernels": r["kernels"]}
        if "clock" in r:
            line["clock"] = r["clock"]
        print(json.dumps(line), flush=True)
        rt.set_stream(None)
        rt.close()
        return

    if args.only:
        lay, m, n, k = args.only.split(":")
        m, n, k = int(m), int(n), int(k)
        r = time_gemm(t0g, torch, rt, stream, m, n, k, lay.upper(), args.steps, args.warmup)
        sec = r["event_ms_per_launch"] * 1e-3
        line = {"only": args.only, "kernel": r["kernel"], "us_per_launch": round(sec * 1e6, 2),
                "tflops": round(r["flop"] / sec / 1e12, 2),
                "frac_of_peak": round(r["flop"] / sec / 1e12 / PEAK_TFLOPS, 4),
                "gbs_min_bytes": round(r["bytes_min"] / sec / 1e9, 1)}
        if args.clock:
            ck = clock_line(torch, rt, r["desc"], r["flop"], seconds=3.0)
            ck.update(_mfma_util(r["flop"] / sec / 1e12, ck.get("sclk_mhz_median")))
            line["clock"] = ck
        if args.timeline:
            line["timeline"] = timeline_summary(t0g, torch, rt, r["desc"], k)
        print(json.dumps(line), flush=True)
        rt.set_stream(None)
        rt.close()
        return

    M = N = K = 4096
    keep = {}
    log(f"[bench] 4096^3 NN bf16: warmup {args.warmup}, steps {args.steps}")
    main_res = time_gemm(t0g, torch, rt, stream, M, N, K, "NN", args.steps, args.warmup, out=keep)
    tflops = main_res["flop"] / (main_res["wall_ms_per_step"] * 1e-3) / 1e12
    kern_tflops = main_res["flop"] / (main_res["event_ms_per_launch"] * 1e-3) / 1e12
    traffic = None
    if os.path.exists(TRAFFIC_FILE):
        with open(TRAFFIC_FILE) as f:
            traffic = json.load(f).get(main_res["kernel"])
    line = {
        "metric": METRIC,
        "value": round(tflops, 2),
        "unit": "TFLOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "warmup_min_load_s": WARM_MIN_MS / 1e3,   # each line also warms until this much load has run
        "ms_per_step": round(main_res["wall_ms_per_step"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: A, B ~ N(0,1)*0.02 from seed (torch.randn on device), bf16",
        "config": {"workload": "gemm_bf16_nn_4096x4096x4096_bf16out", "M": M, "N": N, "K": K,
                   "layout": "NN (C = A*B, row-major)", "accumulate": "fp32", "out": "bf16",
                   "kernel": main_res["kernel"], "parallelism": "single GPU"},
        "roofline": {"bound": "mfma", "achieved": round(kern_tflops, 2), "peak": PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(kern_tflops / PEAK_TFLOPS, 4), "traffic": traffic,
                     "per_launch_flop": main_res["flop"], "avg_launch_ms": round(main_res["event_ms_per_launch"], 5)},
    }
    if not args.no_clock:
        log("[bench] 4096^3 NN bf16: shader clock under sustained load")
        line["clock"] = clock_line(torch, rt, main_res["desc"], main_res["flop"])
        line["clock"].update(_mfma_util(kern_tflops, line["clock"].get("sclk_mhz_median")))

    if not args.no_extra:
        extra = {}
        steps8 = max(5, args.steps // 2)
        log("[bench] 4096^3 NN bf16, operands evicted from the caches before each launch")
        extra["gemm_nn_4096^3_cold_cache"] = cold_gemm(t0g, torch, rt, stream, M, N, K, "NN", 25)
        log(f"[bench] 8192^3 NN bf16: steps {steps8}")
        r8 = time_gemm(t0g, torch, rt, stream, 8192, 8192, 8192, "NN", steps8, max(3, args.warmup // 8), seed=4)
        t8 = r8["flop"] / (r8["event_ms_per_launch"] * 1e-3) / 1e12
        extra["gemm_nn_8192^3"] = {"tflops": round(t8, 2), "frac_of_peak": round(t8 / PEAK_TFLOPS, 4),
                                   "ms_per_launch": round(r8["event_ms_per_launch"], 4), "kernel": r8["kernel"]}
        if not args.no_clock:
            log("[bench] 8192^3 NN bf16: shader clock under sustained load")
            ck8 = clock_line(torch, rt, r8["desc"], r8["flop"], seconds=3.0)
            ck8.update(_mfma_util(t8, ck8.get("sclk_mhz_median")))
            extra["gemm_nn_8192^3"]["clock"] = ck8
        del r8
        log("[bench] 4096^3 NT bf16")
        rnt = time_gemm(t0g, torch, rt, stream, 4096, 4096, 4096, "NT", args.steps, args.warmup, seed=6)
        tnt = rnt["flop"] / (rnt["event_ms_per_launch"] * 1e-3) / 1e12
        extra["gemm_nt_4096^3"] = {"tflops": round(tnt, 2), "frac_of_peak": round(tnt / PEAK_TFLOPS, 4),
                                   "ms_per_launch": round(rnt["event_ms_per_launch"], 4), "kernel": rnt["kernel"]}
        for name, (m, n, k) in {"thin_128x4096x4096": (128, 4096, 4096),
                                "splitk_256x256xK32768": (256, 256, 32768)}.items():
            log(f"[bench] {name}")
            r = time_gemm(t0g, torch, rt, stream, m, n, k, "NT", args.steps, args.warmup, seed=9, dist="uniform")
            sec = r["event_ms_per_launch"] * 1e-3
            extra[name] = {"tflops": round(r["flop"] / sec / 1e12, 2),
                           "gbs_min_bytes": round(r["bytes_min"] / sec / 1e9, 1),
                           "frac_of_hbm": round(r["bytes_min"] / sec / 1e9 / PEAK_GBS, 4),
                           "us_per_gemm": round(sec * 1e6, 2), "kernel": r["kernel"]}
        log("[bench] 256^3 NT (launch-latency config)")
        extra["c1_256^3"] = c1_latency(t0g, torch, rt, stream, max(100, args.steps), max(20, args.warmup // 4))
        log("[bench] 4096^3 NN bf16 with fused bias + SiLU epilogue")
        rf = time_gemm(t0g, torch, rt, stream, M, N, K, "NN", args.steps, args.warmup // 2, epilogue_ops=["bias", "silu"])
        tf = rf["flop"] / (rf["event_ms_per_launch"] * 1e-3) / 1e12
        extra["gemm_nn_4096^3_bias_silu"] = {
            "tflops": round(tf, 2), "ms_per_launch": round(rf["event_ms_per_launch"], 4),
            "overhead_vs_plain_pct": round((rf["event_ms_per_launch"] / main_res["event_ms_per_launch"] - 1) * 100, 2),
            "kernel": rf["kernel"]}
        log("[bench] MLP step")
        extra["mlp_step_1024x4096x11008"] = mlp_step(t0g, torch, rt, stream, max(3, args.steps // 5),
                                                     max(2, args.warmup // 10))
        log("[bench] MLP step, independent GEMMs grouped")
        extra["mlp_step_1024x4096x11008_grouped"] = mlp_step(t0g, torch, rt, stream, max(3, args.steps // 5),
                                                             max(2, args.warmup // 10), grouped=True)
        log("[bench] GemmTuner on the benchmark shapes")
        extra["tuner"] = tuner_extra(t0g, torch, rt, stream, max(10, args.steps // 2), max(10, args.warmup // 4))
        log("[bench] stream-K")
        extra["stream_k"] = stream_k_extra(t0g, torch, rt, stream, max(10, args.steps // 4), max(10, args.warmup // 8))
        log("[bench] Ignis f32 caller path")
        extra["ignis"] = ignis_linear(torch, rt, stream, max(5, args.steps // 2), max(3, args.warmup // 4))
        line["extra"] = extra

    if args.cpu_seconds > 0:
        log("[bench] CPU baseline (oracle on host cores)")
        line["cpu_baseline"] = cpu_baseline(torch, keep["tensors"], M, N, K, args.cpu_seconds)
    else:
        line["cpu_baseline"] = None
    rt.set_stream(None)
    rt.close()
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
