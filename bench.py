"""Benchmark of the MI355X kernel path on the BASELINE.json configs.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME|all]

Prints ONE JSON line. The headline (metric/value) is the workload named by --workload; with
"all" (default) it is the dense GEMM 4096^3 and every other config is
reported in "configs". A step is one pass of the config's kernel(s) over one batch of synthetic
input already resident in HBM. For working sets that fit the 256 MB Infinity Cache, steps rotate
over enough input copies (> 512 MiB in total) that no step reads another step's data from cache.

The timed steps are replayed from one HIP graph (captured from torch's current stream, which
is the stream every kernel is launched on), between device synchronisations, and timed with HIP
events on that stream. Before the timed replay the graph is replayed untimed for >= 50 ms: the
clocks dip at the start of a burst of matrix work and need ~20 ms to reach their sustained
level. roofline.achieved = algorithmic bytes (or FLOPs) per launch / mean launch duration, the
mean taken over a graph of back-to-back launches (rotating input copies); each record also
carries the median of single launches that each follow a 512 MiB cache flush.
cpu_baseline = the oracle (restated reference torch path) on a bounded sample, timed on this
host's cores.

Each timed replay is bracketed by two launches of a marker kernel (a one-element int16
bitwise_not, outside the HIP-event window), so that a rocprofv3 kernel trace of this script can
pick out exactly the timed dispatches: `python bench.py --summarize-trace <kernel_trace.csv>`
prints, per kernel, the statistics of all dispatches and of the dispatches inside each marked
window (window 1: the timed steps; window 2: the back-to-back launch graph behind
roofline.achieved).
"""
import argparse
import itertools
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "tilelang-tpu_amd"))
sys.path.insert(0, ROOT)

import torch  # noqa: E402

HBM_PEAK_GBS = 8000.0
# e4m3 MACs executed per algorithmic MAC in the FP8 MLA decode: Q^T as two terms (576 of the
# 1088 MACs per token and head), P^T as one (the other 512)
MLA_EXEC_FACTOR = (2 * 576 + 512) / (576 + 512)
MFMA_PEAK = {"bf16": 2500.0, "fp16": 2500.0, "fp8": 5000.0}  # dense TFLOP/s (AMD spec)
FLUSH_BYTES = 512 << 20
CACHE_EVICT_BYTES = 512 << 20

METRIC = "TFLOP/s (% MFMA peak) GEMM/FA/FP8-MLA; GB/s (% HBM peak) norm/rope/swiglu"


def cpu_model() -> str:
    """Model name of the host CPU (first 'model name' line of /proc/cpuinfo)."""
    try:
        with open("/proc/cpuinfo") as f:
            for ln in f:
                if ln.startswith("model name"):
                    return ln.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def log(msg):
    print(msg, file=sys.stderr, flush=True)


# ------------------------------------------------------------------------------------------------
# timing helpers


def _copies_for(nbytes):
    return max(1, math.ceil(CACHE_EVICT_BYTES / max(nbytes, 1)))


_MARKER = []  # one-element int16 tensor; its bitwise_not kernel brackets the timed replays
MARKER_KERNEL = "bitwise_not"


def _mark():
    if _MARKER:
        _MARKER[0].bitwise_not_()


def _timed_replay(g):
    """One replay of g timed with HIP events on the current stream, between two marker
    launches (outside the event window); returns the elapsed ms."""
    _mark()
    st, en = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    st.record()
    g.replay()
    en.record()
    _mark()
    torch.cuda.synchronize()
    return st.elapsed_time(en)


def _capture(fns, n):
    """A HIP graph of n launches cycling over fns (None if capture is not possible)."""
    try:
        g = torch.cuda.CUDAGraph()
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            fns[0]()  # warm any lazy state outside the capture
            torch.cuda.synchronize()
            with torch.cuda.graph(g, stream=s):
                for i in range(n):
                    fns[i % len(fns)]()
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        return g
    except Exception as e:  # pragma: no cover - reported in the JSON
        log(f"[bench] graph capture failed ({e}); timing eager launches")
        return None


SETTLE_MS = 50.0


def _settle(g):
    """Replay g untimed until >= SETTLE_MS of GPU time has passed: the clocks dip at the start
    of a burst of matrix work and take ~20 ms to reach their sustained level."""
    spent, n = 0.0, 0
    while spent < SETTLE_MS and n < 1000:
        st, en = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        st.record()
        g.replay()
        en.record()
        torch.cuda.synchronize()
        spent += st.elapsed_time(en)
        n += 1


def time_steps(fns, steps, warmup):
    """ms per step over exactly `steps` steps after `warmup` untimed ones. The steps are
    replayed from one HIP graph (launch-bound host loops would otherwise starve ~10 us
    kernels); bracketed by device synchronisation, timed by HIP events on the replay stream."""
    for i in range(warmup):
        fns[i % len(fns)]()
    torch.cuda.synchronize()
    g = _capture(fns, steps)
    if g is not None:
        _settle(g)
        return _timed_replay(g) / steps, "hip-graph"
    torch.cuda.synchronize()
    st, en = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    st.record()
    for i in range(steps):
        fns[i % len(fns)]()
    en.record()
    torch.cuda.synchronize()
    return st.elapsed_time(en) / steps, "eager"


def time_launches(fns, reps, flush):
    """Mean launch duration (ms): `reps` back-to-back launches replayed from a HIP graph, HIP
    events on the stream they run on, divided by reps. Inputs rotate over copies sized to defeat
    the Infinity Cache. Also returns the median of 100 single launches, each after a 512 MiB
    cache flush."""
    g = _capture(fns, reps)
    mean = None
    if g is not None:
        _settle(g)
        mean = _timed_replay(g) / reps
    n1 = 100
    st = [torch.cuda.Event(enable_timing=True) for _ in range(n1)]
    en = [torch.cuda.Event(enable_timing=True) for _ in range(n1)]
    for i in range(n1):
        flush.zero_()
        st[i].record()
        fns[0]()
        en[i].record()
    torch.cuda.synchronize()
    ts = sorted(a.elapsed_time(b) for a, b in zip(st, en))
    med = ts[len(ts) // 2]
    return (mean if mean is not None else med), med


def cpu_time(fn, reps=3):
    fn()
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    ts.sort()
    return ts[len(ts) // 2]


def _sclk_file():
    """The one GPU's sysfs clock file (amdgpu pp_dpm_sclk: the marked line is the SMU's running
    average of the shader clock), or None when it is absent or there are several cards."""
    import glob
    files = glob.glob("/sys/class/drm/card*/device/pp_dpm_sclk")
    return files[0] if len(files) == 1 and os.access(files[0], os.R_OK) else None


def settled_sclk(fns, seconds=1.5):
    """Shader clock (MHz) while the workload runs back to back for `seconds`: mean of the sysfs
    readings of the last half (the average needs ~0.5 s to settle from idle). Measured after
    the timed steps, so it does not touch them; None without the sysfs file."""
    import re
    import threading
    path = _sclk_file()
    if path is None or not fns:
        return None
    samples, stop = [], threading.Event()

    def sample():
        while not stop.is_set():
            try:
                m = re.search(r"(\d+)\s*Mhz\s*\*", open(path).read())
                if m:
                    samples.append((time.perf_counter(), int(m.group(1))))
            except OSError:
                return
            time.sleep(0.01)

    th = threading.Thread(target=sample, daemon=True)
    t0 = time.perf_counter()
    th.start()
    i = 0
    while time.perf_counter() - t0 < seconds:
        fns[i % len(fns)]()
        i += 1
        if i % 32 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()
    stop.set()
    th.join()
    late = [v for t, v in samples if t - t0 >= seconds / 2]
    return round(sum(late) / len(late), 1) if late else None


def roofline(bound, achieved, unit, peak, traffic=None):
    return {"bound": bound, "achieved": round(achieved, 2), "peak": peak, "unit": unit,
            "frac": round(achieved / peak, 4), "traffic": traffic}


class PmcOnly(Exception):
    """Raised by a config in --pmc-launches mode once its kernel has run the requested times."""


_LAST_FNS = []  # launch closures of the workload being measured (for the clock pass)


def pmc_launches(args, fns, workload):
    """--pmc-launches N: N plain launches for hardware-counter collection (rocprofv3 --pmc),
    no graphs, no timing, no cache flush."""
    _LAST_FNS[:] = fns
    if not args.pmc_launches:
        return
    torch.cuda.synchronize()
    for i in range(args.pmc_launches):
        fns[i % len(fns)]()
    torch.cuda.synchronize()
    raise PmcOnly(workload)


def load_traffic():
    """HBM bytes per launch by workload from profiles/pmc_traffic.md (rocprofv3 --pmc
    FETCH_SIZE + WRITE_SIZE, scaled by the copy-kernel calibration recorded there)."""
    path = os.path.join(ROOT, "profiles", "pmc_traffic.md")
    out = {}
    if not os.path.exists(path):
        return out
    for line in open(path):
        cells = [c.strip() for c in line.strip().strip("|").split("|")]
        if len(cells) >= 6 and cells[0].startswith("`") and cells[5].replace(".", "").isdigit():
            out[cells[0].strip("`")] = float(cells[5])
    return out


# ------------------------------------------------------------------------------------------------
# configs


def bench_rmsnorm(args, dev, flush, cpu):
    import tilelang
    from tilelang.testing import programs, workloads
    w = workloads.rmsnorm(4096, 4096)
    k = tilelang.compile(programs.rms_norm(4096, 4096, 1, "float16", eps=1e-6, with_weight=True),
                         out_idx=-1, target="mi355x")
    nbytes = 2 * 4096 * 4096 * 2 + 4096 * 2
    sets = []
    for _ in range(_copies_for(nbytes)):
        x = w.tensors["x"].to(dev)
        wt = w.tensors["w"].to(dev)
        y = torch.empty_like(x)
        sets.append((x, wt, y))
    fns = [lambda s=s: k(*s) for s in sets]
    pmc_launches(args, fns, "rmsnorm")
    ms, how = time_steps(fns, args.steps, args.warmup)
    mean_ms, med_ms = time_launches(fns, 200, flush)
    res = {"workload": "rmsnorm_fp16_4096x4096", "value": nbytes / (ms * 1e-3) / 1e9,
           "unit": "GB/s", "ms_per_step": ms, "dtype": "f16",
           "roofline": roofline("hbm", nbytes / (mean_ms * 1e-3) / 1e9, "GB/s", HBM_PEAK_GBS),
           "kernel_ms_mean": mean_ms, "kernel_ms_flushed_median": med_ms, "timing": how, "algorithmic_bytes": nbytes}
    if cpu:
        from oracle import ref
        xs, ws = w.tensors["x"], w.tensors["w"]
        t = cpu_time(lambda: ref.rmsnorm_ref(xs, ws, 1e-6))
        res["cpu_baseline"] = {"value": nbytes / t / 1e9, "unit": "GB/s",
                               "cores": torch.get_num_threads(), "kind": "port",
                               "sample": "full 4096x4096 config, oracle.ref.rmsnorm_ref"}
    return res


def bench_swiglu(args, dev, flush, cpu):
    import tilelang
    from tilelang.testing import programs, workloads
    rows, cols = 8192, 14336
    w = workloads.swiglu(rows, cols)
    k = tilelang.compile(programs.swi_glu(32, 32, rows, cols), out_idx=-1)
    nbytes = 3 * rows * cols * 2
    g, u = w.tensors["gate"].to(dev), w.tensors["up"].to(dev)
    o = torch.empty_like(g)
    fns = [lambda: k(g, u, o)]
    pmc_launches(args, fns, "swiglu")
    ms, how = time_steps(fns, args.steps, args.warmup)
    mean_ms, med_ms = time_launches(fns, 50, flush)
    res = {"workload": "swiglu_bf16_8192x14336", "value": nbytes / (ms * 1e-3) / 1e9,
           "unit": "GB/s", "ms_per_step": ms, "dtype": "bf16",
           "roofline": roofline("hbm", nbytes / (mean_ms * 1e-3) / 1e9, "GB/s", HBM_PEAK_GBS),
           "kernel_ms_mean": mean_ms, "kernel_ms_flushed_median": med_ms, "timing": how, "algorithmic_bytes": nbytes}
    if cpu:
        from oracle import ref
        gs, us = w.tensors["gate"][:1024], w.tensors["up"][:1024]
        t = cpu_time(lambda: ref.swiglu_ref(gs, us))
        sb = 3 * gs.numel() * 2
        res["cpu_baseline"] = {"value": sb / t / 1e9, "unit": "GB/s",
                               "cores": torch.get_num_threads(), "kind": "port",
                               "sample": "first 1024 of 8192 rows, oracle.ref.swiglu_ref"}
    return res


def bench_rope(args, dev, flush, cpu):
    import tilelang
    from tilelang.testing import programs, workloads
    T_, H, D = 8192, 32, 128
    w = workloads.rope(T_, H, D)
    k = tilelang.compile(programs.rope_qk(T_, H, H, D), out_idx=[4, 5])
    nbytes = 4 * T_ * H * D * 2 + 2 * T_ * D * 2
    sets = []
    for _ in range(_copies_for(nbytes)):
        t = {n: w.tensors[n].to(dev) for n in ("q", "k", "cos", "sin")}
        sets.append((t["q"], t["k"], t["cos"], t["sin"], torch.empty_like(t["q"]),
                     torch.empty_like(t["k"])))
    fns = [lambda s=s: k(*s) for s in sets]
    pmc_launches(args, fns, "rope")
    ms, how = time_steps(fns, args.steps, args.warmup)
    mean_ms, med_ms = time_launches(fns, 200, flush)
    res = {"workload": "rope_qk_bf16_8192x32x128", "value": nbytes / (ms * 1e-3) / 1e9,
           "unit": "GB/s", "ms_per_step": ms, "dtype": "bf16",
           "roofline": roofline("hbm", nbytes / (mean_ms * 1e-3) / 1e9, "GB/s", HBM_PEAK_GBS),
           "kernel_ms_mean": mean_ms, "kernel_ms_flushed_median": med_ms, "timing": how, "algorithmic_bytes": nbytes}
    if cpu:
        from oracle import ref
        q, kk, c, s = (w.tensors[n][:1024] for n in ("q", "k", "cos", "sin"))
        t = cpu_time(lambda: (ref.rope_ref(q, c, s), ref.rope_ref(kk, c, s)))
        sb = 4 * q.numel() * 2 + 2 * c.numel() * 2
        res["cpu_baseline"] = {"value": sb / t / 1e9, "unit": "GB/s",
                               "cores": torch.get_num_threads(), "kind": "port",
                               "sample": "first 1024 of 8192 tokens, oracle.ref.rope_ref on q,k"}
    return res


def bench_gemm(args, dev, flush, cpu, M=4096, N=4096, K=4096, dtype=torch.float16):
    import tilelang
    from tilelang.testing import programs, workloads
    w = workloads.gemm(M, N, K, dtype=dtype)
    dn = "float16" if dtype == torch.float16 else "bfloat16"
    k = tilelang.compile(programs.matmul(M, N, K, 128, 128, 64, dn, "float16"), out_idx=-1)
    flops = 2 * M * N * K
    nbytes = 2 * (M * K + K * N + M * N)
    sets = []
    for _ in range(_copies_for(nbytes)):
        sets.append((w.tensors["a"].to(dev), w.tensors["b"].to(dev),
                     torch.empty(M, N, dtype=torch.float16, device=dev)))
    fns = [lambda s=s: k(*s) for s in sets]
    pmc_launches(args, fns, "gemm")
    ms, how = time_steps(fns, args.steps, args.warmup)
    mean_ms, med_ms = time_launches(fns, 50, flush)
    skinny = M <= 64
    if skinny:
        rl = roofline("hbm", nbytes / (mean_ms * 1e-3) / 1e9, "GB/s", HBM_PEAK_GBS)
    else:
        rl = roofline("mfma", flops / (mean_ms * 1e-3) / 1e12, "TFLOP/s", MFMA_PEAK["fp16"])
    res = {"workload": f"gemm_{dn}_{M}x{N}x{K}", "value": flops / (ms * 1e-3) / 1e12,
           "unit": "TFLOP/s", "ms_per_step": ms, "dtype": "f16" if dn == "float16" else "bf16",
           "roofline": rl, "kernel_ms_mean": mean_ms, "kernel_ms_flushed_median": med_ms, "timing": how,
           "algorithmic_flops": flops, "algorithmic_bytes": nbytes}
    if cpu:
        from oracle import ref
        rows = min(M, 512)
        a_s, b_s = w.tensors["a"][:rows], w.tensors["b"]
        t = cpu_time(lambda: ref.matmul_ref(a_s, b_s), reps=1)
        res["cpu_baseline"] = {"value": 2 * rows * N * K / t / 1e12, "unit": "TFLOP/s",
                               "cores": torch.get_num_threads(), "kind": "port",
                               "sample": f"first {rows} rows of A, oracle.ref.matmul_ref (fp32 "
                                         f"accumulate)"}
    return res


def bench_gemm_library(args, dev, flush, cpu, M=4096, N=4096, K=4096):
    """Comparator, not this library: torch.matmul on the same fp16 4096^3 operands (ROCm
    dispatches it to hipBLASLt), timed exactly as the gemm workload (graph of back-to-back
    launches over rotating copies, HIP events, settled clocks). Not in the default run."""
    from tilelang.testing import workloads
    w = workloads.gemm(M, N, K, dtype=torch.float16)
    flops = 2 * M * N * K
    nbytes = 2 * (M * K + K * N + M * N)
    sets = []
    for _ in range(_copies_for(nbytes)):
        sets.append((w.tensors["a"].to(dev), w.tensors["b"].to(dev),
                     torch.empty(M, N, dtype=torch.float16, device=dev)))
    fns = [lambda s=s: torch.matmul(s[0], s[1], out=s[2]) for s in sets]
    pmc_launches(args, fns, "gemm_library")
    ms, how = time_steps(fns, args.steps, args.warmup)
    mean_ms, med_ms = time_launches(fns, 50, flush)
    return {"workload": f"gemm_torch_matmul_float16_{M}x{N}x{K}",
            "value": flops / (ms * 1e-3) / 1e12, "unit": "TFLOP/s", "ms_per_step": ms,
            "dtype": "f16", "note": "comparator: torch.matmul (hipBLASLt), not this library",
            "roofline": roofline("mfma", flops / (mean_ms * 1e-3) / 1e12, "TFLOP/s",
                                 MFMA_PEAK["fp16"]),
            "kernel_ms_mean": mean_ms, "kernel_ms_flushed_median": med_ms, "timing": how,
            "algorithmic_flops": flops}


def bench_flashattn(args, dev, flush, cpu, S=4096, causal=True):
    import tilelang
    from tilelang.testing import programs, workloads
    B, H, D = 8, 32, 128
    w = workloads.flashattn(B, S, H, D, causal=causal)
    k = tilelang.compile(programs.flashattn(B, H, S, D, causal), out_idx=-1)
    flops = 4 * B * H * S * S * D * (0.5 if causal else 1.0)
    nbytes = 4 * B * S * H * D * 2  # Q, K, V read once, O written once
    q, kk, v = (w.tensors[n].to(dev) for n in ("q", "k", "v"))
    o = torch.empty_like(q)
    fns = [lambda: k(q, kk, v, o)]
    pmc_launches(args, fns, "flashattn")
    ms, how = time_steps(fns, args.steps, args.warmup)
    mean_ms, med_ms = time_launches(fns, 10, flush)
    res = {"workload": f"flashattn_bf16_b{B}h{H}s{S}d{D}_{'causal' if causal else 'full'}",
           "value": flops / (ms * 1e-3) / 1e12, "unit": "TFLOP/s", "ms_per_step": ms,
           "dtype": "bf16",
           "roofline": roofline("mfma", flops / (mean_ms * 1e-3) / 1e12, "TFLOP/s",
                                MFMA_PEAK["bf16"]),
           "kernel_ms_mean": mean_ms, "kernel_ms_flushed_median": med_ms, "timing": how,
           "algorithmic_flops": flops, "algorithmic_bytes": nbytes}
    if cpu:
        from oracle import ref
        t = cpu_time(lambda: ref.flashattn_ref(w.tensors["q"], w.tensors["k"], w.tensors["v"],
                                               causal, batches=[0], heads=[0, 1]), reps=1)
        sf = flops / (B * H) * 2
        res["cpu_baseline"] = {"value": sf / t / 1e12, "unit": "TFLOP/s",
                               "cores": torch.get_num_threads(), "kind": "port",
                               "sample": "batch 0, heads 0-1, oracle.ref.flashattn_ref"}
    return res


def bench_gemm_fp8(args, dev, flush, cpu):
    """FP8 GEMM (examples/gemm_fp8/example_tilelang_gemm_fp8_2xAcc.py structure: e4m3 A [M,K],
    B [N,K], fp32 C) at the GEMM config's 4096^3."""
    import tilelang
    from tilelang.testing import programs
    M = N = K = 4096
    g = torch.Generator().manual_seed(0)
    a = torch.randn(M, K, generator=g).to(torch.float8_e4m3fn)
    b = torch.randn(N, K, generator=g).to(torch.float8_e4m3fn)
    k = tilelang.compile(programs.matmul_fp8(M, N, K, 128, 128, 64, "e4m3_float8", two_acc=True),
                         out_idx=-1)
    flops = 2 * M * N * K
    nbytes = (M * K + N * K) + M * N * 4
    sets = [(a.to(dev), b.to(dev), torch.empty(M, N, dtype=torch.float32, device=dev))
            for _ in range(_copies_for(nbytes))]
    fns = [lambda s=s: k(*s) for s in sets]
    pmc_launches(args, fns, "gemm_fp8")
    ms, how = time_steps(fns, args.steps, args.warmup)
    mean_ms, med_ms = time_launches(fns, 10, flush)
    res = {"workload": f"gemm_fp8_e4m3_{M}x{N}x{K}_f32out", "value": flops / (ms * 1e-3) / 1e12,
           "unit": "TFLOP/s", "ms_per_step": ms, "dtype": "fp8-e4m3 in, fp32 accumulate",
           "roofline": roofline("mfma", flops / (mean_ms * 1e-3) / 1e12, "TFLOP/s",
                                MFMA_PEAK["fp8"]),
           "kernel_ms_mean": mean_ms, "kernel_ms_flushed_median": med_ms, "timing": how,
           "algorithmic_flops": flops, "algorithmic_bytes": nbytes}
    if cpu:
        from oracle import ref
        rows = 256
        t = cpu_time(lambda: ref.gemm_fp8_ref(a[:rows], b), reps=1)
        res["cpu_baseline"] = {"value": 2 * rows * N * K / t / 1e12, "unit": "TFLOP/s",
                               "cores": torch.get_num_threads(), "kind": "port",
                               "sample": f"first {rows} rows of A, oracle.ref.gemm_fp8_ref"}
    return res


def bench_flashattn_gqa(args, dev, flush, cpu):
    """examples/flash_attention/example_gqa_fwd_bshd.py defaults: batch 1, 64 heads, 16 groups
    (4 K/V heads), seq 8192, dim 128, fp16, non-causal; the upstream program structure."""
    import tilelang
    from tilelang.testing import programs
    B, H, G, S, D = 1, 64, 16, 8192, 128
    g = torch.Generator().manual_seed(0)
    q = torch.randn(B, S, H, D, generator=g).half()
    kk = torch.randn(B, S, H // G, D, generator=g).half()
    v = torch.randn(B, S, H // G, D, generator=g).half()
    k = tilelang.compile(programs.flashattn_gqa(B, H, S, D, False, G), out_idx=[3])
    flops = 4 * B * H * S * S * D
    nbytes = (2 * B * S * H * D + 2 * B * S * (H // G) * D) * 2
    sets = [(q.to(dev), kk.to(dev), v.to(dev), torch.empty(q.shape, dtype=q.dtype, device=dev))
            for _ in range(_copies_for(nbytes))]
    fns = [lambda s=s: k(*s) for s in sets]
    pmc_launches(args, fns, "flashattn_gqa")
    ms, how = time_steps(fns, args.steps, args.warmup)
    mean_ms, med_ms = time_launches(fns, 10, flush)
    res = {"workload": f"flashattn_gqa_fp16_b{B}h{H}g{G}s{S}d{D}_full",
           "value": flops / (ms * 1e-3) / 1e12, "unit": "TFLOP/s", "ms_per_step": ms,
           "dtype": "f16",
           "roofline": roofline("mfma", flops / (mean_ms * 1e-3) / 1e12, "TFLOP/s",
                                MFMA_PEAK["fp16"]),
           "kernel_ms_mean": mean_ms, "kernel_ms_flushed_median": med_ms, "timing": how,
           "algorithmic_flops": flops, "algorithmic_bytes": nbytes}
    if cpu:
        from oracle import ref
        t = cpu_time(lambda: ref.flashattn_ref(q, kk, v, False, heads=[0]), reps=1)
        res["cpu_baseline"] = {"value": flops / H / t / 1e12, "unit": "TFLOP/s",
                               "cores": torch.get_num_threads(), "kind": "port",
                               "sample": "head 0, oracle.ref.flashattn_ref"}
    return res


def bench_flashattn_varlen(args, dev, flush, cpu):
    """examples/flash_attention/example_mha_fwd_varlen.py program structure (unpadded Q/K/V,
    cu_seqlens, non-causal, fp16) at a prefill size: 16 sequences of U[512, 4096] tokens
    (queries and keys of one sequence equally long), 32 heads, dim 128. Algorithmic FLOPs
    = sum over sequences of 4 H D nq nk (the example's 2 matmuls, :372-373, per sequence)."""
    import tilelang
    from tilelang.testing import programs
    B, H, D = 16, 32, 128
    g = torch.Generator().manual_seed(0)
    lens = torch.randint(512, 4097, (B,), generator=g).tolist()
    cu = torch.tensor([0] + list(itertools.accumulate(lens)), dtype=torch.int32)
    T = int(cu[-1])
    q = torch.randn(T, H, D, generator=g).half()
    kk = torch.randn(T, H, D, generator=g).half()
    v = torch.randn(T, H, D, generator=g).half()
    k = tilelang.compile(programs.flashattn_varlen(B, T, T, H, D), out_idx=-1)
    flops = sum(4 * H * D * n * n for n in lens)
    nbytes = 4 * T * H * D * 2
    qd, kd, vd, cud = q.to(dev), kk.to(dev), v.to(dev), cu.to(dev)
    o = torch.empty_like(qd)
    fns = [lambda: k(qd, kd, vd, cud, cud, max(lens), o)]
    pmc_launches(args, fns, "flashattn_varlen")
    ms, how = time_steps(fns, args.steps, args.warmup)
    mean_ms, med_ms = time_launches(fns, 10, flush)
    res = {"workload": f"flashattn_varlen_fp16_b{B}h{H}d{D}_tokens{T}_full",
           "value": flops / (ms * 1e-3) / 1e12, "unit": "TFLOP/s", "ms_per_step": ms,
           "dtype": "f16",
           "roofline": roofline("mfma", flops / (mean_ms * 1e-3) / 1e12, "TFLOP/s",
                                MFMA_PEAK["fp16"]),
           "kernel_ms_mean": mean_ms, "kernel_ms_flushed_median": med_ms, "timing": how,
           "algorithmic_flops": flops, "algorithmic_bytes": nbytes, "seqlens": lens}
    if cpu:
        from oracle import ref
        n0 = lens[0]
        t = cpu_time(lambda: ref.flashattn_varlen_ref(q[:n0, :1], kk[:n0, :1], v[:n0, :1],
                                                      cu[:2], cu[:2]), reps=1)
        res["cpu_baseline"] = {"value": 4 * D * n0 * n0 / t / 1e12, "unit": "TFLOP/s",
                               "cores": torch.get_num_threads(), "kind": "port",
                               "sample": f"sequence 0 ({n0} tokens), head 0, "
                                         "oracle.ref.flashattn_varlen_ref"}
    return res


def bench_flashattn_bhsd(args, dev, flush, cpu):
    """examples/flash_attention/example_mha_fwd_bhsd.py program structure (head-major Q, K, V,
    seq_q != seq_kv, non-causal, fp16) at a chunked-prefill size: 1024 new queries over 8192
    keys, batch 4, 32 heads, dim 128. Algorithmic FLOPs = 4 B H S_q S_kv D (two matmuls)."""
    import tilelang
    from tilelang.testing import programs
    B, H, Sq, Sk, D = 4, 32, 1024, 8192, 128
    g = torch.Generator().manual_seed(0)
    q = torch.randn(B, H, Sq, D, generator=g).half()
    kk = torch.randn(B, H, Sk, D, generator=g).half()
    v = torch.randn(B, H, Sk, D, generator=g).half()
    k = tilelang.compile(programs.flashattn_bhsd(B, H, Sq, Sk, D, False), out_idx=[3])
    flops = 4 * B * H * Sq * Sk * D
    nbytes = (2 * B * H * Sq * D + 2 * B * H * Sk * D) * 2
    qd, kd, vd = q.to(dev), kk.to(dev), v.to(dev)
    o = torch.empty_like(qd)
    fns = [lambda: k(qd, kd, vd, o)]
    pmc_launches(args, fns, "flashattn_bhsd")
    ms, how = time_steps(fns, args.steps, args.warmup)
    mean_ms, med_ms = time_launches(fns, 10, flush)
    res = {"workload": f"flashattn_bhsd_fp16_b{B}h{H}sq{Sq}skv{Sk}d{D}_full",
           "value": flops / (ms * 1e-3) / 1e12, "unit": "TFLOP/s", "ms_per_step": ms,
           "dtype": "f16",
           "roofline": roofline("mfma", flops / (mean_ms * 1e-3) / 1e12, "TFLOP/s",
                                MFMA_PEAK["fp16"]),
           "kernel_ms_mean": mean_ms, "kernel_ms_flushed_median": med_ms, "timing": how,
           "algorithmic_flops": flops, "algorithmic_bytes": nbytes}
    if cpu:
        from oracle import ref
        t = cpu_time(lambda: ref.flashattn_bhsd_ref(q[:1, :1], kk[:1, :1], v[:1, :1], False),
                     reps=1)
        res["cpu_baseline"] = {"value": flops / (B * H) / t / 1e12, "unit": "TFLOP/s",
                               "cores": torch.get_num_threads(), "kind": "port",
                               "sample": "batch 0, head 0, oracle.ref.flashattn_bhsd_ref"}
    return res


def bench_flashattn_inference(args, dev, flush, cpu):
    """examples/flash_attention/example_mha_inference.py at its own defaults (:279-289): batch 1,
    32 heads, 128 queries over 8192 keys, dim 128, fp16, 4 key splits; through
    ``tilelang.compile``, the program's glse / Output_partial written and combined. Algorithmic
    FLOPs = 4 B H S_q S_kv D (two matmuls); algorithmic bytes = Q, K, V read once plus the
    program's three outputs (Output, Output_partial, glse) written once. At 128 queries per key
    the call does 126 FLOP per byte, under the 312 of the MFMA / HBM ridge (2.5 PFLOP/s over
    8 TB/s), so its roofline is HBM."""
    import tilelang
    from tilelang.testing import programs
    B, H, Sq, Sk, D, ns = 1, 32, 128, 8192, 128, 4
    g = torch.Generator().manual_seed(0)
    q = torch.randn(B, Sq, H, D, generator=g).half()
    kk = torch.randn(B, Sk, H, D, generator=g).half()
    v = torch.randn(B, Sk, H, D, generator=g).half()
    k = tilelang.compile(programs.mha_inference(B, H, Sq, Sk, D, num_split=ns), out_idx=[5])
    flops = 4 * B * H * Sq * Sk * D
    nbytes = (2 * B * Sq * H * D + 2 * B * Sk * H * D + B * Sq * H * ns * D + B * H * ns * Sq) * 2
    assert flops / nbytes < MFMA_PEAK["fp16"] * 1e3 / HBM_PEAK_GBS  # below the ridge: HBM-bound
    sets = []
    for _ in range(_copies_for(nbytes)):
        sets.append([q.to(dev), kk.to(dev), v.to(dev),
                     torch.empty(B, H, ns, Sq, dtype=torch.half, device=dev),
                     torch.empty(B, Sq, H, ns, D, dtype=torch.half, device=dev),
                     torch.empty(B, Sq, H, D, dtype=torch.half, device=dev)])
    fns = [lambda t=t: k(*t) for t in sets]
    pmc_launches(args, fns, "flashattn_inference")
    ms, how = time_steps(fns, args.steps, args.warmup)
    mean_ms, med_ms = time_launches(fns, 20, flush)
    res = {"workload": f"flashattn_inference_fp16_b{B}h{H}sq{Sq}skv{Sk}d{D}_split{ns}",
           "value": flops / (ms * 1e-3) / 1e12, "unit": "TFLOP/s", "ms_per_step": ms,
           "dtype": "f16",
           "roofline": roofline("hbm", nbytes / (mean_ms * 1e-3) / 1e9, "GB/s", HBM_PEAK_GBS),
           "mfma_frac": round(flops / (mean_ms * 1e-3) / 1e12 / MFMA_PEAK["fp16"], 4),
           "kernel_ms_mean": mean_ms, "kernel_ms_flushed_median": med_ms, "timing": how,
           "algorithmic_flops": flops, "algorithmic_bytes": nbytes,
           "note": "whole call: the key-part attention kernel plus the split combine"}
    if cpu:
        from oracle import ref
        t = cpu_time(lambda: ref.mha_inference_ref(q[:, :, :1], kk[:, :, :1], v[:, :, :1]),
                     reps=3)
        res["cpu_baseline"] = {"value": flops / H / t / 1e12, "unit": "TFLOP/s",
                               "cores": torch.get_num_threads(), "kind": "port",
                               "sample": "head 0, oracle.ref.mha_inference_ref"}
    return res


def bench_mla(args, dev, flush, cpu):
    from tilelang.jit.adapter.mi355x import ops
    from tilelang.testing import workloads
    w = workloads.mla()
    a = w.attrs
    B, Hq, dv, dpe = a["B"], a["Hq"], a["dv"], a["dpe"]
    sum_l = int(w.tensors["seqlens"].sum())
    nbytes = sum_l * (dv + dpe) + B * Hq * (dv + dpe) * 2 + B * Hq * dv * 2 + \
        w.tensors["block_table"].numel() * 4 + B * 4
    flops = sum_l * Hq * (dv + dpe + dv) * 2
    num_split = args.mla_splits
    ws = torch.empty(ops.mla_workspace_bytes(B, Hq, dv, num_split), dtype=torch.uint8,
                     device=dev)
    # input copies (the whole KV pool, Q, table, lengths, scale) so that no launch reads the
    # previous launch's KV from the Infinity Cache; the workspace is shared (scratch written and
    # read within one call, as in a decode loop)
    sets = []
    for _ in range(_copies_for(nbytes)):
        t = {n: x.to(dev) for n, x in w.tensors.items()}
        t["out"] = torch.empty(B, Hq, dv, dtype=torch.bfloat16, device=dev)
        sets.append(t)

    def run(t):
        q, kv = t["q"], t["kv"]
        ops.mla_decode(q[..., :dv], q[..., dv:], kv[:, :dv], kv[:, dv:], t["block_table"],
                       t["seqlens"], t["out"], ws, a["page"], num_split, a["sm_scale"],
                       t["kv_scale"])

    fns = [lambda t=t: run(t) for t in sets]
    pmc_launches(args, fns, "mla")
    ms, how = time_steps(fns, args.steps, args.warmup)
    mean_ms, med_ms = time_launches(fns, 100, flush)
    # The config is bounded by HBM (576 B per cached token, Q, O, table, lengths), so
    # roofline.frac is against 8 TB/s. The matrix-core rate is reported beside it: algorithmic
    # flops over the bf16-equivalent peak, and the executed e4m3 flops (Q^T runs as two e4m3
    # terms, P^T as one) over the fp8 peak. Durations are whole tlm_mla_decode calls (prep +
    # decode + combine).
    res = {"workload": "mla_decode_fp8_b64_h128_d576", "value": nbytes / (ms * 1e-3) / 1e9,
           "unit": "GB/s", "ms_per_step": ms,
           "dtype": "fp8e4m3 (kv; q as two e4m3 terms, p as one)",
           "roofline": roofline("hbm", nbytes / (mean_ms * 1e-3) / 1e9, "GB/s", HBM_PEAK_GBS),
           "tflops": flops / (mean_ms * 1e-3) / 1e12,
           "mfma_frac_bf16_equivalent": flops / (mean_ms * 1e-3) / 1e12 / MFMA_PEAK["bf16"],
           "executed_fp8_tflops": MLA_EXEC_FACTOR * flops / (mean_ms * 1e-3) / 1e12,
           "kernel_ms_mean": mean_ms, "kernel_ms_flushed_median": med_ms, "timing": how,
           "algorithmic_bytes": nbytes, "algorithmic_flops": flops, "sum_seqlens": sum_l,
           "num_split": num_split}
    if cpu:
        from oracle import ref
        nb = 4
        got = {}

        def oracle_sample():
            got["ref"] = ref.mla_decode_ref(
                w.tensors["q"][:nb, :, :dv], w.tensors["q"][:nb, :, dv:], w.tensors["kv"][:, :dv],
                w.tensors["kv"][:, dv:], w.tensors["block_table"], w.tensors["seqlens"][:nb],
                a["page"], a["sm_scale"], float(w.tensors["kv_scale"]), out_dtype=torch.float32)

        t0 = cpu_time(oracle_sample, reps=1)
        # the error this throughput is bought with: the GPU output of the same sequences against
        # the dequantised fp32 oracle (the FP8 bound of the config is 3% relative RMS)
        run(sets[0])
        o = sets[0]["out"][:nb].float().cpu()
        e = got["ref"]
        res["accuracy"] = {
            "rel_rms": float(((o - e).pow(2).mean() / e.pow(2).mean()).sqrt()),
            "max_abs": float((o - e).abs().max()),
            "sample": f"first {nb} of {B} sequences against oracle.ref.mla_decode_ref (fp32)"}
        sl = int(w.tensors["seqlens"][:nb].sum())
        sb = sl * (dv + dpe) + nb * Hq * (dv + dpe) * 2 + nb * Hq * dv * 2 + \
            w.tensors["block_table"][:nb].numel() * 4 + nb * 4
        res["cpu_baseline"] = {"value": sb / t0 / 1e9, "unit": "GB/s",
                               "cores": torch.get_num_threads(), "kind": "port",
                               "sample": f"first {nb} of {B} sequences ({sl} tokens), "
                                         f"oracle.ref.mla_decode_ref"}
    return res


def bench_mla_program(args, dev, flush, cpu):
    """The reference's split MLA program (example_mla_decode_paged.py with num_split 4, fp8 KV,
    bf16 Q / Output, fp32 glse / Output_partial as it declares them) through tilelang.compile
    at the MLA config: the drop-in path, partials written. Priced against HBM with the
    partials it writes counted in its bytes."""
    import tilelang
    from tilelang.testing import programs, workloads
    w = workloads.mla()
    a = w.attrs
    B, Hq, dv, dpe, page, mp = a["B"], a["Hq"], a["dv"], a["dpe"], a["page"], a["max_pages"]
    ns = 4
    k = tilelang.compile(programs.mla_decode(B, Hq, 1, mp * page, dv, dpe, 64, 64, ns, page,
                                             dtype="bfloat16", kv_dtype="float8_e4m3",
                                             out_dtype="bfloat16"), out_idx=[8])
    sum_l = int(w.tensors["seqlens"].sum())
    nbytes = sum_l * (dv + dpe) + B * Hq * (dv + dpe) * 2 + B * Hq * dv * 2 + \
        w.tensors["block_table"].numel() * 4 + B * 4 + B * Hq * ns * (dv + 1) * 4
    sets = []
    for _ in range(_copies_for(nbytes)):
        T = w.tensors
        pool = T["kv"].view(B * mp * page, 1, dv + dpe)
        sets.append((T["q"][..., :dv].contiguous().to(dev), T["q"][..., dv:].contiguous().to(dev),
                     pool[..., :dv].contiguous().to(dev), pool[..., dv:].contiguous().to(dev),
                     T["block_table"].to(dev), T["seqlens"].to(dev),
                     torch.empty(B, Hq, ns, device=dev), torch.empty(B, Hq, ns, dv, device=dev),
                     torch.empty(B, Hq, dv, dtype=torch.bfloat16, device=dev),
                     T["kv_scale"].to(dev)))
    fns = [lambda s=s: k(*s) for s in sets]
    pmc_launches(args, fns, "mla_program")
    ms, how = time_steps(fns, args.steps, args.warmup)
    mean_ms, med_ms = time_launches(fns, 50, flush)
    return {"workload": "mla_split_program_fp8_b64_h128_d576_split4", "value":
            nbytes / (ms * 1e-3) / 1e9, "unit": "GB/s", "ms_per_step": ms,
            "dtype": "fp8e4m3 (kv; q as two e4m3 terms, p as one)",
            "roofline": roofline("hbm", nbytes / (mean_ms * 1e-3) / 1e9, "GB/s", HBM_PEAK_GBS),
            "kernel_ms_mean": mean_ms, "kernel_ms_flushed_median": med_ms, "timing": how,
            "algorithmic_bytes": nbytes, "path": "tilelang.compile (TPU convention, all "
            "parameters on the device)"}


def bench_copy(args, dev, flush, cpu):
    """Calibration kernel for the HBM counters: a 1 GiB device-to-device copy (torch's copy
    kernel) reads 1 GiB and writes 1 GiB."""
    src = torch.empty(1 << 30, dtype=torch.uint8, device=dev).fill_(1)
    dst = torch.empty_like(src)
    fns = [lambda: dst.copy_(src)]
    pmc_launches(args, fns, "copy")
    ms, how = time_steps(fns, args.steps, args.warmup)
    return {"workload": "copy_1GiB", "value": 2 * src.numel() / (ms * 1e-3) / 1e9, "unit": "GB/s",
            "ms_per_step": ms, "dtype": "u8", "timing": how,
            "roofline": roofline("hbm", 2 * src.numel() / (ms * 1e-3) / 1e9, "GB/s",
                                 HBM_PEAK_GBS)}


def bench_kv_append(args, dev, flush, cpu):
    """Paged KV append + e4m3 quantisation (the step before the MLA decode) at a prefill-sized
    chunk: 64 sequences x 512 new latent tokens x 576 dims, bf16 in, fp8 pages out."""
    from tilelang.jit.adapter.mi355x import ops
    B, T, D, page = 64, 512, 576, 64
    pages = 128
    g = torch.Generator().manual_seed(0)
    x = torch.randn(B, T, D, generator=g).to(torch.bfloat16)
    bt = torch.randperm(B * pages, generator=g).view(B, pages).to(torch.int32)
    start = torch.randint(0, pages * page - T, (B,), generator=g, dtype=torch.int32)
    count = torch.full((B,), T, dtype=torch.int32)
    scale = torch.tensor([float(x.float().abs().max()) / 448.0], dtype=torch.float32)
    nbytes = B * T * D * (2 + 1) + B * pages * 4 + 2 * B * 4
    sets = []
    for _ in range(_copies_for(nbytes)):
        xs, bts, sts, cns, scs = (t.to(dev) for t in (x, bt, start, count, scale))
        kv = torch.zeros(B * pages * page, D, dtype=torch.float8_e4m3fn, device=dev)
        sets.append((xs, sts, cns, bts, kv, page, scs))
    fns = [lambda s=s: ops.kv_append_fp8(*s) for s in sets]
    pmc_launches(args, fns, "kv_append")
    ms, how = time_steps(fns, args.steps, args.warmup)
    mean_ms, med_ms = time_launches(fns, 200, flush)
    res = {"workload": "kv_append_fp8_b64_t512_d576", "value": nbytes / (ms * 1e-3) / 1e9,
           "unit": "GB/s", "ms_per_step": ms, "dtype": "bf16 in, fp8e4m3 out",
           "roofline": roofline("hbm", nbytes / (mean_ms * 1e-3) / 1e9, "GB/s", HBM_PEAK_GBS),
           "kernel_ms_mean": mean_ms, "kernel_ms_flushed_median": med_ms, "timing": how,
           "algorithmic_bytes": nbytes}
    if cpu:
        from oracle import ref
        nb = 4
        pool = torch.zeros(B * pages * page, D, dtype=torch.uint8).numpy()
        t = cpu_time(lambda: ref.kv_append_fp8_ref(x[:nb], start[:nb].numpy(), count[:nb].numpy(),
                                                   bt[:nb].numpy(), pool, page, float(scale)),
                     reps=1)
        res["cpu_baseline"] = {"value": nbytes * nb / B / t / 1e9, "unit": "GB/s",
                               "cores": torch.get_num_threads(), "kind": "port",
                               "sample": f"first {nb} of {B} sequences, oracle.ref.kv_append_fp8_ref"}
    return res


def summarize_trace(path):
    """Markdown summary of a rocprofv3 kernel trace (run_kernel_trace.csv) of this script: per
    kernel, all dispatches and the dispatches inside each marker-bracketed timed window (two
    windows per workload, in run order: the timed steps, then the back-to-back launch graph)."""
    import csv
    rows = []
    with open(path) as f:
        for r in csv.DictReader(f):
            rows.append((int(r["Start_Timestamp"]), int(r["End_Timestamp"]), r["Kernel_Name"]))
    rows.sort()
    windows, cur, inside = [], [], False
    for st, en, name in rows:
        if MARKER_KERNEL in name:
            if inside:
                if cur:  # an empty pair is the marker's warm-up at start-up
                    windows.append(cur)
                cur = []
            inside = not inside
        elif inside:
            cur.append((name, en - st, st, en))

    def short(name):
        n = name.split("(")[0] if not name.startswith("void (") else name
        return n[:110]

    def table(disp, title):
        by = {}
        for name, d, *_ in disp:
            by.setdefault(name, []).append(d)
        out = [f"**{title}**", "", "| Kernel | Calls | Avg ns | Median ns | Min ns | Max ns |",
               "|---|---|---|---|---|---|"]
        for name, ds in sorted(by.items(), key=lambda kv: -sum(kv[1])):
            ds = sorted(ds)
            out.append(f"| `{short(name)}` | {len(ds)} | {sum(ds) / len(ds):.0f} | "
                       f"{ds[len(ds) // 2]} | {ds[0]} | {ds[-1]} |")
        return out

    lines = table([(n, e - s_) for s_, e, n in rows if MARKER_KERNEL not in n],
                  f"All dispatches ({path.split('/')[-1]})")
    for i, w in enumerate(windows):
        span = (w[-1][3] - w[0][2]) if w else 0
        kind = "timed steps" if i % 2 == 0 else "back-to-back launch graph (roofline.achieved)"
        lines += [""] + table(w, f"Window {i + 1}: {kind}, first start to last end "
                                 f"{span / 1e3:.1f} us")
    return "\n".join(lines)


BENCHES = {
    "copy": bench_copy,
    "gemm": bench_gemm,
    "gemm_skinny": lambda a, d, f, c: bench_gemm(a, d, f, c, M=16, N=14336, K=4096),
    "rmsnorm": bench_rmsnorm,
    "rope": bench_rope,
    "swiglu": bench_swiglu,
    "flashattn": bench_flashattn,
    "flashattn_s2048": lambda a, d, f, c: bench_flashattn(a, d, f, c, S=2048, causal=False),
    "flashattn_inference": bench_flashattn_inference,
    "gemm_library": bench_gemm_library,
    "flashattn_gqa": bench_flashattn_gqa,
    "flashattn_varlen": bench_flashattn_varlen,
    "flashattn_bhsd": bench_flashattn_bhsd,
    "gemm_fp8": bench_gemm_fp8,
    "mla": bench_mla,
    "mla_program": bench_mla_program,
    "kv_append": bench_kv_append,
}
ORDER = ["gemm", "gemm_skinny", "rmsnorm", "rope", "swiglu", "flashattn", "flashattn_s2048",
         "flashattn_gqa", "flashattn_varlen", "flashattn_bhsd", "flashattn_inference", "gemm_fp8",
         "mla", "mla_program", "kv_append"]


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", default="all", choices=["all", "copy", "gemm_library"] + ORDER)
    ap.add_argument("--pmc-launches", type=int, default=0,
                    help="only launch the workload's kernel N times (for rocprofv3 --pmc)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--mla-splits", type=int, default=4)
    ap.add_argument("--no-clock", action="store_true",
                    help="skip the shader-clock pass of the matrix-core workloads")
    ap.add_argument("--summarize-trace", metavar="CSV",
                    help="print a markdown summary of a rocprofv3 kernel trace of this script "
                         "(all dispatches and the marker-bracketed timed windows), then exit")
    args = ap.parse_args()
    if args.summarize_trace:
        print(summarize_trace(args.summarize_trace))
        return
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only (every kernel here is a "
                                   "single-GPU kernel); run with --gpus 1"}))
        sys.exit(2)
    if not torch.cuda.is_available():
        print(json.dumps({"error": "no GPU visible"}))
        sys.exit(2)
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    torch.set_num_threads(os.cpu_count() or 1)
    flush = torch.empty(FLUSH_BYTES // 4, dtype=torch.int32, device=dev)
    _MARKER[:] = [torch.zeros(1, dtype=torch.int16, device=dev)]
    # the first launch of the marker kernel loads its code object (a host stall of 40-110 ms);
    # done here, it cannot leave the GPU idle between a settle phase and a timed replay (after
    # such an idle spell the clocks boost and then dip inside the timed window)
    _mark()
    _mark()
    torch.cuda.synchronize()
    names = ORDER if args.workload == "all" else [args.workload]
    traffic = load_traffic()
    results = {}
    for n in names:
        log(f"[bench] {n} ...")
        try:
            results[n] = BENCHES[n](args, dev, flush, not args.no_cpu)
            if results[n].get("cpu_baseline"):
                results[n]["cpu_baseline"]["cpu_model"] = cpu_model()
            tb = traffic.get(results[n].get("workload"))
            if tb is not None and results[n].get("roofline"):
                results[n]["roofline"]["traffic"] = tb
            rl = results[n].get("roofline") or {}
            if rl.get("bound") == "mfma" and not args.no_clock:
                mhz = settled_sclk(_LAST_FNS)
                if mhz:  # the spec peak assumes 2400 MHz; the roofline above keeps the spec peak
                    at_clk = rl["peak"] * mhz / 2400.0
                    results[n]["sclk"] = {
                        "mhz": mhz, "source": "pp_dpm_sclk, last 0.75 s of 1.5 s back to back",
                        "peak_at_sclk": round(at_clk, 1),
                        "frac_at_sclk": round(rl["achieved"] / at_clk, 4)}
            log(f"[bench] {n}: {results[n]['value']:.1f} {results[n]['unit']} "
                f"(roofline {results[n]['roofline']['frac'] * 100:.1f}%)")
        except PmcOnly:
            print(json.dumps({"pmc_launches": args.pmc_launches, "workload": n}))
            return
        except Exception as e:  # a family without a kernel yet is reported, not fatal
            results[n] = {"workload": n, "error": f"{type(e).__name__}: {e}"}
            log(f"[bench] {n}: ERROR {e}")
        torch.cuda.empty_cache()
    head_name = "gemm" if args.workload == "all" else args.workload
    head = results.get(head_name, {})
    if "error" in head:
        ok = [n for n in names if "error" not in results[n]]
        head_name = ok[0] if ok else head_name
        head = results.get(head_name, {})
    line = {
        "metric": METRIC,
        "value": head.get("value"),
        "unit": head.get("unit"),
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": head.get("ms_per_step"),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": head.get("dtype"),
        "data": "synthetic (seed 0, BASELINE.json configs)",
        "config": {"workload": head.get("workload", head_name), "device": torch.cuda.get_device_name(dev)},
        "roofline": head.get("roofline"),
        "sclk": head.get("sclk"),
        "cpu_baseline": head.get("cpu_baseline"),
        "configs": [results[n] for n in names],
        "host": {"cpu_count": os.cpu_count(), "torch_threads": torch.get_num_threads(),
                 "cpu_model": cpu_model()},
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
