"""PoM layer benchmark on one MI355X: forward + backward tokens/s, per-kernel
roofline fractions and a CPU baseline, printed as ONE JSON line.

  python bench.py [--gpus 1] [--steps K] [--warmup W] [--config c2|c3|c4|c5|c2h]
                  [--sub-configs c3,c4,c5,c2h] [--no-cpu] [--no-flush] [--graph]

A step is one forward + backward of one PoM layer over one batch of synthetic
input that is resident in HBM before the timed region starts (x, upstream
gradient and weights).  The default workload is config 2 of the baseline
(image-DiT layer: B=16, N=1024, D=1152, degree 2, expand 2, bf16).  Every
launch of the layer (six projection GEMMs, aggregation and gating kernels) is
bracketed by HIP events on its launch stream in a second, instrumented pass
of the same K steps (events cost ~5 % of a step, so the headline pass runs
without them), giving each kernel's average duration; the roofline object
reports the kernel that takes the most time per step, and "kernels" reports
all of them.

Roofline fractions are in algorithmic units: the bytes (or flops) the
operation itself needs per launch.  A kernel that also writes a channel-major
copy of its output for a backward GEMM on hipBLASLt reports the copy bytes
separately ("copy_bytes", "frac_with_copies"); with the weight gradients on
pom_gemm no copy is written and the fields are absent.

Besides the headline configuration, the same JSON line carries one object per
other configuration ("configs": C3-C5 and c2h by default) with its fwd and
fwd+bwd tokens/s, its dominant-kernel roofline, the streaming / GEMM group
fractions and its own CPU baseline.  "mall_flushed" repeats the headline step
with 1 GiB written before every step (the Infinity Cache and L2 cold at the
layer's start), and times each streaming kernel standalone, back to back
(warm) and after a 1 GiB write before every launch (cold).

The CPU baseline runs the oracle (a pure-PyTorch restatement of the reference
path) on the host cores on a bounded sample of the same workload, fp32 and
bf16, forward and forward + backward.
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

METRIC = "PoM layer fwd+bwd tokens/sec at B=16,N=1024,D=1152 bf16; % HBM/MFMA roofline"
HBM_PEAK = 8.0e12          # B/s, MI355X HBM3E
MFMA_BF16_PEAK = 2.5e15    # FLOP/s, MI355X dense bf16

# name: (B, N, D, degree, expand, variant, extra)
CONFIGS = {
    "c2": dict(B=16, N=1024, D=1152, K=2, E=2, variant="mean",
               workload="C2 image-DiT PoM layer fwd+bwd (B=16, N=1024, D=1152, degree=2, expand=2)"),
    "c3": dict(B=32, N=2048, D=1024, K=3, E=2, variant="masked",
               workload="C3 masked PoM layer fwd+bwd (B=32, N=2048, D=1024, degree=3, expand=2, "
                        "valid length U[256,2048])"),
    "c4": dict(B=4, N=16384, D=1024, K=2, E=4, variant="block", frame_len=1024,
               workload="C4 block-causal video PoM layer fwd+bwd (B=4, 16 frames x 1024, D=1024, "
                        "degree=2, expand=4)"),
    "c5": dict(B=8, N=4096, D=1536, K=2, E=2, variant="rope2d", H=64, W=64,
               workload="C5 2-D RoPE PoM layer fwd+bwd (B=8, N=4096 on 64x64, D=1536, degree=2, expand=2)"),
    # the reference's own benchmarks gate per head (n_sel_heads = num_heads = 16)
    "c2h": dict(B=16, N=1024, D=1152, K=2, E=2, variant="mean", heads=16,
                workload="C2 PoM layer fwd+bwd with n_sel_heads=16 (B=16, N=1024, D=1152, degree=2, expand=2)"),
}


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--config", default="c2", choices=sorted(CONFIGS))
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baselines")
    ap.add_argument("--sub-configs", default="c3,c4,c5,c2h",
                    help="comma-separated other configurations measured into the same JSON line ('' for none)")
    ap.add_argument("--sub-cpu-seconds", type=float, default=6.0, help="CPU baseline budget per sub-config")
    ap.add_argument("--no-flush", action="store_true", help="skip the MALL-flushed measurements")
    ap.add_argument("--cpu-seconds", type=float, default=15.0, help="CPU baseline time budget")
    ap.add_argument("--no-kernel-timing", action="store_true",
                    help="time the steps without per-launch events")
    ap.add_argument("--graph", action="store_true",
                    help="capture one forward+backward step in a HIP graph and time its replays "
                         "(host launch overhead removed); per-kernel events are not available then")
    ap.add_argument("--pmc-summary", nargs=4, metavar=("FETCH_DB", "WRITE_DB", "COPY_FETCH_DB", "COPY_WRITE_DB"),
                    help="turn four rocprofv3 --pmc databases (FETCH_SIZE and WRITE_SIZE of a bench run and "
                         "of a --copy-calib run) into per-kernel HBM traffic; writes profiles/traffic_<config>.json")
    ap.add_argument("--pmc-table", nargs="+", metavar=("DB", "COUNTER"),
                    help="per launch group, the mean of each named counter per dispatch in one rocprofv3 --pmc "
                         "database of a bench run (e.g. MfmaUtil MfmaFlopsBF16 for the GEMMs); writes "
                         "profiles/pmc_<config>_<first counter>.json")
    ap.add_argument("--trace-summary", metavar="TRACE_DIR",
                    help="summarise a rocprofv3 --kernel-trace --stats --output-format csv directory "
                         "(run_kernel_stats.csv, run_kernel_trace.csv) of a bench run: per-kernel calls and "
                         "average duration, projection GEMMs labelled by dispatch order")
    ap.add_argument("--copy-calib", type=float, default=0.0,
                    help="instead of the layer, run a plain device copy of this many MiB "
                         "(calibrates rocprofv3 FETCH_SIZE / WRITE_SIZE)")
    return ap.parse_args()


# ---------------------------------------------------------------------------
# Workload construction (identical seeded inputs for the GPU and CPU legs)
# ---------------------------------------------------------------------------

def make_inputs(cfg):
    import torch
    g1 = torch.Generator().manual_seed(1)
    g2 = torch.Generator().manual_seed(2)
    x = torch.randn(cfg["B"], cfg["N"], cfg["D"], generator=g1)
    go = torch.randn(cfg["B"], cfg["N"], cfg["D"], generator=g2)
    extra = {}
    if cfg["variant"] == "masked":
        g3 = torch.Generator().manual_seed(3)
        lens = torch.randint(256, cfg["N"] + 1, (cfg["B"],), generator=g3)
        extra["mask"] = torch.arange(cfg["N"]).view(1, -1) < lens.view(-1, 1)
        extra["lens"] = lens
    if cfg["variant"] == "rope2d":
        H, W = cfg["H"], cfg["W"]
        extra["positions_hw"] = torch.stack(torch.meshgrid(torch.arange(H), torch.arange(W), indexing="ij"),
                                            -1).reshape(-1, 2)
    return x, go, extra


def _native_sequence() -> bool:
    """Whether the layer's steps run the C++ launch sequence (pom_layer_fwd /
    _bwd) rather than the Python one."""
    from pom_amd import ops
    return ops.native_layer_calls[0] > 0


def make_module(cfg):
    import torch
    import pom_amd
    torch.manual_seed(0)
    heads = cfg.get("heads", 1)
    if cfg["variant"] == "rope2d":
        return pom_amd.PoMRoPE(cfg["D"], cfg["K"], cfg["E"], 1, heads, False, max_h=cfg["H"], max_w=cfg["W"],
                               rope_2d=True)
    return pom_amd.PoM(cfg["D"], cfg["K"], cfg["E"], 1, heads, False)


def forward_fn(cfg, extra_dev):
    import pom_amd
    v = cfg["variant"]
    if v == "mean":
        return lambda m, x: m(x)
    if v == "masked":
        return lambda m, x: m(x, mask=extra_dev["mask"])
    if v == "block":
        desc = pom_amd.block_causal(cfg["frame_len"])
        return lambda m, x: m(x, mask=desc)
    if v == "rope2d":
        return lambda m, x: m(x, positions_hw=extra_dev["positions_hw"])
    raise ValueError(v)


# ---------------------------------------------------------------------------
# Algorithmic work per kernel launch
# ---------------------------------------------------------------------------

def copies_written(cfg):
    """(shᵀ, dYᵀ): whether the layer's bf16 training step writes the channel-major
    copies.  The gate forward writes shᵀ when dW_ag runs on hipBLASLt; the gate and
    aggregation backward write dYᵀ when dW_qc does.  A weight gradient on pom_gemm
    reads the token-major operand in place, and no copy is written."""
    import torch
    from pom_amd import ops
    if not (ops._NT_GEMMS and ops._NT_COPIES == "fused"):
        return False, False
    B, N, D, E = cfg["B"], cfg["N"], cfg["D"], cfg["E"]
    T, P, H = B * N, E * D, cfg.get("heads", 1)
    W = ops._padded_width(P, H if H > 1 else P)
    return (not ops.hip_gemm_fits("gemm_ag_wgrad", D, P, T, torch.bfloat16),
            not ops.hip_gemm_fits("gemm_qc_wgrad", W, D, T, torch.bfloat16))


def kernel_work(cfg, extra):
    """name -> (bound, algorithmic bytes or flops per launch, what one unit is)."""
    B, N, D, K, E = cfg["B"], cfg["N"], cfg["D"], cfg["K"], cfg["E"]
    T, P, e = B * N, E * D, 2
    H = cfg.get("heads", 1)
    S = H if H > 1 else P   # gate columns of Y: one per head, or one per channel
    Q = P + S               # useful projection width (padding columns are not counted)
    G = {"mean": 1, "masked": 1, "block": N // cfg.get("frame_len", N), "rope2d": 1}[cfg["variant"]]
    read_tok = T
    if cfg["variant"] == "masked":
        read_tok = int(extra["lens"].sum())
    agg_out = B * G * P * e
    rope_tab = 0
    if cfg["variant"] == "rope2d":
        rope_tab = 0   # tables are (64, P/4) fp32: cache resident, not counted
    mask_b = B * N * 4 if cfg["variant"] == "masked" else 0
    # channel-major copies written in the same pass: only for a weight gradient that stays on hipBLASLt
    sh_copy, dy_copy = copies_written(cfg)
    cm_sh = T * P * e if sh_copy else 0
    cm = T * P * e if dy_copy else 0
    # name: (bound, algorithmic bytes or flops per launch, channel-major copy bytes written besides)
    w = {
        "gemm_qc_fwd": ("mfma", 2.0 * T * D * Q, 0),
        "gemm_ag_fwd": ("mfma", 2.0 * T * P * D, 0),
        "gemm_ag_dgrad": ("mfma", 2.0 * T * D * P, 0),
        "gemm_ag_wgrad": ("mfma", 2.0 * T * D * P, 0),
        "gemm_qc_dgrad": ("mfma", 2.0 * T * Q * D, 0),
        "gemm_qc_wgrad": ("mfma", 2.0 * T * Q * D, 0),
        # x read (valid tokens only when masked) + aggregate written
        "agg_fwd": ("hbm", float(read_tok * P * e + agg_out + mask_b + rope_tab), 0),
        # x read for valid tokens, grad_x written for every token, fp32 upstream grad read
        "agg_bwd": ("hbm", float(read_tok * P * e + T * P * e + B * G * P * 4 + mask_b), cm),
        # y_s read, sh written, aggregate read
        "gate_fwd": ("hbm", float(2 * T * P * e + B * G * P * e), cm_sh),
        # y_s and dsh read, dy_s written, fp32 dhagg written
        "gate_bwd": ("hbm", float(3 * T * P * e + B * G * P * 4), cm),
        # per-head gate: sh written (y_s and hagg are H / P wide per token / row)
        "gate_heads_fwd": ("hbm", float(T * P * e + T * H * e + B * G * P * e), cm_sh),
        # dsh read once, y_s read, dy_s written, fp32 dhagg written
        "gate_heads_bwd": ("hbm", float(T * P * e + 2 * T * H * e + B * G * P * 4), 0),
        # operand-layout transposes for the backward GEMMs: read + write once
        "transpose_x": ("hbm", float(2 * T * D * e), 0),
        "transpose_sh": ("hbm", float(2 * T * P * e), 0),
        "transpose_g": ("hbm", float(2 * T * D * e), 0),
        # all of dY, or only its gate part when the streaming kernels write the rest
        "transpose_dy": ("hbm", float(2 * T * (S if cm else Q) * e), 0),
        "transpose_w": ("hbm", float(2 * 2 * P * D * e), 0),   # W_qc or W_ag: counted as the larger
    }
    return w


# ---------------------------------------------------------------------------
# GPU leg
# ---------------------------------------------------------------------------

def gpu_run(cfg, steps, warmup, kernel_timing, graph=False):
    import torch
    from pom_amd import ops, _lib
    _lib.load()
    dev = torch.device("cuda:0")
    x, go, extra = make_inputs(cfg)
    m = make_module(cfg).to(dev, torch.bfloat16)
    xd = x.to(dev, torch.bfloat16).requires_grad_(True)
    god = go.to(dev, torch.bfloat16)
    extra_dev = {k: v.to(dev) for k, v in extra.items()}
    fwd = forward_fn(cfg, extra_dev)
    params = list(m.parameters())

    def step():
        for p in params:
            p.grad = None
        xd.grad = None
        # a training step changes every parameter: rebuild the per-parameter
        # derived copies (fp32 coefficients, transposed weights) every step
        ops.invalidate_derived()
        out = fwd(m, xd)
        out.backward(god)

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()

    if graph:
        # capture one step on a side stream (torch's recipe), then replay it
        for p in params:
            p.grad = None
        xd.grad = None
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            step()
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        for p in params:
            p.grad = None
        xd.grad = None
        with torch.cuda.graph(g):
            out = fwd(m, xd)
            out.backward(god)
        for _ in range(warmup):
            g.replay()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            g.replay()
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        return (t1 - t0) / steps * 1e3, None, {}, extra, (None, None)

    # instrumented pass: K steps with HIP events around every launch group on
    # its launch stream -> per-kernel durations and the dominant kernel.  The
    # layer's C++ launch sequence (pom_layer_fwd / _bwd) is one call per
    # direction with no Python between its launches, so the instrumented
    # passes run the Python sequence, which launches the same kernels with the
    # same GEMM solutions on the same operands (bit-identical results,
    # tests/test_gpu_layer_native.py); the timed region runs the default one.
    native = ops._NATIVE_LAYER
    per = {}
    dominant = None
    live = None
    if kernel_timing:
        ops._NATIVE_LAYER = False
        for _ in range(warmup):   # the Python sequence's own first use (torch's GEMM setup)
            step()
        torch.cuda.synchronize()
        ops.kernel_timer = []
        for _ in range(steps):
            step()
        torch.cuda.synchronize()
        for name, s, e in ops.kernel_timer:
            per.setdefault(name, []).append(s.elapsed_time(e) * 1e-3)   # seconds
        # copies on the second stream overlap the GEMMs: their event spans
        # include the wait for free compute units, so they are reported but
        # never taken as the dominant kernel
        dominant = max((k for k in per if k not in overlapped_groups()), key=lambda k: sum(per[k]))
        # a timed pass with events around the dominant kernel only (events
        # around every launch would add ~5 % to the step)
        ops.kernel_timer = []
        ops.kernel_timer_only = {dominant}
        torch.cuda.synchronize()
        for _ in range(steps):
            step()
        torch.cuda.synchronize()
        live = [s.elapsed_time(e) * 1e-3 for _, s, e in ops.kernel_timer]
        ops.kernel_timer = None
        ops.kernel_timer_only = None
        ops._NATIVE_LAYER = native

    # timed region: K fwd+bwd steps
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    ms_step = (t1 - t0) / steps * 1e3

    # forward-only throughput (no autograd graph)
    with torch.no_grad():
        for _ in range(max(2, warmup // 2)):
            fwd(m, xd)
        torch.cuda.synchronize()
        f0 = time.perf_counter()
        for _ in range(steps):
            fwd(m, xd)
        torch.cuda.synchronize()
        f1 = time.perf_counter()
    ms_fwd = (f1 - f0) / steps * 1e3
    return ms_step, ms_fwd, per, extra, (dominant, live)


FLUSH_BYTES = 1 << 30   # 4x the 256 MB Infinity Cache


def _flusher(dev):
    """A 1 GiB fill: evicts the Infinity Cache (MALL) and every XCD's L2."""
    import torch
    buf = torch.empty(FLUSH_BYTES // 4, dtype=torch.float32, device=dev)
    return lambda: buf.fill_(1.0)


def flushed_layer(cfg, steps, warmup):
    """The fwd+bwd step with 1 GiB written before every step: per-step GPU time
    from events around the step only (the fill is outside them), and the
    per-kernel spans of the same steps."""
    import torch
    from pom_amd import ops
    dev = torch.device("cuda:0")
    x, go, extra = make_inputs(cfg)
    m = make_module(cfg).to(dev, torch.bfloat16)
    xd = x.to(dev, torch.bfloat16).requires_grad_(True)
    god = go.to(dev, torch.bfloat16)
    fwd = forward_fn(cfg, {k: v.to(dev) for k, v in extra.items()})
    params = list(m.parameters())
    flush = _flusher(dev)

    def step():
        for p in params:
            p.grad = None
        xd.grad = None
        ops.invalidate_derived()
        fwd(m, xd).backward(god)

    # per-kernel spans need the Python launch sequence (same kernels, same
    # solutions as the C++ one)
    native = ops._NATIVE_LAYER
    ops._NATIVE_LAYER = False
    for _ in range(warmup):
        step()
    spans = []
    ops.kernel_timer = []
    for _ in range(steps):
        flush()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        step()
        e1.record()
        spans.append((e0, e1))
    torch.cuda.synchronize()
    ops._NATIVE_LAYER = native
    per = {}
    for name, a, b in ops.kernel_timer:
        per.setdefault(name, []).append(a.elapsed_time(b) * 1e-3)
    ops.kernel_timer = None
    ms = sum(a.elapsed_time(b) for a, b in spans) / steps
    return ms, per


def stream_kernels_warm_cold(cfg, reps):
    """The four streaming kernels of the full-width layer, standalone on the
    layer's operand shapes (Y's h- and s-parts as strided views, channel-major
    copies as in the training step): mean duration back to back (warm) and
    with 1 GiB written before every launch (cold: operands come from HBM)."""
    import torch
    from pom_amd import ops
    if cfg["variant"] != "mean" or cfg.get("heads", 1) > 1:
        return None
    dev = torch.device("cuda:0")
    B, N, D, K, E = cfg["B"], cfg["N"], cfg["D"], cfg["K"], cfg["E"]
    T, P = B * N, E * D
    W = ops._padded_width(P, P)
    g = torch.Generator().manual_seed(5)
    y = torch.randn(T, W, generator=g).to(dev, torch.bfloat16)
    y3 = y.view(B, N, W)
    h, ys = y3[..., :P], y3[..., P:2 * P]
    c = (torch.randn(P, K, generator=g) * 0.05).to(dev, torch.bfloat16)
    bias = torch.zeros(P, device=dev, dtype=torch.bfloat16)
    dsh = torch.randn(B, N, P, generator=g).to(dev, torch.bfloat16)
    dh = torch.randn(B, 1, P, generator=g).to(dev)
    dy = torch.empty(T, W, device=dev, dtype=torch.bfloat16)
    dy3 = dy.view(B, N, W)
    sh_copy, dy_copy = copies_written(cfg)   # the copies the layer's step writes, and only those
    dyt = torch.empty(W, T, device=dev, dtype=torch.bfloat16) if dy_copy else None
    sht = torch.empty(P, T, device=dev, dtype=torch.bfloat16) if sh_copy else None
    hagg, _ = ops.agg_forward(h, c, K, N)
    calls = {
        "agg_fwd": lambda: ops.agg_forward(h, c, K, N),
        "gate_fwd": lambda: ops.gate_forward(ys, bias, hagg, out_t=sht),
        "gate_bwd": lambda: ops.gate_backward(ys, bias, hagg, dsh, dy3[..., P:],
                                              grad_ys_t=None if dyt is None else dyt[P:], grad_ys_rows=dy[:, P:]),
        "agg_bwd": lambda: ops.agg_backward(h, c, K, N, dh, dy3[..., :P],
                                            grad_x_t=None if dyt is None else dyt[:P], grad_x_rows=dy[:, :P]),
    }
    flush = _flusher(dev)
    work = kernel_work(cfg, {})
    out = {}
    for name, call in calls.items():
        for _ in range(3):
            call()
        res = {}
        for mode in ("warm", "cold"):
            evs = []
            for _ in range(reps):
                if mode == "cold":
                    flush()
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record()
                call()
                e1.record()
                evs.append((e0, e1))
            torch.cuda.synchronize()
            res[mode] = sum(a.elapsed_time(b) for a, b in evs) / reps * 1e-3
        _, amount, copy = work[name]
        out[name] = {"bytes": amount,
                     "warm_us": round(res["warm"] * 1e6, 2), "cold_us": round(res["cold"] * 1e6, 2),
                     "warm_frac": round(amount / res["warm"] / HBM_PEAK, 4),
                     "cold_frac": round(amount / res["cold"] / HBM_PEAK, 4)}
        if copy:
            out[name]["copy_bytes"] = copy
            out[name]["cold_frac_with_copies"] = round((amount + copy) / res["cold"] / HBM_PEAK, 4)
    return out


def copy_calib(mib: float):
    """A plain device-to-device copy of known size, for counter calibration."""
    import torch
    dev = torch.device("cuda:0")
    n = int(mib * (1 << 20)) // 2
    a = torch.randn(n, device=dev).to(torch.bfloat16)
    b = torch.empty_like(a)
    torch.cuda.synchronize()
    for _ in range(10):
        b.copy_(a)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calib_bytes_read": n * 2, "copy_calib_bytes_written": n * 2, "launches": 10}))


# ---------------------------------------------------------------------------
# CPU leg: the oracle, fp32, on the host cores
# ---------------------------------------------------------------------------

def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    import platform
    return platform.processor() or "unknown"


# Threads of the CPU baseline: every core of the process's affinity mask, up to
# the 16 host cores one GPU of the measurement boxes is given (the harness
# sets OMP_NUM_THREADS to that share; more threads would oversubscribe it).
CPU_THREAD_CAP = int(os.environ.get("OMP_NUM_THREADS", "16") or 16)


def cpu_run(cfg, budget_s: float):
    """The oracle (pure-PyTorch restatement of the reference path) on a bounded
    sample of the workload's batch rows: fp32 fwd+bwd (the reported value),
    fp32 forward, and bf16 fwd+bwd and forward.  1 warm-up, median of 3."""
    import torch
    from oracle import pom_oracle as O
    affinity = len(os.sched_getaffinity(0))
    cores = max(1, min(affinity, CPU_THREAD_CAP))
    torch.set_num_threads(cores)
    x, go, extra = make_inputs(cfg)
    torch.manual_seed(0)
    rope2d = True if cfg["variant"] == "rope2d" else None
    prm32 = O.init_params(cfg["D"], cfg["K"], cfg["E"], n_sel_heads=cfg.get("heads", 1), rope_2d=rope2d,
                          max_h=cfg.get("H", 64), max_w=cfg.get("W", 64))
    v = cfg["variant"]

    def params(dt):
        prm = prm32.to(dt)
        for t in (prm.w_qc, prm.se_bias, prm.po_coeff, prm.w_ag):
            t.requires_grad_(True)
        return prm

    def run(prm, nb, dt, backward):
        xs = x[:nb].to(dt).clone().requires_grad_(backward)
        with torch.set_grad_enabled(backward):
            if v == "mean":
                out = O.pom_forward(prm, xs)
            elif v == "masked":
                out = O.pom_forward(prm, xs, mask=extra["mask"][:nb])
            elif v == "block":
                # the O(N) frame-causal route (the reference's state_forward loop
                # computes the same per-frame aggregate)
                out = O.pom_forward(prm, xs, mask=("block_causal", cfg["frame_len"]))
            else:
                out = O.rope_forward(prm, xs, positions_hw=extra["positions_hw"])
            if backward:
                out.backward(go[:nb].to(dt))

    def timed(prm, nb, dt, backward, reps=3):
        ts = []
        for _ in range(reps):
            t0 = time.perf_counter()
            run(prm, nb, dt, backward)
            ts.append(time.perf_counter() - t0)
        ts.sort()
        return ts[len(ts) // 2]

    p32, p16 = params(torch.float32), params(torch.bfloat16)
    t0 = time.perf_counter()
    run(p32, 1, torch.float32, True)                     # warm-up on one batch row
    t_one = time.perf_counter() - t0
    # share of the budget: fp32 fwd+bwd 1/2, the other three legs the rest
    nb = max(1, min(cfg["B"], int(budget_s / 2 / 3 / max(t_one, 1e-3))))
    tok = nb * cfg["N"]
    med = timed(p32, nb, torch.float32, True)
    res = {"value": tok / med, "unit": "tokens/s", "cores": cores, "kind": "port",
           "sample": f"oracle fp32 layer fwd+bwd on {nb} of {cfg['B']} batch rows ({tok} tokens), "
                     f"median of 3 after 1 warm-up, torch.set_num_threads({cores})",
           "fwd_value": tok / timed(p32, nb, torch.float32, False),
           "affinity_cores": affinity, "cpu_model": _cpu_model(),
           "threads_note": f"min(affinity cores, {CPU_THREAD_CAP}): the host-core share of one GPU on the box"}
    run(p16, 1, torch.bfloat16, True)                    # bf16 warm-up
    res["bf16_value"] = tok / timed(p16, nb, torch.bfloat16, True)
    res["bf16_fwd_value"] = tok / timed(p16, nb, torch.bfloat16, False)
    for k in ("value", "fwd_value", "bf16_value", "bf16_fwd_value"):
        res[k] = round(res[k], 1)
    return res


# rocprofv3 kernel names of the launch groups bench.py times
# launch groups that run on the layer's second stream, concurrently with a GEMM
OVERLAPPED = {"transpose_x", "transpose_g"}


def overlapped_groups():
    from pom_amd import ops
    return OVERLAPPED | ({"gemm_ag_wgrad", "gemm_qc_wgrad"} if ops._OVERLAP_GEMMS else set())

KERNEL_NAMES = {
    "agg_fwd": ["agg_fwd_chunk", "agg_fwd_finalize"],
    "agg_bwd": ["agg_bwd_chunk", "coeff_grad_finalize", "agg_frame_weights"],
    "gate_fwd": ["gate_fwd_kernel"],
    "gate_bwd": ["gate_bwd_kernel", "gate_bwd_finalize"],
    "transpose": ["transpose_blocks", "transpose_elems"],   # x^T, g^T and the weights, per step
    "gate_heads_fwd": ["heads_fwd_kernel", "heads_fwd_tile", "heads_fwd_rows"],
    "gate_heads_bwd": ["heads_bwd_token_kernel", "heads_bwd_hagg_kernel", "heads_bwd_finalize", "heads_bwd_tile",
                       "heads_bwd_dz", "heads_tile_finalize", "heads_bwd_rows"],
}


def _pmc_per_kernel(db: str, counter: str):
    """kernel name -> (dispatches, mean counter value per dispatch) from a rocprofv3 database."""
    import sqlite3
    c = sqlite3.connect(db)
    rows = c.execute("select kernel_name, dispatch_id, sum(value) from counters_collection "
                     "where counter_name = ? group by dispatch_id", (counter,)).fetchall()
    agg = {}
    for name, _, v in rows:
        n, t = agg.get(name, (0, 0.0))
        agg[name] = (n + 1, t + v)
    return {k: (n, t / n) for k, (n, t) in agg.items()}


COPY_CALIB_MIB = 144   # pmc_summary expects the calibration run made with --copy-calib 144


def _is_gate_bwd(name: str) -> bool:
    """The gate backward's main kernel (full-width or per-head)."""
    return any(k in name for k in ("gate_bwd_kernel", "heads_bwd_rows", "heads_bwd_tile", "heads_bwd_token_kernel"))


def _is_gemm(name: str) -> bool:
    """A projection GEMM dispatch: a hipBLASLt kernel or this library's pom_gemm kernel (whose
    split-K reduction, when present, is the next dispatch and counts with it)."""
    return "Cijk" in name or "gemm_bf16_kernel" in name


def _label_bwd_gemms(names):
    """Projection of each of a step's four backward GEMM dispatches (in dispatch
    order).  With both weight gradients on pom_gemm they are told apart by
    kernel: the library's products are dsh then dx, pom_gemm's dW_ag then dW_qc,
    whatever their interleaving (dW_ag may be issued first, on the second
    stream); otherwise by the one-stream order."""
    own = [i for i, n in enumerate(names) if "gemm_bf16_kernel" in n]
    if len(names) == 4 and len(own) == 2:
        lib = [i for i in range(4) if i not in own]
        out = [None] * 4
        out[lib[0]], out[lib[1]] = "gemm_ag_dgrad", "gemm_qc_dgrad"
        out[own[0]], out[own[1]] = "gemm_ag_wgrad", "gemm_qc_wgrad"
        return out
    return ["gemm_ag_dgrad", "gemm_ag_wgrad", "gemm_qc_dgrad", "gemm_qc_wgrad"][:len(names)]


def _gemm_dispatches(db: str):
    """Dispatch id and library kernel name of each projection GEMM of the last
    complete fwd+bwd step, from the dispatch order: qc_fwd precedes
    agg_fwd_chunk, ag_fwd follows the gate forward, ag_dgrad and ag_wgrad
    precede the gate backward, qc_dgrad and qc_wgrad follow
    coeff_grad_finalize.  (One library
    kernel can serve several GEMMs, so names alone do not identify them.)"""
    import sqlite3
    c = sqlite3.connect(db)
    seq = [(r[0], r[1]) for r in c.execute("select dispatch_id, kernel_name from counters_collection "
                                           "group by dispatch_id order by dispatch_id")]
    order = ["gemm_qc_fwd", "gemm_ag_fwd", "gemm_ag_dgrad", "gemm_ag_wgrad", "gemm_qc_dgrad", "gemm_qc_wgrad"]
    gb = max(i for i, (_, n) in enumerate(seq) if _is_gate_bwd(n))
    af = max(i for i, (_, n) in enumerate(seq[:gb]) if "agg_fwd_chunk" in n)
    pre = [i for i, d in enumerate(seq[:af]) if _is_gemm(d[1])]
    idx = [pre[-1]] + [af + i for i, d in enumerate(seq[af:]) if _is_gemm(d[1])][:5]
    groups = order[:2] + _label_bwd_gemms([seq[i][1] for i in idx[2:]])
    out = {}
    for g, i in zip(groups, idx):
        ds = [seq[i][0]]
        if i + 1 < len(seq) and "gemm_splitk_reduce" in seq[i + 1][1]:
            ds.append(seq[i + 1][0])
        out[g] = (ds, seq[i][1][:160])
    return out


def _pmc_dispatch(db: str, counter: str):
    """dispatch id -> counter value (summed over instances)."""
    import sqlite3
    c = sqlite3.connect(db)
    return {d: v for d, v in c.execute("select dispatch_id, sum(value) from counters_collection "
                                       "where counter_name = ? group by dispatch_id", (counter,))}


def pmc_summary(cfg_name, dbs):
    """Calibrated HBM bytes per launch group: FETCH_SIZE / WRITE_SIZE (KiB per
    dispatch) of each kernel, scaled by what the same counters read for a
    plain device copy of known size (rocclr's copyBuffer blit)."""
    fetch, write, cfetch, cwrite = (_pmc_per_kernel(d, c) for d, c in
                                    zip(dbs, ["FETCH_SIZE", "WRITE_SIZE", "FETCH_SIZE", "WRITE_SIZE"]))
    copy_bytes = COPY_CALIB_MIB * float(1 << 20)
    ckf = max(((k, v) for k, v in cfetch.items() if "copyBuffer" in k), key=lambda kv: kv[1][1])
    ckw = max(((k, v) for k, v in cwrite.items() if "copyBuffer" in k), key=lambda kv: kv[1][1])
    f_scale = copy_bytes / (ckf[1][1] * 1024.0)
    w_scale = copy_bytes / (ckw[1][1] * 1024.0)
    out = {"config": cfg_name, "copy_calib_bytes_each_way": copy_bytes, "fetch_scale": f_scale,
           "write_scale": w_scale, "kernels": {}}
    for name in fetch:
        fb = fetch[name][1] * 1024.0 * f_scale
        wb = write.get(name, (0, 0.0))[1] * 1024.0 * w_scale
        out["kernels"][name[:160]] = {"fetch_bytes": fb, "write_bytes": wb, "dispatches": fetch[name][0]}
    groups = {}
    for g, names in KERNEL_NAMES.items():
        # the layer's own kernels: the variant with the most dispatches (the
        # training step's, not the forward-only pass's) of each named kernel
        tot = 0.0
        for n in names:
            cand = [(v["dispatches"], v) for k, v in out["kernels"].items() if n in k]
            if cand:
                v = max(cand, key=lambda c: c[0])[1]
                tot += v["fetch_bytes"] + v["write_bytes"]
        groups[g] = tot
    # projection GEMMs: the dispatches of the last complete step, by order
    gd = _gemm_dispatches(dbs[0])
    fd, wd = _pmc_dispatch(dbs[0], "FETCH_SIZE"), _pmc_dispatch(dbs[1], "WRITE_SIZE")
    for g, (ds, _) in gd.items():
        groups[g] = sum(fd.get(d, 0.0) * 1024.0 * f_scale + wd.get(d, 0.0) * 1024.0 * w_scale for d in ds)
    out["gemm_kernels"] = {g: n for g, (_, n) in gd.items()}
    out["groups"] = groups
    path = os.path.join(ROOT, "profiles", f"traffic_{cfg_name}.json")
    with open(path, "w") as f:
        json.dump(out, f, indent=1)
    print(json.dumps({"wrote": path, "groups": groups, "fetch_scale": f_scale, "write_scale": w_scale}))


def pmc_table(cfg_name, db, counters):
    """Mean value per dispatch of each counter, per launch group: the layer's
    streaming kernels by name, the projection GEMMs by dispatch order (the
    last complete fwd+bwd step).  MfmaUtil (rocprofv3's derived metric,
    SQ_VALU_MFMA_BUSY_CYCLES over GRBM_GUI_ACTIVE x SIMDs, in %) and
    MfmaFlopsBF16 (SQ_INSTS_VALU_MFMA_MOPS_BF16 x 512) give the GEMMs' matrix
    core utilisation and the flops they executed."""
    per = {c: _pmc_per_kernel(db, c) for c in counters}
    out = {"config": cfg_name, "database": db, "counters": counters, "groups": {}}
    for g, names in KERNEL_NAMES.items():
        row = {}
        for c in counters:
            tot, found = 0.0, False
            for n in names:
                cand = [(v[0], v[1]) for k, v in per[c].items() if n in k]
                if cand:
                    tot += max(cand)[1]
                    found = True
            if found:
                row[c] = tot
        if row:
            out["groups"][g] = row
    gd = _gemm_dispatches(db)
    for g, (ds, kname) in gd.items():
        out["groups"][g] = {c: _pmc_dispatch(db, c).get(ds[0]) for c in counters}
        out["groups"][g]["kernel"] = kname
    path = os.path.join(ROOT, "profiles", f"pmc_{cfg_name}_{counters[0]}.json")
    with open(path, "w") as f:
        json.dump(out, f, indent=1)
    print(json.dumps({"wrote": path, "groups": out["groups"]}))


def trace_summary(trace_dir):
    """Table of a kernel-trace run: calls, average us, share of GPU time, kernel
    (GEMMs labelled with their projection from the dispatch order of the
    fwd+bwd steps and, in the backward, their kernel: _label_bwd_gemms)."""
    import csv
    stats = list(csv.DictReader(open(os.path.join(trace_dir, "run_kernel_stats.csv"))))
    trace = sorted(csv.DictReader(open(os.path.join(trace_dir, "run_kernel_trace.csv"))),
                   key=lambda r: int(r["Dispatch_Id"]))
    seq = [r["Kernel_Name"] for r in trace]
    dur = [(int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3 for r in trace]
    order = ["gemm_qc_fwd", "gemm_ag_fwd", "gemm_ag_dgrad", "gemm_ag_wgrad", "gemm_qc_dgrad", "gemm_qc_wgrad"]
    # every fwd+bwd step: the GEMM before its agg_fwd_chunk, then the five after it
    per = {g: [] for g in order}
    label = {}
    afs = [i for i, n in enumerate(seq) if "agg_fwd_chunk" in n]
    for k, af in enumerate(afs):
        end = afs[k + 1] if k + 1 < len(afs) else len(seq)
        if not any(_is_gate_bwd(n) for n in seq[af:end]):
            continue   # a forward-only pass
        pre = [i for i in range(af) if _is_gemm(seq[i])]
        idx = [pre[-1]] + [i for i in range(af, end) if _is_gemm(seq[i])][:5]
        for g, i in zip(order[:2] + _label_bwd_gemms([seq[j] for j in idx[2:]]), idx):
            red = i + 1 < len(seq) and "gemm_splitk_reduce" in seq[i + 1]
            per[g].append(dur[i] + (dur[i + 1] if red else 0.0))
            label.setdefault(seq[i], set()).add(g)
            if red:
                label.setdefault(seq[i + 1], set()).add(g)
    print("# columns: calls, avg_us, pct_of_gpu_time, kernel (library GEMM names truncated)")
    for r in sorted(stats, key=lambda r: -float(r["TotalDurationNs"])):
        name = r["Name"]
        tag = f"   [{', '.join(sorted(label[name]))}]" if name in label else ""
        print(f"{int(r['Calls']):6d} {float(r['AverageNs']) / 1e3:10.2f} {float(r['Percentage']):6.2f}  "
              f"{name[:100]}{tag}")
    print("# projection GEMMs of the fwd+bwd steps, labelled by dispatch order (a split-K reduction counted with "
          "its GEMM): group, calls, avg_us")
    for g in order:
        if per[g]:
            print(f"#   {g:14s} {len(per[g]):4d} {sum(per[g]) / len(per[g]):10.2f}")


def traffic_of(cfg_name, group):
    """HBM bytes per launch of a launch group from profiles/traffic_<config>.json, or None."""
    path = os.path.join(ROOT, "profiles", f"traffic_{cfg_name}.json")
    try:
        with open(path) as f:
            return json.load(f).get("groups", {}).get(group)
    except (OSError, ValueError):
        return None


def _kernel_table(per, work, steps):
    kernels = {}
    for name, durs in per.items():
        bound, amount, copy = work[name]
        avg = sum(durs) / len(durs)
        peak = HBM_PEAK if bound == "hbm" else MFMA_BF16_PEAK
        achieved = amount / avg
        k = {"bound": bound, "avg_us": round(avg * 1e6, 2), "us_per_step": round(sum(durs) / steps * 1e6, 2),
             "achieved": round(achieved / (1e9 if bound == "hbm" else 1e12), 2),
             "unit": "GB/s" if bound == "hbm" else "TFLOP/s", "frac": round(achieved / peak, 4),
             "launches_per_step": len(durs) / steps}
        if copy:
            k["copy_bytes"] = copy
            k["frac_with_copies"] = round((amount + copy) / avg / peak, 4)
        if name in overlapped_groups():
            k["overlapped"] = True   # span includes waiting for compute units
        kernels[name] = k
    return kernels


def _groups(kernels, work):
    agg = [n for n in ("agg_fwd", "agg_bwd", "gate_fwd", "gate_bwd", "gate_heads_fwd", "gate_heads_bwd")
           if n in kernels]
    gem = [n for n in kernels if n.startswith("gemm")]
    t_hbm = sum(kernels[n]["us_per_step"] for n in agg)
    t_mf = sum(kernels[n]["us_per_step"] for n in gem)
    b_hbm = sum(work[n][1] for n in agg)
    c_hbm = sum(work[n][2] for n in agg)
    f_mf = sum(work[n][1] for n in gem)
    hbm = {"us_per_step": round(t_hbm, 2),
           "frac_hbm": round(b_hbm / (t_hbm * 1e-6) / HBM_PEAK, 4) if t_hbm else None}
    if c_hbm and t_hbm:
        hbm["frac_hbm_with_copies"] = round((b_hbm + c_hbm) / (t_hbm * 1e-6) / HBM_PEAK, 4)
    return {
        "hip_streaming_kernels": hbm,
        "projection_gemms": {"us_per_step": round(t_mf, 2),
                             "frac_mfma": round(f_mf / (t_mf * 1e-6) / MFMA_BF16_PEAK, 4) if t_mf else None},
        "ideal_step_us": round((b_hbm / HBM_PEAK + f_mf / MFMA_BF16_PEAK) * 1e6, 2),
    }


def measure(name, a, headline):
    """One configuration: GPU step timings, per-kernel table, dominant-kernel
    roofline, group fractions and the CPU baseline."""
    import torch
    cfg = CONFIGS[name]
    steps = a.steps if headline else min(a.steps, 20)
    ms_step, ms_fwd, per, extra, (dominant, live) = gpu_run(cfg, steps, a.warmup,
                                                            not a.no_kernel_timing and not a.graph, a.graph)
    T = cfg["B"] * cfg["N"]
    work = kernel_work(cfg, extra)
    kernels = _kernel_table(per, work, steps)
    roofline = None
    if kernels and dominant and live:
        k = kernels[dominant]
        bound, amount, copy = work[dominant]
        avg = sum(live) / len(live)                      # events of the timed dominant-kernel pass
        achieved = amount / avg
        peak = HBM_PEAK if bound == "hbm" else MFMA_BF16_PEAK
        roofline = {"kernel": dominant, "bound": bound,
                    "achieved": round(achieved / (1e9 if bound == "hbm" else 1e12), 2),
                    "peak": 8000.0 if bound == "hbm" else 2500.0, "unit": k["unit"],
                    "frac": round(achieved / peak, 4), "avg_us": round(avg * 1e6, 2),
                    "launches_timed": len(live), "traffic": traffic_of(name, dominant)}
        if copy:
            roofline["copy_bytes"] = copy
            roofline["frac_with_copies"] = round((amount + copy) / avg / peak, 4)
    res = {"workload": cfg["workload"],
           "config": {"workload": cfg["workload"], "B": cfg["B"], "N": cfg["N"], "D": cfg["D"],
                      "degree": cfg["K"], "expand": cfg["E"], "tokens_per_step": T},
           "steps": steps, "ms_per_step": round(ms_step, 4), "value": round(T / (ms_step * 1e-3), 1),
           "fwd_tokens_per_s": round(T / (ms_fwd * 1e-3), 1) if ms_fwd else None,
           "ms_fwd": round(ms_fwd, 4) if ms_fwd else None, "roofline": roofline, "kernels": kernels}
    if cfg.get("heads", 1) > 1:
        res["config"]["n_sel_heads"] = cfg["heads"]
    if kernels:
        res["roofline_groups"] = _groups(kernels, work)
    if headline and not a.no_flush and not a.graph:
        ms_fl, per_fl = flushed_layer(cfg, min(steps, 20), a.warmup)
        k_fl = _kernel_table(per_fl, work, min(steps, 20))
        res["mall_flushed"] = {
            "note": "1 GiB written before every step; events around the step only",
            "ms_per_step": round(ms_fl, 4), "value": round(T / (ms_fl * 1e-3), 1),
            "kernels": {n: {kk: v[kk] for kk in ("avg_us", "frac") if kk in v} for n, v in k_fl.items()},
            "streaming_kernels_standalone": stream_kernels_warm_cold(cfg, 20)}
    torch.cuda.empty_cache()
    if not a.no_cpu:
        res["cpu_baseline"] = cpu_run(cfg, a.cpu_seconds if headline else a.sub_cpu_seconds)
    return res


def main():
    a = parse()
    if a.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {a.gpus}); "
              "multi-GPU sharding is a design note, not a measured path", file=sys.stderr)
        sys.exit(2)
    if a.copy_calib > 0:
        copy_calib(a.copy_calib)
        return
    if a.pmc_summary:
        pmc_summary(a.config, a.pmc_summary)
        return
    if a.trace_summary:
        trace_summary(a.trace_summary)
        return
    if a.pmc_table:
        pmc_table(a.config, a.pmc_table[0], a.pmc_table[1:])
        return
    head = measure(a.config, a, True)
    res = {
        "metric": METRIC, "value": head["value"], "unit": "tokens/s", "n_gpus": 1,
        "steps": a.steps, "warmup": a.warmup, "ms_per_step": head["ms_per_step"], "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic: x~N(0,1) seed 1, upstream grad~N(0,1) seed 2, weights nn.Linear init seed 0",
        "config": head["config"], "fwd_tokens_per_s": head["fwd_tokens_per_s"], "ms_fwd": head["ms_fwd"],
        "hip_graph": a.graph, "roofline": head["roofline"], "kernels": head["kernels"],
        "launch_sequence": "c++" if _native_sequence() else "python",
    }
    for k in ("roofline_groups", "mall_flushed", "cpu_baseline"):
        if k in head:
            res[k] = head[k]
    subs = [c for c in a.sub_configs.split(",") if c and c != a.config]
    if subs:
        res["configs"] = {}
        for c in subs:
            r = measure(c, a, False)
            res["configs"][c] = {k: v for k, v in r.items() if k != "config"}
            print(f"bench.py: {c} done: {r['ms_per_step']} ms/step", file=sys.stderr, flush=True)
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
