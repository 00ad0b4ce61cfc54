"""PoM layer benchmark on one MI355X: forward + backward tokens/s, per-kernel
roofline fractions and a CPU baseline, printed as ONE JSON line.

  python bench.py [--gpus 1] [--steps K] [--warmup W] [--config c2|c3|c4|c5]
                  [--no-cpu] [--fwd] [--copy-calib MiB]

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

The CPU baseline runs the oracle (a pure-PyTorch restatement of the reference
path) in fp32 on the host cores on a bounded sample of the same workload.
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
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--cpu-seconds", type=float, default=15.0, help="CPU baseline time budget")
    ap.add_argument("--no-kernel-timing", action="store_true",
                    help="time the steps without per-launch events")
    ap.add_argument("--graph", action="store_true",
                    help="capture one forward+backward step in a HIP graph and time its replays "
                         "(host launch overhead removed); per-kernel events are not available then")
    ap.add_argument("--pmc-summary", nargs=4, metavar=("FETCH_DB", "WRITE_DB", "COPY_FETCH_DB", "COPY_WRITE_DB"),
                    help="turn four rocprofv3 --pmc databases (FETCH_SIZE and WRITE_SIZE of a bench run and "
                         "of a --copy-calib run) into per-kernel HBM traffic; writes profiles/traffic_<config>.json")
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
    # channel-major copies written in the same pass (16-bit training path)
    from pom_amd import ops
    cm = T * P * e if (ops._NT_GEMMS and ops._NT_COPIES == "fused") else 0
    w = {
        "gemm_qc_fwd": ("mfma", 2.0 * T * D * Q),
        "gemm_ag_fwd": ("mfma", 2.0 * T * P * D),
        "gemm_ag_dgrad": ("mfma", 2.0 * T * D * P),
        "gemm_ag_wgrad": ("mfma", 2.0 * T * D * P),
        "gemm_qc_dgrad": ("mfma", 2.0 * T * Q * D),
        "gemm_qc_wgrad": ("mfma", 2.0 * T * Q * D),
        # x read (valid tokens only when masked) + aggregate written
        "agg_fwd": ("hbm", float(read_tok * P * e + agg_out + mask_b + rope_tab)),
        # x read for valid tokens, grad_x (and its channel-major copy) written for every token,
        # fp32 upstream grad read
        "agg_bwd": ("hbm", float(read_tok * P * e + T * P * e + cm + B * G * P * 4 + mask_b)),
        # y_s read, sh (and sh^T) written, aggregate read
        "gate_fwd": ("hbm", float(2 * T * P * e + cm + B * G * P * e)),
        # y_s and dsh read, dy_s (and its channel-major copy) written
        "gate_bwd": ("hbm", float(3 * T * P * e + cm + B * G * P * 4)),
        # per-head gate: sh (and sh^T) written (y_s and hagg are H / P wide per token / row)
        "gate_heads_fwd": ("hbm", float(T * P * e + cm + T * H * e + B * G * P * e)),
        # dsh read once, y_s read, dy_s written, fp32 dhagg written
        "gate_heads_bwd": ("hbm", float(T * P * e + 2 * T * H * e + B * G * P * 4)),
        # operand-layout transposes for the backward GEMMs: read + write once
        "transpose_x": ("hbm", float(2 * T * D * e)),
        "transpose_sh": ("hbm", float(2 * T * P * e)),
        "transpose_g": ("hbm", float(2 * T * D * e)),
        # all of dY, or only its gate part when the streaming kernels write the rest
        "transpose_dy": ("hbm", float(2 * T * (S if cm else Q) * e)),
        "transpose_w": ("hbm", float(2 * 2 * P * D * e)),   # W_qc or W_ag: counted as the larger
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
    # its launch stream -> per-kernel durations and the dominant kernel
    per = {}
    dominant = None
    if kernel_timing:
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
        # the timed region records events around the dominant kernel only
        # (events around every launch would add ~5 % to the step)
        ops.kernel_timer = []
        ops.kernel_timer_only = {dominant}

    # timed region: K fwd+bwd steps
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    ms_step = (t1 - t0) / steps * 1e3
    live = None
    if kernel_timing:
        live = [s.elapsed_time(e) * 1e-3 for _, s, e in ops.kernel_timer]
        ops.kernel_timer = None
        ops.kernel_timer_only = None

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

def cpu_run(cfg, budget_s: float):
    import torch
    from oracle import pom_oracle as O
    cores = min(len(os.sched_getaffinity(0)), 16)
    torch.set_num_threads(cores)
    x, go, extra = make_inputs(cfg)
    torch.manual_seed(0)
    rope2d = True if cfg["variant"] == "rope2d" else None
    prm = O.init_params(cfg["D"], cfg["K"], cfg["E"], n_sel_heads=cfg.get("heads", 1), rope_2d=rope2d,
                        max_h=cfg.get("H", 64), max_w=cfg.get("W", 64))
    for t in (prm.w_qc, prm.se_bias, prm.po_coeff, prm.w_ag):
        t.requires_grad_(True)
    # bounded sample: the first batch rows of the workload, as many as the budget allows
    v = cfg["variant"]

    def run(nb):
        xs = x[:nb].clone().requires_grad_(True)
        if v == "mean":
            out = O.pom_forward(prm, xs)
        elif v == "masked":
            out = O.pom_forward(prm, xs, mask=extra["mask"][:nb])
        elif v == "block":
            out = O.pom_forward(prm, xs, mask=("block_causal", cfg["frame_len"]))
        else:
            out = O.rope_forward(prm, xs, positions_hw=extra["positions_hw"])
        out.backward(go[:nb])

    nb = 1
    t0 = time.perf_counter()
    run(nb)                                  # warm-up on one batch row
    t_one = time.perf_counter() - t0
    nb = max(1, min(cfg["B"], int(budget_s / 3 / max(t_one, 1e-3))))
    times = []
    for _ in range(3):
        s = time.perf_counter()
        run(nb)
        times.append(time.perf_counter() - s)
    times.sort()
    med = times[1]
    tok = nb * cfg["N"]
    return {"value": tok / med, "unit": "tokens/s", "cores": cores, "kind": "port",
            "sample": f"oracle fp32 layer fwd+bwd on {nb} of {cfg['B']} batch rows ({tok} tokens), "
                      f"median of 3 after 1 warm-up, torch.set_num_threads({cores})"}


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
    "gate_heads_fwd": ["heads_fwd_kernel", "heads_fwd_tile"],
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
    pre = [d for d in seq[:af] if "Cijk" in d[1]]
    gemms = [pre[-1]] + [d for d in seq[af:] if "Cijk" in d[1]][:5]
    return {g: (d, n[:160]) for g, (d, n) in zip(order, gemms)}


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
    for g, (d, _) in gd.items():
        groups[g] = fd.get(d, 0.0) * 1024.0 * f_scale + wd.get(d, 0.0) * 1024.0 * w_scale
    out["gemm_kernels"] = {g: n for g, (_, n) in gd.items()}
    out["groups"] = groups
    path = os.path.join(ROOT, "profiles", f"traffic_{cfg_name}.json")
    with open(path, "w") as f:
        json.dump(out, f, indent=1)
    print(json.dumps({"wrote": path, "groups": groups, "fetch_scale": f_scale, "write_scale": w_scale}))


def trace_summary(trace_dir):
    """Table of a kernel-trace run: calls, average us, share of GPU time, kernel
    (library GEMMs labelled with their projection from the dispatch order of
    the last fwd+bwd step)."""
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
        pre = [i for i in range(af) if "Cijk" in seq[i]]
        idx = [pre[-1]] + [i for i in range(af, end) if "Cijk" in seq[i]][:5]
        for g, i in zip(order, idx):
            per[g].append(dur[i])
            label.setdefault(seq[i], set()).add(g)
    print("# columns: calls, avg_us, pct_of_gpu_time, kernel (library GEMM names truncated)")
    for r in sorted(stats, key=lambda r: -float(r["TotalDurationNs"])):
        name = r["Name"]
        tag = f"   [{', '.join(sorted(label[name]))}]" if name in label else ""
        print(f"{int(r['Calls']):6d} {float(r['AverageNs']) / 1e3:10.2f} {float(r['Percentage']):6.2f}  "
              f"{name[:100]}{tag}")
    print("# projection GEMMs of the fwd+bwd steps, labelled by dispatch order: group, calls, avg_us")
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
    cfg = CONFIGS[a.config]
    ms_step, ms_fwd, per, extra, (dominant, live) = gpu_run(cfg, a.steps, a.warmup,
                                                            not a.no_kernel_timing and not a.graph, a.graph)
    T = cfg["B"] * cfg["N"]
    work = kernel_work(cfg, extra)
    kernels = {}
    for name, durs in per.items():
        bound, amount = work[name]
        avg = sum(durs) / len(durs)
        per_step = sum(durs) / a.steps
        peak = HBM_PEAK if bound == "hbm" else MFMA_BF16_PEAK
        achieved = amount / avg
        kernels[name] = {"bound": bound, "avg_us": round(avg * 1e6, 2), "us_per_step": round(per_step * 1e6, 2),
                         "achieved": round(achieved / (1e9 if bound == "hbm" else 1e12), 2),
                         "unit": "GB/s" if bound == "hbm" else "TFLOP/s", "frac": round(achieved / peak, 4),
                         "launches_per_step": len(durs) / a.steps}
        if name in overlapped_groups():
            kernels[name]["overlapped"] = True   # span includes waiting for compute units
    roofline = None
    if kernels and dominant and live:
        k = kernels[dominant]
        bound, amount = work[dominant]
        avg = sum(live) / len(live)                      # from the timed region's events
        achieved = amount / avg
        peak = HBM_PEAK if bound == "hbm" else MFMA_BF16_PEAK
        roofline = {"kernel": dominant, "bound": bound,
                    "achieved": round(achieved / (1e9 if bound == "hbm" else 1e12), 2),
                    "peak": 8000.0 if bound == "hbm" else 2500.0, "unit": k["unit"],
                    "frac": round(achieved / peak, 4), "avg_us": round(avg * 1e6, 2),
                    "launches_timed": len(live), "traffic": traffic_of(a.config, dominant)}
    res = {
        "metric": METRIC, "value": round(T / (ms_step * 1e-3), 1), "unit": "tokens/s", "n_gpus": 1,
        "steps": a.steps, "warmup": a.warmup, "ms_per_step": round(ms_step, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic: x~N(0,1) seed 1, upstream grad~N(0,1) seed 2, weights nn.Linear init seed 0",
        "config": {"workload": cfg["workload"], "B": cfg["B"], "N": cfg["N"], "D": cfg["D"], "degree": cfg["K"],
                   "expand": cfg["E"], "tokens_per_step": T},
        "fwd_tokens_per_s": round(T / (ms_fwd * 1e-3), 1) if ms_fwd else None,
        "ms_fwd": round(ms_fwd, 4) if ms_fwd else None, "hip_graph": a.graph,
        "roofline": roofline, "kernels": kernels,
    }
    if kernels:
        agg = [n for n in ("agg_fwd", "agg_bwd", "gate_fwd", "gate_bwd", "gate_heads_fwd", "gate_heads_bwd")
               if n in kernels]
        gem = [n for n in kernels if n.startswith("gemm")]
        t_hbm = sum(kernels[n]["us_per_step"] for n in agg)
        t_mf = sum(kernels[n]["us_per_step"] for n in gem)
        b_hbm = sum(work[n][1] for n in agg)
        f_mf = sum(work[n][1] for n in gem)
        res["roofline_groups"] = {
            "hip_streaming_kernels": {"us_per_step": round(t_hbm, 2),
                                      "frac_hbm": round(b_hbm / (t_hbm * 1e-6) / HBM_PEAK, 4) if t_hbm else None},
            "projection_gemms": {"us_per_step": round(t_mf, 2),
                                 "frac_mfma": round(f_mf / (t_mf * 1e-6) / MFMA_BF16_PEAK, 4) if t_mf else None},
            "ideal_step_us": round((b_hbm / HBM_PEAK + f_mf / MFMA_BF16_PEAK) * 1e6, 2),
        }
    if not a.no_cpu:
        res["cpu_baseline"] = cpu_run(cfg, a.cpu_seconds)
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
