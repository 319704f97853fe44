"""Benchmark of the triangle inference hot path on one MI355X.

One step = the BASELINE.json headline workload at N_res = 512, bf16, B = 1:
  * triangle_attention forward, N_seq = N_res = 512, H = 4, D = 32, pair bias, no mask;
  * triangle_multiplicative_update forward, c_z = c_hidden = 128, 'outgoing';
  * the same with 'incoming' (mask: the last 64 residues padded on both axes).
Every kernel is launched through the C ABI (libgnn_hip.so) with inputs, outputs and
workspaces already resident in HBM. ``ms_per_step`` / ``value`` come from ``--steps`` steps
launched back to back with HIP events around the whole loop (on the launch stream).
Per-kernel (per-entry-point) durations are the median, and the mean, of event pairs around
single launches repeated for at least a 100 ms window after 10 warm-up launches (the window
of the reference's do_bench, benchmarks/_bench_common.py:128-132). Every timed
configuration first passes a parity gate against the fp64 numpy oracle (rel-Frobenius
<= 1e-2; max-abs reported beside it).

Prints ONE JSON line. ``value`` = algorithmic TFLOP/s of the whole step (attention
4 S H N^2 D, softmax excluded; trimul 2 N^3 Ch + N^2 (10 C Ch + 2 C^2)); ``roofline`` is
that of the dominant kernel, its bound chosen by arithmetic intensity against the bf16 ridge
(2516.6 TFLOP/s / 8 TB/s = 315 flop/B). Extra keys:
  * ``configs``: the other BASELINE.json configurations, each timed the same way and
    parity-gated (C2 attention N=256 cueq layout with 26 masked keys, C3 trimul N=512 both
    directions as single gnn_trimul_fwd calls, C4 attention N=768 with ragged lengths, the
    C5 pair-stack block at N=1024 bf16 and at N=384 fp32 under 'ieee' and 'tf32' (bf16x3));
  * ``public_api_ms``: the headline ops through the public Python API (argument checks,
    ctypes marshalling, workspace allocation) beside the C-ABI figure;
  * ``cpu_baseline``: the package's pure-torch path (triangle/_reference/, which follows the
    reference's trimul_torch and triangle_attention_torch op for op) on the host cores, in
    bf16, attention over all 512 N_seq rows in chunks, 1 warm-up and the median of 3; with
    C1's CPU time (trimul outgoing, fp32, N=64);
  * ``cold_ms``: every kernel again after a 512 MiB scratch write (inputs then come from HBM,
    not from the Infinity Cache that holds them in the warm loop);
  * ``graph_ms_per_step``: the step captured once as a HIP graph and replayed;
  * ``hbm_reference``: a 1 GiB device copy (read + write) and fill timed the same way, the
    streaming rate these boxes reach; HBM-bound kernels also report ``frac_of_copy``;
  * ``attention_backward`` / ``trimul_backward``: the gradient paths, outside the step.
"""

import argparse
import ctypes
import gc
import json
import os
import pathlib
import statistics
import sys
import time

ROOT = pathlib.Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "geometric-nn-ops_amd"))
sys.path.insert(0, str(ROOT))

METRIC = "trimul + triangle-attn fwd ms & TFLOP/s at N=512 bf16; % of MFMA peak"
PEAK_BF16_TFLOPS = 2516.6
PEAK_FP32_TFLOPS = 157.3
PEAK_HBM_GBS = 8000.0
RIDGE = PEAK_BF16_TFLOPS * 1e12 / (PEAK_HBM_GBS * 1e9)
TRAFFIC_FILE = ROOT / "profiles" / "traffic_n512_bf16.json"


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--n", type=int, default=512)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-configs", action="store_true", help="skip the other BASELINE configurations")
    ap.add_argument("--cold-steps", type=int, default=3,
                    help="launches of each kernel timed cold, after a 512 MiB scratch write that evicts L2 and "
                         "the 256 MB Infinity Cache (0 skips)")
    ap.add_argument("--only", choices=["attn", "trimul", "configs"], default=None,
                    help="profile helper: run only one op, or only the other BASELINE configurations "
                         "(the JSON line is then partial)")
    ap.add_argument("--no-backward", action="store_true", help="skip the backward timings")
    ap.add_argument("--trace-steps", action="store_true",
                    help="a spin_kernel marker launch before and after the timed eager steps and the timed graph "
                         "replays, which --summarize-trace uses to pick them out of a kernel trace")
    ap.add_argument("--summarize-trace", default=None, metavar="KERNEL_TRACE_CSV",
                    help="print per-kernel durations and launch gaps of a rocprofv3 kernel trace and exit")
    ap.add_argument("--sweep", action=argparse.BooleanOptionalAction, default=True,
                    help="the trimul size sweep and peak-memory table of the public ops")
    ap.add_argument("--copy-calib", action="store_true",
                    help="profile helper: run a plain 256 MiB device copy (known HBM bytes) and exit, "
                         "to scale FETCH_SIZE / WRITE_SIZE counter readings")
    return ap.parse_args()


# --------------------------------------------------------------------------------- timing
def region_marker():
    """One ``spin_kernel`` launch (torch.cuda._sleep), which a kernel trace shows by name:
    ``--trace-steps`` puts one before and one after the timed steps, and
    ``--summarize-trace`` reports the launches between each such pair."""
    import torch

    torch.cuda._sleep(1000)


def summarize_trace(path, steps=None):
    """Markdown tables of a rocprofv3 kernel-trace CSV: for each region between two
    ``spin_kernel`` markers (the whole trace when there are none), per kernel the number of
    launches and their mean / median duration, then the idle gaps between consecutive
    launches and, given ``steps``, the span and kernel time per step."""
    import csv

    rows = []
    with open(path, newline="") as fh:
        for r in csv.DictReader(fh):
            name = r["Kernel_Name"]
            rows.append((int(r["Start_Timestamp"]), int(r["End_Timestamp"]),
                         "spin_kernel" if "::spin_kernel(" in name else
                         name.replace("(anonymous namespace)", "anon").split("(")[0]))
    rows.sort()
    marks = [i for i, r in enumerate(rows) if r[2] == "spin_kernel"]
    regions = [rows[marks[i] + 1:marks[i + 1]] for i in range(0, len(marks) - 1, 2)] if len(marks) >= 2 else [rows]
    out = []
    for ri, reg in enumerate(regions):
        per = {}
        for t0, t1, name in reg:
            per.setdefault(name, []).append((t1 - t0) / 1e3)
        busy = sum(sum(v) for v in per.values())
        out += [f"### region {ri + 1}", "", "| kernel | launches | mean us | median us | share of busy time |",
                "|---|---|---|---|---|"]
        for name, ds in sorted(per.items(), key=lambda kv: -sum(kv[1])):
            out.append(f"| `{name}` | {len(ds)} | {sum(ds) / len(ds):.2f} | {statistics.median(ds):.2f} | "
                       f"{sum(ds) / busy:.3f} |")
        gaps = [(reg[i + 1][0] - reg[i][1]) / 1e3 for i in range(len(reg) - 1)]
        span = (reg[-1][1] - reg[0][0]) / 1e3
        out += ["", f"launches: {len(reg)}; busy {busy:.1f} us of a {span:.1f} us span; gap between launches: "
                    f"mean {sum(gaps) / max(len(gaps), 1):.2f} us, median {statistics.median(gaps) if gaps else 0:.2f} us, "
                    f"max {max(gaps) if gaps else 0:.2f} us"]
        if steps:
            out.append(f"per step ({steps} steps): span {span / steps:.1f} us, kernel time {busy / steps:.1f} us")
        out.append("")
    return "\n".join(out)


def window_ms(fn, stream, window=100.0, warmup=10, min_reps=10, max_reps=5000):
    """(median, mean, reps) of event-pair durations of ``fn`` on ``stream``, repeated until
    the durations add up to ``window`` ms (at least ``min_reps``), after ``warmup`` calls."""
    import torch

    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    ts, total = [], 0.0
    while (total < window or len(ts) < min_reps) and len(ts) < max_reps:
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        fn()
        e1.record(stream)
        e1.synchronize()
        ts.append(e0.elapsed_time(e1))
        total += ts[-1]
    return statistics.median(ts), sum(ts) / len(ts), len(ts)


def rates(flops, nbytes, ms, peak_tflops=PEAK_BF16_TFLOPS):
    tf = flops / (ms * 1e-3) / 1e12
    gbs = nbytes / (ms * 1e-3) / 1e9
    ai = flops / nbytes
    ridge = peak_tflops * 1e12 / (PEAK_HBM_GBS * 1e9)
    return {"ms": round(ms, 5), "tflops": round(tf, 2), "gbs": round(gbs, 1),
            "mfma_frac": round(tf / peak_tflops, 4), "hbm_frac": round(gbs / PEAK_HBM_GBS, 4),
            "ai_flop_per_byte": round(ai, 1), "bound": "mfma" if ai >= ridge else "hbm",
            "algorithmic_flops": flops, "compulsory_bytes": nbytes}


def attn_flops(B, S, N, H, D):
    return 4.0 * B * S * H * N * N * D


def attn_bytes(B, S, N, H, D, e, bias=True, mask=False):
    return e * 4.0 * B * S * N * H * D + (e * B * H * N * N if bias else 0) + (B * S * N if mask else 0)


def trimul_flops(B, N, C, Ch):
    return 2.0 * B * N**3 * Ch + B * N * N * (10.0 * C * Ch + 2.0 * C * C)


def trimul_bytes(B, N, C, Ch, e, mask=True):
    weights = e * (4 * Ch * C + C * Ch + C * C + 2 * C + 2 * Ch)
    return 2.0 * e * B * N * N * C + (e * B * N * N if mask else 0) + weights


def parity(got, want):
    import numpy as np

    from oracle import triangle_oracle as O

    g = got.detach().double().cpu().numpy()
    return {"rel_fro": float(f"{O.rel_fro(g, want):.3e}"), "max_abs": float(f"{np.abs(g - want).max():.3e}")}


def check_parity(where, par, bound=1e-2):
    if not par["rel_fro"] <= bound:
        print(f"bench.py: parity gate failed for {where}: {par}", file=sys.stderr)
        sys.exit(1)
    return par


# --------------------------------------------------------------------------------- inputs
class Gen:
    """Seeded CPU generators, one per tensor in a fixed order (seed 0, 1, 2, ...), so the
    CPU oracle and the GPU kernels see the same bits."""

    def __init__(self):
        self.seed = 0

    def _g(self):
        import torch

        g = torch.Generator().manual_seed(self.seed)
        self.seed += 1
        return g

    def randn(self, *shape, scale=1.0, dtype=None):
        import torch

        t = torch.randn(*shape, generator=self._g()) * scale
        return t if dtype is None else t.to(dtype)

    def rand(self, *shape):
        import torch

        return torch.rand(*shape, generator=self._g())


def trimul_weights(gen, C, Ch, dtype, ln_random):
    import torch

    w = {
        "norm_in_weight": (1 + 0.1 * gen.randn(C)) if ln_random else torch.ones(C),
        "norm_in_bias": (0.1 * gen.randn(C)) if ln_random else torch.zeros(C),
        "p_in_weight": gen.randn(2 * Ch, C, scale=C**-0.5),
        "g_in_weight": gen.randn(2 * Ch, C, scale=C**-0.5),
        "norm_out_weight": (1 + 0.1 * gen.randn(Ch)) if ln_random else torch.ones(Ch),
        "norm_out_bias": (0.1 * gen.randn(Ch)) if ln_random else torch.zeros(Ch),
        "p_out_weight": gen.randn(C, Ch, scale=Ch**-0.5),
        "g_out_weight": gen.randn(C, C, scale=C**-0.5),
    }
    return {k: v.to(dtype) for k, v in w.items()}


class AttnCall:
    """One gnn_triattn_fwd call on device tensors (any strides), with its workspace."""

    def __init__(self, q, k, v, bias=None, mask=None, precision="ieee"):
        import torch

        from geometric_nn_ops_torch import _lib
        from geometric_nn_ops_torch.triangle._kernels import triangle_attention as TA
        from geometric_nn_ops_torch.triangle._masking import rounded_mask_value

        self.lib = _lib.load()
        B, S, N, H, D = q.shape
        self.o = torch.empty((B, S, N, H, D), device=q.device, dtype=q.dtype)
        a = _lib.TriAttnArgs()
        a.q, a.k, a.v, a.o = q.data_ptr(), k.data_ptr(), v.data_ptr(), self.o.data_ptr()
        a.B, a.S, a.N, a.H, a.D = B, S, N, H, D
        for name, t in (("q_stride", q), ("k_stride", k), ("v_stride", v), ("o_stride", self.o)):
            setattr(a, name, _lib.I64x4(*t.stride()[:4]))
        if mask is not None:
            a.mask = mask.data_ptr()
            a.mask_stride = _lib.I64x3(mask.stride(0), mask.stride(1), mask.stride(4))
        a.scale, a.mask_value = D**-0.5, rounded_mask_value(q.dtype)
        a.dtype = _lib.DTYPE_CODE[q.dtype]
        a.precision = _lib.PRECISION_CODE["bf16x3" if precision == "tf32" else "ieee"]
        if bias is not None:
            bias = TA.bias_for_kernel(a, bias, q.dtype)  # the layout the library's kernel reads
        self.ws = TA.workspace_for(a, q.device)
        self.args = a
        self.keep = (q, k, v, bias, mask)

    def __call__(self):
        import torch

        from geometric_nn_ops_torch import _lib

        st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        _lib.check(self.lib.gnn_triattn_fwd(ctypes.byref(self.args), st), "gnn_triattn_fwd")


class TrimulCall:
    """gnn_trimul_fwd (or one of its stages) on device tensors, with its workspace."""

    def __init__(self, x, direction, mask, w, precision="ieee"):
        from geometric_nn_ops_torch import _lib
        from geometric_nn_ops_torch.triangle._kernels import trimul as TK

        self.lib = _lib.load()
        self.args, self.keep, self.out, self.ws, _ = TK.build_args(x, direction, mask, 1e-5, w)
        if x.dtype.itemsize == 4:
            self.args.precision = _lib.PRECISION_CODE["bf16x3" if precision == "tf32" else "ieee"]

    def stage(self, name):
        import torch

        from geometric_nn_ops_torch import _lib

        fn = getattr(self.lib, f"gnn_trimul_{name}")

        def run():
            st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
            _lib.check(fn(ctypes.byref(self.args), st), "trimul")
        return run


# ------------------------------------------------------------------------------ main
def main():
    args = parse()
    if args.summarize_trace:
        print(summarize_trace(args.summarize_trace, args.steps))
        return
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {args.gpus}); "
              "the hot path would shard over (b, s) rows and channels without collectives",
              file=sys.stderr)
        sys.exit(2)

    import torch

    from geometric_nn_ops_torch import _lib
    from geometric_nn_ops_torch.triangle._kernels import triangle_attention as TA
    from oracle import triangle_oracle as O

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.copy_calib:
        src = torch.ones(256 << 20, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calib_bytes_read": src.numel(), "copy_calib_bytes_written": dst.numel()}))
        return
    lib = _lib.load()
    N, H, D, C, CH = args.n, 4, 32, 128, 128
    dt = torch.bfloat16
    f64 = lambda t: t.double().cpu().numpy()  # noqa: E731

    # ---- the headline step's synthetic inputs (CPU, seeded), moved to HBM
    gen = Gen()
    q, k, v = (gen.randn(1, N, N, H, D, dtype=dt) for _ in range(3))
    bias = gen.randn(1, 1, H, N, N, dtype=dt)
    x = gen.randn(1, N, N, C, dtype=dt)
    w = trimul_weights(gen, C, CH, dt, ln_random=True)
    live = torch.arange(N) < N - 64
    tmask = (live[:, None] & live[None, :]).to(dt)[None]
    qd, kd, vd, bd = q.to(dev), k.to(dev), v.to(dev), bias.to(dev)
    wd = {kk: vv.to(dev) for kk, vv in w.items()}
    xd, md = x.to(dev), tmask.to(dev)
    attn = AttnCall(qd, kd, vd, bd)
    tri = {d: TrimulCall(xd, d, md, wd) for d in ("outgoing", "incoming")}
    stream = torch.cuda.current_stream(dev)
    if args.only == "configs":  # profile helper: the other BASELINE configurations alone
        print(json.dumps({"only": "configs", "configs": run_configs(dev, stream)}), flush=True)
        return

    kernels = []  # (name, callable): one C-ABI entry point each
    if args.only in (None, "attn"):
        kernels.append(("triattn_fwd", attn))
    if args.only in (None, "trimul"):
        for direction in ("outgoing", "incoming"):
            for stage in ("proj", "contract", "out"):
                kernels.append((f"trimul_{stage}_{direction}", tri[direction].stage(stage)))

    # ---- parity gate: every output of the step against the fp64 oracle (sampled rows /
    # pixels, the math being row- / pixel-independent)
    for _, fn in kernels:
        fn()
    torch.cuda.synchronize()
    gate = {}
    rows = [0, 1, N // 2, N - 1]
    if args.only in (None, "attn"):
        want = O.triangle_attention(f64(q[:, rows]), f64(k[:, rows]), f64(v[:, rows]), f64(bias), None, D**-0.5)
        gate["triattn_fwd"] = check_parity("triattn_fwd", parity(attn.o[:, rows], want))
    if args.only in (None, "trimul"):
        pr, pc = [0, 100, N - 65, N - 1], [0, 200, N - 64, N - 1]
        for direction in ("outgoing", "incoming"):
            want = O.trimul_grid(f64(x), direction, f64(tmask), pr, pc, **{kk: f64(vv) for kk, vv in w.items()})
            gate[f"trimul_{direction}"] = check_parity(direction, parity(tri[direction].out[:, pr][:, :, pc], want))

    # ---- per-kernel durations (median / mean over a >= 100 ms window each)
    flops, nbytes = {}, {}
    M = N * N
    e = 2
    flops["triattn_fwd"] = attn_flops(1, N, N, H, D)
    nbytes["triattn_fwd"] = attn_bytes(1, N, N, H, D, e)
    for direction in ("outgoing", "incoming"):
        flops[f"trimul_proj_{direction}"] = 2.0 * M * C * (4 * CH + C)  # p_in, g_in, output gate
        nbytes[f"trimul_proj_{direction}"] = e * M * C + e * M + 2 * e * M * CH + e * M * C  # x, mask -> a, b, g
        flops[f"trimul_contract_{direction}"] = 2.0 * N**3 * CH
        nbytes[f"trimul_contract_{direction}"] = 3.0 * e * M * CH
        flops[f"trimul_out_{direction}"] = 2.0 * M * CH * C  # p_out
        nbytes[f"trimul_out_{direction}"] = e * M * CH + 2.0 * e * M * C  # o, g -> out
    per_kernel, kern_mean = {}, {}
    for name, fn in kernels:
        med, mean, reps = window_ms(fn, stream)
        per_kernel[name] = rates(flops[name], nbytes[name], med)
        per_kernel[name].update({"mean_ms": round(mean, 5), "reps": reps})
        kern_mean[name] = mean

    # ---- the step: warm-up, then exactly `steps` steps back to back between two events
    def eager_step():
        for _, fn in kernels:
            fn()

    for _ in range(args.warmup):
        eager_step()

    def timed_steps(run_step, trace=False):
        t_start = torch.cuda.Event(enable_timing=True)
        t_end = torch.cuda.Event(enable_timing=True)
        if trace:
            region_marker()
        torch.cuda.synchronize()
        gc.disable()  # no collector pause inside the timed launches
        t0 = time.perf_counter()
        t_start.record(stream)
        for _ in range(args.steps):
            run_step()
        t_end.record(stream)
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        gc.enable()
        if trace:
            region_marker()
            torch.cuda.synchronize()
        return t_start.elapsed_time(t_end) / args.steps, wall

    outputs = ([attn.o] if args.only in (None, "attn") else []) + \
        ([tri[d].out for d in ("outgoing", "incoming")] if args.only in (None, "trimul") else [])
    ms_step, wall_eager = timed_steps(eager_step, trace=args.trace_steps)

    # ---- in-step durations: the same number of steps again with an event pair around every
    # entry point, so each one runs in the cache state the step leaves it in (the step's other
    # kernels evict its inputs from the 256 MB Infinity Cache, which the warm windows above
    # keep them in); the sum of the per-entry-point means is checked against ms_per_step
    in_ev = {name: [] for name, _ in kernels}
    torch.cuda.synchronize()
    gc.disable()
    for _ in range(args.steps):
        for name, fn in kernels:
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            fn()
            e1.record(stream)
            in_ev[name].append((e0, e1))
    torch.cuda.synchronize()
    gc.enable()
    in_step = {}
    for name, pairs in in_ev.items():
        ts = [e0.elapsed_time(e1) for e0, e1 in pairs]
        in_step[name] = {"mean_ms": round(sum(ts) / len(ts), 5), "median_ms": round(statistics.median(ts), 5),
                         "warm_mean_ms": round(kern_mean[name], 5)}
    in_step_sum = sum(r["mean_ms"] for r in in_step.values())
    want_out = [t.clone() for t in outputs]
    graph_ms, graph_ok = None, None
    try:
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            eager_step()
        for t in outputs:
            t.zero_()
        graph.replay()
        torch.cuda.synchronize()
        graph_ok = all(torch.equal(t, ww) for t, ww in zip(outputs, want_out))
        if graph_ok:
            graph_ms, _ = timed_steps(graph.replay, trace=args.trace_steps)
            graph_ok = all(torch.equal(t, ww) for t, ww in zip(outputs, want_out))
    except Exception as exc:  # pragma: no cover - reported, eager numbers stand
        print(f"bench.py: HIP graph capture failed, eager timing used: {exc}", file=sys.stderr)

    # ---- what plain streaming reaches on this device: a 1 GiB device copy (read + write) and
    # a 1 GiB fill, each timed as the kernels are; the memory-bound kernels' GB/s compare to these
    hbm_ref = None
    if args.only is None:
        csrc = torch.ones(1 << 30, dtype=torch.uint8, device=dev)
        cdst = torch.empty_like(csrc)
        copy_ms, _, _ = window_ms(lambda: cdst.copy_(csrc), stream)
        fill_ms, _, _ = window_ms(lambda: cdst.fill_(1), stream)
        hbm_ref = {"copy_gbs": round(2 * csrc.numel() / (copy_ms * 1e-3) / 1e9, 1),
                   "fill_gbs": round(cdst.numel() / (fill_ms * 1e-3) / 1e9, 1),
                   "copy_frac_of_peak": round(2 * csrc.numel() / (copy_ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4)}
        for r in per_kernel.values():
            if r["bound"] == "hbm":
                r["frac_of_copy"] = round(r["gbs"] / hbm_ref["copy_gbs"], 4)
        del csrc, cdst

    # ---- cold: each launch after a scratch write larger than L2 + Infinity Cache
    cold_ms = {}
    if args.cold_steps > 0:
        scratch = torch.empty(512 << 20, dtype=torch.uint8, device=dev)
        cev = {name: [] for name, _ in kernels}
        for _ in range(args.cold_steps):
            for name, fn in kernels:
                scratch.fill_(1)
                e0 = torch.cuda.Event(enable_timing=True)
                e1 = torch.cuda.Event(enable_timing=True)
                e0.record(stream)
                fn()
                e1.record(stream)
                cev[name].append((e0, e1))
        torch.cuda.synchronize()
        cold_ms = {name: round(statistics.median(e0.elapsed_time(e1) for e0, e1 in pairs), 5)
                   for name, pairs in cev.items()}
        del scratch

    # ---- the public Python API at the headline shape, beside the C-ABI figures
    public = None
    if args.only is None:
        from geometric_nn_ops_torch.triangle import triangle_attention, triangle_multiplicative_update

        with torch.inference_mode():
            pa = window_ms(lambda: triangle_attention(qd, kd, vd, bd), stream)
            pt = window_ms(lambda: triangle_multiplicative_update(xd, "outgoing", md, **wd), stream)
        capi_trimul = window_ms(tri["outgoing"].stage("fwd"), stream)
        public = {"triangle_attention_ms": round(pa[0], 5), "c_abi_triattn_fwd_ms": per_kernel["triattn_fwd"]["ms"],
                  "triangle_multiplicative_update_outgoing_ms": round(pt[0], 5),
                  "c_abi_trimul_fwd_outgoing_ms": round(capi_trimul[0], 5)}
        # the cueq shim's return_aux (o, lse and the row maximum from one forward) against a
        # plain shim call, on the same inputs in cueq's (B, N, H, S, D) layout
        import cuequivariance_ops_torch as cueq

        cq, ck, cv = (t.transpose(2, 3) for t in (qd, kd, vd))
        with torch.inference_mode():
            plain = window_ms(lambda: cueq.triangle_attention(cq, ck, cv, bd, scale=D**-0.5), stream)
            aux = window_ms(lambda: cueq.triangle_attention(cq, ck, cv, bd, scale=D**-0.5, return_aux=True), stream)
        public.update({"cueq_triangle_attention_ms": round(plain[0], 5),
                       "cueq_triangle_attention_return_aux_ms": round(aux[0], 5),
                       "return_aux_over_plain": round(aux[0] / plain[0], 3)})

    # ---- the public ops: the reference harness's trimul size sweep, the attention ops, and
    # peak memory per call
    sweep = None
    if args.sweep and args.only is None:
        sweep = public_sweep(dev, stream)

    # ---- the other BASELINE configurations
    configs = None
    if not args.no_configs and args.only is None:
        configs = run_configs(dev, stream)

    # ---- attention backward (not part of the step): one gnn_triattn_bwd call on the same
    # inputs with a synthetic upstream gradient, after a forward that writes the lse
    backward = None
    if args.only in (None, "attn") and not args.no_backward:
        a = attn.args
        lse = torch.empty((1, N, H, N), device=dev, dtype=torch.float32)
        a.lse = lse.data_ptr()
        attn()
        a.lse = None
        dout = gen.randn(1, N, N, H, D, dtype=dt).to(dev)
        grads = [torch.empty_like(qd) for _ in range(3)]
        dbias = torch.empty((1, H, N, N), device=dev, dtype=torch.float32)
        delta = torch.empty((1, N, H, N), device=dev, dtype=torch.float32)
        splits = TA.dbias_splits(1, N, N, H)
        ws = torch.empty((splits, 1, H, N, N), device=dev, dtype=torch.float32)
        ba = _lib.TriAttnBwdArgs()
        ba.q, ba.k, ba.v, ba.o, ba.dout = qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), attn.o.data_ptr(), dout.data_ptr()
        ba.bias, ba.lse = bd.data_ptr(), lse.data_ptr()
        ba.dq, ba.dk, ba.dv = (t.data_ptr() for t in grads)
        ba.dbias, ba.delta, ba.dbias_ws, ba.dbias_splits = dbias.data_ptr(), delta.data_ptr(), ws.data_ptr(), splits
        ba.B, ba.S, ba.N, ba.H, ba.D = 1, N, N, H, D
        for name in ("q", "k", "v", "o", "do", "dq", "dk", "dv"):
            setattr(ba, f"{name}_stride", _lib.I64x4(*qd.stride()[:4]))
        ba.bias_stride = a.bias_stride
        ba.scale, ba.mask_value, ba.dtype, ba.precision = a.scale, a.mask_value, a.dtype, a.precision

        def bwd():
            _lib.check(lib.gnn_triattn_bwd(ctypes.byref(ba), ctypes.c_void_p(stream.cuda_stream)), "attn bwd")

        bwd_ms = window_ms(bwd, stream, warmup=3)[0]
        bwd_flops = 10.0 * N * H * N * N * D  # QK^T, dO V^T, P^T dO, dS^T Q', dS K
        backward = {"kernel": "gnn_triattn_bwd (dq with Delta, dk/dv, dbias over N_seq, ordered split sum)",
                    "ms": round(bwd_ms, 5), "algorithmic_tflops": round(bwd_flops / (bwd_ms * 1e-3) / 1e12, 2),
                    "mfma_frac": round(bwd_flops / (bwd_ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4),
                    "algorithmic_flops": bwd_flops, "dbias_splits": splits}

    # ---- trimul backward (not part of the step): forward + backward of the public op with
    # gradients on x and every weight, through the HIP path (_TrimulHip) and through autograd
    # over the torch restatement of trimul_torch, which is what the reference runs for
    # gradients (it has no native trimul backward)
    tri_backward = None
    if args.only in (None, "trimul") and not args.no_backward:
        from geometric_nn_ops_torch.triangle import _trimul as TM

        gout = gen.randn(1, N, N, C, dtype=dt).to(dev)

        def fwd_bwd(use_torch):
            xg = xd.detach().requires_grad_()
            wg = {kk: vv.detach().requires_grad_() for kk, vv in wd.items()}
            if use_torch:
                y = TM.trimul_torch(xg, "outgoing", md, eps=1e-5, **wg)
            else:
                y = TM.triangle_multiplicative_update(xg, "outgoing", md, eps=1e-5, **wg)
            y.backward(gout)

        tri_backward = {"direction": "outgoing",
                        "reference_behaviour": "autograd through trimul_torch (no native backward)"}
        for label, use_torch in (("hip_fwd_bwd_ms", False), ("torch_autograd_fwd_bwd_ms", True)):
            tri_backward[label] = round(window_ms(lambda: fwd_bwd(use_torch), stream, warmup=2, min_reps=5)[0], 4)

    # ---- roofline of the dominant kernel: its average launch time inside the step (the warm
    # window's average beside it)
    step_mean = {name: r["mean_ms"] for name, r in in_step.items()}
    dominant = max(step_mean, key=step_mean.get)
    dk = rates(flops[dominant], nbytes[dominant], step_mean[dominant])
    dk_warm = rates(flops[dominant], nbytes[dominant], kern_mean[dominant])
    traffic = None
    if TRAFFIC_FILE.exists():
        try:
            traffic = json.loads(TRAFFIC_FILE.read_text()).get(dominant)
        except Exception:
            traffic = None
    if dk["bound"] == "mfma":
        roof = {"kernel": dominant, "bound": "mfma", "achieved": dk["tflops"], "peak": PEAK_BF16_TFLOPS,
                "unit": "TFLOP/s", "frac": dk["mfma_frac"], "traffic": traffic}
    else:
        roof = {"kernel": dominant, "bound": "hbm", "achieved": dk["gbs"], "peak": PEAK_HBM_GBS,
                "unit": "GB/s", "frac": dk["hbm_frac"], "traffic": traffic}
    roof.update({"algorithmic_flops_per_launch": flops[dominant], "algorithmic_bytes_per_launch": nbytes[dominant],
                 "ai_flop_per_byte": dk["ai_flop_per_byte"], "ridge_flop_per_byte": round(RIDGE, 1),
                 "avg_launch_ms": round(step_mean[dominant], 5), "timing": "mean of its launches in the timed steps",
                 "mfma_frac": dk["mfma_frac"], "hbm_frac": dk["hbm_frac"],
                 "warm": {"avg_launch_ms": round(kern_mean[dominant], 5), "achieved": dk_warm[
                     "tflops" if dk["bound"] == "mfma" else "gbs"], "mfma_frac": dk_warm["mfma_frac"],
                     "hbm_frac": dk_warm["hbm_frac"]}})
    for name, r in in_step.items():
        rr = rates(flops[name], nbytes[name], r["mean_ms"])
        r.update({"tflops": rr["tflops"], "gbs": rr["gbs"], "mfma_frac": rr["mfma_frac"], "hbm_frac": rr["hbm_frac"]})

    step_flops = sum(flops[name] for name, _ in kernels)
    value = step_flops / (ms_step * 1e-3) / 1e12
    line = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "triangle_attention fwd (N_seq=N_res=512, H=4, D=32, pair bias) + "
                               "triangle_multiplicative_update fwd outgoing + incoming (N=512, c_z=c_hidden=128, "
                               "last 64 residues masked)",
                   "N_res": N, "N_seq": N, "heads": H, "head_dim": D, "c_z": C, "c_hidden": CH, "batch": 1,
                   "only": args.only},
        "roofline": roof,
        "mfma_frac_step": round(value / PEAK_BF16_TFLOPS, 4),
        "graph_ms_per_step": round(graph_ms, 5) if graph_ms is not None else None,
        "graph_replays_match_eager": graph_ok,
        "in_step": {"kernels": in_step, "sum_of_means_ms": round(in_step_sum, 5),
                    "sum_over_ms_per_step": round(in_step_sum / ms_step, 4)},
        "kernels": per_kernel,
        "hbm_reference": hbm_ref,
        "parity": gate,
        "cold_ms": cold_ms,
        "cold_ms_per_step": round(sum(cold_ms.values()), 5) if cold_ms else None,
        "public_api_ms": public,
        "configs": configs,
        "public_sweep": sweep,
        "triton_reference": "unavailable: the reference's Triton kernels are not installed on the box and "
                            "the reference does not travel to it",
        "wall_s_timed": round(wall_eager, 4),
        "attention_backward": backward,
        "trimul_backward": tri_backward,
    }
    if args.no_cpu or args.only is not None:
        line["cpu_baseline"] = None
    else:
        line["cpu_baseline"] = cpu_baseline(q, k, v, bias, x, tmask, w, step_flops)
    print(json.dumps(line), flush=True)


# ---------------------------------------------------------- public ops: sweep and memory
GIB = float(1 << 30)


def peak_gib(fn):
    """Peak allocated and reserved GiB over one call of ``fn`` (the reference harness's
    peak_memory_gib, benchmarks/_bench_common.py:74-92: vendor-BLAS workspaces and the
    allocator's cache released first, so the figure does not depend on run order)."""
    import torch

    torch.cuda.synchronize()
    clear = getattr(torch._C, "_cuda_clearCublasWorkspaces", None)
    if clear is not None:
        clear()
    torch.cuda.empty_cache()
    torch.cuda.reset_peak_memory_stats()
    fn()
    torch.cuda.synchronize()
    return {"allocated_gib": round(torch.cuda.max_memory_allocated() / GIB, 4),
            "reserved_gib": round(torch.cuda.max_memory_reserved() / GIB, 4)}


def public_sweep(dev, stream):
    """The reference harness's trimul micro-benchmark through the public op
    (benchmarks/bench_trimul_micro.py:55-98 at its sizes 256 / 384 / 512 / 768, :115), both
    directions, bf16, c_z = 128: ``fwd_train_ms`` (x and the weights require grad, so the
    forward saves what the backward needs), ``fwd_infer_ms`` (inference_mode) and ``bwd_ms``
    (autograd.grad over x and every weight, retain_graph), each the median of a >= 100 ms
    window; with the peak memory of one inference forward and of one forward + backward. The
    same columns for triangle_attention at the headline shape and attention_pair_bias at the
    AF3 pairformer size (its backward runs the torch path: the reference has no other)."""
    import torch

    from geometric_nn_ops_torch.triangle import (attention_pair_bias, triangle_attention,
                                                 triangle_multiplicative_update)

    def columns(fwd, grad_inputs):
        def fwd_infer():
            with torch.inference_mode():
                return fwd()

        out = fwd()
        gout = torch.randn_like(out)

        def bwd():
            torch.autograd.grad([out], grad_inputs, grad_outputs=[gout], retain_graph=True)

        def fwd_bwd():
            y = fwd()
            torch.autograd.grad([y], grad_inputs, grad_outputs=[gout])

        row = {"fwd_train_ms": round(window_ms(fwd, stream, warmup=3, min_reps=5)[0], 5),
               "fwd_infer_ms": round(window_ms(fwd_infer, stream, warmup=3, min_reps=5)[0], 5),
               "bwd_ms": round(window_ms(bwd, stream, warmup=3, min_reps=5)[0], 5)}
        del out
        row["peak_fwd_infer"] = peak_gib(fwd_infer)
        row["peak_fwd_bwd"] = peak_gib(fwd_bwd)
        return row

    res = {"trimul": {}}
    C = 128
    for N in (256, 384, 512, 768):
        gen = Gen()
        x = gen.randn(1, N, N, C, dtype=torch.bfloat16).to(dev).requires_grad_()
        w = {kk: vv.to(dev).requires_grad_() for kk, vv in
             trimul_weights(gen, C, C, torch.bfloat16, ln_random=True).items()}
        live = torch.arange(N, device=dev) < N - N // 8
        mask = (live[:, None] & live[None, :]).to(torch.bfloat16)[None]
        for direction in ("outgoing", "incoming"):
            res["trimul"][f"n{N}_{direction}"] = columns(
                lambda: triangle_multiplicative_update(x, direction, mask, **w), [x, *w.values()])
        del x, w

    gen = Gen()
    N, H, D = 512, 4, 32
    q, k, v = (gen.randn(1, N, N, H, D, dtype=torch.bfloat16).to(dev).requires_grad_() for _ in range(3))
    bias = gen.randn(1, 1, H, N, N, dtype=torch.bfloat16).to(dev).requires_grad_()
    res["triangle_attention_n512"] = columns(lambda: triangle_attention(q, k, v, bias), [q, k, v, bias])
    del q, k, v, bias

    # fp32 attention gradients at the C5 fp32 size (N_seq = N_res = 384): the HIP backward under
    # both fp32 precision settings against autograd through the torch restatement (which
    # materialises the [B, S, H, N, N] fp32 logits), forward + backward and its peak memory
    from geometric_nn_ops_torch.triangle._reference.triangle_attention import triangle_attention_torch

    gen = Gen()
    N, H, D = 384, 4, 32
    q, k, v = (gen.randn(1, N, N, H, D).to(dev).requires_grad_() for _ in range(3))
    bias = gen.randn(1, 1, H, N, N).to(dev).requires_grad_()
    gout = gen.randn(1, N, N, H, D).to(dev)
    fp32 = {}
    old_prec = torch.backends.cuda.matmul.fp32_precision
    try:
        for label, prec, fn in (("hip_ieee", "ieee", triangle_attention), ("hip_tf32", "tf32", triangle_attention),
                                ("torch_autograd", "ieee", triangle_attention_torch)):
            torch.backends.cuda.matmul.fp32_precision = prec

            def fwd_bwd():
                torch.autograd.grad([fn(q, k, v, bias)], [q, k, v, bias], grad_outputs=[gout])

            fp32[label] = {"fwd_bwd_ms": round(window_ms(fwd_bwd, stream, warmup=2, min_reps=3)[0], 4),
                           "peak": peak_gib(fwd_bwd)}
    finally:
        torch.backends.cuda.matmul.fp32_precision = old_prec
    res["triangle_attention_fp32_n384_fwd_bwd"] = fp32
    del q, k, v, bias, gout

    gen = Gen()
    B, H, U, DH, Zc, Cs = 1, 16, 384, 24, 128, 384
    s = gen.randn(B, U, Cs, dtype=torch.bfloat16).to(dev).requires_grad_()
    q, k, v = (gen.randn(B, H, U, DH, dtype=torch.bfloat16).to(dev).requires_grad_() for _ in range(3))
    z = gen.randn(B, U, U, Zc, dtype=torch.bfloat16).to(dev).requires_grad_()
    wts = {"proj_g_weight": gen.randn(Cs, Cs, scale=Cs**-0.5), "proj_o_weight": gen.randn(Cs, Cs, scale=Cs**-0.5),
           "proj_z_weight": gen.randn(H, Zc, scale=Zc**-0.5), "ln_z_weight": 1.0 + gen.randn(Zc, scale=0.1)}
    wts = {kk: vv.to(dev, torch.bfloat16).requires_grad_() for kk, vv in wts.items()}
    mask = (torch.arange(U, device=dev) < U - 40).to(torch.bfloat16)[None]
    res["attention_pair_bias_af3_384"] = columns(
        lambda: attention_pair_bias(s, q, k, v, z, mask=mask, **wts)[0], [s, q, k, v, z, *wts.values()])
    res["attention_pair_bias_af3_384"]["shape"] = "B=1, tokens=384, H=16, DH=24, c_s=384, c_z=128, 40 keys masked"
    return res


# ------------------------------------------------------------------- other configurations
def run_configs(dev, stream):
    """C2, C3, C4 and the C5 blocks of BASELINE.json: median ms over a >= 100 ms window,
    rates against the peaks, and parity against the fp64 oracle on sampled rows / pixels."""
    import torch

    from oracle import triangle_oracle as O

    f64 = lambda t: t.double().cpu().numpy()  # noqa: E731
    out = {}
    dt = torch.bfloat16

    # C2: attention N=256 bf16 in the cueq layout [B, S, H, N, D], read as [B, S, N, H, D]
    # views; keys 230..255 masked
    gen = Gen()
    N, H, D = 256, 4, 32
    q, k, v = (gen.randn(1, N, H, N, D, dtype=dt) for _ in range(3))
    bias = gen.randn(1, 1, H, N, N, dtype=dt)
    mask = torch.ones(1, N, 1, 1, N, dtype=torch.bool)
    mask[..., N - 26:] = False
    sw = lambda t: t.transpose(2, 3)  # noqa: E731
    call = AttnCall(sw(q.to(dev)), sw(k.to(dev)), sw(v.to(dev)), bias.to(dev), mask.to(dev))
    call()
    rows = list(range(0, N, 8))
    want = O.triangle_attention(f64(sw(q)[:, rows]), f64(sw(k)[:, rows]), f64(sw(v)[:, rows]), f64(bias),
                                mask[:, rows].numpy(), D**-0.5)
    par = check_parity("C2", parity(call.o[:, rows], want))
    med = window_ms(call, stream)[0]
    out["C2_triattn_n256_cueq_layout_tail26"] = {
        **rates(attn_flops(1, N, N, H, D), attn_bytes(1, N, N, H, D, 2, mask=True), med),
        "parity": par, "parity_rows": f"{len(rows)} of {N}"}
    del call

    # C3: trimul N=512 bf16 both directions as one gnn_trimul_fwd call each
    gen = Gen()
    N, C = 512, 128
    x = gen.randn(1, N, N, C, dtype=dt)
    w = trimul_weights(gen, C, C, dt, ln_random=True)
    live = torch.arange(N) < N - 64
    tmask = (live[:, None] & live[None, :]).to(dt)[None]
    xd, md, wd = x.to(dev), tmask.to(dev), {kk: vv.to(dev) for kk, vv in w.items()}
    pr, pc = [3, 300, N - 1], [5, 447, N - 1]
    for direction in ("outgoing", "incoming"):
        t = TrimulCall(xd, direction, md, wd)
        fwd = t.stage("fwd")
        fwd()
        want = O.trimul_grid(f64(x), direction, f64(tmask), pr, pc, **{kk: f64(vv) for kk, vv in w.items()})
        par = check_parity(f"C3 {direction}", parity(t.out[:, pr][:, :, pc], want))
        med = window_ms(fwd, stream)[0]
        out[f"C3_trimul_n512_{direction}"] = {**rates(trimul_flops(1, N, C, C), trimul_bytes(1, N, C, C, 2), med),
                                              "parity": par}
        del t

    # C4: attention N=768 bf16, bias 2 N(0,1), each row a random valid length in [384, 768]
    gen = Gen()
    N = 768
    q, k, v = (gen.randn(1, N, N, H, D, dtype=dt) for _ in range(3))
    bias = gen.randn(1, 1, H, N, N, scale=2.0, dtype=dt)
    lengths = (384 + (gen.rand(N) * 385).floor().long()).clamp(max=N)
    mask = (torch.arange(N)[None, :] < lengths[:, None]).view(1, N, 1, 1, N)
    call = AttnCall(q.to(dev), k.to(dev), v.to(dev), bias.to(dev), mask.to(dev))
    call()
    rows = [0, 1, N // 3, N // 2, N - 2, N - 1]
    want = O.triangle_attention(f64(q[:, rows]), f64(k[:, rows]), f64(v[:, rows]), f64(bias), mask[:, rows].numpy(),
                                D**-0.5)
    par = check_parity("C4", parity(call.o[:, rows], want))
    med = window_ms(call, stream)[0]
    out["C4_triattn_n768_ragged"] = {
        **rates(attn_flops(1, N, N, H, D), attn_bytes(1, N, N, H, D, 2, mask=True), med),
        "parity": par, "parity_rows": f"{len(rows)} of {N}", "mean_valid_keys": float(lengths.float().mean())}
    del call

    # C5: the pair-stack block: trimul outgoing, incoming, attention starting node, ending node
    # (transposed views of q / k / v and the bias)
    for N, dtype, precision in ((1024, torch.bfloat16, "ieee"), (384, torch.float32, "ieee"),
                                (384, torch.float32, "tf32")):
        tag = "bf16" if dtype == torch.bfloat16 else f"fp32_{precision}"
        out[f"C5_block_n{N}_{tag}"] = block(dev, stream, N, dtype, precision)
    return out


def block(dev, stream, N, dtype, precision):
    """One pair-stack block (four C-ABI calls), per op and whole; fp32 under ``precision``
    ('ieee' or 'tf32', which resolves to the bf16x3 split on gfx950)."""
    import torch

    from oracle import triangle_oracle as O

    f64 = lambda t: t.double().cpu().numpy()  # noqa: E731
    gen = Gen()
    H, D, C = 4, 32, 128
    x = gen.randn(1, N, N, C, dtype=dtype)
    w = trimul_weights(gen, C, C, dtype, ln_random=False)
    q, k, v = (gen.randn(1, N, N, H, D, dtype=dtype) for _ in range(3))
    bias = gen.randn(1, 1, H, N, N, dtype=dtype)
    xd, wd = x.to(dev), {kk: vv.to(dev) for kk, vv in w.items()}
    qd, kd, vd, bd = q.to(dev), k.to(dev), v.to(dev), bias.to(dev)
    tr = lambda t: t.transpose(1, 2)  # noqa: E731
    t_out = TrimulCall(xd, "outgoing", None, wd, precision)
    t_in = TrimulCall(xd, "incoming", None, wd, precision)
    a_start = AttnCall(qd, kd, vd, bd, None, precision)
    a_end = AttnCall(tr(qd), tr(kd), tr(vd), bd.transpose(-1, -2), None, precision)
    ops = [("trimul_outgoing", t_out.stage("fwd")), ("trimul_incoming", t_in.stage("fwd")),
           ("triattn_starting", a_start), ("triattn_ending", a_end)]

    def run_block():
        for _, fn in ops:
            fn()

    run_block()
    torch.cuda.synchronize()
    # parity: trimul on sampled pixels, attention on sampled N_seq rows of each node
    bound = 1e-2 if dtype == torch.bfloat16 else (1.5e-3 if precision == "ieee" else 2e-3)
    pr, pc = [0, N // 2, N - 1], [1, N // 3, N - 1]
    wn = {kk: f64(vv) for kk, vv in w.items()}
    par = {}
    for name, t, direction in (("trimul_outgoing", t_out, "outgoing"), ("trimul_incoming", t_in, "incoming")):
        want = O.trimul_grid(f64(x), direction, None, pr, pc, **wn)
        par[name] = check_parity(f"C5 {name}", parity(t.out[:, pr][:, :, pc], want), bound)
    rows = [0, N - 1]
    for name, call, (qq, kk, vv, bb) in (("triattn_starting", a_start, (q, k, v, bias)),
                                         ("triattn_ending", a_end, (tr(q), tr(k), tr(v), bias.transpose(-1, -2)))):
        want = O.triangle_attention(f64(qq[:, rows]), f64(kk[:, rows]), f64(vv[:, rows]), f64(bb), None, D**-0.5)
        par[name] = check_parity(f"C5 {name}", parity(call.o[:, rows], want), bound)

    peak = PEAK_BF16_TFLOPS if dtype == torch.bfloat16 else \
        (PEAK_FP32_TFLOPS if precision == "ieee" else PEAK_BF16_TFLOPS / 3)
    e = 2 if dtype == torch.bfloat16 else 4
    fl = {"trimul_outgoing": trimul_flops(1, N, C, C), "trimul_incoming": trimul_flops(1, N, C, C),
          "triattn_starting": attn_flops(1, N, N, H, D), "triattn_ending": attn_flops(1, N, N, H, D)}
    by = {"trimul_outgoing": trimul_bytes(1, N, C, C, e, mask=False),
          "trimul_incoming": trimul_bytes(1, N, C, C, e, mask=False),
          "triattn_starting": attn_bytes(1, N, N, H, D, e), "triattn_ending": attn_bytes(1, N, N, H, D, e)}
    res = {"precision": precision if dtype == torch.float32 else "native", "peak_tflops_used": round(peak, 1),
           "ops": {name: rates(fl[name], by[name], window_ms(fn, stream)[0], peak) for name, fn in ops}}
    res.update(rates(sum(fl.values()), sum(by.values()), window_ms(run_block, stream, warmup=3)[0], peak))
    res["parity"] = par
    if dtype == torch.bfloat16:  # the three trimul kernels on their own (outgoing)
        M, e2 = N * N, 2
        sfl = {"proj": 2.0 * M * C * (4 * C + C), "contract": 2.0 * N**3 * C, "out": 2.0 * M * C * C}
        sby = {"proj": e2 * M * C + 2 * e2 * M * C + e2 * M * C, "contract": 3.0 * e2 * M * C,
               "out": e2 * M * C + 2.0 * e2 * M * C}
        res["trimul_outgoing_kernels"] = {
            name: rates(sfl[name], sby[name], window_ms(t_out.stage(name), stream)[0], peak)
            for name in ("proj", "contract", "out")}
        # the vendor's batched GEMM (torch.bmm, hipBLASLt) on operands of the contraction's
        # shape: C planes of [N, N] x [N, N]^T, the right operand made contiguous first
        va = torch.randn(C, N, N, dtype=dtype, device=dev)
        vb = torch.randn(C, N, N, dtype=dtype, device=dev).transpose(1, 2).contiguous()
        vo = torch.empty(C, N, N, dtype=dtype, device=dev)
        res["trimul_outgoing_kernels"]["contract_vendor_bmm"] = rates(
            sfl["contract"], sby["contract"], window_ms(lambda: torch.bmm(va, vb, out=vo), stream)[0], peak)
        del va, vb, vo
    return res


# --------------------------------------------------------------------------- CPU baseline
def cpu_baseline(q, k, v, bias, x, tmask, w, step_flops):
    """The package's pure-torch path (triangle/_reference/, op for op the reference's
    trimul_torch and triangle_attention_torch) on the host cores, in bf16: the headline step
    (attention over all N_seq rows in chunks of 16, the [B, S, H, N, N] logits otherwise being
    2 GB; trimul both directions) with 1 warm-up and the median of 3, plus C1 (trimul
    outgoing, fp32, N=64) the same way with the median of 5."""
    import torch

    from geometric_nn_ops_torch.triangle._reference.triangle_attention import triangle_attention_torch
    from geometric_nn_ops_torch.triangle._reference.trimul import trimul_torch

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    model = "unknown"
    try:
        for ln in pathlib.Path("/proc/cpuinfo").read_text().splitlines():
            if ln.startswith("model name"):
                model = ln.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    S = q.shape[1]

    def step():
        with torch.inference_mode():
            for s0 in range(0, S, 16):
                triangle_attention_torch(q[:, s0:s0 + 16], k[:, s0:s0 + 16], v[:, s0:s0 + 16], bias=bias)
            for direction in ("outgoing", "incoming"):
                trimul_torch(x, direction, tmask, eps=1e-5, **w)

    def timed(fn, reps=3):
        fn()
        ts = []
        for _ in range(reps):
            t0 = time.perf_counter()
            fn()
            ts.append(time.perf_counter() - t0)
        return statistics.median(ts)

    sec = timed(step)
    gen = Gen()
    x1 = gen.randn(1, 64, 64, 128)
    w1 = trimul_weights(gen, 128, 128, torch.float32, ln_random=False)
    m1 = torch.ones(1, 64, 64)
    with torch.inference_mode():
        c1 = timed(lambda: trimul_torch(x1, "outgoing", m1, eps=1e-5, **w1), reps=5)
    return {"value": round(step_flops / sec / 1e12, 5), "unit": "TFLOP/s", "cores": cores, "kind": "port",
            "implementation": "the package's pure-torch restatement (geometric_nn_ops_torch.triangle._reference), "
                              "the reference's trimul_torch / triangle_attention_torch op for op",
            "cpu_model": model, "threads": torch.get_num_threads(), "dtype": "bf16",
            "sample": "the whole headline step (attention over all 512 N_seq rows in chunks of 16; trimul N=512 "
                      "both directions), 1 warm-up + median of 3",
            "ms_per_step": round(sec * 1e3, 1),
            "C1_trimul_outgoing_fp32_n64_ms": round(c1 * 1e3, 2),
            "C1_tflops": round(trimul_flops(1, 64, 128, 128) / c1 / 1e12, 4)}


if __name__ == "__main__":
    main()
