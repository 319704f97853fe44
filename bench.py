"""Benchmark of the triangle inference hot path on one MI355X.

One step = the BASELINE.json headline workload at N_res = 512, bf16, B = 1:
  * triangle_attention forward, N_seq = N_res = 512, H = 4, D = 32, pair bias, no mask;
  * triangle_multiplicative_update forward, c_z = c_hidden = 128, 'outgoing';
  * the same with 'incoming' (mask: the last 64 residues padded on both axes).
Every kernel is launched through the C ABI (libgnn_hip.so) with inputs, outputs and the
trimul workspace already resident in HBM; per-kernel durations come from HIP events
recorded on the launch stream around each launch, in a loop of their own; ``ms_per_step``
and ``value`` come from ``--steps`` further steps launched back to back with events only
around the whole loop. ``graph_ms_per_step`` times the same step captured once as a HIP graph
and replayed ``--steps`` times (outputs checked bitwise against the eager ones): the entry
points are capturable, and at this size replay gains nothing over eager launches.

Prints ONE JSON line: value = algorithmic TFLOP/s of the whole step (dense attention
FLOPs, softmax excluded; trimul 2 N^3 Ch + N^2 (10 C Ch + 2 C^2)), plus the roofline of
the dominant kernel and a CPU baseline (the numpy oracle in fp32 on a bounded sample of
the same workload, which also serves as the parity gate before timing). ``cold_ms`` times
each kernel again after a 512 MiB scratch write (inputs then come from HBM, not from the
Infinity Cache that holds them in the warm loop); ``value`` is the warm figure.
``attention_backward`` times one gnn_triattn_bwd call (dq, dk, dv and the pair-bias
gradient) on the same attention inputs, outside the step. ``trimul_backward`` times forward +
backward of the outgoing trimul with gradients on x and every weight, on the HIP path and on
autograd through the torch restatement (what the reference runs for gradients), outside the
step.
"""

import argparse
import ctypes
import json
import os
import pathlib
import sys
import time

ROOT = pathlib.Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "geometric-nn-ops_amd"))
sys.path.insert(0, str(ROOT))

METRIC = "trimul + triangle-attn fwd ms & TFLOP/s at N=512 bf16; % of MFMA peak"
PEAK_BF16_TFLOPS = 2516.6
PEAK_HBM_GBS = 8000.0
TRAFFIC_FILE = ROOT / "profiles" / "traffic_n512_bf16.json"


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--n", type=int, default=512)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline / parity gate")
    ap.add_argument("--cold-steps", type=int, default=3,
                    help="steps timed cold: every kernel after a 512 MiB scratch write that evicts L2 and "
                         "the 256 MB Infinity Cache (0 skips)")
    ap.add_argument("--only", choices=["attn", "trimul"], default=None,
                    help="profile helper: run only one op (the JSON line is then partial)")
    ap.add_argument("--no-backward", action="store_true", help="skip the backward timings")
    ap.add_argument("--copy-calib", action="store_true",
                    help="profile helper: run a plain 256 MiB device copy (known HBM bytes) and exit, "
                         "to scale FETCH_SIZE / WRITE_SIZE counter readings")
    return ap.parse_args()


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {args.gpus}); "
              "the hot path shards over (b, s) rows and channels without collectives, see DESIGN.md",
              file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    from geometric_nn_ops_torch import _lib
    from geometric_nn_ops_torch.triangle._kernels import triangle_attention as TA
    from geometric_nn_ops_torch.triangle._kernels import trimul as TK
    from geometric_nn_ops_torch.triangle._masking import rounded_mask_value
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

    # ---- synthetic inputs, drawn on the CPU from seeded generators
    g = torch.Generator().manual_seed(0)
    rn = lambda *s, sc=1.0: (torch.randn(*s, generator=g) * sc).to(dt)  # noqa: E731
    q, k, v = rn(1, N, N, H, D), rn(1, N, N, H, D), rn(1, N, N, H, D)
    bias = rn(1, 1, H, N, N)
    x = rn(1, N, N, C)
    w = {
        "norm_in_weight": 1 + 0.1 * torch.randn(C, generator=g), "norm_in_bias": 0.1 * torch.randn(C, generator=g),
        "p_in_weight": torch.randn(2 * CH, C, generator=g) / C**0.5,
        "g_in_weight": torch.randn(2 * CH, C, generator=g) / C**0.5,
        "norm_out_weight": 1 + 0.1 * torch.randn(CH, generator=g),
        "norm_out_bias": 0.1 * torch.randn(CH, generator=g),
        "p_out_weight": torch.randn(C, CH, generator=g) / CH**0.5,
        "g_out_weight": torch.randn(C, C, generator=g) / C**0.5,
    }
    w = {kk: vv.to(dt) for kk, vv in w.items()}
    live = torch.arange(N) < N - 64
    tmask = (live[:, None] & live[None, :]).to(dt)[None]

    qd, kd, vd, bd = q.to(dev), k.to(dev), v.to(dev), bias.to(dev)
    od = torch.empty_like(qd)
    a = _lib.TriAttnArgs()
    a.q, a.k, a.v, a.o, a.bias = qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), od.data_ptr(), bd.data_ptr()
    a.B, a.S, a.N, a.H, a.D = 1, N, N, H, D
    for name, t in (("q_stride", qd), ("k_stride", kd), ("v_stride", vd), ("o_stride", od)):
        setattr(a, name, _lib.I64x4(*t.stride()[:4]))
    a.bias_stride = _lib.I64x4(bd.stride(0), bd.stride(2), bd.stride(3), bd.stride(4))
    a.scale, a.mask_value = D**-0.5, rounded_mask_value(dt)
    a.dtype, a.precision = _lib.GNN_BF16, _lib.GNN_PREC_IEEE
    attn_ws = TA.workspace_for(a, dev)  # noqa: F841 -- kept alive for every launch below

    wd = {kk: vv.to(dev) for kk, vv in w.items()}
    xd, md = x.to(dev), tmask.to(dev)
    tri = {}
    for direction in ("outgoing", "incoming"):
        targs, keep, tout, ws, _ = TK.build_args(xd, direction, md, 1e-5, wd)
        tri[direction] = (targs, keep, tout, ws)

    stream = torch.cuda.current_stream(dev)
    sh = ctypes.c_void_p(stream.cuda_stream)

    def check(rc, what):
        _lib.check(rc, what)

    def cur():  # the launch stream: the current one (a graph capture switches it)
        return ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)

    kernels = []  # (name, callable)
    if args.only in (None, "attn"):
        kernels.append(("triattn_fwd", lambda: check(lib.gnn_triattn_fwd(ctypes.byref(a), cur()), "attn")))
    if args.only in (None, "trimul"):
        for direction in ("outgoing", "incoming"):
            targs = tri[direction][0]
            for stage in ("proj", "contract", "out"):
                fn = getattr(lib, f"gnn_trimul_{stage}")
                kernels.append((f"trimul_{stage}_{direction}",
                                lambda fn=fn, targs=targs: check(fn(ctypes.byref(targs), cur()), "trimul")))

    # ---- parity gate + CPU baseline (numpy oracle, fp32, bounded sample)
    cpu = None
    parity = {}
    if not args.no_cpu:
        for _, fn in kernels:
            fn()
        torch.cuda.synchronize()
        f32 = lambda t: t.float().numpy()  # noqa: E731
        t_attn = t_tri = 0.0
        rows = list(range(0, N, N // 8))[:8]
        if args.only in (None, "attn"):
            t0 = time.perf_counter()
            want = O.triangle_attention(f32(q[:, rows]), f32(k[:, rows]), f32(v[:, rows]), f32(bias),
                                        None, D**-0.5, dtype=np.float32)
            t_attn = (time.perf_counter() - t0) * (N / len(rows))
            parity["triattn_rel_fro"] = O.rel_fro(od[:, rows].float().cpu().numpy(), want)
        if args.only in (None, "trimul"):
            for direction in ("outgoing", "incoming"):
                t0 = time.perf_counter()
                want = O.trimul(f32(x), direction, f32(tmask), dtype=np.float32,
                                **{kk: f32(vv) for kk, vv in w.items()})
                t_tri += time.perf_counter() - t0
                got = tri[direction][2].float().cpu().numpy()
                parity[f"trimul_{direction}_rel_fro"] = O.rel_fro(got, want)
        bad = {kk: vv for kk, vv in parity.items() if not vv <= 1e-2}
        if bad:
            print(f"bench.py: parity gate failed: {bad}", file=sys.stderr)
            sys.exit(1)
        try:
            from threadpoolctl import threadpool_info

            cores = max((i.get("num_threads", 1) for i in threadpool_info()), default=1)
        except Exception:  # pragma: no cover - threadpoolctl is optional
            cores = os.cpu_count()
        cpu = {"seconds_per_step": t_attn + t_tri, "cores": cores,
               "sample": f"numpy fp32 oracle: attention on {len(rows)} of {N} N_seq rows (time scaled "
                         f"x{N // len(rows)}), trimul full N={N} both directions"}

    # ---- warmup, then `steps` steps with per-kernel events (each kernel's duration), then
    # exactly `steps` timed steps launched eagerly and `steps` replays of the step captured
    # as a HIP graph (the same launches; replays are checked bitwise against the eager
    # outputs)
    for _ in range(args.warmup):
        for _, fn in kernels:
            fn()
    torch.cuda.synchronize()
    ev = {name: [] for name, _ in kernels}
    for _ in range(args.steps):
        for name, fn in kernels:
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            fn()
            e1.record(stream)
            ev[name].append((e0, e1))
    torch.cuda.synchronize()
    kern_ms = {name: sum(e0.elapsed_time(e1) for e0, e1 in pairs) / len(pairs) for name, pairs in ev.items()}

    def timed_steps(run_step):
        t_start = torch.cuda.Event(enable_timing=True)
        t_end = torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        t_start.record(stream)
        for _ in range(args.steps):
            run_step()
        t_end.record(stream)
        torch.cuda.synchronize()
        return t_start.elapsed_time(t_end) / args.steps, time.perf_counter() - t0

    def eager_step():
        for _, fn in kernels:
            fn()

    outputs = ([od] if args.only in (None, "attn") else []) + \
        ([tri[d][2] for d in ("outgoing", "incoming")] if args.only in (None, "trimul") else [])
    eager_ms, wall_eager = timed_steps(eager_step)
    want = [t.clone() for t in outputs]
    graph_ms, graph_ok = None, None
    try:
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            eager_step()
        for t in outputs:
            t.zero_()
        graph.replay()
        torch.cuda.synchronize()
        graph_ok = all(torch.equal(t, w) for t, w in zip(outputs, want))
        if graph_ok:
            graph_ms, _ = timed_steps(graph.replay)
            graph_ok = all(torch.equal(t, w) for t, w in zip(outputs, want))
    except Exception as exc:  # pragma: no cover - reported, eager numbers stand
        print(f"bench.py: HIP graph capture failed, eager timing used: {exc}", file=sys.stderr)
    ms_step = eager_ms

    # ---- cold: each launch after a scratch write larger than L2 + Infinity Cache, so its
    # inputs come from HBM (at N=512 the warm inputs otherwise stay cache resident)
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
        cold_ms = {name: round(sum(e0.elapsed_time(e1) for e0, e1 in pairs) / len(pairs), 5)
                   for name, pairs in cev.items()}
        del scratch

    # ---- attention backward (not part of the step): one gnn_triattn_bwd call on the same
    # inputs with a synthetic upstream gradient, after a forward that writes the lse
    backward = None
    if args.only in (None, "attn") and not args.no_backward:
        lse = torch.empty((1, N, H, N), device=dev, dtype=torch.float32)
        a.lse = lse.data_ptr()
        check(lib.gnn_triattn_fwd(ctypes.byref(a), sh), "attn+lse")
        a.lse = None
        dout = rn(1, N, N, H, D).to(dev)
        grads = [torch.empty_like(qd) for _ in range(3)]
        dbias = torch.empty((1, H, N, N), device=dev, dtype=torch.float32)
        delta = torch.empty((1, N, H, N), device=dev, dtype=torch.float32)
        splits = TA.dbias_splits(1, N, N, H)
        ws = torch.empty((splits, 1, H, N, N), device=dev, dtype=torch.float32)
        ba = _lib.TriAttnBwdArgs()
        ba.q, ba.k, ba.v, ba.o, ba.dout = qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), od.data_ptr(), dout.data_ptr()
        ba.bias, ba.lse = bd.data_ptr(), lse.data_ptr()
        ba.dq, ba.dk, ba.dv = (t.data_ptr() for t in grads)
        ba.dbias, ba.delta, ba.dbias_ws, ba.dbias_splits = dbias.data_ptr(), delta.data_ptr(), ws.data_ptr(), splits
        ba.B, ba.S, ba.N, ba.H, ba.D = 1, N, N, H, D
        for name in ("q", "k", "v", "o", "do", "dq", "dk", "dv"):
            setattr(ba, f"{name}_stride", _lib.I64x4(*qd.stride()[:4]))
        ba.bias_stride = a.bias_stride
        ba.scale, ba.mask_value, ba.dtype, ba.precision = a.scale, a.mask_value, a.dtype, a.precision
        for _ in range(3):
            check(lib.gnn_triattn_bwd(ctypes.byref(ba), sh), "attn bwd")
        bev = []
        for _ in range(10):
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            check(lib.gnn_triattn_bwd(ctypes.byref(ba), sh), "attn bwd")
            e1.record(stream)
            bev.append((e0, e1))
        torch.cuda.synchronize()
        bwd_ms = sorted(e0.elapsed_time(e1) for e0, e1 in bev)[len(bev) // 2]
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

        gout = rn(1, N, N, C).to(dev, dt)

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
            for _ in range(2):
                fwd_bwd(use_torch)
            tev = []
            for _ in range(5):
                e0 = torch.cuda.Event(enable_timing=True)
                e1 = torch.cuda.Event(enable_timing=True)
                e0.record(stream)
                fwd_bwd(use_torch)
                e1.record(stream)
                tev.append((e0, e1))
            torch.cuda.synchronize()
            tri_backward[label] = round(sorted(e0.elapsed_time(e1) for e0, e1 in tev)[len(tev) // 2], 4)

    # ---- algorithmic FLOPs / bytes per launch
    M = N * N
    e = 2
    flops = {"triattn_fwd": 4.0 * N * H * N * N * D}
    nbytes = {"triattn_fwd": e * 4.0 * N * N * H * D + e * H * N * N}
    for direction in ("outgoing", "incoming"):
        flops[f"trimul_proj_{direction}"] = 2.0 * M * C * (4 * CH + C)
        nbytes[f"trimul_proj_{direction}"] = e * M * C + e * M + 2 * e * M * CH + e * M * C
        flops[f"trimul_contract_{direction}"] = 2.0 * N**3 * CH
        nbytes[f"trimul_contract_{direction}"] = 3.0 * e * M * CH
        flops[f"trimul_out_{direction}"] = 2.0 * M * CH * C
        nbytes[f"trimul_out_{direction}"] = e * M * CH + 2.0 * e * M * C
    bound = {"triattn_fwd": "mfma"}
    for direction in ("outgoing", "incoming"):
        bound[f"trimul_proj_{direction}"] = "hbm"
        bound[f"trimul_contract_{direction}"] = "mfma"
        bound[f"trimul_out_{direction}"] = "hbm"

    per_kernel = {}
    for name, ms in kern_ms.items():
        tf = flops[name] / (ms * 1e-3) / 1e12
        gbs = nbytes[name] / (ms * 1e-3) / 1e9
        per_kernel[name] = {"ms": round(ms, 5), "tflops": round(tf, 2), "gbs": round(gbs, 1),
                            "mfma_frac": round(tf / PEAK_BF16_TFLOPS, 4), "hbm_frac": round(gbs / PEAK_HBM_GBS, 4),
                            "bound": bound[name]}
    dominant = max(kern_ms, key=kern_ms.get)
    dk = per_kernel[dominant]
    traffic = None
    if TRAFFIC_FILE.exists():
        try:
            traffic = json.loads(TRAFFIC_FILE.read_text()).get(dominant)
        except Exception:
            traffic = None
    if bound[dominant] == "mfma":
        roof = {"kernel": dominant, "bound": "mfma", "achieved": dk["tflops"], "peak": PEAK_BF16_TFLOPS,
                "unit": "TFLOP/s", "frac": dk["mfma_frac"], "traffic": traffic,
                "algorithmic_flops_per_launch": flops[dominant], "avg_launch_ms": dk["ms"]}
    else:
        roof = {"kernel": dominant, "bound": "hbm", "achieved": dk["gbs"], "peak": PEAK_HBM_GBS,
                "unit": "GB/s", "frac": dk["hbm_frac"], "traffic": traffic,
                "algorithmic_bytes_per_launch": nbytes[dominant], "avg_launch_ms": dk["ms"]}

    step_flops = sum(flops[name] for name in kern_ms)
    value = step_flops / (ms_step * 1e-3) / 1e12
    line = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 5),
        "graph_ms_per_step": round(graph_ms, 5) if graph_ms is not None else None,
        "graph_replays_match_eager": graph_ok,
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
        "kernels": per_kernel,
        "parity_rel_fro": {kk: float(f"{vv:.3e}") for kk, vv in parity.items()},
        "cold_ms": cold_ms,
        "cold_ms_per_step": round(sum(cold_ms.values()), 5) if cold_ms else None,
        "triton_reference": "unavailable: the reference's Triton kernels are not installed on the box and "
                            "the reference does not travel to it",
        "wall_s_timed": round(wall_eager, 4),
        "attention_backward": backward,
        "trimul_backward": tri_backward,
    }
    if cpu is not None:
        cpu_tflops = step_flops / cpu["seconds_per_step"] / 1e12
        line["cpu_baseline"] = {"value": round(cpu_tflops, 5), "unit": "TFLOP/s", "cores": cpu["cores"],
                                "kind": "port", "sample": cpu["sample"],
                                "ms_per_step": round(cpu["seconds_per_step"] * 1e3, 1)}
    else:
        line["cpu_baseline"] = None
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
