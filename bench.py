#!/usr/bin/env python3
"""W4A16 decode-GEMV benchmark on one MI355X (BASELINE.json metric, config 2 shapes).

Workload ("step"): every quantized linear of one Llama-3-8B decode step at batch M (default 1) —
32 layers x {q 4096->4096, k 4096->1024, v 4096->1024, o 4096->4096, gate 4096->14336,
up 4096->14336, down 14336->4096} plus the int4 lm_head 4096->128256 — each an int4-g128 symmetric
(reference format) weight, bf16 activations, through libsqx_hip.so's sqx_int4_linear. Weights are
random N(0, 0.02) quantized on the GPU; 3.99 GB of distinct int4 weights per step keeps the 256 MB
Infinity Cache from serving them. The step is captured once in a HIP graph and replayed.

value = algorithmic HBM bytes per step / time per step, where a linear's bytes are
N*K/2 (codes) + 4*N*K/128 (fp32 scales) + 2*M*K (x) + 2*M*N (y).

roofline: the dominant kernel (the int4 linear instance, the only kernel in the step), with its
average launch duration measured by HIP events around each launch of an eager pass.
cpu_baseline: the reference's CPU path (torch dequantize + F.linear per call, restated in
oracle/torch_path.py) timed on this host's cores over a bounded sample of the same workload.
"""

from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "W4A16 GEMV HBM GB/s (% peak) at Llama-3-8B shapes; decode tok/s at B=1"
HBM_PEAK_GBS = 8000.0
LAYER_SHAPES = [  # (name, N = out_features, K = in_features)
    ("q", 4096, 4096),
    ("k", 1024, 4096),
    ("v", 1024, 4096),
    ("o", 4096, 4096),
    ("gate", 14336, 4096),
    ("up", 14336, 4096),
    ("down", 4096, 14336),
]
LM_HEAD = ("lm_head", 128256, 4096)
GROUP = 128


def algo_bytes(m: int, n: int, k: int) -> int:
    return n * k // 2 + 4 * n * (k // GROUP) + 2 * m * k + 2 * m * n


def log(*a) -> None:
    print(*a, file=sys.stderr, flush=True)


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--m", type=int, default=1, help="activation rows (decode batch)")
    ap.add_argument("--layers", type=int, default=32)
    ap.add_argument("--cpu-seconds", type=float, default=12.0, help="CPU-baseline sample budget")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--eager-passes", type=int, default=3, help="event-timed eager passes for the roofline")
    ap.add_argument("--splits", type=int, default=0, help="split-K override (0 = library default)")
    args = ap.parse_args()

    if args.gpus != 1:
        print(
            f"bench.py measures one GPU only (got --gpus {args.gpus}); this build does not shard across GPUs.",
            file=sys.stderr,
        )
        return 2

    import torch

    from scratch_llm_amd import _lib
    from scratch_llm_amd.quant import int4_group as q4

    if not torch.cuda.is_available():
        log("no ROCm device visible")
        return 1
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    lib = _lib.load()
    m = args.m

    # ------------------------------------------------------------------ weights (quantized on GPU)
    t_setup = time.perf_counter()
    gen = torch.Generator(device=dev)
    linears = []  # (name, N, K, Int4Tiled)
    cpu_sample = []  # layer 0's reference-format codes/scales for the CPU baseline
    for layer in range(args.layers):
        for name, n, k in LAYER_SHAPES:
            gen.manual_seed(1000 + 7 * layer + len(linears) % 7)
            w = (torch.randn(n, k, device=dev, generator=gen) * 0.02).to(torch.bfloat16)
            qc, sc = q4.quantize_groupwise_int4(w)
            del w
            linears.append((name, n, k, q4.tile_int4(qc, sc)))
            if layer == 0 and not args.no_cpu:
                cpu_sample.append((name, n, k, qc.cpu(), sc.cpu()))
            del qc, sc
    name, n, k = LM_HEAD
    gen.manual_seed(999)
    w = (torch.randn(n, k, device=dev, generator=gen) * 0.02).to(torch.bfloat16)
    qc, sc = q4.quantize_groupwise_int4(w)
    del w
    linears.append((name, n, k, q4.tile_int4(qc, sc)))
    del qc, sc
    torch.cuda.synchronize()
    log(f"setup: {len(linears)} int4 linears in {time.perf_counter() - t_setup:.1f}s")

    gen.manual_seed(2001)
    xs = {kk: torch.randn(m, kk, device=dev, generator=gen).to(torch.bfloat16) for kk in (4096, 14336)}
    ys = {}
    for _, n, _, _ in linears:
        ys.setdefault(n, torch.empty(m, n, device=dev, dtype=torch.bfloat16))
    ws_need = max(lib.sqx_int4_linear_workspace_bytes(m, n, k, args.splits) for _, n, k, _ in linears)
    ws = torch.zeros(max(ws_need, 256) // 4 + 64, device=dev, dtype=torch.int32)
    ws_bytes = ws.numel() * 4

    def launch_args(tw, n, k, stream_ptr):
        return (
            tw.wt.data_ptr(), tw.st.data_ptr(), None, _lib.DTYPE_F32, xs[k].data_ptr(), _lib.DTYPE_BF16,
            ys[n].data_ptr(), None, m, n, k, GROUP, args.splits, ws.data_ptr(), ws_bytes, stream_ptr,
        )

    fn = lib.sqx_int4_linear

    def run_step(stream_ptr: int, check: bool = False) -> None:
        for _, n, k, tw in linears:
            rc = fn(*launch_args(tw, n, k, stream_ptr))
            if check:
                _lib.check(rc, "sqx_int4_linear")

    step_bytes = sum(algo_bytes(m, n, k) for _, n, k, _ in linears)
    cur = torch.cuda.current_stream().cuda_stream
    run_step(cur, check=True)
    torch.cuda.synchronize()
    y_eager = {n: t.clone() for n, t in ys.items()}

    # ------------------------------------------------------------------ graph capture of one step
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        run_step(torch.cuda.current_stream().cuda_stream)
    for t in ys.values():
        t.zero_()
    graph.replay()
    torch.cuda.synchronize()
    graph_ok = all(torch.equal(ys[n], y_eager[n]) for n in ys)
    if not graph_ok:
        log("WARNING: graph replay differs from the eager step")

    # ------------------------------------------------------------------ timed region (graph replays)
    for _ in range(args.warmup):
        graph.replay()
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    ev0.record()
    for _ in range(args.steps):
        graph.replay()
    ev1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_per_step = ev0.elapsed_time(ev1) / args.steps
    value_gbs = step_bytes / (ms_per_step * 1e-3) / 1e9
    log(f"graph step: {ms_per_step * 1e3:.1f} us, {value_gbs:.0f} GB/s, wall {wall:.3f}s")

    # ------------------------------------------------------------------ per-launch events (roofline)
    per = {}
    tot_ms = 0.0
    tot_bytes = 0
    n_launch = 0
    for _ in range(args.eager_passes):
        pairs = []
        try:
            torch.cuda._sleep(200_000_000)  # keep the GPU busy while the pass is enqueued
        except Exception:  # pragma: no cover - spin kernel unavailable
            pass
        for name, n, k, tw in linears:
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            fn(*launch_args(tw, n, k, cur))
            b.record()
            pairs.append((name, n, k, a, b))
        torch.cuda.synchronize()
        for name, n, k, a, b in pairs:
            dt = a.elapsed_time(b)
            key = f"{k}->{n}"
            e = per.setdefault(key, {"ms": 0.0, "launches": 0, "bytes": 0})
            e["ms"] += dt
            e["launches"] += 1
            e["bytes"] += algo_bytes(m, n, k)
            tot_ms += dt
            tot_bytes += algo_bytes(m, n, k)
            n_launch += 1
    per_shape = {
        kk: {
            "us_per_launch": round(v["ms"] / v["launches"] * 1e3, 3),
            "gbs": round(v["bytes"] / (v["ms"] * 1e-3) / 1e9, 1),
            "frac_of_8tbs": round(v["bytes"] / (v["ms"] * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        }
        for kk, v in per.items()
    }
    avg_launch_s = tot_ms / n_launch * 1e-3
    bytes_per_launch = tot_bytes / n_launch
    achieved = bytes_per_launch / avg_launch_s / 1e9
    log("per-shape:", json.dumps(per_shape))

    # ------------------------------------------------------------------ measured copy bandwidth
    src = torch.empty(1 << 28, device=dev, dtype=torch.int32)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    c0, c1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    c0.record()
    for _ in range(10):
        dst.copy_(src)
    c1.record()
    torch.cuda.synchronize()
    copy_gbs = 2 * src.numel() * 4 * 10 / (c0.elapsed_time(c1) * 1e-3) / 1e9
    del src, dst

    # ------------------------------------------------------------------ CPU baseline
    cpu_baseline = None
    if not args.no_cpu:
        from oracle import torch_path

        threads = os.cpu_count() or 1
        torch.set_num_threads(threads)
        xc = {kk: xs[kk].cpu() for kk in xs}
        done_bytes = 0
        passes = 0
        c_start = time.perf_counter()
        while True:
            for name, n, k, qc, sc in cpu_sample:
                torch_path.w4a16_linear(xc[k], qc, sc, None, GROUP)
                done_bytes += algo_bytes(m, n, k)
            passes += 1
            if time.perf_counter() - c_start >= args.cpu_seconds:
                break
        c_el = time.perf_counter() - c_start
        cpu_baseline = {
            "value": round(done_bytes / c_el / 1e9, 3),
            "unit": "GB/s",
            "cores": torch.get_num_threads(),
            "kind": "port",
            "sample": (
                f"{passes} passes over layer 0's 7 int4 linears (M={m}, bf16 x), torch CPU dequantize + "
                f"F.linear per call (oracle/torch_path.py), {c_el:.1f}s on '{cpu_model()}', os.cpu_count()={threads}"
            ),
        }
        log(f"cpu baseline: {cpu_baseline['value']} GB/s")

    out = {
        "metric": METRIC,
        "value": round(value_gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": (
                "int4-g128 W4A16 decode GEMV over all linears of a Llama-3-8B decode step "
                f"({args.layers} layers x q,k,v,o,gate,up,down + lm_head), M={m}, HIP-graph replay"
            ),
            "m": m,
            "layers": args.layers,
            "group_size": GROUP,
            "launches_per_step": len(linears),
            "bytes_per_step": step_bytes,
            "splits": args.splits or "default",
        },
        "frac_of_hbm_peak": round(value_gbs / HBM_PEAK_GBS, 4),
        "frac_of_measured_copy": round(value_gbs / copy_gbs, 4),
        "measured_copy_gbs": round(copy_gbs, 1),
        "decode_linear_tok_s": round(1000.0 / ms_per_step, 1),
        "graph_matches_eager": graph_ok,
        "per_shape": per_shape,
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": None,
            "kernel": "sqx::int4_linear_kernel<ActBF16,128,false,false,1>",
            "avg_launch_us": round(avg_launch_s * 1e6, 3),
            "bytes_per_launch": round(bytes_per_launch),
        },
        "cpu_baseline": cpu_baseline,
    }
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
