#!/usr/bin/env python3
"""W4A16 decode-GEMV benchmark on one MI355X (BASELINE.json metric; config 2 shapes, config 5 layout).

Step: every quantized linear of one Llama-3-8B decode step at batch M (default 1), laid out as a
serving engine holds them: per layer a fused QKV projection 4096->6144 (q 4096 + k 1024 + v 1024
rows), o 4096->4096, a fused gate/up projection 4096->28672 and down 14336->4096; 32 layers plus
the lm_head 4096->128256. Every weight is int4 group-128 in the reference's symmetric format
(codes in [-8, 7], fp32 scale per group), random N(0, 0.02) quantized on the GPU, bf16
activations, through libsqx_hip.so's sqx_int4_linear. The step's 3.99 GB of distinct weights is
15x the 256 MB Infinity Cache, so every step streams from HBM. The step is captured once in a HIP
graph and replayed; `--layout unfused` times the seven separate projections per layer instead.

value = algorithmic HBM bytes per step / time per step; a linear's bytes are
N*K/2 (codes) + 4*N*K/128 (fp32 scales) + 2*M*K (x) + 2*M*N (y).

per_shape: each Llama-3-8B linear shape timed on its own (HIP events around each replay of a graph of
back-to-back launches on the launch stream; two untimed replays, then the median replay), rotating over >= 1 GB of distinct weight tiles (views into the
step's tiled weights: any 16-row-tile window of a tiled weight is a tiled weight).
roofline: the dominant kernel of the step, the int4 linear launch that takes the largest share of
the step (the fused gate/up projection), timed the same way; `traffic` is its HBM bytes per launch
from the rocprofv3 FETCH_SIZE / WRITE_SIZE runs of this benchmark recorded in
profiles/int4_linear_gate_up_traffic.md (scaled by the counters' reading of a 1 GiB copy), for M = 1.
cpu_baseline: the reference's CPU path (torch dequantize + F.linear per call, restated in
oracle/torch_path.py) over layer 0's seven projections, on this host's cores, for a bounded time.

decode (not part of `value`; the metric's "decode tok/s at B=1" is decode_tok_s_b1): BASELINE config 5,
the whole decode step of the Llama-3-8B-shaped model with every linear int4-g128
(scratch_llm_amd.decode: embedding, 32 x [RMSNorm, qkv, RoPE + attention over 2048 cached keys,
o, RMSNorm, gate/up, SiLU gate + down], final norm, lm_head, greedy pick), random weights and a
random-filled bf16 KV cache with every row at 2047 cached tokens, captured in one HIP graph and
replayed token after token. Per B: ms per step, tok/s (B / step time), HBM bytes per step (weights
+ KV) and the time share of each kind of launch (qkv, attention, o, gate_up, down, lm_head, other:
a graph of the step's own launches of that kind, same kernels and arguments, timed alone, over the
step time).

fp8_w8a8 (not part of `value`): the FP8 E4M3 W8A8 linear (per-token activations, per-channel weights)
at Llama-3-8B decode shapes, M = 1 and 16, captured graphs over >= 1 GB of rotating weights, next
to hipBLASLt's rowwise torch._scaled_mm (the reference's fp8_linear on ROCm) on the same operands,
with each one's error against the float64 oracle in units of the reference's derived bound.

baseline_configs (not part of `value`): every case BASELINE configs 1-4 name (int8 weight-only
4096x4096 at M = 1, 16; int4 g128 asymmetric at the four Llama-3-8B shapes, M = 1, 4, 8; AWQ at the
same shapes, M = 64, 512, 2048; MXFP4 at the Llama-3-70B MLP shapes, M = 1 and 128, bf16 and MXFP4
activations), each in GB/s or TFLOP/s against its roofline.

prefill (not part of `value`): the prefill GEMMs at their BASELINE configs, captured graphs of
back-to-back calls on inputs already in HBM: config 4's MXFP4 x MXFP4 GEMM at M = 4096 (both
shapes) against the 10.1 PF dense fp4 MFMA peak, config 4's MXFP4-weight x bf16 GEMM at M = 4096
and config 3's AWQ int4 GEMM at M = 2048 against the 2.5 PF bf16 peak.
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
GROUP = 128
D_MODEL, D_FF, VOCAB = 4096, 14336, 128256
# Llama-3-8B projections (name, N = out_features, K = in_features)
UNFUSED = [("q", 4096, 4096), ("k", 1024, 4096), ("v", 1024, 4096), ("o", 4096, 4096),
           ("gate", 14336, 4096), ("up", 14336, 4096), ("down", 4096, 14336)]
FUSED = [("qkv", 6144, 4096), ("o", 4096, 4096), ("gate_up", 28672, 4096), ("down", 4096, 14336)]
LM_HEAD = ("lm_head", VOCAB, D_MODEL)


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
    ap.add_argument("--layout", choices=("fused", "unfused"), default="fused")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-shapes", action="store_true", help="skip the per-shape timing")
    ap.add_argument("--kslices", type=int, default=0, help="waves per 16-row tile (0 = library default)")
    ap.add_argument("--no-prefill", action="store_true", help="skip the prefill GEMM measurements")
    ap.add_argument("--no-decode", action="store_true", help="skip the config-5 decode-step measurement")
    ap.add_argument("--decode-batches", default="1,2,8,32,64", help="batch sizes of the decode-step measurement")
    ap.add_argument("--decode-fp8kv-batches", default="32,64", help="batch sizes also timed with the FP8 KV cache")
    ap.add_argument("--no-fp8", action="store_true", help="skip the FP8 W8A8 linear measurement")
    ap.add_argument("--no-configs", action="store_true", help="skip the per-config cases of BASELINE configs 1-4")
    ap.add_argument("--config-ids", default="1,2,3,4", help="which of BASELINE configs 1-4 the per-config cases run")
    ap.add_argument("--rotate-gb", type=float, default=1.1,
                    help="bytes of rotating weight copies per per-config case (2 copies at least; 0 for counter runs)")
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
    seed = 1000

    def make(n: int, k: int):
        nonlocal seed
        gen.manual_seed(seed)
        seed += 1
        w = (torch.randn(n, k, device=dev, generator=gen) * 0.02).to(torch.bfloat16)
        qc, sc = q4.quantize_groupwise_int4(w)
        del w
        return qc, sc

    shapes = FUSED if args.layout == "fused" else UNFUSED
    linears = []  # (name, N, K, Int4Tiled)
    cpu_sample = []  # layer 0's seven projections in the reference format, for the CPU baseline
    for layer in range(args.layers):
        for name, n, k in shapes:
            qc, sc = make(n, k)
            linears.append((name, n, k, q4.tile_int4(qc, sc)))
            if layer == 0 and not args.no_cpu:
                if args.layout == "fused":  # the fused rows are the seven projections stacked
                    parts = {"qkv": (("q", 4096), ("k", 1024), ("v", 1024)), "gate_up": (("gate", 14336), ("up", 14336))}
                    r0 = 0
                    for pn, pr in parts.get(name, ((name, n),)):
                        cpu_sample.append((pn, pr, k, qc[r0:r0 + pr].cpu(), sc[r0:r0 + pr].cpu()))
                        r0 += pr
                else:
                    cpu_sample.append((name, n, k, qc.cpu(), sc.cpu()))
            del qc, sc
    qc, sc = make(LM_HEAD[1], LM_HEAD[2])
    linears.append((LM_HEAD[0], LM_HEAD[1], LM_HEAD[2], q4.tile_int4(qc, sc)))
    del qc, sc
    torch.cuda.synchronize()
    log(f"setup: {len(linears)} int4 linears ({args.layout}) in {time.perf_counter() - t_setup:.1f}s")

    gen.manual_seed(2001)
    xs = {kk: torch.randn(m, kk, device=dev, generator=gen).to(torch.bfloat16) for kk in (D_MODEL, D_FF)}
    ys = {}
    for n in [n for _, n, _, _ in linears] + [n for _, n, _ in UNFUSED + FUSED]:
        ys.setdefault(n, torch.empty(m, n, device=dev, dtype=torch.bfloat16))
    fn = lib.sqx_int4_linear

    def launch(wt_ptr, st_ptr, n, k, stream_ptr):
        return fn(wt_ptr, st_ptr, None, _lib.DTYPE_F32, xs[k].data_ptr(), _lib.DTYPE_BF16, ys[n].data_ptr(), None,
                  m, n, k, GROUP, args.kslices, stream_ptr)

    def run_step(stream_ptr: int, check: bool = False) -> None:
        for _, n, k, tw in linears:
            rc = launch(tw.wt.data_ptr(), tw.st.data_ptr(), n, k, stream_ptr)
            if check:
                _lib.check(rc, "sqx_int4_linear")

    step_bytes = sum(algo_bytes(m, n, k) for _, n, k, _ in linears)
    run_step(torch.cuda.current_stream().cuda_stream, check=True)
    torch.cuda.synchronize()
    written = {n for _, n, _, _ in linears}
    y_eager = {n: ys[n].clone() for n in written}

    # ------------------------------------------------------------------ graph capture of one step
    cap = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=cap):
        run_step(cap.cuda_stream)
    for t in ys.values():
        t.zero_()
    graph_mismatch = {}
    for r in range(3):  # replays with eager work and synchronisations between them
        graph.replay()
        torch.cuda.synchronize()
        for n in written:
            bad = int((ys[n] != y_eager[n]).sum())
            if bad:
                graph_mismatch[f"replay{r} N={n}"] = bad
        for t in ys.values():
            t.zero_()
        torch.cuda.synchronize()
    graph_ok = not graph_mismatch
    if not graph_ok:
        log("WARNING: graph replay differs from the eager step:", graph_mismatch)

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

    # ------------------------------------------------------------------ per-shape kernel timing
    def shape_time(n: int, k: int, reps: int = 5):
        """us per launch of an (n, k) linear, over windows of the step's tiled weights with matching k."""
        kb = -(-k // 128)
        tiles = -(-n // 16)
        tile_b, tile_p = kb * 1024, kb * 16
        pool = []
        for _, pn, pk, tw in linears:
            if pk != k:
                continue
            for t0 in range(0, -(-pn // 16) - tiles + 1, tiles):
                pool.append((tw.wt[t0 * tile_b:].data_ptr(), tw.st[t0 * tile_p:].data_ptr()))
        need = max(8, min(len(pool), -(-(1 << 30) // (tiles * tile_b))))
        step = max(1, len(pool) // need)
        pool = pool[::step][:need]
        s = torch.cuda.Stream()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            for wp, sp in pool:
                launch(wp, sp, n, k, s.cuda_stream)
        # two untimed replays, then the median of per-replay times: the first replays of a fresh
        # graph run several percent slow
        for _ in range(2):
            g.replay()
        torch.cuda.synchronize()
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(reps + 1)]
        with torch.cuda.stream(s):
            ev[0].record(s)
            for i in range(reps):
                g.replay()
                ev[i + 1].record(s)
        torch.cuda.synchronize()
        times = sorted(ev[i].elapsed_time(ev[i + 1]) for i in range(reps))
        us = times[reps // 2] * 1e3 / len(pool)
        return us, len(pool) * tiles * tile_b

    per_shape = {}
    if not args.no_shapes:
        for name, n, k in UNFUSED + FUSED[:1] + FUSED[2:3] + [LM_HEAD]:
            key = f"{k}->{n}"
            if key in per_shape:
                continue
            us, pool_b = shape_time(n, k)
            gbs = algo_bytes(m, n, k) / us / 1e3
            per_shape[key] = {"name": name, "us": round(us, 3), "gbs": round(gbs, 1),
                              "frac_of_8tbs": round(gbs / HBM_PEAK_GBS, 4), "rotated_mb": pool_b >> 20}
        log("per-shape:", json.dumps(per_shape))

    share_launches = [name for name, _, _, _ in linears]
    # dominant kernel: the launch shape with the largest share of the step
    share = {}
    for name, n, k, _ in linears:
        share[(name, n, k)] = share.get((name, n, k), 0) + 1
    dom = max(share, key=lambda s: share[s] * algo_bytes(m, s[1], s[2]))
    dom_us, _ = shape_time(dom[1], dom[2], reps=9)
    dom_bytes = algo_bytes(m, dom[1], dom[2])
    achieved = dom_bytes / dom_us / 1e3

    # ------------------------------------------------------------------ library bandwidths for reference
    # torch's sum over 1 GiB (read-only) and copy_ of 1 GiB (both directions counted); neither is a
    # roof (the step's own GEMVs outrun the sum), so `value` is compared with 8 TB/s only
    src = torch.ones(1 << 28, device=dev, dtype=torch.float32)
    dst = torch.empty_like(src)

    def lib_gbs(fn, nbytes):
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        c0, c1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        c0.record()
        for _ in range(10):
            fn()
        c1.record()
        torch.cuda.synchronize()
        return nbytes * 10 / (c0.elapsed_time(c1) * 1e-3) / 1e9

    read_gbs = lib_gbs(lambda: src.sum(), src.numel() * 4)
    copy_gbs = lib_gbs(lambda: dst.copy_(src), 2 * src.numel() * 4)
    del src, dst

    # ------------------------------------------------------------------ CPU baseline
    cpu_baseline = None
    if not args.no_cpu:
        cpu_baseline = cpu_baselines(dev, cpu_sample, xs, m, per_shape)
        log(f"cpu baseline: {cpu_baseline['value']} GB/s")

    # ------------------------------------------------------------------ prefill GEMMs
    prefill = None
    if not args.no_prefill:
        prefill = prefill_gemms(dev)
        log("prefill:", json.dumps(prefill))

    fp8 = None
    if not args.no_fp8:
        fp8 = fp8_linears(dev)
        log("fp8:", json.dumps(fp8))

    configs = None
    if not args.no_configs:
        configs = baseline_configs(dev, [int(c) for c in args.config_ids.split(",") if c], args.rotate_gb)
        log("configs:", json.dumps(configs))

    decode = None
    if not args.no_decode:
        del linears, cpu_sample
        torch.cuda.empty_cache()
        decode = decode_steps(dev, [int(b) for b in args.decode_batches.split(",") if b],
                              [int(b) for b in args.decode_fp8kv_batches.split(",") if b])
        log("decode:", json.dumps(decode))

    launches = len(share_launches)
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
                f"int4-g128 W4A16 decode linears of a Llama-3-8B step ({args.layers} layers x "
                + ("qkv,o,gate_up,down" if args.layout == "fused" else "q,k,v,o,gate,up,down")
                + f" + lm_head), M={m}, HIP-graph replay"
            ),
            "m": m,
            "layers": args.layers,
            "layout": args.layout,
            "group_size": GROUP,
            "launches_per_step": launches,
            "bytes_per_step": step_bytes,
            "k_slices": args.kslices or "default",
        },
        "frac_of_hbm_peak": round(value_gbs / HBM_PEAK_GBS, 4),
        "torch_sum_read_gbs": round(read_gbs, 1),
        "torch_copy_gbs": round(copy_gbs, 1),
        "linear_only_tok_s": round(1000.0 / ms_per_step * m, 1),
        "graph_matches_eager": graph_ok,
        "graph_mismatch": graph_mismatch or None,
        "decode_tok_s_b1": None if decode is None or "B=1" not in decode else decode["B=1"]["tok_s"],
        "per_shape": per_shape,
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": measured_traffic(dom, m),
            "kernel": f"gemv_kernel<ActBF16, WInt4<128,false,false>> (sqx_int4_linear) {dom[0]} {dom[2]}->{dom[1]}",
            "avg_launch_us": round(dom_us, 3),
            "bytes_per_launch": dom_bytes,
        },
        "cpu_baseline": cpu_baseline,
        "decode": decode,
        "fp8_w8a8": fp8,
        "prefill": prefill,
        "baseline_configs": configs,
    }
    print(json.dumps(out), flush=True)
    return 0


def _host_stats(fn, warmup: int = 20, iters: int = 50) -> dict:
    """Host-clock timing of ``fn`` (src/scratch_llm/bench/harness.py:52-91's host path): ``warmup``
    untimed calls, then ``iters`` calls timed one by one with time.perf_counter; median and the
    p20-p80 band in ms (bench/_harness.py:51-59)."""
    for _ in range(warmup):
        fn()
    ts = []
    for _ in range(iters):
        t0 = time.perf_counter()
        fn()
        ts.append((time.perf_counter() - t0) * 1e3)
    ts.sort()

    def q(p: float) -> float:
        return ts[min(len(ts) - 1, int(round(p * (len(ts) - 1))))]

    med = q(0.5)
    return {"median_ms": round(med, 4), "p20_ms": round(q(0.2), 4), "p80_ms": round(q(0.8), 4),
            "spread_pct": round(100.0 * (q(0.8) - q(0.2)) / med, 2), "warmup": warmup, "iters": iters}


def cpu_baselines(dev, cpu_sample, xs, m: int, per_shape: dict) -> dict:
    """The reference's CPU path (torch dequantize, then F.linear; oracle/torch_path.py) on this host's
    cores in two variants: (i) dequantizes on every call (what the reference does), (ii) keeps the
    dequantized weight (a CPU upper bound); each timed over 50 calls
    after 20 warm-ups on the host clock, median and p20-p80. Legs: config 2's int4 format over layer
    0's seven projections at the bench's M (the headline leg, ``value``), config 1's int8 4096 x 4096
    at M = 1 and 16, config 3's AWQ 4096 x 4096 at M = 64, and config 4's MXFP4 8192 -> 28672 at
    M = 1 on its first 2048 output rows (a bounded sample of the shape). Weights are quantized on
    the GPU by this library (bit-exact with the reference) and copied to the host."""
    import torch

    from oracle import torch_path
    from scratch_llm_amd.quant import awq, int8 as q8, nvfp4_mxfp4 as f4

    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    t_all = time.perf_counter()
    legs = {}

    def leg(name, byts, call_i, call_ii, extra=None):
        ri, rii = _host_stats(call_i), _host_stats(call_ii)
        legs[name] = {"bytes": byts, "variant_i": ri, "variant_ii": rii,
                      "gbs_i": round(byts / (ri["median_ms"] * 1e-3) / 1e9, 3),
                      "gbs_ii": round(byts / (rii["median_ms"] * 1e-3) / 1e9, 3), **(extra or {})}

    # config 2 / headline: layer 0's seven int4 projections, dequantize + F.linear per call
    xc = {kk: xs[kk].cpu() for kk in xs}
    head_bytes = sum(algo_bytes(m, n, k) for _, n, k, _, _ in cpu_sample)
    cached = [(k, torch_path.dequantize_groupwise_int4(qc, sc).to(torch.bfloat16)) for _, _, k, qc, sc in cpu_sample]

    def int4_i():
        for _, _, k, qc, sc in cpu_sample:
            torch_path.w4a16_linear(xc[k], qc, sc, None, GROUP)

    def int4_ii():
        for k, w in cached:
            torch.nn.functional.linear(xc[k], w)

    shape_us = [per_shape.get(f"{k}->{n}", {}).get("us") for _, n, k, _, _ in cpu_sample]
    gpu_us = None if None in shape_us else round(sum(shape_us), 3)
    leg(f"int4_g128 layer0 q,k,v,o,gate,up,down M={m}", head_bytes, int4_i, int4_ii,
        {"gpu_us": gpu_us})
    hl = legs[f"int4_g128 layer0 q,k,v,o,gate,up,down M={m}"]
    if gpu_us:
        hl["speedup_i"] = round(hl["variant_i"]["median_ms"] * 1e3 / gpu_us, 1)
        hl["speedup_ii"] = round(hl["variant_ii"]["median_ms"] * 1e3 / gpu_us, 1)
    del cached
    g = torch.Generator(device=dev).manual_seed(3001)
    # config 1: int8 weight-only 4096 x 4096
    w = (torch.randn(4096, 4096, generator=g, device=dev) * 0.02).to(torch.bfloat16)
    q, s = q8.quantize_symmetric(w.float(), axis=0)
    qc, sc = q.cpu(), s.cpu()
    wdq = (qc.float() * sc.view(-1, 1)).to(torch.bfloat16)
    for mm in (1, 16):
        x = torch.randn(mm, 4096, generator=g, device=dev).to(torch.bfloat16).cpu()
        leg(f"int8 4096->4096 M={mm}", 4096 * 4096 + 4 * 4096 + 4 * mm * 4096,
            lambda: torch_path.int8_weight_linear(x, qc, sc), lambda: torch.nn.functional.linear(x, wdq))
    # config 3: AWQ 4096 x 4096, M = 64, 1% of channels x20
    w = torch.randn(4096, 4096, generator=g, device=dev) * 0.02
    cs = torch.exp(torch.empty(4096, device=dev).uniform_(-0.6931, 0.6931, generator=g))
    quant = awq.quantize_awq_int4(w, chan_scale=cs)
    aq, ags, acs = quant.q.cpu(), quant.group_scales.cpu(), quant.chan_scale.cpu()
    x = torch.randn(64, 4096, generator=g, device=dev)
    x[:, torch.randperm(4096, generator=torch.Generator().manual_seed(4096))[:40].to(dev)] *= 20.0
    x = x.to(torch.bfloat16).cpu()
    weff = (torch_path.dequantize_groupwise_int4(aq, ags) / acs.view(1, -1)).to(torch.bfloat16)
    leg("awq_int4_g128 4096->4096 M=64", algo_bytes(64, 4096, 4096), lambda: torch_path.awq_linear(x, aq, ags, acs),
        lambda: torch.nn.functional.linear(x, weff), {"flops": 2 * 64 * 4096 * 4096})
    # config 4: MXFP4 8192 -> 28672 at M = 1, first 2048 rows
    rows, k = 2048, 8192
    w = torch.randn(rows, k, generator=g, device=dev) * 0.02
    packed, e8 = f4.mxfp4_pack_weight(f4.mxfp4_quantize(w, 32))
    pc, ec = packed.cpu(), e8.cpu()
    x = torch.randn(1, k, generator=g, device=dev).to(torch.bfloat16).cpu()
    wmx = torch_path.mxfp4_dequantize_packed(pc, ec, rows, k).to(torch.bfloat16)
    leg(f"mxfp4 8192->28672 M=1 (rows 0..{rows - 1})", rows * k // 2 + rows * k // 32 + 2 * k + 2 * rows,
        lambda: torch_path.mxfp4_linear(x, pc, ec, rows, k), lambda: torch.nn.functional.linear(x, wmx))
    del w, q, s, quant
    torch.cuda.empty_cache()
    head = legs[f"int4_g128 layer0 q,k,v,o,gate,up,down M={m}"]
    return {
        "value": head["gbs_i"],
        "unit": "GB/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": (
            f"layer 0's seven int4-g128 projections at M={m} (bf16 x): torch CPU dequantize + F.linear per call "
            f"(oracle/torch_path.py), median of 50 calls after 20 warm-ups; CPU '{cpu_model()}', "
            f"os.cpu_count()={threads}"
        ),
        "p20_gbs": round(head["bytes"] / (head["variant_i"]["p80_ms"] * 1e-3) / 1e9, 3),
        "p80_gbs": round(head["bytes"] / (head["variant_i"]["p20_ms"] * 1e-3) / 1e9, 3),
        "variant_ii_gbs": head["gbs_ii"],
        "cpu_model": cpu_model(),
        "os_cpu_count": threads,
        "legs": legs,
        "wall_s": round(time.perf_counter() - t_all, 1),
    }


def measured_traffic(dom, m: int):
    """HBM bytes per launch of the dominant kernel from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE
    runs of this benchmark (profiles/int4_linear_gate_up_traffic.md), when the shape and M match."""
    path = os.path.join(ROOT, "profiles", "int4_linear_gate_up_traffic.md")
    try:
        text = open(path).read()
        blk = json.loads(text.split("```json", 1)[1].split("```", 1)[0])
    except (OSError, IndexError, ValueError):
        return None
    if blk.get("shape") != f"{dom[2]}->{dom[1]}" or blk.get("m") != m:
        return None
    return int(blk["traffic_bytes_per_launch"])


def _graph_call_us(fn, calls: int = 4, reps: int = 5) -> float:
    """us per call of ``fn`` (device work on the current stream, any host-side allocation graph-safe),
    captured ``calls`` times back to back in one HIP graph and replayed ``reps`` times between HIP
    events: GPU time without the host's launch gaps. ``fn`` may be a list of callables (one per
    rotating weight copy), captured once each in order."""
    import torch

    fns = list(fn) if isinstance(fn, (list, tuple)) else [fn] * calls
    calls = len(fns)
    cs = torch.cuda.Stream()
    cs.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(cs):
        for f in dict.fromkeys(fns):
            f()  # warm any lazily built state outside the capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=cs):
        for f in fns:
            f()
    graph.replay()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(reps):
        graph.replay()
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) * 1e3 / (reps * calls)


def decode_steps(dev, batches: list[int], fp8_batches: list[int], steps: int = 20, warmup: int = 3) -> dict:
    """BASELINE config 5 (module docstring): the captured decode step per batch size; for the batch
    sizes in ``fp8_batches`` also with the per-head FP8 KV cache (entries ``B=..,kv=fp8``)."""
    import torch

    from scratch_llm_amd import _lib
    from scratch_llm_amd.decode import LLAMA3_8B, Int4DecodeLM

    cfg = LLAMA3_8B
    t0 = time.perf_counter()
    model = Int4DecodeLM.random_init(cfg, dev, seed=1005)
    torch.cuda.synchronize()
    log(f"decode model: {model.weight_bytes() / 1e9:.3f} GB of int4 weights in {time.perf_counter() - t0:.1f}s")
    ctx = cfg.context_length
    g = torch.Generator(device=dev).manual_seed(2005)

    def timed(graph, reps):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(reps):
            graph.replay()
        b.record()
        torch.cuda.synchronize()
        return a.elapsed_time(b) / reps

    res = {}
    runs = [(B, "bf16") for B in batches] + [(B, "fp8") for B in fp8_batches]
    for B, kvd in runs:
        st = model.new_state(B, ctx, kv_dtype=kvd)
        if kvd == "bf16":
            st.k.normal_(generator=g)
            st.v.normal_(generator=g)
        else:  # valid E4M3 codes (no NaN encodings) at a fixed per-head scale
            for li in range(cfg.n_layers):
                st.k[li].random_(0, 0x7F, generator=g)
                st.v[li].random_(0, 0x7F, generator=g)
            st.k_scale.fill_(0.01)
            st.v_scale.fill_(0.01)
        st.set_lengths([ctx - 1] * B)
        st.set_tokens(torch.randint(0, cfg.vocab_size, (B,), generator=torch.Generator().manual_seed(B)), cfg.vocab_size)
        model.step(st)
        torch.cuda.synchronize()
        st.set_lengths([ctx - 1] * B)  # every timed step attends 2048 keys (the full slot's last row is rewritten)
        graph = model.capture(st)
        for _ in range(warmup):
            graph.replay()
        torch.cuda.synchronize()
        ms = timed(graph, steps)
        del graph
        kv = 2 * cfg.n_layers * B * cfg.n_kv_heads * ctx * cfg.head_dim * (2 if kvd == "bf16" else 1)
        byts = model.weight_bytes() + kv
        key = f"B={B}" if kvd == "bf16" else f"B={B},kv=fp8"
        res[key] = {
            "ms_per_step": round(ms, 4),
            "tok_s": round(B / (ms * 1e-3), 1),
            "hbm_bytes_per_step": byts,
            "gbs": round(byts / (ms * 1e-3) / 1e9, 1),
            "frac_of_hbm_peak": round(byts / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        }
        log(f"decode B={B} kv={kvd}: {ms:.3f} ms/step, {B / (ms * 1e-3):.1f} tok/s")
        if kvd != "bf16":
            del st
            torch.cuda.empty_cache()
            continue
        # time share of each kind of launch: the step's own launches of that kind (Int4DecodeLM.step's
        # ``only``: same kernels, same arguments), captured and timed alone
        s_parts = {}
        for name in model.STEP_KINDS:
            cs = torch.cuda.Stream()
            gk = torch.cuda.CUDAGraph()
            with torch.cuda.graph(gk, stream=cs):
                model.step(st, only=name)
            gk.replay()
            torch.cuda.synchronize()
            s_parts[name] = timed(gk, 5)
            del gk
        res[key]["share"] = {k: round(v / ms, 4) for k, v in s_parts.items()}
        res[key]["linears_ms"] = round(sum(v for k, v in s_parts.items() if k not in ("attention", "other")), 4)
        del st
        torch.cuda.empty_cache()
    del model
    torch.cuda.empty_cache()
    return res


def _graph_us(launch_all, reps: int = 5) -> float:
    """us per launch of a captured sequence of launches (launch_all(stream) issues them and returns the
    count), replayed ``reps`` times between HIP events."""
    import torch

    cs = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=cs):
        n = launch_all(cs.cuda_stream)
    graph.replay()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(reps):
        graph.replay()
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) * 1e3 / (reps * n)


def fp8_linears(dev) -> dict:
    """FP8 E4M3 W8A8 linears (fp8_weights.py semantics) at the Llama-3-8B decode shapes: the library's
    sqx_fp8_linear (per-token activation quantize + exact-product GEMV, one weight pass), and
    hipBLASLt's rowwise torch._scaled_mm (the reference's fp8_linear path on ROCm) on the same codes
    and scales, each timed as a captured graph of back-to-back launches over >= 1 GB of weights, with
    the max error of each against the float64 oracle in units of the reference's derived bound
    (|ref| eps_bf16 / 2 + sqrt(K) eps_f32 sum|x w|)."""
    import math

    import torch

    from scratch_llm_amd import _lib
    from scratch_llm_amd.quant import fp8_weights as f8

    lib = _lib.load()
    res = {}
    g = torch.Generator(device=dev).manual_seed(1006)
    for n, k in ((4096, 4096), (28672, 4096), (4096, 14336)):
        copies = max(2, min(24, int(1.2e9 // (n * k))))
        ws = []
        for _ in range(copies):
            w = (torch.randn(n, k, generator=g, device=dev) * 0.02).to(torch.bfloat16)
            codes, scale = f8.quantize_per_channel(w)
            ws.append((codes, scale, f8.tile_fp8(codes, scale)))
            del w
        for m in (1, 16):
            x = torch.randn(m, k, generator=g, device=dev).to(torch.bfloat16)
            y = torch.empty(m, n, dtype=torch.bfloat16, device=dev)
            wsp = torch.empty(int(lib.sqx_fp8_linear_workspace_bytes(m, n, k)) // 4 + 4, dtype=torch.float32, device=dev)

            def ours(stream):
                for _, _, tw in ws:
                    lib.sqx_fp8_linear(tw.wt.data_ptr(), tw.scale.data_ptr(), x.data_ptr(), _lib.DTYPE_BF16, y.data_ptr(),
                                       _lib.DTYPE_BF16, None, m, n, k, 0, wsp.data_ptr(), wsp.numel() * 4, stream)
                return copies

            us = _graph_us(ours)
            byts = n * k + 4 * n + 2 * m * k + 2 * m * n
            entry = {"us": round(us, 2), "gbs": round(byts / us / 1e3, 1),
                     "frac_of_hbm_peak": round(byts / us / 1e3 / HBM_PEAK_GBS, 4)}
            codes, scale, tw = ws[0]
            xq, xs = f8.quantize_per_token(x)
            ref = (xq.double() * xs.double()) @ (codes.double() * scale.double()).t()
            mag = (xq.double() * xs.double()).abs() @ (codes.double() * scale.double()).abs().t()
            bound = ref.abs() * 2.0**-8 + mag * math.sqrt(k) * 2.0**-23
            entry["err_over_bound"] = round(float(((f8.fp8_linear_tiled(x, tw).double() - ref).abs() / bound).max()), 3)
            try:
                def theirs(stream):
                    for c, s_, _ in ws:
                        torch._scaled_mm(xq, c.t(), scale_a=xs, scale_b=s_.t(), out_dtype=torch.bfloat16)
                    return copies

                entry["hipblaslt_scaled_mm_us"] = round(_graph_us(theirs), 2)
                out = torch._scaled_mm(xq, codes.t(), scale_a=xs, scale_b=scale.t(), out_dtype=torch.bfloat16)
                out = (out[0] if isinstance(out, tuple) else out).double()
                entry["hipblaslt_err_over_bound"] = round(float(((out - ref).abs() / bound).max()), 3)
            except Exception as e:  # noqa: BLE001 - the comparison is informational
                entry["hipblaslt_scaled_mm_us"] = f"unavailable: {type(e).__name__}: {str(e)[:80]}"
            res[f"{k}->{n} M={m}"] = entry
        del ws
        torch.cuda.empty_cache()
    return res


def prefill_gemms(dev) -> dict:
    """The prefill GEMMs at BASELINE configs 3 and 4 (module docstring)."""
    import torch

    from scratch_llm_amd.quant import awq, nvfp4_mxfp4 as f4

    FP4_PEAK, BF16_PEAK = 10.1e15, 2.5e15
    res = {}
    g = torch.Generator(device=dev).manual_seed(1004)
    for n, k in ((28672, 8192), (8192, 28672)):
        m = 4096
        w = torch.randn(n, k, generator=g, device=dev) * 0.02
        tw = f4.tile_fp4(f4.mxfp4_quantize(w, 32))
        del w
        x = torch.randn(m, k, generator=g, device=dev).to(torch.bfloat16)
        xq = f4.mxfp4_quantize_tiled(x)
        us = _graph_call_us(lambda: f4.mxfp4_gemm(xq, tw))
        fl = 2.0 * m * n * k
        res[f"mxfp4_x_mxfp4 {k}->{n} M={m}"] = {
            "us": round(us, 1), "tflops": round(fl / us / 1e6, 1), "frac_of_fp4_peak": round(fl / us * 1e6 / FP4_PEAK, 4),
            "quantize_x_us": round(_graph_call_us(lambda: f4.mxfp4_quantize_tiled(x)), 1)}
        if n == 28672:
            us = _graph_call_us(lambda: f4.fp4_linear_tiled(x, tw))
            res[f"mxfp4_w_bf16_x {k}->{n} M={m}"] = {
                "us": round(us, 1), "tflops": round(fl / us / 1e6, 1),
                "frac_of_bf16_peak": round(fl / us * 1e6 / BF16_PEAK, 4)}
        del tw, x, xq
        torch.cuda.empty_cache()
    n, k, m = 14336, 4096, 2048
    w = torch.randn(n, k, generator=g, device=dev) * 0.02
    s = torch.exp(torch.empty(k, device=dev).uniform_(-0.6931, 0.6931, generator=g))
    quant = awq.quantize_awq_int4(w, chan_scale=s)
    x = torch.randn(m, k, generator=g, device=dev)
    x[:, torch.randperm(k, generator=torch.Generator().manual_seed(k))[: k // 100].to(dev)] *= 20.0
    x = x.to(torch.bfloat16)
    us = _graph_call_us(lambda: awq.awq_linear(x, quant))
    fl = 2.0 * m * n * k
    res[f"awq_int4_g128 {k}->{n} M={m}"] = {
        "us": round(us, 1), "tflops": round(fl / us / 1e6, 1), "frac_of_bf16_peak": round(fl / us * 1e6 / BF16_PEAK, 4)}
    return res


def baseline_configs(dev, ids=(1, 2, 3, 4), rotate_gb: float = 1.1) -> dict:
    """Every case of BASELINE.json's configs 1-4 on one GPU (config 5 is ``decode``; config 4 at M = 4096
    and config 3's M = 2048 on 4096->14336 are also in ``prefill``). Every case is a captured graph of
    back-to-back calls, each on the next of >= 1.1 GB of rotating weight copies (more than four times
    the 256 MB Infinity Cache, so the weights come from HBM): memory-bound cases (M <= 16, the MXFP4
    GEMV at M = 1) reported in GB/s of algorithmic bytes, GEMMs in TFLOP/s against the dtype's dense
    peak. Weights ~N(0, 0.02), activations bf16 ~N(0, 1) as the configs state; config 3's activation
    scale ~log-uniform[0.5, 2] and 1% of channels x20."""
    import torch

    from scratch_llm_amd import _lib
    from scratch_llm_amd.quant import awq, int4_group as i4, int8 as q8, nvfp4_mxfp4 as f4

    lib = _lib.load()
    BF16_PEAK, FP4_PEAK = 2.5e15, 10.1e15
    g = torch.Generator(device=dev).manual_seed(1007)
    res = {"config1_int8_weight_only": {}, "config2_int4_g128_asym": {}, "config3_awq_int4_g128": {},
           "config4_mxfp4": {}}

    def rotating(n, k, make, per_weight_bytes):
        copies = max(2, min(1024, -(-int(rotate_gb * 1e9) // per_weight_bytes)))
        return [make(torch.randn(n, k, generator=g, device=dev) * 0.02) for _ in range(copies)]

    def gbs_entry(us, byts):
        return {"us": round(us, 2), "gbs": round(byts / us / 1e3, 1),
                "frac_of_hbm_peak": round(byts / us / 1e3 / HBM_PEAK_GBS, 4)}

    # config 1: int8 weight-only 4096x4096, per-output-channel symmetric, M in {1, 16}
    if 1 in ids:
        n = k = 4096
        tws = rotating(n, k, lambda w: q8.tile_int8(*q8.quantize_symmetric(w, axis=0)), n * k)
        for m in (1, 16):
            x = torch.randn(m, k, generator=g, device=dev).to(torch.bfloat16)
            y = torch.empty(m, n, dtype=torch.bfloat16, device=dev)

            def run(stream):
                for tw in tws:
                    lib.sqx_int8_linear(tw.wt.data_ptr(), tw.scale.data_ptr(), x.data_ptr(), _lib.DTYPE_BF16, y.data_ptr(),
                                        None, m, n, k, 0, stream)
                return len(tws)

            res["config1_int8_weight_only"][f"{k}->{n} M={m}"] = gbs_entry(_graph_us(run), n * k + 4 * n + 2 * m * k + 2 * m * n)
        del tws
        torch.cuda.empty_cache()

    # config 2: int4 g128 asymmetric (uint4 codes, bf16 scale and zero per group), M in {1, 4, 8}
    if 2 in ids:
        for n, k in ((4096, 4096), (1024, 4096), (14336, 4096), (4096, 14336)):
            def make(w):
                q, s_, z = i4.quantize_groupwise_uint4_asym(w, 128, torch.bfloat16)
                return i4.tile_int4(q, s_, z, 128)

            tws = rotating(n, k, make, n * k // 2)
            for m in (1, 4, 8):
                x = torch.randn(m, k, generator=g, device=dev).to(torch.bfloat16)
                y = torch.empty(m, n, dtype=torch.bfloat16, device=dev)
                # what w4a16_linear runs (int4_linear_tiled): the GEMV at one row, the library's choice
                # among the GEMV and the row-tiled kernels (K split into a workspace) for 2..64 rows
                nb = int(lib.sqx_int4_skinny_workspace_bytes(m, n, k, 0))
                ws = torch.empty(max(nb, 16), dtype=torch.uint8, device=dev)

                def run(stream):
                    for tw in tws:
                        if m == 1:
                            lib.sqx_int4_linear(tw.wt.data_ptr(), tw.st.data_ptr(), tw.zt.data_ptr(), _lib.DTYPE_BF16,
                                                x.data_ptr(), _lib.DTYPE_BF16, y.data_ptr(), None, m, n, k, 128, 0, stream)
                        else:
                            lib.sqx_int4_skinny(tw.wt.data_ptr(), tw.st.data_ptr(), tw.zt.data_ptr(), _lib.DTYPE_BF16,
                                                x.data_ptr(), _lib.DTYPE_BF16, y.data_ptr(), None, m, n, k, 128, -1, 0, 0,
                                                0, ws.data_ptr() if nb > 0 else None, nb, stream)
                    return len(tws)

                byts = n * k // 2 + 2 * 2 * n * k // 128 + 2 * m * k + 2 * m * n
                res["config2_int4_g128_asym"][f"{k}->{n} M={m}"] = gbs_entry(_graph_us(run), byts)
            del tws
            torch.cuda.empty_cache()

    # config 3: AWQ int4 g128 prefill GEMM, M in {64, 512, 2048}
    if 3 in ids:
        for n, k in ((4096, 4096), (1024, 4096), (14336, 4096), (4096, 14336)):
            sc = torch.exp(torch.empty(k, device=dev).uniform_(-0.6931, 0.6931, generator=g))
            quants = rotating(n, k, lambda w: awq.quantize_awq_int4(w, chan_scale=sc), n * k // 2 + n * k // 32)
            for m in (64, 512, 2048):
                x = torch.randn(m, k, generator=g, device=dev)
                x[:, torch.randperm(k, generator=torch.Generator().manual_seed(k))[: k // 100].to(dev)] *= 20.0
                x = x.to(torch.bfloat16)
                us = _graph_call_us([lambda q=q: awq.awq_linear(x, q) for q in quants])
                fl = 2.0 * m * n * k
                res["config3_awq_int4_g128"][f"{k}->{n} M={m}"] = {
                    "us": round(us, 1), "tflops": round(fl / us / 1e6, 1),
                    "frac_of_bf16_peak": round(fl / us * 1e6 / BF16_PEAK, 4),
                    "weight_gbs": round((n * k // 2 + n * k // 32) / us / 1e3, 1), "rotating_copies": len(quants)}
            del quants
            torch.cuda.empty_cache()

    # config 4: MXFP4 weights (e2m1 + e8m0 per 32 along K), bf16 or MXFP4 activations, M in {1, 128}
    if 4 in ids:
        for n, k in ((28672, 8192), (8192, 28672)):
            tws = rotating(n, k, lambda w: f4.tile_fp4(f4.mxfp4_quantize(w, 32)), n * k // 2)
            x1 = torch.randn(1, k, generator=g, device=dev).to(torch.bfloat16)
            y1 = torch.empty(1, n, dtype=torch.bfloat16, device=dev)

            def run(stream):
                for tw in tws:
                    lib.sqx_fp4_linear(tw.wt.data_ptr(), tw.st.data_ptr(), tw.fmt, _lib.ptr(tw.s_global), x1.data_ptr(),
                                       _lib.DTYPE_BF16, y1.data_ptr(), _lib.DTYPE_BF16, None, 1, n, k, 0, stream)
                return len(tws)

            byts = n * k // 2 + n * k // 32 + 2 * k + 2 * n
            res["config4_mxfp4"][f"bf16_x {k}->{n} M=1"] = gbs_entry(_graph_us(run), byts)
            # MXFP4 activations at M = 1: what mxfp4_linear(quantize_activations=True) runs (the row's
            # quantize-dequantize, then the weight GEMV), and the fp4 MFMA GEMM on the same row
            us = _graph_call_us([lambda tw=tw: f4.fp4_linear_tiled(f4.mxfp4_fake_quant_rows(x1), tw) for tw in tws])
            e = gbs_entry(us, byts)
            e["path"] = "mxfp4_fake_quant_rows + FP4 GEMV (two launches)"
            res["config4_mxfp4"][f"mxfp4_x {k}->{n} M=1"] = e
            xq1 = f4.mxfp4_quantize_tiled(x1)
            e = gbs_entry(_graph_call_us([lambda tw=tw: f4.mxfp4_gemm(xq1, tw) for tw in tws]), byts)
            e["path"] = "fp4 MFMA GEMM (activations quantized beforehand)"
            res["config4_mxfp4"][f"mxfp4_x {k}->{n} M=1 GEMM"] = e
            m = 128
            x = torch.randn(m, k, generator=g, device=dev).to(torch.bfloat16)
            fl = 2.0 * m * n * k
            us = _graph_call_us([lambda tw=tw: f4.fp4_linear_tiled(x, tw) for tw in tws])
            res["config4_mxfp4"][f"bf16_x {k}->{n} M={m}"] = {
                "us": round(us, 1), "tflops": round(fl / us / 1e6, 1), "frac_of_bf16_peak": round(fl / us * 1e6 / BF16_PEAK, 4),
                "weight_gbs": round((n * k // 2 + n * k // 32) / us / 1e3, 1), "rotating_copies": len(tws)}
            xq = f4.mxfp4_quantize_tiled(x)
            us = _graph_call_us([lambda tw=tw: f4.mxfp4_gemm(xq, tw) for tw in tws])
            res["config4_mxfp4"][f"mxfp4_x {k}->{n} M={m}"] = {
                "us": round(us, 1), "tflops": round(fl / us / 1e6, 1), "frac_of_fp4_peak": round(fl / us * 1e6 / FP4_PEAK, 4),
                "weight_gbs": round((n * k // 2 + n * k // 32) / us / 1e3, 1), "rotating_copies": len(tws),
                "quantize_x_us": round(_graph_call_us(lambda: f4.mxfp4_quantize_tiled(x)), 1)}
            del tws
            torch.cuda.empty_cache()
    return res


if __name__ == "__main__":
    sys.exit(main())
