"""Benchmark of the MI355X Swin block forward (BASELINE.json metric).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config c2|c2u|c1|c4]

A step is one forward pass of one SwinTransformerBlock over one batch of
synthetic input (weights: reference trunc-normal init; activations N(0,1)),
through the fused C-ABI call nsw_swin_block_forward.  Prints one JSON line:
tokens/s over K timed steps (inputs resident in HBM), the roofline of the
dominant kernel from HIP events on the launch stream, the per-kernel
breakdown, and a CPU baseline (the fp32 oracle on the host cores, on a
bounded sample of the same workload; with the config-1 block and one
config-3 step assembled from its timed parts beside it).  One GPU only.

The line also carries
  "kernels.metrics_unnorm": the config-5 per-step RMSE/ACC reduction (HBM);
  "gemm_vs_hipblaslt": the block's four GEMM shapes without epilogue, this
              library's GEMM against torch.matmul (hipBLASLt), same operands;
  "config4":  the config-4 block (with its per-kernel breakdown) and one
              forward of the depth-8 p2 model;
  "shard":    one GPU's share of config 2 split 2-way in longitude (the
              block on 180 x 180 tokens), time per token against the full block;
  "achievable": this box's own peaks, the best of a 1 GiB read-only stream
              and 1 GiB device copies (HBM), and the fastest hipBLASLt GEMM
              of an 8192^3 product and the block's four shapes (MFMA); every
              kernel entry and the roofline also give frac_achievable, the
              fraction of those beside the fraction of the spec peaks;
and, unless --no-model is given,
  "forecast": config 3, one SwinTransformer forward (p4, e1024, depth 16,
              16 heads, window 9x18, 70 channels, 720x1440, bf16) = ms per
              forecast step, split into embedding / blocks / head (the
              blocks as one window-order chain), and the same step with one
              fused call per block (ms_per_step_block_calls);
  "rollout":  config 5, 8 autoregressive steps of the config-3 model with
              per-step latitude-weighted RMSE and ACC (nsw.Rollout) in bf16
              and through this library's fp32 path: per-step drift against
              the fp32 oracle rollout of the same weights and inputs, whose
              per-step metrics tests/test_gpu_fullsize.py records in
              tests/golden/rollout_c5_fp32_oracle.json (bench.py does not run
              the oracle outside its CPU-baseline leg).
Inputs there are seeded Gaussian-filtered, per-channel standardised fields
(sigma = 8 px), standing in for ERA5.

Traffic (roofline.traffic): profile this command with --copy-calibration
under two rocprofv3 --pmc runs (FETCH_SIZE, then WRITE_SIZE) and summarise
them with --traffic-summary; the calibration copy and the block's kernels
then come from the same runs.
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "neural-scaling-weather_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "Swin-block fwd tokens/s + % MFMA/HBM roofline, p4 e1024 180x360, 1 GPU"
SPIN_CYCLES = 400_000     # ~0.2 ms spin before diagnostic event sequences
PEAK_BF16_TFLOPS = 2500.0   # MI355X dense bf16 MFMA
PEAK_F32_TFLOPS = 157.3     # MI355X dense fp32 MFMA
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E

CONFIGS = {
    # name: (B, T, H, W, C, heads, ws, shift, dtype, description)
    "c2": (1, 1, 180, 360, 1024, 16, (9, 18), (4, 9), "bf16",
           "config 2: shifted SwinTransformerBlock fwd, B=1 T=1, 180x360 tokens (p4 on 720x1440), "
           "C=1024, 16 heads (hd 64), window 9x18 (400 windows x 162), shift 4x9, mlp 4x"),
    "c2u": (1, 1, 180, 360, 1024, 16, (9, 18), (0, 0), "bf16",
            "config 2, unshifted twin (shift 0x0)"),
    "c1": (1, 1, 90, 180, 192, 6, (9, 18), (4, 9), "f32",
           "config 1: shifted block fp32, 90x180 tokens, C=192, 6 heads (hd 32), window 9x18, shift 4x9"),
    "c4": (1, 1, 360, 720, 512, 8, (9, 18), (4, 9), "bf16",
           "config 4 block: shifted block bf16, 360x720 tokens (p2), C=512, 8 heads (hd 64), window 9x18"),
}


def block_flops(B, T, H, W, C, heads, ws):
    """Algorithmic FLOPs per block (utils/flops_utils.py:15-29 GEMM + attention
    matmul terms, unpadded): QKV, proj, fc1, fc2, QK^T, PV."""
    M = B * T * H * W
    L = T * ws[0] * ws[1]
    nWb = M // L
    hd = C // heads
    qkv = 2 * M * C * 3 * C
    proj = 2 * M * C * C
    fc1 = 2 * M * C * 4 * C
    fc2 = 2 * M * 4 * C * C
    att = 2 * (2 * nWb * heads * L * L * hd)
    return {"qkv": qkv, "proj": proj, "fc1": fc1, "fc2": fc2, "attention": att}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", default="c2", choices=sorted(CONFIGS))
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-model", action="store_true", help="skip the config-3 forecast and config-5 rollout")
    ap.add_argument("--model-steps", type=int, default=10, help="timed forecast steps (config 3)")
    ap.add_argument("--no-rollout", action="store_true", help="skip the config-5 rollout")
    ap.add_argument("--norms", choices=["fold2", "window", "separate"], default="fold2",
                    help="fold2 (default): norm1 as a gather pass, proj scattering to tokens with the norm2 "
                         "sums, fc1 with norm2 as a row scale, 6 launches; window: both norms folded, the "
                         "block as a one-block window-order chain (partition + norm1 sums, QKV with norm1 "
                         "as a row scale, attention, proj with the norm2 sums, fc1, fc2 scattering to "
                         "tokens), 6 launches; separate: both norms as passes of their own, 7 launches")
    ap.add_argument("--cpu-seconds", type=float, default=15.0, help="target CPU-baseline sample time")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="before anything else, run a plain 256 MiB device copy (5 launches): the "
                         "reference kernel whose FETCH_SIZE / WRITE_SIZE counters, read in the same "
                         "rocprofv3 --pmc run as the block's kernels, calibrate the HBM-traffic figures")
    ap.add_argument("--traffic-summary", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"),
                    help="no GPU work: read the counter CSVs of a FETCH_SIZE and a WRITE_SIZE rocprofv3 run "
                         "of 'bench.py --copy-calibration ...', print the calibrated traffic per kernel as "
                         "markdown and write profiles/traffic_<config>.json")
    ap.add_argument("--no-config4", action="store_true", help="skip the config-4 block and model timing")
    ap.add_argument("--no-gemm-compare", action="store_true", help="skip the hipBLASLt comparison leg")
    ap.add_argument("--gemm-only", action="store_true",
                    help="run only the hipBLASLt comparison leg (the block's four GEMM shapes, this library's "
                         "GEMM against torch.matmul) and print its JSON: the command its counter profiles use")
    ap.add_argument("--gemm-phases", action="store_true",
                    help="per-tile phase cycles of the block's GEMMs and of plain GEMMs of the same shapes, "
                         "from nsw/libnsw_stamps.so (build.py --stamps); prints one JSON line and exits")
    ap.add_argument("--no-block-calls", action="store_true",
                    help="skip the config-3 comparison run with one fused call per block (the forward keeps "
                         "the residual stream in window order between blocks)")
    args = ap.parse_args()

    if args.traffic_summary:
        traffic_summary(args.traffic_summary[0], args.traffic_summary[1], args.config)
        return

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(json.dumps({"error": "this build runs on one GPU only; the Swin block path has no "
                                   "multi-GPU mode here; run with --gpus 1 (the value is one GPU's throughput)",
                          "n_gpus": args.gpus}), flush=True)
        sys.exit(2)

    import torch
    import nsw
    from nsw import _lib, ops

    if args.copy_calibration:
        copy_calibration()
    if args.gemm_phases:
        print(json.dumps({"gemm_phases": gemm_phases(torch.device("cuda:0"), args.config, args.norms)}), flush=True)
        return
    if args.gemm_only:
        B, T, H, W, C = CONFIGS[args.config][:5]
        M = B * T * H * W
        print(json.dumps({"gemm_vs_hipblaslt": gemm_compare(torch.device("cuda:0"), M, C, 4 * C, args.steps,
                                                            args.warmup)}), flush=True)
        return

    B, T, H, W, C, heads, ws, shift, dts, desc = CONFIGS[args.config]
    dtype = torch.bfloat16 if dts == "bf16" else torch.float32
    dev = torch.device("cuda:0")
    torch.manual_seed(1001)
    blk = nsw.Block(C, heads, (H, W), ws, T, shift_size=shift).to(device=dev, dtype=dtype).eval()
    blk.fold_norm1 = args.norms == "window"
    blk.fold_norm2 = args.norms != "separate"
    g = torch.Generator().manual_seed(1002)
    x = torch.randn(B, T, H, W, C, generator=g).to(device=dev, dtype=dtype)
    M = B * T * H * W

    # ---------------------------------------------------------------- timed
    with torch.inference_mode():
        for _ in range(args.warmup):
            y = blk(x)
        torch.cuda.synchronize()
        stream = torch.cuda.current_stream(dev)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        e0.record(stream)
        for _ in range(args.steps):
            y = blk(x)
        e1.record(stream)
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        ms_step = e0.elapsed_time(e1) / args.steps
        if not torch.isfinite(y.float()).all():
            raise RuntimeError("non-finite block output")

        kern, same = block_kernels(blk, x, y, (B, T, H, W, C, heads, ws, shift, dtype), args.norms, args.steps,
                                   args.warmup)
        # The same K fused blocks timed again once the GPU has run this
        # workload for a while (the op-by-op loop above): from an idle GPU
        # the first ~25 blocks run slower while the power manager settles
        # the clocks (2.0 -> 1.5 ms per block at config 2), and the timed
        # steps above start right after the W warm-up steps.  Reported
        # beside `value`, which stays the contract's measurement.
        e2, e3 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e2.record(stream)
        for _ in range(args.steps):
            y2 = blk(x)
        e3.record(stream)
        torch.cuda.synchronize()
        ms_settled = e2.elapsed_time(e3) / args.steps
        del y2
    fl = block_flops(B, T, H, W, C, heads, ws)
    peak_f = PEAK_BF16_TFLOPS if dtype == torch.bfloat16 else PEAK_F32_TFLOPS
    names = list(kern)
    dom = max(names, key=lambda n: kern[n]["ms"])
    d = kern[dom]
    traffic = None
    tf_path = os.path.join(ROOT, "profiles", f"traffic_{args.config}.json")
    if os.path.exists(tf_path):
        with open(tf_path) as f:
            traffic = json.load(f).get(dom)
    roofline = {"kernel": dom, "bound": d["bound"], "achieved": d["achieved"],
                "peak": peak_f if d["bound"] == "mfma" else PEAK_HBM_GBS, "unit": d["unit"],
                "frac": d["frac"], "traffic": traffic}

    total_flops = sum(fl.values())
    out = {
        "metric": METRIC,
        "value": round(M / (ms_step * 1e-3), 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": dts,
        "data": "synthetic (N(0,1) activations, reference trunc-normal(0.02) weights)",
        "config": {"workload": desc, "tokens": M, "block_tflop": round(total_flops / 1e12, 4),
                   "block_tflops_achieved": round(total_flops / (ms_step * 1e-3) / 1e12, 1),
                   "wall_s_timed": round(wall, 4), "ops_path_equals_fused": bool(same),
                   "block_launches": len(names), "norms": args.norms,
                   "ms_per_step_settled": round(ms_settled, 4),
                   "settled_note": "the same K fused blocks re-timed after the op-by-op kernel loop; from an idle "
                                   "GPU the first ~25 blocks run slower while the clocks settle"},
        "roofline": roofline,
        "kernels": kern,
    }

    # ----------------------------------------- metrics kernel (config 5 step)
    kern["metrics_unnorm"] = metrics_timing(dev, args.steps, args.warmup)
    # ------------------------------------------------ GEMMs against hipBLASLt
    if not args.no_gemm_compare and args.config in ("c2", "c2u"):
        out["gemm_vs_hipblaslt"] = gemm_compare(dev, M, C, 4 * C, args.steps, args.warmup)
    # ------------------------------- achievable peaks of this box, and fractions
    ach = achievable_peaks(dev, dtype, args.steps, args.warmup, out.get("gemm_vs_hipblaslt"))
    out["achievable"] = ach
    for k in kern.values():
        ref = ach["mfma_tflops"] if k["bound"] == "mfma" else ach["hbm_GBs"]
        k["frac_achievable"] = round(k["achieved"] / ref, 4)
    roofline["frac_achievable"] = kern[dom]["frac_achievable"]
    # ------------------------------------------------------------ config 4
    if not args.no_config4 and args.config in ("c2", "c2u"):
        torch.cuda.empty_cache()
        out["config4"] = config4_section(dev, args.steps, args.warmup, args.model_steps)
        for k in out["config4"]["block_kernels"].values():
            k["frac_achievable"] = round(k["achieved"] / (ach["mfma_tflops"] if k["bound"] == "mfma"
                                                          else ach["hbm_GBs"]), 4)
        out["shard"] = shard_section(dev, args.steps, args.warmup, M, ms_step)

    # ------------------------------------------------- config 3 / config 5
    if not args.no_model:
        del y
        torch.cuda.empty_cache()
        out["forecast"], rollout = model_sections(dev, args.model_steps, args.warmup, not args.no_rollout,
                                                  not args.no_block_calls)
        if rollout is not None:
            out["rollout"] = rollout

    # ----------------------------------------------------------- CPU baseline
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline(blk, B, T, H, W, C, heads, ws, shift, args.cpu_seconds)
    print(json.dumps(out), flush=True)


def block_kernels(blk, x, y_fused, cfg, norms, steps, warmup, after=None):
    """The block's kernels launched one op at a time (the same kernels as the
    fused call) with HIP events between them on the launch stream: per-kernel
    ms, achieved rate and fraction of the binding spec peak.  Returns
    (kernels, whether the op-by-op output equals the fused call's).  `after`,
    if given, is called with each kernel's name right after its launch (the
    phase-stamp reader; its times are then not meaningful)."""
    import torch
    from nsw import _lib, ops
    B, T, H, W, C, heads, ws, shift, dtype = cfg
    M = B * T * H * W
    stream = torch.cuda.current_stream(x.device)
    with torch.inference_mode():
        # ---------------------------------------------- per-kernel breakdown
        # the same kernels, launched one op at a time with HIP events between
        # them on the launch stream
        pk = blk.packed()
        eps = blk._eps(dtype)
        scale = (C // heads) ** -0.5
        st = {}

        def k_gather():
            st["xw"] = ops.rmsnorm_roll_partition(x, pk["norm1_w"], ws, shift, eps)

        def k_qkv():
            st["qkv"] = ops.qkv_projection(st["xw"], pk["wqkv"], pk["bqkv"], pk["qn_w"], pk["kn_w"], heads, eps)

        L = T * ws[0] * ws[1]

        def k_part():
            st["xw"], st["s1"] = ops.window_partition_sumsq(x, ws, shift)

        def k_qkv_rs():
            st["qkv"] = ops.qkv_projection_rowscale(st["xw"].view(-1, C), pk["wqkv_n1"], pk["bqkv"], pk["qn_w"],
                                                    pk["kn_w"], st["s1"], heads, eps).view(-1, L, 3 * C)

        def k_proj_id():
            st["h1"], st["ss"] = ops.linear_remap_residual(st["o"].view(-1, C), pk["wproj"], pk["bproj"],
                                                           st["xw"].view(-1, C), 0)

        def k_fc2_tok():
            y_, _ = ops.linear_remap_residual(st["u"], pk["w2"], pk["b2"], st["h1"], 1, image=(B, T, H, W),
                                              window_size=ws, shift_size=shift)
            st["y"] = y_.view(B, T, H, W, C)

        def k_attn():
            st["o"] = ops.window_attention(st["qkv"], heads, scale, geometry=(H, W, ws, shift, T))

        def k_proj():
            st["h1"] = ops.proj_reverse_residual(st["o"], pk["wproj"], pk["bproj"], x, ws, shift)

        def k_proj_ss():
            st["h1"], st["ss"] = ops.proj_reverse_residual_sumsq(st["o"], pk["wproj"], pk["bproj"], x, ws, shift)

        def k_norm2():
            st["hn"] = ops.rms_norm(st["h1"], pk["norm2_w"], eps)

        def k_fc1():
            st["u"] = ops.linear(st["hn"], pk["w1"], pk["b1"], epilogue=_lib.NSW_EPI_BIAS_GELU)

        def k_fc1_rs():
            st["u"] = ops.linear_rowscale(st["h1"], pk["w1_n2"], st["ss"], pk["b1"],
                                          epilogue=_lib.NSW_EPI_BIAS_GELU, eps=eps)

        def k_fc2():
            st["y"] = ops.linear(st["u"], pk["w2"], pk["b2"], residual=st["h1"])

        if norms == "window":
            seq = [("partition_sumsq", k_part), ("qkv_rowscale", k_qkv_rs), ("attention", k_attn),
                   ("proj_sumsq", k_proj_id), ("fc1_rowscale", k_fc1_rs), ("fc2_to_tokens", k_fc2_tok)]
        else:
            seq = [("gather_norm1", k_gather), ("qkv", k_qkv), ("attention", k_attn)]
            seq += ([("proj_scatter_sumsq", k_proj_ss), ("fc1_rowscale", k_fc1_rs)] if blk.fold_norm2 else
                    [("proj_scatter", k_proj), ("norm2", k_norm2), ("fc1", k_fc1)])
            seq += [("fc2", k_fc2)]
        names = [n for n, _ in seq]
        times = {n: [] for n in names}
        for it in range(warmup + steps):
            ev = [torch.cuda.Event(enable_timing=True) for _ in range(len(names) + 1)]
            # a short spin kernel ahead of the first event keeps the GPU busy
            # while the host enqueues the first op, so that op's interval
            # holds its kernel and not the host's launch latency
            torch.cuda._sleep(SPIN_CYCLES)
            ev[0].record(stream)
            for i, (n_, fn) in enumerate(seq):
                fn()
                ev[i + 1].record(stream)
                if after is not None:
                    after(n_)
            torch.cuda.synchronize()
            if it >= warmup:
                for i, n in enumerate(names):
                    times[n].append(ev[i].elapsed_time(ev[i + 1]))
        same = torch.equal(st["y"], y_fused)

    es = 2 if dtype == torch.bfloat16 else 4
    A = M * C * es
    fl = block_flops(B, T, H, W, C, heads, ws)
    peak_f = PEAK_BF16_TFLOPS if dtype == torch.bfloat16 else PEAK_F32_TFLOPS
    work = {  # (algorithmic units per launch, bound)
        "gather_norm1": (2 * A, "hbm"), "qkv": (fl["qkv"], "mfma"), "attention": (4 * A, "hbm"),
        "proj_scatter": (fl["proj"], "mfma"), "norm2": (2 * A, "hbm"), "fc1": (fl["fc1"], "mfma"),
        "fc2": (fl["fc2"], "mfma"), "fc1_rowscale": (fl["fc1"], "mfma"),
        "proj_scatter_sumsq": (fl["proj"], "mfma"), "partition_sumsq": (2 * A, "hbm"),
        "qkv_rowscale": (fl["qkv"], "mfma"), "proj_sumsq": (fl["proj"], "mfma"), "fc2_to_tokens": (fl["fc2"], "mfma"),
    }
    kern = {}
    for n in names:
        t = statistics.mean(times[n]) * 1e-3
        units, bound = work[n]
        if bound == "mfma":
            ach = units / t / 1e12
            kern[n] = {"ms": round(t * 1e3, 4), "bound": "mfma", "achieved": round(ach, 1), "unit": "TFLOP/s",
                       "frac": round(ach / peak_f, 4)}
        else:
            ach = units / t / 1e9
            kern[n] = {"ms": round(t * 1e3, 4), "bound": "hbm", "achieved": round(ach, 1), "unit": "GB/s",
                       "frac": round(ach / PEAK_HBM_GBS, 4)}
    return kern, same


def stamp_phases(stamps, ntile):
    """Per-tile phase means (cycles of s_memtime) from the GEMM's stamp words
    (start, first stages landed, main loop done, first epilogue phase staged,
    end, HW_ID, XCC_ID, workgroup id per tile), and the mean gap between a
    tile's end and the start of the next tile on the same CU."""
    import numpy as np
    t = stamps[: ntile * 8].reshape(ntile, 8).astype(np.int64)
    hw = t[:, 5]
    # CU of a workgroup: XCC, shader engine (HW_ID 13-15), array (12), CU (8-11)
    cu = (t[:, 6] & 0xF) * 1000 + ((hw >> 13) & 7) * 100 + ((hw >> 12) & 1) * 20 + ((hw >> 8) & 15)
    gaps = []
    for k in np.unique(cu):
        idx = np.where(cu == k)[0]
        o = idx[np.argsort(t[idx, 0])]
        gaps.extend((t[o[1:], 0] - t[o[:-1], 4]).tolist())
    mean = lambda a: round(float(np.mean(a)), 0)
    return {"prologue": mean(t[:, 1] - t[:, 0]), "main_loop": mean(t[:, 2] - t[:, 1]),
            "first_staging": mean(t[:, 3] - t[:, 2]), "rest_of_epilogue": mean(t[:, 4] - t[:, 3]),
            "total": mean(t[:, 4] - t[:, 0]), "gap_to_next_tile_on_cu": mean(gaps) if gaps else None,
            "cus": int(len(np.unique(cu))), "tiles": int(ntile)}


def gemm_phases(dev, config, norms):
    """Per-tile phase cycles (s_memtime) of the block's GEMMs, launched one op
    at a time as in block_kernels, and of plain GEMMs (no epilogue) of the
    same shapes, through nsw/libnsw_stamps.so (the library with the phase
    stamps compiled in).  Means over the tiles of the last of 3 launches of
    each kernel; MFMA issue per tile and SIMD = 16 cycles per
    v_mfma_f32_16x16x32_bf16 (bf16)."""
    import numpy as np
    import torch
    import nsw
    from nsw import _lib, ops
    path = os.path.join(ROOT, "neural-scaling-weather_amd", "nsw", "libnsw_stamps.so")
    if not os.path.exists(path):
        raise SystemExit(f"{path} is not built: python neural-scaling-weather_amd/build.py --stamps")
    _lib.use(path)
    B, T, H, W, C, heads, ws, shift, dts, desc = CONFIGS[config]
    dtype = torch.bfloat16 if dts == "bf16" else torch.float32
    M = B * T * H * W
    buf = np.zeros(65536 * 8, dtype=np.uint64)

    def read(ntile):
        torch.cuda.synchronize()
        _lib.check(_lib.lib().nsw_gemm_read_stamps(buf.ctypes.data, buf.nbytes), "nsw_gemm_read_stamps")
        return stamp_phases(buf, ntile)

    def tiles(n):
        return ((M + 255) // 256) * ((n + 255) // 256)

    def mfma_cycles(k):
        return 256 * 256 * k // (16 * 16 * (32 if dtype == torch.bfloat16 else 4)) // 4 * 16

    shapes = {"qkv": (3 * C, C), "proj_scatter_sumsq": (C, C), "fc1_rowscale": (4 * C, C), "fc2": (C, 4 * C),
              "qkv_rowscale": (3 * C, C), "proj_sumsq": (C, C), "fc2_to_tokens": (C, 4 * C),
              "proj_scatter": (C, C), "fc1": (4 * C, C)}
    res = {"workload": desc, "clock": "s_memtime cycles (shader clock)", "fused": {}, "plain": {}}
    torch.manual_seed(1001)
    blk = nsw.Block(C, heads, (H, W), ws, T, shift_size=shift).to(device=dev, dtype=dtype).eval()
    blk.fold_norm1 = norms == "window"
    blk.fold_norm2 = norms != "separate"
    x = torch.randn(B, T, H, W, C, generator=torch.Generator().manual_seed(1002)).to(device=dev, dtype=dtype)

    def after(name):
        if name in shapes:
            n, k = shapes[name]
            res["fused"][name] = dict(read(tiles(n)), mfma_issue=mfma_cycles(k))

    with torch.inference_mode():
        y = blk(x)
        block_kernels(blk, x, y, (B, T, H, W, C, heads, ws, shift, dtype), norms, 1, 2, after=after)
        g = torch.Generator(device=dev).manual_seed(7)
        for name, (n, k) in (("qkv", (3 * C, C)), ("proj", (C, C)), ("fc1", (4 * C, C)), ("fc2", (C, 4 * C))):
            a = torch.randn(M, k, device=dev, generator=g).to(dtype)
            w = (torch.randn(n, k, device=dev, generator=g) * 0.03).to(dtype)
            for _ in range(3):
                ops.linear(a, w)
            res["plain"][name] = dict(read(tiles(n)), mfma_issue=mfma_cycles(k))
            del a, w
    return res


CALIB_BYTES = 256 << 20
CALIB_LAUNCHES = 5


def traffic_minimum(config):
    """Algorithmic HBM bytes per launch of each block kernel (each operand
    read once, each output written once; weights and row statistics
    included): a calibrated counter figure below it is impossible."""
    B, T, H, W, C, heads, ws, shift, dts, desc = CONFIGS[config]
    es = 2 if dts == "bf16" else 4
    M = B * T * H * W
    A = M * C * es
    wb = C * C * es                       # one C x C weight
    ss = M * ((C * es + 511) // 512) * 4  # row partial sums of squares
    return {"gather_norm1": 2 * A, "partition_sumsq": 2 * A + ss, "qkv": A + 3 * wb + 3 * A,
            "qkv_rowscale": A + ss + 3 * wb + 3 * A, "attention": 4 * A,
            "proj_scatter_sumsq": 3 * A + wb + ss, "proj_sumsq": 3 * A + wb + ss,
            "fc1_rowscale": A + ss + 4 * wb + 4 * A, "fc2": 4 * A + 4 * wb + 2 * A,
            "fc2_to_tokens": 4 * A + 4 * wb + 2 * A, "metrics_unnorm": 2 * 70 * 720 * 1440 * 4}


def copy_calibration():
    """A plain 256 MiB device-to-device copy, 5 launches, before any other
    work: its FETCH_SIZE / WRITE_SIZE per dispatch divided by the bytes it
    moves is the factor that turns those counters into HBM bytes for the
    other kernels of the same profiled run."""
    import torch
    src = torch.empty(CALIB_BYTES, dtype=torch.uint8, device="cuda:0").fill_(1)
    dst = torch.empty_like(src)
    for _ in range(CALIB_LAUNCHES):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_bytes": src.numel(), "launches": CALIB_LAUNCHES}), flush=True)
    del src, dst
    torch.cuda.empty_cache()


# Kernel names in a rocprofv3 trace -> bench.py's kernel names (config 2,
# bf16, the 6-launch blocks of --norms window and fold2).  The GEMM instances
# are told apart by their (mangled) template arguments: gemm_kernel<T, EPI, PRE>.
TRACE_NAMES = [
    ("_ZN3nsw11gemm_kernelIDF16bLi2ELi3E", "fc1_rowscale"),
    ("_ZN3nsw11gemm_kernelIDF16bLi64ELi3E", "qkv_rowscale"),
    ("_ZN3nsw11gemm_kernelIDF16bLi13ELi0E", "proj_sumsq"),
    ("_ZN3nsw11gemm_kernelIDF16bLi14ELi0E", "fc2_to_tokens"),
    ("partition_sumsq_kernel", "partition_sumsq"),
    ("_ZN3nsw11gemm_kernelIDF16bLi3ELi0E", "fc2"),
    ("_ZN3nsw11gemm_kernelIDF16bLi64ELi0E", "qkv"),
    ("_ZN3nsw11gemm_kernelIDF16bLi11ELi0E", "proj_scatter_sumsq"),
    ("attn_dma_kernel", "attention"),
    ("attn_mfma_kernel", "attention"),
    ("row_map_kernel", "gather_norm1"),
    ("wsum_partial_kernel", "metrics_unnorm"),
    ("__amd_rocclr_copyBuffer", "copy_calibration"),
]


def trace_name(kernel_name):
    for key, name in TRACE_NAMES:
        if kernel_name.startswith(key) or key in kernel_name:
            return name
    return None


def traffic_summary(fetch_dir, write_dir, config):
    """Calibrated HBM traffic per kernel from two rocprofv3 --pmc runs (one
    counter each) of the same bench command with --copy-calibration: the
    counters (KB per dispatch) are scaled by what they read for the 256 MiB
    copy of that run."""
    import csv
    import glob

    def load(d, counter):
        acc, copies = {}, []
        for path in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True):
            with open(path) as f:
                for r in csv.DictReader(f):
                    if r["Counter_Name"] != counter:
                        continue
                    n = trace_name(r["Kernel_Name"])
                    v = float(r["Counter_Value"]) * 1024.0
                    if n == "copy_calibration":
                        copies.append((int(r["Dispatch_Id"]), v))
                    elif n is not None:
                        acc.setdefault(n, []).append(v)
        # the calibration copies are the first CALIB_LAUNCHES blit-copy
        # dispatches of the run (copy_calibration runs before any other work;
        # later copies -- the 1 GiB achievable-peak copy, torch's small ones --
        # use the same blit kernel and grid, so neither size nor grid tells
        # them apart); they must agree with each other
        copies.sort()
        cal = [v for _, v in copies[:CALIB_LAUNCHES]]
        if len(cal) < CALIB_LAUNCHES:
            raise SystemExit(f"{counter}: the run holds no calibration copy: profile 'bench.py --copy-calibration ...'")
        if max(cal) > 1.02 * min(cal):
            raise SystemExit(f"{counter}: the first {CALIB_LAUNCHES} copies disagree ({min(cal):.4g}..{max(cal):.4g} B):"
                             " they are not the calibration copies")
        out = {k: sum(vs) / len(vs) for k, vs in acc.items()}
        out["copy_calibration"] = sum(cal) / len(cal)
        return out

    fetch, write = load(fetch_dir, "FETCH_SIZE"), load(write_dir, "WRITE_SIZE")
    nbytes = float(CALIB_BYTES)
    kf, kw = fetch["copy_calibration"] / nbytes, write["copy_calibration"] / nbytes
    minimum = traffic_minimum(config)
    out = {}
    rows = []
    for n in sorted(set(fetch) & set(write)):
        if n == "copy_calibration":
            continue
        f, w = fetch[n] / kf, write[n] / kw
        lo = minimum.get(n)
        if lo is not None and f + w < 0.98 * lo:
            raise SystemExit(f"{n}: calibrated traffic {(f + w) / 1e6:.1f} MB is below the kernel's algorithmic "
                             f"minimum {lo / 1e6:.1f} MB: the calibration is wrong")
        out[n] = int(round(f + w))
        ratio = "" if lo is None else f"{(f + w) / lo:.2f}"
        rows.append(f"| {n} | {f / 1e6:.1f} | {w / 1e6:.1f} | {(f + w) / 1e6:.1f} | "
                    f"{'' if lo is None else f'{lo / 1e6:.1f}'} | {ratio} |")
    print(f"calibration (same runs): FETCH_SIZE reads {kf:.4f} x and WRITE_SIZE {kw:.4f} x the copy's bytes")
    print("| kernel | fetch (MB) | write (MB) | total (MB) | algorithmic (MB) | total / algorithmic |\n"
          "|---|---|---|---|---|---|")
    print("\n".join(rows))
    out["_calibration"] = {"fetch_factor": round(kf, 4), "write_factor": round(kw, 4)}
    with open(os.path.join(ROOT, "profiles", f"traffic_{config}.json"), "w") as fh:
        json.dump(out, fh, indent=1, sort_keys=True)


def timed(fn, steps, warmup):
    """Mean ms of fn() between HIP events on the launch stream (a spin
    kernel ahead of the first event hides the host's enqueue latency)."""
    import torch
    stream = torch.cuda.current_stream()
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda._sleep(SPIN_CYCLES)
    e0.record(stream)
    for _ in range(steps):
        fn()
    e1.record(stream)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps


def metrics_timing(dev, steps, warmup):
    """The rollout's per-step metric call at config 5 (70 channels,
    720 x 1440, fp32 prediction and target, unnormalised RMSE + ACC): HBM
    bound, 2 x 290.3 MB read per call (utils/losses.py:243-257)."""
    import torch
    import nsw
    from nsw import ops
    C, H, W = 70, 720, 1440
    g = torch.Generator(device=dev).manual_seed(4001)
    pred = torch.randn(1, 1, C, H, W, generator=g, device=dev)
    tgt = torch.randn(1, 1, C, H, W, generator=g, device=dev)
    std = torch.rand(C, generator=g, device=dev) + 0.5
    mean = torch.randn(C, generator=g, device=dev)
    clim = torch.randn(C, generator=g, device=dev)
    lat = nsw.misc_utils.era5_latitudes(H)
    w = nsw.build_spherical_area_weights(lat)[:, None].to(dev)
    ms = timed(lambda: ops.weighted_metrics_unnorm(pred, tgt, std, mean, w, clim), steps, warmup)
    nbytes = 2 * C * H * W * 4
    ach = nbytes / (ms * 1e-3) / 1e9
    return {"ms": round(ms, 4), "bound": "hbm", "achieved": round(ach, 1), "unit": "GB/s",
            "frac": round(ach / PEAK_HBM_GBS, 4), "bytes": nbytes,
            "workload": "config 5 per-step metrics: [1,1,70,720,1440] fp32 prediction and target, "
                        "unnormalise + weighted RMSE + ACC (two launches: partial sums, final)"}


def achievable_peaks(dev, dtype, steps, warmup, gemms=None):
    """What this box reaches on its own, the references of the per-kernel
    frac_achievable: HBM, the best of a read-only stream over 1 GiB (this
    library's nsw_hbm_stream probe, read bytes), the probe's 1 GiB copy and
    torch's 1 GiB copy_ (read + write bytes); MFMA, the fastest of an 8192^3
    torch.matmul in the block's dtype and the block's own four GEMM shapes
    through torch.matmul (``gemms``, the gemm_vs_hipblaslt leg), all
    hipBLASLt."""
    import torch
    from nsw import _lib
    n = 1 << 28
    src = torch.ones(n, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    stream = torch.cuda.current_stream(dev).cuda_stream
    L = _lib.lib()

    def probe(d):
        rc = L.nsw_hbm_stream(src.data_ptr(), d, 4 * n, 0, stream)
        if rc != 0:
            raise RuntimeError(L.nsw_last_error().decode())

    t_read = timed(lambda: probe(None), steps, warmup)
    t_pcopy = timed(lambda: probe(dst.data_ptr()), steps, warmup)
    t_copy = timed(lambda: dst.copy_(src), steps, warmup)
    del src, dst
    N = 8192
    g = torch.Generator(device=dev).manual_seed(4102)
    a = torch.randn(N, N, generator=g, device=dev).to(dtype)
    b = torch.randn(N, N, generator=g, device=dev).to(dtype)
    t_mm = timed(lambda: torch.matmul(a, b), steps, warmup)
    del a, b
    read_gbs = n * 4 / (t_read * 1e-3) / 1e9
    pcopy_gbs = 2 * n * 4 / (t_pcopy * 1e-3) / 1e9
    copy_gbs = 2 * n * 4 / (t_copy * 1e-3) / 1e9
    mm = {f"matmul {N}^3": 2.0 * N ** 3 / (t_mm * 1e-3) / 1e12}
    for name, r in (gemms or {}).items():
        mm[f"{name} shape"] = r["hipblaslt_tflops"]
    best = max(mm, key=mm.get)
    return {"hbm_GBs": round(max(read_gbs, pcopy_gbs, copy_gbs), 1), "hbm_read_GBs": round(read_gbs, 1),
            "hbm_copy_GBs": round(max(pcopy_gbs, copy_gbs), 1), "mfma_tflops": round(mm[best], 1),
            "mfma_source": f"hipBLASLt {best} ({str(dtype).replace('torch.', '')})",
            "hbm": "best of a 1 GiB read-only stream (nsw_hbm_stream, read bytes) and 1 GiB copies "
                   "(nsw_hbm_stream, torch copy_; read + write bytes)",
            "gemm_tflops": {k: round(v, 1) for k, v in mm.items()}}


def gemm_compare(dev, M, C, Hm, steps, warmup):
    """The block's four GEMM shapes without epilogue, nsw_linear against
    torch.matmul (hipBLASLt) on the same bf16 operands, interleaved."""
    import torch
    from nsw import ops
    g = torch.Generator(device=dev).manual_seed(4101)
    res = {}
    for name, (N, K) in {"qkv": (3 * C, C), "proj": (C, C), "fc1": (Hm, C), "fc2": (C, Hm)}.items():
        x = torch.randn(M, K, generator=g, device=dev).to(torch.bfloat16)
        w = (torch.randn(N, K, generator=g, device=dev) * 0.02).to(torch.bfloat16)
        wt = w.t()
        t_nsw, t_lib = [], []
        for _ in range(3):
            t_nsw.append(timed(lambda: ops.linear(x, w), steps, warmup))
            t_lib.append(timed(lambda: torch.matmul(x, wt), steps, warmup))
        a, b = ops.linear(x, w), torch.matmul(x, wt)
        diff = (a.float() - b.float()).abs().max().item()
        fl = 2.0 * M * N * K
        tn, tl = min(t_nsw), min(t_lib)
        res[name] = {"M": M, "N": N, "K": K, "nsw_ms": round(tn, 4), "hipblaslt_ms": round(tl, 4),
                     "nsw_tflops": round(fl / (tn * 1e-3) / 1e12, 1), "hipblaslt_tflops": round(fl / (tl * 1e-3) / 1e12, 1),
                     "max_abs_diff": diff}
        del x, w, wt, a, b
    return res


def shard_section(dev, steps, warmup, M_full, ms_full):
    """One GPU's share of config 2 under a 2-way longitude split (sp2 = 2):
    the shifted block on 180 x 180 tokens (200 windows), the kernels one GPU
    would run at that shard's shape; the halo exchange of the roll is not
    part of it (one GPU, local cyclic roll)."""
    import torch
    import nsw
    B, T, H, W, C, heads, ws, shift = 1, 1, 180, 180, 1024, 16, (9, 18), (4, 9)
    torch.manual_seed(5002)
    blk = nsw.Block(C, heads, (H, W), ws, T, shift_size=shift).to(device=dev, dtype=torch.bfloat16).eval()
    x = torch.randn(B, T, H, W, C, device=dev).to(torch.bfloat16)
    with torch.inference_mode():
        ms = timed(lambda: blk(x), steps, warmup)
    del blk, x
    M = B * T * H * W
    return {"workload": "config 2 split 2-way in longitude (sp2 = 2): shifted block on 180 x 180 tokens, "
                        "C=1024, 16 heads, window 9x18 (200 windows), one GPU's shard, no halo exchange",
            "tokens": M, "ms": round(ms, 4), "tokens_per_s": round(M / (ms * 1e-3), 1),
            "per_token_vs_full": round((ms / M) / (ms_full / M_full), 4)}


def config4_section(dev, steps, warmup, model_steps):
    """Config 4: the shifted block (360 x 720 tokens, C = 512, 8 heads) and
    one forward of the depth-8 p2 model on 720 x 1440 x 70 (bf16)."""
    import torch
    import nsw
    B, T, H, W, C, heads, ws, shift, dts, desc = CONFIGS["c4"]
    torch.manual_seed(5001)
    blk = nsw.Block(C, heads, (H, W), ws, T, shift_size=shift).to(device=dev, dtype=torch.bfloat16).eval()
    x = torch.randn(B, T, H, W, C, device=dev).to(torch.bfloat16)
    fl = block_flops(B, T, H, W, C, heads, ws)
    with torch.inference_mode():
        ms_blk = timed(lambda: blk(x), steps, warmup)
        y = blk(x)
    kern, same = block_kernels(blk, x, y, (B, T, H, W, C, heads, ws, shift, torch.bfloat16), "fold2", steps,
                               warmup)
    del blk, x, y
    Cc, Hi, Wi, p, depth = 70, 720, 1440, 2, 8
    lat = nsw.misc_utils.era5_latitudes(Hi)
    lon = nsw.misc_utils.era5_longitudes(Wi)
    meta = {"coords": nsw.get_spatial_coords((lat, lon)).float(), "sp_shapes": [[Hi], [Wi]], "n_channels": Cc}
    model = nsw.SwinTransformer(temporal_context_window_size=T, window_size=ws, patch_size=p, in_chans=Cc,
                                out_chans=Cc, embed_dim=C, depth=depth, num_heads=heads, coord_pos_embed=True,
                                domain_metadata=meta).to(device=dev, dtype=torch.bfloat16).eval()
    xm = smooth_fields((1, T, Cc, Hi, Wi), 8.0, 5002, dev)
    tokens = (Hi // p) * (Wi // p)
    step_flops = depth * sum(fl.values()) + 2 * tokens * (Cc * p * p) * C * 2
    with torch.inference_mode():
        ms_model = timed(lambda: model(xm), model_steps, warmup)
        ok = bool(torch.isfinite(model(xm).float()).all())
    del model, xm
    torch.cuda.empty_cache()
    return {"workload": desc + "; model: p2 e512 depth 8, 8 heads, 70 channels on 720x1440, bf16",
            "block_ms": round(ms_blk, 4), "block_tokens_per_s": round(H * W / (ms_blk * 1e-3), 1),
            "block_tflops": round(sum(fl.values()) / (ms_blk * 1e-3) / 1e12, 1),
            "block_kernels": kern, "ops_path_equals_fused": bool(same),
            "model_ms_per_step": round(ms_model, 3), "model_tflop_per_step": round(step_flops / 1e12, 3),
            "model_tflops": round(step_flops / (ms_model * 1e-3) / 1e12, 1), "finite": ok}


def smooth_fields(shape, sigma, seed, dev):
    """Seeded N(0, 1) noise [..., H, W] convolved with a periodic Gaussian of
    `sigma` pixels (FFT) and standardised per leading index, on the GPU."""
    import math
    import torch
    g = torch.Generator(device=dev).manual_seed(seed)
    x = torch.randn(shape, generator=g, device=dev, dtype=torch.float32)
    H, W = shape[-2], shape[-1]
    ky = torch.fft.fftfreq(H, device=dev).view(H, 1)
    kx = torch.fft.rfftfreq(W, device=dev).view(1, -1)
    filt = torch.exp(-2.0 * (math.pi * sigma) ** 2 * (ky ** 2 + kx ** 2))
    flat = x.view(-1, H, W)
    for i in range(flat.shape[0]):          # one plane at a time: bounded FFT workspace
        y = torch.fft.irfft2(torch.fft.rfft2(flat[i]) * filt, s=(H, W))
        flat[i] = (y - y.mean()) / y.std()
    return x


# config 3's model: (C_in = C_out, H, W, p, E, depth, heads, window, T)
C3 = (70, 720, 1440, 4, 1024, 16, 16, (9, 18), 1)
ROLLOUT_STEPS = 8
# the fp32 oracle rollout of config3_model + rollout_setup, recorded on the
# GPU by tests/test_gpu_fullsize.py::test_rollout_config5_bench_setup
ROLLOUT_GOLDEN = os.path.join(ROOT, "tests", "golden", "rollout_c5_fp32_oracle.json")


def config3_model(dev):
    """The config-3 model (p4, e1024, depth 16, 16 heads, window 9x18, 70
    channels on 720 x 1440, coordinate positional embedding), random init
    from seed 3001 (reference trunc-normal(0.02)) held in bf16, and its
    input field (seed 3002)."""
    import torch
    import nsw
    C, H, W, p, E, depth, heads, ws, T = C3
    lat = nsw.misc_utils.era5_latitudes(H)
    lon = nsw.misc_utils.era5_longitudes(W)
    meta = {"coords": nsw.get_spatial_coords((lat, lon)).float(), "sp_shapes": [[H], [W]], "n_channels": C}
    torch.manual_seed(3001)
    model = nsw.SwinTransformer(temporal_context_window_size=T, window_size=ws, patch_size=p, in_chans=C,
                                out_chans=C, embed_dim=E, depth=depth, num_heads=heads, coord_pos_embed=True,
                                domain_metadata=meta).to(device=dev, dtype=torch.bfloat16).eval()
    x = smooth_fields((1, T, C, H, W), 8.0, 3002, dev)
    return model, x


def rollout_setup(dev):
    """Config 5's statistics and targets: per-channel mean / std (seed 3003),
    a climatology near the mean, cos-latitude area weights over the 720 ERA5
    rows, and ROLLOUT_STEPS normalised target fields (seed 3004)."""
    import torch
    import nsw
    C, H, W = C3[0], C3[1], C3[2]
    g = torch.Generator().manual_seed(3003)
    mean = torch.randn(C, generator=g) * 10.0
    std = torch.rand(C, generator=g) * 1.5 + 0.5
    clim = mean + std * torch.randn(C, generator=g) * 0.01
    w = nsw.build_spherical_area_weights(nsw.misc_utils.era5_latitudes(H))[:, None]
    targets = smooth_fields((ROLLOUT_STEPS, C, H, W), 8.0, 3004, dev)
    return mean, std, clim, w, targets


def model_sections(dev, steps, warmup, with_rollout=True, with_block_calls=True):
    """Config 3 (one forecast step of the d16 model) and config 5 (8-step
    rollout, bf16, drift against the fp32 oracle rollout's recorded
    per-step metrics and against this library's fp32 path)."""
    import numpy as np
    import torch
    import nsw
    C, H, W, p, E, depth, heads, ws, T = C3
    model, x = config3_model(dev)
    tokens = (H // p) * (W // p)
    fl = block_flops(1, T, H // p, W // p, E, heads, ws)
    step_flops = depth * sum(fl.values()) + 2 * tokens * (C * p * p) * E * 2   # blocks + embed + head GEMMs
    stream = torch.cuda.current_stream(dev)
    with torch.inference_mode():
        for _ in range(warmup):
            model(x)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(steps):
            yb = model(x)
        e1.record(stream)
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / steps
        # stage split of the same forward path (model.forward: the embedding
        # into block 0's window order, the window-order chain, the fused
        # head), averaged over `steps` passes with events between the stages
        # and a spin kernel first (see the per-kernel loop of the block).  The
        # chain's argument lists are built once beforehand: in the pipelined
        # steps above the host builds them while the GPU runs the previous step.
        split = [0.0, 0.0, 0.0]
        chain = model._embed_into_chain()
        if chain:
            b0 = model.blocks[0]
            w_pe = model.patch_embed.proj.conv.weight
            pos = model._pos_tokens(x.shape[0], w_pe.dtype, w_pe.device)
            params, shifts, eps, tanh = model._chain_args(model.patch_embed.tokens_windowed(
                x, pos, b0.window_size, b0.shift_size)[0])
        for _ in range(steps):
            ev = [torch.cuda.Event(enable_timing=True) for _ in range(4)]
            torch.cuda._sleep(SPIN_CYCLES)
            ev[0].record(stream)
            if chain:
                yw, ss = model.patch_embed.tokens_windowed(x, pos, b0.window_size, b0.shift_size)
                ev[1].record(stream)
                tok = torch.ops.nsw.swin_blocks_windowed(yw, ss, params, b0.num_heads,
                                                         [int(v) for v in b0.window_size], shifts, eps, tanh)
                del yw, ss
            else:
                tok = model.prepare_tokens(x)
                ev[1].record(stream)
                tok = model.forward_blocks(tok)
            ev[2].record(stream)
            model._head_last(tok)
            ev[3].record(stream)
            torch.cuda.synchronize()
            for i in range(3):
                split[i] += ev[i].elapsed_time(ev[i + 1]) / steps
        if not torch.isfinite(yb.float()).all():
            raise RuntimeError("non-finite forecast")
        # the same step with one fused call per block (no window-order chain)
        ms_per_block = None
        if with_block_calls:
            model.chain_blocks = False
            for _ in range(2):
                model(x)
            e0.record(stream)
            for _ in range(steps):
                model(x)
            e1.record(stream)
            torch.cuda.synchronize()
            ms_per_block = e0.elapsed_time(e1) / steps
            model.chain_blocks = True
    forecast = {
        "workload": "config 3: SwinTransformer fwd, [1,1,70,720,1440] -> [1,1,70,720,1440], p4 e1024 depth 16, "
                    "16 heads, window 9x18, alternating shift 0 / 4x9, coordinate pos-embed, bf16",
        "ms_per_step": round(ms, 3), "steps": steps, "tflop_per_step": round(step_flops / 1e12, 3),
        "tflops_achieved": round(step_flops / (ms * 1e-3) / 1e12, 1),
        "tokens_per_s": round(tokens / (ms * 1e-3), 1),
        "embed_ms": round(split[0], 3), "blocks_ms": round(split[1], 3), "head_ms": round(split[2], 3),
        "ms_per_step_block_calls": None if ms_per_block is None else round(ms_per_block, 3),
    }
    del tok, yb
    if not with_rollout:
        return forecast, None

    # config 5: rollout, bf16 and fp32 copies of the same weights
    S = ROLLOUT_STEPS
    mean, std, clim, w, targets = rollout_setup(dev)
    res = {}
    for name, dt in (("bf16", torch.bfloat16), ("fp32", torch.float32)):
        m = model if dt == torch.bfloat16 else model.float()
        ro = nsw.Rollout(m, mean, std, w, clim=clim)
        with torch.inference_mode():
            torch.cuda.synchronize()
            t0 = torch.cuda.Event(enable_timing=True); t1 = torch.cuda.Event(enable_timing=True)
            t0.record(stream)
            r, a, _ = ro.run(x, targets)
            t1.record(stream)
            torch.cuda.synchronize()
        res[name] = (r.cpu().numpy(), a.cpu().numpy(), t0.elapsed_time(t1) / S)
    rb, ab, msb = res["bf16"]
    rf, af, msf = res["fp32"]
    rnd = lambda a: [round(float(v), 6) for v in a]
    rollout = {
        "workload": "config 5: config-3 model, 8 autoregressive steps from one seeded initial condition, "
                    "per-step latitude-weighted RMSE and ACC over 70 channels (unnormalised fields)",
        "steps": S, "ms_per_step_bf16": round(msb, 3), "ms_per_step_fp32": round(msf, 3),
        "rmse_mean_bf16": rnd(rb.mean(1)), "acc_mean_bf16": rnd(ab.mean(1)),
    }
    golden = None
    if os.path.exists(ROLLOUT_GOLDEN):
        with open(ROLLOUT_GOLDEN) as fh:
            golden = json.load(fh)
    if golden is not None and golden.get("steps") == S and len(golden.get("rmse", [])) == S:
        ro_r, ro_a = np.asarray(golden["rmse"]), np.asarray(golden["acc"])
        rollout["drift_reference"] = ("fp32 oracle rollout (oracle/model_ref.rollout) of the same weights and "
                                      "inputs, per-step RMSE / ACC recorded in tests/golden/"
                                      "rollout_c5_fp32_oracle.json")
        rollout["rmse_rel_drift_max"] = rnd((np.abs(rb - ro_r) / ro_r).max(1))
        rollout["acc_abs_drift_max"] = rnd(np.abs(ab - ro_a).max(1))
        rollout["fp32_path_rmse_rel_drift_max"] = rnd((np.abs(rf - ro_r) / ro_r).max(1))
        rollout["fp32_path_acc_abs_drift_max"] = rnd(np.abs(af - ro_a).max(1))
    else:
        rollout["drift_reference"] = "this library's fp32 path (no recorded fp32 oracle rollout found)"
        rollout["rmse_rel_drift_max"] = rnd((np.abs(rb - rf) / rf).max(1))
        rollout["acc_abs_drift_max"] = rnd(np.abs(ab - af).max(1))
    rollout["bf16_vs_fp32_path_rmse_rel_drift_max"] = rnd((np.abs(rb - rf) / rf).max(1))
    return forecast, rollout


def cpu_baseline(blk, B, T, H, W, C, heads, ws, shift, target_s):
    """The fp32 oracle (eager PyTorch on the host cores) on a sample of the
    same workload: the first `nb` latitude bands of windows (every token costs
    the same; the roll wraps inside the sample)."""
    import torch
    from oracle import swin_ref
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    p = {k: v.detach().float().cpu() for k, v in blk.state_dict().items()}
    g = torch.Generator().manual_seed(7)
    # size the sample: one band first, then as many bands as make a run of
    # ~target_s/5 seconds (at most the whole image), repeated to ~target_s
    x1 = torch.randn(B, T, ws[0], W, C, generator=g)
    swin_ref.block_forward(x1, p, heads, ws, shift)  # warm-up
    t0 = time.perf_counter()
    swin_ref.block_forward(x1, p, heads, ws, shift)
    t1 = time.perf_counter() - t0
    nbands = H // ws[0]
    nb = max(1, min(nbands, int(round(target_s / 5.0 / max(t1, 1e-3)))))
    Hs = ws[0] * nb
    xs = torch.randn(B, T, Hs, W, C, generator=g)
    times = []
    while True:
        t0 = time.perf_counter()
        swin_ref.block_forward(xs, p, heads, ws, shift)
        times.append(time.perf_counter() - t0)
        if sum(times) >= target_s or len(times) >= 20:
            break
    med = statistics.median(times)
    toks = B * T * Hs * W
    extra = cpu_extra_cases(p, xs, heads, ws, shift, med, nbands / nb)
    cpu_model = ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    cpu_model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"value": round(toks / med, 1), "unit": "tokens/s", "cores": torch.get_num_threads(),
            "kind": "port",
            "sample": f"fp32 oracle block (oracle/swin_ref.py, eager torch) on {nb} of {nbands} latitude bands "
                      f"({Hs}x{W} tokens = {toks}, C={C}), median of {len(times)} runs "
                      f"({med:.2f} s each); cpu: {cpu_model}",
            **extra}


def cpu_extra_cases(p, xs, heads, ws, shift, shifted_s, scale):
    """The other CPU figures of the measurement spec, on the same cores: the
    config-1 block (fp32, 90x180 tokens, C=192, 6 heads, median of 5) and one
    config-3 step assembled from its parts -- the patch embedding
    (Conv2d p4 of the [70, 720, 1440] input + the coordinate embedding) and
    the head (Linear 1024 -> 70*16 + unpatchify), each timed once, plus 8
    shifted and 8 unshifted config-2 blocks (the config-3 blocks are config 2's
    shape), the unshifted one timed once on the same sample; ``scale`` lifts a
    sample of latitude bands to the whole image."""
    import torch
    from oracle import model_ref, swin_ref, synth
    out = {}
    p1 = synth.block_params(192, 6, seed=1001)
    x1 = synth.activations((1, 1, 90, 180, 192), seed=1002)
    swin_ref.block_forward(x1, p1, 6, (9, 18), (4, 9))
    t = []
    for _ in range(5):
        t0 = time.perf_counter()
        swin_ref.block_forward(x1, p1, 6, (9, 18), (4, 9))
        t.append(time.perf_counter() - t0)
    out["c1_block_ms"] = round(1e3 * statistics.median(t), 2)
    t0 = time.perf_counter()
    swin_ref.block_forward(xs, p, heads, ws, (0, 0))
    unshifted_s = time.perf_counter() - t0
    E, p4, ch = 1024, 4, 70
    g = torch.Generator().manual_seed(3001)
    x = torch.randn(1, 1, ch, 720, 1440, generator=g)
    pe_w = synth.trunc_normal((E, ch, p4, p4), 0.02, g)
    pos_w = synth.trunc_normal((E, 4, p4, p4), 0.02, g)
    head_w = synth.trunc_normal((ch * p4 * p4, E), 0.02, g)
    lat = torch.linspace(90, -90, 721)[:-1]
    lon = torch.linspace(0, 360, 1441)[:-1]
    coords = model_ref.model_coords(model_ref.spatial_coords(lat, lon), 1)
    t0 = time.perf_counter()
    pos = model_ref.pos_tokens(coords, pos_w, torch.zeros(E), p4)
    tok = model_ref.prepare_tokens(x, pe_w, torch.zeros(E), p4, pos)
    embed_s = time.perf_counter() - t0
    del x, pos
    t0 = time.perf_counter()
    model_ref.forward_head(tok, head_w, p4, ch)
    head_s = time.perf_counter() - t0
    step = embed_s + head_s + 8 * scale * (shifted_s + unshifted_s)
    out["c3_step"] = {"s": round(step, 2), "embed_s": round(embed_s, 3), "head_s": round(head_s, 3),
                      "block_shifted_s": round(scale * shifted_s, 3),
                      "block_unshifted_s": round(scale * unshifted_s, 3),
                      "note": "embed + head timed once at full size, + 8 shifted and 8 unshifted "
                              "config-2 blocks (fp32 oracle, eager torch)"}
    return out


if __name__ == "__main__":
    main()
