#!/usr/bin/env python3
"""Sparse-MoE decode benchmark on one MI355X.

Workload: a 48-layer stack of sparse-MoE blocks at H=2048, I=512, E=512 routed
experts (top-10, softmax renormalised) plus one shared expert (Is=512,
sigmoid-gated), batch-1 decode. All 48 layers' bf16 weights (~155 GB) are
resident in HBM, seeded synthetic with a Zipf(1.1) router bias. One step = one
token through all 48 layers, chained through a pre-norm residual stream
(h_l = rms_norm(r_l), r_{l+1} = bf16(r_l + block_l(h_l))); the whole step is
one persistent kernel launch (k_moe_decode), so the timed region is exactly
the kernel launches.

Prints one JSON line (the driver contract) with:
  value       microseconds per token of the 48-layer step (lower is better)
  roofline    HBM-bound: algorithmic weight bytes per launch / average launch
              time (HIP events on the launch stream) against 8 TB/s
  cpu_baseline the CPU oracle (the reference's scalar path restated in C) on
              the same input, one host thread, 48 layers, block arithmetic only
  mtp         the same step with 2 and 4 tokens (MTP verify widths)
  prefill     8192 tokens through one resident block (router, top-10,
              grouped bf16 MFMA expert GEMMs, ordered combine): tokens/s from
              HIP events on the launch stream; the grouped GEMMs' MFMA
              utilisation from the committed rocprofv3 kernel trace
Progress goes to stderr.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "MoE decode µs/token (batch 1, 48 layers) + HBM GB/s; 8K prefill tokens/s"
SHAPE = dict(hidden=2048, intermediate=512, experts=512, top_k=10, shared_intermediate=512)
HBM_PEAK_GBPS = 8000.0
BF16_PEAK_TFLOPS = 2500.0  # dense bf16 MFMA
F32_PEAK_TFLOPS = 157.3  # dense fp32 MFMA
PREFILL_TOKENS = 8192


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def layer_bytes(union_experts: int) -> int:
    """Algorithmic HBM bytes of one layer: router [E,H], the union of selected
    experts' gate_up [2I,H] + down [H,I], the shared expert (3 x [Is,H]) and the
    shared-expert gate [1,H], all bf16."""
    H, I, E, Is = SHAPE["hidden"], SHAPE["intermediate"], SHAPE["experts"], SHAPE["shared_intermediate"]
    return 2 * (E * H + union_experts * (2 * I * H + H * I) + 3 * Is * H + H)


def time_steps(rt, ctx, x, resid, tokens: int, steps: int, warmup: int):
    """Launch the step on a dedicated default-priority stream and bracket every
    launch with HIP events recorded on that same stream."""
    stream = rt.Stream()
    for _ in range(warmup):
        ctx.moe_step_dev(x.ptr, tokens, resid.ptr, stream=stream.handle)
    stream.synchronize()
    ctx.synchronize()
    starts = [rt.Event() for _ in range(steps)]
    ends = [rt.Event() for _ in range(steps)]
    for i in range(steps):
        starts[i].record(stream)
        ctx.moe_step_dev(x.ptr, tokens, resid.ptr, stream=stream.handle)
        ends[i].record(stream)
    stream.synchronize()
    ctx.synchronize()
    per_launch_ms = [s.elapsed_ms(e) for s, e in zip(starts, ends)]
    total_ms = starts[0].elapsed_ms(ends[-1])
    for e in starts + ends:
        e.destroy()
    stream.destroy()
    return total_ms, per_launch_ms


def union_sizes(ids: np.ndarray) -> list[int]:
    """ids [L, T, K] -> number of distinct experts per layer."""
    return [len(set(ids[l].ravel().tolist())) for l in range(ids.shape[0])]


TRAFFIC_SUMMARY = ROOT / "profiles" / "k_moe_decode_48l_t1_hbm_traffic.md"


def read_traffic():
    """HBM bytes per launch of the decode kernel (FETCH_SIZE + WRITE_SIZE,
    calibrated against a copy of known size) from the committed rocprofv3 PMC
    summary, or None when there is none."""
    if not TRAFFIC_SUMMARY.is_file():
        return None
    for line in TRAFFIC_SUMMARY.read_text().splitlines():
        if line.startswith("hbm_bytes_per_launch:"):
            try:
                return int(line.split(":", 1)[1].strip())
            except ValueError:
                return None
    return None


COPY_CALIBRATION_BYTES = 1 << 30


def copy_calibration(rt, hm) -> None:
    """Three launches of the plain copy kernel over 1 GiB, for the traffic
    counters' scale (each reads and writes exactly 1 GiB)."""
    src = rt.DeviceArray((COPY_CALIBRATION_BYTES // 2,), np.uint16)
    dst = rt.DeviceArray((COPY_CALIBRATION_BYTES // 2,), np.uint16)
    stream = rt.Stream()
    for _ in range(3):
        hm.copy_bytes(dst.ptr, src.ptr, COPY_CALIBRATION_BYTES, stream.handle)
    stream.synchronize()
    stream.destroy()
    src.free()
    dst.free()
    log(f"copy calibration: 3 x {COPY_CALIBRATION_BYTES} bytes")


def prefill_flops(ids: np.ndarray, tokens: int) -> dict:
    """Algorithmic flops of the many-token block: routed expert GEMMs (one
    gate/up [2I,H] and one down [H,I] product per (token, expert) pair), the
    shared expert (every token) and the exact router."""
    H, I, E, Is = SHAPE["hidden"], SHAPE["intermediate"], SHAPE["experts"], SHAPE["shared_intermediate"]
    pairs = int(ids.size)
    return {"routed_gemm": 2 * pairs * (2 * I * H + H * I),
            "shared_gemm": 2 * tokens * (2 * Is * H + H * Is),
            "router": 2 * tokens * (E + 1) * H}


def read_prefill_profile() -> dict | None:
    """Average durations (us) of the prefill kernels from the committed
    rocprofv3 summary of this workload, or None."""
    path = ROOT / "profiles" / "k_pf_prefill_8k_kernel_trace.md"
    if not path.is_file():
        return None
    out = {}
    for line in path.read_text().splitlines():
        if line.startswith("avg_us "):
            _, name, value = line.split()
            out[name] = float(value)
    return out or None


def bench_prefill(rt, hm, ctx, args) -> dict:
    T = PREFILL_TOKENS
    x_host = hm.synth_hidden(args.seed, T, SHAPE["hidden"], True, first_token=100000)
    got = ctx.prefill_block(0, x_host)
    flops = prefill_flops(got["selected_experts"], T)
    x = rt.DeviceArray.from_numpy(x_host)
    out = rt.DeviceArray(x_host.shape, np.uint16)
    stream = rt.Stream()
    for _ in range(2):
        ctx.prefill_block_dev(0, x.ptr, T, out.ptr, stream=stream.handle)
    stream.synchronize()
    steps = max(3, args.steps // 5)
    start, end = rt.Event(), rt.Event()
    start.record(stream)
    for _ in range(steps):
        ctx.prefill_block_dev(0, x.ptr, T, out.ptr, stream=stream.handle)
    end.record(stream)
    stream.synchronize()
    ctx.synchronize()
    ms = start.elapsed_ms(end) / steps
    assert np.array_equal(out.numpy(), got["out"]), "device-pointer prefill differs from host-pointer prefill"
    total = sum(flops.values())
    res = {"tokens": T, "us_per_block": round(ms * 1000, 1), "tokens_per_s": round(T / (ms * 1e-3), 1),
           "pairs": int(got["selected_experts"].size),
           "max_tokens_per_expert": int(np.bincount(got["selected_experts"].ravel()).max()),
           "flops": flops, "block_tflops": round(total / (ms * 1e-3) / 1e12, 1)}
    prof = read_prefill_profile()
    if prof:
        gemm_us = prof.get("k_pf_gemm_gate_up", 0.0) + prof.get("k_pf_gemm_down", 0.0)
        if gemm_us > 0:
            gemm = flops["routed_gemm"] + flops["shared_gemm"]
            tf = gemm / (gemm_us * 1e-6) / 1e12
            res["gemm_roofline"] = {"bound": "mfma", "achieved": round(tf, 1), "peak": BF16_PEAK_TFLOPS,
                                    "unit": "TFLOP/s", "frac": round(tf / BF16_PEAK_TFLOPS, 4),
                                    "source": "profiles/k_pf_prefill_8k_kernel_trace.md"}
        router_us = prof.get("k_pf_router_mx", 0.0) + prof.get("k_pf_router", 0.0)
        if router_us > 0:
            tf = flops["router"] / (router_us * 1e-6) / 1e12
            res["router_roofline"] = {"bound": "mfma", "dtype": "f32 (bf16 operands, one product per step)",
                                      "achieved": round(tf, 1), "peak": F32_PEAK_TFLOPS, "unit": "TFLOP/s",
                                      "frac": round(tf / F32_PEAK_TFLOPS, 4),
                                      "source": "profiles/k_pf_prefill_8k_kernel_trace.md"}
        res["kernel_us"] = prof
    log(f"prefill {T} tokens: {ms * 1000:.1f} us/block, {T / (ms * 1e-3) / 1e6:.2f} M tokens/s")
    stream.destroy()
    start.destroy()
    end.destroy()
    x.free()
    out.free()
    return res


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--layers", type=int, default=48)
    ap.add_argument("--seed", type=lambda s: int(s, 0), default=0x46495245)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-mtp", action="store_true")
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--prefill-only", action="store_true",
                    help="time the 8K-token prefill block alone (for kernel traces)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="also run a 1 GiB plain copy kernel (traffic-counter calibration)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (asked for --gpus {args.gpus}); the sparse-MoE "
              "path is measured on a single MI355X, expert-parallel sharding is design-only.",
              file=sys.stderr)
        return 2

    from firewing_amd import hip_moe as hm
    from firewing_amd import hip_runtime as rt

    if args.prefill_only:
        ctx = hm.MoeContext(layers=1, **SHAPE)
        ctx.generate_layers(0, 1, args.seed, True)
        res = bench_prefill(rt, hm, ctx, args)
        ctx.close()
        print(json.dumps({"prefill": res}), flush=True)
        return 0

    L = args.layers
    T = 1
    log(f"creating context: {L} layers, shape {SHAPE}")
    t0 = time.time()
    ctx = hm.MoeContext(layers=L, **SHAPE)
    log(f"device {ctx.device_name}; generating {L} layers of synthetic weights")
    ctx.generate_layers(0, L, args.seed, True)
    log(f"resident banks ready in {time.time() - t0:.1f} s")

    x_host = hm.synth_hidden(args.seed, T, SHAPE["hidden"], True)
    x = rt.DeviceArray.from_numpy(x_host)
    resid = rt.DeviceArray(x_host.shape, np.uint16)

    # Routed union per layer (10 for one token) from one captured step.
    r_host, _, ids, _ = ctx.moe_step(x_host)
    unions = union_sizes(ids)
    bytes_per_launch = sum(layer_bytes(u) for u in unions)

    log(f"timing {args.steps} steps after {args.warmup} warm-up steps")
    total_ms, per_launch = time_steps(rt, ctx, x, resid, T, args.steps, args.warmup)
    gpu_resid = resid.numpy()
    assert np.array_equal(gpu_resid, r_host), "device-pointer step differs from host-pointer step"
    ms_per_step = total_ms / args.steps
    avg_launch_ms = float(np.mean(per_launch))
    us_per_token = ms_per_step * 1000.0 / T
    achieved = bytes_per_launch / (avg_launch_ms * 1e-3) / 1e9
    log(f"{ms_per_step * 1000:.1f} us/step, kernel avg {avg_launch_ms * 1000:.1f} us, "
        f"{achieved:.0f} GB/s ({achieved / HBM_PEAK_GBPS:.1%} of peak)")

    result = {
        "metric": METRIC,
        "value": round(us_per_token, 3),
        "unit": "us/token",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 6),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": f"{L}-layer sparse-MoE decode step, batch 1 (one persistent launch)",
            "layers": L, "tokens": T, **SHAPE,
            "weights_resident_gb": round(L * (layer_bytes(SHAPE["experts"]) - 2 * SHAPE["hidden"]) / 1e9, 1),
            "router": "tree32 logits (in-model order), total-order top-10, f32 softmax, renormalised",
            "accumulate": "f32, reference summation order, no FMA",
            "router_bias": "Zipf(1.1) popularity via constant feature x[H-1]=1",
            "chaining": "pre-norm residual: h_l = rms_norm(r_l) (h[H-1]=1), r_{l+1} = bf16(r_l + block_l(h_l))",
            "seed": hex(args.seed),
        },
        "hbm_gbps": round(achieved, 1),
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBPS, 4),
            "traffic": read_traffic(),
            "kernel": "fw::k_moe_decode<1, 64, 16, 8>",
            "algorithmic_bytes_per_launch": bytes_per_launch,
            "avg_launch_us": round(avg_launch_ms * 1000.0, 2),
        },
    }

    if args.copy_calibration:
        copy_calibration(rt, hm)

    if not args.no_mtp:
        mtp = {}
        for width in (2, 4):
            xw_host = hm.synth_hidden(args.seed, width, SHAPE["hidden"], True, first_token=1000)
            xw = rt.DeviceArray.from_numpy(xw_host)
            rw = rt.DeviceArray(xw_host.shape, np.uint16)
            _, _, idw, _ = ctx.moe_step(xw_host)
            u = union_sizes(idw)
            b = sum(layer_bytes(n) for n in u)
            tot, per = time_steps(rt, ctx, xw, rw, width, max(5, args.steps // 2), 2)
            ms = tot / max(5, args.steps // 2)
            gbps = b / (float(np.mean(per)) * 1e-3) / 1e9
            mtp[str(width)] = {"us_per_step": round(ms * 1000, 2),
                               "us_per_token": round(ms * 1000 / width, 2),
                               "mean_union_experts_per_layer": round(float(np.mean(u)), 2),
                               "hbm_gbps": round(gbps, 1),
                               "frac": round(gbps / HBM_PEAK_GBPS, 4)}
            log(f"MTP width {width}: {ms * 1000:.1f} us/step, union {np.mean(u):.1f}, {gbps:.0f} GB/s")
        result["mtp"] = mtp

    if not args.no_prefill:
        result["prefill"] = bench_prefill(rt, hm, ctx, args)

    ctx.close()
    x.free()
    resid.free()

    if not args.no_cpu_baseline:
        from oracle import fw_oracle as fo
        log("CPU baseline: oracle 48-layer step, one thread (weights regenerated untimed)")
        t0 = time.time()
        cpu_resid, secs = fo.synth_step_timed(SHAPE, args.seed, L, x_host)
        wall = time.time() - t0
        parity = bool(np.array_equal(cpu_resid, r_host))
        log(f"CPU: {secs * 1e3:.1f} ms of block arithmetic ({wall:.1f} s wall); "
            f"GPU residual {'==' if parity else '!='} CPU residual")
        result["cpu_baseline"] = {
            "value": round(secs * 1e6 / T, 1),
            "unit": "us/token",
            "cores": 1,
            "kind": "port",
            "sample": f"the full {L}-layer chained step for the same token, one thread; "
                      "block arithmetic timed, weight regeneration excluded",
        }
        result["parity"] = {"gpu_vs_cpu_residual_bit_exact": parity}
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
