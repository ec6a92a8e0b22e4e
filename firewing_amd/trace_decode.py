"""Per-task timeline of the persistent decode kernel (a profiling aid).

`python -m firewing_amd.trace_decode build` compiles a second copy of the
library with FW_DECODE_TRACE (every task of the launch records wall-clock marks:
start, dependency met, end, and stage marks) into firewing_amd/_trace/.
`python -m firewing_amd.trace_decode run --tokens T` then runs the 48-layer
synthetic decode step (H=2048, I=512, E=512, K=10, Is=512) through it on GPU 0
and prints the per-layer budget: when, after a layer's router tasks end, its
routed gate/up (B) tasks have their selection and end, and its down/combine
(C) tasks have their activations staged, their down-row dots done, and their
results published. T >= 2 tokens that run as interleaved one-token chains
are reported per launch layer (layer * T + token).

The traced build is slower than the product (each mark is a global store);
its timeline is for finding where a layer's time goes, not for timing.
"""
from __future__ import annotations

import argparse
import ctypes
import os
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

import numpy as np

PKG = Path(__file__).resolve().parent
TRACE_DIR = PKG / "_trace"
TRACE_LIB = TRACE_DIR / "libfirewing_hip_moe_trace.so"
SHAPE = dict(hidden=2048, intermediate=512, experts=512, top_k=10, shared_intermediate=512)
SEED = 0x46495245
WORDS = 18  # per task: start, dependency met, end, workgroup << 8 | kind, 12 marks, 2 cycle counts
TICK_US = 0.01  # the wall clock runs at 100 MHz


def build(verbose: bool = False) -> Path:
    """Compile the traced library (FW_DECODE_TRACE) next to the package."""
    from firewing_amd import build as hip_build

    TRACE_DIR.mkdir(exist_ok=True)
    include = ["-I", str(hip_build.ROOT / "include"), "-I", str(hip_build.CSRC)]
    flags = [f for f in hip_build.HIPCC_FLAGS if f != "-shared"] + ["-DFW_DECODE_TRACE"]
    units = [(hip_build.CSRC / "fw_moe.hip", [], TRACE_DIR / "fw_moe.o"),
             (hip_build.CSRC / "fw_safetensors.cpp", [], TRACE_DIR / "fw_safetensors.o"),
             (hip_build.CSRC / "fw_zstd.hip", [], TRACE_DIR / "fw_zstd.o")]
    for nt in (1, 2, 3, 4):
        units.append((hip_build.CSRC / "fw_decode_kernels.hip", [f"-DFW_NT={nt}"], TRACE_DIR / f"t{nt}.o"))
    jobs = [[hip_build.hipcc(), *flags, *include, *d, "-c", str(src), "-o", str(obj)] for src, d, obj in units]
    with ThreadPoolExecutor(max_workers=max(1, min(len(jobs), os.cpu_count() or 1))) as pool:
        for f in [pool.submit(hip_build._compile, j, verbose) for j in jobs]:
            f.result()
    hip_build._compile([hip_build.hipcc(), f"--offload-arch={hip_build.ARCH}", "-shared", "-fPIC",
                        *[str(o) for _, _, o in units], "-o", str(TRACE_LIB)], verbose)
    return TRACE_LIB


def traced_step(tokens: int, layers: int = 48, warmup: int = 3) -> tuple[np.ndarray, int]:
    """One traced decode step of `tokens` tokens; returns the marks
    [launch layers, tasks per layer, WORDS] and the kernel's token count."""
    from firewing_amd import hip_moe as hm

    if not TRACE_LIB.is_file():
        raise RuntimeError(f"{TRACE_LIB} is missing: run `python -m firewing_amd.trace_decode build` first")
    hm.LIB_PATH = TRACE_LIB
    lib = hm.lib()
    fn = lib.firewing_hip_debug_traced_step
    fn.restype = ctypes.c_bool
    fn.argtypes = [ctypes.c_void_p, ctypes.POINTER(ctypes.c_uint16), ctypes.c_size_t,
                   ctypes.POINTER(ctypes.c_uint64), ctypes.c_size_t, ctypes.POINTER(ctypes.c_size_t)]
    with hm.MoeContext(layers=layers, **SHAPE) as ctx:
        ctx.generate_layers(0, layers, SEED, True)
        x = hm.synth_hidden(SEED, tokens, SHAPE["hidden"], True)
        for _ in range(warmup):
            ctx.moe_step(x)
        chains = ctx.token_chains(tokens)
        cap = layers * tokens * 4000 * WORDS
        buf = np.zeros(cap, dtype=np.uint64)
        n = ctypes.c_size_t(0)
        if not fn(ctx._h, x.ctypes.data_as(ctypes.POINTER(ctypes.c_uint16)), tokens,
                  buf.ctypes.data_as(ctypes.POINTER(ctypes.c_uint64)), cap, ctypes.byref(n)):
            raise RuntimeError(lib.firewing_hip_last_error().decode())
    kernel_tokens = tokens // chains
    launch_layers = layers * chains
    return buf[: n.value * WORDS].reshape(launch_layers, -1, WORDS).astype(np.int64), kernel_tokens


def task_counts(kernel_tokens: int) -> tuple[int, int, int, int]:
    H, I, E, K, Is = (SHAPE[k] for k in ("hidden", "intermediate", "experts", "top_k", "shared_intermediate"))
    return (E + 15) // 16 + 1, (Is + 7) // 8, K * kernel_tokens * (I // 8), H // 4


def summarize(tr: np.ndarray, kernel_tokens: int) -> dict:
    """Per-layer budget (µs), medians over the launch layers after the first."""
    nR, nS, nB, nC = task_counts(kernel_tokens)
    assert tr.shape[1] == nR + nS + nB + nC, tr.shape
    R, B, C = tr[:, :nR], tr[:, nR + nS:nR + nS + nB], tr[:, nR + nS + nB:]

    def rel(col, ref):  # µs after the layer's router end, for recorded marks
        v = col[col > 0]
        return (v - ref) * TICK_US

    per = {k: [] for k in ("b_selected_p50", "b_end_p50", "b_end_max", "c_staged_p50", "c_staged_max",
                           "c_dots_p50", "c_published_max", "layer_period")}
    last_c_end = None
    for li in range(tr.shape[0]):
        r_end = R[li, :, 2].max()
        per["b_selected_p50"].append(np.median(rel(B[li, :, 4], r_end)))
        b_end = rel(B[li, :, 2], r_end)
        per["b_end_p50"].append(np.median(b_end))
        per["b_end_max"].append(b_end.max())
        staged = rel(C[li, :, 4 + 4], r_end)
        per["c_staged_p50"].append(np.median(staged))
        per["c_staged_max"].append(staged.max())
        per["c_dots_p50"].append(np.median(rel(C[li, :, 4], r_end)))
        per["c_published_max"].append(rel(C[li, :, 4 + 1], r_end).max())
        c_end = C[li, :, 2].max()
        if last_c_end is not None:
            per["layer_period"].append((c_end - last_c_end) * TICK_US)
        last_c_end = c_end
    out = {k: round(float(np.median(v[1:] if k != "layer_period" else v)), 2) for k, v in per.items()}
    valid = tr[:, :, 0] > 0
    out["launch_us"] = round(float((tr[:, :, 2][valid].max() - tr[:, :, 0][valid].min()) * TICK_US), 1)
    out["launch_layers"] = int(tr.shape[0])
    return out


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    sub = ap.add_subparsers(dest="cmd", required=True)
    sub.add_parser("build")
    run = sub.add_parser("run")
    run.add_argument("--tokens", type=int, default=1)
    run.add_argument("--layers", type=int, default=48)
    run.add_argument("--save", help="write the raw marks (.npy)")
    args = ap.parse_args(argv)
    if args.cmd == "build":
        print(build(verbose=True))
        return 0
    tr, kt = traced_step(args.tokens, args.layers)
    if args.save:
        np.save(args.save, tr)
    s = summarize(tr, kt)
    print(f"traced decode step: {args.layers} layers, {args.tokens} token(s), "
          f"{s['launch_layers']} launch layers of {kt} token(s)")
    print("per launch layer, µs after its router tasks end (median over layers):")
    for k in ("b_selected_p50", "b_end_p50", "b_end_max", "c_staged_p50", "c_staged_max", "c_dots_p50",
              "c_published_max", "layer_period"):
        print(f"  {k:16s} {s[k]:8.2f}")
    print(f"  traced launch    {s['launch_us']:8.1f} us")
    sys.stdout.flush()
    return 0


if __name__ == "__main__":
    sys.exit(main())
