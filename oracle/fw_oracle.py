"""ctypes view of the CPU oracle (oracle/libfw_oracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, by the smoke check in
__graft_entry__.py and by bench.py's CPU-baseline leg, always as the checker.
The product (firewing_amd) never imports this module.

bf16 values travel as numpy uint16 arrays of bit patterns.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

_DIR = Path(__file__).resolve().parent
_LIB_PATH = _DIR / "libfw_oracle.so"
_REF_TOPK_PATH = _DIR / "_ref" / "libtopk_shim_ref.so"

ORDER_TREE32 = 0
ORDER_FOLD = 1

_u16p = ctypes.POINTER(ctypes.c_uint16)
_i32p = ctypes.POINTER(ctypes.c_int32)
_f32p = ctypes.POINTER(ctypes.c_float)
_size = ctypes.c_size_t


class Shape(ctypes.Structure):
    _fields_ = [
        ("hidden", _size),
        ("intermediate", _size),
        ("experts", _size),
        ("top_k", _size),
        ("shared_intermediate", _size),
    ]


HYPER_OUTPUTS = ("hyper_input_normed", "mix_down", "mix_down_scaled", "mix_down_silu", "mix_up",
                 "input_mix", "products", "mixed", "inject", "inject_scaled", "inject_sigmoid",
                 "injection_weights")


class HyperOutputs(ctypes.Structure):
    _fields_ = [(name, ctypes.POINTER(ctypes.c_uint16)) for name in HYPER_OUTPUTS]


class Layer(ctypes.Structure):
    _fields_ = [
        ("router", _u16p),
        ("gate_up", _u16p),
        ("down", _u16p),
        ("shared_gate", _u16p),
        ("shared_up", _u16p),
        ("shared_down", _u16p),
        ("shared_expert_gate", _u16p),
    ]


class BlockCaptures(ctypes.Structure):
    _fields_ = [
        ("logits", _u16p),
        ("ids", _i32p),
        ("scores", _u16p),
        ("routed_mixture", _u16p),
        ("shared_down", _u16p),
        ("shared_gate_sigmoid", _u16p),
        ("shared_gate", _u16p),
        ("shared_up", _u16p),
        ("shared_swiglu", _u16p),
        ("shared_gate_logit", _u16p),
        ("gated_shared", _u16p),
        ("weighted_down", _u16p),
    ]


class SynthConfig(ctypes.Structure):
    _fields_ = [
        ("seed", ctypes.c_uint64),
        ("bias_feature", ctypes.c_int),
        ("order", ctypes.c_int),
        ("threads", ctypes.c_int),
    ]


def build() -> None:
    """Compile the oracle (and, where the reference is mounted, its top-k shim)."""
    subprocess.run(["make", "-s", "-C", str(_DIR)], check=True)
    if Path("/root/reference/native/topk_shim.cpp").is_file():
        subprocess.run(["make", "-s", "-C", str(_DIR), "ref"], check=True)


_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not _LIB_PATH.is_file():
            build()
        L = ctypes.CDLL(str(_LIB_PATH))
        L.fwo_to_bf16.restype = ctypes.c_uint16
        L.fwo_to_bf16.argtypes = [ctypes.c_float]
        L.fwo_from_bf16.restype = ctypes.c_float
        L.fwo_from_bf16.argtypes = [ctypes.c_uint16]
        L.fwo_expf.restype = ctypes.c_float
        L.fwo_expf.argtypes = [ctypes.c_float]
        L.fwo_expf_array.argtypes = [_f32p, _f32p, _size]
        L.fwo_dot_tree32.restype = ctypes.c_float
        L.fwo_dot_tree32.argtypes = [_u16p, _u16p, _size]
        L.fwo_dot_fold.restype = ctypes.c_float
        L.fwo_dot_fold.argtypes = [_u16p, _u16p, _size]
        L.fwo_linear_bf16.argtypes = [_u16p, _u16p, _size, _size, _u16p]
        L.fwo_linear_fold_bf16.argtypes = [_u16p, _u16p, _size, _size, _u16p]
        L.fwo_swiglu_bf16.argtypes = [_u16p, _u16p, _size, _u16p]
        L.fwo_sigmoid_bf16.restype = ctypes.c_uint16
        L.fwo_sigmoid_bf16.argtypes = [ctypes.c_uint16]
        L.fwo_add_bf16.restype = ctypes.c_uint16
        L.fwo_add_bf16.argtypes = [ctypes.c_uint16, ctypes.c_uint16]
        L.fwo_build_silu_lut.argtypes = [_u16p]
        L.fwo_rms_norm_bf16.argtypes = [_u16p, _size, ctypes.c_int, _u16p]
        L.fwo_inner_square_sum.restype = ctypes.c_float
        L.fwo_inner_square_sum.argtypes = [_f32p, _size]
        L.fwo_grouped_rms.argtypes = [_u16p, _u16p, _size, _size, ctypes.c_float, _u16p]
        L.fwo_stream_mean.restype = ctypes.c_float
        L.fwo_stream_mean.argtypes = [_f32p, _size]
        L.fwo_hyper_connection.restype = ctypes.c_int
        L.fwo_hyper_connection.argtypes = [_u16p, _u16p, _u16p, _u16p, _u16p, _size, _size, _size,
                                           ctypes.POINTER(HyperOutputs)]
        L.fwo_inject_residual.argtypes = [_u16p, _u16p, _u16p, _size, _size, _u16p, _u16p]
        L.fwo_make_hidden.restype = ctypes.c_int
        L.fwo_make_hidden.argtypes = [_size] + [ctypes.c_int64] * 5 + [_size, _u16p]
        L.fwo_topk_total_order.restype = ctypes.c_int
        L.fwo_topk_total_order.argtypes = [_u16p, _size, _size, _i32p]
        L.fwo_route_scores.restype = ctypes.c_int
        L.fwo_route_scores.argtypes = [_u16p, _size, _i32p, _size, _u16p]
        L.fwo_route.restype = ctypes.c_int
        L.fwo_route.argtypes = [_u16p, _u16p, _size, _size, _size, ctypes.c_int, _i32p, _u16p, _u16p]
        L.fwo_equivalent_topk_order.restype = ctypes.c_int
        L.fwo_equivalent_topk_order.argtypes = [_i32p, _i32p, _size, _u16p]
        L.fwo_expert_bf16.argtypes = [_u16p, _u16p, _u16p, _size, _size, ctypes.c_uint16,
                                      _u16p, _u16p, _u16p, _u16p]
        L.fwo_mixture_bf16.restype = ctypes.c_int
        L.fwo_mixture_bf16.argtypes = [ctypes.POINTER(_u16p), ctypes.POINTER(_u16p), _u16p, _size,
                                       _size, _i32p, _u16p, _size, _u16p]
        L.fwo_sparse_moe_block.restype = ctypes.c_int
        L.fwo_sparse_moe_block.argtypes = [ctypes.POINTER(Shape), ctypes.POINTER(Layer), _u16p,
                                           ctypes.c_int, _u16p, ctypes.POINTER(BlockCaptures)]
        L.fwo_synth_tables.argtypes = [_u16p, _u16p]
        L.fwo_synth_hidden.argtypes = [ctypes.c_uint64, ctypes.c_uint32, ctypes.c_uint32,
                                       ctypes.c_uint32, ctypes.c_int, _u16p]
        L.fwo_synth_tensor.argtypes = [ctypes.c_uint64, ctypes.c_uint32, ctypes.c_uint32,
                                       ctypes.c_uint64, ctypes.c_uint64, _u16p]
        L.fwo_synth_router_bias.argtypes = [ctypes.c_uint64, ctypes.c_uint32, ctypes.c_uint32, _u16p]
        L.fwo_synth_block.restype = ctypes.c_int
        L.fwo_synth_block.argtypes = [ctypes.POINTER(Shape), ctypes.POINTER(SynthConfig),
                                      ctypes.c_uint32, _u16p, _size, _u16p, _i32p, _u16p, _u16p]
        L.fwo_synth_block_captured.restype = ctypes.c_int
        L.fwo_synth_block_captured.argtypes = [ctypes.POINTER(Shape), ctypes.POINTER(SynthConfig),
                                               ctypes.c_uint32, _u16p, _size, _u16p,
                                               ctypes.POINTER(BlockCaptures)]
        L.fwo_synth_step.restype = ctypes.c_int
        L.fwo_synth_step.argtypes = [ctypes.POINTER(Shape), ctypes.POINTER(SynthConfig),
                                     ctypes.c_uint32, _u16p, _size, _u16p, _u16p, _i32p, _u16p]
        L.fwo_synth_step_timed.restype = ctypes.c_int
        L.fwo_synth_step_timed.argtypes = [ctypes.POINTER(Shape), ctypes.POINTER(SynthConfig),
                                           ctypes.c_uint32, _u16p, _size, _u16p,
                                           ctypes.POINTER(ctypes.c_double)]
        L.fwo_bench_block.restype = ctypes.c_int
        L.fwo_bench_block.argtypes = [ctypes.POINTER(Shape), ctypes.POINTER(SynthConfig), ctypes.c_uint32,
                                      _u16p, _size, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                      ctypes.POINTER(ctypes.c_double), _u16p]
        L.fwo_synth_route.restype = ctypes.c_int
        L.fwo_synth_route.argtypes = [ctypes.POINTER(Shape), ctypes.POINTER(SynthConfig),
                                      ctypes.c_uint32, _u16p, _size, _i32p, _u16p, _u16p]
        _lib = L
    return _lib


def _p16(a: np.ndarray):
    assert a.dtype == np.uint16 and a.flags.c_contiguous
    return a.ctypes.data_as(_u16p)


def _p32(a: np.ndarray):
    assert a.dtype == np.int32 and a.flags.c_contiguous
    return a.ctypes.data_as(_i32p)


def _pf(a: np.ndarray):
    assert a.dtype == np.float32 and a.flags.c_contiguous
    return a.ctypes.data_as(_f32p)


def _u16(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.uint16)


# ---- scalar and vector primitives -------------------------------------------------

def to_bf16(value: float) -> int:
    return int(lib().fwo_to_bf16(ctypes.c_float(value)))


def from_bf16(bits: int) -> float:
    return float(lib().fwo_from_bf16(bits))


def bf16_array(values) -> np.ndarray:
    return np.array([to_bf16(float(v)) for v in values], dtype=np.uint16)


def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint32) << 16).view(np.float32)


def expf(values: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(values, dtype=np.float32)
    out = np.empty_like(x)
    lib().fwo_expf_array(_pf(x), _pf(out), x.size)
    return out


def dot_tree32(left, right) -> float:
    l, r = _u16(left), _u16(right)
    return float(lib().fwo_dot_tree32(_p16(l), _p16(r), l.size))


def dot_fold(weight, hidden) -> float:
    w, x = _u16(weight), _u16(hidden)
    return float(lib().fwo_dot_fold(_p16(w), _p16(x), w.size))


def linear_bf16(weight, hidden, rows: int, columns: int) -> np.ndarray:
    w, x = _u16(weight), _u16(hidden)
    out = np.empty(rows, dtype=np.uint16)
    lib().fwo_linear_bf16(_p16(w), _p16(x), rows, columns, _p16(out))
    return out


def linear_fold_bf16(weight, hidden, rows: int, columns: int) -> np.ndarray:
    w, x = _u16(weight), _u16(hidden)
    out = np.empty(rows, dtype=np.uint16)
    lib().fwo_linear_fold_bf16(_p16(w), _p16(x), rows, columns, _p16(out))
    return out


def swiglu_bf16(gate, up) -> np.ndarray:
    g, u = _u16(gate), _u16(up)
    out = np.empty(g.size, dtype=np.uint16)
    lib().fwo_swiglu_bf16(_p16(g), _p16(u), g.size, _p16(out))
    return out


def sigmoid_bf16(bits: int) -> int:
    return int(lib().fwo_sigmoid_bf16(bits))


def add_bf16(left: int, right: int) -> int:
    return int(lib().fwo_add_bf16(left, right))


def silu_lut() -> np.ndarray:
    out = np.empty(65536, dtype=np.uint16)
    lib().fwo_build_silu_lut(_p16(out))
    return out


def rms_norm_bf16(r, bias_feature: bool = False) -> np.ndarray:
    """Pre-norm of the chained workload (not part of the reference block)."""
    a = _u16(r)
    out = np.empty(a.size, dtype=np.uint16)
    lib().fwo_rms_norm_bf16(_p16(a), a.size, int(bias_feature), _p16(out))
    return out


def inner_square_sum(values) -> float:
    v = np.ascontiguousarray(values, dtype=np.float32)
    return float(lib().fwo_inner_square_sum(_pf(v), v.size))


def grouped_rms(values, weight, streams: int, width: int, epsilon: float = 1e-6) -> np.ndarray:
    x, w = _u16(values), _u16(weight)
    out = np.empty(streams * width, dtype=np.uint16)
    lib().fwo_grouped_rms(_p16(x), _p16(w), streams, width, epsilon, _p16(out))
    return out


def stream_mean(values) -> float:
    v = np.ascontiguousarray(values, dtype=np.float32)
    return float(lib().fwo_stream_mean(_pf(v), v.size))


def hyper_connection(hidden, hc_norm, mix_down_w, mix_up_w, inject_w, streams: int, width: int,
                     lowrank: int) -> dict:
    """One token's hyper-connection: every output of
    src/hyper_connection.rs:412-490 (inject_w None: run_final_mixer)."""
    sizes = {"hyper_input_normed": streams * width, "mix_down": lowrank, "mix_down_scaled": lowrank,
             "mix_down_silu": lowrank, "mix_up": streams * width, "input_mix": streams * width,
             "products": streams * width, "mixed": width, "inject": streams, "inject_scaled": streams,
             "inject_sigmoid": streams, "injection_weights": streams}
    out = {k: np.zeros(sizes[k], dtype=np.uint16) for k in HYPER_OUTPUTS}
    o = HyperOutputs(*[_p16(out[k]) for k in HYPER_OUTPUTS])
    x, n, d, u = _u16(hidden), _u16(hc_norm), _u16(mix_down_w), _u16(mix_up_w)
    inj = _u16(inject_w) if inject_w is not None else None
    if not lib().fwo_hyper_connection(_p16(x), _p16(n), _p16(d), _p16(u), _p16(inj) if inj is not None else None,
                                      streams, width, lowrank, ctypes.byref(o)):
        raise ValueError("invalid hyper-connection shape")
    return out


def inject_residual(post_attention, moe_output, injection_weights, streams: int, width: int):
    """(products [S*W], layer_output [S*W]) of src/decoder_layer.rs:587-607."""
    p, m, w = _u16(post_attention), _u16(moe_output), _u16(injection_weights)
    products = np.empty(streams * width, dtype=np.uint16)
    out = np.empty(streams * width, dtype=np.uint16)
    lib().fwo_inject_residual(_p16(p), _p16(m), _p16(w), streams, width, _p16(products), _p16(out))
    return products, out


def make_hidden(size: int, spec: dict) -> np.ndarray:
    out = np.empty(size, dtype=np.uint16)
    ok = lib().fwo_make_hidden(size, spec["multiplier"], spec["add"], spec["modulus"],
                               spec["center"], spec["divisor"], spec["sparse_stride"], _p16(out))
    if not ok:
        raise ValueError("invalid input specification")
    return out


def topk_total_order(logits, k: int) -> np.ndarray:
    l = _u16(logits)
    ids = np.empty(k, dtype=np.int32)
    if not lib().fwo_topk_total_order(_p16(l), l.size, k, _p32(ids)):
        raise ValueError("invalid top-k request")
    return ids


def route_scores(logits, ids) -> np.ndarray:
    l = _u16(logits)
    i = np.ascontiguousarray(ids, dtype=np.int32)
    out = np.empty(i.size, dtype=np.uint16)
    lib().fwo_route_scores(_p16(l), l.size, _p32(i), i.size, _p16(out))
    return out


def route(weight, hidden, experts: int, width: int, top_k: int, order: int = ORDER_TREE32):
    """(ids, logits, scores): ids in rank order, full bf16 logits, bf16 scores."""
    w, x = _u16(weight), _u16(hidden)
    ids = np.empty(top_k, dtype=np.int32)
    logits = np.empty(experts, dtype=np.uint16)
    scores = np.empty(top_k, dtype=np.uint16)
    if not lib().fwo_route(_p16(w), _p16(x), experts, width, top_k, order, _p32(ids),
                           _p16(logits), _p16(scores)):
        raise ValueError("route rejected its input")
    return ids, logits, scores


def equivalent_topk_order(expected, actual, logits) -> bool:
    e = np.ascontiguousarray(expected, dtype=np.int32)
    a = np.ascontiguousarray(actual, dtype=np.int32)
    l = _u16(logits)
    if e.size != a.size:
        return False
    return bool(lib().fwo_equivalent_topk_order(_p32(e), _p32(a), e.size, _p16(l)))


def expert_bf16(gate_up_weight, down_weight, hidden, hidden_size: int, intermediate: int,
                route_weight: int) -> dict:
    gu_w, d_w, x = _u16(gate_up_weight), _u16(down_weight), _u16(hidden)
    gate_up = np.empty(2 * intermediate, dtype=np.uint16)
    swiglu = np.empty(intermediate, dtype=np.uint16)
    down = np.empty(hidden_size, dtype=np.uint16)
    weighted = np.empty(hidden_size, dtype=np.uint16)
    lib().fwo_expert_bf16(_p16(gu_w), _p16(d_w), _p16(x), hidden_size, intermediate,
                          route_weight, _p16(gate_up), _p16(swiglu), _p16(down), _p16(weighted))
    return {"gate_up": gate_up, "gate": gate_up[:intermediate], "up": gate_up[intermediate:],
            "swiglu": swiglu, "down": down, "weighted_down": weighted}


def mixture_bf16(gate_up_weights, down_weights, hidden, hidden_size: int, intermediate: int,
                 route_weights) -> np.ndarray:
    n = len(gate_up_weights)
    gus = [_u16(a) for a in gate_up_weights]
    dns = [_u16(a) for a in down_weights]
    gu_arr = (_u16p * n)(*[_p16(a) for a in gus])
    dn_arr = (_u16p * n)(*[_p16(a) for a in dns])
    rw = _u16(route_weights)
    ids = np.arange(n, dtype=np.int32)
    x = _u16(hidden)
    out = np.empty(hidden_size, dtype=np.uint16)
    lib().fwo_mixture_bf16(gu_arr, dn_arr, _p16(x), hidden_size, intermediate, _p32(ids),
                           _p16(rw), n, _p16(out))
    return out


CAPTURE_NAMES = ("logits", "ids", "scores", "routed_mixture", "shared_down", "shared_gate_sigmoid",
                 "shared_gate", "shared_up", "shared_swiglu", "shared_gate_logit", "gated_shared",
                 "weighted_down")


def _capture_arrays(shape: dict, lead: tuple) -> dict:
    H, E, K = shape["hidden"], shape["experts"], shape["top_k"]
    Is = shape["shared_intermediate"]
    dims = {"logits": (E,), "ids": (K,), "scores": (K,), "routed_mixture": (H,), "shared_down": (H,),
            "shared_gate_sigmoid": (1,), "shared_gate": (Is,), "shared_up": (Is,),
            "shared_swiglu": (Is,), "shared_gate_logit": (1,), "gated_shared": (H,),
            "weighted_down": (K, H)}
    return {k: np.empty(lead + dims[k], dtype=np.int32 if k == "ids" else np.uint16)
            for k in CAPTURE_NAMES}


def _captures_of(arrays: dict, index: tuple) -> BlockCaptures:
    ptrs = []
    for k in CAPTURE_NAMES:
        a = arrays[k][index] if index else arrays[k]
        ptrs.append(_p32(a) if k == "ids" else _p16(a))
    return BlockCaptures(*ptrs)


def sparse_moe_block(shape: dict, weights: dict, hidden, order: int = ORDER_TREE32) -> dict:
    """One token through a dense-weight block; returns out and captures."""
    s = Shape(shape["hidden"], shape["intermediate"], shape["experts"], shape["top_k"],
              shape["shared_intermediate"])
    arrs = {k: _u16(v) for k, v in weights.items()}
    layer = Layer(*[_p16(arrs[k]) for k in ("router", "gate_up", "down", "shared_gate",
                                            "shared_up", "shared_down", "shared_expert_gate")])
    H = shape["hidden"]
    out = np.empty(H, dtype=np.uint16)
    cap_arrays = _capture_arrays(shape, ())
    cap = _captures_of(cap_arrays, ())
    x = _u16(hidden)
    if not lib().fwo_sparse_moe_block(ctypes.byref(s), ctypes.byref(layer), _p16(x), order,
                                      _p16(out), ctypes.byref(cap)):
        raise ValueError("sparse-MoE block rejected its input")
    cap_arrays["out"] = out
    return cap_arrays


# ---- synthetic workload -------------------------------------------------------------

def synth_tables():
    unit = np.empty(65536, dtype=np.uint16)
    weight = np.empty(65536, dtype=np.uint16)
    lib().fwo_synth_tables(_p16(unit), _p16(weight))
    return unit, weight


def synth_hidden(seed: int, tokens: int, hidden: int, bias_feature: bool = True,
                 first_token: int = 0) -> np.ndarray:
    out = np.empty((tokens, hidden), dtype=np.uint16)
    lib().fwo_synth_hidden(seed, first_token, tokens, hidden, int(bias_feature), _p16(out))
    return out


def synth_tensor(seed: int, layer: int, tensor: int, first: int, count: int) -> np.ndarray:
    out = np.empty(count, dtype=np.uint16)
    lib().fwo_synth_tensor(seed, layer, tensor, first, count, _p16(out))
    return out


def synth_router_bias(seed: int, layer: int, experts: int) -> np.ndarray:
    out = np.empty(experts, dtype=np.uint16)
    lib().fwo_synth_router_bias(seed, layer, experts, _p16(out))
    return out


def _shape(shape: dict) -> Shape:
    return Shape(shape["hidden"], shape["intermediate"], shape["experts"], shape["top_k"],
                 shape["shared_intermediate"])


def _config(seed: int, bias_feature: bool, order: int, threads: int) -> SynthConfig:
    return SynthConfig(seed, int(bias_feature), order, threads)


def default_threads() -> int:
    return max(1, min(16, os.cpu_count() or 1))


def synth_route(shape: dict, seed: int, layer: int, hidden: np.ndarray, bias_feature=True,
                order=ORDER_TREE32, threads: int | None = None):
    h = _u16(hidden)
    T = h.shape[0]
    K, E = shape["top_k"], shape["experts"]
    ids = np.empty((T, K), dtype=np.int32)
    scores = np.empty((T, K), dtype=np.uint16)
    logits = np.empty((T, E), dtype=np.uint16)
    s, c = _shape(shape), _config(seed, bias_feature, order, threads or default_threads())
    if not lib().fwo_synth_route(ctypes.byref(s), ctypes.byref(c), layer, _p16(h), T, _p32(ids),
                                 _p16(scores), _p16(logits)):
        raise ValueError("synthetic route failed")
    return ids, scores, logits


def synth_block_captures(shape: dict, seed: int, layer: int, hidden: np.ndarray, bias_feature=True,
                         order=ORDER_TREE32, threads: int | None = None) -> dict:
    """synth_block with every capture of the block ([T, ...] arrays named as
    CAPTURE_NAMES; weighted_down [T, K, H] in ascending expert id) and "out"."""
    h = _u16(hidden)
    T = h.shape[0]
    arrays = _capture_arrays(shape, (T,))
    caps = (BlockCaptures * T)(*[_captures_of(arrays, (t,)) for t in range(T)])
    out = np.empty((T, shape["hidden"]), dtype=np.uint16)
    s, c = _shape(shape), _config(seed, bias_feature, order, threads or default_threads())
    if not lib().fwo_synth_block_captured(ctypes.byref(s), ctypes.byref(c), layer, _p16(h), T,
                                          _p16(out), caps):
        raise ValueError("synthetic block failed")
    arrays["out"] = out
    return arrays


def synth_block(shape: dict, seed: int, layer: int, hidden: np.ndarray, bias_feature=True,
                order=ORDER_TREE32, threads: int | None = None):
    h = _u16(hidden)
    T = h.shape[0]
    H, K, E = shape["hidden"], shape["top_k"], shape["experts"]
    out = np.empty((T, H), dtype=np.uint16)
    ids = np.empty((T, K), dtype=np.int32)
    scores = np.empty((T, K), dtype=np.uint16)
    logits = np.empty((T, E), dtype=np.uint16)
    s, c = _shape(shape), _config(seed, bias_feature, order, threads or default_threads())
    if not lib().fwo_synth_block(ctypes.byref(s), ctypes.byref(c), layer, _p16(h), T, _p16(out),
                                 _p32(ids), _p16(scores), _p16(logits)):
        raise ValueError("synthetic block failed")
    return out, ids, scores, logits


def synth_step(shape: dict, seed: int, layers: int, hidden: np.ndarray, bias_feature=True,
               order=ORDER_TREE32, threads: int | None = None):
    """Pre-norm residual decode step; returns (r_L, block outputs, ids, scores)."""
    h = _u16(hidden)
    T = h.shape[0]
    H, K = shape["hidden"], shape["top_k"]
    resid = np.empty((T, H), dtype=np.uint16)
    blocks = np.empty((layers, T, H), dtype=np.uint16)
    ids = np.empty((layers, T, K), dtype=np.int32)
    scores = np.empty((layers, T, K), dtype=np.uint16)
    s, c = _shape(shape), _config(seed, bias_feature, order, threads or default_threads())
    if not lib().fwo_synth_step(ctypes.byref(s), ctypes.byref(c), layers, _p16(h), T, _p16(resid),
                                _p16(blocks), _p32(ids), _p16(scores)):
        raise ValueError("synthetic step failed")
    return resid, blocks, ids, scores


def synth_step_timed(shape: dict, seed: int, layers: int, hidden: np.ndarray, bias_feature=True,
                     order=ORDER_TREE32):
    """Single-thread chained step; returns (x_L, seconds spent in block arithmetic)."""
    h = _u16(hidden)
    T = h.shape[0]
    resid = np.empty((T, shape["hidden"]), dtype=np.uint16)
    secs = ctypes.c_double(0.0)
    s, c = _shape(shape), _config(seed, bias_feature, order, 1)
    if not lib().fwo_synth_step_timed(ctypes.byref(s), ctypes.byref(c), layers, _p16(h), T,
                                      _p16(resid), ctypes.byref(secs)):
        raise ValueError("timed synthetic step failed")
    return resid, secs.value


def bench_block(shape: dict, seed: int, layer: int, hidden: np.ndarray, prenorm: bool, warmups: int, runs: int,
                threads: int = 1, bias_feature=True, order=ORDER_TREE32):
    """CPU baseline timing: (seconds per run [runs], outputs of the last run
    [T, H]) for the block of one synthetic layer over the tokens of `hidden`
    (weights generated untimed; see fwo_bench_block)."""
    h = _u16(hidden).reshape(-1, shape["hidden"])
    T = h.shape[0]
    samples = np.zeros(runs, dtype=np.float64)
    out = np.empty((T, shape["hidden"]), dtype=np.uint16)
    s, c = _shape(shape), _config(seed, bias_feature, order, threads)
    if not lib().fwo_bench_block(ctypes.byref(s), ctypes.byref(c), layer, _p16(h), T, int(prenorm), warmups, runs,
                                 samples.ctypes.data_as(ctypes.POINTER(ctypes.c_double)), _p16(out)):
        raise ValueError("block timing failed")
    return samples, out


# ---- the reference's own top-k shim (built from native/topk_shim.cpp) ---------------

_ref_topk = None


def ref_topk_available() -> bool:
    return _REF_TOPK_PATH.is_file()


def ref_torch_topk_bf16(values, k: int) -> np.ndarray:
    """native/topk_shim.cpp:18-44 built here (libstdc++), via its own C ABI."""
    global _ref_topk
    if _ref_topk is None:
        L = ctypes.CDLL(str(_REF_TOPK_PATH))
        L.firewing_torch_topk_bf16.restype = ctypes.c_bool
        L.firewing_torch_topk_bf16.argtypes = [_u16p, _size, _size, ctypes.POINTER(_size)]
        _ref_topk = L
    v = _u16(values)
    out = (_size * k)()
    if not _ref_topk.firewing_torch_topk_bf16(_p16(v), v.size, k, out):
        raise ValueError("top-k shim rejected its input")
    return np.array(list(out), dtype=np.int64)
