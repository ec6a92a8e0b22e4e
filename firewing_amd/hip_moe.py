"""Host-side mirror of the reference crate's MoE entry points over libfirewing_hip_moe.so.

Names and argument meanings follow the Rust functions they replace:

    linear_bf16(weight, input, rows, columns)        src/expert.rs:554-560
    swiglu_bf16(gate, up)                            src/expert.rs:562-571
    sigmoid_bf16(values)                             src/expert.rs:573-576
    topk_bf16(values, k)                             native/topk_shim.cpp:18-44
    route(weight, hidden, experts, width, top_k)     src/router.rs:220-265
    expert_bf16(gate_up, down, hidden, ...)          src/expert.rs:717-751
    MoeContext.install_layer / mixture / sparse_moe_block / moe_step
                                                     src/metal_moe.rs:95-447,
                                                     src/decoder_layer.rs:460-586

Errors come back as ``FirewingError`` carrying the library's message, as the
Rust wrappers map ``false`` to ``Err(String)`` (src/decoder_layer.rs:28-39).
bf16 values are numpy ``uint16`` bit patterns; ``*_dev`` methods take device
addresses (ints, or objects with a ``data_ptr()``).

Importing this module loads the HIP library and fails loudly if it is absent:
there is no CPU fallback.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

import numpy as np

PKG = Path(__file__).resolve().parent
LIB_PATH = PKG / "libfirewing_hip_moe.so"
HEADER = PKG.parent / "include" / "firewing_hip_moe.h"

LOGITS_TREE32 = 0
LOGITS_FOLD = 1

# tensor ids of firewing_hip_read_tensor (fw_synth.h)
ROUTER, GATE_UP, DOWN, SHARED_GATE, SHARED_UP, SHARED_DOWN, SHARED_EXPERT_GATE = range(1, 8)


class FirewingError(RuntimeError):
    pass


class Shape(ctypes.Structure):
    _fields_ = [("hidden", ctypes.c_size_t), ("intermediate", ctypes.c_size_t),
                ("experts", ctypes.c_size_t), ("top_k", ctypes.c_size_t),
                ("shared_intermediate", ctypes.c_size_t), ("layers", ctypes.c_size_t)]


class TensorSpan(ctypes.Structure):
    _fields_ = [("offset", ctypes.c_uint64), ("bytes", ctypes.c_uint64), ("shard", ctypes.c_uint32)]


# the seven tensors of one MoE layer, in resident-bank order (tensor ids 1..7)
LAYER_TENSORS = ("mlp.gate.weight", "mlp.experts.gate_up_proj", "mlp.experts.down_proj",
                 "mlp.shared_expert.gate_proj.weight", "mlp.shared_expert.up_proj.weight",
                 "mlp.shared_expert.down_proj.weight", "mlp.shared_expert_gate.weight")


def layer_prefix(layer: int) -> str:
    """The checkpoint's name prefix of decoder layer `layer`."""
    return f"model.language_model.layers.{layer}"


HYPER_OUTPUTS = ("hyper_input_normed", "mix_down", "mix_down_scaled", "mix_down_silu", "mix_up",
                 "input_mix", "products", "mixed", "inject", "inject_scaled", "inject_sigmoid",
                 "injection_weights")


class HyperOutputs(ctypes.Structure):
    _fields_ = [(k, ctypes.c_void_p) for k in HYPER_OUTPUTS]


VERIFIER_CAPTURES = ("routed_mixture", "shared_gate", "shared_up", "shared_swiglu", "shared_down",
                     "shared_gate_logit", "gated_shared", "weighted_down")


class BlockCaptures(ctypes.Structure):
    _fields_ = [("router_logits", ctypes.c_void_p), ("selected_experts", ctypes.c_void_p),
                ("selected_scores", ctypes.c_void_p), ("routed_mixture", ctypes.c_void_p),
                ("shared_gate_sigmoid", ctypes.c_void_p), ("shared_gate", ctypes.c_void_p),
                ("shared_up", ctypes.c_void_p), ("shared_swiglu", ctypes.c_void_p),
                ("shared_down", ctypes.c_void_p), ("shared_gate_logit", ctypes.c_void_p),
                ("gated_shared", ctypes.c_void_p), ("weighted_down", ctypes.c_void_p)]


class SublayerCaptures(ctypes.Structure):
    _fields_ = [("hyper", HyperOutputs), ("block", BlockCaptures), ("moe_output", ctypes.c_void_p),
                ("mlp_injection_products", ctypes.c_void_p)]


class ZstdFrame(ctypes.Structure):
    _fields_ = [("src_offset", ctypes.c_uint64), ("src_bytes", ctypes.c_uint64), ("content_bytes", ctypes.c_uint64),
                ("dst", ctypes.c_void_p), ("dst_tail", ctypes.c_void_p), ("split", ctypes.c_uint64)]


ZSTD_STATUS = ["ok", "bad magic", "bad frame header", "truncated", "bad block", "too many blocks",
               "bad literals", "bad huffman", "bad fse", "bad sequences", "bad offset", "content size",
               "scratch", "trailing bytes"]


_u16p = ctypes.POINTER(ctypes.c_uint16)
_szp = ctypes.POINTER(ctypes.c_size_t)
_vp = ctypes.c_void_p
_sz = ctypes.c_size_t
_b = ctypes.c_bool

_SIGNATURES = {
    "firewing_hip_last_error": (ctypes.c_char_p, []),
    "firewing_hip_linear_bf16": (_b, [_u16p, _u16p, _sz, _sz, _u16p]),
    "firewing_hip_swiglu_bf16": (_b, [_u16p, _u16p, _sz, _u16p]),
    "firewing_hip_sigmoid_bf16": (_b, [_u16p, _sz, _u16p]),
    "firewing_hip_topk_bf16": (_b, [_u16p, _sz, _sz, _szp]),
    "firewing_hip_route_bf16": (_b, [_u16p, _u16p, _sz, _sz, _sz, _sz, ctypes.c_int, _szp, _u16p, _u16p]),
    "firewing_hip_route_bf16_noalloc": (_b, [_vp, _vp, _sz, _sz, _sz, _sz, ctypes.c_int, _vp, _vp, _vp, _vp]),
    "firewing_hip_expert_bf16": (_b, [_u16p, _u16p, _u16p, _sz, _sz, ctypes.c_uint16, _u16p, _u16p,
                                      _u16p, _u16p]),
    "firewing_hip_create": (_b, [ctypes.POINTER(Shape), ctypes.POINTER(_vp)]),
    "firewing_hip_destroy": (None, [_vp]),
    "firewing_hip_device_name": (ctypes.c_char_p, [_vp]),
    "firewing_hip_install_layer": (_b, [_vp, _sz, _u16p, _u16p, _u16p, _u16p, _u16p, _u16p, _u16p]),
    "firewing_hip_generate_layers": (_b, [_vp, _sz, _sz, ctypes.c_uint64, _b]),
    "firewing_hip_hyper_connection_bf16": (_b, [_u16p, _sz, _u16p, _u16p, _u16p, _vp, _sz, _sz, _sz,
                                                ctypes.POINTER(HyperOutputs)]),
    "firewing_hip_inject_residual_bf16": (_b, [_u16p, _u16p, _u16p, _sz, _sz, _sz, _vp, _u16p]),
    "firewing_hip_install_hyper_connection": (_b, [_vp, _sz, _sz, _sz, _u16p, _u16p, _u16p, _u16p]),
    "firewing_hip_load_hyper_connection_safetensors": (_b, [_vp, _sz, _sz, _sz, ctypes.c_char_p,
                                                            ctypes.c_char_p]),
    "firewing_hip_moe_sublayer": (_b, [_vp, _sz, _u16p, _sz, ctypes.c_int, _u16p,
                                       ctypes.POINTER(SublayerCaptures)]),
    "firewing_hip_moe_sublayer_dev": (_b, [_vp, _sz, _vp, _sz, ctypes.c_int, _vp, _vp]),
    "firewing_hip_safetensors_layer_plan": (_b, [ctypes.POINTER(Shape), ctypes.c_char_p, ctypes.c_char_p,
                                                 ctypes.POINTER(TensorSpan)]),
    "firewing_hip_load_layer_safetensors": (_b, [_vp, _sz, ctypes.c_char_p, ctypes.c_char_p]),
    "firewing_hip_read_tensor": (_b, [_vp, _sz, ctypes.c_int, _sz, _sz, _u16p]),
    "firewing_hip_route": (_b, [_vp, _sz, _u16p, _sz, ctypes.c_int, _szp, _u16p, _u16p]),
    "firewing_hip_mixture_bf16": (_b, [_vp, _sz, _u16p, _szp, _u16p, _sz, _u16p]),
    "firewing_hip_sparse_moe_block": (_b, [_vp, _sz, _u16p, _sz, ctypes.c_int, _u16p,
                                           ctypes.POINTER(BlockCaptures)]),
    "firewing_hip_sparse_moe_block_dev": (_b, [_vp, _sz, _vp, _sz, ctypes.c_int, _vp, _vp]),
    "firewing_hip_prefill_block": (_b, [_vp, _sz, _u16p, _sz, _u16p, ctypes.POINTER(BlockCaptures)]),
    "firewing_hip_prefill_block_dev": (_b, [_vp, _sz, _vp, _sz, _vp, _vp, _vp, _vp]),
    "firewing_hip_prefill_block_profile": (_b, [_vp, _sz, _vp, _sz, _vp, _vp, ctypes.POINTER(ctypes.c_double), _sz]),
    "firewing_hip_moe_step_dev": (_b, [_vp, _vp, _sz, ctypes.c_int, _b, _vp, _vp, _vp, _vp, _vp]),
    "firewing_hip_moe_step": (_b, [_vp, _u16p, _sz, ctypes.c_int, _b, _u16p, _u16p, _vp, _u16p]),
    "firewing_hip_synchronize": (_b, [_vp]),
    "firewing_hip_token_chains": (_sz, [_vp, _sz]),
    "firewing_hip_install_lm_head": (_b, [_vp, _u16p, _sz]),
    "firewing_hip_generate_lm_head": (_b, [_vp, _sz, ctypes.c_uint64]),
    "firewing_hip_load_lm_head_safetensors": (_b, [_vp, ctypes.c_char_p, ctypes.c_char_p, _sz]),
    "firewing_hip_lm_head": (_b, [_vp, _u16p, _sz, _sz, _vp, _szp, _u16p]),
    "firewing_hip_lm_head_dev": (_b, [_vp, _vp, _sz, _sz, _vp, _vp, _vp, _vp]),
    "firewing_hip_set_wait_timeout": (_b, [_vp, ctypes.c_double]),
    "firewing_hip_synth_hidden": (None, [ctypes.c_uint64, ctypes.c_uint32, ctypes.c_uint32,
                                         ctypes.c_uint32, _b, _u16p]),
    "firewing_hip_expf_host": (None, [ctypes.POINTER(ctypes.c_float), ctypes.POINTER(ctypes.c_float), _sz]),
    "firewing_hip_expf_device": (_b, [ctypes.POINTER(ctypes.c_float), ctypes.POINTER(ctypes.c_float), _sz]),
    "firewing_hip_copy_bytes": (_b, [_vp, _vp, _sz, _vp]),
    "firewing_hip_zstd_create": (_vp, [ctypes.c_int, _sz, _sz]),
    "firewing_hip_zstd_destroy": (None, [_vp]),
    "firewing_hip_zstd_decode": (_b, [_vp, _vp, _sz, ctypes.POINTER(ZstdFrame), _sz, _b,
                                      ctypes.POINTER(ctypes.c_uint32)]),
    "firewing_hip_zstd_decode_dev": (_b, [_vp, _vp, _sz, ctypes.POINTER(ZstdFrame), _sz, _b, _vp]),
    "firewing_hip_zstd_status": (_b, [_vp, ctypes.POINTER(ctypes.c_uint32), _sz]),
    "firewing_hip_install_experts_zstd": (_b, [_vp, _vp, _sz, ctypes.POINTER(ctypes.c_uint32), _sz, _vp, _sz,
                                               ctypes.POINTER(ctypes.c_uint64), ctypes.POINTER(ctypes.c_uint64)]),
}

_lib = None


def lib() -> ctypes.CDLL:
    """Load the HIP library (built by firewing_amd.build)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.is_file():
            raise FirewingError(
                f"{LIB_PATH} is missing: build it with `python -m firewing_amd.build` "
                "(there is no CPU fallback)")
        L = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _err() -> FirewingError:
    msg = lib().firewing_hip_last_error()
    return FirewingError(msg.decode() if msg else "unknown failure")


def _call(name: str, *args) -> None:
    if not getattr(lib(), name)(*args):
        raise _err()


def _u16(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.uint16)


def _p16(a: np.ndarray):
    return a.ctypes.data_as(_u16p)


def _pf(a: np.ndarray):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_float))


def _addr(x) -> int | None:
    if x is None:
        return None
    if hasattr(x, "data_ptr"):
        return int(x.data_ptr())
    return int(x)


# ---- stateless entry points ------------------------------------------------------------

def linear_bf16(weight, hidden, rows: int, columns: int) -> np.ndarray:
    w, x = _u16(weight), _u16(hidden)
    if w.size != rows * columns or x.size != columns:
        raise FirewingError("linear_bf16: weight must be [rows, columns] and input [columns]")
    out = np.empty(rows, dtype=np.uint16)
    _call("firewing_hip_linear_bf16", _p16(w), _p16(x), rows, columns, _p16(out))
    return out


def swiglu_bf16(gate, up) -> np.ndarray:
    g, u = _u16(gate), _u16(up)
    if g.size != u.size:
        raise FirewingError("swiglu_bf16: gate and up differ in length")
    out = np.empty(g.size, dtype=np.uint16)
    _call("firewing_hip_swiglu_bf16", _p16(g), _p16(u), g.size, _p16(out))
    return out


def sigmoid_bf16(values) -> np.ndarray:
    v = _u16(values)
    out = np.empty(v.size, dtype=np.uint16)
    _call("firewing_hip_sigmoid_bf16", _p16(v), v.size, _p16(out))
    return out


def topk_bf16(values, k: int) -> np.ndarray:
    v = _u16(values)
    out = (ctypes.c_size_t * max(k, 1))()
    _call("firewing_hip_topk_bf16", _p16(v), v.size, k, out)
    return np.array(list(out)[:k], dtype=np.int64)


def route(weight, hidden, experts: int, width: int, top_k: int, order: int = LOGITS_TREE32):
    """(ids [T, K], scores [T, K] bf16, logits [T, E] bf16) for hidden [T, H] or [H]."""
    w = _u16(weight)
    x = _u16(hidden)
    tokens = x.size // width
    if x.size != tokens * width or w.size != experts * width:
        raise FirewingError("route: weight must be [experts, width] and hidden [tokens, width]")
    ids = (ctypes.c_size_t * (tokens * top_k))()
    scores = np.empty((tokens, top_k), dtype=np.uint16)
    logits = np.empty((tokens, experts), dtype=np.uint16)
    _call("firewing_hip_route_bf16", _p16(w), _p16(x), tokens, experts, width, top_k, order, ids,
          _p16(scores), _p16(logits))
    return np.array(list(ids), dtype=np.int64).reshape(tokens, top_k), scores, logits


def route_noalloc_dev(weight, hidden, tokens: int, experts: int, width: int, top_k: int, ids, scores,
                      logits=None, order: int = LOGITS_TREE32, stream=None) -> None:
    """firewing_hip_route_bf16_noalloc on device addresses (asynchronous on
    `stream`; ids int32 [T, K], -1 for a rejected token)."""
    _call("firewing_hip_route_bf16_noalloc", _addr(weight), _addr(hidden), tokens, experts, width, top_k,
          order, _addr(ids), _addr(scores), _addr(logits), _addr(stream))


def expert_bf16(gate_up_weight, down_weight, hidden, hidden_size: int, intermediate: int,
                route_weight: int) -> dict:
    gu, dn, x = _u16(gate_up_weight), _u16(down_weight), _u16(hidden)
    gate_up = np.empty(2 * intermediate, dtype=np.uint16)
    swiglu = np.empty(intermediate, dtype=np.uint16)
    down = np.empty(hidden_size, dtype=np.uint16)
    weighted = np.empty(hidden_size, dtype=np.uint16)
    _call("firewing_hip_expert_bf16", _p16(gu), _p16(dn), _p16(x), hidden_size, intermediate,
          route_weight, _p16(gate_up), _p16(swiglu), _p16(down), _p16(weighted))
    return {"gate_up": gate_up, "gate": gate_up[:intermediate], "up": gate_up[intermediate:],
            "swiglu": swiglu, "down": down, "weighted_down": weighted}


def synth_hidden(seed: int, tokens: int, hidden: int, bias_feature: bool = True,
                 first_token: int = 0) -> np.ndarray:
    """Seeded benchmark inputs [tokens, hidden] (bf16 bits)."""
    out = np.empty((tokens, hidden), dtype=np.uint16)
    lib().firewing_hip_synth_hidden(seed, first_token, tokens, hidden, bias_feature, _p16(out))
    return out


def expf_host(values) -> np.ndarray:
    x = np.ascontiguousarray(values, dtype=np.float32)
    out = np.empty_like(x)
    lib().firewing_hip_expf_host(_pf(x), _pf(out), x.size)
    return out


def expf_device(values) -> np.ndarray:
    x = np.ascontiguousarray(values, dtype=np.float32)
    out = np.empty_like(x)
    _call("firewing_hip_expf_device", _pf(x), _pf(out), x.size)
    return out


def copy_bytes(dst_ptr: int, src_ptr: int, nbytes: int, stream: int = 0) -> None:
    """Device-to-device copy of nbytes (multiple of 16) by a plain streaming
    kernel, queued on `stream` (a traffic-counter calibration aid)."""
    _call("firewing_hip_copy_bytes", ctypes.c_void_p(dst_ptr), ctypes.c_void_p(src_ptr), nbytes,
          ctypes.c_void_p(stream))


# ---- resident context ------------------------------------------------------------------

def _hyper_arrays(T: int, S: int, W: int, R: int, inject: bool) -> dict:
    dims = {"hyper_input_normed": S * W, "mix_down": R, "mix_down_scaled": R, "mix_down_silu": R,
            "mix_up": S * W, "input_mix": S * W, "products": S * W, "mixed": W, "inject": S,
            "inject_scaled": S, "inject_sigmoid": S, "injection_weights": S}
    return {k: np.empty((T, dims[k]), dtype=np.uint16) for k in HYPER_OUTPUTS
            if inject or k not in ("inject", "inject_scaled", "inject_sigmoid", "injection_weights")}


def _hyper_struct(arrays: dict) -> HyperOutputs:
    o = HyperOutputs()
    for k, a in arrays.items():
        setattr(o, k, a.ctypes.data)
    return o


def hyper_connection(hidden, hc_norm, mix_down_weight, mix_up_weight, inject_weight, streams: int,
                     width: int, lowrank: int) -> dict:
    """run_hyper_connection (src/hyper_connection.rs:412-490) for hidden
    [T, S*W] on the GPU; every output [T, ...] by name (inject_weight None:
    the final mixer, without the injection outputs)."""
    x = _u16(hidden).reshape(-1, streams * width)
    T = x.shape[0]
    out = _hyper_arrays(T, streams, width, lowrank, inject_weight is not None)
    o = _hyper_struct(out)
    inj = _u16(inject_weight) if inject_weight is not None else None
    _call("firewing_hip_hyper_connection_bf16", _p16(x), T, _p16(_u16(hc_norm)), _p16(_u16(mix_down_weight)),
          _p16(_u16(mix_up_weight)), inj.ctypes.data if inj is not None else None, streams, width, lowrank,
          ctypes.byref(o))
    return out


def inject_residual(post_attention, moe_output, injection_weights, streams: int, width: int):
    """(products, layer_output), each [T, S*W], of src/decoder_layer.rs:587-607."""
    post = _u16(post_attention).reshape(-1, streams * width)
    T = post.shape[0]
    moe = _u16(moe_output).reshape(T, width)
    w = _u16(injection_weights).reshape(T, streams)
    products = np.empty_like(post)
    out = np.empty_like(post)
    _call("firewing_hip_inject_residual_bf16", _p16(post), _p16(moe), _p16(w), T, streams, width,
          products.ctypes.data, _p16(out))
    return products, out


def safetensors_layer_plan(path, prefix: str, hidden: int, intermediate: int, experts: int,
                           shared_intermediate: int, top_k: int = 1) -> list[tuple[int, int, int]]:
    """Host only: (offset, bytes, shard ordinal) of the layer's seven tensors in
    LAYER_TENSORS order, validated against the shape; raises FirewingError with
    the reason otherwise."""
    shape = Shape(hidden, intermediate, experts, top_k, shared_intermediate, 1)
    spans = (TensorSpan * 7)()
    _call("firewing_hip_safetensors_layer_plan", ctypes.byref(shape), os.fsencode(str(path)),
          prefix.encode(), spans)
    return [(int(sp.offset), int(sp.bytes), int(sp.shard)) for sp in spans]


class MoeContext:
    """Resident banks of `layers` sparse-MoE layers in HBM (metal_moe::Runtime)."""

    def __init__(self, hidden: int, intermediate: int, experts: int, top_k: int,
                 shared_intermediate: int, layers: int):
        self.shape = Shape(hidden, intermediate, experts, top_k, shared_intermediate, layers)
        self.H, self.I, self.E, self.K = hidden, intermediate, experts, top_k
        self.Is, self.L = shared_intermediate, layers
        self.hc_streams, self.hc_lowrank = 0, 0
        self.vocab = 0
        handle = ctypes.c_void_p()
        _call("firewing_hip_create", ctypes.byref(self.shape), ctypes.byref(handle))
        self._h = handle

    def close(self) -> None:
        if self._h:
            lib().firewing_hip_destroy(self._h)
            self._h = ctypes.c_void_p()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def device_name(self) -> str:
        return lib().firewing_hip_device_name(self._h).decode()

    def install_layer(self, layer: int, router, gate_up, down, shared_gate, shared_up,
                      shared_down, shared_expert_gate) -> None:
        arrs = [_u16(a) for a in (router, gate_up, down, shared_gate, shared_up, shared_down,
                                  shared_expert_gate)]
        H, I, E, Is = self.H, self.I, self.E, self.Is
        want = [E * H, E * 2 * I * H, E * H * I, Is * H, Is * H, H * Is, H]
        if [a.size for a in arrs] != want:
            raise FirewingError("install_layer: tensor sizes do not match the context shape")
        _call("firewing_hip_install_layer", self._h, layer, *[_p16(a) for a in arrs])

    def generate_layers(self, first: int, count: int, seed: int, bias_feature: bool = True) -> None:
        _call("firewing_hip_generate_layers", self._h, first, count, seed, bias_feature)

    def install_hyper_connection(self, layer: int, streams: int, lowrank: int, hc_norm, mix_down_weight,
                                 mix_up_weight, inject_weight) -> None:
        arrs = [_u16(a) for a in (hc_norm, mix_down_weight, mix_up_weight, inject_weight)]
        SW = streams * self.H
        if [a.size for a in arrs] != [SW, lowrank * SW, SW * lowrank, streams * SW]:
            raise FirewingError("install_hyper_connection: tensor sizes do not match the shape")
        _call("firewing_hip_install_hyper_connection", self._h, layer, streams, lowrank, *[_p16(a) for a in arrs])
        self.hc_streams, self.hc_lowrank = streams, lowrank

    def load_hyper_connection_safetensors(self, layer: int, streams: int, lowrank: int, path,
                                          prefix: str | None = None) -> None:
        pre = layer_prefix(layer) if prefix is None else prefix
        _call("firewing_hip_load_hyper_connection_safetensors", self._h, layer, streams, lowrank,
              os.fsencode(str(path)), pre.encode())
        self.hc_streams, self.hc_lowrank = streams, lowrank

    def moe_sublayer(self, layer: int, post_attention, order: int = LOGITS_TREE32, captures: bool = False) -> dict:
        """The in-model MoE sublayer (src/decoder_layer.rs:451-607) on the S
        residual streams post_attention [T, S*H], T <= 4: {"layer_output"}, and
        with captures every hyper-connection output, the block's captures on
        its mixed input ("block": verifier captures included), "moe_output"
        and "mlp_injection_products"."""
        S, R = self.hc_streams, self.hc_lowrank
        post = _u16(post_attention).reshape(-1, S * self.H)
        T = post.shape[0]
        out = np.empty_like(post)
        res = {"layer_output": out}
        cap = None
        if captures:
            hyper = _hyper_arrays(T, S, self.H, R, True)
            block = {"router_logits": np.empty((T, self.E), dtype=np.uint16),
                     "selected_experts": np.empty((T, self.K), dtype=np.uint64),
                     "selected_scores": np.empty((T, self.K), dtype=np.uint16),
                     "shared_gate_sigmoid": np.empty(T, dtype=np.uint16)}
            dims = {"routed_mixture": (self.H,), "shared_gate": (self.Is,), "shared_up": (self.Is,),
                    "shared_swiglu": (self.Is,), "shared_down": (self.H,), "shared_gate_logit": (),
                    "gated_shared": (self.H,), "weighted_down": (self.K, self.H)}
            block.update({k: np.empty((T,) + dims[k], dtype=np.uint16) for k in VERIFIER_CAPTURES})
            moe = np.empty((T, self.H), dtype=np.uint16)
            products = np.empty_like(post)
            cap = SublayerCaptures()
            cap.hyper = _hyper_struct(hyper)
            for k, a in block.items():
                setattr(cap.block, k, a.ctypes.data)
            cap.moe_output = moe.ctypes.data
            cap.mlp_injection_products = products.ctypes.data
            res.update(hyper=hyper, block=block, moe_output=moe, mlp_injection_products=products)
        _call("firewing_hip_moe_sublayer", self._h, layer, _p16(post), T, order, _p16(out),
              ctypes.byref(cap) if cap is not None else None)
        if captures:
            res["block"]["selected_experts"] = res["block"]["selected_experts"].astype(np.int64)
        return res

    def moe_sublayer_dev(self, layer: int, post_attention, tokens: int, layer_output,
                         order: int = LOGITS_TREE32, stream=None) -> None:
        _call("firewing_hip_moe_sublayer_dev", self._h, layer, _addr(post_attention), tokens, order,
              _addr(layer_output), _addr(stream))

    def install_lm_head(self, weight, vocab: int) -> None:
        w = _u16(weight)
        if w.size != vocab * self.H:
            raise FirewingError("install_lm_head: weight size does not match vocab x hidden")
        _call("firewing_hip_install_lm_head", self._h, _p16(w), vocab)
        self.vocab = vocab

    def generate_lm_head(self, vocab: int, seed: int) -> None:
        _call("firewing_hip_generate_lm_head", self._h, vocab, seed)
        self.vocab = vocab

    def load_lm_head_safetensors(self, path, tensor: str, vocab: int) -> None:
        _call("firewing_hip_load_lm_head_safetensors", self._h, os.fsencode(str(path)), tensor.encode(), vocab)
        self.vocab = vocab

    def lm_head(self, hidden, k: int = 20, logits: bool = True) -> dict:
        """logits [T, vocab] (with logits=True), ids [T, k] and values [T, k]
        of the LM head for T <= 4 tokens (src/text_output.rs:273-287)."""
        x = _u16(hidden).reshape(-1, self.H)
        T = x.shape[0]
        out = np.empty((T, self.vocab), dtype=np.uint16) if logits else None
        ids = (ctypes.c_size_t * (T * k))()
        values = np.empty((T, k), dtype=np.uint16)
        _call("firewing_hip_lm_head", self._h, _p16(x), T, k, out.ctypes.data if logits else None, ids,
              _p16(values))
        res = {"ids": np.array(list(ids), dtype=np.int64).reshape(T, k), "values": values}
        if logits:
            res["logits"] = out
        return res

    def lm_head_dev(self, hidden, tokens: int, k: int, ids, values, logits=None, stream=None) -> None:
        _call("firewing_hip_lm_head_dev", self._h, _addr(hidden), tokens, k, _addr(logits), _addr(ids),
              _addr(values), _addr(stream))

    def token_chains(self, tokens: int) -> int:
        """Independent one-token chains a step of `tokens` tokens interleaves
        (1: the multi-token kernel)."""
        return int(lib().firewing_hip_token_chains(self._h, tokens))

    def load_layer_safetensors(self, layer: int, path, prefix: str | None = None) -> None:
        """Install resident layer `layer` from a safetensors checkpoint (a
        .safetensors file or a model.safetensors.index.json); `prefix` names
        the checkpoint layer (default: layer_prefix(layer))."""
        pre = layer_prefix(layer) if prefix is None else prefix
        _call("firewing_hip_load_layer_safetensors", self._h, layer, os.fsencode(str(path)), pre.encode())

    def read_tensor(self, layer: int, tensor: int, first: int, count: int) -> np.ndarray:
        out = np.empty(count, dtype=np.uint16)
        _call("firewing_hip_read_tensor", self._h, layer, tensor, first, count, _p16(out))
        return out

    def route(self, layer: int, hidden, order: int = LOGITS_TREE32):
        x = _u16(hidden).reshape(-1, self.H)
        T = x.shape[0]
        ids = (ctypes.c_size_t * (T * self.K))()
        scores = np.empty((T, self.K), dtype=np.uint16)
        logits = np.empty((T, self.E), dtype=np.uint16)
        _call("firewing_hip_route", self._h, layer, _p16(x), T, order, ids, _p16(scores), _p16(logits))
        return np.array(list(ids), dtype=np.int64).reshape(T, self.K), scores, logits

    def mixture(self, layer: int, hidden, experts, route_weights) -> np.ndarray:
        x = _u16(hidden)
        ex = (ctypes.c_size_t * len(experts))(*[int(e) for e in experts])
        rw = _u16(route_weights)
        out = np.empty(self.H, dtype=np.uint16)
        _call("firewing_hip_mixture_bf16", self._h, layer, _p16(x), ex, _p16(rw), len(experts),
              _p16(out))
        return out

    def sparse_moe_block(self, layer: int, hidden, order: int = LOGITS_TREE32,
                         captures=()) -> dict:
        """The block for T <= 4 tokens. `captures` names verifier captures to
        take as well (any of VERIFIER_CAPTURES; "all" for every one); they are
        returned under their names, [T, ...] (weighted_down [T, K, H] in
        ascending expert id)."""
        x = _u16(hidden).reshape(-1, self.H)
        T = x.shape[0]
        want = VERIFIER_CAPTURES if captures == "all" else tuple(captures)
        unknown = set(want) - set(VERIFIER_CAPTURES)
        if unknown:
            raise ValueError(f"unknown captures {sorted(unknown)}")
        out = np.empty((T, self.H), dtype=np.uint16)
        logits = np.empty((T, self.E), dtype=np.uint16)
        ids = np.empty((T, self.K), dtype=np.uint64)
        scores = np.empty((T, self.K), dtype=np.uint16)
        sig = np.empty(T, dtype=np.uint16)
        dims = {"routed_mixture": (self.H,), "shared_gate": (self.Is,), "shared_up": (self.Is,),
                "shared_swiglu": (self.Is,), "shared_down": (self.H,), "shared_gate_logit": (),
                "gated_shared": (self.H,), "weighted_down": (self.K, self.H)}
        extra = {k: np.empty((T,) + dims[k], dtype=np.uint16) for k in want}
        cap = BlockCaptures(logits.ctypes.data, ids.ctypes.data, scores.ctypes.data,
                            None, sig.ctypes.data)
        for k, a in extra.items():
            setattr(cap, k, a.ctypes.data)
        _call("firewing_hip_sparse_moe_block", self._h, layer, _p16(x), T, order, _p16(out),
              ctypes.byref(cap))
        res = {"out": out, "router_logits": logits, "selected_experts": ids.astype(np.int64),
               "selected_scores": scores, "shared_gate_sigmoid": sig}
        res.update(extra)
        return res

    def sparse_moe_block_dev(self, layer: int, hidden, tokens: int, out, order: int = LOGITS_TREE32,
                             stream=None) -> None:
        _call("firewing_hip_sparse_moe_block_dev", self._h, layer, _addr(hidden), tokens, order,
              _addr(out), _addr(stream))

    def prefill_block(self, layer: int, hidden) -> dict:
        """The many-token block (any T): ids, scores and logits bit-exact, outputs
        within the MFMA accumulation tolerance."""
        x = _u16(hidden).reshape(-1, self.H)
        T = x.shape[0]
        out = np.empty((T, self.H), dtype=np.uint16)
        logits = np.empty((T, self.E), dtype=np.uint16)
        ids = np.empty((T, self.K), dtype=np.uint64)
        scores = np.empty((T, self.K), dtype=np.uint16)
        mixture = np.empty((T, self.H), dtype=np.uint16)
        sig = np.empty(T, dtype=np.uint16)
        cap = BlockCaptures(logits.ctypes.data, ids.ctypes.data, scores.ctypes.data, mixture.ctypes.data,
                            sig.ctypes.data)
        _call("firewing_hip_prefill_block", self._h, layer, _p16(x), T, _p16(out), ctypes.byref(cap))
        return {"out": out, "router_logits": logits, "selected_experts": ids.astype(np.int64),
                "selected_scores": scores, "routed_mixture": mixture, "shared_gate_sigmoid": sig}

    def prefill_block_dev(self, layer: int, hidden, tokens: int, out, ids=None, scores=None,
                          stream=None) -> None:
        _call("firewing_hip_prefill_block_dev", self._h, layer, _addr(hidden), tokens, _addr(out),
              _addr(ids), _addr(scores), _addr(stream))

    def moe_step(self, hidden, order: int = LOGITS_TREE32, bias_feature: bool = True):
        """All resident layers chained; returns (residual [T,H], block outputs [L,T,H],
        ids [L,T,K], scores [L,T,K])."""
        x = _u16(hidden).reshape(-1, self.H)
        T = x.shape[0]
        resid = np.empty((T, self.H), dtype=np.uint16)
        blocks = np.empty((self.L, T, self.H), dtype=np.uint16)
        ids = np.empty((self.L, T, self.K), dtype=np.int32)
        scores = np.empty((self.L, T, self.K), dtype=np.uint16)
        _call("firewing_hip_moe_step", self._h, _p16(x), T, order, bias_feature, _p16(resid),
              _p16(blocks), ids.ctypes.data, _p16(scores))
        return resid, blocks, ids, scores

    PREFILL_PHASES = ("router", "select", "group", "gemm_gate_up", "gemm_down", "combine")

    def prefill_block_profile(self, layer: int, hidden, tokens: int, out, stream=None) -> dict:
        """The device-pointer prefill block timed by phase (microseconds, HIP
        events on the launch stream); waits for it."""
        us = (ctypes.c_double * 6)()
        _call("firewing_hip_prefill_block_profile", self._h, layer, _addr(hidden), tokens, _addr(out),
              _addr(stream), us, 6)
        return dict(zip(self.PREFILL_PHASES, [float(v) for v in us]))

    def moe_step_dev(self, hidden, tokens: int, residual, block_out=None, ids=None, scores=None,
                     order: int = LOGITS_TREE32, bias_feature: bool = True, stream=None) -> None:
        _call("firewing_hip_moe_step_dev", self._h, _addr(hidden), tokens, order, bias_feature,
              _addr(residual), _addr(block_out), _addr(ids), _addr(scores), _addr(stream))

    def synchronize(self) -> None:
        _call("firewing_hip_synchronize", self._h)

    def install_experts_zstd(self, decoder: "ZstdDecoder", layer: int, experts, container: bytes,
                             offsets, sizes) -> None:
        """Decode container frames (host bytes) into experts' resident rows
        (src/compressed_overlap.rs:1541-1553 decode + unshuffle + install)."""
        ex = np.ascontiguousarray(experts, dtype=np.uint32)
        off = np.ascontiguousarray(offsets, dtype=np.uint64)
        sz = np.ascontiguousarray(sizes, dtype=np.uint64)
        src = np.frombuffer(container, dtype=np.uint8) if len(container) else np.zeros(1, np.uint8)
        _call("firewing_hip_install_experts_zstd", self._h, decoder._h, layer,
              ex.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32)), len(ex), src.ctypes.data, len(container),
              off.ctypes.data_as(ctypes.POINTER(ctypes.c_uint64)), sz.ctypes.data_as(ctypes.POINTER(ctypes.c_uint64)))

    def set_wait_timeout(self, seconds: float) -> None:
        """Time limit of each dependency wait inside the persistent kernel."""
        _call("firewing_hip_set_wait_timeout", self._h, float(seconds))


class ZstdDecoder:
    """GPU decoder of independent zstd frames (the compressed expert container,
    src/compressed_overlap.rs), with scratch for `max_frames` frames in flight
    of at most `max_content` decoded bytes each."""

    def __init__(self, max_frames: int, max_content: int, device: int = 0):
        h = lib().firewing_hip_zstd_create(device, max_frames, max_content)
        if not h:
            raise _err()
        self._h = ctypes.c_void_p(h)
        self.max_frames, self.max_content = max_frames, max_content

    def close(self) -> None:
        if self._h:
            lib().firewing_hip_zstd_destroy(self._h)
            self._h = ctypes.c_void_p()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @staticmethod
    def _frames(specs) -> ctypes.Array:
        arr = (ZstdFrame * max(1, len(specs)))()
        for i, (off, size, content, dst, dst_tail, split) in enumerate(specs):
            arr[i] = ZstdFrame(off, size, content, dst, dst_tail, split)
        return arr

    def decode(self, src: bytes, specs, unshuffle: bool) -> np.ndarray:
        """Host-source decode; specs = [(src_offset, src_bytes, content_bytes,
        dst_ptr, dst_tail_ptr, split)]. Returns per-frame statuses; raises if
        any frame failed (statuses are in the exception's `statuses`)."""
        frames = self._frames(specs)
        st = np.zeros(max(1, len(specs)), dtype=np.uint32)
        buf = np.frombuffer(src, dtype=np.uint8) if len(src) else np.zeros(1, np.uint8)
        ok = lib().firewing_hip_zstd_decode(self._h, buf.ctypes.data, len(src), frames, len(specs), unshuffle,
                                            st.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32)))
        if not ok:
            e = _err()
            e.statuses = st[:len(specs)]
            raise e
        return st[:len(specs)]

    def decode_dev(self, src_ptr: int, src_bytes: int, specs, unshuffle: bool, stream=None) -> None:
        """Device-source decode queued on `stream` (asynchronous)."""
        frames = self._frames(specs)
        _call("firewing_hip_zstd_decode_dev", self._h, src_ptr, src_bytes, frames, len(specs), unshuffle,
              _addr(stream))

    def status(self, n: int) -> np.ndarray:
        """Wait for the last call; its per-frame statuses (raises if any failed)."""
        st = np.zeros(max(1, n), dtype=np.uint32)
        ok = lib().firewing_hip_zstd_status(self._h, st.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32)), n)
        if not ok:
            e = _err()
            e.statuses = st[:n]
            raise e
        return st[:n]


def header_symbols() -> list[str]:
    """Every function the public header declares."""
    import re
    text = HEADER.read_text()
    return sorted(set(re.findall(r"\b(firewing_hip_[a-z0-9_]+)\s*\(", text)))
