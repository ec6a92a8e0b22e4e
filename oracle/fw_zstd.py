"""CPU checker of the compressed expert container path. Test infrastructure:
only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline use it, never
the product.

- shuffle_bf16 / unshuffle_bf16 restate the container's BF16 byte transform
  (tools/analyze_sequential_q2_zstd_oracle.py:33-46; the reader's inverse,
  src/compressed_overlap.rs:1385-1395), pinned by the reference's own vector
  0102030405060708 -> 0103050702040608
  (tests/test_analyze_sequential_q2_zstd_oracle.py:14-19).
- zstd itself is a third-party dependency: the reference decodes with the zstd
  crate 0.13.3 (zstd-sys 2.0.16+zstd.1.5.7, Cargo.lock) and its container was
  written by python-zstandard's ZstdCompressor(level=1), content size written,
  no checksum (tools/build_sequential_shuffle_container.py:147,166-167). The
  format (RFC 8878) fixes the decoded bytes of a frame, so any conforming
  decoder is an exact oracle; this module binds the system libzstd
  (libzstd.so.1) through ctypes to make frames and to decode them. Every check
  built on it is a round trip: decode(compress(x)) == x.
"""
from __future__ import annotations

import ctypes
import ctypes.util

import numpy as np

_z = None

# ZSTD_cParameter values (zstd.h, stable API)
_C_COMPRESSION_LEVEL = 100
_C_WINDOW_LOG = 101
_C_CONTENT_SIZE_FLAG = 200
_C_CHECKSUM_FLAG = 201


def _lib() -> ctypes.CDLL:
    global _z
    if _z is None:
        name = ctypes.util.find_library("zstd") or "libzstd.so.1"
        z = ctypes.CDLL(name)
        z.ZSTD_versionNumber.restype = ctypes.c_uint
        z.ZSTD_compressBound.restype = ctypes.c_size_t
        z.ZSTD_compressBound.argtypes = [ctypes.c_size_t]
        z.ZSTD_isError.restype = ctypes.c_uint
        z.ZSTD_isError.argtypes = [ctypes.c_size_t]
        z.ZSTD_createCCtx.restype = ctypes.c_void_p
        z.ZSTD_freeCCtx.argtypes = [ctypes.c_void_p]
        z.ZSTD_CCtx_setParameter.restype = ctypes.c_size_t
        z.ZSTD_CCtx_setParameter.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int]
        z.ZSTD_compress2.restype = ctypes.c_size_t
        z.ZSTD_compress2.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p,
                                     ctypes.c_size_t]
        z.ZSTD_decompress.restype = ctypes.c_size_t
        z.ZSTD_decompress.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_size_t]
        _z = z
    return _z


def version() -> str:
    v = _lib().ZSTD_versionNumber()
    return f"{v // 10000}.{v // 100 % 100}.{v % 100}"


def compress(data: bytes, level: int = 1, checksum: bool = False, content_size: bool = True,
             window_log: int = 0) -> bytes:
    """One zstd frame of `data` (libzstd ZSTD_compress2)."""
    z = _lib()
    src = np.frombuffer(data, dtype=np.uint8) if len(data) else np.zeros(1, np.uint8)
    cap = z.ZSTD_compressBound(len(data))
    dst = np.empty(cap, dtype=np.uint8)
    c = z.ZSTD_createCCtx()
    try:
        for param, value in ((_C_COMPRESSION_LEVEL, level), (_C_CHECKSUM_FLAG, int(checksum)),
                             (_C_CONTENT_SIZE_FLAG, int(content_size)), (_C_WINDOW_LOG, window_log)):
            if z.ZSTD_isError(z.ZSTD_CCtx_setParameter(c, param, value)):
                raise ValueError(f"zstd parameter {param}={value} rejected")
        n = z.ZSTD_compress2(c, dst.ctypes.data, cap, src.ctypes.data, len(data))
        if z.ZSTD_isError(n):
            raise ValueError("zstd compression failed")
    finally:
        z.ZSTD_freeCCtx(c)
    return dst[:n].tobytes()


def decompress(frame: bytes, size: int) -> bytes:
    """Decode one frame of exactly `size` bytes (libzstd ZSTD_decompress)."""
    z = _lib()
    src = np.frombuffer(frame, dtype=np.uint8)
    dst = np.empty(max(1, size), dtype=np.uint8)
    n = z.ZSTD_decompress(dst.ctypes.data, size, src.ctypes.data, len(frame))
    if z.ZSTD_isError(n) or n != size:
        raise ValueError("zstd decompression failed")
    return dst[:size].tobytes()


def shuffle_bf16(source: bytes) -> bytes:
    """Every low byte, then every high byte (analyze_sequential_q2_zstd_oracle.py:33-36)."""
    if len(source) % 2:
        raise ValueError("BF16 byte shuffle requires an even byte count")
    a = np.frombuffer(source, dtype=np.uint8)
    return np.concatenate([a[0::2], a[1::2]]).tobytes()


def unshuffle_bf16(shuffled: bytes) -> bytes:
    """The inverse (compressed_overlap.rs:1385-1395)."""
    if len(shuffled) % 2:
        raise ValueError("BF16 byte unshuffle requires an even byte count")
    a = np.frombuffer(shuffled, dtype=np.uint8)
    half = len(a) // 2
    out = np.empty_like(a)
    out[0::2] = a[:half]
    out[1::2] = a[half:]
    return out.tobytes()


def expert_frame(gate_up: np.ndarray, down: np.ndarray, level: int = 1) -> tuple[bytes, bytes]:
    """An expert's container frame as the reference's builder writes it: source
    = gate_up bytes + down bytes (bf16), shuffled, zstd level 1
    (build_sequential_shuffle_container.py:156-167). Returns (source, frame)."""
    source = np.ascontiguousarray(gate_up, dtype=np.uint16).tobytes() + \
        np.ascontiguousarray(down, dtype=np.uint16).tobytes()
    return source, compress(shuffle_bf16(source), level=level)
