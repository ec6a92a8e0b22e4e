"""The compressed expert container and its install path.

Format (tools/build_sequential_shuffle_container.py:143-237): one file of
records, one per (layer, expert); a record is one zstd frame (level 1, content
size written, no checksum) of the expert's source bytes, gate_up [2I, H] then
down [H, I] as bf16, BF16 byte-shuffled (every low byte, then every high
byte), padded with zeros to a 16 KiB page; a JSON manifest lists each record's
identity "layer:expert", offset, compressed and physical bytes and the SHA-256
of the frame and of the source.

Reading follows the reference's miss path (src/compressed_overlap.rs:1426-1560):
a page-aligned read plan per record (src/ngram.rs:940-969 aligned_read_plan),
preads of the physical pages, then decode + unshuffle + install, here on the
GPU straight into the resident banks (MoeContext.install_experts_zstd).

write_container builds a container the way the reference's builder does, from
weights in memory (for synthetic checkpoints); its compressor is the system
libzstd.
"""
from __future__ import annotations

import ctypes
import ctypes.util
import hashlib
import json
import os
from dataclasses import dataclass
from pathlib import Path

import numpy as np

PAGE_BYTES = 16 * 1024  # tools/build_q2_zstd_container.py:40, src/compressed_overlap.rs:29
SEMANTIC = "firewing_amd_bf16_shuffle_zstd1_page_aligned_expert_container"

_zstd = None


def _lib() -> ctypes.CDLL:
    global _zstd
    if _zstd is None:
        z = ctypes.CDLL(ctypes.util.find_library("zstd") or "libzstd.so.1")
        z.ZSTD_compressBound.restype = ctypes.c_size_t
        z.ZSTD_compressBound.argtypes = [ctypes.c_size_t]
        z.ZSTD_isError.restype = ctypes.c_uint
        z.ZSTD_isError.argtypes = [ctypes.c_size_t]
        z.ZSTD_compress.restype = ctypes.c_size_t
        z.ZSTD_compress.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_size_t,
                                    ctypes.c_int]
        _zstd = z
    return _zstd


def shuffle_bf16(source: bytes) -> bytes:
    """Every low byte of the bf16 values, then every high byte."""
    if len(source) % 2:
        raise ValueError("BF16 byte shuffle requires an even byte count")
    a = np.frombuffer(source, dtype=np.uint8)
    return np.concatenate([a[0::2], a[1::2]]).tobytes()


def compress_frame(data: bytes, level: int = 1) -> bytes:
    """One zstd frame with the content size written and no checksum."""
    z = _lib()
    src = np.frombuffer(data, dtype=np.uint8) if data else np.zeros(1, np.uint8)
    cap = z.ZSTD_compressBound(len(data))
    dst = np.empty(cap, dtype=np.uint8)
    n = z.ZSTD_compress(dst.ctypes.data, cap, src.ctypes.data, len(data), level)
    if z.ZSTD_isError(n):
        raise ValueError("zstd compression failed")
    return dst[:n].tobytes()


def expert_source(gate_up: np.ndarray, down: np.ndarray) -> bytes:
    return np.ascontiguousarray(gate_up, dtype=np.uint16).tobytes() + \
        np.ascontiguousarray(down, dtype=np.uint16).tobytes()


def align_up(value: int, alignment: int = PAGE_BYTES) -> int:
    return (value + alignment - 1) & -alignment


@dataclass(frozen=True)
class ReadPlan:
    physical_offset: int
    physical_bytes: int
    logical_offset: int


def aligned_read_plan(offset: int, logical_bytes: int, file_bytes: int, page_bytes: int = PAGE_BYTES) -> ReadPlan:
    """The pages that hold [offset, offset + logical_bytes) of a file of
    file_bytes (src/ngram.rs:940-969)."""
    if logical_bytes <= 0 or page_bytes <= 0 or page_bytes & (page_bytes - 1):
        raise ValueError("invalid aligned read parameters")
    end = offset + logical_bytes
    if offset < 0 or end > file_bytes:
        raise ValueError("aligned read exceeds the file")
    mask = page_bytes - 1
    start = offset & ~mask
    stop = min((end + mask) & ~mask, file_bytes)
    return ReadPlan(start, stop - start, offset - start)


def write_container(path, manifest_path, experts, level: int = 1) -> dict:
    """Write a container of `experts`, an iterable of (layer, expert, gate_up
    [2I*H] bf16, down [H*I] bf16), in the order given; returns the manifest
    (also written to manifest_path)."""
    path, manifest_path = Path(path), Path(manifest_path)
    records = []
    offset = 0
    content = None
    with open(path, "wb") as out:
        for layer, expert, gate_up, down in experts:
            source = expert_source(gate_up, down)
            if content is None:
                content = len(source)
            elif len(source) != content:
                raise ValueError("every expert of a container has the same source size")
            frame = compress_frame(shuffle_bf16(source), level)
            physical = align_up(len(frame))
            out.write(frame)
            out.write(bytes(physical - len(frame)))
            records.append({"identity": f"{layer}:{expert}", "layer": int(layer), "expert": int(expert),
                            "offset": offset, "compressed_bytes": len(frame), "physical_bytes": physical,
                            "frame_sha256": hashlib.sha256(frame).hexdigest(),
                            "source_sha256": hashlib.sha256(source).hexdigest()})
            offset += physical
    manifest = {"schema_version": 1, "semantic": SEMANTIC,
                "codec": {"name": "zstd", "level": level, "frame_content_size": True, "independent_frames": True},
                "exact_transform": "bf16_byte_shuffle", "page_bytes": PAGE_BYTES,
                "source_bytes_per_expert": content or 0, "records": records,
                "container_file": path.name, "physical_bytes": offset,
                "compressed_bytes": sum(r["compressed_bytes"] for r in records)}
    manifest_path.write_text(json.dumps(manifest, indent=1))
    return manifest


class Container:
    """A container opened from its manifest (the container file sits next to it)."""

    def __init__(self, manifest_path):
        manifest_path = Path(manifest_path)
        m = json.loads(manifest_path.read_text())
        if m.get("schema_version") != 1 or m.get("page_bytes") != PAGE_BYTES:
            raise ValueError("unsupported container manifest")
        if m.get("codec", {}).get("name") != "zstd" or m.get("exact_transform") != "bf16_byte_shuffle":
            raise ValueError("container codec is not BF16-shuffled zstd")
        self.path = manifest_path.parent / m["container_file"]
        if "/" in m["container_file"] or m["container_file"] in ("", ".", ".."):
            raise ValueError("container_file must be a plain file name")
        self.file_bytes = self.path.stat().st_size
        self.source_bytes = int(m["source_bytes_per_expert"])
        self.records = {}
        for r in m["records"]:
            if r["identity"] != f"{r['layer']}:{r['expert']}" or r["identity"] in self.records:
                raise ValueError(f"bad or repeated record identity {r['identity']}")
            if r["offset"] % PAGE_BYTES or r["physical_bytes"] != align_up(r["compressed_bytes"]):
                raise ValueError(f"record {r['identity']} is not page-aligned")
            if r["offset"] + r["physical_bytes"] > self.file_bytes:
                raise ValueError(f"record {r['identity']} runs past the container file")
            self.records[r["identity"]] = r
        self.manifest = m

    def read(self, identities, verify: bool = False) -> tuple[bytes, list[int], list[int]]:
        """The frames of `identities` read through page-aligned preads, packed
        back to back: (bytes, offsets, sizes)."""
        parts, offsets, sizes = [], [], []
        at = 0
        fd = os.open(self.path, os.O_RDONLY)
        try:
            for ident in identities:
                r = self.records[ident]
                plan = aligned_read_plan(r["offset"], r["compressed_bytes"], self.file_bytes)
                pages = os.pread(fd, plan.physical_bytes, plan.physical_offset)
                if len(pages) != plan.physical_bytes:
                    raise OSError(f"short read of record {ident}")
                frame = pages[plan.logical_offset:plan.logical_offset + r["compressed_bytes"]]
                if verify and hashlib.sha256(frame).hexdigest() != r["frame_sha256"]:
                    raise ValueError(f"record {ident}: frame hash mismatch")
                parts.append(frame)
                offsets.append(at)
                sizes.append(len(frame))
                at += len(frame)
        finally:
            os.close(fd)
        return b"".join(parts), offsets, sizes

    def install(self, ctx, decoder, layer: int, experts, verify: bool = False) -> None:
        """Read the records of `experts` of `layer` and decode them into the
        context's resident banks."""
        if self.source_bytes != 6 * ctx.I * ctx.H:
            raise ValueError("container experts do not match the context's shape")
        data, offsets, sizes = self.read([f"{layer}:{e}" for e in experts], verify)
        ctx.install_experts_zstd(decoder, layer, experts, data, offsets, sizes)
