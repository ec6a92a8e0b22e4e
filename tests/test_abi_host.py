"""CPU checks of the HIP library: it loads, exports every declared entry point,
and its expf restatement equals the platform's glibc expf (Rust's f32::exp on
Linux) on the domains the path uses. No GPU calls."""
import os

import numpy as np
import pytest

from firewing_amd import hip_moe as hm
from oracle import fw_oracle as fo


def test_library_exports_every_header_symbol():
    lib = hm.lib()
    declared = hm.header_symbols()
    assert len(declared) >= 20
    missing = [name for name in declared if not hasattr(lib, name)]
    assert missing == []


def test_python_signatures_cover_the_header():
    assert sorted(hm._SIGNATURES) == hm.header_symbols()


def _compare_expf(x: np.ndarray) -> int:
    ours = hm.expf_host(x).view(np.uint32)
    glibc = fo.expf(x).view(np.uint32)
    nan = np.isnan(fo.expf(x))
    return int(np.count_nonzero((ours != glibc) & ~nan))


def test_expf_matches_glibc_on_every_bf16_argument():
    # SiLU and sigmoid evaluate exp(-g) for bf16 g (src/expert.rs:566, 575).
    bits = (np.arange(65536, dtype=np.uint32) << 16)
    x = bits.view(np.float32)
    assert _compare_expf(x) == 0
    assert _compare_expf(-x) == 0


def test_expf_matches_glibc_on_the_softmax_domain():
    # Softmax evaluates exp(v - max) <= 0 (src/router.rs:250-253): every f32 in
    # [-104, 0] with a stride of 13 bit patterns, plus the range edges.
    lo, hi = np.uint32(0x80000000), np.uint32(0xC2D00000)
    step = 13
    for start in range(int(lo), int(hi), 1 << 26):
        stop = min(int(hi), start + (1 << 26))
        bits = np.arange(start, stop, step, dtype=np.uint64).astype(np.uint32)
        assert _compare_expf(bits.view(np.float32)) == 0, hex(start)
    edges = np.array([0.0, -0.0, -87.3, -88.0, -88.7, -103.9, -103.97, -104.0, -1e-45, np.inf,
                      -np.inf, 88.72, 88.73, np.nan], dtype=np.float32)
    assert _compare_expf(edges) == 0


@pytest.mark.skipif(os.environ.get("FIREWING_SLOW") != "1", reason="exhaustive 2^32 sweep (FIREWING_SLOW=1)")
def test_expf_matches_glibc_on_all_floats():
    for start in range(0, 1 << 32, 1 << 26):
        bits = np.arange(start, start + (1 << 26), dtype=np.uint64).astype(np.uint32)
        assert _compare_expf(bits.view(np.float32)) == 0, hex(start)


def test_invalid_arguments_fail_with_a_message():
    # Host-side validation runs before any device call.
    with pytest.raises(hm.FirewingError, match="invalid top-k"):
        hm.topk_bf16(np.zeros(4, dtype=np.uint16), 0)
    with pytest.raises(hm.FirewingError, match="invalid top-k"):
        hm.topk_bf16(np.zeros(4, dtype=np.uint16), 5)
    with pytest.raises(hm.FirewingError, match="top_k"):
        hm.route(np.zeros(64, dtype=np.uint16), np.zeros(32, dtype=np.uint16), 2, 32, 3)
    with pytest.raises(hm.FirewingError, match="hidden must be"):
        hm.MoeContext(hidden=100, intermediate=32, experts=8, top_k=2, shared_intermediate=32,
                      layers=1)
