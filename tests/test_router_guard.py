"""The matrix-unit router's input guard, checked in IEEE f32 on the CPU.

The many-token router accumulates each 32-column chain of a logit with one
product per matrix-unit step (src/expert.rs:514-552 order); those units flush
denormal products and partial sums to zero. A tile runs there only when every
nonzero |x| and |w| it stages lies in [kPfMxSmall, kPfMxLarge) (bf16 bit
patterns in firewing_amd/csrc/fw_prefill.h); other tiles are recomputed on the
vector units. These tests read the two bounds from the kernel source and check
the property the guard relies on: inside the range every product is exact and
normal, every partial sum of a chain is zero or normal, and a chain of H / 32
= 64 terms stays finite.
"""
import re
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[1]
F32_MIN_NORMAL = np.float32(2.0 ** -126)


def kernel_bound(name: str) -> int:
    text = (ROOT / "firewing_amd" / "csrc" / "fw_prefill.h").read_text()
    m = re.search(rf"constexpr uint16_t {name} = (0x[0-9A-Fa-f]+);", text)
    assert m, name
    return int(m.group(1), 16)


def bf16_values(bits: np.ndarray) -> np.ndarray:
    return (bits.astype(np.uint32) << 16).view(np.float32)


def guarded_magnitudes() -> np.ndarray:
    """Every positive bf16 magnitude the guard lets through."""
    lo, hi = kernel_bound("kPfMxSmall"), kernel_bound("kPfMxLarge")
    return bf16_values(np.arange(lo, hi, dtype=np.uint16))


def test_bounds_are_the_documented_powers_of_two():
    assert bf16_values(np.array([kernel_bound("kPfMxSmall")], np.uint16))[0] == np.float32(2.0 ** -55)
    assert bf16_values(np.array([kernel_bound("kPfMxLarge")], np.uint16))[0] == np.float32(2.0 ** 57)


def test_products_at_the_range_edges_are_exact_and_normal():
    mags = guarded_magnitudes()
    edge = np.concatenate([mags[:256], mags[-256:]])  # two full binades at each end
    a = edge[:, None].astype(np.float32)
    b = edge[None, :].astype(np.float32)
    prod32 = a * b
    prod64 = a.astype(np.float64) * b.astype(np.float64)
    assert np.array_equal(prod32.astype(np.float64), prod64)  # bf16 x bf16 fits 24 bits
    assert np.abs(prod32).min() >= F32_MIN_NORMAL
    assert np.isfinite(prod32).all()


def test_partial_sums_near_the_lower_edge_are_zero_or_normal():
    """Chains of products of the smallest guarded magnitudes with random signs
    cancel often; every partial sum stays a multiple of the product grid, so a
    nonzero one is at least 2^-125."""
    rng = np.random.default_rng(7)
    mags = guarded_magnitudes()[:512]  # the four smallest binades
    n_chains, terms = 20000, 64
    x = rng.choice(mags, (n_chains, terms)) * rng.choice([-1.0, 1.0], (n_chains, terms)).astype(np.float32)
    w = rng.choice(mags, (n_chains, terms)) * rng.choice([-1.0, 1.0], (n_chains, terms)).astype(np.float32)
    acc = np.zeros(n_chains, np.float32)
    zeros = 0
    smallest = np.float32(np.inf)
    for j in range(terms):
        acc = (acc + (x[:, j] * w[:, j]).astype(np.float32)).astype(np.float32)
        nz = acc != 0
        zeros += int((~nz).sum())
        if nz.any():
            smallest = min(smallest, np.abs(acc[nz]).min())
    assert zeros > 0  # exact cancellations happen, and are zeros, not denormals
    assert smallest >= np.float32(2.0 ** -125)


def test_longest_chain_at_the_upper_edge_is_finite():
    top = guarded_magnitudes()[-1]
    acc = np.float32(0.0)
    for _ in range(64):
        acc = np.float32(acc + np.float32(top * top))
    assert np.isfinite(acc) and acc < np.float32(2.0 ** 121)
