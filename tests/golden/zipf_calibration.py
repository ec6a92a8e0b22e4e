#!/usr/bin/env python3
"""Calibrate the router-bias slope of the synthetic workload.

Router logits of the synthetic layers are approximately
N(0, (0.02 * sqrt(H - 1))^2) plus a bias -slope * ln(rank + 1) carried by the
constant input feature x[H-1] = 1.0. This script finds the slope at which the
top-K selection frequency of the popularity ranks 3..300 follows a power law
of exponent -s (Zipf s = 1.1) by Monte Carlo on that logit model; the chosen
value is FW_SYNTH_ZIPF_BIAS_SLOPE in firewing_amd/csrc/fw_synth.h. The two
most popular experts saturate (selected for most tokens), so the fit excludes
them. tests/test_workload.py fits the same exponent on the selections of the
real synthetic layers (the oracle's exact route of seeded tokens).
"""
from __future__ import annotations

import argparse

import numpy as np


def loglog_slope(slope: float, hidden: int, experts: int, top_k: int, samples: int,
                 seed: int = 0) -> float:
    rng = np.random.default_rng(seed)
    sigma = 0.02 * np.sqrt(hidden - 1)
    ranks = np.arange(1, experts + 1)
    logits = rng.standard_normal((samples, experts)) * sigma - slope * np.log(ranks)
    top = np.argpartition(-logits, top_k, axis=1)[:, :top_k]
    freq = np.bincount(top.ravel(), minlength=experts) / samples
    r, f = ranks[2:300], freq[2:300]
    keep = f > 0
    return float(np.polyfit(np.log(r[keep]), np.log(f[keep]), 1)[0])


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--hidden", type=int, default=2048)
    ap.add_argument("--experts", type=int, default=512)
    ap.add_argument("--top-k", type=int, default=10)
    ap.add_argument("--zipf-s", type=float, default=1.1)
    ap.add_argument("--samples", type=int, default=20000)
    args = ap.parse_args()
    lo, hi = 0.2, 1.0
    for _ in range(12):
        mid = 0.5 * (lo + hi)
        s = loglog_slope(mid, args.hidden, args.experts, args.top_k, args.samples)
        if -s < args.zipf_s:
            lo = mid
        else:
            hi = mid
    print(f"bias slope {0.5 * (lo + hi):.3f} gives selection frequency ~ rank^-{args.zipf_s}")


if __name__ == "__main__":
    main()
