"""Checks of the synthetic workload's definition (firewing_amd/csrc/fw_synth.h):
the inverse-normal table behind every seeded weight and input, and the
Zipf(1.1) expert popularity that the router-bias column realises. CPU only."""
import numpy as np

from oracle import fw_oracle as fo

SHAPE = dict(hidden=2048, intermediate=512, experts=512, top_k=10, shared_intermediate=512)
SEED = 0x46495245


def _bf16_of_f64(values: np.ndarray) -> np.ndarray:
    f = values.astype(np.float32).view(np.uint32).astype(np.uint64)
    return ((f + 0x7FFF + ((f >> 16) & 1)) >> 16).astype(np.uint16)


def test_normal_tables_equal_scipy_ndtri():
    # table[u] = bf16(f32(sigma * Phi^-1((u + 0.5) / 65536))) for sigma 1 (inputs)
    # and 0.02 (weights); scipy's ndtri is an independent quantile.
    from scipy.special import ndtri
    unit, weight = fo.synth_tables()
    p = (np.arange(65536, dtype=np.float64) + 0.5) / 65536.0
    assert np.array_equal(unit, _bf16_of_f64(ndtri(p)))
    assert np.array_equal(weight, _bf16_of_f64(0.02 * ndtri(p)))


def test_router_bias_realises_zipf_popularity():
    # Selection frequency by popularity rank over the exact in-model route of
    # seeded tokens, fitted on ranks 3..300 (the two most popular experts
    # saturate) as tests/golden/zipf_calibration.py models it: the exponent is
    # within 0.08 of 1.1 on each of three layers.
    for layer in (0, 7, 31):
        x = fo.synth_hidden(SEED, 2000, SHAPE["hidden"], True, first_token=10000 * layer)
        ids, _, _ = fo.synth_route(SHAPE, SEED, layer, x)
        bias = fo.bf16_to_f32(fo.synth_router_bias(SEED, layer, SHAPE["experts"]))
        by_rank = np.argsort(-bias, kind="stable")
        freq = np.bincount(ids.ravel(), minlength=SHAPE["experts"])[by_rank] / ids.shape[0]
        ranks = np.arange(1, SHAPE["experts"] + 1)
        r, f = ranks[2:300], freq[2:300]
        keep = f > 0
        slope = np.polyfit(np.log(r[keep]), np.log(f[keep]), 1)[0]
        assert abs(-slope - 1.1) < 0.08, (layer, slope)


def test_cpu_baseline_timing_computes_the_same_block():
    # The benchmark's CPU leg (fwo_bench_block) must time the oracle's own
    # block: outputs equal synth_block for one thread, for row-parallel
    # threads (one token) and for token-parallel threads (several tokens).
    shape = dict(hidden=256, intermediate=128, experts=64, top_k=6, shared_intermediate=128)
    x1 = fo.synth_hidden(SEED, 1, shape["hidden"], True, first_token=5)
    x4 = fo.synth_hidden(SEED, 4, shape["hidden"], True, first_token=9)
    ref1 = fo.synth_block(shape, SEED, 3, x1)[0]
    ref4 = fo.synth_block(shape, SEED, 3, x4)[0]
    for threads in (1, 4):
        t, out = fo.bench_block(shape, SEED, 3, x1, prenorm=False, warmups=1, runs=3, threads=threads)
        assert t.shape == (3,) and (t > 0).all()
        assert np.array_equal(out, ref1), threads
        t, out = fo.bench_block(shape, SEED, 3, x4, prenorm=False, warmups=0, runs=2, threads=threads)
        assert np.array_equal(out, ref4), threads
    # with the pre-norm of the chained step
    normed = fo.rms_norm_bf16(x1[0], True)
    ref_n = fo.synth_block(shape, SEED, 3, normed[None])[0]
    _, out = fo.bench_block(shape, SEED, 3, x1, prenorm=True, warmups=0, runs=1, threads=2)
    assert np.array_equal(out, ref_n)
