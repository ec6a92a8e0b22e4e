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


def test_block_captures_compose_to_the_block_output():
    """The oracle's per-token captures are the block's own intermediate vectors:
    they recombine, by the reference's formulas (src/expert.rs:1138-1153,
    src/decoder_layer.rs:532-607), into the block output synth_block gives."""
    shape = dict(hidden=256, intermediate=64, experts=64, top_k=6, shared_intermediate=96)
    x = fo.synth_hidden(11, 3, shape["hidden"], first_token=5)
    cap = fo.synth_block_captures(shape, 11, 0, x)
    out, ids, scores, logits = fo.synth_block(shape, 11, 0, x)
    assert np.array_equal(cap["out"], out) and np.array_equal(cap["ids"], ids)
    assert np.array_equal(cap["scores"], scores) and np.array_equal(cap["logits"], logits)
    for t in range(3):
        assert np.array_equal(cap["shared_swiglu"][t], fo.swiglu_bf16(cap["shared_gate"][t], cap["shared_up"][t]))
        assert cap["shared_gate_sigmoid"][t, 0] == fo.sigmoid_bf16(int(cap["shared_gate_logit"][t, 0]))
        sig = fo.from_bf16(int(cap["shared_gate_sigmoid"][t, 0]))
        gated = [fo.to_bf16(np.float32(sig) * np.float32(fo.from_bf16(int(v)))) for v in cap["shared_down"][t]]
        assert list(cap["gated_shared"][t]) == gated
        mix = fo.to_bf16(0.0)
        mixed = []
        for h in range(shape["hidden"]):
            m = mix
            for n in range(shape["top_k"]):
                m = fo.add_bf16(m, int(cap["weighted_down"][t, n, h]))
            mixed.append(m)
        assert list(cap["routed_mixture"][t]) == mixed
        assert list(out[t]) == [fo.add_bf16(a, b) for a, b in zip(mixed, gated)]
        # weighted rows in ascending expert id, each bf16(down * score) of its expert
        order = np.argsort(ids[t], kind="stable")
        for n, r in enumerate(order):
            e = int(ids[t, r])
            gu = fo.synth_tensor(11, 0, 2, e * 2 * 64 * 256, 2 * 64 * 256)
            dn = fo.synth_tensor(11, 0, 3, e * 256 * 64, 256 * 64)
            ex = fo.expert_bf16(gu, dn, x[t], 256, 64, int(scores[t, r]))
            assert np.array_equal(cap["weighted_down"][t, n], ex["weighted_down"]), (t, n, e)
