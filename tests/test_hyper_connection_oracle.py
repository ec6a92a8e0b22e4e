"""Pins of the oracle's hyper-connection (src/hyper_connection.rs) and the
block's injection into the residual streams (src/decoder_layer.rs:587-607).
CPU only.

The reference's hash-only hyper-connection fixture needs the checkpoint's
weights, so the pins are: the reference's own unit tests
(src/hyper_connection.rs:660-679, tests/test_generate_ple_fixture.py:28-33),
exact sums, and an independent evaluation of the square-sum cascade's order
on inputs where every other order gives a different f32 result.
"""
import numpy as np
import pytest

from oracle import fw_oracle as fo

S, W, R = 4, 2560, 320  # src/hyper_connection.rs:13-16


def f32(x):
    return np.float32(x)


def test_grouped_rms_is_independent_per_stream():
    # src/hyper_connection.rs:664-671: ones in, zero weight -> ones out
    ones = np.full(S * W, fo.to_bf16(1.0), dtype=np.uint16)
    out = fo.grouped_rms(ones, np.zeros(S * W, dtype=np.uint16), S, W)
    assert np.all(out == fo.to_bf16(1.0))
    # tests/test_generate_ple_fixture.py:28-33: stream s holds s + 1 -> ones
    values = np.concatenate([np.full(W, fo.to_bf16(float(s + 1)), dtype=np.uint16) for s in range(S)])
    out = fo.grouped_rms(values, np.zeros(S * W, dtype=np.uint16), S, W)
    assert np.all(out == fo.to_bf16(1.0))


def test_four_stream_mean_uses_sequential_reduction():
    # src/hyper_connection.rs:673-678
    assert fo.stream_mean([1.0e8, 1.0, -1.0e8, 1.0]) == 0.25


@pytest.mark.parametrize("n", [1, 3, 4, 15, 16, 17, 63, 64, 65, 255, 256, 257, 1023, 1024, 2560, 4099, 10240, 70001])
def test_square_sum_is_exact_on_small_integers(n):
    # every partial sum is an integer below 2^24: any order gives the exact
    # sum, so a dropped, repeated or wrong element fails
    rng = np.random.default_rng(n)
    v = rng.integers(-7, 8, size=n).astype(np.float32)
    assert fo.inner_square_sum(v) == float((v.astype(np.int64) ** 2).sum())


def cascade_by_structure(v: np.ndarray) -> np.float32:
    """The cascade written from its structure: 16 chains c = 4r + l take every
    16th element (offset c) of the first 16 * (n // 16) elements; a chain's
    squares are summed in runs of `step` terms, runs accumulate into blocks of
    `step` runs, blocks into level 3; terms after the last full run, the
    levels, the 4-element vectors past the chains (into register 0) and the
    registers are then folded as the reduction does, lanes last, after the
    scalar tail."""
    n = v.size
    vectors, groups = n // 4, n // 16
    ceil_log2 = 0 if groups <= 1 else int(groups - 1).bit_length()
    power = max(4, ceil_log2 // 4)
    step = 1 << power
    full_runs = groups // step

    def seq(terms, start=f32(0.0)):
        acc = start
        for t in terms:
            acc = f32(acc + t)
        return acc

    chain = np.zeros((4, 4), dtype=np.float32)  # [register][lane]
    for r in range(4):
        for lane in range(4):
            c = 4 * r + lane
            sq = [f32(x * x) for x in v[c:16 * groups:16]]
            runs = [seq(sq[k * step:(k + 1) * step]) for k in range(full_runs)]
            # level 1 holds the runs since the last multiple of step^2, level 2
            # the level-1 blocks since the last multiple of step^3, level 3 the rest
            lv = [f32(0.0)] * 4
            for k, run in enumerate(runs, start=1):
                lv[1] = f32(lv[1] + run)
                if k % step == 0:
                    lv[2] = f32(lv[2] + lv[1])
                    lv[1] = f32(0.0)
                    if k % (step * step) == 0:
                        lv[3] = f32(lv[3] + lv[2])
                        lv[2] = f32(0.0)
            lv[0] = seq(sq[full_runs * step:])
            chain[r, lane] = f32(f32(f32(lv[0] + lv[1]) + lv[2]) + lv[3])
    for vec in range(groups * 4, vectors):
        for lane in range(4):
            chain[0, lane] = f32(chain[0, lane] + f32(v[vec * 4 + lane] * v[vec * 4 + lane]))
    lanes = [seq(chain[1:, lane], chain[0, lane]) for lane in range(4)]
    result = seq([f32(x * x) for x in v[vectors * 4:]])
    return seq(lanes, result)


def square_sum_in_lanes(v: np.ndarray, lanes: int) -> np.float32:
    """A plain `lanes`-wide vector order (AVX2: 8, AVX-512: 16): lane sums,
    then the scalar tail, then the lanes in order."""
    n = v.size
    acc = np.zeros(lanes, dtype=np.float32)
    for i in range(0, n - n % lanes, lanes):
        acc = (acc + v[i:i + lanes] * v[i:i + lanes]).astype(np.float32)
    folded = f32(0.0)
    for x in v[n - n % lanes:]:
        folded = f32(folded + f32(x * x))
    for lane in acc:
        folded = f32(folded + lane)
    return folded


@pytest.mark.parametrize("n", [2560, 2560 + 7, 16 * 16 * 16 + 48, 16 * 256 * 3 + 20, 16 * 4096 + 16 * 17 + 9])
def test_square_sum_order_matches_its_structure(n):
    # Over eight draws the oracle equals the structural evaluation every time,
    # and each plausible mistake (one sequential chain, an 8- or 16-lane
    # order, registers and lanes transposed) differs in at least one draw.
    rng = np.random.default_rng(1000 + n)
    differs = {"sequential": False, "lanes8": False, "lanes16": False, "transposed": False}
    for _ in range(8):
        v = (rng.standard_normal(n) * np.exp2(rng.integers(-6, 7, size=n))).astype(np.float32)
        got = fo.inner_square_sum(v)
        assert got == float(cascade_by_structure(v))
        sequential = f32(0.0)
        for x in v:
            sequential = f32(sequential + f32(x * x))
        m = 16 * (n // 16)
        t = v.copy()
        t[:m] = v[:m].reshape(-1, 4, 4).transpose(0, 2, 1).reshape(-1)
        differs["sequential"] |= got != float(sequential)
        differs["lanes8"] |= got != float(square_sum_in_lanes(v, 8))
        differs["lanes16"] |= got != float(square_sum_in_lanes(v, 16))
        differs["transposed"] |= got != float(cascade_by_structure(t))
    assert all(differs.values()), differs


def test_hyper_connection_outputs_compose():
    # small shape, random weights: each output from the previous ones by the
    # reference's formulas (src/hyper_connection.rs:412-490)
    s, w, r = 4, 96, 32
    rng = np.random.default_rng(5)

    def rand(n, scale):
        return fo.bf16_array(rng.standard_normal(n) * scale)

    x, norm = rand(s * w, 1.0), rand(s * w, 0.1)
    down, up, inj = rand(r * s * w, 0.05), rand(s * w * r, 0.05), rand(s * s * w, 0.05)
    o = fo.hyper_connection(x, norm, down, up, inj, s, w, r)
    assert np.array_equal(o["hyper_input_normed"], fo.grouped_rms(x, norm, s, w))
    assert np.array_equal(o["mix_down"], fo.linear_bf16(down, o["hyper_input_normed"], r, s * w))
    assert np.array_equal(o["mix_down_scaled"], fo.bf16_array(fo.bf16_to_f32(o["mix_down"]) / 4))
    assert np.array_equal(o["mix_down_silu"], np.array([fo.swiglu_bf16([gb], [fo.to_bf16(1.0)])[0]
                                                        for gb in o["mix_down_scaled"]], dtype=np.uint16))
    assert np.array_equal(o["mix_up"], fo.linear_bf16(up, o["mix_down_silu"], s * w, r))
    assert np.array_equal(o["input_mix"], np.array([fo.sigmoid_bf16(int(b)) for b in o["mix_up"]], dtype=np.uint16))
    prod = fo.bf16_to_f32(o["input_mix"]) * fo.bf16_to_f32(o["hyper_input_normed"])
    assert np.array_equal(o["products"], fo.bf16_array(prod.astype(np.float32)))
    p = fo.bf16_to_f32(o["products"]).reshape(s, w)
    mean = [fo.to_bf16(f32(f32(f32(f32(f32(0) + p[0, c]) + p[1, c]) + p[2, c]) + p[3, c]) / f32(4)) for c in range(w)]
    assert list(o["mixed"]) == mean
    assert np.array_equal(o["inject"], fo.linear_bf16(inj, o["hyper_input_normed"], s, s * w))
    assert np.array_equal(o["inject_scaled"], fo.bf16_array(fo.bf16_to_f32(o["inject"]) / 4))
    sig = [fo.sigmoid_bf16(int(b)) for b in o["inject_scaled"]]
    assert list(o["inject_sigmoid"]) == sig
    assert list(o["injection_weights"]) == [fo.to_bf16(2.0 * fo.from_bf16(b)) for b in sig]


def test_inject_residual():
    s, w = 4, 64
    rng = np.random.default_rng(6)
    post = fo.bf16_array(rng.standard_normal(s * w))
    moe = fo.bf16_array(rng.standard_normal(w))
    weights = fo.bf16_array([0.5, 1.25, 1.9921875, 0.0078125])
    products, out = fo.inject_residual(post, moe, weights, s, w)
    for i in range(s):
        ref_p = fo.bf16_array(fo.bf16_to_f32(moe) * np.float32(fo.from_bf16(int(weights[i]))))
        assert np.array_equal(products[i * w:(i + 1) * w], ref_p)
        assert list(out[i * w:(i + 1) * w]) == [fo.add_bf16(int(a), int(b)) for a, b in
                                                zip(post[i * w:(i + 1) * w], ref_p)]
