"""Pins the CPU oracle against the reference's own known answers.

Every test names the reference test or fixture it restates. None retypes the
oracle's formula: each checks a value fixed by the reference's tests or
fixtures, by the reference's own top-k source built here (oracle/_ref), or by
exact arithmetic.
"""
import hashlib
import struct

import numpy as np
import pytest

from oracle import fw_oracle as fo


def bf16(values):
    return fo.bf16_array(values)


def f32(bits):
    return [float(v) for v in fo.bf16_to_f32(np.asarray(bits, dtype=np.uint16))]


def sha_bf16(bits) -> str:
    return hashlib.sha256(np.ascontiguousarray(bits, dtype="<u2").tobytes()).hexdigest()


# ---- R1 to_bf16 / from_bf16 ---------------------------------------------------------

def test_bf16_conversion_matches_known_value():
    # src/router.rs:416-418
    assert fo.from_bf16(fo.to_bf16(0.1)) == np.float32(0.100097656)


def test_capture_hash_is_over_little_endian_bf16(golden):
    # tests/test_generate_expert_fixture.py:29-35
    assert sha_bf16(bf16([1.0, -2.0])) == golden["capture_hash_bf16_one_minus_two"]


def test_to_bf16_rounds_half_to_even_and_wraps_like_rust():
    # Closed forms of bits + 0x7fff + lsb >> 16 (src/expert.rs:315-318).
    def f(bits):
        return struct.unpack("<f", struct.pack("<I", bits))[0]
    assert fo.to_bf16(f(0x3f808000)) == 0x3f80  # tie, even stays
    assert fo.to_bf16(f(0x3f818000)) == 0x3f82  # tie, odd rounds up
    assert fo.to_bf16(f(0x3f808001)) == 0x3f81
    assert fo.to_bf16(f(0x7f7fffff)) == 0x7f80  # max finite rounds to +inf
    assert fo.to_bf16(f(0xffffffff)) == 0x0000  # u32 wrapping_add: all-ones NaN wraps to +0
    assert fo.to_bf16(f(0x7fc00001)) == 0x7fc0


# ---- R2 make_hidden -------------------------------------------------------------------

def test_affine_mod_input_is_deterministic_bf16():
    # tests/test_generate_router_fixture.py:9-18
    spec = {"multiplier": 3, "add": 1, "modulus": 7, "center": 3, "divisor": 2, "sparse_stride": 1}
    assert f32(fo.make_hidden(5, spec)) == [-1.0, 0.5, -1.5, 0.0, 1.5]
    spec["sparse_stride"] = 2
    assert f32(fo.make_hidden(5, spec)) == [-1.0, 0.0, -1.5, 0.0, 1.5]


def test_committed_input_specs_match_hashes(golden):
    # src/router.rs:421-433 and src/expert.rs:1266-1274
    for case in golden["router"]["cases"]:
        assert sha_bf16(fo.make_hidden(2560, case["input_spec"])) == case["input_bf16_sha256"]
    case = golden["expert"]["case"]
    assert sha_bf16(fo.make_hidden(2560, case["input_spec"])) == case["input_bf16_sha256"]
    sm = golden["sparse_moe"]
    assert sha_bf16(fo.make_hidden(2560, sm["input_spec"])) == sm["input_bf16_sha256"]


def test_invalid_input_spec_is_rejected():
    # src/expert.rs:342-344
    with pytest.raises(ValueError):
        fo.make_hidden(4, {"multiplier": 1, "add": 0, "modulus": 0, "center": 0, "divisor": 1,
                           "sparse_stride": 1})


# ---- R3 / R4 dot orders ---------------------------------------------------------------

def _lcg_values():
    # src/expert.rs:1247-1263
    state = 25
    out = []
    for _ in range(128):
        state = (state * 1664525 + 1013904223) & 0xFFFFFFFF
        raw = ((state >> 8) % 65535) - 32768
        out.append(fo.to_bf16(np.float32(raw) / np.float32(64.0)))
    return np.array(out, dtype=np.uint16)


def test_vector_dot_reduction_is_not_a_forward_sum():
    # src/expert.rs:1247-1263: tree 0x48e4807c, forward fold 0x48e4807e
    values = _lcg_values()
    left, right = values[:64], values[64:]
    tree = np.float32(fo.dot_tree32(left, right)).view(np.uint32)
    fold = np.float32(fo.dot_fold(left, right)).view(np.uint32)
    assert int(tree) == 0x48E4807C
    assert int(fold) == 0x48E4807E


def test_tree32_is_exact_when_every_partial_sum_is_exact():
    # Small integers: every product and partial sum is exact in f32, so any
    # summation order must return the exact integer dot product.
    rng = np.random.default_rng(7)
    for n in (32, 64, 96, 2048, 40, 45):
        a = rng.integers(-8, 9, n)
        b = rng.integers(-8, 9, n)
        exact = float(np.dot(a, b))
        assert fo.dot_tree32(bf16(a), bf16(b)) == exact
        assert fo.dot_fold(bf16(a), bf16(b)) == exact


def test_tree32_pairs_chains_in_the_reference_tree():
    # Column j of each 32-block feeds chain j; the tree adds chain j+16 into j,
    # then j+8, then j+4, then (a0+a1)+(a2+a3) (src/expert.rs:536-545). With a
    # 2^24 term, adding 1.0 to it is lost (ties to even) while adding 2.0 is
    # exact, so where the 1.0 terms meet decides the result.
    big = 16777216.0
    ones = bf16([1.0] * 32)

    def vec(entries):
        v = np.zeros(32)
        for index, value in entries.items():
            v[index] = value
        return bf16(v)

    # chains 1 and 17 pair first (1 + 1 = 2), then meet the 2^24 of chain 0
    # at (a0 + a1): exact. The fold meets 2^24 first and loses both.
    v = vec({0: big, 1: 1.0, 17: 1.0})
    assert fo.dot_tree32(v, ones) == big + 2
    assert fo.dot_fold(v, ones) == big
    # chain 16 pairs with chain 0 first: 2^24 + 1 is lost there.
    v = vec({0: big, 16: 1.0, 1: 1.0})
    assert fo.dot_tree32(v, ones) == big
    # chain 31 reaches a3 (31 -> 15 -> 7 -> 3); chains 1 and 2 meet it
    # one at a time in (a0+a1)+(a2+a3), so both are lost; the fold adds
    # 1 + 1 first and keeps them.
    v = vec({31: big, 1: 1.0, 2: 1.0})
    assert fo.dot_tree32(v, ones) == big
    assert fo.dot_fold(v, ones) == big + 2


def test_negative_zero_sum_leaves_as_positive_zero():
    # src/expert.rs:543: the tail add always runs, so a -0.0 block sum
    # becomes +0.0 before rounding to bf16.
    neg = bf16([-1.0] * 32)
    zero = bf16([0.0] * 32)
    assert np.float32(fo.dot_tree32(neg, zero)).view(np.uint32) == 0
    # the fold keeps -0.0 + (-0.0) ... starting from +0.0: stays +0.0 too.
    assert np.float32(fo.dot_fold(neg, zero)).view(np.uint32) == 0


# ---- R6 / R7 / R10 expert -------------------------------------------------------------

def test_tiny_expert_equation_rounds_each_bf16_boundary():
    # src/expert.rs:1227-1244 and tests/test_generate_expert_fixture.py:9-27
    hidden = bf16([1.0, -2.0])
    gate_up_w = bf16([1.0, 2.0, 0.5, -0.5, 2.0, 0.0, -1.0, 1.0])
    gate_up = fo.linear_bf16(gate_up_w, hidden, 4, 2)
    assert f32(gate_up) == [-3.0, 1.5, 2.0, -3.0]
    activated = fo.swiglu_bf16(gate_up[:2], gate_up[2:])
    down_w = bf16([1.0, 0.0, 0.0, 1.0])
    assert np.array_equal(fo.linear_bf16(down_w, activated, 2, 2), activated)
    out = fo.expert_bf16(gate_up_w, down_w, hidden, 2, 2, fo.to_bf16(0.5))
    assert np.array_equal(out["down"], activated)
    # weighted = bf16(down * 0.5) is exact for bf16 down
    assert f32(out["weighted_down"]) == [v * 0.5 for v in f32(activated)]
    # silu(-3) * 2 and silu(1.5) * (-3), each bf16-rounded twice
    silu = [-3.0 / (1.0 + np.exp(3.0)), 1.5 / (1.0 + np.exp(-1.5))]
    expect = [silu[0] * 2.0, silu[1] * -3.0]
    assert np.allclose(f32(activated), expect, rtol=2 ** -7)


def test_silu_lut_preserves_cpu_bf16_boundary_for_every_finite_gate():
    # src/metal_moe.rs:669-680, exhaustive over the 65,536 gate patterns
    lut = fo.silu_lut()
    gates = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    finite = (gates & 0x7F80) != 0x7F80
    via_swiglu = fo.swiglu_bf16(gates, np.full(65536, 0x3F80, dtype=np.uint16))
    assert np.array_equal(lut[finite], via_swiglu[finite])


# ---- R9 / R11 / R12 -------------------------------------------------------------------

def test_shared_gate_and_combination_round_at_bf16_boundaries():
    # src/expert.rs:1290-1293
    assert fo.from_bf16(fo.sigmoid_bf16(fo.to_bf16(0.0))) == 0.5
    assert fo.from_bf16(fo.add_bf16(fo.to_bf16(256.0), fo.to_bf16(1.0))) == 256.0


def test_real_checkpoint_shared_gate_sigmoid(golden):
    # fixtures/sparse_moe/qwen3_8_flash_next_layer0.json: the one-element
    # shared_gate_logit and shared_gate_sigmoid captures, recovered from their
    # SHA-256s; sigmoid_bf16 must map one to the other.
    sm = golden["sparse_moe"]
    assert fo.sigmoid_bf16(sm["shared_gate_logit_bits"]) == sm["shared_gate_sigmoid_bits"]


def test_bf16_mixture_order_is_observable():
    # src/expert.rs:1276-1287 and tests/test_generate_mixture_fixture.py:9-29
    def accumulate(values):
        acc = fo.to_bf16(0.0)
        for v in values:
            acc = fo.add_bf16(acc, fo.to_bf16(v))
        return fo.from_bf16(acc)
    assert accumulate([256.0, -256.0, 1.0]) == 1.0
    assert accumulate([256.0, 1.0, -256.0]) == 0.0


def test_mixture_accumulates_in_given_order_with_bf16_rounding():
    # A one-column "expert" whose down output equals its input lets the mixture
    # be driven by chosen contributions: [256, 1, -256] -> 0 (rounds after
    # each expert), and [256, -256, 1] -> 1.
    # gate_up rows: gate = big positive (silu(g) ~= g), up = 1.0
    def expert_weights(value):
        # hidden = [1.0]; gate row = [64.0] -> gate=64 -> silu=64;
        # up row = [value/64] -> up = value/64; act = bf16(64 * value/64) = value
        gu = bf16([64.0, value / 64.0])
        down = bf16([1.0])
        return gu, down
    hidden = bf16([1.0])
    w = [expert_weights(v) for v in (256.0, 1.0, -256.0)]
    out = fo.mixture_bf16([a for a, _ in w], [b for _, b in w], hidden, 1, 1,
                          bf16([1.0, 1.0, 1.0]))
    assert f32(out) == [0.0]
    w = [expert_weights(v) for v in (256.0, -256.0, 1.0)]
    out = fo.mixture_bf16([a for a, _ in w], [b for _, b in w], hidden, 1, 1,
                          bf16([1.0, 1.0, 1.0]))
    assert f32(out) == [1.0]


def test_tiny_shared_expert_and_gate():
    # tests/test_generate_sparse_moe_block_fixture.py:9-26, through the whole
    # block: a router that always picks expert 0, whose weighted output is
    # known, so the combination routed + sigmoid(0) * shared_down is checked.
    shape = {"hidden": 2, "intermediate": 2, "experts": 1, "top_k": 1, "shared_intermediate": 2}
    weights = {
        "router": bf16([0.0, 0.0]),
        # routed expert: gate = x, up = x -> act = silu(x) * x
        "gate_up": bf16([1.0, 0.0, 0.0, 1.0, 1.0, 0.0, 0.0, 1.0]),
        "down": bf16([1.0, 0.0, 0.0, 1.0]),
        "shared_gate": bf16([1.0, 0.0, 0.0, 1.0]),
        "shared_up": bf16([2.0, 0.0, 0.0, 3.0]),
        "shared_down": bf16([1.0, 0.0, 0.0, 1.0]),
        "shared_expert_gate": bf16([0.0, 0.0]),
    }
    hidden = bf16([1.0, -2.0])
    res = fo.sparse_moe_block(shape, weights, hidden)
    assert fo.from_bf16(int(res["shared_gate_sigmoid"][0])) == 0.5
    assert list(res["ids"]) == [0]
    assert f32(res["scores"]) == [1.0]  # one selected expert renormalises to 1
    gated = [fo.to_bf16(0.5 * v) for v in f32(res["shared_down"])]
    combined = [fo.add_bf16(int(a), g) for a, g in zip(res["routed_mixture"], gated)]
    assert list(res["out"]) == combined
    # shared: gate=[1,-2], up=[2,-6], swiglu = silu*up, down = identity
    expect_shared = fo.swiglu_bf16(bf16([1.0, -2.0]), bf16([2.0, -6.0]))
    assert np.array_equal(res["shared_down"], expect_shared)


# ---- R4 / R5 routing ------------------------------------------------------------------

def test_router_fixture_scores_follow_from_selected_logits(golden):
    # fixtures/router/qwen3_8_flash_next_real.json: renormalised scores depend
    # only on the selected logits (exp(l_i - m) / sum over the selection), so
    # routing the ten selected logits alone must reproduce the fixture's
    # scores within the reference's own tolerance (src/router.rs:375, 2^-9).
    for case in golden["router"]["cases"]:
        logits = bf16(case["selected_logits_bf16"])
        ids = fo.topk_total_order(logits, 10)
        assert list(ids) == list(range(10))  # already in rank order, ties by index
        scores = f32(fo.route_scores(logits, ids))
        err = max(abs(a - b) for a, b in zip(scores, case["normalized_scores_bf16"]))
        assert err <= 2 ** -9, (case["name"], err)


def test_mixture_fixture_rank_and_execution_orders(golden):
    # src/expert.rs:811-815 and fixtures/mixture: execution order is the
    # ascending sort of the selection; score bits match the router authority.
    mix = golden["mixture"]
    assert sorted(mix["selection"]) == mix["execution"]
    assert mix["case"]["expert_execution_order"] == mix["execution"]
    router0 = golden["router"]["cases"][0]
    assert router0["selected_experts"] == mix["selection"]
    assert [fo.to_bf16(v) for v in router0["normalized_scores_bf16"]] == mix["score_bits_by_selection"]


def test_topk_total_order_against_brute_force_sort():
    # src/router.rs:241-247: sort by (total_cmp desc, index asc), truncate.
    rng = np.random.default_rng(3)
    for trial in range(200):
        n = int(rng.integers(1, 80))
        k = int(rng.integers(1, n + 1))
        # few distinct values to force ties, including -0.0/+0.0 and negatives
        pool = bf16([0.0, -0.0, 1.0, -1.0, 0.5, 2.0, -3.0, 1e-30])
        logits = pool[rng.integers(0, len(pool), n)]
        as_f = fo.bf16_to_f32(logits)
        # total_cmp: -0.0 < +0.0; emulate with a signed-zero-aware key
        key = [(float(v), 1 if (v == 0 and not np.signbit(v)) else 0) for v in as_f]
        expect = sorted(range(n), key=lambda i: (-key[i][0], -key[i][1], i))[:k]
        assert list(fo.topk_total_order(logits, k)) == expect


def test_route_matches_pinned_torch_topk_where_no_tie_order_is_involved():
    # src/decoder_layer.rs:667-672: all-zero logits select [0..9]. The second
    # case there (src/decoder_layer.rs:674-679) depends on libc++'s
    # nth_element tie order, [90,80,...,10,9]; the total-order rule selects
    # the same nine maxima and breaks the boundary tie by lowest index.
    zeros = np.full(512, fo.to_bf16(0.0), dtype=np.uint16)
    assert list(fo.topk_total_order(zeros, 10)) == list(range(10))
    logits = zeros.copy()
    for i in (10, 20, 30, 40, 50, 60, 70, 80, 90):
        logits[i] = fo.to_bf16(1.0)
    ours = list(fo.topk_total_order(logits, 10))
    assert ours == [10, 20, 30, 40, 50, 60, 70, 80, 90, 0]
    libcxx = [90, 80, 70, 60, 50, 40, 30, 20, 10, 9]
    assert sorted(ours[:9]) == sorted(libcxx[:9])
    assert all(logits[a] == logits[b] for a, b in zip(ours, libcxx))


def test_selected_tie_permutations_are_semantically_equivalent():
    # src/decoder_layer.rs:682-689
    logits = np.full(512, fo.to_bf16(-1.0), dtype=np.uint16)
    logits[202] = fo.to_bf16(0.5)
    logits[468] = fo.to_bf16(0.5)
    assert fo.equivalent_topk_order([468, 202], [202, 468], logits)
    logits[468] = fo.to_bf16(0.75)
    assert not fo.equivalent_topk_order([468, 202], [202, 468], logits)


@pytest.mark.skipif(not fo.ref_topk_available(), reason="oracle/_ref not built (no reference mounted)")
def test_reference_topk_shim_agrees_up_to_ties():
    # native/topk_shim.cpp built from the reference's source (libstdc++ here):
    # without ties its order is the value order, which the total order
    # reproduces exactly; with ties the two lists must be tie-equivalent
    # (src/decoder_layer.rs:309-322) whenever the k-th value is not tied
    # outside the selection.
    rng = np.random.default_rng(11)
    for trial in range(300):
        distinct = trial % 2 == 0
        if distinct:
            vals = rng.permutation(np.arange(-256, 256))[:512].astype(np.float32) / 64.0
        else:
            vals = rng.integers(-20, 20, 512).astype(np.float32) / 8.0
        logits = bf16(vals)
        shim = fo.ref_torch_topk_bf16(logits, 10)
        ours = fo.topk_total_order(logits, 10)
        f = fo.bf16_to_f32(logits)
        kth = f[ours[9]]
        boundary_tie = np.count_nonzero(f == kth) > np.count_nonzero(f[ours] == kth)
        if distinct:
            assert list(shim) == list(ours)
        elif not boundary_tie:
            assert fo.equivalent_topk_order(shim.astype(np.int32), ours, logits)
        # either way the selected values are identical rank by rank
        assert np.array_equal(f[shim], f[ours])


@pytest.mark.skipif(not fo.ref_topk_available(), reason="oracle/_ref not built (no reference mounted)")
def test_reference_topk_shim_agrees_at_vocabulary_size():
    # The LM head's top-20 over 248,320 logits (src/text_output.rs:275): the
    # shim's partial_sort branch (k * 64 <= count). With no tie in the top 21
    # its list is the value order; with ties the selected values still agree
    # rank by rank.
    rng = np.random.default_rng(12)
    for trial in range(4):
        vals = rng.standard_normal(248320).astype(np.float32) * (4.0 if trial % 2 else 0.5)
        logits = bf16(vals)
        shim = fo.ref_torch_topk_bf16(logits, 20)
        ours = fo.topk_total_order(logits, 20)
        f = fo.bf16_to_f32(logits)
        top = np.sort(f)[::-1][:21]
        if len(np.unique(top)) == 21:
            assert list(shim) == list(ours)
        assert np.array_equal(f[shim], f[ours])


def test_route_rejects_nan_logits_in_model_order():
    # src/decoder_layer.rs:279-281
    H, E = 32, 16
    w = np.zeros(E * H, dtype=np.uint16)
    w[0] = 0x7FC0  # NaN weight -> NaN logit for expert 0
    x = bf16([1.0] * H)
    with pytest.raises(ValueError):
        fo.route(w, x, E, H, 4, fo.ORDER_TREE32)
    ids, logits, scores = fo.route(w, x, E, H, 4, fo.ORDER_FOLD)  # router.rs does not reject
    assert ids[0] == 0


def test_expf_is_glibc_on_known_values():
    # Rust f32::exp is the platform expf; spot values with exactly known results.
    x = np.array([0.0, -0.0, 1.0, -np.inf, np.inf, -200.0, 100.0], dtype=np.float32)
    y = fo.expf(x)
    assert y[0] == 1.0 and y[1] == 1.0
    assert y[2] == np.float32(2.7182817)
    assert y[3] == 0.0 and np.isinf(y[4]) and y[5] == 0.0 and np.isinf(y[6])


# ---- pins whose failure a plausible oracle mistake would cause ----------------------

def _bf16_rne_f64(value: float) -> float:
    """Round an f64 to the nearest bf16 value, ties to even (8 significant
    bits), by exact rational arithmetic: independent of the oracle's float
    path."""
    from fractions import Fraction
    import math
    if value == 0.0:
        return 0.0
    v = Fraction(value)
    sign = -1 if v < 0 else 1
    v = abs(v)
    e = math.floor(math.log2(v))
    while Fraction(2) ** e > v:
        e -= 1
    while Fraction(2) ** (e + 1) <= v:
        e += 1
    ulp = Fraction(2) ** (e - 7)
    q, r = divmod(v, ulp)
    if r * 2 > ulp or (r * 2 == ulp and q % 2 == 1):
        q += 1
    return sign * float(q * ulp)


def test_tiny_expert_swiglu_bits_are_exact():
    # tests/test_generate_expert_fixture.py:9-27 asserts torch.equal on
    # bf16(bf16(silu(gate)) * up): silu is rounded to bf16 before the multiply
    # (src/expert.rs:562-571). Derived here in f64 with exact rounding:
    #   silu(-3) = -0.1422776 -> bf16 -0.142578125; * 2.0  = -0.28515625
    #   silu(1.5) = 1.2263618 -> bf16 1.2265625; * -3.0 = -3.6796875 -> -3.6875
    # Without the inner rounding the second would be bf16(-3.67908...) =
    # -3.671875.
    import math
    gate, up = [-3.0, 1.5], [2.0, -3.0]
    expect = []
    for g, u in zip(gate, up):
        silu = _bf16_rne_f64(g / (1.0 + math.exp(-g)))
        expect.append(_bf16_rne_f64(silu * u))
    assert expect == [-0.28515625, -3.6875]
    hidden = bf16([1.0, -2.0])
    gate_up_w = bf16([1.0, 2.0, 0.5, -0.5, 2.0, 0.0, -1.0, 1.0])
    out = fo.expert_bf16(gate_up_w, bf16([1.0, 0.0, 0.0, 1.0]), hidden, 2, 2, fo.to_bf16(0.5))
    assert f32(out["swiglu"]) == expect
    assert f32(out["down"]) == expect
    assert f32(out["weighted_down"]) == [v * 0.5 for v in expect]


def test_route_renormalises_over_the_selection():
    # src/router.rs:248-262 and src/decoder_layer.rs:290-306: softmax over all
    # E logits, then each selected probability divided by the selection's
    # sum. With 502 unselected experts holding most of the mass, the
    # un-renormalised probabilities are ~19x smaller than the scores, so an
    # oracle that skipped the division would fail by far more than the
    # tolerance; the f64 closed form exp(l_i) / sum_sel exp(l_j) is what the
    # renormalised score must equal up to f32 rounding and the bf16 output.
    import math
    E, K = 512, 10
    sel_values = [1.0 - 0.125 * i for i in range(K)]      # exact in bf16
    logits = np.full(E, fo.to_bf16(-0.25), dtype=np.uint16)  # below every selected value
    chosen = [7, 501, 3, 260, 99, 18, 444, 130, 311, 58]  # rank order of the values above
    for e, v in zip(chosen, sel_values):
        logits[e] = fo.to_bf16(v)
    ids = fo.topk_total_order(logits, K)
    assert list(ids) == chosen
    scores = f32(fo.route_scores(logits, ids))
    z = sum(math.exp(v) for v in sel_values)
    full = sum(math.exp(v) for v in sel_values) + (E - K) * math.exp(-0.25)
    for s, v in zip(scores, sel_values):
        closed = math.exp(v) / z
        assert abs(s - closed) <= 2 ** -8 * closed, (s, closed)
        assert closed / (math.exp(v) / full) > 10.0  # skipping renormalisation is far off
    assert abs(sum(scores) - 1.0) <= K * 2 ** -9


def test_block_mixture_runs_in_ascending_expert_id_not_rank():
    # src/decoder_layer.rs:422-424 (execution order = ascending id) and the
    # src/expert.rs:1276-1287 pattern: with contributions w0 = -w1 (experts 0
    # and 1 tie in the router, so their scores are equal) and a small w2 from
    # the top-ranked expert 2, the ascending-id sum is (w0 + w1) + w2 = w2,
    # while the rank-order sum (w2 + w0) + w1 loses w2 to rounding and gives 0.
    # Expert e: gate row 64 -> silu = 64 exactly; up row u_e -> act = 64 u_e;
    # down = identity, so its down output is 64 u_e: 1024, -1024 and 0.5.
    shape = {"hidden": 2, "intermediate": 1, "experts": 3, "top_k": 3, "shared_intermediate": 2}
    u = [16.0, -16.0, 1.0 / 128.0]
    gate_up = []
    for ue in u:
        gate_up += [64.0, 0.0, ue, 0.0]  # rows [gate; up] of [2I, H] = [2, 2]
    weights = {
        "router": bf16([0.0, 0.0, 0.0, 0.0, 1.0, 0.0]),  # logits [0, 0, 1]
        "gate_up": bf16(gate_up),
        "down": bf16([1.0, 0.0] * 3),                     # [H, I] = [2, 1] per expert
        "shared_gate": bf16([0.0] * 4),
        "shared_up": bf16([0.0] * 4),
        "shared_down": bf16([0.0] * 4),                   # shared output 0
        "shared_expert_gate": bf16([0.0, 0.0]),
    }
    hidden = bf16([1.0, 0.0])
    res = fo.sparse_moe_block(shape, weights, hidden)
    assert list(res["ids"]) == [2, 0, 1]  # rank order differs from id order
    s = f32(res["scores"])               # rank order: experts 2, 0, 1
    assert s[1] == s[2]
    w = {0: _bf16_rne_f64(1024.0 * s[1]), 1: _bf16_rne_f64(-1024.0 * s[2]), 2: _bf16_rne_f64(0.5 * s[0])}
    assert w[0] == -w[1] and 0 < w[2] < 0.5  # below half an ulp of w0 (ulp 1 in [128, 256))
    ascending = _bf16_rne_f64(_bf16_rne_f64(w[0] + w[1]) + w[2])
    rank_order = _bf16_rne_f64(_bf16_rne_f64(w[2] + w[0]) + w[1])
    assert ascending == w[2] and rank_order == 0.0
    assert f32(res["routed_mixture"])[0] == ascending
    assert f32(res["out"])[0] == ascending
