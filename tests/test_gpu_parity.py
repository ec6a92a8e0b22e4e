"""GPU parity: every HIP entry point against the CPU oracle, bit for bit.

All calls go through the C ABI (firewing_amd.hip_moe over
libfirewing_hip_moe.so). Shapes are the workload's (H=2048, I=512, E=512,
K=10, Is=512) unless a test needs a tiny case. The bar is bit-exact equality
for every bf16 output, selected id and score.
"""
import numpy as np
import pytest

from firewing_amd import hip_moe as hm
from oracle import fw_oracle as fo

pytestmark = pytest.mark.gpu

SEED = 0x46495245
CFG = dict(hidden=2048, intermediate=512, experts=512, top_k=10, shared_intermediate=512)


def rand_bf16(rng, n, scale=1.0):
    return fo.bf16_array(rng.standard_normal(n) * scale)


def first_diff(a, b):
    a, b = np.asarray(a).ravel(), np.asarray(b).ravel()
    idx = np.flatnonzero(a != b)
    return None if idx.size == 0 else (int(idx[0]), int(a[idx[0]]), int(b[idx[0]]), int(idx.size))


# ---- numerics -----------------------------------------------------------------------

def test_device_expf_matches_glibc():
    rng = np.random.default_rng(1)
    bits = (np.arange(65536, dtype=np.uint32) << 16).view(np.float32)
    soft = -rng.uniform(0, 104, 1 << 22).astype(np.float32)
    edges = np.array([0.0, -0.0, -87.3, -88.0, -103.9, -103.97, -104.0, np.inf, -np.inf, 88.72,
                      np.nan], dtype=np.float32)
    for x in (bits, -bits, soft, edges):
        dev = hm.expf_device(x)
        ref = fo.expf(x)
        same = (dev.view(np.uint32) == ref.view(np.uint32)) | (np.isnan(dev) & np.isnan(ref))
        assert same.all(), x[~same][:5]


def test_swiglu_and_sigmoid_exhaustive_over_bf16():
    gates = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    rng = np.random.default_rng(2)
    ups = rand_bf16(rng, 65536)
    assert first_diff(hm.swiglu_bf16(gates, ups), fo.swiglu_bf16(gates, ups)) is None
    assert first_diff(hm.sigmoid_bf16(gates), [fo.sigmoid_bf16(int(g)) for g in gates]) is None


@pytest.mark.parametrize("rows,cols", [(1024, 2048), (2048, 512), (7, 64), (5, 40), (3, 46), (1, 2)])
def test_linear_bf16_bit_exact(rows, cols):
    rng = np.random.default_rng(rows * 7 + cols)
    w = rand_bf16(rng, rows * cols, 0.02)
    x = rand_bf16(rng, cols)
    assert first_diff(hm.linear_bf16(w, x, rows, cols), fo.linear_bf16(w, x, rows, cols)) is None


def test_linear_bf16_special_values():
    rng = np.random.default_rng(5)
    rows, cols = 64, 256
    w = rand_bf16(rng, rows * cols)
    x = rand_bf16(rng, cols)
    w[:cols] = 0x8000          # row 0: -0.0 weights -> -0.0 sum -> +0.0 result
    x[5] = 0x0001              # subnormal input
    w[cols:2 * cols] = 0x0080  # row 1: smallest normal weights x subnormal products
    w[2 * cols + 3] = 0x7F7F   # row 2: huge weight -> large products
    w[3 * cols + 7] = 0x7F80   # row 3: +inf
    got = hm.linear_bf16(w, x, rows, cols)
    assert first_diff(got, fo.linear_bf16(w, x, rows, cols)) is None
    assert got[0] == 0x0000


def test_topk_matches_total_order():
    rng = np.random.default_rng(3)
    for trial in range(40):
        count = int(rng.integers(1, 1025))
        k = int(rng.integers(1, min(32, count) + 1))
        pool = fo.bf16_array([0.0, -0.0, 1.0, -1.0, 0.5, 2.0, -3.0, 1e-30])
        if trial % 2:
            vals = pool[rng.integers(0, len(pool), count)]
        else:
            vals = rand_bf16(rng, count)
        assert list(hm.topk_bf16(vals, k)) == list(fo.topk_total_order(vals, k)), trial


@pytest.mark.parametrize("order", [hm.LOGITS_TREE32, hm.LOGITS_FOLD])
def test_route_bit_exact(order):
    rng = np.random.default_rng(4 + order)
    H, E, K, T = 2048, 512, 10, 9
    w = fo.synth_tensor(SEED, 0, 1, 0, E * H)
    w.reshape(E, H)[:, H - 1] = fo.synth_router_bias(SEED, 0, E)
    x = fo.synth_hidden(SEED, T, H)
    ids, scores, logits = hm.route(w, x, E, H, K, order)
    for t in range(T):
        rid, rlog, rsc = fo.route(w, x[t], E, H, K, order)
        assert first_diff(logits[t], rlog) is None
        assert list(ids[t]) == list(rid)
        assert first_diff(scores[t], rsc) is None


def test_route_rejects_nan_logits_in_model_order():
    H, E = 64, 16
    w = np.zeros(E * H, dtype=np.uint16)
    w[0] = 0x7FC0
    x = fo.bf16_array([1.0] * H)
    with pytest.raises(hm.FirewingError, match="NaN"):
        hm.route(w, x, E, H, 4, hm.LOGITS_TREE32)
    ids, _, _ = hm.route(w, x, E, H, 4, hm.LOGITS_FOLD)
    assert ids[0][0] == 0


def test_expert_bf16_all_captures():
    H, I = CFG["hidden"], CFG["intermediate"]
    e = 137
    gu = fo.synth_tensor(SEED, 0, 2, e * 2 * I * H, 2 * I * H)
    dn = fo.synth_tensor(SEED, 0, 3, e * H * I, H * I)
    x = fo.synth_hidden(SEED, 1, H)[0]
    rw = fo.to_bf16(0.11962890625)
    got = hm.expert_bf16(gu, dn, x, H, I, rw)
    ref = fo.expert_bf16(gu, dn, x, H, I, rw)
    for name in ("gate_up", "swiglu", "down", "weighted_down"):
        assert first_diff(got[name], ref[name]) is None, name


# ---- resident context, tiny shapes with installed weights ---------------------------------

TINY = dict(hidden=64, intermediate=32, experts=16, top_k=4, shared_intermediate=32)


def tiny_weights(rng, router_scale=0.2):
    H, I, E, Is = TINY["hidden"], TINY["intermediate"], TINY["experts"], TINY["shared_intermediate"]
    return {
        "router": rand_bf16(rng, E * H, router_scale),
        "gate_up": rand_bf16(rng, E * 2 * I * H, 0.2),
        "down": rand_bf16(rng, E * H * I, 0.2),
        "shared_gate": rand_bf16(rng, Is * H, 0.2),
        "shared_up": rand_bf16(rng, Is * H, 0.2),
        "shared_down": rand_bf16(rng, H * Is, 0.2),
        "shared_expert_gate": rand_bf16(rng, H, 0.2),
    }


@pytest.fixture(scope="module")
def tiny_ctx():
    with hm.MoeContext(layers=3, **TINY) as ctx:
        yield ctx


def install(ctx, layer, w):
    ctx.install_layer(layer, w["router"], w["gate_up"], w["down"], w["shared_gate"],
                      w["shared_up"], w["shared_down"], w["shared_expert_gate"])


@pytest.mark.parametrize("tokens", [1, 2, 3, 4])
@pytest.mark.parametrize("order", [hm.LOGITS_TREE32, hm.LOGITS_FOLD])
def test_block_tiny_installed(tiny_ctx, tokens, order):
    rng = np.random.default_rng(10 * tokens + order)
    w = tiny_weights(rng)
    install(tiny_ctx, 1, w)
    x = rand_bf16(rng, tokens * TINY["hidden"]).reshape(tokens, -1)
    got = tiny_ctx.sparse_moe_block(1, x, order)
    for t in range(tokens):
        ref = fo.sparse_moe_block(TINY, w, x[t], order)
        assert list(got["selected_experts"][t]) == list(ref["ids"])
        assert first_diff(got["selected_scores"][t], ref["scores"]) is None
        assert first_diff(got["router_logits"][t], ref["logits"]) is None
        assert got["shared_gate_sigmoid"][t] == ref["shared_gate_sigmoid"][0]
        assert first_diff(got["out"][t], ref["out"]) is None, (t, first_diff(got["out"][t], ref["out"]))


def assert_captures_equal(got, ref, t, where):
    """Every verifier capture of token t bit for bit (src/expert.rs:1154-1199,
    src/decoder_layer.rs:528-586), and the capture identity the reference's
    verifier ends with: out = add_bf16(routed_mixture, gated_shared)."""
    for name in hm.VERIFIER_CAPTURES:
        g = np.asarray(got[name][t]).ravel()
        r = np.asarray(ref[name]).ravel()
        assert g.shape == r.shape and first_diff(g, r) is None, (where, t, name, first_diff(g, r))
    combined = np.array([fo.add_bf16(int(a), int(b)) for a, b in
                         zip(got["routed_mixture"][t], got["gated_shared"][t])], dtype=np.uint16)
    assert first_diff(combined, got["out"][t]) is None, (where, t)


@pytest.mark.parametrize("tokens,order", [(1, hm.LOGITS_TREE32), (4, hm.LOGITS_TREE32), (3, hm.LOGITS_FOLD)])
def test_block_tiny_verifier_captures(tiny_ctx, tokens, order):
    rng = np.random.default_rng(70 + 10 * tokens + order)
    w = tiny_weights(rng)
    install(tiny_ctx, 2, w)
    x = rand_bf16(rng, tokens * TINY["hidden"]).reshape(tokens, -1)
    got = tiny_ctx.sparse_moe_block(2, x, order, captures="all")
    for t in range(tokens):
        ref = fo.sparse_moe_block(TINY, w, x[t], order)
        assert first_diff(got["out"][t], ref["out"]) is None
        assert got["shared_gate_sigmoid"][t] == ref["shared_gate_sigmoid"][0]
        assert_captures_equal(got, ref, t, "tiny")


def test_block_tiny_router_ties(tiny_ctx):
    # A zero router: every logit is +0.0, so selection is experts 0..K-1 by the
    # index rule and the scores are uniform.
    rng = np.random.default_rng(99)
    w = tiny_weights(rng)
    w["router"][:] = 0
    install(tiny_ctx, 0, w)
    x = rand_bf16(rng, 2 * TINY["hidden"]).reshape(2, -1)
    got = tiny_ctx.sparse_moe_block(0, x)
    for t in range(2):
        ref = fo.sparse_moe_block(TINY, w, x[t])
        assert list(got["selected_experts"][t]) == [0, 1, 2, 3] == list(ref["ids"])
        assert first_diff(got["out"][t], ref["out"]) is None


def test_mixture_resident_tiny(tiny_ctx):
    rng = np.random.default_rng(7)
    w = tiny_weights(rng)
    install(tiny_ctx, 2, w)
    H, I = TINY["hidden"], TINY["intermediate"]
    x = rand_bf16(rng, H)
    experts = [1, 4, 9, 15]
    rws = fo.bf16_array([0.4, 0.3, 0.2, 0.1])
    got = tiny_ctx.mixture(2, x, experts, rws)
    gus = [w["gate_up"][e * 2 * I * H:(e + 1) * 2 * I * H] for e in experts]
    dns = [w["down"][e * H * I:(e + 1) * H * I] for e in experts]
    assert first_diff(got, fo.mixture_bf16(gus, dns, x, H, I, rws)) is None


def test_step_tiny_chained(tiny_ctx):
    rng = np.random.default_rng(8)
    ws = [tiny_weights(rng) for _ in range(3)]
    for l, w in enumerate(ws):
        install(tiny_ctx, l, w)
    x = rand_bf16(rng, 2 * TINY["hidden"]).reshape(2, -1)
    resid, blocks, ids, scores = tiny_ctx.moe_step(x, bias_feature=False)
    cur = x.copy()
    for l, w in enumerate(ws):
        for t in range(2):
            ref = fo.sparse_moe_block(TINY, w, fo.rms_norm_bf16(cur[t]))
            assert list(ids[l, t]) == list(ref["ids"])
            assert first_diff(blocks[l, t], ref["out"]) is None
            cur[t] = [fo.add_bf16(int(a), int(b)) for a, b in zip(cur[t], ref["out"])]
    assert first_diff(resid, cur) is None


def _norms_with_tree(r, partner3):
    """bf16 rms_norm of every row of r ([N, H] bf16, no bias feature) with the
    32-chain sum of squares (TREE32) whose third tree level adds chain
    partner3[j] to chain j (j + 4 in the reference)."""
    v = (np.asarray(r, np.uint16).astype(np.uint32) << 16).view(np.float32)
    n, H = v.shape
    acc = np.zeros((n, 32), np.float32)
    for b in range(H // 32):
        blk = v[:, 32 * b:32 * b + 32]
        acc = (acc + (blk * blk).astype(np.float32)).astype(np.float32)
    a = acc.copy()
    a[:, :16] = (a[:, :16] + a[:, 16:]).astype(np.float32)
    a[:, :8] = (a[:, :8] + a[:, 8:16]).astype(np.float32)
    a[:, :4] = (a[:, :4] + a[:, partner3]).astype(np.float32)
    ss = ((a[:, 0] + a[:, 1]).astype(np.float32) + (a[:, 2] + a[:, 3]).astype(np.float32)).astype(np.float32)
    ss = (ss + np.float32(0)).astype(np.float32)
    inv = (np.float32(1.0) / np.sqrt((ss / np.float32(H) + np.float32(1e-6)).astype(np.float32))).astype(np.float32)
    bits = (v * inv[:, None]).astype(np.float32).view(np.uint32)
    return ((bits + 0x7FFF + ((bits >> 16) & 1)) >> 16).astype(np.uint16)


def test_step_prenorm_summation_order(tiny_ctx):
    # A one-ulp change in the sum of squares rarely shows after the bf16
    # rounding, so the residuals are chosen (on the CPU, from many random
    # candidates) where it does: those whose normalised vector changes if the
    # last tree level paired chain j with j ^ 6 (what a DPP row rotate in the
    # wrong direction gives) instead of j + 4. A wrong pairing in the kernel
    # then fails every one of them.
    rng = np.random.default_rng(21)
    ws = [tiny_weights(rng) for _ in range(3)]
    for l, w in enumerate(ws):
        install(tiny_ctx, l, w)
    H = TINY["hidden"]
    cand = rng.standard_normal((200000, H)).astype(np.float32).view(np.uint32)
    cand = ((cand + 0x7FFF + ((cand >> 16) & 1)) >> 16).astype(np.uint16)
    right = _norms_with_tree(cand, [4, 5, 6, 7])
    wrong = _norms_with_tree(cand, [6, 7, 4, 5])
    picked = cand[(right != wrong).any(axis=1)][:32]
    assert len(picked) >= 8, len(picked)
    for x in picked[:4]:
        assert first_diff(fo.rms_norm_bf16(x), _norms_with_tree(x[None], [4, 5, 6, 7])[0]) is None
    for i in range(0, len(picked) - len(picked) % 4, 4):
        x4 = picked[i:i + 4]
        resid, blocks, _, _ = tiny_ctx.moe_step(x4, bias_feature=False)
        for t in range(4):
            ref = fo.sparse_moe_block(TINY, ws[0], fo.rms_norm_bf16(x4[t]))
            assert first_diff(blocks[0, t], ref["out"]) is None, (i + t)


def test_step_after_timed_out_launch(tiny_ctx):
    # A wait limit of 10 ns makes the chained step's dependency waits time
    # out (forced from the host; every workgroup still exits). The failed
    # launch leaves phase counters partly counted; the next launch with the
    # normal limit must still be exact.
    rng = np.random.default_rng(12)
    ws = [tiny_weights(rng) for _ in range(3)]
    for l, w in enumerate(ws):
        install(tiny_ctx, l, w)
    x = rand_bf16(rng, TINY["hidden"]).reshape(1, -1)
    tiny_ctx.set_wait_timeout(1e-8)
    try:
        with pytest.raises(hm.FirewingError, match="time limit"):
            tiny_ctx.moe_step(x, bias_feature=False)
    finally:
        tiny_ctx.set_wait_timeout(10.0)
    for _ in range(2):
        resid, blocks, ids, _ = tiny_ctx.moe_step(x, bias_feature=False)
        cur = x[0].copy()
        for l, w in enumerate(ws):
            ref = fo.sparse_moe_block(TINY, w, fo.rms_norm_bf16(cur))
            assert list(ids[l, 0]) == list(ref["ids"])
            assert first_diff(blocks[l, 0], ref["out"]) is None
            cur = np.array([fo.add_bf16(int(a), int(b)) for a, b in zip(cur, ref["out"])], dtype=np.uint16)
        assert first_diff(resid[0], cur) is None


def test_block_rejects_bad_arguments(tiny_ctx):
    x = np.zeros((5, TINY["hidden"]), dtype=np.uint16)
    with pytest.raises(hm.FirewingError, match="tokens"):
        tiny_ctx.sparse_moe_block(0, x)
    with pytest.raises(hm.FirewingError, match="layer out of range"):
        tiny_ctx.sparse_moe_block(3, x[:1])


# ---- resident context at the workload's shapes ------------------------------------------

@pytest.fixture(scope="module")
def ctx3():
    with hm.MoeContext(layers=3, **CFG) as ctx:
        ctx.generate_layers(0, 3, SEED, True)
        yield ctx


def test_generated_weights_match_cpu_generator(ctx3):
    H, I, E, Is = CFG["hidden"], CFG["intermediate"], CFG["experts"], CFG["shared_intermediate"]
    rng = np.random.default_rng(11)
    sizes = {hm.ROUTER: E * H, hm.GATE_UP: E * 2 * I * H, hm.DOWN: E * H * I,
             hm.SHARED_GATE: Is * H, hm.SHARED_UP: Is * H, hm.SHARED_DOWN: H * Is,
             hm.SHARED_EXPERT_GATE: H}
    for layer in range(3):
        for tensor, n in sizes.items():
            span = min(4096, n)
            for start in (0, int(rng.integers(0, n - span + 1)) & ~3, n - span):
                count = span
                got = ctx3.read_tensor(layer, tensor, start, count)
                ref = fo.synth_tensor(SEED, layer, tensor, start, count)
                if tensor == hm.ROUTER:
                    bias = fo.synth_router_bias(SEED, layer, E)
                    idx = np.arange(start, start + count)
                    col = idx % H == H - 1
                    ref[col] = bias[idx[col] // H]
                assert first_diff(got, ref) is None, (layer, tensor, start)


@pytest.mark.parametrize("tokens", [1, 2, 4])
def test_block_workload_shape(ctx3, tokens):
    x = fo.synth_hidden(SEED, tokens, CFG["hidden"], first_token=100)
    got = ctx3.sparse_moe_block(1, x)
    out, ids, scores, logits = fo.synth_block(CFG, SEED, 1, x)
    assert np.array_equal(got["selected_experts"], ids)
    assert first_diff(got["selected_scores"], scores) is None
    assert first_diff(got["router_logits"], logits) is None
    assert first_diff(got["out"], out) is None


def test_block_workload_shape_fold_order(ctx3):
    x = fo.synth_hidden(SEED, 2, CFG["hidden"], first_token=200)
    got = ctx3.sparse_moe_block(2, x, hm.LOGITS_FOLD)
    out, ids, scores, logits = fo.synth_block(CFG, SEED, 2, x, order=fo.ORDER_FOLD)
    assert np.array_equal(got["selected_experts"], ids)
    assert first_diff(got["selected_scores"], scores) is None
    assert first_diff(got["out"], out) is None


@pytest.mark.parametrize("tokens,order", [(1, hm.LOGITS_TREE32), (2, hm.LOGITS_FOLD), (4, hm.LOGITS_TREE32)])
def test_block_verifier_captures_workload_shape(ctx3, tokens, order):
    x = fo.synth_hidden(SEED, tokens, CFG["hidden"], first_token=900 + tokens)
    got = ctx3.sparse_moe_block(0, x, order, captures="all")
    ref = fo.synth_block_captures(CFG, SEED, 0, x, order=order)
    assert first_diff(got["out"], ref["out"]) is None
    assert np.array_equal(got["selected_experts"], ref["ids"])
    assert first_diff(got["shared_gate_sigmoid"], ref["shared_gate_sigmoid"].ravel()) is None
    for t in range(tokens):
        assert_captures_equal(got, {k: ref[k][t] for k in hm.VERIFIER_CAPTURES}, t, "workload")


def test_mixture_resident_workload_shape(ctx3):
    H, I = CFG["hidden"], CFG["intermediate"]
    x = fo.synth_hidden(SEED, 1, H, first_token=300)[0]
    experts = [3, 77, 130, 250, 511]
    rws = fo.bf16_array([0.3, 0.25, 0.2, 0.15, 0.1])
    got = ctx3.mixture(0, x, experts, rws)
    gus = [fo.synth_tensor(SEED, 0, 2, e * 2 * I * H, 2 * I * H) for e in experts]
    dns = [fo.synth_tensor(SEED, 0, 3, e * H * I, H * I) for e in experts]
    assert first_diff(got, fo.mixture_bf16(gus, dns, x, H, I, rws)) is None


@pytest.mark.parametrize("tokens", [1, 3])
def test_step_workload_shape_three_layers(ctx3, tokens):
    x = fo.synth_hidden(SEED, tokens, CFG["hidden"], first_token=400)
    resid, blocks, ids, scores = ctx3.moe_step(x)
    r_resid, r_blocks, r_ids, r_scores = fo.synth_step(CFG, SEED, 3, x)
    assert np.array_equal(ids, r_ids)
    assert first_diff(scores, r_scores) is None
    assert first_diff(blocks, r_blocks) is None
    assert first_diff(resid, r_resid) is None
    # a second launch reuses the counters the first one zeroed
    again = ctx3.moe_step(x)
    assert np.array_equal(again[0], resid)


def test_calls_on_different_streams_are_ordered(ctx3):
    # The context's calls share its scratch (launch parameters, phase
    # counters, prefill buffers). moe_step_dev on one user stream,
    # prefill_block_dev on another (the first time growing the prefill
    # scratch) and host-pointer calls on the context's stream follow each
    # other with no host wait: each must still run after the previous one.
    from firewing_amd import hip_runtime as rt
    H = CFG["hidden"]
    x = fo.synth_hidden(SEED, 1, H, first_token=41)
    xb = fo.synth_hidden(SEED, 2, H, first_token=42)
    xp = fo.synth_hidden(SEED, 96, H, first_token=43)
    xq = fo.synth_hidden(SEED, 300, H, first_token=44)
    want_step = ctx3.moe_step(x)[0]
    want_block = ctx3.sparse_moe_block(1, xb)["out"]
    want_pf = ctx3.prefill_block(0, xp)["out"]
    a, b = rt.Stream(), rt.Stream()
    xd, rd = rt.DeviceArray.from_numpy(x), rt.DeviceArray(x.shape, np.uint16)
    xpd, opd = rt.DeviceArray.from_numpy(xp), rt.DeviceArray(xp.shape, np.uint16)
    xqd, oqd = rt.DeviceArray.from_numpy(xq), rt.DeviceArray(xq.shape, np.uint16)
    for i in range(3):
        ctx3.moe_step_dev(xd.ptr, 1, rd.ptr, stream=a.handle)
        if i == 0:
            ctx3.prefill_block_dev(1, xqd.ptr, 300, oqd.ptr, stream=b.handle)  # grows the scratch
        blk = ctx3.sparse_moe_block(1, xb)["out"]
        ctx3.prefill_block_dev(0, xpd.ptr, 96, opd.ptr, stream=b.handle)
        ctx3.moe_step_dev(xd.ptr, 1, rd.ptr, stream=a.handle)
        pf = ctx3.prefill_block(0, xp)["out"]
        assert np.array_equal(blk, want_block), i
        assert np.array_equal(pf, want_pf), i
    a.synchronize()
    b.synchronize()
    ctx3.synchronize()
    assert np.array_equal(rd.numpy(), want_step)
    assert np.array_equal(opd.numpy(), want_pf)
    out_q = oqd.numpy()
    assert np.array_equal(out_q, ctx3.prefill_block(1, xq)["out"])
    for arr in (xd, rd, xpd, opd, xqd, oqd):
        arr.free()
    a.destroy()
    b.destroy()
