"""GPU parity at the reference model's real block shape: H=2560, I=Is=640,
E=512, K=10 (docs/ARCHITECTURE.md:16-21, src/decoder_layer.rs:15,40-42), with
seeded synthetic weights (no checkpoint is mounted), and at E=1024, the top-k
variant for more than 512 experts.

Decode blocks, chained steps, route ids/scores/logits: bit-exact against the
oracle. Prefill outputs: the MFMA tolerance of tests/test_gpu_prefill.py
(per-token cosine >= 0.9999, max |got - ref| <= 2^-6 max |ref|); its router
logits, ids and scores bit-exact.
"""
import numpy as np
import pytest

from firewing_amd import hip_moe as hm
from oracle import fw_oracle as fo

pytestmark = pytest.mark.gpu

SEED = 0x46495245
REAL = dict(hidden=2560, intermediate=640, experts=512, top_k=10, shared_intermediate=640)
WIDE_E = dict(hidden=256, intermediate=128, experts=1024, top_k=10, shared_intermediate=128)


def as_f32(bits):
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def assert_close(got, ref, what):
    g, r = as_f32(got).astype(np.float64), as_f32(ref).astype(np.float64)
    cos = (g * r).sum(-1) / np.maximum(np.linalg.norm(g, axis=-1) * np.linalg.norm(r, axis=-1), 1e-30)
    rel = np.abs(g - r).max(-1) / np.maximum(np.abs(r).max(-1), 1e-30)
    msg = f"{what}: min cosine {cos.min():.7f}, max rel {rel.max():.3e}"
    print(msg)
    assert cos.min() >= 0.9999 and rel.max() <= 2.0 ** -6, msg


@pytest.fixture(scope="module")
def real3():
    # 3 layers x 5.04 GB of resident banks
    with hm.MoeContext(layers=3, **REAL) as ctx:
        ctx.generate_layers(0, 3, SEED, True)
        yield ctx


@pytest.mark.parametrize("tokens", [1, 2, 3, 4])
def test_real_shape_block(real3, tokens):
    x = fo.synth_hidden(SEED, tokens, REAL["hidden"], first_token=50 + tokens)
    got = real3.sparse_moe_block(1, x)
    out, ids, scores, logits = fo.synth_block(REAL, SEED, 1, x)
    assert np.array_equal(got["selected_experts"], ids)
    assert np.array_equal(got["selected_scores"], scores)
    assert np.array_equal(got["router_logits"], logits)
    assert np.array_equal(got["out"], out)


@pytest.mark.parametrize("tokens", [1, 4])
def test_real_shape_step_three_layers(real3, tokens):
    x = fo.synth_hidden(SEED, tokens, REAL["hidden"], first_token=600 + tokens)
    resid, blocks, ids, scores = real3.moe_step(x)
    r_resid, r_blocks, r_ids, r_scores = fo.synth_step(REAL, SEED, 3, x)
    assert np.array_equal(ids, r_ids)
    assert np.array_equal(scores, r_scores)
    assert np.array_equal(blocks, r_blocks)
    assert np.array_equal(resid, r_resid)


def test_real_shape_fold_route(real3):
    x = fo.synth_hidden(SEED, 3, REAL["hidden"], first_token=700)
    ids, scores, logits = real3.route(2, x, hm.LOGITS_FOLD)
    r_ids, r_scores, r_logits = fo.synth_route(REAL, SEED, 2, x, order=fo.ORDER_FOLD)
    assert np.array_equal(ids, r_ids)
    assert np.array_equal(scores, r_scores)
    assert np.array_equal(logits, r_logits)


def test_real_shape_prefill_300_tokens(real3):
    x = fo.synth_hidden(SEED, 300, REAL["hidden"], first_token=800)
    got = real3.prefill_block(0, x)
    out, ids, scores, logits = fo.synth_block(REAL, SEED, 0, x)
    assert np.array_equal(got["router_logits"], logits)
    assert np.array_equal(got["selected_experts"], ids)
    assert np.array_equal(got["selected_scores"], scores)
    assert_close(got["out"], out, "real-shape prefill T=300")


def test_real_shape_prefill_8k_router_bits(real3):
    T = 8192
    x = fo.synth_hidden(SEED, T, REAL["hidden"], first_token=30000)
    got = real3.prefill_block(2, x)
    ids, scores, logits = fo.synth_route(REAL, SEED, 2, x)
    assert np.array_equal(got["router_logits"], logits)
    assert np.array_equal(got["selected_experts"], ids)
    assert np.array_equal(got["selected_scores"], scores)
    # every token of two popular experts (multi-tile groups) within tolerance
    counts = np.bincount(ids.ravel(), minlength=REAL["experts"])
    top = np.argsort(-counts)[:2]
    rows = np.flatnonzero(np.isin(ids, top).any(axis=1))[:512]
    out, _, _, _ = fo.synth_block(REAL, SEED, 2, x[rows])
    assert_close(got["out"][rows], out, f"real-shape prefill T=8192 ({rows.size} tokens of experts {top})")


@pytest.fixture(scope="module")
def wide_e():
    with hm.MoeContext(layers=2, **WIDE_E) as ctx:
        ctx.generate_layers(0, 2, SEED, True)
        yield ctx


@pytest.mark.parametrize("tokens", [1, 2, 4])
def test_wide_expert_count_block(wide_e, tokens):
    x = fo.synth_hidden(SEED, tokens, WIDE_E["hidden"], first_token=70 + tokens)
    got = wide_e.sparse_moe_block(1, x)
    out, ids, scores, logits = fo.synth_block(WIDE_E, SEED, 1, x)
    assert np.array_equal(got["selected_experts"], ids)
    assert np.array_equal(got["selected_scores"], scores)
    assert np.array_equal(got["router_logits"], logits)
    assert np.array_equal(got["out"], out)


def test_wide_expert_count_step_and_prefill(wide_e):
    x = fo.synth_hidden(SEED, 2, WIDE_E["hidden"], first_token=90)
    resid, blocks, ids, _ = wide_e.moe_step(x)
    r_resid, r_blocks, r_ids, _ = fo.synth_step(WIDE_E, SEED, 2, x)
    assert np.array_equal(ids, r_ids)
    assert np.array_equal(blocks, r_blocks)
    assert np.array_equal(resid, r_resid)
    xp = fo.synth_hidden(SEED, 37, WIDE_E["hidden"], first_token=95)
    got = wide_e.prefill_block(0, xp)
    out, pids, pscores, plogits = fo.synth_block(WIDE_E, SEED, 0, xp)
    assert np.array_equal(got["router_logits"], plogits)
    assert np.array_equal(got["selected_experts"], pids)
    assert np.array_equal(got["selected_scores"], pscores)
    assert_close(got["out"], out, "E=1024 prefill T=37")
