"""GPU parity of the LM head (src/text_output.rs:204-317): logits =
linear_bf16(lm_head, mixed) bit-exact against the oracle, and their top-k in
the total order (value descending, index ascending), at small vocabularies,
with ties, after the final mixer, from a safetensors checkpoint, and at the
reference model's full head (248,320 x 2560, seeded synthetic weights)."""
import json

import numpy as np
import pytest

from firewing_amd import hip_moe as hm
from oracle import fw_oracle as fo

pytestmark = pytest.mark.gpu

SEED = 0x46495245


def bf16(rng, shape, scale):
    v = (rng.standard_normal(shape) * scale).astype(np.float32)
    return (v.view(np.uint32) >> 16).astype(np.uint16)


def small_ctx(hidden):
    # the LM head uses only the context's hidden size; the MoE banks are tiny
    return hm.MoeContext(hidden=hidden, intermediate=32, experts=16, top_k=4, shared_intermediate=32, layers=1)


def reference(weight, x, V, H, k):
    logits = np.stack([fo.linear_bf16(weight, x[t], V, H) for t in range(x.shape[0])])
    ids = np.stack([fo.topk_total_order(logits[t], k) for t in range(x.shape[0])])
    return logits, ids


@pytest.mark.parametrize("H", [2048, 2560])
@pytest.mark.parametrize("V,T,k", [(37, 1, 20), (4099, 3, 20), (20000, 4, 64), (20, 2, 20)])
def test_lm_head_bit_exact(H, V, T, k):
    rng = np.random.default_rng(V + T + H)
    w = bf16(rng, (V, H), 0.02)
    x = bf16(rng, (T, H), 1.0)
    with small_ctx(H) as ctx:
        ctx.install_lm_head(w, V)
        got = ctx.lm_head(x, k)
    logits, ids = reference(w, x, V, H, k)
    assert np.array_equal(got["logits"], logits)
    assert np.array_equal(got["ids"], ids)
    assert np.array_equal(got["values"], np.take_along_axis(logits, ids, 1))


def test_lm_head_ties_take_the_lower_index():
    rng = np.random.default_rng(3)
    H, V, k = 2048, 9000, 32
    base = bf16(rng, (16, H), 0.02)
    w = base[rng.integers(0, 16, size=V)]  # 16 distinct rows: every logit is tied ~560 times
    x = bf16(rng, (2, H), 1.0)
    with small_ctx(H) as ctx:
        ctx.install_lm_head(w, V)
        got = ctx.lm_head(x, k)
    logits, ids = reference(w, x, V, H, k)
    assert np.array_equal(got["ids"], ids)
    # within a tied value the ids ascend
    for t in range(2):
        vals = logits[t, ids[t]]
        for a in range(k - 1):
            if vals[a] == vals[a + 1]:
                assert ids[t, a] < ids[t, a + 1]


def test_final_mixer_then_lm_head():
    # src/text_output.rs:266-273: run_final_mixer on the decoder output, then the head
    S, W, R, V, k = 4, 2560, 320, 5000, 20
    rng = np.random.default_rng(11)
    norm, down, up = bf16(rng, S * W, 0.1), bf16(rng, (R, S * W), 0.02), bf16(rng, (S * W, R), 0.05)
    head = bf16(rng, (V, W), 0.02)
    decoder_out = bf16(rng, (1, S * W), 1.0)
    mixed = hm.hyper_connection(decoder_out, norm, down, up, None, S, W, R)["mixed"]
    ref_mixed = fo.hyper_connection(decoder_out[0], norm, down, up, None, S, W, R)["mixed"]
    assert np.array_equal(mixed[0], ref_mixed)
    with small_ctx(W) as ctx:
        ctx.install_lm_head(head, V)
        got = ctx.lm_head(mixed, k)
    logits, ids = reference(head, mixed, V, W, k)
    assert np.array_equal(got["logits"], logits)
    assert np.array_equal(got["ids"], ids)


def test_lm_head_from_safetensors_and_device_pointers(tmp_path):
    import torch
    from safetensors.torch import save_file
    from firewing_amd import hip_runtime as rt
    rng = np.random.default_rng(13)
    H, V, T, k = 2560, 3001, 2, 20
    w = bf16(rng, (V, H), 0.02)
    x = bf16(rng, (T, H), 1.0)
    save_file({"lm_head.weight": torch.from_numpy(w.view(np.int16)).view(torch.bfloat16)},
              str(tmp_path / "head.safetensors"))
    (tmp_path / "model.safetensors.index.json").write_text(json.dumps({"weight_map": {"lm_head.weight": "head.safetensors"}}))
    with small_ctx(H) as ctx:
        ctx.load_lm_head_safetensors(tmp_path / "model.safetensors.index.json", "lm_head.weight", V)
        got = ctx.lm_head(x, k)
        dx = rt.DeviceArray.from_numpy(x)
        dl = rt.DeviceArray((T, V), np.uint16)
        di = rt.DeviceArray((T, k), np.int32)
        dv = rt.DeviceArray((T, k), np.uint16)
        ctx.lm_head_dev(dx.ptr, T, k, di.ptr, dv.ptr, logits=dl.ptr)
        ctx.synchronize()
        assert np.array_equal(dl.numpy(), got["logits"])
        assert np.array_equal(di.numpy(), got["ids"])
        assert np.array_equal(dv.numpy(), got["values"])
        for a in (dx, dl, di, dv):
            a.free()
        with pytest.raises(hm.FirewingError, match="shape"):
            ctx.load_lm_head_safetensors(tmp_path / "model.safetensors.index.json", "lm_head.weight", V + 1)
    logits, ids = reference(w, x, V, H, k)
    assert np.array_equal(got["logits"], logits)
    assert np.array_equal(got["ids"], ids)


def test_full_vocabulary_head():
    # the reference model's head: 248,320 x 2560 (src/text_output.rs:256-262)
    H, V, T, k = 2560, 248320, 2, 20
    with small_ctx(H) as ctx:
        ctx.generate_lm_head(V, SEED)
        x = hm.synth_hidden(SEED, T, H, False, first_token=123)
        got = ctx.lm_head(x, k)
    w = fo.synth_tensor(SEED, 0, 10, 0, V * H)
    logits, ids = reference(w, x, V, H, k)
    assert np.array_equal(got["logits"], logits)
    assert np.array_equal(got["ids"], ids)
