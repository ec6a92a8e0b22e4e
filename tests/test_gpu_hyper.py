"""GPU parity of the hyper-connection (src/hyper_connection.rs:211-490), the
block's injection into the residual streams (src/decoder_layer.rs:587-607)
and the in-model MoE sublayer that joins them around the block
(src/decoder_layer.rs:451-607): every output bit-exact against the oracle.
Weights are seeded synthetic (no checkpoint is mounted)."""
import json

import numpy as np
import pytest

from firewing_amd import hip_moe as hm
from oracle import fw_oracle as fo

pytestmark = pytest.mark.gpu

SEED = 0x46495245
CFG = dict(hidden=2048, intermediate=512, experts=512, top_k=10, shared_intermediate=512)


def bf16(rng, shape, scale):
    v = (rng.standard_normal(shape) * scale).astype(np.float32)
    return (v.view(np.uint32) >> 16).astype(np.uint16)  # truncation: any bf16 pattern will do


def hyper_weights(rng, S, W, R):
    return {"hc_norm": bf16(rng, S * W, 0.1), "down": bf16(rng, (R, S * W), 0.02),
            "up": bf16(rng, (S * W, R), 0.05), "inject": bf16(rng, (S, S * W), 0.02)}


def oracle_hyper(x, w, S, W, R, inject=True):
    return fo.hyper_connection(x, w["hc_norm"], w["down"], w["up"], w["inject"] if inject else None, S, W, R)


@pytest.mark.parametrize("S,W,R,T", [(4, 2560, 320, 1), (4, 2560, 320, 3), (3, 1000, 96, 2), (2, 4098, 64, 1),
                                     (2, 5, 2, 2), (4, 2048, 320, 5)])
@pytest.mark.parametrize("inject", [True, False])
def test_hyper_connection_bit_exact(S, W, R, T, inject):
    rng = np.random.default_rng(S * 100000 + W + R + T)
    w = hyper_weights(rng, S, W, R)
    x = bf16(rng, (T, S * W), 1.0)
    got = hm.hyper_connection(x, w["hc_norm"], w["down"], w["up"], w["inject"] if inject else None, S, W, R)
    for t in range(T):
        ref = oracle_hyper(x[t], w, S, W, R, inject)
        for k in got:
            assert np.array_equal(got[k][t], ref[k]), (k, t)


def test_inject_residual_bit_exact():
    rng = np.random.default_rng(3)
    S, W, T = 4, 2560, 3
    post = bf16(rng, (T, S * W), 1.0)
    moe = bf16(rng, (T, W), 0.5)
    weights = bf16(rng, (T, S), 1.0)
    products, out = hm.inject_residual(post, moe, weights, S, W)
    for t in range(T):
        rp, ro = fo.inject_residual(post[t], moe[t], weights[t], S, W)
        assert np.array_equal(products[t], rp)
        assert np.array_equal(out[t], ro)


@pytest.fixture(scope="module")
def sublayer_ctx():
    with hm.MoeContext(layers=2, **CFG) as ctx:
        ctx.generate_layers(0, 2, SEED, True)
        yield ctx


def sublayer_reference(post, hw, S, R, layer, t):
    H = CFG["hidden"]
    hyper = oracle_hyper(post[t], hw, S, H, R)
    block = fo.synth_block_captures(CFG, SEED, layer, hyper["mixed"].reshape(1, H))
    products, out = fo.inject_residual(post[t], block["out"][0], hyper["injection_weights"], S, H)
    return hyper, block, products, out


@pytest.mark.parametrize("tokens", [1, 2, 4])
def test_moe_sublayer_bit_exact(sublayer_ctx, tokens):
    S, R, layer = 4, 320, 1
    rng = np.random.default_rng(40 + tokens)
    hw = hyper_weights(rng, S, CFG["hidden"], R)
    sublayer_ctx.install_hyper_connection(layer, S, R, hw["hc_norm"], hw["down"], hw["up"], hw["inject"])
    post = bf16(rng, (tokens, S * CFG["hidden"]), 1.0)
    got = sublayer_ctx.moe_sublayer(layer, post, captures=True)
    for t in range(tokens):
        hyper, block, products, out = sublayer_reference(post, hw, S, R, layer, t)
        for k in hm.HYPER_OUTPUTS:
            assert np.array_equal(got["hyper"][k][t], hyper[k]), (k, t)
        assert np.array_equal(got["moe_output"][t], block["out"][0])
        assert np.array_equal(got["block"]["selected_experts"][t], block["ids"][0])
        assert np.array_equal(got["block"]["router_logits"][t], block["logits"][0])
        for k in hm.VERIFIER_CAPTURES:
            assert np.array_equal(np.ravel(got["block"][k][t]), np.ravel(block[k][0])), (k, t)
        assert np.array_equal(got["mlp_injection_products"][t], products)
        assert np.array_equal(got["layer_output"][t], out)
    # the device-pointer form gives the same streams
    from firewing_amd import hip_runtime as rt
    dpost = rt.DeviceArray.from_numpy(post)
    dout = rt.DeviceArray(post.shape, np.uint16)
    sublayer_ctx.moe_sublayer_dev(layer, dpost.ptr, tokens, dout.ptr)
    sublayer_ctx.synchronize()
    assert np.array_equal(dout.numpy(), got["layer_output"])
    dpost.free()
    dout.free()


def test_hyper_connection_from_safetensors(sublayer_ctx, tmp_path):
    import torch
    from safetensors.torch import save_file
    S, R, H = 4, 320, CFG["hidden"]
    rng = np.random.default_rng(77)
    hw = hyper_weights(rng, S, H, R)
    pre = "model.language_model.layers.7.mlp_hyper_connection."
    names = {"hc_norm": "hc_norm.weight", "down": "input_mix_weight_down.weight",
             "up": "input_mix_weight_up.weight", "inject": "block_inject_weight.weight"}
    save_file({pre + names[k]: torch.from_numpy(v.view(np.int16)).view(torch.bfloat16) for k, v in hw.items()},
              str(tmp_path / "hc.safetensors"))
    (tmp_path / "model.safetensors.index.json").write_text(
        json.dumps({"weight_map": {pre + n: "hc.safetensors" for n in names.values()}}))
    sublayer_ctx.load_hyper_connection_safetensors(0, S, R, tmp_path / "model.safetensors.index.json",
                                                   hm.layer_prefix(7))
    post = bf16(rng, (2, S * H), 1.0)
    got = sublayer_ctx.moe_sublayer(0, post)
    for t in range(2):
        _, _, _, out = sublayer_reference(post, hw, S, R, 0, t)
        assert np.array_equal(got["layer_output"][t], out)
    with pytest.raises(hm.FirewingError, match="same for every layer"):
        sublayer_ctx.install_hyper_connection(1, S, 256, hw["hc_norm"], hw["down"][:256], hw["up"][:, :256],
                                              hw["inject"])
