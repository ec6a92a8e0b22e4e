"""GPU parity at the benchmark's full size: the 48-layer decode step with all
weights resident (~155 GB), compared bit for bit with the oracle's chained
step for every layer's expert ids, scores and block output."""
import numpy as np
import pytest

from firewing_amd import hip_moe as hm
from oracle import fw_oracle as fo

pytestmark = pytest.mark.gpu

SEED = 0x46495245
CFG = dict(hidden=2048, intermediate=512, experts=512, top_k=10, shared_intermediate=512)
LAYERS = 48


@pytest.fixture(scope="module")
def ctx48():
    with hm.MoeContext(layers=LAYERS, **CFG) as ctx:
        ctx.generate_layers(0, LAYERS, SEED, True)
        yield ctx


@pytest.mark.parametrize("tokens", [1, 4])
def test_step_48_layers_bit_exact(ctx48, tokens):
    x = hm.synth_hidden(SEED, tokens, CFG["hidden"], True, first_token=7 + tokens)
    resid, blocks, ids, scores = ctx48.moe_step(x)
    r_resid, r_blocks, r_ids, r_scores = fo.synth_step(CFG, SEED, LAYERS, x, threads=16)
    bad_layers = [l for l in range(LAYERS) if not np.array_equal(ids[l], r_ids[l])]
    assert bad_layers == [], f"expert ids differ at layers {bad_layers}"
    assert np.array_equal(scores, r_scores)
    assert np.array_equal(blocks, r_blocks)
    assert np.array_equal(resid, r_resid)


def test_step_48_layers_repeatable_and_device_path(ctx48):
    from firewing_amd import hip_runtime as rt
    x = hm.synth_hidden(SEED, 1, CFG["hidden"], True, first_token=99)
    first = ctx48.moe_step(x)[0]
    xd = rt.DeviceArray.from_numpy(x)
    rd = rt.DeviceArray(x.shape, np.uint16)
    stream = rt.Stream()
    for _ in range(3):
        ctx48.moe_step_dev(xd.ptr, 1, rd.ptr, stream=stream.handle)
    stream.synchronize()
    ctx48.synchronize()
    assert np.array_equal(rd.numpy(), first)
    assert np.array_equal(ctx48.moe_step(x)[0], first)
    stream.destroy()
