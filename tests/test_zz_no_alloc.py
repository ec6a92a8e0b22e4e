"""The route entry point that allocates nothing (firewing_hip_route_bf16_noalloc)
against the allocating one (firewing_hip_route_bf16), through the C ABI: two
calls in a row, the second with fewer tokens and experts, every id, score and
logit bit-identical, with the logits both in the library's scratch and in a
caller buffer."""
import numpy as np
import pytest

from firewing_amd import hip_moe as hm
from firewing_amd import hip_runtime as rt
from oracle import fw_oracle as fo

pytestmark = pytest.mark.gpu

SEED = 0x46495245


def _case(tokens, experts, width, top_k, layer):
    w = fo.synth_tensor(SEED, layer, 1, 0, experts * width)
    w.reshape(experts, width)[:, width - 1] = fo.synth_router_bias(SEED, layer, experts)
    x = fo.synth_hidden(SEED, tokens, width, first_token=300 + layer)
    return w, x


def _noalloc(w, x, tokens, experts, width, top_k, order, keep_logits, stream):
    dw, dx = rt.DeviceArray.from_numpy(w), rt.DeviceArray.from_numpy(x)
    ids = rt.DeviceArray((tokens, top_k), np.int32)
    scores = rt.DeviceArray((tokens, top_k), np.uint16)
    logits = rt.DeviceArray((tokens, experts), np.uint16) if keep_logits else None
    hm.route_noalloc_dev(dw.ptr, dx.ptr, tokens, experts, width, top_k, ids.ptr, scores.ptr,
                         logits.ptr if logits else None, order=order, stream=stream.handle)
    stream.synchronize()
    out = (ids.numpy(), scores.numpy(), logits.numpy() if logits else None)
    for a in (dw, dx, ids, scores) + ((logits,) if logits else ()):
        a.free()
    return out


@pytest.mark.parametrize("order", [hm.LOGITS_TREE32, hm.LOGITS_FOLD])
@pytest.mark.parametrize("keep_logits", [False, True])
def test_noalloc_route_matches_allocating_route(order, keep_logits):
    stream = rt.Stream()
    # two calls in a row on one stream: the second smaller, so stale scratch
    # from the first would show
    for tokens, experts, width, top_k, layer in ((700, 512, 2048, 10, 0), (9, 64, 256, 4, 1)):
        w, x = _case(tokens, experts, width, top_k, layer)
        ids, scores, logits = _noalloc(w, x, tokens, experts, width, top_k, order, keep_logits, stream)
        r_ids, r_scores, r_logits = hm.route(w, x, experts, width, top_k, order)
        assert np.array_equal(ids, r_ids), (tokens, experts)
        assert np.array_equal(scores, r_scores), (tokens, experts)
        if keep_logits:
            assert np.array_equal(logits, r_logits), (tokens, experts)
    stream.destroy()


def test_noalloc_route_rejects_oversized_scratch_and_nan():
    stream = rt.Stream()
    tokens, experts, width = 1025, 512, 64  # 1025 * 512 logits exceed the 1 MiB scratch
    w = np.zeros(experts * width, dtype=np.uint16)
    dw = rt.DeviceArray.from_numpy(w)
    dx = rt.DeviceArray((tokens, width), np.uint16)
    ids = rt.DeviceArray((tokens, 4), np.int32)
    scores = rt.DeviceArray((tokens, 4), np.uint16)
    with pytest.raises(hm.FirewingError, match="524288"):
        hm.route_noalloc_dev(dw.ptr, dx.ptr, tokens, experts, width, 4, ids.ptr, scores.ptr,
                             stream=stream.handle)
    # a NaN router weight makes token 0's in-model logits NaN: its ids read -1
    w[0] = 0x7FC0
    nan_w = rt.DeviceArray.from_numpy(w)
    x = rt.DeviceArray.from_numpy(fo.bf16_array([1.0] * width * 2).reshape(2, width))
    hm.route_noalloc_dev(nan_w.ptr, x.ptr, 2, experts, width, 4, ids.ptr, scores.ptr, stream=stream.handle)
    stream.synchronize()
    assert (ids.numpy()[:2] == -1).all()
    for a in (dw, dx, ids, scores, nan_w, x):
        a.free()
    stream.destroy()
