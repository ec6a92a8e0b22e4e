"""safetensors checkpoints into the resident banks (include/firewing_hip_moe.h
firewing_hip_safetensors_layer_plan / firewing_hip_load_layer_safetensors),
replacing the reference's slice readers (src/expert.rs:362-512) and mapped
catalog (src/checkpoint_catalog.rs:146-245, 405-443).

CPU tests: plans of checkpoints written by the `safetensors` library itself (an
independent writer) and by hand, single files and index + shards, and every
rejection the reference's readers make. GPU tests: a layer loaded from a
checkpoint holds exactly the file's bytes and computes the oracle's block.
"""
import json
import struct

import numpy as np
import pytest

from firewing_amd import hip_moe as hm

TINY = dict(hidden=64, intermediate=32, experts=16, top_k=4, shared_intermediate=32)
# gate_up is 64 MiB here: more than one 32 MiB staging chunk, with a tail
WIDE = dict(hidden=1024, intermediate=256, experts=72, top_k=8, shared_intermediate=256)


def layer_shapes(shape):
    H, I, E, Is = shape["hidden"], shape["intermediate"], shape["experts"], shape["shared_intermediate"]
    return [(E, H), (E, 2 * I, H), (E, H, I), (Is, H), (Is, H), (H, Is), (1, H)]


def layer_weights(rng, shape, scale=0.2):
    out = []
    for dims in layer_shapes(shape):
        v = (rng.standard_normal(int(np.prod(dims))) * scale).astype(np.float32)
        out.append((v.view(np.uint32) >> 16).astype(np.uint16).reshape(dims))
    return out


def names(layer):
    return [f"{hm.layer_prefix(layer)}.{t}" for t in hm.LAYER_TENSORS]


def save_with_library(path, tensors: dict, metadata=None):
    """Write with the safetensors package (bf16 through torch)."""
    import torch
    from safetensors.torch import save_file
    save_file({k: torch.from_numpy(v.view(np.int16)).view(torch.bfloat16) for k, v in tensors.items()},
              str(path), metadata=metadata)


def save_by_hand(path, entries, header_patch=None, raw_header=None, truncate=0):
    """entries: name -> (dtype, shape, bytes). Offsets are laid out in order;
    header_patch(header dict) may edit the header before it is written."""
    header, blobs, at = {}, [], 0
    for name, (dtype, shape, blob) in entries.items():
        header[name] = {"dtype": dtype, "shape": list(shape), "data_offsets": [at, at + len(blob)]}
        blobs.append(blob)
        at += len(blob)
    if header_patch:
        header_patch(header)
    text = raw_header if raw_header is not None else json.dumps(header).encode()
    data = struct.pack("<Q", len(text)) + text + b"".join(blobs)
    path.write_bytes(data[:len(data) - truncate] if truncate else data)


def plan(path, prefix, shape):
    return hm.safetensors_layer_plan(path, prefix, shape["hidden"], shape["intermediate"], shape["experts"],
                                     shape["shared_intermediate"])


def check_spans(spans, files, weights):
    for (off, nbytes, shard), w in zip(spans, weights):
        assert nbytes == w.nbytes
        got = np.fromfile(files[shard], dtype=np.uint16, count=w.size, offset=off)
        assert np.array_equal(got, w.ravel())


def test_plan_of_a_file_written_by_the_safetensors_library(tmp_path):
    rng = np.random.default_rng(1)
    w0, w1 = layer_weights(rng, TINY), layer_weights(rng, TINY)
    tensors = dict(zip(names(0), w0)) | dict(zip(names(1), w1))
    tensors["model.language_model.layers.1.self_attn.q_proj.weight"] = w1[3].copy()
    path = tmp_path / "model.safetensors"
    save_with_library(path, tensors, metadata={"format": "pt"})
    spans = plan(path, hm.layer_prefix(1), TINY)
    assert {s for _, _, s in spans} == {0}
    check_spans(spans, [path], w1)


def test_plan_through_an_index_and_two_shards(tmp_path):
    rng = np.random.default_rng(2)
    w = layer_weights(rng, TINY)
    n = names(3)
    save_with_library(tmp_path / "model-00001-of-00002.safetensors", dict(zip(n[:2], w[:2])))
    save_with_library(tmp_path / "model-00002-of-00002.safetensors", dict(zip(n[2:], w[2:])))
    index = {"metadata": {"total_size": 0},
             "weight_map": {k: f"model-0000{1 if i < 2 else 2}-of-00002.safetensors" for i, k in enumerate(n)}}
    (tmp_path / "model.safetensors.index.json").write_text(json.dumps(index))
    spans = plan(tmp_path / "model.safetensors.index.json", hm.layer_prefix(3), TINY)
    assert [s for _, _, s in spans] == [0, 0, 1, 1, 1, 1, 1]
    files = [tmp_path / "model-00001-of-00002.safetensors", tmp_path / "model-00002-of-00002.safetensors"]
    check_spans(spans, files, w)


def test_escaped_names_and_padded_header(tmp_path):
    # a tensor name spelt with JSON escapes, spaces after the object (the
    # library pads headers to 8 bytes), and a __metadata__ object
    rng = np.random.default_rng(3)
    w = layer_weights(rng, TINY)
    entries = {k: ("BF16", a.shape, a.tobytes()) for k, a in zip(names(0), w)}
    text = json.dumps({"__metadata__": {"format": "pt"},
                       **{k: {"dtype": d, "shape": list(s), "data_offsets": [0, 0]} for k, (d, s, _) in entries.items()}})
    at, header = 0, json.loads(text)
    for k, (_, _, b) in entries.items():
        header[k]["data_offsets"] = [at, at + len(b)]
        at += len(b)
    raw = json.dumps(header).replace('"model.language_model.layers.0.mlp.gate.weight"',
                                     '"model\\u002elanguage_model.layers.0.mlp.g\\u0061te.weight"')
    raw = (raw + " " * (-len(raw) % 8)).encode()
    path = tmp_path / "escaped.safetensors"
    save_by_hand(path, entries, raw_header=raw)
    check_spans(plan(path, hm.layer_prefix(0), TINY), [path], w)


def _entries(w, layer=0):
    return {k: ("BF16", a.shape, a.tobytes()) for k, a in zip(names(layer), w)}


@pytest.mark.parametrize("case,message", [
    ("missing", "tensor absent from shard: model.language_model.layers.0.mlp.experts.down_proj"),
    ("f16", "expected BF16, got F16"),
    ("shape", "mlp.experts.gate_up_proj: shape [16, 64, 32], expected [16, 64, 64]"),
    ("short_offsets", "payload layout mismatch"),
    ("truncated", "payload layout mismatch"),
    ("overlap", "overlapping tensor"),
    ("unknown_dtype", "unknown dtype Q4"),
    ("zero_dim", "empty shape"),
    ("duplicate", "duplicate member"),
    ("bad_json", "header"),
    ("header_zero", "invalid safetensors header"),
    ("header_huge", "invalid safetensors header"),
])
def test_rejections(tmp_path, case, message):
    rng = np.random.default_rng(4)
    w = layer_weights(rng, TINY)
    e = _entries(w)
    n = names(0)
    path = tmp_path / f"{case}.safetensors"
    if case == "missing":
        del e[n[2]]
        save_by_hand(path, e)
    elif case == "f16":
        e[n[5]] = ("F16",) + e[n[5]][1:]
        save_by_hand(path, e)
    elif case == "shape":
        a = w[1].reshape(16, 64, 64)[:, :, :32].copy()
        e[n[1]] = ("BF16", a.shape, a.tobytes())
        save_by_hand(path, e)
    elif case == "short_offsets":
        save_by_hand(path, e, header_patch=lambda h: h[n[6]]["data_offsets"].__setitem__(1, h[n[6]]["data_offsets"][1] - 2))
    elif case == "truncated":
        save_by_hand(path, e, truncate=2)
    elif case == "overlap":
        def patch(h):
            h[n[4]]["data_offsets"] = list(h[n[3]]["data_offsets"])
        save_by_hand(path, e, header_patch=patch)
    elif case == "unknown_dtype":
        e["model.language_model.layers.0.other"] = ("Q4", (4,), b"\0" * 8)
        save_by_hand(path, e)
    elif case == "zero_dim":
        e["model.language_model.layers.0.other"] = ("BF16", (0, 4), b"")
        save_by_hand(path, e)
    elif case == "duplicate":
        text = json.dumps({k: {"dtype": "BF16", "shape": [1], "data_offsets": [0, 2]} for k in ["a"]})
        save_by_hand(path, {"a": ("BF16", (1,), b"\0\0")}, raw_header=text.replace("}}", "}, \"a\": {}}").encode())
    elif case == "bad_json":
        save_by_hand(path, {"a": ("BF16", (1,), b"\0\0")}, raw_header=b'{"a": {"dtype": "BF16",')
    elif case == "header_zero":
        path.write_bytes(struct.pack("<Q", 0) + b"\0" * 64)
    elif case == "header_huge":
        path.write_bytes(struct.pack("<Q", (16 << 20) + 1) + b"{}" + b" " * 64)
    with pytest.raises(hm.FirewingError, match=message.replace("[", r"\[").replace("]", r"\]")):
        plan(path, hm.layer_prefix(0), TINY)


@pytest.mark.parametrize("shard,message", [
    ("../model.safetensors", "unbound checkpoint shard"),
    ("sub/model.safetensors", "unbound checkpoint shard"),
    ("absent.safetensors", "cannot open"),
])
def test_index_rejections(tmp_path, shard, message):
    rng = np.random.default_rng(5)
    w = layer_weights(rng, TINY)
    save_with_library(tmp_path / "model.safetensors", dict(zip(names(0), w)))
    wm = {k: "model.safetensors" for k in names(0)}
    wm[names(0)[2]] = shard
    (tmp_path / "model.safetensors.index.json").write_text(json.dumps({"weight_map": wm}))
    with pytest.raises(hm.FirewingError, match=message):
        plan(tmp_path / "model.safetensors.index.json", hm.layer_prefix(0), TINY)


def test_index_missing_tensor(tmp_path):
    rng = np.random.default_rng(6)
    w = layer_weights(rng, TINY)
    save_with_library(tmp_path / "model.safetensors", dict(zip(names(0), w)))
    wm = {k: "model.safetensors" for k in names(0)[:-1]}
    (tmp_path / "model.safetensors.index.json").write_text(json.dumps({"weight_map": wm}))
    with pytest.raises(hm.FirewingError, match="tensor absent from index: .*shared_expert_gate.weight"):
        plan(tmp_path / "model.safetensors.index.json", hm.layer_prefix(0), TINY)


# ---- GPU: loading into the resident banks ---------------------------------------------------

def write_index_checkpoint(tmp_path, layers: dict):
    """layers: checkpoint layer -> weights; tensors alternate between two shards."""
    shards = [{}, {}]
    wm = {}
    for layer, w in layers.items():
        for i, (k, a) in enumerate(zip(names(layer), w)):
            shards[i % 2][k] = a
            wm[k] = f"model-0000{i % 2 + 1}-of-00002.safetensors"
    for s, t in enumerate(shards):
        save_with_library(tmp_path / f"model-0000{s + 1}-of-00002.safetensors", t)
    index = tmp_path / "model.safetensors.index.json"
    index.write_text(json.dumps({"metadata": {}, "weight_map": wm}))
    return index


def read_back(ctx, layer, shape):
    return [ctx.read_tensor(layer, t + 1, 0, int(np.prod(d))) for t, d in enumerate(layer_shapes(shape))]


@pytest.mark.gpu
@pytest.mark.parametrize("shape", [TINY, WIDE], ids=["tiny", "wide"])
def test_loaded_layer_holds_the_file_and_computes_the_block(tmp_path, shape):
    from oracle import fw_oracle as fo
    rng = np.random.default_rng(7)
    w5, w9 = layer_weights(rng, shape, 0.05), layer_weights(rng, shape, 0.05)
    index = write_index_checkpoint(tmp_path, {5: w5, 9: w9})
    with hm.MoeContext(layers=2, **shape) as ctx:
        ctx.load_layer_safetensors(1, index, hm.layer_prefix(9))
        ctx.load_layer_safetensors(0, index, hm.layer_prefix(5))
        for layer, w in ((0, w5), (1, w9)):
            for t, (got, ref) in enumerate(zip(read_back(ctx, layer, shape), w)):
                assert np.array_equal(got, ref.ravel()), (layer, t + 1)
        # a failing plan copies nothing
        with pytest.raises(hm.FirewingError, match="tensor absent from index"):
            ctx.load_layer_safetensors(1, index, hm.layer_prefix(6))
        assert np.array_equal(ctx.read_tensor(1, 2, 0, 4096), w9[1].ravel()[:4096])
        x = (rng.standard_normal((2, shape["hidden"])).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
        got = ctx.sparse_moe_block(1, x)
        weights = dict(zip(("router", "gate_up", "down", "shared_gate", "shared_up", "shared_down",
                            "shared_expert_gate"), [a.ravel() for a in w9]))
        for t in range(2):
            ref = fo.sparse_moe_block(shape, weights, x[t])
            assert list(got["selected_experts"][t]) == list(ref["ids"])
            assert np.array_equal(got["out"][t], ref["out"])
