"""GPU decoding of the compressed expert container (src/compressed_overlap.rs):
frames made by libzstd decode on the GPU to exactly their source bytes, with the
BF16 byte shuffle undone and the output split at the gate_up / down boundary as
the reference's reader does (decompress_to_buffer, the EXPERT_BYTES check,
unshuffle_bf16, the install copy: src/compressed_overlap.rs:1541-1553), across
the format's block, literal and sequence-table kinds; bad frames report their
status; installs land in the resident banks a step reads."""
import numpy as np
import pytest

from firewing_amd import hip_moe as hm
from firewing_amd import hip_runtime as rt
from oracle import fw_oracle as fo
from oracle import fw_zstd as fz

pytestmark = pytest.mark.gpu

REAL = dict(hidden=2560, intermediate=640)  # src/decoder_layer.rs:15,40-42
EXPERT_BYTES = 6 * REAL["hidden"] * REAL["intermediate"]  # 9,830,400 (src/compressed_overlap.rs:28)


def bf16_weights(rng, n, scale=0.02):
    v = (rng.standard_normal(n) * scale).astype(np.float32)
    return (v.view(np.uint32) >> 16).astype(np.uint16)


def expert_source(rng, H, I):
    return bf16_weights(rng, 2 * I * H), bf16_weights(rng, H * I)


def run_decode(frames, contents, unshuffle, splits=None, max_frames=8, device_source=False):
    """Decode frames (bytes) into fresh device buffers; returns (statuses,
    decoded bytes per frame as head + tail)."""
    splits = splits or [c for c in contents]
    src = b"".join(frames)
    offs = np.cumsum([0] + [len(f) for f in frames])[:-1]
    heads = [rt.DeviceArray((max(1, s),), np.uint8) for s in splits]
    tails = [rt.DeviceArray((max(1, c - s),), np.uint8) for c, s in zip(contents, splits)]
    specs = [(int(o), len(f), c, h.ptr, t.ptr if c > s else None, s)
             for o, f, c, s, h, t in zip(offs, frames, contents, splits, heads, tails)]
    with hm.ZstdDecoder(max_frames, max(max(contents), 1)) as dec:
        if device_source:
            dsrc = rt.DeviceArray.from_numpy(np.frombuffer(src, dtype=np.uint8).copy())
            stream = rt.Stream()
            dec.decode_dev(dsrc.ptr, len(src), specs, unshuffle, stream.handle)
            try:
                st = dec.status(len(frames))
            except hm.FirewingError as e:
                st = e.statuses
            stream.synchronize()
            stream.destroy()
            dsrc.free()
        else:
            try:
                st = dec.decode(src, specs, unshuffle)
            except hm.FirewingError as e:
                st = e.statuses
    out = []
    for c, s, h, t in zip(contents, splits, heads, tails):
        b = h.numpy().tobytes()[:s] + (t.numpy().tobytes()[:c - s] if c > s else b"")
        out.append(b)
        h.free()
        t.free()
    return list(st), out


# The sequence pass's table entries: four bytes or two (the decoder picks per
# call by how many blocks must run at once; both forms are checked here).
TABLE_FORMS = ["wide", "narrow"]


@pytest.mark.parametrize("tables", TABLE_FORMS)
@pytest.mark.parametrize("level", [1, 3])
def test_real_shape_expert_frames(level, tables, monkeypatch):
    monkeypatch.setenv("FIREWING_ZSTD_SEQ_TABLES", tables)
    rng = np.random.default_rng(level)
    H, I = REAL["hidden"], REAL["intermediate"]
    sources, frames = [], []
    for _ in range(3 if level == 1 else 1):
        gu, dn = expert_source(rng, H, I)
        s, f = fz.expert_frame(gu, dn, level=level)
        assert len(s) == EXPERT_BYTES
        sources.append(s)
        frames.append(f)
    split = 2 * I * H * 2
    st, out = run_decode(frames, [EXPERT_BYTES] * len(frames), True, [split] * len(frames))
    assert st == [0] * len(frames)
    for s, o in zip(sources, out):
        assert o == s


def format_cases():
    rng = np.random.default_rng(5)
    words = [b"expert ", b"router ", b"the ", b"shared ", b"gate ", b"mixture ", b"token ", b"layer\n"]
    text = b"".join(words[i] for i in rng.integers(0, len(words), size=120_000))
    runs = b"".join(bytes([int(rng.integers(0, 4))]) * int(rng.integers(1, 200_000)) for _ in range(8))
    rnd = rng.integers(0, 256, size=300_001, dtype=np.uint8).tobytes()
    periodic = (b"abcdefg" * 40_000)[:250_000]
    w = bf16_weights(rng, 400_000).tobytes()
    cases = [
        ("text-1", text, dict(level=1)),
        ("text-5-checksum", text, dict(level=5, checksum=True)),
        ("text-19", text, dict(level=19)),
        ("text-neg", text, dict(level=-1)),
        ("text-no-size", text, dict(level=3, content_size=False)),
        ("text-window-10", text[:200_000], dict(level=3, window_log=10)),
        ("runs", runs, dict(level=1)),
        ("runs-12", runs, dict(level=12, checksum=True)),
        ("random", rnd, dict(level=1)),
        ("periodic", periodic, dict(level=1)),
        ("weights-plain-1", w, dict(level=1)),
        ("weights-shuffled-19", fz.shuffle_bf16(w[:300_000]), dict(level=19)),
        ("empty", b"", dict(level=3)),
    ]
    for n in (1, 2, 5, 17, 255, 256, 1000, 4097, 70_000, 131_072, 131_073):
        v = bytes(((np.arange(n) * 7 + rng.integers(0, 3, size=n)) & 0x3F).astype(np.uint8))
        cases.append((f"small-{n}", v, dict(level=3, checksum=True)))
    return cases


def pyarrow_cases():
    # frames from another encoder: pyarrow's bundled libzstd (a newer release
    # than the system's), when pyarrow is importable
    try:
        import pyarrow as pa
    except ImportError:
        return []
    rng = np.random.default_rng(17)
    w = bf16_weights(rng, 300_000).tobytes()
    words = [b"expert ", b"router ", b"gate ", b"token "]
    text = b"".join(words[i] for i in rng.integers(0, len(words), size=60_000))
    out = []
    for name, data, lvl in (("pa-weights-shuffled-1", fz.shuffle_bf16(w), 1), ("pa-weights-9", w, 9),
                            ("pa-text-19", text, 19), ("pa-text-neg", text, -3)):
        out.append((name, data, pa.Codec("zstd", compression_level=lvl).compress(data, asbytes=True)))
    return out


@pytest.mark.parametrize("tables", TABLE_FORMS)
def test_format_features(tables, monkeypatch):
    monkeypatch.setenv("FIREWING_ZSTD_SEQ_TABLES", tables)
    cases = format_cases()
    frames = [fz.compress(data, **kw) for _, data, kw in cases]
    extra = pyarrow_cases()
    cases += [(name, data, {}) for name, data, _ in extra]
    frames += [f for _, _, f in extra]
    for (_, data, _), f in zip(cases, frames):
        assert fz.decompress(f, len(data)) == data  # the frames are good
    st, out = run_decode(frames, [len(d) for _, d, _ in cases], False, max_frames=len(cases))
    for (name, data, _), s, o in zip(cases, st, out):
        assert s == 0, (name, hm.ZSTD_STATUS[s])
        assert o == data, name


def test_unshuffle_split_at_odd_places_and_chunked_calls():
    # more frames than the decoder holds (chunks of 2), splits that are not
    # word multiples, device-resident source
    rng = np.random.default_rng(9)
    sources = [bf16_weights(rng, n).tobytes() for n in (1, 3, 1000, 33_333, 70_001)]
    frames = [fz.compress(fz.shuffle_bf16(s), level=1) for s in sources]
    contents = [len(s) for s in sources]
    splits = [1, 5, 998, 2 * 33_333 - 2, 70_001]
    st, out = run_decode(frames, contents, True, splits, max_frames=2, device_source=True)
    assert st == [0] * len(frames)
    for s, o in zip(sources, out):
        assert o == s


def test_bad_frames_report_their_status():
    rng = np.random.default_rng(2)
    data = bf16_weights(rng, 60_000).tobytes()
    good = fz.compress(data, level=1)
    cases = [
        (b"\x00" + good[1:], len(data), hm.ZSTD_STATUS.index("bad magic")),
        (good[: len(good) // 2], len(data), hm.ZSTD_STATUS.index("truncated")),
        (good + b"\x00\x01", len(data), hm.ZSTD_STATUS.index("trailing bytes")),
        (good, len(data) - 2, hm.ZSTD_STATUS.index("content size")),
        (good, len(data), 0),
    ]
    st, out = run_decode([c[0] for c in cases], [c[1] for c in cases], False)
    assert st == [c[2] for c in cases]
    assert out[-1] == data


SMALL = dict(hidden=256, intermediate=64, experts=16, top_k=4, shared_intermediate=64)


def test_install_experts_then_block_matches_oracle():
    H, I, E = SMALL["hidden"], SMALL["intermediate"], SMALL["experts"]
    rng = np.random.default_rng(4)
    with hm.MoeContext(layers=2, **SMALL) as ctx, hm.ZstdDecoder(4, 6 * I * H) as dec:
        ctx.generate_layers(0, 2, 77, True)
        layer = 1
        w = {}
        for name, tensor, n in (("router", hm.ROUTER, E * H), ("gate_up", hm.GATE_UP, E * 2 * I * H),
                                ("down", hm.DOWN, E * H * I), ("shared_gate", hm.SHARED_GATE, 64 * H),
                                ("shared_up", hm.SHARED_UP, 64 * H), ("shared_down", hm.SHARED_DOWN, H * 64),
                                ("shared_expert_gate", hm.SHARED_EXPERT_GATE, H)):
            w[name] = ctx.read_tensor(layer, tensor, 0, n).copy()
        experts = [3, 7, 12, 0, 15]
        frames = []
        for e in experts:
            gu, dn = bf16_weights(rng, 2 * I * H, 0.2), bf16_weights(rng, H * I, 0.2)
            w["gate_up"][e * 2 * I * H:(e + 1) * 2 * I * H] = gu
            w["down"][e * H * I:(e + 1) * H * I] = dn
            frames.append(fz.expert_frame(gu, dn)[1])
        offs = np.cumsum([0] + [len(f) for f in frames])[:-1]
        ctx.install_experts_zstd(dec, layer, experts, b"".join(frames), offs, [len(f) for f in frames])
        assert np.array_equal(ctx.read_tensor(layer, hm.GATE_UP, 0, E * 2 * I * H), w["gate_up"])
        assert np.array_equal(ctx.read_tensor(layer, hm.DOWN, 0, E * H * I), w["down"])
        x = hm.synth_hidden(5, 2, H, True)
        got = ctx.sparse_moe_block(layer, x)
        for t in range(2):
            ref = fo.sparse_moe_block(SMALL, w, x[t], hm.LOGITS_TREE32)
            assert np.array_equal(got["out"][t], ref["out"])
        with pytest.raises(hm.FirewingError, match="repeated expert"):
            ctx.install_experts_zstd(dec, layer, [1, 1], b"".join(frames[:2]), offs[:2], [len(f) for f in frames[:2]])
        bad = bytearray(frames[0])
        bad[0] ^= 0xFF
        with pytest.raises(hm.FirewingError, match="not a zstd frame"):
            ctx.install_experts_zstd(dec, layer, [2], bytes(bad), [0], [len(bad)])


def test_install_real_shape_experts():
    H, I = REAL["hidden"], REAL["intermediate"]
    rng = np.random.default_rng(6)
    shape = dict(hidden=H, intermediate=I, experts=512, top_k=10, shared_intermediate=I)
    experts = [0, 17, 255, 300, 511]
    with hm.MoeContext(layers=1, **shape) as ctx, hm.ZstdDecoder(len(experts), EXPERT_BYTES) as dec:
        ctx.generate_layers(0, 1, 3, True)
        frames, srcs = [], []
        for e in experts:
            gu, dn = expert_source(rng, H, I)
            srcs.append((gu, dn))
            frames.append(fz.expert_frame(gu, dn)[1])
        offs = np.cumsum([0] + [len(f) for f in frames])[:-1]
        ctx.install_experts_zstd(dec, 0, experts, b"".join(frames), offs, [len(f) for f in frames])
        for e, (gu, dn) in zip(experts, srcs):
            assert np.array_equal(ctx.read_tensor(0, hm.GATE_UP, e * 2 * I * H, 2 * I * H), gu), e
            assert np.array_equal(ctx.read_tensor(0, hm.DOWN, e * H * I, H * I), dn), e
        # neighbours untouched
        ref = fo.synth_tensor(3, 0, hm.GATE_UP, 18 * 2 * I * H, 4096)
        assert np.array_equal(ctx.read_tensor(0, hm.GATE_UP, 18 * 2 * I * H, 4096), ref)


def test_install_from_container_file(tmp_path):
    # the reference's miss path: page-aligned preads of the records, then
    # decode + unshuffle + install (src/compressed_overlap.rs:1426-1560)
    from firewing_amd import container as fc
    H, I, E = SMALL["hidden"], SMALL["intermediate"], SMALL["experts"]
    rng = np.random.default_rng(8)
    weights = {}
    recs = []
    for layer in (0, 1):
        for e in range(E):
            gu, dn = bf16_weights(rng, 2 * I * H, 0.2), bf16_weights(rng, H * I, 0.2)
            weights[(layer, e)] = (gu, dn)
            recs.append((layer, e, gu, dn))
    fc.write_container(tmp_path / "experts.fwz", tmp_path / "experts.json", recs)
    c = fc.Container(tmp_path / "experts.json")
    with hm.MoeContext(layers=2, **SMALL) as ctx, hm.ZstdDecoder(E, 6 * I * H) as dec:
        ctx.generate_layers(0, 2, 12, True)
        for layer in (0, 1):
            c.install(ctx, dec, layer, list(range(E)), verify=True)
        for (layer, e), (gu, dn) in weights.items():
            assert np.array_equal(ctx.read_tensor(layer, hm.GATE_UP, e * 2 * I * H, 2 * I * H), gu)
            assert np.array_equal(ctx.read_tensor(layer, hm.DOWN, e * H * I, H * I), dn)
