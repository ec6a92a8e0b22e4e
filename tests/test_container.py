"""CPU checks of the container format and reader (firewing_amd/container.py):
page-aligned read plans as src/ngram.rs:940-969 computes them, and a written
container whose records read back, checked by the oracle's libzstd decode and
unshuffle."""
import hashlib
import json

import numpy as np
import pytest

from firewing_amd import container as fc
from oracle import fw_zstd as fz


def test_aligned_read_plan():
    P = fc.PAGE_BYTES
    assert fc.aligned_read_plan(0, 1, 10 * P) == fc.ReadPlan(0, P, 0)
    assert fc.aligned_read_plan(P + 5, P, 10 * P) == fc.ReadPlan(P, 2 * P, 5)
    assert fc.aligned_read_plan(3 * P, 2 * P, 10 * P) == fc.ReadPlan(3 * P, 2 * P, 0)
    # the last page is clipped to the file
    assert fc.aligned_read_plan(9 * P + 10, 100, 9 * P + 200) == fc.ReadPlan(9 * P, 200, 10)
    for bad in ((0, 0, P), (0, P + 1, P), (-1, 4, P)):
        with pytest.raises(ValueError):
            fc.aligned_read_plan(*bad)
    with pytest.raises(ValueError):
        fc.aligned_read_plan(0, 4, P, page_bytes=3000)


def test_shuffle_matches_the_checker():
    rng = np.random.default_rng(0)
    b = rng.integers(0, 256, size=1000, dtype=np.uint8).tobytes()
    assert fc.shuffle_bf16(b) == fz.shuffle_bf16(b)
    assert fc.shuffle_bf16(bytes.fromhex("0102030405060708")) == bytes.fromhex("0103050702040608")


def test_container_round_trip(tmp_path):
    H, I = 64, 16
    rng = np.random.default_rng(1)
    experts = []
    for layer, expert in ((0, 3), (0, 9), (2, 1), (5, 511)):
        gu = rng.integers(0, 1 << 16, size=2 * I * H, dtype=np.uint16)
        dn = (rng.standard_normal(H * I) * 0.02).astype(np.float32).view(np.uint32) >> 16
        experts.append((layer, expert, gu, dn.astype(np.uint16)))
    m = fc.write_container(tmp_path / "c.fwz", tmp_path / "c.json", experts)
    assert m["source_bytes_per_expert"] == 6 * I * H
    c = fc.Container(tmp_path / "c.json")
    want = ["5:511", "0:3", "2:1"]
    data, offs, sizes = c.read(want, verify=True)
    for ident, o, s in zip(want, offs, sizes):
        layer, expert = map(int, ident.split(":"))
        gu, dn = next((g, d) for l, e, g, d in experts if (l, e) == (layer, expert))
        frame = data[o:o + s]
        source = fz.unshuffle_bf16(fz.decompress(frame, 6 * I * H))
        assert source == gu.tobytes() + dn.tobytes()
        assert hashlib.sha256(source).hexdigest() == c.records[ident]["source_sha256"]
    for r in m["records"]:
        assert r["offset"] % fc.PAGE_BYTES == 0


def test_manifest_validation(tmp_path):
    H, I = 32, 8
    rng = np.random.default_rng(2)
    gu, dn = rng.integers(0, 1 << 16, size=2 * I * H, dtype=np.uint16), rng.integers(0, 1 << 16, size=H * I,
                                                                                        dtype=np.uint16)
    fc.write_container(tmp_path / "c.fwz", tmp_path / "c.json", [(0, 0, gu, dn), (0, 1, gu, dn)])
    m = json.loads((tmp_path / "c.json").read_text())
    for mutate, msg in ((lambda m: m["records"][1].__setitem__("offset", 5), "page-aligned"),
                        (lambda m: m["records"][1].__setitem__("identity", "0:0"), "identity"),
                        (lambda m: m.__setitem__("container_file", "../c.fwz"), "plain file name"),
                        (lambda m: m["records"][1].__setitem__("offset", 1 << 30), "runs past")):
        mm = json.loads(json.dumps(m))
        mutate(mm)
        (tmp_path / "bad.json").write_text(json.dumps(mm))
        with pytest.raises(ValueError, match=msg):
            fc.Container(tmp_path / "bad.json")
    c = fc.Container(tmp_path / "c.json")
    bad = bytearray((tmp_path / "c.fwz").read_bytes())
    bad[10] ^= 1
    (tmp_path / "c.fwz").write_bytes(bytes(bad))
    with pytest.raises(ValueError, match="hash"):
        c.read(["0:0"], verify=True)
