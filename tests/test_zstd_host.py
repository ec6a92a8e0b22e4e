"""The zstd format core (firewing_amd/csrc/fw_zstd.h: frame index, FSE and
Huffman tables, Huffman streams, sequence decoding; the functions the GPU
passes run) on the host under AddressSanitizer: frames made by libzstd decode
to their bytes, and corrupted frames decode or fail with a status without a
read or write outside the frame and the decoder's buffers."""
import struct
import subprocess

import numpy as np
import pytest

from firewing_amd import build as fw_build
from oracle import fw_zstd as fz


@pytest.fixture(scope="module")
def checker():
    if not fw_build.HOST_CHECK.is_file():
        fw_build.host_check()
    return str(fw_build.HOST_CHECK)


def cases():
    rng = np.random.default_rng(21)
    w = (rng.standard_normal(300_000) * 0.02).astype(np.float32)
    weights = ((w.view(np.uint32) >> 16).astype(np.uint16)).tobytes()
    words = [b"expert ", b"router ", b"gate ", b"mixture ", b"token ", b"layer\n"]
    text = b"".join(words[i] for i in rng.integers(0, len(words), size=40_000))
    runs = b"".join(bytes([int(rng.integers(0, 3))]) * int(rng.integers(1, 70_000)) for _ in range(6))
    out = []
    for level in (1, 3, 19):
        out.append((fz.shuffle_bf16(weights), dict(level=level)))
    out += [(weights, dict(level=1)), (text, dict(level=1)), (text, dict(level=19, checksum=True)),
            (text, dict(level=3, content_size=False)), (text[:100_000], dict(level=3, window_log=10)),
            (runs, dict(level=1)), (rng.integers(0, 256, 50_000, dtype=np.uint8).tobytes(), dict(level=1)),
            (b"", dict(level=3))]
    for n in (1, 17, 256, 1000, 4097, 131_073):
        out.append((bytes(((np.arange(n) * 7) & 0x3F).astype(np.uint8)), dict(level=3)))
    made = [(data, fz.compress(data, **kw)) for data, kw in out]
    try:  # frames from another encoder: pyarrow's bundled libzstd
        import pyarrow as pa
        for data, lvl in ((fz.shuffle_bf16(weights), 1), (text, 19), (weights, -3)):
            made.append((data, pa.Codec("zstd", compression_level=lvl).compress(data, asbytes=True)))
    except ImportError:
        pass
    return made


def write_cases(path, items):
    with open(path, "wb") as f:
        f.write(struct.pack("<I", len(items)))
        for data, frame in items:
            f.write(struct.pack("<QQ", len(data), len(frame)))
            f.write(frame)
            f.write(data)


def run(checker, *args):
    env = {"ASAN_OPTIONS": "detect_leaks=0:abort_on_error=0:exitcode=99", "PATH": "/usr/bin:/bin"}
    return subprocess.run([checker, *args], capture_output=True, text=True, env=env, timeout=600)


def test_libzstd_frames_decode_on_the_host_core(checker, tmp_path):
    items = cases()
    write_cases(tmp_path / "cases.bin", items)
    r = run(checker, "decode", str(tmp_path / "cases.bin"))
    assert r.returncode == 0, r.stdout + r.stderr
    assert r.stdout.count(" ok ") == len(items)


def test_corrupted_frames_stay_in_bounds(checker, tmp_path):
    items = cases()
    write_cases(tmp_path / "cases.bin", items)
    r = run(checker, "fuzz", str(tmp_path / "cases.bin"), "120", "0x5eed")
    # AddressSanitizer exits 99 on any read or write outside an allocation
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-4000:]
    counts = {int(a.split()[1].rstrip(":")): int(a.split()[2]) for a in r.stdout.splitlines() if a.startswith("status")}
    assert sum(counts.values()) > 0.9 * 120 * (len(items) - 1)
    assert sum(v for k, v in counts.items() if k != 0) > 0  # corruptions are reported, not decoded silently
