"""CPU checks of the container checker (oracle/fw_zstd.py): the BF16 byte
shuffle against the reference's own vector, and the libzstd binding's round
trips with the settings the reference's container builder uses."""
import numpy as np
import pytest

from oracle import fw_zstd as fz


def test_shuffle_matches_the_reference_vector():
    # tests/test_analyze_sequential_q2_zstd_oracle.py:14-19
    source = bytes.fromhex("0102030405060708")
    assert fz.shuffle_bf16(source) == bytes.fromhex("0103050702040608")
    assert fz.unshuffle_bf16(fz.shuffle_bf16(source)) == source
    with pytest.raises(ValueError):
        fz.shuffle_bf16(b"x")
    with pytest.raises(ValueError):
        fz.unshuffle_bf16(b"xyz")


def test_a_swapped_unshuffle_fails_the_vector():
    # the mistake a reader could make (high bytes first) does not pass the vector
    def swapped(shuffled):
        a = np.frombuffer(shuffled, dtype=np.uint8)
        half = len(a) // 2
        out = np.empty_like(a)
        out[1::2], out[0::2] = a[:half], a[half:]
        return out.tobytes()
    assert swapped(bytes.fromhex("0103050702040608")) != bytes.fromhex("0102030405060708")


def test_unshuffle_inverts_shuffle_on_bf16_weights():
    rng = np.random.default_rng(1)
    w = (rng.standard_normal(4099) * 0.02).astype(np.float32)
    src = ((w.view(np.uint32) >> 16).astype(np.uint16)).tobytes()
    sh = fz.shuffle_bf16(src)
    assert sh[:4099] == src[0::2] and sh[4099:] == src[1::2]
    assert fz.unshuffle_bf16(sh) == src


@pytest.mark.parametrize("level,checksum,content_size", [(1, False, True), (3, True, True), (19, False, False),
                                                         (-5, False, True)])
def test_libzstd_round_trip(level, checksum, content_size):
    rng = np.random.default_rng(level + 7)
    data = bytes(rng.integers(0, 8, size=200_000, dtype=np.uint8)) + b"expert " * 5000
    frame = fz.compress(data, level=level, checksum=checksum, content_size=content_size)
    assert frame[:4] == bytes.fromhex("28b52ffd")
    fhd = frame[4]
    assert bool(fhd & 4) == checksum
    assert ((fhd >> 6) != 0 or bool(fhd & 0x20)) == content_size
    assert fz.decompress(frame, len(data)) == data
    with pytest.raises(ValueError):
        fz.decompress(frame, len(data) + 1)


def test_expert_frame_has_the_builders_settings():
    # python-zstandard ZstdCompressor(level=1): content size, no checksum, no
    # dictionary (tools/build_sequential_shuffle_container.py:147,166-167)
    rng = np.random.default_rng(3)
    gu = rng.integers(0, 1 << 16, size=2 * 8 * 64, dtype=np.uint16)
    dn = rng.integers(0, 1 << 16, size=64 * 8, dtype=np.uint16)
    source, frame = fz.expert_frame(gu, dn)
    assert len(source) == 6 * 8 * 64
    fhd = frame[4]
    assert fhd & 4 == 0 and fhd & 3 == 0 and ((fhd >> 6) != 0 or fhd & 0x20)
    assert fz.unshuffle_bf16(fz.decompress(frame, len(source))) == source
    assert fz.version().count(".") == 2
