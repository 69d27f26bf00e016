"""Oracle of the reference connector's torch-op codecs (payload modes 0, 1, 2,
src/unchain_kv/vllm_connector.py:3204-3404, 5168-5252), on the CPU.

Pinned by: the bit packing against an independent big-integer unpacking and the
C oracle's fixed5 decoder on the reference's own hand-built fixed5 payload
(tests/test_vllm_connector.py:2551-2584, packed with the same helper); the two
inputs of the reference's codec round-trip tests (:2437-2549), which the
reference's codec choice sends to sign/magnitude (their payloads must be smaller
than the words); round trips of every mode and width; the restore validation's
refusals; and planted mistakes that a wrong bit order or palette index would
make."""

import numpy as np
import pytest

import oracle


@pytest.mark.parametrize("width", [1, 2, 3, 4, 5, 6, 7])
def test_bit_packing_is_lsb_first(width):
    rng = np.random.default_rng(width)
    codes = rng.integers(0, 1 << width, 333)
    packed = oracle.pack_bits_lsb(codes, width)
    assert packed.size == (333 * width + 7) // 8
    assert oracle.unpack_bits_py(bytes(packed), 333, width) == codes.tolist()
    assert np.array_equal(oracle.unpack_bits_lsb(packed, 333, width), codes)


def test_reference_fixed5_payload_decodes_with_the_c_oracle():
    """tests/test_vllm_connector.py:2551-2584: palette 0x40..0x5f, code i % 32, low
    i % 251, codes packed by the torch helper (width 5)."""
    index = np.arange(256)
    palette = np.arange(0x40, 0x60, dtype=np.uint8)
    codes = index % 32
    low = (index % 251).astype(np.uint8)
    words = ((palette[codes].astype(np.uint16) << 8) | low).astype(np.uint16)
    comp = np.concatenate([np.array([4], np.uint8), palette, low, oracle.pack_bits_lsb(codes, 5)])
    assert comp.size == 33 + 256 + (256 * 5 + 7) // 8
    assert np.array_equal(oracle.palette_decode(comp, 256, 5), words)


@pytest.mark.parametrize("highs,low_mod", [
    ([0x3F, 0xBF, 0x40, 0xC0], 251),      # tests/test_vllm_connector.py:2459-2467
    ([0x30 + i for i in range(32)], 256),  # :2513-2521 (more than 16 high bytes)
])
def test_reference_roundtrip_inputs(highs, low_mod):
    index = np.arange(256)
    high = np.array(highs)[index % len(highs)]
    words = ((high << 8) | (index % low_mod)).astype(np.uint16)
    payload = oracle.encode_torchop(words)
    assert payload is not None and payload.size < 512 and payload[0] == 2
    assert np.array_equal(oracle.decode_torchop(payload, 256), words)


def _words_for(rng, n, mode, width):
    if mode == 2:   # magnitudes within 2**width, either sign
        mag = rng.integers(0x20, 0x20 + (1 << width), n)
        high = mag | (rng.integers(0, 2, n) << 7)
    elif mode == 0:  # 2**width distinct high bytes spread over the magnitude range
        values = np.linspace(0, 255, 1 << width).astype(np.int64)
        values[1] = 0x7F if width == 1 else values[1]
        high = rng.choice(values, n)
    else:            # every high byte, low nibbles of 2 and 4 values
        high = rng.integers(0, 256, n)
        low = rng.choice([3, 12], n) | (rng.choice([1, 5, 9, 15], n) << 4)
        return ((high << 8) | low).astype(np.uint16)
    return ((high << 8) | rng.integers(0, 256, n)).astype(np.uint16)


@pytest.mark.parametrize("mode,width", [(2, w) for w in range(1, 7)] + [(0, w) for w in range(1, 8)]
                         + [(1, 0)])
@pytest.mark.parametrize("n", [4000, 4093])
def test_each_mode_round_trips(mode, width, n):
    rng = np.random.default_rng(mode * 10 + width + n)
    words = _words_for(rng, n, mode, width)
    payload = oracle.encode_torchop(words)
    assert payload is not None and payload[0] == mode
    if mode != 1:
        assert payload[1] == width
    assert np.array_equal(oracle.decode_torchop(payload, n), words)


def test_nibble_plane_widths_and_layout():
    rng = np.random.default_rng(3)
    n = 5000
    w = (rng.integers(0, 16, n) | (rng.integers(0, 4, n) << 4) | (rng.integers(0, 2, n) << 8)
         | (rng.integers(0, 256, n) << 8)).astype(np.uint16)
    payload = oracle.encode_nibbles(w)
    widths = [int(x) for x in payload[1:5]]
    assert widths[0] == 4 and widths[1] == 2
    assert payload.size == 69 + sum((n * x + 7) // 8 for x in widths)
    assert np.array_equal(oracle.decode_torchop(payload, n), w)


def test_restore_validation_refuses_bad_payloads():
    rng = np.random.default_rng(4)
    words = _words_for(rng, 1000, 2, 3)
    good = oracle.encode_torchop(words)
    assert oracle.decode_torchop(good[:-1], 1000) is None          # size mismatch
    bad = good.copy()
    bad[1] = 7                                                      # sign/mag width 7
    assert oracle.decode_torchop(bad, 1000) is None
    pal = oracle.encode_palette(_words_for(rng, 1000, 0, 5))
    bad = pal.copy()
    bad[1] = 0
    assert oracle.decode_torchop(bad, 1000) is None
    nib = oracle.encode_nibbles(_words_for(rng, 1000, 1, 0))
    bad = nib.copy()
    bad[3] = 3
    assert oracle.decode_torchop(bad, 1000) is None
    assert oracle.decode_torchop(np.array([7], np.uint8), 1) is None


def test_planted_mistakes_are_caught():
    index = np.arange(256)
    high = np.array([0x30 + i for i in range(32)])[index % 32]
    words = ((high << 8) | index).astype(np.uint16)
    payload = oracle.encode_torchop(words)
    # most-significant-bit-first packing of the magnitudes decodes differently
    n, width = 256, int(payload[1])
    mag = oracle.unpack_bits_lsb(payload[3 + n + 32:], n, width)
    msb = np.packbits(((mag[:, None] >> np.arange(width)[::-1]) & 1).astype(np.uint8).reshape(-1))
    mutant = payload.copy()
    mutant[3 + n + 32:] = msb
    assert not np.array_equal(oracle.decode_torchop(mutant, n), words)
    # a palette read one entry off
    pal_words = _words_for(np.random.default_rng(9), 600, 0, 4)
    p0 = oracle.encode_palette(pal_words)
    shifted = p0.copy()
    shifted[2:257] = p0[3:258]
    assert not np.array_equal(oracle.decode_torchop(shifted, 600), pal_words)
