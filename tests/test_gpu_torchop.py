"""GPU decode + scatter of the reference connector's torch-op payloads (modes 0,
1, 2) against the oracle: every width of each mode, odd sizes and block
geometries, mixed modes in one launch with a refused header left unapplied, two
launches, the connector's restore of the reference tests' own inputs
(tests/test_vllm_connector.py:2437-2549) into a (2, 16, 8) layer, and payloads the
reference connector itself wrote or accepts (tests/golden/torchop_payloads.npz)
decoded to the words the reference restored."""

import numpy as np
import pytest

import oracle
from unchainkv_amd.connector import CodecConfig, SplitzipLayerCodec
from unchainkv_amd.trace import RecordingTrace

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def sz():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU visible")
    from unchainkv_amd import splitzip_cuda

    assert splitzip_cuda.available(), splitzip_cuda.load_error()
    return splitzip_cuda


def say(*parts):
    print("[case]", *parts, flush=True)


def u16(t):
    return t.detach().contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def words_for(rng, n, mode, width):
    if mode == 2:
        mag = rng.integers(0x20, 0x20 + (1 << width), n)
        high = mag | (rng.integers(0, 2, n) << 7)
    elif mode == 0:
        values = np.linspace(0, 255, 1 << width).astype(np.int64)
        values[1] = 0x7F if width == 1 else values[1]
        high = rng.choice(values, n)
    else:
        high = rng.integers(0, 256, n)
        low = rng.choice([3, 12], n) | (rng.choice([1, 5, 9, 15], n) << 4)
        return ((high << 8) | low).astype(np.uint16)
    return ((high << 8) | rng.integers(0, 256, n)).astype(np.uint16)


def run_batch(sz, bw, pool, requests, payload_words, marker=0x3C3C):
    """Payloads (list of (payload, words)) decoded through random block tables;
    returns (got layer words, expected layer words)."""
    rng = np.random.default_rng(bw + pool)
    perm = rng.permutation(pool).tolist()
    tables, at = [], 0
    for c in requests:
        tables.append(perm[at:at + c])
        at += c
    batch = sz.PagedBatch(tables, bw, "cuda")
    offsets, buf = [], bytearray()
    for payload, _ in payload_words:
        offsets.append(len(buf))
        buf += bytes(payload)
        buf += bytes((-len(buf)) % 7)          # odd alignments on purpose
    source = torch.tensor(list(buf), dtype=torch.uint8, device="cuda")
    layer = torch.full((2, pool, bw), marker, dtype=torch.int16, device="cuda").view(torch.bfloat16)
    got = sz.decode_torchop_paged(source, offsets, [len(p) for p, _ in payload_words], layer, batch)
    torch.cuda.synchronize()
    assert got == sum(2 * 2 * c * bw for c in requests)
    expected = np.full((2, pool, bw), marker, np.uint16)
    for (payload, words), t in zip(payload_words, tables):
        if words is not None:
            expected[:, t] = words.reshape(2, len(t), bw)
    return u16(layer).reshape(2, pool, bw), expected


@pytest.mark.parametrize("mode,width", [(2, w) for w in range(1, 7)] + [(0, w) for w in range(1, 8)]
                         + [(1, 0)])
def test_each_mode_and_width(sz, mode, width):
    say("torchop", mode, width)
    rng = np.random.default_rng(100 * mode + width)
    bw, requests = 2048, [3, 1, 4]
    items = []
    for c in requests:
        words = words_for(rng, 2 * c * bw, mode, width)
        payload = oracle.encode_torchop(words)
        assert payload is not None and payload[0] == mode
        assert np.array_equal(oracle.decode_torchop(payload, words.size), words)
        items.append((payload, words))
    got, expected = run_batch(sz, bw, 20, requests, items)
    assert np.array_equal(got, expected)


@pytest.mark.parametrize("bw", [16384, 40, 24])
def test_mixed_modes_odd_geometry_and_a_refused_header(sz, bw):
    say("torchop mixed", bw)
    rng = np.random.default_rng(bw)
    requests = [2, 3, 1, 2] if bw > 1000 else [20, 30, 10, 20]
    pool = 12 if bw > 1000 else 100
    items = []
    for c, (mode, width) in zip(requests, [(0, 5), (1, 0), (2, 3), (2, 6)]):
        words = words_for(rng, 2 * c * bw, mode, width)
        items.append((oracle.encode_torchop(words), words))
    bad = items[3][0].copy()
    bad[1] = 7                                  # width 7 is refused: left unapplied
    items[3] = (bad, None)
    got, expected = run_batch(sz, bw, pool, requests, items)
    assert np.array_equal(got, expected)


def test_two_launches(sz):
    say("torchop 70 payloads")
    rng = np.random.default_rng(70)
    bw, requests = 1024, [1] * 66 + [3, 2, 2, 1]
    items = []
    for r, c in enumerate(requests):
        mode = r % 3
        words = words_for(rng, 2 * c * bw, mode, 1 + r % 6)
        payload = oracle.encode_torchop(words)
        assert payload is not None
        items.append((payload, words))
    got, expected = run_batch(sz, bw, 100, requests, items)
    assert np.array_equal(got, expected)


@pytest.mark.parametrize("highs,low_mod", [
    ([0x3F, 0xBF, 0x40, 0xC0], 251),
    ([0x30 + i for i in range(32)], 256),
])
def test_connector_restores_the_reference_test_inputs(sz, highs, low_mod):
    """tests/test_vllm_connector.py:2437-2549: a (2, 16, 8) layer of 256 words sent
    by the reference's torch-op codec (sign/magnitude for both inputs) and restored
    into blocks 0..15."""
    say("torchop connector", len(highs))
    index = np.arange(256)
    words = ((np.array(highs)[index % len(highs)] << 8) | (index % low_mod)).astype(np.uint16)
    payload = oracle.encode_torchop(words)
    trace = RecordingTrace()
    codec = SplitzipLayerCodec(CodecConfig(), trace=trace)
    target = torch.zeros((2, 16, 8), dtype=torch.bfloat16, device="cuda")
    meta = {"raw_bytes": 512, "encoded_bytes": payload.size, "codec": "splitzip_bf16"}
    got = codec.load_kv_layer_batch(0, target, [(list(range(16)), bytes(payload), meta)])
    torch.cuda.synchronize()
    assert got == [(16, 512)]
    assert np.array_equal(u16(target).reshape(-1), words)
    assert ("splitzip_native_decode", {"blocks": 16, "bytes": 512, "mode": 2}) in trace.rows


def test_connector_restores_every_torchop_mode_in_one_call(sz):
    say("torchop connector mixed")
    rng = np.random.default_rng(5)
    bw, pool = 16 * 8 * 128, 24
    codec = SplitzipLayerCodec(CodecConfig(), trace=RecordingTrace())
    target = torch.zeros((2, pool, 16, 8, 128), dtype=torch.bfloat16, device="cuda")
    requests, expect = [], []
    for r, (mode, width) in enumerate([(0, 6), (1, 0), (2, 2)]):
        ids = [3 * r + 1, 3 * r + 5]
        words = words_for(rng, 2 * 2 * bw, mode, width)
        payload = oracle.encode_torchop(words)
        assert payload[0] == mode
        requests.append((ids, bytes(payload), {"raw_bytes": 2 * words.size,
                                               "encoded_bytes": payload.size}))
        expect.append((ids, words))
    assert codec.load_kv_layer_batch(0, target, requests) == [(2, 4 * 2 * bw)] * 3
    torch.cuda.synchronize()
    layer = u16(target).reshape(2, pool, bw)
    for ids, words in expect:
        assert np.array_equal(layer[:, ids].reshape(-1), words)


def _golden_cases():
    import json
    from pathlib import Path

    golden = Path(__file__).resolve().parent / "golden"
    index = json.loads((golden / "torchop_cases.json").read_text())["cases"]
    with np.load(golden / "torchop_payloads.npz") as z:
        arrays = {k: z[k] for k in z.files}
    return [dict(c, payload=arrays.get(c["key"] + "_payload"), out=arrays.get(c["key"] + "_out"))
            for c in index if c["kind"] in ("encode", "decode")
            and arrays.get(c["key"] + "_payload") is not None]


def test_reference_produced_payloads(sz):
    """Payloads the reference connector wrote (its torch-op encoders and
    hand-made ones its restore decoders accept or refuse; tests/golden/
    make_torchop_golden.py) decode to the words the reference restored, one launch
    per block geometry; refused payloads leave their blocks unapplied."""
    groups = {}
    for c in _golden_cases():
        groups.setdefault(c["block_words"], []).append(c)
    for bw, cases in sorted(groups.items()):
        say("torchop golden", bw, len(cases))
        requests = [c["blocks"] for c in cases]
        items = [(c["payload"], None if c["declined"] else c["out"]) for c in cases]
        got, expected = run_batch(sz, bw, sum(requests) + 5, requests, items)
        assert np.array_equal(got, expected), bw


def test_connector_restores_reference_produced_payloads(sz):
    """The encoder fixtures through the connector's restore (host validation, one
    pinned staging copy, the torch-op launch) into their own block spans."""
    cases = [c for c in _golden_cases() if c["kind"] == "encode" and not c["declined"]]
    say("torchop golden connector", len(cases))
    for c in cases:
        bw, nblk, start = c["block_words"], c["blocks"], c["start"]
        codec = SplitzipLayerCodec(CodecConfig(), trace=RecordingTrace())
        target = torch.zeros((2, start + nblk + 2, bw), dtype=torch.bfloat16, device="cuda")
        meta = {"raw_bytes": 2 * c["n"], "encoded_bytes": int(c["payload"].size)}
        ids = list(range(start, start + nblk))
        got = codec.load_kv_layer_batch(0, target, [(ids, bytes(c["payload"]), meta)])
        torch.cuda.synchronize()
        assert got == [(nblk, 2 * c["n"])], c["name"]
        assert np.array_equal(u16(target)[:, start:start + nblk].reshape(-1), c["out"]), c["name"]
