"""GPU torch-op encode (the reference connector's sender formats for small
requests: sign/magnitude mode 2, high-byte palette mode 0, nibble planes mode 1,
src/unchain_kv/vllm_connector.py:3204-3343) through the C ABI's plan and encode
entry points: byte-exact against the payloads the reference connector itself
wrote (tests/golden/torchop_payloads.npz, including its two declines), against
the oracle on seeded inputs of every mode and width with odd block geometries,
mixed modes and more than 64 requests (two launches), and round-tripped through
the torch-op decode."""

import json

import numpy as np
import pytest

import oracle

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


def encode_batch(sz, words_list, bw, pool, seed, marker=0x5A):
    """Each request's words (2 * blocks * bw, plane-major) laid into random blocks of
    a (2, pool, bw) layer, then planned and encoded in one batch. Returns (plans,
    payload bytes per request or None, tables, layer)."""
    rng = np.random.default_rng(seed)
    perm = rng.permutation(pool).tolist()
    layer_np = rng.integers(0, 1 << 16, (2, pool, bw)).astype(np.uint16)
    tables, at = [], 0
    for words in words_list:
        blocks = words.size // (2 * bw)
        tables.append(perm[at:at + blocks])
        layer_np[:, perm[at:at + blocks]] = words.reshape(2, blocks, bw)
        at += blocks
    layer = torch.from_numpy(layer_np.view(np.int16)).to("cuda").view(torch.bfloat16)
    batch = sz.PagedBatch(tables, bw, "cuda")
    plans = sz.plan_torchop_paged(layer, batch)
    assert plans is not None
    fields = sz.read_torchop_plans(plans.cpu().numpy())
    sizes = [size for _, size in fields]
    offsets, end = [], 0
    for r, size in enumerate(sizes):
        start = end + (r * 3) % 11               # odd offsets on purpose
        offsets.append(start)
        end = start + size
    out = torch.full((max(end, 1) + 64,), marker, dtype=torch.uint8, device="cuda")
    got = sz.encode_torchop_paged(layer, batch, plans, out, offsets, sizes)
    torch.cuda.synchronize()
    assert got == sum(sizes) or (got is None and not any(sizes))
    host = out.cpu().numpy()
    payloads = [bytes(host[o:o + s]) if s else None for o, s in zip(offsets, sizes)]
    # bytes between and after the payloads are untouched
    mask = np.ones(host.size, bool)
    for o, s in zip(offsets, sizes):
        mask[o:o + s] = False
    assert (host[mask] == marker).all()
    return fields, payloads, tables, layer, batch


def test_reference_connector_payloads(sz, golden_dir):
    """Every encoder fixture: the plan's mode and size and the payload bytes are the
    reference connector's; its declines are declined."""
    cases = [c for c in json.loads((golden_dir / "torchop_cases.json").read_text())["cases"]
             if c["kind"] == "encode"]
    data = np.load(golden_dir / "torchop_payloads.npz")
    assert len(cases) == 39
    for case in cases:
        say("torchop encode fixture", case["name"])
        words = data[case["key"] + "_words"]
        fields, payloads, *_ = encode_batch(sz, [words], case["block_words"],
                                            case["blocks"] + 5, seed=len(case["name"]))
        mode, size = fields[0]
        if case["declined"]:
            assert (mode, size, payloads[0]) == (255, 0, None), case["name"]
            continue
        expected = data[case["key"] + "_payload"]
        assert mode == case["mode"] and size == expected.size, case["name"]
        assert payloads[0] == expected.tobytes(), case["name"]


def words_for(rng, n, mode, width):
    """Words the reference's choice encodes with `mode` at `width` (nibble planes:
    `width` picks the plane widths)."""
    if mode == 2:
        lo = int(rng.integers(0, 128 - (1 << width) + 1))
        mag = rng.integers(lo, lo + (1 << width), n)
        mag[0], mag[-1] = lo, lo + (1 << width) - 1
        high = mag | (rng.integers(0, 2, n) << 7)
    elif mode == 0:
        # magnitudes spanning 7 bits (0 and 127 present), so sign/magnitude is out
        others = [v for v in range(256) if v not in (0x00, 0x7F)]
        values = np.array([0x00, 0x7F] + list(rng.choice(others, (1 << (width - 1)) - 1,
                                                         replace=False)))
        high = rng.choice(values, n)
        k = min(n, values.size)
        high[:k] = values[:k]
    else:
        high = rng.integers(0, 256, n)
        high[:min(n, 256)] = np.arange(min(n, 256))
        counts = [(2, 2), (3, 4), (16, 3), (1, 5)][width % 4]
        low = rng.choice(counts[0] if counts[0] > 1 else [7], n) | \
            (rng.choice(counts[1], n) << 4)
        return ((high << 8) | (low & 0xFF)).astype(np.uint16)
    return ((high << 8) | rng.integers(0, 256, n)).astype(np.uint16)


def check_against_oracle(sz, words_list, bw, pool, seed):
    fields, payloads, tables, layer, batch = encode_batch(sz, words_list, bw, pool, seed)
    for r, words in enumerate(words_list):
        expected = oracle.encode_torchop(words)
        if expected is None:
            assert fields[r] == (255, 0) and payloads[r] is None, r
            continue
        assert fields[r] == (int(expected[0]), expected.size), r
        assert payloads[r] == expected.tobytes(), r
    return fields, payloads, tables, layer, batch


@pytest.mark.parametrize("mode,width", [(2, w) for w in range(1, 7)] + [(0, w) for w in range(1, 8)]
                         + [(1, k) for k in range(4)])
@pytest.mark.parametrize("bw", [2048, 131, 7])
def test_seeded_modes_and_widths(sz, mode, width, bw):
    say("torchop encode", mode, width, bw)
    rng = np.random.default_rng(1000 * mode + 10 * width + bw)
    blocks = [3, 1, 5] if bw > 1000 else [37, 4, 291]
    words_list = [words_for(rng, 2 * c * bw, mode, width) for c in blocks]
    fields, *_ = check_against_oracle(sz, words_list, bw, sum(blocks) + 9, seed=width)
    # the largest request takes the format (a shorter one may not fit its header and
    # take the reference's next choice)
    assert fields[2][0] == mode


def test_mixed_modes_declines_and_two_launches(sz):
    """70 requests (two launches of the kernels' 64 payloads) of every mode plus
    incompressible ones, then each payload decoded by the torch-op decode into an
    independent block table."""
    say("torchop encode 70 requests")
    rng = np.random.default_rng(70)
    bw = 256
    words_list = []
    for r in range(70):
        blocks = 1 + r % 4
        n = 2 * blocks * bw
        if r % 9 == 4:
            words_list.append(rng.integers(0, 1 << 16, n).astype(np.uint16))  # declined
        else:
            mode = (2, 0, 1)[r % 3]
            width = 1 + r % (6 if mode == 2 else 7 if mode == 0 else 4)
            words_list.append(words_for(rng, n, mode, width))
    pool = sum(w.size // (2 * bw) for w in words_list) + 3
    fields, payloads, tables, layer, batch = check_against_oracle(sz, words_list, bw, pool, seed=7)
    assert {m for m, _ in fields} == {0, 1, 2, 255}
    # round trip of the encoded ones through the torch-op decode
    keep = [r for r in range(70) if payloads[r] is not None]
    # independent receiver blocks: a permutation split into runs
    perm = np.random.default_rng(11).permutation(pool).tolist()
    recv_tables, at = [], 0
    for r in keep:
        recv_tables.append(perm[at:at + len(tables[r])])
        at += len(tables[r])
    recv = sz.PagedBatch(recv_tables, bw, "cuda")
    buf = b"".join(payloads[r] for r in keep)
    offsets = np.cumsum([0] + [len(payloads[r]) for r in keep])[:-1].tolist()
    source = torch.tensor(list(buf), dtype=torch.uint8, device="cuda")
    target = torch.zeros((2, pool, bw), dtype=torch.bfloat16, device="cuda")
    got = sz.decode_torchop_paged(source, offsets, [len(payloads[r]) for r in keep], target, recv)
    torch.cuda.synchronize()
    assert got == sum(2 * words_list[r].size for r in keep)
    out = u16(target).reshape(2, pool, bw)
    for k, r in enumerate(keep):
        assert np.array_equal(out[:, recv_tables[k]].reshape(-1), words_list[r]), r


def test_llama3_8b_small_requests(sz):
    """Requests of 1-15 blocks of a Llama-3-8B layer (below 1 MiB: what the reference
    sends with torch ops), natural K/V statistics."""
    say("torchop encode llama3-8b small")
    from unchainkv_amd import workloads

    shape = workloads.LLAMA3_8B
    kv = workloads.make_kv_layer(torch, shape, 64, seed=3, layer=5, device=torch.device("cuda"))
    tables = [[1], [2, 9, 4], list(range(10, 25)), [63, 0]]
    batch = sz.PagedBatch(tables, shape.block_words, "cuda")
    plans = sz.plan_torchop_paged(kv, batch)
    fields = sz.read_torchop_plans(plans.cpu().numpy())
    sizes = [s for _, s in fields]
    offsets = np.cumsum([0] + sizes)[:-1].tolist()
    out = torch.zeros(sum(sizes), dtype=torch.uint8, device="cuda")
    assert sz.encode_torchop_paged(kv, batch, plans, out, offsets, sizes) == sum(sizes)
    host = out.cpu().numpy()
    layer = u16(kv).reshape(2, 64, -1)
    for r, t in enumerate(tables):
        expected = oracle.encode_torchop(layer[:, t].reshape(-1))
        assert expected is not None
        assert fields[r] == (int(expected[0]), expected.size)
        assert bytes(host[offsets[r]:offsets[r] + sizes[r]]) == expected.tobytes()


def test_more_than_256_requests(sz):
    """300 one-block requests (five presence launches of at most 64 payloads, two
    plan launches of at most 256): every plan and payload is the oracle's."""
    say("torchop encode 300 requests")
    rng = np.random.default_rng(300)
    bw = 1024
    words_list = []
    for r in range(300):
        mode = (2, 0, 1)[r % 3]
        width = 1 + r % (6 if mode == 2 else 7 if mode == 0 else 4)
        words_list.append(words_for(rng, 2 * bw, mode, width))
    fields, *_ = check_against_oracle(sz, words_list, bw, 310, seed=3)
    assert {m for m, _ in fields} <= {0, 1, 2, 255}


def test_misaligned_layer_takes_the_generic_kernels(sz):
    """Block words a multiple of 1024 but the layer 2 bytes off 16-byte alignment:
    plan, encode and decode take the generic kernels and still give the oracle's
    payloads and an exact round trip."""
    say("torchop misaligned layer")
    rng = np.random.default_rng(77)
    bw, pool = 2048, 12
    words_list = [words_for(rng, 2 * 3 * bw, 2, 4), words_for(rng, 2 * 2 * bw, 0, 5),
                  words_for(rng, 2 * 4 * bw, 1, 2)]
    tables = [[1, 7, 3], [10, 0], [2, 4, 5, 9]]
    host = rng.integers(0, 1 << 16, (2, pool, bw)).astype(np.uint16)
    for words, t in zip(words_list, tables):
        host[:, t] = words.reshape(2, len(t), bw)
    backing = torch.zeros(2 * pool * bw + 1, dtype=torch.int16, device="cuda")
    backing[1:] = torch.from_numpy(host.reshape(-1).view(np.int16)).cuda()
    layer = backing[1:].view(torch.bfloat16).view(2, pool, bw)
    assert layer.data_ptr() % 16 == 2
    batch = sz.PagedBatch(tables, bw, "cuda")
    plans = sz.plan_torchop_paged(layer, batch)
    fields = sz.read_torchop_plans(plans.cpu().numpy())
    sizes = [s for _, s in fields]
    offsets = np.cumsum([0] + sizes)[:-1].tolist()
    out = torch.zeros(sum(sizes), dtype=torch.uint8, device="cuda")
    assert sz.encode_torchop_paged(layer, batch, plans, out, offsets, sizes) == sum(sizes)
    got = out.cpu().numpy()
    for r, words in enumerate(words_list):
        expected = oracle.encode_torchop(words)
        assert fields[r] == (int(expected[0]), expected.size)
        assert bytes(got[offsets[r]:offsets[r] + sizes[r]]) == expected.tobytes(), r
    # decode into a misaligned receiver through other blocks
    recv_backing = torch.zeros_like(backing)
    target = recv_backing[1:].view(torch.bfloat16).view(2, pool, bw)
    recv_tables = [[11, 6, 8], [3, 1], [0, 2, 4, 5]]
    recv = sz.PagedBatch(recv_tables, bw, "cuda")
    assert sz.decode_torchop_paged(out, offsets, sizes, target, recv) == \
        sum(2 * w.size for w in words_list)
    torch.cuda.synchronize()
    res = target.view(torch.int16).cpu().numpy().view(np.uint16).reshape(2, pool, bw)
    for words, t in zip(words_list, recv_tables):
        assert np.array_equal(res[:, t].reshape(-1), words)
