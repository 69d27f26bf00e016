"""GPU parity of the HIP palette codecs (fixed6 mode 3, fixed5 mode 4) against the
CPU oracle: byte-exact canonical encode (ascending palette, zeroed unused entries),
exact decode + scatter, overflow marking (byte 0 = 255 and nothing else written),
and decode of payloads whose palette is in another order (the reference builds
its palette first-come)."""

import numpy as np
import pytest

import oracle
from unchainkv_amd import codec_format

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def sz():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU visible")
    from unchainkv_amd import splitzip_cuda

    assert splitzip_cuda.available(), splitzip_cuda.load_error()
    return splitzip_cuda


def u16(t) -> np.ndarray:
    return t.detach().contiguous().view(torch.int16).cpu().numpy().view(np.uint16).reshape(-1)


def bf16(words: np.ndarray, device="cuda"):
    return torch.from_numpy(np.ascontiguousarray(words).view(np.int16).copy()).to(device).view(
        torch.bfloat16)


def palette_words(rng, n, distinct):
    highs = np.array(sorted(rng.choice(256, distinct, replace=False)), np.uint16)
    return ((highs[rng.integers(0, distinct, n)] << 8) | rng.integers(0, 256, n)).astype(np.uint16)


def say(*parts):
    print("[case]", *parts, flush=True)


def limit(bits):
    return 64 if bits == 6 else 32


# ---------------------------------------------------------------------------
# drop-in entry points (kvq_splitzip_bf16_encode_mode / decode_fixed6[_blocks])

@pytest.mark.parametrize("bits", [6, 5])
@pytest.mark.parametrize("n,shift", [(1000, 0), (8203, 3), (2 * 8192, 0), (2 * 8192, 15),
                                     (2 * 4096 * 5, 31), (2 * 4096 * 5, 15)])
@pytest.mark.parametrize("roomy", [True, False])
def test_dropin_encode_matches_oracle(sz, bits, n, shift, roomy):
    say("dropin palette encode", bits, n, shift, roomy)
    rng = np.random.default_rng(n + shift + bits)
    words = palette_words(rng, n, limit(bits) - 3)
    ref = oracle.palette_encode(words, bits)
    size = codec_format.palette_encoded_size(n, bits)
    minimum = ((size + 3) & ~3) + 1032  # the reference's capacity rule
    if 2 * n < minimum:
        short = torch.empty(minimum - 1, dtype=torch.uint8, device="cuda")
        assert sz.encode_bf16(bf16(words), short, bits=bits) == 0  # declined, as the reference
    capacity = max(2 * n, minimum) + 4096 if roomy else minimum
    backing = torch.full((capacity + shift + 64,), 0xA5, dtype=torch.uint8, device="cuda")
    out = backing[shift:shift + capacity]
    got = sz.encode_bf16(bf16(words), out, bits=bits)
    torch.cuda.synchronize()
    assert got == size
    assert bytes(out[:size].cpu().numpy()) == bytes(ref)
    assert bytes(backing[:shift].cpu().numpy()) == b"\xa5" * shift


@pytest.mark.parametrize("bits", [6, 5])
def test_dropin_encode_overflow_writes_only_the_mode_byte(sz, bits):
    say("dropin palette overflow", bits)
    rng = np.random.default_rng(3)
    n = 2 * 8192
    words = palette_words(rng, n, limit(bits) + 1)
    size = codec_format.palette_encoded_size(n, bits)
    out = torch.full((2 * n,), 0x3C, dtype=torch.uint8, device="cuda")
    assert sz.encode_bf16(bf16(words), out, bits=bits) == size
    torch.cuda.synchronize()
    host = out.cpu().numpy()
    assert host[0] == 255 and not (host[1:size] != 0x3C).any()


@pytest.mark.parametrize("bw,blocks,pool,contiguous", [
    (2048, 8, 40, False), (16384, 3, 12, False), (2048, 6, 20, True), (40, 30, 90, False),
    (48, 50, 120, True)])
def test_dropin_decode_fixed6_scatter(sz, bw, blocks, pool, contiguous):
    say("dropin fixed6 decode", bw, blocks, contiguous)
    rng = np.random.default_rng(bw + blocks)
    n = 2 * blocks * bw
    words = palette_words(rng, n, 50)
    payload = oracle.fixed6_encode(words)
    ids = (list(range(5, 5 + blocks)) if contiguous
           else rng.permutation(pool)[:blocks].tolist())
    target = torch.full((2, pool, bw), 1.5, dtype=torch.bfloat16, device="cuda")
    before = u16(target).reshape(2, pool, bw).copy()
    comp = torch.from_numpy(payload.copy()).cuda()
    assert sz.decode_fixed6(comp, target, ids, 2 * n) == 2 * n
    torch.cuda.synchronize()
    expected = before.copy()
    expected[:, ids] = words.reshape(2, blocks, bw)
    assert np.array_equal(u16(target).reshape(2, pool, bw), expected)


@pytest.mark.parametrize("blocks", [256, 257])
def test_dropin_decode_fixed6_host_table_limit(sz, blocks):
    """256 shuffled ids ride in the kernel arguments, 257 go through a device copy."""
    say("dropin fixed6 decode host table", blocks)
    rng = np.random.default_rng(blocks + 1)
    bw, pool = 1024, 600
    n = 2 * blocks * bw
    words = palette_words(rng, n, 40)
    comp = torch.from_numpy(oracle.fixed6_encode(words).copy()).cuda()
    ids = rng.permutation(pool)[:blocks].tolist()
    target = torch.zeros((2, pool, bw), dtype=torch.bfloat16, device="cuda")
    assert sz.decode_fixed6(comp, target, ids, 2 * n) == 2 * n
    got = u16(target).reshape(2, pool, bw)
    assert np.array_equal(got[:, ids].reshape(-1), words)
    assert not got[:, np.setdiff1d(np.arange(pool), ids)].any()


def test_dropin_decode_accepts_any_palette_order_and_skips_other_modes(sz):
    say("fixed6 permuted palette")
    rng = np.random.default_rng(9)
    bw, blocks, pool = 2048, 4, 10
    n = 2 * blocks * bw
    words = palette_words(rng, n, 7)
    canon = oracle.fixed6_encode(words)
    palette = list(canon[1:8])
    perm = [3, 6, 0, 5, 1, 2, 4]
    codes = oracle.unpack_bits_py(bytes(canon[65 + n:]), n, 6)
    remap = {old: new for new, old in enumerate(perm)}
    value = sum(remap[c] << (6 * i) for i, c in enumerate(codes))
    packed = value.to_bytes(len(canon) - 65 - n, "little")
    payload = bytes([3]) + bytes(palette[i] for i in perm) + bytes(57) + bytes(canon[65:65 + n]) + packed
    ids = [9, 2, 7, 4]
    target = torch.zeros((2, pool, bw), dtype=torch.bfloat16, device="cuda")
    comp = torch.tensor(list(payload), dtype=torch.uint8, device="cuda")
    assert sz.decode_fixed6(comp, target, ids, 2 * n) == 2 * n
    torch.cuda.synchronize()
    assert np.array_equal(u16(target).reshape(2, pool, bw)[:, ids].reshape(-1), words)
    # byte 0 other than 3: nothing is written
    comp[0] = 255
    fresh = torch.zeros_like(target)
    assert sz.decode_fixed6(comp, fresh, ids, 2 * n) == 2 * n
    torch.cuda.synchronize()
    assert not fresh.view(torch.int16).any()


# ---------------------------------------------------------------------------
# batched paged entry points

@pytest.mark.parametrize("bits", [6, 5])
@pytest.mark.parametrize("bw,pool,requests,offset", [
    (16384, 64, [8, 16, 3], 0),      # Llama-3-8B block: tile kernels
    (2048, 300, [8, 40, 17, 64], 0),  # 70B TP8 share: tile kernels
    (48, 400, [50, 7, 99], 0),        # small blocks: generic kernels
    (2048, 100, [10, 20], 1),         # KV view at a 2-byte offset: generic kernels
    (2048, 400, [3] * 70, 0),         # 70 payloads: two launches of 64 and 6
    (48, 600, [8] * 66, 0),           # 66 payloads on the generic kernels
])
def test_paged_encode_decode_matches_oracle(sz, bits, bw, pool, requests, offset):
    say("paged palette", bits, bw, requests, offset)
    rng = np.random.default_rng(bw * 7 + pool + bits)
    words = palette_words(rng, 2 * pool * bw + offset, limit(bits) - 2)
    # one request's blocks use few high bytes: its palette differs from the others'
    perm = rng.permutation(pool).tolist()
    kv_host = words[offset:].reshape(2, pool, bw)
    block_tables, at = [], 0
    for r in requests:
        block_tables.append(perm[at:at + r])
        at += r
    for b in block_tables[1]:
        kv_host[:, b] = (kv_host[:, b] & 0x01FF) | 0x3C00
    backing = bf16(np.concatenate([words[:offset], kv_host.reshape(-1)]))
    kv = backing[offset:].view(2, pool, bw)
    batch = sz.PagedBatch(block_tables, bw, "cuda")
    offsets, sizes, total = batch.palette_layout(bits)
    out = batch.new_palette_buffer(bits)
    out.fill_(0x5A)
    ws = batch.new_palette_workspace()
    assert sz.encode_bf16_paged(kv, batch, out, ws, bits=bits) == sum(sizes)
    torch.cuda.synchronize()
    host = out.cpu().numpy()
    for r, t in enumerate(block_tables):
        ref = oracle.palette_encode(kv_host[:, t].reshape(-1), bits)
        assert bytes(host[offsets[r]:offsets[r] + sizes[r]]) == bytes(ref), f"payload {r}"
    rperm = rng.permutation(pool).tolist()
    recv_tables, at = [], 0
    for r in requests:
        recv_tables.append(rperm[at:at + r])
        at += r
    recv = sz.PagedBatch(recv_tables, bw, "cuda")
    target = torch.zeros((2, pool, bw), dtype=torch.bfloat16, device="cuda")
    assert sz.decode_bf16_paged(out, offsets, sizes, target, recv, bits=bits) == \
        batch.total_raw_bytes
    torch.cuda.synchronize()
    got = u16(target).reshape(2, pool, bw)
    for src_t, dst_t in zip(block_tables, recv_tables):
        assert np.array_equal(got[:, dst_t], kv_host[:, src_t])
    used = {b for t in recv_tables for b in t}
    assert not got[:, [b for b in range(pool) if b not in used]].any()


@pytest.mark.parametrize("bits", [6, 5])
@pytest.mark.parametrize("shift", [1, 7])
def test_paged_decode_of_payloads_at_unaligned_offsets(sz, bits, shift):
    """Payloads from the oracle packed back to back at odd offsets (low bytes and
    codes at any byte address) decode on the tile kernels, exactly."""
    say("paged palette unaligned offsets", bits, shift)
    rng = np.random.default_rng(90 + bits + shift)
    bw, pool = 2048, 60
    kv_host = palette_words(rng, 2 * pool * bw, limit(bits) - 4).reshape(2, pool, bw)
    perm = rng.permutation(pool).tolist()
    block_tables = [perm[0:5], perm[5:6], perm[6:20]]
    payloads = [oracle.palette_encode(kv_host[:, t].reshape(-1), bits) for t in block_tables]
    offsets, packed = [], bytearray()
    for p in payloads:
        packed += bytes(shift)
        offsets.append(len(packed))
        packed += bytes(p)
    assert any(o % 16 for o in offsets)
    source = torch.tensor(list(packed), dtype=torch.uint8, device="cuda")
    recv_tables = [[(b + 11) % pool for b in t] for t in block_tables]
    recv = sz.PagedBatch(recv_tables, bw, "cuda")
    target = torch.zeros((2, pool, bw), dtype=torch.bfloat16, device="cuda")
    assert sz.decode_bf16_paged(source, offsets, [len(p) for p in payloads], target, recv,
                                bits=bits) == recv.total_raw_bytes
    torch.cuda.synchronize()
    got = u16(target).reshape(2, pool, bw)
    for src_t, dst_t in zip(block_tables, recv_tables):
        assert np.array_equal(got[:, dst_t], kv_host[:, src_t])


@pytest.mark.parametrize("bits", [6, 5])
def test_paged_overflow_marks_only_that_payload(sz, bits):
    say("paged palette overflow", bits)
    rng = np.random.default_rng(17)
    bw, pool = 2048, 40
    kv_host = palette_words(rng, 2 * pool * bw, 20).reshape(2, pool, bw)
    tables = [[1, 2, 3], [10, 11], [20, 21, 22, 23]]
    # payload 1 gets limit + 1 distinct high bytes
    spread = np.arange(limit(bits) + 1, dtype=np.uint16)
    kv_host[:, 10] = (spread[np.arange(bw) % spread.size] << 8) | 1
    batch = sz.PagedBatch(tables, bw, "cuda")
    offsets, sizes, _ = batch.palette_layout(bits)
    out = batch.new_palette_buffer(bits)
    out.fill_(0x5A)
    ws = batch.new_palette_workspace()
    assert sz.encode_bf16_paged(bf16(kv_host.reshape(-1)).view(2, pool, bw), batch, out, ws,
                                bits=bits) == sum(sizes)
    torch.cuda.synchronize()
    host = out.cpu().numpy()
    assert host[offsets[1]] == 255
    assert not (host[offsets[1] + 1:offsets[1] + sizes[1]] != 0x5A).any()
    for r in (0, 2):
        ref = oracle.palette_encode(kv_host[:, tables[r]].reshape(-1), bits)
        assert bytes(host[offsets[r]:offsets[r] + sizes[r]]) == bytes(ref)
