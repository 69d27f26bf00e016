"""Fused Top-16 decode + decode attention against decode-then-attend.

The reference pairs its decoder with a separate attention (scripts/
bench_codec_attention.py, torch SDPA); no reference test checks attention outputs,
so parity here is against (a) the CPU oracle's decode followed by float64
attention, (b) attention over the original (pre-encode) words, which the exact
decode must reproduce, and (c) at the Llama-3-8B decode shape, the GPU decoder
followed by float32 attention. Tolerance: 1e-2 relative to each output row's
largest magnitude (bf16 output and bf16 softmax weights).
"""

import os

import numpy as np
import pytest

import oracle
from attention_ref import attention_f64

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

HEAD_DIM = 128
TOL = 1e-2
# seeds of the shape sweep below (UNCHAIN_KV_TEST_SEEDS=<count> for a wider one)
SEEDS = int(os.environ.get("UNCHAIN_KV_TEST_SEEDS", "16"))


@pytest.fixture(scope="module")
def sz():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU visible")
    from unchainkv_amd import splitzip_cuda

    assert splitzip_cuda.available(), splitzip_cuda.load_error()
    return splitzip_cuda


def say(*parts):
    print("[case]", *parts, flush=True)


def span_of(tokens):
    return -(-tokens // 16) * 16


def kv_words(rng, books, tokens, kv_heads, escape_rate):
    """Plane words [2][span][kv_heads][128] (span = tokens rounded up to whole
    16-token blocks) with exponents from the codebooks; escapes take exponents
    outside them."""
    shape = (span_of(tokens), kv_heads, HEAD_DIM)
    planes = []
    for p in range(2):
        book = np.frombuffer(books[16 * p:16 * (p + 1)], np.uint8).astype(np.uint16)
        exps = book[rng.integers(0, 16, shape)]
        outside = np.array([e for e in range(100, 140) if e not in set(books[16 * p:16 * p + 16])],
                           np.uint16)
        # an exact count per plane keeps every payload within its 0.5% capacity
        hits = rng.choice(exps.size, int(escape_rate * exps.size), replace=False)
        exps.reshape(-1)[hits] = outside[rng.integers(0, outside.size, hits.size)]
        sign = rng.integers(0, 2, shape).astype(np.uint16) << 15
        planes.append(sign | (exps << 7) | rng.integers(0, 128, shape).astype(np.uint16))
    return np.stack(planes)


def bf16_to_f64(words):
    return (words.astype(np.uint32) << 16).view(np.float32).astype(np.float64)


def encode_sequences(sz, words_per_seq, kv_heads, books):
    """Payload of each sequence through the batched encoder (block table in token
    order over a shared pool)."""
    bw = 16 * kv_heads * HEAD_DIM
    blocks = [w.shape[1] // 16 for w in words_per_seq]
    pool = sum(blocks)
    cache = np.zeros((2, pool, 16, kv_heads, HEAD_DIM), np.uint16)
    tables, at = [], 0
    for w, nb in zip(words_per_seq, blocks):
        ids = list(range(at, at + nb))
        cache[:, at:at + nb] = w.reshape(2, nb, 16, kv_heads, HEAD_DIM)
        tables.append(ids)
        at += nb
    kv = torch.from_numpy(cache.view(np.int16)).cuda().view(torch.bfloat16)
    batch = sz.PagedBatch(tables, bw, "cuda")
    out = batch.new_payload_buffer()
    assert sz.encode_top16_paged(kv, batch, out, batch.new_workspace(), codebooks=books) == \
        batch.total_encoded_bytes
    return out, batch


def random_q(rng, batch, q_heads):
    q = rng.standard_normal((batch, q_heads, HEAD_DIM)).astype(np.float32)
    qb = torch.from_numpy(q).to(torch.bfloat16)
    return qb.cuda(), qb.float().numpy().astype(np.float64)


def check_close(got, ref):
    for row_got, row_ref in zip(got.reshape(-1, HEAD_DIM), ref.reshape(-1, HEAD_DIM)):
        scale = max(np.abs(row_ref).max(), 1e-6)
        assert np.abs(row_got - row_ref).max() <= TOL * scale, (np.abs(row_got - row_ref).max(), scale)


@pytest.mark.parametrize("kv_heads,contexts,rate", [
    (2, [208, 64, 1040, 16], 0.004),
    (1, [3000, 4096, 1], 0.002),
    (4, [128, 2048, 80], 0.0),
    (1, [32 + 16 * (i % 7) for i in range(70)], 0.004),  # more than one launch of 64
])
def test_fused_attention_matches_oracle_decode_then_attend(sz, codebooks, kv_heads, contexts, rate):
    say("fused attention", kv_heads, contexts, rate)
    rng = np.random.default_rng(kv_heads * 101 + len(contexts))
    books = codebooks[6 * 32:7 * 32]
    tables = oracle.top16_tables(books)
    words = [kv_words(rng, books, t, kv_heads, rate) for t in contexts]
    payloads, batch = encode_sequences(sz, words, kv_heads, books)
    q, q64 = random_q(rng, len(contexts), 4 * kv_heads)
    out = sz.decode_attention_top16(q, payloads, batch.out_offsets, contexts, kv_heads,
                                    codebooks=books)
    torch.cuda.synchronize()
    assert out is not None
    got = out.float().cpu().numpy()
    host = payloads.cpu().numpy()
    for b, (w, t) in enumerate(zip(words, contexts)):
        a = batch.out_offsets[b]
        payload = host[a:a + batch.encoded_bytes[b]]
        assert payload[0] == 5
        decoded = oracle.top16_decode(payload, w.size, tables)
        assert np.array_equal(decoded, w.reshape(-1))  # the exact decode the kernel must match
        kv = bf16_to_f64(decoded).reshape(2, span_of(t), kv_heads, HEAD_DIM)[:, :t]
        check_close(got[b], attention_f64(q64[b], kv[0], kv[1]))


@pytest.mark.parametrize("seed", range(SEEDS))
def test_seeded_attention_shapes(sz, codebooks, seed):
    """Seeded sweep: 1, 2, 4 or 8 kv heads, one to six sequences of 1 to 3000
    tokens (partial last blocks included), escape rates up to 0.4 %, any layer's
    codebooks; every output row within the tolerance of the oracle's decode
    followed by float64 attention."""
    rng = np.random.default_rng(9000 + seed)
    kv_heads = int(rng.choice([1, 2, 4, 8]))
    contexts = rng.integers(1, 3001, int(rng.integers(1, 7))).tolist()
    rate = float(rng.choice([0.0, 0.001, 0.004]))
    layer = int(rng.integers(0, 32))
    say("seeded attention", seed, kv_heads, contexts, rate, layer)
    books = codebooks[32 * layer:32 * layer + 32]
    tables = oracle.top16_tables(books)
    words = [kv_words(rng, books, t, kv_heads, rate) for t in contexts]
    payloads, batch = encode_sequences(sz, words, kv_heads, books)
    q, q64 = random_q(rng, len(contexts), 4 * kv_heads)
    out = sz.decode_attention_top16(q, payloads, batch.out_offsets, contexts, kv_heads,
                                    codebooks=books)
    torch.cuda.synchronize()
    assert out is not None
    got = out.float().cpu().numpy()
    host = payloads.cpu().numpy()
    for b, (w, t) in enumerate(zip(words, contexts)):
        a = batch.out_offsets[b]
        decoded = oracle.top16_decode(host[a:a + batch.encoded_bytes[b]], w.size, tables)
        kv = bf16_to_f64(decoded).reshape(2, span_of(t), kv_heads, HEAD_DIM)[:, :t]
        check_close(got[b], attention_f64(q64[b], kv[0], kv[1]))


def test_escapes_change_the_result_and_are_applied(sz, codebooks):
    """Escapes carry the outliers: attention without them differs grossly, so a
    kernel that skipped them could not pass the comparison."""
    say("fused attention escapes")
    rng = np.random.default_rng(5)
    books = codebooks[:32]
    kv_heads, ctx = 2, 1024
    w = kv_words(rng, books, ctx, kv_heads, 0.0)
    # 0.4% escapes with exponents far above the codebooks in both planes
    for p in range(2):
        hit = rng.random(w[p].shape) < 0.004
        w[p][hit] = (w[p][hit] & 0x807F) | (np.uint16(140) << 7)
    payloads, batch = encode_sequences(sz, [w], kv_heads, books)
    q, q64 = random_q(rng, 1, 4 * kv_heads)
    out = sz.decode_attention_top16(q, payloads, batch.out_offsets, [ctx], kv_heads,
                                    codebooks=books)
    torch.cuda.synchronize()
    kv = bf16_to_f64(w.reshape(-1)).reshape(2, ctx, kv_heads, HEAD_DIM)
    ref = attention_f64(q64[0], kv[0], kv[1])
    check_close(out.float().cpu().numpy()[0], ref)
    no_esc = w.copy()
    for p in range(2):
        mask = ((no_esc[p] >> 7) & 0xFF) == 140
        no_esc[p][mask] = (no_esc[p][mask] & 0x807F) | (np.uint16(books[16 * p]) << 7)
    kv0 = bf16_to_f64(no_esc.reshape(-1)).reshape(2, ctx, kv_heads, HEAD_DIM)
    assert np.abs(attention_f64(q64[0], kv0[0], kv0[1]) - ref).max() > 10 * TOL * np.abs(ref).max()


def test_overflowed_or_unsorted_payload_gives_nan_for_that_sequence_only(sz, codebooks):
    say("fused attention nan marking")
    rng = np.random.default_rng(6)
    books = codebooks[:32]
    kv_heads = 1
    words = [kv_words(rng, books, 1024, kv_heads, 0.004) for _ in range(3)]
    payloads, batch = encode_sequences(sz, words, kv_heads, books)
    # sequence 0: mode 255; sequence 2: escape entries in reverse order
    payloads[batch.out_offsets[0]] = 255
    n = words[2].size
    a = batch.out_offsets[2]
    count = int.from_bytes(bytes(payloads[a + 1:a + 5].cpu().numpy()), "little")
    assert count > 300
    lo = a + 5 + n + n // 2
    entries = payloads[lo:lo + 5 * count].view(count, 5).flip(0).contiguous().view(-1)
    payloads[lo:lo + 5 * count] = entries
    q, _ = random_q(rng, 3, 4 * kv_heads)
    out = sz.decode_attention_top16(q, payloads, batch.out_offsets, [1024] * 3, kv_heads,
                                    codebooks=books).float().cpu()
    assert torch.isnan(out[0]).all() and torch.isnan(out[2]).all()
    assert torch.isfinite(out[1]).all()


@pytest.mark.parametrize("disorder", ["shuffled", "one_swap_at_the_end", "one_swap_at_the_start"])
def test_unordered_escape_list_gives_nan_for_every_head_of_that_sequence(sz, codebooks, disorder):
    """Escape lists written in another order (the reference's encoder appends in
    atomic order) are refused as a whole: every query head of the sequence is NaN,
    even heads whose own escapes were walked in order, and even when the one
    misplaced pair sits where no wave's walk meets it."""
    say("fused attention escape order", disorder)
    rng = np.random.default_rng(7)
    books = codebooks[:32]
    kv_heads = 4
    words = [kv_words(rng, books, 512, kv_heads, 0.004) for _ in range(3)]
    payloads, batch = encode_sequences(sz, words, kv_heads, books)
    n = words[1].size
    a = batch.out_offsets[1]
    count = int.from_bytes(bytes(payloads[a + 1:a + 5].cpu().numpy()), "little")
    assert count > 100
    lo = a + 5 + n + n // 2
    entries = payloads[lo:lo + 5 * count].view(count, 5).clone()
    if disorder == "shuffled":
        order = torch.from_numpy(rng.permutation(count)).cuda()
    else:
        order = torch.arange(count, device="cuda")
        i = count - 2 if disorder == "one_swap_at_the_end" else 0
        order[i], order[i + 1] = i + 1, i
    payloads[lo:lo + 5 * count] = entries[order].reshape(-1)
    q, _ = random_q(rng, 3, 4 * kv_heads)
    out = sz.decode_attention_top16(q, payloads, batch.out_offsets, [512] * 3, kv_heads,
                                    codebooks=books).float().cpu()
    assert torch.isnan(out[1]).all()
    assert torch.isfinite(out[0]).all() and torch.isfinite(out[2]).all()


@pytest.mark.parametrize("outliers", [0.0, 0.001])
def test_llama3_8b_decode_step_against_decode_then_attend(sz, outliers):
    """Llama-3-8B GQA (32 q heads, 8 kv heads), batch 32, 8192 tokens each, KV in
    the Top-16 format: the natural ~0.05% escapes, and the benchmark's input with
    0.1% of the elements replaced by outliers of magnitude logU[1e2, 1e4];
    reference = GPU decode into bf16 KV (checked equal to the original KV), then
    float32 attention."""
    from unchainkv_amd import workloads

    say("llama3-8b decode attention 32 x 8192", outliers)
    shape = workloads.LLAMA3_8B
    batch_size, ctx, kv_heads = 32, 8192, 8
    blocks = ctx // 16
    pool = batch_size * blocks
    kv = workloads.make_kv_layer(torch, shape, pool, seed=4, layer=0, device="cuda",
                                 outlier_rate=outliers)
    tables = [list(range(b * blocks, (b + 1) * blocks)) for b in range(batch_size)]
    books = workloads.fit_codebook(torch, kv, tables)
    batch = sz.PagedBatch(tables, shape.block_words, "cuda")
    payloads = batch.new_payload_buffer()
    assert sz.encode_top16_paged(kv, batch, payloads, batch.new_workspace(), codebooks=books)
    g = torch.Generator(device="cuda")
    g.manual_seed(7)
    q = torch.randn((batch_size, 32, HEAD_DIM), generator=g, device="cuda").to(torch.bfloat16)
    out = sz.decode_attention_top16(q, payloads, batch.out_offsets, [ctx] * batch_size, kv_heads,
                                    codebooks=books)
    # decode-then-attend: the codec's decoder restores the KV, then float32 attention
    restored = torch.zeros_like(kv)
    assert sz.decode_top16_paged(payloads, batch.out_offsets, batch.encoded_bytes, restored,
                                 batch, codebooks=books) == batch.total_raw_bytes
    assert torch.equal(restored.view(torch.int16), kv.view(torch.int16))
    k = restored[0].reshape(batch_size, ctx, kv_heads, HEAD_DIM).float()
    v = restored[1].reshape(batch_size, ctx, kv_heads, HEAD_DIM).float()
    qf = q.float().reshape(batch_size, kv_heads, 4, HEAD_DIM)
    kt = k.permute(0, 2, 3, 1).contiguous()                    # (b, h, d, t)
    s = torch.matmul(qf, kt) / HEAD_DIM ** 0.5                  # (b, h, 4, t)
    p = torch.softmax(s, dim=-1)
    ref = torch.matmul(p, v.permute(0, 2, 1, 3).contiguous())   # (b, h, 4, d)
    ref = ref.reshape(batch_size, 32, HEAD_DIM)
    torch.cuda.synchronize()
    escapes = sum(int.from_bytes(bytes(payloads[o + 1:o + 5].cpu().numpy()), "little")
                  for o in batch.out_offsets)
    assert escapes > (0.0008 if outliers else 0.0002) * 2 * pool * shape.block_words, escapes
    assert torch.isfinite(out.float()).all()
    err = (out.float() - ref).abs().amax(dim=-1)
    scale = ref.abs().amax(dim=-1).clamp_min(1e-6)
    assert (err <= TOL * scale).all(), float((err / scale).max())
