/*
 * CPU oracle for the splitzip bf16 KV-cache codec (Top-16 mode 5, fixed6 mode 3).
 *
 * TEST INFRASTRUCTURE ONLY. This file restates, in plain C, the algorithm of the
 * reference codec so the HIP kernels can be checked against it. Only tests/,
 * __graft_entry__.smoke() and the CPU-baseline leg of bench.py may load the
 * library built from it, and only to check results against or as the timed CPU
 * baseline.
 * The product path (unchainkv_amd) never links, imports or calls it.
 *
 * Canonical form. The reference encoder places escape entries with a global
 * atomicAdd (native/unchain_kv/kvq_splitzip_cuda.cu:177), so their order varies
 * between runs, and it never writes unused escape slots. The oracle emits the
 * canonical form: escapes in ascending position order, unused slots zeroed.
 * Every byte the reference writes deterministically (header, count, body,
 * nibble codes) is produced by the same per-element arithmetic.
 *
 * fixed6: the reference builds its 64-entry palette first-come through atomicCAS
 * (kvq_splitzip_cuda.cu:28-49), so palette order is nondeterministic; the
 * canonical palette here is the distinct high bytes in ascending order with the
 * unused palette bytes zeroed. Decoding reads the palette from the payload, so
 * any palette order decodes to the same words.
 *
 * Parity pins for every function are listed in tests/test_oracle_golden.py.
 */
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

#define SZ_EXPORT __attribute__((visibility("default")))

/* ---- closed-form sizes: kvq_splitzip_cuda.cu:389-391 (top16), :300-303 (fixed6/5) ---- */

SZ_EXPORT uint64_t sz_top16_escape_capacity(uint64_t n) { return (n + 199) / 200; }

SZ_EXPORT uint64_t sz_top16_encoded_size(uint64_t n) {
  return 5 + n + (n + 1) / 2 + 5 * sz_top16_escape_capacity(n);
}

SZ_EXPORT uint64_t sz_fixed6_encoded_size(uint64_t n) {
  return 65 + n + ((n + 3) / 4) * 3;
}

/* ---- 544-byte lookup table: splitzip_cuda.py:290-297 ----
 * bytes [p*256 + exp] -> code (255 = not in the codebook; a later code overwrites
 * an earlier one for a duplicated exponent), then the 32 codebook bytes. */
SZ_EXPORT void sz_top16_tables(const uint8_t* codebooks32, uint8_t* out544) {
  memset(out544, 255, 512);
  for (int plane = 0; plane < 2; ++plane)
    for (int code = 0; code < 16; ++code)
      out544[plane * 256 + codebooks32[plane * 16 + code]] = (uint8_t)code;
  memcpy(out544 + 512, codebooks32, 32);
}

/* ---- gather through a block table: vllm_connector.py:2827-2869 ----
 * Payload word order is plane (K then V), then block in block-table order, then
 * the block's words: the order of kv_layer[:, ids] made contiguous. */
SZ_EXPORT void sz_gather(const uint16_t* kv, uint64_t plane_stride, uint64_t block_stride,
                         uint64_t block_words, const int64_t* ids, uint64_t block_count,
                         uint16_t* out) {
  for (uint64_t p = 0; p < 2; ++p)
    for (uint64_t j = 0; j < block_count; ++j)
      memcpy(out + (p * block_count + j) * block_words,
             kv + p * plane_stride + (uint64_t)ids[j] * block_stride,
             block_words * sizeof(uint16_t));
}

/* ---- scatter into a paged cache: Top16DstIndex, kvq_splitzip_cuda.cu:210-224 ----
 * ids == NULL means the contiguous run block_start, block_start+1, ... */
static inline uint64_t dst_index(uint64_t index, uint64_t block_count, uint64_t block_words,
                                 uint64_t plane_stride, uint64_t block_stride,
                                 uint64_t block_start, const int64_t* ids) {
  uint64_t plane_words = block_count * block_words;
  uint64_t plane = index / plane_words;
  uint64_t in_plane = index % plane_words;
  uint64_t block = in_plane / block_words;
  uint64_t within = in_plane % block_words;
  uint64_t dst_block = ids ? (uint64_t)ids[block] : block_start + block;
  return plane * plane_stride + dst_block * block_stride + within;
}

SZ_EXPORT void sz_scatter(const uint16_t* words, uint64_t n, uint64_t block_count,
                          uint64_t block_words, uint64_t plane_stride, uint64_t block_stride,
                          uint64_t block_start, const int64_t* ids, uint16_t* kv) {
  for (uint64_t i = 0; i < n; ++i)
    kv[dst_index(i, block_count, block_words, plane_stride, block_stride, block_start, ids)] =
        words[i];
}

/* ---- Top-16 encode of one element: EncodeTop16, kvq_splitzip_cuda.cu:170-191 ---- */
static inline uint8_t body_byte(uint16_t w) {
  return (uint8_t)((w & 0x7F) | ((w >> 8) & 0x80));
}

/* Header and escape region: FinalizeTop16, kvq_splitzip_cuda.cu:197-208 (byte 0 =
 * 255 on overflow, count clamped to capacity); entries {u32 LE position, u8 exponent}
 * (.cu:179-185). Canonical: ascending order, zeroed padding. */
static void write_header(uint8_t* out, uint64_t n, uint64_t escapes) {
  uint64_t cap = sz_top16_escape_capacity(n);
  uint64_t count = escapes > cap ? cap : escapes;
  out[0] = escapes > cap ? 255 : 5;
  out[1] = (uint8_t)count;
  out[2] = (uint8_t)(count >> 8);
  out[3] = (uint8_t)(count >> 16);
  out[4] = (uint8_t)(count >> 24);
}

static inline void put_entry(uint8_t* entries, uint64_t slot, uint32_t pos, uint8_t exponent) {
  uint8_t* e = entries + slot * 5;
  e[0] = (uint8_t)pos;
  e[1] = (uint8_t)(pos >> 8);
  e[2] = (uint8_t)(pos >> 16);
  e[3] = (uint8_t)(pos >> 24);
  e[4] = exponent;
}

/* Preconditions of kvq_splitzip_bf16_encode_top16 (.cu:385-395) other than the
 * buffer capacity: 0 < n <= 2^32-1 and E(n) < 2n. Returns 0 where the reference
 * declines. */
SZ_EXPORT uint64_t sz_top16_encode(const uint16_t* words, uint64_t n, const uint8_t* tables,
                                   uint8_t* out) {
  if (n == 0 || n > 0xFFFFFFFFULL) return 0;
  uint64_t encoded = sz_top16_encoded_size(n);
  if (encoded >= 2 * n) return 0;
  uint64_t cap = sz_top16_escape_capacity(n);
  uint8_t* body = out + 5;
  uint8_t* codes = body + n;
  uint8_t* entries = codes + (n + 1) / 2;
  memset(entries, 0, cap * 5);
  uint64_t half = n / 2; /* plane = index >= count_words / 2 (.cu:172) */
  uint64_t slot = 0;
  for (uint64_t i = 0; i < n; ++i) {
    uint16_t w = words[i];
    unsigned exponent = (w >> 7) & 0xFF;
    unsigned code = tables[(i >= half ? 256u : 0u) + exponent];
    body[i] = body_byte(w);
    if (code == 255) {
      /* sequential scan: slots are taken in ascending position order */
      if (slot < cap) put_entry(entries, slot, (uint32_t)i, (uint8_t)exponent);
      ++slot;
      code = 0;
    }
    /* even index in the low nibble (.cu:191) */
    if (i & 1)
      codes[i >> 1] |= (uint8_t)((code & 0x0F) << 4);
    else
      codes[i >> 1] = (uint8_t)(code & 0x0F);
  }
  write_header(out, n, slot);
  return encoded;
}

/* Decode: DecodeTop16 + ApplyTop16Escapes, kvq_splitzip_cuda.cu:226-284. Words are
 * produced in payload order. If byte 0 != 5 nothing is written and 0 is returned
 * (the reference kernels return early but the C call still reports 2n). */
SZ_EXPORT int sz_top16_decode(const uint8_t* payload, uint64_t n, const uint8_t* tables,
                              uint16_t* words) {
  if (payload[0] != 5) return 0;
  const uint8_t* body = payload + 5;
  const uint8_t* codes = body + n;
  const uint8_t* codebooks = tables + 512;
  uint64_t half = n / 2;
  for (uint64_t i = 0; i < n; ++i) {
    unsigned code = (codes[i / 2] >> ((i % 2) * 4)) & 0x0F;
    unsigned exponent = codebooks[(i >= half ? 16u : 0u) + code];
    uint8_t v = body[i];
    words[i] = (uint16_t)((v & 0x7F) | ((uint16_t)(v & 0x80) << 8) | (uint16_t)(exponent << 7));
  }
  uint64_t cap = sz_top16_escape_capacity(n);
  uint64_t count = (uint64_t)payload[1] | ((uint64_t)payload[2] << 8) |
                   ((uint64_t)payload[3] << 16) | ((uint64_t)payload[4] << 24);
  const uint8_t* entries = codes + (n + 1) / 2;
  for (uint64_t slot = 0; slot < count && slot < cap; ++slot) {
    const uint8_t* e = entries + slot * 5;
    uint64_t pos = (uint64_t)e[0] | ((uint64_t)e[1] << 8) | ((uint64_t)e[2] << 16) |
                   ((uint64_t)e[3] << 24);
    if (pos >= n) continue;
    words[pos] = (uint16_t)((words[pos] & 0x807F) | ((unsigned)e[4] << 7));
  }
  return 1;
}

/* Decode straight into a paged cache (decode + scatter in one call). */
SZ_EXPORT int sz_top16_decode_scatter(const uint8_t* payload, uint64_t n, const uint8_t* tables,
                                      uint64_t block_count, uint64_t block_words,
                                      uint64_t plane_stride, uint64_t block_stride,
                                      uint64_t block_start, const int64_t* ids, uint16_t* kv) {
  uint16_t* words = (uint16_t*)malloc(n * sizeof(uint16_t));
  if (!words) return -1;
  int ok = sz_top16_decode(payload, n, tables, words);
  if (ok)
    sz_scatter(words, n, block_count, block_words, plane_stride, block_stride, block_start, ids,
               kv);
  free(words);
  return ok;
}

/* ---- exponent histogram per plane: vllm_connector.py:2871-2904 ----
 * counts[p*256 + ((w >> 7) & 0xFF)] over the K plane (p=0, first n/2 words) and the
 * V plane (p=1). */
SZ_EXPORT void sz_exponent_histogram(const uint16_t* words, uint64_t n, uint64_t* counts) {
  memset(counts, 0, 512 * sizeof(uint64_t));
  uint64_t half = n / 2;
  for (uint64_t i = 0; i < n; ++i) counts[(i >= half ? 256 : 0) + ((words[i] >> 7) & 0xFF)]++;
}

/* ---- palette codecs: fixed6 (mode 3) and fixed5 (mode 4) ----
 * kvq_splitzip_cuda.cu:20-111 (encode), :113-144 (fixed6 decode); the fixed5 decode
 * follows the connector's torch decoder for mode 4 (vllm_connector.py:5266-5275:
 * LSB-first 5-bit codes, `_unpack_splitzip_bits` :3345-3404).
 * Payload: [mode][palette of high bytes: 64 (fixed6) or 32 (fixed5) bytes][n low
 * bytes][codes: groups of 4 x 6 bits in 3 bytes, or 8 x 5 bits in 5 bytes,
 * little-endian, first word in the low bits]. More distinct high bytes than
 * palette entries: byte 0 = 255 and nothing else is written (.cu:58-61, 86-88).
 * Canonical palette: ascending, zero padded. */
SZ_EXPORT uint64_t sz_palette_encoded_size(uint64_t n, int bits) {
  return bits == 6 ? 65 + n + ((n + 3) / 4) * 3 : 33 + n + ((n + 7) / 8) * 5;
}

SZ_EXPORT uint64_t sz_palette_encode(const uint16_t* words, uint64_t n, int bits, uint8_t* out) {
  if (n == 0 || (bits != 5 && bits != 6)) return 0;
  const int limit = bits == 6 ? 64 : 32, group = bits == 6 ? 4 : 8, group_bytes = bits == 6 ? 3 : 5;
  const uint64_t encoded = sz_palette_encoded_size(n, bits);
  if (encoded >= 2 * n) return 0;
  uint8_t present[256] = {0};
  for (uint64_t i = 0; i < n; ++i) present[words[i] >> 8] = 1;
  int rank[256];
  int distinct = 0;
  for (int h = 0; h < 256; ++h) rank[h] = present[h] ? distinct++ : -1;
  if (distinct > limit) {
    out[0] = 255;
    return encoded;
  }
  out[0] = (uint8_t)(bits == 6 ? 3 : 4);
  memset(out + 1, 0, (size_t)limit);
  for (int h = 0; h < 256; ++h)
    if (rank[h] >= 0) out[1 + rank[h]] = (uint8_t)h;
  uint8_t* low = out + 1 + limit;
  uint8_t* codes = low + n;
  for (uint64_t g = 0; g < (n + group - 1) / group; ++g) {
    uint64_t packed = 0;
    for (int k = 0; k < group; ++k) {
      uint64_t i = g * group + k;
      if (i >= n) break;
      low[i] = (uint8_t)(words[i] & 0xFF);
      packed |= (uint64_t)(rank[words[i] >> 8] & (limit - 1)) << (k * bits);
    }
    for (int b = 0; b < group_bytes; ++b) codes[g * group_bytes + b] = (uint8_t)(packed >> (8 * b));
  }
  return encoded;
}

SZ_EXPORT int sz_palette_decode(const uint8_t* payload, uint64_t n, int bits, uint16_t* words) {
  const int limit = bits == 6 ? 64 : 32, group = bits == 6 ? 4 : 8, group_bytes = bits == 6 ? 3 : 5;
  if (payload[0] != (bits == 6 ? 3 : 4)) return 0;
  const uint8_t* palette = payload + 1;
  const uint8_t* low = payload + 1 + limit;
  const uint8_t* codes = low + n;
  for (uint64_t i = 0; i < n; ++i) {
    uint64_t g = i / group, packed = 0;
    for (int b = 0; b < group_bytes; ++b) packed |= (uint64_t)codes[g * group_bytes + b] << (8 * b);
    uint32_t code = (uint32_t)(packed >> ((i % group) * bits)) & (uint32_t)(limit - 1);
    words[i] = (uint16_t)(((uint16_t)palette[code] << 8) | low[i]);
  }
  return 1;
}

SZ_EXPORT uint64_t sz_fixed6_encode(const uint16_t* words, uint64_t n, uint8_t* out) {
  return sz_palette_encode(words, n, 6, out);
}

SZ_EXPORT int sz_fixed6_decode(const uint8_t* payload, uint64_t n, uint16_t* words) {
  return sz_palette_decode(payload, n, 6, words);
}

/* ---- multi-threaded CPU baseline: gather + canonical Top-16 encode of a batch ----
 * Payload r holds the blocks ids[block_offsets[r] .. block_offsets[r+1]) of one
 * paged layer; its bytes go to out + out_offsets[r]. Work is split into chunks of
 * `chunk` words so every core has work; escapes are placed in ascending order by a
 * second pass over the per-chunk counts. */
typedef struct {
  uint64_t payload, lo, hi, escapes, base;
} sz_chunk;

static uint16_t load_paged(const uint16_t* kv, uint64_t plane_stride, uint64_t block_stride,
                           uint64_t block_words, const int64_t* ids, uint64_t block_count,
                           uint64_t i) {
  uint64_t plane_words = block_count * block_words;
  uint64_t p = i / plane_words, r = i % plane_words;
  return kv[p * plane_stride + (uint64_t)ids[r / block_words] * block_stride + r % block_words];
}

SZ_EXPORT int sz_top16_encode_paged_batch(const uint16_t* kv, uint64_t plane_stride,
                                          uint64_t block_stride, uint64_t block_words,
                                          const int64_t* ids, const uint64_t* block_offsets,
                                          uint64_t payloads, uint8_t* out,
                                          const uint64_t* out_offsets, const uint8_t* tables,
                                          uint64_t chunk, int threads) {
  if (chunk == 0 || (chunk & 1)) return -1;
  uint64_t total = 0;
  for (uint64_t r = 0; r < payloads; ++r) {
    uint64_t n = 2 * (block_offsets[r + 1] - block_offsets[r]) * block_words;
    total += (n + chunk - 1) / chunk;
  }
  sz_chunk* chunks = (sz_chunk*)calloc(total ? total : 1, sizeof(sz_chunk));
  if (!chunks) return -1;
  uint64_t c = 0;
  for (uint64_t r = 0; r < payloads; ++r) {
    uint64_t n = 2 * (block_offsets[r + 1] - block_offsets[r]) * block_words;
    for (uint64_t lo = 0; lo < n; lo += chunk) {
      chunks[c].payload = r;
      chunks[c].lo = lo;
      chunks[c].hi = lo + chunk < n ? lo + chunk : n;
      ++c;
    }
  }
#ifdef _OPENMP
  if (threads > 0) omp_set_num_threads(threads);
#else
  (void)threads;
#endif
  /* pass 1: body + codes + escape counts per chunk */
#pragma omp parallel for schedule(dynamic, 4)
  for (int64_t k = 0; k < (int64_t)total; ++k) {
    sz_chunk* ch = &chunks[k];
    uint64_t r = ch->payload;
    const int64_t* pid = ids + block_offsets[r];
    uint64_t nblk = block_offsets[r + 1] - block_offsets[r];
    uint64_t n = 2 * nblk * block_words;
    uint8_t* o = out + out_offsets[r];
    uint8_t* body = o + 5;
    uint8_t* codes = body + n;
    uint64_t half = n / 2, esc = 0;
    for (uint64_t i = ch->lo; i < ch->hi; ++i) {
      uint16_t w = load_paged(kv, plane_stride, block_stride, block_words, pid, nblk, i);
      unsigned e = (w >> 7) & 0xFF;
      unsigned code = tables[(i >= half ? 256u : 0u) + e];
      body[i] = body_byte(w);
      if (code == 255) {
        ++esc;
        code = 0;
      }
      if (i & 1)
        codes[i >> 1] |= (uint8_t)((code & 0x0F) << 4);
      else
        codes[i >> 1] = (uint8_t)(code & 0x0F);
    }
    ch->escapes = esc;
  }
  /* prefix over chunks of each payload; header; zero the escape region */
  for (uint64_t k = 0, r = (uint64_t)-1, run = 0; k < total; ++k) {
    if (chunks[k].payload != r) {
      r = chunks[k].payload;
      run = 0;
    }
    chunks[k].base = run;
    run += chunks[k].escapes;
    if (k + 1 == total || chunks[k + 1].payload != r) {
      uint64_t n = 2 * (block_offsets[r + 1] - block_offsets[r]) * block_words;
      uint8_t* o = out + out_offsets[r];
      write_header(o, n, run);
      memset(o + 5 + n + (n + 1) / 2, 0, 5 * sz_top16_escape_capacity(n));
    }
  }
  /* pass 2: place the escapes of chunks that have any */
#pragma omp parallel for schedule(dynamic, 4)
  for (int64_t k = 0; k < (int64_t)total; ++k) {
    sz_chunk* ch = &chunks[k];
    if (!ch->escapes) continue;
    uint64_t r = ch->payload;
    const int64_t* pid = ids + block_offsets[r];
    uint64_t nblk = block_offsets[r + 1] - block_offsets[r];
    uint64_t n = 2 * nblk * block_words, half = n / 2;
    uint64_t cap = sz_top16_escape_capacity(n);
    uint8_t* entries = out + out_offsets[r] + 5 + n + (n + 1) / 2;
    uint64_t slot = ch->base;
    for (uint64_t i = ch->lo; i < ch->hi && slot < cap; ++i) {
      uint16_t w = load_paged(kv, plane_stride, block_stride, block_words, pid, nblk, i);
      unsigned e = (w >> 7) & 0xFF;
      if (tables[(i >= half ? 256u : 0u) + e] == 255) put_entry(entries, slot++, (uint32_t)i, e);
    }
  }
  free(chunks);
  return 0;
}

/* Multi-threaded decode + scatter of a batch (CPU baseline for the decode leg). */
SZ_EXPORT int sz_top16_decode_paged_batch(const uint8_t* src, const uint64_t* src_offsets,
                                          uint64_t payloads, uint16_t* kv,
                                          uint64_t plane_stride, uint64_t block_stride,
                                          uint64_t block_words, const int64_t* ids,
                                          const uint64_t* block_offsets, const uint8_t* tables,
                                          uint64_t chunk, int threads) {
  if (chunk == 0) return -1;
  uint64_t total = 0;
  for (uint64_t r = 0; r < payloads; ++r) {
    uint64_t n = 2 * (block_offsets[r + 1] - block_offsets[r]) * block_words;
    total += (n + chunk - 1) / chunk;
  }
  uint64_t* cr = (uint64_t*)calloc(total ? 2 * total : 2, sizeof(uint64_t));
  if (!cr) return -1;
  uint64_t c = 0;
  for (uint64_t r = 0; r < payloads; ++r) {
    uint64_t n = 2 * (block_offsets[r + 1] - block_offsets[r]) * block_words;
    for (uint64_t lo = 0; lo < n; lo += chunk) {
      cr[2 * c] = r;
      cr[2 * c + 1] = lo;
      ++c;
    }
  }
#ifdef _OPENMP
  if (threads > 0) omp_set_num_threads(threads);
#else
  (void)threads;
#endif
#pragma omp parallel for schedule(dynamic, 4)
  for (int64_t k = 0; k < (int64_t)total; ++k) {
    uint64_t r = cr[2 * k], lo = cr[2 * k + 1];
    const uint8_t* p = src + src_offsets[r];
    if (p[0] != 5) continue;
    const int64_t* pid = ids + block_offsets[r];
    uint64_t nblk = block_offsets[r + 1] - block_offsets[r];
    uint64_t n = 2 * nblk * block_words, half = n / 2;
    uint64_t hi = lo + chunk < n ? lo + chunk : n;
    const uint8_t* body = p + 5;
    const uint8_t* codes = body + n;
    const uint8_t* cb = tables + 512;
    for (uint64_t i = lo; i < hi; ++i) {
      unsigned code = (codes[i / 2] >> ((i % 2) * 4)) & 0x0F;
      unsigned e = cb[(i >= half ? 16u : 0u) + code];
      uint8_t v = body[i];
      kv[dst_index(i, nblk, block_words, plane_stride, block_stride, 0, pid)] =
          (uint16_t)((v & 0x7F) | ((uint16_t)(v & 0x80) << 8) | (uint16_t)(e << 7));
    }
  }
  /* escapes after every word of the payload is written */
#pragma omp parallel for schedule(dynamic, 1)
  for (int64_t r = 0; r < (int64_t)payloads; ++r) {
    const uint8_t* p = src + src_offsets[r];
    if (p[0] != 5) continue;
    const int64_t* pid = ids + block_offsets[r];
    uint64_t nblk = block_offsets[r + 1] - block_offsets[r];
    uint64_t n = 2 * nblk * block_words;
    uint64_t cap = sz_top16_escape_capacity(n);
    uint64_t count = (uint64_t)p[1] | ((uint64_t)p[2] << 8) | ((uint64_t)p[3] << 16) |
                     ((uint64_t)p[4] << 24);
    const uint8_t* entries = p + 5 + n + (n + 1) / 2;
    for (uint64_t s = 0; s < count && s < cap; ++s) {
      const uint8_t* e = entries + s * 5;
      uint64_t pos = (uint64_t)e[0] | ((uint64_t)e[1] << 8) | ((uint64_t)e[2] << 16) |
                     ((uint64_t)e[3] << 24);
      if (pos >= n) continue;
      uint64_t d = dst_index(pos, nblk, block_words, plane_stride, block_stride, 0, pid);
      kv[d] = (uint16_t)((kv[d] & 0x807F) | ((unsigned)e[4] << 7));
    }
  }
  free(cr);
  return 0;
}
