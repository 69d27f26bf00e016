// Decode + scatter of the reference connector's torch-op codec payloads (payload
// modes 0, 1, 2), gfx950. The reference decodes them with torch ops on restore
// (src/unchain_kv/vllm_connector.py:5168-5252); a sender without the native codec
// produces them (:3204-3343). Layouts, n words per payload, codes packed LSB-first
// (code i at bits [i*w, i*w + w), :3345-3404):
//   mode 0  [0][w][256-byte palette][n low bytes][codes, w = 1..7]
//           word = palette[code] << 8 | low
//   mode 1  [1][w0 w1 w2 w3][4 x 16-byte palettes][plane 0 codes]..[plane 3 codes],
//           w_p in {1, 2, 4}; word = OR_p palette_p[code_p] << 4p (16 bits kept)
//   mode 2  [2][w][mag_min][n low bytes][n sign bits][magnitude codes, w = 1..6]
//           word = ((sign << 7 | (code + mag_min)) << 8 | low) (16 bits kept)
// A payload whose header does not give exactly its encoded size (the reference's
// restore checks) is left unapplied.
//
// Encode (the sender's choice for a request below 1 MiB without the native codec,
// :3043-3046, 3204-3343): a presence pass records which high-byte and low-nibble
// values occur in each 4096-word tile, a plan pass ORs a payload's tiles and picks
// the format in the reference's order -- sign/magnitude if the magnitudes span
// fewer than 7 bits and the payload is smaller than the raw words, else the
// high-byte palette if it has at most 128 entries and is smaller, else the nibble
// planes if smaller, else none -- with its widths and encoded size, and the encode
// pass writes the chosen format (palettes ascending, unused palette bytes zero,
// codes LSB-first with zero padding bits). The host reads the plans' sizes between
// the plan and the encode to lay the payloads out.
//
// Kernels: `*_tile` for layers whose block words are a multiple of 1024 (a
// 1024-word wave chunk lies in one block; one workgroup per 4096-word tile of the
// launch, XCD-remapped, lanes own two 8-word runs so that every section access of
// a wave instruction is one contiguous span), `*_generic` for any other geometry
// (workgroup (x, y): words [4096 x, 4096 x + 4096) of payload y, 16 consecutive
// words per thread, byte-granular section accesses). A launch covers at most 64
// payloads; the plan kernel runs once for up to 256 after all presence launches.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>

#include "splitzip_common.h"

namespace unchainkv {
namespace {

constexpr unsigned int kTorchopTile = kThreads * kWordsPerLane;  // 4096 words

struct TorchopSizes {
  unsigned long long encoded[kMaxPayloads];
};

// Header of one payload as the decode reads it.
struct TorchopHeader {
  unsigned int mode;
  unsigned int width[4];
  unsigned int mag_min;
  unsigned long long low_at, code_at[4], sign_at;  // byte offsets of the sections
  bool ok;
};

// From the payload's first eight bytes (little-endian in `first8`).
__device__ TorchopHeader parse_header(unsigned long long first8, unsigned long long size,
                                      unsigned long long n) {
  unsigned int h[5];
#pragma unroll
  for (int k = 0; k < 5; ++k) h[k] = (unsigned int)(first8 >> (8 * k)) & 0xFFu;
  TorchopHeader t{};
  t.mode = h[0];
  t.ok = false;
  if (t.mode == 0) {
    t.width[0] = h[1];
    t.low_at = 258;
    t.code_at[0] = 258 + n;
    t.ok = size >= 258 && t.width[0] >= 1 && t.width[0] < 8 &&
           size == 258 + n + (n * t.width[0] + 7) / 8;
  } else if (t.mode == 1) {
    unsigned long long at = 69;
    bool widths_ok = true;
    for (int p = 0; p < 4; ++p) {
      t.width[p] = h[1 + p];
      widths_ok = widths_ok && (t.width[p] == 1 || t.width[p] == 2 || t.width[p] == 4);
      t.code_at[p] = at;
      at += (n * t.width[p] + 7) / 8;
    }
    t.ok = size >= 69 && widths_ok && size == at;
  } else if (t.mode == 2) {
    t.width[0] = h[1];
    t.mag_min = h[2];
    t.low_at = 3;
    t.sign_at = 3 + n;
    t.code_at[0] = 3 + n + (n + 7) / 8;
    t.ok = size >= 3 && t.width[0] >= 1 && t.width[0] < 7 &&
           size == 3 + n + (n + 7) / 8 + (n * t.width[0] + 7) / 8;
  }
  return t;
}

// Code i of width w (w <= 8, so within two bytes) from the section at `sec`; the
// byte past the section's end reads as zero (the reference unpacks from a copy
// padded with one zero byte).
__device__ __forceinline__ unsigned int code_at(const unsigned char* sec, unsigned long long end,
                                                unsigned long long i, unsigned int w) {
  const unsigned long long bit = i * w;
  const unsigned long long byte = bit >> 3;
  const unsigned int lo = sec[byte];
  const unsigned int hi = byte + 1 < end ? sec[byte + 1] : 0u;
  return ((lo | (hi << 8)) >> (bit & 7)) & ((1u << w) - 1u);
}

__global__ __launch_bounds__(kThreads) void torchop_decode_generic(LaunchArgs a,
                                                                   TorchopSizes sizes) {
  __shared__ unsigned char s_hdr[260];
  const unsigned int tid = threadIdx.x;
  const unsigned int r = blockIdx.y;
  const PayloadDesc d = a.p[r];
  const unsigned long long n = 2ull * d.block_count * a.block_words;
  const unsigned long long size = sizes.encoded[r];
  const unsigned char* payload = a.buf + d.buf_offset;
  // palettes and widths, from the first bytes of the payload
  for (unsigned int k = tid; k < 258; k += kThreads) s_hdr[k] = k < size ? payload[k] : 0;
  __syncthreads();
  unsigned long long first8 = 0;
#pragma unroll
  for (int k = 0; k < 8; ++k) first8 |= (unsigned long long)s_hdr[k] << (8 * k);
  const TorchopHeader h = parse_header(first8, size, n);
  if (!h.ok) return;
  const unsigned long long i0 =
      (unsigned long long)blockIdx.x * kTorchopTile + (unsigned long long)tid * kWordsPerLane;
  if (i0 >= n) return;
  const unsigned int count = (unsigned int)std::min<unsigned long long>(kWordsPerLane, n - i0);

  uint32_t out[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  for (unsigned int k = 0; k < count; ++k) {
    const unsigned long long i = i0 + k;
    uint32_t word;
    if (h.mode == 0) {
      const unsigned int code = code_at(payload + h.code_at[0], size - h.code_at[0], i, h.width[0]);
      word = ((uint32_t)s_hdr[2 + code] << 8) | payload[h.low_at + i];
    } else if (h.mode == 1) {
      word = 0;
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        const unsigned long long end = (p < 3 ? h.code_at[p + 1] : size) - h.code_at[p];
        const unsigned int code = code_at(payload + h.code_at[p], end, i, h.width[p]);
        word |= (uint32_t)s_hdr[5 + 16 * p + code] << (4 * p);
      }
    } else {
      const unsigned int sign = (payload[h.sign_at + (i >> 3)] >> (i & 7)) & 1u;
      const unsigned int mag = code_at(payload + h.code_at[0], size - h.code_at[0], i, h.width[0]);
      word = (((sign << 7) | (mag + h.mag_min)) << 8) | payload[h.low_at + i];
    }
    out[k >> 1] |= (word & 0xFFFFu) << (16 * (k & 1));
  }

  // scatter: 16 words in one block go out as two 16-byte stores
  const unsigned long long half = n >> 1;
  const unsigned int plane = i0 >= half ? 1u : 0u;
  const unsigned long long in_plane = i0 - plane * half;
  const unsigned long long j = in_plane / a.block_words;
  const unsigned long long within = in_plane - j * a.block_words;
  const bool whole = count == kWordsPerLane && within + kWordsPerLane <= a.block_words &&
                     (i0 + kWordsPerLane <= (plane + 1) * half);
  if (whole) {
    const unsigned long long blk = a.ids ? (unsigned long long)a.ids[d.ids_offset + j] : j;
    uint16_t* dst = a.kv + plane * a.plane_stride + blk * a.block_stride + within;
    if (((uintptr_t)dst & 15) == 0) {
      reinterpret_cast<uint4*>(dst)[0] = make_uint4(out[0], out[1], out[2], out[3]);
      reinterpret_cast<uint4*>(dst)[1] = make_uint4(out[4], out[5], out[6], out[7]);
      return;
    }
  }
  for (unsigned int k = 0; k < count; ++k)
    a.kv[word_offset(a, d, i0 + k)] = (uint16_t)(out[k >> 1] >> (16 * (k & 1)));
}


// ---------------------------------------------------------------------------
// encode

// Presence of word values in one 4096-word tile (workspace record, 16 u32):
// [0..8) 256-bit mask of the high bytes, [8] bits 0-15: values of bits 0-3 of the
// words, bits 16-31: values of bits 4-7.
constexpr unsigned int kTorchopRecordWords = 16;

// Plan of one payload's torch-op encode (64 bytes, device memory; the host reads
// encoded_bytes).
struct TorchopPlan {
  unsigned int high[8];              // presence of each high byte value
  unsigned int nibbles;              // presence of bits 0-3 values | bits 4-7 values << 16
  unsigned char mode;                // 2, 0 or 1; kTorchopNone when none is smaller
  unsigned char width[4];            // modes 2 and 0: width[0]; mode 1: per nibble plane
  unsigned char mag_min;             // mode 2: smallest magnitude (high byte & 0x7F)
  unsigned char pad0[6];
  unsigned long long encoded_bytes;  // 0 when declined
  unsigned long long words;          // n
};
static_assert(sizeof(TorchopPlan) == 64, "torch-op plan record");
constexpr unsigned char kTorchopNone = 255;

// Up to 16 consecutive words i0 .. of payload d (count of them valid) into w (two
// bf16 per dword): two 16-byte loads when they lie in one block and are 16-byte
// aligned, else word by word.
__device__ __forceinline__ unsigned int load_words16(const LaunchArgs& a, const PayloadDesc& d,
                                                     unsigned long long n, unsigned long long i0,
                                                     uint32_t (&w)[8]) {
  const unsigned int count = (unsigned int)std::min<unsigned long long>(kWordsPerLane, n - i0);
  const unsigned long long half = n >> 1;
  const unsigned int plane = i0 >= half ? 1u : 0u;
  const unsigned long long in_plane = i0 - plane * half;
  const unsigned long long j = in_plane / a.block_words;
  const unsigned long long within = in_plane - j * a.block_words;
  if (count == kWordsPerLane && within + kWordsPerLane <= a.block_words &&
      i0 + kWordsPerLane <= (plane + 1ull) * half) {
    const unsigned long long blk = a.ids ? (unsigned long long)a.ids[d.ids_offset + j] : j;
    const uint16_t* src = a.kv + plane * a.plane_stride + blk * a.block_stride + within;
    if (((uintptr_t)src & 15) == 0) {
      const u32x4 v0 = load_stream16(src), v1 = load_stream16(src + 8);
      w[0] = v0.x; w[1] = v0.y; w[2] = v0.z; w[3] = v0.w;
      w[4] = v1.x; w[5] = v1.y; w[6] = v1.z; w[7] = v1.w;
      return count;
    }
  }
#pragma unroll
  for (int k = 0; k < 8; ++k) w[k] = 0;
  for (unsigned int k = 0; k < count; ++k)
    w[k >> 1] |= (uint32_t)a.kv[word_offset(a, d, i0 + k)] << (16 * (k & 1));
  return count;
}

__device__ __forceinline__ unsigned int word_at(const uint32_t (&w)[8], unsigned int k) {
  return (w[k >> 1] >> (16 * (k & 1))) & 0xFFFFu;
}

// Any geometry. Workgroup (x, y): tile x of payload y; each thread marks the values
// of its 16 words in LDS byte maps, one ballot per wave turns them into mask bits.
__global__ __launch_bounds__(kThreads) void torchop_presence_generic(LaunchArgs a,
                                                                     unsigned int record_base) {
  __shared__ unsigned char s_high[256];
  __shared__ unsigned char s_nib[64];
  const unsigned int tid = threadIdx.x;
  const PayloadDesc d = a.p[blockIdx.y];
  const unsigned long long n = payload_words(a, d);
  const unsigned long long tile0 = (unsigned long long)blockIdx.x * kTorchopTile;
  if (tile0 >= n) return;  // the whole workgroup
  s_high[tid] = 0;
  if (tid < 64) s_nib[tid] = 0;
  __syncthreads();
  const unsigned long long i0 = tile0 + (unsigned long long)tid * kWordsPerLane;
  if (i0 < n) {
    uint32_t w[8];
    const unsigned int count = load_words16(a, d, n, i0, w);
    for (unsigned int k = 0; k < count; ++k) {
      const unsigned int v = word_at(w, k);
      s_high[v >> 8] = 1;
      s_nib[v & 15] = 1;
      s_nib[16 + ((v >> 4) & 15)] = 1;
    }
  }
  __syncthreads();
  const unsigned int lane = tid & (kWave - 1), wave = tid >> 6;
  unsigned int* rec =
      a.workspace + kTorchopRecordWords * (record_base + d.tile_begin + blockIdx.x);
  const unsigned long long high = __ballot(s_high[tid] != 0);
  if (lane == 0) {
    rec[2 * wave] = (unsigned int)high;
    rec[2 * wave + 1] = (unsigned int)(high >> 32);
  }
  if (wave == 0) {
    const unsigned long long nib = __ballot(lane < 32 && s_nib[lane] != 0);
    if (lane == 0) rec[8] = (unsigned int)nib;
  }
}

__device__ __forceinline__ unsigned int bit_length(unsigned int x) {
  return x ? 32u - (unsigned int)__clz((int)x) : 0u;
}

// Width of a nibble plane with k distinct values (vllm_connector.py:3287).
__device__ __forceinline__ unsigned int nibble_width(unsigned int mask) {
  const unsigned int k = (unsigned int)__popc(mask);
  return k <= 2 ? 1u : k <= 4 ? 2u : 4u;
}

// The four nibble planes' value masks (bits 0-3, 4-7, 8-11, 12-15 of the words)
// from a plan's presence masks.
__device__ __forceinline__ void nibble_masks(const unsigned int (&high)[8], unsigned int nibbles,
                                             unsigned int (&m)[4]) {
  m[0] = nibbles & 0xFFFFu;
  m[1] = nibbles >> 16;
  unsigned int lo = 0, hi = 0;
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    lo |= (high[k] & 0xFFFFu) | (high[k] >> 16);        // high byte & 15 (bits 8-11)
    hi |= ((high[k] & 0xFFFFu) != 0 ? 1u : 0u) << (2 * k);  // high byte >> 4 (bits 12-15)
    hi |= ((high[k] >> 16) != 0 ? 1u : 0u) << (2 * k + 1);
  }
  m[2] = lo;
  m[3] = hi;
}

// One workgroup per payload: OR of its tile records, then the reference's format
// choice (vllm_connector.py:3210-3213, 3219-3222, 3250-3253, 3279-3290, 3310-3311).
// Payloads of one plan launch: each payload's first tile record and its blocks per
// plane (the presence launches cover at most kMaxPayloads payloads each; one plan
// launch follows all of them).
constexpr unsigned int kPlanPayloads = 256;
struct PlanArgs {
  const unsigned int* workspace;
  unsigned long long block_words;
  unsigned int record_begin[kPlanPayloads];
  unsigned int blocks[kPlanPayloads];
};

__global__ __launch_bounds__(kThreads) void torchop_plan(PlanArgs a, TorchopPlan* plans) {
  __shared__ unsigned int s_or[9];
  const unsigned int tid = threadIdx.x;
  const unsigned long long n = 2ull * a.blocks[blockIdx.x] * a.block_words;
  const unsigned int record0 = a.record_begin[blockIdx.x];
  const unsigned int tiles = (unsigned int)((n + kTorchopTile - 1) / kTorchopTile);
  if (tid < 9) s_or[tid] = 0;
  __syncthreads();
  unsigned int part[9] = {0, 0, 0, 0, 0, 0, 0, 0, 0};
  for (unsigned int t = tid; t < tiles; t += kThreads) {
    const unsigned int* rec = a.workspace + kTorchopRecordWords * (record0 + t);
#pragma unroll
    for (int k = 0; k < 9; ++k) part[k] |= rec[k];
  }
#pragma unroll
  for (int k = 0; k < 9; ++k)
#pragma unroll
    for (int off = kWave / 2; off > 0; off >>= 1) part[k] |= __shfl_xor(part[k], off, kWave);
  if ((tid & (kWave - 1)) == 0) {
#pragma unroll
    for (int k = 0; k < 9; ++k)
      if (part[k]) atomicOr(&s_or[k], part[k]);
  }
  __syncthreads();
  if (tid != 0) return;
  TorchopPlan p{};
  for (int k = 0; k < 8; ++k) p.high[k] = s_or[k];
  p.nibbles = s_or[8];
  p.words = n;
  p.mode = kTorchopNone;
  const unsigned long long raw = 2 * n;
  // sign / magnitude: magnitudes present = high bytes with the sign bit dropped
  unsigned int mags[4];
  for (int k = 0; k < 4; ++k) mags[k] = p.high[k] | p.high[k + 4];
  unsigned int mag_min = 0, mag_max = 0;
  bool seen = false;
  for (int k = 0; k < 4; ++k) {
    if (!mags[k]) continue;
    if (!seen) mag_min = 32 * k + (unsigned int)__ffs((int)mags[k]) - 1;
    mag_max = 32 * k + 31 - (unsigned int)__clz((int)mags[k]);
    seen = true;
  }
  const unsigned int mag_width = max(1u, bit_length(mag_max - mag_min));
  if (mag_width < 7) {
    const unsigned long long size = 3 + n + (n + 7) / 8 + (n * mag_width + 7) / 8;
    if (size < raw) {
      p.mode = 2;
      p.width[0] = (unsigned char)mag_width;
      p.mag_min = (unsigned char)mag_min;
      p.encoded_bytes = size;
    }
  }
  if (p.mode == kTorchopNone) {
    unsigned int distinct = 0;
    for (int k = 0; k < 8; ++k) distinct += (unsigned int)__popc(p.high[k]);
    const unsigned int width = max(1u, bit_length(distinct - 1));
    if (width < 8) {
      const unsigned long long size = 258 + n + (n * width + 7) / 8;
      if (size < raw) {
        p.mode = 0;
        p.width[0] = (unsigned char)width;
        p.encoded_bytes = size;
      }
    }
  }
  if (p.mode == kTorchopNone) {
    unsigned int m[4];
    nibble_masks(p.high, p.nibbles, m);
    unsigned long long size = 69;
    for (int q = 0; q < 4; ++q) {
      const unsigned int w = nibble_width(m[q]);
      p.width[q] = (unsigned char)w;
      size += (n * w + 7) / 8;
    }
    if (size < raw) {
      p.mode = 1;
      p.encoded_bytes = size;
    } else {
      for (int q = 0; q < 4; ++q) p.width[q] = 0;
    }
  }
  plans[blockIdx.x] = p;
}

// Code section write of one thread: 16 codes (count of them valid, the others 0)
// of `width` bits each, LSB-first, at bit 16 * width * (i0 / 16) of the section:
// whole bytes, ceil(count * width / 8) of them.
__device__ __forceinline__ void put_codes(unsigned char* sec, unsigned long long i0,
                                          const unsigned int (&code)[16], unsigned int count,
                                          unsigned int width) {
  unsigned long long lo = 0, hi = 0;
#pragma unroll
  for (unsigned int k = 0; k < 16; ++k) {
    const unsigned long long c = k < count ? code[k] : 0u;
    const unsigned int b = k * width;
    if (b < 64) {
      lo |= c << b;
      if (b + width > 64) hi |= c >> (64 - b);
    } else {
      hi |= c << (b - 64);
    }
  }
  unsigned char* dst = sec + (i0 * width) / 8;
  const unsigned int bytes = (count * width + 7) / 8;
  for (unsigned int j = 0; j < bytes; ++j)
    dst[j] = (unsigned char)(j < 8 ? lo >> (8 * j) : hi >> (8 * (j - 8)));
}

// The plan's fields, the rank tables in LDS (mode 0: high byte -> palette index;
// mode 1: entry 16q + v -> index of nibble value v in plane q's palette) and, with
// `header`, the payload's header and palettes (vllm_connector.py:3226-3228,
// 3259-3261, 3300-3307). `ok`: the plan encodes the payload (a format was chosen,
// for n words, at the size the host laid out); nothing is written otherwise. The
// record is read as 16 aligned dwords (scalar loads), and no register array is
// indexed per thread (such an array would be placed in memory). The caller
// synchronises before reading s_rank.
struct EncodeFields {
  unsigned int mode;
  unsigned int widths;  // one byte per nibble plane (mode 1); mode 0 and 2: byte 0
  unsigned int mag_min;
  bool ok;
};

__device__ __forceinline__ unsigned int plane_width(const EncodeFields& f, int q) {
  return (f.widths >> (8 * q)) & 0xFFu;
}

__device__ __forceinline__ unsigned int pick4(unsigned int i, unsigned int a0, unsigned int a1,
                                              unsigned int a2, unsigned int a3) {
  return i == 0 ? a0 : i == 1 ? a1 : i == 2 ? a2 : a3;
}

__device__ __forceinline__ EncodeFields encode_prologue(const TorchopPlan* plan,
                                                        unsigned long long n,
                                                        unsigned long long size,
                                                        unsigned char* out,
                                                        unsigned char* s_rank, bool header) {
  const unsigned int tid = threadIdx.x;
  const unsigned int* pw = reinterpret_cast<const unsigned int*>(plan);
  unsigned int high[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) high[k] = pw[k];
  const unsigned int nibbles = pw[8], w9 = pw[9], w10 = pw[10];
  const unsigned long long encoded = pw[12] | ((unsigned long long)pw[13] << 32);
  const unsigned long long words = pw[14] | ((unsigned long long)pw[15] << 32);
  EncodeFields f;
  f.mode = w9 & 0xFFu;                  // byte 36
  f.widths = (w9 >> 8) | (w10 << 24);   // bytes 37-40
  f.mag_min = (w10 >> 8) & 0xFFu;       // byte 41
  f.ok = f.mode != kTorchopNone && encoded == size && words == n;
  unsigned int nib[4];
  nibble_masks(high, nibbles, nib);
  unsigned int rank = 0, present = 0;
  if (f.mode == 0) {
    const unsigned int h = tid, hw = h >> 5;
    unsigned int word = 0, below = 0;
#pragma unroll
    for (unsigned int k = 0; k < 8; ++k) {
      word = k == hw ? high[k] : word;
      below += k < hw ? (unsigned int)__popc(high[k]) : 0u;
    }
    rank = below + (unsigned int)__popc(word & ((1u << (h & 31)) - 1u));
    present = (word >> (h & 31)) & 1u;
  } else if (f.mode == 1 && tid < 64) {
    const unsigned int q = tid >> 4, v = tid & 15;
    const unsigned int m = pick4(q, nib[0], nib[1], nib[2], nib[3]);
    rank = (unsigned int)__popc(m & ((1u << v) - 1u));
    present = (m >> v) & 1u;
  }
  s_rank[tid] = (unsigned char)rank;
  if (header && f.ok) {
    if (f.mode == 2) {
      if (tid == 0) out[0] = 2;
      if (tid == 1) out[1] = (unsigned char)plane_width(f, 0);
      if (tid == 2) out[2] = (unsigned char)f.mag_min;
    } else if (f.mode == 0) {
      unsigned int distinct = 0;
#pragma unroll
      for (int k = 0; k < 8; ++k) distinct += (unsigned int)__popc(high[k]);
      if (tid == 0) {
        out[0] = 0;
        out[1] = (unsigned char)plane_width(f, 0);
      }
      if (present) out[2 + rank] = (unsigned char)tid;
      if (tid >= distinct) out[2 + tid] = 0;
    } else if (tid < 64) {
      const unsigned int q = tid >> 4, v = tid & 15;
      const unsigned int m = pick4(q, nib[0], nib[1], nib[2], nib[3]);
      if (present) out[5 + 16 * q + rank] = (unsigned char)v;
      if (v >= (unsigned int)__popc(m)) out[5 + 16 * q + v] = 0;
      if (tid == 0) out[0] = 1;
      if (tid < 4) out[1 + tid] = (unsigned char)(f.widths >> (8 * tid));
    }
  }
  return f;
}

// Any geometry. Workgroup (x, y): words [4096 x, 4096 x + 4096) of payload y, 16
// per thread; workgroup x == 0 also writes the header. Payloads whose plan
// declined, or whose plan size is not the size the host laid out, are skipped.
__global__ __launch_bounds__(kThreads) void torchop_encode_generic(LaunchArgs a,
                                                                   const TorchopPlan* plans,
                                                                   TorchopSizes sizes) {
  __shared__ unsigned char s_rank[256];
  const unsigned int tid = threadIdx.x;
  const unsigned int r = blockIdx.y;
  const PayloadDesc d = a.p[r];
  const unsigned long long n = payload_words(a, d);
  const unsigned long long tile0 = (unsigned long long)blockIdx.x * kTorchopTile;
  if (tile0 >= n) return;  // the whole workgroup
  unsigned char* out = a.buf + d.buf_offset;
  const EncodeFields f = encode_prologue(plans + r, n, sizes.encoded[r], out, s_rank,
                                         blockIdx.x == 0);
  if (!f.ok) return;
  const unsigned int mode = f.mode, mag_min = f.mag_min;
  const unsigned int width[4] = {plane_width(f, 0), plane_width(f, 1), plane_width(f, 2),
                                 plane_width(f, 3)};
  __syncthreads();
  const unsigned long long i0 = tile0 + (unsigned long long)tid * kWordsPerLane;
  if (i0 >= n) return;
  uint32_t w[8];
  const unsigned int count = load_words16(a, d, n, i0, w);
  unsigned int code[16];
  if (mode == 2 || mode == 0) {
    // low bytes, then (mode 2) sign bits and magnitudes, (mode 0) palette indices
    const unsigned long long low_at = mode == 2 ? 3 : 258;
    for (unsigned int k = 0; k < count; ++k) out[low_at + i0 + k] = (unsigned char)word_at(w, k);
    if (mode == 2) {
      unsigned int signs = 0;
#pragma unroll
      for (unsigned int k = 0; k < 16; ++k) {
        const unsigned int v = word_at(w, k);
        signs |= (k < count ? (v >> 15) : 0u) << k;
        code[k] = ((v >> 8) & 0x7Fu) - mag_min;
      }
      unsigned char* sign_sec = out + 3 + n;
      sign_sec[i0 / 8] = (unsigned char)signs;
      if (count > 8) sign_sec[i0 / 8 + 1] = (unsigned char)(signs >> 8);
      put_codes(out + 3 + n + (n + 7) / 8, i0, code, count, width[0]);
    } else {
#pragma unroll
      for (unsigned int k = 0; k < 16; ++k) code[k] = s_rank[word_at(w, k) >> 8];
      put_codes(out + 258 + n, i0, code, count, width[0]);
    }
    return;
  }
  unsigned long long at = 69;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
#pragma unroll
    for (unsigned int k = 0; k < 16; ++k) code[k] = s_rank[16 * q + ((word_at(w, k) >> (4 * q)) & 15)];
    put_codes(out + at, i0, code, count, width[q]);
    at += (n * width[q] + 7) / 8;
  }
}

// ---------------------------------------------------------------------------
// tile kernels: block words a multiple of 1024 (a 1024-word wave chunk lies in one
// block), the layer 16-byte aligned. Workgroup (x, y): words [4096 x, 4096 x +
// 4096) of payload y; wave w owns the chunk at 4096 x + 1024 w (its block found
// with scalar loads), lane l the two 8-word runs at 8 l and 512 + 8 l of it. Every
// section access of a wave instruction is then one contiguous span: the run's 16
// source bytes, its 8 low bytes, its sign byte and its w code bytes (w-bit codes of
// 8 words fill whole bytes) at the section offset of word i, w * i / 8. Payload
// sections start at any byte (global memory takes unaligned accesses).

typedef unsigned short u16_unaligned __attribute__((aligned(1)));
typedef unsigned int u32_unaligned __attribute__((aligned(1)));

// Little-endian bytes [0, w) at p, 1 <= w <= 7 (w uniform): one access per set bit.
__device__ __forceinline__ unsigned long long load_bytes(const unsigned char* p, unsigned int w) {
  unsigned long long v = 0;
  unsigned int at = 0;
  if (w & 4) {
    v = *reinterpret_cast<const u32_unaligned*>(p);
    at = 4;
  }
  if (w & 2) {
    v |= (unsigned long long)*reinterpret_cast<const u16_unaligned*>(p + at) << (8 * at);
    at += 2;
  }
  if (w & 1) v |= (unsigned long long)p[at] << (8 * at);
  return v;
}

__device__ __forceinline__ void store_bytes(unsigned char* p, unsigned long long v,
                                            unsigned int w) {
  unsigned int at = 0;
  if (w & 4) {
    *reinterpret_cast<u32_unaligned*>(p) = (unsigned int)v;
    at = 4;
  }
  if (w & 2) {
    *reinterpret_cast<u16_unaligned*>(p + at) = (unsigned short)(v >> (8 * at));
    at += 2;
  }
  if (w & 1) p[at] = (unsigned char)(v >> (8 * at));
}

// Element offset in the layer of the wave chunk starting at payload word c.
__device__ __forceinline__ unsigned long long chunk_source(const LaunchArgs& a,
                                                           const PayloadDesc& d,
                                                           const EncodeGeom& geo,
                                                           unsigned long long n,
                                                           unsigned long long c) {
  const unsigned long long half = n >> 1;
  const unsigned int plane = c >= half ? 1u : 0u;
  const unsigned int in_plane = uniform((unsigned int)(c - plane * half));
  const unsigned int j = uniform(div_u32(in_plane, geo.bw_magic, geo.bw));
  const unsigned int within = in_plane - j * geo.bw;
  const unsigned long long blk = uniform64((unsigned long long)a.ids[d.ids_offset + j]);
  return uniform64(plane * a.plane_stride + blk * a.block_stride + within);
}

// Codes k = 0..7 of a run, `width` bits each, LSB-first.
__device__ __forceinline__ unsigned int run_code(unsigned long long codes, unsigned int width,
                                                 int k) {
  return (unsigned int)(codes >> (width * k)) & ((1u << width) - 1u);
}

__global__ __launch_bounds__(kThreads) void torchop_presence_tile(LaunchArgs a, EncodeGeom geo,
                                                                  unsigned int record_base) {
  __shared__ unsigned char s_high[256];
  __shared__ unsigned int s_nib;
  const unsigned int tid = threadIdx.x;
  const unsigned int lane = tid & (kWave - 1), wave = uniform(tid >> 6);
  const unsigned int tile = group_index();
  const PayloadDesc d = a.p[find_payload(a, tile)];
  const unsigned long long n = payload_words(a, d);
  const unsigned long long c = (unsigned long long)(tile - d.tile_begin) * kTorchopTile + wave * 1024ull;
  const bool active = c < n;
  u32x4 v0 = {0, 0, 0, 0}, v1 = {0, 0, 0, 0};
  if (active) {
    const uint16_t* src = a.kv + chunk_source(a, d, geo, n, c);
    v0 = load_stream16(src + 8 * lane);
    v1 = load_stream16(src + 512 + 8 * lane);
  }
  if (tid < 64) reinterpret_cast<unsigned int*>(s_high)[tid] = 0;
  if (tid == 0) s_nib = 0;
  __syncthreads();
  if (active) {
    const uint32_t x[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
    unsigned int nib = 0;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      s_high[(x[k] >> 8) & 0xFF] = 1;
      s_high[x[k] >> 24] = 1;
      nib |= (1u << (x[k] & 15)) | (1u << (16 + ((x[k] >> 4) & 15)));
      nib |= (1u << ((x[k] >> 16) & 15)) | (1u << (16 + ((x[k] >> 20) & 15)));
    }
#pragma unroll
    for (int off = kWave / 2; off > 0; off >>= 1) nib |= __shfl_xor(nib, off, kWave);
    if (lane == 0) atomicOr(&s_nib, nib);
  }
  __syncthreads();
  unsigned int* rec = a.workspace + kTorchopRecordWords * (record_base + tile);
  const unsigned long long high = __ballot(s_high[tid] != 0);
  if (lane == 0) {
    rec[2 * wave] = (unsigned int)high;
    rec[2 * wave + 1] = (unsigned int)(high >> 32);
  }
  if (tid == 0) rec[8] = s_nib;
}

__global__ __launch_bounds__(kThreads) void torchop_encode_tile(LaunchArgs a, EncodeGeom geo,
                                                                const TorchopPlan* plans,
                                                                TorchopSizes sizes) {
  __shared__ unsigned char s_rank[256];
  const unsigned int tid = threadIdx.x;
  const unsigned int lane = tid & (kWave - 1), wave = uniform(tid >> 6);
  const unsigned int tile = group_index();
  const unsigned int r = find_payload(a, tile);
  const PayloadDesc d = a.p[r];
  const unsigned long long n = payload_words(a, d);
  const unsigned int local = tile - d.tile_begin;
  const unsigned long long c = (unsigned long long)local * kTorchopTile + wave * 1024ull;
  const bool active = c < n;
  // the words first: the plan's round trip overlaps with theirs
  u32x4 v0 = {0, 0, 0, 0}, v1 = {0, 0, 0, 0};
  if (active) {
    const uint16_t* src = a.kv + chunk_source(a, d, geo, n, c);
    v0 = load_stream16(src + 8 * lane);
    v1 = load_stream16(src + 512 + 8 * lane);
  }
  unsigned char* out = a.buf + d.buf_offset;
  const EncodeFields f = encode_prologue(plans + r, n, sizes.encoded[r], out, s_rank, local == 0);
  if (!f.ok) return;  // the whole workgroup
  __syncthreads();
  if (!active) return;
  const uint32_t x[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
#pragma unroll
  for (int run = 0; run < 2; ++run) {
    const uint32_t* xr = x + 4 * run;
    const unsigned long long i = c + 512 * run + 8 * lane;  // the run's first word
    if (f.mode == 1) {
      unsigned long long at = 69;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const unsigned int w = plane_width(f, q);
        unsigned long long codes = 0;
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          const unsigned int word = (xr[k >> 1] >> (16 * (k & 1))) & 0xFFFFu;
          const unsigned int v = s_rank[16 * q + ((word >> (4 * q)) & 15)] & ((1u << w) - 1u);
          codes |= (unsigned long long)v << (w * k);
        }
        store_bytes(out + at + w * (i >> 3), codes, w);
        at += n * w / 8;
      }
      continue;
    }
    // low bytes: bytes 0 and 2 of each dword
    const u32x2 low = {__builtin_amdgcn_perm(xr[1], xr[0], 0x06040200u),
                       __builtin_amdgcn_perm(xr[3], xr[2], 0x06040200u)};
    const unsigned int w = plane_width(f, 0);
    unsigned long long codes = 0;
    unsigned int signs = 0;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const unsigned int word = (xr[k >> 1] >> (16 * (k & 1))) & 0xFFFFu;
      unsigned int v;
      if (f.mode == 2) {
        signs |= (word >> 15) << k;
        v = ((word >> 8) & 0x7Fu) - f.mag_min;
      } else {
        v = s_rank[word >> 8];
      }
      codes |= (unsigned long long)(v & ((1u << w) - 1u)) << (w * k);
    }
    if (f.mode == 2) {
      store_stream8(out + 3 + i, low);
      out[3 + n + (i >> 3)] = (unsigned char)signs;
      store_bytes(out + 3 + n + n / 8 + w * (i >> 3), codes, w);
    } else {
      store_stream8(out + 258 + i, low);
      store_bytes(out + 258 + n + w * (i >> 3), codes, w);
    }
  }
}

__global__ __launch_bounds__(kThreads) void torchop_decode_tile(LaunchArgs a, EncodeGeom geo,
                                                                TorchopSizes sizes) {
  __shared__ unsigned char s_pal[256];
  const unsigned int tid = threadIdx.x;
  const unsigned int lane = tid & (kWave - 1), wave = uniform(tid >> 6);
  const unsigned int tile = group_index();
  const unsigned int r = find_payload(a, tile);
  const PayloadDesc d = a.p[r];
  const unsigned long long n = 2ull * d.block_count * a.block_words;
  const unsigned long long size = sizes.encoded[r];
  const unsigned char* payload = a.buf + d.buf_offset;
  const unsigned long long c =
      (unsigned long long)(tile - d.tile_begin) * kTorchopTile + wave * 1024ull;
  // a payload of these kernels holds at least 2048 words; a shorter size fails its
  // header check below, and the header reads stay inside 16 bytes of the payload
  if (size < 16) return;
  // header bytes 0-7 from the aligned dwords that cover them (scalar loads, in
  // parallel with the destination block's)
  const uintptr_t addr = reinterpret_cast<uintptr_t>(payload);
  const unsigned int* hw = reinterpret_cast<const unsigned int*>(addr & ~(uintptr_t)3);
  const unsigned int sh = (unsigned int)(addr & 3) * 8;
  const unsigned long long lo64 = hw[0] | ((unsigned long long)hw[1] << 32);
  const unsigned long long first8 =
      sh ? (lo64 >> sh) | ((unsigned long long)hw[2] << (64 - sh)) : lo64;
  const bool active = c < n;
  uint16_t* dst = active ? a.kv + chunk_source(a, d, geo, n, c) : nullptr;
  const TorchopHeader h = parse_header(first8, size, n);
  if (!h.ok) return;  // the whole workgroup
  // the palette bytes first, then every section load of both runs, so that the
  // palette's LDS write waits for its own load only
  unsigned int pal = 0;
  if (h.mode == 0) pal = payload[2 + tid];
  else if (h.mode == 1 && tid < 64) pal = payload[5 + tid];
  u32x2 low[2] = {{0, 0}, {0, 0}};
  unsigned long long codes[2][4] = {{0, 0, 0, 0}, {0, 0, 0, 0}};
  unsigned int signs[2] = {0, 0};
  if (active) {
#pragma unroll
    for (int run = 0; run < 2; ++run) {
      const unsigned long long i = c + 512 * run + 8 * lane;
      if (h.mode == 1) {
#pragma unroll
        for (int q = 0; q < 4; ++q)
          codes[run][q] = load_bytes(payload + h.code_at[q] + h.width[q] * (i >> 3), h.width[q]);
      } else {
        low[run] = load_stream8(payload + h.low_at + i);
        codes[run][0] = load_bytes(payload + h.code_at[0] + h.width[0] * (i >> 3), h.width[0]);
        if (h.mode == 2) signs[run] = payload[h.sign_at + (i >> 3)];
      }
    }
  }
  if (h.mode != 2) s_pal[tid] = (unsigned char)pal;
  __syncthreads();
  if (!active) return;
  u32x4 o[2];
#pragma unroll
  for (int run = 0; run < 2; ++run) {
    unsigned int word[8];
    if (h.mode == 1) {
#pragma unroll
      for (int k = 0; k < 8; ++k) word[k] = 0;
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int k = 0; k < 8; ++k)
          word[k] |= (unsigned int)s_pal[16 * q + run_code(codes[run][q], h.width[q], k)]
                     << (4 * q);
    } else {
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const unsigned int code = run_code(codes[run][0], h.width[0], k);
        const unsigned int hi = h.mode == 2
                                    ? (((signs[run] >> k) & 1u) << 7) | (code + h.mag_min)
                                    : (unsigned int)s_pal[code];
        const unsigned int lo = ((k < 4 ? low[run].x : low[run].y) >> (8 * (k & 3))) & 0xFFu;
        word[k] = (hi << 8) | lo;
      }
    }
    o[run].x = (word[0] & 0xFFFFu) | (word[1] << 16);
    o[run].y = (word[2] & 0xFFFFu) | (word[3] << 16);
    o[run].z = (word[4] & 0xFFFFu) | (word[5] << 16);
    o[run].w = (word[6] & 0xFFFFu) | (word[7] << 16);
  }
  // write-through stores after the last load (the compiler's waits do not see them)
  asm volatile("" ::"v"(o[0]), "v"(o[1]));
  store_through16(dst + 8 * lane, o[0]);
  store_through16(dst + 512 + 8 * lane, o[1]);
}

}  // namespace
}  // namespace unchainkv

using namespace unchainkv;

namespace {

unsigned long long torchop_tiles(unsigned long long n) {
  return (n + kTorchopTile - 1) / kTorchopTile;
}

// The tile kernels' geometry: 1024-word wave chunks inside one block, 16-byte
// aligned runs of the layer.
bool torchop_tile_geometry(unsigned long long kv_ptr, unsigned long long plane_stride,
                           unsigned long long block_stride, unsigned long long block_words) {
  return block_words % 1024 == 0 && kv_ptr % 16 == 0 && plane_stride % 8 == 0 &&
         block_stride % 8 == 0;
}

}  // namespace

// Decodes payload r (src + src_offsets[r], encoded_bytes[r] long; byte 0 is its
// mode, 0, 1 or 2) and scatters it into blocks ids[block_offsets[r] ..
// block_offsets[r+1]) of one paged layer. Returns the total raw bytes, 0 on a failed
// precondition, -1 on a launch error.
extern "C" long long kvq_splitzip_bf16_decode_torchop_paged(
    unsigned long long src_ptr, const unsigned long long* src_offsets,
    const unsigned long long* encoded_bytes, unsigned long long payload_count,
    unsigned long long kv_ptr, unsigned long long plane_stride, unsigned long long block_stride,
    unsigned long long block_words, unsigned long long block_ids_ptr,
    const unsigned long long* block_offsets, unsigned long long stream_ptr) {
  if (src_ptr == 0 || kv_ptr == 0 || block_ids_ptr == 0 || src_offsets == nullptr ||
      encoded_bytes == nullptr || block_offsets == nullptr || payload_count == 0 ||
      block_words == 0 || block_words > 0xFFFFFFFFULL || kv_ptr % 2 != 0)
    return 0;
  unsigned long long total = 0, max_n = 0;
  for (unsigned long long r = 0; r < payload_count; ++r) {
    if (block_offsets[r + 1] <= block_offsets[r] || encoded_bytes[r] == 0) return 0;
    const unsigned long long n = 2 * (block_offsets[r + 1] - block_offsets[r]) * block_words;
    if (n > 0xFFFFFFFFULL) return 0;
    total += 2 * n;
    max_n = std::max(max_n, n);
  }
  const bool tiles = torchop_tile_geometry(kv_ptr, plane_stride, block_stride, block_words);
  const EncodeGeom geo = make_geom(block_words);
  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_ptr);
  for (unsigned long long first = 0; first < payload_count; first += kMaxPayloads) {
    LaunchArgs a{};
    TorchopSizes sizes{};
    a.kv = reinterpret_cast<uint16_t*>(kv_ptr);
    a.ids = reinterpret_cast<const long long*>(block_ids_ptr);
    a.buf = reinterpret_cast<unsigned char*>(src_ptr);
    a.plane_stride = plane_stride;
    a.block_stride = block_stride;
    a.block_words = block_words;
    const unsigned int count =
        (unsigned int)std::min<unsigned long long>(kMaxPayloads, payload_count - first);
    unsigned long long launch_max = 0, launch_tiles = 0;
    bool uniform_size = true;
    for (unsigned int k = 0; k < count; ++k) {
      const unsigned long long r = first + k;
      a.p[k].buf_offset = src_offsets[r];
      a.p[k].ids_offset = block_offsets[r];
      a.p[k].block_count = (unsigned int)(block_offsets[r + 1] - block_offsets[r]);
      a.p[k].tile_begin = (unsigned int)launch_tiles;
      sizes.encoded[k] = encoded_bytes[r];
      const unsigned long long n = 2ull * a.p[k].block_count * block_words;
      launch_max = std::max(launch_max, n);
      launch_tiles += torchop_tiles(n);
      uniform_size = uniform_size && a.p[k].block_count == a.p[0].block_count;
    }
    a.payload_count = count;
    const dim3 grid((unsigned int)((launch_max + kTorchopTile - 1) / kTorchopTile), count);
    if (tiles && launch_tiles <= 0xFFFFFFFFULL) {
      a.total_tiles = (unsigned int)launch_tiles;
      a.uniform_tiles = uniform_size ? (unsigned int)(launch_tiles / count) : 0;
      hipLaunchKernelGGL(torchop_decode_tile, dim3(a.total_tiles), dim3(kThreads), 0, stream, a,
                         geo, sizes);
    } else
      hipLaunchKernelGGL(torchop_decode_generic, grid, dim3(kThreads), 0, stream, a, sizes);
    const hipError_t st = hipGetLastError();
    if (st != hipSuccess) return fail("torchop_decode", st);
  }
  return (long long)total;
}

namespace {


// Fills the launch arguments of payloads [first, first + count): descriptors with
// their first tile within the launch, the launch's tile count and, when every
// payload has the same size, its tiles per payload. The launch's tile records
// start at record tile_prefix. False when a word or tile count is past the
// kernels' limits.
bool torchop_args(LaunchArgs& a, unsigned long long kv_ptr, unsigned long long plane_stride,
                  unsigned long long block_stride, unsigned long long block_words,
                  unsigned long long block_ids_ptr, const unsigned long long* block_offsets,
                  unsigned long long first, unsigned int count, unsigned long long tile_prefix,
                  unsigned long long& max_n) {
  a = LaunchArgs{};
  a.kv = reinterpret_cast<uint16_t*>(kv_ptr);
  a.ids = reinterpret_cast<const long long*>(block_ids_ptr);
  a.plane_stride = plane_stride;
  a.block_stride = block_stride;
  a.block_words = block_words;
  a.payload_count = count;
  max_n = 0;
  unsigned long long tile = 0;  // tiles of the launch before payload k
  bool uniform_size = true;
  for (unsigned int k = 0; k < count; ++k) {
    const unsigned long long r = first + k;
    const unsigned long long blocks = block_offsets[r + 1] - block_offsets[r];
    const unsigned long long n = 2 * blocks * block_words;
    if (n > 0x7FFFFFFFULL || tile_prefix + tile > 0xFFFFFFFFULL) return false;
    a.p[k].ids_offset = block_offsets[r];
    a.p[k].block_count = (unsigned int)blocks;
    a.p[k].tile_begin = (unsigned int)tile;
    tile += torchop_tiles(n);
    max_n = std::max(max_n, n);
    uniform_size = uniform_size && blocks == block_offsets[first + 1] - block_offsets[first];
  }
  if (tile > 0xFFFFFFFFULL) return false;
  a.total_tiles = (unsigned int)tile;
  a.uniform_tiles = uniform_size ? (unsigned int)(tile / count) : 0;
  return true;
}

bool torchop_tables_ok(unsigned long long kv_ptr, unsigned long long block_words,
                       unsigned long long block_ids_ptr, const unsigned long long* block_offsets,
                       unsigned long long payload_count) {
  if (kv_ptr == 0 || block_ids_ptr == 0 || block_offsets == nullptr || payload_count == 0 ||
      block_words == 0 || block_words > 0xFFFFFFFFULL || kv_ptr % 2 != 0)
    return false;
  for (unsigned long long r = 0; r < payload_count; ++r)
    if (block_offsets[r + 1] <= block_offsets[r]) return false;
  return true;
}

}  // namespace

// Plan records are 64 bytes per payload.
extern "C" unsigned long long kvq_splitzip_torchop_plan_bytes() { return sizeof(TorchopPlan); }

// Workspace of kvq_splitzip_bf16_plan_torchop_paged: 64 bytes per 4096-word tile of
// every payload; 0 when the block offsets do not increase.
extern "C" unsigned long long kvq_splitzip_torchop_workspace_bytes(
    unsigned long long block_words, const unsigned long long* block_offsets,
    unsigned long long payload_count) {
  if (block_offsets == nullptr || payload_count == 0 || block_words == 0) return 0;
  unsigned long long tiles = 0;
  for (unsigned long long r = 0; r < payload_count; ++r) {
    if (block_offsets[r + 1] <= block_offsets[r]) return 0;
    tiles += torchop_tiles(2 * (block_offsets[r + 1] - block_offsets[r]) * block_words);
  }
  return tiles * kTorchopRecordWords * 4;
}

extern "C" long long kvq_splitzip_bf16_plan_torchop_paged(
    unsigned long long kv_ptr, unsigned long long plane_stride, unsigned long long block_stride,
    unsigned long long block_words, unsigned long long block_ids_ptr,
    const unsigned long long* block_offsets, unsigned long long payload_count,
    unsigned long long workspace_ptr, unsigned long long workspace_bytes,
    unsigned long long plans_ptr, unsigned long long stream_ptr) {
  if (!torchop_tables_ok(kv_ptr, block_words, block_ids_ptr, block_offsets, payload_count) ||
      workspace_ptr == 0 || plans_ptr == 0 || workspace_ptr % 4 != 0 || plans_ptr % 8 != 0)
    return 0;
  const unsigned long long need =
      kvq_splitzip_torchop_workspace_bytes(block_words, block_offsets, payload_count);
  if (need == 0 || workspace_bytes < need) return 0;
  const bool tiles = torchop_tile_geometry(kv_ptr, plane_stride, block_stride, block_words);
  const EncodeGeom geo = make_geom(block_words);
  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_ptr);
  unsigned long long tile_prefix = 0;
  for (unsigned long long first = 0; first < payload_count; first += kMaxPayloads) {
    const unsigned int count =
        (unsigned int)std::min<unsigned long long>(kMaxPayloads, payload_count - first);
    LaunchArgs a;
    unsigned long long max_n = 0;
    if (!torchop_args(a, kv_ptr, plane_stride, block_stride, block_words, block_ids_ptr,
                      block_offsets, first, count, tile_prefix, max_n))
      return 0;
    a.workspace = reinterpret_cast<unsigned int*>(workspace_ptr);
    const unsigned int base = (unsigned int)tile_prefix;
    if (tiles)
      hipLaunchKernelGGL(torchop_presence_tile, dim3(a.total_tiles), dim3(kThreads), 0, stream, a,
                         geo, base);
    else
      hipLaunchKernelGGL(torchop_presence_generic, dim3((unsigned int)torchop_tiles(max_n), count),
                         dim3(kThreads), 0, stream, a, base);
    const hipError_t st = hipGetLastError();
    if (st != hipSuccess) return fail("torchop_presence", st);
    tile_prefix += a.total_tiles;
  }
  // one plan launch for up to kPlanPayloads payloads, after every presence launch
  unsigned long long record = 0;
  for (unsigned long long first = 0; first < payload_count; first += kPlanPayloads) {
    const unsigned int count =
        (unsigned int)std::min<unsigned long long>(kPlanPayloads, payload_count - first);
    PlanArgs pa{};
    pa.workspace = reinterpret_cast<const unsigned int*>(workspace_ptr);
    pa.block_words = block_words;
    for (unsigned int k = 0; k < count; ++k) {
      const unsigned long long blocks = block_offsets[first + k + 1] - block_offsets[first + k];
      pa.record_begin[k] = (unsigned int)record;
      pa.blocks[k] = (unsigned int)blocks;
      record += torchop_tiles(2 * blocks * block_words);
    }
    hipLaunchKernelGGL(torchop_plan, dim3(count), dim3(kThreads), 0, stream, pa,
                       reinterpret_cast<TorchopPlan*>(plans_ptr) + first);
    const hipError_t st = hipGetLastError();
    if (st != hipSuccess) return fail("torchop_plan", st);
  }
  return (long long)payload_count;
}

extern "C" long long kvq_splitzip_bf16_encode_torchop_paged(
    unsigned long long kv_ptr, unsigned long long plane_stride, unsigned long long block_stride,
    unsigned long long block_words, unsigned long long block_ids_ptr,
    const unsigned long long* block_offsets, unsigned long long payload_count,
    unsigned long long plans_ptr, unsigned long long out_ptr,
    const unsigned long long* out_offsets, const unsigned long long* encoded_bytes,
    unsigned long long out_capacity, unsigned long long stream_ptr) {
  if (!torchop_tables_ok(kv_ptr, block_words, block_ids_ptr, block_offsets, payload_count) ||
      plans_ptr == 0 || plans_ptr % 8 != 0 || out_ptr == 0 || out_offsets == nullptr ||
      encoded_bytes == nullptr)
    return 0;
  const bool tiles = torchop_tile_geometry(kv_ptr, plane_stride, block_stride, block_words);
  const EncodeGeom geo = make_geom(block_words);
  unsigned long long total = 0;
  for (unsigned long long r = 0; r < payload_count; ++r) {
    const unsigned long long n = 2 * (block_offsets[r + 1] - block_offsets[r]) * block_words;
    const unsigned long long size = encoded_bytes[r];
    if (size == 0) continue;  // declined by its plan: nothing to write
    if (size >= 2 * n || out_offsets[r] > out_capacity || size > out_capacity - out_offsets[r])
      return 0;
    total += size;
  }
  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_ptr);
  for (unsigned long long first = 0; first < payload_count; first += kMaxPayloads) {
    const unsigned int count =
        (unsigned int)std::min<unsigned long long>(kMaxPayloads, payload_count - first);
    LaunchArgs a;
    unsigned long long max_n = 0;
    if (!torchop_args(a, kv_ptr, plane_stride, block_stride, block_words, block_ids_ptr,
                      block_offsets, first, count, 0, max_n))
      return 0;
    a.buf = reinterpret_cast<unsigned char*>(out_ptr);
    TorchopSizes sizes{};
    for (unsigned int k = 0; k < count; ++k) {
      a.p[k].buf_offset = out_offsets[first + k];
      sizes.encoded[k] = encoded_bytes[first + k];
    }
    const dim3 grid((unsigned int)torchop_tiles(max_n), count);
    const TorchopPlan* plans = reinterpret_cast<const TorchopPlan*>(plans_ptr) + first;
    if (tiles)
      hipLaunchKernelGGL(torchop_encode_tile, dim3(a.total_tiles), dim3(kThreads), 0, stream, a,
                         geo, plans, sizes);
    else
      hipLaunchKernelGGL(torchop_encode_generic, grid, dim3(kThreads), 0, stream, a, plans, sizes);
    const hipError_t st = hipGetLastError();
    if (st != hipSuccess) return fail("torchop_encode", st);
  }
  return (long long)total;
}
