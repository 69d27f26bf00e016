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
// Workgroup (x, y): payload y of the launch, words [4096 x, 4096 x + 4096); a thread
// decodes 16 consecutive words. Byte-granular reads (these are fallback formats),
// 16-byte stores when a thread's words lie in one block.
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

__device__ TorchopHeader parse_header(const unsigned char* h, unsigned long long size,
                                      unsigned long long n) {
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

__global__ __launch_bounds__(kThreads) void torchop_decode(LaunchArgs a, TorchopSizes sizes) {
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
  const TorchopHeader h = parse_header(s_hdr, size, n);
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

}  // namespace
}  // namespace unchainkv

using namespace unchainkv;

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
    unsigned long long launch_max = 0;
    for (unsigned int k = 0; k < count; ++k) {
      const unsigned long long r = first + k;
      a.p[k].buf_offset = src_offsets[r];
      a.p[k].ids_offset = block_offsets[r];
      a.p[k].block_count = (unsigned int)(block_offsets[r + 1] - block_offsets[r]);
      sizes.encoded[k] = encoded_bytes[r];
      launch_max = std::max(launch_max, 2ull * a.p[k].block_count * block_words);
    }
    a.payload_count = count;
    const dim3 grid((unsigned int)((launch_max + kTorchopTile - 1) / kTorchopTile), count);
    hipLaunchKernelGGL(torchop_decode, grid, dim3(kThreads), 0, stream, a, sizes);
    const hipError_t st = hipGetLastError();
    if (st != hipSuccess) return fail("torchop_decode", st);
  }
  return (long long)total;
}
