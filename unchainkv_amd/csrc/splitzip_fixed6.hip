// Palette codecs fixed6 (mode 3) and fixed5 (mode 4) for bf16 KV cache, gfx950.
// They are the Top-16 overflow fallback of the connector.
//
// Wire format (native/unchain_kv/kvq_splitzip_cuda.cu:57-111, 292-333):
//   fixed6: [3][64-byte palette of high bytes][n low bytes][ceil(n/4) x 3 code bytes]
//   fixed5: [4][32-byte palette][n low bytes][ceil(n/8) x 5 code bytes]
// A group's codes are packed little-endian, first word in the low bits. With more
// distinct high bytes than palette entries byte 0 is 255.
//
// The palette is the set of distinct high bytes in ascending order, unused entries
// zeroed (the reference builds it first-come with atomicCAS, so its order varies
// from run to run; every order decodes to the same words).
//
// Kernels: palette_clear (zero the 256-bit presence mask), palette_presence
// (presence of every high byte, LDS mask per workgroup), palette_encode (rank
// table from the mask, low bytes + codes), fixed6_decode (decode + scatter).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>

#include "splitzip_common.h"

namespace unchainkv {
namespace {

__global__ void palette_clear(unsigned int* mask) {
  if (threadIdx.x < 8) mask[threadIdx.x] = 0;
}

__global__ __launch_bounds__(kThreads) void palette_presence(const uint16_t* src,
                                                             unsigned long long n,
                                                             unsigned int* mask) {
  __shared__ unsigned int s_mask[8];
  if (threadIdx.x < 8) s_mask[threadIdx.x] = 0;
  __syncthreads();
  unsigned int local[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  unsigned int last = 0x100;  // runs of one high byte are common; skip repeats
  for (unsigned long long i = (unsigned long long)blockIdx.x * kThreads + threadIdx.x; i < n;
       i += (unsigned long long)gridDim.x * kThreads) {
    const unsigned int h = src[i] >> 8;
    if (h == last) continue;
    last = h;
#pragma unroll
    for (int k = 0; k < 8; ++k)
      if ((h >> 5) == (unsigned int)k) local[k] |= 1u << (h & 31);
  }
#pragma unroll
  for (int k = 0; k < 8; ++k)
    if (local[k]) atomicOr(&s_mask[k], local[k]);
  __syncthreads();
  if (threadIdx.x < 8 && s_mask[threadIdx.x]) atomicOr(&mask[threadIdx.x], s_mask[threadIdx.x]);
}

template <int kBits>
__global__ __launch_bounds__(kThreads) void palette_encode(const uint16_t* src,
                                                           unsigned long long n,
                                                           unsigned char* dst,
                                                           const unsigned int* mask) {
  constexpr int kLimit = kBits == 6 ? 64 : 32;
  constexpr int kGroup = kBits == 6 ? 4 : 8;
  constexpr int kGroupBytes = kBits == 6 ? 3 : 5;
  constexpr int kHeader = 1 + kLimit;
  __shared__ unsigned char s_rank[256];
  __shared__ unsigned char s_pal[kLimit];
  __shared__ unsigned int s_mask[8];
  const unsigned int tid = threadIdx.x;
  if (tid < 8) s_mask[tid] = mask[tid];
  if (tid < kLimit) s_pal[tid] = 0;
  __syncthreads();
  unsigned int distinct = 0;
  for (int k = 0; k < 8; ++k) distinct += __popc(s_mask[k]);
  if (distinct > (unsigned int)kLimit) {
    if (blockIdx.x == 0 && tid == 0) dst[0] = 255;
    return;
  }
  {
    const unsigned int h = tid;  // 256 threads, one high byte each
    unsigned int rank = 0;
    for (unsigned int k = 0; k < (h >> 5); ++k) rank += __popc(s_mask[k]);
    rank += __popc(s_mask[h >> 5] & ((1u << (h & 31)) - 1u));
    const bool present = (s_mask[h >> 5] >> (h & 31)) & 1u;
    s_rank[h] = (unsigned char)(present ? rank : 0);
    if (present) s_pal[rank] = (unsigned char)h;
  }
  __syncthreads();
  if (blockIdx.x == 0) {
    if (tid == 0) dst[0] = kBits == 6 ? 3 : 4;
    if (tid < kLimit) dst[1 + tid] = s_pal[tid];
  }
  unsigned char* low = dst + kHeader;
  unsigned char* codes = low + n;
  const unsigned long long groups = (n + kGroup - 1) / kGroup;
  for (unsigned long long g = (unsigned long long)blockIdx.x * kThreads + tid; g < groups;
       g += (unsigned long long)gridDim.x * kThreads) {
    unsigned long long bits = 0;
#pragma unroll
    for (int k = 0; k < kGroup; ++k) {
      const unsigned long long i = g * kGroup + k;
      if (i >= n) break;
      const unsigned int w = src[i];
      low[i] = (unsigned char)(w & 0xFF);
      bits |= (unsigned long long)(s_rank[w >> 8] & (kLimit - 1)) << (k * kBits);
    }
#pragma unroll
    for (int k = 0; k < kGroupBytes; ++k)
      codes[g * kGroupBytes + k] = (unsigned char)(bits >> (8 * k));
  }
}

// DecodeFixed6 semantics (kvq_splitzip_cuda.cu:113-144): no-op unless byte 0 is 3.
__global__ __launch_bounds__(kThreads) void fixed6_decode(LaunchArgs a) {
  __shared__ unsigned char s_pal[64];
  const unsigned char* payload = a.buf;
  if (payload[0] != 3) return;
  if (threadIdx.x < 64) s_pal[threadIdx.x] = payload[1 + threadIdx.x];
  __syncthreads();
  const PayloadDesc d = a.p[0];
  const unsigned long long n = 2ull * d.block_count * a.block_words;
  const unsigned char* low = payload + 65;
  const unsigned char* codes = low + n;
  const unsigned long long groups = (n + 3) / 4;
  for (unsigned long long g = (unsigned long long)blockIdx.x * kThreads + threadIdx.x; g < groups;
       g += (unsigned long long)gridDim.x * kThreads) {
    const unsigned int packed = (unsigned int)codes[g * 3] |
                                ((unsigned int)codes[g * 3 + 1] << 8) |
                                ((unsigned int)codes[g * 3 + 2] << 16);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const unsigned long long i = g * 4 + k;
      if (i >= n) break;
      const unsigned int code = (packed >> (6 * k)) & 0x3F;
      a.kv[word_offset(a, d, i)] = (uint16_t)(((unsigned int)s_pal[code] << 8) | low[i]);
    }
  }
}

unsigned int grid_for(unsigned long long items) {
  return (unsigned int)std::max<unsigned long long>(
      1, std::min<unsigned long long>((items + kThreads - 1) / kThreads, 4096));
}

}  // namespace
}  // namespace unchainkv

using namespace unchainkv;

// kvq_splitzip_cuda.cu:292-333: same preconditions, same return values. The
// 8-word presence mask lives in the caller's buffer at align4(encoded).
extern "C" long long kvq_splitzip_bf16_encode_mode(unsigned long long src_ptr,
                                                   unsigned long long dst_ptr,
                                                   unsigned long long count,
                                                   unsigned long long capacity,
                                                   unsigned long long stream_ptr, int bits) {
  if (src_ptr == 0 || dst_ptr == 0 || count == 0) return 0;
  if (bits != 5 && bits != 6) return 0;
  const unsigned long long code_bytes = bits == 5 ? ((count + 7) / 8) * 5 : ((count + 3) / 4) * 3;
  const unsigned long long header_bytes = bits == 5 ? 33 : 65;
  const unsigned long long encoded = header_bytes + count + code_bytes;
  const unsigned long long scratch_offset = (encoded + 3) & ~3ULL;
  const unsigned long long scratch = 256 * sizeof(int) + 2 * sizeof(int);
  if (encoded >= count * 2 || scratch_offset + scratch > capacity) return 0;
  const uint16_t* src = reinterpret_cast<const uint16_t*>(src_ptr);
  unsigned char* dst = reinterpret_cast<unsigned char*>(dst_ptr);
  // 4-byte aligned place for the mask inside the scratch area
  const unsigned long long mask_addr = (dst_ptr + scratch_offset + 3) & ~3ULL;
  unsigned int* mask = reinterpret_cast<unsigned int*>(mask_addr);
  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_ptr);
  hipLaunchKernelGGL(palette_clear, dim3(1), dim3(64), 0, stream, mask);
  hipError_t st = hipGetLastError();
  if (st != hipSuccess) return fail("palette_clear", st);
  hipLaunchKernelGGL(palette_presence, dim3(grid_for(count)), dim3(kThreads), 0, stream, src,
                     count, mask);
  st = hipGetLastError();
  if (st != hipSuccess) return fail("palette_presence", st);
  const unsigned long long groups = bits == 5 ? (count + 7) / 8 : (count + 3) / 4;
  if (bits == 5)
    hipLaunchKernelGGL(palette_encode<5>, dim3(grid_for(groups)), dim3(kThreads), 0, stream, src,
                       count, dst, mask);
  else
    hipLaunchKernelGGL(palette_encode<6>, dim3(grid_for(groups)), dim3(kThreads), 0, stream, src,
                       count, dst, mask);
  st = hipGetLastError();
  if (st != hipSuccess) return fail(bits == 5 ? "EncodeFixed5" : "EncodeFixed6", st);
  return (long long)encoded;
}

extern "C" long long kvq_splitzip_bf16_encode(unsigned long long src_ptr,
                                              unsigned long long dst_ptr,
                                              unsigned long long count,
                                              unsigned long long capacity,
                                              unsigned long long stream_ptr) {
  return kvq_splitzip_bf16_encode_mode(src_ptr, dst_ptr, count, capacity, stream_ptr, 6);
}

extern "C" long long kvq_splitzip_bf16_decode_fixed6_blocks(
    unsigned long long src_ptr, unsigned long long encoded_bytes, unsigned long long dst_ptr,
    unsigned long long count_words, unsigned long long block_count,
    unsigned long long block_words, unsigned long long plane_stride,
    unsigned long long block_stride, unsigned long long block_start,
    unsigned long long block_ids_ptr, unsigned long long stream_ptr) {
  // kvq_splitzip_cuda.cu:351-357
  if (src_ptr == 0 || dst_ptr == 0 || count_words == 0 || block_count == 0 || block_words == 0 ||
      count_words != 2 * block_count * block_words)
    return 0;
  if (encoded_bytes != 65 + count_words + ((count_words + 3) / 4) * 3) return 0;
  if (block_count > 0xFFFFFFFFULL)
    return fail_msg("decode_fixed6: block_count must fit in 32 bits");
  LaunchArgs a{};
  a.kv = reinterpret_cast<uint16_t*>(dst_ptr);
  a.ids = reinterpret_cast<const long long*>(block_ids_ptr);
  a.buf = reinterpret_cast<unsigned char*>(src_ptr);
  a.plane_stride = plane_stride;
  a.block_stride = block_stride;
  a.block_words = block_words;
  a.block_start = block_start;
  a.payload_count = 1;
  a.p[0].block_count = (unsigned int)block_count;
  hipLaunchKernelGGL(fixed6_decode, dim3(grid_for((count_words + 3) / 4)), dim3(kThreads), 0,
                     reinterpret_cast<hipStream_t>(stream_ptr), a);
  hipError_t st = hipGetLastError();
  if (st != hipSuccess) return fail("DecodeFixed6", st);
  return (long long)(count_words * sizeof(uint16_t));
}

extern "C" long long kvq_splitzip_bf16_decode_fixed6(
    unsigned long long src_ptr, unsigned long long encoded_bytes, unsigned long long dst_ptr,
    unsigned long long count_words, unsigned long long block_count,
    unsigned long long block_words, unsigned long long plane_stride,
    unsigned long long block_stride, unsigned long long block_start,
    unsigned long long stream_ptr) {
  return kvq_splitzip_bf16_decode_fixed6_blocks(src_ptr, encoded_bytes, dst_ptr, count_words,
                                                block_count, block_words, plane_stride,
                                                block_stride, block_start, 0, stream_ptr);
}
