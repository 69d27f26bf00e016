// bf16 exponent histograms of a paged KV layer (gfx950): the statistics the Top-16
// codebooks are fit from.
//
// The reference computes, per K/V plane of a gathered request, a 256-bin count of
// (word >> 7) & 0xFF with torch.bincount (src/unchain_kv/vllm_connector.py:2871-2904)
// and ranks it offline (scripts/extract_llama_top16_codebooks.py:15-60). Here one
// call counts every listed block of a paged layer, K plane and V plane separately,
// straight from the cache (no gather copy).
//
// Two kernels, no global atomics, deterministic output:
//   exponent_hist_partial: each wave streams 1024-word chunks (one KV block each)
//     and adds every word's exponent into an LDS histogram of its own; a bin is
//     kept in 4 copies selected by lane % 4, interleaved so the copies sit in
//     different banks, which cuts the serialisation of same-bin LDS atomics (a
//     bf16 plane concentrates on ~16 exponents). The workgroup then writes one
//     512-bin partial (K bins, then V bins).
//   exponent_hist_reduce: sums the partials into 64-bit counts.
// Layouts that the chunk kernel cannot take (block words not a multiple of 1024,
// misaligned cache) go through a one-word-per-thread kernel with the same output.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>

#include "splitzip_common.h"

namespace unchainkv {
namespace {

constexpr int kBins = 256;
constexpr int kCopies = 4;
constexpr int kChunk = 1024;                   // words per wave step (one block)
constexpr unsigned int kMaxPartials = 2048;    // workgroups of the partial kernel

struct HistArgs {
  const uint16_t* kv;
  const long long* ids;
  unsigned int* partial;  // [workgroup][2 * kBins]
  unsigned long long plane_stride, block_stride, block_words, block_count;
  unsigned long long chunks_per_plane;  // block_count * block_words / kChunk (chunk kernel)
};

// LDS histogram of one wave: [plane][bin][copy]
__device__ __forceinline__ unsigned int hist_index(unsigned int plane, unsigned int bin,
                                                   unsigned int copy) {
  return (plane * kBins + bin) * kCopies + copy;
}

__device__ __forceinline__ void add_word(unsigned int* h, unsigned int plane, uint32_t w,
                                         unsigned int copy) {
  atomicAdd(&h[hist_index(plane, (w >> 7) & 0xFFu, copy)], 1u);
}

// Sums the 4 waves x 4 copies of every bin and writes the workgroup's partial.
__device__ __forceinline__ void write_partial(const unsigned int (*h)[2 * kBins * kCopies],
                                              unsigned int* partial) {
  for (unsigned int b = threadIdx.x; b < 2 * kBins; b += kThreads) {
    unsigned int s = 0;
#pragma unroll
    for (int w = 0; w < kThreads / kWave; ++w)
#pragma unroll
      for (int c = 0; c < kCopies; ++c) s += h[w][b * kCopies + c];
    partial[(unsigned long long)blockIdx.x * 2 * kBins + b] = s;
  }
}

__device__ __forceinline__ u32x4 load_chunk_part(const HistArgs& a, unsigned long long chunk,
                                                 unsigned int half_lane_word) {
  const unsigned int plane = chunk >= a.chunks_per_plane ? 1u : 0u;
  const unsigned long long word = (chunk - plane * a.chunks_per_plane) * kChunk;
  const unsigned long long j = word / a.block_words;
  const unsigned long long within = word - j * a.block_words;
  const uint16_t* src = a.kv + plane * a.plane_stride +
                        (unsigned long long)a.ids[j] * a.block_stride + within;
  return load_stream16(src + half_lane_word);
}

__global__ __launch_bounds__(kThreads) void exponent_hist_partial(HistArgs a) {
  __shared__ unsigned int h[kThreads / kWave][2 * kBins * kCopies];
  const unsigned int lane = threadIdx.x & (kWave - 1);
  const unsigned int wave = threadIdx.x / kWave;
  unsigned int* mine = h[wave];
  for (unsigned int i = lane; i < 2 * kBins * kCopies; i += kWave) mine[i] = 0;
  const unsigned int copy = lane % kCopies;
  const unsigned long long chunks = 2 * a.chunks_per_plane;
  const unsigned long long stride = (unsigned long long)gridDim.x * (kThreads / kWave);
  unsigned long long chunk = (unsigned long long)blockIdx.x * (kThreads / kWave) + wave;
  // one chunk ahead in registers: its loads are in flight while this one is counted
  u32x4 cur0 = {0, 0, 0, 0}, cur1 = {0, 0, 0, 0};
  if (chunk < chunks) {
    cur0 = load_chunk_part(a, chunk, 8 * lane);
    cur1 = load_chunk_part(a, chunk, 512 + 8 * lane);
  }
  for (; chunk < chunks; chunk += stride) {
    const unsigned long long next = chunk + stride;
    u32x4 nxt0 = {0, 0, 0, 0}, nxt1 = {0, 0, 0, 0};
    if (next < chunks) {
      nxt0 = load_chunk_part(a, next, 8 * lane);
      nxt1 = load_chunk_part(a, next, 512 + 8 * lane);
    }
    const unsigned int plane = chunk >= a.chunks_per_plane ? 1u : 0u;
    const uint32_t x[8] = {cur0.x, cur0.y, cur0.z, cur0.w, cur1.x, cur1.y, cur1.z, cur1.w};
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      add_word(mine, plane, x[k], copy);
      add_word(mine, plane, x[k] >> 16, copy);
    }
    cur0 = nxt0;
    cur1 = nxt1;
  }
  __syncthreads();
  write_partial(h, a.partial);
}

// Any layout: one word per thread, grid-stride.
__global__ __launch_bounds__(kThreads) void exponent_hist_generic(HistArgs a) {
  __shared__ unsigned int h[kThreads / kWave][2 * kBins * kCopies];
  const unsigned int lane = threadIdx.x & (kWave - 1);
  unsigned int* mine = h[threadIdx.x / kWave];
  for (unsigned int i = lane; i < 2 * kBins * kCopies; i += kWave) mine[i] = 0;
  const unsigned long long plane_words = a.block_count * a.block_words;
  const unsigned long long total = 2 * plane_words;
  for (unsigned long long i = (unsigned long long)blockIdx.x * kThreads + threadIdx.x; i < total;
       i += (unsigned long long)gridDim.x * kThreads) {
    const unsigned int plane = i >= plane_words ? 1u : 0u;
    const unsigned long long in_plane = i - plane * plane_words;
    const unsigned long long j = in_plane / a.block_words;
    const unsigned long long within = in_plane - j * a.block_words;
    const uint32_t w = a.kv[plane * a.plane_stride + (unsigned long long)a.ids[j] * a.block_stride +
                            within];
    add_word(mine, plane, w, lane % kCopies);
  }
  __syncthreads();
  write_partial(h, a.partial);
}

__global__ __launch_bounds__(kThreads) void exponent_hist_reduce(const unsigned int* partial,
                                                                 unsigned int groups,
                                                                 unsigned long long* counts) {
  const unsigned int b = blockIdx.x * kThreads + threadIdx.x;  // grid covers 2 * kBins
  unsigned long long s = 0;
  for (unsigned int g = 0; g < groups; ++g) s += partial[(unsigned long long)g * 2 * kBins + b];
  counts[b] = s;
}

unsigned int partial_groups(unsigned long long block_count, unsigned long long block_words,
                            bool chunked) {
  const unsigned long long words = 2 * block_count * block_words;
  const unsigned long long per_group = chunked ? 4ull * kChunk * 8 : (unsigned long long)kThreads * 64;
  const unsigned long long g = (words + per_group - 1) / per_group;
  return (unsigned int)(g < 1 ? 1 : (g > kMaxPartials ? kMaxPartials : g));
}

bool chunk_layout(unsigned long long kv_ptr, unsigned long long plane_stride,
                  unsigned long long block_stride, unsigned long long block_words) {
  return block_words % kChunk == 0 && kv_ptr % 16 == 0 && plane_stride % 8 == 0 &&
         block_stride % 8 == 0;
}

}  // namespace
}  // namespace unchainkv

using namespace unchainkv;

// Workspace bytes kvq_splitzip_exponent_histogram_paged needs (no counterpart in the
// reference).
extern "C" unsigned long long kvq_splitzip_exponent_histogram_workspace_bytes(
    unsigned long long block_count, unsigned long long block_words) {
  if (block_count == 0 || block_words == 0) return 0;
  // the larger of the two kernels' partial counts
  const unsigned int g = std::max(partial_groups(block_count, block_words, true),
                                  partial_groups(block_count, block_words, false));
  return (unsigned long long)g * 2 * kBins * sizeof(unsigned int);
}

// Exponent histograms of blocks ids[0 .. block_count) of one paged layer: counts[b]
// (b < 256) = K-plane words whose bits 7..14 equal b, counts[256 + b] the same for
// the V plane (torch.bincount of (word >> 7) & 0xFF per plane, as the reference's
// exponent trace, src/unchain_kv/vllm_connector.py:2871-2904). counts is a device
// array of 512 u64, overwritten. Returns the words counted (2 * block_count *
// block_words), 0 on a failed precondition, -1 on a launch error.
extern "C" long long kvq_splitzip_exponent_histogram_paged(
    unsigned long long kv_ptr, unsigned long long plane_stride, unsigned long long block_stride,
    unsigned long long block_words, unsigned long long block_ids_ptr,
    unsigned long long block_count, unsigned long long counts_ptr,
    unsigned long long workspace_ptr, unsigned long long workspace_bytes,
    unsigned long long stream_ptr) {
  if (kv_ptr == 0 || block_ids_ptr == 0 || counts_ptr == 0 || workspace_ptr == 0 ||
      block_count == 0 || block_words == 0 || counts_ptr % 8 != 0 || workspace_ptr % 4 != 0 ||
      kv_ptr % 2 != 0)
    return 0;
  if (kvq_splitzip_exponent_histogram_workspace_bytes(block_count, block_words) > workspace_bytes)
    return 0;
  const bool chunked = chunk_layout(kv_ptr, plane_stride, block_stride, block_words);
  HistArgs a{};
  a.kv = reinterpret_cast<const uint16_t*>(kv_ptr);
  a.ids = reinterpret_cast<const long long*>(block_ids_ptr);
  a.partial = reinterpret_cast<unsigned int*>(workspace_ptr);
  a.plane_stride = plane_stride;
  a.block_stride = block_stride;
  a.block_words = block_words;
  a.block_count = block_count;
  a.chunks_per_plane = block_count * block_words / kChunk;
  const unsigned int groups = partial_groups(block_count, block_words, chunked);
  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_ptr);
  if (chunked)
    hipLaunchKernelGGL(exponent_hist_partial, dim3(groups), dim3(kThreads), 0, stream, a);
  else
    hipLaunchKernelGGL(exponent_hist_generic, dim3(groups), dim3(kThreads), 0, stream, a);
  hipError_t st = hipGetLastError();
  if (st != hipSuccess) return fail("exponent_hist_partial", st);
  hipLaunchKernelGGL(exponent_hist_reduce, dim3(2 * kBins / kThreads), dim3(kThreads), 0, stream,
                     a.partial, groups, reinterpret_cast<unsigned long long*>(counts_ptr));
  st = hipGetLastError();
  if (st != hipSuccess) return fail("exponent_hist_reduce", st);
  return (long long)(2 * block_count * block_words);
}
