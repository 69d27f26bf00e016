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
//   exponent_hist_partial: 512-thread workgroups, about one per CU; each wave
//     streams batches of two 1024-word chunks, two batches in flight (block ids
//     fetched a batch ahead), sixteen batches per wave, and adds every word's
//     exponent into the workgroup's LDS histogram. Lane l counts into copy l % 16
//     of the histogram, two 16-bit bins per dword, copy c in bank c: of the 32
//     lanes an LDS instruction serves at once only lanes l and l + 16 can meet on
//     one address (a bf16 plane concentrates on ~16 exponents, and colliding LDS
//     atomics serialise). A chunk's 16 addresses per lane are computed before its
//     16 LDS adds, so the adds go out back to back. The 16 KiB histogram leaves
//     the CU's LDS and registers to deep streaming (Llama-3-8B layer: 64 copies
//     and twelve-chunk batches 42.2 us, four-chunk batches 28.2 us, two-chunk
//     batches 26.3 us: as fast as the same loop with no LDS adds at all). The
//     workgroup then writes one 512-bin partial (K bins, then V bins).
//   exponent_hist_reduce: sums the partials into 64-bit counts, every bin's
//     groups split over sixteen threads.
// Layouts that the chunk kernel cannot take (block words not a multiple of 1024,
// misaligned cache) go through a one-word-per-thread kernel with the same output.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <mutex>

#include "splitzip_common.h"

namespace unchainkv {
namespace {

constexpr int kBins = 256;
constexpr int kCopies = 16;                    // lane l counts into copy l % 16
// 16-bit counters: a workgroup counts at most kCopies * 65535 words
constexpr int kChunk = 1024;                   // words per wave step (one block)
constexpr unsigned int kMaxPartials = 2048;    // workgroups of the partial kernel

// Chunks per wave step: 4 KiB of loads per wave, two steps in flight (63 VGPRs;
// Llama-3-8B call with 1, 2, 3, 4 and 6 chunks: 26.4, 26.3, 27.5, 28.1, 32.1 us).
constexpr int kBatch = 2;
// Threads of a partial-kernel workgroup and wave steps per wave (the grid size).
constexpr int kHistThreads = 512;
constexpr int kBatchesPerWave = 16;

struct HistArgs {
  const uint16_t* kv;
  const long long* ids;
  unsigned int* partial;  // [workgroup][2 * kBins]
  unsigned long long plane_stride, block_stride, block_words, block_count;
  // chunk kernel: chunks of one plane, chunks per block and its divider
  unsigned int chunks_per_plane, chunks_per_block;
  unsigned long long cpb_magic;
};

constexpr unsigned long long kMaxWordsPerGroup = (unsigned long long)kCopies * 65535;
constexpr int kHistWords = kBins * kCopies;     // dwords: 2 planes x 256 bins / 2 per dword,
                                                // per copy

// LDS histogram of a workgroup: dword [plane][bin / 2][copy], bin parity selects
// the 16-bit half.
__device__ __forceinline__ void add_word(unsigned int* h, unsigned int plane, uint32_t w,
                                         unsigned int copy) {
  const unsigned int bin = (w >> 7) & 0xFFu;
  atomicAdd(&h[(plane * (kBins / 2) + (bin >> 1)) * kCopies + copy], 1u << (16 * (bin & 1)));
}

__device__ __forceinline__ void zero_hist(unsigned int* h) {
  for (unsigned int i = threadIdx.x; i < kHistWords; i += blockDim.x) h[i] = 0;
  __syncthreads();
}

// Sums the copies of every bin and writes the workgroup's partial: thread t < 256
// sums the bin pair t (both halves of the copies' dwords).
__device__ __forceinline__ void write_partial(const unsigned int* h, unsigned int* partial) {
  __syncthreads();
  const unsigned int pair = threadIdx.x;  // 256 pairs = 512 bins
  if (pair >= kBins) return;
  unsigned int lo = 0, hi = 0;
#pragma unroll 8
  for (int c = 0; c < kCopies; ++c) {
    const unsigned int v = h[pair * kCopies + (c + pair) % kCopies];
    lo += v & 0xFFFFu;
    hi += v >> 16;
  }
  unsigned int* out = partial + (unsigned long long)blockIdx.x * 2 * kBins + 2 * pair;
  out[0] = lo;
  out[1] = hi;
}

// Block id of chunk c (lanes 0..kBatch-1 of a wave each fetch one chunk of a batch).
__device__ __forceinline__ long long chunk_block_id(const HistArgs& a, unsigned int c) {
  const unsigned int plane = c >= a.chunks_per_plane ? 1u : 0u;
  const unsigned int cin = c - plane * a.chunks_per_plane;
  return a.ids[div_u32(cin, a.cpb_magic, a.chunks_per_block)];
}

// Element offset of chunk c's first word, given its block id.
__device__ __forceinline__ unsigned long long chunk_offset(const HistArgs& a, unsigned int c,
                                                           unsigned long long id) {
  const unsigned int plane = c >= a.chunks_per_plane ? 1u : 0u;
  const unsigned int cin = c - plane * a.chunks_per_plane;
  const unsigned int j = div_u32(cin, a.cpb_magic, a.chunks_per_block);
  return plane * a.plane_stride + id * a.block_stride +
         (unsigned long long)(cin - j * a.chunks_per_block) * kChunk;
}

struct Batch {
  u32x4 d[2 * kBatch];
};

// Issues the loads of batch b (chunks kBatch*b ..), lane k of `idv` holding chunk
// k's block id. Chunks past the end re-read the last chunk, so that every load is
// issued unconditionally (a load under a branch makes the compiler wait for all
// outstanding loads where the paths join); count_batch skips them.
__device__ __forceinline__ Batch load_batch(const HistArgs& a, unsigned int b, long long idv,
                                            unsigned int total, unsigned int lane) {
  Batch r;
#pragma unroll
  for (int k = 0; k < kBatch; ++k) {
    const unsigned int c = min(b * kBatch + k, total - 1);
    const long long id = __builtin_amdgcn_readlane((int)idv, k) |
                         ((long long)__builtin_amdgcn_readlane((int)(idv >> 32), k) << 32);
    const uint16_t* src = a.kv + chunk_offset(a, c, (unsigned long long)id);
    r.d[2 * k] = load_stream16(src + 8 * lane);
    r.d[2 * k + 1] = load_stream16(src + 512 + 8 * lane);
  }
  return r;
}

// Block ids of batch b: lane k < kBatch loads chunk k's (clamped like the data).
__device__ __forceinline__ long long load_ids(const HistArgs& a, unsigned int b,
                                              unsigned int total, unsigned int lane) {
  return chunk_block_id(a, min(b * kBatch + (lane < (unsigned int)kBatch ? lane : 0u), total - 1));
}

// Adds the words of batch b (held in r) to the LDS histogram.
__device__ __forceinline__ void count_batch(unsigned int* h, const Batch& r, unsigned int b,
                                            unsigned int total, unsigned int chunks_per_plane,
                                            unsigned int copy) {
#pragma unroll
  for (int k = 0; k < kBatch; ++k) {
    const unsigned int c = b * kBatch + k;
    if (c >= total) break;
    const unsigned int plane = c >= chunks_per_plane ? 1u : 0u;
    const u32x4 x0 = r.d[2 * k], x1 = r.d[2 * k + 1];
    const uint32_t x[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
    // every address and increment first, then the 16 LDS adds
    unsigned int addr[16], inc[16];
#pragma unroll
    for (int q = 0; q < 16; ++q) {
      const unsigned int bin = (x[q >> 1] >> (7 + 16 * (q & 1))) & 0xFFu;
      addr[q] = (plane * (kBins / 2) + (bin >> 1)) * kCopies + copy;
      inc[q] = 1u << (16 * (bin & 1));
    }
#pragma unroll
    for (int q = 0; q < 16; ++q) atomicAdd(&h[addr[q]], inc[q]);
  }
}

__global__ __launch_bounds__(kHistThreads) void exponent_hist_partial(HistArgs a) {
  __shared__ unsigned int h[kHistWords];
  const unsigned int lane = threadIdx.x & (kWave - 1);
  const unsigned int wave = uniform(threadIdx.x / kWave);
  zero_hist(h);
  const unsigned int copy = lane % kCopies;
  const unsigned int total = 2 * a.chunks_per_plane;
  const unsigned int batches = (total + kBatch - 1) / kBatch;
  const unsigned int stride = gridDim.x * (kHistThreads / kWave);
  unsigned int b0 = blockIdx.x * (kHistThreads / kWave) + wave;
  if (b0 < batches) {
    // Two batches in flight, in two buffers used in turn (a copy from one to the
    // other would wait for its loads). The block ids of a batch are loaded one
    // step ahead and issued before the batch that precedes it, so waiting for them
    // (outstanding loads complete in issue order) does not wait for that batch.
    const long long id0 = load_ids(a, b0, total, lane);
    unsigned int bb = b0 + stride;
    long long id_b = load_ids(a, min(bb, batches - 1), total, lane);
    Batch ba = load_batch(a, b0, id0, total, lane);
    Batch bbuf;
    for (;;) {
      // past the last batch the loads repeat it and nothing is counted
      const unsigned int b2 = bb + stride;
      const long long id_a = load_ids(a, min(b2, batches - 1), total, lane);
      bbuf = load_batch(a, min(bb, batches - 1), id_b, total, lane);
      count_batch(h, ba, b0, total, a.chunks_per_plane, copy);
      if (bb >= batches) break;
      const unsigned int b3 = b2 + stride;
      id_b = load_ids(a, min(b3, batches - 1), total, lane);
      ba = load_batch(a, min(b2, batches - 1), id_a, total, lane);
      count_batch(h, bbuf, bb, total, a.chunks_per_plane, copy);
      if (b2 >= batches) break;
      b0 = b2;
      bb = b3;
    }
  }
  write_partial(h, a.partial);
}

// Any layout: one word per thread, grid-stride.
__global__ __launch_bounds__(kThreads) void exponent_hist_generic(HistArgs a) {
  __shared__ unsigned int h[kHistWords];
  const unsigned int lane = threadIdx.x & (kWave - 1);
  zero_hist(h);
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
    add_word(h, plane, w, lane % kCopies);
  }
  write_partial(h, a.partial);
}

// Sums the partials into 64-bit counts. Workgroup w owns bins [16w, 16w + 16); its
// threads split the groups into 16 slices (each row of 16 bins is one 64-byte
// segment) and keep sixteen loads in flight (one round for a grid of 256 partials:
// Llama-3-8B call 28.5 -> 28.1 us against two rounds of eight), then add the slices
// in LDS.
constexpr unsigned int kReduceBins = 16;
constexpr unsigned int kReduceSlices = kThreads / kReduceBins;

__global__ __launch_bounds__(kThreads) void exponent_hist_reduce(const unsigned int* partial,
                                                                 unsigned int groups,
                                                                 unsigned long long* counts) {
  __shared__ unsigned long long s_sum[kThreads];
  const unsigned int bin = blockIdx.x * kReduceBins + threadIdx.x % kReduceBins;
  const unsigned int slice = threadIdx.x / kReduceBins;
  unsigned long long s = 0;
  unsigned int g = slice;
  for (; g + 15 * kReduceSlices < groups; g += 16 * kReduceSlices) {
    unsigned int v[16];
#pragma unroll
    for (int k = 0; k < 16; ++k)
      v[k] = partial[(unsigned long long)(g + k * kReduceSlices) * 2 * kBins + bin];
#pragma unroll
    for (int k = 0; k < 16; ++k) s += v[k];
  }
  for (; g < groups; g += kReduceSlices) s += partial[(unsigned long long)g * 2 * kBins + bin];
  s_sum[threadIdx.x] = s;
  __syncthreads();
  if (slice == 0) {
    for (unsigned int j = 1; j < kReduceSlices; ++j) s += s_sum[j * kReduceBins + threadIdx.x];
    counts[bin] = s;
  }
}

// Compute units of the current device, cached per device.
unsigned long long device_cus() {
  static std::mutex mu;
  static unsigned long long cached[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  std::lock_guard<std::mutex> lock(mu);
  if (cached[dev] == 0) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        cus <= 0)
      cus = 256;
    cached[dev] = (unsigned long long)cus;
  }
  return cached[dev];
}

unsigned int partial_groups(unsigned long long block_count, unsigned long long block_words,
                            bool chunked) {
  const unsigned long long words = 2 * block_count * block_words;
  unsigned long long g;
  if (chunked) {
    // about 32 chunks per wave (per-layer call, Llama-3-8B, four-chunk batches:
    // 4 batches per wave 30.1 us, 8 28.2, 16 42.4 with too few workgroups to fill
    // the GPU; two-chunk batches: 16 per wave 26.3 us, 8 27.5), rounded to
    // whole rounds of one workgroup per CU (Llama-3-70B TP8 layer: 381 workgroups
    // 48.9 us, 256 40.4 us, 512 41.8 us); a small layer still spreads over up to
    // 64 workgroups, one batch per wave
    const unsigned long long batches = (words / kChunk + kBatch - 1) / kBatch;
    const unsigned long long waves = kHistThreads / kWave;
    g = (batches + kBatchesPerWave * waves - 1) / (kBatchesPerWave * waves);
    const unsigned long long cus = device_cus();
    if (2 * g >= cus) g = std::max(1ull, (g + cus / 2) / cus) * cus;
    const unsigned long long spread = (batches + waves - 1) / waves;
    const unsigned long long floor_g = spread < 64 ? spread : 64;
    if (g < floor_g) g = floor_g;
  } else {
    g = (words + (unsigned long long)kThreads * 64 - 1) / ((unsigned long long)kThreads * 64);
  }
  // a group's share stays within its 16-bit counters (the caller declines layers
  // too large for kMaxPartials groups)
  const unsigned long long need = (words + kMaxWordsPerGroup / 2 - 1) / (kMaxWordsPerGroup / 2);
  if (g < need) g = need;
  g = g > kMaxPartials ? kMaxPartials : (g < 1 ? 1 : g);
  return (unsigned int)g;
}

bool chunk_layout(unsigned long long kv_ptr, unsigned long long plane_stride,
                  unsigned long long block_stride, unsigned long long block_words,
                  unsigned long long block_count) {
  return block_words % kChunk == 0 && kv_ptr % 16 == 0 && plane_stride % 8 == 0 &&
         block_stride % 8 == 0 && 2 * block_count * (block_words / kChunk) < (1ull << 31);
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
  // a workgroup's share of the words must fit its 16-bit counters (every lane
  // counts at most one word in 64 of the group's words)
  if ((2 * block_count * block_words + kMaxPartials - 1) / kMaxPartials > kMaxWordsPerGroup / 2)
    return 0;
  const bool chunked = chunk_layout(kv_ptr, plane_stride, block_stride, block_words, block_count);
  HistArgs a{};
  a.kv = reinterpret_cast<const uint16_t*>(kv_ptr);
  a.ids = reinterpret_cast<const long long*>(block_ids_ptr);
  a.partial = reinterpret_cast<unsigned int*>(workspace_ptr);
  a.plane_stride = plane_stride;
  a.block_stride = block_stride;
  a.block_words = block_words;
  a.block_count = block_count;
  if (chunked) {
    a.chunks_per_plane = (unsigned int)(block_count * block_words / kChunk);
    a.chunks_per_block = (unsigned int)(block_words / kChunk);
    a.cpb_magic = make_divider(a.chunks_per_block).m;
  }
  const unsigned int groups = partial_groups(block_count, block_words, chunked);
  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_ptr);
  if (chunked)
    hipLaunchKernelGGL(exponent_hist_partial, dim3(groups), dim3(kHistThreads), 0, stream, a);
  else
    hipLaunchKernelGGL(exponent_hist_generic, dim3(groups), dim3(kThreads), 0, stream, a);
  hipError_t st = hipGetLastError();
  if (st != hipSuccess) return fail("exponent_hist_partial", st);
  hipLaunchKernelGGL(exponent_hist_reduce, dim3(2 * kBins / kReduceBins), dim3(kThreads), 0, stream,
                     a.partial, groups, reinterpret_cast<unsigned long long*>(counts_ptr));
  st = hipGetLastError();
  if (st != hipSuccess) return fail("exponent_hist_reduce", st);
  return (long long)(2 * block_count * block_words);
}
