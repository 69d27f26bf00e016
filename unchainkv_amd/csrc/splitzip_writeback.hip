// Codec writeback for gfx950: moves encoded Top-16 payloads out of the codec
// buffer into the sending request's own KV blocks, so the codec buffer can be
// reused while the payload is still being copied to the host.
//
// Reference behaviour (src/unchain_kv/vllm_connector.py:3460-3563, segments
// :3720-3738): for a request whose blocks form one contiguous run
// [start, start + count), the payload's first bytes fill the K-plane run
// kv[0, start:start+count] and the rest the V-plane run kv[1, start:start+count]
// (two torch copies per request); the host copy is then taken from those runs.
// The reference keeps its gathered source tensor for the overflow fallback. This
// library gathers inside the encode kernel and has no such copy, so a payload
// whose mode byte is not 5 (an overflow, header 255) is not written: its blocks
// stay intact for the fixed6 re-encode, and the mode byte each payload had is
// reported in status[r] for the host to check.
//
// One launch moves up to 64 payloads. A workgroup moves 8 KiB of one payload,
// two 16-byte chunks per lane: for each, a lane reads its 16 source bytes with one
// load at their byte address (a payload starts 5 bytes before a 256-byte boundary;
// global memory takes unaligned accesses) and writes one aligned 16-byte store.
// Loads and stores keep the default cache policy: with nontemporal stores the
// Llama-3-8B layer's 102 MB took 41 us, with write-through stores 42 us, with
// plain stores 33 us (four chunks per lane: 35.6 us).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <utility>
#include <vector>

#include "splitzip_common.h"

namespace unchainkv {
namespace {

constexpr int kWbMaxPayloads = 64;
constexpr int kWbChunks = 2;                                // 16-byte chunks per lane
constexpr unsigned int kWbSpan = kThreads * 16;             // one chunk of every lane
constexpr unsigned int kWbGroupBytes = kWbSpan * kWbChunks;  // payload bytes per workgroup
constexpr unsigned int kModeTop16 = 5;

struct WbDesc {
  const unsigned char* src;  // first payload byte
  unsigned char* k_dst;      // first byte of the K-plane run
  unsigned char* v_dst;      // first byte of the V-plane run
  unsigned long long bytes;  // encoded bytes
  unsigned long long seg;    // bytes of one plane's run
  unsigned int group_begin;  // first workgroup of this payload within the launch
  unsigned int pad;
};

struct WbArgs {
  unsigned char* status;  // per payload of the launch: its mode byte
  unsigned int payload_count;
  unsigned int uniform_groups;  // workgroups of every payload when all are equal, else 0
  WbDesc p[kWbMaxPayloads];
};

static_assert(kWbMaxPayloads == 64, "one payload descriptor per lane");

__device__ __forceinline__ unsigned int find_wb_payload(const WbArgs& a, unsigned int group) {
  if (a.uniform_groups) return group / a.uniform_groups;
  if (a.payload_count <= 1) return 0;
  const unsigned int lane = __lane_id();
  const unsigned int begin = lane < a.payload_count ? a.p[lane].group_begin : 0xFFFFFFFFu;
  const unsigned long long starts = __ballot(begin <= group);
  return __builtin_amdgcn_readfirstlane((unsigned int)__popcll(starts) - 1u);
}

__device__ __forceinline__ unsigned char* wb_target(const WbDesc& d, unsigned long long j) {
  return j < d.seg ? d.k_dst + j : d.v_dst + (j - d.seg);
}

// 16 bytes at any byte address.
typedef unsigned int u32x4_a1 __attribute__((ext_vector_type(4), aligned(1)));

// kAligned: both runs start 16-byte aligned, a run holds a multiple of 16 bytes
// (a lane's 16 destination bytes never straddle the two runs) and every payload
// has at least 16 bytes. A lane moves chunks base + k * 4 KiB (k < 2) of its
// workgroup's 8 KiB: chunk 0 is loaded together with the mode byte, chunk 1 once
// the mode byte has shown a payload to move (an overflowed payload costs half of
// its bytes in reads, not all of them), and every load is issued before the first
// store.
template <bool kAligned>
__global__ __launch_bounds__(kThreads) void top16_writeback(WbArgs a) {
  const unsigned int g = group_index();
  const unsigned int r = find_wb_payload(a, g);
  const WbDesc d = a.p[r];
  const unsigned long long base =
      (unsigned long long)(g - d.group_begin) * kWbGroupBytes + threadIdx.x * 16u;
  // the mode byte is read per lane (through an index the compiler cannot prove
  // uniform) so that testing it does not wait for it before the data loads issue
  unsigned int zero;
  __asm__ volatile("v_mov_b32 %0, 0" : "=v"(zero));
  const unsigned int mode = d.src[zero];
  // Chunks that are not whole inside the payload (its last bytes, or past its end)
  // load the payload's first 16 bytes instead, which every payload of an aligned
  // launch holds: the loads need no branch and all issue together.
  u32x4 v[kWbChunks];
  auto load_chunk = [&](int k) {
    const unsigned long long c = base + (unsigned long long)k * kWbSpan;
    v[k] = *reinterpret_cast<const u32x4_a1*>(d.src + (c + 16 <= d.bytes ? c : 0));
  };
  if (kAligned) load_chunk(0);
  if (g == d.group_begin && threadIdx.x == 0) a.status[r] = (unsigned char)mode;
  if (mode != kModeTop16) return;
  if (kAligned) {
#pragma unroll
    for (int k = 1; k < kWbChunks; ++k) load_chunk(k);
  }
#pragma unroll
  for (int k = 0; k < kWbChunks; ++k) {
    const unsigned long long c = base + (unsigned long long)k * kWbSpan;
    if (c >= d.bytes) return;
    if (kAligned && c + 16 <= d.bytes) {
      *reinterpret_cast<u32x4*>(wb_target(d, c)) = v[k];
    } else {
      const unsigned long long stop = c + 16 < d.bytes ? c + 16 : d.bytes;
      for (unsigned long long j = c; j < stop; ++j) *wb_target(d, j) = d.src[j];
    }
  }
}

struct Interval {
  unsigned long long lo, hi;
};

bool overlaps_any(std::vector<Interval>& v) {
  std::sort(v.begin(), v.end(), [](const Interval& x, const Interval& y) { return x.lo < y.lo; });
  for (size_t i = 1; i < v.size(); ++i)
    if (v[i].lo < v[i - 1].hi) return true;
  return false;
}

}  // namespace
}  // namespace unchainkv

using namespace unchainkv;

// Moves payload r (payloads_ptr + payload_offsets[r], encoded_bytes[r] bytes) into
// the K-plane run then the V-plane run of blocks [run_starts[r], run_starts[r] +
// run_blocks[r]) of a paged bf16 layer (strides in words), for r < payload_count,
// if byte 0 of the payload is 5; status[r] (device u8) receives byte 0. Returns
// the bytes of all payloads, 0 on a failed precondition (a run that is not
// contiguous in memory, a payload longer than its two runs, runs that overlap
// each other or the payload buffer), -1 on a launch error.
extern "C" long long kvq_splitzip_top16_writeback_paged(
    unsigned long long payloads_ptr, const unsigned long long* payload_offsets,
    const unsigned long long* encoded_bytes, unsigned long long payload_count,
    unsigned long long kv_ptr, unsigned long long plane_stride, unsigned long long block_stride,
    unsigned long long block_words, const unsigned long long* run_starts,
    const unsigned long long* run_blocks, unsigned long long status_ptr,
    unsigned long long stream_ptr) {
  if (payloads_ptr == 0 || payload_offsets == nullptr || encoded_bytes == nullptr ||
      payload_count == 0 || kv_ptr == 0 || block_words == 0 || run_starts == nullptr ||
      run_blocks == nullptr || status_ptr == 0 || kv_ptr % 2 != 0)
    return 0;
  std::vector<Interval> runs;
  runs.reserve(2 * payload_count + 1);
  unsigned long long src_lo = ~0ull, src_hi = 0, total = 0, launch_groups = 0;
  for (unsigned long long r = 0; r < payload_count; ++r) {
    const unsigned long long count = run_blocks[r], bytes = encoded_bytes[r];
    if (count == 0 || bytes == 0 || (count > 1 && block_stride != block_words)) return 0;
    if (count > (~0ull >> 2) / block_words) return 0;
    const unsigned long long seg = 2 * count * block_words;
    if (bytes > 2 * seg) return 0;
    // a launch's work-items (64 payloads at most) are counted in 32 bits
    if (r % kWbMaxPayloads == 0) launch_groups = 0;
    launch_groups += (bytes + kWbGroupBytes - 1) / kWbGroupBytes;
    if (launch_groups > 0xFFFFFFFFull / kThreads) return 0;
    const unsigned long long k = kv_ptr + 2 * run_starts[r] * block_stride;
    const unsigned long long v = k + 2 * plane_stride;
    runs.push_back({k, k + seg});
    runs.push_back({v, v + seg});
    src_lo = std::min(src_lo, payloads_ptr + payload_offsets[r]);
    src_hi = std::max(src_hi, payloads_ptr + payload_offsets[r] + bytes);
    total += bytes;
  }
  runs.push_back({src_lo, src_hi});
  if (overlaps_any(runs)) return 0;

  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_ptr);
  for (unsigned long long first = 0; first < payload_count; first += kWbMaxPayloads) {
    const unsigned int n =
        (unsigned int)std::min<unsigned long long>(kWbMaxPayloads, payload_count - first);
    WbArgs a{};
    a.status = reinterpret_cast<unsigned char*>(status_ptr + first);
    a.payload_count = n;
    unsigned long long groups = 0, first_groups = 0;
    bool aligned = true, uniform = true;
    for (unsigned int i = 0; i < n; ++i) {
      const unsigned long long r = first + i;
      WbDesc& d = a.p[i];
      const unsigned long long k = kv_ptr + 2 * run_starts[r] * block_stride;
      d.src = reinterpret_cast<const unsigned char*>(payloads_ptr + payload_offsets[r]);
      d.k_dst = reinterpret_cast<unsigned char*>(k);
      d.v_dst = reinterpret_cast<unsigned char*>(k + 2 * plane_stride);
      d.bytes = encoded_bytes[r];
      d.seg = 2 * run_blocks[r] * block_words;
      d.group_begin = (unsigned int)groups;
      const unsigned long long own = (d.bytes + kWbGroupBytes - 1) / kWbGroupBytes;
      if (i == 0) first_groups = own;
      uniform = uniform && own == first_groups;
      groups += own;
      aligned = aligned && k % 16 == 0 && (k + 2 * plane_stride) % 16 == 0 &&
                d.seg % 16 == 0 && d.bytes >= 16;
    }
    a.uniform_groups = uniform ? (unsigned int)first_groups : 0u;
    if (aligned)
      hipLaunchKernelGGL(top16_writeback<true>, dim3((unsigned int)groups), dim3(kThreads), 0,
                         stream, a);
    else
      hipLaunchKernelGGL(top16_writeback<false>, dim3((unsigned int)groups), dim3(kThreads), 0,
                         stream, a);
    hipError_t st = hipGetLastError();
    if (st != hipSuccess) return fail("top16_writeback", st);
  }
  return (long long)total;
}
