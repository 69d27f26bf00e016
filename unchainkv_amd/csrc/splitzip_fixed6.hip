// Palette codecs fixed6 (mode 3) and fixed5 (mode 4) for bf16 KV cache, gfx950.
// They are the Top-16 overflow fallback of the connector.
//
// Wire format (native/unchain_kv/kvq_splitzip_cuda.cu:57-111, 292-333):
//   fixed6: [3][64-byte palette of high bytes][n low bytes][ceil(n/4) x 3 code bytes]
//   fixed5: [4][32-byte palette][n low bytes][ceil(n/8) x 5 code bytes]
// A group's codes are packed little-endian, first word in the low bits. With more
// distinct high bytes than palette entries only byte 0 is written, as 255.
//
// The palette is the set of distinct high bytes in ascending order, unused entries
// zeroed (the reference builds it first-come with atomicCAS, so its order varies
// from run to run; every order decodes to the same words).
//
// Kernels (one payload or every request of a paged layer per launch):
//   palette_presence_tile / _generic   256-bit presence mask of the high bytes, one
//       mask per 4096-word tile (or per workgroup of a grid-stride pass)
//   palette_reduce                     per payload: OR of its masks -> ascending
//       palette, rank table and distinct count (PaletteInfo in the workspace)
//   palette_encode_tile / _generic     header + palette, low bytes, packed codes
//   palette_decode_tile / _generic     decode + scatter (no-op unless byte 0 is the
//       format's mode byte)
// The tile kernels take block words a multiple of 1024 and a payload at any byte
// address (global memory takes unaligned vector accesses): waves own 1024 words of
// one block, lanes two 8-word runs, and the packed codes of a tile are staged in
// LDS so they move as whole dwords.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <vector>

#include "splitzip_common.h"

namespace unchainkv {
namespace {

template <int kBits>
struct Palette {
  static constexpr int kLimit = kBits == 6 ? 64 : 32;   // palette entries
  static constexpr int kHeader = 1 + kLimit;            // mode byte + palette
  static constexpr unsigned int kMode = kBits == 6 ? 3 : 4;
  static constexpr int kGroup = kBits == 6 ? 4 : 8;     // words per packed group
  static constexpr int kGroupBytes = kBits == 6 ? 3 : 5;
  static constexpr int kRunBytes = kBits;               // code bytes of 8 words
};

inline unsigned long long palette_encoded_size(unsigned long long n, int bits) {
  return bits == 6 ? 65 + n + ((n + 3) / 4) * 3 : 33 + n + ((n + 7) / 8) * 5;
}

constexpr unsigned int kGenericGroups = 64;  // workgroups per payload, generic kernels

// ---------------------------------------------------------------------------
// presence

// LDS byte map of the high bytes seen by a workgroup -> 8 dwords at out.
__device__ __forceinline__ void presence_flush(unsigned char* s_seen, unsigned int* out) {
  __syncthreads();
  const unsigned int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid >> 6;
  const unsigned long long bits = __ballot(s_seen[tid] != 0);  // high bytes 64w .. 64w+63
  if (lane == 0) {
    out[2 * wave] = (unsigned int)bits;
    out[2 * wave + 1] = (unsigned int)(bits >> 32);
  }
}

__device__ __forceinline__ void seen_clear(unsigned char* s_seen) {
  if (threadIdx.x < 64) reinterpret_cast<unsigned int*>(s_seen)[threadIdx.x] = 0;
  __syncthreads();
}

template <bool kIds>
__global__ __launch_bounds__(kThreads) void palette_presence_tile(LaunchArgs a, EncodeGeom geo,
                                                                  unsigned int* masks) {
  __shared__ unsigned char s_seen[256];
  const unsigned int lane = threadIdx.x & (kWave - 1);
  const unsigned int wave = uniform(threadIdx.x >> 6);
  const unsigned int tile = group_index();
  const PlaneTile t = plane_tile<kTileShift>(a, tile);
  const unsigned int in_plane = t.in_plane0 + wave * 1024;
  const bool active = wave * 1024 < t.words;
  u32x4 v0 = {0, 0, 0, 0}, v1 = {0, 0, 0, 0};
  if (active) {
    const uint16_t* src = a.kv + wave_source<kIds>(a, t, geo, in_plane);
    v0 = load_stream16(src + 8 * lane);
    v1 = load_stream16(src + 512 + 8 * lane);
  }
  seen_clear(s_seen);
  if (active) {
    const uint32_t x[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      s_seen[(x[k] >> 8) & 0xFF] = 1;
      s_seen[x[k] >> 24] = 1;
    }
  }
  presence_flush(s_seen, masks + (unsigned long long)tile * 8);
}

// Grid-stride presence pass over any geometry: grid = payload_count x groups.
__global__ __launch_bounds__(kThreads) void palette_presence_generic(LaunchArgs a,
                                                                     unsigned int groups,
                                                                     unsigned int* masks) {
  __shared__ unsigned char s_seen[256];
  const unsigned int r = blockIdx.x / groups, g = blockIdx.x % groups;
  const PayloadDesc d = a.p[r];
  const unsigned long long n = payload_words(a, d);
  seen_clear(s_seen);
  for (unsigned long long i = (unsigned long long)g * kThreads + threadIdx.x; i < n;
       i += (unsigned long long)groups * kThreads)
    s_seen[a.kv[word_offset(a, d, i)] >> 8] = 1;
  presence_flush(s_seen, masks + (unsigned long long)blockIdx.x * 8);
}

// Per payload: OR of masks [first, first + count) -> PaletteInfo. Masks of payload
// r start at mask_begin (one mask per tile: the presence tile kernel's, or the
// Top-16 tile kernel's) or r * groups (generic masks).
template <int kBits>
__global__ __launch_bounds__(kThreads) void palette_reduce(LaunchArgs a, unsigned int groups,
                                                           const unsigned int* masks,
                                                           PaletteInfo* info) {
  __shared__ unsigned int s_mask[8];
  const unsigned int r = blockIdx.x;
  const PayloadDesc d = a.p[r];
  const unsigned long long n = payload_words(a, d);
  const unsigned long long first = groups ? (unsigned long long)r * groups : d.mask_begin;
  const unsigned long long count = groups ? groups : payload_tiles(a, n);
  palette_info_from_masks(masks + first * 8, count, info[r], s_mask);
}

// ---------------------------------------------------------------------------
// encode

// Header and palette of a payload (from its info); 255 alone on overflow.
template <int kBits>
__device__ __forceinline__ void write_palette_header(unsigned char* payload,
                                                     const PaletteInfo& info) {
  using P = Palette<kBits>;
  const unsigned int tid = threadIdx.x;
  if (info.distinct > (unsigned int)P::kLimit) {
    if (tid == 0) payload[0] = 255;
    return;
  }
  if (tid == 0) payload[0] = (unsigned char)P::kMode;
  if (tid < (unsigned int)P::kLimit) payload[1 + tid] = info.palette[tid];
}

// Codes of one 8-word run (4 dwords of 2 words) packed little-endian, kBits each.
template <int kBits>
__device__ __forceinline__ unsigned long long pack_run(const uint32_t* x, const unsigned char* rank) {
  constexpr unsigned int kMask = (1u << kBits) - 1u;
  unsigned long long bits = 0;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    bits |= (unsigned long long)(rank[(x[k] >> 8) & 0xFF] & kMask) << (kBits * (2 * k));
    bits |= (unsigned long long)(rank[x[k] >> 24] & kMask) << (kBits * (2 * k + 1));
  }
  return bits;
}

// Low bytes of an 8-word run: bytes 0 and 2 of each dword.
__device__ __forceinline__ u32x2 low_run(const uint32_t* x) {
  return u32x2{__builtin_amdgcn_perm(x[1], x[0], 0x06040200u),
               __builtin_amdgcn_perm(x[3], x[2], 0x06040200u)};
}

// Writes kBits code bytes at LDS byte offset `at`.
template <int kBits>
__device__ __forceinline__ void stage_run(unsigned char* s, unsigned int at,
                                          unsigned long long bits) {
  if (kBits == 6) {  // at is even
#pragma unroll
    for (int k = 0; k < 3; ++k)
      *reinterpret_cast<uint16_t*>(s + at + 2 * k) = (uint16_t)(bits >> (16 * k));
  } else {
#pragma unroll
    for (int k = 0; k < kBits; ++k) s[at + k] = (unsigned char)(bits >> (8 * k));
  }
}

template <int kBits>
__device__ __forceinline__ unsigned long long unstage_run(const unsigned char* s, unsigned int at) {
  unsigned long long bits = 0;
  if (kBits == 6) {
#pragma unroll
    for (int k = 0; k < 3; ++k)
      bits |= (unsigned long long)*reinterpret_cast<const uint16_t*>(s + at + 2 * k) << (16 * k);
  } else {
#pragma unroll
    for (int k = 0; k < kBits; ++k) bits |= (unsigned long long)s[at + k] << (8 * k);
  }
  return bits;
}

// kIndexed: payload r's palette is info[a.p[r].mask_begin] (palettes computed by a
// Top-16 probe encode for a larger batch), else info[r].
template <bool kIds, int kBits, bool kIndexed = false>
__global__ __launch_bounds__(kThreads) void palette_encode_tile(LaunchArgs a, EncodeGeom geo,
                                                                const PaletteInfo* info) {
  using P = Palette<kBits>;
  constexpr unsigned int kWaveCodeBytes = 128 * kBits;  // 1024 words
  __shared__ uint32_t s_rank[64];
  __shared__ __align__(16) uint32_t s_code[(kThreads / kWave) * kWaveCodeBytes / 4];
  const unsigned int tid = threadIdx.x;
  const unsigned int lane = tid & (kWave - 1);
  const unsigned int wave = uniform(tid >> 6);
  const PlaneTile t = plane_tile<kTileShift>(a, group_index());
  const PaletteInfo& pi = info[kIndexed ? a.p[t.payload_index].mask_begin : t.payload_index];
  const unsigned int in_plane = t.in_plane0 + wave * 1024;
  const unsigned long long wstart = t.plane * (t.n >> 1) + in_plane;  // payload word
  const bool active = wave * 1024 < t.words;
  uint32_t x[8];
  if (active) {
    const uint16_t* src = a.kv + wave_source<kIds>(a, t, geo, in_plane);
    const u32x4 v0 = load_stream16(src + 8 * lane);
    const u32x4 v1 = load_stream16(src + 512 + 8 * lane);
    x[0] = v0.x; x[1] = v0.y; x[2] = v0.z; x[3] = v0.w;
    x[4] = v1.x; x[5] = v1.y; x[6] = v1.z; x[7] = v1.w;
  } else {
#pragma unroll
    for (int k = 0; k < 8; ++k) x[k] = 0;
  }
  if (tid < 64) s_rank[tid] = reinterpret_cast<const uint32_t*>(pi.rank)[tid];
  const unsigned int distinct = pi.distinct;
  if (t.local_tile == 0) write_palette_header<kBits>(t.payload, pi);
  // overflow: the reference writes byte 0 only (kvq_splitzip_cuda.cu:58-61)
  if (distinct > (unsigned int)P::kLimit) return;
  __syncthreads();  // s_rank ready
  const unsigned char* rank = reinterpret_cast<const unsigned char*>(s_rank);
  unsigned char* stage = reinterpret_cast<unsigned char*>(s_code) + wave * kWaveCodeBytes;
  if (active) {
    unsigned char* low = t.payload + P::kHeader + wstart;
    store_stream8(low + 8 * lane, low_run(x));
    store_stream8(low + 512 + 8 * lane, low_run(x + 4));
    stage_run<kBits>(stage, kBits * lane, pack_run<kBits>(x, rank));
    stage_run<kBits>(stage, kBits * (64 + lane), pack_run<kBits>(x + 4, rank));
  }
  __syncthreads();
  // the tile's code bytes as whole dwords (a tile's share is a multiple of 16
  // bytes, so no dword reaches into a neighbour tile's share)
  const unsigned long long tile_word = t.plane * (t.n >> 1) + t.in_plane0;
  uint32_t* codes = reinterpret_cast<uint32_t*>(t.payload + P::kHeader + t.n +
                                                tile_word * kBits / 8);
  const unsigned int dwords = t.words * kBits / 32;
  for (unsigned int k = tid; k < dwords; k += kThreads) store_stream4(codes + k, s_code[k]);
}

// Any geometry: grid = payload_count x kGenericGroups, grid-stride over groups.
template <int kBits>
__global__ __launch_bounds__(kThreads) void palette_encode_generic(LaunchArgs a,
                                                                   const PaletteInfo* info) {
  using P = Palette<kBits>;
  __shared__ unsigned char s_rank[256];
  const unsigned int r = blockIdx.x / kGenericGroups, g = blockIdx.x % kGenericGroups;
  const PayloadDesc d = a.p[r];
  const PaletteInfo& pi = info[r];
  const unsigned long long n = payload_words(a, d);
  unsigned char* payload = a.buf + d.buf_offset;
  if (g == 0) write_palette_header<kBits>(payload, pi);
  if (pi.distinct > (unsigned int)P::kLimit) return;
  s_rank[threadIdx.x] = pi.rank[threadIdx.x];
  __syncthreads();
  unsigned char* low = payload + P::kHeader;
  unsigned char* codes = low + n;
  const unsigned long long groups = (n + P::kGroup - 1) / P::kGroup;
  for (unsigned long long q = (unsigned long long)g * kThreads + threadIdx.x; q < groups;
       q += (unsigned long long)kGenericGroups * kThreads) {
    unsigned long long bits = 0;
#pragma unroll
    for (int k = 0; k < P::kGroup; ++k) {
      const unsigned long long i = q * P::kGroup + k;
      if (i >= n) break;
      const unsigned int w = a.kv[word_offset(a, d, i)];
      low[i] = (unsigned char)(w & 0xFF);
      bits |= (unsigned long long)(s_rank[w >> 8] & (P::kLimit - 1)) << (k * kBits);
    }
#pragma unroll
    for (int k = 0; k < P::kGroupBytes; ++k)
      codes[q * P::kGroupBytes + k] = (unsigned char)(bits >> (8 * k));
  }
}

// ---------------------------------------------------------------------------
// decode (DecodeFixed6 semantics, kvq_splitzip_cuda.cu:113-144)

// Decode + scatter of one tile; the destination's j-th block from block_of(t, j).
template <int kBits, typename BlockOf>
__device__ __forceinline__ void palette_decode_tile_body(const LaunchArgs& a,
                                                         const EncodeGeom& geo,
                                                         BlockOf block_of) {
  using P = Palette<kBits>;
  constexpr unsigned int kWaveCodeBytes = 128 * kBits;
  constexpr unsigned int kMask = (1u << kBits) - 1u;
  __shared__ unsigned char s_pal[64];
  __shared__ __align__(16) uint32_t s_code[(kThreads / kWave) * kWaveCodeBytes / 4];
  const unsigned int tid = threadIdx.x;
  const unsigned int lane = tid & (kWave - 1);
  const unsigned int wave = uniform(tid >> 6);
  const PlaneTile t = plane_tile<kTileShift>(a, group_index());
  const unsigned int mode = t.payload[0];
  const unsigned int in_plane = t.in_plane0 + wave * 1024;
  const unsigned long long wstart = t.plane * (t.n >> 1) + in_plane;
  const bool active = wave * 1024 < t.words;
  const unsigned long long tile_word = t.plane * (t.n >> 1) + t.in_plane0;
  const uint32_t* codes = reinterpret_cast<const uint32_t*>(t.payload + P::kHeader + t.n +
                                                            tile_word * kBits / 8);
  // the tile's code bytes, 16 at a time (a tile's share is a multiple of 16 bytes)
  const unsigned int quads = t.words * kBits / 128;
  for (unsigned int k = tid; k < quads; k += kThreads)
    reinterpret_cast<u32x4*>(s_code)[k] = load_stream16(codes + 4 * k);
  if (tid < (unsigned int)P::kLimit) s_pal[tid] = t.payload[1 + tid];
  u32x2 low_a = {0, 0}, low_b = {0, 0};
  uint16_t* dst = nullptr;
  if (active) {
    const unsigned char* low = t.payload + P::kHeader + wstart;
    low_a = load_stream8(low + 8 * lane);
    low_b = load_stream8(low + 512 + 8 * lane);
    dst = a.kv + wave_offset_by(a, t, geo, in_plane,
                                [&](unsigned int j) { return block_of(t, j); });
  }
  __syncthreads();
  if (mode != P::kMode || !active) return;  // the reference leaves other payloads untouched
  const unsigned char* stage = reinterpret_cast<const unsigned char*>(s_code) + wave * kWaveCodeBytes;
#pragma unroll
  for (int run = 0; run < 2; ++run) {
    const unsigned long long bits = unstage_run<kBits>(stage, kBits * (run * 64 + lane));
    const u32x2 low = run ? low_b : low_a;
    const uint32_t lw[2] = {low.x, low.y};
    uint32_t out[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const uint32_t lo = (lw[k >> 1] >> (16 * (k & 1))) & 0xFFFF;  // two low bytes
      const uint32_t h0 = s_pal[(bits >> (kBits * (2 * k))) & kMask];
      const uint32_t h1 = s_pal[(bits >> (kBits * (2 * k + 1))) & kMask];
      out[k] = (lo & 0xFF) | (h0 << 8) | ((lo >> 8) << 16) | (h1 << 24);
    }
    store_through16(dst + run * 512 + 8 * lane, u32x4{out[0], out[1], out[2], out[3]});
  }
}

template <bool kIds, int kBits>
__global__ __launch_bounds__(kThreads) void palette_decode_tile(LaunchArgs a, EncodeGeom geo) {
  palette_decode_tile_body<kBits>(a, geo, [&](const PlaneTile& t, unsigned int j) {
    return kIds ? (unsigned long long)t.ids[j] : a.block_start + j;
  });
}

// One request whose block table rides in the kernel arguments.
template <int kBits>
__global__ __launch_bounds__(kThreads) void palette_decode_tile_inline(LaunchArgs a,
                                                                       EncodeGeom geo,
                                                                       InlineBlocks table) {
  palette_decode_tile_body<kBits>(a, geo, [&](const PlaneTile&, unsigned int j) {
    return (unsigned long long)table.id[j];
  });
}

// Any geometry: grid = payload_count x kGenericGroups, grid-stride over words.
template <int kBits>
__global__ __launch_bounds__(kThreads) void palette_decode_generic(LaunchArgs a) {
  using P = Palette<kBits>;
  __shared__ unsigned char s_pal[64];
  const unsigned int r = blockIdx.x / kGenericGroups, g = blockIdx.x % kGenericGroups;
  const PayloadDesc d = a.p[r];
  const unsigned char* payload = a.buf + d.buf_offset;
  if (payload[0] != P::kMode) return;
  if (threadIdx.x < (unsigned int)P::kLimit) s_pal[threadIdx.x] = payload[1 + threadIdx.x];
  __syncthreads();
  const unsigned long long n = payload_words(a, d);
  const unsigned char* low = payload + P::kHeader;
  const unsigned char* codes = low + n;
  for (unsigned long long i = (unsigned long long)g * kThreads + threadIdx.x; i < n;
       i += (unsigned long long)kGenericGroups * kThreads) {
    const unsigned long long q = i / P::kGroup;
    unsigned long long packed = 0;
#pragma unroll
    for (int k = 0; k < P::kGroupBytes; ++k)
      packed |= (unsigned long long)codes[q * P::kGroupBytes + k] << (8 * k);
    const unsigned int code = (packed >> ((i % P::kGroup) * kBits)) & (P::kLimit - 1);
    a.kv[word_offset(a, d, i)] = (uint16_t)(((unsigned int)s_pal[code] << 8) | low[i]);
  }
}

// ---------------------------------------------------------------------------
// host side

long long check(const char* what) {
  const hipError_t st = hipGetLastError();
  return st == hipSuccess ? 0 : fail(what, st);
}

inline bool tile_geometry(unsigned long long kv_ptr, unsigned long long plane_stride,
                          unsigned long long block_stride, unsigned long long block_words,
                          unsigned long long max_plane_words) {
  return block_words % 1024 == 0 && kv_ptr % 16 == 0 && plane_stride % 8 == 0 &&
         block_stride % 8 == 0 && max_plane_words < (1ull << 31);
}

// A payload of n words suits the tile kernels at any byte address when its
// sections are whole multiples of 16 bytes.
inline bool palette_sections(unsigned long long n) { return n % 16 == 0; }

unsigned int tiles_of(unsigned long long n) {
  return 2u * (unsigned int)(((n >> 1) + kTileWords - 1) >> kTileShift);
}

// masks_given: `masks` already holds one mask per tile of every payload (from the
// Top-16 encode), at each payload's mask_begin; the presence pass is skipped.
template <int kBits>
long long launch_palette_encode(LaunchArgs& a, const EncodeGeom& g, bool tiles,
                                unsigned int presence_groups, PaletteInfo* info,
                                unsigned int* masks, bool masks_given, hipStream_t stream) {
  const dim3 block(kThreads);
  if (masks_given) {
    presence_groups = 0;
  } else if (tiles) {
    if (a.ids)
      hipLaunchKernelGGL(palette_presence_tile<true>, dim3(a.total_tiles), block, 0, stream, a, g,
                         masks);
    else
      hipLaunchKernelGGL(palette_presence_tile<false>, dim3(a.total_tiles), block, 0, stream, a,
                         g, masks);
  } else {
    hipLaunchKernelGGL(palette_presence_generic, dim3(a.payload_count * presence_groups), block, 0,
                       stream, a, presence_groups, masks);
  }
  if (long long rc = check("palette_presence")) return rc;
  hipLaunchKernelGGL(palette_reduce<kBits>, dim3(a.payload_count), block, 0, stream, a,
                     tiles || masks_given ? 0u : presence_groups, masks, info);
  if (long long rc = check("palette_reduce")) return rc;
  if (tiles) {
    if (a.ids)
      hipLaunchKernelGGL((palette_encode_tile<true, kBits>), dim3(a.total_tiles), block, 0, stream,
                         a, g, info);
    else
      hipLaunchKernelGGL((palette_encode_tile<false, kBits>), dim3(a.total_tiles), block, 0,
                         stream, a, g, info);
  } else {
    hipLaunchKernelGGL(palette_encode_generic<kBits>, dim3(a.payload_count * kGenericGroups),
                       block, 0, stream, a, info);
  }
  return check("palette_encode");
}

template <int kBits>
long long launch_palette_decode(LaunchArgs& a, const EncodeGeom& g, bool tiles,
                                hipStream_t stream, const InlineBlocks* table) {
  const dim3 block(kThreads);
  if (tiles) {
    if (table)
      hipLaunchKernelGGL(palette_decode_tile_inline<kBits>, dim3(a.total_tiles), block, 0, stream,
                         a, g, *table);
    else if (a.ids)
      hipLaunchKernelGGL((palette_decode_tile<true, kBits>), dim3(a.total_tiles), block, 0, stream,
                         a, g);
    else
      hipLaunchKernelGGL((palette_decode_tile<false, kBits>), dim3(a.total_tiles), block, 0,
                         stream, a, g);
  } else {
    hipLaunchKernelGGL(palette_decode_generic<kBits>, dim3(a.payload_count * kGenericGroups),
                       block, 0, stream, a);
  }
  return check("palette_decode");
}

// Encodes with the palettes a Top-16 probe encode computed: payload r's is
// info[a.p[r].mask_begin]; the presence and reduce passes are skipped (tile
// geometry only).
template <int kBits>
long long launch_palette_encode_info(LaunchArgs& a, const EncodeGeom& g, const PaletteInfo* info,
                                     hipStream_t stream) {
  const dim3 block(kThreads);
  if (a.ids)
    hipLaunchKernelGGL((palette_encode_tile<true, kBits, true>), dim3(a.total_tiles), block, 0,
                       stream, a, g, info);
  else
    hipLaunchKernelGGL((palette_encode_tile<false, kBits, true>), dim3(a.total_tiles), block, 0,
                       stream, a, g, info);
  return check("palette_encode (probe palettes)");
}

long long palette_encode(LaunchArgs& a, const EncodeGeom& g, bool tiles,
                         unsigned int presence_groups, PaletteInfo* info, unsigned int* masks,
                         hipStream_t stream, int bits, bool masks_given = false) {
  return bits == 6 ? launch_palette_encode<6>(a, g, tiles, presence_groups, info, masks,
                                              masks_given, stream)
                   : launch_palette_encode<5>(a, g, tiles, presence_groups, info, masks,
                                              masks_given, stream);
}

// `table`: one request's block table in the kernel arguments (tile kernels only).
long long palette_decode(LaunchArgs& a, const EncodeGeom& g, bool tiles, hipStream_t stream,
                         int bits, const InlineBlocks* table = nullptr) {
  return bits == 6 ? launch_palette_decode<6>(a, g, tiles, stream, table)
                   : launch_palette_decode<5>(a, g, tiles, stream, table);
}

// Fills a.p for payloads [first, first + count) of a batch (tiles of 4096 words
// per plane) and returns the tile total.
unsigned int fill_batch(LaunchArgs& a, const unsigned long long* block_offsets,
                        const unsigned long long* buf_offsets, unsigned long long first,
                        unsigned int count, unsigned long long block_words) {
  unsigned int tiles = 0;
  bool uniform_size = true;
  for (unsigned int k = 0; k < count; ++k) {
    const unsigned long long r = first + k;
    const unsigned long long nblk = block_offsets[r + 1] - block_offsets[r];
    a.p[k].buf_offset = buf_offsets[r];
    a.p[k].ids_offset = block_offsets[r];
    a.p[k].block_count = (unsigned int)nblk;
    a.p[k].tile_begin = tiles;
    a.p[k].mask_begin = tiles;
    tiles += tiles_of(2 * nblk * block_words);
    uniform_size = uniform_size && nblk == block_offsets[first + 1] - block_offsets[first];
  }
  a.payload_count = count;
  a.total_tiles = tiles;
  a.tiles_per_plane_mode = 1;
  a.tile_shift = kTileShift;
  a.uniform_tiles = uniform_size ? tiles / count : 0;
  // equal payloads whose block tables lie back to back from the start: block-table
  // offsets follow from the payload index (see plane_tile)
  const unsigned long long nblk0 = block_offsets[first + 1] - block_offsets[first];
  bool packed = uniform_size && block_offsets[first] == 0;
  for (unsigned int k = 0; k < count && packed; ++k)
    packed = block_offsets[first + k] == k * nblk0;
  a.uniform_blocks = packed ? (unsigned int)nblk0 : 0;
  return tiles;
}

unsigned long long batch_workspace_bytes(const unsigned long long* block_offsets,
                                         unsigned long long payload_count,
                                         unsigned long long block_words) {
  unsigned long long bytes = 0;
  for (unsigned long long first = 0; first < payload_count; first += kMaxPayloads) {
    const unsigned long long count = std::min<unsigned long long>(kMaxPayloads, payload_count - first);
    unsigned long long tiles = 0;
    for (unsigned long long r = first; r < first + count; ++r)
      tiles += tiles_of(2 * (block_offsets[r + 1] - block_offsets[r]) * block_words);
    const unsigned long long slots = std::max<unsigned long long>(tiles, count * kGenericGroups);
    bytes += count * sizeof(PaletteInfo) + slots * 32;
  }
  return bytes;
}

}  // namespace
}  // namespace unchainkv

using namespace unchainkv;

// kvq_splitzip_cuda.cu:292-333: same preconditions and return values. The palette
// state lives in the caller's buffer past the payload (the reference keeps an
// 8-byte counter/flag and a 256-entry map there, align4(encoded) + 1032 bytes); with
// room for one presence mask per tile the tile kernels run, else the generic ones.
extern "C" long long kvq_splitzip_bf16_encode_mode(unsigned long long src_ptr,
                                                   unsigned long long dst_ptr,
                                                   unsigned long long count,
                                                   unsigned long long capacity,
                                                   unsigned long long stream_ptr, int bits) {
  if (src_ptr == 0 || dst_ptr == 0 || count == 0) return 0;
  if (bits != 5 && bits != 6) return 0;
  const unsigned long long encoded = palette_encoded_size(count, bits);
  const unsigned long long scratch_offset = (encoded + 3) & ~3ULL;
  if (encoded >= count * 2 || scratch_offset + 256 * sizeof(int) + 2 * sizeof(int) > capacity)
    return 0;
  LaunchArgs a{};
  a.kv = reinterpret_cast<uint16_t*>(src_ptr);
  a.buf = reinterpret_cast<unsigned char*>(dst_ptr);
  a.linear_words = count;
  a.payload_count = 1;
  a.block_words = count / 2;
  a.plane_stride = count / 2;
  a.p[0].block_count = 1;
  a.tiles_per_plane_mode = 1;
  a.tile_shift = kTileShift;
  const unsigned long long ws = (dst_ptr + encoded + 15) / 16 * 16;  // 16-byte aligned scratch
  const unsigned long long room = dst_ptr + capacity > ws ? dst_ptr + capacity - ws : 0;
  const bool tiles = count % 2 == 0 &&
                     tile_geometry(src_ptr, count / 2, 0, count / 2, count / 2) &&
                     palette_sections(count) &&
                     room >= sizeof(PaletteInfo) + 32ull * tiles_of(count);
  a.total_tiles = tiles ? tiles_of(count) : 0;
  // Generic path: one presence mask per workgroup of the presence pass, as many as
  // the room holds (the reference's minimum capacity leaves room for 15).
  const unsigned int presence_groups = (unsigned int)std::min<unsigned long long>(
      kGenericGroups, room > sizeof(PaletteInfo) ? (room - sizeof(PaletteInfo)) / 32 : 0);
  if (!tiles && presence_groups == 0) return fail_msg("encode_mode: no room for the palette state");
  PaletteInfo* info = reinterpret_cast<PaletteInfo*>(ws);
  unsigned int* masks = reinterpret_cast<unsigned int*>(info + 1);
  const long long rc = palette_encode(a, make_geom(count / 2), tiles, presence_groups, info, masks,
                                      reinterpret_cast<hipStream_t>(stream_ptr), bits);
  return rc < 0 ? rc : (long long)encoded;
}

extern "C" long long kvq_splitzip_bf16_encode(unsigned long long src_ptr,
                                              unsigned long long dst_ptr,
                                              unsigned long long count,
                                              unsigned long long capacity,
                                              unsigned long long stream_ptr) {
  return kvq_splitzip_bf16_encode_mode(src_ptr, dst_ptr, count, capacity, stream_ptr, 6);
}

namespace {

long long decode_blocks(unsigned long long src_ptr, unsigned long long encoded_bytes,
                        unsigned long long dst_ptr, unsigned long long count_words,
                        unsigned long long block_count, unsigned long long block_words,
                        unsigned long long plane_stride, unsigned long long block_stride,
                        unsigned long long block_start, unsigned long long block_ids_ptr,
                        unsigned long long stream_ptr, int bits,
                        const long long* host_ids = nullptr) {
  // kvq_splitzip_cuda.cu:351-357
  if (src_ptr == 0 || dst_ptr == 0 || count_words == 0 || block_count == 0 || block_words == 0 ||
      count_words != 2 * block_count * block_words)
    return 0;
  if (encoded_bytes != palette_encoded_size(count_words, bits)) return 0;
  if (block_count > 0xFFFFFFFFULL || block_words > 0xFFFFFFFFULL)
    return fail_msg("decode_fixed6: block_count and block_words must fit in 32 bits");
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
  a.tiles_per_plane_mode = 1;
  a.tile_shift = kTileShift;
  const bool tiles = tile_geometry(dst_ptr, plane_stride, block_stride, block_words,
                                   count_words / 2) &&
                     palette_sections(count_words);
  a.total_tiles = tiles_of(count_words);
  // a host block table rides in the kernel arguments (tile kernels only)
  InlineBlocks table{};
  if (host_ids) {
    if (!tiles || block_count > kInlineBlocks) return 0;
    for (unsigned long long j = 0; j < block_count; ++j) {
      if (host_ids[j] < 0 || host_ids[j] > 0xFFFFFFFFll) return 0;
      table.id[j] = (unsigned int)host_ids[j];
    }
  }
  const long long rc = palette_decode(a, make_geom(block_words), tiles,
                                      reinterpret_cast<hipStream_t>(stream_ptr), bits,
                                      host_ids ? &table : nullptr);
  return rc < 0 ? rc : (long long)(count_words * sizeof(uint16_t));
}

}  // namespace

extern "C" long long kvq_splitzip_bf16_decode_fixed6_blocks(
    unsigned long long src_ptr, unsigned long long encoded_bytes, unsigned long long dst_ptr,
    unsigned long long count_words, unsigned long long block_count,
    unsigned long long block_words, unsigned long long plane_stride,
    unsigned long long block_stride, unsigned long long block_start,
    unsigned long long block_ids_ptr, unsigned long long stream_ptr) {
  return decode_blocks(src_ptr, encoded_bytes, dst_ptr, count_words, block_count, block_words,
                       plane_stride, block_stride, block_start, block_ids_ptr, stream_ptr, 6);
}

extern "C" long long kvq_splitzip_bf16_decode_fixed6(
    unsigned long long src_ptr, unsigned long long encoded_bytes, unsigned long long dst_ptr,
    unsigned long long count_words, unsigned long long block_count,
    unsigned long long block_words, unsigned long long plane_stride,
    unsigned long long block_stride, unsigned long long block_start,
    unsigned long long stream_ptr) {
  return decode_blocks(src_ptr, encoded_bytes, dst_ptr, count_words, block_count, block_words,
                       plane_stride, block_stride, block_start, 0, stream_ptr, 6);
}

extern "C" long long kvq_splitzip_bf16_decode_fixed6_host_blocks(
    unsigned long long src_ptr, unsigned long long encoded_bytes, unsigned long long dst_ptr,
    unsigned long long count_words, unsigned long long block_count,
    unsigned long long block_words, unsigned long long plane_stride,
    unsigned long long block_stride, const long long* host_block_ids,
    unsigned long long stream_ptr) {
  if (host_block_ids == nullptr) return 0;
  return decode_blocks(src_ptr, encoded_bytes, dst_ptr, count_words, block_count, block_words,
                       plane_stride, block_stride, 0, 0, stream_ptr, 6, host_block_ids);
}

// ---------------------------------------------------------------------------
// batched paged palette entry points (no counterpart in the reference)

extern "C" unsigned long long kvq_splitzip_palette_paged_workspace_bytes(
    unsigned long long block_words, const unsigned long long* block_offsets,
    unsigned long long payload_count) {
  if (block_offsets == nullptr || payload_count == 0) return 0;
  return batch_workspace_bytes(block_offsets, payload_count, block_words);
}

namespace {

long long encode_mode_paged_impl(
    unsigned long long kv_ptr, unsigned long long plane_stride, unsigned long long block_stride,
    unsigned long long block_words, unsigned long long block_ids_ptr,
    const unsigned long long* block_offsets, unsigned long long payload_count,
    unsigned long long out_ptr, const unsigned long long* out_offsets,
    unsigned long long out_capacity, unsigned long long workspace_ptr,
    unsigned long long workspace_bytes, unsigned long long stream_ptr, int bits,
    unsigned long long presence_ptr, const unsigned long long* presence_first,
    unsigned long long info_ptr = 0, const unsigned long long* info_first = nullptr,
    unsigned long long info_count = 0) {
  // info mode (palettes from a Top-16 probe encode): no workspace and no masks
  const bool with_info = info_ptr != 0;
  if (kv_ptr == 0 || block_ids_ptr == 0 || out_ptr == 0 || (workspace_ptr == 0 && !with_info) ||
      block_offsets == nullptr || out_offsets == nullptr || payload_count == 0 ||
      block_words == 0 || block_words > 0xFFFFFFFFULL || (bits != 5 && bits != 6) ||
      workspace_ptr % 16 != 0 || presence_ptr % 16 != 0 ||
      (presence_ptr != 0 && presence_first == nullptr) ||
      (with_info && (info_ptr % 16 != 0 || info_first == nullptr || presence_ptr != 0)))
    return 0;
  if (presence_ptr != 0)
    for (unsigned long long r = 0; r < payload_count; ++r)
      if (presence_first[r] > 0xFFFFFFFFULL) return 0;
  if (with_info)
    for (unsigned long long r = 0; r < payload_count; ++r)
      if (info_first[r] >= info_count) return 0;
  unsigned long long total = 0, max_plane = 0;
  bool sections = true;
  std::vector<std::pair<unsigned long long, unsigned long long>> spans;
  for (unsigned long long r = 0; r < payload_count; ++r) {
    if (block_offsets[r + 1] <= block_offsets[r]) return 0;
    const unsigned long long n = 2 * (block_offsets[r + 1] - block_offsets[r]) * block_words;
    const unsigned long long e = palette_encoded_size(n, bits);
    if (n > 0xFFFFFFFFULL || e >= 2 * n || out_offsets[r] + e > out_capacity) return 0;
    spans.emplace_back(out_offsets[r], out_offsets[r] + e);
    total += e;
    max_plane = std::max(max_plane, n >> 1);
    sections = sections && palette_sections(n);
  }
  std::sort(spans.begin(), spans.end());
  for (size_t k = 1; k < spans.size(); ++k)
    if (spans[k].first < spans[k - 1].second) return 0;  // overlapping payloads
  if (!with_info && batch_workspace_bytes(block_offsets, payload_count, block_words) >
                        workspace_bytes)
    return 0;
  const bool tiles =
      sections && tile_geometry(kv_ptr, plane_stride, block_stride, block_words, max_plane);
  if (with_info && !tiles) return 0;  // the probe palettes come with the tile geometry
  const EncodeGeom g = make_geom(block_words);
  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_ptr);
  unsigned char* ws = reinterpret_cast<unsigned char*>(workspace_ptr);
  for (unsigned long long first = 0; first < payload_count; first += kMaxPayloads) {
    LaunchArgs a{};
    a.kv = reinterpret_cast<uint16_t*>(kv_ptr);
    a.ids = reinterpret_cast<const long long*>(block_ids_ptr);
    a.buf = reinterpret_cast<unsigned char*>(out_ptr);
    a.plane_stride = plane_stride;
    a.block_stride = block_stride;
    a.block_words = block_words;
    const unsigned int count =
        (unsigned int)std::min<unsigned long long>(kMaxPayloads, payload_count - first);
    fill_batch(a, block_offsets, out_offsets, first, count, block_words);
    if (with_info) {
      for (unsigned int k = 0; k < count; ++k) a.p[k].mask_begin = (unsigned int)info_first[first + k];
      const PaletteInfo* probe = reinterpret_cast<const PaletteInfo*>(info_ptr);
      const long long rc = bits == 6 ? launch_palette_encode_info<6>(a, g, probe, stream)
                                     : launch_palette_encode_info<5>(a, g, probe, stream);
      if (rc < 0) return rc;
      continue;
    }
    PaletteInfo* info = reinterpret_cast<PaletteInfo*>(ws);
    unsigned int* masks = reinterpret_cast<unsigned int*>(info + count);
    if (presence_ptr != 0) {
      masks = reinterpret_cast<unsigned int*>(presence_ptr);
      for (unsigned int k = 0; k < count; ++k) a.p[k].mask_begin = (unsigned int)presence_first[first + k];
    }
    const long long rc =
        palette_encode(a, g, tiles, kGenericGroups, info, masks, stream, bits, presence_ptr != 0);
    if (rc < 0) return rc;
    ws += count * sizeof(PaletteInfo) +
          32 * std::max<unsigned long long>(a.total_tiles, (unsigned long long)count * kGenericGroups);
  }
  return (long long)total;
}

}  // namespace

extern "C" long long kvq_splitzip_bf16_encode_mode_paged(
    unsigned long long kv_ptr, unsigned long long plane_stride, unsigned long long block_stride,
    unsigned long long block_words, unsigned long long block_ids_ptr,
    const unsigned long long* block_offsets, unsigned long long payload_count,
    unsigned long long out_ptr, const unsigned long long* out_offsets,
    unsigned long long out_capacity, unsigned long long workspace_ptr,
    unsigned long long workspace_bytes, unsigned long long stream_ptr, int bits) {
  return encode_mode_paged_impl(kv_ptr, plane_stride, block_stride, block_words, block_ids_ptr,
                                block_offsets, payload_count, out_ptr, out_offsets, out_capacity,
                                workspace_ptr, workspace_bytes, stream_ptr, bits, 0, nullptr);
}

extern "C" long long kvq_splitzip_bf16_encode_mode_paged_presence(
    unsigned long long kv_ptr, unsigned long long plane_stride, unsigned long long block_stride,
    unsigned long long block_words, unsigned long long block_ids_ptr,
    const unsigned long long* block_offsets, unsigned long long payload_count,
    unsigned long long out_ptr, const unsigned long long* out_offsets,
    unsigned long long out_capacity, unsigned long long workspace_ptr,
    unsigned long long workspace_bytes, unsigned long long presence_ptr,
    const unsigned long long* presence_first, unsigned long long stream_ptr, int bits) {
  if (presence_ptr == 0) return 0;
  return encode_mode_paged_impl(kv_ptr, plane_stride, block_stride, block_words, block_ids_ptr,
                                block_offsets, payload_count, out_ptr, out_offsets, out_capacity,
                                workspace_ptr, workspace_bytes, stream_ptr, bits, presence_ptr,
                                presence_first);
}

extern "C" long long kvq_splitzip_bf16_encode_mode_paged_info(
    unsigned long long kv_ptr, unsigned long long plane_stride, unsigned long long block_stride,
    unsigned long long block_words, unsigned long long block_ids_ptr,
    const unsigned long long* block_offsets, unsigned long long payload_count,
    unsigned long long out_ptr, const unsigned long long* out_offsets,
    unsigned long long out_capacity, unsigned long long info_ptr,
    const unsigned long long* info_first, unsigned long long info_count,
    unsigned long long stream_ptr, int bits) {
  if (info_ptr == 0) return 0;
  return encode_mode_paged_impl(kv_ptr, plane_stride, block_stride, block_words, block_ids_ptr,
                                block_offsets, payload_count, out_ptr, out_offsets, out_capacity,
                                0, 0, stream_ptr, bits, 0, nullptr, info_ptr, info_first,
                                info_count);
}

extern "C" long long kvq_splitzip_bf16_decode_mode_paged(
    unsigned long long src_ptr, const unsigned long long* src_offsets,
    const unsigned long long* encoded_bytes, unsigned long long payload_count,
    unsigned long long kv_ptr, unsigned long long plane_stride, unsigned long long block_stride,
    unsigned long long block_words, unsigned long long block_ids_ptr,
    const unsigned long long* block_offsets, unsigned long long stream_ptr, int bits) {
  if (src_ptr == 0 || kv_ptr == 0 || block_ids_ptr == 0 || src_offsets == nullptr ||
      encoded_bytes == nullptr || block_offsets == nullptr || payload_count == 0 ||
      block_words == 0 || block_words > 0xFFFFFFFFULL || (bits != 5 && bits != 6))
    return 0;
  unsigned long long total = 0, max_plane = 0;
  bool sections = true;
  for (unsigned long long r = 0; r < payload_count; ++r) {
    if (block_offsets[r + 1] <= block_offsets[r]) return 0;
    const unsigned long long n = 2 * (block_offsets[r + 1] - block_offsets[r]) * block_words;
    if (encoded_bytes[r] != palette_encoded_size(n, bits) || (n >> 1) > 0xFFFFFFFFULL) return 0;
    total += 2 * n;
    max_plane = std::max(max_plane, n >> 1);
    sections = sections && palette_sections(n);
  }
  const bool tiles =
      sections && tile_geometry(kv_ptr, plane_stride, block_stride, block_words, max_plane);
  const EncodeGeom g = make_geom(block_words);
  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_ptr);
  for (unsigned long long first = 0; first < payload_count; first += kMaxPayloads) {
    LaunchArgs a{};
    a.kv = reinterpret_cast<uint16_t*>(kv_ptr);
    a.ids = reinterpret_cast<const long long*>(block_ids_ptr);
    a.buf = reinterpret_cast<unsigned char*>(src_ptr);
    a.plane_stride = plane_stride;
    a.block_stride = block_stride;
    a.block_words = block_words;
    const unsigned int count =
        (unsigned int)std::min<unsigned long long>(kMaxPayloads, payload_count - first);
    fill_batch(a, block_offsets, src_offsets, first, count, block_words);
    const long long rc = palette_decode(a, g, tiles, stream, bits);
    if (rc < 0) return rc;
  }
  return (long long)total;
}
