// Top-16 palette codec for bf16 KV cache (payload mode 5), gfx950.
//
// Wire format of one payload of n bf16 words (n = 2 * blocks * block_words for a
// paged layer; K plane first, then V), identical to the reference's
// (native/unchain_kv/kvq_splitzip_cuda.cu:146-208):
//   [0]                 5, or 255 when the escapes overflow the capacity
//   [1..4]              u32 LE escape count, clamped to cap = ceil(n / 200)
//   [5, 5+n)            body: (w & 0x7F) | ((w >> 8) & 0x80)  (mantissa + sign)
//   [5+n, 5+n+n/2)      codes: 4-bit codebook index, even word in the low nibble
//   [.., +5*cap)        escapes: {u32 LE position, u8 exponent}, code 0 in codes
// The code of word i is tables[p * 256 + exponent(i)] with p = (i >= n / 2);
// 255 there means "escape". Escapes are emitted in ascending position order and
// unused slots are zeroed, which is one of the byte streams the reference
// encoder can produce (its order is set by a global atomicAdd) and makes the
// payload deterministic.
//
// Kernels (all launched on the caller's stream, no host synchronisation):
//   top16_encode_tile        block words a multiple of 1024, payload at any byte
//       address: gather through the block table + encode one 4096-word tile per
//       workgroup, one block per wave so addressing is scalar; escapes are
//       counted per tile and up to kStageSlots of them staged in the workspace.
//   top16_encode_lanes<fast, sequential>  any geometry: 16 consecutive words per
//       lane (stores realigned through neighbour-lane shuffles); or one workgroup
//       walking every tile in order.
//   top16_encode_finalize    per payload (8, 16 or 32 workgroups): scan tile counts,
//       place escapes in ascending order, write the header (the tile kernel
//       zeroes the escape slots of its span).
//   top16_decode_tile / top16_decode_lanes / top16_decode_generic
//       decode + scatter for the tile geometry, 16-word lanes, any geometry.
// Global memory takes unaligned vector accesses (the code object's unaligned
// access mode), so a payload's sections need no alignment: the reference
// connector's payloads start at a buffer's first byte, their body at byte 5.
//   top16_patch_escapes      apply escapes (any order) after decode.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "splitzip_common.h"

namespace unchainkv {

thread_local std::string g_last_error;

long long fail(const char* what, hipError_t status) {
  g_last_error = std::string(what) + ": " + hipGetErrorString(status);
  return -1;
}

long long fail_msg(const std::string& msg) {
  g_last_error = msg;
  return -1;
}

namespace {

// Finalize workgroups per payload: each scans every tile count and places the
// escapes of every kGroups-th tile; a thread holds kGroups counts per pass. Per
// Llama-3-8B layer call (2048 tiles per payload), encode: 8 groups 48.6 us, 16
// groups 48.1 us, 32 groups 48.4 us (the 1 % outlier encode: 135.9, 134.4, 133.0);
// the Llama-3.2-1B payload (256 tiles): 8 groups 8.4 us, 16 groups 8.9 us.
// payloads from this size take 16 finalize groups, smaller ones 8 (fewer, fuller
// workgroups: Llama-3-70B TP8 encode call 73.5 -> 72.9 us with 8 for its largest
// payloads of 2048 tiles)
constexpr unsigned int kFinLargeTiles = 4096;
constexpr unsigned int kFinFewTiles = 1024;
constexpr int kFinPresenceGroups = 32;
constexpr int kFinPreload = 8;                         // staged escapes loaded with the counts
// Dense tiles (more staged escapes than the preload) placed per wave pass by the
// finalize: 2 normally; 8 after a presence-mask encode, the variant for a layer
// that overflowed before (1 % outlier layer encode call 112.0 -> 108.7 us; with 8
// in every finalize the Llama-3-8B call lost 0.9 us to the larger kernel).
constexpr int kDenseItemsSparse = 2;
constexpr int kDenseItemsDense = 8;

__host__ __device__ inline unsigned long long escape_capacity(unsigned long long n) {
  return (n + 199) / 200;
}

__host__ __device__ inline unsigned long long encoded_size(unsigned long long n) {
  return 5 + n + (n + 1) / 2 + 5 * escape_capacity(n);
}

// A 4-byte type at any address: global memory takes unaligned dword accesses, so
// an entry is one dword store and one byte store instead of five byte stores.
typedef unsigned int u32_unaligned __attribute__((aligned(1)));

__device__ __forceinline__ void put_entry(unsigned char* entries, unsigned long long slot,
                                          unsigned int pos, unsigned int exponent) {
  unsigned char* e = entries + slot * 5;
  *reinterpret_cast<u32_unaligned*>(e) = pos;  // little-endian, as the format
  e[4] = (unsigned char)exponent;
}

__device__ __forceinline__ void write_header(unsigned char* payload, unsigned long long n,
                                             unsigned long long escapes) {
  unsigned long long cap = escape_capacity(n);
  unsigned long long count = escapes > cap ? cap : escapes;
  payload[0] = escapes > cap ? 255 : 5;
  payload[1] = (unsigned char)count;
  payload[2] = (unsigned char)(count >> 8);
  payload[3] = (unsigned char)(count >> 16);
  payload[4] = (unsigned char)(count >> 24);
}

// Workgroup-cooperative zeroing of [p, p + len).
__device__ void zero_fill(unsigned char* p, unsigned long long len) {
  const unsigned int tid = threadIdx.x;
  unsigned long long head = (16 - ((uintptr_t)p & 15)) & 15;
  if (head > len) head = len;
  if (tid < head) p[tid] = 0;
  unsigned char* q = p + head;
  unsigned long long rest = len - head;
  unsigned long long vecs = rest >> 4;
  for (unsigned long long k = tid; k < vecs; k += kThreads)
    reinterpret_cast<uint4*>(q)[k] = make_uint4(0, 0, 0, 0);
  unsigned long long tail = rest & 15;
  if (tid < tail) q[(vecs << 4) + tid] = 0;
}

// Exclusive scan of one value per thread across the workgroup; returns the
// exclusive prefix and sets total. Uses s_wave[4]; contains barriers.
__device__ __forceinline__ unsigned int block_exclusive_sum(unsigned int v, unsigned int* s_wave,
                                                            unsigned int& total) {
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x >> 6;
  unsigned int incl = wave_inclusive_sum(v);
  if (lane == kWave - 1) s_wave[wave] = incl;
  __syncthreads();
  unsigned int before = 0;
  total = 0;
#pragma unroll
  for (int k = 0; k < kThreads / kWave; ++k) {
    unsigned int t = s_wave[k];
    if (k < wave) before += t;
    total += t;
  }
  __syncthreads();
  return before + incl - v;
}


// Same for a 64-bit value holding up to four 16-bit counters (no carries: every
// counter stays below 2^16). Uses s_wave64[4]; contains barriers.
__device__ __forceinline__ unsigned long long block_exclusive_sum64(unsigned long long v,
                                                                    unsigned long long* s_wave64,
                                                                    unsigned long long& total) {
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x >> 6;
  unsigned long long incl = v;
#pragma unroll
  for (int d = 1; d < kWave; d <<= 1) {
    unsigned long long t = __shfl_up(incl, d, kWave);
    if (lane >= d) incl += t;
  }
  if (lane == kWave - 1) s_wave64[wave] = incl;
  __syncthreads();
  unsigned long long before = 0;
  total = 0;
#pragma unroll
  for (int k = 0; k < kThreads / kWave; ++k) {
    unsigned long long t = s_wave64[k];
    if (k < wave) before += t;
    total += t;
  }
  __syncthreads();
  return before + incl - v;
}

// ---------------------------------------------------------------------------
// misaligned stores/loads of per-lane byte runs

// Each active lane owns 16 bytes for [dst, dst + 16); the active lanes of a wave
// cover one contiguous range and share the misalignment s = dst & 15. Interior
// 16-byte aligned chunks are written whole (own tail + next lane's head);
// the wave's edges are written bytewise.
__device__ __forceinline__ void store16_run(unsigned char* dst, const uint32_t (&v)[4],
                                            bool active, bool first, bool last) {
  const uint32_t s = (uint32_t)((uintptr_t)dst & 15);
  if (s == 0) {
    if (active) *reinterpret_cast<uint4*>(dst) = make_uint4(v[0], v[1], v[2], v[3]);
    return;
  }
  uint32_t c[8];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    c[k] = v[k];
    c[k + 4] = shfl_next(v[k]);
  }
  if (!active) return;
  unsigned char* x = dst - s + 16;
  if (first) store_bytes(dst, v, 0, 16 - s);
  if (last) {
    store_bytes(x, v, 16 - s, s);
  } else {
    uint32_t o[4];
    window4(c, 16 - s, o);
    *reinterpret_cast<uint4*>(x) = make_uint4(o[0], o[1], o[2], o[3]);
  }
}

// Same for 8-byte runs.
__device__ __forceinline__ void store8_run(unsigned char* dst, const uint32_t (&v)[2],
                                           bool active, bool first, bool last) {
  const uint32_t s = (uint32_t)((uintptr_t)dst & 7);
  if (s == 0) {
    if (active) *reinterpret_cast<uint2*>(dst) = make_uint2(v[0], v[1]);
    return;
  }
  uint32_t c[4] = {v[0], v[1], shfl_next(v[0]), shfl_next(v[1])};
  if (!active) return;
  unsigned char* x = dst - s + 8;
  if (first) store_bytes(dst, v, 0, 8 - s);
  if (last) {
    store_bytes(x, v, 8 - s, s);
  } else {
    uint32_t o[2];
    window2(c, 8 - s, o);
    *reinterpret_cast<uint2*>(x) = make_uint2(o[0], o[1]);
  }
}

// Loads [src, src + 16) for each active lane (lanes contiguous, shared
// misalignment). Only aligned chunks that hold wanted bytes are read.
__device__ __forceinline__ void load16_run(const unsigned char* src, bool active, bool last,
                                           uint32_t (&o)[4]) {
  const uint32_t s = (uint32_t)((uintptr_t)src & 15);
  if (s == 0) {
    uint4 v = active ? *reinterpret_cast<const uint4*>(src) : make_uint4(0, 0, 0, 0);
    o[0] = v.x; o[1] = v.y; o[2] = v.z; o[3] = v.w;
    return;
  }
  const unsigned char* f = src - s;
  uint4 own = active ? *reinterpret_cast<const uint4*>(f) : make_uint4(0, 0, 0, 0);
  uint32_t c[8] = {own.x, own.y, own.z, own.w, 0, 0, 0, 0};
#pragma unroll
  for (int k = 0; k < 4; ++k) c[k + 4] = shfl_next(c[k]);
  if (active && last) {
    uint4 nx = *reinterpret_cast<const uint4*>(f + 16);
    c[4] = nx.x; c[5] = nx.y; c[6] = nx.z; c[7] = nx.w;
  }
  window4(c, s, o);
}

__device__ __forceinline__ void load8_run(const unsigned char* src, bool active, bool last,
                                          uint32_t (&o)[2]) {
  const uint32_t s = (uint32_t)((uintptr_t)src & 7);
  if (s == 0) {
    uint2 v = active ? *reinterpret_cast<const uint2*>(src) : make_uint2(0, 0);
    o[0] = v.x; o[1] = v.y;
    return;
  }
  const unsigned char* f = src - s;
  uint2 own = active ? *reinterpret_cast<const uint2*>(f) : make_uint2(0, 0);
  uint32_t c[4] = {own.x, own.y, 0, 0};
  c[2] = shfl_next(c[0]);
  c[3] = shfl_next(c[1]);
  if (active && last) {
    uint2 nx = *reinterpret_cast<const uint2*>(f + 8);
    c[2] = nx.x; c[3] = nx.y;
  }
  window2(c, s, o);
}

// ---------------------------------------------------------------------------
// encode

// Geometry of one tile of a launch (wave-uniform values).
struct TileInfo {
  unsigned long long n, half, start, end, ids_offset;
  unsigned char* payload;
  unsigned int plane;
  unsigned int local_tile;  // tile index within its payload
};

__device__ __forceinline__ TileInfo tile_info(const LaunchArgs& a, unsigned int tile) {
  TileInfo t;
  const unsigned int r = find_payload(a, tile);
  const PayloadDesc d = a.p[r];
  t.n = payload_words(a, d);
  t.half = t.n >> 1;
  t.local_tile = tile - d.tile_begin;
  tile_range(a, d, t.local_tile, t.n, t.start, t.end);
  t.plane = t.start >= t.half ? 1u : 0u;
  t.payload = a.buf + d.buf_offset;
  t.ids_offset = d.ids_offset;
  return t;
}

// Zeroes tile `local_tile`'s share of its payload's escape section; the finalize
// kernel then writes the used slots over it (workgroup-cooperative, no barrier).
__device__ __forceinline__ void zero_escape_share(unsigned char* payload, unsigned long long n,
                                                  unsigned int local_tile, unsigned int tiles) {
  const unsigned int len = (unsigned int)(5 * escape_capacity(n));  // < 2^30 for n < 2^32
  const unsigned int share = (len + tiles - 1) / tiles;
  const unsigned int lo = share * local_tile;
  if (lo >= len) return;
  const unsigned int hi = min(lo + share, len);
  zero_fill(payload + 5 + n + (n + 1) / 2 + lo, hi - lo);
}

// Element offset in the paged layer of payload word i (i inside plane t.plane).
__device__ __forceinline__ unsigned long long chunk_offset(const LaunchArgs& a, const TileInfo& t,
                                                           const EncodeGeom& geo,
                                                           unsigned long long i) {
  const unsigned int in_plane = (unsigned int)(i - t.plane * t.half);
  const unsigned int j = div_u32(in_plane, geo.bw_magic, geo.bw);
  const unsigned int within = in_plane - j * geo.bw;
  const unsigned long long blk =
      a.ids ? (unsigned long long)a.ids[t.ids_offset + j] : a.block_start + j;
  return t.plane * a.plane_stride + blk * a.block_stride + within;
}

// Fills s_tab[512] with code (0..15) or 0x10 for an escape, from the 544-byte table
// (a code byte other than 255 keeps its low nibble, as the reference's
// `(code & 0x0F)` does).
__device__ __forceinline__ void load_code_table(const unsigned char* tables, unsigned char* s_tab) {
  for (int k = threadIdx.x; k < 512; k += kThreads) {
    unsigned int t = tables[k];
    s_tab[k] = (unsigned char)(t == 255 ? 0x10 : (t & 0x0F));
  }
}

// Encodes the 16 words of one lane (packed 2 per dword) with the code table of one
// plane: 16 body bytes, 8 code bytes, and a 16-bit escape mask.
__device__ __forceinline__ void encode_lane(const uint32_t (&x)[8], const unsigned char* tab,
                                            uint32_t (&body)[4], uint32_t (&codes)[2],
                                            uint32_t& emask) {
  body[0] = body[1] = body[2] = body[3] = 0;
  codes[0] = codes[1] = 0;
  emask = 0;
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const uint32_t v = x[k];
    const uint32_t c0 = tab[(v >> 7) & 0xFF];
    const uint32_t c1 = tab[(v >> 23) & 0xFF];
    const uint32_t b0 = (v & 0x7F) | ((v >> 8) & 0x80);
    const uint32_t b1 = ((v >> 16) & 0x7F) | ((v >> 24) & 0x80);
    body[k >> 1] |= (b0 | (b1 << 8)) << (16 * (k & 1));
    codes[k >> 2] |= ((c0 & 0x0F) | ((c1 & 0x0F) << 4)) << (8 * (k & 3));
    emask |= ((c0 >> 4) | ((c1 >> 4) << 1)) << (2 * k);
  }
}

template <bool kFast, bool kSequential>
__global__ __launch_bounds__(kThreads) void top16_encode_lanes(LaunchArgs a, EncodeGeom g) {
  __shared__ unsigned char s_tab[512];
  __shared__ unsigned int s_wave[kThreads / kWave];
  const unsigned int tid = threadIdx.x;
  const unsigned int lane = tid & (kWave - 1);
  load_code_table(a.tables, s_tab);
  __syncthreads();

  unsigned int first, stop;
  if (kSequential) {
    first = 0;
    stop = a.total_tiles;
  } else {
    first = xcd_remap(blockIdx.x, gridDim.x);
    stop = first + 1;
  }
  unsigned long long running = 0;  // sequential mode: escapes in earlier tiles
  const unsigned int inbody = a.inbody_slots;  // body bytes hold the staging (see below)

  for (unsigned int tile = first; tile < stop; ++tile) {
    const unsigned int r = find_payload(a, tile);
    const PayloadDesc d = a.p[r];
    const unsigned long long n = payload_words(a, d);
    const unsigned long long half = n >> 1;
    unsigned long long start, end;
    tile_range(a, d, tile - d.tile_begin, n, start, end);
    unsigned char* payload = a.buf + d.buf_offset;
    const unsigned long long i0 = start + (unsigned long long)tid * kWordsPerLane;
    const bool active = i0 < end;

    uint32_t x[8];
    uint32_t body[4], codes[2], emask;
    if (kFast) {
      // Tiles never cross the K/V split and every lane is wholly inside or
      // outside the tile (plane_words % 16 == 0).
      const unsigned int plane = start >= half ? 1u : 0u;
      if (active) {
        const unsigned int in_plane = (unsigned int)(i0 - plane * half);
        const unsigned int j = div_u32(in_plane, g.bw_magic, g.bw);
        const unsigned int within = in_plane - j * g.bw;
        const unsigned long long blk =
            a.ids ? (unsigned long long)a.ids[d.ids_offset + j] : a.block_start + j;
        const uint4* src = reinterpret_cast<const uint4*>(
            a.kv + plane * a.plane_stride + blk * a.block_stride + within);
        const uint4 v0 = src[0];
        const uint4 v1 = src[1];
        x[0] = v0.x; x[1] = v0.y; x[2] = v0.z; x[3] = v0.w;
        x[4] = v1.x; x[5] = v1.y; x[6] = v1.z; x[7] = v1.w;
      } else {
#pragma unroll
        for (int k = 0; k < 8; ++k) x[k] = 0;
      }
      encode_lane(x, s_tab + plane * 256, body, codes, emask);
      if (!active) emask = 0;
      const bool first_lane = active && lane == 0;
      const bool last_lane = active && (lane == kWave - 1 || i0 + kWordsPerLane >= end);
      if (!inbody) store16_run(payload + 5 + i0, body, active, first_lane, last_lane);
      store8_run(payload + 5 + n + (i0 >> 1), codes, active, first_lane, last_lane);
    } else {
      // Generic geometry: per-word addressing and plane, byte stores.
#pragma unroll
      for (int k = 0; k < 8; ++k) x[k] = 0;
      body[0] = body[1] = body[2] = body[3] = 0;
      codes[0] = codes[1] = 0;
      emask = 0;
#pragma unroll 4
      for (int k = 0; k < kWordsPerLane; ++k) {
        const unsigned long long i = i0 + k;
        if (i >= end) break;
        const uint32_t w = a.kv[word_offset(a, d, i)];
        const uint32_t c = s_tab[(i >= half ? 256u : 0u) + ((w >> 7) & 0xFF)];
        if (!inbody) payload[5 + i] = (unsigned char)((w & 0x7F) | ((w >> 8) & 0x80));
        emask |= (c >> 4) << k;
        x[k >> 1] = (k & 1) ? (x[k >> 1] | (w << 16)) : w;
        codes[k >> 3] |= (c & 0x0F) << (4 * (k & 7));
      }
      // code bytes: a lane starts at an even index, so no byte is shared
      for (int k = 0; k < kWordsPerLane; k += 2) {
        const unsigned long long i = i0 + k;
        if (i >= end) break;
        payload[5 + n + (i >> 1)] = (unsigned char)((codes[k >> 3] >> (4 * (k & 7))) & 0xFF);
      }
    }

    // ---- escapes: per-lane count, workgroup prefix (ascending positions) ----
    const unsigned int cnt = __popc(emask);
    unsigned int tile_total;
    const unsigned int lane_base = block_exclusive_sum(cnt, s_wave, tile_total);
    if (kSequential) {
      if (emask) {
        const unsigned long long cap = escape_capacity(n);
        unsigned char* entries = payload + 5 + n + (n + 1) / 2;
        unsigned long long slot = running + lane_base;
#pragma unroll
        for (int k = 0; k < kWordsPerLane; ++k) {
          if (!((emask >> k) & 1)) continue;
          if (slot < cap)
            put_entry(entries, slot, (unsigned int)(i0 + k), (x[k >> 1] >> (7 + 16 * (k & 1))) & 0xFF);
          ++slot;
        }
      }
      running += tile_total;
    } else if (inbody) {
      // the count, then up to `slots` escapes, in the tile's own body bytes (the
      // body is written from the source after the finalize has read them)
      unsigned char* hdr = payload + 5 + start;
      const unsigned int slots = min(inbody, (unsigned int)((end - start) >> 2) - 1u);
      if (emask) {
        unsigned int idx = lane_base;
#pragma unroll
        for (int k = 0; k < kWordsPerLane; ++k) {
          if (!((emask >> k) & 1)) continue;
          if (idx < slots)
            *reinterpret_cast<u32_unaligned*>(hdr + 4 + 4 * idx) =
                ((unsigned int)(i0 + k - start) << 8) | ((x[k >> 1] >> (7 + 16 * (k & 1))) & 0xFF);
          ++idx;
        }
      }
      if (tid == 0) *reinterpret_cast<u32_unaligned*>(hdr) = tile_total;
      zero_escape_share(payload, n, tile - d.tile_begin, payload_tiles(a, n));
    } else {
      unsigned int* staged = a.workspace + a.total_tiles + (unsigned long long)tile * kStageSlots;
      if (emask) {
        unsigned int idx = lane_base;
#pragma unroll
        for (int k = 0; k < kWordsPerLane; ++k) {
          if (!((emask >> k) & 1)) continue;
          if (idx < kStageSlots)
            staged[idx] = ((unsigned int)(i0 + k - start) << 8) |
                          ((x[k >> 1] >> (7 + 16 * (k & 1))) & 0xFF);
          ++idx;
        }
      }
      if (tid == 0) a.workspace[tile] = tile_total;
      zero_escape_share(payload, n, tile - d.tile_begin, payload_tiles(a, n));
    }
  }

  if (kSequential) {
    // one payload: zero unused slots, then the header
    const PayloadDesc d = a.p[0];
    const unsigned long long n = payload_words(a, d);
    const unsigned long long cap = escape_capacity(n);
    unsigned char* payload = a.buf + d.buf_offset;
    unsigned char* entries = payload + 5 + n + (n + 1) / 2;
    const unsigned long long used = running < cap ? running : cap;
    zero_fill(entries + 5 * used, 5 * (cap - used));
    if (tid == 0) write_header(payload, n, running);
  }
}


// Body bytes of every tile, from the source (the last pass of the drop-in encode
// whose escapes were staged in the body bytes).
template <bool kFast>
__global__ __launch_bounds__(kThreads) void top16_body_lanes(LaunchArgs a, EncodeGeom g) {
  const unsigned int tid = threadIdx.x;
  const unsigned int lane = tid & (kWave - 1);
  const unsigned int tile = xcd_remap(blockIdx.x, gridDim.x);
  const unsigned int r = find_payload(a, tile);
  const PayloadDesc d = a.p[r];
  const unsigned long long n = payload_words(a, d);
  const unsigned long long half = n >> 1;
  unsigned long long start, end;
  tile_range(a, d, tile - d.tile_begin, n, start, end);
  unsigned char* payload = a.buf + d.buf_offset;
  const unsigned long long i0 = start + (unsigned long long)tid * kWordsPerLane;
  const bool active = i0 < end;
  if (kFast) {
    const unsigned int plane = start >= half ? 1u : 0u;
    uint32_t x[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    if (active) {
      const unsigned int in_plane = (unsigned int)(i0 - plane * half);
      const unsigned int j = div_u32(in_plane, g.bw_magic, g.bw);
      const unsigned int within = in_plane - j * g.bw;
      const unsigned long long blk =
          a.ids ? (unsigned long long)a.ids[d.ids_offset + j] : a.block_start + j;
      const uint4* src = reinterpret_cast<const uint4*>(
          a.kv + plane * a.plane_stride + blk * a.block_stride + within);
      const uint4 v0 = src[0];
      const uint4 v1 = src[1];
      x[0] = v0.x; x[1] = v0.y; x[2] = v0.z; x[3] = v0.w;
      x[4] = v1.x; x[5] = v1.y; x[6] = v1.z; x[7] = v1.w;
    }
    uint32_t body[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint32_t w0 = x[2 * q], w1 = x[2 * q + 1];
      const uint32_t t0 = (w0 & 0x007F007Fu) | ((w0 >> 8) & ~0x007F007Fu);
      const uint32_t t1 = (w1 & 0x007F007Fu) | ((w1 >> 8) & ~0x007F007Fu);
      body[q] = __builtin_amdgcn_perm(t1, t0, 0x06040200u);
    }
    const bool first_lane = active && lane == 0;
    const bool last_lane = active && (lane == kWave - 1 || i0 + kWordsPerLane >= end);
    store16_run(payload + 5 + i0, body, active, first_lane, last_lane);
  } else {
    for (int k = 0; k < kWordsPerLane; ++k) {
      const unsigned long long i = i0 + k;
      if (i >= end) break;
      const uint32_t w = a.kv[word_offset(a, d, i)];
      payload[5 + i] = (unsigned char)((w & 0x7F) | ((w >> 8) & 0x80));
    }
  }
}

// ---------------------------------------------------------------------------
// Tile kernels: block words a multiple of 1024, one block per wave.
//
// A workgroup handles one 4096-word tile of one plane; wave w covers words
// [start + 1024w, start + 1024w + 1024), which lie in one KV block (block words a
// multiple of 1024), so block lookup and every base address are wave-uniform
// scalars. Lane l handles two 8-word runs of its wave's range, words 8l .. 8l + 7
// ("run A") and 512 + 8l .. 512 + 8l + 7 ("run B"), so that every vector memory
// instruction of the wave covers one contiguous span (1 KiB of bf16, 512 B of body
// bytes, 256 B of code bytes). The per-word work is a handful of VALU operations
// (byte permutes, bit-field inserts) plus one LDS lookup for the encoder. Body and
// code spans may start at any byte (a payload at a buffer's first byte has its
// body at byte 5): the memory system splits an unaligned access, and each store
// writes only bytes of its own tile.

// Code table byte for each of four exponents packed in a dword of the 544-byte
// table: the code (0..15), or 0x10 for an escape (a code byte other than 255 keeps
// its low nibble, as the reference's `(code & 0x0F)` does).
__device__ __forceinline__ uint32_t pack_codes4(uint32_t raw) {
  uint32_t packed = 0;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const uint32_t c = (raw >> (8 * e)) & 0xFF;
    packed |= (c == 255 ? 0x10u : (c & 0x0Fu)) << (8 * e);
  }
  return packed;
}

// Encodes one 8-word run (4 dwords) with the code table of its plane: 8 body
// bytes, 4 code bytes, and an 8-bit escape mask.
__device__ __forceinline__ void encode_run8(const uint32_t* x, const unsigned char* tab,
                                            uint32_t (&body)[2], uint32_t& codes,
                                            uint32_t& emask) {
  uint32_t D[2], flags = 0;
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    // body bytes of 4 words: mantissa bits 0-6 and the sign bit into bit 7
    // (bytes 1 and 3 of t0/t1 are don't-care: the permute keeps bytes 0 and 2)
    const uint32_t w0 = x[2 * q], w1 = x[2 * q + 1];
    const uint32_t t0 = (w0 & 0x007F007Fu) | ((w0 >> 8) & ~0x007F007Fu);
    const uint32_t t1 = (w1 & 0x007F007Fu) | ((w1 >> 8) & ~0x007F007Fu);
    body[q] = __builtin_amdgcn_perm(t1, t0, 0x06040200u);
    // codes of 4 words, one per byte (0x10 marks an escape)
    const uint32_t c0 = tab[(w0 >> 7) & 0xFF];
    const uint32_t c1 = tab[(w0 >> 23) & 0xFF];
    const uint32_t c2 = tab[(w1 >> 7) & 0xFF];
    const uint32_t c3 = tab[(w1 >> 23) & 0xFF];
    D[q] = c0 | (c1 << 8) | (c2 << 16) | (c3 << 24);
    flags |= D[q];
  }
  const uint32_t ta = D[0] & 0x0F0F0F0Fu, tb = D[1] & 0x0F0F0F0Fu;
  codes = __builtin_amdgcn_perm(tb | (tb >> 4), ta | (ta >> 4), 0x06040200u);
  emask = 0;
  if (flags & 0x10101010u) {
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const uint32_t m = D[q] & 0x10101010u;
      emask |= (((m >> 4) & 1) | ((m >> 11) & 2) | ((m >> 18) & 4) | ((m >> 25) & 8)) << (4 * q);
    }
  }
}

// Zeroes the payload's escape section in 4 KiB spans of 16-byte stores, one span per
// tile of the payload from its first tile on (a section is at most n / 40 + 5 bytes,
// fewer than the payload's 4096-word tiles can cover): wide, line-filling stores
// instead of a sliver per tile.
__device__ __forceinline__ void zero_escape_span(unsigned char* payload, unsigned long long n,
                                                 unsigned int local_tile) {
  const unsigned long long len = 5 * escape_capacity(n);
  const unsigned long long lo = (unsigned long long)local_tile * (kThreads * 16);
  if (lo >= len) return;
  const unsigned long long hi = min(lo + kThreads * 16, len);
  zero_fill(payload + 5 + n + (n + 1) / 2 + lo, hi - lo);
}

// kSeen: also writes the tile's high-byte presence mask to a.presence (the
// variant for a layer likely to overflow, whose palette fallback then needs no
// presence pass of its own).
// kInBody (drop-in encode with no room for a workspace): the tile's escape count
// and its first kInBodySlots escapes are staged in the tile's first 512 body
// bytes (run A of wave 0, left unwritten here); top16_body_tile writes those
// body bytes once the finalize has read the staging.
template <bool kIds, bool kSeen, bool kInBody>
__global__ __launch_bounds__(kThreads) void top16_encode_tile(LaunchArgs a, EncodeGeom geo) {
  static_assert(!(kSeen && kInBody), "presence masks come with a workspace");
  __shared__ uint32_t s_tab[64];  // this tile's plane, 4 code bytes per dword
  __shared__ unsigned int s_wave[kThreads / kWave];
  __shared__ uint32_t s_seen[kSeen ? 64 : 1];  // one byte per high byte value
  const unsigned int tid = threadIdx.x;
  const unsigned int lane = tid & (kWave - 1);
  const unsigned int wave = uniform(tid >> 6);
  const unsigned int tile = group_index();
  const PlaneTile t = plane_tile<kTileShift>(a, tile);
  const unsigned int in_plane = t.in_plane0 + wave * 1024;
  const unsigned long long wstart = t.plane * (t.n >> 1) + in_plane;  // payload word
  const bool active = wave * 1024 < t.words;  // whole waves
  // source loads first, then the code table, so the table's round trip overlaps them
  uint32_t x[8];
  if (active) {
    const uint16_t* src = a.kv + wave_source<kIds>(a, t, geo, in_plane);
    const u32x4 v0 = load_stream16(src + 8 * lane);
    const u32x4 v1 = load_stream16(src + 512 + 8 * lane);
    x[0] = v0.x; x[1] = v0.y; x[2] = v0.z; x[3] = v0.w;
    x[4] = v1.x; x[5] = v1.y; x[6] = v1.z; x[7] = v1.w;
  } else {
#pragma unroll
    for (int q = 0; q < 8; ++q) x[q] = 0;
  }
  if (tid < 64) {
    s_tab[tid] = pack_codes4(reinterpret_cast<const uint32_t*>(a.tables + t.plane * 256)[tid]);
    if (kSeen) s_seen[tid] = 0;
  }
  __syncthreads();  // s_tab ready
  const unsigned char* tab = reinterpret_cast<const unsigned char*>(s_tab);

  uint32_t body_a[2], body_b[2], code_a, code_b, mask_a, mask_b;
  encode_run8(x, tab, body_a, code_a, mask_a);
  encode_run8(x + 4, tab, body_b, code_b, mask_b);
  if (kSeen && active) {
    unsigned char* seen = reinterpret_cast<unsigned char*>(s_seen);
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      seen[(x[k] >> 8) & 0xFF] = 1;
      seen[x[k] >> 24] = 1;
    }
  }
  unsigned char* const tile_body = t.payload + 5 + t.plane * (t.n >> 1) + t.in_plane0;
  if (active) {
    unsigned char* pbody = t.payload + 5 + wstart;
    unsigned char* pcode = t.payload + 5 + t.n + (wstart >> 1);
    if (!kInBody || wave != 0) store_through8(pbody + 8 * lane, u32x2{body_a[0], body_a[1]});
    store_through8(pbody + 512 + 8 * lane, u32x2{body_b[0], body_b[1]});
    store_through4(pcode + 4 * lane, code_a);
    store_through4(pcode + 256 + 4 * lane, code_b);
  } else {
    mask_a = mask_b = 0;
  }

  // escapes (rare), in ascending word order: run A of every lane of the wave,
  // then run B of every lane, then the next wave. Per-lane counts of both runs are
  // packed into one word (16 bits each) for a single shuffle scan; a wave without
  // escapes skips the scan.
  const unsigned int cnt = __popc(mask_a) | (__popc(mask_b) << 16);
  unsigned int incl = 0;
  if (__ballot(cnt != 0)) {
    incl = cnt;
#pragma unroll
    for (int d = 1; d < kWave; d <<= 1) {
      const unsigned int v = (unsigned int)__shfl_up((int)incl, d, kWave);
      if (lane >= (unsigned int)d) incl += v;
    }
  }
  const unsigned int wave_tot = uniform((unsigned int)__shfl((int)incl, kWave - 1, kWave));
  const unsigned int wave_a = wave_tot & 0xFFFFu;
  if (lane == 0) s_wave[wave] = wave_a + (wave_tot >> 16);
  __syncthreads();
  if (kSeen) {
    // wave w reports high bytes 64w .. 64w + 63
    const unsigned long long bits =
        __ballot(reinterpret_cast<const unsigned char*>(s_seen)[tid] != 0);
    if (lane == 0) {
      a.presence[8ull * tile + 2 * wave] = (uint32_t)bits;
      a.presence[8ull * tile + 2 * wave + 1] = (uint32_t)(bits >> 32);
    }
  }
  unsigned int before = 0, total = 0;
#pragma unroll
  for (int w = 0; w < kThreads / kWave; ++w) {
    const unsigned int v = s_wave[w];
    if (w < (int)wave) before += v;
    total += v;
  }
  if (tid == 0) {
    if (kInBody)
      *reinterpret_cast<u32_unaligned*>(tile_body) = total;
    else
      a.workspace[tile] = total;
  }
  // directory record of this wave's chunk: its first escape's slot within the tile,
  // its escape count, and its first kDirInline escapes (written by the lanes that
  // hold them, below)
  uint32_t* rec = a.dir_rec ? a.dir_rec + 4 * (4 * (unsigned long long)tile + wave) : nullptr;
  if (rec && lane == 0) rec[0] = before | ((wave_a + (wave_tot >> 16)) << 16);
  if (mask_a | mask_b) {
    const unsigned int excl = incl - cnt;
    unsigned int* staged =
        kInBody ? nullptr : a.workspace + a.total_tiles + (unsigned long long)tile * kStageSlots;
    auto stage = [&](unsigned int idx, uint32_t e) {
      if (kInBody) {
        if (idx < kInBodySlots) *reinterpret_cast<u32_unaligned*>(tile_body + 4 + 4 * idx) = e;
      } else if (idx < kStageSlots) {
        staged[idx] = e;
      }
    };
    const unsigned int local = wave * 1024 + lane * 8;
    unsigned int idx = before + (excl & 0xFFFFu);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      if (!((mask_a >> j) & 1)) continue;
      const uint32_t e = ((local + j) << 8) | ((x[j >> 1] >> (7 + 16 * (j & 1))) & 0xFF);
      stage(idx, e);
      if (rec && idx - before < kDirInline) rec[1 + idx - before] = e;
      ++idx;
    }
    idx = before + wave_a + (excl >> 16);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      if (!((mask_b >> j) & 1)) continue;
      const uint32_t e =
          ((local + 512 + j) << 8) | ((x[4 + (j >> 1)] >> (7 + 16 * (j & 1))) & 0xFF);
      stage(idx, e);
      if (rec && idx - before < kDirInline) rec[1 + idx - before] = e;
      ++idx;
    }
  }
  zero_escape_span(t.payload, t.n, t.local_tile);
}

// The first 512 body bytes of every tile (run A of wave 0), from the source: the
// last pass of a drop-in encode whose tiles staged their escapes there. One wave
// per tile, 8 words per lane.
template <bool kIds>
__global__ __launch_bounds__(kThreads) void top16_body_tile(LaunchArgs a, EncodeGeom geo) {
  const unsigned int lane = threadIdx.x & (kWave - 1);
  const unsigned int tile = blockIdx.x * (kThreads / kWave) + uniform(threadIdx.x >> 6);
  if (tile >= a.total_tiles) return;  // whole waves
  const PlaneTile t = plane_tile<kTileShift>(a, tile);
  const uint16_t* src = a.kv + wave_source<kIds>(a, t, geo, t.in_plane0);
  const u32x4 v = load_stream16(src + 8 * lane);
  uint32_t body[2];
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const uint32_t w0 = q ? v.z : v.x, w1 = q ? v.w : v.y;
    const uint32_t t0 = (w0 & 0x007F007Fu) | ((w0 >> 8) & ~0x007F007Fu);
    const uint32_t t1 = (w1 & 0x007F007Fu) | ((w1 >> 8) & ~0x007F007Fu);
    body[q] = __builtin_amdgcn_perm(t1, t0, 0x06040200u);
  }
  unsigned char* pbody = t.payload + 5 + t.plane * (t.n >> 1) + t.in_plane0;
  store_through8(pbody + 8 * lane, u32x2{body[0], body[1]});
}

// Decode + scatter of one tile; the destination's j-th block from block_of(t, j).
template <typename BlockOf>
__device__ __forceinline__ void decode_tile(const LaunchArgs& a, const EncodeGeom& geo,
                                            BlockOf block_of) {
  const unsigned int lane = threadIdx.x & (kWave - 1);
  const unsigned int wave = uniform(threadIdx.x >> 6);
  const PlaneTile t = plane_tile<kTileShift>(a, group_index());
  const unsigned int in_plane = t.in_plane0 + wave * 1024;
  const unsigned long long wstart = t.plane * (t.n >> 1) + in_plane;  // payload word
  if (wave * 1024 >= t.words) return;  // whole waves; no barrier in this kernel
  const unsigned int mode = t.payload[0];
  const uint32_t* cbw = reinterpret_cast<const uint32_t*>(a.tables + 512 + t.plane * 16);
  const uint32_t cb[4] = {cbw[0], cbw[1], cbw[2], cbw[3]};
  const unsigned char* pbody = t.payload + 5 + wstart;
  const unsigned char* pcode = t.payload + 5 + t.n + (wstart >> 1);
  const u32x2 body_a = load_stream8(pbody + 8 * lane);
  const u32x2 body_b = load_stream8(pbody + 512 + 8 * lane);
  const uint32_t code_a = load_stream4(pcode + 4 * lane);
  const uint32_t code_b = load_stream4(pcode + 256 + 4 * lane);
  // The block-id load and the destination address come after the payload loads
  // are issued, so the two round trips overlap.
  __builtin_amdgcn_sched_barrier(0);
  uint16_t* dst =
      a.kv + wave_offset_by(a, t, geo, in_plane, [&](unsigned int j) { return block_of(t, j); });
  const u32x4 out_a = decode_run8(body_a, code_a, cb);
  const u32x4 out_b = decode_run8(body_b, code_b, cb);
  // Keeps the payload loads ahead of the mode test below: without this use the
  // compiler sinks them under the test and the mode byte's round trip comes first.
  asm volatile("" ::"v"(out_a), "v"(out_b));
  // the reference decoder leaves a payload whose byte 0 is not 5 untouched
  if (mode != 5) return;
  store_through16(dst + 8 * lane, out_a);
  store_through16(dst + 512 + 8 * lane, out_b);
}

template <bool kIds>
__global__ __launch_bounds__(kThreads) void top16_decode_tile(LaunchArgs a, EncodeGeom geo) {
  decode_tile(a, geo, [&](const PlaneTile& t, unsigned int j) {
    return kIds ? (unsigned long long)t.ids[j] : a.block_start + j;
  });
}

// One request whose block table rides in the kernel arguments.
__global__ __launch_bounds__(kThreads) void top16_decode_tile_inline(LaunchArgs a, EncodeGeom geo,
                                                                     InlineBlocks table) {
  decode_tile(a, geo, [&](const PlaneTile&, unsigned int j) {
    return (unsigned long long)table.id[j];
  });
}

// Replaces the exponent of word w (0..1023) of this wave's chunk, held in run A
// (w < 512) or run B of lane (w & 511) / 8, by `exponent` (kvq_splitzip_cuda.cu:
// 276-281: sign and mantissa stay, bits 7-14 take the escape's exponent). w and
// exponent are wave-uniform; only the owning lane's dword changes. Branch-free
// selects over the eight dwords (no register indexing).
__device__ __forceinline__ void patch_word(u32x4& run_a, u32x4& run_b, unsigned int lane,
                                           unsigned int w, unsigned int exponent) {
  const unsigned int half = 16 * (w & 1);
  const uint32_t clear = lane == ((w & 511) >> 3) ? (0x7F80u << half) : 0u;
  const uint32_t bits = (exponent << (7 + half)) & clear;
  const unsigned int d = ((w >> 9) << 2) | ((w >> 1) & 3);  // dword of the two runs
#define UKV_PATCH(v, k) v = (d == (k)) ? ((v & ~clear) | bits) : v
  UKV_PATCH(run_a.x, 0); UKV_PATCH(run_a.y, 1); UKV_PATCH(run_a.z, 2); UKV_PATCH(run_a.w, 3);
  UKV_PATCH(run_b.x, 4); UKV_PATCH(run_b.y, 5); UKV_PATCH(run_b.z, 6); UKV_PATCH(run_b.w, 7);
#undef UKV_PATCH
}

// Decode + scatter with the escape directory the encoder wrote (one kernel, no
// patch pass): each wave reads its chunk's record and its tile's base slot along
// with the payload, and puts the chunk's escapes into its registers before the
// stores. A chunk with more than kDirInline escapes reads them from the payload's
// (ascending) escape list at slots base + first .. + count.
template <bool kIds>
__global__ __launch_bounds__(kThreads) void top16_decode_tile_dir(LaunchArgs a, EncodeGeom geo) {
  const unsigned int lane = threadIdx.x & (kWave - 1);
  const unsigned int wave = uniform(threadIdx.x >> 6);
  const unsigned int tile = group_index();
  const PlaneTile t = plane_tile<kTileShift>(a, tile);
  const unsigned int in_plane = t.in_plane0 + wave * 1024;
  const unsigned long long wstart = t.plane * (t.n >> 1) + in_plane;  // payload word
  if (wave * 1024 >= t.words) return;  // whole waves; no barrier in this kernel
  const u32x4 rec =
      *reinterpret_cast<const u32x4*>(a.dir_rec + 4 * (4 * (unsigned long long)tile + wave));
  const unsigned int tile_base = a.dir_base[tile];
  const unsigned int mode = t.payload[0];
  const uint32_t* cbw = reinterpret_cast<const uint32_t*>(a.tables + 512 + t.plane * 16);
  const uint32_t cb[4] = {cbw[0], cbw[1], cbw[2], cbw[3]};
  const unsigned char* pbody = t.payload + 5 + wstart;
  const unsigned char* pcode = t.payload + 5 + t.n + (wstart >> 1);
  const u32x2 body_a = load_stream8(pbody + 8 * lane);
  const u32x2 body_b = load_stream8(pbody + 512 + 8 * lane);
  const uint32_t code_a = load_stream4(pcode + 4 * lane);
  const uint32_t code_b = load_stream4(pcode + 256 + 4 * lane);
  __builtin_amdgcn_sched_barrier(0);
  uint16_t* dst = a.kv + wave_source<kIds>(a, t, geo, in_plane);
  u32x4 out_a = decode_run8(body_a, code_a, cb);
  u32x4 out_b = decode_run8(body_b, code_b, cb);
  const unsigned int first = uniform(rec.x & 0xFFFFu);
  const unsigned int count = uniform(rec.x >> 16);
  const unsigned int chunk0 = wave * 1024;  // tile-local position of the chunk's first word
  if (count != 0) {
    if (count <= (unsigned int)kDirInline) {
      const uint32_t inl[kDirInline] = {uniform(rec.y), uniform(rec.z), uniform(rec.w)};
#pragma unroll
      for (int i = 0; i < kDirInline; ++i)
        if ((unsigned int)i < count)
          patch_word(out_a, out_b, lane, ((inl[i] >> 8) - chunk0) & 1023u, inl[i] & 0xFF);
    } else if (mode == 5 && (unsigned long long)tile_base + first + count <=
                                escape_capacity(t.n)) {
      // escape-dense chunk: entries from the payload, 64 per round (an overflowed
      // payload, whose slots stop at the capacity, is not stored at all)
      const unsigned char* entries = t.payload + 5 + t.n + (t.n >> 1);
      const unsigned long long slot0 = (unsigned long long)tile_base + first;
      for (unsigned int r0 = 0; r0 < count; r0 += kWave) {
        unsigned int pos = 0xFFFFFFFFu, ex = 0;
        if (r0 + lane < count) {
          const unsigned char* e = entries + 5 * (slot0 + r0 + lane);
          pos = *reinterpret_cast<const u32_unaligned*>(e);
          ex = e[4];
        }
        const unsigned int m = min(count - r0, (unsigned int)kWave);
        for (unsigned int i = 0; i < m; ++i) {
          const unsigned long long p = (unsigned int)__builtin_amdgcn_readlane((int)pos, i);
          const unsigned int xe = (unsigned int)__builtin_amdgcn_readlane((int)ex, i);
          if (p >= wstart && p < wstart + 1024)
            patch_word(out_a, out_b, lane, (unsigned int)(p - wstart), xe);
        }
      }
    }
  }
  asm volatile("" ::"v"(out_a), "v"(out_b));
  if (mode != 5) return;
  store_through16(dst + 8 * lane, out_a);
  store_through16(dst + 512 + 8 * lane, out_b);
}

// Scans the escapes of one tile from the source words (tiles with more escapes
// than were staged) and places them from slot `base` on.
__device__ void rescan_tile(const LaunchArgs& a, const PayloadDesc& d, unsigned int local_tile,
                            unsigned long long n, unsigned long long base,
                            const unsigned char* s_tab, unsigned int* s_wave,
                            unsigned char* entries, unsigned long long cap) {
  unsigned long long start, end;
  tile_range(a, d, local_tile, n, start, end);
  const unsigned long long half = n >> 1;
  for (unsigned long long sub = start; sub < end; sub += kTileWords) {
    const unsigned long long i0 = sub + (unsigned long long)threadIdx.x * kWordsPerLane;
    uint32_t emask = 0;
    uint32_t ex[kWordsPerLane];
#pragma unroll
    for (int k = 0; k < kWordsPerLane; ++k) {
      const unsigned long long i = i0 + k;
      ex[k] = 0;
      if (i < end) {
        const uint32_t w = a.kv[word_offset(a, d, i)];
        const uint32_t e = (w >> 7) & 0xFF;
        ex[k] = e;
        emask |= (uint32_t)(s_tab[(i >= half ? 256u : 0u) + e] >> 4) << k;
      }
    }
    unsigned int total;
    const unsigned int lane_base = block_exclusive_sum(__popc(emask), s_wave, total);
    unsigned long long slot = base + lane_base;
#pragma unroll
    for (int k = 0; k < kWordsPerLane; ++k) {
      if (!((emask >> k) & 1)) continue;
      if (slot < cap) put_entry(entries, slot, (unsigned int)(i0 + k), ex[k]);
      ++slot;
    }
    base += total;
  }
}

// kProbe (a probe encode of a layer that overflowed before, whose caller re-encodes
// an overflowed payload as fixed6 / fixed5): a payload found to overflow gets its
// header but no escape placement (its escape section is left zeroed; the
// reference's is in atomic order and discarded the same way), and
// a.payload_count more workgroups after the finalize groups compute each payload's
// palette from the presence masks the tile kernel wrote (a.palette_info).
template <int kFinGroups, bool kInBody, int kDenseItems, bool kProbe = false>
__global__ __launch_bounds__(kThreads) void top16_encode_finalize(LaunchArgs a) {
  constexpr int kFinPerThread = kFinGroups;             // tile counts per thread per pass
  constexpr int kFinChunk = kThreads * kFinPerThread;   // tiles scanned per pass
  if (kProbe && blockIdx.x >= a.payload_count * kFinGroups) {
    __shared__ unsigned int s_mask[8];
    const unsigned int r = blockIdx.x - a.payload_count * kFinGroups;
    const PayloadDesc d = a.p[r];
    const unsigned long long n = 2ull * d.block_count * a.block_words;
    palette_info_from_masks(a.presence + 8ull * d.tile_begin,
                            payload_tiles(a, n), a.palette_info[r], s_mask);
    return;
  }
  __shared__ unsigned int s_over_tile[kFinChunk / kFinGroups];
  __shared__ unsigned int s_over_base[kFinChunk / kFinGroups];
  __shared__ unsigned int s_over_count;
  __shared__ unsigned int s_dense_tile[kFinChunk / kFinGroups];  // tile | escapes << 24
  __shared__ unsigned int s_dense_base[kFinChunk / kFinGroups];
  __shared__ unsigned int s_dense_count;
  __shared__ unsigned int s_wave[kThreads / kWave];
  __shared__ unsigned char s_tab[512];
  const unsigned int tid = threadIdx.x;
  const unsigned int r = blockIdx.x / kFinGroups;
  const unsigned int grp = blockIdx.x % kFinGroups;
  // Every kernel argument of the common path is read here, before any branch on
  // one of them: the scalar loads then go out together instead of as a chain of
  // dependent round trips (a cold constant cache makes each one an L2 access).
  const PayloadDesc d = a.p[r];
  const unsigned long long linear = a.linear_words;
  const unsigned long long bw = a.block_words;
  const unsigned int per_plane = a.tiles_per_plane_mode;
  const unsigned int shift = a.tile_shift;
  const unsigned int total_tiles = a.total_tiles;
  unsigned char* const buf = a.buf;
  unsigned int* const ws = a.workspace;
  uint32_t* const dir_base = a.dir_base;
  // (the compiler would otherwise sink each load to its first use, behind branches)
  asm volatile("" ::"s"(d.buf_offset), "s"(d.block_count), "s"(d.tile_begin), "s"(linear),
               "s"(bw), "s"(per_plane), "s"(shift), "s"(total_tiles), "s"(buf), "s"(ws),
               "s"(dir_base));
  asm volatile("" ::"s"(a.kv), "s"(a.ids), "s"(a.tables), "s"(a.plane_stride),
               "s"(a.block_stride), "s"(a.block_start), "s"(d.ids_offset));
  const unsigned long long n = linear ? linear : 2ull * d.block_count * bw;
  const unsigned long long cap = escape_capacity(n);
  const unsigned long long tile_words = 1ull << shift;
  const unsigned int tiles =
      per_plane ? 2u * (unsigned int)(((n >> 1) + tile_words - 1) >> shift)
                : (unsigned int)((n + tile_words - 1) >> shift);
  unsigned char* payload = buf + d.buf_offset;
  unsigned char* entries = payload + 5 + n + (n + 1) / 2;
  const unsigned int* counts = ws + d.tile_begin;
  const unsigned int* staged = ws + total_tiles + (unsigned long long)d.tile_begin * kStageSlots;
  // kInBody (drop-in encode without a workspace): each tile's count and staged
  // escapes sit in its own body bytes (u32 count, then the entries; tiles of at
  // least 64 words)
  const unsigned int inbody = kInBody ? a.inbody_slots : 0u;
  if (tid == 0) {  // ordered by the barriers of the first scan
    s_over_count = 0;
    s_dense_count = 0;
  }

  unsigned long long running = 0;  // escapes in earlier chunks
  for (unsigned int chunk0 = 0; chunk0 < tiles; chunk0 += kFinChunk) {
    const unsigned int m = min((unsigned int)kFinChunk, tiles - chunk0);
    // Thread tid holds the counts of tiles chunk0 + tid * kFinPerThread + k and
    // places the escapes of the one among them that belongs to this group
    // (k == grp). Its first staged escapes are loaded along with the counts, so
    // the common tile (few escapes) needs a single round trip.
    static_assert(kFinPerThread == kFinGroups, "one tile of each group per thread");
    unsigned int mine[kFinPerThread];
    unsigned int sum = 0;
#pragma unroll
    for (int k = 0; k < kFinPerThread; ++k) {
      // loads without branches: indices past the chunk read its last count
      const unsigned int t = tid * kFinPerThread + k;
      const unsigned int tt = chunk0 + min(t, m - 1);
      unsigned int v;
      if (kInBody) {
        unsigned long long ts, te;
        tile_range(a, d, tt, n, ts, te);
        v = *reinterpret_cast<const u32_unaligned*>(payload + 5 + ts);
      } else {
        v = counts[tt];
      }
      mine[k] = t < m ? v : 0;
      sum += mine[k];
    }
    const unsigned int own = tid * kFinPerThread + grp;  // this thread's tile of the group
    const unsigned int own_c = chunk0 + min(own, m - 1);
    const unsigned int* st = staged + (unsigned long long)own_c * kStageSlots;
    const unsigned char* st_body = nullptr;
    unsigned int slots = kStageSlots;
    if (kInBody) {
      unsigned long long ts, te;
      tile_range(a, d, own_c, n, ts, te);
      st_body = payload + 5 + ts + 4;
      slots = min(inbody, (unsigned int)((te - ts) >> 2) - 1u);
    }
    auto staged_at = [&](unsigned int q) -> unsigned int {
      return kInBody ? *reinterpret_cast<const u32_unaligned*>(st_body + 4 * q) : st[q];
    };
    unsigned int pre[kFinPreload];
#pragma unroll
    for (int q = 0; q < kFinPreload; ++q) pre[q] = staged_at(q);
    unsigned int chunk_total;
    unsigned int prefix = block_exclusive_sum(sum, s_wave, chunk_total);
    if (kProbe && chunk0 == 0 && m == tiles && chunk_total > cap) {
      // the whole payload in one pass and over its capacity: header only
      running = chunk_total;
      break;
    }

    // staged escapes of this group's tile go straight to their slots
    unsigned int c = 0;
#pragma unroll
    for (int k = 0; k < kFinPerThread; ++k) {
      if ((unsigned int)k < grp) prefix += mine[k];
      if ((unsigned int)k == grp) c = mine[k];
    }
    const unsigned long long base = running + prefix;
    if (dir_base && own < m)
      dir_base[d.tile_begin + chunk0 + own] = (unsigned int)min(base, 0xFFFFFFFFull);
    if (c != 0 && base < cap) {
      if (c > slots) {
        const unsigned int q = atomicAdd(&s_over_count, 1u);
        s_over_tile[q] = chunk0 + own;
        s_over_base[q] = (unsigned int)base;
      } else if (c > (unsigned int)kFinPreload) {
        // more than the preloaded batch (dense escapes, e.g. outliers): placed
        // below by a whole wave, one entry per lane, instead of batch after
        // batch of dependent loads by this thread (c <= kStageSlots < 2^8,
        // chunk tiles < 2^24)
        const unsigned int q = atomicAdd(&s_dense_count, 1u);
        s_dense_tile[q] = own | (c << 24);
        s_dense_base[q] = (unsigned int)base;
      } else {
        unsigned long long start, end;
        tile_range(a, d, chunk0 + own, n, start, end);
        // batches of kFinPreload entries: the first came with the counts, later
        // batches are loaded together before they are stored
        for (unsigned int q0 = 0; q0 < c && base + q0 < cap; q0 += kFinPreload) {
          unsigned int v[kFinPreload];
#pragma unroll
          for (int e = 0; e < kFinPreload; ++e) {
            const unsigned int q = q0 + e;
            v[e] = q0 == 0 ? pre[e] : (q < c ? staged_at(q) : 0u);
          }
#pragma unroll
          for (int e = 0; e < kFinPreload; ++e) {
            const unsigned int q = q0 + e;
            if (q < c && base + q < cap)
              put_entry(entries, base + q, (unsigned int)(start + (v[e] >> 8)), v[e] & 0xFF);
          }
        }
      }
    }
    __syncthreads();
    // dense tiles: wave w places the entries of list items w, w + 4, ...;
    // kDenseItems items per pass so that their loads are in flight together
    const unsigned int dense = s_dense_count;
    for (unsigned int i0 = uniform(tid >> 6); i0 < dense;
         i0 += kDenseItems * (kThreads / kWave)) {
      const unsigned int lane = tid & (kWave - 1);
      unsigned int v[kDenseItems][kStageSlots / kWave], tile[kDenseItems], cnt[kDenseItems];
      unsigned long long start[kDenseItems], bases[kDenseItems];
#pragma unroll
      for (int h = 0; h < kDenseItems; ++h) {
        const unsigned int i = min(i0 + h * (kThreads / kWave), dense - 1);
        const unsigned int packed = s_dense_tile[i];
        tile[h] = chunk0 + (packed & 0xFFFFFFu);
        cnt[h] = i0 + h * (kThreads / kWave) < dense ? packed >> 24 : 0u;
        bases[h] = s_dense_base[i];
        unsigned long long end;
        tile_range(a, d, tile[h], n, start[h], end);
        const unsigned int* tst = staged + (unsigned long long)tile[h] * kStageSlots;
        const unsigned char* tbody = nullptr;
        if (kInBody) tbody = payload + 5 + start[h] + 4;
#pragma unroll
        for (int k = 0; k < kStageSlots / kWave; ++k) {
          const unsigned int q = min(lane + k * kWave, cnt[h] > 0 ? cnt[h] - 1 : 0u);
          v[h][k] = kInBody ? *reinterpret_cast<const u32_unaligned*>(tbody + 4 * q) : tst[q];
        }
      }
#pragma unroll
      for (int h = 0; h < kDenseItems; ++h)
#pragma unroll
        for (int k = 0; k < kStageSlots / kWave; ++k) {
          const unsigned int q = lane + k * kWave;
          if (q < cnt[h] && bases[h] + q < cap)
            put_entry(entries, bases[h] + q, (unsigned int)(start[h] + (v[h][k] >> 8)),
                      v[h][k] & 0xFF);
        }
    }
    // tiles with more escapes than were staged are scanned again from the source
    const unsigned int over = s_over_count;
    if (over) {
      load_code_table(a.tables, s_tab);
      __syncthreads();
      for (unsigned int q = 0; q < over; ++q)
        rescan_tile(a, d, s_over_tile[q], n, s_over_base[q], s_tab, s_wave, entries, cap);
    }
    running += chunk_total;
    __syncthreads();
    if (tid == 0) {
      s_over_count = 0;
      s_dense_count = 0;
    }
  }

  // unused escape slots were zeroed by the tile kernel
  if (grp == 0 && tid == 0) write_header(payload, n, running);
}

// ---------------------------------------------------------------------------
// decode

// Decode + scatter for any section alignment (block words a multiple of 16,
// destination 16-byte aligned): 16 consecutive words per lane, misaligned
// sections read as aligned chunks and realigned with the neighbour lane's data.
__global__ __launch_bounds__(kThreads) void top16_decode_lanes(LaunchArgs a, EncodeGeom geo) {
  __shared__ unsigned char s_cb[32];
  const unsigned int tid = threadIdx.x;
  const unsigned int lane = tid & (kWave - 1);
  if (tid < 32) s_cb[tid] = a.tables[512 + tid];
  const unsigned int tile = xcd_remap(blockIdx.x, gridDim.x);
  const TileInfo t = tile_info(a, tile);
  const unsigned int mode = t.payload[0];
  const unsigned long long i0 = t.start + (unsigned long long)tid * kWordsPerLane;
  const bool active = i0 < t.end;
  const bool last_lane = active && (lane == kWave - 1 || i0 + kWordsPerLane >= t.end);
  uint32_t body[4], codes[2];
  load16_run(t.payload + 5 + i0, active, last_lane, body);
  load8_run(t.payload + 5 + t.n + (i0 >> 1), active, last_lane, codes);
  __syncthreads();  // s_cb ready
  if (!active || mode != 5) return;
  const unsigned char* cb = s_cb + t.plane * 16;
  uint32_t out[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const uint32_t nb = (codes[k >> 2] >> (8 * (k & 3))) & 0xFF;
    const uint32_t e0 = cb[nb & 0x0F];
    const uint32_t e1 = cb[nb >> 4];
    const uint32_t bb = (body[k >> 1] >> (16 * (k & 1))) & 0xFFFF;
    const uint32_t w0 = (bb & 0x7F) | ((bb & 0x80) << 8) | (e0 << 7);
    const uint32_t w1 = ((bb >> 8) & 0x7F) | (bb & 0x8000) | (e1 << 7);
    out[k] = w0 | (w1 << 16);
  }
  uint4* dst = reinterpret_cast<uint4*>(a.kv + chunk_offset(a, t, geo, i0));
  dst[0] = make_uint4(out[0], out[1], out[2], out[3]);
  dst[1] = make_uint4(out[4], out[5], out[6], out[7]);
}

// Any geometry: one word per thread, grid-stride over every payload of the launch.
__global__ __launch_bounds__(kThreads) void top16_decode_generic(LaunchArgs a) {
  const unsigned int r = blockIdx.y;
  const PayloadDesc d = a.p[r];
  const unsigned char* payload = a.buf + d.buf_offset;
  if (payload[0] != 5) return;
  const unsigned long long n = payload_words(a, d);
  const unsigned long long half = n >> 1;
  const unsigned char* body = payload + 5;
  const unsigned char* codes = body + n;
  const unsigned char* cb = a.tables + 512;
  for (unsigned long long i = (unsigned long long)blockIdx.x * kThreads + threadIdx.x; i < n;
       i += (unsigned long long)gridDim.x * kThreads) {
    const uint32_t code = (codes[i >> 1] >> ((i & 1) * 4)) & 0x0F;
    const uint32_t e = cb[(i >= half ? 16u : 0u) + code];
    const uint32_t b = body[i];
    a.kv[word_offset(a, d, i)] = (uint16_t)((b & 0x7F) | ((b & 0x80) << 8) | (e << 7));
  }
}

// ApplyTop16Escapes semantics (kvq_splitzip_cuda.cu:253-284): for slot <
// min(count, cap) with position < n, the word gets the escape's exponent bits.
// The decode kernel wrote sign and mantissa from the body byte, so the patched word
// is rebuilt from that byte and stored (no read of the destination). One thread
// per escape slot; payload r owns workgroups [slot_group_begin, + ceil(cap_r/256)).
// The destination's j-th block of payload d from block_of(d, j).
template <typename BlockOf>
__device__ __forceinline__ void patch_escapes(const LaunchArgs& a, BlockOf block_of) {
  const unsigned int r = find_slot_payload(a, blockIdx.x);
  const PayloadDesc d = a.p[r];
  const unsigned long long s =
      (unsigned long long)(blockIdx.x - d.slot_group_begin) * kThreads + threadIdx.x;
  const unsigned long long n = payload_words(a, d);
  const unsigned long long cap = escape_capacity(n);
  if (s >= cap) return;
  const unsigned char* payload = a.buf + d.buf_offset;
  const unsigned char* e = payload + 5 + n + (n + 1) / 2 + s * 5;
  // header and entry are independent loads
  const unsigned int mode = payload[0];
  const unsigned long long count = (unsigned long long)payload[1] |
                                   ((unsigned long long)payload[2] << 8) |
                                   ((unsigned long long)payload[3] << 16) |
                                   ((unsigned long long)payload[4] << 24);
  const unsigned long long pos = (unsigned long long)e[0] | ((unsigned long long)e[1] << 8) |
                                 ((unsigned long long)e[2] << 16) |
                                 ((unsigned long long)e[3] << 24);
  const unsigned int exponent = e[4];
  if (mode != 5 || s >= count || pos >= n) return;
  const unsigned int b = payload[5 + pos];
  const unsigned int word = (b & 0x7F) | ((b & 0x80) << 8) | (exponent << 7);
  // written through like the tile kernels' output (after the kernel's last load):
  // the scattered 2-byte writes leave no dirty lines for the write-back at the
  // kernel's end (Llama-3-8B decode call 50.4 -> 50.3 us, step 3.166 -> 3.152 ms)
  const unsigned long long at =
      word_offset_by(a, d, pos, [&](unsigned long long j) { return block_of(d, j); });
  asm volatile("global_store_short %0, %1, off nt sc1" ::"v"(a.kv + at), "v"(word) : "memory");
}

__global__ __launch_bounds__(kThreads) void top16_patch_escapes(LaunchArgs a) {
  patch_escapes(a, [&](const PayloadDesc& d, unsigned long long j) {
    return a.ids ? (unsigned long long)a.ids[d.ids_offset + j] : a.block_start + j;
  });
}

__global__ __launch_bounds__(kThreads) void top16_patch_escapes_inline(LaunchArgs a,
                                                                       InlineBlocks table) {
  patch_escapes(a, [&](const PayloadDesc&, unsigned long long j) {
    return (unsigned long long)table.id[j];
  });
}

// ---------------------------------------------------------------------------
// host side

inline unsigned long long align_up(unsigned long long v, unsigned long long a) {
  return (v + a - 1) / a * a;
}

constexpr unsigned int kMinTileShift = kTileShift;
// The tile kernels use 32-bit in-plane word arithmetic.
constexpr unsigned long long kTilePlaneLimit = 1ull << 31;

enum class Kernel { kTile, kLanes, kGeneric };

struct Plan {
  Kernel kernel;
  bool sequential;
  unsigned int tile_shift;
  bool per_plane;
};

inline unsigned int host_payload_tiles(unsigned long long n, bool per_plane,
                                       unsigned int shift) {
  const unsigned long long tile = 1ull << shift;
  if (per_plane) return 2u * (unsigned int)(((n >> 1) + tile - 1) >> shift);
  return (unsigned int)((n + tile - 1) >> shift);
}

// tile_ok: every wave's 1024 words lie in one block (block words a multiple of
// 1024) and the code table is dword aligned.
Plan make_plan(bool geometry_fast, bool tile_ok, bool sequential) {
  Plan p;
  p.sequential = sequential;
  p.tile_shift = kTileShift;
  if (geometry_fast && tile_ok && !sequential) {
    p.kernel = Kernel::kTile;
  } else {
    p.kernel = geometry_fast ? Kernel::kLanes : Kernel::kGeneric;
  }
  p.per_plane = geometry_fast;
  return p;
}

// Decode tiles every payload per plane.
Plan make_decode_plan(bool geometry_fast, bool tile_ok) {
  Plan p = make_plan(geometry_fast, tile_ok, false);
  p.per_plane = true;
  return p;
}

void apply_plan(LaunchArgs& a, const Plan& p) {
  a.tiles_per_plane_mode = p.per_plane ? 1 : 0;
  a.tile_shift = p.tile_shift;
}

long long check_launch(const char* what) {
  hipError_t st = hipGetLastError();
  if (st != hipSuccess) return fail(what, st);
  return 0;
}

// Encodes payloads a.p[0 .. a.payload_count) (descriptors and tiling set).
long long launch_encode(LaunchArgs& a, const EncodeGeom& g, const Plan& p, hipStream_t stream) {
  const dim3 block(kThreads);
  if (p.sequential) {
    if (p.kernel == Kernel::kGeneric)
      hipLaunchKernelGGL((top16_encode_lanes<false, true>), dim3(1), block, 0, stream, a, g);
    else
      hipLaunchKernelGGL((top16_encode_lanes<true, true>), dim3(1), block, 0, stream, a, g);
    return check_launch("top16_encode_lanes");
  }
  switch (p.kernel) {
    case Kernel::kTile:
      if (a.presence) {
        if (a.ids)
          hipLaunchKernelGGL((top16_encode_tile<true, true, false>), dim3(a.total_tiles), block,
                             0, stream, a, g);
        else
          hipLaunchKernelGGL((top16_encode_tile<false, true, false>), dim3(a.total_tiles), block,
                             0, stream, a, g);
      } else if (a.inbody_slots) {
        if (a.ids)
          hipLaunchKernelGGL((top16_encode_tile<true, false, true>), dim3(a.total_tiles), block,
                             0, stream, a, g);
        else
          hipLaunchKernelGGL((top16_encode_tile<false, false, true>), dim3(a.total_tiles), block,
                             0, stream, a, g);
      } else if (a.ids) {
        hipLaunchKernelGGL((top16_encode_tile<true, false, false>), dim3(a.total_tiles), block, 0,
                           stream, a, g);
      } else {
        hipLaunchKernelGGL((top16_encode_tile<false, false, false>), dim3(a.total_tiles), block,
                           0, stream, a, g);
      }
      break;
    case Kernel::kLanes:
      hipLaunchKernelGGL((top16_encode_lanes<true, false>), dim3(a.total_tiles), block, 0, stream,
                         a, g);
      break;
    case Kernel::kGeneric:
      hipLaunchKernelGGL((top16_encode_lanes<false, false>), dim3(a.total_tiles), block, 0,
                         stream, a, g);
      break;
  }
  if (long long rc = check_launch("top16_encode")) return rc;
  unsigned int max_tiles = 0;
  for (unsigned int r = 0; r < a.payload_count; ++r) {
    const unsigned int end = r + 1 < a.payload_count ? a.p[r + 1].tile_begin : a.total_tiles;
    max_tiles = std::max(max_tiles, end - a.p[r].tile_begin);
  }
  const bool large = max_tiles >= kFinLargeTiles;
  // a presence-mask encode (a layer that overflowed before: dense tiles
  // everywhere) spreads its placement over 32 groups per payload: 1 % outlier
  // layer encode call 109.2 -> 105.8 us (16 groups: 106.5 us). So does an encode of
  // one or two payloads of at least 1024 tiles (the drop-in per-request call),
  // whose escapes would otherwise be placed by 8 workgroups: 8.4 M-word request with
  // an escape every 200 words 32.3 -> 20.2 us, with the benchmark's natural escapes
  // 14.9 -> 15.5 us. (A 1 M-word layer with natural escapes, a launch-bound call,
  // keeps 8 groups: 8.3 us, 9.3 us with 32.)
  const bool few = a.payload_count <= 2 && max_tiles >= kFinFewTiles;
  const dim3 fin_grid(a.payload_count * ((a.presence || few) && !a.inbody_slots
                                             ? kFinPresenceGroups
                                             : large ? 16 : 8) +
                      (a.palette_info ? a.payload_count : 0));
  if (a.inbody_slots) {
    if (large)
      hipLaunchKernelGGL((top16_encode_finalize<16, true, kDenseItemsSparse>), fin_grid, block, 0,
                         stream, a);
    else
      hipLaunchKernelGGL((top16_encode_finalize<8, true, kDenseItemsSparse>), fin_grid, block, 0,
                         stream, a);
  } else if (a.presence && a.palette_info) {
    hipLaunchKernelGGL((top16_encode_finalize<kFinPresenceGroups, false, kDenseItemsDense, true>),
                       fin_grid, block, 0, stream, a);
  } else if (a.presence) {
    hipLaunchKernelGGL((top16_encode_finalize<kFinPresenceGroups, false, kDenseItemsDense>),
                       fin_grid, block, 0, stream, a);
  } else if (few) {
    hipLaunchKernelGGL((top16_encode_finalize<kFinPresenceGroups, false, kDenseItemsSparse>),
                       fin_grid, block, 0, stream, a);
  } else if (large) {
    hipLaunchKernelGGL((top16_encode_finalize<16, false, kDenseItemsSparse>), fin_grid, block, 0,
                       stream, a);
  } else {
    hipLaunchKernelGGL((top16_encode_finalize<8, false, kDenseItemsSparse>), fin_grid, block, 0,
                       stream, a);
  }
  if (long long rc = check_launch("top16_encode_finalize")) return rc;
  if (a.inbody_slots) {
    // the staging in the body bytes has been read: write the body
    if (p.kernel == Kernel::kTile) {
      const dim3 grid((a.total_tiles + kThreads / kWave - 1) / (kThreads / kWave));
      if (a.ids)
        hipLaunchKernelGGL(top16_body_tile<true>, grid, block, 0, stream, a, g);
      else
        hipLaunchKernelGGL(top16_body_tile<false>, grid, block, 0, stream, a, g);
      return check_launch("top16_body_tile");
    }
    if (p.kernel == Kernel::kGeneric)
      hipLaunchKernelGGL(top16_body_lanes<false>, dim3(a.total_tiles), block, 0, stream, a, g);
    else
      hipLaunchKernelGGL(top16_body_lanes<true>, dim3(a.total_tiles), block, 0, stream, a, g);
    return check_launch("top16_body_lanes");
  }
  return 0;
}

// `table`: the request's block table in the kernel arguments (one payload on the
// tile plan) instead of a.ids.
long long launch_decode(LaunchArgs& a, const EncodeGeom& g, const Plan& p, hipStream_t stream,
                        const InlineBlocks* table = nullptr) {
  const dim3 block(kThreads);
  if (a.dir_rec) {  // the host only passes a directory with the tile plan
    if (a.ids)
      hipLaunchKernelGGL(top16_decode_tile_dir<true>, dim3(a.total_tiles), block, 0, stream, a, g);
    else
      hipLaunchKernelGGL(top16_decode_tile_dir<false>, dim3(a.total_tiles), block, 0, stream, a, g);
    return check_launch("top16_decode_tile_dir");
  }
  switch (p.kernel) {
    case Kernel::kTile:
      if (table)
        hipLaunchKernelGGL(top16_decode_tile_inline, dim3(a.total_tiles), block, 0, stream, a, g,
                           *table);
      else if (a.ids)
        hipLaunchKernelGGL(top16_decode_tile<true>, dim3(a.total_tiles), block, 0, stream, a, g);
      else
        hipLaunchKernelGGL(top16_decode_tile<false>, dim3(a.total_tiles), block, 0, stream, a, g);
      break;
    case Kernel::kLanes:
      hipLaunchKernelGGL(top16_decode_lanes, dim3(a.total_tiles), block, 0, stream, a, g);
      break;
    case Kernel::kGeneric: {
      unsigned long long max_n = 0;
      for (unsigned int r = 0; r < a.payload_count; ++r)
        max_n = std::max(max_n, 2ull * a.p[r].block_count * a.block_words);
      const unsigned int blocks = (unsigned int)std::min<unsigned long long>(
          (max_n + kThreads - 1) / kThreads, 2048);
      hipLaunchKernelGGL(top16_decode_generic, dim3(std::max(blocks, 1u), a.payload_count), block,
                         0, stream, a);
      break;
    }
  }
  if (long long rc = check_launch("top16_decode")) return rc;
  unsigned long long groups = 0, first_groups = 0;
  bool uniform = true;
  for (unsigned int r = 0; r < a.payload_count; ++r) {
    const unsigned long long n =
        a.linear_words ? a.linear_words : 2ull * a.p[r].block_count * a.block_words;
    const unsigned long long own = (escape_capacity(n) + kThreads - 1) / kThreads;
    if (r == 0) first_groups = own;
    uniform = uniform && own == first_groups;
    a.p[r].slot_group_begin = (unsigned int)groups;
    groups += own;
  }
  // equal payloads: a workgroup finds its payload by one division
  a.uniform_slot_groups = uniform ? (unsigned int)first_groups : 0u;
  if (table)
    hipLaunchKernelGGL(top16_patch_escapes_inline, dim3((unsigned int)groups), block, 0, stream, a,
                       *table);
  else
    hipLaunchKernelGGL(top16_patch_escapes, dim3((unsigned int)groups), block, 0, stream, a);
  return check_launch("top16_patch_escapes");
}

unsigned long long workspace_words(unsigned long long tiles) {
  return tiles * (1ull + kStageSlots);
}

}  // namespace
}  // namespace unchainkv

using namespace unchainkv;

extern "C" const char* kvq_splitzip_last_error() { return g_last_error.c_str(); }

extern "C" long long kvq_splitzip_bf16_encode_top16(unsigned long long src_ptr,
                                                    unsigned long long dst_ptr,
                                                    unsigned long long count,
                                                    unsigned long long capacity,
                                                    unsigned long long tables_ptr,
                                                    unsigned long long stream_ptr) {
  // Preconditions and declines of kvq_splitzip_cuda.cu:385-395.
  if (src_ptr == 0 || dst_ptr == 0 || tables_ptr == 0 || count == 0 || count > 0xFFFFFFFFULL)
    return 0;
  const unsigned long long encoded = encoded_size(count);
  const unsigned long long scratch_offset = (encoded + 3) & ~3ULL;
  if (encoded >= count * 2 || scratch_offset + 2 * sizeof(unsigned int) > capacity) return 0;

  LaunchArgs a{};
  a.kv = reinterpret_cast<uint16_t*>(src_ptr);
  a.buf = reinterpret_cast<unsigned char*>(dst_ptr);
  a.tables = reinterpret_cast<const unsigned char*>(tables_ptr);
  a.linear_words = count;
  a.payload_count = 1;
  // 16-byte loads need halves made of whole 16-word lanes and an aligned source;
  // the contiguous source is addressed as one block per plane
  const bool geometry_fast = (count % 32 == 0) && (src_ptr % 16 == 0);
  a.plane_stride = count / 2;
  a.block_words = count / 2;
  a.block_stride = 0;
  a.block_start = 0;
  a.p[0].block_count = 1;
  const EncodeGeom g = make_geom(count / 2);
  const bool tile_ok = tables_ptr % 4 == 0 && (count / 2) % 1024 == 0;
  // Parallel tiles need a workspace for per-tile escape counts and staged escapes;
  // it lives in the caller's buffer past the payload when the capacity allows.
  // Without that room (the ABI only promises align4(E) + 8 bytes) the tiles are still
  // encoded in parallel: each stages its escape count and escapes in its own body
  // bytes, the finalize places them, and a last pass writes those body bytes from
  // the source (the first 512 of each tile after the tile kernel, the whole body
  // after the lanes kernels, whose tiles need 64 words for the staging); otherwise
  // one workgroup walks the tiles in order.
  Plan plan = make_plan(geometry_fast, tile_ok, false);
  unsigned int tiles = host_payload_tiles(count, plan.per_plane, plan.tile_shift);
  const unsigned long long ws_offset = align_up(dst_ptr + encoded, 16) - dst_ptr;
  const unsigned long long ws_bytes = workspace_words(tiles) * 4;
  if (tiles > 1 && ws_offset + ws_bytes <= capacity) {
    a.workspace = reinterpret_cast<unsigned int*>(dst_ptr + ws_offset);
  } else {
    const unsigned long long tile_words = 1ull << plan.tile_shift;
    const unsigned long long span = plan.per_plane ? count / 2 : count;
    const unsigned long long last = span % tile_words ? span % tile_words : tile_words;
    if (tiles > 1 && std::min(last, span) >= 64) {
      a.inbody_slots = kInBodySlots;  // 512 bytes: count + 127 escapes
    } else {
      plan = make_plan(geometry_fast, tile_ok, true);
      tiles = host_payload_tiles(count, plan.per_plane, plan.tile_shift);
    }
  }
  apply_plan(a, plan);
  a.total_tiles = tiles;
  long long rc = launch_encode(a, g, plan, reinterpret_cast<hipStream_t>(stream_ptr));
  if (rc < 0) return rc;
  return (long long)encoded;
}

namespace unchainkv {
namespace {

// One payload's decode + scatter; the block table from block_ids_ptr (device),
// host_ids (host, carried in the kernel arguments: tile plan only, else declined),
// or neither (block_start + j).
long long decode_top16_one(unsigned long long src_ptr, unsigned long long encoded_bytes,
                           unsigned long long dst_ptr, unsigned long long count_words,
                           unsigned long long block_count, unsigned long long block_words,
                           unsigned long long plane_stride, unsigned long long block_stride,
                           unsigned long long block_start, unsigned long long block_ids_ptr,
                           const long long* host_ids, unsigned long long tables_ptr,
                           unsigned long long stream_ptr) {
  // Preconditions of kvq_splitzip_cuda.cu:423-432.
  if (src_ptr == 0 || dst_ptr == 0 || tables_ptr == 0 || count_words == 0 || block_count == 0 ||
      block_words == 0 || count_words != 2 * block_count * block_words)
    return 0;
  if (encoded_bytes != encoded_size(count_words)) return 0;
  if (block_count > 0xFFFFFFFFULL || block_words > 0xFFFFFFFFULL)
    return fail_msg("decode_top16: block_count and block_words must fit in 32 bits");

  LaunchArgs a{};
  a.kv = reinterpret_cast<uint16_t*>(dst_ptr);
  a.ids = reinterpret_cast<const long long*>(block_ids_ptr);
  a.buf = reinterpret_cast<unsigned char*>(src_ptr);
  a.tables = reinterpret_cast<const unsigned char*>(tables_ptr);
  a.plane_stride = plane_stride;
  a.block_stride = block_stride;
  a.block_words = block_words;
  a.block_start = block_start;
  a.payload_count = 1;
  a.p[0].block_count = (unsigned int)block_count;
  const bool geometry_fast = block_words % 16 == 0 && dst_ptr % 16 == 0 && plane_stride % 8 == 0 &&
                             block_stride % 8 == 0 && (count_words >> 1) <= 0xFFFFFFFFULL;
  const Plan plan = make_decode_plan(geometry_fast, tables_ptr % 4 == 0 && block_words % 1024 == 0 &&
                                                        (count_words >> 1) < kTilePlaneLimit);
  apply_plan(a, plan);
  a.total_tiles = host_payload_tiles(count_words, true, plan.tile_shift);
  InlineBlocks table{};
  if (host_ids) {
    if (plan.kernel != Kernel::kTile || block_count > kInlineBlocks) return 0;
    for (unsigned long long j = 0; j < block_count; ++j) {
      if (host_ids[j] < 0 || host_ids[j] > 0xFFFFFFFFll) return 0;
      table.id[j] = (unsigned int)host_ids[j];
    }
  }
  long long rc = launch_decode(a, make_geom(block_words), plan,
                               reinterpret_cast<hipStream_t>(stream_ptr),
                               host_ids ? &table : nullptr);
  if (rc < 0) return rc;
  return (long long)(count_words * sizeof(uint16_t));
}

}  // namespace
}  // namespace unchainkv

extern "C" long long kvq_splitzip_bf16_decode_top16_blocks(
    unsigned long long src_ptr, unsigned long long encoded_bytes, unsigned long long dst_ptr,
    unsigned long long count_words, unsigned long long block_count,
    unsigned long long block_words, unsigned long long plane_stride,
    unsigned long long block_stride, unsigned long long block_start,
    unsigned long long block_ids_ptr, unsigned long long tables_ptr,
    unsigned long long stream_ptr) {
  return decode_top16_one(src_ptr, encoded_bytes, dst_ptr, count_words, block_count, block_words,
                          plane_stride, block_stride, block_start, block_ids_ptr, nullptr,
                          tables_ptr, stream_ptr);
}

extern "C" long long kvq_splitzip_bf16_decode_top16_host_blocks(
    unsigned long long src_ptr, unsigned long long encoded_bytes, unsigned long long dst_ptr,
    unsigned long long count_words, unsigned long long block_count,
    unsigned long long block_words, unsigned long long plane_stride,
    unsigned long long block_stride, const long long* host_block_ids,
    unsigned long long tables_ptr, unsigned long long stream_ptr) {
  if (host_block_ids == nullptr) return 0;
  return decode_top16_one(src_ptr, encoded_bytes, dst_ptr, count_words, block_count, block_words,
                          plane_stride, block_stride, 0, 0, host_block_ids, tables_ptr,
                          stream_ptr);
}

extern "C" long long kvq_splitzip_bf16_decode_top16(
    unsigned long long src_ptr, unsigned long long encoded_bytes, unsigned long long dst_ptr,
    unsigned long long count_words, unsigned long long block_count,
    unsigned long long block_words, unsigned long long plane_stride,
    unsigned long long block_stride, unsigned long long block_start,
    unsigned long long tables_ptr, unsigned long long stream_ptr) {
  return kvq_splitzip_bf16_decode_top16_blocks(src_ptr, encoded_bytes, dst_ptr, count_words,
                                               block_count, block_words, plane_stride,
                                               block_stride, block_start, 0, tables_ptr,
                                               stream_ptr);
}

// ---------------------------------------------------------------------------
// batched paged entry points (no counterpart in the reference: it encodes one
// gathered request per call)

extern "C" unsigned long long kvq_splitzip_top16_paged_workspace_bytes(
    unsigned long long block_words, const unsigned long long* block_offsets,
    unsigned long long payload_count) {
  if (block_offsets == nullptr) return 0;
  unsigned long long tiles = 0;
  for (unsigned long long r = 0; r < payload_count; ++r) {
    if (block_offsets[r + 1] <= block_offsets[r]) return 0;  // refused by the encode too
    const unsigned long long n = 2 * (block_offsets[r + 1] - block_offsets[r]) * block_words;
    // the smallest tile of any plan bounds the tile count
    tiles += host_payload_tiles(n, true, kMinTileShift);
  }
  return workspace_words(tiles) * 4;
}

// Escape directory bytes of a batch (0 when block_words is not a multiple of 1024,
// the geometry of the tile kernels, which alone read and write a directory).
extern "C" unsigned long long kvq_splitzip_top16_paged_directory_bytes(
    unsigned long long block_words, const unsigned long long* block_offsets,
    unsigned long long payload_count) {
  if (block_offsets == nullptr || block_words == 0 || block_words % 1024 != 0) return 0;
  unsigned long long tiles = 0;
  for (unsigned long long r = 0; r < payload_count; ++r) {
    if (block_offsets[r + 1] <= block_offsets[r]) return 0;
    tiles += host_payload_tiles(2 * (block_offsets[r + 1] - block_offsets[r]) * block_words, true,
                                kTileShift);
  }
  return tiles * kDirBytesPerTile;
}

namespace {

// Points launch `a` (whose first tile is call tile `tile_offset`) at its part of a
// call's directory of `call_tiles` tiles: the chunk records of every tile, then
// the tile base slots.
void set_directory(LaunchArgs& a, unsigned long long directory_ptr, unsigned long long call_tiles,
                   unsigned long long tile_offset) {
  if (directory_ptr == 0) return;
  uint32_t* dir = reinterpret_cast<uint32_t*>(directory_ptr);
  a.dir_rec = dir + 16 * tile_offset;
  a.dir_base = dir + 16 * call_tiles + tile_offset;
}

struct PagedGeometry {
  unsigned long long kv_ptr, plane_stride, block_stride, block_words, ids_ptr;
};

bool paged_fast(const PagedGeometry& pg) {
  return pg.block_words % 16 == 0 && pg.kv_ptr % 16 == 0 && pg.plane_stride % 8 == 0 &&
         pg.block_stride % 8 == 0;
}

// Fills a.p for payloads [first, first + count) and returns the tile total.
unsigned int fill_descs(LaunchArgs& a, const PagedGeometry& pg,
                        const unsigned long long* block_offsets,
                        const unsigned long long* buf_offsets, unsigned long long first,
                        unsigned int count, const Plan& plan) {
  unsigned int tiles = 0;
  bool uniform = true;
  for (unsigned int k = 0; k < count; ++k) {
    const unsigned long long r = first + k;
    const unsigned long long nblk = block_offsets[r + 1] - block_offsets[r];
    a.p[k].buf_offset = buf_offsets[r];
    a.p[k].ids_offset = block_offsets[r];
    a.p[k].block_count = (unsigned int)nblk;
    a.p[k].tile_begin = tiles;
    tiles += host_payload_tiles(2 * nblk * pg.block_words, plan.per_plane, plan.tile_shift);
    uniform = uniform && nblk == block_offsets[first + 1] - block_offsets[first];
  }
  a.payload_count = count;
  a.total_tiles = tiles;
  // every payload has the same tile count: the kernels find a tile's payload by
  // one division instead of a search of the descriptors
  a.uniform_tiles = uniform ? tiles / count : 0;
  // ... and its block-table offset by one multiplication, when the block tables
  // are laid out back to back (as the host's block_offsets are)
  const unsigned long long nblk0 = block_offsets[first + 1] - block_offsets[first];
  bool packed = uniform;
  for (unsigned int k = 0; k < count && packed; ++k)
    packed = block_offsets[first + k] == block_offsets[first] + k * nblk0;
  a.uniform_blocks = packed && block_offsets[first] == 0 ? (unsigned int)nblk0 : 0;
  return tiles;
}

}  // namespace

namespace {

// Gathers and encodes payload r = blocks ids[block_offsets[r] .. block_offsets[r+1])
// of one paged layer into out + out_offsets[r], for every r, in one launch per 64
// payloads, with the workspace at workspace_ptr. Returns the total encoded bytes, 0
// on a failed precondition (a workspace smaller than the batch needs included), or
// -1 with the error recorded.
long long encode_top16_paged_impl(
    unsigned long long kv_ptr, unsigned long long plane_stride, unsigned long long block_stride,
    unsigned long long block_words, unsigned long long block_ids_ptr,
    const unsigned long long* block_offsets, unsigned long long payload_count,
    unsigned long long out_ptr, const unsigned long long* out_offsets,
    unsigned long long out_capacity, unsigned long long tables_ptr,
    unsigned long long workspace_ptr, unsigned long long workspace_bytes,
    unsigned long long directory_ptr, unsigned long long presence_ptr,
    unsigned long long stream_ptr, unsigned long long info_ptr = 0) {
  if (info_ptr != 0 && (presence_ptr == 0 || info_ptr % 16 != 0)) return 0;
  if (kv_ptr == 0 || block_ids_ptr == 0 || out_ptr == 0 || tables_ptr == 0 || workspace_ptr == 0 ||
      block_offsets == nullptr || out_offsets == nullptr || payload_count == 0 || block_words == 0 ||
      block_words > 0xFFFFFFFFULL)
    return 0;
  unsigned long long total = 0;
  std::vector<std::pair<unsigned long long, unsigned long long>> spans;
  spans.reserve(payload_count);
  for (unsigned long long r = 0; r < payload_count; ++r) {
    if (block_offsets[r + 1] <= block_offsets[r]) return 0;
    const unsigned long long n = 2 * (block_offsets[r + 1] - block_offsets[r]) * block_words;
    const unsigned long long e = encoded_size(n);
    if (n > 0xFFFFFFFFULL || e >= 2 * n || out_offsets[r] + e > out_capacity) return 0;
    spans.emplace_back(out_offsets[r], out_offsets[r] + e);
    total += e;
  }
  std::sort(spans.begin(), spans.end());
  for (size_t k = 1; k < spans.size(); ++k)
    if (spans[k].first < spans[k - 1].second) return 0;  // overlapping payloads
  if (kvq_splitzip_top16_paged_workspace_bytes(block_words, block_offsets, payload_count) >
      workspace_bytes)
    return 0;
  if (workspace_ptr % 4 != 0) return 0;

  const PagedGeometry pg{kv_ptr, plane_stride, block_stride, block_words, block_ids_ptr};
  const Plan plan =
      make_plan(paged_fast(pg), tables_ptr % 4 == 0 && block_words % 1024 == 0, false);
  const unsigned long long dir_tiles =
      kvq_splitzip_top16_paged_directory_bytes(block_words, block_offsets, payload_count) /
      kDirBytesPerTile;
  // a directory and presence masks are written by the tile kernels only
  if (directory_ptr != 0 && (plan.kernel != Kernel::kTile || directory_ptr % 16 != 0 ||
                             dir_tiles == 0))
    return 0;
  if (presence_ptr != 0 && (plan.kernel != Kernel::kTile || presence_ptr % 16 != 0)) return 0;
  const EncodeGeom g = make_geom(block_words);
  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_ptr);
  unsigned int* ws = reinterpret_cast<unsigned int*>(workspace_ptr);
  unsigned long long tile_offset = 0;
  for (unsigned long long first = 0; first < payload_count; first += kMaxPayloads) {
    LaunchArgs a{};
    a.kv = reinterpret_cast<uint16_t*>(kv_ptr);
    a.ids = reinterpret_cast<const long long*>(block_ids_ptr);
    a.buf = reinterpret_cast<unsigned char*>(out_ptr);
    a.tables = reinterpret_cast<const unsigned char*>(tables_ptr);
    a.plane_stride = plane_stride;
    a.block_stride = block_stride;
    a.block_words = block_words;
    apply_plan(a, plan);
    const unsigned int count =
        (unsigned int)std::min<unsigned long long>(kMaxPayloads, payload_count - first);
    const unsigned int tiles = fill_descs(a, pg, block_offsets, out_offsets, first, count, plan);
    a.workspace = ws;
    set_directory(a, directory_ptr, dir_tiles, tile_offset);
    if (presence_ptr) a.presence = reinterpret_cast<uint32_t*>(presence_ptr) + 8 * tile_offset;
    if (info_ptr) a.palette_info = reinterpret_cast<PaletteInfo*>(info_ptr) + first;
    long long rc = launch_encode(a, g, plan, stream);
    if (rc < 0) return rc;
    ws += workspace_words(tiles);
    tile_offset += tiles;
  }
  return (long long)total;
}

// ---------------------------------------------------------------------------
// Library-owned scratch for the entry point that allocates nothing: the encode's
// per-tile escape counts and staged escapes live in this array instead of a
// caller workspace. Each GPU holds its own copy for the life of the process; its
// device address is looked up once per device (the array's host-side name is not
// a device address) and every call on that GPU shares it.
constexpr unsigned long long kStaticScratchBytes = 16ull << 20;
constexpr int kMaxDevices = 64;
static __device__ __align__(256) unsigned char scratch[kStaticScratchBytes];

std::mutex g_scratch_mutex;
unsigned long long g_scratch_ptr[kMaxDevices];  // 0: not looked up yet

// Device address of `scratch` on the device that runs `stream` (0 on failure, with
// the error recorded).
unsigned long long scratch_address(hipStream_t stream) {
  int device = 0;
  hipError_t st = stream ? hipStreamGetDevice(stream, &device) : hipGetDevice(&device);
  if (st != hipSuccess) {
    fail("encode_top16_paged_noalloc: device of the stream", st);
    return 0;
  }
  if (device < 0 || device >= kMaxDevices) {
    fail_msg("encode_top16_paged_noalloc: device index out of range");
    return 0;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_ptr[device] == 0) {
    int current = 0;
    st = hipGetDevice(&current);
    if (st == hipSuccess && current != device) st = hipSetDevice(device);
    void* ptr = nullptr;
    if (st == hipSuccess) st = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (current != device) (void)hipSetDevice(current);
    if (st != hipSuccess || ptr == nullptr) {
      fail("encode_top16_paged_noalloc: scratch address", st);
      return 0;
    }
    g_scratch_ptr[device] = reinterpret_cast<unsigned long long>(ptr);
  }
  return g_scratch_ptr[device];
}

}  // namespace

extern "C" long long kvq_splitzip_bf16_encode_top16_paged(
    unsigned long long kv_ptr, unsigned long long plane_stride, unsigned long long block_stride,
    unsigned long long block_words, unsigned long long block_ids_ptr,
    const unsigned long long* block_offsets, unsigned long long payload_count,
    unsigned long long out_ptr, const unsigned long long* out_offsets,
    unsigned long long out_capacity, unsigned long long tables_ptr,
    unsigned long long workspace_ptr, unsigned long long workspace_bytes,
    unsigned long long directory_ptr, unsigned long long stream_ptr) {
  return encode_top16_paged_impl(kv_ptr, plane_stride, block_stride, block_words, block_ids_ptr,
                                 block_offsets, payload_count, out_ptr, out_offsets,
                                 out_capacity, tables_ptr, workspace_ptr, workspace_bytes,
                                 directory_ptr, 0, stream_ptr);
}

extern "C" unsigned long long kvq_splitzip_top16_paged_presence_bytes(
    unsigned long long block_words, const unsigned long long* block_offsets,
    unsigned long long payload_count) {
  if (block_offsets == nullptr || block_words == 0 || block_words % 1024 != 0) return 0;
  unsigned long long tiles = 0;
  for (unsigned long long r = 0; r < payload_count; ++r) {
    if (block_offsets[r + 1] <= block_offsets[r]) return 0;
    tiles += host_payload_tiles(2 * (block_offsets[r + 1] - block_offsets[r]) * block_words, true,
                                kTileShift);
  }
  return 32 * tiles;
}

extern "C" long long kvq_splitzip_bf16_encode_top16_paged_presence(
    unsigned long long kv_ptr, unsigned long long plane_stride, unsigned long long block_stride,
    unsigned long long block_words, unsigned long long block_ids_ptr,
    const unsigned long long* block_offsets, unsigned long long payload_count,
    unsigned long long out_ptr, const unsigned long long* out_offsets,
    unsigned long long out_capacity, unsigned long long tables_ptr,
    unsigned long long workspace_ptr, unsigned long long workspace_bytes,
    unsigned long long directory_ptr, unsigned long long presence_ptr,
    unsigned long long stream_ptr) {
  if (presence_ptr == 0) return 0;
  return encode_top16_paged_impl(kv_ptr, plane_stride, block_stride, block_words, block_ids_ptr,
                                 block_offsets, payload_count, out_ptr, out_offsets,
                                 out_capacity, tables_ptr, workspace_ptr, workspace_bytes,
                                 directory_ptr, presence_ptr, stream_ptr);
}

extern "C" long long kvq_splitzip_bf16_encode_top16_paged_probe(
    unsigned long long kv_ptr, unsigned long long plane_stride, unsigned long long block_stride,
    unsigned long long block_words, unsigned long long block_ids_ptr,
    const unsigned long long* block_offsets, unsigned long long payload_count,
    unsigned long long out_ptr, const unsigned long long* out_offsets,
    unsigned long long out_capacity, unsigned long long tables_ptr,
    unsigned long long workspace_ptr, unsigned long long workspace_bytes,
    unsigned long long directory_ptr, unsigned long long presence_ptr,
    unsigned long long palette_info_ptr, unsigned long long stream_ptr) {
  if (presence_ptr == 0 || palette_info_ptr == 0) return 0;
  return encode_top16_paged_impl(kv_ptr, plane_stride, block_stride, block_words, block_ids_ptr,
                                 block_offsets, payload_count, out_ptr, out_offsets,
                                 out_capacity, tables_ptr, workspace_ptr, workspace_bytes,
                                 directory_ptr, presence_ptr, stream_ptr, palette_info_ptr);
}

extern "C" unsigned long long kvq_splitzip_top16_noalloc_scratch_bytes() {
  return kStaticScratchBytes;
}

extern "C" long long kvq_splitzip_bf16_encode_top16_paged_noalloc(
    unsigned long long kv_ptr, unsigned long long plane_stride, unsigned long long block_stride,
    unsigned long long block_words, unsigned long long block_ids_ptr,
    const unsigned long long* block_offsets, unsigned long long payload_count,
    unsigned long long out_ptr, const unsigned long long* out_offsets,
    unsigned long long out_capacity, unsigned long long tables_ptr,
    unsigned long long directory_ptr, unsigned long long stream_ptr) {
  // the workspace entry point's checks of the host arrays first, so that a bad
  // batch declines with 0 as it does there (the device pointers are checked there)
  if (block_offsets == nullptr || out_offsets == nullptr || payload_count == 0 ||
      block_words == 0 || block_words > 0xFFFFFFFFULL)
    return 0;
  for (unsigned long long r = 0; r < payload_count; ++r)
    if (block_offsets[r + 1] <= block_offsets[r]) return 0;
  {
    const unsigned long long need =
        kvq_splitzip_top16_paged_workspace_bytes(block_words, block_offsets, payload_count);
    if (need > kStaticScratchBytes)
      return fail_msg("encode_top16_paged_noalloc: the batch needs " + std::to_string(need) +
                      " bytes of scratch, above the library's fixed " +
                      std::to_string(kStaticScratchBytes) + " bytes; split the batch");
  }
  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_ptr);
  const unsigned long long ws = scratch_address(stream);
  if (ws == 0) return -1;
  return encode_top16_paged_impl(kv_ptr, plane_stride, block_stride, block_words, block_ids_ptr,
                                 block_offsets, payload_count, out_ptr, out_offsets,
                                 out_capacity, tables_ptr, ws, kStaticScratchBytes,
                                 directory_ptr, 0, stream_ptr);
}

// Decodes payload r (src + src_offsets[r], encoded_bytes[r] long) and scatters it
// into blocks ids[block_offsets[r] .. block_offsets[r+1]) of one paged layer.
// Returns the total raw bytes written, 0 on a failed precondition, -1 on error.
extern "C" long long kvq_splitzip_bf16_decode_top16_paged(
    unsigned long long src_ptr, const unsigned long long* src_offsets,
    const unsigned long long* encoded_bytes, unsigned long long payload_count,
    unsigned long long kv_ptr, unsigned long long plane_stride, unsigned long long block_stride,
    unsigned long long block_words, unsigned long long block_ids_ptr,
    const unsigned long long* block_offsets, unsigned long long tables_ptr,
    unsigned long long directory_ptr, unsigned long long stream_ptr) {
  if (src_ptr == 0 || kv_ptr == 0 || block_ids_ptr == 0 || tables_ptr == 0 ||
      src_offsets == nullptr || encoded_bytes == nullptr || block_offsets == nullptr ||
      payload_count == 0 || block_words == 0 || block_words > 0xFFFFFFFFULL)
    return 0;
  unsigned long long total = 0, max_plane = 0;
  for (unsigned long long r = 0; r < payload_count; ++r) {
    if (block_offsets[r + 1] <= block_offsets[r]) return 0;
    const unsigned long long n = 2 * (block_offsets[r + 1] - block_offsets[r]) * block_words;
    if (encoded_bytes[r] != encoded_size(n) || (n >> 1) > 0xFFFFFFFFULL) return 0;
    total += 2 * n;
    max_plane = std::max(max_plane, n >> 1);
  }
  const PagedGeometry pg{kv_ptr, plane_stride, block_stride, block_words, block_ids_ptr};
  const Plan plan = make_decode_plan(
      paged_fast(pg),
      tables_ptr % 4 == 0 && block_words % 1024 == 0 && max_plane < kTilePlaneLimit);
  const unsigned long long dir_tiles =
      kvq_splitzip_top16_paged_directory_bytes(block_words, block_offsets, payload_count) /
      kDirBytesPerTile;
  if (directory_ptr != 0 && (plan.kernel != Kernel::kTile || directory_ptr % 16 != 0 ||
                             dir_tiles == 0))
    return 0;
  const EncodeGeom g = make_geom(block_words);
  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_ptr);
  unsigned long long tile_offset = 0;
  for (unsigned long long first = 0; first < payload_count; first += kMaxPayloads) {
    LaunchArgs a{};
    a.kv = reinterpret_cast<uint16_t*>(kv_ptr);
    a.ids = reinterpret_cast<const long long*>(block_ids_ptr);
    a.buf = reinterpret_cast<unsigned char*>(src_ptr);
    a.tables = reinterpret_cast<const unsigned char*>(tables_ptr);
    a.plane_stride = plane_stride;
    a.block_stride = block_stride;
    a.block_words = block_words;
    apply_plan(a, plan);
    const unsigned int count =
        (unsigned int)std::min<unsigned long long>(kMaxPayloads, payload_count - first);
    const unsigned int tiles = fill_descs(a, pg, block_offsets, src_offsets, first, count, plan);
    set_directory(a, directory_ptr, dir_tiles, tile_offset);
    long long rc = launch_decode(a, g, plan, stream);
    if (rc < 0) return rc;
    tile_offset += tiles;
  }
  return (long long)total;
}

// ---------------------------------------------------------------------------
// host-built escape directory (payloads that arrive in host memory)

extern "C" long long kvq_splitzip_top16_build_directory(
    unsigned char* host_buf, const unsigned long long* offsets,
    const unsigned long long* encoded_bytes, unsigned long long payload_count,
    unsigned long long block_words, const unsigned long long* block_offsets,
    unsigned char* host_directory, unsigned long long directory_bytes) {
  if (host_buf == nullptr || offsets == nullptr || encoded_bytes == nullptr ||
      host_directory == nullptr || payload_count == 0)
    return 0;
  const unsigned long long need =
      kvq_splitzip_top16_paged_directory_bytes(block_words, block_offsets, payload_count);
  if (need == 0 || need > directory_bytes) return 0;
  for (unsigned long long r = 0; r < payload_count; ++r) {
    const unsigned long long n = 2 * (block_offsets[r + 1] - block_offsets[r]) * block_words;
    if (encoded_bytes[r] != encoded_size(n)) return 0;
  }
  const unsigned long long call_tiles = need / kDirBytesPerTile;
  uint32_t* rec = reinterpret_cast<uint32_t*>(host_directory);
  uint32_t* tile_base = rec + 16 * call_tiles;
  std::fill(rec, rec + 17 * call_tiles, 0u);

  std::vector<std::pair<uint32_t, uint8_t>> list;
  unsigned long long tile0 = 0;  // call tile of the payload's first tile
  for (unsigned long long r = 0; r < payload_count; ++r) {
    const unsigned long long n = 2 * (block_offsets[r + 1] - block_offsets[r]) * block_words;
    const unsigned long long half = n / 2;
    const unsigned long long tpp = (half + kTileWords - 1) / kTileWords;
    unsigned char* payload = host_buf + offsets[r];
    const unsigned long long cap = escape_capacity(n);
    unsigned long long count = (unsigned long long)payload[1] | (payload[2] << 8) |
                               ((unsigned long long)payload[3] << 16) |
                               ((unsigned long long)payload[4] << 24);
    count = std::min(count, cap);
    if (payload[0] == 5 && count != 0) {
      // the list in position order (stable: a repeated position keeps its order, so
      // the last entry still wins as it would in slot order)
      unsigned char* entries = payload + 5 + n + (n + 1) / 2;
      list.resize(count);
      for (unsigned long long s = 0; s < count; ++s) {
        uint32_t pos;
        std::memcpy(&pos, entries + 5 * s, 4);
        list[s] = {pos, entries[5 * s + 4]};
      }
      std::stable_sort(list.begin(), list.end(),
                       [](const std::pair<uint32_t, uint8_t>& x,
                          const std::pair<uint32_t, uint8_t>& y) { return x.first < y.first; });
      for (unsigned long long s = 0; s < count; ++s) {
        std::memcpy(entries + 5 * s, &list[s].first, 4);
        entries[5 * s + 4] = list[s].second;
      }
      // entries at or beyond n are not applied and sort last
      unsigned long long slot = 0;
      for (unsigned long long j = 0; j < 2 * tpp; ++j) {
        tile_base[tile0 + j] = (uint32_t)slot;
        const unsigned long long plane = j >= tpp ? 1 : 0;
        const unsigned long long lo = plane * half + (j - plane * tpp) * kTileWords;
        const unsigned long long hi = std::min(lo + kTileWords, (plane + 1) * half);
        const unsigned long long first_slot = slot;
        while (slot < count && list[slot].first < hi) {
          const unsigned long long local = list[slot].first - lo;  // tile-local position
          uint32_t* c = rec + 16 * (tile0 + j) + 4 * (local >> 10);
          const uint32_t k = c[0] >> 16;
          if (k == 0) c[0] = (uint32_t)(slot - first_slot);
          if (k < (uint32_t)kDirInline) c[1 + k] = (uint32_t)(local << 8) | list[slot].second;
          c[0] = (c[0] & 0xFFFFu) | ((k + 1) << 16);
          ++slot;
        }
      }
    }
    tile0 += 2 * tpp;
  }
  return (long long)need;
}
