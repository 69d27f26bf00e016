// Shared device helpers for the splitzip bf16 codec kernels (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <string>

namespace unchainkv {

// Error reporting shared by every C entry point: the message is kept per host
// thread and returned by kvq_splitzip_last_error().
long long fail(const char* what, hipError_t status);
long long fail_msg(const std::string& msg);

constexpr int kThreads = 256;                         // 4 waves of 64
constexpr int kWave = 64;
// Lane-run kernels: each lane owns 16 consecutive words (any alignment).
constexpr int kWordsPerLane = 16;
constexpr int kTileWords = kThreads * kWordsPerLane;  // 4096 words per workgroup tile
constexpr int kTileShift = 12;
static_assert((1 << kTileShift) == kTileWords, "tile size");

// Escapes staged per tile by the encode kernel (3.1% of a 4096-word tile, three
// times the 0.5% escape capacity of a payload, so that a payload with 1% outliers
// rarely has a tile to re-scan); tiles with more are re-scanned by the finalize
// kernel.
constexpr int kStageSlots = 128;
// Escapes staged in a tile's own first 512 body bytes after its u32 count, when
// a drop-in encode has no room for a workspace.
constexpr unsigned int kInBodySlots = kStageSlots - 1;
// Payload descriptors passed by value in the kernel arguments.
constexpr int kMaxPayloads = 64;

// Per-payload palette of the fixed6 / fixed5 codecs, from the OR of the payload's
// high-byte presence masks (palette_info_from_masks).
struct PaletteInfo {
  unsigned int mask[8];     // presence of each high byte
  unsigned int distinct;    // number of distinct high bytes
  unsigned int pad0[7];
  unsigned char rank[256];  // high byte -> code (0 for absent bytes)
  unsigned char palette[64];
  unsigned char pad1[128];
};
static_assert(sizeof(PaletteInfo) == 512, "palette info");

struct PayloadDesc {
  unsigned long long buf_offset;  // byte offset of the payload inside the payload buffer
  unsigned long long ids_offset;  // first block id of this payload inside `ids`
  unsigned int block_count;       // blocks per plane
  unsigned int tile_begin;        // first tile of this payload within the launch
  unsigned int slot_group_begin;  // first escape-patch workgroup of this payload
  unsigned int mask_begin;        // palette codecs: first high-byte presence mask
};
static_assert(sizeof(PayloadDesc) == 32, "payload descriptor");

// One launch covers up to kMaxPayloads payloads of one paged layer (or one
// contiguous payload). Word i of a payload lives at
//   kv[p * plane_stride + block(j) * block_stride + within]
// with p = i / plane_words, j = (i % plane_words) / block_words, within =
// i % block_words, block(j) = ids[ids_offset + j] or block_start + j, and
// plane_words = block_count * block_words. `linear` payloads are contiguous
// (word i at kv[i]) with the K/V split at n / 2 for any n.
struct LaunchArgs {
  uint16_t* kv;
  const long long* ids;
  unsigned char* buf;
  const unsigned char* tables;  // 544 B: [p*256+exp] -> code, then 2 x 16 codebook bytes
  unsigned int* workspace;      // encode: per-tile escape counts, then staged escapes
  unsigned long long plane_stride;
  unsigned long long block_stride;
  unsigned long long block_words;
  unsigned long long block_start;
  unsigned long long linear_words;  // n of a linear payload, else 0
  unsigned int payload_count;
  unsigned int total_tiles;
  unsigned int tiles_per_plane_mode;  // 1: tiles never cross a plane (fast path); 0: one range [0, n)
  unsigned int tile_shift;            // log2 of the tile size in words
  unsigned int uniform_tiles;         // tiles of every payload when all are equal, else 0
  unsigned int uniform_slot_groups;   // escape-patch workgroups of every payload, likewise
  unsigned int uniform_blocks;        // blocks per plane of every payload when uniform_tiles
  // Drop-in encode without room for a workspace: 0, or the escapes staged per tile
  // inside the tile's own body bytes (u32 count, then staged entries), which the
  // body pass writes last (top16_body_lanes).
  unsigned int inbody_slots;
  // Escape directory of the launch's tiles (Top-16 tile kernels only; null when
  // absent): per 1024-word wave chunk of tile t a record dir_rec[4 * (4t + wave)
  // .. + 4) = {tile-relative slot of the chunk's first escape | chunk escapes << 16,
  // up to kDirInline of them as (tile-local position << 8 | exponent)}, and per
  // tile dir_base[t] = payload slot of the tile's first escape.
  uint32_t* dir_rec;
  uint32_t* dir_base;
  // 256-bit presence mask of the high bytes of each of the launch's tiles, written
  // by the Top-16 tile kernel when not null (8 dwords per tile): the palette
  // fallback encode of an overflowed payload then starts from these masks instead
  // of reading the words again.
  uint32_t* presence;
  // Palette of each payload of the launch, computed from its presence masks by the
  // Top-16 probe encode's finalize launch (null otherwise); the fixed6 / fixed5
  // re-encode of an overflowed payload then starts from it.
  PaletteInfo* palette_info;
  PayloadDesc p[kMaxPayloads];
};

// Escapes of a wave chunk held in its directory record.
constexpr int kDirInline = 3;
// Directory bytes per tile: four 16-byte chunk records and the tile's base slot.
constexpr unsigned long long kDirBytesPerTile = 4 * 16 + 4;

// ---------------------------------------------------------------------------
// streaming (nontemporal) vector memory access: the codec reads its source once
// and writes its destination once, so neither should displace cached data.

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

template <typename T>
__device__ __forceinline__ T load_stream(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const T*>(p));
}
template <typename T>
__device__ __forceinline__ void store_stream(void* p, T v) {
  __builtin_nontemporal_store(v, reinterpret_cast<T*>(p));
}
__device__ __forceinline__ u32x4 load_stream16(const void* p) { return load_stream<u32x4>(p); }
__device__ __forceinline__ u32x2 load_stream8(const void* p) { return load_stream<u32x2>(p); }
__device__ __forceinline__ uint32_t load_stream4(const void* p) { return load_stream<uint32_t>(p); }
// Streaming stores that also write through to the device's coherence point
// (cache policy nt sc1): a tile kernel that writes its whole output this way
// leaves little dirty data in L2 for the write-back at its end, so the kernel
// that follows it starts sooner (Llama-3-8B encode call 49.5 -> 48.7 us). No
// builtin sets sc1 on a vector store, hence the inline assembly; the compiler's
// memory-counter waits do not see these stores, so a kernel issues them only
// after its last global load.
__device__ __forceinline__ void store_through16(void* p, u32x4 v) {
  asm volatile("global_store_dwordx4 %0, %1, off nt sc1" ::"v"(p), "v"(v) : "memory");
}
__device__ __forceinline__ void store_through8(void* p, u32x2 v) {
  asm volatile("global_store_dwordx2 %0, %1, off nt sc1" ::"v"(p), "v"(v) : "memory");
}
__device__ __forceinline__ void store_through4(void* p, uint32_t v) {
  asm volatile("global_store_dword %0, %1, off nt sc1" ::"v"(p), "v"(v) : "memory");
}
__device__ __forceinline__ void store_stream16(void* p, u32x4 v) { store_stream<u32x4>(p, v); }
__device__ __forceinline__ void store_stream8(void* p, u32x2 v) { store_stream<u32x2>(p, v); }
__device__ __forceinline__ void store_stream4(void* p, uint32_t v) { store_stream<uint32_t>(p, v); }

// ---------------------------------------------------------------------------
// launch-shape helpers

// Workgroups are handed to the 8 XCDs round-robin; remap so each XCD walks a
// contiguous run of tiles (neighbouring tiles share partial cache lines).
__device__ __forceinline__ unsigned int xcd_remap(unsigned int wg, unsigned int count) {
  unsigned int q = count >> 3, rem = count & 7, xcd = wg & 7, local = wg >> 3;
  return xcd * q + min(xcd, rem) + local;
}

// Payload of a (wave-uniform) tile. Equal-size payloads: one division. Otherwise
// lane k reads payload k's first tile (kMaxPayloads == wave size) and a ballot
// counts the payloads that start at or before the tile: one round trip instead of
// a chain of dependent loads. Every lane of the wave must be active.
static_assert(kMaxPayloads == 64, "one payload descriptor per lane");
__device__ __forceinline__ unsigned int find_payload(const LaunchArgs& a, unsigned int tile) {
  if (a.uniform_tiles) return tile / a.uniform_tiles;
  if (a.payload_count <= 1) return 0;
  const unsigned int lane = __lane_id();
  const unsigned int begin = lane < a.payload_count ? a.p[lane].tile_begin : 0xFFFFFFFFu;
  const unsigned long long starts = __ballot(begin <= tile);
  return __builtin_amdgcn_readfirstlane((unsigned int)__popcll(starts) - 1u);
}

// Same search over the escape-patch workgroups of each payload.
__device__ __forceinline__ unsigned int find_slot_payload(const LaunchArgs& a, unsigned int group) {
  if (a.uniform_slot_groups) return group / a.uniform_slot_groups;
  if (a.payload_count <= 1) return 0;
  const unsigned int lane = __lane_id();
  const unsigned int begin =
      lane < a.payload_count ? a.p[lane].slot_group_begin : 0xFFFFFFFFu;
  const unsigned long long starts = __ballot(begin <= group);
  return __builtin_amdgcn_readfirstlane((unsigned int)__popcll(starts) - 1u);
}

__device__ __forceinline__ unsigned long long payload_words(const LaunchArgs& a,
                                                            const PayloadDesc& d) {
  return a.linear_words ? a.linear_words : 2ull * d.block_count * a.block_words;
}

// Tiles of payload d: planes are tiled separately when tiles_per_plane_mode is set
// (so a tile never crosses the K/V split), else [0, n) is tiled as one range.
__device__ __forceinline__ unsigned int tiles_per_plane(const LaunchArgs& a,
                                                        unsigned long long plane_words) {
  return (unsigned int)((plane_words + (1ull << a.tile_shift) - 1) >> a.tile_shift);
}

__device__ __forceinline__ void tile_range(const LaunchArgs& a, const PayloadDesc& d,
                                           unsigned int local_tile, unsigned long long n,
                                           unsigned long long& start, unsigned long long& end) {
  if (a.tiles_per_plane_mode) {
    unsigned long long plane_words = n >> 1;
    unsigned int tpp = tiles_per_plane(a, plane_words);
    unsigned int plane = local_tile >= tpp ? 1u : 0u;
    const unsigned long long tile = 1ull << a.tile_shift;
    start = plane * plane_words + ((unsigned long long)(local_tile - plane * tpp) << a.tile_shift);
    unsigned long long stop = (plane + 1ull) * plane_words;
    end = start + tile < stop ? start + tile : stop;
  } else {
    const unsigned long long tile = 1ull << a.tile_shift;
    start = (unsigned long long)local_tile << a.tile_shift;
    end = start + tile < n ? start + tile : n;
  }
}

__device__ __forceinline__ unsigned int payload_tiles(const LaunchArgs& a, unsigned long long n) {
  if (a.tiles_per_plane_mode) return 2u * tiles_per_plane(a, n >> 1);
  return (unsigned int)((n + (1ull << a.tile_shift) - 1) >> a.tile_shift);
}

// Element offset of payload word i in the KV cache (any geometry).
// Element offset of word i with the payload's j-th block from block_of(j).
template <typename BlockOf>
__device__ __forceinline__ unsigned long long word_offset_by(const LaunchArgs& a,
                                                             const PayloadDesc& d,
                                                             unsigned long long i,
                                                             BlockOf block_of) {
  if (a.linear_words) return i;
  unsigned long long plane_words = (unsigned long long)d.block_count * a.block_words;
  unsigned long long plane = i / plane_words;
  unsigned long long in_plane = i - plane * plane_words;
  unsigned long long j = in_plane / a.block_words;
  unsigned long long within = in_plane - j * a.block_words;
  return plane * a.plane_stride + block_of(j) * a.block_stride + within;
}

__device__ __forceinline__ unsigned long long word_offset(const LaunchArgs& a,
                                                          const PayloadDesc& d,
                                                          unsigned long long i) {
  return word_offset_by(a, d, i, [&](unsigned long long j) {
    return a.ids ? (unsigned long long)a.ids[d.ids_offset + j] : a.block_start + j;
  });
}

// ---------------------------------------------------------------------------
// tile geometry shared by the tile kernels of both codecs

// q = x / d for x, d < 2^32 via m = floor(2^64 / d) + 1 (exact for every 32-bit x).
struct Divider {
  unsigned long long m;
  unsigned int d;
};

inline Divider make_divider(unsigned int d) {
  Divider r;
  r.d = d;
  r.m = d <= 1 ? 0 : (~0ull / d) + 1;
  return r;
}

__device__ __forceinline__ unsigned int div_u32(unsigned int x, unsigned long long m,
                                                unsigned int d) {
  return d <= 1 ? x : (unsigned int)__umul64hi((unsigned long long)x, m);
}


struct EncodeGeom {
  unsigned long long bw_magic;  // divider for block_words
  unsigned int bw;
};


#ifndef UKV_XCD_REMAP
#define UKV_XCD_REMAP 1
#endif

// Index of this workgroup's tile (XCD-aware: each XCD walks a contiguous run).
__device__ __forceinline__ unsigned int group_index() {
#if UKV_XCD_REMAP
  return xcd_remap(blockIdx.x, gridDim.x);
#else
  return blockIdx.x;
#endif
}

// Scalar (SGPR) copies of wave-uniform values.
__device__ __forceinline__ unsigned int uniform(unsigned int v) {
  return __builtin_amdgcn_readfirstlane(v);
}
__device__ __forceinline__ unsigned long long uniform64(unsigned long long v) {
  return ((unsigned long long)__builtin_amdgcn_readfirstlane((unsigned int)(v >> 32)) << 32) |
         __builtin_amdgcn_readfirstlane((unsigned int)v);
}

// One 4096-word tile of the per-plane tiling that the tile kernels use. In-plane
// arithmetic is 32-bit (the host only picks these kernels for plane words < 2^31)
// and free of branches on the launch layout, so the kernel-argument loads of the
// prologue can be issued together.
struct PlaneTile {
  unsigned long long n;   // payload words
  unsigned char* payload;
  const long long* ids;   // the payload's block table (when there is one)
  unsigned int plane;
  unsigned int in_plane0;  // first word of the tile within its plane
  unsigned int words;      // words in the tile: a multiple of 1024, at most the tile size
  unsigned int local_tile;
  unsigned int payload_tiles;
  unsigned int payload_index;  // index of the payload within the launch
};

// With equal payloads whose block tables lie back to back, the payload's tile and
// block-table offsets follow from its index, so the block-id load that gates a
// wave's source address does not wait for the payload descriptor.
template <int kShift>
__device__ __forceinline__ PlaneTile plane_tile(const LaunchArgs& a, unsigned int tile) {
  constexpr unsigned int kWords = 1u << kShift;
  const unsigned int ut = a.uniform_tiles, ub = a.uniform_blocks;
  const unsigned int bw = (unsigned int)a.block_words;
  const long long* const ids = a.ids;
  unsigned char* const buf = a.buf;
  PlaneTile t;
  unsigned int block_count, tile_begin;
  unsigned long long ids_offset;
  if (ut != 0 && ub != 0) {
    t.payload_index = tile / ut;
    block_count = ub;
    tile_begin = t.payload_index * ut;
    ids_offset = (unsigned long long)t.payload_index * ub;
  } else {
    t.payload_index = find_payload(a, tile);
    const PayloadDesc d = a.p[t.payload_index];
    block_count = d.block_count;
    tile_begin = d.tile_begin;
    ids_offset = d.ids_offset;
  }
  const unsigned int plane_words = block_count * bw;
  const unsigned int tpp = (plane_words + kWords - 1) >> kShift;
  t.local_tile = tile - tile_begin;
  t.plane = t.local_tile >= tpp ? 1u : 0u;
  t.in_plane0 = (t.local_tile - t.plane * tpp) << kShift;
  t.words = min(kWords, plane_words - t.in_plane0);
  t.n = 2ull * plane_words;
  t.payload = buf + a.p[t.payload_index].buf_offset;
  t.ids = ids + ids_offset;
  t.payload_tiles = 2 * tpp;
  return t;
}

// Wave-uniform element offset in the layer of in-plane word `in_plane` of tile t,
// with the payload's j-th block from block_of(j).
template <typename BlockOf>
__device__ __forceinline__ unsigned long long wave_offset_by(const LaunchArgs& a,
                                                             const PlaneTile& t,
                                                             const EncodeGeom& geo,
                                                             unsigned int in_plane,
                                                             BlockOf block_of) {
  const unsigned int j = uniform(div_u32(in_plane, geo.bw_magic, geo.bw));
  const unsigned int within = in_plane - j * geo.bw;
  const unsigned long long blk = block_of(j);
  return uniform64(t.plane * a.plane_stride + uniform64(blk) * a.block_stride + within);
}

// The same with the block from the payload's block table, or block_start + j
// without one.
template <bool kIds>
__device__ __forceinline__ unsigned long long wave_source(const LaunchArgs& a, const PlaneTile& t,
                                                          const EncodeGeom& geo,
                                                          unsigned int in_plane) {
  return wave_offset_by(a, t, geo, in_plane, [&](unsigned int j) {
    return kIds ? (unsigned long long)t.ids[j] : a.block_start + j;
  });
}

// A request's block table of at most kInlineBlocks ids carried in the kernel
// arguments: a table that is a host list then needs no copy to the device before
// the decode (its ids are read with scalar loads from the kernel-argument segment).
constexpr unsigned int kInlineBlocks = 256;
struct InlineBlocks {
  unsigned int id[kInlineBlocks];
};


inline EncodeGeom make_geom(unsigned long long block_words) {
  EncodeGeom g{};
  const Divider dv = make_divider((unsigned int)(block_words > 1 ? block_words : 1));
  g.bw = dv.d;
  g.bw_magic = dv.m;
  return g;
}


// ---------------------------------------------------------------------------
// byte-window helpers: c[] holds consecutive little-endian dwords; take 4 (or 2)
// dwords starting at byte offset off (wave-uniform, 0 <= off < 16 or < 8).

__device__ __forceinline__ uint32_t funnel(uint32_t lo, uint32_t hi, uint32_t r) {
  return (uint32_t)((((uint64_t)hi << 32) | lo) >> (8 * r));
}

template <int Q>
__device__ __forceinline__ void window4_q(const uint32_t (&c)[8], uint32_t r, uint32_t (&o)[4]) {
#pragma unroll
  for (int k = 0; k < 4; ++k) o[k] = funnel(c[Q + k], c[Q + k + 1], r);
}

__device__ __forceinline__ void window4(const uint32_t (&c)[8], uint32_t off, uint32_t (&o)[4]) {
  uint32_t r = off & 3;
  switch (off >> 2) {
    case 0: window4_q<0>(c, r, o); break;
    case 1: window4_q<1>(c, r, o); break;
    case 2: window4_q<2>(c, r, o); break;
    default: window4_q<3>(c, r, o); break;
  }
}

__device__ __forceinline__ void window2(const uint32_t (&c)[4], uint32_t off, uint32_t (&o)[2]) {
  uint32_t r = off & 3;
  if (off >> 2) {
    o[0] = funnel(c[1], c[2], r);
    o[1] = funnel(c[2], c[3], r);
  } else {
    o[0] = funnel(c[0], c[1], r);
    o[1] = funnel(c[1], c[2], r);
  }
}

__device__ __forceinline__ uint32_t shfl_next(uint32_t v) {
  // value of the next lane in the wave (lane 63 receives its own value)
  return (uint32_t)__shfl_down((int)v, 1, kWave);
}

__device__ __forceinline__ uint32_t byte_of(const uint32_t* v, int k) {
  return (v[k >> 2] >> (8 * (k & 3))) & 0xFF;
}

// Writes `count` bytes of v (starting at byte `first` of the dword array) to dst.
__device__ __forceinline__ void store_bytes(unsigned char* dst, const uint32_t* v, int first,
                                            int count) {
  for (int k = 0; k < count; ++k) dst[k] = (unsigned char)byte_of(v, first + k);
}

// Wave-wide inclusive prefix sum.
__device__ __forceinline__ uint32_t wave_inclusive_sum(uint32_t v) {
  const int lane = threadIdx.x & (kWave - 1);
#pragma unroll
  for (int d = 1; d < kWave; d <<= 1) {
    uint32_t t = (uint32_t)__shfl_up((int)v, d, kWave);
    if (lane >= d) v += t;
  }
  return v;
}

// ---------------------------------------------------------------------------
// Top-16 decode of 8 words in registers (the decode tile kernels and the fused
// attention)

// Per-byte 0xFF/0x00 masks from bit 3 of each byte of s (byte permute with the
// sign-replicating selectors 8-11).
__device__ __forceinline__ uint32_t bit3_mask(uint32_t s) {
  return __builtin_amdgcn_perm(s << 12, s << 4, 0x090B080Au);
}

// Exponents of four 4-bit codes (one per byte of s) from a 16-byte codebook held
// in four dwords: two byte permutes (codes 0-7 and 8-15) merged by bit 3.
__device__ __forceinline__ uint32_t codebook_lookup4(uint32_t s, const uint32_t (&cb)[4]) {
  const uint32_t s7 = s & 0x07070707u;
  const uint32_t lo = __builtin_amdgcn_perm(cb[1], cb[0], s7);
  const uint32_t hi = __builtin_amdgcn_perm(cb[3], cb[2], s7);
  const uint32_t mask = bit3_mask(s);
  return (hi & mask) | (lo & ~mask);
}

// Two decoded words from bytes [b0, e0, b1, e1] (body byte, exponent): mantissa
// from b, exponent into bits 7-14, b's bit 7 into the sign bit 15.
__device__ __forceinline__ uint32_t assemble_pair(uint32_t x) {
  const uint32_t y = (x & 0x007F007Fu) | ((x >> 1) & ~0x007F007Fu);
  return ((x << 8) & 0x80008000u) | (y & ~0x80008000u);
}

// Decodes one 8-word run: 8 body bytes (2 dwords) and 4 code bytes -> 4 dwords.
__device__ __forceinline__ u32x4 decode_run8(u32x2 body, uint32_t cd, const uint32_t (&cb)[4]) {
  const uint32_t u = cd >> 4;
  // codes of the 8 words as bytes (low nibble first)
  const uint32_t sa = __builtin_amdgcn_perm(u, cd, 0x05010400u) & 0x0F0F0F0Fu;
  const uint32_t sb = __builtin_amdgcn_perm(u, cd, 0x07030602u) & 0x0F0F0F0Fu;
  const uint32_t ea = codebook_lookup4(sa, cb);
  const uint32_t eb = codebook_lookup4(sb, cb);
  return u32x4{assemble_pair(__builtin_amdgcn_perm(ea, body.x, 0x05010400u)),
               assemble_pair(__builtin_amdgcn_perm(ea, body.x, 0x07030602u)),
               assemble_pair(__builtin_amdgcn_perm(eb, body.y, 0x05010400u)),
               assemble_pair(__builtin_amdgcn_perm(eb, body.y, 0x07030602u))};
}

// Workgroup-cooperative: OR of `count` 32-byte presence masks at `masks` -> the
// palette record `out` (ascending palette, rank table, distinct count). Thread tid
// ORs whole masks tid, tid + 256, ... (four loads in flight), then the wave by
// shuffles and the workgroup through LDS (s_mask, 8 dwords).
__device__ __forceinline__ void palette_info_from_masks(const unsigned int* masks,
                                                        unsigned long long count,
                                                        PaletteInfo& out, unsigned int* s_mask) {
  const unsigned int tid = threadIdx.x;
  if (tid < 8) s_mask[tid] = 0;
  __syncthreads();
  u32x4 lo = {0, 0, 0, 0}, hi = {0, 0, 0, 0};
  const u32x4* m4 = reinterpret_cast<const u32x4*>(masks);
  for (unsigned long long s = tid; s < count; s += 4 * kThreads) {
    u32x4 a[4], b[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const unsigned long long slot = s + (unsigned long long)k * kThreads;
      a[k] = slot < count ? m4[2 * slot] : u32x4{0, 0, 0, 0};
      b[k] = slot < count ? m4[2 * slot + 1] : u32x4{0, 0, 0, 0};
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      lo |= a[k];
      hi |= b[k];
    }
  }
  // one LDS atomic per wave and dword (an atomic from every lane compiles to a loop
  // over the active lanes)
  unsigned int part[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
#pragma unroll
  for (int k = 0; k < 8; ++k)
#pragma unroll
    for (int off = kWave / 2; off > 0; off >>= 1) part[k] |= __shfl_xor(part[k], off, kWave);
  if ((tid & (kWave - 1)) == 0) {
#pragma unroll
    for (int k = 0; k < 8; ++k)
      if (part[k]) atomicOr(&s_mask[k], part[k]);
  }
  __syncthreads();
  unsigned int distinct = 0;
#pragma unroll
  for (int k = 0; k < 8; ++k) distinct += __popc(s_mask[k]);
  if (tid < 8) out.mask[tid] = s_mask[tid];
  if (tid == 0) out.distinct = distinct;
  // code of high byte h = number of present bytes below h (ascending palette)
  const unsigned int h = tid;
  unsigned int rank = __popc(s_mask[h >> 5] & ((1u << (h & 31)) - 1u));
  for (unsigned int k = 0; k < (h >> 5); ++k) rank += __popc(s_mask[k]);
  const bool present = (s_mask[h >> 5] >> (h & 31)) & 1u;
  out.rank[h] = (unsigned char)(present ? rank : 0);
  if (tid < 64) out.palette[tid] = 0;
  __syncthreads();
  // (a palette of more than 32 entries is an overflow for fixed5, which reads 32)
  if (present && rank < 64) out.palette[rank] = (unsigned char)h;
}

}  // namespace unchainkv
