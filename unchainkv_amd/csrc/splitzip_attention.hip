// Fused Top-16 decode + paged decode attention (one query token per sequence),
// gfx950.
//
// The KV of each sequence is one Top-16 payload (mode 5) of its K plane then its V
// plane, words ordered [token][kv head][dim] (what the batched encoder produces for
// a sequence's block table in token order). The kernel never materialises bf16 KV
// in HBM: it reads the packed body and code bytes once, decodes 16-token steps into
// LDS, patches the step's escapes there, and runs QK^T and PV on the MFMA units
// with an online softmax.
//
// Work split (flash-decoding): one workgroup per (sequence, context split, pair of
// kv heads); waves 0-1 walk two consecutive token ranges of the split for the first
// head, waves 2-3 the same ranges for the second (the two heads' rows of a token
// are adjacent in the payload and are read together), with a workgroup barrier
// every second step. Per 16-token step a wave decodes K and V into its LDS (lane l:
// tokens l/8 and l/8 + 8, dims 16*(l%8) .. +15, so 8 lanes read a token's row),
// patches the step's escapes there, and then:
//   * S^T = K Q^T on v_mfma_f32_16x16x32_bf16 with K as the A operand (rows =
//     tokens, lane l reads row l%16) and the GQA group's 4 query heads as B
//     columns, which leaves lane l with tokens 4*(l/16)+j of head l%16;
//   * online softmax in f32 (the column max over the lane groups by gfx950's
//     VALU row swaps);
//   * O += P V on the 16-block v_mfma_f32_4x4x4_16b_bf16: block b makes O[4 heads]
//     [dims 4b..4b+3] (+64 for the second half) over 4 tokens per instruction, its
//     A operand P broadcast from the lanes that hold it (cbsz 4, abid 4g for token
//     group g) and its B operand (4 tokens of one dim) read from the token-major V
//     in LDS by the transposing ds_read_b64_tr_b16. The accumulators hold O's 4
//     query rows only (8 VGPRs; the 16-row MFMA tiles used before held 12 padding
//     rows in 24 more), which keeps the kernel at 4 waves per SIMD.
// The waves' softmax states are merged in LDS; a second kernel merges the splits
// and writes bf16.
//
// Escapes: the kernel needs the escape list in ascending position order (what the
// encoder of this library writes; the reference's encoder appends escapes in
// atomic order, so its lists may be unordered). Each wave finds its first K and V
// escape with a 64-way search and then walks the list with its steps, one 64-entry
// window per plane. The search and the walk are only meaningful on an ordered
// list, so the list's order is checked as well: the split kernel's workgroups of a
// sequence share the check of every neighbouring pair of entries between them. A
// decrease anywhere in the list, or a payload whose byte 0 is not 5, makes every
// output of the sequence NaN (the combine kernel looks at all of the sequence's
// partials) rather than silently wrong.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <mutex>

#include "splitzip_common.h"

namespace unchainkv {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kHeadDim = 128;
constexpr int kGroup = 4;                   // query heads per kv head
constexpr int kStep = 16;                   // tokens per wave step
// u16 per row of sK and sV: 288-byte rows (16-byte aligned for the b128 accesses).
// The padding spreads the LDS banks of the 16 rows one MFMA operand read spans: on
// the Llama-3-8B decode step, unpadded 256-byte rows ran 10 us slower; with the
// chunk order below, 272- and 288-byte rows run alike (before it, 288 was 3 us
// ahead). Longer rows would not leave room for 4 workgroups per CU.
constexpr int kKStride = kHeadDim + 16;

// Position in an LDS row of dim d: the row's 8-dim (16-byte) chunks are stored even
// chunks first, then odd ones (chunk c in slot (c >> 1) | (c & 1) << 3), so that the
// 8 lanes of one decode store, which hold chunks 2p (then 2p + 1), write 128
// contiguous bytes. Reads take whole chunks, or 4 dims inside one.
__device__ __forceinline__ constexpr unsigned int row_pos(unsigned int d) {
  return ((((d >> 3) >> 1) | (((d >> 3) & 1u) << 3)) << 3) | (d & 7u);
}
constexpr int kWaveLds = 2 * kStep * kKStride;  // u16 per wave: K and V of a step, token-major
constexpr int kMaxSeqs = 64;                // sequences per launch (kernel arguments)
constexpr int kPartial = kHeadDim + 2;      // m, l, acc[128] per (split, query head)
constexpr int kMaxSplits = 64;
constexpr int kCheck = 8;                   // escape-order pairs per thread held through the walk
// Independent accumulator chains of the PV product: one chain keeps the kernel at
// 125 VGPRs (4 waves per SIMD); two reached 128 with a spill and ran 1 us slower.
constexpr int kPvChains = 1;
static_assert(4 * kGroup * kPartial * 4 <= 4 * kWaveLds * 2, "merge area fits the wave LDS");

struct AttnArgs {
  const uint16_t* q;             // [batch][q_heads][128] bf16
  uint16_t* out;                 // [batch][q_heads][128] bf16
  const unsigned char* payloads;
  const unsigned char* tables;   // 544 B; K codebook at +512, V at +528
  float* partial;                // [batch][kv_heads][splits][kGroup][kPartial]
  unsigned int batch, q_heads, kv_heads, splits, tokens_per_wave;
  float scale_log2;              // scale * log2(e)
  unsigned int head_magic;       // 2^24 / kv_heads + 1
  unsigned long long offset[kMaxSeqs];  // payload byte offset of each sequence
  unsigned int ctx[kMaxSeqs];           // context tokens of each sequence
  unsigned int span[kMaxSeqs];          // tokens the payload holds (whole blocks, >= ctx)
};

__device__ __forceinline__ unsigned int bf16_bits(float v) {
  return __builtin_bit_cast(unsigned short, (__bf16)v);  // round to nearest even
}

// Decode table of one plane in LDS: entry x (a byte of two 4-bit codes, even word
// in the low nibble) = (cb[x & 15] << 7) | (cb[x >> 4] << 23), i.e. both words'
// exponents already in place inside a dword of two bf16 words.
__device__ __forceinline__ uint32_t table_entry(const unsigned char* cb, unsigned int x) {
  return ((uint32_t)cb[x & 15] << 7) | ((uint32_t)cb[x >> 4] << 23);
}

// 8 words (4 dwords of bf16 pairs) from 8 body bytes (mantissa | sign << 7) and 4
// code bytes: exponent bits 7..14 of each word come from the table, bits 0..6 and
// 15 from the body byte repeated into both bytes of its word.
__device__ __forceinline__ void decode8(uint32_t b0, uint32_t b1, uint32_t cd,
                                        const uint32_t* tab, uint32_t* o) {
  constexpr uint32_t kExp = 0x7F807F80u;
  const uint32_t t0 = tab[cd & 0xFFu], t1 = tab[(cd >> 8) & 0xFFu];
  const uint32_t t2 = tab[(cd >> 16) & 0xFFu], t3 = tab[cd >> 24];
  o[0] = (t0 & kExp) | (__builtin_amdgcn_perm(b0, b0, 0x01010000u) & ~kExp);
  o[1] = (t1 & kExp) | (__builtin_amdgcn_perm(b0, b0, 0x03030202u) & ~kExp);
  o[2] = (t2 & kExp) | (__builtin_amdgcn_perm(b1, b1, 0x01010000u) & ~kExp);
  o[3] = (t3 & kExp) | (__builtin_amdgcn_perm(b1, b1, 0x03030202u) & ~kExp);
}

// Position (u32 LE) of escape entry i by one unaligned dword load (entries are
// 5 bytes apart; the load stays inside the entry).
typedef unsigned int u32_unaligned __attribute__((aligned(1)));
__device__ __forceinline__ unsigned int entry_pos(const unsigned char* entries, unsigned int i) {
  return *reinterpret_cast<const u32_unaligned*>(entries + 5u * i);
}

// Packed bytes of one lane's share of a step, per plane: 16 body bytes (mantissa |
// sign << 7) and 8 code bytes of 16 consecutive words of each of two tokens.
// Lane l takes tokens l/8 and l/8 + 8 of the step, dims 16*(l%8) .. +15, so that
// 8 consecutive lanes read a token's whole 128-byte body row and 64-byte code row.
struct RawShare {
  u32x4 kb[2], vb[2];
  u32x2 kc[2], vc[2];
};

// Section starts of one payload (wave-uniform, so the loads take a scalar base and
// a 32-bit per-lane offset): K plane body and codes, V plane body and codes.
struct PlaneBases {
  const unsigned char* kb;
  const unsigned char* kc;
  const unsigned char* vb;
  const unsigned char* vc;
};

// `w0`, `w1` = word of the share's first K word within its plane, for each token
// (even: a token row and a lane's share are whole code bytes). Every lane loads (no
// branch): a lane whose token is past the range passes a clamped, in-range token
// instead and its words are ignored.
__device__ __forceinline__ RawShare load_share(const PlaneBases& pb, unsigned int w0,
                                               unsigned int w1) {
  RawShare r;
  r.kb[0] = load_stream16(pb.kb + w0);
  r.kb[1] = load_stream16(pb.kb + w1);
  r.kc[0] = load_stream8(pb.kc + (w0 >> 1));
  r.kc[1] = load_stream8(pb.kc + (w1 >> 1));
  r.vb[0] = load_stream16(pb.vb + w0);
  r.vb[1] = load_stream16(pb.vb + w1);
  r.vc[0] = load_stream8(pb.vc + (w0 >> 1));
  r.vc[1] = load_stream8(pb.vc + (w1 >> 1));
  return r;
}

// First indices in [0, count) whose positions are >= target_k and >= target_v
// (entries ascending): lanes 0-31 search for target_k and lanes 32-63 for target_v
// at once, 32 ways per round, so that both searches share each memory round trip.
// Results uniform across the wave.
__device__ uint2 lower_bound_escapes2(const unsigned char* entries, unsigned int count,
                                      unsigned int target_k, unsigned int target_v) {
  const unsigned int lane = __lane_id(), half = lane >> 5, sub = lane & 31;
  const unsigned int target = half ? target_v : target_k;
  unsigned int lo = 0, hi = count;  // uniform within each half
  for (;;) {
    const unsigned int span_k = __builtin_amdgcn_readlane(hi - lo, 0);
    const unsigned int span_v = __builtin_amdgcn_readlane(hi - lo, 32);
    if (span_k <= 32 && span_v <= 32) break;
    const unsigned int step = (hi - lo + 31) / 32;
    const unsigned int idx = lo + sub * step;
    const bool below = idx < hi && entry_pos(entries, idx) < target;
    const unsigned int k = (unsigned int)__popcll((__ballot(below) >> (32 * half)) & 0xFFFFFFFFull);
    const unsigned int new_lo = k ? lo + (k - 1) * step + 1 : lo;
    const unsigned int new_hi = min(hi, lo + k * step);
    lo = new_lo;
    hi = max(new_hi, new_lo);
  }
  const unsigned int idx = lo + sub;
  const bool below = idx < hi && entry_pos(entries, idx) < target;
  const unsigned int r = lo + (unsigned int)__popcll((__ballot(below) >> (32 * half)) & 0xFFFFFFFFull);
  return uint2{__builtin_amdgcn_readlane(r, 0), __builtin_amdgcn_readlane(r, 32)};
}

// One 64-entry window of a plane's escape list (entry base + lane); positions past
// the list read as 0xFFFFFFFF.
struct Window {
  unsigned int pos, exp;
};

// Maximum of v over lanes l, l ^ 16, l ^ 32 and l ^ 48, on the VALU (gfx950 row
// swaps: max(r[0], r[1]) of a swap of v with itself is the lane pair's maximum).
__device__ __forceinline__ float max_over_lane_groups(float v) {
  const unsigned int u = __builtin_bit_cast(unsigned int, v);
  const auto a = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  v = fmaxf(__builtin_bit_cast(float, (unsigned int)a[0]), __builtin_bit_cast(float, (unsigned int)a[1]));
  const unsigned int w = __builtin_bit_cast(unsigned int, v);
  const auto b = __builtin_amdgcn_permlane32_swap(w, w, false, false);
  return fmaxf(__builtin_bit_cast(float, (unsigned int)b[0]), __builtin_bit_cast(float, (unsigned int)b[1]));
}

__device__ __forceinline__ Window load_window(const unsigned char* entries, unsigned int count,
                                              unsigned int i) {
  Window w{0xFFFFFFFFu, 0u};
  if (i < count) {
    w.pos = entry_pos(entries, i);
    w.exp = entries[5u * i + 4];
  }
  return w;
}

// Per-wave state of the walk over a token range.
struct WaveWalk {
  float m_run;      // running max (log2 units) of head l%16
  float l_run;      // this lane's share of the running sum of head l%16
  // O[head j][dim 64*half + l] = sum over k of acc[half + 2k][j]: token group g of
  // a step goes to acc[half + 2 (g % kPvChains)], so that with two chains no 4x4x4
  // MFMA waits for the one just before it
  f32x4 acc[2 * kPvChains];
  Window wk, wv;    // escape windows of the K and V planes
  unsigned int ptr_k, ptr_v;    // next entry of each plane's walk
  unsigned int base_k, base_v;  // entry index of each window's lane 0
  bool ok;
};

struct StepConst {
  const unsigned char* entries;
  unsigned int count, half, row_words, head, we, kv_heads, head_magic;
  float scale_log2;
  const uint32_t* tab_k;
  const uint32_t* tab_v;
  uint16_t* sK;
  uint16_t* sV;
};

// Applies the escapes of one plane that fall in tokens [ts, t_stop) to the wave's
// LDS copy of the step (`dst`: sK or sV) and advances the plane's list pointer past
// them. `base` is the plane's first position (0 or n/2). An escape at position
// lo + r (lo = the step's first position) belongs to step token x / kv_heads and
// head x % kv_heads, x = r >> 7; the quotient is (x * head_magic) >> 24, exact for
// x < 16 * kv_heads and kv_heads < 1024 (head_magic = 2^24 / kv_heads + 1). The
// exponent is replaced by two LDS atomics on the word's dword (and, or) that need
// no reply. Lane l of the window holds entry wbase + l; entries below ptr were
// taken by earlier steps; the window is reloaded when this step takes its last
// entry, and after the step once more than half of it is used. The list's order
// is checked once for the whole list (the walk assumes it ascending).
// Wave-uniform control flow.
__device__ __forceinline__ void apply_escapes(Window& win, unsigned int& ptr, unsigned int& wbase,
                                              const StepConst& c, unsigned int base,
                                              unsigned int ts, unsigned int t_stop,
                                              uint16_t* dst) {
  const unsigned int lane = __lane_id();
  const unsigned int lo = base + ts * c.row_words, hi = base + t_stop * c.row_words;
  for (;;) {
    const bool in = wbase + lane >= ptr && win.pos < hi;
    if (in) {
      const unsigned int r = win.pos - lo;
      const unsigned int x = r >> 7;  // step token * kv_heads + head
      const unsigned int tt = (x * c.head_magic) >> 24;
      if (x - tt * c.kv_heads == c.head) {
        const unsigned int word = tt * kKStride + row_pos(r & (kHeadDim - 1));
        const unsigned int shift = (word & 1u) * 16u;
        uint32_t* dw = reinterpret_cast<uint32_t*>(dst) + (word >> 1);
        __hip_atomic_fetch_and(dw, ~(0x7F80u << shift), __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_WAVEFRONT);
        __hip_atomic_fetch_or(dw, (win.exp << 7) << shift, __ATOMIC_RELAXED,
                              __HIP_MEMORY_SCOPE_WAVEFRONT);
      }
    }
    ptr += (unsigned int)__popcll(__ballot(in));
    if (ptr < wbase + 64) break;
    wbase = ptr;  // every entry of the window taken: more may be in range
    win = load_window(c.entries, c.count, ptr + lane);
  }
}

// O[head][dim] += P[head][t] V[t][dim] over the 4 tokens 4G .. 4G + 3 of the step,
// both halves of the dims (accumulators half + 2 * (G % kPvChains)). B operand by the transposing LDS read: within each
// 16-lane group, lane i receives element i % 4 of the 4-element rows that lanes
// 4j + i/4 read (j = 0..3); lane s of group q reads dims 64*half + 16q + 4*(s%4)
// .. + 3 of token 4G + s/4, so lane l ends up with dim 64*half + l of the 4 tokens.
template <int G>
__device__ __forceinline__ void pv_group(i16x4 pa, const uint16_t* sV, f32x4 (&acc)[2 * kPvChains]) {
  const unsigned int lane = __lane_id(), col = lane % 16, grp = lane / 16;
  const uint16_t* vrow = sV + (4 * G + col / 4) * kKStride;
#pragma unroll
  for (int half = 0; half < 2; ++half) {
    const uint16_t* vsrc = vrow + row_pos(64 * half + 16 * grp + 4 * (col % 4));
    const i16x4 vb = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) i16x4*)(vsrc));
    f32x4& o = acc[half + 2 * (G % kPvChains)];
    o = __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(pa, vb, o, 4, 4 * G, 0);
  }
}

// One 16-token step of a wave: decode into the wave's LDS, patch escapes, S^T on
// MFMA, online softmax, O += P V on MFMA.
__device__ __forceinline__ void attend_step(const RawShare& cur, unsigned int ts,
                                            const StepConst& c, const bf16x8 (&qb)[4],
                                            WaveWalk& w) {
  const unsigned int lane = __lane_id(), col = lane % 16, grp = lane / 16;
  const bool tail = ts + kStep > c.we;  // wave-uniform
  {
    const unsigned int tt0 = lane / 8, part = lane % 8;  // tokens tt0 and tt0 + 8
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const unsigned int tt = tt0 + 8 * i;
      uint32_t o[8];
      decode8(cur.kb[i].x, cur.kb[i].y, cur.kc[i].x, c.tab_k, o);
      decode8(cur.kb[i].z, cur.kb[i].w, cur.kc[i].y, c.tab_k, o + 4);
      // dims 16p .. 16p + 7 and 16p + 8 .. 16p + 15: chunks 2p and 2p + 1
      uint16_t* rowk = c.sK + tt * kKStride;
      *reinterpret_cast<u32x4*>(rowk + row_pos(part * 16)) = u32x4{o[0], o[1], o[2], o[3]};
      *reinterpret_cast<u32x4*>(rowk + row_pos(part * 16 + 8)) = u32x4{o[4], o[5], o[6], o[7]};
      decode8(cur.vb[i].x, cur.vb[i].y, cur.vc[i].x, c.tab_v, o);
      decode8(cur.vb[i].z, cur.vb[i].w, cur.vc[i].y, c.tab_v, o + 4);
      uint16_t* rowv = c.sV + tt * kKStride;
      *reinterpret_cast<u32x4*>(rowv + row_pos(part * 16)) = u32x4{o[0], o[1], o[2], o[3]};
      *reinterpret_cast<u32x4*>(rowv + row_pos(part * 16 + 8)) = u32x4{o[4], o[5], o[6], o[7]};
    }
  }
  if (tail) {
    // tokens past the range (their lanes decoded a clamped, in-range token without
    // its escapes): zero their V rows so that p = 0 cannot meet an Inf or NaN. The
    // stores sit behind the wave-uniform branch, so full steps skip them.
    const unsigned int tt0 = lane / 8, part = lane % 8;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const unsigned int tt = tt0 + 8 * i;
      if (ts + tt >= c.we) {
        uint16_t* rowv = c.sV + tt * kKStride;
        *reinterpret_cast<u32x4*>(rowv + row_pos(part * 16)) = u32x4{0u, 0u, 0u, 0u};
        *reinterpret_cast<u32x4*>(rowv + row_pos(part * 16 + 8)) = u32x4{0u, 0u, 0u, 0u};
      }
    }
  }

  // escapes of this step; then prefetch the windows of the next one
  const unsigned int t_stop = min(ts + kStep, c.we);
  apply_escapes(w.wk, w.ptr_k, w.base_k, c, 0u, ts, t_stop, c.sK);
  apply_escapes(w.wv, w.ptr_v, w.base_v, c, c.half, ts, t_stop, c.sV);
  if (w.ptr_k - w.base_k > 32) {
    w.base_k = w.ptr_k;
    w.wk = load_window(c.entries, c.count, w.ptr_k + lane);
  }
  if (w.ptr_v - w.base_v > 32) {
    w.base_v = w.ptr_v;
    w.wv = load_window(c.entries, c.count, w.ptr_v + lane);
  }
  // LDS accesses of one wave complete in order; this keeps the compiler from
  // moving the reads below above the writes
  __builtin_amdgcn_wave_barrier();

  // ---- S^T = K Q^T: lane l gets tokens 4*(l/16)+j of head l%16 ----
  f32x4 st = {0, 0, 0, 0};
  {
    const uint16_t* krow = c.sK + col * kKStride;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const bf16x8 ka = __builtin_bit_cast(
          bf16x8, *reinterpret_cast<const u32x4*>(krow + row_pos(grp * 32 + 8 * ks)));
      st = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ka, qb[ks], st, 0, 0, 0);
    }
  }
  // columns 4..15 (zero query rows) stay finite and only feed output rows that are
  // never read
  float sc[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) sc[j] = st[j] * c.scale_log2;
  if (tail) {
#pragma unroll
    for (int j = 0; j < 4; ++j) sc[j] = ts + grp * 4 + j < c.we ? sc[j] : -INFINITY;
  }
  float mloc = fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3]));
  mloc = max_over_lane_groups(mloc);
  const float m_new = fmaxf(w.m_run, mloc);  // finite: every step holds a token
  if (__ballot(m_new > w.m_run) & 0xFull) {
    // a head's max moved: rescale its sum share and its acc row
    const float alpha = __builtin_amdgcn_exp2f(w.m_run - m_new);
    w.l_run *= alpha;
    float al[4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
      al[j] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, alpha), j));
#pragma unroll
    for (int k = 0; k < 2 * kPvChains; ++k)
#pragma unroll
      for (int j = 0; j < 4; ++j) w.acc[k][j] *= al[j];
    w.m_run = m_new;
  }
  float p[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) p[j] = __builtin_amdgcn_exp2f(sc[j] - w.m_run);
  w.l_run += (p[0] + p[1]) + (p[2] + p[3]);

  // ---- O += P V on the 16-block 4x4x4 MFMA: block b (lanes 4b..4b+3) makes
  // O[4 heads][dims 64*half + 4b .. + 3] over 4 tokens per instruction. Lanes
  // 16g .. 16g + 3 (block 4g) hold P[head l%4][tokens 4g .. 4g + 3], the A operand
  // of token group g, which the instruction broadcasts to all 16 blocks (cbsz 4,
  // abid 4g); no accumulator register holds a padding row ----
  i16x4 pa;
#pragma unroll
  for (int j = 0; j < 4; ++j) pa[j] = (short)bf16_bits(p[j]);
  pv_group<0>(pa, c.sV, w.acc);
  pv_group<1>(pa, c.sV, w.acc);
  pv_group<2>(pa, c.sV, w.acc);
  pv_group<3>(pa, c.sV, w.acc);
  __builtin_amdgcn_wave_barrier();
}

// kWaves waves per workgroup serve kHeads consecutive kv heads, kRanges =
// kWaves / kHeads token ranges of each per context split. Measured on the
// Llama-3-8B decode step: 2 heads x 2 ranges ahead of 4 heads x 1 range (1.5 us)
// and of 8 heads x 1 range in 8-wave workgroups (6 us); 4 waves per SIMD (at most
// 128 VGPRs) ahead of 3 (6 us): the payload loads alone ran 134 against 152 us.
constexpr int kWaves = 4;
constexpr int kHeads = 2;
constexpr int kRanges = kWaves / kHeads;
constexpr int kT = 64 * kWaves;
static_assert(kRanges * kHeads == kWaves, "whole ranges per head");

__global__ __launch_bounds__(kT) __attribute__((amdgpu_waves_per_eu(4, 4))) void
top16_attention_split(AttnArgs a) {
  __shared__ __align__(16) uint16_t lds[kWaves * kWaveLds];
  __shared__ uint32_t sTab[2][256];
  __shared__ unsigned int sBad[kWaves];

  const unsigned int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  // work item = (sequence, split, head group) with the group fastest, each XCD
  // taking a contiguous run of items (xcd_remap). Waves r, r + kRanges, ... serve
  // range r of the group's heads: the heads' rows of one token are adjacent in the
  // payload (body kHeads * 128 bytes, codes kHeads * 64), which the group's waves
  // then read together.
  const unsigned int hkv = a.kv_heads;
  const unsigned int groups = (hkv + kHeads - 1) / kHeads;
  const unsigned int w_item = xcd_remap(blockIdx.x, gridDim.x);
  const unsigned int hg = w_item % groups;
  const unsigned int split = (w_item / groups) % a.splits;
  const unsigned int b = w_item / (groups * a.splits);
  const unsigned int h = kHeads * hg + wave / kRanges;
  const unsigned int range = wave % kRanges;
  const bool head_ok = h < hkv;  // the last group may be partly empty
  const unsigned int ctx = a.ctx[b];
  const unsigned char* payload = a.payloads + a.offset[b];
  const unsigned long long n = 2ull * a.span[b] * hkv * kHeadDim;
  const unsigned char* body = payload + 5;
  const unsigned char* codes = body + n;
  const unsigned char* entries = codes + n / 2;
  const unsigned int cap = (unsigned int)((n + 199) / 200);
  const unsigned int header_count = (unsigned int)payload[1] | ((unsigned int)payload[2] << 8) |
                                    ((unsigned int)payload[3] << 16) |
                                    ((unsigned int)payload[4] << 24);
  const unsigned int row_words = hkv * kHeadDim;  // payload words per token per plane
  const unsigned int wb = (split * kRanges + range) * a.tokens_per_wave;
  StepConst c;
  c.entries = entries;
  c.count = min(header_count, cap);
  c.half = (unsigned int)(n / 2);
  c.row_words = row_words;
  c.head = h;
  c.we = head_ok ? min(ctx, wb + a.tokens_per_wave) : wb;
  c.kv_heads = hkv;
  c.head_magic = a.head_magic;
  c.scale_log2 = a.scale_log2;
  c.tab_k = sTab[0];
  c.tab_v = sTab[1];
  c.sK = static_cast<uint16_t*>(__builtin_assume_aligned(lds + wave * kWaveLds, 16));
  c.sV = static_cast<uint16_t*>(__builtin_assume_aligned(c.sK + kStep * kKStride, 16));
  const unsigned int col = lane % 16, grp = lane / 16;
  const PlaneBases pb{body, codes, body + c.half, codes + c.half / 2};

  for (unsigned int i = tid; i < 512; i += kT)
    sTab[i >> 8][i & 255] = table_entry(a.tables + 512 + 16 * (i >> 8), i & 255);

  // query heads of the group as the B operand of S^T = K Q^T: lane l holds head
  // l%16 (columns 4..15 zero), dims 32*(l/16) + 8*ks + j
  bf16x8 qb[4];
  {
    const uint16_t* qrow = a.q + ((unsigned long long)b * a.q_heads + h * kGroup + col) * kHeadDim +
                           grp * 32;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      u32x4 v = {0, 0, 0, 0};
      if (col < kGroup && head_ok) v = *reinterpret_cast<const u32x4*>(qrow + 8 * ks);
      qb[ks] = __builtin_bit_cast(bf16x8, v);
    }
  }

  WaveWalk w;
  w.m_run = -INFINITY;
  w.l_run = 0.f;
#pragma unroll
  for (int k = 0; k < 2 * kPvChains; ++k) w.acc[k] = f32x4{0, 0, 0, 0};
  w.ok = payload[0] == 5;
  // This workgroup's share of the order check: entry pairs (i, i + 1) for i in
  // [chk_first, chk_last), the list split evenly over the sequence's splits * groups
  // workgroups. Thread t holds the positions of entries chk_first + kCheck*t ..
  // + kCheck; their loads go out now and are compared once the walk's first loads
  // are in flight, so they add no round trip of their own (entries past chk_last
  // repeat its position).
  const unsigned int chk_groups = a.splits * groups, chk_g = split * groups + hg;
  const unsigned int chk_chunk = (c.count + chk_groups - 1) / chk_groups;
  const unsigned int chk_first = min(chk_g * chk_chunk, c.count);
  const unsigned int chk_last = min(chk_first + chk_chunk, c.count > 0 ? c.count - 1 : 0u);
  const unsigned int chk0 = chk_first + tid * kCheck;
  unsigned int chk[kCheck + 1];
#pragma unroll
  for (int k = 0; k <= kCheck; ++k) chk[k] = entry_pos(entries, min(chk0 + k, chk_last));
  __syncthreads();  // decode tables

  // The waves meet at a barrier after every second step, so that the heads' waves
  // of a token range read each cache line they share within two steps of each
  // other and the later reads hit L2 (unsynchronised waves drifted apart and
  // fetched ~12 % of the payload bytes twice). Every wave runs the step count of
  // the longest of the workgroup's ranges.
  unsigned int steps_max = 0;
#pragma unroll
  for (int r = 0; r < kRanges; ++r) {
    const unsigned int s0 = (split * kRanges + r) * a.tokens_per_wave;
    const unsigned int e0 = min(ctx, s0 + a.tokens_per_wave);
    steps_max = max(steps_max, e0 > s0 ? (e0 - s0 + kStep - 1) / kStep : 0u);
  }
  const unsigned int steps = wb < c.we ? (c.we - wb + kStep - 1) / kStep : 0u;
  bool order_bad = false;
  auto check_order = [&]() {
#pragma unroll
    for (int k = 0; k < kCheck; ++k) order_bad |= chk0 + k < chk_last && chk[k + 1] < chk[k];
  };
  if (wb < c.we) {
    const unsigned int we = c.we;
    const unsigned int share = h * kHeadDim + (lane % 8) * 16;
    // two register sets of raw bytes alternate: one is decoded while the next
    // step's loads are in flight
    auto load_step = [&](unsigned int ts) {
      const unsigned int t0 = ts + lane / 8;
      return load_share(pb, min(t0, we - 1) * row_words + share,
                        min(t0 + 8, we - 1) * row_words + share);
    };
    auto step = [&](const RawShare& r, unsigned int ts) { attend_step(r, ts, c, qb, w); };
    // the first step's loads go out before the escape searches, whose round trips
    // they then overlap
    RawShare r0 = load_step(wb);
    const uint2 first = lower_bound_escapes2(entries, c.count, wb * row_words,
                                             c.half + wb * row_words);
    w.ptr_k = w.base_k = first.x;
    w.ptr_v = w.base_v = first.y;
    w.wk = load_window(entries, c.count, w.ptr_k + lane);
    w.wv = load_window(entries, c.count, w.ptr_v + lane);
    check_order();
    RawShare r1;
    unsigned int ts = wb;
    for (unsigned int i = 0; i < steps_max; i += 2) {
      if (i < steps) {
        r1 = load_step(ts + kStep);
        step(r0, ts);
      }
      if (i + 1 < steps) {
        r0 = load_step(ts + 2 * kStep);
        step(r1, ts + kStep);
      }
      __builtin_amdgcn_s_barrier();
      ts += 2 * kStep;
    }
  } else {
    check_order();
    for (unsigned int i = 0; i < steps_max; i += 2) __builtin_amdgcn_s_barrier();
  }

  // the rest of the order check (long lists only)
  for (unsigned int i = chk_first + kT * kCheck + tid; i < chk_last; i += kT)
    order_bad |= entry_pos(entries, i + 1) < entry_pos(entries, i);

  // ---- merge each head's kRanges waves (m, l, acc), then write the split's partials ----
  float l_run = w.l_run;
  const float m_run = w.m_run;
  l_run += __shfl_xor(l_run, 16, 64);
  l_run += __shfl_xor(l_run, 32, 64);
  const bool wave_bad = __ballot(!w.ok || order_bad) != 0;
  if (lane == 0) sBad[wave] = wave_bad ? 1u : 0u;
  __syncthreads();  // every wave is done with its LDS region
  float* sm = reinterpret_cast<float*>(lds);  // [wave][query row][kPartial]
  if (lane < kGroup) {
    sm[(wave * kGroup + lane) * kPartial] = m_run;
    sm[(wave * kGroup + lane) * kPartial + 1] = l_run;
  }
#pragma unroll
  for (int half = 0; half < 2; ++half)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float v = w.acc[half][j];
#pragma unroll
      for (int k = 1; k < kPvChains; ++k) v += w.acc[half + 2 * k][j];
      sm[(wave * kGroup + j) * kPartial + 2 + 64 * half + lane] = v;
    }
  __syncthreads();
  bool bad = false;
#pragma unroll
  for (int k = 0; k < kWaves; ++k) bad |= sBad[k] != 0;
  (void)grp;
  {
    // thread t: head m of the group, query row j, dims d0 .. d0 + kVals - 1
    constexpr int kPerHead = kT / kHeads;           // threads per head
    constexpr int kPerRow = kPerHead / kGroup;      // threads per query row
    constexpr int kVals = kHeadDim / kPerRow;       // dims per thread
    const unsigned int m = tid / kPerHead, u = tid % kPerHead;
    const unsigned int j = u / kPerRow, d0 = (u % kPerRow) * kVals;
    const unsigned int hm = kHeads * hg + m;
    if (hm < hkv) {
      const float* src[kRanges];
      float mr[kRanges];
      float big = -INFINITY;
#pragma unroll
      for (int r = 0; r < kRanges; ++r) {
        src[r] = sm + ((m * kRanges + r) * kGroup + j) * kPartial;
        mr[r] = src[r][0];
        big = fmaxf(big, mr[r]);
      }
      float l_sum = 0.f, o[kVals];
#pragma unroll
      for (int k = 0; k < kVals; ++k) o[k] = 0.f;
      if (big != -INFINITY) {
        // a wave with no tokens has m = -inf and weight 0
#pragma unroll
        for (int r = 0; r < kRanges; ++r) {
          const float wr = mr[r] == -INFINITY ? 0.f : exp2f(mr[r] - big);
          l_sum += src[r][1] * wr;
#pragma unroll
          for (int k = 0; k < kVals; ++k) o[k] += src[r][2 + d0 + k] * wr;
        }
      }
      float* dst = a.partial +
                   ((((unsigned long long)b * hkv + hm) * a.splits + split) * kGroup + j) * kPartial;
#pragma unroll
      for (int k = 0; k < kVals; ++k) dst[2 + d0 + k] = bad ? NAN : o[k];
      if (u % kPerRow == 0) {
        dst[0] = bad ? NAN : big;
        dst[1] = bad ? NAN : l_sum;
      }
    }
  }
}

// Merges the splits of one query head: out = sum_s acc_s 2^(m_s - M) / sum_s l_s 2^(m_s - M).
// A NaN running max in any partial of the sequence (a rejected payload or escape
// list, flagged by the split kernel) makes the whole output row NaN. The splits are
// read in batches of kCombineBatch with every load of a batch issued before any is
// used (one memory round trip per batch; a loop over the splits waited for each
// load in turn); with a single batch the sums run in split order against the
// global max.
constexpr int kCombineBatch = 16;

__global__ __launch_bounds__(kHeadDim) void top16_attention_combine(AttnArgs a) {
  const unsigned int qh = blockIdx.x, b = blockIdx.y, d = threadIdx.x;
  const unsigned int h = qh / kGroup, g = qh % kGroup;
  const float* seq = a.partial + (unsigned long long)b * a.kv_heads * a.splits * kGroup * kPartial;
  // the running max of the sequence's partials d, d + kHeadDim, ... (kv heads x
  // splits of them): the first four loaded now, tested after the merge
  float flag[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const unsigned int k = d + j * kHeadDim;
    flag[j] = k < a.kv_heads * a.splits ? seq[(unsigned long long)k * kGroup * kPartial] : 0.f;
  }
  const float* part = seq + (unsigned long long)h * a.splits * kGroup * kPartial + g * kPartial;
  float big = -INFINITY, num = 0.f, den = 0.f;
  for (unsigned int s0 = 0; s0 < a.splits; s0 += kCombineBatch) {
    float m[kCombineBatch], l[kCombineBatch], v[kCombineBatch];
#pragma unroll
    for (int k = 0; k < kCombineBatch; ++k) {
      // splits past the last one load split s0 again and are ignored
      const bool in = s0 + k < a.splits;
      const float* p = part + (unsigned long long)(in ? s0 + k : s0) * kGroup * kPartial;
      m[k] = p[0];
      l[k] = p[1];
      v[k] = p[2 + d];
      if (!in) m[k] = -INFINITY;
    }
    float top = big;
#pragma unroll
    for (int k = 0; k < kCombineBatch; ++k) top = fmaxf(top, m[k]);
    if (top == -INFINITY) continue;  // no split of this batch holds a token
    if (big != -INFINITY && top != big) {
      const float r = exp2f(big - top);
      num *= r;
      den *= r;
    }
    big = top;
#pragma unroll
    for (int k = 0; k < kCombineBatch; ++k) {
      if (m[k] == -INFINITY) continue;  // a split with no tokens
      const float wgt = exp2f(m[k] - big);
      den += l[k] * wgt;
      num += v[k] * wgt;
    }
  }
  int flagged = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) flagged |= isnan(flag[j]) ? 1 : 0;
  for (unsigned int k = d + 4 * kHeadDim; k < a.kv_heads * a.splits; k += kHeadDim)
    flagged |= isnan(seq[(unsigned long long)k * kGroup * kPartial]) ? 1 : 0;
  const bool bad = __syncthreads_or(flagged) != 0;
  a.out[((unsigned long long)b * a.q_heads + qh) * kHeadDim + d] =
      (uint16_t)bf16_bits(bad ? NAN : num / den);
}

}  // namespace
}  // namespace unchainkv

using namespace unchainkv;

namespace {

// Split-kernel workgroups the current device keeps resident at once (CUs x
// workgroups per CU at the kernel's register and LDS use), cached per device.
unsigned long long resident_workgroups() {
  static std::mutex mu;
  static unsigned long long cached[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 512;
  std::lock_guard<std::mutex> lock(mu);
  if (cached[dev] == 0) {
    int cus = 0, per_cu = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        cus <= 0)
      cus = 256;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
            &per_cu, reinterpret_cast<const void*>(top16_attention_split), kT, 0) != hipSuccess ||
        per_cu <= 0)
      per_cu = 1;
    cached[dev] = (unsigned long long)cus * (unsigned long long)per_cu;
  }
  return cached[dev];
}

struct SplitPlan {
  unsigned int groups;           // workgroups per (sequence, split)
  unsigned int splits, tokens_per_wave;
};

// Context splits per (sequence, head group): the count whose workgroups fill whole
// rounds of the resident slots with the fewest tokens per wave (a wave walks its
// range serially; a round that is partly empty wastes the rest of the chip). A split
// gives every head kRanges token ranges of tokens_per_wave.
SplitPlan plan_splits(unsigned long long sequences, unsigned long long kv_heads,
                      unsigned long long max_ctx) {
  SplitPlan best{(unsigned int)((kv_heads + kHeads - 1) / kHeads), 1, 0};
  const unsigned long long ranges = kRanges;
  const unsigned long long per_split = sequences * best.groups;
  const unsigned long long slots = resident_workgroups();
  constexpr unsigned long long kWaveOverhead = 32;  // start-up cost in token steps
  unsigned long long best_cost = ~0ull;
  for (unsigned int s = 1; s <= kMaxSplits; ++s) {
    const unsigned long long per_wave = (max_ctx + ranges * s - 1) / (ranges * s);
    const unsigned long long tpw = (per_wave + kStep - 1) / kStep * kStep;
    if (s > 1 && (unsigned long long)(s - 1) * ranges * tpw >= max_ctx) break;  // empty splits
    const unsigned long long rounds = (per_split * s + slots - 1) / slots;
    const unsigned long long cost = rounds * (tpw + kWaveOverhead);
    if (cost < best_cost) {
      best_cost = cost;
      best.splits = s;
      best.tokens_per_wave = (unsigned int)tpw;
    }
  }
  return best;
}

}  // namespace

// Workspace bytes that kvq_splitzip_top16_decode_attention needs (no counterpart in
// the reference).
extern "C" unsigned long long kvq_splitzip_top16_decode_attention_workspace_bytes(
    unsigned long long batch, unsigned long long kv_heads, unsigned long long max_ctx) {
  if (batch == 0 || kv_heads == 0 || max_ctx == 0) return 0;
  const unsigned long long per_launch = batch < kMaxSeqs ? batch : kMaxSeqs;
  const SplitPlan plan = plan_splits(per_launch, kv_heads, max_ctx);
  return per_launch * kv_heads * plan.splits * kGroup * kPartial * sizeof(float);
}

// Decode attention of one query token per sequence over Top-16 packed KV (no
// counterpart in the reference: it decodes the payload into the KV cache and then
// runs attention). See the header for the layout and the preconditions.
extern "C" long long kvq_splitzip_top16_decode_attention(
    unsigned long long q_ptr, unsigned long long out_ptr, unsigned long long payloads_ptr,
    const unsigned long long* payload_offsets, const unsigned long long* context_tokens,
    unsigned long long block_tokens, unsigned long long batch, unsigned long long q_heads,
    unsigned long long kv_heads, unsigned long long head_dim, unsigned long long tables_ptr,
    unsigned long long workspace_ptr, unsigned long long workspace_bytes, float scale,
    unsigned long long stream_ptr) {
  if (q_ptr == 0 || out_ptr == 0 || payloads_ptr == 0 || payload_offsets == nullptr ||
      context_tokens == nullptr || tables_ptr == 0 || workspace_ptr == 0 || batch == 0 ||
      block_tokens == 0 ||
      kv_heads == 0 || kv_heads >= 1024 || head_dim != kHeadDim || q_heads != kGroup * kv_heads ||
      q_ptr % 16 != 0 || tables_ptr % 4 != 0 || workspace_ptr % 16 != 0)
    return 0;
  unsigned long long max_ctx = 0;
  for (unsigned long long r = 0; r < batch; ++r) {
    const unsigned long long ctx = context_tokens[r];
    const unsigned long long span = (ctx + block_tokens - 1) / block_tokens * block_tokens;
    const unsigned long long n = 2 * span * kv_heads * kHeadDim;
    // positions are u32 and the body/code sections must be 16-byte aligned
    if (ctx == 0 || n > 0xFFFFFFFFULL || (payloads_ptr + payload_offsets[r] + 5) % 16 != 0)
      return 0;
    max_ctx = ctx > max_ctx ? ctx : max_ctx;
  }
  if (kvq_splitzip_top16_decode_attention_workspace_bytes(batch, kv_heads, max_ctx) >
      workspace_bytes)
    return 0;
  const unsigned long long per_launch = batch < kMaxSeqs ? batch : kMaxSeqs;
  const SplitPlan plan = plan_splits(per_launch, kv_heads, max_ctx);
  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_ptr);
  for (unsigned long long first = 0; first < batch; first += kMaxSeqs) {
    const unsigned int count = (unsigned int)(batch - first < kMaxSeqs ? batch - first : kMaxSeqs);
    AttnArgs a{};
    a.q = reinterpret_cast<const uint16_t*>(q_ptr) + first * q_heads * kHeadDim;
    a.out = reinterpret_cast<uint16_t*>(out_ptr) + first * q_heads * kHeadDim;
    a.payloads = reinterpret_cast<const unsigned char*>(payloads_ptr);
    a.tables = reinterpret_cast<const unsigned char*>(tables_ptr);
    a.partial = reinterpret_cast<float*>(workspace_ptr);
    a.batch = count;
    a.q_heads = (unsigned int)q_heads;
    a.kv_heads = (unsigned int)kv_heads;
    a.splits = plan.splits;
    a.tokens_per_wave = plan.tokens_per_wave;
    a.scale_log2 = scale * 1.4426950408889634f;
    a.head_magic = (unsigned int)((1ull << 24) / kv_heads + 1);
    for (unsigned int r = 0; r < count; ++r) {
      a.offset[r] = payload_offsets[first + r];
      const unsigned long long ctx = context_tokens[first + r];
      a.ctx[r] = (unsigned int)ctx;
      a.span[r] = (unsigned int)((ctx + block_tokens - 1) / block_tokens * block_tokens);
    }
    hipLaunchKernelGGL(top16_attention_split, dim3(plan.splits * plan.groups * count), dim3(kT),
                       0, stream, a);
    hipError_t st = hipGetLastError();
    if (st != hipSuccess) return fail("top16_attention_split", st);
    hipLaunchKernelGGL(top16_attention_combine, dim3((unsigned int)q_heads, count),
                       dim3(kHeadDim), 0, stream, a);
    st = hipGetLastError();
    if (st != hipSuccess) return fail("top16_attention_combine", st);
  }
  return (long long)(batch * q_heads * kHeadDim * sizeof(uint16_t));
}
