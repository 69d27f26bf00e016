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
// Work split (flash-decoding): one workgroup per (context split, kv head, sequence);
// its 4 waves take 4 consecutive token ranges of the split and run independently
// (wave-private LDS, no workgroup barrier until the final merge). Per 16-token
// step, lane l decodes token l%16, dims 32*(l/16) .. +31 of K and V:
//   * S^T = K Q^T on v_mfma_f32_16x16x32_bf16 with K as the A operand (rows =
//     tokens) and the GQA group's 4 query heads as B columns; the dims are taken in
//     the order lane-group-major so the A operand is the lane's own row of sK;
//   * the result leaves lane l with tokens 4*(l/16)+j of head l%16, which is
//     exactly the A operand (P) of v_mfma_f32_16x16x16_bf16 for O = P V, whose B
//     operand (4 tokens of one dim) comes from the token-major V in LDS through
//     the transposing read ds_read_b64_tr_b16 (V is stored like K, two 16-byte
//     writes per token and lane instead of sixteen 2-byte transposed writes:
//     Llama-3-8B decode step 167.4 -> 159.0 us).
// The 4 waves' softmax states are merged in LDS; a second kernel merges the splits
// and writes bf16.
//
// Escapes: the kernel needs the escape list in ascending position order (what the
// encoder of this library writes; the reference's encoder appends escapes in
// atomic order, so its lists may be unordered). Each wave finds its first K and V
// escape with a 64-way search and then walks the list with its steps, one 64-entry
// window per plane prefetched a step ahead. The search is only meaningful on an
// ordered list, so the list's order is checked up front as well: the split
// kernel's workgroups of a sequence share the check of every neighbouring pair of
// entries between them. A decrease anywhere in the list, an entry found below the
// current step, or a payload whose byte 0 is not 5, makes every output of the
// sequence NaN (the combine kernel looks at all of the sequence's partials)
// rather than silently wrong.
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
constexpr int kKStride = kHeadDim + 8;      // u16 per row of sK and sV (bank spread, 16 B aligned)
constexpr int kWaveLds = 2 * kStep * kKStride;  // u16 per wave: K and V of a step, token-major
constexpr int kMaxSeqs = 64;                // sequences per launch (kernel arguments)
constexpr int kPartial = kHeadDim + 2;      // m, l, acc[128] per (split, query head)
constexpr int kMaxSplits = 64;
constexpr int kCheck = 8;                   // escape-order pairs per thread held through the walk
static_assert(4 * kGroup * kPartial * 4 <= 4 * kWaveLds * 2, "merge area fits the wave LDS");

struct AttnArgs {
  const uint16_t* q;             // [batch][q_heads][128] bf16
  uint16_t* out;                 // [batch][q_heads][128] bf16
  const unsigned char* payloads;
  const unsigned char* tables;   // 544 B; K codebook at +512, V at +528
  float* partial;                // [batch][kv_heads][splits][kGroup][kPartial]
  unsigned int batch, q_heads, kv_heads, splits, tokens_per_wave;
  float scale_log2;              // scale * log2(e)
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
  return *reinterpret_cast<const u32_unaligned*>(entries + 5ull * i);
}

// Packed bytes of one lane's share of a step, per plane: 16 body bytes (mantissa |
// sign << 7) and 8 code bytes of 16 consecutive words of each of two tokens.
// Lane l takes tokens l/8 and l/8 + 8 of the step, dims 16*(l%8) .. +15, so that
// 8 consecutive lanes read a token's whole 128-byte body row and 64-byte code row.
struct RawShare {
  u32x4 kb[2], vb[2];
  u32x2 kc[2], vc[2];
};

// `w0`, `w1` = payload word of the share's first K word for each token. Every lane
// loads (no branch): a lane whose token is past the range passes a clamped,
// in-range token instead and its words are ignored.
__device__ __forceinline__ RawShare load_share(const unsigned char* body,
                                               const unsigned char* codes,
                                               unsigned long long w0, unsigned long long w1,
                                               unsigned int half) {
  RawShare r;
  r.kb[0] = load_stream16(body + w0);
  r.kb[1] = load_stream16(body + w1);
  r.kc[0] = load_stream8(codes + w0 / 2);
  r.kc[1] = load_stream8(codes + w1 / 2);
  r.vb[0] = load_stream16(body + half + w0);
  r.vb[1] = load_stream16(body + half + w1);
  r.vc[0] = load_stream8(codes + (half + w0) / 2);
  r.vc[1] = load_stream8(codes + (half + w1) / 2);
  return r;
}

// First index in [0, count) whose position is >= target (entries ascending);
// wave-cooperative 64-way search, result uniform across the wave.
__device__ unsigned int lower_bound_escapes(const unsigned char* entries, unsigned int count,
                                            unsigned int target) {
  const unsigned int lane = __lane_id();
  unsigned int lo = 0, hi = count;
  while (hi - lo > 64) {
    const unsigned int step = (hi - lo + 63) / 64;
    const unsigned int idx = lo + lane * step;
    const bool below = idx < hi && entry_pos(entries, idx) < target;
    const unsigned int k = (unsigned int)__popcll(__ballot(below));
    const unsigned int new_lo = k ? lo + (k - 1) * step + 1 : lo;
    const unsigned int new_hi = min(hi, lo + k * step);
    lo = new_lo;
    hi = max(new_hi, new_lo);
  }
  const unsigned int idx = lo + lane;
  const bool below = idx < hi && entry_pos(entries, idx) < target;
  return __builtin_amdgcn_readfirstlane(lo + (unsigned int)__popcll(__ballot(below)));
}

// One 64-entry window of a plane's escape list (entry ptr + lane); positions past
// the list read as 0xFFFFFFFF.
struct Window {
  unsigned int pos, exp;
};

__device__ __forceinline__ Window load_window(const unsigned char* entries, unsigned int count,
                                              unsigned int i) {
  Window w{0xFFFFFFFFu, 0u};
  if (i < count) {
    w.pos = entry_pos(entries, i);
    w.exp = entries[5ull * i + 4];
  }
  return w;
}

// Applies the escapes of one plane that fall in tokens [ts, t_stop) to the wave's
// LDS copy of the step and advances the plane's list pointer past them. `base` is
// the plane's first position (0 or n/2), `row_words` the payload words per token.
// Returns false when the list is found out of order. Wave-uniform control flow.
template <bool kV>
__device__ __forceinline__ bool apply_escapes(Window& win, unsigned int& ptr,
                                              const unsigned char* entries, unsigned int count,
                                              unsigned int base, unsigned int ts,
                                              unsigned int t_stop, unsigned int row_words,
                                              unsigned int head, uint16_t* sK, uint16_t* sV) {
  const unsigned int lane = __lane_id();
  const unsigned int lo = base + ts * row_words, hi = base + t_stop * row_words;
  bool ok = true;
  for (;;) {
    const bool in = win.pos < hi;
    if (in) {
      if (win.pos < lo) {
        ok = false;  // below this step: the list is not ascending
      } else {
        const unsigned int q = win.pos - base;
        const unsigned int t = q / row_words, rem = q - t * row_words;
        if (rem / kHeadDim == head) {
          const unsigned int dim = rem % kHeadDim, tt = t - ts;
          uint16_t* w = kV ? &sV[tt * kKStride + dim] : &sK[tt * kKStride + dim];
          *w = (uint16_t)((*w & 0x807Fu) | (win.exp << 7));
        }
      }
    }
    const unsigned int next = __shfl_down(win.pos, 1, 64);
    if (lane < 63 && next < win.pos) ok = false;
    const unsigned int taken = (unsigned int)__popcll(__ballot(in));
    ptr += taken;
    if (taken < 64) break;
    win = load_window(entries, count, ptr + lane);  // > 64 escapes in one step
  }
  return ok;
}

// Per-wave state of the walk over a token range.
struct WaveWalk {
  float m_run;      // running max (log2 units) of head l%16
  float l_run;      // this lane's share of the running sum of head l%16
  f32x4 acc[8];     // O rows 4*(l/16)+j (heads on lanes 0..15), dims 16*nt + l%16
  Window wk, wv;    // escape windows of the K and V planes
  unsigned int ptr_k, ptr_v;
  bool ok;
};

struct StepConst {
  const unsigned char* entries;
  unsigned int count, half, row_words, head, we;
  float scale_log2;
  const uint32_t* tab_k;
  const uint32_t* tab_v;
  uint16_t* sK;
  uint16_t* sV;
};

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
      u32x4* dstk = reinterpret_cast<u32x4*>(c.sK + tt * kKStride + part * 16);
      dstk[0] = u32x4{o[0], o[1], o[2], o[3]};
      dstk[1] = u32x4{o[4], o[5], o[6], o[7]};
      decode8(cur.vb[i].x, cur.vb[i].y, cur.vc[i].x, c.tab_v, o);
      decode8(cur.vb[i].z, cur.vb[i].w, cur.vc[i].y, c.tab_v, o + 4);
      if (tail && ts + tt >= c.we) {
        // a token past the range: zero V so that p = 0 cannot meet an Inf or NaN
#pragma unroll
        for (int r = 0; r < 8; ++r) o[r] = 0u;
      }
      u32x4* dstv = reinterpret_cast<u32x4*>(c.sV + tt * kKStride + part * 16);
      dstv[0] = u32x4{o[0], o[1], o[2], o[3]};
      dstv[1] = u32x4{o[4], o[5], o[6], o[7]};
    }
  }

  // escapes of this step; then prefetch the windows of the next one
  const unsigned int t_stop = min(ts + kStep, c.we);
  w.ok &= apply_escapes<false>(w.wk, w.ptr_k, c.entries, c.count, 0u, ts, t_stop, c.row_words,
                               c.head, c.sK, c.sV);
  w.ok &= apply_escapes<true>(w.wv, w.ptr_v, c.entries, c.count, c.half, ts, t_stop, c.row_words,
                              c.head, c.sK, c.sV);
  w.wk = load_window(c.entries, c.count, w.ptr_k + lane);
  w.wv = load_window(c.entries, c.count, w.ptr_v + lane);
  // LDS accesses of one wave complete in order; this keeps the compiler from
  // moving the reads below above the writes
  __builtin_amdgcn_wave_barrier();

  // ---- S^T = K Q^T: lane l gets tokens 4*(l/16)+j of head l%16 ----
  f32x4 st = {0, 0, 0, 0};
  {
    const uint16_t* krow = c.sK + col * kKStride + grp * 32;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const bf16x8 ka = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(krow + 8 * ks));
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
  mloc = fmaxf(mloc, __shfl_xor(mloc, 16, 64));
  mloc = fmaxf(mloc, __shfl_xor(mloc, 32, 64));
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
    for (int nt = 0; nt < 8; ++nt)
#pragma unroll
      for (int j = 0; j < 4; ++j) w.acc[nt][j] *= al[j];
    w.m_run = m_new;
  }
  float p[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) p[j] = __builtin_amdgcn_exp2f(sc[j] - w.m_run);
  w.l_run += (p[0] + p[1]) + (p[2] + p[3]);

  // ---- O += P V: P is already the A operand (head l%16, tokens 4*(l/16)+j) ----
  i16x4 pa;
#pragma unroll
  for (int j = 0; j < 4; ++j) pa[j] = (short)bf16_bits(p[j]);
#pragma unroll
  for (int nt = 0; nt < 8; ++nt) {
    // transposing read: within each 16-lane group, lane i receives element i % 4
    // of the 4-element rows that lanes 4j + i/4 read (j = 0..3). Lane s reads dims
    // nt*16 + 4*(s%4) .. + 3 of token 4*grp + s/4, so lane i ends up with dim
    // nt*16 + i of tokens 4*grp .. + 3: the B operand, from token-major V
    const uint16_t* vsrc = c.sV + (grp * 4 + col / 4) * kKStride + nt * 16 + 4 * (col % 4);
    const i16x4 vb = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) i16x4*)(vsrc));
    w.acc[nt] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(pa, vb, w.acc[nt], 0, 0, 0);
  }
  __builtin_amdgcn_wave_barrier();
}

__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(3, 3))) void
top16_attention_split(AttnArgs a) {
  __shared__ __align__(16) uint16_t lds[4 * kWaveLds];
  __shared__ uint32_t sTab[2][256];
  __shared__ unsigned int sBad[4];

  const unsigned int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  // work item = (sequence, split, head pair) with the pair fastest, each XCD taking
  // a contiguous run of items (xcd_remap). Waves 0-1 serve head 2p and waves 2-3
  // head 2p+1 over the same two token ranges: the two heads' 64-byte code rows
  // share one 128-byte cache line, which the two waves then read together.
  const unsigned int hkv = a.kv_heads;
  const unsigned int pairs = (hkv + 1) / 2;
  const unsigned int w_item = xcd_remap(blockIdx.x, gridDim.x);
  const unsigned int hp = w_item % pairs;
  const unsigned int split = (w_item / pairs) % a.splits;
  const unsigned int b = w_item / (pairs * a.splits);
  const unsigned int h = 2 * hp + (wave >> 1);
  const bool head_ok = h < hkv;  // an odd head count leaves the last pair half empty
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
  const unsigned int wb = (split * 2 + (wave & 1)) * a.tokens_per_wave;
  StepConst c;
  c.entries = entries;
  c.count = min(header_count, cap);
  c.half = (unsigned int)(n / 2);
  c.row_words = row_words;
  c.head = h;
  c.we = head_ok ? min(ctx, wb + a.tokens_per_wave) : wb;
  c.scale_log2 = a.scale_log2;
  c.tab_k = sTab[0];
  c.tab_v = sTab[1];
  c.sK = static_cast<uint16_t*>(__builtin_assume_aligned(lds + wave * kWaveLds, 16));
  c.sV = static_cast<uint16_t*>(__builtin_assume_aligned(c.sK + kStep * kKStride, 16));
  const unsigned int col = lane % 16, grp = lane / 16;

  sTab[0][tid] = table_entry(a.tables + 512, tid);
  sTab[1][tid] = table_entry(a.tables + 528, tid);

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
  for (int nt = 0; nt < 8; ++nt) w.acc[nt] = f32x4{0, 0, 0, 0};
  w.ok = payload[0] == 5;
  // This workgroup's share of the order check: entry pairs (i, i + 1) for i in
  // [chk_first, chk_last), the list split evenly over the sequence's splits * pairs
  // workgroups. Thread t holds the positions of entries chk_first + kCheck*t ..
  // + kCheck; their loads go out now and are compared once the walk's first loads
  // are in flight, so they add no round trip of their own (entries past chk_last
  // repeat its position).
  const unsigned int chk_groups = a.splits * pairs, chk_g = split * pairs + hp;
  const unsigned int chk_chunk = (c.count + chk_groups - 1) / chk_groups;
  const unsigned int chk_first = min(chk_g * chk_chunk, c.count);
  const unsigned int chk_last = min(chk_first + chk_chunk, c.count > 0 ? c.count - 1 : 0u);
  const unsigned int chk0 = chk_first + tid * kCheck;
  unsigned int chk[kCheck + 1];
#pragma unroll
  for (int k = 0; k <= kCheck; ++k) chk[k] = entry_pos(entries, min(chk0 + k, chk_last));
  __syncthreads();  // decode tables

  // The four waves meet at a barrier after every second step, so that the two
  // heads' waves of a token range read each 128-byte code line they share within
  // two steps of each other and the second read hits L2 (unsynchronised waves
  // drifted apart and fetched ~12 % of the payload bytes twice). Every wave runs
  // the step count of the longer of the workgroup's two ranges.
  auto range_steps = [&](unsigned int r) -> unsigned int {
    const unsigned int s0 = (split * 2 + r) * a.tokens_per_wave;
    const unsigned int e0 = min(ctx, s0 + a.tokens_per_wave);
    return e0 > s0 ? (e0 - s0 + kStep - 1) / kStep : 0u;
  };
  const unsigned int steps_max = max(range_steps(0), range_steps(1));
  const unsigned int steps = wb < c.we ? (c.we - wb + kStep - 1) / kStep : 0u;
  bool order_bad = false;
  auto check_order = [&]() {
#pragma unroll
    for (int k = 0; k < kCheck; ++k) order_bad |= chk0 + k < chk_last && chk[k + 1] < chk[k];
  };
  if (wb < c.we) {
    const unsigned int we = c.we;
    w.ptr_k = lower_bound_escapes(entries, c.count, wb * row_words);
    w.ptr_v = lower_bound_escapes(entries, c.count, c.half + wb * row_words);
    w.wk = load_window(entries, c.count, w.ptr_k + lane);
    w.wv = load_window(entries, c.count, w.ptr_v + lane);
    const unsigned int share = h * kHeadDim + (lane % 8) * 16;
    // two register sets of raw bytes alternate: one is decoded while the next
    // step's loads are in flight
    auto load_step = [&](unsigned int ts) {
      const unsigned int t0 = ts + lane / 8;
      return load_share(body, codes, (unsigned long long)min(t0, we - 1) * row_words + share,
                        (unsigned long long)min(t0 + 8, we - 1) * row_words + share, c.half);
    };
    RawShare r0 = load_step(wb);
    check_order();
    RawShare r1;
    unsigned int ts = wb;
    for (unsigned int i = 0; i < steps_max; i += 2) {
      if (i < steps) {
        r1 = load_step(ts + kStep);
        attend_step(r0, ts, c, qb, w);
      }
      if (i + 1 < steps) {
        r0 = load_step(ts + 2 * kStep);
        attend_step(r1, ts + kStep, c, qb, w);
      }
      __builtin_amdgcn_s_barrier();
      ts += 2 * kStep;
    }
  } else {
    check_order();
    for (unsigned int i = 0; i < steps_max; i += 2) __builtin_amdgcn_s_barrier();
  }

  // the rest of the order check (long lists only)
  for (unsigned int i = chk_first + kThreads * kCheck + tid; i < chk_last; i += kThreads)
    order_bad |= entry_pos(entries, i + 1) < entry_pos(entries, i);

  // ---- merge each head's 2 waves (m, l, acc), then write the split's partials ----
  float l_run = w.l_run;
  const float m_run = w.m_run;
  l_run += __shfl_xor(l_run, 16, 64);
  l_run += __shfl_xor(l_run, 32, 64);
  const bool wave_bad = __ballot(!w.ok || order_bad) != 0;
  if (lane == 0) sBad[wave] = wave_bad ? 1u : 0u;
  __syncthreads();  // every wave is done with its LDS region
  float* sm = reinterpret_cast<float*>(lds);  // [wave][head][kPartial]
  if (lane < kGroup) {
    sm[(wave * kGroup + lane) * kPartial] = m_run;
    sm[(wave * kGroup + lane) * kPartial + 1] = l_run;
  }
  if (lane < 16) {
#pragma unroll
    for (int nt = 0; nt < 8; ++nt)
#pragma unroll
      for (int j = 0; j < 4; ++j) sm[(wave * kGroup + j) * kPartial + 2 + nt * 16 + lane] = w.acc[nt][j];
  }
  __syncthreads();
  const bool bad = (sBad[0] | sBad[1] | sBad[2] | sBad[3]) != 0;
  (void)grp;
  {
    // thread t: head 2p + (t >> 7), query row (t >> 5) & 3, dims 4 * (t & 31) .. +3
    const unsigned int m = tid >> 7, j = (tid >> 5) & 3, d0 = (tid & 31) * 4;
    const unsigned int hm = 2 * hp + m;
    if (hm < hkv) {
      const float* s0 = sm + ((2 * m) * kGroup + j) * kPartial;
      const float* s1 = sm + ((2 * m + 1) * kGroup + j) * kPartial;
      const float m0 = s0[0], m1 = s1[0];
      const float big = fmaxf(m0, m1);
      float l_sum = 0.f, o[4] = {0.f, 0.f, 0.f, 0.f};
      if (big != -INFINITY) {
        // a wave with no tokens has m = -inf and weight 0
        const float w0 = m0 == -INFINITY ? 0.f : exp2f(m0 - big);
        const float w1 = m1 == -INFINITY ? 0.f : exp2f(m1 - big);
        l_sum = s0[1] * w0 + s1[1] * w1;
#pragma unroll
        for (int k = 0; k < 4; ++k) o[k] = s0[2 + d0 + k] * w0 + s1[2 + d0 + k] * w1;
      }
      float* dst = a.partial +
                   ((((unsigned long long)b * hkv + hm) * a.splits + split) * kGroup + j) * kPartial;
#pragma unroll
      for (int k = 0; k < 4; ++k) dst[2 + d0 + k] = bad ? NAN : o[k];
      if ((tid & 31) == 0) {
        dst[0] = bad ? NAN : big;
        dst[1] = bad ? NAN : l_sum;
      }
    }
  }
}

// Merges the splits of one query head: out = sum_s acc_s 2^(m_s - M) / sum_s l_s 2^(m_s - M).
// A NaN running max in any partial of the sequence (a rejected payload or escape
// list, flagged by the split kernel) makes the whole output row NaN.
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
  float big = -INFINITY;
  for (unsigned int s = 0; s < a.splits; ++s) big = fmaxf(big, part[s * kGroup * kPartial]);
  float num = 0.f, den = 0.f;
  for (unsigned int s = 0; s < a.splits; ++s) {
    const float* p = part + s * kGroup * kPartial;
    const float m = p[0];
    if (m == -INFINITY) continue;  // a split with no tokens
    const float wgt = exp2f(m - big);
    den += p[1] * wgt;
    num += p[2 + d] * wgt;
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
// workgroups per CU at this kernel's register and LDS use), cached per device.
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
            &per_cu, reinterpret_cast<const void*>(top16_attention_split), kThreads, 0) !=
            hipSuccess ||
        per_cu <= 0)
      per_cu = 2;
    cached[dev] = (unsigned long long)cus * (unsigned long long)per_cu;
  }
  return cached[dev];
}

struct SplitPlan {
  unsigned int splits, tokens_per_wave;
};

// Context splits per (sequence, kv head): the count whose workgroups fill whole
// rounds of the resident slots with the fewest tokens per wave (a wave walks its
// range serially; a round that is partly empty wastes the rest of the chip).
SplitPlan plan_splits(unsigned long long groups, unsigned long long max_ctx) {
  // groups: workgroups per split (sequences x head pairs); a split gives every head
  // 2 token ranges of tokens_per_wave
  const unsigned long long slots = resident_workgroups();
  constexpr unsigned long long kWaveOverhead = 32;  // start-up cost in token steps
  SplitPlan best{1, 0};
  unsigned long long best_cost = ~0ull;
  for (unsigned int s = 1; s <= kMaxSplits; ++s) {
    const unsigned long long per_wave = (max_ctx + 2ull * s - 1) / (2ull * s);
    const unsigned long long tpw = (per_wave + kStep - 1) / kStep * kStep;
    if (s > 1 && (unsigned long long)(s - 1) * 2 * tpw >= max_ctx) break;  // empty splits
    const unsigned long long rounds = (groups * s + slots - 1) / slots;
    const unsigned long long cost = rounds * (tpw + kWaveOverhead);
    if (cost < best_cost) {
      best_cost = cost;
      best = SplitPlan{s, (unsigned int)tpw};
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
  const SplitPlan plan = plan_splits(per_launch * ((kv_heads + 1) / 2), max_ctx);
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
      kv_heads == 0 || head_dim != kHeadDim || q_heads != kGroup * kv_heads ||
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
  const SplitPlan plan = plan_splits(per_launch * ((kv_heads + 1) / 2), max_ctx);
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
    for (unsigned int r = 0; r < count; ++r) {
      a.offset[r] = payload_offsets[first + r];
      const unsigned long long ctx = context_tokens[first + r];
      a.ctx[r] = (unsigned int)ctx;
      a.span[r] = (unsigned int)((ctx + block_tokens - 1) / block_tokens * block_tokens);
    }
    hipLaunchKernelGGL(top16_attention_split,
                       dim3(plan.splits * (unsigned int)((kv_heads + 1) / 2) * count),
                       dim3(kThreads), 0, stream, a);
    hipError_t st = hipGetLastError();
    if (st != hipSuccess) return fail("top16_attention_split", st);
    hipLaunchKernelGGL(top16_attention_combine, dim3((unsigned int)q_heads, count),
                       dim3(kHeadDim), 0, stream, a);
    st = hipGetLastError();
    if (st != hipSuccess) return fail("top16_attention_combine", st);
  }
  return (long long)(batch * q_heads * kHeadDim * sizeof(uint16_t));
}
