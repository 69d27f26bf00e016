// Fused Top-16 decode + paged decode attention (one query token per sequence),
// gfx950.
//
// The KV of each sequence is one Top-16 payload (mode 5) of its K plane then its V
// plane, words ordered [token][kv head][dim] (what the batched encoder produces for
// a sequence's block table in token order). The kernel never materialises bf16 KV
// in HBM: it reads the packed body and code bytes once, decodes 64-token chunks
// into LDS, patches the chunk's escapes there, and runs QK^T and PV on the MFMA
// units (v_mfma_f32_16x16x32_bf16) with an online softmax.
//
// Work split: one workgroup per (context split, kv head, sequence); wave w owns
// tokens 16w .. 16w+15 of a chunk for QK and output dims 32w .. 32w+31 for PV. The
// GQA group (4 query heads per kv head) fills rows 0..3 of the 16-row MFMA A tile.
// A second kernel merges the splits (flash-decoding) and writes bf16.
//
// Escapes: the kernel needs the escape list in ascending position order (what the
// encoder of this library writes). Each workgroup finds its first escape with a
// 64-way search and then walks the list with its chunks; a decrease between
// neighbouring entries it reads, or a payload whose byte 0 is not 5, makes its
// output NaN rather than silently wrong.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>

#include "splitzip_common.h"

namespace unchainkv {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kHeadDim = 128;
constexpr int kGroup = 4;                  // query heads per kv head
constexpr int kChunk = 64;                 // tokens per inner step
constexpr int kKStride = kHeadDim + 8;     // bf16 per row of sK (bank spread)
constexpr int kVtStride = kChunk + 8;      // bf16 per row of the transposed V
constexpr int kPStride = kChunk + 8;       // bf16 per row of P
constexpr int kMaxSeqs = 64;               // sequences per launch (kernel arguments)
constexpr int kPartial = kHeadDim + 2;     // m, l, acc[128] per (split, query head)

struct AttnArgs {
  const uint16_t* q;             // [batch][q_heads][128] bf16
  uint16_t* out;                 // [batch][q_heads][128] bf16
  const unsigned char* payloads;
  const unsigned char* tables;   // 544 B; K codebook at +512, V at +528
  float* partial;                // [batch][kv_heads][splits][kGroup][kPartial]
  unsigned int batch, q_heads, kv_heads, splits, tokens_per_split;
  float scale_log2;              // log2(e) / sqrt(head_dim)
  unsigned long long offset[kMaxSeqs];  // payload byte offset of each sequence
  unsigned int ctx[kMaxSeqs];           // context tokens of each sequence
  unsigned int span[kMaxSeqs];          // tokens the payload holds (whole blocks, >= ctx)
};

__device__ __forceinline__ unsigned int bf16_bits(float v) {
  return __builtin_bit_cast(unsigned short, (__bf16)v);  // round to nearest even
}

// Exponents of four 4-bit codes (one per byte of s) from a 16-byte codebook.
__device__ __forceinline__ uint32_t lookup4(uint32_t s, const uint32_t (&cb)[4]) {
  const uint32_t s7 = s & 0x07070707u;
  const uint32_t lo = __builtin_amdgcn_perm(cb[1], cb[0], s7);
  const uint32_t hi = __builtin_amdgcn_perm(cb[3], cb[2], s7);
  const uint32_t mask = __builtin_amdgcn_perm(s << 12, s << 4, 0x090B080Au);
  return (hi & mask) | (lo & ~mask);
}

__device__ __forceinline__ uint32_t pair_of(uint32_t x) {
  const uint32_t y = (x & 0x007F007Fu) | ((x >> 1) & ~0x007F007Fu);
  return ((x << 8) & 0x80008000u) | (y & ~0x80008000u);
}

// 8 words (4 dwords of bf16 pairs) from 8 body bytes and 4 code bytes.
__device__ __forceinline__ void decode8(uint32_t b0, uint32_t b1, uint32_t cd,
                                        const uint32_t (&cb)[4], uint32_t* o) {
  const uint32_t u = cd >> 4;
  const uint32_t sa = __builtin_amdgcn_perm(u, cd, 0x05010400u) & 0x0F0F0F0Fu;
  const uint32_t sb = __builtin_amdgcn_perm(u, cd, 0x07030602u) & 0x0F0F0F0Fu;
  const uint32_t ea = lookup4(sa, cb), eb = lookup4(sb, cb);
  o[0] = pair_of(__builtin_amdgcn_perm(ea, b0, 0x05010400u));
  o[1] = pair_of(__builtin_amdgcn_perm(ea, b0, 0x07030602u));
  o[2] = pair_of(__builtin_amdgcn_perm(eb, b1, 0x05010400u));
  o[3] = pair_of(__builtin_amdgcn_perm(eb, b1, 0x07030602u));
}

// Position (u32 LE) of escape entry i.
__device__ __forceinline__ unsigned int entry_pos(const unsigned char* entries, unsigned int i) {
  const unsigned char* e = entries + 5ull * i;
  return (unsigned int)e[0] | ((unsigned int)e[1] << 8) | ((unsigned int)e[2] << 16) |
         ((unsigned int)e[3] << 24);
}

// Packed bytes of one thread's share of a chunk: 32 body bytes and 16 code bytes
// of the K plane and of the V plane (32 words each).
struct RawShare {
  u32x4 kb0, kb1, kc, vb0, vb1, vc;
};

__device__ __forceinline__ RawShare load_share(const unsigned char* body,
                                               const unsigned char* codes,
                                               unsigned long long w, unsigned int half,
                                               bool live) {
  RawShare r;
  if (live) {
    r.kb0 = load_stream16(body + w);
    r.kb1 = load_stream16(body + w + 16);
    r.kc = load_stream16(codes + w / 2);
    r.vb0 = load_stream16(body + half + w);
    r.vb1 = load_stream16(body + half + w + 16);
    r.vc = load_stream16(codes + (half + w) / 2);
  } else {
    r.kb0 = r.kb1 = r.kc = r.vb0 = r.vb1 = r.vc = u32x4{0, 0, 0, 0};
  }
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

__global__ __launch_bounds__(kThreads) void top16_attention_split(AttnArgs a) {
  __shared__ __align__(16) uint16_t sK[kChunk * kKStride];
  __shared__ __align__(16) uint16_t sVt[kHeadDim * kVtStride];
  __shared__ __align__(16) uint16_t sP[16 * kPStride];
  __shared__ float sRed[4][2 * kGroup];
  __shared__ unsigned int sCount[4];
  __shared__ unsigned int sPtr[2];
  __shared__ unsigned int sBad;

  const unsigned int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const unsigned int split = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const unsigned int hkv = a.kv_heads;
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
  const unsigned int count = min(header_count, cap);
  const unsigned int mode = payload[0];
  const unsigned int t_begin = split * a.tokens_per_split;
  const unsigned int t_end = min(ctx, t_begin + a.tokens_per_split);
  const unsigned int row_words = hkv * kHeadDim;  // payload words per token per plane
  const unsigned int half = (unsigned int)(n / 2);

  // Q rows of the GQA group as the MFMA A operand: lane l holds row l%16 (rows 0..3
  // are the group's query heads, the rest zero), k = 32ks + (l/16)*8 + j
  bf16x8 qa[4];
  {
    const unsigned int row = lane % 16, kq = (lane / 16) * 8;
    const uint16_t* qrow = a.q + ((unsigned long long)b * a.q_heads + h * kGroup + row) * kHeadDim;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      u32x4 v = {0, 0, 0, 0};
      if (row < kGroup) v = *reinterpret_cast<const u32x4*>(qrow + 32 * ks + kq);
      qa[ks] = __builtin_bit_cast(bf16x8, v);
    }
  }
  // P rows 4..15 stay zero
  for (unsigned int i = tid; i < 16 * kPStride; i += kThreads) sP[i] = 0;
  if (tid == 0) sBad = mode != 5 ? 1u : 0u;
  if (wave < 2) {
    const unsigned int target = (wave ? half : 0u) + t_begin * row_words;
    const unsigned int ptr = lower_bound_escapes(entries, count, target);
    if (lane == 0) sPtr[wave] = ptr;
  }
  uint32_t cbk[4], cbv[4];
  {
    const uint32_t* t32 = reinterpret_cast<const uint32_t*>(a.tables + 512);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      cbk[k] = t32[k];
      cbv[k] = t32[4 + k];
    }
  }

  // per-lane online-softmax state: lanes 0..15 own rows 0..3 (the query heads)
  float m_run[kGroup], l_run[kGroup];
#pragma unroll
  for (int j = 0; j < kGroup; ++j) {
    m_run[j] = -INFINITY;
    l_run[j] = 0.f;
  }
  f32x4 acc[2] = {{0, 0, 0, 0}, {0, 0, 0, 0}};

  // this thread's share of a chunk: token tid/4, dims (tid%4)*32 .. +32
  const unsigned int tok = tid >> 2, part = tid & 3;
  const unsigned long long share_word = (unsigned long long)tok * row_words + h * kHeadDim + part * 32;
  RawShare next = load_share(body, codes, (unsigned long long)t_begin * row_words + share_word,
                             half, t_begin + tok < t_end);
  __syncthreads();
  unsigned int ptr[2] = {sPtr[0], sPtr[1]};

  for (unsigned int t0 = t_begin; t0 < t_end; t0 += kChunk) {
    // ---- decode this chunk into LDS, prefetch the next one ----
    const RawShare cur = next;
    const unsigned int tn = t0 + kChunk;
    next = load_share(body, codes, (unsigned long long)tn * row_words + share_word, half,
                      tn + tok < t_end);
    const u32x4 k0 = cur.kb0, k1 = cur.kb1, k2 = cur.kc, v0 = cur.vb0, v1 = cur.vb1, v2 = cur.vc;
    {
      // tokens past the context are written as zeros (their scores are masked)
      const bool live = t0 + tok < t_end;
      const uint32_t bk[8] = {k0.x, k0.y, k0.z, k0.w, k1.x, k1.y, k1.z, k1.w};
      const uint32_t ck[4] = {k2.x, k2.y, k2.z, k2.w};
      uint32_t o[16];
#pragma unroll
      for (int r = 0; r < 4; ++r) decode8(bk[2 * r], bk[2 * r + 1], ck[r], cbk, o + 4 * r);
#pragma unroll
      for (int r = 0; r < 16; ++r) o[r] = live ? o[r] : 0u;
      u32x4* dstk = reinterpret_cast<u32x4*>(sK + tok * kKStride + part * 32);
#pragma unroll
      for (int r = 0; r < 4; ++r) dstk[r] = u32x4{o[4 * r], o[4 * r + 1], o[4 * r + 2], o[4 * r + 3]};
      const uint32_t bv[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
      const uint32_t cv[4] = {v2.x, v2.y, v2.z, v2.w};
#pragma unroll
      for (int r = 0; r < 4; ++r) decode8(bv[2 * r], bv[2 * r + 1], cv[r], cbv, o + 4 * r);
#pragma unroll
      for (int r = 0; r < 16; ++r) o[r] = live ? o[r] : 0u;
#pragma unroll
      for (int d = 0; d < 32; ++d)
        sVt[(part * 32 + d) * kVtStride + tok] = (uint16_t)(o[d >> 1] >> (16 * (d & 1)));
    }
    __syncthreads();

    // ---- escapes of this chunk (K plane, then V plane) ----
    const unsigned int t_stop = min(t0 + kChunk, t_end);
#pragma unroll
    for (int plane = 0; plane < 2; ++plane) {
      const unsigned int base = plane ? half : 0u;
      const unsigned int hi = base + t_stop * row_words;
      for (;;) {
        const unsigned int i = ptr[plane] + tid;
        const bool valid = i < count;
        const unsigned int p = valid ? entry_pos(entries, i) : 0xFFFFFFFFu;
        const bool in = p < hi;
        // p >= base holds for an ascending list; checked so that an out-of-order
        // entry can never address outside the chunk
        if (in && p >= base) {
          const unsigned int e = entries[5ull * i + 4];
          const unsigned int q = p - base;
          const unsigned int t = q / row_words, rem = q - t * row_words;
          if (rem / kHeadDim == h && t >= t0) {
            const unsigned int dim = rem % kHeadDim, tt = t - t0;
            uint16_t* w = plane ? &sVt[dim * kVtStride + tt] : &sK[tt * kKStride + dim];
            *w = (uint16_t)((*w & 0x807F) | (e << 7));
          }
        }
        // ascending order check between this entry and the next one read
        const unsigned int next = __shfl_down(p, 1, 64);
        if (valid && lane < 63 && i + 1 < count && next < p) sBad = 1;
        const unsigned int wave_in = (unsigned int)__popcll(__ballot(in));
        if (lane == 0) sCount[wave] = wave_in;
        __syncthreads();
        const unsigned int total = sCount[0] + sCount[1] + sCount[2] + sCount[3];
        ptr[plane] += total;
        __syncthreads();
        if (total < kThreads) break;
      }
    }

    // ---- S = Q K^T for tokens 16w .. 16w+15 of the chunk ----
    f32x4 s = {0, 0, 0, 0};
    {
      const uint16_t* krow = sK + (wave * 16 + lane % 16) * kKStride + (lane / 16) * 8;
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const bf16x8 kb = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(krow + 32 * ks));
        s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qa[ks], kb, s, 0, 0, 0);
      }
    }
    // lane l < 16 holds rows 0..3 (query heads) of token 16w + l
    const bool tok_ok = t0 + wave * 16 + (lane % 16) < t_end;
    float sc[kGroup], mx[kGroup];
#pragma unroll
    for (int j = 0; j < kGroup; ++j) {
      sc[j] = (lane < 16 && tok_ok) ? s[j] * a.scale_log2 : -INFINITY;
      mx[j] = sc[j];
#pragma unroll
      for (int o = 8; o >= 1; o >>= 1) mx[j] = fmaxf(mx[j], __shfl_xor(mx[j], o, 16));
    }
    if (lane == 0) {
#pragma unroll
      for (int j = 0; j < kGroup; ++j) sRed[wave][j] = mx[j];
    }
    __syncthreads();
    float alpha[kGroup], pr[kGroup], sum[kGroup];
#pragma unroll
    for (int j = 0; j < kGroup; ++j) {
      const float cmax = fmaxf(fmaxf(sRed[0][j], sRed[1][j]), fmaxf(sRed[2][j], sRed[3][j]));
      const float m_new = fmaxf(m_run[j], cmax);
      alpha[j] = exp2f(m_run[j] - m_new);
      m_run[j] = m_new;
      pr[j] = lane < 16 && tok_ok ? exp2f(sc[j] - m_new) : 0.f;
      sum[j] = pr[j];
#pragma unroll
      for (int o = 8; o >= 1; o >>= 1) sum[j] += __shfl_xor(sum[j], o, 16);
    }
    if (lane < 16) {
#pragma unroll
      for (int j = 0; j < kGroup; ++j)
        sP[j * kPStride + wave * 16 + lane] = (uint16_t)bf16_bits(pr[j]);
    }
    if (lane == 0) {
#pragma unroll
      for (int j = 0; j < kGroup; ++j) sRed[wave][kGroup + j] = sum[j];
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < kGroup; ++j) {
      l_run[j] = l_run[j] * alpha[j] + sRed[0][kGroup + j] + sRed[1][kGroup + j] +
                 sRed[2][kGroup + j] + sRed[3][kGroup + j];
    }
    // rows held by this lane: (lane/16)*4 + j; only lanes 0..15 hold real rows
#pragma unroll
    for (int nt = 0; nt < 2; ++nt)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[nt][j] *= lane < 16 ? alpha[j] : 0.f;

    // ---- O += P V for dims 32w .. 32w+31 ----
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const bf16x8 pa = __builtin_bit_cast(
          bf16x8, *reinterpret_cast<const u32x4*>(sP + (lane % 16) * kPStride + 32 * ks + (lane / 16) * 8));
#pragma unroll
      for (int nt = 0; nt < 2; ++nt) {
        const uint16_t* vrow = sVt + (wave * 32 + nt * 16 + lane % 16) * kVtStride + 32 * ks + (lane / 16) * 8;
        const bf16x8 vb = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(vrow));
        acc[nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pa, vb, acc[nt], 0, 0, 0);
      }
    }
    __syncthreads();  // sK, sVt and sP are rewritten by the next chunk
  }

  // ---- partial results of this split ----
  const bool bad = sBad != 0;
  float* out = a.partial +
               (((unsigned long long)b * hkv + h) * a.splits + split) * kGroup * kPartial;
  if (lane < 16) {
#pragma unroll
    for (int nt = 0; nt < 2; ++nt)
#pragma unroll
      for (int j = 0; j < kGroup; ++j)
        out[j * kPartial + 2 + wave * 32 + nt * 16 + lane] = bad ? NAN : acc[nt][j];
  }
  if (wave == 0 && lane < kGroup) {
    out[lane * kPartial] = bad ? NAN : m_run[lane];
    out[lane * kPartial + 1] = bad ? NAN : l_run[lane];
  }
}

// Merges the splits of one query head: out = sum_s acc_s 2^(m_s - M) / sum_s l_s 2^(m_s - M).
__global__ __launch_bounds__(kHeadDim) void top16_attention_combine(AttnArgs a) {
  const unsigned int qh = blockIdx.x, b = blockIdx.y, d = threadIdx.x;
  const unsigned int h = qh / kGroup, g = qh % kGroup;
  const float* part = a.partial + (((unsigned long long)b * a.kv_heads + h) * a.splits) * kGroup * kPartial +
                      g * kPartial;
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
  if (isnan(big)) num = NAN;
  a.out[((unsigned long long)b * a.q_heads + qh) * kHeadDim + d] = (uint16_t)bf16_bits(num / den);
}

}  // namespace
}  // namespace unchainkv

using namespace unchainkv;

namespace {

unsigned int attention_splits(unsigned long long max_ctx) {
  const unsigned long long s = (max_ctx + 1023) / 1024;
  return (unsigned int)(s < 1 ? 1 : (s > 64 ? 64 : s));
}

}  // namespace

// Workspace bytes that kvq_splitzip_top16_decode_attention needs (no counterpart in
// the reference).
extern "C" unsigned long long kvq_splitzip_top16_decode_attention_workspace_bytes(
    unsigned long long batch, unsigned long long kv_heads, unsigned long long max_ctx) {
  const unsigned long long per_launch = batch < kMaxSeqs ? batch : kMaxSeqs;
  return per_launch * kv_heads * attention_splits(max_ctx) * kGroup * kPartial * sizeof(float);
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
  const unsigned int splits = attention_splits(max_ctx);
  const unsigned int per = (unsigned int)(((max_ctx + splits - 1) / splits + kChunk - 1) / kChunk * kChunk);
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
    a.splits = splits;
    a.tokens_per_split = per;
    a.scale_log2 = scale * 1.4426950408889634f;
    for (unsigned int r = 0; r < count; ++r) {
      a.offset[r] = payload_offsets[first + r];
      const unsigned long long ctx = context_tokens[first + r];
      a.ctx[r] = (unsigned int)ctx;
      a.span[r] = (unsigned int)((ctx + block_tokens - 1) / block_tokens * block_tokens);
    }
    hipLaunchKernelGGL(top16_attention_split, dim3(splits, (unsigned int)kv_heads, count),
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
