// GQA decode attention over the paged KV cache, gfx950.
//
// A unit is the token range [split*split_tokens, (split+1)*split_tokens) of
// stream b, KV head h, and 2^(qsplit + vsplit) workgroups of 8 wavefronts
// share it (1 to 32: V's dims in 1 or 2 parts times the group's query heads
// in 1 to 16): each computes the scores of its share of the group's query
// heads over all of the unit's K, and their output over its share of V's
// dims (all, or one half). With B*Hkv >= 128 the host uses one split (no merge at all); smaller
// batches split the context so the launch still spreads over the CUs, and a
// second small kernel merges the splits.
//
// A wavefront walks the 32-token spans wave, wave + 8, ... of its range with
// two spans' loads in flight: while one span is used the next one's loads
// are outstanding, and a span's registers are refilled as soon as it has been
// used. Per span:
//   1. the block ids of its tokens (scalar loads, one pair of spans ahead),
//      then all K and V loads;
//   2. QK^T: two v_mfma_f32_16x16x32_bf16 tiles x 4 k-steps. A = 16 K rows
//      (tokens), B = the G query heads of the group padded to 16 columns;
//   3. online softmax in fp32 in the exp2 domain (two lane swaps per column
//      reduction), rescaling the running output when a maximum grew; spans
//      whose tokens are all live skip every mask;
//   4. PV: one v_mfma_f32_16x16x32_bf16 per 16-dim tile of V the workgroup
//      computes (8, or 4 for a half), A = P straight from the QK
//      accumulators, B = V.
// MFMA multiplies along the 8 contiguous elements a lane holds, so the cache
// keeps K as 16-byte units of 8 dims of one token, tiled in the order the QK
// tiles read them (pdk::k_unit: one K load instruction reads 512 contiguous
// bytes of each of its two blocks), and V dim-major ([blk][h][D][16]: a
// lane's 8 tokens are 16 contiguous bytes). The reduction index of each
// product is permuted identically on both operands (dims in QK, tokens in
// PV), which leaves the sums unchanged:
//   QK  k-step s, lane group g, element e  <->  dim s*32 + g*8 + e;
//   QK  tile 0 row r <-> token 8(r/4) + r%4, tile 1 row r <-> that + 4, so a
//       lane's two accumulators hold tokens 8g..8g+7 of the span: exactly the
//       A-operand row segment PV needs.
// The wavefronts of a workgroup merge (max, sum, O) through LDS. Nothing is
// cleared with a memset and no state survives a launch, so the kernels can be
// captured in a HIP graph.

#include <math.h>
#include <stdlib.h>

#include <algorithm>
#include <mutex>
#include <type_traits>

#include "pdk_common.h"

namespace {

using pdk::v8;

typedef __bf16 bf16x8_t __attribute__((__vector_size__(16)));
typedef float f32x4 __attribute__((__vector_size__(16)));

constexpr int kD = 128;          // head_dim handled by the kernel
constexpr int kMaxWaves = 8;
constexpr int kSpan = 32;        // tokens per span
constexpr int kMaxG = 16;
constexpr int kMaxSplits = 32;
constexpr int kMaxCtx = 16384;   // longest context a call accepts
// LDS row stride of the wavefront merge: kD + 4 puts lane groups g and g+1
// (rows 4 apart) on different banks.
constexpr int kOStride = kD + 4;
// LDS row of the merge: the 8 wavefronts' O rows of one query head. With
// kORow = 4 (mod 8), rows 4 apart (lane groups g, g+1) start 16 banks apart.
constexpr int kORow = 8 * kOStride + 4;
constexpr int kMergeRows = 8;     // query rows merged per LDS pass

__device__ __forceinline__ bf16x8_t as_bf(const v8& v) { return __builtin_bit_cast(bf16x8_t, v); }

__device__ __forceinline__ f32x4 mfma(const v8& a, const v8& b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf(a), as_bf(b), c, 0, 0, 0);
}

struct AttnArgs {
  const uint16_t* q;
  const uint16_t* ck;
  const uint16_t* cv;
  const int32_t* tables;
  const int32_t* ctx;
  uint16_t* out;
  float* ws_ml;                  // [B*Hq][nsplit][2]
  float* ws_o;                   // [B*Hq][nsplit][D]
  int num_blocks, max_blocks, Hq, Hkv, G, nsplit, split_tokens;
  float scale_log2;              // scale * log2(e)
};

// Registers of one span between its loads and its use.
struct Span {
  v8 ka[4], kb[4], vf[8];
};

__device__ __forceinline__ bool valid_block(int blk, int num_blocks) {
  return blk >= 0 && blk < num_blocks;
}

// Issue every load of the 32-token span starting at `span`, whose tokens lie
// in the blocks blk_lo (tokens span..span+15) and blk_hi (span+16..span+31).
// kVStream: V with non-temporal loads (each V byte has one reader; K has one
// per workgroup sharing the unit); kKnt: K too, for units whose K has two
// readers (the two V halves).
// Loads are unconditional from in-bounds addresses (an invalid block id reads
// block 0) so they are all in flight together; V of tokens >= lim and of
// invalid blocks is zeroed before use, K of tokens >= lim needs nothing (their
// scores become -inf). live = false (wavefront-uniform): a span that is never
// used, loaded only so that every path issues the same loads; each
// instruction then reads one 16-byte piece of block 0 in all lanes.
template <int kNV, bool kVStream, bool kKnt>
__device__ __forceinline__ void load_span(const AttnArgs& a, int h, int span, int g, int j,
                                          int blk_lo, int blk_hi, Span& r, bool live = true) {
  // QK tile 0 row j is token span + 8(j/4) + j%4 and tile 1 row j that token
  // + 4: slots (j%8 -> j8 = j%8) of blk_lo for j < 8, of blk_hi otherwise. In
  // the tiled K block (pdk::k_unit) lanes j%8 = 0..7 of one dim group g read
  // one 128-byte line, and the four groups g four consecutive lines.
  const int tv = span + 8 * g;                   // this lane's 8 V tokens; blk_lo iff g < 2
  const int bk = (j < 8) ? blk_lo : blk_hi;
  const int bv = (g < 2) ? blk_lo : blk_hi;
  const int cbk = valid_block(bk, a.num_blocks) ? bk : 0;
  const int cbv = valid_block(bv, a.num_blocks) ? bv : 0;
  const uint16_t* pk = a.ck + ((int64_t)cbk * a.Hkv + h) * 16 * kD + (live ? (g * 8 + (j & 7)) * 8 : 0);
  const uint16_t* pv = a.cv + ((int64_t)cbv * a.Hkv + h) * kD * 16 + (live ? (tv & 15) + j * 16 : 0);
  // unit(t, s) = ((t * 4 + s) * 4 + g) * 8 + j8 with kD / 32 = 4 dim groups per tile
  if constexpr (kKnt) {
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      r.ka[s] = pdk::ld16_stream(pk + (s * 4 * 8) * 8);
      r.kb[s] = pdk::ld16_stream(pk + ((4 + s) * 4 * 8) * 8);
    }
  } else {
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      r.ka[s] = pdk::ld16(pk + (s * 4 * 8) * 8);
      r.kb[s] = pdk::ld16(pk + ((4 + s) * 4 * 8) * 8);
    }
  }
#pragma unroll
  for (int n = 0; n < kNV; ++n) r.vf[n] = pdk::ld16_as<kVStream>(pv + 16 * 16 * n);
}

// Reductions over the four lanes of one query column {i, i^16, i^32, i^48}
// with the gfx950 lane-swap instructions (VALU, no LDS round trip): after
// v_permlane32_swap each lane holds {x[i], x[i^32]}, after v_permlane16_swap
// {y[i], y[i^16]}. Both operands of each step are exchanged symmetrically, so
// every lane of the column ends with the same bits.
// Maximum that propagates NaN (v_maximum3_f32 on gfx950): unlike fmaxf it
// needs no operand canonicalisation.
__device__ __forceinline__ float vmax(float a, float b) { return __builtin_elementwise_maximum(a, b); }

// n / d for 0 <= n < 2^24 and 1 <= d < 2^24 (wavefront-uniform values):
// n * rcp(d) in fp32 is within 1 of the quotient, and one step corrects it.
__device__ __forceinline__ int div_u24(int n, int d) {
  int q = (int)((float)n * __builtin_amdgcn_rcpf((float)d));
  const int r = n - q * d;
  q += (r >= d) - (r < 0);
  return q;
}

__device__ __forceinline__ float column_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = vmax(__uint_as_float(r[0]), __uint_as_float(r[1]));
  const auto t = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return vmax(__uint_as_float(t[0]), __uint_as_float(t[1]));
}

__device__ __forceinline__ float column_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  const auto t = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(t[0]) + __uint_as_float(t[1]);
}

// The new token of the fused RoPE path: its position and its rotated k and
// its v (bf16, in LDS).
struct NewToken {
  int pos;
  const uint16_t* k;
  const uint16_t* v;
};

// Block of the new token in the span starting at `span` (its ids lo, hi), or
// -1 when the span does not hold it or the id is invalid (the block the
// token's slot was written to in the cache, if any; V of an invalid block is
// zeroed by attend_span anyway).
__device__ __forceinline__ int new_token_block(const NewToken& nt, int span, int lo, int hi,
                                               int num_blocks) {
  if (nt.pos < span || nt.pos >= span + kSpan) return -1;   // wavefront-uniform
  const int blk = (nt.pos - span < 16) ? lo : hi;
  return (blk >= 0 && blk < num_blocks) ? blk : -1;
}

// The span's K tiles take the new token's k in place of the cache's old
// contents (lane (g, j): tile 0 row j is token span + 16 (j / 8) + 8 ((j % 8)
// / 4) + j % 4, tile 1 the same + 4, pdk::k_unit's slot order). Value selects,
// not a branch choosing which register to store, keep the span in registers;
// they sit right before the QK products, which wait for these loads anyway.
__device__ __forceinline__ void patch_k(Span& r, int span, const NewToken& nt, int g, int j) {
  const int j8 = j & 7;
  const int ta = span + ((j >> 3) << 4) + ((j8 >> 2) << 3) + (j8 & 3);
  const bool in_a = ta == nt.pos, in_b = ta + 4 == nt.pos;
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const v8 k = *reinterpret_cast<const v8*>(nt.k + 32 * s + 8 * g);
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      r.ka[s].w[w] = in_a ? k.w[w] : r.ka[s].w[w];
      r.kb[s].w[w] = in_b ? k.w[w] : r.kb[s].w[w];
    }
  }
}

// The span's V rows take the new token's v (lane (g, j) holds dims j + 16n of
// tokens span + 8g .. + 7), right before the PV products.
template <int kNV>
__device__ __forceinline__ void patch_v(Span& r, int span, const NewToken& nt, int g, int j) {
  const int tv = span + 8 * g;
  const bool in_v = nt.pos >= tv && nt.pos < tv + 8;
  const int e = nt.pos - tv, word = e >> 1;
  const uint32_t keep = (e & 1) ? 0x0000ffffu : 0xffff0000u;
#pragma unroll
  for (int n = 0; n < kNV; ++n) {
    const uint32_t bits = (uint32_t)nt.v[j + 16 * n] << ((e & 1) * 16);
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const bool hit = in_v && w == word;
      r.vf[n].w[w] = hit ? ((r.vf[n].w[w] & keep) | bits) : r.vf[n].w[w];
    }
  }
}

// The read probe's stand-in for attend_span: every loaded word is folded into
// one register, so the loads stay but no arithmetic of attention is done.
template <int kNV>
__device__ __forceinline__ void fold_span(const Span& r, f32x4 o[8]) {
  uint32_t x = 0;
#pragma unroll
  for (int s = 0; s < 4; ++s)
#pragma unroll
    for (int w = 0; w < 4; ++w) x ^= r.ka[s].w[w] ^ r.kb[s].w[w];
#pragma unroll
  for (int n = 0; n < kNV; ++n)
#pragma unroll
    for (int w = 0; w < 4; ++w) x ^= r.vf[n].w[w];
  o[0][0] += (float)(x & 1u);
}

// Fold one span into the running state of query column j = lane & 15: m, the
// largest raw score so far (the same in the column's four lanes), lsum, this
// lane's own sum of weights 2^(c*s - c*m) (c = scale * log2(e) > 0; the
// column's four sums are added once, at the end), and o, the weighted sum of
// V rows (lane (g, j) holds query rows 4g..4g+3, dims 16n + j of the kNV
// 16-dim tiles the workgroup computes: all 8, or one half of V). Spans whose
// 32 tokens are all live and whose block ids are valid (a wavefront-uniform
// test) skip every mask; the others give tokens >= lim the score -inf and
// zero V of those tokens and of invalid blocks. O is rescaled only when some
// column's maximum grew, by a factor that is exactly 1 for the other columns,
// so the arithmetic of a query column is the same whatever columns share its
// wavefront.
// With kPatch (the fused RoPE path) the span's K and V take the new token nt
// in place of the cache's contents.
template <bool kPatch, int kNV>
__device__ __forceinline__ void attend_span(const AttnArgs& a, Span& r, const v8 qv[4], int span,
                                            int lo, int hi, int lim, int g, int j, bool first,
                                            float& m, float& lsum, f32x4 o[8],
                                            const NewToken& nt) {
  const int tv = span + 8 * g;
  const bool full = span + kSpan <= lim && valid_block(lo, a.num_blocks) &&
                    valid_block(hi, a.num_blocks);
  int blk = -1;
  if constexpr (kPatch) {
    blk = new_token_block(nt, span, lo, hi, a.num_blocks);
    if (blk >= 0) patch_k(r, span, nt, g, j);
  }
  f32x4 s0 = {0.f, 0.f, 0.f, 0.f}, s1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    s0 = mfma(r.ka[s], qv[s], s0);
    s1 = mfma(r.kb[s], qv[s], s1);
  }
  float sc[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    sc[i] = s0[i];
    sc[4 + i] = s1[i];
  }
  // This lane's 8 tokens lie in one block: lo for lane groups 0-1, hi for 2-3.
  const bool blk_ok = valid_block(g < 2 ? lo : hi, a.num_blocks);
  if (!full) {
    // Tokens past the context and tokens of an invalid block id take no part.
#pragma unroll
    for (int e = 0; e < 8; ++e)
      if (!blk_ok || tv + e >= lim) sc[e] = -INFINITY;
  }
  float mx = vmax(vmax(vmax(sc[0], sc[1]), vmax(sc[2], sc[3])),
                  vmax(vmax(sc[4], sc[5]), vmax(sc[6], sc[7])));
  mx = column_max(mx);                           // -inf when no token of the span is live
  const float m_new = first ? mx : vmax(m, mx);
  // With no live token so far (m_new = -inf) every weight must come out 0:
  // exp2(-inf - 0), not exp2(-inf + inf).
  const float mc = m_new == -INFINITY ? 0.f : m_new * a.scale_log2;
  float p[8], ps = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    p[e] = __builtin_amdgcn_exp2f(fmaf(sc[e], a.scale_log2, -mc));   // <= 0; exp2(-inf) = 0
    ps += p[e];
  }
  if (first) {
    lsum = ps;
  } else {
    // Exactly 1 unless this column's maximum grew (the fma would otherwise
    // leave the rounding residual of m * c in the exponent): a column's sums
    // then never depend on which other columns share the wavefront.
    // m = -inf (nothing live before this span): exp2(-inf) = 0, and O and lsum are 0.
    const float alpha = m_new > m ? __builtin_amdgcn_exp2f(fmaf(m, a.scale_log2, -mc)) : 1.f;
    lsum = lsum * alpha + ps;
    if (__any(m_new > m)) {
      float ar[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) ar[i] = __shfl(alpha, 4 * g + i);
#pragma unroll
      for (int n = 0; n < kNV; ++n)
#pragma unroll
        for (int i = 0; i < 4; ++i) o[n][i] *= ar[i];
    }
  }
  m = m_new;
  if constexpr (kPatch) {
    if (blk >= 0) patch_v<kNV>(r, span, nt, g, j);
  }
  if (!full) {
    uint32_t mk[4];
#pragma unroll
    for (int w = 0; w < 4; ++w)
      mk[w] = (blk_ok && tv + 2 * w < lim ? 0x0000ffffu : 0u) |
              (blk_ok && tv + 2 * w + 1 < lim ? 0xffff0000u : 0u);
#pragma unroll
    for (int n = 0; n < kNV; ++n)
#pragma unroll
      for (int w = 0; w < 4; ++w) r.vf[n].w[w] &= mk[w];
  }
  // Rows j >= G of P belong to padding columns; they only reach O rows that
  // are never read.
  v8 pv;
#pragma unroll
  for (int w = 0; w < 4; ++w) pv.w[w] = pdk::pack_bf16x2_rne(p[2 * w], p[2 * w + 1]);   // in [0, 1]
#pragma unroll
  for (int n = 0; n < kNV; ++n) o[n] = mfma(pv, r.vf[n], o[n]);
}

// Scalar arguments, those the first loads need first: the compiler preloads
// the leading ones into SGPRs (-amdgpu-kernarg-preload-count), so the query,
// context-length and block-id loads issue without waiting for a kernarg read.
// The first 14 dwords arrive preloaded in SGPRs, and they hold everything
// the first loads need: hgw packs Hkv (16 bits), G (8) and log2 of the
// query-head split (8); mb_b the table width max_blocks (16) and B (16);
// st_ns the split length split_tokens (16) and the split count nsplit (16).
// (gridDim would be a load from the hidden kernel arguments: one more round
// trip before any address exists.)
//
// The grid is 1-D: 2^(qsplit + kVS) workgroups share each unit (split, KV
// head, stream), each taking G / 2^qsplit of the group's query heads and, with
// kNV = 4 (kVS = 1), one half of V's dims, over the same K (part id p: query
// part p >> kVS, V half p & kVS). Units go in groups of 8 and the workgroups
// of a unit are 8 ids apart, so that they run on one XCD (workgroups are
// handed to the XCDs round robin) and read the unit's K/V once from HBM: the
// others find it in the XCD's L2. The last group, of U % 8 units, is laid out
// the same way with a stride of U % 8 (correct anywhere, local when it
// happens to be).
//
// kRope = 0: src is q [B][Hq][D] bf16. kRope = 1, 2 or 4: src is the q, k and
// v of the new token as kRope fp32 split-K partial sums of the q|k|v
// projection ([kRope][B][(Hq + 2 Hkv) D]; passing them in q's place keeps them
// among the preloaded arguments, so their loads, and the K/V loads behind
// them, do not wait for a kernel-argument read): the
// workgroup adds them in split order, rounds to bf16, rotates q and k (RoPE at
// position ctx-1, angle pos * inv_freq[i]) into LDS, writes the new k and v to
// their cache slot (the workgroup whose split holds that position), and uses
// them for the new token in place of the cache's contents. Every value is the
// one pdk_rope_cache_append_partials computes, so the result is bit-identical
// to that kernel followed by the kRope = 0 path.
// kRope = -1 is the read probe (pdk_attn_read_probe): the same launch, block
// ids and K/V loads, none of the arithmetic, one store per thread.
// kAct: out in the decode step's tiled activation layout (pdk::act_at, row b,
// column qh * D + d of Hq * D) instead of row-major [B][Hq][D].
// kKnt: K with non-temporal loads (plain path and probe with V split in two
// halves and the query heads not split, so the two halves are K's only
// readers): B=16 8.37 -> 8.26 us per layer; with 4 or 8 readers no faster.
// It is a template argument because a choice made at run time puts each K
// load between two alternative instructions, and the compiler's wait counts
// then ignore the loads on both sides of that choice: every K/V wait of the
// wavefront became a wait for nearly all of its loads.
template <int kRope, int kNV, bool kAct = false, bool kKnt = false>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2))) void decode_attn_kernel(
    const void* src, const uint16_t* ck, const uint16_t* cv, const int32_t* tables,
    const int32_t* ctx_lens, uint32_t hgw, uint32_t mb_b, int num_blocks, uint32_t st_ns,
    float scale_log2, uint16_t* out, float* ws_ml, float* ws_o, const float* inv_freq,
    uint16_t* ck_w, uint16_t* cv_w, const float* ssq, int n_ssq, float eps) {
  const uint16_t* q = static_cast<const uint16_t*>(src);
  const float* part = static_cast<const float*>(src);
  __shared__ __align__(16) float sm_m[kMaxG][kMaxWaves];
  __shared__ __align__(16) float sm_l[kMaxG][kMaxWaves];
  __shared__ __align__(16) uint16_t q_rot[kRope ? kMaxG : 1][kD];   // rotated q of the group
  __shared__ __align__(16) uint16_t kv_new[2][kD];                  // rotated k, v of the new token
  extern __shared__ float sm_o[];                // [min(G, kMergeRows)][kORow]

  AttnArgs a;
  a.Hkv = hgw & 0xffff;
  a.G = (hgw >> 16) & 0xff;
  a.Hq = a.Hkv * a.G;
  a.q = q; a.ck = ck; a.cv = cv; a.tables = tables; a.ctx = ctx_lens; a.out = out;
  a.ws_ml = ws_ml; a.ws_o = ws_o; a.num_blocks = num_blocks; a.max_blocks = mb_b & 0xffff;
  a.nsplit = st_ns >> 16; a.split_tokens = st_ns & 0xffff; a.scale_log2 = scale_log2;
  constexpr int W = kMaxWaves;                   // every launch runs 8 wavefronts
  const int nsplit = a.nsplit;
  constexpr int kVS = kNV == 8 ? 0 : 1;         // log2 of the parts V's dims are split in
  constexpr int kDV = 16 * kNV;                  // dims of O this workgroup computes
  // Non-temporal V loads: measured per layer at ctx 512 (32-layer graph) on the
  // plain path B=16 8.71 -> 8.37 us, B=8 6.98 -> 6.75, B=4 6.06 -> 5.88; on
  // the fused RoPE path no faster, and 0.15-0.3 us slower between streaming
  // kernels, so it keeps ordinary loads.
  constexpr bool kVStream = kRope <= 0;
  const int qsplit = hgw >> 24;
  static_assert(!kKnt || (kRope <= 0 && kNV == 4), "non-temporal K only on the plain V-split path");
  constexpr bool knt = kKnt;
  const int gs = qsplit + kVS;                   // log2 of the workgroups sharing a unit
  const int units = nsplit * a.Hkv * (int)(mb_b >> 16);
  const int wg = blockIdx.x, full = (units >> 3) << (3 + gs);
  int u, part_id;
  if (wg < full) {
    part_id = (wg >> 3) & ((1 << gs) - 1);
    u = ((wg >> (3 + gs)) << 3) | (wg & 7);
  } else {                                       // the last, partial group of units
    const int r = units & 7, x = wg - full;
    part_id = div_u24(x, r);
    u = (units & ~7) + (x - part_id * r);
  }
  const int qpart = part_id >> kVS, vd0 = (part_id & kVS) * kDV;
  a.cv += vd0 * 16;                              // V rows (dims) vd0 .. vd0 + kDV - 1
  const int hb = div_u24(u, nsplit), split = u - hb * nsplit;
  const int b = div_u24(hb, a.Hkv), h = hb - b * a.Hkv;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int g = lane >> 4, j = lane & 15;
  const int G = a.G >> qsplit;                   // query heads of this workgroup
  const int qh0 = h * a.G + qpart * G;           // the first of them
  int ctx_raw = a.ctx[b];
  const int s_begin = split * a.split_tokens;
  const int32_t* table = a.tables + (int64_t)b * a.max_blocks;

  v8 qv[4];
  if constexpr (kRope == 0) {
    const uint16_t* qp = a.q + ((int64_t)b * a.Hq + qh0 + min(j, G - 1)) * kD + g * 8;
#pragma unroll
    for (int s = 0; s < 4; ++s) qv[s] = pdk::ld16(qp + 32 * s);
  }
  // Columns j >= G repeat query G-1 (index clamped); their P rows only reach
  // O rows that are never read, and their (m, lsum) are never read either, so
  // Q needs no mask.

  float m = -INFINITY, lsum = 0.f;
  f32x4 o[8];
#pragma unroll
  for (int n = 0; n < 8; ++n) o[n] = f32x4{0.f, 0.f, 0.f, 0.f};

  // The wavefront index is uniform: spans and their block ids live in SGPRs,
  // so the block ids of both spans come in as scalar loads before any data
  // load is issued (a vector load here would make the second span's data
  // wait, in-order, behind the first span's). Those of the first pair do not
  // depend on the context length: they are read (at indices clamped into the
  // table) together with it, and the asm statement keeps the compiler from
  // waiting for the length first. An id read past the context is harmless:
  // load_span maps an invalid id to block 0, and tokens >= s_end are masked.
  const int wv = __builtin_amdgcn_readfirstlane(wave);
  const int stride = W * kSpan;
  const int mb = a.max_blocks - 1;
  // Fused RoPE, first phase: the partial sums of this wavefront's rows, loaded
  // before its K/V loads so that using them does not wait for those (a
  // wavefront's loads complete in order). Rows of 64 lanes: r < G the group's
  // query heads (dims lane and lane + 64), r == G the new k, r == G+1, G+2 the
  // new v (dims 64 (r - G - 1) + lane); row r belongs to wavefront r % W.
  constexpr int kPre = 4;                        // rows per wavefront loaded early
  constexpr int kParts = kRope > 0 ? kRope : 1;
  const int n_rows = G + 3;
  const int64_t n_qkv = (int64_t)(a.Hq + 2 * a.Hkv) * kD;
  const int64_t part_stride = (int64_t)(mb_b >> 16) * n_qkv;   // one split of the partials
  const float* prow = part + (int64_t)b * n_qkv;
  auto row_col = [&](int r) -> int64_t {
    return r < G ? (int64_t)(qh0 + r) * kD
         : r == G ? (int64_t)(a.Hq + h) * kD
                  : (int64_t)(a.Hq + a.Hkv + h) * kD + (r - G - 1) * 64;
  };
  float raw[kPre][2][kParts];
  float ifreq = 0.f;
  pdk::RowRms rr{};
  if constexpr (kRope > 0) {
#pragma unroll
    for (int k = 0; k < kPre; ++k) {
      const int r = wv + k * W;
      if (r < n_rows) {
        const int64_t c = row_col(r) + lane;
#pragma unroll
        for (int sp = 0; sp < kRope; ++sp) {
          raw[k][0][sp] = prow[sp * part_stride + c];
          raw[k][1][sp] = r <= G ? prow[sp * part_stride + c + 64] : 0.f;
        }
      }
    }
  }
  // Block ids of the spans at sa and sa + stride, read with scalar loads
  // (constant address space: the table is not written during the launch), so
  // that waiting for them never waits for the wavefront's K/V loads.
  typedef const __attribute__((address_space(4))) int32_t* ctable_t;
  const ctable_t ctab = (ctable_t)table;
  auto ids = [&](int sa, int* id) {
    const int sb = sa + stride;
    id[0] = ctab[min(sa >> 4, mb)];
    id[1] = ctab[min((sa >> 4) + 1, mb)];
    id[2] = ctab[min(sb >> 4, mb)];
    id[3] = ctab[min((sb >> 4) + 1, mb)];
  };
  const int sa0 = s_begin + wv * kSpan;
  int id0[4];
  ids(sa0, id0);
  asm volatile("" : "+s"(ctx_raw) : "s"(id0[0]), "s"(id0[1]), "s"(id0[2]), "s"(id0[3]));
  // The arguments past the preloaded ones (inv_freq, ssq) arrive with the
  // block ids; the row scale's loads and the frequencies go out after the
  // partial sums' and before any K/V load (a wavefront's loads complete in
  // order), and the scale is finished after the K/V loads are issued.
  if constexpr (kRope > 0) {
    if (ssq) rr = pdk::row_rms_load(ssq, b, n_ssq, lane);
    ifreq = inv_freq[lane];
  }
  const int ctx = min(ctx_raw, a.max_blocks * 16);
  const int s_end = (split == a.nsplit - 1) ? ctx : min(ctx, s_begin + a.split_tokens);
  const int pos = ctx_raw - 1;                   // the new token (fused RoPE path)
  // Loads and waits. A wavefront's loads complete in order, and the compiler
  // waits for a register with a count of the loads issued after it, taken
  // over every path that reaches the wait. So no load of the span loop sits
  // under a branch that a path around it could skip: on such a path fewer
  // loads follow, and the wait before a span's first product would drain the
  // next span's loads too (measured: waiting for 25 of a wavefront's 28 loads
  // before its first product; without it, ctx 512, 32-layer graph, B=16 8.36
  // -> 7.92 us per layer, B=8 6.84 -> 6.42, B=4 5.97 -> 5.60).
  // The first two spans' loads are issued together, and in the span loop every
  // refill is issued; a span without tokens is loaded as a dead span (one
  // 16-byte piece of block 0 per instruction, see load_span).
  const bool active = sa0 < s_end;
  const int sb0 = sa0 + stride;
  const bool has_b0 = sb0 < s_end;
  Span ra0, rb0;
  auto first_loads = [&]() __attribute__((always_inline)) {
    load_span<kNV, kVStream, knt>(a, h, sa0, g, j, active ? id0[0] : 0, active ? id0[1] : 0, ra0,
                                  active);
    load_span<kNV, kVStream, knt>(a, h, sb0, g, j, has_b0 ? id0[2] : 0, has_b0 ? id0[3] : 0, rb0,
                                  has_b0);
  };
  // With the fused RoPE a wavefront without tokens issues them too (the
  // barrier after the rotation keeps every wavefront on one path up to it);
  // on the other paths such a wavefront skips the loads and the spans at once.
  if constexpr (kRope > 0) first_loads();
  if constexpr (kRope > 0) {
    // Second phase, while the first pair's K/V loads are in flight: add the
    // partials in split order, round to bf16 (the projection's output), rotate
    // q and k with the angle pos * inv_freq[lane], and put the group's q and
    // the new k and v into LDS.
    float sn, cs;
    sincosf((float)max(pos, 0) * ifreq, &sn, &cs);
    const float rb = ssq ? pdk::row_rms_finish(rr, ssq, b, n_ssq, 16 * n_ssq, eps, lane)
                         : 1.f;
    auto rnd = [&](float x) {
      return pdk::bf16_to_f32(pdk::f32_to_bf16_rne(ssq ? x * rb : x));
    };
    auto put = [&](int r, float x0, float x1) {
      if (r <= G) {
        uint16_t* dst = r < G ? q_rot[r] : kv_new[0];
        float y0, y1;
        pdk::rope_pair(x0, x1, cs, sn, y0, y1);
        dst[lane] = (uint16_t)pdk::f32_to_bf16_rne(y0);
        dst[lane + 64] = (uint16_t)pdk::f32_to_bf16_rne(y1);
      } else {
        kv_new[1][(r - G - 1) * 64 + lane] = (uint16_t)pdk::f32_to_bf16_rne(x0);
      }
    };
#pragma unroll
    for (int k = 0; k < kPre; ++k) {
      const int r = wv + k * W;
      if (r < n_rows) {
        float x0 = raw[k][0][0], x1 = raw[k][1][0];
#pragma unroll
        for (int sp = 1; sp < kRope; ++sp) {
          x0 += raw[k][0][sp];
          x1 += raw[k][1][sp];
        }
        put(r, rnd(x0), rnd(x1));
      }
    }
    for (int r = wv + kPre * W; r < n_rows; r += W) {      // one wavefront, G = 16: late rows
      const int64_t c = row_col(r) + lane;
      float x0 = prow[c], x1 = r <= G ? prow[c + 64] : 0.f;
#pragma unroll
      for (int sp = 1; sp < kRope; ++sp) {
        x0 += prow[sp * part_stride + c];
        x1 += r <= G ? prow[sp * part_stride + c + 64] : 0.f;
      }
      put(r, rnd(x0), rnd(x1));
    }
    __syncthreads();
#pragma unroll
    for (int s = 0; s < 4; ++s)
      qv[s] = *reinterpret_cast<const v8*>(&q_rot[min(j, G - 1)][32 * s + 8 * g]);
    // The new token's k and v into its cache slot, by one wavefront of the
    // unit's first workgroup (part 0), in the split that holds the position: issued now, behind every K/V load of the wavefront, the
    // stores complete while the loads' data arrives (the spans that hold the
    // token take its k and v from LDS, not from the cache).
    if (part_id == 0 && wv == 0 && pos >= s_begin && pos < s_end) {
      const int blk = ctab[min(pos >> 4, mb)];
      if (valid_block(blk, a.num_blocks)) {
        const int slot = pos & 15;
        uint16_t* kb = ck_w + ((int64_t)blk * a.Hkv + h) * 16 * kD;
        uint16_t* vb = cv_w + ((int64_t)blk * a.Hkv + h) * kD * 16;
        if (lane < kD / 8)
          pdk::st16(kb + pdk::k_unit(slot, 8 * lane, kD) * 8,
                    *reinterpret_cast<const v8*>(&kv_new[0][8 * lane]));
#pragma unroll
        for (int d = lane; d < kD; d += 64) vb[(int64_t)d * 16 + slot] = kv_new[1][d];
      }
    }
  }
  const NewToken nt{pos, kv_new[0], kv_new[1] + vd0};
  // A wavefront's spans are sa0 + k * stride. Two of them are in registers at
  // a time (ra, rb): while one is used the other's loads are in flight, and a
  // span's registers are refilled with the span two ahead as soon as it has
  // been used. The block ids of the next pair are read one pair ahead.
  auto use = [&](auto first_c, Span& r, int s, int lo, int hi) __attribute__((always_inline)) {
    if constexpr (kRope < 0) fold_span<kNV>(r, o);
    else attend_span<(kRope > 0), kNV>(a, r, qv, s, lo, hi, s_end, g, j,
                                       decltype(first_c)::value, m, lsum, o, nt);
  };
  // Spans sa and sa + stride with the span sa + 2 stride still to come: use
  // both and refill both (the second refill dead when sa + 3 stride has no
  // tokens).
  auto pair = [&](auto first_c, int sa, const int* cur, int* nxt) __attribute__((always_inline)) {
    const int sc = sa + 2 * stride, sd = sc + stride;
    const bool has_d = sd < s_end;
    ids(sc, nxt);
    use(first_c, ra0, sa, cur[0], cur[1]);
    load_span<kNV, kVStream, knt>(a, h, sc, g, j, nxt[0], nxt[1], ra0);
    use(std::false_type{}, rb0, sa + stride, cur[2], cur[3]);
    load_span<kNV, kVStream, knt>(a, h, sd, g, j, has_d ? nxt[2] : 0, has_d ? nxt[3] : 0, rb0, has_d);
  };
  // The last one or two spans, already in registers: no loads.
  auto last = [&](auto first_c, int sa, const int* cur) __attribute__((always_inline)) {
    use(first_c, ra0, sa, cur[0], cur[1]);
    if (sa + stride < s_end) use(std::false_type{}, rb0, sa + stride, cur[2], cur[3]);
  };
  auto spans = [&]() __attribute__((always_inline)) {
    if (sa0 + 2 * stride < s_end) {
      int cur[4], nxt[4];
      pair(std::true_type{}, sa0, id0, nxt);
      int sa = sa0 + 2 * stride;
      for (; sa + 2 * stride < s_end; sa += 2 * stride) {
#pragma unroll
        for (int i = 0; i < 4; ++i) cur[i] = nxt[i];
        pair(std::false_type{}, sa, cur, nxt);
      }
      last(std::false_type{}, sa, nxt);
    } else {
      last(std::true_type{}, sa0, id0);
    }
  };
  // The fused RoPE path with whole V (kNV = 8) keeps a loop whose refills are
  // conditional: there the loop above needs more than the 256 registers a
  // lane has (it spilled; a serving step at contexts up to 1152, split in two
  // then and so run with whole V, went from 3.07 to 5.1 ms). With V split in
  // halves it runs the loop above (190 registers): 16-stream steps at
  // contexts U[128, 1152] 3.028-3.031 -> 3.020-3.025 ms.
  auto pair_cond = [&](auto first_c, int sa, const int* cur, int* nxt) __attribute__((always_inline)) {
    const int sb = sa + stride, sc = sa + 2 * stride, sd = sa + 3 * stride;
    if (sc < s_end) ids(sc, nxt);
    use(first_c, ra0, sa, cur[0], cur[1]);
    if (sc < s_end) load_span<kNV, kVStream, knt>(a, h, sc, g, j, nxt[0], nxt[1], ra0);
    if (sb < s_end) use(std::false_type{}, rb0, sb, cur[2], cur[3]);
    if (sd < s_end) load_span<kNV, kVStream, knt>(a, h, sd, g, j, nxt[2], nxt[3], rb0);
    return sc;
  };
  if (active) {
    if constexpr (kRope <= 0) {
      first_loads();
      spans();
    } else if constexpr (kNV == 4) {
      spans();                                   // first pair issued before the rotation
    } else {
      int cur[4], nxt[4];
      for (int sa = pair_cond(std::true_type{}, sa0, id0, cur); sa < s_end;) {
#pragma unroll
        for (int i = 0; i < 4; ++i) nxt[i] = cur[i];
        sa = pair_cond(std::false_type{}, sa, nxt, cur);
      }
    }
  }
  const int64_t bq0 = (int64_t)b * a.Hq + qh0;
  if constexpr (kRope < 0) {
    const int t = threadIdx.x;
    if (t < G * kDV) a.out[(bq0 + t / kDV) * kD + vd0 + t % kDV] = (uint16_t)__float_as_uint(o[0][0]);
    return;
  }
  lsum = column_sum(lsum);
  m *= a.scale_log2;                             // log2 domain for the merge (-inf stays)

  // Merge the 8 wavefronts through LDS, one barrier per 8 query rows. Lane
  // (g, j) holds O rows 4g..4g+3 (the group's query heads), dims 16n+j; the
  // four lanes of column j hold the same (m, lsum). Every wavefront writes its
  // slot, also one without tokens (m = -inf, lsum = 0, O = 0), so the combine
  // reads all 8 slots unconditionally: (m, lsum) as two 16-byte vectors per
  // row, O at fixed offsets from one address. A slot with m = -inf weighs 0.
  if (g == 0 && j < G) {
    sm_m[j][wave] = m;
    sm_l[j][wave] = lsum;
  }
  const int R = min(G, kMergeRows);              // rows per pass; one pass for G <= 8
  for (int r0 = 0; r0 < G; r0 += R) {
    if (r0 > 0) __syncthreads();                 // the previous pass has read sm_o
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = 4 * g + i - r0;
      if (row >= 0 && row < R && row + r0 < G) {
#pragma unroll
        for (int n = 0; n < kNV; ++n) sm_o[row * kORow + wave * kOStride + 16 * n + j] = o[n][i];
      }
    }
    __syncthreads();
    for (int idx = threadIdx.x; idx < R * kDV; idx += 64 * kMaxWaves) {
      const int row = idx / kDV, d = idx % kDV;
      const f32x4 ma = *reinterpret_cast<const f32x4*>(&sm_m[r0 + row][0]);
      const f32x4 mb = *reinterpret_cast<const f32x4*>(&sm_m[r0 + row][4]);
      const f32x4 la = *reinterpret_cast<const f32x4*>(&sm_l[r0 + row][0]);
      const f32x4 lb = *reinterpret_cast<const f32x4*>(&sm_l[r0 + row][4]);
      const float* po = &sm_o[row * kORow + d];
      float ow[kMaxWaves];
#pragma unroll
      for (int w = 0; w < kMaxWaves; ++w) ow[w] = po[w * kOStride];
      const float mw[kMaxWaves] = {ma[0], ma[1], ma[2], ma[3], mb[0], mb[1], mb[2], mb[3]};
      const float lw[kMaxWaves] = {la[0], la[1], la[2], la[3], lb[0], lb[1], lb[2], lb[3]};
      const float M = vmax(vmax(vmax(mw[0], mw[1]), vmax(mw[2], mw[3])),
                           vmax(vmax(mw[4], mw[5]), vmax(mw[6], mw[7])));
      // M = -inf: no token at all in this split (m = -inf everywhere).
      const float Mc = M == -INFINITY ? 0.f : M;
      float L = 0.f, O = 0.f;
#pragma unroll
      for (int w = 0; w < kMaxWaves; ++w) {
        const float c = __builtin_amdgcn_exp2f(mw[w] - Mc);   // <= 0; exp2(-inf) = 0
        L = fmaf(lw[w], c, L);
        O = fmaf(ow[w], c, O);
      }
      const int64_t bq = bq0 + r0 + row;
      if (a.nsplit == 1) {
        const float inv = L > 0.f ? __builtin_amdgcn_rcpf(L) : 0.f;
        const int64_t at = kAct ? pdk::act_at(b, (qh0 + r0 + row) * kD + vd0 + d, a.Hq * kD)
                                : bq * kD + vd0 + d;
        a.out[at] = (uint16_t)pdk::f32_to_bf16_rne(O * inv);
      } else {
        a.ws_o[(bq * a.nsplit + split) * kD + vd0 + d] = O;
        if (vd0 + d == 0) {
          a.ws_ml[(bq * a.nsplit + split) * 2 + 0] = M;
          a.ws_ml[(bq * a.nsplit + split) * 2 + 1] = L;
        }
      }
    }
  }
}

// out = sum_s 2^(m_s-M) O_s / sum_s 2^(m_s-M) l_s, all partial loads independent.
// kAct: out in the tiled activation layout (row bq / Hq, column (bq % Hq) * D + d).
template <bool kAct>
__global__ __launch_bounds__(128) void merge_kernel(const float* ws_ml, const float* ws_o,
                                                    int nsplit, uint16_t* out, int Hq) {
  const int64_t bq = blockIdx.x;
  const int d = threadIdx.x;
  const float* ml = ws_ml + bq * nsplit * 2;
  const float* po = ws_o + bq * nsplit * kD + d;
  float mv[kMaxSplits], lv[kMaxSplits], ov[kMaxSplits];
  float M = -INFINITY;
#pragma unroll
  for (int s = 0; s < kMaxSplits; ++s) {
    if (s < nsplit) {
      mv[s] = ml[2 * s];
      lv[s] = ml[2 * s + 1];
      ov[s] = po[(int64_t)s * kD];
      M = fmaxf(M, mv[s]);
    }
  }
  float L = 0.f, O = 0.f;
  if (M != -INFINITY) {
#pragma unroll
    for (int s = 0; s < kMaxSplits; ++s) {
      if (s < nsplit && mv[s] != -INFINITY) {
        const float c = __builtin_amdgcn_exp2f(mv[s] - M);   // argument <= 0
        L += lv[s] * c;
        O += ov[s] * c;
      }
    }
  }
  const int64_t at = kAct ? pdk::act_at((int)(bq / Hq), (int)(bq % Hq) * kD + d, Hq * kD)
                          : bq * kD + d;
  out[at] = (uint16_t)pdk::f32_to_bf16_rne(L > 0.f ? O * __builtin_amdgcn_rcpf(L) : 0.f);
}

// New token's k/v into slot ctx[b]-1 (kernels/decode_batch.py:81-82 as a store).
__global__ void cache_append_kernel(const uint16_t* k_new, const uint16_t* v_new, uint16_t* ck,
                                    uint16_t* cv, int num_blocks, const int32_t* tables,
                                    int max_blocks, const int32_t* ctx, int Hkv, int D) {
  const int b = blockIdx.x, h = blockIdx.y;
  const int t = ctx[b] - 1;
  if (t < 0 || t >= max_blocks * 16) return;
  const int blk = tables[(int64_t)b * max_blocks + (t >> 4)];
  if (blk < 0 || blk >= num_blocks) return;
  const int slot = t & 15;
  uint16_t* kb = ck + ((int64_t)blk * Hkv + h) * 16 * D;
  for (int d = threadIdx.x; d < D; d += blockDim.x) {
    const int64_t src = ((int64_t)b * Hkv + h) * D + d;
    kb[pdk::k_unit(slot, d & ~7, D) * 8 + (d & 7)] = k_new[src];
    cv[(((int64_t)blk * Hkv + h) * D + d) * 16 + slot] = v_new[src];
  }
}

int64_t round_up(int64_t x, int64_t m) { return (x + m - 1) / m * m; }

// Scratch of pdk_decode_attn_noalloc: the split partials (what the workspace
// argument of pdk_decode_attn holds) in a file-scope device array, so that a
// caller that cannot allocate needs none. Each GPU holds its own copy. Host
// code never passes `scratch` itself to a kernel (in host code the name is a
// stand-in, not a device address): the device address comes from
// hipGetSymbolAddress, once per device, and is kept in scratch_ptr.
static __device__ __align__(256) char scratch[PDK_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
void* scratch_ptr[kMaxDevices];
std::mutex scratch_mu;

// The current device's scratch address (looked up on the first call on that
// device, with it current); null and an error message on failure.
void* device_scratch() {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    (void)hipGetLastError();
    pdk::set_error("no current HIP device (or device index >= %d)", kMaxDevices);
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(scratch_mu);
  if (!scratch_ptr[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      pdk::hip_fail(e != hipSuccess ? e : hipErrorInvalidSymbol,
                    "hipGetSymbolAddress(scratch)");
      return nullptr;
    }
    scratch_ptr[dev] = p;
  }
  return scratch_ptr[dev];
}

// Launch plan. One workgroup per (stream, KV head, split), up to 8
// wavefronts of 64 tokens each in flight. The context is split across
// workgroups until about 256 of them (one per CU) exist, in splits of at least
// min_split tokens, because a split costs the partial-result merge (an extra
// launch): 2048 once B*Hkv alone reaches 128 workgroups, 512 from 32, 128
// below. Measured per layer on MI355X, Hq=32, Hkv=8 (32-layer graph), B=16:
// ctx 1152 one split 14.85 us vs two 17.20, ctx 2048 one 24.02 vs two 25.47,
// ctx 4096 two 45.1 vs one 47.2, ctx 8192 two 83.8 vs one 95.4; B=8 and B=4
// at ctx 1152-4096: splits of 512 the fastest or within 4 % of it; at ctx 512
// one split: B=4 5.60 us against 7.22-7.87 in splits of 256, 128 or 64 tokens,
// B=8 6.19 against 8.46-8.79. (Before
// the span loads were issued on every path, B=16 ctx 2048 was faster in two
// splits, 28.9 vs 32.3 us, and the threshold was 1024: a decode step whose
// tables hold 1152 tokens took 3.21 ms at ctx 512 instead of 3.01.)
struct Plan {
  int nsplit, split_tokens;
  int qsplit;                    // log2 of the parts a unit's query heads are split in
  int vsplit;                    // 1: V's dims split in two halves, 0: whole
};

constexpr int kTargetWorkgroups = 256;

// After the context split, units (split, KV head, stream) that still leave
// CUs idle are shared by 2, 4 or 8 workgroups on one XCD, which read the same
// K from HBM once (the others find it in the XCD's L2). First V's dims are
// split in two halves (each workgroup reads all of K, half of V, and computes
// all the group's scores and half of their output), then the group's query
// heads. A query's arithmetic is the same whichever workgroup computes it and
// whatever other queries share its wavefront, so the plan never changes a
// result. Measured per layer at ctx 512, Hq 32, Hkv 8 (32-layer graph, MI355X,
// us, heads split in 2^q, V split in 2^v, as (q, v)): B=16 (1, 0) 9.12,
// (0, 1) 8.72, (1, 1) 13.0 (512 workgroups); B=8 (2, 0) 7.91, (0, 1) 7.26,
// (1, 1) 6.99; B=4 (2, 0) 7.13, (1, 1) 6.17, (2, 1) 6.07.
// The context split is chosen for plan_B streams (it orders the fp32 sums, so
// a decoder keeps it fixed across steps), the sharing for the B launched.
Plan plan_for(int B, int plan_B, int Hkv, int G, int max_ctx) {
  const int64_t pairs = (int64_t)plan_B * Hkv;
  const int min_split = pairs >= 128 ? 2048 : pairs >= 32 ? 512 : 128;
  int64_t nsplit = (kTargetWorkgroups + pairs - 1) / pairs;
  nsplit = std::min<int64_t>(nsplit, (max_ctx + min_split - 1) / min_split);
  nsplit = std::max<int64_t>(1, std::min<int64_t>(nsplit, kMaxSplits));
  const int split_tokens = (int)round_up((max_ctx + nsplit - 1) / nsplit, kSpan);
  const int ns = (max_ctx + split_tokens - 1) / split_tokens;
  const int64_t units = (int64_t)B * Hkv * ns;
  const int vs = units * 2 <= kTargetWorkgroups ? 1 : 0;
  int qs = 0;
  while ((2 << qs) <= G && (units << (vs + qs + 1)) <= kTargetWorkgroups) ++qs;
  return {ns, split_tokens, qs, vs};
}

size_t ws_bytes(int B, int Hq, int nsplit) {
  if (nsplit <= 1) return 0;
  const int64_t bq = (int64_t)B * Hq;
  return (size_t)(round_up(bq * nsplit * 2 * 4, 256) + bq * nsplit * kD * 4);
}

}  // namespace

extern "C" size_t pdk_decode_attn_workspace_bytes(int B, int n_q_heads, int max_ctx, int head_dim) {
  if (B <= 0 || n_q_heads <= 0 || head_dim <= 0 || max_ctx <= 0) return 0;
  // The most splits a plan uses for any n_kv_heads <= n_q_heads.
  return ws_bytes(B, n_q_heads, min(kMaxSplits, max(1, (max_ctx + 127) / 128)));
}

namespace {

// Inputs of the fused RoPE path (null part: q given).
struct RopeIn {
  const float* part;
  int splits;
  const float* inv_freq;
  uint16_t* ck_w;
  uint16_t* cv_w;
  const float* ssq = nullptr;    // folded-norm row scale (pdk::row_rms), or none
  int n_ssq = 0;
  float eps = 0.f;
  bool probe = false;            // pdk_attn_read_probe: loads only
  bool act = false;              // out in the tiled activation layout (pdk::act_at)
};

// The kernel for a plan: V in halves or whole, and on the plain path and the
// probe non-temporal K when the two V halves are K's only readers.
template <int kRope, bool kAct>
auto attn_kernel_for(const Plan& p) {
  if constexpr (kRope <= 0) {
    if (p.vsplit && p.qsplit == 0) return decode_attn_kernel<kRope, 4, kAct, true>;
  }
  return p.vsplit ? decode_attn_kernel<kRope, 4, kAct, false> : decode_attn_kernel<kRope, 8, kAct, false>;
}

int launch_attn(const uint16_t* q, const uint16_t* cache_k, const uint16_t* cache_v,
                int num_blocks, const int32_t* block_tables, int max_blocks,
                const int32_t* ctx_lens, int max_ctx, int B, int n_q_heads, int n_kv_heads,
                int head_dim, float scale, void* workspace, size_t workspace_bytes, uint16_t* out,
                uintptr_t stream, const RopeIn& rope, int plan_B) {
  if (head_dim != kD) {
    pdk::set_error("decode attention implements head_dim %d only (got %d)", kD, head_dim);
    return PDK_ENOTSUP;
  }
  PDK_REQUIRE(B >= 1 && B <= 65535, "B must be in [1, 65535] (got %d)", B);
  PDK_REQUIRE(n_kv_heads >= 1 && n_kv_heads <= 65535, "n_kv_heads out of range (%d)", n_kv_heads);
  PDK_REQUIRE(n_q_heads >= n_kv_heads && n_q_heads % n_kv_heads == 0,
              "n_q_heads=%d must be a multiple of n_kv_heads=%d", n_q_heads, n_kv_heads);
  const int G = n_q_heads / n_kv_heads;
  if (G > kMaxG || (G & (G - 1)) != 0) {
    pdk::set_error("GQA group %d not in {1,2,4,8,16}", G);
    return PDK_ENOTSUP;
  }
  PDK_REQUIRE((q || rope.part || rope.probe) && cache_k && cache_v && out && block_tables && ctx_lens,
              "null pointer argument");
  PDK_REQUIRE((!q || pdk::aligned16(q)) && pdk::aligned16(cache_k) && pdk::aligned16(cache_v),
              "q/cache_k/cache_v must be 16-byte aligned");
  PDK_REQUIRE(num_blocks >= 1 && max_blocks >= 1 && max_blocks <= 65535,
              "num_blocks must be >= 1 and max_blocks in [1, 65535]");
  PDK_REQUIRE(max_ctx >= 1 && max_ctx <= max_blocks * 16,
              "max_ctx=%d outside [1, max_blocks*16=%d]", max_ctx, max_blocks * 16);
  // The largest context the tests cover (and the header promises).
  if (max_ctx > kMaxCtx) {
    pdk::set_error("max_ctx=%d above the supported %d", max_ctx, kMaxCtx);
    return PDK_ENOTSUP;
  }
  PDK_REQUIRE(scale > 0.f && scale < INFINITY, "scale must be positive and finite (got %g)",
              (double)scale);
  PDK_REQUIRE(plan_B >= B && plan_B <= 65535, "plan_batch=%d must be in [B=%d, 65535]", plan_B, B);
  const Plan p = plan_for(B, plan_B, n_kv_heads, G, max_ctx);
  AttnArgs a{};
  a.q = q;
  a.ck = cache_k;
  a.cv = cache_v;
  a.tables = block_tables;
  a.ctx = ctx_lens;
  a.out = out;
  a.num_blocks = num_blocks;
  a.max_blocks = max_blocks;
  a.Hq = n_q_heads;
  a.Hkv = n_kv_heads;
  a.G = G;
  a.nsplit = p.nsplit;
  a.split_tokens = p.split_tokens;
  a.scale_log2 = scale * 1.4426950408889634f;
  if (p.nsplit > 1 && !rope.probe) {
    const size_t need = ws_bytes(B, n_q_heads, p.nsplit);
    PDK_REQUIRE(workspace && workspace_bytes >= need && pdk::aligned16(workspace),
                "workspace of %zu bytes needed (got %zu)", need, workspace_bytes);
    char* base = static_cast<char*>(workspace);
    const int64_t bq = (int64_t)B * n_q_heads;
    a.ws_ml = reinterpret_cast<float*>(base);
    a.ws_o = reinterpret_cast<float*>(base + round_up(bq * p.nsplit * 2 * 4, 256));
  }
  hipStream_t st = pdk::as_stream(stream);
  const size_t lds = (size_t)min(G, kMergeRows) * kORow * sizeof(float);
  const int64_t units = (int64_t)p.nsplit * n_kv_heads * B;
  PDK_REQUIRE(units < (1 << 24), "B * n_kv_heads * splits = %lld is too large", (long long)units);
  const int64_t n_wg = units << (p.qsplit + p.vsplit);
  const uint32_t hgw = (uint32_t)n_kv_heads | ((uint32_t)G << 16) | ((uint32_t)p.qsplit << 24);
  const uint32_t mb_b = (uint32_t)max_blocks | ((uint32_t)B << 16);
  const uint32_t st_ns = (uint32_t)p.split_tokens | ((uint32_t)p.nsplit << 16);
  const dim3 grid((uint32_t)n_wg), block(64 * kMaxWaves);
  const void* src = rope.part ? static_cast<const void*>(rope.part) : static_cast<const void*>(a.q);
#define PDK_ATTN_LAUNCH(R, A)                                                                   \
  do {                                                                                         \
    const auto kern = attn_kernel_for<R, A>(p);                                                \
    hipLaunchKernelGGL(kern, grid, block, lds, st, src, a.ck, a.cv, a.tables, a.ctx, hgw, mb_b, \
                       a.num_blocks, st_ns, a.scale_log2, a.out, a.ws_ml, a.ws_o,              \
                       rope.inv_freq, rope.ck_w, rope.cv_w, rope.ssq, rope.n_ssq, rope.eps);   \
  } while (0)
  const int mode = rope.probe ? -1 : rope.part ? rope.splits : 0;
  if (rope.act) {
    switch (mode) {
      case 1: PDK_ATTN_LAUNCH(1, true); break;
      case 2: PDK_ATTN_LAUNCH(2, true); break;
      case 4: PDK_ATTN_LAUNCH(4, true); break;
      default:
        pdk::set_error("splits must be 1, 2 or 4 (got %d)", rope.splits);
        return PDK_EINVAL;
    }
  } else {
    switch (mode) {
      case -1: PDK_ATTN_LAUNCH(-1, false); break;
      case 0: PDK_ATTN_LAUNCH(0, false); break;
      case 1: PDK_ATTN_LAUNCH(1, false); break;
      case 2: PDK_ATTN_LAUNCH(2, false); break;
      case 4: PDK_ATTN_LAUNCH(4, false); break;
      default:
        pdk::set_error("splits must be 1, 2 or 4 (got %d)", rope.splits);
        return PDK_EINVAL;
    }
  }
#undef PDK_ATTN_LAUNCH
  int rc = pdk::check_launch("decode_attn_kernel");
  if (rc || p.nsplit == 1 || rope.probe) return rc;
  if (rope.act)
    hipLaunchKernelGGL(merge_kernel<true>, dim3(B * n_q_heads), dim3(kD), 0, st, a.ws_ml, a.ws_o,
                       p.nsplit, out, n_q_heads);
  else
    hipLaunchKernelGGL(merge_kernel<false>, dim3(B * n_q_heads), dim3(kD), 0, st, a.ws_ml,
                       a.ws_o, p.nsplit, out, n_q_heads);
  return pdk::check_launch("merge_kernel");
}

}  // namespace

extern "C" int pdk_decode_attn(const uint16_t* q, const uint16_t* cache_k, const uint16_t* cache_v,
                               int num_blocks, const int32_t* block_tables, int max_blocks,
                               const int32_t* ctx_lens, int max_ctx, int B, int n_q_heads,
                               int n_kv_heads, int head_dim, float scale, void* workspace,
                               size_t workspace_bytes, uint16_t* out, uintptr_t stream) {
  pdk::clear_error();
  PDK_REQUIRE(q, "null pointer argument");
  return launch_attn(q, cache_k, cache_v, num_blocks, block_tables, max_blocks, ctx_lens, max_ctx,
                     B, n_q_heads, n_kv_heads, head_dim, scale, workspace, workspace_bytes, out,
                     stream, RopeIn{nullptr, 0, nullptr, nullptr, nullptr}, B);
}

extern "C" int pdk_decode_attn_noalloc(const uint16_t* q, const uint16_t* cache_k,
                                       const uint16_t* cache_v, int num_blocks,
                                       const int32_t* block_tables, int max_blocks,
                                       const int32_t* ctx_lens, int max_ctx, int B,
                                       int n_q_heads, int n_kv_heads, int head_dim, float scale,
                                       uint16_t* out, uintptr_t stream) {
  pdk::clear_error();
  PDK_REQUIRE(q, "null pointer argument");
  PDK_REQUIRE(B >= 1 && n_q_heads >= 1 && n_kv_heads >= 1 && max_ctx >= 1 && head_dim == kD,
              "bad shape (B=%d, Hq=%d, Hkv=%d, max_ctx=%d, D=%d)", B, n_q_heads, n_kv_heads,
              max_ctx, head_dim);
  PDK_REQUIRE(n_q_heads % n_kv_heads == 0, "n_q_heads=%d must be a multiple of n_kv_heads=%d",
              n_q_heads, n_kv_heads);
  const Plan p = plan_for(B, B, n_kv_heads, n_q_heads / n_kv_heads, max_ctx);
  const size_t need = ws_bytes(B, n_q_heads, p.nsplit);
  if (need > PDK_NOALLOC_SCRATCH_BYTES) {
    pdk::set_error("this launch needs %zu bytes of split partials; the no-allocation entry "
                   "point holds at most %zu (use pdk_decode_attn with a workspace)",
                   need, (size_t)PDK_NOALLOC_SCRATCH_BYTES);
    return PDK_ENOMEM;
  }
  void* ws = nullptr;
  if (need > 0) {
    ws = device_scratch();
    if (!ws) return PDK_EHIP;
  }
  return launch_attn(q, cache_k, cache_v, num_blocks, block_tables, max_blocks, ctx_lens, max_ctx,
                     B, n_q_heads, n_kv_heads, head_dim, scale, ws, need, out, stream,
                     RopeIn{nullptr, 0, nullptr, nullptr, nullptr}, B);
}

extern "C" int pdk_decode_attn_rope(const float* qkv_partials, int splits, const float* inv_freq,
                                    uint16_t* cache_k, uint16_t* cache_v, int num_blocks,
                                    const int32_t* block_tables, int max_blocks,
                                    const int32_t* ctx_lens, int max_ctx, int B, int n_q_heads,
                                    int n_kv_heads, int head_dim, float scale, void* workspace,
                                    size_t workspace_bytes, uint16_t* out, int plan_batch,
                                    uintptr_t stream) {
  pdk::clear_error();
  PDK_REQUIRE(qkv_partials && inv_freq, "null pointer argument");
  PDK_REQUIRE(splits == 1 || splits == 2 || splits == 4, "splits must be 1, 2 or 4 (got %d)",
              splits);
  return launch_attn(nullptr, cache_k, cache_v, num_blocks, block_tables, max_blocks, ctx_lens,
                     max_ctx, B, n_q_heads, n_kv_heads, head_dim, scale, workspace,
                     workspace_bytes, out, stream,
                     RopeIn{qkv_partials, splits, inv_freq, cache_k, cache_v},
                     plan_batch > 0 ? plan_batch : B);
}

extern "C" int pdk_decode_attn_rope_xt(const float* qkv_partials, int splits,
                                       const float* inv_freq, uint16_t* cache_k,
                                       uint16_t* cache_v, int num_blocks,
                                       const int32_t* block_tables, int max_blocks,
                                       const int32_t* ctx_lens, int max_ctx, int B, int n_q_heads,
                                       int n_kv_heads, int head_dim, float scale, void* workspace,
                                       size_t workspace_bytes, uint16_t* out, int plan_batch,
                                       uintptr_t stream) {
  pdk::clear_error();
  PDK_REQUIRE(qkv_partials && inv_freq, "null pointer argument");
  PDK_REQUIRE(splits == 1 || splits == 2 || splits == 4, "splits must be 1, 2 or 4 (got %d)",
              splits);
  PDK_REQUIRE((int64_t)n_q_heads * head_dim % 128 == 0,
              "tiled activations need n_q_heads * head_dim %% 128 == 0");
  RopeIn rope{qkv_partials, splits, inv_freq, cache_k, cache_v};
  rope.act = true;
  return launch_attn(nullptr, cache_k, cache_v, num_blocks, block_tables, max_blocks, ctx_lens,
                     max_ctx, B, n_q_heads, n_kv_heads, head_dim, scale, workspace,
                     workspace_bytes, out, stream, rope, plan_batch > 0 ? plan_batch : B);
}

extern "C" int pdk_decode_attn_rope_rms(const float* qkv_partials, int splits,
                                        const float* ssq, int n_ssq, float eps,
                                        const float* inv_freq, uint16_t* cache_k,
                                        uint16_t* cache_v, int num_blocks,
                                        const int32_t* block_tables, int max_blocks,
                                        const int32_t* ctx_lens, int max_ctx, int B, int n_q_heads,
                                        int n_kv_heads, int head_dim, float scale, void* workspace,
                                        size_t workspace_bytes, uint16_t* out, int plan_batch,
                                        uintptr_t stream) {
  pdk::clear_error();
  PDK_REQUIRE(qkv_partials && inv_freq && ssq, "null pointer argument");
  PDK_REQUIRE(splits == 1 || splits == 2 || splits == 4, "splits must be 1, 2 or 4 (got %d)",
              splits);
  PDK_REQUIRE(n_ssq >= 1 && eps > 0.f, "n_ssq must be >= 1 and eps positive");
  RopeIn rope{qkv_partials, splits, inv_freq, cache_k, cache_v};
  rope.ssq = ssq;
  rope.n_ssq = n_ssq;
  rope.eps = eps;
  return launch_attn(nullptr, cache_k, cache_v, num_blocks, block_tables, max_blocks, ctx_lens,
                     max_ctx, B, n_q_heads, n_kv_heads, head_dim, scale, workspace,
                     workspace_bytes, out, stream, rope, plan_batch > 0 ? plan_batch : B);
}

extern "C" int pdk_attn_read_probe(const uint16_t* cache_k, const uint16_t* cache_v,
                                   int num_blocks, const int32_t* block_tables, int max_blocks,
                                   const int32_t* ctx_lens, int max_ctx, int B, int n_q_heads,
                                   int n_kv_heads, int head_dim, uint16_t* out, uintptr_t stream) {
  pdk::clear_error();
  RopeIn probe{nullptr, 0, nullptr, nullptr, nullptr};
  probe.probe = true;
  return launch_attn(nullptr, cache_k, cache_v, num_blocks, block_tables, max_blocks, ctx_lens,
                     max_ctx, B, n_q_heads, n_kv_heads, head_dim, 1.f, nullptr, 0, out, stream,
                     probe, B);
}

extern "C" int pdk_cache_append(const uint16_t* k_new, const uint16_t* v_new, uint16_t* cache_k,
                                uint16_t* cache_v, int num_blocks, const int32_t* block_tables,
                                int max_blocks, const int32_t* ctx_lens, int B, int n_kv_heads,
                                int head_dim, uintptr_t stream) {
  pdk::clear_error();
  PDK_REQUIRE(k_new && v_new && cache_k && cache_v && block_tables && ctx_lens,
              "null pointer argument");
  PDK_REQUIRE(B >= 1 && B <= 65535 && n_kv_heads >= 1 && n_kv_heads <= 65535,
              "B/n_kv_heads out of range");
  PDK_REQUIRE(head_dim >= 32 && head_dim % 32 == 0 && head_dim <= 4096,
              "head_dim must be a multiple of 32 in [32, 4096] (got %d)", head_dim);
  PDK_REQUIRE(num_blocks >= 1 && max_blocks >= 1, "num_blocks and max_blocks must be >= 1");
  hipLaunchKernelGGL(cache_append_kernel, dim3(B, n_kv_heads), dim3(128), 0,
                     pdk::as_stream(stream), k_new, v_new, cache_k, cache_v, num_blocks,
                     block_tables, max_blocks, ctx_lens, n_kv_heads, head_dim);
  return pdk::check_launch("cache_append_kernel");
}
