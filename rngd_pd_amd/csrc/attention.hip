// GQA decode attention over the paged KV cache, gfx950.
//
// Grid (nsplit, Hkv, B); a workgroup of W wavefronts (W <= 8) owns the token
// range [split*split_tokens, (split+1)*split_tokens) of stream b, KV head h.
// With B*Hkv >= 128 the host uses one split (no merge at all); smaller batches
// split the context so the launch still spreads over the CUs, and a second
// small kernel merges the splits.
//
// A wavefront walks 32-token spans, two per iteration (both spans' loads in
// flight together); per span:
//   1. the block ids of its tokens (three loads), then all K and V loads;
//   2. QK^T: two v_mfma_f32_16x16x32_bf16 tiles x 4 k-steps. A = 16 K rows
//      (tokens), B = the G query heads of the group padded to 16 columns;
//   3. online softmax in fp32 in the exp2 domain (two lane shuffles per
//      reduction), rescaling the running output;
//   4. PV: 8 v_mfma_f32_16x16x32_bf16 (one per 16-dim tile), A = P straight
//      from the QK accumulators, B = V.
// MFMA multiplies along the 8 contiguous elements a lane holds, so the cache
// keeps K token-major ([blk][h][16][D]: a lane's 8 dims are 16 contiguous
// bytes) and V dim-major ([blk][h][D][16]: a lane's 8 tokens are 16 contiguous
// bytes). The reduction index of each product is permuted identically on both
// operands (dims in QK, tokens in PV), which leaves the sums unchanged:
//   QK  k-step s, lane group g, element e  <->  dim s*32 + g*8 + e
//       (the four lanes of one token row read 64 contiguous bytes per step);
//   QK  tile 0 row r <-> token 8(r/4) + r%4, tile 1 row r <-> that + 4, so a
//       lane's two accumulators hold tokens 8g..8g+7 of the span: exactly the
//       A-operand row segment PV needs.
// The wavefronts of a workgroup merge (max, sum, O) through LDS. Nothing is
// cleared with a memset and no state survives a launch, so the kernels can be
// captured in a HIP graph.

#include <math.h>

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

// Issue every load of the span starting at `span` (< lim). Loads are
// unconditional from in-bounds addresses (indices clamped, invalid block ids
// read block 0) so they are all in flight together; V of tokens >= lim is
// zeroed afterwards, K of such tokens needs nothing (their scores become -inf).
__device__ __forceinline__ void load_span(const AttnArgs& a, const int32_t* table, int h, int span,
                                          int lim, int g, int j, Span& r) {
  const int tau0 = 8 * (j >> 2) + (j & 3);      // QK tile-0 row j -> token offset
  const int ta = span + tau0, tb = ta + 4;
  const int tv = span + 8 * g;                   // this lane's 8 V tokens
  const int last = lim - 1;
  const int ba = table[min(ta, last) >> 4];
  const int bb = table[min(tb, last) >> 4];
  const int bv = table[min(tv, last) >> 4];
  const int cba = (ba >= 0 && ba < a.num_blocks) ? ba : 0;
  const int cbb = (bb >= 0 && bb < a.num_blocks) ? bb : 0;
  const int cbv = (bv >= 0 && bv < a.num_blocks) ? bv : 0;
  const uint16_t* pa = a.ck + (((int64_t)cba * a.Hkv + h) * 16 + (ta & 15)) * kD + g * 8;
  const uint16_t* pb = a.ck + (((int64_t)cbb * a.Hkv + h) * 16 + (tb & 15)) * kD + g * 8;
  const uint16_t* pv = a.cv + ((int64_t)cbv * a.Hkv + h) * kD * 16 + (tv & 15) + j * 16;
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    r.ka[s] = pdk::ld16(pa + 32 * s);
    r.kb[s] = pdk::ld16(pb + 32 * s);
  }
#pragma unroll
  for (int n = 0; n < 8; ++n) r.vf[n] = pdk::ld16(pv + 16 * 16 * n);
}

// Fold one loaded span into the running (m, lsum, o) of query j = lane & 15.
__device__ __forceinline__ void attend_span(const AttnArgs& a, const int32_t* table, Span& r,
                                            const v8 qv[4], int span, int lim, int g, int j,
                                            float& m, float& lsum, f32x4 o[8]) {
  const int tv = span + 8 * g;
  const int bv = table[min(tv, lim - 1) >> 4];
  if (tv >= lim || bv < 0 || bv >= a.num_blocks) {
#pragma unroll
    for (int n = 0; n < 8; ++n) r.vf[n] = pdk::zero8();
  } else if (tv + 8 > lim) {
#pragma unroll
    for (int n = 0; n < 8; ++n) pdk::mask_tail(r.vf[n], tv, lim);
  }
  f32x4 s0 = {0.f, 0.f, 0.f, 0.f}, s1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    s0 = mfma(r.ka[s], qv[s], s0);
    s1 = mfma(r.kb[s], qv[s], s1);
  }
  // Lane (g, j): query j, tokens tv + e, e = 0..7.
  float sc[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    sc[i] = s0[i] * a.scale_log2;
    sc[4 + i] = s1[i] * a.scale_log2;
  }
#pragma unroll
  for (int e = 0; e < 8; ++e)
    if (tv + e >= lim) sc[e] = -INFINITY;
  float mx = sc[0];
#pragma unroll
  for (int e = 1; e < 8; ++e) mx = fmaxf(mx, sc[e]);
  mx = fmaxf(mx, __shfl_xor(mx, 16));
  mx = fmaxf(mx, __shfl_xor(mx, 32));
  const float m_new = fmaxf(m, mx);             // finite: token `span` is valid
  const float alpha = exp2f(m - m_new);
  float p[8], ps = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    p[e] = exp2f(sc[e] - m_new);
    ps += p[e];
  }
  ps += __shfl_xor(ps, 16);
  ps += __shfl_xor(ps, 32);
  lsum = lsum * alpha + ps;
  m = m_new;
  v8 pv;
  const uint32_t pmask = j < a.G ? 0xffffffffu : 0u;
#pragma unroll
  for (int w = 0; w < 4; ++w)
    pv.w[w] = (pdk::f32_to_bf16_rne(p[2 * w]) | (pdk::f32_to_bf16_rne(p[2 * w + 1]) << 16)) & pmask;
  float ar[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) ar[i] = __shfl(alpha, 4 * g + i);
#pragma unroll
  for (int n = 0; n < 8; ++n) {
#pragma unroll
    for (int i = 0; i < 4; ++i) o[n][i] *= ar[i];
    o[n] = mfma(pv, r.vf[n], o[n]);
  }
}

__global__ __launch_bounds__(512) void decode_attn_kernel(const AttnArgs a) {
  __shared__ float sm_m[kMaxWaves][kMaxG];
  __shared__ float sm_l[kMaxWaves][kMaxG];
  __shared__ float sm_o[kMaxWaves][4][kD];      // rows of the group, 4 at a time

  const int split = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int W = blockDim.x >> 6;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int g = lane >> 4, j = lane & 15;
  const int G = a.G;
  const int ctx = min(a.ctx[b], a.max_blocks * 16);
  const int s_begin = split * a.split_tokens;
  const int s_end = (split == a.nsplit - 1) ? ctx : min(ctx, s_begin + a.split_tokens);
  const int32_t* table = a.tables + (int64_t)b * a.max_blocks;

  const uint16_t* qp = a.q + ((int64_t)b * a.Hq + h * G + min(j, G - 1)) * kD + g * 8;
  v8 qv[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) qv[s] = pdk::ld16(qp + 32 * s);
  const uint32_t qmask = j < G ? 0xffffffffu : 0u;
#pragma unroll
  for (int s = 0; s < 4; ++s)
#pragma unroll
    for (int w = 0; w < 4; ++w) qv[s].w[w] &= qmask;

  float m = -INFINITY, lsum = 0.f;
  f32x4 o[8];
#pragma unroll
  for (int n = 0; n < 8; ++n) o[n] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int stride = W * kSpan;
  for (int sa = s_begin + wave * kSpan; sa < s_end; sa += 2 * stride) {
    const int sb = sa + stride;
    Span ra, rb;
    load_span(a, table, h, sa, s_end, g, j, ra);
    if (sb < s_end) load_span(a, table, h, sb, s_end, g, j, rb);
    attend_span(a, table, ra, qv, sa, s_end, g, j, m, lsum, o);
    if (sb < s_end) attend_span(a, table, rb, qv, sb, s_end, g, j, m, lsum, o);
  }

  // Merge the W wavefronts. Lane (g, j) holds O rows 4g..4g+3, dim 16n+j;
  // rows go through LDS four at a time (one lane group g per pass).
  if (g == 0 && j < G) {
    sm_m[wave][j] = m;
    sm_l[wave][j] = lsum;
  }
  const int64_t bq0 = (int64_t)b * a.Hq + h * G;
  for (int gg = 0; 4 * gg < G; ++gg) {
    __syncthreads();                             // sm_m/sm_l written; sm_o free
    if (g == gg) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int n = 0; n < 8; ++n) sm_o[wave][i][16 * n + j] = o[n][i];
    }
    __syncthreads();
    const int rows = min(4, G - 4 * gg);
    for (int idx = threadIdx.x; idx < rows * kD; idx += blockDim.x) {
      const int i = idx / kD, d = idx - i * kD;
      const int row = 4 * gg + i;
      float M = -INFINITY;
      for (int w = 0; w < W; ++w) M = fmaxf(M, sm_m[w][row]);
      float L = 0.f, O = 0.f;
      if (M != -INFINITY) {
        for (int w = 0; w < W; ++w) {
          const float mw = sm_m[w][row];
          if (mw != -INFINITY) {
            const float c = exp2f(mw - M);
            L += sm_l[w][row] * c;
            O += sm_o[w][i][d] * c;
          }
        }
      }
      const int64_t bq = bq0 + row;
      if (a.nsplit == 1) {
        a.out[bq * kD + d] = (uint16_t)pdk::f32_to_bf16_rne(L > 0.f ? O / L : 0.f);
      } else {
        a.ws_o[(bq * a.nsplit + split) * kD + d] = O;
        if (d == 0) {
          a.ws_ml[(bq * a.nsplit + split) * 2 + 0] = M;
          a.ws_ml[(bq * a.nsplit + split) * 2 + 1] = L;
        }
      }
    }
  }
}

// out = sum_s 2^(m_s-M) O_s / sum_s 2^(m_s-M) l_s, all partial loads independent.
__global__ __launch_bounds__(128) void merge_kernel(const float* ws_ml, const float* ws_o,
                                                    int nsplit, uint16_t* out) {
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
        const float c = exp2f(mv[s] - M);
        L += lv[s] * c;
        O += ov[s] * c;
      }
    }
  }
  out[bq * kD + d] = (uint16_t)pdk::f32_to_bf16_rne(L > 0.f ? O / L : 0.f);
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
  for (int d = threadIdx.x; d < D; d += blockDim.x) {
    const int64_t src = ((int64_t)b * Hkv + h) * D + d;
    ck[(((int64_t)blk * Hkv + h) * 16 + slot) * D + d] = k_new[src];
    cv[(((int64_t)blk * Hkv + h) * D + d) * 16 + slot] = v_new[src];
  }
}

int64_t round_up(int64_t x, int64_t m) { return (x + m - 1) / m * m; }

// Launch plan: one split once B*Hkv workgroups reach 128 (each up to 8
// wavefronts = 512 tokens in flight); below that, enough splits for ~256
// workgroups, each at least 64 tokens.
struct Plan {
  int nsplit, split_tokens, waves;
};

Plan plan_for(int B, int Hkv, int max_ctx) {
  const int64_t pairs = (int64_t)B * Hkv;
  int nsplit = 1;
  if (pairs < 128) nsplit = (int)((256 + pairs - 1) / pairs);
  const int max_splits = max(1, (max_ctx + 63) / 64);
  nsplit = min(min(nsplit, max_splits), kMaxSplits);
  const int split_tokens = (int)round_up((max_ctx + nsplit - 1) / nsplit, kSpan);
  nsplit = (max_ctx + split_tokens - 1) / split_tokens;
  const int waves = max(1, min(kMaxWaves, (split_tokens + 2 * kSpan - 1) / (2 * kSpan)));
  return {nsplit, split_tokens, waves};
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
  return ws_bytes(B, n_q_heads, min(kMaxSplits, max(1, (max_ctx + 63) / 64)));
}

extern "C" int pdk_decode_attn(const uint16_t* q, const uint16_t* cache_k, const uint16_t* cache_v,
                               int num_blocks, const int32_t* block_tables, int max_blocks,
                               const int32_t* ctx_lens, int max_ctx, int B, int n_q_heads,
                               int n_kv_heads, int head_dim, float scale, void* workspace,
                               size_t workspace_bytes, uint16_t* out, uintptr_t stream) {
  pdk::clear_error();
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
  PDK_REQUIRE(q && cache_k && cache_v && out && block_tables && ctx_lens,
              "null pointer argument");
  PDK_REQUIRE(pdk::aligned16(q) && pdk::aligned16(cache_k) && pdk::aligned16(cache_v),
              "q/cache_k/cache_v must be 16-byte aligned");
  PDK_REQUIRE(num_blocks >= 1 && max_blocks >= 1, "num_blocks and max_blocks must be >= 1");
  PDK_REQUIRE(max_ctx >= 1 && max_ctx <= max_blocks * 16,
              "max_ctx=%d outside [1, max_blocks*16=%d]", max_ctx, max_blocks * 16);
  const Plan p = plan_for(B, n_kv_heads, max_ctx);
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
  if (p.nsplit > 1) {
    const size_t need = ws_bytes(B, n_q_heads, p.nsplit);
    PDK_REQUIRE(workspace && workspace_bytes >= need && pdk::aligned16(workspace),
                "workspace of %zu bytes needed (got %zu)", need, workspace_bytes);
    char* base = static_cast<char*>(workspace);
    const int64_t bq = (int64_t)B * n_q_heads;
    a.ws_ml = reinterpret_cast<float*>(base);
    a.ws_o = reinterpret_cast<float*>(base + round_up(bq * p.nsplit * 2 * 4, 256));
  }
  hipStream_t st = pdk::as_stream(stream);
  hipLaunchKernelGGL(decode_attn_kernel, dim3(p.nsplit, n_kv_heads, B), dim3(64 * p.waves), 0, st,
                     a);
  int rc = pdk::check_launch("decode_attn_kernel");
  if (rc || p.nsplit == 1) return rc;
  hipLaunchKernelGGL(merge_kernel, dim3(B * n_q_heads), dim3(kD), 0, st, a.ws_ml, a.ws_o,
                     p.nsplit, out);
  return pdk::check_launch("merge_kernel");
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
  PDK_REQUIRE(head_dim >= 1 && head_dim <= 4096, "head_dim out of range");
  PDK_REQUIRE(num_blocks >= 1 && max_blocks >= 1, "num_blocks and max_blocks must be >= 1");
  hipLaunchKernelGGL(cache_append_kernel, dim3(B, n_kv_heads), dim3(128), 0,
                     pdk::as_stream(stream), k_new, v_new, cache_k, cache_v, num_blocks,
                     block_tables, max_blocks, ctx_lens, n_kv_heads, head_dim);
  return pdk::check_launch("cache_append_kernel");
}
