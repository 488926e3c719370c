// GQA decode attention over the paged KV cache, gfx950.
//
// One workgroup (4 wavefronts) owns one (stream b, KV head h, token split).
// A wavefront walks 32-token spans of its split (span s, s+4, ...); per span:
//   QK^T  two v_mfma_f32_16x16x32_bf16 tiles x 4 k-steps: A = 16 K rows
//         (tokens), B = the G query heads of the group padded to 16 columns;
//   softmax  online, fp32, in the exp2 domain, across the 32 tokens with two
//         lane shuffles;
//   PV    8 v_mfma_f32_16x16x32_bf16 (one per 16-dim tile): A = P (queries x
//         32 tokens, straight from the QK accumulators), B = V.
// MFMA multiplies along the 8 contiguous elements a lane holds, so the cache
// keeps K token-major ([blk][h][16][D]: a lane's 8 dims are 16 contiguous
// bytes) and V dim-major ([blk][h][D][16]: a lane's 8 tokens are 16 contiguous
// bytes). The reduction index of each product is permuted consistently on both
// operands (dims in QK, tokens in PV), which leaves the sums unchanged:
//   QK  k-step s, lane group g, element e  <->  dim g*32 + s*8 + e
//   QK  tile 0 row r <-> token 8(r/4) + r%4, tile 1 row r <-> that + 4, so a
//       lane's two accumulators hold tokens 8g..8g+7 of the span, which is
//       exactly the A-operand row segment PV needs.
// The four wavefronts merge (max, sum, O) through LDS; with more than one
// split the partials go to the workspace and a small kernel merges them.

#include <math.h>

#include "pdk_common.h"

namespace {

using pdk::v8;

typedef __bf16 bf16x8_t __attribute__((__vector_size__(16)));
typedef float f32x4 __attribute__((__vector_size__(16)));

constexpr int kD = 128;          // head_dim handled by the kernel
constexpr int kWaves = 4;
constexpr int kSpan = 32;        // tokens per wavefront step
constexpr int kSplitTokens = kWaves * kSpan;   // tokens per workgroup split
constexpr int kMaxG = 16;

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
  float* ws_o;                   // [B*Hq][nsplit][D]
  float* ws_ml;                  // [B*Hq][nsplit][2]
  int num_blocks, max_blocks, Hq, Hkv, G, nsplit;
  float scale_log2;              // scale * log2(e)
};

__global__ __launch_bounds__(256) void decode_attn_kernel(const AttnArgs a) {
  __shared__ float sm_m[kWaves][kMaxG];
  __shared__ float sm_l[kWaves][kMaxG];
  __shared__ float sm_o[kWaves][kMaxG][kD];

  const int split = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int g = lane >> 4, j = lane & 15;
  const int G = a.G, Hkv = a.Hkv;
  int ctx = a.ctx[b];
  ctx = min(ctx, a.max_blocks * 16);
  const int s_begin = split * kSplitTokens;
  const int s_end = (split == a.nsplit - 1) ? ctx : min(ctx, s_begin + kSplitTokens);

  v8 qv[4];
  if (j < G) {
    const uint16_t* qp = a.q + ((int64_t)b * a.Hq + h * G + j) * kD + g * 32;
#pragma unroll
    for (int s = 0; s < 4; ++s) qv[s] = pdk::ld16(qp + 8 * s);
  } else {
#pragma unroll
    for (int s = 0; s < 4; ++s) qv[s] = pdk::zero8();
  }

  float m = -INFINITY, lsum = 0.f;
  f32x4 o[8];
#pragma unroll
  for (int n = 0; n < 8; ++n) o[n] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int32_t* table = a.tables + (int64_t)b * a.max_blocks;
  const int tau0 = 8 * (j >> 2) + (j & 3);      // QK tile-0 row j -> token offset

  for (int span = s_begin + wave * kSpan; span < s_end; span += kSplitTokens) {
    // K rows for tiles 0 and 1: 64 contiguous bytes per lane each.
    v8 ka[4], kb[4];
    {
      const int ta = span + tau0, tb = ta + 4;
      const int ba = ta < ctx ? table[ta >> 4] : -1;
      const int bb = tb < ctx ? table[tb >> 4] : -1;
      if (ba >= 0 && ba < a.num_blocks) {
        const uint16_t* p = a.ck + (((int64_t)ba * Hkv + h) * 16 + (ta & 15)) * kD + g * 32;
#pragma unroll
        for (int s = 0; s < 4; ++s) ka[s] = pdk::ld16(p + 8 * s);
      } else {
#pragma unroll
        for (int s = 0; s < 4; ++s) ka[s] = pdk::zero8();
      }
      if (bb >= 0 && bb < a.num_blocks) {
        const uint16_t* p = a.ck + (((int64_t)bb * Hkv + h) * 16 + (tb & 15)) * kD + g * 32;
#pragma unroll
        for (int s = 0; s < 4; ++s) kb[s] = pdk::ld16(p + 8 * s);
      } else {
#pragma unroll
        for (int s = 0; s < 4; ++s) kb[s] = pdk::zero8();
      }
    }
    // V: tokens tv..tv+7 (one block, 8 slots) of dims 16n + j.
    const int tv = span + 8 * g;
    v8 vf[8];
    {
      const int bv = tv < ctx ? table[tv >> 4] : -1;
      if (bv >= 0 && bv < a.num_blocks) {
        const uint16_t* p = a.cv + ((int64_t)bv * Hkv + h) * kD * 16 + (tv & 15);
#pragma unroll
        for (int n = 0; n < 8; ++n) {
          vf[n] = pdk::ld16(p + (16 * n + j) * 16);
          if (tv + 8 > ctx) pdk::mask_tail(vf[n], tv, ctx);
        }
      } else {
#pragma unroll
        for (int n = 0; n < 8; ++n) vf[n] = pdk::zero8();
      }
    }

    f32x4 s0 = {0.f, 0.f, 0.f, 0.f}, s1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      s0 = mfma(ka[s], qv[s], s0);
      s1 = mfma(kb[s], qv[s], s1);
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
      if (tv + e >= ctx) sc[e] = -INFINITY;
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
    if (j < G) {
#pragma unroll
      for (int w = 0; w < 4; ++w)
        pv.w[w] = pdk::f32_to_bf16_rne(p[2 * w]) | (pdk::f32_to_bf16_rne(p[2 * w + 1]) << 16);
    } else {
      pv = pdk::zero8();
    }
    float ar[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) ar[i] = __shfl(alpha, 4 * g + i);
#pragma unroll
    for (int n = 0; n < 8; ++n) {
#pragma unroll
      for (int i = 0; i < 4; ++i) o[n][i] *= ar[i];
      o[n] = mfma(pv, vf[n], o[n]);
    }
  }

  // Merge the four wavefronts. Lane (g, j) holds O rows 4g..4g+3, dim 16n+j.
  if (g == 0 && j < G) {
    sm_m[wave][j] = m;
    sm_l[wave][j] = lsum;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row = 4 * g + i;
    if (row < G) {
#pragma unroll
      for (int n = 0; n < 8; ++n) sm_o[wave][row][16 * n + j] = o[n][i];
    }
  }
  __syncthreads();

  for (int idx = threadIdx.x; idx < G * kD; idx += blockDim.x) {
    const int row = idx / kD, d = idx - row * kD;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) M = fmaxf(M, sm_m[w][row]);
    float L = 0.f, O = 0.f;
    if (M != -INFINITY) {
#pragma unroll
      for (int w = 0; w < kWaves; ++w) {
        const float mw = sm_m[w][row];
        if (mw != -INFINITY) {
          const float c = exp2f(mw - M);
          L += sm_l[w][row] * c;
          O += sm_o[w][row][d] * c;
        }
      }
    }
    const int64_t bq = (int64_t)b * a.Hq + h * G + row;
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

// Combine split partials: out = sum_s 2^(m_s-M) O_s / sum_s 2^(m_s-M) l_s.
__global__ __launch_bounds__(128) void merge_kernel(const float* ws_o, const float* ws_ml,
                                                    int nsplit, uint16_t* out) {
  const int64_t bq = blockIdx.x;
  const int d = threadIdx.x;
  float M = -INFINITY;
  for (int s = 0; s < nsplit; ++s) M = fmaxf(M, ws_ml[(bq * nsplit + s) * 2]);
  float L = 0.f, O = 0.f;
  if (M != -INFINITY) {
    for (int s = 0; s < nsplit; ++s) {
      const float ms = ws_ml[(bq * nsplit + s) * 2];
      if (ms != -INFINITY) {
        const float c = exp2f(ms - M);
        L += ws_ml[(bq * nsplit + s) * 2 + 1] * c;
        O += ws_o[(bq * nsplit + s) * kD + d] * c;
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

int nsplit_for(int max_ctx) { return max_ctx <= 0 ? 1 : (max_ctx + kSplitTokens - 1) / kSplitTokens; }

}  // namespace

extern "C" size_t pdk_decode_attn_workspace_bytes(int B, int n_q_heads, int max_ctx, int head_dim) {
  if (B <= 0 || n_q_heads <= 0 || head_dim <= 0) return 0;
  const int ns = nsplit_for(max_ctx);
  if (ns == 1) return 0;
  return (size_t)B * n_q_heads * ns * (head_dim + 2) * sizeof(float);
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
  const int nsplit = nsplit_for(max_ctx);
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
  a.nsplit = nsplit;
  a.scale_log2 = scale * 1.4426950408889634f;
  if (nsplit > 1) {
    const size_t need = pdk_decode_attn_workspace_bytes(B, n_q_heads, max_ctx, head_dim);
    PDK_REQUIRE(workspace && workspace_bytes >= need && pdk::aligned16(workspace),
                "workspace of %zu bytes needed (got %zu)", need, workspace_bytes);
    a.ws_o = static_cast<float*>(workspace);
    a.ws_ml = a.ws_o + (size_t)B * n_q_heads * nsplit * kD;
  }
  hipStream_t st = pdk::as_stream(stream);
  hipLaunchKernelGGL(decode_attn_kernel, dim3(nsplit, n_kv_heads, B), dim3(256), 0, st, a);
  int rc = pdk::check_launch("decode_attn_kernel");
  if (rc || nsplit == 1) return rc;
  hipLaunchKernelGGL(merge_kernel, dim3(B * n_q_heads), dim3(kD), 0, st, a.ws_o, a.ws_ml, nsplit,
                     out);
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
