// The non-GEMM kernels of the Llama decode step for gfx950: RMSNorm with the
// residual add fused in, RoPE fused with the new token's paged-cache write,
// and SwiGLU. The projections and the lm_head are plain GEMMs (the caller's
// BLAS); attention is decode_attn_kernel.
//
// Each is bound by the bytes it moves (a few KiB per stream per layer); they
// exist to keep the step to one launch per operation with fp32 arithmetic
// inside and bf16 at every tensor boundary, as the reference's step keeps its
// activations in bf16 (kernels/decode_batch.py:73-91).

#include <math.h>

#include "pdk_common.h"

namespace {

using pdk::v8;

__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) x += __shfl_xor(x, o);
  return x;
}

// One workgroup per row of H (H % 8 == 0, H <= 8192), 256 threads, 8 bf16 per
// 16-byte access, the row held in registers between the two passes. Before
// the norm, kAdd == 1: x <- bf16(x + add) (the residual add, zipadd_dsl of
// kernels/dsl_batch.py), written back; kAdd == 2: x <- bf16(x + sum over
// `splits` fp32 partial rows) (the residual add of a split-K projection,
// summed in a fixed order), written back. Then
// out = bf16(x * rsqrt(mean(x^2) + eps) * w) (rms_dsl: x * (sum x^2 + eps*H)^-1/2
// * w*sqrt(H), the same value).
constexpr int kNormThreads = 256, kNormChunks = 4;     // 8 elements per chunk

template <int kAdd>
__global__ __launch_bounds__(kNormThreads) void rmsnorm_kernel(uint16_t* x, const void* add,
                                                               int splits, int B,
                                                               const uint16_t* w, float eps,
                                                               int H, uint16_t* out) {
  __shared__ float part[kNormThreads / 64];
  const int64_t row = (int64_t)blockIdx.x * H;
  const int n8 = H >> 3;
  v8 keep[kNormChunks], gain[kNormChunks];
  float ss = 0.f;
  // The weights are loaded with the row, before the reduction, so the second
  // pass waits on no memory.
#pragma unroll
  for (int j = 0; j < kNormChunks; ++j) {
    const int c = threadIdx.x + j * kNormThreads;
    gain[j] = c < n8 ? pdk::ld16(w + 8 * c) : pdk::zero8();
  }
#pragma unroll
  for (int j = 0; j < kNormChunks; ++j) {
    const int c = threadIdx.x + j * kNormThreads;
    keep[j] = pdk::zero8();
    if (c < n8) {
      v8 a = pdk::ld16(x + row + 8 * c);
      if (kAdd == 1) {
        const v8 b = pdk::ld16(static_cast<const uint16_t*>(add) + row + 8 * c);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const float lo = pdk::bf16_to_f32(a.w[k] & 0xffffu) + pdk::bf16_to_f32(b.w[k] & 0xffffu);
          const float hi = pdk::bf16_to_f32(a.w[k] >> 16) + pdk::bf16_to_f32(b.w[k] >> 16);
          a.w[k] = pdk::f32_to_bf16_rne(lo) | (pdk::f32_to_bf16_rne(hi) << 16);
        }
      } else if (kAdd == 2) {
        float acc[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) acc[k] = 0.f;
        const float* p = static_cast<const float*>(add) + row + 8 * c;
        for (int s = 0; s < splits; ++s) {
          const float4 u = *reinterpret_cast<const float4*>(p + (int64_t)s * B * H);
          const float4 v = *reinterpret_cast<const float4*>(p + (int64_t)s * B * H + 4);
          acc[0] += u.x; acc[1] += u.y; acc[2] += u.z; acc[3] += u.w;
          acc[4] += v.x; acc[5] += v.y; acc[6] += v.z; acc[7] += v.w;
        }
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const float lo = pdk::bf16_to_f32(a.w[k] & 0xffffu) + acc[2 * k];
          const float hi = pdk::bf16_to_f32(a.w[k] >> 16) + acc[2 * k + 1];
          a.w[k] = pdk::f32_to_bf16_rne(lo) | (pdk::f32_to_bf16_rne(hi) << 16);
        }
      }
      if (kAdd) pdk::st16(x + row + 8 * c, a);
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const float lo = pdk::bf16_to_f32(a.w[k] & 0xffffu), hi = pdk::bf16_to_f32(a.w[k] >> 16);
        ss += lo * lo + hi * hi;
      }
      keep[j] = a;
    }
  }
  ss = wave_sum(ss);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = ss;
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int i = 0; i < kNormThreads / 64; ++i) tot += part[i];
  const float r = rsqrtf(tot / (float)H + eps);
#pragma unroll
  for (int j = 0; j < kNormChunks; ++j) {
    const int c = threadIdx.x + j * kNormThreads;
    if (c < n8) {
      const v8 a = keep[j];
      const v8 g = gain[j];
      v8 o;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const float lo = pdk::bf16_to_f32(a.w[k] & 0xffffu) * r * pdk::bf16_to_f32(g.w[k] & 0xffffu);
        const float hi = pdk::bf16_to_f32(a.w[k] >> 16) * r * pdk::bf16_to_f32(g.w[k] >> 16);
        o.w[k] = pdk::f32_to_bf16_rne(lo) | (pdk::f32_to_bf16_rne(hi) << 16);
      }
      pdk::st16(out + row + 8 * c, o);
    }
  }
}

__device__ __forceinline__ float bf(uint16_t h) { return pdk::bf16_to_f32(h); }
__device__ __forceinline__ uint16_t to_bf(float f) { return (uint16_t)pdk::f32_to_bf16_rne(f); }

// Grid (NH + 2*NKV, B), HD/2 threads. Row b of qkv holds q (NH heads), k (NKV)
// and v (NKV), HD each. Rotate-half RoPE at position pos = ctx[b]-1 (HF's
// rotate_half, engines/model.py:55-64; angle pos*inv_freq[i] in fp32 as the
// reference's tables, engines/decode_batch.py:244-255): q heads go to q_out
// [B][NH][HD]; the rotated k and the v of the new token go to slot pos of the
// paged cache (the one-hot injection of kernels/decode_batch.py:81-82 as a
// store), K in the tiled block order of pdk::k_unit.
//
// With kSplits > 0 the row comes as kSplits fp32 partial sums of the q|k|v
// projection (split-K, [split][B][ld]): they are added in split order and
// rounded to bf16 once, the value the unsplit projection would have written.
//
// With ssq (kSplits > 0 only) the projection's input was the un-normalised
// residual and its weights carry the norm's gain: the summed row is scaled by
// the row's r (pdk::row_rms over ssq [B][n_ssq], K = 16 n_ssq) before the one
// rounding, the value pdk_decode_attn_rope_rms uses.
template <int kSplits>
__global__ void rope_append_kernel(const void* src_, int64_t ld, int64_t split_stride,
                                   uint16_t* q_out, const float* inv_freq, const int32_t* ctx,
                                   const int32_t* tables, int max_blocks, uint16_t* ck,
                                   uint16_t* cv, int num_blocks, int NH, int NKV, int HD,
                                   const float* ssq, int n_ssq, float eps) {
  const int head = blockIdx.x, b = blockIdx.y, i = threadIdx.x, half = HD >> 1;
  const int pos = ctx[b] - 1;
  float rb = 1.f;
  if (kSplits > 0 && ssq) {
    const pdk::RowRms rr = pdk::row_rms_load(ssq, b, n_ssq, i);
    rb = pdk::row_rms_finish(rr, ssq, b, n_ssq, 16 * n_ssq, eps, i);
  }
  // Element c of row b, already rounded to bf16.
  auto val = [&](int64_t c) -> uint16_t {
    if constexpr (kSplits == 0) {
      return static_cast<const uint16_t*>(src_)[(int64_t)b * ld + c];
    } else {
      const float* p = static_cast<const float*>(src_) + (int64_t)b * ld + c;
      float sum = p[0];
#pragma unroll
      for (int s = 1; s < kSplits; ++s) sum += p[s * split_stride];
      return to_bf(ssq ? sum * rb : sum);
    }
  };
  int blk = -1;
  if (pos >= 0 && pos < max_blocks * 16) {
    const int id = tables[(int64_t)b * max_blocks + (pos >> 4)];
    if (id >= 0 && id < num_blocks) blk = id;
  }
  const int slot = pos & 15;
  if (head < NH + NKV) {
    const int64_t c0 = (int64_t)head * HD;
    const float a = bf(val(c0 + i)), c = bf(val(c0 + i + half));
    float s, co;
    sincosf((float)max(pos, 0) * inv_freq[i], &s, &co);
    float y0, y1;
    pdk::rope_pair(a, c, co, s, y0, y1);
    const uint16_t o0 = to_bf(y0), o1 = to_bf(y1);
    if (head < NH) {
      uint16_t* q = q_out + ((int64_t)b * NH + head) * HD;
      q[i] = o0;
      q[i + half] = o1;
    } else if (blk >= 0) {
      uint16_t* kb = ck + ((int64_t)blk * NKV + (head - NH)) * 16 * HD;
      kb[pdk::k_unit(slot, i & ~7, HD) * 8 + (i & 7)] = o0;
      kb[pdk::k_unit(slot, (i + half) & ~7, HD) * 8 + ((i + half) & 7)] = o1;
    }
  } else if (blk >= 0) {
    const int vh = head - NH - NKV;
    const int64_t c0 = (int64_t)(NH + NKV + vh) * HD;
    uint16_t* vb = cv + ((int64_t)blk * NKV + vh) * HD * 16;
    vb[(int64_t)i * 16 + slot] = val(c0 + i);
    vb[(int64_t)(i + half) * 16 + slot] = val(c0 + i + half);
  }
}

// out[b][m] = bf16(silu(g) * u), g = gu[b][m], u = gu[b][M+m], fp32 inside
// (swiglu_dsl of kernels/dsl_batch.py: g * sigmoid(g) * u). 8 per thread.
__global__ __launch_bounds__(256) void swiglu_kernel(const uint16_t* gu, int M, int64_t n8,
                                                     uint16_t* out) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= n8) return;
  const int64_t per_row = M >> 3;
  const int64_t b = t / per_row, c = t - b * per_row;
  const v8 g = pdk::ld16(gu + b * 2 * M + 8 * c);
  const v8 u = pdk::ld16(gu + b * 2 * M + M + 8 * c);
  v8 o;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const float g0 = pdk::bf16_to_f32(g.w[k] & 0xffffu), g1 = pdk::bf16_to_f32(g.w[k] >> 16);
    const float u0 = pdk::bf16_to_f32(u.w[k] & 0xffffu), u1 = pdk::bf16_to_f32(u.w[k] >> 16);
    const float r0 = g0 / (1.f + expf(-g0)) * u0, r1 = g1 / (1.f + expf(-g1)) * u1;
    o.w[k] = pdk::f32_to_bf16_rne(r0) | (pdk::f32_to_bf16_rne(r1) << 16);
  }
  pdk::st16(out + b * M + 8 * c, o);
}

// The sum of squares of 16 bf16 values (lo: elements 0..7, hi: 8..15), in
// index order.
__device__ __forceinline__ float tile_ssq(const v8& lo, const v8& hi) {
  float s = 0.f;
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const v8& v = k < 4 ? lo : hi;
    const float a = pdk::bf16_to_f32(v.w[k & 3] & 0xffffu), c = pdk::bf16_to_f32(v.w[k & 3] >> 16);
    s += a * a;
    s += c * c;
  }
  return s;
}

// ssq[b][t] = the sum over x[b][16t .. 16t+15] (bf16) of x^2, in index order:
// the per-tile sums of squares a folded RMSNorm's consumer scales rows by.
__global__ __launch_bounds__(256) void row_ssq_kernel(const uint16_t* x, int B, int H, float* ssq) {
  const int b = blockIdx.x;
  for (int t = threadIdx.x; t < H / 16; t += 256) {
    const uint16_t* p = x + (int64_t)b * H + 16 * t;
    ssq[(int64_t)b * (H / 16) + t] = tile_ssq(pdk::ld16(p), pdk::ld16(p + 8));
  }
}

// x[b] = table[tokens[b]] and its per-tile sums of squares (row_ssq_kernel's
// values, bit for bit): the step's embedding lookup and the first layer's
// folded-norm input in one launch. A token outside [0, vocab) gives a zero row.
// kAct: x in the tiled activation layout (pdk::act_at; H % 128 == 0).
template <typename Tok, bool kAct = false>
__global__ __launch_bounds__(256) void embed_ssq_kernel(const uint16_t* table, int64_t vocab,
                                                        const Tok* tokens, int H, uint16_t* x,
                                                        float* ssq) {
  const int b = blockIdx.x;
  const int64_t tok = (int64_t)tokens[b];
  const bool ok = tok >= 0 && tok < vocab;
  const uint16_t* row = table + (ok ? tok : 0) * (int64_t)H;
  for (int t = threadIdx.x; t < H / 16; t += 256) {
    v8 lo = pdk::ld16(row + 16 * t), hi = pdk::ld16(row + 16 * t + 8);
    if (!ok) lo = hi = pdk::zero8();
    pdk::st16(x + (kAct ? pdk::act_at(b, 16 * t, H) : (int64_t)b * H + 16 * t), lo);
    pdk::st16(x + (kAct ? pdk::act_at(b, 16 * t + 8, H) : (int64_t)b * H + 16 * t + 8), hi);
    ssq[(int64_t)b * (H / 16) + t] = tile_ssq(lo, hi);
  }
}

}  // namespace

extern "C" int pdk_row_ssq(const uint16_t* x, int B, int H, float* ssq, uintptr_t stream) {
  pdk::clear_error();
  PDK_REQUIRE(x && ssq, "null pointer argument");
  PDK_REQUIRE(B >= 1 && B <= 65535, "B must be in [1, 65535] (got %d)", B);
  PDK_REQUIRE(H >= 16 && H % 16 == 0, "H must be a positive multiple of 16 (got %d)", H);
  PDK_REQUIRE(pdk::aligned16(x), "x must be 16-byte aligned");
  hipLaunchKernelGGL(row_ssq_kernel, dim3(B), dim3(256), 0, pdk::as_stream(stream), x, B, H, ssq);
  return pdk::check_launch("row_ssq_kernel");
}

namespace {
template <bool kAct>
int embed_ssq(const uint16_t* table, int64_t vocab, const void* tokens, int tok_bytes, int B,
              int H, uint16_t* x, float* ssq, uintptr_t stream) {
  pdk::clear_error();
  PDK_REQUIRE(!kAct || H % 128 == 0, "tiled activations need H %% 128 == 0 (got %d)", H);
  PDK_REQUIRE(table && tokens && x && ssq, "null pointer argument");
  PDK_REQUIRE(vocab >= 1, "vocab must be >= 1");
  PDK_REQUIRE(tok_bytes == 4 || tok_bytes == 8, "tok_bytes must be 4 (int32) or 8 (int64)");
  PDK_REQUIRE(B >= 1 && B <= 65535, "B must be in [1, 65535] (got %d)", B);
  PDK_REQUIRE(H >= 16 && H % 16 == 0, "H must be a positive multiple of 16 (got %d)", H);
  PDK_REQUIRE(pdk::aligned16(table) && pdk::aligned16(x), "table and x must be 16-byte aligned");
  PDK_REQUIRE(reinterpret_cast<uintptr_t>(tokens) % tok_bytes == 0,
              "tokens must be aligned to their %d-byte size", tok_bytes);
  hipStream_t st = pdk::as_stream(stream);
  if (tok_bytes == 4)
    hipLaunchKernelGGL((embed_ssq_kernel<int32_t, kAct>), dim3(B), dim3(256), 0, st, table, vocab,
                       static_cast<const int32_t*>(tokens), H, x, ssq);
  else
    hipLaunchKernelGGL((embed_ssq_kernel<int64_t, kAct>), dim3(B), dim3(256), 0, st, table, vocab,
                       static_cast<const int64_t*>(tokens), H, x, ssq);
  return pdk::check_launch("embed_ssq_kernel");
}
}  // namespace

extern "C" int pdk_embed_ssq(const uint16_t* table, int64_t vocab, const void* tokens,
                             int tok_bytes, int B, int H, uint16_t* x, float* ssq,
                             uintptr_t stream) {
  return embed_ssq<false>(table, vocab, tokens, tok_bytes, B, H, x, ssq, stream);
}

extern "C" int pdk_embed_ssq_xt(const uint16_t* table, int64_t vocab, const void* tokens,
                                int tok_bytes, int B, int H, uint16_t* x, float* ssq,
                                uintptr_t stream) {
  return embed_ssq<true>(table, vocab, tokens, tok_bytes, B, H, x, ssq, stream);
}

static int check_norm(const void* x, const void* weight, const void* out, int B, int H) {
  PDK_REQUIRE(x && weight && out, "null pointer argument");
  PDK_REQUIRE(B >= 1 && B <= 65535, "B must be in [1, 65535] (got %d)", B);
  PDK_REQUIRE(H >= 8 && H % 8 == 0 && H <= kNormThreads * kNormChunks * 8,
              "H must be a multiple of 8 in [8, %d] (got %d)", kNormThreads * kNormChunks * 8, H);
  PDK_REQUIRE(pdk::aligned16(x) && pdk::aligned16(weight) && pdk::aligned16(out),
              "tensors must be 16-byte aligned");
  return PDK_OK;
}

extern "C" int pdk_rmsnorm(uint16_t* x, const uint16_t* add, const uint16_t* weight, int B,
                           int H, float eps, uint16_t* out, uintptr_t stream) {
  pdk::clear_error();
  if (int rc = check_norm(x, weight, out, B, H)) return rc;
  PDK_REQUIRE(!add || pdk::aligned16(add), "tensors must be 16-byte aligned");
  PDK_REQUIRE(eps >= 0.f, "eps must be >= 0");
  hipStream_t st = pdk::as_stream(stream);
  if (add)
    hipLaunchKernelGGL(rmsnorm_kernel<1>, dim3(B), dim3(kNormThreads), 0, st, x, add, 0, B,
                       weight, eps, H, out);
  else
    hipLaunchKernelGGL(rmsnorm_kernel<0>, dim3(B), dim3(kNormThreads), 0, st, x, nullptr, 0, B,
                       weight, eps, H, out);
  return pdk::check_launch("rmsnorm_kernel");
}

extern "C" int pdk_rmsnorm_partials(uint16_t* x, const float* partials, int splits,
                                    const uint16_t* weight, int B, int H, float eps,
                                    uint16_t* out, uintptr_t stream) {
  pdk::clear_error();
  if (int rc = check_norm(x, weight, out, B, H)) return rc;
  PDK_REQUIRE(partials && pdk::aligned16(partials), "partials must be 16-byte aligned");
  PDK_REQUIRE(splits >= 1 && splits <= 64, "splits must be in [1, 64] (got %d)", splits);
  PDK_REQUIRE(eps >= 0.f, "eps must be >= 0");
  hipLaunchKernelGGL(rmsnorm_kernel<2>, dim3(B), dim3(kNormThreads), 0, pdk::as_stream(stream),
                     x, partials, splits, B, weight, eps, H, out);
  return pdk::check_launch("rmsnorm_kernel");
}

static int check_rope(const void* src, const uint16_t* q_out, const float* inv_freq,
                      const int32_t* ctx_lens, const int32_t* block_tables, int max_blocks,
                      const uint16_t* cache_k, const uint16_t* cache_v, int num_blocks, int B,
                      int n_q_heads, int n_kv_heads, int head_dim, int64_t ld) {
  PDK_REQUIRE(src && q_out && inv_freq && ctx_lens && block_tables && cache_k && cache_v,
              "null pointer argument");
  PDK_REQUIRE(B >= 1 && B <= 65535, "B must be in [1, 65535] (got %d)", B);
  PDK_REQUIRE(n_q_heads >= 1 && n_kv_heads >= 1 && n_q_heads + 2 * n_kv_heads <= 65535,
              "head counts out of range");
  PDK_REQUIRE(head_dim >= 32 && head_dim % 32 == 0 && head_dim <= 2048,
              "head_dim must be a multiple of 32 in [32, 2048] (got %d)", head_dim);
  PDK_REQUIRE(ld >= (int64_t)(n_q_heads + 2 * n_kv_heads) * head_dim,
              "row stride %lld shorter than a (q, k, v) row", (long long)ld);
  PDK_REQUIRE(num_blocks >= 1 && max_blocks >= 1, "num_blocks and max_blocks must be >= 1");
  return PDK_OK;
}

extern "C" int pdk_rope_cache_append(const uint16_t* qkv, int64_t qkv_ld, uint16_t* q_out,
                                     const float* inv_freq, const int32_t* ctx_lens,
                                     const int32_t* block_tables, int max_blocks,
                                     uint16_t* cache_k, uint16_t* cache_v, int num_blocks, int B,
                                     int n_q_heads, int n_kv_heads, int head_dim,
                                     uintptr_t stream) {
  pdk::clear_error();
  if (int rc = check_rope(qkv, q_out, inv_freq, ctx_lens, block_tables, max_blocks, cache_k,
                          cache_v, num_blocks, B, n_q_heads, n_kv_heads, head_dim, qkv_ld))
    return rc;
  hipLaunchKernelGGL(rope_append_kernel<0>, dim3(n_q_heads + 2 * n_kv_heads, B),
                     dim3(head_dim / 2), 0, pdk::as_stream(stream), qkv, qkv_ld, (int64_t)0,
                     q_out, inv_freq, ctx_lens, block_tables, max_blocks, cache_k, cache_v,
                     num_blocks, n_q_heads, n_kv_heads, head_dim, nullptr, 0, 0.f);
  return pdk::check_launch("rope_append_kernel");
}

static int rope_partials(const float* partials, int splits, int N, uint16_t* q_out,
                         const float* inv_freq, const int32_t* ctx_lens,
                         const int32_t* block_tables, int max_blocks, uint16_t* cache_k,
                         uint16_t* cache_v, int num_blocks, int B, int n_q_heads, int n_kv_heads,
                         int head_dim, const float* ssq, int n_ssq, float eps,
                         uintptr_t stream) {
  if (int rc = check_rope(partials, q_out, inv_freq, ctx_lens, block_tables, max_blocks, cache_k,
                          cache_v, num_blocks, B, n_q_heads, n_kv_heads, head_dim, N))
    return rc;
  if (ssq) {
    PDK_REQUIRE(n_ssq >= 1, "n_ssq must be >= 1 (got %d)", n_ssq);
    PDK_REQUIRE(eps > 0.f, "eps must be positive");
    PDK_REQUIRE(head_dim >= 64, "the row scale needs head_dim >= 64 (got %d)", head_dim);
  }
  const dim3 grid(n_q_heads + 2 * n_kv_heads, B), block(head_dim / 2);
  const int64_t stride = (int64_t)B * N;
  hipStream_t st = pdk::as_stream(stream);
  switch (splits) {
    case 1: hipLaunchKernelGGL(rope_append_kernel<1>, grid, block, 0, st, partials, (int64_t)N, stride, q_out, inv_freq, ctx_lens, block_tables, max_blocks, cache_k, cache_v, num_blocks, n_q_heads, n_kv_heads, head_dim, ssq, n_ssq, eps); break;
    case 2: hipLaunchKernelGGL(rope_append_kernel<2>, grid, block, 0, st, partials, (int64_t)N, stride, q_out, inv_freq, ctx_lens, block_tables, max_blocks, cache_k, cache_v, num_blocks, n_q_heads, n_kv_heads, head_dim, ssq, n_ssq, eps); break;
    case 4: hipLaunchKernelGGL(rope_append_kernel<4>, grid, block, 0, st, partials, (int64_t)N, stride, q_out, inv_freq, ctx_lens, block_tables, max_blocks, cache_k, cache_v, num_blocks, n_q_heads, n_kv_heads, head_dim, ssq, n_ssq, eps); break;
    default:
      pdk::set_error("splits must be 1, 2 or 4 (got %d)", splits);
      return PDK_EINVAL;
  }
  return pdk::check_launch("rope_append_kernel");
}

extern "C" int pdk_rope_cache_append_partials(const float* partials, int splits, int N,
                                              uint16_t* q_out, const float* inv_freq,
                                              const int32_t* ctx_lens,
                                              const int32_t* block_tables, int max_blocks,
                                              uint16_t* cache_k, uint16_t* cache_v,
                                              int num_blocks, int B, int n_q_heads,
                                              int n_kv_heads, int head_dim, uintptr_t stream) {
  pdk::clear_error();
  return rope_partials(partials, splits, N, q_out, inv_freq, ctx_lens, block_tables, max_blocks,
                       cache_k, cache_v, num_blocks, B, n_q_heads, n_kv_heads, head_dim, nullptr,
                       0, 0.f, stream);
}

extern "C" int pdk_rope_cache_append_partials_rms(
    const float* partials, int splits, int N, const float* ssq, int n_ssq, float eps,
    uint16_t* q_out, const float* inv_freq, const int32_t* ctx_lens, const int32_t* block_tables,
    int max_blocks, uint16_t* cache_k, uint16_t* cache_v, int num_blocks, int B, int n_q_heads,
    int n_kv_heads, int head_dim, uintptr_t stream) {
  pdk::clear_error();
  PDK_REQUIRE(ssq, "null pointer argument");
  return rope_partials(partials, splits, N, q_out, inv_freq, ctx_lens, block_tables, max_blocks,
                       cache_k, cache_v, num_blocks, B, n_q_heads, n_kv_heads, head_dim, ssq,
                       n_ssq, eps, stream);
}

extern "C" int pdk_swiglu(const uint16_t* gate_up, int B, int M, uint16_t* out,
                          uintptr_t stream) {
  pdk::clear_error();
  PDK_REQUIRE(gate_up && out, "null pointer argument");
  PDK_REQUIRE(B >= 1 && M >= 8 && M % 8 == 0, "B >= 1 and M a positive multiple of 8");
  PDK_REQUIRE(pdk::aligned16(gate_up) && pdk::aligned16(out), "tensors must be 16-byte aligned");
  const int64_t n8 = (int64_t)B * (M / 8);
  const int64_t blocks = (n8 + 255) / 256;
  PDK_REQUIRE(blocks < (1ll << 31), "launch too large");
  hipLaunchKernelGGL(swiglu_kernel, dim3((unsigned)blocks), dim3(256), 0,
                     pdk::as_stream(stream), gate_up, M, n8, out);
  return pdk::check_launch("swiglu_kernel");
}
