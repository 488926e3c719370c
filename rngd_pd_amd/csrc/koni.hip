// KONI token blocks into the paged KV cache (gfx950).
//
// The Furiosa native connector ships KV as units of one token of one tensor:
// tensor t = 2*layer + (0: K, 1: V), a unit = [Hkv][D] bf16, token-major
// (native_v4/kv.py:1-20). The reference's receiver writes each unit into
// host ATOM buffers (native_v4/kv.py:100-118); here a batch of units, uploaded
// as it arrived, goes straight into the paged cache.
//
// index[t][tok] = the unit holding token tok of tensor t, or -1 (not in this
// batch). One workgroup per (tensor, 16-token cache block): it loads the
// block's present units into LDS (coalesced: a unit is H*D*2 contiguous
// bytes; all of a thread's loads in flight at once), then writes the cache
// block in its own order, K as the tiled units of pdk::k_unit (16 contiguous
// bytes per (token, 8 dims), 128-byte runs of 8 tokens) and V as [D][16] rows
// (16 bytes = 8 consecutive slots, from an 8x8 register transpose of 16-byte
// LDS reads). Slots whose token is absent are not written. HBM-bound: read +
// write once. One 512-token Llama-3.1-8B request: 30.7 us, against 32-34 us
// when each load waited for the one before and V was gathered 2 bytes at a
// time.

#include "pdk_common.h"

namespace {

using pdk::v8;

constexpr int kThreads = 256;
constexpr int kMaxUnit8 = 128;     // H*D <= 1024: 16 tokens x 2 KiB = 32 KiB of LDS at most

__global__ __launch_bounds__(kThreads) void koni_scatter_kernel(
    const uint16_t* __restrict__ units, int64_t n_units, const int32_t* __restrict__ index,
    int n_tokens, const int32_t* __restrict__ table, int max_blocks, int num_blocks, int H,
    int D, uint16_t* ck, uint16_t* cv, int64_t layer_stride) {
  extern __shared__ v8 lds[];                      // [16][H*D/8]
  const int j = blockIdx.x, t = blockIdx.y;
  const int layer = t >> 1, kind = t & 1;
  const int u8 = (H * D) >> 3;                     // 16-byte pieces per unit
  if (j >= max_blocks) return;
  const int blk = table[j];
  if (blk < 0 || blk >= num_blocks) return;
  __shared__ int32_t src[16];
  __shared__ uint32_t present;                     // bit s: slot s's token is in the batch
  if (threadIdx.x < 64) {
    const int tok = j * 16 + threadIdx.x;
    int32_t u = (threadIdx.x < 16 && tok < n_tokens) ? index[(int64_t)t * n_tokens + tok] : -1;
    u = (u >= 0 && u < n_units) ? u : -1;
    if (threadIdx.x < 16) src[threadIdx.x] = u;
    const uint64_t bits = __ballot(u >= 0);
    if (threadIdx.x == 0) present = (uint32_t)bits;
  }
  __syncthreads();
  // Every piece's load is issued before any is stored (absent slots read unit
  // 0, in bounds, and are never written out): one round trip, not eight.
  constexpr int kPer = 16 * kMaxUnit8 / kThreads;  // pieces per thread at the largest unit
  v8 in[kPer];
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int p = threadIdx.x + i * kThreads;
    if (p < 16 * u8) {
      const int s = p / u8, c = p - s * u8;
      const int32_t u = src[s];
      in[i] = pdk::ld16(units + (int64_t)(u >= 0 ? u : 0) * (H * D) + 8 * c);
    }
  }
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int p = threadIdx.x + i * kThreads;
    if (p < 16 * u8) lds[p] = in[i];
  }
  __syncthreads();
  if (kind == 0) {
    // K: per head a block of 16 * D/8 tiled units; q is the unit's position in it.
    uint16_t* base = ck + (int64_t)layer * layer_stride + (int64_t)blk * H * 16 * D;
    const int per_head = 2 * D;                    // 16 * D / 8
    const int s32n = D >> 5;
    for (int o = threadIdx.x; o < H * per_head; o += kThreads) {
      const int h = o / per_head, q = o - h * per_head;
      const int j8 = q & 7, g = (q >> 3) & 3, rest = q >> 5;
      const int tt = rest / s32n, s32 = rest - tt * s32n;
      const int slot = ((j8 >> 2) << 3) | (tt << 2) | (j8 & 3);
      const int d0 = s32 * 32 + g * 8;
      if ((present >> slot) & 1u)
        pdk::st16(base + (int64_t)h * 16 * D + 8 * q, lds[slot * u8 + ((h * D + d0) >> 3)]);
    }
  } else {
    // V: rows (h, d) of 16 slots. A thread takes 8 dims x 8 slots: the eight
    // slots' 16-byte pieces of those dims, transposed in registers, give eight
    // 16-byte row pieces (8 consecutive slots of one dim each).
    uint16_t* base = cv + (int64_t)layer * layer_stride + (int64_t)blk * H * D * 16;
    for (int o = threadIdx.x; o < 2 * u8; o += kThreads) {
      const int dg = o % u8, half = o / u8;        // dims 8 dg .. 8 dg + 7, slots 8 half ..
      const uint32_t bits = (present >> (8 * half)) & 0xffu;
      if (!bits) continue;
      v8 rows[8], cols[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) rows[k] = lds[(8 * half + k) * u8 + dg];
      pdk::transpose8x8(rows, cols);               // cols[c]: dim 8 dg + c, slots 8 half + 0..7
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        uint16_t* dst = base + (int64_t)(8 * dg + c) * 16 + 8 * half;
        if (bits == 0xffu) {
          pdk::st16(dst, cols[c]);
        } else {
#pragma unroll
          for (int k = 0; k < 8; ++k)
            if ((bits >> k) & 1u)
              dst[k] = (uint16_t)(cols[c].w[k >> 1] >> (16 * (k & 1)));
        }
      }
    }
  }
}

}  // namespace

extern "C" int pdk_scatter_koni(const uint16_t* units, int64_t n_units, const int32_t* index,
                                int n_tensors, int n_tokens, const int32_t* block_table,
                                int max_blocks, uint16_t* cache_k, uint16_t* cache_v,
                                int64_t layer_stride, int num_blocks, int n_kv_heads,
                                int head_dim, uintptr_t stream) {
  pdk::clear_error();
  PDK_REQUIRE(units && index && block_table && cache_k && cache_v, "null pointer argument");
  PDK_REQUIRE(n_units >= 1 && n_tokens >= 1 && n_tensors >= 2 && n_tensors % 2 == 0 &&
                  n_tensors <= 65535,
              "bad counts: %lld units, %d tokens, %d tensors", (long long)n_units, n_tokens,
              n_tensors);
  PDK_REQUIRE(head_dim >= 32 && head_dim % 32 == 0, "head_dim must be a multiple of 32");
  PDK_REQUIRE(n_kv_heads >= 1 && n_kv_heads * head_dim <= kMaxUnit8 * 8 &&
                  (n_kv_heads * head_dim) % 8 == 0,
              "a unit of %d x %d exceeds %d elements", n_kv_heads, head_dim, kMaxUnit8 * 8);
  PDK_REQUIRE(max_blocks >= (n_tokens + 15) / 16, "block table holds %d blocks, %d tokens need %d",
              max_blocks, n_tokens, (n_tokens + 15) / 16);
  PDK_REQUIRE(num_blocks >= 1 && layer_stride >= (int64_t)num_blocks * n_kv_heads * 16 * head_dim,
              "layer stride too small");
  PDK_REQUIRE(pdk::aligned16(units) && pdk::aligned16(cache_k) && pdk::aligned16(cache_v),
              "tensors must be 16-byte aligned");
  const size_t lds = (size_t)16 * n_kv_heads * head_dim * 2;
  hipLaunchKernelGGL(koni_scatter_kernel, dim3((n_tokens + 15) / 16, n_tensors), dim3(kThreads),
                     lds, pdk::as_stream(stream), units, n_units, index, n_tokens, block_table,
                     max_blocks, num_blocks, n_kv_heads, head_dim, cache_k, cache_v,
                     layer_stride);
  return pdk::check_launch("koni_scatter_kernel");
}
