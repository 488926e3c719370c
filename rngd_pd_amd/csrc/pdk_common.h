// Internal helpers shared by the librngdpd HIP sources (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "rngdpd.h"

namespace pdk {

// Thread-local error text behind pdk_last_error().
void set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
void clear_error();
// Records a HIP failure and returns PDK_EHIP.
int hip_fail(hipError_t e, const char* what);
// Reports a launch error (hipGetLastError) after a kernel launch.
int check_launch(const char* what);
// Asynchronous copy between pinned or pageable host memory and device memory
// on stream st (DMA engines when the host range is pinned).
int copy_host_device(void* host, void* dev, size_t bytes, bool to_host, hipStream_t st);

inline hipStream_t as_stream(uintptr_t s) { return reinterpret_cast<hipStream_t>(s); }
inline hipEvent_t as_event(uintptr_t e) { return reinterpret_cast<hipEvent_t>(e); }
inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// 8 bf16 values in one 16-byte register group: word w holds elements 2w (low
// half) and 2w+1 (high half).
struct v8 {
  uint32_t w[4];
};

__device__ __forceinline__ v8 ld16(const uint16_t* p) {
  const uint4 x = *reinterpret_cast<const uint4*>(p);
  return v8{{x.x, x.y, x.z, x.w}};
}

__device__ __forceinline__ void st16(uint16_t* p, const v8& v) {
  *reinterpret_cast<uint4*>(p) = make_uint4(v.w[0], v.w[1], v.w[2], v.w[3]);
}

// Streaming (non-temporal) variants: the same data movement with a hint that
// the lines are not reused soon. Use the store for full 128-byte lines only:
// a partial-line streaming store loses the L2's write combining.
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ v8 ld16_stream(const uint16_t* p) {
  const u32x4_t x = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
  return v8{{x[0], x[1], x[2], x[3]}};
}

__device__ __forceinline__ void st16_stream(uint16_t* p, const v8& v) {
  const u32x4_t x = {v.w[0], v.w[1], v.w[2], v.w[3]};
  __builtin_nontemporal_store(x, reinterpret_cast<u32x4_t*>(p));
}

template <bool kStream>
__device__ __forceinline__ v8 ld16_as(const uint16_t* p) {
  return kStream ? ld16_stream(p) : ld16(p);
}

template <bool kStream>
__device__ __forceinline__ void st16_as(uint16_t* p, const v8& v) {
  if (kStream) st16_stream(p, v);
  else st16(p, v);
}

__device__ __forceinline__ v8 zero8() { return v8{{0u, 0u, 0u, 0u}}; }

// Paged K-cache block layout. One (block, KV head) holds 16 tokens x D dims of
// bf16 (D % 32 == 0) as 16-byte units of 8 consecutive dims of one token, in
// the order the decode-attention QK tiles read them, so that each of those
// load instructions reads whole 128-byte lines. The unit of token `slot`
// (0..15) and dims d0..d0+7 (d0 % 8 == 0) is
//   ((t * (D / 32) + s) * 4 + g) * 8 + j8,
//   t = (slot >> 2) & 1,  j8 = (slot >> 3) * 4 + (slot & 3),
//   s = d0 / 32,          g = (d0 / 8) % 4.
// Tile t holds the 8 tokens whose slot has bit 2 equal to t; within it, the
// 8 tokens of one 8-dim group are contiguous (128 bytes).
__host__ __device__ __forceinline__ int k_unit(int slot, int d0, int D) {
  const int t = (slot >> 2) & 1, j8 = ((slot >> 3) << 2) | (slot & 3);
  return ((t * (D >> 5) + (d0 >> 5)) * 4 + ((d0 >> 3) & 3)) * 8 + j8;
}

// Tiled activation layout of the decode step's bf16 [rows][K] operands (K %
// 128 == 0; rows padded to a multiple of 16): the 16 x 128 block of rows
// 16t..16t+15 and columns 128s..128s+127 is 2048 contiguous elements, in the
// order the GEMM lanes read their MFMA operand (lane l = 16 kg + r, r the row
// in the tile, reads 8 columns 32c + 8kg .. + 7 at element (c * 64 + l) * 8),
// so each load instruction of a GEMM reads 1 KiB of consecutive bytes instead
// of 64-byte pieces of 16 rows. Element (m, n) of such an operand is at
//   ((m / 16) * (K / 128) + n / 128) * 2048 + (((n % 128) / 8) * 16 + m % 16) * 8 + n % 8
// (columns 32c + 8kg .. + 7 of a block are its 16-byte group 4c + kg).
__host__ __device__ __forceinline__ int64_t act_at(int m, int n, int K) {
  return ((int64_t)(m >> 4) * (K >> 7) + (n >> 7)) * 2048 +
         ((((n & 127) >> 3) << 4) + (m & 15)) * 8 + (n & 7);
}

// Zero the elements e with first + e >= limit (first..first+7 are the token
// indices of the 8 elements).
__device__ __forceinline__ void mask_tail(v8& v, int first, int limit) {
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const uint32_t lo = (first + 2 * w < limit) ? 0x0000ffffu : 0u;
    const uint32_t hi = (first + 2 * w + 1 < limit) ? 0xffff0000u : 0u;
    v.w[w] &= (lo | hi);
  }
}

// 8x8 transpose of 16-bit elements held by one lane: in[r] is row r
// (elements c = 0..7); out[c] becomes column c (elements r = 0..7).
__device__ __forceinline__ void transpose8x8(const v8 in[8], v8 out[8]) {
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    const int w = c >> 1;
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const uint32_t a = in[2 * p].w[w];
      const uint32_t b = in[2 * p + 1].w[w];
      out[c].w[p] = (c & 1) ? ((a >> 16) | (b & 0xffff0000u))
                            : ((a & 0x0000ffffu) | (b << 16));
    }
  }
}

// fp32 -> bf16 bits, round to nearest even (inputs here are finite).
__device__ __forceinline__ uint32_t f32_to_bf16_rne(float f) {
  uint32_t u = __float_as_uint(f);
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}

// Two floats rounded to nearest-even bf16 and packed (a in the low half): one
// v_cvt_pk_bf16_f32 on gfx950. Equal to f32_to_bf16_rne on every finite input.
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_bf16x2_rne(float a, float b) {
  const f32x2_t v = {a, b};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}

// Row scale of an RMSNorm whose gain is folded into the next weights:
// rsqrt(sum_t ssq[row * n_tiles + t] / K + eps), t < n_tiles, ssq [rows]
// [n_tiles] holding each 16-column tile's sum of squares of the row. Lane l
// (l = lane & 31) of a 32-lane group adds tiles l, l + 32, ... in increasing
// order, then a fixed xor butterfly (every lane of the group ends with the
// same bits), so the value depends on nothing but the row's data. The 32
// lanes of the group must all be active. row_rms_load issues the first 256
// tiles' loads (unconditional, from clamped addresses; one 128-byte line per
// instruction) and returns at once, so a caller can issue other loads before
// row_rms_finish waits for these.
struct RowRms {
  float v[8];
};

__device__ __forceinline__ RowRms row_rms_load(const float* ssq, int row, int n_tiles, int lane) {
  const int l = lane & 31;
  const float* p = ssq + (int64_t)row * n_tiles;
  RowRms r;
#pragma unroll
  for (int i = 0; i < 8; ++i) r.v[i] = p[min(l + 32 * i, n_tiles - 1)];
  return r;
}

__device__ __forceinline__ float row_rms_finish(const RowRms& r, const float* ssq, int row,
                                                int n_tiles, int K, float eps, int lane) {
  const int l = lane & 31;
  const float* p = ssq + (int64_t)row * n_tiles;
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) s += l + 32 * i < n_tiles ? r.v[i] : 0.f;
  for (int t = l + 256; t < n_tiles; t += 32) s += p[t];
#pragma unroll
  for (int o = 1; o < 32; o <<= 1) s += __shfl_xor(s, o);
  return rsqrtf(s / (float)K + eps);
}

__device__ __forceinline__ float bf16_to_f32(uint32_t h) {
  return __uint_as_float(h << 16);
}

// RoPE on one pair of dims (x0, x1) = (dim i, dim i + D/2) with cos c and sin
// s: (x0 c - x1 s, x1 c + x0 s), each as one fused multiply-add on a rounded
// product. Written out so that every kernel that rotates (the fused attention
// and the separate cache append) rounds the same way whatever the compiler
// would contract on its own: their outputs are compared bit for bit.
__device__ __forceinline__ void rope_pair(float x0, float x1, float c, float s, float& y0,
                                          float& y1) {
  y0 = __builtin_fmaf(x0, c, -(x1 * s));
  y1 = __builtin_fmaf(x1, c, x0 * s);
}

}  // namespace pdk

#define PDK_TRY_HIP(call)                              \
  do {                                                 \
    hipError_t _pdk_e = (call);                        \
    if (_pdk_e != hipSuccess) return pdk::hip_fail(_pdk_e, #call); \
  } while (0)

#define PDK_REQUIRE(cond, ...)        \
  do {                                \
    if (!(cond)) {                    \
      pdk::set_error(__VA_ARGS__);    \
      return PDK_EINVAL;              \
    }                                 \
  } while (0)
