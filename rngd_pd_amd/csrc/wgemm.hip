// Weight-streaming GEMMs of the decode step for gfx950:
//   Y[B][N] = X[B][K] . W[N][K]^T            (+ R[B][N] when a residual is given)
//   Y[B][M] = silu(X . Wg^T) * (X . Wu^T)     (W = [Wg; Wu], 2M rows: gate then up)
// for B <= 64 streams. W is [out][in] (torch Linear layout), bf16; fp32
// accumulation on the matrix cores; bf16 out.
//
// At decode batch sizes each weight element is used B times, so these GEMMs
// are bound by HBM: the kernel's job is to read W once, as fast as HBM
// delivers it, and keep the few activation rows in cache. Mapping:
//   * one workgroup per kCols tiles of 16 output columns, kWaves waves
//     splitting K in steps of 128 (wave w takes steps w, w + kWaves, ...);
//   * per step a lane loads 4 x 16 bytes of one W row, (column lane % 16, k
//     offsets 32c + 8 (lane / 16)), and the same k offsets of one X row (row
//     lane % 16 of each 16-row tile), then issues 4 v_mfma_f32_16x16x32_bf16
//     per tile: the 16x16 result tile is [stream][column];
//   * rows past B read row B-1 and columns past N read column N-1 (in bounds,
//     results dropped), so no masking;
//   * the waves' partial tiles meet in LDS, and the epilogue (residual add or
//     SwiGLU) runs on the fp32 sums before the single bf16 rounding.
// A [out][in] W is read with ordinary loads: non-temporal ones measured
// 10-25 % slower in that layout, although a decode step streams every weight
// once. A tiled W (below) is read with non-temporal loads, which are faster
// there: gate|up at Llama-3.1-8B shape 40.3 -> 37.1 us, the lm_head 200 ->
// 185 us at B = 16.
//
// Tiled weights. The same GEMMs also take W as a tiled copy (pdk_weight_tile)
// in which the 4 KiB that a wavefront reads for one 16-column tile and one
// 128-long k step are contiguous, in the order the lanes read them: each load
// instruction then reads 1 KiB of consecutive bytes instead of 64 bytes of
// each of 16 rows.
//   tile t = rows 16t .. 16t+15 (rows >= N zero); block (t, s) holds its k
//   step s (2048 elements) and starts at (s * tiles + t) * 2048; element
//   ((c * 4 + kg) * 16 + col) * 8 + e of it is W[16t + col][128 s + 32 c +
//   8 kg + e].
// The blocks are step-major: the workgroups of a launch advance through K
// together, so at any time they read one region a few MiB wide instead of a
// separate run per column tile spread over the whole matrix (HBM serves the
// former faster). Tile-major, each column tile's K contiguous, the decode step
// of Llama-3.1-8B took 2.985-2.988 ms at B = 16 and 2.855-2.857 at B = 4;
// step-major 2.929-2.932 and 2.796-2.809 (three alternating runs of each on
// one box, bit-identical results).
//
// Tiled activations. The _xt entry points take the decode step's bf16
// activations (x, the residual and the output y) in the tiled layout of
// pdk::act_at, the same order for rows that the tiled weights use for
// columns: an X load instruction then reads 1 KiB of consecutive bytes
// instead of a 64-byte piece of each of 16 rows. At Llama-3.1-8B shapes and
// B = 16 (32 launches of each in a HIP graph, tiled weights) that took the
// five GEMMs of a layer from 82.1 to 78.5 us: O 9.55 -> 8.28, q|k|v 11.84 ->
// 11.02, gate|up 38.04 -> 37.30, down 22.68 -> 21.89. Rows past B are never
// read (lanes of rows >= B read row B - 1, as in the row-major layout), so
// the padding rows of a tile may hold anything. fp32 partials, logits and
// the sums of squares keep their row-major layouts.

#include <math.h>

#include "pdk_common.h"

namespace {

using pdk::v8;


typedef __bf16 bf16x8_t __attribute__((__vector_size__(16)));
typedef float f32x4 __attribute__((__vector_size__(16)));

__device__ __forceinline__ f32x4 mfma(const v8& a, const v8& b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                 __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}

constexpr int kStepK = 128;        // k per wave step: 4 MFMA of 32
constexpr int kWaves = 8;
constexpr int kBlock = 16 * kStepK;  // tiled W: one tile's k step, 4 KiB

// kResidualSsq: kResidual that also writes, per 16-column tile and row, the
// sum of squares of the bf16 outputs (ssq[row][tile]): the raw material of the
// next RMSNorm. kSwiGLURms: kSwiGLU on weights with that norm's gain folded
// into their columns, whose input x is the un-normalised residual: each row's
// two sums are scaled by r = rsqrt(sum(ssq[row][.]) / K + eps) before SwiGLU,
// so rmsnorm(x) . W^T = r * (x . (W diag g)^T) takes no launch of its own.
//
// kPartialFinal: kPartial whose last-arriving split of each column group adds
// the splits' partials in split order to the residual (y = bf16(r + sum), r
// may alias y: the update pdk_rmsnorm_partials makes) and writes that
// group's sums of squares as kResidualSsq does, so the next RMSNorm needs no
// launch. kArgmaxRms: kArgmax on weights with the final norm's gain folded in,
// each row's logits scaled by its r (from ssq) before rounding. kPartialRms:
// kPartial on weights with a norm's gain folded in, each row's partial scaled
// by its r (the q|k|v projection: its consumer adds the scaled halves).
enum Epilogue { kPlain = 0, kResidual = 1, kSwiGLU = 2, kArgmax = 3, kPartial = 4,
                kResidualSsq = 5, kSwiGLURms = 6, kPartialFinal = 7, kArgmaxRms = 8,
                kPartialRms = 9 };

// Greedy-token key of one bf16 logit: the value in an order-preserving code
// above the complement of the column, so the unsigned maximum is the largest
// value at its lowest column (torch.argmax: NaN above every number, the first
// of equal values; -0 counts as +0). 0 is below every key.
__device__ __forceinline__ uint64_t argmax_key(uint32_t h, int n) {
  h &= 0xffffu;
  if (h == 0x8000u) h = 0;                                   // -0 -> +0
  uint32_t ord;
  if ((h & 0x7fffu) > 0x7f80u) ord = 0xffffu;               // NaN
  else ord = (h & 0x8000u) ? (~h & 0xffffu) : (h | 0x8000u);
  return ((uint64_t)ord << 32) | (uint64_t)(0xffffffffu - (uint32_t)n);
}

// Loads in flight per wave: kDepth steps of W (and X), no more than about 160
// VGPRs of load buffers, and at most 4. With step-major tiled weights fewer
// steps in flight pay at one row tile (B <= 16), measured on the Llama-3.1-8B
// decode step (32-layer graph, three alternating runs of each on one box):
// one column tile (the O and down projections) at depth 2 instead of 4, B=16
// 2.931-2.933 -> 2.907-2.911 ms, B=4 2.772-2.774 -> 2.759-2.762 (depth 1: B=16
// 2.915-2.921); q|k|v (3 column tiles) at depth 1 instead of 2, B=16
// 2.906-2.911 -> 2.895-2.908, B=4 unchanged. Before the weights were
// step-major, depth 4 had been the fastest for one column tile.
constexpr int depth_for(int row_tiles, int w_tiles) {
  if (row_tiles == 1 && w_tiles == 1) return 2;
  if (row_tiles == 1 && w_tiles == 3) return 1;
  const int tiles = row_tiles + w_tiles;
  return 160 / (16 * tiles) < 1 ? 1 : 160 / (16 * tiles) > 4 ? 4 : 160 / (16 * tiles);
}

// kTiles = ceil(B / 16) row tiles; kCols = 16-column tiles per workgroup (all
// its waves share them and split K); kEpi selects the epilogue. For kSwiGLU the
// workgroup also computes the matching up columns (rows n and M + n of W) and
// writes silu(g) * u.
template <int kTiles, int kCols, int kEpi, bool kTiled, bool kAct>
__global__ __launch_bounds__(kWaves * 64) void wgemm_kernel(const uint16_t* __restrict__ x,
                                                            const uint16_t* __restrict__ w, int B,
                                                            int K, int N, int splits, float* ssq,
                                                            const uint16_t* r, uint16_t* y,
                                                            uint64_t* keys, float* part,
                                                            float eps, int* counters) {
  // The arguments up to y (14 dwords) arrive preloaded in SGPRs: everything
  // the first loads need, including the split count (gridDim.y would be a
  // load from the hidden kernel arguments, a round trip before the first
  // weight load) and the row sums of squares. Their row length is K / 16.
  const int n_ssq = K >> 4;
  constexpr bool kGLU = kEpi == kSwiGLU || kEpi == kSwiGLURms;
  constexpr bool kRowScale = kEpi == kSwiGLURms || kEpi == kArgmaxRms || kEpi == kPartialRms;
  constexpr bool kArg = kEpi == kArgmax || kEpi == kArgmaxRms;
  constexpr int kPairs = kGLU ? 2 : 1;
  constexpr int kW = kPairs * kCols;                 // W tiles per step
  constexpr int kDepth = depth_for(kTiles, kW);
  __shared__ float red[kWaves][kW][256];
  __shared__ float rms[kRowScale ? 64 : 1];
  __shared__ int is_last;
  __shared__ uint64_t kbest[kArg ? 16 : 1][kArg ? kCols : 1];   // per row of a tile, per column tile
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int col = lane & 15, kg = lane >> 4;
  const int n0 = blockIdx.x * 16 * kCols;
  const uint16_t* wp[kW];
  const int n_tiles = (N + 15) >> 4;
  // Tiled W is step-major: k step s of every tile (gate and up tiles for
  // SwiGLU), then step s + 1.
  const int64_t step_stride = (int64_t)kPairs * n_tiles * kBlock;
#pragma unroll
  for (int p = 0; p < kPairs; ++p)
#pragma unroll
    for (int c = 0; c < kCols; ++c) {
      if (kTiled)   // tile of columns n0 + 16c (the last one past N), rows of pair p after it
        wp[p * kCols + c] =
            w + ((int64_t)p * n_tiles + min((n0 >> 4) + c, n_tiles - 1)) * kBlock + lane * 8;
      else
        wp[p * kCols + c] = w + ((int64_t)p * N + min(n0 + 16 * c + col, N - 1)) * K + kg * 8;
    }
  // X operand of row tile t: row min(16t + col, B - 1), k offsets 32c + 8kg.
  // Tiled activations (kAct): that row's 16-byte group 4c + kg of each
  // 2048-element block, pdk::act_at.
  const uint16_t* xp[kTiles];
#pragma unroll
  for (int t = 0; t < kTiles; ++t) {
    const int row = min(t * 16 + col, B - 1);
    xp[t] = kAct ? x + (int64_t)(row >> 4) * 16 * K + (kg * 16 + (row & 15)) * 8
                 : x + (int64_t)row * K + kg * 8;
  }
  // The residual under this thread's epilogue element (at most one per row
  // tile when the workgroup's columns fit one pass of its threads), loaded
  // before any weight from a clamped address, so every lane loads and the
  // weights' waits stay exact: the epilogue then adds it without a round trip
  // to memory after the products. y may be the residual itself (in place);
  // only this thread writes that element, and only after this read.
  constexpr bool kResPre =
      (kEpi == kResidual || kEpi == kResidualSsq) && 256 * kCols <= kWaves * 64;
  uint16_t rpre[kResPre ? kTiles : 1];
  if constexpr (kResPre) {
    const int e = min((int)threadIdx.x, 256 * kCols - 1);
#pragma unroll
    for (int t = 0; t < kTiles; ++t) {
      const int m = min(t * 16 + ((e >> 4) & 15), B - 1);
      const int n = min(n0 + 16 * (e >> 8) + (e & 15), N - 1);
      rpre[t] = r[kAct ? pdk::act_at(m, n, N) : (int64_t)m * N + n];
    }
  }

  f32x4 acc[kW][kTiles];
#pragma unroll
  for (int q = 0; q < kW; ++q)
#pragma unroll
    for (int t = 0; t < kTiles; ++t) acc[q][t] = f32x4{0.f, 0.f, 0.f, 0.f};

  // This wave's steps are first, first + stride, ...: n_mine of them. Buffers
  // cycle through kDepth slots; a slot past the wave's last step loads that
  // last step again (a valid address) and its X operand is zeroed, so every
  // load is unconditional and the tail adds nothing.
  // Split-K over `splits` (= gridDim.y) workgroups: this one takes steps [s_lo, s_hi).
  const int steps_all = K / kStepK;
  const int s_lo = (int)((int64_t)blockIdx.y * steps_all / splits);
  const int s_hi = (int)((int64_t)(blockIdx.y + 1) * steps_all / splits);
  const int steps = s_hi - s_lo;
  // Steps of this wave: wave, wave + kWaves, ... (so the workgroup's waves
  // read consecutive k blocks together). Each wave's share, and so the order
  // of the fp32 sums, is the same for both weight layouts.
  const int first = wave;
  const int n_mine = steps > wave ? (steps - wave + kWaves - 1) / kWaves : 0;
  constexpr int stride = kWaves;
  const int last = min(first + (max(n_mine, 1) - 1) * stride, steps - 1);
  v8 wv[kDepth][kW][4], xv[kDepth][kTiles][4];
  auto load = [&](int slot, int j) {
    const int k = (s_lo + min(first + j * stride, last)) * kStepK;
#pragma unroll
    for (int q = 0; q < kW; ++q)
#pragma unroll
      for (int c = 0; c < 4; ++c)
        wv[slot][q][c] = kTiled ? pdk::ld16_stream(wp[q] + (k / kStepK) * step_stride + 512 * c)
                                : pdk::ld16(wp[q] + k + 32 * c);
#pragma unroll
    for (int t = 0; t < kTiles; ++t)
#pragma unroll
      for (int c = 0; c < 4; ++c)
        xv[slot][t][c] = kAct ? pdk::ld16(xp[t] + (int64_t)k * 16 + 512 * c)
                              : pdk::ld16(xp[t] + k + 32 * c);
  };
  // Row scales (kRowScale): 32 lanes per row (16 rows per pass over the
  // workgroup, kTiles passes), each adding every 32nd tile's sum of squares,
  // then a fixed butterfly: a row's scale depends neither on B nor on timing.
  // A lane's loads are issued before the first steps' weight loads
  // (unconditional, from clamped addresses). With at most 256 tiles and one row
  // tile (two, but for the register-heavy SwiGLU epilogue) the values stay in registers and are summed in the epilogue, so
  // nothing waits for them before the main loop; otherwise they are summed
  // right after the first weight loads are issued.
  constexpr int kTpr = 32, kPer = 8;                 // 32 lanes x 8 tiles per pass
  constexpr bool kLate = kRowScale && (kTiles == 1 || (kTiles == 2 && kEpi != kSwiGLURms));
  const int srow = threadIdx.x / kTpr, ssub = threadIdx.x % kTpr;
  const bool late = kLate && n_ssq <= kTpr * kPer;
  float sv[kLate ? kTiles : 1][kPer];
  if constexpr (kRowScale) {
    if (late) {
#pragma unroll
      for (int t = 0; t < (kLate ? kTiles : 1); ++t) {
        const float* sp = ssq + (int64_t)min(t * 16 + srow, B - 1) * n_ssq;
#pragma unroll
        for (int i = 0; i < kPer; ++i) sv[t][i] = sp[min(ssub + i * kTpr, n_ssq - 1)];
      }
#pragma unroll
      for (int d = 0; d < kDepth; ++d) load(d, d);
    } else {
      float sq_part[kTiles];
#pragma unroll
      for (int t = 0; t < kTiles; ++t) sq_part[t] = 0.f;
      for (int base = 0; base < n_ssq; base += kTpr * kPer) {
        float v[kTiles][kPer];
#pragma unroll
        for (int t = 0; t < kTiles; ++t) {
          const float* sp = ssq + (int64_t)min(t * 16 + srow, B - 1) * n_ssq;
#pragma unroll
          for (int i = 0; i < kPer; ++i) v[t][i] = sp[min(base + ssub + i * kTpr, n_ssq - 1)];
        }
        if (base + kTpr * kPer >= n_ssq) {
#pragma unroll
          for (int d = 0; d < kDepth; ++d) load(d, d);
        }
#pragma unroll
        for (int t = 0; t < kTiles; ++t)
#pragma unroll
          for (int i = 0; i < kPer; ++i)
            sq_part[t] += base + ssub + i * kTpr < n_ssq ? v[t][i] : 0.f;
      }
#pragma unroll
      for (int t = 0; t < kTiles; ++t) {
#pragma unroll
        for (int o = 1; o < kTpr; o <<= 1) sq_part[t] += __shfl_xor(sq_part[t], o);
        if (ssub == 0) rms[t * 16 + srow] = rsqrtf(sq_part[t] / (float)K + eps);
      }
    }
  } else {
#pragma unroll
    for (int d = 0; d < kDepth; ++d) load(d, d);
  }
  for (int j0 = 0; j0 < n_mine; j0 += kDepth) {
#pragma unroll
    for (int d = 0; d < kDepth; ++d) {
      const int j = j0 + d;
      if (j >= n_mine) {                       // wave-uniform: zero the stale operand
#pragma unroll
        for (int t = 0; t < kTiles; ++t)
#pragma unroll
          for (int c = 0; c < 4; ++c) xv[d][t][c] = pdk::zero8();
      }
#pragma unroll
      for (int c = 0; c < 4; ++c)
#pragma unroll
        for (int q = 0; q < kW; ++q)
#pragma unroll
          for (int t = 0; t < kTiles; ++t) acc[q][t] = mfma(xv[d][t][c], wv[d][q][c], acc[q][t]);
      if (j + kDepth < n_mine) load(d, j + kDepth);
    }
  }

  if constexpr (kLate) {
    if (late) {                              // the same sums in the same order, now
#pragma unroll
      for (int t = 0; t < kTiles; ++t) {
        float sq = 0.f;
#pragma unroll
        for (int i = 0; i < kPer; ++i) sq += ssub + i * kTpr < n_ssq ? sv[t][i] : 0.f;
#pragma unroll
        for (int o = 1; o < kTpr; o <<= 1) sq += __shfl_xor(sq, o);
        if (ssub == 0) rms[t * 16 + srow] = rsqrtf(sq / (float)K + eps);
      }
    }
  }
  // acc[q][t][i] = partial Y[t*16 + 4*kg + i][column tile q, column col]; one
  // row tile at a time through LDS, summed over the waves.
#pragma unroll
  for (int t = 0; t < kTiles; ++t) {
    if (t) __syncthreads();
#pragma unroll
    for (int q = 0; q < kW; ++q)
#pragma unroll
      for (int i = 0; i < 4; ++i) red[wave][q][(4 * kg + i) * 16 + col] = acc[q][t][i];
    __syncthreads();
    for (int e = threadIdx.x; e < 256 * kCols; e += kWaves * 64) {
      const int c = e >> 8, m = t * 16 + ((e >> 4) & 15), n = n0 + 16 * c + (e & 15);
      const bool ok = m < B && n < N;
      float v[kPairs];
#pragma unroll
      for (int p = 0; p < kPairs; ++p) {
        float sum = 0.f;
#pragma unroll
        for (int q = 0; q < kWaves; ++q) sum += red[q][p * kCols + c][e & 255];
        v[p] = sum;
      }
      // Logits (the argmax epilogues) stay row-major; y and the residual are
      // activations, tiled with kAct.
      const int64_t at = kAct && !kArg ? pdk::act_at(m, n, N) : (int64_t)m * N + n;
      if (kEpi == kPartial || kEpi == kPartialRms) {
        const float pv = kEpi == kPartialRms ? v[0] * rms[m < 64 ? m : 63] : v[0];
        if (ok) part[((int64_t)blockIdx.y * B + m) * N + n] = pv;
        continue;
      }
      if (kEpi == kPartialFinal) {
        // Device-coherent stores: the split that finishes last reads them
        // from another workgroup, possibly on another XCD.
        if (ok)
          __hip_atomic_store(&part[((int64_t)blockIdx.y * B + m) * N + n], v[0], __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
        continue;
      }
      float out = v[0];
      if constexpr (kResPre) {
        if (ok) out += pdk::bf16_to_f32(rpre[t]);          // e == threadIdx.x here
      } else if ((kEpi == kResidual || kEpi == kResidualSsq) && ok) {
        out += pdk::bf16_to_f32(r[at]);
      }
      if (kEpi == kSwiGLU) out = v[0] / (1.f + expf(-v[0])) * v[kPairs - 1];
      if (kEpi == kSwiGLURms) {
        const float s = rms[m < 64 ? m : 63];
        const float a = v[0] * s, b = v[kPairs - 1] * s;
        out = a / (1.f + expf(-a)) * b;
      }
      if (kEpi == kArgmaxRms) out = v[0] * rms[m < 64 ? m : 63];
      const uint32_t h = pdk::f32_to_bf16_rne(out);
      if (ok && y) y[at] = (uint16_t)h;
      if (kEpi == kResidualSsq) {
        // Lanes e .. e|15 hold one row's 16 columns of this tile.
        const float hv = pdk::bf16_to_f32(h);
        float sq = ok ? hv * hv : 0.f;
#pragma unroll
        for (int o = 1; o < 16; o <<= 1) sq += __shfl_xor(sq, o);
        if ((e & 15) == 0 && m < B) ssq[(int64_t)m * (N >> 4) + blockIdx.x * kCols + c] = sq;
      }
      if (kArg) {
        // The 16 lanes e .. e|15 hold one row's 16 columns of this tile: the
        // best of them goes to LDS, and below the best of the workgroup's
        // column tiles to keys[m].
        uint64_t key = ok ? argmax_key(h, n) : 0;
#pragma unroll
        for (int o = 1; o < 16; o <<= 1) {
          const uint64_t other = __shfl_xor(key, o);
          key = other > key ? other : key;
        }
        if ((e & 15) == 0) kbest[(e >> 4) & 15][c] = key;
      }
    }
    if constexpr (kArg) {
      // One thread per row: the best key of the workgroup's columns goes to
      // keys[m], with an atomic only when it beats the value already there
      // (so few workgroups write). One device-scope round trip per row and
      // workgroup instead of one per row and column tile: the lm_head at
      // B = 16 went from 128 to 16 of them per workgroup.
      __syncthreads();
      const int mr = threadIdx.x, m = t * 16 + mr;
      if (mr < 16 && m < B) {
        uint64_t best = kbest[mr][0];
#pragma unroll
        for (int c = 1; c < kCols; ++c) best = kbest[mr][c] > best ? kbest[mr][c] : best;
        uint64_t* slot = keys + m;
        if (best > __hip_atomic_load(slot, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT))
          __hip_atomic_fetch_max(slot, best, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  }
  if constexpr (kEpi == kPartialFinal) {
    // This split's partial stores are complete before it counts itself in
    // (counters[blockIdx.x] counts the splits of this column group that are
    // done); the last one resets the count for the next call and finishes the
    // group. No workgroup waits for another.
    //
    // Ordering. Every access to the partials and the counter is an
    // agent-scope atomic, which gfx950 performs at the device's coherence
    // point (sc1: through the XCD's L2, not cached in it), so no write-back
    // or invalidation of a cache is needed for them to meet across XCDs. What
    // remains is order: s_waitcnt vmcnt(0) completes this workgroup's partial
    // stores (gfx9 counts stores in vmcnt) before the barrier and the ticket;
    // in the last split the loads of the partials follow the ticket's result
    // through the barrier and the is_last branch, so they issue after it
    // returned. The C++ model would want an acquire-release ticket instead,
    // but at agent scope that is a buffer_wbl2 + buffer_inv pair per
    // workgroup, which measured +80 us (B = 4) and +120 us (B = 16) on the
    // Llama-3.1-8B decode step (3-4 us per launch); the GPU tests hold this
    // launch bit-identical to the separate partials-plus-norm path, on two
    // calls in a row.
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0) {
      int* cnt = counters + blockIdx.x;
      const int done = __hip_atomic_fetch_add(cnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      const int last = done == splits - 1;
      if (last) __hip_atomic_store(cnt, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      is_last = last;
    }
    __syncthreads();
    if (!is_last) return;
    const int S = splits;
#pragma unroll
    for (int t = 0; t < kTiles; ++t) {
      for (int e = threadIdx.x; e < 256 * kCols; e += kWaves * 64) {
        const int c = e >> 8, m = t * 16 + ((e >> 4) & 15), n = n0 + 16 * c + (e & 15);
        const bool ok = m < B && n < N;
        const int mc = min(m, B - 1), nc = min(n, N - 1);
        const int64_t at = (int64_t)mc * N + nc;  // the fp32 partials are row-major
        const int64_t ra = kAct ? pdk::act_at(mc, nc, N) : at;
        float pv[16];
#pragma unroll
        for (int sp = 0; sp < 16; ++sp)
          if (sp < S)
            pv[sp] = __hip_atomic_load(&part[(int64_t)sp * B * N + at], __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
        float acc = 0.f;                         // in split order, as pdk_rmsnorm_partials adds
#pragma unroll
        for (int sp = 0; sp < 16; ++sp)
          if (sp < S) acc += pv[sp];
        const uint32_t h = pdk::f32_to_bf16_rne(pdk::bf16_to_f32(r[ra]) + acc);
        if (ok) y[ra] = (uint16_t)h;
        const float hv = pdk::bf16_to_f32(h);
        float sq = ok ? hv * hv : 0.f;
#pragma unroll
        for (int o = 1; o < 16; o <<= 1) sq += __shfl_xor(sq, o);
        if ((e & 15) == 0 && m < B) ssq[(int64_t)m * (N >> 4) + blockIdx.x * kCols + c] = sq;
      }
    }
  }
}

// tokens[b] = the column of keys[b]; keys[b] back to 0 for the next call.
__global__ void argmax_finish_kernel(uint64_t* keys, int B, int32_t* tokens) {
  const int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= B) return;
  const uint64_t k = keys[b];
  tokens[b] = (int32_t)(0xffffffffu - (uint32_t)k);
  keys[b] = 0;
}

template <int kCols, int kEpi, bool kTiled, bool kAct = false>
int launch_cols(const uint16_t* x, const uint16_t* w, int B, int K, int N, const uint16_t* r,
                uint16_t* y, uint64_t* keys, hipStream_t st, float* part = nullptr,
                int splits = 1, float* ssq = nullptr, int n_ssq = 0, float eps = 0.f,
                int* counters = nullptr) {
  const dim3 grid((N + 16 * kCols - 1) / (16 * kCols), splits), block(kWaves * 64);
#define PDK_WGEMM(T) \
  hipLaunchKernelGGL((wgemm_kernel<T, kCols, kEpi, kTiled, kAct>), grid, block, 0, st, x, w, B, K, N, splits, ssq, r, y, keys, part, eps, counters)
  switch ((B + 15) / 16) {
    case 1: PDK_WGEMM(1); break;
    case 2: PDK_WGEMM(2); break;
    case 3: PDK_WGEMM(3); break;
    default: PDK_WGEMM(4); break;
  }
#undef PDK_WGEMM
  return pdk::check_launch("wgemm_kernel");
}

// Column tiles per workgroup. Wider tiles read each X row once for more
// columns (X traffic from L2 is (N / 16 kCols) * B * K * 2 bytes, as much as W
// itself at B = 16 with one tile) but leave fewer workgroups. Measured at the
// Llama-3.1-8B shapes: gate|up (M = 14336) and the lm_head at B > 8 run best
// with 4 tiles; N = 4096 and 6144 need every workgroup one tile gives.
template <int kEpi, bool kTiled, bool kAct = false>
int launch(const uint16_t* x, const uint16_t* w, int B, int K, int N, const uint16_t* r,
           uint16_t* y, uint64_t* keys, hipStream_t st, float* ssq = nullptr, int n_ssq = 0,
           float eps = 0.f) {
  const int64_t wide = (N + 63) / 64;                // workgroups with 4 tiles
  // Wide SwiGLU tiles hold 8 weight tiles per step in registers: beyond 32
  // streams they would spill, and one tile is used instead. The lm_head with
  // tiled weights runs 4 tiles wide at every B (B = 4: 181 -> 178 us).
  constexpr bool kGLU = kEpi == kSwiGLU || kEpi == kSwiGLURms;
  // The lm_head on tiled activations runs 8 tiles wide up to B = 32: each
  // workgroup reads the activation rows once for 128 columns instead of 64,
  // and the decode step at B = 16 went 3.022 -> 3.007 ms (B = 4 unchanged).
  if (kAct && kEpi == kArgmaxRms && B <= 32 && wide >= 1024)
    return launch_cols<8, kEpi, kTiled, kAct>(x, w, B, K, N, r, y, keys, st, nullptr, 1, ssq,
                                              n_ssq, eps);
  const bool four = kGLU ? (wide >= 192 && B <= 32) : ((B > 8 || kTiled) && wide >= 1024);
  if (four) return launch_cols<4, kEpi, kTiled, kAct>(x, w, B, K, N, r, y, keys, st, nullptr, 1,
                                                      ssq, n_ssq, eps);
  return launch_cols<1, kEpi, kTiled, kAct>(x, w, B, K, N, r, y, keys, st, nullptr, 1, ssq, n_ssq,
                                            eps);
}

// Tiled copy of W [N][K]: one thread per 16-byte group of the copy.
__global__ void weight_tile_kernel(const uint16_t* __restrict__ w, int N, int K,
                                   uint16_t* __restrict__ wt, int64_t groups) {
  const int64_t gi = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gi >= groups) return;
  const int lane = (int)(gi & 63);                   // (kg, col) = (lane >> 4, lane & 15)
  const int c = (int)((gi >> 6) & 3);
  const int64_t blk = gi >> 8;                       // block: step * tiles + tile
  const int64_t n_t = (N + 15) / 16;
  const int s = (int)(blk / n_t);
  const int64_t t = blk - (int64_t)s * n_t;
  const int64_t row = t * 16 + (lane & 15);
  v8 v = pdk::zero8();
  if (row < N) v = pdk::ld16(w + row * K + s * kStepK + 32 * c + 8 * (lane >> 4));
  pdk::st16(wt + gi * 8, v);
}

int check_shape(const void* x, const void* w, const void* y, int B, int K, int N) {
  PDK_REQUIRE(x && w && y, "null pointer argument");
  PDK_REQUIRE(B >= 1 && B <= 64, "B must be in [1, 64] (got %d)", B);
  PDK_REQUIRE(K >= kStepK && K % kStepK == 0, "K must be a positive multiple of %d (got %d)",
              kStepK, K);
  PDK_REQUIRE(N >= 1, "N must be positive (got %d)", N);
  PDK_REQUIRE(pdk::aligned16(x) && pdk::aligned16(w), "x and w must be 16-byte aligned");
  return PDK_OK;
}


template <bool kTiled>
int linear(const uint16_t* x, const uint16_t* w, int B, int K, int N, const uint16_t* residual,
           uint16_t* y, uintptr_t stream) {
  pdk::clear_error();
  if (int rc = check_shape(x, w, y, B, K, N)) return rc;
  if (residual)
    return launch<kResidual, kTiled>(x, w, B, K, N, residual, y, nullptr, pdk::as_stream(stream));
  return launch<kPlain, kTiled>(x, w, B, K, N, nullptr, y, nullptr, pdk::as_stream(stream));
}

template <bool kTiled>
int linear_swiglu(const uint16_t* x, const uint16_t* w_gate_up, int B, int K, int M, uint16_t* y,
                  uintptr_t stream) {
  pdk::clear_error();
  if (int rc = check_shape(x, w_gate_up, y, B, K, M)) return rc;
  // The up rows start at tile M / 16 of the tiled copy of [2M][K].
  PDK_REQUIRE(!kTiled || M % 16 == 0, "tiled gate|up weights need M %% 16 == 0 (got %d)", M);
  return launch<kSwiGLU, kTiled>(x, w_gate_up, B, K, M, nullptr, y, nullptr,
                                 pdk::as_stream(stream));
}

template <bool kTiled, bool kAct = false>
int linear_ssq(const uint16_t* x, const uint16_t* w, int B, int K, int N, const uint16_t* residual,
               uint16_t* y, float* ssq, uintptr_t stream) {
  pdk::clear_error();
  if (int rc = check_shape(x, w, y, B, K, N)) return rc;
  PDK_REQUIRE(residual && ssq, "null pointer argument");
  PDK_REQUIRE(N % 16 == 0, "N must be a multiple of 16 (got %d)", N);
  PDK_REQUIRE(!kAct || N % kStepK == 0, "tiled activations need N %% %d == 0 (got %d)", kStepK, N);
  return launch<kResidualSsq, kTiled, kAct>(x, w, B, K, N, residual, y, nullptr, pdk::as_stream(stream),
                                      ssq);
}

template <bool kTiled, bool kAct = false>
int linear_swiglu_rms(const uint16_t* x, const uint16_t* w_gate_up, int B, int K, int M,
                      const float* ssq, int n_ssq, float eps, uint16_t* y, uintptr_t stream) {
  pdk::clear_error();
  if (int rc = check_shape(x, w_gate_up, y, B, K, M)) return rc;
  PDK_REQUIRE(ssq, "null pointer argument");
  PDK_REQUIRE(n_ssq >= 1 && n_ssq * 16 == K, "n_ssq must be K / 16 = %d (got %d)", K / 16, n_ssq);
  PDK_REQUIRE(eps > 0.f, "eps must be positive");
  PDK_REQUIRE(!kTiled || M % 16 == 0, "tiled gate|up weights need M %% 16 == 0 (got %d)", M);
  PDK_REQUIRE(!kAct || M % kStepK == 0, "tiled activations need M %% %d == 0 (got %d)", kStepK, M);
  return launch<kSwiGLURms, kTiled, kAct>(x, w_gate_up, B, K, M, nullptr, y, nullptr,
                                    pdk::as_stream(stream), const_cast<float*>(ssq), n_ssq, eps);
}

template <bool kTiled>
int linear_argmax(const uint16_t* x, const uint16_t* w, int B, int K, int N, uint16_t* logits,
                  uint64_t* keys, int32_t* tokens, uintptr_t stream) {
  pdk::clear_error();
  // y may be null here: check_shape only needs a non-null stand-in.
  if (int rc = check_shape(x, w, keys, B, K, N)) return rc;
  PDK_REQUIRE(tokens, "null pointer argument");
  PDK_REQUIRE(((uintptr_t)keys & 7u) == 0, "keys must be 8-byte aligned");
  hipStream_t st = pdk::as_stream(stream);
  if (int rc = launch<kArgmax, kTiled>(x, w, B, K, N, nullptr, logits, keys, st)) return rc;
  hipLaunchKernelGGL(argmax_finish_kernel, dim3((B + 63) / 64), dim3(64), 0, st, keys, B, tokens);
  return pdk::check_launch("argmax_finish_kernel");
}

template <bool kTiled, bool kAct = false>
int linear_argmax_rms(const uint16_t* x, const uint16_t* w, int B, int K, int N, const float* ssq,
                      int n_ssq, float eps, uint16_t* logits, uint64_t* keys, int32_t* tokens,
                      uintptr_t stream) {
  pdk::clear_error();
  if (int rc = check_shape(x, w, keys, B, K, N)) return rc;
  PDK_REQUIRE(tokens && ssq, "null pointer argument");
  PDK_REQUIRE(((uintptr_t)keys & 7u) == 0, "keys must be 8-byte aligned");
  PDK_REQUIRE(n_ssq >= 1 && n_ssq * 16 == K, "n_ssq must be K / 16 = %d (got %d)", K / 16, n_ssq);
  PDK_REQUIRE(eps > 0.f, "eps must be positive");
  hipStream_t st = pdk::as_stream(stream);
  if (int rc = launch<kArgmaxRms, kTiled, kAct>(x, w, B, K, N, nullptr, logits, keys, st,
                                          const_cast<float*>(ssq), n_ssq, eps))
    return rc;
  hipLaunchKernelGGL(argmax_finish_kernel, dim3((B + 63) / 64), dim3(64), 0, st, keys, B, tokens);
  return pdk::check_launch("argmax_finish_kernel");
}

template <bool kTiled, bool kAct = false>
int linear_splitk_rms(const uint16_t* x, const uint16_t* w, int B, int K, int N, int splits,
                      const float* ssq, int n_ssq, float eps, float* partials, uintptr_t stream) {
  pdk::clear_error();
  if (int rc = check_shape(x, w, partials, B, K, N)) return rc;
  PDK_REQUIRE(ssq, "null pointer argument");
  PDK_REQUIRE(n_ssq >= 1 && n_ssq * 16 == K, "n_ssq must be K / 16 = %d (got %d)", K / 16, n_ssq);
  PDK_REQUIRE(eps > 0.f, "eps must be positive");
  PDK_REQUIRE(splits >= 1 && splits <= 16 && splits <= K / kStepK,
              "splits must be in [1, min(16, K/%d)] (got %d)", kStepK, splits);
  hipStream_t st = pdk::as_stream(stream);
  float* q = const_cast<float*>(ssq);
  // Three column tiles per workgroup where that fills the 256 CUs exactly and
  // four would leave some idle (q|k|v at Llama-3.1-8B: 384 tiles x 2 splits =
  // 256 workgroups, not 192): with tiled activations, 11.59 -> 10.54 us per
  // launch at B = 16 and 10.41 -> 10.39 at B = 4 (32 launches in a HIP graph).
  const int64_t tiles = (N + 15) / 16;
  if (kAct && tiles % 3 == 0 && tiles / 3 * splits <= 256 && tiles / 4 * splits < 256)
    return launch_cols<3, kPartialRms, kTiled, kAct>(x, w, B, K, N, nullptr, nullptr, nullptr, st,
                                                     partials, splits, q, n_ssq, eps);
  if (N >= 1024)
    return launch_cols<4, kPartialRms, kTiled, kAct>(x, w, B, K, N, nullptr, nullptr, nullptr, st,
                                               partials, splits, q, n_ssq, eps);
  return launch_cols<1, kPartialRms, kTiled, kAct>(x, w, B, K, N, nullptr, nullptr, nullptr, st,
                                             partials, splits, q, n_ssq, eps);
}

template <bool kTiled, bool kAct = false>
int linear_splitk_final(const uint16_t* x, const uint16_t* w, int B, int K, int N, int splits,
                        float* partials, uint16_t* residual, float* ssq, int* counters,
                        uintptr_t stream) {
  pdk::clear_error();
  if (int rc = check_shape(x, w, partials, B, K, N)) return rc;
  PDK_REQUIRE(residual && ssq && counters, "null pointer argument");
  PDK_REQUIRE(N % 16 == 0, "N must be a multiple of 16 (got %d)", N);
  PDK_REQUIRE(!kAct || N % kStepK == 0, "tiled activations need N %% %d == 0 (got %d)", kStepK, N);
  PDK_REQUIRE(splits >= 1 && splits <= 16 && splits <= K / kStepK,
              "splits must be in [1, min(16, K/%d)] (got %d)", kStepK, splits);
  hipStream_t st = pdk::as_stream(stream);
  // Two column tiles (with the caller's two K splits at the Llama-8B down
  // projection: 128 x 2 workgroups, 7 steps per wave) rather than four with
  // four splits (28 steps per workgroup: waves 0-3 take 4 and waves 4-7 take 3):
  // the decode step B=4 2.890 -> 2.848 ms, B=16 3.100 -> 3.097 in one process.
  // One tile per workgroup without a split (pdk_linear_ssq, no partials) was
  // faster at B=4 but slower at B=16, where x's loads are as many bytes as
  // the weights, until the tiled weights became step-major; since then it is
  // as fast at B=16 and faster at B=4, and the decode step uses it for the
  // down projection.
  if (N >= 1024)
    return launch_cols<2, kPartialFinal, kTiled, kAct>(x, w, B, K, N, residual, residual, nullptr, st,
                                                 partials, splits, ssq, 0, 0.f, counters);
  return launch_cols<1, kPartialFinal, kTiled, kAct>(x, w, B, K, N, residual, residual, nullptr, st,
                                               partials, splits, ssq, 0, 0.f, counters);
}

template <bool kTiled>
int linear_splitk(const uint16_t* x, const uint16_t* w, int B, int K, int N, int splits,
                  float* partials, uintptr_t stream) {
  pdk::clear_error();
  if (int rc = check_shape(x, w, partials, B, K, N)) return rc;
  PDK_REQUIRE(splits >= 1 && splits <= 16 && splits <= K / kStepK,
              "splits must be in [1, min(16, K/%d)] (got %d)", kStepK, splits);
  // Wide column tiles (fewer re-reads of x) with the K split restoring the
  // workgroup count.
  hipStream_t st = pdk::as_stream(stream);
  if (N >= 1024)
    return launch_cols<4, kPartial, kTiled>(x, w, B, K, N, nullptr, nullptr, nullptr, st,
                                            partials, splits);
  return launch_cols<1, kPartial, kTiled>(x, w, B, K, N, nullptr, nullptr, nullptr, st, partials,
                                          splits);
}

}  // namespace

extern "C" int pdk_linear(const uint16_t* x, const uint16_t* w, int B, int K, int N,
                          const uint16_t* residual, uint16_t* y, uintptr_t stream) {
  return linear<false>(x, w, B, K, N, residual, y, stream);
}

extern "C" int pdk_linear_swiglu(const uint16_t* x, const uint16_t* w_gate_up, int B, int K, int M,
                                 uint16_t* y, uintptr_t stream) {
  return linear_swiglu<false>(x, w_gate_up, B, K, M, y, stream);
}

extern "C" int pdk_linear_argmax(const uint16_t* x, const uint16_t* w, int B, int K, int N,
                                 uint16_t* logits, uint64_t* keys, int32_t* tokens,
                                 uintptr_t stream) {
  return linear_argmax<false>(x, w, B, K, N, logits, keys, tokens, stream);
}

extern "C" int pdk_linear_splitk(const uint16_t* x, const uint16_t* w, int B, int K, int N,
                                 int splits, float* partials, uintptr_t stream) {
  return linear_splitk<false>(x, w, B, K, N, splits, partials, stream);
}

extern "C" int64_t pdk_weight_tiled_elems(int N, int K) {
  if (N < 1 || K < kStepK || K % kStepK != 0) return 0;
  return (int64_t)((N + 15) / 16) * 16 * K;
}

extern "C" int pdk_weight_tile(const uint16_t* w, int N, int K, uint16_t* wt, uintptr_t stream) {
  pdk::clear_error();
  PDK_REQUIRE(w && wt, "null pointer argument");
  PDK_REQUIRE(N >= 1, "N must be positive (got %d)", N);
  PDK_REQUIRE(K >= kStepK && K % kStepK == 0, "K must be a positive multiple of %d (got %d)",
              kStepK, K);
  PDK_REQUIRE(pdk::aligned16(w) && pdk::aligned16(wt), "w and wt must be 16-byte aligned");
  const int64_t groups = pdk_weight_tiled_elems(N, K) / 8;
  const int64_t blocks = (groups + 255) / 256;
  PDK_REQUIRE(blocks < (1ll << 31), "weight too large");
  hipLaunchKernelGGL(weight_tile_kernel, dim3((unsigned)blocks), dim3(256), 0,
                     pdk::as_stream(stream), w, N, K, wt, groups);
  return pdk::check_launch("weight_tile_kernel");
}

extern "C" int pdk_linear_tiled(const uint16_t* x, const uint16_t* wt, int B, int K, int N,
                                const uint16_t* residual, uint16_t* y, uintptr_t stream) {
  return linear<true>(x, wt, B, K, N, residual, y, stream);
}

extern "C" int pdk_linear_swiglu_tiled(const uint16_t* x, const uint16_t* wt_gate_up, int B,
                                       int K, int M, uint16_t* y, uintptr_t stream) {
  return linear_swiglu<true>(x, wt_gate_up, B, K, M, y, stream);
}

extern "C" int pdk_linear_argmax_tiled(const uint16_t* x, const uint16_t* wt, int B, int K, int N,
                                       uint16_t* logits, uint64_t* keys, int32_t* tokens,
                                       uintptr_t stream) {
  return linear_argmax<true>(x, wt, B, K, N, logits, keys, tokens, stream);
}

extern "C" int pdk_linear_ssq(const uint16_t* x, const uint16_t* w, int B, int K, int N,
                              const uint16_t* residual, uint16_t* y, float* ssq, uintptr_t stream) {
  return linear_ssq<false>(x, w, B, K, N, residual, y, ssq, stream);
}

extern "C" int pdk_linear_ssq_tiled(const uint16_t* x, const uint16_t* wt, int B, int K, int N,
                                    const uint16_t* residual, uint16_t* y, float* ssq,
                                    uintptr_t stream) {
  return linear_ssq<true>(x, wt, B, K, N, residual, y, ssq, stream);
}

extern "C" int pdk_linear_swiglu_rms(const uint16_t* x, const uint16_t* w_gate_up, int B, int K,
                                     int M, const float* ssq, int n_ssq, float eps, uint16_t* y,
                                     uintptr_t stream) {
  return linear_swiglu_rms<false>(x, w_gate_up, B, K, M, ssq, n_ssq, eps, y, stream);
}

extern "C" int pdk_linear_swiglu_rms_tiled(const uint16_t* x, const uint16_t* wt_gate_up, int B,
                                           int K, int M, const float* ssq, int n_ssq, float eps,
                                           uint16_t* y, uintptr_t stream) {
  return linear_swiglu_rms<true>(x, wt_gate_up, B, K, M, ssq, n_ssq, eps, y, stream);
}

extern "C" int pdk_linear_argmax_rms(const uint16_t* x, const uint16_t* w, int B, int K, int N,
                                     const float* ssq, int n_ssq, float eps, uint16_t* logits,
                                     uint64_t* keys, int32_t* tokens, uintptr_t stream) {
  return linear_argmax_rms<false>(x, w, B, K, N, ssq, n_ssq, eps, logits, keys, tokens, stream);
}

extern "C" int pdk_linear_argmax_rms_tiled(const uint16_t* x, const uint16_t* wt, int B, int K,
                                           int N, const float* ssq, int n_ssq, float eps,
                                           uint16_t* logits, uint64_t* keys, int32_t* tokens,
                                           uintptr_t stream) {
  return linear_argmax_rms<true>(x, wt, B, K, N, ssq, n_ssq, eps, logits, keys, tokens, stream);
}

extern "C" int pdk_linear_splitk_rms(const uint16_t* x, const uint16_t* w, int B, int K, int N,
                                     int splits, const float* ssq, int n_ssq, float eps,
                                     float* partials, uintptr_t stream) {
  return linear_splitk_rms<false>(x, w, B, K, N, splits, ssq, n_ssq, eps, partials, stream);
}

extern "C" int pdk_linear_splitk_rms_tiled(const uint16_t* x, const uint16_t* wt, int B, int K,
                                           int N, int splits, const float* ssq, int n_ssq,
                                           float eps, float* partials, uintptr_t stream) {
  return linear_splitk_rms<true>(x, wt, B, K, N, splits, ssq, n_ssq, eps, partials, stream);
}

extern "C" int pdk_linear_splitk_final(const uint16_t* x, const uint16_t* w, int B, int K, int N,
                                       int splits, float* partials, uint16_t* residual,
                                       float* ssq, int* counters, uintptr_t stream) {
  return linear_splitk_final<false>(x, w, B, K, N, splits, partials, residual, ssq, counters,
                                    stream);
}

extern "C" int pdk_linear_splitk_final_tiled(const uint16_t* x, const uint16_t* wt, int B, int K,
                                             int N, int splits, float* partials,
                                             uint16_t* residual, float* ssq, int* counters,
                                             uintptr_t stream) {
  return linear_splitk_final<true>(x, wt, B, K, N, splits, partials, residual, ssq, counters,
                                   stream);
}

extern "C" int pdk_linear_splitk_tiled(const uint16_t* x, const uint16_t* wt, int B, int K, int N,
                                       int splits, float* partials, uintptr_t stream) {
  return linear_splitk<true>(x, wt, B, K, N, splits, partials, stream);
}

// ---- tiled activations (pdk::act_at) with tiled weights ---------------------
extern "C" int pdk_linear_ssq_xt(const uint16_t* x, const uint16_t* wt, int B, int K, int N,
                                 const uint16_t* residual, uint16_t* y, float* ssq,
                                 uintptr_t stream) {
  return linear_ssq<true, true>(x, wt, B, K, N, residual, y, ssq, stream);
}

extern "C" int pdk_linear_swiglu_rms_xt(const uint16_t* x, const uint16_t* wt_gate_up, int B,
                                        int K, int M, const float* ssq, int n_ssq, float eps,
                                        uint16_t* y, uintptr_t stream) {
  return linear_swiglu_rms<true, true>(x, wt_gate_up, B, K, M, ssq, n_ssq, eps, y, stream);
}

extern "C" int pdk_linear_argmax_rms_xt(const uint16_t* x, const uint16_t* wt, int B, int K,
                                        int N, const float* ssq, int n_ssq, float eps,
                                        uint16_t* logits, uint64_t* keys, int32_t* tokens,
                                        uintptr_t stream) {
  return linear_argmax_rms<true, true>(x, wt, B, K, N, ssq, n_ssq, eps, logits, keys, tokens,
                                       stream);
}

extern "C" int pdk_linear_splitk_rms_xt(const uint16_t* x, const uint16_t* wt, int B, int K,
                                        int N, int splits, const float* ssq, int n_ssq,
                                        float eps, float* partials, uintptr_t stream) {
  return linear_splitk_rms<true, true>(x, wt, B, K, N, splits, ssq, n_ssq, eps, partials, stream);
}

extern "C" int pdk_linear_splitk_final_xt(const uint16_t* x, const uint16_t* wt, int B, int K,
                                          int N, int splits, float* partials,
                                          uint16_t* residual, float* ssq, int* counters,
                                          uintptr_t stream) {
  return linear_splitk_final<true, true>(x, wt, B, K, N, splits, partials, residual, ssq,
                                         counters, stream);
}
