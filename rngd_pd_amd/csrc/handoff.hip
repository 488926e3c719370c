// Prefill->decode KV handoff kernels for gfx950: pack (prefill KV -> transport
// frame), scatter (frame -> paged decode cache) and gather (its inverse).
//
// All three are pure permutations of bf16 bits, bound by HBM bandwidth. Each
// wavefront owns a 64-token x 64-dim tile of one (request, layer, head); a lane
// owns an 8x8 sub-tile, moves it with 16-byte loads and stores, and transposes
// it in registers where the two layouts disagree (K in pack; K and V in
// scatter/gather), so no LDS round trip is needed. Lane (ti, di) = (lane>>3,
// lane&7) holds tokens 8ti..8ti+7 and dims 8di..8di+7 of the tile: for every
// load and store instruction the 64 lanes touch eight full 128-byte lines.
//
// Requests are batched through the kernel argument block: their tiles are laid
// end to end over grid.x, so a launch moves up to PDK_MAX_BATCH requests of any
// mix of lengths without a device-side descriptor buffer or an allocation.
//
// Cache policy. A launch that moves more bytes than the last-level cache holds
// (kStreamBytes) uses streaming (non-temporal) accesses on its read-once side:
// pack streams its prefill reads and whole-line frame writes, gather its frame
// writes, scatter its frame reads. Scatter's cache-block stores stay ordinary:
// on 8 Llama-3.1-8B requests (452 MiB scattered right after their pack) they
// take the scatter from 95 us with streaming stores to 78 us, and the pack
// that follows is no slower for it. Ordinary stores for pack's transposed
// tiles (the zero tails kept streaming) make the pack itself faster, 142 ->
// 123 us when packs run back to back, but the write-back they defer lands in
// whatever runs next: right before the scatter, pack takes 138 us and the
// scatter 90 instead of 78, so the pair is slower (228 against 224 us) and
// pack keeps streaming stores. A smaller launch keeps ordinary accesses, so a
// just-written frame can still be in the cache when its consumer (a copy or
// the scatter) reads it: one 512-token request packs in 22 us that way and in
// 28 us streaming.

#include <algorithm>

#include "pdk_common.h"

namespace {

using pdk::v8;

constexpr int kWaves = 4;        // wavefronts per workgroup
constexpr int kTileT = 64;       // tokens per wavefront tile
constexpr int kTileD = 64;       // dims per wavefront tile
constexpr int64_t kStreamBytes = 256ll << 20;   // the MI355X last-level (Infinity) cache

// Requests of a batched launch are laid end to end over grid.x: request r owns
// wavefront tiles off[r] .. off[r+1]-1, so a launch holds only tiles with
// work, however different the requests' lengths are. Pack lays out the
// tiles that move tokens first (off[]), for all requests, and the zero-fill
// chunks of the frames' tails after them (zoff[], counted from off[n_req]): on
// the 8-request Llama-3.1-8B batch that is 2-5 us faster (of about 145) than
// each request's zero chunks right after its own tiles.
struct PackArgs {
  pdk_pack_req req[PDK_MAX_BATCH];
  int64_t off[PDK_MAX_BATCH + 1];
  int64_t zoff[PDK_MAX_BATCH + 1];
  int32_t nT[PDK_MAX_BATCH];     // 64-token tiles of request r holding valid tokens
  int32_t nvalid[PDK_MAX_BATCH]; // its units that move tokens
  int32_t Pz[PDK_MAX_BATCH];     // first column of its all-zero tail: min(64 nT, S)
  int32_t nZ[PDK_MAX_BATCH];     // zero-fill chunks per (layer, head)
  uint32_t magic[PDK_MAX_BATCH]; // ceil(2^32 / ((S - Pz) / 8)): row of a K tail group
  int n_req, S, Hkv, D, nD;
};

// 16-byte stores per lane per zero chunk: 2 (2 KiB per wavefront, 8 KiB per
// workgroup). On the 8-request Llama-3.1-8B batch the 311 MB of zero tails
// take 48 us this way (6.5 TB/s) against 56 us with 16 stores per lane; one
// store per lane was slower again (160 us for the whole pack against 142).
constexpr int kZeroInstr = 2;
constexpr int kZeroElems = kZeroInstr * 64 * 8;   // 1024 bf16 = 2 KiB per chunk

// The all-zero tail of one (layer, head) of a frame: K rows (h, d) columns
// [Pz, S) and the V block rows t in [Pz, S), flattened into 2 * D * (S - Pz)
// elements (the K tails first, row by row, then the contiguous V tail). Each
// store instruction of a chunk writes 1 KiB of consecutive elements of that
// space: whole K-row runs and the V tail linearly, instead of the 128-byte
// pieces a transposed tile would write.
template <bool kStream>
__device__ __forceinline__ void pack_zero_chunk(const PackArgs& a, int r, uint32_t z, int lane) {
  const pdk_pack_req& R = a.req[r];
  const int nZ = a.nZ[r];
  const int zc = (int)(z % (uint32_t)nZ);
  z /= (uint32_t)nZ;
  const int h = (int)(z % (uint32_t)a.Hkv);
  const int l = (int)(z / (uint32_t)a.Hkv);
  const int S = a.S, D = a.D, Pz = a.Pz[r];
  const uint32_t g_row = (uint32_t)(S - Pz) >> 3;   // 8-element groups per K tail row
  const uint32_t gK = (uint32_t)D * g_row;         // groups of the K tails (= of the V tail)
  const int64_t F = (int64_t)a.Hkv * D * S;
  uint16_t* fk = R.frame + (int64_t)(2 * l) * F;
  uint16_t* fv = fk + F + ((int64_t)h * S + Pz) * D;
  const v8 zero = pdk::zero8();
#pragma unroll
  for (int i = 0; i < kZeroInstr; ++i) {
    const uint32_t g = (uint32_t)zc * (kZeroElems / 8) + i * 64 + lane;
    if (g < gK) {
      const uint32_t row = __umulhi(g, a.magic[r]);
      const uint32_t col = Pz + (g - row * g_row) * 8;
      pdk::st16_as<kStream>(fk + ((int64_t)h * D + row) * S + col, zero);
    } else if (g < 2 * gK) {
      pdk::st16_as<kStream>(fv + (int64_t)(g - gK) * 8, zero);
    }
  }
}

// Request of wavefront tile `unit` (uniform across the wavefront).
__device__ __forceinline__ int request_of(const int64_t* off, int n_req, int64_t unit) {
  int r = 0;
  while (r + 1 < n_req && unit >= off[r + 1]) ++r;
  return r;
}

__device__ __forceinline__ int64_t wave_unit() {
  return (int64_t)blockIdx.x * kWaves + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
}

// Frame layout per request: [L][2][F], F = Hkv*D*S; K frame [Hkv][D][S],
// V frame [Hkv][S][D]; columns t >= P are zero (engines/prefill_full.py:378-379).
// kNarrow: some request of the launch is narrow (its V rows past P are not
// stored). Without it every V store is unconditional: dropping the per-lane
// test took the 8-request Llama-3.1-8B batch of full-width frames from
// 146.0-146.3 to 141.6-142.1 us (both libraries in one process).
template <bool kStream, bool kNarrow>
__global__ __launch_bounds__(256) void pack_kernel(const PackArgs a) {
  const int64_t unit = wave_unit();
  const int64_t n_moving = a.off[a.n_req];
  const int lane = threadIdx.x & 63;
  if (unit >= n_moving) {                     // uniform across the wavefront
    const int64_t z = unit - n_moving;
    if (z >= a.zoff[a.n_req]) return;
    const int rz = request_of(a.zoff, a.n_req, z);
    pack_zero_chunk<kStream>(a, rz, (uint32_t)(z - a.zoff[rz]), lane);
    return;
  }
  const int r = request_of(a.off, a.n_req, unit);
  const pdk_pack_req& R = a.req[r];
  uint32_t u = (uint32_t)(unit - a.off[r]);   // units of one request fit 32 bits
  const int dt = (int)(u % (uint32_t)a.nD); u /= (uint32_t)a.nD;
  const int tt = (int)(u % (uint32_t)a.nT[r]); u /= (uint32_t)a.nT[r];
  const int h = (int)(u % (uint32_t)a.Hkv); u /= (uint32_t)a.Hkv;
  const int l = (int)u;
  const int ti = lane >> 3, di = lane & 7;
  const int S = a.S, D = a.D, P = R.P;
  const int t0 = tt * kTileT + ti * 8;
  const int d0 = dt * kTileD + di * 8;
  const int64_t F = (int64_t)a.Hkv * D * S;

  const uint16_t* sk = R.src_k + (int64_t)l * R.layer_stride + (int64_t)h * D + d0;
  const uint16_t* sv = R.src_v + (int64_t)l * R.layer_stride + (int64_t)h * D + d0;
  v8 kin[8], vin[8];
#pragma unroll
  for (int r = 0; r < 8; ++r) {
    const int t = t0 + r;
    if (t < P) {
      kin[r] = pdk::ld16_as<kStream>(sk + (int64_t)t * R.tok_stride);
      vin[r] = pdk::ld16_as<kStream>(sv + (int64_t)t * R.tok_stride);
    } else {
      kin[r] = pdk::zero8();
      vin[r] = pdk::zero8();
    }
  }
  if (t0 >= S) return;           // S % 8 == 0: the lane's 8 tokens are all in or all out
  // Narrow frames still get whole 64-token tiles of K (zeros past P): a K row
  // then ends on a 128-byte line, which keeps the stores whole lines when the
  // frame is in host memory. V rows past P are left unwritten.
  const bool narrow = kNarrow && (R.flags & PDK_PACK_NARROW) != 0;
  uint16_t* fk = R.frame + (int64_t)(2 * l) * F;
  uint16_t* fv = fk + F;
#pragma unroll
  for (int r = 0; r < 8; ++r)
    if (!narrow || t0 + r < P) pdk::st16_as<kStream>(fv + ((int64_t)h * S + t0 + r) * D + d0, vin[r]);
  v8 kout[8];
  pdk::transpose8x8(kin, kout);  // kout[c]: dim d0+c, tokens t0..t0+7
#pragma unroll
  for (int c = 0; c < 8; ++c)
    pdk::st16_as<kStream>(fk + ((int64_t)h * D + d0 + c) * S + t0, kout[c]);
}

struct ScatterArgs {
  pdk_scatter_req req[PDK_MAX_BATCH];
  int64_t off[PDK_MAX_BATCH + 1];
  int32_t nC[PDK_MAX_BATCH];     // 64-token chunks of request r
  uint16_t* cache_k;
  uint16_t* cache_v;
  int64_t cache_ls;              // elements between layers of the cache
  int32_t* skipped;              // or null: += block ids outside [0, num_blocks) not written
  int n_req, num_blocks, S, Hkv, D, nD;
};

// Frame -> paged cache. K cache block [Hkv][16 x D] in the tiled token order of
// pdk::k_unit (8 dims of one token per 16-byte unit), V cache block [Hkv][D][16]
// (dim rows): both need an 8x8 transpose from the frame.
//
// A lane's 8 transposed K rows are 8 consecutive tokens, but each 128-byte line
// of the tiled K block holds tokens from two lanes, and a V dim row (32 bytes)
// holds a quarter line. Stored directly, every instruction would write 16-byte
// pieces of 32 lines. So each wavefront stages its tile through LDS (8 KiB):
// lanes write their vectors at their destination positions, then read them
// back in destination order, and each store instruction writes 1 KiB of one
// block contiguously. An XOR swizzle of the 16-byte slot index keeps both the
// writes and the reads free of bank conflicts.
__device__ __forceinline__ int swizzle_k(int i) { return i ^ ((i >> 3) & 7); }
__device__ __forceinline__ int swizzle_v(int i) { return i ^ ((i >> 4) & 7); }

template <bool kStream>
__global__ __launch_bounds__(256) void scatter_kernel(const ScatterArgs a) {
  __shared__ uint4 stage[kWaves][512];
  const int64_t unit = wave_unit();
  if (unit >= a.off[a.n_req]) return;           // uniform across the wavefront
  const int r = request_of(a.off, a.n_req, unit);
  const pdk_scatter_req& R = a.req[r];
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  uint32_t u = (uint32_t)(unit - a.off[r]);
  const int dt = (int)(u % (uint32_t)a.nD); u /= (uint32_t)a.nD;
  const int ct = (int)(u % (uint32_t)a.nC[r]); u /= (uint32_t)a.nC[r];
  const int h = (int)(u % (uint32_t)a.Hkv); u /= (uint32_t)a.Hkv;
  const int l = (int)u;
  const int ti = lane >> 3, di = lane & 7;
  const int S = a.S, D = a.D, P = R.P;           // P >= 1: a request with P = 0 has no tiles
  const int rP = (P + 15) & ~15;                 // tokens of the request's blocks, <= S
  const int t0 = ct * kTileT + ti * 8;
  const int tl = min(t0, rP - 8);                // lanes past the last block load in bounds
  const int d0 = dt * kTileD + di * 8;
  const int64_t F = (int64_t)a.Hkv * D * S;
  const uint16_t* fk = R.frame + (int64_t)(2 * l) * F;
  const uint16_t* fv = fk + F;

  // The frame loads are unconditional and tokens >= P are zeroed afterwards:
  // a load whose register a divergent branch later overwrites with zero makes
  // the compiler wait for it before the next load.
  v8 kin[8], vin[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    // K frame row d0+i holds tokens contiguously; V frame row tl+i holds dims.
    kin[i] = pdk::ld16_as<kStream>(fk + ((int64_t)h * D + d0 + i) * S + tl);
    vin[i] = pdk::ld16_as<kStream>(fv + ((int64_t)h * S + tl + i) * D + d0);
  }
  // Block ids of the chunk's four blocks: uniform scalar loads from clamped,
  // in-bounds indices (no branch, so nothing waits on them before the stores);
  // blocks past the request's last one are dropped afterwards.
  const int nblk = min(rP >> 4, R.n_table);
  const int j0 = ct * (kTileT / 16);
  int blk[4];
  int bad = 0;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int id = R.table[min(j0 + q, nblk - 1)];
    blk[q] = (j0 + q < nblk && id >= 0 && id < a.num_blocks) ? id : -1;
    bad += j0 + q < nblk && blk[q] < 0;
  }
  // Invalid ids are skipped (nothing is written for their tokens); with a
  // counter, the first unit of each chunk (layer 0, head 0, dims 0..63)
  // reports them, so each (request, block) counts once per launch.
  if (a.skipped && bad && l == 0 && h == 0 && dt == 0 && lane == 0)
    atomicAdd(a.skipped, bad);
  if (t0 + 8 > P) {              // a narrow frame leaves tokens >= P unwritten
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      pdk::mask_tail(kin[i], t0, P);
      if (t0 + i >= P) vin[i] = pdk::zero8();
    }
  }
  v8 kout[8], vout[8];
  pdk::transpose8x8(kin, kout);  // kout[c]: token t0+c, dims d0..d0+7
  pdk::transpose8x8(vin, vout);  // vout[c]: dim d0+c, tokens t0..t0+7
  // Materialise vout here. Computed later (next to its use, after the K
  // stores), its first input would need a wait that also covers every K
  // store issued meanwhile, as loads and stores share one counter.
#pragma unroll
  for (int c = 0; c < 8; ++c)
    asm volatile("" ::"v"(vout[c].w[0]), "v"(vout[c].w[1]), "v"(vout[c].w[2]), "v"(vout[c].w[3]));
  uint4* st = stage[wave];
  const int q_lane = ti >> 1;                    // the lane's block within the chunk

  // K: run (q, t) of 64 units = tile t of block q for this wavefront's two
  // 32-dim groups; inside it unit di*8 + j8 (pdk::k_unit with s, g from di).
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    const int i = (q_lane * 2 + (c >> 2)) * 64 + di * 8 + (ti & 1) * 4 + (c & 3);
    st[swizzle_k(i)] = make_uint4(kout[c].w[0], kout[c].w[1], kout[c].w[2], kout[c].w[3]);
  }
  const int nS = D >> 5;
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const uint4 x = st[swizzle_k(k * 64 + lane)];
    const int b = blk[k >> 1];
    if (b >= 0) {
      uint16_t* ck = a.cache_k + (int64_t)l * a.cache_ls + ((int64_t)b * a.Hkv + h) * 16 * D;
      pdk::st16(ck + ((int64_t)((k & 1) * nS + 2 * dt) * 32 + lane) * 8,
                            v8{{x.x, x.y, x.z, x.w}});
    }
  }
  // V: block q's dims d0 of this wavefront are 128 contiguous units (2 per dim
  // row); lane vector c is unit (8di + c)*2 + (ti & 1).
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    const int i = q_lane * 128 + (8 * di + c) * 2 + (ti & 1);
    st[swizzle_v(i)] = make_uint4(vout[c].w[0], vout[c].w[1], vout[c].w[2], vout[c].w[3]);
  }
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const uint4 x = st[swizzle_v(k * 64 + lane)];
    const int b = blk[k >> 1];
    if (b >= 0) {
      uint16_t* cv = a.cache_v + (int64_t)l * a.cache_ls + ((int64_t)b * a.Hkv + h) * D * 16;
      pdk::st16(cv + ((int64_t)dt * 128 + (k & 1) * 64 + lane) * 8,
                            v8{{x.x, x.y, x.z, x.w}});
    }
  }
}

struct GatherArgs {
  const uint16_t* cache_k;
  const uint16_t* cache_v;
  const int32_t* table;
  uint16_t* frame;
  int64_t cache_ls;
  int num_blocks, n_table, P, S, Hkv, D, nC, nD;
  int64_t units;
};

// Paged cache -> S-wide frame (zero for t >= P).
template <bool kStream>
__global__ __launch_bounds__(256) void gather_kernel(const GatherArgs a) {
  const int64_t unit = (int64_t)blockIdx.x * kWaves + (threadIdx.x >> 6);
  if (unit >= a.units) return;
  const int lane = threadIdx.x & 63;
  uint32_t u = (uint32_t)unit;
  const int dt = (int)(u % (uint32_t)a.nD); u /= (uint32_t)a.nD;
  const int ct = (int)(u % (uint32_t)a.nC); u /= (uint32_t)a.nC;
  const int h = (int)(u % (uint32_t)a.Hkv); u /= (uint32_t)a.Hkv;
  const int l = (int)u;
  const int ti = lane >> 3, di = lane & 7;
  const int S = a.S, D = a.D, P = a.P;
  const int t0 = ct * kTileT + ti * 8;
  if (t0 >= S) return;
  const int d0 = dt * kTileD + di * 8;
  const int64_t F = (int64_t)a.Hkv * D * S;
  uint16_t* fk = a.frame + (int64_t)(2 * l) * F;
  uint16_t* fv = fk + F;

  int blk = -1;
  if (t0 < P && (t0 >> 4) < a.n_table) blk = a.table[t0 >> 4];
  const bool ok = blk >= 0 && blk < a.num_blocks;
  const int slot0 = t0 & 15;
  const uint16_t* ck = a.cache_k + (int64_t)l * a.cache_ls + ((int64_t)(ok ? blk : 0) * a.Hkv + h) * 16 * D;
  const uint16_t* cv = a.cache_v + (int64_t)l * a.cache_ls + ((int64_t)(ok ? blk : 0) * a.Hkv + h) * D * 16;
  // Loads are unconditional from in-bounds addresses (block 0 stands in for a
  // missing block) and masked afterwards, so they are all in flight at once.
  v8 kin[8], vin[8];
#pragma unroll
  for (int r = 0; r < 8; ++r) {
    kin[r] = pdk::ld16(ck + (int64_t)pdk::k_unit(slot0 + r, d0, D) * 8);
    vin[r] = pdk::ld16(cv + (int64_t)(d0 + r) * 16 + slot0);
  }
#pragma unroll
  for (int r = 0; r < 8; ++r) {
    if (!ok || t0 + r >= P) kin[r] = pdk::zero8();
    if (!ok) vin[r] = pdk::zero8();
    else if (t0 + 8 > P) pdk::mask_tail(vin[r], t0, P);
  }
  v8 kout[8], vout[8];
  pdk::transpose8x8(kin, kout);  // kout[c]: dim d0+c, tokens t0..t0+7
  pdk::transpose8x8(vin, vout);  // vout[c]: token t0+c, dims d0..d0+7
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    pdk::st16_as<kStream>(fk + ((int64_t)h * D + d0 + c) * S + t0, kout[c]);
    pdk::st16_as<kStream>(fv + ((int64_t)h * S + t0 + c) * D + d0, vout[c]);
  }
}

int check_common(int n_layers, int S, int Hkv, int D) {
  PDK_REQUIRE(n_layers >= 1, "n_layers must be >= 1 (got %d)", n_layers);
  PDK_REQUIRE(Hkv >= 1, "n_kv_heads must be >= 1 (got %d)", Hkv);
  if (D < 64 || D % 64 != 0 || D > 1024) {
    pdk::set_error("head_dim must be a multiple of 64 in [64, 1024] (got %d)", D);
    return PDK_ENOTSUP;
  }
  PDK_REQUIRE(S >= 16 && S % 16 == 0, "S must be a positive multiple of 16 (got %d)", S);
  return PDK_OK;
}

int64_t grid_x(int64_t units) { return (units + kWaves - 1) / kWaves; }

}  // namespace

extern "C" int pdk_pack_kv_batch(const pdk_pack_req* reqs, int n_reqs, int n_layers,
                                 int S, int n_kv_heads, int head_dim, uintptr_t stream) {
  pdk::clear_error();
  int rc = check_common(n_layers, S, n_kv_heads, head_dim);
  if (rc) return rc;
  PDK_REQUIRE(reqs != nullptr, "reqs is null");
  PDK_REQUIRE(n_reqs >= 1 && n_reqs <= PDK_MAX_BATCH, "n_reqs must be in [1, %d] (got %d)",
              PDK_MAX_BATCH, n_reqs);
  // The zero-fill chunks find a K row by a multiply-high by ceil(2^32 / g),
  // exact while (row groups) * g^2 < 2^32: S <= 32768 keeps it so.
  PDK_REQUIRE(S <= 32768, "S must be <= 32768 (got %d)", S);
  PackArgs a{};
  for (int i = 0; i < n_reqs; ++i) {
    const pdk_pack_req& r = reqs[i];
    PDK_REQUIRE(r.frame && pdk::aligned16(r.frame), "request %d: frame null or not 16-byte aligned", i);
    PDK_REQUIRE(r.P >= 0 && r.P <= S, "request %d: P=%d outside [0, S=%d]", i, r.P, S);
    PDK_REQUIRE((r.flags & ~PDK_PACK_NARROW) == 0, "request %d: unknown flags 0x%x", i, r.flags);
    if (r.P > 0) {
      PDK_REQUIRE(r.src_k && r.src_v && pdk::aligned16(r.src_k) && pdk::aligned16(r.src_v),
                  "request %d: src_k/src_v null or not 16-byte aligned", i);
      PDK_REQUIRE(r.tok_stride >= (int64_t)n_kv_heads * head_dim && r.tok_stride % 8 == 0,
                  "request %d: tok_stride=%lld must be a multiple of 8 and >= Hkv*D", i,
                  (long long)r.tok_stride);
      PDK_REQUIRE(r.layer_stride % 8 == 0 && (n_layers == 1 || r.layer_stride != 0),
                  "request %d: layer_stride=%lld must be a multiple of 8", i,
                  (long long)r.layer_stride);
    }
    a.req[i] = r;
  }
  a.n_req = n_reqs;
  a.S = S;
  a.Hkv = n_kv_heads;
  a.D = head_dim;
  a.nD = head_dim / kTileD;
  a.off[0] = 0;
  a.zoff[0] = 0;
  for (int i = 0; i < n_reqs; ++i) {
    // Tiles that hold valid tokens move them (and zero their own columns >= P);
    // a full-width frame's tail past them is zero-filled by separate chunks.
    const int P = a.req[i].P;
    a.nT[i] = (P + kTileT - 1) / kTileT;
    a.nvalid[i] = n_layers * n_kv_heads * a.nT[i] * a.nD;
    a.Pz[i] = std::min(a.nT[i] * kTileT, S);
    const bool narrow = (a.req[i].flags & PDK_PACK_NARROW) != 0;
    const int64_t tail = (int64_t)2 * head_dim * (S - a.Pz[i]);
    a.nZ[i] = narrow ? 0 : (int)((tail + kZeroElems - 1) / kZeroElems);
    const uint32_t g_row = (uint32_t)(S - a.Pz[i]) / 8;
    a.magic[i] = g_row ? (uint32_t)((((uint64_t)1 << 32) + g_row - 1) / g_row) : 0;
    a.off[i + 1] = a.off[i] + a.nvalid[i];
    a.zoff[i + 1] = a.zoff[i] + (int64_t)n_layers * n_kv_heads * a.nZ[i];
  }
  const int64_t units = a.off[n_reqs] + a.zoff[n_reqs];
  if (units == 0) return PDK_OK;
  const int64_t gx = grid_x(units);
  PDK_REQUIRE(gx < (1ll << 31), "launch too large");
  // Bytes the launch moves: valid tokens read, frame columns written.
  int64_t moved = 0;
  bool any_narrow = false;
  for (int i = 0; i < n_reqs; ++i) {
    const bool narrow = (a.req[i].flags & PDK_PACK_NARROW) != 0;
    any_narrow = any_narrow || narrow;
    moved += (int64_t)n_layers * 2 * n_kv_heads * head_dim * 2 *
             (a.req[i].P + (int64_t)(narrow ? a.req[i].P : S));
  }
  const bool stream_io = moved > kStreamBytes;
  const auto kern = stream_io ? (any_narrow ? pack_kernel<true, true> : pack_kernel<true, false>)
                              : (any_narrow ? pack_kernel<false, true> : pack_kernel<false, false>);
  hipLaunchKernelGGL(kern, dim3((unsigned)gx), dim3(256), 0, pdk::as_stream(stream), a);
  return pdk::check_launch("pack_kernel");
}

extern "C" int pdk_pack_kv(const uint16_t* src_k, const uint16_t* src_v, int64_t layer_stride,
                           int64_t tok_stride, int n_layers, int P, int S, int n_kv_heads,
                           int head_dim, uint16_t* frame, uintptr_t stream) {
  pdk_pack_req r{src_k, src_v, frame, layer_stride, tok_stride, P, 0};
  return pdk_pack_kv_batch(&r, 1, n_layers, S, n_kv_heads, head_dim, stream);
}

namespace {
int scatter_batch(const pdk_scatter_req* reqs, int n_reqs, int n_layers, int S, int n_kv_heads,
                  int head_dim, uint16_t* cache_k, uint16_t* cache_v, int64_t cache_layer_stride,
                  int num_blocks, int32_t* skipped, uintptr_t stream) {
  pdk::clear_error();
  int rc = check_common(n_layers, S, n_kv_heads, head_dim);
  if (rc) return rc;
  PDK_REQUIRE(reqs != nullptr, "reqs is null");
  PDK_REQUIRE(n_reqs >= 1 && n_reqs <= PDK_MAX_BATCH, "n_reqs must be in [1, %d] (got %d)",
              PDK_MAX_BATCH, n_reqs);
  PDK_REQUIRE(cache_k && cache_v && pdk::aligned16(cache_k) && pdk::aligned16(cache_v),
              "cache_k/cache_v null or not 16-byte aligned");
  PDK_REQUIRE(num_blocks >= 1, "num_blocks must be >= 1");
  const int64_t per_layer = (int64_t)num_blocks * n_kv_heads * 16 * head_dim;
  PDK_REQUIRE(n_layers == 1 || cache_layer_stride >= per_layer,
              "cache_layer_stride=%lld smaller than one layer (%lld)",
              (long long)cache_layer_stride, (long long)per_layer);
  PDK_REQUIRE(cache_layer_stride % 8 == 0, "cache_layer_stride must be a multiple of 8");
  ScatterArgs a{};
  a.skipped = skipped;
  int max_p = 0;
  for (int i = 0; i < n_reqs; ++i) {
    const pdk_scatter_req& r = reqs[i];
    PDK_REQUIRE(r.P >= 0 && r.P <= S, "request %d: P=%d outside [0, S=%d]", i, r.P, S);
    if (r.P > 0) {
      PDK_REQUIRE(r.frame && pdk::aligned16(r.frame), "request %d: frame null or not 16-byte aligned", i);
      PDK_REQUIRE(r.table != nullptr, "request %d: block table is null", i);
      PDK_REQUIRE(r.n_table >= (r.P + 15) / 16, "request %d: table has %d blocks, P=%d needs %d",
                  i, r.n_table, r.P, (r.P + 15) / 16);
    }
    a.req[i] = r;
    if (r.P > max_p) max_p = r.P;
  }
  if (max_p == 0) return PDK_OK;
  a.cache_k = cache_k;
  a.cache_v = cache_v;
  a.cache_ls = cache_layer_stride;
  a.num_blocks = num_blocks;
  a.n_req = n_reqs;
  a.S = S;
  a.Hkv = n_kv_heads;
  a.D = head_dim;
  a.nD = head_dim / kTileD;
  a.off[0] = 0;
  for (int i = 0; i < n_reqs; ++i) {
    a.nC[i] = (a.req[i].P + kTileT - 1) / kTileT;
    a.off[i + 1] = a.off[i] + (int64_t)n_layers * n_kv_heads * a.nC[i] * a.nD;
  }
  const int64_t gx = grid_x(a.off[n_reqs]);
  PDK_REQUIRE(gx < (1ll << 31), "launch too large");
  int64_t moved = 0;                             // valid frame columns read, blocks written
  for (int i = 0; i < n_reqs; ++i)
    moved += (int64_t)n_layers * 2 * n_kv_heads * head_dim * 2 * 2 * a.req[i].P;
  if (moved > kStreamBytes)
    hipLaunchKernelGGL(scatter_kernel<true>, dim3((unsigned)gx), dim3(256), 0, pdk::as_stream(stream), a);
  else
    hipLaunchKernelGGL(scatter_kernel<false>, dim3((unsigned)gx), dim3(256), 0, pdk::as_stream(stream), a);
  return pdk::check_launch("scatter_kernel");
}
}  // namespace

extern "C" int pdk_scatter_paged_batch(const pdk_scatter_req* reqs, int n_reqs, int n_layers,
                                       int S, int n_kv_heads, int head_dim, uint16_t* cache_k,
                                       uint16_t* cache_v, int64_t cache_layer_stride,
                                       int num_blocks, uintptr_t stream) {
  return scatter_batch(reqs, n_reqs, n_layers, S, n_kv_heads, head_dim, cache_k, cache_v,
                       cache_layer_stride, num_blocks, nullptr, stream);
}

extern "C" int pdk_scatter_paged_batch_counted(const pdk_scatter_req* reqs, int n_reqs,
                                               int n_layers, int S, int n_kv_heads, int head_dim,
                                               uint16_t* cache_k, uint16_t* cache_v,
                                               int64_t cache_layer_stride, int num_blocks,
                                               int32_t* skipped, uintptr_t stream) {
  PDK_REQUIRE(skipped && ((uintptr_t)skipped & 3u) == 0, "skipped must be a 4-byte aligned int32");
  return scatter_batch(reqs, n_reqs, n_layers, S, n_kv_heads, head_dim, cache_k, cache_v,
                       cache_layer_stride, num_blocks, skipped, stream);
}

extern "C" int pdk_scatter_paged(const uint16_t* frame, const int32_t* block_table, int n_table,
                                 int n_layers, int P, int S, int n_kv_heads, int head_dim,
                                 uint16_t* cache_k, uint16_t* cache_v,
                                 int64_t cache_layer_stride, int num_blocks, uintptr_t stream) {
  pdk_scatter_req r{frame, block_table, P, n_table};
  return pdk_scatter_paged_batch(&r, 1, n_layers, S, n_kv_heads, head_dim, cache_k, cache_v,
                                 cache_layer_stride, num_blocks, stream);
}

extern "C" int pdk_gather_paged(const uint16_t* cache_k, const uint16_t* cache_v,
                                int64_t cache_layer_stride, int num_blocks,
                                const int32_t* block_table, int n_table, int n_layers, int P,
                                int S, int n_kv_heads, int head_dim, uint16_t* frame,
                                uintptr_t stream) {
  pdk::clear_error();
  int rc = check_common(n_layers, S, n_kv_heads, head_dim);
  if (rc) return rc;
  PDK_REQUIRE(frame && pdk::aligned16(frame), "frame null or not 16-byte aligned");
  PDK_REQUIRE(P >= 0 && P <= S, "P=%d outside [0, S=%d]", P, S);
  PDK_REQUIRE(cache_k && cache_v && pdk::aligned16(cache_k) && pdk::aligned16(cache_v),
              "cache_k/cache_v null or not 16-byte aligned");
  PDK_REQUIRE(num_blocks >= 1, "num_blocks must be >= 1");
  PDK_REQUIRE(cache_layer_stride % 8 == 0, "cache_layer_stride must be a multiple of 8");
  PDK_REQUIRE(P == 0 || (block_table && n_table >= (P + 15) / 16),
              "block table null or shorter than ceil(P/16)");
  GatherArgs a{};
  a.cache_k = cache_k;
  a.cache_v = cache_v;
  a.table = block_table;
  a.frame = frame;
  a.cache_ls = cache_layer_stride;
  a.num_blocks = num_blocks;
  a.n_table = n_table;
  a.P = P;
  a.S = S;
  a.Hkv = n_kv_heads;
  a.D = head_dim;
  a.nC = (S + kTileT - 1) / kTileT;
  a.nD = head_dim / kTileD;
  a.units = (int64_t)n_layers * n_kv_heads * a.nC * a.nD;
  const int64_t gx = grid_x(a.units);
  PDK_REQUIRE(gx < (1ll << 31), "launch too large");
  const int64_t moved = (int64_t)n_layers * 2 * n_kv_heads * head_dim * 2 * ((int64_t)P + S);
  if (moved > kStreamBytes)
    hipLaunchKernelGGL(gather_kernel<true>, dim3((unsigned)gx), dim3(256), 0, pdk::as_stream(stream), a);
  else
    hipLaunchKernelGGL(gather_kernel<false>, dim3((unsigned)gx), dim3(256), 0, pdk::as_stream(stream), a);
  return pdk::check_launch("gather_kernel");
}
