/*
 * CPU oracle for the KV handoff and decode attention -- TEST INFRASTRUCTURE.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load this library, and only as the oracle results are compared with. It is a plain-loop restatement
 * of what the reference computes, written for clarity, not speed.
 *
 * Layouts match include/rngdpd.h:
 *   prefill KV  [L][T][Hkv][D] with free layer/token strides (elements)
 *   frame       [L][2][F], F = Hkv*D*S; K [Hkv][D][S], V [Hkv][S][D]
 *   paged cache K [L][nb][Hkv][16][D], V [L][nb][Hkv][D][16]
 * bf16 values are carried as uint16 bit patterns.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define BS 16

static float widen(uint16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* ser() bf16 encode: keep the high 16 bits of the f32 pattern (truncation),
 * connector/transport.py:33-35 `(f.view(np.uint32) >> 16).astype(np.uint16)`. */
void orc_bf16_truncate(const float* x, int64_t n, uint16_t* out) {
  for (int64_t i = 0; i < n; ++i) {
    uint32_t u;
    memcpy(&u, &x[i], 4);
    out[i] = (uint16_t)(u >> 16);
  }
}

/* deser() bf16 decode, connector/transport.py:41-42
 * `(o["bf16"].astype(np.uint32) << 16).view(np.float32)`. */
void orc_bf16_widen(const uint16_t* x, int64_t n, float* out) {
  for (int64_t i = 0; i < n; ++i) out[i] = widen(x[i]);
}

/* Frame step of FullPrefillEngine.prefill_stream
 * (engines/prefill_full.py:378-382): K keeps columns < P and is zero from P
 * to S, in the [Hkv][D][S] order the reference's K cache uses
 * (engines/prefill_full.py:9-10, kv_nixl.py:18-20); V likewise in
 * [Hkv][S][D]. */
int orc_pack_kv(const uint16_t* src_k, const uint16_t* src_v, int64_t layer_stride,
                int64_t tok_stride, int L, int P, int S, int Hkv, int D, uint16_t* frame) {
  if (P < 0 || P > S) return -22;
  const int64_t F = (int64_t)Hkv * D * S;
  for (int l = 0; l < L; ++l) {
    uint16_t* fk = frame + (int64_t)(2 * l) * F;
    uint16_t* fv = fk + F;
    for (int h = 0; h < Hkv; ++h)
      for (int t = 0; t < S; ++t)
        for (int d = 0; d < D; ++d) {
          const int64_t s = (int64_t)l * layer_stride + (int64_t)t * tok_stride + (int64_t)h * D + d;
          fk[((int64_t)h * D + d) * S + t] = t < P ? src_k[s] : 0;
          fv[((int64_t)h * S + t) * D + d] = t < P ? src_v[s] : 0;
        }
  }
  return 0;
}

/* Element offset, inside one (block, KV head) K block of 16*D values, of
 * token `slot` (0..15) and dim d. The block is 16-byte units of 8 dims of one
 * token in tiled order: the unit of (slot, d/8) is
 * ((t*(D/32) + d/32)*4 + (d/8)%4)*8 + j8, t = (slot>>2)&1,
 * j8 = (slot>>3)*4 + (slot&3). A layout of this package's paged cache (the reference keeps
 * dense per-stream K, engines/decode_batch.py:305-330). Needs D % 32 == 0. */
static int64_t k_index(int slot, int d, int D) {
  const int t = (slot >> 2) & 1, j8 = ((slot >> 3) << 2) | (slot & 3);
  const int64_t unit = ((int64_t)(t * (D / 32) + d / 32) * 4 + (d / 8) % 4) * 8 + j8;
  return unit * 8 + d % 8;
}

/* Decode-side placement of a delivered frame (connector/rngd_kv.py:160-165)
 * into a paged cache: token t of the request goes to block table[t/16],
 * slot t%16; slots >= P of the last block are zero. */
int orc_scatter_paged(const uint16_t* frame, const int32_t* table, int n_table, int L, int P,
                      int S, int Hkv, int D, uint16_t* cache_k, uint16_t* cache_v,
                      int64_t cache_ls, int num_blocks) {
  if (P < 0 || P > S || n_table < (P + BS - 1) / BS || D % 32 != 0) return -22;
  const int64_t F = (int64_t)Hkv * D * S;
  for (int j = 0; j < (P + BS - 1) / BS; ++j) {
    const int blk = table[j];
    if (blk < 0 || blk >= num_blocks) continue;
    for (int l = 0; l < L; ++l) {
      const uint16_t* fk = frame + (int64_t)(2 * l) * F;
      const uint16_t* fv = fk + F;
      for (int h = 0; h < Hkv; ++h)
        for (int slot = 0; slot < BS; ++slot) {
          const int t = j * BS + slot;
          for (int d = 0; d < D; ++d) {
            const uint16_t k = t < P ? fk[((int64_t)h * D + d) * S + t] : 0;
            const uint16_t v = t < P ? fv[((int64_t)h * S + t) * D + d] : 0;
            cache_k[(int64_t)l * cache_ls + ((int64_t)blk * Hkv + h) * BS * D + k_index(slot, d, D)] = k;
            cache_v[(int64_t)l * cache_ls + (((int64_t)blk * Hkv + h) * D + d) * BS + slot] = v;
          }
        }
    }
  }
  return 0;
}

/* Inverse of orc_scatter_paged: an S-wide frame, zero for t >= P. */
int orc_gather_paged(const uint16_t* cache_k, const uint16_t* cache_v, int64_t cache_ls,
                     int num_blocks, const int32_t* table, int n_table, int L, int P, int S,
                     int Hkv, int D, uint16_t* frame) {
  if (P < 0 || P > S || n_table < (P + BS - 1) / BS || D % 32 != 0) return -22;
  const int64_t F = (int64_t)Hkv * D * S;
  memset(frame, 0, (size_t)L * 2 * F * sizeof(uint16_t));
  for (int l = 0; l < L; ++l) {
    uint16_t* fk = frame + (int64_t)(2 * l) * F;
    uint16_t* fv = fk + F;
    for (int t = 0; t < P; ++t) {
      const int blk = table[t / BS];
      if (blk < 0 || blk >= num_blocks) continue;
      const int slot = t % BS;
      for (int h = 0; h < Hkv; ++h)
        for (int d = 0; d < D; ++d) {
          fk[((int64_t)h * D + d) * S + t] =
              cache_k[(int64_t)l * cache_ls + ((int64_t)blk * Hkv + h) * BS * D + k_index(slot, d, D)];
          fv[((int64_t)h * S + t) * D + d] =
              cache_v[(int64_t)l * cache_ls + (((int64_t)blk * Hkv + h) * D + d) * BS + slot];
        }
    }
  }
  return 0;
}

/* One-hot injection of the new token's k/v at slot pos = ctx-1
 * (kernels/decode_batch.py:81-82; cpu_layer writes it at :148-150). */
int orc_cache_append(const uint16_t* k_new, const uint16_t* v_new, uint16_t* cache_k,
                     uint16_t* cache_v, int num_blocks, const int32_t* tables, int max_blocks,
                     const int32_t* ctx, int B, int Hkv, int D) {
  if (D % 32 != 0) return -22;
  for (int b = 0; b < B; ++b) {
    const int t = ctx[b] - 1;
    if (t < 0 || t >= max_blocks * BS) continue;
    const int blk = tables[(int64_t)b * max_blocks + t / BS];
    if (blk < 0 || blk >= num_blocks) continue;
    for (int h = 0; h < Hkv; ++h)
      for (int d = 0; d < D; ++d) {
        const int64_t s = ((int64_t)b * Hkv + h) * D + d;
        cache_k[((int64_t)blk * Hkv + h) * BS * D + k_index(t % BS, d, D)] = k_new[s];
        cache_v[(((int64_t)blk * Hkv + h) * D + d) * BS + t % BS] = v_new[s];
      }
  }
  return 0;
}

/* Attention part of cpu_layer (kernels/decode_batch.py:151-156): scores
 * q.k * scale over slots 0..pos (pos = ctx-1; slots > pos get -1e4, whose
 * exp underflows to exactly 0 after the max subtraction, so they drop out),
 * max-subtracted softmax, then p.V. Query head qh reads KV head qh/(Hq/Hkv)
 * (q.reshape(B, NKV, G, HD), :151). Accumulates in double, returns float.
 * The paged cache adds one case the reference's dense per-lane cache cannot
 * have: a block id outside [0, num_blocks) inside the context. Its tokens
 * are masked like slots past pos (they take no part in the softmax); a
 * stream with no token left gets a zero output. */
int orc_decode_attn(const uint16_t* q, const uint16_t* cache_k, const uint16_t* cache_v,
                    int num_blocks, const int32_t* tables, int max_blocks, const int32_t* ctx,
                    int B, int Hq, int Hkv, int D, float scale, float* out) {
  if (Hq % Hkv != 0 || D % 32 != 0) return -22;
  const int G = Hq / Hkv;
  double* sc = (double*)malloc(sizeof(double) * (size_t)max_blocks * BS);
  if (!sc) return -12;
  for (int b = 0; b < B; ++b) {
    int n = ctx[b];
    if (n > max_blocks * BS) n = max_blocks * BS;
    for (int qh = 0; qh < Hq; ++qh) {
      const int h = qh / G;
      const uint16_t* qp = q + ((int64_t)b * Hq + qh) * D;
      float* op = out + ((int64_t)b * Hq + qh) * D;
      double mx = -INFINITY;
      int live = 0;
      for (int t = 0; t < n; ++t) {
        const int blk = tables[(int64_t)b * max_blocks + t / BS];
        if (blk < 0 || blk >= num_blocks) continue;          /* masked */
        const uint16_t* kb = cache_k + ((int64_t)blk * Hkv + h) * BS * D;
        double s = 0.0;
        for (int d = 0; d < D; ++d) s += (double)widen(qp[d]) * (double)widen(kb[k_index(t % BS, d, D)]);
        sc[t] = s * scale;
        if (sc[t] > mx) mx = sc[t];
        ++live;
      }
      double sum = 0.0;
      for (int t = 0; t < n; ++t) {
        const int blk = tables[(int64_t)b * max_blocks + t / BS];
        if (blk < 0 || blk >= num_blocks) continue;
        sc[t] = exp(sc[t] - mx);
        sum += sc[t];
      }
      for (int d = 0; d < D; ++d) {
        double acc = 0.0;
        for (int t = 0; t < n; ++t) {
          const int blk = tables[(int64_t)b * max_blocks + t / BS];
          if (blk < 0 || blk >= num_blocks) continue;
          acc += sc[t] * (double)widen(cache_v[(((int64_t)blk * Hkv + h) * D + d) * BS + t % BS]);
        }
        op[d] = live > 0 ? (float)(acc / sum) : 0.0f;
      }
    }
  }
  free(sc);
  return 0;
}

/* greedy_tokens (engines/decode_batch.py:162-171): torch.argmax over the
 * vocabulary, first maximum wins; NaN counts as the maximum. */
int orc_greedy_argmax(const uint16_t* logits, int B, int V, int64_t ld, int32_t* out) {
  for (int b = 0; b < B; ++b) {
    int best = 0;
    float bv = widen(logits[(int64_t)b * ld]);
    for (int i = 1; i < V; ++i) {
      const float x = widen(logits[(int64_t)b * ld + i]);
      if (bv != bv) break;
      if (x != x || x > bv) {
        bv = x;
        best = i;
      }
    }
    out[b] = best;
  }
  return 0;
}
