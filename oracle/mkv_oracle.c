/*
 * CPU oracle for the paged-KV hot path.
 *
 * TEST INFRASTRUCTURE ONLY. This file is the checker: only tests/, the smoke()
 * entry and bench.py's CPU-baseline leg may load it. The product path (the HIP
 * library under mitten_amd/) never links, calls or falls back to it.
 *
 * It restates, in plain C, what the reference engine does (or, where the
 * reference has no implementation, the closed form the reference's design
 * fixes) for each operation on the path:
 *
 *   orc_pool_bytes       inference-engine/src/kv_pool.rs:58-68 (required_bytes)
 *   orc_append           inference-model-qwen/src/model.rs:390-392 (Tensor::cat
 *                        of the new K/V rows), addressed through the slot
 *                        mapping slot = page*page_size + pos%page_size implied by
 *                        inference-engine/src/prefill.rs:72-81 and
 *                        inference-engine/src/scheduler.rs:42-47,56-57
 *   orc_gather           design/phase0-deliverable.md:278 (gather-then-attend);
 *                        output layout inference-model-common/src/lib.rs:5-8
 *                        ([batch, heads, seq, head_dim] per sequence)
 *   orc_copy_blocks      no reference counterpart (the reference has no COW or
 *                        compaction); closed-form per-block memcpy over all
 *                        layers, K and V
 *   orc_decode_attention inference-model-qwen/src/model.rs:394-416 (GQA repeat,
 *                        q.k^T * scaling, additive causal mask, softmax, .v),
 *                        scaling = head_dim^-0.5 (model.rs:298)
 *   orc_norm_rope_rows   inference-model-qwen/src/model.rs:104-108 (RmsNorm::forward4:
 *                        x * (mean(x^2) + eps)^-1/2 * (w + 1)) followed by
 *                        model.rs:508-540 (apply_rope, NeoX half-rotation of
 *                        dims [0, rotary_dim), the rest passed through), as
 *                        GatedAttention::forward applies them (model.rs:380-384)
 *   orc_wire_*           no reference implementation (the reference hands pages
 *                        between workers as indices, design/phase2b-deliverable.md:
 *                        272-289, and sketches per-layer SSD KV files,
 *                        design/phase1-deliverable.md:253-339); the closed form of
 *                        the byte format declared in include/mitten_kv.h:
 *                        payload [n][layers][K,V][page][heads][dim], per-block
 *                        sum64 checksum
 *   orc_ref_faithful_*   the same attention, executed the way the reference
 *                        executes it (contiguous cache grown by a copy per
 *                        token, repeat_kv materialised, mask built per call);
 *                        used only as the timed CPU baseline
 *
 * Pool layout (design/rust-inference-engine-design.md:1385):
 *   [num_layers][2 (K,V)][num_blocks][page_size][num_kv_heads][head_dim]
 *
 * Parity pins for every function are listed in tests/test_oracle.py.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define ORC_API __attribute__((visibility("default")))

/* ------------------------------------------------------------------ */
/* Seeded synthetic data: SplitMix64 -> uniform -> Box-Muller N(0,1).  */
/* ------------------------------------------------------------------ */

static inline uint64_t splitmix64_next(uint64_t *s) {
  uint64_t z = (*s += 0x9E3779B97F4A7C15ull);
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

ORC_API uint64_t orc_splitmix64(uint64_t *state) { return splitmix64_next(state); }

/* Uniform in (0,1]: top 53 bits, offset so log() never sees 0. */
static inline double u01_open0(uint64_t *s) {
  return ((double)(splitmix64_next(s) >> 11) + 1.0) * (1.0 / 9007199254740992.0);
}

ORC_API void orc_fill_normal_f32(uint64_t seed, int64_t n, float *out) {
  uint64_t s = seed;
  int64_t i = 0;
  while (i < n) {
    double u1 = u01_open0(&s), u2 = u01_open0(&s);
    double r = sqrt(-2.0 * log(u1));
    double t = 6.283185307179586476925286766559 * u2;
    out[i++] = (float)(r * cos(t));
    if (i < n) out[i++] = (float)(r * sin(t));
  }
}

/* Lemire's nearly-divisionless bounded integer in [0, range). */
ORC_API uint32_t orc_bounded(uint64_t *state, uint32_t range) {
  uint32_t x = (uint32_t)(splitmix64_next(state) >> 32);
  uint64_t m = (uint64_t)x * range;
  uint32_t l = (uint32_t)m;
  if (l < range) {
    uint32_t t = (uint32_t)(-range) % range;
    while (l < t) {
      x = (uint32_t)(splitmix64_next(state) >> 32);
      m = (uint64_t)x * range;
      l = (uint32_t)m;
    }
  }
  return (uint32_t)(m >> 32);
}

/* f32 -> bf16, round to nearest even; NaN stays NaN (quietened). */
ORC_API void orc_f32_to_bf16(const float *in, uint16_t *out, int64_t n) {
  for (int64_t i = 0; i < n; i++) {
    uint32_t u;
    memcpy(&u, &in[i], 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) {
      out[i] = (uint16_t)((u >> 16) | 0x0040u);
    } else {
      u += 0x7fffu + ((u >> 16) & 1u);
      out[i] = (uint16_t)(u >> 16);
    }
  }
}

ORC_API void orc_bf16_to_f32(const uint16_t *in, float *out, int64_t n) {
  for (int64_t i = 0; i < n; i++) {
    uint32_t u = (uint32_t)in[i] << 16;
    memcpy(&out[i], &u, 4);
  }
}

/* ------------------------------------------------------------------ */
/* Pool geometry.                                                      */
/* ------------------------------------------------------------------ */

typedef struct {
  int32_t num_layers;
  int32_t num_kv_heads;
  int32_t head_dim;
  int32_t page_size;
  int64_t num_blocks;
  int32_t elem_bytes; /* 4 = f32, 2 = bf16 */
} orc_pool_desc;

/* kv_pool.rs:58-68: 2 * layers * pages * page_size * kv_heads * head_dim * dtype */
ORC_API int64_t orc_pool_bytes(const orc_pool_desc *d) {
  return 2ll * d->num_layers * d->num_blocks * d->page_size * d->num_kv_heads * d->head_dim *
         d->elem_bytes;
}

static inline int64_t row_bytes(const orc_pool_desc *d) {
  return (int64_t)d->num_kv_heads * d->head_dim * d->elem_bytes;
}
static inline int64_t block_bytes(const orc_pool_desc *d) { return d->page_size * row_bytes(d); }
/* Byte offset of (layer, kv, block, 0, 0, 0). */
static inline int64_t plane_off(const orc_pool_desc *d, int layer, int kv, int64_t block) {
  return (((int64_t)layer * 2 + kv) * d->num_blocks + block) * block_bytes(d);
}

/* Append: for every token t, pool[layer][K|V][slot/ps][slot%ps][:][:] = src[t][:][:].
 * Returns the index of the first token whose slot is out of range, or -1. */
ORC_API int64_t orc_append(const orc_pool_desc *d, uint8_t *pool, int layer, const void *k,
                           const void *v, const int32_t *slots, int64_t n_tok) {
  const int64_t rb = row_bytes(d);
  const int64_t nslots = d->num_blocks * d->page_size;
  for (int64_t t = 0; t < n_tok; t++) {
    int64_t s = slots[t];
    if (s < 0 || s >= nslots) return t;
    int64_t blk = s / d->page_size, off = s % d->page_size;
    memcpy(pool + plane_off(d, layer, 0, blk) + off * rb, (const uint8_t *)k + t * rb, rb);
    memcpy(pool + plane_off(d, layer, 1, blk) + off * rb, (const uint8_t *)v + t * rb, rb);
  }
  return -1;
}

/* Gather: sequence b's first ctx_len[b] tokens, addressed through its block
 * table indices[indptr[b] .. indptr[b+1]), are written contiguously as
 * [num_kv_heads][ctx_len[b]][head_dim] at element offset
 * num_kv_heads*head_dim*sum_{b'<b} ctx_len[b'] of dst_k / dst_v. */
ORC_API int orc_gather(const orc_pool_desc *d, const uint8_t *pool, int layer,
                       const int32_t *indptr, const int32_t *indices, const int32_t *ctx_len,
                       int32_t num_seqs, void *dst_k, void *dst_v) {
  const int64_t es = d->elem_bytes, D = d->head_dim, H = d->num_kv_heads, ps = d->page_size;
  const int64_t rb = row_bytes(d);
  int64_t base = 0; /* token offset of this sequence in the ragged output */
  for (int b = 0; b < num_seqs; b++) {
    int64_t n = ctx_len[b];
    if (n < 0 || (n + ps - 1) / ps > indptr[b + 1] - indptr[b]) return -1;
    for (int64_t t = 0; t < n; t++) {
      int64_t blk = indices[indptr[b] + t / ps];
      if (blk < 0 || blk >= d->num_blocks) return -1;
      for (int kv = 0; kv < 2; kv++) {
        const uint8_t *src = pool + plane_off(d, layer, kv, blk) + (t % ps) * rb;
        uint8_t *dst = (uint8_t *)(kv ? dst_v : dst_k);
        for (int64_t h = 0; h < H; h++)
          memcpy(dst + ((base * H + h * n + t) * D) * es, src + h * D * es, D * es);
      }
    }
    base += n;
  }
  return 0;
}

/* Copy blocks: for every pair i and every layer, K and V:
 * pool[l][kv][dst[i]] = pool[l][kv][src[i]] (whole block, page_size rows). */
ORC_API int orc_copy_blocks(const orc_pool_desc *d, uint8_t *pool, const int32_t *src,
                            const int32_t *dst, int64_t n) {
  const int64_t bb = block_bytes(d);
  for (int64_t i = 0; i < n; i++) {
    if (src[i] < 0 || src[i] >= d->num_blocks || dst[i] < 0 || dst[i] >= d->num_blocks) return -1;
    for (int l = 0; l < d->num_layers; l++)
      for (int kv = 0; kv < 2; kv++)
        memmove(pool + plane_off(d, l, kv, dst[i]), pool + plane_off(d, l, kv, src[i]), bb);
  }
  return 0;
}

/* RMSNorm then partial NeoX RoPE, in place, on `rows` rows of D f32 values
 * (model.rs:104-108, 508-540). Row r sits at position pos[r]. w == NULL skips
 * the norm. All arithmetic f32 in the reference's order: the mean of squares,
 * + eps, sqrt, reciprocal, x * that, then * (w + 1); then for i < half =
 * rotary_dim/2, a = (float)pos * inv_freq[i],
 *   x[i] * cos a - x[i+half] * sin a,  x[i+half] * cos a + x[i] * sin a.
 * (Built with -std=c11: no contraction into FMAs.) */
ORC_API void orc_norm_rope_rows(float *x, int64_t rows, int32_t D, const float *w, float eps,
                                const float *inv_freq, int32_t rotary_dim, const int32_t *pos) {
  const int half = rotary_dim / 2;
  for (int64_t r = 0; r < rows; r++) {
    float *row = x + r * D;
    if (w) {
      float ss = 0.0f;
      for (int i = 0; i < D; i++) ss += row[i] * row[i];
      const float inv = 1.0f / sqrtf(ss / (float)D + eps);
      for (int i = 0; i < D; i++) row[i] = (row[i] * inv) * (w[i] + 1.0f);
    }
    const float p = (float)pos[r];
    for (int i = 0; i < half; i++) {
      const float a = p * inv_freq[i];
      const float c = cosf(a), sn = sinf(a);
      const float x1 = row[i], x2 = row[i + half];
      row[i] = x1 * c - x2 * sn;
      row[i + half] = x2 * c + x1 * sn;
    }
  }
}

/* sum64 of one block's payload: sum over little-endian u64 words w_j of
 * mix(w_j + (j + 1) * golden), mix the splitmix64 output function, mod 2^64.
 * splitmix64_next(&s) with s = w_j + j * golden adds golden and mixes: the
 * same value. */
static uint64_t wire_sum64(const uint8_t *p, int64_t nbytes) {
  uint64_t acc = 0;
  for (int64_t j = 0; j < nbytes / 8; j++) {
    uint64_t w;
    memcpy(&w, p + 8 * j, 8);
    uint64_t s = w + (uint64_t)j * 0x9E3779B97F4A7C15ull;
    acc += splitmix64_next(&s);
  }
  return acc;
}

ORC_API void orc_wire_checksums(const uint8_t *payload, int64_t n, int64_t block_bytes, uint64_t *out) {
  for (int64_t i = 0; i < n; i++) out[i] = wire_sum64(payload + i * block_bytes, block_bytes);
}

/* Export: payload[i][l][kv] = pool[layer_begin + l][kv][ids[i]] (one whole
 * block plane, page_size rows), checksums per block. Returns -1, or the index
 * of the first id outside the pool (nothing written for it). */
ORC_API int64_t orc_wire_export(const orc_pool_desc *d, const uint8_t *pool, const int32_t *ids, int64_t n,
                                int layer_begin, int num_layers, uint8_t *payload, uint64_t *sums) {
  const int64_t bb = block_bytes(d), per = (int64_t)num_layers * 2 * bb;
  for (int64_t i = 0; i < n; i++) {
    if (ids[i] < 0 || ids[i] >= d->num_blocks) return i;
    for (int l = 0; l < num_layers; l++)
      for (int kv = 0; kv < 2; kv++)
        memcpy(payload + i * per + ((int64_t)l * 2 + kv) * bb, pool + plane_off(d, layer_begin + l, kv, ids[i]), bb);
    sums[i] = wire_sum64(payload + i * per, per);
  }
  return -1;
}

/* Import: the inverse scatter; sums of the payload as received. */
ORC_API int64_t orc_wire_import(const orc_pool_desc *d, uint8_t *pool, const int32_t *ids, int64_t n,
                                int layer_begin, int num_layers, const uint8_t *payload, uint64_t *sums) {
  const int64_t bb = block_bytes(d), per = (int64_t)num_layers * 2 * bb;
  for (int64_t i = 0; i < n; i++) {
    if (ids[i] < 0 || ids[i] >= d->num_blocks) return i;
    for (int l = 0; l < num_layers; l++)
      for (int kv = 0; kv < 2; kv++)
        memcpy(pool + plane_off(d, layer_begin + l, kv, ids[i]), payload + i * per + ((int64_t)l * 2 + kv) * bb, bb);
    sums[i] = wire_sum64(payload + i * per, per);
  }
  return -1;
}

/* Element load from the pool as f32 (bf16 is widened exactly). */
static inline float pool_elem(const orc_pool_desc *d, const uint8_t *p) {
  if (d->elem_bytes == 4) {
    float f;
    memcpy(&f, p, 4);
    return f;
  }
  uint32_t u = (uint32_t)(*(const uint16_t *)p) << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* Decode attention, f32 arithmetic in the reference's order (model.rs:394-416):
 *   scores_t = (sum_d q_d * k_td) * scale           (q.matmul(k^T) * scaling)
 *   (+ mask: with one query row nothing is masked,   model.rs:542-555)
 *   p = softmax(scores) = exp(s - max) / sum exp(s - max)
 *   o_d = sum_t p_t * v_td
 * Query head h reads KV head h / (num_q_heads / num_kv_heads) (repeat along the
 * group axis, model.rs:398-408).  zero_sink = 1 adds the reference's phantom
 * all-zero key/value (init_cache, model.rs:210-213): one extra score 0 with
 * value 0.  q: [num_seqs][num_q_heads][head_dim] f32, o likewise. */
ORC_API int orc_decode_attention_f32(const orc_pool_desc *d, const uint8_t *pool, int layer,
                                     const float *q, int32_t num_seqs, int32_t num_q_heads,
                                     const int32_t *indptr, const int32_t *indices,
                                     const int32_t *ctx_len, float scale, int zero_sink,
                                     float *o) {
  const int64_t D = d->head_dim, H = d->num_kv_heads, ps = d->page_size, es = d->elem_bytes;
  const int64_t rb = row_bytes(d);
  if (num_q_heads % H) return -1;
  const int rep = num_q_heads / (int)H;
  int err = 0;
#pragma omp parallel for collapse(2) schedule(dynamic)
  for (int b = 0; b < num_seqs; b++) {
    for (int hq = 0; hq < num_q_heads; hq++) {
      const int64_t n = ctx_len[b];
      const int hk = hq / rep;
      const float *qv = q + ((int64_t)b * num_q_heads + hq) * D;
      float *ov = o + ((int64_t)b * num_q_heads + hq) * D;
      if (n <= 0 || (n + ps - 1) / ps > indptr[b + 1] - indptr[b]) {
        err = 1;
        continue;
      }
      float *s = (float *)malloc(sizeof(float) * (n + 1));
      float mx = zero_sink ? 0.0f : -INFINITY;
      for (int64_t t = 0; t < n; t++) {
        int64_t blk = indices[indptr[b] + t / ps];
        const uint8_t *kr = pool + plane_off(d, layer, 0, blk) + (t % ps) * rb + hk * D * es;
        float acc = 0.0f;
        for (int64_t i = 0; i < D; i++) acc += qv[i] * pool_elem(d, kr + i * es);
        s[t] = acc * scale;
        if (s[t] > mx) mx = s[t];
      }
      float sum = 0.0f;
      for (int64_t t = 0; t < n; t++) {
        s[t] = expf(s[t] - mx);
        sum += s[t];
      }
      if (zero_sink) sum += expf(0.0f - mx);
      for (int64_t i = 0; i < D; i++) ov[i] = 0.0f;
      for (int64_t t = 0; t < n; t++) {
        int64_t blk = indices[indptr[b] + t / ps];
        const uint8_t *vr = pool + plane_off(d, layer, 1, blk) + (t % ps) * rb + hk * D * es;
        const float p = s[t] / sum;
        for (int64_t i = 0; i < D; i++) ov[i] += p * pool_elem(d, vr + i * es);
      }
      free(s);
    }
  }
  return err ? -1 : 0;
}

/* Same computation in double precision throughout (q given as f32 values). */
ORC_API int orc_decode_attention_f64(const orc_pool_desc *d, const uint8_t *pool, int layer,
                                     const float *q, int32_t num_seqs, int32_t num_q_heads,
                                     const int32_t *indptr, const int32_t *indices,
                                     const int32_t *ctx_len, double scale, int zero_sink,
                                     double *o) {
  const int64_t D = d->head_dim, H = d->num_kv_heads, ps = d->page_size, es = d->elem_bytes;
  const int64_t rb = row_bytes(d);
  if (num_q_heads % H) return -1;
  const int rep = num_q_heads / (int)H;
  int err = 0;
#pragma omp parallel for collapse(2) schedule(dynamic)
  for (int b = 0; b < num_seqs; b++) {
    for (int hq = 0; hq < num_q_heads; hq++) {
      const int64_t n = ctx_len[b];
      const int hk = hq / rep;
      const float *qv = q + ((int64_t)b * num_q_heads + hq) * D;
      double *ov = o + ((int64_t)b * num_q_heads + hq) * D;
      if (n <= 0 || (n + ps - 1) / ps > indptr[b + 1] - indptr[b]) {
        err = 1;
        continue;
      }
      double *s = (double *)malloc(sizeof(double) * n);
      double mx = zero_sink ? 0.0 : -INFINITY;
      for (int64_t t = 0; t < n; t++) {
        int64_t blk = indices[indptr[b] + t / ps];
        const uint8_t *kr = pool + plane_off(d, layer, 0, blk) + (t % ps) * rb + hk * D * es;
        double acc = 0.0;
        for (int64_t i = 0; i < D; i++) acc += (double)qv[i] * (double)pool_elem(d, kr + i * es);
        s[t] = acc * scale;
        if (s[t] > mx) mx = s[t];
      }
      double sum = 0.0;
      for (int64_t t = 0; t < n; t++) {
        s[t] = exp(s[t] - mx);
        sum += s[t];
      }
      if (zero_sink) sum += exp(-mx);
      for (int64_t i = 0; i < D; i++) ov[i] = 0.0;
      for (int64_t t = 0; t < n; t++) {
        int64_t blk = indices[indptr[b] + t / ps];
        const uint8_t *vr = pool + plane_off(d, layer, 1, blk) + (t % ps) * rb + hk * D * es;
        const double p = s[t] / sum;
        for (int64_t i = 0; i < D; i++) ov[i] += p * (double)pool_elem(d, vr + i * es);
      }
      free(s);
    }
  }
  return err ? -1 : 0;
}

/* ------------------------------------------------------------------ */
/* Reference-faithful CPU baseline (timed beside the GPU; not a parity  */
/* checker).  One decode step of one attention layer for one sequence,  */
/* executed the way model.rs:390-416 executes it on Burn's CPU backend: */
/*   cat:    new cache [Hkv][T+1][D] = old cache ++ new row (full copy)  */
/*   repeat: K_ext, V_ext [Hq][T+1][D] materialised                      */
/*   mask:   [T+1] additive zeros built per call                         */
/*   scores = q . K_ext^T * scale + mask;  softmax;  out = p . V_ext     */
/* Caches are f32 (the reference's only KV dtype). Returns 0.            */
/* ------------------------------------------------------------------ */

__attribute__((target_clones("avx512f", "avx2", "default"))) static float dotf(const float *a,
                                                                              const float *b,
                                                                              int64_t n) {
  float s = 0.0f;
  for (int64_t i = 0; i < n; i++) s += a[i] * b[i];
  return s;
}

__attribute__((target_clones("avx512f", "avx2", "default"))) static void axpyf(float *y,
                                                                              const float *x,
                                                                              float a, int64_t n) {
  for (int64_t i = 0; i < n; i++) y[i] += a * x[i];
}

/* kcache/vcache: [Hkv][T][D] f32 owned by the caller (malloc'd); on return they
 * are replaced by freshly allocated [Hkv][T+1][D] buffers (the old ones freed),
 * mirroring Tensor::cat producing a new tensor. */
ORC_API int orc_ref_faithful_decode(float **kcache, float **vcache, int64_t T, int32_t Hkv,
                                    int32_t Hq, int32_t D, const float *k_new, const float *v_new,
                                    const float *q, float scale, float *out) {
  const int64_t T1 = T + 1;
  const int rep = Hq / Hkv;
  float *kc = (float *)malloc(sizeof(float) * Hkv * T1 * D);
  float *vc = (float *)malloc(sizeof(float) * Hkv * T1 * D);
  for (int h = 0; h < Hkv; h++) {
    memcpy(kc + (int64_t)h * T1 * D, *kcache + (int64_t)h * T * D, sizeof(float) * T * D);
    memcpy(kc + ((int64_t)h * T1 + T) * D, k_new + (int64_t)h * D, sizeof(float) * D);
    memcpy(vc + (int64_t)h * T1 * D, *vcache + (int64_t)h * T * D, sizeof(float) * T * D);
    memcpy(vc + ((int64_t)h * T1 + T) * D, v_new + (int64_t)h * D, sizeof(float) * D);
  }
  free(*kcache);
  free(*vcache);
  *kcache = kc;
  *vcache = vc;
  float *kext = (float *)malloc(sizeof(float) * Hq * T1 * D);
  float *vext = (float *)malloc(sizeof(float) * Hq * T1 * D);
  for (int h = 0; h < Hq; h++) {
    memcpy(kext + (int64_t)h * T1 * D, kc + (int64_t)(h / rep) * T1 * D, sizeof(float) * T1 * D);
    memcpy(vext + (int64_t)h * T1 * D, vc + (int64_t)(h / rep) * T1 * D, sizeof(float) * T1 * D);
  }
  float *mask = (float *)calloc(T1, sizeof(float));
  float *sc = (float *)malloc(sizeof(float) * T1);
  for (int h = 0; h < Hq; h++) {
    const float *qh = q + (int64_t)h * D;
    float mx = -INFINITY;
    for (int64_t t = 0; t < T1; t++) {
      sc[t] = dotf(qh, kext + ((int64_t)h * T1 + t) * D, D) * scale + mask[t];
      if (sc[t] > mx) mx = sc[t];
    }
    float sum = 0.0f;
    for (int64_t t = 0; t < T1; t++) {
      sc[t] = expf(sc[t] - mx);
      sum += sc[t];
    }
    float *oh = out + (int64_t)h * D;
    memset(oh, 0, sizeof(float) * D);
    for (int64_t t = 0; t < T1; t++) axpyf(oh, vext + ((int64_t)h * T1 + t) * D, sc[t] / sum, D);
  }
  free(mask);
  free(sc);
  free(kext);
  free(vext);
  return 0;
}

/* orc_ref_faithful_decode on malloc'd copies of the caller's caches
 * ([Hkv][T][D] each), which it grows and frees as the reference does; the
 * caller's arrays are unchanged. For the tests that check the baseline
 * against orc_decode_attention_f32. */
ORC_API int orc_ref_faithful_decode_copy(const float *kcache, const float *vcache, int64_t T, int32_t Hkv,
                                         int32_t Hq, int32_t D, const float *k_new, const float *v_new,
                                         const float *q, float scale, float *out) {
  const size_t n = (size_t)Hkv * (size_t)(T > 0 ? T : 1) * (size_t)D;
  float *kc = (float *)malloc(sizeof(float) * n);
  float *vc = (float *)malloc(sizeof(float) * n);
  if (!kc || !vc) {
    free(kc);
    free(vc);
    return -1;
  }
  memcpy(kc, kcache, sizeof(float) * (size_t)Hkv * (size_t)T * (size_t)D);
  memcpy(vc, vcache, sizeof(float) * (size_t)Hkv * (size_t)T * (size_t)D);
  const int rc = orc_ref_faithful_decode(&kc, &vc, T, Hkv, Hq, D, k_new, v_new, q, scale, out);
  free(kc);
  free(vc);
  return rc;
}

/* Thread count the OpenMP runtime will use (1 without OpenMP). */
ORC_API int orc_num_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

ORC_API void orc_set_num_threads(int n) {
#ifdef _OPENMP
  omp_set_num_threads(n);
#else
  (void)n;
#endif
}

/* Threads that fill orc_ref_faithful_batch's caches before its timed region
 * (0: the current thread count). A one-thread timing of a large sample need
 * not fill gigabytes of seeded values on one thread. */
static int g_setup_threads = 0;

ORC_API void orc_set_setup_threads(int n) { g_setup_threads = n > 0 ? n : 0; }

/* Timed CPU baseline over a batch: for every sequence b (in parallel over
 * sequences with OpenMP), one decode step of one layer executed as
 * orc_ref_faithful_decode does, starting from a contiguous cache of
 * ctx[b] - 1 tokens (filled with seeded N(0,1) values) and appending one
 * token. Cache set-up is outside the timed region; returns the wall time of
 * the decode steps in seconds. */
ORC_API double orc_ref_faithful_batch(const int32_t *ctx, int32_t num_seqs, int32_t Hkv, int32_t Hq,
                                      int32_t D, uint64_t seed) {
  float **kc = (float **)calloc(num_seqs, sizeof(float *));
  float **vc = (float **)calloc(num_seqs, sizeof(float *));
  float **qn = (float **)calloc(num_seqs, sizeof(float *));
  float **on = (float **)calloc(num_seqs, sizeof(float *));
#ifdef _OPENMP
  const int setup_threads = g_setup_threads > 0 ? g_setup_threads : omp_get_max_threads();
#endif
#pragma omp parallel for schedule(dynamic) num_threads(setup_threads)
  for (int b = 0; b < num_seqs; b++) {
    const int64_t T = ctx[b] - 1;
    kc[b] = (float *)malloc(sizeof(float) * Hkv * (T > 0 ? T : 1) * D);
    vc[b] = (float *)malloc(sizeof(float) * Hkv * (T > 0 ? T : 1) * D);
    qn[b] = (float *)malloc(sizeof(float) * (Hq + 2 * Hkv) * D);
    on[b] = (float *)malloc(sizeof(float) * Hq * D);
    orc_fill_normal_f32(seed + 3 * (uint64_t)b, Hkv * T * D, kc[b]);
    orc_fill_normal_f32(seed + 3 * (uint64_t)b + 1, Hkv * T * D, vc[b]);
    orc_fill_normal_f32(seed + 3 * (uint64_t)b + 2, (Hq + 2 * Hkv) * D, qn[b]);
  }
  double t0 = 0.0, t1 = 0.0;
#ifdef _OPENMP
  t0 = omp_get_wtime();
#endif
#pragma omp parallel for schedule(dynamic)
  for (int b = 0; b < num_seqs; b++) {
    const float scale = 1.0f / sqrtf((float)D);
    orc_ref_faithful_decode(&kc[b], &vc[b], ctx[b] - 1, Hkv, Hq, D, qn[b] + Hq * D,
                            qn[b] + (Hq + Hkv) * D, qn[b], scale, on[b]);
  }
#ifdef _OPENMP
  t1 = omp_get_wtime();
#endif
  for (int b = 0; b < num_seqs; b++) {
    free(kc[b]);
    free(vc[b]);
    free(qn[b]);
    free(on[b]);
  }
  free(kc);
  free(vc);
  free(qn);
  free(on);
  return t1 - t0;
}
