// Paged GQA/MQA decode attention, straight from the block pool.
//
// Work decomposition: one wave64 per unit (sequence b, context split, KV head
// h, query chunk qc); a 256-thread workgroup holds four consecutive units, so
// with 4 KV heads one workgroup streams all heads of the same blocks. Each
// unit runs an online (max-subtracted, base-2) softmax over its split and
// either writes the final normalised row (single split) or an unnormalised
// partial (m, l, o[D]) that merge_kernel combines by log-sum-exp.
//
// Two kernels:
//   attn_mfma_kernel  bf16 KV, head_dim 64/128/256, up to 16 query heads per
//                     wave. S^T = K.Q^T on v_mfma_f32_16x16x32_bf16 with K
//                     loaded straight into the A-operand layout (16 B per
//                     lane, no LDS), O^T = V^T.P^T on v_mfma_f32_16x16x16_bf16
//                     with V transposed in registers by a 4x4 DPP quad
//                     transpose. The S^T accumulator layout equals the P^T
//                     operand layout, and the O^T accumulator puts query row
//                     q = lane%16 where the softmax state lives, so no
//                     cross-lane traffic is needed for the rescale.
//   attn_valu_kernel  any dtype, head_dim 32/64/128/256: lanes split each
//                     token row into 16-byte chunks, scores reduce across
//                     the row's lanes with shuffles. f32 pools use this one.
//
// Arithmetic follows inference-model-qwen/src/model.rs:394-416: scores are
// (q.k) * scale with scale = head_dim^-0.5 (model.rs:298), softmax is the
// max-subtracted exponential, the output is p.v; the KV head of query head h
// is h / (num_q_heads/num_kv_heads) (repeat_kv, model.rs:398-408).
#include <algorithm>
#include <cmath>

#include "mkv_internal.h"

namespace mkv {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

constexpr float kLog2e = 1.4426950408889634f;

struct AttnArgs {
  const uint8_t *k_plane;  // layer's K plane
  const uint8_t *v_plane;  // layer's V plane
  const void *q;
  void *o;
  const int32_t *indptr;
  const int32_t *ids;
  const int32_t *ctx_lens;
  float *ws_ml;  // [B][Hq][S] (m, l) pairs
  float *ws_o;   // [B][Hq][S][D]
  uint32_t *d_err;
  int64_t nblocks;
  int64_t row_bytes;
  int64_t block_bytes;
  int64_t total_units;
  int32_t B, Hq, Hkv, G, nqc, S, split_tokens, max_ctx;
  float sl2;  // scale * log2(e)
  int32_t zero_sink;
};

struct Unit {
  int b, split, h, qc;
  int ctx, t_begin, t_end, nsp, tab0;
};

// Decodes the wave's unit and validates its sequence; false = nothing to do.
__device__ __forceinline__ bool decode_unit(const AttnArgs &a, int lane, Unit &u) {
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  int64_t id = (int64_t)blockIdx.x * 4 + wave;
  if (id >= a.total_units) return false;
  u.qc = (int)(id % a.nqc);
  id /= a.nqc;
  u.h = (int)(id % a.Hkv);
  id /= a.Hkv;
  u.split = (int)(id % a.S);
  u.b = (int)(id / a.S);
  const bool first = u.split == 0 && u.h == 0 && u.qc == 0 && lane == 0;
  u.ctx = a.ctx_lens[u.b];
  if (u.ctx < 1 || u.ctx > a.max_ctx) {
    if (first) record_error(a.d_err, MKV_DEVERR_CTX);
    return false;
  }
  u.t_begin = u.split * a.split_tokens;
  if (u.t_begin >= u.ctx) return false;
  u.t_end = min(u.ctx, u.t_begin + a.split_tokens);
  u.nsp = (u.ctx + a.split_tokens - 1) / a.split_tokens;
  u.tab0 = a.indptr[u.b];
  const int tabn = a.indptr[u.b + 1] - u.tab0;
  if (u.tab0 < 0 || tabn < (u.ctx + kPageSize - 1) / kPageSize) {
    if (first) record_error(a.d_err, MKV_DEVERR_TABLE);
    return false;
  }
  return true;
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Final normalisation of one row, including the optional phantom zero key
// (score 0, value 0) of the reference's Qwen cache (model.rs:210-213).
__device__ __forceinline__ float final_scale(float m, float l, int zero_sink) {
  if (zero_sink) {
    const float M = fmaxf(m, 0.0f);
    const float f = fast_exp2(m - M);
    return f / (l * f + fast_exp2(-M));
  }
  return 1.0f / l;
}

// ---------------------------------------------------------------------------
// VALU kernel.
// ---------------------------------------------------------------------------
template <int D, bool BF16>
__global__ void __launch_bounds__(256) attn_valu_kernel(AttnArgs a) {
  constexpr int ES = BF16 ? 2 : 4;
  constexpr int VEC = 16 / ES;
  constexpr int LPT = D / VEC;
  static_assert(LPT >= 1 && LPT <= 64 && (64 % LPT) == 0, "unsupported head_dim");
  constexpr int TPI = 64 / LPT;
  constexpr int QC = 8;
  const int lane = threadIdx.x & 63;
  Unit u;
  if (!decode_unit(a, lane, u)) return;
  const int lt = lane / LPT, ld = lane % LPT;
  const int q0 = u.qc * QC;
  const int nq = min(QC, a.G - q0);
  const int hq0 = u.h * a.G + q0;

  auto load_chunk = [&](const uint8_t *p, float (&f)[VEC]) {
    const u32x4 w = *reinterpret_cast<const u32x4 *>(p);
    if constexpr (BF16) {
#pragma unroll
      for (int e = 0; e < 4; e++) {
        f[2 * e] = bf16_lo(w[e]);
        f[2 * e + 1] = bf16_hi(w[e]);
      }
    } else {
#pragma unroll
      for (int e = 0; e < 4; e++) f[e] = __uint_as_float(w[e]);
    }
  };

  float qv[QC][VEC];
#pragma unroll
  for (int g = 0; g < QC; g++) {
    if (g < nq) {
      const uint8_t *qp = reinterpret_cast<const uint8_t *>(a.q) +
                          ((int64_t)(u.b * a.Hq + hq0 + g) * D + ld * VEC) * ES;
      load_chunk(qp, qv[g]);
#pragma unroll
      for (int e = 0; e < VEC; e++) qv[g][e] *= a.sl2;
    } else {
#pragma unroll
      for (int e = 0; e < VEC; e++) qv[g][e] = 0.0f;
    }
  }
  float m[QC], l[QC], acc[QC][VEC];
#pragma unroll
  for (int g = 0; g < QC; g++) {
    m[g] = -INFINITY;
    l[g] = 0.0f;
#pragma unroll
    for (int e = 0; e < VEC; e++) acc[g][e] = 0.0f;
  }
  const int64_t head_off = (int64_t)u.h * D * ES + ld * 16;
  const int n_iter = (u.t_end - u.t_begin + TPI - 1) / TPI;
  for (int it = 0; it < n_iter; it++) {
    const int t = u.t_begin + it * TPI + lt;
    bool valid = t < u.t_end;
    float kf[VEC], vf[VEC];
#pragma unroll
    for (int e = 0; e < VEC; e++) kf[e] = vf[e] = 0.0f;
    if (valid) {
      const int32_t blk = a.ids[u.tab0 + t / kPageSize];
      if (blk < 0 || blk >= a.nblocks) {
        record_error(a.d_err, MKV_DEVERR_BLOCK);
        valid = false;
      } else {
        const int64_t off = (int64_t)blk * a.block_bytes + (t % kPageSize) * a.row_bytes + head_off;
        load_chunk(a.k_plane + off, kf);
        load_chunk(a.v_plane + off, vf);
      }
    }
#pragma unroll
    for (int g = 0; g < QC; g++) {
      if (g >= nq) break;
      float s = 0.0f;
#pragma unroll
      for (int e = 0; e < VEC; e++) s = fmaf(qv[g][e], kf[e], s);
#pragma unroll
      for (int o = LPT / 2; o >= 1; o >>= 1) s += __shfl_xor(s, o);
      if (valid) {
        const float mn = fmaxf(m[g], s);
        const float al = fast_exp2(m[g] - mn);
        const float p = fast_exp2(s - mn);
        l[g] = l[g] * al + p;
#pragma unroll
        for (int e = 0; e < VEC; e++) acc[g][e] = fmaf(p, vf[e], acc[g][e] * al);
        m[g] = mn;
      }
    }
  }
  // Merge the TPI token slots of the wave (lanes sharing ld).
#pragma unroll
  for (int o = LPT; o < 64; o <<= 1) {
#pragma unroll
    for (int g = 0; g < QC; g++) {
      if (g >= nq) break;
      const float mo = __shfl_xor(m[g], o);
      const float lo = __shfl_xor(l[g], o);
      const float M = fmaxf(m[g], mo);
      const float fa = m[g] == -INFINITY ? 0.0f : fast_exp2(m[g] - M);
      const float fb = mo == -INFINITY ? 0.0f : fast_exp2(mo - M);
      l[g] = l[g] * fa + lo * fb;
#pragma unroll
      for (int e = 0; e < VEC; e++) acc[g][e] = acc[g][e] * fa + __shfl_xor(acc[g][e], o) * fb;
      m[g] = M;
    }
  }
  if (lt != 0) return;
#pragma unroll
  for (int g = 0; g < QC; g++) {
    if (g >= nq) break;
    const int hq = hq0 + g;
    if (u.nsp == 1) {
      const float f = final_scale(m[g], l[g], a.zero_sink);
      uint8_t *op = reinterpret_cast<uint8_t *>(a.o) + ((int64_t)(u.b * a.Hq + hq) * D + ld * VEC) * ES;
      u32x4 w;
      if constexpr (BF16) {
#pragma unroll
        for (int e = 0; e < 4; e++) w[e] = pack_bf16x2(acc[g][2 * e] * f, acc[g][2 * e + 1] * f);
      } else {
#pragma unroll
        for (int e = 0; e < 4; e++) w[e] = __float_as_uint(acc[g][e] * f);
      }
      *reinterpret_cast<u32x4 *>(op) = w;
    } else {
      const int64_t idx = ((int64_t)u.b * a.Hq + hq) * a.S + u.split;
      float *wo = a.ws_o + idx * D + ld * VEC;
#pragma unroll
      for (int e = 0; e < VEC; e++) wo[e] = acc[g][e];
      if (ld == 0) {
        a.ws_ml[2 * idx] = m[g];
        a.ws_ml[2 * idx + 1] = l[g];
      }
    }
  }
}

// ---------------------------------------------------------------------------
// MFMA kernel (bf16).
// ---------------------------------------------------------------------------

// 4x4 transpose of 32-bit words inside each DPP quad (lanes 4k..4k+3): on
// return x[k] of lane r holds what x[r] of lane k held. Two butterfly stages
// (quad_perm [2,3,0,1] then [1,0,3,2]), each exchanging two words per lane.
__device__ __forceinline__ void quad_transpose(uint32_t (&x)[4], int lane) {
  const bool b1 = (lane >> 1) & 1, b0 = lane & 1;
  {
    const uint32_t t0 = b1 ? x[0] : x[2], t1 = b1 ? x[1] : x[3];
    const uint32_t u0 = (uint32_t)__builtin_amdgcn_mov_dpp((int)t0, 0x4E, 0xF, 0xF, false);
    const uint32_t u1 = (uint32_t)__builtin_amdgcn_mov_dpp((int)t1, 0x4E, 0xF, 0xF, false);
    if (b1) { x[0] = u0; x[1] = u1; } else { x[2] = u0; x[3] = u1; }
  }
  {
    const uint32_t t0 = b0 ? x[0] : x[1], t1 = b0 ? x[2] : x[3];
    const uint32_t u0 = (uint32_t)__builtin_amdgcn_mov_dpp((int)t0, 0xB1, 0xF, 0xF, false);
    const uint32_t u1 = (uint32_t)__builtin_amdgcn_mov_dpp((int)t1, 0xB1, 0xF, 0xF, false);
    if (b0) { x[0] = u0; x[2] = u1; } else { x[1] = u0; x[3] = u1; }
  }
}

template <int D>
__global__ void __launch_bounds__(256) attn_mfma_kernel(AttnArgs a) {
  static_assert(D % 32 == 0 && D <= 256, "unsupported head_dim");
  constexpr int NR = D / 32;  // 16-byte K loads and V loads per lane per block
  const int lane = threadIdx.x & 63;
  Unit u;
  if (!decode_unit(a, lane, u)) return;
  const int m16 = lane & 15, g4 = lane >> 4, a4 = m16 >> 2, rq = m16 & 3;
  const int q0 = u.qc * 16;
  const int nq = min(16, a.G - q0);

  // Q^T operand of S^T = K.Q^T: lane holds Q[q0+m16][32r + 8*g4 .. +8].
  bf16x8 qop[NR];
  {
    const uint16_t *qp = reinterpret_cast<const uint16_t *>(a.q) +
                         (int64_t)(u.b * a.Hq + u.h * a.G + q0 + min(m16, nq - 1)) * D;
#pragma unroll
    for (int r = 0; r < NR; r++) {
      u32x4 w = *reinterpret_cast<const u32x4 *>(qp + 32 * r + 8 * g4);
      if (m16 >= nq) w = u32x4{0, 0, 0, 0};
      qop[r] = __builtin_bit_cast(bf16x8, w);
    }
  }
  f32x4 O[NR][2];
#pragma unroll
  for (int s = 0; s < NR; s++) O[s][0] = O[s][1] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m = -INFINITY, l = 0.0f;

  const int64_t head_off = (int64_t)u.h * D * 2;
  const int64_t k_lane = (int64_t)m16 * a.row_bytes + head_off + 16 * g4;          // + 64*r
  const int64_t v_lane = (int64_t)(4 * g4 + rq) * a.row_bytes + head_off + 16 * a4;  // + 64*s
  const int j0 = u.t_begin / kPageSize, j1 = (u.t_end + kPageSize - 1) / kPageSize;

  for (int j = j0; j < j1; j++) {
    int32_t blk = a.ids[u.tab0 + j];
    const bool bad = blk < 0 || blk >= a.nblocks;
    if (bad) {
      if (lane == 0) record_error(a.d_err, MKV_DEVERR_BLOCK);
      continue;
    }
    const uint8_t *kb = a.k_plane + (int64_t)blk * a.block_bytes + k_lane;
    const uint8_t *vb = a.v_plane + (int64_t)blk * a.block_bytes + v_lane;
    u32x4 kq[NR], vq[NR];
#pragma unroll
    for (int r = 0; r < NR; r++) kq[r] = *reinterpret_cast<const u32x4 *>(kb + 64 * r);
#pragma unroll
    for (int s = 0; s < NR; s++) vq[s] = *reinterpret_cast<const u32x4 *>(vb + 64 * s);

    // Scores: lane holds S[token 4*g4+i][q = m16].
    f32x4 S = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int r = 0; r < NR; r++)
      S = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, kq[r]), qop[r], S, 0, 0, 0);
    const int tb = j * kPageSize;
    float x[4];
#pragma unroll
    for (int i = 0; i < 4; i++) x[i] = (tb + 4 * g4 + i < u.t_end) ? S[i] * a.sl2 : -INFINITY;
    float mloc = fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3]));
    mloc = fmaxf(mloc, __shfl_xor(mloc, 16));
    mloc = fmaxf(mloc, __shfl_xor(mloc, 32));
    const float mn = fmaxf(m, mloc);
    const float al = fast_exp2(m - mn);
    float p[4];
#pragma unroll
    for (int i = 0; i < 4; i++) p[i] = fast_exp2(x[i] - mn);
    l = l * al + ((p[0] + p[1]) + (p[2] + p[3]));
    m = mn;
#pragma unroll
    for (int s = 0; s < NR; s++) {
      O[s][0] *= al;
      O[s][1] *= al;
    }
    // P^T operand: tokens 4*g4 .. +4 for query m16, bf16.
    const uint32_t p01 = pack_bf16x2(p[0], p[1]), p23 = pack_bf16x2(p[2], p[3]);
    const i16x4 pb = __builtin_bit_cast(i16x4, (uint64_t)p01 | ((uint64_t)p23 << 32));
    // V rows past the context are zeroed (stale slots may hold any bits).
    const bool vvalid = tb + 4 * g4 + rq < u.t_end;
#pragma unroll
    for (int s = 0; s < NR; s++) {
      uint32_t w[4] = {vq[s][0], vq[s][1], vq[s][2], vq[s][3]};
      if (!vvalid) w[0] = w[1] = w[2] = w[3] = 0u;
      quad_transpose(w, lane);
      // w[k] = (V[4*g4+k][32s + 2*m16], V[4*g4+k][32s + 2*m16 + 1])
      const uint32_t e01 = (w[0] & 0xffffu) | (w[1] << 16), e23 = (w[2] & 0xffffu) | (w[3] << 16);
      const uint32_t o01 = (w[0] >> 16) | (w[1] & 0xffff0000u), o23 = (w[2] >> 16) | (w[3] & 0xffff0000u);
      const i16x4 ve = __builtin_bit_cast(i16x4, (uint64_t)e01 | ((uint64_t)e23 << 32));
      const i16x4 vo = __builtin_bit_cast(i16x4, (uint64_t)o01 | ((uint64_t)o23 << 32));
      O[s][0] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(ve, pb, O[s][0], 0, 0, 0);
      O[s][1] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(vo, pb, O[s][1], 0, 0, 0);
    }
  }
  l += __shfl_xor(l, 16);
  l += __shfl_xor(l, 32);
  if (m16 >= nq || m == -INFINITY) return;
  // Lane holds O[q0+m16][32s + 8*g4 + 2i + hh] = O[s][hh][i].
  const int hq = u.h * a.G + q0 + m16;
  if (u.nsp == 1) {
    const float f = final_scale(m, l, a.zero_sink);
    uint16_t *op = reinterpret_cast<uint16_t *>(a.o) + (int64_t)(u.b * a.Hq + hq) * D + 8 * g4;
#pragma unroll
    for (int s = 0; s < NR; s++) {
      u32x4 w;
#pragma unroll
      for (int i = 0; i < 4; i++) w[i] = pack_bf16x2(O[s][0][i] * f, O[s][1][i] * f);
      *reinterpret_cast<u32x4 *>(op + 32 * s) = w;
    }
  } else {
    const int64_t idx = ((int64_t)u.b * a.Hq + hq) * a.S + u.split;
    float *wo = a.ws_o + idx * D + 8 * g4;
#pragma unroll
    for (int s = 0; s < NR; s++) {
      f32x4 lo4 = {O[s][0][0], O[s][1][0], O[s][0][1], O[s][1][1]};
      f32x4 hi4 = {O[s][0][2], O[s][1][2], O[s][0][3], O[s][1][3]};
      *reinterpret_cast<f32x4 *>(wo + 32 * s) = lo4;
      *reinterpret_cast<f32x4 *>(wo + 32 * s + 4) = hi4;
    }
    if (g4 == 0) {
      a.ws_ml[2 * idx] = m;
      a.ws_ml[2 * idx + 1] = l;
    }
  }
}

// ---------------------------------------------------------------------------
// Split-K merge: one wave per (sequence, query head) with more than one split.
// ---------------------------------------------------------------------------
template <bool BF16>
__global__ void __launch_bounds__(256) merge_kernel(AttnArgs a, int D) {
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t row = (int64_t)blockIdx.x * 4 + wave;
  if (row >= (int64_t)a.B * a.Hq) return;
  const int b = (int)(row / a.Hq);
  const int ctx = a.ctx_lens[b];
  if (ctx < 1 || ctx > a.max_ctx) return;
  const int nsp = (ctx + a.split_tokens - 1) / a.split_tokens;
  if (nsp <= 1) return;
  const float *ml = a.ws_ml + 2 * row * a.S;
  float M = -INFINITY;
  for (int s = 0; s < nsp; s++) M = fmaxf(M, ml[2 * s]);
  float L = 0.0f;
  for (int s = 0; s < nsp; s++) L += ml[2 * s + 1] * fast_exp2(ml[2 * s] - M);
  const float f = final_scale(M, L, a.zero_sink);
  const float *wo = a.ws_o + row * a.S * D;
  for (int d = lane; d < D; d += 64) {
    float acc = 0.0f;
    for (int s = 0; s < nsp; s++) acc += wo[(int64_t)s * D + d] * fast_exp2(ml[2 * s] - M);
    acc *= f;
    if constexpr (BF16)
      reinterpret_cast<uint16_t *>(a.o)[row * D + d] = (uint16_t)f32_to_bf16_bits(acc);
    else
      reinterpret_cast<float *>(a.o)[row * D + d] = acc;
  }
}

// ---------------------------------------------------------------------------
// Host side.
// ---------------------------------------------------------------------------

static int choose_split(const Geom &g, int B, int max_ctx) {
  // Enough units to give every SIMD of the 256 CUs several waves, with at
  // least 128 tokens per split so partials stay small next to the KV bytes.
  const int64_t per_split_units = (int64_t)B * g.Hkv;
  const int64_t target_units = 4096;
  int64_t splits = std::max<int64_t>(1, (target_units + per_split_units - 1) / per_split_units);
  int64_t tokens = (max_ctx + splits - 1) / splits;
  tokens = std::max<int64_t>(128, (tokens + kPageSize - 1) / kPageSize * kPageSize);
  return (int)std::min<int64_t>(tokens, std::max(kPageSize, (max_ctx + kPageSize - 1) / kPageSize * kPageSize));
}

static uint64_t ws_bytes_for(const Geom &g, int B, int S) {
  if (S <= 1) return 0;
  const uint64_t rows = (uint64_t)B * g.Hq * S;
  const uint64_t ml = (rows * 8 + 255) / 256 * 256;
  return ml + rows * g.D * 4;
}

static bool mfma_applies(const Geom &g) {
  return g.dtype == MKV_DTYPE_BF16 && (g.D == 64 || g.D == 128 || g.D == 256);
}

}  // namespace mkv

using namespace mkv;

extern "C" int mkv_decode_attention_workspace_size(const mkv_pool *pool, int32_t num_seqs,
                                                   int32_t max_ctx_len, int32_t split_tokens,
                                                   uint64_t *out_bytes) {
  if (!pool || !out_bytes) return set_error(MKV_ERR_INVALID_ARGUMENT, "NULL argument");
  const Pool *p = reinterpret_cast<const Pool *>(pool);
  if (num_seqs < 0 || max_ctx_len < 0 || split_tokens < 0 || split_tokens % kPageSize)
    return set_error(MKV_ERR_INVALID_ARGUMENT, "bad sizes");
  const int st = split_tokens ? split_tokens : choose_split(p->g, num_seqs, max_ctx_len);
  const int S = max_ctx_len > 0 ? (max_ctx_len + st - 1) / st : 1;
  *out_bytes = ws_bytes_for(p->g, num_seqs, S);
  return MKV_OK;
}

extern "C" int mkv_decode_attention(mkv_pool *pool, int32_t layer, const void *d_q, void *d_o,
                                    const int32_t *d_block_indptr, const int32_t *d_block_ids,
                                    const int32_t *d_ctx_lens, int32_t num_seqs,
                                    int32_t max_ctx_len, float scale, uint32_t flags,
                                    int32_t split_tokens, void *d_workspace,
                                    uint64_t workspace_bytes, void *stream) {
  if (!pool) return set_error(MKV_ERR_INVALID_ARGUMENT, "pool is NULL");
  Pool *p = reinterpret_cast<Pool *>(pool);
  const Geom &g = p->g;
  if (layer < 0 || layer >= g.L)
    return set_error(MKV_ERR_INVALID_ARGUMENT, "layer %d out of range [0, %d)", layer, g.L);
  if (num_seqs < 0 || max_ctx_len < 0)
    return set_error(MKV_ERR_INVALID_ARGUMENT, "num_seqs and max_ctx_len must be >= 0");
  if (num_seqs == 0) return MKV_OK;
  if (max_ctx_len == 0) return set_error(MKV_ERR_INVALID_ARGUMENT, "max_ctx_len must be >= 1");
  if (!d_q || !d_o || !d_block_indptr || !d_block_ids || !d_ctx_lens)
    return set_error(MKV_ERR_INVALID_ARGUMENT, "NULL device pointer");
  if (!aligned16(d_q) || !aligned16(d_o))
    return set_error(MKV_ERR_INVALID_ARGUMENT, "q and o must be 16-byte aligned");
  if (g.D != 32 && g.D != 64 && g.D != 128 && g.D != 256)
    return set_error(MKV_ERR_INVALID_ARGUMENT, "decode attention supports head_dim 32/64/128/256 (pool has %d)", g.D);
  if (split_tokens < 0 || split_tokens % kPageSize)
    return set_error(MKV_ERR_INVALID_ARGUMENT, "split_tokens must be a multiple of %d", kPageSize);
  if (!(scale > 0.0f) || !std::isfinite(scale))
    return set_error(MKV_ERR_INVALID_ARGUMENT, "scale must be finite and > 0");
  const bool use_mfma = mfma_applies(g) && !(flags & MKV_ATTN_FORCE_VALU);
  if ((flags & MKV_ATTN_FORCE_MFMA) && !use_mfma)
    return set_error(MKV_ERR_INVALID_ARGUMENT, "MFMA kernel needs bf16 KV and head_dim 64/128/256");
  const int G = g.Hq / g.Hkv;
  const int qcw = use_mfma ? 16 : 8;
  const int nqc = (G + qcw - 1) / qcw;
  const int st = split_tokens ? split_tokens : choose_split(g, num_seqs, max_ctx_len);
  const int S = (max_ctx_len + st - 1) / st;
  const uint64_t need = ws_bytes_for(g, num_seqs, S);
  DeviceGuard guard(p->device);
  hipStream_t hs = reinterpret_cast<hipStream_t>(stream);
  void *ws = d_workspace;
  if (need) {
    if (ws) {
      if (workspace_bytes < need)
        return set_error(MKV_ERR_INVALID_ARGUMENT, "workspace of %llu bytes < %llu needed",
                         (unsigned long long)workspace_bytes, (unsigned long long)need);
    } else {
      if (p->ws_bytes < need) {
        // Earlier launches may still read the old buffer.
        MKV_CHECK_HIP(hipStreamSynchronize(hs));
        if (p->ws) MKV_CHECK_HIP(hipFree(p->ws));
        p->ws = nullptr;
        p->ws_bytes = 0;
        MKV_CHECK_HIP(hipMalloc(&p->ws, need));
        p->ws_bytes = need;
      }
      ws = p->ws;
    }
  }
  AttnArgs a;
  a.k_plane = p->data + (int64_t)layer * 2 * g.plane_bytes;
  a.v_plane = a.k_plane + g.plane_bytes;
  a.q = d_q;
  a.o = d_o;
  a.indptr = d_block_indptr;
  a.ids = d_block_ids;
  a.ctx_lens = d_ctx_lens;
  const uint64_t rows = (uint64_t)num_seqs * g.Hq * S;
  a.ws_ml = reinterpret_cast<float *>(ws);
  a.ws_o = ws ? reinterpret_cast<float *>(reinterpret_cast<uint8_t *>(ws) + (rows * 8 + 255) / 256 * 256)
              : nullptr;
  a.d_err = p->d_err;
  a.nblocks = g.nblocks;
  a.row_bytes = g.row_bytes;
  a.block_bytes = g.block_bytes;
  a.B = num_seqs;
  a.Hq = g.Hq;
  a.Hkv = g.Hkv;
  a.G = G;
  a.nqc = nqc;
  a.S = S;
  a.split_tokens = st;
  a.max_ctx = max_ctx_len;
  a.total_units = (int64_t)num_seqs * S * g.Hkv * nqc;
  a.sl2 = scale * kLog2e;
  a.zero_sink = (flags & MKV_ATTN_ZERO_SINK) ? 1 : 0;
  const int64_t wgs = (a.total_units + 3) / 4;
  if (wgs > INT32_MAX) return set_error(MKV_ERR_INVALID_ARGUMENT, "launch too large");
  const dim3 grid((unsigned)wgs), block(256);
  if (use_mfma) {
    switch (g.D) {
      case 64: hipLaunchKernelGGL(attn_mfma_kernel<64>, grid, block, 0, hs, a); break;
      case 128: hipLaunchKernelGGL(attn_mfma_kernel<128>, grid, block, 0, hs, a); break;
      default: hipLaunchKernelGGL(attn_mfma_kernel<256>, grid, block, 0, hs, a); break;
    }
    MKV_CHECK_LAUNCH("attn_mfma_kernel");
  } else if (g.dtype == MKV_DTYPE_BF16) {
    switch (g.D) {
      case 32: hipLaunchKernelGGL((attn_valu_kernel<32, true>), grid, block, 0, hs, a); break;
      case 64: hipLaunchKernelGGL((attn_valu_kernel<64, true>), grid, block, 0, hs, a); break;
      case 128: hipLaunchKernelGGL((attn_valu_kernel<128, true>), grid, block, 0, hs, a); break;
      default: hipLaunchKernelGGL((attn_valu_kernel<256, true>), grid, block, 0, hs, a); break;
    }
    MKV_CHECK_LAUNCH("attn_valu_kernel");
  } else {
    switch (g.D) {
      case 32: hipLaunchKernelGGL((attn_valu_kernel<32, false>), grid, block, 0, hs, a); break;
      case 64: hipLaunchKernelGGL((attn_valu_kernel<64, false>), grid, block, 0, hs, a); break;
      case 128: hipLaunchKernelGGL((attn_valu_kernel<128, false>), grid, block, 0, hs, a); break;
      default: hipLaunchKernelGGL((attn_valu_kernel<256, false>), grid, block, 0, hs, a); break;
    }
    MKV_CHECK_LAUNCH("attn_valu_kernel");
  }
  if (S > 1) {
    const int64_t mwgs = ((int64_t)num_seqs * g.Hq + 3) / 4;
    if (g.dtype == MKV_DTYPE_BF16)
      hipLaunchKernelGGL(merge_kernel<true>, dim3((unsigned)mwgs), dim3(256), 0, hs, a, g.D);
    else
      hipLaunchKernelGGL(merge_kernel<false>, dim3((unsigned)mwgs), dim3(256), 0, hs, a, g.D);
    MKV_CHECK_LAUNCH("merge_kernel");
  }
  return MKV_OK;
}
