// Fused pre-attention step for the tokens of one layer: q/k RMSNorm with
// weight (1 + w), partial NeoX RoPE, then the new K/V rows appended into the
// pool at their slots and the prepared q written out for attention.
//
// Follows inference-model-qwen/src/model.rs:369-392:
//   q  = qg[:, :, :, 0, :]               (q_proj output, q then gate per head, :371-374)
//   q  = RMSNorm(q), k = RMSNorm(k)      (forward4, :104-108: x * (mean(x^2) + eps)^-1/2 * (w + 1))
//   q  = RoPE(q, pos), k = RoPE(k, pos)  (apply_rope, :508-540: dims [0, rotary_dim) rotate the
//                                         first half against the second, the rest pass through)
//   k, v appended to the cache           (Tensor::cat, :390-392; here the slot scatter of mkv_append)
// A wave works on (token, head) rows: lane l holds EPL = max(1, D/64)
// contiguous elements of a row; the sum of squares is a wave reduction and
// the RoPE partner (d +- rotary_dim/2) comes from lane l +- rotary_dim/(2*EPL)
// by a shuffle.
// Arithmetic is f32 in the reference's operation order, with no contraction
// into FMAs; a bf16 pool gets one round-to-nearest-even per output element.
#include <cstring>

#include "mkv_internal.h"

namespace mkv {

struct PrepArgs {
  const uint8_t *q;        // [n][Hq][2][D] (q then gate) or [n][Hq][D] with MKV_PREP_PLAIN_Q
  const uint8_t *k;        // [n][Hkv][D]
  const uint8_t *v;        // [n][Hkv][D]
  const float *wq, *wk;    // [D] RMSNorm weights, applied as (1 + w)
  const float *inv_freq;   // [rotary_dim / 2]
  const int32_t *pos;      // [n]
  const int32_t *slots;    // [n]
  uint8_t *q_out;          // [n][Hq][D]
  uint8_t *k_plane, *v_plane;
  uint32_t *d_err;
  int64_t nslots, row_bytes;
  int32_t n, Hq, Hkv, rd, q_head_stride;  // q_head_stride in elements: 2*D or D
  float eps;
  bool norm;
};

template <int N> struct RawT;
template <> struct RawT<2> { typedef uint16_t type; };
template <> struct RawT<4> { typedef uint32_t type; };
template <> struct RawT<8> { typedef uint2 type; };
template <> struct RawT<16> { typedef uint4 type; };

// EPL consecutive elements at element index i0 (aligned to EPL) as f32.
template <int EPL, bool BF16>
__device__ __forceinline__ void load_row_part(const uint8_t *p, int i0, float (&x)[EPL]) {
  constexpr int ES = BF16 ? 2 : 4;
  typedef typename RawT<EPL * ES>::type R;
  const R r = *reinterpret_cast<const R *>(p + (int64_t)i0 * ES);
  if constexpr (BF16) {
    uint16_t h[EPL];
    __builtin_memcpy(h, &r, sizeof(r));
#pragma unroll
    for (int e = 0; e < EPL; e++) x[e] = __uint_as_float((uint32_t)h[e] << 16);
  } else {
    __builtin_memcpy(x, &r, sizeof(r));
  }
}

template <int EPL, bool BF16>
__device__ __forceinline__ void store_row_part(uint8_t *p, int i0, const float (&x)[EPL]) {
  constexpr int ES = BF16 ? 2 : 4;
  typedef typename RawT<EPL * ES>::type R;
  R r;
  if constexpr (BF16) {
    uint16_t h[EPL];
#pragma unroll
    for (int e = 0; e < EPL; e++) h[e] = (uint16_t)f32_to_bf16_bits(x[e]);
    __builtin_memcpy(&r, h, sizeof(r));
  } else {
    __builtin_memcpy(&r, x, sizeof(r));
  }
  *reinterpret_cast<R *>(p + (int64_t)i0 * ES) = r;
}

// Sum over the 64 lanes of a wave, the same value in every lane: DPP steps
// inside each 16-lane row (pairs, quads, half-rows, rows), then the four row
// sums read out and added as ((r0 + r1) + (r2 + r3)).
__device__ __forceinline__ float wave_sum(float v) {
  v += dpp_f<0xb1>(v);   // quad_perm [1,0,3,2]
  v += dpp_f<0x4e>(v);   // quad_perm [2,3,0,1]
  v += dpp_f<0x141>(v);  // row_half_mirror
  v += dpp_f<0x140>(v);  // row_mirror
  const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
  const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
  return (r0 + r1) + (r2 + r3);
}

// One workgroup (4 waves) per token. Every global load is issued first and
// unconditionally (out-of-range rows read a clamped, valid address and are
// discarded; absent weights and frequencies are replaced on the host by a
// valid dummy address), so that no load waits on another: the weights, the
// frequencies, one 16-byte chunk of the token's v rows per thread, each
// wave's kPrepRows head rows (q heads, then k heads), position and slot. Then the token's cos/sin table (rotary_dim/2 angles, shared by all its
// heads) goes to LDS, the v rows are stored, and each wave normalises,
// rotates and stores its rows.
constexpr int kPrepRows = 8;

template <int D, bool BF16>
__global__ void __launch_bounds__(256) qk_norm_rope_append_kernel(PrepArgs a) {
#pragma clang fp contract(off)
  constexpr int ES = BF16 ? 2 : 4;
  constexpr int EPL = D >= 64 ? D / 64 : 1;  // elements per lane
  constexpr int LANES = D / EPL;             // lanes holding a row: 64, or 32 when D == 32
  typedef typename RawT<EPL * ES>::type R;
  __shared__ float cs[2][D / 2];
  const int t = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // known wave-uniform: no divergent branches
  const bool active = lane < LANES;
  const int d0 = active ? lane * EPL : 0;  // idle lanes stay in bounds
  const int heads = a.Hq + a.Hkv;
  // Loads in the order their results are needed (the wait counter is in
  // order): weights, frequency and the token's v chunk, then the head rows.
  float wq[EPL], wk[EPL];
#pragma unroll
  for (int e = 0; e < EPL; e++) {
    wq[e] = a.wq[d0 + e];
    wk[e] = a.wk[d0 + e];
  }
  const int half = a.rd >> 1;
  const float f = a.inv_freq[min(tid, max(half - 1, 0))];
  const int vchunks = (int)(a.row_bytes >> 4);  // 16-byte chunks of the token's v rows
  const uint4 *vsrc = reinterpret_cast<const uint4 *>(a.v + (int64_t)t * a.row_bytes);
  const uint4 v0 = vsrc[min(tid, vchunks - 1)];
  R xr[kPrepRows];
  auto load_rows = [&](int h0) {
#pragma unroll
    for (int u = 0; u < kPrepRows; u++) {
      const int hh = min(h0 + u, heads - 1);
      const uint8_t *src = hh < a.Hq ? a.q + ((int64_t)t * a.Hq + hh) * a.q_head_stride * ES
                                     : a.k + ((int64_t)t * a.Hkv + (hh - a.Hq)) * D * ES;
      xr[u] = *reinterpret_cast<const R *>(src + (int64_t)d0 * ES);
    }
  };
  load_rows(wave * kPrepRows);
  const float p = (float)a.pos[t];
  const int64_t slot = a.slots[t];
  const bool slot_ok = slot >= 0 && slot < a.nslots;
  if (tid < half) {  // angle = pos * inv_freq[i], in f32 as the reference forms it
    float sn, c;
    sincosf(p * f, &sn, &c);
    cs[0][tid] = c;
    cs[1][tid] = sn;
  }
#pragma unroll
  for (int e = 0; e < EPL; e++) {  // RMSNorm weight is applied as (1 + w)
    wq[e] = a.norm ? wq[e] + 1.0f : 1.0f;
    wk[e] = a.norm ? wk[e] + 1.0f : 1.0f;
  }
  if (slot_ok) {  // v rows are appended as is
    uint4 *vdst = reinterpret_cast<uint4 *>(a.v_plane + slot * a.row_bytes);  // slot s = block s/16, row s%16
    if (tid < vchunks) vdst[tid] = v0;
    for (int i = tid + 256; i < vchunks; i += 256) vdst[i] = vsrc[i];
  } else if (tid == 0) {
    record_error(a.d_err, MKV_DEVERR_SLOT);
  }
  // Lane's RoPE partner (d +- half sits at the same e: half is a multiple of EPL).
  const int partner = (d0 < half ? lane + half / EPL : lane - half / EPL) & 63;
  __syncthreads();
  float c[EPL], sgn_s[EPL];
  bool rot[EPL];
#pragma unroll
  for (int e = 0; e < EPL; e++) {
    const int d = d0 + e;
    rot[e] = d < a.rd;
    const int i = d < half ? d : d - half;
    c[e] = rot[e] ? cs[0][i] : 1.0f;
    // first half x1*c - x2*s, second half x2*c + x1*s (a - b*s == a + b*(-s) exactly)
    sgn_s[e] = rot[e] ? (d < half ? -cs[1][i] : cs[1][i]) : 0.0f;
  }
  for (int h0 = wave * kPrepRows; h0 < heads; h0 += 4 * kPrepRows) {
    if (h0 != wave * kPrepRows) load_rows(h0);  // more than 4 * kPrepRows heads
    float out[kPrepRows][EPL];
#pragma unroll
    for (int u = 0; u < kPrepRows; u++) {
      const bool is_q = h0 + u < a.Hq;
      float x[EPL];
      if constexpr (BF16) {
        uint16_t hb[EPL];
        __builtin_memcpy(hb, &xr[u], sizeof(R));
#pragma unroll
        for (int e = 0; e < EPL; e++) x[e] = active ? __uint_as_float((uint32_t)hb[e] << 16) : 0.0f;
      } else {
        __builtin_memcpy(x, &xr[u], sizeof(R));
#pragma unroll
        for (int e = 0; e < EPL; e++) x[e] = active ? x[e] : 0.0f;
      }
      if (a.norm) {  // x * (mean(x^2) + eps)^-1/2, then * (1 + w)
        float ss = 0.0f;
#pragma unroll
        for (int e = 0; e < EPL; e++) ss += x[e] * x[e];
        const float inv = 1.0f / sqrtf(wave_sum(ss) / (float)D + a.eps);
#pragma unroll
        for (int e = 0; e < EPL; e++) x[e] = (x[e] * inv) * (is_q ? wq[e] : wk[e]);
      }
#pragma unroll
      for (int e = 0; e < EPL; e++) {
        const float other = __shfl(x[e], partner);
        out[u][e] = rot[e] ? x[e] * c[e] + other * sgn_s[e] : x[e];
      }
    }
    if (!active) continue;
#pragma unroll
    for (int u = 0; u < kPrepRows; u++) {
      const int hh = h0 + u;
      if (hh < a.Hq) {
        store_row_part<EPL, BF16>(a.q_out + ((int64_t)t * a.Hq + hh) * D * ES, d0, out[u]);
      } else if (hh < heads && slot_ok) {
        store_row_part<EPL, BF16>(a.k_plane + slot * a.row_bytes + (int64_t)(hh - a.Hq) * D * ES, d0, out[u]);
      }
    }
  }
}


// Vector form, one wave per token: lane holds VEC = 16 / ES contiguous
// elements of a head row (one 16-byte load), a row spans LPR = D / VEC lanes
// and one load instruction covers RPI = 64 / LPR rows. Used when
// rotary_dim / 2 is a multiple of VEC, so that a lane's elements all rotate
// or all pass through and their partners (d +- rotary_dim/2) sit at the same
// element index of lane +- rotary_dim / (2 VEC). Per wave: position and slot
// by scalar loads, then weights, frequencies, the token's first v chunk and
// kPrepLoads row loads, all issued before any is used; the token's cos/sin
// table goes to the wave's own LDS slice (no workgroup barrier: waves of a
// workgroup are independent tokens).
constexpr int kPrepTokens = 4;  // waves (tokens) per workgroup
constexpr int kPrepLoads = 4;   // row loads in flight per lane (8: 56.5 us, 4: 53.4, 2: 54.7 at 16k tokens)

template <int D, bool BF16>
__global__ void __launch_bounds__(256) prep_wave_kernel(PrepArgs a) {
#pragma clang fp contract(off)
  constexpr int ES = BF16 ? 2 : 4;
  constexpr int VEC = 16 / ES;
  constexpr int LPR = D / VEC;
  constexpr int RPI = 64 / LPR;
  __shared__ float cs[kPrepTokens][2][D / 2];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int t = blockIdx.x * kPrepTokens + wave;
  if (t >= a.n) return;  // wave-uniform
  typedef const __attribute__((address_space(4))) int32_t const_i32;
  const int pos = *(const const_i32 *)(a.pos + t);
  const int64_t slot = *(const const_i32 *)(a.slots + t);
  const bool slot_ok = slot >= 0 && slot < a.nslots;
  const int sub = lane % LPR, rin = lane / LPR;
  const int d0 = sub * VEC;
  const int heads = a.Hq + a.Hkv;
  const int half = a.rd >> 1;

  float wq[VEC], wk[VEC];
#pragma unroll
  for (int e = 0; e < VEC; e += 4) {
    const float4 q4 = *reinterpret_cast<const float4 *>(a.wq + d0 + e);
    const float4 k4 = *reinterpret_cast<const float4 *>(a.wk + d0 + e);
    wq[e] = q4.x, wq[e + 1] = q4.y, wq[e + 2] = q4.z, wq[e + 3] = q4.w;
    wk[e] = k4.x, wk[e + 1] = k4.y, wk[e + 2] = k4.z, wk[e + 3] = k4.w;
  }
  constexpr int NF = (D / 2 + 63) / 64;  // angles per lane
  float fr[NF];
#pragma unroll
  for (int j = 0; j < NF; j++) fr[j] = a.inv_freq[min(lane + 64 * j, max(half - 1, 0))];
  const int vchunks = (int)(a.row_bytes >> 4);
  const uint4 *vsrc = reinterpret_cast<const uint4 *>(a.v + (int64_t)t * a.row_bytes);
  const uint4 v0 = vsrc[min(lane, vchunks - 1)];
  uint4 xr[kPrepLoads];
  auto load_rows = [&](int r0) {
#pragma unroll
    for (int u = 0; u < kPrepLoads; u++) {
      const int r = min(r0 + u * RPI + rin, heads - 1);
      const uint8_t *src = r < a.Hq ? a.q + ((int64_t)t * a.Hq + r) * a.q_head_stride * ES
                                    : a.k + ((int64_t)t * a.Hkv + (r - a.Hq)) * D * ES;
      xr[u] = *reinterpret_cast<const uint4 *>(src + (int64_t)d0 * ES);
    }
  };
  load_rows(0);

  float *cw = cs[wave][0], *sw = cs[wave][1];
#pragma unroll
  for (int j = 0; j < NF; j++) {  // angle = pos * inv_freq[i], in f32 as the reference forms it
    const int i = lane + 64 * j;
    if (i < half) {
      float sn, c;
      sincosf((float)pos * fr[j], &sn, &c);
      cw[i] = c;
      sw[i] = sn;
    }
  }
#pragma unroll
  for (int e = 0; e < VEC; e++) {  // RMSNorm weight is applied as (1 + w)
    wq[e] = a.norm ? wq[e] + 1.0f : 1.0f;
    wk[e] = a.norm ? wk[e] + 1.0f : 1.0f;
  }
  if (slot_ok) {  // v rows are appended as is
    uint4 *vdst = reinterpret_cast<uint4 *>(a.v_plane + slot * a.row_bytes);  // slot s = block s/16, row s%16
    if (lane < vchunks) vdst[lane] = v0;
    for (int i = lane + 64; i < vchunks; i += 64) vdst[i] = vsrc[i];
  } else if (lane == 0) {
    record_error(a.d_err, MKV_DEVERR_SLOT);
  }
  // The table written by other lanes of this wave, read below.
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  const bool rot = d0 < a.rd;
  const int i0 = !rot ? 0 : d0 < half ? d0 : d0 - half;
  const int hl = half / VEC;  // partner distance in lanes
  const int partner = !rot ? lane : sub < hl ? lane + hl : lane - hl;
  float c[VEC], sg[VEC];
#pragma unroll
  for (int e = 0; e < VEC; e++) {
    c[e] = rot ? cw[i0 + e] : 1.0f;
    // first half x1*c - x2*s, second half x2*c + x1*s (a - b*s == a + b*(-s) exactly)
    sg[e] = rot ? (d0 < half ? -sw[i0 + e] : sw[i0 + e]) : 0.0f;
  }

  for (int r0 = 0; r0 < heads; r0 += kPrepLoads * RPI) {
    if (r0) load_rows(r0);  // more than kPrepLoads * RPI heads
#pragma unroll
    for (int u = 0; u < kPrepLoads; u++) {
      const int r = r0 + u * RPI + rin;
      const bool is_q = r < a.Hq;
      float x[VEC];
      if constexpr (BF16) {
        const uint32_t w32[4] = {xr[u].x, xr[u].y, xr[u].z, xr[u].w};
#pragma unroll
        for (int j = 0; j < 4; j++) {
          x[2 * j] = __uint_as_float(w32[j] << 16);
          x[2 * j + 1] = __uint_as_float(w32[j] & 0xffff0000u);
        }
      } else {
        x[0] = __uint_as_float(xr[u].x), x[1] = __uint_as_float(xr[u].y);
        x[2] = __uint_as_float(xr[u].z), x[3] = __uint_as_float(xr[u].w);
      }
      if (a.norm) {  // x * (mean(x^2) + eps)^-1/2, then * (1 + w)
        float ss = x[0] * x[0];
#pragma unroll
        for (int e = 1; e < VEC; e++) ss += x[e] * x[e];
        const float inv = 1.0f / sqrtf(row_sum<LPR>(ss) / (float)D + a.eps);
#pragma unroll
        for (int e = 0; e < VEC; e++) x[e] = (x[e] * inv) * (is_q ? wq[e] : wk[e]);
      }
      if (a.rd) {
#pragma unroll
        for (int e = 0; e < VEC; e++) {
          const float other = __shfl(x[e], partner);
          x[e] = rot ? x[e] * c[e] + other * sg[e] : x[e];
        }
      }
      uint4 o;
      if constexpr (BF16) {
        o.x = pack_bf16x2(x[0], x[1]), o.y = pack_bf16x2(x[2], x[3]);
        o.z = pack_bf16x2(x[4], x[5]), o.w = pack_bf16x2(x[6], x[7]);
      } else {
        o.x = __float_as_uint(x[0]), o.y = __float_as_uint(x[1]);
        o.z = __float_as_uint(x[2]), o.w = __float_as_uint(x[3]);
      }
      if (is_q) {
        *reinterpret_cast<uint4 *>(a.q_out + (((int64_t)t * a.Hq + r) * D + d0) * ES) = o;
      } else if (r < heads && slot_ok) {
        *reinterpret_cast<uint4 *>(a.k_plane + slot * a.row_bytes + ((int64_t)(r - a.Hq) * D + d0) * ES) = o;
      }
    }
  }
}

}  // namespace mkv

using namespace mkv;

extern "C" int mkv_qk_norm_rope_append(mkv_pool *pool, int32_t layer, const void *d_q, const void *d_k,
                                       const void *d_v, const float *d_q_norm_w, const float *d_k_norm_w,
                                       const float *d_inv_freq, int32_t rotary_dim, float eps,
                                       const int32_t *d_positions, const int32_t *d_slot_mapping,
                                       int32_t num_tokens, void *d_q_out, uint32_t flags, void *stream) {
  if (!pool) return set_error(MKV_ERR_INVALID_ARGUMENT, "NULL pool");
  Pool *p = reinterpret_cast<Pool *>(pool);
  const Geom &g = p->g;
  if (layer < 0 || layer >= g.L)
    return set_error(MKV_ERR_INVALID_ARGUMENT, "layer %d out of range [0, %d)", layer, g.L);
  if (flags & ~(uint32_t)(MKV_PREP_PLAIN_Q | MKV_PREP_NO_NORM))
    return set_error(MKV_ERR_INVALID_ARGUMENT, "unknown flags 0x%x", flags);
  if (num_tokens < 0) return set_error(MKV_ERR_INVALID_ARGUMENT, "num_tokens < 0");
  if (num_tokens == 0) return MKV_OK;
  const bool norm = !(flags & MKV_PREP_NO_NORM);
  if (!d_q || !d_k || !d_v || !d_positions || !d_slot_mapping || !d_q_out ||
      (norm && (!d_q_norm_w || !d_k_norm_w)) || (rotary_dim > 0 && !d_inv_freq))
    return set_error(MKV_ERR_INVALID_ARGUMENT, "NULL device pointer");
  if (!aligned16(d_q) || !aligned16(d_k) || !aligned16(d_v) || !aligned16(d_q_out))
    return set_error(MKV_ERR_INVALID_ARGUMENT, "q, k, v and q_out must be 16-byte aligned");
  if (g.D != 32 && g.D != 64 && g.D != 128 && g.D != 256)
    return set_error(MKV_ERR_INVALID_ARGUMENT, "head_dim must be 32/64/128/256 (pool has %d)", g.D);
  const int epl = g.D >= 64 ? g.D / 64 : 1;
  if (rotary_dim < 0 || rotary_dim > g.D || rotary_dim % (2 * epl))
    return set_error(MKV_ERR_INVALID_ARGUMENT, "rotary_dim %d must be in [0, %d] and a multiple of %d",
                     rotary_dim, g.D, 2 * epl);
  if (norm && !(eps >= 0.0f && eps < INFINITY))
    return set_error(MKV_ERR_INVALID_ARGUMENT, "eps must be finite and >= 0");
  PrepArgs a;
  a.q = static_cast<const uint8_t *>(d_q);
  a.k = static_cast<const uint8_t *>(d_k);
  a.v = static_cast<const uint8_t *>(d_v);
  // The kernel loads weights and frequencies unconditionally; where they are
  // absent it reads (and ignores) the start of the pool, which holds at least
  // page_size * head_dim elements.
  const float *dummy = reinterpret_cast<const float *>(p->data);
  a.wq = norm ? d_q_norm_w : dummy;
  a.wk = norm ? d_k_norm_w : dummy;
  a.inv_freq = rotary_dim > 0 ? d_inv_freq : dummy;
  a.pos = d_positions;
  a.slots = d_slot_mapping;
  a.q_out = static_cast<uint8_t *>(d_q_out);
  a.k_plane = p->data + (int64_t)layer * 2 * g.plane_bytes;
  a.v_plane = a.k_plane + g.plane_bytes;
  a.d_err = p->d_err;
  a.nslots = g.nblocks * kPageSize;
  a.row_bytes = g.row_bytes;
  a.n = num_tokens;
  a.Hq = g.Hq;
  a.Hkv = g.Hkv;
  a.rd = rotary_dim;
  a.q_head_stride = (flags & MKV_PREP_PLAIN_Q) ? g.D : 2 * g.D;
  a.eps = eps;
  a.norm = norm;
  DeviceGuard guard(p->device);
  hipStream_t hs = reinterpret_cast<hipStream_t>(stream);
  const bool bf = g.dtype == MKV_DTYPE_BF16;
  // The wave-per-token kernel needs rotary_dim / 2 to be a multiple of its
  // 16-byte vector (8 bf16 or 4 f32 elements) and reads the weights as
  // 16-byte vectors; other rotary widths, or unaligned weights, take the
  // workgroup-per-token kernel (1 to 4 elements per lane).
  const bool wave_form = rotary_dim % (2 * (bf ? 8 : 4)) == 0 && aligned16(a.wq) && aligned16(a.wk);
  const dim3 block(256);
  const dim3 grid(wave_form ? (unsigned)((num_tokens + kPrepTokens - 1) / kPrepTokens) : (unsigned)num_tokens);
#define MKV_PREP(DD)                                                                              \
  do {                                                                                            \
    if (wave_form && bf) hipLaunchKernelGGL((prep_wave_kernel<DD, true>), grid, block, 0, hs, a);  \
    else if (wave_form) hipLaunchKernelGGL((prep_wave_kernel<DD, false>), grid, block, 0, hs, a);  \
    else if (bf) hipLaunchKernelGGL((qk_norm_rope_append_kernel<DD, true>), grid, block, 0, hs, a); \
    else hipLaunchKernelGGL((qk_norm_rope_append_kernel<DD, false>), grid, block, 0, hs, a);        \
  } while (0)
  switch (g.D) {
    case 32: MKV_PREP(32); break;
    case 64: MKV_PREP(64); break;
    case 128: MKV_PREP(128); break;
    default: MKV_PREP(256); break;
  }
#undef MKV_PREP
  MKV_CHECK_LAUNCH("qk_norm_rope_append_kernel");
  return MKV_OK;
}

extern "C" int mkv_qk_norm_rope_append_host(mkv_pool *pool, int32_t layer, const void *d_q, const void *d_k,
                                            const void *d_v, const float *d_q_norm_w, const float *d_k_norm_w,
                                            const float *d_inv_freq, int32_t rotary_dim, float eps,
                                            const int32_t *h_positions, const uint32_t *h_slot_mapping,
                                            int32_t num_tokens, void *d_q_out, uint32_t flags, void *stream) {
  if (!pool) return set_error(MKV_ERR_INVALID_ARGUMENT, "NULL pool");
  Pool *p = reinterpret_cast<Pool *>(pool);
  int rc = check_host_slots(p->g, h_slot_mapping, num_tokens);
  if (rc) return rc;
  if (num_tokens == 0) return MKV_OK;
  if (!h_positions) return set_error(MKV_ERR_INVALID_ARGUMENT, "NULL positions");
  for (int32_t t = 0; t < num_tokens; t++)
    if (h_positions[t] < 0) return set_error(MKV_ERR_INVALID_ARGUMENT, "position[%d] = %d < 0", t, h_positions[t]);
  DeviceGuard guard(p->device);
  hipStream_t hs = reinterpret_cast<hipStream_t>(stream);
  // Every layer of a step passes the same positions and slots: staged once
  // per step, so a step of many layers does not cycle the staging ring (and
  // wait on the launch from a full ring earlier) at every layer.
  std::vector<int32_t> &st = p->stage_tmp;
  st.resize(2 * (size_t)num_tokens);
  std::memcpy(st.data(), h_positions, (size_t)num_tokens * 4);
  std::memcpy(st.data() + num_tokens, h_slot_mapping, (size_t)num_tokens * 4);
  MetaSlot *sl = nullptr;
  if ((rc = stage_cached(p, p->prep_cache, st.data(), st.size(), hs, &sl))) return rc;
  rc = mkv_qk_norm_rope_append(pool, layer, d_q, d_k, d_v, d_q_norm_w, d_k_norm_w, d_inv_freq, rotary_dim, eps,
                               sl->d, sl->d + num_tokens, num_tokens, d_q_out, flags, stream);
  const int rr = meta_release(sl, hs);
  return rc ? rc : rr;
}
