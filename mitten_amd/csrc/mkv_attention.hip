// Paged GQA/MQA decode attention, straight from the block pool.
//
// Arithmetic follows inference-model-qwen/src/model.rs:394-416: scores are
// (q.k) * scale with scale = head_dim^-0.5 (model.rs:298), softmax is the
// max-subtracted exponential, the output is p.v; query head h reads KV head
// h / (num_q_heads/num_kv_heads) (repeat_kv, model.rs:398-408). Softmax runs
// online in base 2 with f32 state; a sequence's context can be cut into
// segments whose unnormalised partials (m, l, o[D]) merge by log-sum-exp.
//
// Hot loop (one wave64 per (sequence segment, KV head, chunk of <= 16 query
// heads)), bf16 KV with head_dim 64/128/256:
//   S^T = K.Q^T  v_mfma_f32_16x16x32_bf16: each lane loads 16 B of one K row
//                straight into the A-operand layout (no LDS);
//   O^T = V^T.P^T v_mfma_f32_16x16x16_bf16: the S^T accumulator layout is
//                already the P^T operand layout; V is transposed in registers
//                by a 4x4 DPP quad transpose; the O^T accumulator keeps query
//                row q = lane%16, where that row's softmax state lives;
//   loads run three blocks deep in a register ring, so two blocks stay in
//   flight while one is computed; the running max moves only when it grows
//   by more than 2^8, so O is rarely rescaled.
// Other dtypes/shapes use a VALU loop: lanes split a token row into 16-byte
// chunks and reduce scores across the row's lanes with DPP steps; a batch of
// tokens inside one block is loaded while the previous batch is used.
//
// Two work decompositions:
//   split grid (mkv_decode_attention): units (sequence, split, KV head, query
//     chunk) over a grid sized by max_ctx_len; partials merge in merge_split.
//   plan (mkv_decode_attention_planned / mkv_decode_step): the host cuts the
//     concatenation of all sequences' blocks into equal pieces, one workgroup
//     per piece (all KV heads of the same blocks in one workgroup), so every
//     workgroup streams the same bytes whatever the context lengths;
//     sequences cut by a piece boundary merge in merge_planned (a second
//     launch: merging inside the first through an arrival counter needs an
//     agent-scope release/acquire per piece, which measured slower).
#include <algorithm>
#include <cmath>
#include <cstring>
#include <mutex>
#include <new>
#include <type_traits>
#include <vector>

#include "mkv_internal.h"

namespace mkv {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kRescaleSlack = 8.0f;  // log2 units: p <= 2^8 between rescales
constexpr int kQChunkMfma = 16;
constexpr int kQChunkValu = 8;       // query heads per wave on the per-head (VALU) kernels
constexpr int kQChunkValuSmall = 1;  // the same for launches too small to fill the device (see the plan)
constexpr int kRing = 3;       // MFMA loop: blocks loaded ahead + 1
constexpr int kBlockWeight = 8;    // plan: weight of one block in a piece ...
constexpr int kSwitchWeight = 12;  // ... and of a sequence start inside it (about 1.5 blocks)
constexpr int kFirstRoundWeight = 116;  // plan: cap of the first-dispatched pieces, percent
constexpr int kOddXcdWeight = 96;       // plan: cap of pieces dealt to odd-numbered XCDs, percent
constexpr int kMinPieceBlocks = 4;      // plan: fewest blocks per piece of a small cooperative plan ...
constexpr int kSmallPlanBlocks = 8;     // ... one with fewer blocks than this per resident workgroup
constexpr int kCoopRing = 3;   // register stages of the cooperative kernel (one less when
                               // its slots carry four Q loads per lane, or at head_dim 256,
                               // where three stages spilled registers)
constexpr int coop_ring(int D, int QL) { return D >= 256 || QL >= 4 ? kCoopRing - 1 : kCoopRing; }

// Kernel-side geometry and per-call arguments shared by every variant.
struct KArgs {
  const uint8_t *k_plane;  // layer's K plane
  const uint8_t *v_plane;  // layer's V plane
  uint8_t *k_plane_w;      // same planes, writable (fused append)
  uint8_t *v_plane_w;
  const void *q;           // [B][Hq][D]
  void *o;                 // [B][Hq][D]
  const uint8_t *new_k;    // fused append: [B][Hkv][D] or nullptr
  const uint8_t *new_v;
  const int32_t *indptr;
  const int32_t *ids;
  float *ws_ml;  // partial (m, l) pairs
  float *ws_o;   // partial o rows, f32 [D]
  uint32_t *d_err;
  int64_t nblocks;
  int64_t row_bytes;
  int64_t block_bytes;
  int32_t Hq, Hkv, G, nqc;
  float sl2;  // scale * log2(e)
  int32_t zero_sink;
  // Fused block-table gather (the per-head kernel of the planned path):
  // every row the attention reads is also stored at gather row
  // gtok0[b] * Hkv + h * ctx_b + t of gk / gv ([Hkv][ctx][D] per sequence).
  uint8_t *gk, *gv;
  const int32_t *gtok0;
};

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Normalisation factor of one row, including the optional phantom zero key
// (score 0, value 0) of the reference's Qwen cache (model.rs:210-213).
__device__ __forceinline__ float final_scale(float m, float l, int zero_sink) {
  if (zero_sink) {
    const float M = fmaxf(m, 0.0f);
    const float f = fast_exp2(m - M);
    return f / (l * f + fast_exp2(-M));
  }
  return 1.0f / l;
}

// Writes the step's new K/V row of (sequence, KV head) into its slot:
// block `blk`, row `row`. Lanes split the two D-element rows in 16 B chunks.
template <int D, int ES>
__device__ __forceinline__ void store_new_row(const KArgs &a, int lane, int b, int h, int32_t blk,
                                              int row) {
  constexpr int NC = D * ES / 16;
  const int64_t src = ((int64_t)b * a.Hkv + h) * D * ES;
  const int64_t dst = (int64_t)blk * a.block_bytes + (int64_t)row * a.row_bytes + (int64_t)h * D * ES;
  for (int c = lane; c < 2 * NC; c += 64) {
    const int kv = c >= NC, cc = c - kv * NC;
    const u32x4 w = *reinterpret_cast<const u32x4 *>((kv ? a.new_v : a.new_k) + src + 16 * cc);
    *reinterpret_cast<u32x4 *>((kv ? a.v_plane_w : a.k_plane_w) + dst + 16 * cc) = w;
  }
}

// Byte offset of the block that this workgroup's spare ring loads (past the
// end of its work) read: spreads them over the pool instead of one hot line.
__device__ __forceinline__ int64_t dummy_offset(const KArgs &a) {
  return (int64_t)(blockIdx.x % (uint32_t)min<int64_t>(a.nblocks, 1 << 30)) * a.block_bytes;
}

// One (sequence, KV head, query chunk) stretch of blocks [j0, j1) of a
// sequence with `ctx` tokens whose block table starts at ids + tab0.
struct Seg {
  int b, h, qc;
  int ctx;
  int j0, j1;
  const int32_t *table;  // ids + tab0
  const uint8_t *nk;     // fused append: new K row (this head) or nullptr
  const uint8_t *nv;
  int64_t gtok = 0;      // fused gather: the sequence's first token in the outputs
};

// ===========================================================================
// MFMA path (bf16).
// ===========================================================================

template <int D>
struct MState {
  f32x4 O[D / 32][2];
  float m, l;
};

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

// Q^T operand of S^T = K.Q^T: lane holds Q[q0 + lane%16][32r + 8*(lane/16) .. +8].
// Columns past the group repeat its last query; their results are never
// stored. (No select on the loaded words, so nothing waits for the load
// before the operand is used.)
template <int D>
__device__ __forceinline__ void mfma_load_q(const KArgs &a, int lane, int b, int h, int qc,
                                            bf16x8 (&qop)[D / 32]) {
  const int m16 = lane & 15, g4 = lane >> 4;
  const int q0 = qc * kQChunkMfma;
  const int nq = min(kQChunkMfma, a.G - q0);
  const uint16_t *qp = reinterpret_cast<const uint16_t *>(a.q) +
                       (int64_t)(b * a.Hq + h * a.G + q0 + min(m16, nq - 1)) * D;
#pragma unroll
  for (int r = 0; r < D / 32; r++)
    qop[r] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4 *>(qp + 32 * r + 8 * g4));
}

// One 16-token block whose first `nvalid` rows are context: scores, online
// softmax update, O += P.V.
template <int D>
__device__ __forceinline__ void mfma_block(const u32x4 (&kq)[D / 32], const u32x4 (&vq)[D / 32],
                                           int nvalid, bool bad, const bf16x8 (&qop)[D / 32],
                                           float sl2, int lane, MState<D> &st) {
  constexpr int NR = D / 32;
  const int g4 = lane >> 4, rq = lane & 3;
  f32x4 S = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int r = 0; r < NR; r++)
    S = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, kq[r]), qop[r], S, 0, 0, 0);
  // Lane holds S[token tb + 4*g4 + i][q = lane%16].
  float x[4];
#pragma unroll
  for (int i = 0; i < 4; i++) x[i] = (!bad && 4 * g4 + i < nvalid) ? S[i] * sl2 : -INFINITY;
  // The column-wide max (two cross-lane steps) only when a lane's own
  // scores pass the running max by the slack: the same rescale decisions.
  float mloc = fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3]));
  if (__ballot(mloc > st.m + kRescaleSlack)) {
    mloc = fmaxf(mloc, __shfl_xor(mloc, 16));
    mloc = fmaxf(mloc, __shfl_xor(mloc, 32));
    const bool need = mloc > st.m + kRescaleSlack;
    const float mn = need ? mloc : st.m;
    const float al = fast_exp2(st.m - mn);
    st.l *= al;
#pragma unroll
    for (int s = 0; s < NR; s++) {
      st.O[s][0] *= al;
      st.O[s][1] *= al;
    }
    st.m = mn;
  }
  float p[4];
#pragma unroll
  for (int i = 0; i < 4; i++) p[i] = fast_exp2(x[i] - st.m);
  st.l += (p[0] + p[1]) + (p[2] + p[3]);
  // P^T operand: tokens 4*g4 .. +4 of query lane%16, bf16.
  const uint32_t p01 = pack_bf16x2(p[0], p[1]), p23 = pack_bf16x2(p[2], p[3]);
  const i16x4 pb = __builtin_bit_cast(i16x4, (uint64_t)p01 | ((uint64_t)p23 << 32));
  // V rows past the context (or of a rejected block) are zeroed: stale slots
  // may hold any bit pattern, and 0 * NaN would poison the sum.
  const bool vvalid = !bad && 4 * g4 + rq < nvalid;
#pragma unroll
  for (int s = 0; s < NR; s++) {
    uint32_t w[4] = {vq[s][0], vq[s][1], vq[s][2], vq[s][3]};
    if (!vvalid) w[0] = w[1] = w[2] = w[3] = 0u;
    quad_transpose(w, lane);
    // w[k] = (V[4*g4+k][32s + 2*(lane%16)], V[4*g4+k][32s + 2*(lane%16) + 1])
    const uint32_t e01 = (w[0] & 0xffffu) | (w[1] << 16), e23 = (w[2] & 0xffffu) | (w[3] << 16);
    const uint32_t o01 = (w[0] >> 16) | (w[1] & 0xffff0000u), o23 = (w[2] >> 16) | (w[3] & 0xffff0000u);
    const i16x4 ve = __builtin_bit_cast(i16x4, (uint64_t)e01 | ((uint64_t)e23 << 32));
    const i16x4 vo = __builtin_bit_cast(i16x4, (uint64_t)o01 | ((uint64_t)o23 << 32));
    st.O[s][0] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(ve, pb, st.O[s][0], 0, 0, 0);
    st.O[s][1] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(vo, pb, st.O[s][1], 0, 0, 0);
  }
}

// Blocks [sg.j0, sg.j1) (at most 64) of one segment, loads kRing deep.
template <int D>
__device__ __forceinline__ void mfma_run(const KArgs &a, const Seg &sg, int lane,
                                         const bf16x8 (&qop)[D / 32], MState<D> &st) {
  constexpr int NR = D / 32;
  const int m16 = lane & 15, g4 = lane >> 4, a4 = m16 >> 2, rq = m16 & 3;
  const int n = sg.j1 - sg.j0;
  // Block ids of the stretch, one per lane; rejected ids read block 0 and
  // are masked.
  int32_t idv = lane < n ? sg.table[sg.j0 + lane] : 0;
  const bool badv = lane < n && (idv < 0 || idv >= a.nblocks);
  if (badv) {
    record_error(a.d_err, MKV_DEVERR_BLOCK);
    idv = 0;
  }
  const uint64_t badmask = __ballot(badv);
  const int64_t head_off = (int64_t)sg.h * D * 2;
  const int64_t k_lane = (int64_t)m16 * a.row_bytes + head_off + 16 * g4;          // + 64 r
  const int64_t v_lane = (int64_t)(4 * g4 + rq) * a.row_bytes + head_off + 16 * a4;  // + 64 s
  const int last_blk = (sg.ctx - 1) / kPageSize, new_row = (sg.ctx - 1) % kPageSize;
  u32x4 kb[kRing][NR], vb[kRing][NR];
  // Blocks past the stretch load the first 128 bytes of a block picked by the
  // workgroup index instead (so workgroups do not all hit the same lines):
  // the loads are issued unconditionally and the compiler's static wait
  // counts cover exactly the block about to be used.
  const int64_t spare = dummy_offset(a) + 16 * (lane & 7);
  auto issue = [&](u32x4 (&kd)[NR], u32x4 (&vd)[NR], int jj) {
    const bool live = jj < sg.j1;
    const int32_t blk = __builtin_amdgcn_readlane(idv, live ? jj - sg.j0 : 0);
    const uint8_t *kp = a.k_plane + (live ? (int64_t)blk * a.block_bytes + k_lane : spare);
    const uint8_t *vp = a.v_plane + (live ? (int64_t)blk * a.block_bytes + v_lane : spare);
    if (live && sg.nk && jj == last_blk) {  // the step's new row comes from the input
      if (m16 == new_row) kp = sg.nk + 16 * g4;
      if (4 * g4 + rq == new_row) vp = sg.nv + 16 * a4;
    }
#pragma unroll
    for (int r = 0; r < NR; r++) kd[r] = *reinterpret_cast<const u32x4 *>(kp + 64 * r);
#pragma unroll
    for (int s = 0; s < NR; s++) vd[s] = *reinterpret_cast<const u32x4 *>(vp + 64 * s);
  };
#pragma unroll
  for (int s = 0; s < kRing - 1; s++) issue(kb[s], vb[s], sg.j0 + s);
  for (int j = sg.j0; j < sg.j1; j += kRing) {
#pragma unroll
    for (int s = 0; s < kRing; s++) {
      const int jj = j + s;
      if (jj < sg.j1) {
        issue(kb[(s + kRing - 1) % kRing], vb[(s + kRing - 1) % kRing], jj + kRing - 1);
        const bool bad = (badmask >> (jj - sg.j0)) & 1;
        mfma_block<D>(kb[s], vb[s], min(kPageSize, sg.ctx - jj * kPageSize), bad, qop, a.sl2, lane, st);
      }
    }
  }
}

template <int D>
__device__ __forceinline__ void mfma_segment(const KArgs &a, const Seg &sg, int lane, MState<D> &st) {
  bf16x8 qop[D / 32];
  mfma_load_q<D>(a, lane, sg.b, sg.h, sg.qc, qop);
#pragma unroll
  for (int s = 0; s < D / 32; s++) st.O[s][0] = st.O[s][1] = f32x4{0.f, 0.f, 0.f, 0.f};
  st.m = -INFINITY;
  st.l = 0.0f;
  for (int c = sg.j0; c < sg.j1; c += 64) {
    Seg part = sg;
    part.j0 = c;
    part.j1 = min(sg.j1, c + 64);
    mfma_run<D>(a, part, lane, qop, st);
  }
  st.l += __shfl_xor(st.l, 16);
  st.l += __shfl_xor(st.l, 32);
}

// Lane holds O[q0 + lane%16][32s + 8*(lane/16) + c], c = 2i + hh, in O[s][hh][i].
template <int D>
__device__ __forceinline__ void mfma_store(const KArgs &a, const Seg &sg, int lane, const MState<D> &st,
                                           bool final, int64_t prow_base, int64_t prow_stride) {
  const int m16 = lane & 15, g4 = lane >> 4;
  const int q0 = sg.qc * kQChunkMfma;
  if (m16 >= min(kQChunkMfma, a.G - q0)) return;
  const int hq = sg.h * a.G + q0 + m16;
  if (final) {
    const float f = final_scale(st.m, st.l, a.zero_sink);
    uint16_t *op = reinterpret_cast<uint16_t *>(a.o) + (int64_t)(sg.b * a.Hq + hq) * D + 8 * g4;
#pragma unroll
    for (int s = 0; s < D / 32; s++) {
      u32x4 w;
#pragma unroll
      for (int i = 0; i < 4; i++) w[i] = pack_bf16x2(st.O[s][0][i] * f, st.O[s][1][i] * f);
      *reinterpret_cast<u32x4 *>(op + 32 * s) = w;
    }
  } else {
    const int64_t prow = prow_base + (int64_t)hq * prow_stride;
    float *wo = a.ws_o + prow * D + 8 * g4;
#pragma unroll
    for (int s = 0; s < D / 32; s++) {
      *reinterpret_cast<f32x4 *>(wo + 32 * s) = f32x4{st.O[s][0][0], st.O[s][1][0], st.O[s][0][1], st.O[s][1][1]};
      *reinterpret_cast<f32x4 *>(wo + 32 * s + 4) = f32x4{st.O[s][0][2], st.O[s][1][2], st.O[s][0][3], st.O[s][1][3]};
    }
    if (g4 == 0) *reinterpret_cast<float2 *>(a.ws_ml + 2 * prow) = make_float2(st.m, st.l);
  }
}

// ===========================================================================
// VALU path (any dtype).
// ===========================================================================

template <int D, bool BF16>
struct VTraits {
  static constexpr int ES = BF16 ? 2 : 4;
  static constexpr int VEC = 16 / ES;  // elements per 16 B chunk
  static constexpr int LPT = D / VEC;  // lanes per token row
  static constexpr int TPI = 64 / LPT; // tokens per wave iteration
  static_assert(LPT >= 1 && LPT <= 64 && (64 % LPT) == 0, "unsupported head_dim");
};

template <int D, bool BF16, int QC = kQChunkValu>
struct VState {
  float m[QC], l[QC], acc[QC][VTraits<D, BF16>::VEC];
};

template <bool BF16, int VEC>
__device__ __forceinline__ void load_chunk(const uint8_t *p, float (&f)[VEC]) {
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
}

// BATCHED: the U tokens of a lane's batch are scored first and enter the
// online softmax together (one rescale and U + 1 exponentials per query head,
// not 2U of each), at the cost of holding their V rows.
template <int D, bool BF16, int QC, bool BATCHED = false>
__device__ __forceinline__ void valu_segment(const KArgs &a, const Seg &sg, int lane, VState<D, BF16, QC> &st) {
  using T = VTraits<D, BF16>;
  constexpr int ES = T::ES, VEC = T::VEC, LPT = T::LPT, TPI = T::TPI;
  const int lt = lane / LPT, ld = lane % LPT;
  const int q0 = sg.qc * QC;
  const int nq = min(QC, a.G - q0);
  const int hq0 = sg.h * a.G + q0;
  float qv[QC][VEC];
#pragma unroll
  for (int g = 0; g < QC; g++) {
    if (g < nq) {
      load_chunk<BF16, VEC>(reinterpret_cast<const uint8_t *>(a.q) +
                                ((int64_t)(sg.b * a.Hq + hq0 + g) * D + ld * VEC) * ES,
                            qv[g]);
#pragma unroll
      for (int e = 0; e < VEC; e++) qv[g][e] *= a.sl2;
    } else {
#pragma unroll
      for (int e = 0; e < VEC; e++) qv[g][e] = 0.0f;
    }
    st.m[g] = -INFINITY;
    st.l[g] = 0.0f;
#pragma unroll
    for (int e = 0; e < VEC; e++) st.acc[g][e] = 0.0f;
  }
  const int64_t head_off = (int64_t)sg.h * D * ES + ld * 16;
  const int t_begin = sg.j0 * kPageSize, t_end = min(sg.ctx, sg.j1 * kPageSize);
  // Tokens go in batches of BT = TPI * U (U loads of K and of V per lane),
  // a batch inside one block: its block id is wave-uniform and comes by a
  // scalar load. The next batch's loads are issued before this batch is
  // used, so a block costs about one memory round trip instead of a block-id
  // load and a K/V load per TPI tokens.
  constexpr int U = (kPageSize / TPI) < 1 ? 1 : (kPageSize / TPI) > 4 ? 4 : kPageSize / TPI;
  constexpr int BT = TPI * U;
  static_assert(kPageSize % BT == 0, "a batch lies inside one block");
  typedef const __attribute__((address_space(4))) int32_t const_i32;
  const const_i32 *tab = (const const_i32 *)sg.table;
  const int nbat = t_end > t_begin ? (t_end - t_begin + BT - 1) / BT : 0;
  u32x4 kr[2][U], vr[2][U];
  bool okr[2];
  auto fetch = [&](u32x4 (&kd)[U], u32x4 (&vd)[U], bool &okb, int bi) {
    const int tb = t_begin + min(bi, nbat - 1) * BT;  // batches past the end re-read the last one
    const int32_t blk = tab[tb / kPageSize];           // uniform: a scalar load
    okb = blk >= 0 && blk < a.nblocks;
    const int64_t boff = (int64_t)(okb ? blk : 0) * a.block_bytes + head_off;
#pragma unroll
    for (int u = 0; u < U; u++) {
      const int t = tb + u * TPI + lt;
      const bool fresh = sg.nk && t == sg.ctx - 1;  // the step's new row, read from its input
      const int64_t off = boff + (int64_t)(t % kPageSize) * a.row_bytes;
      kd[u] = *reinterpret_cast<const u32x4 *>(fresh ? sg.nk + ld * 16 : a.k_plane + off);
      vd[u] = *reinterpret_cast<const u32x4 *>(fresh ? sg.nv + ld * 16 : a.v_plane + off);
    }
  };
  auto consume = [&](const u32x4 (&kd)[U], const u32x4 (&vd)[U], bool okb, int bi) {
    if (!okb && lane == 0) record_error(a.d_err, MKV_DEVERR_BLOCK);
    const int tb = t_begin + bi * BT;
    if constexpr (BATCHED) {
      float vfu[U][VEC], su[U][QC];
      bool vu[U];
#pragma unroll
      for (int u = 0; u < U; u++) {
        const int t = tb + u * TPI + lt;
        vu[u] = okb && t < t_end;
        if (a.gk && sg.qc == 0 && vu[u]) {  // fused gather: the row as read (the new row from its input)
          const int64_t go = ((sg.gtok * a.Hkv + (int64_t)sg.h * sg.ctx + t) * D) * ES + ld * 16;
          *reinterpret_cast<u32x4 *>(a.gk + go) = kd[u];
          *reinterpret_cast<u32x4 *>(a.gv + go) = vd[u];
        }
        float kf[VEC];
        if constexpr (BF16) {
#pragma unroll
          for (int e = 0; e < 4; e++) {
            kf[2 * e] = bf16_lo(kd[u][e]), kf[2 * e + 1] = bf16_hi(kd[u][e]);
            vfu[u][2 * e] = bf16_lo(vd[u][e]), vfu[u][2 * e + 1] = bf16_hi(vd[u][e]);
          }
        } else {
#pragma unroll
          for (int e = 0; e < 4; e++) kf[e] = __uint_as_float(kd[u][e]), vfu[u][e] = __uint_as_float(vd[u][e]);
        }
#pragma unroll
        for (int g = 0; g < QC; g++) {
          if (g >= nq) break;
          float sc = 0.0f;
#pragma unroll
          for (int e = 0; e < VEC; e++) sc = fmaf(qv[g][e], kf[e], sc);
          su[u][g] = row_sum<LPT>(sc);  // DPP steps within the token's lanes (no LDS round trips)
        }
      }
#pragma unroll
      for (int g = 0; g < QC; g++) {
        if (g >= nq) break;
        float mx = st.m[g];
#pragma unroll
        for (int u = 0; u < U; u++)
          if (vu[u]) mx = fmaxf(mx, su[u][g]);
        if (mx == -INFINITY) continue;  // nothing visible yet
        const float al = st.m[g] == -INFINITY ? 0.0f : fast_exp2(st.m[g] - mx);
        float pu[U], lsum = 0.0f;
#pragma unroll
        for (int u = 0; u < U; u++) {
          pu[u] = vu[u] ? fast_exp2(su[u][g] - mx) : 0.0f;
          lsum += pu[u];
        }
        st.l[g] = fmaf(st.l[g], al, lsum);
#pragma unroll
        for (int e = 0; e < VEC; e++) {
          float acc = st.acc[g][e] * al;
#pragma unroll
          for (int u = 0; u < U; u++) acc = fmaf(pu[u], vfu[u][e], acc);
          st.acc[g][e] = acc;
        }
        st.m[g] = mx;
      }
      return;
    }
#pragma unroll
    for (int u = 0; u < U; u++) {
      const int t = tb + u * TPI + lt;
      const bool valid = okb && t < t_end;
      if (a.gk && sg.qc == 0 && valid) {  // fused gather: the row as read (the new row from its input)
        const int64_t go = ((sg.gtok * a.Hkv + (int64_t)sg.h * sg.ctx + t) * D) * ES + ld * 16;
        *reinterpret_cast<u32x4 *>(a.gk + go) = kd[u];
        *reinterpret_cast<u32x4 *>(a.gv + go) = vd[u];
      }
      float kf[VEC], vf[VEC];
      if constexpr (BF16) {
#pragma unroll
        for (int e = 0; e < 4; e++) {
          kf[2 * e] = bf16_lo(kd[u][e]), kf[2 * e + 1] = bf16_hi(kd[u][e]);
          vf[2 * e] = bf16_lo(vd[u][e]), vf[2 * e + 1] = bf16_hi(vd[u][e]);
        }
      } else {
#pragma unroll
        for (int e = 0; e < 4; e++) kf[e] = __uint_as_float(kd[u][e]), vf[e] = __uint_as_float(vd[u][e]);
      }
#pragma unroll
      for (int g = 0; g < QC; g++) {
        if (g >= nq) break;
        float s = 0.0f;
#pragma unroll
        for (int e = 0; e < VEC; e++) s = fmaf(qv[g][e], kf[e], s);
        s = row_sum<LPT>(s);  // DPP steps within the token's lanes (no LDS round trips)
        if (valid) {
          const float mn = fmaxf(st.m[g], s);
          const float al = fast_exp2(st.m[g] - mn);
          const float p = fast_exp2(s - mn);
          st.l[g] = st.l[g] * al + p;
#pragma unroll
          for (int e = 0; e < VEC; e++) st.acc[g][e] = fmaf(p, vf[e], st.acc[g][e] * al);
          st.m[g] = mn;
        }
      }
    }
  };
  if (nbat > 0) {
    fetch(kr[0], vr[0], okr[0], 0);
    for (int bi = 0; bi < nbat; bi += 2) {
      fetch(kr[1], vr[1], okr[1], bi + 1);
      consume(kr[0], vr[0], okr[0], bi);
      if (bi + 1 < nbat) {
        fetch(kr[0], vr[0], okr[0], bi + 2);
        consume(kr[1], vr[1], okr[1], bi + 1);
      }
    }
  }
  // Merge the TPI token slots of the wave (lanes sharing ld).
#pragma unroll
  for (int o = LPT; o < 64; o <<= 1) {
#pragma unroll
    for (int g = 0; g < QC; g++) {
      if (g >= nq) break;
      const float mo = __shfl_xor(st.m[g], o);
      const float lo = __shfl_xor(st.l[g], o);
      const float M = fmaxf(st.m[g], mo);
      const float fa = st.m[g] == -INFINITY ? 0.0f : fast_exp2(st.m[g] - M);
      const float fb = mo == -INFINITY ? 0.0f : fast_exp2(mo - M);
      st.l[g] = st.l[g] * fa + lo * fb;
#pragma unroll
      for (int e = 0; e < VEC; e++) st.acc[g][e] = st.acc[g][e] * fa + __shfl_xor(st.acc[g][e], o) * fb;
      st.m[g] = M;
    }
  }
}

template <int D, bool BF16, int QC>
__device__ __forceinline__ void valu_store(const KArgs &a, const Seg &sg, int lane, const VState<D, BF16, QC> &st,
                                           bool final, int64_t prow_base, int64_t prow_stride) {
  using T = VTraits<D, BF16>;
  constexpr int ES = T::ES, VEC = T::VEC, LPT = T::LPT;
  if (lane >= LPT) return;
  const int ld = lane;
  const int q0 = sg.qc * QC;
  const int nq = min(QC, a.G - q0);
#pragma unroll
  for (int g = 0; g < QC; g++) {
    if (g >= nq) break;
    const int hq = sg.h * a.G + q0 + g;
    if (final) {
      const float f = final_scale(st.m[g], st.l[g], a.zero_sink);
      uint8_t *op = reinterpret_cast<uint8_t *>(a.o) + ((int64_t)(sg.b * a.Hq + hq) * D + ld * VEC) * ES;
      u32x4 w;
      if constexpr (BF16) {
#pragma unroll
        for (int e = 0; e < 4; e++) w[e] = pack_bf16x2(st.acc[g][2 * e] * f, st.acc[g][2 * e + 1] * f);
      } else {
#pragma unroll
        for (int e = 0; e < 4; e++) w[e] = __float_as_uint(st.acc[g][e] * f);
      }
      *reinterpret_cast<u32x4 *>(op) = w;
    } else {
      const int64_t prow = prow_base + (int64_t)hq * prow_stride;
      float *wo = a.ws_o + prow * D + ld * VEC;
#pragma unroll
      for (int e = 0; e < VEC; e += 4)
        *reinterpret_cast<f32x4 *>(wo + e) = f32x4{st.acc[g][e], st.acc[g][e + 1], st.acc[g][e + 2], st.acc[g][e + 3]};
      if (ld == 0) *reinterpret_cast<float2 *>(a.ws_ml + 2 * prow) = make_float2(st.m[g], st.l[g]);
    }
  }
}

// Processes one segment with the selected path and stores its result. QC:
// query heads per wave on the VALU path (KArgs::nqc must be ceil(G / QC)).
template <int D, bool BF16, bool MFMA, int QC = kQChunkValu>
__device__ __forceinline__ void run_segment(const KArgs &a, const Seg &sg, int lane, bool final,
                                            int64_t prow_base, int64_t prow_stride) {
  if constexpr (MFMA) {
    MState<D> st;
    mfma_segment<D>(a, sg, lane, st);
    mfma_store<D>(a, sg, lane, st, final, prow_base, prow_stride);
  } else {
    VState<D, BF16, QC> st;
    valu_segment<D, BF16, QC>(a, sg, lane, st);
    valu_store<D, BF16, QC>(a, sg, lane, st, final, prow_base, prow_stride);
  }
}

// Log-sum-exp merge of n partial rows: partial s has (m, l) at ml_at(s) and
// its D floats at o_at(s). Lane s holds partial s's (m, l); lane d holds dims
// d * DPL .. +DPL of every partial. Up to 16 partials merge in one memory
// round trip: all their loads are issued before the first use; weights
// exp2(m_s - M) are broadcast with readlane. More partials take further
// rounds of 16. Leaves the merged (M, L) (wave-uniform) and the lane's dims
// of the unnormalised row in acc; n = 0 leaves (-inf, 0, 0).
template <int D>
struct MergeVec {
  static constexpr int DPL = (D + 63) / 64;  // dims per lane (one vector load per partial row)
  typedef float type __attribute__((ext_vector_type(DPL)));
};

template <int D, class MlAt, class OAt>
__device__ __forceinline__ void merge_partials_state(int lane, int n, MlAt ml_at, OAt o_at, float &M, float &L,
                                                     typename MergeVec<D>::type &acc) {
  constexpr int DPL = MergeVec<D>::DPL;
  constexpr int SB = 16;
  typedef typename MergeVec<D>::type fvec;
  const int d0 = lane * DPL;
  const bool has = d0 < D;  // D = 32 leaves half the lanes idle
  acc = fvec{};
  M = -INFINITY;
  L = 0.0f;
  for (int s0 = 0; s0 < n; s0 += SB) {
    const int cnt = min(SB, n - s0);
    float2 ml = make_float2(-INFINITY, 0.0f);
    if (lane < cnt) ml = *reinterpret_cast<const float2 *>(ml_at(s0 + lane));
    fvec ov[SB];
#pragma unroll
    for (int i = 0; i < SB; i++) {
      ov[i] = fvec{};
      if (i < cnt && has) ov[i] = *reinterpret_cast<const fvec *>(o_at(s0 + i) + d0);
    }
    // Max and weighted sum over lanes 0..15 (the partials) by DPP row steps,
    // read from lane 0 (no LDS round trips).
    float mb = row16_max(ml.x);
    mb = __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, mb)));
    const float Mn = fmaxf(M, mb);
    const float carry = M == -INFINITY ? 0.0f : fast_exp2(M - Mn);
    const float w = (lane < cnt && ml.x != -INFINITY) ? fast_exp2(ml.x - Mn) : 0.0f;
    const float lw = row_sum<16>(ml.y * w);
    L = L * carry + __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, lw)));
    acc *= carry;
#pragma unroll
    for (int i = 0; i < SB; i++) {
      const float wi = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, w), i));
      acc += wi * ov[i];
    }
    M = Mn;
  }
}

// Row out_row of o from a merged (M, L, acc): the lane's DPL dims.
template <int D, bool BF16>
__device__ __forceinline__ void store_merged_row(const KArgs &a, int lane, float M, float L,
                                                 const typename MergeVec<D>::type &acc, int64_t out_row) {
  constexpr int DPL = MergeVec<D>::DPL;
  typedef typename MergeVec<D>::type fvec;
  const int d0 = lane * DPL;
  if (d0 >= D) return;
  const float f = final_scale(M, L, a.zero_sink);
  if constexpr (BF16) {
    uint16_t *op = reinterpret_cast<uint16_t *>(a.o) + out_row * D + d0;
    if constexpr (DPL == 1) {
      *op = (uint16_t)f32_to_bf16_bits(acc[0] * f);
    } else {
      uint32_t w[DPL / 2];
#pragma unroll
      for (int k = 0; k < DPL / 2; k++) w[k] = pack_bf16x2(acc[2 * k] * f, acc[2 * k + 1] * f);
      if constexpr (DPL == 2) *reinterpret_cast<uint32_t *>(op) = w[0];
      else *reinterpret_cast<uint2 *>(op) = make_uint2(w[0], w[1]);
    }
  } else {
    *reinterpret_cast<fvec *>(reinterpret_cast<float *>(a.o) + out_row * D + d0) = acc * f;
  }
}

template <int D, bool BF16, class MlAt, class OAt>
__device__ __forceinline__ void merge_partials(const KArgs &a, int lane, int n, MlAt ml_at, OAt o_at,
                                               int64_t out_row) {
  float M, L;
  typename MergeVec<D>::type acc;
  merge_partials_state<D>(lane, n, ml_at, o_at, M, L, acc);
  store_merged_row<D, BF16>(a, lane, M, L, acc, out_row);
}

// Partials ws[base + s*stride], s < n, of the kernel's workspace.
template <int D, bool BF16>
__device__ __forceinline__ void merge_rows(const KArgs &a, int lane, int64_t base, int64_t stride, int n,
                                           int64_t out_row) {
  merge_partials<D, BF16>(
      a, lane, n, [&](int s) { return a.ws_ml + 2 * (base + (int64_t)s * stride); },
      [&](int s) { return a.ws_o + (base + (int64_t)s * stride) * D; }, out_row);
}

// ===========================================================================
// Split-grid decomposition.
// ===========================================================================

struct SplitArgs {
  const int32_t *ctx_lens;
  int64_t total_units;
  int32_t B, S, split_tokens, max_ctx;
};

template <int D, bool BF16, bool MFMA>
__global__ void __launch_bounds__(256) attn_split_kernel(KArgs a, SplitArgs sp) {
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  int64_t id = (int64_t)blockIdx.x * 4 + wave;
  if (id >= sp.total_units) return;
  Seg sg;
  sg.qc = (int)(id % a.nqc);
  id /= a.nqc;
  sg.h = (int)(id % a.Hkv);
  id /= a.Hkv;
  const int split = (int)(id % sp.S);
  sg.b = (int)(id / sp.S);
  const bool first = split == 0 && sg.h == 0 && sg.qc == 0 && lane == 0;
  sg.ctx = sp.ctx_lens[sg.b];
  if (sg.ctx < 1 || sg.ctx > sp.max_ctx) {
    if (first) record_error(a.d_err, MKV_DEVERR_CTX);
    return;
  }
  const int t_begin = split * sp.split_tokens;
  if (t_begin >= sg.ctx) return;
  const int nsp = (sg.ctx + sp.split_tokens - 1) / sp.split_tokens;
  const int nb = (sg.ctx + kPageSize - 1) / kPageSize;
  const int tab0 = a.indptr[sg.b];
  if (tab0 < 0 || a.indptr[sg.b + 1] - tab0 < nb) {
    if (first) record_error(a.d_err, MKV_DEVERR_TABLE);
    return;
  }
  sg.table = a.ids + tab0;
  sg.j0 = t_begin / kPageSize;
  sg.j1 = min(nb, (t_begin + sp.split_tokens) / kPageSize);
  sg.nk = sg.nv = nullptr;
  run_segment<D, BF16, MFMA>(a, sg, lane, nsp == 1, ((int64_t)sg.b * a.Hq) * sp.S + split, sp.S);
}

// Extend attention on the decode kernels' per-sequence segments, for pools
// the MFMA extend kernel does not take (f32, head_dim 32, more than 16
// query heads per KV head): query token t of sequence b, at position p,
// is decode attention over keys 0..p through b's block table, with q and o
// rows addressed by t (a virtual sequence per token). One unit per
// (token, KV head, query-head chunk), whole context, final stores.
struct ExtSplitArgs {
  const int32_t *q_indptr;  // [B+1]
  const int32_t *ctx;       // [B] tokens in the cache, the chunk included
  int64_t total_units;      // tokens (upper bound) * Hkv * nqc
  int32_t B, max_ctx;
};

template <int D, bool BF16, bool MFMA>
__global__ void __launch_bounds__(256) attn_ext_split_kernel(KArgs a, ExtSplitArgs x) {
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  int64_t id = (int64_t)blockIdx.x * 4 + wave;
  if (id >= x.total_units) return;
  Seg sg;
  sg.qc = (int)(id % a.nqc);
  id /= a.nqc;
  sg.h = (int)(id % a.Hkv);
  const int t = (int)(id / a.Hkv);
  if (t >= x.q_indptr[x.B]) return;
  int lo = 0, hi = x.B - 1;  // the sequence holding token t: last b with q_indptr[b] <= t
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (x.q_indptr[mid] <= t) lo = mid;
    else hi = mid - 1;
  }
  const int b = lo;
  const int q0 = x.q_indptr[b], nq = x.q_indptr[b + 1] - q0, ctx = x.ctx[b];
  const bool first = t == q0 && sg.h == 0 && sg.qc == 0 && lane == 0;
  if (t < q0 || nq < 1 || nq > ctx || ctx > x.max_ctx) {
    if (first || (t < q0 && sg.h == 0 && sg.qc == 0 && lane == 0)) record_error(a.d_err, MKV_DEVERR_CTX);
    return;
  }
  const int nb = (ctx + kPageSize - 1) / kPageSize;
  const int tab0 = a.indptr[b];
  if (tab0 < 0 || a.indptr[b + 1] - tab0 < nb) {
    if (first) record_error(a.d_err, MKV_DEVERR_TABLE);
    return;
  }
  sg.b = t;
  sg.ctx = ctx - nq + (t - q0) + 1;  // keys 0..p
  sg.table = a.ids + tab0;
  sg.j0 = 0;
  sg.j1 = (sg.ctx + kPageSize - 1) / kPageSize;
  sg.nk = sg.nv = nullptr;
  run_segment<D, BF16, MFMA>(a, sg, lane, true, 0, 1);
}

template <int D, bool BF16>
__global__ void __launch_bounds__(256) merge_split_kernel(KArgs a, SplitArgs sp) {
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t row = (int64_t)blockIdx.x * 4 + wave;
  if (row >= (int64_t)sp.B * a.Hq) return;
  const int b = (int)(row / a.Hq);
  const int ctx = sp.ctx_lens[b];
  if (ctx < 1 || ctx > sp.max_ctx) return;
  const int nsp = (ctx + sp.split_tokens - 1) / sp.split_tokens;
  if (nsp <= 1) return;
  merge_rows<D, BF16>(a, lane, row * sp.S, 1, nsp, row);
}

// ===========================================================================
// Planned decomposition.
// ===========================================================================

struct PlanDev {
  const int32_t *ctx;         // [B] tokens attended
  const int32_t *seq_blk0;    // [B+1] first flattened block of each sequence
  const int32_t *piece_f0;    // [P+1] first flattened block of each piece (<= 64 per piece)
  const int32_t *piece_seq;   // [P] sequence holding each piece's first block
  const int32_t *seq_piece0;  // [B] first piece of each sequence
  const int32_t *seq_npiece;  // [B] pieces a sequence spans
  const int32_t *merge_seqs;  // [n_merge] sequences cut by a piece boundary
  const int32_t *tok0;        // [B+1] first token of each sequence (sum of the earlier contexts)
  const int32_t *flat_seq;    // [total] sequence of each flattened block
  const int32_t *flat_meta;   // [total] kMetaValid | kMetaLast | kMetaSingle bits
  int32_t *flat_id;           // [total] block id (written per step from the tables)
  int32_t B, P, total_blocks, n_merge;
};

// flat_meta bits of a flattened block.
constexpr int kMetaValid = 31;       // rows of the block inside the context (1..16)
constexpr int kMetaLast = 1 << 5;    // last block of its sequence (holds the new row)
constexpr int kMetaSingle = 1 << 6;  // its sequence lies inside one piece (final store)

// Once per plan build: flat_id[f] = block id of flattened block f from the
// caller's block tables; an id outside the pool or a short table becomes -1
// and is reported.
__global__ void __launch_bounds__(256) flatten_ids_kernel(PlanDev pd, const int32_t *__restrict__ indptr,
                                                          const int32_t *__restrict__ ids, int64_t nblocks,
                                                          uint32_t *__restrict__ d_err) {
  const int f = blockIdx.x * blockDim.x + threadIdx.x;
  if (f >= pd.total_blocks) return;
  const int b = pd.flat_seq[f];
  const int j = f - pd.seq_blk0[b];
  const int tab0 = indptr[b], tabn = indptr[b + 1] - tab0;
  int32_t id = -1;
  if (tab0 < 0 || j >= tabn) {
    record_error(d_err, MKV_DEVERR_TABLE);
  } else {
    id = ids[tab0 + j];
    if (id < 0 || id >= nblocks) {
      record_error(d_err, MKV_DEVERR_BLOCK);
      id = -1;
    }
  }
  pd.flat_id[f] = id;
}

// Writes the step's new K/V rows of KV head h for the piece's items that are
// the last block of their sequence (flattened items in lanes < n).
template <int D>
__device__ __forceinline__ void store_new_rows(const KArgs &a, int lane, int h, int32_t idv, int32_t seqv,
                                               int32_t metav, int n, bool badv) {
  uint64_t last = __ballot(lane < n && (metav & kMetaLast) && !badv);
  while (last) {
    const int k = __builtin_ctzll(last);
    last &= last - 1;
    store_new_row<D, 2>(a, lane, __builtin_amdgcn_readlane(seqv, k), h, __builtin_amdgcn_readlane(idv, k),
                        (__builtin_amdgcn_readlane(metav, k) & kMetaValid) - 1);
  }
}

// MFMA attention over one piece as a single block stream: the three-deep
// load ring runs across sequence boundaries, and the next sequence's Q is
// loaded while the current one is computed.
template <int D>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(D <= 128 ? 2 : 1)))
attn_stream_kernel(KArgs a, PlanDev pd) {
  constexpr int NR = D / 32;
  constexpr int RG = D >= 256 ? 2 : kRing;  // register stages (three spilled at head_dim 256)
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int hc = (int)blockIdx.y * (int)(blockDim.x >> 6) + wave;
  if (hc >= a.Hkv * a.nqc) return;
  const int h = hc / a.nqc, qc = hc % a.nqc;
  const int m16 = lane & 15, g4 = lane >> 4, a4 = m16 >> 2, rq = m16 & 3;
  const int p = blockIdx.x;
  const int f0 = pd.piece_f0[p];
  const int n = pd.piece_f0[p + 1] - f0;  // 1..64 items
  int32_t idv = -1, seqv = 0, metav = 0;
  if (lane < n) {
    idv = pd.flat_id[f0 + lane];
    seqv = pd.flat_seq[f0 + lane];
    metav = pd.flat_meta[f0 + lane];
  }
  const bool badv = lane < n && (idv < 0 || idv >= a.nblocks);
  if (badv) idv = 0;
  const uint64_t badmask = __ballot(badv);
  const int prev_seq = __shfl_up(seqv, 1);
  const uint64_t startmask = __ballot(lane < n && (lane == 0 || seqv != prev_seq));
  auto seq_at = [&](int k) { return __builtin_amdgcn_readlane(seqv, k); };
  auto next_start = [&](int k) {  // first segment start after item k, or 64
    const uint64_t m = k >= 63 ? 0 : (startmask >> (k + 1)) << (k + 1);
    return m ? __builtin_ctzll(m) : 64;
  };

  const int64_t head_off = (int64_t)h * D * 2;
  const int64_t k_lane = (int64_t)m16 * a.row_bytes + head_off + 16 * g4;
  const int64_t v_lane = (int64_t)(4 * g4 + rq) * a.row_bytes + head_off + 16 * a4;
  u32x4 kb[RG][NR], vb[RG][NR];
  // Items k >= n (past the piece) load the first 128 bytes of a block picked
  // by the workgroup index instead: every iteration then issues the same loads
  // with no branch around them, so the compiler's static wait counts cover
  // exactly the block about to be used rather than draining the whole ring.
  const int64_t spare = dummy_offset(a) + 16 * (lane & 7);
  auto issue = [&](u32x4 (&kd)[NR], u32x4 (&vd)[NR], int k) {
    const bool live = k < n;
    const int kk = live ? k : n - 1;
    const int32_t blk = __builtin_amdgcn_readlane(idv, kk);
    const int meta = __builtin_amdgcn_readlane(metav, kk);
    const uint8_t *kp = a.k_plane + (live ? (int64_t)blk * a.block_bytes + k_lane : spare);
    const uint8_t *vp = a.v_plane + (live ? (int64_t)blk * a.block_bytes + v_lane : spare);
    if (live && a.new_k && (meta & kMetaLast) && !((badmask >> k) & 1)) {
      // The sequence's new row is read from the input (it is written into
      // its slot after the loop).
      const int b = seq_at(k), row = (meta & kMetaValid) - 1;
      const int64_t src = ((int64_t)b * a.Hkv + h) * D * 2;
      if (m16 == row) kp = a.new_k + src + 16 * g4;
      if (4 * g4 + rq == row) vp = a.new_v + src + 16 * a4;
    }
#pragma unroll
    for (int r = 0; r < NR; r++) kd[r] = *reinterpret_cast<const u32x4 *>(kp + 64 * r);
#pragma unroll
    for (int r = 0; r < NR; r++) vd[r] = *reinterpret_cast<const u32x4 *>(vp + 64 * r);
  };

  bf16x8 qcur[NR], qnext[NR];
  int seg = seq_at(0);
  mfma_load_q<D>(a, lane, seg, h, qc, qcur);
  int nxt = next_start(0);
  if (nxt < n) mfma_load_q<D>(a, lane, seq_at(nxt), h, qc, qnext);
#pragma unroll
  for (int s = 0; s < RG - 1; s++) issue(kb[s], vb[s], s);

  MState<D> st;
  auto reset = [&]() {
#pragma unroll
    for (int s = 0; s < NR; s++) st.O[s][0] = st.O[s][1] = f32x4{0.f, 0.f, 0.f, 0.f};
    st.m = -INFINITY;
    st.l = 0.0f;
  };
  auto finish = [&](int b, int first_item) {
    st.l += __shfl_xor(st.l, 16);
    st.l += __shfl_xor(st.l, 32);
    Seg sg;
    sg.b = b;
    sg.h = h;
    sg.qc = qc;
    const bool single = __builtin_amdgcn_readlane(metav, first_item) & kMetaSingle;
    mfma_store<D>(a, sg, lane, st, single, (int64_t)(p + b) * a.Hq, 1);
  };
  reset();
  int seg_first = 0;
  auto stage = [&](int s, int k) {
    issue(kb[(s + RG - 1) % RG], vb[(s + RG - 1) % RG], k + RG - 1);
    if (k > 0 && ((startmask >> k) & 1)) {  // a new sequence starts at item k
      finish(seg, seg_first);
      reset();
      seg = seq_at(k);
      seg_first = k;
#pragma unroll
      for (int r = 0; r < NR; r++) qcur[r] = qnext[r];
      nxt = next_start(k);
      if (nxt < n) mfma_load_q<D>(a, lane, seq_at(nxt), h, qc, qnext);
    }
    const int meta = __builtin_amdgcn_readlane(metav, k);
    mfma_block<D>(kb[s], vb[s], meta & kMetaValid, (badmask >> k) & 1, qcur, a.sl2, lane, st);
  };
  // No branch around any stage of the main loop (a path that skipped one
  // would make the compiler's wait counts drain the ring); the last
  // n mod RG items run after it.
  const int nfull = n / RG;
  int k0 = 0;
  for (int it = 0; it < nfull; it++, k0 += RG) {
#pragma unroll
    for (int s = 0; s < RG; s++) stage(s, k0 + s);
  }
#pragma unroll
  for (int s = 0; s < RG - 1; s++)
    if (k0 + s < n) stage(s, k0 + s);
  finish(seg, seg_first);
  if (a.new_k && qc == 0) store_new_rows<D>(a, lane, h, idv, seqv, metav, n, badv);
}

// One workgroup per (piece, group of <= 4 (KV head, query chunk) waves). QC:
// query heads per wave on the VALU path.
template <int D, bool BF16, bool MFMA, int QC = kQChunkValu>
__global__ void __launch_bounds__(256) attn_planned_kernel(KArgs a, PlanDev pd) {
  constexpr int ES = BF16 ? 2 : 4;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int hc = (int)blockIdx.y * (int)(blockDim.x >> 6) + wave;
  if (hc >= a.Hkv * a.nqc) return;
  Seg sg;
  sg.h = hc / a.nqc;
  sg.qc = hc % a.nqc;
  const int p = blockIdx.x;
  int f = pd.piece_f0[p];
  const int f_end = pd.piece_f0[p + 1];
  int b = pd.piece_seq[p];
  for (; f < f_end; ++b) {
    const int sb = pd.seq_blk0[b], nb = pd.seq_blk0[b + 1] - sb;
    sg.b = b;
    sg.ctx = pd.ctx[b];
    sg.j0 = f - sb;
    sg.j1 = min(nb, f_end - sb);
    f = sb + sg.j1;
    const int tab0 = a.indptr[b];
    if (tab0 < 0 || a.indptr[b + 1] - tab0 < nb) {
      if (lane == 0) record_error(a.d_err, MKV_DEVERR_TABLE);
      continue;
    }
    sg.table = a.ids + tab0;
    sg.nk = sg.nv = nullptr;
    if (a.new_k && sg.j1 == nb) {
      // This piece holds the sequence's last block: the step's new row.
      const int32_t blk = sg.table[nb - 1];
      if (blk < 0 || blk >= a.nblocks) {
        if (lane == 0) record_error(a.d_err, MKV_DEVERR_BLOCK);
      } else {
        const int64_t src = ((int64_t)b * a.Hkv + sg.h) * D * ES;
        sg.nk = a.new_k + src;
        sg.nv = a.new_v + src;
        if (sg.qc == 0) store_new_row<D, ES>(a, lane, b, sg.h, blk, (sg.ctx - 1) % kPageSize);
      }
    }
    const bool single = pd.flat_meta[sb] & kMetaSingle;
    if (a.gk) sg.gtok = a.gtok0[b];
    run_segment<D, BF16, MFMA, QC>(a, sg, lane, single, (int64_t)(p + b) * a.Hq, 1);
  }
}

// A latency-bound step on the per-head kernel (few blocks for the device:
// the plan's small query chunks) without split-K partials: one workgroup of
// kSeqWaves waves per (sequence, KV head, query chunk); wave w takes the
// w-th contiguous share of the sequence's blocks, and the waves' softmax
// states merge through LDS into the final rows. No merge launch follows.
// Measured on the Qwen2.5-0.5B f32 step: 8 waves 0.255 ms, 16 waves 0.261 ms
// (and bf16 state spills past the 128 registers of 16 waves), 4 waves 0.327.
constexpr int kSeqWaves = 8;

template <int D, bool BF16, bool MFMA, int QC>
__global__ void __launch_bounds__(64 * kSeqWaves) attn_seq_kernel(KArgs a, PlanDev pd) {
  static_assert(!MFMA, "per-head path only");
  using T = VTraits<D, BF16>;
  constexpr int ES = T::ES, VEC = T::VEC, LPT = T::LPT;
  __shared__ float part[kSeqWaves][QC][2 + D];  // per wave and query head: m, l, unnormalised row
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int b = blockIdx.x;
  Seg sg;
  sg.b = b;
  sg.h = (int)blockIdx.y / a.nqc;
  sg.qc = (int)blockIdx.y % a.nqc;
  sg.ctx = pd.ctx[b];
  const int sb = pd.seq_blk0[b], nb = pd.seq_blk0[b + 1] - sb;
  const int tab0 = a.indptr[b];
  if (tab0 < 0 || a.indptr[b + 1] - tab0 < nb) {  // uniform over the workgroup
    if (threadIdx.x == 0 && sg.qc == 0) record_error(a.d_err, MKV_DEVERR_TABLE);
    return;
  }
  sg.table = a.ids + tab0;
  sg.j0 = (int)((int64_t)nb * wave / kSeqWaves);
  sg.j1 = (int)((int64_t)nb * (wave + 1) / kSeqWaves);
  sg.nk = sg.nv = nullptr;
  if (a.new_k && sg.j0 < sg.j1 && sg.j1 == nb) {
    // This wave holds the sequence's last block: the step's new row.
    const int32_t blk = sg.table[nb - 1];
    if (blk < 0 || blk >= a.nblocks) {
      if (lane == 0) record_error(a.d_err, MKV_DEVERR_BLOCK);
    } else {
      const int64_t src = ((int64_t)b * a.Hkv + sg.h) * D * ES;
      sg.nk = a.new_k + src;
      sg.nv = a.new_v + src;
      if (sg.qc == 0) store_new_row<D, ES>(a, lane, b, sg.h, blk, (sg.ctx - 1) % kPageSize);
    }
  }
  if (a.gk) sg.gtok = a.gtok0[b];
  VState<D, BF16, QC> st;
  valu_segment<D, BF16, QC, true>(a, sg, lane, st);  // an empty share leaves m = -inf, l = 0, row 0
  const int q0 = sg.qc * QC;
  const int nq = min(QC, a.G - q0);
  if (lane < LPT) {
#pragma unroll
    for (int g = 0; g < QC; g++) {
      if (g >= nq) break;
      part[wave][g][0] = st.m[g];
      part[wave][g][1] = st.l[g];
#pragma unroll
      for (int e = 0; e < VEC; e++) part[wave][g][2 + lane * VEC + e] = st.acc[g][e];
    }
  }
  __syncthreads();
  // Wave g merges query head q0 + g: lane ld the dims ld*VEC .. +VEC.
  if (wave >= nq || lane >= LPT) return;
  const int g = wave;
  float M = -INFINITY;
#pragma unroll
  for (int w = 0; w < kSeqWaves; w++) M = fmaxf(M, part[w][g][0]);
  float L = 0.0f, acc[VEC];
#pragma unroll
  for (int e = 0; e < VEC; e++) acc[e] = 0.0f;
#pragma unroll
  for (int w = 0; w < kSeqWaves; w++) {
    const float mw = part[w][g][0];
    const float f = mw == -INFINITY ? 0.0f : fast_exp2(mw - M);
    L = fmaf(part[w][g][1], f, L);
#pragma unroll
    for (int e = 0; e < VEC; e++) acc[e] = fmaf(part[w][g][2 + lane * VEC + e], f, acc[e]);
  }
  const float f = final_scale(M, L, a.zero_sink);
  const int hq = sg.h * a.G + q0 + g;
  uint8_t *op = reinterpret_cast<uint8_t *>(a.o) + ((int64_t)(b * a.Hq + hq) * D + lane * VEC) * ES;
  u32x4 wv;
  if constexpr (BF16) {
#pragma unroll
    for (int e = 0; e < 4; e++) wv[e] = pack_bf16x2(acc[2 * e] * f, acc[2 * e + 1] * f);
  } else {
#pragma unroll
    for (int e = 0; e < 4; e++) wv[e] = __float_as_uint(acc[e] * f);
  }
  *reinterpret_cast<u32x4 *>(op) = wv;
}

// ---- LDS-fed MFMA block (cooperative kernel) -------------------------------
//
// Same online-softmax step as mfma_block, but V^T comes straight from the
// LDS tile through ds_read_tr16_b64 (gfx950 transpose read): within each group
// of 16 lanes, lane i receives element (i mod 4) of the 8 bytes read by lane
// 4j + i/4, for j = 0..3. Lane 4j + q of group g reads token row 4g + j at
// dims 16n + 4q .. +3, so lane i of group g receives V[4g + j][16n + i] for
// j = 0..3: the A operand of O^T[16n..+16][q] += V^T . P^T. O^T tile n holds
// O[q = lane%16][16n + 4*(lane/16) + i] in O[n][i].
template <int D>
struct MStateT {
  f32x4 O[D / 16];
  float m, l;
};

typedef short i16x4s __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) i16x4s lds_i16x4;

template <int D>
__device__ __forceinline__ void mfma_block_t(const u32x4 (&kq)[D / 32], const uint8_t *tv,
                                             const int (&v_rd)[D / 16], int nvalid, bool bad,
                                             const bf16x8 (&qop)[D / 32], float sl2, int lane,
                                             MStateT<D> &st) {
  constexpr int NR = D / 32, NT = D / 16;
  const int g4 = lane >> 4;
  f32x4 S = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int r = 0; r < NR; r++)
    S = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, kq[r]), qop[r], S, 0, 0, 0);
  // Lane holds S[token 4*g4 + i][q = lane%16]. Only a sequence's last block
  // (or a rejected one) has rows past the context.
  const bool partial = bad || nvalid < kPageSize;
  float x[4];
#pragma unroll
  for (int i = 0; i < 4; i++) x[i] = S[i] * sl2;
  if (partial) {
#pragma unroll
    for (int i = 0; i < 4; i++)
      if (bad || 4 * g4 + i >= nvalid) x[i] = -INFINITY;
  }
  // The column-wide max (two cross-lane steps) only when a lane's own
  // scores pass the running max by the slack: the same rescale decisions.
  float mloc = fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3]));
  if (__ballot(mloc > st.m + kRescaleSlack)) {
    mloc = fmaxf(mloc, __shfl_xor(mloc, 16));
    mloc = fmaxf(mloc, __shfl_xor(mloc, 32));
    const bool need = mloc > st.m + kRescaleSlack;
    const float mn = need ? mloc : st.m;
    const float al = fast_exp2(st.m - mn);
    st.l *= al;
#pragma unroll
    for (int n = 0; n < NT; n++) st.O[n] *= al;
    st.m = mn;
  }
  float p[4];
#pragma unroll
  for (int i = 0; i < 4; i++) p[i] = fast_exp2(x[i] - st.m);
  st.l += (p[0] + p[1]) + (p[2] + p[3]);
  const uint32_t p01 = pack_bf16x2(p[0], p[1]), p23 = pack_bf16x2(p[2], p[3]);
  const i16x4 pb = __builtin_bit_cast(i16x4, (uint64_t)p01 | ((uint64_t)p23 << 32));
  // V rows past the context (or of a rejected block) are zeroed: stale slots
  // may hold any bit pattern, and 0 * NaN would poison the sum.
  uint32_t vm0 = ~0u, vm1 = ~0u;
  if (partial) {
    const int t0 = 4 * g4;
    vm0 = (bad || t0 >= nvalid ? 0u : 0xffffu) | (bad || t0 + 1 >= nvalid ? 0u : 0xffff0000u);
    vm1 = (bad || t0 + 2 >= nvalid ? 0u : 0xffffu) | (bad || t0 + 3 >= nvalid ? 0u : 0xffff0000u);
  }
#pragma unroll
  for (int n = 0; n < NT; n++) {
    const i16x4s raw = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4 *)(tv + v_rd[n]));
    uint64_t w = __builtin_bit_cast(uint64_t, raw);
    if (partial) w &= (uint64_t)vm0 | ((uint64_t)vm1 << 32);
    st.O[n] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(i16x4, w), pb, st.O[n], 0, 0, 0);
  }
}

// Stores one (sequence, KV head) result of the LDS-fed path: the final bf16
// rows, or f32 partial rows plus (m, l) for the split-K merge.
template <int D>
__device__ __forceinline__ void mfma_store_t(const KArgs &a, int b, int h, int lane, const MStateT<D> &st,
                                             bool final, int64_t prow_base) {
  const int m16 = lane & 15, g4 = lane >> 4;
  if (m16 >= min(kQChunkMfma, a.G)) return;
  const int hq = h * a.G + m16;
  if (final) {
    const float f = final_scale(st.m, st.l, a.zero_sink);
    uint16_t *op = reinterpret_cast<uint16_t *>(a.o) + (int64_t)(b * a.Hq + hq) * D + 4 * g4;
#pragma unroll
    for (int n = 0; n < D / 16; n++) {
      const uint2 w = make_uint2(pack_bf16x2(st.O[n][0] * f, st.O[n][1] * f),
                                 pack_bf16x2(st.O[n][2] * f, st.O[n][3] * f));
      *reinterpret_cast<uint2 *>(op + 16 * n) = w;
    }
  } else {
    const int64_t prow = prow_base + hq;
    float *wo = a.ws_o + prow * D + 4 * g4;
#pragma unroll
    for (int n = 0; n < D / 16; n++) *reinterpret_cast<f32x4 *>(wo + 16 * n) = st.O[n];
    if (g4 == 0) *reinterpret_cast<float2 *>(a.ws_ml + 2 * prow) = make_float2(st.m, st.l);
  }
}

// Cooperative variant of the stream kernel for workgroups that hold every
// KV head (num_kv_heads 1, 2 or 4 and at most 16 query heads per KV head).
// The workgroup reads each block as whole token rows of all heads, every
// wave load instruction one contiguous KiB (non-temporal when NT), which the
// memory system serves faster than per-head 64-byte row pieces. NT = false
// (MKV_ATTN_CACHED_LOADS) keeps the blocks in the caches: with a prefix
// shared by 256 sequences its blocks are then re-read from the MALL
// (10.7 -> 7.2 ms per 28-layer step), while a batch of distinct blocks
// streams 13% slower that way (102 -> 117 us per layer). A block passes
// through a double-buffered LDS tile (one barrier per block); each wave then
// reads its head's MFMA operands from it. The Q rows of a sequence ride in
// the same load ring as its first block in the piece and are kept in LDS, so
// nothing waits for them at a sequence boundary.
//
// LDS layout: tile rows of RB = W*D*2 bytes with 16-byte chunk c of row r
// stored at chunk c ^ swz(r), swz(r) = 2 * (r / rows-per-512-bytes) (2r for
// rows of 512 bytes or more). Measured with the LDS bank-conflict counter on
// gfx950, for the K reads (ds_read_b128: rows m16, chunks g4 + 4r) and the
// transposed V reads (ds_read_b64_tr_b16: 4 rows x 4 half-chunks per 16
// lanes) of 512- and 1024-byte rows: no conflicts (the previous swizzle, row
// bits 0-1 and 2-3 swapped: both reads 2-way). Q rows (D*2 bytes, [Hq][D]
// order) use chunk c ^ (row mod chunks-per-row).
__device__ __forceinline__ int tile_swz(int row, int cpr) {
  const int rpw = cpr >= 32 ? 1 : 32 / cpr;  // rows per 512 bytes
  return (2 * (row / rpw)) & (cpr - 1);
}

// The extend kernel's one-head tiles (rows of 2 * head_dim bytes) take a
// swizzle per tile, each measured free of bank conflicts at head_dim 64, 128
// and 256 (no single row swizzle is, for both reads, at all three):
//   K tile: chunk c of row r at c ^ r          (ds_read_b128 reads)
//   V tile: chunk c of row r at c ^ v_swz(r)   (ds_read_b64_tr_b16 reads),
// v_swz linear over GF(2) in the row's four bits, which flip chunk bits by
// 2, 4, 11 and 1. With the decode swizzle above both reads were 2-way
// conflicted at head_dim 128 (47% of the kernel's LDS cycles stalled).
__device__ __forceinline__ int ext_k_swz(int row, int cpr) { return row & (cpr - 1); }
__device__ __forceinline__ int ext_v_swz(int row, int cpr) {
  const int s = ((row & 1) << 1) ^ ((row & 2) << 1) ^ (((row >> 2) & 1) * 11) ^ ((row >> 3) & 1);
  return s & (cpr - 1);
}

template <int D, int W, int QL, int R, bool NT>
__global__ void __launch_bounds__(64 * W) __attribute__((amdgpu_waves_per_eu(D <= 128 ? 2 : 1)))
attn_coop_kernel(KArgs a, PlanDev pd) {
  constexpr int NR = D / 32;
  constexpr int RB = W * D * 2;          // tile row bytes (all KV heads)
  constexpr int CPR = RB / 16;           // 16-byte chunks per tile row
  constexpr int BLK = 16 * RB;           // K (or V) bytes of one block
  constexpr int CH = BLK / 1024 / W;     // 1 KiB loads per wave per block, K (and V)
  constexpr int CPQ = D / 8;             // 16-byte chunks per Q row
  constexpr int QCAP = QL * 64 * W * 16; // Q bytes the ring slots can carry
  static_assert(BLK % (1024 * W) == 0, "block must split into 1 KiB loads per wave");
  __shared__ __attribute__((aligned(16))) uint8_t tiles[2][2][BLK];  // [buffer][K|V]
  __shared__ __attribute__((aligned(16))) uint8_t qtile[QCAP];
  const int lane = threadIdx.x & 63;
  const int h = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave = KV head
  const int m16 = lane & 15, g4 = lane >> 4, a4 = m16 >> 2, rq = m16 & 3;
  const int p = blockIdx.x;
  const int f0 = pd.piece_f0[p];
  const int n = pd.piece_f0[p + 1] - f0;  // 1..64 items
  const int qchunks = a.Hq * CPQ;        // Q chunks of one sequence (<= QCAP / 16)
  int32_t idv = -1, seqv = 0, metav = 0;
  if (lane < n) {
    idv = pd.flat_id[f0 + lane];
    seqv = pd.flat_seq[f0 + lane];
    metav = pd.flat_meta[f0 + lane];
  }
  const bool badv = lane < n && (idv < 0 || idv >= a.nblocks);
  if (badv) idv = 0;
  const uint64_t badmask = __ballot(badv);
  const int prev_seq = __shfl_up(seqv, 1);
  const uint64_t startmask = __ballot(lane < n && (lane == 0 || seqv != prev_seq));
  auto seq_at = [&](int k) { return __builtin_amdgcn_readlane(seqv, k); };

  // Ring slot: wave h holds bytes [(i*W + h)*1024 + 16*lane, +16) of the
  // block's K and V (i < CH), and Q chunks (i*W + h)*64 + lane (i < QL) of the
  // sequence when the item starts one. Items k >= n load the first 128 bytes
  // of a block picked by the workgroup index instead (so workgroups do not all
  // hit the same lines), and Q of items that start no sequence a fixed span:
  // every iteration issues the same loads, so the compiler's static wait
  // counts cover exactly the block about to be used.
  u32x4 kb[R][CH], vb[R][CH], qb[R][QL];
  const int64_t spare = dummy_offset(a);
  auto issue = [&](u32x4 (&kd)[CH], u32x4 (&vd)[CH], u32x4 (&qd)[QL], int k) {
    const bool live = k < n;
    const int kk = live ? k : n - 1;
    const int32_t blk = __builtin_amdgcn_readlane(idv, kk);
    const int meta = __builtin_amdgcn_readlane(metav, kk);
    const uint8_t *kbase = a.k_plane + (live ? (int64_t)blk * a.block_bytes : spare);
    const uint8_t *vbase = a.v_plane + (live ? (int64_t)blk * a.block_bytes : spare);
    const bool fresh = live && a.new_k && (meta & kMetaLast) && !((badmask >> k) & 1);
    const int b = seq_at(kk), row_new = (meta & kMetaValid) - 1;
#pragma unroll
    for (int i = 0; i < CH; i++) {
      const int off = live ? (i * W + h) * 1024 + 16 * lane : 16 * (lane & 7);
      const uint8_t *kp = kbase + off, *vp = vbase + off;
      if (fresh && off / RB == row_new) {  // the step's new row comes from the input
        kp = a.new_k + (int64_t)b * RB + off % RB;
        vp = a.new_v + (int64_t)b * RB + off % RB;
      }
      if constexpr (NT) {
        kd[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(kp));
        vd[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(vp));
      } else {
        kd[i] = *reinterpret_cast<const u32x4 *>(kp);
        vd[i] = *reinterpret_cast<const u32x4 *>(vp);
      }
    }
    const bool qload = live && ((startmask >> k) & 1);
    const uint8_t *qbase = static_cast<const uint8_t *>(a.q) + (qload ? (int64_t)b * a.Hq * D * 2 : 0);
#pragma unroll
    for (int i = 0; i < QL; i++) {
      const int c = (i * W + h) * 64 + lane;
      // (The fallback offset stays lane-varying: a uniform one invites the
      // compiler to branch around the load, which costs a full wait.)
      qd[i] = *reinterpret_cast<const u32x4 *>(qbase + 16 * (qload ? min(c, qchunks - 1) : (lane & 7)));
    }
  };

  MStateT<D> st;
  auto reset = [&]() {
#pragma unroll
    for (int n = 0; n < D / 16; n++) st.O[n] = f32x4{0.f, 0.f, 0.f, 0.f};
    st.m = -INFINITY;
    st.l = 0.0f;
  };
  auto finish = [&](int b, int first_item) {
    st.l += __shfl_xor(st.l, 16);
    st.l += __shfl_xor(st.l, 32);
    const bool single = __builtin_amdgcn_readlane(metav, first_item) & kMetaSingle;
    mfma_store_t<D>(a, b, h, lane, st, single, (int64_t)(p + b) * a.Hq);
  };
  // LDS byte offsets of this lane's operands: K (16 B, r < NR), V^T
  // transpose reads (8 B, tile n < D/16: token row 4*g4 + (lane%16)/4, dims
  // 16n + 4*(lane%4)), Q (16 B, r < NR).
  int k_rd[NR], v_rd[D / 16], q_rd[NR];
  const int qrow = h * a.G + min(m16, a.G - 1);
  const int vrow = 4 * g4 + a4, vq4 = rq;
#pragma unroll
  for (int r = 0; r < NR; r++) {
    k_rd[r] = m16 * RB + (((h * D / 8 + g4 + 4 * r) ^ tile_swz(m16, CPR)) << 4);
    q_rd[r] = qrow * D * 2 + (((4 * r + g4) ^ (qrow & (CPQ - 1))) << 4);
  }
#pragma unroll
  for (int n = 0; n < D / 16; n++)
    v_rd[n] = vrow * RB + (((h * D / 8 + 2 * n + (vq4 >> 1)) ^ tile_swz(vrow, CPR)) << 4) + 8 * (vq4 & 1);
  bf16x8 qop[NR];

#pragma unroll
  for (int s = 0; s < R - 1; s++) issue(kb[s], vb[s], qb[s], s);
  reset();
  int seg = seq_at(0), seg_first = 0;
  // One item: load item k + R - 1 into the slot freed last, stage slot s
  // (item k) in LDS, compute.
  auto stage = [&](int s, int k) {
    issue(kb[(s + R - 1) % R], vb[(s + R - 1) % R], qb[(s + R - 1) % R], k + R - 1);
    uint8_t *tk = tiles[k & 1][0], *tv = tiles[k & 1][1];
#pragma unroll
    for (int i = 0; i < CH; i++) {
      const int off = (i * W + h) * 1024 + 16 * lane;
      const int row = off / RB, c = (off % RB) >> 4;
      const int t = row * RB + ((c ^ tile_swz(row, CPR)) << 4);
      *reinterpret_cast<u32x4 *>(tk + t) = kb[s][i];
      *reinterpret_cast<u32x4 *>(tv + t) = vb[s][i];
    }
    __syncthreads();
    if ((startmask >> k) & 1) {  // item k starts a sequence: its Q goes to LDS
      // Every wave has passed the barrier above, so none still reads the
      // previous sequence's Q.
#pragma unroll
      for (int i = 0; i < QL; i++) {
        const int c = (i * W + h) * 64 + lane;
        if (c < qchunks) {
          const int row = c / CPQ, cc = c % CPQ;
          *reinterpret_cast<u32x4 *>(qtile + row * D * 2 + ((cc ^ (row & (CPQ - 1))) << 4)) = qb[s][i];
        }
      }
      if (k > 0) {
        // The previous sequence's result. Its stores go after the wait on
        // this item's Q above: the wait's count assumes no stores, and
        // would otherwise also wait for the loads issued this stage.
        finish(seg, seg_first);
        reset();
        seg = seq_at(k);
        seg_first = k;
      }
      __syncthreads();
#pragma unroll
      for (int r = 0; r < NR; r++) qop[r] = *reinterpret_cast<const bf16x8 *>(qtile + q_rd[r]);
    }
    u32x4 kq[NR];
#pragma unroll
    for (int r = 0; r < NR; r++) kq[r] = *reinterpret_cast<const u32x4 *>(tk + k_rd[r]);
    const int meta = __builtin_amdgcn_readlane(metav, k);
    mfma_block_t<D>(kq, tv, v_rd, meta & kMetaValid, (badmask >> k) & 1, qop, a.sl2, lane, st);
  };
  // The main loop has no branch around any stage: a path that skipped one
  // would make the compiler's wait counts assume fewer loads in flight and
  // drain the ring. The last n mod R items run after it.
  const int nfull = n / R;
  int k0 = 0;
  for (int it = 0; it < nfull; it++, k0 += R) {
#pragma unroll
    for (int s = 0; s < R; s++) stage(s, k0 + s);
  }
#pragma unroll
  for (int s = 0; s < R - 1; s++)
    if (k0 + s < n) stage(s, k0 + s);
  finish(seg, seg_first);
  if (a.new_k) store_new_rows<D>(a, lane, h, idv, seqv, metav, n, badv);
}

// ===========================================================================
// Extend (chunked prefill) attention: causal attention of each sequence's
// newest q_len tokens over its whole cache (the chunk's own K/V already
// appended), the seq_q > 1 path of inference-model-qwen/src/model.rs:410-416
// with the causal mask of model.rs:542-555 (a key at position j is visible to
// the query at position p iff j <= p).
//
// One workgroup per (query tile of 16 or 32 positions, KV head, sequence,
// key-range split); per 16-position sub-tile, W/TP >= G waves, wave g
// computing query head h*G + g for the sub-tile's positions (the MFMA column
// dimension). The workgroup streams the head's K/V blocks 0..(last tile
// position)/16 (its split's share of them) through a double-buffered LDS
// tile (rows of one head: D*2 bytes; K and V tiles each with their own
// bank-conflict-free swizzle), loaded cooperatively one step of two blocks
// ahead; scores, online softmax and the V^T transpose reads follow the
// decode kernel, with the causal mask applied on blocks that reach past a
// sub-tile's first position. Steps whose keys every query of the workgroup
// sees (all but the last one or two of a tile) run a lean form: block ids
// staged in LDS and checked once, wave-uniform load bases, no masks, and the
// PV product on one full-rate 16x16x32 MFMA per 16 dims over both blocks.
// ===========================================================================

// Extend kernel: two blocks (32 keys) per softmax step, steps loaded one
// ahead (two blocks in flight). Measured against one block per step with a
// 4-step ring: equal at head_dim 128, 3.5% faster at 256; four blocks per
// step raise the register count past two workgroups per CU.
constexpr int kExtKB = 2;  // blocks per softmax step of the extend kernel
constexpr int kExtR = 2;   // ring depth (steps) of the extend kernel
// Block ids a workgroup stages in LDS for its unmasked steps (16k keys);
// a longer key range takes the scalar table reads throughout.
constexpr int kExtIdCap = 1024;

struct ExtArgs {
  const int32_t *q_indptr;  // [B+1] query tokens of each sequence in q / o; null: one sequence of
                            // v_nq queries over v_ctx tokens of the table a.ids (no indptr, no ctx)
  const int32_t *ctx;       // [B] tokens in the cache, the chunk included
  int32_t B, max_ctx;
  int32_t tiles, per_xcd;   // query tiles per sequence; logical workgroups per XCD
  int32_t splits;           // key-range splits per (tile, KV head, sequence); > 1: f32 partials + merge
  int32_t max_q;            // max_q_len: with splits, partial rows exist for B * max_q tokens
  int32_t causal;           // 0: every query sees all ctx keys (a shared prefix's decode queries)
  int32_t partial;          // 1: f32 partials whatever the split count, merged by the caller
  int32_t v_nq, v_ctx;      // the one sequence when q_indptr is null
  int32_t hgroups;          // workgroups per (tile, KV head): each takes W / TP consecutive query heads
};

// Workgroups are dealt to the 8 XCDs round-robin by linear index. The
// launch has 8 * per_xcd workgroups; workgroup L becomes logical index
// (L % 8) * per_xcd + L / 8, so each XCD receives a contiguous run of
// logical indices: the query tiles of one (sequence, KV head) share that
// XCD's L2 while they stream the same K/V. Logical index = (tiles - 1 -
// tile) + tiles * (group + hgroups * (head + Hkv * (sequence + B * split)));
// false for the padding past the last one. `h` returns head * hgroups +
// group. The last tile of a chunk attends the most keys,
// so a sequence's tiles start longest first (causal 2k-token prompts: 518 ->
// 487 us), leaving the short ones for the tail.
__device__ __forceinline__ bool ext_tile(const ExtArgs &e, int Hkv, int &t, int &h, int &b, int &sp) {
  const int L = blockIdx.x;
  const int logical = (L & 7) * e.per_xcd + (L >> 3);
  const int heads = Hkv * e.hgroups;
  const int per_split = e.tiles * heads * e.B;
  if (logical >= per_split * e.splits) return false;
  const int r = logical % per_split;
  sp = logical / per_split;
  t = e.tiles - 1 - r % e.tiles;
  h = (r / e.tiles) % heads;
  b = r / (e.tiles * heads);
  return true;
}

template <int D, int W, int KB, int R, int TP>
__global__ void __launch_bounds__(64 * W) attn_extend_kernel(KArgs a, ExtArgs e) {
  constexpr int NR = D / 32, NT = D / 16;
  constexpr int RB = D * 2;                           // LDS tile row: one head's K or V row
  constexpr int CPR = RB / 16;                        // 16-byte chunks per tile row
  constexpr int TILE = 16 * RB;
  constexpr int BCH = 2 * 16 * CPR;                   // chunks of K + V of one block
  constexpr int NCH = KB * BCH;                       // chunks of one step (KB blocks)
  constexpr int LPL = (NCH + 64 * W - 1) / (64 * W);  // loads per lane per step
  static_assert(R % 2 == 0, "even ring: stage s of an unrolled round uses LDS buffer s & 1");
  constexpr int WG = W / TP;                          // waves per 16-position sub-tile
  static_assert(W % TP == 0, "whole sub-tiles per workgroup");
  __shared__ __attribute__((aligned(16))) uint8_t tiles[2][KB][2][TILE];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int m16 = lane & 15, g4 = lane >> 4, a4 = m16 >> 2, rq = m16 & 3;
  int t, hx, b, sp;
  if (!ext_tile(e, a.Hkv, t, hx, b, sp)) return;
  const int h = hx / e.hgroups, hg = hx % e.hgroups;  // KV head; group of W / TP query heads
  const bool virt = e.q_indptr == nullptr;  // one sequence; the host checked its table length
  const int q0 = virt ? 0 : e.q_indptr[b], nq = virt ? e.v_nq : e.q_indptr[b + 1] - q0;
  if (nq <= 0 || 16 * TP * t >= nq) return;
  const int ctx = virt ? e.v_ctx : e.ctx[b];
  // (With partials, a chunk longer than max_q_len or a q_indptr past
  // num_seqs * max_q_len tokens would address partial rows past the workspace.)
  if ((e.causal && nq > ctx) || ctx < 1 || ctx > e.max_ctx ||
      ((e.splits > 1 || e.partial) && (nq > e.max_q || q0 < 0 || (int64_t)q0 + nq > (int64_t)e.B * e.max_q))) {
    if (threadIdx.x == 0 && t == 0) record_error(a.d_err, MKV_DEVERR_CTX);
    return;
  }
  const int tab0 = virt ? 0 : a.indptr[b], nbt = (ctx + kPageSize - 1) / kPageSize;
  if (!virt && (tab0 < 0 || a.indptr[b + 1] - tab0 < nbt)) {
    if (threadIdx.x == 0 && t == 0) record_error(a.d_err, MKV_DEVERR_TABLE);
    return;
  }
  // The table is read through the constant address space: scalar loads,
  // whose wait does not drain the vector-load ring (a vector load of a block
  // id needs vmcnt(0) before its readfirstlane).
  typedef const __attribute__((address_space(4))) int32_t const_i32;
  const const_i32 *table = (const const_i32 *)(a.ids + tab0);
  // The workgroup holds TP sub-tiles of 16 positions; wave = (sub-tile, head slot).
  const int sub = wave / WG, hw = wave % WG;
  const int row0 = 16 * (TP * t + sub);                  // first chunk row of this wave's sub-tile
  // Its first query position; without the causal mask every query stands at
  // the last position and sees all ctx keys.
  const int qlo = e.causal ? ctx - nq + row0 : ctx - 1;
  const int qhi_wg = e.causal ? min(ctx - nq + 16 * TP * (t + 1) - 1, ctx - 1) : ctx - 1;
  const int n = qhi_wg / kPageSize + 1;                  // blocks the workgroup streams: keys 0..qhi_wg
  const int nw = min(n, (qlo + 15) / kPageSize + 1);     // blocks this wave's sub-tile sees
  // Steps of KB blocks; with splits, this workgroup takes its share of them
  // (a short context can leave a split none: it stores an empty partial).
  const int nsteps_all = (n + KB - 1) / KB;
  const int sps = (nsteps_all + e.splits - 1) / e.splits;
  const int st0 = min(sp * sps, nsteps_all), st1 = min(st0 + sps, nsteps_all);
  const int hslot = hg * WG + hw;  // this wave's query head among the KV head's G
  const bool computes = hslot < a.G;
  const int hq = h * a.G + min(hslot, a.G - 1);
  const int qp = e.causal ? qlo + m16 : ctx - 1;  // this lane's query position (rows past nq: unused)
  const int64_t spare = dummy_offset(a);

  // Q^T operand: lane holds Q[row 16t + lane%16][32r + 8*(lane/16) .. +8].
  bf16x8 qop[NR];
  {
    const int row = min(row0 + m16, nq - 1);
    const uint8_t *qp8 = static_cast<const uint8_t *>(a.q) + ((int64_t)(q0 + row) * a.Hq + hq) * D * 2;
#pragma unroll
    for (int r = 0; r < NR; r++)
      qop[r] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4 *>(qp8 + 2 * (32 * r + 8 * g4)));
  }

  // Ring slot of one step: lane loads chunks c = threadIdx.x + 64*W*i of the
  // step's KB blocks (block kb = c / BCH: K rows then V rows of head h).
  // Blocks past n and chunks past the step read 128 bytes of a block picked
  // by the workgroup index, so every stage issues the same loads.
  u32x4 ring[R][LPL];
  uint32_t badr[R];  // bit kb: block kb of the step was rejected
  auto issue = [&](u32x4 (&d)[LPL], uint32_t &bad, int step) {
    int32_t blk[KB];
    bad = 0;
#pragma unroll
    for (int kb = 0; kb < KB; kb++) {
      const int k = step * KB + kb;
      blk[kb] = k < n ? table[k] : 0;  // uniform: a scalar load
      if (k < n && (blk[kb] < 0 || blk[kb] >= a.nblocks)) {
        bad |= 1u << kb;
        blk[kb] = 0;
      }
    }
#pragma unroll
    for (int i = 0; i < LPL; i++) {
      const int c = (int)threadIdx.x + 64 * W * i;
      const int kb = min(c / BCH, KB - 1), rem = c % BCH;
      const int kv = rem / (16 * CPR), rem2 = rem % (16 * CPR), row = rem2 / CPR, cc = rem2 % CPR;
      int32_t bk = blk[0];
#pragma unroll
      for (int j = 1; j < KB; j++) bk = kb == j ? blk[j] : bk;
      const bool real = c < NCH && step * KB + kb < n;
      const uint8_t *plane = kv ? a.v_plane : a.k_plane;
      const int64_t off = real ? (int64_t)bk * a.block_bytes + (int64_t)row * a.row_bytes + h * RB + 16 * cc
                               : spare + 16 * (lane & 7);
      d[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>((real ? plane : a.k_plane) + off));
    }
  };

  // Unmasked steps take a lean path. The ids of the workgroup's blocks
  // [kfirst, kend) are staged in LDS and range-checked once (any rejected id:
  // the generic path throughout, which masks it and records the error).
  // Chunk c = 64 * (wave + W * i) + lane of a step lies in one (block, K/V)
  // plane per wave, so a load is a wave-uniform base (block id, plane) plus a
  // lane offset (row, chunk, head) fixed for the whole launch.
  // (More than four loads per lane and step would hold more registers than the
  // lean path saves: those launches keep the generic path.)
  constexpr bool kLean = LPL <= 4;
  __shared__ int32_t ids_s[kLean ? kExtIdCap : 1];
  const int kfirst = st0 * KB, kend = min(st1 * KB, n);
  int fast = kLean && kend - kfirst <= kExtIdCap;
  if (fast) {
    int badl = 0;
    const int32_t *tg = a.ids + tab0 + kfirst;
    for (int i = (int)threadIdx.x; i < kend - kfirst; i += 64 * W) {
      const int32_t id = tg[i];
      badl |= (id < 0) | (id >= a.nblocks);
      ids_s[i] = id;
    }
    fast = !__syncthreads_or(badl);
  }
  fast = __builtin_amdgcn_readfirstlane(fast);
  // A wave past the step's chunks (head_dim 64 with 16 waves) loads the
  // step's last chunks again and does not store them: one load form, so the
  // compiler's in-order load counting stays exact.
  constexpr bool kAllVal = NCH % (64 * W) == 0;
  uint32_t flo[LPL], fwr[LPL];  // lane offset in the block; LDS offset in one ring buffer
  int fkb[LPL];                 // wave-uniform block of the step
  const uint8_t *fpl[LPL];      // wave-uniform plane (K or V)
  bool fval[LPL];               // wave-uniform: the wave's chunk is stored
#pragma unroll
  for (int i = 0; i < LPL; i++) {
    const int cw = 64 * (wave + W * i);
    fval[i] = kAllVal || cw < NCH;
    const int cu = min(cw, NCH - 64);
    const int pl = cu / (16 * CPR), kv = pl & 1;
    fkb[i] = pl >> 1;
    fpl[i] = kv ? a.v_plane : a.k_plane;
    const int rem2 = cu % (16 * CPR) + lane, row = rem2 / CPR, cc = rem2 % CPR;
    flo[i] = (uint32_t)(row * (int)a.row_bytes + h * RB + 16 * cc);
    fwr[i] = (uint32_t)((2 * fkb[i] + kv) * TILE + row * RB + ((cc ^ (kv ? ext_v_swz(row, CPR) : ext_k_swz(row, CPR))) << 4));
  }
  // A step whose KB blocks all lie in [kfirst, kend).
  auto issue_fast = [&](u32x4 (&d)[LPL], uint32_t &bad, int step) {
    bad = 0;
#pragma unroll
    for (int i = 0; i < LPL; i++) {
      const int32_t bk = __builtin_amdgcn_readfirstlane(ids_s[step * KB + fkb[i] - kfirst]);
      d[i] = __builtin_nontemporal_load(
          reinterpret_cast<const u32x4 *>(fpl[i] + (int64_t)bk * a.block_bytes + flo[i]));
    }
  };

  MStateT<D> st;
#pragma unroll
  for (int nn = 0; nn < NT; nn++) st.O[nn] = f32x4{0.f, 0.f, 0.f, 0.f};
  st.m = -INFINITY;
  st.l = 0.0f;
  const float inv_sl2 = 1.0f / a.sl2;
  float thr = -INFINITY;  // raw-score rescale threshold
  int k_rd[NR], v_rd[NT];
  const int vrow = 4 * g4 + a4;
#pragma unroll
  for (int r = 0; r < NR; r++) k_rd[r] = m16 * RB + (((g4 + 4 * r) ^ ext_k_swz(m16, CPR)) << 4);
#pragma unroll
  for (int nn = 0; nn < NT; nn++)
    v_rd[nn] = vrow * RB + (((2 * nn + (rq >> 1)) ^ ext_v_swz(vrow, CPR)) << 4) + 8 * (rq & 1);

  // FAST: every block of the step is in range and fully visible to every
  // query of the workgroup (no mask), and the step issued R - 1 ahead lies
  // in the staged ids.
  auto stage = [&](auto fast_c, int s, int step) {
    constexpr bool FAST = decltype(fast_c)::value;
    if constexpr (FAST) issue_fast(ring[(s + R - 1) % R], badr[(s + R - 1) % R], step + R - 1);
    else issue(ring[(s + R - 1) % R], badr[(s + R - 1) % R], step + R - 1);
    // step = (multiple of R) + s: buffer s & 1 alternates like step & 1 and
    // is a compile-time constant here (immediate LDS offsets).
#pragma unroll
    for (int i = 0; i < LPL; i++) {
      if constexpr (FAST) {
        if (kAllVal || fval[i]) *reinterpret_cast<u32x4 *>(&tiles[s & 1][0][0][0] + fwr[i]) = ring[s][i];
        continue;
      }
      const int c = (int)threadIdx.x + 64 * W * i;
      if (c < NCH) {
        const int kb = c / BCH, rem = c % BCH;
        const int kv = rem / (16 * CPR), rem2 = rem % (16 * CPR), row = rem2 / CPR, cc = rem2 % CPR;
        // V rows past the context or of a rejected block are stored as
        // zeros (stale slots may hold any bit pattern, and p = 0 times NaN
        // would poison O); K rows there are masked in the scores instead.
        u32x4 val = ring[s][i];
        if (kv && (((badr[s] >> kb) & 1) || kPageSize * (step * KB + kb) + row >= ctx)) val = u32x4{0u, 0u, 0u, 0u};
        *reinterpret_cast<u32x4 *>(tiles[s & 1][kb][kv] + row * RB + ((cc ^ (kv ? ext_v_swz(row, CPR) : ext_k_swz(row, CPR))) << 4)) = val;
      }
    }
    __syncthreads();
    if (!computes) return;
    const uint32_t bad = FAST ? 0u : badr[s];
    if (!FAST && bad && lane == 0) record_error(a.d_err, MKV_DEVERR_BLOCK);
    // Raw scores of the step's blocks (masked ones -inf). Lane holds
    // sr[kb][i] = S[key 16k + 4*g4 + i][query position qlo + lane%16].
    float sr[KB][4];
    float mloc = -INFINITY;
    bool masked = false;  // some block of the step needs the causal / context mask (uniform)
#pragma unroll
    for (int kb = 0; kb < KB; kb++) {
      const int k = step * KB + kb;
      if (!FAST && k >= nw) {  // uniform: past this sub-tile's last position (or past n in the last step)
#pragma unroll
        for (int i = 0; i < 4; i++) sr[kb][i] = -INFINITY;
        masked = true;
        continue;
      }
      const uint8_t *tk = tiles[s & 1][kb][0];
      u32x4 kq[NR];
#pragma unroll
      for (int r = 0; r < NR; r++) kq[r] = *reinterpret_cast<const u32x4 *>(tk + k_rd[r]);
      f32x4 S = {0.f, 0.f, 0.f, 0.f};
      // Where one workgroup fills a CU (two sub-tiles, or head_dim 256 with
      // 8 or more waves) the score MFMAs issue at raised wave priority, so a
      // wave that reaches them overtakes the waves busy with exponentials
      // and the matrix pipe stays fed (8 x 512 after 4k: 455 -> 435-445 us at priority 1, about
      // 1% more at 3; head_dim 256: 259 -> 255 us). The same around the PV
      // products or the load issue gained nothing, and with one sub-tile at
      // head_dim <= 128 (two workgroups per CU) it cost 16-token chunks 15%.
      constexpr bool kPrio = TP == 2 || (D == 256 && W >= 8);
      if constexpr (kPrio) __builtin_amdgcn_s_setprio(3);
#pragma unroll
      for (int r = 0; r < NR; r++)
        S = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, kq[r]), qop[r], S, 0, 0, 0);
      if constexpr (kPrio) __builtin_amdgcn_s_setprio(0);
      const bool kbad = (bad >> kb) & 1;
      const bool full = FAST || (!kbad && kPageSize * k + kPageSize - 1 <= qlo && kPageSize * k + kPageSize <= ctx);
#pragma unroll
      for (int i = 0; i < 4; i++) sr[kb][i] = S[i];
      if (!full) {  // only the last blocks of a tile (and rejected ones)
        masked = true;
        const int kp0 = kPageSize * k + 4 * g4;
#pragma unroll
        for (int i = 0; i < 4; i++)
          if (kbad || kp0 + i > qp || kp0 + i >= ctx) sr[kb][i] = -INFINITY;
      }
#pragma unroll
      for (int i = 0; i < 4; i++) mloc = fmaxf(mloc, sr[kb][i]);
    }
    // Rescale only when some score passes the running max by the slack
    // (st.m in scaled log2 units, thr = (st.m + slack) / (scale * log2 e) in
    // raw ones): checked on the lane's own scores first, so the column-wide
    // max (two cross-lane steps) runs only on the rare steps that need it.
    if (__ballot(mloc > thr)) {
      mloc = fmaxf(mloc, __shfl_xor(mloc, 16));
      mloc = fmaxf(mloc, __shfl_xor(mloc, 32));
      const float ms = mloc * a.sl2;
      const bool need = ms > st.m + kRescaleSlack;
      const float mn = need ? ms : st.m;
      // A column with nothing visible yet (possible in a later key range)
      // keeps m = -inf, l = 0, O = 0: scale 0, not exp2(-inf - -inf) = NaN.
      const float al = st.m == -INFINITY ? 0.0f : fast_exp2(st.m - mn);
      st.l *= al;
#pragma unroll
      for (int nn = 0; nn < NT; nn++) st.O[nn] *= al;
      st.m = mn;
      thr = (mn + kRescaleSlack) * inv_sl2;
    }
    if constexpr (FAST && KB == 2) {
      // Both blocks in one full-rate 16x16x32 product per 16 dims: lane
      // group g4's k-slots 0-3 are keys 4*g4..+3 of the first block and 4-7
      // the same keys of the second, in P^T (the score layout) and in V^T
      // (one transposed read per block).
      uint32_t pk[4];
#pragma unroll
      for (int kb = 0; kb < 2; kb++) {
        float pr[4];
#pragma unroll
        for (int i = 0; i < 4; i++) pr[i] = fast_exp2(fmaf(sr[kb][i], a.sl2, -st.m));
        st.l += (pr[0] + pr[1]) + (pr[2] + pr[3]);
        pk[2 * kb] = pack_bf16x2(pr[0], pr[1]);
        pk[2 * kb + 1] = pack_bf16x2(pr[2], pr[3]);
      }
      const bf16x8 pb = __builtin_bit_cast(bf16x8, u32x4{pk[0], pk[1], pk[2], pk[3]});
      const uint8_t *tv0 = tiles[s & 1][0][1], *tv1 = tiles[s & 1][1][1];
#pragma unroll
      for (int nn = 0; nn < NT; nn++) {
        const i16x4s r0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4 *)(tv0 + v_rd[nn]));
        const i16x4s r1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4 *)(tv1 + v_rd[nn]));
        const uint64_t w0 = __builtin_bit_cast(uint64_t, r0), w1 = __builtin_bit_cast(uint64_t, r1);
        const bf16x8 va = __builtin_bit_cast(bf16x8, u32x4{(uint32_t)w0, (uint32_t)(w0 >> 32), (uint32_t)w1,
                                                            (uint32_t)(w1 >> 32)});
        st.O[nn] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va, pb, st.O[nn], 0, 0, 0);
      }
      return;
    }
#pragma unroll
    for (int kb = 0; kb < KB; kb++) {
      const int k = step * KB + kb;
      if (!FAST && k >= nw) continue;  // uniform
      float pr[4];
#pragma unroll
      for (int i = 0; i < 4; i++) pr[i] = fast_exp2(fmaf(sr[kb][i], a.sl2, -st.m));
      if (!FAST && masked) {  // a fully masked column has m = -inf: keep its p at 0, not NaN
#pragma unroll
        for (int i = 0; i < 4; i++)
          if (sr[kb][i] == -INFINITY) pr[i] = 0.0f;
      }
      st.l += (pr[0] + pr[1]) + (pr[2] + pr[3]);
      const uint32_t p01 = pack_bf16x2(pr[0], pr[1]), p23 = pack_bf16x2(pr[2], pr[3]);
      const i16x4 pb = __builtin_bit_cast(i16x4, (uint64_t)p01 | ((uint64_t)p23 << 32));
      // O^T += V^T . P^T (V rows past the context were zeroed in LDS;
      // causally hidden rows have p = 0).
      const uint8_t *tv = tiles[s & 1][kb][1];
#pragma unroll
      for (int nn = 0; nn < NT; nn++) {
        const i16x4s raw = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4 *)(tv + v_rd[nn]));
        st.O[nn] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(i16x4, raw), pb, st.O[nn], 0, 0, 0);
      }
    }
  };

#pragma unroll
  for (int s = 0; s < R - 1; s++) issue(ring[s], badr[s], st0 + s);
  // Fast steps: [st0, fast_end), blocks below the workgroup's first query
  // position and below ctx (all keys visible to all its queries), with the
  // steps issued R - 1 ahead inside [kfirst, kend).
  const int fb = e.causal ? min((ctx - nq + 16 * TP * t + 1) / kPageSize, ctx / kPageSize) : ctx / kPageSize;
  const int fast_end = fast ? max(st0, min(min(st1, fb / KB), kend / KB - (R - 1))) : st0;
  const std::integral_constant<bool, true> kFast;
  const std::integral_constant<bool, false> kGeneric;
  int k0 = st0;
  for (int it = 0, nit = (fast_end - st0) / R; it < nit; it++, k0 += R) {
#pragma unroll
    for (int s = 0; s < R; s++) stage(kFast, s, k0 + s);
  }
  for (int it = 0, nit = (st1 - k0) / R; it < nit; it++, k0 += R) {
#pragma unroll
    for (int s = 0; s < R; s++) stage(kGeneric, s, k0 + s);
  }
#pragma unroll
  for (int s = 0; s < R - 1; s++)
    if (k0 + s < st1) stage(kGeneric, s, k0 + s);

  if (!computes) return;
  st.l += __shfl_xor(st.l, 16);
  st.l += __shfl_xor(st.l, 32);
  const int row = row0 + m16;
  if (row >= nq) return;
  if (e.splits > 1 || e.partial) {  // f32 partial (m, l, O) of this key range, merged later
    const int64_t prow = ((int64_t)(q0 + row) * a.Hq + hq) * e.splits + sp;
    float *wo = a.ws_o + prow * D + 4 * g4;
#pragma unroll
    for (int nn = 0; nn < NT; nn++) *reinterpret_cast<f32x4 *>(wo + 16 * nn) = st.O[nn];
    if (g4 == 0) *reinterpret_cast<float2 *>(a.ws_ml + 2 * prow) = make_float2(st.m, st.l);
    return;
  }
  const float f = final_scale(st.m, st.l, a.zero_sink);
  uint16_t *op = reinterpret_cast<uint16_t *>(a.o) + ((int64_t)(q0 + row) * a.Hq + hq) * D + 4 * g4;
#pragma unroll
  for (int nn = 0; nn < NT; nn++)
    *reinterpret_cast<uint2 *>(op + 16 * nn) = make_uint2(pack_bf16x2(st.O[nn][0] * f, st.O[nn][1] * f),
                                                          pack_bf16x2(st.O[nn][2] * f, st.O[nn][3] * f));
}

// Log-sum-exp merge of the extend kernel's key-range partials: one wave per
// (query token, query head) row, partials row * splits + s.
template <int D, bool BF16>
__global__ void __launch_bounds__(256) merge_ext_kernel(KArgs a, ExtArgs e) {
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t row = (int64_t)blockIdx.x * 4 + wave;
  const int64_t tokens = min((int64_t)e.q_indptr[e.B], (int64_t)e.B * e.max_q);
  if (row >= tokens * a.Hq) return;
  merge_rows<D, BF16>(a, lane, row * e.splits, 1, e.splits, row);
}

template <int D, bool BF16>
__global__ void __launch_bounds__(256) merge_planned_kernel(KArgs a, PlanDev pd) {
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t row = (int64_t)blockIdx.x * 4 + wave;
  if (row >= (int64_t)pd.n_merge * a.Hq) return;
  const int b = pd.merge_seqs[row / a.Hq];
  const int hq = (int)(row % a.Hq);
  const int first = pd.seq_piece0[b];
  merge_rows<D, BF16>(a, lane, (int64_t)(first + b) * a.Hq + hq, a.Hq, pd.seq_npiece[b],
                      (int64_t)b * a.Hq + hq);
}

// A sequence cut into many pieces (a batch too small to fill the device with
// long pieces): one workgroup per (sequence, query head) row, wave w merging
// the w-th share of the row's partials (one round of loads each), the waves'
// states combined in LDS by wave 0. The grid is n_merge * Hq.
constexpr int kWideMergeWaves = 8;
constexpr int kWideMergeMin = 16;  // partials per row above which the wide merge runs (one round of merge_rows)

template <int D, bool BF16>
__global__ void __launch_bounds__(64 * kWideMergeWaves) merge_wide_kernel(KArgs a, PlanDev pd) {
  constexpr int DPL = MergeVec<D>::DPL;
  typedef typename MergeVec<D>::type fvec;
  __shared__ float part[kWideMergeWaves][2 + 64 * DPL];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t row = blockIdx.x;
  const int b = pd.merge_seqs[row / a.Hq];
  const int hq = (int)(row % a.Hq);
  const int n = pd.seq_npiece[b];
  const int s0 = (int)((int64_t)n * wave / kWideMergeWaves);
  const int s1 = (int)((int64_t)n * (wave + 1) / kWideMergeWaves);
  // Partial s of the row at workspace row (seq_piece0[b] + b + s) * Hq + hq.
  const int64_t base = ((int64_t)pd.seq_piece0[b] + b + s0) * a.Hq + hq;
  float M, L;
  fvec acc;
  merge_partials_state<D>(
      lane, s1 - s0, [&](int s) { return a.ws_ml + 2 * (base + (int64_t)s * a.Hq); },
      [&](int s) { return a.ws_o + (base + (int64_t)s * a.Hq) * D; }, M, L, acc);
  if (lane == 0) {
    part[wave][0] = M;
    part[wave][1] = L;
  }
#pragma unroll
  for (int k = 0; k < DPL; k++) part[wave][2 + lane * DPL + k] = acc[k];
  __syncthreads();
  if (wave != 0) return;
  float Mx = -INFINITY;
#pragma unroll
  for (int w = 0; w < kWideMergeWaves; w++) Mx = fmaxf(Mx, part[w][0]);
  float Lx = 0.0f;
  fvec ax = fvec{};
#pragma unroll
  for (int w = 0; w < kWideMergeWaves; w++) {
    const float mw = part[w][0];
    const float f = mw == -INFINITY ? 0.0f : fast_exp2(mw - Mx);  // an empty share adds nothing
    Lx = fmaf(part[w][1], f, Lx);
#pragma unroll
    for (int k = 0; k < DPL; k++) ax[k] = fmaf(part[w][2 + lane * DPL + k], f, ax[k]);
  }
  store_merged_row<D, BF16>(a, lane, Mx, Lx, ax, (int64_t)b * a.Hq + hq);
}

// Decode over a shared prefix: row (sequence b, query head hq) merges b's
// suffix partials (one per piece, in the plan's workspace, as
// merge_planned_kernel reads them) with the prefix's S key-range partials
// (extend workspace rows (b * Hq + hq) * S + s); one wave per row, every
// sequence of the plan.
struct PrefixParts {
  const float *ml;  // (m, l) pairs of the prefix partials
  const float *o;   // their f32 rows
  int32_t S;        // key-range partials per (sequence, query head)
};

template <int D, bool BF16>
__global__ void __launch_bounds__(256) merge_prefix_kernel(KArgs a, PlanDev pd, PrefixParts pp) {
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t row = (int64_t)blockIdx.x * 4 + wave;
  if (row >= (int64_t)pd.B * a.Hq) return;
  const int b = (int)(row / a.Hq), hq = (int)(row % a.Hq);
  const int n1 = pd.seq_npiece[b];
  const int64_t base1 = (int64_t)(pd.seq_piece0[b] + b) * a.Hq + hq, base2 = row * pp.S;
  merge_partials<D, BF16>(
      a, lane, n1 + pp.S,
      [&](int s) { return s < n1 ? a.ws_ml + 2 * (base1 + (int64_t)s * a.Hq) : pp.ml + 2 * (base2 + s - n1); },
      [&](int s) { return s < n1 ? a.ws_o + (base1 + (int64_t)s * a.Hq) * D : pp.o + (base2 + s - n1) * D; }, row);
}

// ===========================================================================
// Host side.
// ===========================================================================

static bool mfma_applies(const Geom &g) {
  return g.dtype == MKV_DTYPE_BF16 && (g.D == 64 || g.D == 128 || g.D == 256);
}

static int check_common(const Pool *p, int32_t layer, uint32_t flags, float scale, bool &use_mfma) {
  const Geom &g = p->g;
  if (layer < 0 || layer >= g.L)
    return set_error(MKV_ERR_INVALID_ARGUMENT, "layer %d out of range [0, %d)", layer, g.L);
  if (g.D != 32 && g.D != 64 && g.D != 128 && g.D != 256)
    return set_error(MKV_ERR_INVALID_ARGUMENT,
                     "decode attention supports head_dim 32/64/128/256 (pool has %d)", g.D);
  if (!(scale > 0.0f) || !std::isfinite(scale))
    return set_error(MKV_ERR_INVALID_ARGUMENT, "scale must be finite and > 0");
  use_mfma = mfma_applies(g) && !(flags & MKV_ATTN_FORCE_VALU);
  if ((flags & MKV_ATTN_FORCE_MFMA) && !use_mfma)
    return set_error(MKV_ERR_INVALID_ARGUMENT, "MFMA kernel needs bf16 KV and head_dim 64/128/256");
  return MKV_OK;
}

static KArgs make_kargs(Pool *p, int32_t layer, const void *d_q, void *d_o, const int32_t *indptr,
                        const int32_t *ids, float scale, uint32_t flags, bool use_mfma) {
  const Geom &g = p->g;
  KArgs a;
  a.k_plane_w = p->data + (int64_t)layer * 2 * g.plane_bytes;
  a.v_plane_w = a.k_plane_w + g.plane_bytes;
  a.k_plane = a.k_plane_w;
  a.v_plane = a.v_plane_w;
  a.q = d_q;
  a.o = d_o;
  a.new_k = a.new_v = nullptr;
  a.indptr = indptr;
  a.ids = ids;
  a.ws_ml = a.ws_o = nullptr;
  a.d_err = p->d_err;
  a.nblocks = g.nblocks;
  a.row_bytes = g.row_bytes;
  a.block_bytes = g.block_bytes;
  a.Hq = g.Hq;
  a.Hkv = g.Hkv;
  a.G = g.Hq / g.Hkv;
  const int qcw = use_mfma ? kQChunkMfma : kQChunkValu;
  a.nqc = (a.G + qcw - 1) / qcw;
  a.sl2 = scale * kLog2e;
  a.zero_sink = (flags & MKV_ATTN_ZERO_SINK) ? 1 : 0;
  a.gk = a.gv = nullptr;
  a.gtok0 = nullptr;
  return a;
}

// Launches attention kernel `Kern<D, BF16, MFMA>` for the pool geometry.
#define MKV_DISPATCH(KERNEL, GRID, BLOCK, STREAM, ...)                                             \
  do {                                                                                             \
    if (use_mfma) {                                                                                \
      if (g.D == 64) hipLaunchKernelGGL((KERNEL<64, true, true>), GRID, BLOCK, 0, STREAM, __VA_ARGS__);   \
      else if (g.D == 128) hipLaunchKernelGGL((KERNEL<128, true, true>), GRID, BLOCK, 0, STREAM, __VA_ARGS__); \
      else hipLaunchKernelGGL((KERNEL<256, true, true>), GRID, BLOCK, 0, STREAM, __VA_ARGS__);         \
    } else if (g.dtype == MKV_DTYPE_BF16) {                                                        \
      if (g.D == 32) hipLaunchKernelGGL((KERNEL<32, true, false>), GRID, BLOCK, 0, STREAM, __VA_ARGS__);   \
      else if (g.D == 64) hipLaunchKernelGGL((KERNEL<64, true, false>), GRID, BLOCK, 0, STREAM, __VA_ARGS__); \
      else if (g.D == 128) hipLaunchKernelGGL((KERNEL<128, true, false>), GRID, BLOCK, 0, STREAM, __VA_ARGS__); \
      else hipLaunchKernelGGL((KERNEL<256, true, false>), GRID, BLOCK, 0, STREAM, __VA_ARGS__);         \
    } else {                                                                                       \
      if (g.D == 32) hipLaunchKernelGGL((KERNEL<32, false, false>), GRID, BLOCK, 0, STREAM, __VA_ARGS__);  \
      else if (g.D == 64) hipLaunchKernelGGL((KERNEL<64, false, false>), GRID, BLOCK, 0, STREAM, __VA_ARGS__); \
      else if (g.D == 128) hipLaunchKernelGGL((KERNEL<128, false, false>), GRID, BLOCK, 0, STREAM, __VA_ARGS__); \
      else hipLaunchKernelGGL((KERNEL<256, false, false>), GRID, BLOCK, 0, STREAM, __VA_ARGS__);        \
    }                                                                                              \
  } while (0)

// Launches VALU kernel `KERNEL<D, BF16, false, QC>` for the pool geometry.
#define MKV_DISPATCH_VALU_QC(KERNEL, QC, GRID, BLOCK, STREAM, ...)                                      \
  do {                                                                                                 \
    const bool bf = g.dtype == MKV_DTYPE_BF16;                                                         \
    switch (g.D) {                                                                                     \
      case 32: if (bf) hipLaunchKernelGGL((KERNEL<32, true, false, QC>), GRID, BLOCK, 0, STREAM, __VA_ARGS__);  \
               else hipLaunchKernelGGL((KERNEL<32, false, false, QC>), GRID, BLOCK, 0, STREAM, __VA_ARGS__); break; \
      case 64: if (bf) hipLaunchKernelGGL((KERNEL<64, true, false, QC>), GRID, BLOCK, 0, STREAM, __VA_ARGS__);  \
               else hipLaunchKernelGGL((KERNEL<64, false, false, QC>), GRID, BLOCK, 0, STREAM, __VA_ARGS__); break; \
      case 128: if (bf) hipLaunchKernelGGL((KERNEL<128, true, false, QC>), GRID, BLOCK, 0, STREAM, __VA_ARGS__); \
                else hipLaunchKernelGGL((KERNEL<128, false, false, QC>), GRID, BLOCK, 0, STREAM, __VA_ARGS__); break; \
      default: if (bf) hipLaunchKernelGGL((KERNEL<256, true, false, QC>), GRID, BLOCK, 0, STREAM, __VA_ARGS__); \
               else hipLaunchKernelGGL((KERNEL<256, false, false, QC>), GRID, BLOCK, 0, STREAM, __VA_ARGS__); break; \
    }                                                                                                  \
  } while (0)

// Launches merge kernel `KERNEL<D, BF16>` for the pool geometry.
#define MKV_DISPATCH_MERGE(KERNEL, GRID, BLOCK, STREAM, ...)                                 \
  do {                                                                                       \
    const bool bf = g.dtype == MKV_DTYPE_BF16;                                               \
    switch (g.D) {                                                                           \
      case 32: if (bf) hipLaunchKernelGGL((KERNEL<32, true>), GRID, BLOCK, 0, STREAM, __VA_ARGS__);  \
               else hipLaunchKernelGGL((KERNEL<32, false>), GRID, BLOCK, 0, STREAM, __VA_ARGS__); break; \
      case 64: if (bf) hipLaunchKernelGGL((KERNEL<64, true>), GRID, BLOCK, 0, STREAM, __VA_ARGS__);  \
               else hipLaunchKernelGGL((KERNEL<64, false>), GRID, BLOCK, 0, STREAM, __VA_ARGS__); break; \
      case 128: if (bf) hipLaunchKernelGGL((KERNEL<128, true>), GRID, BLOCK, 0, STREAM, __VA_ARGS__); \
                else hipLaunchKernelGGL((KERNEL<128, false>), GRID, BLOCK, 0, STREAM, __VA_ARGS__); break; \
      default: if (bf) hipLaunchKernelGGL((KERNEL<256, true>), GRID, BLOCK, 0, STREAM, __VA_ARGS__); \
               else hipLaunchKernelGGL((KERNEL<256, false>), GRID, BLOCK, 0, STREAM, __VA_ARGS__); break; \
    }                                                                                        \
  } while (0)

// ---- split grid -------------------------------------------------------------

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

static uint64_t split_ws_bytes(const Geom &g, int B, int S) {
  if (S <= 1) return 0;
  const uint64_t rows = (uint64_t)B * g.Hq * S;
  return (rows * 8 + 255) / 256 * 256 + rows * g.D * 4;
}

// ---- plan ---------------------------------------------------------------------

struct Plan {
  Pool *pool = nullptr;
  int device = 0;
  int32_t B = 0, P = 0, BP = 0, total = 0, n_merge = 0;
  int32_t *d_meta = nullptr;  // ctx[B] | seq_blk0[B+1] | piece_f0[P+1] | piece_seq[P] |
                              // seq_piece0[B] | seq_npiece[B] | merge_seqs[n_merge] |
                              // tok0[B+1] | flat_seq[total] | flat_meta[total] |
                              // flat_id[total] | prefix_ids[n_prefix] | dev_flat_id[total]
  size_t meta_cap = 0;        // ints
  int32_t *h_meta = nullptr;  // pinned staging
  size_t h_cap = 0;
  hipEvent_t uploaded = nullptr;
  bool pending = false;
  void *d_ws = nullptr;
  uint64_t ws_cap = 0;
  uint64_t ws_ml_bytes = 0;   // offset of the o rows inside d_ws
  size_t flat_off = 0;        // offset (ints) of flat_id inside d_meta
  size_t dev_flat_off = 0;    // offset (ints) of the ids flattened from a call's device tables
  bool has_tables = false;    // flat_id holds the block ids given at build time
  int32_t n_prefix = 0;       // shared-prefix ids given at build time (0: none)
  bool all_partial = false;   // every sequence stores partials (built for a shared prefix's suffixes)
  bool beside = false;        // suffix pieces sized to run beside the prefix tiles (one per CU)
  int32_t max_npiece = 0;     // most pieces any merged sequence spans
  int32_t valu_qc = kQChunkValu;  // query heads per wave when the per-head (VALU) kernel runs the plan
  int64_t tokens = 0;         // sum of the context lengths
  int32_t max_ctx = 0;        // the longest context
};

static PlanDev plan_dev(const Plan *pl) {
  PlanDev d;
  d.ctx = pl->d_meta;
  d.seq_blk0 = d.ctx + pl->B;
  d.piece_f0 = d.seq_blk0 + pl->B + 1;
  d.piece_seq = d.piece_f0 + pl->P + 1;
  d.seq_piece0 = d.piece_seq + pl->P;
  d.seq_npiece = d.seq_piece0 + pl->B;
  d.merge_seqs = d.seq_npiece + pl->B;
  d.tok0 = d.merge_seqs + pl->n_merge;
  d.flat_seq = d.tok0 + pl->B + 1;
  d.flat_meta = d.flat_seq + pl->total;
  d.flat_id = pl->d_meta + pl->flat_off;
  d.B = pl->B;
  d.P = pl->P;
  d.total_blocks = pl->total;
  d.n_merge = pl->n_merge;
  return d;
}

}  // namespace mkv

using namespace mkv;

// ---- C ABI: split grid ------------------------------------------------------------------

extern "C" int mkv_decode_attention_workspace_size(const mkv_pool *pool, int32_t num_seqs,
                                                   int32_t max_ctx_len, int32_t split_tokens,
                                                   uint64_t *out_bytes) {
  if (!pool || !out_bytes) return set_error(MKV_ERR_INVALID_ARGUMENT, "NULL argument");
  const Pool *p = reinterpret_cast<const Pool *>(pool);
  if (num_seqs < 0 || max_ctx_len < 0 || split_tokens < 0 || split_tokens % kPageSize)
    return set_error(MKV_ERR_INVALID_ARGUMENT, "bad sizes");
  const int st = split_tokens ? split_tokens : choose_split(p->g, num_seqs, max_ctx_len);
  const int S = max_ctx_len > 0 ? (max_ctx_len + st - 1) / st : 1;
  *out_bytes = split_ws_bytes(p->g, num_seqs, S);
  return MKV_OK;
}

// The split-grid decode of mkv_decode_attention. ws / ws_bytes: the
// caller's workspace, or NULL to use (and grow) the pool-owned one; with
// fixed_ws the given buffer is the only one and nothing is allocated: an
// automatic split count shrinks until its partials fit, and an explicit one
// whose partials do not fit is refused.
static int decode_split(Pool *p, int32_t layer, const void *d_q, void *d_o, const int32_t *d_block_indptr,
                        const int32_t *d_block_ids, const int32_t *d_ctx_lens, int32_t num_seqs, int32_t max_ctx_len,
                        float scale, uint32_t flags, int32_t split_tokens, void *ws, uint64_t ws_bytes, bool fixed_ws,
                        void *stream) {
  const Geom &g = p->g;
  bool use_mfma = false;
  int rc = check_common(p, layer, flags, scale, use_mfma);
  if (rc) return rc;
  if (num_seqs < 0 || max_ctx_len < 0)
    return set_error(MKV_ERR_INVALID_ARGUMENT, "num_seqs and max_ctx_len must be >= 0");
  if (num_seqs == 0) return MKV_OK;
  if (max_ctx_len == 0) return set_error(MKV_ERR_INVALID_ARGUMENT, "max_ctx_len must be >= 1");
  if (!d_q || !d_o || !d_block_indptr || !d_block_ids || !d_ctx_lens)
    return set_error(MKV_ERR_INVALID_ARGUMENT, "NULL device pointer");
  if (!aligned16(d_q) || !aligned16(d_o))
    return set_error(MKV_ERR_INVALID_ARGUMENT, "q and o must be 16-byte aligned");
  if (split_tokens < 0 || split_tokens % kPageSize)
    return set_error(MKV_ERR_INVALID_ARGUMENT, "split_tokens must be a multiple of %d", kPageSize);
  int st = split_tokens ? split_tokens : choose_split(g, num_seqs, max_ctx_len);
  int S = (max_ctx_len + st - 1) / st;
  uint64_t need = split_ws_bytes(g, num_seqs, S);
  if (fixed_ws && need > ws_bytes) {
    if (split_tokens)
      return set_error(MKV_ERR_INVALID_ARGUMENT, "split-K partials of %llu bytes exceed the %llu-byte scratch",
                       (unsigned long long)need, (unsigned long long)ws_bytes);
    while (S > 1 && need > ws_bytes) {  // fewer, longer splits until the partials fit (S = 1 needs none)
      S = (S + 1) / 2;
      st = ((max_ctx_len + S - 1) / S + kPageSize - 1) / kPageSize * kPageSize;
      S = (max_ctx_len + st - 1) / st;
      need = split_ws_bytes(g, num_seqs, S);
    }
  }
  DeviceGuard guard(p->device);
  hipStream_t hs = reinterpret_cast<hipStream_t>(stream);
  if (need) {
    if (ws) {
      if (ws_bytes < need)
        return set_error(MKV_ERR_INVALID_ARGUMENT, "workspace of %llu bytes < %llu needed",
                         (unsigned long long)ws_bytes, (unsigned long long)need);
    } else {
      if (p->ws_bytes < need) {
        const uint64_t cap = std::max<uint64_t>(need, p->ws_bytes + p->ws_bytes / 2);
        MKV_CHECK_HIP(hipStreamSynchronize(hs));  // earlier launches may read the old buffer
        if (p->ws) MKV_CHECK_HIP(hipFree(p->ws));
        p->ws = nullptr;
        p->ws_bytes = 0;
        MKV_CHECK_HIP(hipMalloc(&p->ws, cap));
        p->ws_bytes = cap;
      }
      ws = p->ws;
    }
  }
  KArgs a = make_kargs(p, layer, d_q, d_o, d_block_indptr, d_block_ids, scale, flags, use_mfma);
  const uint64_t rows = (uint64_t)num_seqs * g.Hq * S;
  a.ws_ml = reinterpret_cast<float *>(ws);
  a.ws_o = ws ? reinterpret_cast<float *>(reinterpret_cast<uint8_t *>(ws) + (rows * 8 + 255) / 256 * 256)
              : nullptr;
  SplitArgs sp;
  sp.ctx_lens = d_ctx_lens;
  sp.B = num_seqs;
  sp.S = S;
  sp.split_tokens = st;
  sp.max_ctx = max_ctx_len;
  sp.total_units = (int64_t)num_seqs * S * g.Hkv * a.nqc;
  const int64_t wgs = (sp.total_units + 3) / 4;
  if (wgs > INT32_MAX) return set_error(MKV_ERR_INVALID_ARGUMENT, "launch too large");
  MKV_DISPATCH(attn_split_kernel, dim3((unsigned)wgs), dim3(256), hs, a, sp);
  MKV_CHECK_LAUNCH("attn_split_kernel");
  if (S > 1) {
    const int64_t mwgs = ((int64_t)num_seqs * g.Hq + 3) / 4;
    MKV_DISPATCH_MERGE(merge_split_kernel, dim3((unsigned)mwgs), dim3(256), hs, a, sp);
    MKV_CHECK_LAUNCH("merge_split_kernel");
  }
  return MKV_OK;
}

extern "C" int mkv_decode_attention(mkv_pool *pool, int32_t layer, const void *d_q, void *d_o,
                                    const int32_t *d_block_indptr, const int32_t *d_block_ids,
                                    const int32_t *d_ctx_lens, int32_t num_seqs,
                                    int32_t max_ctx_len, float scale, uint32_t flags,
                                    int32_t split_tokens, void *d_workspace,
                                    uint64_t workspace_bytes, void *stream) {
  if (!pool) return set_error(MKV_ERR_INVALID_ARGUMENT, "pool is NULL");
  return decode_split(reinterpret_cast<Pool *>(pool), layer, d_q, d_o, d_block_indptr, d_block_ids, d_ctx_lens,
                      num_seqs, max_ctx_len, scale, flags, split_tokens, d_workspace, workspace_bytes, false,
                      stream);
}

// ---- C ABI: split grid without allocation ------------------------------------------
//
// mkv_decode_attention_static keeps its split-K partials in `scratch`, a
// file-scope device array: each GPU holds its own copy (kStaticScratchBytes)
// from the moment the library's code is loaded on it until the process
// ends. In host code `scratch` names a host-side stand-in, not the device
// memory: its device address on each GPU comes from hipGetSymbolAddress,
// looked up once per device when the first pool is created there (with that
// device current) and kept in g_scratch, and only that address is passed to
// the kernels. No partial needs to start at zero: the split kernel writes
// every partial the merge then reads. Calls on one GPU share the array, so
// calls that overlap on one GPU (other streams, other threads) race.

constexpr uint64_t kStaticScratchBytes = MKV_STATIC_SCRATCH_BYTES;
constexpr int kMaxDevices = 64;
static __device__ __align__(256) uint8_t scratch[kStaticScratchBytes];
static void *g_scratch[kMaxDevices];
static std::mutex g_scratch_mu;

int mkv::static_scratch_setup(int device) {
  if (device < 0 || device >= kMaxDevices)
    return set_error(MKV_ERR_INVALID_ARGUMENT, "device %d beyond the %d this library tracks", device, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch[device]) return MKV_OK;
  DeviceGuard guard(device);
  if (!guard.ok) return set_error(MKV_ERR_HIP, "hipSetDevice(%d) failed", device);
  void *ptr = nullptr;
  MKV_CHECK_HIP(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)));
  if (!ptr) return set_error(MKV_ERR_HIP, "hipGetSymbolAddress returned NULL for the static scratch");
  g_scratch[device] = ptr;
  return MKV_OK;
}

extern "C" int mkv_decode_attention_static(mkv_pool *pool, int32_t layer, const void *d_q, void *d_o,
                                           const int32_t *d_block_indptr, const int32_t *d_block_ids,
                                           const int32_t *d_ctx_lens, int32_t num_seqs, int32_t max_ctx_len,
                                           float scale, uint32_t flags, int32_t split_tokens, void *stream) {
  if (!pool) return set_error(MKV_ERR_INVALID_ARGUMENT, "pool is NULL");
  Pool *p = reinterpret_cast<Pool *>(pool);
  void *ws = nullptr;
  {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (p->device >= 0 && p->device < kMaxDevices) ws = g_scratch[p->device];
  }
  if (!ws) return set_error(MKV_ERR_HIP, "the static scratch of device %d was not set up", p->device);
  return decode_split(p, layer, d_q, d_o, d_block_indptr, d_block_ids, d_ctx_lens, num_seqs, max_ctx_len, scale,
                      flags, split_tokens, ws, kStaticScratchBytes, true, stream);
}

// ---- C ABI: plan --------------------------------------------------------------------

extern "C" int mkv_decode_plan_create(mkv_pool *pool, mkv_decode_plan **out_plan) {
  if (!pool || !out_plan) return set_error(MKV_ERR_INVALID_ARGUMENT, "NULL argument");
  Plan *pl = new (std::nothrow) Plan();
  if (!pl) return set_error(MKV_ERR_OUT_OF_MEMORY, "host allocation failed");
  pl->pool = reinterpret_cast<Pool *>(pool);
  pl->device = pl->pool->device;
  DeviceGuard guard(pl->device);
  hipError_t e = hipEventCreateWithFlags(&pl->uploaded, hipEventDisableTiming);
  if (e != hipSuccess) {
    delete pl;
    return hip_fail(e, "hipEventCreate");
  }
  *out_plan = reinterpret_cast<mkv_decode_plan *>(pl);
  return MKV_OK;
}

extern "C" int mkv_decode_plan_destroy(mkv_decode_plan *plan) {
  if (!plan) return MKV_OK;
  Plan *pl = reinterpret_cast<Plan *>(plan);
  DeviceGuard guard(pl->device);
  (void)hipDeviceSynchronize();
  if (pl->d_meta) (void)hipFree(pl->d_meta);
  if (pl->h_meta) (void)hipHostFree(pl->h_meta);
  if (pl->d_ws) (void)hipFree(pl->d_ws);
  if (pl->uploaded) (void)hipEventDestroy(pl->uploaded);
  delete pl;
  return MKV_OK;
}

// Compute units of the pool's device, queried once (-1 when unknown).
static int device_cus(Pool *p) {
  if (p->cus == 0) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, p->device) != hipSuccess) {
      (void)hipGetLastError();
      cus = 0;
    }
    p->cus = cus > 0 ? cus : -1;
  }
  return p->cus;
}

// Workgroups of the cooperative decode kernel the device holds at once
// (CUs x resident workgroups per CU for the instantiation the pool's
// geometry selects), or 0 when that kernel does not apply. Pieces beyond it
// run in a second round; fewer leave CUs idle. Queried once per pool.
static int64_t coop_resident(Pool *p) {
  if (p->coop_slots >= 0) return p->coop_slots;
  const Geom &g = p->g;
  p->coop_slots = 0;
  const int G = g.Hq / g.Hkv;
  if (!mfma_applies(g) || G > kQChunkMfma || !(g.Hkv == 1 || g.Hkv == 2 || g.Hkv == 4)) return 0;
  const int ql = (g.Hq * g.D / 8 + 64 * g.Hkv - 1) / (64 * g.Hkv);
  if (ql > 4) return 0;
  const void *fn = nullptr;
#define MKV_COOP_FN(DD, WW)                                                                        \
  fn = ql == 1   ? reinterpret_cast<const void *>(&attn_coop_kernel<DD, WW, 1, coop_ring(DD, 1), true>)  \
       : ql == 2 ? reinterpret_cast<const void *>(&attn_coop_kernel<DD, WW, 2, coop_ring(DD, 2), true>)  \
                 : reinterpret_cast<const void *>(&attn_coop_kernel<DD, WW, 4, coop_ring(DD, 4), true>)
#define MKV_COOP_FN_W(DD)              \
  do {                                 \
    if (g.Hkv == 1) MKV_COOP_FN(DD, 1); \
    else if (g.Hkv == 2) MKV_COOP_FN(DD, 2); \
    else MKV_COOP_FN(DD, 4);            \
  } while (0)
  switch (g.D) {
    case 64: MKV_COOP_FN_W(64); break;
    case 128: MKV_COOP_FN_W(128); break;
    default: MKV_COOP_FN_W(256); break;
  }
#undef MKV_COOP_FN_W
#undef MKV_COOP_FN
  DeviceGuard guard(p->device);
  int per_cu = 0, cus = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, 64 * g.Hkv, 0) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, p->device) != hipSuccess) {
    (void)hipGetLastError();  // leave no sticky error: fall back to the fixed rule
    return 0;
  }
  p->coop_slots = per_cu > 0 && cus > 0 ? (int64_t)per_cu * cus : 0;
  return p->coop_slots;
}

static const void *ext_kernel(int D, int W, int TP);
static int ext_resident_per_cu(Pool *p, const void *fn, int W, int TP);

// Whether the shared-prefix step runs its prefix tiles beside the suffix
// pieces, on a second stream. The suffixes are HBM-bound and the prefix is
// bound by issue and the matrix cores, so a CU that holds one workgroup of
// each keeps both busy. That pairing fits when the decode kernel and the
// one-sub-tile prefix instantiation each hold two workgroups per CU: each
// then takes at most half of every CU resource. The plan then cuts one
// suffix piece per CU, and the prefix is split to about one workgroup per
// CU (Qwen2.5-7B heads, 256 sequences over a 4,100-token prefix: 2.86 ->
// 2.42 ms per 28-layer step). Queried once per pool.
static bool prefix_beside(Pool *p) {
  if (p->beside == 0) {
    p->beside = -1;
    const Geom &g = p->g;
    const int G = g.Hq / g.Hkv;
    const int cus = device_cus(p);
    if (cus > 0 && g.D <= 128 && G <= 8 && coop_resident(p) == 2 * (int64_t)cus) {
      const int WG = G <= 1 ? 1 : G <= 2 ? 2 : G <= 4 ? 4 : 8;
      if (ext_resident_per_cu(p, ext_kernel(g.D, WG, 1), WG, 1) >= 2) p->beside = 1;
    }
  }
  return p->beside > 0;
}

// Host tables given to a plan build (the engine's form; all NULL when the
// calls bring device tables).
struct HostTables {
  const uint32_t *indptr = nullptr;  // [B+1]
  const uint32_t *ids = nullptr;
  const uint32_t *prefix = nullptr;  // shared prefix [n_prefix]
  int32_t n_prefix = 0;
};

static int plan_build(mkv_decode_plan *plan, const int32_t *h_ctx_lens, int32_t num_seqs, int32_t pieces,
                      bool all_partial, const HostTables &ht, void *stream) {
  if (!plan) return set_error(MKV_ERR_INVALID_ARGUMENT, "plan is NULL");
  Plan *pl = reinterpret_cast<Plan *>(plan);
  const Geom &g = pl->pool->g;
  if (num_seqs < 1 || !h_ctx_lens) return set_error(MKV_ERR_INVALID_ARGUMENT, "need num_seqs >= 1 context lengths");
  if (pieces < 0) return set_error(MKV_ERR_INVALID_ARGUMENT, "pieces must be >= 0");
  if (ht.indptr || ht.ids) {
    int rc = check_host_tables(g, ht.indptr, ht.ids, h_ctx_lens, num_seqs, nullptr);
    if (rc) return rc;
  }
  if (ht.n_prefix < 0 || (ht.n_prefix > 0 && !ht.prefix))
    return set_error(MKV_ERR_INVALID_ARGUMENT, "bad prefix ids");
  if (ht.n_prefix > INT32_MAX / (2 * kPageSize)) return set_error(MKV_ERR_INVALID_ARGUMENT, "prefix too long");
  for (int32_t i = 0; i < ht.n_prefix; i++)
    if (ht.prefix[i] >= (uint64_t)g.nblocks)
      return set_error(MKV_ERR_INVALID_ARGUMENT, "prefix block id %u (entry %d) outside the pool of %lld",
                       ht.prefix[i], i, (long long)g.nblocks);
  int64_t total = 0;
  for (int32_t b = 0; b < num_seqs; b++) {
    if (h_ctx_lens[b] < 1) return set_error(MKV_ERR_INVALID_ARGUMENT, "ctx_len[%d] = %d < 1", b, h_ctx_lens[b]);
    total += (h_ctx_lens[b] + kPageSize - 1) / kPageSize;
  }
  if (total > INT32_MAX / 2) return set_error(MKV_ERR_INVALID_ARGUMENT, "batch too large");
  // Pieces: as many as the cooperative kernel's resident workgroups (one
  // round), else ~8 waves per CU on 256 CUs, one wave per (KV head, query
  // chunk); a piece is one workgroup of the grid.
  const int G = g.Hq / g.Hkv;
  const int nqc = (G + kQChunkMfma - 1) / kQChunkMfma;
  // A shared prefix's suffixes run beside the prefix tiles: one piece per CU.
  const bool beside = !pieces && all_partial && prefix_beside(pl->pool);
  const int64_t resident = pieces ? 0 : beside ? device_cus(pl->pool) : coop_resident(pl->pool);
  int64_t P = pieces ? pieces : resident ? resident : std::max<int64_t>(1, 2048 / std::max(1, g.Hkv * nqc));
  // A batch too small to give every resident workgroup kSmallPlanBlocks
  // blocks is latency-bound. Its cooperative plan takes at most one piece per
  // CU (a second workgroup on a CU only competes for it) and at least
  // kMinPieceBlocks blocks per piece (shorter ones only add partials for the
  // merge to read back). Batches of 1-8 sequences at Qwen2.5-7B heads,
  // us per layer: 1 x 4k 17.3 -> 14.6, 1 x 8k 19.5 -> 14.7, 8 x 2k 17.1 ->
  // 15.1 (with the wide merge for rows of many partials).
  if (!pieces && resident > 0 && total < resident * kSmallPlanBlocks) {
    const int cus = device_cus(pl->pool);
    if (cus > 0) P = std::min<int64_t>(P, cus);
    P = std::min<int64_t>(P, std::max<int64_t>(1, (total + kMinPieceBlocks - 1) / kMinPieceBlocks));
  }
  P = std::max<int64_t>(P, (total + 63) / 64);  // a piece is at most 64 blocks (one per lane)
  P = std::min<int64_t>(P, total);
  std::vector<int32_t> blk0v(num_seqs + 1);
  {
    int64_t acc = 0;
    for (int32_t b = 0; b < num_seqs; b++) {
      blk0v[b] = (int32_t)acc;
      acc += (h_ctx_lens[b] + kPageSize - 1) / kPageSize;
    }
    blk0v[num_seqs] = (int32_t)acc;
  }
  // Piece boundaries: a greedy fill of the flattened blocks under a weight
  // cap, the smallest that gives at most P pieces. A block weighs
  // kBlockWeight; a sequence that starts inside a piece (not at its first
  // block) adds kSwitchWeight, what its predecessor's partial stores and the
  // Q reload cost that piece (measured: about 1.5 blocks' time).
  std::vector<int32_t> f0s;
  // With two resident workgroups per CU, the pieces dispatched first (the
  // first `first` indices, one per CU) get kFirstRoundWeight percent of the
  // cap: their waves are older and win issue arbitration over the second
  // workgroup of their CU.
  const int64_t first = (!pieces && resident > 0 && device_cus(pl->pool) > 0 &&
                         resident == 2 * (int64_t)device_cus(pl->pool)) ? device_cus(pl->pool) : 0;
  // Workgroup L runs on XCD L mod 8, and in a launch of one round of
  // resident pieces the odd-numbered XCDs finish last: per-workgroup stamps
  // on every box measured put their last workgroups about 5 us (6%) after
  // the even XCDs'. Pieces with an odd index, dealt to those XCDs, get
  // kOddXcdWeight percent of the cap (the 28-layer Qwen2.5-7B step of 64
  // sequences 72.7 -> 73.4% of peak, Gemma-2B MQA 72.3 -> 73.3%). Launches of several rounds, whose freed slots take
  // the next piece whatever its XCD, keep equal caps.
  const bool odd_light = !pieces && resident > 0 && P == resident;
  auto cut = [&](int64_t cap) {
    f0s.clear();
    int64_t w = 0;
    int cnt = 0;
    int32_t b = 0;
    const int64_t cap_first = cap * kFirstRoundWeight / 100;
    for (int64_t f = 0; f < total; f++) {
      while (blk0v[b + 1] <= f) b++;
      int64_t wi = kBlockWeight + ((f == blk0v[b] && cnt > 0) ? kSwitchWeight : 0);
      const int64_t idx = (int64_t)f0s.size() - 1;  // the piece being filled
      const int64_t cq0 = idx < first ? cap_first : cap;
      const int64_t cq = odd_light && (idx & 1) ? cq0 * kOddXcdWeight / 100 : cq0;
      if (cnt > 0 && (cnt == 64 || w + wi > cq)) {
        cnt = 0;
        w = 0;
        wi = kBlockWeight;
      }
      if (cnt == 0) f0s.push_back((int32_t)f);
      w += wi;
      cnt++;
    }
    f0s.push_back((int32_t)total);
  };
  {  // smallest cap giving at most P pieces (the count falls as the cap grows)
    int64_t lo = kBlockWeight, hi = 64 * (kBlockWeight + kSwitchWeight);
    while (lo < hi) {
      const int64_t mid = (lo + hi) / 2;
      cut(mid);
      if ((int64_t)f0s.size() - 1 <= P) hi = mid;
      else lo = mid + 1;
    }
    for (cut(lo); (int64_t)f0s.size() - 1 > P; cut(++lo)) {
    }
  }
  P = (int64_t)f0s.size() - 1;
  // The per-head (VALU) kernel takes kQChunkValu query heads per wave. A
  // launch with fewer (block, KV head) units than two per CU cannot fill the
  // device and is latency-bound: there each wave takes kQChunkValuSmall
  // heads, which divides a wave's arithmetic by eight for the price of more
  // waves reading the same (cache-resident) K/V (8 f32 sequences at
  // Qwen2.5-0.5B heads, per-sequence form, 24 layers: 0.251 ms per step with
  // 2 heads per wave, 0.212 ms with 1). Larger launches keep the wide chunk,
  // which reads each block once per KV head.
  const int cus_now = device_cus(pl->pool);
  const int32_t valu_qc = cus_now > 0 && total * g.Hkv <= 2 * (int64_t)cus_now ? kQChunkValuSmall : kQChunkValu;
  int64_t BP = 0;
  for (int64_t q = 0; q < P; q++) BP = std::max<int64_t>(BP, f0s[q + 1] - f0s[q]);
  DeviceGuard guard(pl->pool->device);
  hipStream_t hs = reinterpret_cast<hipStream_t>(stream);
  const size_t n_ints = (size_t)num_seqs + (num_seqs + 1) + (P + 1) + P + 3 * (size_t)num_seqs +
                        (num_seqs + 1) + 3 * (size_t)total + ht.n_prefix;
  // Staging: wait for the previous upload to leave the pinned buffer.
  if (pl->pending) {
    MKV_CHECK_HIP(hipEventSynchronize(pl->uploaded));
    pl->pending = false;
  }
  // Buffers grow by half again their size when they must grow: an engine's
  // tables gain blocks every few steps, and each reallocation costs a stream
  // synchronisation (measured: 0.2-0.5 ms per step when it happened on every
  // step).
  const auto grown = [](size_t need, size_t cap) { return std::max(need, cap + cap / 2); };
  if (pl->h_cap < n_ints) {
    const size_t cap = grown(n_ints, pl->h_cap);
    if (pl->h_meta) MKV_CHECK_HIP(hipHostFree(pl->h_meta));
    pl->h_meta = nullptr;
    pl->h_cap = 0;
    MKV_CHECK_HIP(hipHostMalloc(reinterpret_cast<void **>(&pl->h_meta), cap * 4));
    pl->h_cap = cap;
  }
  int32_t *ctx = pl->h_meta, *blk0 = ctx + num_seqs, *pf0 = blk0 + num_seqs + 1, *pseq = pf0 + P + 1;
  int32_t *spiece0 = pseq + P, *snpiece = spiece0 + num_seqs, *mseq = snpiece + num_seqs;
  for (int32_t b = 0; b < num_seqs; b++) ctx[b] = h_ctx_lens[b];
  for (int32_t b = 0; b <= num_seqs; b++) blk0[b] = blk0v[b];
  for (int64_t q = 0; q <= P; q++) pf0[q] = f0s[q];
  for (int32_t b = 0, q = 0; q < P; q++) {
    while (blk0[b + 1] <= pf0[q]) b++;
    pseq[q] = b;
  }
  // Pieces of each sequence: first = the piece holding its first block.
  for (int32_t b = 0, q = 0; b < num_seqs; b++) {
    while (pf0[q + 1] <= blk0[b]) q++;
    int32_t last = q;
    while (pf0[last + 1] < blk0[b + 1]) last++;
    spiece0[b] = q;
    snpiece[b] = last - q + 1;
  }
  int n_merge = 0, max_npiece = 0;
  for (int32_t b = 0; b < num_seqs; b++)
    if (snpiece[b] > 1 || all_partial) {
      mseq[n_merge++] = b;
      max_npiece = std::max(max_npiece, snpiece[b]);
    }
  int32_t *tok0 = mseq + n_merge, *fseq = tok0 + num_seqs + 1, *fmeta = fseq + total;
  // Gather rows: sequence b's tokens start after the earlier contexts
  // (clamped where they pass 2^31 - 1: the fused gather then refuses the plan).
  int64_t tokens = 0;
  int32_t max_ctx = 0;
  for (int32_t b = 0; b < num_seqs; b++) {
    tok0[b] = (int32_t)std::min<int64_t>(tokens, INT32_MAX);
    tokens += ctx[b];
    max_ctx = std::max(max_ctx, ctx[b]);
  }
  tok0[num_seqs] = (int32_t)std::min<int64_t>(tokens, INT32_MAX);
  for (int32_t b = 0; b < num_seqs; b++) {
    const int nb = blk0[b + 1] - blk0[b];
    const int single = snpiece[b] == 1 && !all_partial ? kMetaSingle : 0;
    for (int j = 0; j < nb; j++) {
      const int last = j == nb - 1;
      fseq[blk0[b] + j] = b;
      fmeta[blk0[b] + j] = (last ? ctx[b] - kPageSize * j : kPageSize) | (last ? kMetaLast : 0) | single;
    }
  }
  // Block ids in piece order (flattened order: sequence b's first
  // ceil(ctx_b / 16) table entries at seq_blk0[b]), then the prefix ids.
  const size_t flat_off = (size_t)num_seqs + (num_seqs + 1) + (P + 1) + P + 2 * (size_t)num_seqs + n_merge +
                          (num_seqs + 1) + 2 * (size_t)total;
  const bool tables = ht.indptr != nullptr;
  if (tables) {
    int32_t *fid = pl->h_meta + flat_off;
    for (int32_t b = 0; b < num_seqs; b++) {
      const uint32_t *t = ht.ids + ht.indptr[b];
      for (int32_t j = 0, nb = blk0[b + 1] - blk0[b]; j < nb; j++) fid[blk0[b] + j] = (int32_t)t[j];
    }
    for (int32_t i = 0; i < ht.n_prefix; i++) fid[total + i] = (int32_t)ht.prefix[i];
  }
  const size_t used = flat_off + (tables ? (size_t)total + ht.n_prefix : 0);
  // A call that brings device tables flattens their ids into a region of its
  // own after the held ids, so the ids given at build time stay intact for
  // later calls without tables.
  const size_t dev_flat_off = flat_off + (size_t)total + ht.n_prefix;
  if (pl->meta_cap < dev_flat_off + total) {
    const size_t cap = grown(dev_flat_off + total, pl->meta_cap);
    MKV_CHECK_HIP(hipStreamSynchronize(hs));  // earlier launches may read the old buffer
    if (pl->d_meta) MKV_CHECK_HIP(hipFree(pl->d_meta));
    pl->d_meta = nullptr;
    pl->meta_cap = 0;
    MKV_CHECK_HIP(hipMalloc(reinterpret_cast<void **>(&pl->d_meta), cap * 4));
    pl->meta_cap = cap;
  }
  const uint64_t slots = (uint64_t)P + num_seqs;
  const uint64_t rows = slots * g.Hq;
  const uint64_t ml = (rows * 8 + 255) / 256 * 256;
  const uint64_t need = ml + rows * g.D * 4;
  if (pl->ws_cap < need) {
    const uint64_t cap = std::max<uint64_t>(need, pl->ws_cap + pl->ws_cap / 2);
    MKV_CHECK_HIP(hipStreamSynchronize(hs));
    if (pl->d_ws) MKV_CHECK_HIP(hipFree(pl->d_ws));
    pl->d_ws = nullptr;
    pl->ws_cap = 0;
    MKV_CHECK_HIP(hipMalloc(&pl->d_ws, cap));
    pl->ws_cap = cap;
  }
  pl->ws_ml_bytes = ml;
  pl->flat_off = flat_off;
  pl->dev_flat_off = dev_flat_off;
  pl->has_tables = tables;
  pl->n_prefix = ht.n_prefix;
  MKV_CHECK_HIP(hipMemcpyAsync(pl->d_meta, pl->h_meta, used * 4, hipMemcpyHostToDevice, hs));
  MKV_CHECK_HIP(hipEventRecord(pl->uploaded, hs));
  pl->pending = true;
  pl->B = num_seqs;
  pl->P = (int32_t)P;
  pl->BP = (int32_t)BP;
  pl->total = (int32_t)total;
  pl->n_merge = n_merge;
  pl->max_npiece = max_npiece;
  pl->all_partial = all_partial;
  pl->beside = beside;
  pl->valu_qc = valu_qc;
  pl->tokens = tokens;
  pl->max_ctx = max_ctx;
  return MKV_OK;
}

extern "C" int mkv_decode_plan_build(mkv_decode_plan *plan, const int32_t *h_ctx_lens, int32_t num_seqs,
                                     int32_t pieces, void *stream) {
  return plan_build(plan, h_ctx_lens, num_seqs, pieces, false, HostTables(), stream);
}

extern "C" int mkv_decode_plan_build_suffixes(mkv_decode_plan *plan, const int32_t *h_suffix_lens,
                                              int32_t num_seqs, int32_t pieces, void *stream) {
  return plan_build(plan, h_suffix_lens, num_seqs, pieces, true, HostTables(), stream);
}

extern "C" int mkv_decode_plan_build_tables(mkv_decode_plan *plan, const int32_t *h_ctx_lens,
                                            const uint32_t *h_block_indptr, const uint32_t *h_block_ids,
                                            int32_t num_seqs, int32_t pieces, void *stream) {
  if (!h_block_indptr) return set_error(MKV_ERR_INVALID_ARGUMENT, "NULL block_indptr");
  HostTables ht;
  ht.indptr = h_block_indptr;
  ht.ids = h_block_ids;
  return plan_build(plan, h_ctx_lens, num_seqs, pieces, false, ht, stream);
}

extern "C" int mkv_decode_plan_build_shared_prefix(mkv_decode_plan *plan, const uint32_t *h_prefix_ids,
                                                   int32_t prefix_blocks, const int32_t *h_suffix_lens,
                                                   const uint32_t *h_block_indptr, const uint32_t *h_block_ids,
                                                   int32_t num_seqs, int32_t pieces, void *stream) {
  if (!h_block_indptr) return set_error(MKV_ERR_INVALID_ARGUMENT, "NULL block_indptr");
  if (!h_prefix_ids || prefix_blocks < 1) return set_error(MKV_ERR_INVALID_ARGUMENT, "need a prefix of >= 1 block ids");
  HostTables ht;
  ht.indptr = h_block_indptr;
  ht.ids = h_block_ids;
  ht.prefix = h_prefix_ids;
  ht.n_prefix = prefix_blocks;
  return plan_build(plan, h_suffix_lens, num_seqs, pieces, true, ht, stream);
}

extern "C" int mkv_decode_plan_info(const mkv_decode_plan *plan, int32_t *out_pieces,
                                    int32_t *out_blocks_per_piece, int32_t *out_merge_seqs) {
  if (!plan) return set_error(MKV_ERR_INVALID_ARGUMENT, "plan is NULL");
  const Plan *pl = reinterpret_cast<const Plan *>(plan);
  if (out_pieces) *out_pieces = pl->P;
  if (out_blocks_per_piece) *out_blocks_per_piece = pl->BP;
  if (out_merge_seqs) *out_merge_seqs = pl->n_merge;
  return MKV_OK;
}

static int launch_planned(Pool *p, const Plan *pl, int32_t layer, const void *d_k_new, const void *d_v_new,
                          const void *d_q, void *d_o, const int32_t *d_block_indptr,
                          const int32_t *d_block_ids, float scale, uint32_t flags, void *stream,
                          bool merge = true, void *d_gk = nullptr, void *d_gv = nullptr, int64_t gcap = 0) {
  const Geom &g = p->g;
  if (pl->pool != p) return set_error(MKV_ERR_INVALID_ARGUMENT, "plan belongs to another pool");
  if (pl->B < 1) return set_error(MKV_ERR_INVALID_ARGUMENT, "plan was never built");
  const bool gather = d_gk || d_gv;
  if (gather) {
    if (!d_gk || !d_gv) return set_error(MKV_ERR_INVALID_ARGUMENT, "give both gather outputs");
    if (!aligned16(d_gk) || !aligned16(d_gv))
      return set_error(MKV_ERR_INVALID_ARGUMENT, "gather outputs must be 16-byte aligned");
    if (pl->tokens > INT32_MAX) return set_error(MKV_ERR_INVALID_ARGUMENT, "more than 2^31 - 1 tokens to gather");
    if (pl->tokens > gcap)
      return set_error(MKV_ERR_INVALID_ARGUMENT, "gather outputs hold %lld tokens, the plan's contexts %lld",
                       (long long)gcap, (long long)pl->tokens);
  }
  bool use_mfma = false;
  int rc = check_common(p, layer, flags, scale, use_mfma);
  if (rc) return rc;
  if (!d_q || !d_o) return set_error(MKV_ERR_INVALID_ARGUMENT, "NULL device pointer");
  const bool dev_tables = d_block_indptr || d_block_ids;
  if (dev_tables && !(d_block_indptr && d_block_ids))
    return set_error(MKV_ERR_INVALID_ARGUMENT, "give both device table arrays, or neither");
  if (!dev_tables && !pl->has_tables)
    return set_error(MKV_ERR_INVALID_ARGUMENT,
                     "no block tables: pass device tables, or build the plan with its host tables");
  if (!aligned16(d_q) || !aligned16(d_o) || !aligned16(d_k_new) || !aligned16(d_v_new))
    return set_error(MKV_ERR_INVALID_ARGUMENT, "q, o and new K/V rows must be 16-byte aligned");
  DeviceGuard guard(p->device);
  hipStream_t hs = reinterpret_cast<hipStream_t>(stream);
  PlanDev pd = plan_dev(pl);
  if (dev_tables) {
    // Device tables are read on every call: the MFMA kernels' piece-order
    // ids are gathered from them here, so a table rewritten in place between
    // calls is seen by the next call. They land in their own region, never
    // over the ids the plan holds from its build.
    pd.flat_id = pl->d_meta + pl->dev_flat_off;
    if (use_mfma) hipLaunchKernelGGL(flatten_ids_kernel, dim3((unsigned)((pl->total + 255) / 256)), dim3(256), 0, hs, pd,
                       d_block_indptr, d_block_ids, g.nblocks, p->d_err);
    MKV_CHECK_LAUNCH("flatten_ids_kernel");
  } else {
    // The plan's own tables: flattened ids indexed by seq_blk0 form a CSR
    // table of exactly ceil(ctx_b / 16) ids per sequence.
    d_block_indptr = pd.seq_blk0;
    d_block_ids = pd.flat_id;
  }
  KArgs a = make_kargs(p, layer, d_q, d_o, d_block_indptr, d_block_ids, scale, flags, use_mfma);
  const bool small_qc = !use_mfma && pl->valu_qc == kQChunkValuSmall;
  if (small_qc) a.nqc = (a.G + kQChunkValuSmall - 1) / kQChunkValuSmall;
  a.new_k = reinterpret_cast<const uint8_t *>(d_k_new);
  a.new_v = reinterpret_cast<const uint8_t *>(d_v_new);
  a.ws_ml = reinterpret_cast<float *>(pl->d_ws);
  a.ws_o = reinterpret_cast<float *>(reinterpret_cast<uint8_t *>(pl->d_ws) + pl->ws_ml_bytes);
  // The per-head kernel stores the gather's rows as it reads them; after the
  // MFMA kernels the gather kernel runs on the same stream.
  const bool fused_gather = gather && !use_mfma;
  if (fused_gather) {
    a.gk = reinterpret_cast<uint8_t *>(d_gk);
    a.gv = reinterpret_cast<uint8_t *>(d_gv);
    a.gtok0 = pd.tok0;
  }
  const int hcs = g.Hkv * a.nqc;
  const int wpw = std::min(4, hcs);
  const dim3 grid((unsigned)pl->P, (unsigned)((hcs + wpw - 1) / wpw)), block(64 * wpw);
  // A caller's measurement events bracket the attention kernel alone (one shot).
  hipEvent_t ev_start = p->ev_start, ev_end = p->ev_end;
  p->ev_start = p->ev_end = nullptr;
  if (ev_start) MKV_CHECK_HIP(hipEventRecord(ev_start, hs));
  bool merged = false;  // the attention kernel wrote the final rows of every sequence
  if (use_mfma) {
    // Cooperative kernel: Q rows of one sequence (Hq * D * 2 bytes) must fit
    // the QL loads per lane its ring slots carry.
    const int qlanes = 64 * g.Hkv;
    const int qchunks = g.Hq * g.D / 8;
    const int ql = (qchunks + qlanes - 1) / qlanes;
    const bool coop = a.nqc == 1 && (g.Hkv == 1 || g.Hkv == 2 || g.Hkv == 4) && ql <= 4 &&
                      !(flags & MKV_ATTN_PER_HEAD_LOADS);
    if (coop) {
      // Non-temporal K/V loads stream best; a batch whose tables share blocks
      // (a radix-shared prefix) reads them again from the caches instead.
      const bool cached = flags & MKV_ATTN_CACHED_LOADS;
      const dim3 cgrid((unsigned)pl->P), cblock(64 * g.Hkv);
#define MKV_COOP_NT(DD, WW, NT)                                                                          \
  do {                                                                                                   \
    if (ql == 1) hipLaunchKernelGGL((attn_coop_kernel<DD, WW, 1, coop_ring(DD, 1), NT>), cgrid, cblock, 0, hs, a, pd); \
    else if (ql == 2) hipLaunchKernelGGL((attn_coop_kernel<DD, WW, 2, coop_ring(DD, 2), NT>), cgrid, cblock, 0, hs, a, pd); \
    else hipLaunchKernelGGL((attn_coop_kernel<DD, WW, 4, coop_ring(DD, 4), NT>), cgrid, cblock, 0, hs, a, pd);    \
  } while (0)
#define MKV_COOP_QL(DD, WW)                     \
  do {                                          \
    if (cached) MKV_COOP_NT(DD, WW, false);     \
    else MKV_COOP_NT(DD, WW, true);             \
  } while (0)
#define MKV_COOP(DD)                                   \
  do {                                                 \
    if (g.Hkv == 1) MKV_COOP_QL(DD, 1);                \
    else if (g.Hkv == 2) MKV_COOP_QL(DD, 2);           \
    else MKV_COOP_QL(DD, 4);                           \
  } while (0)
      switch (g.D) {
        case 64: MKV_COOP(64); break;
        case 128: MKV_COOP(128); break;
        default: MKV_COOP(256); break;
      }
#undef MKV_COOP
#undef MKV_COOP_QL
#undef MKV_COOP_NT
      MKV_CHECK_LAUNCH("attn_coop_kernel");
    } else {
      switch (g.D) {
        case 64: hipLaunchKernelGGL(attn_stream_kernel<64>, grid, block, 0, hs, a, pd); break;
        case 128: hipLaunchKernelGGL(attn_stream_kernel<128>, grid, block, 0, hs, a, pd); break;
        default: hipLaunchKernelGGL(attn_stream_kernel<256>, grid, block, 0, hs, a, pd); break;
      }
      MKV_CHECK_LAUNCH("attn_stream_kernel");
    }
  } else if (small_qc && merge && !pl->all_partial) {
    // Latency-bound: one workgroup per (sequence, KV head, query chunk),
    // the waves' states merged in LDS; no partials, no merge launch.
    const dim3 sgrid((unsigned)pl->B, (unsigned)(g.Hkv * a.nqc)), sblock(64 * kSeqWaves);
    MKV_DISPATCH_VALU_QC(attn_seq_kernel, kQChunkValuSmall, sgrid, sblock, hs, a, pd);
    MKV_CHECK_LAUNCH("attn_seq_kernel");
    merged = true;
  } else if (small_qc) {
    MKV_DISPATCH_VALU_QC(attn_planned_kernel, kQChunkValuSmall, grid, block, hs, a, pd);
    MKV_CHECK_LAUNCH("attn_planned_kernel");
  } else {
    MKV_DISPATCH(attn_planned_kernel, grid, block, hs, a, pd);
    MKV_CHECK_LAUNCH("attn_planned_kernel");
  }
  if (ev_end) MKV_CHECK_HIP(hipEventRecord(ev_end, hs));
  if (pl->n_merge && merge && !merged) {
    // Rows of many partials spread over 8 waves, where the rows are few (at
    // most two per CU): with thousands of rows (64 sequences at Qwen2.5-7B
    // heads have 1,792, 446 cut sequences 12,488) the eightfold waves cost
    // more than the rounds they save (2.80 -> 2.97 ms per 28-layer step).
    const int64_t rows = (int64_t)pl->n_merge * g.Hq;
    const int cus = device_cus(p);
    if (pl->max_npiece > kWideMergeMin && cus > 0 && rows <= 2 * (int64_t)cus) {
      MKV_DISPATCH_MERGE(merge_wide_kernel, dim3((unsigned)rows), dim3(64 * kWideMergeWaves), hs, a, pd);
      MKV_CHECK_LAUNCH("merge_wide_kernel");
    } else {
      const int64_t mwgs = ((int64_t)pl->n_merge * g.Hq + 3) / 4;
      MKV_DISPATCH_MERGE(merge_planned_kernel, dim3((unsigned)mwgs), dim3(256), hs, a, pd);
      MKV_CHECK_LAUNCH("merge_planned_kernel");
    }
  }
  if (gather && !fused_gather)
    return mkv_gather(reinterpret_cast<mkv_pool *>(p), layer, d_block_indptr, d_block_ids, pd.tok0, pl->B,
                      pl->max_ctx, d_gk, d_gv, gcap, stream);
  return MKV_OK;
}

extern "C" int mkv_decode_attention_planned(mkv_pool *pool, const mkv_decode_plan *plan, int32_t layer,
                                            const void *d_q, void *d_o, const int32_t *d_block_indptr,
                                            const int32_t *d_block_ids, float scale, uint32_t flags,
                                            void *stream) {
  if (!pool || !plan) return set_error(MKV_ERR_INVALID_ARGUMENT, "NULL pool or plan");
  return launch_planned(reinterpret_cast<Pool *>(pool), reinterpret_cast<const Plan *>(plan), layer,
                        nullptr, nullptr, d_q, d_o, d_block_indptr, d_block_ids, scale, flags, stream);
}

extern "C" int mkv_decode_step(mkv_pool *pool, const mkv_decode_plan *plan, int32_t layer,
                               const void *d_k_new, const void *d_v_new, const void *d_q, void *d_o,
                               const int32_t *d_block_indptr, const int32_t *d_block_ids, float scale,
                               uint32_t flags, void *stream) {
  if (!pool || !plan) return set_error(MKV_ERR_INVALID_ARGUMENT, "NULL pool or plan");
  if (!d_k_new || !d_v_new) return set_error(MKV_ERR_INVALID_ARGUMENT, "NULL new K/V rows");
  return launch_planned(reinterpret_cast<Pool *>(pool), reinterpret_cast<const Plan *>(plan), layer,
                        d_k_new, d_v_new, d_q, d_o, d_block_indptr, d_block_ids, scale, flags, stream);
}

extern "C" int mkv_decode_step_gather(mkv_pool *pool, const mkv_decode_plan *plan, int32_t layer,
                                      const void *d_k_new, const void *d_v_new, const void *d_q, void *d_o,
                                      const int32_t *d_block_indptr, const int32_t *d_block_ids, void *d_out_k,
                                      void *d_out_v, int64_t out_capacity_tokens, float scale, uint32_t flags,
                                      void *stream) {
  if (!pool || !plan) return set_error(MKV_ERR_INVALID_ARGUMENT, "NULL pool or plan");
  if (!d_k_new || !d_v_new) return set_error(MKV_ERR_INVALID_ARGUMENT, "NULL new K/V rows");
  if (!d_out_k || !d_out_v) return set_error(MKV_ERR_INVALID_ARGUMENT, "NULL gather outputs");
  if (reinterpret_cast<const Plan *>(plan)->all_partial)
    return set_error(MKV_ERR_INVALID_ARGUMENT, "a suffix plan's contexts are not whole sequences");
  return launch_planned(reinterpret_cast<Pool *>(pool), reinterpret_cast<const Plan *>(plan), layer, d_k_new,
                        d_v_new, d_q, d_o, d_block_indptr, d_block_ids, scale, flags, stream, true, d_out_k,
                        d_out_v, out_capacity_tokens);
}

static int launch_ext_tiles(Pool *p, KArgs &a, ExtArgs &e, int split_cap, hipStream_t hs, bool beside = false);

extern "C" int mkv_decode_step_shared_prefix(mkv_pool *pool, const mkv_decode_plan *plan, int32_t layer,
                                             const void *d_k_new, const void *d_v_new, const void *d_q,
                                             void *d_o, const int32_t *d_prefix_ids, int32_t prefix_blocks,
                                             const int32_t *d_block_indptr, const int32_t *d_block_ids,
                                             float scale, uint32_t flags, void *stream) {
  if (!pool || !plan) return set_error(MKV_ERR_INVALID_ARGUMENT, "NULL pool or plan");
  Pool *p = reinterpret_cast<Pool *>(pool);
  const Plan *pl = reinterpret_cast<const Plan *>(plan);
  const Geom &g = p->g;
  if (pl->pool != p) return set_error(MKV_ERR_INVALID_ARGUMENT, "plan belongs to another pool");
  if (pl->B < 1) return set_error(MKV_ERR_INVALID_ARGUMENT, "plan was never built");
  if (!pl->all_partial)
    return set_error(MKV_ERR_INVALID_ARGUMENT, "the plan must be built with mkv_decode_plan_build_suffixes");
  if (!d_prefix_ids) {  // the prefix given at build time
    if (!pl->has_tables || pl->n_prefix < 1)
      return set_error(MKV_ERR_INVALID_ARGUMENT,
                       "no prefix ids: pass device ids, or build the plan with mkv_decode_plan_build_shared_prefix");
    d_prefix_ids = pl->d_meta + pl->flat_off + pl->total;
    prefix_blocks = pl->n_prefix;
  }
  if (prefix_blocks < 1 || prefix_blocks > INT32_MAX / (2 * kPageSize))
    return set_error(MKV_ERR_INVALID_ARGUMENT, "need a prefix of >= 1 block ids");
  if ((d_k_new == nullptr) != (d_v_new == nullptr))
    return set_error(MKV_ERR_INVALID_ARGUMENT, "give both new K and V rows, or neither");
  bool use_mfma = false;
  int rc = check_common(p, layer, flags, scale, use_mfma);
  if (rc) return rc;
  if (!use_mfma || g.Hq / g.Hkv > kQChunkMfma)
    return set_error(MKV_ERR_INVALID_ARGUMENT,
                     "shared-prefix decode needs bf16 KV, head_dim 64/128/256 and at most 16 query heads per KV head");
  if (!d_q || !d_o) return set_error(MKV_ERR_INVALID_ARGUMENT, "NULL device pointer");
  if ((d_block_indptr == nullptr) != (d_block_ids == nullptr))
    return set_error(MKV_ERR_INVALID_ARGUMENT, "give both device table arrays, or neither");
  if (!d_block_indptr && !pl->has_tables)
    return set_error(MKV_ERR_INVALID_ARGUMENT,
                     "no suffix tables: pass device tables, or build the plan with its host tables");
  if (!aligned16(d_q) || !aligned16(d_o)) return set_error(MKV_ERR_INVALID_ARGUMENT, "q and o must be 16-byte aligned");
  DeviceGuard guard(p->device);
  hipStream_t hs = reinterpret_cast<hipStream_t>(stream);
  // 1. The prefix: the B decode queries as one chunk over the prefix's keys,
  //    no causal mask, f32 partials per key range (pool workspace). When the
  //    plan's suffix pieces leave room for it (one per CU), it runs on the
  //    pool's second stream, forked from the caller's stream here and joined
  //    back before the merge, beside the suffixes. The events order device
  //    work only, so they skip the system-scope fence.
  const bool beside = pl->beside;
  if (beside && !p->aux) {
    // The stream is published last, so a failed creation leaves none of the
    // three half made for the next call.
    if (!p->aux_fork)
      MKV_CHECK_HIP(hipEventCreateWithFlags(&p->aux_fork, hipEventDisableTiming | hipEventDisableSystemFence));
    if (!p->aux_join)
      MKV_CHECK_HIP(hipEventCreateWithFlags(&p->aux_join, hipEventDisableTiming | hipEventDisableSystemFence));
    hipStream_t aux = nullptr;
    MKV_CHECK_HIP(hipStreamCreateWithFlags(&aux, hipStreamNonBlocking));
    p->aux = aux;
  }
  KArgs ap = make_kargs(p, layer, d_q, d_o, nullptr, d_prefix_ids, scale, flags, true);
  ExtArgs e{};
  e.B = 1;
  e.max_ctx = e.v_ctx = prefix_blocks * kPageSize;
  e.max_q = e.v_nq = pl->B;
  e.causal = 0;
  e.partial = 1;
  if (beside) {
    MKV_CHECK_HIP(hipEventRecord(p->aux_fork, hs));
    MKV_CHECK_HIP(hipStreamWaitEvent(p->aux, p->aux_fork, 0));
    rc = launch_ext_tiles(p, ap, e, 16, p->aux, true);
    MKV_CHECK_HIP(hipEventRecord(p->aux_join, p->aux));
  } else {
    rc = launch_ext_tiles(p, ap, e, 16, hs);
  }
  // 2. The suffixes (and the fused append): every sequence's partials, one
  //    per piece, in the plan's workspace.
  if (!rc)
    rc = launch_planned(p, pl, layer, d_k_new, d_v_new, d_q, d_o, d_block_indptr, d_block_ids, scale, flags,
                        stream, false);
  // The join comes before any return: nothing the caller enqueues after this
  // call (nor the merge) may overtake the prefix tiles.
  if (beside) MKV_CHECK_HIP(hipStreamWaitEvent(hs, p->aux_join, 0));
  if (rc) return rc;
  // 3. Both runs of partials merged into o.
  KArgs am = make_kargs(p, layer, d_q, d_o, d_block_indptr, d_block_ids, scale, flags, true);
  am.ws_ml = reinterpret_cast<float *>(pl->d_ws);
  am.ws_o = reinterpret_cast<float *>(reinterpret_cast<uint8_t *>(pl->d_ws) + pl->ws_ml_bytes);
  const PlanDev pd = plan_dev(pl);
  const PrefixParts pp{ap.ws_ml, ap.ws_o, e.splits};
  const dim3 mgrid((unsigned)(((int64_t)pl->B * g.Hq + 3) / 4));
  switch (g.D) {
    case 64: hipLaunchKernelGGL((merge_prefix_kernel<64, true>), mgrid, dim3(256), 0, hs, am, pd, pp); break;
    case 128: hipLaunchKernelGGL((merge_prefix_kernel<128, true>), mgrid, dim3(256), 0, hs, am, pd, pp); break;
    default: hipLaunchKernelGGL((merge_prefix_kernel<256, true>), mgrid, dim3(256), 0, hs, am, pd, pp); break;
  }
  MKV_CHECK_LAUNCH("merge_prefix_kernel");
  return MKV_OK;
}

extern "C" int mkv_extend_attention(mkv_pool *pool, int32_t layer, const void *d_q, void *d_o,
                                    const int32_t *d_q_indptr, const int32_t *d_block_indptr,
                                    const int32_t *d_block_ids, const int32_t *d_ctx_lens, int32_t num_seqs,
                                    int32_t max_q_len, int32_t max_ctx_len, float scale, uint32_t flags,
                                    void *stream) {
  if (!pool) return set_error(MKV_ERR_INVALID_ARGUMENT, "NULL pool");
  Pool *p = reinterpret_cast<Pool *>(pool);
  const Geom &g = p->g;
  bool use_mfma = false;
  int rc = check_common(p, layer, flags, scale, use_mfma);
  if (rc) return rc;
  if (!d_q || !d_o || !d_q_indptr || !d_block_indptr || !d_block_ids || !d_ctx_lens)
    return set_error(MKV_ERR_INVALID_ARGUMENT, "NULL device pointer");
  if (num_seqs < 0 || max_q_len < 0 || max_ctx_len < 0)
    return set_error(MKV_ERR_INVALID_ARGUMENT, "negative sizes");
  if (num_seqs == 0 || max_q_len == 0) return MKV_OK;
  if (max_q_len > max_ctx_len)
    return set_error(MKV_ERR_INVALID_ARGUMENT, "max_q_len %d > max_ctx_len %d", max_q_len, max_ctx_len);
  const int G = g.Hq / g.Hkv;
  if (!aligned16(d_q) || !aligned16(d_o)) return set_error(MKV_ERR_INVALID_ARGUMENT, "q and o must be 16-byte aligned");
  if (!use_mfma || G > 16) {  // per-token segments on the decode kernels (see attn_ext_split_kernel)
    const int64_t tokens = (int64_t)num_seqs * max_q_len;  // upper bound; the kernel reads q_indptr[B]
    DeviceGuard guard(p->device);
    hipStream_t hs = reinterpret_cast<hipStream_t>(stream);
    KArgs a = make_kargs(p, layer, d_q, d_o, d_block_indptr, d_block_ids, scale, flags, use_mfma);
    ExtSplitArgs x;
    x.q_indptr = d_q_indptr;
    x.ctx = d_ctx_lens;
    x.B = num_seqs;
    x.max_ctx = max_ctx_len;
    x.total_units = tokens * g.Hkv * a.nqc;
    const int64_t wgs = (x.total_units + 3) / 4;
    if (wgs > INT32_MAX) return set_error(MKV_ERR_INVALID_ARGUMENT, "launch too large");
    MKV_DISPATCH(attn_ext_split_kernel, dim3((unsigned)wgs), dim3(256), hs, a, x);
    MKV_CHECK_LAUNCH("attn_ext_split_kernel");
    return MKV_OK;
  }
  DeviceGuard guard(p->device);
  hipStream_t hs = reinterpret_cast<hipStream_t>(stream);
  KArgs a = make_kargs(p, layer, d_q, d_o, d_block_indptr, d_block_ids, scale, flags, true);
  ExtArgs e{};
  e.q_indptr = d_q_indptr;
  e.ctx = d_ctx_lens;
  e.B = num_seqs;
  e.max_ctx = max_ctx_len;
  e.max_q = max_q_len;
  e.causal = 1;
  return launch_ext_tiles(p, a, e, 4, hs);
}

extern "C" int mkv_extend_attention_host(mkv_pool *pool, int32_t layer, const void *d_q, void *d_o,
                                         const int32_t *h_q_lens, const int32_t *h_ctx_lens,
                                         const uint32_t *h_block_indptr, const uint32_t *h_block_ids,
                                         int32_t num_seqs, float scale, uint32_t flags, void *stream) {
  if (!pool) return set_error(MKV_ERR_INVALID_ARGUMENT, "NULL pool");
  Pool *p = reinterpret_cast<Pool *>(pool);
  if (num_seqs < 0) return set_error(MKV_ERR_INVALID_ARGUMENT, "num_seqs < 0");
  if (num_seqs == 0) return MKV_OK;
  if (!h_q_lens) return set_error(MKV_ERR_INVALID_ARGUMENT, "NULL q_lens");
  int32_t max_ctx = 0;
  int rc = check_host_tables(p->g, h_block_indptr, h_block_ids, h_ctx_lens, num_seqs, &max_ctx);
  if (rc) return rc;
  int32_t max_q = 0;
  int64_t rows = 0;
  for (int32_t b = 0; b < num_seqs; b++) {
    if (h_q_lens[b] < 0 || h_q_lens[b] > h_ctx_lens[b])
      return set_error(MKV_ERR_INVALID_ARGUMENT, "sequence %d: %d new tokens outside [0, ctx %d]", b, h_q_lens[b],
                       h_ctx_lens[b]);
    max_q = std::max(max_q, h_q_lens[b]);
    rows += h_q_lens[b];
  }
  if (rows > INT32_MAX) return set_error(MKV_ERR_INVALID_ARGUMENT, "more than 2^31 - 1 query rows");
  if (max_q == 0) return MKV_OK;
  const size_t nids = h_block_indptr[num_seqs];
  const size_t n = 3 * (size_t)num_seqs + 2 + nids;  // q_indptr | indptr | ctx | ids
  DeviceGuard guard(p->device);
  hipStream_t hs = reinterpret_cast<hipStream_t>(stream);
  // Every layer of a step passes the same chunks and tables: uploaded once
  // per step.
  std::vector<int32_t> &stg = p->stage_tmp;
  stg.resize(n);
  int32_t *qp = stg.data(), *ip = qp + num_seqs + 1, *cl = ip + num_seqs + 1, *ix = cl + num_seqs;
  qp[0] = 0;
  for (int32_t b = 0; b < num_seqs; b++) qp[b + 1] = qp[b] + h_q_lens[b];
  for (int32_t b = 0; b <= num_seqs; b++) ip[b] = (int32_t)h_block_indptr[b];
  std::memcpy(cl, h_ctx_lens, (size_t)num_seqs * 4);
  if (nids) std::memcpy(ix, h_block_ids, nids * 4);
  MetaSlot *sl = nullptr;
  if ((rc = stage_cached(p, p->extend_cache, stg.data(), n, hs, &sl))) return rc;
  const int32_t *d = sl->d;
  rc = mkv_extend_attention(pool, layer, d_q, d_o, d, d + num_seqs + 1, d + 3 * num_seqs + 2, d + 2 * num_seqs + 2,
                            num_seqs, max_q, max_ctx, scale, flags, stream);
  const int rr = meta_release(sl, hs);
  return rc ? rc : rr;
}

// The extend kernel's instantiation for head_dim D, W waves and TP
// sub-tiles of 16 positions per workgroup.
static const void *ext_kernel(int D, int W, int TP) {
  const void *fn = nullptr;
#define MKV_EXT_FN(DD, TT)                                                                                  \
  do {                                                                                                      \
    switch (W / TT) {                                                                                       \
      case 1: fn = reinterpret_cast<const void *>(&attn_extend_kernel<DD, 1 * TT, kExtKB, kExtR, TT>); break; \
      case 2: fn = reinterpret_cast<const void *>(&attn_extend_kernel<DD, 2 * TT, kExtKB, kExtR, TT>); break; \
      case 4: fn = reinterpret_cast<const void *>(&attn_extend_kernel<DD, 4 * TT, kExtKB, kExtR, TT>); break; \
      case 8: fn = reinterpret_cast<const void *>(&attn_extend_kernel<DD, 8 * TT, kExtKB, kExtR, TT>); break; \
      default: fn = reinterpret_cast<const void *>(&attn_extend_kernel<DD, 16, kExtKB, kExtR, 1>); break;     \
    }                                                                                                       \
  } while (0)
  switch (D) {
    case 64: if (TP == 2) MKV_EXT_FN(64, 2); else MKV_EXT_FN(64, 1); break;
    case 128: if (TP == 2) MKV_EXT_FN(128, 2); else MKV_EXT_FN(128, 1); break;
    default:
      fn = W == 4 ? reinterpret_cast<const void *>(&attn_extend_kernel<256, 4, kExtKB, kExtR, 1>)
                  : reinterpret_cast<const void *>(&attn_extend_kernel<256, 8, kExtKB, kExtR, 1>);
      break;
  }
#undef MKV_EXT_FN
  return fn;
}

// Resident workgroups per CU of an extend instantiation (occupancy query,
// once per pool and instantiation); -1 when unknown.
static int ext_resident_per_cu(Pool *p, const void *fn, int W, int TP) {
  const Geom &g = p->g;
  int &per_cu = p->ext_per_cu[g.D == 64 ? 0 : g.D == 128 ? 1 : 2][W == 1 ? 0 : W == 2 ? 1 : W == 4 ? 2 : W == 8 ? 3 : 4][TP - 1];
  if (per_cu == 0) {
    int n_cu = 0;
    DeviceGuard guard(p->device);
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n_cu, fn, 64 * W, 0) != hipSuccess) {
      (void)hipGetLastError();  // leave no sticky error: no splitting
      n_cu = 0;
    }
    per_cu = n_cu > 0 ? n_cu : -1;
  }
  return per_cu;
}

// MFMA query tiles of the extend kernel for e (B, max_q, max_ctx, causal,
// partial and the sequence arguments set): picks the instantiation and the
// key-range split (at most split_cap), grows the pool workspace when
// partials are stored, launches, and merges the splits unless e.partial
// (then a.ws_ml / a.ws_o and e.splits describe the partials left). With
// beside, the tiles share the device with a decode launch that holds one
// workgroup per CU: one sub-tile per workgroup, and the split aims at one
// workgroup per CU.
static int launch_ext_tiles(Pool *p, KArgs &a, ExtArgs &e, int split_cap, hipStream_t hs, bool beside) {
  const Geom &g = p->g;
  const int G = g.Hq / g.Hkv;
  const int64_t num_seqs = e.B, max_q_len = e.max_q, max_ctx_len = e.max_ctx;
  if (((max_q_len + 15) / 16 * g.Hq * num_seqs) * split_cap + 8 > INT32_MAX)
    return set_error(MKV_ERR_INVALID_ARGUMENT, "grid too large");
  e.splits = 1;
  // Waves per 16-position sub-tile: the next power of two >= G. Two
  // sub-tiles per workgroup share each K/V tile (K/V streamed once per 32
  // positions) where that stays within 16 waves and their register budget
  // (head_dim <= 128) and chunks are longer than one sub-tile. Measured at
  // Qwen-7B heads: 8 x 512 after 4k 526 -> 480 us, 8 x 2,048 prompts 560 ->
  // 534 us; 16-token chunks would leave half the waves idle (168 -> 220 us).
  // At head_dim 256 a workgroup has at least 4 waves: waves past G only
  // share the loads, and one or two waves would each carry 16-32 loads per
  // ring stage (register spills). It has at most 8: more than 8 query heads
  // per KV head go to groups of 8 in workgroups of their own (16 waves cap
  // the registers at 128, and the head_dim-256 state then spills).
  const int WG = G <= 1 && g.D < 256 ? 1 : G <= 2 && g.D < 256 ? 2 : G <= 4 ? 4 : G <= 8 || g.D == 256 ? 8 : 16;
  e.hgroups = (G + WG - 1) / WG;
  const int TP = (!beside && WG <= 8 && g.D <= 128 && max_q_len > 16) ? 2 : 1;
  const int W = WG * TP;
  const int64_t tiles = ((int64_t)max_q_len + 16 * TP - 1) / (16 * TP);
  // (tile, KV head, head group, sequence) workgroups
  const int64_t per_split = tiles * g.Hkv * e.hgroups * num_seqs;
  const void *fn = ext_kernel(g.D, W, TP);
  // When the launch leaves resident workgroup slots empty (short chunks over
  // long contexts: one workgroup per (sequence, KV head) streams a whole
  // context), each key range splits in up to 4, at least 8 steps apiece;
  // the f32 partials go to the pool-owned workspace and a second launch
  // merges them. Slots = resident workgroups per CU of this instantiation
  // (occupancy query, once per pool) x CUs; one per CU beside a decode launch.
  const int per_cu = ext_resident_per_cu(p, fn, W, TP);
  const int cus = device_cus(p);
  const int64_t slots = per_cu > 0 && cus > 0 ? (beside ? 1 : (int64_t)per_cu) * cus : 0;
  const int64_t steps_max = ((int64_t)(max_ctx_len + kPageSize - 1) / kPageSize + kExtKB - 1) / kExtKB;
  if (per_split < slots)
    e.splits = (int32_t)std::min<int64_t>({(int64_t)split_cap, (slots + per_split - 1) / per_split,
                                           std::max<int64_t>(1, steps_max / 8)});
  const int64_t rows = (int64_t)num_seqs * max_q_len * g.Hq;  // bounds the (token, query head) rows
  if (e.splits > 1 || e.partial) {
    const uint64_t ml_bytes = ((uint64_t)rows * e.splits * 8 + 255) / 256 * 256;
    const uint64_t need = ml_bytes + (uint64_t)rows * e.splits * g.D * 4;
    if (p->ws_bytes < need) {
      const uint64_t cap = std::max<uint64_t>(need, p->ws_bytes + p->ws_bytes / 2);
      MKV_CHECK_HIP(hipStreamSynchronize(hs));  // earlier launches may read the old buffer
      if (p->ws) MKV_CHECK_HIP(hipFree(p->ws));
      p->ws = nullptr;
      p->ws_bytes = 0;
      MKV_CHECK_HIP(hipMalloc(&p->ws, cap));
      p->ws_bytes = cap;
    }
    a.ws_ml = reinterpret_cast<float *>(p->ws);
    a.ws_o = reinterpret_cast<float *>(reinterpret_cast<uint8_t *>(p->ws) + ml_bytes);
  }
  const int64_t total = per_split * e.splits;  // linear index -> (tile, KV head, group, sequence, split), by XCD
  e.tiles = (int32_t)tiles;
  e.per_xcd = (int32_t)((total + 7) / 8);
  const dim3 grid((unsigned)(8 * (int64_t)e.per_xcd)), block(64 * W);
  void *args[] = {&a, &e};
  MKV_CHECK_HIP(hipLaunchKernel(fn, grid, block, args, 0, hs));
  MKV_CHECK_LAUNCH("attn_extend_kernel");
  if (e.splits > 1 && !e.partial) {
    const dim3 mgrid((unsigned)((rows + 3) / 4));
    switch (g.D) {
      case 64: hipLaunchKernelGGL((merge_ext_kernel<64, true>), mgrid, dim3(256), 0, hs, a, e); break;
      case 128: hipLaunchKernelGGL((merge_ext_kernel<128, true>), mgrid, dim3(256), 0, hs, a, e); break;
      default: hipLaunchKernelGGL((merge_ext_kernel<256, true>), mgrid, dim3(256), 0, hs, a, e); break;
    }
    MKV_CHECK_LAUNCH("merge_ext_kernel");
  }
  return MKV_OK;
}
