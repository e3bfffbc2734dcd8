// Internal definitions shared by the libmitten_kv translation units.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <string>
#include <vector>

#include "mitten_kv.h"

namespace mkv {

constexpr int kPageSize = 16;
constexpr int kWave = 64;

// Pool geometry in bytes. Layout: [L][2][blocks][page][Hkv][D].
struct Geom {
  int32_t L, Hkv, Hq, D, ps, dtype;
  int64_t nblocks;
  int32_t es;          // element bytes
  int64_t row_bytes;   // one token, all KV heads: Hkv*D*es
  int64_t block_bytes; // ps * row_bytes
  int64_t plane_bytes; // nblocks * block_bytes (one layer, K or V)
};

// Host metadata staging for the *_host entry points. The caller's host
// arrays are copied into a pinned slot before the call returns and uploaded
// on the caller's stream ahead of the launch that reads them. Slots are used
// round-robin; a slot is reused once the stream has passed the launches that
// read it (its `done` event), so the wait almost never blocks.
constexpr int kMetaSlots = 8;
struct MetaSlot {
  int32_t *h = nullptr;  // pinned host
  int32_t *d = nullptr;  // device
  size_t cap = 0;        // int32 elements of both
  hipEvent_t done = nullptr;
  bool pending = false;
  uint64_t gen = 0;  // counts acquisitions (a staged array is current while gen is unchanged)
};

// The last array one entry point staged: the slot that holds it, that
// slot's generation then, the stream it was uploaded on, and the values.
struct StagedCache {
  int slot = -1;
  uint64_t gen = 0;
  hipStream_t stream = nullptr;
  std::vector<int32_t> vals;
};

struct Pool {
  mkv_pool_desc desc;
  Geom g;
  int device = 0;
  uint8_t *data = nullptr;   // pool buffer
  uint64_t bytes = 0;
  uint32_t *d_err = nullptr; // device error word
  void *ws = nullptr;        // pool-owned attention workspace
  uint64_t ws_bytes = 0;
  int64_t coop_slots = -1;   // resident workgroups of the decode kernel (-1: not yet queried)
  int cus = 0;               // compute units of the device (0: not yet queried)
  int ext_per_cu[3][5][2] = {};  // resident extend workgroups per CU by (head_dim, waves, sub-tiles); 0: not yet queried
  // The shared-prefix step's second stream, which runs the prefix tiles
  // beside the suffix pieces, and its fork / join events (created on first
  // use). beside: 1 when one prefix workgroup fits beside one decode-kernel
  // workgroup on every CU, -1 when not, 0 before the first query.
  hipStream_t aux = nullptr;
  hipEvent_t aux_fork = nullptr, aux_join = nullptr;
  int beside = 0;
  // Caller events recorded around the next decode attention kernel (one
  // shot; mkv_pool_set_launch_events).
  hipEvent_t ev_start = nullptr, ev_end = nullptr;
  MetaSlot meta[kMetaSlots];
  int meta_next = 0;
  // The last host arrays staged by the append, gather, extend and fused prep
  // entry points (an engine step passes the same ones to every layer), and a
  // scratch array to assemble a staged array in.
  StagedCache app_cache, gather_cache, extend_cache, prep_cache;
  std::vector<int32_t> stage_tmp;
};

// Next staging slot with room for n int32 values (waits for its previous
// readers, grows it when needed). Fill s->h[0..n), then meta_upload, launch,
// meta_release.
int meta_acquire(Pool *p, size_t n, hipStream_t hs, MetaSlot **out);
int meta_upload(MetaSlot *s, size_t n, hipStream_t hs);
int meta_release(MetaSlot *s, hipStream_t hs);
void meta_free(Pool *p);
// meta_acquire + fill + meta_upload of h[0..n), unless the cache's last
// array equals it, was uploaded on the same stream, and its slot has not
// been claimed since: then that device copy is handed out again. Either
// way the caller launches from (*out)->d and calls meta_release.
int stage_cached(Pool *p, StagedCache &c, const int32_t *h, size_t n, hipStream_t hs, MetaSlot **out);

// Looks up this device's address of the static scratch of
// mkv_decode_attention_static (once per device; called by mkv_pool_create).
int static_scratch_setup(int device);

// Host-side checks of the engine's u32 metadata against the pool (pure CPU).
int check_host_slots(const Geom &g, const uint32_t *slots, int32_t n);
// Tables of num_seqs sequences: indptr monotone from 0, every id < nblocks,
// table b holds >= ceil(len_b / page) ids, 1 <= len_b. Returns the largest
// len in *max_len (when non-NULL).
int check_host_tables(const Geom &g, const uint32_t *indptr, const uint32_t *ids, const int32_t *lens,
                      int32_t num_seqs, int32_t *max_len);

// Thread-local last-error message and status helpers.
int set_error(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
int hip_fail(hipError_t e, const char *what);

// Sets the pool's device current for the lifetime of the guard.
struct DeviceGuard {
  int prev = -1;
  bool ok = true;
  explicit DeviceGuard(int dev) {
    if (hipGetDevice(&prev) != hipSuccess) prev = -1;
    if (prev != dev) ok = hipSetDevice(dev) == hipSuccess;
    if (!ok) (void)hipGetLastError();  // reported by the caller's status, not left for the next HIP check
  }
  ~DeviceGuard() {
    int cur = -1;
    if (prev >= 0 && hipGetDevice(&cur) == hipSuccess && cur != prev) (void)hipSetDevice(prev);
  }
};

inline bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

#define MKV_CHECK_HIP(expr)                      \
  do {                                           \
    hipError_t e_ = (expr);                      \
    if (e_ != hipSuccess) return ::mkv::hip_fail(e_, #expr); \
  } while (0)

// After a kernel launch.
#define MKV_CHECK_LAUNCH(name)                   \
  do {                                           \
    hipError_t e_ = hipGetLastError();           \
    if (e_ != hipSuccess) return ::mkv::hip_fail(e_, name); \
  } while (0)

// ---- device helpers -------------------------------------------------------

__device__ __forceinline__ void record_error(uint32_t *d_err, uint32_t bit) {
  atomicOr(d_err, bit);
}

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// DPP lane move within 16-lane rows (CTRL a dpp_ctrl code; all lanes active).
template <int CTRL>
__device__ __forceinline__ float dpp_f(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xf, 0xf, false));
}

// Sum over the LPR lanes of each row group (LPR = 4, 8, ..., 64 consecutive
// lanes); every lane of the group gets the same bits (each step adds two
// values that are equal up to the order of a commutative addition).
template <int LPR>
__device__ __forceinline__ float row_sum(float v) {
  v += dpp_f<0xb1>(v);                             // quad_perm [1,0,3,2]: lane ^ 1
  if constexpr (LPR >= 4) v += dpp_f<0x4e>(v);     // quad_perm [2,3,0,1]: lane ^ 2
  if constexpr (LPR >= 8) v += dpp_f<0x141>(v);    // row_half_mirror: the other quad
  if constexpr (LPR >= 16) v += dpp_f<0x140>(v);   // row_mirror: the other half-row
  if constexpr (LPR >= 32) v += __shfl_xor(v, 16);
  if constexpr (LPR >= 64) v += __shfl_xor(v, 32);
  return v;
}

// Maximum over the 16 lanes of each DPP row, in every lane of the row.
__device__ __forceinline__ float row16_max(float v) {
  v = fmaxf(v, dpp_f<0xb1>(v));   // lane ^ 1
  v = fmaxf(v, dpp_f<0x4e>(v));   // lane ^ 2
  v = fmaxf(v, dpp_f<0x141>(v));  // the other quad of the half-row
  v = fmaxf(v, dpp_f<0x140>(v));  // the other half-row
  return v;
}

// f32 -> bf16 bits, round to nearest even (NaN kept NaN).
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x40u;
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}
// Two f32 -> packed bf16 pair (lo in bits 0-15), round to nearest even: one
// v_cvt_pk_bf16_f32 on gfx950.
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  const bf16x2_t v = {(__bf16)lo, (__bf16)hi};
  return __builtin_bit_cast(uint32_t, v);
}

}  // namespace mkv
