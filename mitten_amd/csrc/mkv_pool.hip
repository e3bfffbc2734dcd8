// Device KV pool, KV data movement kernels (append, gather, copy_blocks),
// host-side validators, device buffers and the error API of libmitten_kv.
//
// All three movement kernels are pure HBM streams: every thread moves whole
// 16-byte chunks (global_load_dwordx4 / global_store_dwordx4), consecutive
// lanes touch consecutive chunks of one contiguous row or block, and every
// slot / block id is range-checked before it is dereferenced.
#include <algorithm>
#include <cstring>
#include <new>
#include <vector>

#include "mkv_internal.h"

namespace mkv {

typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));

static thread_local std::string g_last_error;

int set_error(int code, const char *fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int hip_fail(hipError_t e, const char *what) {
  // The failure is the call's status: clear the thread's last HIP error so
  // that the caller's own next error check (torch's, after its next launch)
  // does not report it a second time.
  (void)hipGetLastError();
  int code = (e == hipErrorOutOfMemory) ? MKV_ERR_OUT_OF_MEMORY : MKV_ERR_HIP;
  return set_error(code, "%s failed: %s (%d)", what, hipGetErrorString(e), (int)e);
}

static int validate_desc(const mkv_pool_desc *d) {
  if (!d) return set_error(MKV_ERR_INVALID_ARGUMENT, "desc is NULL");
  if (d->num_layers < 1 || d->num_kv_heads < 1 || d->num_q_heads < 1 || d->num_blocks < 1)
    return set_error(MKV_ERR_INVALID_ARGUMENT,
                     "num_layers, num_kv_heads, num_q_heads and num_blocks must be >= 1");
  if (d->num_q_heads % d->num_kv_heads)
    return set_error(MKV_ERR_INVALID_ARGUMENT, "num_q_heads (%d) is not a multiple of num_kv_heads (%d)",
                     d->num_q_heads, d->num_kv_heads);
  if (d->head_dim < 8 || d->head_dim > 512 || d->head_dim % 8)
    return set_error(MKV_ERR_INVALID_ARGUMENT, "head_dim (%d) must be a multiple of 8 in [8, 512]",
                     d->head_dim);
  if (d->page_size != kPageSize)
    return set_error(MKV_ERR_INVALID_ARGUMENT, "page_size must be %d (got %d)", kPageSize,
                     d->page_size);
  if (d->dtype != MKV_DTYPE_F32 && d->dtype != MKV_DTYPE_BF16)
    return set_error(MKV_ERR_INVALID_ARGUMENT, "unknown dtype %d", d->dtype);
  if (d->num_blocks > (int64_t)INT32_MAX / kPageSize)
    return set_error(MKV_ERR_INVALID_ARGUMENT, "num_blocks too large for int32 slot ids");
  return MKV_OK;
}

static Geom make_geom(const mkv_pool_desc *d) {
  Geom g;
  g.L = d->num_layers;
  g.Hkv = d->num_kv_heads;
  g.Hq = d->num_q_heads;
  g.D = d->head_dim;
  g.ps = d->page_size;
  g.dtype = d->dtype;
  g.nblocks = d->num_blocks;
  g.es = d->dtype == MKV_DTYPE_F32 ? 4 : 2;
  g.row_bytes = (int64_t)g.Hkv * g.D * g.es;
  g.block_bytes = g.ps * g.row_bytes;
  g.plane_bytes = g.nblocks * g.block_bytes;
  return g;
}

// ---- kernels ------------------------------------------------------------------

// grid.y = layer. The chunk space of a launch is num_tokens * 2 * cpr
// 16-byte chunks (token-major, then K/V, then the row's chunks); a thread
// takes PER chunks 256 apart per pass, issues all their loads and the slot
// ids of their tokens, then the stores. Loads and stores are nontemporal (a
// row is moved once). Indices are 32-bit (the host keeps the chunk count of
// one launch below 2^31). PER is 1 for small appends (a 512-token chunk
// batch is latency-bound: as many waves as possible in flight) and grows to
// 8 for large ones (loads in flight per thread).
template <int PER>
__global__ void __launch_bounds__(256)
append_kernel(uint8_t *__restrict__ pool, int32_t layer0, const uint8_t *__restrict__ k,
              const uint8_t *__restrict__ v, const int32_t *__restrict__ slots, uint32_t total,
              uint32_t cpr, int64_t src_layer_stride, Geom g, uint32_t *__restrict__ d_err) {
  const uint32_t per_tok = 2 * cpr;
  const uint32_t nslots = (uint32_t)(g.nblocks * kPageSize);  // < 2^31 (checked at pool creation)
  const int layer = layer0 + (int)blockIdx.y;
  uint8_t *const kbase = pool + (int64_t)layer * 2 * g.plane_bytes;
  const int64_t src_off = (int64_t)blockIdx.y * src_layer_stride;
  const uint32_t stride = gridDim.x * 256u * PER;
  for (uint32_t base = blockIdx.x * 256u * PER + threadIdx.x; base < total; base += stride) {
    u32x4v r[PER];
    int32_t sl[PER];
#pragma unroll
    for (int u = 0; u < PER; u++) {  // clamped past the end: loaded, never stored
      const uint32_t c = min(base + u * 256u, total - 1);
      const uint32_t t = c / per_tok, rem = c - t * per_tok;
      const uint32_t kv = rem >= cpr, cc = rem - kv * cpr;
      r[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4v *>(
          (kv ? v : k) + src_off + ((int64_t)t * cpr + cc) * 16));
      sl[u] = slots[t];
    }
#pragma unroll
    for (int u = 0; u < PER; u++) {
      const uint32_t c = base + u * 256u;
      if (c >= total) break;
      const uint32_t t = c / per_tok, rem = c - t * per_tok;
      const uint32_t kv = rem >= cpr, cc = rem - kv * cpr;
      const uint32_t s = (uint32_t)sl[u];
      if (s >= nslots) {  // negative ids wrap above nslots
        if (rem == 0) record_error(d_err, MKV_DEVERR_SLOT);
        continue;
      }
      uint8_t *dst = kbase + kv * g.plane_bytes + (int64_t)(s / kPageSize) * g.block_bytes +
                     (int64_t)(s % kPageSize) * g.row_bytes;
      __builtin_nontemporal_store(r[u], reinterpret_cast<u32x4v *>(dst) + cc);
    }
  }
}

// grid.x = block index within a sequence, grid.y = sequence. A workgroup
// moves one block's rows of K and V: every thread issues all its 16-byte
// loads (K chunks, then V chunks) before its stores; loads and stores are
// nontemporal (nothing is reused).
constexpr int kGatherPer = 8;  // 16-byte chunks per thread and pass

__global__ void __launch_bounds__(256)
gather_kernel(const uint8_t *__restrict__ pool, int32_t layer, const int32_t *__restrict__ indptr,
              const int32_t *__restrict__ ids, const int32_t *__restrict__ ctx_indptr,
              int32_t max_ctx, uint8_t *__restrict__ out_k, uint8_t *__restrict__ out_v,
              int64_t out_cap, Geom g, uint32_t *__restrict__ d_err) {
  const int b = blockIdx.y, j = blockIdx.x, tid = threadIdx.x;
  const int64_t c0 = ctx_indptr[b];
  const int64_t n = (int64_t)ctx_indptr[b + 1] - c0;
  if (n < 0 || n > max_ctx || c0 < 0 || c0 + n > out_cap) {
    if (j == 0 && tid == 0) record_error(d_err, MKV_DEVERR_CTX);
    return;
  }
  const int64_t t0 = (int64_t)j * kPageSize;
  if (t0 >= n) return;
  const int64_t tab0 = indptr[b];
  const int64_t tabn = (int64_t)indptr[b + 1] - tab0;
  if (tabn < (n + kPageSize - 1) / kPageSize || tab0 < 0) {
    if (j == 0 && tid == 0) record_error(d_err, MKV_DEVERR_TABLE);
    return;
  }
  const int32_t blk = ids[tab0 + j];
  if (blk < 0 || blk >= g.nblocks) {
    if (tid == 0) record_error(d_err, MKV_DEVERR_BLOCK);
    return;
  }
  const int nt = (int)min<int64_t>(kPageSize, n - t0);
  const uint32_t cph = (uint32_t)(g.D * g.es) >> 4;  // 16-byte chunks per head row
  const uint32_t per_kv = (uint32_t)nt * g.Hkv * cph;  // chunks of K (or V) in this block
  const uint32_t total = 2 * per_kv;
  const uint8_t *kplane = pool + (int64_t)layer * 2 * g.plane_bytes + (int64_t)blk * g.block_bytes;
  for (uint32_t base = tid; base < total; base += 256u * kGatherPer) {
    u32x4v r[kGatherPer];
#pragma unroll
    for (int u = 0; u < kGatherPer; u++) {  // all loads first (clamped past the end, not stored)
      const uint32_t c = min(base + u * 256u, total - 1);
      const uint32_t kv = c >= per_kv, cc = c - kv * per_kv;
      r[u] = __builtin_nontemporal_load(
          reinterpret_cast<const u32x4v *>(kplane + kv * g.plane_bytes + (int64_t)cc * 16));
    }
#pragma unroll
    for (int u = 0; u < kGatherPer; u++) {
      const uint32_t c = base + u * 256u;
      if (c >= total) break;
      const uint32_t kv = c >= per_kv, cc = c - kv * per_kv;
      const uint32_t t = cc / (g.Hkv * cph), h = (cc / cph) % g.Hkv, w = cc % cph;
      const int64_t elem = (c0 * g.Hkv + (int64_t)h * n + t0 + t) * g.D;
      __builtin_nontemporal_store(r[u], reinterpret_cast<u32x4v *>((kv ? out_v : out_k) + elem * g.es) + w);
    }
  }
}

// grid.x = pair, grid.y = group of kCopyPlanes planes (layer * 2 + kv). A
// workgroup copies kCopyPlanes whole block planes: all loads first, then the
// stores, nontemporal.
constexpr int kCopyPlanes = 2;
constexpr int kCopyPer = 8;  // 16-byte chunks per thread and pass

__global__ void __launch_bounds__(256)
copy_blocks_kernel(uint8_t *__restrict__ pool, const int32_t *__restrict__ src,
                   const int32_t *__restrict__ dst, Geom g, uint32_t *__restrict__ d_err) {
  const int i = blockIdx.x, tid = threadIdx.x;
  const int32_t s = src[i], d = dst[i];
  if (s < 0 || s >= g.nblocks || d < 0 || d >= g.nblocks) {
    if (blockIdx.y == 0 && tid == 0) record_error(d_err, MKV_DEVERR_COPY);
    return;
  }
  const int p0 = blockIdx.y * kCopyPlanes;
  const int planes = min(kCopyPlanes, 2 * g.L - p0);
  const uint32_t per_plane = (uint32_t)(g.block_bytes >> 4);
  const uint32_t total = planes * per_plane;
  const uint8_t *sp = pool + p0 * g.plane_bytes + s * g.block_bytes;
  uint8_t *dp = pool + p0 * g.plane_bytes + d * g.block_bytes;
  for (uint32_t base = tid; base < total; base += 256u * kCopyPer) {
    u32x4v r[kCopyPer];
#pragma unroll
    for (int u = 0; u < kCopyPer; u++) {
      const uint32_t c = min(base + u * 256u, total - 1);
      const uint32_t pl = c / per_plane, cc = c - pl * per_plane;
      r[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4v *>(sp + pl * g.plane_bytes) + cc);
    }
#pragma unroll
    for (int u = 0; u < kCopyPer; u++) {
      const uint32_t c = base + u * 256u;
      if (c >= total) break;
      const uint32_t pl = c / per_plane, cc = c - pl * per_plane;
      __builtin_nontemporal_store(r[u], reinterpret_cast<u32x4v *>(dp + pl * g.plane_bytes) + cc);
    }
  }
}

// ---- host metadata staging ----------------------------------------------------------

int meta_acquire(Pool *p, size_t n, hipStream_t hs, MetaSlot **out) {
  MetaSlot *sl = &p->meta[p->meta_next];
  p->meta_next = (p->meta_next + 1) % kMetaSlots;
  // The slot's event only tells the host that the launches reading the
  // slot are done (the device never writes it), so it skips the
  // system-scope cache fence: recorded after every host-form call, a fenced
  // event held the next launch back by about 4.6 us.
  if (!sl->done)
    MKV_CHECK_HIP(hipEventCreateWithFlags(&sl->done, hipEventDisableTiming | hipEventDisableSystemFence));
  if (sl->pending) {  // the launches that read this slot last time are done
    MKV_CHECK_HIP(hipEventSynchronize(sl->done));
    sl->pending = false;
  }
  sl->gen++;
  n = std::max<size_t>(n, 1);
  // A slot starts at 64k values (256 KiB pinned, as much on the device): an
  // engine step's slots, copy pairs and tables of a few thousand sequences fit
  // from the first use. It grows by half again at least, since a batch's
  // tables grow step by step, and each growth frees the old buffers, which
  // synchronises the device.
  if (sl->cap < n) {
    const size_t cap = std::max<size_t>({n, (size_t)1 << 16, sl->cap + sl->cap / 2});
    if (sl->h) MKV_CHECK_HIP(hipHostFree(sl->h));
    if (sl->d) MKV_CHECK_HIP(hipFree(sl->d));
    sl->h = nullptr;
    sl->d = nullptr;
    sl->cap = 0;
    MKV_CHECK_HIP(hipHostMalloc(reinterpret_cast<void **>(&sl->h), cap * 4));
    MKV_CHECK_HIP(hipMalloc(reinterpret_cast<void **>(&sl->d), cap * 4));
    sl->cap = cap;
  }
  (void)hs;
  *out = sl;
  return MKV_OK;
}

int meta_upload(MetaSlot *sl, size_t n, hipStream_t hs) {
  if (n) MKV_CHECK_HIP(hipMemcpyAsync(sl->d, sl->h, n * 4, hipMemcpyHostToDevice, hs));
  return MKV_OK;
}

int meta_release(MetaSlot *sl, hipStream_t hs) {
  MKV_CHECK_HIP(hipEventRecord(sl->done, hs));
  sl->pending = true;
  return MKV_OK;
}

void meta_free(Pool *p) {
  for (MetaSlot &sl : p->meta) {
    if (sl.h) (void)hipHostFree(sl.h);
    if (sl.d) (void)hipFree(sl.d);
    if (sl.done) (void)hipEventDestroy(sl.done);
    sl = MetaSlot();
  }
}

int check_host_slots(const Geom &g, const uint32_t *slots, int32_t n) {
  if (n < 0) return set_error(MKV_ERR_INVALID_ARGUMENT, "num_tokens < 0");
  if (n > 0 && !slots) return set_error(MKV_ERR_INVALID_ARGUMENT, "NULL slot mapping");
  const uint64_t nslots = (uint64_t)g.nblocks * kPageSize;
  for (int32_t i = 0; i < n; i++)
    if (slots[i] >= nslots)
      return set_error(MKV_ERR_INVALID_ARGUMENT, "slot[%d] = %u outside [0, %llu)", i, slots[i],
                       (unsigned long long)nslots);
  return MKV_OK;
}

int check_host_tables(const Geom &g, const uint32_t *indptr, const uint32_t *ids, const int32_t *lens,
                      int32_t num_seqs, int32_t *max_len) {
  if (num_seqs < 0) return set_error(MKV_ERR_INVALID_ARGUMENT, "num_seqs < 0");
  if (!indptr || !lens) return set_error(MKV_ERR_INVALID_ARGUMENT, "NULL indptr or lengths");
  if (indptr[0] != 0) return set_error(MKV_ERR_INVALID_ARGUMENT, "block_indptr[0] = %u, expected 0", indptr[0]);
  if (indptr[num_seqs] > (uint32_t)INT32_MAX)
    return set_error(MKV_ERR_INVALID_ARGUMENT, "more than 2^31 - 1 block ids");
  if (indptr[num_seqs] > 0 && !ids) return set_error(MKV_ERR_INVALID_ARGUMENT, "NULL block ids");
  // Monotone over the whole array before any id is read: the ids array
  // holds indptr[num_seqs] entries, and a later entry that falls back would
  // otherwise let an earlier sequence's reads run past it.
  for (int32_t b = 0; b < num_seqs; b++)
    if (indptr[b + 1] < indptr[b])
      return set_error(MKV_ERR_INVALID_ARGUMENT, "block_indptr not monotone at %d", b);
  int32_t mx = 0;
  for (int32_t b = 0; b < num_seqs; b++) {
    const int32_t n = lens[b];
    if (n < 1) return set_error(MKV_ERR_INVALID_ARGUMENT, "length[%d] = %d < 1", b, n);
    const uint32_t need = (uint32_t)((n + kPageSize - 1) / kPageSize);
    if (indptr[b + 1] - indptr[b] < need)
      return set_error(MKV_ERR_INVALID_ARGUMENT, "sequence %d: %u blocks cannot hold %d tokens", b,
                       indptr[b + 1] - indptr[b], n);
    for (uint32_t i = indptr[b]; i < indptr[b] + need; i++)
      if (ids[i] >= (uint64_t)g.nblocks)
        return set_error(MKV_ERR_INVALID_ARGUMENT, "sequence %d: block id %u (table entry %u) outside the pool of %lld",
                         b, ids[i], i - indptr[b], (long long)g.nblocks);
    mx = std::max(mx, n);
  }
  if (max_len) *max_len = mx;
  return MKV_OK;
}

}  // namespace mkv

using namespace mkv;

// ---- C ABI: pool lifecycle -------------------------------------------------------

extern "C" int mkv_pool_required_bytes(const mkv_pool_desc *desc, uint64_t *out_bytes) {
  int rc = validate_desc(desc);
  if (rc) return rc;
  if (!out_bytes) return set_error(MKV_ERR_INVALID_ARGUMENT, "out_bytes is NULL");
  Geom g = make_geom(desc);
  *out_bytes = (uint64_t)2 * g.L * (uint64_t)g.plane_bytes;
  return MKV_OK;
}

extern "C" int mkv_pool_create(const mkv_pool_desc *desc, int device, mkv_pool **out_pool) {
  int rc = validate_desc(desc);
  if (rc) return rc;
  if (!out_pool) return set_error(MKV_ERR_INVALID_ARGUMENT, "out_pool is NULL");
  *out_pool = nullptr;
  int ndev = 0;
  if (hipGetDeviceCount(&ndev) != hipSuccess || ndev == 0) {
    (void)hipGetLastError();
    return set_error(MKV_ERR_NO_DEVICE, "no HIP device available");
  }
  if (device < 0 || device >= ndev)
    return set_error(MKV_ERR_INVALID_ARGUMENT, "device %d out of range (%d devices)", device, ndev);
  DeviceGuard guard(device);
  if (!guard.ok) return set_error(MKV_ERR_HIP, "hipSetDevice(%d) failed", device);
  int rs = static_scratch_setup(device);  // once per device: the no-allocation entry point's scratch
  if (rs) return rs;
  Pool *p = new (std::nothrow) Pool();
  if (!p) return set_error(MKV_ERR_OUT_OF_MEMORY, "host allocation failed");
  p->desc = *desc;
  p->g = make_geom(desc);
  p->device = device;
  p->bytes = (uint64_t)2 * p->g.L * (uint64_t)p->g.plane_bytes;
  hipError_t e = hipMalloc(reinterpret_cast<void **>(&p->data), p->bytes);
  if (e != hipSuccess) {
    delete p;
    (void)hipGetLastError();
    return set_error(e == hipErrorOutOfMemory ? MKV_ERR_OUT_OF_MEMORY : MKV_ERR_HIP,
                     "pool allocation of %llu bytes failed: %s", (unsigned long long)p->bytes,
                     hipGetErrorString(e));
  }
  e = hipMalloc(reinterpret_cast<void **>(&p->d_err), 256);
  if (e == hipSuccess) e = hipMemset(p->d_err, 0, 256);
  if (e != hipSuccess) {
    (void)hipFree(p->data);
    if (p->d_err) (void)hipFree(p->d_err);
    delete p;
    return hip_fail(e, "error word allocation");
  }
  *out_pool = reinterpret_cast<mkv_pool *>(p);
  return MKV_OK;
}

extern "C" int mkv_pool_destroy(mkv_pool *pool) {
  if (!pool) return MKV_OK;
  Pool *p = reinterpret_cast<Pool *>(pool);
  DeviceGuard guard(p->device);
  (void)hipDeviceSynchronize();
  if (p->ws) (void)hipFree(p->ws);
  if (p->aux_fork) (void)hipEventDestroy(p->aux_fork);
  if (p->aux_join) (void)hipEventDestroy(p->aux_join);
  if (p->aux) (void)hipStreamDestroy(p->aux);
  meta_free(p);
  (void)hipFree(p->d_err);
  (void)hipFree(p->data);
  delete p;
  return MKV_OK;
}

extern "C" int mkv_pool_get_desc(const mkv_pool *pool, mkv_pool_desc *out_desc) {
  if (!pool || !out_desc) return set_error(MKV_ERR_INVALID_ARGUMENT, "NULL argument");
  *out_desc = reinterpret_cast<const Pool *>(pool)->desc;
  return MKV_OK;
}

extern "C" int mkv_pool_buffer(const mkv_pool *pool, void **out_dev_ptr, uint64_t *out_bytes) {
  if (!pool) return set_error(MKV_ERR_INVALID_ARGUMENT, "pool is NULL");
  const Pool *p = reinterpret_cast<const Pool *>(pool);
  if (out_dev_ptr) *out_dev_ptr = p->data;
  if (out_bytes) *out_bytes = p->bytes;
  return MKV_OK;
}

extern "C" int mkv_pool_check(mkv_pool *pool, void *stream, uint32_t *out_bits) {
  if (!pool) return set_error(MKV_ERR_INVALID_ARGUMENT, "pool is NULL");
  Pool *p = reinterpret_cast<Pool *>(pool);
  DeviceGuard guard(p->device);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  uint32_t bits = 0;
  MKV_CHECK_HIP(hipStreamSynchronize(s));
  MKV_CHECK_HIP(hipMemcpy(&bits, p->d_err, sizeof(bits), hipMemcpyDeviceToHost));
  if (bits) MKV_CHECK_HIP(hipMemset(p->d_err, 0, sizeof(bits)));
  if (out_bits) *out_bits = bits;
  if (bits)
    return set_error(MKV_ERR_DEVICE_INDEX, "kernel met out-of-range ids (error bits 0x%x)", bits);
  return MKV_OK;
}

extern "C" int mkv_pool_set_launch_events(mkv_pool *pool, void *ev_start, void *ev_end) {
  if (!pool) return set_error(MKV_ERR_INVALID_ARGUMENT, "pool is NULL");
  if (!ev_start != !ev_end) return set_error(MKV_ERR_INVALID_ARGUMENT, "give both events, or neither");
  Pool *p = reinterpret_cast<Pool *>(pool);
  p->ev_start = reinterpret_cast<hipEvent_t>(ev_start);
  p->ev_end = reinterpret_cast<hipEvent_t>(ev_end);
  return MKV_OK;
}

// ---- C ABI: data movement -----------------------------------------------------------

static int check_layer(const Pool *p, int32_t layer) {
  if (layer < 0 || layer >= p->g.L)
    return set_error(MKV_ERR_INVALID_ARGUMENT, "layer %d out of range [0, %d)", layer, p->g.L);
  return MKV_OK;
}

static int launch_append(Pool *p, int32_t layer0, int32_t nlayers, const void *d_k,
                         const void *d_v, const int32_t *d_slots, int32_t n, void *stream) {
  if (n < 0) return set_error(MKV_ERR_INVALID_ARGUMENT, "num_tokens < 0");
  if (n == 0) return MKV_OK;
  if (!d_k || !d_v || !d_slots) return set_error(MKV_ERR_INVALID_ARGUMENT, "NULL device pointer");
  if (!aligned16(d_k) || !aligned16(d_v))
    return set_error(MKV_ERR_INVALID_ARGUMENT, "K/V source must be 16-byte aligned");
  DeviceGuard guard(p->device);
  const int64_t cpr = p->g.row_bytes >> 4;
  hipStream_t hs = reinterpret_cast<hipStream_t>(stream);
  // Launches of at most 2^30 chunks, so 32-bit chunk indices never overflow.
  const int64_t tok_per_launch = std::max<int64_t>(1, ((int64_t)1 << 30) / (2 * cpr));
  for (int64_t t0 = 0; t0 < n; t0 += tok_per_launch) {
    const int64_t nt = std::min<int64_t>(tok_per_launch, n - t0);
    const int64_t total = nt * 2 * cpr;
    // Chunks per thread: 1 while that leaves under 8 workgroups per CU of
    // 256 (2,048 in all), then up to 8.
    const int64_t chunks = total * nlayers;
    const int per = chunks <= (int64_t)256 * 2048 * 2 ? 1 : chunks <= (int64_t)256 * 2048 * 8 ? 2
                    : chunks <= (int64_t)256 * 2048 * 32 ? 4 : 8;
    const int64_t per_wg = 256 * per;
    const int64_t wgs = std::min<int64_t>((total + per_wg - 1) / per_wg, 65535);
    const int64_t off = t0 * p->g.row_bytes;
    const uint8_t *kk = reinterpret_cast<const uint8_t *>(d_k) + off, *vv = reinterpret_cast<const uint8_t *>(d_v) + off;
    const dim3 grid((unsigned)wgs, (unsigned)nlayers);
#define MKV_APPEND(PP)                                                                                        \
  hipLaunchKernelGGL(append_kernel<PP>, grid, dim3(256), 0, hs, p->data, layer0, kk, vv, d_slots + t0,        \
                     (uint32_t)total, (uint32_t)cpr, (int64_t)n * p->g.row_bytes, p->g, p->d_err)
    switch (per) {
      case 1: MKV_APPEND(1); break;
      case 2: MKV_APPEND(2); break;
      case 4: MKV_APPEND(4); break;
      default: MKV_APPEND(8); break;
    }
#undef MKV_APPEND
    MKV_CHECK_LAUNCH("append_kernel");
  }
  return MKV_OK;
}

extern "C" int mkv_append(mkv_pool *pool, int32_t layer, const void *d_k, const void *d_v,
                          const int32_t *d_slot_mapping, int32_t num_tokens, void *stream) {
  if (!pool) return set_error(MKV_ERR_INVALID_ARGUMENT, "pool is NULL");
  Pool *p = reinterpret_cast<Pool *>(pool);
  int rc = check_layer(p, layer);
  if (rc) return rc;
  return launch_append(p, layer, 1, d_k, d_v, d_slot_mapping, num_tokens, stream);
}

extern "C" int mkv_append_all_layers(mkv_pool *pool, const void *d_k, const void *d_v,
                                     const int32_t *d_slot_mapping, int32_t num_tokens,
                                     void *stream) {
  if (!pool) return set_error(MKV_ERR_INVALID_ARGUMENT, "pool is NULL");
  Pool *p = reinterpret_cast<Pool *>(pool);
  return launch_append(p, 0, p->g.L, d_k, d_v, d_slot_mapping, num_tokens, stream);
}

extern "C" int mkv_gather(mkv_pool *pool, int32_t layer, const int32_t *d_block_indptr,
                          const int32_t *d_block_ids, const int32_t *d_ctx_indptr,
                          int32_t num_seqs, int32_t max_ctx_len, void *d_out_k, void *d_out_v,
                          int64_t out_capacity_tokens, void *stream) {
  if (!pool) return set_error(MKV_ERR_INVALID_ARGUMENT, "pool is NULL");
  Pool *p = reinterpret_cast<Pool *>(pool);
  int rc = check_layer(p, layer);
  if (rc) return rc;
  if (num_seqs < 0 || max_ctx_len < 0 || out_capacity_tokens < 0)
    return set_error(MKV_ERR_INVALID_ARGUMENT, "num_seqs, max_ctx_len and out_capacity_tokens must be >= 0");
  if (num_seqs == 0 || max_ctx_len == 0) return MKV_OK;
  if (num_seqs > 65535) return set_error(MKV_ERR_INVALID_ARGUMENT, "num_seqs > 65535");
  if (!d_block_indptr || !d_block_ids || !d_ctx_indptr || !d_out_k || !d_out_v)
    return set_error(MKV_ERR_INVALID_ARGUMENT, "NULL device pointer");
  if (!aligned16(d_out_k) || !aligned16(d_out_v))
    return set_error(MKV_ERR_INVALID_ARGUMENT, "gather outputs must be 16-byte aligned");
  DeviceGuard guard(p->device);
  const int nblk = (max_ctx_len + kPageSize - 1) / kPageSize;
  hipLaunchKernelGGL(gather_kernel, dim3(nblk, num_seqs), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), p->data, layer, d_block_indptr,
                     d_block_ids, d_ctx_indptr, max_ctx_len,
                     reinterpret_cast<uint8_t *>(d_out_k), reinterpret_cast<uint8_t *>(d_out_v),
                     (int64_t)out_capacity_tokens, p->g, p->d_err);
  MKV_CHECK_LAUNCH("gather_kernel");
  return MKV_OK;
}

extern "C" int mkv_copy_blocks(mkv_pool *pool, const int32_t *d_src_blocks,
                               const int32_t *d_dst_blocks, int32_t num_pairs, void *stream) {
  if (!pool) return set_error(MKV_ERR_INVALID_ARGUMENT, "pool is NULL");
  Pool *p = reinterpret_cast<Pool *>(pool);
  if (num_pairs < 0) return set_error(MKV_ERR_INVALID_ARGUMENT, "num_pairs < 0");
  if (num_pairs == 0) return MKV_OK;
  if (!d_src_blocks || !d_dst_blocks)
    return set_error(MKV_ERR_INVALID_ARGUMENT, "NULL device pointer");
  if (2 * p->g.L > 65535) return set_error(MKV_ERR_INVALID_ARGUMENT, "too many layers");
  DeviceGuard guard(p->device);
  hipLaunchKernelGGL(copy_blocks_kernel, dim3(num_pairs, (2 * p->g.L + kCopyPlanes - 1) / kCopyPlanes), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), p->data, d_src_blocks, d_dst_blocks,
                     p->g, p->d_err);
  MKV_CHECK_LAUNCH("copy_blocks_kernel");
  return MKV_OK;
}

// ---- C ABI: host metadata (the engine's u32 form) --------------------------------------

int mkv::stage_cached(Pool *p, StagedCache &c, const int32_t *h, size_t n, hipStream_t hs, MetaSlot **out) {
  if (c.slot >= 0 && c.stream == hs && c.vals.size() == n) {
    MetaSlot *sl = &p->meta[c.slot];
    if (sl->gen == c.gen && std::memcmp(c.vals.data(), h, n * 4) == 0) {
      *out = sl;
      return MKV_OK;
    }
  }
  c.slot = -1;
  const int idx = p->meta_next;  // the slot meta_acquire hands out
  MetaSlot *sl = nullptr;
  int rc = meta_acquire(p, n, hs, &sl);
  if (rc) return rc;
  std::memcpy(sl->h, h, n * 4);
  if ((rc = meta_upload(sl, n, hs))) return rc;
  c.slot = idx;
  c.gen = sl->gen;
  c.stream = hs;
  c.vals.assign(h, h + n);
  *out = sl;
  return MKV_OK;
}

// Stages a host slot mapping for the append entry points. Every layer of an
// engine step appends the same tokens, so the mapping is uploaded once per
// step (stage_cached).
static int stage_append_slots(Pool *p, const uint32_t *h, int32_t n, hipStream_t hs, MetaSlot **out) {
  return stage_cached(p, p->app_cache, reinterpret_cast<const int32_t *>(h), (size_t)n, hs, out);
}

extern "C" int mkv_append_host(mkv_pool *pool, int32_t layer, const void *d_k, const void *d_v,
                               const uint32_t *h_slot_mapping, int32_t num_tokens, void *stream) {
  if (!pool) return set_error(MKV_ERR_INVALID_ARGUMENT, "pool is NULL");
  Pool *p = reinterpret_cast<Pool *>(pool);
  int rc = check_layer(p, layer);
  if (rc) return rc;
  if ((rc = check_host_slots(p->g, h_slot_mapping, num_tokens))) return rc;
  if (num_tokens == 0) return MKV_OK;
  if (!d_k || !d_v) return set_error(MKV_ERR_INVALID_ARGUMENT, "NULL device pointer");
  DeviceGuard guard(p->device);
  hipStream_t hs = reinterpret_cast<hipStream_t>(stream);
  MetaSlot *sl = nullptr;
  if ((rc = stage_append_slots(p, h_slot_mapping, num_tokens, hs, &sl))) return rc;
  rc = launch_append(p, layer, 1, d_k, d_v, sl->d, num_tokens, stream);
  const int rr = meta_release(sl, hs);
  return rc ? rc : rr;
}

extern "C" int mkv_append_all_layers_host(mkv_pool *pool, const void *d_k, const void *d_v,
                                          const uint32_t *h_slot_mapping, int32_t num_tokens, void *stream) {
  if (!pool) return set_error(MKV_ERR_INVALID_ARGUMENT, "pool is NULL");
  Pool *p = reinterpret_cast<Pool *>(pool);
  int rc = check_host_slots(p->g, h_slot_mapping, num_tokens);
  if (rc) return rc;
  if (num_tokens == 0) return MKV_OK;
  if (!d_k || !d_v) return set_error(MKV_ERR_INVALID_ARGUMENT, "NULL device pointer");
  DeviceGuard guard(p->device);
  hipStream_t hs = reinterpret_cast<hipStream_t>(stream);
  MetaSlot *sl = nullptr;
  if ((rc = stage_append_slots(p, h_slot_mapping, num_tokens, hs, &sl))) return rc;
  rc = launch_append(p, 0, p->g.L, d_k, d_v, sl->d, num_tokens, stream);
  const int rr = meta_release(sl, hs);
  return rc ? rc : rr;
}

extern "C" int mkv_gather_host(mkv_pool *pool, int32_t layer, const uint32_t *h_block_indptr,
                               const uint32_t *h_block_ids, const int32_t *h_ctx_lens, int32_t num_seqs,
                               void *d_out_k, void *d_out_v, int64_t out_capacity_tokens, void *stream) {
  if (!pool) return set_error(MKV_ERR_INVALID_ARGUMENT, "pool is NULL");
  Pool *p = reinterpret_cast<Pool *>(pool);
  int rc = check_layer(p, layer);
  if (rc) return rc;
  if (num_seqs < 0 || out_capacity_tokens < 0)
    return set_error(MKV_ERR_INVALID_ARGUMENT, "num_seqs and out_capacity_tokens must be >= 0");
  if (num_seqs == 0) return MKV_OK;
  if (num_seqs > 65535) return set_error(MKV_ERR_INVALID_ARGUMENT, "num_seqs > 65535");
  int32_t max_ctx = 0;
  if ((rc = check_host_tables(p->g, h_block_indptr, h_block_ids, h_ctx_lens, num_seqs, &max_ctx))) return rc;
  int64_t tokens = 0;
  for (int32_t b = 0; b < num_seqs; b++) tokens += h_ctx_lens[b];
  if (tokens > out_capacity_tokens)
    return set_error(MKV_ERR_INVALID_ARGUMENT, "outputs hold %lld tokens, the tables give %lld",
                     (long long)out_capacity_tokens, (long long)tokens);
  if (tokens > INT32_MAX) return set_error(MKV_ERR_INVALID_ARGUMENT, "more than 2^31 - 1 tokens");
  const size_t nids = h_block_indptr[num_seqs];
  const size_t n = 2 * ((size_t)num_seqs + 1) + nids;  // indptr | ctx_indptr | ids
  DeviceGuard guard(p->device);
  hipStream_t hs = reinterpret_cast<hipStream_t>(stream);
  // Every layer of a step gathers the same tables: uploaded once per step.
  std::vector<int32_t> &st = p->stage_tmp;
  st.resize(n);
  int32_t *ip = st.data(), *cp = ip + num_seqs + 1, *ix = cp + num_seqs + 1;
  cp[0] = 0;
  for (int32_t b = 0; b <= num_seqs; b++) ip[b] = (int32_t)h_block_indptr[b];
  for (int32_t b = 0; b < num_seqs; b++) cp[b + 1] = cp[b] + h_ctx_lens[b];
  if (nids) std::memcpy(ix, h_block_ids, nids * 4);
  MetaSlot *sl = nullptr;
  if ((rc = stage_cached(p, p->gather_cache, st.data(), n, hs, &sl))) return rc;
  rc = mkv_gather(pool, layer, sl->d, sl->d + 2 * (num_seqs + 1), sl->d + num_seqs + 1, num_seqs, max_ctx,
                  d_out_k, d_out_v, out_capacity_tokens, stream);
  const int rr = meta_release(sl, hs);
  return rc ? rc : rr;
}

extern "C" int mkv_copy_blocks_host(mkv_pool *pool, const uint32_t *h_src_blocks, const uint32_t *h_dst_blocks,
                                    int32_t num_pairs, void *stream) {
  if (!pool) return set_error(MKV_ERR_INVALID_ARGUMENT, "pool is NULL");
  Pool *p = reinterpret_cast<Pool *>(pool);
  if (num_pairs < 0) return set_error(MKV_ERR_INVALID_ARGUMENT, "num_pairs < 0");
  if (num_pairs == 0) return MKV_OK;
  if (!h_src_blocks || !h_dst_blocks) return set_error(MKV_ERR_INVALID_ARGUMENT, "NULL block arrays");
  for (int32_t i = 0; i < num_pairs; i++)
    if (h_src_blocks[i] >= (uint64_t)p->g.nblocks || h_dst_blocks[i] >= (uint64_t)p->g.nblocks)
      return set_error(MKV_ERR_INVALID_ARGUMENT, "pair %d (%u -> %u) outside the pool of %lld blocks", i,
                       h_src_blocks[i], h_dst_blocks[i], (long long)p->g.nblocks);
  DeviceGuard guard(p->device);
  hipStream_t hs = reinterpret_cast<hipStream_t>(stream);
  MetaSlot *sl = nullptr;
  int rc = meta_acquire(p, 2 * (size_t)num_pairs, hs, &sl);
  if (rc) return rc;
  std::memcpy(sl->h, h_src_blocks, (size_t)num_pairs * 4);
  std::memcpy(sl->h + num_pairs, h_dst_blocks, (size_t)num_pairs * 4);
  // Distinct destinations, no block both a source and a destination: the
  // copies of one launch then do not depend on each other's order.
  if ((rc = mkv_validate_copy_pairs(&p->desc, sl->h, sl->h + num_pairs, num_pairs))) return rc;
  if ((rc = meta_upload(sl, 2 * (size_t)num_pairs, hs))) return rc;
  rc = mkv_copy_blocks(pool, sl->d, sl->d + num_pairs, num_pairs, stream);
  const int rr = meta_release(sl, hs);
  return rc ? rc : rr;
}

// ---- C ABI: host validation ------------------------------------------------------------

extern "C" int mkv_validate_slots(const mkv_pool_desc *desc, const int32_t *slots, int32_t n) {
  int rc = validate_desc(desc);
  if (rc) return rc;
  if (n < 0 || (n > 0 && !slots)) return set_error(MKV_ERR_INVALID_ARGUMENT, "bad slot array");
  const int64_t nslots = desc->num_blocks * desc->page_size;
  for (int32_t i = 0; i < n; i++)
    if (slots[i] < 0 || slots[i] >= nslots)
      return set_error(MKV_ERR_INVALID_ARGUMENT, "slot[%d] = %d outside [0, %lld)", i, slots[i],
                       (long long)nslots);
  return MKV_OK;
}

extern "C" int mkv_validate_block_tables(const mkv_pool_desc *desc, const int32_t *indptr,
                                         const int32_t *ids, const int32_t *ctx_lens,
                                         int32_t num_seqs, int32_t max_ctx_len) {
  int rc = validate_desc(desc);
  if (rc) return rc;
  if (num_seqs < 0 || !indptr) return set_error(MKV_ERR_INVALID_ARGUMENT, "bad indptr");
  if (indptr[0] < 0) return set_error(MKV_ERR_INVALID_ARGUMENT, "indptr[0] < 0");
  // The whole array first: ids holds indptr[num_seqs] entries.
  for (int32_t b = 0; b < num_seqs; b++)
    if (indptr[b + 1] < indptr[b])
      return set_error(MKV_ERR_INVALID_ARGUMENT, "indptr not monotone at %d", b);
  for (int32_t b = 0; b < num_seqs; b++) {
    for (int32_t i = indptr[b]; i < indptr[b + 1]; i++)
      if (!ids || ids[i] < 0 || ids[i] >= desc->num_blocks)
        return set_error(MKV_ERR_INVALID_ARGUMENT, "block id at %d (sequence %d) out of range", i, b);
    if (ctx_lens) {
      const int32_t n = ctx_lens[b];
      if (n < 1 || n > max_ctx_len)
        return set_error(MKV_ERR_INVALID_ARGUMENT, "ctx_len[%d] = %d outside [1, %d]", b, n,
                         max_ctx_len);
      if ((int64_t)(n + desc->page_size - 1) / desc->page_size > indptr[b + 1] - indptr[b])
        return set_error(MKV_ERR_INVALID_ARGUMENT,
                         "sequence %d: %d blocks cannot hold %d tokens", b,
                         indptr[b + 1] - indptr[b], n);
    }
  }
  return MKV_OK;
}

extern "C" int mkv_validate_copy_pairs(const mkv_pool_desc *desc, const int32_t *src,
                                       const int32_t *dst, int32_t n) {
  int rc = validate_desc(desc);
  if (rc) return rc;
  if (n < 0 || (n > 0 && (!src || !dst))) return set_error(MKV_ERR_INVALID_ARGUMENT, "bad pairs");
  std::vector<uint8_t> role((size_t)desc->num_blocks, 0);  // bit0 = source, bit1 = destination
  for (int32_t i = 0; i < n; i++) {
    if (src[i] < 0 || src[i] >= desc->num_blocks || dst[i] < 0 || dst[i] >= desc->num_blocks)
      return set_error(MKV_ERR_INVALID_ARGUMENT, "pair %d (%d -> %d) out of range", i, src[i], dst[i]);
    if (role[dst[i]] & 2) return set_error(MKV_ERR_INVALID_ARGUMENT, "destination %d repeats", dst[i]);
    role[src[i]] |= 1;
    role[dst[i]] |= 2;
  }
  for (int32_t i = 0; i < n; i++)
    if (role[src[i]] == 3 || role[dst[i]] == 3)
      return set_error(MKV_ERR_INVALID_ARGUMENT, "block %d is both a source and a destination",
                       role[src[i]] == 3 ? src[i] : dst[i]);
  return MKV_OK;
}

// ---- C ABI: device buffers ------------------------------------------------------------

extern "C" int mkv_buffer_alloc(int device, uint64_t bytes, void **out_dev_ptr) {
  if (!out_dev_ptr) return set_error(MKV_ERR_INVALID_ARGUMENT, "out pointer is NULL");
  *out_dev_ptr = nullptr;
  int ndev = 0;
  if (hipGetDeviceCount(&ndev) != hipSuccess || ndev == 0) {
    (void)hipGetLastError();
    return set_error(MKV_ERR_NO_DEVICE, "no HIP device available");
  }
  if (device < 0 || device >= ndev)
    return set_error(MKV_ERR_INVALID_ARGUMENT, "device %d out of range (%d devices)", device, ndev);
  DeviceGuard guard(device);
  if (!guard.ok) return set_error(MKV_ERR_NO_DEVICE, "cannot select device %d", device);
  MKV_CHECK_HIP(hipMalloc(out_dev_ptr, bytes ? bytes : 1));
  return MKV_OK;
}

extern "C" int mkv_buffer_free(void *dev_ptr) {
  if (dev_ptr) MKV_CHECK_HIP(hipFree(dev_ptr));
  return MKV_OK;
}

extern "C" int mkv_memcpy_h2d(void *d_dst, const void *h_src, uint64_t bytes, void *stream) {
  if (!bytes) return MKV_OK;
  if (!d_dst || !h_src) return set_error(MKV_ERR_INVALID_ARGUMENT, "NULL pointer");
  MKV_CHECK_HIP(hipMemcpyAsync(d_dst, h_src, bytes, hipMemcpyHostToDevice,
                               reinterpret_cast<hipStream_t>(stream)));
  return MKV_OK;
}

extern "C" int mkv_memcpy_d2h(void *h_dst, const void *d_src, uint64_t bytes, void *stream) {
  if (!bytes) return MKV_OK;
  if (!h_dst || !d_src) return set_error(MKV_ERR_INVALID_ARGUMENT, "NULL pointer");
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  MKV_CHECK_HIP(hipMemcpyAsync(h_dst, d_src, bytes, hipMemcpyDeviceToHost, s));
  MKV_CHECK_HIP(hipStreamSynchronize(s));
  return MKV_OK;
}

extern "C" int mkv_stream_synchronize(void *stream) {
  MKV_CHECK_HIP(hipStreamSynchronize(reinterpret_cast<hipStream_t>(stream)));
  return MKV_OK;
}

extern "C" const char *mkv_last_error(void) { return g_last_error.c_str(); }

extern "C" int mkv_version(void) { return 100; }
