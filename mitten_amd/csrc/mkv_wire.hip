// Wire / disk form of KV blocks: export a list of pool blocks (a range of
// layers, K and V) into one contiguous payload with a checksum per block,
// and import such a payload into other blocks of a pool, verifying it.
//
// The reference moves KV between workers only as page indices into one pool
// (KvHandoff, design/phase2b-deliverable.md:272-289) and sketches per-layer
// KV files streamed from SSD (KvOffloadManager, design/phase1-deliverable.md:
// 253-339); it defines no byte format. This file defines one:
//   payload = [n][num_layers][2 (K, V)][page_size][num_kv_heads][head_dim],
// block-major, so each block's state is contiguous (a page is the unit of
// handoff) and, with num_layers = 1, one layer's blocks form the per-layer
// offload chunk. The checksum of a block's payload, seen as little-endian
// u64 words w_0 .. w_{m-1}, is
//   sum64 = sum_j mix(w_j + (j + 1) * 0x9E3779B97F4A7C15)  (mod 2^64),
// mix being the splitmix64 output function. A sum is order-free, so
// workgroups add their parts with atomics and the result is deterministic;
// mix is a bijection, so any single-word change alters the sum, and the
// index term makes it position-sensitive.
#include <cstring>
#include <vector>

#include "mkv_internal.h"

namespace mkv {

typedef uint32_t w32x4 __attribute__((ext_vector_type(4)));

constexpr uint64_t kWireGolden = 0x9E3779B97F4A7C15ull;
constexpr int kWireUnroll = 8;  // 16-byte chunks per thread: 32 KiB per workgroup

__device__ __forceinline__ uint64_t wire_mix(uint64_t w, uint64_t j) {
  uint64_t z = w + (j + 1) * kWireGolden;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

struct WireArgs {
  uint8_t *pool;
  const int32_t *ids;
  uint8_t *payload;
  unsigned long long *sums;
  uint32_t *d_err;
  int64_t nblocks, plane_bytes, block_bytes;
  uint32_t chunks;        // 16-byte chunks of one block's payload: nl * 2 * block_bytes / 16
  uint32_t plane_chunks;  // block_bytes / 16
  int32_t layer0;
};

// grid.x: 32 KiB slices of one block's payload; grid.y: position in the id
// list. EXPORT copies pool -> payload, else payload -> pool; the sum is over
// the bytes copied (the pool's on export, the received payload's on import).
template <bool EXPORT>
__global__ void __launch_bounds__(256) wire_kernel(WireArgs a) {
  const int i = blockIdx.y, tid = threadIdx.x;
  const int32_t b = a.ids[i];
  if (b < 0 || b >= a.nblocks) {
    if (blockIdx.x == 0 && tid == 0) record_error(a.d_err, MKV_DEVERR_BLOCK);
    return;
  }
  const uint32_t c0 = blockIdx.x * (256u * kWireUnroll) + tid;
  w32x4 *pay = reinterpret_cast<w32x4 *>(a.payload + (int64_t)i * a.chunks * 16);
  int64_t poff[kWireUnroll];
  w32x4 r[kWireUnroll];
#pragma unroll
  for (int u = 0; u < kWireUnroll; u++) {  // all loads first; nontemporal: the data is not reused
    const uint32_t c = min(c0 + u * 256u, a.chunks - 1);  // lanes past the end reload the last chunk
    const uint32_t p = c / a.plane_chunks, o = c - p * a.plane_chunks;
    poff[u] = (int64_t)(a.layer0 * 2 + (int)p) * a.plane_bytes + (int64_t)b * a.block_bytes + (int64_t)o * 16;
    r[u] = EXPORT ? __builtin_nontemporal_load(reinterpret_cast<const w32x4 *>(a.pool + poff[u])) : __builtin_nontemporal_load(&pay[c]);
  }
  unsigned long long acc = 0;
#pragma unroll
  for (int u = 0; u < kWireUnroll; u++) {
    const uint32_t c = c0 + u * 256u;
    if (c < a.chunks) {
      if (EXPORT) __builtin_nontemporal_store(r[u], &pay[c]);
      else __builtin_nontemporal_store(r[u], reinterpret_cast<w32x4 *>(a.pool + poff[u]));
      const uint64_t lo = ((uint64_t)r[u][1] << 32) | r[u][0], hi = ((uint64_t)r[u][3] << 32) | r[u][2];
      acc += wire_mix(lo, 2ull * c) + wire_mix(hi, 2ull * c + 1);
    }
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) acc += __shfl_xor(acc, o);
  if ((tid & 63) == 0) atomicAdd(&a.sums[i], acc);
}

__global__ void __launch_bounds__(256) wire_zero_kernel(unsigned long long *sums, int32_t n) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i < n) sums[i] = 0;
}

__global__ void __launch_bounds__(256) wire_compare_kernel(const unsigned long long *got,
                                                           const unsigned long long *expected, int32_t n,
                                                           uint32_t *d_err) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i < n && got[i] != expected[i]) record_error(d_err, MKV_DEVERR_CHECKSUM);
}

}  // namespace mkv

using namespace mkv;

namespace {

int wire_args(mkv_pool *pool, const int32_t *d_block_ids, int32_t num_blocks, int32_t layer_begin,
              int32_t num_layers, void *d_payload, uint64_t *d_checksums, WireArgs *a) {
  if (!pool) return set_error(MKV_ERR_INVALID_ARGUMENT, "NULL pool");
  Pool *p = reinterpret_cast<Pool *>(pool);
  const Geom &g = p->g;
  if (num_blocks < 0) return set_error(MKV_ERR_INVALID_ARGUMENT, "num_blocks < 0");
  if (layer_begin < 0 || num_layers < 1 || layer_begin > g.L - num_layers)
    return set_error(MKV_ERR_INVALID_ARGUMENT, "layers [%d, %d) outside the pool's %d", layer_begin,
                     layer_begin + num_layers, g.L);
  if (num_blocks > 0 && (!d_block_ids || !d_payload || !d_checksums))
    return set_error(MKV_ERR_INVALID_ARGUMENT, "NULL device pointer");
  if (!aligned16(d_payload) || (reinterpret_cast<uintptr_t>(d_checksums) & 7u))
    return set_error(MKV_ERR_INVALID_ARGUMENT, "payload must be 16-byte and checksums 8-byte aligned");
  const uint64_t chunks = (uint64_t)num_layers * 2 * (uint64_t)g.block_bytes / 16;
  if (chunks > (uint64_t)INT32_MAX)
    return set_error(MKV_ERR_INVALID_ARGUMENT, "a block's payload exceeds 32 GiB");
  if (num_blocks > 65535) return set_error(MKV_ERR_INVALID_ARGUMENT, "at most 65535 blocks per call");
  a->pool = p->data;
  a->ids = d_block_ids;
  a->payload = static_cast<uint8_t *>(d_payload);
  a->sums = reinterpret_cast<unsigned long long *>(d_checksums);
  a->d_err = p->d_err;
  a->nblocks = g.nblocks;
  a->plane_bytes = g.plane_bytes;
  a->block_bytes = g.block_bytes;
  a->chunks = (uint32_t)chunks;
  a->plane_chunks = (uint32_t)(g.block_bytes / 16);
  a->layer0 = layer_begin;
  return MKV_OK;
}

template <bool EXPORT>
int wire_launch(mkv_pool *pool, const WireArgs &a, int32_t n, void *stream) {
  Pool *p = reinterpret_cast<Pool *>(pool);
  DeviceGuard guard(p->device);
  hipStream_t hs = reinterpret_cast<hipStream_t>(stream);
  // Sums start at zero through a kernel (no memset node if the caller
  // captures the stream into a graph).
  hipLaunchKernelGGL(wire_zero_kernel, dim3((n + 255) / 256), dim3(256), 0, hs, a.sums, n);
  MKV_CHECK_LAUNCH("wire_zero_kernel");
  const unsigned slices = (a.chunks + 256u * kWireUnroll - 1) / (256u * kWireUnroll);
  hipLaunchKernelGGL(wire_kernel<EXPORT>, dim3(slices, n), dim3(256), 0, hs, a);
  MKV_CHECK_LAUNCH("wire_kernel");
  return MKV_OK;
}

}  // namespace

extern "C" int mkv_wire_export(mkv_pool *pool, const int32_t *d_block_ids, int32_t num_blocks,
                               int32_t layer_begin, int32_t num_layers, void *d_payload, uint64_t *d_checksums,
                               void *stream) {
  WireArgs a;
  const int st = wire_args(pool, d_block_ids, num_blocks, layer_begin, num_layers, d_payload, d_checksums, &a);
  if (st != MKV_OK || num_blocks == 0) return st;
  return wire_launch<true>(pool, a, num_blocks, stream);
}

extern "C" int mkv_wire_import(mkv_pool *pool, const int32_t *d_block_ids, int32_t num_blocks,
                               int32_t layer_begin, int32_t num_layers, const void *d_payload,
                               const uint64_t *d_expected, uint64_t *d_checksums, void *stream) {
  WireArgs a;
  const int st = wire_args(pool, d_block_ids, num_blocks, layer_begin, num_layers, const_cast<void *>(d_payload),
                           d_checksums, &a);
  if (st != MKV_OK || num_blocks == 0) return st;
  const int st2 = wire_launch<false>(pool, a, num_blocks, stream);
  if (st2 != MKV_OK || !d_expected) return st2;
  Pool *p = reinterpret_cast<Pool *>(pool);
  DeviceGuard guard(p->device);
  hipLaunchKernelGGL(wire_compare_kernel, dim3((num_blocks + 255) / 256), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), a.sums,
                     reinterpret_cast<const unsigned long long *>(d_expected), num_blocks, p->d_err);
  MKV_CHECK_LAUNCH("wire_compare_kernel");
  return MKV_OK;
}

// ---- host block ids (the engine's u32 pages) ----------------------------------

static int stage_wire_ids(Pool *p, const uint32_t *h_ids, int32_t n, bool distinct, hipStream_t hs, MetaSlot **out) {
  if (n < 0) return set_error(MKV_ERR_INVALID_ARGUMENT, "num_blocks < 0");
  if (n > 0 && !h_ids) return set_error(MKV_ERR_INVALID_ARGUMENT, "NULL block ids");
  std::vector<uint8_t> seen(distinct ? (size_t)p->g.nblocks : 0, 0);
  for (int32_t i = 0; i < n; i++) {
    if (h_ids[i] >= (uint64_t)p->g.nblocks)
      return set_error(MKV_ERR_INVALID_ARGUMENT, "block id %u (entry %d) outside the pool of %lld", h_ids[i], i,
                       (long long)p->g.nblocks);
    if (distinct) {
      if (seen[h_ids[i]]) return set_error(MKV_ERR_INVALID_ARGUMENT, "destination block %u repeats", h_ids[i]);
      seen[h_ids[i]] = 1;
    }
  }
  int rc = meta_acquire(p, n, hs, out);
  if (rc) return rc;
  if (n) std::memcpy((*out)->h, h_ids, (size_t)n * 4);
  return meta_upload(*out, n, hs);
}

extern "C" int mkv_wire_export_host(mkv_pool *pool, const uint32_t *h_block_ids, int32_t num_blocks,
                                    int32_t layer_begin, int32_t num_layers, void *d_payload, uint64_t *d_checksums,
                                    void *stream) {
  if (!pool) return set_error(MKV_ERR_INVALID_ARGUMENT, "pool is NULL");
  Pool *p = reinterpret_cast<Pool *>(pool);
  if (num_blocks == 0) return MKV_OK;
  DeviceGuard guard(p->device);
  hipStream_t hs = reinterpret_cast<hipStream_t>(stream);
  MetaSlot *sl = nullptr;
  int rc = stage_wire_ids(p, h_block_ids, num_blocks, false, hs, &sl);
  if (rc) return rc;
  rc = mkv_wire_export(pool, sl->d, num_blocks, layer_begin, num_layers, d_payload, d_checksums, stream);
  const int rr = meta_release(sl, hs);
  return rc ? rc : rr;
}

extern "C" int mkv_wire_import_host(mkv_pool *pool, const uint32_t *h_block_ids, int32_t num_blocks,
                                    int32_t layer_begin, int32_t num_layers, const void *d_payload,
                                    const uint64_t *d_expected, uint64_t *d_checksums, void *stream) {
  if (!pool) return set_error(MKV_ERR_INVALID_ARGUMENT, "pool is NULL");
  Pool *p = reinterpret_cast<Pool *>(pool);
  if (num_blocks == 0) return MKV_OK;
  DeviceGuard guard(p->device);
  hipStream_t hs = reinterpret_cast<hipStream_t>(stream);
  MetaSlot *sl = nullptr;
  int rc = stage_wire_ids(p, h_block_ids, num_blocks, true, hs, &sl);
  if (rc) return rc;
  rc = mkv_wire_import(pool, sl->d, num_blocks, layer_begin, num_layers, d_payload, d_expected, d_checksums, stream);
  const int rr = meta_release(sl, hs);
  return rc ? rc : rr;
}

// ---- header (host only) -------------------------------------------------------

extern "C" int mkv_wire_header_init(const mkv_pool_desc *desc, int32_t layer_begin, int32_t num_layers,
                                    int32_t num_blocks, int64_t cached_len, mkv_wire_header *out) {
  if (!desc || !out) return set_error(MKV_ERR_INVALID_ARGUMENT, "NULL argument");
  if (layer_begin < 0 || num_layers < 1 || layer_begin > desc->num_layers - num_layers)
    return set_error(MKV_ERR_INVALID_ARGUMENT, "layers [%d, %d) outside the pool's %d", layer_begin,
                     layer_begin + num_layers, desc->num_layers);
  if (num_blocks < 0 || cached_len < 0 || cached_len > (int64_t)num_blocks * desc->page_size)
    return set_error(MKV_ERR_INVALID_ARGUMENT, "cached_len %lld does not fit %d blocks",
                     (long long)cached_len, num_blocks);
  if (desc->dtype != MKV_DTYPE_F32 && desc->dtype != MKV_DTYPE_BF16)
    return set_error(MKV_ERR_INVALID_ARGUMENT, "unknown dtype %d", desc->dtype);
  std::memset(out, 0, sizeof(*out));
  out->magic = MKV_WIRE_MAGIC;
  out->version = MKV_WIRE_VERSION;
  out->dtype = (uint16_t)desc->dtype;
  out->page_size = desc->page_size;
  out->num_kv_heads = desc->num_kv_heads;
  out->head_dim = desc->head_dim;
  out->layer_begin = layer_begin;
  out->num_layers = num_layers;
  out->num_blocks = num_blocks;
  out->cached_len = cached_len;
  const uint64_t es = desc->dtype == MKV_DTYPE_F32 ? 4 : 2;
  out->block_bytes = (uint64_t)num_layers * 2 * desc->page_size * desc->num_kv_heads * desc->head_dim * es;
  out->payload_offset = (sizeof(mkv_wire_header) + 8ull * num_blocks + 4095) / 4096 * 4096;
  return MKV_OK;
}

extern "C" int mkv_wire_header_check(const mkv_pool_desc *desc, const mkv_wire_header *h) {
  if (!desc || !h) return set_error(MKV_ERR_INVALID_ARGUMENT, "NULL argument");
  if (h->magic != MKV_WIRE_MAGIC) return set_error(MKV_ERR_INVALID_ARGUMENT, "not a KV block payload (magic)");
  if (h->version != MKV_WIRE_VERSION)
    return set_error(MKV_ERR_INVALID_ARGUMENT, "wire version %u, this library reads %u", h->version,
                     MKV_WIRE_VERSION);
  mkv_wire_header want;
  if (mkv_wire_header_init(desc, h->layer_begin, h->num_layers, h->num_blocks, h->cached_len, &want) != MKV_OK)
    return MKV_ERR_INVALID_ARGUMENT;
  if (h->dtype != want.dtype || h->page_size != want.page_size || h->num_kv_heads != want.num_kv_heads ||
      h->head_dim != want.head_dim || h->block_bytes != want.block_bytes ||
      h->payload_offset != want.payload_offset)
    return set_error(MKV_ERR_INVALID_ARGUMENT,
                     "payload geometry (dtype %u, page %d, %d heads x %d) does not match the pool", h->dtype,
                     h->page_size, h->num_kv_heads, h->head_dim);
  return MKV_OK;
}
