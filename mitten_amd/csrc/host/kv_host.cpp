// Host-side paged-KV bookkeeping: page allocator, page table, radix prefix
// cache (with the reference engine's semantics) and the block manager that
// drives the device pool. Plain C++17; no device code.
//
//   KvPool      inference-engine/src/kv_pool.rs:4-69
//   PageTable   inference-engine/src/kv_pool.rs:71-102
//   Radix       inference-engine/src/radix_cache.rs:37-303
//   BlockMgr    the engine's page lifecycle (prefill.rs:39-81, decode.rs:6-47,
//               scheduler.rs:117,164-172) with reference counts, decode-time
//               growth, copy-on-write and compaction added
#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <map>
#include <new>
#include <queue>
#include <string>
#include <unordered_map>
#include <unordered_set>
#include <vector>

#include "mitten_kv_host.h"

namespace mkvh {

static thread_local std::string g_err;

static int fail(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
static int fail(int code, const char *fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

// ---------------------------------------------------------------------------
// KvCachePool: LIFO free stack; new() pushes 0..n reversed so pages come out
// 0, 1, 2, ... (kv_pool.rs:18-27). Each page carries an owner tag and, for the
// block manager, a reference count.
// ---------------------------------------------------------------------------
struct KvPool {
  int64_t num_pages;
  int32_t page_size;
  std::vector<uint32_t> free_stack;  // back() is the top
  std::vector<uint8_t> in_use;
  std::vector<uint64_t> owner;
  std::vector<int32_t> refcnt;

  KvPool(int64_t n, int32_t ps) : num_pages(n), page_size(ps), in_use(n, 0), owner(n, 0), refcnt(n, 0) {
    free_stack.reserve(n);
    for (int64_t i = n - 1; i >= 0; i--) free_stack.push_back((uint32_t)i);
  }
  bool valid(uint32_t p) const { return (int64_t)p < num_pages; }
  [[nodiscard]] int allocate(uint64_t who, uint32_t *out) {
    if (free_stack.empty()) return fail(MKVH_ERR_EXHAUSTED, "KV pool exhausted (%lld pages)", (long long)num_pages);
    const uint32_t p = free_stack.back();
    free_stack.pop_back();
    in_use[p] = 1;
    owner[p] = who;
    refcnt[p] = 1;
    *out = p;
    return MKVH_OK;
  }
  int free(uint32_t p) {
    if (!valid(p)) return fail(MKVH_ERR_INVALID_ARGUMENT, "page %u out of range", p);
    if (!in_use[p]) return fail(MKVH_ERR_NOT_IN_USE, "Attempted to free a page that is not in use (%u)", p);
    in_use[p] = 0;
    refcnt[p] = 0;
    free_stack.push_back(p);
    return MKVH_OK;
  }
  [[nodiscard]] int retain(uint32_t p) {
    if (!valid(p) || !in_use[p]) return fail(MKVH_ERR_NOT_IN_USE, "retain of page %u that is not in use", p);
    refcnt[p]++;
    return MKVH_OK;
  }
  [[nodiscard]] int release(uint32_t p, bool *freed) {
    if (!valid(p) || !in_use[p]) return fail(MKVH_ERR_NOT_IN_USE, "release of page %u that is not in use", p);
    *freed = --refcnt[p] == 0;
    if (*freed) return free(p);
    return MKVH_OK;
  }
};

// ---------------------------------------------------------------------------
// PageTable: (request, slot) -> page (kv_pool.rs:71-102).
// ---------------------------------------------------------------------------
struct PageTable {
  std::map<std::pair<uint64_t, int64_t>, uint32_t> m;
};

// ---------------------------------------------------------------------------
// RadixCache (radix_cache.rs:37-303). Node ids follow the slab the reference
// uses: a removed id is the next one reused. Time is a logical clock (each
// "now" is a fresh, larger tick), which orders LRU exactly as distinct
// Instant::now() calls do. The LRU heap pops the oldest stamp first and, on
// equal stamps, the larger node id (BinaryHeap<(Reverse<Instant>, NodeId)>).
// ---------------------------------------------------------------------------
struct Node {
  std::vector<uint32_t> edge;
  std::vector<uint32_t> pages;
  std::unordered_map<uint32_t, size_t> children;
  int64_t parent = -1;
  int32_t lock_ref = 0;
  uint64_t last_used = 0;
  bool live = false;
  bool is_leaf() const { return children.empty(); }
  bool evictable() const { return is_leaf() && lock_ref == 0 && !pages.empty(); }
};

struct HeapCmp {  // std::priority_queue pops the "largest": oldest stamp, then larger id
  bool operator()(const std::pair<uint64_t, size_t> &a, const std::pair<uint64_t, size_t> &b) const {
    if (a.first != b.first) return a.first > b.first;
    return a.second < b.second;
  }
};

struct Radix {
  std::vector<Node> nodes;
  std::vector<size_t> vacant;  // slab free list, last removed reused first
  size_t live_count = 0;
  size_t root = 0;
  std::priority_queue<std::pair<uint64_t, size_t>, std::vector<std::pair<uint64_t, size_t>>, HeapCmp> heap;
  int32_t page_size;
  int64_t total_pages = 0;
  int64_t max_pages;
  uint64_t clock = 0;
  std::vector<uint32_t> evicted;  // pages evicted and not yet drained

  Radix(int32_t ps, int64_t maxp) : page_size(ps), max_pages(maxp) {
    Node r;
    r.live = true;
    r.last_used = now();
    root = insert_node(std::move(r));
  }
  uint64_t now() { return ++clock; }
  size_t insert_node(Node &&n) {
    n.live = true;
    live_count++;
    if (!vacant.empty()) {
      const size_t id = vacant.back();
      vacant.pop_back();
      nodes[id] = std::move(n);
      return id;
    }
    nodes.push_back(std::move(n));
    return nodes.size() - 1;
  }
  void remove_node(size_t id) {
    nodes[id] = Node();
    live_count--;
    vacant.push_back(id);
  }
  bool contains(size_t id) const { return id < nodes.size() && nodes[id].live; }

  static size_t common(const std::vector<uint32_t> &edge, const uint32_t *t, size_t n) {
    size_t k = 0;
    while (k < edge.size() && k < n && edge[k] == t[k]) k++;
    return k;
  }

  // match_prefix (radix_cache.rs:64-117).
  void match_prefix(const uint32_t *tokens, size_t n, size_t *matched, std::vector<uint32_t> &pages,
                    std::vector<size_t> &locked) {
    size_t offset = 0, cur = root;
    while (offset < n) {
      auto it = nodes[cur].children.find(tokens[offset]);
      if (it == nodes[cur].children.end()) break;
      const size_t child = it->second;
      Node &c = nodes[child];
      const size_t match_len = common(c.edge, tokens + offset, n - offset);
      if (match_len == 0) break;
      const size_t full_pages = match_len / page_size;
      if (full_pages == 0) break;
      const size_t take = std::min(full_pages, c.pages.size());
      pages.insert(pages.end(), c.pages.begin(), c.pages.begin() + take);
      offset += full_pages * page_size;
      const bool partial = match_len < c.edge.size();
      locked.push_back(child);
      c.lock_ref += 1;
      c.last_used = now();
      if (partial) break;
      cur = child;
    }
    *matched = offset;
  }

  // split_edge (radix_cache.rs:191-223).
  size_t split_edge(size_t parent, size_t child, size_t split_at) {
    const size_t page_split = std::min(split_at / page_size, nodes[child].pages.size());
    Node mid;
    mid.edge.assign(nodes[child].edge.begin(), nodes[child].edge.begin() + split_at);
    mid.pages.assign(nodes[child].pages.begin(), nodes[child].pages.begin() + page_split);
    std::vector<uint32_t> suffix(nodes[child].edge.begin() + split_at, nodes[child].edge.end());
    std::vector<uint32_t> suffix_pages(nodes[child].pages.begin() + page_split, nodes[child].pages.end());
    const uint32_t first_suffix = suffix[0], first_prefix = mid.edge[0];
    nodes[child].edge = std::move(suffix);
    nodes[child].pages = std::move(suffix_pages);
    mid.children[first_suffix] = child;
    mid.parent = (int64_t)parent;
    mid.last_used = now();
    const size_t mid_id = insert_node(std::move(mid));
    nodes[child].parent = (int64_t)mid_id;
    nodes[parent].children[first_prefix] = mid_id;
    return mid_id;
  }

  // evict_pages (radix_cache.rs:243-282); freed pages are appended to `out`.
  void evict_pages(size_t target, std::vector<uint32_t> &out) {
    size_t freed = 0;
    while (freed < target) {
      size_t cand = SIZE_MAX;
      while (!heap.empty()) {
        const size_t id = heap.top().second;
        heap.pop();
        if (contains(id) && nodes[id].evictable()) {
          cand = id;
          break;
        }
      }
      if (cand == SIZE_MAX) return;
      std::vector<uint32_t> pg = std::move(nodes[cand].pages);
      nodes[cand].pages.clear();
      total_pages -= (int64_t)pg.size();
      freed += pg.size();
      out.insert(out.end(), pg.begin(), pg.end());
      if (nodes[cand].parent >= 0) {
        const size_t parent = (size_t)nodes[cand].parent;
        if (!nodes[cand].edge.empty()) {
          nodes[parent].children.erase(nodes[cand].edge[0]);
          if (nodes[parent].evictable()) heap.push({nodes[parent].last_used, parent});
        }
      }
      remove_node(cand);
    }
  }

  // insert_prefix (radix_cache.rs:123-187). Pages evicted to make room go to
  // `evicted_out` (the reference discards them, radix_cache.rs:132-134); the
  // pages a new leaf adopts go to `adopted`.
  void insert_prefix(const uint32_t *tokens, const uint32_t *pages, size_t full_pages,
                     std::vector<uint32_t> &evicted_out, std::vector<uint32_t> &adopted) {
    if (full_pages == 0) return;
    const size_t len = full_pages * page_size;
    if (total_pages + (int64_t)full_pages > max_pages)
      evict_pages((size_t)(total_pages + (int64_t)full_pages - max_pages), evicted_out);
    size_t offset = 0, cur = root;
    while (offset < len) {
      const uint32_t first = tokens[offset];
      auto it = nodes[cur].children.find(first);
      if (it == nodes[cur].children.end()) {
        Node leaf;
        leaf.edge.assign(tokens + offset, tokens + len);
        const size_t p0 = std::min(offset / page_size, full_pages);
        leaf.pages.assign(pages + p0, pages + full_pages);
        leaf.parent = (int64_t)cur;
        leaf.last_used = now();
        const size_t added = leaf.pages.size();
        adopted.insert(adopted.end(), leaf.pages.begin(), leaf.pages.end());
        const size_t id = insert_node(std::move(leaf));
        nodes[cur].children[first] = id;
        total_pages += (int64_t)added;
        heap.push({now(), id});
        break;
      }
      const size_t child = it->second;
      const size_t edge_len = nodes[child].edge.size();
      const size_t match_len = common(nodes[child].edge, tokens + offset, len - offset);
      if (match_len == edge_len) {
        nodes[child].last_used = now();
        offset += edge_len;
        cur = child;
      } else {
        const size_t mid = split_edge(cur, child, match_len);
        offset += match_len;
        cur = mid;
      }
    }
  }

  // unlock_nodes (radix_cache.rs:227-238).
  void unlock_nodes(const uint64_t *ids, size_t n) {
    for (size_t i = 0; i < n; i++) {
      const size_t id = (size_t)ids[i];
      if (!contains(id)) continue;
      Node &nd = nodes[id];
      nd.lock_ref = std::max(nd.lock_ref - 1, 0);
      nd.last_used = now();
      if (nd.evictable()) heap.push({nd.last_used, id});
    }
  }
  void lock_nodes(const std::vector<size_t> &ids) {
    for (size_t id : ids)
      if (contains(id)) nodes[id].lock_ref += 1;
  }
};

// ---------------------------------------------------------------------------
// Block manager.
// ---------------------------------------------------------------------------
struct Seq {
  std::vector<uint32_t> blocks;
  int64_t len = 0;     // tokens written
  int64_t prompt = 0;  // prompt length given at admission
  std::vector<size_t> locked;
};

// Reference counts of blocks the manager's books say are in use. Every
// block is processed; a failure (the books disagree with the pool) is
// returned after the loop, with the pool's message.
static int retain_all(KvPool &pool, const std::vector<uint32_t> &blocks) {
  int rc = MKVH_OK;
  for (uint32_t b : blocks) {
    const int r = pool.retain(b);
    if (r != MKVH_OK && rc == MKVH_OK) rc = r;
  }
  return rc;
}
static int release_all(KvPool &pool, const std::vector<uint32_t> &blocks) {
  int rc = MKVH_OK;
  for (uint32_t b : blocks) {
    bool freed = false;
    const int r = pool.release(b, &freed);
    if (r != MKVH_OK && rc == MKVH_OK) rc = r;
  }
  return rc;
}

struct BlockMgr {
  KvPool pool;
  Radix radix;
  std::unordered_map<uint64_t, Seq> seqs;
  int32_t ps;
  BlockMgr(int64_t n, int32_t page, int64_t maxc) : pool(n, page), radix(page, maxc), ps(page) {}

  // Releases the tree's reference to each evicted page.
  int64_t drop_tree_pages(const std::vector<uint32_t> &pages) {
    int64_t freed = 0;
    for (uint32_t p : pages) {
      bool f = false;
      if (pool.release(p, &f) == MKVH_OK && f) freed++;
    }
    return freed;
  }
  // Frees room for `need` pages by evicting tree leaves once (prefill.rs:44-49).
  void make_room(int64_t need) {
    const int64_t free_now = (int64_t)pool.free_stack.size();
    if (free_now >= need) return;
    std::vector<uint32_t> ev;
    radix.evict_pages((size_t)(need - free_now), ev);
    drop_tree_pages(ev);
  }
};

}  // namespace mkvh

using namespace mkvh;

#define H_CHECK(p) \
  if (!(p)) return fail(MKVH_ERR_INVALID_ARGUMENT, "NULL handle")

extern "C" {

const char *mkvh_last_error(void) { return g_err.c_str(); }

uint64_t mkvh_required_bytes(uint64_t num_pages, uint64_t page_size, uint64_t num_layers,
                             uint64_t num_kv_heads, uint64_t head_dim, uint64_t dtype_bytes) {
  return 2 * num_layers * num_pages * page_size * num_kv_heads * head_dim * dtype_bytes;
}

// ---- KvCachePool ------------------------------------------------------------------

int mkvh_kv_pool_create(int64_t num_pages, int32_t page_size, mkvh_kv_pool **out) {
  if (!out || num_pages < 0 || num_pages > UINT32_MAX || page_size < 1)
    return fail(MKVH_ERR_INVALID_ARGUMENT, "bad pool size");
  KvPool *p = new (std::nothrow) KvPool(num_pages, page_size);
  if (!p) return fail(MKVH_ERR_EXHAUSTED, "host allocation failed");
  *out = reinterpret_cast<mkvh_kv_pool *>(p);
  return MKVH_OK;
}
void mkvh_kv_pool_destroy(mkvh_kv_pool *pool) { delete reinterpret_cast<KvPool *>(pool); }
int mkvh_kv_pool_allocate(mkvh_kv_pool *pool, uint64_t owner, uint32_t *out_page) {
  H_CHECK(pool && out_page);
  return reinterpret_cast<KvPool *>(pool)->allocate(owner, out_page);
}
int mkvh_kv_pool_free(mkvh_kv_pool *pool, uint32_t page) {
  H_CHECK(pool);
  return reinterpret_cast<KvPool *>(pool)->free(page);
}
int64_t mkvh_kv_pool_free_pages(const mkvh_kv_pool *pool) {
  return pool ? (int64_t)reinterpret_cast<const KvPool *>(pool)->free_stack.size() : -1;
}
int64_t mkvh_kv_pool_total_pages(const mkvh_kv_pool *pool) {
  return pool ? reinterpret_cast<const KvPool *>(pool)->num_pages : -1;
}
int mkvh_kv_pool_page_state(const mkvh_kv_pool *pool, uint32_t page, int32_t *in_use, uint64_t *owner,
                            int32_t *refcount) {
  H_CHECK(pool);
  const KvPool *p = reinterpret_cast<const KvPool *>(pool);
  if (!p->valid(page)) return fail(MKVH_ERR_INVALID_ARGUMENT, "page %u out of range", page);
  if (in_use) *in_use = p->in_use[page];
  if (owner) *owner = p->owner[page];
  if (refcount) *refcount = p->refcnt[page];
  return MKVH_OK;
}
int mkvh_kv_pool_retain(mkvh_kv_pool *pool, uint32_t page) {
  H_CHECK(pool);
  return reinterpret_cast<KvPool *>(pool)->retain(page);
}
int mkvh_kv_pool_release(mkvh_kv_pool *pool, uint32_t page, int32_t *out_freed) {
  H_CHECK(pool);
  bool f = false;
  int rc = reinterpret_cast<KvPool *>(pool)->release(page, &f);
  if (out_freed) *out_freed = f;
  return rc;
}

// ---- PageTable ----------------------------------------------------------------------

int mkvh_page_table_create(mkvh_page_table **out) {
  if (!out) return fail(MKVH_ERR_INVALID_ARGUMENT, "NULL out");
  *out = reinterpret_cast<mkvh_page_table *>(new (std::nothrow) PageTable());
  return *out ? MKVH_OK : fail(MKVH_ERR_EXHAUSTED, "host allocation failed");
}
void mkvh_page_table_destroy(mkvh_page_table *pt) { delete reinterpret_cast<PageTable *>(pt); }
int mkvh_page_table_insert(mkvh_page_table *pt, uint64_t req, int64_t slot, uint32_t page) {
  H_CHECK(pt);
  reinterpret_cast<PageTable *>(pt)->m[{req, slot}] = page;
  return MKVH_OK;
}
int mkvh_page_table_lookup(const mkvh_page_table *pt, uint64_t req, int64_t slot, uint32_t *out_page) {
  H_CHECK(pt && out_page);
  const auto &m = reinterpret_cast<const PageTable *>(pt)->m;
  auto it = m.find({req, slot});
  if (it == m.end()) return fail(MKVH_ERR_NOT_FOUND, "no page for (request, slot %lld)", (long long)slot);
  *out_page = it->second;
  return MKVH_OK;
}
int mkvh_page_table_remove_request(mkvh_page_table *pt, uint64_t req, uint32_t *out_pages, int64_t cap,
                                   int64_t *out_n) {
  H_CHECK(pt && out_n);
  auto &m = reinterpret_cast<PageTable *>(pt)->m;
  auto lo = m.lower_bound({req, INT64_MIN}), hi = m.upper_bound({req, INT64_MAX});
  const int64_t n = std::distance(lo, hi);
  if (n > cap) return fail(MKVH_ERR_BUFFER_TOO_SMALL, "need room for %lld pages", (long long)n);
  if (n && !out_pages) return fail(MKVH_ERR_INVALID_ARGUMENT, "NULL out_pages");
  int64_t i = 0;
  for (auto it = lo; it != hi; ++it) out_pages[i++] = it->second;
  m.erase(lo, hi);
  *out_n = n;
  return MKVH_OK;
}

// ---- RadixCache -----------------------------------------------------------------------

int mkvh_radix_create(int32_t page_size, int64_t max_pages, mkvh_radix **out) {
  if (!out || page_size < 1 || max_pages < 0) return fail(MKVH_ERR_INVALID_ARGUMENT, "bad radix arguments");
  *out = reinterpret_cast<mkvh_radix *>(new (std::nothrow) Radix(page_size, max_pages));
  return *out ? MKVH_OK : fail(MKVH_ERR_EXHAUSTED, "host allocation failed");
}
void mkvh_radix_destroy(mkvh_radix *r) { delete reinterpret_cast<Radix *>(r); }

int mkvh_radix_match_prefix(mkvh_radix *r, const uint32_t *tokens, int64_t n_tokens, int64_t *out_matched_len,
                            uint32_t *out_pages, int64_t pages_cap, int64_t *out_n_pages, uint64_t *out_nodes,
                            int64_t nodes_cap, int64_t *out_n_nodes) {
  H_CHECK(r);
  Radix *x = reinterpret_cast<Radix *>(r);
  if (n_tokens < 0 || (n_tokens && !tokens) || !out_matched_len || !out_n_pages || !out_n_nodes)
    return fail(MKVH_ERR_INVALID_ARGUMENT, "bad arguments");
  const int64_t bound = n_tokens / x->page_size;
  if (pages_cap < bound || nodes_cap < bound)
    return fail(MKVH_ERR_BUFFER_TOO_SMALL, "capacities must be >= n_tokens / page_size = %lld", (long long)bound);
  if (bound && (!out_pages || !out_nodes)) return fail(MKVH_ERR_INVALID_ARGUMENT, "NULL output arrays");
  size_t matched = 0;
  std::vector<uint32_t> pages;
  std::vector<size_t> nodes;
  x->match_prefix(tokens, (size_t)n_tokens, &matched, pages, nodes);
  *out_matched_len = (int64_t)matched;
  *out_n_pages = (int64_t)pages.size();
  *out_n_nodes = (int64_t)nodes.size();
  std::copy(pages.begin(), pages.end(), out_pages);
  for (size_t i = 0; i < nodes.size(); i++) out_nodes[i] = nodes[i];
  return MKVH_OK;
}

int mkvh_radix_insert_prefix(mkvh_radix *r, const uint32_t *tokens, int64_t n_tokens, const uint32_t *pages,
                             int64_t n_pages) {
  H_CHECK(r);
  Radix *x = reinterpret_cast<Radix *>(r);
  if (n_pages < 0 || n_tokens < n_pages * x->page_size || (n_pages && (!tokens || !pages)))
    return fail(MKVH_ERR_INVALID_ARGUMENT, "insert_prefix needs n_tokens >= n_pages * page_size");
  std::vector<uint32_t> adopted;
  x->insert_prefix(tokens, pages, (size_t)n_pages, x->evicted, adopted);
  return MKVH_OK;
}

int mkvh_radix_unlock_nodes(mkvh_radix *r, const uint64_t *nodes, int64_t n) {
  H_CHECK(r);
  if (n < 0 || (n && !nodes)) return fail(MKVH_ERR_INVALID_ARGUMENT, "bad node list");
  reinterpret_cast<Radix *>(r)->unlock_nodes(nodes, (size_t)n);
  return MKVH_OK;
}

int mkvh_radix_evict_pages(mkvh_radix *r, int64_t target, int64_t *out_n_freed) {
  H_CHECK(r);
  if (target < 0) return fail(MKVH_ERR_INVALID_ARGUMENT, "target < 0");
  Radix *x = reinterpret_cast<Radix *>(r);
  const size_t before = x->evicted.size();
  x->evict_pages((size_t)target, x->evicted);
  if (out_n_freed) *out_n_freed = (int64_t)(x->evicted.size() - before);
  return MKVH_OK;
}

int mkvh_radix_drain_evicted(mkvh_radix *r, uint32_t *out_pages, int64_t cap, int64_t *out_n) {
  H_CHECK(r);
  if (!out_n || cap < 0 || (cap && !out_pages)) return fail(MKVH_ERR_INVALID_ARGUMENT, "bad buffer");
  Radix *x = reinterpret_cast<Radix *>(r);
  const int64_t n = std::min<int64_t>(cap, (int64_t)x->evicted.size());
  std::copy(x->evicted.begin(), x->evicted.begin() + n, out_pages);
  x->evicted.erase(x->evicted.begin(), x->evicted.begin() + n);
  *out_n = n;
  return MKVH_OK;
}

int mkvh_radix_promote_request(mkvh_radix *r, const uint32_t *input_ids, int64_t n_input, int64_t device_len,
                               const uint32_t *kv_pages, int64_t n_pages) {
  H_CHECK(r);
  Radix *x = reinterpret_cast<Radix *>(r);
  const int64_t full = device_len / x->page_size;
  if (full == 0) return MKVH_OK;
  if (device_len < 0 || n_input < full * x->page_size || n_pages < full || !input_ids || !kv_pages)
    return fail(MKVH_ERR_INVALID_ARGUMENT, "promote_request: input_ids or kv_pages shorter than device_len");
  std::vector<uint32_t> adopted;
  x->insert_prefix(input_ids, kv_pages, (size_t)full, x->evicted, adopted);
  return MKVH_OK;
}

int64_t mkvh_radix_total_cached_pages(const mkvh_radix *r) {
  return r ? reinterpret_cast<const Radix *>(r)->total_pages : -1;
}
int64_t mkvh_radix_num_nodes(const mkvh_radix *r) {
  return r ? (int64_t)reinterpret_cast<const Radix *>(r)->live_count : -1;
}

// ---- Block manager ----------------------------------------------------------------------

int mkvh_bm_create(int64_t num_blocks, int32_t page_size, int64_t max_cached_pages, mkvh_block_manager **out) {
  if (!out || num_blocks < 0 || num_blocks > UINT32_MAX || page_size < 1 || max_cached_pages < 0)
    return fail(MKVH_ERR_INVALID_ARGUMENT, "bad block manager arguments");
  // Slots (block * page_size + offset) and the batch's block ids are int32.
  if (num_blocks * (int64_t)page_size > INT32_MAX)
    return fail(MKVH_ERR_INVALID_ARGUMENT, "%lld blocks of %d tokens: slots would not fit int32",
                (long long)num_blocks, page_size);
  *out = reinterpret_cast<mkvh_block_manager *>(new (std::nothrow) BlockMgr(num_blocks, page_size, max_cached_pages));
  return *out ? MKVH_OK : fail(MKVH_ERR_EXHAUSTED, "host allocation failed");
}
void mkvh_bm_destroy(mkvh_block_manager *bm) { delete reinterpret_cast<BlockMgr *>(bm); }

int mkvh_bm_admit(mkvh_block_manager *bm, uint64_t seq, const uint32_t *tokens, int64_t n_tokens,
                  int64_t *out_cached_len) {
  H_CHECK(bm);
  BlockMgr *m = reinterpret_cast<BlockMgr *>(bm);
  if (n_tokens < 1 || !tokens) return fail(MKVH_ERR_INVALID_ARGUMENT, "a prompt needs >= 1 token");
  if (m->seqs.count(seq)) return fail(MKVH_ERR_INVALID_ARGUMENT, "sequence %llu already admitted", (unsigned long long)seq);
  const int64_t need = (n_tokens + m->ps - 1) / m->ps;
  // prefill.rs:44-55: evict the deficit once, then admit only if it fits.
  m->make_room(need);
  if ((int64_t)m->pool.free_stack.size() < need) {
    // Matched pages need no fresh block; count them before refusing.
    size_t matched = 0;
    std::vector<uint32_t> pg;
    std::vector<size_t> nd;
    Radix probe = m->radix;  // match without touching locks or LRU stamps
    probe.match_prefix(tokens, (size_t)n_tokens, &matched, pg, nd);
    if ((int64_t)m->pool.free_stack.size() < need - (int64_t)pg.size())
      return fail(MKVH_ERR_EXHAUSTED, "cannot admit %lld-token prompt: %zu free blocks", (long long)n_tokens,
                  m->pool.free_stack.size());
  }
  Seq s;
  size_t matched = 0;
  m->radix.match_prefix(tokens, (size_t)n_tokens, &matched, s.blocks, s.locked);
  const int held = retain_all(m->pool, s.blocks);
  while ((int64_t)s.blocks.size() < need) {
    uint32_t b;
    if (m->pool.allocate(seq, &b) != MKVH_OK) {  // not reachable after the check above
      std::vector<uint64_t> ids(s.locked.begin(), s.locked.end());
      m->radix.unlock_nodes(ids.data(), ids.size());
      (void)release_all(m->pool, s.blocks);
      return MKVH_ERR_EXHAUSTED;
    }
    s.blocks.push_back(b);
  }
  s.len = (int64_t)matched;
  s.prompt = n_tokens;
  m->seqs.emplace(seq, std::move(s));
  if (out_cached_len) *out_cached_len = (int64_t)matched;
  return held;
}

int mkvh_bm_fork(mkvh_block_manager *bm, uint64_t parent, uint64_t child) {
  H_CHECK(bm);
  BlockMgr *m = reinterpret_cast<BlockMgr *>(bm);
  auto it = m->seqs.find(parent);
  if (it == m->seqs.end()) return fail(MKVH_ERR_NOT_FOUND, "unknown sequence %llu", (unsigned long long)parent);
  if (m->seqs.count(child)) return fail(MKVH_ERR_INVALID_ARGUMENT, "sequence %llu exists", (unsigned long long)child);
  Seq c = it->second;
  const int held = retain_all(m->pool, c.blocks);
  m->radix.lock_nodes(c.locked);
  m->seqs.emplace(child, std::move(c));
  return held;
}

int mkvh_bm_append(mkvh_block_manager *bm, uint64_t seq, int32_t n_new, int32_t *out_slots, int32_t *out_cow_src,
                   int32_t *out_cow_dst, int32_t *out_n_cow) {
  H_CHECK(bm);
  BlockMgr *m = reinterpret_cast<BlockMgr *>(bm);
  auto it = m->seqs.find(seq);
  if (it == m->seqs.end()) return fail(MKVH_ERR_NOT_FOUND, "unknown sequence %llu", (unsigned long long)seq);
  if (n_new < 0 || (n_new && !out_slots) || !out_n_cow) return fail(MKVH_ERR_INVALID_ARGUMENT, "bad arguments");
  Seq &s = it->second;
  const int64_t ps = m->ps;
  const int64_t end = s.len + n_new;
  const int64_t grow = std::max<int64_t>(0, (end + ps - 1) / ps - (int64_t)s.blocks.size());
  // Every block this append writes that another holder shares (a fork, or
  // blocks reserved at admission and shared before they were written) gets
  // a private block first. Only the block holding position len with rows
  // already written (len % ps != 0) needs its contents copied: the others
  // hold none of this sequence's rows yet.
  const int64_t j0 = s.len / ps;
  const int64_t j_end = n_new > 0 ? std::min<int64_t>((end + ps - 1) / ps, (int64_t)s.blocks.size()) : j0;
  std::vector<int64_t> shared;
  for (int64_t j = j0; j < j_end; j++)
    if (m->pool.refcnt[s.blocks[j]] > 1) shared.push_back(j);
  const bool copy_needed = !shared.empty() && shared[0] == j0 && s.len % ps != 0;
  if (copy_needed && !(out_cow_src && out_cow_dst))
    return fail(MKVH_ERR_INVALID_ARGUMENT, "append writes a shared partial block: pass the copy-pair outputs");
  const int64_t need = grow + (int64_t)shared.size();
  m->make_room(need);
  if ((int64_t)m->pool.free_stack.size() < need)
    return fail(MKVH_ERR_EXHAUSTED, "append needs %lld blocks, %zu free", (long long)need, m->pool.free_stack.size());
  *out_n_cow = 0;
  // The allocations below cannot fail: `need` free blocks were checked above.
  for (int64_t j : shared) {
    uint32_t fresh = 0;
    if (m->pool.allocate(seq, &fresh) != MKVH_OK) return MKVH_ERR_EXHAUSTED;
    const uint32_t old = s.blocks[j];
    bool freed = false;
    if (m->pool.release(old, &freed) != MKVH_OK) return MKVH_ERR_NOT_IN_USE;
    s.blocks[j] = fresh;
    if (j * ps < s.len) {  // rows [j*ps, len) of this block are written: copy them
      out_cow_src[0] = (int32_t)old;
      out_cow_dst[0] = (int32_t)fresh;
      *out_n_cow = 1;
    }
  }
  for (int64_t p = s.len; p < end; p++) {
    if (p / ps == (int64_t)s.blocks.size()) {
      uint32_t b = 0;
      if (m->pool.allocate(seq, &b) != MKVH_OK) return MKVH_ERR_EXHAUSTED;
      s.blocks.push_back(b);
    }
    out_slots[p - s.len] = (int32_t)(s.blocks[p / ps] * ps + p % ps);
  }
  s.len = end;
  return MKVH_OK;
}

// schedule_prefill_chunk (prefill.rs:99-114) for one request: min(remaining,
// budget - used), nothing when the request has no prompt left.
static int64_t prefill_chunk(int64_t remaining, int64_t budget, int64_t &used) {
  if (remaining <= 0) return 0;
  const int64_t chunk = std::min(remaining, budget - used);
  if (chunk <= 0) return 0;
  used += chunk;
  return chunk;
}

int mkvh_schedule_prefill_chunks(int64_t budget, const int64_t *remaining, int32_t n, int64_t *out_chunks,
                                 int64_t *out_used) {
  if (budget < 0 || n < 0 || (n && (!remaining || !out_chunks)))
    return fail(MKVH_ERR_INVALID_ARGUMENT, "bad chunk-schedule arguments");
  for (int32_t i = 0; i < n; i++)
    if (remaining[i] < 0) return fail(MKVH_ERR_INVALID_ARGUMENT, "remaining[%d] = %lld < 0", i, (long long)remaining[i]);
  int64_t used = 0;
  for (int32_t i = 0; i < n; i++) out_chunks[i] = 0;
  // prefill.rs:27-36: in order, stopping once the budget is used up.
  for (int32_t i = 0; i < n && used < budget; i++) out_chunks[i] = prefill_chunk(remaining[i], budget, used);
  if (out_used) *out_used = used;
  return MKVH_OK;
}

int mkvh_bm_schedule_prefill(mkvh_block_manager *bm, int64_t budget, const uint64_t *in_progress, int32_t n_in_progress,
                             const uint64_t *waiting, const int64_t *waiting_indptr, const uint32_t *waiting_tokens,
                             int32_t n_waiting, int64_t *out_chunks, int32_t *out_n_admitted,
                             int64_t *out_cached_lens) {
  H_CHECK(bm);
  BlockMgr *m = reinterpret_cast<BlockMgr *>(bm);
  if (budget < 0 || n_in_progress < 0 || n_waiting < 0 || !out_n_admitted ||
      (n_in_progress && !in_progress) || (n_in_progress + n_waiting > 0 && !out_chunks) ||
      (n_waiting && (!waiting || !waiting_indptr || !out_cached_lens)))
    return fail(MKVH_ERR_INVALID_ARGUMENT, "bad prefill-schedule arguments");
  // Every argument is checked before the books change: each sequence id
  // appears once in the two lists together.
  std::unordered_set<uint64_t> seen;
  for (int32_t i = 0; i < n_in_progress; i++) {
    if (!m->seqs.count(in_progress[i]))
      return fail(MKVH_ERR_NOT_FOUND, "unknown sequence %llu", (unsigned long long)in_progress[i]);
    if (!seen.insert(in_progress[i]).second)
      return fail(MKVH_ERR_INVALID_ARGUMENT, "sequence %llu listed twice", (unsigned long long)in_progress[i]);
  }
  if (n_waiting && waiting_indptr[0] != 0) return fail(MKVH_ERR_INVALID_ARGUMENT, "waiting_indptr[0] != 0");
  for (int32_t i = 0; i < n_waiting; i++) {
    if (waiting_indptr[i + 1] <= waiting_indptr[i])
      return fail(MKVH_ERR_INVALID_ARGUMENT, "waiting request %d has no prompt tokens", i);
    if (m->seqs.count(waiting[i]))
      return fail(MKVH_ERR_INVALID_ARGUMENT, "sequence %llu already admitted", (unsigned long long)waiting[i]);
    if (!seen.insert(waiting[i]).second)
      return fail(MKVH_ERR_INVALID_ARGUMENT, "sequence %llu listed twice", (unsigned long long)waiting[i]);
  }
  if (n_waiting && !waiting_tokens) return fail(MKVH_ERR_INVALID_ARGUMENT, "NULL waiting tokens");
  for (int32_t i = 0; i < n_in_progress + n_waiting; i++) out_chunks[i] = 0;
  *out_n_admitted = 0;
  int64_t used = 0;
  // 1. In-progress prefills first (prefill.rs:27-36).
  for (int32_t i = 0; i < n_in_progress && used < budget; i++) {
    const Seq &s = m->seqs.at(in_progress[i]);
    out_chunks[i] = prefill_chunk(s.prompt - s.len, budget, used);
  }
  // 2. Admission from the waiting queue while budget remains (prefill.rs:39-93).
  for (int32_t i = 0; i < n_waiting && used < budget; i++) {
    int64_t cached = 0;
    const uint32_t *tok = waiting_tokens + waiting_indptr[i];
    const int64_t n_tok = waiting_indptr[i + 1] - waiting_indptr[i];
    const int rc = mkvh_bm_admit(bm, waiting[i], tok, n_tok, &cached);
    if (rc == MKVH_ERR_EXHAUSTED) break;  // cannot admit this request yet
    if (rc != MKVH_OK) return rc;
    out_cached_lens[i] = cached;
    *out_n_admitted = i + 1;
    out_chunks[n_in_progress + i] = prefill_chunk(n_tok - cached, budget, used);
  }
  return MKVH_OK;
}

int mkvh_bm_promote(mkvh_block_manager *bm, uint64_t seq, const uint32_t *tokens, int64_t n_tokens) {
  H_CHECK(bm);
  BlockMgr *m = reinterpret_cast<BlockMgr *>(bm);
  auto it = m->seqs.find(seq);
  if (it == m->seqs.end()) return fail(MKVH_ERR_NOT_FOUND, "unknown sequence %llu", (unsigned long long)seq);
  Seq &s = it->second;
  const int64_t full = std::min<int64_t>(s.len, n_tokens) / m->ps;
  if (full == 0) return MKVH_OK;
  if (!tokens) return fail(MKVH_ERR_INVALID_ARGUMENT, "NULL tokens");
  std::vector<uint32_t> evicted, adopted;
  m->radix.insert_prefix(tokens, s.blocks.data(), (size_t)full, evicted, adopted);
  const int held = retain_all(m->pool, adopted);
  m->drop_tree_pages(evicted);
  return held;
}

int mkvh_bm_release(mkvh_block_manager *bm, uint64_t seq) {
  H_CHECK(bm);
  BlockMgr *m = reinterpret_cast<BlockMgr *>(bm);
  auto it = m->seqs.find(seq);
  if (it == m->seqs.end()) return fail(MKVH_ERR_NOT_FOUND, "unknown sequence %llu", (unsigned long long)seq);
  std::vector<uint64_t> ids(it->second.locked.begin(), it->second.locked.end());
  m->radix.unlock_nodes(ids.data(), ids.size());
  const int rc = release_all(m->pool, it->second.blocks);
  m->seqs.erase(it);
  return rc;
}

int mkvh_bm_evict(mkvh_block_manager *bm, int64_t target_pages, int64_t *out_freed_blocks) {
  H_CHECK(bm);
  if (target_pages < 0) return fail(MKVH_ERR_INVALID_ARGUMENT, "target < 0");
  BlockMgr *m = reinterpret_cast<BlockMgr *>(bm);
  std::vector<uint32_t> ev;
  m->radix.evict_pages((size_t)target_pages, ev);
  const int64_t freed = m->drop_tree_pages(ev);
  if (out_freed_blocks) *out_freed_blocks = freed;
  return MKVH_OK;
}

int mkvh_bm_plan_compaction(mkvh_block_manager *bm, int32_t *out_src, int32_t *out_dst, int64_t cap,
                            int64_t *out_n) {
  H_CHECK(bm);
  BlockMgr *m = reinterpret_cast<BlockMgr *>(bm);
  KvPool &pool = m->pool;
  if (!out_n) return fail(MKVH_ERR_INVALID_ARGUMENT, "NULL out_n");
  const int64_t N = pool.num_pages;
  const int64_t live = N - (int64_t)pool.free_stack.size();
  std::vector<uint32_t> holes, movers;
  for (int64_t b = 0; b < live; b++)
    if (!pool.in_use[b]) holes.push_back((uint32_t)b);
  for (int64_t b = live; b < N; b++)
    if (pool.in_use[b]) movers.push_back((uint32_t)b);
  if ((int64_t)movers.size() > cap)
    return fail(MKVH_ERR_BUFFER_TOO_SMALL, "compaction needs room for %zu moves", movers.size());
  if (!movers.empty() && !(out_src && out_dst))
    return fail(MKVH_ERR_INVALID_ARGUMENT, "compaction moves %zu blocks: pass out_src and out_dst", movers.size());
  std::vector<int64_t> remap(N, -1);
  for (size_t i = 0; i < movers.size(); i++) {
    const uint32_t s = movers[i], d = holes[i];
    remap[s] = d;
    pool.in_use[d] = 1;
    pool.owner[d] = pool.owner[s];
    pool.refcnt[d] = pool.refcnt[s];
    pool.in_use[s] = 0;
    pool.refcnt[s] = 0;
    pool.owner[s] = 0;
    out_src[i] = (int32_t)s;
    out_dst[i] = (int32_t)d;
  }
  for (auto &kv : m->seqs)
    for (uint32_t &b : kv.second.blocks)
      if (remap[b] >= 0) b = (uint32_t)remap[b];
  for (Node &nd : m->radix.nodes)
    if (nd.live)
      for (uint32_t &p : nd.pages)
        if (remap[p] >= 0) p = (uint32_t)remap[p];
  // Free ids are now exactly [live, N): the stack hands them out ascending.
  pool.free_stack.clear();
  for (int64_t b = N - 1; b >= live; b--) pool.free_stack.push_back((uint32_t)b);
  *out_n = (int64_t)movers.size();
  return MKVH_OK;
}

int mkvh_bm_seq_len(const mkvh_block_manager *bm, uint64_t seq, int64_t *out_len) {
  H_CHECK(bm && out_len);
  const BlockMgr *m = reinterpret_cast<const BlockMgr *>(bm);
  auto it = m->seqs.find(seq);
  if (it == m->seqs.end()) return fail(MKVH_ERR_NOT_FOUND, "unknown sequence %llu", (unsigned long long)seq);
  *out_len = it->second.len;
  return MKVH_OK;
}

int mkvh_bm_table(const mkvh_block_manager *bm, uint64_t seq, int32_t *out_blocks, int64_t cap, int64_t *out_n) {
  H_CHECK(bm && out_n);
  const BlockMgr *m = reinterpret_cast<const BlockMgr *>(bm);
  auto it = m->seqs.find(seq);
  if (it == m->seqs.end()) return fail(MKVH_ERR_NOT_FOUND, "unknown sequence %llu", (unsigned long long)seq);
  const auto &b = it->second.blocks;
  if ((int64_t)b.size() > cap) return fail(MKVH_ERR_BUFFER_TOO_SMALL, "table has %zu blocks", b.size());
  for (size_t i = 0; i < b.size(); i++) out_blocks[i] = (int32_t)b[i];
  *out_n = (int64_t)b.size();
  return MKVH_OK;
}

int mkvh_bm_batch(const mkvh_block_manager *bm, const uint64_t *seqs, int32_t n_seqs, int32_t *out_indptr,
                  int32_t *out_ids, int64_t ids_cap, int32_t *out_ctx_lens) {
  H_CHECK(bm);
  const BlockMgr *m = reinterpret_cast<const BlockMgr *>(bm);
  if (n_seqs < 0 || (n_seqs && (!seqs || !out_ctx_lens)) || !out_indptr)
    return fail(MKVH_ERR_INVALID_ARGUMENT, "bad arguments");
  int64_t total = 0;
  for (int32_t i = 0; i < n_seqs; i++) {
    auto it = m->seqs.find(seqs[i]);
    if (it == m->seqs.end()) return fail(MKVH_ERR_NOT_FOUND, "unknown sequence %llu", (unsigned long long)seqs[i]);
    total += (int64_t)it->second.blocks.size();
  }
  if (total > ids_cap) return fail(MKVH_ERR_BUFFER_TOO_SMALL, "batch holds %lld block ids", (long long)total);
  out_indptr[0] = 0;
  int64_t k = 0;
  for (int32_t i = 0; i < n_seqs; i++) {
    const Seq &s = m->seqs.at(seqs[i]);
    for (uint32_t b : s.blocks) out_ids[k++] = (int32_t)b;
    out_indptr[i + 1] = (int32_t)k;
    out_ctx_lens[i] = (int32_t)s.len;
  }
  return MKVH_OK;
}

int64_t mkvh_bm_free_blocks(const mkvh_block_manager *bm) {
  return bm ? (int64_t)reinterpret_cast<const BlockMgr *>(bm)->pool.free_stack.size() : -1;
}
int64_t mkvh_bm_live_blocks(const mkvh_block_manager *bm) {
  if (!bm) return -1;
  const BlockMgr *m = reinterpret_cast<const BlockMgr *>(bm);
  return m->pool.num_pages - (int64_t)m->pool.free_stack.size();
}
int32_t mkvh_bm_refcount(const mkvh_block_manager *bm, uint32_t block) {
  if (!bm) return -1;
  const BlockMgr *m = reinterpret_cast<const BlockMgr *>(bm);
  return m->pool.valid(block) ? m->pool.refcnt[block] : -1;
}
int64_t mkvh_bm_cached_pages(const mkvh_block_manager *bm) {
  return bm ? reinterpret_cast<const BlockMgr *>(bm)->radix.total_pages : -1;
}

int mkvh_bm_check_invariants(const mkvh_block_manager *bm) {
  H_CHECK(bm);
  const BlockMgr *m = reinterpret_cast<const BlockMgr *>(bm);
  const KvPool &pool = m->pool;
  std::vector<int32_t> holders(pool.num_pages, 0);
  for (const auto &kv : m->seqs)
    for (uint32_t b : kv.second.blocks) {
      if (!pool.valid(b)) return fail(MKVH_ERR_INVALID_ARGUMENT, "sequence holds block %u out of range", b);
      holders[b]++;
    }
  int64_t tree_pages = 0;
  for (const Node &nd : m->radix.nodes)
    if (nd.live)
      for (uint32_t p : nd.pages) {
        if (!pool.valid(p)) return fail(MKVH_ERR_INVALID_ARGUMENT, "tree holds page %u out of range", p);
        holders[p]++;
        tree_pages++;
      }
  if (tree_pages != m->radix.total_pages)
    return fail(MKVH_ERR_INVALID_ARGUMENT, "tree counts %lld pages, nodes hold %lld",
                (long long)m->radix.total_pages, (long long)tree_pages);
  std::vector<uint8_t> on_stack(pool.num_pages, 0);
  for (uint32_t p : pool.free_stack) {
    if (on_stack[p]) return fail(MKVH_ERR_INVALID_ARGUMENT, "page %u twice on the free stack", p);
    on_stack[p] = 1;
  }
  for (int64_t b = 0; b < pool.num_pages; b++) {
    if (pool.in_use[b] == on_stack[b])
      return fail(MKVH_ERR_INVALID_ARGUMENT, "page %lld: in_use=%d but on free stack=%d", (long long)b,
                  pool.in_use[b], on_stack[b]);
    if (pool.in_use[b] && pool.refcnt[b] != holders[b])
      return fail(MKVH_ERR_INVALID_ARGUMENT, "block %lld: refcount %d, holders %d", (long long)b, pool.refcnt[b],
                  holders[b]);
    if (!pool.in_use[b] && holders[b])
      return fail(MKVH_ERR_INVALID_ARGUMENT, "free block %lld still held %d times", (long long)b, holders[b]);
  }
  return MKVH_OK;
}

}  // extern "C"
