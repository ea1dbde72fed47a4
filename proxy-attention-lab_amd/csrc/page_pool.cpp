// Page-pool allocator and compaction planner (host side) of libpal_hip.so.
//
// The reference has no allocator: page tables come from the caller
// (src/proxy_attention_lab/ops.py:61-63, paged_attention_decode_primitive.cpp
// takes them as an input array).  This is the allocator a serving engine
// puts in front of the paged pools: page ids handed out lowest-first, freed
// back, and a compaction plan that moves every live page above the live
// count into a hole below it, so the live pages end up as [0, live).  The
// plan is applied on the GPU by pal_copy_pages and pal_remap_pages
// (page_ops.hip).  A pool object is internally locked; its calls are safe
// from several threads.
#include <algorithm>
#include <cstdint>
#include <cstring>
#include <mutex>
#include <new>
#include <set>
#include <string>
#include <vector>

#include "../../include/pal_hip.h"
#include "pal_log.h"

namespace {

struct PagePool {
  std::mutex mu;
  int64_t num_pages = 0;
  std::vector<uint8_t> used;  // used[p] != 0: page p is allocated
  std::set<uint32_t> free_ids;  // ascending: allocation takes the lowest ids
};

int pool_fail(int code, const std::string& msg) {
  pal::set_last_error(msg.c_str());
  return code;
}

PagePool* as_pool(void* h) { return static_cast<PagePool*>(h); }

}  // namespace

extern "C" {

int pal_page_pool_create(int64_t num_pages, void** pool) {
  if (!pool) return pool_fail(PAL_ERR_INVALID_ARGUMENT, "[page_pool] null handle pointer");
  *pool = nullptr;
  if (num_pages < 0 || num_pages > 0xFFFFFFFFLL)
    return pool_fail(PAL_ERR_INVALID_ARGUMENT, "[page_pool] num_pages must be in [0, 2^32)");
  PagePool* p = new (std::nothrow) PagePool();
  if (!p) return pool_fail(PAL_ERR_RUNTIME, "[page_pool] out of host memory");
  p->num_pages = num_pages;
  p->used.assign(static_cast<size_t>(num_pages), 0);
  for (int64_t i = 0; i < num_pages; ++i) p->free_ids.insert(p->free_ids.end(), static_cast<uint32_t>(i));
  *pool = p;
  PAL_LOG("page_pool create %p pages=%lld", static_cast<void*>(p), static_cast<long long>(num_pages));
  pal::clear_last_error();
  return PAL_OK;
}

int pal_page_pool_destroy(void* pool) {
  delete as_pool(pool);
  pal::clear_last_error();
  return PAL_OK;
}

int64_t pal_page_pool_num_free(void* pool) {
  PagePool* p = as_pool(pool);
  if (!p) return pool_fail(PAL_ERR_INVALID_ARGUMENT, "[page_pool] null pool");
  std::lock_guard<std::mutex> lock(p->mu);
  return static_cast<int64_t>(p->free_ids.size());
}

int pal_page_pool_alloc(void* pool, int64_t n, uint32_t* out_ids) {
  PagePool* p = as_pool(pool);
  if (!p) return pool_fail(PAL_ERR_INVALID_ARGUMENT, "[page_pool] null pool");
  if (n < 0 || (n > 0 && !out_ids)) return pool_fail(PAL_ERR_INVALID_ARGUMENT, "[page_pool] bad allocation request");
  std::lock_guard<std::mutex> lock(p->mu);
  if (static_cast<int64_t>(p->free_ids.size()) < n)
    return pool_fail(PAL_ERR_RUNTIME, "[page_pool] out of pages: " + std::to_string(n) + " requested, " +
                                          std::to_string(p->free_ids.size()) + " free");
  auto it = p->free_ids.begin();
  for (int64_t i = 0; i < n; ++i) {
    const uint32_t id = *it;
    it = p->free_ids.erase(it);
    p->used[id] = 1;
    out_ids[i] = id;
  }
  pal::clear_last_error();
  return PAL_OK;
}

int pal_page_pool_free(void* pool, const uint32_t* ids, int64_t n) {
  PagePool* p = as_pool(pool);
  if (!p) return pool_fail(PAL_ERR_INVALID_ARGUMENT, "[page_pool] null pool");
  if (n < 0 || (n > 0 && !ids)) return pool_fail(PAL_ERR_INVALID_ARGUMENT, "[page_pool] bad free request");
  std::lock_guard<std::mutex> lock(p->mu);
  // validate everything first: a rejected call changes nothing
  std::vector<uint32_t> sorted(ids, ids + n);
  std::sort(sorted.begin(), sorted.end());
  for (int64_t i = 0; i < n; ++i) {
    const uint32_t id = sorted[i];
    if (id >= p->num_pages)
      return pool_fail(PAL_ERR_INVALID_ARGUMENT, "[page_pool] page " + std::to_string(id) + " out of range");
    if (!p->used[id])
      return pool_fail(PAL_ERR_INVALID_ARGUMENT, "[page_pool] page " + std::to_string(id) + " is not allocated");
    if (i > 0 && sorted[i - 1] == id)
      return pool_fail(PAL_ERR_INVALID_ARGUMENT, "[page_pool] page " + std::to_string(id) + " freed twice");
  }
  for (const uint32_t id : sorted) {
    p->used[id] = 0;
    p->free_ids.insert(id);
  }
  pal::clear_last_error();
  return PAL_OK;
}

int pal_page_pool_compaction_plan(void* pool, uint32_t* src, uint32_t* dst, int64_t capacity, int64_t* n_moves) {
  PagePool* p = as_pool(pool);
  if (!p || !n_moves) return pool_fail(PAL_ERR_INVALID_ARGUMENT, "[page_pool] null pool or count pointer");
  std::lock_guard<std::mutex> lock(p->mu);
  const int64_t live = p->num_pages - static_cast<int64_t>(p->free_ids.size());
  // movers: live ids >= live, ascending; holes: free ids < live, ascending
  std::vector<uint32_t> movers, holes;
  for (int64_t id = live; id < p->num_pages; ++id)
    if (p->used[id]) movers.push_back(static_cast<uint32_t>(id));
  for (auto it = p->free_ids.begin(); it != p->free_ids.end() && *it < live; ++it) holes.push_back(*it);
  const int64_t m = static_cast<int64_t>(movers.size());
  *n_moves = m;
  if (m != static_cast<int64_t>(holes.size()))
    return pool_fail(PAL_ERR_RUNTIME, "[page_pool] inconsistent free set");  // cannot happen
  if (capacity < m || (m > 0 && (!src || !dst))) {
    if (capacity == 0 && !src && !dst) {  // a size query
      pal::clear_last_error();
      return PAL_OK;
    }
    return pool_fail(PAL_ERR_INVALID_ARGUMENT, "[page_pool] compaction needs " + std::to_string(m) +
                                                   " moves, room for " + std::to_string(capacity));
  }
  for (int64_t i = 0; i < m; ++i) {
    src[i] = movers[i];
    dst[i] = holes[i];
    p->used[movers[i]] = 0;
    p->used[holes[i]] = 1;
    p->free_ids.erase(holes[i]);
    p->free_ids.insert(movers[i]);
  }
  PAL_LOG("page_pool compaction %p live=%lld moves=%lld", static_cast<void*>(p), static_cast<long long>(live),
          static_cast<long long>(m));
  pal::clear_last_error();
  return PAL_OK;
}

}  // extern "C"
