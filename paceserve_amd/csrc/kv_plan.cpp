// Native block allocation, batch planning and single-call promotion.
//
// The allocator keeps the reference's LIFO order exactly: a fresh pool hands
// out num_pages-1, num_pages-2, ...; allocation pops from the back of the
// free list; a free appends each distinct page of the table once.  Planning
// allocates every request's destination pages in request order and remaps
// positionally: a table of n pages receives n source pages, a table of n+1
// pages receives them in its first n pages and its last page is left
// untouched.
//
// pace_kv_promote runs plan + id upload + page movement in one call: both id
// lists are written into one of two pinned host slots and copied to the
// matching device slot with one asynchronous copy on the caller's stream; a
// slot is reused only after the events recorded by its previous copy and its
// previous kernels, so back-to-back promotions never overwrite ids in use.
#include <string.h>

#include <mutex>
#include <vector>

#include "internal.h"

using pace_kv::fail;
using pace_kv::hip_status;

struct pace_kv_allocator {
  int64_t num_pages = 0;
  std::vector<int32_t> free_list;  // back() is allocated next
  std::vector<uint32_t> stamp;     // per page: last free() call that saw it (lazy)
  uint32_t generation = 0;
  std::mutex mu;
};

namespace {

// Pops n pages (LIFO) into out; caller holds the lock and checked the count.
void pop_pages(pace_kv_allocator* a, int64_t n, int32_t* out) {
  const int64_t size = static_cast<int64_t>(a->free_list.size());
  for (int64_t i = 0; i < n; ++i) out[i] = a->free_list[size - 1 - i];
  a->free_list.resize(size - n);
}

// Undoes pop_pages: pushing the pages back in reverse pop order restores the
// free list exactly.
void unpop_pages(pace_kv_allocator* a, int64_t n, const int32_t* pages) {
  for (int64_t i = n - 1; i >= 0; --i) a->free_list.push_back(pages[i]);
}

int check_page_range(const int32_t* ids, int64_t n, int64_t limit, const char* what) {
  for (int64_t i = 0; i < n; ++i) {
    if (ids[i] < 0 || ids[i] >= limit)
      return fail(PACE_KV_ERANGE, "%s: page id %d at position %lld outside [0, %lld)", what, ids[i],
                  (long long)i, (long long)limit);
  }
  return PACE_KV_OK;
}

struct Plan {
  int64_t n_src = 0;       // total source pages
  int64_t n_dst_table = 0;  // total destination pages allocated
};

// Validates a batch and computes its totals (no allocation).
int plan_sizes(int num_requests, const int64_t* indptr, const int32_t* src_ids,
               int64_t src_pool_pages, const int32_t* dst_pages, Plan* plan) {
  if (num_requests < 0) return fail(PACE_KV_EINVAL, "num_requests must be >= 0");
  if (num_requests == 0) return PACE_KV_OK;
  if (indptr == nullptr) return fail(PACE_KV_EINVAL, "indptr is NULL");
  if (indptr[0] != 0) return fail(PACE_KV_EINVAL, "indptr[0] must be 0");
  for (int r = 0; r < num_requests; ++r) {
    const int64_t n = indptr[r + 1] - indptr[r];
    if (n < 0) return fail(PACE_KV_EINVAL, "indptr decreases at request %d", r);
    const int64_t m = dst_pages ? dst_pages[r] : n;
    if (m != n && m != n + 1)
      return fail(PACE_KV_EINVAL, "request %d: %lld destination pages cannot receive %lld pages", r,
                  (long long)m, (long long)n);
    plan->n_dst_table += m;
  }
  plan->n_src = indptr[num_requests];
  if (plan->n_src > 0 && src_ids == nullptr) return fail(PACE_KV_EINVAL, "src_ids is NULL");
  if (plan->n_src > INT32_MAX) return fail(PACE_KV_ERANGE, "more than 2^31 pages in one batch");
  return check_page_range(src_ids, plan->n_src, src_pool_pages, "source ids");
}

// Allocates and remaps; dst_tables receives every request's full table,
// dst_ids the pages that receive data (CSR like the source ids).
int plan_allocate(pace_kv_allocator* a, int num_requests, const int64_t* indptr,
                  const int32_t* dst_pages, const Plan& plan, int32_t* dst_tables,
                  int32_t* dst_ids) {
  {
    std::lock_guard<std::mutex> lock(a->mu);
    if (plan.n_dst_table > static_cast<int64_t>(a->free_list.size()))
      return fail(PACE_KV_ENOMEM, "Out of memory! No free blocks are available. "
                  "(need %lld pages, %lld free)", (long long)plan.n_dst_table,
                  (long long)a->free_list.size());
    pop_pages(a, plan.n_dst_table, dst_tables);
  }
  int64_t pos = 0;
  for (int r = 0; r < num_requests; ++r) {
    const int64_t n = indptr[r + 1] - indptr[r];
    const int64_t m = dst_pages ? dst_pages[r] : n;
    memcpy(dst_ids + indptr[r], dst_tables + pos, n * sizeof(int32_t));
    pos += m;
  }
  return PACE_KV_OK;
}

}  // namespace

struct pace_kv_promoter {
  int device = -1;
  int64_t capacity = 0;           // int32 entries per slot
  int32_t* host[2] = {nullptr, nullptr};
  int32_t* dev[2] = {nullptr, nullptr};
  hipEvent_t copied[2] = {nullptr, nullptr};  // H2D out of host[s] finished
  hipEvent_t done[2] = {nullptr, nullptr};    // kernels reading dev[s] finished
  uint64_t calls = 0;
};

namespace {

void promoter_free_buffers(pace_kv_promoter* p) {
  for (int s = 0; s < 2; ++s) {
    if (p->host[s]) (void)hipHostFree(p->host[s]);
    if (p->dev[s]) (void)hipFree(p->dev[s]);
    p->host[s] = nullptr;
    p->dev[s] = nullptr;
  }
  p->capacity = 0;
}

int promoter_reserve(pace_kv_promoter* p, int64_t entries) {
  if (entries <= p->capacity) return PACE_KV_OK;
  for (int s = 0; s < 2; ++s) {
    PACE_KV_TRY(hip_status(hipEventSynchronize(p->copied[s]), "promoter grow"));
    PACE_KV_TRY(hip_status(hipEventSynchronize(p->done[s]), "promoter grow"));
  }
  promoter_free_buffers(p);
  int64_t cap = 1024;
  while (cap < entries) cap *= 2;
  for (int s = 0; s < 2; ++s) {
    PACE_KV_TRY(hip_status(hipHostMalloc(reinterpret_cast<void**>(&p->host[s]), cap * sizeof(int32_t),
                                         hipHostMallocDefault), "promoter pinned ids"));
    PACE_KV_TRY(hip_status(hipMalloc(reinterpret_cast<void**>(&p->dev[s]), cap * sizeof(int32_t)),
                           "promoter device ids"));
  }
  p->capacity = cap;
  return PACE_KV_OK;
}

// Small batches: both id lists travel in the kernel arguments, so no upload
// (and no slot of the promoter) is involved.
int promote_inline(pace_kv_promoter* pr, pace_kv_allocator* dst_alloc,
                   const void* const* src_layers, int64_t src_pool_pages, void* const* dst_layers,
                   int64_t dst_pool_pages, int num_layers, int64_t page_bytes, int num_requests,
                   const int64_t* src_indptr, const int32_t* src_ids, const int32_t* dst_pages,
                   void* buffer, int64_t buffer_layer_stride, int buffer_layers,
                   int32_t* out_dst_tables, int32_t* err_count, const Plan& plan,
                   hipStream_t stream) {
  (void)pr;
  const int64_t n = plan.n_src;
  int32_t dst_ids[PACE_KV_INLINE_IDS];
  PACE_KV_TRY(plan_allocate(dst_alloc, num_requests, src_indptr, dst_pages, plan, out_dst_tables,
                            dst_ids));
  using pace_kv::Side;
  const char* const* src_tab = reinterpret_cast<const char* const*>(src_layers);
  const char* const* dst_tab = reinterpret_cast<const char* const*>(dst_layers);
  int rc = PACE_KV_OK;
  if (n > 0 && num_layers > 0) {
    if (buffer == nullptr) {
      rc = pace_kv::launch_page_copy(Side{src_tab, nullptr, src_pool_pages},
                                     Side{dst_tab, nullptr, dst_pool_pages}, num_layers, n,
                                     page_bytes, err_count, stream, src_ids, dst_ids);
    } else {
      std::vector<const char*> buf(buffer_layers);
      pace_kv::buffer_layers(buffer, buffer_layer_stride, buffer_layers, buf.data());
      for (int l0 = 0; l0 < num_layers && rc == PACE_KV_OK; l0 += buffer_layers) {
        const int nl = num_layers - l0 < buffer_layers ? num_layers - l0 : buffer_layers;
        rc = pace_kv::launch_page_copy(Side{src_tab + l0, nullptr, src_pool_pages},
                                       Side{buf.data(), nullptr, n}, nl, n, page_bytes, err_count,
                                       stream, src_ids, nullptr,
                                       pace_kv::StorePolicy::kPack);
        if (rc == PACE_KV_OK)
          rc = pace_kv::launch_page_copy(Side{buf.data(), nullptr, n},
                                         Side{dst_tab + l0, nullptr, dst_pool_pages}, nl, n,
                                         page_bytes, err_count, stream, nullptr, dst_ids);
      }
    }
  }
  if (rc) {
    // As in pace_kv_promote: pages go back once the copies into them are done.
    (void)hipStreamSynchronize(stream);
    std::lock_guard<std::mutex> lock(dst_alloc->mu);
    unpop_pages(dst_alloc, plan.n_dst_table, out_dst_tables);
  }
  return rc;
}

}  // namespace

extern "C" {

int pace_kv_allocator_create(int64_t num_pages, const int32_t* free_list, int64_t free_len,
                             pace_kv_allocator** out) {
  if (out == nullptr) return fail(PACE_KV_EINVAL, "allocator_create: out is NULL");
  *out = nullptr;
  if (num_pages < 0 || num_pages > INT32_MAX) return fail(PACE_KV_EINVAL, "num_pages outside [0, 2^31)");
  if (free_list == nullptr && free_len != 0) return fail(PACE_KV_EINVAL, "free_list is NULL");
  pace_kv_allocator* a = new pace_kv_allocator();
  a->num_pages = num_pages;
  if (free_list == nullptr) {
    a->free_list.resize(static_cast<size_t>(num_pages));
    for (int64_t i = 0; i < num_pages; ++i) a->free_list[i] = static_cast<int32_t>(i);
  } else {
    int rc = check_page_range(free_list, free_len, num_pages, "free list");
    if (rc) {
      delete a;
      return rc;
    }
    a->free_list.assign(free_list, free_list + free_len);
  }
  *out = a;
  return PACE_KV_OK;
}

int pace_kv_allocator_destroy(pace_kv_allocator* a) {
  delete a;
  return PACE_KV_OK;
}

int pace_kv_allocator_num_free(pace_kv_allocator* a, int64_t* out) {
  if (a == nullptr || out == nullptr) return fail(PACE_KV_EINVAL, "allocator_num_free: NULL argument");
  std::lock_guard<std::mutex> lock(a->mu);
  *out = static_cast<int64_t>(a->free_list.size());
  return PACE_KV_OK;
}

int pace_kv_allocator_allocate(pace_kv_allocator* a, int64_t n, int32_t* out_ids) {
  if (a == nullptr) return fail(PACE_KV_EINVAL, "allocator is NULL");
  if (n < 0) return fail(PACE_KV_EINVAL, "n must be >= 0");
  if (n > 0 && out_ids == nullptr) return fail(PACE_KV_EINVAL, "out_ids is NULL");
  std::lock_guard<std::mutex> lock(a->mu);
  if (n > static_cast<int64_t>(a->free_list.size()))
    return fail(PACE_KV_ENOMEM, "Out of memory! No free blocks are available.");
  pop_pages(a, n, out_ids);
  return PACE_KV_OK;
}

int pace_kv_allocator_free(pace_kv_allocator* a, const int32_t* ids, int64_t n) {
  if (a == nullptr) return fail(PACE_KV_EINVAL, "allocator is NULL");
  if (n < 0) return fail(PACE_KV_EINVAL, "n must be >= 0");
  if (n > 0 && ids == nullptr) return fail(PACE_KV_EINVAL, "ids is NULL");
  PACE_KV_TRY(check_page_range(ids, n, a->num_pages, "free"));
  std::lock_guard<std::mutex> lock(a->mu);
  if (a->stamp.empty()) a->stamp.assign(static_cast<size_t>(a->num_pages), 0u);
  if (++a->generation == 0) {  // stamps wrapped: clear them once
    std::fill(a->stamp.begin(), a->stamp.end(), 0u);
    a->generation = 1;
  }
  for (int64_t i = 0; i < n; ++i) {
    uint32_t& st = a->stamp[ids[i]];
    if (st == a->generation) continue;  // a page repeated within this table
    st = a->generation;
    a->free_list.push_back(ids[i]);
  }
  return PACE_KV_OK;
}

int pace_kv_allocator_snapshot(pace_kv_allocator* a, int32_t* out, int64_t capacity, int64_t* len) {
  if (a == nullptr || len == nullptr) return fail(PACE_KV_EINVAL, "allocator_snapshot: NULL argument");
  std::lock_guard<std::mutex> lock(a->mu);
  const int64_t size = static_cast<int64_t>(a->free_list.size());
  *len = size;
  if (capacity < size) return fail(PACE_KV_ERANGE, "snapshot needs %lld entries", (long long)size);
  if (size > 0) memcpy(out, a->free_list.data(), size * sizeof(int32_t));
  return PACE_KV_OK;
}

int pace_kv_plan(pace_kv_allocator* dst_alloc, int num_requests, const int64_t* src_indptr,
                 const int32_t* src_ids, int64_t src_pool_pages, const int32_t* dst_pages,
                 int32_t* out_dst_tables, int32_t* out_dst_ids) {
  if (dst_alloc == nullptr) return fail(PACE_KV_EINVAL, "plan: allocator is NULL");
  Plan plan;
  PACE_KV_TRY(plan_sizes(num_requests, src_indptr, src_ids, src_pool_pages, dst_pages, &plan));
  if (num_requests == 0 || plan.n_dst_table == 0) return PACE_KV_OK;
  if (out_dst_tables == nullptr || (plan.n_src > 0 && out_dst_ids == nullptr))
    return fail(PACE_KV_EINVAL, "plan: NULL output");
  return plan_allocate(dst_alloc, num_requests, src_indptr, dst_pages, plan, out_dst_tables,
                       out_dst_ids);
}

int pace_kv_promoter_create(pace_kv_promoter** out) {
  if (out == nullptr) return fail(PACE_KV_EINVAL, "promoter_create: out is NULL");
  *out = nullptr;
  pace_kv_promoter* p = new pace_kv_promoter();
  hipError_t e = hipGetDevice(&p->device);
  for (int s = 0; s < 2 && e == hipSuccess; ++s) {
    e = hipEventCreateWithFlags(&p->copied[s], hipEventDisableTiming);
    if (e == hipSuccess) e = hipEventCreateWithFlags(&p->done[s], hipEventDisableTiming);
  }
  if (e != hipSuccess) {
    int rc = hip_status(e, "promoter_create");
    pace_kv_promoter_destroy(p);
    return rc;
  }
  *out = p;
  return PACE_KV_OK;
}

int pace_kv_promoter_destroy(pace_kv_promoter* p) {
  if (p == nullptr) return PACE_KV_OK;
  for (int s = 0; s < 2; ++s) {
    if (p->copied[s]) (void)hipEventSynchronize(p->copied[s]);
    if (p->done[s]) (void)hipEventSynchronize(p->done[s]);
  }
  promoter_free_buffers(p);
  for (int s = 0; s < 2; ++s) {
    if (p->copied[s]) (void)hipEventDestroy(p->copied[s]);
    if (p->done[s]) (void)hipEventDestroy(p->done[s]);
  }
  delete p;
  return PACE_KV_OK;
}

int pace_kv_promote(pace_kv_promoter* pr, pace_kv_allocator* dst_alloc,
                    const void* const* src_layers, int64_t src_pool_pages,
                    void* const* dst_layers, int64_t dst_pool_pages, int num_layers,
                    int64_t page_bytes, int num_requests, const int64_t* src_indptr,
                    const int32_t* src_ids, const int32_t* dst_pages, void* buffer,
                    int64_t buffer_layer_stride, int buffer_layers, int32_t* out_dst_tables,
                    int32_t* err_count, void* stream_) {
  if (pr == nullptr || dst_alloc == nullptr) return fail(PACE_KV_EINVAL, "promote: NULL promoter or allocator");
  int dev = -1;
  PACE_KV_TRY(hip_status(hipGetDevice(&dev), "hipGetDevice"));
  if (dev != pr->device)
    return fail(PACE_KV_ESTATE, "promoter belongs to device %d but device %d is current", pr->device, dev);
  Plan plan;
  PACE_KV_TRY(plan_sizes(num_requests, src_indptr, src_ids, src_pool_pages, dst_pages, &plan));
  if (num_requests == 0 || plan.n_dst_table == 0) return PACE_KV_OK;
  if (out_dst_tables == nullptr) return fail(PACE_KV_EINVAL, "promote: out_dst_tables is NULL");
  if (buffer != nullptr && buffer_layers <= 0)
    return fail(PACE_KV_EINVAL, "promote: buffer_layers must be >= 1 with a buffer");
  const int64_t n = plan.n_src;
  // Argument checks of the copies, before any page is allocated.
  if (num_layers < 0) return fail(PACE_KV_EINVAL, "num_layers must be >= 0");
  if (page_bytes <= 0 || page_bytes % 16 != 0)
    return fail(PACE_KV_EINVAL, "page_bytes must be a positive multiple of 16");
  if (num_layers > 0 && (src_layers == nullptr || dst_layers == nullptr))
    return fail(PACE_KV_EINVAL, "promote: NULL layer table");
  if (buffer != nullptr && (n > INT64_MAX / page_bytes || buffer_layer_stride < n * page_bytes ||
                            buffer_layer_stride % 16 != 0))
    return fail(PACE_KV_ERANGE, "promote: buffer_layer_stride must be >= n_pages*page_bytes and a multiple of 16");
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  if (n <= PACE_KV_INLINE_IDS) return promote_inline(pr, dst_alloc, src_layers, src_pool_pages,
                                                      dst_layers, dst_pool_pages, num_layers,
                                                      page_bytes, num_requests, src_indptr, src_ids,
                                                      dst_pages, buffer, buffer_layer_stride,
                                                      buffer_layers, out_dst_tables, err_count,
                                                      plan, stream);

  PACE_KV_TRY(promoter_reserve(pr, 2 * n));
  const int s = static_cast<int>(pr->calls & 1);
  // host[s] is rewritten below: its previous copy must have left it.
  PACE_KV_TRY(hip_status(hipEventSynchronize(pr->copied[s]), "promoter slot"));
  int32_t* host = pr->host[s];
  memcpy(host, src_ids, n * sizeof(int32_t));
  PACE_KV_TRY(plan_allocate(dst_alloc, num_requests, src_indptr, dst_pages, plan, out_dst_tables,
                            host + n));
  auto rollback = [&](int rc) {
    std::lock_guard<std::mutex> lock(dst_alloc->mu);
    unpop_pages(dst_alloc, plan.n_dst_table, out_dst_tables);
    return rc;
  };
  int32_t* dev_ids = pr->dev[s];
  int rc = hip_status(hipStreamWaitEvent(stream, pr->done[s], 0), "promoter slot wait");
  if (rc == PACE_KV_OK)
    rc = hip_status(hipMemcpyAsync(dev_ids, host, 2 * n * sizeof(int32_t), hipMemcpyHostToDevice, stream),
                    "promoter id upload");
  if (rc == PACE_KV_OK) rc = hip_status(hipEventRecord(pr->copied[s], stream), "promoter record");
  if (rc) return rollback(rc);
  ++pr->calls;
  if (buffer == nullptr) {
    rc = pace_kv_move(src_layers, src_pool_pages, dev_ids, dst_layers, dst_pool_pages, dev_ids + n,
                      num_layers, n, page_bytes, err_count, stream);
  } else {
    for (int l0 = 0; l0 < num_layers && rc == PACE_KV_OK; l0 += buffer_layers) {
      const int nl = num_layers - l0 < buffer_layers ? num_layers - l0 : buffer_layers;
      rc = pace_kv_pack(src_layers + l0, nl, src_pool_pages, dev_ids, n, page_bytes, buffer,
                        buffer_layer_stride, err_count, stream);
      if (rc == PACE_KV_OK)
        rc = pace_kv_unpack(buffer, buffer_layer_stride, dst_layers + l0, nl, dst_pool_pages,
                            dev_ids + n, n, page_bytes, err_count, stream);
    }
  }
  // Record even on failure: the slot's next user waits on this event.
  const int rc2 = hip_status(hipEventRecord(pr->done[s], stream), "promoter record");
  if (rc) {
    // The destination pages go back to the free list only after every copy
    // enqueued into them has finished, so that their next owner, on any
    // stream, cannot see a late partial write.
    (void)hipStreamSynchronize(stream);
    return rollback(rc);
  }
  return rc2;
}

}  // extern "C"
