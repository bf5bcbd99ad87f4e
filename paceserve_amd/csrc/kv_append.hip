// Paged KV append (the producer of page contents): writes newly computed K/V
// rows of appended tokens into their page slots, in the layout the migration
// path moves.  Equivalent to the three FlashInfer calls the reference makes per
// layer (paceserve/model_executor/attention/flashinfer_attention_wrapper.py:
// 241-255): get_seq_lens, get_batch_indices_positions, append_paged_kv_cache.
//
//   seq_len[b]   = max(kv_indptr[b+1] - kv_indptr[b] - 1, 0) * P + kv_last_page_len[b]
//                  (computed by the caller: get_seq_lens)
//   token i of request b (append_indptr[b] <= i < append_indptr[b+1]) sits at
//   pos = seq_len[b] - (append_indptr[b+1] - append_indptr[b]) + (i - append_indptr[b])
//   cache[kv_indices[kv_indptr[b] + pos / P]][0 (K) | 1 (V)][pos % P] = key[i] | value[i]
//
// One wave64 workgroup copies one 1 KiB row of one token's K or V (lanes move
// 16-byte vectors, as in the page copy).  Every index is checked: a token whose
// request, page slot or page id is out of range is skipped and counted.
#include "internal.h"

namespace pace_kv {
namespace {

constexpr int kThreads = 64;
constexpr int kVecBytes = 16;
constexpr int kRowBytes = kThreads * kVecBytes;

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

struct AppendParams {
  const char* key;
  const char* value;
  int64_t token_stride;      // bytes between tokens in key / value
  const int32_t* batch_indices;
  const int32_t* positions;
  const int32_t* kv_indices;
  const int32_t* kv_indptr;  // batch_size + 1 entries
  int64_t num_indices;       // entries of kv_indices
  char* cache;               // [num_pages, 2, P, H, D]
  int32_t* err;
  int64_t row_bytes;         // H * D * elem: one token's K (or V) row
  uint32_t batch_size;
  uint32_t num_pages;
  uint32_t page_size;
  uint32_t chunks_per_row;   // ceil(row_bytes / kRowBytes)
  uint32_t total_items;      // nnz * 2 * chunks_per_row
  uint32_t row_vecs;         // row_bytes / 16
};

template <bool GUARD>
__global__ __launch_bounds__(kThreads) void append_kernel(const AppendParams p) {
  const uint32_t item = blockIdx.x;
  if (item >= p.total_items) return;
  const uint32_t per_token = 2 * p.chunks_per_row;
  const uint32_t i = item / per_token;
  const uint32_t rem = item - i * per_token;
  const uint32_t kv = rem / p.chunks_per_row;
  const uint32_t chunk = rem - kv * p.chunks_per_row;
  const uint32_t b = static_cast<uint32_t>(p.batch_indices[i]);
  const int32_t pos = p.positions[i];
  bool ok = b < p.batch_size && pos >= 0;
  uint32_t page = 0;
  if (ok) {
    const int64_t first = p.kv_indptr[b];
    const int64_t last = p.kv_indptr[b + 1];
    const int64_t it = first + pos / static_cast<int32_t>(p.page_size);
    ok = first >= 0 && it < last && it < p.num_indices;
    if (ok) {
      page = static_cast<uint32_t>(p.kv_indices[it]);
      ok = page < p.num_pages;
    }
  }
  if (!ok) {
    if (kv == 0 && chunk == 0 && threadIdx.x == 0 && p.err != nullptr) atomicAdd(p.err, 1);
    return;
  }
  const uint32_t vec = chunk * kThreads + threadIdx.x;
  if (GUARD && vec >= p.row_vecs) return;
  const uint32_t slot = static_cast<uint32_t>(pos) % p.page_size;
  const char* src = (kv ? p.value : p.key) + static_cast<int64_t>(i) * p.token_stride;
  const int64_t page_bytes = 2 * static_cast<int64_t>(p.page_size) * p.row_bytes;
  char* dst = p.cache + static_cast<int64_t>(page) * page_bytes +
              (static_cast<int64_t>(kv) * p.page_size + slot) * p.row_bytes;
  const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src) + vec);
  // A plain nontemporal store: unlike the page copy, the append measured
  // slower with the device-scope write-through store (prefill 16 x 1024
  // tokens 25.3 us against 23.9-24.7 us per launch, decode 2.37 against 2.22).
  __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(dst) + vec);
}

// One thread per appended token: finds its request by binary search over
// append_indptr and derives its position from the request's sequence length.
__global__ __launch_bounds__(256) void positions_kernel(const int32_t* __restrict__ append_indptr,
                                                        const int32_t* __restrict__ seq_lens,
                                                        uint32_t batch_size, uint32_t nnz,
                                                        int32_t* __restrict__ batch_indices,
                                                        int32_t* __restrict__ positions) {
  const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= nnz) return;
  // largest b in [0, batch_size) with append_indptr[b] <= i
  uint32_t lo = 0, hi = batch_size;
  while (hi - lo > 1) {
    const uint32_t mid = lo + (hi - lo) / 2;
    if (append_indptr[mid] <= static_cast<int32_t>(i)) lo = mid; else hi = mid;
  }
  const int32_t a0 = append_indptr[lo], a1 = append_indptr[lo + 1];
  if (static_cast<int32_t>(i) < a0 || static_cast<int32_t>(i) >= a1) {
    batch_indices[i] = -1;   // not covered by any request: the append skips it
    positions[i] = -1;
    return;
  }
  batch_indices[i] = static_cast<int32_t>(lo);
  positions[i] = seq_lens[lo] - (a1 - a0) + (static_cast<int32_t>(i) - a0);
}

}  // namespace
}  // namespace pace_kv

using pace_kv::fail;
using pace_kv::hip_status;

extern "C" {

int pace_kv_append(const void* keys, const void* values, int64_t token_stride_bytes, int64_t nnz,
                   const int32_t* batch_indices, const int32_t* positions, int batch_size,
                   void* cache, int64_t num_pages, const int32_t* kv_indices, int64_t num_indices,
                   const int32_t* kv_indptr, int page_size, int64_t row_bytes, int32_t* err_count,
                   void* stream) {
  using namespace pace_kv;
  if (nnz < 0 || batch_size < 0 || num_pages < 0 || num_indices < 0)
    return fail(PACE_KV_EINVAL, "append: negative size");
  if (nnz == 0) return PACE_KV_OK;
  if (!keys || !values || !batch_indices || !positions || !cache || !kv_indices || !kv_indptr)
    return fail(PACE_KV_EINVAL, "append: NULL argument");
  if (page_size <= 0) return fail(PACE_KV_EINVAL, "append: page_size must be >= 1");
  if (row_bytes <= 0 || row_bytes % kVecBytes != 0)
    return fail(PACE_KV_EINVAL, "append: row bytes (H*D*elem) must be a positive multiple of 16");
  if (token_stride_bytes < row_bytes || token_stride_bytes % kVecBytes != 0)
    return fail(PACE_KV_EINVAL, "append: token stride must be >= row bytes and a multiple of 16");
  if ((reinterpret_cast<uintptr_t>(keys) | reinterpret_cast<uintptr_t>(values) |
       reinterpret_cast<uintptr_t>(cache)) & 15u)
    return fail(PACE_KV_EINVAL, "append: keys, values and cache must be 16-byte aligned");
  if (num_pages > INT32_MAX) return fail(PACE_KV_ERANGE, "append: too many pages");
  const int64_t chunks = (row_bytes + kRowBytes - 1) / kRowBytes;
  if (nnz * 2 * chunks >= (int64_t(1) << 25))
    return fail(PACE_KV_ERANGE, "append: too many tokens for one launch (%lld)", (long long)nnz);
  AppendParams p;
  p.key = static_cast<const char*>(keys);
  p.value = static_cast<const char*>(values);
  p.token_stride = token_stride_bytes;
  p.batch_indices = batch_indices;
  p.positions = positions;
  p.kv_indices = kv_indices;
  p.kv_indptr = kv_indptr;
  p.num_indices = num_indices;
  p.cache = static_cast<char*>(cache);
  p.err = err_count;
  p.row_bytes = row_bytes;
  p.batch_size = static_cast<uint32_t>(batch_size);
  p.num_pages = static_cast<uint32_t>(num_pages);
  p.page_size = static_cast<uint32_t>(page_size);
  p.chunks_per_row = static_cast<uint32_t>(chunks);
  p.total_items = static_cast<uint32_t>(nnz * 2 * chunks);
  p.row_vecs = static_cast<uint32_t>(row_bytes / kVecBytes);
  void* args[] = {&p};
  const bool guard = row_bytes % kRowBytes != 0;
  const void* fn = guard ? reinterpret_cast<const void*>(&append_kernel<true>)
                         : reinterpret_cast<const void*>(&append_kernel<false>);
  return hip_status(hipLaunchKernel(fn, dim3(p.total_items), dim3(kThreads), args, 0,
                                    static_cast<hipStream_t>(stream)),
                    "append launch");
}

int pace_kv_batch_indices_positions(const int32_t* append_indptr, const int32_t* seq_lens,
                                    int batch_size, int64_t nnz, int32_t* batch_indices,
                                    int32_t* positions, void* stream) {
  using namespace pace_kv;
  if (nnz < 0 || batch_size < 0) return fail(PACE_KV_EINVAL, "positions: negative size");
  if (nnz == 0) return PACE_KV_OK;
  if (batch_size == 0) return fail(PACE_KV_EINVAL, "positions: tokens without requests");
  if (!append_indptr || !seq_lens || !batch_indices || !positions)
    return fail(PACE_KV_EINVAL, "positions: NULL argument");
  if (nnz > INT32_MAX) return fail(PACE_KV_ERANGE, "positions: too many tokens");
  uint32_t n = static_cast<uint32_t>(nnz);
  uint32_t bs = static_cast<uint32_t>(batch_size);
  const uint32_t blocks = (n + 255) / 256;
  void* args[] = {const_cast<int32_t**>(&append_indptr), const_cast<int32_t**>(&seq_lens), &bs, &n,
                  &batch_indices, &positions};
  return hip_status(hipLaunchKernel(reinterpret_cast<const void*>(&positions_kernel), dim3(blocks),
                                    dim3(256), args, 0, static_cast<hipStream_t>(stream)),
                    "positions launch");
}

}  // extern "C"
