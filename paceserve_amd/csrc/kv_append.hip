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
// pace_kv_append takes b and pos per token (get_batch_indices_positions);
// pace_kv_append_indptr derives them in the same launch from append_indptr,
// kv_indptr and kv_last_page_len, so a layer's append is one launch.
//
// One wave64 workgroup copies one token's K or V row (or a 16 KiB chunk of a
// longer row): every lane loads its vectors of the row, then stores them,
// with the page copy's device-scope write-through store.  Measured on MI355X
// (Llama-3-8B rows of 2 KiB, 16 x 1024 tokens): 20.6 us per launch against
// 23.3-24.5 us for a wave per 1 KiB half row with nontemporal stores, and
// 22.3 us for the half-row waves with these stores; nontemporal
// write-through stores ran at 23.9 us.  Every index is checked: a token whose
// request, page slot or page id is out of range is skipped and counted.
#include "internal.h"

namespace pace_kv {
namespace {

constexpr int kThreads = 64;
constexpr int kVecBytes = 16;
// Longest row one wave carries: 16 vectors of 16 bytes per lane.
constexpr int kMaxVecsPerLane = 16;

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

struct AppendParams {
  const char* key;
  const char* value;
  int64_t token_stride;      // bytes between tokens in key / value
  const int32_t* batch_indices;  // precomputed token -> request (or nullptr: derive from append_indptr)
  const int32_t* positions;
  const int32_t* append_indptr;  // batch_size + 1 entries (the fused form)
  const int32_t* kv_last_page_len;  // batch_size entries (the fused form)
  const int32_t* kv_indices;
  const int32_t* kv_indptr;  // batch_size + 1 entries
  int64_t num_indices;       // entries of kv_indices
  char* cache;               // [num_pages, 2, P, H, D]
  int32_t* err;
  int64_t row_bytes;         // H * D * elem: one token's K (or V) row
  uint32_t batch_size;
  uint32_t num_pages;
  uint32_t page_size;
  uint32_t chunks_per_row;   // ceil(row_vecs / (V * 64))
  uint32_t total_items;      // nnz * 2 * chunks_per_row
  uint32_t row_vecs;         // row_bytes / 16
  uint32_t guess_own_request;  // fused form, nnz <= batch_size: try request i for token i first
};

// A store of more than 64 bits reads its data registers after it issues; the
// asm carries the wait states the compiler cannot add for it (s_nop 1).
__device__ __forceinline__ void store_row_vec(u32x4* d, const u32x4 v) {
  asm volatile("global_store_dwordx4 %0, %1, off sc1\n\ts_nop 1" : : "v"(d), "v"(v) : "memory");
}

// Request of token i in the fused form: the largest b < batch_size with
// append_indptr[b] <= i, found by the whole wave at once: each lane loads
// one entry of each block of 64 (four blocks per round, loaded before any is
// tested, so up to 256 requests cost one load latency), and the entries that
// pass are counted; -1 if none.
__device__ __forceinline__ int32_t request_of(const AppendParams& p, int32_t i) {
  constexpr int kBlocks = 4;
  uint32_t count = 0;
  for (uint32_t base = 0; base < p.batch_size; base += kBlocks * kThreads) {
    int32_t x[kBlocks];
#pragma unroll
    for (int k = 0; k < kBlocks; ++k) {
      const uint32_t e = base + k * kThreads + threadIdx.x;
      x[k] = e < p.batch_size ? p.append_indptr[e] : INT32_MAX;
    }
#pragma unroll
    for (int k = 0; k < kBlocks; ++k) count += __popcll(__ballot(x[k] <= i));
  }
  return static_cast<int32_t>(count) - 1;
}

// Page and slot of token i, or false when any index is out of range.
template <bool FUSED>
__device__ __forceinline__ bool locate(const AppendParams& p, uint32_t i, uint32_t* page, uint32_t* slot) {
  int32_t pos;
  int64_t first, last;
  if (FUSED) {
    const int32_t t = static_cast<int32_t>(i);
    int32_t a0 = 0, a1 = 0, k0 = 0, k1 = 0, len = 0;
    bool found = false;
    if (p.guess_own_request && i < p.batch_size) {
      // A decode batch (no more tokens than requests) usually appends one
      // token per request: guess that token i is request i's and load every
      // index that places it in one round.  The guess holds exactly when
      // append_indptr[i] <= i < append_indptr[i+1], which is when the
      // search below finds request i.
      a0 = p.append_indptr[i];
      a1 = p.append_indptr[i + 1];
      k0 = p.kv_indptr[i];
      k1 = p.kv_indptr[i + 1];
      len = p.kv_last_page_len[i];
      found = a0 <= t && t < a1;
    }
    if (!found) {
      const int32_t b = request_of(p, t);
      if (b < 0) return false;
      // b < batch_size: every offset of request b is loaded in one round,
      // before the range check.
      a0 = p.append_indptr[b];
      a1 = p.append_indptr[b + 1];
      k0 = p.kv_indptr[b];
      k1 = p.kv_indptr[b + 1];
      len = p.kv_last_page_len[b];
      if (t >= a1) return false;
    }
    const int32_t pages = k1 - k0;
    const int32_t seq_len = (pages > 1 ? pages - 1 : 0) * static_cast<int32_t>(p.page_size) + len;
    pos = seq_len - (a1 - a0) + (t - a0);
    first = k0;
    last = k1;
  } else {
    const int32_t b = p.batch_indices[i];
    pos = p.positions[i];
    if (b < 0 || static_cast<uint32_t>(b) >= p.batch_size) return false;
    first = p.kv_indptr[b];
    last = p.kv_indptr[b + 1];
  }
  if (pos < 0) return false;
  const int64_t it = first + pos / static_cast<int32_t>(p.page_size);
  if (first < 0 || it >= last || it >= p.num_indices) return false;
  *page = static_cast<uint32_t>(p.kv_indices[it]);
  if (*page >= p.num_pages) return false;
  *slot = static_cast<uint32_t>(pos) % p.page_size;
  return true;
}

// V: vectors per lane (the row, or its chunk, is V * 64 vectors); GUARD: the
// row is not a multiple of that; MULTI: rows longer than one chunk.
template <int V, bool GUARD, bool MULTI, bool FUSED>
__global__ __launch_bounds__(kThreads) void append_kernel(const AppendParams p) {
  const uint32_t item = blockIdx.x;
  if (item >= p.total_items) return;
  uint32_t i, kv, chunk;
  if (MULTI) {
    const uint32_t per_token = 2 * p.chunks_per_row;
    i = item / per_token;
    const uint32_t rem = item - i * per_token;
    kv = rem / p.chunks_per_row;
    chunk = rem - kv * p.chunks_per_row;
  } else {
    i = item >> 1;
    kv = item & 1;
    chunk = 0;
  }
  // The row's loads depend on the token alone (always in range): they are
  // issued before the index loads that place it, so their latencies overlap.
  const u32x4* src = reinterpret_cast<const u32x4*>((kv ? p.value : p.key) + static_cast<int64_t>(i) * p.token_stride);
  const uint32_t first_vec = chunk * (V * kThreads) + threadIdx.x;
  u32x4 v[V];
#pragma unroll
  for (int c = 0; c < V; ++c) {
    const uint32_t vec = first_vec + c * kThreads;
    if (!GUARD || vec < p.row_vecs) v[c] = __builtin_nontemporal_load(src + vec);
  }
  // Without this barrier the compiler sinks the row loads below the index
  // loads (into the block that stores the row), and the two latencies add up
  // again (measured: 1 us of a 20.8 us prefill launch).
  __builtin_amdgcn_sched_barrier(0);
  uint32_t page = 0, slot = 0;
  if (!locate<FUSED>(p, i, &page, &slot)) {
    if (kv == 0 && chunk == 0 && threadIdx.x == 0 && p.err != nullptr) atomicAdd(p.err, 1);
    return;
  }
  const int64_t page_bytes = 2 * static_cast<int64_t>(p.page_size) * p.row_bytes;
  u32x4* dst = reinterpret_cast<u32x4*>(p.cache + static_cast<int64_t>(page) * page_bytes +
                                        (static_cast<int64_t>(kv) * p.page_size + slot) * p.row_bytes);
#pragma unroll
  for (int c = 0; c < V; ++c) {
    const uint32_t vec = first_vec + c * kThreads;
    if (!GUARD || vec < p.row_vecs) store_row_vec(dst + vec, v[c]);
  }
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

namespace pace_kv {
namespace {

template <int V, bool GUARD, bool MULTI, bool FUSED>
const void* kernel_of() {
  return reinterpret_cast<const void*>(&append_kernel<V, GUARD, MULTI, FUSED>);
}

template <bool FUSED>
const void* pick_kernel(int v, bool guard, bool multi) {
  switch (v) {
    case 1: return guard ? kernel_of<1, true, false, FUSED>() : kernel_of<1, false, false, FUSED>();
    case 2: return guard ? kernel_of<2, true, false, FUSED>() : kernel_of<2, false, false, FUSED>();
    case 4: return guard ? kernel_of<4, true, false, FUSED>() : kernel_of<4, false, false, FUSED>();
    case 8: return guard ? kernel_of<8, true, false, FUSED>() : kernel_of<8, false, false, FUSED>();
    default:
      if (multi) return guard ? kernel_of<16, true, true, FUSED>() : kernel_of<16, false, true, FUSED>();
      return guard ? kernel_of<16, true, false, FUSED>() : kernel_of<16, false, false, FUSED>();
  }
}

// Checks the arguments both forms share, sizes the grid and launches.
int launch_append(AppendParams& p, int64_t nnz, int batch_size, int64_t num_pages, int64_t num_indices,
                  int page_size, int64_t token_stride_bytes, int64_t row_bytes, bool fused, hipStream_t stream) {
  if (nnz < 0 || batch_size < 0 || num_pages < 0 || num_indices < 0)
    return fail(PACE_KV_EINVAL, "append: negative size");
  if (nnz == 0) return PACE_KV_OK;
  if (!p.key || !p.value || !p.cache || !p.kv_indices || !p.kv_indptr)
    return fail(PACE_KV_EINVAL, "append: NULL argument");
  if (page_size <= 0) return fail(PACE_KV_EINVAL, "append: page_size must be >= 1");
  if (row_bytes <= 0 || row_bytes % kVecBytes != 0)
    return fail(PACE_KV_EINVAL, "append: row bytes (H*D*elem) must be a positive multiple of 16");
  if (token_stride_bytes < row_bytes || token_stride_bytes % kVecBytes != 0)
    return fail(PACE_KV_EINVAL, "append: token stride must be >= row bytes and a multiple of 16");
  if ((reinterpret_cast<uintptr_t>(p.key) | reinterpret_cast<uintptr_t>(p.value) |
       reinterpret_cast<uintptr_t>(p.cache)) & 15u)
    return fail(PACE_KV_EINVAL, "append: keys, values and cache must be 16-byte aligned");
  if (num_pages > INT32_MAX) return fail(PACE_KV_ERANGE, "append: too many pages");
  const int64_t row_vecs = row_bytes / kVecBytes;
  const int64_t per_lane = (row_vecs + kThreads - 1) / kThreads;
  int v = 1;
  while (v < per_lane && v < kMaxVecsPerLane) v *= 2;
  const int64_t chunk_vecs = static_cast<int64_t>(v) * kThreads;
  const int64_t chunks = (row_vecs + chunk_vecs - 1) / chunk_vecs;
  if (nnz > INT32_MAX || nnz * 2 * chunks >= (int64_t(1) << 25))
    return fail(PACE_KV_ERANGE, "append: too many tokens for one launch (%lld)", (long long)nnz);
  p.token_stride = token_stride_bytes;
  p.num_indices = num_indices;
  p.row_bytes = row_bytes;
  p.batch_size = static_cast<uint32_t>(batch_size);
  p.num_pages = static_cast<uint32_t>(num_pages);
  p.page_size = static_cast<uint32_t>(page_size);
  p.chunks_per_row = static_cast<uint32_t>(chunks);
  p.total_items = static_cast<uint32_t>(nnz * 2 * chunks);
  p.row_vecs = static_cast<uint32_t>(row_vecs);
  p.guess_own_request = fused && nnz <= batch_size ? 1u : 0u;
  const bool guard = row_vecs % chunk_vecs != 0;
  const void* fn = fused ? pick_kernel<true>(v, guard, chunks > 1) : pick_kernel<false>(v, guard, chunks > 1);
  void* args[] = {&p};
  return hip_status(hipLaunchKernel(fn, dim3(p.total_items), dim3(kThreads), args, 0, stream), "append launch");
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
  if (nnz > 0 && (!batch_indices || !positions)) return fail(PACE_KV_EINVAL, "append: NULL argument");
  pace_kv::AppendParams p = {};
  p.key = static_cast<const char*>(keys);
  p.value = static_cast<const char*>(values);
  p.batch_indices = batch_indices;
  p.positions = positions;
  p.kv_indices = kv_indices;
  p.kv_indptr = kv_indptr;
  p.cache = static_cast<char*>(cache);
  p.err = err_count;
  return pace_kv::launch_append(p, nnz, batch_size, num_pages, num_indices, page_size, token_stride_bytes,
                                row_bytes, false, static_cast<hipStream_t>(stream));
}

int pace_kv_append_indptr(const void* keys, const void* values, int64_t token_stride_bytes, int64_t nnz,
                          const int32_t* append_indptr, int batch_size, void* cache, int64_t num_pages,
                          const int32_t* kv_indices, int64_t num_indices, const int32_t* kv_indptr,
                          const int32_t* kv_last_page_len, int page_size, int64_t row_bytes,
                          int32_t* err_count, void* stream) {
  if (nnz > 0 && batch_size == 0) return fail(PACE_KV_EINVAL, "append: tokens without requests");
  if (nnz > 0 && (!append_indptr || !kv_last_page_len)) return fail(PACE_KV_EINVAL, "append: NULL argument");
  pace_kv::AppendParams p = {};
  p.key = static_cast<const char*>(keys);
  p.value = static_cast<const char*>(values);
  p.append_indptr = append_indptr;
  p.kv_last_page_len = kv_last_page_len;
  p.kv_indices = kv_indices;
  p.kv_indptr = kv_indptr;
  p.cache = static_cast<char*>(cache);
  p.err = err_count;
  return pace_kv::launch_append(p, nnz, batch_size, num_pages, num_indices, page_size, token_stride_bytes,
                                row_bytes, true, static_cast<hipStream_t>(stream));
}

int pace_kv_batch_indices_positions(const int32_t* append_indptr, const int32_t* seq_lens,
                                    int batch_size, int64_t nnz, int32_t* batch_indices,
                                    int32_t* positions, void* stream) {
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
  return hip_status(hipLaunchKernel(reinterpret_cast<const void*>(&pace_kv::positions_kernel), dim3(blocks),
                                    dim3(256), args, 0, static_cast<hipStream_t>(stream)),
                    "positions launch");
}

}  // extern "C"
