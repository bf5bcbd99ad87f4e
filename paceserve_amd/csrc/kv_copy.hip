// Paged KV-cache page copies for MI355X (gfx950): pack (gather), unpack
// (scatter) and move (fused gather+scatter), and their C ABI.
//
// Data movement only: no arithmetic, no MFMA.  The kernels are bound by HBM
// bandwidth, so the design goals are (1) every byte read and written exactly
// once, in full 16-byte vectors, fully coalesced per wavefront; (2) many bytes
// in flight per CU: each thread issues all of its loads before its first
// store; (3) no per-page host work: one launch covers every (layer, page)
// pair of a batch of requests, with page ids read from the device block table
// once per workgroup (a uniform, scalar load).
//
// Work decomposition.  A page of one layer is `page_bytes` contiguous bytes
// (K half then V half).  It is split into chunks of kThreads*VPT*16 bytes
// (32 KiB for VPT=8, exactly one K or V half of a Llama-3-8B page).  One
// workgroup (4 wave64) copies one chunk per loop trip; work items are ordered
// layer-major, then page, then chunk, so consecutive workgroups write (pack)
// or read (unpack) consecutive bytes of the contiguous transfer buffer.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <vector>

#include "internal.h"

namespace pace_kv {

namespace {

constexpr int kThreads = 256;
constexpr int kVecBytes = 16;
constexpr int kMaxLayers = PACE_KV_MAX_LAYERS_PER_LAUNCH;
// Upper bound on workgroups per launch; beyond it workgroups loop.
constexpr uint32_t kGridCap = 1u << 20;

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

thread_local char g_last_error[512] = "";

struct CopyParams {
  const char* src[kMaxLayers];
  char* dst[kMaxLayers];
  const int32_t* src_ids;  // nullptr: identity (page j)
  const int32_t* dst_ids;  // nullptr: identity (page j)
  int32_t* err;            // optional skipped-tile counter
  int64_t page_bytes;
  uint32_t src_pool_pages;
  uint32_t dst_pool_pages;
  uint32_t n_pages;
  uint32_t chunks_per_page;
  uint32_t total_items;    // layers * n_pages * chunks_per_page
  uint32_t page_vecs;      // page_bytes / 16
};

__device__ __forceinline__ u32x4 load_stream(const u32x4* p) {
  return __builtin_nontemporal_load(p);
}

__device__ __forceinline__ void store_stream(u32x4* p, u32x4 v) {
  __builtin_nontemporal_store(v, p);
}

// VPT: 16-byte vectors per thread per chunk.  GUARD: the last chunk of a page
// may be partial (page_bytes not a multiple of the chunk size).
template <int VPT, bool GUARD>
__global__ __launch_bounds__(kThreads) void page_copy_kernel(const CopyParams p) {
  constexpr uint32_t kChunkVecs = kThreads * VPT;
  const uint32_t tid = threadIdx.x;
  for (uint32_t item = blockIdx.x; item < p.total_items; item += gridDim.x) {
    const uint32_t page_linear = item / p.chunks_per_page;
    const uint32_t chunk = item - page_linear * p.chunks_per_page;
    const uint32_t layer = page_linear / p.n_pages;
    const uint32_t j = page_linear - layer * p.n_pages;
    const uint32_t sp = p.src_ids ? static_cast<uint32_t>(p.src_ids[j]) : j;
    const uint32_t dp = p.dst_ids ? static_cast<uint32_t>(p.dst_ids[j]) : j;
    // Negative ids wrap to large unsigned values and fail the same test.
    if (sp >= p.src_pool_pages || dp >= p.dst_pool_pages) {
      if (chunk == 0 && tid == 0 && p.err != nullptr) atomicAdd(p.err, 1);
      continue;
    }
    const uint32_t first = chunk * kChunkVecs + tid;
    const u32x4* s = reinterpret_cast<const u32x4*>(
                         p.src[layer] + static_cast<int64_t>(sp) * p.page_bytes) + first;
    u32x4* d = reinterpret_cast<u32x4*>(
                   p.dst[layer] + static_cast<int64_t>(dp) * p.page_bytes) + first;
    u32x4 v[VPT];
#pragma unroll
    for (int u = 0; u < VPT; ++u) {
      if (!GUARD || first + u * kThreads < p.page_vecs) v[u] = load_stream(s + u * kThreads);
    }
#pragma unroll
    for (int u = 0; u < VPT; ++u) {
      if (!GUARD || first + u * kThreads < p.page_vecs) store_stream(d + u * kThreads, v[u]);
    }
  }
}

template <int VPT, bool GUARD>
hipError_t launch(const CopyParams& p, hipStream_t stream) {
  const uint32_t grid = p.total_items < kGridCap ? p.total_items : kGridCap;
  void* args[] = {const_cast<CopyParams*>(&p)};
  return hipLaunchKernel(reinterpret_cast<const void*>(&page_copy_kernel<VPT, GUARD>),
                         dim3(grid), dim3(kThreads), args, 0, stream);
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int check_layers(const char* const* layers, int num_layers, const char* what) {
  if (num_layers > 0 && layers == nullptr) return fail(PACE_KV_EINVAL, "%s: layer table is NULL", what);
  for (int l = 0; l < num_layers; ++l) {
    if (layers[l] == nullptr) return fail(PACE_KV_EINVAL, "%s: layer %d pointer is NULL", what, l);
    if (!aligned16(layers[l]))
      return fail(PACE_KV_EINVAL, "%s: layer %d pointer is not 16-byte aligned", what, l);
  }
  return PACE_KV_OK;
}

}  // namespace

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int hip_status(hipError_t err, const char* what) {
  if (err == hipSuccess) return PACE_KV_OK;
  return fail(static_cast<int>(err), "%s: %s (hipError %d)", what, hipGetErrorString(err),
              static_cast<int>(err));
}

void buffer_layers(const void* base, int64_t layer_stride, int num_layers, const char** out) {
  for (int l = 0; l < num_layers; ++l)
    out[l] = static_cast<const char*>(base) + static_cast<int64_t>(l) * layer_stride;
}

int launch_page_copy(const Side& src, const Side& dst, int num_layers, int64_t n_pages,
                     int64_t page_bytes, int32_t* err_count, hipStream_t stream) {
  if (num_layers < 0) return fail(PACE_KV_EINVAL, "num_layers must be >= 0 (got %d)", num_layers);
  if (n_pages < 0) return fail(PACE_KV_EINVAL, "n_pages must be >= 0 (got %lld)", (long long)n_pages);
  if (page_bytes <= 0 || page_bytes % kVecBytes != 0)
    return fail(PACE_KV_EINVAL, "page_bytes must be a positive multiple of 16 (got %lld)",
                (long long)page_bytes);
  if (page_bytes / kVecBytes > INT32_MAX)
    return fail(PACE_KV_ERANGE, "page_bytes too large (%lld)", (long long)page_bytes);
  if (n_pages > INT32_MAX) return fail(PACE_KV_ERANGE, "n_pages exceeds int32 range");
  if (src.pool_pages < 0 || dst.pool_pages < 0) return fail(PACE_KV_EINVAL, "pool_pages must be >= 0");
  if (num_layers == 0 || n_pages == 0) return PACE_KV_OK;
  if ((src.ids == nullptr && src.pool_pages < n_pages) || (dst.ids == nullptr && dst.pool_pages < n_pages))
    return fail(PACE_KV_ERANGE, "contiguous buffer holds fewer pages than n_pages");
  int rc = check_layers(src.layers, num_layers, "source");
  if (rc) return rc;
  rc = check_layers(dst.layers, num_layers, "destination");
  if (rc) return rc;
  if (src.ids != nullptr && (reinterpret_cast<uintptr_t>(src.ids) & 3u))
    return fail(PACE_KV_EINVAL, "source page ids are not 4-byte aligned");
  if (dst.ids != nullptr && (reinterpret_cast<uintptr_t>(dst.ids) & 3u))
    return fail(PACE_KV_EINVAL, "destination page ids are not 4-byte aligned");

  // Largest chunk (up to 32 KiB per workgroup) that divides the page.
  int vpt = 0;
  for (int v : {8, 4, 2, 1}) {
    if (page_bytes % (int64_t(kThreads) * kVecBytes * v) == 0) { vpt = v; break; }
  }
  const bool guard = vpt == 0;
  if (guard) vpt = 1;
  const int64_t chunk_bytes = int64_t(kThreads) * kVecBytes * vpt;
  const int64_t chunks_per_page = (page_bytes + chunk_bytes - 1) / chunk_bytes;

  const auto clamp_pool = [](int64_t pages) -> uint32_t {
    return pages > INT32_MAX ? static_cast<uint32_t>(INT32_MAX) : static_cast<uint32_t>(pages);
  };

  for (int l0 = 0; l0 < num_layers; l0 += kMaxLayers) {
    const int nl = num_layers - l0 < kMaxLayers ? num_layers - l0 : kMaxLayers;
    // Keep layers * pages * chunks below 2^31 per launch.
    const int64_t max_pages = (int64_t(INT32_MAX) / (int64_t(nl) * chunks_per_page));
    for (int64_t j0 = 0; j0 < n_pages; j0 += max_pages) {
      const int64_t nj = n_pages - j0 < max_pages ? n_pages - j0 : max_pages;
      CopyParams p;
      memset(&p, 0, sizeof(p));
      for (int l = 0; l < nl; ++l) {
        p.src[l] = src.layers[l0 + l] + (src.ids ? 0 : j0 * page_bytes);
        p.dst[l] = const_cast<char*>(dst.layers[l0 + l]) + (dst.ids ? 0 : j0 * page_bytes);
      }
      p.src_ids = src.ids ? src.ids + j0 : nullptr;
      p.dst_ids = dst.ids ? dst.ids + j0 : nullptr;
      p.err = err_count;
      p.page_bytes = page_bytes;
      p.src_pool_pages = src.ids ? clamp_pool(src.pool_pages) : static_cast<uint32_t>(nj);
      p.dst_pool_pages = dst.ids ? clamp_pool(dst.pool_pages) : static_cast<uint32_t>(nj);
      p.n_pages = static_cast<uint32_t>(nj);
      p.chunks_per_page = static_cast<uint32_t>(chunks_per_page);
      p.total_items = static_cast<uint32_t>(int64_t(nl) * nj * chunks_per_page);
      p.page_vecs = static_cast<uint32_t>(page_bytes / kVecBytes);
      hipError_t e;
      if (guard) e = launch<1, true>(p, stream);
      else if (vpt == 8) e = launch<8, false>(p, stream);
      else if (vpt == 4) e = launch<4, false>(p, stream);
      else if (vpt == 2) e = launch<2, false>(p, stream);
      else e = launch<1, false>(p, stream);
      rc = hip_status(e, "page copy launch");
      if (rc) return rc;
    }
  }
  return PACE_KV_OK;
}

}  // namespace pace_kv

using pace_kv::fail;
using pace_kv::Side;

extern "C" {

int pace_kv_abi_version(void) { return PACE_KV_ABI_VERSION; }

const char* pace_kv_last_error(void) { return pace_kv::g_last_error; }

int pace_kv_pack(const void* const* src_layers, int num_layers, int64_t pool_pages,
                 const int32_t* page_ids, int64_t n_pages, int64_t page_bytes, void* out,
                 int64_t out_layer_stride, int32_t* err_count, void* stream) {
  if (num_layers < 0) return fail(PACE_KV_EINVAL, "num_layers must be >= 0");
  if (num_layers == 0 || n_pages == 0) return PACE_KV_OK;
  if (page_ids == nullptr || out == nullptr) return fail(PACE_KV_EINVAL, "pack: NULL page_ids or out");
  if (n_pages > 0 && page_bytes > 0 && out_layer_stride < n_pages * page_bytes)
    return fail(PACE_KV_ERANGE, "pack: out_layer_stride %lld < n_pages*page_bytes",
                (long long)out_layer_stride);
  if (out_layer_stride % 16 != 0) return fail(PACE_KV_EINVAL, "pack: out_layer_stride not a multiple of 16");
  std::vector<const char*> buf(num_layers);
  pace_kv::buffer_layers(out, out_layer_stride, num_layers, buf.data());
  Side src{reinterpret_cast<const char* const*>(src_layers), page_ids, pool_pages};
  Side dst{buf.data(), nullptr, n_pages};
  return pace_kv::launch_page_copy(src, dst, num_layers, n_pages, page_bytes, err_count,
                                   static_cast<hipStream_t>(stream));
}

int pace_kv_unpack(const void* buf, int64_t buf_layer_stride, void* const* dst_layers,
                   int num_layers, int64_t pool_pages, const int32_t* page_ids, int64_t n_pages,
                   int64_t page_bytes, int32_t* err_count, void* stream) {
  if (num_layers < 0) return fail(PACE_KV_EINVAL, "num_layers must be >= 0");
  if (num_layers == 0 || n_pages == 0) return PACE_KV_OK;
  if (page_ids == nullptr || buf == nullptr) return fail(PACE_KV_EINVAL, "unpack: NULL page_ids or buf");
  if (n_pages > 0 && page_bytes > 0 && buf_layer_stride < n_pages * page_bytes)
    return fail(PACE_KV_ERANGE, "unpack: buf_layer_stride %lld < n_pages*page_bytes",
                (long long)buf_layer_stride);
  if (buf_layer_stride % 16 != 0) return fail(PACE_KV_EINVAL, "unpack: buf_layer_stride not a multiple of 16");
  std::vector<const char*> src_tab(num_layers);
  pace_kv::buffer_layers(buf, buf_layer_stride, num_layers, src_tab.data());
  Side src{src_tab.data(), nullptr, n_pages};
  Side dst{reinterpret_cast<const char* const*>(dst_layers), page_ids, pool_pages};
  return pace_kv::launch_page_copy(src, dst, num_layers, n_pages, page_bytes, err_count,
                                   static_cast<hipStream_t>(stream));
}

int pace_kv_move(const void* const* src_layers, int64_t src_pool_pages, const int32_t* src_ids,
                 void* const* dst_layers, int64_t dst_pool_pages, const int32_t* dst_ids,
                 int num_layers, int64_t n_pages, int64_t page_bytes, int32_t* err_count,
                 void* stream) {
  if (num_layers < 0) return fail(PACE_KV_EINVAL, "num_layers must be >= 0");
  if (num_layers == 0 || n_pages == 0) return PACE_KV_OK;
  if (src_ids == nullptr || dst_ids == nullptr) return fail(PACE_KV_EINVAL, "move: NULL page ids");
  Side src{reinterpret_cast<const char* const*>(src_layers), src_ids, src_pool_pages};
  Side dst{reinterpret_cast<const char* const*>(dst_layers), dst_ids, dst_pool_pages};
  return pace_kv::launch_page_copy(src, dst, num_layers, n_pages, page_bytes, err_count,
                                   static_cast<hipStream_t>(stream));
}

}  // extern "C"
