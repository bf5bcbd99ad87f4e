// Paged KV-cache page copies for MI355X (gfx950): pack (gather), unpack
// (scatter) and move (fused gather+scatter), and their C ABI.
//
// Data movement only: no arithmetic, no MFMA.  The kernels are bound by HBM
// bandwidth, so the design goals are (1) every byte read and written exactly
// once, in full 16-byte vectors, fully coalesced per wavefront; (2) no per-page
// host work: one launch covers every (layer, page) pair of a batch of
// requests, with each page id read from the device block table once per
// wavefront (a uniform load, served from L2 after the first wavefront of the
// page); (3) a compact set of in-flight addresses.
//
// Work decomposition.  A page of one layer is `page_bytes` contiguous bytes
// (K half then V half).  It is split into 1 KiB rows; one workgroup of one
// wave64 copies one row, each lane moving one 16-byte vector with a
// nontemporal load and a write-through store, and then retires.  The grid is
// (rows x pages) x layers: blockIdx.x walks the rows of a layer's pages, row
// fastest, and blockIdx.y is the layer, so workgroups dispatched together read
// (unpack) or write (pack) adjacent rows of the transfer buffer and adjacent
// rows of each pool page.  A wave splits blockIdx.x into page and row with a
// shift when a page has a power-of-two number of rows (every common KV page),
// else with one division.  An unpack wave issues its buffer load before its
// destination page id arrives.  Measured on MI355X, this fine grain keeps
// the chip's in-flight accesses within a narrow address window and copies at
// ~6.6 TB/s, against ~5.6-5.9 TB/s for 8-32 KiB per workgroup, persistent
// grid-stride loops or ids staged in LDS (a persistent loop serialises each
// trip's loads behind the previous trip's stores on the shared vmcnt counter).
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <vector>

#include "internal.h"

namespace pace_kv {

namespace {

constexpr int kThreads = 64;              // one wave64 per workgroup
constexpr int kVecBytes = 16;
constexpr int kRowBytes = kThreads * kVecBytes;  // 1 KiB per workgroup
constexpr int kMaxLayers = PACE_KV_MAX_LAYERS_PER_LAUNCH;
// Workgroups per launch stay below 2^25 so that grid * 64 threads fits the
// 32-bit launch limit with room to spare; larger batches use more launches.
constexpr int64_t kMaxItemsPerLaunch = int64_t(1) << 25;

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
  uint32_t page_vecs;      // page_bytes / 16
  uint32_t rows_per_page;  // ceil(page_bytes / kRowBytes)
  uint32_t rows_log2;      // log2(rows_per_page) when that is a power of two
};

// Page ids carried in the kernel arguments (small promotions): no device id
// array, so no upload has to precede the launch.
struct CopyParamsInline {
  CopyParams base;
  int32_t src_ids[PACE_KV_INLINE_IDS];
  int32_t dst_ids[PACE_KV_INLINE_IDS];
};

__device__ __forceinline__ uint32_t page_of(const int32_t* ids, uint32_t j) {
  return ids ? static_cast<uint32_t>(ids[j]) : j;
}

// Stores carry the device-scope bit (sc1): an XCD's L2 is not coherent with
// the other XCDs', so such a store writes through it to the memory side, and
// the launch leaves no dirty L2 lines to write back when it ends.  A pack
// (PACK) stores with sc1 alone, so the rows also stay in the memory-side cache
// for the unpack that reads them next; every other copy adds nt (streaming).
// Measured on MI355X against plain (launches <= 1 GiB) or nontemporal pack
// stores and nontemporal unpack stores, pack+unpack runs 0.8% (16 GiB of
// 256 KiB pages) to 5.9% (64 MiB) faster, and a fused move 0.5% to 4.2%.
// A store of more than 64 bits reads its data registers after it issues, so
// the next instructions must not overwrite them; the compiler inserts those
// wait states for the stores it emits itself but cannot for one written as
// asm, so the asm carries them (s_nop 1: two wait states).  Without them a
// variant that computed its next address into the stored registers wrote
// wrong data.
template <bool PACK>
__device__ __forceinline__ void store_vec(const u32x4 v, u32x4* d) {
  if (PACK) asm volatile("global_store_dwordx4 %0, %1, off sc1\n\ts_nop 1" : : "v"(d), "v"(v) : "memory");
  else asm volatile("global_store_dwordx4 %0, %1, off nt sc1\n\ts_nop 1" : : "v"(d), "v"(v) : "memory");
}

// The copy of one 1 KiB row: item blockIdx.x (page j, row r of it) of layer
// blockIdx.y; the grid is exactly (rows x pages) x layers.  POW2: the page has
// a power-of-two number of rows.  sids / dids are the sides' page ids (device
// or kernel-argument arrays), nullptr for a contiguous side.  Loads are
// always nontemporal; PACK selects the pack's store policy (store_vec).
template <bool GUARD, bool PACK, bool POW2>
__device__ __forceinline__ void copy_row(const CopyParams& p, const int32_t* sids,
                                         const int32_t* dids) {
  const uint32_t x = blockIdx.x;
  const uint32_t j = POW2 ? x >> p.rows_log2 : x / p.rows_per_page;
  const uint32_t row = POW2 ? x & (p.rows_per_page - 1) : x - j * p.rows_per_page;
  const uint32_t layer = blockIdx.y;
  const uint32_t vec = row * kThreads + threadIdx.x;
  // Lane 0 of row 0 is never guarded out, so a skipped tile is still counted.
  if (GUARD && vec >= p.page_vecs) return;
  if (sids == nullptr) {
    // Contiguous source (unpack): page j of the buffer is always in bounds,
    // so the load is issued before the destination id is known.
    const u32x4 v = __builtin_nontemporal_load(
        reinterpret_cast<const u32x4*>(p.src[layer] + static_cast<int64_t>(j) * p.page_bytes) + vec);
    const uint32_t dp = page_of(dids, j);
    if (dp >= p.dst_pool_pages) {
      if (row == 0 && threadIdx.x == 0 && p.err != nullptr) atomicAdd(p.err, 1);
      return;
    }
    store_vec<PACK>(v, reinterpret_cast<u32x4*>(p.dst[layer] + static_cast<int64_t>(dp) * p.page_bytes) + vec);
    return;
  }
  const uint32_t sp = static_cast<uint32_t>(sids[j]);
  const uint32_t dp = page_of(dids, j);
  // Negative ids wrap to large unsigned values and fail the same test.
  if (sp >= p.src_pool_pages || dp >= p.dst_pool_pages) {
    if (row == 0 && threadIdx.x == 0 && p.err != nullptr) atomicAdd(p.err, 1);
    return;
  }
  const u32x4 v = __builtin_nontemporal_load(
      reinterpret_cast<const u32x4*>(p.src[layer] + static_cast<int64_t>(sp) * p.page_bytes) + vec);
  store_vec<PACK>(v, reinterpret_cast<u32x4*>(p.dst[layer] + static_cast<int64_t>(dp) * p.page_bytes) + vec);
}

// GUARD: page_bytes is not a multiple of kRowBytes, so the last row of a page
// is partial.
template <bool GUARD, bool PACK, bool POW2>
__global__ __launch_bounds__(kThreads) void page_copy_kernel(const CopyParams p) {
  copy_row<GUARD, PACK, POW2>(p, p.src_ids, p.dst_ids);
}

// Same copy with the ids in the kernel arguments.  A side whose ids are not
// inline (the contiguous buffer of a pack or unpack) indexes pages by
// position.
template <bool GUARD, bool PACK, bool POW2, bool SRC_INLINE, bool DST_INLINE>
__global__ __launch_bounds__(kThreads) void page_copy_inline_kernel(const CopyParamsInline p) {
  copy_row<GUARD, PACK, POW2>(p.base, SRC_INLINE ? p.src_ids : nullptr,
                              DST_INLINE ? p.dst_ids : nullptr);
}

template <bool GUARD, bool PACK, bool POW2>
hipError_t launch_t(const CopyParams& p, dim3 grid, hipStream_t stream) {
  void* args[] = {const_cast<CopyParams*>(&p)};
  return hipLaunchKernel(reinterpret_cast<const void*>(&page_copy_kernel<GUARD, PACK, POW2>), grid,
                         dim3(kThreads), args, 0, stream);
}

// Inline ids on both sides (move), the source only (pack) or the destination
// only (unpack).
enum InlineSides { kBothInline = 0, kSrcInline = 1, kDstInline = 2 };

template <bool GUARD, bool PACK, bool POW2, int SIDES>
hipError_t launch_inline_t(const CopyParamsInline& p, dim3 grid, hipStream_t stream) {
  void* args[] = {const_cast<CopyParamsInline*>(&p)};
  constexpr bool kS = SIDES != kDstInline, kD = SIDES != kSrcInline;
  return hipLaunchKernel(
      reinterpret_cast<const void*>(&page_copy_inline_kernel<GUARD, PACK, POW2, kS, kD>), grid,
      dim3(kThreads), args, 0, stream);
}

using LaunchFn = hipError_t (*)(const CopyParams&, dim3, hipStream_t);
using LaunchInlineFn = hipError_t (*)(const CopyParamsInline&, dim3, hipStream_t);

// Instances indexed [GUARD][PACK][POW2] (and [SIDES] for inline ids).
constexpr LaunchFn kLaunch[2][2][2] = {
    {{launch_t<false, false, false>, launch_t<false, false, true>},
     {launch_t<false, true, false>, launch_t<false, true, true>}},
    {{launch_t<true, false, false>, launch_t<true, false, true>},
     {launch_t<true, true, false>, launch_t<true, true, true>}}};

template <bool GUARD, bool PACK, bool POW2>
constexpr LaunchInlineFn kInlineSides[3] = {launch_inline_t<GUARD, PACK, POW2, kBothInline>,
                                            launch_inline_t<GUARD, PACK, POW2, kSrcInline>,
                                            launch_inline_t<GUARD, PACK, POW2, kDstInline>};

LaunchInlineFn launch_inline_fn(bool guard, bool pack, bool pow2, int sides) {
  if (guard) {
    if (pack) return pow2 ? kInlineSides<true, true, true>[sides] : kInlineSides<true, true, false>[sides];
    return pow2 ? kInlineSides<true, false, true>[sides] : kInlineSides<true, false, false>[sides];
  }
  if (pack) return pow2 ? kInlineSides<false, true, true>[sides] : kInlineSides<false, true, false>[sides];
  return pow2 ? kInlineSides<false, false, true>[sides] : kInlineSides<false, false, false>[sides];
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
                     int64_t page_bytes, int32_t* err_count, hipStream_t stream,
                     const int32_t* host_src_ids, const int32_t* host_dst_ids,
                     StorePolicy policy) {
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
  const bool src_indexed = src.ids != nullptr || host_src_ids != nullptr;
  const bool dst_indexed = dst.ids != nullptr || host_dst_ids != nullptr;
  if ((!src_indexed && src.pool_pages < n_pages) || (!dst_indexed && dst.pool_pages < n_pages))
    return fail(PACE_KV_ERANGE, "contiguous buffer holds fewer pages than n_pages");
  int rc = check_layers(src.layers, num_layers, "source");
  if (rc) return rc;
  rc = check_layers(dst.layers, num_layers, "destination");
  if (rc) return rc;
  const bool inline_ids = host_src_ids != nullptr || host_dst_ids != nullptr;
  // The inline kernels index a side without inline ids by position.
  if (inline_ids && ((host_src_ids == nullptr && src.ids != nullptr) ||
                     (host_dst_ids == nullptr && dst.ids != nullptr)))
    return fail(PACE_KV_EINVAL, "a launch cannot mix device and kernel-argument page ids");
  if (inline_ids && n_pages > PACE_KV_INLINE_IDS)
    return fail(PACE_KV_ERANGE, "more than %d pages cannot travel in the kernel arguments",
                PACE_KV_INLINE_IDS);
  if (src.ids != nullptr && (reinterpret_cast<uintptr_t>(src.ids) & 3u))
    return fail(PACE_KV_EINVAL, "source page ids are not 4-byte aligned");
  if (dst.ids != nullptr && (reinterpret_cast<uintptr_t>(dst.ids) & 3u))
    return fail(PACE_KV_EINVAL, "destination page ids are not 4-byte aligned");

  const bool guard = page_bytes % kRowBytes != 0;
  const int64_t rows_per_page = (page_bytes + kRowBytes - 1) / kRowBytes;

  const auto clamp_pool = [](int64_t pages) -> uint32_t {
    return pages > INT32_MAX ? static_cast<uint32_t>(INT32_MAX) : static_cast<uint32_t>(pages);
  };

  uint32_t rows_log2 = 0;
  while ((int64_t(1) << rows_log2) < rows_per_page) ++rows_log2;
  const bool pow2 = (int64_t(1) << rows_log2) == rows_per_page;

  for (int l0 = 0; l0 < num_layers; l0 += kMaxLayers) {
    const int nl = num_layers - l0 < kMaxLayers ? num_layers - l0 : kMaxLayers;
    const int64_t max_pages = kMaxItemsPerLaunch / (int64_t(nl) * rows_per_page);
    if (max_pages < 1)
      return fail(PACE_KV_ERANGE, "page_bytes too large for one launch (%lld)", (long long)page_bytes);
    for (int64_t j0 = 0; j0 < n_pages; j0 += max_pages) {
      const int64_t nj = n_pages - j0 < max_pages ? n_pages - j0 : max_pages;
      CopyParams p;
      memset(&p, 0, sizeof(p));
      for (int l = 0; l < nl; ++l) {
        p.src[l] = src.layers[l0 + l] + (src_indexed ? 0 : j0 * page_bytes);
        p.dst[l] = const_cast<char*>(dst.layers[l0 + l]) + (dst_indexed ? 0 : j0 * page_bytes);
      }
      p.src_ids = src.ids ? src.ids + j0 : nullptr;
      p.dst_ids = dst.ids ? dst.ids + j0 : nullptr;
      p.err = err_count;
      p.page_bytes = page_bytes;
      p.src_pool_pages = src_indexed ? clamp_pool(src.pool_pages) : static_cast<uint32_t>(nj);
      p.dst_pool_pages = dst_indexed ? clamp_pool(dst.pool_pages) : static_cast<uint32_t>(nj);
      p.page_vecs = static_cast<uint32_t>(page_bytes / kVecBytes);
      p.rows_per_page = static_cast<uint32_t>(rows_per_page);
      p.rows_log2 = rows_log2;
      const dim3 grid(static_cast<uint32_t>(rows_per_page * nj), static_cast<uint32_t>(nl));
      const bool pack = policy == StorePolicy::kPack;
      if (inline_ids) {
        CopyParamsInline q;
        q.base = p;
        if (host_src_ids) memcpy(q.src_ids, host_src_ids + j0, nj * sizeof(int32_t));
        if (host_dst_ids) memcpy(q.dst_ids, host_dst_ids + j0, nj * sizeof(int32_t));
        const int sides = host_src_ids && host_dst_ids ? kBothInline : (host_src_ids ? kSrcInline : kDstInline);
        rc = hip_status(launch_inline_fn(guard, pack, pow2, sides)(q, grid, stream), "page copy launch");
      } else {
        rc = hip_status(kLaunch[guard][pack][pow2](p, grid, stream), "page copy launch");
      }
      if (rc) return rc;
    }
  }
  return PACE_KV_OK;
}

// Resolves num_layers host or device layer pointers to the addresses the
// kernel uses, after checking that each lies in a registered allocation of
// the expected kind (pinned host memory mapped for the device, or device
// memory of the current device) that holds pool_bytes from the pointer on.
// Unregistered (pageable) host memory is rejected: the kernel would fault.
int resolve_layers(const void* const* layers, int num_layers, int64_t pool_bytes, bool host,
                   std::vector<const char*>& out, const char* what) {
  if (num_layers > 0 && layers == nullptr) return fail(PACE_KV_EINVAL, "%s: layer table is NULL", what);
  int dev = -1;
  PACE_KV_TRY(hip_status(hipGetDevice(&dev), "hipGetDevice"));
  out.resize(num_layers);
  for (int l = 0; l < num_layers; ++l) {
    const void* p = layers[l];
    hipPointerAttribute_t attr;
    memset(&attr, 0, sizeof(attr));
    hipError_t e = hipPointerGetAttributes(&attr, p);
    const hipMemoryType want = host ? hipMemoryTypeHost : hipMemoryTypeDevice;
    if (e != hipSuccess || attr.type != want || attr.devicePointer == nullptr) {
      (void)hipGetLastError();
      return fail(PACE_KV_EINVAL, "%s: layer %d is not %s memory", what, l,
                  host ? "pinned host (hipHostMalloc)" : "device");
    }
    if (!host && attr.device != dev)
      return fail(PACE_KV_EINVAL, "%s: layer %d lives on device %d, current device is %d", what, l,
                  attr.device, dev);
    // The allocation's range comes from hipMemGetAddressRange: on ROCm 7.2,
    // hipPointerGetAttribute(HIP_POINTER_ATTRIBUTE_RANGE_SIZE) reports the
    // size modulo 2^32 (a 4 GiB allocation reads 0), which would reject a
    // valid pool carved out of a large allocation or accept a short one.
    hipDeviceptr_t start = nullptr;
    size_t size = 0;
    e = hipMemGetAddressRange(&start, &size, const_cast<void*>(p));
    if (e != hipSuccess) {
      (void)hipGetLastError();
      return fail(PACE_KV_EINVAL, "%s: layer %d allocation range unknown", what, l);
    }
    const uintptr_t begin = reinterpret_cast<uintptr_t>(p);
    const uintptr_t lo = reinterpret_cast<uintptr_t>(start);
    if (begin < lo || begin - lo + static_cast<uint64_t>(pool_bytes) > size)
      return fail(PACE_KV_ERANGE, "%s: layer %d allocation holds %zu bytes from its start, "
                  "the pool needs %lld from offset %llu", what, l, size, (long long)pool_bytes,
                  (unsigned long long)(begin - lo));
    out[l] = static_cast<const char*>(attr.devicePointer);
  }
  return PACE_KV_OK;
}

int swap_copy(const void* const* src_layers, int64_t src_pool_pages, const int32_t* src_ids,
              bool src_host, const void* const* dst_layers, int64_t dst_pool_pages,
              const int32_t* dst_ids, bool dst_host, int num_layers, int64_t n_pages,
              int64_t page_bytes, int32_t* err_count, hipStream_t stream, const char* what) {
  if (num_layers < 0 || n_pages < 0) return fail(PACE_KV_EINVAL, "%s: negative size", what);
  if (num_layers == 0 || n_pages == 0) return PACE_KV_OK;
  if (src_ids == nullptr || dst_ids == nullptr) return fail(PACE_KV_EINVAL, "%s: NULL page ids", what);
  if (page_bytes <= 0 || page_bytes % kVecBytes != 0)
    return fail(PACE_KV_EINVAL, "%s: page_bytes must be a positive multiple of 16", what);
  if (src_pool_pages < 0 || dst_pool_pages < 0 || src_pool_pages > INT64_MAX / page_bytes ||
      dst_pool_pages > INT64_MAX / page_bytes)
    return fail(PACE_KV_EINVAL, "%s: bad pool size", what);
  std::vector<const char*> s, d;
  PACE_KV_TRY(resolve_layers(src_layers, num_layers, src_pool_pages * page_bytes, src_host, s, what));
  PACE_KV_TRY(resolve_layers(dst_layers, num_layers, dst_pool_pages * page_bytes, dst_host, d, what));
  Side src{s.data(), src_ids, src_pool_pages};
  Side dst{d.data(), dst_ids, dst_pool_pages};
  return launch_page_copy(src, dst, num_layers, n_pages, page_bytes, err_count, stream);
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
  if (n_pages > 0 && page_bytes > 0 &&
      (n_pages > INT64_MAX / page_bytes || out_layer_stride < n_pages * page_bytes))
    return fail(PACE_KV_ERANGE, "pack: out_layer_stride %lld < n_pages*page_bytes",
                (long long)out_layer_stride);
  if (out_layer_stride % 16 != 0) return fail(PACE_KV_EINVAL, "pack: out_layer_stride not a multiple of 16");
  std::vector<const char*> buf(num_layers);
  pace_kv::buffer_layers(out, out_layer_stride, num_layers, buf.data());
  Side src{reinterpret_cast<const char* const*>(src_layers), page_ids, pool_pages};
  Side dst{buf.data(), nullptr, n_pages};
  return pace_kv::launch_page_copy(src, dst, num_layers, n_pages, page_bytes, err_count,
                                   static_cast<hipStream_t>(stream), nullptr, nullptr,
                                   pace_kv::StorePolicy::kPack);
}

int pace_kv_unpack(const void* buf, int64_t buf_layer_stride, void* const* dst_layers,
                   int num_layers, int64_t pool_pages, const int32_t* page_ids, int64_t n_pages,
                   int64_t page_bytes, int32_t* err_count, void* stream) {
  if (num_layers < 0) return fail(PACE_KV_EINVAL, "num_layers must be >= 0");
  if (num_layers == 0 || n_pages == 0) return PACE_KV_OK;
  if (page_ids == nullptr || buf == nullptr) return fail(PACE_KV_EINVAL, "unpack: NULL page_ids or buf");
  if (n_pages > 0 && page_bytes > 0 &&
      (n_pages > INT64_MAX / page_bytes || buf_layer_stride < n_pages * page_bytes))
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

int pace_kv_swap_out(const void* const* dev_layers, int64_t dev_pool_pages, const int32_t* dev_ids,
                     void* const* host_layers, int64_t host_pool_pages, const int32_t* host_ids,
                     int num_layers, int64_t n_pages, int64_t page_bytes, int32_t* err_count,
                     void* stream) {
  return pace_kv::swap_copy(dev_layers, dev_pool_pages, dev_ids, false,
                            reinterpret_cast<const void* const*>(host_layers), host_pool_pages,
                            host_ids, true, num_layers, n_pages, page_bytes, err_count,
                            static_cast<hipStream_t>(stream), "swap_out");
}

int pace_kv_swap_in(const void* const* host_layers, int64_t host_pool_pages, const int32_t* host_ids,
                    void* const* dev_layers, int64_t dev_pool_pages, const int32_t* dev_ids,
                    int num_layers, int64_t n_pages, int64_t page_bytes, int32_t* err_count,
                    void* stream) {
  return pace_kv::swap_copy(host_layers, host_pool_pages, host_ids, true,
                            reinterpret_cast<const void* const*>(dev_layers), dev_pool_pages,
                            dev_ids, false, num_layers, n_pages, page_bytes, err_count,
                            static_cast<hipStream_t>(stream), "swap_in");
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
