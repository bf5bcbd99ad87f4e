// Shared declarations between the translation units of libpace_kv.so.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "pace_kv.h"

// Returns from the enclosing function with the status of `expr` if non-zero.
#define PACE_KV_TRY(expr)  \
  do {                     \
    int rc_ = (expr);      \
    if (rc_) return rc_;   \
  } while (0)

namespace pace_kv {

// Records `msg` (printf-style) as the calling thread's last error and returns
// `code`, so call sites read `return fail(PACE_KV_EINVAL, "...")`.
int fail(int code, const char* fmt, ...);

// Converts a HIP error into the ABI's status convention (positive hipError_t)
// and records its message; returns 0 for hipSuccess.
int hip_status(hipError_t err, const char* what);

// One side of a page copy: per-layer base pointers plus an optional device
// page-id array (NULL means page j of layer l is at base[l] + j*page_bytes,
// which is how the contiguous transfer buffer is addressed).
struct Side {
  const char* const* layers;  // host array, num_layers entries
  const int32_t* ids;         // device array of n_pages ids, or nullptr
  int64_t pool_pages;         // ids must lie in [0, pool_pages)
};

// Most page ids per side that a launch carries in its kernel arguments.
#define PACE_KV_INLINE_IDS 512

// Store flavour of a copy: both write through the L2 at device scope; kStream
// also marks the stores nontemporal, while kPack (a pack into a transfer
// buffer) leaves them cacheable, so that the unpack reading the rows next
// finds them in the memory-side cache.
enum class StorePolicy { kStream, kPack };

// Validates arguments and enqueues the copy dst[l][dst_id(j)] = src[l][src_id(j)]
// for l < num_layers, j < n_pages on `stream`, in launches of at most
// PACE_KV_MAX_LAYERS_PER_LAUNCH layers.  host_src_ids / host_dst_ids (host
// arrays, n_pages <= PACE_KV_INLINE_IDS) replace the sides' device ids and
// travel in the kernel arguments.

int launch_page_copy(const Side& src, const Side& dst, int num_layers,
                     int64_t n_pages, int64_t page_bytes, int32_t* err_count,
                     hipStream_t stream, const int32_t* host_src_ids = nullptr,
                     const int32_t* host_dst_ids = nullptr,
                     StorePolicy policy = StorePolicy::kStream);

// Builds the layer table of a contiguous buffer [num_layers][layer_stride].
void buffer_layers(const void* base, int64_t layer_stride, int num_layers,
                   const char** out);

}  // namespace pace_kv
