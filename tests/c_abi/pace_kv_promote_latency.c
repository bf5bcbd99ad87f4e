/*
 * Promote latency seen by a native caller: pace_kv_promote timed from C with
 * no Python in the loop.  One request of n pages (default: 4096 tokens of
 * Llama-3-8B KV, 256 pages of 64 KiB in each of 32 layers) moves from a
 * 2048-page source pool into a fresh 2048-page destination pool on GPU 0:
 * destination allocation and remap, then pack into a transfer buffer and
 * unpack (buffer mode) or one fused pass (fused mode).  Each run is timed from
 * the call to the completion of an event recorded after it on the same
 * stream (CLOCK_MONOTONIC); the destination pages go back to the allocator
 * after each run, in the order that makes the next run allocate the same
 * pages.  After each mode's runs, three layers of every moved page (and, in
 * buffer mode, of the transfer buffer) are checked on the host against the
 * source contents; the destination pool and the buffer are zeroed between
 * the modes, so a mode that wrote nothing cannot pass on the other's bytes.
 *
 * Usage: pace_kv_promote_latency [layers pool_pages n_pages page_bytes runs warmup]
 * Prints one JSON line: p50/p90 microseconds per mode and whether the check
 * passed; exit status 0 when it did.
 *
 * Build (the package build does this): gcc -std=c99 -D__HIP_PLATFORM_AMD__
 *   -I/opt/rocm/include -Iinclude pace_kv_promote_latency.c -Lpaceserve_amd
 *   -lpace_kv -L/opt/rocm/lib -lamdhip64
 */
#define _POSIX_C_SOURCE 200809L
#include <hip/hip_runtime_api.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

#include "pace_kv.h"

#define MAX_LAYERS 128

#define HIP_OK(expr)                                                      \
  do {                                                                    \
    hipError_t e_ = (expr);                                               \
    if (e_ != hipSuccess) {                                               \
      fprintf(stderr, "%s failed: %s\n", #expr, hipGetErrorString(e_));   \
      return 2;                                                           \
    }                                                                     \
  } while (0)

#define PACE_OK(expr)                                                     \
  do {                                                                    \
    int r_ = (expr);                                                      \
    if (r_ != PACE_KV_OK) {                                               \
      fprintf(stderr, "%s failed (%d): %s\n", #expr, r_, pace_kv_last_error()); \
      return 2;                                                           \
    }                                                                     \
  } while (0)

/* The 32-bit word every source page (layer, page) is filled with. */
static uint32_t word_of(int layer, int page) { return 0x5A000000u ^ ((uint32_t)layer << 16) ^ (uint32_t)page; }

static double now_us(void) {
  struct timespec ts;
  clock_gettime(CLOCK_MONOTONIC, &ts);
  return ts.tv_sec * 1e6 + ts.tv_nsec / 1e3;
}

static int cmp_double(const void* a, const void* b) {
  const double x = *(const double*)a, y = *(const double*)b;
  return (x > y) - (x < y);
}

/* Checks that every 32-bit word of the page_bytes at dev equals want. */
static int page_is(const void* dev, int64_t page_bytes, uint32_t want, uint32_t* scratch) {
  if (hipMemcpy(scratch, dev, (size_t)page_bytes, hipMemcpyDeviceToHost) != hipSuccess) return 0;
  for (int64_t i = 0; i < page_bytes / 4; ++i)
    if (scratch[i] != want) return 0;
  return 1;
}

int main(int argc, char** argv) {
  const int layers = argc > 1 ? atoi(argv[1]) : 32;
  const int64_t pool = argc > 2 ? atoll(argv[2]) : 2048;
  const int64_t n = argc > 3 ? atoll(argv[3]) : 256;
  const int64_t page_bytes = argc > 4 ? atoll(argv[4]) : 65536;
  const int runs = argc > 5 ? atoi(argv[5]) : 100;
  const int warmup = argc > 6 ? atoi(argv[6]) : 10;
  if (layers < 1 || layers > MAX_LAYERS || pool < 1 || n < 1 || n > pool || page_bytes < 16 ||
      page_bytes % 16 != 0 || runs < 1 || warmup < 0) {
    fprintf(stderr, "bad arguments\n");
    return 2;
  }
  void* src_layers[MAX_LAYERS];
  void* dst_layers[MAX_LAYERS];
  int32_t* src_ids = malloc((size_t)n * sizeof(int32_t));
  int32_t* perm = malloc((size_t)pool * sizeof(int32_t));
  int32_t* tables = malloc((size_t)n * sizeof(int32_t));
  int32_t* back = malloc((size_t)n * sizeof(int32_t));
  double* lat = malloc((size_t)(runs + warmup) * sizeof(double));
  uint32_t* scratch = malloc((size_t)page_bytes);
  if (!src_ids || !perm || !tables || !back || !lat || !scratch) return 2;

  HIP_OK(hipSetDevice(0));
  hipStream_t stream;
  hipEvent_t done;
  HIP_OK(hipStreamCreate(&stream));
  HIP_OK(hipEventCreateWithFlags(&done, hipEventDisableTiming));

  /* source ids: the first n of a seeded permutation of the pool */
  uint64_t s = 1100;
  for (int64_t i = 0; i < pool; ++i) perm[i] = (int32_t)i;
  for (int64_t i = pool - 1; i > 0; --i) {
    s = s * 6364136223846793005ull + 1442695040888963407ull;
    const int64_t j = (int64_t)((s >> 33) % (uint64_t)(i + 1));
    const int32_t t = perm[i];
    perm[i] = perm[j];
    perm[j] = t;
  }
  memcpy(src_ids, perm, (size_t)n * sizeof(int32_t));
  const int64_t indptr[2] = {0, n};

  for (int l = 0; l < layers; ++l) {
    HIP_OK(hipMalloc(&src_layers[l], (size_t)(pool * page_bytes)));
    HIP_OK(hipMalloc(&dst_layers[l], (size_t)(pool * page_bytes)));
    HIP_OK(hipMemsetD32Async((hipDeviceptr_t)dst_layers[l], 0, (size_t)(pool * page_bytes / 4), stream));
    for (int64_t j = 0; j < n; ++j)
      HIP_OK(hipMemsetD32Async((hipDeviceptr_t)((char*)src_layers[l] + src_ids[j] * page_bytes),
                               (int)word_of(l, src_ids[j]), (size_t)(page_bytes / 4), stream));
  }
  void* buf = NULL;
  HIP_OK(hipMalloc(&buf, (size_t)(layers * n * page_bytes)));
  HIP_OK(hipStreamSynchronize(stream));

  pace_kv_allocator* alloc = NULL;
  pace_kv_promoter* pr = NULL;
  PACE_OK(pace_kv_allocator_create(pool, NULL, 0, &alloc));
  PACE_OK(pace_kv_promoter_create(&pr));

  const char* modes[2] = {"buffer", "fused"};
  double p50[2], p90[2];
  int ok = 1;
  const int check_layers[3] = {0, layers / 2, layers - 1};
  for (int m = 0; m < 2; ++m) {
    void* b = m == 0 ? buf : NULL;
    for (int l = 0; l < layers; ++l)
      HIP_OK(hipMemsetD32Async((hipDeviceptr_t)dst_layers[l], 0, (size_t)(pool * page_bytes / 4), stream));
    HIP_OK(hipMemsetD32Async((hipDeviceptr_t)buf, 0, (size_t)(layers * n * page_bytes / 4), stream));
    HIP_OK(hipStreamSynchronize(stream));
    for (int r = 0; r < warmup + runs; ++r) {
      const double t0 = now_us();
      PACE_OK(pace_kv_promote(pr, alloc, (const void* const*)src_layers, pool, dst_layers, pool, layers,
                              page_bytes, 1, indptr, src_ids, NULL, b, n * page_bytes, layers, tables, NULL,
                              stream));
      HIP_OK(hipEventRecord(done, stream));
      HIP_OK(hipEventSynchronize(done));
      lat[r] = now_us() - t0;
      /* give the pages back so that the next run pops the same ones */
      for (int64_t i = 0; i < n; ++i) back[i] = tables[n - 1 - i];
      PACE_OK(pace_kv_allocator_free(alloc, back, n));
    }
    qsort(lat + warmup, (size_t)runs, sizeof(double), cmp_double);
    p50[m] = runs % 2 ? lat[warmup + runs / 2] : 0.5 * (lat[warmup + runs / 2 - 1] + lat[warmup + runs / 2]);
    p90[m] = lat[warmup + (int)(0.9 * (runs - 1))];
    /* the last run's pages: tables[j] of the destination holds src_ids[j]
     * (and so does page j of the buffer in buffer mode) */
    for (int c = 0; c < 3 && ok; ++c) {
      const int l = check_layers[c];
      for (int64_t j = 0; j < n && ok; ++j) {
        const uint32_t want = word_of(l, src_ids[j]);
        ok = page_is((char*)dst_layers[l] + tables[j] * page_bytes, page_bytes, want, scratch) &&
             (b == NULL || page_is((char*)buf + (l * n + j) * page_bytes, page_bytes, want, scratch));
      }
    }
    if (!ok) fprintf(stderr, "%s mode: a moved page differs from its source\n", modes[m]);
  }

  printf("{\"layers\": %d, \"pool_pages\": %lld, \"n_pages\": %lld, \"page_bytes\": %lld, \"runs\": %d, "
         "\"warmup\": %d", layers, (long long)pool, (long long)n, (long long)page_bytes, runs, warmup);
  for (int m = 0; m < 2; ++m)
    printf(", \"%s\": {\"p50_us\": %.1f, \"p90_us\": %.1f}", modes[m], p50[m], p90[m]);
  printf(", \"verified\": %s}\n", ok ? "true" : "false");

  PACE_OK(pace_kv_promoter_destroy(pr));
  PACE_OK(pace_kv_allocator_destroy(alloc));
  for (int l = 0; l < layers; ++l) {
    HIP_OK(hipFree(src_layers[l]));
    HIP_OK(hipFree(dst_layers[l]));
  }
  HIP_OK(hipFree(buf));
  HIP_OK(hipEventDestroy(done));
  HIP_OK(hipStreamDestroy(stream));
  free(src_ids);
  free(perm);
  free(tables);
  free(back);
  free(lat);
  free(scratch);
  return ok ? 0 : 1;
}
