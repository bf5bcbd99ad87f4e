/*
 * A C (C99) user of libpace_kv.so through include/pace_kv.h alone: no Python,
 * no torch.  Allocates two 3-layer pools with the HIP runtime, packs four
 * pages of the source pool into a transfer buffer, unpacks them into other
 * pages of the destination pool, and checks every byte on the host against a
 * plain memcpy restatement.  Then sends four pages through a cross-process
 * channel (both endpoints in this process: the message fits the ring) into
 * further destination pages, and checks them the same way.  Then moves the
 * same pages through pinned host memory with a stager (pack to host, unpack
 * from host, round trip), once with one chunk of all layers and once with a
 * chunk per layer, checking the host bytes and both pools.  Then swaps the
 * same pages out to a pinned host pool and back into zeroed destination
 * pages, checking the host pool and the destination.  Then appends three
 * tokens (two requests, one launch with positions derived in the kernel) into
 * the destination's first layer, read as [pages, 2, 16, 128 B rows], and
 * checks every layer against the rows placed by hand, and moves the source
 * pages into zeroed destination pages with the fused move, and packs them to
 * pinned host memory with the allocation-free entry point.  Also checks that
 * an argument error returns PACE_KV_EINVAL with a message.  Exit status 0
 * means every check passed.
 *
 * Build (the package build does this): gcc -std=c99 -D__HIP_PLATFORM_AMD__
 *   -I/opt/rocm/include -Iinclude pace_kv_check.c -Lpaceserve_amd -lpace_kv
 *   -L/opt/rocm/lib -lamdhip64
 */
#define _POSIX_C_SOURCE 200809L
#include <hip/hip_runtime_api.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

#include "pace_kv.h"

#define LAYERS 3
#define POOL_PAGES 16
#define PAGE_BYTES 4096
#define N 4

#define HIP_OK(expr)                                                      \
  do {                                                                    \
    hipError_t e_ = (expr);                                               \
    if (e_ != hipSuccess) {                                               \
      fprintf(stderr, "%s failed: %s\n", #expr, hipGetErrorString(e_));   \
      return 2;                                                           \
    }                                                                     \
  } while (0)

static unsigned char pattern(int pool, int layer, int page, int offset) {
  return (unsigned char)(pool * 101 + layer * 37 + page * 13 + offset * 7 + (offset >> 8));
}

int main(void) {
  const size_t pool_bytes = (size_t)POOL_PAGES * PAGE_BYTES;
  const int32_t src_ids[N] = {5, 0, 11, 3};
  const int32_t dst_ids[N] = {2, 9, 14, 7};
  const int32_t ch_ids[N] = {12, 1, 4, 8};    /* destination pages of the channel message */
  unsigned char* host_src[LAYERS];
  unsigned char* host_dst[LAYERS];
  void* src_layers[LAYERS];
  void* dst_layers[LAYERS];
  void *buf, *ids_src, *ids_dst, *ids_ch;
  unsigned char* host_buf = malloc((size_t)LAYERS * N * PAGE_BYTES);
  unsigned char* got = malloc(pool_bytes);
  int l, j, p, failures = 0;

  if (host_buf == NULL || got == NULL) return 2;
  HIP_OK(hipSetDevice(0));
  for (l = 0; l < LAYERS; ++l) {
    host_src[l] = malloc(pool_bytes);
    host_dst[l] = malloc(pool_bytes);
    if (host_src[l] == NULL || host_dst[l] == NULL) return 2;
    for (p = 0; p < POOL_PAGES; ++p)
      for (j = 0; j < PAGE_BYTES; ++j) {
        host_src[l][(size_t)p * PAGE_BYTES + j] = pattern(0, l, p, j);
        host_dst[l][(size_t)p * PAGE_BYTES + j] = pattern(1, l, p, j);
      }
    HIP_OK(hipMalloc(&src_layers[l], pool_bytes));
    HIP_OK(hipMalloc(&dst_layers[l], pool_bytes));
    HIP_OK(hipMemcpy(src_layers[l], host_src[l], pool_bytes, hipMemcpyHostToDevice));
    HIP_OK(hipMemcpy(dst_layers[l], host_dst[l], pool_bytes, hipMemcpyHostToDevice));
  }
  HIP_OK(hipMalloc(&buf, (size_t)LAYERS * N * PAGE_BYTES));
  HIP_OK(hipMalloc(&ids_src, sizeof(src_ids)));
  HIP_OK(hipMalloc(&ids_dst, sizeof(dst_ids)));
  HIP_OK(hipMalloc(&ids_ch, sizeof(ch_ids)));
  HIP_OK(hipMemcpy(ids_ch, ch_ids, sizeof(ch_ids), hipMemcpyHostToDevice));
  HIP_OK(hipMemcpy(ids_src, src_ids, sizeof(src_ids), hipMemcpyHostToDevice));
  HIP_OK(hipMemcpy(ids_dst, dst_ids, sizeof(dst_ids), hipMemcpyHostToDevice));

  if (pace_kv_abi_version() != PACE_KV_ABI_VERSION) {
    fprintf(stderr, "ABI version %d, header %d\n", pace_kv_abi_version(), PACE_KV_ABI_VERSION);
    return 1;
  }
  /* NULL stream: the device's null stream. */
  int rc = pace_kv_pack((const void* const*)src_layers, LAYERS, POOL_PAGES, (const int32_t*)ids_src, N,
                        PAGE_BYTES, buf, (int64_t)N * PAGE_BYTES, NULL, NULL);
  if (rc == PACE_KV_OK)
    rc = pace_kv_unpack(buf, (int64_t)N * PAGE_BYTES, dst_layers, LAYERS, POOL_PAGES,
                        (const int32_t*)ids_dst, N, PAGE_BYTES, NULL, NULL);
  if (rc != PACE_KV_OK) {
    fprintf(stderr, "pack/unpack status %d: %s\n", rc, pace_kv_last_error());
    return 1;
  }
  HIP_OK(hipDeviceSynchronize());

  /* transfer buffer: buf[l][j] = src[l][src_ids[j]] */
  HIP_OK(hipMemcpy(host_buf, buf, (size_t)LAYERS * N * PAGE_BYTES, hipMemcpyDeviceToHost));
  for (l = 0; l < LAYERS; ++l)
    for (j = 0; j < N; ++j)
      if (memcmp(host_buf + ((size_t)l * N + j) * PAGE_BYTES,
                 host_src[l] + (size_t)src_ids[j] * PAGE_BYTES, PAGE_BYTES) != 0) {
        fprintf(stderr, "buffer layer %d page %d differs\n", l, j);
        ++failures;
      }
  /* destination: named pages receive the source pages, the rest is unchanged */
  for (l = 0; l < LAYERS; ++l) {
    for (j = 0; j < N; ++j)
      memcpy(host_dst[l] + (size_t)dst_ids[j] * PAGE_BYTES, host_src[l] + (size_t)src_ids[j] * PAGE_BYTES,
             PAGE_BYTES);
    HIP_OK(hipMemcpy(got, dst_layers[l], pool_bytes, hipMemcpyDeviceToHost));
    if (memcmp(got, host_dst[l], pool_bytes) != 0) {
      fprintf(stderr, "destination layer %d differs\n", l);
      ++failures;
    }
    HIP_OK(hipMemcpy(got, src_layers[l], pool_bytes, hipMemcpyDeviceToHost));
    if (memcmp(got, host_src[l], pool_bytes) != 0) {
      fprintf(stderr, "source layer %d was written\n", l);
      ++failures;
    }
  }

  /* the same pages through a channel: src[l][src_ids[j]] -> dst[l][ch_ids[j]] */
  {
    char name[64], meta[16];
    pace_kv_channel *rx = NULL, *tx = NULL;
    uint64_t sent = 0, got_id = 0;
    int64_t meta_len = 0, n_pages = 0, page_bytes = 0;
    int num_layers = 0;
    snprintf(name, sizeof(name), "pace_c_check_%d", (int)getpid());
    rc = pace_kv_channel_create(name, 65536, 4, 2, &rx);
    if (rc == PACE_KV_OK) rc = pace_kv_channel_open(name, 2, 1000, &tx);
    if (rc == PACE_KV_OK)
      rc = pace_kv_channel_send(tx, (const void* const*)src_layers, LAYERS, POOL_PAGES, (const int32_t*)ids_src, N,
                                PAGE_BYTES, "four", 4, 1000, &sent, NULL);
    if (rc == PACE_KV_OK)
      rc = pace_kv_channel_recv_header(rx, meta, sizeof(meta), &meta_len, &num_layers, &n_pages, &page_bytes,
                                       &got_id, 1000);
    if (rc == PACE_KV_OK &&
        (meta_len != 4 || memcmp(meta, "four", 4) != 0 || num_layers != LAYERS || n_pages != N ||
         page_bytes != PAGE_BYTES || got_id != sent)) {
      fprintf(stderr, "channel header differs\n");
      ++failures;
    }
    if (rc == PACE_KV_OK)
      rc = pace_kv_channel_recv(rx, dst_layers, LAYERS, POOL_PAGES, (const int32_t*)ids_ch, N, PAGE_BYTES, NULL,
                                1000, NULL);
    if (rc != PACE_KV_OK) {
      fprintf(stderr, "channel status %d: %s\n", rc, pace_kv_last_error());
      return 1;
    }
    HIP_OK(hipDeviceSynchronize());
    pace_kv_channel_close(tx);
    pace_kv_channel_close(rx);
    for (l = 0; l < LAYERS; ++l) {
      for (j = 0; j < N; ++j)
        memcpy(host_dst[l] + (size_t)ch_ids[j] * PAGE_BYTES, host_src[l] + (size_t)src_ids[j] * PAGE_BYTES,
               PAGE_BYTES);
      HIP_OK(hipMemcpy(got, dst_layers[l], pool_bytes, hipMemcpyDeviceToHost));
      if (memcmp(got, host_dst[l], pool_bytes) != 0) {
        fprintf(stderr, "destination layer %d differs after the channel message\n", l);
        ++failures;
      }
    }
  }

  /* through pinned host memory with a stager: pack to host, unpack from host
     into stage pages, round trip into rt pages; one chunk, then a chunk per
     layer, with the target pages zeroed before each pass */
  {
    const int32_t page_sets[2][N] = {{13, 6, 10, 15}, {0, 3, 5, 11}};
    const size_t payload = (size_t)LAYERS * N * PAGE_BYTES;
    const int chunks[2] = {LAYERS, 1};
    pace_kv_stager* st = NULL;
    void *pinned = NULL, *ids_sets[2] = {NULL, NULL};
    int pass, s;
    HIP_OK(hipHostMalloc(&pinned, payload, 0));
    for (s = 0; s < 2; ++s) {
      HIP_OK(hipMalloc(&ids_sets[s], sizeof(page_sets[s])));
      HIP_OK(hipMemcpy(ids_sets[s], page_sets[s], sizeof(page_sets[s]), hipMemcpyHostToDevice));
    }
    rc = pace_kv_stager_create((int64_t)payload, 2, &st);
    for (pass = 0; pass < 2 && rc == PACE_KV_OK; ++pass) {
      const int32_t* stage_ids = page_sets[pass];
      const int32_t* rt_ids = page_sets[1 - pass];
      for (l = 0; l < LAYERS; ++l)
        for (s = 0; s < 2; ++s)
          for (j = 0; j < N; ++j) {
            HIP_OK(hipMemset((char*)dst_layers[l] + (size_t)page_sets[s][j] * PAGE_BYTES, 0, PAGE_BYTES));
            memset(host_dst[l] + (size_t)page_sets[s][j] * PAGE_BYTES, 0, PAGE_BYTES);
          }
      memset(pinned, 0, payload);
      HIP_OK(hipDeviceSynchronize());
      rc = pace_kv_pack_to_host(st, (const void* const*)src_layers, LAYERS, POOL_PAGES, (const int32_t*)ids_src, N,
                                PAGE_BYTES, chunks[pass], pinned, NULL, NULL);
      if (rc == PACE_KV_OK) {
        HIP_OK(hipDeviceSynchronize());
        for (l = 0; l < LAYERS; ++l)
          for (j = 0; j < N; ++j)
            if (memcmp((unsigned char*)pinned + ((size_t)l * N + j) * PAGE_BYTES,
                       host_src[l] + (size_t)src_ids[j] * PAGE_BYTES, PAGE_BYTES) != 0) {
              fprintf(stderr, "pack to host, %d layers per chunk: layer %d page %d differs\n", chunks[pass], l, j);
              ++failures;
            }
        rc = pace_kv_unpack_from_host(st, pinned, dst_layers, LAYERS, POOL_PAGES, (const int32_t*)ids_sets[pass], N,
                                      PAGE_BYTES, chunks[pass], NULL, NULL);
      }
      if (rc == PACE_KV_OK)
        rc = pace_kv_roundtrip(st, (const void* const*)src_layers, POOL_PAGES, (const int32_t*)ids_src, dst_layers,
                               POOL_PAGES, (const int32_t*)ids_sets[1 - pass], LAYERS, N, PAGE_BYTES, chunks[pass],
                               pinned, (int64_t)payload, NULL, NULL);
      if (rc != PACE_KV_OK) break;
      HIP_OK(hipDeviceSynchronize());
      for (l = 0; l < LAYERS; ++l) {
        for (j = 0; j < N; ++j) {
          memcpy(host_dst[l] + (size_t)stage_ids[j] * PAGE_BYTES, host_src[l] + (size_t)src_ids[j] * PAGE_BYTES,
                 PAGE_BYTES);
          memcpy(host_dst[l] + (size_t)rt_ids[j] * PAGE_BYTES, host_src[l] + (size_t)src_ids[j] * PAGE_BYTES,
                 PAGE_BYTES);
        }
        HIP_OK(hipMemcpy(got, dst_layers[l], pool_bytes, hipMemcpyDeviceToHost));
        if (memcmp(got, host_dst[l], pool_bytes) != 0) {
          fprintf(stderr, "destination layer %d differs after staging with %d layers per chunk\n", l, chunks[pass]);
          ++failures;
        }
        HIP_OK(hipMemcpy(got, src_layers[l], pool_bytes, hipMemcpyDeviceToHost));
        if (memcmp(got, host_src[l], pool_bytes) != 0) {
          fprintf(stderr, "source layer %d was written by staging\n", l);
          ++failures;
        }
      }
    }
    if (rc != PACE_KV_OK) {
      fprintf(stderr, "staging status %d: %s\n", rc, pace_kv_last_error());
      return 1;
    }
    rc = pace_kv_stager_destroy(st);
    if (rc != PACE_KV_OK) {
      fprintf(stderr, "stager_destroy status %d: %s\n", rc, pace_kv_last_error());
      return 1;
    }
    HIP_OK(hipHostFree(pinned));
    for (s = 0; s < 2; ++s) HIP_OK(hipFree(ids_sets[s]));
  }

  /* swap out to a pinned host pool (src[l][src_ids[j]] -> host[l][host_ids[j]]),
     then into zeroed destination pages (host[l][host_ids[j]] -> dst[l][in_ids[j]]) */
  {
    const int32_t host_ids[N] = {7, 2, 5, 0};
    const int32_t in_ids[N] = {13, 6, 10, 15};
    const int host_pages = 8;
    const size_t host_pool_bytes = (size_t)host_pages * PAGE_BYTES;
    void* host_layers[LAYERS];
    void *ids_host = NULL, *ids_in = NULL;
    HIP_OK(hipMalloc(&ids_host, sizeof(host_ids)));
    HIP_OK(hipMalloc(&ids_in, sizeof(in_ids)));
    HIP_OK(hipMemcpy(ids_host, host_ids, sizeof(host_ids), hipMemcpyHostToDevice));
    HIP_OK(hipMemcpy(ids_in, in_ids, sizeof(in_ids), hipMemcpyHostToDevice));
    for (l = 0; l < LAYERS; ++l) {
      HIP_OK(hipHostMalloc(&host_layers[l], host_pool_bytes, 0));
      memset(host_layers[l], 0, host_pool_bytes);
      for (j = 0; j < N; ++j) {
        HIP_OK(hipMemset((char*)dst_layers[l] + (size_t)in_ids[j] * PAGE_BYTES, 0, PAGE_BYTES));
        memset(host_dst[l] + (size_t)in_ids[j] * PAGE_BYTES, 0, PAGE_BYTES);
      }
    }
    HIP_OK(hipDeviceSynchronize());
    rc = pace_kv_swap_out((const void* const*)src_layers, POOL_PAGES, (const int32_t*)ids_src, host_layers,
                          host_pages, (const int32_t*)ids_host, LAYERS, N, PAGE_BYTES, NULL, NULL);
    if (rc == PACE_KV_OK) {
      HIP_OK(hipDeviceSynchronize());
      for (l = 0; l < LAYERS; ++l)
        for (p = 0; p < host_pages; ++p) {
          const unsigned char* want = NULL;
          for (j = 0; j < N; ++j)
            if (host_ids[j] == p) want = host_src[l] + (size_t)src_ids[j] * PAGE_BYTES;
          const unsigned char* have = (const unsigned char*)host_layers[l] + (size_t)p * PAGE_BYTES;
          int bad = 0;
          if (want != NULL) {
            bad = memcmp(have, want, PAGE_BYTES) != 0;
          } else {
            for (j = 0; j < PAGE_BYTES && !bad; ++j) bad = have[j] != 0;
          }
          if (bad) {
            fprintf(stderr, "swap out: host layer %d page %d differs\n", l, p);
            ++failures;
          }
        }
      rc = pace_kv_swap_in((const void* const*)host_layers, host_pages, (const int32_t*)ids_host, dst_layers,
                           POOL_PAGES, (const int32_t*)ids_in, LAYERS, N, PAGE_BYTES, NULL, NULL);
    }
    if (rc != PACE_KV_OK) {
      fprintf(stderr, "swap status %d: %s\n", rc, pace_kv_last_error());
      return 1;
    }
    HIP_OK(hipDeviceSynchronize());
    for (l = 0; l < LAYERS; ++l) {
      for (j = 0; j < N; ++j)
        memcpy(host_dst[l] + (size_t)in_ids[j] * PAGE_BYTES, host_src[l] + (size_t)src_ids[j] * PAGE_BYTES,
               PAGE_BYTES);
      HIP_OK(hipMemcpy(got, dst_layers[l], pool_bytes, hipMemcpyDeviceToHost));
      if (memcmp(got, host_dst[l], pool_bytes) != 0) {
        fprintf(stderr, "destination layer %d differs after the swap in\n", l);
        ++failures;
      }
      HIP_OK(hipHostFree(host_layers[l]));
    }
    HIP_OK(hipFree(ids_host));
    HIP_OK(hipFree(ids_in));
  }

  /* paged append into layer 0: request 0 holds pages {2, 9} with 5 tokens in
     the last (21 tokens after its 2 new ones: positions 19, 20 -> page 9 slots
     3, 4); request 1 holds page {14} with 1 token (its new one: page 14 slot 0) */
  {
    enum { P = 16, ROW = PAGE_BYTES / (2 * P), NNZ = 3, BATCH = 2 };
    const int32_t append_indptr[BATCH + 1] = {0, 2, 3};
    const int32_t kv_indptr[BATCH + 1] = {0, 2, 3};
    const int32_t kv_indices[3] = {2, 9, 14};
    const int32_t last_len[BATCH] = {5, 1};
    const int32_t where[NNZ][2] = {{9, 3}, {9, 4}, {14, 0}};   /* page, slot of token i */
    unsigned char keys[NNZ * ROW], values[NNZ * ROW];
    void *d_keys, *d_values, *d_ai, *d_ip, *d_idx, *d_last;
    for (j = 0; j < NNZ * ROW; ++j) {
      keys[j] = (unsigned char)(j * 5 + 1);
      values[j] = (unsigned char)(j * 3 + 200);
    }
    HIP_OK(hipMalloc(&d_keys, sizeof(keys)));
    HIP_OK(hipMalloc(&d_values, sizeof(values)));
    HIP_OK(hipMalloc(&d_ai, sizeof(append_indptr)));
    HIP_OK(hipMalloc(&d_ip, sizeof(kv_indptr)));
    HIP_OK(hipMalloc(&d_idx, sizeof(kv_indices)));
    HIP_OK(hipMalloc(&d_last, sizeof(last_len)));
    HIP_OK(hipMemcpy(d_keys, keys, sizeof(keys), hipMemcpyHostToDevice));
    HIP_OK(hipMemcpy(d_values, values, sizeof(values), hipMemcpyHostToDevice));
    HIP_OK(hipMemcpy(d_ai, append_indptr, sizeof(append_indptr), hipMemcpyHostToDevice));
    HIP_OK(hipMemcpy(d_ip, kv_indptr, sizeof(kv_indptr), hipMemcpyHostToDevice));
    HIP_OK(hipMemcpy(d_idx, kv_indices, sizeof(kv_indices), hipMemcpyHostToDevice));
    HIP_OK(hipMemcpy(d_last, last_len, sizeof(last_len), hipMemcpyHostToDevice));
    rc = pace_kv_append_indptr(d_keys, d_values, ROW, NNZ, (const int32_t*)d_ai, BATCH, dst_layers[0], POOL_PAGES,
                               (const int32_t*)d_idx, 3, (const int32_t*)d_ip, (const int32_t*)d_last, P, ROW,
                               NULL, NULL);
    if (rc != PACE_KV_OK) {
      fprintf(stderr, "append status %d: %s\n", rc, pace_kv_last_error());
      return 1;
    }
    HIP_OK(hipDeviceSynchronize());
    for (j = 0; j < NNZ; ++j) {
      unsigned char* page = host_dst[0] + (size_t)where[j][0] * PAGE_BYTES;
      memcpy(page + (size_t)where[j][1] * ROW, keys + (size_t)j * ROW, ROW);
      memcpy(page + (size_t)(P + where[j][1]) * ROW, values + (size_t)j * ROW, ROW);
    }
    for (l = 0; l < LAYERS; ++l) {
      HIP_OK(hipMemcpy(got, dst_layers[l], pool_bytes, hipMemcpyDeviceToHost));
      if (memcmp(got, host_dst[l], pool_bytes) != 0) {
        fprintf(stderr, "destination layer %d differs after the append\n", l);
        ++failures;
      }
    }
    HIP_OK(hipFree(d_keys));
    HIP_OK(hipFree(d_values));
    HIP_OK(hipFree(d_ai));
    HIP_OK(hipFree(d_ip));
    HIP_OK(hipFree(d_idx));
    HIP_OK(hipFree(d_last));
  }

  /* fused move: src[l][src_ids[j]] -> dst[l][move_ids[j]], no buffer */
  {
    const int32_t move_ids[N] = {0, 3, 5, 11};
    void* ids_move = NULL;
    HIP_OK(hipMalloc(&ids_move, sizeof(move_ids)));
    HIP_OK(hipMemcpy(ids_move, move_ids, sizeof(move_ids), hipMemcpyHostToDevice));
    for (l = 0; l < LAYERS; ++l)
      for (j = 0; j < N; ++j) {
        HIP_OK(hipMemset((char*)dst_layers[l] + (size_t)move_ids[j] * PAGE_BYTES, 0, PAGE_BYTES));
        memset(host_dst[l] + (size_t)move_ids[j] * PAGE_BYTES, 0, PAGE_BYTES);
      }
    HIP_OK(hipDeviceSynchronize());
    rc = pace_kv_move((const void* const*)src_layers, POOL_PAGES, (const int32_t*)ids_src, dst_layers, POOL_PAGES,
                      (const int32_t*)ids_move, LAYERS, N, PAGE_BYTES, NULL, NULL);
    if (rc != PACE_KV_OK) {
      fprintf(stderr, "move status %d: %s\n", rc, pace_kv_last_error());
      return 1;
    }
    HIP_OK(hipDeviceSynchronize());
    for (l = 0; l < LAYERS; ++l) {
      for (j = 0; j < N; ++j)
        memcpy(host_dst[l] + (size_t)move_ids[j] * PAGE_BYTES, host_src[l] + (size_t)src_ids[j] * PAGE_BYTES,
               PAGE_BYTES);
      HIP_OK(hipMemcpy(got, dst_layers[l], pool_bytes, hipMemcpyDeviceToHost));
      if (memcmp(got, host_dst[l], pool_bytes) != 0) {
        fprintf(stderr, "destination layer %d differs after the move\n", l);
        ++failures;
      }
    }
    HIP_OK(hipFree(ids_move));
  }

  /* the allocation-free pack into pinned host memory, twice in a row */
  {
    const size_t payload = (size_t)LAYERS * N * PAGE_BYTES;
    void* out = NULL;
    int rep;
    HIP_OK(hipHostMalloc(&out, payload, 0));
    for (rep = 0; rep < 2; ++rep) {
      memset(out, 0, payload);
      rc = pace_kv_pack_to_host_noalloc((const void* const*)src_layers, LAYERS, POOL_PAGES, (const int32_t*)ids_src, N,
                                        PAGE_BYTES, out, (int64_t)payload, NULL, NULL);
      if (rc != PACE_KV_OK) {
        fprintf(stderr, "pack_to_host_noalloc status %d: %s\n", rc, pace_kv_last_error());
        return 1;
      }
      HIP_OK(hipDeviceSynchronize());
      for (l = 0; l < LAYERS; ++l)
        for (j = 0; j < N; ++j)
          if (memcmp((unsigned char*)out + ((size_t)l * N + j) * PAGE_BYTES,
                     host_src[l] + (size_t)src_ids[j] * PAGE_BYTES, PAGE_BYTES) != 0) {
            fprintf(stderr, "pack_to_host_noalloc call %d: layer %d page %d differs\n", rep, l, j);
            ++failures;
          }
    }
    HIP_OK(hipHostFree(out));
  }

  /* an argument error is caught on the host, before any launch */
  rc = pace_kv_pack((const void* const*)src_layers, LAYERS, POOL_PAGES, (const int32_t*)ids_src, N, 100,
                    buf, (int64_t)N * PAGE_BYTES, NULL, NULL);
  if (rc != PACE_KV_EINVAL || strlen(pace_kv_last_error()) == 0) {
    fprintf(stderr, "page_bytes 100: status %d, message '%s'\n", rc, pace_kv_last_error());
    ++failures;
  }

  for (l = 0; l < LAYERS; ++l) {
    HIP_OK(hipFree(src_layers[l]));
    HIP_OK(hipFree(dst_layers[l]));
    free(host_src[l]);
    free(host_dst[l]);
  }
  HIP_OK(hipFree(buf));
  HIP_OK(hipFree(ids_src));
  HIP_OK(hipFree(ids_dst));
  HIP_OK(hipFree(ids_ch));
  free(host_buf);
  free(got);
  if (failures) return 1;
  printf("pace_kv C ABI check passed: %d layers x %d pages of %d B packed and unpacked, sent through "
         "a channel, staged through pinned host memory, swapped out and in, appended, moved and packed without allocating\n", LAYERS, N, PAGE_BYTES);
  return 0;
}
