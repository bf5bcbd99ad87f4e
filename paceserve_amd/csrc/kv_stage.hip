// Pinned-host staging of packed KV pages: the host leg of a migration.
//
// A migration through host DRAM moves every payload byte over PCIe twice
// (device->host, host->device), at <= ~64 GB/s per direction, i.e. two orders
// of magnitude slower than the on-device pack/unpack.  The pipeline therefore
// aims to keep both DMA directions busy at once and to hide pack/unpack under
// them: layers are processed in chunks, and the round trip uses three streams
//   work stream : unpack(c-S), pack(c+1)   (S = the stager's slots)
//   H2D stream  : H2D(c-1)                 (hipMemcpyAsync: a DMA engine)
//   D2H stream  : D2H(c)                   (a 16-wave copy kernel; see below)
// chunk c's device-to-host copy overlaps chunk c-1's host-to-device copy and
// the kernels of neighbouring chunks.  Events carry every dependency; nothing
// blocks the host.  The work stream waits for the caller's stream at the start
// of a call, and the caller's stream waits for it at the end.
//
// Enqueue order matters as much as the dependencies.  The runtime maps a
// process's streams onto a few hardware queues (4 by default), shared in an
// order that depends on every stream the process has used, and on a shared
// queue a wait or an event record that follows a copy holds back everything
// enqueued behind it until that copy finishes.  Enqueued chunk by chunk
// (pack, D2H, H2D, unpack), the round trip ran at 47-48 GB/s per direction
// with private queues but at 27.5 when the H2D stream shared the caller's
// queue or the D2H stream's, since each pack or D2H copy then waited for the
// previous H2D copy.  Each step therefore enqueues unpack(c-S) and pack(c+1)
// first, then the waits of both copies, both copies, and both completion
// records last, so anything a step enqueues is held back only until the
// previous step's copies finish (measured: 45.6-47.2 GB/s per direction for
// every way the three streams shared queues).  The one-way legs lead in the
// same way: pack(c+1) before D2H(c), H2D(c+1) before unpack(c).
//
// In a torch process the HIP runtime is the one torch ships.  It carried
// hipMemcpyAsync D2H copies as blit kernels whose waves hold the CUs until
// the copy drains, so that packs and unpacks ran only between those copies,
// and switched some of them, by rules of its own, to a DMA engine, where they
// ran one after the other with the H2D copies (12.8 GB/s).  The round trip
// therefore copies device to host with a kernel of its own, sized to leave
// the CUs to the packs and unpacks (copy_to_host_kernel).  Its packs and
// unpacks run on a work stream of the stager's own, which keeps them off
// whatever else the caller's stream carries; measured against the caller's
// stream on stagers kept for the whole run, it was 2% and 6% faster for 2048-
// and 4096-token requests and within 2% either way for 256-1024 and 8192
// tokens.
//
// A call whose layers fit one chunk has nothing to overlap, so all its stages
// run on the caller's stream: each wait between streams adds latency, 30-36 us
// per call on 2-8 MiB requests.  Its device-to-host copy is the copy kernel
// too, which follows a pack on the same stream sooner than a DMA copy does;
// so is the allocation-free pack's.
//
// Device slots are reused round-robin; before a slot is overwritten, the
// stream that writes it waits for the event recorded after the last read of
// that slot, so back-to-back calls on one stager are ordered correctly.
#include <string.h>

#include <mutex>
#include <vector>

#include "internal.h"

using pace_kv::fail;
using pace_kv::hip_status;

// Device staging of pace_kv_pack_to_host_noalloc: one array per GPU, which
// the runtime places when it loads this code object on that GPU and which
// stays until the process ends.  Host code never uses this name as an
// address (on the host it is a stand-in): the device address comes from
// hipGetSymbolAddress, once per device, and is kept in g_scratch.
static __device__ __align__(256) char scratch[PACE_KV_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
char* g_scratch[kMaxDevices];  // device address of `scratch` on each device, once looked up

// The address of the current device's scratch array, looked up on the first
// call on that device.
int current_scratch(char** out) {
  int dev = -1;
  PACE_KV_TRY(hip_status(hipGetDevice(&dev), "hipGetDevice"));
  if (dev < 0 || dev >= kMaxDevices)
    return fail(PACE_KV_ESTATE, "device %d is outside the %d devices the scratch table covers", dev,
                kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch[dev] == nullptr) {
    void* p = nullptr;
    PACE_KV_TRY(hip_status(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)"));
    if (p == nullptr) return fail(PACE_KV_ESTATE, "hipGetSymbolAddress(scratch) returned NULL");
    g_scratch[dev] = static_cast<char*>(p);
  }
  *out = g_scratch[dev];
  return PACE_KV_OK;
}

// host_out of the allocation-free pack: pinned host memory (hipHostMalloc or
// torch's pin_memory) holding `bytes` from host_out on.  With pageable memory
// the runtime would stage each copy through buffers of its own, and the copy
// could not run under graph capture.
int check_pinned_host_out(const void* host_out, int64_t bytes) {
  hipPointerAttribute_t attr;
  memset(&attr, 0, sizeof(attr));
  hipError_t e = hipPointerGetAttributes(&attr, host_out);
  if (e != hipSuccess || attr.type != hipMemoryTypeHost) {
    (void)hipGetLastError();
    return fail(PACE_KV_EINVAL, "pack_to_host_noalloc: host_out is not pinned host memory (hipHostMalloc)");
  }
  hipDeviceptr_t start = nullptr;
  size_t size = 0;
  e = hipMemGetAddressRange(&start, &size, const_cast<void*>(host_out));
  if (e != hipSuccess) {
    (void)hipGetLastError();
    return fail(PACE_KV_EINVAL, "pack_to_host_noalloc: the range of host_out's allocation is unknown");
  }
  const uintptr_t begin = reinterpret_cast<uintptr_t>(host_out);
  const uintptr_t lo = reinterpret_cast<uintptr_t>(start);
  if (begin < lo || begin - lo + static_cast<uint64_t>(bytes) > size)
    return fail(PACE_KV_ERANGE, "pack_to_host_noalloc: host_out's allocation holds %zu bytes from its start, "
                "the payload needs %lld from offset %llu", size, (long long)bytes,
                (unsigned long long)(begin - lo));
  return PACE_KV_OK;
}

}  // namespace

struct pace_kv_stager {
  int device = -1;
  int64_t slot_bytes = 0;
  int num_slots = 0;
  char* out_ring = nullptr;  // num_slots device slots written by pack, read by D2H
  char* in_ring = nullptr;   // num_slots device slots written by H2D, read by unpack
  hipStream_t work = nullptr;  // the round trip's packs and unpacks
  hipStream_t d2h = nullptr;
  hipStream_t h2d = nullptr;
  hipEvent_t work_start = nullptr;  // the caller's stream at the start of a round trip
  hipEvent_t work_done = nullptr;   // everything a round trip enqueued
  hipEvent_t start = nullptr;
  hipEvent_t d2h_done = nullptr;
  hipEvent_t h2d_done = nullptr;  // the last round trip's last H2D copy
  // The kernel stream below is the work stream in a round trip and the
  // caller's stream in the one-way legs.
  std::vector<hipEvent_t> packed;    // out slot s filled (kernel stream)
  std::vector<hipEvent_t> out_free;  // out slot s drained by D2H (D2H stream)
  std::vector<hipEvent_t> in_ready;  // in slot s filled by H2D (H2D stream)
  std::vector<hipEvent_t> in_free;   // in slot s drained by unpack (kernel stream)
  std::vector<hipEvent_t> host_full;  // host region r written by D2H
  std::vector<hipEvent_t> host_free;  // host region r read by H2D
};

namespace {

hipError_t make_events(std::vector<hipEvent_t>& v, size_t n) {
  while (v.size() < n) {
    hipEvent_t e;
    hipError_t err = hipEventCreateWithFlags(&e, hipEventDisableTiming);
    if (err != hipSuccess) return err;
    v.push_back(e);
  }
  return hipSuccess;
}

void destroy_events(std::vector<hipEvent_t>& v) {
  for (hipEvent_t e : v) (void)hipEventDestroy(e);
  v.clear();
}

void release(pace_kv_stager* s) {
  if (s->out_ring) (void)hipFree(s->out_ring);
  if (s->in_ring) (void)hipFree(s->in_ring);
  if (s->work) (void)hipStreamDestroy(s->work);
  if (s->work_start) (void)hipEventDestroy(s->work_start);
  if (s->work_done) (void)hipEventDestroy(s->work_done);
  if (s->d2h) (void)hipStreamDestroy(s->d2h);
  if (s->h2d) (void)hipStreamDestroy(s->h2d);
  if (s->start) (void)hipEventDestroy(s->start);
  if (s->d2h_done) (void)hipEventDestroy(s->d2h_done);
  if (s->h2d_done) (void)hipEventDestroy(s->h2d_done);
  destroy_events(s->packed);
  destroy_events(s->out_free);
  destroy_events(s->in_ready);
  destroy_events(s->in_free);
  destroy_events(s->host_full);
  destroy_events(s->host_free);
  delete s;
}

int check_stager(pace_kv_stager* s) {
  if (s == nullptr) return fail(PACE_KV_EINVAL, "stager is NULL");
  int dev = -1;
  int rc = hip_status(hipGetDevice(&dev), "hipGetDevice");
  if (rc) return rc;
  if (dev != s->device)
    return fail(PACE_KV_ESTATE, "stager belongs to device %d but device %d is current", s->device, dev);
  return PACE_KV_OK;
}

struct ChunkPlan {
  int num_layers;
  int layers_per_chunk;
  int64_t n_pages;
  int64_t page_bytes;
  int64_t layer_bytes;  // n_pages * page_bytes
  int num_chunks() const { return (num_layers + layers_per_chunk - 1) / layers_per_chunk; }
  int first(int c) const { return c * layers_per_chunk; }
  int count(int c) const {
    const int rest = num_layers - first(c);
    return rest < layers_per_chunk ? rest : layers_per_chunk;
  }
};

int make_plan(const pace_kv_stager* s, int num_layers, int64_t n_pages, int64_t page_bytes,
              int layers_per_chunk, ChunkPlan* plan) {
  if (num_layers < 0 || n_pages < 0) return fail(PACE_KV_EINVAL, "negative num_layers or n_pages");
  if (page_bytes <= 0 || page_bytes % 16 != 0)
    return fail(PACE_KV_EINVAL, "page_bytes must be a positive multiple of 16");
  if (layers_per_chunk <= 0) return fail(PACE_KV_EINVAL, "layers_per_chunk must be >= 1");
  if (n_pages > INT64_MAX / page_bytes) return fail(PACE_KV_ERANGE, "payload size overflows");
  plan->num_layers = num_layers;
  plan->layers_per_chunk = layers_per_chunk < num_layers ? layers_per_chunk : (num_layers > 0 ? num_layers : 1);
  plan->n_pages = n_pages;
  plan->page_bytes = page_bytes;
  plan->layer_bytes = n_pages * page_bytes;
  if (plan->layer_bytes > 0 && int64_t(plan->layers_per_chunk) > s->slot_bytes / plan->layer_bytes)
    return fail(PACE_KV_ERANGE,
                "a chunk of %d layers needs %lld bytes but a stager slot holds %lld",
                plan->layers_per_chunk, (long long)(plan->layer_bytes * plan->layers_per_chunk),
                (long long)s->slot_bytes);
  return PACE_KV_OK;
}

#define PACE_HIP(expr, what) PACE_KV_TRY(hip_status((expr), (what)))

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// The round trip's device-to-host copies.  In a torch process the HIP runtime
// carries hipMemcpyAsync from device memory to pinned host memory as a blit
// kernel whose waves fill every CU until the copy drains, or, copy by copy
// and by rules of its own, on a DMA engine, which moved 32 MiB copies at
// 12.8 GB/s beside the round trip's host-to-device copies.  This kernel moves
// a chunk with 16 waves (4 workgroups, each lane keeping 16 vectors in
// flight: 256 KiB per pass), which leaves the other CUs to the packs and
// unpacks and keeps up with the link.  Measured on MI355X against the
// runtime's copy: the same or faster for requests of 32 MiB-1 GiB, 2% slower
// on 4 GiB and 16 GiB round trips in a fresh process, and free of the runtime's
// slow cases.  Stores are write-through at device scope and streaming (the
// swap kernel's host stores); as in the page copy, the asm carries the wait
// states a store of more than 64 bits needs before its data registers are
// overwritten.
constexpr int kHostCopyThreads = 256;
constexpr int kHostCopyGroups = 4;
constexpr int kHostCopyUnroll = 16;

__device__ __forceinline__ void host_store(u32x4* d, const u32x4 v) {
  asm volatile("global_store_dwordx4 %0, %1, off nt sc1\n\ts_nop 1" : : "v"(d), "v"(v) : "memory");
}

__global__ __launch_bounds__(kHostCopyThreads) void copy_to_host_kernel(const u32x4* __restrict__ src,
                                                                        u32x4* __restrict__ dst,
                                                                        uint64_t n_vec) {
  const uint64_t stride = static_cast<uint64_t>(gridDim.x) * kHostCopyThreads;
  uint64_t i = static_cast<uint64_t>(blockIdx.x) * kHostCopyThreads + threadIdx.x;
  for (; i + (kHostCopyUnroll - 1) * stride < n_vec; i += kHostCopyUnroll * stride) {
    u32x4 v[kHostCopyUnroll];
#pragma unroll
    for (int u = 0; u < kHostCopyUnroll; ++u) v[u] = __builtin_nontemporal_load(src + i + u * stride);
#pragma unroll
    for (int u = 0; u < kHostCopyUnroll; ++u) host_store(dst + i + u * stride, v[u]);
  }
  for (; i < n_vec; i += stride) host_store(dst + i, __builtin_nontemporal_load(src + i));
}

// Whether [p, p + bytes) lies in one pinned host allocation that the device
// addresses at the same pointer (hipHostMalloc, torch's pin_memory).
bool device_addressable_host(const void* p, int64_t bytes) {
  hipPointerAttribute_t attr;
  memset(&attr, 0, sizeof(attr));
  if (hipPointerGetAttributes(&attr, p) != hipSuccess || attr.type != hipMemoryTypeHost ||
      attr.devicePointer != p) {
    (void)hipGetLastError();
    return false;
  }
  hipDeviceptr_t start = nullptr;
  size_t size = 0;
  if (hipMemGetAddressRange(&start, &size, const_cast<void*>(p)) != hipSuccess) {
    (void)hipGetLastError();
    return false;
  }
  const uintptr_t begin = reinterpret_cast<uintptr_t>(p);
  const uintptr_t lo = reinterpret_cast<uintptr_t>(start);
  return begin >= lo && begin - lo + static_cast<uint64_t>(bytes) <= size;
}

// One device-to-host copy of the round trip on `stream`: the copy kernel
// when the host side is device-addressable pinned memory (`kernel`) and both
// sides are 16-byte aligned, else hipMemcpyAsync (pageable host memory).
hipError_t copy_to_host(void* host, const void* dev, int64_t bytes, bool kernel, hipStream_t stream) {
  if (!kernel || bytes % 16 != 0 || reinterpret_cast<uintptr_t>(host) % 16 != 0 ||
      reinterpret_cast<uintptr_t>(dev) % 16 != 0)
    return hipMemcpyAsync(host, dev, static_cast<size_t>(bytes), hipMemcpyDeviceToHost, stream);
  copy_to_host_kernel<<<kHostCopyGroups, kHostCopyThreads, 0, stream>>>(
      static_cast<const u32x4*>(dev), static_cast<u32x4*>(host), static_cast<uint64_t>(bytes) / 16);
  return hipGetLastError();
}

// pack(chunk c) of the source pool into out slot `slot`, on `stream`.
int pack_chunk(pace_kv_stager* s, const ChunkPlan& p, int c, const void* const* src_layers,
               int64_t pool_pages, const int32_t* ids, int32_t* err, hipStream_t stream) {
  char* slot = s->out_ring + (c % s->num_slots) * s->slot_bytes;
  return pace_kv_pack(src_layers + p.first(c), p.count(c), pool_pages, ids, p.n_pages,
                      p.page_bytes, slot, p.layer_bytes, err, stream);
}

int unpack_chunk(pace_kv_stager* s, const ChunkPlan& p, int c, void* const* dst_layers,
                 int64_t pool_pages, const int32_t* ids, int32_t* err, hipStream_t stream) {
  const char* slot = s->in_ring + (c % s->num_slots) * s->slot_bytes;
  return pace_kv_unpack(slot, p.layer_bytes, dst_layers + p.first(c), p.count(c), pool_pages, ids,
                        p.n_pages, p.page_bytes, err, stream);
}

// Makes `caller` wait for everything a round trip enqueued: now() on the
// success path (reporting a failure), where the last unpack on the work
// stream already follows every copy; the destructor on an early error return
// (best effort: the call is failing already), where copies may still be in
// flight on the copy streams, so the work stream first waits for those too.
struct WorkJoin {
  pace_kv_stager* s;
  hipStream_t caller;
  bool joined = false;
  int now() {
    joined = true;
    PACE_HIP(hipEventRecord(s->work_done, s->work), "record work_done");
    PACE_HIP(hipStreamWaitEvent(caller, s->work_done, 0), "wait work_done");
    return PACE_KV_OK;
  }
  ~WorkJoin() {
    if (joined) return;
    if (hipEventRecord(s->d2h_done, s->d2h) == hipSuccess) (void)hipStreamWaitEvent(s->work, s->d2h_done, 0);
    if (hipEventRecord(s->h2d_done, s->h2d) == hipSuccess) (void)hipStreamWaitEvent(s->work, s->h2d_done, 0);
    if (hipEventRecord(s->work_done, s->work) == hipSuccess) (void)hipStreamWaitEvent(caller, s->work_done, 0);
  }
};

// Makes `stream` wait for the copies a one-way leg enqueued on its copy
// stream `side` when the leg fails part-way (best effort: the call is failing
// already), so that the caller's stream is ordered after every copy of the
// caller's host buffer.  The success path orders `stream` itself (ok).
struct SideJoin {
  hipStream_t side;
  hipStream_t stream;
  hipEvent_t event;
  bool ok = false;
  ~SideJoin() {
    if (ok) return;
    if (hipEventRecord(event, side) == hipSuccess) (void)hipStreamWaitEvent(stream, event, 0);
  }
};

}  // namespace

extern "C" {

int pace_kv_stager_create(int64_t slot_bytes, int num_slots, pace_kv_stager** out) {
  if (out == nullptr) return fail(PACE_KV_EINVAL, "stager_create: out is NULL");
  *out = nullptr;
  if (slot_bytes <= 0 || slot_bytes % 256 != 0)
    return fail(PACE_KV_EINVAL, "slot_bytes must be a positive multiple of 256");
  if (num_slots < 2 || num_slots > 64) return fail(PACE_KV_EINVAL, "num_slots must be in [2, 64]");
  pace_kv_stager* s = new pace_kv_stager();
  s->slot_bytes = slot_bytes;
  s->num_slots = num_slots;
  hipError_t e = hipGetDevice(&s->device);
  if (e == hipSuccess) e = hipMalloc(reinterpret_cast<void**>(&s->out_ring), slot_bytes * num_slots);
  if (e == hipSuccess) e = hipMalloc(reinterpret_cast<void**>(&s->in_ring), slot_bytes * num_slots);
  if (e == hipSuccess) e = hipStreamCreateWithFlags(&s->work, hipStreamNonBlocking);
  if (e == hipSuccess) e = hipStreamCreateWithFlags(&s->d2h, hipStreamNonBlocking);
  if (e == hipSuccess) e = hipStreamCreateWithFlags(&s->h2d, hipStreamNonBlocking);
  if (e == hipSuccess) e = hipEventCreateWithFlags(&s->work_start, hipEventDisableTiming);
  if (e == hipSuccess) e = hipEventCreateWithFlags(&s->work_done, hipEventDisableTiming);
  if (e == hipSuccess) e = hipEventCreateWithFlags(&s->start, hipEventDisableTiming);
  if (e == hipSuccess) e = hipEventCreateWithFlags(&s->d2h_done, hipEventDisableTiming);
  if (e == hipSuccess) e = hipEventCreateWithFlags(&s->h2d_done, hipEventDisableTiming);
  if (e == hipSuccess) e = make_events(s->packed, num_slots);
  if (e == hipSuccess) e = make_events(s->out_free, num_slots);
  if (e == hipSuccess) e = make_events(s->in_ready, num_slots);
  if (e == hipSuccess) e = make_events(s->in_free, num_slots);
  if (e != hipSuccess) {
    int rc = hip_status(e, "stager_create");
    release(s);
    return rc;
  }
  *out = s;
  return PACE_KV_OK;
}

int pace_kv_stager_destroy(pace_kv_stager* s) {
  if (s == nullptr) return PACE_KV_OK;
  // Work enqueued through the stager may still use its slots and streams.
  (void)hipStreamSynchronize(s->work);
  hipError_t e1 = hipStreamSynchronize(s->d2h);
  hipError_t e2 = hipStreamSynchronize(s->h2d);
  for (hipEvent_t e : s->in_free) (void)hipEventSynchronize(e);
  for (hipEvent_t e : s->packed) (void)hipEventSynchronize(e);
  for (hipEvent_t e : s->out_free) (void)hipEventSynchronize(e);  // one-chunk copies on the caller's stream
  release(s);
  if (e1 != hipSuccess) return hip_status(e1, "stager_destroy (D2H stream)");
  return hip_status(e2, "stager_destroy (H2D stream)");
}

int pace_kv_pack_to_host(pace_kv_stager* s, const void* const* src_layers, int num_layers,
                         int64_t pool_pages, const int32_t* page_ids, int64_t n_pages,
                         int64_t page_bytes, int layers_per_chunk, void* host_out,
                         int32_t* err_count, void* stream_) {
  PACE_KV_TRY(check_stager(s));
  ChunkPlan p;
  PACE_KV_TRY(make_plan(s, num_layers, n_pages, page_bytes, layers_per_chunk, &p));
  if (num_layers == 0 || n_pages == 0) return PACE_KV_OK;
  if (host_out == nullptr) return fail(PACE_KV_EINVAL, "pack_to_host: host_out is NULL");
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  const int chunks = p.num_chunks();
  if (chunks == 1) {
    // One chunk leaves nothing to overlap: the pack and the copy run on
    // `stream`, without the waits between streams (measured on MI355X: 30-36
    // us less per call for 2-8 MiB requests, about 1% less at 128 MiB).  The
    // copy kernel starts sooner after the pack than a DMA copy does (62 against
    // 73 us for 2 MiB, the same from 32 MiB).
    PACE_HIP(hipStreamWaitEvent(stream, s->out_free[0], 0), "wait out slot");
    PACE_KV_TRY(pack_chunk(s, p, 0, src_layers, pool_pages, page_ids, err_count, stream));
    // out_free follows the pack also when the copy fails to enqueue.
    const int64_t bytes = p.count(0) * p.layer_bytes;
    const hipError_t d2h =
        copy_to_host(host_out, s->out_ring, bytes, device_addressable_host(host_out, bytes), stream);
    PACE_HIP(hipEventRecord(s->out_free[0], stream), "record out_free");
    PACE_HIP(d2h, "D2H copy");
    return PACE_KV_OK;
  }
  SideJoin join{s->d2h, stream, s->d2h_done};
  // Step i enqueues pack(i + 1), then the copy of chunk i: the copy's
  // completion record, which holds back whatever follows it when the D2H
  // stream shares the caller's hardware queue, then only delays pack(i + 2).
  // pack(i + 1) refills the slot of chunk i + 1 - num_slots, whose copy was
  // enqueued in an earlier step (num_slots >= 2).
  for (int i = -1; i < chunks; ++i) {
    if (i + 1 < chunks) {
      const int slot = (i + 1) % s->num_slots;
      PACE_HIP(hipStreamWaitEvent(stream, s->out_free[slot], 0), "wait out slot");
      PACE_KV_TRY(pack_chunk(s, p, i + 1, src_layers, pool_pages, page_ids, err_count, stream));
      PACE_HIP(hipEventRecord(s->packed[slot], stream), "record packed");
    }
    if (i >= 0) {
      const int slot = i % s->num_slots;
      PACE_HIP(hipStreamWaitEvent(s->d2h, s->packed[slot], 0), "wait packed");
      PACE_HIP(hipMemcpyAsync(static_cast<char*>(host_out) + p.first(i) * p.layer_bytes,
                              s->out_ring + slot * s->slot_bytes, p.count(i) * p.layer_bytes,
                              hipMemcpyDeviceToHost, s->d2h),
               "D2H copy");
      PACE_HIP(hipEventRecord(s->out_free[slot], s->d2h), "record out_free");
    }
  }
  PACE_HIP(hipEventRecord(s->d2h_done, s->d2h), "record d2h_done");
  PACE_HIP(hipStreamWaitEvent(stream, s->d2h_done, 0), "join D2H");
  join.ok = true;
  return PACE_KV_OK;
}

int pace_kv_unpack_from_host(pace_kv_stager* s, const void* host_in, void* const* dst_layers,
                             int num_layers, int64_t pool_pages, const int32_t* page_ids,
                             int64_t n_pages, int64_t page_bytes, int layers_per_chunk,
                             int32_t* err_count, void* stream_) {
  PACE_KV_TRY(check_stager(s));
  ChunkPlan p;
  PACE_KV_TRY(make_plan(s, num_layers, n_pages, page_bytes, layers_per_chunk, &p));
  if (num_layers == 0 || n_pages == 0) return PACE_KV_OK;
  if (host_in == nullptr) return fail(PACE_KV_EINVAL, "unpack_from_host: host_in is NULL");
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  const int chunks = p.num_chunks();
  if (chunks == 1) {
    // One chunk: the copy and the unpack run on `stream` (as in the pack).
    PACE_HIP(hipStreamWaitEvent(stream, s->in_free[0], 0), "wait in slot");
    PACE_HIP(hipMemcpyAsync(s->in_ring, host_in, p.count(0) * p.layer_bytes, hipMemcpyHostToDevice, stream),
             "H2D copy");
    // in_free follows the copy also when the unpack fails to launch.
    const int rc = unpack_chunk(s, p, 0, dst_layers, pool_pages, page_ids, err_count, stream);
    PACE_HIP(hipEventRecord(s->in_free[0], stream), "record in_free");
    return rc;
  }
  // The caller's earlier work (e.g. writes of host_in by a kernel) comes first.
  PACE_HIP(hipEventRecord(s->start, stream), "record start");
  PACE_HIP(hipStreamWaitEvent(s->h2d, s->start, 0), "wait start");
  // On success the last unpack, on `stream`, follows every copy.
  SideJoin join{s->h2d, stream, s->start};
  // Step i enqueues the copy of chunk i + 1, then unpack(i), whose wait for
  // chunk i's copy then holds back (on a shared hardware queue) only the copy
  // of chunk i + 2.  That copy refills the slot of chunk i + 2 - num_slots,
  // whose unpack was enqueued in an earlier step (num_slots >= 2).
  for (int i = -1; i < chunks; ++i) {
    if (i + 1 < chunks) {
      const int c = i + 1;
      const int slot = c % s->num_slots;
      PACE_HIP(hipStreamWaitEvent(s->h2d, s->in_free[slot], 0), "wait in slot");
      PACE_HIP(hipMemcpyAsync(s->in_ring + slot * s->slot_bytes,
                              static_cast<const char*>(host_in) + p.first(c) * p.layer_bytes,
                              p.count(c) * p.layer_bytes, hipMemcpyHostToDevice, s->h2d),
               "H2D copy");
      PACE_HIP(hipEventRecord(s->in_ready[slot], s->h2d), "record in_ready");
    }
    if (i >= 0) {
      const int slot = i % s->num_slots;
      PACE_HIP(hipStreamWaitEvent(stream, s->in_ready[slot], 0), "wait in_ready");
      PACE_KV_TRY(unpack_chunk(s, p, i, dst_layers, pool_pages, page_ids, err_count, stream));
      PACE_HIP(hipEventRecord(s->in_free[slot], stream), "record in_free");
    }
  }
  join.ok = true;
  return PACE_KV_OK;
}

int pace_kv_roundtrip(pace_kv_stager* s, const void* const* src_layers, int64_t src_pool_pages,
                      const int32_t* src_ids, void* const* dst_layers, int64_t dst_pool_pages,
                      const int32_t* dst_ids, int num_layers, int64_t n_pages, int64_t page_bytes,
                      int layers_per_chunk, void* host_buf, int64_t host_bytes,
                      int32_t* err_count, void* stream_) {
  PACE_KV_TRY(check_stager(s));
  ChunkPlan p;
  PACE_KV_TRY(make_plan(s, num_layers, n_pages, page_bytes, layers_per_chunk, &p));
  if (num_layers == 0 || n_pages == 0) return PACE_KV_OK;
  if (host_buf == nullptr) return fail(PACE_KV_EINVAL, "roundtrip: host_buf is NULL");
  const int64_t chunk_bytes = p.layer_bytes * p.layers_per_chunk;
  if (host_bytes < chunk_bytes)
    return fail(PACE_KV_ERANGE, "roundtrip: host buffer (%lld bytes) is smaller than one chunk (%lld)",
                (long long)host_bytes, (long long)chunk_bytes);
  const int chunks = p.num_chunks();
  int64_t regions64 = host_bytes / chunk_bytes;
  const int regions = regions64 < chunks ? static_cast<int>(regions64) : chunks;
  PACE_HIP(make_events(s->host_full, regions), "create host events");
  PACE_HIP(make_events(s->host_free, regions), "create host events");
  char* host = static_cast<char*>(host_buf);
  const bool host_kernel = device_addressable_host(host_buf, regions * chunk_bytes);
  if (chunks == 1) {
    // One chunk leaves nothing to overlap: its four stages run on the
    // caller's stream, without the waits between streams.  They follow the
    // packs and unpacks of earlier calls on this stager (work_done), the last
    // reads of both slots and the previous call's last read of its host
    // buffer, and leave the records a later call waits on.
    hipStream_t caller = static_cast<hipStream_t>(stream_);
    const int64_t bytes = p.count(0) * p.layer_bytes;
    PACE_HIP(hipStreamWaitEvent(caller, s->work_done, 0), "wait earlier calls");
    PACE_HIP(hipStreamWaitEvent(caller, s->out_free[0], 0), "wait out slot");
    PACE_HIP(hipStreamWaitEvent(caller, s->h2d_done, 0), "wait previous round trip");
    PACE_KV_TRY(pack_chunk(s, p, 0, src_layers, src_pool_pages, src_ids, err_count, caller));
    // out_free follows the pack also when the copy fails to enqueue.
    const hipError_t d2h = copy_to_host(host, s->out_ring, bytes, host_kernel, caller);
    PACE_HIP(hipEventRecord(s->out_free[0], caller), "record out_free");
    PACE_HIP(d2h, "D2H copy");
    PACE_HIP(hipStreamWaitEvent(caller, s->in_free[0], 0), "wait in slot");
    PACE_HIP(hipMemcpyAsync(s->in_ring, host, bytes, hipMemcpyHostToDevice, caller), "H2D copy");
    PACE_HIP(hipEventRecord(s->h2d_done, caller), "record h2d_done");
    // The records follow the H2D copy also when the unpack fails to launch.
    const int rc = unpack_chunk(s, p, 0, dst_layers, dst_pool_pages, dst_ids, err_count, caller);
    PACE_HIP(hipEventRecord(s->in_free[0], caller), "record in_free");
    PACE_HIP(hipEventRecord(s->work_done, caller), "record work_done");
    return rc;
  }
  // Packs and unpacks run on the stager's work stream, created together with
  // its two copy streams (see the file comment); the work stream starts after
  // the caller's earlier work, and the caller's stream waits for everything
  // the call enqueued on it, on every return path.
  hipStream_t caller = static_cast<hipStream_t>(stream_);
  hipStream_t stream = s->work;
  WorkJoin join{s, caller};
  PACE_HIP(hipEventRecord(s->work_start, caller), "record work_start");
  PACE_HIP(hipStreamWaitEvent(stream, s->work_start, 0), "wait work_start");
  const int S = s->num_slots;
  // A region's events order its reuse within a call and between calls of one
  // chunk size; a call with another chunk size (or host buffer) carves other
  // regions, so its first D2H copy waits for the previous call's last H2D
  // copy to have read the host buffer.
  PACE_HIP(hipStreamWaitEvent(s->d2h, s->h2d_done, 0), "wait previous round trip");
  // The stages of chunk c; each wait names an event whose record for the
  // chunk it must follow is the latest one enqueued when the wait is.
  auto pack = [&](int c) -> int {
    const int slot = c % S;
    PACE_HIP(hipStreamWaitEvent(stream, s->out_free[slot], 0), "wait out slot");
    PACE_KV_TRY(pack_chunk(s, p, c, src_layers, src_pool_pages, src_ids, err_count, stream));
    PACE_HIP(hipEventRecord(s->packed[slot], stream), "record packed");
    return PACE_KV_OK;
  };
  auto d2h_wait = [&](int c) -> int {
    PACE_HIP(hipStreamWaitEvent(s->d2h, s->packed[c % S], 0), "wait packed");
    PACE_HIP(hipStreamWaitEvent(s->d2h, s->host_free[c % regions], 0), "wait host region");
    return PACE_KV_OK;
  };
  auto d2h_copy = [&](int c) -> int {
    PACE_HIP(copy_to_host(host + static_cast<int64_t>(c % regions) * chunk_bytes,
                          s->out_ring + (c % S) * s->slot_bytes, p.count(c) * p.layer_bytes, host_kernel,
                          s->d2h),
             "D2H copy");
    return PACE_KV_OK;
  };
  auto d2h_record = [&](int c) -> int {
    PACE_HIP(hipEventRecord(s->out_free[c % S], s->d2h), "record out_free");
    PACE_HIP(hipEventRecord(s->host_full[c % regions], s->d2h), "record host_full");
    return PACE_KV_OK;
  };
  auto h2d_wait = [&](int c) -> int {
    PACE_HIP(hipStreamWaitEvent(s->h2d, s->host_full[c % regions], 0), "wait host_full");
    PACE_HIP(hipStreamWaitEvent(s->h2d, s->in_free[c % S], 0), "wait in slot");
    return PACE_KV_OK;
  };
  auto h2d_copy = [&](int c) -> int {
    PACE_HIP(hipMemcpyAsync(s->in_ring + (c % S) * s->slot_bytes,
                            host + static_cast<int64_t>(c % regions) * chunk_bytes,
                            p.count(c) * p.layer_bytes, hipMemcpyHostToDevice, s->h2d),
             "H2D copy");
    return PACE_KV_OK;
  };
  auto h2d_record = [&](int c) -> int {
    PACE_HIP(hipEventRecord(s->in_ready[c % S], s->h2d), "record in_ready");
    PACE_HIP(hipEventRecord(s->host_free[c % regions], s->h2d), "record host_free");
    return PACE_KV_OK;
  };
  auto unpack = [&](int c) -> int {
    const int slot = c % S;
    PACE_HIP(hipStreamWaitEvent(stream, s->in_ready[slot], 0), "wait in_ready");
    PACE_KV_TRY(unpack_chunk(s, p, c, dst_layers, dst_pool_pages, dst_ids, err_count, stream));
    PACE_HIP(hipEventRecord(s->in_free[slot], stream), "record in_free");
    return PACE_KV_OK;
  };
  if (regions == 1) {
    // One host region: each chunk's D2H copy must wait for the previous
    // chunk's H2D copy to leave the region, so the stages run one chunk at
    // a time.
    for (int c = 0; c < chunks; ++c) {
      PACE_KV_TRY(pack(c));
      PACE_KV_TRY(d2h_wait(c));
      PACE_KV_TRY(d2h_copy(c));
      PACE_KV_TRY(d2h_record(c));
      PACE_KV_TRY(h2d_wait(c));
      PACE_KV_TRY(h2d_copy(c));
      PACE_KV_TRY(h2d_record(c));
      PACE_KV_TRY(unpack(c));
    }
    PACE_HIP(hipEventRecord(s->h2d_done, s->h2d), "record h2d_done");
    return join.now();
  }
  // Step i enqueues unpack(i-S) and pack(i+1) on `stream`, then both copy
  // directions grouped: the waits of H2D(i-1) and D2H(i), the two copies,
  // then their completion records.  The runtime may map the three streams
  // onto shared hardware queues, where a wait or a record that follows a copy
  // holds back everything enqueued behind it.  In this order everything a
  // step enqueues is held back at most until the copies of the step before
  // it finish, which is when the copies of this step are due to start, so the
  // D2H and H2D copies overlap whichever queues the streams share.  The
  // unpack trails by S steps (not 2) so that the H2D copies queued behind it
  // are not held back by its wait for the H2D copy that just ended (measured:
  // 60 us lost per chunk, 8% of a 32 MiB chunk's copy).  Within a step,
  // every wait names the record of the right chunk: unpack(i-S) follows
  // H2D(i-S) (step i-S+1), pack(i+1) follows D2H(i+1-S) (step i+1-S <= i-1),
  // H2D(i-1) follows D2H(i-1) (step i-1) and unpack(i-1-S) (step i-1), and
  // D2H(i) follows pack(i) (step i-1) and H2D(i-regions) (step
  // i-regions+1 <= i-1), which needs S >= 2 and regions >= 2.
  for (int i = -1; i < chunks + S; ++i) {
    const bool h = i - 1 >= 0 && i - 1 < chunks;
    const bool d = i >= 0 && i < chunks;
    if (i - S >= 0 && i - S < chunks) PACE_KV_TRY(unpack(i - S));
    if (i + 1 < chunks) PACE_KV_TRY(pack(i + 1));
    if (h) PACE_KV_TRY(h2d_wait(i - 1));
    if (d) PACE_KV_TRY(d2h_wait(i));
    if (h) PACE_KV_TRY(h2d_copy(i - 1));
    if (d) PACE_KV_TRY(d2h_copy(i));
    if (h) PACE_KV_TRY(h2d_record(i - 1));
    if (d) PACE_KV_TRY(d2h_record(i));
  }
  PACE_HIP(hipEventRecord(s->h2d_done, s->h2d), "record h2d_done");
  // The last unpack is on the work stream: the caller's later work comes
  // after it.
  return join.now();
}

int pace_kv_pack_to_host_noalloc(const void* const* src_layers, int num_layers, int64_t pool_pages,
                                 const int32_t* page_ids, int64_t n_pages, int64_t page_bytes,
                                 void* host_out, int64_t host_out_bytes, int32_t* err_count,
                                 void* stream_) {
  const int64_t cap = PACE_KV_NOALLOC_SCRATCH_BYTES;
  if (num_layers < 0 || n_pages < 0) return fail(PACE_KV_EINVAL, "negative num_layers or n_pages");
  if (page_bytes <= 0 || page_bytes % 16 != 0)
    return fail(PACE_KV_EINVAL, "page_bytes must be a positive multiple of 16");
  if (page_bytes > cap)
    return fail(PACE_KV_ERANGE, "pack_to_host_noalloc: a page of %lld bytes exceeds the %lld-byte scratch",
                (long long)page_bytes, (long long)cap);
  if (n_pages > INT64_MAX / page_bytes) return fail(PACE_KV_ERANGE, "payload size overflows");
  if (num_layers == 0 || n_pages == 0) return PACE_KV_OK;
  if (host_out == nullptr) return fail(PACE_KV_EINVAL, "pack_to_host_noalloc: host_out is NULL");
  if (num_layers > INT64_MAX / (n_pages * page_bytes)) return fail(PACE_KV_ERANGE, "payload size overflows");
  const int64_t payload = num_layers * n_pages * page_bytes;
  if (payload > host_out_bytes)
    return fail(PACE_KV_ERANGE, "pack_to_host_noalloc: the payload needs %lld bytes, host_out holds %lld",
                (long long)payload, (long long)host_out_bytes);
  PACE_KV_TRY(check_pinned_host_out(host_out, payload));
  char* slot = nullptr;
  PACE_KV_TRY(current_scratch(&slot));
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  char* host = static_cast<char*>(host_out);
  const int64_t layer_bytes = n_pages * page_bytes;
  // The copies are the copy kernel's when the device addresses host_out at
  // the same pointer (hipHostMalloc's default), which follows each pack
  // sooner than a DMA copy does.
  const bool kernel = device_addressable_host(host_out, payload);
  // Every pack and copy runs on `stream`, so a chunk's pack overwrites the
  // scratch only after the previous chunk's copy has read it.
  if (layer_bytes <= cap) {
    // chunks of whole layers
    const int64_t k64 = cap / layer_bytes;
    const int k = k64 < num_layers ? static_cast<int>(k64) : num_layers;
    for (int l0 = 0; l0 < num_layers; l0 += k) {
      const int nl = num_layers - l0 < k ? num_layers - l0 : k;
      PACE_KV_TRY(pace_kv_pack(src_layers + l0, nl, pool_pages, page_ids, n_pages, page_bytes, slot,
                               layer_bytes, err_count, stream));
      PACE_HIP(copy_to_host(host + l0 * layer_bytes, slot, nl * layer_bytes, kernel, stream), "D2H copy");
    }
  } else {
    // runs of pages of one layer
    const int64_t run = cap / page_bytes;
    for (int l = 0; l < num_layers; ++l) {
      for (int64_t p0 = 0; p0 < n_pages; p0 += run) {
        const int64_t np = n_pages - p0 < run ? n_pages - p0 : run;
        PACE_KV_TRY(pace_kv_pack(src_layers + l, 1, pool_pages, page_ids + p0, np, page_bytes, slot,
                                 np * page_bytes, err_count, stream));
        PACE_HIP(copy_to_host(host + l * layer_bytes + p0 * page_bytes, slot, np * page_bytes, kernel, stream),
                 "D2H copy");
      }
    }
  }
  return PACE_KV_OK;
}

}  // extern "C"
