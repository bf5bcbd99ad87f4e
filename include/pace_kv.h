/*
 * pace_kv.h — C ABI of the MI355X (gfx950) paged KV-cache migration library
 * (libpace_kv.so).
 *
 * The path moves a request's paged KV cache out of one cache pool and into
 * another.  Each pool is a list of L separately allocated per-layer device
 * buffers, each laid out as [num_pages, 2, page_size, num_kv_heads, head_dim]
 * (dim 1: 0 = K, 1 = V).  A "page" is one slice [2, page_size, H, D] of one
 * layer: page_bytes = 2 * page_size * H * D * sizeof(elem) contiguous bytes.
 * The library copies whole pages as raw bytes, so every dtype (fp16, bf16,
 * fp8, fp32) is handled bit-exactly and the partial last page of a request is
 * copied with all of its slots, stale ones included.
 *
 * Conventions
 *  - Every entry point returns an int status: 0 (PACE_KV_OK) on success, a
 *    negative PACE_KV_E* code for an argument error detected on the host, or a
 *    positive hipError_t value from the HIP runtime.  pace_kv_last_error()
 *    returns a message for the calling thread's last failure.
 *  - Layer tables (src_layers / dst_layers) are HOST arrays of num_layers
 *    DEVICE pointers.  Page-id arrays are DEVICE arrays of int32.
 *  - All device pointers and page_bytes must be multiples of 16 bytes.
 *  - Work is enqueued on `stream` (a hipStream_t; NULL = the null stream) and
 *    the calls return without waiting for it.  The kernels never read or
 *    write a page whose id lies outside [0, pool_pages): such a (layer, page)
 *    tile is skipped and, when err_count (a device int32) is non-NULL, counted
 *    there with an atomic add.
 *  - Entry points are reentrant; none holds global locks or synchronises the
 *    device.  A pace_kv_stager or pace_kv_promoter must be driven by one host
 *    thread at a time; a pace_kv_allocator serialises its callers with its own
 *    mutex.
 */
#ifndef PACE_KV_H_
#define PACE_KV_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PACE_KV_ABI_VERSION 2

/* Largest number of layers one kernel launch addresses; entry points split
 * longer layer lists into several launches on the same stream. */
#define PACE_KV_MAX_LAYERS_PER_LAUNCH 64

enum pace_kv_status {
  PACE_KV_OK = 0,
  PACE_KV_EINVAL = -1,   /* null pointer, negative size, misalignment        */
  PACE_KV_ERANGE = -2,   /* page id or size outside what a buffer holds      */
  PACE_KV_ENOMEM = -3,   /* allocator exhausted (no free pages)              */
  PACE_KV_ESTATE = -4,   /* object used in a state that does not allow it    */
  PACE_KV_ETIMEDOUT = -5, /* a channel wait passed its deadline               */
  PACE_KV_ECLOSED = -6   /* the channel was closed by either side            */
};

/* ABI version this library was built with (PACE_KV_ABI_VERSION). */
int pace_kv_abi_version(void);

/* Message describing the calling thread's most recent failing call. */
const char* pace_kv_last_error(void);

/* ------------------------------------------------------------------------ */
/* Device-to-device page copies                                              */
/* ------------------------------------------------------------------------ */

/*
 * PACK (multi-layer gather).
 *   out[l][j] = src_layers[l][page_ids[j]]   for l < num_layers, j < n_pages
 * where out[l] = (char*)out + l * out_layer_stride and each element is one
 * page of page_bytes.  Several requests are packed in one call by
 * concatenating their block tables in page_ids (CSR order); request r's
 * slice is then out[:, indptr[r]:indptr[r+1]].
 *
 * Replaces the per-layer gather in KVhelper.get_kv_cache
 *   (paceserve/kv_transfer/kv_utils.py:44-46:
 *    seq_cache[i] = gpu_cache[i][torch.tensor(kv_page_indices)]).
 */
int pace_kv_pack(const void* const* src_layers, int num_layers,
                 int64_t pool_pages, const int32_t* page_ids, int64_t n_pages,
                 int64_t page_bytes, void* out, int64_t out_layer_stride,
                 int32_t* err_count, void* stream);

/*
 * UNPACK (multi-layer scatter through a remapped block table).
 *   dst_layers[l][page_ids[j]] = buf[l][j]
 * where buf[l] = (const char*)buf + l * buf_layer_stride.  Pages of the
 * destination pools not named in page_ids are left untouched.  page_ids must
 * not repeat a page (the host layer removes repeats, keeping the last
 * occurrence, as a sequential index_put_ would).
 *
 * Replaces the per-layer scatter in KVhelper.insert_kv_cache
 *   (paceserve/kv_transfer/kv_utils.py:49-52:
 *    gpu_cache[i][torch.tensor(kv_indices)] = cached_content[i].to(device)).
 */
int pace_kv_unpack(const void* buf, int64_t buf_layer_stride,
                   void* const* dst_layers, int num_layers, int64_t pool_pages,
                   const int32_t* page_ids, int64_t n_pages, int64_t page_bytes,
                   int32_t* err_count, void* stream);

/*
 * MOVE (pack and unpack fused, pool to pool on one device, no transfer buffer).
 *   dst_layers[l][dst_ids[j]] = src_layers[l][src_ids[j]]
 * Produces the same destination bytes as PACK followed by UNPACK with half of
 * their HBM traffic.  Source and destination pages must not overlap.
 *
 * Replaces get_kv_cache followed by insert_kv_cache when both caches live on
 * the same GPU (paceserve/worker/base_worker.py:236-281).
 */
int pace_kv_move(const void* const* src_layers, int64_t src_pool_pages,
                 const int32_t* src_ids, void* const* dst_layers,
                 int64_t dst_pool_pages, const int32_t* dst_ids,
                 int num_layers, int64_t n_pages, int64_t page_bytes,
                 int32_t* err_count, void* stream);

/*
 * SWAP OUT / SWAP IN between a device pool and a host-resident pool of pages
 * in pinned memory (hipHostMalloc / torch pin_memory), in one kernel that
 * reads or writes the host pages across PCIe directly (no staging buffer):
 *   swap_out: host_layers[l][host_ids[j]] = dev_layers[l][dev_ids[j]]
 *   swap_in:  dev_layers[l][dev_ids[j]]   = host_layers[l][host_ids[j]]
 * Host layers have the device pool's layout [host_pool_pages, 2, P, H, D].
 * Every layer pointer is checked on the host before launch: host layers must
 * be pinned host memory mapped for the device and device layers memory of the
 * current device, each allocation holding pool_pages * page_bytes from the
 * pointer (else PACE_KV_EINVAL / PACE_KV_ERANGE).  Page ids are device int32.
 *
 * Replaces the preemption swap of a decode instance: get_kv_cache without
 * free into host DRAM and the later re-insertion
 * (paceserve/engine/decode_llm_engine.py:31-41,
 *  paceserve/disutil/decode_instance.py:176-192).
 */
int pace_kv_swap_out(const void* const* dev_layers, int64_t dev_pool_pages,
                     const int32_t* dev_ids, void* const* host_layers,
                     int64_t host_pool_pages, const int32_t* host_ids,
                     int num_layers, int64_t n_pages, int64_t page_bytes,
                     int32_t* err_count, void* stream);
int pace_kv_swap_in(const void* const* host_layers, int64_t host_pool_pages,
                    const int32_t* host_ids, void* const* dev_layers,
                    int64_t dev_pool_pages, const int32_t* dev_ids,
                    int num_layers, int64_t n_pages, int64_t page_bytes,
                    int32_t* err_count, void* stream);

/* ------------------------------------------------------------------------ */
/* Pinned-host staging (the host leg of a migration)                         */
/* ------------------------------------------------------------------------ */

/*
 * A stager owns two rings of device slots (one feeding device-to-host copies,
 * one fed by host-to-device copies), three side streams created one after
 * another (the round trip's packs and unpacks, D2H copies, H2D copies; default
 * priority) and the events that order them against the caller's stream.
 * Each slot holds slot_bytes; a layer chunk of k layers needs
 * k * n_pages * page_bytes <= slot_bytes.
 */
typedef struct pace_kv_stager pace_kv_stager;

int pace_kv_stager_create(int64_t slot_bytes, int num_slots,
                          pace_kv_stager** out);
int pace_kv_stager_destroy(pace_kv_stager* stager);

/*
 * Pack into host memory: for every chunk of layers_per_chunk layers, PACK into
 * a device slot on `stream`, then copy the slot to
 * host_out + layer_begin * n_pages * page_bytes on the D2H side stream, so the
 * copy of chunk c overlaps the pack of chunk c+1.  host_out receives the
 * layout [num_layers, n_pages, page_size-slice...] of PACK with
 * out_layer_stride = n_pages * page_bytes.  Pinned host memory gives
 * asynchronous DMA; pageable memory works but the runtime stages it.
 * When the call returns, `stream` is ordered after the last copy enqueued,
 * also when it fails part-way.  A call of one chunk
 * (layers_per_chunk >= num_layers) packs and copies on `stream`, the copy by
 * a 16-wave kernel when host_out is pinned memory the device addresses.
 *
 * Replaces the gather + pageable device-to-host copy loop of
 * KVhelper.get_kv_cache (paceserve/kv_transfer/kv_utils.py:44-47).
 */
int pace_kv_pack_to_host(pace_kv_stager* stager,
                         const void* const* src_layers, int num_layers,
                         int64_t pool_pages, const int32_t* page_ids,
                         int64_t n_pages, int64_t page_bytes,
                         int layers_per_chunk, void* host_out,
                         int32_t* err_count, void* stream);

/*
 * Unpack from host memory: the mirror of pace_kv_pack_to_host.  Chunk c is
 * copied host-to-device on the H2D side stream while chunk c-1 is unpacked on
 * `stream`; a call of one chunk copies and unpacks on `stream`.  When the
 * call returns, `stream` is ordered after every copy it enqueued, also when
 * it fails part-way.
 *
 * Replaces the pageable host-to-device copy + scatter loop of
 * KVhelper.insert_kv_cache (paceserve/kv_transfer/kv_utils.py:49-52).
 */
int pace_kv_unpack_from_host(pace_kv_stager* stager, const void* host_in,
                             void* const* dst_layers, int num_layers,
                             int64_t pool_pages, const int32_t* page_ids,
                             int64_t n_pages, int64_t page_bytes,
                             int layers_per_chunk, int32_t* err_count,
                             void* stream);

/* Bytes of the device scratch array through which
 * pace_kv_pack_to_host_noalloc stages its chunks (64 MiB per GPU). */
#define PACE_KV_NOALLOC_SCRATCH_BYTES (64 << 20)

/*
 * Allocation-free pack into host memory.  No counterpart in the reference:
 * it is for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc), which
 * cannot create a pace_kv_stager.  It writes the same host_out bytes as
 * pace_kv_pack_to_host, with no stager: each chunk is packed into a device
 * scratch array of PACE_KV_NOALLOC_SCRATCH_BYTES, which the library holds on
 * every GPU it runs on until the process ends, and copied from there to
 * host_out, pack and copy both on `stream` (no side stream, so a chunk's pack
 * does not overlap the previous chunk's copy); the copy is a 16-wave kernel
 * when the device addresses host_out at the same pointer (hipHostMalloc's
 * default), else hipMemcpyAsync.  Chunks are whole layers when
 * one layer's n_pages * page_bytes fits the scratch, else runs of pages of
 * one layer; a page larger than the scratch is rejected (PACE_KV_ERANGE).
 * host_out must be pinned host memory (hipHostMalloc) and host_out_bytes the
 * bytes the caller gives it: a payload (num_layers * n_pages * page_bytes)
 * larger than host_out_bytes, or running past the end of host_out's pinned
 * allocation, is rejected (PACE_KV_ERANGE) before anything is enqueued.
 * Pageable memory is rejected (PACE_KV_EINVAL), since the runtime would stage
 * its copies through buffers of its own.
 * It calls no hipMalloc or hipFree, and once a call has run on a device (the
 * first call looks up that device's scratch address) later calls there make
 * only kernel launches and hipMemcpyAsync copies on `stream`, so they can be
 * captured into a HIP graph.  Every call on one GPU shares that GPU's
 * scratch: calls on one stream from one host thread are ordered, while calls
 * that overlap (on several streams, or from several host threads, or a graph
 * replayed beside other calls) race on it.
 */
int pace_kv_pack_to_host_noalloc(const void* const* src_layers, int num_layers,
                                 int64_t pool_pages, const int32_t* page_ids,
                                 int64_t n_pages, int64_t page_bytes,
                                 void* host_out, int64_t host_out_bytes,
                                 int32_t* err_count, void* stream);

/*
 * Full host round trip in one pipeline: pack(c) -> D2H(c) -> H2D(c) ->
 * unpack(c) per layer chunk, with pack(c+1), D2H(c), H2D(c-1) and the
 * unpacks of earlier chunks in flight together.  The D2H copies are a copy
 * kernel of 16 waves when host_buf is pinned host memory the device can
 * address (hipHostMalloc, torch's pin_memory), else hipMemcpyAsync; the H2D
 * copies are hipMemcpyAsync.  Packs and unpacks, D2H copies and H2D copies run
 * on three streams of the stager's own: the packs
 * start after the work enqueued on `stream` before the call, and `stream`
 * waits for everything the call enqueued, so `stream`'s later work comes
 * after the last unpack (also when the call fails part-way).  The copies
 * overlap however the runtime maps these streams onto its hardware queues.
 * Calls on one stager run their packs and unpacks in call order, whichever
 * `stream` each names.  A call of one chunk has nothing to overlap and runs
 * its four stages on `stream`, after the stager's earlier calls.
 * host_buf holds host_bytes of host memory used as a ring of chunk-sized
 * regions (host_bytes >= one chunk; pass the full payload to keep a complete
 * host copy, as the reference's KVobj does).
 *
 * Replaces KVhelper.get_kv_cache followed by KVhelper.insert_kv_cache through
 * host DRAM (paceserve/worker/base_worker.py:236-281,
 * paceserve/engine/decode_llm_engine.py:31-41).
 */
int pace_kv_roundtrip(pace_kv_stager* stager,
                      const void* const* src_layers, int64_t src_pool_pages,
                      const int32_t* src_ids, void* const* dst_layers,
                      int64_t dst_pool_pages, const int32_t* dst_ids,
                      int num_layers, int64_t n_pages, int64_t page_bytes,
                      int layers_per_chunk, void* host_buf, int64_t host_bytes,
                      int32_t* err_count, void* stream);

/* ------------------------------------------------------------------------ */
/* Paged append (the producer of page contents)                              */
/* ------------------------------------------------------------------------ */

/*
 * Writes the K and V rows of nnz appended tokens into one layer's paged cache
 * [num_pages, 2, page_size, H, D]:
 *   b = batch_indices[i], pos = positions[i],
 *   page = kv_indices[kv_indptr[b] + pos / page_size], slot = pos % page_size,
 *   cache[page][0][slot] = keys[i], cache[page][1][slot] = values[i]
 * keys / values hold nnz rows of row_bytes = H * D * elem bytes, token_stride
 * bytes apart (device).  batch_indices, positions (nnz), kv_indptr
 * (batch_size + 1) and kv_indices (num_indices) are device int32 arrays.
 * A token whose request, page slot (outside its request's pages) or page id
 * is out of range is skipped and counted in err_count.
 *
 * Replaces flashinfer.append_paged_kv_cache as called in
 * paceserve/model_executor/attention/flashinfer_attention_wrapper.py:245-255.
 */
int pace_kv_append(const void* keys, const void* values, int64_t token_stride_bytes,
                   int64_t nnz, const int32_t* batch_indices, const int32_t* positions,
                   int batch_size, void* cache, int64_t num_pages,
                   const int32_t* kv_indices, int64_t num_indices,
                   const int32_t* kv_indptr, int page_size, int64_t row_bytes,
                   int32_t* err_count, void* stream);

/*
 * The same append with each token's request and position derived in the
 * launch itself from the request offsets, so one launch does what
 * get_seq_lens, get_batch_indices_positions and append_paged_kv_cache do:
 *   token i of request b (append_indptr[b] <= i < append_indptr[b+1]),
 *   seq_len = max(kv_indptr[b+1] - kv_indptr[b] - 1, 0) * page_size + kv_last_page_len[b],
 *   pos = seq_len - (append_indptr[b+1] - append_indptr[b]) + (i - append_indptr[b]).
 * append_indptr, kv_indptr (batch_size + 1 entries), kv_last_page_len
 * (batch_size) and kv_indices are device int32 arrays.  A token outside
 * every request, or whose slot or page is out of range, is skipped and
 * counted in err_count.
 *
 * Replaces the three calls the reference makes for each layer
 * (paceserve/model_executor/attention/flashinfer_attention_wrapper.py:
 * 241-255).
 */
int pace_kv_append_indptr(const void* keys, const void* values,
                          int64_t token_stride_bytes, int64_t nnz,
                          const int32_t* append_indptr, int batch_size,
                          void* cache, int64_t num_pages,
                          const int32_t* kv_indices, int64_t num_indices,
                          const int32_t* kv_indptr,
                          const int32_t* kv_last_page_len, int page_size,
                          int64_t row_bytes, int32_t* err_count, void* stream);

/*
 * Request index and sequence position of every appended token (device):
 *   for append_indptr[b] <= i < append_indptr[b+1]:
 *     batch_indices[i] = b,
 *     positions[i] = seq_lens[b] - (append_indptr[b+1] - append_indptr[b]) + (i - append_indptr[b])
 * where seq_lens[b] counts the request's tokens including the appended ones
 * (max(pages - 1, 0) * page_size + last_page_len).  Tokens beyond
 * append_indptr[batch_size] get -1, which the append skips.
 *
 * Replaces flashinfer.get_batch_indices_positions as called in
 * paceserve/model_executor/attention/flashinfer_attention_wrapper.py:242.
 */
int pace_kv_batch_indices_positions(const int32_t* append_indptr, const int32_t* seq_lens,
                                    int batch_size, int64_t nnz, int32_t* batch_indices,
                                    int32_t* positions, void* stream);

/* ------------------------------------------------------------------------ */
/* Native block allocation, batch planning and single-call promotion          */
/* ------------------------------------------------------------------------ */

/*
 * LIFO free list of page ids over [0, num_pages), guarded by a mutex.
 * free_list NULL means the fresh pool [0, 1, ..., num_pages-1], which hands
 * out num_pages-1 first; otherwise free_list[free_len-1] is handed out first.
 *
 * Replaces BlockAllocator
 *   (paceserve/core/block_space_manager/base_block_space_manager.py:11-47).
 */
typedef struct pace_kv_allocator pace_kv_allocator;

int pace_kv_allocator_create(int64_t num_pages, const int32_t* free_list,
                             int64_t free_len, pace_kv_allocator** out);
int pace_kv_allocator_destroy(pace_kv_allocator* alloc);
int pace_kv_allocator_num_free(pace_kv_allocator* alloc, int64_t* out);

/* n pages in the order n successive pops return them; all-or-nothing:
 * PACE_KV_ENOMEM ("Out of memory! No free blocks are available.") leaves the
 * list unchanged.  Replaces BlockAllocator.allocate (:34-39) and
 * BaseBlockSpaceManager.allocate (:89-97). */
int pace_kv_allocator_allocate(pace_kv_allocator* alloc, int64_t n, int32_t* out_ids);

/* Returns each distinct page of ids[0..n) once, in first-occurrence order.
 * Replaces BaseBlockSpaceManager._free_block_table (:119-121). */
int pace_kv_allocator_free(pace_kv_allocator* alloc, const int32_t* ids, int64_t n);

/* Copies the free list (allocation order: last entry first) into out. */
int pace_kv_allocator_snapshot(pace_kv_allocator* alloc, int32_t* out,
                               int64_t capacity, int64_t* len);

/*
 * Plans a batch of num_requests migrations: request r's source pages are
 * src_ids[src_indptr[r] .. src_indptr[r+1]) (host arrays, ids in
 * [0, src_pool_pages)); it receives dst_pages[r] destination pages (NULL:
 * as many as its source pages), which must be n_r or n_r + 1.  Pages are
 * allocated request by request from dst_alloc, all-or-nothing.  Outputs (host):
 * out_dst_tables, every request's full destination table (sum of dst_pages
 * entries); out_dst_ids, the pages that receive data, CSR like src_ids (a
 * table of n_r + 1 pages leaves its last page untouched).
 *
 * Replaces the destination allocation and remap of BaseWorker._insert_kv_cache
 * (paceserve/worker/base_worker.py:255-277) for a whole batch.
 */
int pace_kv_plan(pace_kv_allocator* dst_alloc, int num_requests,
                 const int64_t* src_indptr, const int32_t* src_ids,
                 int64_t src_pool_pages, const int32_t* dst_pages,
                 int32_t* out_dst_tables, int32_t* out_dst_ids);

/*
 * A promoter owns two pinned host slots and two device slots for block-table
 * ids, and the events that guard their reuse.
 */
typedef struct pace_kv_promoter pace_kv_promoter;

int pace_kv_promoter_create(pace_kv_promoter** out);
int pace_kv_promoter_destroy(pace_kv_promoter* promoter);

/*
 * One-call promotion of a batch: pace_kv_plan, one host-to-device copy of
 * both id lists on `stream`, then the page movement: with buffer == NULL a
 * fused pace_kv_move; otherwise pace_kv_pack into `buffer` followed by
 * pace_kv_unpack, in chunks of buffer_layers layers (the buffer holds
 * buffer_layers layers of buffer_layer_stride bytes).  out_dst_tables is as in
 * pace_kv_plan.  On failure no destination page stays allocated.
 *
 * Replaces KVhelper.get_kv_cache + BaseWorker._insert_kv_cache for requests
 * whose source and destination caches share a GPU
 * (paceserve/worker/base_worker.py:236-281, kv_utils.py:33-56).
 */
int pace_kv_promote(pace_kv_promoter* promoter, pace_kv_allocator* dst_alloc,
                    const void* const* src_layers, int64_t src_pool_pages,
                    void* const* dst_layers, int64_t dst_pool_pages,
                    int num_layers, int64_t page_bytes, int num_requests,
                    const int64_t* src_indptr, const int32_t* src_ids,
                    const int32_t* dst_pages, void* buffer,
                    int64_t buffer_layer_stride, int buffer_layers,
                    int32_t* out_dst_tables, int32_t* err_count, void* stream);

/* ------------------------------------------------------------------------ */
/* Cross-process channel                                                     */
/* ------------------------------------------------------------------------ */

/*
 * A named shared-memory ring (POSIX shm "/<name>") that carries packed KV
 * pages from a sender process to a receiver process, with no serialization
 * and no object store: the sender packs a layer chunk, copies it to pinned
 * memory and from there into a ring slot (a pool of copy_threads host threads
 * does that copy); the receiver copies a slot out to pinned memory, uploads
 * it and unpacks it, chunk by chunk, overlapped.  A message is a header (its
 * shape and an opaque metadata blob of at most slot_bytes, e.g. the sequence
 * id and source block table) followed by its payload in the transfer-buffer
 * layout [num_layers][n_pages][page_bytes], in chunks of whole layers when a
 * layer fits in a slot, else of pages of one layer (a page must fit).
 * Messages larger than the ring stream through it, so the receiver must be
 * receiving while the sender sends.
 *
 * One sender and one receiver per channel; each endpoint serialises its own
 * sends (whole messages) and its own receives.  Every blocking call waits at
 * most timeout_ms milliseconds (PACE_KV_ETIMEDOUT; 0 = do not wait) and
 * returns PACE_KV_ECLOSED once either side has closed the channel or the peer
 * process has exited (checked at least every 10 ms while waiting).  A send
 * on a closed channel fails with PACE_KV_ECLOSED before it writes anything;
 * a receiver still takes the messages published before the sender closed
 * (those in shared-memory slots, and those in device slots while the ring is
 * alive: see pace_kv_channel_create_device).  A sender that fails after the
 * header marks the message abandoned, and the receiver's next wait for its
 * chunks fails with PACE_KV_ESTATE.
 *
 * Replaces the transfer of a KVobj from a prefill instance to a decode
 * instance through Ray's object store (paceserve/disutil/prefill_instance.py:
 * 96-107 transfer_kv_cache returns the KVobj holding the host tensor;
 * paceserve/disutil/decode_instance.py:165-171 ray.get()s it and inserts it;
 * paceserve/core/datatypes/kv_cache_obj.py:7-21 KVobj): only the sequence id
 * crosses the control plane, the pages cross the ring.
 */
typedef struct pace_kv_channel pace_kv_channel;

/* Creates the channel "/<name>" (fails with PACE_KV_ESTATE if it exists):
 * num_slots (a power of two in [2, 64]) slots of slot_bytes (a multiple of
 * 4096).  The
 * creator's close unlinks the name.  copy_threads in [1, 64]. */
int pace_kv_channel_create(const char* name, int64_t slot_bytes, int num_slots,
                           int copy_threads, pace_kv_channel** out);
/* As pace_kv_channel_create, plus a device ring on the current GPU for peers
 * on the same GPU: num_slots device slots of dev_slot_bytes (a multiple of
 * 4096; num_slots * dev_slot_bytes at most 1 GiB), allocated here and
 * exported with hipIpcGetMemHandle.  A pace_kv_channel_send made on that GPU
 * packs each chunk straight into a device slot (chunks sized to
 * dev_slot_bytes), and the receiving endpoint unpacks straight out of it, so
 * the payload never leaves HBM; the other endpoint opens the ring on its
 * first device transfer.  Sends from another GPU, sends while the receiver's
 * GPU (recorded at its last pace_kv_channel_recv_header) is another one or
 * none, and send_host, use the shared-memory slots as before.
 * Lifetime: endpoints in the creator's process share the ring, which is
 * freed when the last of them closes, in any order.  Another process that
 * has opened the ring uses it only while the creator's endpoint is open:
 * once the creator has closed, its sends and its receives of device-slot
 * messages fail with PACE_KV_ECLOSED, so the creator must outlive the
 * device transfers of its peers.  Replaces, for two instance processes on
 * one GPU, the same object-store hop as pace_kv_channel_create
 * (paceserve/disutil/prefill_instance.py:96-107,
 *  paceserve/disutil/decode_instance.py:165-171). */
int pace_kv_channel_create_device(const char* name, int64_t slot_bytes,
                                  int num_slots, int copy_threads,
                                  int64_t dev_slot_bytes,
                                  pace_kv_channel** out);
/* The device ring's slot bytes (0: the channel has none) and whether it lives
 * on the current GPU (sends from this GPU then use it). */
int pace_kv_channel_device_info(pace_kv_channel* channel,
                                int64_t* dev_slot_bytes, int* on_current_gpu);
/* Opens a channel created by the peer, waiting up to timeout_ms for it. */
int pace_kv_channel_open(const char* name, int copy_threads, int timeout_ms,
                         pace_kv_channel** out);
/* Marks the channel closed for both sides, waits for this endpoint's device
 * work, and unmaps it.  No call may be in progress on this endpoint. */
int pace_kv_channel_close(pace_kv_channel* channel);
int pace_kv_channel_info(pace_kv_channel* channel, int64_t* slot_bytes,
                         int* num_slots);
/* Removes the name "/<name>" (a channel left behind by a creator that died
 * before closing it); endpoints already open keep working.  A name that does
 * not exist is not an error. */
int pace_kv_channel_unlink(const char* name);

/* Sends one message whose payload is packed from device pools:
 *   payload[l][j] = src_layers[l][page_ids[j]].
 * page_ids: int32, in device memory, or in host memory (pageable or pinned)
 * when n_pages <= 512: host ids travel in each pack's kernel arguments, so no
 * upload precedes the first pack (more than 512 host ids: PACE_KV_ERANGE).
 * Packs run on `stream` after its earlier work.  Returns once every chunk is
 * in the ring (host-synchronous); *msg_id receives the message's id.  On the
 * GPU of a channel's device ring the chunks go into device slots. */
int pace_kv_channel_send(pace_kv_channel* channel,
                         const void* const* src_layers, int num_layers,
                         int64_t pool_pages, const int32_t* page_ids,
                         int64_t n_pages, int64_t page_bytes,
                         const void* meta, int64_t meta_bytes, int timeout_ms,
                         uint64_t* msg_id, void* stream);
/* Sends one message whose payload is already in host memory, contiguous in
 * the transfer-buffer layout (num_layers * n_pages * page_bytes bytes). */
int pace_kv_channel_send_host(pace_kv_channel* channel, const void* payload,
                              int num_layers, int64_t n_pages,
                              int64_t page_bytes, const void* meta,
                              int64_t meta_bytes, int timeout_ms,
                              uint64_t* msg_id);

/* Receives the next message's header: its metadata (into meta, meta_cap
 * bytes; with a smaller buffer PACE_KV_ERANGE reports the size in
 * *meta_bytes and leaves the message in place) and its shape.  The payload
 * must then be received (pace_kv_channel_recv or _recv_host) before the next
 * header; a header with num_layers or n_pages 0 has none. */
int pace_kv_channel_recv_header(pace_kv_channel* channel, void* meta,
                                int64_t meta_cap, int64_t* meta_bytes,
                                int* num_layers, int64_t* n_pages,
                                int64_t* page_bytes, uint64_t* msg_id,
                                int timeout_ms);
/* Receives the current message's payload into device pools:
 *   dst_layers[l][page_ids[j]] = payload[l][j] (page_ids: int32, distinct,
 * in device memory or, with n_pages <= 512, in host memory as for
 * pace_kv_channel_send).  The shape must equal the header's.  Unpacks run on `stream`
 * after its earlier work; the call returns once every chunk has left the
 * ring, with the last unpacks still enqueued (a payload in device slots:
 * with every unpack finished, since a slot is released only then).  Ids outside [0, pool_pages)
 * are skipped and counted in err_count, as in pace_kv_unpack.  After a
 * PACE_KV_ETIMEDOUT the call may be repeated and continues where it
 * stopped. */
int pace_kv_channel_recv(pace_kv_channel* channel, void* const* dst_layers,
                         int num_layers, int64_t pool_pages,
                         const int32_t* page_ids, int64_t n_pages,
                         int64_t page_bytes, int32_t* err_count,
                         int timeout_ms, void* stream);
/* Receives the current message's payload into host memory (payload_bytes
 * must equal the payload's size), or discards it when payload is NULL (a
 * receiver that cannot take the message must still drain it). */
int pace_kv_channel_recv_host(pace_kv_channel* channel, void* payload,
                              int64_t payload_bytes, int timeout_ms);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif /* PACE_KV_H_ */
