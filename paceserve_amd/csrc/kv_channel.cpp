// Cross-process KV channel: moves packed KV pages from one process to
// another through a named shared-memory ring, in place of pickling the host
// tensor through an object store.
//
// Layout of the shared object (POSIX shm, /dev/shm/<name>):
//   ChannelCtl (control block: ring counters, per-slot records)
//   num_slots data slots of slot_bytes each, page-aligned
// One sender and one receiver (single producer, single consumer).  The sender
// owns `head` (slots published), the receiver owns `tail` (slots released);
// both are 32-bit futex words, compared modulo 2^32, and the slot count is a
// power of two so that the slot of a record stays the count modulo num_slots
// across the wrap.  A slot holds one record:
// a message header (shape + an opaque metadata blob) or one chunk of the
// message's payload.  The payload is the contiguous transfer-buffer layout
// [num_layers][n_pages][page_bytes]; a chunk is a run of whole layers when a
// layer fits in a slot, else a run of pages of one layer.
//
// The device legs stage through pinned memory, since a kernel or DMA engine
// cannot reach the shared mapping (it is pageable; pinning memory that already
// exists is not available): the sender packs chunk c into a device slot,
// copies it to a pinned slot, and copies that into the shared slot with a pool
// of host threads while chunk c+1 is packed and copied down; the receiver
// copies a shared slot into a pinned slot (releasing the shared slot at once),
// then uploads it and unpacks it while the next chunk is copied.
//
// Same-GPU device ring: a creator may also allocate a ring of device slots
// (pace_kv_channel_create_device) and export it with hipIpcGetMemHandle; the
// other process opens the handle on its first device transfer.  A device
// send then packs each chunk straight into a device slot and publishes it
// once its pack has finished; the receiver unpacks from that slot and
// releases it once its unpack has finished.  Those payload bytes never leave
// HBM.  Headers still travel in the shared-memory slots, and a message is
// wholly in device slots or wholly in host slots (the header says which).
//
// Failures: every wait has a deadline and ends when either side closes the
// channel; the control block records which process plays each role, so a
// wait also ends when the peer process has exited.  A sender that fails
// part-way marks its message abandoned; a receiver skips chunks left over
// from a message it failed to take.
#include <errno.h>
#include <stddef.h>
#include <fcntl.h>
#include <signal.h>
#include <stdio.h>
#include <linux/futex.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <sys/syscall.h>
#include <time.h>
#include <unistd.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <condition_variable>
#include <map>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

#include "internal.h"

using pace_kv::fail;
using pace_kv::hip_status;

namespace {

constexpr uint64_t kMagic = 0x50414345'4b564348ull;  // "PACEKVCH"
constexpr uint32_t kVersion = 4;
constexpr int kMaxSlots = 64;
constexpr int kNameMax = 200;
// Largest device ring: one shared allocation, kept well under the 2 GiB
// beyond which opening an exported allocation was seen not to return.
constexpr int64_t kMaxDeviceRing = int64_t(1) << 30;
constexpr int kBusIdBytes = 64;

enum RecordKind : uint32_t { kEmpty = 0, kHeader = 1, kData = 2, kDevData = 3 };
// Header flags.
constexpr int32_t kDevicePayload = 1;  // the payload's chunks are in device slots

static_assert(sizeof(std::atomic<uint32_t>) == 4, "futex words are 32-bit");
static_assert(std::atomic<uint32_t>::is_always_lock_free, "shared counters must be lock-free");
static_assert(std::atomic<uint64_t>::is_always_lock_free, "shared counters must be lock-free");

struct alignas(64) SlotRecord {
  uint32_t kind;
  uint32_t chunk;        // data: chunk index within the message
  uint64_t msg_id;
  int64_t offset;        // data: byte offset of the chunk in the payload
  int64_t bytes;         // data: chunk bytes; header: metadata bytes
  int64_t n_pages;       // header
  int64_t page_bytes;    // header
  int32_t num_layers;    // header
  int32_t flags;         // header: kDevicePayload
};

// Which process plays a role (sender or receiver): its pid, its pid
// namespace and its start time, so that a waiting peer can tell that the
// process has exited (or that its pid now names another process).
struct ProcessId {
  std::atomic<int32_t> pid;      // 0: no process has taken the role yet
  std::atomic<uint64_t> pidns;   // inode of /proc/<pid>/ns/pid
  std::atomic<uint64_t> start;   // start time, field 22 of /proc/<pid>/stat
};

struct alignas(64) ChannelCtl {
  uint64_t magic;
  uint32_t version;
  uint32_t num_slots;
  int64_t slot_bytes;
  int64_t data_offset;   // first data slot, from the start of the mapping
  int64_t total_bytes;
  alignas(64) std::atomic<uint32_t> head;    // sender: records published
  alignas(64) std::atomic<uint32_t> tail;    // receiver: records released
  alignas(64) std::atomic<uint32_t> closed;  // either side closed the channel
  std::atomic<uint64_t> next_msg_id;         // sender: id of the next message
  std::atomic<uint64_t> aborted_msg;         // sender: id of a message it gave up (0 = none)
  ProcessId sender, receiver;
  SlotRecord slots[kMaxSlots];
  // Device ring (dev_slot_bytes 0: none): num_slots device slots of
  // dev_slot_bytes, allocated by the process dev_owner_pid on the GPU
  // dev_bus_id, exported as dev_handle.
  int64_t dev_slot_bytes;
  int32_t dev_owner_pid;
  int32_t dev_pad;
  char dev_bus_id[kBusIdBytes];
  hipIpcMemHandle_t dev_handle;
  // The creator has closed its endpoint: a ring it exported is freed (or
  // about to be), so other processes no longer touch it.
  std::atomic<uint32_t> creator_closed;
  // PCI bus id of the GPU that was current when the receiver last asked for
  // a header, as 8 words of 8 bytes (all zero: not known yet; kNoGpu: the
  // receiver had no GPU).  A sender uses the device ring only when the
  // receiver is not known yet or is on the ring's GPU.
  std::atomic<uint64_t> rx_bus_id[kBusIdBytes / 8];
};

// head and tail count records modulo 2^32 and a record's slot is the count
// modulo num_slots; a power-of-two slot count divides 2^32, so consecutive
// records keep consecutive slots across the counters' wrap.
static_assert(offsetof(ChannelCtl, num_slots) == 12 && offsetof(ChannelCtl, head) == 64 &&
                  offsetof(ChannelCtl, tail) == 128,
              "control-block layout (the CPU tests write num_slots, head and tail at these offsets)");

bool valid_slot_count(int64_t n) { return n >= 2 && n <= kMaxSlots && (n & (n - 1)) == 0; }

int64_t round_up(int64_t v, int64_t a) { return (v + a - 1) / a * a; }

// State (field 3) and start time (field 22) of /proc/<pid>/stat; false if the
// process does not exist.
bool proc_stat(int pid, char* state, uint64_t* start) {
  char path[64];
  snprintf(path, sizeof(path), "/proc/%d/stat", pid);
  FILE* f = fopen(path, "r");
  if (f == nullptr) return false;
  char buf[1024];
  const size_t n = fread(buf, 1, sizeof(buf) - 1, f);
  fclose(f);
  buf[n] = '\0';
  const char* p = strrchr(buf, ')');  // the command name may hold spaces
  if (p == nullptr) return false;
  unsigned long long st = 0;
  // after ") ": state, then 18 fields, then the start time
  if (sscanf(p + 2, "%c %*s %*s %*s %*s %*s %*s %*s %*s %*s %*s %*s %*s %*s %*s %*s %*s %*s %*s %llu",
             state, &st) != 2)
    return false;
  *start = st;
  return true;
}

uint64_t pid_namespace(const char* who) {
  char path[64];
  snprintf(path, sizeof(path), "/proc/%s/ns/pid", who);
  struct stat st;
  return stat(path, &st) == 0 ? static_cast<uint64_t>(st.st_ino) : 0;
}

// Records the calling process as the one playing `role`.
void take_role(ProcessId& role) {
  static const int32_t pid = static_cast<int32_t>(getpid());
  static const uint64_t ns = pid_namespace("self");
  static const uint64_t start = [] {
    char state = 0;
    uint64_t t = 0;
    return proc_stat(static_cast<int>(getpid()), &state, &t) ? t : 0;
  }();
  if (role.pid.load(std::memory_order_acquire) == pid) return;
  role.pid.store(0, std::memory_order_release);
  role.pidns.store(ns, std::memory_order_relaxed);
  role.start.store(start, std::memory_order_relaxed);
  role.pid.store(pid, std::memory_order_release);
}

// True when the process recorded in `role` is known to have exited.  A role
// not yet taken, taken by this process, or taken in another pid namespace
// (whose pids this process cannot check) counts as alive.
bool role_gone(const ProcessId& role) {
  const int32_t pid = role.pid.load(std::memory_order_acquire);
  if (pid <= 0 || pid == static_cast<int32_t>(getpid())) return false;
  static const uint64_t own_ns = pid_namespace("self");
  if (own_ns == 0 || role.pidns.load(std::memory_order_relaxed) != own_ns) return false;
  if (kill(pid, 0) != 0 && errno == ESRCH) return true;
  char state = 0;
  uint64_t start = 0;
  if (!proc_stat(pid, &state, &start)) return false;  // cannot tell
  return state == 'Z' || state == 'X' || start != role.start.load(std::memory_order_relaxed);
}

long futex(std::atomic<uint32_t>* word, int op, uint32_t val, const timespec* ts) {
  return syscall(SYS_futex, reinterpret_cast<uint32_t*>(word), op, val, ts, nullptr, 0);
}

void wake_all(std::atomic<uint32_t>* word) { (void)futex(word, FUTEX_WAKE, INT32_MAX, nullptr); }

// Splits large host copies over a pool of threads (the caller takes a share).
// A job's fields change only while no worker is inside work(): a worker joins
// a job under the lock (active_), and the caller waits for active_ == 0 both
// before setting up a job and before returning from it.
class CopyPool {
 public:
  explicit CopyPool(int threads) {
    for (int i = 1; i < threads; ++i) workers_.emplace_back([this] { run(); });
  }
  ~CopyPool() {
    {
      std::lock_guard<std::mutex> lock(mu_);
      stop_ = true;
    }
    cv_.notify_all();
    for (auto& t : workers_) t.join();
  }
  void copy(void* dst, const void* src, int64_t bytes) {
    constexpr int64_t kPart = 2 << 20;
    if (workers_.empty() || bytes <= 2 * kPart) {
      memcpy(dst, src, static_cast<size_t>(bytes));
      return;
    }
    std::lock_guard<std::mutex> one_job(job_mu_);  // one job at a time
    std::unique_lock<std::mutex> lock(mu_);
    done_cv_.wait(lock, [this] { return active_ == 0; });
    dst_ = static_cast<char*>(dst);
    src_ = static_cast<const char*>(src);
    bytes_ = bytes;
    const int64_t want = static_cast<int64_t>(workers_.size()) + 1;
    part_ = round_up((bytes + want - 1) / want, 4096);
    parts_ = (bytes + part_ - 1) / part_;
    next_.store(0);
    finished_ = 0;
    ++generation_;
    lock.unlock();
    cv_.notify_all();
    const int64_t mine = work();
    lock.lock();
    finished_ += mine;
    done_cv_.wait(lock, [this] { return finished_ == parts_ && active_ == 0; });
  }

 private:
  int64_t work() {
    int64_t done = 0;
    for (;;) {
      const int64_t i = next_.fetch_add(1);
      if (i >= parts_) return done;
      const int64_t off = i * part_;
      const int64_t n = bytes_ - off < part_ ? bytes_ - off : part_;
      memcpy(dst_ + off, src_ + off, static_cast<size_t>(n));
      ++done;
    }
  }
  void run() {
    uint64_t seen = 0;
    std::unique_lock<std::mutex> lock(mu_);
    for (;;) {
      cv_.wait(lock, [&] { return stop_ || generation_ != seen; });
      if (stop_) return;
      seen = generation_;
      ++active_;
      lock.unlock();
      const int64_t mine = work();
      lock.lock();
      finished_ += mine;
      --active_;
      done_cv_.notify_all();
    }
  }

  std::vector<std::thread> workers_;
  std::mutex job_mu_;
  std::mutex mu_;
  std::condition_variable cv_, done_cv_;
  bool stop_ = false;
  uint64_t generation_ = 0;
  int active_ = 0;
  char* dst_ = nullptr;
  const char* src_ = nullptr;
  int64_t bytes_ = 0, part_ = 0, parts_ = 0, finished_ = 0;
  std::atomic<int64_t> next_{0};
};

// Chunks of a message: whole layers per chunk when a layer fits in a slot,
// else runs of pages of one layer.
struct Chunking {
  int num_layers = 0;
  int64_t n_pages = 0, page_bytes = 0, layer_bytes = 0;
  int layers_per_chunk = 0;     // > 0: layer chunks
  int64_t pages_per_chunk = 0;  // > 0: page chunks
  int64_t chunks_per_layer = 0;
  int64_t num_chunks = 0;

  struct Chunk {
    int layer, nl;     // first layer and layer count
    int64_t j0, nj;    // first page and page count (all pages for layer chunks)
    int64_t offset, bytes;
  };
  Chunk at(int64_t c) const {
    Chunk k;
    if (layers_per_chunk > 0) {
      k.layer = static_cast<int>(c * layers_per_chunk);
      k.nl = num_layers - k.layer < layers_per_chunk ? num_layers - k.layer : layers_per_chunk;
      k.j0 = 0;
      k.nj = n_pages;
      k.offset = k.layer * layer_bytes;
      k.bytes = k.nl * layer_bytes;
    } else {
      k.layer = static_cast<int>(c / chunks_per_layer);
      k.nl = 1;
      k.j0 = (c % chunks_per_layer) * pages_per_chunk;
      k.nj = n_pages - k.j0 < pages_per_chunk ? n_pages - k.j0 : pages_per_chunk;
      k.offset = k.layer * layer_bytes + k.j0 * page_bytes;
      k.bytes = k.nj * page_bytes;
    }
    return k;
  }
};

int make_chunking(int num_layers, int64_t n_pages, int64_t page_bytes, int64_t slot_bytes, Chunking* out) {
  if (num_layers < 0 || n_pages < 0) return fail(PACE_KV_EINVAL, "channel: negative num_layers or n_pages");
  if (page_bytes <= 0 || page_bytes % 16 != 0)
    return fail(PACE_KV_EINVAL, "channel: page_bytes must be a positive multiple of 16");
  if (page_bytes > slot_bytes)
    return fail(PACE_KV_ERANGE, "channel: a page (%lld bytes) does not fit a slot (%lld bytes)",
                (long long)page_bytes, (long long)slot_bytes);
  if (n_pages > INT64_MAX / page_bytes / (num_layers > 0 ? num_layers : 1))
    return fail(PACE_KV_ERANGE, "channel: payload size overflows");
  Chunking& k = *out;
  k.num_layers = num_layers;
  k.n_pages = n_pages;
  k.page_bytes = page_bytes;
  k.layer_bytes = n_pages * page_bytes;
  if (num_layers == 0 || n_pages == 0) {
    k.num_chunks = 0;
    k.layers_per_chunk = 1;
    return PACE_KV_OK;
  }
  if (k.layer_bytes <= slot_bytes) {
    const int64_t per = slot_bytes / k.layer_bytes;
    k.layers_per_chunk = static_cast<int>(per < num_layers ? per : num_layers);
    k.num_chunks = (num_layers + k.layers_per_chunk - 1) / k.layers_per_chunk;
  } else {
    k.layers_per_chunk = 0;
    k.pages_per_chunk = slot_bytes / page_bytes;
    k.chunks_per_layer = (n_pages + k.pages_per_chunk - 1) / k.pages_per_chunk;
    k.num_chunks = k.chunks_per_layer * num_layers;
  }
  return PACE_KV_OK;
}

// Device-side staging of one endpoint: two device slots and two pinned slots
// of slot_bytes, a copy stream and the events that guard slot reuse.
struct Staging {
  int device = -1;
  char* dev[2] = {nullptr, nullptr};
  char* pinned[2] = {nullptr, nullptr};
  hipStream_t copy = nullptr;
  hipEvent_t filled[2] = {nullptr, nullptr};  // device slot written (pack, or upload)
  hipEvent_t copied[2] = {nullptr, nullptr};  // copy between device and pinned slot finished
  hipEvent_t drained[2] = {nullptr, nullptr}; // receiver: unpack of the device slot finished
  bool ready = false;
};

}  // namespace

struct pace_kv_channel {
  std::string name;
  bool creator = false;
  int fd = -1;
  char* base = nullptr;
  int64_t map_bytes = 0;
  ChannelCtl* ctl = nullptr;
  CopyPool* pool = nullptr;
  std::mutex send_mu;   // one message at a time from this endpoint
  std::mutex recv_mu;
  Staging tx, rx;       // device staging of sends and of receives
  // receiver state of the message in progress
  bool rx_active = false;
  bool rx_device = false;  // its payload is in device slots
  uint64_t rx_msg = 0;
  Chunking rx_chunks;
  int64_t rx_next = 0;
  // Device receive: records read whose slots are not released yet (their
  // unpacks are in flight), oldest first; the next record to read sits
  // rx_held positions past `tail`.  Zero outside pace_kv_channel_recv.
  uint32_t rx_held = 0;
  // this process's view of the device ring
  char* dev_ring = nullptr;
  int dev_device = -1;
  bool dev_local = false;     // allocated by this process: holds a reference in g_rings
  bool dev_imported = false;  // opened from the exported handle (closed at close)
  std::vector<hipEvent_t> dev_packed;    // sender: pack into slot i finished
  std::vector<hipEvent_t> dev_unpacked;  // receiver: unpack out of slot i finished
};

namespace {

char* slot_data(pace_kv_channel* ch, uint32_t idx) {
  return ch->base + ch->ctl->data_offset + static_cast<int64_t>(idx) * ch->ctl->slot_bytes;
}

// Waits until cond() holds.  `word` is the futex word the other side bumps
// when it may have made cond() true; closing the channel also wakes it.  The
// peer process is checked at every wake-up (at least every 10 ms), so a wait
// on a peer that died ends then rather than at the deadline.
// A sender's wait (closed_first) fails on a closed channel even when cond()
// holds, so nothing is published into a channel either side has closed; a
// receiver's wait still takes records published before the sender closed.
// The first kSpinUs of a wait poll without sleeping: the peer's next record
// often follows within one chunk's copy time, and a futex wake-up would add
// its own latency to every hand-over.
constexpr int kSpinUs = 200;

template <class Cond>
int wait_for(pace_kv_channel* ch, std::atomic<uint32_t>* word, const ProcessId& peer, Cond cond,
             int timeout_ms, const char* what, bool closed_first = false) {
  using clock = std::chrono::steady_clock;
  const auto start = clock::now();
  const auto deadline = start + std::chrono::milliseconds(timeout_ms < 0 ? 0 : timeout_ms);
  const auto spin_end = std::min(deadline, start + std::chrono::microseconds(kSpinUs));
  bool spinning = true;
  for (int spin = 0;; ++spin) {
    const uint32_t seen = word->load(std::memory_order_acquire);
    const bool closed = ch->ctl->closed.load(std::memory_order_acquire) != 0;
    if (!(closed && closed_first) && cond()) return PACE_KV_OK;
    if (closed)
      return fail(PACE_KV_ECLOSED, "channel %s: closed while waiting for %s", ch->name.c_str(), what);
    if (spinning) {
      __builtin_ia32_pause();
      if ((spin & 63) != 63 || clock::now() < spin_end) continue;
      spinning = false;
    }
    if (role_gone(peer))
      return fail(PACE_KV_ECLOSED, "channel %s: the peer process %d exited while this side waited for %s",
                  ch->name.c_str(), peer.pid.load(), what);
    const auto left = std::chrono::duration_cast<std::chrono::microseconds>(deadline - clock::now()).count();
    if (left <= 0)
      return fail(PACE_KV_ETIMEDOUT, "channel %s: timed out after %d ms waiting for %s", ch->name.c_str(),
                  timeout_ms, what);
    const long us = left < 10000 ? left : 10000;
    timespec ts{us / 1000000, (us % 1000000) * 1000};
    (void)futex(word, FUTEX_WAIT, seen, &ts);
  }
}

// Sender: waits for a free slot and returns its index.
int acquire_slot(pace_kv_channel* ch, int timeout_ms, uint32_t* idx) {
  ChannelCtl* c = ch->ctl;
  const uint32_t h = c->head.load(std::memory_order_relaxed);
  PACE_KV_TRY(wait_for(ch, &c->tail, c->receiver,
                       [&] { return h - c->tail.load(std::memory_order_acquire) < c->num_slots; },
                       timeout_ms, "a free slot", true));
  *idx = h % c->num_slots;
  return PACE_KV_OK;
}

void publish(pace_kv_channel* ch) {
  ChannelCtl* c = ch->ctl;
  c->head.store(c->head.load(std::memory_order_relaxed) + 1, std::memory_order_release);
  wake_all(&c->head);
}

// Receiver: waits for the next record and returns its slot index.
int next_record(pace_kv_channel* ch, int timeout_ms, uint32_t* idx, const char* what) {
  ChannelCtl* c = ch->ctl;
  take_role(c->receiver);
  const uint32_t t = c->tail.load(std::memory_order_relaxed) + ch->rx_held;
  const uint64_t msg = ch->rx_msg;
  const bool active = ch->rx_active;
  PACE_KV_TRY(wait_for(ch, &c->head, c->sender,
                       [&] {
                         return c->head.load(std::memory_order_acquire) != t ||
                                (active && c->aborted_msg.load(std::memory_order_acquire) == msg);
                       },
                       timeout_ms, what));
  if (c->head.load(std::memory_order_acquire) == t) {
    ch->rx_active = false;
    return fail(PACE_KV_ESTATE, "channel %s: the sender abandoned message %llu", ch->name.c_str(),
                (unsigned long long)msg);
  }
  *idx = t % c->num_slots;
  return PACE_KV_OK;
}

void release(pace_kv_channel* ch) {
  ChannelCtl* c = ch->ctl;
  c->tail.store(c->tail.load(std::memory_order_relaxed) + 1, std::memory_order_release);
  wake_all(&c->tail);
}

int check_name(const char* name) {
  if (name == nullptr || name[0] == '\0') return fail(PACE_KV_EINVAL, "channel: empty name");
  if (strlen(name) > kNameMax) return fail(PACE_KV_EINVAL, "channel: name longer than %d bytes", kNameMax);
  for (const char* p = name; *p; ++p)
    if (*p == '/') return fail(PACE_KV_EINVAL, "channel: name must not contain '/'");
  return PACE_KV_OK;
}

int map_channel(pace_kv_channel* ch, int64_t bytes) {
  void* p = mmap(nullptr, static_cast<size_t>(bytes), PROT_READ | PROT_WRITE, MAP_SHARED, ch->fd, 0);
  if (p == MAP_FAILED) return fail(PACE_KV_ESTATE, "channel %s: mmap failed: %s", ch->name.c_str(), strerror(errno));
  ch->base = static_cast<char*>(p);
  ch->map_bytes = bytes;
  ch->ctl = reinterpret_cast<ChannelCtl*>(p);
  return PACE_KV_OK;
}

void free_staging(Staging& s) {
  for (int i = 0; i < 2; ++i) {
    if (s.dev[i]) (void)hipFree(s.dev[i]);
    if (s.pinned[i]) (void)hipHostFree(s.pinned[i]);
    if (s.filled[i]) (void)hipEventDestroy(s.filled[i]);
    if (s.copied[i]) (void)hipEventDestroy(s.copied[i]);
    if (s.drained[i]) (void)hipEventDestroy(s.drained[i]);
  }
  if (s.copy) (void)hipStreamDestroy(s.copy);
  s = Staging();
}

// Process-local registry of the device rings this process allocated, by the
// inode of their channel's shared-memory object: an endpoint that opens a
// channel created in its own process uses the ring's address directly, since
// an exported handle is not opened in the process that exported it.  Each
// endpoint of this process holds one reference to the ring while it is open
// (the creator from its creation, another endpoint from its open), and the
// ring is freed when the last of them closes, whichever closes first.
struct RingRef {
  char* ring = nullptr;
  int device = -1;  // the device it was allocated on
  int refs = 0;
};
std::mutex g_rings_mu;
std::map<uint64_t, RingRef> g_rings;

uint64_t shm_inode(int fd) {
  struct stat st;
  return fd >= 0 && fstat(fd, &st) == 0 ? static_cast<uint64_t>(st.st_ino) : 0;
}

void free_device_ring(pace_kv_channel* ch) {
  for (std::vector<hipEvent_t>* v : {&ch->dev_packed, &ch->dev_unpacked}) {
    for (hipEvent_t e : *v) {
      (void)hipEventSynchronize(e);
      (void)hipEventDestroy(e);
    }
    v->clear();
  }
  if (ch->dev_ring != nullptr) {
    if (ch->dev_imported) (void)hipIpcCloseMemHandle(ch->dev_ring);
    if (ch->dev_local) {
      char* last = nullptr;
      {
        std::lock_guard<std::mutex> lock(g_rings_mu);
        auto it = g_rings.find(shm_inode(ch->fd));
        if (it != g_rings.end() && it->second.ring == ch->dev_ring && --it->second.refs == 0) {
          last = it->second.ring;
          g_rings.erase(it);
        }
      }
      if (last != nullptr) (void)hipFree(last);
    }
  }
  ch->dev_ring = nullptr;
  ch->dev_imported = ch->dev_local = false;
}

void destroy(pace_kv_channel* ch) {
  free_device_ring(ch);
  free_staging(ch->tx);
  free_staging(ch->rx);
  delete ch->pool;
  if (ch->base) munmap(ch->base, static_cast<size_t>(ch->map_bytes));
  if (ch->creator && ch->fd >= 0) {
    // The name is removed only while it still names this channel's object:
    // after an unlink and a new create under the same name it names another.
    const std::string shm_name = "/" + ch->name;
    const int cur = shm_open(shm_name.c_str(), O_RDONLY, 0);
    struct stat mine, now;
    if (cur >= 0 && fstat(ch->fd, &mine) == 0 && fstat(cur, &now) == 0 && mine.st_ino == now.st_ino &&
        mine.st_dev == now.st_dev)
      shm_unlink(shm_name.c_str());
    if (cur >= 0) close(cur);
  }
  if (ch->fd >= 0) close(ch->fd);
  delete ch;
}

int new_endpoint(const char* name, int copy_threads, pace_kv_channel** out) {
  if (out == nullptr) return fail(PACE_KV_EINVAL, "channel: out is NULL");
  *out = nullptr;
  PACE_KV_TRY(check_name(name));
  if (copy_threads < 1 || copy_threads > 64) return fail(PACE_KV_EINVAL, "channel: copy_threads must be in [1, 64]");
  pace_kv_channel* ch = new pace_kv_channel();
  ch->name = name;
  *out = ch;
  return PACE_KV_OK;
}

// Device staging of one direction of an endpoint, created on its first
// device transfer.
int staging_ready(pace_kv_channel* ch, Staging& s) {
  int dev = -1;
  PACE_KV_TRY(hip_status(hipGetDevice(&dev), "hipGetDevice"));
  if (s.ready) {
    if (dev != s.device)
      return fail(PACE_KV_ESTATE, "channel %s: staging lives on device %d, device %d is current",
                  ch->name.c_str(), s.device, dev);
    return PACE_KV_OK;
  }
  const size_t bytes = static_cast<size_t>(ch->ctl->slot_bytes);
  hipError_t e = hipSuccess;
  for (int i = 0; i < 2 && e == hipSuccess; ++i) {
    e = hipMalloc(reinterpret_cast<void**>(&s.dev[i]), bytes);
    if (e == hipSuccess) e = hipHostMalloc(reinterpret_cast<void**>(&s.pinned[i]), bytes, hipHostMallocDefault);
    if (e == hipSuccess) e = hipEventCreateWithFlags(&s.filled[i], hipEventDisableTiming);
    if (e == hipSuccess) e = hipEventCreateWithFlags(&s.copied[i], hipEventDisableTiming);
    if (e == hipSuccess) e = hipEventCreateWithFlags(&s.drained[i], hipEventDisableTiming);
  }
  if (e == hipSuccess) e = hipStreamCreateWithFlags(&s.copy, hipStreamNonBlocking);
  if (e != hipSuccess) {
    free_staging(s);
    return hip_status(e, "channel staging");
  }
  s.device = dev;
  s.ready = true;
  return PACE_KV_OK;
}

// Publishes the header record of a new message; returns its id.
int send_header(pace_kv_channel* ch, int num_layers, int64_t n_pages, int64_t page_bytes, const void* meta,
                int64_t meta_bytes, int timeout_ms, uint64_t* msg_id, int32_t flags = 0) {
  ChannelCtl* c = ch->ctl;
  take_role(c->sender);
  if (meta_bytes < 0 || (meta_bytes > 0 && meta == nullptr))
    return fail(PACE_KV_EINVAL, "channel: bad metadata");
  if (meta_bytes > c->slot_bytes)
    return fail(PACE_KV_ERANGE, "channel: metadata (%lld bytes) does not fit a slot (%lld bytes)",
                (long long)meta_bytes, (long long)c->slot_bytes);
  uint32_t idx = 0;
  PACE_KV_TRY(acquire_slot(ch, timeout_ms, &idx));
  const uint64_t id = c->next_msg_id.fetch_add(1) + 1;
  if (meta_bytes > 0) memcpy(slot_data(ch, idx), meta, static_cast<size_t>(meta_bytes));
  SlotRecord& r = c->slots[idx];
  r.kind = kHeader;
  r.chunk = 0;
  r.msg_id = id;
  r.offset = 0;
  r.bytes = meta_bytes;
  r.n_pages = n_pages;
  r.page_bytes = page_bytes;
  r.num_layers = num_layers;
  r.flags = flags;
  publish(ch);
  if (msg_id) *msg_id = id;
  return PACE_KV_OK;
}

int send_chunk_from(pace_kv_channel* ch, uint64_t id, int64_t c, const Chunking::Chunk& k, const char* src,
                    int timeout_ms) {
  uint32_t idx = 0;
  PACE_KV_TRY(acquire_slot(ch, timeout_ms, &idx));
  ch->pool->copy(slot_data(ch, idx), src, k.bytes);
  SlotRecord& r = ch->ctl->slots[idx];
  r.kind = kData;
  r.chunk = static_cast<uint32_t>(c);
  r.msg_id = id;
  r.offset = k.offset;
  r.bytes = k.bytes;
  publish(ch);
  return PACE_KV_OK;
}

// Marks a message whose chunks will not all arrive, so that the receiver
// fails at once instead of waiting out its deadline.
int abandon(pace_kv_channel* ch, uint64_t id, int rc) {
  ch->ctl->aborted_msg.store(id, std::memory_order_release);
  wake_all(&ch->ctl->head);
  return rc;
}

// Sender: nothing goes into a channel that either side has closed.
int check_open(pace_kv_channel* ch) {
  if (ch->ctl->closed.load(std::memory_order_acquire))
    return fail(PACE_KV_ECLOSED, "channel %s is closed", ch->name.c_str());
  return PACE_KV_OK;
}

int check_rx_shape(pace_kv_channel* ch, int num_layers, int64_t n_pages, int64_t page_bytes) {
  if (!ch->rx_active)
    return fail(PACE_KV_ESTATE, "channel %s: no message header received", ch->name.c_str());
  const Chunking& k = ch->rx_chunks;
  if (num_layers != k.num_layers || n_pages != k.n_pages || page_bytes != k.page_bytes)
    return fail(PACE_KV_EINVAL,
                "channel %s: message %llu holds %d layers x %lld pages x %lld bytes, the receiver "
                "asked for %d x %lld x %lld", ch->name.c_str(), (unsigned long long)ch->rx_msg,
                k.num_layers, (long long)k.n_pages, (long long)k.page_bytes, num_layers,
                (long long)n_pages, (long long)page_bytes);
  return PACE_KV_OK;
}

// Receiver: waits for chunk rx_next of the current message and checks it.
int next_chunk(pace_kv_channel* ch, int timeout_ms, uint32_t* idx, Chunking::Chunk* k) {
  PACE_KV_TRY(next_record(ch, timeout_ms, idx, "a payload chunk"));
  const SlotRecord& r = ch->ctl->slots[*idx];
  *k = ch->rx_chunks.at(ch->rx_next);
  const uint32_t kind = ch->rx_device ? kDevData : kData;
  if (r.kind != kind || r.msg_id != ch->rx_msg || r.chunk != static_cast<uint32_t>(ch->rx_next) ||
      r.offset != k->offset || r.bytes != k->bytes) {
    ch->rx_active = false;
    return fail(PACE_KV_ESTATE, "channel %s: expected chunk %lld of message %llu, found a record of "
                "kind %u for message %llu chunk %u", ch->name.c_str(), (long long)ch->rx_next,
                (unsigned long long)ch->rx_msg, r.kind, (unsigned long long)r.msg_id, r.chunk);
  }
  return PACE_KV_OK;
}

void finish_chunk(pace_kv_channel* ch) {
  release(ch);
  if (++ch->rx_next == ch->rx_chunks.num_chunks) ch->rx_active = false;
}

// ------------------------------------------------------------ page ids

// The page ids of a send or a receive: device memory, or host memory of at
// most PACE_KV_INLINE_IDS entries, which each launch carries in its kernel
// arguments (no upload has to precede the first pack or unpack).
struct PageIds {
  const int32_t* ptr = nullptr;
  bool host = false;
};

int classify_ids(const int32_t* ids, int64_t n, PageIds* out) {
  out->ptr = ids;
  hipPointerAttribute_t attr;
  memset(&attr, 0, sizeof(attr));
  const hipError_t e = hipPointerGetAttributes(&attr, ids);
  if (e != hipSuccess) (void)hipGetLastError();  // pageable host memory is not known to the runtime
  out->host = e != hipSuccess || (attr.type != hipMemoryTypeDevice && attr.type != hipMemoryTypeManaged);
  if (out->host && n > PACE_KV_INLINE_IDS)
    return fail(PACE_KV_ERANGE, "channel: %lld page ids in host memory (at most %d; pass device ids)",
                (long long)n, PACE_KV_INLINE_IDS);
  return PACE_KV_OK;
}

// pack of pages [j0, j0 + nj) of layers [0, nl) into out[l][j - j0]
// (layer stride `stride`), as pace_kv_pack.
int pack_pages(const void* const* src_layers, int nl, int64_t pool_pages, const PageIds& ids, int64_t j0,
               int64_t nj, int64_t page_bytes, char* out, int64_t stride, int32_t* err, hipStream_t stream) {
  if (!ids.host)
    return pace_kv_pack(src_layers, nl, pool_pages, ids.ptr + j0, nj, page_bytes, out, stride, err, stream);
  std::vector<const char*> buf(static_cast<size_t>(nl));
  pace_kv::buffer_layers(out, stride, nl, buf.data());
  return pace_kv::launch_page_copy(
      pace_kv::Side{reinterpret_cast<const char* const*>(src_layers), nullptr, pool_pages},
      pace_kv::Side{buf.data(), nullptr, nj}, nl, nj, page_bytes, err, stream, ids.ptr + j0, nullptr,
      pace_kv::StorePolicy::kPack);
}

// unpack of in[l][j - j0] into pages [j0, j0 + nj) of layers [0, nl), as
// pace_kv_unpack.
int unpack_pages(const char* in, int64_t stride, void* const* dst_layers, int nl, int64_t pool_pages,
                 const PageIds& ids, int64_t j0, int64_t nj, int64_t page_bytes, int32_t* err, hipStream_t stream) {
  if (!ids.host)
    return pace_kv_unpack(in, stride, dst_layers, nl, pool_pages, ids.ptr + j0, nj, page_bytes, err, stream);
  std::vector<const char*> buf(static_cast<size_t>(nl));
  pace_kv::buffer_layers(in, stride, nl, buf.data());
  return pace_kv::launch_page_copy(pace_kv::Side{buf.data(), nullptr, nj},
                                   pace_kv::Side{reinterpret_cast<const char* const*>(dst_layers), nullptr,
                                                 pool_pages},
                                   nl, nj, page_bytes, err, stream, nullptr, ids.ptr + j0);
}

// ------------------------------------------------------------ device ring

// PCI bus ids of this process's devices, looked up once per device: a
// device ordinal names the same GPU for the whole process.
constexpr int kMaxBusDevices = 64;
std::mutex g_bus_mu;
char g_bus_ids[kMaxBusDevices][kBusIdBytes];
bool g_bus_known[kMaxBusDevices];

int bus_id_of(int dev, char* bus) {
  if (dev >= 0 && dev < kMaxBusDevices) {
    std::lock_guard<std::mutex> lock(g_bus_mu);
    if (!g_bus_known[dev]) {
      PACE_KV_TRY(hip_status(hipDeviceGetPCIBusId(g_bus_ids[dev], kBusIdBytes, dev), "hipDeviceGetPCIBusId"));
      g_bus_ids[dev][kBusIdBytes - 1] = '\0';
      g_bus_known[dev] = true;
    }
    memcpy(bus, g_bus_ids[dev], kBusIdBytes);
    return PACE_KV_OK;
  }
  return hip_status(hipDeviceGetPCIBusId(bus, kBusIdBytes, dev), "hipDeviceGetPCIBusId");
}

int current_bus_id(int* dev, char* bus) {
  PACE_KV_TRY(hip_status(hipGetDevice(dev), "hipGetDevice"));
  return bus_id_of(*dev, bus);
}

// Whether the channel has a device ring on the current GPU.
int device_ring_here(pace_kv_channel* ch, bool* here) {
  *here = false;
  if (ch->ctl->dev_slot_bytes <= 0) return PACE_KV_OK;
  int dev = -1;
  char bus[kBusIdBytes] = {0};
  PACE_KV_TRY(current_bus_id(&dev, bus));
  *here = strncmp(bus, ch->ctl->dev_bus_id, kBusIdBytes) == 0;
  return PACE_KV_OK;
}

constexpr uint64_t kNoGpu = ~uint64_t(0);

// Receiver: records the GPU current in this thread (or that there is none)
// for the sender's choice of ring.
void record_receiver_gpu(pace_kv_channel* ch) {
  uint64_t words[kBusIdBytes / 8] = {0};
  int dev = -1;
  char bus[kBusIdBytes] = {0};
  if (hipGetDevice(&dev) == hipSuccess && bus_id_of(dev, bus) == PACE_KV_OK) {
    bus[kBusIdBytes - 1] = '\0';
    memcpy(words, bus, sizeof(words));
  } else {
    (void)hipGetLastError();
    words[0] = kNoGpu;
  }
  for (int i = 0; i < kBusIdBytes / 8; ++i) ch->ctl->rx_bus_id[i].store(words[i], std::memory_order_relaxed);
}

// Sender: whether the receiver can take a message in device slots: its GPU
// is not known yet, or it is the ring's GPU.
bool receiver_on_ring_gpu(pace_kv_channel* ch) {
  uint64_t words[kBusIdBytes / 8];
  bool unknown = true;
  for (int i = 0; i < kBusIdBytes / 8; ++i) {
    words[i] = ch->ctl->rx_bus_id[i].load(std::memory_order_relaxed);
    unknown = unknown && words[i] == 0;
  }
  if (unknown) return true;
  if (words[0] == kNoGpu) return false;
  char bus[kBusIdBytes];
  memcpy(bus, words, sizeof(bus));
  bus[kBusIdBytes - 1] = '\0';
  return strncmp(bus, ch->ctl->dev_bus_id, kBusIdBytes) == 0;
}

int make_slot_events(pace_kv_channel* ch) {
  const size_t n = ch->ctl->num_slots;
  for (std::vector<hipEvent_t>* v : {&ch->dev_packed, &ch->dev_unpacked}) {
    while (v->size() < n) {
      hipEvent_t e = nullptr;
      PACE_KV_TRY(hip_status(hipEventCreateWithFlags(&e, hipEventDisableTiming), "channel slot event"));
      v->push_back(e);
    }
  }
  return PACE_KV_OK;
}

// Maps the device ring into this process on the current GPU (once).
int ring_ready(pace_kv_channel* ch) {
  ChannelCtl* c = ch->ctl;
  if (c->dev_slot_bytes <= 0) return fail(PACE_KV_ESTATE, "channel %s has no device ring", ch->name.c_str());
  int dev = -1;
  char bus[kBusIdBytes] = {0};
  PACE_KV_TRY(current_bus_id(&dev, bus));
  if (strncmp(bus, c->dev_bus_id, kBusIdBytes) != 0)
    return fail(PACE_KV_ESTATE, "channel %s: its device ring is on the GPU at %.64s, the current GPU is at %s",
                ch->name.c_str(), c->dev_bus_id, bus);
  if (ch->dev_imported && c->creator_closed.load(std::memory_order_acquire))
    return fail(PACE_KV_ECLOSED, "channel %s: the process that created its device ring has closed it",
                ch->name.c_str());
  if (ch->dev_ring != nullptr) {
    if (dev != ch->dev_device)
      return fail(PACE_KV_ESTATE, "channel %s: device ring mapped on device %d, device %d is current",
                  ch->name.c_str(), ch->dev_device, dev);
    return make_slot_events(ch);
  }
  void* p = nullptr;
  if (c->dev_owner_pid == static_cast<int32_t>(getpid())) {
    std::lock_guard<std::mutex> lock(g_rings_mu);
    auto it = g_rings.find(shm_inode(ch->fd));
    if (it == g_rings.end())
      return fail(PACE_KV_ESTATE, "channel %s: its device ring was allocated by this process and is freed",
                  ch->name.c_str());
    p = it->second.ring;
    ++it->second.refs;
    ch->dev_local = true;
  } else {
    if (c->creator_closed.load(std::memory_order_acquire))
      return fail(PACE_KV_ECLOSED, "channel %s: the process that created its device ring has closed it",
                  ch->name.c_str());
    PACE_KV_TRY(hip_status(hipIpcOpenMemHandle(&p, c->dev_handle, hipIpcMemLazyEnablePeerAccess),
                           "hipIpcOpenMemHandle (channel device ring)"));
    ch->dev_imported = true;
  }
  ch->dev_ring = static_cast<char*>(p);
  ch->dev_device = dev;
  return make_slot_events(ch);
}

// A not-ready query is no error: it must not be left as the thread's last
// HIP error for the caller's next error check to find.
void clear_not_ready() {
  if (hipPeekAtLastError() == hipErrorNotReady) (void)hipGetLastError();
}

// Waits for `e` by polling it, so that the host sees the completion within a
// poll rather than after a blocking wait's wake-up (the hand-overs of the
// device ring are on the path of every message).
hipError_t poll_event(hipEvent_t e) {
  for (;;) {
    const hipError_t q = hipEventQuery(e);
    if (q != hipErrorNotReady) {
      clear_not_ready();
      return q;
    }
    __builtin_ia32_pause();
  }
}

char* dev_slot(pace_kv_channel* ch, uint32_t idx) {
  return ch->dev_ring + static_cast<int64_t>(idx) * ch->ctl->dev_slot_bytes;
}

// Sender: waits until the record at position `pos` (head plus the records
// reserved but not yet published) has a free slot.
int acquire_slot_at(pace_kv_channel* ch, uint32_t pos, int timeout_ms, uint32_t* idx) {
  ChannelCtl* c = ch->ctl;
  PACE_KV_TRY(wait_for(ch, &c->tail, c->receiver,
                       [&] { return pos - c->tail.load(std::memory_order_acquire) < c->num_slots; },
                       timeout_ms, "a free slot", true));
  *idx = pos % c->num_slots;
  return PACE_KV_OK;
}

// Sender: publishes device chunk `c` of message `id` once its pack into slot
// idx has finished.
int publish_dev_chunk(pace_kv_channel* ch, uint64_t id, int64_t c, const Chunking::Chunk& k, uint32_t idx) {
  PACE_KV_TRY(hip_status(poll_event(ch->dev_packed[idx]), "channel pack into the device ring"));
  SlotRecord& r = ch->ctl->slots[idx];
  r.kind = kDevData;
  r.chunk = static_cast<uint32_t>(c);
  r.msg_id = id;
  r.offset = k.offset;
  r.bytes = k.bytes;
  publish(ch);
  return PACE_KV_OK;
}

// Sender: gives up a device message after packs into the ring may have been
// enqueued.  An unpublished slot is reserved again by the next record at its
// position, whose pack may run on another stream: the packs enqueued here
// finish before this returns, so no late write lands in a slot that a later
// message owns.
int abandon_device(pace_kv_channel* ch, uint64_t id, int rc, hipStream_t stream) {
  (void)hipStreamSynchronize(stream);
  return abandon(ch, id, rc);
}

// Sender: packs every chunk straight into a device slot.  Chunk c is packed
// before chunk c-1 is published, so the GPU has the next pack queued while
// this thread waits for the previous one; at most one slot is reserved and
// unpublished, so the receiver can always drain what precedes it.
int send_device(pace_kv_channel* ch, const void* const* src_layers, int64_t pool_pages,
                const PageIds& page_ids, const Chunking& k, uint64_t id, int timeout_ms, hipStream_t stream) {
  const uint32_t first = ch->ctl->head.load(std::memory_order_relaxed);
  uint32_t prev = 0;
  for (int64_t c = 0; c < k.num_chunks; ++c) {
    const Chunking::Chunk ck = k.at(c);
    uint32_t idx = 0;
    int rc = acquire_slot_at(ch, first + static_cast<uint32_t>(c), timeout_ms, &idx);
    if (rc == PACE_KV_OK) {
      const int64_t stride = k.layers_per_chunk > 0 ? k.layer_bytes : ck.bytes;
      rc = pack_pages(src_layers + ck.layer, ck.nl, pool_pages, page_ids, ck.j0, ck.nj, k.page_bytes,
                      dev_slot(ch, idx), stride, nullptr, stream);
    }
    if (rc == PACE_KV_OK) rc = hip_status(hipEventRecord(ch->dev_packed[idx], stream), "channel send record");
    if (rc == PACE_KV_OK && c > 0) rc = publish_dev_chunk(ch, id, c - 1, k.at(c - 1), prev);
    if (rc) return abandon_device(ch, id, rc, stream);
    prev = idx;
  }
  if (k.num_chunks > 0) {
    const int rc = publish_dev_chunk(ch, id, k.num_chunks - 1, k.at(k.num_chunks - 1), prev);
    if (rc) return abandon_device(ch, id, rc, stream);
  }
  return PACE_KV_OK;
}

// Receiver: a device chunk whose copy to host memory failed still releases
// its slot (the copy is synchronous), and the rest of its message is dropped
// by the next header receive.
int fail_rx(pace_kv_channel* ch, int rc) {
  ch->rx_active = false;
  release(ch);
  return rc;
}

// Receiver: releases the oldest held slot once its unpack has finished.
int release_held(pace_kv_channel* ch, bool wait) {
  const uint32_t idx = (ch->ctl->tail.load(std::memory_order_relaxed)) % ch->ctl->num_slots;
  hipEvent_t e = ch->dev_unpacked[idx];
  int rc = PACE_KV_OK;
  if (wait) {
    rc = hip_status(poll_event(e), "channel unpack out of the device ring");
  } else {
    const hipError_t q = hipEventQuery(e);
    if (q == hipErrorNotReady) {
      clear_not_ready();
      return PACE_KV_OK;  // still reading: keep the slot
    }
    rc = hip_status(q, "channel unpack out of the device ring");
  }
  if (rc) return rc;
  --ch->rx_held;
  release(ch);
  return PACE_KV_OK;
}

// Receiver: gives every held slot back, after the unpacks enqueued on
// `stream` have stopped reading them; returns rc.
int release_all_held(pace_kv_channel* ch, int rc, hipStream_t stream) {
  if (ch->rx_held > 0) (void)hipStreamSynchronize(stream);
  while (ch->rx_held > 0) {
    --ch->rx_held;
    release(ch);
  }
  return rc;
}

// Receiver: a chunk read but not unpacked (its unpack could not be
// enqueued) also goes back, and the rest of the message is dropped by the
// next header receive.
int fail_rx_device(pace_kv_channel* ch, int rc, hipStream_t stream) {
  release_all_held(ch, rc, stream);
  (void)hipStreamSynchronize(stream);
  release(ch);
  ch->rx_active = false;
  return rc;
}

// Receiver: unpacks every chunk straight out of its device slot.  A slot
// goes back to the sender once its unpack has finished, in ring order.
// While it waits for the next chunk, the receiver keeps at most
// num_slots - 2 slots whose unpacks are still in flight, so that its GPU
// queue does not drain between chunks; the sender, which reserves one slot
// beyond the chunk it publishes, can then always publish the chunk waited for.
// With two slots every unpack finishes before the next wait.
int recv_device(pace_kv_channel* ch, void* const* dst_layers, int64_t pool_pages, const PageIds& page_ids,
                int32_t* err_count, int timeout_ms, hipStream_t stream) {
  PACE_KV_TRY(ring_ready(ch));
  const Chunking k = ch->rx_chunks;
  const uint32_t max_held = ch->ctl->num_slots - 2;
  while (ch->rx_active) {
    // release what has finished, and enough to stay within max_held
    while (ch->rx_held > 0) {
      const uint32_t before = ch->rx_held;
      const int rc = release_held(ch, ch->rx_held > max_held);
      if (rc) {
        ch->rx_active = false;
        return release_all_held(ch, rc, stream);
      }
      if (ch->rx_held == before) break;   // the oldest is still in flight
    }
    uint32_t idx = 0;
    Chunking::Chunk ck;
    // A failed wait (deadline, closed channel, abandoned or unexpected
    // record) leaves rx_active as next_chunk set it: after a deadline the
    // message is still pending and can be received or drained again.
    int rc = next_chunk(ch, timeout_ms, &idx, &ck);
    if (rc) return release_all_held(ch, rc, stream);
    const int64_t stride = k.layers_per_chunk > 0 ? k.layer_bytes : ck.bytes;
    rc = unpack_pages(dev_slot(ch, idx), stride, dst_layers + ck.layer, ck.nl, pool_pages, page_ids, ck.j0,
                      ck.nj, k.page_bytes, err_count, stream);
    if (rc == PACE_KV_OK) rc = hip_status(hipEventRecord(ch->dev_unpacked[idx], stream), "channel recv record");
    if (rc) return fail_rx_device(ch, rc, stream);
    ++ch->rx_held;
    if (++ch->rx_next == k.num_chunks) ch->rx_active = false;
  }
  // the message is read: its slots go back as their unpacks finish
  while (ch->rx_held > 0) {
    const int rc = release_held(ch, true);
    if (rc) return release_all_held(ch, rc, stream);
  }
  return PACE_KV_OK;
}

// An endpoint opened in the process that created the channel's device ring
// shares that ring from the start (one more reference), so that the ring
// outlives the creator's endpoint while this one is open.
void take_local_ring(pace_kv_channel* ch) {
  ChannelCtl* c = ch->ctl;
  if (c->dev_slot_bytes <= 0 || c->dev_owner_pid != static_cast<int32_t>(getpid())) return;
  std::lock_guard<std::mutex> lock(g_rings_mu);
  auto it = g_rings.find(shm_inode(ch->fd));
  if (it == g_rings.end()) return;
  ++it->second.refs;
  ch->dev_ring = it->second.ring;
  ch->dev_device = it->second.device;
  ch->dev_local = true;
}

// Creates the ring (and, with dev_slot_bytes > 0, the device ring on the
// current GPU); the magic goes in last.
int create_channel(const char* name, int64_t slot_bytes, int num_slots, int copy_threads, int64_t dev_slot_bytes,
                   pace_kv_channel** out) {
  PACE_KV_TRY(new_endpoint(name, copy_threads, out));
  pace_kv_channel* ch = *out;
  *out = nullptr;
  if (slot_bytes <= 0 || slot_bytes % 4096 != 0) {
    delete ch;
    return fail(PACE_KV_EINVAL, "channel: slot_bytes must be a positive multiple of 4096");
  }
  if (!valid_slot_count(num_slots)) {
    delete ch;
    return fail(PACE_KV_EINVAL, "channel: num_slots must be a power of two in [2, %d] (got %d)", kMaxSlots,
                num_slots);
  }
  if (slot_bytes > (INT64_MAX / 2) / num_slots) {
    delete ch;
    return fail(PACE_KV_ERANGE, "channel: ring size overflows");
  }
  if (dev_slot_bytes < 0 || dev_slot_bytes % 4096 != 0) {
    delete ch;
    return fail(PACE_KV_EINVAL, "channel: dev_slot_bytes must be a non-negative multiple of 4096");
  }
  if (dev_slot_bytes > kMaxDeviceRing / num_slots) {
    delete ch;
    return fail(PACE_KV_ERANGE, "channel: a device ring of %d x %lld bytes exceeds %lld bytes", num_slots,
                (long long)dev_slot_bytes, (long long)kMaxDeviceRing);
  }
  const int64_t data_offset = round_up(static_cast<int64_t>(sizeof(ChannelCtl)), 1 << 21);
  const int64_t total = data_offset + slot_bytes * num_slots;
  ch->fd = shm_open(("/" + ch->name).c_str(), O_CREAT | O_EXCL | O_RDWR, 0600);
  if (ch->fd < 0) {
    const int err = errno;
    delete ch;
    return fail(err == EEXIST ? PACE_KV_ESTATE : PACE_KV_EINVAL, "channel %s: shm_open failed: %s", name,
                strerror(err));
  }
  ch->creator = true;
  ch->pool = new CopyPool(copy_threads);
  if (ftruncate(ch->fd, total) != 0) {
    const int err = errno;
    destroy(ch);
    return fail(PACE_KV_ENOMEM, "channel %s: cannot size the ring to %lld bytes: %s", name, (long long)total,
                strerror(err));
  }
  int rc = map_channel(ch, total);
  if (rc) {
    destroy(ch);
    return rc;
  }
  ChannelCtl* c = ch->ctl;
  c->version = kVersion;
  c->num_slots = static_cast<uint32_t>(num_slots);
  c->slot_bytes = slot_bytes;
  c->data_offset = data_offset;
  c->total_bytes = total;
  c->head.store(0);
  c->tail.store(0);
  c->closed.store(0);
  c->next_msg_id.store(0);
  c->aborted_msg.store(0);
  for (ProcessId* r : {&c->sender, &c->receiver}) {
    r->pid.store(0);
    r->pidns.store(0);
    r->start.store(0);
  }
  c->dev_slot_bytes = 0;
  c->dev_owner_pid = 0;
  c->creator_closed.store(0);
  for (auto& w : c->rx_bus_id) w.store(0);
  if (dev_slot_bytes > 0) {
    int dev = -1;
    void* ring = nullptr;
    rc = current_bus_id(&dev, c->dev_bus_id);
    if (rc == PACE_KV_OK)
      rc = hip_status(hipMalloc(&ring, static_cast<size_t>(dev_slot_bytes * num_slots)), "channel device ring");
    if (rc == PACE_KV_OK) {
      ch->dev_ring = static_cast<char*>(ring);
      ch->dev_device = dev;
      ch->dev_local = true;
      std::lock_guard<std::mutex> lock(g_rings_mu);
      g_rings[shm_inode(ch->fd)] = RingRef{ch->dev_ring, dev, 1};
    }
    if (rc == PACE_KV_OK)
      rc = hip_status(hipIpcGetMemHandle(&c->dev_handle, ring), "hipIpcGetMemHandle (channel device ring)");
    if (rc == PACE_KV_OK) {
      c->dev_slot_bytes = dev_slot_bytes;
      c->dev_owner_pid = static_cast<int32_t>(getpid());
      rc = make_slot_events(ch);
    }
    if (rc) {
      destroy(ch);
      return rc;
    }
  }
  std::atomic_thread_fence(std::memory_order_release);
  // The magic goes in last: an opener that sees it sees a complete block.
  __atomic_store_n(&c->magic, kMagic, __ATOMIC_RELEASE);
  *out = ch;
  return PACE_KV_OK;
}

}  // namespace

extern "C" {

int pace_kv_channel_create(const char* name, int64_t slot_bytes, int num_slots, int copy_threads,
                           pace_kv_channel** out) {
  return create_channel(name, slot_bytes, num_slots, copy_threads, 0, out);
}

int pace_kv_channel_create_device(const char* name, int64_t slot_bytes, int num_slots, int copy_threads,
                                  int64_t dev_slot_bytes, pace_kv_channel** out) {
  if (dev_slot_bytes <= 0) {
    if (out) *out = nullptr;
    return fail(PACE_KV_EINVAL, "channel: dev_slot_bytes must be a positive multiple of 4096");
  }
  return create_channel(name, slot_bytes, num_slots, copy_threads, dev_slot_bytes, out);
}

int pace_kv_channel_device_info(pace_kv_channel* ch, int64_t* dev_slot_bytes, int* on_current_gpu) {
  if (ch == nullptr) return fail(PACE_KV_EINVAL, "channel is NULL");
  if (dev_slot_bytes) *dev_slot_bytes = ch->ctl->dev_slot_bytes;
  if (on_current_gpu) {
    bool here = false;
    PACE_KV_TRY(device_ring_here(ch, &here));
    *on_current_gpu = here ? 1 : 0;
  }
  return PACE_KV_OK;
}

int pace_kv_channel_open(const char* name, int copy_threads, int timeout_ms, pace_kv_channel** out) {
  PACE_KV_TRY(new_endpoint(name, copy_threads, out));
  pace_kv_channel* ch = *out;
  *out = nullptr;
  using clock = std::chrono::steady_clock;
  const auto deadline = clock::now() + std::chrono::milliseconds(timeout_ms < 0 ? 0 : timeout_ms);
  // Waits for the creator: the name, then its size, then the magic.
  struct stat st;
  for (;;) {
    if (ch->fd < 0) ch->fd = shm_open(("/" + ch->name).c_str(), O_RDWR, 0600);
    if (ch->fd >= 0 && fstat(ch->fd, &st) == 0 && st.st_size >= static_cast<off_t>(sizeof(ChannelCtl))) {
      if (!ch->base) {
        int rc = map_channel(ch, st.st_size);
        if (rc) {
          destroy(ch);
          return rc;
        }
      }
      if (__atomic_load_n(&ch->ctl->magic, __ATOMIC_ACQUIRE) == kMagic) break;
    }
    if (clock::now() >= deadline) {
      destroy(ch);
      return fail(PACE_KV_ETIMEDOUT, "channel %s: not created within %d ms", name, timeout_ms);
    }
    std::this_thread::sleep_for(std::chrono::milliseconds(1));
  }
  ChannelCtl* c = ch->ctl;
  if (c->version != kVersion || c->total_bytes != ch->map_bytes ||
      !valid_slot_count(static_cast<int64_t>(c->num_slots))) {
    destroy(ch);
    return fail(PACE_KV_ESTATE, "channel %s: incompatible control block", name);
  }
  ch->pool = new CopyPool(copy_threads);
  take_local_ring(ch);
  *out = ch;
  return PACE_KV_OK;
}

int pace_kv_channel_close(pace_kv_channel* ch) {
  if (ch == nullptr) return PACE_KV_OK;
  if (ch->ctl) {
    if (ch->creator) ch->ctl->creator_closed.store(1, std::memory_order_release);
    ch->ctl->closed.store(1, std::memory_order_release);
    wake_all(&ch->ctl->head);
    wake_all(&ch->ctl->tail);
  }
  // Copies and kernels this endpoint enqueued may still use its staging.
  for (Staging* s : {&ch->tx, &ch->rx}) {
    if (!s->ready) continue;
    (void)hipStreamSynchronize(s->copy);
    for (int i = 0; i < 2; ++i) (void)hipEventSynchronize(s->drained[i]);
  }
  destroy(ch);
  return PACE_KV_OK;
}

int pace_kv_channel_unlink(const char* name) {
  PACE_KV_TRY(check_name(name));
  if (shm_unlink(("/" + std::string(name)).c_str()) != 0 && errno != ENOENT)
    return fail(PACE_KV_EINVAL, "channel %s: shm_unlink failed: %s", name, strerror(errno));
  return PACE_KV_OK;
}

int pace_kv_channel_info(pace_kv_channel* ch, int64_t* slot_bytes, int* num_slots) {
  if (ch == nullptr) return fail(PACE_KV_EINVAL, "channel is NULL");
  if (slot_bytes) *slot_bytes = ch->ctl->slot_bytes;
  if (num_slots) *num_slots = static_cast<int>(ch->ctl->num_slots);
  return PACE_KV_OK;
}

int pace_kv_channel_send(pace_kv_channel* ch, const void* const* src_layers, int num_layers,
                         int64_t pool_pages, const int32_t* page_ids, int64_t n_pages, int64_t page_bytes,
                         const void* meta, int64_t meta_bytes, int timeout_ms, uint64_t* msg_id,
                         void* stream_) {
  if (ch == nullptr) return fail(PACE_KV_EINVAL, "channel is NULL");
  std::lock_guard<std::mutex> lock(ch->send_mu);
  PACE_KV_TRY(check_open(ch));
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  bool device = false;
  PageIds ids;
  if (num_layers > 0 && n_pages > 0) {
    if (src_layers == nullptr || page_ids == nullptr) return fail(PACE_KV_EINVAL, "channel send: NULL argument");
    PACE_KV_TRY(classify_ids(page_ids, n_pages, &ids));
    PACE_KV_TRY(device_ring_here(ch, &device));
    device = device && receiver_on_ring_gpu(ch);
  }
  if (device) {
    // Same GPU as the device ring: the payload never leaves HBM.
    Chunking kd;
    PACE_KV_TRY(make_chunking(num_layers, n_pages, page_bytes, ch->ctl->dev_slot_bytes, &kd));
    PACE_KV_TRY(ring_ready(ch));
    uint64_t id = 0;
    PACE_KV_TRY(send_header(ch, num_layers, n_pages, page_bytes, meta, meta_bytes, timeout_ms, &id,
                            kDevicePayload));
    if (msg_id) *msg_id = id;
    return send_device(ch, src_layers, pool_pages, ids, kd, id, timeout_ms, stream);
  }
  Chunking k;
  PACE_KV_TRY(make_chunking(num_layers, n_pages, page_bytes, ch->ctl->slot_bytes, &k));
  if (k.num_chunks > 0) PACE_KV_TRY(staging_ready(ch, ch->tx));
  uint64_t id = 0;
  PACE_KV_TRY(send_header(ch, num_layers, n_pages, page_bytes, meta, meta_bytes, timeout_ms, &id));
  if (msg_id) *msg_id = id;
  Staging& s = ch->tx;
  // Chunk c: pack into device slot c%2 (caller stream), copy down to pinned
  // slot c%2 (copy stream); chunk c-1 is copied into the ring meanwhile.
  for (int64_t c = 0; c <= k.num_chunks; ++c) {
    if (c < k.num_chunks) {
      const int b = static_cast<int>(c & 1);
      const Chunking::Chunk ck = k.at(c);
      int rc = hip_status(hipStreamWaitEvent(stream, s.copied[b], 0), "channel send wait");
      if (rc == PACE_KV_OK) {
        const int64_t stride = k.layers_per_chunk > 0 ? k.layer_bytes : ck.bytes;
        rc = pack_pages(src_layers + ck.layer, ck.nl, pool_pages, ids, ck.j0, ck.nj, page_bytes, s.dev[b],
                        stride, nullptr, stream);
      }
      if (rc == PACE_KV_OK) rc = hip_status(hipEventRecord(s.filled[b], stream), "channel send record");
      if (rc == PACE_KV_OK) rc = hip_status(hipStreamWaitEvent(s.copy, s.filled[b], 0), "channel send wait");
      if (rc == PACE_KV_OK)
        rc = hip_status(hipMemcpyAsync(s.pinned[b], s.dev[b], static_cast<size_t>(ck.bytes),
                                       hipMemcpyDeviceToHost, s.copy), "channel device-to-host copy");
      if (rc == PACE_KV_OK) rc = hip_status(hipEventRecord(s.copied[b], s.copy), "channel send record");
      if (rc) return abandon(ch, id, rc);
    }
    if (c > 0) {
      const int b = static_cast<int>((c - 1) & 1);
      int rc = hip_status(hipEventSynchronize(s.copied[b]), "channel device-to-host copy");
      if (rc == PACE_KV_OK) rc = send_chunk_from(ch, id, c - 1, k.at(c - 1), s.pinned[b], timeout_ms);
      if (rc) return abandon(ch, id, rc);
    }
  }
  return PACE_KV_OK;
}

int pace_kv_channel_send_host(pace_kv_channel* ch, const void* payload, int num_layers, int64_t n_pages,
                              int64_t page_bytes, const void* meta, int64_t meta_bytes, int timeout_ms,
                              uint64_t* msg_id) {
  if (ch == nullptr) return fail(PACE_KV_EINVAL, "channel is NULL");
  std::lock_guard<std::mutex> lock(ch->send_mu);
  PACE_KV_TRY(check_open(ch));
  Chunking k;
  PACE_KV_TRY(make_chunking(num_layers, n_pages, page_bytes, ch->ctl->slot_bytes, &k));
  if (k.num_chunks > 0 && payload == nullptr) return fail(PACE_KV_EINVAL, "channel send: payload is NULL");
  uint64_t id = 0;
  PACE_KV_TRY(send_header(ch, num_layers, n_pages, page_bytes, meta, meta_bytes, timeout_ms, &id));
  if (msg_id) *msg_id = id;
  for (int64_t c = 0; c < k.num_chunks; ++c) {
    const Chunking::Chunk ck = k.at(c);
    int rc = send_chunk_from(ch, id, c, ck, static_cast<const char*>(payload) + ck.offset, timeout_ms);
    if (rc) return abandon(ch, id, rc);
  }
  return PACE_KV_OK;
}

int pace_kv_channel_recv_header(pace_kv_channel* ch, void* meta, int64_t meta_cap, int64_t* meta_bytes,
                                int* num_layers, int64_t* n_pages, int64_t* page_bytes, uint64_t* msg_id,
                                int timeout_ms) {
  if (ch == nullptr) return fail(PACE_KV_EINVAL, "channel is NULL");
  std::lock_guard<std::mutex> lock(ch->recv_mu);
  if (ch->rx_active)
    return fail(PACE_KV_ESTATE, "channel %s: the payload of message %llu has not been received",
                ch->name.c_str(), (unsigned long long)ch->rx_msg);
  if (ch->ctl->dev_slot_bytes > 0) record_receiver_gpu(ch);
  uint32_t idx = 0;
  for (;;) {
    PACE_KV_TRY(next_record(ch, timeout_ms, &idx, "a message"));
    if (ch->ctl->slots[idx].kind == kHeader) break;
    // A chunk without its header: the rest of a message whose receive
    // failed part-way.  It is dropped.
    release(ch);
  }
  const SlotRecord& r = ch->ctl->slots[idx];
  if (meta_bytes) *meta_bytes = r.bytes;
  if (r.bytes > meta_cap || (r.bytes > 0 && meta == nullptr))
    return fail(PACE_KV_ERANGE, "channel %s: metadata needs %lld bytes, the buffer holds %lld (message kept)",
                ch->name.c_str(), (long long)r.bytes, (long long)meta_cap);
  const bool device = (r.flags & kDevicePayload) != 0;
  if (device && ch->ctl->dev_slot_bytes <= 0) {
    release(ch);
    return fail(PACE_KV_ESTATE, "channel %s: message %llu is in device slots but the channel has none",
                ch->name.c_str(), (unsigned long long)r.msg_id);
  }
  Chunking k;
  int rc = make_chunking(r.num_layers, r.n_pages, r.page_bytes,
                         device ? ch->ctl->dev_slot_bytes : ch->ctl->slot_bytes, &k);
  if (rc) {
    release(ch);
    return rc;
  }
  if (r.bytes > 0) memcpy(meta, slot_data(ch, idx), static_cast<size_t>(r.bytes));
  if (num_layers) *num_layers = r.num_layers;
  if (n_pages) *n_pages = r.n_pages;
  if (page_bytes) *page_bytes = r.page_bytes;
  if (msg_id) *msg_id = r.msg_id;
  ch->rx_msg = r.msg_id;
  ch->rx_chunks = k;
  ch->rx_next = 0;
  ch->rx_device = device;
  ch->rx_active = k.num_chunks > 0;
  release(ch);
  return PACE_KV_OK;
}

int pace_kv_channel_recv(pace_kv_channel* ch, void* const* dst_layers, int num_layers, int64_t pool_pages,
                         const int32_t* page_ids, int64_t n_pages, int64_t page_bytes, int32_t* err_count,
                         int timeout_ms, void* stream_) {
  if (ch == nullptr) return fail(PACE_KV_EINVAL, "channel is NULL");
  std::lock_guard<std::mutex> lock(ch->recv_mu);
  PACE_KV_TRY(check_rx_shape(ch, num_layers, n_pages, page_bytes));
  if (dst_layers == nullptr || page_ids == nullptr) return fail(PACE_KV_EINVAL, "channel recv: NULL argument");
  PageIds ids;
  PACE_KV_TRY(classify_ids(page_ids, n_pages, &ids));
  if (ch->rx_device)
    return recv_device(ch, dst_layers, pool_pages, ids, err_count, timeout_ms, static_cast<hipStream_t>(stream_));
  PACE_KV_TRY(staging_ready(ch, ch->rx));
  const Chunking k = ch->rx_chunks;
  Staging& s = ch->rx;
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  // The caller's earlier work on `stream` (e.g. the upload of page_ids, or
  // earlier use of the destination pages) comes before the unpacks, which
  // run on `stream` itself.
  while (ch->rx_active) {
    const int64_t c = ch->rx_next;
    const int b = static_cast<int>(c & 1);
    uint32_t idx = 0;
    Chunking::Chunk ck;
    PACE_KV_TRY(next_chunk(ch, timeout_ms, &idx, &ck));
    // pinned slot b was last read by the upload of chunk c-2
    int rc = hip_status(hipEventSynchronize(s.copied[b]), "channel host-to-device copy");
    if (rc) {
      ch->rx_active = false;
      return rc;
    }
    ch->pool->copy(s.pinned[b], slot_data(ch, idx), ck.bytes);
    finish_chunk(ch);
    // device slot b was last read by the unpack of chunk c-2
    rc = hip_status(hipStreamWaitEvent(s.copy, s.drained[b], 0), "channel recv wait");
    if (rc == PACE_KV_OK)
      rc = hip_status(hipMemcpyAsync(s.dev[b], s.pinned[b], static_cast<size_t>(ck.bytes), hipMemcpyHostToDevice,
                                     s.copy), "channel host-to-device copy");
    if (rc == PACE_KV_OK) rc = hip_status(hipEventRecord(s.copied[b], s.copy), "channel recv record");
    if (rc == PACE_KV_OK) rc = hip_status(hipStreamWaitEvent(stream, s.copied[b], 0), "channel recv wait");
    if (rc == PACE_KV_OK) {
      const int64_t stride = k.layers_per_chunk > 0 ? k.layer_bytes : ck.bytes;
      rc = unpack_pages(s.dev[b], stride, dst_layers + ck.layer, ck.nl, pool_pages, ids, ck.j0, ck.nj,
                        page_bytes, err_count, stream);
    }
    if (rc == PACE_KV_OK) rc = hip_status(hipEventRecord(s.drained[b], stream), "channel recv record");
    if (rc) {
      ch->rx_active = false;
      return rc;
    }
  }
  return PACE_KV_OK;
}

int pace_kv_channel_recv_host(pace_kv_channel* ch, void* payload, int64_t payload_bytes, int timeout_ms) {
  if (ch == nullptr) return fail(PACE_KV_EINVAL, "channel is NULL");
  std::lock_guard<std::mutex> lock(ch->recv_mu);
  if (!ch->rx_active) return fail(PACE_KV_ESTATE, "channel %s: no message header received", ch->name.c_str());
  const Chunking& k = ch->rx_chunks;
  const int64_t total = k.num_layers * k.layer_bytes;
  if (payload != nullptr && payload_bytes != total)
    return fail(PACE_KV_EINVAL, "channel %s: message %llu holds %lld payload bytes, the buffer %lld",
                ch->name.c_str(), (unsigned long long)ch->rx_msg, (long long)total, (long long)payload_bytes);
  if (ch->rx_device && payload != nullptr) PACE_KV_TRY(ring_ready(ch));
  while (ch->rx_active) {
    uint32_t idx = 0;
    Chunking::Chunk ck;
    PACE_KV_TRY(next_chunk(ch, timeout_ms, &idx, &ck));
    if (payload != nullptr) {
      char* to = static_cast<char*>(payload) + ck.offset;
      if (ch->rx_device) {
        const int rc = hip_status(hipMemcpy(to, dev_slot(ch, idx), static_cast<size_t>(ck.bytes),
                                            hipMemcpyDeviceToHost), "channel copy out of the device ring");
        if (rc) return fail_rx(ch, rc);
      } else {
        ch->pool->copy(to, slot_data(ch, idx), ck.bytes);
      }
    }
    finish_chunk(ch);
  }
  return PACE_KV_OK;
}

}  // extern "C"
