// Host-side stress of libpace_kv's CPU code, built with the host pass under
// AddressSanitizer + UndefinedBehaviorSanitizer and, separately, under
// ThreadSanitizer (tests/sanitize/Makefile; device code is not instrumented,
// and nothing here touches a GPU):
//   - pace_kv_allocator_* and pace_kv_plan from 8 threads sharing one
//     allocator: no page handed out twice, none lost;
//   - the channel between two processes through the host payload path
//     (pace_kv_channel_send_host / recv_header / recv_host): messages larger
//     than the ring, metadata, a discarded payload, two receiving threads
//     taking whole messages, deadlines and closing.
// Exits 0 when every check passes; prints what failed otherwise.
#include <pace_kv.h>

#include <sys/wait.h>
#include <unistd.h>

#include <atomic>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <random>
#include <string>
#include <thread>
#include <vector>

namespace {

int failures = 0;
std::mutex report_mu;

void check(bool ok, const char* what) {
  if (!ok) {
    std::lock_guard<std::mutex> lock(report_mu);
    ++failures;
    std::fprintf(stderr, "FAILED: %s (%s)\n", what, pace_kv_last_error());
  }
}

// ---------------------------------------------------------------- allocator

void allocator_stress() {
  constexpr int kPages = 4096, kThreads = 8, kRounds = 3000;
  pace_kv_allocator* a = nullptr;
  check(pace_kv_allocator_create(kPages, nullptr, 0, &a) == PACE_KV_OK, "allocator_create");
  std::vector<std::atomic<int>> owner(kPages);
  for (auto& o : owner) o.store(-1);
  std::vector<std::thread> ts;
  for (int t = 0; t < kThreads; ++t) {
    ts.emplace_back([&, t] {
      std::mt19937 rng(1234 + t);
      std::vector<int32_t> got(64);
      for (int r = 0; r < kRounds; ++r) {
        const int n = 1 + static_cast<int>(rng() % 48);
        const int rc = pace_kv_allocator_allocate(a, n, got.data());
        if (rc == PACE_KV_ENOMEM) continue;
        check(rc == PACE_KV_OK, "allocator_allocate");
        for (int i = 0; i < n; ++i) {
          int expect = -1;
          check(owner[got[i]].compare_exchange_strong(expect, t), "a page handed out twice");
        }
        for (int i = 0; i < n; ++i) owner[got[i]].store(-1);
        // free with a repeat: the page goes back once
        std::vector<int32_t> back(got.begin(), got.begin() + n);
        back.push_back(got[0]);
        check(pace_kv_allocator_free(a, back.data(), static_cast<int64_t>(back.size())) == PACE_KV_OK,
              "allocator_free");
        if (r % 97 == 0) {
          int64_t nf = -1;
          check(pace_kv_allocator_num_free(a, &nf) == PACE_KV_OK && nf >= 0 && nf <= kPages, "num_free");
        }
      }
    });
  }
  // a planner sharing the allocator
  ts.emplace_back([&] {
    std::vector<int32_t> src(64), tables(80), ids(64);
    for (int i = 0; i < 64; ++i) src[i] = i;
    const int64_t indptr[3] = {0, 20, 64};
    const int32_t dst_pages[2] = {21, 44};
    for (int r = 0; r < kRounds; ++r) {
      const int rc = pace_kv_plan(a, 2, indptr, src.data(), 64, dst_pages, tables.data(), ids.data());
      if (rc == PACE_KV_ENOMEM) continue;
      check(rc == PACE_KV_OK, "plan");
      check(std::memcmp(ids.data(), tables.data(), 20 * sizeof(int32_t)) == 0, "plan remap of request 0");
      check(std::memcmp(ids.data() + 20, tables.data() + 21, 44 * sizeof(int32_t)) == 0, "plan remap of request 1");
      check(pace_kv_allocator_free(a, tables.data(), 65) == PACE_KV_OK, "free planned tables");
    }
  });
  for (auto& t : ts) t.join();
  int64_t nf = 0, len = 0;
  check(pace_kv_allocator_num_free(a, &nf) == PACE_KV_OK && nf == kPages, "every page returned");
  std::vector<int32_t> snap(kPages);
  check(pace_kv_allocator_snapshot(a, snap.data(), kPages, &len) == PACE_KV_OK && len == kPages, "snapshot");
  std::vector<int> seen(kPages, 0);
  for (int64_t i = 0; i < len; ++i) ++seen[snap[i]];
  bool once = true;
  for (int c : seen) once = once && c == 1;
  check(once, "each page in the free list exactly once");
  check(pace_kv_allocator_destroy(a) == PACE_KV_OK, "allocator_destroy");
}

// ------------------------------------------------------------------ channel

constexpr int kLayers = 3;
constexpr int64_t kPageBytes = 64 << 10;  // a layer of 90 pages (5.6 MiB) goes through the copy threads

uint8_t byte_of(int msg, int64_t off) { return static_cast<uint8_t>((msg * 131 + off * 7 + off / 4099) & 0xff); }

int64_t pages_of(int msg) { return 1 + (msg * 37) % 90; }  // up to 90 pages x 3 layers x 64 KiB: more than the 32 MiB ring

int sender_process(const std::string& name, int messages) {
  pace_kv_channel* ch = nullptr;
  if (pace_kv_channel_open(name.c_str(), 3, 20000, &ch) != PACE_KV_OK) {
    std::fprintf(stderr, "sender: open failed: %s\n", pace_kv_last_error());
    return 1;
  }
  int rc = 0;
  for (int m = 0; m < messages && rc == 0; ++m) {
    const int64_t n = pages_of(m);
    std::vector<uint8_t> payload(static_cast<size_t>(kLayers * n * kPageBytes));
    for (size_t i = 0; i < payload.size(); ++i) payload[i] = byte_of(m, static_cast<int64_t>(i));
    const std::string meta = "message " + std::to_string(m);
    uint64_t id = 0;
    rc = pace_kv_channel_send_host(ch, payload.data(), kLayers, n, kPageBytes, meta.data(),
                                   static_cast<int64_t>(meta.size()), 20000, &id);
    if (rc) std::fprintf(stderr, "sender: message %d failed: %s\n", m, pace_kv_last_error());
  }
  pace_kv_channel_close(ch);
  return rc == 0 ? 0 : 1;
}

void channel_test() {
  const std::string name = "pace_sanitize_" + std::to_string(getpid());
  constexpr int kMessages = 40;
  (void)pace_kv_channel_unlink(name.c_str());
  // fork before any thread exists in this process (the allocator threads
  // have been joined; the endpoints' copy threads start after the fork)
  const pid_t child = fork();
  if (child == 0) _exit(sender_process(name, kMessages));
  pace_kv_channel* rx = nullptr;
  check(pace_kv_channel_create(name.c_str(), 8 << 20, 4, 3, &rx) == PACE_KV_OK, "channel_create");
  if (rx == nullptr) return;
  // a wait with no deadline left ends at once
  char meta0[64];
  int64_t mb = 0;
  int nl = 0;
  int64_t np = 0, pb = 0;
  uint64_t id = 0;
  std::mutex rx_mu;  // whole messages per thread: header + payload under one lock
  std::atomic<int> next{0};
  std::vector<int> got(kMessages, 0);
  auto receiver = [&] {
    for (;;) {
      std::lock_guard<std::mutex> lock(rx_mu);
      const int m = next.load();
      if (m >= kMessages) return;
      char meta[64];
      int64_t meta_bytes = 0;
      int num_layers = 0;
      int64_t n_pages = 0, page_bytes = 0;
      uint64_t msg = 0;
      if (pace_kv_channel_recv_header(rx, meta, sizeof(meta), &meta_bytes, &num_layers, &n_pages, &page_bytes,
                                      &msg, 20000) != PACE_KV_OK) {
        check(false, "recv_header");
        next.store(kMessages);
        return;
      }
      const std::string want = "message " + std::to_string(m);
      check(std::string(meta, static_cast<size_t>(meta_bytes)) == want, "metadata in order");
      check(num_layers == kLayers && n_pages == pages_of(m) && page_bytes == kPageBytes, "header shape");
      if (m % 7 == 3) {
        check(pace_kv_channel_recv_host(rx, nullptr, 0, 20000) == PACE_KV_OK, "discard");
      } else {
        std::vector<uint8_t> payload(static_cast<size_t>(kLayers * n_pages * kPageBytes));
        check(pace_kv_channel_recv_host(rx, payload.data(), static_cast<int64_t>(payload.size()), 20000) ==
                  PACE_KV_OK, "recv_host");
        bool same = true;
        for (size_t i = 0; i < payload.size() && same; ++i) same = payload[i] == byte_of(m, static_cast<int64_t>(i));
        check(same, "payload bytes");
      }
      ++got[m];
      next.store(m + 1);
    }
  };
  std::thread t1(receiver), t2(receiver);
  t1.join();
  t2.join();
  bool all = true;
  for (int c : got) all = all && c == 1;
  check(all, "every message received once");
  int status = 0;
  check(waitpid(child, &status, 0) == child && WIFEXITED(status) && WEXITSTATUS(status) == 0, "sender exited 0");
  // nothing left: a zero deadline times out; after close, calls fail
  check(pace_kv_channel_recv_header(rx, meta0, sizeof(meta0), &mb, &nl, &np, &pb, &id, 0) != PACE_KV_OK,
        "empty ring: recv_header fails (closed or timed out)");
  check(pace_kv_channel_close(rx) == PACE_KV_OK, "channel_close");
}

}  // namespace

int main() {
  allocator_stress();
  channel_test();
  if (failures) {
    std::fprintf(stderr, "%d check(s) failed\n", failures);
    return 1;
  }
  std::printf("host stress ok\n");
  return 0;
}
