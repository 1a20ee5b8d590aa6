// Host-side copy engine of the manager: a process-wide pool of threads that
// splits large host copies and compares into slices.  The manager stages
// every transfer through pinned memory, so each upload is a host copy into
// pinned memory followed by a DMA, and each download a DMA followed by a host
// copy out; at the c3 shape these host copies move 16 MiB per activation,
// which one thread cannot keep up with against PCIe.  Shadow compares of
// resident activations (is the host array still what the device holds?)
// read two such arrays.
#include <sched.h>

#include <algorithm>
#include <atomic>
#include <condition_variable>
#include <cstdlib>
#include <cstring>
#include <deque>
#include <functional>
#include <map>
#include <new>
#include <memory>
#include <mutex>
#include <thread>

#include "cdml_host.h"

namespace cdml_host {

namespace {

constexpr size_t kSlice = size_t(1) << 20;       // bytes per task
constexpr size_t kParallelMin = size_t(2) << 20;  // below this, the caller does it alone

int pool_threads() {
  if (const char *e = std::getenv("CDML_HOST_COPY_THREADS")) {
    const int n = std::atoi(e);
    if (n >= 0) return std::min(n, 64);
  }
  int cpus = 0;
  cpu_set_t set;
  if (sched_getaffinity(0, sizeof(set), &set) == 0) cpus = CPU_COUNT(&set);
  if (cpus <= 0) cpus = (int)std::thread::hardware_concurrency();
  return std::max(0, std::min(12, 3 * cpus / 4));  // plus the calling thread
}

class Pool {
 public:
  Pool() {
    const int n = pool_threads();
    for (int i = 0; i < n; ++i) std::thread([this] { worker(); }).detach();
    threads_ = n;
  }
  int threads() const { return threads_; }

  // fn(i) for every i in [0, n); the caller takes tasks too, so this also
  // completes with no worker threads.
  void run(int n, const std::function<void(int)> &fn) {
    if (n <= 0) return;
    auto job = std::make_shared<Job>();
    job->fn = &fn;
    job->n = n;
    if (threads_ > 0 && n > 1) {
      std::lock_guard<std::mutex> lock(mu_);
      jobs_.push_back(job);
      cv_.notify_all();
    }
    work_on(*job);
    std::unique_lock<std::mutex> lock(job->mu);
    job->cv.wait(lock, [&] { return job->done.load() == job->n; });
  }

 private:
  struct Job {
    const std::function<void(int)> *fn = nullptr;
    int n = 0;
    std::atomic<int> next{0}, done{0};
    std::mutex mu;
    std::condition_variable cv;
  };

  static void work_on(Job &j) {
    for (int i = j.next.fetch_add(1); i < j.n; i = j.next.fetch_add(1)) {
      (*j.fn)(i);
      if (j.done.fetch_add(1) + 1 == j.n) {
        std::lock_guard<std::mutex> lock(j.mu);
        j.cv.notify_all();
      }
    }
  }

  void worker() {
    for (;;) {
      std::shared_ptr<Job> job;
      {
        std::unique_lock<std::mutex> lock(mu_);
        cv_.wait(lock, [&] { return !jobs_.empty(); });
        job = jobs_.front();
        if (job->next.load() >= job->n) {  // fully handed out: retire it
          jobs_.pop_front();
          continue;
        }
      }
      work_on(*job);
    }
  }

  int threads_ = 0;
  std::mutex mu_;
  std::condition_variable cv_;
  std::deque<std::shared_ptr<Job>> jobs_;
};

Pool &pool() {
  static Pool *p = new Pool();  // never destroyed: its threads live until the process ends
  return *p;
}

int slices(size_t bytes) {
  const size_t per = std::max(kSlice, bytes / (size_t)(4 * (pool().threads() + 1)));
  return (int)((bytes + per - 1) / per);
}

// Idle large blocks by exact size.
constexpr size_t kRecycleMin = size_t(1) << 20;
constexpr size_t kRecycleCap = size_t(1) << 30;

struct BlockCache {
  std::mutex mu;
  std::multimap<size_t, void *> idle;
  size_t idle_bytes = 0;
};

BlockCache &blocks() {
  static BlockCache *c = new BlockCache();  // idle blocks live until the process ends
  return *c;
}

}  // namespace

void *HostArrayAlloc(size_t bytes) {
  if (bytes >= kRecycleMin) {
    BlockCache &c = blocks();
    std::lock_guard<std::mutex> lock(c.mu);
    auto it = c.idle.find(bytes);
    if (it != c.idle.end()) {
      void *p = it->second;
      c.idle.erase(it);
      c.idle_bytes -= bytes;
      return p;
    }
  }
  void *p = std::malloc(bytes ? bytes : 1);
  if (!p) throw std::bad_alloc();
  return p;
}

void HostArrayFree(void *p, size_t bytes) {
  if (!p) return;
  if (bytes >= kRecycleMin) {
    BlockCache &c = blocks();
    std::lock_guard<std::mutex> lock(c.mu);
    // make room by dropping the largest idle blocks
    while (c.idle_bytes + bytes > kRecycleCap && !c.idle.empty()) {
      auto last = std::prev(c.idle.end());
      c.idle_bytes -= last->first;
      std::free(last->second);
      c.idle.erase(last);
    }
    if (bytes <= kRecycleCap) {
      c.idle.emplace(bytes, p);
      c.idle_bytes += bytes;
      return;
    }
  }
  std::free(p);
}

int HostCopyThreads() { return pool().threads() + 1; }

void ParallelMemcpy(void *dst, const void *src, size_t bytes) {
  if (bytes < kParallelMin) {
    if (bytes) std::memcpy(dst, src, bytes);
    return;
  }
  const int n = slices(bytes);
  const size_t per = ((bytes + n - 1) / n + 63) & ~size_t(63);
  pool().run(n, [&](int i) {
    const size_t off = (size_t)i * per;
    if (off < bytes)
      std::memcpy(static_cast<char *>(dst) + off, static_cast<const char *>(src) + off,
                  std::min(per, bytes - off));
  });
}

void ParallelZero(void *dst, size_t bytes) {
  if (bytes < kParallelMin) {
    if (bytes) std::memset(dst, 0, bytes);
    return;
  }
  const int n = slices(bytes);
  const size_t per = ((bytes + n - 1) / n + 63) & ~size_t(63);
  pool().run(n, [&](int i) {
    const size_t off = (size_t)i * per;
    if (off < bytes) std::memset(static_cast<char *>(dst) + off, 0, std::min(per, bytes - off));
  });
}

bool ParallelEqual(const void *a, const void *b, size_t bytes) {
  if (bytes < kParallelMin) return bytes == 0 || std::memcmp(a, b, bytes) == 0;
  const int n = slices(bytes);
  const size_t per = ((bytes + n - 1) / n + 63) & ~size_t(63);
  std::atomic<bool> differ{false};
  pool().run(n, [&](int i) {
    const size_t off = (size_t)i * per;
    if (off >= bytes || differ.load(std::memory_order_relaxed)) return;
    if (std::memcmp(static_cast<const char *>(a) + off, static_cast<const char *>(b) + off,
                    std::min(per, bytes - off)) != 0)
      differ.store(true, std::memory_order_relaxed);
  });
  return !differ.load();
}

}  // namespace cdml_host
