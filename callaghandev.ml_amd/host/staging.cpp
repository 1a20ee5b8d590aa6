// Host-side copy engine of the manager: a process-wide pool of threads that
// splits large host copies and compares into slices.  The manager stages
// every transfer through pinned memory, so each upload is a host copy into
// pinned memory followed by a DMA, and each download a DMA followed by a host
// copy out; at the c3 shape these host copies move 16 MiB per activation,
// which one thread cannot keep up with against PCIe.  Shadow compares of
// resident activations (is the host array still what the device holds?)
// read two such arrays.
#include <immintrin.h>
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
  // plus the calling thread; eight threads in all already saturate the
  // host memory beside a running DMA on the GPU box (16 CPUs: 4.05 ms per
  // c3 drop-in sequence with 8 threads against 4.2 ms with 13)
  return std::max(0, std::min(7, 3 * cpus / 4));
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
      posted_.fetch_add(1, std::memory_order_release);
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

  // A worker that finished a job polls for the next one for a while before
  // it sleeps: the jobs of one manager call (the chunks of a download, each
  // posted when its DMA lands) come tens of microseconds apart, and a
  // condition-variable wake-up of a dozen sleeping threads costs about that.
  void worker() {
    uint64_t seen = posted_.load(std::memory_order_acquire);
    for (;;) {
      for (int spin = 0; spin < kSpin && posted_.load(std::memory_order_acquire) == seen; ++spin)
        __builtin_ia32_pause();
      seen = posted_.load(std::memory_order_acquire);
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

  static constexpr int kSpin = 20000;  // pause instructions, roughly 100-200 us
  int threads_ = 0;
  std::atomic<uint64_t> posted_{0};
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

namespace {

// A slice copy with non-temporal 64-byte stores: the destination is written
// without being read into the cache first, a third less memory traffic than
// a cached copy, which matters while a DMA into the pinned buffers competes
// for the same memory (measured on the GPU box: 115 against 100 GB/s from
// pinned memory beside a running device-to-host DMA, 160 against 136 GB/s
// alone, with eight threads).
__attribute__((target("avx512f"))) void stream_copy_avx512(char *d, const char *s, size_t n) {
  size_t head = (64 - (reinterpret_cast<uintptr_t>(d) & 63)) & 63;
  if (head > n) head = n;
  std::memcpy(d, s, head);
  size_t i = head;
  for (; i + 256 <= n; i += 256) {
    const __m512i a = _mm512_loadu_si512(s + i), b = _mm512_loadu_si512(s + i + 64),
                  c = _mm512_loadu_si512(s + i + 128), e = _mm512_loadu_si512(s + i + 192);
    _mm512_stream_si512(reinterpret_cast<__m512i *>(d + i), a);
    _mm512_stream_si512(reinterpret_cast<__m512i *>(d + i + 64), b);
    _mm512_stream_si512(reinterpret_cast<__m512i *>(d + i + 128), c);
    _mm512_stream_si512(reinterpret_cast<__m512i *>(d + i + 192), e);
  }
  std::memcpy(d + i, s + i, n - i);
  _mm_sfence();  // the streaming stores are visible before the slice is reported done
}

const bool kHaveAvx512 = __builtin_cpu_supports("avx512f");

void copy_slice(void *dst, const void *src, size_t n) {
  if (kHaveAvx512 && n >= 4096)
    stream_copy_avx512(static_cast<char *>(dst), static_cast<const char *>(src), n);
  else
    std::memcpy(dst, src, n);
}

}  // namespace

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
      copy_slice(static_cast<char *>(dst) + off, static_cast<const char *>(src) + off, std::min(per, bytes - off));
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
