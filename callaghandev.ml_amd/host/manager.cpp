// HipAccelerationManager: the hot-path IAccelerationManager methods on the
// gfx950 kernels of libcdml_hip.so.  Each method validates its arguments in
// the order the reference's CPU manager does (citations per method), stages
// activations through the manager's device buffers, reuses resident copies of
// weight arrays, runs the kernel(s) on the manager's stream and returns host
// arrays.  Nothing here computes on the CPU: a missing device or library is
// an InvalidOperationException.
#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <functional>

#include "cdml_host.h"

namespace cdml_host {

namespace {

// Activation-cache memory of every manager in the process: device bytes, each
// paired with as many pinned host bytes.  The process-wide budget bounds the
// pinned memory however many managers a caller creates (the reference builds
// one manager per FFN); a manager over it gives back its own least recently
// used entries, and when it has none left to give, the array takes the
// uncached scratch path.
std::atomic<size_t> g_act_bytes{0};
std::atomic<size_t> g_act_budget{size_t(4) << 30};
std::atomic<int> g_act_alloc_failures{0};  // injected failures (tests)

void check(int rc, const char *what) {
  if (rc != CDML_OK)
    throw InvalidOperationException(std::string(what) + ": " + cdml_last_error());
}

// Scratch slots of the manager's device buffer pool.
enum Slot {
  S_X = 0, S_Q, S_K, S_V, S_O, S_MASK, S_IDS, S_KVLEN, S_WS, S_BIAS,
  S_DQ, S_DK, S_DV, S_GW0, S_GW1, S_GW2, S_GB0, S_GB1, S_GB2, S_COUNT
};

}  // namespace

HipAccelerationManager::HipAccelerationManager(int device) : device_(device) {
  if (device < 0) throw ArgumentOutOfRangeException("device");
}

HipAccelerationManager::~HipAccelerationManager() {
  try {
    Dispose();
  } catch (...) {
  }
}

void HipAccelerationManager::Dispose() {
  std::lock_guard<std::mutex> lock(mu_);
  if (disposed_) return;
  disposed_ = true;
  if (!ready_) return;
  cdml_stream_synchronize(stream_);
  for (auto &kv : resident_) cdml_free(kv.second.dev);
  resident_.clear();
  for (auto &b : scratch_) cdml_free(b.p);
  scratch_.clear();
  for (auto &kv : decode_) {
    cdml_free(kv.second.k);
    cdml_free(kv.second.v);
  }
  decode_.clear();
  for (auto &kv : acts_) act_release(kv.second);
  acts_.clear();
  for (const ActEntry &e : act_parked_) act_release(e);
  act_parked_.clear();
  for (auto &kv : act_free_) act_destroy(kv.second);
  act_free_.clear();
  for (auto &kv : pin_spare_) cdml_host_free_pinned(kv.second);
  pin_spare_.clear();
  cdml_host_free_pinned(stage_);
  stage_ = nullptr;
  stage_cap_ = stage_off_ = 0;
  for (LseRecord &r : lse_) cdml_free(r.lse);
  lse_.clear();
  cdml_free(lse_spare_);
  lse_spare_ = nullptr;
  lse_spare_bytes_ = 0;
  for (DeviceBuf &b : ffn_scratch_) cdml_free(b.p);
  ffn_scratch_.clear();
  for (cdml_event e : events_) cdml_event_destroy(e);
  events_.clear();
  if (copy_) {
    cdml_stream_synchronize(copy_);
    cdml_stream_destroy(copy_);
    copy_ = nullptr;
    for (cdml_event &e : kev_) {
      cdml_event_destroy(e);
      e = nullptr;
    }
  }
  cdml_stream_destroy(stream_);
  stream_ = nullptr;
}

void HipAccelerationManager::ensure_ready() {
  if (disposed_) throw InvalidOperationException("HipAccelerationManager has been disposed.");
  if (!ready_) {
    check(cdml_init(device_), "cdml_init");
    check(cdml_stream_create(&stream_), "cdml_stream_create");
    scratch_.assign(S_COUNT, DeviceBuf{});
    ready_ = true;
  }
  begin_call();
}

// Every public method that touches the device starts here (through
// ensure_ready, with mu_ held): the staging buffer is handed out from its
// start again, and the call gets a new id that marks the activation entries
// it uses as not evictable.
void HipAccelerationManager::begin_call() {
  if (dirty_ || !act_parked_.empty()) sync();  // an earlier call that threw may have left transfers in flight
  for (const ActEntry &e : act_parked_) act_release(e);  // the earlier call is over: its dropped buffers are free
  act_parked_.clear();
  stage_off_ = 0;
  ++call_;
  defer_ = false;
  pending_.clear();
}

bool HipAccelerationManager::settle() {
  defer_ = false;
  bool current = true;
  for (const Pending &p : pending_) {
    if (ParallelEqual(p.host, p.shadow, p.bytes)) {
      if (!p.weight) stats_.h2d_skipped_bytes += p.bytes;
      continue;
    }
    current = false;
    if (p.weight) {
      ParallelMemcpy(p.shadow, p.host, p.bytes);
      upload(p.dev, p.shadow, p.bytes);
    } else {
      stage_upload(p.dev, p.host, p.bytes, p.shadow);
      auto it = acts_.find(static_cast<const float *>(p.host));
      if (it != acts_.end() && it->second.dev == p.dev) it->second.ver = ++ver_;
    }
  }
  pending_.clear();
  return current;
}

cdml_stream HipAccelerationManager::stream() {
  std::lock_guard<std::mutex> lock(mu_);
  ensure_ready();
  return stream_;
}

void *HipAccelerationManager::scratch(int slot, size_t bytes) {
  DeviceBuf &b = scratch_[slot];
  if (bytes == 0) bytes = 4;
  if (b.bytes < bytes) {
    sync();
    check(cdml_free(b.p), "cdml_free");
    b.p = nullptr;
    b.bytes = 0;
    size_t grow = bytes + bytes / 4;  // some headroom for the next, larger call
    check(cdml_malloc(&b.p, grow), "cdml_malloc");
    b.bytes = grow;
  }
  return b.p;
}

// Like scratch(), but a failed allocation returns NULL (the slot is left
// empty) instead of throwing.
void *HipAccelerationManager::try_scratch(int slot, size_t bytes) {
  DeviceBuf &b = scratch_[slot];
  if (bytes == 0) bytes = 4;
  if (b.bytes >= bytes) return b.p;
  sync();
  check(cdml_free(b.p), "cdml_free");
  b.p = nullptr;
  b.bytes = 0;
  void *p = nullptr;
  if (cdml_malloc(&p, bytes) != CDML_OK) return nullptr;
  b.p = p;
  b.bytes = bytes;
  return p;
}

size_t SdpaBackwardWorkspaceChoice(size_t base_bytes, size_t stored_ds_bytes, size_t extra_cap) {
  if (stored_ds_bytes <= base_bytes) return base_bytes;
  return stored_ds_bytes - base_bytes <= extra_cap ? stored_ds_bytes : base_bytes;
}

// ---- pinned staging ----------------------------------------------------------
// Every host<->device copy of the manager goes through pinned memory: either
// the shadow buffer of a resident activation, or a region of the grow-only
// staging buffer.  Regions are handed out front to back within one call, so
// no region is reused while a transfer from it may still be in flight.
namespace {
// Bytes per DMA of a staged transfer (CDML_STAGE_CHUNK_MB, default 8): a
// chunk's host copy overlaps the next chunk's DMA.
size_t stage_chunk() {
  static const size_t c = [] {
    const char *e = std::getenv("CDML_STAGE_CHUNK_MB");
    const int mb = e ? std::atoi(e) : 0;
    return size_t(mb > 0 && mb <= 256 ? mb : 8) << 20;
  }();
  return c;
}
size_t round_up(size_t n, size_t a) { return (n + a - 1) / a * a; }
}  // namespace

void *HipAccelerationManager::stage_region(size_t bytes) {
  bytes = round_up(std::max<size_t>(bytes, 1), 256);
  if (stage_off_ + bytes > stage_cap_) {
    sync();  // transfers that still read the current buffer finish first
    const size_t cap = std::max(round_up(bytes, size_t(1) << 20), std::max(stage_cap_ * 2, size_t(4) << 20));
    check(cdml_host_free_pinned(stage_), "cdml_host_free_pinned");
    stage_ = nullptr;
    stage_cap_ = 0;
    check(cdml_host_alloc_pinned(&stage_, cap), "cdml_host_alloc_pinned");
    stage_cap_ = cap;
    stage_off_ = 0;
  }
  void *p = static_cast<char *>(stage_) + stage_off_;
  stage_off_ += bytes;
  return p;
}

// Host -> pinned -> device in chunks: the host copy of chunk i + 1 runs
// while the DMA of chunk i is in flight.
void HipAccelerationManager::stage_upload(void *dev, const void *host, size_t bytes, void *pin) {
  const size_t kChunk = stage_chunk();
  for (size_t off = 0; off < bytes; off += kChunk) {
    const size_t n = std::min(kChunk, bytes - off);
    ParallelMemcpy(static_cast<char *>(pin) + off, static_cast<const char *>(host) + off, n);
    check(cdml_memcpy_h2d_async(static_cast<char *>(dev) + off, static_cast<char *>(pin) + off, n, stream_),
          "cdml_memcpy_h2d_async");
    dirty_ = true;
  }
  stats_.h2d_bytes += bytes;
}

// Device -> pinned -> host for a group of transfers: every chunk's DMA is
// enqueued first, each followed by an event, then each chunk is copied out as
// soon as its event has completed, while the later chunks are still moving.
void HipAccelerationManager::download_all(const std::vector<Xfer> &xs) {
  download_enqueue(xs);
  download_finish(xs);
}

// The chunks of a group of downloads, stage_chunk() bytes each.  (Splitting
// the final chunk into quarters, so that less of the copy out trails the last
// DMA, measured slower: every chunk costs a DMA submission and an event, and
// below 8 MiB those costs outweigh the overlap.)
namespace {
struct Chunk {
  size_t xfer, off, bytes;
};
std::vector<Chunk> plan_chunks(const std::vector<size_t> &sizes) {
  const size_t big = stage_chunk();
  std::vector<Chunk> out;
  for (size_t i = 0; i < sizes.size(); ++i)
    for (size_t off = 0; off < sizes[i]; off += big) out.push_back(Chunk{i, off, std::min(big, sizes[i] - off)});
  return out;
}
template <class X>
std::vector<size_t> sizes_of(const std::vector<X> &xs) {
  std::vector<size_t> v;
  for (const X &x : xs) v.push_back(x.bytes);
  return v;
}
}  // namespace

// The DMA half of download_all: every chunk's copy into pinned memory, each
// followed by an event.  Enqueuing the same transfers again re-records the
// events, so download_finish then waits for the later copies.
void HipAccelerationManager::download_enqueue(const std::vector<Xfer> &xs, cdml_stream st, size_t ev0) {
  if (!st) st = stream_;
  const std::vector<Chunk> chunks = plan_chunks(sizes_of(xs));
  while (events_.size() < ev0 + chunks.size()) {
    cdml_event e = nullptr;
    check(cdml_event_create_sync_only(&e), "cdml_event_create_sync_only");
    events_.push_back(e);
  }
  for (size_t c = 0; c < chunks.size(); ++c) {
    const Xfer &x = xs[chunks[c].xfer];
    check(cdml_memcpy_d2h_async(static_cast<char *>(x.pin) + chunks[c].off,
                                static_cast<const char *>(x.dev) + chunks[c].off, chunks[c].bytes, st),
          "cdml_memcpy_d2h_async");
    check(cdml_event_record(events_[ev0 + c], st), "cdml_event_record");
    dirty_ = true;
  }
}

// The host half: each chunk is copied out of pinned memory as soon as its
// event has completed.
void HipAccelerationManager::download_finish(const std::vector<Xfer> &xs, size_t ev0) {
  const std::vector<Chunk> chunks = plan_chunks(sizes_of(xs));
  for (size_t c = 0; c < chunks.size(); ++c) {
    const Xfer &x = xs[chunks[c].xfer];
    check(cdml_event_synchronize(events_[ev0 + c]), "cdml_event_synchronize");
    ParallelMemcpy(static_cast<char *>(x.host) + chunks[c].off, static_cast<const char *>(x.pin) + chunks[c].off,
                   chunks[c].bytes);
  }
  for (const Xfer &x : xs) stats_.d2h_bytes += x.bytes;
}

void HipAccelerationManager::upload(void *dev, const void *host, size_t bytes) {
  if (bytes == 0) return;
  stage_upload(dev, host, bytes, stage_region(bytes));
}

void HipAccelerationManager::download(void *host, const void *dev, size_t bytes) {
  if (bytes == 0) return;
  download_all({Xfer{host, const_cast<void *>(dev), bytes, stage_region(bytes)}});
}

cdml_stream HipAccelerationManager::copy_stream() {
  if (!copy_) {
    check(cdml_stream_create(&copy_), "cdml_stream_create");
    for (cdml_event &e : kev_) check(cdml_event_create_sync_only(&e), "cdml_event_create_sync_only");
  }
  return copy_;
}

void HipAccelerationManager::sync() {
  if (copy_) check(cdml_stream_synchronize(copy_), "cdml_stream_synchronize");
  check(cdml_stream_synchronize(stream_), "cdml_stream_synchronize");
  dirty_ = false;
}

// ---- resident activations ------------------------------------------------------
// An entry pairs a device buffer with a pinned buffer of the same capacity;
// the pinned one holds exactly the bits of the device one (it was the staging
// buffer of the last transfer in either direction), so comparing the host
// array with it tells whether the device copy is still current.
HipAccelerationManager::ActEntry HipAccelerationManager::act_acquire(size_t bytes) {
  const size_t cap = round_up(std::max<size_t>(bytes, 1), size_t(64) << 10);
  auto fit = act_free_.lower_bound(cap);
  if (fit != act_free_.end() && fit->first <= 2 * cap) {
    ActEntry e = fit->second;
    act_free_.erase(fit);
    return e;
  }
  // give back one buffer: an idle one first, else the least recently used
  // entry that this call does not use; false when nothing is left to give
  auto evict_one = [this]() -> bool {
    if (!act_free_.empty()) {
      auto it = std::prev(act_free_.end());
      act_destroy(it->second);
      act_free_.erase(it);
      return true;
    }
    auto lru = acts_.end();
    for (auto it = acts_.begin(); it != acts_.end(); ++it)
      if (it->second.busy != call_ && (lru == acts_.end() || it->second.last < lru->second.last)) lru = it;
    if (lru == acts_.end()) return false;
    const ActEntry old = lru->second;
    acts_.erase(lru);
    act_destroy(old);
    return true;
  };
  while (act_held_ + cap > act_limit_ || g_act_bytes.load() + cap > g_act_budget.load())
    if (!evict_one()) return ActEntry{};  // over a limit with nothing to give back: the scratch path
  for (;;) {
    ActEntry e;
    e.cap = cap;
    bool ok = true;
    int injected = g_act_alloc_failures.load();
    while (injected > 0 && !g_act_alloc_failures.compare_exchange_weak(injected, injected - 1)) {
    }
    if (injected > 0 || cdml_malloc(&e.dev, cap) != CDML_OK) {
      ok = false;
    } else if (cdml_host_alloc_pinned(&e.pin, cap) != CDML_OK) {
      cdml_free(e.dev);
      ok = false;
    }
    if (ok) {
      act_held_ += cap;
      g_act_bytes += cap;
      return e;
    }
    // out of device or pinned memory: give back more and try again, or
    // leave the array to the scratch path, which the reference's contract
    // (no cache at all) needs anyway
    ++stats_.act_alloc_failures;
    if (!evict_one()) return ActEntry{};
  }
}

void HipAccelerationManager::act_destroy(const ActEntry &e) {
  cdml_free(e.dev);
  cdml_host_free_pinned(e.pin);
  act_held_ -= e.cap;
  g_act_bytes -= e.cap;
}

void HipAccelerationManager::act_release(const ActEntry &e) {
  ActEntry idle;
  idle.dev = e.dev;
  idle.pin = e.pin;
  idle.cap = e.cap;
  act_free_.emplace(e.cap, idle);
}

void HipAccelerationManager::act_drop(const float *key) {
  auto it = acts_.find(key);
  if (it == acts_.end()) return;
  // An entry this call already handed out (the same host pointer with
  // another shape, as x and x[:n] give) may be an argument of a launch still
  // to come: it is parked until the call ends instead of going back to the
  // idle pool, where the next acquire could reuse or free it.
  if (it->second.busy == call_)
    act_parked_.push_back(it->second);
  else
    act_release(it->second);
  acts_.erase(it);
}

// The device copy of activation `m` (uploaded only when it is new or its
// host contents changed since the last transfer).  With the cache off, `m`
// is uploaded into scratch slot `slot`.
const float *HipAccelerationManager::act_in(MatView m, int slot) {
  const size_t bytes = (size_t)m.rows * m.cols * sizeof(float);
  if (act_limit_ == 0 || bytes == 0) {
    void *d = scratch(slot, bytes);
    upload(d, m.data, bytes);
    return static_cast<const float *>(d);
  }
  auto it = acts_.find(m.data);
  if (it != acts_.end() && it->second.rows == m.rows && it->second.cols == m.cols && it->second.dev) {
    ActEntry &e = it->second;
    e.last = ++tick_;
    if (e.busy != call_ && defer_) {
      pending_.push_back(Pending{m.data, e.pin, e.dev, bytes, false});
    } else if (e.busy != call_ && ParallelEqual(m.data, e.pin, bytes)) {
      stats_.h2d_skipped_bytes += bytes;
    } else if (e.busy != call_) {
      stage_upload(e.dev, m.data, bytes, e.pin);
      e.ver = ++ver_;
    }
    e.busy = call_;
    return static_cast<const float *>(e.dev);
  }
  act_drop(m.data);
  ActEntry e = act_acquire(bytes);
  if (!e.dev) {  // no cache memory: the uncached path
    void *d = scratch(slot, bytes);
    upload(d, m.data, bytes);
    return static_cast<const float *>(d);
  }
  e.rows = m.rows;
  e.cols = m.cols;
  e.last = ++tick_;
  e.busy = call_;
  e.ver = ++ver_;
  stage_upload(e.dev, m.data, bytes, e.pin);
  acts_[m.data] = e;
  return static_cast<const float *>(e.dev);
}

// The device copy of an array that the method changes in place (RoPE,
// gradient accumulators): as act_in, and the caller writes the result back
// with act_done, which refreshes the shadow.  A failure in between must drop
// the entry (act_drop), since the device copy may then differ from both.
float *HipAccelerationManager::act_inplace(MatRef m, int slot) {
  float *d = const_cast<float *>(act_in(MatView(m.data, m.rows, m.cols), slot));
  auto it = acts_.find(m.data);
  if (it != acts_.end() && it->second.dev == d) it->second.ver = ++ver_;
  return d;
}

// A device buffer for a result whose host storage `host` [rows, cols] this
// call allocated (or the caller keeps); its entry is keyed by that storage.
float *HipAccelerationManager::act_out(float *host, int rows, int cols, int slot) {
  const size_t bytes = (size_t)rows * cols * sizeof(float);
  if (act_limit_ == 0 || bytes == 0) return static_cast<float *>(scratch(slot, bytes));
  act_drop(host);  // an entry left by a freed array at the same address
  ActEntry e = act_acquire(bytes);
  if (!e.dev) return static_cast<float *>(scratch(slot, bytes));  // no cache memory: the uncached path
  e.rows = rows;
  e.cols = cols;
  e.last = ++tick_;
  e.busy = call_;
  e.ver = ++ver_;
  acts_[host] = e;
  return static_cast<float *>(e.dev);
}

// Downloads each result from its device buffer, through its entry's shadow
// when the buffer belongs to one (the shadow then matches the host again).
void HipAccelerationManager::act_done(std::initializer_list<Out> outs) { download_all(act_transfers(outs)); }

std::vector<HipAccelerationManager::Xfer> HipAccelerationManager::act_transfers(std::initializer_list<Out> outs) {
  std::vector<Xfer> xs;
  for (const Out &o : outs) {
    const size_t bytes = o.floats * sizeof(float);
    if (bytes == 0) continue;
    auto it = acts_.find(o.host);
    void *pin = (it != acts_.end() && it->second.dev == o.dev) ? it->second.pin : stage_region(bytes);
    xs.push_back(Xfer{o.host, const_cast<float *>(o.dev), bytes, pin});
  }
  return xs;
}

// For methods whose kernels write nothing but their results, into buffers
// the caller cannot see yet: the kernel runs on the device copies of the
// inputs and the results' downloads into pinned memory are enqueued behind
// it before the deferred compares of the inputs run, so the compares
// overlap the kernel and the DMA.  If an input changed on the host, it is
// uploaded and the kernel and the downloads run again (the stream orders
// them after the first ones); the results reach the host arrays only after
// the compares, from the last downloads.
void HipAccelerationManager::launch_settle_download(const std::function<void()> &launch,
                                                    std::initializer_list<Out> outs) {
  launch();
  std::vector<Xfer> xs = act_transfers(outs);
  download_enqueue(xs);
  if (!settle()) {
    launch();
    xs = act_transfers(outs);  // an upload may have moved the staging buffer
    download_enqueue(xs);
  }
  download_finish(xs);
}

// The same for a long result computed in two row ranges: launch_rows(0, h),
// then launch_rows(h, rows - h), with the first range's rows of every output
// moving on the copy stream (behind an event) while the kernel computes the
// second, so most of the kernel time hides behind the DMA that bounds the
// call.  before_finish runs after the compares, before the results reach the
// host arrays.
void HipAccelerationManager::launch_split_download(const std::function<void(int, int)> &launch_rows, int rows,
                                                   int h, std::initializer_list<Out> outs,
                                                   const std::function<void()> &before_finish) {
  std::vector<Xfer> xs0, xs1;
  auto plan = [&] {
    const std::vector<Xfer> all = act_transfers(outs);
    xs0.clear();
    xs1.clear();
    for (const Xfer &x : all) {
      const size_t row = x.bytes / rows, off = (size_t)h * row;
      xs0.push_back(Xfer{x.host, x.dev, off, x.pin});
      xs1.push_back(Xfer{static_cast<char *>(x.host) + off, static_cast<char *>(x.dev) + off, x.bytes - off,
                         static_cast<char *>(x.pin) + off});
    }
  };
  plan();
  size_t n0 = plan_chunks(sizes_of(xs0)).size();
  cdml_stream cs = copy_stream();
  auto run = [&] {
    launch_rows(0, h);
    check(cdml_event_record(kev_[0], stream_), "cdml_event_record");
    check(cdml_stream_wait_event(cs, kev_[0]), "cdml_stream_wait_event");
    download_enqueue(xs0, cs, 0);
    launch_rows(h, rows - h);
    check(cdml_event_record(kev_[1], stream_), "cdml_event_record");
    check(cdml_stream_wait_event(cs, kev_[1]), "cdml_stream_wait_event");
    download_enqueue(xs1, cs, n0);
  };
  run();
  if (!settle()) {  // an input changed: the first downloads finish before the kernel runs again
    check(cdml_stream_synchronize(cs), "cdml_stream_synchronize");
    plan();  // an upload may have moved the staging buffer
    n0 = plan_chunks(sizes_of(xs0)).size();
    run();
  }
  if (before_finish) before_finish();
  download_finish(xs0, 0);
  download_finish(xs1, n0);
}

// ---- attention row statistics kept for the backward --------------------------
namespace {
constexpr size_t kLseRecords = 64;
}  // namespace

// A buffer of at least `bytes` for the next record's statistics.
float *HipAccelerationManager::lse_slot(size_t bytes) {
  if (lse_spare_bytes_ < bytes) {
    sync();
    cdml_free(lse_spare_);
    lse_spare_ = nullptr;
    lse_spare_bytes_ = 0;
    check(cdml_malloc(&lse_spare_, bytes), "cdml_malloc");
    lse_spare_bytes_ = bytes;
  }
  return static_cast<float *>(lse_spare_);
}

// Files `r` (whose lse is the spare buffer): it replaces a record of the same
// arrays, or the least recently used one when all slots are taken; the
// replaced record's buffer becomes the spare.
void HipAccelerationManager::lse_record(const LseRecord &r) {
  LseRecord *slot = nullptr;
  for (LseRecord &x : lse_)
    if (x.q == r.q && x.k == r.k && x.v == r.v) slot = &x;
  if (!slot && lse_.size() < kLseRecords) {
    lse_.push_back(LseRecord{});
    slot = &lse_.back();
  }
  if (!slot) {
    slot = &lse_.front();
    for (LseRecord &x : lse_)
      if (x.last < slot->last) slot = &x;
  }
  void *old = slot->lse;
  const size_t old_bytes = slot->lse_bytes;
  *slot = r;
  slot->lse = lse_spare_;
  slot->lse_bytes = lse_spare_bytes_;
  slot->last = ++tick_;
  lse_spare_ = old;
  lse_spare_bytes_ = old ? old_bytes : 0;
}

// The record of a forward on exactly these arrays, if every array's device
// copy is still the one (and the version) the forward saw.
const HipAccelerationManager::LseRecord *HipAccelerationManager::lse_find(
    const float *q, const float *k, const float *v, int batch, int lq, int lk, int dim, int heads, float scale,
    bool causal) {
  auto same = [&](const float *key, void *dev, uint64_t ver) {
    auto it = acts_.find(key);
    return it != acts_.end() && it->second.dev == dev && it->second.ver == ver;
  };
  for (LseRecord &r : lse_) {
    if (r.q != q || r.k != k || r.v != v || r.batch != batch || r.lq != lq || r.lk != lk || r.dim != dim ||
        r.heads != heads || r.scale != scale || r.causal != causal)
      continue;
    if (same(r.q, r.qd, r.qv) && same(r.k, r.kd, r.kv) && same(r.v, r.vd, r.vv) && same(r.o, r.od, r.ov)) {
      r.last = ++tick_;
      return &r;
    }
  }
  return nullptr;
}

// ---- arrays the manager changes in place ---------------------------------------
// A resident weight (MatrixUpdate on a model's weights) is updated in its
// resident copy, whose shadow then follows the new host contents; any other
// array takes the activation path.
float *HipAccelerationManager::inplace_begin(float *host, int rows, int cols, int slot) {
  auto it = resident_.find(host);
  if (it != resident_.end() && it->second.rows == rows && it->second.cols == cols) {
    Resident &r = it->second;
    const size_t bytes = (size_t)rows * cols * sizeof(float);
    if (bytes && !ParallelEqual(r.shadow.data(), host, bytes)) {
      ParallelMemcpy(r.shadow.data(), host, bytes);
      upload(r.dev, r.shadow.data(), bytes);
    }
    return static_cast<float *>(r.dev);
  }
  return act_inplace(MatRef(host, rows, cols), slot);
}

void HipAccelerationManager::inplace_end(float *host, int rows, int cols, const float *dev) {
  const size_t n = (size_t)rows * cols;
  act_done({Out{host, n, dev}});
  auto it = resident_.find(host);
  if (it != resident_.end() && it->second.dev == dev) ParallelMemcpy(it->second.shadow.data(), host, n * sizeof(float));
}

// After a failure between inplace_begin and inplace_end the device copy may
// differ from the host array and its shadow alike: forget it.
void HipAccelerationManager::inplace_fail(float *host) {
  act_drop(host);
  auto it = resident_.find(host);
  if (it != resident_.end()) {
    cdml_stream_synchronize(stream_);
    cdml_free(it->second.dev);
    resident_.erase(it);
  }
}

void HipAccelerationManager::SetActivationCacheLimit(size_t bytes) {
  std::lock_guard<std::mutex> lock(mu_);
  act_limit_ = bytes;
  if (!ready_) return;
  sync();
  for (auto &kv : acts_) act_release(kv.second);
  acts_.clear();
  for (const ActEntry &e : act_parked_) act_release(e);
  act_parked_.clear();
  for (auto &kv : act_free_) act_destroy(kv.second);
  act_free_.clear();
  for (auto &kv : pin_spare_) cdml_host_free_pinned(kv.second);
  pin_spare_.clear();
}

void HipAccelerationManager::SetProcessActivationCacheBudget(size_t bytes) { g_act_budget.store(bytes); }
size_t HipAccelerationManager::ProcessActivationCacheBudget() { return g_act_budget.load(); }
size_t HipAccelerationManager::ProcessActivationCacheBytes() { return g_act_bytes.load(); }
void HipAccelerationManager::InjectActivationAllocFailures(int count) { g_act_alloc_failures.store(count); }

int HipAccelerationManager::activation_cache_entries() {
  std::lock_guard<std::mutex> lock(mu_);
  return (int)acts_.size();
}

HipAccelerationManager::TransferStats HipAccelerationManager::transfer_stats() {
  std::lock_guard<std::mutex> lock(mu_);
  return stats_;
}

// Identity-keyed resident copy with a shadow compare
// (AccelerationManagers/GPU/DeviceResidentCache.cs:44-120): the first call
// with an array uploads it; later calls upload again only when the shape or
// the contents changed.
const float *HipAccelerationManager::resident(const float *host, int rows, int cols) {
  const size_t n = (size_t)rows * cols;
  auto it = resident_.find(host);
  if (it == resident_.end() || it->second.rows != rows || it->second.cols != cols) {
    if (it != resident_.end()) {
      sync();
      cdml_free(it->second.dev);
      resident_.erase(it);
    }
    Resident r;
    r.rows = rows;
    r.cols = cols;
    check(cdml_malloc(&r.dev, n * sizeof(float) + 4), "cdml_malloc");
    r.shadow.assign(host, host + n);
    upload(r.dev, r.shadow.data(), n * sizeof(float));
    auto res = resident_.emplace(host, std::move(r));
    return static_cast<const float *>(res.first->second.dev);
  }
  Resident &r = it->second;
  if (defer_ && n) {
    pending_.push_back(Pending{host, r.shadow.data(), r.dev, n * sizeof(float), true});
  } else if (n && !ParallelEqual(r.shadow.data(), host, n * sizeof(float))) {
    ParallelMemcpy(r.shadow.data(), host, n * sizeof(float));
    upload(r.dev, r.shadow.data(), n * sizeof(float));
  }
  return static_cast<const float *>(r.dev);
}

// ---- ProjectQKV: AccelerationCPU.cs:2005-2069 -----------------------------
std::tuple<Matrix, Matrix, Matrix> HipAccelerationManager::ProjectQKV(MatView input, MatView WQ,
                                                                      VecView biasQ, MatView WK,
                                                                      VecView biasK, MatView WV,
                                                                      VecView biasV) {
  if (input.null()) throw ArgumentNullException("input");
  if (WQ.null()) throw ArgumentNullException("WQ");
  if (WK.null()) throw ArgumentNullException("WK");
  if (WV.null()) throw ArgumentNullException("WV");
  if (biasQ.null()) throw ArgumentNullException("biasQ");
  if (biasK.null()) throw ArgumentNullException("biasK");
  if (biasV.null()) throw ArgumentNullException("biasV");
  const int rows = input.rows, inputDim = input.cols;
  const int qDim = WQ.rows, kDim = WK.rows, vDim = WV.rows;
  if (WQ.cols != inputDim) throw ArgumentException("WQ input dimension does not match input width.", "WQ");
  if (WK.cols != inputDim) throw ArgumentException("WK input dimension does not match input width.", "WK");
  if (WV.cols != inputDim) throw ArgumentException("WV input dimension does not match input width.", "WV");
  if (biasQ.length != qDim) throw ArgumentException("biasQ length does not match WQ output dimension.", "biasQ");
  if (biasK.length != kDim) throw ArgumentException("biasK length does not match WK output dimension.", "biasK");
  if (biasV.length != vDim) throw ArgumentException("biasV length does not match WV output dimension.", "biasV");
  if (qDim != kDim || qDim != vDim) throw ArgumentException("Q, K and V output dimensions must match.");

  if (rows == 0 || qDim == 0) return {Matrix(rows, qDim), Matrix(rows, kDim), Matrix(rows, vDim)};
  std::lock_guard<std::mutex> lock(mu_);
  ensure_ready();
  defer_ = true;
  const float *wq = resident(WQ.data, qDim, inputDim), *wk = resident(WK.data, kDim, inputDim),
              *wv = resident(WV.data, vDim, inputDim);
  const float *bq = resident(biasQ.data, 1, qDim), *bk = resident(biasK.data, 1, kDim),
              *bv = resident(biasV.data, 1, vDim);
  const float *dx = act_in(input, S_X);
  defer_ = false;
  Matrix Q = Matrix::Uninit(rows, qDim), K = Matrix::Uninit(rows, kDim), V = Matrix::Uninit(rows, vDim);
  float *dq = act_out(Q, S_Q), *dk = act_out(K, S_K), *dv = act_out(V, S_V);
  auto launch_rows = [&](int r0, int n) {
    const size_t o = (size_t)r0 * qDim;
    check(cdml_project_qkv(dx + (size_t)r0 * inputDim, wq, bq, wk, bk, wv, bv, dq + o, dk + o, dv + o, n, inputDim,
                           qDim, stream_),
          "cdml_project_qkv");
  };
  const size_t outBytes = (size_t)rows * qDim * sizeof(float);
  if (rows < 2048 || outBytes < (size_t(16) << 20)) {
    launch_settle_download([&] { launch_rows(0, rows); }, {out_of(Q, dq), out_of(K, dk), out_of(V, dv)});
  } else {
    // Two row halves, the first half's rows downloaded while the kernel
    // computes the second.
    const int h = (rows / 2 + 255) / 256 * 256;
    launch_split_download(launch_rows, rows, h, {out_of(Q, dq), out_of(K, dk), out_of(V, dv)}, nullptr);
  }
  sync();
  return {std::move(Q), std::move(K), std::move(V)};
}

// ---- attention core shared by SDPA and MultiHeadAttentionForward -----------
// `batch` independent sequences: q [batch * lq, D], k and v [batch * lk, D].
// Without a mask (head dims up to 128) the forward keeps each row's softmax
// statistics, so a MultiHeadAttentionBackward on the same arrays can start
// from them instead of repeating this pass.
Matrix HipAccelerationManager::attention(MatView q, MatView k, MatView v, int numHeads,
                                         float scale, MaskView mask, bool causal, int batch) {
  const int rq = q.rows, rk = k.rows, dim = q.cols;
  if (rq == 0 || rk == 0 || dim == 0) return Matrix(rq, dim);
  const int lq = rq / batch, lk = rk / batch;
  std::lock_guard<std::mutex> lock(mu_);
  ensure_ready();
  defer_ = true;
  const float *dq = act_in(q, S_Q), *dk = act_in(k, S_K), *dv = act_in(v, S_V);
  defer_ = false;
  Matrix out = Matrix::Uninit(rq, dim);
  float *dout = act_out(out, S_O);
  const uint8_t *dm = nullptr;
  if (!mask.null()) {
    void *m = scratch(S_MASK, (size_t)lq * lk);
    upload(m, mask.data, (size_t)lq * lk);
    dm = static_cast<const uint8_t *>(m);
  }
  const bool keep = act_limit_ > 0 && mask.null() && dim / numHeads <= 128;
  float *lse = keep ? lse_slot((size_t)batch * numHeads * lq * sizeof(float)) : nullptr;
  auto launch = [&] {
    if (lse)
      check(cdml_sdpa_fwd_lse(dq, dim, dk, dim, dv, dim, dout, dim, lse, batch, lq, lk, dim, numHeads, scale,
                              causal ? 1 : 0, nullptr, stream_),
            "cdml_sdpa_fwd_lse");
    else
      check(cdml_sdpa_fwd(dq, dim, dk, dim, dv, dim, dout, dim, batch, lq, lk, dim, numHeads, scale,
                          causal ? 1 : 0, dm, stream_),
            "cdml_sdpa_fwd");
  };
  launch();
  std::vector<Xfer> xs = act_transfers({out_of(out, dout)});
  download_enqueue(xs);  // overlaps the compares below (launch_settle_download)
  if (!settle()) {
    launch();
    xs = act_transfers({out_of(out, dout)});
    download_enqueue(xs);
  }
  if (lse) {
    auto eq = acts_.find(q.data), ek = acts_.find(k.data), ev = acts_.find(v.data), eo = acts_.find(out.ptr());
    if (eq != acts_.end() && ek != acts_.end() && ev != acts_.end() && eo != acts_.end()) {
      LseRecord r;
      r.q = q.data;
      r.k = k.data;
      r.v = v.data;
      r.o = out.ptr();
      r.qd = eq->second.dev;
      r.kd = ek->second.dev;
      r.vd = ev->second.dev;
      r.od = eo->second.dev;
      r.qv = eq->second.ver;
      r.kv = ek->second.ver;
      r.vv = ev->second.ver;
      r.ov = eo->second.ver;
      r.batch = batch;
      r.lq = lq;
      r.lk = lk;
      r.dim = dim;
      r.heads = numHeads;
      r.scale = scale;
      r.causal = causal;
      lse_record(r);
    }
  }
  download_finish(xs);
  sync();
  return out;
}

// ---- ScaledDotProductAttention: AccelerationCPU.cs:1797-1956 ---------------
Matrix HipAccelerationManager::ScaledDotProductAttention(MatView q, MatView k, MatView v,
                                                         int numHeads, MaskView mask, bool causal) {
  if (q.null()) throw ArgumentNullException("q");
  if (k.null()) throw ArgumentNullException("k");
  if (v.null()) throw ArgumentNullException("v");
  if (numHeads <= 0) throw ArgumentOutOfRangeException("numHeads");
  const int queryLen = q.rows, keyLen = k.rows, valueLen = v.rows, dim = q.cols;
  if (queryLen <= 0) throw ArgumentException("Q must contain at least one row.", "q");
  if (keyLen <= 0) throw ArgumentException("K must contain at least one row.", "k");
  if (dim <= 0) throw ArgumentException("Q must contain at least one column.", "q");
  if (k.cols != dim) throw ArgumentException("K width must match Q width.", "k");
  if (v.cols != dim) throw ArgumentException("V width must match Q width.", "v");
  if (valueLen != keyLen) throw ArgumentException("V row count must match K row count.", "v");
  if (dim % numHeads != 0)
    throw ArgumentException("Embedding dimension must be divisible by numHeads.", "numHeads");
  if (!mask.null() && (mask.rows != queryLen || mask.cols != keyLen))
    throw ArgumentException("Mask shape must be [" + std::to_string(queryLen) + "," +
                                std::to_string(keyLen) + "], got [" + std::to_string(mask.rows) +
                                "," + std::to_string(mask.cols) + "].",
                            "mask");
  if (causal && queryLen != keyLen)
    throw ArgumentException(
        "The simple causal path assumes queryLen == keyLen. Use an explicit mask for "
        "cross-attention or cached decoding.");
  const int headDim = dim / numHeads;
  const float scale = 1.0f / std::sqrt((float)headDim);  // AccelerationCPU.cs:1865
  return attention(q, k, v, numHeads, scale, mask, causal);
}

// ---- MultiHeadAttentionForward: AccelerationCPU.cs:1647-1792 ---------------
Matrix HipAccelerationManager::MultiHeadAttentionForward(MatView Q, MatView K, MatView V,
                                                         int numHeads, float scale, MaskView mask) {
  if (Q.null()) throw ArgumentNullException("Q");
  if (K.null()) throw ArgumentNullException("K");
  if (V.null()) throw ArgumentNullException("V");
  const int seqLenQ = Q.rows, seqLenK = K.rows, dim = Q.cols;
  if (K.cols != dim || V.cols != dim)
    throw ArgumentException("Q, K and V must have the same embedding dimension.");
  if (V.rows != seqLenK) throw ArgumentException("K and V must have the same sequence length.");
  if (numHeads <= 0) throw ArgumentOutOfRangeException("numHeads");
  if (dim % numHeads != 0) throw ArgumentException("Embedding dim must be divisible by numHeads.");
  if (!mask.null() && (mask.rows != seqLenQ || mask.cols != seqLenK))
    throw ArgumentException("Mask shape must be [seqLenQ, seqLenK].");
  if (seqLenQ == 0 || seqLenK == 0 || dim / numHeads == 0) return Matrix(seqLenQ, dim);
  return attention(Q, K, V, numHeads, scale, mask, false);
}

// ---- ProjectOutputBatch / BatchDotProductAddBias ---------------------------
Matrix HipAccelerationManager::linear(MatView x, int rowStart, int rowCount, MatView w, VecView b,
                                      int act) {
  const int in = w.cols, out = w.rows;
  if (rowCount == 0 || out == 0) return Matrix(rowCount, out);
  std::lock_guard<std::mutex> lock(mu_);
  ensure_ready();
  defer_ = true;
  const float *dw = resident(w.data, out, in);
  const float *db = resident(b.data, 1, out);
  const float *dx;
  if (rowStart == 0 && rowCount == x.rows) {
    dx = act_in(x, S_X);
  } else {  // a row range of a larger array: staged on its own
    const size_t xb = (size_t)rowCount * in * sizeof(float);
    float *d = static_cast<float *>(scratch(S_X, xb));
    upload(d, x.data + (size_t)rowStart * x.cols, xb);
    dx = d;
  }
  defer_ = false;
  Matrix y = Matrix::Uninit(rowCount, out);
  float *dy = act_out(y, S_O);
  auto launch = [&] {
    check(cdml_linear(dx, in, dw, db, dy, out, rowCount, in, out, act, stream_), "cdml_linear");
  };
  launch_settle_download(launch, {out_of(y, dy)});
  sync();
  return y;
}

// AccelerationCPU.cs:2694-2715.  The reference reads hidden[i, :] for i <
// seqLen and projection rows j < outputDim without checks (an out-of-range
// shape raises IndexOutOfRangeException there); the same shapes are rejected
// here with ArgumentException before any device work.
Matrix HipAccelerationManager::ProjectOutputBatch(MatView hidden, MatView outputProjection,
                                                  VecView outputBias, int seqLen, int outputDim) {
  if (hidden.null()) throw ArgumentNullException("hidden");
  if (outputProjection.null()) throw ArgumentNullException("outputProjection");
  if (outputBias.null()) throw ArgumentNullException("outputBias");
  if (seqLen < 0 || seqLen > hidden.rows) throw ArgumentException("seqLen exceeds the hidden rows.", "seqLen");
  if (outputDim < 0 || outputDim > outputProjection.rows || outputDim > outputBias.length)
    throw ArgumentException("outputDim exceeds the projection rows or bias length.", "outputDim");
  if (outputProjection.cols != hidden.cols)
    throw ArgumentException("Projection width must match the hidden width.", "outputProjection");
  MatView w(outputProjection.data, outputDim, outputProjection.cols);
  return linear(hidden, 0, seqLen, w, VecView(outputBias.data, outputDim), CDML_ACT_NONE);
}

Matrix HipAccelerationManager::BatchDotProductAddBias(MatView weights, MatView inputMatrix,
                                                      VecView bias) {
  if (inputMatrix.null()) throw ArgumentNullException("inputMatrix");
  return BatchDotProductAddBias(weights, inputMatrix, 0, inputMatrix.rows, bias);
}

// AccelerationCPU.cs:352-404
Matrix HipAccelerationManager::BatchDotProductAddBias(MatView weights, MatView inputMatrix,
                                                      int rowStart, int rowCount, VecView bias) {
  if (weights.null()) throw ArgumentNullException("weights");
  if (inputMatrix.null()) throw ArgumentNullException("inputMatrix");
  if (bias.null()) throw ArgumentNullException("bias");
  if (rowStart < 0 || rowCount < 0 || (long long)rowStart + rowCount > inputMatrix.rows)
    throw ArgumentOutOfRangeException("rowStart");
  if (inputMatrix.cols != weights.cols)
    throw ArgumentException("Expected input columns " + std::to_string(weights.cols) + ", got " +
                                std::to_string(inputMatrix.cols),
                            "inputMatrix");
  if (bias.length != weights.rows) throw ArgumentException("Bias length must match output dimension.", "bias");
  if (rowCount == 0 || weights.rows == 0 || weights.cols == 0) {
    Matrix y(rowCount, weights.rows);
    if (weights.cols == 0)  // an empty dot product leaves only the bias
      for (int i = 0; i < rowCount; ++i)
        for (int j = 0; j < weights.rows; ++j) y.at(i, j) = bias.data[j];
    return y;
  }
  return linear(inputMatrix, rowStart, rowCount, weights, bias, CDML_ACT_NONE);
}

// ---- in-place kernels on resident activations ---------------------------------
// A spare pinned buffer of exactly `cap` bytes (nullptr when none can be
// allocated), and its return; at most two spares stay idle per manager.
void *HipAccelerationManager::spare_pin(size_t cap) {
  auto it = pin_spare_.find(cap);
  if (it != pin_spare_.end()) {
    void *p = it->second;
    pin_spare_.erase(it);
    return p;
  }
  void *p = nullptr;
  if (cdml_host_alloc_pinned(&p, cap) != CDML_OK) return nullptr;
  return p;
}

void HipAccelerationManager::spare_put(void *p, size_t cap) {
  pin_spare_.emplace(cap, p);
  while (pin_spare_.size() > 2) {
    auto last = std::prev(pin_spare_.end());
    cdml_host_free_pinned(last->second);
    pin_spare_.erase(last);
  }
}

// An in-place kernel on the resident copy of `m` with the shadow compare
// overlapped: the kernel runs on the device copy and its result is
// downloaded into a spare pinned buffer while the host array is compared
// with the shadow.  If the host array is unchanged, the spare's contents go
// to the host array and the spare becomes the shadow; otherwise the host
// contents are uploaded and the kernel runs again, as without the cache.
// Returns false (nothing done) when `m` has no resident entry this call may
// use, or is too small for the overlap to pay; the caller then takes the
// plain path.
bool HipAccelerationManager::inplace_overlapped(MatRef m, const std::function<void(float *)> &launch) {
  const size_t bytes = (size_t)m.rows * m.cols * sizeof(float);
  if (act_limit_ == 0 || bytes < (size_t(4) << 20)) return false;
  auto it = acts_.find(m.data);
  if (it == acts_.end() || it->second.rows != m.rows || it->second.cols != m.cols || it->second.busy == call_)
    return false;
  const size_t cap = it->second.cap;
  void *spare = spare_pin(cap);
  if (!spare) return false;
  ActEntry &e = it->second;
  e.busy = call_;
  e.last = ++tick_;
  e.ver = ++ver_;  // the device copy changes in every outcome
  float *d = static_cast<float *>(e.dev);
  try {
    launch(d);
    std::vector<Xfer> xs{Xfer{m.data, d, bytes, spare}};
    download_enqueue(xs);
    if (ParallelEqual(m.data, e.pin, bytes)) {
      stats_.h2d_skipped_bytes += bytes;
      download_finish(xs);
      spare_put(e.pin, cap);
      e.pin = spare;
      return true;
    }
    sync();  // the speculative download is done with the device buffer and the spare
    spare_put(spare, cap);
    spare = nullptr;
    stage_upload(d, m.data, bytes, e.pin);
    launch(d);
    download_all({Xfer{m.data, d, bytes, e.pin}});
    return true;
  } catch (...) {
    if (spare) spare_put(spare, cap);
    throw;
  }
}

// ---- RoPE: AccelerationCPU.cs:4855-4982 --------------------------------------
void HipAccelerationManager::ApplyRotaryPositionEmbeddingInPlace(MatRef matrix, int numHeads,
                                                                 float baseTheta, bool inverse) {
  if (!matrix.data) throw ArgumentNullException("matrix");
  if (numHeads <= 0) throw ArgumentOutOfRangeException("numHeads");
  if (!(baseTheta > 0.f) || std::isinf(baseTheta)) throw ArgumentOutOfRangeException("baseTheta");
  const int dim = matrix.cols;
  if (dim % numHeads != 0)
    throw ArgumentException("Embedding dimension must be divisible by number of heads.");
  const int headDim = dim / numHeads;
  if (headDim & 1) throw ArgumentException("RoPE requires an even per-head dimension.");
  if (matrix.rows == 0 || headDim == 0) return;
  std::lock_guard<std::mutex> lock(mu_);
  ensure_ready();
  auto launch = [&](float *dx) {
    check(cdml_rope(dx, matrix.rows, dim, 0, headDim, numHeads, baseTheta, inverse ? 1 : 0, 0, 0,
                    nullptr, stream_),
          "cdml_rope");
  };
  try {
    if (inplace_overlapped(matrix, launch)) {
      sync();
      return;
    }
    float *dx = act_inplace(matrix, S_X);
    launch(dx);
    act_done({Out{matrix.data, (size_t)matrix.rows * dim, dx}});
    sync();
  } catch (...) {
    act_drop(matrix.data);
    throw;
  }
}

void HipAccelerationManager::ApplyRotaryPositionEmbeddingHeadInPlace(MatRef matrix, int startCol,
                                                                     int headDim, float baseTheta,
                                                                     bool inverse) {
  if (!matrix.data) throw ArgumentNullException("matrix");
  if (startCol < 0) throw ArgumentOutOfRangeException("startCol");
  if (headDim < 0) throw ArgumentOutOfRangeException("headDim");
  if (headDim & 1) throw ArgumentException("RoPE requires an even per-head dimension.", "headDim");
  if (!(baseTheta > 0.f) || std::isinf(baseTheta)) throw ArgumentOutOfRangeException("baseTheta");
  if ((long long)startCol + headDim > matrix.cols)
    throw ArgumentException("Head range exceeds matrix embedding dimension.");
  if (matrix.rows == 0 || headDim == 0) return;
  std::lock_guard<std::mutex> lock(mu_);
  ensure_ready();
  float *dx = act_inplace(matrix, S_X);
  try {
    check(cdml_rope(dx, matrix.rows, matrix.cols, startCol, headDim, 1, baseTheta, inverse ? 1 : 0,
                    0, 0, nullptr, stream_),
          "cdml_rope");
    act_done({Out{matrix.data, (size_t)matrix.rows * matrix.cols, dx}});
    sync();
  } catch (...) {
    act_drop(matrix.data);
    throw;
  }
}

// ---- ResidualLayerNorm: AccelerationCPU.cs:1376-1438 ----------------------
Matrix HipAccelerationManager::ResidualLayerNorm(MatView input, MatView subLayer, VecView gamma,
                                                 VecView beta, float epsilon) {
  if (input.null()) throw ArgumentNullException("input");
  if (subLayer.null()) throw ArgumentNullException("subLayer");
  if (gamma.null()) throw ArgumentNullException("gamma");
  if (beta.null()) throw ArgumentNullException("beta");
  const int rows = input.rows, f = input.cols;
  if (subLayer.rows != rows || subLayer.cols != f)
    throw ArgumentException("Residual input dimensions must match.", "subLayer");
  if (gamma.length != f || beta.length != f)
    throw ArgumentException("Layer norm gamma/beta must match the feature dimension.");
  if (rows == 0 || f == 0) return Matrix(rows, f);
  std::lock_guard<std::mutex> lock(mu_);
  ensure_ready();
  defer_ = true;
  const float *dg = resident(gamma.data, 1, f), *db = resident(beta.data, 1, f);
  const float *da = act_in(input, S_X), *dbb = act_in(subLayer, S_Q);
  defer_ = false;
  Matrix out = Matrix::Uninit(rows, f);
  float *dy = act_out(out, S_O);
  auto launch = [&] {
    check(cdml_residual_layernorm(da, dbb, dg, db, dy, rows, f, epsilon, stream_),
          "cdml_residual_layernorm");
  };
  launch_settle_download(launch, {out_of(out, dy)});
  sync();
  return out;
}

// ---- EmbedTokenIds: AccelerationCPU.cs:3463-3515 --------------------------
Matrix HipAccelerationManager::EmbedTokenIds(const std::vector<int> &tokenIds, MatView embedding,
                                             int embeddingDim) {
  if (tokenIds.empty()) return Matrix(0, embeddingDim);
  return EmbedTokenIds(tokenIds, 0, (int)tokenIds.size(), embedding, embeddingDim);
}

Matrix HipAccelerationManager::EmbedTokenIds(const std::vector<int> &tokenIds, int tokenStart,
                                             int tokenCount, MatView embedding, int embeddingDim) {
  if (tokenIds.empty() || tokenCount == 0) return Matrix(0, embeddingDim);
  if (embedding.null()) throw ArgumentNullException("embedding");
  if (tokenStart < 0 || tokenCount < 0 || (long long)tokenStart + tokenCount > (long long)tokenIds.size())
    throw ArgumentOutOfRangeException("tokenStart");
  const int vocab = embedding.rows;
  if (embedding.cols != embeddingDim) throw ArgumentException("Embedding dimension mismatch.", "embedding");
  for (int i = 0; i < tokenCount; ++i) {
    const int t = tokenIds[tokenStart + i];
    if ((unsigned)t >= (unsigned)vocab)
      throw ArgumentOutOfRangeException("tokenIds", "Token out of range: " + std::to_string(t));
  }
  if (embeddingDim == 0) return Matrix(tokenCount, embeddingDim);
  std::lock_guard<std::mutex> lock(mu_);
  ensure_ready();
  const float *dt = resident(embedding.data, vocab, embeddingDim);
  int *dids = static_cast<int *>(scratch(S_IDS, (size_t)tokenCount * sizeof(int)));
  upload(dids, tokenIds.data() + tokenStart, (size_t)tokenCount * sizeof(int));
  Matrix out = Matrix::Uninit(tokenCount, embeddingDim);
  float *dout = act_out(out, S_O);
  check(cdml_embed_tokens(dids, tokenCount, dt, vocab, embeddingDim, dout, nullptr, stream_),
        "cdml_embed_tokens");
  act_done({out_of(out, dout)});
  sync();
  return out;
}

// ---- CreateCausalMask: AccelerationCPU.cs:1566-1586 (host data only) --------
BoolMatrix HipAccelerationManager::CreateCausalMask(int seqLen) {
  if (seqLen < 0) throw ArgumentOutOfRangeException("seqLen");
  BoolMatrix m;
  m.rows = m.cols = seqLen;
  m.data.assign((size_t)seqLen * seqLen, 0);
  for (int i = 0; i < seqLen; ++i)
    for (int j = 0; j <= i; ++j) m.data[(size_t)i * seqLen + j] = 1;
  return m;
}

// ---- FFNForwardBatch: AccelerationCPU.cs:1957-2002 + NeuralNetwork.cs:629-668
Matrix HipAccelerationManager::FFNForwardBatch(MatView input, int seqLen, int outputDim,
                                               const FeedForwardNetwork &ffn) {
  if (input.null()) throw ArgumentNullException("input");
  if (seqLen < 0 || seqLen > input.rows) throw ArgumentOutOfRangeException("seqLen");
  if (ffn.weights.empty()) throw InvalidOperationException("Neural network must have at least input and output layers.");
  if (seqLen == 0) return Matrix(0, ffn.output_size());
  if (input.cols != ffn.input_size())
    throw ArgumentException("Input matrix column count (" + std::to_string(input.cols) +
                                ") must match network input size (" +
                                std::to_string(ffn.input_size()) + ").",
                            "input");
  (void)outputDim;  // the reference's batched route returns the network's own output width
  {
    int w_in = input.cols;
    for (size_t l = 0; l < ffn.weights.size(); ++l) {
      const Matrix &w = ffn.weights[l];
      if (w.cols != w_in) throw ArgumentException("FFN layer widths do not chain.", "ffn");
      if ((int)ffn.biases[l].size() != w.rows) throw ArgumentException("FFN bias length mismatch.", "ffn");
      w_in = w.rows;
    }
  }
  std::lock_guard<std::mutex> lock(mu_);
  ensure_ready();
  int width = input.cols;
  size_t maxw = width;
  for (auto &w : ffn.weights) maxw = std::max(maxw, (size_t)w.rows);
  defer_ = true;
  const float *in0;
  if (seqLen == input.rows) {
    in0 = act_in(input, S_X);
  } else {
    float *d = static_cast<float *>(scratch(S_X, (size_t)seqLen * width * sizeof(float)));
    upload(d, input.data, (size_t)seqLen * width * sizeof(float));
    in0 = d;
  }
  std::vector<const float *> dws(ffn.weights.size()), dbs(ffn.weights.size());
  for (size_t l = 0; l < ffn.weights.size(); ++l) {
    const Matrix &w = ffn.weights[l];
    dws[l] = resident(w.ptr(), w.rows, w.cols);
    dbs[l] = resident(ffn.biases[l].data(), 1, w.rows);
  }
  defer_ = false;
  // hidden layers alternate between two scratch buffers; the last layer
  // writes the result's own buffer
  float *tmp[2] = {static_cast<float *>(scratch(S_Q, (size_t)seqLen * maxw * sizeof(float))),
                   static_cast<float *>(scratch(S_K, (size_t)seqLen * maxw * sizeof(float)))};
  Matrix out = Matrix::Uninit(seqLen, ffn.output_size());
  float *dout = act_out(out, S_O);
  auto launch = [&] {
    const float *cur = in0;
    int wdt = input.cols;
    for (size_t l = 0; l < ffn.weights.size(); ++l) {
      const Matrix &w = ffn.weights[l];
      float *dst = l + 1 == ffn.weights.size() ? dout : tmp[l & 1];
      check(cdml_linear(cur, wdt, dws[l], dbs[l], dst, w.rows, seqLen, wdt, w.rows, ffn.activations[l], stream_),
            "cdml_linear");
      cur = dst;
      wdt = w.rows;
    }
  };
  launch_settle_download(launch, {out_of(out, dout)});
  sync();
  return out;
}

// ---- MultiHeadAttentionBackward: AccelerationCPU.cs:1011-1280 ----------------
std::tuple<Matrix, Matrix, Matrix> HipAccelerationManager::MultiHeadAttentionBackward(
    MatView Q, MatView K, MatView V, MatView dConcatenated, int numHeads, float scale,
    bool useDecoderMask) {
  return attention_backward(Q, K, V, dConcatenated, numHeads, scale, MaskView{}, useDecoderMask);
}

std::tuple<Matrix, Matrix, Matrix> HipAccelerationManager::MultiHeadAttentionBackward(
    MatView Q, MatView K, MatView V, MatView dConcatenated, int numHeads, float scale,
    MaskView mask) {
  return attention_backward(Q, K, V, dConcatenated, numHeads, scale, mask, false);
}

// MultiHeadAttentionBackwardCore's checks (AccelerationCPU.cs:1037-1063) in
// order, then cdml_sdpa_bwd on the manager's stream.
std::tuple<Matrix, Matrix, Matrix> HipAccelerationManager::attention_backward(
    MatView Q, MatView K, MatView V, MatView dO, int numHeads, float scale, MaskView mask,
    bool causal, int batch) {
  if (Q.null()) throw ArgumentNullException("Q");
  if (K.null()) throw ArgumentNullException("K");
  if (V.null()) throw ArgumentNullException("V");
  if (dO.null()) throw ArgumentNullException("dConcatenated");
  if (numHeads <= 0) throw ArgumentOutOfRangeException("numHeads");
  const int lq = Q.rows, lk = K.rows, dim = Q.cols;
  if (K.cols != dim || V.cols != dim)
    throw ArgumentException("Q, K and V must have the same embedding dimension.");
  if (V.rows != lk) throw ArgumentException("K and V must have the same sequence length.");
  if (dO.rows != lq || dO.cols != dim)
    throw ArgumentException("dConcatenated shape must match Q shape.", "dConcatenated");
  if (dim % numHeads != 0)
    throw ArgumentException("Embedding dim must be divisible by numHeads.", "numHeads");
  if (!mask.null() && (mask.rows != lq || mask.cols != lk))
    throw ArgumentException("Mask shape must be [" + std::to_string(lq) + "," + std::to_string(lk) +
                                "], got [" + std::to_string(mask.rows) + "," +
                                std::to_string(mask.cols) + "].",
                            "mask");
  if (lq == 0 || lk == 0 || dim == 0) return {Matrix(lq, dim), Matrix(lk, dim), Matrix(lk, dim)};
  std::lock_guard<std::mutex> lock(mu_);
  ensure_ready();
  const int sq = lq / batch, sk = lk / batch;  // rows per sequence
  const int cflag = causal && mask.null() ? 1 : 0;
  // Workspaces of both forms: recomputing the forward (cdml_sdpa_bwd) and
  // starting from the forward's saved statistics (cdml_sdpa_bwd_saved); each
  // with room for the dS blocks when the shape can use them (dQ as one
  // product), as long as the extra bytes stay under the cap and allocate.
  size_t base_ws = 0, stored_ws = 0, saved_stored_ws = 0;
  check(cdml_sdpa_bwd_workspace_size(batch, sq, sk, dim, numHeads, &base_ws), "cdml_sdpa_bwd_workspace_size");
  check(cdml_sdpa_bwd_stored_ds_workspace_size(batch, sq, sk, dim, numHeads, cflag, &stored_ws),
        "cdml_sdpa_bwd_stored_ds_workspace_size");
  check(cdml_sdpa_bwd_saved_workspace_size(batch, sq, sk, dim, numHeads, cflag, &saved_stored_ws),
        "cdml_sdpa_bwd_saved_workspace_size");
  const size_t saved_base_ws = (size_t)batch * numHeads * sq * sizeof(float);
  size_t ws = SdpaBackwardWorkspaceChoice(base_ws, stored_ws, kStoredDsExtraBytesCap);
  size_t ws_saved = SdpaBackwardWorkspaceChoice(saved_base_ws, saved_stored_ws, kStoredDsExtraBytesCap);
  void *dws = try_scratch(S_WS, std::max(ws, ws_saved));
  if (!dws) {
    ws = base_ws;
    ws_saved = saved_base_ws;
    dws = scratch(S_WS, std::max(ws, ws_saved));
  }
  defer_ = true;
  const float *dq_in = act_in(Q, S_Q), *dk_in = act_in(K, S_K), *dv_in = act_in(V, S_V);
  const float *ddo = act_in(dO, S_O);
  defer_ = false;
  Matrix dQ = Matrix::Uninit(lq, dim), dK = Matrix::Uninit(lk, dim), dV = Matrix::Uninit(lk, dim);
  float *gq = act_out(dQ, S_DQ), *gk = act_out(dK, S_DK), *gv = act_out(dV, S_DV);
  const uint8_t *dm = nullptr;
  if (!mask.null()) {
    void *m = scratch(S_MASK, (size_t)lq * lk);
    upload(m, mask.data, (size_t)lq * lk);
    dm = static_cast<const uint8_t *>(m);
  }
  // the forward's statistics, when it ran on these very arrays (no mask)
  auto saved = [&]() -> const LseRecord * {
    return mask.null() ? lse_find(Q.data, K.data, V.data, batch, sq, sk, dim, numHeads, scale, causal) : nullptr;
  };
  auto launch = [&](const LseRecord *r) {
    if (r)
      check(cdml_sdpa_bwd_saved(dq_in, dim, dk_in, dim, dv_in, dim, static_cast<const float *>(r->od), dim,
                                static_cast<const float *>(r->lse), ddo, dim, gq, dim, gk, dim, gv, dim, batch, sq,
                                sk, dim, numHeads, scale, cflag, nullptr, dws, ws_saved, stream_),
            "cdml_sdpa_bwd_saved");
    else
      check(cdml_sdpa_bwd(dq_in, dim, dk_in, dim, dv_in, dim, ddo, dim, gq, dim, gk, dim, gv, dim, batch, sq, sk,
                          dim, numHeads, scale, causal ? 1 : 0, dm, dws, ws, stream_),
            "cdml_sdpa_bwd");
  };
  const LseRecord *rec = saved();
  launch(rec);
  if (!settle()) {  // an input changed on the host: its record, if any, no longer holds
    rec = saved();
    launch(rec);
  }
  if (rec) ++stats_.backward_from_saved;
  act_done({out_of(dQ, gq), out_of(dK, gk), out_of(dV, gv)});
  sync();
  return {std::move(dQ), std::move(dK), std::move(dV)};
}

// ---- BackpropQKV: AccelerationCPU.cs:2071-2186 ------------------------------
Matrix HipAccelerationManager::BackpropQKV(MatView input, MatView dQ, MatView dK, MatView dV,
                                           MatView WQ, MatView WK, MatView WV, MatRef WQGrad,
                                           VecRef biasQGrad, MatRef WKGrad, VecRef biasKGrad,
                                           MatRef WVGrad, VecRef biasVGrad) {
  if (input.null()) throw ArgumentNullException("input");
  if (dQ.null()) throw ArgumentNullException("dQ");
  if (dK.null()) throw ArgumentNullException("dK");
  if (dV.null()) throw ArgumentNullException("dV");
  if (WQ.null()) throw ArgumentNullException("WQ");
  if (WK.null()) throw ArgumentNullException("WK");
  if (WV.null()) throw ArgumentNullException("WV");
  if (!WQGrad.data) throw ArgumentNullException("WQGrad");
  if (!WKGrad.data) throw ArgumentNullException("WKGrad");
  if (!WVGrad.data) throw ArgumentNullException("WVGrad");
  if (biasQGrad.null()) throw ArgumentNullException("biasQGrad");
  if (biasKGrad.null()) throw ArgumentNullException("biasKGrad");
  if (biasVGrad.null()) throw ArgumentNullException("biasVGrad");
  const int rows = input.rows, inputDim = input.cols;
  const int outputDim = WQ.rows;
  if (WK.rows != outputDim || WV.rows != outputDim)
    throw ArgumentException("Q, K and V dimensions must match.");
  if (WQ.cols != inputDim || WK.cols != inputDim || WV.cols != inputDim)
    throw ArgumentException("Q/K/V weight input dimensions must match input width.");
  if (dQ.rows != rows || dK.rows != rows || dV.rows != rows)
    throw ArgumentException("dQ, dK and dV row counts must match input row count.");
  if (dQ.cols != outputDim || dK.cols != outputDim || dV.cols != outputDim)
    throw ArgumentException("dQ, dK and dV widths must match Q/K/V output dimension.");
  if (WQGrad.rows != outputDim || WQGrad.cols != inputDim)
    throw ArgumentException("WQGrad shape mismatch.", "WQGrad");
  if (WKGrad.rows != outputDim || WKGrad.cols != inputDim)
    throw ArgumentException("WKGrad shape mismatch.", "WKGrad");
  if (WVGrad.rows != outputDim || WVGrad.cols != inputDim)
    throw ArgumentException("WVGrad shape mismatch.", "WVGrad");
  if (biasQGrad.length != outputDim || biasKGrad.length != outputDim || biasVGrad.length != outputDim)
    throw ArgumentException("Q/K/V bias gradient lengths must match output dimension.");
  if (rows == 0 || inputDim == 0 || outputDim == 0) return Matrix(rows, inputDim);
  std::lock_guard<std::mutex> lock(mu_);
  ensure_ready();
  const size_t wb = (size_t)outputDim * inputDim * sizeof(float), bb = (size_t)outputDim * sizeof(float);
  const float *wq = resident(WQ.data, outputDim, inputDim), *wk = resident(WK.data, outputDim, inputDim),
              *wv = resident(WV.data, outputDim, inputDim);
  const float *dx_in = act_in(input, S_X);
  const float *ddq = act_in(dQ, S_DQ), *ddk = act_in(dK, S_DK), *ddv = act_in(dV, S_DV);
  Matrix dInput = Matrix::Uninit(rows, inputDim);
  float *ddx = act_out(dInput, S_O);
  float *gw[3] = {static_cast<float *>(scratch(S_GW0, wb)), static_cast<float *>(scratch(S_GW1, wb)),
                  static_cast<float *>(scratch(S_GW2, wb))};
  float *gb[3] = {static_cast<float *>(scratch(S_GB0, bb)), static_cast<float *>(scratch(S_GB1, bb)),
                  static_cast<float *>(scratch(S_GB2, bb))};
  MatRef hw[3] = {WQGrad, WKGrad, WVGrad};
  VecRef hb[3] = {biasQGrad, biasKGrad, biasVGrad};
  for (int i = 0; i < 3; ++i) {
    upload(gw[i], hw[i].data, wb);
    upload(gb[i], hb[i].data, bb);
  }
  size_t ws = 0;
  check(cdml_backprop_qkv_workspace_size(rows, inputDim, outputDim, &ws),
        "cdml_backprop_qkv_workspace_size");
  void *dws = ws ? scratch(S_WS, ws) : nullptr;
  check(cdml_backprop_qkv(dx_in, ddq, ddk, ddv, wq, wk, wv, gw[0], gb[0], gw[1], gb[1], gw[2], gb[2],
                          ddx, rows, inputDim, outputDim, dws, ws, stream_),
        "cdml_backprop_qkv");
  act_done({out_of(dInput, ddx), Out{hw[0].data, wb / 4, gw[0]}, Out{hb[0].data, bb / 4, gb[0]},
            Out{hw[1].data, wb / 4, gw[1]}, Out{hb[1].data, bb / 4, gb[1]}, Out{hw[2].data, wb / 4, gw[2]},
            Out{hb[2].data, bb / 4, gb[2]}});
  sync();
  return dInput;
}

// Shared body of BackpropLinearProjection / BackpropOutputProjection
// (AccelerationCPU.cs:2188-2270): wgrad += dy^T x, bgrad += column sums of
// dy, dx (+)= dy w, over `rows` rows of x and dy.
void HipAccelerationManager::linear_backward(MatView x, MatView dy, int rows, MatView w,
                                             MatRef wgrad, VecRef bgrad, float *dx_host,
                                             bool accumulate_dx) {
  const int in = w.cols, out = w.rows;
  if (rows == 0 || in == 0) return;
  std::lock_guard<std::mutex> lock(mu_);
  ensure_ready();
  const size_t xb = (size_t)rows * in * sizeof(float);
  const size_t wb = (size_t)out * in * sizeof(float), bb = (size_t)out * sizeof(float);
  const float *dw = resident(w.data, out, in);
  // x and dy are whole arrays when `rows` covers them, else row prefixes
  auto rows_of = [&](MatView m, int slot) -> const float * {
    if (m.rows == rows) return act_in(m, slot);
    const size_t b = (size_t)rows * m.cols * sizeof(float);
    float *d = static_cast<float *>(scratch(slot, b));
    upload(d, m.data, b);
    return d;
  };
  const float *dxin = rows_of(x, S_X);
  const float *ddy = out > 0 ? rows_of(dy, S_Q) : nullptr;
  float *gw = static_cast<float *>(scratch(S_GW0, wb > 0 ? wb : 4));
  float *gb = static_cast<float *>(scratch(S_GB0, bb > 0 ? bb : 4));
  if (out > 0) {
    upload(gw, wgrad.data, wb);
    upload(gb, bgrad.data, bb);
  }
  // dX: accumulated in place into the caller's array, or a new result
  float *ddx = accumulate_dx ? act_inplace(MatRef(dx_host, rows, in), S_O) : act_out(dx_host, rows, in, S_O);
  try {
  if (out > 0) {
    size_t ws = 0;
    check(cdml_linear_backward_workspace_size(rows, in, out, &ws),
          "cdml_linear_backward_workspace_size");
    void *dws = ws ? scratch(S_WS, ws) : nullptr;
    check(cdml_linear_backward(dxin, in, ddy, out, dw, ddx, in, gw, gb, rows, in, out,
                               accumulate_dx ? 1 : 0, dws, ws, stream_),
          "cdml_linear_backward");
  } else if (!accumulate_dx) {
    check(cdml_zero_f32_async(ddx, (size_t)rows * in, stream_), "cdml_zero_f32_async");
  }
  if (out > 0)
    act_done({Out{dx_host, xb / 4, ddx}, Out{wgrad.data, wb / 4, gw}, Out{bgrad.data, bb / 4, gb}});
  else
    act_done({Out{dx_host, xb / 4, ddx}});
  sync();
  } catch (...) {
    act_drop(dx_host);
    throw;
  }
}

// ---- BackpropLinearProjection: AccelerationCPU.cs:2188-2227 -----------------
// The reference indexes the arrays without checks (a mismatch surfaces as an
// IndexOutOfRangeException mid-update); here every shape is checked before
// any device work, with ArgumentException.
void HipAccelerationManager::BackpropLinearProjection(MatView input, MatView dOutput,
                                                      MatView weights, MatRef weightGrad,
                                                      VecRef biasGrad, MatRef dInput) {
  if (input.null()) throw ArgumentNullException("input");
  if (dOutput.null()) throw ArgumentNullException("dOutput");
  if (weights.null()) throw ArgumentNullException("weights");
  if (!weightGrad.data) throw ArgumentNullException("weightGrad");
  if (biasGrad.null()) throw ArgumentNullException("biasGrad");
  if (!dInput.data) throw ArgumentNullException("dInput");
  const int rows = input.rows, in = input.cols, out = dOutput.cols;
  if (dOutput.rows != rows) throw ArgumentException("dOutput rows must match input rows.", "dOutput");
  if (weights.rows != out || weights.cols != in)
    throw ArgumentException("weights must be [outDim, inDim].", "weights");
  if (weightGrad.rows != out || weightGrad.cols != in)
    throw ArgumentException("weightGrad must be [outDim, inDim].", "weightGrad");
  if (biasGrad.length != out) throw ArgumentException("biasGrad length must match outDim.", "biasGrad");
  if (dInput.rows != rows || dInput.cols != in)
    throw ArgumentException("dInput must be [seqLen, inDim].", "dInput");
  linear_backward(input, dOutput, rows, weights, weightGrad, biasGrad, dInput.data, true);
}

// ---- BackpropOutputProjection: AccelerationCPU.cs:2229-2270 ------------------
Matrix HipAccelerationManager::BackpropOutputProjection(MatView dLogits, MatView input,
                                                        MatView weights, MatRef weightGrad,
                                                        VecRef biasGrad, int seqLen, int outputDim,
                                                        int embeddingDim) {
  if (dLogits.null()) throw ArgumentNullException("dLogits");
  if (input.null()) throw ArgumentNullException("input");
  if (weights.null()) throw ArgumentNullException("weights");
  if (!weightGrad.data) throw ArgumentNullException("weightGrad");
  if (biasGrad.null()) throw ArgumentNullException("biasGrad");
  if (seqLen < 0 || seqLen > dLogits.rows || seqLen > input.rows)
    throw ArgumentException("seqLen exceeds the dLogits or input rows.", "seqLen");
  if (outputDim < 0 || dLogits.cols != outputDim)
    throw ArgumentException("dLogits width must equal outputDim.", "outputDim");
  if (embeddingDim < 0 || input.cols != embeddingDim)
    throw ArgumentException("input width must equal embeddingDim.", "embeddingDim");
  if (weights.rows != outputDim || weights.cols != embeddingDim)
    throw ArgumentException("weights must be [outputDim, embeddingDim].", "weights");
  if (weightGrad.rows != outputDim || weightGrad.cols != embeddingDim)
    throw ArgumentException("weightGrad must be [outputDim, embeddingDim].", "weightGrad");
  if (biasGrad.length != outputDim) throw ArgumentException("biasGrad length must match outputDim.", "biasGrad");
  Matrix dX(seqLen, embeddingDim);
  linear_backward(input, dLogits, seqLen, weights, weightGrad, biasGrad, dX.ptr(), false);
  return dX;
}

// ---- BackpropInputProjection: AccelerationCPU.cs:2280-2330 -------------------
// The weight gradient is the same dY^T X product as the other projections'
// (cdml_linear_backward with no input gradient): X is the input's row slice
// at its own row stride, dY the first seqLen * embeddingDim floats of dX.
void HipAccelerationManager::BackpropInputProjection(MatView dX, MatView continuousInput, int inputRowStart,
                                                     MatRef weightGrad, VecRef biasGrad, int seqLen,
                                                     int embeddingDim, int inputFeatureDim) {
  if (dX.null()) throw ArgumentNullException("dX");
  if (continuousInput.null()) throw ArgumentNullException("continuousInput");
  if (!weightGrad.data) throw ArgumentNullException("weightGrad");
  if (biasGrad.null()) throw ArgumentNullException("biasGrad");
  if (inputRowStart < 0 || seqLen < 0 || (long long)inputRowStart + seqLen > continuousInput.rows)
    throw ArgumentOutOfRangeException("inputRowStart", "Invalid input row slice: start=" + std::to_string(inputRowStart) +
                                                           ", count=" + std::to_string(seqLen) + ", rows=" +
                                                           std::to_string(continuousInput.rows) + ".");
  if (inputFeatureDim > continuousInput.cols || dX.rows < seqLen || dX.cols < embeddingDim)
    throw ArgumentException("Input or gradient dimensions are smaller than the requested projection dimensions.");
  // the reference indexes weightGrad[e * inputFeatureDim + f] and biasGrad[e]
  // without a check (IndexOutOfRangeException mid-update); checked up front
  if (embeddingDim < 0 || inputFeatureDim < 0 ||
      (long long)weightGrad.rows * weightGrad.cols < (long long)embeddingDim * inputFeatureDim ||
      biasGrad.length < embeddingDim)
    throw ArgumentException("weightGrad or biasGrad is smaller than embeddingDim x inputFeatureDim.");
  if (seqLen == 0 || embeddingDim == 0) return;
  std::lock_guard<std::mutex> lock(mu_);
  ensure_ready();
  const int ldin = continuousInput.cols;
  const float *din = act_in(continuousInput, S_X) + (size_t)inputRowStart * ldin;
  const float *ddx = act_in(dX, S_Q);
  const size_t wb = (size_t)embeddingDim * inputFeatureDim * sizeof(float), bb = (size_t)embeddingDim * sizeof(float);
  float *gw = static_cast<float *>(scratch(S_GW0, wb > 0 ? wb : 4));
  float *gb = static_cast<float *>(scratch(S_GB0, bb));
  if (wb > 0) upload(gw, weightGrad.data, wb);
  upload(gb, biasGrad.data, bb);
  size_t ws = 0;
  check(cdml_linear_backward_workspace_size(seqLen, inputFeatureDim, embeddingDim, &ws),
        "cdml_linear_backward_workspace_size");
  void *dws = ws ? scratch(S_WS, ws) : nullptr;
  check(cdml_linear_backward(din, ldin, ddx, embeddingDim, nullptr, nullptr, inputFeatureDim, wb > 0 ? gw : nullptr,
                             gb, seqLen, inputFeatureDim, embeddingDim, 0, dws, ws, stream_),
        "cdml_linear_backward");
  if (wb > 0)
    act_done({Out{weightGrad.data, wb / 4, gw}, Out{biasGrad.data, bb / 4, gb}});
  else
    act_done({Out{biasGrad.data, bb / 4, gb}});
  sync();
}

// ---- MatrixMultiply / MatrixMultiplyTranspose: AccelerationCPU.cs:159-250 ----
Matrix HipAccelerationManager::MatrixMultiply(MatView A, MatView B) {
  if (A.null()) throw ArgumentNullException("A");
  if (B.null()) throw ArgumentNullException("B");
  if (A.cols != B.rows)
    throw ArgumentException("Matrix dimensions don't match: [" + std::to_string(A.rows) + "x" +
                            std::to_string(A.cols) + "] * [" + std::to_string(B.rows) + "x" +
                            std::to_string(B.cols) + "]");
  if (A.rows == 0 || B.cols == 0 || A.cols == 0) return Matrix(A.rows, B.cols);
  std::lock_guard<std::mutex> lock(mu_);
  ensure_ready();
  const float *da = act_in(A, S_X), *db = act_in(B, S_Q);
  Matrix Cm = Matrix::Uninit(A.rows, B.cols);
  float *dc = act_out(Cm, S_O);
  check(cdml_matmul(da, A.cols, db, B.cols, dc, B.cols, A.rows, A.cols, B.cols, stream_), "cdml_matmul");
  act_done({out_of(Cm, dc)});
  sync();
  return Cm;
}

Matrix HipAccelerationManager::MatrixMultiplyTranspose(MatView A, MatView B) {
  if (A.null()) throw ArgumentNullException("A");
  if (B.null()) throw ArgumentNullException("B");
  if (A.cols != B.cols) throw ArgumentException("Matrix dimensions don't match for A*B^T");
  if (A.rows == 0 || B.rows == 0 || A.cols == 0) return Matrix(A.rows, B.rows);
  std::lock_guard<std::mutex> lock(mu_);
  ensure_ready();
  const float *da = act_in(A, S_X), *db = act_in(B, S_Q);
  Matrix Cm = Matrix::Uninit(A.rows, B.rows);
  float *dc = act_out(Cm, S_O);
  check(cdml_linear(da, A.cols, db, nullptr, dc, B.rows, A.rows, A.cols, B.rows, CDML_ACT_NONE, stream_),
        "cdml_linear");
  act_done({out_of(Cm, dc)});
  sync();
  return Cm;
}

// ---- ResidualLayerNormForward: AccelerationCPU.cs:1440-1514 -------------------
std::tuple<Matrix, std::vector<float>, std::vector<float>, Matrix, Matrix>
HipAccelerationManager::ResidualLayerNormForward(MatView input, MatView subLayer, VecView gamma,
                                                 VecView beta, float epsilon) {
  if (input.null()) throw ArgumentNullException("input");
  if (subLayer.null()) throw ArgumentNullException("subLayer");
  if (gamma.null()) throw ArgumentNullException("gamma");
  if (beta.null()) throw ArgumentNullException("beta");
  const int rows = input.rows, f = input.cols;
  if (subLayer.rows != rows || subLayer.cols != f)
    throw ArgumentException("Residual input dimensions must match.", "subLayer");
  if (gamma.length != f || beta.length != f)
    throw ArgumentException("Layer norm gamma/beta must match the feature dimension.");
  if (f > 2048) throw ArgumentException("ResidualLayerNormForward supports up to 2048 features.", "input");
  std::vector<float> mean(rows), var(rows);
  if (rows == 0 || f == 0)
    return {Matrix(rows, f), std::move(mean), std::move(var), Matrix(rows, f), Matrix(rows, f)};
  std::lock_guard<std::mutex> lock(mu_);
  ensure_ready();
  const float *dg = resident(gamma.data, 1, f), *dbt = resident(beta.data, 1, f);
  const float *da = act_in(input, S_X), *dbb = act_in(subLayer, S_Q);
  Matrix out = Matrix::Uninit(rows, f), norm = Matrix::Uninit(rows, f), res = Matrix::Uninit(rows, f);
  float *dy = act_out(out, S_O), *dn = act_out(norm, S_K), *dr = act_out(res, S_V);
  float *dm = static_cast<float *>(scratch(S_DQ, (size_t)rows * 8));
  check(cdml_residual_layernorm_fwd(da, dbb, dg, dbt, dy, dm, dm + rows, dr, dn, rows, f, epsilon, stream_),
        "cdml_residual_layernorm_fwd");
  act_done({out_of(out, dy), out_of(norm, dn), out_of(res, dr), Out{mean.data(), (size_t)rows, dm},
            Out{var.data(), (size_t)rows, dm + rows}});
  sync();
  return {std::move(out), std::move(mean), std::move(var), std::move(norm), std::move(res)};
}

// ---- LayerNormBackward: AccelerationCPU.cs:1516-1564 ----------------------------
// The reference indexes its arguments without checks; every shape is checked
// here first (ArgumentException).
std::tuple<Matrix, std::vector<float>, std::vector<float>>
HipAccelerationManager::LayerNormBackward(MatView dOut, MatView normalized, VecView gamma, MatView input,
                                          VecView mean, VecView variance, float epsilon) {
  if (dOut.null()) throw ArgumentNullException("dOut");
  if (normalized.null()) throw ArgumentNullException("normalized");
  if (gamma.null()) throw ArgumentNullException("gamma");
  if (input.null()) throw ArgumentNullException("input");
  if (mean.null()) throw ArgumentNullException("mean");
  if (variance.null()) throw ArgumentNullException("variance");
  const int rows = dOut.rows, f = dOut.cols;
  if (normalized.rows != rows || normalized.cols != f || input.rows != rows || input.cols != f)
    throw ArgumentException("normalized and input must have dOut's shape.");
  if (gamma.length != f) throw ArgumentException("gamma must match the feature dimension.", "gamma");
  if (mean.length < rows || variance.length < rows)
    throw ArgumentException("mean and variance need one entry per row.");
  if (f > 2048) throw ArgumentException("LayerNormBackward supports up to 2048 features.", "dOut");
  std::vector<float> dg(f), db(f);
  if (rows == 0 || f == 0) return {Matrix(rows, f), std::move(dg), std::move(db)};
  std::lock_guard<std::mutex> lock(mu_);
  ensure_ready();
  const float *dd = act_in(dOut, S_X), *dn = act_in(normalized, S_Q), *di = act_in(input, S_K);
  Matrix dx = Matrix::Uninit(rows, f);
  float *dxo = act_out(dx, S_O);
  float *dmv = static_cast<float *>(scratch(S_DQ, (size_t)rows * 8));
  float *dgb = static_cast<float *>(scratch(S_GB0, (size_t)f * 8 + 4 * (size_t)f));
  float *dgam = dgb + 2 * (size_t)f;
  size_t ws = 0;
  check(cdml_layernorm_backward_workspace_size(rows, f, &ws), "cdml_layernorm_backward_workspace_size");
  void *dws = scratch(S_WS, ws);
  upload(dmv, mean.data, (size_t)rows * 4);
  upload(dmv + rows, variance.data, (size_t)rows * 4);
  upload(dgam, gamma.data, (size_t)f * 4);
  check(cdml_layernorm_backward(dd, nullptr, dn, dgam, di, dmv, dmv + rows, dxo, dgb, dgb + f, rows, f, epsilon,
                                0, dws, ws, stream_),
        "cdml_layernorm_backward");
  act_done({out_of(dx, dxo), Out{dg.data(), (size_t)f, dgb}, Out{db.data(), (size_t)f, dgb + f}});
  sync();
  return {std::move(dx), std::move(dg), std::move(db)};
}

// ---- CrossEntropyLossAndGradient: AccelerationCPU.cs:2372-2440 -----------------
std::pair<float, Matrix> HipAccelerationManager::CrossEntropyLossAndGradient(
    MatView logits, const std::vector<int> &targets, int targetStart, int effectiveLen) {
  if (logits.null()) throw ArgumentNullException("logits");
  if (targetStart < 0 || effectiveLen < 0 || (long long)targetStart + effectiveLen > (long long)targets.size())
    throw ArgumentOutOfRangeException("targetStart");
  const int rows = logits.rows, v = logits.cols;
  if (effectiveLen == 0) return {0.f, Matrix(rows, v)};
  // the reference reads row i < effectiveLen and the target's column without
  // checks; both are checked here
  if (effectiveLen > rows) throw ArgumentException("effectiveLen exceeds the logits rows.", "effectiveLen");
  for (int i = 0; i < effectiveLen; ++i)
    if ((unsigned)targets[targetStart + i] >= (unsigned)v)
      throw ArgumentOutOfRangeException("targets", "Target out of range: " + std::to_string(targets[targetStart + i]));
  std::lock_guard<std::mutex> lock(mu_);
  ensure_ready();
  const float *dlog = act_in(logits, S_X);
  int *dt = static_cast<int *>(scratch(S_IDS, (size_t)effectiveLen * 4));
  float *dloss = static_cast<float *>(scratch(S_BIAS, 4));
  size_t ws = 0;
  check(cdml_cross_entropy_workspace_size(rows, &ws), "cdml_cross_entropy_workspace_size");
  void *dws = scratch(S_WS, ws);
  upload(dt, targets.data() + targetStart, (size_t)effectiveLen * 4);
  Matrix dl = Matrix::Uninit(rows, v);
  float *dgrad = act_out(dl, S_O);
  check(cdml_cross_entropy(dlog, v, dt, rows, v, effectiveLen, 1.0f, 1.0f, dloss, dgrad, v, dws, ws, stream_),
        "cdml_cross_entropy");
  float loss = 0.f;
  act_done({out_of(dl, dgrad), Out{&loss, 1, dloss}});
  sync();
  return {loss, std::move(dl)};
}

// ---- MSELossAndGradient: AccelerationCPU.cs:2442-2490 -------------------------
std::pair<float, Matrix> HipAccelerationManager::MSELossAndGradient(MatView predictions, MatView targets,
                                                                    int targetStart, int effectiveLen) {
  if (predictions.null()) throw ArgumentNullException("predictions");
  if (targets.null()) throw ArgumentNullException("targets");
  const int rows = predictions.rows, o = predictions.cols;
  if (targetStart < 0 || effectiveLen < 0 || (long long)targetStart + effectiveLen > targets.rows || targets.cols != o)
    throw ArgumentException("Target shape must match predictions for the effective length and target offset.",
                            "targets");
  if (effectiveLen == 0 || o == 0) return {0.f, Matrix(rows, o)};
  // the reference reads prediction rows i < effectiveLen without a check
  if (effectiveLen > rows) throw ArgumentException("effectiveLen exceeds the prediction rows.", "effectiveLen");
  std::lock_guard<std::mutex> lock(mu_);
  ensure_ready();
  const size_t tbytes = (size_t)effectiveLen * o * 4;
  const float *dp = act_in(predictions, S_X);
  float *dt = static_cast<float *>(scratch(S_Q, tbytes));
  float *dloss = static_cast<float *>(scratch(S_BIAS, 4));
  void *dws = scratch(S_WS, (size_t)rows * 4);
  upload(dt, targets.data + (size_t)targetStart * o, tbytes);
  Matrix d = Matrix::Uninit(rows, o);
  float *dd = act_out(d, S_K);
  check(cdml_mse_loss(dp, o, dt, o, rows, o, effectiveLen, 1.0f, 1.0f, dloss, dd, o, dws, (size_t)rows * 4, stream_),
        "cdml_mse_loss");
  float loss = 0.f;
  act_done({out_of(d, dd), Out{&loss, 1, dloss}});
  sync();
  return {loss, std::move(d)};
}

// ---- AccumulateTokenEmbeddingGrad: AccelerationCPU.cs:2339-2370 ----------------
void HipAccelerationManager::AccumulateTokenEmbeddingGrad(MatRef embeddingGrad, MatView dX,
                                                          const std::vector<int> &tokenIds, int tokenStart,
                                                          int seqLen, int embeddingDim) {
  if (!embeddingGrad.data) throw ArgumentNullException("embeddingGrad");
  if (dX.null()) throw ArgumentNullException("dX");
  if (tokenStart < 0 || seqLen < 0 || (long long)tokenStart + seqLen > (long long)tokenIds.size())
    throw ArgumentOutOfRangeException("tokenStart");
  if (embeddingGrad.cols != embeddingDim || dX.cols != embeddingDim || dX.rows < seqLen)
    throw ArgumentException("embeddingGrad and dX must be [*, embeddingDim] with seqLen rows of dX.");
  const int vocab = embeddingGrad.rows;
  for (int i = 0; i < seqLen; ++i)
    if ((unsigned)tokenIds[tokenStart + i] >= (unsigned)vocab)
      throw ArgumentOutOfRangeException("tokenIds", "Token out of range: " + std::to_string(tokenIds[tokenStart + i]));
  if (seqLen == 0 || embeddingDim == 0) return;
  // rows grouped by token, each group in row order (the reference's summation order)
  std::vector<int> order(seqLen);
  for (int i = 0; i < seqLen; ++i) order[i] = i;
  std::stable_sort(order.begin(), order.end(),
                   [&](int a, int b) { return tokenIds[tokenStart + a] < tokenIds[tokenStart + b]; });
  std::vector<int> start, token;
  for (int i = 0; i < seqLen; ++i)
    if (i == 0 || tokenIds[tokenStart + order[i]] != tokenIds[tokenStart + order[i - 1]]) {
      start.push_back(i);
      token.push_back(tokenIds[tokenStart + order[i]]);
    }
  start.push_back(seqLen);
  std::lock_guard<std::mutex> lock(mu_);
  ensure_ready();
  float *dg = act_inplace(embeddingGrad, S_O);
  const float *dx;
  if (dX.rows == seqLen) {
    dx = act_in(dX, S_X);
  } else {
    const size_t xb = (size_t)seqLen * embeddingDim * 4;
    float *d = static_cast<float *>(scratch(S_X, xb));
    upload(d, dX.data, xb);
    dx = d;
  }
  int *di = static_cast<int *>(scratch(S_IDS, ((size_t)seqLen * 3 + 1) * 4));
  upload(di, order.data(), (size_t)seqLen * 4);
  upload(di + seqLen, start.data(), start.size() * 4);
  upload(di + 2 * seqLen + 1, token.data(), token.size() * 4);
  try {
    check(cdml_embedding_grad(dg, dx, nullptr, embeddingDim, di, di + seqLen, di + 2 * seqLen + 1,
                              (int)token.size(), embeddingDim, stream_),
          "cdml_embedding_grad");
    act_done({Out{embeddingGrad.data, (size_t)vocab * embeddingDim, dg}});
    sync();
  } catch (...) {
    act_drop(embeddingGrad.data);
    throw;
  }
}

// ---- elementwise methods of the training step ----------------------------------
namespace {
enum ElemOp { OP_ZERO, OP_ADD, OP_SCALE, OP_UPDATE };
}  // namespace

// One in-place elementwise operation on host array `host` [rows, cols]:
// zero, += src, *= a, or -= a * src (MatrixUpdate), on its device copy, with
// the result written back to the host array.
void HipAccelerationManager::elementwise_inplace(float *host, int rows, int cols, const float *src, int op,
                                                 float a) {
  const size_t n = (size_t)rows * cols;
  if (n == 0) return;
  std::lock_guard<std::mutex> lock(mu_);
  ensure_ready();
  float *d = nullptr;
  if (op == OP_ZERO) {  // the old contents do not matter: no compare, no upload
    auto it = resident_.find(host);
    d = (it != resident_.end() && it->second.rows == rows && it->second.cols == cols)
            ? static_cast<float *>(it->second.dev)
            : act_out(host, rows, cols, S_O);
  } else {
    d = inplace_begin(host, rows, cols, S_O);
  }
  try {
    const float *ds = src ? act_in(MatView(src, rows, cols), S_X) : nullptr;
    switch (op) {
      case OP_ZERO: check(cdml_zero_f32_async(d, n, stream_), "cdml_zero_f32_async"); break;
      case OP_ADD: check(cdml_add_inplace(d, ds, n, stream_), "cdml_add_inplace"); break;
      case OP_SCALE: check(cdml_scale_f32(d, a, n, stream_), "cdml_scale_f32"); break;
      default: check(cdml_update_f32(d, ds, a, n, stream_), "cdml_update_f32"); break;
    }
    inplace_end(host, rows, cols, d);
    sync();
  } catch (...) {
    inplace_fail(host);
    throw;
  }
}

float HipAccelerationManager::elementwise_norm(const float *host, int rows, int cols) {
  const size_t n = (size_t)rows * cols;
  if (n == 0) return 0.f;
  std::lock_guard<std::mutex> lock(mu_);
  ensure_ready();
  const float *d = act_in(MatView(host, rows, cols), S_X);
  size_t ws = 0;
  check(cdml_sum_squares_workspace_size(&ws), "cdml_sum_squares_workspace_size");
  float *dws = static_cast<float *>(scratch(S_WS, ws + sizeof(float)));
  check(cdml_sum_squares(d, n, dws + ws / sizeof(float), dws, ws, stream_), "cdml_sum_squares");
  float out = 0.f;
  act_done({Out{&out, 1, dws + ws / sizeof(float)}});
  sync();
  return out;
}

// ZeroMatrix / ZeroVector: AccelerationCPU.cs:507-520
void HipAccelerationManager::ZeroMatrix(MatRef matrix) {
  if (!matrix.data) throw ArgumentNullException("matrix");
  elementwise_inplace(matrix.data, matrix.rows, matrix.cols, nullptr, OP_ZERO, 0.f);
}
void HipAccelerationManager::ZeroVector(VecRef vector) {
  if (vector.null()) throw ArgumentNullException("vector");
  elementwise_inplace(vector.data, 1, vector.length, nullptr, OP_ZERO, 0.f);
}
// MatrixAddInPlace: AccelerationCPU.cs:522-546
void HipAccelerationManager::MatrixAddInPlace(MatRef target, MatView addend) {
  if (!target.data) throw ArgumentNullException("target");
  if (addend.null()) throw ArgumentNullException("addend");
  if (addend.rows != target.rows || addend.cols != target.cols)
    throw ArgumentException("Matrix dimensions must match.", "addend");
  elementwise_inplace(target.data, target.rows, target.cols, addend.data, OP_ADD, 0.f);
}
// VectorAccumulate: AccelerationCPU.cs:548-568 (the reference reads
// source[j] for every j < target.Length; a shorter source is rejected here)
void HipAccelerationManager::VectorAccumulate(VecRef target, VecView source) {
  if (target.null()) throw ArgumentNullException("target");
  if (source.null()) throw ArgumentNullException("source");
  if (source.length < target.length) throw ArgumentException("source is shorter than target.", "source");
  elementwise_inplace(target.data, 1, target.length, source.data, OP_ADD, 0.f);
}
// MatrixSquaredNorm / VectorSquaredNorm: AccelerationCPU.cs:2493-2512
float HipAccelerationManager::MatrixSquaredNorm(MatView matrix) {
  if (matrix.null()) throw ArgumentNullException("matrix");
  return elementwise_norm(matrix.data, matrix.rows, matrix.cols);
}
float HipAccelerationManager::VectorSquaredNorm(VecView vector) {
  if (vector.null()) throw ArgumentNullException("vector");
  return elementwise_norm(vector.data, 1, vector.length);
}
// MatrixScaleInPlace / VectorScaleInPlace: AccelerationCPU.cs:2514-2546
void HipAccelerationManager::MatrixScaleInPlace(MatRef matrix, float scale) {
  if (!matrix.data) throw ArgumentNullException("matrix");
  elementwise_inplace(matrix.data, matrix.rows, matrix.cols, nullptr, OP_SCALE, scale);
}
void HipAccelerationManager::VectorScaleInPlace(VecRef vector, float scale) {
  if (vector.null()) throw ArgumentNullException("vector");
  elementwise_inplace(vector.data, 1, vector.length, nullptr, OP_SCALE, scale);
}
// MatrixUpdate / VectorUpdate: AccelerationCPU.cs:2548-2597
void HipAccelerationManager::MatrixUpdate(MatRef weights, MatView gradients, float learningRate) {
  if (!weights.data) throw ArgumentNullException("weights");
  if (gradients.null()) throw ArgumentNullException("gradients");
  if (gradients.rows != weights.rows || gradients.cols != weights.cols)
    throw ArgumentException("Matrix dimensions must match.", "gradients");
  elementwise_inplace(weights.data, weights.rows, weights.cols, gradients.data, OP_UPDATE, learningRate);
}
void HipAccelerationManager::VectorUpdate(VecRef weights, VecView gradients, float learningRate) {
  if (weights.null()) throw ArgumentNullException("weights");
  if (gradients.null()) throw ArgumentNullException("gradients");
  if (gradients.length < weights.length) throw ArgumentException("gradients is shorter than weights.", "gradients");
  elementwise_inplace(weights.data, 1, weights.length, gradients.data, OP_UPDATE, learningRate);
}

// ---- capabilities the reference's trainer runs inline ----------------------------
Matrix HipAccelerationManager::SegmentedAttentionForward(MatView q, MatView k, MatView v, int numHeads,
                                                         int segmentLength, int segmentCount, bool causal) {
  if (q.null()) throw ArgumentNullException("q");
  if (k.null()) throw ArgumentNullException("k");
  if (v.null()) throw ArgumentNullException("v");
  if (numHeads <= 0) throw ArgumentOutOfRangeException("numHeads");
  const int totalRows = q.rows, dim = q.cols;
  // TransformerTrainer.cs:726-731
  if (segmentLength <= 0 || segmentCount <= 0 || (long long)totalRows != (long long)segmentLength * segmentCount)
    throw ArgumentException("Invalid segmented attention shape.");
  if (k.rows != totalRows || v.rows != totalRows || k.cols != dim || v.cols != dim)
    throw ArgumentException("Q, K and V must have the same shape.");
  if (dim % numHeads != 0) throw ArgumentException("Embedding dimension must be divisible by numHeads.", "numHeads");
  const float scale = 1.0f / std::sqrt((float)(dim / numHeads));  // :734
  return attention(q, k, v, numHeads, scale, MaskView{}, causal, segmentCount);
}

std::tuple<Matrix, Matrix, Matrix> HipAccelerationManager::SegmentedMultiHeadAttentionBackward(
    MatView Q, MatView K, MatView V, MatView dConcatenated, int numHeads, float scale, int segmentLength,
    int segmentCount, bool causal) {
  if (Q.null()) throw ArgumentNullException("Q");
  if (numHeads <= 0) throw ArgumentOutOfRangeException("numHeads");
  // TransformerTrainer.cs:1000-1006
  if (segmentLength <= 0 || segmentCount <= 0 || (long long)Q.rows != (long long)segmentLength * segmentCount)
    throw ArgumentException("Invalid segmented attention backward shape.");
  return attention_backward(Q, K, V, dConcatenated, numHeads, scale, MaskView{}, causal, segmentCount);
}

void HipAccelerationManager::ApplySegmentedRotaryInPlace(MatRef q, MatRef k, int numHeads, int segmentLength,
                                                         bool inverse) {
  if (!q.data) throw ArgumentNullException("q");
  if (!k.data) throw ArgumentNullException("k");
  if (numHeads <= 0) throw ArgumentOutOfRangeException("numHeads");
  if (segmentLength <= 0) throw ArgumentOutOfRangeException("segmentLength");
  if (k.rows != q.rows || k.cols != q.cols) throw ArgumentException("Q and K must have the same shape.");
  const int dim = q.cols;
  if (dim % numHeads != 0)
    throw ArgumentException("Embedding dimension must be divisible by number of heads.");
  const int headDim = dim / numHeads;
  if (headDim & 1) throw ArgumentException("RoPE requires an even per-head dimension.");
  if (q.rows == 0 || headDim == 0) return;
  std::lock_guard<std::mutex> lock(mu_);
  ensure_ready();
  float *dq = act_inplace(q, S_Q);
  float *dk = act_inplace(k, S_K);
  try {
    for (float *d : {dq, dk})
      check(cdml_rope(d, q.rows, dim, 0, headDim, numHeads, 10000.0f, inverse ? 1 : 0, 0, segmentLength, nullptr,
                      stream_),
            "cdml_rope");
    act_done({Out{q.data, (size_t)q.rows * dim, dq}, Out{k.data, (size_t)k.rows * dim, dk}});
    sync();
  } catch (...) {
    act_drop(q.data);
    act_drop(k.data);
    throw;
  }
}

// NeuralNetwork.ComputeInputGradientBatch: NeuralNetwork.cs:773-882
Matrix HipAccelerationManager::FFNInputGradientBatch(MatView input, MatView dOutput, const FeedForwardNetwork &ffn,
                                                     const std::vector<MatRef> &weightGradients,
                                                     const std::vector<VecRef> &biasGradients) {
  if (input.null()) throw ArgumentNullException("input");
  if (dOutput.null()) throw ArgumentNullException("dOutput");
  if (ffn.weights.empty()) throw InvalidOperationException("Neural network must have at least input and output layers.");
  const int rows = input.rows, inputDim = input.cols, outputDim = dOutput.cols;
  const int nl = (int)ffn.weights.size();
  if (dOutput.rows != rows) throw ArgumentException("dOutput row count must match input row count.", "dOutput");
  if (inputDim != ffn.input_size())
    throw ArgumentException("Input matrix column count (" + std::to_string(inputDim) +
                                ") must match network input size (" + std::to_string(ffn.input_size()) + ").",
                            "input");
  if (outputDim != ffn.output_size())
    throw ArgumentException("dOutput column count (" + std::to_string(outputDim) +
                                ") must match network output size (" + std::to_string(ffn.output_size()) + ").",
                            "dOutput");
  if ((int)weightGradients.size() != nl || (int)biasGradients.size() != nl)
    throw ArgumentException("Gradient storage must contain one entry per non-input layer.");
  for (int l = 0; l < nl; ++l) {
    const Matrix &w = ffn.weights[l];
    if (l > 0 && w.cols != ffn.weights[l - 1].rows) throw ArgumentException("FFN layer widths do not chain.", "ffn");
    if ((int)ffn.biases[l].size() != w.rows) throw ArgumentException("FFN bias length mismatch.", "ffn");
    if (!weightGradients[l].data || weightGradients[l].rows != w.rows || weightGradients[l].cols != w.cols)
      throw ArgumentException("Weight gradient shape does not match layer shape.", "weightGradients");
    if (biasGradients[l].null() || biasGradients[l].length != w.rows)
      throw ArgumentException("Bias gradient length does not match layer size.", "biasGradients");
  }
  if (ffn.activations.back() != None)
    throw ArgumentException("FFNInputGradientBatch takes networks whose output layer has no activation.", "ffn");
  if (rows == 0) return Matrix(0, inputDim);
  std::lock_guard<std::mutex> lock(mu_);
  ensure_ready();
  // forward with pre-activations for the hidden layers (the output layer's
  // own values are not needed: its derivative is 1)
  if ((int)ffn_scratch_.size() < 2 * nl + 2) ffn_scratch_.resize(2 * nl + 2);
  auto buf = [&](int i, size_t bytes) -> float * {
    DeviceBuf &b = ffn_scratch_[i];
    if (b.bytes < bytes) {
      sync();
      check(cdml_free(b.p), "cdml_free");
      b.p = nullptr;
      b.bytes = 0;
      check(cdml_malloc(&b.p, bytes), "cdml_malloc");
      b.bytes = bytes;
    }
    return static_cast<float *>(b.p);
  };
  const float *x0 = act_in(input, S_X);
  const float *dy = act_in(dOutput, S_Q);
  std::vector<const float *> dw(nl), db(nl), xin(nl);
  std::vector<float *> z(nl, nullptr);
  xin[0] = x0;
  for (int l = 0; l < nl; ++l) {
    const Matrix &w = ffn.weights[l];
    dw[l] = resident(w.ptr(), w.rows, w.cols);
    db[l] = resident(ffn.biases[l].data(), 1, w.rows);
    if (l + 1 < nl) {
      z[l] = buf(2 * l, (size_t)rows * w.rows * sizeof(float));
      float *y = buf(2 * l + 1, (size_t)rows * w.rows * sizeof(float));
      check(cdml_linear_preact(xin[l], w.cols, dw[l], db[l], z[l], y, w.rows, rows, w.cols, w.rows,
                               ffn.activations[l], stream_),
            "cdml_linear_preact");
      xin[l + 1] = y;
    }
  }
  std::vector<float *> gw(nl), gb(nl);
  size_t ws = 0;
  for (int l = 0; l < nl; ++l) {
    size_t w1 = 0;
    check(cdml_linear_backward_workspace_size(rows, ffn.weights[l].cols, ffn.weights[l].rows, &w1),
          "cdml_linear_backward_workspace_size");
    ws = std::max(ws, w1);
  }
  void *dws = ws ? scratch(S_WS, ws) : nullptr;
  Matrix dInput = Matrix::Uninit(rows, inputDim);
  float *dxo = act_out(dInput, S_O);
  int started = 0;
  try {
    for (int l = 0; l < nl; ++l, ++started) {
      gw[l] = inplace_begin(weightGradients[l].data, weightGradients[l].rows, weightGradients[l].cols, S_GW0);
      gb[l] = inplace_begin(biasGradients[l].data, 1, biasGradients[l].length, S_GB0);
    }
    // deltas from the output layer down (currentDeltas = dOutput for an
    // output layer without activation); layer l's input gradient carries
    // act'(z of layer l - 1) into the next delta
    const float *delta = dy;
    for (int l = nl - 1; l >= 0; --l) {
      const Matrix &w = ffn.weights[l];
      float *dxl = l > 0 ? buf(2 * nl + (l & 1), (size_t)rows * w.cols * sizeof(float)) : dxo;
      check(cdml_linear_backward_act(xin[l], w.cols, delta, w.rows, dw[l], l > 0 ? z[l - 1] : nullptr,
                                     l > 0 ? ffn.activations[l - 1] : CDML_ACT_NONE, nullptr, dxl, w.cols, gw[l],
                                     gb[l], rows, w.cols, w.rows, dws, ws, stream_),
            "cdml_linear_backward_act");
      delta = dxl;
    }
    std::vector<Xfer> xs;
    act_done({out_of(dInput, dxo)});
    for (int l = 0; l < nl; ++l) {
      inplace_end(weightGradients[l].data, weightGradients[l].rows, weightGradients[l].cols, gw[l]);
      inplace_end(biasGradients[l].data, 1, biasGradients[l].length, gb[l]);
    }
    sync();
  } catch (...) {
    for (int l = 0; l < started; ++l) {
      inplace_fail(weightGradients[l].data);
      inplace_fail(biasGradients[l].data);
    }
    throw;
  }
  return dInput;
}

// ---- decode capability ------------------------------------------------------
Matrix HipAccelerationManager::DecodeSelfAttention(MatRef q, MatRef k, MatView v, MatRef keys,
                                                   MatRef values, int absolutePosition,
                                                   int numHeads) {
  if (!q.data) throw ArgumentNullException("q");
  if (!k.data) throw ArgumentNullException("k");
  if (v.null()) throw ArgumentNullException("v");
  if (!keys.data) throw ArgumentNullException("keys");
  if (!values.data) throw ArgumentNullException("values");
  if (q.rows != 1 || k.rows != 1 || v.rows != 1)
    throw ArgumentException("Incremental RoPE expects single-row Q and K matrices.");
  const int dim = q.cols;
  if (k.cols != dim || v.cols != dim) throw ArgumentException("Q and K must have the same embedding dimension.");
  if (numHeads <= 0 || dim % numHeads != 0)
    throw ArgumentException("Embedding dimension must be divisible by number of heads.", "numHeads");
  const int headDim = dim / numHeads;
  if (headDim & 1) throw ArgumentException("RoPE requires an even per-head dimension.");
  if (keys.cols != dim || values.cols != dim || values.rows != keys.rows)
    throw ArgumentException("Key/value caches must be [maxSeq, D] with D the query width.");
  if (absolutePosition < 0 || absolutePosition >= keys.rows)
    throw InvalidOperationException("Decoder KV cache is full.");
  Matrix out(1, dim);
  if (dim == 0) return out;
  std::lock_guard<std::mutex> lock(mu_);
  ensure_ready();
  const size_t row = (size_t)dim * sizeof(float);
  DecodeMirror &m = decode_[keys.data];
  if (m.rows != keys.rows || m.cols != dim) {
    sync();
    cdml_free(m.k);
    cdml_free(m.v);
    m = DecodeMirror{};
    check(cdml_malloc(&m.k, keys.rows * row), "cdml_malloc");
    check(cdml_malloc(&m.v, keys.rows * row), "cdml_malloc");
    m.rows = keys.rows;
    m.cols = dim;
  }
  if (m.uploaded != absolutePosition) {  // not the rows this manager appended: refresh
    upload(m.k, keys.data, (size_t)absolutePosition * row);
    upload(m.v, values.data, (size_t)absolutePosition * row);
  }
  float *dq = static_cast<float *>(scratch(S_Q, row));
  float *dout = static_cast<float *>(scratch(S_O, row));
  int *dlen = static_cast<int *>(scratch(S_KVLEN, sizeof(int)));
  float *dk = static_cast<float *>(m.k) + (size_t)absolutePosition * dim;
  float *dv = static_cast<float *>(m.v) + (size_t)absolutePosition * dim;
  size_t ws = 0;
  check(cdml_decode_attn_workspace_size(1, keys.rows, dim, numHeads, &ws),
        "cdml_decode_attn_workspace_size");
  void *dws = scratch(S_WS, ws);
  upload(dq, q.data, row);
  upload(dk, k.data, row);
  upload(dv, v.data, row);
  check(cdml_rope(dq, 1, dim, 0, headDim, numHeads, 10000.0f, 0, absolutePosition, 0, nullptr, stream_),
        "cdml_rope");
  check(cdml_rope(dk, 1, dim, 0, headDim, numHeads, 10000.0f, 0, absolutePosition, 0, nullptr, stream_),
        "cdml_rope");
  check(cdml_fill_i32_async(dlen, 1, absolutePosition + 1, stream_), "cdml_fill_i32_async");
  const float scale = 1.0f / std::sqrt((float)headDim);  // LanguageModel.cs:368
  check(cdml_decode_attn(dq, static_cast<const float *>(m.k), static_cast<const float *>(m.v), dlen,
                         dout, 1, keys.rows, dim, numHeads, scale, dws, ws, stream_),
        "cdml_decode_attn");
  download(q.data, dq, row);
  download(k.data, dk, row);
  download(out.ptr(), dout, row);
  sync();
  m.uploaded = absolutePosition + 1;
  std::memcpy(keys.data + (size_t)absolutePosition * dim, k.data, row);
  std::memcpy(values.data + (size_t)absolutePosition * dim, v.data, row);
  return out;
}

}  // namespace cdml_host
