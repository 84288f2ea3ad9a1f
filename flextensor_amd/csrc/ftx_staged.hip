// Staged host-to-device copies from pageable memory, and a parallel host memcpy.
//
// A pageable source (an ordinary allocation, or a POSIX shared-memory mapping
// that cannot be page-locked in place) cannot be read by the SDMA engines
// directly. The staged engine copies it in pieces through three page-locked
// staging buffers per device:
//
//   for piece j:  wait until buffer j%3's previous DMA has finished (host wait
//                 on its event), copy the piece into it with the host thread
//                 pool, enqueue hipMemcpyAsync(buffer -> device) on the caller's
//                 stream and record the buffer's event after it.
//
// The host copy of piece j+1 runs while the SDMA engine moves the pieces
// before it; with three buffers two DMAs stay queued while the host fills the
// third, so jitter in the host copy (which shares host memory bandwidth with
// the DMA) does not idle the link. Pieces ramp from a sixteenth of the policy
// size up to the full size so the first DMA starts early. A copy runs at
// about the slower of the two rates. The call returns once the
// last piece is enqueued; the DMA itself stays stream-ordered. The host work
// happens at call time, so a staged copy cannot be captured into a graph
// (the entry point rejects capturing streams).
//
// The host thread pool: a fixed set of worker threads plus the caller share
// one copy job, split into parts that each thread claims with an atomic
// counter. Every job is a separate object held by the threads working on it,
// so a slow worker that wakes after its job finished finds no parts left and
// cannot touch the next job.
#include <algorithm>
#include <atomic>
#include <condition_variable>
#include <cstring>
#include <memory>
#include <mutex>
#include <thread>
#include <vector>

#include "ftx_internal.h"

namespace ftx {
namespace {

constexpr int kMaxDevices = 64;
constexpr size_t kMinPartBytes = size_t(1) << 20;

struct CopyJob {
  uint8_t *dst = nullptr;
  const uint8_t *src = nullptr;
  size_t n = 0;
  size_t part = 0;
  size_t parts = 0;
  std::atomic<size_t> next{0};
  std::atomic<size_t> done{0};
};

class HostCopyPool {
 public:
  ~HostCopyPool() { shutdown(); }

  // Stops and joins the worker threads. Later copies run on the caller alone.
  void shutdown() {
    std::vector<std::thread> workers;
    {
      std::lock_guard<std::mutex> lock(m_);
      stop_ = true;
      workers.swap(workers_);
    }
    cv_.notify_all();
    for (auto &t : workers) t.join();
  }

  // Copies n bytes with up to `threads` threads (the caller is one of them).
  void copy(void *dst, const void *src, size_t n, int threads) {
    if (n == 0) return;
    threads = std::max(1, threads);
    size_t part = std::max(kMinPartBytes, (n + 4 * threads - 1) / (4 * threads));
    part = (part + 63) / 64 * 64;
    const size_t parts = (n + part - 1) / part;
    auto job = std::make_shared<CopyJob>();
    job->dst = static_cast<uint8_t *>(dst);
    job->src = static_cast<const uint8_t *>(src);
    job->n = n;
    job->part = part;
    job->parts = parts;
    bool shared = false;
    if (parts > 1 && threads > 1) {
      std::lock_guard<std::mutex> lock(m_);
      if (!stop_) {
        while (static_cast<int>(workers_.size()) < threads - 1) workers_.emplace_back([this] { loop(); });
        job_ = job;
        ++gen_;
        shared = true;
      }
    }
    if (shared) cv_.notify_all();
    run(*job);
    std::unique_lock<std::mutex> lock(m_);
    done_cv_.wait(lock, [&] { return job->done.load() == job->parts; });
    if (job_ == job) job_.reset();
  }

 private:
  void run(CopyJob &j) {
    size_t count = 0;
    for (size_t i; (i = j.next.fetch_add(1)) < j.parts;) {
      const size_t off = i * j.part;
      std::memcpy(j.dst + off, j.src + off, std::min(j.part, j.n - off));
      ++count;
    }
    if (count != 0 && j.done.fetch_add(count) + count == j.parts) {
      std::lock_guard<std::mutex> lock(m_);
      done_cv_.notify_all();
    }
  }

  void loop() {
    uint64_t seen = 0;
    for (;;) {
      std::shared_ptr<CopyJob> job;
      {
        std::unique_lock<std::mutex> lock(m_);
        cv_.wait(lock, [&] { return stop_ || gen_ != seen; });
        if (stop_) return;
        seen = gen_;
        job = job_;
      }
      if (job) run(*job);
    }
  }

  std::mutex m_;
  std::condition_variable cv_;
  std::condition_variable done_cv_;
  std::vector<std::thread> workers_;
  std::shared_ptr<CopyJob> job_;
  uint64_t gen_ = 0;
  bool stop_ = false;
};

constexpr int kStagingBuffers = 3;  // two DMAs stay queued while the host fills the third

struct StagingState {
  void *buf[kStagingBuffers] = {};
  hipEvent_t done[kStagingBuffers] = {};
  size_t bytes = 0;  // per buffer
};

std::mutex g_stage_mutex;  // guards the policy and the staging buffers
size_t g_piece_bytes = size_t(64) << 20;
int g_threads = 0;  // 0: chosen from the host's core count
StagingState g_stage[kMaxDevices];

HostCopyPool &pool() {
  static HostCopyPool p;
  return p;
}

int default_threads() {
  const unsigned hw = std::thread::hardware_concurrency();
  return static_cast<int>(std::clamp<unsigned>(hw / 2, 1u, 8u));
}

// Staging buffers of the current device, (re)allocated to `bytes` each.
int staging(size_t bytes, StagingState **out) {
  int dev = 0;
  FTX_HIP(hipGetDevice(&dev));
  if (dev < 0 || dev >= kMaxDevices) return fail(FTX_ERR_UNSUPPORTED, "device index out of range");
  StagingState &st = g_stage[dev];
  if (st.bytes != bytes) {
    for (int b = 0; b < kStagingBuffers; ++b) {
      if (st.done[b]) FTX_HIP(hipEventSynchronize(st.done[b]));
      if (st.buf[b]) FTX_HIP(hipHostFree(st.buf[b]));
      st.buf[b] = nullptr;
    }
    st.bytes = 0;
    for (int b = 0; b < kStagingBuffers; ++b) {
      hipError_t err = hipHostMalloc(&st.buf[b], bytes, hipHostMallocDefault);
      if (err != hipSuccess) {
        (void)hipGetLastError();
        st.buf[b] = nullptr;
        return fail(FTX_ERR_OOM, "hipHostMalloc of a staging buffer failed");
      }
      if (!st.done[b]) FTX_HIP(hipEventCreateWithFlags(&st.done[b], hipEventDisableTiming));
    }
    st.bytes = bytes;
  }
  *out = &st;
  return FTX_OK;
}

}  // namespace

int staged_shutdown() {
  pool().shutdown();
  int first = FTX_OK;
  auto keep = [&first](hipError_t err, const char *what) {
    if (err != hipSuccess && first == FTX_OK) first = hip_fail(err, what);
    if (err != hipSuccess) (void)hipGetLastError();
  };
  std::lock_guard<std::mutex> lock(g_stage_mutex);
  int prev = -1;
  bool any = false;
  for (int d = 0; d < kMaxDevices; ++d) {
    StagingState &st = g_stage[d];
    bool held = false;
    for (int b = 0; b < kStagingBuffers; ++b) held = held || st.buf[b] || st.done[b];
    if (!held) continue;
    if (!any) {
      any = true;
      if (hipGetDevice(&prev) != hipSuccess) {
        (void)hipGetLastError();
        prev = -1;
      }
    }
    hipError_t err = hipSetDevice(d);
    keep(err, "hipSetDevice at shutdown");
    if (err != hipSuccess) continue;
    for (int b = 0; b < kStagingBuffers; ++b) {
      if (st.done[b]) {
        keep(hipEventSynchronize(st.done[b]), "hipEventSynchronize(staging buffer)");
        keep(hipEventDestroy(st.done[b]), "hipEventDestroy(staging buffer)");
        st.done[b] = nullptr;
      }
      if (st.buf[b]) {
        keep(hipHostFree(st.buf[b]), "hipHostFree(staging buffer)");
        st.buf[b] = nullptr;
      }
    }
    st.bytes = 0;
  }
  if (prev >= 0 && hipSetDevice(prev) != hipSuccess) (void)hipGetLastError();
  return first;
}

int set_staging_policy(size_t piece_bytes, int threads) {
  if (piece_bytes < (size_t(1) << 20) || piece_bytes > (size_t(1) << 30))
    return fail(FTX_ERR_INVALID, "staging piece must be between 1 MiB and 1 GiB");
  if (threads < 0 || threads > 64) return fail(FTX_ERR_INVALID, "threads must be 0 (automatic) or in [1, 64]");
  std::lock_guard<std::mutex> lock(g_stage_mutex);
  g_piece_bytes = piece_bytes;
  g_threads = threads;
  return FTX_OK;
}

void get_staging_policy(size_t *piece_bytes, int *threads) {
  std::lock_guard<std::mutex> lock(g_stage_mutex);
  if (piece_bytes) *piece_bytes = g_piece_bytes;
  if (threads) *threads = g_threads ? g_threads : default_threads();
}

int host_memcpy(void *dst, const void *src, size_t nbytes) {
  int threads;
  {
    std::lock_guard<std::mutex> lock(g_stage_mutex);
    threads = g_threads ? g_threads : default_threads();
  }
  pool().copy(dst, src, nbytes, threads);
  return FTX_OK;
}

int staged_copy_h2d(void *dst, const void *src, size_t nbytes, hipStream_t stream) {
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  FTX_HIP(hipStreamIsCapturing(stream, &cap));
  if (cap != hipStreamCaptureStatusNone)
    return fail(FTX_ERR_UNSUPPORTED, "a staged copy copies on the host at call time and cannot be captured");
  std::lock_guard<std::mutex> lock(g_stage_mutex);
  const int threads = g_threads ? g_threads : default_threads();
  StagingState *st = nullptr;
  int rc = staging(g_piece_bytes, &st);
  if (rc != FTX_OK) return rc;
  uint8_t *d = static_cast<uint8_t *>(dst);
  const uint8_t *s = static_cast<const uint8_t *>(src);
  // The first piece's host copy has no DMA to overlap with, so pieces start
  // small (a sixteenth of the policy's piece, at least 1 MiB) and double up to
  // the full piece: the link starts early and the pipeline fills at once.
  size_t piece = std::min(st->bytes, std::max(kMinPartBytes, st->bytes / 16));
  size_t off = 0;
  for (int j = 0; off < nbytes; ++j) {
    const int b = j % kStagingBuffers;
    const size_t len = std::min(piece, nbytes - off);
    FTX_HIP(hipEventSynchronize(st->done[b]));  // the buffer's previous DMA has read it
    pool().copy(st->buf[b], s + off, len, threads);
    FTX_HIP(hipMemcpyAsync(d + off, st->buf[b], len, hipMemcpyHostToDevice, stream));
    FTX_HIP(hipEventRecord(st->done[b], stream));
    off += len;
    piece = std::min(st->bytes, piece * 2);
  }
  return FTX_OK;
}

}  // namespace ftx
