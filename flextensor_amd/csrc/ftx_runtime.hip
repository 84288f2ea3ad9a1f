// C ABI of the MI355X weight-streaming engine: host arenas, copy engines,
// streams/events, scatter plans and checksums. Declarations and the reference
// constructs each entry point replaces are in include/ftx.h.
#include <algorithm>
#include <atomic>
#include <cstdio>
#include <cstring>
#include <map>
#include <mutex>
#include <vector>

#include "ftx_internal.h"

// Split-K partial sums of ftx_fp8_linear_static, for callers that cannot
// allocate: one array per GPU, held until the process ends. On the host this
// name is a stand-in, not a device address: host code only ever uses the
// address hipGetSymbolAddress returns for the current device (static_scratch).
static __device__ __align__(256) uint8_t scratch[FTX_FP8_STATIC_SCRATCH_BYTES];

namespace ftx {

namespace {

thread_local std::string g_last_error;

constexpr int kMaxDevices = 64;
constexpr int kMaxCopyStreams = 8;

struct CopyPolicy {
  size_t kernel_max_bytes = 1u << 20;  // AUTO: chunks up to 1 MiB go to the zero-copy kernel
  size_t split_min_bytes = ~size_t(0); // SDMA splitting disabled until measured
  int n_copy_streams = 1;
  int kernel_grid = 0;                 // 0: kZeroCopyDefaultGrid
};

int check_policy(size_t kernel_max_bytes, size_t split_min_bytes, int n_copy_streams, int kernel_grid,
                 CopyPolicy *out);

struct DeviceState {
  bool ready = false;
  int cu_count = 0;
  int xcd_count = 1;
  size_t total_mem = 0;
  hipStream_t copy_streams[kMaxCopyStreams] = {};
  hipEvent_t fork_event = nullptr;
  hipEvent_t join_events[kMaxCopyStreams] = {};
  void *static_scratch = nullptr;  // this device's address of `scratch`, resolved on first use
  size_t copy_reserve_lds = 0;     // LDS a small zero-copy grid reserves per CU (0: not available)
};

struct ArenaRecord {
  size_t nbytes;
  void *dev;  // device-visible address of the arena (hipHostGetDevicePointer)
};

std::atomic<bool> g_shut_down{false};
std::mutex g_mutex;      // guards g_policy and g_arenas
std::mutex g_dev_mutex;  // guards first-use setup of g_devices
CopyPolicy g_policy;
// fp8 linear launch shape; 0 = chosen per call from the shape and the CU count.
int g_fp8_waves = 0;
int g_fp8_slice_k = 0;
DeviceState g_devices[kMaxDevices];
std::map<uintptr_t, ArenaRecord> g_arenas;

int current_device(int *dev) {
  FTX_HIP(hipGetDevice(dev));
  if (*dev < 0 || *dev >= kMaxDevices) return fail(FTX_ERR_UNSUPPORTED, "device index out of range");
  return FTX_OK;
}

// Per-device copy streams and fork/join events, created on first use with the
// device current. Streams are non-blocking and at default priority.
int device_state(DeviceState **out) {
  int dev = 0;
  int rc = current_device(&dev);
  if (rc != FTX_OK) return rc;
  DeviceState &st = g_devices[dev];
  std::lock_guard<std::mutex> lock(g_dev_mutex);
  if (!st.ready) {
    int cus = 0;
    FTX_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
    int xccs = 0;
    if (hipDeviceGetAttribute(&xccs, hipDeviceAttributeNumberOfXccs, dev) != hipSuccess || xccs <= 0) {
      (void)hipGetLastError();
      hipDeviceProp_t prop;
      xccs = 1;
      if (hipGetDeviceProperties(&prop, dev) == hipSuccess && std::strncmp(prop.gcnArchName, "gfx950", 6) == 0)
        xccs = 8;
      (void)hipGetLastError();
    }
    size_t free_b = 0, total_b = 0;
    FTX_HIP(hipMemGetInfo(&free_b, &total_b));
    // Copy streams are created on the first split copy (copy_streams_ready):
    // every extra stream changes how streams share the device's hardware queues.
    // The whole LDS of a CU, for small zero-copy grids: the per-CU figure,
    // capped at what one workgroup may ask for. Where the runtime will not
    // grant it, copies share their CUs as before.
    int lds_cu = 0, lds_block = 0;
    if (hipDeviceGetAttribute(&lds_cu, hipDeviceAttributeMaxSharedMemoryPerMultiprocessor, dev) != hipSuccess)
      lds_cu = 0;
    if (hipDeviceGetAttribute(&lds_block, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess)
      lds_block = 0;
    const int lds = lds_cu > 0 && lds_block > 0 ? std::min(lds_cu, lds_block) : std::max(lds_cu, lds_block);
    if (lds > 0 && allow_zero_copy_lds(static_cast<size_t>(lds)) == hipSuccess &&
        allow_expcode_lds(static_cast<size_t>(lds)) == hipSuccess)
      st.copy_reserve_lds = static_cast<size_t>(lds);
    (void)hipGetLastError();
    st.cu_count = cus;
    st.xcd_count = xccs;
    st.total_mem = total_b;
    st.ready = true;
  }
  *out = &st;
  return FTX_OK;
}

// This device's copy of the static scratch array: its address is looked up
// once per device, with the device current, and kept.
int static_scratch(void **out) {
  DeviceState *st = nullptr;
  int rc = device_state(&st);
  if (rc != FTX_OK) return rc;
  std::lock_guard<std::mutex> lock(g_dev_mutex);
  if (st->static_scratch == nullptr) {
    void *ptr = nullptr;
    FTX_HIP(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)));
    if (ptr == nullptr) return fail(FTX_ERR_HIP, "hipGetSymbolAddress(scratch) returned no address");
    st->static_scratch = ptr;
  }
  *out = st->static_scratch;
  return FTX_OK;
}

// Device-visible address of the pinned host range [host, host+nbytes):
// arenas created here are looked up in the registry; other pinned memory
// (e.g. torch pin_memory) is resolved through hipPointerGetAttributes and
// hipMemGetAddressRange. The whole range must lie in one pinned allocation.
int mapped_source(const void *host, size_t nbytes, const void **dev) {
  const uintptr_t a = reinterpret_cast<uintptr_t>(host);
  {
    std::lock_guard<std::mutex> lock(g_mutex);
    auto it = g_arenas.upper_bound(a);
    if (it != g_arenas.begin()) {
      --it;
      if (a < it->first + it->second.nbytes) {
        if (a + nbytes > it->first + it->second.nbytes)
          return fail(FTX_ERR_INVALID, "host range exceeds its pinned arena");
        *dev = static_cast<const uint8_t *>(it->second.dev) + (a - it->first);
        return FTX_OK;
      }
    }
  }
  hipPointerAttribute_t attr;
  hipError_t err = hipPointerGetAttributes(&attr, host);
  if (err != hipSuccess) {
    (void)hipGetLastError();
    return fail(FTX_ERR_UNSUPPORTED, "zero-copy source is not pinned host memory");
  }
  if (attr.type != hipMemoryTypeHost || attr.devicePointer == nullptr)
    return fail(FTX_ERR_UNSUPPORTED, "zero-copy source is not device-mapped pinned host memory");
  hipDeviceptr_t base = nullptr;
  size_t size = 0;
  err = hipMemGetAddressRange(&base, &size, const_cast<void *>(host));
  if (err != hipSuccess) {
    (void)hipGetLastError();
    return fail(FTX_ERR_UNSUPPORTED, "extent of the pinned source is unknown");
  }
  if (a + nbytes > reinterpret_cast<uintptr_t>(base) + size)
    return fail(FTX_ERR_INVALID, "host range exceeds its pinned allocation");
  *dev = attr.devicePointer;
  return FTX_OK;
}

// [p, p+nbytes) must lie inside one device allocation; anything else (host
// memory, unmapped addresses, overruns past the allocation) is rejected on
// the host before a kernel or copy can touch it.
int check_device_range(const void *p, size_t nbytes, const char *what) {
  hipPointerAttribute_t attr;
  hipError_t err = hipPointerGetAttributes(&attr, p);
  if (err != hipSuccess || attr.type != hipMemoryTypeDevice) {
    (void)hipGetLastError();
    return fail(FTX_ERR_INVALID, std::string(what) + " is not device memory");
  }
  hipDeviceptr_t base = nullptr;
  size_t size = 0;
  err = hipMemGetAddressRange(&base, &size, const_cast<void *>(p));
  if (err != hipSuccess) {
    (void)hipGetLastError();
    return fail(FTX_ERR_INVALID, std::string(what) + ": device allocation extent unknown");
  }
  if (reinterpret_cast<uintptr_t>(p) + nbytes > reinterpret_cast<uintptr_t>(base) + size)
    return fail(FTX_ERR_INVALID, std::string(what) + " range exceeds its device allocation");
  return FTX_OK;
}

int copy_sdma(void *dst, const void *src, size_t nbytes, hipStream_t stream, const CopyPolicy &pol) {
  int vrc = check_device_range(dst, nbytes, "copy destination");
  if (vrc != FTX_OK) return vrc;
  if (pol.n_copy_streams <= 1 || nbytes < pol.split_min_bytes) {
    FTX_HIP(hipMemcpyAsync(dst, src, nbytes, hipMemcpyHostToDevice, stream));
    return FTX_OK;
  }
  DeviceState *st = nullptr;
  int rc = device_state(&st);
  if (rc != FTX_OK) return rc;
  const int k = std::min(pol.n_copy_streams, kMaxCopyStreams);
  // Every split copy on this device shares the fork and join events, so one
  // copy's record-and-wait sequence is enqueued whole: a copy made from another
  // host thread in between would re-record the fork event, and this copy's
  // pieces would then wait on the other caller's stream instead of this one.
  std::lock_guard<std::mutex> lock(g_dev_mutex);
  if (!st->fork_event) FTX_HIP(hipEventCreateWithFlags(&st->fork_event, hipEventDisableTiming));
  for (int i = 0; i < k; ++i) {
    if (!st->copy_streams[i]) FTX_HIP(hipStreamCreateWithFlags(&st->copy_streams[i], hipStreamNonBlocking));
    if (!st->join_events[i]) FTX_HIP(hipEventCreateWithFlags(&st->join_events[i], hipEventDisableTiming));
  }
  const size_t align = size_t(1) << 16;
  size_t piece = (nbytes + k - 1) / k;
  piece = (piece + align - 1) / align * align;
  FTX_HIP(hipEventRecord(st->fork_event, stream));
  size_t off = 0;
  for (int i = 0; i < k && off < nbytes; ++i) {
    const size_t n = std::min(piece, nbytes - off);
    FTX_HIP(hipStreamWaitEvent(st->copy_streams[i], st->fork_event, 0));
    FTX_HIP(hipMemcpyAsync(static_cast<uint8_t *>(dst) + off, static_cast<const uint8_t *>(src) + off, n,
                           hipMemcpyHostToDevice, st->copy_streams[i]));
    FTX_HIP(hipEventRecord(st->join_events[i], st->copy_streams[i]));
    FTX_HIP(hipStreamWaitEvent(stream, st->join_events[i], 0));
    off += n;
  }
  return FTX_OK;
}

int copy_kernel(void *dst, const void *src, size_t nbytes, hipStream_t stream, const CopyPolicy &pol,
                bool allow_fallback) {
  int rc = check_device_range(dst, nbytes, "copy destination");
  if (rc != FTX_OK) return rc;
  const void *src_dev = nullptr;
  rc = mapped_source(src, nbytes, &src_dev);
  const bool congruent =
      rc == FTX_OK && ((reinterpret_cast<uintptr_t>(src_dev) ^ reinterpret_cast<uintptr_t>(dst)) & 15) == 0;
  if (!congruent) {
    if (allow_fallback) return copy_sdma(dst, src, nbytes, stream, pol);
    if (rc != FTX_OK) return rc;
    return fail(FTX_ERR_UNSUPPORTED, "zero-copy kernel needs src and dst congruent modulo 16");
  }
  DeviceState *st = nullptr;
  rc = device_state(&st);
  if (rc != FTX_OK) return rc;
  const int grid = pol.kernel_grid > 0 ? pol.kernel_grid : kZeroCopyDefaultGrid;
  const size_t reserve = grid <= kZeroCopyReserveMaxGrid ? st->copy_reserve_lds : 0;
  FTX_HIP(launch_zero_copy(dst, src_dev, nbytes, grid, reserve, stream));
  return FTX_OK;
}

int check_policy(size_t kernel_max_bytes, size_t split_min_bytes, int n_copy_streams, int kernel_grid,
                 CopyPolicy *out) {
  if (n_copy_streams < 1 || n_copy_streams > kMaxCopyStreams)
    return fail(FTX_ERR_INVALID, "n_copy_streams must be in [1, 8]");
  if (kernel_grid < 0 || kernel_grid > (1 << 20)) return fail(FTX_ERR_INVALID, "kernel_grid must be in [0, 2^20]");
  out->kernel_max_bytes = kernel_max_bytes;
  out->split_min_bytes = split_min_bytes;
  out->n_copy_streams = n_copy_streams;
  out->kernel_grid = kernel_grid;
  return FTX_OK;
}

// Waits for every device, then destroys the split-copy streams and events of
// each device the library set up. Every device is tried; the first failure
// is returned.
int release_devices() {
  int first = FTX_OK;
  auto keep = [&first](int rc) {
    if (first == FTX_OK) first = rc;
  };
  int count = 0;
  if (hipGetDeviceCount(&count) != hipSuccess) {  // no device or no driver: nothing ran, nothing to release
    (void)hipGetLastError();
    count = 0;
  }
  int prev = -1;
  if (count > 0 && hipGetDevice(&prev) != hipSuccess) {
    (void)hipGetLastError();
    prev = -1;
  }
  std::lock_guard<std::mutex> lock(g_dev_mutex);
  for (int d = 0; d < std::min(count, kMaxDevices); ++d) {
    hipError_t err = hipSetDevice(d);
    if (err == hipSuccess) err = hipDeviceSynchronize();
    if (err != hipSuccess) {
      keep(hip_fail(err, "hipDeviceSynchronize at shutdown"));
      continue;
    }
    DeviceState &st = g_devices[d];
    for (int i = 0; i < kMaxCopyStreams; ++i) {
      if (st.copy_streams[i]) {
        err = hipStreamDestroy(st.copy_streams[i]);
        if (err != hipSuccess) keep(hip_fail(err, "hipStreamDestroy(copy stream)"));
        st.copy_streams[i] = nullptr;
      }
      if (st.join_events[i]) {
        err = hipEventDestroy(st.join_events[i]);
        if (err != hipSuccess) keep(hip_fail(err, "hipEventDestroy(join event)"));
        st.join_events[i] = nullptr;
      }
    }
    if (st.fork_event) {
      err = hipEventDestroy(st.fork_event);
      if (err != hipSuccess) keep(hip_fail(err, "hipEventDestroy(fork event)"));
      st.fork_event = nullptr;
    }
  }
  if (prev >= 0 && hipSetDevice(prev) != hipSuccess) (void)hipGetLastError();
  return first;
}

}  // namespace

bool is_shut_down() { return g_shut_down.load(); }

void set_error(const std::string &msg) { g_last_error = msg; }

int fail(int code, const std::string &msg) {
  set_error(msg);
  return code;
}

int hip_fail(hipError_t err, const char *what) {
  std::string msg = std::string(what) + ": " + hipGetErrorName(err) + " (" + hipGetErrorString(err) + ")";
  (void)hipGetLastError();  // do not leave the error for the next caller of the runtime
  set_error(msg);
  return err == hipErrorOutOfMemory || err == hipErrorMemoryAllocation ? FTX_ERR_OOM : FTX_ERR_HIP;
}

}  // namespace ftx

struct ftx_scatter_plan {
  ftx::ScatterPlanDev dev;
  void *storage;  // one device allocation holding the three tables
  int n_desc_in;
  uint64_t total_bytes;
  uint64_t max_src_end;
};

namespace {

// Host-side tables of a scatter plan, laid out as one contiguous buffer:
// [descs | tile_start | group_desc0], each section 256-byte aligned.
struct PlanTables {
  std::vector<uint8_t> buf;
  size_t off_tile_start = 0, off_group = 0;
  int n_desc = 0;
  int64_t n_tiles = 0, n_groups = 0;
  uint64_t total_bytes = 0;
  uint64_t max_src_end = 0;  // chunk bytes the descriptors read
};

size_t align256(size_t x) { return (x + 255) / 256 * 256; }

int build_plan_tables(const ftx_desc *descs, int n_desc, size_t tile_bytes, PlanTables *t) {
  if (n_desc < 0) return ftx::fail(FTX_ERR_INVALID, "n_desc must be >= 0");
  if (n_desc > 0 && descs == nullptr) return ftx::fail(FTX_ERR_INVALID, "descs is null");
  if (tile_bytes == 0) tile_bytes = ftx::kScatterTileBytes;
  if (tile_bytes % 16 != 0) return ftx::fail(FTX_ERR_INVALID, "tile_bytes must be a multiple of 16");
  std::vector<ftx_desc> kept;
  kept.reserve(static_cast<size_t>(n_desc));
  uint64_t max_src_end = 0;
  for (int i = 0; i < n_desc; ++i) {
    if (descs[i].nbytes == 0) continue;
    if (descs[i].dst == 0) return ftx::fail(FTX_ERR_INVALID, "descriptor with null destination");
    if (descs[i].src_off + descs[i].nbytes < descs[i].src_off)
      return ftx::fail(FTX_ERR_INVALID, "descriptor source range overflows");
    int vrc = ftx::check_device_range(reinterpret_cast<const void *>(descs[i].dst), descs[i].nbytes,
                                      "scatter destination");
    if (vrc != FTX_OK) return vrc;
    max_src_end = std::max<uint64_t>(max_src_end, descs[i].src_off + descs[i].nbytes);
    kept.push_back(descs[i]);
  }
  t->max_src_end = max_src_end;
  const size_t nd = kept.size();
  std::vector<uint64_t> tile_start(nd + 1, 0);
  uint64_t total = 0;
  for (size_t i = 0; i < nd; ++i) {
    tile_start[i + 1] = tile_start[i] + (kept[i].nbytes + tile_bytes - 1) / tile_bytes;
    total += kept[i].nbytes;
  }
  const int64_t n_tiles = static_cast<int64_t>(tile_start[nd]);
  const int64_t n_groups = (n_tiles + ftx::kScatterWavesPerGroup - 1) / ftx::kScatterWavesPerGroup;
  if (n_groups > 0x7fffffff) return ftx::fail(FTX_ERR_INVALID, "scatter plan too large for one launch");
  std::vector<uint32_t> group_desc0(static_cast<size_t>(n_groups));
  size_t d = 0;
  for (int64_t g = 0; g < n_groups; ++g) {
    const uint64_t tile = static_cast<uint64_t>(g) * ftx::kScatterWavesPerGroup;
    while (tile_start[d + 1] <= tile) ++d;
    group_desc0[static_cast<size_t>(g)] = static_cast<uint32_t>(d);
  }
  t->off_tile_start = align256(nd * sizeof(ftx_desc));
  t->off_group = t->off_tile_start + align256((nd + 1) * sizeof(uint64_t));
  const size_t total_sz = t->off_group + align256(std::max<size_t>(1, group_desc0.size()) * sizeof(uint32_t));
  t->buf.assign(total_sz, 0);
  if (nd) std::memcpy(t->buf.data(), kept.data(), nd * sizeof(ftx_desc));
  std::memcpy(t->buf.data() + t->off_tile_start, tile_start.data(), (nd + 1) * sizeof(uint64_t));
  if (!group_desc0.empty())
    std::memcpy(t->buf.data() + t->off_group, group_desc0.data(), group_desc0.size() * sizeof(uint32_t));
  t->n_desc = static_cast<int>(nd);
  t->n_tiles = n_tiles;
  t->n_groups = n_groups;
  t->total_bytes = total;
  return FTX_OK;
}

ftx::ScatterPlanDev plan_view(const PlanTables &t, void *storage, size_t tile_bytes) {
  ftx::ScatterPlanDev p;
  uint8_t *base = static_cast<uint8_t *>(storage);
  p.descs = reinterpret_cast<const ftx_desc *>(base);
  p.tile_start = reinterpret_cast<const uint64_t *>(base + t.off_tile_start);
  p.group_desc0 = reinterpret_cast<const uint32_t *>(base + t.off_group);
  p.n_desc = t.n_desc;
  p.n_tiles = t.n_tiles;
  p.n_groups = t.n_groups;
  p.tile_bytes = tile_bytes ? tile_bytes : ftx::kScatterTileBytes;
  return p;
}

}  // namespace

extern "C" {

const char *ftx_last_error(void) { return ftx::g_last_error.c_str(); }

int ftx_version(void) { return 1; }

int ftx_shutdown(void) {
  if (ftx::g_shut_down.exchange(true)) return FTX_OK;  // already done
  // Devices first: the staging buffers and events are only released once no
  // queued copy can still read them.
  const int rc_dev = ftx::release_devices();
  const int rc_stage = ftx::staged_shutdown();
  return rc_dev != FTX_OK ? rc_dev : rc_stage;
}

int ftx_device_count(int *count) {
  if (!count) return ftx::fail(FTX_ERR_INVALID, "count is null");
  FTX_HIP(hipGetDeviceCount(count));
  return FTX_OK;
}

int ftx_set_device(int device) {
  FTX_HIP(hipSetDevice(device));
  return FTX_OK;
}

int ftx_get_device(int *device) {
  if (!device) return ftx::fail(FTX_ERR_INVALID, "device is null");
  FTX_HIP(hipGetDevice(device));
  return FTX_OK;
}

int ftx_device_synchronize(void) {
  FTX_HIP(hipDeviceSynchronize());
  return FTX_OK;
}

int ftx_device_info(int *cu_count, int *xcd_count, size_t *total_mem) {
  ftx::DeviceState *st = nullptr;
  int rc = ftx::device_state(&st);
  if (rc != FTX_OK) return rc;
  if (cu_count) *cu_count = st->cu_count;
  if (xcd_count) *xcd_count = st->xcd_count;
  if (total_mem) *total_mem = st->total_mem;
  return FTX_OK;
}

int ftx_arena_alloc(size_t nbytes, unsigned flags, void **host) {
  FTX_REQUIRE_LIVE();
  if (!host) return ftx::fail(FTX_ERR_INVALID, "host is null");
  if (nbytes == 0) return ftx::fail(FTX_ERR_INVALID, "arena size must be > 0");
  if ((flags & FTX_ARENA_COHERENT) && (flags & FTX_ARENA_NONCOHERENT))
    return ftx::fail(FTX_ERR_INVALID, "arena cannot be both coherent and non-coherent");
  unsigned hflags = hipHostMallocPortable | hipHostMallocMapped;
  if (flags & FTX_ARENA_COHERENT) hflags |= hipHostMallocCoherent;
  if (flags & FTX_ARENA_NONCOHERENT) hflags |= hipHostMallocNonCoherent;
  if (flags & FTX_ARENA_WRITECOMBINED) hflags |= hipHostMallocWriteCombined;
  if (flags & FTX_ARENA_NUMA_USER) hflags |= hipHostMallocNumaUser;
  void *p = nullptr;
  FTX_HIP(hipHostMalloc(&p, nbytes, hflags));
  void *dev = nullptr;
  hipError_t err = hipHostGetDevicePointer(&dev, p, 0);
  if (err != hipSuccess) {
    (void)hipHostFree(p);
    return ftx::hip_fail(err, "hipHostGetDevicePointer");
  }
  {
    std::lock_guard<std::mutex> lock(ftx::g_mutex);
    ftx::g_arenas[reinterpret_cast<uintptr_t>(p)] = ftx::ArenaRecord{nbytes, dev};
  }
  *host = p;
  return FTX_OK;
}

int ftx_arena_free(void *host) {
  if (!host) return FTX_OK;
  {
    std::lock_guard<std::mutex> lock(ftx::g_mutex);
    auto it = ftx::g_arenas.find(reinterpret_cast<uintptr_t>(host));
    if (it == ftx::g_arenas.end()) return ftx::fail(FTX_ERR_INVALID, "pointer is not an arena from ftx_arena_alloc");
    ftx::g_arenas.erase(it);
  }
  FTX_HIP(hipHostFree(host));
  return FTX_OK;
}

int ftx_arena_register(void *host, size_t nbytes, unsigned flags) {
  (void)host;
  (void)nbytes;
  (void)flags;
  return ftx::fail(FTX_ERR_UNSUPPORTED,
                   "in-place page-locking (hipHostRegister of existing memory) is refused in this build: the MI355X "
                   "hosts it targets reject it, and the failed call's error can surface in the next GPU call; "
                   "allocate the block with ftx_arena_alloc, or stream a pageable source with FTX_COPY_STAGED");
}

int ftx_arena_unregister(void *host) {
  (void)host;
  return ftx::fail(FTX_ERR_INVALID, "nothing is registered in place: ftx_arena_register is refused in this build");
}

int ftx_host_device_ptr(void *host, void **dev) {
  if (!host || !dev) return ftx::fail(FTX_ERR_INVALID, "null argument");
  const void *d = nullptr;
  int rc = ftx::mapped_source(host, 1, &d);
  if (rc != FTX_OK) return rc;
  *dev = const_cast<void *>(d);
  return FTX_OK;
}

int ftx_device_alloc(size_t nbytes, void **dev) {
  FTX_REQUIRE_LIVE();
  if (!dev || nbytes == 0) return ftx::fail(FTX_ERR_INVALID, "dev is null or size is 0");
  FTX_HIP(hipMalloc(dev, nbytes));
  return FTX_OK;
}

int ftx_device_free(void *dev) {
  if (!dev) return FTX_OK;
  FTX_HIP(hipFree(dev));
  return FTX_OK;
}

int ftx_memset_async(void *dev, int value, size_t nbytes, void *stream) {
  FTX_REQUIRE_LIVE();
  if (nbytes == 0) return FTX_OK;
  if (!dev) return ftx::fail(FTX_ERR_INVALID, "dev is null");
  int rc = ftx::check_device_range(dev, nbytes, "memset destination");
  if (rc != FTX_OK) return rc;
  FTX_HIP(ftx::launch_fill_u8(dev, static_cast<uint8_t>(value), nbytes, static_cast<hipStream_t>(stream)));
  return FTX_OK;
}

int ftx_copy_d2h(void *dst_host, const void *src_dev, size_t nbytes, void *stream) {
  FTX_REQUIRE_LIVE();
  if ((!dst_host || !src_dev) && nbytes) return ftx::fail(FTX_ERR_INVALID, "null argument");
  if (nbytes == 0) return FTX_OK;
  int rc = ftx::check_device_range(src_dev, nbytes, "copy source");
  if (rc != FTX_OK) return rc;
  FTX_HIP(hipMemcpyAsync(dst_host, src_dev, nbytes, hipMemcpyDeviceToHost, static_cast<hipStream_t>(stream)));
  return FTX_OK;
}

int ftx_stream_create(void **stream) {
  FTX_REQUIRE_LIVE();
  if (!stream) return ftx::fail(FTX_ERR_INVALID, "stream is null");
  hipStream_t s = nullptr;
  FTX_HIP(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
  *stream = s;
  return FTX_OK;
}

int ftx_stream_destroy(void *stream) {
  if (!stream) return FTX_OK;
  FTX_HIP(hipStreamDestroy(static_cast<hipStream_t>(stream)));
  return FTX_OK;
}

int ftx_stream_synchronize(void *stream) {
  FTX_HIP(hipStreamSynchronize(static_cast<hipStream_t>(stream)));
  return FTX_OK;
}

int ftx_stream_query(void *stream, int *done) {
  if (!done) return ftx::fail(FTX_ERR_INVALID, "done is null");
  hipError_t err = hipStreamQuery(static_cast<hipStream_t>(stream));
  if (err == hipErrorNotReady) {
    (void)hipGetLastError();
    *done = 0;
    return FTX_OK;
  }
  FTX_HIP(err);
  *done = 1;
  return FTX_OK;
}

int ftx_event_create(unsigned flags, void **event) {
  FTX_REQUIRE_LIVE();
  if (!event) return ftx::fail(FTX_ERR_INVALID, "event is null");
  if (flags & ~(FTX_EVENT_TIMING | FTX_EVENT_DEVICE_ONLY)) return ftx::fail(FTX_ERR_INVALID, "unknown event flags");
  unsigned hflags = (flags & FTX_EVENT_TIMING) ? hipEventDefault : hipEventDisableTiming;
  if (flags & FTX_EVENT_DEVICE_ONLY) hflags |= hipEventDisableSystemFence;
  hipEvent_t e = nullptr;
  FTX_HIP(hipEventCreateWithFlags(&e, hflags));
  *event = e;
  return FTX_OK;
}

int ftx_event_destroy(void *event) {
  if (!event) return FTX_OK;
  FTX_HIP(hipEventDestroy(static_cast<hipEvent_t>(event)));
  return FTX_OK;
}

int ftx_event_record(void *event, void *stream) {
  FTX_REQUIRE_LIVE();
  if (!event) return ftx::fail(FTX_ERR_INVALID, "event is null");
  FTX_HIP(hipEventRecord(static_cast<hipEvent_t>(event), static_cast<hipStream_t>(stream)));
  return FTX_OK;
}

int ftx_timestamp(void *dev_slot, void *stream) {
  FTX_REQUIRE_LIVE();
  if (!dev_slot) return ftx::fail(FTX_ERR_INVALID, "timestamp slot is null");
  if (reinterpret_cast<uintptr_t>(dev_slot) % 8) return ftx::fail(FTX_ERR_INVALID, "timestamp slot is not 8-byte aligned");
  int rc = ftx::check_device_range(dev_slot, 8, "timestamp slot");
  if (rc != FTX_OK) return rc;
  FTX_HIP(ftx::launch_timestamp(static_cast<uint64_t *>(dev_slot), static_cast<hipStream_t>(stream)));
  return FTX_OK;
}

int ftx_wall_clock_khz(int *khz) {
  if (!khz) return ftx::fail(FTX_ERR_INVALID, "khz is null");
  int dev = 0;
  FTX_HIP(hipGetDevice(&dev));
  FTX_HIP(hipDeviceGetAttribute(khz, hipDeviceAttributeWallClockRate, dev));
  return FTX_OK;
}

int ftx_stream_wait_event(void *stream, void *event) {
  FTX_REQUIRE_LIVE();
  if (!event) return ftx::fail(FTX_ERR_INVALID, "event is null");
  FTX_HIP(hipStreamWaitEvent(static_cast<hipStream_t>(stream), static_cast<hipEvent_t>(event), 0));
  return FTX_OK;
}

int ftx_event_query(void *event, int *done) {
  if (!event || !done) return ftx::fail(FTX_ERR_INVALID, "null argument");
  hipError_t err = hipEventQuery(static_cast<hipEvent_t>(event));
  if (err == hipErrorNotReady) {
    (void)hipGetLastError();
    *done = 0;
    return FTX_OK;
  }
  FTX_HIP(err);
  *done = 1;
  return FTX_OK;
}

int ftx_event_synchronize(void *event) {
  if (!event) return ftx::fail(FTX_ERR_INVALID, "event is null");
  FTX_HIP(hipEventSynchronize(static_cast<hipEvent_t>(event)));
  return FTX_OK;
}

int ftx_event_elapsed_ms(void *start, void *end, float *ms) {
  if (!start || !end || !ms) return ftx::fail(FTX_ERR_INVALID, "null argument");
  FTX_HIP(hipEventElapsedTime(ms, static_cast<hipEvent_t>(start), static_cast<hipEvent_t>(end)));
  return FTX_OK;
}

int ftx_copy_h2d(void *dst, const void *src, size_t nbytes, int mode, void *stream) {
  return ftx_copy_h2d_policy(dst, src, nbytes, mode, nullptr, stream);
}

int ftx_copy_h2d_policy(void *dst, const void *src, size_t nbytes, int mode, const ftx_copy_policy *policy,
                        void *stream) {
  FTX_REQUIRE_LIVE();
  ftx::CopyPolicy pol;
  if (policy != nullptr) {
    int rc = ftx::check_policy(policy->kernel_max_bytes, policy->split_min_bytes, policy->n_copy_streams,
                               policy->kernel_grid, &pol);
    if (rc != FTX_OK) return rc;
  } else {
    std::lock_guard<std::mutex> lock(ftx::g_mutex);
    pol = ftx::g_policy;
  }
  if (nbytes == 0) return FTX_OK;
  if (!dst || !src) return ftx::fail(FTX_ERR_INVALID, "null pointer");
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (mode) {
    case FTX_COPY_SDMA:
      return ftx::copy_sdma(dst, src, nbytes, s, pol);
    case FTX_COPY_KERNEL:
      return ftx::copy_kernel(dst, src, nbytes, s, pol, false);
    case FTX_COPY_STAGED: {
      int rc = ftx::check_device_range(dst, nbytes, "copy destination");
      if (rc != FTX_OK) return rc;
      return ftx::staged_copy_h2d(dst, src, nbytes, s);
    }
    case FTX_COPY_AUTO: {
      const void *mapped = nullptr;
      if (ftx::mapped_source(src, nbytes, &mapped) != FTX_OK) {  // pageable: stage it
        int rc = ftx::check_device_range(dst, nbytes, "copy destination");
        if (rc != FTX_OK) return rc;
        return ftx::staged_copy_h2d(dst, src, nbytes, s);
      }
      if (nbytes <= pol.kernel_max_bytes) return ftx::copy_kernel(dst, src, nbytes, s, pol, true);
      return ftx::copy_sdma(dst, src, nbytes, s, pol);
    }
    default:
      return ftx::fail(FTX_ERR_INVALID, "unknown copy mode");
  }
}

int ftx_expcode_encode(const void *raw, size_t nbytes, void *out, size_t out_capacity, size_t *out_bytes) {
  FTX_REQUIRE_LIVE();
  if (!out_bytes) return ftx::fail(FTX_ERR_INVALID, "out_bytes is null");
  if (nbytes > 0 && !raw) return ftx::fail(FTX_ERR_INVALID, "raw is null");
  if (out != nullptr) {
    const uintptr_t o = reinterpret_cast<uintptr_t>(out), r = reinterpret_cast<uintptr_t>(raw);
    if (nbytes > 0 && o < r + nbytes && r < o + out_capacity)
      return ftx::fail(FTX_ERR_INVALID, "raw and out ranges overlap");
  }
  return ftx::expcode_encode(raw, nbytes, out, out_capacity, out_bytes);
}

int ftx_expcode_raw_bytes(const void *src, size_t src_bytes, size_t *raw_bytes) {
  if (!src || !raw_bytes) return ftx::fail(FTX_ERR_INVALID, "null argument");
  uint32_t version = 0;
  if (src_bytes >= 8) std::memcpy(&version, static_cast<const uint8_t *>(src) + 4, 4);
  if (version == 2) {
    ftx::DenseLayout d;
    const int rc = ftx::expcode_parse_dense(src, src_bytes, &d);
    if (rc != FTX_OK) return rc;
    *raw_bytes = static_cast<size_t>(d.n);
    return FTX_OK;
  }
  ftx::ExpcodeInfo info;
  int rc = ftx::expcode_parse(src, src_bytes, &info);
  if (rc != FTX_OK) return rc;
  *raw_bytes = static_cast<size_t>(info.n);
  return FTX_OK;
}

int ftx_expcode_decode_h2d(void *dst, const void *src, size_t src_bytes, const ftx_copy_policy *policy,
                           void *stream) {
  FTX_REQUIRE_LIVE();
  if (!dst || !src) return ftx::fail(FTX_ERR_INVALID, "null pointer");
  // The header is read on the host (src is host memory): version 1, or the dense version 2
  uint32_t version = 0;
  if (src_bytes >= 8) std::memcpy(&version, static_cast<const uint8_t *>(src) + 4, 4);
  const bool dense = version == 2;
  uint64_t n = 0;
  int rc;
  if (dense) {
    ftx::DenseLayout d;
    rc = ftx::expcode_parse_dense(src, src_bytes, &d);
    n = d.n;
  } else {
    ftx::ExpcodeInfo info;
    rc = ftx::expcode_parse(src, src_bytes, &info);
    n = info.n;
  }
  if (rc != FTX_OK) return rc;
  if (n == 0) return FTX_OK;
  if (reinterpret_cast<uintptr_t>(dst) % 16 != 0) return ftx::fail(FTX_ERR_INVALID, "decode destination needs 16-byte alignment");
  rc = ftx::check_device_range(dst, static_cast<size_t>(n), "decode destination");
  if (rc != FTX_OK) return rc;
  const void *src_dev = nullptr;
  rc = ftx::mapped_source(src, src_bytes, &src_dev);  // the kernel may read up to src_bytes (a re-encoded block)
  if (rc != FTX_OK) return rc;
  if (reinterpret_cast<uintptr_t>(src_dev) % 16 != 0)
    return ftx::fail(FTX_ERR_INVALID, "encoded block needs 16-byte alignment");
  int grid = ftx::kExpcodeDefaultGrid;
  if (policy != nullptr) {
    ftx::CopyPolicy pol;
    rc = ftx::check_policy(policy->kernel_max_bytes, policy->split_min_bytes, policy->n_copy_streams,
                           policy->kernel_grid, &pol);
    if (rc != FTX_OK) return rc;
    if (pol.kernel_grid > 0) grid = pol.kernel_grid;
  }
  ftx::DeviceState *st = nullptr;
  rc = ftx::device_state(&st);
  if (rc != FTX_OK) return rc;
  const size_t reserve = grid <= ftx::kZeroCopyReserveMaxGrid ? st->copy_reserve_lds : 0;
  if (dense)
    FTX_HIP(ftx::launch_expcode_dense_link_decode(dst, src_dev, src_bytes, n, grid, reserve,
                                                  static_cast<hipStream_t>(stream)));
  else
    FTX_HIP(ftx::launch_expcode_decode(dst, src_dev, src_bytes, n, grid, reserve, static_cast<hipStream_t>(stream)));
  return FTX_OK;
}

int ftx_expcode_decode_d2d(void *dst, const void *src, size_t src_bytes, size_t raw_bytes, int grid,
                           void *stream) {
  FTX_REQUIRE_LIVE();
  if (raw_bytes == 0) return FTX_OK;
  if (!dst || !src) return ftx::fail(FTX_ERR_INVALID, "null pointer");
  if (grid < 0 || grid > (1 << 20)) return ftx::fail(FTX_ERR_INVALID, "grid must be in [0, 2^20]");
  if (reinterpret_cast<uintptr_t>(dst) % 16 != 0 || reinterpret_cast<uintptr_t>(src) % 16 != 0)
    return ftx::fail(FTX_ERR_INVALID, "decode source and destination need 16-byte alignment");
  // The header is in device memory: the caller states the raw size, and the kernel reads the rest of the
  // header when it runs (a header of another raw size writes nothing; escape reads stay within src_bytes).
  const uint64_t groups = (raw_bytes / 2 + ftx::kExpcodeGroupWords - 1) / ftx::kExpcodeGroupWords;
  const uint64_t off_x = ftx::kExpcodeHeaderBytes + ftx::kExpcodeGroupWords * groups +
                         ftx::kExpcodeGroupWords / 2 * groups + (4 * (groups + 1) + 15) / 16 * 16;
  if (src_bytes < off_x) return ftx::fail(FTX_ERR_INVALID, "encoded block is shorter than its raw size needs");
  int rc = ftx::check_device_range(dst, raw_bytes, "decode destination");
  if (rc == FTX_OK) rc = ftx::check_device_range(src, src_bytes, "encoded block");
  if (rc != FTX_OK) return rc;
  ftx::DeviceState *st = nullptr;
  rc = ftx::device_state(&st);
  if (rc != FTX_OK) return rc;
  // HBM to HBM: eight workgroups per CU by default (a 7B-shape layer decodes at 5.4 TB/s of encoded plus raw
  // bytes, the rate of a device-to-device copy; one per CU reaches 4.6 TB/s)
  const int g = grid > 0 ? grid : 8 * st->cu_count;
  // A larger grid asks for 1 KiB of LDS per workgroup. A link decode or zero-copy copy running beside it holds
  // all the LDS of its CUs, so these workgroups keep off those CUs, where its slow host reads would hold up
  // their loads (in the 7B decode a 90 MB unit took 105 us there against 34 us elsewhere).
  const size_t reserve = g <= ftx::kZeroCopyReserveMaxGrid ? st->copy_reserve_lds
                                                           : (st->copy_reserve_lds ? size_t{1024} : size_t{0});
  FTX_HIP(ftx::launch_expcode_decode(dst, src, src_bytes, raw_bytes, g, reserve, static_cast<hipStream_t>(stream)));
  return FTX_OK;
}

int ftx_expcode_encode_dense(const void *raw, size_t n, void *out, size_t capacity, size_t *out_bytes) {
  FTX_REQUIRE_LIVE();
  if (!out_bytes) return ftx::fail(FTX_ERR_INVALID, "out_bytes is null");
  if (n > 0 && !raw) return ftx::fail(FTX_ERR_INVALID, "raw is null");
  if (out && raw && n > 0) {
    const auto r = reinterpret_cast<uintptr_t>(raw), o = reinterpret_cast<uintptr_t>(out);
    if (o < r + n && r < o + capacity) return ftx::fail(FTX_ERR_INVALID, "output overlaps the raw block");
  }
  return ftx::expcode_encode_dense(raw, n, out, capacity, out_bytes);
}

int ftx_expcode_decode_dense_d2d(void *dst, const void *src, size_t src_bytes, size_t raw_bytes, int grid,
                                 void *stream) {
  FTX_REQUIRE_LIVE();
  if (raw_bytes == 0) return FTX_OK;
  if (!dst || !src) return ftx::fail(FTX_ERR_INVALID, "null pointer");
  if (grid < 0 || grid > (1 << 20)) return ftx::fail(FTX_ERR_INVALID, "grid must be in [0, 2^20]");
  if (reinterpret_cast<uintptr_t>(dst) % 16 != 0 || reinterpret_cast<uintptr_t>(src) % 16 != 0)
    return ftx::fail(FTX_ERR_INVALID, "decode source and destination need 16-byte alignment");
  const ftx::DenseLayout d = ftx::dense_layout(raw_bytes, 0, 0);
  if (src_bytes < d.off_y) return ftx::fail(FTX_ERR_INVALID, "encoded block is shorter than its raw size needs");
  int rc = ftx::check_device_range(dst, raw_bytes, "decode destination");
  if (rc == FTX_OK) rc = ftx::check_device_range(src, src_bytes, "encoded block");
  if (rc != FTX_OK) return rc;
  ftx::DeviceState *st = nullptr;
  rc = ftx::device_state(&st);
  if (rc != FTX_OK) return rc;
  const int g = grid > 0 ? grid : 16 * st->cu_count;  // a 7B layer: 150 us at 16 per CU, 162 us at 8
  const size_t reserve = g <= ftx::kZeroCopyReserveMaxGrid ? st->copy_reserve_lds
                                                           : (st->copy_reserve_lds ? size_t{1024} : size_t{0});
  FTX_HIP(ftx::launch_expcode_dense_decode(dst, src, src_bytes, raw_bytes, g, reserve,
                                           static_cast<hipStream_t>(stream)));
  return FTX_OK;
}

int ftx_set_staging_policy(size_t piece_bytes, int n_threads) { return ftx::set_staging_policy(piece_bytes, n_threads); }

int ftx_get_staging_policy(size_t *piece_bytes, int *n_threads) {
  ftx::get_staging_policy(piece_bytes, n_threads);
  return FTX_OK;
}

int ftx_host_memcpy(void *dst, const void *src, size_t nbytes) {
  FTX_REQUIRE_LIVE();
  if (nbytes == 0) return FTX_OK;
  if (!dst || !src) return ftx::fail(FTX_ERR_INVALID, "null pointer");
  const uintptr_t d = reinterpret_cast<uintptr_t>(dst), sp = reinterpret_cast<uintptr_t>(src);
  if (d < sp + nbytes && sp < d + nbytes) return ftx::fail(FTX_ERR_INVALID, "host copy ranges overlap");
  return ftx::host_memcpy(dst, src, nbytes);
}

int ftx_set_copy_policy(size_t kernel_max_bytes, size_t split_min_bytes, int n_copy_streams, int kernel_grid) {
  ftx::CopyPolicy pol;
  int rc = ftx::check_policy(kernel_max_bytes, split_min_bytes, n_copy_streams, kernel_grid, &pol);
  if (rc != FTX_OK) return rc;
  std::lock_guard<std::mutex> lock(ftx::g_mutex);
  ftx::g_policy = pol;
  return FTX_OK;
}

int ftx_get_copy_policy(size_t *kernel_max_bytes, size_t *split_min_bytes, int *n_copy_streams, int *kernel_grid) {
  std::lock_guard<std::mutex> lock(ftx::g_mutex);
  if (kernel_max_bytes) *kernel_max_bytes = ftx::g_policy.kernel_max_bytes;
  if (split_min_bytes) *split_min_bytes = ftx::g_policy.split_min_bytes;
  if (n_copy_streams) *n_copy_streams = ftx::g_policy.n_copy_streams;
  if (kernel_grid) *kernel_grid = ftx::g_policy.kernel_grid;
  return FTX_OK;
}

int ftx_set_fp8_linear_config(int waves, int slice_k) {
  if (waves < 0 || waves > 8) return ftx::fail(FTX_ERR_INVALID, "waves must be 0 (automatic) or in [1, 8]");
  if (slice_k < 0 || slice_k % 256 != 0)
    return ftx::fail(FTX_ERR_INVALID, "slice_k must be 0 (automatic) or a positive multiple of 256");
  std::lock_guard<std::mutex> lock(ftx::g_mutex);
  ftx::g_fp8_waves = waves;
  ftx::g_fp8_slice_k = slice_k;
  return FTX_OK;
}

namespace {

int plan_fp8(int64_t m, const int64_t *n, int group, int64_t k, ftx::Fp8LinearLaunch *p,
             int epilogue = ftx::kFp8EpilogueNone) {
  if (group < 1 || group > ftx::kFp8MaxGroup)
    return ftx::fail(FTX_ERR_INVALID, "a grouped fp8 linear takes 1 to " + std::to_string(ftx::kFp8MaxGroup) +
                                          " weight matrices");
  if (!n) return ftx::fail(FTX_ERR_INVALID, "n is null");
  int64_t n_total = 0;
  for (int s = 0; s < group; ++s) {
    if (n[s] < 0) return ftx::fail(FTX_ERR_INVALID, "negative dimension");
    if (n[s] > (int64_t(1) << 30)) return ftx::fail(FTX_ERR_INVALID, "fp8 linear dimensions too large");
    n_total += n[s];
  }
  if (m < 0 || k < 0) return ftx::fail(FTX_ERR_INVALID, "negative dimension");
  if (k % 16 != 0) return ftx::fail(FTX_ERR_INVALID, "k must be a multiple of 16");
  if (n_total > (int64_t(1) << 30) || k > (int64_t(1) << 30) || m * n_total > (int64_t(1) << 31))
    return ftx::fail(FTX_ERR_INVALID, "fp8 linear dimensions too large");
  if (epilogue == ftx::kFp8EpilogueSwiglu) {
    if (group != 2 || n[0] != n[1])
      return ftx::fail(FTX_ERR_INVALID, "the SwiGLU epilogue takes two matrices (gate, up) with the same n");
  } else if (epilogue == ftx::kFp8EpilogueResidual) {
    if (group != 1) return ftx::fail(FTX_ERR_INVALID, "the residual epilogue takes one matrix");
  } else if (epilogue != ftx::kFp8EpilogueNone) {
    return ftx::fail(FTX_ERR_INVALID, "unknown fp8 linear epilogue");
  }
  if (epilogue != ftx::kFp8EpilogueNone && m > ftx::kFp8LinearMaxRows)
    return ftx::fail(FTX_ERR_UNSUPPORTED, "fp8 linear epilogues run in the decode kernel only (at most " +
                                              std::to_string(ftx::kFp8LinearMaxRows) + " rows)");
  if (m == 0 || n_total == 0) {
    *p = ftx::Fp8LinearLaunch{};
    p->group = group;
    p->m = m;
    p->k = k;
    p->epilogue = epilogue;
    return FTX_OK;
  }
  int waves, slice_k;
  {
    std::lock_guard<std::mutex> lock(ftx::g_mutex);
    waves = ftx::g_fp8_waves;
    slice_k = ftx::g_fp8_slice_k;
  }
  int cus = 256, xcds = 8;
  {
    ftx::DeviceState *st = nullptr;
    if (ftx::device_state(&st) == FTX_OK) {
      cus = st->cu_count;
      xcds = st->xcd_count;
    }
  }
  *p = ftx::plan_fp8_linear(m, n, group, k, cus, xcds, waves, slice_k, epilogue);
  if (p->grid > (int64_t(1) << 31) - 1) return ftx::fail(FTX_ERR_INVALID, "fp8 linear grid too large");
  return FTX_OK;
}

}  // namespace

int ftx_fp8_linear_workspace(int64_t m, int64_t n, int64_t k, size_t *bytes) {
  return ftx_fp8_linear_group_workspace(m, &n, 1, k, bytes);
}

int ftx_fp8_linear_group_workspace(int64_t m, const int64_t *n, int group, int64_t k, size_t *bytes) {
  if (!bytes) return ftx::fail(FTX_ERR_INVALID, "bytes is null");
  ftx::Fp8LinearLaunch p;
  int rc = plan_fp8(m, n, group, k, &p);
  if (rc != FTX_OK) return rc;
  *bytes = p.workspace_bytes;
  return FTX_OK;
}

namespace {

// Checks the operands of one planned fp8 linear launch and launches it. The
// workspace is checked against its allocation unless it is the static scratch.
int run_fp8(ftx::Fp8LinearLaunch &p, const void *x, const void *const *w, const void *const *scale, void *const *y,
            void *workspace, size_t workspace_bytes, bool static_workspace, void *stream) {
  const int64_t m = p.m, k = p.k;
  if (!w || !scale || !y) return ftx::fail(FTX_ERR_INVALID, "null pointer");
  for (int s = 0; s < p.group; ++s) {
    const int64_t n = p.n[s];
    if (n == 0) continue;
    if (!y[s] || !scale[s]) return ftx::fail(FTX_ERR_INVALID, "null pointer");
    if (reinterpret_cast<uintptr_t>(y[s]) % 2 != 0 || reinterpret_cast<uintptr_t>(scale[s]) % 2 != 0)
      return ftx::fail(FTX_ERR_INVALID, "y and scale need 2-byte alignment");
    int rc = ftx::check_device_range(y[s], static_cast<size_t>(m * n * 2), "fp8 linear output");
    if (rc == FTX_OK) rc = ftx::check_device_range(scale[s], static_cast<size_t>(n * 2), "fp8 linear scale");
    if (rc != FTX_OK) return rc;
    if (k > 0) {
      if (!w[s]) return ftx::fail(FTX_ERR_INVALID, "null pointer");
      if (reinterpret_cast<uintptr_t>(w[s]) % 16 != 0)
        return ftx::fail(FTX_ERR_INVALID, "x and w need 16-byte alignment");
      rc = ftx::check_device_range(w[s], static_cast<size_t>(n * k), "fp8 linear weight");
      if (rc != FTX_OK) return rc;
    }
    p.w[s] = w[s];
    p.scale[s] = scale[s];
    p.y[s] = y[s];
  }
  if (k > 0) {
    if (!x) return ftx::fail(FTX_ERR_INVALID, "null pointer");
    if (reinterpret_cast<uintptr_t>(x) % 16 != 0) return ftx::fail(FTX_ERR_INVALID, "x and w need 16-byte alignment");
    int rc = ftx::check_device_range(x, static_cast<size_t>(m * k * 2), "fp8 linear input");
    if (rc != FTX_OK) return rc;
  }
  if (p.epilogue == ftx::kFp8EpilogueResidual) {
    if (!p.residual) return ftx::fail(FTX_ERR_INVALID, "the residual epilogue needs a residual");
    if (reinterpret_cast<uintptr_t>(p.residual) % 2 != 0)
      return ftx::fail(FTX_ERR_INVALID, "residual needs 2-byte alignment");
    int rc = ftx::check_device_range(p.residual, static_cast<size_t>(m * p.n[0] * 2), "fp8 linear residual");
    if (rc != FTX_OK) return rc;
  }
  if (p.workspace_bytes > 0 && !static_workspace) {
    if (!workspace || workspace_bytes < p.workspace_bytes)
      return ftx::fail(FTX_ERR_INVALID, "fp8 linear needs a workspace of " + std::to_string(p.workspace_bytes) +
                                            " bytes (ftx_fp8_linear_workspace)");
    if (reinterpret_cast<uintptr_t>(workspace) % 16 != 0)
      return ftx::fail(FTX_ERR_INVALID, "workspace needs 16-byte alignment");
    int rc = ftx::check_device_range(workspace, p.workspace_bytes, "fp8 linear workspace");
    if (rc != FTX_OK) return rc;
  }
  p.x = x;
  p.workspace = workspace;
  FTX_HIP(ftx::launch_fp8_linear(p, static_cast<hipStream_t>(stream)));
  return FTX_OK;
}

}  // namespace

int ftx_fp8_linear(const void *x, const void *w, const void *scale, void *y, int64_t m, int64_t n, int64_t k,
                   void *workspace, size_t workspace_bytes, void *stream) {
  return ftx_fp8_linear_group(x, 1, &w, &scale, &y, &n, m, k, workspace, workspace_bytes, stream);
}

int ftx_fp8_linear_group(const void *x, int group, const void *const *w, const void *const *scale, void *const *y,
                         const int64_t *n, int64_t m, int64_t k, void *workspace, size_t workspace_bytes,
                         void *stream) {
  FTX_REQUIRE_LIVE();
  ftx::Fp8LinearLaunch p;
  int rc = plan_fp8(m, n, group, k, &p);
  if (rc != FTX_OK) return rc;
  if (m == 0 || p.n_total == 0) return FTX_OK;
  return run_fp8(p, x, w, scale, y, workspace, workspace_bytes, false, stream);
}

int ftx_fp8_linear_fused_workspace(int64_t m, const int64_t *n, int group, int64_t k, int epilogue, size_t *bytes) {
  if (!bytes) return ftx::fail(FTX_ERR_INVALID, "bytes is null");
  ftx::Fp8LinearLaunch p;
  int rc = plan_fp8(m, n, group, k, &p, epilogue);
  if (rc != FTX_OK) return rc;
  *bytes = p.workspace_bytes;
  return FTX_OK;
}

int ftx_fp8_linear_fused(const void *x, int group, const void *const *w, const void *const *scale, void *y,
                         const int64_t *n, int64_t m, int64_t k, int epilogue, const void *residual, void *workspace,
                         size_t workspace_bytes, void *stream) {
  FTX_REQUIRE_LIVE();
  ftx::Fp8LinearLaunch p;
  int rc = plan_fp8(m, n, group, k, &p, epilogue);
  if (rc != FTX_OK) return rc;
  if (m == 0 || p.n_total == 0) return FTX_OK;
  if (!y) return ftx::fail(FTX_ERR_INVALID, "null pointer");
  // Each matrix's output slot is the one output: the SwiGLU reduce writes only the gate's, and the
  // up matrix's slot (same shape) is checked and never written.
  void *const ys[ftx::kFp8MaxGroup] = {y, y, y, y};
  p.residual = residual;
  return run_fp8(p, x, w, scale, ys, workspace, workspace_bytes, false, stream);
}

int ftx_fp8_linear_static(const void *x, const void *w, const void *scale, void *y, int64_t m, int64_t n, int64_t k,
                          void *stream) {
  FTX_REQUIRE_LIVE();
  ftx::Fp8LinearLaunch p;
  int rc = plan_fp8(m, &n, 1, k, &p);
  if (rc != FTX_OK) return rc;
  if (m == 0 || n == 0) return FTX_OK;
  if (p.workspace_bytes > FTX_FP8_STATIC_SCRATCH_BYTES)
    return ftx::fail(FTX_ERR_UNSUPPORTED,
                     "fp8 linear of " + std::to_string(m) + " x " + std::to_string(n) + " x " + std::to_string(k) +
                         " needs " + std::to_string(p.workspace_bytes) + " bytes of split-K partial sums, more than "
                         "the static scratch's " + std::to_string(FTX_FP8_STATIC_SCRATCH_BYTES) +
                         " bytes; call ftx_fp8_linear with a workspace instead");
  void *ws = nullptr;
  if (p.workspace_bytes > 0) {
    rc = ftx::static_scratch(&ws);
    if (rc != FTX_OK) return rc;
  }
  return run_fp8(p, x, &w, &scale, &y, ws, p.workspace_bytes, true, stream);
}

int ftx_scatter_plan_create(const ftx_desc *descs, int n_desc, size_t tile_bytes, ftx_scatter_plan **plan) {
  FTX_REQUIRE_LIVE();
  if (!plan) return ftx::fail(FTX_ERR_INVALID, "plan is null");
  PlanTables t;
  int rc = build_plan_tables(descs, n_desc, tile_bytes, &t);
  if (rc != FTX_OK) return rc;
  void *storage = nullptr;
  FTX_HIP(hipMalloc(&storage, t.buf.size()));
  hipError_t err = hipMemcpy(storage, t.buf.data(), t.buf.size(), hipMemcpyHostToDevice);
  if (err != hipSuccess) {
    (void)hipFree(storage);
    return ftx::hip_fail(err, "hipMemcpy(scatter plan)");
  }
  auto *p = new ftx_scatter_plan;
  p->dev = plan_view(t, storage, tile_bytes);
  p->storage = storage;
  p->n_desc_in = n_desc;
  p->total_bytes = t.total_bytes;
  p->max_src_end = t.max_src_end;
  *plan = p;
  return FTX_OK;
}

int ftx_scatter_plan_destroy(ftx_scatter_plan *plan) {
  if (!plan) return FTX_OK;
  hipError_t err = hipFree(plan->storage);
  delete plan;
  FTX_HIP(err);
  return FTX_OK;
}

int ftx_scatter_plan_info(const ftx_scatter_plan *plan, int *n_desc, int64_t *n_tiles, uint64_t *total_bytes) {
  if (!plan) return ftx::fail(FTX_ERR_INVALID, "plan is null");
  if (n_desc) *n_desc = plan->n_desc_in;
  if (n_tiles) *n_tiles = plan->dev.n_tiles;
  if (total_bytes) *total_bytes = plan->total_bytes;
  return FTX_OK;
}

int ftx_scatter_run(const ftx_scatter_plan *plan, const void *chunk, void *stream) {
  FTX_REQUIRE_LIVE();
  if (!plan) return ftx::fail(FTX_ERR_INVALID, "plan is null");
  if (plan->dev.n_tiles == 0) return FTX_OK;
  if (!chunk) return ftx::fail(FTX_ERR_INVALID, "chunk is null");
  int rc = ftx::check_device_range(chunk, plan->max_src_end, "scatter chunk");
  if (rc != FTX_OK) return rc;
  FTX_HIP(ftx::launch_scatter(plan->dev, chunk, static_cast<hipStream_t>(stream)));
  return FTX_OK;
}

int ftx_scatter(const void *chunk, const ftx_desc *descs, int n_desc, void *stream) {
  FTX_REQUIRE_LIVE();
  PlanTables t;
  int rc = build_plan_tables(descs, n_desc, 0, &t);
  if (rc != FTX_OK) return rc;
  if (t.n_tiles == 0) return FTX_OK;
  if (!chunk) return ftx::fail(FTX_ERR_INVALID, "chunk is null");
  rc = ftx::check_device_range(chunk, t.max_src_end, "scatter chunk");
  if (rc != FTX_OK) return rc;
  hipStream_t s = static_cast<hipStream_t>(stream);
  void *storage = nullptr;
  FTX_HIP(hipMallocAsync(&storage, t.buf.size(), s));
  hipError_t err = hipMemcpyAsync(storage, t.buf.data(), t.buf.size(), hipMemcpyHostToDevice, s);
  if (err == hipSuccess) err = ftx::launch_scatter(plan_view(t, storage, 0), chunk, s);
  if (err == hipSuccess) {
    // The pageable source table must stay valid until the upload has been
    // staged; synchronizing keeps the one-shot form simple and safe.
    err = hipStreamSynchronize(s);
  }
  hipError_t ferr = hipFreeAsync(storage, s);
  FTX_HIP(err);
  FTX_HIP(ferr);
  return FTX_OK;
}

int ftx_hbm_read_probe(const void *dev, size_t nbytes, void *sink, int grid, void *stream) {
  FTX_REQUIRE_LIVE();
  if (nbytes == 0) return FTX_OK;
  if (!dev || !sink) return ftx::fail(FTX_ERR_INVALID, "null pointer");
  if (reinterpret_cast<uintptr_t>(dev) % 16 != 0 || nbytes % 16 != 0)
    return ftx::fail(FTX_ERR_INVALID, "the read probe needs a 16-byte aligned range of whole 16-byte vectors");
  if (reinterpret_cast<uintptr_t>(sink) % 4 != 0) return ftx::fail(FTX_ERR_INVALID, "sink needs 4-byte alignment");
  if (grid <= 0 || grid > (1 << 20)) return ftx::fail(FTX_ERR_INVALID, "grid must be in [1, 2^20]");
  int rc = ftx::check_device_range(dev, nbytes, "read probe input");
  if (rc == FTX_OK) rc = ftx::check_device_range(sink, 4, "read probe sink");
  if (rc != FTX_OK) return rc;
  FTX_HIP(ftx::launch_read_probe(dev, nbytes, static_cast<uint32_t *>(sink), grid, static_cast<hipStream_t>(stream)));
  return FTX_OK;
}

int ftx_mfma_probe(int workgroups, int iters, void *sink, void *stream) {
  return ftx_mfma_probe_shape(ftx::kMfmaProbe16x16x32, workgroups, iters, sink, stream);
}

int ftx_mfma_probe_shape(int shape, int workgroups, int iters, void *sink, void *stream) {
  FTX_REQUIRE_LIVE();
  if (shape != ftx::kMfmaProbe16x16x32 && shape != ftx::kMfmaProbe32x32x16)
    return ftx::fail(FTX_ERR_INVALID, "shape must be 0 (16x16x32) or 1 (32x32x16)");
  if (!sink) return ftx::fail(FTX_ERR_INVALID, "null pointer");
  if (reinterpret_cast<uintptr_t>(sink) % 4 != 0) return ftx::fail(FTX_ERR_INVALID, "sink needs 4-byte alignment");
  if (workgroups <= 0 || workgroups > (1 << 20)) return ftx::fail(FTX_ERR_INVALID, "workgroups must be in [1, 2^20]");
  if (iters <= 0 || iters > (1 << 20)) return ftx::fail(FTX_ERR_INVALID, "iters must be in [1, 2^20]");
  int rc = ftx::check_device_range(sink, 4, "mfma probe sink");
  if (rc != FTX_OK) return rc;
  FTX_HIP(ftx::launch_mfma_probe(shape, workgroups, iters, static_cast<float *>(sink),
                                 static_cast<hipStream_t>(stream)));
  return FTX_OK;
}

int ftx_checksum64(const void *dev, size_t nbytes, void *stream, uint64_t *out) {
  FTX_REQUIRE_LIVE();
  if (!out) return ftx::fail(FTX_ERR_INVALID, "out is null");
  if (nbytes == 0) {
    *out = ftx::splitmix64(0);
    return FTX_OK;
  }
  if (!dev) return ftx::fail(FTX_ERR_INVALID, "dev is null");
  if (reinterpret_cast<uintptr_t>(dev) % 8 != 0) return ftx::fail(FTX_ERR_INVALID, "checksum needs 8-byte alignment");
  {
    int vrc = ftx::check_device_range(dev, nbytes, "checksum input");
    if (vrc != FTX_OK) return vrc;
  }
  int cus = 256;
  {
    ftx::DeviceState *st = nullptr;
    if (ftx::device_state(&st) == FTX_OK) cus = st->cu_count;
  }
  const uint64_t n_blocks = (nbytes + ftx::kChecksumBlockBytes - 1) / ftx::kChecksumBlockBytes;
  uint64_t waves = std::min<uint64_t>(n_blocks, static_cast<uint64_t>(cus) * 32);
  waves = (waves + 3) / 4 * 4;
  hipStream_t s = static_cast<hipStream_t>(stream);
  uint64_t *partials = nullptr;
  FTX_HIP(hipMalloc(&partials, waves * sizeof(uint64_t)));
  std::vector<uint64_t> host(waves, 0);
  hipError_t err = ftx::launch_checksum(dev, nbytes, partials, static_cast<int>(waves), s);
  if (err == hipSuccess) err = hipMemcpyAsync(host.data(), partials, waves * sizeof(uint64_t), hipMemcpyDeviceToHost, s);
  if (err == hipSuccess) err = hipStreamSynchronize(s);
  hipError_t ferr = hipFree(partials);
  FTX_HIP(err);
  FTX_HIP(ferr);
  uint64_t sum = 0;
  for (uint64_t v : host) sum += v;
  *out = ftx::splitmix64(sum + static_cast<uint64_t>(nbytes));
  return FTX_OK;
}

}  // extern "C"
