// HIP kernels of the streaming engine, written for gfx950 (CDNA4, wave64).
//
//  * zero_copy_kernel  - host-to-device copy executed by the CUs: every lane
//                        issues 16-byte non-temporal loads from mapped pinned
//                        host memory (PCIe reads) and stores into HBM. A small
//                        grid is launched with the CU's whole LDS as dynamic
//                        shared memory, which the kernel never touches: no
//                        workgroup that uses LDS (a GEMM's) can then share a CU
//                        with a copy workgroup. Sharing one slowed both: an
//                        LDS-using HBM reader beside an 8-workgroup copy ran
//                        1.63-1.79x its time alone and the copy 49 GB/s; with
//                        the CUs reserved, 1.15-1.25x and 56.6-56.9 GB/s.
//  * scatter_kernel    - places one streamed chunk into many destination
//                        tensors in one launch. Work is split into fixed-size
//                        byte tiles; each workgroup stages the (at most four)
//                        descriptors its tiles touch in LDS and each wavefront
//                        copies one tile, so a small tensor is one wavefront
//                        and a large one is spread over many workgroups.
//  * checksum_kernel   - order-sensitive 64-bit checksum used to check
//                        streamed bytes at full size without a host copy.
//  * fill_kernel       - byte fill (memset replacement that is safe to
//                        capture in a graph).
//  * timestamp_kernel  - writes the wall clock to device memory; the timing
//                        points of captured graphs.
//  * read_probe_kernel - a plain streaming read (measurement only): the HBM
//                        read rate the HBM-bound kernels are compared with.
//
// None of these kernels has data reuse, so blockIdx is mapped linearly: the
// round-robin dispatch over the 8 XCDs only spreads independent tiles.
#include "ftx_internal.h"

namespace ftx {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;
constexpr int kWave = 64;
constexpr int kZeroCopyUnroll = 8;

__device__ __forceinline__ uint64_t d_splitmix64(uint64_t x) {
  x += 0x9e3779b97f4a7c15ull;
  uint64_t z = x;
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}

__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t v, int mask) {
  int lo = static_cast<int>(static_cast<uint32_t>(v));
  int hi = static_cast<int>(static_cast<uint32_t>(v >> 32));
  lo = __shfl_xor(lo, mask, kWave);
  hi = __shfl_xor(hi, mask, kWave);
  return (static_cast<uint64_t>(static_cast<uint32_t>(hi)) << 32) | static_cast<uint32_t>(lo);
}

// Host-to-device copy by the CUs. `src` is the device-visible address of
// pinned host memory; src and dst are congruent modulo 16 (checked on host).
// Block 0 copies the head bytes before the first 16-byte boundary, the last
// block copies the tail bytes after the last full 16-byte word.
__global__ __launch_bounds__(kThreads) void zero_copy_kernel(uint8_t *__restrict__ dst,
                                                             const uint8_t *__restrict__ src,
                                                             uint64_t nbytes, uint64_t head,
                                                             uint64_t n16) {
  const uint64_t tid = threadIdx.x;
  if (blockIdx.x == 0 && tid < head) dst[tid] = src[tid];
  const uint64_t body_end = head + n16 * 16;
  const uint64_t tail = nbytes - body_end;
  if (blockIdx.x == gridDim.x - 1 && tid < tail) dst[body_end + tid] = src[body_end + tid];

  const u32x4 *s = reinterpret_cast<const u32x4 *>(src + head);
  u32x4 *d = reinterpret_cast<u32x4 *>(dst + head);
  const uint64_t per_iter = static_cast<uint64_t>(gridDim.x) * kThreads * kZeroCopyUnroll;
  for (uint64_t base = static_cast<uint64_t>(blockIdx.x) * kThreads * kZeroCopyUnroll + tid;
       base < n16; base += per_iter) {
    u32x4 v[kZeroCopyUnroll];
#pragma unroll
    for (int k = 0; k < kZeroCopyUnroll; ++k) {
      const uint64_t i = base + static_cast<uint64_t>(k) * kThreads;
      if (i < n16) v[k] = __builtin_nontemporal_load(s + i);
    }
#pragma unroll
    for (int k = 0; k < kZeroCopyUnroll; ++k) {
      const uint64_t i = base + static_cast<uint64_t>(k) * kThreads;
      if (i < n16) __builtin_nontemporal_store(v[k], d + i);
    }
  }
}

// One wavefront copies `len` bytes. The widest access that both pointers
// allow is used: 16 bytes when src and dst are congruent modulo 16, 4 bytes
// when congruent modulo 4, single bytes otherwise.
// Pointers in the global address space. Destinations come from descriptor
// tables, so without the cast the compiler cannot tell they are global and
// emits flat stores (which also count against the LDS counter and add waits).
typedef __attribute__((address_space(1))) u32x4 g_u32x4;
typedef __attribute__((address_space(1))) uint32_t g_u32;
typedef __attribute__((address_space(1))) uint8_t g_u8;
typedef __attribute__((address_space(1))) uint64_t g_u64;

template <typename T>
__device__ __forceinline__ T *as_global(const void *p) {
  return (T *)(p);  // generic -> global address-space cast
}

// One wavefront copies `len` bytes. The widest access that both pointers
// allow is used: 16 bytes when src and dst are congruent modulo 16, 4 bytes
// when congruent modulo 4, single bytes otherwise. In the 16-byte path each
// lane issues UNROLL loads before the matching stores (both non-temporal: the
// bytes are not touched again by this kernel, and streaming stores copy about
// 7% faster than write-allocating ones on a 512 MiB copy); whole rounds of
// 64 x UNROLL words run without bounds checks, and what is left of a partial
// round is copied one word per lane at a time. An 8 KiB tile with UNROLL 8 (the
// default) or a 16 KiB tile with UNROLL 16
// is exactly one round.
template <int UNROLL>
__device__ __forceinline__ void wave_copy(uint8_t *__restrict__ dst_, const uint8_t *__restrict__ src_,
                                          uint64_t len, int lane) {
  g_u8 *dst = as_global<g_u8>(dst_);
  const g_u8 *src = as_global<const g_u8>(src_);
  const uint64_t sa = reinterpret_cast<uint64_t>(src_);
  const uint64_t da = reinterpret_cast<uint64_t>(dst_);
  const uint64_t ln = static_cast<uint64_t>(lane);
  if (((sa ^ da) & 15) == 0) {
    const uint64_t head = min<uint64_t>((16 - (sa & 15)) & 15, len);
    if (ln < head) dst[ln] = src[ln];
    const uint64_t n16 = (len - head) / 16;
    const g_u32x4 *s = as_global<const g_u32x4>(src_ + head);
    g_u32x4 *d = as_global<g_u32x4>(dst_ + head);
    constexpr uint64_t kRound = static_cast<uint64_t>(kWave) * UNROLL;
    const uint64_t full = n16 / kRound * kRound;
    for (uint64_t base = ln; base < full; base += kRound) {
      u32x4 v[UNROLL];
#pragma unroll
      for (int k = 0; k < UNROLL; ++k) v[k] = __builtin_nontemporal_load(s + base + k * kWave);
#pragma unroll
      for (int k = 0; k < UNROLL; ++k) __builtin_nontemporal_store(v[k], d + base + k * kWave);
    }
    for (uint64_t i = full + ln; i < n16; i += kWave) __builtin_nontemporal_store(__builtin_nontemporal_load(s + i), d + i);
    const uint64_t done = head + n16 * 16;
    if (ln < len - done) dst[done + ln] = src[done + ln];
  } else if (((sa ^ da) & 3) == 0) {
    const uint64_t head = min<uint64_t>((4 - (sa & 3)) & 3, len);
    if (ln < head) dst[ln] = src[ln];
    const uint64_t n4 = (len - head) / 4;
    const g_u32 *s = as_global<const g_u32>(src_ + head);
    g_u32 *d = as_global<g_u32>(dst_ + head);
    for (uint64_t i = ln; i < n4; i += kWave) d[i] = s[i];
    const uint64_t done = head + n4 * 4;
    if (ln < len - done) dst[done + ln] = src[done + ln];
  } else {
    for (uint64_t i = ln; i < len; i += kWave) dst[i] = src[i];
  }
}

// Batched scatter. Descriptors with zero bytes are dropped when the plan is
// built, so every descriptor owns at least one tile and the
// kScatterWavesPerGroup consecutive tiles of a workgroup touch at most
// kScatterWavesPerGroup consecutive descriptors starting at group_desc0.
template <int UNROLL>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(6))) void scatter_kernel(const ftx_desc *__restrict__ descs,
                                                           const uint64_t *__restrict__ tile_start,
                                                           const uint32_t *__restrict__ group_desc0,
                                                           int n_desc, int64_t n_tiles,
                                                           uint64_t tile_bytes,
                                                           const uint8_t *__restrict__ chunk) {
  __shared__ ftx_desc s_desc[kScatterWavesPerGroup];
  __shared__ uint64_t s_tile_start[kScatterWavesPerGroup + 1];

  const int t = threadIdx.x;
  const uint32_t d0 = group_desc0[blockIdx.x];
  const int nd = min(kScatterWavesPerGroup, n_desc - static_cast<int>(d0));
  if (t < nd) s_desc[t] = descs[d0 + t];
  if (t <= nd) s_tile_start[t] = tile_start[d0 + t];
  __syncthreads();

  const int wave = t / kWave;
  const int lane = t % kWave;
  const int64_t tile = static_cast<int64_t>(blockIdx.x) * kScatterWavesPerGroup + wave;
  if (tile >= n_tiles) return;

  int j = 0;
  for (int q = 1; q < nd; ++q)
    if (s_tile_start[q] <= static_cast<uint64_t>(tile)) j = q;

  const ftx_desc dsc = s_desc[j];
  const uint64_t off = (static_cast<uint64_t>(tile) - s_tile_start[j]) * tile_bytes;
  const uint64_t len = min<uint64_t>(tile_bytes, dsc.nbytes - off);
  wave_copy<UNROLL>(reinterpret_cast<uint8_t *>(dsc.dst) + off, chunk + dsc.src_off + off, len, lane);
}

// Checksum: word w (8 bytes, little endian, zero padded past nbytes) belongs
// to block w / 512, lane (w % 512) % 64, step (w % 512) / 64. Each lane folds
// its 8 words with FNV-1a (64-bit words); a block sums splitmix64(h + lane)
// over its lanes; each wave accumulates splitmix64(block_sum + block) over
// its blocks and writes one partial. The host finishes with
// splitmix64(sum(partials) + nbytes).
__global__ __launch_bounds__(kThreads) void checksum_kernel(const uint8_t *__restrict__ p,
                                                            uint64_t nbytes, uint64_t n_blocks,
                                                            uint64_t *__restrict__ partials) {
  const int lane = threadIdx.x % kWave;
  const uint64_t gw = static_cast<uint64_t>(blockIdx.x) * (kThreads / kWave) + threadIdx.x / kWave;
  const uint64_t nw = static_cast<uint64_t>(gridDim.x) * (kThreads / kWave);
  const uint64_t full_words = nbytes / 8;
  const uint64_t *p64 = reinterpret_cast<const uint64_t *>(p);
  uint64_t acc = 0;
  for (uint64_t b = gw; b < n_blocks; b += nw) {
    uint64_t h = 0xcbf29ce484222325ull;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const uint64_t w = b * 512 + static_cast<uint64_t>(k) * kWave + lane;
      uint64_t x = 0;
      if (w < full_words) {
        x = p64[w];
      } else if (w * 8 < nbytes) {
        for (uint64_t q = w * 8; q < nbytes; ++q) x |= static_cast<uint64_t>(p[q]) << (8 * (q - w * 8));
      }
      h = (h ^ x) * 0x100000001b3ull;
    }
    uint64_t v = d_splitmix64(h + static_cast<uint64_t>(lane));
    for (int m = kWave / 2; m >= 1; m >>= 1) v += shfl_xor_u64(v, m);
    acc += d_splitmix64(v + b);
  }
  if (lane == 0) partials[gw] = acc;
}

__global__ __launch_bounds__(kThreads) void fill_kernel(uint8_t *__restrict__ p, uint8_t value,
                                                        uint64_t nbytes, uint64_t head, uint64_t n16) {
  const uint64_t tid = static_cast<uint64_t>(blockIdx.x) * kThreads + threadIdx.x;
  const uint64_t stride = static_cast<uint64_t>(gridDim.x) * kThreads;
  if (tid < head) p[tid] = value;
  const uint64_t body_end = head + n16 * 16;
  if (tid < nbytes - body_end) p[body_end + tid] = value;
  const uint32_t w = 0x01010101u * value;
  u32x4 vv = {w, w, w, w};
  u32x4 *d = reinterpret_cast<u32x4 *>(p + head);
  for (uint64_t i = tid; i < n16; i += stride) d[i] = vv;
}

// Streams n16 16-byte vectors with eight non-temporal loads in flight per
// lane (grid-stride), folds them into one word and stores it only when it
// equals `never` (practically never): the loads cannot be optimised away and
// nothing is written. Measures the plain read rate of HBM.
constexpr int kReadProbeUnroll = 8;
__global__ __launch_bounds__(kThreads) void read_probe_kernel(const u32x4 *__restrict__ p, uint64_t n16,
                                                              uint32_t never, uint32_t *__restrict__ sink) {
  const uint64_t stride = static_cast<uint64_t>(gridDim.x) * kThreads;
  uint64_t i = static_cast<uint64_t>(blockIdx.x) * kThreads + threadIdx.x;
  uint32_t acc = 0;
  for (; i + (kReadProbeUnroll - 1) * stride < n16; i += kReadProbeUnroll * stride) {
    u32x4 v[kReadProbeUnroll];
#pragma unroll
    for (int j = 0; j < kReadProbeUnroll; ++j) v[j] = __builtin_nontemporal_load(p + i + j * stride);
#pragma unroll
    for (int j = 0; j < kReadProbeUnroll; ++j) acc ^= v[j][0] ^ v[j][1] ^ v[j][2] ^ v[j][3];
  }
  for (; i < n16; i += stride) {
    const u32x4 v = __builtin_nontemporal_load(p + i);
    acc ^= v[0] ^ v[1] ^ v[2] ^ v[3];
  }
  if (acc == never) sink[0] = acc;
}

// One lane writes the constant-rate wall clock (a vector store).
__global__ __launch_bounds__(kWave) void timestamp_kernel(uint64_t *__restrict__ slot) {
  if (threadIdx.x == 0) *as_global<g_u64>(slot) = static_cast<uint64_t>(wall_clock64());
}

}  // namespace

hipError_t launch_timestamp(uint64_t *slot, hipStream_t stream) {
  hipLaunchKernelGGL(timestamp_kernel, dim3(1), dim3(kWave), 0, stream, slot);
  return hipGetLastError();
}

hipError_t allow_zero_copy_lds(size_t bytes) {
  return hipFuncSetAttribute(reinterpret_cast<const void *>(zero_copy_kernel),
                             hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(bytes));
}

hipError_t launch_zero_copy(void *dst, const void *src_dev, size_t nbytes, int grid, size_t reserve_lds,
                            hipStream_t stream) {
  if (nbytes == 0) return hipSuccess;
  const uint64_t sa = reinterpret_cast<uint64_t>(src_dev);
  const uint64_t head = std::min<uint64_t>((16 - (sa & 15)) & 15, nbytes);
  const uint64_t n16 = (nbytes - head) / 16;
  const uint64_t per_block = static_cast<uint64_t>(kThreads) * kZeroCopyUnroll;
  uint64_t need = (n16 + per_block - 1) / per_block;
  if (need < 1) need = 1;
  const int g = static_cast<int>(std::min<uint64_t>(need, static_cast<uint64_t>(grid)));
  hipLaunchKernelGGL(zero_copy_kernel, dim3(g), dim3(kThreads), static_cast<unsigned>(reserve_lds), stream,
                     static_cast<uint8_t *>(dst), static_cast<const uint8_t *>(src_dev),
                     static_cast<uint64_t>(nbytes), head, n16);
  return hipGetLastError();
}

hipError_t launch_scatter(const ScatterPlanDev &plan, const void *chunk, hipStream_t stream) {
  if (plan.n_tiles == 0) return hipSuccess;
  // 16 KiB and larger tiles: 16 loads in flight per lane; smaller tiles: 8.
  if (plan.tile_bytes >= 16 * 1024)
    hipLaunchKernelGGL(scatter_kernel<16>, dim3(static_cast<unsigned>(plan.n_groups)), dim3(kThreads), 0,
                       stream, plan.descs, plan.tile_start, plan.group_desc0, plan.n_desc,
                       plan.n_tiles, plan.tile_bytes, static_cast<const uint8_t *>(chunk));
  else
    hipLaunchKernelGGL(scatter_kernel<8>, dim3(static_cast<unsigned>(plan.n_groups)), dim3(kThreads), 0,
                       stream, plan.descs, plan.tile_start, plan.group_desc0, plan.n_desc,
                       plan.n_tiles, plan.tile_bytes, static_cast<const uint8_t *>(chunk));
  return hipGetLastError();
}

hipError_t launch_checksum(const void *dev, size_t nbytes, uint64_t *partials, int n_waves,
                           hipStream_t stream) {
  const uint64_t n_blocks = (nbytes + kChecksumBlockBytes - 1) / kChecksumBlockBytes;
  const int groups = n_waves / (kThreads / kWave);
  hipLaunchKernelGGL(checksum_kernel, dim3(groups), dim3(kThreads), 0, stream,
                     static_cast<const uint8_t *>(dev), static_cast<uint64_t>(nbytes), n_blocks,
                     partials);
  return hipGetLastError();
}

hipError_t launch_read_probe(const void *dev, size_t nbytes, uint32_t *sink, int grid, hipStream_t stream) {
  hipLaunchKernelGGL(read_probe_kernel, dim3(static_cast<unsigned>(grid)), dim3(kThreads), 0, stream,
                     static_cast<const u32x4 *>(dev), static_cast<uint64_t>(nbytes / 16), 0x9e3779b9u, sink);
  return hipGetLastError();
}

hipError_t launch_fill_u8(void *dev, uint8_t value, size_t nbytes, hipStream_t stream) {
  if (nbytes == 0) return hipSuccess;
  const uint64_t a = reinterpret_cast<uint64_t>(dev);
  const uint64_t head = std::min<uint64_t>((16 - (a & 15)) & 15, nbytes);
  const uint64_t n16 = (nbytes - head) / 16;
  uint64_t need = (n16 + kThreads - 1) / kThreads;
  if (need < 1) need = 1;
  const int g = static_cast<int>(std::min<uint64_t>(need, 4096));
  hipLaunchKernelGGL(fill_kernel, dim3(g), dim3(kThreads), 0, stream, static_cast<uint8_t *>(dev),
                     value, static_cast<uint64_t>(nbytes), head, n16);
  return hipGetLastError();
}

}  // namespace ftx
