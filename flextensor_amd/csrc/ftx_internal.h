// Internal declarations shared by the runtime (C ABI) and the kernel file.
#pragma once

#include <hip/hip_runtime.h>
#include <cstddef>
#include <cstdint>
#include <string>

#include "../../include/ftx.h"

namespace ftx {

// Thread-local error message behind ftx_last_error().
void set_error(const std::string &msg);
int fail(int code, const std::string &msg);
int hip_fail(hipError_t err, const char *what);

#define FTX_HIP(expr)                                   \
  do {                                                  \
    hipError_t ftx_err_ = (expr);                       \
    if (ftx_err_ != hipSuccess) return ::ftx::hip_fail(ftx_err_, #expr); \
  } while (0)

// Set once by ftx_shutdown. Entry points that start work or allocate refuse
// afterwards (FTX_REQUIRE_LIVE); releasing, waiting and querying still work.
bool is_shut_down();
#define FTX_REQUIRE_LIVE()                                                                        \
  do {                                                                                            \
    if (::ftx::is_shut_down())                                                                    \
      return ::ftx::fail(FTX_ERR_UNSUPPORTED, "the library has been shut down (ftx_shutdown)"); \
  } while (0)

// Default bytes per wave tile of the scatter kernel: one round of 8 loads and
// 8 non-temporal stores of 16 bytes per lane (fastest of 8/16/32 KiB on the
// 2000-tensor set's 512 MiB chunks: 5.94 TB/s against 5.78 and 5.77).
constexpr size_t kScatterTileBytes = 8 * 1024;
// Default zero-copy grid: 64 workgroups keep the link at its peak (more
// workgroups only add outstanding PCIe reads).
constexpr int kZeroCopyDefaultGrid = 64;
// A zero-copy launch of at most this many workgroups takes each CU it runs on
// whole (its workgroups reserve the CU's LDS).
constexpr int kZeroCopyReserveMaxGrid = 16;
// Wave tiles handled by one workgroup (one tile per wavefront).
constexpr int kScatterWavesPerGroup = 4;
// Checksum block: 64 lanes x 8 bytes x 8 steps.
constexpr size_t kChecksumBlockBytes = 4096;

// Device-resident scatter plan.
struct ScatterPlanDev {
  const ftx_desc *descs;        // n_desc descriptors
  const uint64_t *tile_start;   // n_desc + 1 exclusive prefix of tiles per descriptor
  const uint32_t *group_desc0;  // n_groups: descriptor of each workgroup's first tile
  int n_desc;
  int64_t n_tiles;
  int64_t n_groups;
  uint64_t tile_bytes;
};

// One launch of the fp8-weight linear kernel (ftx_gemm.hip), as planned by
// plan_fp8_linear from the shapes, the CU count and optional overrides. A
// launch covers `group` weight matrices (segments) that share the input x and
// k: y_s = bf16(scale_s * x @ w_s^T) for each segment s.
constexpr int kFp8MaxGroup = 4;
// Epilogues the decode kernel's reduce can apply (FTX_FP8_EPILOGUE_* in ftx.h).
constexpr int kFp8EpilogueNone = FTX_FP8_EPILOGUE_NONE;
constexpr int kFp8EpilogueSwiglu = FTX_FP8_EPILOGUE_SWIGLU;
constexpr int kFp8EpilogueResidual = FTX_FP8_EPILOGUE_RESIDUAL;
struct Fp8LinearLaunch {
  const void *x;                       // bf16 [m, k]
  int group;                           // segments in this launch, 1..kFp8MaxGroup
  const void *w[kFp8MaxGroup];         // e4m3fn [n_s, k]
  const void *scale[kFp8MaxGroup];     // bf16 [n_s]
  void *y[kFp8MaxGroup];               // bf16 [m, n_s]
  int64_t n[kFp8MaxGroup];             // output rows of each segment
  int64_t n_total;                     // sum of n
  void *workspace;    // fp32 partial sums [splits, m, n_s] per segment, back to back, when splits > 1
  int64_t m, k;
  int batch_blocks;   // 16-column batch blocks: 1, 2 or 4 (m <= 16 * batch_blocks)
  int waves;          // wavefronts per workgroup, 16 output rows each
  int splits;         // K slices, one workgroup each per row group
  int64_t kc;         // K values per slice (multiple of 256)
  int64_t row_groups; // groups of 16 * waves output rows, summed over segments
  int64_t grid;       // workgroups = row_groups * splits
  size_t lds_bytes;   // activation slice + one weight tile per wave
  size_t workspace_bytes;
  int epilogue;         // kFp8Epilogue*: what the reduce kernel applies to the outputs
  const void *residual; // bf16 [m, n[0]] for kFp8EpilogueResidual
  bool prefill;       // more than kFp8LinearMaxRows rows: the tiled prefill kernel (no split, no workspace)
  int64_t m_tiles;    // prefill: tiles of 128 activation rows (row_groups then counts tiles of 128 channels)
  int xcds;           // prefill: L2 domains the block order is arranged for
};
constexpr int kFp8LinearMaxRows = 64;
constexpr size_t kFp8LinearMaxLds = 64 * 1024;
Fp8LinearLaunch plan_fp8_linear(int64_t m, const int64_t *n, int group, int64_t k, int cus, int xcds, int waves,
                                int kc, int epilogue);
hipError_t launch_fp8_linear(const Fp8LinearLaunch &p, hipStream_t stream);
// MFMA rate probe: `workgroups` x 4 waves, each iters x 32 v_mfma_f32_16x16x32_bf16.
constexpr int kMfmaProbe16x16x32 = 0;  // v_mfma_f32_16x16x32_bf16, the prefill kernel's instruction
constexpr int kMfmaProbe32x32x16 = 1;  // v_mfma_f32_32x32x16_bf16
hipError_t launch_mfma_probe(int shape, int workgroups, int iters, float *sink, hipStream_t stream);

// Staged copies from pageable host memory and the parallel host memcpy
// (ftx_staged.hip).
int staged_copy_h2d(void *dst, const void *src, size_t nbytes, hipStream_t stream);
int host_memcpy(void *dst, const void *src, size_t nbytes);
int set_staging_policy(size_t piece_bytes, int threads);
void get_staging_policy(size_t *piece_bytes, int *threads);
// Joins the host threads and frees every device's staging buffers and events
// (each device made current in turn). Returns the first failure, after trying all.
int staged_shutdown();

// Kernel launchers (ftx_kernels.hip). Each returns hipSuccess or the launch error.
// `reserve_lds` bytes of dynamic LDS per workgroup (0: none); see zero_copy_kernel.
hipError_t launch_zero_copy(void *dst, const void *src_dev, size_t nbytes, int grid, size_t reserve_lds,
                            hipStream_t stream);
// Lets zero_copy_kernel take `bytes` of dynamic LDS on the current device.
hipError_t allow_zero_copy_lds(size_t bytes);
hipError_t launch_scatter(const ScatterPlanDev &plan, const void *chunk, hipStream_t stream);
hipError_t launch_checksum(const void *dev, size_t nbytes, uint64_t *partials, int n_waves,
                           hipStream_t stream);
hipError_t launch_fill_u8(void *dev, uint8_t value, size_t nbytes, hipStream_t stream);
hipError_t launch_timestamp(uint64_t *slot, hipStream_t stream);
hipError_t launch_read_probe(const void *dev, size_t nbytes, uint32_t *sink, int grid, hipStream_t stream);

// Exponent-coded blocks (ftx_expcode.hip): the layout of one encoded block.
constexpr uint64_t kExpcodeHeaderBytes = 256;
constexpr uint64_t kExpcodeGroupWords = 1024;
// Default decode grid: workgroups of 8 waves, each lane with eight groups' loads in flight.
constexpr int kExpcodeDefaultGrid = 16;
struct ExpcodeInfo {
  uint64_t n;        // raw bytes
  uint64_t n_words;  // n / 2
  uint64_t groups;   // groups of kExpcodeGroupWords words
  uint64_t escapes;  // escaped words
  uint64_t off_b, off_s, off_x, total;  // section offsets and encoded size (plane A starts at the header's end)
  uint8_t table[16];                    // exponent of each code below 15
  uint8_t tail;                         // the odd last raw byte
};
// out == nullptr: only *out_bytes (the encoded size) is computed.
int expcode_encode(const void *raw, size_t nbytes, void *out, size_t out_capacity, size_t *out_bytes);
// Reads and checks the header of an encoded block of src_bytes bytes in host memory.
int expcode_parse(const void *src, size_t src_bytes, ExpcodeInfo *info);
// Decodes the block of raw size n at src_dev (a device-visible address, `capacity` bytes readable) into
// dst; the kernel reads the block's header when it runs. `reserve_lds` as for launch_zero_copy.
hipError_t launch_expcode_decode(void *dst, const void *src_dev, uint64_t capacity, uint64_t n, int grid,
                                 size_t reserve_lds, hipStream_t stream);
hipError_t allow_expcode_lds(size_t bytes);

// Dense exponent-coded blocks (version 2): 3-bit primary codes for the 7 most frequent exponents in three
// bit planes, a 4-bit secondary code per primary escape for the next 15, a list for the rest. Sections
// after the 256-byte header: plane A (1024 bytes a group), plane P (384 a group), S1 and S2 (G + 1 u32
// each, 16-byte aligned), Y (a nibble per primary escape, 16-byte aligned), X (a u32 per secondary escape).
constexpr uint64_t kDensePlaneBytes = 384;
struct DenseLayout {
  uint64_t n, n_words, groups, e1, e2;
  uint64_t off_p, off_s1, off_s2, off_y, off_x, total;
};
// The section offsets of a dense block of raw size n with e1 primary and e2 secondary escapes.
DenseLayout dense_layout(uint64_t n, uint64_t e1, uint64_t e2);
// out == nullptr: only *out_bytes (the encoded size) is computed.
int expcode_encode_dense(const void *raw, size_t nbytes, void *out, size_t out_capacity, size_t *out_bytes);
// Decodes the dense block of raw size n at src_dev (device memory, `capacity` bytes readable) into dst; the
// kernel reads the block's header when it runs and writes nothing for a header of another raw size.
hipError_t launch_expcode_dense_decode(void *dst, const void *src_dev, uint64_t capacity, uint64_t n, int grid,
                                       size_t reserve_lds, hipStream_t stream);
// Reads and checks the header of a dense block of src_bytes bytes in host memory.
int expcode_parse_dense(const void *src, size_t src_bytes, DenseLayout *layout);
// The dense decode from mapped host memory (over the link): `reserve_lds` as for launch_zero_copy.
hipError_t launch_expcode_dense_link_decode(void *dst, const void *src_dev, uint64_t capacity, uint64_t n, int grid,
                                            size_t reserve_lds, hipStream_t stream);

// Host-side helpers shared with the oracle's definition of the checksum.
inline uint64_t splitmix64(uint64_t x) {
  x += 0x9e3779b97f4a7c15ull;
  uint64_t z = x;
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}

}  // namespace ftx
