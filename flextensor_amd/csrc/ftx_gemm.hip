// fp8-weight linear layer for decode-sized batches, written for gfx950.
//
//   y[m, n] = bf16( scale[n] * sum_k x[m, k] * w[n, k] )
//
// x is bf16 [M, K], w is float8 e4m3fn [N, K] (row-major, K contiguous),
// scale is one bf16 per output channel, y is bf16 [M, N]. Up to 64 rows
// (decode) run fp8_linear_kernel below; more rows (prefill) run the tiled
// fp8_prefill_kernel further down.
//
// Decode multiplies a few activation rows by a large weight matrix, so the
// kernel is bound by reading the fp8 weights from HBM once (1 byte per
// weight). Each lane loads 16 weight bytes of one row, converts them to bf16
// in registers with v_cvt_scalef32_pk_bf16_fp8 (scale 1.0; every e4m3 value is
// exact in bf16) and feeds v_mfma_f32_16x16x32_bf16 with the weights as the A
// operand (16 output channels) and the activations as the B operand (16 batch
// columns). The activations stay bf16, so the products are exactly those of
// dequantizing the weights and running a bf16 GEMM; only the fp32
// accumulation order differs.
//
// Grouping: one launch can cover up to four weight matrices that share x and
// K (a layer's q/k/v projections, its gate/up projections). Their row groups
// are laid end to end in the grid, so the group pays one launch (and one
// reduce) instead of one per matrix.
//
// Work split: a workgroup of S wavefronts owns 16*S output channels (16 per
// wave) of one matrix and one K slice; the grid is row groups x K slices.
// Each workgroup stages its slice of x in LDS once, so L2 serves activations about 2M/(16 S)
// times the weight bytes. With one slice the kernel writes y directly;
// otherwise it writes fp32 partials [slice][M][N] and fp8_linear_reduce_kernel
// sums them in slice order, so results do not depend on timing. The split is
// a separate kernel: an in-kernel last-arriver reduction needs either
// agent-scope release/acquire (a whole-L2 writeback per workgroup) or
// device-coherent partials and counters, and the coherent form measured
// slower than two launches (218 against 172 us for a 70B layer's projections).
//
// MFMA 16x16x32 operand layout (gfx950): lane l supplies row/column l%16 and
// the eight k values 8*(l/16)..8*(l/16)+7 of the 32-wide k block; lane l
// receives D rows 4*(l/16)..4*(l/16)+3 of column l%16. Any permutation of k
// that A and B share gives the same sum, so here lane group g = l/16 holds the
// k values g*16..g*16+15 of a 64-byte piece: the first eight go to one MFMA,
// the last eight to a second one.
#include <algorithm>

#include "ftx_internal.h"

namespace ftx {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;
constexpr int kPieceBytes = 16;              // fp8 bytes one lane loads per row and step
constexpr int kStepBytes = 4 * kPieceBytes;  // K bytes one step covers per row (4 lane groups)

__device__ __forceinline__ bf16x8 join8(bf16x2 a, bf16x2 b, bf16x2 c, bf16x2 d) {
  const bf16x4 lo = __builtin_shufflevector(a, b, 0, 1, 2, 3);
  const bf16x4 hi = __builtin_shufflevector(c, d, 0, 1, 2, 3);
  return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
}

// 16 e4m3fn bytes -> bf16 of bytes 0-7 (lo) and bytes 8-15 (hi), in byte order.
__device__ __forceinline__ void fp8x16_to_bf16(u32x4 w, bf16x8 &lo, bf16x8 &hi) {
  const bf16x2 p0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w[0], 1.0f, false);
  const bf16x2 p1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w[0], 1.0f, true);
  const bf16x2 p2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w[1], 1.0f, false);
  const bf16x2 p3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w[1], 1.0f, true);
  const bf16x2 p4 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w[2], 1.0f, false);
  const bf16x2 p5 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w[2], 1.0f, true);
  const bf16x2 p6 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w[3], 1.0f, false);
  const bf16x2 p7 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w[3], 1.0f, true);
  lo = join8(p0, p1, p2, p3);
  hi = join8(p4, p5, p6, p7);
}

__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }

// fp32 -> bf16 bits, round to nearest even; NaN stays NaN.
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

// Bytes of one weight row loaded per iteration: 16 lanes x 16 bytes, so one
// load instruction covers 4 rows x 256 contiguous bytes. Fewer, longer runs
// per instruction keep HBM near its streaming rate; the MFMA layout (16 rows
// per 16 lanes, 64 bytes each) is reached through a per-wave LDS tile.
constexpr int kIterK = 256;
constexpr int kRowsPerLoad = kWave * kPieceBytes / kIterK;   // 4
constexpr int kLoads = 16 / kRowsPerLoad;                     // 4 per 16 rows
constexpr int kSteps = kIterK / kStepBytes;                   // 4 MFMA steps per iteration
constexpr int kTileRow = kIterK + 16;                         // LDS bytes per staged row (+16: bank spread)
constexpr int kTileBytes = 16 * kTileRow;                     // per wave

// The weight matrices of one launch. Matrix s owns row groups
// [rg0[s], rg0[s+1]), its partial sums start at float offset part0[s]
// ([splits][M][n[s]]) and its outputs are reduced by blocks [rb0[s], rb0[s+1])
// of the reduce kernel.
struct SegTable {
  const uint8_t *w[kFp8MaxGroup];
  const uint16_t *scale[kFp8MaxGroup];
  uint16_t *y[kFp8MaxGroup];
  int n[kFp8MaxGroup];
  int rg0[kFp8MaxGroup + 1];
  int64_t part0[kFp8MaxGroup];
  int rb0[kFp8MaxGroup + 1];
  int count;
};

// Output tile of the prefill kernel (more than kFp8LinearMaxRows rows), below.
constexpr int kPTileM = 128;  // activation rows
constexpr int kPTileN = 128;  // output channels

// MB: 16-column batch blocks (M <= 16*MB). Workgroup b owns rows
// [rg*16*S, rg*16*S + 16*S) (S waves, 16 rows each), rg = b / splits, and
// the K slice [sp*Kc, min(K, (sp+1)*Kc)), sp = b % splits.
template <int MB>
__global__ __launch_bounds__(512) void fp8_linear_kernel(const uint8_t *__restrict__ x, SegTable seg,
                                                         float *__restrict__ part, int M, int K, int Kc, int splits) {
  extern __shared__ __align__(16) uint8_t lds[];  // [M][row_bytes] activations, then S weight tiles
  const int S = blockDim.x / kWave;
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int r = lane & 15;
  const int g = lane >> 4;
  const int rg_all = blockIdx.x / splits;
  const int sp = blockIdx.x % splits;
  int s = 0;  // the matrix this workgroup's row group belongs to (uniform per workgroup)
  while (s + 1 < seg.count && rg_all >= seg.rg0[s + 1]) ++s;
  const int rg = rg_all - seg.rg0[s];
  const int N = seg.n[s];
  const uint8_t *__restrict__ w = seg.w[s];
  const uint16_t *__restrict__ scale = seg.scale[s];
  uint16_t *__restrict__ y = seg.y[s];
  const int kb = sp * Kc;
  const int klen = min(K - kb, Kc);  // multiple of 16
  const int kpad = (klen + kIterK - 1) / kIterK * kIterK;
  const int row_bytes = kpad * 2 + 16;  // +16 spreads the 16 rows one MFMA operand load touches over all banks
  uint8_t *xs = lds;
  uint8_t *tile = lds + M * row_bytes + wave * kTileBytes;
  const int n0 = (rg * S + wave) * 16;

  // Load mapping: instruction j reads rows n0 + 4j + lane/16, bytes (lane%16)*16
  // of the iteration's 256-byte window. Rows past N read the last row.
  const int lrow = lane >> 4;
  const int lcol = (lane & 15) * kPieceBytes;
  const uint8_t *wr[kLoads];
#pragma unroll
  for (int j = 0; j < kLoads; ++j)
    wr[j] = w + static_cast<size_t>(min(n0 + j * kRowsPerLoad + lrow, N - 1)) * K + kb + lcol;

  // Two register stages: iterations it+1 and it+2 are in flight while it is
  // multiplied. A piece that starts at or past the slice end reads as zero
  // (the slice length is a multiple of 16).
  u32x4 va[kLoads], vb[kLoads];
  auto load = [&](u32x4(&v)[kLoads], int it) {
    const bool ok = it * kIterK + lcol < klen;
#pragma unroll
    for (int j = 0; j < kLoads; ++j)
      v[j] = ok ? __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(wr[j] + it * kIterK))
                : u32x4{0u, 0u, 0u, 0u};
  };
  const int n_iter = kpad / kIterK;
  load(va, 0);
  if (n_iter > 1) load(vb, 1);

  // Stage x[0:M, kb:kb+kpad) in LDS (zero past the slice end) while the first
  // weight loads are in flight.
  const int vec_per_row = kpad / 8;
  for (int v = threadIdx.x; v < M * vec_per_row; v += blockDim.x) {
    const int m = v / vec_per_row;
    const int kk = (v - m * vec_per_row) * 8;
    u32x4 val = u32x4{0u, 0u, 0u, 0u};
    if (kk < klen) val = *reinterpret_cast<const u32x4 *>(x + (static_cast<size_t>(m) * K + kb + kk) * 2);
    *reinterpret_cast<u32x4 *>(xs + m * row_bytes + kk * 2) = val;
  }
  __syncthreads();

  const uint8_t *brow[MB];
#pragma unroll
  for (int b = 0; b < MB; ++b) brow[b] = xs + min(b * 16 + r, M - 1) * row_bytes;
  f32x4 acc[MB];
#pragma unroll
  for (int b = 0; b < MB; ++b) acc[b] = f32x4{0.f, 0.f, 0.f, 0.f};

  // One iteration: registers -> wave tile (row-contiguous), then MFMA
  // operands read back in the MFMA layout: lane (r, g) takes row r, bytes
  // s*64 + g*16 .. +15 of the window for step s.
  auto multiply = [&](const u32x4(&v)[kLoads], int it) {
#pragma unroll
    for (int j = 0; j < kLoads; ++j)
      *reinterpret_cast<u32x4 *>(tile + (j * kRowsPerLoad + lrow) * kTileRow + lcol) = v[j];
    // The tile is written and read back by different lanes of this wave:
    // order the LDS writes before the reads explicitly.
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (int st = 0; st < kSteps; ++st) {
      const u32x4 a = *reinterpret_cast<const u32x4 *>(tile + r * kTileRow + st * kStepBytes + g * kPieceBytes);
      bf16x8 a_lo, a_hi;
      fp8x16_to_bf16(a, a_lo, a_hi);
      const int kk = it * kIterK + st * kStepBytes + g * kPieceBytes;
#pragma unroll
      for (int b = 0; b < MB; ++b) {
        const u32x4 *bp = reinterpret_cast<const u32x4 *>(brow[b] + kk * 2);
        acc[b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a_lo, as_bf16x8(bp[0]), acc[b], 0, 0, 0);
        acc[b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a_hi, as_bf16x8(bp[1]), acc[b], 0, 0, 0);
      }
    }
    // Every lane's reads of this tile come before the next iteration overwrites it.
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  };
  for (int it = 0; it < n_iter; it += 2) {
    multiply(va, it);
    if (it + 2 < n_iter) load(va, it + 2);
    if (it + 1 < n_iter) {
      multiply(vb, it + 1);
      if (it + 3 < n_iter) load(vb, it + 3);
    }
  }

  // Lane l holds rows n0 + 4*(l/16) + i, column b*16 + l%16.
  const int nb = n0 + 4 * g;
  if (part == nullptr) {  // one slice and no epilogue: the kernel writes y itself
#pragma unroll
    for (int b = 0; b < MB; ++b) {
      const int m = b * 16 + r;
      if (m >= M) continue;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (nb + i < N) {
          const float sc = __uint_as_float(static_cast<uint32_t>(scale[nb + i]) << 16);
          y[static_cast<size_t>(m) * N + nb + i] = f32_to_bf16_bits(acc[b][i] * sc);
        }
    }
    return;
  }
  float *__restrict__ pseg = part + seg.part0[s];
#pragma unroll
  for (int b = 0; b < MB; ++b) {
    const int m = b * 16 + r;
    if (m >= M) continue;
    float *dst = pseg + (static_cast<size_t>(sp) * M + m) * N;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (nb + i < N) dst[nb + i] = acc[b][i];
  }
}

// y_s[i] = bf16(scale_s[i % n_s] * sum over slices of part_s[slice][i]),
// summed in slice order. Blocks [rb0[s], rb0[s+1]) reduce matrix s; each
// thread owns kReduceVec consecutive outputs and keeps up to kReduceBatch
// independent loads in flight.
//
// Epilogues fold the operation that consumes the output into the reduce, with
// the rounding of that operation run on its own in bf16 (each value rounded to
// bf16 where the separate operation would round it):
//   kFp8EpilogueSwiglu (two matrices of equal n, gate then up):
//     y_0[i] = bf16(bf16(silu(g)) * u), g = bf16(gate), u = bf16(up);
//   kFp8EpilogueResidual (one matrix): y_0[i] = bf16(residual[i] + bf16(...)).
constexpr int kReduceVec = 4;
constexpr int kReduceBatch = 8;
constexpr int kReduceThreads = 256;
// LDS the reduce asks for and never touches: one allocation granule. A ring
// copy running beside a streamed decode holds its CUs' whole LDS (a small
// zero-copy grid), so with any LDS request the reduce's workgroups stay off
// those CUs. A workgroup that does share a CU with the copy queues behind the
// copy's outstanding host reads: in a streamed 70B decode the SwiGLU reduce
// took 45 us (median) against 5 us alone, the q/k/v reduce 26 against 5.
constexpr unsigned kReduceLdsToken = 512;

__device__ __forceinline__ float bf16_bits_to_f32(uint16_t b) { return __uint_as_float(static_cast<uint32_t>(b) << 16); }

// Sum over slices of kReduceVec consecutive partials starting at i0 (fewer at the end of MN).
__device__ __forceinline__ void sum_slices(const float *__restrict__ p, int64_t MN, int64_t i0, int splits,
                                           float (&acc)[kReduceVec]) {
#pragma unroll
  for (int e = 0; e < kReduceVec; ++e) acc[e] = 0.f;
  if (MN % kReduceVec == 0) {
    for (int p0 = 0; p0 < splits; p0 += kReduceBatch) {
      f32x4 v[kReduceBatch];
#pragma unroll
      for (int j = 0; j < kReduceBatch; ++j)
        v[j] = p0 + j < splits ? *reinterpret_cast<const f32x4 *>(p + (p0 + j) * MN + i0)
                               : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j = 0; j < kReduceBatch; ++j)
#pragma unroll
        for (int e = 0; e < kReduceVec; ++e) acc[e] += v[j][e];
    }
  } else {
    for (int q = 0; q < splits; ++q)
      for (int e = 0; e < kReduceVec; ++e)
        if (i0 + e < MN) acc[e] += p[q * MN + i0 + e];
  }
}

__global__ __launch_bounds__(kReduceThreads) void fp8_linear_reduce_kernel(const float *__restrict__ part,
                                                                           SegTable seg, int M, int splits,
                                                                           int epilogue,
                                                                           const uint16_t *__restrict__ residual) {
  int s = 0;
  while (s + 1 < seg.count && static_cast<int>(blockIdx.x) >= seg.rb0[s + 1]) ++s;
  const int N = seg.n[s];
  const int64_t MN = static_cast<int64_t>(M) * N;
  const int64_t i0 = (static_cast<int64_t>(blockIdx.x - seg.rb0[s]) * blockDim.x + threadIdx.x) * kReduceVec;
  if (i0 >= MN) return;
  const uint16_t *__restrict__ scale = seg.scale[s];
  uint16_t *__restrict__ y = seg.y[s];
  float acc[kReduceVec];
  sum_slices(part + seg.part0[s], MN, i0, splits, acc);
  if (epilogue == kFp8EpilogueSwiglu) {  // s is 0: the gate; the up matrix is segment 1, same shape
    float up[kReduceVec];
    sum_slices(part + seg.part0[1], MN, i0, splits, up);
    const uint16_t *__restrict__ scale_up = seg.scale[1];
#pragma unroll
    for (int e = 0; e < kReduceVec; ++e) {
      const int64_t i = i0 + e;
      if (i < MN) {
        const float g = bf16_bits_to_f32(f32_to_bf16_bits(acc[e] * bf16_bits_to_f32(scale[i % N])));
        const float u = bf16_bits_to_f32(f32_to_bf16_bits(up[e] * bf16_bits_to_f32(scale_up[i % N])));
        const float act = bf16_bits_to_f32(f32_to_bf16_bits(g / (1.0f + expf(-g))));
        y[i] = f32_to_bf16_bits(act * u);
      }
    }
    return;
  }
#pragma unroll
  for (int e = 0; e < kReduceVec; ++e) {
    const int64_t i = i0 + e;
    if (i < MN) {
      const uint16_t out = f32_to_bf16_bits(acc[e] * bf16_bits_to_f32(scale[i % N]));
      y[i] = epilogue == kFp8EpilogueResidual
                 ? f32_to_bf16_bits(bf16_bits_to_f32(residual[i]) + bf16_bits_to_f32(out))
                 : out;
    }
  }
}

SegTable seg_table(const Fp8LinearLaunch &p) {
  SegTable t{};
  t.count = p.group;
  const int64_t rows = p.prefill ? kPTileN : 16 * static_cast<int64_t>(p.waves);
  int rg = 0, rb = 0;
  int64_t off = 0;
  for (int s = 0; s < p.group; ++s) {
    t.w[s] = static_cast<const uint8_t *>(p.w[s]);
    t.scale[s] = static_cast<const uint16_t *>(p.scale[s]);
    t.y[s] = static_cast<uint16_t *>(p.y[s]);
    t.n[s] = static_cast<int>(p.n[s]);
    t.rg0[s] = rg;
    t.part0[s] = off;
    t.rb0[s] = rb;
    rg += static_cast<int>((p.n[s] + rows - 1) / rows);
    off += static_cast<int64_t>(p.splits) * p.m * p.n[s];
    rb += static_cast<int>((p.m * p.n[s] + kReduceVec * kReduceThreads - 1) / (kReduceVec * kReduceThreads));
  }
  t.rg0[p.group] = rg;
  t.rb0[p.group] = rb;
  return t;
}

// ---- prefill: inputs of more than kFp8LinearMaxRows rows -------------------
//
// Many activation rows make the layer a compute-bound GEMM. This is a tiled
// MFMA GEMM that still reads the weights as fp8 and widens them in registers
// (no bf16 copy of the weights is ever written).
//
// Workgroup tile: 128 output channels x 128 activation rows, K in steps of 64.
// Each step's tiles go straight from global memory into an S-stage LDS ring
// with global_load_lds_dwordx4 (no register staging): the activation tile as
// 128 rows of 128 bytes, then the weight tile as 128 rows of 64 bytes. Each
// load instruction writes 1 KB of LDS, lane l at +16 l, so the layout is
// chosen by which global chunk each lane fetches:
//   activation row R, 16-byte chunk c (k = 8c..8c+7) at slot c ^ rot3(R & 7),
//     rot3(v) = (v & 3) << 1 | v >> 2 (a rotation of the row's low three bits),
//   weight row R,     16-byte chunk c (k = 16c..16c+15) at slot c ^ ((R >> 1) & 3).
// Both keep the MFMA operand reads below (ds_read_b128, 1 KB per wave) free
// of bank conflicts on gfx950: 6 LDS cycles per read, measured with the
// SQ_LDS_BANK_CONFLICT counter. The plain c ^ (R & 7) for the activations
// costs 8, two of them bank-conflict cycles.
//
// k permutation within a step (any one that both operands share gives the
// same sum): lane group g feeds k = 16g + 8kb + (0..7) to the kb-th of the
// step's two MFMAs, so one 16-byte weight read per lane covers both MFMAs.
//
// Two launch shapes, chosen by the planner (measured on the 70B projection
// shapes at 512 rows):
//   * more tiles than CUs: 4 waves (2 x 2, 64 x 64 each), 2 stages (48 KB
//     LDS, three workgroups per CU);
//   * at most one tile per CU: 8 waves (2 x 4, 64 x 32 each), 4 stages
//     (96 KB, one workgroup per CU), so two waves share each SIMD; waves 0-3
//     issue the loads (all eight issuing them measured slower, by 5% to 50%
//     over runs).
// Both accumulate every output over the same MFMA sequence, so they give
// identical results.
//
// Rows past M or N read the last valid row (their products land in outputs
// that are never stored). A K that is not a multiple of 64 ends in a partial
// step: its loads past K are clamped into the row and both operands are
// zeroed for the lane groups past K.
//
// Block order: the hardware hands workgroup b to XCD b % xcds. The m-tiles of
// one n-tile get consecutive slots on one XCD, so each weight tile comes from
// HBM once and from that XCD's L2 for the other m-tiles.
constexpr int kPTileK = 64;
constexpr int kPXStage = kPTileM * kPTileK * 2;      // 16 KiB activation tile
constexpr int kPWStage = kPTileN * kPTileK;          // 8 KiB weight tile
constexpr int kPStage = kPXStage + kPWStage;
constexpr int kPLoadsPerWave = 6;                    // load instructions per loading wave and step

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(3))) void lds_void;

__device__ __forceinline__ bf16x8 fp8x8_to_bf16(uint32_t w0, uint32_t w1) {
  const bf16x2 p0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w0, 1.0f, false);
  const bf16x2 p1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w0, 1.0f, true);
  const bf16x2 p2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w1, 1.0f, false);
  const bf16x2 p3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w1, 1.0f, true);
  return join8(p0, p1, p2, p3);
}

// Activation-tile swizzle: rotate a row's low three bits (see the layout above).
__device__ __forceinline__ int rot3(int v) { return ((v & 3) << 1) | ((v >> 2) & 1); }

// s_waitcnt vmcnt(n) (expcnt and lgkmcnt left free); n is a constant at every call.
__device__ __forceinline__ void wait_vmcnt(int n) {
  switch (n) {
    case 0: __builtin_amdgcn_s_waitcnt(0x0f70); break;
    case 6: __builtin_amdgcn_s_waitcnt(0x0f76); break;
    case 12: __builtin_amdgcn_s_waitcnt(0x0f7c); break;
    default: __builtin_amdgcn_s_waitcnt(0x0f70); break;
  }
}

// Workgroup barrier that also keeps the compiler from moving memory accesses
// across it; the LDS ring's ordering is carried by vmcnt waits and this.
__device__ __forceinline__ void ring_barrier() {
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's LDS reads are done
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// seg.rg0 holds each matrix's first n-tile (tiles of kPTileN output channels).
// SADDR: the activations and every weight matrix are under 2 GiB, so each load
// takes a scalar base (the matrix plus the step's K offset) and a per-lane
// 32-bit offset, and the loading wave's LDS address is scalar arithmetic: the
// per-step address work leaves the vector ALU (about 3% per layer, measured).
template <int WAVES, int S, bool SADDR>
__global__ __launch_bounds__(WAVES * 64) void fp8_prefill_kernel(const uint8_t *__restrict__ x, SegTable seg, int M,
                                                                 int K, int m_tiles, int n_tiles, int xcds) {
  static_assert(WAVES == 4 || WAVES == 8, "4 or 8 waves");
  constexpr int JT = 16 / WAVES;             // 16-row activation tiles per wave
  constexpr int WROWS = 16 * JT;             // activation rows per wave
  __shared__ __align__(1024) uint8_t lds[S * kPStage];
  const int xcd = blockIdx.x % xcds;
  const int slot = blockIdx.x / xcds;
  const int nt = (slot / m_tiles) * xcds + xcd;
  const int mt = slot % m_tiles;
  if (nt >= n_tiles) return;  // the last round of n-tiles does not fill every XCD
  int s = 0;
  while (s + 1 < seg.count && nt >= seg.rg0[s + 1]) ++s;
  const int N = seg.n[s];
  const uint8_t *__restrict__ w = seg.w[s];
  const int n_base = (nt - seg.rg0[s]) * kPTileN;
  const int m_base = mt * kPTileM;

  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int r = lane & 15;
  const int g = lane >> 4;
  const int wn = wave & 1;
  const int wm = wave >> 1;
  const bool loads = WAVES == 4 || wave < 4;
  const int lw = __builtin_amdgcn_readfirstlane(wave & 3);  // uniform: LDS destinations stay scalar

  // This lane's load sources: activation rows (lw*4 + t)*8 + lane/8, weight
  // rows (lw*2 + t)*16 + lane/4, at the chunk the swizzle assigns.
  const int xc = ((lane & 7) ^ rot3(lane >> 3)) * 8;        // k offset (elements) within a step
  const int wc = ((lane & 3) ^ ((lane >> 3) & 3)) * 16;     // k offset (bytes) within a step
  const uint8_t *xrow[4];
  const uint8_t *wrow[2];
  uint32_t xoff[4], woff[2];  // SADDR: byte offsets of this lane's chunk in step 0
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const int gm = min(m_base + (lw * 4 + t) * 8 + (lane >> 3), M - 1);
    xrow[t] = x + static_cast<size_t>(gm) * K * 2;
    xoff[t] = static_cast<uint32_t>((static_cast<size_t>(gm) * K + xc) * 2);
  }
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int gn = min(n_base + (lw * 2 + t) * 16 + (lane >> 2), N - 1);
    wrow[t] = w + static_cast<size_t>(gn) * K;
    woff[t] = static_cast<uint32_t>(static_cast<size_t>(gn) * K + wc);
  }
  const int full = K / kPTileK;                 // whole steps
  const int tail = K % kPTileK;                 // k values of a final partial step, a multiple of 16
  const int steps = full + (tail ? 1 : 0);
  auto issue = [&](int st) {
    uint8_t *base = lds + (st % S) * kPStage;
    if (SADDR && st < full) {  // whole step: scalar base, per-lane offsets fixed for the whole kernel
      const uint8_t *xb = x + static_cast<size_t>(st) * kPTileK * 2;
      const uint8_t *wb = w + static_cast<size_t>(st) * kPTileK;
#pragma unroll
      for (int t = 0; t < 4; ++t)
        __builtin_amdgcn_global_load_lds(xb + xoff[t], (lds_void *)(base + (lw * 4 + t) * 1024), 16, 0, 0);
#pragma unroll
      for (int t = 0; t < 2; ++t)
        __builtin_amdgcn_global_load_lds(wb + woff[t], (lds_void *)(base + kPXStage + (lw * 2 + t) * 1024), 16, 0,
                                         0);
      return;
    }
    // the clamps only bind in a partial step (a whole step ends at K - 8 and K - 16)
    const int kx = min(st * kPTileK + xc, K - 8);
    const int kw = min(st * kPTileK + wc, K - 16);
    if (SADDR) {  // the same 32-bit offsets, moved by the clamped k
#pragma unroll
      for (int t = 0; t < 4; ++t)
        __builtin_amdgcn_global_load_lds(x + (xoff[t] + static_cast<uint32_t>(kx - xc) * 2),
                                         (lds_void *)(base + (lw * 4 + t) * 1024), 16, 0, 0);
#pragma unroll
      for (int t = 0; t < 2; ++t)
        __builtin_amdgcn_global_load_lds(w + (woff[t] + static_cast<uint32_t>(kw - wc)),
                                         (lds_void *)(base + kPXStage + (lw * 2 + t) * 1024), 16, 0, 0);
      return;
    }
#pragma unroll
    for (int t = 0; t < 4; ++t)
      __builtin_amdgcn_global_load_lds(xrow[t] + static_cast<size_t>(kx) * 2,
                                       (lds_void *)(base + (lw * 4 + t) * 1024), 16, 0, 0);
#pragma unroll
    for (int t = 0; t < 2; ++t)
      __builtin_amdgcn_global_load_lds(wrow[t] + kw, (lds_void *)(base + kPXStage + (lw * 2 + t) * 1024), 16, 0,
                                       0);
  };

  int aoff[4], boff0[JT], boff1[JT];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int R = wn * 64 + i * 16 + r;
    aoff[i] = kPXStage + R * kPTileK + ((g ^ ((R >> 1) & 3)) << 4);
  }
#pragma unroll
  for (int j = 0; j < JT; ++j) {
    const int R = wm * WROWS + j * 16 + r;
    boff0[j] = R * 128 + (((2 * g) ^ rot3(R & 7)) << 4);
    boff1[j] = R * 128 + (((2 * g + 1) ^ rot3(R & 7)) << 4);
  }

  f32x4 acc[4][JT];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < JT; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  if (loads) {
#pragma unroll
    for (int st = 0; st < S - 1; ++st)
      if (st < steps) issue(st);
  }
  // One step: this wave's loads of step st are in LDS once at most the later
  // steps' loads are outstanding; the barrier then covers every loading wave,
  // and every wave has finished reading the buffer the next loads overwrite.
  // `partial` (the final step of a K that is not a multiple of 64) zeroes both
  // operands of the lane groups past K.
  auto step = [&](int st, bool partial) {
    if (loads) {
      if (st + S - 2 < steps)
        wait_vmcnt((S - 2) * kPLoadsPerWave);
      else
        wait_vmcnt(0);
    }
    ring_barrier();
    if (loads && st + S - 1 < steps) issue(st + S - 1);
    const uint8_t *sb = lds + (st % S) * kPStage;
    u32x4 A[4], B0[JT], B1[JT];
#pragma unroll
    for (int i = 0; i < 4; ++i) A[i] = *reinterpret_cast<const u32x4 *>(sb + aoff[i]);
#pragma unroll
    for (int j = 0; j < JT; ++j) {
      B0[j] = *reinterpret_cast<const u32x4 *>(sb + boff0[j]);
      B1[j] = *reinterpret_cast<const u32x4 *>(sb + boff1[j]);
    }
    if (partial && 16 * g >= tail) {
#pragma unroll
      for (int i = 0; i < 4; ++i) A[i] = u32x4{0u, 0u, 0u, 0u};
#pragma unroll
      for (int j = 0; j < JT; ++j) B0[j] = B1[j] = u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const bf16x8 a0 = fp8x8_to_bf16(A[i][0], A[i][1]);
      const bf16x8 a1 = fp8x8_to_bf16(A[i][2], A[i][3]);
#pragma unroll
      for (int j = 0; j < JT; ++j) {
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0, as_bf16x8(B0[j]), acc[i][j], 0, 0, 0);
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, as_bf16x8(B1[j]), acc[i][j], 0, 0, 0);
      }
    }
  };
  for (int st = 0; st < full; ++st) step(st, false);
  if (tail) step(full, true);

  // lane holds D rows (output channels) 4g..4g+3 of column (activation row) r of every tile
  const uint16_t *__restrict__ scale = seg.scale[s];
  uint16_t *__restrict__ y = seg.y[s];
  const bool vec = (N & 3) == 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int nb = n_base + wn * 64 + i * 16 + 4 * g;
    float sc[4];
#pragma unroll
    for (int v = 0; v < 4; ++v) sc[v] = nb + v < N ? __uint_as_float(static_cast<uint32_t>(scale[nb + v]) << 16) : 0.f;
#pragma unroll
    for (int j = 0; j < JT; ++j) {
      const int m = m_base + wm * WROWS + j * 16 + r;
      if (m >= M) continue;
      uint16_t *dst = y + static_cast<size_t>(m) * N + nb;
      if (vec && nb + 3 < N) {
        const uint32_t lo = f32_to_bf16_bits(acc[i][j][0] * sc[0]) |
                            (static_cast<uint32_t>(f32_to_bf16_bits(acc[i][j][1] * sc[1])) << 16);
        const uint32_t hi = f32_to_bf16_bits(acc[i][j][2] * sc[2]) |
                            (static_cast<uint32_t>(f32_to_bf16_bits(acc[i][j][3] * sc[3])) << 16);
        *reinterpret_cast<u32x2 *>(dst) = u32x2{lo, hi};
      } else {
#pragma unroll
        for (int v = 0; v < 4; ++v)
          if (nb + v < N) dst[v] = f32_to_bf16_bits(acc[i][j][v] * sc[v]);
      }
    }
  }
}

// ---- measurement: the sustained MFMA rate -------------------------------
//
// Each wave keeps 16 independent accumulators and cycles through 8 operand
// pairs of random bf16 values (finite, magnitude 0.5 to 4, from a hash of the
// lane), so the operands change from one MFMA to the next as in a GEMM; the
// MFMA pipe runs at a lower clock on changing data than on constant data.
// Writes nothing: sink is written only if the sum equals a fixed sentinel.
__device__ __forceinline__ uint32_t probe_hash(uint32_t x) {
  x ^= x >> 16;
  x *= 0x7feb352du;
  x ^= x >> 15;
  x *= 0x846ca68bu;
  x ^= x >> 16;
  return x;
}

__global__ __launch_bounds__(256) void mfma_probe_kernel(float *sink, int iters) {
  const uint32_t id = blockIdx.x * 256u + threadIdx.x;
  u32x4 av[8], bv[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint32_t h = probe_hash(id * 64u + e * 8u + q);
      const uint32_t h2 = probe_hash(h);
      // two bf16 per dword: sign, exponent 126..129, 7 mantissa bits
      auto bf = [](uint32_t r) { return ((r & 1u) << 15) | ((126u + ((r >> 1) & 3u)) << 7) | ((r >> 3) & 0x7fu); };
      av[e][q] = bf(h) | (bf(h >> 10) << 16);
      bv[e][q] = bf(h2) | (bf(h2 >> 10) << 16);
    }
  }
  f32x4 acc[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int i = 0; i < 16; ++i)
        acc[i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(av[(i + h) & 7]), as_bf16x8(bv[(3 * i + h) & 7]),
                                                         acc[i], 0, 0, 0);
  }
  float sum = 0.f;
#pragma unroll
  for (int i = 0; i < 16; ++i) sum += acc[i][0] + acc[i][1] + acc[i][2] + acc[i][3];
  if (sum == 1234.5f) sink[0] = sum;
}

// The same probe on v_mfma_f32_32x32x16_bf16 (32768 flops each): 8
// independent accumulators per wave, 16 MFMAs per iteration, so an iteration
// has the flops of the 16 x 16 probe's. It reads half the operand registers
// per flop, and on changing data it sustains a higher rate.
__global__ __launch_bounds__(256) void mfma_probe_32x32_kernel(float *sink, int iters) {
  const uint32_t id = blockIdx.x * 256u + threadIdx.x;
  u32x4 av[8], bv[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint32_t h = probe_hash(id * 64u + e * 8u + q);
      const uint32_t h2 = probe_hash(h);
      auto bf = [](uint32_t r) { return ((r & 1u) << 15) | ((126u + ((r >> 1) & 3u)) << 7) | ((r >> 3) & 0x7fu); };
      av[e][q] = bf(h) | (bf(h >> 10) << 16);
      bv[e][q] = bf(h2) | (bf(h2 >> 10) << 16);
    }
  }
  f32x16 acc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[i][e] = 0.f;
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int i = 0; i < 8; ++i)
        acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(av[(i + h) & 7]), as_bf16x8(bv[(3 * i + h) & 7]),
                                                         acc[i], 0, 0, 0);
  }
  float sum = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int e = 0; e < 16; ++e) sum += acc[i][e];
  if (sum == 1234.5f) sink[0] = sum;
}

template <int MB>
hipError_t launch_mb(const Fp8LinearLaunch &p, hipStream_t stream) {
  const SegTable seg = seg_table(p);
  const bool reduce = p.workspace_bytes > 0;  // split K, or an epilogue: partials, then the reduce kernel
  hipLaunchKernelGGL((fp8_linear_kernel<MB>), dim3(static_cast<unsigned>(p.grid)), dim3(p.waves * kWave),
                     p.lds_bytes, stream, static_cast<const uint8_t *>(p.x), seg,
                     reduce ? static_cast<float *>(p.workspace) : nullptr, static_cast<int>(p.m), static_cast<int>(p.k),
                     static_cast<int>(p.kc), p.splits);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess || !reduce) return err;
  // the SwiGLU epilogue writes one output per gate/up pair: the gate's blocks only
  const int blocks = p.epilogue == kFp8EpilogueSwiglu ? seg.rb0[1] : seg.rb0[p.group];
  hipLaunchKernelGGL(fp8_linear_reduce_kernel, dim3(static_cast<unsigned>(blocks)), dim3(kReduceThreads),
                     kReduceLdsToken, stream, static_cast<const float *>(p.workspace), seg, static_cast<int>(p.m),
                     p.splits, p.epilogue, static_cast<const uint16_t *>(p.residual));
  return hipGetLastError();
}

}  // namespace

Fp8LinearLaunch plan_fp8_linear(int64_t m, const int64_t *n, int group, int64_t k, int cus, int xcds, int waves,
                                int kc_override, int epilogue) {
  Fp8LinearLaunch p{};
  p.epilogue = epilogue;
  p.m = m;
  p.k = k;
  p.group = group;
  for (int s = 0; s < group; ++s) {
    p.n[s] = n[s];
    p.n_total += n[s];
  }
  if (m > kFp8LinearMaxRows) {
    // prefill: one workgroup per 128 x 128 output tile, whole K, no workspace
    p.prefill = true;
    p.splits = 1;
    p.kc = k;
    p.xcds = std::max(1, xcds);
    const int64_t m_tiles = (m + kPTileM - 1) / kPTileM;
    int64_t n_tiles = 0;
    for (int s = 0; s < group; ++s) n_tiles += (n[s] + kPTileN - 1) / kPTileN;
    p.m_tiles = m_tiles;
    p.row_groups = n_tiles;
    p.grid = p.xcds * m_tiles * ((n_tiles + p.xcds - 1) / p.xcds);
    // at most one tile per CU: 8 waves (two per SIMD) and 4 LDS stages in one
    // workgroup; more tiles: 4 waves and 2 stages, three workgroups per CU
    p.waves = (waves == 4 || waves == 8) ? waves : (m_tiles * n_tiles <= cus ? 8 : 4);
    return p;
  }
  p.batch_blocks = m <= 16 ? 1 : (m <= 32 ? 2 : 4);
  // LDS: m activation rows of (2*Kc + 16) bytes plus one weight tile per
  // wave, within kFp8LinearMaxLds (less a margin for the kernel's own flag).
  const int64_t budget = static_cast<int64_t>(kFp8LinearMaxLds) - 256;
  const int64_t kblocks = std::max<int64_t>(1, (k + kIterK - 1) / kIterK);
  p.waves = waves ? waves : 8;
  int64_t min_slice_blocks = 4;
  if (!waves && !kc_override && ((p.n_total + 127) / 128) * std::max<int64_t>(1, kblocks / 4) < 2 * cus) {
    // Narrow outputs (the 1024-channel k/v projections of a 70B layer) give
    // fewer than two workgroups per CU at 8 waves and 4-iteration slices;
    // 4 waves and 2-iteration slices give four times as many (7.1 against
    // 9.3 us for 1024 x 8192 at 8 rows, measured).
    p.waves = 4;
    min_slice_blocks = 2;
  }
  while (p.waves > 1 && m * (2 * kIterK + 16) + static_cast<int64_t>(p.waves) * kTileBytes > budget) --p.waves;
  const int64_t rows = 16 * static_cast<int64_t>(p.waves);
  int64_t row_groups = 0;
  for (int s = 0; s < group; ++s) row_groups += (n[s] + rows - 1) / rows;
  const int64_t tiles = static_cast<int64_t>(p.waves) * kTileBytes;
  const int64_t x_budget = budget - tiles;
  const int64_t lds_blocks = std::max<int64_t>(1, ((x_budget / m - 16) / 2) / kIterK);
  int64_t kc_blocks;
  if (kc_override) {
    kc_blocks = std::max<int64_t>(1, kc_override / kIterK);
  } else {
    // Aim for at least 4 workgroups per CU, with slices of at least
    // min_slice_blocks iterations.
    const int64_t want_splits = std::max<int64_t>(1, (4 * static_cast<int64_t>(cus) + row_groups - 1) / row_groups);
    kc_blocks = std::max<int64_t>(std::min<int64_t>(min_slice_blocks, kblocks),
                                  (kblocks + want_splits - 1) / want_splits);
  }
  kc_blocks = std::min(std::min(kc_blocks, kblocks), lds_blocks);
  p.splits = static_cast<int>((kblocks + kc_blocks - 1) / kc_blocks);
  p.kc = kc_blocks * kIterK;
  p.grid = row_groups * p.splits;
  p.row_groups = row_groups;
  p.lds_bytes = static_cast<size_t>(m) * (2 * p.kc + 16) + static_cast<size_t>(tiles);
  // partials when K is split, and always under an epilogue (the reduce kernel applies it)
  p.workspace_bytes = p.splits > 1 || epilogue != kFp8EpilogueNone
                          ? static_cast<size_t>(p.splits) * m * p.n_total * sizeof(float)
                          : 0;
  return p;
}

hipError_t launch_mfma_probe(int shape, int workgroups, int iters, float *sink, hipStream_t stream) {
  if (shape == kMfmaProbe32x32x16)
    hipLaunchKernelGGL(mfma_probe_32x32_kernel, dim3(static_cast<unsigned>(workgroups)), dim3(256), 0, stream, sink,
                       iters);
  else
    hipLaunchKernelGGL(mfma_probe_kernel, dim3(static_cast<unsigned>(workgroups)), dim3(256), 0, stream, sink,
                       iters);
  return hipGetLastError();
}

hipError_t launch_fp8_linear(const Fp8LinearLaunch &p, hipStream_t stream) {
  if (p.prefill) {
    const SegTable seg = seg_table(p);
    // 32-bit load offsets reach every byte of x and of each weight matrix (kept under 2^31, so they read
    // the same whether the hardware widens the offset as signed or unsigned)
    bool small = static_cast<uint64_t>(p.m) * p.k * 2 < (uint64_t(1) << 31);
    for (int s = 0; s < p.group; ++s) small = small && static_cast<uint64_t>(p.n[s]) * p.k < (uint64_t(1) << 31);
    const auto *x = static_cast<const uint8_t *>(p.x);
    const int m = static_cast<int>(p.m), k = static_cast<int>(p.k), mt = static_cast<int>(p.m_tiles),
              nt = static_cast<int>(p.row_groups);
    const dim3 grid(static_cast<unsigned>(p.grid));
    if (p.waves == 8) {
      if (small)
        hipLaunchKernelGGL((fp8_prefill_kernel<8, 4, true>), grid, dim3(8 * kWave), 0, stream, x, seg, m, k, mt, nt,
                           p.xcds);
      else
        hipLaunchKernelGGL((fp8_prefill_kernel<8, 4, false>), grid, dim3(8 * kWave), 0, stream, x, seg, m, k, mt, nt,
                           p.xcds);
    } else {
      if (small)
        hipLaunchKernelGGL((fp8_prefill_kernel<4, 2, true>), grid, dim3(4 * kWave), 0, stream, x, seg, m, k, mt, nt,
                           p.xcds);
      else
        hipLaunchKernelGGL((fp8_prefill_kernel<4, 2, false>), grid, dim3(4 * kWave), 0, stream, x, seg, m, k, mt, nt,
                           p.xcds);
    }
    return hipGetLastError();
  }
  switch (p.batch_blocks) {
    case 1: return launch_mb<1>(p, stream);
    case 2: return launch_mb<2>(p, stream);
    default: return launch_mb<4>(p, stream);
  }
}

}  // namespace ftx
