/*
 * ftx.h - C ABI of the MI355X weight-streaming engine (libftx_hip.so).
 *
 * Plain pointers, sizes and opaque handles only; no C++ or torch types cross
 * this boundary. Every entry point returns an int status (FTX_OK on success);
 * ftx_last_error() returns the calling thread's message for the last failure.
 * Streams are hipStream_t values passed as void* (on the Python side they come
 * from torch.cuda.Stream.cuda_stream). All calls for one engine instance must
 * come from one host thread, as in the reference (core/transfer.py:42-46).
 *
 * Each declaration names the reference construct it replaces. The reference is
 * pure Python over PyTorch, so "replaces" means the PyTorch call the reference
 * makes on this path.
 */
#ifndef FTX_H_
#define FTX_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ------------------------------------------------------ */
#define FTX_OK 0
#define FTX_ERR_INVALID 1     /* bad argument (null, misaligned, out of range) */
#define FTX_ERR_HIP 2         /* the HIP runtime returned an error           */
#define FTX_ERR_OOM 3         /* host or device allocation failed            */
#define FTX_ERR_UNSUPPORTED 4 /* request not possible for this memory/device */

/* ---- copy engines ------------------------------------------------------ */
/* FTX_COPY_SDMA is hipMemcpyAsync. From page-locked host memory the runtime
 * hands the copy to an SDMA engine (traced as MEMORY_COPY_HOST_TO_DEVICE, no
 * kernel dispatch), so it uses no CUs and does not slow kernels running
 * beside it. Copies may be split over dedicated copy streams.
 * FTX_COPY_KERNEL is this library's zero-copy kernel: CUs load from mapped
 * host memory. It starts faster on small copies, but while it runs its
 * outstanding host reads delay the memory accesses of other kernels on the
 * same CUs, so FTX_COPY_AUTO keeps it to small chunks. */
#define FTX_COPY_SDMA 0   /* hipMemcpyAsync, optionally split over copy streams   */
#define FTX_COPY_KERNEL 1 /* zero-copy kernel: CUs read mapped pinned host memory */
#define FTX_COPY_AUTO 2   /* pageable source: FTX_COPY_STAGED; pinned: per chunk from ftx_set_copy_policy */
#define FTX_COPY_STAGED 3 /* pageable source staged through pinned buffers by a host thread pool */

/* ---- host arena flags -------------------------------------------------- */
#define FTX_ARENA_DEFAULT 0u
#define FTX_ARENA_COHERENT 1u      /* hipHostMallocCoherent (fine-grained)     */
#define FTX_ARENA_NONCOHERENT 2u   /* hipHostMallocNonCoherent (coarse-grained) */
#define FTX_ARENA_WRITECOMBINED 4u /* hipHostMallocWriteCombined              */
#define FTX_ARENA_NUMA_USER 8u     /* hipHostMallocNumaUser: pages follow the calling thread's NUMA policy */

/* ---- events ------------------------------------------------------------ */
#define FTX_EVENT_DEFAULT 0u /* no timing: cheapest record/wait */
#define FTX_EVENT_TIMING 1u  /* timing enabled (ftx_event_elapsed_ms) */
/* Only streams of this device wait on the event: recording it skips the
 * system-scope fence (cache writeback and invalidation for the host's view,
 * hipEventDisableSystemFence); device-scope ordering between the streams is
 * kept. Host waits still see it complete, but device writes before it are not
 * made visible to the host. For the ring's ready and slot-release events. */
#define FTX_EVENT_DEVICE_ONLY 2u

/* One scatter descriptor: dst[0:nbytes) = chunk[src_off : src_off+nbytes).
 * Replaces the per-tensor copies the reference makes when it places tensors
 * (allocation_block.py:179-186 pack; tensor_processors.py:685-742 move of
 * unmapped tensors; loaders.py:592-617 per-tensor .to()). */
typedef struct ftx_desc {
  uint64_t src_off; /* byte offset inside the streamed chunk */
  uint64_t dst;     /* device address of the destination     */
  uint64_t nbytes;  /* bytes to copy                         */
} ftx_desc;

/* Opaque scatter plan: descriptor table + per-tile work table resident in HBM. */
typedef struct ftx_scatter_plan ftx_scatter_plan;

/* ---- library / device -------------------------------------------------- */
const char *ftx_last_error(void);
int ftx_version(void);                 /* returns the ABI version number (not a status) */
/* Releases what the library holds for the process, while the HIP runtime is
 * still up: waits for every device, joins the staged engine's host threads,
 * frees its page-locked staging buffers and events, and destroys the copy
 * streams and events of split SDMA copies. Idempotent. Afterwards every call
 * that would start work or allocate returns FTX_ERR_UNSUPPORTED; calls that
 * release, wait on or query existing handles still work. Meant for process
 * exit, ahead of the runtime's own teardown. Replaces
 * CudaTransferRuntime.close (core/transfer.py:133-142): synchronize, then
 * refuse further work. */
int ftx_shutdown(void);
int ftx_device_count(int *count);
int ftx_set_device(int device);
int ftx_get_device(int *device);
int ftx_device_synchronize(void);
/* CU count and L2-domain (XCD) count of the current device, for launch shaping. */
int ftx_device_info(int *cu_count, int *xcd_count, size_t *total_mem);

/* ---- host arenas ---------------------------------------------------------
 * Replace HostPinner.pin in "torch" mode (host_pinning.py:374-400: a fresh
 * pinned copy via Tensor.pin_memory) with one page-locked, device-mapped arena
 * per packed block. */
int ftx_arena_alloc(size_t nbytes, unsigned flags, void **host);
int ftx_arena_free(void *host);
/* Stand in for HostPinRegistry.pin_in_place (host_pinning.py:206-265, the
 * cudaHostRegister(ptr, n, Portable) call at :257) and SHM pinning
 * (shm/flexible_shm.py:832-848): page-locking existing memory in place.
 * Refused in this build: the MI355X hosts it targets reject hipHostRegister,
 * and the failed call's error can surface in the next GPU call. So
 * ftx_arena_register returns FTX_ERR_UNSUPPORTED for every input without
 * calling the runtime, and ftx_arena_unregister (nothing is ever registered)
 * returns FTX_ERR_INVALID. Allocate blocks with ftx_arena_alloc instead;
 * pageable or shared-memory sources stream through FTX_COPY_STAGED. */
int ftx_arena_register(void *host, size_t nbytes, unsigned flags);
int ftx_arena_unregister(void *host);
/* Device-visible address of pinned host memory (zero-copy kernel source). */
int ftx_host_device_ptr(void *host, void **dev);

/* ---- device memory (ring slots when no torch allocator is in use) -------
 * Replace AllocationManager.create_max_block (allocation_block.py:260-280). */
int ftx_device_alloc(size_t nbytes, void **dev);
int ftx_device_free(void *dev);
int ftx_memset_async(void *dev, int value, size_t nbytes, void *stream);
int ftx_copy_d2h(void *dst_host, const void *src_dev, size_t nbytes, void *stream);

/* ---- streams and events --------------------------------------------------
 * Replace torch.cuda.Stream / Stream.record_event / Stream.wait_event /
 * Stream.synchronize as used by CudaTransferRuntime (core/transfer.py:49,
 * 69-70, 92, 97, 109, 116, 124-125, 20). Streams are created at default
 * priority. */
int ftx_stream_create(void **stream);
int ftx_stream_destroy(void *stream);
int ftx_stream_synchronize(void *stream);
int ftx_stream_query(void *stream, int *done);
int ftx_event_create(unsigned flags, void **event);
int ftx_event_destroy(void *event);
int ftx_event_record(void *event, void *stream);
/* Device timestamps for timing captured graphs: writes the GPU's constant-rate
 * wall clock into dev_slot (8 bytes of device memory) when the stream reaches
 * it. Captured in a graph it is a kernel node, so every replay writes a new
 * time. Replaces torch.cuda.Event(external=True).record() of the graph-replay
 * timing mode (offload_timing.py:319-352); ticks per millisecond come from
 * ftx_wall_clock_khz. */
int ftx_timestamp(void *dev_slot, void *stream);
int ftx_wall_clock_khz(int *khz);
int ftx_stream_wait_event(void *stream, void *event);
int ftx_event_query(void *event, int *done);
int ftx_event_synchronize(void *event);
int ftx_event_elapsed_ms(void *start, void *end, float *ms);

/* ---- host-to-device copy engines ------------------------------------------
 * Replace AllocationBlock.copy_to (allocation_block.py:104-106) and
 * RawBlockController.schedule_transfer (loaders.py:1064-1067), i.e.
 * gpu_view.copy_(pinned_block, non_blocking=True) on the transfer stream.
 * Stream-ordered on `stream`: work split over internal copy streams is forked
 * from and joined back into `stream`. `src` must be pinned host memory. */
int ftx_copy_h2d(void *dst, const void *src, size_t nbytes, int mode, void *stream);
/* A copy policy: how FTX_COPY_AUTO picks the engine per chunk and how the
 * engines run.
 *   kernel_max_bytes  chunks <= this go to the zero-copy kernel under AUTO;
 *   split_min_bytes   SDMA copies >= this are split over n_copy_streams;
 *   n_copy_streams    1..8 dedicated copy streams;
 *   kernel_grid       zero-copy kernel workgroups, 0..2^20 (0 = 64, enough to hold the link at
 *                     its peak). A grid of at most 16 reserves each CU it runs on: its
 *                     workgroups take the CU's whole LDS, so kernels that use LDS run on the
 *                     other CUs. */
typedef struct ftx_copy_policy {
  uint64_t kernel_max_bytes;
  uint64_t split_min_bytes;
  int32_t n_copy_streams;
  int32_t kernel_grid;
} ftx_copy_policy;
/* ftx_copy_h2d under a policy the caller owns. Each named offload manager
 * copies independently in the reference (offload_manager.py:2817-2850; each
 * controller's AllocationBlock.copy_to, allocation_block.py:104-106), so each
 * carries its own measured policy into every copy instead of changing the
 * process's. policy NULL is the library default below. */
int ftx_copy_h2d_policy(void *dst, const void *src, size_t nbytes, int mode, const ftx_copy_policy *policy,
                        void *stream);
/* The library default, used by ftx_copy_h2d (process-wide; 1 MiB kernel cut,
 * no SDMA split, grid 0 until set). */
int ftx_set_copy_policy(size_t kernel_max_bytes, size_t split_min_bytes, int n_copy_streams,
                        int kernel_grid);
int ftx_get_copy_policy(size_t *kernel_max_bytes, size_t *split_min_bytes, int *n_copy_streams,
                        int *kernel_grid);

/* ---- exponent-coded blocks -------------------------------------------------
 * No reference counterpart: the reference copies each label's packed block as
 * raw bytes (allocation_block.py:104-106). These entry points carry the same
 * block over the link encoded, and the GPU rebuilds the raw bytes exactly.
 * The block is read as little-endian 16-bit words (bf16 bit patterns):
 * sign and mantissa travel as one byte per word, the exponent as a 4-bit code
 * for the block's 15 most frequent exponents, and the others as escapes.
 * Blocks of bf16 weights from one distribution encode to about 0.75 of their
 * raw size; other contents may grow (compare sizes before using it).
 * ftx_expcode_encode: host only, no GPU. out NULL stores only the encoded size
 * in *out_bytes; otherwise the block is written to out (out_capacity bytes,
 * not overlapping raw). The format is exponent-coded block v1 ("FTXE").
 * ftx_expcode_raw_bytes: the raw size recorded in an encoded block's header.
 * ftx_expcode_decode_h2d: the host-to-device copy of an encoded block: src is
 * the encoded block in pinned, device-mapped host memory (src_bytes bytes,
 * 16-byte aligned), dst a 16-byte aligned device range of the raw size. A
 * zero-copy kernel reads src over the link and writes the raw bytes, ordered
 * on `stream`; policy->kernel_grid sets its workgroups (NULL or 0: 16), and a
 * grid of at most 16 reserves its CUs as the zero-copy copy does. The header
 * is read on the host at call time; the block must not change until the copy
 * has run. A dense block (version 2, ftx_expcode_encode_dense) is decoded by
 * the dense kernel's link variant, whose nibble reads follow each batch's rank
 * scans; ftx_expcode_raw_bytes reads either version. */
int ftx_expcode_encode(const void *raw, size_t nbytes, void *out, size_t out_capacity, size_t *out_bytes);
int ftx_expcode_raw_bytes(const void *src, size_t src_bytes, size_t *raw_bytes);
int ftx_expcode_decode_h2d(void *dst, const void *src, size_t src_bytes, const ftx_copy_policy *policy,
                           void *stream);
/* The same decode from an encoded block kept in device memory (src_bytes
 * bytes, 16-byte aligned) into dst (raw_bytes). The header stays on the
 * device: the caller states the raw size, and the kernel reads the table and
 * escape count when it runs (a block of another raw size writes nothing).
 * grid 0 runs eight workgroups per CU. Serves units kept encoded in HBM
 * (OffloadConfig.encode_resident_blocks). */
int ftx_expcode_decode_d2d(void *dst, const void *src, size_t src_bytes, size_t raw_bytes, int grid, void *stream);
/* Dense exponent-coded blocks (FTXE version 2), for units kept encoded in
 * device memory: 3-bit codes for a block's 7 most frequent exponents in three
 * bit planes, a 4-bit code for each other word's exponent among the next 15,
 * and a list for the rest; about 0.70 of the raw size for bf16 weights, against
 * 0.75 for version 1. A decoder ranks each escaped word among the group's
 * escapes, which costs a dependent read: cheap from HBM, so version 2 is decoded
 * only from device memory. Same contracts as ftx_expcode_encode and
 * ftx_expcode_decode_d2d, except that grid 0 runs sixteen workgroups per CU.
 * No reference counterpart. */
int ftx_expcode_encode_dense(const void *raw, size_t n, void *out, size_t capacity, size_t *out_bytes);
int ftx_expcode_decode_dense_d2d(void *dst, const void *src, size_t src_bytes, size_t raw_bytes, int grid,
                                 void *stream);

/* ---- staged copies from pageable host memory ------------------------------
 * Replace the reference's copy from pageable or shared-memory blocks that are
 * not page-locked (pinned_memory=False blocks, allocation_block.py:104-106 with
 * an unpinned source; FlexibleSharedMemory blocks without in-place
 * registration, shm/flexible_shm.py:832-848): FTX_COPY_STAGED copies the
 * source in pieces (ramping up to `piece_bytes`, 64 MiB by default) into
 * three page-locked staging buffers per device with `n_threads` host threads,
 * each piece then crossing the link by SDMA while the next one is copied. The call returns once the last piece is
 * enqueued; the source may be reused then. Staged copies are refused on a
 * capturing stream. ftx_host_memcpy is the same thread pool's parallel host
 * copy (no overlap allowed). n_threads 0 = half the host's cores, at most 8. */
int ftx_set_staging_policy(size_t piece_bytes, int n_threads);
int ftx_get_staging_policy(size_t *piece_bytes, int *n_threads);
int ftx_host_memcpy(void *dst, const void *src, size_t nbytes);

/* ---- batched scatter / unpack --------------------------------------------
 * No reference counterpart; it places a streamed chunk into many tensors in
 * one launch where the reference copies tensor by tensor (see ftx_desc).
 * A plan uploads descriptors once (device memory) and can be run any number
 * of times on any stream; tile_bytes 0 selects the default (8 KiB). */
int ftx_scatter_plan_create(const ftx_desc *descs, int n_desc, size_t tile_bytes,
                            ftx_scatter_plan **plan);
int ftx_scatter_plan_destroy(ftx_scatter_plan *plan);
int ftx_scatter_plan_info(const ftx_scatter_plan *plan, int *n_desc, int64_t *n_tiles,
                          uint64_t *total_bytes);
int ftx_scatter_run(const ftx_scatter_plan *plan, const void *chunk, void *stream);
/* One-shot form: stream-ordered upload of the table, launch, stream-ordered free. */
int ftx_scatter(const void *chunk, const ftx_desc *descs, int n_desc, void *stream);

/* ---- fp8-weight linear (the decode and prefill forward's GEMMs) ------------
 * No reference counterpart: the reference streams weights for whatever
 * nn.Linear the user's model holds. This replaces the forward of an fp8 linear
 * layer, F.linear(x, w.to(bfloat16)) * scale:
 *   y[i, j] = bf16(scale[j] * sum_k x[i, k] * w[j, k])
 * x: bf16 [m, k] contiguous, 16-byte aligned; w: float8 e4m3fn [n, k]
 * contiguous, 16-byte aligned; scale: bf16 [n]; y: bf16 [m, n] contiguous;
 * k a multiple of 16. The weights are widened to bf16 in registers and
 * multiplied on the MFMA units in fp32; no bf16 copy of them is written.
 * Up to 64 rows (decode) K is split over workgroups; each slice's partial
 * sums go to `workspace` (device memory of at least ftx_fp8_linear_workspace
 * bytes, 16-byte aligned; it may be NULL when that size is 0) and a second
 * kernel adds them in slice order, so results are deterministic for a given
 * launch shape. More rows (prefill) run a tiled GEMM (128 x 128 output tiles,
 * whole K per tile) that needs no workspace.
 * Calls that share a workspace must be ordered on one stream.
 * ftx_set_fp8_linear_config fixes the decode launch shape (0 = chosen per
 * call): waves (wavefronts per workgroup, 16 output rows each, 1..8) and
 * slice_k (K values per workgroup, a multiple of 256). For more than 64 rows
 * waves 4 or 8 fixes the prefill launch shape (4: two LDS stages; 8: four);
 * any other value lets the tile count choose. Every launch shape gives the
 * same results. */
int ftx_fp8_linear_workspace(int64_t m, int64_t n, int64_t k, size_t *bytes);
int ftx_fp8_linear(const void *x, const void *w, const void *scale, void *y, int64_t m, int64_t n, int64_t k,
                   void *workspace, size_t workspace_bytes, void *stream);
int ftx_set_fp8_linear_config(int waves, int slice_k);
/* Grouped form: `group` (1..4) weight matrices w[s] [n[s], k] with scales
 * scale[s] and outputs y[s] [m, n[s]] that share the input x, in one launch
 * (one reduce launch when K is split): a layer's q/k/v projections, or its
 * gate/up projections. Each y[s] equals what ftx_fp8_linear computes for that
 * matrix to within fp32 rounding (the K split may differ); results are
 * deterministic for a given group. Workspace sizes from
 * ftx_fp8_linear_group_workspace. */
int ftx_fp8_linear_group_workspace(int64_t m, const int64_t *n, int group, int64_t k, size_t *bytes);
int ftx_fp8_linear_group(const void *x, int group, const void *const *w, const void *const *scale, void *const *y,
                         const int64_t *n, int64_t m, int64_t k, void *workspace, size_t workspace_bytes,
                         void *stream);

/* Fused forms for decode batches (m <= 64): the reduce kernel that sums the
 * split-K partials also applies the operation that consumes the output, so it
 * is not a launch of its own. No counterpart in the reference, whose models
 * run these as separate PyTorch operations; each epilogue rounds to bf16
 * where those operations do.
 *   FTX_FP8_EPILOGUE_SWIGLU   group 2 (gate, up), n[0] == n[1]:
 *                             y = bf16(bf16(silu(g)) * u), g and u the bf16
 *                             outputs of the two matrices (F.silu(g) * u);
 *   FTX_FP8_EPILOGUE_RESIDUAL group 1: y = bf16(residual + bf16(out))
 *                             (residual + F.linear(...)); residual is bf16
 *                             [m, n] and may be y itself.
 * y is one bf16 [m, n[0]] output. Every call goes through the workspace
 * (ftx_fp8_linear_fused_workspace, non-zero). More than 64 rows, or an
 * epilogue of the wrong group shape, returns FTX_ERR_UNSUPPORTED or
 * FTX_ERR_INVALID before any operand is touched. */
#define FTX_FP8_EPILOGUE_NONE 0
#define FTX_FP8_EPILOGUE_SWIGLU 1
#define FTX_FP8_EPILOGUE_RESIDUAL 2
int ftx_fp8_linear_fused_workspace(int64_t m, const int64_t *n, int group, int64_t k, int epilogue, size_t *bytes);
int ftx_fp8_linear_fused(const void *x, int group, const void *const *w, const void *const *scale, void *y,
                         const int64_t *n, int64_t m, int64_t k, int epilogue, const void *residual, void *workspace,
                         size_t workspace_bytes, void *stream);

/* Bytes of the static scratch array behind ftx_fp8_linear_static (64 MiB per GPU). */
#define FTX_FP8_STATIC_SCRATCH_BYTES ((size_t)64 << 20)
/* No counterpart in the reference. For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): ftx_fp8_linear with its split-K partial sums in a static
 * device array of FTX_FP8_STATIC_SCRATCH_BYTES that each GPU the library runs
 * on holds until the process ends. Same operands, results and launch shape as
 * ftx_fp8_linear; allocates nothing (no hipMalloc, hipFree or allocating
 * library call). Returns FTX_ERR_UNSUPPORTED, before touching any operand,
 * when the call's partial sums (ftx_fp8_linear_workspace) exceed the array.
 * Every call on one GPU shares that GPU's array: calls that may overlap on one
 * GPU (unordered streams, other host threads) race and must be ordered, e.g.
 * on one stream. Every partial sum a call reads is written by that call
 * first, so nothing needs clearing between calls. */
int ftx_fp8_linear_static(const void *x, const void *w, const void *scale, void *y, int64_t m, int64_t n, int64_t k,
                          void *stream);

/* ---- checksums (size-independent parity checks on device data) ----------- */
/* Order-sensitive 64-bit checksum of nbytes at dev (FNV-1a over 8-byte lanes,
 * folded per 4 KiB block); result written to *out after stream sync. */
int ftx_checksum64(const void *dev, size_t nbytes, void *stream, uint64_t *out);

/* ---- measurement ----------------------------------------------------------
 * No reference counterpart. Reads nbytes at dev (16-byte aligned, a multiple
 * of 16) with `grid` workgroups of 256 lanes, eight 16-byte non-temporal loads
 * in flight per lane, and writes nothing (sink, 4 bytes of device memory, is
 * written only if the folded data equals a fixed sentinel): the plain HBM
 * read rate the HBM-bound kernels are measured against. */
int ftx_hbm_read_probe(const void *dev, size_t nbytes, void *sink, int grid, void *stream);
/* No reference counterpart. Runs `workgroups` workgroups of 4 waves, each
 * wave iters x 32 independent v_mfma_f32_16x16x32_bf16 (16384 flops each) on
 * random bf16 operands that change from one MFMA to the next, and writes
 * nothing (sink, 4 bytes of device memory, only on a fixed sentinel): the
 * sustained MFMA rate the compute-bound kernels are measured against. */
int ftx_mfma_probe(int workgroups, int iters, void *sink, void *stream);
/* No reference counterpart. ftx_mfma_probe on another MFMA shape:
 * FTX_MFMA_PROBE_16X16X32 (as above) or FTX_MFMA_PROBE_32X32X16 (each wave
 * iters x 16 independent v_mfma_f32_32x32x16_bf16 of 32768 flops, the same
 * flops per iteration). The better of the two is the measured ceiling. */
#define FTX_MFMA_PROBE_16X16X32 0
#define FTX_MFMA_PROBE_32X32X16 1
int ftx_mfma_probe_shape(int shape, int workgroups, int iters, void *sink, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* FTX_H_ */
