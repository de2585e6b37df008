/*
 * libmoegemm: MI355X (gfx950) grouped and single GEMM kernels behind a plain C ABI.
 *
 * This is the native boundary of the MoE expert-GEMM hot path.  The Python layer
 * (kernels/grouped_gemm.py and kernels/matmul.py of this project) keeps the reference's Python
 * signatures and calls these functions through ctypes; any other host language binds the same
 * symbols.  Conventions:
 *   - all matrix, table and stream arguments are plain device pointers / a hipStream_t as void*;
 *   - strides are in elements; dims tables are int32 (m, n, k) triples; pointer tables are int64
 *     device addresses, read by the kernel at run time (callers may rewrite them between calls);
 *   - a call performs exactly one kernel launch on `stream` (or none for an empty problem set),
 *     never allocates, copies or synchronizes, and is therefore capturable in a HIP graph;
 *   - the return value is MOEGEMM_OK or a negative error code; moegemm_last_error() returns the
 *     message of the most recent failure on the calling thread;
 *   - every launching call takes `b_stream` (0 or 1) just before `stream`: 1 issues the LDS-DMA
 *     kernels' B copies as non-temporal loads (streamed, evicted first from the caches), 0 as
 *     ordinary loads.  It changes no result, only speed, and which is faster depends on the
 *     workload (it is a tuning choice, like the tile config; the general kernel ignores it).  It
 *     has no counterpart in the reference's Triton launches, which take no cache policy.
 */
#ifndef MOEGEMM_H
#define MOEGEMM_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MOEGEMM_ABI_VERSION 9

#define MOEGEMM_OK 0
#define MOEGEMM_ERR_INVALID (-1)   /* bad shape, pointer, dtype or parameter (Python: ValueError) */
#define MOEGEMM_ERR_NO_KERNEL (-2) /* no compiled instantiation for the tile config (RuntimeError) */
#define MOEGEMM_ERR_LAUNCH (-3)    /* the HIP runtime rejected the launch (RuntimeError) */

#define MOEGEMM_DTYPE_F16 0
#define MOEGEMM_DTYPE_BF16 1
#define MOEGEMM_DTYPE_F32 2

#define MOEGEMM_PRECISION_IEEE 0 /* operands used as given */
#define MOEGEMM_PRECISION_TF32 1 /* fp32 operands rounded to a 10-bit mantissa (ties away) */

/* Size of the tile queue of the work-stealing launches (17 int32 counters, each in a 256-byte
 * block of its own; the buffer is 256-byte aligned). */
#define MOEGEMM_QUEUE_BYTES 4352

/* ABI version of the loaded library (MOEGEMM_ABI_VERSION when header and library agree). */
int moegemm_abi_version(void);

/* Message of the last failed call on this thread ("" if none). */
const char* moegemm_last_error(void);

/*
 * Compiled tile configurations.  Replaces the Triton config pools
 * (reference kernels/matmul.py:54-98 _MATMUL_CONFIG_POOL and kernels/grouped_gemm.py:41-64
 * _GROUPED_EXTRA_CONFIG_POOL): the Python candidate generators enumerate this table instead.
 * moegemm_kernel_info fills out7 = {block_m, block_n, block_k, num_warps (wave64 per
 * workgroup), num_stages (LDS stages), lds_bytes, waves_m}.
 */
int moegemm_kernel_count(int dtype);
int moegemm_kernel_info(int dtype, int index, int32_t* out7);

/*
 * Persistent grouped GEMM: for each problem e, C_e[m, n] = sum_k A_e[m, k] * B_e[k, n] with fp32
 * accumulation, stored in the operand dtype.  Replaces the two Triton kernels launched by
 * reference kernels/grouped_gemm.py:618-760 (launch_grouped):
 *   homogeneous != 0 -> _homogeneous_grouped_kernel_impl (kernels/grouped_gemm.py:321-397):
 *       every problem is (m, k) @ (k, n), all row-major contiguous; dims/strides may be NULL.
 *   homogeneous == 0 -> _generic_grouped_kernel_impl (kernels/grouped_gemm.py:399-482):
 *       per-problem dims [G,3] = (m, n, k) and strides [G,6] = (am, ak, bk, bn, cm, cn), the
 *       tables built at kernels/grouped_gemm.py:536-544; total_tiles = sum over problems of
 *       ceil(m/block_m) * ceil(n/block_n); m, n, k are ignored.
 * group_size_m is the GROUP_M traversal width inside each problem; grid_size is the persistent
 * grid (reference _grid_size, kernels/grouped_gemm.py:597-599); <= 0 means one workgroup per tile.
 * vector_layout != 0 promises that every problem is fp16/bf16 with unit inner strides, row
 * pitches and K, N multiples of 8 elements, C row pitch a multiple of 4, 16-byte aligned A/B and
 * 8-byte aligned C bases, A and C row pitches under 2^22 elements (256 rows under 2 GiB; any
 * number of rows) and B under 2 GiB: the launch then uses the LDS-DMA kernel.
 * Otherwise (or for fp32) the general kernel runs, which accepts any strides and alignment.
 */
int moegemm_grouped_gemm(const int64_t* a_ptrs, const int64_t* b_ptrs, const int64_t* c_ptrs,
                         const int32_t* dims, const int64_t* strides, int32_t problem_count,
                         int32_t m, int32_t n, int32_t k, int32_t homogeneous, int32_t total_tiles,
                         int32_t dtype, int32_t input_precision, int32_t block_m, int32_t block_n,
                         int32_t block_k, int32_t group_size_m, int32_t num_warps,
                         int32_t num_stages, int32_t grid_size, int32_t vector_layout, int32_t b_stream,
                         void* stream);

/*
 * moegemm_grouped_gemm with a work-stealing tile scheduler instead of the static one: the
 * "persistent tile scheduler over (expert, m-tile, n-tile)" of reference
 * kernels/grouped_gemm.py:321-482, whose programs take the fixed tiles pid, pid + grid, ...
 * (:346-353, :397, :481); here the tiles are drawn at run time.  When grid_size is a multiple of 8 each XCD owns a
 * contiguous eighth of the tiles (its workgroups take them from an atomic ticket counter) and a
 * workgroup whose XCD has none left steals from the other XCDs' counters; otherwise one counter
 * serves all.  `queue` is MOEGEMM_QUEUE_BYTES of device memory, zero before the first call; every
 * call leaves it zero, so it can be reused without clearing (and replayed in a captured graph).
 * Calls sharing a queue must not overlap (use one per stream).  Results are identical to
 * moegemm_grouped_gemm's (each tile is computed the same way by whichever workgroup takes it).
 */
int moegemm_grouped_gemm_stealing(const int64_t* a_ptrs, const int64_t* b_ptrs,
                                  const int64_t* c_ptrs, const int32_t* dims,
                                  const int64_t* strides, int32_t problem_count, int32_t m,
                                  int32_t n, int32_t k, int32_t homogeneous, int32_t total_tiles,
                                  int32_t dtype, int32_t input_precision, int32_t block_m,
                                  int32_t block_n, int32_t block_k, int32_t group_size_m,
                                  int32_t num_warps, int32_t num_stages, int32_t grid_size,
                                  int32_t vector_layout, void* queue, int32_t b_stream, void* stream);

/*
 * Packed Gate+Up projection with the SwiGLU activation fused into the epilogue: for each problem e
 * with B_e = [gate | up] of n = 2F columns (the packed W13 weights of reference
 * kernels/grouped_gemm.py:575-594 build_fused_gate_up_workspace), H_e[m, j] =
 * silu(sum_k A_e[m,k] B_e[k,j]) * sum_k A_e[m,k] B_e[k,F+j] for j < F, computed from the fp32
 * accumulators and stored in the operand dtype into H_e [M_e, F] (h_ptrs; in generic mode the
 * strides table's cm/cn are H's).  The reference keeps the activation outside its timed GEMM
 * (README.md:55-57) and has no such kernel; this is the next step of the path, timed as a
 * separate labelled variant.  Same tables, tile config and grid as moegemm_grouped_gemm; requires
 * fp16/bf16, vector_layout != 0, F a multiple of 8 and a tile with moegemm_kernel_swiglu() == 1.
 */
int moegemm_grouped_gemm_swiglu(const int64_t* a_ptrs, const int64_t* b_ptrs, const int64_t* h_ptrs,
                                const int32_t* dims, const int64_t* strides, int32_t problem_count,
                                int32_t m, int32_t n, int32_t k, int32_t homogeneous,
                                int32_t total_tiles, int32_t dtype, int32_t block_m,
                                int32_t block_n, int32_t block_k, int32_t group_size_m,
                                int32_t num_warps, int32_t num_stages, int32_t grid_size,
                                int32_t vector_layout, int32_t b_stream, void* stream);

/*
 * Split-K in one launch, for problems with fewer output tiles than CUs (the reference's G = 1
 * Mixtral EP path, kernels/grouped_gemm.py:629-640 -> kernels/matmul.py:332-392, runs one
 * workgroup per tile and leaves most of the GPU idle on a skinny-N, long-K W2).  Each output tile
 * is computed by `splits` units over K ranges of whole block_k slices; each unit writes its fp32
 * partial tile into `workspace`, and the last unit of a tile (counted with one atomic per unit)
 * sums the partials in split order (deterministic), casts and stores C, and re-arms the counter.
 * `workspace` (256-byte aligned, at least moegemm_splitk_workspace_bytes() bytes) holds a fixed
 * 256 KiB area of int32 tile counters (at most 65536 output tiles) then the fp32 partials; the
 * counter area must be zero before the first call and every call leaves it zero, whatever its
 * tile count or shape, so one workspace serves calls of any shape in any order and a captured
 * graph can be replayed without clearing it.  Calls that share a workspace must not overlap (use
 * one workspace per stream).  fp16/bf16 in the vector layout only
 * (the LDS-DMA kernels); `splits` is clamped to the number of non-empty K ranges.
 */
int moegemm_splitk_workspace_bytes(int32_t tiles, int32_t splits, int32_t block_m, int32_t block_n,
                                   int64_t* bytes);
int moegemm_matmul_splitk(const void* a, const void* b, void* c, int32_t m, int32_t n, int32_t k,
                          int64_t stride_am, int64_t stride_ak, int64_t stride_bk,
                          int64_t stride_bn, int64_t stride_cm, int64_t stride_cn, int32_t dtype,
                          int32_t block_m, int32_t block_n, int32_t block_k, int32_t group_size_m,
                          int32_t num_warps, int32_t num_stages, int32_t splits, int32_t grid_size,
                          void* workspace, int64_t workspace_bytes, int32_t b_stream, void* stream);
/*
 * moegemm_matmul_splitk without the workspace argument: the partials and tile counters live in a
 * static device array of MOEGEMM_NOALLOC_SCRATCH_BYTES inside the library (one per GPU, held until
 * the process ends), so the call allocates nothing, not even on its first use.  No counterpart in
 * the reference: it is for callers that cannot allocate (code under HIP graph capture, serving
 * loops, harnesses that forbid hipMalloc).  Limits and rules:
 *   - a launch whose split partials need more than MOEGEMM_NOALLOC_SCRATCH_BYTES (256 KiB of
 *     counters + tiles * splits * block_m * block_n * 4 bytes) is rejected with
 *     MOEGEMM_ERR_INVALID before anything runs;
 *   - every call on one GPU shares that GPU's area: calls that overlap on one GPU (different
 *     streams or threads without ordering) race and may produce wrong results;
 *   - the first call on a GPU also launches one small kernel on `stream` that clears the counters
 *     (later launches leave them zero); the results equal moegemm_matmul_splitk's bit for bit;
 *   - footprint: the array is part of the library's code object, so every process that loads the
 *     library holds MOEGEMM_NOALLOC_SCRATCH_BYTES of device memory on each GPU the library is
 *     loaded on, whether or not this entry point is ever called.
 */
#define MOEGEMM_NOALLOC_SCRATCH_BYTES (64 * 1024 * 1024 + 256 * 1024)
int moegemm_matmul_splitk_noalloc(const void* a, const void* b, void* c, int32_t m, int32_t n, int32_t k,
                                  int64_t stride_am, int64_t stride_ak, int64_t stride_bk,
                                  int64_t stride_bn, int64_t stride_cm, int64_t stride_cn, int32_t dtype,
                                  int32_t block_m, int32_t block_n, int32_t block_k, int32_t group_size_m,
                                  int32_t num_warps, int32_t num_stages, int32_t splits, int32_t grid_size,
                                  int32_t b_stream, void* stream);
/* Homogeneous grouped counterpart (equal contiguous problems, vector_layout must be 1). */
int moegemm_grouped_gemm_splitk(const int64_t* a_ptrs, const int64_t* b_ptrs, const int64_t* c_ptrs,
                                int32_t problem_count, int32_t m, int32_t n, int32_t k,
                                int32_t dtype, int32_t block_m, int32_t block_n, int32_t block_k,
                                int32_t group_size_m, int32_t num_warps, int32_t num_stages,
                                int32_t splits, int32_t grid_size, int32_t vector_layout,
                                void* workspace, int64_t workspace_bytes, int32_t b_stream, void* stream);

/*
 * Stream-K tail in one launch, for launches whose tile count leaves the last round of a persistent
 * grid partly idle (T = R * grid_size + r tiles take R + 1 rounds for R + r / grid_size rounds of
 * work).  Replaces the same reference launches as the split-K entry points above (G = 1:
 * kernels/matmul.py:332-392, homogeneous: kernels/grouped_gemm.py:321-397, dispatched by
 * launch_grouped, :618-760), whose programs each take whole tiles pid, pid + grid, ...
 * (:346-353, :397).  The first T - tail_tiles output tiles run whole, on the static schedule; the
 * K slices (block_k each) of the last tail_tiles tiles are cut into grid_size equal runs in tile
 * order, one per workgroup.  A run that covers part of a tile writes its fp32 partial into
 * `workspace`; the last piece of a tile to arrive sums the tile's partials in K order
 * (deterministic), casts and stores C.  With tail_tiles = r every workgroup ends after R + r /
 * grid_size tile times.  `workspace` (256-byte aligned, at least moegemm_streamk_workspace_bytes()
 * bytes) holds the 256 KiB counter area of the split-K workspace (zero before the first call, left
 * zero by every call; one workspace can serve split-K and stream-K calls alike) then grid_size +
 * tail_tiles partial slots of block_m * block_n floats.  Calls that share a workspace must not
 * overlap.  Requirements: fp16/bf16 in the vector layout, grid_size >= 1, 1 <= tail_tiles <=
 * min(T, 65536), and runs of at least ceil(K / block_k) / 63 slices (no tile cut into more than 64
 * pieces).  Results differ from the unsplit launch's only in the order of the fp32 sums.
 */
int moegemm_streamk_workspace_bytes(int32_t tail_tiles, int32_t grid_size, int32_t block_m, int32_t block_n,
                                    int64_t* bytes);
int moegemm_matmul_streamk(const void* a, const void* b, void* c, int32_t m, int32_t n, int32_t k,
                           int64_t stride_am, int64_t stride_ak, int64_t stride_bk, int64_t stride_bn,
                           int64_t stride_cm, int64_t stride_cn, int32_t dtype, int32_t block_m,
                           int32_t block_n, int32_t block_k, int32_t group_size_m, int32_t num_warps,
                           int32_t num_stages, int32_t tail_tiles, int32_t grid_size, void* workspace,
                           int64_t workspace_bytes, int32_t b_stream, void* stream);
/* Homogeneous grouped counterpart (equal contiguous problems, vector_layout must be 1). */
int moegemm_grouped_gemm_streamk(const int64_t* a_ptrs, const int64_t* b_ptrs, const int64_t* c_ptrs,
                                 int32_t problem_count, int32_t m, int32_t n, int32_t k, int32_t dtype,
                                 int32_t block_m, int32_t block_n, int32_t block_k, int32_t group_size_m,
                                 int32_t num_warps, int32_t num_stages, int32_t tail_tiles,
                                 int32_t grid_size, int32_t vector_layout, void* workspace,
                                 int64_t workspace_bytes, int32_t b_stream, void* stream);

/* 1 when compiled kernel `index` of `dtype` can run the SwiGLU epilogue, 0 when not, < 0 on a bad
 * index.  No counterpart in the reference (its Triton pools have no fused epilogue). */
int moegemm_kernel_swiglu(int dtype, int index);

/*
 * Grouped GEMM over the expert-sorted layout of torch.nn.functional.grouped_mm (2-D A, 3-D B):
 * for each group e, C[r0:r1, :] = A[r0:r1, :] @ B[e] with r0 = offs[e-1] (0 for e = 0) and
 * r1 = offs[e], fp32 accumulation.  A is [rows, k] (row stride stride_am), B is [group_count, k, n]
 * (strides stride_bg, stride_bk), C is [rows, n] (row stride stride_cm), all with unit inner stride;
 * offs is a device int32 [group_count] array of cumulative end rows that the kernel reads at run
 * time (it may be produced on the device by a router; no host copy is needed).  Offsets are
 * clamped to [0, rows] and a decreasing offset is an empty group, so no access leaves A or C; rows
 * at or past offs[group_count-1] are not written.  Replaces the one-call grouped_mm provider of
 * reference kernels/torch_grouped_gemm.py:121-174 (build_torch_grouped_workspace +
 * launch_torch_grouped; layout :139-158) with the persistent HIP kernel: the grid walks an upper
 * bound of the tile count computed on the host from rows and group_count and stops at the total
 * computed on the device from offs.  Tile config and grid_size as for moegemm_grouped_gemm; the
 * LDS-DMA kernel is chosen automatically when the layout allows it.
 */
int moegemm_grouped_mm_offs(const void* a, const void* b, void* c, const int32_t* offs,
                            int32_t group_count, int32_t rows, int32_t n, int32_t k,
                            int64_t stride_am, int64_t stride_bg, int64_t stride_bk,
                            int64_t stride_cm, int32_t dtype, int32_t input_precision,
                            int32_t block_m, int32_t block_n, int32_t block_k,
                            int32_t group_size_m, int32_t num_warps, int32_t num_stages,
                            int32_t grid_size, int32_t b_stream, void* stream);
/*
 * Packed Gate+Up over the expert-sorted layout with the SwiGLU epilogue: B is [group_count, k, n]
 * with n = 2F columns [gate | up] per group (the packed W13 weights of reference
 * kernels/grouped_gemm.py:575-594, stored as the 3-D grouped_mm operand of
 * kernels/torch_grouped_gemm.py:139-158), and H [rows, F] (row stride stride_hm) receives
 * silu(A[r0:r1] @ B[e][:, :F]) * (A[r0:r1] @ B[e][:, F:]) for each group, from the fp32 accumulators.
 * Offsets, clamping and untouched rows as in moegemm_grouped_mm_offs.  No counterpart in the reference
 * (it keeps the activation outside its timed GEMM, README.md:55-57).  Requires fp16/bf16, the vector
 * layout, n a multiple of 16 and a tile with moegemm_kernel_swiglu() == 1.
 */
int moegemm_grouped_mm_offs_swiglu(const void* a, const void* b, void* h, const int32_t* offs,
                                   int32_t group_count, int32_t rows, int32_t n, int32_t k,
                                   int64_t stride_am, int64_t stride_bg, int64_t stride_bk,
                                   int64_t stride_hm, int32_t dtype, int32_t block_m,
                                   int32_t block_n, int32_t block_k, int32_t group_size_m,
                                   int32_t num_warps, int32_t num_stages, int32_t grid_size,
                                   int32_t b_stream, void* stream);
/* The same launch with the work-stealing tile scheduler and queue of
 * moegemm_grouped_gemm_stealing; ragged offsets give tiles of unequal cost (partial M tiles). */
int moegemm_grouped_mm_offs_stealing(const void* a, const void* b, void* c, const int32_t* offs,
                                     int32_t group_count, int32_t rows, int32_t n, int32_t k,
                                     int64_t stride_am, int64_t stride_bg, int64_t stride_bk,
                                     int64_t stride_cm, int32_t dtype, int32_t input_precision,
                                     int32_t block_m, int32_t block_n, int32_t block_k,
                                     int32_t group_size_m, int32_t num_warps,
                                     int32_t num_stages, int32_t grid_size, void* queue,
                                     int32_t b_stream, void* stream);

/*
 * Masked single GEMM with arbitrary strides, C = A @ B.  Replaces the Triton launch of
 * reference kernels/matmul.py:332-392 (launch_matmul -> _matmul_kernel_impl, :223-273); shape
 * and dtype validation (_validate_matrices, kernels/matmul.py:318-329) stays in Python.  grid_size <= 0 launches one
 * workgroup per output tile like the reference's 1-D grid; a positive value makes it persistent.
 * The LDS-DMA kernel is chosen automatically when the operands meet its layout preconditions.
 */
int moegemm_matmul(const void* a, const void* b, void* c, int32_t m, int32_t n, int32_t k,
                   int64_t stride_am, int64_t stride_ak, int64_t stride_bk, int64_t stride_bn,
                   int64_t stride_cm, int64_t stride_cn, int32_t dtype, int32_t input_precision,
                   int32_t block_m, int32_t block_n, int32_t block_k, int32_t group_size_m,
                   int32_t num_warps, int32_t num_stages, int32_t grid_size, int32_t b_stream, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MOEGEMM_H */
