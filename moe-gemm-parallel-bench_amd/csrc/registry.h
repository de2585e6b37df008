// Table of compiled kernel instantiations.  Each entry is one tile configuration for one dtype,
// with up to two kernels: the LDS-DMA fast path (16-bit operands in vector layouts) and the
// general register-staged kernel (any strides/alignment, and all fp32 work).
#pragma once
#include <hip/hip_runtime.h>

#include "gemm_fast.h"
#include "gemm_kernel.h"
#include "gemm_pingpong.h"

namespace moegemm {

typedef hipError_t (*LaunchFn)(const KParams&, int grid, hipStream_t stream);

struct KernelEntry {
  int dtype;
  int block_m, block_n, block_k;
  int num_warps;   // wave64 wavefronts per workgroup
  int num_stages;  // LDS stages of the fast path's K pipeline
  int waves_m, waves_n;
  int lds_bytes;   // fast path if present, else general
  int swiglu_ok;   // the fast path can run the packed Gate+Up SwiGLU epilogue (even FN)
  LaunchFn launch_fast;     // null when the dtype has no fast path
  LaunchFn launch_general;
  LaunchFn launch_fast_split;  // the fast path's split-K kernel (null without a fast path)
  LaunchFn launch_fast_streamk;  // the fast path's stream-K kernel (null without a fast path)
};

template <class T, bool SPLIT = false, bool STREAMK = false>
hipError_t launch_tile(const KParams& p, int grid, hipStream_t stream) {
  hipLaunchKernelGGL((grouped_gemm_kernel<T, SPLIT, STREAMK>), dim3(grid), dim3(T::NT), 0, stream, p);
  return hipGetLastError();
}

// X-macro menus: X(E, BM, BN, BK, WAVES_M, WAVES_N, STAGES).  Each translation unit expands a
// menu into explicit kernel instantiations (device and host passes) and into the host table.
// The 8-wave 256x256 tiles with at least three stages run the ping-pong schedule
// (gemm_pingpong.h); every other 16-bit vector-layout tile runs FastTile's schedule.
template <class E, int BM, int BN, int BK, int WM, int WN, int S>
struct FastTileFor {
  using type = typename std::conditional<BM == 256 && BN == 256 && WM == 2 && WN == 4 && S >= 3,
                                         PingPongTile<E, BK, S>, FastTile<E, BM, BN, BK, WM, WN, S>>::type;
};
template <class E, int BM, int BN, int BK, int WM, int WN, int S>
using FastTileT = typename FastTileFor<E, BM, BN, BK, WM, WN, S>::type;
#define MOEGEMM_FAST(E, BM, BN, BK, WM, WN, S) FastTileT<E, BM, BN, BK, WM, WN, S>
// The general kernel has no stage count; the wrapper keeps one instantiation per menu entry even
// when two entries differ only in the fast path's stages.
template <class E, int BM, int BN, int BK, int WM, int WN, int S>
struct GemmTileEntry : GemmTile<E, BM, BN, BK, WM, WN> {};
#define MOEGEMM_GEN(E, BM, BN, BK, WM, WN, S) GemmTileEntry<E, BM, BN, BK, WM, WN, S>

#define MOEGEMM_INST16(E, BM, BN, BK, WM, WN, S)                                                     \
  template __global__ void grouped_gemm_kernel<MOEGEMM_FAST(E, BM, BN, BK, WM, WN, S), false>(KParams); \
  template __global__ void grouped_gemm_kernel<MOEGEMM_FAST(E, BM, BN, BK, WM, WN, S), true>(KParams);  \
  template __global__ void grouped_gemm_kernel<MOEGEMM_GEN(E, BM, BN, BK, WM, WN, S), false>(KParams);
// The stream-K kernels live in translation units of their own (inst_*_sk.hip): compiled next to
// the other kernels of a tile, their presence in the module changed the register allocation of
// those kernels (18 of 54 moved, one from 8 to 72 bytes of scratch).  Each such unit instantiates
// the kernel and its host launcher; the tables refer to the launchers through these declarations.
#define MOEGEMM_INST16_SK(E, BM, BN, BK, WM, WN, S)                                                        \
  template __global__ void grouped_gemm_kernel<MOEGEMM_FAST(E, BM, BN, BK, WM, WN, S), true, true>(KParams); \
  template hipError_t launch_tile<MOEGEMM_FAST(E, BM, BN, BK, WM, WN, S), true, true>(const KParams&, int,   \
                                                                                      hipStream_t);
#define MOEGEMM_EXTERN16_SK(E, BM, BN, BK, WM, WN, S)                                                          \
  extern template hipError_t launch_tile<MOEGEMM_FAST(E, BM, BN, BK, WM, WN, S), true, true>(const KParams&, int, \
                                                                                             hipStream_t);
#define MOEGEMM_ENTRY16(E, BM, BN, BK, WM, WN, S)                                             \
  KernelEntry{E::dtype, BM, BN, BK, (WM) * (WN), S, WM, WN,                                   \
              MOEGEMM_FAST(E, BM, BN, BK, WM, WN, S)::LDS_BYTES,                              \
              MOEGEMM_FAST(E, BM, BN, BK, WM, WN, S)::SWIGLU_OK ? 1 : 0,                      \
              &launch_tile<MOEGEMM_FAST(E, BM, BN, BK, WM, WN, S)>,                          \
              &launch_tile<MOEGEMM_GEN(E, BM, BN, BK, WM, WN, S)>,                           \
              &launch_tile<MOEGEMM_FAST(E, BM, BN, BK, WM, WN, S), true>,                    \
              &launch_tile<MOEGEMM_FAST(E, BM, BN, BK, WM, WN, S), true, true>},

#define MOEGEMM_INST32(E, BM, BN, BK, WM, WN, S) \
  template __global__ void grouped_gemm_kernel<MOEGEMM_GEN(E, BM, BN, BK, WM, WN, S), false>(KParams);
#define MOEGEMM_ENTRY32(E, BM, BN, BK, WM, WN, S)                                             \
  KernelEntry{E::dtype, BM, BN, BK, (WM) * (WN), S, WM, WN,                                   \
              MOEGEMM_GEN(E, BM, BN, BK, WM, WN, S)::LDS_BYTES, 0, nullptr,                      \
              &launch_tile<MOEGEMM_GEN(E, BM, BN, BK, WM, WN, S)>, nullptr, nullptr},

// 16-bit menu (bf16 and f16 share it): large-M MFMA-bound tiles down to skinny-M streaming tiles.
// STAGES is sized to the 160 KiB LDS of a CU; the 2-stage narrow tiles at the end fit two
// workgroups per CU (16x128 fits four; LDS, and registers via FastTile::WAVES_PER_EU), so one
// workgroup's prologue overlaps another's work on short-K groups.
#define MOEGEMM_MENU_16BIT(X, E)                                                             \
  X(E, 256, 256, 64, 2, 4, 2) X(E, 256, 256, 64, 2, 2, 2) X(E, 256, 256, 32, 2, 2, 4)        \
  X(E, 256, 256, 32, 2, 4, 4)                                                                \
  X(E, 256, 128, 64, 2, 2, 3) X(E, 128, 256, 64, 2, 4, 3)                                   \
  X(E, 128, 256, 64, 2, 2, 3) X(E, 128, 128, 64, 2, 2, 4) X(E, 128, 64, 64, 2, 2, 4)         \
  X(E, 64, 256, 64, 1, 4, 3) X(E, 64, 128, 64, 2, 2, 4) X(E, 64, 64, 64, 2, 2, 4)            \
  X(E, 32, 256, 64, 1, 4, 4) X(E, 32, 128, 64, 1, 4, 4) X(E, 32, 128, 128, 1, 4, 3)          \
  X(E, 16, 256, 64, 1, 4, 4) X(E, 16, 256, 128, 1, 4, 2) X(E, 16, 128, 128, 1, 4, 4)         \
  X(E, 16, 64, 128, 1, 4, 4) X(E, 16, 64, 128, 1, 4, 7)                                    \
  X(E, 16, 256, 64, 1, 4, 2) X(E, 32, 256, 64, 1, 4, 2) X(E, 64, 128, 64, 2, 2, 2)        \
  X(E, 16, 128, 64, 1, 4, 2) X(E, 16, 512, 64, 1, 4, 2) X(E, 64, 512, 64, 1, 4, 2)        \
  X(E, 32, 512, 32, 1, 4, 4)

// fp32 menu (general kernel, v_mfma_f32_16x16x4_f32); STAGES is the register-staged double buffer.
#define MOEGEMM_MENU_F32(X, E)                                                               \
  X(E, 128, 128, 32, 2, 2, 2) X(E, 64, 64, 32, 2, 2, 2) X(E, 32, 64, 32, 1, 4, 2)            \
  X(E, 16, 64, 32, 1, 4, 2) X(E, 32, 32, 32, 1, 2, 2)

extern const KernelEntry kEntriesBf16[];
extern const int kNumBf16;
extern const KernelEntry kEntriesF16[];
extern const int kNumF16;
extern const KernelEntry kEntriesF32[];
extern const int kNumF32;

}  // namespace moegemm
