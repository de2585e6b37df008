// Table of compiled kernel instantiations.  Each entry is one tile configuration for one dtype.
#pragma once
#include <hip/hip_runtime.h>
#include "gemm_kernel.h"

namespace moegemm {

struct KernelEntry {
  int dtype;
  int block_m, block_n, block_k;
  int num_warps;   // wave64 wavefronts per workgroup
  int num_stages;  // LDS pipeline stages
  int waves_m, waves_n;
  int lds_bytes;
  hipError_t (*launch)(const KParams&, int grid, hipStream_t stream);
};

template <class T>
hipError_t launch_tile(const KParams& p, int grid, hipStream_t stream) {
  hipLaunchKernelGGL(grouped_gemm_kernel<T>, dim3(grid), dim3(T::NT), 0, stream, p);
  return hipGetLastError();
}

// X-macro menus: X(E, BM, BN, BK, WAVES_M, WAVES_N).  Each translation unit expands a menu twice:
// once into explicit kernel instantiations (device and host passes) and once into the host-side
// launch table.
#define MOEGEMM_INST(E, BM, BN, BK, WM, WN) \
  template __global__ void grouped_gemm_kernel<GemmTile<E, BM, BN, BK, WM, WN>>(KParams);
#define MOEGEMM_ENTRY(E, BM, BN, BK, WM, WN)                                                  \
  KernelEntry{E::dtype, BM, BN, BK, (WM) * (WN), 2, WM, WN,                                   \
              GemmTile<E, BM, BN, BK, WM, WN>::LDS_BYTES, &launch_tile<GemmTile<E, BM, BN, BK, WM, WN>>},

// 16-bit menu (bf16 and f16 share it): large-M MFMA-bound tiles down to skinny-M streaming tiles.
#define MOEGEMM_MENU_16BIT(X, E)                                                             \
  X(E, 256, 256, 64, 2, 2) X(E, 256, 128, 64, 2, 2) X(E, 128, 256, 64, 2, 2)                 \
  X(E, 128, 128, 64, 2, 2) X(E, 128, 64, 64, 2, 2) X(E, 64, 256, 64, 1, 4)                   \
  X(E, 64, 128, 64, 2, 2) X(E, 64, 64, 64, 2, 2) X(E, 64, 64, 32, 2, 2)                      \
  X(E, 32, 256, 64, 1, 4) X(E, 32, 128, 64, 1, 4) X(E, 32, 128, 128, 1, 4)                   \
  X(E, 16, 256, 64, 1, 4) X(E, 16, 256, 128, 1, 4) X(E, 16, 128, 128, 1, 4)                  \
  X(E, 16, 64, 128, 1, 4)

#define MOEGEMM_MENU_F32(X, E)                                                               \
  X(E, 128, 128, 32, 2, 2) X(E, 64, 64, 32, 2, 2) X(E, 32, 64, 32, 1, 4)                     \
  X(E, 16, 64, 32, 1, 4) X(E, 32, 32, 32, 1, 2)

extern const KernelEntry kEntriesBf16[];
extern const int kNumBf16;
extern const KernelEntry kEntriesF16[];
extern const int kNumF16;
extern const KernelEntry kEntriesF32[];
extern const int kNumF32;

}  // namespace moegemm
