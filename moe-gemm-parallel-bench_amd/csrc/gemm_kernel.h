// Persistent grouped GEMM for gfx950 (CDNA4): C_e = A_e @ B_e over per-problem pointer tables.
//
// Semantics follow kernels/grouped_gemm.py:321-482 and kernels/matmul.py:223-273 of the reference:
// fp32 accumulation of fp16/bf16/fp32 operands, masked M/N/K tails, cast of the accumulator to C's
// dtype on store, GROUP_M traversal inside each problem, and a persistent grid that walks a flat
// (problem, m-tile, n-tile) index space.  The implementation is CDNA4-native:
//
//  * Work unit: one BM x BN output tile, computed by WM x WN wave64 wavefronts with
//    v_mfma_f32_32x32x16 / v_mfma_f32_16x16x32 (bf16, f16) or v_mfma_f32_16x16x4_f32 (fp32).
//  * Operands are swapped (D^T = B^T A^T) so that each lane owns four consecutive N columns of one
//    output row: the epilogue stores 8-byte (bf16/f16) or 16-byte (fp32) vectors.
//  * A tiles live in LDS as [BM][BK] (K contiguous) and are read with ds_read_b128; B tiles live
//    as [BK][BN] (N contiguous, the layout of the caller's B) and are read K-packed with the gfx950
//    transpose load ds_read_b64_tr_b16, so B never needs a transposed copy in HBM.
//  * 16-byte chunks are XOR-swizzled inside each LDS row so that fragment reads of 16 consecutive
//    rows (A) or of 4x2 row/chunk groups (B transpose reads) fall on distinct banks.
//  * Global -> LDS staging goes through registers with double-buffered LDS stages: the next K
//    slice is in flight while MFMAs consume the current one; one workgroup barrier per K slice.
//  * Persistent schedule: each of the 8 XCDs (workgroups are dispatched to them round-robin by
//    id) owns a contiguous eighth of the tile index space, which its workgroups walk in lockstep;
//    the tiles of one expert, and so the A/B panels they share, stay in that XCD's L2.
//  * Generic groups (heterogeneous shapes/strides) map tile -> problem with an LDS prefix sum of
//    per-problem tile counts and a binary search, instead of a per-tile scan over all problems.
//  * Offsets mode (the expert-sorted layout of torch.nn.functional.grouped_mm: A [rows, K] and
//    C [rows, N] split by cumulative int32 end rows `offs`, B [G, K, N]) derives each group's row
//    count from `offs` on the device, so a router can produce `offs` without a host round trip;
//    the host passes only an upper bound on the tile count and the grid stops at the device total.
//    Offsets are clamped to [0, rows], so no access leaves A or C whatever `offs` holds.
//  * Every problem is checked at run time for the vector preconditions (unit inner stride, row
//    stride and extent multiples of the 16-byte chunk, 16-byte aligned base); a problem that fails
//    them is staged element by element with arbitrary strides.  Pointer tables are read from
//    device memory on every tile, so callers may rewrite them between launches.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

namespace moegemm {

typedef short i16x4_t __attribute__((ext_vector_type(4)));
typedef short i16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

enum DType : int { DT_F16 = 0, DT_BF16 = 1, DT_F32 = 2 };
enum Mode : int { MODE_SINGLE = 0, MODE_HOMOGENEOUS = 1, MODE_GENERIC = 2, MODE_OFFSETS = 3 };

// Kernel arguments, passed by value.  Strides are in elements.
struct KParams {
  const int64_t* a_ptrs;
  const int64_t* b_ptrs;
  const int64_t* c_ptrs;
  const int32_t* dims;     // [G,3] = (m, n, k) per problem (generic mode)
  const int64_t* strides;  // [G,6] = (am, ak, bk, bn, cm, cn) per problem (generic mode)
  const void* a;           // single mode operands
  const void* b;
  void* c;
  int64_t sam, sak, sbk, sbn, scm, scn;  // single / offsets mode strides
  const int32_t* offs;   // offsets mode: [G] cumulative end rows of the expert-sorted A and C
  int64_t sbg;           // offsets mode: B stride between groups (elements)
  int32_t rows;          // offsets mode: rows of A and C; offsets are clamped to it
  int32_t mode;
  int32_t G;
  int32_t M, N, K;       // single / homogeneous shape
  int32_t total_tiles;
  int32_t group_m;
  int32_t tf32;          // fp32 only: round operands to TF32 (10-bit mantissa, ties away)
  int32_t swiglu;        // packed Gate+Up epilogue: B = [gate | up] (n columns), output n/2 columns
  // Split-K (single and homogeneous modes, LDS-DMA tiles): each output tile is computed by
  // `splits` units over K ranges of k_chunk elements; units write fp32 partial tiles to
  // `partials` ([tiles][splits][BM*BN]) and count arrivals in `counters` ([tiles], zero between
  // launches); the last unit of a tile sums the partials in split order and stores C.
  int32_t splits;
  int32_t k_chunk;
  int32_t split_polls;  // polls of a tile's counter a unit makes while waiting for the tile's other units
  float* partials;
  int32_t* counters;
  // Work-stealing schedule (null = static): ticket counters and exit counts, one per 256-byte
  // block (the layout is at kQueueStride); zero between launches (the last workgroup of a launch
  // re-arms them).
  int32_t* queue;
  // Stream-K tail (the stream-K kernel, single and homogeneous modes; 0 = off): the first
  // total_tiles - sk_tiles tiles run whole on the static schedule, the last sk_tiles tiles are
  // cut into `grid` equal runs of K slices, one per workgroup (see streamk_units).
  int32_t sk_tiles;
  // B copy policy of the LDS-DMA tiles: 1 issues B's global -> LDS copies non-temporal (streamed
  // data, evicted first from the caches), 0 as ordinary loads.  A's copies are always ordinary.
  int32_t b_stream;
};

struct ProblemDesc {
  const char* a;
  const char* b;
  char* c;
  int32_t m, n, k;
  int64_t sam, sak, sbk, sbn, scm, scn;
  int32_t swiglu;  // C holds silu(A @ B[:, :n/2]) * (A @ B[:, n/2:]), n/2 columns
  int32_t splits;  // > 1: this unit covers one K range of output tile `tile`
  int32_t split;
  int32_t tile;
  int32_t split_wait;  // > 0 when every unit of the launch has a workgroup of its own: a tile's units
                       // may then wait for each other, up to this many polls, to share its reduction
  float* partials;
  int32_t* counters;
  int32_t slot0;       // partial slot of the tile's unit 0; unit s writes slot slot0 + s
  int32_t b_stream;    // KParams::b_stream
};


// Epilogue of a unit: the C store, the fp32 partial of a split-K unit (split_store), or either,
// chosen per unit by its piece count (stream-K launches: whole tiles store C, pieces store partials).
enum Epilogue : int { EPI_C = 0, EPI_SPLIT = 1, EPI_EITHER = 2 };

// Wave-uniform copies: values derived from LDS (the generic-mode prefix search) are treated as
// divergent by the compiler; reading lane 0 makes every descriptor scalar again, so table loads
// become scalar loads and buffer resources need no waterfall loops.
__device__ __forceinline__ int32_t uniform(int32_t x) { return __builtin_amdgcn_readfirstlane(x); }
__device__ __forceinline__ int64_t uniform(int64_t x) {
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)(uint64_t)x);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)((uint64_t)x >> 32));
  return (int64_t)(((uint64_t)hi << 32) | lo);
}
template <class P>
__device__ __forceinline__ P* uniform(P* x) {
  return reinterpret_cast<P*>(uniform(reinterpret_cast<int64_t>(x)));
}
__device__ __forceinline__ void make_uniform(ProblemDesc& pd) {
  pd.a = uniform(pd.a);
  pd.b = uniform(pd.b);
  pd.c = uniform(pd.c);
  pd.m = uniform(pd.m);
  pd.n = uniform(pd.n);
  pd.k = uniform(pd.k);
  pd.sam = uniform(pd.sam);
  pd.sak = uniform(pd.sak);
  pd.sbk = uniform(pd.sbk);
  pd.sbn = uniform(pd.sbn);
  pd.scm = uniform(pd.scm);
  pd.scn = uniform(pd.scn);
  pd.swiglu = uniform(pd.swiglu);
  pd.splits = uniform(pd.splits);
  pd.split = uniform(pd.split);
  pd.tile = uniform(pd.tile);
  pd.split_wait = uniform(pd.split_wait);
  pd.partials = uniform(pd.partials);
  pd.counters = uniform(pd.counters);
  pd.slot0 = uniform(pd.slot0);
  pd.b_stream = uniform(pd.b_stream);
}

// ---------------------------------------------------------------------------------------------
// Element traits
struct EBf16 {
  using raw = uint16_t;
  static constexpr int dtype = DT_BF16;
  static constexpr bool is_f32 = false;
};
struct EF16 {
  using raw = uint16_t;
  static constexpr int dtype = DT_F16;
  static constexpr bool is_f32 = false;
};
struct EF32 {
  using raw = uint32_t;
  static constexpr int dtype = DT_F32;
  static constexpr bool is_f32 = true;
};

__device__ __forceinline__ uint32_t tf32_round(uint32_t u) {
  // Round-to-nearest, ties away from zero, to a 10-bit mantissa.  Inf/NaN pass through.
  if ((u & 0x7f800000u) == 0x7f800000u) return u;
  return (u + 0x1000u) & 0xffffe000u;
}

// Four fp32 results converted to the output type and stored (8 or 16 bytes).  These stores cover
// part of a cache line; L2 merges the neighbouring pieces before the line goes out.
template <class E>
__device__ __forceinline__ void store4(char* dst, f32x4_t v);

#define MOEGEMM_GLOBAL(T, p) ((__attribute__((address_space(1))) T*)(p))
template <>
__device__ __forceinline__ void store4<EBf16>(char* dst, f32x4_t v) {
  typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
  bf16x4_t o;
  o[0] = (__bf16)v[0]; o[1] = (__bf16)v[1]; o[2] = (__bf16)v[2]; o[3] = (__bf16)v[3];
  *MOEGEMM_GLOBAL(bf16x4_t, dst) = o;
}
template <>
__device__ __forceinline__ void store4<EF16>(char* dst, f32x4_t v) {
  typedef _Float16 f16x4_t __attribute__((ext_vector_type(4)));
  f16x4_t o;
  o[0] = (_Float16)v[0]; o[1] = (_Float16)v[1]; o[2] = (_Float16)v[2]; o[3] = (_Float16)v[3];
  *MOEGEMM_GLOBAL(f16x4_t, dst) = o;
}
template <>
__device__ __forceinline__ void store4<EF32>(char* dst, f32x4_t v) {
  *MOEGEMM_GLOBAL(f32x4_t, dst) = v;
}

// Four fp32 values converted to the 16-bit type, as the 8 bytes of one packed pair of dwords.
template <class E>
__device__ __forceinline__ u32x2_t pack4(f32x4_t v) {
  static_assert(E::dtype != DT_F32, "16-bit outputs only");
  if constexpr (E::dtype == DT_BF16) {
    typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
    bf16x4_t o;
    o[0] = (__bf16)v[0]; o[1] = (__bf16)v[1]; o[2] = (__bf16)v[2]; o[3] = (__bf16)v[3];
    return __builtin_bit_cast(u32x2_t, o);
  } else {
    typedef _Float16 f16x4_t __attribute__((ext_vector_type(4)));
    f16x4_t o;
    o[0] = (_Float16)v[0]; o[1] = (_Float16)v[1]; o[2] = (_Float16)v[2]; o[3] = (_Float16)v[3];
    return __builtin_bit_cast(u32x2_t, o);
  }
}

// Four fp32 values converted to the 16-bit type, written to LDS (8 bytes).
template <class E>
__device__ __forceinline__ void store4_lds(char* dst, f32x4_t v) {
  static_assert(E::dtype != DT_F32, "16-bit staging only");
  if constexpr (E::dtype == DT_BF16) {
    typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
    bf16x4_t o;
    o[0] = (__bf16)v[0]; o[1] = (__bf16)v[1]; o[2] = (__bf16)v[2]; o[3] = (__bf16)v[3];
    *reinterpret_cast<bf16x4_t*>(dst) = o;
  } else {
    typedef _Float16 f16x4_t __attribute__((ext_vector_type(4)));
    f16x4_t o;
    o[0] = (_Float16)v[0]; o[1] = (_Float16)v[1]; o[2] = (_Float16)v[2]; o[3] = (_Float16)v[3];
    *reinterpret_cast<f16x4_t*>(dst) = o;
  }
}

template <class E>
__device__ __forceinline__ void store1(char* dst, float v);
template <>
__device__ __forceinline__ void store1<EBf16>(char* dst, float v) { *reinterpret_cast<__bf16*>(dst) = (__bf16)v; }
template <>
__device__ __forceinline__ void store1<EF16>(char* dst, float v) { *reinterpret_cast<_Float16*>(dst) = (_Float16)v; }
template <>
__device__ __forceinline__ void store1<EF32>(char* dst, float v) { *reinterpret_cast<float*>(dst) = v; }

// ---------------------------------------------------------------------------------------------
// XOR swizzles on 16-byte chunk indices (see header comment).
// Both were chosen with the SQ_LDS_BANK_CONFLICT counter on gfx950 over every fragment-read
// pattern the tiles use (ds_read_b128 A reads with the 32x32 and 16x16 MFMA lane maps at 4, 8 and
// 16 chunks per row; ds_read_b64_tr_b16 B reads at 8, 16 and 32 chunks per row): each read then
// takes the minimum LDS cycles (4 for b128, 2 for tr_b64).
__device__ __forceinline__ int swz_a(int row, int chunks) {
  int f = (chunks >= 16) ? (row & 15) : (row ^ (row >> 2));
  return f & (chunks - 1);
}
__device__ __forceinline__ int swz_b(int row, int chunks) {
  // Independent of row bit 2: the transpose reads fetch rows r and r + 4 (r bit 2 clear) with
  // one chunk index.
  if (chunks == 8) return ((row << 1) & 4) | ((row >> 2) & 2);
  // h = [0, 3, 6, 5] on row bits 0-1, doubled to chunk pairs, plus row bit 3 moving by 8 chunks.
  int r = row & 3;
  int h = (r << 1) ^ r;
  int f = (h << 1) ^ (((row >> 3) & 1) << 3);
  return f & (chunks - 1);
}

// ---------------------------------------------------------------------------------------------
template <class E, int BM_, int BN_, int BK_, int WM_, int WN_>
struct GemmTile {
  using raw_t = typename E::raw;
  static constexpr int BM = BM_, BN = BN_, BK = BK_, WM = WM_, WN = WN_;
  static constexpr int ES = sizeof(raw_t);
  static constexpr int NW = WM * WN;
  static constexpr int NT = NW * 64;
  static constexpr int WTM = BM / WM;
  static constexpr int WTN = BN / WN;
  static constexpr bool F32 = E::is_f32;
  static constexpr int MI = F32 ? 16 : ((WTM >= 32 && WTN >= 32) ? 32 : 16);
  static constexpr int MIK = F32 ? 4 : (MI == 32 ? 16 : 32);
  static constexpr int FM = WTM / MI;
  static constexpr int FN = WTN / MI;
  static constexpr int ACC = MI * MI / 64;
  static constexpr int EPC = 16 / ES;  // elements per 16-byte chunk
  static constexpr int CA = BK / EPC;  // chunks per A row
  static constexpr int CB = BN / EPC;  // chunks per B row
  static constexpr int A_CHUNKS = BM * CA;
  static constexpr int B_CHUNKS = BK * CB;
  static constexpr int A_PT = (A_CHUNKS + NT - 1) / NT;
  static constexpr int B_PT = (B_CHUNKS + NT - 1) / NT;
  static constexpr int A_BYTES = BM * BK * ES;
  static constexpr int B_BYTES = BK * BN * ES;
  static constexpr int STAGE_BYTES = A_BYTES + B_BYTES;
  static constexpr int PREFIX = 1024;  // problems per prefix-sum chunk (generic mode)
  static constexpr int PREFIX_OFFSET = 2 * STAGE_BYTES;
  static constexpr int LDS_BYTES = PREFIX_OFFSET + (PREFIX + 1) * 4 + NT * 4;
  static constexpr int WAVES_PER_EU = 1;
  static constexpr bool CHAIN_OK = false;  // no cross-tile copy chaining (LDS-DMA tiles only)
  static constexpr bool CHAIN_STEALING = false;

  static_assert(BM % WM == 0 && BN % WN == 0, "tile must split evenly over waves");
  static_assert(WTM % MI == 0 && WTN % MI == 0, "wave tile must be a multiple of the MFMA tile");
  static_assert(BK % MIK == 0 && BK % EPC == 0, "BK must cover whole MFMA K steps and chunks");
  static_assert(F32 || CB >= 4, "transpose reads need at least 32 columns");
  static_assert(F32 || MIK % 16 == 0, "B swizzle assumes K steps of 16 rows");

  using acc_t = typename std::conditional<ACC == 16, f32x16_t, f32x4_t>::type;

  // -------------------------------------------------------------------------------------------
  // Global -> register staging for one K slice.  Each thread owns A_PT + B_PT 16-byte chunks.
  struct Stage {
    u32x4_t a[A_PT];
    u32x4_t b[B_PT];
  };

  __device__ static __forceinline__ u32x4_t load_chunk_gather(const char* base, int64_t s_outer, int64_t s_inner,
                                                              int outer, int inner0, int outer_lim, int inner_lim,
                                                              bool tf32) {
    // Element-wise masked gather of EPC consecutive inner elements (arbitrary strides).
    u32x4_t v = {0u, 0u, 0u, 0u};
    if (outer < outer_lim) {
      const raw_t* p = reinterpret_cast<const raw_t*>(base) + (int64_t)outer * s_outer;
      raw_t tmp[EPC];
#pragma unroll
      for (int e = 0; e < EPC; ++e) {
        int in = inner0 + e;
        tmp[e] = (in < inner_lim) ? p[(int64_t)in * s_inner] : (raw_t)0;
      }
      v = *reinterpret_cast<u32x4_t*>(tmp);
    }
    if (F32 && tf32) {
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = tf32_round(v[e]);
    }
    return v;
  }

  __device__ static __forceinline__ void load_stage(Stage& st, const ProblemDesc& pd, bool vec_a, bool vec_b,
                                                    int m0, int n0, int k0, bool tf32) {
    const int tid = threadIdx.x;
#pragma unroll
    for (int i = 0; i < A_PT; ++i) {
      int cl = tid + i * NT;
      st.a[i] = u32x4_t{0u, 0u, 0u, 0u};
      if (A_CHUNKS % NT == 0 || cl < A_CHUNKS) {
        int r = cl / CA, c = cl % CA;
        int gm = m0 + r, gk = k0 + c * EPC;
        if (vec_a) {
          if (gm < pd.m && gk < pd.k) {
            const u32x4_t* p = reinterpret_cast<const u32x4_t*>(pd.a + ((int64_t)gm * pd.sam + gk) * ES);
            st.a[i] = *p;
            if (F32 && tf32) {
#pragma unroll
              for (int e = 0; e < 4; ++e) st.a[i][e] = tf32_round(st.a[i][e]);
            }
          }
        } else {
          st.a[i] = load_chunk_gather(pd.a, pd.sam, pd.sak, gm, gk, pd.m, pd.k, tf32);
        }
      }
    }
#pragma unroll
    for (int i = 0; i < B_PT; ++i) {
      int cl = tid + i * NT;
      st.b[i] = u32x4_t{0u, 0u, 0u, 0u};
      if (B_CHUNKS % NT == 0 || cl < B_CHUNKS) {
        int r = cl / CB, c = cl % CB;
        int gk = k0 + r, gn = n0 + c * EPC;
        if (vec_b) {
          if (gk < pd.k && gn < pd.n) {
            const u32x4_t* p = reinterpret_cast<const u32x4_t*>(pd.b + ((int64_t)gk * pd.sbk + gn) * ES);
            st.b[i] = *p;
            if (F32 && tf32) {
#pragma unroll
              for (int e = 0; e < 4; ++e) st.b[i][e] = tf32_round(st.b[i][e]);
            }
          }
        } else {
          st.b[i] = load_chunk_gather(pd.b, pd.sbk, pd.sbn, gk, gn, pd.k, pd.n, tf32);
        }
      }
    }
  }

  __device__ static __forceinline__ void store_stage(const Stage& st, char* lds_a, char* lds_b) {
    const int tid = threadIdx.x;
#pragma unroll
    for (int i = 0; i < A_PT; ++i) {
      int cl = tid + i * NT;
      if (A_CHUNKS % NT == 0 || cl < A_CHUNKS) {
        int r = cl / CA, c = cl % CA;
        int pc = c ^ swz_a(r, CA);
        *reinterpret_cast<u32x4_t*>(lds_a + (r * CA + pc) * 16) = st.a[i];
      }
    }
#pragma unroll
    for (int i = 0; i < B_PT; ++i) {
      int cl = tid + i * NT;
      if (B_CHUNKS % NT == 0 || cl < B_CHUNKS) {
        int r = cl / CB, c = cl % CB;
        int pc = c ^ swz_b(r, CB);
        *reinterpret_cast<u32x4_t*>(lds_b + (r * CB + pc) * 16) = st.b[i];
      }
    }
  }

  // -------------------------------------------------------------------------------------------
  // MFMA over one K slice held in LDS.
  __device__ static __forceinline__ void compute_stage(acc_t (&acc)[FM][FN], const char* lds_a, const char* lds_b,
                                                       int wave_m, int wave_n) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int kk = 0; kk < BK / MIK; ++kk) {
      if constexpr (F32) {
        // v_mfma_f32_16x16x4_f32, swapped: first operand B^T (row n = lane%16, k = lane/16),
        // second operand A^T (col m = lane%16, k = lane/16).
        float af[FM], bf[FN];
        const int k = kk * 4 + (lane >> 4);
#pragma unroll
        for (int fm = 0; fm < FM; ++fm) {
          int row = wave_m * WTM + fm * 16 + (lane & 15);
          int c = k >> 2;
          int pc = c ^ swz_a(row, CA);
          af[fm] = *reinterpret_cast<const float*>(lds_a + (row * CA + pc) * 16 + (k & 3) * 4);
        }
#pragma unroll
        for (int fn = 0; fn < FN; ++fn) {
          int col = wave_n * WTN + fn * 16 + (lane & 15);
          int c = col >> 2;
          int pc = c ^ swz_b(k, CB);
          bf[fn] = *reinterpret_cast<const float*>(lds_b + (k * CB + pc) * 16 + (col & 3) * 4);
        }
#pragma unroll
        for (int fm = 0; fm < FM; ++fm)
#pragma unroll
          for (int fn = 0; fn < FN; ++fn)
            acc[fm][fn] = __builtin_amdgcn_mfma_f32_16x16x4f32(bf[fn], af[fm], acc[fm][fn], 0, 0, 0);
      } else {
        i16x8_t af[FM], bf[FN];
#pragma unroll
        for (int fm = 0; fm < FM; ++fm) {
          int row = wave_m * WTM + fm * MI + (lane % MI);
          int c = (kk * MIK) / 8 + lane / MI;
          int pc = c ^ swz_a(row, CA);
          af[fm] = *reinterpret_cast<const i16x8_t*>(lds_a + (row * CA + pc) * 16);
        }
#pragma unroll
        for (int fn = 0; fn < FN; ++fn) {
          const int g = lane >> 4, s = lane & 15;
          int row, col;
          if constexpr (MI == 32) {
            row = kk * MIK + 8 * (g >> 1) + (s >> 2);
            col = wave_n * WTN + fn * 32 + 16 * (g & 1) + 4 * (s & 3);
          } else {
            row = kk * MIK + 8 * g + (s >> 2);
            col = wave_n * WTN + fn * 16 + 4 * (s & 3);
          }
          int pc = (col >> 3) ^ swz_b(row, CB);
          const char* p0 = lds_b + (row * CB + pc) * 16 + (col & 7) * 2;
          const char* p1 = p0 + 4 * CB * 16;  // rows + 4 (same swizzle: bits 0-1 and 3 unchanged)
          i16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (__attribute__((address_space(3))) i16x4_t*)(p0));
          i16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (__attribute__((address_space(3))) i16x4_t*)(p1));
          bf[fn] = i16x8_t{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        }
#pragma unroll
        for (int fm = 0; fm < FM; ++fm)
#pragma unroll
          for (int fn = 0; fn < FN; ++fn) {
            if constexpr (E::dtype == DT_BF16) {
              if constexpr (MI == 32)
                acc[fm][fn] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                    __builtin_bit_cast(bf16x8_t, bf[fn]), __builtin_bit_cast(bf16x8_t, af[fm]), acc[fm][fn], 0, 0, 0);
              else
                acc[fm][fn] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                    __builtin_bit_cast(bf16x8_t, bf[fn]), __builtin_bit_cast(bf16x8_t, af[fm]), acc[fm][fn], 0, 0, 0);
            } else {
              if constexpr (MI == 32)
                acc[fm][fn] = __builtin_amdgcn_mfma_f32_32x32x16_f16(
                    __builtin_bit_cast(f16x8_t, bf[fn]), __builtin_bit_cast(f16x8_t, af[fm]), acc[fm][fn], 0, 0, 0);
              else
                acc[fm][fn] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                    __builtin_bit_cast(f16x8_t, bf[fn]), __builtin_bit_cast(f16x8_t, af[fm]), acc[fm][fn], 0, 0, 0);
            }
          }
      }
    }
  }

  // -------------------------------------------------------------------------------------------
  // Epilogue: lane owns output row m = mbase + lane%MI and, per group of 4 accumulators, four
  // consecutive columns.
  __device__ static __forceinline__ void store_tile(const acc_t (&acc)[FM][FN], const ProblemDesc& pd, int m0,
                                                    int n0, int wave_m, int wave_n) {
    const int lane = threadIdx.x & 63;
    // The SwiGLU and split-K epilogues run only in the LDS-DMA tiles (the host enforces it).
    if (pd.swiglu || pd.splits > 1) return;
    const bool vec_c = pd.scn == 1 && (pd.scm % 4) == 0 && (pd.n % 4) == 0 &&
                       ((reinterpret_cast<uintptr_t>(pd.c) & (4 * ES - 1)) == 0);
#pragma unroll
    for (int fm = 0; fm < FM; ++fm) {
      const int gm = m0 + wave_m * WTM + fm * MI + (lane % MI);
      if (gm >= pd.m) continue;
      char* crow = pd.c + (int64_t)gm * pd.scm * ES;
#pragma unroll
      for (int fn = 0; fn < FN; ++fn) {
#pragma unroll
        for (int q = 0; q < ACC / 4; ++q) {
          int nloc = (MI == 32) ? (q * 8 + (lane >> 5) * 4) : ((lane >> 4) * 4);
          const int gn = n0 + wave_n * WTN + fn * MI + nloc;
          f32x4_t v = {acc[fm][fn][q * 4 + 0], acc[fm][fn][q * 4 + 1], acc[fm][fn][q * 4 + 2],
                       acc[fm][fn][q * 4 + 3]};
          if (vec_c) {
            if (gn < pd.n) store4<E>(crow + (int64_t)gn * ES, v);
          } else {
#pragma unroll
            for (int e = 0; e < 4; ++e)
              if (gn + e < pd.n) store1<E>(crow + (int64_t)(gn + e) * pd.scn * ES, v[e]);
          }
        }
      }
    }
  }

  // -------------------------------------------------------------------------------------------
  // `before_store` runs once the K loop is done, before the C stores (the work-stealing scheduler
  // draws its next ticket there).  Split-K runs only on the LDS-DMA tiles: EPI is always EPI_C here.
  template <int EPI, class Hook>
  __device__ static __forceinline__ void run_tile(const ProblemDesc& pd, int tm, int tn, char* smem, bool tf32,
                                                  Hook&& before_store) {
    static_assert(EPI == EPI_C, "the general kernel has no split-K epilogue");
    const int wave = threadIdx.x >> 6;
    const int wave_m = wave / WN, wave_n = wave % WN;
    const int m0 = tm * BM, n0 = tn * BN;
    const bool vec_a = pd.sak == 1 && (pd.k % EPC) == 0 && (pd.sam % EPC) == 0 &&
                       ((reinterpret_cast<uintptr_t>(pd.a) & 15) == 0);
    const bool vec_b = pd.sbn == 1 && (pd.n % EPC) == 0 && (pd.sbk % EPC) == 0 &&
                       ((reinterpret_cast<uintptr_t>(pd.b) & 15) == 0);

    acc_t acc[FM][FN];
#pragma unroll
    for (int fm = 0; fm < FM; ++fm)
#pragma unroll
      for (int fn = 0; fn < FN; ++fn)
#pragma unroll
        for (int i = 0; i < ACC; ++i) acc[fm][fn][i] = 0.0f;

    char* lds0 = smem;
    char* lds1 = smem + STAGE_BYTES;
    const int kt_count = (pd.k + BK - 1) / BK;

    Stage st;
    load_stage(st, pd, vec_a, vec_b, m0, n0, 0, tf32);
    store_stage(st, lds0, lds0 + A_BYTES);
    __syncthreads();
    for (int kt = 0; kt < kt_count; ++kt) {
      char* cur = (kt & 1) ? lds1 : lds0;
      char* nxt = (kt & 1) ? lds0 : lds1;
      const bool more = kt + 1 < kt_count;
      if (more) load_stage(st, pd, vec_a, vec_b, m0, n0, (kt + 1) * BK, tf32);
      compute_stage(acc, cur, cur + A_BYTES, wave_m, wave_n);
      if (more) store_stage(st, nxt, nxt + A_BYTES);
      __syncthreads();
    }
    before_store();
    store_tile(acc, pd, m0, n0, wave_m, wave_n);
  }
};

// ---------------------------------------------------------------------------------------------
// GROUP_M traversal inside one problem (kernels/grouped_gemm.py:354-360).
__device__ __forceinline__ void group_m_order(int local, int m_tiles, int n_tiles, int group_m, int& tm, int& tn) {
  const int width = group_m * n_tiles;
  const int group_id = local / width;
  const int first_m = group_id * group_m;
  const int gsz = min(m_tiles - first_m, group_m);
  tm = first_m + (local % gsz);
  tn = (local % width) / gsz;
}

// Offsets mode: first row and row count of group e, with the offsets clamped to [0, rows] and a
// decreasing offset read as an empty group.
__device__ __forceinline__ int offsets_rows(const KParams& p, int e, int& m) {
  const int lo = e == 0 ? 0 : min(max(p.offs[e - 1], 0), p.rows);
  const int hi = min(max(p.offs[e], 0), p.rows);
  m = hi > lo ? hi - lo : 0;
  return lo;
}

// Generic and offsets modes: s_pref[i] = tile offset of problem first+i, for one chunk of PREFIX
// problems.
template <class T>
__device__ __forceinline__ void load_prefix(const KParams& p, int* s_pref, int* s_tot, int first, int base) {
  constexpr int PER = (T::PREFIX + T::NT - 1) / T::NT;
  int vals[PER];
  int local = 0;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int i = threadIdx.x * PER + j;
    const int prob = first + i;
    int cnt = 0;
    if (i < T::PREFIX && prob < p.G) {
      int m, n;
      if (p.mode == MODE_OFFSETS) {
        offsets_rows(p, prob, m);
        n = p.N;
      } else {
        m = p.dims[prob * 3 + 0];
        n = p.dims[prob * 3 + 1];
      }
      cnt = (m > 0 && n > 0) ? ((m + T::BM - 1) / T::BM) * ((n + T::BN - 1) / T::BN) : 0;
    }
    local += cnt;
    vals[j] = local;
  }
  s_tot[threadIdx.x] = local;
  __syncthreads();
  for (int off = 1; off < T::NT; off <<= 1) {  // Hillis-Steele inclusive scan over NT totals
    const int v = (threadIdx.x >= (unsigned)off) ? s_tot[threadIdx.x - off] : 0;
    __syncthreads();
    s_tot[threadIdx.x] += v;
    __syncthreads();
  }
  const int excl = s_tot[threadIdx.x] - local;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int i = threadIdx.x * PER + j;
    if (i < T::PREFIX) s_pref[i + 1] = base + excl + vals[j];
  }
  if (threadIdx.x == 0) s_pref[0] = base;
  __syncthreads();
}

// Work-stealing tile queues (KParams::queue).  When the grid is a multiple of 8, workgroup b runs
// on XCD b % 8 (round-robin dispatch) and XCD x owns units [lo(x), lo(x + 1)) — a contiguous run,
// so the tiles sharing an expert's B panel stay in one XCD's L2; otherwise one queue owns all
// units.  The `per` workgroups of an XCD take their first units statically (lo(x) + b / 8) and
// draw later ones from ticket counter x (ticket c is unit lo(x) + per + c).  The ticket for
// the next unit is drawn after the current tile's K loop, before its C stores: vector memory
// operations complete in issue order, so an atomic issued earlier would hold up the tile's copy
// waits, while here its latency overlaps the epilogue.  When a queue is drained, wave 0 reads all
// counters at once (one lane each) and moves to the queue with the most units left, so units left
// on a slow XCD are taken by idle ones and a drained workgroup learns that every queue is empty in
// one round trip.  Every workgroup counts itself out after its last claim has returned (two-level
// exit counts, below), and the last one re-arms all counters to zero for the next launch.  Chained
// two-stage tiles draw their ticket earlier, right after the tile's first copies, where the wave's
// next wait is for every copy anyway (see the chained loop of grouped_gemm_kernel).
constexpr int kQueues = 8;
// Counters of the queue buffer, each in a 256-byte block of its own (int32 index = slot *
// kQueueStride): tickets of queue y in slot y, the exit count of the workgroups b with b % 8 == x
// in slot kQueues + x, and the exit count of those eight groups in slot 2 * kQueues.  Device-scope
// atomics are performed at the memory side; counters that shared one cache line serialised every
// claim and exit of a launch there.
constexpr int kQueueStride = 64;
constexpr int kQueueSlots = 2 * kQueues + 1;

struct TileQueue {
  int32_t* q;
  int nx, per, units;
  int cur;           // queue of the last claim (starts at this workgroup's XCD)
  uint32_t drained;  // bit y: queue y has no units left (known to wave 0)

  int lg;            // log2(nx): nx is 8 or 1

  __device__ int lo(int y) const { return (int)(((int64_t)y * units) >> lg); }

  // Wave 0 only (every lane, uniform control flow).  Lane 0 holds `c`, a ticket already drawn from
  // queue `cur`, or -1.  Returns the next unit, or -1 when every queue is drained.  Each round
  // either claims a unit or marks at least one more queue drained, so it ends within nx + 1 rounds.
  __device__ int claim(int c) {
    const int lane = (int)(threadIdx.x & 63);
    for (int round = 0; round <= kQueues; ++round) {
      if (!((drained >> cur) & 1u)) {
        int u = -1;
        if (lane == 0) {
          if (c < 0) c = atomicAdd(q + cur * kQueueStride, 1);
          u = lo(cur) + per + c;
          if (u >= lo(cur + 1)) u = -1;
        }
        u = __builtin_amdgcn_readfirstlane(u);
        c = -1;
        if (u >= 0) return u;
        drained |= 1u << cur;
      }
      int left = 0;
      if (lane < nx && !((drained >> lane) & 1u))
        left = lo(lane + 1) - lo(lane) - per -
               __hip_atomic_load(q + lane * kQueueStride, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      drained |= (uint32_t)__builtin_amdgcn_ballot_w64(lane < nx && left <= 0) & ((1u << nx) - 1u);
      int best = -1, most = 0;
      for (int y = 0; y < nx; ++y) {
        const int l = __builtin_amdgcn_readlane(left, y);
        if (l > most) {
          most = l;
          best = y;
        }
      }
      if (best < 0) return -1;
      cur = best;
    }
    return -1;
  }
};

// Problem and tile coordinates of tile t in a generic or offsets launch (unsplit fields only).  The
// loaded prefix chunk (s_pref, problems chunk_first ..) must cover t: s_pref[0] <= t < s_pref[PREFIX].
template <class T>
__device__ __forceinline__ void searched_tile(const KParams& p, const int* s_pref, int chunk_first, int t,
                                              ProblemDesc& pd, int& tm, int& tn) {
  int lo = 0, hi = T::PREFIX;  // largest i with s_pref[i] <= t
  while (hi - lo > 1) {
    const int mid = (lo + hi) >> 1;
    if (s_pref[mid] <= t) lo = mid; else hi = mid;
  }
  const int e = uniform(chunk_first + lo);
  const int local = uniform(t - s_pref[lo]);
  if (p.mode == MODE_OFFSETS) {
    int m;
    const int row0 = uniform(offsets_rows(p, e, m));
    pd.m = uniform(m); pd.n = p.N; pd.k = p.K;
    pd.sam = p.sam; pd.sak = 1; pd.sbk = p.sbk; pd.sbn = 1; pd.scm = p.scm; pd.scn = 1;
    constexpr int ES = T::ES;
    pd.a = static_cast<const char*>(p.a) + (int64_t)row0 * p.sam * ES;
    pd.b = static_cast<const char*>(p.b) + (int64_t)e * p.sbg * ES;
    pd.c = static_cast<char*>(p.c) + (int64_t)row0 * p.scm * ES;
  } else {
    pd.m = p.dims[e * 3 + 0]; pd.n = p.dims[e * 3 + 1]; pd.k = p.dims[e * 3 + 2];
    const int64_t* s = p.strides + (int64_t)e * 6;
    pd.sam = s[0]; pd.sak = s[1]; pd.sbk = s[2]; pd.sbn = s[3]; pd.scm = s[4]; pd.scn = s[5];
    pd.a = reinterpret_cast<const char*>(p.a_ptrs[e]);
    pd.b = reinterpret_cast<const char*>(p.b_ptrs[e]);
    pd.c = reinterpret_cast<char*>(p.c_ptrs[e]);
  }
  pd.b_stream = p.b_stream;
  const int mt = (pd.m + T::BM - 1) / T::BM, nt = (pd.n + T::BN - 1) / T::BN;
  group_m_order(local, mt, nt, p.group_m, tm, tn);
}

// The three schedule hooks of FastTile::run_tile_chained, as one object.
template <class BeforeBarrier, class Next, class Started>
struct ChainHooks {
  BeforeBarrier before_barrier;
  Next next;
  Started started;
};
template <class BeforeBarrier, class Next, class Started>
__device__ __forceinline__ ChainHooks<BeforeBarrier, Next, Started> chain_hooks(BeforeBarrier b, Next n, Started s) {
  return {b, n, s};
}

// Problem and tile coordinates of tile t in a single or homogeneous launch (unsplit fields only).
template <class T>
__device__ __forceinline__ void simple_tile(const KParams& p, int t, ProblemDesc& pd, int& tm, int& tn) {
  const int mt = (p.M + T::BM - 1) / T::BM, nt = (p.N + T::BN - 1) / T::BN;
  pd.b_stream = p.b_stream;
  if (p.mode == MODE_SINGLE) {
    pd.a = static_cast<const char*>(p.a);
    pd.b = static_cast<const char*>(p.b);
    pd.c = static_cast<char*>(p.c);
    pd.m = p.M; pd.n = p.N; pd.k = p.K;
    pd.sam = p.sam; pd.sak = p.sak; pd.sbk = p.sbk; pd.sbn = p.sbn; pd.scm = p.scm; pd.scn = p.scn;
    group_m_order(t, mt, nt, p.group_m, tm, tn);
  } else {
    const int per = mt * nt;
    const int e = t / per;
    group_m_order(t - e * per, mt, nt, p.group_m, tm, tn);
    pd.a = reinterpret_cast<const char*>(p.a_ptrs[e]);
    pd.b = reinterpret_cast<const char*>(p.b_ptrs[e]);
    pd.c = reinterpret_cast<char*>(p.c_ptrs[e]);
    pd.m = p.M; pd.n = p.N; pd.k = p.K;
    pd.sam = p.K; pd.sak = 1; pd.sbk = p.N; pd.sbn = 1; pd.scm = p.swiglu ? p.N / 2 : p.N; pd.scn = 1;
  }
}

// Stream-K tail of a single or homogeneous launch (KParams::sk_tiles > 0), the body of the stream-K
// kernel.  A launch of T equal tiles on a grid of W workgroups takes ceil(T / W) rounds, so with
// T = R W + r (0 < r < W) its last round leaves W - r workgroups idle: 448 tiles on 256 CUs cost
// two rounds for 1.75 rounds of work.  Here the first T - sk_tiles tiles run whole on the static
// XCD-aware schedule (sk_tiles = r makes that R rounds), and the K slices of the last sk_tiles
// tiles, I = sk_tiles * KT of them, are cut into W runs of I / W consecutive slices (in tile
// order), one per workgroup, so every workgroup ends after R + r / W tile times.  A run that
// covers part of a tile computes that piece and stores it as an fp32 partial (split_store, the
// protocol in which the last arrival reduces and nobody waits); a run that covers a whole tile
// stores C directly.  Runs are numbered XCD-contiguously (run v on XCD v / (W / 8)) so the pieces
// of one tile, and the panels of neighbouring tiles, are read by workgroups of one XCD.
// Bookkeeping, all from integers: slice i of the tail belongs to run floor(((i + 1) W - 1) / I);
// tile j's pieces are runs first(j) .. last(j) (the owners of its first and last slice), piece
// s = v - first(j) is unit s of the tile, and its partial goes to slot v + j: distinct pieces
// (v, j) have distinct sums v + j (both indices grow along the tail), and the pieces of one tile
// take the consecutive slots first(j) + j .. last(j) + j.  The workspace holds W + sk_tiles slots.
template <class T>
__device__ __forceinline__ void streamk_units(const KParams& p, char* smem) {
  const int grid = gridDim.x;
  const int b = (int)blockIdx.x;
  const int main_tiles = p.total_tiles - p.sk_tiles;
  auto describe = [&](int t, ProblemDesc& pd, int& tm, int& tn) {
    simple_tile<T>(p, t, pd, tm, tn);
    pd.swiglu = 0;
    pd.splits = 1;
    pd.split = 0;
    pd.tile = 0;
    pd.slot0 = 0;
    pd.split_wait = 0;  // single protocol: the last piece to arrive reduces, nobody waits
    pd.partials = p.partials;
    pd.counters = p.counters;
  };
  // Whole tiles: the static schedule of the unsplit kernel over the first main_tiles tiles.
  int u = b, u_step = grid, u_end = main_tiles;
  if ((grid & 7) == 0) {
    const int xcd = b & 7, per = grid >> 3;
    u = (int)((int64_t)xcd * main_tiles / 8) + (b >> 3);
    u_step = per;
    u_end = (int)((int64_t)(xcd + 1) * main_tiles / 8);
  }
  for (; u < u_end; u += u_step) {
    ProblemDesc pd;
    int tm, tn;
    describe(u, pd, tm, tn);
    make_uniform(pd);
    T::template run_tile<EPI_EITHER>(pd, uniform(tm), uniform(tn), smem, false, [] {});
  }
  // The tail: run v covers slices [v I / W, (v + 1) I / W).
  const int64_t kt = (p.K + T::BK - 1) / T::BK;
  const int64_t iters = (int64_t)p.sk_tiles * kt;
  const int v = (grid & 7) == 0 ? (b & 7) * (grid >> 3) + (b >> 3) : b;
  int64_t it = (int64_t)v * iters / grid;
  const int64_t end = (int64_t)(v + 1) * iters / grid;
  while (it < end) {
    const int j = (int)(it / kt);
    const int64_t k0 = it - (int64_t)j * kt;
    const int64_t k1 = min(kt, k0 + (end - it));
    const int first = (int)((((int64_t)j * kt + 1) * grid - 1) / iters);
    const int last = (int)((((int64_t)j + 1) * kt * grid - 1) / iters);
    ProblemDesc pd;
    int tm, tn;
    describe(main_tiles + j, pd, tm, tn);
    pd.splits = last - first + 1;
    pd.split = v - first;
    pd.slot0 = first + j;
    pd.tile = j;  // the tile's arrival counter
    const int kb = (int)(k0 * T::BK);
    pd.a += (int64_t)kb * pd.sak * T::ES;
    pd.b += (int64_t)kb * pd.sbk * T::ES;
    pd.k = min((int)((k1 - k0) * T::BK), pd.k - kb);
    make_uniform(pd);
    T::template run_tile<EPI_EITHER>(pd, uniform(tm), uniform(tn), smem, false, [] {});
    it += k1 - k0;
  }
}

// SPLIT: the split-K kernel (units are K ranges of tiles, split_store epilogue).  It is a kernel of
// its own so that the split epilogue's registers do not weigh on the unsplit kernel's loops.
// STREAMK (with SPLIT): the stream-K kernel, a kernel of its own for the same reason.
template <class T, bool SPLIT, bool STREAMK = false>
__global__ void __launch_bounds__(T::NT) __attribute__((amdgpu_waves_per_eu(T::WAVES_PER_EU)))
grouped_gemm_kernel(KParams p) {
  __shared__ __attribute__((aligned(16))) char smem[T::LDS_BYTES];
  if constexpr (STREAMK) {
    static_assert(SPLIT, "stream-K pieces use the split-K epilogue");
    streamk_units<T>(p, smem);
    return;
  }
  int* s_pref = reinterpret_cast<int*>(smem + T::PREFIX_OFFSET);
  int* s_tot = s_pref + T::PREFIX + 1;

  const int grid = gridDim.x;

  int chunk_first = 0;
  const bool searched = p.mode == MODE_GENERIC || p.mode == MODE_OFFSETS;
  if (searched) load_prefix<T>(p, s_pref, s_tot, 0, 0);

  // Units: tile t, K split u / total_tiles (one split outside split-K launches).  Generic and
  // offsets launches whose groups fit one prefix chunk know their exact tile count on the device
  // (offsets mode gets only an upper bound from the host): the schedules partition that.
  const int splits = SPLIT && p.splits > 1 ? p.splits : 1;
  int units = p.total_tiles * splits;
  if (searched && p.G <= T::PREFIX) units = min(units, s_pref[T::PREFIX] * splits);
  const bool stealing = p.queue != nullptr;
  __shared__ int s_next[2];  // unit broadcast, alternating slots so a slow reader never sees the next
  int parity = 0;
  TileQueue tq{};
  // Static schedule.  When the grid is a multiple of 8, workgroup b runs on XCD b % 8 (round-robin
  // dispatch).  Single and homogeneous launches (tiles of equal cost): XCD x owns the contiguous
  // unit range [x * units / 8, (x + 1) * units / 8), which its grid / 8 workgroups walk with stride
  // grid / 8, so every tile of an expert (both M tiles of a B panel, whatever GROUP_M) is computed
  // on one XCD and its B panel is fetched into one L2.  Generic and offsets launches (tiles of
  // unequal cost: ragged groups, partial M tiles) split each round of grid units into eight
  // contiguous runs instead, which spreads every part of the tile space over all XCDs.  Otherwise
  // workgroup b takes units b, b + grid, ...
  int u = blockIdx.x, u_step = grid, u_end = units;
  if ((grid & 7) == 0) {
    const int xcd = (int)blockIdx.x & 7, per = grid >> 3;
    if (searched) {
      u = xcd * per + (int)(blockIdx.x >> 3);
    } else {
      u = (int)((int64_t)xcd * units / 8) + (int)(blockIdx.x >> 3);
      u_step = per;
      u_end = (int)((int64_t)(xcd + 1) * units / 8);
    }
  }
  // Wave 0 claims the next unit (-1: none left) and the workgroup takes it from LDS.
  auto next_unit = [&](int ticket) {
    if (threadIdx.x < 64) {
      const int claimed = tq.claim(ticket);
      if (threadIdx.x == 0) s_next[parity] = claimed;
    }
    __syncthreads();
    u = uniform(s_next[parity]);
    parity ^= 1;
  };
  if (stealing) {
    tq.q = p.queue;
    tq.nx = (grid & 7) == 0 ? kQueues : 1;
    tq.lg = tq.nx == kQueues ? 3 : 0;
    tq.per = grid / tq.nx;
    tq.units = units;
    tq.cur = (int)blockIdx.x & (tq.nx - 1);
    tq.drained = 0;
    u = tq.lo(tq.cur) + (int)blockIdx.x / tq.nx;
    if (u >= tq.lo(tq.cur + 1)) next_unit(-1);  // this XCD has fewer units than workgroups
  }
  // Every workgroup counts itself out of the stealing queues after its last claim has returned, in
  // two levels: into the exit count of its group (b % 8), and the group's last member into the
  // count of groups.  The last group's last member re-arms every counter for the next launch.
  auto count_out = [&] {
    if (stealing && threadIdx.x == 0) {
      const int x = (int)blockIdx.x & 7;
      const int members = (grid - x + 7) >> 3, groups = min(grid, 8);
      if (atomicAdd(p.queue + (kQueues + x) * kQueueStride, 1) == members - 1 &&
          atomicAdd(p.queue + 2 * kQueues * kQueueStride, 1) == groups - 1) {
        for (int y = 0; y < kQueueSlots; ++y) atomicExch(p.queue + y * kQueueStride, 0);
      }
    }
  };
  // CHAIN_OK tiles (two-stage FastTiles, the ping-pong tile) chain their copies across tiles in
  // single, homogeneous and offsets launches; offsets launches only when their groups fit the one
  // prefix chunk loaded above, so locating a tile needs no workgroup barrier.  A tile issues the
  // next unit's first K slices before its own last ones (FastTile::run_tile_chained,
  // PingPongTile::run_tile_chained), so the next unit must be known by then.  The static schedule
  // knows it in advance.  Under work stealing (two-stage FastTiles and the ping-pong tile), lane 0 of
  // wave 0 draws the ticket for the next unit and wave 0 resolves it before a barrier that publishes
  // it to the workgroup: a two-stage tile draws once its slice-1 copies are issued and resolves at
  // its first slice boundary, the ping-pong tile does both just before its prologue barrier.  Each
  // tile claims exactly its successor, as the unchained loop does, only earlier: a workgroup never
  // holds more than one unit ahead, so the last units of a queue still go to whichever workgroups
  // reach them first.  Every ticket is resolved within the tile that drew it, so none is
  // outstanding when the workgroup counts itself out.
  if constexpr (T::CHAIN_OK && !SPLIT) {
    if (!p.swiglu &&
        (p.mode == MODE_SINGLE || p.mode == MODE_HOMOGENEOUS || (p.mode == MODE_OFFSETS && p.G <= T::PREFIX)) &&
        (!stealing || T::CHAIN_STEALING) && (p.K + T::BK - 1) / T::BK <= T::CHAIN_MAX_SLICES &&
        (p.K + T::BK - 1) / T::BK >= T::CHAIN_MIN_SLICES) {
      auto describe = [&](int unit, ProblemDesc& pd, int& tm, int& tn) {
        if (p.mode == MODE_OFFSETS)
          searched_tile<T>(p, s_pref, 0, unit, pd, tm, tn);
        else
          simple_tile<T>(p, unit, pd, tm, tn);
        pd.swiglu = 0;
        pd.splits = 1;
        pd.split = 0;
        pd.tile = unit;
        pd.slot0 = 0;
        pd.split_wait = 0;
        pd.partials = p.partials;
        pd.counters = p.counters;
        make_uniform(pd);
        tm = uniform(tm);
        tn = uniform(tn);
      };
      // The loop is compiled once per schedule, so the static one carries no queue code.
      auto chain_loop = [&](auto steal) {
        constexpr bool STEAL = decltype(steal)::value;
        int ticket = -1;  // lane 0 of wave 0: drawn from queue tq.cur, not yet resolved
        auto hooks = chain_hooks(
            [&] {
              if constexpr (STEAL) {
                if (threadIdx.x < 64) {
                  const int claimed = tq.claim(ticket);
                  if (threadIdx.x == 0) s_next[parity] = claimed;
                  ticket = -1;
                }
              }
            },
            [&](ProblemDesc& next, int& ntm, int& ntn) -> bool {
              if constexpr (STEAL) {
                u = uniform(s_next[parity]);
                parity ^= 1;
              } else {
                u += u_step;
                if (u >= u_end) u = -1;
              }
              if (u < 0) return false;
              describe(u, next, ntm, ntn);
              return true;
            },
            [&] {
              if constexpr (STEAL) {
                if (threadIdx.x == 0 && !((tq.drained >> tq.cur) & 1u))
                  ticket = atomicAdd(tq.q + tq.cur * kQueueStride, 1);
              }
            });
        typename T::Chain ch;
        ch.rot = 0;
        ch.prefetched = false;
        ProblemDesc pd, pdn;
        int tm = 0, tn = 0, tmn = 0, tnn = 0;
        if (STEAL ? u >= 0 : u < u_end) {
          describe(u, pd, tm, tn);
          while (T::run_tile_chained(pd, tm, tn, smem, ch, hooks, pdn, tmn, tnn)) {
            pd = pdn;
            tm = tmn;
            tn = tnn;
          }
        }
      };
      if constexpr (T::CHAIN_STEALING) {
        if (stealing)
          chain_loop(std::true_type{});
        else
          chain_loop(std::false_type{});
      } else {
        chain_loop(std::false_type{});  // the condition above excludes stealing for these tiles
      }
      count_out();
      return;
    }
  }
  while (stealing ? u >= 0 : u < u_end) {
    const int t = u % p.total_tiles;
    ProblemDesc pd;
    int tm, tn;
    if (p.mode == MODE_SINGLE || p.mode == MODE_HOMOGENEOUS) {
      simple_tile<T>(p, t, pd, tm, tn);
    } else {
      // A stolen unit may precede the loaded prefix chunk: restart from the first chunk.
      if (t < s_pref[0]) {
        chunk_first = 0;
        __syncthreads();
        load_prefix<T>(p, s_pref, s_tot, 0, 0);
      }
      // Advance prefix chunks until this tile falls inside the current one (t is block-uniform).
      while (t >= s_pref[T::PREFIX] && chunk_first + T::PREFIX < p.G) {
        const int base = s_pref[T::PREFIX];
        chunk_first += T::PREFIX;
        __syncthreads();
        load_prefix<T>(p, s_pref, s_tot, chunk_first, base);
      }
      if (t >= s_pref[T::PREFIX]) {  // device dims describe fewer tiles than the host count
        if (!stealing) break;
        // Later units of this queue lie past the count too: mark it drained and move on.
        tq.drained |= 1u << tq.cur;
        next_unit(-1);
        continue;
      }
      searched_tile<T>(p, s_pref, chunk_first, t, pd, tm, tn);
    }
    pd.swiglu = p.swiglu;
    pd.splits = splits;
    pd.split = u / p.total_tiles;
    pd.tile = t;
    pd.slot0 = t * splits;
    pd.split_wait = units <= grid ? p.split_polls : 0;
    pd.partials = p.partials;
    pd.counters = p.counters;
    if (splits > 1) {  // this unit's K range: shift A's columns and B's rows, shorten K
      const int k_begin = pd.split * p.k_chunk;
      pd.a += (int64_t)k_begin * pd.sak * T::ES;
      pd.b += (int64_t)k_begin * pd.sbk * T::ES;
      pd.k = min(p.k_chunk, pd.k - k_begin);
    }
    make_uniform(pd);
    int ticket = -1;  // the next unit's ticket: drawn before the C stores, resolved after the tile
    T::template run_tile<SPLIT ? EPI_SPLIT : EPI_C>(pd, uniform(tm), uniform(tn), smem, p.tf32 != 0, [&] {
      if (stealing && threadIdx.x == 0 && !((tq.drained >> tq.cur) & 1u))
        ticket = atomicAdd(tq.q + tq.cur * kQueueStride, 1);
    });
    if (stealing)
      next_unit(ticket);
    else
      u += u_step;
  }
  count_out();
}

}  // namespace moegemm
