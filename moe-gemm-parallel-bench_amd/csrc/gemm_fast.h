// Fast path of the grouped GEMM for 16-bit operands in vector layouts (gfx950).
//
// Same tile semantics, LDS layout and MFMA fragment reads as GemmTile (gemm_kernel.h); what
// differs is how K slices reach LDS:
//  * Each tile builds two buffer resources: the A row panel (num_records = valid rows * row
//    pitch) and the B column panel (base at column n0, num_records up to the end of B).  Rows past
//    M or K fall outside the range and chunks past K (A) or N (B) get an out-of-range offset, so
//    the hardware writes zeros into LDS for every tail element: no branches, no per-element masks.
//  * K slices are copied global -> LDS by buffer_load_dwordx4 ... lds (no VGPR staging).  One
//    wave instruction moves 1 KiB: lane l's 16 bytes land at M0 + 16*l, so each lane fetches the
//    global chunk that the XOR swizzle assigns to its LDS slot.
//  * STAGES LDS buffers form a ring; STAGES-1 slices are in flight while the MFMAs consume the
//    current one.  The copies are issued from inline asm, so the compiler neither sees nor waits
//    on them (its own tracking would put s_waitcnt vmcnt(0) before every ds_read_b64_tr_b16,
//    serialising each K slice behind the newest copies' global-memory latency).  The loop waits
//    explicitly instead: s_waitcnt vmcnt(<copies issued after the slice it needs>) then s_barrier
//    (each wave has seen its own copies land; the barrier makes that true for all waves).  The
//    slice refilled after the barrier is the one every wave finished reading in the previous
//    iteration, so one barrier per K slice suffices.  Compiler memory barriers keep LDS reads
//    from moving across.  No other vector-memory loads are issued while copies are in flight.
//  * Fragment reads for K step kk+1 are issued before the MFMAs of step kk (register double
//    buffering) so the MFMA pipe does not wait on LDS latency inside a slice.
//  * SwiGLU epilogue (packed W13, B = [gate | up] with n = 2F columns): a tile of output columns
//    [n0/2, n0/2 + BN/2) loads the gate columns into the first half of the LDS B row and the
//    matching up columns (F further on) into the second half, so every B row is read as two
//    contiguous runs.  A wave's fragments fn < FN/2 read its WTN/2 gate columns and fragments
//    fn + FN/2 the same output columns' up values, so the epilogue forms silu(gate) * up from the
//    fp32 accumulators in registers and stores F-wide rows.  Needs an even FN and F a multiple of 8
//    (checked by the host).
//  * Split-K units (ProblemDesc::splits > 1: a K range of a split-K tile or a piece of a stream-K
//    tail tile) end with split_store instead of the C store: the fp32 partial tile goes to slot
//    slot0 + split of the caller's workspace with device-coherent (sc1) 16-byte stores, the
//    workgroup waits for them to complete before one atomic increment of the tile's counter, and
//    the unit that brings the counter to `splits` re-arms it (writes 0) and reads all partials of
//    the tile with device-coherent loads, summing them in split order — the same order whichever
//    unit is last, so results are deterministic — then casts and stores C.  No L2 writeback or
//    invalidation is involved (a device-scope fence would write back or invalidate the whole L2
//    of the XCD in every unit).
//  * C epilogue through LDS (STAGED_OK tiles): the 32x32 / 16x16 accumulator layout leaves each
//    lane 4 consecutive columns of one row, so direct stores write 8 bytes per row per lane and one
//    store instruction touches 32 (or 16) rows.  Instead each wave converts its WTM x WTN sub-tile
//    to 16-bit and writes it to the LDS slots that only it fills by DMA (slot j of every stage
//    belongs to wave j % NW: once the wave's own copies have landed and the K loop is over, no
//    other wave reads or writes them), row-major with the 16-byte chunk index XOR-swizzled by the
//    row, then reads it back 16 bytes per lane along rows, so every store instruction writes whole
//    row segments (8 rows x 128 bytes for a 64-column sub-tile).  The next tile's copies into
//    those slots are issued by the same wave after its reads have returned.
// Preconditions (checked by the host before choosing this variant): fp16/bf16, unit inner strides,
// row pitches and the K, N extents multiples of 8 elements, 256 rows of A or C under 2 GiB (their
// resources span one tile's rows, at most 256, and every byte offset in them stays below
// kOutOfRange), and B under 2 GiB (its resource runs to the end of the matrix).  A and C may hold
// any number of rows: each tile's resource base is a 64-bit address.
#pragma once

#include "gemm_kernel.h"

namespace moegemm {

// Raw buffer resource word 3 for gfx9 untyped buffer loads (32-bit data format).
constexpr uint32_t kBufferFlags = 0x00020000u;
constexpr uint32_t kOutOfRange = 0x80000000u;
// Cache-policy operand of the buffer load/store builtins: sc1, device (agent) scope coherence.
constexpr int kDeviceCoherent = 16;
// ... and the non-temporal (streaming) hint.
constexpr int kNonTemporal = 2;

__device__ __forceinline__ void compiler_fence() { asm volatile("" ::: "memory"); }

// Raw buffer resource (V#) for untyped loads: 48-bit base, stride 0, num_records bytes.
__device__ __forceinline__ u32x4_t make_rsrc(const void* base, uint32_t num_records) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  return u32x4_t{(uint32_t)a, (uint32_t)(a >> 32) & 0xffffu, num_records, kBufferFlags};
}

// LDS byte address of a shared-memory pointer (what M0 holds for an LDS-DMA copy).
__device__ __forceinline__ uint32_t lds_address(const void* p) {
  return (uint32_t)reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const char*)(p));
}

// One LDS-DMA copy: every lane reads 16 bytes at rsrc.base + voffset (zero when voffset is past
// num_records) and the wave's 64 x 16 bytes land contiguously at LDS byte address `lds`.  M0
// holds the LDS address; one wait state separates the M0 write from the copy that reads it.
// M0 has no other use in these kernels (gfx9 LDS instructions do not read it).
__device__ __forceinline__ void dma_copy16(u32x4_t rsrc, uint32_t voffset, uint32_t lds) {
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds"
               :
               : "v"(voffset), "s"(rsrc), "s"(lds)
               : "memory", "m0");
#pragma clang diagnostic pop
}

// dma_copy16 with a non-temporal (nt) read: streamed data, evicted first from the caches.
__device__ __forceinline__ void dma_copy16_nt(u32x4_t rsrc, uint32_t voffset, uint32_t lds) {
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tbuffer_load_dwordx4 %0, %1, 0 offen nt lds"
               :
               : "v"(voffset), "s"(rsrc), "s"(lds)
               : "memory", "m0");
#pragma clang diagnostic pop
}

// dma_copy16 with device-coherent (sc1) reads: for data that other workgroups, possibly on other
// XCDs, wrote with sc1 stores (the split-K partials).
__device__ __forceinline__ void dma_copy16_coherent(u32x4_t rsrc, uint32_t voffset, uint32_t lds) {
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tbuffer_load_dwordx4 %0, %1, 0 offen sc1 lds"
               :
               : "v"(voffset), "s"(rsrc), "s"(lds)
               : "memory", "m0");
#pragma clang diagnostic pop
}

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt field is 6 bits");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

template <class E, int BM_, int BN_, int BK_, int WM_, int WN_, int STAGES_>
struct FastTile {
  static_assert(!E::is_f32, "the DMA fast path is for 16-bit operands");
  static constexpr int BM = BM_, BN = BN_, BK = BK_, WM = WM_, WN = WN_, STAGES = STAGES_;
  static constexpr int ES = 2;  // element size in bytes
  static constexpr int NW = WM * WN;
  static constexpr int NT = NW * 64;
  static constexpr int WTM = BM / WM;
  static constexpr int WTN = BN / WN;
  static constexpr int MI = (WTM >= 32 && WTN >= 32) ? 32 : 16;
  static constexpr int MIK = MI == 32 ? 16 : 32;
  static constexpr int KK = BK / MIK;
  static constexpr int FM = WTM / MI;
  static constexpr int FN = WTN / MI;
  static constexpr int ACC = MI * MI / 64;
  static constexpr int CA = BK / 8;  // 16-byte chunks per A row
  static constexpr int CB = BN / 8;  // 16-byte chunks per B row
  static constexpr int A_BYTES = BM * BK * 2;
  static constexpr int B_BYTES = BK * BN * 2;
  static constexpr int STAGE_BYTES = A_BYTES + B_BYTES;
  static constexpr int IA = A_BYTES / 1024;  // 1 KiB DMA issues per stage
  static constexpr int IB = B_BYTES / 1024;
  static constexpr int QA = (IA + NW - 1) / NW;  // A issues per wave (upper bound)
  static constexpr int QB = (IB + NW - 1) / NW;
  static constexpr int XMIN = IA / NW + IB / NW;  // issues per stage every wave makes
  static constexpr int RPA = 64 / CA;             // A rows per issue
  static constexpr int RPB = 64 / CB;             // B rows per issue
  static constexpr int CPW = WTN / 8;             // B chunks per wave column block
  static constexpr bool SWIGLU_OK = FN % 2 == 0;  // gate and up fragments pair up inside a wave
  // Staged C epilogue: 16-bit rows of ROWB bytes, whole rows per 1 KiB slot, and the wave's
  // sub-tile fits the slots it owns (XMIN per stage when every wave issues the same copies).
  static constexpr int ROWB = WTN * 2;
  static constexpr int ROW_CHUNKS = ROWB / 16;
  static constexpr bool STAGED_OK = IA % NW == 0 && IB % NW == 0 && ROWB >= 32 && 1024 % ROWB == 0 &&
                                    WTM * ROWB <= STAGES * XMIN * 1024 && (WTM * ROWB) % 1024 == 0;
  static constexpr int PREFIX = 512;
  static constexpr int PREFIX_OFFSET = STAGES * STAGE_BYTES;
  static constexpr int LDS_BYTES = PREFIX_OFFSET + (PREFIX + 1) * 4 + NT * 4;
  // Two-stage narrow tiles are meant to run two workgroups per CU (one's prologue under the other's
  // work): that needs two waves per SIMD, i.e. at most 256 registers per wave, which the kernel
  // asks the compiler for.  Every other tile takes what it needs.
  static constexpr int WAVES_PER_EU = (STAGES == 2 && 2 * LDS_BYTES <= 160 * 1024 && BM * BN <= 32 * 256) ? 2 : 1;

  static_assert(STAGES >= 2, "need at least double buffering");
  static_assert(A_BYTES % 1024 == 0 && B_BYTES % 1024 == 0, "stages must be whole 1 KiB DMA issues");
  static_assert(CA <= 64 && CB <= 64 && 64 % CA == 0 && 64 % CB == 0, "rows must tile a 1 KiB issue");
  static_assert(CB >= 4, "transpose reads need at least 32 columns");
  static_assert(WTM % MI == 0 && WTN % MI == 0 && BK % MIK == 0, "tile shape");
  static_assert(STAGES * (QA + QB) < 64, "vmcnt budget: every copy in flight must fit the 6-bit counter");
  static_assert(LDS_BYTES <= 160 * 1024, "LDS budget of one CU");

  using acc_t = typename std::conditional<ACC == 16, f32x16_t, f32x4_t>::type;

  struct Dma {
    u32x4_t ra, rb;
    uint32_t a_off[QA];  // byte offset at k0 = 0, or kOutOfRange
    uint32_t a_kch[QA];  // k index of the lane's chunk at k0 = 0
    uint32_t b_off[QB];
    int32_t k;
    uint32_t ldb_bytes;
    uint32_t lds_wave;   // LDS byte address of this wave's first 1 KiB slot in stage 0
    int32_t b_stream;    // B copies non-temporal (ProblemDesc::b_stream)
  };

  __device__ static __forceinline__ void setup_dma(Dma& d, const ProblemDesc& pd, int m0, int n0, const char* smem) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t lda_bytes = (uint32_t)pd.sam * 2u;
    d.ldb_bytes = (uint32_t)pd.sbk * 2u;
    d.k = pd.k;
    d.b_stream = pd.b_stream;
    const int rows = min(BM, pd.m - m0);
    d.ra = make_rsrc(pd.a + (int64_t)m0 * lda_bytes, (uint32_t)rows * lda_bytes);
    if (pd.swiglu)
      d.rb = make_rsrc(pd.b, (uint32_t)pd.k * d.ldb_bytes);
    else
      d.rb = make_rsrc(pd.b + (int64_t)n0 * 2, (uint32_t)pd.k * d.ldb_bytes - (uint32_t)n0 * 2u);
    d.lds_wave = lds_address(smem) + (uint32_t)__builtin_amdgcn_readfirstlane(wave) * 1024u;
#pragma unroll
    for (int q = 0; q < QA; ++q) {
      const int j = wave + q * NW;
      const int r = j * RPA + lane / CA;
      const int pc = lane % CA;
      const int c = pc ^ swz_a(r, CA);
      d.a_kch[q] = (uint32_t)(c * 8);
      d.a_off[q] = (uint32_t)r * lda_bytes + (uint32_t)c * 16u;
    }
#pragma unroll
    for (int q = 0; q < QB; ++q) {
      const int j = wave + q * NW;
      const int r = j * RPB + lane / CB;
      const int pc = lane % CB;
      const int c = pc ^ swz_b(r, CB);
      if (pd.swiglu) {
        // Logical chunk c of the tile: the first half of the row holds the gate columns of output
        // columns [n0/2, n0/2 + BN/2), the second half the matching up columns (F further on), so
        // each B row is read as two contiguous BN-byte runs.
        const int f = pd.n >> 1, half = CB / 2;
        const int ocol = (n0 >> 1) + (c % half) * 8;
        const int gcol = c < half ? ocol : f + ocol;
        d.b_off[q] = ocol < f ? (uint32_t)r * d.ldb_bytes + (uint32_t)gcol * 2u : kOutOfRange;
      } else {
        d.b_off[q] = (n0 + c * 8 < pd.n) ? (uint32_t)r * d.ldb_bytes + (uint32_t)c * 16u : kOutOfRange;
      }
    }
  }

  // Copy K slice [k0, k0 + BK) into LDS stage `stage`.
  // Slot j of a stage is written by wave j % NW; `wave` below is wave-uniform.  NTB fixes B's copy
  // policy at compile time (0 ordinary, 1 non-temporal); -1 reads d.b_stream at run time.
  template <int NTB = -1>
  __device__ static __forceinline__ void issue_stage(const Dma& d, int stage, int k0) {
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t base = d.lds_wave + (uint32_t)(stage * STAGE_BYTES);
#pragma unroll
    for (int q = 0; q < QA; ++q) {
      const int j = wave + q * NW;
      if (IA % NW == 0 || j < IA) {
        const uint32_t off = ((int)d.a_kch[q] + k0 < d.k) ? d.a_off[q] + (uint32_t)k0 * 2u : kOutOfRange;
        dma_copy16(d.ra, off, base + (uint32_t)(q * NW * 1024));
      }
    }
    const uint32_t kstep = (uint32_t)k0 * d.ldb_bytes;
    if constexpr (NTB >= 0)
      issue_b<NTB == 1>(d, base, kstep, wave);
    else if (d.b_stream)
      issue_b<true>(d, base, kstep, wave);
    else
      issue_b<false>(d, base, kstep, wave);
  }

  template <bool NT>
  __device__ static __forceinline__ void issue_b(const Dma& d, uint32_t base, uint32_t kstep, int wave) {
#pragma unroll
    for (int q = 0; q < QB; ++q) {
      const int j = wave + q * NW;
      if (IB % NW == 0 || j < IB) {
        const uint32_t off = d.b_off[q] == kOutOfRange ? kOutOfRange : d.b_off[q] + kstep;
        if constexpr (NT)
          dma_copy16_nt(d.rb, off, base + (uint32_t)(A_BYTES + q * NW * 1024));
        else
          dma_copy16(d.rb, off, base + (uint32_t)(A_BYTES + q * NW * 1024));
      }
    }
  }

  // First LDS column of B fragment fn: the wave's WTN-column block, or under the SwiGLU layout the
  // wave's WTN/2 gate columns (fragments fn < FN/2) and, BN/2 further on, the matching up columns.
  __device__ static __forceinline__ int b_frag_col(int fn, int wave_n, bool swiglu) {
    if (SWIGLU_OK && swiglu)
      return (fn < FN / 2 ? 0 : BN / 2) + wave_n * (WTN / 2) + (fn % (FN / 2 > 0 ? FN / 2 : 1)) * MI;
    return wave_n * WTN + fn * MI;
  }

  __device__ static __forceinline__ void load_frags(i16x8_t (&af)[FM], i16x8_t (&bf)[FN], const char* lds_a,
                                                    const char* lds_b, int kk, int wave_m, int wave_n,
                                                    bool swiglu = false) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int fm = 0; fm < FM; ++fm) {
      const int row = wave_m * WTM + fm * MI + (lane % MI);
      const int c = (kk * MIK) / 8 + lane / MI;
      const int pc = c ^ swz_a(row, CA);
      af[fm] = *reinterpret_cast<const i16x8_t*>(lds_a + (row * CA + pc) * 16);
    }
#pragma unroll
    for (int fn = 0; fn < FN; ++fn) {
      const int g = lane >> 4, s = lane & 15;
      int row, col;
      if constexpr (MI == 32) {
        row = kk * MIK + 8 * (g >> 1) + (s >> 2);
        col = b_frag_col(fn, wave_n, swiglu) + 16 * (g & 1) + 4 * (s & 3);
      } else {
        row = kk * MIK + 8 * g + (s >> 2);
        col = b_frag_col(fn, wave_n, swiglu) + 4 * (s & 3);
      }
      const int pc = (col >> 3) ^ swz_b(row, CB);
      const char* p0 = lds_b + (row * CB + pc) * 16 + (col & 7) * 2;
      const char* p1 = p0 + 4 * CB * 16;
      i16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) i16x4_t*)(p0));
      i16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) i16x4_t*)(p1));
      bf[fn] = i16x8_t{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    }
  }

  __device__ static __forceinline__ void mfmas(acc_t (&acc)[FM][FN], const i16x8_t (&af)[FM], const i16x8_t (&bf)[FN]) {
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

  // MFMAs of fragment columns [fm0, fm1) of one K step.
  template <int FM0, int FM1>
  __device__ static __forceinline__ void mfma_rows(acc_t (&acc)[FM][FN], const i16x8_t (&af)[FM],
                                                   const i16x8_t (&bf)[FN]) {
#pragma unroll
    for (int fm = FM0; fm < FM1; ++fm)
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

  // Scheduling hints: interleave `mfma` MFMAs with `ds` LDS reads and `vm` DMA issues.
  template <int NMFMA, int NDS, int NVM>
  __device__ static __forceinline__ void interleave() {
    constexpr int vm_per = NMFMA > 0 ? (NVM + NMFMA - 1) / NMFMA : 0;
    constexpr int ds_per = NMFMA > 0 ? (NDS + NMFMA - 1) / NMFMA : 0;
#pragma unroll
    for (int i = 0; i < NMFMA; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
      if constexpr (vm_per > 0) __builtin_amdgcn_sched_group_barrier(0x020, vm_per, 0);  // VMEM reads
      if constexpr (ds_per > 0) __builtin_amdgcn_sched_group_barrier(0x100, ds_per, 0);  // LDS reads
    }
  }

  // silu(x) = x * sigmoid(x) = x / (1 + e^-x), with the hardware reciprocal (1 ulp) in place of an
  // IEEE divide: the result is rounded to 16 bits, far coarser than either error.
  __device__ static __forceinline__ float silu(float x) { return x * __builtin_amdgcn_rcpf(1.0f + __expf(-x)); }

  // Split-K reduction through LDS: after the K loop the DMA ring is free, and each wave takes
  // RED_SLOTS 1 KiB slots of it.  The wave's share of one partial is RED_CH 1 KiB chunks (each lane
  // fetches the 16 bytes of its own accumulator chunk, landing at slot + 16 * lane).  A chunk range
  // is reduced in rounds: each round copies as many (split, chunk) pairs as fit RED_CAP slots per
  // wave, waits once, and adds them from LDS, so many partials share one memory round trip.  The sum
  // of every element runs in split order, whichever unit reduces it.  KEEP_OWN tiles add their own
  // partial from the accumulators; larger tiles read it back like the others, so that the
  // accumulators are dead and the registers free.
  static constexpr int RED_CH = FM * FN * (ACC / 4);
  static constexpr int RED_SLOTS = (STAGES * STAGE_BYTES / NW) / 1024;
  static constexpr int RED_CAP = RED_SLOTS < 48 ? RED_SLOTS : 48;
  static constexpr bool KEEP_OWN = 2 * FM * FN * ACC <= 160;
  static_assert(RED_CAP >= 1, "at least one 1 KiB slot per wave for the split-K reduction");
  // Shared reductions (split_store): at most this many splits, and only when one unit would read at
  // least this many chunks per wave of the other units' partials; below that the extra round trips
  // of waiting cost more than the reads they spread.
  static constexpr int kSharedMaxSplits = 16;
  static constexpr int kSharedMinChunks = 48;

  // Byte offset, inside one partial tile, of this lane's 16-byte accumulator chunk c (= (fm * FN +
  // fn) * ACC / 4 + q).  Partials are private scratch, laid out in accumulator order
  // [wave][chunk][lane][4 floats]: each wave's store or load of one chunk is one contiguous 1 KiB
  // access (a row-major tile would give every instruction 16 bytes in each of 32 rows).  Every unit
  // of a tile runs the same tile, so chunk (wave, c) holds the same output elements in every split's
  // partial.
  __device__ static __forceinline__ int chunk_offset(int c, int wave) {
    const int lane = threadIdx.x & 63;
    return ((wave * RED_CH + c) * 64 + lane) * 16;
  }

  // Sums chunks [lo, hi) of every split's partial (split order) and stores them to C.
  __device__ static __forceinline__ void reduce_chunks(const acc_t (&acc)[FM][FN], const ProblemDesc& pd, int m0,
                                                       int n0, int wave_m, int wave_n, char* smem, int lo, int hi) {
    constexpr uint32_t kSlotBytes = BM * BN * 4;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int splits = pd.splits;
    char* region = smem + wave * RED_SLOTS * 1024;
    const uint32_t region_lds = lds_address(region);
    acc_t tot[FM][FN];
#pragma unroll
    for (int fm = 0; fm < FM; ++fm)
#pragma unroll
      for (int fn = 0; fn < FN; ++fn)
#pragma unroll
        for (int i = 0; i < ACC; ++i) tot[fm][fn][i] = 0.0f;
    // Rounds of `per` chunks x `ways` splits (at most RED_CAP copies in flight per wave).
    const int per = min(hi - lo, RED_CAP), ways = max(1, RED_CAP / per);
    for (int c0 = lo; c0 < hi; c0 += per) {
      const int cn = min(per, hi - c0);
      for (int g0 = 0; g0 < splits; g0 += ways) {
        const int count = min(ways, splits - g0);
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the previous round's LDS reads are done
        for (int r = 0; r < count; ++r) {
          if (KEEP_OWN && g0 + r == pd.split) continue;
          const u32x4_t rs = make_rsrc(pd.partials + ((int64_t)pd.slot0 + g0 + r) * (BM * BN), kSlotBytes);
          for (int i = 0; i < cn; ++i)
            dma_copy16_coherent(rs, (uint32_t)chunk_offset(c0 + i, wave), region_lds + (uint32_t)((r * per + i) * 1024));
        }
        wait_vmcnt<0>();
        compiler_fence();
#pragma unroll
        for (int fm = 0; fm < FM; ++fm)
#pragma unroll
          for (int fn = 0; fn < FN; ++fn)
#pragma unroll
            for (int q = 0; q < ACC / 4; ++q) {
              const int c = (fm * FN + fn) * (ACC / 4) + q;
              if (c < c0 || c >= c0 + cn) continue;
              for (int r = 0; r < count; ++r) {
                f32x4_t v;
                if (KEEP_OWN && g0 + r == pd.split)
                  v = f32x4_t{acc[fm][fn][q * 4 + 0], acc[fm][fn][q * 4 + 1], acc[fm][fn][q * 4 + 2],
                              acc[fm][fn][q * 4 + 3]};
                else
                  v = *reinterpret_cast<const f32x4_t*>(region + (r * per + (c - c0)) * 1024 + lane * 16);
#pragma unroll
                for (int i = 0; i < 4; ++i) tot[fm][fn][q * 4 + i] += v[i];
              }
            }
        compiler_fence();
      }
    }
#pragma unroll
    for (int fm = 0; fm < FM; ++fm) {
      const int gm = m0 + wave_m * WTM + fm * MI + (lane % MI);
      char* crow = pd.c + (int64_t)gm * pd.scm * 2;
#pragma unroll
      for (int fn = 0; fn < FN; ++fn)
#pragma unroll
        for (int q = 0; q < ACC / 4; ++q) {
          const int c = (fm * FN + fn) * (ACC / 4) + q;
          if (c < lo || c >= hi) continue;
          const int cl = wave_n * WTN + fn * MI + ((MI == 32) ? (q * 8 + (lane >> 5) * 4) : ((lane >> 4) * 4));
          if (gm >= pd.m || n0 + cl >= pd.n) continue;
          const f32x4_t v = {tot[fm][fn][q * 4 + 0], tot[fm][fn][q * 4 + 1], tot[fm][fn][q * 4 + 2],
                             tot[fm][fn][q * 4 + 3]};
          store4<E>(crow + (int64_t)(n0 + cl) * 2, v);
        }
    }
  }

  // Split-K epilogue of one unit.  The unit stores its fp32 partial (device-coherent sc1 stores),
  // waits for them, and arrives at the tile's counter, one int32 per tile.  Then one of two
  // protocols, the same for every unit of the tile:
  //  * single (few chunks to read, or the units of the launch share workgroups, pd.split_wait 0):
  //    the last unit to arrive reduces the whole tile and re-arms the counter to zero;
  //  * shared: the tile's chunks form `splits` slices (slice s = chunks [s RED_CH / S,
  //    (s + 1) RED_CH / S)), and unit s reduces slice s once every unit has arrived.  Counter
  //    fields: arrivals (bits 0-7), a mask of units that stopped waiting (bits 8-23) and departures
  //    (bits 24-31).  A unit that is not the last to arrive polls the counter up to pd.split_wait
  //    times, each after a sleep of about 1000 cycles (the host's default of 16 polls waits some
  //    20-30 us); if the others have still not arrived, it sets its bit with a compare-and-swap that
  //    succeeds only while arrivals are short, and leaves its slice.  The last unit to arrive reads
  //    the mask in the value its arrival returned (every bit was set before that arrival) and
  //    reduces those slices as well as its own, so every slice is reduced exactly once.  Each unit
  //    then departs, and the unit whose departure completes the count re-arms the counter.
  // Launches and graph replays need no memset.
  __device__ static __forceinline__ void split_store(const acc_t (&acc)[FM][FN], const ProblemDesc& pd, int m0,
                                                     int n0, int wave_m, int wave_n, char* smem) {
    __shared__ uint32_t s_work;  // bit s: reduce slice s; bit 31: reduce the whole tile
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int splits = pd.splits;
    const auto mine = __builtin_amdgcn_make_buffer_rsrc(pd.partials + ((int64_t)pd.slot0 + pd.split) * (BM * BN),
                                                        (short)0, (int)(BM * BN * 4), (int)kBufferFlags);
#pragma unroll
    for (int fm = 0; fm < FM; ++fm)
#pragma unroll
      for (int fn = 0; fn < FN; ++fn)
#pragma unroll
        for (int q = 0; q < ACC / 4; ++q) {
          const f32x4_t v = {acc[fm][fn][q * 4 + 0], acc[fm][fn][q * 4 + 1], acc[fm][fn][q * 4 + 2],
                             acc[fm][fn][q * 4 + 3]};
          __builtin_amdgcn_raw_buffer_store_b128(v, mine, chunk_offset((fm * FN + fn) * (ACC / 4) + q, wave), 0,
                                                 kDeviceCoherent);
        }
    // The partials are device-coherent (sc1) stores, the encoding of relaxed agent-scope atomic
    // stores: once this wave's stores have completed they are visible to sc1 loads from any XCD,
    // so no L2 writeback (release fence) is needed.  The barrier makes every wave's stores complete
    // before the counter moves.
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    const bool shared = pd.split_wait > 0 && splits <= kSharedMaxSplits && RED_CH * (splits - 1) >= kSharedMinChunks;
    int32_t* word = pd.counters + pd.tile;
    if (threadIdx.x == 0) {
      const uint32_t old = (uint32_t)atomicAdd(word, 1);
      const bool last = (int)(old & 0xffu) == splits - 1;
      uint32_t work = 0;
      if (!shared) {
        if (last) {
          atomicExch(word, 0);
          work = 1u << 31;
        }
      } else if (last) {
        work = ((old >> 8) & 0xffffu) | (1u << pd.split);
      } else {
        work = 1u << pd.split;
        uint32_t w = 0;
        for (int poll = 0;; ++poll) {
          __builtin_amdgcn_s_sleep(16);
          w = (uint32_t)__hip_atomic_load(word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          if ((int)(w & 0xffu) >= splits || poll + 1 >= pd.split_wait) break;
        }
        // Stop waiting: set this unit's bit while arrivals are still short.  Each failed
        // compare-and-swap means another arrival or another unit's bit changed the word, at most
        // 2 x splits times.
        while ((int)(w & 0xffu) < splits) {
          const uint32_t seen = (uint32_t)atomicCAS(word, (int)w, (int)(w | (1u << (8 + pd.split))));
          if (seen == w) {
            work = 0;
            break;
          }
          w = seen;
        }
      }
      s_work = work;
    }
    __syncthreads();
    // Every partial of the tile has completed once this unit has work: its sc1 loads see them (no
    // L2 invalidation, acquire fence, is needed).
    const uint32_t work = (uint32_t)uniform((int32_t)s_work);
    if (work >> 31) {
      reduce_chunks(acc, pd, m0, n0, wave_m, wave_n, smem, 0, RED_CH);
    } else if (work) {
      for (int sl = 0; sl < splits; ++sl) {
        const int lo = sl * RED_CH / splits, hi = (sl + 1) * RED_CH / splits;
        if (((work >> sl) & 1u) && lo < hi) reduce_chunks(acc, pd, m0, n0, wave_m, wave_n, smem, lo, hi);
      }
    }
    if (shared && threadIdx.x == 0 && (int)(((uint32_t)atomicAdd(word, 1 << 24) >> 24) & 0xffu) == splits - 1)
      atomicExch(word, 0);
    // Each wave reduced through a contiguous LDS region of its own, which is not the slot ownership
    // of the copies: the workgroup's next unit must not issue its first copies (into other waves'
    // regions) until every wave has finished reading.
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __syncthreads();
  }

  // LDS byte offset (from the tile's LDS base) of the s-th 1 KiB slot this wave fills by DMA:
  // per stage, its A slots then its B slots, in issue order.
  __device__ static __forceinline__ int owned_slot(int s, int wave) {
    constexpr int PA = IA / NW;
    const int stage = s / XMIN, t = s % XMIN;
    return stage * STAGE_BYTES + (t < PA ? (wave + t * NW) * 1024 : A_BYTES + (wave + (t - PA) * NW) * 1024);
  }

  // Staged C epilogue (see the header comment).  Row r of the wave's sub-tile occupies bytes
  // [r * ROWB, (r + 1) * ROWB) of its slot sequence; 16-byte chunk c of the row sits at c ^ (r % ROW_CHUNKS).
  __device__ static __forceinline__ void staged_store(const acc_t (&acc)[FM][FN], const ProblemDesc& pd, int m0,
                                                      int n0, int wave_m, int wave_n, char* smem) {
    static_assert(STAGED_OK, "tile cannot stage its C sub-tile");
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    // The caller has waited for this wave's copies (the zero-filled slices past K included).
#pragma unroll
    for (int fm = 0; fm < FM; ++fm) {
      const int r = fm * MI + (lane % MI);
#pragma unroll
      for (int fn = 0; fn < FN; ++fn)
#pragma unroll
        for (int q = 0; q < ACC / 4; ++q) {
          const int c = fn * MI + ((MI == 32) ? (q * 8 + (lane >> 5) * 4) : ((lane >> 4) * 4));
          const int lin = r * ROWB + (((c >> 3) ^ (r % ROW_CHUNKS)) << 4) + (c & 7) * 2;
          const f32x4_t v = {acc[fm][fn][q * 4 + 0], acc[fm][fn][q * 4 + 1], acc[fm][fn][q * 4 + 2],
                             acc[fm][fn][q * 4 + 3]};
          store4_lds<E>(smem + owned_slot(lin >> 10, wave) + (lin & 1023), v);
        }
    }
    compiler_fence();
    const bool c16 = ((reinterpret_cast<uintptr_t>(pd.c) & 15) == 0) && (pd.scm & 7) == 0;
    constexpr int RPI = 1024 / ROWB;  // rows per 1 KiB read
#pragma unroll
    for (int j = 0; j < WTM * ROWB / 1024; ++j) {
      const int r = j * RPI + lane / ROW_CHUNKS, chunk = lane % ROW_CHUNKS;
      const u32x4_t v = *reinterpret_cast<const u32x4_t*>(smem + owned_slot(j, wave) +
                                                          (r % RPI) * ROWB + ((chunk ^ (r % ROW_CHUNKS)) << 4));
      const int gm = m0 + wave_m * WTM + r, gn = n0 + wave_n * WTN + chunk * 8;
      if (gm < pd.m && gn < pd.n) {
        char* dst = pd.c + ((int64_t)gm * pd.scm + gn) * 2;
        if (c16) {
          // A wave's row segment covers whole 128-byte lines when ROWB >= 128.  Such lines are
          // written once and never re-read by the launch, so non-temporal stores stream them
          // through L2 instead of evicting the A and B panels that other workgroups of the XCD
          // are about to re-read.  DSV3 TP W2 at M_e = 512 writes 1.9 GB of C per launch; its
          // measured HBM fetch fell from 1.88 to 1.37 GB with these stores.  Narrower segments
          // stay in L2 until the neighbouring wave completes the line.
          if constexpr (ROWB >= 128) __builtin_nontemporal_store(v, MOEGEMM_GLOBAL(u32x4_t, dst));
          else *MOEGEMM_GLOBAL(u32x4_t, dst) = v;
        } else {
          *MOEGEMM_GLOBAL(u32x2_t, dst) = u32x2_t{v[0], v[1]};
          *MOEGEMM_GLOBAL(u32x2_t, dst + 8) = u32x2_t{v[2], v[3]};
        }
      }
    }
  }

  // Stores the tile (C, the SwiGLU output, or split-K partials; see Epilogue).  The wave's copies
  // must have landed (the staged epilogue reuses its LDS slots).
  template <int EPI = EPI_C>
  __device__ static __forceinline__ void store_tile(const acc_t (&acc)[FM][FN], const ProblemDesc& pd, int m0,
                                                    int n0, int wave_m, int wave_n, char* smem) {
    const int lane = threadIdx.x & 63;
    if constexpr (EPI == EPI_SPLIT) {
      split_store(acc, pd, m0, n0, wave_m, wave_n, smem);
      return;
    } else if constexpr (EPI == EPI_EITHER) {
      if (pd.splits > 1) {  // a piece; a whole tile takes the regular epilogue below
        split_store(acc, pd, m0, n0, wave_m, wave_n, smem);
        return;
      }
    }
    if constexpr (SWIGLU_OK) {
      if (pd.swiglu) {
        const int f = pd.n >> 1;
#pragma unroll
        for (int fm = 0; fm < FM; ++fm) {
          const int gm = m0 + wave_m * WTM + fm * MI + (lane % MI);
          if (gm >= pd.m) continue;
          char* crow = pd.c + (int64_t)gm * pd.scm * 2;
#pragma unroll
          for (int fn = 0; fn < FN / 2; ++fn) {
#pragma unroll
            for (int q = 0; q < ACC / 4; ++q) {
              const int nloc = (MI == 32) ? (q * 8 + (lane >> 5) * 4) : ((lane >> 4) * 4);
              const int gn = (n0 >> 1) + wave_n * (WTN / 2) + fn * MI + nloc;
              if (gn < f) {
                f32x4_t v;
#pragma unroll
                for (int i = 0; i < 4; ++i) v[i] = silu(acc[fm][fn][q * 4 + i]) * acc[fm][fn + FN / 2][q * 4 + i];
                store4<E>(crow + (int64_t)gn * 2, v);
              }
            }
          }
        }
        return;
      }
    } else {
      if (pd.swiglu) return;  // the host never selects this tile for the epilogue; store nothing
    }
    if constexpr (STAGED_OK) {
      staged_store(acc, pd, m0, n0, wave_m, wave_n, smem);
      return;
    }
#pragma unroll
    for (int fm = 0; fm < FM; ++fm) {
      const int gm = m0 + wave_m * WTM + fm * MI + (lane % MI);
      if (gm >= pd.m) continue;
      char* crow = pd.c + (int64_t)gm * pd.scm * 2;
#pragma unroll
      for (int fn = 0; fn < FN; ++fn) {
#pragma unroll
        for (int q = 0; q < ACC / 4; ++q) {
          const int nloc = (MI == 32) ? (q * 8 + (lane >> 5) * 4) : ((lane >> 4) * 4);
          const int gn = n0 + wave_n * WTN + fn * MI + nloc;
          if (gn < pd.n) {
            f32x4_t v = {acc[fm][fn][q * 4 + 0], acc[fm][fn][q * 4 + 1], acc[fm][fn][q * 4 + 2],
                         acc[fm][fn][q * 4 + 3]};
            store4<E>(crow + (int64_t)gn * 2, v);
          }
        }
      }
    }
  }

  // `before_store` runs once every copy has landed, before the epilogue barrier and the C stores
  // (a global atomic issued there overlaps them instead of delaying the in-order copy waits).
  // EPI: the unit's epilogue (Epilogue; EPI_SPLIT for one K range of a split-K tile).
  template <int EPI, class Hook>
  __device__ static __forceinline__ void run_tile(const ProblemDesc& pd, int tm, int tn, char* smem, bool,
                                                  Hook&& before_store) {
    static_assert(KK % 2 == 0, "fragment double buffer alternates by K step");
    constexpr int HALF = FM / 2 > 0 ? FM / 2 : 1;  // fragment rows issued before the mid-slice barrier
    constexpr int NDS = FM + 2 * FN;                 // LDS reads per K step
    constexpr int NVM = QA + QB;                      // DMA issues per slice (upper bound per wave)
    const int wave = threadIdx.x >> 6;
    const int wave_m = wave / WN, wave_n = wave % WN;
    const int m0 = tm * BM, n0 = tn * BN;
    Dma d;
    setup_dma(d, pd, m0, n0, smem);

    acc_t acc[FM][FN];
#pragma unroll
    for (int fm = 0; fm < FM; ++fm)
#pragma unroll
      for (int fn = 0; fn < FN; ++fn)
#pragma unroll
        for (int i = 0; i < ACC; ++i) acc[fm][fn][i] = 0.0f;

    // Prologue: slices 0..STAGES-1 in flight, then slice 0 resident and its first fragments read.
    // Slices at or past K read out of range and land as zeros, so every copy is unconditional.
#pragma unroll
    for (int s = 0; s < STAGES; ++s) issue_stage(d, s, s * BK);
    wait_vmcnt<(STAGES - 1) * XMIN>();
    compiler_fence();
    __builtin_amdgcn_s_barrier();
    compiler_fence();
    i16x8_t af[2][FM], bf[2][FN];
    load_frags(af[0], bf[0], smem, smem + A_BYTES, 0, wave_m, wave_n, pd.swiglu != 0);

    const int kt_count = (pd.k + BK - 1) / BK;
    for (int kt = 0; kt < kt_count; ++kt) {
      const char* cur = smem + (kt % STAGES) * STAGE_BYTES;
      const char* nxt = smem + ((kt + 1) % STAGES) * STAGE_BYTES;
#pragma unroll
      for (int kk = 0; kk < KK - 1; ++kk) {
        load_frags(af[(kk + 1) & 1], bf[(kk + 1) & 1], cur, cur + A_BYTES, kk + 1, wave_m, wave_n,
                   pd.swiglu != 0);
        mfma_rows<0, FM>(acc, af[kk & 1], bf[kk & 1]);
        interleave<FM * FN, NDS, 0>();
      }
      constexpr int L = (KK - 1) & 1;
      // Last K step: first half of its MFMAs, then slice kt+1 becomes readable (this wave's copies
      // landed, then every wave's), the drained buffer of slice kt is refilled with slice
      // kt+STAGES, and slice kt+1's first fragments load under the second half of the MFMAs.
      mfma_rows<0, HALF>(acc, af[L], bf[L]);
      wait_vmcnt<(STAGES - 2) * XMIN>();
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      compiler_fence();
      __builtin_amdgcn_s_barrier();
      compiler_fence();
      issue_stage(d, kt % STAGES, (kt + STAGES) * BK);
      load_frags(af[0], bf[0], nxt, nxt + A_BYTES, 0, wave_m, wave_n, pd.swiglu != 0);
      mfma_rows<HALF, FM>(acc, af[L], bf[L]);
      interleave<(FM - HALF) * FN, NDS, NVM>();
    }
    // All copies (including the out-of-range tail slices) landed and every wave is done reading
    // LDS before the next tile's prologue refills it.
    wait_vmcnt<0>();
    before_store();
    compiler_fence();
    __builtin_amdgcn_s_barrier();
    compiler_fence();
    store_tile<EPI>(acc, pd, m0, n0, wave_m, wave_n, smem);
  }

  // Cross-tile chaining of the two-stage tiles.  A workgroup on the static schedule knows its next
  // unit.  So the copy that would fill the drained buffer with a zero slice past K fetches the next
  // tile's slice 0 instead, and the next tile starts with that slice in flight.  It sits in the
  // buffer after this tile's last one: buffer roles rotate by the K slice count at every tile.  This
  // tile's C then leaves with exactly CHAIN_STORES buffer stores per wave, every lane active;
  // out-of-range lanes are dropped by the range check.  A wave's vector memory operations complete
  // in issue order, so the next tile knows its slice 0 has landed once at most CHAIN_STORES
  // operations are outstanding.  It does not wait for the stores themselves.  Staged tiles stage C
  // through the wave's slots in the last slice's buffer (the other one holds the prefetch), in
  // rounds of CH_ROWS rows.  Workgroup tiles over 32768 outputs are left out: the chained loop
  // made them spill (the 8-wave 256x256x64 tile from 7 to about 200 spilled VGPRs).  Tiles with
  // more than 64 accumulator registers per wave chain only short-K launches (CHAIN_MAX_SLICES):
  // 64x512x64 gained 8 % at K = 256 (4 slices) and lost 2-3 % at K = 2048 (32 slices).
  //
  // Four-stage tiles of at most 32768 outputs and 64 accumulator registers per wave chain deeper,
  // on the static schedule (run_tile_chained_deep): the last STAGES - 1 refills of a tile fetch the
  // next tile's slices 0 .. STAGES - 2, and its slice STAGES - 1 follows the C stores, so the next
  // tile starts with STAGES slices in flight as an unchained tile's prologue would have them.  A
  // two-stage tile can prefetch only one slice, which leaves one slice's memory latency exposed at
  // every tile: short-K launches (DSV3 TP W2, K = 256, four 64-deep slices per tile) paid it 4 times
  // per 4 slices.
  // Deep chaining is kept to launches of STAGES to 8 slices: with fewer the tile has no slice
  // boundary to prefetch from, and on long-K launches (32 slices) it measured 1-2 % slower than
  // run_tile's own prologue.
  static constexpr bool CHAIN_DEEP = STAGES == 4 && FM * FN * ACC <= 64 && BM * BN <= 32768;
  static constexpr bool CHAIN_OK = (STAGES == 2 && FM * FN * ACC <= 128 && BM * BN <= 32768) || CHAIN_DEEP;
  static constexpr int CHAIN_MIN_SLICES = CHAIN_DEEP ? STAGES : 1;
  static constexpr int CHAIN_MAX_SLICES = CHAIN_DEEP ? 8 : FM * FN * ACC <= 64 ? (1 << 30) : 8;
  static constexpr bool CHAIN_STEALING = STAGES == 2;  // the two-stage loop also runs the stealing schedule
  static constexpr int CH_ROWS_FIT = STAGED_OK ? (XMIN * 1024 / ROWB) / MI * MI : MI;
  static constexpr int CH_ROWS = CH_ROWS_FIT < WTM ? CH_ROWS_FIT : WTM;  // staged rows per round
  static constexpr int CHAIN_STORES = STAGED_OK ? WTM * ROWB / 1024 : FM * FN * (ACC / 4);
  static_assert(!CHAIN_OK || CHAIN_STORES + (STAGES - 1) * (QA + QB) < 64,
                "outstanding operations must fit the 6-bit vmcnt");
  static_assert(!(CHAIN_OK && STAGED_OK) || (CH_ROWS > 0 && WTM % CH_ROWS == 0 && (CH_ROWS * ROWB) % 1024 == 0),
                "staging rounds must cover the wave tile in whole slots");
  struct Chain {
    int rot;          // LDS buffer holding the slice 0 the previous tile issued
    bool prefetched;  // false: the next tile issues its own prologue
  };

  // Direct C stores with a fixed instruction count per wave: CHAIN_STORES 8-byte buffer stores.
  __device__ static __forceinline__ void store_tile_counted(const acc_t (&acc)[FM][FN], const ProblemDesc& pd,
                                                            int m0, int n0, int wave_m, int wave_n) {
    const int lane = threadIdx.x & 63;
    const int rows = min(BM, pd.m - m0);
    const auto rc = __builtin_amdgcn_make_buffer_rsrc(pd.c + (int64_t)m0 * pd.scm * 2, (short)0,
                                                      (int)((uint32_t)rows * (uint32_t)pd.scm * 2u), (int)kBufferFlags);
#pragma unroll
    for (int fm = 0; fm < FM; ++fm) {
      const int rl = wave_m * WTM + fm * MI + (lane % MI);
#pragma unroll
      for (int fn = 0; fn < FN; ++fn)
#pragma unroll
        for (int q = 0; q < ACC / 4; ++q) {
          const int nloc = (MI == 32) ? (q * 8 + (lane >> 5) * 4) : ((lane >> 4) * 4);
          const int gn = n0 + wave_n * WTN + fn * MI + nloc;
          const uint32_t off =
              (rl < rows && gn < pd.n) ? ((uint32_t)rl * (uint32_t)pd.scm + (uint32_t)gn) * 2u : kOutOfRange;
          const f32x4_t v = {acc[fm][fn][q * 4 + 0], acc[fm][fn][q * 4 + 1], acc[fm][fn][q * 4 + 2],
                             acc[fm][fn][q * 4 + 3]};
          __builtin_amdgcn_raw_buffer_store_b64(pack4<E>(v), rc, (int)off, 0, 0);
        }
    }
  }

  // Staged C stores with a fixed instruction count per wave: the wave's sub-tile in rounds of
  // CH_ROWS rows through its XMIN slots of LDS buffer `stage` (layout as in staged_store), each
  // round's rows leaving as 16-byte buffer stores along the rows: CHAIN_STORES in all.  Needs a
  // 16-byte aligned C with a row pitch of a multiple of 8 elements.
  __device__ static __forceinline__ void staged_store_counted(const acc_t (&acc)[FM][FN], const ProblemDesc& pd,
                                                              int m0, int n0, int wave_m, int wave_n, char* smem,
                                                              int stage) {
    static_assert(STAGED_OK, "tile cannot stage its C sub-tile");
    constexpr int FMR = CH_ROWS / MI;  // fragment rows per round
    constexpr int RPI = 1024 / ROWB;   // rows per 1 KiB read
    // Full 128-byte lines stream through L2 as non-temporal stores (as in staged_store).
    constexpr int kAux = ROWB >= 128 ? kNonTemporal : 0;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int rows = min(BM, pd.m - m0);
    const auto rc = __builtin_amdgcn_make_buffer_rsrc(pd.c + (int64_t)m0 * pd.scm * 2, (short)0,
                                                      (int)((uint32_t)rows * (uint32_t)pd.scm * 2u), (int)kBufferFlags);
#pragma unroll
    for (int rd = 0; rd < WTM / CH_ROWS; ++rd) {
#pragma unroll
      for (int f = 0; f < FMR; ++f) {
        const int fm = rd * FMR + f;
        const int r = f * MI + (lane % MI);
#pragma unroll
        for (int fn = 0; fn < FN; ++fn)
#pragma unroll
          for (int q = 0; q < ACC / 4; ++q) {
            const int c = fn * MI + ((MI == 32) ? (q * 8 + (lane >> 5) * 4) : ((lane >> 4) * 4));
            const int lin = r * ROWB + (((c >> 3) ^ (r % ROW_CHUNKS)) << 4) + (c & 7) * 2;
            const f32x4_t v = {acc[fm][fn][q * 4 + 0], acc[fm][fn][q * 4 + 1], acc[fm][fn][q * 4 + 2],
                               acc[fm][fn][q * 4 + 3]};
            store4_lds<E>(smem + owned_slot(stage * XMIN + (lin >> 10), wave) + (lin & 1023), v);
          }
      }
      compiler_fence();
#pragma unroll
      for (int j = 0; j < CH_ROWS * ROWB / 1024; ++j) {
        const int r = j * RPI + lane / ROW_CHUNKS, chunk = lane % ROW_CHUNKS;
        const u32x4_t v = *reinterpret_cast<const u32x4_t*>(smem + owned_slot(stage * XMIN + j, wave) +
                                                            (r % RPI) * ROWB + ((chunk ^ (r % ROW_CHUNKS)) << 4));
        const int rl = wave_m * WTM + rd * CH_ROWS + r;
        const int gn = n0 + wave_n * WTN + chunk * 8;
        const uint32_t off =
            (rl < rows && gn < pd.n) ? ((uint32_t)rl * (uint32_t)pd.scm + (uint32_t)gn) * 2u : kOutOfRange;
        __builtin_amdgcn_raw_buffer_store_b128(v, rc, (int)off, 0, kAux);
      }
      compiler_fence();
    }
  }

  // run_tile's schedule with deep cross-tile chaining (CHAIN_DEEP tiles, static schedule).  The K
  // loop is run_tile's.  In buffer terms, slice kt of a tile lives in buffer (kt + rot) % STAGES,
  // where rot is where the previous tile left the next tile's slice 0.  Once the next tile is known
  // (at the prologue barrier), the refill that would copy slice kt + STAGES of this tile when that
  // lies past K copies the next tile's slice kt + STAGES - kt_count instead: slices 0 .. STAGES - 2
  // of the next tile, at the last STAGES - 1 slice boundaries.  The last slice has no boundary: its
  // MFMAs run, every wave reads its buffer to the end (a barrier), C leaves through the wave's slots
  // there in CHAIN_STORES counted stores, and each wave then copies the next tile's slice
  // STAGES - 1 into its own slots of that buffer.  A wave's vector memory operations complete in
  // issue order, so the next tile's wait for its slice j counts the younger slices plus, for
  // j <= STAGES - 2, the stores issued after them: it never waits for the stores themselves before
  // slice STAGES - 1 is needed.  Tiles of fewer than STAGES slices, the workgroup's last tile, and C
  // that is not 16-byte aligned (staged tiles) use run_tile's zero slices and unchained epilogue.
  template <class Sched>
  __device__ static __forceinline__ bool run_tile_chained_deep(const ProblemDesc& pd, int tm, int tn, char* smem,
                                                               Chain& ch, Sched& sched, ProblemDesc& next, int& ntm,
                                                               int& ntn) {
    static_assert(CHAIN_DEEP && (STAGES & (STAGES - 1)) == 0, "buffer rotation needs a power-of-two ring");
    static_assert(KK % 2 == 0, "fragment double buffer alternates by K step");
    constexpr int S = STAGES;
    constexpr int HALF = FM / 2 > 0 ? FM / 2 : 1;
    constexpr int NDS = FM + 2 * FN;
    constexpr int NVM = QA + QB;
    const int wave = threadIdx.x >> 6;
    const int wave_m = wave / WN, wave_n = wave % WN;
    const int m0 = tm * BM, n0 = tn * BN;

    acc_t acc[FM][FN];
#pragma unroll
    for (int fm = 0; fm < FM; ++fm)
#pragma unroll
      for (int fn = 0; fn < FN; ++fn)
#pragma unroll
        for (int i = 0; i < ACC; ++i) acc[fm][fn][i] = 0.0f;

    Dma d;
    setup_dma(d, pd, m0, n0, smem);
    const bool pre = ch.prefetched;
    const int rot = uniform(pre ? ch.rot : 0);  // buffer indices are wave-uniform (LDS-DMA's M0)
    if (pre) {
      // In flight: slices 0 .. S-2, the previous tile's CHAIN_STORES stores, slice S-1.
      wait_vmcnt<(S - 1) * XMIN + CHAIN_STORES>();
    } else {
#pragma unroll
      for (int st = 0; st < S; ++st) issue_stage(d, st, st * BK);
      wait_vmcnt<(S - 1) * XMIN>();
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    compiler_fence();
    __builtin_amdgcn_s_barrier();
    compiler_fence();
    sched.started();
    sched.before_barrier();
    const bool has_next = sched.next(next, ntm, ntn);
    const int kt_count = (pd.k + BK - 1) / BK;
    const bool c16 = ((reinterpret_cast<uintptr_t>(pd.c) & 15) == 0) && (pd.scm & 7) == 0;
    const bool chain = has_next && kt_count >= S && (!STAGED_OK || c16);
    i16x8_t af[2][FM], bf[2][FN];
    load_frags(af[0], bf[0], smem + rot * STAGE_BYTES, smem + rot * STAGE_BYTES + A_BYTES, 0, wave_m, wave_n, false);

    for (int kt = 0; kt < kt_count; ++kt) {
      const int b = uniform((kt + rot) & (S - 1));
      const char* cur = smem + b * STAGE_BYTES;
      const char* nxt = smem + ((b + 1) & (S - 1)) * STAGE_BYTES;
#pragma unroll
      for (int kk = 0; kk < KK - 1; ++kk) {
        load_frags(af[(kk + 1) & 1], bf[(kk + 1) & 1], cur, cur + A_BYTES, kk + 1, wave_m, wave_n, false);
        mfma_rows<0, FM>(acc, af[kk & 1], bf[kk & 1]);
        interleave<FM * FN, NDS, 0>();
      }
      constexpr int L = (KK - 1) & 1;
      if (!chain || kt + 1 < kt_count) {
        mfma_rows<0, HALF>(acc, af[L], bf[L]);
        // Slice kt + 1 complete: younger are slices kt + 2 .. kt + S - 1, plus the previous tile's
        // stores while slice kt + 1 is one of the first S - 1 prefetched slices.
        if (pre && kt + 1 <= S - 2)
          wait_vmcnt<(S - 2) * XMIN + CHAIN_STORES>();
        else
          wait_vmcnt<(S - 2) * XMIN>();
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        compiler_fence();
        __builtin_amdgcn_s_barrier();
        compiler_fence();
        const int st = kt + S;
        if (chain && st >= kt_count) {
          Dma dn;  // the next tile's copy state, recomputed for each of its prefetched slices
          setup_dma(dn, next, ntm * BM, ntn * BN, smem);
          issue_stage(dn, b, (st - kt_count) * BK);
        } else {
          issue_stage(d, b, st * BK);
        }
        load_frags(af[0], bf[0], nxt, nxt + A_BYTES, 0, wave_m, wave_n, false);
        mfma_rows<HALF, FM>(acc, af[L], bf[L]);
        interleave<(FM - HALF) * FN, NDS, NVM>();
      } else {
        mfma_rows<0, FM>(acc, af[L], bf[L]);  // the last slice of a chained tile
      }
    }
    if (chain) {
      const int last = uniform((kt_count - 1 + rot) & (S - 1));
      // Every wave has read the last slice's buffer before any stages C in its slots there.
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      compiler_fence();
      __builtin_amdgcn_s_barrier();
      compiler_fence();
      if constexpr (STAGED_OK)
        staged_store_counted(acc, pd, m0, n0, wave_m, wave_n, smem, last);
      else
        store_tile_counted(acc, pd, m0, n0, wave_m, wave_n);
      {
        Dma dn;
        setup_dma(dn, next, ntm * BM, ntn * BN, smem);
        issue_stage(dn, last, (S - 1) * BK);
      }
      ch.rot = (kt_count + rot) & (S - 1);
      ch.prefetched = true;
    } else {
      // Copies of this tile (zero slices past K) landed and every wave is done with LDS before
      // the next tile's own prologue refills it.
      wait_vmcnt<0>();
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      compiler_fence();
      __builtin_amdgcn_s_barrier();
      compiler_fence();
      store_tile(acc, pd, m0, n0, wave_m, wave_n, smem);
      ch.prefetched = false;
    }
    return has_next;
  }

  // run_tile's schedule for CHAIN_OK tiles.  `ch` carries the prefetch from one call to the next;
  // start a workgroup with ch.prefetched false.  The workgroup's next tile comes from `sched`, whose
  // hooks every wave runs once per tile, in this order:
  //   sched.started()               after the tile's slice-1 copies are issued.  The wave's next
  //                                 vector-memory wait is vmcnt(0), so one more vector memory
  //                                 operation issued here never breaks a counted wait;
  //   sched.before_barrier()        after that vmcnt(0) wait, before the barrier of the first slice
  //                                 boundary (of the epilogue for a one-slice tile); LDS writes
  //                                 made here are visible after the barrier;
  //   sched.next(next, ntm, ntn)    after that barrier: true and the next tile's description, or
  //                                 false when this is the workgroup's last tile.  The next tile is
  //                                 needed no earlier: its slice 0 is issued at the boundary before
  //                                 this tile's last slice.
  // Returns whether there is a next tile (then `next`, `ntm`, `ntn` describe it).
  template <class Sched>
  __device__ static __forceinline__ bool run_tile_chained(const ProblemDesc& pd, int tm, int tn, char* smem, Chain& ch,
                                                          Sched& sched, ProblemDesc& next, int& ntm, int& ntn) {
    if constexpr (CHAIN_DEEP) return run_tile_chained_deep(pd, tm, tn, smem, ch, sched, next, ntm, ntn);
    static_assert(CHAIN_OK, "the chained schedule is for two-stage and four-stage tiles");
    static_assert(KK % 2 == 0, "fragment double buffer alternates by K step");
    constexpr int HALF = FM / 2 > 0 ? FM / 2 : 1;
    constexpr int NDS = FM + 2 * FN;
    constexpr int NVM = QA + QB;
    const int wave = threadIdx.x >> 6;
    const int wave_m = wave / WN, wave_n = wave % WN;
    const int m0 = tm * BM, n0 = tn * BN;

    acc_t acc[FM][FN];
#pragma unroll
    for (int fm = 0; fm < FM; ++fm)
#pragma unroll
      for (int fn = 0; fn < FN; ++fn)
#pragma unroll
        for (int i = 0; i < ACC; ++i) acc[fm][fn][i] = 0.0f;

    Dma d;
    int rot = 0;
    if (ch.prefetched) {
      // Slice 0 was issued before the previous tile's CHAIN_STORES stores, with nothing else of
      // this wave outstanding; the previous tile's LDS reads are done once every wave is here.
      // The copy state is recomputed rather than carried (fewer registers live across the
      // previous tile's epilogue).
      setup_dma(d, pd, m0, n0, smem);
      rot = ch.rot;
      wait_vmcnt<CHAIN_STORES>();
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      compiler_fence();
      __builtin_amdgcn_s_barrier();
      compiler_fence();
      issue_stage(d, rot ^ 1, BK);  // slice 1, into the buffer of the previous tile's last slice
    } else {
      setup_dma(d, pd, m0, n0, smem);
      issue_stage(d, 0, 0);
      issue_stage(d, 1, BK);
      wait_vmcnt<XMIN>();
      compiler_fence();
      __builtin_amdgcn_s_barrier();
      compiler_fence();
    }
    sched.started();
    bool has_next = false;
    i16x8_t af[2][FM], bf[2][FN];
    load_frags(af[0], bf[0], smem + rot * STAGE_BYTES, smem + rot * STAGE_BYTES + A_BYTES, 0, wave_m, wave_n,
               false);

    const int kt_count = (pd.k + BK - 1) / BK;
    const bool c16 = ((reinterpret_cast<uintptr_t>(pd.c) & 15) == 0) && (pd.scm & 7) == 0;
    bool chain = false;  // set at the first slice boundary, once the next tile is known
    for (int kt = 0; kt < kt_count; ++kt) {
      const int b = (kt + rot) & 1;
      const char* cur = smem + b * STAGE_BYTES;
      const char* nxt = smem + (b ^ 1) * STAGE_BYTES;
#pragma unroll
      for (int kk = 0; kk < KK - 1; ++kk) {
        load_frags(af[(kk + 1) & 1], bf[(kk + 1) & 1], cur, cur + A_BYTES, kk + 1, wave_m, wave_n, false);
        mfma_rows<0, FM>(acc, af[kk & 1], bf[kk & 1]);
        interleave<FM * FN, NDS, 0>();
      }
      constexpr int L = (KK - 1) & 1;
      if (kt + 1 < kt_count) {
        // As run_tile: slice kt+1 becomes readable, and the drained buffer of slice kt is refilled
        // with slice kt+2, or with the next tile's slice 0 when slice kt+2 would lie past K.
        mfma_rows<0, HALF>(acc, af[L], bf[L]);
        wait_vmcnt<0>();
        if (kt == 0) sched.before_barrier();
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        compiler_fence();
        __builtin_amdgcn_s_barrier();
        compiler_fence();
        if (kt == 0) {
          has_next = sched.next(next, ntm, ntn);
          chain = has_next && (!STAGED_OK || c16);
        }
        if (chain && kt + 2 == kt_count) {
          Dma dn;  // the next tile's copy state, only for its slice 0
          setup_dma(dn, next, ntm * BM, ntn * BN, smem);
          issue_stage(dn, b, 0);
        } else {
          issue_stage(d, b, (kt + 2) * BK);
        }
        load_frags(af[0], bf[0], nxt, nxt + A_BYTES, 0, wave_m, wave_n, false);
        mfma_rows<HALF, FM>(acc, af[L], bf[L]);
        interleave<(FM - HALF) * FN, NDS, NVM>();
      } else {
        mfma_rows<0, FM>(acc, af[L], bf[L]);  // the last slice: nothing left to fetch for this tile
      }
    }
    if (chain) {
      if constexpr (STAGED_OK) {
        // Every wave has read the last slice's buffer before any stages C in its slots there.
        const int last = (kt_count - 1 + rot) & 1;
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        compiler_fence();
        __builtin_amdgcn_s_barrier();
        compiler_fence();
        staged_store_counted(acc, pd, m0, n0, wave_m, wave_n, smem, last);
      } else {
        store_tile_counted(acc, pd, m0, n0, wave_m, wave_n);
      }
      ch.rot = (kt_count + rot) & 1;
      ch.prefetched = true;
    } else {
      // Copies of this tile (zero slices past K) landed and every wave is done with LDS before
      // the next tile's own prologue refills it.  Chained launches have no split-K and no SwiGLU,
      // so only the plain C epilogue is needed.
      wait_vmcnt<0>();
      if (kt_count <= 1) sched.before_barrier();
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      compiler_fence();
      __builtin_amdgcn_s_barrier();
      compiler_fence();
      if (kt_count <= 1) has_next = sched.next(next, ntm, ntn);
      if constexpr (STAGED_OK) {
        staged_store(acc, pd, m0, n0, wave_m, wave_n, smem);
      } else {
        const int lane = threadIdx.x & 63;
#pragma unroll
        for (int fm = 0; fm < FM; ++fm) {
          const int gm = m0 + wave_m * WTM + fm * MI + (lane % MI);
          if (gm >= pd.m) continue;
          char* crow = pd.c + (int64_t)gm * pd.scm * 2;
#pragma unroll
          for (int fn = 0; fn < FN; ++fn)
#pragma unroll
            for (int q = 0; q < ACC / 4; ++q) {
              const int nloc = (MI == 32) ? (q * 8 + (lane >> 5) * 4) : ((lane >> 4) * 4);
              const int gn = n0 + wave_n * WTN + fn * MI + nloc;
              if (gn < pd.n)
                store4<E>(crow + (int64_t)gn * 2, f32x4_t{acc[fm][fn][q * 4 + 0], acc[fm][fn][q * 4 + 1],
                                                          acc[fm][fn][q * 4 + 2], acc[fm][fn][q * 4 + 3]});
            }
        }
      }
      ch.prefetched = false;
    }
    return has_next;
  }
};

}  // namespace moegemm
