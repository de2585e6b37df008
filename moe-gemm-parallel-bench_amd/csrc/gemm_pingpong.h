// Ping-pong schedule of the LDS-DMA grouped GEMM tile for large, MFMA-bound problems (gfx950).
//
// Same tile semantics, LDS layout, DMA copies, fragment reads and epilogue as FastTile
// (gemm_fast.h); only the order of work inside a tile differs.  The 8 waves of a workgroup form
// two groups, waves 0..3 (group 0) and 4..7 (group 1); the hardware places wave w and wave w + 4
// on the same SIMD, so every SIMD holds one wave of each group.  Group 1 runs one workgroup
// barrier behind group 0, and each wave alternates two phases per K slice:
//   memory phase : issue its share of the LDS-DMA copies for a later slice, read every MFMA
//                  fragment of the current slice from LDS into registers, wait for the reads;
//   compute phase: the slice's MFMAs, from registers only.
// Between consecutive barriers one group computes while the other loads, so each SIMD's MFMA
// pipe is fed by its two waves in turn and never waits on LDS latency or on a barrier with work
// left in the other wave.  Per slice k (buffer k % S), with barrier j numbered from the prologue:
//   group 0: memory(k) between barriers 2k and 2k+1, compute(k) between 2k+1 and 2k+2;
//   group 1: memory(k) between barriers 2k+1 and 2k+2, compute(k) between 2k+2 and 2k+3.
// Slice k is last read in group 1's memory(k), so its buffer is refilled (with slice k + S) from
// memory(k + 1) on, by both groups.  Slice k + 1 must be complete at barrier 2k + 2: group 0 waits
// for its own copies at the end of compute(k), group 1 at the end of memory(k) (each wave has
// S - 2 younger slices of copies in flight at that point), and the barrier publishes them.
// Group 0 executes one extra barrier after its last compute phase (storing its outputs first,
// except for split-K units, whose epilogue synchronises the workgroup and so runs after it) so
// both groups pass the same number of barriers per tile.  Copies of slices past K read
// zeros into buffers nobody reads; every LDS slot is always written by the same wave, which waits
// for its own copies before its epilogue (the staged C store reuses its slots).  When group 0
// stages C after barrier 2K, group 1 has finished its last fragment reads (before that barrier),
// and each wave touches only its own slots.
#pragma once

#include "gemm_fast.h"

namespace moegemm {

// Workgroup barrier that neither the compiler nor the machine scheduler moves work across.
__device__ __forceinline__ void phase_barrier() {
  __builtin_amdgcn_sched_barrier(0);
  compiler_fence();
  __builtin_amdgcn_s_barrier();
  compiler_fence();
  __builtin_amdgcn_sched_barrier(0);
}

template <class E, int BK_, int STAGES_>
struct PingPongTile : FastTile<E, 256, 256, BK_, 2, 4, STAGES_> {
  using Base = FastTile<E, 256, 256, BK_, 2, 4, STAGES_>;
  using typename Base::acc_t;
  using typename Base::Dma;
  static constexpr int BM = Base::BM, BN = Base::BN, BK = Base::BK, STAGES = Base::STAGES;
  static constexpr int NW = Base::NW, WN = Base::WN, FM = Base::FM, FN = Base::FN, KK = Base::KK;
  static constexpr int ACC = Base::ACC, A_BYTES = Base::A_BYTES, STAGE_BYTES = Base::STAGE_BYTES;
  static constexpr int XMIN = Base::XMIN;
  static_assert(NW == 8, "two groups of four waves, one wave of each per SIMD");
  static_assert(Base::IA % NW == 0 && Base::IB % NW == 0, "every wave issues the same number of copies");
  static_assert(STAGES >= 3, "group 1 needs at least one phase between issuing and publishing a slice");

  template <class Hook>
  __device__ static __forceinline__ void run_tile(const ProblemDesc& pd, int tm, int tn, char* smem, bool,
                                                  Hook&& before_store) {
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int wave_m = wave / WN, wave_n = wave % WN;
    const bool second = wave >= NW / 2;
    const int m0 = tm * BM, n0 = tn * BN;
    Dma d;
    Base::setup_dma(d, pd, m0, n0, smem);

    acc_t acc[FM][FN];
#pragma unroll
    for (int fm = 0; fm < FM; ++fm)
#pragma unroll
      for (int fn = 0; fn < FN; ++fn)
#pragma unroll
        for (int i = 0; i < ACC; ++i) acc[fm][fn][i] = 0.0f;

    // Prologue: slices 0..S-1 in flight; slice 0 published by barrier 0.
#pragma unroll
    for (int s = 0; s < STAGES; ++s) Base::issue_stage(d, s, s * BK);
    wait_vmcnt<(STAGES - 1) * XMIN>();
    phase_barrier();
    if (second) phase_barrier();  // group 1 runs one barrier behind

    i16x8_t af[KK][FM], bf[KK][FN];
    const int kt_count = (pd.k + BK - 1) / BK;
    for (int kt = 0; kt < kt_count; ++kt) {
      // Memory phase.
      const char* cur = smem + (kt % STAGES) * STAGE_BYTES;
      if (kt >= 1) Base::issue_stage(d, (kt - 1) % STAGES, (kt - 1 + STAGES) * BK);
#pragma unroll
      for (int kk = 0; kk < KK; ++kk)
        Base::load_frags(af[kk], bf[kk], cur, cur + A_BYTES, kk, wave_m, wave_n, pd.swiglu != 0);
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      if (second) wait_vmcnt<(STAGES - 2) * XMIN>();
      phase_barrier();
      // Compute phase.
#pragma unroll
      for (int kk = 0; kk < KK; ++kk) Base::template mfma_rows<0, FM>(acc, af[kk], bf[kk]);
      if (!second) wait_vmcnt<(STAGES - 2) * XMIN>();
      phase_barrier();
    }
    // This wave's remaining copies (zero-filled slices past K) land before the epilogue, which may
    // stage C in the wave's own LDS slots; then the hook, as in FastTile.
    wait_vmcnt<0>();
    before_store();
    if (pd.splits > 1) {
      // The split epilogue has workgroup barriers of its own: align the groups first.
      if (!second) phase_barrier();
      Base::store_tile(acc, pd, m0, n0, wave_m, wave_n, smem);
    } else if (!second) {
      Base::store_tile(acc, pd, m0, n0, wave_m, wave_n, smem);
      phase_barrier();
    } else {
      Base::store_tile(acc, pd, m0, n0, wave_m, wave_n, smem);
    }
  }
};

}  // namespace moegemm
