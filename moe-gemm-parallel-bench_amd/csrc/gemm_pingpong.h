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

  template <int EPI, class Hook>
  __device__ static __forceinline__ void run_tile(const ProblemDesc& pd, int tm, int tn, char* smem, bool tf32,
                                                  Hook&& before_store) {
    // Each group runs a copy of the schedule compiled for it and for the launch's B copy policy
    // (no group or policy tests inside the K loop).
    const bool second = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)) >= NW / 2;
    if (pd.b_stream) {
      if (second) group_tile<EPI, true, 1>(pd, tm, tn, smem, before_store);
      else group_tile<EPI, false, 1>(pd, tm, tn, smem, before_store);
    } else {
      if (second) group_tile<EPI, true, 0>(pd, tm, tn, smem, before_store);
      else group_tile<EPI, false, 0>(pd, tm, tn, smem, before_store);
    }
  }

  template <int EPI, bool SECOND, int NTB, class Hook>
  __device__ static __forceinline__ void group_tile(const ProblemDesc& pd, int tm, int tn, char* smem,
                                                    Hook&& before_store) {
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int wave_m = wave / WN, wave_n = wave % WN;
    constexpr bool second = SECOND;
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
    for (int s = 0; s < STAGES; ++s) Base::template issue_stage<NTB>(d, s, s * BK);
    wait_vmcnt<(STAGES - 1) * XMIN>();
    phase_barrier();
    if constexpr (second) phase_barrier();  // group 1 runs one barrier behind

    i16x8_t af[KK][FM], bf[KK][FN];
    const int kt_count = (pd.k + BK - 1) / BK;
    for (int kt = 0; kt < kt_count; ++kt) {
      // Memory phase.
      const char* cur = smem + (kt % STAGES) * STAGE_BYTES;
      if (kt >= 1) Base::template issue_stage<NTB>(d, (kt - 1) % STAGES, (kt - 1 + STAGES) * BK);
#pragma unroll
      for (int kk = 0; kk < KK; ++kk)
        Base::load_frags(af[kk], bf[kk], cur, cur + A_BYTES, kk, wave_m, wave_n, pd.swiglu != 0);
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      if constexpr (second) wait_vmcnt<(STAGES - 2) * XMIN>();
      phase_barrier();
      // Compute phase.
#pragma unroll
      for (int kk = 0; kk < KK; ++kk) Base::template mfma_rows<0, FM>(acc, af[kk], bf[kk]);
      if constexpr (!second) wait_vmcnt<(STAGES - 2) * XMIN>();
      phase_barrier();
    }
    // This wave's remaining copies (zero-filled slices past K) land before the epilogue, which may
    // stage C in the wave's own LDS slots; then the hook, as in FastTile.
    wait_vmcnt<0>();
    before_store();
    if constexpr (EPI != EPI_C) {
      if (EPI == EPI_SPLIT || pd.splits > 1) {
        // The split epilogue has workgroup barriers of its own: align the groups first.
        if constexpr (!second) phase_barrier();
        Base::template store_tile<EPI_SPLIT>(acc, pd, m0, n0, wave_m, wave_n, smem);
        return;
      }
    }
    // Unsplit tiles, also the whole tiles of a stream-K tail.
    Base::store_tile(acc, pd, m0, n0, wave_m, wave_n, smem);
    if constexpr (!second) phase_barrier();
  }

  // Cross-tile chaining on the static schedule of single and homogeneous launches, and of offsets
  // launches whose groups fit one LDS prefix chunk (ragged groups, partial M tiles).  A tile's last
  // three memory phases would refill their buffers with zero slices past K; instead they copy the
  // next tile's slices 0..2 (each wave into its own slots, as always).  C then leaves through the
  // wave's slots of the last slice's buffer, in CHAIN_STORES counted stores
  // (FastTile::staged_store_counted): group 1 read that slice in its memory phase before the
  // barrier that ends group 0's last compute phase, so both groups may stage there.  After its
  // stores each wave copies the next tile's slice 3 into the same slots (its staging reads have
  // returned: the stores consumed them).  A wave's vector memory operations complete in issue
  // order, so the next tile waits for slice 0 with 3 * XMIN + CHAIN_STORES younger operations
  // outstanding, and for slices 1 and 2 with the stores still counted; only slice 3's wait
  // (end of the memory or compute phase of K step 2) needs the stores done.  The next tile's buffers
  // rotate by K slices.  Tiles of fewer than STAGES slices, the last tile, and C that is not
  // 16-byte aligned run the unchained epilogue (zero slices, wait for every copy).  The next unit
  // is known right after the prologue barrier: the static schedule computes it, and under work
  // stealing wave 0 claims it just before that barrier (see chained_group).
  static constexpr bool CHAIN_OK = Base::STAGED_OK && (STAGES & (STAGES - 1)) == 0;
  static constexpr int CHAIN_MIN_SLICES = 1;
  static constexpr int CHAIN_MAX_SLICES = 1 << 30;
  static constexpr bool CHAIN_STEALING = true;
  static constexpr int CHAIN_STORES = Base::CHAIN_STORES;
  static_assert(!CHAIN_OK || 3 * XMIN + CHAIN_STORES < 64, "outstanding operations must fit the 6-bit vmcnt");
  static_assert(!CHAIN_OK || (Base::CH_ROWS > 0 && Base::WTM % Base::CH_ROWS == 0 &&
                              (Base::CH_ROWS * Base::ROWB) % 1024 == 0),
                "staging rounds must cover the wave tile in whole slots of one stage");
  using Chain = typename Base::Chain;

  template <class Sched>
  __device__ static __forceinline__ bool run_tile_chained(const ProblemDesc& pd, int tm, int tn, char* smem, Chain& ch,
                                                          Sched& sched, ProblemDesc& next, int& ntm, int& ntn) {
    static_assert(CHAIN_OK, "the chained epilogue stages C in one stage's slots");
    // Each group runs a copy of the tile's schedule compiled for it, so the group tests of the K
    // steps (which wait comes where, the extra barriers) cost no branches.
    // The B copy policy is uniform over a launch, so the next tile's prefetched slices take this
    // tile's.
    const bool second = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)) >= NW / 2;
    if (pd.b_stream) {
      if (second) return chained_group<true, 1>(pd, tm, tn, smem, ch, sched, next, ntm, ntn);
      return chained_group<false, 1>(pd, tm, tn, smem, ch, sched, next, ntm, ntn);
    }
    if (second) return chained_group<true, 0>(pd, tm, tn, smem, ch, sched, next, ntm, ntn);
    return chained_group<false, 0>(pd, tm, tn, smem, ch, sched, next, ntm, ntn);
  }

  template <bool SECOND, int NTB, class Sched>
  __device__ static __forceinline__ bool chained_group(const ProblemDesc& pd, int tm, int tn, char* smem, Chain& ch,
                                                       Sched& sched, ProblemDesc& next, int& ntm, int& ntn) {
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int wave_m = wave / WN, wave_n = wave % WN;
    constexpr bool second = SECOND;
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

    const bool pre = ch.prefetched;
    const int rot = pre ? ch.rot : 0;
    // Under work stealing, wave 0 claims the workgroup's next unit here and the first barrier
    // publishes it.  Reading the claim waits for every vector memory operation of wave 0
    // (vmcnt(0)): at this point that is the tile's own first slices and the previous tile's C
    // stores, which the first K steps wait for anyway, or on a workgroup's first tile nothing.
    if (pre) {
      // Issued by the previous tile: slices 0, 1, 2, then its CHAIN_STORES stores, then slice 3.
      wait_vmcnt<3 * XMIN + CHAIN_STORES>();
      sched.started();
      sched.before_barrier();
    } else {
      sched.started();
      sched.before_barrier();
#pragma unroll
      for (int s = 0; s < STAGES; ++s) Base::template issue_stage<NTB>(d, s, s * BK);
      wait_vmcnt<(STAGES - 1) * XMIN>();
    }
    phase_barrier();
    if constexpr (second) phase_barrier();  // group 1 runs one barrier behind
    const bool has_next = sched.next(next, ntm, ntn);
    const int kt_count = (pd.k + BK - 1) / BK;
    const bool c16 = ((reinterpret_cast<uintptr_t>(pd.c) & 15) == 0) && (pd.scm & 7) == 0;
    const bool chain = has_next && kt_count >= STAGES && c16;

    // One K step.  ISSUE: 0 none (kt = 0), 1 this tile's slice kt + STAGES - 1 (zeros past K),
    // 2 chosen at run time (the next tile's slices once that index passes K).  GENERIC: the wait for
    // slice kt + 1 depends on kt (stores of the previous tile still counted, no successor).  The
    // steady-state steps (ISSUE 1, fixed wait) carry no branches.
    i16x8_t af[KK][FM], bf[KK][FN];
    auto step = [&](int kt, auto issue_kind, auto generic) {
      constexpr int ISSUE = decltype(issue_kind)::value;
      constexpr bool GENERIC = decltype(generic)::value;
      // Memory phase.
      const char* cur = smem + ((kt + rot) & (STAGES - 1)) * STAGE_BYTES;
      const int buf = (kt - 1 + rot) & (STAGES - 1), s = kt - 1 + STAGES;
      if constexpr (ISSUE == 1) {
        Base::template issue_stage<NTB>(d, buf, s * BK);
      } else if constexpr (ISSUE == 2) {
        if (chain && s >= kt_count) {
          Dma dn;  // the next tile's copy state, recomputed for each of its first slices
          Base::setup_dma(dn, next, ntm * BM, ntn * BN, smem);
          Base::template issue_stage<NTB>(dn, buf, (s - kt_count) * BK);
        } else {
          Base::template issue_stage<NTB>(d, buf, s * BK);
        }
      }
#pragma unroll
      for (int kk = 0; kk < KK; ++kk)
        Base::load_frags(af[kk], bf[kk], cur, cur + A_BYTES, kk, wave_m, wave_n, false);
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      // Slice kt + 1 complete (the chained last slice has no successor in this tile).
      auto wait_next = [&] {
        if constexpr (GENERIC) {
          if (!chain || kt + 1 < kt_count) {
            if (pre && kt < 2) wait_vmcnt<(STAGES - 2) * XMIN + CHAIN_STORES>();
            else wait_vmcnt<(STAGES - 2) * XMIN>();
          }
        } else {
          wait_vmcnt<(STAGES - 2) * XMIN>();
        }
      };
      if constexpr (second) wait_next();
      phase_barrier();
      // Compute phase.
#pragma unroll
      for (int kk = 0; kk < KK; ++kk) Base::template mfma_rows<0, FM>(acc, af[kk], bf[kk]);
      if constexpr (!second) wait_next();
      phase_barrier();
    };
    using no_issue = std::integral_constant<int, 0>;
    using own_issue = std::integral_constant<int, 1>;
    using any_issue = std::integral_constant<int, 2>;
    step(0, no_issue{}, std::true_type{});
    int kt = 1;
    for (; kt < 2 && kt < kt_count; ++kt) step(kt, any_issue{}, std::true_type{});
    for (; kt + STAGES - 1 < kt_count; ++kt) step(kt, own_issue{}, std::false_type{});
    for (; kt < kt_count; ++kt) step(kt, any_issue{}, std::true_type{});
    if (chain) {
      const int last = (kt_count - 1 + rot) & (STAGES - 1);
      Base::staged_store_counted(acc, pd, m0, n0, wave_m, wave_n, smem, last);
      {
        Dma dn;
        Base::setup_dma(dn, next, ntm * BM, ntn * BN, smem);
        Base::template issue_stage<NTB>(dn, last, (STAGES - 1) * BK);
      }
      if constexpr (!second) phase_barrier();
      ch.rot = (kt_count + rot) & (STAGES - 1);
      ch.prefetched = true;
    } else {
      wait_vmcnt<0>();
      Base::store_tile(acc, pd, m0, n0, wave_m, wave_n, smem);
      if constexpr (!second) phase_barrier();
      ch.prefetched = false;
    }
    return has_next;
  }
};

}  // namespace moegemm
