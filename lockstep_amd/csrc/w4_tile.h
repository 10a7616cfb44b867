// Four-wave int8 MFMA main loop for gfx950 (dense contract GEMMs).
//
// A block of 256 threads computes a BM x BN tile of C = A * W^T over all of K with one wave per
// SIMD; each wave owns a (BM/2) x (BN/2) sub-tile (TM x TN v_mfma_i32_32x32x32_i8 tiles whose
// accumulators fill the accumulation registers).  Against the eight-wave ping-pong (pp_tile.h),
// a wave's sub-tile is twice as large, so each fragment read from LDS feeds more MFMAs: a 256x256
// tile reads 512 bytes of LDS per MFMA instead of 768.
//
// K is staged 64 bytes at a time through a ring of RING LDS stages filled by direct global ->
// LDS loads (buffer_load_dwordx4 ... lds), issued RING - 1 stages ahead of the stage being
// multiplied (in the second half of a stage, so they interleave with its MFMAs), with the chunk
// swizzle of pp_tile.h.  Within a wave the fragments of the next 32-byte K-step are read from LDS while the
// MFMAs of the current one run (two fragment register sets).  One barrier per stage, placed
// where the wave moves on to the next stage's fragments: after it, every wave's loads of that
// stage have landed and every wave has finished reading the stage before, whose slot the next
// stage's loads then refill.  Integer accumulation is exact in any order, so nothing here
// changes a bit of the result.
#pragma once
#include <type_traits>

#include "pp_tile.h"

namespace lsk {

template <int BM, int BN, int RING = 4>
struct W4Cfg {
  static_assert(RING >= 3 && RING <= 5, "ring of 3..5 stages");
  static constexpr int kThreads = 256;
  static constexpr int kBM = BM, kBN = BN, kWM = 2, kWN = 2;
  static constexpr int kBK = 64, kChunks = 4, kKS = 2;
  static constexpr int kRing = RING, kAhead = RING - 1;
  static constexpr int WTM = BM / 2, WTN = BN / 2;
  static constexpr int TM = WTM / 32, TN = WTN / 32;
  static constexpr int kStageA = BM * kBK, kStageB = BN * kBK, kStage = kStageA + kStageB;
  static constexpr int kLA = kStageA / 16 / kThreads, kLB = kStageB / 16 / kThreads;
  static constexpr int kMainBytes = kRing * kStage;
  static constexpr int kLdc = WTN + 4;
  static constexpr int kStripBytes = 32 * kLdc * 4;
  static constexpr int kEpiBytes = 4 * kStripBytes;
  static constexpr int kScaleOff = kMainBytes > kEpiBytes ? kMainBytes : kEpiBytes;
  static constexpr int kFlagOff = kScaleOff + (BM + 3 * BN) * 4;
  static constexpr int kSmemBytes = kFlagOff + 8 * 4;
  static_assert(BM <= kThreads && BN <= kThreads, "one epilogue operand per thread");
  static_assert(kStageA % (16 * kThreads) == 0 && kStageB % (16 * kThreads) == 0, "tile / threads");
  static_assert(WTM % 32 == 0 && WTN % 32 == 0, "wave tile must be a multiple of 32");
  static_assert(kSmemBytes <= 160 * 1024, "LDS");
  typedef v16i Acc[TM][TN];
  typedef uint32_t RowsA[kLA];
  typedef uint32_t RowsB[kLB];
};

// N times: one MFMA, then one instruction of class MASK (0x100 LDS read, 0x020 global load), in
// the scheduling region that ends here.
template <int N, int MASK, int ID>
LSK_DEV void sched_pairs() {
#pragma unroll
  for (int t = 0; t < N; ++t) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, ID);
    __builtin_amdgcn_sched_group_barrier(MASK, 1, ID);
  }
}

template <class C>
LSK_DEV void w4_mainloop(typename C::Acc& acc, __amdgpu_buffer_rsrc_t ra, const typename C::RowsA& pa,
                         __amdgpu_buffer_rsrc_t rb, const typename C::RowsB& pb, int K, char* smem) {
  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
  const int wm = wave / C::kWN, wn = wave % C::kWN;
  const int nk = (K + C::kBK - 1) / C::kBK;

  int ka[C::kLA], kb[C::kLB];
#pragma unroll
  for (int j = 0; j < C::kLA; ++j) {
    int r;
    pp_slot<C::kThreads, C::kChunks>(tid, j, r, ka[j]);
  }
#pragma unroll
  for (int j = 0; j < C::kLB; ++j) {
    int r;
    pp_slot<C::kThreads, C::kChunks>(tid, j, r, kb[j]);
  }
  // this thread's direct-to-LDS loads of stage s (CHECK: the stage may reach past K)
  auto issue = [&](int s, auto check) {
    constexpr bool kCheck = decltype(check)::value;
    char* st = smem + (s % C::kRing) * C::kStage;
    const int k0 = s * C::kBK;
#pragma unroll
    for (int j = 0; j < C::kLA; ++j) {
      const int kk = k0 + ka[j];
      const uint32_t off = (!kCheck || kk < K) ? pa[j] + (uint32_t)kk : kOob;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (lds_void_t)(st + (j * C::kThreads + wave * 64) * 16), 16, off, 0,
                                               0, 0);
    }
#pragma unroll
    for (int j = 0; j < C::kLB; ++j) {
      const int kk = k0 + kb[j];
      const uint32_t off = (!kCheck || kk < K) ? pb[j] + (uint32_t)kk : kOob;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rb, (lds_void_t)(st + C::kStageA + (j * C::kThreads + wave * 64) * 16), 16, off, 0, 0, 0);
    }
  };
  constexpr int kPer = C::kLA + C::kLB;

  // fragment addresses: row base + (lane & 31), logical chunk 2 ks + (lane >> 5)
  const int lr = lane & 31, sw = pp_swz<C::kChunks>(lr), kg = lane >> 5;
  const int offA = (wm * C::WTM + lr) * C::kBK, offB = C::kStageA + (wn * C::WTN + lr) * C::kBK;
  const int slot0 = 16 * ((0 + kg) ^ sw), slot1 = 16 * ((2 + kg) ^ sw);

  v4i fa0[C::TM], fb0[C::TN], fa1[C::TM], fb1[C::TN];
  auto read = [&](int s, int slot, v4i (&fa)[C::TM], v4i (&fb)[C::TN]) {
    const char* st = smem + (s % C::kRing) * C::kStage;
#pragma unroll
    for (int i = 0; i < C::TM; ++i) fa[i] = *(const v4i*)(st + offA + i * 32 * C::kBK + slot);
#pragma unroll
    for (int j = 0; j < C::TN; ++j) fb[j] = *(const v4i*)(st + offB + j * 32 * C::kBK + slot);
  };
  // MFMAs t in [T0, T1) of one K-step (t = i * TN + j)
  auto mma = [&](const v4i (&fa)[C::TM], const v4i (&fb)[C::TN], auto t0, auto t1) {
#pragma unroll
    for (int t = decltype(t0)::value; t < decltype(t1)::value; ++t)
      acc[t / C::TN][t % C::TN] = mfma_i8_32(fa[t / C::TN], fb[t % C::TN], acc[t / C::TN][t % C::TN]);
  };
  constexpr int kMF = C::TM * C::TN;  // MFMAs per K-step
  constexpr int kR = C::TM + C::TN;   // fragment reads per K-step
  constexpr int kPre = 2;             // MFMAs of K-step 1 issued before the stage barrier
  using I0 = std::integral_constant<int, 0>;
  using IPre = std::integral_constant<int, kPre>;
  using IMF = std::integral_constant<int, kMF>;

  // one stage: read K-step 1 | MFMAs of K-step 0, each followed by one read; then, when a stage
  // follows: two MFMAs of K-step 1, own loads of stage kt + 1 landed (WAIT younger loads may stay
  // outstanding), barrier, read its K-step 0, [issue stage kt + kAhead into the slot of stage
  // kt - 1, which every wave finished reading before the previous barrier] | the other MFMAs of
  // K-step 1, each followed by one read, then by one load.  The schedule is pinned: the compiler
  // would otherwise hoist the waits for the reads above most of the MFMAs they overlap.
  using Chk = std::true_type;
  using NoChk = std::false_type;
  auto stage = [&](int kt, auto wait_n, auto do_issue, auto check, auto has_next) {
    constexpr int kWait = decltype(wait_n)::value;
    constexpr bool kIssue = decltype(do_issue)::value, kNext = decltype(has_next)::value;
    static_assert(kNext || !kIssue, "a stage that issues has a successor");
    read(kt, slot1, fa1, fb1);
    mma(fa0, fb0, I0{}, IMF{});
    sched_pairs<(kR < kMF ? kR : kMF), 0x100, 0>();
    __builtin_amdgcn_sched_barrier(0);
    wait_lgkm0();
    if constexpr (kNext) {
      mma(fa1, fb1, I0{}, IPre{});
      __builtin_amdgcn_sched_barrier(0);
      wait_vm<kWait>();
      phase_barrier();
      read(kt + 1, slot0, fa0, fb0);
      if constexpr (kIssue) issue(kt + C::kAhead, check);
      mma(fa1, fb1, IPre{}, IMF{});
      constexpr int nDS = kR < kMF - kPre ? kR : kMF - kPre;
      sched_pairs<nDS, 0x100, 1>();
      if constexpr (kIssue) sched_pairs<(kPer < kMF - kPre - nDS ? kPer : kMF - kPre - nDS), 0x010, 1>();
    } else {
      mma(fa1, fb1, I0{}, IMF{});
    }
    __builtin_amdgcn_sched_barrier(0);
    wait_lgkm0();
  };
  using W0 = std::integral_constant<int, 0>;
  using Yes = std::true_type;
  using No = std::false_type;

  // prologue: stages 0 .. kAhead-1 in flight, all waited for, K-step 0 of stage 0 read
#pragma unroll
  for (int s = 0; s < C::kAhead; ++s)
    if (s < nk) issue(s, Chk{});
  wait_vm<0>();
  phase_barrier();
  read(0, slot0, fa0, fb0);
  wait_lgkm0();

  if (nk > C::kAhead) {
    // stage kt waits for stage kt + 1 with stages up to kt - 1 + kAhead issued
    using WSteady = std::integral_constant<int, (C::kAhead - 2) * kPer>;
    const int nfull = K / C::kBK;
    int kt = 0;
    for (; kt + C::kAhead < nfull; ++kt) stage(kt, WSteady{}, Yes{}, NoChk{}, Yes{});
    for (; kt + C::kAhead < nk; ++kt) stage(kt, WSteady{}, Yes{}, Chk{}, Yes{});
    // drain: the last kAhead stages issue nothing; stage kt + d leaves kAhead - 2 - d stages younger
    // than the next one outstanding
    stage(kt, std::integral_constant<int, (C::kAhead >= 2 ? C::kAhead - 2 : 0) * kPer>{}, No{}, NoChk{}, Yes{});
    if constexpr (C::kAhead >= 3)
      stage(kt + 1, std::integral_constant<int, (C::kAhead >= 3 ? C::kAhead - 3 : 0) * kPer>{}, No{}, NoChk{}, Yes{});
    if constexpr (C::kAhead >= 4)
      stage(kt + 2, std::integral_constant<int, (C::kAhead >= 4 ? C::kAhead - 4 : 0) * kPer>{}, No{}, NoChk{}, Yes{});
    stage(kt + C::kAhead - 1, W0{}, No{}, NoChk{}, No{});
  } else {
    // every stage was issued and waited for in the prologue
    for (int kt = 0; kt + 1 < nk; ++kt) stage(kt, W0{}, No{}, NoChk{}, Yes{});
    stage(nk - 1, W0{}, No{}, NoChk{}, No{});
  }
  __syncthreads();  // every wave is past its last read of the ring (the epilogue reuses it)
}

}  // namespace lsk
