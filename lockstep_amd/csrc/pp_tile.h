// Eight-wave ping-pong int8 MFMA main loop for gfx950 (dense and grouped contract GEMMs).
//
// A block of 512 threads computes a BM x BN tile of C = A * W^T over all of K.  Its eight
// waves form two groups of four, one wave of each group per SIMD; the groups run half a
// period apart, so while one group issues its MFMAs the other reads its operand fragments
// from LDS and issues the next global loads.  Each SIMD's matrix core therefore always has a
// wave with operands ready, and the LDS port is used by one group at a time.
//
// K is staged 64 (or 128) bytes at a time through a ring of LDS stages filled by direct
// global -> LDS loads (buffer_load_dwordx4 ... lds: no registers, no LDS write instructions).
// Loads run RING - 1 stages ahead of the stage being multiplied.  A stage holds BM + BN rows
// of 16-byte chunks, XOR-swizzled per row (pp_swz) so that the 16 lanes one LDS cycle serves
// (16 consecutive rows, one logical chunk) touch 16 distinct 16-byte bank groups of the
// 256-byte bank row.
//
// v_mfma_i32_32x32x32_i8: lane l supplies 16 bytes of row l % 32 at K-group l / 32 of both
// operands; the 64-byte stage is two such K-steps.  Integer accumulation is exact in any
// order (|acc| <= K * 127^2 < 2^31), so staging and the chunk permutation never change a bit.
#pragma once
#include <type_traits>

#include "mfma_tile.h"

namespace lsk {

typedef __attribute__((address_space(3))) void* lds_void_t;

template <int BM, int BN, int WM, int WN, int RING = 4, int BKB = 64>
struct PPCfg {
  static_assert(WM * WN == 8, "eight waves");
  static_assert(RING >= 3 && RING <= 5, "ring of 3..5 stages (the ping-pong waits one phase after issue)");
  static constexpr int kThreads = 512;
  static constexpr int kBM = BM, kBN = BN, kWM = WM, kWN = WN;
  static_assert(BKB == 64 || BKB == 128, "64- or 128-byte K stages");
  static constexpr int kBK = BKB;         // bytes of K per stage
  static constexpr int kChunks = BKB / 16;  // 16-byte chunks per row per stage
  static constexpr int kKS = BKB / 32;      // 32-byte MFMA K-steps per stage
  static constexpr int kRing = RING;      // LDS stages
  static constexpr int kAhead = RING - 1; // stages loaded ahead of the one being multiplied
  static constexpr int WTM = BM / WM, WTN = BN / WN;
  static constexpr int TM = WTM / 32, TN = WTN / 32;
  static constexpr int kStageA = BM * kBK, kStageB = BN * kBK, kStage = kStageA + kStageB;  // bytes
  static constexpr int kLA = kStageA / 16 / kThreads;  // 16-byte loads per thread per stage
  static constexpr int kLB = kStageB / 16 / kThreads;
  static constexpr int kMainBytes = kRing * kStage;
  static constexpr int kLdc = WTN + 4;                 // int32 row stride of a staged 32-row strip
  static constexpr int kStripBytes = 32 * kLdc * 4;
  static constexpr int kEpiBytes = 8 * kStripBytes;
  // epilogue operands of the tile: row operand [BM], ws / bias / column exponent [BN] each
  static constexpr int kScaleOff = kMainBytes > kEpiBytes ? kMainBytes : kEpiBytes;
  // eight per-wave flags of the epilogue's fast-path test follow the operands
  static constexpr int kFlagOff = kScaleOff + (BM + 3 * BN) * 4;
  static constexpr int kSmemBytes = kFlagOff + 8 * 4;
  static_assert(BM <= kThreads && BN <= kThreads, "one epilogue operand per thread");
  static_assert(kStageA % (16 * kThreads) == 0 && kStageB % (16 * kThreads) == 0, "tile / threads");
  static_assert(WTM % 32 == 0 && WTN % 32 == 0, "wave tile must be a multiple of 32");
  typedef v16i Acc[TM][TN];
  typedef uint32_t RowsA[kLA];  // byte offset of each load slot's row in its resource (kOob: zero row)
  typedef uint32_t RowsB[kLB];
};

// Tile row loaded by thread `tid` in load slot j of a stage with CHUNKS 16-byte chunks per row,
// and the byte offset within the row's stage segment that it fetches: the logical chunk that
// its LDS slot holds.  Chunk c of row r sits in slot c ^ ((r >> SHIFT) & (CHUNKS - 1)), SHIFT
// chosen so that 16 consecutive rows reading one logical chunk fall in 16 distinct 16-byte
// bank groups of the 256-byte bank row.
template <int CHUNKS>
LSK_DEV int pp_swz(int r) {
  constexpr int kShift = CHUNKS == 4 ? 2 : 1;
  return (r >> kShift) & (CHUNKS - 1);
}
template <int THREADS, int CHUNKS = 4>
LSK_DEV void pp_slot(int tid, int j, int& row, int& kbyte) {
  const int p = j * THREADS + tid;  // 16-byte LDS slot index inside the operand's stage
  row = p / CHUNKS;
  kbyte = 16 * ((p % CHUNKS) ^ pp_swz<CHUNKS>(row));
}

// s_waitcnt vmcnt(n) with the other counters left alone (gfx9 encoding).
template <int N>
LSK_DEV void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}
LSK_DEV void wait_lgkm0() { __builtin_amdgcn_s_waitcnt(0xC07F); }  // lgkmcnt(0), vmcnt/expcnt max

// Keeps the compiler from moving memory operations across this point (a plain load is
// otherwise free to sink to its first use, past a barrier or a counted wait that assumes it
// was issued).
LSK_DEV void compiler_fence() { asm volatile("" ::: "memory"); }

// s_barrier that the instruction scheduler may not move anything across (the phases of the
// ping-pong are defined by where the MFMAs and LDS reads sit relative to the barriers).
LSK_DEV void phase_barrier() {
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_sched_barrier(0);
}

// Byte offset of K byte kk of an operand row relative to the row's offset: kk in the row-major
// layout; kk + (kk & ~63) in the row-pair layout (rows 2i and 2i+1 interleaved by 64-byte K
// chunks, so each 128-byte line holds one chunk of both rows).  `pairs`: bit 0 the A operand,
// bit 1 the B operand in the row-pair layout.
LSK_DEV uint32_t pair_koff(int kk, int paired) { return (uint32_t)(paired ? kk + (kk & ~63) : kk); }

// Issue this thread's direct-to-LDS loads of the first kRing stages of a tile into ring slots
// 0 .. kRing-1, the whole ring (a persistent kernel's next tile, ahead of the current tile's
// stores); chunks past K read zeros.
template <int BM, int BN, int WM, int WN, int RING, int BKB = 64>
LSK_DEV void pp_issue_prologue(__amdgpu_buffer_rsrc_t ra, const typename PPCfg<BM, BN, WM, WN, RING, BKB>::RowsA& pa,
                               __amdgpu_buffer_rsrc_t rb, const typename PPCfg<BM, BN, WM, WN, RING, BKB>::RowsB& pb,
                               int K, char* smem, int pairs = 0) {
  using C = PPCfg<BM, BN, WM, WN, RING, BKB>;
  const int tid = threadIdx.x, wave = wave_id();
  const int nk = (K + C::kBK - 1) / C::kBK;
#pragma unroll
  for (int s = 0; s < C::kRing; ++s) {
    if (s >= nk) break;
    char* st = smem + s * C::kStage;
    const int k0 = s * C::kBK;
#pragma unroll
    for (int j = 0; j < C::kLA; ++j) {
      int r, kbyte;
      pp_slot<C::kThreads, C::kChunks>(tid, j, r, kbyte);
      const int kk = k0 + kbyte;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (lds_void_t)(st + (j * C::kThreads + wave * 64) * 16), 16,
                                               kk < K ? pa[j] + pair_koff(kk, pairs & 1) : kOob, 0, 0, 0);
    }
#pragma unroll
    for (int j = 0; j < C::kLB; ++j) {
      int r, kbyte;
      pp_slot<C::kThreads, C::kChunks>(tid, j, r, kbyte);
      const int kk = k0 + kbyte;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rb, (lds_void_t)(st + C::kStageA + (j * C::kThreads + wave * 64) * 16),
                                               16, kk < K ? pb[j] + pair_koff(kk, pairs & 2) : kOob, 0, 0, 0);
    }
  }
}

// PRE: the first kRing stages were issued by pp_issue_prologue before at least 63 more vector
// memory instructions of this thread (the previous tile's stores).  Vector memory instructions
// complete in issue order and at most 63 are outstanding, so those stages are complete: no wait
// for them; the first step issues nothing (its stage kAhead is in the ring already) and the
// first three steps (which wait for stages 1 .. 3) wait for nothing, leaving the stores to
// drain while stages 0 .. 2 are multiplied.  Needs K / kBK >= kRing + 2 whole stages.
// SKIP (two 32-row strips per wave): only the wave's first na strips hold rows of the tile
// (na in 0 .. 2, wave-uniform), so the fragment reads and MFMAs of the others are left out; their
// accumulators stay zero.  The loads and barriers are the same for every wave.
// PREWAIT (with PRE): the first kRing stages were issued by pp_issue_prologue, and the loop starts
// by waiting for every outstanding vector memory instruction of the thread (for callers whose
// stores after the prologue are fewer or data-dependent).  The lane-dependent offsets are then
// computed afresh on every call (a persistent caller's loop does not keep them live through its
// epilogue).
template <int BM, int BN, int WM, int WN, int RING, int BKB = 64, bool PRE = false, bool SKIP = false,
          bool PREWAIT = false>
LSK_DEV void pp_mainloop(typename PPCfg<BM, BN, WM, WN, RING, BKB>::Acc& acc, __amdgpu_buffer_rsrc_t ra,
                         const typename PPCfg<BM, BN, WM, WN, RING, BKB>::RowsA& pa, __amdgpu_buffer_rsrc_t rb,
                         const typename PPCfg<BM, BN, WM, WN, RING, BKB>::RowsB& pb, int K, char* smem, int na = 0,
                         int pairs = 0) {
  using C = PPCfg<BM, BN, WM, WN, RING, BKB>;
  int tid = threadIdx.x;
  if constexpr (PREWAIT) asm volatile("" : "+v"(tid));
  const int lane = tid & 63, wave = wave_id();
  const int group = wave >> 2;
  const int wm = wave / WN, wn = wave % WN;
  const int nk = (K + C::kBK - 1) / C::kBK;

  // per-slot chunk byte offsets (the LDS side of each load is fixed by the lane); an operand's K
  // offset in its layout is k0x + kx[j] for stage start k0 (a multiple of 64): k0 + k in the
  // row-major layout, 2 k0 + k + (k & 64) in the row-pair layout
  const int ap = pairs & 1, bp = (pairs >> 1) & 1;
  int ka[C::kLA], kb[C::kLB], kax[C::kLA], kbx[C::kLB];
#pragma unroll
  for (int j = 0; j < C::kLA; ++j) {
    int r;
    pp_slot<C::kThreads, C::kChunks>(tid, j, r, ka[j]);
    kax[j] = ka[j] + (ap ? (ka[j] & 64) : 0);
  }
#pragma unroll
  for (int j = 0; j < C::kLB; ++j) {
    int r;
    pp_slot<C::kThreads, C::kChunks>(tid, j, r, kb[j]);
    kbx[j] = kb[j] + (bp ? (kb[j] & 64) : 0);
  }

  // issue this thread's direct-to-LDS loads of stage s; CHECK: the stage may reach past K
  // (chunks there read zeros), otherwise it lies wholly inside K and needs no test
  auto issue = [&](int s, auto check) {
    constexpr bool kCheck = decltype(check)::value;
    char* st = smem + (s % C::kRing) * C::kStage;
    const int k0 = s * C::kBK;
    const int k0a = ap ? 2 * k0 : k0, k0b = bp ? 2 * k0 : k0;
#pragma unroll
    for (int j = 0; j < C::kLA; ++j) {
      const int kk = k0 + ka[j];
      const uint32_t off = (!kCheck || kk < K) ? pa[j] + (uint32_t)(k0a + kax[j]) : kOob;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (lds_void_t)(st + (j * C::kThreads + wave * 64) * 16), 16, off, 0,
                                               0, 0);
    }
#pragma unroll
    for (int j = 0; j < C::kLB; ++j) {
      const int kk = k0 + kb[j];
      const uint32_t off = (!kCheck || kk < K) ? pb[j] + (uint32_t)(k0b + kbx[j]) : kOob;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rb, (lds_void_t)(st + C::kStageA + (j * C::kThreads + wave * 64) * 16), 16, off, 0, 0, 0);
    }
  };
  constexpr int kPer = C::kLA + C::kLB;  // loads per thread per stage

  // fragment addresses: row r = base + (lane & 31), logical chunk 2*ks + (lane >> 5)
  const int lr = lane & 31, sw = pp_swz<C::kChunks>(lr), kg = lane >> 5;
  const int offA = (wm * C::WTM + lr) * C::kBK, offB = C::kStageA + (wn * C::WTN + lr) * C::kBK;
  int slot[C::kKS];
#pragma unroll
  for (int ks = 0; ks < C::kKS; ++ks) slot[ks] = 16 * ((2 * ks + kg) ^ sw);

  // one iteration: [next loads] fragments of stage kt; own part of stage kt+1 complete (at
  // most WAIT younger loads outstanding); barrier; MFMAs; barrier.  WAIT is a compile-time
  // count: the steady state and each step of the drain get their own copy (no branches).
  using Chk = std::true_type;
  using NoChk = std::false_type;
  auto step = [&](int kt, auto wait_n, bool do_issue, auto check) {
    constexpr int kWait = decltype(wait_n)::value;
    if (do_issue) issue(kt + C::kAhead, check);
    const char* st = smem + (kt % C::kRing) * C::kStage;
    v4i fa[C::kKS][C::TM], fb[C::kKS][C::TN];
    // strip i's fragments and MFMAs only where it holds rows (SKIP; na is wave-uniform)
    auto live = [&](int i) { return !SKIP || i < na; };
    const bool any = !SKIP || na > 0;
    if (any) {
#pragma unroll
      for (int ks = 0; ks < C::kKS; ++ks) {
#pragma unroll
        for (int i = 0; i < C::TM; ++i)
          if (live(i)) fa[ks][i] = *(const v4i*)(st + offA + i * 32 * C::kBK + slot[ks]);
#pragma unroll
        for (int j = 0; j < C::TN; ++j) fb[ks][j] = *(const v4i*)(st + offB + j * 32 * C::kBK + slot[ks]);
      }
    }
    wait_vm<kWait>();
    wait_lgkm0();
    phase_barrier();
    if (any) {
#pragma unroll
      for (int ks = 0; ks < C::kKS; ++ks)
#pragma unroll
        for (int i = 0; i < C::TM; ++i)
          if (live(i)) {
#pragma unroll
            for (int j = 0; j < C::TN; ++j) acc[i][j] = mfma_i8_32(fa[ks][i], fb[ks][j], acc[i][j]);
          }
    }
    phase_barrier();
  };
  static_assert(!SKIP || C::TM == 2, "strip skipping takes two 32-row strips per wave");
  using W0 = std::integral_constant<int, 0>;

  // prologue: stages 0 .. kAhead-1 issued together and all waited for (about one latency,
  // like waiting for stage 0 alone).  A counted wait here could also count a caller's plain
  // loads that the compiler placed among these; inside the loop only ring loads are issued,
  // so the counted waits there are exact.
  if constexpr (!PRE) {
#pragma unroll
    for (int s = 0; s < C::kAhead; ++s)
      if (s < nk) issue(s, Chk{});
    wait_vm<0>();
  } else if constexpr (PREWAIT) {
    wait_vm<0>();
  }
  phase_barrier();
  if (group == 1) phase_barrier();

  if (nk >= C::kAhead) {
    // steady state: every iteration issues a whole stage; kAhead - 1 stages stay younger
    // (stages below K / kBK lie wholly inside K; only a last partial stage needs the test)
    using WSteady = std::integral_constant<int, (C::kAhead - 1) * kPer>;
    const int nfull = K / C::kBK;
    int kt = 0;
    if constexpr (PRE) {
      using WNone = std::integral_constant<int, 63>;
      step(0, WNone{}, false, NoChk{});
      step(1, WNone{}, true, NoChk{});
      step(2, WNone{}, true, NoChk{});
      kt = 3;
    }
    for (; kt + C::kAhead < nfull; ++kt) step(kt, WSteady{}, true, NoChk{});
    for (; kt + C::kAhead < nk; ++kt) step(kt, WSteady{}, true, Chk{});
    // drain: the last kAhead stages, nothing more to issue
    step(kt, std::integral_constant<int, (C::kAhead >= 2 ? C::kAhead - 2 : 0) * kPer>{}, false, NoChk{});
    if (C::kAhead >= 2)
      step(kt + 1, std::integral_constant<int, (C::kAhead >= 3 ? C::kAhead - 3 : 0) * kPer>{}, false, NoChk{});
    if (C::kAhead >= 3)
      step(kt + 2, std::integral_constant<int, (C::kAhead >= 4 ? C::kAhead - 4 : 0) * kPer>{}, false, NoChk{});
    if (C::kAhead >= 4) step(kt + 3, W0{}, false, NoChk{});
  } else {
    // fewer stages than the ring holds: all were issued and waited for in the prologue
    for (int kt = 0; kt < nk; ++kt) step(kt, W0{}, false, NoChk{});
  }
  if (group == 0) phase_barrier();
}

// Stage 32-row strip i of the wave's accumulators (rows 32i .. 32i+31 of the wave tile) into
// the wave's LDS region, row stride LDC int32.  MFMA layout: register r of lane l holds row
// 8 (r / 4) + 4 (l / 32) + r % 4, column l % 32 of each 32 x 32 block.
template <int TN, int LDC>
LSK_DEV void pp_stage_strip(const v16i* strip, int32_t* region) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int j = 0; j < TN; ++j)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int row = 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
      region[row * LDC + j * 32 + (lane & 31)] = strip[j][r];
    }
}

}  // namespace lsk
