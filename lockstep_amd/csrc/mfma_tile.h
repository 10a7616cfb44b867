// The exact int8 MFMA tile main loop shared by the dense and grouped (MoE) GEMMs on gfx950.
//
// One block computes a BM x BN tile of C = A * W^T over the whole K range.  Rows of A and W
// are addressed through per-thread row pointers fixed before the K loop, so a caller can
// gather rows (MoE token rows), interleave weight rows (gate/up pairs) or clip at the matrix
// edge (a null pointer loads zeros).  K stages of 128 bytes are double-buffered in LDS as
// 16-byte chunks whose position within a row is XOR-swizzled by the row index, so the
// 16 lanes that read one MFMA operand column hit 16 distinct bank groups.
//
// v_mfma_i32_16x16x64_i8: lane l supplies 16 bytes of row (l % 16) at K-group (l / 16) of the
// A operand and of the W operand alike; D[i][j] lands in lane j + 16 * (i / 4), register i % 4.
// Integer accumulation is exact in any order (|acc| <= K * 127^2 < 2^31), so the K blocking
// never changes a result.
//
// Results leave the registers through LDS one 16-row strip at a time (per wave, static
// register indices), and are read back four consecutive columns per lane so the epilogue
// issues full-width, coalesced stores.
#pragma once
#include "lsk_common.h"

namespace lsk {

constexpr int kBK = 128;  // bytes of K per LDS stage

LSK_DEV v4i mfma_i8(v4i a, v4i b, v4i c) { return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0); }
LSK_DEV v4i zero4() { return v4i{0, 0, 0, 0}; }

template <int BM, int BN, int WM, int WN>
struct TileCfg {
  static constexpr int kThreads = WM * WN * 64;
  static constexpr int WTM = BM / WM, WTN = BN / WN;
  static constexpr int TM = WTM / 16, TN = WTN / 16;
  static constexpr int kAPer = BM * kBK / 16 / kThreads;  // 16-byte chunks per thread per stage
  static constexpr int kBPer = BN * kBK / 16 / kThreads;
  static constexpr int kSmemA = BM * 8, kSmemB = BN * 8;  // v4i chunks per stage
  static constexpr int kLdc = WTN + 4;                     // int32 row stride of a staged strip
  static constexpr int kStripInts = 16 * kLdc;             // per wave
  static constexpr int kMainBytes = 2 * (kSmemA + kSmemB) * 16;
  static constexpr int kEpiBytes = WM * WN * kStripInts * 4;
  static constexpr int kSmemBytes = kMainBytes > kEpiBytes ? kMainBytes : kEpiBytes;
  static_assert((BM * kBK / 16) % kThreads == 0 && (BN * kBK / 16) % kThreads == 0, "tile/threads");
  static_assert(WTM % 16 == 0 && WTN % 16 == 0, "wave tile must be a multiple of 16");
  typedef v4i Acc[TM][TN];
  typedef const int8_t* RowsA[kAPer];
  typedef const int8_t* RowsB[kBPer];
};

// Row index (within the tile) and 16-byte chunk index that thread `tid` loads in slot j.
template <int THREADS>
LSK_DEV void chunk_of(int tid, int j, int& row, int& c) {
  const int i = tid + j * THREADS;
  row = i >> 3;
  c = i & 7;
}

// acc[TM][TN] += A_tile * W_tile^T over K (K % 16 == 0; row pointers 16-byte aligned).
// pa / pb: the global row pointers of this thread's load slots (null = zero row).
template <int BM, int BN, int WM, int WN>
LSK_DEV void mfma_mainloop(typename TileCfg<BM, BN, WM, WN>::Acc& acc, const typename TileCfg<BM, BN, WM, WN>::RowsA& pa,
                           const typename TileCfg<BM, BN, WM, WN>::RowsB& pb, int K, v4i* smem) {
  using C = TileCfg<BM, BN, WM, WN>;
  v4i* sA = smem;
  v4i* sB = smem + 2 * C::kSmemA;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;

  v4i ra[C::kAPer], rb[C::kBPer];
  auto gload = [&](int k0) {
#pragma unroll
    for (int j = 0; j < C::kAPer; ++j) {
      int row, c;
      chunk_of<C::kThreads>(tid, j, row, c);
      const int gk = k0 + c * 16;
      ra[j] = (pa[j] && gk < K) ? *(const v4i*)(pa[j] + gk) : zero4();
    }
#pragma unroll
    for (int j = 0; j < C::kBPer; ++j) {
      int row, c;
      chunk_of<C::kThreads>(tid, j, row, c);
      const int gk = k0 + c * 16;
      rb[j] = (pb[j] && gk < K) ? *(const v4i*)(pb[j] + gk) : zero4();
    }
  };
  auto sstore = [&](int buf) {
#pragma unroll
    for (int j = 0; j < C::kAPer; ++j) {
      int row, c;
      chunk_of<C::kThreads>(tid, j, row, c);
      sA[buf * C::kSmemA + row * 8 + (c ^ (row & 7))] = ra[j];
    }
#pragma unroll
    for (int j = 0; j < C::kBPer; ++j) {
      int row, c;
      chunk_of<C::kThreads>(tid, j, row, c);
      sB[buf * C::kSmemB + row * 8 + (c ^ (row & 7))] = rb[j];
    }
  };

  const int nk = (K + kBK - 1) / kBK;
  gload(0);
  sstore(0);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < nk) gload((kt + 1) * kBK);
    const v4i* a_s = sA + buf * C::kSmemA;
    const v4i* b_s = sB + buf * C::kSmemB;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const int c = ks * 4 + (lane >> 4);
      v4i af[C::TM], bf[C::TN];
#pragma unroll
      for (int i = 0; i < C::TM; ++i) {
        const int r = wm * C::WTM + i * 16 + (lane & 15);
        af[i] = a_s[r * 8 + (c ^ (r & 7))];
      }
#pragma unroll
      for (int j = 0; j < C::TN; ++j) {
        const int r = wn * C::WTN + j * 16 + (lane & 15);
        bf[j] = b_s[r * 8 + (c ^ (r & 7))];
      }
#pragma unroll
      for (int i = 0; i < C::TM; ++i)
#pragma unroll
        for (int j = 0; j < C::TN; ++j) acc[i][j] = mfma_i8(af[i], bf[j], acc[i][j]);
    }
    if (kt + 1 < nk) sstore(buf ^ 1);
    __syncthreads();
  }
}

// Write the 16-row strip `strip` of this wave's accumulators into the wave's LDS region
// (row stride TileCfg::kLdc int32).  Called after the main loop's final barrier; the region
// is private to the wave, and a wave's LDS accesses complete in program order.
template <int TN, int LDC>
LSK_DEV void stage_strip(const v4i* strip, int32_t* region) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int j = 0; j < TN; ++j)
#pragma unroll
    for (int r = 0; r < 4; ++r) region[((lane >> 4) * 4 + r) * LDC + j * 16 + (lane & 15)] = strip[j][r];
}

// Map a hardware block id to a logical tile id so the blocks one XCD runs (hardware ids
// congruent mod 8: dispatch is round-robin over the 8 XCDs) form one contiguous run of
// logical ids, sharing their operand panels in that XCD's L2.
LSK_DEV int xcd_logical_id(int b, int nblocks) {
  const int per = nblocks / 8, rem = nblocks % 8;
  const int x = b % 8, i = b / 8;
  return x * per + (x < rem ? x : rem) + i;
}

}  // namespace lsk
