// The exact int8 MFMA tile main loop shared by the dense and grouped (MoE) GEMMs on gfx950.
//
// One block computes a BM x BN tile of C = A * W^T over the whole K range.  Rows of A and W
// are addressed through per-thread row pointers fixed before the K loop, so a caller can
// gather rows (MoE token rows), interleave weight rows (gate/up pairs) or clip at the matrix
// edge (a null pointer loads zeros).  K stages of 128 bytes are double-buffered in LDS as
// 16-byte chunks; chunk c of row r sits at position c ^ ((r >> 1) & 7), so any 16 consecutive
// rows reading one logical chunk hit 16 distinct 16-byte bank groups (two 128-byte rows span
// the 64 four-byte banks).
//
// v_mfma_i32_32x32x32_i8 (measured at 97% of the 5.0 POPS int8 peak in a register-only loop
// with constant operands; the 16x16x64 form stalls near 55-70%): lane l supplies 16 bytes of row (l % 32) at K-group
// (l / 32) of the A operand and of the W operand alike; D[i][j] lands in lane j + 32 * ((i / 4) % 2),
// register 4 * (i / 8) + i % 4.  Integer accumulation is exact in any order (|acc| <= K * 127^2
// < 2^31), so the K blocking never changes a result.
//
// Results leave the registers through LDS 16 rows at a time (per wave, static register indices)
// and are read back four consecutive columns per lane, so the epilogue issues full-width,
// coalesced stores.
#pragma once
#include "lsk_common.h"

namespace lsk {

constexpr int kBK = 128;  // bytes of K per LDS stage

LSK_DEV v16i mfma_i8_32(v4i a, v4i b, v16i c) { return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0); }
LSK_DEV v4i mfma_i8(v4i a, v4i b, v4i c) { return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0); }
LSK_DEV v4i zero4() { return v4i{0, 0, 0, 0}; }
LSK_DEV v16i zero16() { return v16i{0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0}; }

// Raw buffer loads: an access at or beyond the resource's byte range returns zero in hardware,
// so edge rows and the K tail need no branch around the load (branches around loads also stop
// the compiler from counting outstanding loads, which serialises the prefetch).
constexpr uint32_t kOob = 0x80000000u;  // an offset beyond any resource range used here

LSK_DEV __amdgpu_buffer_rsrc_t make_rsrc(const void* base, int64_t bytes) {
  const int n = bytes > 0x7fffffff ? 0x7fffffff : (int)bytes;
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, n, 0x00020000);
}

LSK_DEV v4i buf_load16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0));
}

// Position of 16-byte chunk c (0..7) of row r in a tile of 128-byte rows.
LSK_DEV int swz8(int r, int c) { return r * 8 + (c ^ ((r >> 1) & 7)); }

template <int BM, int BN, int WM, int WN>
struct TileCfg {
  static constexpr int kThreads = WM * WN * 64;
  static constexpr int WTM = BM / WM, WTN = BN / WN;
  static constexpr int TM = WTM / 32, TN = WTN / 32;       // 32x32 MFMA tiles per wave
  static constexpr int kAPer = BM * kBK / 16 / kThreads;  // 16-byte chunks per thread per stage
  static constexpr int kBPer = BN * kBK / 16 / kThreads;
  static constexpr int kSmemA = BM * 8, kSmemB = BN * 8;  // v4i chunks per stage
  static constexpr int kLdc = WTN + 8;                     // int32 row stride of a staged half strip
  static constexpr int kStripInts = 16 * kLdc;             // per wave
  static constexpr int kMainBytes = 2 * (kSmemA + kSmemB) * 16;
  static constexpr int kEpiBytes = WM * WN * kStripInts * 4;
  static constexpr int kSmemBytes = kMainBytes > kEpiBytes ? kMainBytes : kEpiBytes;
  static_assert((BM * kBK / 16) % kThreads == 0 && (BN * kBK / 16) % kThreads == 0, "tile/threads");
  static_assert(WTM % 32 == 0 && WTN % 32 == 0, "wave tile must be a multiple of 32");
  typedef v16i Acc[TM][TN];
  typedef uint32_t RowsA[kAPer];  // byte offset of each load slot's row in its resource (kOob: zero row)
  typedef uint32_t RowsB[kBPer];
};

// Row index (within the tile) and 16-byte chunk index that thread `tid` loads in slot j.
template <int THREADS>
LSK_DEV void chunk_of(int tid, int j, int& row, int& c) {
  const int i = tid + j * THREADS;
  row = i >> 3;
  c = i & 7;
}

// acc[TM][TN] += A_tile * W_tile^T over K (K % 16 == 0; rows 16-byte aligned).
// ra_res / rb_res: buffer resources over the operands; pa / pb: the byte offsets of this thread's
// load-slot rows in them (kOob = zero row).
template <int BM, int BN, int WM, int WN>
LSK_DEV void mfma_mainloop(typename TileCfg<BM, BN, WM, WN>::Acc& acc, __amdgpu_buffer_rsrc_t ra_res,
                           const typename TileCfg<BM, BN, WM, WN>::RowsA& pa, __amdgpu_buffer_rsrc_t rb_res,
                           const typename TileCfg<BM, BN, WM, WN>::RowsB& pb, int K, v4i* smem) {
  using C = TileCfg<BM, BN, WM, WN>;
  v4i* sA = smem;
  v4i* sB = smem + 2 * C::kSmemA;
  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
  const int wm = wave / WN, wn = wave % WN;

  v4i ra[C::kAPer], rb[C::kBPer];
  auto gload = [&](int k0) {
#pragma unroll
    for (int j = 0; j < C::kAPer; ++j) {
      int row, c;
      chunk_of<C::kThreads>(tid, j, row, c);
      const int gk = k0 + c * 16;
      ra[j] = buf_load16(ra_res, gk < K ? pa[j] + (uint32_t)gk : kOob);
    }
#pragma unroll
    for (int j = 0; j < C::kBPer; ++j) {
      int row, c;
      chunk_of<C::kThreads>(tid, j, row, c);
      const int gk = k0 + c * 16;
      rb[j] = buf_load16(rb_res, gk < K ? pb[j] + (uint32_t)gk : kOob);
    }
  };
  auto sstore = [&](int buf) {
#pragma unroll
    for (int j = 0; j < C::kAPer; ++j) {
      int row, c;
      chunk_of<C::kThreads>(tid, j, row, c);
      sA[buf * C::kSmemA + swz8(row, c)] = ra[j];
    }
#pragma unroll
    for (int j = 0; j < C::kBPer; ++j) {
      int row, c;
      chunk_of<C::kThreads>(tid, j, row, c);
      sB[buf * C::kSmemB + swz8(row, c)] = rb[j];
    }
  };
  auto compute = [&](int buf) {
    const v4i* a_s = sA + buf * C::kSmemA;
    const v4i* b_s = sB + buf * C::kSmemB;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const int c = ks * 2 + (lane >> 5);
      v4i af[C::TM], bf[C::TN];
#pragma unroll
      for (int i = 0; i < C::TM; ++i) af[i] = a_s[swz8(wm * C::WTM + i * 32 + (lane & 31), c)];
#pragma unroll
      for (int j = 0; j < C::TN; ++j) bf[j] = b_s[swz8(wn * C::WTN + j * 32 + (lane & 31), c)];
#pragma unroll
      for (int i = 0; i < C::TM; ++i)
#pragma unroll
        for (int j = 0; j < C::TN; ++j) acc[i][j] = mfma_i8_32(af[i], bf[j], acc[i][j]);
    }
  };

  const int nk = (K + kBK - 1) / kBK;
  gload(0);
  sstore(0);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < nk) gload((kt + 1) * kBK);
    compute(buf);
    if (kt + 1 < nk) sstore(buf ^ 1);
    __syncthreads();
  }
}

// Write half h (rows 16h .. 16h+15) of the wave's 32-row strip `strip` into the wave's LDS
// region (row stride LDC int32).  Called after the main loop's final barrier.
template <int TN, int LDC>
LSK_DEV void stage_half(const v16i* strip, int h, int32_t* region) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int j = 0; j < TN; ++j)
#pragma unroll
    for (int rr = 0; rr < 8; ++rr) {
      const int row = 8 * (rr >> 2) + 4 * (lane >> 5) + (rr & 3);
      region[row * LDC + j * 32 + (lane & 31)] = strip[j][8 * h + rr];
    }
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
