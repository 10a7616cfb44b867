// The MXFP4-consuming operand (contract addendum item 5, reference/moe_ref.py:233-255) on gfx950.
//
//   for every 32-wide K block b, ascending:
//     s_b = sum_{j in b} a[m, j] * m2[n, j]             exact (|s_b| <= 32 * 127 * 12 < 2^16)
//     acc = fl32(acc + s_b * 2^(kexp[n, b] - 128))     one rounding per block, from +0
//
// Operands are staged into LDS as bf16: int8 activations and doubled fp4 mantissas m2 are small
// integers, exact in bf16.  v_mfma_f32_16x16x32_bf16 contracts exactly one block (K = 32) from a
// zero accumulator, so its result is the exact integer s_b (every partial sum is an integer
// below 2^16, exact in any summation order).  The block update is one FMA: s_b * 2^(k-128) is
// exact in binary32 unless it overflows, which needs an exponent byte >= 240, so
// fma(s_b, 2^(k-128), acc) rounds exactly once, like the reference's multiply-then-add.  Weight
// sets holding an exponent byte >= 240 take the SAFE variant (a multiply, then an add).
// Blocks are never summed together before rounding and K is never split.
//
// ROWSCALE adds a per-row block exponent ka[m, b] (block-scaled activations, moe_ref.py:317-326):
// the update becomes acc = fl32(acc + fl32(s_b * p)) with p = fl32(2^ka * 2^(kexp - 128)), the
// correctly rounded 2^(ka + kexp - 128) (0 below 2^-149, inf from 2^128), always as a multiply
// and then an add.
#pragma once
#include "mfma_tile.h"

namespace lsk {

typedef __bf16 v8bf __attribute__((ext_vector_type(8)));

LSK_DEV v4f mfma_bf16(v4i a, v4i b) {
  const v4f z = {0.0f, 0.0f, 0.0f, 0.0f};
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8bf, a), __builtin_bit_cast(v8bf, b), z, 0, 0, 0);
}

// bf16 bit patterns of the doubled E2M1 magnitudes 0, 1, 2, 3, 4, 6, 8, 12.
LSK_DEV uint32_t m2_bf16(uint32_t code) {
  const uint32_t mag = code & 7u;
  const uint32_t b = mag >= 2u ? mag * 64u + 16256u : (mag == 1u ? 16256u : 0u);
  return b | ((code & 8u) << 12);
}

// int8 value -> bf16 bits (exact for |v| <= 256)
LSK_DEV uint32_t i8_bf16(int v) { return __float_as_uint((float)v) >> 16; }

// 16 int8 -> 16 bf16 (two 16-byte chunks)
LSK_DEV void i8x16_to_bf16(v4i in, v4i& lo, v4i& hi) {
  uint32_t o[8];
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const uint32_t u = (uint32_t)in[w];
    const int b0 = (int)(int8_t)(u & 0xff), b1 = (int)(int8_t)((u >> 8) & 0xff);
    const int b2 = (int)(int8_t)((u >> 16) & 0xff), b3 = (int)(int8_t)(u >> 24);
    o[2 * w] = i8_bf16(b0) | (i8_bf16(b1) << 16);
    o[2 * w + 1] = i8_bf16(b2) | (i8_bf16(b3) << 16);
  }
  lo = v4i{(int)o[0], (int)o[1], (int)o[2], (int)o[3]};
  hi = v4i{(int)o[4], (int)o[5], (int)o[6], (int)o[7]};
}

// 32 packed fp4 codes (element 2i in the low nibble of byte i) -> 32 bf16 m2 values (4 chunks).
// gfx950's v_cvt_scalef32_pk_bf16_fp4 with scale 2 converts the two codes of one byte (low
// nibble first) to bf16 2 * fp4 = m2, exactly (checked against m2_bf16 over every code byte on
// MI355X).
LSK_DEV void fp4x32_to_bf16(v4i in, v4i (&out)[4]) {
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const uint32_t u = (uint32_t)in[w];
    const uint32_t o0 = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(u, 2.0f, 0));
    const uint32_t o1 = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(u, 2.0f, 1));
    const uint32_t o2 = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(u, 2.0f, 2));
    const uint32_t o3 = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(u, 2.0f, 3));
    out[w] = v4i{(int)o0, (int)o1, (int)o2, (int)o3};
  }
}

// Tile configuration: BM x BN outputs, BK = 32 * NB elements of K per LDS stage.
template <int BM, int BN, int WM, int WN, int NB>
struct MxCfg {
  static constexpr int kThreads = WM * WN * 64;
  static constexpr int WTM = BM / WM, WTN = BN / WN;
  static constexpr int TM = WTM / 16, TN = WTN / 16;
  static constexpr int BK = 32 * NB;
  static constexpr int kRowChunks = BK * 2 / 16;                 // 16-byte bf16 chunks per LDS row
  static constexpr int kSmemA = BM * kRowChunks, kSmemB = BN * kRowChunks;  // v4i per stage
  static constexpr int kScale = BN * NB;                          // floats per stage
  static constexpr int kScaleA = BM * NB;                         // row scales per stage (ROWSCALE)
  static constexpr int kStageBytes = (kSmemA + kSmemB) * 16 + (kScale + kScaleA) * 4;
  static constexpr int kLdc = WTN + 4;
  static constexpr int kStripFloats = 16 * kLdc;
  static constexpr int kEpiBytes = WM * WN * kStripFloats * 4;
  static constexpr int kSmemBytes = 2 * kStageBytes > kEpiBytes ? 2 * kStageBytes : kEpiBytes;
  typedef v4f Acc[TM][TN];
  static_assert(WTM % 16 == 0 && WTN % 16 == 0, "wave tile");
  static_assert(kRowChunks <= 16, "swizzle assumes at most 16 chunks per row");
};

// Physical LDS chunk of logical chunk c in row r (XOR swizzle over the row's chunks).
template <int RC>
LSK_DEV int swz(int r, int c) {
  return r * RC + (c ^ (r & (RC - 1)));
}

// acc[TM][TN] (binary32) accumulates the MX blocks of this tile in ascending order.
// rowA(r): tile row r's activation row (bf16 [K] or int8 [K]; null = zero row);
// rowB(r): tile row r's weight row (packed fp4 [K/2] or m2 int8 [K]; null = zero row);
// rowS(r): its e8m0 exponents [K/32]; rowK(r) (ROWSCALE only): tile row r's block exponents
// ka [K/32] (int32; null = all 0).  Each is evaluated once per load slot, before the K loop.
template <int BM, int BN, int WM, int WN, int NB, bool A_I8, bool B_FP4, bool SAFE, bool ROWSCALE, class FA, class FB,
          class FS, class FK>
LSK_DEV void mx_mainloop(typename MxCfg<BM, BN, WM, WN, NB>::Acc& acc, FA rowA, FB rowB, FS rowS, FK rowK, int K,
                         char* smem) {
  using C = MxCfg<BM, BN, WM, WN, NB>;
  constexpr int T = C::kThreads;
  constexpr int RC = C::kRowChunks;
  // per stage: A global chunks (16 B): bf16 rows BM * RC, int8 rows BM * RC / 2
  constexpr int kAG = A_I8 ? BM * RC / 2 : BM * RC;
  constexpr int kAPer = (kAG + T - 1) / T;
  // B global chunks: fp4 rows hold BK / 2 bytes = RC / 4 chunks; m2 rows RC / 2 chunks
  constexpr int kBG = B_FP4 ? BN * RC / 4 : BN * RC / 2;
  constexpr int kBPer = (kBG + T - 1) / T;
  constexpr int kAChunksPerRow = A_I8 ? RC / 2 : RC;
  constexpr int kBChunksPerRow = B_FP4 ? RC / 4 : RC / 2;

  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
  const int wm = wave / WN, wn = wave % WN;

  constexpr int kSPer = (BN * NB + T - 1) / T;  // scale bytes per thread per stage
  constexpr int kKPer = ROWSCALE ? (BM * NB + T - 1) / T : 0;  // row exponents per thread per stage
  const char* pa[kAPer];
  const uint8_t* pb[kBPer];
  const uint8_t* ps[kSPer];
  const int32_t* pk[kKPer > 0 ? kKPer : 1];
#pragma unroll
  for (int j = 0; j < kAPer; ++j) {
    const int i = tid + j * T;
    pa[j] = i < kAG ? (const char*)rowA(i / kAChunksPerRow) : nullptr;
  }
#pragma unroll
  for (int j = 0; j < kBPer; ++j) {
    const int i = tid + j * T;
    pb[j] = i < kBG ? rowB(i / kBChunksPerRow) : nullptr;
  }
#pragma unroll
  for (int j = 0; j < kSPer; ++j) {
    const int i = tid + j * T;
    ps[j] = i < BN * NB ? rowS(i / NB) : nullptr;
  }
#pragma unroll
  for (int j = 0; j < kKPer; ++j) {
    const int i = tid + j * T;
    pk[j] = i < BM * NB ? rowK(i / NB) : nullptr;
  }
  v4i ra[kAPer], rb[kBPer];
  uint32_t rs[kSPer];
  int rk[kKPer > 0 ? kKPer : 1];
  auto gload = [&](int k0) {
#pragma unroll
    for (int j = 0; j < kAPer; ++j) {
      const int i = tid + j * T;
      const int c = i % kAChunksPerRow;
      const int elem = k0 + c * (A_I8 ? 16 : 8);
      ra[j] = (pa[j] && elem < K) ? *(const v4i*)(pa[j] + (A_I8 ? elem : 2 * elem)) : zero4();
    }
#pragma unroll
    for (int j = 0; j < kBPer; ++j) {
      const int i = tid + j * T;
      const int c = i % kBChunksPerRow;
      const int elem = k0 + c * (B_FP4 ? 32 : 16);
      rb[j] = (pb[j] && elem < K) ? *(const v4i*)(pb[j] + (B_FP4 ? elem / 2 : elem)) : zero4();
    }
#pragma unroll
    for (int j = 0; j < kSPer; ++j) {
      const int i = tid + j * T;
      const int b = i % NB;
      rs[j] = (ps[j] && k0 + 32 * b < K) ? ps[j][k0 / 32 + b] : 128u;
    }
#pragma unroll
    for (int j = 0; j < kKPer; ++j) {
      const int i = tid + j * T;
      const int b = i % NB;
      rk[j] = (pk[j] && k0 + 32 * b < K) ? pk[j][k0 / 32 + b] : 0;
    }
  };
  auto sstore = [&](int buf) {
    v4i* sA = (v4i*)(smem + buf * C::kStageBytes);
    v4i* sB = sA + C::kSmemA;
    float* sS = (float*)(sB + C::kSmemB);
#pragma unroll
    for (int j = 0; j < kAPer; ++j) {
      const int i = tid + j * T;
      if (i < kAG) {
        const int row = i / kAChunksPerRow, c = i - row * kAChunksPerRow;
        if (A_I8) {
          v4i lo, hi;
          i8x16_to_bf16(ra[j], lo, hi);
          sA[swz<RC>(row, 2 * c)] = lo;
          sA[swz<RC>(row, 2 * c + 1)] = hi;
        } else {
          sA[swz<RC>(row, c)] = ra[j];
        }
      }
    }
#pragma unroll
    for (int j = 0; j < kBPer; ++j) {
      const int i = tid + j * T;
      if (i < kBG) {
        const int row = i / kBChunksPerRow, c = i - row * kBChunksPerRow;
        if (B_FP4) {
          v4i o[4];
          fp4x32_to_bf16(rb[j], o);
#pragma unroll
          for (int q = 0; q < 4; ++q) sB[swz<RC>(row, 4 * c + q)] = o[q];
        } else {
          v4i lo, hi;
          i8x16_to_bf16(rb[j], lo, hi);
          sB[swz<RC>(row, 2 * c)] = lo;
          sB[swz<RC>(row, 2 * c + 1)] = hi;
        }
      }
    }
#pragma unroll
    for (int j = 0; j < kSPer; ++j) {
      const int i = tid + j * T;
      if (i < BN * NB) sS[i] = pow2f((int)rs[j] - 128);
    }
#pragma unroll
    for (int j = 0; j < kKPer; ++j) {
      const int i = tid + j * T;
      if (i < BM * NB) sS[C::kScale + (i % NB) * BM + i / NB] = pow2f(rk[j]);  // ka in [-126, 127]
    }
  };

  const int nk = (K + C::BK - 1) / C::BK;
  gload(0);
  sstore(0);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < nk) gload((kt + 1) * C::BK);
    const v4i* sA = (const v4i*)(smem + buf * C::kStageBytes);
    const v4i* sB = sA + C::kSmemA;
    const float* sS = (const float*)(sB + C::kSmemB);
    const int kbase = kt * C::BK;
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      if (kbase + 32 * b >= K) break;
      const int c = b * 4 + (lane >> 4);
      v4i af[C::TM], bf[C::TN];
      float sc[C::TN];
      v4f sa[C::TM];
      if (ROWSCALE) {
        // the C rows of lane l in a 16x16 tile are 4 (l / 16) + r
#pragma unroll
        for (int i = 0; i < C::TM; ++i) sa[i] = *(const v4f*)(sS + C::kScale + b * BM + wm * C::WTM + i * 16 + 4 * (lane >> 4));
      }
#pragma unroll
      for (int i = 0; i < C::TM; ++i) af[i] = sA[swz<RC>(wm * C::WTM + i * 16 + (lane & 15), c)];
#pragma unroll
      for (int j = 0; j < C::TN; ++j) {
        const int r = wn * C::WTN + j * 16 + (lane & 15);
        bf[j] = sB[swz<RC>(r, c)];
        sc[j] = sS[r * NB + b];
      }
#pragma unroll
      for (int i = 0; i < C::TM; ++i)
#pragma unroll
        for (int j = 0; j < C::TN; ++j) {
          const v4f d = mfma_bf16(af[i], bf[j]);
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            if (ROWSCALE) acc[i][j][r] = f32_add(acc[i][j][r], f32_mul(d[r], f32_mul(sa[i][r], sc[j])));
            else if (SAFE) acc[i][j][r] = f32_add(acc[i][j][r], f32_mul(d[r], sc[j]));
            else acc[i][j][r] = __builtin_fmaf(d[r], sc[j], acc[i][j][r]);
          }
        }
    }
    if (kt + 1 < nk) sstore(buf ^ 1);
    __syncthreads();
  }
}

// Write the 16-row strip of this wave's binary32 accumulators into its LDS region.
template <int TN, int LDC>
LSK_DEV void stage_strip_f(const v4f* strip, float* region) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int j = 0; j < TN; ++j)
#pragma unroll
    for (int r = 0; r < 4; ++r) region[((lane >> 4) * 4 + r) * LDC + j * 16 + (lane & 15)] = strip[j][r];
}

}  // namespace lsk
