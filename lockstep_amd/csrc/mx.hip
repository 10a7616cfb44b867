// MXFP4 kernels on gfx950: the MX-operand GEMM (dense and grouped for the MoE layer), the exact
// E2M1/E8M0 dequant, and the doubled-mantissa packer.  See mx_tile.h for the exactness argument.
#include <atomic>

#include "contract_act.h"
#include "moe_internal.h"
#include "moe_route.h"
#include "mx_pp.h"
#include "mx_tile.h"

namespace {

constexpr float kAmaxFloor = 0x1.5798eep-27f;  // fl32(1e-8)
constexpr int NB = 2;                          // MX blocks per LDS stage (K = 64)
using Cfg = lsk::MxCfg<128, 128, 2, 2, NB>;

template <class K>
int reserve_lds(K kern, int bytes, const char* name) {
  if (hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, bytes) != hipSuccess) {
    lsk::set_error("%s: cannot reserve %d bytes of LDS", name, bytes);
    return LSK_ERR_HIP;
  }
  return LSK_OK;
}

// ---------------------------------------------------------------- quantisers emitting bf16 values
LSK_DEV uint16_t q_bf16(float v, float s, float r) {
  const float t = fminf(fmaxf(rint_div8(v, s, r), -127.0f), 127.0f);
  return (uint16_t)(__float_as_uint(t) >> 16);  // an integer of magnitude <= 127: exact in bf16
}

__global__ __launch_bounds__(256) void rowquant_bf16_kernel(const uint16_t* __restrict__ x, int64_t H,
                                                            uint16_t* __restrict__ q, float* __restrict__ asc) {
  __shared__ float red[4];
  const int64_t t = blockIdx.x;
  const uint16_t* row = x + t * H;
  float am = 0.0f;
  for (int64_t i = threadIdx.x; i < H; i += 256) am = fmaxf(am, fabsf(bf16_to_f32(row[i])));
  am = wave_fmax(am);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = am;
  __syncthreads();
  am = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  const float s = f32_div(fmaxf(am, kAmaxFloor), 127.0f), rs = f32_div(1.0f, s);
  if (threadIdx.x == 0) asc[t] = s;
  for (int64_t i = threadIdx.x; i < H; i += 256) q[t * H + i] = q_bf16(bf16_to_f32(row[i]), s, rs);
}

__global__ __launch_bounds__(256) void requant_bf16_kernel(const uint16_t* __restrict__ h, const uint32_t* __restrict__ amax,
                                                           const int32_t* __restrict__ nrows, int I,
                                                           uint16_t* __restrict__ q, float* __restrict__ asc) {
  const int R = *nrows;
  const int chunks = I / 8;
  const int64_t total = (int64_t)R * chunks;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
    const int64_t p = i / chunks;
    const int c = (int)(i - p * chunks);
    const float s = f32_div(fmaxf(__uint_as_float(amax[p]), kAmaxFloor), 127.0f), rs = f32_div(1.0f, s);
    if (c == 0) asc[p] = s;
    const uint4 u = *(const uint4*)(h + p * I + c * 8);
    const uint32_t wd[4] = {u.x, u.y, u.z, u.w};
    uint32_t o[4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
      o[j] = (uint32_t)q_bf16(bf16_to_f32((uint16_t)(wd[j] & 0xffff)), s, rs) |
             ((uint32_t)q_bf16(bf16_to_f32((uint16_t)(wd[j] >> 16)), s, rs) << 16);
    store16_split(q + p * I + c * 8, o[0], o[1], o[2], o[3]);
  }
}

// ---------------------------------------------------------------- block quant (block-scaled activations)
// moe_ref.py:299-314.  ka = the least k with 127 * 2^k >= am (am = max |x| over the 32-wide
// block), clamped to [-126, 127]; -126 for an all-zero block.  With am = 1.f * 2^(be - 127) (its
// binary32 fields), 127 * 2^k >= am  <=>  k >= be - 133 when 1.f <= 127/64 (fraction field
// <= 0x7E0000), else k >= be - 132.  The reference's ceil(log2(fl32(am / 127))), raised by one
// where fl32(127 * 2^ka) < am, is the same least k.  q = clamp(rint(x * 2^-ka), +-127): x * 2^-ka
// and the reference's x / 2^ka are the same correctly rounded quotient.  Infinite inputs give
// ka = 127 and q = +-127; NaN has no defined quantisation in the reference.
LSK_DEV int mx2_block_exp(float am) {
  const uint32_t u = __float_as_uint(am);
  const int be = (int)(u >> 23);
  if (be == 0) return -126;   // zero or subnormal
  if (be >= 255) return 127;  // infinity
  const int k = be - ((u & 0x7fffffu) <= 0x7e0000u ? 133 : 132);
  return k < -126 ? -126 : k;
}

LSK_DEV float mx2_q(float v, float inv) { return fminf(fmaxf(rintf(f32_mul(v, inv)), -127.0f), 127.0f); }

// 8 consecutive elements (bf16 bits or binary32) as binary32
template <bool X_F32>
LSK_DEV void load8(const void* x, int64_t off, float (&v)[8]) {
  if (X_F32) {
    const float4 a = *(const float4*)((const float*)x + off), b = *(const float4*)((const float*)x + off + 4);
    v[0] = a.x, v[1] = a.y, v[2] = a.z, v[3] = a.w, v[4] = b.x, v[5] = b.y, v[6] = b.z, v[7] = b.w;
  } else {
    const uint4 u = *(const uint4*)((const uint16_t*)x + off);
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      v[2 * j] = bf16_to_f32((uint16_t)(w[j] & 0xffff));
      v[2 * j + 1] = bf16_to_f32((uint16_t)(w[j] >> 16));
    }
  }
}

// the block maximum of the 8 values of this thread and the 3 neighbours sharing its block
LSK_DEV float block_amax(const float (&v)[8]) {
  float am = 0.0f;
#pragma unroll
  for (int t = 0; t < 8; ++t) am = fmaxf(am, fabsf(v[t]));
  am = fmaxf(am, __shfl_xor(am, 1, 64));
  return fmaxf(am, __shfl_xor(am, 2, 64));
}

// x [M, K] -> q int8 [M, K], ka int32 [M, K/32].  One block per row; a thread quantises 8
// consecutive elements and the 4 threads of a 32-wide block share its maximum (K % 32 == 0, so
// the groups of 4 never straddle the loop's end).
template <bool X_F32>
__global__ __launch_bounds__(256) void blockquant_i8_kernel(const void* __restrict__ x, int64_t ldx, int K,
                                                            int8_t* __restrict__ q, int64_t ldq, int32_t* __restrict__ ka,
                                                            int64_t ldka) {
  const int64_t r = blockIdx.x;
  for (int c = threadIdx.x; c < K / 8; c += 256) {
    float v[8];
    load8<X_F32>(x, r * ldx + 8 * c, v);
    const int e = mx2_block_exp(block_amax(v));
    const float inv = pow2f(-e);
    uint32_t w[2] = {0u, 0u};
#pragma unroll
    for (int t = 0; t < 8; ++t) w[t >> 2] |= ((uint32_t)(int)mx2_q(v[t], inv) & 0xffu) << (8 * (t & 3));
    *(uint2*)(q + r * ldq + 8 * c) = make_uint2(w[0], w[1]);
    if ((c & 3) == 0) ka[r * ldka + c / 4] = e;
  }
}

// Block quant of bf16 rows for the grouped MX GEMMs.  Each row gets the dequantised values
// q * 2^ka as bf16 (exact: |q| <= 127 has 7 significant bits and 2^ka is in range whenever the
// row is not flagged), its exponents ka [rows, K/32] and a flag set when some nonzero block has
// ka outside [lo, hi], the range in which the fused block update on the dequantised values is
// exact for the experts' weight exponents.  A flagged row is rewritten with the integer values q
// (as bf16), which the general kernel pairs with ka, and *any is raised.  One block per row; rows
// from *nrows on (when given) are skipped; q and ka rows are packed (strides K and K/32).
__global__ __launch_bounds__(256) void blockquant_mx2_kernel(const uint16_t* __restrict__ x, int64_t ldx,
                                                             const int32_t* __restrict__ nrows, int K,
                                                             uint16_t* __restrict__ q, int32_t* __restrict__ ka,
                                                             int32_t* __restrict__ flag, int32_t* __restrict__ any,
                                                             int lo, int hi) {
  const int64_t r = blockIdx.x;
  if (nrows && r >= *nrows) return;
  int bad = 0;
  for (int c = threadIdx.x; c < K / 8; c += 256) {
    float v[8];
    load8<false>(x, r * ldx + 8 * c, v);
    const float am = block_amax(v);
    const int e = mx2_block_exp(am);
    const float inv = pow2f(-e), sc = pow2f(e);
    uint32_t w[4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
      w[j] = (uint32_t)f32_to_bf16(f32_mul(mx2_q(v[2 * j], inv), sc)) |
             ((uint32_t)f32_to_bf16(f32_mul(mx2_q(v[2 * j + 1], inv), sc)) << 16);
    store16_split(q + r * K + 8 * c, w[0], w[1], w[2], w[3]);
    if ((c & 3) == 0) ka[r * (K / 32) + c / 4] = e;
    if (am > 0.0f && (e < lo || e > hi)) bad = 1;
  }
  bad = __syncthreads_or(bad);
  if (bad) {
    for (int c = threadIdx.x; c < K / 8; c += 256) {
      float v[8];
      load8<false>(x, r * ldx + 8 * c, v);
      const float inv = pow2f(-mx2_block_exp(block_amax(v)));
      uint32_t w[4];
#pragma unroll
      for (int j = 0; j < 4; ++j)
        w[j] = (uint32_t)f32_to_bf16(mx2_q(v[2 * j], inv)) | ((uint32_t)f32_to_bf16(mx2_q(v[2 * j + 1], inv)) << 16);
      store16_split(q + r * K + 8 * c, w[0], w[1], w[2], w[3]);
    }
  }
  if (threadIdx.x == 0) {
    flag[r] = bad;
    if (bad) atomicOr(any, 1);
  }
}

// ---------------------------------------------------------------- dense MX GEMM (int_mm_mx, int_mm_mx2)
// ROWSCALE: the activation rows carry block exponents ka [M, K/32] (int_mm_mx2); asc == null: the
// epilogue has no row scale (y = bfr(acc)).
template <bool B_FP4, bool SAFE, bool ROWSCALE>
__global__ __launch_bounds__(256) void mx_gemm_kernel(const int8_t* __restrict__ A, int64_t lda, const int32_t* __restrict__ KA,
                                                      int64_t ldka, const uint8_t* __restrict__ B,
                                                      int64_t ldb, const uint8_t* __restrict__ S, int64_t lds, int M, int N,
                                                      int K, int epi, const float* __restrict__ asc,
                                                      const float* __restrict__ bias, float* __restrict__ out,
                                                      int64_t ldo) {
  extern __shared__ char mx_smem[];
  const int ntiles = (N + 127) / 128;
  const int L = lsk::xcd_logical_id(blockIdx.x, gridDim.x);
  const int m0 = (L / ntiles) * 128, n0 = (L % ntiles) * 128;
  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
  const int wm = wave / 2, wn = wave % 2;
  typename Cfg::Acc acc;
#pragma unroll
  for (int i = 0; i < Cfg::TM; ++i)
#pragma unroll
    for (int j = 0; j < Cfg::TN; ++j) acc[i][j] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
  auto rowA = [&](int r) -> const void* { return m0 + r < M ? (const void*)(A + (int64_t)(m0 + r) * lda) : nullptr; };
  auto rowB = [&](int r) -> const uint8_t* { return n0 + r < N ? B + (int64_t)(n0 + r) * ldb : nullptr; };
  auto rowS = [&](int r) -> const uint8_t* { return n0 + r < N ? S + (int64_t)(n0 + r) * lds : nullptr; };
  auto rowK = [&](int r) -> const int32_t* { return m0 + r < M ? KA + (int64_t)(m0 + r) * ldka : nullptr; };
  lsk::mx_mainloop<128, 128, 2, 2, NB, true, B_FP4, SAFE, ROWSCALE>(acc, rowA, rowB, rowS, rowK, K, mx_smem);

  float* region = (float*)mx_smem + wave * Cfg::kStripFloats;
#pragma unroll
  for (int i = 0; i < Cfg::TM; ++i) {
    lsk::stage_strip_f<Cfg::TN, Cfg::kLdc>(acc[i], region);
    __syncthreads();
    for (int q = lane; q < 16 * 16; q += 64) {
      const int row = q >> 4, c4 = (q & 15) * 4;
      const int m = m0 + wm * 64 + i * 16 + row;
      const int n = n0 + wn * 64 + c4;
      if (m < M) {
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          if (n + t >= N) break;
          float v = region[row * Cfg::kLdc + c4 + t];
          if (epi) {
            v = bfr(asc ? f32_mul(v, asc[m]) : v);
            if (bias) v = bfr(f32_add(v, bias[n + t]));
          }
          out[(int64_t)m * ldo + n + t] = v;
        }
      }
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------- grouped MX GEMM (MoE)
// MODE 0: gate/up + activation (tile columns interleave 16 gate / 16 up weight rows); MODE 1:
// down + routing weight into the token-major slot rows.

// Weight row of tile row r (tile column block nt), or -1.
template <int MODE>
LSK_DEV int moe_mx_wrow(const lsk::MoeGemmArgs& a, int nt, int r) {
  if (MODE == 0) {
    const int blk = r >> 4;
    const int hc = nt * 64 + (blk >> 1) * 16 + (r & 15);
    return hc < a.N ? ((blk & 1) ? a.N + hc : hc) : -1;
  }
  const int n = nt * 128 + r;
  return n < a.N ? n : -1;
}

// The tile's epilogue from the binary32 block accumulators (128 x 128, four waves of 64 x 64):
// MODE 0 the gate / up values and the activation into h (with its row maxima); MODE 1 the
// routing-weighted down values into the token-major slot rows.  The operands of every row and
// column a lane stores (row scales, routing weights and slots, biases) are loaded together before
// the first store: loads after a store to memory the compiler cannot prove distinct would each
// wait a round trip.
template <int MODE>
LSK_DEV void moe_mx_epilogue(const lsk::MoeGemmArgs& a, const Cfg::Acc& acc, int nt, int p0, int p1, const float* bias,
                             char* smem) {
  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
  const int wm = wave / 2, wn = wave % 2;
  float* region = (float*)smem + wave * Cfg::kStripFloats;
  constexpr int NPASS = MODE == 0 ? 2 : 4;  // passes of 64 lanes over a 16-row strip
  constexpr int QPR = MODE == 0 ? 8 : 16;   // lanes per row
  const int c4 = MODE == 0 ? ((lane & 7) & 3) * 4 : (lane & 15) * 4;
  const int pair = MODE == 0 ? (lane & 7) >> 2 : 0;
  const int col0 = MODE == 0 ? nt * 64 + wn * 32 + pair * 16 + c4 : nt * 128 + wn * 64 + c4;
  const bool whole = col0 + 4 <= a.N;
  float b0[4], b1[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    b0[t] = 0.0f;
    b1[t] = 0.0f;
    if (bias && col0 + t < a.N) {
      b0[t] = bias[col0 + t];
      if (MODE == 0) b1[t] = bias[a.N + col0 + t];
    }
  }
  float r_asc[Cfg::TM][NPASS], r_w[Cfg::TM][NPASS];
  int r_dst[Cfg::TM][NPASS];
#pragma unroll
  for (int i = 0; i < Cfg::TM; ++i)
#pragma unroll
    for (int pass = 0; pass < NPASS; ++pass) {
      const int p = p0 + wm * 64 + i * 16 + (pass * 64 + lane) / QPR;
      r_asc[i][pass] = 0.0f;
      r_w[i][pass] = 1.0f;
      r_dst[i][pass] = p;
      if (p < p1) {
        if (MODE == 0) {
          r_asc[i][pass] = a.a_scale ? a.a_scale[a.row_tok[p]] : 1.0f;  // none for block-scaled rows
        } else {
          r_asc[i][pass] = a.a_scale ? a.a_scale[p] : 1.0f;
          if (a.row_w) r_w[i][pass] = a.row_w[p];  // none: a plain grouped linear
          if (a.row_dst) r_dst[i][pass] = a.row_dst[p];
        }
      }
    }
#pragma unroll
  for (int i = 0; i < Cfg::TM; ++i) {
    lsk::stage_strip_f<Cfg::TN, Cfg::kLdc>(acc[i], region);
    __syncthreads();
    if (MODE == 0) {
#pragma unroll
      for (int pass = 0; pass < NPASS; ++pass) {
        const int row = (pass * 64 + lane) / QPR;
        const int p = p0 + wm * 64 + i * 16 + row;
        const float asc = r_asc[i][pass];
        float am = 0.0f;
        if (p < p1) {
          float hv[4];
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            hv[t] = 0.0f;
            if (whole || col0 + t < a.N) {
              float yg = bfr(f32_mul(region[row * Cfg::kLdc + pair * 32 + c4 + t], asc));
              float yu = bfr(f32_mul(region[row * Cfg::kLdc + pair * 32 + 16 + c4 + t], asc));
              if (bias) {
                yg = bfr(f32_add(yg, b0[t]));
                yu = bfr(f32_add(yu, b1[t]));
              }
              hv[t] = lsk::act_eval(a.act, yg, yu, a.frac, a.act_tab);
              am = fmaxf(am, fabsf(hv[t]));
            }
          }
          uint16_t* dst = a.h + (int64_t)p * a.N + col0;
          if (whole) {
            *(uint2*)dst = make_uint2(pack_bf16x2(hv[0], hv[1]), pack_bf16x2(hv[2], hv[3]));
          } else {
            for (int t = 0; t < 4; ++t)
              if (col0 + t < a.N) dst[t] = f32_to_bf16(hv[t]);
          }
        }
        am = fmaxf(am, __shfl_xor(am, 1, 64));
        am = fmaxf(am, __shfl_xor(am, 2, 64));
        am = fmaxf(am, __shfl_xor(am, 4, 64));
        if ((lane & 7) == 0 && p < p1) atomicMax(&a.h_amax[p], __float_as_uint(am));
      }
    } else {
#pragma unroll
      for (int pass = 0; pass < NPASS; ++pass) {
        const int row = (pass * 64 + lane) / QPR;
        const int p = p0 + wm * 64 + i * 16 + row;
        if (p < p1 && col0 < a.N) {
          const float asc = r_asc[i][pass], wt = r_w[i][pass];
          float o[4];
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            o[t] = 0.0f;
            if (whole || col0 + t < a.N) {
              float yv = bfr(f32_mul(region[row * Cfg::kLdc + c4 + t], asc));
              if (bias) yv = bfr(f32_add(yv, b0[t]));
              o[t] = f32_mul(wt, yv);
            }
          }
          uint16_t* dst = a.y + (int64_t)r_dst[i][pass] * a.N + col0;
          if (whole) {
            *(uint2*)dst = make_uint2(pack_bf16x2(o[0], o[1]), pack_bf16x2(o[2], o[3]));
          } else {
            for (int t = 0; t < 4; ++t)
              if (col0 + t < a.N) dst[t] = f32_to_bf16(o[t]);
          }
        }
      }
    }
    __syncthreads();
  }
}

// Block-scaled activations: a tile goes to the fused-update kernel (mx2 == 1) when none of its
// rows is flagged, to the general one (mx2 == 2) otherwise; with mx2 == 3 (after the skinny GEMM,
// which runs only when no row is flagged) every tile goes to the general kernel when some row is.  Every thread of the block calls it;
// when no row at all is flagged (the usual case) it decides without a barrier.
template <int MODE>
LSK_DEV bool mx2_takes_tile(const lsk::MoeGemmArgs& a, int p0, int p1) {
  if (a.mx2 == 3) return *a.any_flag != 0;  // every tile, when some row is flagged
  if (*a.any_flag == 0) return a.mx2 == 1;
  int f = 0;
  const int t = threadIdx.x;
  if (t < lsk::kMoeBM && p0 + t < p1) f = a.row_flag[MODE == 0 ? a.row_tok[p0 + t] : p0 + t];
  const int any = __syncthreads_or(f);
  return a.mx2 == 1 ? any == 0 : any != 0;
}

// Register-staged main loop (mx_tile.h), kept as a selectable variant; with ROWSCALE the general
// kernel of block-scaled activations (flagged rows: integer values and their exponents ka;
// other rows: the dequantised values with exponent 0).
template <int MODE, bool SAFE, bool ROWSCALE>
__global__ __launch_bounds__(256) void moe_mx_gemm_kernel(lsk::MoeGemmArgs a) {
  extern __shared__ char mx_smem[];
  const int ntiles = MODE == 0 ? (a.N + 63) / 64 : (a.N + 127) / 128;
  const int L = lsk::xcd_logical_id(blockIdx.x, gridDim.x);
  const int mt = L / ntiles, nt = L - (L / ntiles) * ntiles;
  if (mt >= a.tiles[0]) return;
  const int e = a.tiles[1 + 2 * mt];
  const int p0 = a.tiles[2 + 2 * mt];
  const int p1 = min(a.offs[e + 1], p0 + lsk::kMoeBM);
  if (a.mx2 && !mx2_takes_tile<MODE>(a, p0, p1)) return;
  const uint8_t* wb = (const uint8_t*)a.w_ptrs[e];
  const uint8_t* sb = (const uint8_t*)a.ws_ptrs[e];
  const float* bias = a.b_ptrs ? (const float*)a.b_ptrs[e] : nullptr;
  const uint16_t* A = (const uint16_t*)a.A;
  auto rowA = [&](int r) -> const void* {
    const int p = p0 + r;
    if (p >= p1) return nullptr;
    const int src = MODE == 0 ? a.row_tok[p] : p;
    return (const void*)(A + (int64_t)src * a.lda);
  };
  auto rowB = [&](int r) -> const uint8_t* {
    const int w = moe_mx_wrow<MODE>(a, nt, r);
    return w >= 0 ? wb + (int64_t)w * a.ldw : nullptr;
  };
  auto rowS = [&](int r) -> const uint8_t* {
    const int w = moe_mx_wrow<MODE>(a, nt, r);
    return w >= 0 ? sb + (int64_t)w * a.lds : nullptr;
  };
  auto rowK = [&](int r) -> const int32_t* {
    const int p = p0 + r;
    if (p >= p1) return nullptr;
    const int src = MODE == 0 ? a.row_tok[p] : p;
    return a.row_flag[src] ? a.a_ka + (int64_t)src * a.ldka : nullptr;
  };
  typename Cfg::Acc acc;
#pragma unroll
  for (int i = 0; i < Cfg::TM; ++i)
#pragma unroll
    for (int j = 0; j < Cfg::TN; ++j) acc[i][j] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
  lsk::mx_mainloop<128, 128, 2, 2, NB, false, true, SAFE, ROWSCALE>(acc, rowA, rowB, rowS, rowK, a.K, mx_smem);
  moe_mx_epilogue<MODE>(a, acc, nt, p0, p1, bias, mx_smem);
}

// Direct-to-LDS main loop (mx_pp.h): the default.
template <int MODE, bool SAFE, int RING>
__global__ __launch_bounds__(256, RING == 2 ? 3 : 2) void moe_mx_pp_kernel(lsk::MoeGemmArgs a) {
  extern __shared__ char mx_smem[];
  const int ntiles = MODE == 0 ? (a.N + 63) / 64 : (a.N + 127) / 128;
  const int L = lsk::xcd_logical_id(blockIdx.x, gridDim.x);
  const int mt = L / ntiles, nt = L - (L / ntiles) * ntiles;
  if (mt >= a.tiles[0]) return;
  const int e = a.tiles[1 + 2 * mt];
  const int p0 = a.tiles[2 + 2 * mt];
  const int p1 = min(a.offs[e + 1], p0 + lsk::kMoeBM);
  if (a.mx2 && !mx2_takes_tile<MODE>(a, p0, p1)) return;
  const float* bias = a.b_ptrs ? (const float*)a.b_ptrs[e] : nullptr;
  const int nrows_w = MODE == 0 ? 2 * a.N : a.N;  // weight rows of one expert
  const __amdgpu_buffer_rsrc_t ra = lsk::make_rsrc(a.A, a.a_bytes);
  // the expert's code and exponent resources in scalar registers (a tile's expert is one value)
  const __amdgpu_buffer_rsrc_t rb = lsk::make_rsrc((const void*)wave_uniform64(a.w_ptrs[e]), a.w_bytes);
  const __amdgpu_buffer_rsrc_t rs =
      lsk::make_rsrc((const void*)wave_uniform64(a.ws_ptrs[e]), (int64_t)nrows_w * a.lds);
  const lsk::MxPPRows rows = lsk::mx_pp_rows(
      [&](int r) -> uint32_t {
        const int p = p0 + r;
        if (p >= p1) return lsk::kOob;
        const int src = MODE == 0 ? a.row_tok[p] : p;
        return (uint32_t)((int64_t)src * a.lda * 2);
      },
      [&](int r) -> uint32_t {
        const int w = moe_mx_wrow<MODE>(a, nt, r);
        return w >= 0 ? (uint32_t)((int64_t)w * a.ldw) : lsk::kOob;
      },
      [&](int r) -> uint32_t {
        const int w = moe_mx_wrow<MODE>(a, nt, r);
        return w >= 0 ? (uint32_t)((int64_t)w * a.lds) : lsk::kOob;
      });
  typename lsk::MxPPCfg<RING>::Acc acc;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
  lsk::mx_pp_mainloop<SAFE, RING>(acc, ra, rb, rs, rows, a.K, mx_smem);
  moe_mx_epilogue<MODE>(a, acc, nt, p0, p1, bias, mx_smem);
}

// ---------------------------------------------------------------- dequant and packing
__global__ __launch_bounds__(256) void dequant_mxfp4_kernel(const uint8_t* __restrict__ packed,
                                                            const uint8_t* __restrict__ scale, int64_t rows, int64_t K,
                                                            int block, void* __restrict__ out, int odt) {
  const int64_t half = K / 2;
  const int64_t total = rows * half;
  const int64_t nsb = K / block;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
    const int64_t r = i / half, c = i - r * half;
    const uint32_t byte = packed[i];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int64_t k = 2 * c + t;
      const uint32_t code = t ? (byte >> 4) : (byte & 15u);
      const int e = (int)scale[r * nsb + k / block] - 127;
      const float sc = e > 127 ? __builtin_inff() : pow2f(e);
      // fp4 value = m2 / 2 (exact), times 2^e: one binary32 multiply, as the reference's vals * sc
      const float v = f32_mul(f32_mul(__uint_as_float(lsk::m2_bf16(code) << 16), 0.5f), sc);
      if (odt == LSK_BF16) ((uint16_t*)out)[r * K + k] = f32_to_bf16(v);
      else ((float*)out)[r * K + k] = v;
    }
  }
}

__global__ __launch_bounds__(256) void mx_pack_kernel(const int8_t* __restrict__ m2, int64_t n, uint8_t* __restrict__ packed,
                                                      int32_t* __restrict__ bad) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n / 2; i += (int64_t)gridDim.x * 256) {
    uint32_t codes[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int v = m2[2 * i + t];
      const int a = v < 0 ? -v : v;
      int mag = -1;
      switch (a) {
        case 0: mag = 0; break;
        case 1: mag = 1; break;
        case 2: mag = 2; break;
        case 3: mag = 3; break;
        case 4: mag = 4; break;
        case 6: mag = 5; break;
        case 8: mag = 6; break;
        case 12: mag = 7; break;
        default: break;
      }
      if (mag < 0) {
        atomicOr(bad, 1);
        mag = 0;
      }
      codes[t] = (uint32_t)mag | (v < 0 ? 8u : 0u);
    }
    packed[i] = (uint8_t)(codes[0] | (codes[1] << 4));
  }
}

unsigned grid_for(int64_t n) {
  int64_t b = (n + 255) / 256;
  return (unsigned)(b > 8192 ? 8192 : (b < 1 ? 1 : b));
}

thread_local int g_mx_variant = 0;  // grouped MX main loop: 0 direct-to-LDS, two-stage ring, three blocks per CU (mx_pp.h);
                       // 1 register-staged (mx_tile.h); 2 direct-to-LDS, three-stage ring, two blocks per CU;
                       // 3 as 0, with the skinny grouped GEMM wherever the layer can take it

template <int MODE, bool SAFE>
int launch_grouped(const lsk::MoeGemmArgs& ga, int64_t max_tiles, hipStream_t s) {
  const int ntiles = MODE == 0 ? (ga.N + 63) / 64 : (ga.N + 127) / 128;
  const int64_t blocks = max_tiles * ntiles;
  if (blocks == 0) return LSK_OK;
  LSK_REQUIRE(blocks <= 0x7fffffff, "moe_mx_gemm_kernel: grid too large");
  if (ga.mx2 >= 2) {
    static std::atomic<bool> attr_rs{false};
    auto kern = moe_mx_gemm_kernel<MODE, true, true>;
    if (!attr_rs) {
      if (int rc = reserve_lds(kern, Cfg::kSmemBytes, "moe_mx_gemm_kernel")) return rc;
      attr_rs = true;
    }
    hipLaunchKernelGGL(kern, dim3((unsigned)blocks), dim3(256), Cfg::kSmemBytes, s, ga);
    return lsk::check_launch(MODE == 0 ? "moe_mx_gemm_kernel<gate_up, block exponents>"
                                       : "moe_mx_gemm_kernel<down, block exponents>");
  }
  if (g_mx_variant == 1) {
    static std::atomic<bool> attr{false};
    auto kern = moe_mx_gemm_kernel<MODE, SAFE, false>;
    if (!attr) {
      if (int rc = reserve_lds(kern, Cfg::kSmemBytes, "moe_mx_gemm_kernel")) return rc;
      attr = true;
    }
    hipLaunchKernelGGL(kern, dim3((unsigned)blocks), dim3(256), Cfg::kSmemBytes, s, ga);
    return lsk::check_launch(MODE == 0 ? "moe_mx_gemm_kernel<gate_up>" : "moe_mx_gemm_kernel<down>");
  }
  static_assert(lsk::MxPPCfg<2>::kRingBytes >= Cfg::kEpiBytes, "the epilogue strips fit in the ring");
  if (g_mx_variant == 0 || g_mx_variant == 3) {
    static std::atomic<bool> attr_pp2{false};
    auto kern = moe_mx_pp_kernel<MODE, SAFE, 2>;
    if (!attr_pp2) {
      if (int rc = reserve_lds(kern, lsk::MxPPCfg<2>::kRingBytes, "moe_mx_pp_kernel")) return rc;
      attr_pp2 = true;
    }
    hipLaunchKernelGGL(kern, dim3((unsigned)blocks), dim3(256), lsk::MxPPCfg<2>::kRingBytes, s, ga);
    return lsk::check_launch(MODE == 0 ? "moe_mx_pp_kernel<gate_up>" : "moe_mx_pp_kernel<down>");
  }
  static std::atomic<bool> attr_pp{false};
  auto kern = moe_mx_pp_kernel<MODE, SAFE, 3>;
  if (!attr_pp) {
    if (int rc = reserve_lds(kern, lsk::MxPPCfg<3>::kRingBytes, "moe_mx_pp_kernel")) return rc;
    attr_pp = true;
  }
  hipLaunchKernelGGL(kern, dim3((unsigned)blocks), dim3(256), lsk::MxPPCfg<3>::kRingBytes, s, ga);
  return lsk::check_launch(MODE == 0 ? "moe_mx_pp_kernel<gate_up>" : "moe_mx_pp_kernel<down>");
}

template <bool B_FP4, bool SAFE, bool ROWSCALE>
int launch_dense(const int8_t* a, int64_t lda, const int32_t* ka, int64_t ldka, const uint8_t* b, int64_t ldb,
                 const uint8_t* kexp, int64_t lds, int M, int N, int K, int epi, const float* asc, const float* bias,
                 float* out, int64_t ldo, hipStream_t s) {
  static std::atomic<bool> attr{false};
  auto kern = mx_gemm_kernel<B_FP4, SAFE, ROWSCALE>;
  if (!attr) {
    if (int rc = reserve_lds(kern, Cfg::kSmemBytes, "mx_gemm_kernel")) return rc;
    attr = true;
  }
  const int64_t blocks = (int64_t)((M + 127) / 128) * ((N + 127) / 128);
  LSK_REQUIRE(blocks <= 0x7fffffff, "mx_gemm_kernel: grid too large");
  hipLaunchKernelGGL(kern, dim3((unsigned)blocks), dim3(256), Cfg::kSmemBytes, s, a, lda, ka, ldka, b, ldb, kexp, lds, M, N,
                     K, epi, asc, bias, out, ldo);
  return lsk::check_launch("mx_gemm_kernel");
}

// ---------------------------------------------------------------- decode-sized grouped MX GEMV
// Decode-sized MX expert GEMV.  Lane l owns MX block b = l + 64 j (j < NCH) of every weight row
// the wave streams: its 16 code bytes and its exponent byte, loaded coalesced.  gfx950's
// v_cvt_scalef32_pk_bf16_fp4 with scale 2 turns two codes into the bf16 doubled mantissas m2
// (exact; checked over every code byte on MI355X), and v_dot2_f32_bf16 against the activation
// (int8 values held as bf16) sums a block: every product and partial sum is an integer below
// 2^16, so the block sum s_b is exact.  The block sums go to LDS, and one lane per (row, column)
// then runs the contract's ordered update acc = fl32(acc + s_b * 2^(k_b - 128)) over the
// blocks in ascending order from +0 (one FMA, exact product; SAFE: multiply, then add).  MODE
// 0: gate row c and up row N + c, bias-added bfr values into gu for the activation-and-requant
// kernel; MODE 1: bfr(w * y) into the token's slot row.
// MX2 (block-scaled activations, integer-valued rows with block exponents ka): the update is
// acc = fl32(acc + fl32(s_b * fl32(2^ka_b * 2^(k_b - 128)))) with no row scale, and MODE 0 writes
// the activation h = act(gate, up) straight into h (the owner lane holds both values).
// MODE 2 (one token, at most four experts): the down projection and the combine in one launch --
// wave s of a block computes slot s's MODE 1 values bfr(w * y) for the block's RPW columns into
// LDS, and wave 0 adds the slots in order from +0 (the token's rows are its experts in ascending
// order, the combine's order), then bfr(shared) when given, and writes the token's row of y (gu).
typedef __bf16 v2bf_t __attribute__((ext_vector_type(2)));

template <int MODE, int MR, int NCH, int RPW, bool SAFE, bool MX2>
__global__ __launch_bounds__(256) void moe_mx_gemv_kernel(lsk::MoeGemmArgs a, uint16_t* __restrict__ gu,
                                                          const float* __restrict__ shared) {
  constexpr int kRows = MODE == 0 ? 2 : 1;
  constexpr int V = MR * RPW * kRows;  // chains per row chunk, q = (m * RPW + i) * kRows + r
  static_assert(V <= 64, "one lane per chain");
  constexpr int kB = 64 * NCH;          // blocks a wave covers
  constexpr int kSbStride = kB + 4;     // floats per chain row in LDS (16-byte aligned, skewed banks)
  constexpr int kWaveBytes = V * kSbStride * 4 + RPW * kRows * kB * 4 + (MX2 ? MR * kB * 4 : 0);
  extern __shared__ __attribute__((aligned(16))) char gemv_smem[];
  const int cols_blk = MODE == 2 ? RPW : 4 * RPW;
  const int nchunk = (a.N + cols_blk - 1) / cols_blk;
  const int lane = threadIdx.x & 63, wave = wave_id();
  const int mt = MODE == 2 ? wave : (int)(blockIdx.x / nchunk);
  const int ch = MODE == 2 ? (int)blockIdx.x : (int)(blockIdx.x - mt * nchunk);
  const bool tile_ok = mt < a.tiles[0];
  if (MODE != 2 && !tile_ok) return;  // (MODE 2: every wave reaches the combine's barrier)
  const int e = tile_ok ? a.tiles[1 + 2 * mt] : 0;
  const int p0 = tile_ok ? a.tiles[2 + 2 * mt] : 0;
  const int p1 = tile_ok ? min(a.offs[e + 1], p0 + lsk::kMoeBM) : 0;
  const int nb = a.K / 32;
  const int c0 = MODE == 2 ? ch * RPW : ch * cols_blk + wave * RPW;
  const int nw = MODE == 0 ? 2 * a.N : a.N;  // weight rows of the expert
  float* sb = (float*)(gemv_smem + wave * kWaveBytes);
  float* scl = sb + V * kSbStride;  // 2^(k - 128) per (weight row, block)
  float* sa = scl + RPW * kRows * kB;  // MX2: 2^ka per (activation row of the chunk, block)
  const __amdgpu_buffer_rsrc_t rw = lsk::make_rsrc((const void*)a.w_ptrs[e], (int64_t)nw * a.ldw);
  const __amdgpu_buffer_rsrc_t rsc = lsk::make_rsrc((const void*)a.ws_ptrs[e], (int64_t)nw * a.lds);
  const __amdgpu_buffer_rsrc_t ra = lsk::make_rsrc(a.A, a.a_bytes);

  // the wave's weight rows: the lane's code bytes and exponent bytes per (column, row, block)
  v4i codes[RPW][kRows][NCH];
  uint32_t kxs[RPW][kRows][NCH];
#pragma unroll
  for (int i = 0; i < RPW; ++i)
#pragma unroll
    for (int r = 0; r < kRows; ++r) {
      const int c = c0 + i;
      const int wr = MODE == 0 && r ? a.N + c : c;
#pragma unroll
      for (int j = 0; j < NCH; ++j) {
        const int b = lane + 64 * j;
        const bool in = tile_ok && c < a.N && b < nb;
        codes[i][r][j] = lsk::buf_load16(rw, in ? (uint32_t)(wr * a.ldw + b * 16) : lsk::kOob);
        kxs[i][r][j] = __builtin_amdgcn_raw_buffer_load_b8(rsc, in ? (int)(wr * a.lds + b) : (int)lsk::kOob, 0, 0);
      }
    }
  // the chain this lane runs (lanes >= V idle in that phase)
  const int q = lane;
  const int q_m = q / (RPW * kRows), q_i = (q / kRows) % RPW, q_r = q % kRows;
  const int c = c0 + q_i;
  const bool chain = q < V;
  const bool owner = chain && q_r == 0 && c < a.N;
  const float* bias = a.b_ptrs ? (const float*)a.b_ptrs[e] : nullptr;
  float b0 = 0.0f, b1 = 0.0f;
  if (owner && bias) {
    b0 = bias[c];
    if (MODE == 0) b1 = bias[a.N + c];
  }
  const uint16_t* A = (const uint16_t*)a.A;
  for (int rb = p0; rb < p1; rb += MR) {
    // the lane's blocks of the chunk's activation rows: 32 bf16 values each (16 pairs)
    v4i act[MR][NCH][4];
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      const int p = rb + m;
      const int src = p < p1 ? (MODE == 0 ? a.row_tok[p] : p) : -1;
#pragma unroll
      for (int j = 0; j < NCH; ++j) {
        const int b = lane + 64 * j;
        const bool in = src >= 0 && b < nb;
        const uint32_t off = in ? (uint32_t)((src * a.lda + b * 32) * 2) : lsk::kOob;
#pragma unroll
        for (int h = 0; h < 4; ++h) act[m][j][h] = lsk::buf_load16(ra, in ? off + 16 * h : lsk::kOob);
        // (this wave alone writes and reads its LDS area, in program order)
        if constexpr (MX2) sa[m * kB + b] = in ? pow2f(a.a_ka[(int64_t)src * a.ldka + b]) : 0.0f;
      }
    }
    (void)A;
    const int p = rb + q_m;
    const bool rowok = owner && p < p1;
    float asc = 0.0f, wt = 0.0f;
    int dst = 0;
    if (rowok) {
      asc = a.a_scale ? a.a_scale[MODE == 0 ? a.row_tok[p] : p] : 1.0f;
      if (MODE >= 1) {
        wt = a.row_w ? a.row_w[p] : 1.0f;
        dst = a.row_dst ? a.row_dst[p] : p;
      }
    }
    if (rb == p0) {
      // block scales into LDS, after the first chunk's loads are issued (its wait covers them)
#pragma unroll
      for (int i = 0; i < RPW; ++i)
#pragma unroll
        for (int r = 0; r < kRows; ++r)
#pragma unroll
          for (int j = 0; j < NCH; ++j)
            scl[(i * kRows + r) * kB + lane + 64 * j] = pow2f((int)(kxs[i][r][j] & 0xffu) - 128);
    }
    // exact block sums into LDS: decode the codes of (i, r, j), dot with every row of the chunk
#pragma unroll
    for (int i = 0; i < RPW; ++i)
#pragma unroll
      for (int r = 0; r < kRows; ++r)
#pragma unroll
        for (int j = 0; j < NCH; ++j) {
          uint32_t m2[16];  // pair d = elements 2d, 2d + 1 of the block
          // decoded per row chunk (kept out of registers between chunks: 16 words per row block)
          v4i cw = codes[i][r][j];
          asm volatile("" : "+v"(cw));
#pragma unroll
          for (int w = 0; w < 4; ++w) {
            const uint32_t x = (uint32_t)cw[w];
            m2[4 * w + 0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(x, 2.0f, 0));
            m2[4 * w + 1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(x, 2.0f, 1));
            m2[4 * w + 2] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(x, 2.0f, 2));
            m2[4 * w + 3] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(x, 2.0f, 3));
          }
#pragma unroll
          for (int m = 0; m < MR; ++m) {
            float t = 0.0f;
#pragma unroll
            for (int d = 0; d < 16; ++d) {
              // through a plain int: a bit cast of a vector element lvalue read the vector's first
              // element here
              const int av = act[m][j][d >> 2][d & 3];
              t = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(v2bf_t, av), __builtin_bit_cast(v2bf_t, m2[d]), t,
                                                  false);
            }
            sb[((m * RPW + i) * kRows + r) * kSbStride + lane + 64 * j] = t;
          }
        }
    // the ordered update, one chain per lane (LDS written and read by this wave only: in order)
    float acc = 0.0f;
    if (chain) {
      const float* srow = sb + q * kSbStride;
      const float* crow = scl + (q_i * kRows + q_r) * kB;
      auto upd = [&](float sv, float sc) {
        acc = SAFE ? f32_add(acc, f32_mul(sv, sc)) : __builtin_fmaf(sv, sc, acc);
      };
      int b = 0;
      if constexpr (MX2) {
        const float* arow = sa + q_m * kB;
        auto upd2 = [&](float sv, float av, float sc) { acc = f32_add(acc, f32_mul(sv, f32_mul(av, sc))); };
#pragma unroll 2
        for (; b + 4 <= nb; b += 4) {
          const v4f s4 = *(const v4f*)(srow + b);
          const v4f a4 = *(const v4f*)(arow + b);
          const v4f c4 = *(const v4f*)(crow + b);
          upd2(s4[0], a4[0], c4[0]);
          upd2(s4[1], a4[1], c4[1]);
          upd2(s4[2], a4[2], c4[2]);
          upd2(s4[3], a4[3], c4[3]);
        }
        for (; b < nb; ++b) upd2(srow[b], arow[b], crow[b]);
      } else {
#pragma unroll 2
        for (; b + 4 <= nb; b += 4) {
          const v4f s4 = *(const v4f*)(srow + b);
          const v4f c4 = *(const v4f*)(crow + b);
          upd(s4[0], c4[0]);
          upd(s4[1], c4[1]);
          upd(s4[2], c4[2]);
          upd(s4[3], c4[3]);
        }
        for (; b < nb; ++b) upd(srow[b], crow[b]);
      }
    }
    const float accu = MODE == 0 ? __shfl_down(acc, 1, 64) : 0.0f;  // the up chain sits in lane q + 1
    if (rowok) {
      if (MODE == 0) {
        float yg = bfr(f32_mul(acc, asc));
        float yu = bfr(f32_mul(accu, asc));
        if (bias) {
          yg = bfr(f32_add(yg, b0));
          yu = bfr(f32_add(yu, b1));
        }
        if constexpr (MX2) {
          a.h[(int64_t)p * a.N + c] = f32_to_bf16(lsk::act_eval(a.act, yg, yu, a.frac, a.act_tab));
        } else {
          uint16_t* row = gu + (int64_t)p * 2 * a.N;
          row[c] = f32_to_bf16(yg);
          row[a.N + c] = f32_to_bf16(yu);
        }
      } else {
        float yv = bfr(f32_mul(acc, asc));
        if (bias) yv = bfr(f32_add(yv, b0));
        if (MODE == 1) a.y[(int64_t)dst * a.N + c] = f32_to_bf16(f32_mul(wt, yv));
        else ((float*)(gemv_smem + 4 * kWaveBytes))[mt * RPW + q_i] = bfr(f32_mul(wt, yv));
      }
    }
  }
  if constexpr (MODE == 2) {
    __syncthreads();
    const float* comb = (const float*)(gemv_smem + 4 * kWaveBytes);  // [slot][RPW]
    const int cc = c0 + lane;
    if (wave == 0 && lane < RPW && cc < a.N) {
      const int n = a.tiles[0];
      float acc = 0.0f;
      for (int s2 = 0; s2 < n; ++s2) acc = f32_add(acc, comb[s2 * RPW + lane]);
      if (shared) acc = f32_add(acc, bfr(shared[cc]));
      gu[cc] = f32_to_bf16(acc);
    }
  }
}

template <int MODE, int MR, int NCH, bool SAFE, bool MX2>
int launch_mx_gemv_k(const lsk::MoeGemmArgs& ga, int64_t max_tiles, uint16_t* gu, hipStream_t s, const char* name,
                     const float* shared = nullptr) {
  constexpr int RPW = MODE == 0 ? 2 : 4;
  constexpr int kRows = MODE == 0 ? 2 : 1;
  constexpr int V = MR * RPW * kRows;
  constexpr int smem = 4 * (V * (64 * NCH + 4) * 4 + RPW * kRows * 64 * NCH * 4 + (MX2 ? MR * 64 * NCH * 4 : 0)) +
                       (MODE == 2 ? 4 * RPW * 4 : 0);
  static std::atomic<bool> attr{false};
  auto kern = moe_mx_gemv_kernel<MODE, MR, NCH, RPW, SAFE, MX2>;
  if (!attr) {
    if (int rc = reserve_lds(kern, smem, name)) return rc;
    attr = true;
  }
  const int nchunk = MODE == 2 ? (ga.N + RPW - 1) / RPW : (ga.N + 4 * RPW - 1) / (4 * RPW);
  const int64_t blocks = MODE == 2 ? nchunk : max_tiles * nchunk;
  if (blocks == 0) return LSK_OK;
  LSK_REQUIRE(blocks <= 0x7fffffff, "%s: grid too large", name);
  hipLaunchKernelGGL(kern, dim3((unsigned)blocks), dim3(256), smem, s, ga, gu, shared);
  return lsk::check_launch(name);
}

// MR: activation rows per pass (their bf16 blocks live in registers: 16 words per row and block
// sweep), fewer when K needs more sweeps.
template <int MODE, int MR, bool SAFE, bool MX2>
int launch_mx_gemv_mr(const lsk::MoeGemmArgs& ga, int64_t max_tiles, uint16_t* gu, hipStream_t s, const char* name) {
  const int nch = (ga.K / 32 + 63) / 64;
  if (nch <= 1) return launch_mx_gemv_k<MODE, MR, 1, SAFE, MX2>(ga, max_tiles, gu, s, name);
  if (nch <= 2) return launch_mx_gemv_k<MODE, (MR > 2 ? 2 : MR), 2, SAFE, MX2>(ga, max_tiles, gu, s, name);
  return launch_mx_gemv_k<MODE, 1, 4, SAFE, MX2>(ga, max_tiles, gu, s, name);
}

template <int MODE, bool SAFE, bool MX2 = false>
int launch_mx_gemv(const lsk::MoeGemmArgs& ga, int64_t max_tiles, int64_t T, uint16_t* gu, hipStream_t s,
                   const char* name) {
  if (T <= 1) return launch_mx_gemv_mr<MODE, 1, SAFE, MX2>(ga, max_tiles, gu, s, name);
  if (T <= 2) return launch_mx_gemv_mr<MODE, 2, SAFE, MX2>(ga, max_tiles, gu, s, name);
  return launch_mx_gemv_mr<MODE, 4, SAFE, MX2>(ga, max_tiles, gu, s, name);
}

// ---------------------------------------------------------------- skinny grouped MX GEMM
// MXFP4 experts holding few routed rows each (layers of tens of tokens): the layout of moe.hip's
// skinny int8 kernel on the bf16 MFMA.  A block takes one expert tile's rows 16 at a time, copied
// into LDS as their bf16 values, and 16 groups of 16 weight rows, one per wave, each over the whole
// K (the ordered block updates cannot be split over K).  For block b, lane (col, g) of a wave holds
// the 4 code bytes of k = 32 b + 8 g .. + 7 of weight row 16 w + col, converted to the doubled
// mantissas as moe_mx_pp's main loop does, and the same k of activation row col; the MFMA's sum
// s_b of (row 4 g + i, col) is applied in block order as acc = fl32(acc + s_b 2^(e - 128)) (one
// FMA; with SAFE the product and the sum apart), e the weight row's E8M0 byte of block b, staged
// in LDS per wave with one contiguous copy of the group's rows.  The codes come from the experts'
// skinny-layout copies (lsk_mx_skinny_pack: per group of 16 rows and step of 4 blocks, lane
// (col, g)'s 4 code bytes of the 4 blocks side by side, so a wave reads each step as one
// contiguous 1 KB; the codes' own layout, 16 bytes per row and block, measured 2.6x slower for the
// whole layer) and stream D steps ahead of their MFMAs in registers, so each expert's codes are read
// once per chunk.  The epilogue is
// moe_mx_gemv_kernel's: the bias-added gate / up values into gu (mode 0), the routing-weighted slot
// rows (mode 1).  WPB waves per block (one group each); chunks of cr <= 16 rows, the most any
// expert holds when that is fewer (one token: one row, so the LDS holds one row and more blocks fit
// a CU; MFMA rows past the chunk read its last row and their outputs are dropped).  LDS: the
// chunk's rows [cr][ldsk], the waves' E8M0 bytes [WPB][scb], the rows' operands.
// ROUTE = EPL > 0 (MODE 0, one token, one-row chunks): the token is routed from its logits in the
// launch itself -- every wave runs the router's selection (route_select), the block takes the
// mt-th of the k experts ascending, quantises the token's row of x into its LDS row (rowquant's
// arithmetic, the values as bf16), and block 0's first wave writes the routing outputs and the
// one-token dispatch the later launches read (as moe_route_gemv1_kernel does for int8 experts).
template <int MODE, bool SAFE, int D, int WPB, int ROUTE = 0>
__global__ __launch_bounds__(WPB * 64) void moe_mx_skinny_kernel(lsk::MoeGemmArgs a, uint16_t* __restrict__ gu,
                                                                 int sets, int ldsk, int scb, int cr,
                                                                 lsk::MxRouteArgs rt) {
  extern __shared__ __attribute__((aligned(16))) char smem_mxs[];
  const int lane = threadIdx.x & 63, wave = wave_id(), tid = threadIdx.x;
  const int mt = blockIdx.x / sets, gs = blockIdx.x - (blockIdx.x / sets) * sets;
  int e, p0, p1;
  int e_r = 0, s_r = 0, S = 1, pos = 0;
  int ek[8];
  uint4 xr[4];  // ROUTE: this thread's 8-element chunks of the token's row of x
  if constexpr (ROUTE > 0) {
    if (mt >= rt.k) return;  // the whole block leaves
    // x first (its wait then leaves the code loads issued below in flight), then the routing
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int c = tid + WPB * 64 * j;
      xr[j] = c < (a.K >> 3) ? *(const uint4*)(rt.x + 8 * c) : make_uint4(0, 0, 0, 0);
    }
    lsk::route_select<ROUTE>(rt.g, rt.gdt, rt.ldg, 0, rt.E, rt.k, rt.renorm, rt.rtab, e_r, s_r, S);
#pragma unroll
    for (int j = 0; j < 8; ++j) ek[j] = __shfl(e_r, j < rt.k ? j : 0, 64);
#pragma unroll
    for (int j = 0; j < 8; ++j) pos += (j < rt.k && ek[j] < e_r) ? 1 : 0;
    const uint64_t sel = __builtin_amdgcn_ballot_w64(lane < rt.k && pos == mt);
    e = __shfl(e_r, (int)__builtin_ctzll(sel), 64);
    p0 = mt;
    p1 = mt + 1;
  } else {
    if (mt >= a.tiles[0]) return;  // the whole block leaves
    if (a.mx2 == 1 && *a.any_flag != 0) return;  // block-scaled rows with a flagged row: not here
    e = a.tiles[1 + 2 * mt];
    p0 = a.tiles[2 + 2 * mt];
    p1 = min(a.offs[e + 1], p0 + lsk::kMoeBM);
  }
  const int K = a.K, nb = K >> 5;
  const int NWR = MODE == 0 ? 2 * a.N : a.N;  // weight rows
  const int G = (NWR + 15) >> 4;
  const int g = gs * WPB + wave;  // this wave's group of 16 weight rows (wave-uniform)
  const int col = lane & 15, kg = lane >> 4;
  const int n = g * 16 + col;
  const bool live = g < G && n < NWR;
  const float* bp = a.b_ptrs ? (const float*)a.b_ptrs[e] : nullptr;
  const __amdgpu_buffer_rsrc_t rcb = lsk::make_rsrc(bp, bp ? 4 * (int64_t)NWR : 0);
  const float c_b =
      __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rcb, (live && bp) ? (uint32_t)(4 * n) : lsk::kOob, 0, 0));
  const __amdgpu_buffer_rsrc_t rw = lsk::make_rsrc((const void*)wave_uniform64(a.w_ptrs[e]), a.w_bytes);
  const __amdgpu_buffer_rsrc_t rsc =
      lsk::make_rsrc((const void*)wave_uniform64(a.ws_ptrs[e]), (int64_t)NWR * a.lds);
  const __amdgpu_buffer_rsrc_t ra = lsk::make_rsrc(a.A, a.a_bytes);
  const int nst = (nb + 3) >> 2;  // steps of 4 blocks
  // this lane's 16 code bytes of step s (blocks 4 s .. 4 s + 3, 4 bytes each) at wbase + 1024 s
  const uint32_t wbase = g < G ? (uint32_t)(((g * nst) * 16 + col) * 64 + kg * 16) : lsk::kOob;
  char* sc_w = smem_mxs + cr * ldsk + wave * scb;
  int* r_src = (int*)(smem_mxs + cr * ldsk + WPB * scb);
  float* r_asc = (float*)(r_src + 16);
  float* r_w = r_asc + 16;
  int* r_dst = (int*)(r_w + 16);
  float* r_red = (float*)(r_dst + 16);  // ROUTE: the waves' maxima of |x|
  // the group's E8M0 rows 16 g .. 16 g + 15: one contiguous run of 16 lds bytes (zeros past NWR)
  {
    const int sbytes = 16 * (int)a.lds;
    const uint32_t sbase = (uint32_t)(g * 16) * (uint32_t)a.lds;
    for (int j = 0; j * 1024 < sbytes; ++j) {
      const int o = j * 1024 + lane * 16;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rsc, (lsk::lds_void_t)(sc_w + j * 1024), 16,
                                               (g < G && o < sbytes) ? sbase + (uint32_t)o : lsk::kOob, 0, 0, 0);
    }
  }
  const int cpr = (2 * K + 1023) >> 10;  // 1 KB chunks of an activation row
  const char* arow = smem_mxs + min(col, cr - 1) * ldsk + 16 * kg;  // A fragment of block b at + 64 b
  const uint8_t* srow = (const uint8_t*)sc_w + col * (int)a.lds;  // E8M0 byte of block b at [b]
  lsk::compiler_fence();
  for (int q0 = p0; q0 < p1; q0 += cr) {
    const int nr = min(cr, p1 - q0);
    if (q0 > p0) __syncthreads();  // the previous chunk's LDS reads are done
    v4i cw[D];
#pragma unroll
    for (int u = 0; u < D; ++u)
      cw[u] = lsk::buf_load16(rw, (u < nst && wbase != lsk::kOob) ? wbase + 1024u * u : lsk::kOob);
    float rsc_x = 0.0f;  // ROUTE: the token's row scale
    if constexpr (ROUTE > 0) {
      // the token's row of x quantised into LDS row 0: q = clamp(rint(x / asc)) as bf16 values
      constexpr int NTH = WPB * 64;
      const int K8 = K >> 3;
      float am = 0.0f;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t wd[4] = {xr[j].x, xr[j].y, xr[j].z, xr[j].w};
#pragma unroll
        for (int q = 0; q < 4; ++q)
          am = fmaxf(am, fmaxf(fabsf(bf16_to_f32((uint16_t)(wd[q] & 0xffff))),
                               fabsf(bf16_to_f32((uint16_t)(wd[q] >> 16)))));
      }
      am = wave_fmax(am);
      if (lane == 0) r_red[wave] = am;
      __syncthreads();
      am = r_red[0];
#pragma unroll
      for (int w2 = 1; w2 < WPB; ++w2) am = fmaxf(am, r_red[w2]);
      const float sc = f32_div(fmaxf(am, kAmaxFloor), 127.0f), rs = f32_div(1.0f, sc);
      rsc_x = sc;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int c = tid + NTH * j;
        if (c < K8) {
          const uint32_t wd[4] = {xr[j].x, xr[j].y, xr[j].z, xr[j].w};
          uint32_t ob[4];
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const float q0v = fminf(fmaxf(rint_div8(bf16_to_f32((uint16_t)(wd[q] & 0xffff)), sc, rs), -127.0f), 127.0f);
            const float q1v = fminf(fmaxf(rint_div8(bf16_to_f32((uint16_t)(wd[q] >> 16)), sc, rs), -127.0f), 127.0f);
            ob[q] = (__float_as_uint(q0v) >> 16) | (__float_as_uint(q1v) & 0xffff0000u);  // exact bf16
          }
          *(uint2*)(smem_mxs + 16 * c) = make_uint2(ob[0], ob[1]);
          *(uint2*)(smem_mxs + 16 * c + 8) = make_uint2(ob[2], ob[3]);
        }
      }
      // block 0's first wave: the routing outputs and the one-token dispatch
      if (blockIdx.x == 0 && wave == 0) {
        if (lane < rt.k) {
          const uint16_t wb = f32_to_bf16(f32_div((float)s_r, (float)S));
          rt.idx_out[lane] = e_r;
          rt.w_out[lane] = wb;
          rt.tiles[1 + 2 * pos] = e_r;
          rt.tiles[2 + 2 * pos] = pos;
          rt.row_tok[pos] = 0;
          rt.row_dst[pos] = pos;
          rt.row_w[pos] = bf16_to_f32(wb);
        }
        for (int ee = lane; ee <= rt.E; ee += 64) {
          int before = 0;
#pragma unroll
          for (int j = 0; j < 8; ++j) before += (j < rt.k && ek[j] < ee) ? 1 : 0;
          rt.offs[ee] = before;
        }
        if (lane == 0) {
          rt.tiles[0] = rt.k;
          rt.tok_cnt[0] = rt.k;
          rt.ascx[0] = sc;
        }
      }
    } else if (MODE == 0) {
      // the token rows of the chunk: loaded behind the first code steps, waited for alone
      const int src = tid < nr ? a.row_tok[q0 + tid] : 0;
      lsk::compiler_fence();
      if (tid < nr) r_src[tid] = src;
      __syncthreads();
    }
    // the chunk's rows into LDS (bf16 values, zeros past K), then the rows' operands
    for (int c = wave; c < (ROUTE > 0 ? 0 : nr * cpr); c += WPB) {
      const int r = c / cpr, j = c - (c / cpr) * cpr;
      const int kb = j * 1024 + lane * 16;
      const int src = MODE == 0 ? r_src[r] : q0 + r;
      const uint32_t off = kb < 2 * K ? (uint32_t)(src * 2 * a.lda + kb) : lsk::kOob;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (lsk::lds_void_t)(smem_mxs + r * ldsk + j * 1024), 16, off, 0, 0,
                                               0);
    }
    float o_asc = 1.0f, o_w = 1.0f;
    int o_dst = 0;
    if (tid < nr) {
      const int p = q0 + tid;
      if (ROUTE > 0) o_asc = rsc_x;
      else if (a.a_scale) o_asc = a.a_scale[MODE == 0 ? r_src[tid] : p];
      if (MODE == 1) {
        o_w = a.row_w ? a.row_w[p] : 1.0f;
        o_dst = a.row_dst ? a.row_dst[p] : p;
      }
    }
    lsk::compiler_fence();
    lsk::wait_vm<0>();  // rows, E8M0 bytes, the rows' operands and the first code steps
    if (tid < nr) {
      r_asc[tid] = o_asc;
      r_w[tid] = o_w;
      r_dst[tid] = o_dst;
    }
    __syncthreads();
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    // block b's exact sums: the MFMA of the rows' fragments with the weight row's doubled mantissas
    auto bsum = [&](int b, uint32_t q) -> v4f {
      const v4i af = *(const v4i*)(arow + 64 * b);
      const v4i bf = v4i{(int)__builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(q, 2.0f, 0)),
                         (int)__builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(q, 2.0f, 1)),
                         (int)__builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(q, 2.0f, 2)),
                         (int)__builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(q, 2.0f, 3))};
      return lsk::mfma_bf16(af, bf);
    };
    // the ordered update with the weight row's 2^(e - 128): v_ldexp_f32 of 1 is exact for every E8M0
    // byte (2^-128 and 2^-127 as binary32 subnormals, denormals kept)
    auto upd = [&](const v4f& d, int b) {
      const float sc = __builtin_amdgcn_ldexpf(1.0f, (int)srow[b] - 128);
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[i] = SAFE ? f32_add(acc[i], f32_mul(d[i], sc)) : __builtin_fmaf(d[i], sc, acc[i]);
    };
    // a whole step: its four MFMAs issued before the first of its updates, which stay in block order
    auto step4 = [&](int st, const v4i& q4) {
      const int b0 = 4 * st;
      const v4f d0 = bsum(b0, (uint32_t)q4[0]);
      const v4f d1 = bsum(b0 + 1, (uint32_t)q4[1]);
      const v4f d2 = bsum(b0 + 2, (uint32_t)q4[2]);
      const v4f d3 = bsum(b0 + 3, (uint32_t)q4[3]);
      upd(d0, b0);
      upd(d1, b0 + 1);
      upd(d2, b0 + 2);
      upd(d3, b0 + 3);
    };
    if (g < G) {
      const int nfs = nb >> 2;          // whole steps (the last step may hold fewer blocks)
      const int nfull = nfs / D * D;    // rounds of D whole steps
      for (int s0 = 0; s0 < nfull; s0 += D) {
#pragma unroll
        for (int u = 0; u < D; ++u) {
          step4(s0 + u, cw[u]);
          const int nx = s0 + u + D;
          cw[u] = lsk::buf_load16(rw, (nx < nst && wbase != lsk::kOob) ? wbase + 1024u * nx : lsk::kOob);
        }
      }
      // the rest: up to D - 1 whole steps and the partial one, already loaded
#pragma unroll
      for (int u = 0; u < D; ++u) {
        const int st = nfull + u;
        if (st < nfs) {
          step4(st, cw[u]);
        } else if (st < nst) {
#pragma unroll
          for (int j = 0; j < 4; ++j)
            if (4 * st + j < nb) upd(bsum(4 * st + j, (uint32_t)cw[u][j]), 4 * st + j);
        }
      }
    }
    lsk::wait_vm<0>();  // no code load outlives the chunk (the next one reuses the registers)
    if (live) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int m = 4 * kg + i;
        if (m < nr) {
          float yv = bfr(f32_mul(acc[i], r_asc[m]));
          if (bp) yv = bfr(f32_add(yv, c_b));
          if (MODE == 0) gu[(int64_t)(q0 + m) * NWR + n] = f32_to_bf16(yv);
          else a.y[(int64_t)r_dst[m] * a.N + n] = f32_to_bf16(f32_mul(r_w[m], yv));
        }
      }
    }
  }
}

template <int MODE, bool SAFE>
int launch_mx_skinny(const lsk::MoeGemmArgs& ga, int64_t max_tiles, int64_t rows, uint16_t* gu, hipStream_t s,
                     const char* name) {
  const int NWR = MODE == 0 ? 2 * ga.N : ga.N;
  const int G = (NWR + 15) / 16;
  // chunks of up to 16 rows, fewer when no expert holds more; with few rows four waves per block
  // (more blocks over the CUs, the LDS a few rows deep)
  const int cr = (int)(rows < 1 ? 1 : (rows > 16 ? 16 : rows));
  const bool small = cr <= 8;
  const int wpb = small ? 4 : 16;
  const int sets = (G + wpb - 1) / wpb;
  const int ldsk = (2 * ga.K + 1023) / 1024 * 1024 + 16;
  const int scb = (16 * (int)ga.lds + 1023) / 1024 * 1024;
  const int smem = cr * ldsk + wpb * scb + 5 * 16 * 4;
  LSK_REQUIRE(smem <= 160 * 1024, "%s: %d bytes of LDS", name, smem);
  const int64_t blocks = max_tiles * sets;
  if (blocks == 0) return LSK_OK;
  LSK_REQUIRE(blocks <= 0x7fffffff, "%s: grid too large", name);
  constexpr int D = SAFE ? 4 : 8;  // steps of 4 blocks in flight
  if (small) {
    auto kern = moe_mx_skinny_kernel<MODE, SAFE, D, 4>;
    static std::atomic<bool> attr{false};
    if (!attr) {
      if (int rc = reserve_lds(kern, 160 * 1024, name)) return rc;
      attr = true;
    }
    hipLaunchKernelGGL(kern, dim3((unsigned)blocks), dim3(256), smem, s, ga, gu, sets, ldsk, scb, cr, lsk::MxRouteArgs{});
  } else {
    auto kern = moe_mx_skinny_kernel<MODE, SAFE, D, 16>;
    static std::atomic<bool> attr{false};
    if (!attr) {
      if (int rc = reserve_lds(kern, 160 * 1024, name)) return rc;
      attr = true;
    }
    hipLaunchKernelGGL(kern, dim3((unsigned)blocks), dim3(1024), smem, s, ga, gu, sets, ldsk, scb, cr, lsk::MxRouteArgs{});
  }
  return lsk::check_launch(name);
}

// One token routed inside the gate/up launch (ROUTE = EPL): four-wave blocks, one-row chunks, k
// experts x the column groups' sets.
template <bool SAFE, int EPL>
int launch_mx_route_skinny1(const lsk::MoeGemmArgs& ga, const lsk::MxRouteArgs& ra, uint16_t* gu, hipStream_t s,
                            const char* name) {
  const int G = (2 * ga.N + 15) / 16;
  const int sets = (G + 3) / 4;
  const int ldsk = (2 * ga.K + 1023) / 1024 * 1024 + 16;
  const int scb = (16 * (int)ga.lds + 1023) / 1024 * 1024;
  const int smem = ldsk + 4 * scb + 5 * 16 * 4;
  LSK_REQUIRE(smem <= 160 * 1024, "%s: %d bytes of LDS", name, smem);
  const int64_t blocks = (int64_t)ra.k * sets;
  if (blocks == 0) return LSK_OK;
  auto kern = moe_mx_skinny_kernel<0, SAFE, SAFE ? 4 : 8, 4, EPL>;
  static std::atomic<bool> attr{false};
  if (!attr) {
    if (int rc = reserve_lds(kern, 160 * 1024, name)) return rc;
    attr = true;
  }
  hipLaunchKernelGGL(kern, dim3((unsigned)blocks), dim3(256), smem, s, ga, gu, sets, ldsk, scb, 1, ra);
  return lsk::check_launch(name);
}

}  // namespace

namespace lsk {

int launch_moe_mx_route_skinny1(const MoeGemmArgs& ga, const MxRouteArgs& ra, int safe, uint16_t* gu, hipStream_t s) {
  LSK_REQUIRE(ga.K % 32 == 0 && ga.K <= 8192 && gu && ra.x && ((uintptr_t)ra.x & 15) == 0 && ra.k >= 1 &&
                  ra.k <= 8 && ra.E >= ra.k && ra.E <= 256,
              "moe_mx_route_skinny1: arguments");
  const char* name = "moe_mx_skinny_kernel<gate_up, routed>";
  const int epl = ra.E <= 64 ? 1 : (ra.E <= 128 ? 2 : 4);
  if (safe) {
    if (epl == 1) return launch_mx_route_skinny1<true, 1>(ga, ra, gu, s, name);
    if (epl == 2) return launch_mx_route_skinny1<true, 2>(ga, ra, gu, s, name);
    return launch_mx_route_skinny1<true, 4>(ga, ra, gu, s, name);
  }
  if (epl == 1) return launch_mx_route_skinny1<false, 1>(ga, ra, gu, s, name);
  if (epl == 2) return launch_mx_route_skinny1<false, 2>(ga, ra, gu, s, name);
  return launch_mx_route_skinny1<false, 4>(ga, ra, gu, s, name);
}

int launch_moe_mx_gemm(int mode, const MoeGemmArgs& ga, int64_t max_tiles, int safe, hipStream_t s) {
  if (mode == 0) return safe ? launch_grouped<0, true>(ga, max_tiles, s) : launch_grouped<0, false>(ga, max_tiles, s);
  return safe ? launch_grouped<1, true>(ga, max_tiles, s) : launch_grouped<1, false>(ga, max_tiles, s);
}

// Bytes of a skinny-layout copy of rows x K packed E2M1 codes (see lsk_mx_skinny_pack).
int64_t mx_skinny_bytes(int64_t rows, int64_t K) { return (rows + 15) / 16 * ((K / 32 + 3) / 4) * 1024; }

// LDS bytes the skinny grouped MX GEMM needs for K and an E8M0 row stride lds (<= 160 KB to run).
int moe_mx_skinny_lds(int64_t K, int64_t lds) {
  return (int)((2 * K + 1023) / 1024 * 1024 + 16) * 16 + (int)((16 * lds + 1023) / 1024 * 1024) * 16 + 320;
}

int launch_moe_mx_skinny(int mode, const MoeGemmArgs& ga, int64_t max_tiles, int64_t rows, int safe, uint16_t* gu,
                         hipStream_t s) {
  LSK_REQUIRE((!ga.a_ka || ga.mx2 == 1) && ga.K % 32 == 0 && (mode == 1 || gu), "moe_mx_skinny: arguments");
  if (mode == 0)
    return safe ? launch_mx_skinny<0, true>(ga, max_tiles, rows, gu, s, "moe_mx_skinny_kernel<gate_up>")
                : launch_mx_skinny<0, false>(ga, max_tiles, rows, gu, s, "moe_mx_skinny_kernel<gate_up>");
  return safe ? launch_mx_skinny<1, true>(ga, max_tiles, rows, nullptr, s, "moe_mx_skinny_kernel<down>")
              : launch_mx_skinny<1, false>(ga, max_tiles, rows, nullptr, s, "moe_mx_skinny_kernel<down>");
}

int launch_moe_mx_down_combine1(const MoeGemmArgs& ga, int safe, const float* shared, uint16_t* y, hipStream_t s) {
  LSK_REQUIRE(!ga.a_ka && ga.K % 32 == 0 && y, "moe_mx_down_combine1: arguments");
  const int nch = (ga.K / 32 + 63) / 64;
  const char* name = "moe_mx_gemv_kernel<down + combine>";
#define LSK_DC1(NCHV) \
  return safe ? launch_mx_gemv_k<2, 1, NCHV, true, false>(ga, 1, y, s, name, shared) \
              : launch_mx_gemv_k<2, 1, NCHV, false, false>(ga, 1, y, s, name, shared)
  if (nch <= 1) LSK_DC1(1);
  if (nch <= 2) LSK_DC1(2);
  LSK_DC1(4);
#undef LSK_DC1
}

int launch_moe_mx_gemv(int mode, const MoeGemmArgs& ga, int64_t max_tiles, int64_t T, int safe, uint16_t* gu,
                       hipStream_t s) {
  if (ga.a_ka) {  // block-scaled activations: one update form, whatever safe says
    LSK_REQUIRE(!ga.a_scale && ga.ldka >= ga.K / 32 && (mode == 1 || ga.h), "moe_mx_gemv: MX2 arguments");
    return mode == 0 ? launch_mx_gemv<0, false, true>(ga, max_tiles, T, gu, s, "moe_mx_gemv_kernel<gate_up, mx2>")
                     : launch_mx_gemv<1, false, true>(ga, max_tiles, T, gu, s, "moe_mx_gemv_kernel<down, mx2>");
  }
  if (mode == 0)
    return safe ? launch_mx_gemv<0, true>(ga, max_tiles, T, gu, s, "moe_mx_gemv_kernel<gate_up>")
                : launch_mx_gemv<0, false>(ga, max_tiles, T, gu, s, "moe_mx_gemv_kernel<gate_up>");
  return safe ? launch_mx_gemv<1, true>(ga, max_tiles, T, gu, s, "moe_mx_gemv_kernel<down>")
              : launch_mx_gemv<1, false>(ga, max_tiles, T, gu, s, "moe_mx_gemv_kernel<down>");
}

int launch_rowquant_bf16(const uint16_t* x, int64_t T, int64_t H, uint16_t* q, float* asc, hipStream_t s) {
  if (T == 0) return LSK_OK;
  LSK_REQUIRE(T <= 0x7fffffff, "rowquant_bf16: too many rows");
  hipLaunchKernelGGL(rowquant_bf16_kernel, dim3((unsigned)T), dim3(256), 0, s, x, H, q, asc);
  return check_launch("rowquant_bf16_kernel");
}

int launch_blockquant_mx2(const uint16_t* x, int64_t ldx, int64_t R, const int32_t* nrows, int K, uint16_t* q,
                          int32_t* ka, int32_t* flag, int32_t* any, int lo, int hi, hipStream_t s) {
  if (R == 0) return LSK_OK;
  LSK_REQUIRE(R <= 0x7fffffff, "blockquant_mx2: too many rows");
  hipLaunchKernelGGL(blockquant_mx2_kernel, dim3((unsigned)R), dim3(256), 0, s, x, ldx, nrows, K, q, ka, flag, any, lo,
                     hi);
  return check_launch("blockquant_mx2_kernel");
}

int launch_requant_bf16(const uint16_t* h, const uint32_t* amax, const int32_t* nrows, int64_t R, int I, uint16_t* q,
                        float* asc, hipStream_t s) {
  hipLaunchKernelGGL(requant_bf16_kernel, dim3(grid_for(R * (I / 8))), dim3(256), 0, s, h, amax, nrows, I, q, asc);
  return check_launch("requant_bf16_kernel");
}

}  // namespace lsk

extern "C" int lsk_gemm_mx(const int8_t* a, int64_t lda, const void* b, int b_fmt, int64_t ldb, const uint8_t* kexp,
                           int64_t lds, int64_t M, int64_t N, int64_t K, int epilogue, const float* asc, const float* bias,
                           float* out, int64_t ldo, void* stream) {
  LSK_REQUIRE(M >= 0 && N >= 0 && K >= 0, "lsk_gemm_mx: negative size");
  LSK_REQUIRE(K % 32 == 0, "lsk_gemm_mx: K=%lld not a multiple of the 32-element block", (long long)K);
  LSK_REQUIRE(b_fmt == 0 || b_fmt == 1, "lsk_gemm_mx: b_fmt %d not 0 (m2 int8) or 1 (packed E2M1)", b_fmt);
  LSK_REQUIRE(epilogue == 0 || epilogue == 1, "lsk_gemm_mx: epilogue must be 0 or 1");
  if (M == 0 || N == 0) return LSK_OK;
  LSK_REQUIRE(a && b && kexp && out && (epilogue == 0 || asc), "lsk_gemm_mx: null pointer");
  LSK_REQUIRE(M <= 0x7fffffff && N <= 0x7fffffff && K <= 0x7fffffff, "lsk_gemm_mx: size too large");
  const int64_t rowbytes = b_fmt == 1 ? K / 2 : K;
  LSK_REQUIRE(lda >= K && lda % 16 == 0 && ((uintptr_t)a & 15) == 0, "lsk_gemm_mx: a rows must be 16-byte aligned");
  LSK_REQUIRE(ldb >= rowbytes && ldb % 16 == 0 && ((uintptr_t)b & 15) == 0, "lsk_gemm_mx: weight rows must be 16-byte aligned");
  LSK_REQUIRE(lds >= K / 32 && ldo >= N, "lsk_gemm_mx: leading dimension too small");
  // the fused block update is exact unless an exponent byte >= 240 can overflow the product;
  // the host cannot see device data, so the general entry point always takes the SAFE update
  hipStream_t s = (hipStream_t)stream;
  if (b_fmt == 1)
    return launch_dense<true, true, false>(a, lda, nullptr, 0, (const uint8_t*)b, ldb, kexp, lds, (int)M, (int)N, (int)K,
                                           epilogue, asc, bias, out, ldo, s);
  return launch_dense<false, true, false>(a, lda, nullptr, 0, (const uint8_t*)b, ldb, kexp, lds, (int)M, (int)N, (int)K,
                                          epilogue, asc, bias, out, ldo, s);
}

extern "C" int lsk_blockquant(const void* x, int x_dtype, int64_t ldx, int64_t M, int64_t K, int8_t* q, int64_t ldq,
                              int32_t* ka, int64_t ldka, void* stream) {
  LSK_REQUIRE(M >= 0 && K >= 0, "lsk_blockquant: negative size");
  LSK_REQUIRE(K % 32 == 0, "lsk_blockquant: K=%lld not a multiple of the 32-element block", (long long)K);
  LSK_REQUIRE(x_dtype == LSK_BF16 || x_dtype == LSK_F32, "lsk_blockquant: x must be bf16 or f32");
  if (M == 0 || K == 0) return LSK_OK;
  LSK_REQUIRE(x && q && ka, "lsk_blockquant: null pointer");
  LSK_REQUIRE(M <= 0x7fffffff && K <= 0x7fffffff, "lsk_blockquant: size too large");
  const int esz = x_dtype == LSK_F32 ? 4 : 2;
  LSK_REQUIRE(ldx >= K && (ldx * esz) % 16 == 0 && ((uintptr_t)x & 15) == 0,
              "lsk_blockquant: x rows must be 16-byte aligned");
  LSK_REQUIRE(ldq >= K && ldq % 8 == 0 && ((uintptr_t)q & 7) == 0, "lsk_blockquant: q rows must be 8-byte aligned");
  LSK_REQUIRE(ldka >= K / 32, "lsk_blockquant: ldka too small");
  hipStream_t s = (hipStream_t)stream;
  if (x_dtype == LSK_F32)
    hipLaunchKernelGGL(blockquant_i8_kernel<true>, dim3((unsigned)M), dim3(256), 0, s, x, ldx, (int)K, q, ldq, ka, ldka);
  else
    hipLaunchKernelGGL(blockquant_i8_kernel<false>, dim3((unsigned)M), dim3(256), 0, s, x, ldx, (int)K, q, ldq, ka, ldka);
  return lsk::check_launch("blockquant_i8_kernel");
}

extern "C" int lsk_gemm_mx2(const int8_t* q, int64_t ldq, const int32_t* ka, int64_t ldka, const void* b, int b_fmt,
                            int64_t ldb, const uint8_t* kexp, int64_t lds, int64_t M, int64_t N, int64_t K, int epilogue,
                            const float* bias, float* out, int64_t ldo, void* stream) {
  LSK_REQUIRE(M >= 0 && N >= 0 && K >= 0, "lsk_gemm_mx2: negative size");
  LSK_REQUIRE(K % 32 == 0, "lsk_gemm_mx2: K=%lld not a multiple of the 32-element block", (long long)K);
  LSK_REQUIRE(b_fmt == 0 || b_fmt == 1, "lsk_gemm_mx2: b_fmt %d not 0 (m2 int8) or 1 (packed E2M1)", b_fmt);
  LSK_REQUIRE(epilogue == 0 || epilogue == 1, "lsk_gemm_mx2: epilogue must be 0 or 1");
  if (M == 0 || N == 0) return LSK_OK;
  LSK_REQUIRE(q && ka && b && kexp && out, "lsk_gemm_mx2: null pointer");
  LSK_REQUIRE(M <= 0x7fffffff && N <= 0x7fffffff && K <= 0x7fffffff, "lsk_gemm_mx2: size too large");
  const int64_t rowbytes = b_fmt == 1 ? K / 2 : K;
  LSK_REQUIRE(ldq >= K && ldq % 16 == 0 && ((uintptr_t)q & 15) == 0, "lsk_gemm_mx2: q rows must be 16-byte aligned");
  LSK_REQUIRE(ldb >= rowbytes && ldb % 16 == 0 && ((uintptr_t)b & 15) == 0,
              "lsk_gemm_mx2: weight rows must be 16-byte aligned");
  LSK_REQUIRE(ldka >= K / 32 && lds >= K / 32 && ldo >= N, "lsk_gemm_mx2: leading dimension too small");
  // the exponent of each product depends on the row and the column; the general entry point
  // always takes the multiply-then-add update with the correctly rounded 2^(ka + kexp - 128)
  hipStream_t s = (hipStream_t)stream;
  if (b_fmt == 1)
    return launch_dense<true, true, true>(q, ldq, ka, ldka, (const uint8_t*)b, ldb, kexp, lds, (int)M, (int)N, (int)K,
                                          epilogue, nullptr, bias, out, ldo, s);
  return launch_dense<false, true, true>(q, ldq, ka, ldka, (const uint8_t*)b, ldb, kexp, lds, (int)M, (int)N, (int)K,
                                         epilogue, nullptr, bias, out, ldo, s);
}

extern "C" int lsk_dequant_mxfp4(const uint8_t* packed, const uint8_t* scale, int64_t rows, int64_t K, int block,
                                 void* out, int out_dtype, void* stream) {
  LSK_REQUIRE(rows >= 0 && K >= 0 && block > 0, "lsk_dequant_mxfp4: bad sizes");
  LSK_REQUIRE(K % 2 == 0 && K % block == 0, "lsk_dequant_mxfp4: K=%lld must be even and a multiple of block=%d",
              (long long)K, block);
  LSK_REQUIRE(out_dtype == LSK_BF16 || out_dtype == LSK_F32, "lsk_dequant_mxfp4: out_dtype must be bf16 or f32");
  if (rows == 0 || K == 0) return LSK_OK;
  LSK_REQUIRE(packed && scale && out, "lsk_dequant_mxfp4: null pointer");
  hipLaunchKernelGGL(dequant_mxfp4_kernel, dim3(grid_for(rows * K / 2)), dim3(256), 0, (hipStream_t)stream, packed, scale,
                     rows, K, block, out, out_dtype);
  return lsk::check_launch("dequant_mxfp4_kernel");
}

extern "C" int lsk_mx_pack_m2(const int8_t* m2, int64_t n, uint8_t* packed, int32_t* bad, void* stream) {
  LSK_REQUIRE(n >= 0 && n % 2 == 0, "lsk_mx_pack_m2: n=%lld must be even", (long long)n);
  if (n == 0) return LSK_OK;
  LSK_REQUIRE(m2 && packed && bad, "lsk_mx_pack_m2: null pointer");
  hipLaunchKernelGGL(mx_pack_kernel, dim3(grid_for(n / 2)), dim3(256), 0, (hipStream_t)stream, m2, n, packed, bad);
  return lsk::check_launch("mx_pack_kernel");
}

namespace {
// moe_ref.py:258-261: y = bfr(acc * asc[m]); y = bfr(y + b[n])
__global__ __launch_bounds__(256) void mx_epilogue_kernel(const float* __restrict__ acc, int64_t M, int64_t N,
                                                          const float* __restrict__ asc, const float* __restrict__ bias,
                                                          float* __restrict__ out) {
  const int64_t total = M * N;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
    const int64_t m = i / N, n = i - m * N;
    float y = bfr(f32_mul(acc[i], asc[m]));
    if (bias) y = bfr(f32_add(y, bias[n]));
    out[i] = y;
  }
}
}  // namespace

extern "C" int lsk_mx_epilogue(const float* acc, int64_t M, int64_t N, const float* asc, const float* bias, float* out,
                               void* stream) {
  LSK_REQUIRE(M >= 0 && N >= 0, "lsk_mx_epilogue: negative size");
  if (M == 0 || N == 0) return LSK_OK;
  LSK_REQUIRE(acc && asc && out, "lsk_mx_epilogue: null pointer");
  hipLaunchKernelGGL(mx_epilogue_kernel, dim3(grid_for(M * N)), dim3(256), 0, (hipStream_t)stream, acc, M, N, asc, bias,
                     out);
  return lsk::check_launch("mx_epilogue_kernel");
}

namespace lsk {
int mx_variant() { return g_mx_variant; }
}  // namespace lsk

// ---------------------------------------------------------------- skinny-layout copies of MXFP4 codes
// codes: rows x K/2 packed E2M1 bytes, row stride ldw (ldw % 4 == 0); out [ceil(rows / 16)]
// [ceil(K / 128)][16][4][16] bytes: group of 16 rows, step of 4 blocks of 32, row of the group,
// lane group g, then the 4 code bytes of k = 32 b + 8 g .. + 7 for the step's blocks b; zeros
// past `rows` and past K / 32 blocks.  One thread per output dword (4-byte loads and stores).
__global__ __launch_bounds__(256) void mx_skinny_pack_kernel(const uint8_t* __restrict__ codes, int64_t ldw,
                                                             int64_t rows, int64_t nb, uint32_t* __restrict__ out,
                                                             int64_t nwords) {
  const int64_t nst = (nb + 3) / 4;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < nwords; i += (int64_t)gridDim.x * 256) {
    const int64_t j = i & 3, kg = (i >> 2) & 3, c = (i >> 4) & 15, rest = i >> 8;
    const int64_t st = rest % nst, gi = rest / nst;
    const int64_t r = gi * 16 + c, b = 4 * st + j;
    uint32_t v = 0;
    if (r < rows && b < nb) v = *(const uint32_t*)(codes + r * ldw + 16 * b + 4 * kg);
    out[i] = v;
  }
}

extern "C" int64_t lsk_mx_skinny_bytes(int64_t rows, int64_t K) {
  return (rows > 0 && K > 0 && K % 32 == 0) ? lsk::mx_skinny_bytes(rows, K) : 0;
}

extern "C" int lsk_mx_skinny_pack(const uint8_t* codes, int64_t ldw, int64_t rows, int64_t K, uint8_t* out,
                                  void* stream) {
  LSK_REQUIRE(rows >= 0 && K > 0 && K % 32 == 0, "lsk_mx_skinny_pack: rows=%lld, K=%lld (K %% 32 == 0)",
              (long long)rows, (long long)K);
  if (rows == 0) return LSK_OK;
  LSK_REQUIRE(codes && out, "lsk_mx_skinny_pack: null pointer");
  LSK_REQUIRE(ldw >= K / 2 && ldw % 4 == 0 && ((uintptr_t)codes & 3) == 0 && ((uintptr_t)out & 15) == 0,
              "lsk_mx_skinny_pack: ldw=%lld below K/2 or not a multiple of 4, or misaligned pointers", (long long)ldw);
  const int64_t nwords = lsk::mx_skinny_bytes(rows, K) / 4;
  hipLaunchKernelGGL(mx_skinny_pack_kernel, dim3(grid_for(nwords)), dim3(256), 0, (hipStream_t)stream, codes, ldw,
                     rows, K / 32, (uint32_t*)out, nwords);
  return lsk::check_launch("mx_skinny_pack_kernel");
}

extern "C" int lsk_moe_mx_select(int variant) {
  LSK_REQUIRE(variant >= 0 && variant <= 3, "lsk_moe_mx_select: variant %d not in [0, 3]", variant);
  g_mx_variant = variant;
  return LSK_OK;
}
