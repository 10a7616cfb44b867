// Dense contract GEMM on gfx950: exact int8 x int8 -> int32 on MFMA, fused binary32 epilogue.
//
//   prefill (M > 128): eight-wave ping-pong MFMA tiles (pp_tile.h), v_mfma_i32_32x32x32_i8,
//                     four 64-byte K stages in flight through direct-to-LDS loads, XCD-aware
//                     tile order, epilogue operands staged in LDS.
//   small   (32 < M <= 128): register-staged 128x128 MFMA tiles (mfma_tile.h).
//   decode  (M <= 32): weight-streaming GEMV on the same MFMA (rows padded to 16 in registers),
//                     K split over the block's waves and reduced exactly in LDS.
//   generic:          any stride / alignment / K, one thread per output (correctness path).
//
// Integer accumulation is exact in any order (|acc| <= K * 127^2 < 2^31 for K <= 133144), so
// tiling and K-splits never change a bit; the epilogue is applied once per output element.
#include <algorithm>
#include <atomic>

#include "mfma_tile.h"
#include "pp_tile.h"
#include "w4_tile.h"

// Tile order: consecutive tiles walk LSK_GROUP_M M-tiles down one N column before the next
// column, inside each XCD's contiguous run of tiles.  The 32 tiles one XCD runs at a time then
// cover 4 M-tiles x 8 N-tiles, whose activation and weight panels its L2 shares (measured on the
// Qwen2.5-7B block and Llama-3.1-8B MLP shapes: 1 to 2.5% faster than 16 x 2, 32 x 1 slower).
#ifndef LSK_GROUP_M
#define LSK_GROUP_M 4
#endif

namespace {

using lsk::zero4;

// Dense tile kernel: C[m, n] = sum_k A[m, k] * W[n, k] with the epilogue applied per element.
// A and W are K-contiguous with 16-byte aligned rows and K % 16 == 0.  Logical tile ids walk
// M-fastest inside groups of 16 M-tiles after the XCD remap.
template <int BM, int BN, int WM, int WN>
__global__ __launch_bounds__(WM * WN * 64) void gemm_i8_mfma_kernel(
    const int8_t* __restrict__ A, int lda, const int8_t* __restrict__ W, int ldw, int M, int N, int K,
    EpiParams ep, int vec_ok) {
  using C = lsk::TileCfg<BM, BN, WM, WN>;
  extern __shared__ v4i smem[];
  const int mtiles = (M + BM - 1) / BM, ntiles = (N + BN - 1) / BN;
  const int L = lsk::xcd_logical_id(blockIdx.x, mtiles * ntiles);
  constexpr int GM = LSK_GROUP_M;
  const int group = L / (GM * ntiles);
  const int first_m = group * GM;
  const int gsize = (mtiles - first_m) < GM ? (mtiles - first_m) : GM;
  const int r = L - group * GM * ntiles;
  const int m0 = (first_m + r % gsize) * BM, n0 = (r / gsize) * BN;

  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
  const int wm = wave / WN, wn = wave % WN;
  // resources start at the tile's first row: offsets stay below BM * lda
  const __amdgpu_buffer_rsrc_t ra_res = lsk::make_rsrc(A + (int64_t)m0 * lda, (int64_t)(M - m0) * lda);
  const __amdgpu_buffer_rsrc_t rb_res = lsk::make_rsrc(W + (int64_t)n0 * ldw, (int64_t)(N - n0) * ldw);
  typename C::RowsA pa;
  typename C::RowsB pb;
#pragma unroll
  for (int j = 0; j < C::kAPer; ++j) {
    int row, c;
    lsk::chunk_of<C::kThreads>(tid, j, row, c);
    pa[j] = (m0 + row < M) ? (uint32_t)(row * lda) : lsk::kOob;
  }
#pragma unroll
  for (int j = 0; j < C::kBPer; ++j) {
    int row, c;
    lsk::chunk_of<C::kThreads>(tid, j, row, c);
    pb[j] = (n0 + row < N) ? (uint32_t)(row * ldw) : lsk::kOob;
  }
  typename C::Acc acc;
#pragma unroll
  for (int i = 0; i < C::TM; ++i)
#pragma unroll
    for (int j = 0; j < C::TN; ++j) acc[i][j] = lsk::zero16();

  lsk::mfma_mainloop<BM, BN, WM, WN>(acc, ra_res, pa, rb_res, pb, K, smem);

  int32_t* region = (int32_t*)smem + wave * C::kStripInts;
  constexpr int kQuads = C::WTN / 4;
#pragma unroll
  for (int i = 0; i < C::TM; ++i)
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      lsk::stage_half<C::TN, C::kLdc>(acc[i], h, region);
      __syncthreads();
      for (int q = lane; q < 16 * kQuads; q += 64) {
        const int row = q / kQuads, c4 = q - row * kQuads;
        const v4i v = *(const v4i*)(region + row * C::kLdc + c4 * 4);
        const int m = m0 + wm * C::WTM + i * 32 + h * 16 + row;
        const int n = n0 + wn * C::WTN + c4 * 4;
        if (m < M && n < N) epilogue_store4(ep, m, n, N, v, vec_ok && n + 4 <= N);
      }
      __syncthreads();
    }
}

// Epilogue of the ping-pong kernel, one staged 32-row strip (strip i of the wave's tile, in the
// wave's LDS region): the contract epilogue over four consecutive columns per lane (a lane
// always covers the same four columns), with the tile's operands read from LDS.  ORDER / ODT /
// BIAS specialise the common cases; -1 evaluates them at run time.
template <class C, int ORDER, int ODT, bool BIAS>
__device__ __forceinline__ void pp_strip_store(int i, const int32_t* region, const EpiParams& ep, int m0, int n0,
                                               int M, int N, int vec_ok, const char* smem) {
  const int order = ORDER >= 0 ? ORDER : ep.order;
  const int odt = ODT >= 0 ? ODT : ep.out_dtype;
  const bool has_bias = ORDER >= 0 ? BIAS : ep.bias != nullptr;
  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
  const int wm = wave / C::kWN, wn = wave % C::kWN;
  const float* sc_row = (const float*)(smem + C::kScaleOff);
  const float* sc_ws = sc_row + C::kBM;
  const float* sc_b = sc_ws + C::kBN;
  const int* sc_ec = (const int*)(sc_b + C::kBN);
  constexpr int kQuads = C::WTN / 4;
  static_assert(64 % kQuads == 0, "a lane keeps one column quad");
  const int c4 = lane % kQuads;
  const int nl = wn * C::WTN + c4 * 4;  // tile-local first column of the lane's quad
  const int n = n0 + nl;
  const v4f wsq = *(const v4f*)(sc_ws + nl);
  const v4f bq = *(const v4f*)(sc_b + nl);
  const v4i ecq = *(const v4i*)(sc_ec + nl);
  const float wsv[4] = {wsq[0], wsq[1], wsq[2], wsq[3]}, bv[4] = {bq[0], bq[1], bq[2], bq[3]};
  const int ecv[4] = {ecq[0], ecq[1], ecq[2], ecq[3]};
  const bool pow2 = order == LSK_EPI_POW2;
  const bool vec = vec_ok && n + 4 <= N;
#pragma unroll
  for (int t = 0; t < 32 * kQuads / 64; ++t) {
    const int row = (lane + 64 * t) / kQuads;
    const v4i v = *(const v4i*)(region + row * C::kLdc + c4 * 4);
    const int ml = wm * C::WTM + i * 32 + row;
    const int m = m0 + ml;
    const float rv = sc_row[ml];
    if (ORDER < 0 && order == LSK_EPI_V25) {  // the outlier side term needs (m, n): operands from memory
      if (m < M && n < N) epilogue_store4(ep, m, n, N, v, vec);
      continue;
    }
    if (m < M && n < N)
      epilogue_store4_pre(ep.out, ep.ldo, order, odt, has_bias, ep.shift, m, n, N, v, rv, wsv, bv,
                          pow2 ? __float_as_int(rv) : 0, ecv, vec);
  }
}

// Fast epilogue of a whole tile under the v2.1 order, bf16 output, no bias, taken when no output
// of the tile can be NaN: every ws of the tile finite with |ws| < 2^96 and every asc finite, so
// fl32(acc) * ws is finite (|acc| < 2^31) and its product with a finite asc is finite or
// infinite, never NaN.  Per four columns: the two binary32 products per element, gfx950's bf16
// conversion (round to nearest even, equal to f32_to_bf16 away from NaN), and one 8-byte buffer
// store at a 32-bit offset from the tile's first output (the host checks the tile span fits).
// Stores stay 8 bytes wide: 16-byte buffer stores scheduled a few instructions ahead of VALU
// writes to their data registers were measured on MI355X to store the newer values.
template <class C>
__device__ __forceinline__ void pp_strip_store_fast(int i, const int32_t* region, __amdgpu_buffer_rsrc_t ro,
                                                    int ldo_bytes, const char* smem) {
  const int lane = threadIdx.x & 63, wave = wave_id();
  const int wm = wave / C::kWN, wn = wave % C::kWN;
  const float* sc_row = (const float*)(smem + C::kScaleOff);
  const float* sc_ws = sc_row + C::kBM;
  constexpr int kQuads = C::WTN / 4;
  constexpr int kRowStep = 64 / kQuads;  // rows one pass of the wave covers
  const int c4 = lane % kQuads, r0 = lane / kQuads;
  const int nl = wn * C::WTN + c4 * 4;
  const v4f wsq = *(const v4f*)(sc_ws + nl);
  const int ml0 = wm * C::WTM + i * 32 + r0;
  const uint32_t off = (uint32_t)(ml0 * ldo_bytes + nl * 2);
#pragma unroll
  for (int t = 0; t < 32 / kRowStep; ++t) {
    const v4i v = *(const v4i*)(region + (r0 + kRowStep * t) * C::kLdc + c4 * 4);
    const float rv = sc_row[ml0 + kRowStep * t];
    float y[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) y[k] = f32_mul(f32_mul((float)v[k], wsq[k]), rv);
    const v2u32 u = {pack_bf16x2_nonan(y[0], y[1]), pack_bf16x2_nonan(y[2], y[3])};
    __builtin_amdgcn_raw_buffer_store_b64(u, ro, off, kRowStep * t * ldo_bytes, 0);
  }
}

// Fast epilogue of a whole tile under the POW2 order (ref_block_v1.py:167,193,198,218) with
// binary32 output and no column exponents: y = fl32(acc) * fl32(2^-(shift + erow[m])), one
// factor per row (the row exponent sits in the tile's row-operand slot).  Stored straight from
// the accumulators, no LDS staging: register r of lane l of a 32 x 32 block holds row
// 8 (r / 4) + 4 (l / 32) + r % 4, column l % 32, so each 4-byte store instruction writes 32
// consecutive binary32 values (128 bytes) of two rows.  (On MI355X at the Qwen2.5-7B gate/up
// shape, 8192 x 37888 x 3584, this is 3-4% faster than staging 32-row strips through LDS for
// 8-byte stores.)
template <class C>
__device__ __forceinline__ void pp_epilogue_direct_pow2(const typename C::Acc& acc, __amdgpu_buffer_rsrc_t ro,
                                                        int ldo_bytes, int shift, const float* sc_row) {
  const int lane = threadIdx.x & 63, wave = wave_id();
  const int wm = wave / C::kWN, wn = wave % C::kWN;
  const int colb = (wn * C::WTN + (lane & 31)) * 4;
#pragma unroll
  for (int i = 0; i < C::TM; ++i)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      // rows row0 .. row0 + 3 of this lane (registers 4 g .. 4 g + 3 of each block)
      const int row0 = wm * C::WTM + i * 32 + 8 * g + 4 * (lane >> 5);
      const v4f e4 = *(const v4f*)(sc_row + row0);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float sc = pow2_descale(shift + __float_as_int(e4[q]));
        const uint32_t off = (uint32_t)((row0 + q) * ldo_bytes + colb);
#pragma unroll
        for (int j = 0; j < C::TN; ++j)
          __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(f32_mul((float)acc[i][j][4 * g + q], sc)), ro,
                                                off + j * 128, 0, 0);
      }
    }
}

template <class C, int I>
__device__ __forceinline__ void pp_epilogue_fast(const typename C::Acc& acc, __amdgpu_buffer_rsrc_t ro, int ldo_bytes,
                                                 char* smem) {
  if constexpr (I < C::TM) {
    int32_t* region = (int32_t*)(smem + wave_id() * C::kStripBytes);
    lsk::pp_stage_strip<C::TN, C::kLdc>(acc[I], region);
    pp_strip_store_fast<C>(I, region, ro, ldo_bytes, smem);
    pp_epilogue_fast<C, I + 1>(acc, ro, ldo_bytes, smem);
  }
}

// All strips of the wave's tile, strip index a compile-time constant (the accumulators stay in
// registers): stage strip I in the wave's LDS region, store it, recurse.
template <class C, int ORDER, int ODT, bool BIAS, int I>
__device__ __forceinline__ void pp_epilogue(const typename C::Acc& acc, const EpiParams& ep, int m0, int n0, int M,
                                            int N, int vec_ok, char* smem) {
  if constexpr (I < C::TM) {
    int32_t* region = (int32_t*)(smem + wave_id() * C::kStripBytes);
    lsk::pp_stage_strip<C::TN, C::kLdc>(acc[I], region);
    pp_strip_store<C, ORDER, ODT, BIAS>(I, region, ep, m0, n0, M, N, vec_ok, smem);
    pp_epilogue<C, ORDER, ODT, BIAS, I + 1>(acc, ep, m0, n0, M, N, vec_ok, smem);
  }
}

// One dense tile (eight-wave ping-pong or four-wave main loop, MAIN); same operand contract and
// tile order as gemm_i8_mfma_kernel.  The epilogue operands of the tile (asc / row exponents,
// ws, bias, column exponents) are loaded into registers before the main loop and parked in LDS
// after it, so the epilogue itself touches global memory only to store.
template <class C, class MAIN>
__device__ __forceinline__ void contract_tile(const int8_t* __restrict__ A, int lda, const int8_t* __restrict__ W,
                                              int ldw, int M, int N, int K, const EpiParams& ep, int vec_ok,
                                              char* smem_pp, MAIN main) {
  constexpr int BM = C::kBM, BN = C::kBN;
  constexpr int kWaves = C::kThreads / 64;
  const int mtiles = (M + BM - 1) / BM, ntiles = (N + BN - 1) / BN;
  const int L = lsk::xcd_logical_id(blockIdx.x, mtiles * ntiles);
  constexpr int GM = LSK_GROUP_M;
  const int group = L / (GM * ntiles);
  const int first_m = group * GM;
  const int gsize = (mtiles - first_m) < GM ? (mtiles - first_m) : GM;
  const int r = L - group * GM * ntiles;
  const int m0 = (first_m + r % gsize) * BM, n0 = (r / gsize) * BN;

  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();

  // epilogue operands: thread t holds row m0 + t and column n0 + t
  float s_row = 0.0f, s_ws = 0.0f, s_b = 0.0f;
  int s_ec = 0;
  if (tid < BM && m0 + tid < M) {
    if (ep.order == LSK_EPI_POW2) s_row = __int_as_float(ep.erow ? ep.erow[m0 + tid] : 0);
    else if (ep.order != LSK_EPI_RAW) s_row = ep.asc[m0 + tid];
  }
  if (tid < BN && n0 + tid < N) {
    if (ep.order == LSK_EPI_POW2) {
      s_ec = ep.ecol ? ep.ecol[n0 + tid] : 0;
    } else if (ep.order != LSK_EPI_RAW) {
      s_ws = ep.ws[n0 + tid];
      if (ep.bias) s_b = ep.bias[n0 + tid];
    }
  }

  // (the row-pair layouts: m0 and n0 are even, so a tile's rows start at byte m0 * lda / n0 * ldw
  // as well; an odd M or N ends in a pair whose second row is never read)
  const int ap = ep.pairs & 1, bp = ep.pairs & 2;
  const int64_t a_rows = ap ? (int64_t)((M - m0 + 1) & ~1) : (int64_t)(M - m0);
  const int64_t b_rows = bp ? (int64_t)((N - n0 + 1) & ~1) : (int64_t)(N - n0);
  const __amdgpu_buffer_rsrc_t ra_res = lsk::make_rsrc(A + (int64_t)m0 * lda, a_rows * lda);
  const __amdgpu_buffer_rsrc_t rb_res = lsk::make_rsrc(W + (int64_t)n0 * ldw, b_rows * ldw);
  typename C::RowsA pa;
  typename C::RowsB pb;
#pragma unroll
  for (int j = 0; j < C::kLA; ++j) {
    int row, kb;
    lsk::pp_slot<C::kThreads, C::kChunks>(tid, j, row, kb);
    const uint32_t ro = ap ? (uint32_t)((row >> 1) * 2 * lda + (row & 1) * 64) : (uint32_t)(row * lda);
    pa[j] = (m0 + row < M) ? ro : lsk::kOob;
  }
#pragma unroll
  for (int j = 0; j < C::kLB; ++j) {
    int row, kb;
    lsk::pp_slot<C::kThreads, C::kChunks>(tid, j, row, kb);
    const uint32_t ro = bp ? (uint32_t)((row >> 1) * 2 * ldw + (row & 1) * 64) : (uint32_t)(row * ldw);
    pb[j] = (n0 + row < N) ? ro : lsk::kOob;
  }
  typename C::Acc acc;
#pragma unroll
  for (int i = 0; i < C::TM; ++i)
#pragma unroll
    for (int j = 0; j < C::TN; ++j) acc[i][j] = lsk::zero16();

  main(acc, ra_res, pa, rb_res, pb, K, smem_pp, ep.pairs);

  // every wave is past its last read of the LDS ring
  float* sc_row = (float*)(smem_pp + C::kScaleOff);
  float* sc_ws = sc_row + BM;
  float* sc_b = sc_ws + BN;
  int* sc_ec = (int*)(sc_b + BN);
  if (tid < BM) sc_row[tid] = s_row;
  if (tid < BN) {
    sc_ws[tid] = s_ws;
    sc_b[tid] = s_b;
    sc_ec[tid] = s_ec;
  }
  // per wave: whether one of its operands rules out the fast epilogue (a NaN output possible);
  // eight flag words, the unused ones clear
  int* sc_flag = (int*)(smem_pp + C::kFlagOff);
  const bool odd = (tid < BM && !(__builtin_fabsf(s_row) < __builtin_inff())) ||
                   (tid < BN && !(__builtin_fabsf(s_ws) < 0x1p96f));
  const bool wave_odd = __builtin_amdgcn_ballot_w64(odd) != 0;
  if (lane == 0) sc_flag[wave] = wave_odd ? 1 : 0;
  if (kWaves < 8 && tid < 8 - kWaves) sc_flag[kWaves + tid] = 0;
  __syncthreads();
  // each wave stages its own 32-row strips, then stores them through the epilogue
  const bool bias = ep.bias != nullptr;
  if (ep.order == LSK_EPI_V21 && !bias && vec_ok == 2 && m0 + BM <= M && n0 + BN <= N &&
      ep.out_dtype == LSK_BF16) {
    const v4i f0 = *(const v4i*)sc_flag, f1 = *(const v4i*)(sc_flag + 4);
    if (((f0 | f1)[0] | (f0 | f1)[1] | (f0 | f1)[2] | (f0 | f1)[3]) == 0) {
      const int ldo_bytes = (int)(ep.ldo * 2);
      char* base = (char*)ep.out + ((int64_t)m0 * ep.ldo + n0) * 2;
      const __amdgpu_buffer_rsrc_t ro = lsk::make_rsrc(base, (int64_t)(BM - 1) * ldo_bytes + BN * 2);
      pp_epilogue_fast<C, 0>(acc, ro, ldo_bytes, smem_pp);
      return;
    }
  }
  if (ep.order == LSK_EPI_POW2 && ep.ecol == nullptr && vec_ok == 2 && m0 + BM <= M && n0 + BN <= N &&
      ep.out_dtype == LSK_F32) {
    const int ldo_bytes = (int)(ep.ldo * 4);
    char* base = (char*)ep.out + ((int64_t)m0 * ep.ldo + n0) * 4;
    const __amdgpu_buffer_rsrc_t ro = lsk::make_rsrc(base, (int64_t)(BM - 1) * ldo_bytes + BN * 4);
    pp_epilogue_direct_pow2<C>(acc, ro, ldo_bytes, ep.shift, (const float*)(smem_pp + C::kScaleOff));
    return;
  }
#define LSK_PP_EPI(O, D, B)                                                        \
  if (ep.order == O && ep.out_dtype == D && bias == B) {                           \
    pp_epilogue<C, O, D, B, 0>(acc, ep, m0, n0, M, N, vec_ok, smem_pp);            \
    return;                                                                        \
  }
  LSK_PP_EPI(LSK_EPI_V21, LSK_BF16, false)
  LSK_PP_EPI(LSK_EPI_V21, LSK_BF16, true)
  LSK_PP_EPI(LSK_EPI_V21, LSK_F32, false)
  LSK_PP_EPI(LSK_EPI_V21, LSK_BF16_AS_F32, false)
  LSK_PP_EPI(LSK_EPI_V2, LSK_BF16, false)
  LSK_PP_EPI(LSK_EPI_POW2, LSK_F32, false)
  LSK_PP_EPI(LSK_EPI_RAW, LSK_I32, false)
#undef LSK_PP_EPI
  pp_epilogue<C, -1, -1, false, 0>(acc, ep, m0, n0, M, N, vec_ok, smem_pp);  // any other combination
}

// Dense ping-pong tile kernel (512 threads, eight waves in two alternating groups).
template <int BM, int BN, int WM, int WN, int RING, int BKB>
__global__ __launch_bounds__(512, (RING == 3 && BKB == 64 ? 2 : 1)) void gemm_i8_pp_kernel(const int8_t* __restrict__ A, int lda,
                                                         const int8_t* __restrict__ W, int ldw, int M, int N, int K,
                                                         EpiParams ep, int vec_ok) {
  using C = lsk::PPCfg<BM, BN, WM, WN, RING, BKB>;
  extern __shared__ __attribute__((aligned(16))) char smem_pp[];
  contract_tile<C>(A, lda, W, ldw, M, N, K, ep, vec_ok, smem_pp,
                   [](typename C::Acc& acc, __amdgpu_buffer_rsrc_t ra, const typename C::RowsA& pa,
                      __amdgpu_buffer_rsrc_t rb, const typename C::RowsB& pb, int K_, char* sm, int pairs) {
                     lsk::pp_mainloop<BM, BN, WM, WN, RING, BKB>(acc, ra, pa, rb, pb, K_, sm, 0, pairs);
                   });
}

// Persistent form of the ping-pong kernel for whole tiles under the POW2 order with binary32
// output and no column exponents (the ref_block_v1 GEMMs, ref_block_v1.py:167,193,198,218): one
// block per CU walks tiles blockIdx.x, blockIdx.x + gridDim.x, ... in the one-tile-per-block
// launch's order (hardware ids congruent mod 8 stay on one XCD).  After a tile's main loop the
// block fills the whole ring with the next tile's first stages (no wave reads it any more) and
// only then stores the finished tile from its accumulators: the next tile's first loads and the
// block start leave the critical path, and the stores drain while the next tile's first three
// stages are multiplied.  M % BM == 0, N % BN == 0, K % BKB == 0 with at least kRing + 2 stages.
// (Measured on MI355X: the Qwen2.5-7B block GEMMs at 8192 rows 1.5% faster than one tile per
// block.)
template <int BM, int BN, int WM, int WN, int RING, int BKB>
__global__ __launch_bounds__(512, 1) void gemm_i8_pp_pow2_persist_kernel(const int8_t* __restrict__ A, int lda,
                                                                         const int8_t* __restrict__ W, int ldw, int M,
                                                                         int N, int K, EpiParams ep) {
  using C = lsk::PPCfg<BM, BN, WM, WN, RING, BKB>;
  extern __shared__ __attribute__((aligned(16))) char smem_pp[];
  const int mtiles = M / BM, ntiles = N / BN, tiles = mtiles * ntiles;
  const int tid = threadIdx.x;
  float* sc_row = (float*)(smem_pp + C::kScaleOff);
  constexpr int GM = LSK_GROUP_M;
  struct Tile {
    int m0, n0;
    __amdgpu_buffer_rsrc_t ra, rb;
    typename C::RowsA pa;
    typename C::RowsB pb;
    float erow;
  };
  auto setup = [&](int v, Tile& t) {
    const int L = lsk::xcd_logical_id(v, tiles);
    const int group = L / (GM * ntiles);
    const int first_m = group * GM;
    const int gsize = (mtiles - first_m) < GM ? (mtiles - first_m) : GM;
    const int r = L - group * GM * ntiles;
    t.m0 = (first_m + r % gsize) * BM;
    t.n0 = (r / gsize) * BN;
    t.ra = lsk::make_rsrc(A + (int64_t)t.m0 * lda, (int64_t)BM * lda);
    t.rb = lsk::make_rsrc(W + (int64_t)t.n0 * ldw, (int64_t)BN * ldw);
#pragma unroll
    for (int j = 0; j < C::kLA; ++j) {
      int row, kb;
      lsk::pp_slot<C::kThreads, C::kChunks>(tid, j, row, kb);
      t.pa[j] = (ep.pairs & 1) ? (uint32_t)((row >> 1) * 2 * lda + (row & 1) * 64) : (uint32_t)(row * lda);
    }
#pragma unroll
    for (int j = 0; j < C::kLB; ++j) {
      int row, kb;
      lsk::pp_slot<C::kThreads, C::kChunks>(tid, j, row, kb);
      t.pb[j] = (ep.pairs & 2) ? (uint32_t)((row >> 1) * 2 * ldw + (row & 1) * 64) : (uint32_t)(row * ldw);
    }
    t.erow = (tid < BM && ep.erow) ? __int_as_float(ep.erow[t.m0 + tid]) : 0.0f;
  };
  const int ldo_bytes = (int)(ep.ldo * 4);
  Tile cur;
  setup(blockIdx.x, cur);
  for (int v = blockIdx.x, it = 0; v < tiles; v += gridDim.x, ++it) {
    typename C::Acc acc;
#pragma unroll
    for (int i = 0; i < C::TM; ++i)
#pragma unroll
      for (int j = 0; j < C::TN; ++j) acc[i][j] = lsk::zero16();
    if (it == 0)
      lsk::pp_mainloop<BM, BN, WM, WN, RING, BKB, false>(acc, cur.ra, cur.pa, cur.rb, cur.pb, K, smem_pp, 0, ep.pairs);
    else
      lsk::pp_mainloop<BM, BN, WM, WN, RING, BKB, true>(acc, cur.ra, cur.pa, cur.rb, cur.pb, K, smem_pp, 0, ep.pairs);
    // every wave is past its last read of the ring; the previous tile's epilogue (the last
    // reader of sc_row) ended before this tile's first barrier
    if (tid < BM) sc_row[tid] = cur.erow;
    const __amdgpu_buffer_rsrc_t ro =
        lsk::make_rsrc((char*)ep.out + ((int64_t)cur.m0 * ep.ldo + cur.n0) * 4, (int64_t)(BM - 1) * ldo_bytes + BN * 4);
    if (v + (int)gridDim.x < tiles) {
      setup(v + gridDim.x, cur);
      lsk::pp_issue_prologue<BM, BN, WM, WN, RING, BKB>(cur.ra, cur.pa, cur.rb, cur.pb, K, smem_pp, ep.pairs);
    }
    __syncthreads();
    pp_epilogue_direct_pow2<C>(acc, ro, ldo_bytes, ep.shift, sc_row);
  }
}

// Dense four-wave tile kernel (256 threads, one wave per SIMD, 128-row wave tiles; w4_tile.h).
template <int BM, int BN, int RING>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1))) void gemm_i8_w4_kernel(
    const int8_t* __restrict__ A, int lda, const int8_t* __restrict__ W, int ldw, int M, int N, int K, EpiParams ep,
    int vec_ok) {
  using C = lsk::W4Cfg<BM, BN, RING>;
  extern __shared__ __attribute__((aligned(16))) char smem_pp[];
  contract_tile<C>(A, lda, W, ldw, M, N, K, ep, vec_ok, smem_pp,
                   [](typename C::Acc& acc, __amdgpu_buffer_rsrc_t ra, const typename C::RowsA& pa,
                      __amdgpu_buffer_rsrc_t rb, const typename C::RowsB& pb, int K_, char* sm, int) {
                     lsk::w4_mainloop<C>(acc, ra, pa, rb, pb, K_, sm);  // row-major A only
                   });
}

// Decode GEMV (M <= 32), bandwidth-bound on the weight stream: one block per 16 output
// columns, its KW waves splitting K into 64-byte-aligned slices.  Lane l streams 16 bytes of
// weight row n0 + l % 16 at K-group l / 16 of each 64-byte step (one v_mfma_i32_16x16x64_i8
// per step and 16-row tile of activations); batches of U steps are loaded one batch ahead of
// their MFMAs.  The waves' partial sums are added exactly in LDS; wave 0 applies the
// epilogue.  Edge rows, the K tail and slice ends load zeros through the buffer range.
template <int MT, int U>
__global__ __launch_bounds__(1024) void gemv_i8_stream_kernel(const int8_t* __restrict__ A, int lda,
                                                              const int8_t* __restrict__ W, int ldw, int M, int N,
                                                              int K, int kslice, EpiParams ep) {
  extern __shared__ v4i red_gemv[];  // [(KW - 1) * MT][64]
  const int lane = threadIdx.x & 63, wave = wave_id(), KW = blockDim.x >> 6;
  const int col = lane & 15, kg = lane >> 4;
  const int n0 = blockIdx.x * 16;
  const int nrows = (N - n0) < 16 ? (N - n0) : 16;
  const __amdgpu_buffer_rsrc_t rw = lsk::make_rsrc(W + (int64_t)n0 * ldw, (int64_t)nrows * ldw);
  const __amdgpu_buffer_rsrc_t ra = lsk::make_rsrc(A, (int64_t)M * lda);
  const uint32_t wrow = (col < nrows) ? (uint32_t)(col * ldw) : lsk::kOob;
  uint32_t arow[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t) arow[t] = (t * 16 + col < M) ? (uint32_t)((t * 16 + col) * lda) : lsk::kOob;
  const int kb = wave * kslice;
  const int ke = (kb + kslice) < K ? (kb + kslice) : K;
  // wave 0's epilogue operands, requested first (used at the end)
  const EpiRaw er_ = epi_raw(ep, M, N);
  const uint32_t c0w = epi_raw_col0(er_, n0 + col, wave == 0 && col < nrows);
  const uint32_t c1w = epi_raw_col1(er_, n0 + col, wave == 0 && col < nrows);
  // (the row operands too with one activation tile; with two, their registers would spill)
  uint32_t rw_[MT][4];
#pragma unroll
  for (int t = 0; t < MT; ++t)
#pragma unroll
    for (int r = 0; r < 4; ++r)
      rw_[t][r] = MT == 1 ? epi_raw_row(er_, t * 16 + kg * 4 + r, wave == 0 && t * 16 + kg * 4 + r < M) : 0u;

  // one batch = U 64-byte steps: weights (non-temporal) and activations, loaded one batch
  // ahead of the MFMAs that consume them (register double buffer)
  auto load_batch = [&](v4i* w, v4i (*a)[MT], int k) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int kk = k + u * 64 + kg * 16;
      const bool in = kk < ke;
#pragma unroll
      for (int t = 0; t < MT; ++t) a[u][t] = lsk::buf_load16(ra, in ? arow[t] + (uint32_t)kk : lsk::kOob);
      w[u] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(rw, in ? wrow + (uint32_t)kk : lsk::kOob,
                                                                           0, 2 /* non-temporal */));
    }
  };
  v4i acc[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t) acc[t] = zero4();
  auto mma_batch = [&](const v4i* w, const v4i (*a)[MT]) {
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int t = 0; t < MT; ++t) acc[t] = lsk::mfma_i8(a[u][t], w[u], acc[t]);
  };
  // two register sets in turn (no copies between them, so no wait on the newer loads)
  v4i w0[U], a0[U][MT], w1[U], a1[U][MT];
  load_batch(w0, a0, kb);
  lsk::compiler_fence();
  for (int k = kb; k < ke; k += 128 * U) {
    load_batch(w1, a1, k + 64 * U);
    __builtin_amdgcn_sched_barrier(0);
    mma_batch(w0, a0);
    __builtin_amdgcn_sched_barrier(0);
    if (k + 64 * U >= ke) break;
    load_batch(w0, a0, k + 128 * U);
    __builtin_amdgcn_sched_barrier(0);
    mma_batch(w1, a1);
    __builtin_amdgcn_sched_barrier(0);
  }
  if (wave > 0) {
#pragma unroll
    for (int t = 0; t < MT; ++t) red_gemv[((wave - 1) * MT + t) * 64 + lane] = acc[t];
  }
  __syncthreads();
  if (wave != 0) return;
  const int n = n0 + col;
  const EpiCol ec = epi_col_of(ep, c0w, c1w);
  if (MT > 1) {
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) rw_[t][r] = epi_raw_row(er_, t * 16 + kg * 4 + r, t * 16 + kg * 4 + r < M);
  }
  for (int w2 = 1; w2 < KW; ++w2)
#pragma unroll
    for (int t = 0; t < MT; ++t) acc[t] += red_gemv[((w2 - 1) * MT + t) * 64 + lane];
#pragma unroll
  for (int t = 0; t < MT; ++t)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int m = t * 16 + kg * 4 + r;
      if (m < M && n < N) epilogue_store_rc(ep, m, n, acc[t][r], epi_row_of(ep, rw_[t][r]), ec);
    }
}

// Decode GEMV (4 < M <= 32) with whole-row weight streaming through LDS.  A block owns 16
// weight rows; its NW waves split K into slices of whole SB-byte stages.  Each wave streams its
// slice of the 16 rows into its own LDS ring by direct loads, each instruction reading 1024 / SB
// whole SB-byte row segments (long contiguous runs stream faster from HBM than the MFMA
// operand's 64-byte pieces), then reads them back in the v_mfma_i32_16x16x64_i8 B layout (chunk c
// of row r stored at c ^ r: the 16 rows one LDS cycle serves hit distinct bank groups).  The
// activation fragments (MT tiles of 16 rows) are loaded into registers one stage ahead.  A wave
// waits only for its own loads (exact counts, no barrier in the loop); the K-slices' exact int32
// sums are added in LDS and wave 0 applies the epilogue.  Rows past N, activation rows past M and
// bytes past K load zeros through the buffer ranges.
template <int MT, int SB, int R>
__global__ __launch_bounds__(1024) void gemv_i8_lds_kernel(const int8_t* __restrict__ A, int lda,
                                                           const int8_t* __restrict__ W, int ldw, int M, int N,
                                                           int K, int kslice, EpiParams ep) {
  extern __shared__ __attribute__((aligned(16))) char smem_lds[];
  constexpr int kRPI = 1024 / SB;        // rows per load instruction
  constexpr int kCPR = SB / 16;          // 16-byte chunks per row per stage
  constexpr int kWL = 16 / kRPI;         // weight loads per lane per stage
  constexpr int kKS = SB / 64;           // MFMA K-steps per stage
  constexpr int kAL = kKS * MT;          // activation loads per lane per stage
  constexpr int kStage = 16 * SB;        // bytes of one ring stage
  const int lane = threadIdx.x & 63, wave = wave_id(), NW = blockDim.x >> 6;
  const int n0 = blockIdx.x * 16;
  const int nrows = (N - n0) < 16 ? (N - n0) : 16;
  const int kb = wave * kslice;
  const int ke = (kb + kslice) < K ? (kb + kslice) : K;
  const int nst = ke > kb ? (ke - kb + SB - 1) / SB : 0;
  char* ring = smem_lds + wave * R * kStage;
  // wave 0's epilogue operands, requested first (used at the end)
  const int rr0 = lane & 15, kg0 = lane >> 4;
  const EpiRaw er_ = epi_raw(ep, M, N);
  const uint32_t c0w = epi_raw_col0(er_, n0 + rr0, wave == 0 && rr0 < nrows);
  const uint32_t c1w = epi_raw_col1(er_, n0 + rr0, wave == 0 && rr0 < nrows);
  uint32_t rw_[MT][4];
#pragma unroll
  for (int t = 0; t < MT; ++t)
#pragma unroll
    for (int r = 0; r < 4; ++r) rw_[t][r] = epi_raw_row(er_, t * 16 + kg0 * 4 + r, wave == 0 && t * 16 + kg0 * 4 + r < M);
  const __amdgpu_buffer_rsrc_t rw = lsk::make_rsrc(W + (int64_t)n0 * ldw, (int64_t)nrows * ldw);
  const __amdgpu_buffer_rsrc_t ra = lsk::make_rsrc(A, (int64_t)M * lda);

  // this lane's weight slots: instruction j reads its row's logical chunk.  (The load offsets are
  // computed into locals before the direct-load builtin: with the conditional expression inside
  // its argument list the host pass silently emitted no launch stub for this kernel.)
  struct Slots {
    uint32_t off[kWL];  // byte offset of the slot's row
    int k[kWL];         // byte offset of the slot's logical chunk within a stage
  } ws_;
#pragma unroll
  for (int j = 0; j < kWL; ++j) {
    const int row = j * kRPI + lane / kCPR;
    ws_.off[j] = (uint32_t)(row * ldw);
    ws_.k[j] = 16 * ((lane % kCPR) ^ row);
  }
  uint32_t arow[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t) arow[t] = (t * 16 + (lane & 15) < M) ? (uint32_t)((t * 16 + (lane & 15)) * lda) : lsk::kOob;
  const int ag = 16 * (lane >> 4);

  auto issue_w = [&](int st) {
    char* slot = ring + (st % R) * kStage;
    const int k0 = kb + st * SB;
#pragma unroll
    for (int j = 0; j < kWL; ++j) {
      const int kk = k0 + ws_.k[j];
      const uint32_t off = kk < ke ? ws_.off[j] + (uint32_t)kk : lsk::kOob;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rw, (lsk::lds_void_t)(slot + j * 1024), 16, off, 0, 0,
                                               2 /* non-temporal */);
    }
  };
  auto issue_a = [&](int st, v4i (&a)[kKS][MT]) {
    const int k0 = kb + st * SB;
#pragma unroll
    for (int s = 0; s < kKS; ++s)
#pragma unroll
      for (int t = 0; t < MT; ++t) {
        const int kk = k0 + s * 64 + ag;
        a[s][t] = lsk::buf_load16(ra, kk < ke ? arow[t] + (uint32_t)kk : lsk::kOob);
      }
  };
  v4i acc[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t) acc[t] = zero4();
  const int rr = lane & 15;
  auto compute = [&](int st, const v4i (&a)[kKS][MT]) {
    const char* slot = ring + (st % R) * kStage + rr * SB;
#pragma unroll
    for (int s = 0; s < kKS; ++s) {
      const v4i w = *(const v4i*)(slot + 16 * ((4 * s + (lane >> 4)) ^ rr));
#pragma unroll
      for (int t = 0; t < MT; ++t) acc[t] = lsk::mfma_i8(a[s][t], w, acc[t]);
    }
  };
  // issue order: A(0) W(0) W(1) | step t: A(t+1) W(t+2), then wait for everything up to A(t)
  v4i a0[kKS][MT], a1[kKS][MT];
  auto step = [&](int st, v4i (&acur)[kKS][MT], v4i (&anext)[kKS][MT]) {
    const bool n1 = st + 1 < nst, n2 = st + 2 < nst;
    if (n1) issue_a(st + 1, anext);
    if (n2) issue_w(st + 2);
    lsk::compiler_fence();
    // younger than A(st): W(st+1), A(st+1), W(st+2) when issued
    if (n2) lsk::wait_vm<2 * kWL + kAL>();
    else if (n1) lsk::wait_vm<kWL + kAL>();
    else lsk::wait_vm<0>();
    compute(st, acur);
  };
  if (nst > 0) {
    issue_a(0, a0);
    issue_w(0);
    if (nst > 1) issue_w(1);
    for (int st = 0; st < nst; st += 2) {
      step(st, a0, a1);
      if (st + 1 < nst) step(st + 1, a1, a0);
    }
  }
  // the K-slices: waves 1.. park their sums, wave 0 adds them in any order (exact) and stores
  __syncthreads();
  v4i* red = (v4i*)smem_lds;
  if (wave > 0) {
#pragma unroll
    for (int t = 0; t < MT; ++t) red[((wave - 1) * MT + t) * 64 + lane] = acc[t];
  }
  __syncthreads();
  if (wave != 0) return;
  const int n = n0 + rr;
  const EpiCol ec = epi_col_of(ep, c0w, c1w);
  for (int w2 = 1; w2 < NW; ++w2)
#pragma unroll
    for (int t = 0; t < MT; ++t) acc[t] += red[((w2 - 1) * MT + t) * 64 + lane];
#pragma unroll
  for (int t = 0; t < MT; ++t)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int m = t * 16 + 4 * (lane >> 4) + r;
      if (m < M && n < N) epilogue_store_rc(ep, m, n, acc[t][r], epi_row_of(ep, rw_[t][r]), ec);
    }
}

// Decode GEMV (4 < M <= 32) with the activation rows staged once per block in LDS and the weight
// rows streamed straight into v_mfma_i32_16x16x64_i8 B registers.  A block of GPB x KW waves owns
// GPB groups of 16 weight rows; the KW waves of a group split its K steps.  Prologue, all in
// flight together: the epilogue operands of the lanes that will store, A by direct-to-LDS loads
// (1 KB of one row per instruction; row r at r * ldsk, ldsk a multiple of 1024 plus 16 so that
// consecutive rows start 16 bytes apart in the bank space; zeros past K), then each wave's first
// D weight steps -- and a wait for everything but those D.  Then the weight stream is the only
// traffic counted by a wave's vmcnt: lane l loads 16 bytes of weight row n0 + l % 16 at K-group
// l / 16 of every 64-byte step, D steps in flight, and the matching A fragment comes from LDS.
// With PAIRS the weights are a row-pair copy (rows 2i and 2i + 1 interleaved by 64-byte K chunks,
// row stride ldw a multiple of 64): each load instruction then reads 8 whole 128-byte lines
// instead of 16 half lines.  Weight bytes past K multiply zeros of A; rows past N and steps past
// the slice load zeros through the buffer range.  The K-slices' exact int32 sums are added in LDS
// (over the A area, after a barrier) and the group's first wave applies the epilogue.
template <int MT, int D, bool PAIRS>
__global__ __launch_bounds__(1024) void gemv_i8_skinny_kernel(const int8_t* __restrict__ A, int lda,
                                                              const int8_t* __restrict__ W, int ldw, int M, int N,
                                                              int K, int gpb, int kw, int sps, int ldsk, EpiParams ep) {
  extern __shared__ __attribute__((aligned(16))) char smem_sk[];
  const int lane = threadIdx.x & 63, wave = wave_id(), nw = blockDim.x >> 6;
  const int steps = (K + 63) >> 6;
  const int G = (N + 15) >> 4;
  const int g = blockIdx.x * gpb + wave / kw;
  const int ks = wave - (wave / kw) * kw;
  const int s0 = ks * sps;
  const int nst = g < G ? max(0, min(steps, s0 + sps) - s0) : 0;
  const int col = lane & 15, kg = lane >> 4;
  const int n = g * 16 + col;
  // the raw epilogue operands of this lane's outputs (row: asc, or erow under POW2; column: ws and
  // bias, or ecol), loaded ahead of everything else by branch-free buffer loads (zeros past M / N
  // and for absent operands) and only combined at the stores, so no load waits here
  const bool mine = ks == 0 && g < G;
  const EpiRaw er_ = epi_raw(ep, M, N);
  const uint32_t col0 = epi_raw_col0(er_, n, mine && n < N), col1 = epi_raw_col1(er_, n, mine && n < N);
  uint32_t rowv[MT][4];
#pragma unroll
  for (int t = 0; t < MT; ++t)
#pragma unroll
    for (int r = 0; r < 4; ++r) rowv[t][r] = epi_raw_row(er_, t * 16 + kg * 4 + r, mine && t * 16 + kg * 4 + r < M);
  lsk::compiler_fence();
  // A into LDS: chunk c = (row, 1 KB piece) per wave instruction
  {
    const int cpr = (K + 1023) >> 10;
    const __amdgpu_buffer_rsrc_t ra = lsk::make_rsrc(A, (int64_t)(M - 1) * lda + K);
    for (int c = wave; c < M * cpr; c += nw) {
      const int r = c / cpr, j = c - r * cpr;
      const int kb = j * 1024 + lane * 16;
      const uint32_t off = kb < K ? (uint32_t)(r * lda + kb) : lsk::kOob;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (lsk::lds_void_t)(smem_sk + r * ldsk + j * 1024), 16, off, 0, 0,
                                               0);
    }
  }
  // the first D weight steps
  const int n0 = g * 16;
  const int nrows = g < G ? ((N - n0) < 16 ? (N - n0) : 16) : 0;
  const int64_t wbytes = PAIRS ? (int64_t)((nrows + 1) >> 1) * 2 * ldw : (int64_t)nrows * ldw;
  const __amdgpu_buffer_rsrc_t rw = lsk::make_rsrc(W + (int64_t)(g < G ? n0 : 0) * ldw, wbytes);
  const uint32_t wbase = col < nrows ? (PAIRS ? (uint32_t)((col >> 1) * 2 * ldw + (col & 1) * 64 + kg * 16 + s0 * 128)
                                              : (uint32_t)(col * ldw + s0 * 64 + kg * 16))
                                     : lsk::kOob;
  constexpr uint32_t kStep = PAIRS ? 128 : 64;
  v4i w[D];
#pragma unroll
  for (int u = 0; u < D; ++u)
    w[u] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(rw, u < nst ? wbase + u * kStep : lsk::kOob,
                                                                         0, 2 /* non-temporal */));
  lsk::compiler_fence();
  lsk::wait_vm<D>();  // everything older than the D weight steps: A and the epilogue operands
  __syncthreads();
  v4i acc[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t) acc[t] = zero4();
  if (nst > 0) {
    // activation rows of this lane's A fragments (clamped to a staged row; zeroed past M)
    const char* arow[MT];
    bool alive[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      const int r = t * 16 + col;
      alive[t] = r < M;
      arow[t] = smem_sk + (r < M ? r : M - 1) * ldsk + s0 * 64 + kg * 16;
    }
    for (int s = 0; s < nst; s += D) {
      // each step's A fragments are read one step ahead, so their LDS latency overlaps an MFMA
      v4i a[2][MT];
#pragma unroll
      for (int t = 0; t < MT; ++t) a[0][t] = *(const v4i*)(arow[t] + s * 64);
#pragma unroll
      for (int u = 0; u < D; ++u) {
        if (u + 1 < D) {
          const int st = s + u + 1 < nst ? s + u + 1 : 0;
#pragma unroll
          for (int t = 0; t < MT; ++t) a[(u + 1) & 1][t] = *(const v4i*)(arow[t] + st * 64);
        }
#pragma unroll
        for (int t = 0; t < MT; ++t) acc[t] = lsk::mfma_i8(alive[t] ? a[u & 1][t] : zero4(), w[u], acc[t]);
        const int nx = s + u + D;
        w[u] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(
                                           rw, nx < nst ? wbase + nx * kStep : lsk::kOob, 0, 2 /* non-temporal */));
      }
    }
  }
  if (kw > 1) {
    __syncthreads();  // every wave is past its last A read: the partial sums reuse the LDS
    v4i* red = (v4i*)smem_sk;
#pragma unroll
    for (int t = 0; t < MT; ++t) red[(wave * MT + t) * 64 + lane] = acc[t];
    __syncthreads();
    if (ks != 0) return;
    for (int j = 1; j < kw; ++j)
#pragma unroll
      for (int t = 0; t < MT; ++t) acc[t] += red[((wave + j) * MT + t) * 64 + lane];
  }
  if (g >= G) return;
  const EpiCol ec = epi_col_of(ep, col0, col1);
#pragma unroll
  for (int t = 0; t < MT; ++t)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int m = t * 16 + kg * 4 + r;
      if (m < M && n < N) epilogue_store_rc(ep, m, n, acc[t][r], epi_row_of(ep, rowv[t][r]), ec);
    }
}

// Batch-few decode GEMV (M <= MR <= 8) on the VALU (v_dot4c_i32_i8), bandwidth-bound on the
// weight stream.  A block is four waves; each wave owns 8 weight rows and one of WK K-slices
// (WK = 1, 2 or 4 waves per row group).  Lane l reads 16 bytes of row l / 8 at chunk l % 8 of
// every 128-byte step, so each load instruction covers 8 whole 128-byte row segments; U steps
// of loads are in flight while the previous U are multiplied (register double buffer).  The
// activation rows sit in LDS (zero-padded to 128 bytes).  Partial sums are exact int32 and
// reduced across the 8 lanes of a row, then across the K-slices, in any order.
template <int MR, int U>
__global__ __launch_bounds__(256) void gemv_i8_dot_kernel(const int8_t* __restrict__ A, int lda,
                                                          const int8_t* __restrict__ W, int ldw, int M, int N, int K,
                                                          int wk, int kslice, EpiParams ep) {
  extern __shared__ __attribute__((aligned(16))) char smem_dot[];
  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
  const int Kp = (K + 127) & ~127;
  v4i* sa = (v4i*)smem_dot;                           // [MR][Kp / 16]
  int* red = (int*)(smem_dot + MR * Kp);              // [4 waves][8 rows][MR]
  const int rg = wave / wk, ks = wave % wk;
  const int rows_blk = 8 * (4 / wk);
  const int n0 = blockIdx.x * rows_blk;
  const int rl = rg * 8 + (lane >> 3), c = lane & 7;
  const int nrows = (N - n0) < rows_blk ? (N - n0) : rows_blk;
  const __amdgpu_buffer_rsrc_t rw = lsk::make_rsrc(W + (int64_t)n0 * ldw, (int64_t)nrows * ldw);
  const uint32_t wrow = rl < nrows ? (uint32_t)(rl * ldw) : lsk::kOob;
  const int kb = ks * kslice;
  const int ke = (kb + kslice) < K ? (kb + kslice) : K;

  // epilogue operands of the lanes that store (first K-slice, first lane of each row), loaded
  // before the stream so the tail does not wait on them
  const int n = n0 + rl;
  EpiOps eo[MR];
#pragma unroll
  for (int m = 0; m < MR; ++m) eo[m] = EpiOps{0.0f, 0.0f, 0.0f, 0};
  if (ks == 0 && c == 0 && n < N) {
#pragma unroll
    for (int m = 0; m < MR; ++m)
      if (m < M) eo[m] = epi_ops_load(ep, m, n);
  }

  // activation rows -> LDS by direct-to-LDS loads, issued before the weight stream (loads
  // complete in order, so waiting for these never waits for the weights behind them)
  const int kc16 = Kp / 16;
  const __amdgpu_buffer_rsrc_t ra = lsk::make_rsrc(A, (int64_t)M * lda);
  int na = 0;  // this thread's activation loads
  for (int i0 = wave * 64; i0 < MR * kc16; i0 += 256, ++na) {
    const int i = i0 + lane;
    const int m = i / kc16, kc = i - m * kc16;
    const uint32_t off = (m < M && kc * 16 < K) ? (uint32_t)(m * lda + kc * 16) : lsk::kOob;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (lsk::lds_void_t)(smem_dot + i0 * 16), 16, off, 0, 0, 0);
  }
  auto load_batch = [&](v4i* w, int s) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int kk = s + u * 128 + c * 16;
      w[u] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(
                                         rw, kk < ke ? wrow + (uint32_t)kk : lsk::kOob, 0, 2 /* non-temporal */));
    }
  };
  int acc[MR];
#pragma unroll
  for (int m = 0; m < MR; ++m) acc[m] = 0;
  auto dot_batch = [&](const v4i* w, int s) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int kk = s + u * 128 + c * 16;
      if (s + u * 128 < ke) {
#pragma unroll
        for (int m = 0; m < MR; ++m) {
          const v4i a = sa[m * kc16 + kk / 16];
          acc[m] = __builtin_amdgcn_sdot4(a[0], w[u][0], acc[m], false);
          acc[m] = __builtin_amdgcn_sdot4(a[1], w[u][1], acc[m], false);
          acc[m] = __builtin_amdgcn_sdot4(a[2], w[u][2], acc[m], false);
          acc[m] = __builtin_amdgcn_sdot4(a[3], w[u][3], acc[m], false);
        }
      }
    }
  };
  // two register sets in turn (no copies between them, so no wait on the newer loads)
  v4i w0[U], w1[U];
  load_batch(w0, kb);
  // The activation loads must have landed before the barrier.  The compiler may place the
  // first weight batch on either side of this wait, so it cannot be counted on to be
  // outstanding: wait for everything.
  lsk::wait_vm<0>();
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_sched_barrier(0);
  for (int s = kb; s < ke; s += 256 * U) {
    load_batch(w1, s + 128 * U);
    __builtin_amdgcn_sched_barrier(0);
    dot_batch(w0, s);
    __builtin_amdgcn_sched_barrier(0);
    if (s + 128 * U >= ke) break;
    load_batch(w0, s + 256 * U);
    __builtin_amdgcn_sched_barrier(0);
    dot_batch(w1, s + 128 * U);
    __builtin_amdgcn_sched_barrier(0);
  }
  // the 8 lanes of a row, then the K-slices of the row group
#pragma unroll
  for (int m = 0; m < MR; ++m) {
    acc[m] += __shfl_xor(acc[m], 1, 64);
    acc[m] += __shfl_xor(acc[m], 2, 64);
    acc[m] += __shfl_xor(acc[m], 4, 64);
  }
  if (c == 0) {
#pragma unroll
    for (int m = 0; m < MR; ++m) red[(wave * 8 + (lane >> 3)) * MR + m] = acc[m];
  }
  __syncthreads();
  if (ks != 0 || c != 0) return;
#pragma unroll
  for (int m = 0; m < MR; ++m) {
    int sum = 0;
    for (int k2 = 0; k2 < wk; ++k2) sum += red[((rg * wk + k2) * 8 + (lane >> 3)) * MR + m];
    if (m < M && n < N) epilogue_store_ops(ep, m, n, sum, eo[m]);
  }
}

// s_waitcnt vmcnt(n) for a run-time n in [0, 15] (larger n waits for 15).
__device__ __forceinline__ void wait_vm_upto15(int n) {
  switch (n < 0 ? 0 : (n > 15 ? 15 : n)) {
    case 0: lsk::wait_vm<0>(); break;
    case 1: lsk::wait_vm<1>(); break;
    case 2: lsk::wait_vm<2>(); break;
    case 3: lsk::wait_vm<3>(); break;
    case 4: lsk::wait_vm<4>(); break;
    case 5: lsk::wait_vm<5>(); break;
    case 6: lsk::wait_vm<6>(); break;
    case 7: lsk::wait_vm<7>(); break;
    case 8: lsk::wait_vm<8>(); break;
    case 9: lsk::wait_vm<9>(); break;
    case 10: lsk::wait_vm<10>(); break;
    case 11: lsk::wait_vm<11>(); break;
    case 12: lsk::wait_vm<12>(); break;
    case 13: lsk::wait_vm<13>(); break;
    case 14: lsk::wait_vm<14>(); break;
    default: lsk::wait_vm<15>(); break;
  }
}

// Batch-few decode GEMV (M <= MR <= 4), weights streamed through per-wave LDS rings.  A block
// is four waves; each wave owns 8 weight rows and one of WK K-slices.  A step is 128 bytes of
// K of the wave's 8 rows: one direct-to-LDS load (lane l: row l / 8, 16-byte chunk l % 8), so
// every load instruction covers 8 whole 128-byte row segments.  Steps travel in batches of U;
// the wave keeps R batches in flight in its private ring (R * U slots of 1 KB) and waits on its
// own loads only (exact counts: no other vector-memory load is issued in the loop), so the
// stream needs no barrier and no registers.  The activation rows (zero-padded to 128 bytes)
// are staged once per block.  Each lane multiplies its 16-byte chunks on the VALU
// (v_dot4c_i32_i8); the exact int32 sums are reduced across the 8 lanes of a row, then across
// the K-slices, in any order.
template <int MR, int U, int R>
__global__ __launch_bounds__(256) void gemv_i8_ring_kernel(const int8_t* __restrict__ A, int lda,
                                                           const int8_t* __restrict__ W, int ldw, int M, int N, int K,
                                                           int wk, int kslice, EpiParams ep) {
  extern __shared__ __attribute__((aligned(16))) char smem_ring[];
  constexpr int kSlots = U * R;
  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
  const int Kp = (K + 127) & ~127;
  const int kc16 = Kp / 16;
  char* sa = smem_ring;                                         // [MR][Kp] activations
  char* ring = smem_ring + MR * Kp + wave * kSlots * 1024;      // this wave's slots
  int* red = (int*)(smem_ring + MR * Kp + 4 * kSlots * 1024);   // [4 waves][8 rows][MR]
  const int rg = wave / wk, ks = wave % wk;
  const int rows_blk = 8 * (4 / wk);
  const int n0 = blockIdx.x * rows_blk;
  const int rl = rg * 8 + (lane >> 3), c = lane & 7;
  const int nrows = (N - n0) < rows_blk ? (N - n0) : rows_blk;
  const int n = n0 + rl;
  const int kb = ks * kslice;
  const int ke = (kb + kslice) < K ? (kb + kslice) : K;
  const int nbatch = ke > kb ? (ke - kb + 128 * U - 1) / (128 * U) : 0;
  const __amdgpu_buffer_rsrc_t rw = lsk::make_rsrc(W + (int64_t)n0 * ldw, (int64_t)nrows * ldw);
  const __amdgpu_buffer_rsrc_t ra = lsk::make_rsrc(A, (int64_t)M * lda);
  const uint32_t wrow = rl < nrows ? (uint32_t)(rl * ldw) : lsk::kOob;

  // activations -> LDS (every wave a share), then the first R weight batches of this wave
  for (int i0 = wave * 64; i0 < MR * kc16; i0 += 256) {
    const int i = i0 + lane;
    const int m = i / kc16, kc = i - m * kc16;
    const uint32_t off = (m < M && kc * 16 < K) ? (uint32_t)(m * lda + kc * 16) : lsk::kOob;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (lsk::lds_void_t)(sa + i0 * 16), 16, off, 0, 0, 0);
  }
  auto issue = [&](int bt) {
    char* slot = ring + (bt % R) * U * 1024;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int kk = kb + (bt * U + u) * 128 + c * 16;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rw, (lsk::lds_void_t)(slot + u * 1024), 16,
                                               kk < ke ? wrow + (uint32_t)kk : lsk::kOob, 0, 0, 2 /* non-temporal */);
    }
  };
#pragma unroll
  for (int bt = 0; bt < R; ++bt)
    if (bt < nbatch) issue(bt);
  // everything issued so far has landed (one latency for all of it); the activations are
  // visible to the block after the barrier
  lsk::wait_vm<0>();
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_sched_barrier(0);

  int acc[MR];
#pragma unroll
  for (int m = 0; m < MR; ++m) acc[m] = 0;
  for (int bt = 0; bt < nbatch; ++bt) {
    // batches issued after batch bt: min(nbatch, bt + R) - bt - 1 (those before R landed already)
    if (bt >= R) {
      if (nbatch - bt - 1 >= R - 1) lsk::wait_vm<U * (R - 1)>();
      else wait_vm_upto15(U * (nbatch - bt - 1));
    }
    const char* slot = ring + (bt % R) * U * 1024;
    v4i w[U], a[U][MR];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      w[u] = *(const v4i*)(slot + u * 1024 + lane * 16);
      const int kl = (kb + (bt * U + u) * 128) / 16 + c;
#pragma unroll
      for (int m = 0; m < MR; ++m) a[u][m] = *(const v4i*)(sa + m * Kp + (kl < kc16 ? kl : 0) * 16);
    }
    lsk::wait_lgkm0();  // the batch is in registers: its slots can be refilled
    if (bt + R < nbatch) issue(bt + R);
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int m = 0; m < MR; ++m) {
        acc[m] = __builtin_amdgcn_sdot4(a[u][m][0], w[u][0], acc[m], false);
        acc[m] = __builtin_amdgcn_sdot4(a[u][m][1], w[u][1], acc[m], false);
        acc[m] = __builtin_amdgcn_sdot4(a[u][m][2], w[u][2], acc[m], false);
        acc[m] = __builtin_amdgcn_sdot4(a[u][m][3], w[u][3], acc[m], false);
      }
  }
  EpiOps eo[MR];
#pragma unroll
  for (int m = 0; m < MR; ++m) eo[m] = EpiOps{0.0f, 0.0f, 0.0f, 0};
  if (ks == 0 && c == 0 && n < N) {
#pragma unroll
    for (int m = 0; m < MR; ++m)
      if (m < M) eo[m] = epi_ops_load(ep, m, n);
  }
  // the 8 lanes of a row, then the K-slices of the row group
#pragma unroll
  for (int m = 0; m < MR; ++m) {
    acc[m] += __shfl_xor(acc[m], 1, 64);
    acc[m] += __shfl_xor(acc[m], 2, 64);
    acc[m] += __shfl_xor(acc[m], 4, 64);
  }
  if (c == 0) {
#pragma unroll
    for (int m = 0; m < MR; ++m) red[(wave * 8 + (lane >> 3)) * MR + m] = acc[m];
  }
  __syncthreads();
  if (ks != 0 || c != 0) return;
#pragma unroll
  for (int m = 0; m < MR; ++m) {
    int sum = 0;
    for (int k2 = 0; k2 < wk; ++k2) sum += red[((rg * wk + k2) * 8 + (lane >> 3)) * MR + m];
    if (m < M && n < N) epilogue_store_ops(ep, m, n, sum, eo[m]);
  }
}

// Batch-few decode GEMV (M <= MR <= 4) streaming whole weight rows.  Each load instruction of
// a wave reads 1 KB of one row (lane l: bytes 16 l .. 16 l + 15 of a 1 KB chunk): contiguous
// streams reach a higher HBM rate than several rows per instruction.  A wave owns RPW rows
// and one of WK K-slices of NC chunks; the activations of its K-slice sit in registers
// (loaded once), the next row is loaded while the current one is multiplied on the VALU
// (v_dot4c_i32_i8), and each row's exact int32 sum is reduced across the wave; the K-slices
// of a row are added in LDS.  Everything outside [0, K) and past the last row loads zero
// through the buffer range.
template <int MR, int NC>
__global__ __launch_bounds__(256) void gemv_i8_row_kernel(const int8_t* __restrict__ A, int lda,
                                                          const int8_t* __restrict__ W, int ldw, int M, int N, int K,
                                                          int wk, int rpw, EpiParams ep) {
  __shared__ int red[4][16][MR];  // [wave][row of the wave][m], rpw <= 16
  const int lane = threadIdx.x & 63, wave = wave_id();
  const int rg = wave / wk, ks = wave % wk;
  const int rows_blk = rpw * (4 / wk);
  const int n0 = blockIdx.x * rows_blk;
  const int nrows = (N - n0) < rows_blk ? (N - n0) : rows_blk;
  const int kb = ks * NC * 1024;
  const int ke = (kb + NC * 1024) < K ? (kb + NC * 1024) : K;
  const __amdgpu_buffer_rsrc_t rw = lsk::make_rsrc(W + (int64_t)n0 * ldw, (int64_t)nrows * ldw);
  const __amdgpu_buffer_rsrc_t ra = lsk::make_rsrc(A, (int64_t)M * lda);

  // this lane's byte offsets within the K-slice (kOob past its end)
  uint32_t koff[NC];
#pragma unroll
  for (int j = 0; j < NC; ++j) {
    const int kk = kb + j * 1024 + lane * 16;
    koff[j] = kk < ke ? (uint32_t)kk : lsk::kOob;
  }
  v4i a[MR][NC];
#pragma unroll
  for (int m = 0; m < MR; ++m)
#pragma unroll
    for (int j = 0; j < NC; ++j)
      a[m][j] = lsk::buf_load16(ra, (m < M && koff[j] != lsk::kOob) ? (uint32_t)(m * lda) + koff[j] : lsk::kOob);

  const int r0 = rg * rpw;  // first row of this wave within the block
  // the epilogue operands of the lane that stores row r0 + lane (requested now, used at the end)
  const bool owner = ks == 0 && lane < rpw && r0 + lane < nrows;
  const EpiRaw er_ = epi_raw(ep, M, N);
  const uint32_t c0w = epi_raw_col0(er_, n0 + r0 + lane, owner), c1w = epi_raw_col1(er_, n0 + r0 + lane, owner);
  uint32_t rw_[MR];
#pragma unroll
  for (int m = 0; m < MR; ++m) rw_[m] = epi_raw_row(er_, m, owner && m < M);
  auto load_row = [&](v4i* w, int i) {
    const int rl = r0 + i;
    const uint32_t rowoff = rl < nrows ? (uint32_t)(rl * ldw) : lsk::kOob;
#pragma unroll
    for (int j = 0; j < NC; ++j)
      w[j] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(
                                         rw, (rowoff == lsk::kOob || koff[j] == lsk::kOob) ? lsk::kOob : rowoff + koff[j],
                                         0, 2 /* non-temporal */));
  };
  auto row_sum = [&](const v4i* w, int i) {
    int acc[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      acc[m] = 0;
#pragma unroll
      for (int j = 0; j < NC; ++j) {
        acc[m] = __builtin_amdgcn_sdot4(a[m][j][0], w[j][0], acc[m], false);
        acc[m] = __builtin_amdgcn_sdot4(a[m][j][1], w[j][1], acc[m], false);
        acc[m] = __builtin_amdgcn_sdot4(a[m][j][2], w[j][2], acc[m], false);
        acc[m] = __builtin_amdgcn_sdot4(a[m][j][3], w[j][3], acc[m], false);
      }
      acc[m] = wave_sum_i32(acc[m]);
    }
    if (lane == 0) {
#pragma unroll
      for (int m = 0; m < MR; ++m) red[wave][i][m] = acc[m];
    }
  };
  // two register sets in turn (no copies between them, so no wait on the newer loads)
  v4i w0[NC], w1[NC];
  load_row(w0, 0);
  for (int i = 0; i < rpw; i += 2) {
    if (i + 1 < rpw) load_row(w1, i + 1);
    __builtin_amdgcn_sched_barrier(0);
    row_sum(w0, i);
    __builtin_amdgcn_sched_barrier(0);
    if (i + 1 >= rpw) break;
    if (i + 2 < rpw) load_row(w0, i + 2);
    __builtin_amdgcn_sched_barrier(0);
    row_sum(w1, i + 1);
    __builtin_amdgcn_sched_barrier(0);
  }
  __syncthreads();
  // the K-slices of each row: one lane per (row of the row group)
  if (!owner) return;
  const int rl = r0 + lane;
  const int n = n0 + rl;
  const EpiCol ec = epi_col_of(ep, c0w, c1w);
#pragma unroll
  for (int m = 0; m < MR; ++m) {
    if (m < M) {
      int sum = 0;
      for (int k2 = 0; k2 < wk; ++k2) sum += red[rg * wk + k2][lane][m];
      epilogue_store_rc(ep, m, n, sum, epi_row_of(ep, rw_[m]), ec);
    }
  }
}

// The whole-row GEMV for one activation row with the contract's row quant fused in (the drop-in
// w8a8_matmul at M = 1: one launch instead of the row quant and the GEMV).  Every block quantises
// the row itself: thread t holds the 8-element chunks t, t + 256, ... of x in registers (x read
// once per block, from L2 after the first block), the block takes their maximum, derives asc =
// fl32(max(amax, 1e-8) / 127) and writes q = clamp(rint(x / asc)) to LDS with rowquant's arithmetic
// (quant_one), then streams its weight rows as gemv_i8_row_kernel does, its first weight row
// requested before x.  All blocks compute the same asc and q.  K % 16 == 0, K <= 512 NV WV; x 16-byte
// aligned.
template <int NC, int NV, int DT, int WV = 4, int PF = 2>
__global__ __launch_bounds__(WV * 64) void gemv_i8_rowq_kernel(const void* __restrict__ X, const int8_t* __restrict__ W,
                                                               int ldw, int N, int K, int wk, int rpw, EpiParams ep) {
  constexpr int kThr = WV * 64;
  __shared__ int red[WV][16];  // [wave][row of the wave], rpw <= 16
  __shared__ float bred[WV];
  __shared__ __attribute__((aligned(16))) int8_t qs[NV * kThr * 8];
  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
  const int rg = wave / wk, ks = wave % wk;
  const int rows_blk = rpw * (WV / wk);
  const int n0 = blockIdx.x * rows_blk;
  const int nrows = (N - n0) < rows_blk ? (N - n0) : rows_blk;
  const int kb = ks * NC * 1024;
  const int ke = (kb + NC * 1024) < K ? (kb + NC * 1024) : K;
  const __amdgpu_buffer_rsrc_t rw = lsk::make_rsrc(W + (int64_t)n0 * ldw, (int64_t)nrows * ldw);
  uint32_t koff[NC];
#pragma unroll
  for (int j = 0; j < NC; ++j) {
    const int kk = kb + j * 1024 + lane * 16;
    koff[j] = kk < ke ? (uint32_t)kk : lsk::kOob;
  }
  const int r0 = rg * rpw;
  auto load_row = [&](v4i* w, int i) {
    const int rl = r0 + i;
    const uint32_t rowoff = rl < nrows ? (uint32_t)(rl * ldw) : lsk::kOob;
#pragma unroll
    for (int j = 0; j < NC; ++j)
      w[j] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(
                                         rw, (rowoff == lsk::kOob || koff[j] == lsk::kOob) ? lsk::kOob : rowoff + koff[j],
                                         0, 2 /* non-temporal */));
  };
  // x first, then the first two weight rows: vector loads complete in issue order, so the wait
  // for x below leaves the weight rows in flight while x is quantised
  const int K8 = K >> 3;
  constexpr int kXW = DT == LSK_F32 ? 2 : 1;  // 16-byte loads per 8 elements
  uint4 xr[NV][kXW];
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int c = tid + j * kThr;
#pragma unroll
    for (int h = 0; h < kXW; ++h)
      xr[j][h] = c < K8 ? ((const uint4*)X)[(int64_t)c * kXW + h] : make_uint4(0, 0, 0, 0);
  }
  __builtin_amdgcn_sched_barrier(0);
  // the wave's first PF weight rows, all in flight while x is quantised
  v4i w[PF][NC];
#pragma unroll
  for (int p = 0; p < PF; ++p)
    if (p < rpw) load_row(w[p], p);
  __builtin_amdgcn_sched_barrier(0);
  // the column operands of the lane that stores row r0 + lane (used at the end)
  const bool owner = ks == 0 && lane < rpw && r0 + lane < nrows;
  const EpiRaw er_ = epi_raw(ep, 1, N);
  const uint32_t c0w = epi_raw_col0(er_, n0 + r0 + lane, owner), c1w = epi_raw_col1(er_, n0 + r0 + lane, owner);
  __builtin_amdgcn_sched_barrier(0);

  // the activation row: maximum, scale, quantised values into LDS
  float v[NV][8];
  float am = 0.0f;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    // (bf16 / f16: the first four words hold the eight elements)
    const uint32_t wd[8] = {xr[j][0].x, xr[j][0].y, xr[j][0].z, xr[j][0].w,
                            xr[j][kXW - 1].x, xr[j][kXW - 1].y, xr[j][kXW - 1].z, xr[j][kXW - 1].w};
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      if (DT == LSK_F32) v[j][e] = __uint_as_float(wd[e]);
      else if (DT == LSK_BF16) v[j][e] = bf16_to_f32((uint16_t)(wd[e >> 1] >> (16 * (e & 1))));
      else v[j][e] = (float)__builtin_bit_cast(_Float16, (uint16_t)(wd[e >> 1] >> (16 * (e & 1))));
      am = fmaxf(am, fabsf(v[j][e]));
    }
  }
  am = wave_fmax(am);
  if (lane == 0) bred[wave] = am;
  __syncthreads();
  am = bred[0];
#pragma unroll
  for (int w2 = 1; w2 < WV; ++w2) am = fmaxf(am, bred[w2]);
  am = fmaxf(am, kAmaxFloor);
  const float sc = f32_div(am, 127.0f), rs = f32_div(1.0f, sc);
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int c = tid + j * kThr;
    if (c < K8) {
      *(uint2*)(qs + 8 * c) = quant8_pack(v[j], sc, rs);
    }
  }
  __syncthreads();
  v4i a[NC];
#pragma unroll
  for (int j = 0; j < NC; ++j) a[j] = koff[j] != lsk::kOob ? *(const v4i*)(qs + koff[j]) : v4i{0, 0, 0, 0};

  auto row_sum = [&](const v4i* w, int i) {
    int acc = 0;
#pragma unroll
    for (int j = 0; j < NC; ++j) {
      acc = __builtin_amdgcn_sdot4(a[j][0], w[j][0], acc, false);
      acc = __builtin_amdgcn_sdot4(a[j][1], w[j][1], acc, false);
      acc = __builtin_amdgcn_sdot4(a[j][2], w[j][2], acc, false);
      acc = __builtin_amdgcn_sdot4(a[j][3], w[j][3], acc, false);
    }
    acc = wave_sum_i32(acc);
    if (lane == 0) red[wave][i] = acc;
  };
  // PF register sets in turn, each reloaded as soon as its row is summed
  for (int i = 0; i < rpw; i += PF) {
#pragma unroll
    for (int p = 0; p < PF; ++p) {
      if (i + p >= rpw) break;
      row_sum(w[p], i + p);
      __builtin_amdgcn_sched_barrier(0);
      if (i + p + PF < rpw) load_row(w[p], i + p + PF);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  __syncthreads();
  // the K-slices of each row: one lane per row of the row group
  if (!owner) return;
  const int rl = r0 + lane;
  const int n = n0 + rl;
  const EpiCol ec = epi_col_of(ep, c0w, c1w);
  int sum = 0;
  for (int k2 = 0; k2 < wk; ++k2) sum += red[rg * wk + k2][lane];
  epilogue_store_rc(ep, 0, n, sum, EpiRow{sc, 0}, ec);
}

// Correctness path for shapes the tiled kernels do not take (odd K, unaligned rows).
__global__ __launch_bounds__(256) void gemm_i8_generic_kernel(const int8_t* __restrict__ A, int64_t lda,
                                                              const int8_t* __restrict__ W, int64_t ldw, int64_t M,
                                                              int64_t N, int64_t K, EpiParams ep) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= M * N) return;
  const int64_t m = idx / N, n = idx - m * N;
  const int8_t* a = A + m * lda;
  const int8_t* w = W + n * ldw;
  int32_t s = 0;
  for (int64_t k = 0; k < K; ++k) s += (int32_t)a[k] * (int32_t)w[k];
  epilogue_store(ep, m, n, s);
}

// The epilogue alone over an existing int32 accumulator (the reference's separate
// lin_epilogue / lin_epilogue_b calls on the result of int_mm).
__global__ __launch_bounds__(256) void epilogue_apply_kernel(const int32_t* __restrict__ acc, int64_t ldc,
                                                             int64_t M, int64_t N, EpiParams ep) {
  const int64_t total = M * N;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
    const int64_t m = i / N, n = i - m * N;
    epilogue_store(ep, m, n, acc[m * ldc + n]);
  }
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

}  // namespace

namespace lsk {

// Shape checks shared by the dense and grouped entry points.
int validate_epilogue(int order, int out_dtype, const float* asc, const float* ws, int64_t M, const char* who) {
  LSK_REQUIRE(order >= LSK_EPI_V21 && order <= LSK_EPI_V25, "%s: unknown epilogue order %d", who, order);
  if (order == LSK_EPI_RAW) {
    LSK_REQUIRE(out_dtype == LSK_I32, "%s: the RAW epilogue writes int32 (out_dtype %d)", who, out_dtype);
  } else if (order == LSK_EPI_POW2) {
    LSK_REQUIRE(out_dtype == LSK_F32, "%s: the POW2 epilogue writes binary32 (out_dtype %d)", who, out_dtype);
  } else {
    LSK_REQUIRE(out_dtype == LSK_F32 || out_dtype == LSK_BF16 || out_dtype == LSK_F16 || out_dtype == LSK_BF16_AS_F32,
                "%s: out_dtype %d not one of f32/bf16/f16/bf16-as-f32", who, out_dtype);
    LSK_REQUIRE(M == 0 || (asc && ws), "%s: asc and ws are required by the V21/V2/V25 epilogues", who);
  }
  return LSK_OK;
}

// Tile configurations of the dense kernel; id -1 lets the shape decide.
thread_local int g_force_tile = -1;
thread_local int g_row_rpw = 0;       // rows per wave of the whole-row GEMV (0: by shape)
thread_local int g_rowq = 1;          // w8a8_matmul at M = 1: the row quant fused into the whole-row GEMV
thread_local int g_gemv_variant = 0;  // M <= 4: 0 whole-row GEMV, 1 register double-buffered 8-row GEMV, 2 LDS-ring 8-row GEMV
thread_local int g_gemv_mid = 0;      // M <= 32: 0 by shape, 1 direct 64-byte row pieces, 2 whole rows through LDS, 3 A staged in LDS (skinny)
// the skinny GEMV's launch shape: groups per block, waves per group, weight steps in flight (0: by shape)
thread_local int g_skinny_gpb = 0, g_skinny_kw = 0, g_skinny_d = 0;

// the persistent POW2 kernel: 1 on (one block per CU), 0 off, > 1 that many blocks (tests)
thread_local int g_pp_persist = 1;

// Compute units of the current device (the persistent kernels' grid), cached per device.
static int cu_count() {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
  int n = cache[dev].load(std::memory_order_relaxed);
  if (n <= 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cache[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

template <int BM, int BN, int WM, int WN>
static int launch_tile(const int8_t* a, int lda, const int8_t* w, int ldw, int M, int N, int K,
                       const EpiParams& ep, int vec_ok, hipStream_t s, const char* name) {
  using C = TileCfg<BM, BN, WM, WN>;
  static std::atomic<bool> attr_set{false};
  auto kern = gemm_i8_mfma_kernel<BM, BN, WM, WN>;
  if (!attr_set) {
    if (hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, C::kSmemBytes) !=
        hipSuccess) {
      set_error("%s: cannot reserve %d bytes of LDS", name, C::kSmemBytes);
      return LSK_ERR_HIP;
    }
    attr_set = true;
  }
  const int64_t tiles = (int64_t)((M + BM - 1) / BM) * ((N + BN - 1) / BN);
  LSK_REQUIRE(tiles <= 0x7fffffff, "gemm: too many tiles");
  hipLaunchKernelGGL(kern, dim3((unsigned)tiles), dim3(C::kThreads), C::kSmemBytes, s, a, lda, w, ldw, M, N, K, ep,
                     vec_ok);
  return check_launch(name);
}

template <int BM, int BN, int WM, int WN, int RING = 4, int BKB = 64>
static int launch_pp(const int8_t* a, int lda, const int8_t* w, int ldw, int M, int N, int K, const EpiParams& ep,
                     int vec_ok, hipStream_t s, const char* name) {
  using C = PPCfg<BM, BN, WM, WN, RING, BKB>;
  static std::atomic<bool> attr_set{false};
  auto kern = gemm_i8_pp_kernel<BM, BN, WM, WN, RING, BKB>;
  if (!attr_set) {
    if (hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, C::kSmemBytes) !=
        hipSuccess) {
      set_error("%s: cannot reserve %d bytes of LDS", name, C::kSmemBytes);
      return LSK_ERR_HIP;
    }
    attr_set = true;
  }
  const int64_t tiles = (int64_t)((M + BM - 1) / BM) * ((N + BN - 1) / BN);
  LSK_REQUIRE(tiles <= 0x7fffffff, "gemm: too many tiles");
  // 2: vector stores allowed and a whole tile's output span addressable by 32-bit offsets
  // (the kernel's fast epilogue)
  const int64_t esz = (ep.out_dtype == LSK_BF16 || ep.out_dtype == LSK_F16) ? 2 : 4;
  const int vflag = (vec_ok && (int64_t)(BM - 1) * ep.ldo * esz + BN * esz < 0x7fffffff) ? 2 : vec_ok;
  if constexpr (BM == 256 && BN == 256 && WM == 4 && WN == 2 && RING == 4 && BKB == 64) {
    // whole tiles under POW2 with binary32 out: the persistent kernel, one block per CU
    if (g_pp_persist != 0 && ep.order == LSK_EPI_POW2 && ep.ecol == nullptr && ep.out_dtype == LSK_F32 &&
        vflag == 2 && M % BM == 0 && N % BN == 0 && K % BKB == 0 && K / BKB >= C::kRing + 2) {
      auto pk = gemm_i8_pp_pow2_persist_kernel<BM, BN, WM, WN, RING, BKB>;
      static std::atomic<bool> pattr{false};
      if (!pattr) {
        if (hipFuncSetAttribute((const void*)pk, hipFuncAttributeMaxDynamicSharedMemorySize, C::kSmemBytes) !=
            hipSuccess) {
          set_error("%s: cannot reserve %d bytes of LDS", name, C::kSmemBytes);
          return LSK_ERR_HIP;
        }
        pattr = true;
      }
      int64_t grid = g_pp_persist > 1 ? g_pp_persist : cu_count();
      grid = grid < tiles ? grid : tiles;
      hipLaunchKernelGGL(pk, dim3((unsigned)grid), dim3(C::kThreads), C::kSmemBytes, s, a, lda, w, ldw, M, N, K, ep);
      return check_launch(name);
    }
  }
  hipLaunchKernelGGL(kern, dim3((unsigned)tiles), dim3(C::kThreads), C::kSmemBytes, s, a, lda, w, ldw, M, N, K, ep,
                     vflag);
  return check_launch(name);
}

template <int BM, int BN, int RING = 4>
static int launch_w4(const int8_t* a, int lda, const int8_t* w, int ldw, int M, int N, int K, const EpiParams& ep,
                     int vec_ok, hipStream_t s, const char* name) {
  using C = W4Cfg<BM, BN, RING>;
  static std::atomic<bool> attr_set{false};
  auto kern = gemm_i8_w4_kernel<BM, BN, RING>;
  if (!attr_set) {
    if (hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, C::kSmemBytes) !=
        hipSuccess) {
      set_error("%s: cannot reserve %d bytes of LDS", name, C::kSmemBytes);
      return LSK_ERR_HIP;
    }
    attr_set = true;
  }
  const int64_t tiles = (int64_t)((M + BM - 1) / BM) * ((N + BN - 1) / BN);
  LSK_REQUIRE(tiles <= 0x7fffffff, "gemm: too many tiles");
  const int64_t esz = (ep.out_dtype == LSK_BF16 || ep.out_dtype == LSK_F16) ? 2 : 4;
  const int vflag = (vec_ok && (int64_t)(BM - 1) * ep.ldo * esz + BN * esz < 0x7fffffff) ? 2 : vec_ok;
  hipLaunchKernelGGL(kern, dim3((unsigned)tiles), dim3(C::kThreads), C::kSmemBytes, s, a, lda, w, ldw, M, N, K, ep,
                     vflag);
  return check_launch(name);
}

static int pick_tile(int64_t M, int64_t N) {
  if (g_force_tile >= 0) return g_force_tile;
  if (M <= 128) return 0;  // few rows: the 128x128 register-staged tile wastes least
  // Ping-pong tiles: whole rounds of 256 blocks (one per CU) are what a launch costs.  A
  // 256x128 tile takes 0.68 of a 256x256 tile's time (measured on MI355X at the Llama-3.1-8B /
  // Qwen2.5-7B prefill shapes), so pick the shape with the smaller rounds x tile cost.  The
  // 256x128 tile stages K 128 bytes at a time (three stages, 144 KB): half the barriers per MFMA
  // of 64-byte stages, 15% faster on the Llama-3.1-8B down projection.
  const int64_t r256 = ((M + 255) / 256 * ((N + 255) / 256) + 255) / 256;
  const int64_t r128 = ((M + 255) / 256 * ((N + 127) / 128) + 255) / 256;
  return (double)r128 * 0.68 < (double)r256 ? 18 : 1;
}

// Columns to cover with whole rounds of 256x256 tiles before finishing with 256x128 tiles, or 0
// when one tile shape is cheaper: a launch of 256x256 tiles that ends in a partial round of 256
// blocks leaves CUs idle through that round; splitting the columns so the 256x256 part fills
// whole rounds and the rest takes 256x128 tiles (0.68 of a 256x256 tile's time) costs
// rounds1 + 0.68 * rounds2 instead.
static int64_t split_columns(int64_t M, int64_t N) {
  if (M <= 128) return 0;
  const int64_t mt = (M + 255) / 256;
  const int64_t t256 = mt * ((N + 255) / 256);
  const int64_t full = t256 / 256;
  if (full == 0 || t256 % 256 == 0) return 0;
  const int64_t nt1 = full * 256 / mt;  // 256-column tiles the whole rounds cover
  const int64_t n1 = nt1 * 256;
  if (n1 <= 0 || n1 >= N) return 0;
  const int64_t r1 = (nt1 * mt + 255) / 256;
  const int64_t r2 = (mt * ((N - n1 + 127) / 128) + 255) / 256;
  const int64_t r256 = (t256 + 255) / 256;
  const int64_t r128 = (mt * ((N + 127) / 128) + 255) / 256;
  const double best_one = (double)r128 * 0.68 < (double)r256 ? (double)r128 * 0.68 : (double)r256;
  return ((double)r1 + 0.68 * (double)r2 < best_one) ? n1 : 0;
}

// The epilogue parameters of the output columns from n1 on.
static EpiParams shift_columns(const EpiParams& ep, int64_t n1) {
  EpiParams e = ep;
  const int esz = (ep.out_dtype == LSK_BF16 || ep.out_dtype == LSK_F16) ? 2 : 4;
  e.out = (char*)ep.out + n1 * esz;
  if (e.ws) e.ws += n1;
  if (e.bias) e.bias += n1;
  if (e.ecol) e.ecol += n1;
  if (e.wo) e.wo = (const char*)e.wo + n1 * e.ko * (e.wo_dtype == LSK_BF16 ? 2 : 4);
  return e;
}

// Launch shape of gemv_i8_skinny_kernel: A (M rows of ceil(K / 1024) KB + 16 bytes) must fit in
// LDS.  Groups of 16 weight rows are dealt to one block per CU (one round of blocks covers them),
// then each group's K steps are split over waves up to 16 waves per block.  (Measured on MI355X,
// Llama-3.1-8B gate_up, graph replays over weight copies, us for gpb x kw at M = 8 / 32: 7 x 2
// 25.9 / 30.4, 4 x 2 (two blocks per CU) 27.5 / 35.4, 8 x 2 27.5 / 32.5, 8 x 1 29.6 / 31.8, 4 x 4
// 28.2 / 36.8.)
struct SkinnyShape {
  int gpb, kw, sps, ldsk, blocks, D;
  size_t smem;
};

static bool skinny_shape(int M, int N, int K, SkinnyShape& sh) {
  if (M < 1 || M > 32 || N < 1 || K < 16) return false;
  const int steps = (K + 63) / 64, MT = M <= 16 ? 1 : 2;
  sh.ldsk = (K + 1023) / 1024 * 1024 + 16;
  const int64_t lds_a = (int64_t)M * sh.ldsk;
  if (lds_a > 160 * 1024) return false;
  const int64_t G = (N + 15) / 16;
  int64_t gpb = std::min<int64_t>(16, std::max<int64_t>(1, (G + 255) / 256));
  if (g_skinny_gpb > 0) gpb = g_skinny_gpb;
  const int64_t blocks = (G + gpb - 1) / gpb;
  int64_t kw = std::max<int64_t>(1, 16 / gpb);
  if (g_skinny_kw > 0 && g_skinny_kw * gpb <= 16) kw = g_skinny_kw;
  const int64_t sps = (steps + kw - 1) / kw;
  kw = (steps + sps - 1) / sps;
  sh.gpb = (int)gpb;
  sh.kw = (int)kw;
  sh.sps = (int)sps;
  sh.blocks = (int)blocks;
  sh.D = g_skinny_d > 0 ? g_skinny_d : (sps <= 4 ? 4 : 8);
  sh.smem = (size_t)std::max<int64_t>(lds_a, gpb * kw * MT * 1024);
  return blocks <= 0x7fffffff && sh.smem <= 160 * 1024;
}

// Whether launch_gemv runs (M, N, K) on gemv_i8_skinny_kernel under the calling thread's
// selection: by shape for 4 < M <= 32 and N >= 8192 wherever A fits in LDS, or for any M <= 32
// when selected.  (Measured on MI355X, graph replays over weight copies, the GEMV alone: Llama-3.1-8B
// gate_up M = 8 / 16 / 32 29.1 / 32.1 / 47.5 -> 25.9 / 28.3 / 30.4 us.  With N <= 4096 a block
// holds one group of weight rows, A is staged once per 16 weight rows, and the GEMVs that stream
// whole rows through LDS stay ahead: down M = 8 14.5 against 16.2 us, the Qwen2.5-7B o_proj at
// M = 16 6.9 against 7.3 us.)
bool gemv_takes_skinny(int64_t M, int64_t N, int64_t K) {
  SkinnyShape sh;
  if (M > 32 || !skinny_shape((int)M, (int)std::min<int64_t>(N, 0x7fffffff), (int)K, sh)) return false;
  return g_gemv_mid == 3 || (g_gemv_mid == 0 && g_gemv_variant == 0 && M > 4 && N >= 8192);
}

static int launch_skinny(const int8_t* a, int lda, const int8_t* w, int ldw, int M, int N, int K, const EpiParams& ep,
                         hipStream_t s) {
  SkinnyShape sh;
  if (!skinny_shape(M, N, K, sh)) return set_error("gemv: M=%d K=%d does not fit the skinny GEMV", M, K), LSK_ERR_ARG;
  const bool pairs = (ep.pairs & 2) != 0;
#define LSK_SK(MTV, DV, PV)                                                                                    \
  {                                                                                                            \
    auto kern = gemv_i8_skinny_kernel<MTV, DV, PV>;                                                            \
    if (sh.smem > 65536 &&                                                                                     \
        hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024) != hipSuccess) \
      return set_error("gemv: cannot reserve LDS"), LSK_ERR_HIP;                                               \
    hipLaunchKernelGGL(kern, dim3((unsigned)sh.blocks), dim3(64 * sh.gpb * sh.kw), sh.smem, s, a, lda, w, ldw, M, N, \
                       K, sh.gpb, sh.kw, sh.sps, sh.ldsk, ep);                                                 \
    return check_launch("gemv_i8_skinny_kernel");                                                              \
  }
#define LSK_SK_D(MTV, PV) \
  if (sh.D == 4) LSK_SK(MTV, 4, PV) else LSK_SK(MTV, 8, PV)
  if (M <= 16) {
    if (pairs) LSK_SK_D(1, true) else LSK_SK_D(1, false)
  } else {
    if (pairs) LSK_SK_D(2, true) else LSK_SK_D(2, false)
  }
#undef LSK_SK_D
#undef LSK_SK
}

// Waves per block of the decode GEMV: enough blocks x waves (about 8192) to keep every CU's
// memory pipeline full, K split into 64-byte-aligned slices.
static int launch_gemv(const int8_t* a, int lda, const int8_t* w, int ldw, int M, int N, int K, const EpiParams& ep,
                       hipStream_t s) {
  if ((ep.pairs & 2) || gemv_takes_skinny(M, N, K)) return launch_skinny(a, lda, w, ldw, M, N, K, ep, s);
  const int64_t Kp = (K + 127) / 128 * 128;
  if (M <= 4 && g_gemv_variant == 0 && K <= 4 * 8 * 1024) {
    // whole-row streaming: K-slices of NC <= 8 chunks (WK <= 4 waves per row).  (With 8 or 16
    // activation rows the VALU dot products outweigh the better stream: Llama-3.1-8B gate_up
    // M = 8 37.8 us against 28.8 on the MFMA GEMV, M = 16 96.7 against 32.3.)
    const int nch = (K + 1023) / 1024;
    int wk = 1;
    while (wk < 4 && (nch + wk - 1) / wk > 4) wk *= 2;
    const int nc = (nch + wk - 1) / wk;
    // rows per wave (measured on MI355X, Llama-3.1-8B decode shapes): one row per wave streams
    // best for a single activation row; more activation rows amortise their registers over
    // more weight rows.  Fewer when N leaves under about 2048 waves.
    const int mr = M <= 1 ? 1 : (M <= 2 ? 2 : 4);
    int rpw = mr == 1 ? (wk == 1 ? 1 : 2) : (mr == 2 ? 4 : 8);
    while (rpw > 1 && (int64_t)((N + rpw * (4 / wk) - 1) / (rpw * (4 / wk))) * 4 < 2048) rpw /= 2;
    if (g_row_rpw > 0) rpw = g_row_rpw;
    const int rows_blk = rpw * (4 / wk);
    const int rblocks = (N + rows_blk - 1) / rows_blk;
#define LSK_ROW(MRV, NCV)                                                                                  \
  {                                                                                                        \
    hipLaunchKernelGGL((gemv_i8_row_kernel<MRV, NCV>), dim3((unsigned)rblocks), dim3(256), 0, s, a, lda, w, ldw, M, N, \
                       K, wk, rpw, ep);                                                                    \
    return check_launch("gemv_i8_row_kernel");                                                             \
  }
#define LSK_ROW_NC(MRV) \
  if (nc <= 1) LSK_ROW(MRV, 1) else if (nc <= 2) LSK_ROW(MRV, 2) else if (nc <= 4) LSK_ROW(MRV, 4) else LSK_ROW(MRV, 8)
    if (mr == 1) LSK_ROW_NC(1) else if (mr == 2) LSK_ROW_NC(2) else LSK_ROW_NC(4)
#undef LSK_ROW_NC
#undef LSK_ROW
  }
  if (M <= 4 && 4 * Kp <= 65536) {
    // WK waves per 8-row group so that about 2048 waves stream the weights
    int wk = 1;
    while (wk < 4 && (int64_t)((N + 8 * (4 / wk) - 1) / (8 * (4 / wk))) * 4 < 2048) wk *= 2;
    const int rows_blk = 8 * (4 / wk);
    const int dblocks = (N + rows_blk - 1) / rows_blk;
    const int kslice = (int)(((K + wk - 1) / wk + 127) / 128 * 128);
    const int mr = M <= 1 ? 1 : (M <= 2 ? 2 : 4);
    if (g_gemv_variant == 1) {
      const size_t smem = (size_t)mr * Kp + 4 * 8 * mr * sizeof(int);
      if (mr == 1)
        hipLaunchKernelGGL((gemv_i8_dot_kernel<1, 8>), dim3((unsigned)dblocks), dim3(256), smem, s, a, lda, w, ldw, M,
                           N, K, wk, kslice, ep);
      else if (mr == 2)
        hipLaunchKernelGGL((gemv_i8_dot_kernel<2, 8>), dim3((unsigned)dblocks), dim3(256), smem, s, a, lda, w, ldw, M,
                           N, K, wk, kslice, ep);
      else
        hipLaunchKernelGGL((gemv_i8_dot_kernel<4, 8>), dim3((unsigned)dblocks), dim3(256), smem, s, a, lda, w, ldw, M,
                           N, K, wk, kslice, ep);
      return check_launch("gemv_i8_dot_kernel");
    }
    // ring: batches of 4 steps, 3 or 2 batches deep as the LDS share of the blocks one CU
    // must hold allows
    const int64_t per_cu = (dblocks + 255) / 256;
    const int64_t budget = (160 * 1024) / (per_cu < 1 ? 1 : per_cu) - mr * Kp - 4 * 8 * mr * 4;
    const int R = budget >= 4 * 12 * 1024 ? 3 : 2;
    const size_t smem = (size_t)mr * Kp + (size_t)4 * 4 * R * 1024 + 4 * 8 * mr * sizeof(int);
    if (smem > 160 * 1024) return set_error("gemv: %zu bytes of LDS exceed the 160 KB limit", smem), LSK_ERR_ARG;
#define LSK_RING(MRV, RV)                                                                                         \
  {                                                                                                               \
    auto kern = gemv_i8_ring_kernel<MRV, 4, RV>;                                                                  \
    if (smem > 65536 &&                                                                                           \
        hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024) != hipSuccess) \
      return set_error("gemv: cannot reserve LDS"), LSK_ERR_HIP;                                                  \
    hipLaunchKernelGGL(kern, dim3((unsigned)dblocks), dim3(256), smem, s, a, lda, w, ldw, M, N, K, wk, kslice, ep); \
    return check_launch("gemv_i8_ring_kernel");                                                                   \
  }
    if (mr == 1) {
      if (R == 3) LSK_RING(1, 3) else LSK_RING(1, 2)
    } else if (mr == 2) {
      if (R == 3) LSK_RING(2, 3) else LSK_RING(2, 2)
    } else {
      if (R == 3) LSK_RING(4, 3) else LSK_RING(4, 2)
    }
#undef LSK_RING
  }
  const int blocks = (N + 15) / 16;
  // whole-row streaming through LDS wins over 64-byte row pieces for one activation tile (M <= 16)
  // except where N leaves just over one round of 256 blocks or is very wide (measured on MI355X,
  // graph replays over weight copies, us LDS / pieces: K = 3584 and N = 2048 .. 4096 at M = 8 / 16
  // 5.9-7.0 / 7.1-7.9; N = 4608 10.8 / 10.4 and 11.9 / 11.4; N = 3584, K = 2048 / 5120 5.1-5.4 /
  // 5.6-6.0 and 7.4-8.2 / 9.8-10.4; N = 14336, K = 4096 17.6 / 20.3 and 19.9 / 22.7; N = 28672,
  // K = 4096 level at M = 8 (the whole w8a8_matmul call 33.3 / 32.2), 34.2 / 32.9 at M = 16;
  // K = 14336 14.5 / 17.0 and 16.4 / 19.5; two activation tiles (M > 16) about 2x slower)
  // (one activation tile only: the two-tile form spilled registers and measured about 2x slower)
  const bool use_lds = M <= 16 && (g_gemv_mid == 2 ||
                                   (g_gemv_mid == 0 && (K >= 8192 || N <= 4096 || (N >= 8192 && N <= 16384))));
  if (use_lds) {
    // waves per block so that at least 1024 waves stream, each K-slice a whole number of
    // 512-byte stages
    constexpr int SB = 512, R = 3;
    const int nstg = (K + SB - 1) / SB;
    int nw = 1;  // up to four waves per block (96 KB of rings): at least 1024 waves stream
    while (nw < 4 && (int64_t)blocks * nw < 1024 && nstg >= 2 * nw) nw *= 2;
    const int kslice = ((nstg + nw - 1) / nw) * SB;
    const size_t smem = (size_t)nw * R * 16 * SB;
    if (smem > 160 * 1024) return set_error("gemv: %zu bytes of LDS exceed the 160 KB limit", smem), LSK_ERR_ARG;
#define LSK_LDS(MTV)                                                                                          \
  {                                                                                                           \
    auto kern = gemv_i8_lds_kernel<MTV, SB, R>;                                                               \
    if (smem > 65536 &&                                                                                       \
        hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024) != hipSuccess) \
      return set_error("gemv: cannot reserve LDS"), LSK_ERR_HIP;                                              \
    hipLaunchKernelGGL(kern, dim3((unsigned)blocks), dim3(64 * nw), smem, s, a, lda, w, ldw, M, N, K, kslice, ep); \
    return check_launch("gemv_i8_lds_kernel");                                                                \
  }
    LSK_LDS(1)
#undef LSK_LDS
  }
  int kw = 1;
  while (kw < 16 && (int64_t)blocks * kw < 2048 && (int64_t)(kw * 2) * 64 * 4 * 2 <= K) kw *= 2;
  const int kslice = ((K + kw * 64 - 1) / (kw * 64)) * 64;
  const size_t smem = (size_t)(kw - 1) * (M <= 16 ? 1 : 2) * 64 * sizeof(v4i);
  if (M <= 16)
    hipLaunchKernelGGL((gemv_i8_stream_kernel<1, 4>), dim3((unsigned)blocks), dim3(64 * kw), smem, s, a, lda, w, ldw, M,
                       N, K, kslice, ep);
  else
    hipLaunchKernelGGL((gemv_i8_stream_kernel<2, 4>), dim3((unsigned)blocks), dim3(64 * kw), smem, s, a, lda, w, ldw, M,
                       N, K, kslice, ep);
  return check_launch("gemv_i8_stream_kernel");
}

// Whether lsk_w8a8_matmul takes the fused row-quant GEMV for one activation row: the decode GEMV
// would run (no forced tile other than the GEMV, the whole-row variant), K % 16 == 0 and
// K <= 16384, x and w 16-byte aligned, the v2.1 or v2 order.  (Every block reads x, so long rows
// take 16-wave blocks that serve 16 weight rows per read of x: on MI355X, graph replays over weight
// copies, Llama-3.1-8B gate_up M = 1 (K = 4096) 21.2 us fused against 22.1 us as two launches; the
// down projection (K = 14336, 57 KB of x per block) 13.5 us against 16.0 us; with four-wave blocks
// it measured 16.0 us.)
bool rowq_gemv_ok(const void* x, const int8_t* w, int64_t ldw, int64_t M, int64_t N, int64_t K, int order) {
  return g_rowq && M == 1 && N >= 1 && N < (1 << 29) && K >= 16 && K <= 16384 && K % 16 == 0 && ldw % 16 == 0 &&
         aligned16(x) && aligned16(w) && (g_force_tile < 0 || g_force_tile == 5) && g_gemv_variant == 0 &&
         g_gemv_mid != 3 &&
         (order == LSK_EPI_V21 || order == LSK_EPI_V2) && ldw * 64 < 0x7fffffff;
}

int launch_gemv_rowq(const void* x, int x_dtype, const int8_t* w, int ldw, int N, int K, const EpiParams& ep,
                     hipStream_t s) {
  if (K > 4096) {
    // long rows: 16-wave blocks (four K-slices of up to 4 KB per row, RPW rows per wave) so that
    // each block's read of x serves 4 RPW weight rows and about 256 blocks cover N.  (Llama-3.1-8B
    // down, M = 1, graph replays: 16.0 us as two launches -> 13.5 us; RPW 1 / 2 / 4 / 8: 22.0 / 17.2
    // / 13.5 / 16.1 us.  Up to K = 4096 the four-wave blocks measured level with this form.  All four
    // rows of a wave in flight before the quant, PF = 4: 14.5 against 13.4 us.)
    const int wk = 4;
    int rpw = (N * wk / 16 + 255) / 256;
    rpw = rpw < 1 ? 1 : (rpw > 16 ? 16 : rpw);
    if (g_row_rpw > 0) rpw = g_row_rpw;
    const int rows_blk = rpw * (16 / wk);
    const int blocks = (N + rows_blk - 1) / rows_blk;
#define LSK_RQL(DTV)                                                                                       \
  {                                                                                                        \
    hipLaunchKernelGGL((gemv_i8_rowq_kernel<4, 2, DTV, 16, 2>), dim3((unsigned)blocks), dim3(1024), 0, s, x, w, ldw, N, \
                       K, wk, rpw, ep);                                                                    \
    return check_launch("gemv_i8_rowq_kernel");                                                            \
  }
    if (x_dtype == LSK_F32) LSK_RQL(LSK_F32) else if (x_dtype == LSK_BF16) LSK_RQL(LSK_BF16) else LSK_RQL(LSK_F16)
#undef LSK_RQL
  }
  const int nch = (K + 1023) / 1024;
  int wk = 1;
  while (wk < 4 && (nch + wk - 1) / wk > 4) wk *= 2;
  const int nc = (nch + wk - 1) / wk;
  // rows per wave: each block reads x once, so more than one row per wave amortises it (two
  // measured best: 21.2 us at gate_up M = 1 against 26.9 / 23.0 / 23.5 us at 1 / 4 / 8); fewer
  // when N leaves under about 2048 waves
  int rpw = 2;
  while (rpw > 1 && (int64_t)((N + rpw * (4 / wk) - 1) / (rpw * (4 / wk))) * 4 < 2048) rpw /= 2;
  if (g_row_rpw > 0) rpw = g_row_rpw;
  const int rows_blk = rpw * (4 / wk);
  const int blocks = (N + rows_blk - 1) / rows_blk;
#define LSK_RQ(NCV, NVV, DTV)                                                                              \
  {                                                                                                        \
    hipLaunchKernelGGL((gemv_i8_rowq_kernel<NCV, NVV, DTV>), dim3((unsigned)blocks), dim3(256), 0, s, x, w, ldw, N, K, \
                       wk, rpw, ep);                                                                       \
    return check_launch("gemv_i8_rowq_kernel");                                                            \
  }
#define LSK_RQ_DT(NCV, NVV) \
  if (x_dtype == LSK_F32) LSK_RQ(NCV, NVV, LSK_F32) else if (x_dtype == LSK_BF16) LSK_RQ(NCV, NVV, LSK_BF16) else LSK_RQ(NCV, NVV, LSK_F16)
  if (nc <= 1) LSK_RQ_DT(1, 2)
  if (nc <= 2) LSK_RQ_DT(2, 2)
  LSK_RQ_DT(4, 2)
#undef LSK_RQ_DT
#undef LSK_RQ
}

static bool tiles_fast(const int8_t* a, int64_t lda, const int8_t* w, int64_t ldw, int64_t M, int64_t N, int64_t K) {
  // the tile kernels address rows by 32-bit offsets inside a 256-row tile
  return (K % 16 == 0) && (lda % 16 == 0) && (ldw % 16 == 0) && aligned16(a) && aligned16(w) && M <= 0x7fffffff &&
         N <= 0x7fffffff && K > 0 && lda * 256 < 0x7fffffff && ldw * 256 < 0x7fffffff;
}

// Whether launch_gemm runs (M, N, K) on the decode GEMV that reads the weight's row-pair copy
// (gemv_i8_skinny_kernel), for a weight of row stride ldw at a 16-byte aligned address.
bool gemm_takes_skinny(const int8_t* w, int64_t ldw, int64_t M, int64_t N, int64_t K, int64_t lda) {
  if (M <= 0 || M > 32 || N <= 0 || !epi_raw_fits(M, N) || !tiles_fast(w, lda, w, ldw, M, N, K)) return false;
  return (g_force_tile < 0 || g_force_tile == 5) && gemv_takes_skinny(M, N, K);
}

// Whether launch_gemm runs (M, N, K) on the ping-pong tile kernels only (the kernels that read an
// A operand in the row-pair layout), for an A of row stride lda at a 16-byte aligned address.
bool gemm_takes_pp(const int8_t* w, int64_t ldw, int64_t M, int64_t N, int64_t K, int64_t lda) {
  if (M <= 0 || N <= 0 || !tiles_fast(w, lda, w, ldw, M, N, K)) return false;  // (A aligned: the caller)
  if (M <= 32 && (g_force_tile < 0 || g_force_tile == 5)) return false;
  if (g_force_tile < 0 && split_columns(M, N) > 0) return true;
  const int t = pick_tile(M, N);
  return t == 1 || t == 2 || t == 3 || t == 4 || t == 12 || t == 13 || t == 18;
}

int launch_gemm(const int8_t* a, int64_t lda, const int8_t* w, int64_t ldw, int64_t M, int64_t N, int64_t K,
                const EpiParams& ep, hipStream_t s) {
  if (M == 0 || N == 0) return LSK_OK;
  LSK_REQUIRE(!ep.pairs || (ep.pairs == 2 && ldw % 64 == 0 && gemm_takes_skinny(w, ldw, M, N, K, lda)) ||
                  (aligned16(a) && gemm_takes_pp(w, ldw, M, N, K, lda) && (!(ep.pairs & 1) || lda % 64 == 0) &&
                   (!(ep.pairs & 2) || ldw % 64 == 0)),
              "gemm: operands in the row-pair layout need the ping-pong tiles or the skinny decode GEMV (M=%lld "
              "N=%lld K=%lld lda=%lld ldw=%lld)",
              (long long)M, (long long)N, (long long)K, (long long)lda, (long long)ldw);
  const bool fast = tiles_fast(a, lda, w, ldw, M, N, K);
  if (!fast) {
    const int64_t total = M * N;
    const int64_t blocks = (total + 255) / 256;
    LSK_REQUIRE(blocks <= 0x7fffffff, "gemm: M*N=%lld too large for the generic path", (long long)total);
    hipLaunchKernelGGL(gemm_i8_generic_kernel, dim3((unsigned)blocks), dim3(256), 0, s, a, lda, w, ldw, M, N, K, ep);
    return check_launch("gemm_i8_generic_kernel");
  }
  const int iM = (int)M, iN = (int)N, iK = (int)K;
  if (M <= 32 && (g_force_tile < 0 || g_force_tile == 5)) {
    if (!epi_raw_fits(M, N)) {  // (the GEMVs address their epilogue operands by 32-bit offsets)
      hipLaunchKernelGGL(gemm_i8_generic_kernel, dim3((unsigned)((M * N + 255) / 256)), dim3(256), 0, s, a, lda, w,
                         ldw, M, N, K, ep);
      return check_launch("gemm_i8_generic_kernel");
    }
    return launch_gemv(a, (int)lda, w, (int)ldw, iM, iN, iK, ep, s);
  }
  const int vec_ok = out_vec_ok(ep.out, ep.out_dtype, ep.ldo) ? 1 : 0;
  const int ilda = (int)lda, ildw = (int)ldw;
  int64_t n1 = 0;
  if (g_force_tile < 0 && (n1 = split_columns(M, N)) > 0) {
    // whole rounds of 256x256 tiles over the first n1 columns, the rest in 256x128 tiles
    int rc = launch_pp<256, 256, 4, 2>(a, ilda, w, ildw, iM, (int)n1, iK, ep, vec_ok, s, "gemm_i8_pp<256x256,4x2>");
    if (rc) return rc;
    const EpiParams ep2 = shift_columns(ep, n1);
    return launch_pp<256, 128, 4, 2, 3, 128>(a, ilda, w + n1 * ldw, ildw, iM, (int)(N - n1), iK, ep2,
                                             out_vec_ok(ep2.out, ep2.out_dtype, ep2.ldo) ? 1 : 0, s,
                                             "gemm_i8_pp<256x128,4x2,r3,k128>");
  }
  switch (pick_tile(M, N)) {
    case 1: return launch_pp<256, 256, 4, 2>(a, ilda, w, ildw, iM, iN, iK, ep, vec_ok, s, "gemm_i8_pp<256x256,4x2>");
    case 2: return launch_pp<256, 256, 2, 4>(a, ilda, w, ildw, iM, iN, iK, ep, vec_ok, s, "gemm_i8_pp<256x256,2x4>");
    case 3: return launch_pp<256, 128, 4, 2>(a, ilda, w, ildw, iM, iN, iK, ep, vec_ok, s, "gemm_i8_pp<256x128,4x2>");
    case 4: return launch_pp<128, 256, 2, 4>(a, ilda, w, ildw, iM, iN, iK, ep, vec_ok, s, "gemm_i8_pp<128x256,2x4>");
    case 12: return launch_pp<256, 128, 4, 2, 3>(a, ilda, w, ildw, iM, iN, iK, ep, vec_ok, s, "gemm_i8_pp<256x128,4x2,r3>");
    case 13: return launch_pp<128, 256, 2, 4, 3>(a, ilda, w, ildw, iM, iN, iK, ep, vec_ok, s, "gemm_i8_pp<128x256,2x4,r3>");
    case 17: return launch_w4<256, 128>(a, ilda, w, ildw, iM, iN, iK, ep, vec_ok, s, "gemm_i8_w4<256x128>");
    case 18: return launch_pp<256, 128, 4, 2, 3, 128>(a, ilda, w, ildw, iM, iN, iK, ep, vec_ok, s,
                                                      "gemm_i8_pp<256x128,4x2,r3,k128>");
    default: return launch_tile<128, 128, 2, 2>(a, ilda, w, ildw, iM, iN, iK, ep, vec_ok, s, "gemm_i8<128x128,2x2>");
  }
}

}  // namespace lsk

extern "C" int lsk_gemm_w8a8(const int8_t* a, int64_t lda, const int8_t* w, int64_t ldw, int64_t M, int64_t N,
                             int64_t K, int order, const float* asc, const float* ws, const float* bias,
                             const int32_t* erow, const int32_t* ecol, int shift, void* out, int out_dtype,
                             int64_t ldo, void* stream) {
  LSK_REQUIRE(M >= 0 && N >= 0 && K >= 0, "lsk_gemm_w8a8: negative size M=%lld N=%lld K=%lld", (long long)M,
              (long long)N, (long long)K);
  LSK_REQUIRE(K <= 133144, "lsk_gemm_w8a8: K=%lld exceeds the int32-exact bound 133144", (long long)K);
  LSK_REQUIRE(order != LSK_EPI_V25, "lsk_gemm_w8a8: the V25 epilogue takes its side inputs through lsk_gemm_w8a8_outlier");
  int rc = lsk::validate_epilogue(order, out_dtype, asc, ws, M, "lsk_gemm_w8a8");
  if (rc) return rc;
  if (M == 0 || N == 0) return LSK_OK;
  LSK_REQUIRE(out && ((a && w) || K == 0), "lsk_gemm_w8a8: null pointer");
  LSK_REQUIRE(lda >= K && ldw >= K && ldo >= N, "lsk_gemm_w8a8: leading dimension too small");
  EpiParams ep{order, out_dtype, ws, asc, bias, erow, ecol, shift, out, ldo};
  return lsk::launch_gemm(a, lda, w, ldw, M, N, K, ep, (hipStream_t)stream);
}

namespace lsk {
bool rowquant_pair_ok(const void* x, int x_dtype, int64_t ldx, int64_t K);
int rowquant_pair(const void* x, int x_dtype, int64_t M, int64_t K, int64_t ldx, int8_t* q, int64_t ldq, float* asc,
                  hipStream_t s);
}  // namespace lsk

// The quantised rows' share of lsk_w8a8_matmul's workspace: room for either layout (row-major
// rows of K rounded up to 16, or row pairs of K rounded up to 64).
static int64_t w8a8_q_bytes(int64_t M, int64_t K) {
  const int64_t major = M * ((K + 15) / 16 * 16), pair = ((M + 1) & ~(int64_t)1) * ((K + 63) / 64 * 64);
  return ((major > pair ? major : pair) + 255) / 256 * 256;
}

extern "C" int64_t lsk_w8a8_matmul_workspace(int64_t M, int64_t K) {
  return w8a8_q_bytes(M, K) + ((M * 4 + 255) / 256) * 256;
}

extern "C" int lsk_w8a8_matmul_pairs(const void* x, int x_dtype, int64_t ldx, int64_t M, int64_t K,
                                     const int8_t* w, int64_t ldw, const int8_t* w_pairs, int64_t N, const float* ws,
                                     const float* bias, int order, void* out, int out_dtype, int64_t ldo,
                                     void* workspace, int64_t workspace_bytes, void* stream);

extern "C" int lsk_w8a8_matmul(const void* x, int x_dtype, int64_t ldx, int64_t M, int64_t K, const int8_t* w,
                               int64_t ldw, int64_t N, const float* ws, const float* bias, int order, void* out,
                               int out_dtype, int64_t ldo, void* workspace, int64_t workspace_bytes, void* stream) {
  return lsk_w8a8_matmul_pairs(x, x_dtype, ldx, M, K, w, ldw, nullptr, N, ws, bias, order, out, out_dtype, ldo,
                               workspace, workspace_bytes, stream);
}

extern "C" int lsk_w8a8_matmul_pairs(const void* x, int x_dtype, int64_t ldx, int64_t M, int64_t K,
                                     const int8_t* w, int64_t ldw, const int8_t* w_pairs, int64_t N, const float* ws,
                                     const float* bias, int order, void* out, int out_dtype, int64_t ldo,
                                     void* workspace, int64_t workspace_bytes, void* stream) {
  LSK_REQUIRE(order == LSK_EPI_V21 || order == LSK_EPI_V2, "lsk_w8a8_matmul: order must be V21 or V2");
  LSK_REQUIRE(M >= 0 && N >= 0 && K >= 0, "lsk_w8a8_matmul: negative size");
  int rc = lsk::validate_epilogue(order, out_dtype, (const float*)1, ws, M, "lsk_w8a8_matmul");
  if (rc) return rc;
  if (M == 0 || N == 0) return LSK_OK;
  const int64_t need = lsk_w8a8_matmul_workspace(M, K);
  LSK_REQUIRE(workspace && workspace_bytes >= need, "lsk_w8a8_matmul: workspace of %lld bytes needed",
              (long long)need);
  LSK_REQUIRE(((uintptr_t)workspace & 255) == 0, "lsk_w8a8_matmul: workspace must be 256-byte aligned");
  // one activation row: the row quant fused into the whole-row GEMV (one launch)
  if (lsk::rowq_gemv_ok(x, w, ldw, M, N, K, order) && (x_dtype == LSK_F32 || x_dtype == LSK_BF16 || x_dtype == LSK_F16)) {
    LSK_REQUIRE(x && w && out && ldw >= K && ldo >= N, "lsk_w8a8_matmul: bad operand");
    EpiParams ep{order, out_dtype, ws, nullptr, bias, nullptr, nullptr, 0, out, ldo};
    return lsk::launch_gemv_rowq(x, x_dtype, w, (int)ldw, (int)N, (int)K, ep, (hipStream_t)stream);
  }
  // the row-pair layout when every tile of the GEMM is a ping-pong tile; row-major otherwise
  const int64_t kp = (K + 63) / 64 * 64;
  const bool pair = lsk::rowquant_pair_ok(x, x_dtype, ldx, K) && lsk::gemm_takes_pp(w, ldw, M, N, K, kp);
  const int64_t ldq = pair ? kp : (K + 15) / 16 * 16;
  int8_t* q = (int8_t*)workspace;
  float* asc = (float*)((char*)workspace + w8a8_q_bytes(M, K));
  if (!pair && w_pairs && lsk::gemm_takes_skinny(w_pairs, kp, M, N, K, ldq)) {
    // decode rows: row-major q, the weight's row-pair copy streamed by the skinny GEMV
    LSK_REQUIRE(w && out && ldw >= K && ldo >= N, "lsk_w8a8_matmul: bad operand");
    if ((rc = lsk_rowquant(x, x_dtype, M, K, ldx, q, ldq, asc, stream))) return rc;
    EpiParams ep{order, out_dtype, ws, asc, bias, nullptr, nullptr, 0, out, ldo};
    ep.pairs = 2;
    return lsk::launch_gemm(q, ldq, w_pairs, kp, M, N, K, ep, (hipStream_t)stream);
  }
  if (!pair)
    return (rc = lsk_rowquant(x, x_dtype, M, K, ldx, q, ldq, asc, stream))
               ? rc
               : lsk_gemm_w8a8(q, ldq, w, ldw, M, N, K, order, asc, ws, bias, nullptr, nullptr, 0, out, out_dtype,
                               ldo, stream);
  LSK_REQUIRE(x && w && out && ldw >= K && ldo >= N, "lsk_w8a8_matmul: bad operand");
  if ((rc = lsk::rowquant_pair(x, x_dtype, M, K, ldx, q, ldq, asc, (hipStream_t)stream))) return rc;
  EpiParams ep{order, out_dtype, ws, asc, bias, nullptr, nullptr, 0, out, ldo};
  ep.pairs = 1;
  // the weight's row-pair copy with the quantised rows' row-pair layout
  if (w_pairs && lsk::gemm_takes_pp(w_pairs, kp, M, N, K, kp)) {
    ep.pairs = 3;
    return lsk::launch_gemm(q, ldq, w_pairs, kp, M, N, K, ep, (hipStream_t)stream);
  }
  return lsk::launch_gemm(q, ldq, w, ldw, M, N, K, ep, (hipStream_t)stream);
}

extern "C" int lsk_epilogue_apply(const int32_t* acc, int64_t ldc, int64_t M, int64_t N, int order,
                                  const float* asc, const float* ws, const float* bias, const int32_t* erow,
                                  const int32_t* ecol, int shift, void* out, int out_dtype, int64_t ldo,
                                  void* stream) {
  LSK_REQUIRE(M >= 0 && N >= 0, "lsk_epilogue_apply: negative size");
  LSK_REQUIRE(order != LSK_EPI_RAW, "lsk_epilogue_apply: RAW is a copy, not an epilogue");
  LSK_REQUIRE(order != LSK_EPI_V25, "lsk_epilogue_apply: V25 is applied by lsk_gemm_w8a8_outlier");
  int rc = lsk::validate_epilogue(order, out_dtype, asc, ws, M, "lsk_epilogue_apply");
  if (rc) return rc;
  if (M == 0 || N == 0) return LSK_OK;
  LSK_REQUIRE(acc && out, "lsk_epilogue_apply: null pointer");
  LSK_REQUIRE(ldc >= N && ldo >= N, "lsk_epilogue_apply: leading dimension below N");
  EpiParams ep{order, out_dtype, ws, asc, bias, erow, ecol, shift, out, ldo};
  int64_t blocks = (M * N + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  hipLaunchKernelGGL(epilogue_apply_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, acc, ldc, M,
                     N, ep);
  return lsk::check_launch("epilogue_apply_kernel");
}

extern "C" int lsk_gemm_fuse_rowquant(int on) {
  LSK_REQUIRE(on == 0 || on == 1, "lsk_gemm_fuse_rowquant: %d not 0 or 1", on);
  lsk::g_rowq = on;
  return LSK_OK;
}

extern "C" int lsk_gemm_skinny_shape(int gpb, int kw, int depth) {
  LSK_REQUIRE(gpb >= 0 && gpb <= 16 && kw >= 0 && kw <= 16 && (gpb == 0 || kw == 0 || gpb * kw <= 16) &&
                  (depth == 0 || depth == 4 || depth == 8),
              "lsk_gemm_skinny_shape: gpb=%d kw=%d depth=%d (gpb * kw <= 16, depth 0, 4 or 8)", gpb, kw, depth);
  lsk::g_skinny_gpb = gpb;
  lsk::g_skinny_kw = kw;
  lsk::g_skinny_d = depth;
  return LSK_OK;
}

extern "C" int lsk_gemm_persist(int blocks) {
  LSK_REQUIRE(blocks >= 0 && blocks <= 65536, "lsk_gemm_persist: %d blocks", blocks);
  lsk::g_pp_persist = blocks;
  return LSK_OK;
}

extern "C" int lsk_gemm_select(int tile_id) {
  LSK_REQUIRE(tile_id >= -1 && tile_id <= 19 && tile_id != 16,
              "lsk_gemm_select: tile id %d not in [-1, 19] (16, the four-wave 256x256 tile, was removed)", tile_id);
  lsk::g_force_tile = ((tile_id >= 6 && tile_id <= 11) || tile_id == 14 || tile_id == 15 || tile_id == 19) ? 5 : tile_id;
  lsk::g_gemv_mid = tile_id == 14 ? 1 : (tile_id == 15 ? 2 : (tile_id == 19 ? 3 : 0));
  lsk::g_gemv_variant = (tile_id == 6 || tile_id == 7) ? tile_id - 5 : 0;
  lsk::g_row_rpw = (tile_id >= 8 && tile_id <= 11) ? (1 << (tile_id - 8)) : 0;
  return LSK_OK;
}
