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
#include "mfma_tile.h"
#include "pp_tile.h"

namespace {

using lsk::zero4;

// Dense tile kernel: C[m, n] = sum_k A[m, k] * W[n, k] with the epilogue applied per element.
// A and W are K-contiguous with 16-byte aligned rows and K % 16 == 0.  Logical tile ids walk
// M-fastest inside groups of 16 M-tiles after the XCD remap.
template <int BM, int BN, int WM, int WN, int PF>
__global__ __launch_bounds__(WM * WN * 64) void gemm_i8_mfma_kernel(
    const int8_t* __restrict__ A, int lda, const int8_t* __restrict__ W, int ldw, int M, int N, int K,
    EpiParams ep, int vec_ok) {
  using C = lsk::TileCfg<BM, BN, WM, WN>;
  extern __shared__ v4i smem[];
  const int mtiles = (M + BM - 1) / BM, ntiles = (N + BN - 1) / BN;
  const int L = lsk::xcd_logical_id(blockIdx.x, mtiles * ntiles);
  constexpr int GM = 16;
  const int group = L / (GM * ntiles);
  const int first_m = group * GM;
  const int gsize = (mtiles - first_m) < GM ? (mtiles - first_m) : GM;
  const int r = L - group * GM * ntiles;
  const int m0 = (first_m + r % gsize) * BM, n0 = (r / gsize) * BN;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
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

  lsk::mfma_mainloop<BM, BN, WM, WN, PF>(acc, ra_res, pa, rb_res, pb, K, smem);

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
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
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
    if (m < M && n < N)
      epilogue_store4_pre(ep.out, ep.ldo, order, odt, has_bias, ep.shift, m, n, N, v, rv, wsv, bv,
                          pow2 ? __float_as_int(rv) : 0, ecv, vec);
  }
}

// All strips of the wave's tile, strip index a compile-time constant (the accumulators stay in
// registers): stage strip I in the wave's LDS region, store it, recurse.
template <class C, int ORDER, int ODT, bool BIAS, int I>
__device__ __forceinline__ void pp_epilogue(const typename C::Acc& acc, const EpiParams& ep, int m0, int n0, int M,
                                            int N, int vec_ok, char* smem) {
  if constexpr (I < C::TM) {
    int32_t* region = (int32_t*)(smem + (threadIdx.x >> 6) * C::kStripBytes);
    lsk::pp_stage_strip<C::TN, C::kLdc>(acc[I], region);
    pp_strip_store<C, ORDER, ODT, BIAS>(I, region, ep, m0, n0, M, N, vec_ok, smem);
    pp_epilogue<C, ORDER, ODT, BIAS, I + 1>(acc, ep, m0, n0, M, N, vec_ok, smem);
  }
}

// Dense ping-pong tile kernel (512 threads, eight waves in two alternating groups); same
// operand contract and tile order as gemm_i8_mfma_kernel.  The epilogue operands of the tile
// (asc / row exponents, ws, bias, column exponents) are loaded into registers before the main
// loop and parked in LDS after it, so the epilogue itself touches global memory only to store.
template <int BM, int BN, int WM, int WN, int RING>
__global__ __launch_bounds__(512) void gemm_i8_pp_kernel(const int8_t* __restrict__ A, int lda,
                                                         const int8_t* __restrict__ W, int ldw, int M, int N, int K,
                                                         EpiParams ep, int vec_ok) {
  using C = lsk::PPCfg<BM, BN, WM, WN, RING>;
  extern __shared__ __attribute__((aligned(16))) char smem_pp[];
  const int mtiles = (M + BM - 1) / BM, ntiles = (N + BN - 1) / BN;
  const int L = lsk::xcd_logical_id(blockIdx.x, mtiles * ntiles);
  constexpr int GM = 16;
  const int group = L / (GM * ntiles);
  const int first_m = group * GM;
  const int gsize = (mtiles - first_m) < GM ? (mtiles - first_m) : GM;
  const int r = L - group * GM * ntiles;
  const int m0 = (first_m + r % gsize) * BM, n0 = (r / gsize) * BN;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;

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

  const __amdgpu_buffer_rsrc_t ra_res = lsk::make_rsrc(A + (int64_t)m0 * lda, (int64_t)(M - m0) * lda);
  const __amdgpu_buffer_rsrc_t rb_res = lsk::make_rsrc(W + (int64_t)n0 * ldw, (int64_t)(N - n0) * ldw);
  typename C::RowsA pa;
  typename C::RowsB pb;
#pragma unroll
  for (int j = 0; j < C::kLA; ++j) {
    int row, kb;
    lsk::pp_slot<C::kThreads>(tid, j, row, kb);
    pa[j] = (m0 + row < M) ? (uint32_t)(row * lda) : lsk::kOob;
  }
#pragma unroll
  for (int j = 0; j < C::kLB; ++j) {
    int row, kb;
    lsk::pp_slot<C::kThreads>(tid, j, row, kb);
    pb[j] = (n0 + row < N) ? (uint32_t)(row * ldw) : lsk::kOob;
  }
  typename C::Acc acc;
#pragma unroll
  for (int i = 0; i < C::TM; ++i)
#pragma unroll
    for (int j = 0; j < C::TN; ++j) acc[i][j] = lsk::zero16();

  lsk::pp_mainloop<BM, BN, WM, WN, RING>(acc, ra_res, pa, rb_res, pb, K, smem_pp);

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
  __syncthreads();
  // each wave stages its own 32-row strips, then stores them through the epilogue
  const bool bias = ep.bias != nullptr;
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

// Decode GEMV: one block per 16 output columns; its 4 waves take interleaved 256-byte K slabs;
// each lane streams 64 contiguous weight bytes per slab (4 MFMAs).  MT 16-row tiles cover M.
template <int MT>
__global__ __launch_bounds__(256) void gemv_i8_mfma_kernel(const int8_t* __restrict__ A, int64_t lda,
                                                           const int8_t* __restrict__ W, int64_t ldw, int M,
                                                           int N, int K, EpiParams ep) {
  __shared__ v4i red[3][MT][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int col = lane & 15, kg = lane >> 4;
  const int n0 = blockIdx.x * 16;
  const int n = n0 + col;
  const bool nvalid = n < N;
  const int8_t* wrow = W + (int64_t)(nvalid ? n : 0) * ldw;

  v4i acc[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t) acc[t] = zero4();

  for (int kb = wave * 256; kb < K; kb += 4 * 256) {
    const int k = kb + kg * 64;
    v4i w4[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) w4[j] = (nvalid && k + j * 16 < K) ? *(const v4i*)(wrow + k + j * 16) : zero4();
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      const int m = t * 16 + col;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const v4i a = (m < M && k + j * 16 < K) ? *(const v4i*)(A + (int64_t)m * lda + k + j * 16) : zero4();
        acc[t] = lsk::mfma_i8(a, w4[j], acc[t]);
      }
    }
  }
  if (wave > 0) {
#pragma unroll
    for (int t = 0; t < MT; ++t) red[wave - 1][t][lane] = acc[t];
  }
  __syncthreads();
  if (wave != 0) return;
#pragma unroll
  for (int t = 0; t < MT; ++t) {
    v4i s = acc[t];
#pragma unroll
    for (int w = 0; w < 3; ++w) s += red[w][t][lane];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int m = t * 16 + (lane >> 4) * 4 + r;
      if (m < M && nvalid) epilogue_store(ep, m, n, s[r]);
    }
  }
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
  LSK_REQUIRE(order >= LSK_EPI_V21 && order <= LSK_EPI_RAW, "%s: unknown epilogue order %d", who, order);
  if (order == LSK_EPI_RAW) {
    LSK_REQUIRE(out_dtype == LSK_I32, "%s: the RAW epilogue writes int32 (out_dtype %d)", who, out_dtype);
  } else if (order == LSK_EPI_POW2) {
    LSK_REQUIRE(out_dtype == LSK_F32, "%s: the POW2 epilogue writes binary32 (out_dtype %d)", who, out_dtype);
  } else {
    LSK_REQUIRE(out_dtype == LSK_F32 || out_dtype == LSK_BF16 || out_dtype == LSK_F16 || out_dtype == LSK_BF16_AS_F32,
                "%s: out_dtype %d not one of f32/bf16/f16/bf16-as-f32", who, out_dtype);
    LSK_REQUIRE(M == 0 || (asc && ws), "%s: asc and ws are required by the V21/V2 epilogues", who);
  }
  return LSK_OK;
}

// Tile configurations of the dense kernel; id -1 lets the shape decide.
static int g_force_tile = -1;

template <int BM, int BN, int WM, int WN, int PF = 1>
static int launch_tile(const int8_t* a, int lda, const int8_t* w, int ldw, int M, int N, int K,
                       const EpiParams& ep, int vec_ok, hipStream_t s, const char* name) {
  using C = TileCfg<BM, BN, WM, WN>;
  static bool attr_set = false;
  auto kern = gemm_i8_mfma_kernel<BM, BN, WM, WN, PF>;
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

template <int BM, int BN, int WM, int WN, int RING = 4>
static int launch_pp(const int8_t* a, int lda, const int8_t* w, int ldw, int M, int N, int K, const EpiParams& ep,
                     int vec_ok, hipStream_t s, const char* name) {
  using C = PPCfg<BM, BN, WM, WN, RING>;
  static bool attr_set = false;
  auto kern = gemm_i8_pp_kernel<BM, BN, WM, WN, RING>;
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

static int pick_tile(int64_t M, int64_t N) {
  if (g_force_tile >= 0) return g_force_tile;
  if (M <= 128) return 2;  // few rows: the 128x128 register-staged tile wastes least
  // Ping-pong tiles: whole rounds of 256 blocks (one per CU) are what a launch costs.  A
  // 256x128 tile takes 0.68 of a 256x256 tile's time (measured on MI355X at the Llama-3.1-8B /
  // Qwen2.5-7B prefill shapes), so pick the shape with the smaller rounds x tile cost.
  const int64_t r256 = ((M + 255) / 256 * ((N + 255) / 256) + 255) / 256;
  const int64_t r128 = ((M + 255) / 256 * ((N + 127) / 128) + 255) / 256;
  return (double)r128 * 0.68 < (double)r256 ? 11 : 10;
}

int launch_gemm(const int8_t* a, int64_t lda, const int8_t* w, int64_t ldw, int64_t M, int64_t N, int64_t K,
                const EpiParams& ep, hipStream_t s) {
  if (M == 0 || N == 0) return LSK_OK;
  // the tile kernels address rows by 32-bit offsets inside a 256-row tile
  const bool fast = (K % 16 == 0) && (lda % 16 == 0) && (ldw % 16 == 0) && aligned16(a) && aligned16(w) &&
                    M <= 0x7fffffff && N <= 0x7fffffff && K > 0 && lda * 256 < 0x7fffffff && ldw * 256 < 0x7fffffff;
  if (!fast) {
    const int64_t total = M * N;
    const int64_t blocks = (total + 255) / 256;
    LSK_REQUIRE(blocks <= 0x7fffffff, "gemm: M*N=%lld too large for the generic path", (long long)total);
    hipLaunchKernelGGL(gemm_i8_generic_kernel, dim3((unsigned)blocks), dim3(256), 0, s, a, lda, w, ldw, M, N, K, ep);
    return check_launch("gemm_i8_generic_kernel");
  }
  const int iM = (int)M, iN = (int)N, iK = (int)K;
  if (M <= 16) {
    hipLaunchKernelGGL(gemv_i8_mfma_kernel<1>, dim3((unsigned)((N + 15) / 16)), dim3(256), 0, s, a, lda, w, ldw, iM,
                       iN, iK, ep);
    return check_launch("gemv_i8_mfma_kernel<1>");
  }
  if (M <= 32) {
    hipLaunchKernelGGL(gemv_i8_mfma_kernel<2>, dim3((unsigned)((N + 15) / 16)), dim3(256), 0, s, a, lda, w, ldw, iM,
                       iN, iK, ep);
    return check_launch("gemv_i8_mfma_kernel<2>");
  }
  const int vec_ok = out_vec_ok(ep.out, ep.out_dtype, ep.ldo) ? 1 : 0;
  const int ilda = (int)lda, ildw = (int)ldw;
  switch (pick_tile(M, N)) {
    case 0: return launch_tile<256, 256, 2, 2>(a, ilda, w, ildw, iM, iN, iK, ep, vec_ok, s, "gemm_i8<256x256,2x2>");
    case 1: return launch_tile<256, 128, 4, 2>(a, ilda, w, ildw, iM, iN, iK, ep, vec_ok, s, "gemm_i8<256x128,4x2>");
    case 3: return launch_tile<256, 256, 4, 2>(a, ilda, w, ildw, iM, iN, iK, ep, vec_ok, s, "gemm_i8<256x256,4x2>");
    case 4: return launch_tile<128, 256, 2, 4>(a, ilda, w, ildw, iM, iN, iK, ep, vec_ok, s, "gemm_i8<128x256,2x4>");
    case 5: return launch_tile<128, 128, 2, 2, 2>(a, ilda, w, ildw, iM, iN, iK, ep, vec_ok, s, "gemm_i8<128x128,2x2,pf2>");
    case 6: return launch_tile<256, 128, 4, 2, 2>(a, ilda, w, ildw, iM, iN, iK, ep, vec_ok, s, "gemm_i8<256x128,4x2,pf2>");
    case 7: return launch_tile<256, 256, 4, 2, 2>(a, ilda, w, ildw, iM, iN, iK, ep, vec_ok, s, "gemm_i8<256x256,4x2,pf2>");
    case 8: return launch_tile<128, 256, 2, 4, 2>(a, ilda, w, ildw, iM, iN, iK, ep, vec_ok, s, "gemm_i8<128x256,2x4,pf2>");
    case 9: return launch_pp<256, 256, 2, 4>(a, ilda, w, ildw, iM, iN, iK, ep, vec_ok, s, "gemm_i8_pp<256x256,2x4>");
    case 10: return launch_pp<256, 256, 4, 2>(a, ilda, w, ildw, iM, iN, iK, ep, vec_ok, s, "gemm_i8_pp<256x256,4x2>");
    case 11: return launch_pp<256, 128, 4, 2>(a, ilda, w, ildw, iM, iN, iK, ep, vec_ok, s, "gemm_i8_pp<256x128,4x2>");
    case 12: return launch_pp<128, 256, 2, 4>(a, ilda, w, ildw, iM, iN, iK, ep, vec_ok, s, "gemm_i8_pp<128x256,2x4>");
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
  int rc = lsk::validate_epilogue(order, out_dtype, asc, ws, M, "lsk_gemm_w8a8");
  if (rc) return rc;
  if (M == 0 || N == 0) return LSK_OK;
  LSK_REQUIRE(out && ((a && w) || K == 0), "lsk_gemm_w8a8: null pointer");
  LSK_REQUIRE(lda >= K && ldw >= K && ldo >= N, "lsk_gemm_w8a8: leading dimension too small");
  EpiParams ep{order, out_dtype, ws, asc, bias, erow, ecol, shift, out, ldo};
  return lsk::launch_gemm(a, lda, w, ldw, M, N, K, ep, (hipStream_t)stream);
}

extern "C" int64_t lsk_w8a8_matmul_workspace(int64_t M, int64_t K) {
  const int64_t ldq = (K + 15) / 16 * 16;
  return ((M * ldq + 255) / 256) * 256 + ((M * 4 + 255) / 256) * 256;
}

extern "C" int lsk_w8a8_matmul(const void* x, int x_dtype, int64_t ldx, int64_t M, int64_t K, const int8_t* w,
                               int64_t ldw, int64_t N, const float* ws, const float* bias, int order, void* out,
                               int out_dtype, int64_t ldo, void* workspace, int64_t workspace_bytes, void* stream) {
  LSK_REQUIRE(order == LSK_EPI_V21 || order == LSK_EPI_V2, "lsk_w8a8_matmul: order must be V21 or V2");
  LSK_REQUIRE(M >= 0 && N >= 0 && K >= 0, "lsk_w8a8_matmul: negative size");
  int rc = lsk::validate_epilogue(order, out_dtype, (const float*)1, ws, M, "lsk_w8a8_matmul");
  if (rc) return rc;
  if (M == 0 || N == 0) return LSK_OK;
  const int64_t need = lsk_w8a8_matmul_workspace(M, K);
  LSK_REQUIRE(workspace && workspace_bytes >= need, "lsk_w8a8_matmul: workspace of %lld bytes needed",
              (long long)need);
  LSK_REQUIRE(((uintptr_t)workspace & 255) == 0, "lsk_w8a8_matmul: workspace must be 256-byte aligned");
  const int64_t ldq = (K + 15) / 16 * 16;
  int8_t* q = (int8_t*)workspace;
  float* asc = (float*)((char*)workspace + ((M * ldq + 255) / 256) * 256);
  rc = lsk_rowquant(x, x_dtype, M, K, ldx, q, ldq, asc, stream);
  if (rc) return rc;
  return lsk_gemm_w8a8(q, ldq, w, ldw, M, N, K, order, asc, ws, bias, nullptr, nullptr, 0, out, out_dtype, ldo,
                       stream);
}

extern "C" int lsk_epilogue_apply(const int32_t* acc, int64_t ldc, int64_t M, int64_t N, int order,
                                  const float* asc, const float* ws, const float* bias, const int32_t* erow,
                                  const int32_t* ecol, int shift, void* out, int out_dtype, int64_t ldo,
                                  void* stream) {
  LSK_REQUIRE(M >= 0 && N >= 0, "lsk_epilogue_apply: negative size");
  LSK_REQUIRE(order != LSK_EPI_RAW, "lsk_epilogue_apply: RAW is a copy, not an epilogue");
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

extern "C" int lsk_gemm_select(int tile_id) {
  LSK_REQUIRE(tile_id >= -1 && tile_id <= 12, "lsk_gemm_select: tile id %d not in [-1, 12]", tile_id);
  lsk::g_force_tile = tile_id;
  return LSK_OK;
}
