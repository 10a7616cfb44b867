// The contract v2.5 outlier side path on gfx950 (lockstep_fullstack.py:549-578).
//
// A norm-fed linear with declared outlier channels oidx: the channels leave the row as their
// exact values ho, the masked row takes the 256-block butterfly / 16 (R1 online; none for the
// v2.5.1 o_proj form) and the per-row int8 quant, the exact int8 GEMM runs on the published
// weight, and the epilogue (order LSK_EPI_V25, fused into the GEMM kernels) adds the side term
//   side[m, n] = sum_j fl32(ho[m, j] * wo[n, j])   (sequential in j from +0)
// to the bf16-rounded v2.1 value before a second bf16 rounding.
//
// Stages: (1) a convert-copy of the row into binary32 workspace, (2) the outlier gather +
// mask, (3) the butterfly in place (rot), (4) the row quant, (5) the GEMM with the V25
// epilogue.  Every stage is stream-ordered; none allocates.
#include "lsk_common.h"

namespace lsk {
int launch_gemm(const int8_t* a, int64_t lda, const int8_t* w, int64_t ldw, int64_t M, int64_t N, int64_t K,
                const EpiParams& ep, hipStream_t s);
int validate_epilogue(int order, int out_dtype, const float* asc, const float* ws, int64_t M, const char* who);
}  // namespace lsk

namespace {

// x [M, K] of x_dtype (row stride ldx) -> xm binary32 [M, K] (row stride ldm), exact widening.
__global__ __launch_bounds__(256) void widen_rows_kernel(const void* __restrict__ x, int x_dtype, int64_t ldx,
                                                         int64_t M, int64_t K, float* __restrict__ xm, int64_t ldm,
                                                         int64_t chunks) {
  const int64_t b = blockIdx.x;
  const int64_t m = b / chunks;
  const int64_t k0 = (b - m * chunks) * 1024;
  if (m >= M) return;
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const int64_t k = k0 + t * 256 + threadIdx.x;
    if (k < K) xm[m * ldm + k] = load_as_f32(x, x_dtype, m * ldx + k);
  }
}

// Resolve a declared channel like torch indexing does (negative counts from the end); -1 when
// out of range (the gather then yields NaN and nothing is masked).
LSK_DEV int64_t resolve_channel(int32_t i, int64_t K) {
  int64_t c = i < 0 ? (int64_t)i + K : (int64_t)i;
  return (c >= 0 && c < K) ? c : -1;
}

// ho[m, j] = x[m, oidx[j]] (binary32); xm[m, oidx[j]] = 0 (when xm is given).
__global__ __launch_bounds__(256) void outlier_gather_kernel(const void* __restrict__ x, int x_dtype, int64_t ldx,
                                                             int64_t M, int64_t K, const int32_t* __restrict__ oidx,
                                                             int ko, float* __restrict__ ho, float* xm, int64_t ldm) {
  const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (e >= M * ko) return;
  const int64_t m = e / ko;
  const int j = (int)(e - m * ko);
  const int64_t c = resolve_channel(oidx[j], K);
  ho[e] = c >= 0 ? load_as_f32(x, x_dtype, m * ldx + c) : __builtin_nanf("");
  if (xm && c >= 0) xm[m * ldm + c] = 0.0f;
}

// side[m, n] = sum_j fl32(ho[m, j] * wo[n, j]), sequential in j from +0 (binary32 out).
__global__ __launch_bounds__(256) void outlier_side_kernel(const void* __restrict__ ho, int ho_dtype, int64_t M,
                                                           int ko, const void* __restrict__ wo, int wo_dtype,
                                                           int64_t N, float* __restrict__ side) {
  const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (e >= M * N) return;
  const int64_t m = e / N, n = e - m * N;
  float s = 0.0f;
  for (int j = 0; j < ko; ++j)
    s = f32_add(s, f32_mul(load_as_f32(ho, ho_dtype, m * ko + j), load_as_f32(wo, wo_dtype, n * ko + j)));
  side[e] = s;
}

bool side_dtype_ok(int d) { return d == LSK_F32 || d == LSK_BF16 || d == LSK_F16; }

}  // namespace

extern "C" int lsk_outlier_side(const void* ho, int ho_dtype, int64_t M, int64_t ko, const void* wo, int wo_dtype,
                                int64_t N, float* side, void* stream) {
  LSK_REQUIRE(M >= 0 && N >= 0 && ko >= 0, "lsk_outlier_side: negative size");
  LSK_REQUIRE(ko <= 0x7fffffff, "lsk_outlier_side: ko too large");
  LSK_REQUIRE(side_dtype_ok(ho_dtype) && side_dtype_ok(wo_dtype), "lsk_outlier_side: ho/wo dtype must be f32/bf16/f16");
  if (M == 0 || N == 0) return LSK_OK;
  LSK_REQUIRE(side && ((ho && wo) || ko == 0), "lsk_outlier_side: null pointer");
  const int64_t blocks = (M * N + 255) / 256;
  LSK_REQUIRE(blocks <= 0x7fffffff, "lsk_outlier_side: M*N too large");
  hipLaunchKernelGGL(outlier_side_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, ho, ho_dtype, M,
                     (int)ko, wo, wo_dtype, N, side);
  return lsk::check_launch("outlier_side_kernel");
}

extern "C" int lsk_outlier_split(const void* x, int x_dtype, int64_t ldx, int64_t M, int64_t K, const int32_t* oidx,
                                 int64_t ko, float* xm, int64_t ldm, float* ho, void* stream) {
  LSK_REQUIRE(M >= 0 && K >= 0 && ko >= 0, "lsk_outlier_split: negative size");
  LSK_REQUIRE(ko <= 4096, "lsk_outlier_split: ko=%lld above 4096", (long long)ko);
  LSK_REQUIRE(x_dtype == LSK_F32 || x_dtype == LSK_BF16 || x_dtype == LSK_F16, "lsk_outlier_split: x dtype %d",
              x_dtype);
  if (M == 0) return LSK_OK;
  LSK_REQUIRE(ldx >= K && (!xm || ldm >= K), "lsk_outlier_split: leading dimension below K");
  LSK_REQUIRE(x || K == 0, "lsk_outlier_split: null x");
  LSK_REQUIRE((oidx && ho) || ko == 0, "lsk_outlier_split: null oidx/ho");
  hipStream_t s = (hipStream_t)stream;
  if (xm && K > 0) {
    const int64_t chunks = (K + 1023) / 1024;
    LSK_REQUIRE(M * chunks <= 0x7fffffff, "lsk_outlier_split: too many rows");
    hipLaunchKernelGGL(widen_rows_kernel, dim3((unsigned)(M * chunks)), dim3(256), 0, s, x, x_dtype, ldx, M, K, xm,
                       ldm, chunks);
    int rc = lsk::check_launch("widen_rows_kernel");
    if (rc) return rc;
  }
  if (ko == 0) return LSK_OK;
  LSK_REQUIRE(K > 0, "lsk_outlier_split: declared channels of an empty row");
  const int64_t blocks = (M * ko + 255) / 256;
  LSK_REQUIRE(blocks <= 0x7fffffff, "lsk_outlier_split: M*ko too large");
  hipLaunchKernelGGL(outlier_gather_kernel, dim3((unsigned)blocks), dim3(256), 0, s, x, x_dtype, ldx, M, K, oidx,
                     (int)ko, ho, xm, ldm);
  return lsk::check_launch("outlier_gather_kernel");
}

extern "C" int lsk_gemm_w8a8_outlier(const int8_t* a, int64_t lda, const int8_t* w, int64_t ldw, int64_t M, int64_t N,
                                     int64_t K, const float* asc, const float* ws, const float* bias, const float* ho,
                                     int64_t ko, const void* wo, int wo_dtype, void* out, int out_dtype, int64_t ldo,
                                     void* stream) {
  LSK_REQUIRE(M >= 0 && N >= 0 && K >= 0 && ko >= 0, "lsk_gemm_w8a8_outlier: negative size");
  LSK_REQUIRE(K <= 133144, "lsk_gemm_w8a8_outlier: K=%lld exceeds the int32-exact bound 133144", (long long)K);
  LSK_REQUIRE(ko <= 4096, "lsk_gemm_w8a8_outlier: ko=%lld above 4096", (long long)ko);
  LSK_REQUIRE(wo_dtype == LSK_BF16 || wo_dtype == LSK_F32, "lsk_gemm_w8a8_outlier: wo must be bf16 or f32");
  int rc = lsk::validate_epilogue(LSK_EPI_V25, out_dtype, asc, ws, M, "lsk_gemm_w8a8_outlier");
  if (rc) return rc;
  if (M == 0 || N == 0) return LSK_OK;
  LSK_REQUIRE(out && ((a && w) || K == 0) && ((ho && wo) || ko == 0), "lsk_gemm_w8a8_outlier: null pointer");
  LSK_REQUIRE(lda >= K && ldw >= K && ldo >= N, "lsk_gemm_w8a8_outlier: leading dimension too small");
  EpiParams ep{LSK_EPI_V25, out_dtype, ws, asc, bias, nullptr, nullptr, 0, out, ldo};
  ep.ho = ho;
  ep.wo = wo;
  ep.ko = (int)ko;
  ep.wo_dtype = wo_dtype;
  return lsk::launch_gemm(a, lda, w, ldw, M, N, K, ep, (hipStream_t)stream);
}

namespace {
int64_t align256(int64_t b) { return (b + 255) / 256 * 256; }
}  // namespace

extern "C" int64_t lsk_w8a8_outlier_linear_workspace(int64_t M, int64_t K, int64_t ko) {
  const int64_t ldq = (K + 15) / 16 * 16;
  return align256(M * K * 4) + align256(M * ko * 4) + align256(M * ldq) + align256(M * 4);
}

extern "C" int lsk_w8a8_outlier_linear(const void* x, int x_dtype, int64_t ldx, int64_t M, int64_t K,
                                       const int32_t* oidx, int64_t ko, const void* wo, int wo_dtype, const int8_t* w,
                                       int64_t ldw, int64_t N, const float* ws, const float* bias, int rot, void* out,
                                       int out_dtype, int64_t ldo, void* workspace, int64_t workspace_bytes,
                                       void* stream) {
  LSK_REQUIRE(M >= 0 && N >= 0 && K >= 0 && ko >= 0, "lsk_w8a8_outlier_linear: negative size");
  LSK_REQUIRE(!rot || K % 256 == 0, "lsk_w8a8_outlier_linear: K=%lld is not a multiple of the 256-wide rotation block",
              (long long)K);
  int rc = lsk::validate_epilogue(LSK_EPI_V25, out_dtype, (const float*)1, ws, M, "lsk_w8a8_outlier_linear");
  if (rc) return rc;
  if (M == 0 || N == 0) return LSK_OK;
  const int64_t need = lsk_w8a8_outlier_linear_workspace(M, K, ko);
  LSK_REQUIRE(workspace && workspace_bytes >= need, "lsk_w8a8_outlier_linear: workspace of %lld bytes needed",
              (long long)need);
  LSK_REQUIRE(((uintptr_t)workspace & 255) == 0, "lsk_w8a8_outlier_linear: workspace must be 256-byte aligned");
  char* p = (char*)workspace;
  float* xm = (float*)p;
  p += align256(M * K * 4);
  float* ho = (float*)p;
  p += align256(M * ko * 4);
  const int64_t ldq = (K + 15) / 16 * 16;
  int8_t* q = (int8_t*)p;
  p += align256(M * ldq);
  float* asc = (float*)p;
  if ((rc = lsk_outlier_split(x, x_dtype, ldx, M, K, oidx, ko, xm, K, ho, stream))) return rc;
  if (rot && K > 0 && (rc = lsk_fwht_blocks(xm, M, K, K, 256, 1.0f / 16.0f, xm, K, stream))) return rc;
  if ((rc = lsk_rowquant(xm, LSK_F32, M, K, K, q, ldq, asc, stream))) return rc;
  return lsk_gemm_w8a8_outlier(q, ldq, w, ldw, M, N, K, asc, ws, bias, ho, ko, wo, wo_dtype, out, out_dtype, ldo,
                               stream);
}
