// Two-plane int8 carriers of wider integers (the lm_head / linear variants a<A>w<W> of
// t16h_lmvariants.py:71-125) on gfx950.
//
// A <B>-bit value a (|a| <= 2^(B-1) - 1, B in {8, 11, 15}) is carried exactly by two int8
// planes: hi = a >> (B - 8) in [-128, 127] (arithmetic shift = floor division) and
// lo = a - (hi << (B - 8)) in [0, 2^(B-8) - 1]; B = 8 is one plane.  Every plane product is an
// exact int32 GEMM (|plane acc| <= 128 * 128 * K < 2^31 for K <= 131071) and the planes are combined exactly in int64:
//   s[m, n] = sum_{pa, pw} acc_{pa,pw}[m, n] << (sh_a(pa) + sh_w(pw)).
// The logits epilogue is fl32(fl32(fl32(s) * asc[m]) * ws[n]) (t16h_lmvariants.py:125), fl32(s)
// rounded to nearest even from int64, then (with a bias) fl32(y + b[n]) and the output cast.
//
// Layouts: activation planes q [Pa * M, ldq] int8 (plane p of row m at row p * M + m, the hi
// plane first); weight planes [Pw * N, ldw] int8 the same way; the plane GEMM is one exact GEMM
// of the stacked operands, C [Pa * M, Pw * N] int32, whose blocks are the four products.
#include "lsk_common.h"

namespace lsk {
int launch_gemm(const int8_t* a, int64_t lda, const int8_t* w, int64_t ldw, int64_t M, int64_t N, int64_t K,
                const EpiParams& ep, hipStream_t s);
}  // namespace lsk

namespace {

constexpr float kAmaxFloor = 0x1.5798eep-27f;  // binary32 nearest 1e-8 (torch clamp(min=1e-8))

// The element the quantiser sees: x, or fl32(x / sdiv[k]) (op 1, the runtime SmoothQuant
// divide) or fl32(x * sdiv[k]) (op 2, the prepare-time weight fold).
LSK_DEV float col_op(float v, const float* sdiv, int op, int64_t k) {
  if (op == 1) return f32_div(v, sdiv[k]);
  if (op == 2) return f32_mul(v, sdiv[k]);
  return v;
}

template <int THREADS>
LSK_DEV float block_max(float v, float* red) {
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  if (lane == 0) red[wave] = v;
  __syncthreads();
  float r = red[0];
  for (int w = 1; w < THREADS / 64; ++w) r = fmaxf(r, red[w]);
  __syncthreads();
  return r;
}

// One block per row: amax (exact, order-free), asc = fl32(max(amax, 1e-8) / amax_q),
// a = clamp(rint_even(fl32(v / asc)), +-amax_q); then either the int32 value (q32) or its planes.
template <int THREADS>
__global__ __launch_bounds__(THREADS) void quant_planes_kernel(const void* __restrict__ x, int dtype, int64_t M,
                                                               int64_t K, int64_t ldx, int bits,
                                                               const float* __restrict__ sdiv, int op,
                                                               int8_t* __restrict__ q, int64_t ldq,
                                                               int32_t* __restrict__ q32, float* __restrict__ asc) {
  __shared__ float red[THREADS / 64];
  const int64_t m = blockIdx.x;
  const int tid = threadIdx.x;
  const int64_t base = m * ldx;
  float am = 0.0f;
  for (int64_t k = tid; k < K; k += THREADS) am = fmaxf(am, fabsf(col_op(load_as_f32(x, dtype, base + k), sdiv, op, k)));
  am = block_max<THREADS>(am, red);
  am = fmaxf(am, kAmaxFloor);
  const float qmax = (float)((1 << (bits - 1)) - 1);
  const float s = f32_div(am, qmax);
  if (tid == 0) asc[m] = s;
  const int sh = bits - 8;
  for (int64_t k = tid; k < K; k += THREADS) {
    float t = rintf(f32_div(col_op(load_as_f32(x, dtype, base + k), sdiv, op, k), s));
    t = fminf(fmaxf(t, -qmax), qmax);
    const int a = (int)t;
    if (q32) {
      q32[m * K + k] = a;
    } else if (sh == 0) {
      q[m * ldq + k] = (int8_t)a;
    } else {
      const int hi = a >> sh;
      q[m * ldq + k] = (int8_t)hi;
      q[(M + m) * ldq + k] = (int8_t)(a - (hi << sh));
    }
  }
}

// Split int32 values into planes: hi = a >> sh, lo = a - (hi << sh) (sh = 0: one plane, a itself).
__global__ __launch_bounds__(256) void split_planes_kernel(const int32_t* __restrict__ a, int64_t n, int sh,
                                                           int8_t* __restrict__ hi, int8_t* __restrict__ lo) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const int v = a[i];
  const int h = v >> sh;
  hi[i] = (int8_t)h;
  if (sh) lo[i] = (int8_t)(v - (h << sh));
}

// int64 -> binary32, round to nearest even (the conversion torch's `.to(torch.float32)` of an
// int64 tensor performs): normalise |s| to bit 63, keep 24 bits, round the 40 below them.
LSK_DEV float i64_to_f32_rne(int64_t s) {
  if (s == 0) return 0.0f;
  const uint32_t sign = s < 0 ? 0x80000000u : 0u;
  uint64_t u = s < 0 ? (uint64_t)0 - (uint64_t)s : (uint64_t)s;
  const int lz = __builtin_clzll(u);
  u <<= lz;
  uint32_t mant = (uint32_t)(u >> 40);  // 24 bits, leading one at bit 23
  const uint64_t rest = u & ((1ull << 40) - 1);
  const uint64_t half = 1ull << 39;
  int e = 63 - lz;  // value = mant * 2^(e - 23)
  if (rest > half || (rest == half && (mant & 1u))) {
    ++mant;
    if (mant == (1u << 24)) {
      mant >>= 1;
      ++e;
    }
  }
  return __uint_as_float(sign | ((uint32_t)(e + 127) << 23) | (mant & 0x7fffffu));
}

struct CombineArgs {
  const int32_t* c;
  int64_t ldc;
  int64_t M, N;  // logical rows / columns; C holds pa * M rows and pw * N columns
  int pa, pw, sha, shw;
  const float* asc;
  const float* ws;
  const float* bias;
  void* out;
  int out_dtype;
  int64_t ldo;
};

__global__ __launch_bounds__(256) void planes_combine_kernel(CombineArgs p) {
  const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (e >= p.M * p.N) return;
  const int64_t m = e / p.N, n = e - m * p.N;
  int64_t s = 0;
  for (int i = 0; i < p.pa; ++i) {
    const int ai = (i == 0 && p.pa == 2) ? p.sha : 0;  // the hi plane carries the shift
    for (int j = 0; j < p.pw; ++j) {
      const int wj = (j == 0 && p.pw == 2) ? p.shw : 0;
      s += (int64_t)p.c[(i * p.M + m) * p.ldc + j * p.N + n] << (ai + wj);
    }
  }
  float y = f32_mul(f32_mul(i64_to_f32_rne(s), p.asc[m]), p.ws[n]);
  if (p.bias) y = f32_add(y, p.bias[n]);
  store_out(p.out, p.out_dtype, m * p.ldo + n, y);
}

bool bits_ok(int b) { return b == 8 || b == 11 || b == 15; }
int64_t align256(int64_t b) { return (b + 255) / 256 * 256; }

// Rows of one chunk of the plane linear: the chunk's int32 plane products stay under 256 MB.
int64_t chunk_rows(int64_t M, int64_t N, int pa, int pw) {
  const int64_t per_row = (int64_t)pa * pw * N * 4;
  int64_t mc = per_row > 0 ? ((int64_t)1 << 28) / per_row : M;
  if (mc < 32) mc = 32;
  return mc < M ? mc : M;
}

}  // namespace

extern "C" int lsk_quant_planes(const void* x, int x_dtype, int64_t ldx, int64_t M, int64_t K, int bits,
                                const float* sdiv, int sdiv_op, int8_t* q, int64_t ldq, int32_t* q32, float* asc,
                                void* stream) {
  LSK_REQUIRE(M >= 0 && K >= 0, "lsk_quant_planes: negative size");
  LSK_REQUIRE(bits_ok(bits), "lsk_quant_planes: bits=%d not one of 8, 11, 15", bits);
  LSK_REQUIRE(x_dtype == LSK_F32 || x_dtype == LSK_BF16 || x_dtype == LSK_F16, "lsk_quant_planes: x dtype %d", x_dtype);
  LSK_REQUIRE(sdiv_op >= 0 && sdiv_op <= 2 && (sdiv_op == 0 || sdiv), "lsk_quant_planes: bad sdiv / sdiv_op");
  if (M == 0) return LSK_OK;
  LSK_REQUIRE(asc && (q || q32) && (x || K == 0), "lsk_quant_planes: null pointer");
  LSK_REQUIRE(ldx >= K && (q32 || ldq >= K), "lsk_quant_planes: leading dimension below K");
  LSK_REQUIRE(M <= 0x7fffffff, "lsk_quant_planes: too many rows");
  hipLaunchKernelGGL(quant_planes_kernel<256>, dim3((unsigned)M), dim3(256), 0, (hipStream_t)stream, x, x_dtype, M, K,
                     ldx, bits, sdiv, sdiv_op, q, ldq, q32, asc);
  return lsk::check_launch("quant_planes_kernel");
}

extern "C" int lsk_split_planes(const int32_t* a, int64_t n, int sh, int8_t* hi, int8_t* lo, void* stream) {
  LSK_REQUIRE(n >= 0 && sh >= 0 && sh <= 24, "lsk_split_planes: bad size or shift");
  if (n == 0) return LSK_OK;
  LSK_REQUIRE(a && hi && (lo || sh == 0), "lsk_split_planes: null pointer");
  const int64_t blocks = (n + 255) / 256;
  LSK_REQUIRE(blocks <= 0x7fffffff, "lsk_split_planes: too many elements");
  hipLaunchKernelGGL(split_planes_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, a, n, sh, hi, lo);
  return lsk::check_launch("split_planes_kernel");
}

extern "C" int lsk_planes_combine(const int32_t* c, int64_t ldc, int64_t M, int64_t N, int abits, int wbits,
                                  const float* asc, const float* ws, const float* bias, void* out, int out_dtype,
                                  int64_t ldo, void* stream) {
  LSK_REQUIRE(M >= 0 && N >= 0, "lsk_planes_combine: negative size");
  LSK_REQUIRE(bits_ok(abits) && bits_ok(wbits), "lsk_planes_combine: widths must be 8, 11 or 15");
  LSK_REQUIRE(out_dtype == LSK_F32 || out_dtype == LSK_BF16 || out_dtype == LSK_F16 || out_dtype == LSK_BF16_AS_F32,
              "lsk_planes_combine: out_dtype %d", out_dtype);
  if (M == 0 || N == 0) return LSK_OK;
  const int pa = abits == 8 ? 1 : 2, pw = wbits == 8 ? 1 : 2;
  LSK_REQUIRE(c && asc && ws && out, "lsk_planes_combine: null pointer");
  LSK_REQUIRE(ldc >= pw * N && ldo >= N, "lsk_planes_combine: leading dimension too small");
  const int64_t blocks = (M * N + 255) / 256;
  LSK_REQUIRE(blocks <= 0x7fffffff, "lsk_planes_combine: M*N too large");
  CombineArgs p{c, ldc, M, N, pa, pw, abits - 8, wbits - 8, asc, ws, bias, out, out_dtype, ldo};
  hipLaunchKernelGGL(planes_combine_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, p);
  return lsk::check_launch("planes_combine_kernel");
}

extern "C" int64_t lsk_planes_linear_workspace(int64_t M, int64_t K, int64_t N, int abits, int wbits) {
  if (!bits_ok(abits) || !bits_ok(wbits) || M < 0 || K < 0 || N < 0) return -1;
  const int pa = abits == 8 ? 1 : 2, pw = wbits == 8 ? 1 : 2;
  const int64_t ldq = (K + 15) / 16 * 16;
  const int64_t mc = chunk_rows(M, N, pa, pw);
  return align256((int64_t)pa * mc * ldq) + align256(M * 4) + align256((int64_t)pa * mc * pw * N * 4);
}

extern "C" int lsk_planes_linear(const void* x, int x_dtype, int64_t ldx, int64_t M, int64_t K, int abits,
                                 const float* sdiv, const int8_t* w, int64_t ldw, int64_t N, int wbits, const float* ws,
                                 const float* bias, void* out, int out_dtype, int64_t ldo, void* workspace,
                                 int64_t workspace_bytes, void* stream) {
  LSK_REQUIRE(M >= 0 && N >= 0 && K >= 0, "lsk_planes_linear: negative size");
  LSK_REQUIRE(bits_ok(abits) && bits_ok(wbits), "lsk_planes_linear: widths must be 8, 11 or 15");
  // every plane product is bounded by 128 * 128 * K; int32 is exact for K <= 131071
  LSK_REQUIRE(K <= 131071, "lsk_planes_linear: K=%lld exceeds the int32-exact plane bound 131071", (long long)K);
  LSK_REQUIRE(out_dtype == LSK_F32 || out_dtype == LSK_BF16 || out_dtype == LSK_F16 || out_dtype == LSK_BF16_AS_F32,
              "lsk_planes_linear: out_dtype %d", out_dtype);
  if (M == 0 || N == 0) return LSK_OK;
  const int pa = abits == 8 ? 1 : 2, pw = wbits == 8 ? 1 : 2;
  const int64_t need = lsk_planes_linear_workspace(M, K, N, abits, wbits);
  LSK_REQUIRE(workspace && workspace_bytes >= need, "lsk_planes_linear: workspace of %lld bytes needed",
              (long long)need);
  LSK_REQUIRE(((uintptr_t)workspace & 255) == 0, "lsk_planes_linear: workspace must be 256-byte aligned");
  LSK_REQUIRE(ws && out && (w || K == 0) && ldw >= K && ldo >= N, "lsk_planes_linear: bad weight or output");
  hipStream_t s = (hipStream_t)stream;
  const int64_t ldq = (K + 15) / 16 * 16;
  const int64_t mc = chunk_rows(M, N, pa, pw);
  char* p = (char*)workspace;
  int8_t* q = (int8_t*)p;
  p += align256((int64_t)pa * mc * ldq);
  float* asc = (float*)p;
  p += align256(M * 4);
  int32_t* c = (int32_t*)p;
  const int osz = (out_dtype == LSK_BF16 || out_dtype == LSK_F16) ? 2 : 4;
  for (int64_t m0 = 0; m0 < M; m0 += mc) {
    const int64_t rows = (M - m0) < mc ? (M - m0) : mc;
    // the chunk's planes: plane i of chunk row r at row i * rows + r, so one GEMM of pa * rows
    // rows reads the weight planes once for every activation plane
    int rc = lsk_quant_planes((const char*)x + m0 * ldx * (x_dtype == LSK_F32 ? 4 : 2), x_dtype, ldx, rows, K, abits,
                              sdiv, sdiv ? 1 : 0, q, ldq, nullptr, asc + m0, stream);
    if (rc) return rc;
    EpiParams ep{LSK_EPI_RAW, LSK_I32, nullptr, nullptr, nullptr, nullptr, nullptr, 0, c, (int64_t)pw * N};
    if ((rc = lsk::launch_gemm(q, ldq, w, ldw, (int64_t)pa * rows, (int64_t)pw * N, K, ep, s))) return rc;
    if ((rc = lsk_planes_combine(c, (int64_t)pw * N, rows, N, abits, wbits, asc + m0, ws, bias,
                                 (char*)out + m0 * ldo * osz, out_dtype, ldo, stream)))
      return rc;
  }
  return LSK_OK;
}
