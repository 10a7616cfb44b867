// The contract 2.6 float RMSNorm (t16n_ref.py:38-92) on gfx950, and its fusion with the row quant
// that feeds the contract GEMM.
//
// Per row of width N (N % 8 == 0): sq = fl32(x * x); group g = elements 8g..8g+7 summed as a chain
// in index order; S = T(groups) where T splits at the largest power of two below the count (a
// power-of-two count is halved): the adjacent-pairs balanced tree.  That tree equals the perfect
// binary tree over the groups padded with -0 to the next power of two G' (x + (-0) == x for every
// binary32 x, so a padded subtree passes its real part through unchanged, and the splits of the
// padded tree land where T's do).  So: a row is split over W waves x 64 lanes, lane l of wave w
// holding C = G' / (64 W) consecutive groups; the lane reduces its groups as a perfect tree, the
// wave by xor-shuffles 1, 2, ..., 32 (adjacent pairs first), and the W wave sums by a tree in LDS.
// Then S = fl32(S + ne) (when eps), max(S, 2^-126), rs = fl32(sN / fl32(sqrt S)) (IEEE sqrt and
// division, correctly rounded by the build flags), out = bf16(fl32(fl32(x * rs) * g)).  The fused
// quant is the contract row quant of the bf16 outputs: asc = fl32(max(amax, 1e-8) / 127),
// q = clamp(rint_even(fl32(out / asc)), +-127).
#include "lsk_common.h"

namespace {

constexpr float kAmaxFloor = 0x1.5798eep-27f;  // binary32 nearest 1e-8
constexpr float kNegZero = -0.0f;              // the additive identity of binary32 RNE addition

struct NormArgs {
  const void* x;
  int x_dtype;
  int64_t ldx;
  int64_t R, N;
  const void* g;      // gain [N] or null (ones)
  int g_dtype;
  float sN, ne;
  int has_eps;
  void* out;          // [R, N] or null
  int out_dtype;
  int64_t ldo;
  int8_t* q;          // [R, N] or null (the fused row quant)
  int64_t ldq;
  float* asc;         // [R] (with q)
  float* S;           // [R] or null
};

// Perfect pairwise tree over v[0..n), n a power of two, adjacent pairs first.
template <int n>
LSK_DEV float local_tree(float* v) {
#pragma unroll
  for (int h = 1; h < n; h *= 2)
#pragma unroll
    for (int i = 0; i < n; i += 2 * h) v[i] = f32_add(v[i], v[i + h]);
  return v[0];
}

// The row's sum of squares by the pinned tree; every lane of the row's waves gets it.  xv holds the
// lane's C groups of 8 elements (binary32), groups past the row hold anything (masked here).
template <int C>
LSK_DEV float row_tree(const float (*xv)[8], int64_t g0, int64_t G, float* red, int W) {
  float a[C];
#pragma unroll
  for (int c = 0; c < C; ++c) {
    float s = f32_mul(xv[c][0], xv[c][0]);
#pragma unroll
    for (int i = 1; i < 8; ++i) s = f32_add(s, f32_mul(xv[c][i], xv[c][i]));
    a[c] = (g0 + c < G) ? s : kNegZero;
  }
  float v = local_tree<C>(a);
#pragma unroll
  for (int o = 1; o < 64; o *= 2) v = f32_add(v, __shfl_xor(v, o, 64));
  if (W == 1) return v;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  if (lane == 0) red[wave] = v;
  __syncthreads();
  float w[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) w[i] = i < W ? red[i] : kNegZero;
  // W is a power of two <= 16: the same adjacent-pairs tree over the wave sums
  for (int h = 1; h < W; h *= 2)
    for (int i = 0; i < W; i += 2 * h) w[i] = f32_add(w[i], w[i + h]);
  __syncthreads();
  return w[0];
}

LSK_DEV void load_group(const NormArgs& p, int64_t m, int64_t grp, float* v) {
  const int64_t k0 = grp * 8;
  if (p.x_dtype == LSK_BF16) {
    const uint4 u = *(const uint4*)((const uint16_t*)p.x + m * p.ldx + k0);
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      v[2 * j] = bf16_to_f32((uint16_t)(w[j] & 0xffff));
      v[2 * j + 1] = bf16_to_f32((uint16_t)(w[j] >> 16));
    }
  } else {
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = load_as_f32(p.x, p.x_dtype, m * p.ldx + k0 + j);
  }
}

// One row per block of W waves (blockDim.x = 64 W); lane l of wave w holds groups
// (w * 64 + l) * C .. + C - 1.
template <int C>
__global__ __launch_bounds__(1024) void rmsnorm_float_kernel(NormArgs p, int vec) {
  __shared__ float red[16];
  __shared__ float redq[16];
  const int64_t m = blockIdx.x;
  const int W = blockDim.x >> 6;
  const int64_t G = p.N / 8;
  const int64_t g0 = (int64_t)threadIdx.x * C;
  float xv[C][8];
#pragma unroll
  for (int c = 0; c < C; ++c) {
    if (g0 + c < G) {
      if (vec) load_group(p, m, g0 + c, xv[c]);
      else
#pragma unroll
        for (int j = 0; j < 8; ++j) xv[c][j] = load_as_f32(p.x, p.x_dtype, m * p.ldx + (g0 + c) * 8 + j);
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) xv[c][j] = 0.0f;
    }
  }
  float S = row_tree<C>(xv, g0, G, red, W);
  if (p.S && threadIdx.x == 0) p.S[m] = S;
  if (p.has_eps) S = f32_add(S, p.ne);
  S = (S < 0x1p-126f) ? 0x1p-126f : S;  // clamp(min=2^-126); a NaN sum stays NaN, as torch's clamp keeps it
  const float rs = f32_div(p.sN, __builtin_sqrtf(S));
  float amax = 0.0f;
#pragma unroll
  for (int c = 0; c < C; ++c) {
    const int64_t grp = g0 + c;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      float y = f32_mul(xv[c][j], rs);
      if (p.g && grp < G) y = f32_mul(y, load_as_f32(p.g, p.g_dtype, grp * 8 + j));
      y = bfr(y);
      xv[c][j] = y;
      if (grp < G) amax = fmaxf(amax, fabsf(y));
    }
    if (grp < G && p.out) {
      const int64_t o = m * p.ldo + grp * 8;
      if (vec && p.out_dtype == LSK_BF16) {
        uint4 u;
        u.x = (uint32_t)f32_to_bf16(xv[c][0]) | ((uint32_t)f32_to_bf16(xv[c][1]) << 16);
        u.y = (uint32_t)f32_to_bf16(xv[c][2]) | ((uint32_t)f32_to_bf16(xv[c][3]) << 16);
        u.z = (uint32_t)f32_to_bf16(xv[c][4]) | ((uint32_t)f32_to_bf16(xv[c][5]) << 16);
        u.w = (uint32_t)f32_to_bf16(xv[c][6]) | ((uint32_t)f32_to_bf16(xv[c][7]) << 16);
        store16_split((uint16_t*)p.out + o, u.x, u.y, u.z, u.w);
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) store_out(p.out, p.out_dtype, o + j, xv[c][j]);
      }
    }
  }
  if (!p.q) return;
  // the contract row quant of the bf16 outputs (max is exact and order-free)
  amax = wave_fmax(amax);
  if (W > 1) {
    if ((threadIdx.x & 63) == 0) redq[threadIdx.x >> 6] = amax;
    __syncthreads();
    amax = redq[0];
    for (int i = 1; i < W; ++i) amax = fmaxf(amax, redq[i]);
  }
  const float s = f32_div(fmaxf(amax, kAmaxFloor), 127.0f), rcp = f32_div(1.0f, s);
  if (threadIdx.x == 0) p.asc[m] = s;
#pragma unroll
  for (int c = 0; c < C; ++c) {
    const int64_t grp = g0 + c;
    if (grp >= G) continue;
    uint32_t lo = 0, hi = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      float t = rint_div8(xv[c][j], s, rcp);
      t = fminf(fmaxf(t, -127.0f), 127.0f);
      const uint32_t b = (uint32_t)(uint8_t)(int8_t)(int)t;
      if (j < 4) lo |= b << (8 * j);
      else hi |= b << (8 * (j - 4));
    }
    int8_t* qp = p.q + m * p.ldq + grp * 8;
    if (vec) {
      *(uint2*)qp = make_uint2(lo, hi);
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) qp[j] = (int8_t)((j < 4 ? lo >> (8 * j) : hi >> (8 * (j - 4))) & 0xff);
    }
  }
}

// The pinned tree over given leaves v [R, n] (t16n_ref.tree_sum): one row per block of W waves,
// C leaves per lane, padded with -0.
template <int C>
__global__ __launch_bounds__(1024) void tree_sum_kernel(const float* __restrict__ v, int64_t ldv, int64_t n,
                                                        float* __restrict__ out) {
  __shared__ float red[16];
  const int64_t m = blockIdx.x;
  const int W = blockDim.x >> 6;
  const int64_t i0 = (int64_t)threadIdx.x * C;
  float a[C];
#pragma unroll
  for (int c = 0; c < C; ++c) a[c] = (i0 + c < n) ? v[m * ldv + i0 + c] : kNegZero;
  float s = local_tree<C>(a);
#pragma unroll
  for (int o = 1; o < 64; o *= 2) s = f32_add(s, __shfl_xor(s, o, 64));
  if (W > 1) {
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
    __syncthreads();
    float w[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) w[i] = i < W ? red[i] : kNegZero;
    for (int h = 1; h < W; h *= 2)
      for (int i = 0; i < W; i += 2 * h) w[i] = f32_add(w[i], w[i + h]);
    s = w[0];
  }
  if (threadIdx.x == 0) out[m] = s;
}

int64_t next_pow2(int64_t n) {
  int64_t p = 1;
  while (p < n) p *= 2;
  return p;
}

// Waves per row and leaves per lane for `leaves` leaves: C <= 8 leaves per lane, W <= 16 waves.
bool tree_shape(int64_t leaves, int& W, int& C) {
  const int64_t P = next_pow2(leaves < 1 ? 1 : leaves);
  int64_t w = P / (64 * 8);
  if (w < 1) w = 1;
  if (w > 16) return false;
  W = (int)w;
  int64_t c = P / (64 * w);
  C = (int)(c < 1 ? 1 : c);
  return C <= 8;
}

}  // namespace

extern "C" int lsk_rmsnorm_float(const void* x, int x_dtype, int64_t ldx, int64_t R, int64_t N, const void* g,
                                 int g_dtype, float sN, double eps, void* out, int out_dtype, int64_t ldo, int8_t* q,
                                 int64_t ldq, float* asc, float* S, void* stream) {
  LSK_REQUIRE(R >= 0 && N >= 0, "lsk_rmsnorm_float: negative size");
  LSK_REQUIRE(N % 8 == 0, "lsk_rmsnorm_float: N=%lld is not a multiple of 8", (long long)N);
  LSK_REQUIRE(x_dtype == LSK_F32 || x_dtype == LSK_BF16 || x_dtype == LSK_F16, "lsk_rmsnorm_float: x dtype %d", x_dtype);
  LSK_REQUIRE(!g || g_dtype == LSK_F32 || g_dtype == LSK_BF16 || g_dtype == LSK_F16, "lsk_rmsnorm_float: gain dtype");
  LSK_REQUIRE(!out || out_dtype == LSK_BF16 || out_dtype == LSK_F32 || out_dtype == LSK_F16,
              "lsk_rmsnorm_float: out dtype %d", out_dtype);
  LSK_REQUIRE(!q || asc, "lsk_rmsnorm_float: the fused quant needs asc");
  if (R == 0 || N == 0) return LSK_OK;
  LSK_REQUIRE(x && (out || q || S), "lsk_rmsnorm_float: null input or no output");
  LSK_REQUIRE(ldx >= N && (!out || ldo >= N) && (!q || ldq >= N), "lsk_rmsnorm_float: leading dimension below N");
  LSK_REQUIRE(R <= 0x7fffffff, "lsk_rmsnorm_float: too many rows");
  int W, C;
  LSK_REQUIRE(tree_shape(N / 8, W, C), "lsk_rmsnorm_float: N=%lld above 65536", (long long)N);
  NormArgs p{x, x_dtype, ldx, R, N, g, g_dtype, sN, 0.0f, 0, out, out_dtype, ldo, q, ldq, asc, S};
  if (!(sN > 0.0f)) p.sN = (float)__builtin_sqrt((double)N);  // the width constant fl32(sqrt(N))
  if (eps != 0.0) {
    p.ne = (float)((double)N * eps);  // one binary64 product, one rounding
    p.has_eps = 1;
  }
  const int esz = x_dtype == LSK_F32 ? 4 : 2;
  const int vec = (((uintptr_t)x % 16) == 0 && (ldx * esz) % 16 == 0 && (!out || ((uintptr_t)out % 16 == 0 &&
                   (ldo * 2) % 16 == 0)) && (!q || ((uintptr_t)q % 8 == 0 && ldq % 8 == 0))) ? 1 : 0;
  hipStream_t s = (hipStream_t)stream;
#define LSK_NORM(CV) hipLaunchKernelGGL(rmsnorm_float_kernel<CV>, dim3((unsigned)R), dim3(64 * W), 0, s, p, vec)
  switch (C) {
    case 1: LSK_NORM(1); break;
    case 2: LSK_NORM(2); break;
    case 4: LSK_NORM(4); break;
    default: LSK_NORM(8); break;
  }
#undef LSK_NORM
  return lsk::check_launch("rmsnorm_float_kernel");
}

extern "C" int lsk_tree_sum(const float* v, int64_t ldv, int64_t R, int64_t n, float* out, void* stream) {
  LSK_REQUIRE(R >= 0 && n >= 1, "lsk_tree_sum: bad size (n must be at least 1)");
  if (R == 0) return LSK_OK;
  LSK_REQUIRE(v && out && ldv >= n && R <= 0x7fffffff, "lsk_tree_sum: bad pointer or stride");
  int W, C;
  LSK_REQUIRE(tree_shape(n, W, C), "lsk_tree_sum: n=%lld above 65536", (long long)n);
  hipStream_t s = (hipStream_t)stream;
#define LSK_TREE(CV) hipLaunchKernelGGL(tree_sum_kernel<CV>, dim3((unsigned)R), dim3(64 * W), 0, s, v, ldv, n, out)
  switch (C) {
    case 1: LSK_TREE(1); break;
    case 2: LSK_TREE(2); break;
    case 4: LSK_TREE(4); break;
    default: LSK_TREE(8); break;
  }
#undef LSK_TREE
  return lsk::check_launch("tree_sum_kernel");
}
