// Activation quantisers: the contract's per-row int8 quant (true-division scale) and the
// power-of-two quantisers of the golden training block.
#include <hip/hip_cooperative_groups.h>

#include <atomic>

#include "lsk_common.h"
#include "pp_tile.h"

namespace lsk {
int launch_gemm(const int8_t* a, int64_t lda, const int8_t* w, int64_t ldw, int64_t M, int64_t N, int64_t K,
                const EpiParams& ep, hipStream_t s);
bool gemm_takes_pp(const int8_t* w, int64_t ldw, int64_t M, int64_t N, int64_t K, int64_t lda);
bool gemm_takes_skinny(const int8_t* w, int64_t ldw, int64_t M, int64_t N, int64_t K, int64_t lda);
}  // namespace lsk

namespace {

// Block-wide max of non-negative floats; every thread gets the result.
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

// One block per row.  Pass 1: amax over the row (exact, order-free).  Pass 2: quantise.
// Vector path: 8 elements per thread-step when the row is 16-byte aligned and K % 8 == 0.
template <int THREADS>
__global__ __launch_bounds__(THREADS) void rowquant_kernel(const void* __restrict__ x, int dtype,
                                                           int64_t K, int64_t ldx,
                                                           int8_t* __restrict__ q, int64_t ldq,
                                                           float* __restrict__ asc, int vec) {
  __shared__ float red[THREADS / 64];
  const int64_t m = blockIdx.x;
  const int tid = threadIdx.x;
  const int64_t base = m * ldx;
  float am = 0.0f;
  if (vec) {
    const int64_t K8 = K >> 3;
    for (int64_t c = tid; c < K8; c += THREADS) {
      if (dtype == LSK_F32) {
        const float4* p = (const float4*)((const float*)x + base) + 2 * c;
        float4 a = p[0], b = p[1];
        am = fmaxf(am, fmaxf(fmaxf(fabsf(a.x), fabsf(a.y)), fmaxf(fabsf(a.z), fabsf(a.w))));
        am = fmaxf(am, fmaxf(fmaxf(fabsf(b.x), fabsf(b.y)), fmaxf(fabsf(b.z), fabsf(b.w))));
      } else {
        const uint4 u = ((const uint4*)((const uint16_t*)x + base))[c];
        const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          float lo, hi;
          if (dtype == LSK_BF16) {
            lo = bf16_to_f32((uint16_t)(w[j] & 0xffff));
            hi = bf16_to_f32((uint16_t)(w[j] >> 16));
          } else {
            lo = (float)__builtin_bit_cast(_Float16, (uint16_t)(w[j] & 0xffff));
            hi = (float)__builtin_bit_cast(_Float16, (uint16_t)(w[j] >> 16));
          }
          am = fmaxf(am, fmaxf(fabsf(lo), fabsf(hi)));
        }
      }
    }
  } else {
    for (int64_t k = tid; k < K; k += THREADS) am = fmaxf(am, fabsf(load_as_f32(x, dtype, base + k)));
  }
  am = block_max<THREADS>(am, red);
  am = fmaxf(am, kAmaxFloor);
  const float s = f32_div(am, 127.0f), rs = f32_div(1.0f, s);
  if (tid == 0) asc[m] = s;
  int8_t* qrow = q + m * ldq;
  if (vec) {
    const int64_t K8 = K >> 3;
    for (int64_t c = tid; c < K8; c += THREADS) {
      float v[8];
      if (dtype == LSK_F32) {
        const float4* p = (const float4*)((const float*)x + base) + 2 * c;
        float4 a = p[0], b = p[1];
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
        v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
      } else {
        const uint4 u = ((const uint4*)((const uint16_t*)x + base))[c];
        const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          if (dtype == LSK_BF16) {
            v[2 * j] = bf16_to_f32((uint16_t)(w[j] & 0xffff));
            v[2 * j + 1] = bf16_to_f32((uint16_t)(w[j] >> 16));
          } else {
            v[2 * j] = (float)__builtin_bit_cast(_Float16, (uint16_t)(w[j] & 0xffff));
            v[2 * j + 1] = (float)__builtin_bit_cast(_Float16, (uint16_t)(w[j] >> 16));
          }
        }
      }
      ((uint2*)qrow)[c] = quant8_pack(v, s, rs);
    }
  } else {
    for (int64_t k = tid; k < K; k += THREADS) qrow[k] = quant_one(load_as_f32(x, dtype, base + k), s, rs);
  }
}

// Single-pass row quant: one block per row, the row held in registers (NV chunks of 8
// elements per thread, K <= 8 * NV * THREADS), so x is read from memory once.  Same
// arithmetic as rowquant_kernel: exact amax, asc = fl32(max(amax, 1e-8) / 127), q = clamp(rint(x / asc)).
// PAIR: q in the row-pair layout of the ping-pong GEMM tiles (rows 2i and 2i+1 interleaved by
// 64-byte K chunks: element (m, k) at byte (m >> 1) * 2 ldq + (k >> 6) * 128 + (m & 1) * 64 +
// (k & 63); ldq % 64 == 0).
template <int THREADS, int NV, int DT, bool PAIR = false>
__global__ __launch_bounds__(THREADS) void rowquant_reg_kernel(const void* __restrict__ x, int64_t K, int64_t ldx,
                                                               int8_t* __restrict__ q, int64_t ldq,
                                                               float* __restrict__ asc) {
  __shared__ float red[THREADS / 64];
  const int64_t m = blockIdx.x;
  const int tid = threadIdx.x;
  const int64_t K8 = K >> 3;
  const void* row = (const char*)x + m * ldx * (DT == LSK_F32 ? 4 : 2);
  float v[NV][8];
  float am = 0.0f;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int64_t c = tid + (int64_t)j * THREADS;
    if (c < K8) {
      load8_as_f32<DT>(row, c, v[j]);
#pragma unroll
      for (int e = 0; e < 8; ++e) am = fmaxf(am, fabsf(v[j][e]));
    }
  }
  am = block_max<THREADS>(am, red);
  am = fmaxf(am, kAmaxFloor);
  const float s = f32_div(am, 127.0f), rs = f32_div(1.0f, s);
  if (tid == 0) asc[m] = s;
  int8_t* qrow = PAIR ? q + (m >> 1) * 2 * ldq + (m & 1) * 64 : q + m * ldq;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int64_t c = tid + (int64_t)j * THREADS;
    if (c < K8) {
      // 8 elements from K byte 8c: ((8c) >> 6) * 128 + (8c & 63) in the row-pair layout
      *(uint2*)(qrow + (PAIR ? (c >> 3) * 128 + (c & 7) * 8 : c * 8)) = quant8_pack(v[j], s, rs);
    }
  }
}

template <int THREADS, int NV, bool PAIR = false>
int launch_rowquant_reg(const void* x, int dt, int64_t M, int64_t K, int64_t ldx, int8_t* q, int64_t ldq, float* asc,
                        hipStream_t s) {
  if (dt == LSK_F32)
    hipLaunchKernelGGL((rowquant_reg_kernel<THREADS, NV, LSK_F32, PAIR>), dim3((unsigned)M), dim3(THREADS), 0, s, x, K,
                       ldx, q, ldq, asc);
  else if (dt == LSK_BF16)
    hipLaunchKernelGGL((rowquant_reg_kernel<THREADS, NV, LSK_BF16, PAIR>), dim3((unsigned)M), dim3(THREADS), 0, s, x,
                       K, ldx, q, ldq, asc);
  else
    hipLaunchKernelGGL((rowquant_reg_kernel<THREADS, NV, LSK_F16, PAIR>), dim3((unsigned)M), dim3(THREADS), 0, s, x, K,
                       ldx, q, ldq, asc);
  return lsk::check_launch("rowquant_reg_kernel");
}

// ---------------------------------------------------------------- power-of-two quantisers
// e = 6 - (biased_exp(m) - 127); e -= 1 if fl32(m * 2^e) > 127; e = 0 where m == 0; clip [-32, 40]
LSK_DEV int pow2_exponent(float m) {
  if (m == 0.0f) return 0;
  int e = 6 - ((int)(__float_as_uint(m) >> 23) - 127);
  // The decrement can change the clipped result only for e in [-31, 40]; there 2^e is a
  // normal binary32 and m * 2^e is exact (a power-of-two scaling of a normal number).
  if (e >= -31 && e <= 40 && f32_mul(m, pow2f(e)) > 127.0f) e -= 1;
  return e < -32 ? -32 : (e > 40 ? 40 : e);
}

LSK_DEV int8_t quant_pow2_one(float v, float scale) {
  float t = rintf(f32_mul(v, scale));
  t = fminf(fmaxf(t, -127.0f), 127.0f);
  return (int8_t)(int)t;
}

__global__ __launch_bounds__(256) void amax_cols_kernel(const float* __restrict__ x, int64_t M, int64_t K,
                                                        int64_t ldx, uint32_t* __restrict__ out) {
  const int64_t c = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (c >= K) return;
  const int64_t r0 = (int64_t)blockIdx.y * 64, r1 = r0 + 64 < M ? r0 + 64 : M;
  float am = 0.0f;
  for (int64_t r = r0; r < r1; ++r) am = fmaxf(am, fabsf(x[r * ldx + c]));
  atomicMax(out + c, __float_as_uint(am));
}

// per-column exponents from the column maxima amax_bits[K] (float bits)
__global__ __launch_bounds__(256) void quant_pow2_cols_kernel(const float* __restrict__ x, int64_t M, int64_t K,
                                                              int64_t ldx, const uint32_t* __restrict__ amax_bits,
                                                              int8_t* __restrict__ q, int64_t ldq,
                                                              int32_t* __restrict__ e_out) {
  const int64_t total = M * K;
  for (int64_t c = (int64_t)blockIdx.x * 256 + threadIdx.x; c < K; c += (int64_t)gridDim.x * 256)
    e_out[c] = pow2_exponent(__uint_as_float(amax_bits[c]));
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
    const int64_t r = i / K, c = i - r * K;
    q[r * ldq + c] = quant_pow2_one(x[r * ldx + c], pow2f(pow2_exponent(__uint_as_float(amax_bits[c]))));
  }
}

__global__ __launch_bounds__(256) void quant_pow2_rows_kernel(const float* __restrict__ x, int64_t K, int64_t ldx,
                                                              int8_t* __restrict__ q, int64_t ldq,
                                                              int32_t* __restrict__ e_out) {
  __shared__ float red[4];
  const int64_t m = blockIdx.x;
  float am = 0.0f;
  for (int64_t k = threadIdx.x; k < K; k += 256) am = fmaxf(am, fabsf(x[m * ldx + k]));
  am = block_max<256>(am, red);
  const int e = pow2_exponent(am);
  if (threadIdx.x == 0) e_out[m] = e;
  const float sc = pow2f(e);
  for (int64_t k = threadIdx.x; k < K; k += 256) q[m * ldq + k] = quant_pow2_one(x[m * ldx + k], sc);
}

// ---------------------------------------------------------------- quant8_dyn (one exponent per tensor)
// Two launches, nothing to clear beforehand (so the pair can be captured in a graph): pass 1
// writes one |x| maximum per block to partial[blockIdx.x]; pass 2 has every block reduce those
// partials (at most kDynBlocks floats, read from L2), derive the tensor exponent and quantise its
// share of the tensor.  The maximum is exact in any order, so the grid shape does not matter.
constexpr int kDynBlocks = 2048;

// Contiguous tensors ([M, K] with ldx == K) are walked as one flat array of float4s, each block
// a contiguous run of them (eight 4 KB block-wide loads in flight per step, non-temporal: the
// tensor is read twice, once per pass, and nothing else should be evicted for it); other strides
// go row by row.
constexpr int kDynUnroll = 8;

LSK_DEV float4 ld_nt(const float4* p) {
  const v4f v = __builtin_nontemporal_load((const v4f*)p);
  return make_float4(v[0], v[1], v[2], v[3]);
}

LSK_DEV void block_run(int64_t n, int64_t& b0, int64_t& b1) {
  const int64_t per = (n + gridDim.x - 1) / gridDim.x;
  b0 = (int64_t)blockIdx.x * per;
  b1 = b0 + per < n ? b0 + per : n;
}

template <bool NT = true>
__global__ __launch_bounds__(256) void dyn_amax_kernel(const float* __restrict__ x, int64_t M, int64_t K,
                                                       int64_t ldx, int flat, float* __restrict__ partial) {
  auto ld = [](const float4* p) {
    if constexpr (NT) return ld_nt(p);
    return *p;
  };
  __shared__ float red[4];
  float am = 0.0f;
  if (flat) {
    const int64_t n4 = (M * K) >> 2;
    const float4* x4 = (const float4*)x;
    int64_t b0, b1;
    block_run(n4, b0, b1);
    int64_t i = b0 + threadIdx.x;
    for (; i + 256 * (kDynUnroll - 1) < b1; i += 256 * kDynUnroll) {
      float4 v[kDynUnroll];
#pragma unroll
      for (int u = 0; u < kDynUnroll; ++u) v[u] = ld(x4 + i + 256 * u);
#pragma unroll
      for (int u = 0; u < kDynUnroll; ++u)
        am = fmaxf(am, fmaxf(fmaxf(fabsf(v[u].x), fabsf(v[u].y)), fmaxf(fabsf(v[u].z), fabsf(v[u].w))));
    }
    for (; i < b1; i += 256) {
      const float4 v = ld(x4 + i);
      am = fmaxf(am, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
    }
    if (blockIdx.x == gridDim.x - 1)
      for (int64_t j = (n4 << 2) + threadIdx.x; j < M * K; j += 256) am = fmaxf(am, fabsf(x[j]));
  } else {
    for (int64_t r = blockIdx.x; r < M; r += gridDim.x)
      for (int64_t c = threadIdx.x; c < K; c += 256) am = fmaxf(am, fabsf(x[r * ldx + c]));
  }
  am = block_max<256>(am, red);
  if (threadIdx.x == 0) partial[blockIdx.x] = am;
}

LSK_DEV uint32_t quant_pow2_x4(float4 v, float sc) {
  return (uint32_t)(uint8_t)quant_pow2_one(v.x, sc) | ((uint32_t)(uint8_t)quant_pow2_one(v.y, sc) << 8) |
         ((uint32_t)(uint8_t)quant_pow2_one(v.z, sc) << 16) | ((uint32_t)(uint8_t)quant_pow2_one(v.w, sc) << 24);
}

__global__ __launch_bounds__(256) void dyn_quant_kernel(const float* __restrict__ x, int64_t M, int64_t K,
                                                        int64_t ldx, int flat, const float* __restrict__ partial,
                                                        int nparts, int8_t* __restrict__ q, int64_t ldq,
                                                        int32_t* __restrict__ e_out, int32_t* __restrict__ erow) {
  __shared__ float red[4];
  float am = 0.0f;
  for (int j = threadIdx.x; j < nparts; j += 256) am = fmaxf(am, partial[j]);
  am = block_max<256>(am, red);
  const int e = pow2_exponent(am);   // 0 for an all-zero tensor, whose q is then 0 as well
  const float sc = pow2f(e);         // e in [-32, 40]: a normal power of two
  const int64_t stride = (int64_t)gridDim.x * 256;
  if (blockIdx.x == 0 && threadIdx.x == 0) e_out[0] = e;
  if (erow)
    for (int64_t r = (int64_t)blockIdx.x * 256 + threadIdx.x; r < M; r += stride) erow[r] = e;
  if (flat) {
    // pairs of float4 (eight elements, one 8-byte store of q), each block a contiguous run
    const int64_t n8 = (M * K) >> 3;
    const float4* x4 = (const float4*)x;
    int64_t b0, b1;
    block_run(n8, b0, b1);
    int64_t i = b0 + threadIdx.x;
    constexpr int U = kDynUnroll / 2;
    for (; i + 256 * (U - 1) < b1; i += 256 * U) {
      float4 v[U][2];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        v[u][0] = ld_nt(x4 + 2 * (i + 256 * u));
        v[u][1] = ld_nt(x4 + 2 * (i + 256 * u) + 1);
      }
#pragma unroll
      for (int u = 0; u < U; ++u)
        *(v2u32*)(q + 8 * (i + 256 * u)) = v2u32{quant_pow2_x4(v[u][0], sc), quant_pow2_x4(v[u][1], sc)};
    }
    for (; i < b1; i += 256) {
      const float4 a = ld_nt(x4 + 2 * i), b = ld_nt(x4 + 2 * i + 1);
      *(v2u32*)(q + 8 * i) = v2u32{quant_pow2_x4(a, sc), quant_pow2_x4(b, sc)};
    }
    if (blockIdx.x == gridDim.x - 1)
      for (int64_t j = (n8 << 3) + threadIdx.x; j < M * K; j += 256) q[j] = quant_pow2_one(x[j], sc);
  } else {
    for (int64_t r = blockIdx.x; r < M; r += gridDim.x)
      for (int64_t c = threadIdx.x; c < K; c += 256) q[r * ldq + c] = quant_pow2_one(x[r * ldx + c], sc);
  }
}

// Pass 2 of quant8_dyn writing q in the row-pair layout the ping-pong GEMM tiles read (rows 2i
// and 2i+1 interleaved by 64-byte K chunks: element (m, k) at byte (m >> 1) * 2 ldq + (k >> 6) *
// 128 + (m & 1) * 64 + (k & 63); ldq % 64 == 0, K % 8 == 0, x rows 16-byte aligned).  A block
// takes whole row pairs; thread t writes 8-byte items t, t + 256, ... of the pair's 2 ldq bytes
// (contiguous stores), each from 8 consecutive elements of one x row.  Bytes past K (and the
// second row of a last pair when M is odd) are written as 0 and never read.
__global__ __launch_bounds__(256) void dyn_quant_pair_kernel(const float* __restrict__ x, int64_t M, int64_t K,
                                                             int64_t ldx, const float* __restrict__ partial,
                                                             int nparts, int8_t* __restrict__ q, int64_t ldq,
                                                             int32_t* __restrict__ e_out,
                                                             int32_t* __restrict__ erow) {
  __shared__ float red[4];
  const int64_t npair = (M + 1) >> 1;
  const int per = (int)(ldq >> 2);  // 8-byte items per row pair
  constexpr int U = 4;
  // the loads of one step: every load issued before the first use, none under a branch (a lane
  // without an element reads its pair's first row start and discards it)
  auto load_step = [&](int64_t p, int r0, float4 (&v)[U][2], bool (&ok)[U]) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int o = (r0 + 256 * u) * 8;
      const int64_t m = 2 * p + ((o >> 6) & 1);
      const int64_t k = (int64_t)(o >> 7) * 64 + (o & 63);
      ok[u] = r0 + 256 * u < per && m < M && k < K;
      const float4* src = (const float4*)(x + (ok[u] ? m * ldx + k : 2 * p * ldx));
      v[u][0] = ld_nt(src);
      v[u][1] = ld_nt(src + 1);
    }
  };
  // the block's first step requested before the partial maxima are reduced (it does not depend on
  // the exponent), so the reduction's latency overlaps the first loads
  float4 v0[U][2];
  bool ok0[U];
  const bool first = (int64_t)blockIdx.x < npair && (int)threadIdx.x < per;
  if (first) load_step(blockIdx.x, threadIdx.x, v0, ok0);
  float am = 0.0f;
  for (int j = threadIdx.x; j < nparts; j += 256) am = fmaxf(am, partial[j]);
  am = block_max<256>(am, red);
  const int e = pow2_exponent(am);
  const float sc = pow2f(e);
  if (blockIdx.x == 0 && threadIdx.x == 0) e_out[0] = e;
  if (erow)
    for (int64_t r = (int64_t)blockIdx.x * 256 + threadIdx.x; r < M; r += (int64_t)gridDim.x * 256) erow[r] = e;
  for (int64_t p = blockIdx.x; p < npair; p += gridDim.x) {
    int8_t* qp = q + p * 2 * ldq;
    for (int r0 = threadIdx.x; r0 < per; r0 += 256 * U) {
      float4 v[U][2];
      bool ok[U];
      if (p == (int64_t)blockIdx.x && r0 == (int)threadIdx.x) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
          v[u][0] = v0[u][0];
          v[u][1] = v0[u][1];
          ok[u] = ok0[u];
        }
      } else {
        load_step(p, r0, v, ok);
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if (r0 + 256 * u >= per) continue;
        v2u32 out = v2u32{0u, 0u};
        if (ok[u]) out = v2u32{quant_pow2_x4(v[u][0], sc), quant_pow2_x4(v[u][1], sc)};
        *(v2u32*)(qp + (int64_t)(r0 + 256 * u) * 8) = out;
      }
    }
  }
}

// Pass 2 of quant8_dyn into the row-pair layout for a contiguous tensor with no padding bytes
// (ldx == ldq == K, K % 64 == 0, M even, M K < 2^31), walked in the order of q: unit f is q bytes
// 4 f .. 4 f + 3, which (q byte o = p 2K + c 128 + r 64 + j: row pair p, K chunk c, row 2p + r,
// column 64 c + j) come from one float4 of x.  Each block takes a contiguous run of units, lane-
// contiguous, so a wave's store covers 256 contiguous bytes of q (two whole 128-byte lines, both
// rows of a pair) and its load four 256-byte runs of x (a chunk of each row of the pair, twice).
// Every load of a step is issued before any is used, none under a branch (a lane past the run
// re-reads the run's first float4 and stores nothing).
constexpr int kDynU2 = 8;

template <bool NT>
__global__ __launch_bounds__(256) void dyn_quant_pair_flat_kernel(const float* __restrict__ x, int64_t M, int64_t K,
                                                                  const float* __restrict__ partial, int nparts,
                                                                  int8_t* __restrict__ q, int32_t* __restrict__ e_out,
                                                                  int32_t* __restrict__ erow) {
  __shared__ float red[4];
  const int n4 = (int)((M * K) >> 2);
  const int per = (n4 + (int)gridDim.x - 1) / (int)gridDim.x;
  const int b0 = (int)blockIdx.x * per, b1 = min(b0 + per, n4);
  const float4* x4 = (const float4*)x;
  const int K2 = 2 * (int)K;
  // q byte 4 f as (row pair pp, offset rem in the pair's 2K bytes); each step of 256 units adds 1024
  const int f0 = b0 + (int)threadIdx.x;
  int pp = (4 * f0) / K2, rem = 4 * f0 - pp * K2;
  const int dp = 1024 / K2, drem = 1024 - dp * K2;
  auto src = [&](int f, int p, int r) {
    // element (2p + (r >> 6 & 1), 64 (r >> 7) + (r & 63)) of x, as a float4 index
    const int e = (2 * p + ((r >> 6) & 1)) * (int)K + 64 * (r >> 7) + (r & 63);
    return x4 + (f < b1 ? (e >> 2) : b0);
  };
  auto load = [&](const float4* p) {
    if constexpr (NT) return ld_nt(p);
    return *p;
  };
  int lp[kDynU2], lr[kDynU2];
  auto addrs = [&]() {
#pragma unroll
    for (int u = 0; u < kDynU2; ++u) {
      lp[u] = pp;
      lr[u] = rem;
      pp += dp;
      rem += drem;
      if (rem >= K2) {
        rem -= K2;
        ++pp;
      }
    }
  };
  // the first step requested before the partial maxima are reduced (it does not depend on them)
  float4 v[kDynU2];
  int f = f0;
  if (b0 < b1) {
    addrs();
#pragma unroll
    for (int u = 0; u < kDynU2; ++u) v[u] = load(src(f + 256 * u, lp[u], lr[u]));
  }
  float am = 0.0f;
  for (int j = threadIdx.x; j < nparts; j += 256) am = fmaxf(am, partial[j]);
  am = block_max<256>(am, red);
  const int e = pow2_exponent(am);
  const float sc = pow2f(e);
  if (blockIdx.x == 0 && threadIdx.x == 0) e_out[0] = e;
  if (erow)
    for (int64_t r = (int64_t)blockIdx.x * 256 + threadIdx.x; r < M; r += (int64_t)gridDim.x * 256) erow[r] = e;
  if (b0 >= b1) return;
  uint32_t* q4 = (uint32_t*)q;
  for (;;) {
#pragma unroll
    for (int u = 0; u < kDynU2; ++u)
      if (f + 256 * u < b1) q4[f + 256 * u] = quant_pow2_x4(v[u], sc);
    f += 256 * kDynU2;
    if (f >= b1) break;
    addrs();
#pragma unroll
    for (int u = 0; u < kDynU2; ++u) v[u] = load(src(f + 256 * u, lp[u], lr[u]));
  }
}

// Single-pass quant8_dyn into the row-pair layout for a tensor that fits on chip (a cooperative
// launch: every block resident, one grid-wide barrier).  Block b holds the contiguous run of
// 256 * (kQ1Regs + kQ1Lds) float4s from b * 256 * (kQ1Regs + kQ1Lds): step j of thread t is float4
// run + 256 j + t, kQ1Regs steps in registers and kQ1Lds in LDS (direct-to-LDS loads), so x is read
// from memory once, each block from one contiguous run.  Each block writes its |x| maximum to
// partial[block]; after the barrier every block reduces the G partials, derives the tensor exponent
// (pow2_exponent) and quantises its float4s from registers and LDS into q (element (m, k) at
// (m >> 1) 2 ldq + (k >> 6) 128 + (m & 1) 64 + (k & 63)).  Needs ldx == K, K % 64 == 0 (no padding
// bytes), M even, M K < 2^31 and M K <= G * 256 * (kQ1Regs + kQ1Lds) * 4.  Same exponent and q as
// the two-pass kernels: the maximum is exact in any order.
constexpr int kQ1Regs = 19, kQ1Lds = 9;

__global__ __launch_bounds__(256, 4) void dyn_quant1_pair_kernel(const float* __restrict__ x, int64_t M, int64_t K,
                                                                float* __restrict__ partial, int8_t* __restrict__ q,
                                                                int64_t ldq, int32_t* __restrict__ e_out,
                                                                int32_t* __restrict__ erow) {
  constexpr int NT = kQ1Regs + kQ1Lds;
  __shared__ __attribute__((aligned(16))) char xs[kQ1Lds * 4096];  // [step][wave][lane] 16 bytes each
  __shared__ float red[4];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int n4 = (int)((M * K) >> 2);
  const int i0 = (int)blockIdx.x * 256 * NT + tid;  // float4 of step 0
  const float4* x4 = (const float4*)x;
  const __amdgpu_buffer_rsrc_t rx = lsk::make_rsrc(x, (int64_t)n4 * 16);
  float4 r[kQ1Regs];
#pragma unroll
  for (int j = 0; j < kQ1Regs; ++j) {
    const int i = i0 + 256 * j;
    r[j] = i < n4 ? ld_nt(x4 + i) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  }
#pragma unroll
  for (int j = 0; j < kQ1Lds; ++j) {
    const int i = i0 + 256 * (kQ1Regs + j);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, (lsk::lds_void_t)(xs + (j * 4 + wave) * 1024), 16,
                                             i < n4 ? (uint32_t)i * 16u : lsk::kOob, 0, 0, 0);
  }
  float am = 0.0f;
#pragma unroll
  for (int j = 0; j < kQ1Regs; ++j)
    am = fmaxf(am, fmaxf(fmaxf(fabsf(r[j].x), fabsf(r[j].y)), fmaxf(fabsf(r[j].z), fabsf(r[j].w))));
  lsk::wait_vm<0>();
  __syncthreads();
#pragma unroll
  for (int j = 0; j < kQ1Lds; ++j) {
    const float4 v = *(const float4*)(xs + (j * 4 + wave) * 1024 + lane * 16);
    am = fmaxf(am, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
  }
  am = block_max<256>(am, red);
  if (tid == 0) partial[blockIdx.x] = am;
  cooperative_groups::this_grid().sync();
  float m = 0.0f;
  for (int j = tid; j < (int)gridDim.x; j += 256) m = fmaxf(m, partial[j]);
  m = block_max<256>(m, red);
  const int e = pow2_exponent(m);
  const float sc = pow2f(e);
  if (blockIdx.x == 0 && tid == 0) e_out[0] = e;
  if (erow)
    for (int64_t rr = (int64_t)blockIdx.x * 256 + tid; rr < M; rr += (int64_t)gridDim.x * 256) erow[rr] = e;
  // element 4 i of x is (row mr, column kc); each step adds 1024 elements (dm rows + dk columns)
  const int Ki = (int)K;
  int mr = (4 * i0) / Ki, kc = (4 * i0) - mr * Ki;
  const int dm = 1024 / Ki, dk = 1024 - dm * Ki;
  auto put = [&](float4 v) {
    *(uint32_t*)(q + (int64_t)(mr >> 1) * 2 * ldq + (kc >> 6) * 128 + (mr & 1) * 64 + (kc & 63)) = quant_pow2_x4(v, sc);
  };
  auto advance = [&]() {
    mr += dm;
    kc += dk;
    if (kc >= Ki) {
      kc -= Ki;
      ++mr;
    }
  };
#pragma unroll
  for (int j = 0; j < kQ1Regs; ++j) {
    if (i0 + 256 * j < n4) put(r[j]);
    advance();
  }
#pragma unroll
  for (int j = 0; j < kQ1Lds; ++j) {
    if (i0 + 256 * (kQ1Regs + j) < n4) put(*(const float4*)(xs + (j * 4 + wave) * 1024 + lane * 16));
    advance();
  }
}

// w [N, K] int8 (row stride ldw) into the row-pair layout (row stride (K + 63) / 64 * 64 per row of
// a pair): one 16-byte chunk of the output per thread and step (two 8-byte stores); bytes past K,
// and the second row of a last pair when N is odd, are 0.  K % 16 == 0.
__global__ __launch_bounds__(256) void pack_row_pairs_kernel(const int8_t* __restrict__ w, int64_t N, int64_t K,
                                                             int64_t ldw, int8_t* __restrict__ out) {
  const int64_t kp = (K + 63) / 64 * 64;
  const int64_t chunks = ((N + 1) >> 1) * 2 * kp / 16;
  for (int64_t c = (int64_t)blockIdx.x * 256 + threadIdx.x; c < chunks; c += (int64_t)gridDim.x * 256) {
    const int64_t o = c * 16;
    const int64_t p = o / (2 * kp), r = o - p * 2 * kp;
    const int64_t n = 2 * p + ((r >> 6) & 1), k = (r >> 7) * 64 + (r & 63);
    uint4 v = make_uint4(0u, 0u, 0u, 0u);
    if (n < N && k < K) v = *(const uint4*)(w + n * ldw + k);
    store16_split(out + o, v.x, v.y, v.z, v.w);
  }
}

__global__ __launch_bounds__(256) void fill_u32_kernel(uint32_t* __restrict__ p, int64_t n, uint32_t v) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) p[i] = v;
}

// Launches of quant8_dyn on a workspace of kDynBlocks floats.
int launch_quant8_dyn(const float* x, int64_t M, int64_t K, int64_t ldx, int8_t* q, int64_t ldq, int32_t* e_out,
                      int32_t* erow, float* partial, hipStream_t s) {
  const int64_t total = M * K;
  const int flat = (ldx == K && ldq == K && ((uintptr_t)x % 16) == 0 && ((uintptr_t)q % 8) == 0) ? 1 : 0;
  int64_t blocks = flat ? (total + 256 * 16 - 1) / (256 * 16) : M;
  blocks = blocks < 1 ? 1 : (blocks > kDynBlocks ? kDynBlocks : blocks);
  hipLaunchKernelGGL(dyn_amax_kernel<true>, dim3((unsigned)blocks), dim3(256), 0, s, x, M, K, ldx, flat, partial);
  int rc = lsk::check_launch("dyn_amax_kernel");
  if (rc) return rc;
  hipLaunchKernelGGL(dyn_quant_kernel, dim3((unsigned)blocks), dim3(256), 0, s, x, M, K, ldx, flat,
                     (const float*)partial, (int)blocks, q, ldq, e_out, erow);
  return lsk::check_launch("dyn_quant_kernel");
}

// quant8_dyn in one pass where the tensor fits on chip: off by default.  Measured on MI355X
// (ROCm 7.2, Qwen2.5-7B block at 8192 rows, alternating on one box): 171-178 us per 117 MB
// activation against 60-65 us for the two passes (maxima 20 us, quantise 33 us); the cooperative
// launch and its grid barrier cost more than the second read of x saves.
thread_local int g_quant1 = 0;

// Pass 2 of the row-pair quant8_dyn: 0 row pairs per block; 1 (the default) the walk in the order
// of q (non-temporal loads in both passes); 2 as 1 with ordinary loads in both passes.  Measured on
// MI355X (Qwen2.5-7B block at 8192 rows, both passes): 117 MB of x 51.7 / 45.7 / 41.2 us and 620 MB
// 248 / 228 / 274 us alone; in the block step the sites' quant 450 / 418 / 486 us in all (2 takes
// the second pass from the Infinity Cache alone, but loses it to the GEMMs between the sites).
thread_local int g_dynq = 1;

// Blocks of the single-pass kernel that the device keeps resident at once (four per CU when its
// registers and LDS allow), cached per device; 0 when the device cannot launch it cooperatively.
static int quant1_blocks() {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  int n = cache[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    int coop = 0, cus = 0, per = 0;
    if (hipDeviceGetAttribute(&coop, hipDeviceAttributeCooperativeLaunch, dev) != hipSuccess || !coop ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, dyn_quant1_pair_kernel, 256, 0) != hipSuccess)
      n = -1;
    else
      n = per >= 4 ? 4 * cus : -1;
    cache[dev].store(n, std::memory_order_relaxed);
  }
  return n > 0 ? (n > kDynBlocks ? kDynBlocks : n) : 0;
}

// quant8_dyn into the row-pair layout (ldq % 64 == 0, K % 8 == 0, x rows 16-byte aligned).
int launch_quant8_dyn_pair(const float* x, int64_t M, int64_t K, int64_t ldx, int8_t* q, int64_t ldq, int32_t* e_out,
                           int32_t* erow, float* partial, hipStream_t s) {
  const int64_t total = M * K;
  // one pass when the tensor fits on chip and the stream is not being captured (a cooperative
  // launch is not captured into graphs)
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  int G = 0;
  if (g_quant1 && ldx == K && K % 64 == 0 && M % 2 == 0 && ldq == K && total < (int64_t)1 << 31 &&
      ((uintptr_t)x % 16) == 0 && ((uintptr_t)q % 4) == 0 && hipStreamIsCapturing(s, &cap) == hipSuccess &&
      cap == hipStreamCaptureStatusNone && (G = quant1_blocks()) > 0 &&
      total <= (int64_t)G * 256 * (kQ1Regs + kQ1Lds) * 4) {
    void* args[] = {(void*)&x, (void*)&M, (void*)&K, (void*)&partial, (void*)&q, (void*)&ldq, (void*)&e_out,
                    (void*)&erow};
    if (hipLaunchCooperativeKernel((const void*)dyn_quant1_pair_kernel, dim3((unsigned)G), dim3(256), args, 0, s) !=
        hipSuccess)
      return lsk::set_error("quant8_dyn: cooperative launch failed: %s", hipGetErrorString(hipGetLastError())),
             LSK_ERR_HIP;
    return LSK_OK;
  }
  const int flat = (ldx == K && ((uintptr_t)x % 16) == 0) ? 1 : 0;
  int64_t blocks = flat ? (total + 256 * 16 - 1) / (256 * 16) : M;
  blocks = blocks < 1 ? 1 : (blocks > kDynBlocks ? kDynBlocks : blocks);
  const bool nt = g_dynq != 2;
  if (nt)
    hipLaunchKernelGGL(dyn_amax_kernel<true>, dim3((unsigned)blocks), dim3(256), 0, s, x, M, K, ldx, flat, partial);
  else
    hipLaunchKernelGGL(dyn_amax_kernel<false>, dim3((unsigned)blocks), dim3(256), 0, s, x, M, K, ldx, flat, partial);
  int rc = lsk::check_launch("dyn_amax_kernel");
  if (rc) return rc;
  if (g_dynq && flat && ldq == K && K % 64 == 0 && M % 2 == 0 && total < (int64_t)1 << 31 && ((uintptr_t)q % 4) == 0) {
    int64_t fb = (total / 4 + 256 * kDynU2 * 2 - 1) / (256 * kDynU2 * 2);
    fb = fb < 1 ? 1 : (fb > kDynBlocks ? kDynBlocks : fb);
    if (nt)
      hipLaunchKernelGGL(dyn_quant_pair_flat_kernel<true>, dim3((unsigned)fb), dim3(256), 0, s, x, M, K,
                         (const float*)partial, (int)blocks, q, e_out, erow);
    else
      hipLaunchKernelGGL(dyn_quant_pair_flat_kernel<false>, dim3((unsigned)fb), dim3(256), 0, s, x, M, K,
                         (const float*)partial, (int)blocks, q, e_out, erow);
    return lsk::check_launch("dyn_quant_pair_flat_kernel");
  }
  int64_t qblocks = (M + 1) / 2;
  qblocks = qblocks < 1 ? 1 : (qblocks > kDynBlocks ? kDynBlocks : qblocks);
  hipLaunchKernelGGL(dyn_quant_pair_kernel, dim3((unsigned)qblocks), dim3(256), 0, s, x, M, K, ldx,
                     (const float*)partial, (int)blocks, q, ldq, e_out, erow);
  return lsk::check_launch("dyn_quant_pair_kernel");
}

// Workspace of lsk_linear_dyn: the quant8_dyn partial maxima, the per-row exponents and q
// (rows rounded up to a pair, K up to a multiple of 64), each 256-byte aligned.
struct LinDynWs {
  int64_t partial, erow, q, bytes;
};
LinDynWs lindyn_layout(int64_t M, int64_t K) {
  auto up = [](int64_t v) { return (v + 255) / 256 * 256; };
  LinDynWs l;
  l.partial = 0;
  l.erow = up((int64_t)kDynBlocks * 4);
  l.q = l.erow + up(M * 4);
  l.bytes = l.q + up(((M + 1) & ~(int64_t)1) * ((K + 63) / 64 * 64));
  return l;
}

}  // namespace

namespace lsk {
// Whether rowquant_pair can quantise x (the single-pass register kernels: K % 8 == 0, K <= 32768,
// 16-byte aligned rows).
bool rowquant_pair_ok(const void* x, int x_dtype, int64_t ldx, int64_t K) {
  const int esz = x_dtype == LSK_F32 ? 4 : 2;
  return K > 0 && K % 8 == 0 && K <= 32768 && ldx % 8 == 0 && ((uintptr_t)x % 16) == 0 && ((ldx * esz) % 16) == 0 &&
         (x_dtype == LSK_F32 || x_dtype == LSK_BF16 || x_dtype == LSK_F16);
}

// The contract's per-row int8 quant (as lsk_rowquant) with q in the row-pair layout (ldq % 64 == 0).
int rowquant_pair(const void* x, int x_dtype, int64_t M, int64_t K, int64_t ldx, int8_t* q, int64_t ldq, float* asc,
                  hipStream_t s) {
  LSK_REQUIRE(rowquant_pair_ok(x, x_dtype, ldx, K) && ldq % 64 == 0 && ldq >= K && ((uintptr_t)q % 64) == 0 &&
                  M <= 0x7fffffff,
              "rowquant_pair: unsupported operand (K=%lld ldx=%lld ldq=%lld)", (long long)K, (long long)ldx,
              (long long)ldq);
  if (M == 0) return LSK_OK;
  const int64_t K8 = K >> 3;
  if (K8 <= 256) return launch_rowquant_reg<256, 1, true>(x, x_dtype, M, K, ldx, q, ldq, asc, s);
  if (K8 <= 512) return launch_rowquant_reg<256, 2, true>(x, x_dtype, M, K, ldx, q, ldq, asc, s);
  if (K8 <= 1024) return launch_rowquant_reg<256, 4, true>(x, x_dtype, M, K, ldx, q, ldq, asc, s);
  if (K8 <= 2048) return launch_rowquant_reg<512, 4, true>(x, x_dtype, M, K, ldx, q, ldq, asc, s);
  return launch_rowquant_reg<512, 8, true>(x, x_dtype, M, K, ldx, q, ldq, asc, s);
}
}  // namespace lsk

extern "C" int64_t lsk_quant8_dyn_workspace(void) { return (int64_t)kDynBlocks * sizeof(float); }

extern "C" int64_t lsk_linear_dyn_workspace(int64_t M, int64_t K) {
  if (M < 0 || K < 0) return -1;
  return lindyn_layout(M, K).bytes;
}

extern "C" int64_t lsk_row_pairs_bytes(int64_t N, int64_t K) {
  if (N < 0 || K < 0) return -1;
  return ((N + 1) & ~(int64_t)1) * ((K + 63) / 64 * 64);
}

extern "C" int lsk_pack_row_pairs(const int8_t* w, int64_t N, int64_t K, int64_t ldw, int8_t* out, void* stream) {
  LSK_REQUIRE(N >= 0 && K >= 0 && ldw >= K, "lsk_pack_row_pairs: bad sizes N=%lld K=%lld ldw=%lld", (long long)N,
              (long long)K, (long long)ldw);
  LSK_REQUIRE(K % 16 == 0 && ldw % 16 == 0, "lsk_pack_row_pairs: K and ldw must be multiples of 16");
  if (N == 0 || K == 0) return LSK_OK;
  LSK_REQUIRE(w && out && ((uintptr_t)w % 16) == 0 && ((uintptr_t)out % 16) == 0,
              "lsk_pack_row_pairs: null or unaligned pointer");
  const int64_t chunks = lsk_row_pairs_bytes(N, K) / 16;
  int64_t blocks = (chunks + 255) / 256;
  blocks = blocks > 8192 ? 8192 : blocks;
  hipLaunchKernelGGL(pack_row_pairs_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, w, N, K, ldw,
                     out);
  return lsk::check_launch("pack_row_pairs_kernel");
}

extern "C" int lsk_gemm_reads_row_pairs(int64_t M, int64_t N, int64_t K) {
  // the question lsk_w8a8_matmul and lsk_linear_dyn ask of a 16-byte aligned weight copy whose
  // rows are kp bytes apart, with the calling thread's tile selection
  if (M <= 0 || N <= 0 || K <= 0 || K % 16 != 0) return 0;
  const int64_t kp = (K + 63) / 64 * 64;
  return (lsk::gemm_takes_pp((const int8_t*)(uintptr_t)256, kp, M, N, K, kp) ||
          lsk::gemm_takes_skinny((const int8_t*)(uintptr_t)256, kp, M, N, K, (K + 15) / 16 * 16))
             ? 1
             : 0;
}

extern "C" int lsk_quant8_dyn_variant(int v) {
  LSK_REQUIRE(v >= 0 && v <= 2, "lsk_quant8_dyn_variant: %d not in [0, 2]", v);
  g_dynq = v;
  return LSK_OK;
}

extern "C" int lsk_quant8_dyn_single_pass(int on) {
  LSK_REQUIRE(on == 0 || on == 1, "lsk_quant8_dyn_single_pass: %d not 0 or 1", on);
  g_quant1 = on;
  return LSK_OK;
}

extern "C" int lsk_linear_dyn(const float* x, int64_t M, int64_t K, int64_t ldx, const int8_t* w, int64_t ldw,
                              const int8_t* w_pairs, int64_t N, int ew, float* y, int64_t ldy, int32_t* ex_out,
                              int stages, void* workspace, int64_t workspace_bytes, void* stream) {
  LSK_REQUIRE(stages >= 1 && stages <= 3, "lsk_linear_dyn: stages=%d not 1, 2 or 3", stages);
  LSK_REQUIRE(M >= 0 && N >= 0 && K >= 0, "lsk_linear_dyn: negative size M=%lld N=%lld K=%lld", (long long)M,
              (long long)N, (long long)K);
  LSK_REQUIRE(K <= 133144, "lsk_linear_dyn: K=%lld exceeds the int32-exact bound 133144", (long long)K);
  LSK_REQUIRE(ldx >= K && ldw >= K && ldy >= N, "lsk_linear_dyn: leading dimension too small");
  LSK_REQUIRE(ex_out || !(stages & 1), "lsk_linear_dyn: ex_out is required");
  const LinDynWs l = lindyn_layout(M, K);
  LSK_REQUIRE(workspace && workspace_bytes >= l.bytes && ((uintptr_t)workspace & 255) == 0,
              "lsk_linear_dyn: workspace of %lld bytes (256-byte aligned) required (%lld given)", (long long)l.bytes,
              (long long)workspace_bytes);
  LSK_REQUIRE(M * K == 0 || (x && w), "lsk_linear_dyn: null pointer");
  LSK_REQUIRE(M * N == 0 || y, "lsk_linear_dyn: null pointer");
  hipStream_t s = (hipStream_t)stream;
  char* ws = (char*)workspace;
  float* partial = (float*)(ws + l.partial);
  int32_t* erow = (int32_t*)(ws + l.erow);
  int8_t* q = (int8_t*)(ws + l.q);
  // the row-pair layout when every tile of the GEMM is a ping-pong tile; row-major otherwise
  const int64_t kp = (K + 63) / 64 * 64;
  const bool pair = M > 0 && N > 0 && K > 0 && K % 8 == 0 && ldx % 4 == 0 && ((uintptr_t)x % 16) == 0 &&
                    lsk::gemm_takes_pp(w, ldw, M, N, K, kp);
  const int64_t ldq = pair ? kp : (K + 15) / 16 * 16;
  if (stages & 1) {
    const int rc = pair ? launch_quant8_dyn_pair(x, M, K, ldx, q, ldq, ex_out, erow, partial, s)
                        : launch_quant8_dyn(x, M, K, ldx, q, ldq, ex_out, erow, partial, s);
    if (rc) return rc;
  }
  if (!(stages & 2) || M == 0 || N == 0) return LSK_OK;
  EpiParams ep{LSK_EPI_POW2, LSK_F32, nullptr, nullptr, nullptr, erow, nullptr, ew, y, ldy};
  ep.pairs = pair ? 1 : 0;
  // the weight's row-pair copy with the quantised rows' row-pair layout
  if (pair && w_pairs && lsk::gemm_takes_pp(w_pairs, kp, M, N, K, kp)) {
    ep.pairs = 3;
    return lsk::launch_gemm(q, ldq, w_pairs, kp, M, N, K, ep, s);
  }
  // decode rows: the skinny GEMV streams the weight's row-pair copy
  if (!pair && w_pairs && lsk::gemm_takes_skinny(w_pairs, kp, M, N, K, ldq)) {
    ep.pairs = 2;
    return lsk::launch_gemm(q, ldq, w_pairs, kp, M, N, K, ep, s);
  }
  return lsk::launch_gemm(q, ldq, w, ldw, M, N, K, ep, s);
}

extern "C" int lsk_quant8_dyn(const float* x, int64_t M, int64_t K, int64_t ldx, int8_t* q, int64_t ldq,
                              int32_t* e_out, int32_t* erow_out, void* workspace, int64_t workspace_bytes,
                              void* stream) {
  LSK_REQUIRE(M >= 0 && K >= 0, "lsk_quant8_dyn: negative size M=%lld K=%lld", (long long)M, (long long)K);
  LSK_REQUIRE(ldx >= K && ldq >= K, "lsk_quant8_dyn: ldx=%lld / ldq=%lld below K=%lld", (long long)ldx,
              (long long)ldq, (long long)K);
  LSK_REQUIRE(e_out, "lsk_quant8_dyn: e_out is required");
  LSK_REQUIRE(workspace && workspace_bytes >= lsk_quant8_dyn_workspace(),
              "lsk_quant8_dyn: workspace of %lld bytes required (%lld given)", (long long)lsk_quant8_dyn_workspace(),
              (long long)workspace_bytes);
  LSK_REQUIRE(M * K == 0 || (x && q), "lsk_quant8_dyn: null pointer");
  return launch_quant8_dyn(x, M, K, ldx, q, ldq, e_out, erow_out, (float*)workspace, (hipStream_t)stream);
}

extern "C" int lsk_rowquant(const void* x, int x_dtype, int64_t M, int64_t K, int64_t ldx, int8_t* q,
                            int64_t ldq, float* asc, void* stream) {
  LSK_REQUIRE(M >= 0 && K >= 0, "lsk_rowquant: negative size M=%lld K=%lld", (long long)M, (long long)K);
  LSK_REQUIRE(x_dtype == LSK_F32 || x_dtype == LSK_BF16 || x_dtype == LSK_F16,
              "lsk_rowquant: x_dtype %d not one of f32/bf16/f16", x_dtype);
  if (M == 0) return LSK_OK;
  LSK_REQUIRE(x && q && asc, "lsk_rowquant: null pointer");
  LSK_REQUIRE(ldx >= K && ldq >= K, "lsk_rowquant: ldx=%lld / ldq=%lld below K=%lld", (long long)ldx,
              (long long)ldq, (long long)K);
  LSK_REQUIRE(M <= 0x7fffffff, "lsk_rowquant: M=%lld exceeds the grid", (long long)M);
  const int esz = x_dtype == LSK_F32 ? 4 : 2;
  const int vec = (K % 8 == 0) && (ldx % 8 == 0) && (ldq % 8 == 0) && ((uintptr_t)x % 16 == 0) &&
                  ((uintptr_t)q % 8 == 0) && ((ldx * esz) % 16 == 0);
  hipStream_t s = (hipStream_t)stream;
  if (vec) {
    // single pass with the row in registers: chunks of 8 elements per thread
    const int64_t K8 = K >> 3;
    if (K8 <= 256) return launch_rowquant_reg<256, 1>(x, x_dtype, M, K, ldx, q, ldq, asc, s);
    if (K8 <= 512) return launch_rowquant_reg<256, 2>(x, x_dtype, M, K, ldx, q, ldq, asc, s);
    if (K8 <= 1024) return launch_rowquant_reg<256, 4>(x, x_dtype, M, K, ldx, q, ldq, asc, s);
    if (K8 <= 2048) return launch_rowquant_reg<512, 4>(x, x_dtype, M, K, ldx, q, ldq, asc, s);
    if (K8 <= 4096) return launch_rowquant_reg<512, 8>(x, x_dtype, M, K, ldx, q, ldq, asc, s);
  }
  hipLaunchKernelGGL(rowquant_kernel<256>, dim3((unsigned)M), dim3(256), 0, s, x, x_dtype, K, ldx, q, ldq, asc, vec);
  return lsk::check_launch("rowquant_kernel");
}

extern "C" int lsk_quant8_pow2(const float* x, int64_t M, int64_t K, int64_t ldx, int mode, int8_t* q,
                               int64_t ldq, int32_t* e_out, void* workspace, void* stream) {
  LSK_REQUIRE(M >= 0 && K >= 0, "lsk_quant8_pow2: negative size");
  LSK_REQUIRE(mode >= 0 && mode <= 2, "lsk_quant8_pow2: mode %d not in {0,1,2}", mode);
  LSK_REQUIRE(ldx >= K && ldq >= K, "lsk_quant8_pow2: leading dimension below K");
  hipStream_t s = (hipStream_t)stream;
  if (mode == 1) {
    if (M == 0) return LSK_OK;
    LSK_REQUIRE(M <= 0x7fffffff, "lsk_quant8_pow2: M too large");
    hipLaunchKernelGGL(quant_pow2_rows_kernel, dim3((unsigned)M), dim3(256), 0, s, x, K, ldx, q, ldq, e_out);
    return lsk::check_launch("quant_pow2_rows_kernel");
  }
  LSK_REQUIRE(workspace, "lsk_quant8_pow2: workspace required");
  if (mode == 0) {
    // the workspace (4 * (M + K + 64) bytes) holds the partial maxima of every grid quant8_dyn
    // launches for this size
    return launch_quant8_dyn(x, M, K, ldx, q, ldq, e_out, nullptr, (float*)workspace, s);
  }
  uint32_t* amax = (uint32_t*)workspace;
  if (K > 0) {
    // column maxima are integer atomics on the float bits: clear them with a kernel (no memset
    // node if the caller captures this into a graph)
    int64_t fb = (K + 255) / 256;
    hipLaunchKernelGGL(fill_u32_kernel, dim3((unsigned)(fb > 1024 ? 1024 : fb)), dim3(256), 0, s, amax, K, 0u);
    int rc = lsk::check_launch("fill_u32_kernel");
    if (rc) return rc;
  }
  if (M > 0 && K > 0) {
    dim3 g((unsigned)((K + 255) / 256), (unsigned)((M + 63) / 64));
    hipLaunchKernelGGL(amax_cols_kernel, g, dim3(256), 0, s, x, M, K, ldx, amax);
    int rc = lsk::check_launch("amax kernel");
    if (rc) return rc;
  }
  int64_t blocks = (M * K + 255) / 256;
  if (blocks < 1) blocks = 1;
  if (blocks > 4096) blocks = 4096;
  hipLaunchKernelGGL(quant_pow2_cols_kernel, dim3((unsigned)blocks), dim3(256), 0, s, x, M, K, ldx, amax, q, ldq,
                     e_out);
  return lsk::check_launch("quant_pow2_cols_kernel");
}
