// Elementwise contract operators exposed on their own (the reference's separate calls):
// the table activations, the router's table scores, and the R1/R4 block butterfly.
#include "contract_act.h"

namespace {

__global__ __launch_bounds__(256) void act_kernel(const float* __restrict__ g, const float* __restrict__ u, int64_t n,
                                                  int op, const int32_t* __restrict__ frac, float* __restrict__ out) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
    const float x = g[i];
    float y;
    switch (op) {
      case LSK_OP_SILU: y = lsk::silu_contract(x, frac); break;
      case LSK_OP_SIGMOID: y = lsk::sigmoid_contract(x, frac); break;
      case LSK_OP_ACT_SILU: y = lsk::act_silu(x, u[i], frac); break;
      default: y = lsk::act_swigluoai(x, u[i], frac); break;
    }
    out[i] = y;
  }
}

// The activation's gate table over the 65536 bf16 bit patterns (contract_act.h).
__global__ __launch_bounds__(256) void act_table_kernel(const int32_t* __restrict__ frac, int act,
                                                        float* __restrict__ tab) {
  const uint32_t i = blockIdx.x * 256 + threadIdx.x;
  tab[i] = lsk::act_table_entry(act, i, frac);
}

// moe_ref.py:64-74
__global__ __launch_bounds__(256) void table_scores_kernel(const float* __restrict__ dgap, int64_t n,
                                                           const int32_t* __restrict__ tab, int64_t* __restrict__ out) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
    const float v = rintf(f32_mul(dgap[i], 0x1.715476p+26f));
    int64_t s = 0;
    if (v < 1073741824.0f) {
      const int d = v > 0.0f ? (int)v : 0;
      s = tab[(d >> 13) & 8191] >> (d >> 26);
    }
    out[i] = s;
  }
}

// lockstep_fullstack.py:533-546: per blk-wide block, pairs (i, i + h) -> (a + b, a - b) for
// h = 1, 2, ..., blk / 2 in binary32, then one multiply by `scale`.  One block per (row, block).
__global__ __launch_bounds__(512) void fwht_kernel(const float* __restrict__ x, int64_t ldx, int nb, int blk,
                                                   float scale, float* __restrict__ y, int64_t ldy) {
  __shared__ float v[1024];
  const int64_t row = blockIdx.x / nb;
  const int b = blockIdx.x - (int)(row * nb);
  const float* src = x + row * ldx + (int64_t)b * blk;
  for (int i = threadIdx.x; i < blk; i += blockDim.x) v[i] = src[i];
  __syncthreads();
  for (int h = 1; h < blk; h <<= 1) {
    for (int i = threadIdx.x; i < blk / 2; i += blockDim.x) {
      const int grp = i / h, off = i - grp * h;
      const int i0 = grp * 2 * h + off, i1 = i0 + h;
      const float a = v[i0], c = v[i1];
      v[i0] = f32_add(a, c);
      v[i1] = a - c;
    }
    __syncthreads();
  }
  float* dst = y + row * ldy + (int64_t)b * blk;
  for (int i = threadIdx.x; i < blk; i += blockDim.x) dst[i] = f32_mul(v[i], scale);
}

unsigned grid_for(int64_t n) {
  int64_t b = (n + 255) / 256;
  return (unsigned)(b > 8192 ? 8192 : (b < 1 ? 1 : b));
}

}  // namespace

extern "C" int lsk_act_elementwise(const float* g, const float* u, int64_t n, int op, const int32_t* frac, float* out,
                                   void* stream) {
  LSK_REQUIRE(n >= 0, "lsk_act_elementwise: negative size");
  LSK_REQUIRE(op >= LSK_OP_SILU && op <= LSK_OP_ACT_SWIGLUOAI, "lsk_act_elementwise: unknown op %d", op);
  if (n == 0) return LSK_OK;
  LSK_REQUIRE(g && frac && out && (u || op < LSK_OP_ACT_SILU), "lsk_act_elementwise: null pointer");
  hipLaunchKernelGGL(act_kernel, dim3(grid_for(n)), dim3(256), 0, (hipStream_t)stream, g, u, n, op, frac, out);
  return lsk::check_launch("act_kernel");
}

extern "C" int lsk_table_scores(const float* dgap, int64_t n, const int32_t* tab, int64_t* out, void* stream) {
  LSK_REQUIRE(n >= 0, "lsk_table_scores: negative size");
  if (n == 0) return LSK_OK;
  LSK_REQUIRE(dgap && tab && out, "lsk_table_scores: null pointer");
  hipLaunchKernelGGL(table_scores_kernel, dim3(grid_for(n)), dim3(256), 0, (hipStream_t)stream, dgap, n, tab, out);
  return lsk::check_launch("table_scores_kernel");
}

extern "C" int lsk_fwht_blocks(const float* x, int64_t rows, int64_t D, int64_t ldx, int blk, float scale, float* y,
                               int64_t ldy, void* stream) {
  LSK_REQUIRE(rows >= 0 && D >= 0, "lsk_fwht_blocks: negative size");
  LSK_REQUIRE(blk >= 2 && blk <= 1024 && (blk & (blk - 1)) == 0, "lsk_fwht_blocks: blk=%d not a power of two in [2, 1024]",
              blk);
  LSK_REQUIRE(D % blk == 0, "lsk_fwht_blocks: D=%lld not a multiple of blk=%d", (long long)D, blk);
  LSK_REQUIRE(ldx >= D && ldy >= D, "lsk_fwht_blocks: leading dimension below D");
  const int64_t nb = D / blk;
  if (rows == 0 || nb == 0) return LSK_OK;
  LSK_REQUIRE(x && y, "lsk_fwht_blocks: null pointer");
  LSK_REQUIRE(rows * nb <= 0x7fffffff, "lsk_fwht_blocks: too many blocks");
  const int threads = blk / 2 < 64 ? 64 : blk / 2;
  hipLaunchKernelGGL(fwht_kernel, dim3((unsigned)(rows * nb)), dim3(threads), 0, (hipStream_t)stream, x, ldx, (int)nb, blk,
                     scale, y, ldy);
  return lsk::check_launch("fwht_kernel");
}

extern "C" int lsk_act_table(const int32_t* frac, int act, float* table, void* stream) {
  LSK_REQUIRE(act == LSK_ACT_SILU || act == LSK_ACT_SWIGLUOAI, "lsk_act_table: unknown act %d", act);
  LSK_REQUIRE(frac && table, "lsk_act_table: null pointer");
  hipLaunchKernelGGL(act_table_kernel, dim3(65536 / 256), dim3(256), 0, (hipStream_t)stream, frac, act, table);
  return lsk::check_launch("act_table_kernel");
}
