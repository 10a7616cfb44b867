// The int8 MFMA ceiling of the part, for the bench's roofline context: a register-only loop of
// v_mfma_i32_32x32x32_i8 on operands the caller provides (constant or uniformly random int8), no
// memory traffic inside the loop.  The sustained rate on random operands is what the power budget
// lets the GEMM kernels reach at most; on constant operands it approaches the nominal peak.
#include "lsk_common.h"
#include "mfma_tile.h"
#include "mx_tile.h"

namespace {

// Each wave keeps four independent accumulators (four MFMAs in flight hide the MFMA latency)
// and two operand pairs per accumulator, loaded once from ops (16 bytes per lane per operand).
__global__ __launch_bounds__(256) void mfma_probe_kernel(const v4i* __restrict__ ops, int64_t nops, int iters,
                                                         int32_t* __restrict__ sink) {
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  v4i a[4], b[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    a[j] = ops[(t * 8 + 2 * j) % nops];
    b[j] = ops[(t * 8 + 2 * j + 1) % nops];
  }
  v16i c[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) c[j] = v16i{};
  for (int i = 0; i < iters; ++i) {
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int j = 0; j < 4; ++j) c[j] = lsk::mfma_i8_32(a[(j + r) & 3], b[j], c[j]);
  }
  int s = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int e = 0; e < 16; ++e) s += c[j][e];
  sink[t] = s;
}

// Every binary32 pattern start .. start + count - 1: gfx950's packed bf16 conversion
// (pack_bf16x2_nonan, both halves, patterns that are not NaN) and the library's f32_to_bf16 and
// pack_bf16x2 (every pattern, NaN included) against the round-to-nearest-even bit method
// (f32_to_bf16_bits).
// Disagreements are counted (integer atomics) and the smallest such pattern kept.
__global__ __launch_bounds__(256) void bf16_cvt_check_kernel(uint64_t start, uint64_t count,
                                                             uint32_t* __restrict__ mismatches,
                                                             uint32_t* __restrict__ first) {
  uint32_t bad = 0, lo = 0xffffffffu;
  for (uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x; i < count; i += (uint64_t)gridDim.x * 256) {
    const uint32_t u = (uint32_t)(start + i);
    const float f = __uint_as_float(u), g = __uint_as_float(u ^ 0x80000000u);
    const bool nan = (u & 0x7fffffffu) > 0x7f800000u;  // excluded by pack_bf16x2_nonan's contract
    const uint32_t sw = (uint32_t)f32_to_bf16_bits(f) | ((uint32_t)f32_to_bf16_bits(g) << 16);
    const uint32_t hw = nan ? sw : pack_bf16x2_nonan(f, g);
    const uint32_t lib = (uint32_t)f32_to_bf16(f) | ((uint32_t)f32_to_bf16(g) << 16);
    if (hw != sw || lib != sw || pack_bf16x2(f, g) != sw) {
      ++bad;
      lo = u < lo ? u : lo;
    }
  }
  if (bad) {
    atomicAdd(mismatches, bad);
    atomicMin(first, lo);
  }
}

// One v_mfma_f32_16x16x32_bf16 per case with the caller's accumulator input: D = A B^T + C over
// K = 32 (one MX block).  Case c: a [16][32] and b [16][32] bf16 (rows M / N, K contiguous), cin and
// d [16][16] binary32 (row M, column N).  Lane l supplies row l % 16 of A and of B at K elements
// 8 (l / 16) .. 8 (l / 16) + 7; register r of lane l holds D row 4 (l / 16) + r, column l % 16.
// Four cases per 256-thread block; the grid covers ncases exactly.
__global__ __launch_bounds__(256) void mfma_bf16_acc_kernel(const uint16_t* __restrict__ a,
                                                            const uint16_t* __restrict__ b,
                                                            const float* __restrict__ cin, float* __restrict__ d,
                                                            int ncases) {
  const int c = blockIdx.x * 4 + (int)(threadIdx.x >> 6);
  if (c >= ncases) return;
  const int l = threadIdx.x & 63, row = l & 15, kg = l >> 4;
  const v4i av = *(const v4i*)(a + (int64_t)c * 512 + row * 32 + 8 * kg);
  const v4i bv = *(const v4i*)(b + (int64_t)c * 512 + row * 32 + 8 * kg);
  v4f acc;
#pragma unroll
  for (int r = 0; r < 4; ++r) acc[r] = cin[(int64_t)c * 256 + (4 * kg + r) * 16 + row];
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(lsk::v8bf, av), __builtin_bit_cast(lsk::v8bf, bv),
                                                acc, 0, 0, 0);
#pragma unroll
  for (int r = 0; r < 4; ++r) d[(int64_t)c * 256 + (4 * kg + r) * 16 + row] = acc[r];
}

}  // namespace

extern "C" int lsk_mfma_bf16_acc_probe(const uint16_t* a, const uint16_t* b, const float* cin, float* d, int ncases,
                                       void* stream) {
  LSK_REQUIRE(a && b && cin && d && ncases > 0 && ncases <= (1 << 24), "lsk_mfma_bf16_acc_probe: bad arguments");
  LSK_REQUIRE(((uintptr_t)a & 15) == 0 && ((uintptr_t)b & 15) == 0, "lsk_mfma_bf16_acc_probe: a, b 16-byte aligned");
  hipLaunchKernelGGL(mfma_bf16_acc_kernel, dim3((unsigned)((ncases + 3) / 4)), dim3(256), 0, (hipStream_t)stream, a, b,
                     cin, d, ncases);
  return lsk::check_launch("mfma_bf16_acc_kernel");
}

extern "C" int lsk_bf16_cvt_check(uint64_t start, uint64_t count, uint32_t* mismatches, uint32_t* first,
                                  void* stream) {
  LSK_REQUIRE(mismatches && first && count > 0 && start + count <= (1ull << 32),
              "lsk_bf16_cvt_check: bad arguments");
  hipLaunchKernelGGL(bf16_cvt_check_kernel, dim3(8192), dim3(256), 0, (hipStream_t)stream, start, count, mismatches,
                     first);
  return lsk::check_launch("bf16_cvt_check_kernel");
}

extern "C" int lsk_mfma_probe(const void* ops, int64_t nops, int64_t blocks, int iters, int32_t* sink, void* stream) {
  LSK_REQUIRE(ops && sink && nops > 0 && blocks > 0 && blocks <= 65536 && iters > 0,
              "lsk_mfma_probe: bad arguments");
  hipLaunchKernelGGL(mfma_probe_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, (const v4i*)ops,
                     nops, iters, sink);
  return lsk::check_launch("mfma_probe_kernel");
}
