// Shared device helpers for the contract GEMM kernels (gfx950 only).
//
// Every binary32 operation in an epilogue must be one IEEE operation rounded to nearest
// even, in the declared order.  The build passes -ffp-contract=off; the pragma below makes
// the sources safe under any flag set, so no multiply and add are ever fused into an FMA.
#pragma once
#pragma clang fp contract(off)

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "lockstep_amd.h"

#define LSK_DEV __device__ __forceinline__

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef short v8s __attribute__((ext_vector_type(8)));
typedef unsigned int v2u32 __attribute__((ext_vector_type(2)));
typedef unsigned int v4u32 __attribute__((ext_vector_type(4)));

// Index of the calling wave in its block, as a wave-uniform (scalar) value: the compiler cannot
// prove threadIdx.x / 64 uniform by itself, and treats code that depends on it as divergent.
LSK_DEV int wave_id() { return __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)); }

// A 64-bit value the caller knows to be equal in every lane (an entry of a per-block table, say)
// moved to scalar registers.  Without it a buffer resource built from such a pointer can end up
// in vector registers, and every load through it is wrapped in a loop over distinct resources.
LSK_DEV int64_t wave_uniform64(int64_t v) {
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)v);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)((uint64_t)v >> 32));
  return (int64_t)(((uint64_t)hi << 32) | lo);
}

// Wave-wide reductions by DPP row moves: two quad swaps and the half-row and row mirrors leave
// each row's total in all 16 of its lanes, the row broadcasts 15 and 31 carry rows 0-2 into row 3,
// and lane 63's total is returned as a wave-uniform value.  Lanes of the rows a broadcast does not
// write keep their value (the identity is passed as the DPP "old" operand).  Six VALU steps and a
// readlane, against six LDS-crossbar round trips for a __shfl_xor butterfly.  Every lane of the
// wave must be active.
template <class Op>
LSK_DEV uint32_t wave_reduce_dpp(uint32_t v, uint32_t ident, Op op) {
  v = op(v, (uint32_t)__builtin_amdgcn_update_dpp((int)ident, (int)v, 0xb1, 0xf, 0xf, false));   // quad [1,0,3,2]
  v = op(v, (uint32_t)__builtin_amdgcn_update_dpp((int)ident, (int)v, 0x4e, 0xf, 0xf, false));   // quad [2,3,0,1]
  v = op(v, (uint32_t)__builtin_amdgcn_update_dpp((int)ident, (int)v, 0x141, 0xf, 0xf, false));  // half-row mirror
  v = op(v, (uint32_t)__builtin_amdgcn_update_dpp((int)ident, (int)v, 0x140, 0xf, 0xf, false));  // row mirror
  v = op(v, (uint32_t)__builtin_amdgcn_update_dpp((int)ident, (int)v, 0x142, 0xa, 0xf, false));  // row bcast 15
  v = op(v, (uint32_t)__builtin_amdgcn_update_dpp((int)ident, (int)v, 0x143, 0xc, 0xf, false));  // row bcast 31
  return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}
LSK_DEV uint32_t wave_max_u32(uint32_t v) {
  return wave_reduce_dpp(v, 0u, [](uint32_t a, uint32_t b) { return a > b ? a : b; });
}
LSK_DEV int wave_sum_i32(int v) {
  return (int)wave_reduce_dpp((uint32_t)v, 0u, [](uint32_t a, uint32_t b) { return (uint32_t)((int)a + (int)b); });
}
// fmaxf over the wave (a NaN lane is passed over as fmaxf passes it; -inf is the identity).
LSK_DEV float wave_fmax(float v) {
  return __uint_as_float(wave_reduce_dpp(__float_as_uint(v), 0xff800000u, [](uint32_t a, uint32_t b) {
    return __float_as_uint(fmaxf(__uint_as_float(a), __uint_as_float(b)));
  }));
}

// binary32 -> bf16, round to nearest even; every NaN becomes 0x7FC0 (the conversion torch's
// c10::BFloat16 performs, which is what the reference's `.to(torch.bfloat16)` runs).
// binary32 -> bf16 by the round-to-nearest-even bit method torch uses, every NaN to 0x7FC0: the
// definition the conversions below are checked against.
LSK_DEV uint16_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0;
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

LSK_DEV float bf16_to_f32(uint16_t b) { return __uint_as_float(((uint32_t)b) << 16); }

// Two binary32 values to packed bf16 (a in the low half) with gfx950's conversion instruction:
// round to nearest even, denormals kept; equal to f32_to_bf16_bits for every binary32 that is
// not a NaN (checked exhaustively over all 2^32 patterns on MI355X).  NaN inputs are the
// caller's to exclude.
typedef float v2f_t __attribute__((ext_vector_type(2)));
typedef __bf16 v2bf16_t __attribute__((ext_vector_type(2)));
LSK_DEV uint32_t pack_bf16x2_nonan(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((v2f_t){a, b}, v2bf16_t));
}

// binary32 -> bf16, equal to f32_to_bf16_bits for every input (checked over all 2^32 patterns on
// MI355X): the conversion instruction, with a NaN replaced by 0x7FC0 (three VALU instructions
// against the bit method's six or seven).
LSK_DEV uint16_t f32_to_bf16(float f) {
  const uint16_t h = (uint16_t)pack_bf16x2_nonan(f, f);
  return f != f ? (uint16_t)0x7fc0 : h;
}

// Two binary32 values to packed bf16 (a in the low half), each equal to f32_to_bf16.
LSK_DEV uint32_t pack_bf16x2(float a, float b) {
  uint32_t h = pack_bf16x2_nonan(a, b);
  if (a != a) h = (h & 0xffff0000u) | 0x7fc0u;
  if (b != b) h = (h & 0xffffu) | 0x7fc00000u;
  return h;
}

// 16 bytes to global memory as two 8-byte stores.  On MI355X a 16-byte global / buffer store
// followed three to four instructions later by VALU writes to its data registers was measured to
// store the newer values, and the compiler separates the two by one wait state only; 8-byte
// stores have no such hazard.  The empty asm with a memory clobber between the halves keeps the
// load/store vectoriser from fusing them back into one 16-byte store.  p is 8-byte aligned.
LSK_DEV void store16_split(void* p, uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
  ((v2u32*)p)[0] = v2u32{a, b};
  __asm__ volatile("" ::: "memory");
  ((v2u32*)p)[1] = v2u32{c, d};
}
LSK_DEV void store16_split(void* p, v4u32 v) { store16_split(p, v[0], v[1], v[2], v[3]); }

// fl32 -> bf16 -> fl32 (one bf16 rounding, kept in binary32)
LSK_DEV float bfr(float f) { return bf16_to_f32(f32_to_bf16(f)); }

// exact 2^e for e in [-149, 127] (subnormal powers included), built from bits
LSK_DEV float pow2f(int e) {
  if (e >= -126) return __uint_as_float((uint32_t)(e + 127) << 23);
  return __uint_as_float(1u << (e + 149));
}

// The POW2 dequant factor fl32(2^-s) (ref_block_v1.py:167: F(2.0**(-e)), binary64 rounded once to
// binary32): exact for s in [-127, 149], +0 above (2^-150 and below round to zero), +inf below.
LSK_DEV float pow2_descale(int s) {
  return s > 149 ? 0.0f : (s < -127 ? __uint_as_float(0x7f800000u) : pow2f(-s));
}

LSK_DEV float f32_mul(float a, float b) { return a * b; }
LSK_DEV float f32_add(float a, float b) { return a + b; }
LSK_DEV float f32_div(float a, float b) { return a / b; }   // correctly rounded (build flag)

// rint(fl32(v / s)) for the 8-bit row quantisers, given r = fl32(1 / s); there |v / s| is about 127
// at most (|v| is at most the row maximum and s = fl32(max / 127)), and the argument holds for any
// |v / s| < 256: y = fl32(v * r) differs from v / s by at most 256 * 2^-23 = 2^-15 (two roundings of
// relative error <= 2^-24 each) and fl32(v / s) from v / s by at most half an ulp, 2^-17, so
// |y - fl32(v / s)| < 2^-14.  Unless y lies within 2^-13 of a half-integer, both therefore round to
// the same integer; only there is the division evaluated, behind a branch on the wave's ballot (a
// select would have the compiler evaluate the division for every element).  (y - floor(y) is exact for |y| < 2^23; infinities and NaNs give what the division
// gives: v * 0 for s = inf, NaN for NaN or infinite v over an infinite s.)
LSK_DEV float rint_div8(float v, float s, float r) {
  const float y = f32_mul(v, r);
  const bool near = fabsf(y - floorf(y) - 0.5f) < 0x1p-13f;
  float t = rintf(y);
  if (__builtin_amdgcn_ballot_w64(near) != 0) {
    if (near) t = rintf(f32_div(v, s));
  }
  return t;
}

// The contract's per-row int8 quant of one element: clamp(rint(fl32(x / asc)), -127, 127) with
// r = fl32(1 / asc); asc = fl32(max(amax, kAmaxFloor) / 127) over the row.
constexpr float kAmaxFloor = 0x1.5798eep-27f;  // binary32 nearest 1e-8 (torch clamp(min=1e-8))

LSK_DEV int8_t quant_one(float v, float s, float r) {
  float t = rint_div8(v, s, r);
  t = fminf(fmaxf(t, -127.0f), 127.0f);
  return (int8_t)(int)t;
}

// quant_one of eight elements, packed as int8 bytes (element e in byte e % 4 of word e / 4), in
// fewer VALU instructions: the near-half-integer test of an element is |(|y - rint(y)|) - 0.5| <
// 2^-13, the same set as rint_div8's |y - floor(y) - 0.5| < 2^-13 (with f = y - floor(y),
// |y - rint(y)| = min(f, 1 - f), and both differences are exact for |y| < 2^23, where the test is
// decided), with one ballot for the eight; the clamped value (a NaN becomes -127 through fmaxf, as
// in quant_one) plus 128 is an integer in [1, 255] that v_cvt_pk_u8_f32 writes into its byte
// exactly, and the xor with 0x80 turns that byte into the value's two's-complement byte.
LSK_DEV uint2 quant8_pack(const float (&v)[8], float s, float r) {
  float t[8];
  bool near = false;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float y = f32_mul(v[e], r);
    t[e] = rintf(y);
    near |= fabsf(fabsf(y - t[e]) - 0.5f) < 0x1p-13f;
  }
  if (__builtin_amdgcn_ballot_w64(near) != 0) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float y = f32_mul(v[e], r);
      if (fabsf(fabsf(y - t[e]) - 0.5f) < 0x1p-13f) t[e] = rintf(f32_div(v[e], s));
    }
  }
  uint32_t w[2] = {0, 0};
#pragma unroll
  for (int e = 0; e < 8; ++e)
    w[e >> 2] = __builtin_amdgcn_cvt_pk_u8_f32(f32_add(fminf(fmaxf(t[e], -127.0f), 127.0f), 128.0f), e & 3, w[e >> 2]);
  return make_uint2(w[0] ^ 0x80808080u, w[1] ^ 0x80808080u);
}

// Load 8 consecutive elements of dtype DT (16-byte aligned) as binary32.
template <int DT>
LSK_DEV void load8_as_f32(const void* x, int64_t i8, float* v) {
  if (DT == LSK_F32) {
    const float4* p = (const float4*)x + 2 * i8;
    const float4 a = p[0], b = p[1];
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
  } else {
    const uint4 u = ((const uint4*)x)[i8];
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (DT == LSK_BF16) {
        v[2 * j] = bf16_to_f32((uint16_t)(w[j] & 0xffff));
        v[2 * j + 1] = bf16_to_f32((uint16_t)(w[j] >> 16));
      } else {
        v[2 * j] = (float)__builtin_bit_cast(_Float16, (uint16_t)(w[j] & 0xffff));
        v[2 * j + 1] = (float)__builtin_bit_cast(_Float16, (uint16_t)(w[j] >> 16));
      }
    }
  }
}

// Load one activation element of the given dtype as binary32 (bf16 and f16 widen exactly).
LSK_DEV float load_as_f32(const void* p, int dtype, int64_t i) {
  switch (dtype) {
    case LSK_BF16: return bf16_to_f32(((const uint16_t*)p)[i]);
    case LSK_F16: return (float)(((const _Float16*)p)[i]);
    default: return ((const float*)p)[i];
  }
}

// Store binary32 `y` rounded to the output dtype.  Returns the stored value widened back to
// binary32 (what the reference's next `.float()` sees).
LSK_DEV float store_out(void* out, int dtype, int64_t i, float y) {
  switch (dtype) {
    case LSK_BF16: {
      uint16_t b = f32_to_bf16(y);
      ((uint16_t*)out)[i] = b;
      return bf16_to_f32(b);
    }
    case LSK_F16: {
      _Float16 h = (_Float16)y;
      ((_Float16*)out)[i] = h;
      return (float)h;
    }
    case LSK_BF16_AS_F32: {
      float r = bfr(y);
      ((float*)out)[i] = r;
      return r;
    }
    default:
      ((float*)out)[i] = y;
      return y;
  }
}

LSK_DEV float round_out(int dtype, float y) {
  switch (dtype) {
    case LSK_BF16:
    case LSK_BF16_AS_F32: return bfr(y);
    case LSK_F16: return (float)(_Float16)y;
    default: return y;
  }
}

// The contract epilogues, applied to one exact int32 accumulator.
//   V21  (moe_ref.py:40-42, lockstep_fullstack.py:524-527): y = fl32(fl32(acc)*ws[n])*asc[m],
//        rounded to the output type; a bias is a second rounding: out(fl32(y_out) + b[n]).
//   V2   (contract_common.py:172-174): y = fl32(fl32(acc)*asc[m])*ws[n] (+ b[n]) then one cast.
//   POW2 (ref_block_v1.py:167,193,198,218): fl32(acc) * 2^-(shift + erow[m] + ecol[n]), exact.
struct EpiParams {
  int order;                 // lsk_epilogue
  int out_dtype;             // lsk_dtype
  const float* ws;           // [N]
  const float* asc;          // [M] (indexed by the logical output row)
  const float* bias;         // [N] or null
  const int32_t* erow;       // [M] or null (POW2)
  const int32_t* ecol;       // [N] or null (POW2)
  int shift;                 // POW2 scalar
  void* out;
  int64_t ldo;               // elements
  // V25 (the v2.5 outlier side path): ho binary32 [M, ko] (row stride ko), wo [N, ko] of
  // wo_dtype (LSK_BF16 or LSK_F32, row stride ko)
  const float* ho = nullptr;
  const void* wo = nullptr;
  int ko = 0;
  int wo_dtype = LSK_BF16;
  // operand layouts (read by the ping-pong tile kernels only): bit 0 A, bit 1 B in the row-pair
  // layout -- row pairs interleaved by 64-byte K chunks, element (m, k) at byte (m >> 1) * 2 ld +
  // (k >> 6) * 128 + (m & 1) * 64 + (k & 63), ld % 64 == 0 -- instead of rows of ld bytes
  int pairs = 0;
};

// The v2.5 side term of output (m, n) (lockstep_fullstack.py:549-557): sequential in j from +0,
// each step one binary32 product and one binary32 add.
LSK_DEV float outlier_side_value(const EpiParams& p, int64_t m, int64_t n) {
  float s = 0.0f;
  const float* h = p.ho + m * p.ko;
  if (p.wo_dtype == LSK_BF16) {
    const uint16_t* w = (const uint16_t*)p.wo + n * p.ko;
    for (int j = 0; j < p.ko; ++j) s = f32_add(s, f32_mul(h[j], bf16_to_f32(w[j])));
  } else {
    const float* w = (const float*)p.wo + n * p.ko;
    for (int j = 0; j < p.ko; ++j) s = f32_add(s, f32_mul(h[j], w[j]));
  }
  return s;
}

// The V25 value of one element (lockstep_fullstack.py:575-578): bf16-valued binary32.
LSK_DEV float epi_v25(const EpiParams& p, int64_t m, int64_t n, int32_t acc) {
  float y = bfr(f32_mul(f32_mul((float)acc, p.ws[n]), p.asc[m]));
  y = bfr(f32_add(y, outlier_side_value(p, m, n)));
  if (p.bias) y = bfr(f32_add(y, p.bias[n]));
  return y;
}

LSK_DEV void epilogue_store(const EpiParams& p, int64_t m, int64_t n, int32_t acc) {
  const int64_t o = m * p.ldo + n;
  if (p.order == LSK_EPI_RAW) {
    ((int32_t*)p.out)[o] = acc;
    return;
  }
  if (p.order == LSK_EPI_V25) {
    store_out(p.out, p.out_dtype, o, epi_v25(p, m, n, acc));
    return;
  }
  const float v = (float)acc;  // int32 -> binary32, round to nearest even
  if (p.order == LSK_EPI_V21) {
    float y = f32_mul(f32_mul(v, p.ws[n]), p.asc[m]);
    if (p.bias) {
      y = round_out(p.out_dtype, y);
      y = f32_add(y, p.bias[n]);
    }
    store_out(p.out, p.out_dtype, o, y);
  } else if (p.order == LSK_EPI_V2) {
    float y = f32_mul(f32_mul(v, p.asc[m]), p.ws[n]);
    if (p.bias) y = f32_add(y, p.bias[n]);
    store_out(p.out, p.out_dtype, o, y);
  } else {  // LSK_EPI_POW2
    int s = p.shift;
    if (p.erow) s += p.erow[m];
    if (p.ecol) s += p.ecol[n];
    store_out(p.out, p.out_dtype, o, f32_mul(v, pow2_descale(s)));
  }
}

// Epilogue value of one element, before the final rounding to the output type.
LSK_DEV float epi_value(const EpiParams& p, int64_t m, int64_t n, int32_t acc) {
  if (p.order == LSK_EPI_V25) return epi_v25(p, m, n, acc);
  const float v = (float)acc;  // int32 -> binary32, round to nearest even
  if (p.order == LSK_EPI_V21) {
    float y = f32_mul(f32_mul(v, p.ws[n]), p.asc[m]);
    if (p.bias) y = f32_add(round_out(p.out_dtype, y), p.bias[n]);
    return y;
  }
  if (p.order == LSK_EPI_V2) {
    float y = f32_mul(f32_mul(v, p.asc[m]), p.ws[n]);
    if (p.bias) y = f32_add(y, p.bias[n]);
    return y;
  }
  int s = p.shift;
  if (p.erow) s += p.erow[m];
  if (p.ecol) s += p.ecol[n];
  return f32_mul(v, pow2_descale(s));
}

// Epilogue value of one element from operands already in registers: the row operand (asc[m],
// or the POW2 row exponent), the column operands (ws[n], bias[n] or 0) and, for POW2, the
// total exponent shift + erow[m] + ecol[n].  The same binary32 operations as epi_value.
LSK_DEV float epi_value_pre(int order, int out_dtype, bool has_bias, int32_t acc, float ascm, float wsn, float bn,
                            int pshift) {
  const float v = (float)acc;  // int32 -> binary32, round to nearest even
  if (order == LSK_EPI_V21) {
    float y = f32_mul(f32_mul(v, wsn), ascm);
    if (has_bias) y = f32_add(round_out(out_dtype, y), bn);
    return y;
  }
  if (order == LSK_EPI_V2) {
    float y = f32_mul(f32_mul(v, ascm), wsn);
    if (has_bias) y = f32_add(y, bn);
    return y;
  }
  return f32_mul(v, pow2_descale(pshift));
}

// The per-element epilogue operands of output (m, n), loaded ahead of the accumulator so a
// kernel's tail does not wait on them: the row operand (asc[m]), ws[n], bias[n] (0 if none),
// and for POW2 the total exponent shift + erow[m] + ecol[n].
struct EpiOps {
  float row, ws, b;
  int sh;
};

LSK_DEV EpiOps epi_ops_load(const EpiParams& p, int64_t m, int64_t n) {
  EpiOps o{0.0f, 0.0f, 0.0f, 0};
  if (p.order == LSK_EPI_V21 || p.order == LSK_EPI_V2) {
    o.row = p.asc[m];
    o.ws = p.ws[n];
    if (p.bias) o.b = p.bias[n];
  } else if (p.order == LSK_EPI_POW2) {
    o.sh = p.shift + (p.erow ? p.erow[m] : 0) + (p.ecol ? p.ecol[n] : 0);
  }
  return o;
}

// epilogue_store with the operands from epi_ops_load.
LSK_DEV void epilogue_store_ops(const EpiParams& p, int64_t m, int64_t n, int32_t acc, const EpiOps& o) {
  const int64_t off = m * p.ldo + n;
  if (p.order == LSK_EPI_V25) {
    store_out(p.out, p.out_dtype, off, epi_v25(p, m, n, acc));
    return;
  }
  if (p.order == LSK_EPI_RAW) {
    ((int32_t*)p.out)[off] = acc;
    return;
  }
  store_out(p.out, p.out_dtype, off, epi_value_pre(p.order, p.out_dtype, p.bias != nullptr, acc, o.row, o.ws, o.b, o.sh));
}

// The operands of output row m and of output column n, loaded apart so a kernel that owns a
// block of rows and columns loads each once, all ahead of its first store (loads after a store
// to memory the compiler cannot prove distinct would each wait a round trip): the row operand
// (asc[m]; POW2: shift + erow[m]) and the column operands (ws[n], bias[n] or 0; POW2: ecol[n]).
struct EpiRow {
  float row;
  int sh;
};
struct EpiCol {
  float ws, b;
  int sh;
};

LSK_DEV EpiRow epi_row_load(const EpiParams& p, int64_t m) {
  EpiRow r{0.0f, 0};
  if (p.order == LSK_EPI_V21 || p.order == LSK_EPI_V2) r.row = p.asc[m];
  else if (p.order == LSK_EPI_POW2) r.sh = p.shift + (p.erow ? p.erow[m] : 0);
  return r;
}

LSK_DEV EpiCol epi_col_load(const EpiParams& p, int64_t n) {
  EpiCol c{0.0f, 0.0f, 0};
  if (p.order == LSK_EPI_V21 || p.order == LSK_EPI_V2) {
    c.ws = p.ws[n];
    if (p.bias) c.b = p.bias[n];
  } else if (p.order == LSK_EPI_POW2) {
    c.sh = p.ecol ? p.ecol[n] : 0;
  }
  return c;
}

LSK_DEV void epilogue_store_rc(const EpiParams& p, int64_t m, int64_t n, int32_t acc, const EpiRow& r,
                               const EpiCol& c) {
  epilogue_store_ops(p, m, n, acc, EpiOps{r.row, c.ws, c.b, r.sh + c.sh});
}

// The same row and column operands as raw 32-bit words from branch-free buffer loads, for kernels
// that request them at their start and combine them only at their stores: a load whose value is
// used at once (the POW2 shift added, a branch on the order around it) makes the compiler wait for
// it there, so the operands of a short kernel would cost a round trip each.  Offsets of absent
// operands (the other orders' arrays, a null bias or exponent vector, rows / columns out of range)
// read zero.  Row m < 2^29 and column n < 2^29 (4-byte offsets inside one buffer range).
struct EpiRaw {
  __amdgpu_buffer_rsrc_t row, col0, col1;
};

LSK_DEV EpiRaw epi_raw(const EpiParams& p, int64_t M, int64_t N) {
  const bool pow2 = p.order == LSK_EPI_POW2, v2x = p.order == LSK_EPI_V21 || p.order == LSK_EPI_V2;
  const int64_t rb = (pow2 ? p.erow != nullptr : v2x) ? 4 * M : 0;
  const int64_t cb = (pow2 ? p.ecol != nullptr : v2x) ? 4 * N : 0;
  const int64_t bb = v2x && p.bias ? 4 * N : 0;
  EpiRaw r;
  r.row = __builtin_amdgcn_make_buffer_rsrc(pow2 ? (void*)p.erow : (void*)p.asc, (short)0,
                                            (int)(rb > 0x7fffffff ? 0x7fffffff : rb), 0x00020000);
  r.col0 = __builtin_amdgcn_make_buffer_rsrc(pow2 ? (void*)p.ecol : (void*)p.ws, (short)0,
                                             (int)(cb > 0x7fffffff ? 0x7fffffff : cb), 0x00020000);
  r.col1 = __builtin_amdgcn_make_buffer_rsrc((void*)p.bias, (short)0, (int)(bb > 0x7fffffff ? 0x7fffffff : bb),
                                             0x00020000);
  return r;
}

LSK_DEV uint32_t epi_raw_row(const EpiRaw& r, int64_t m, bool ok) {
  return __builtin_amdgcn_raw_buffer_load_b32(r.row, ok ? (int)(4 * m) : (int)0x80000000u, 0, 0);
}
LSK_DEV uint32_t epi_raw_col0(const EpiRaw& r, int64_t n, bool ok) {
  return __builtin_amdgcn_raw_buffer_load_b32(r.col0, ok ? (int)(4 * n) : (int)0x80000000u, 0, 0);
}
LSK_DEV uint32_t epi_raw_col1(const EpiRaw& r, int64_t n, bool ok) {
  return __builtin_amdgcn_raw_buffer_load_b32(r.col1, ok ? (int)(4 * n) : (int)0x80000000u, 0, 0);
}
// The EpiRow / EpiCol those words stand for (epi_row_load / epi_col_load's values).
LSK_DEV EpiRow epi_row_of(const EpiParams& p, uint32_t raw) {
  EpiRow r{0.0f, 0};
  if (p.order == LSK_EPI_POW2) r.sh = p.shift + (int)raw;
  else r.row = __uint_as_float(raw);
  return r;
}
LSK_DEV EpiCol epi_col_of(const EpiParams& p, uint32_t raw0, uint32_t raw1) {
  EpiCol c{0.0f, 0.0f, 0};
  if (p.order == LSK_EPI_POW2) c.sh = (int)raw0;
  else {
    c.ws = __uint_as_float(raw0);
    c.b = __uint_as_float(raw1);
  }
  return c;
}
// Whether epi_raw's offsets cover M rows and N columns.
inline bool epi_raw_fits(int64_t M, int64_t N) { return M < (1 << 29) && N < (1 << 29); }

// Round four epilogue values to the output type and store them at element offset o with one
// vector store (the row segment is aligned and in range).  RAW stores the accumulators.
LSK_DEV void store4_out(void* out, int order, int out_dtype, int64_t o, const float* y, v4i acc) {
  if (order == LSK_EPI_RAW) {
    store16_split((int32_t*)out + o, (uint32_t)acc[0], (uint32_t)acc[1], (uint32_t)acc[2], (uint32_t)acc[3]);
    return;
  }
  switch (out_dtype) {
    case LSK_BF16: {
      uint2 u;
      u.x = (uint32_t)f32_to_bf16(y[0]) | ((uint32_t)f32_to_bf16(y[1]) << 16);
      u.y = (uint32_t)f32_to_bf16(y[2]) | ((uint32_t)f32_to_bf16(y[3]) << 16);
      *(uint2*)((uint16_t*)out + o) = u;
      break;
    }
    case LSK_F16: {
      uint2 u;
      u.x = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)y[0]) |
            ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)y[1]) << 16);
      u.y = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)y[2]) |
            ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)y[3]) << 16);
      *(uint2*)((uint16_t*)out + o) = u;
      break;
    }
    case LSK_BF16_AS_F32:
      store16_split((float*)out + o, __float_as_uint(bfr(y[0])), __float_as_uint(bfr(y[1])),
                    __float_as_uint(bfr(y[2])), __float_as_uint(bfr(y[3])));
      break;
    default:
      store16_split((float*)out + o, __float_as_uint(y[0]), __float_as_uint(y[1]), __float_as_uint(y[2]),
                    __float_as_uint(y[3]));
  }
}

// Four consecutive columns n..n+3 of row m: epilogue, rounding and one vector store when
// `vec` (the row segment is aligned and in range), else element stores up to column N.
LSK_DEV void epilogue_store4(const EpiParams& p, int64_t m, int64_t n, int64_t N, v4i acc, bool vec) {
  if (!vec) {
    for (int t = 0; t < 4; ++t)
      if (n + t < N) epilogue_store(p, m, n + t, acc[t]);
    return;
  }
  float y[4];
  if (p.order != LSK_EPI_RAW) {
#pragma unroll
    for (int t = 0; t < 4; ++t) y[t] = epi_value(p, m, n + t, acc[t]);
  }
  store4_out(p.out, p.order, p.out_dtype, m * p.ldo + n, y, acc);
}

// The same with the row and column operands already loaded (see epi_value_pre), the
// epilogue given as plain values so the common cases fold to constants; stores element-wise
// up to column N when not `vec`.
LSK_DEV void epilogue_store4_pre(void* out, int64_t ldo, int order, int out_dtype, bool has_bias, int shift,
                                 int64_t m, int64_t n, int64_t N, v4i acc, float ascm, const float* wsn,
                                 const float* bn, int rshift, const int* cshift, bool vec) {
  float y[4];
  if (order != LSK_EPI_RAW) {
#pragma unroll
    for (int t = 0; t < 4; ++t)
      y[t] = epi_value_pre(order, out_dtype, has_bias, acc[t], ascm, wsn[t], bn[t], shift + rshift + cshift[t]);
  }
  if (vec) {
    store4_out(out, order, out_dtype, m * ldo + n, y, acc);
    return;
  }
  for (int t = 0; t < 4; ++t) {
    if (n + t >= N) break;
    if (order == LSK_EPI_RAW) ((int32_t*)out)[m * ldo + n + t] = acc[t];
    else store_out(out, out_dtype, m * ldo + n + t, y[t]);
  }
}

// Whether rows of the output allow 4-wide vector stores (16-byte rows for 4-byte types,
// 8-byte for 2-byte types).
inline bool out_vec_ok(const void* out, int out_dtype, int64_t ldo) {
  const int esz = (out_dtype == LSK_BF16 || out_dtype == LSK_F16) ? 2 : 4;
  return ((uintptr_t)out % (4 * esz) == 0) && ((ldo * esz) % (4 * esz) == 0);
}

// Thread-local last-error string shared by every entry point.
namespace lsk {
void set_error(const char* fmt, ...);
int check_launch(const char* what);
}  // namespace lsk

#define LSK_REQUIRE(cond, ...)        \
  do {                                \
    if (!(cond)) {                    \
      lsk::set_error(__VA_ARGS__);    \
      return LSK_ERR_ARG;             \
    }                                 \
  } while (0)
