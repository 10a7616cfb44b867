// The contract's table activations (no libm): silu_contract, sigmoid_contract, act_silu and
// act_swigluoai, one binary32 operation per declared step.
#pragma once
#include "lsk_common.h"

namespace lsk {

constexpr float kSiluC = -0x1.715476p+0f;   // binary32 nearest -log2(e) (lockstep_fullstack.py:175)
constexpr float kAlpha = 0x1.b3b646p+0f;    // fl32(1.702) (moe_ref.py:146)
constexpr float kMinNormal = 0x1p-126f;

// Steps (2)-(9) of silu_contract / sigmoid_contract (lockstep_fullstack.py:590-604,
// moe_ref.py:150-161) on the flushed input xc: 1 / (1 + FRAC[k] * 2^-15 * 2^i).
LSK_DEV float sigmoid_steps(float xc, const int32_t* __restrict__ frac) {
  float t = f32_mul(xc, kSiluC);
  t = fminf(fmaxf(t, -30.0f), 30.0f);
  const float i = ceilf(t);
  const float g = i - t;
  const float kf = fminf(truncf(f32_mul(g, 8192.0f)), 8191.0f);
  const float f = f32_mul((float)frac[(int)kf], 0x1p-15f);
  const float e2 = f32_mul(f, pow2f((int)i));
  return f32_div(1.0f, f32_add(1.0f, e2));
}

// Step (0): subnormal inputs are flushed to +0.
LSK_DEV float flush_sub(float x) { return fabsf(x) < kMinNormal ? 0.0f : x; }

LSK_DEV float silu_contract(float x, const int32_t* frac) {
  const float xc = flush_sub(x);
  return f32_mul(xc, sigmoid_steps(xc, frac));
}

LSK_DEV float sigmoid_contract(float x, const int32_t* frac) { return sigmoid_steps(flush_sub(x), frac); }

// moe_ref.py:183-186: bfr(fl32(silu(g)) * u)
LSK_DEV float act_silu(float g, float u, const int32_t* frac) { return bfr(f32_mul(silu_contract(g, frac), u)); }

// moe_ref.py:172-180: gc = min(g, 7); uc = clamp(u, -7, 7); arg = bfr(gc * 1.702);
// glu = bfr(gc * sig(arg)); h = bfr((uc + 1) * glu)
LSK_DEV float glu_oai(float g, const int32_t* frac) {
  const float gc = fminf(g, 7.0f);
  const float arg = bfr(f32_mul(gc, kAlpha));
  return bfr(f32_mul(gc, sigmoid_contract(arg, frac)));
}
LSK_DEV float swigluoai_up(float u, float glu) {
  const float uc = fminf(fmaxf(u, -7.0f), 7.0f);
  return bfr(f32_mul(f32_add(uc, 1.0f), glu));
}
LSK_DEV float act_swigluoai(float g, float u, const int32_t* frac) { return swigluoai_up(u, glu_oai(g, frac)); }

// The gate's part of an activation depends on g alone, and in the MoE epilogues g is always
// bf16-valued (a bfr result), so it can be read from a table of the 65536 bf16 bit patterns built
// once by the functions above (lsk_act_table): SiLU tab[g] = silu_contract(g) (binary32, the
// unrounded factor of bfr(silu(g) * u)); SwiGLU-OAI tab[g] = glu_oai(g).  The lookup then replaces
// the FRAC gather, the divide and the rest of the per-element steps with the same values.
LSK_DEV float act_table_entry(int act, uint32_t bits, const int32_t* frac) {
  const float g = __uint_as_float(bits << 16);
  return act == LSK_ACT_SILU ? silu_contract(g, frac) : glu_oai(g, frac);
}

// act(g, u) from the table entry t = tab[g] of the gate value.
LSK_DEV float act_from_entry(int act, float t, float u) {
  return act == LSK_ACT_SILU ? bfr(f32_mul(t, u)) : swigluoai_up(u, t);
}

// act(g, u) for bf16-valued g: from the table when one is given, else step by step.
LSK_DEV float act_eval(int act, float g, float u, const int32_t* frac, const float* tab) {
  if (tab) return act_from_entry(act, tab[__float_as_uint(g) >> 16], u);
  return act == LSK_ACT_SILU ? act_silu(g, u, frac) : act_swigluoai(g, u, frac);
}

}  // namespace lsk
