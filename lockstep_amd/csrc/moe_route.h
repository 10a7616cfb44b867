#pragma once
// The router's top-k selection of one token, shared by the router kernels (moe.hip) and the
// one-token MXFP4 launch that routes its token itself (mx.hip).
#include "lsk_common.h"

namespace lsk {

constexpr float kRouterC = 0x1.715476p+26f;  // fl32(2^26 / ln 2) (moe_ref.py:61)

// One wave per token; lane l owns experts l, l + 64, ... (EPL per lane, E <= 64 * EPL).  The
// reference's ranking key s * E + (E - 1 - e) orders like the pair (s, E - 1 - e); with scores
// below 2^16 (entries of the FRAC table are at most 2^15, and a score is an entry shifted right) and
// E <= 2^16 the pair packs into one 32-bit key s << 16 | (0xffff - e), so each of the k rounds is
// one DPP maximum over the wave and the winner is decoded from the wave-uniform key.  The
// selection: lane r < k gets the rank-r expert e_r and its score s_r; S is the score sum the
// weights divide by (the selected scores, or all of them without renormalisation), clamped to >= 1.
template <int EPL>
LSK_DEV void route_select(const void* __restrict__ g, int gdt, int64_t ldg, int t, int E, int k, int renorm,
                          const int32_t* __restrict__ tab, int& e_mine, int& s_mine, int& S) {
  const int lane = threadIdx.x & 63;
  float gv[EPL];
  float m = -__builtin_inff();
#pragma unroll
  for (int j = 0; j < EPL; ++j) {
    const int e = lane + 64 * j;
    gv[j] = 0.0f;
    if (e < E) {
      gv[j] = gdt == LSK_BF16 ? bf16_to_f32(((const uint16_t*)g)[(int64_t)t * ldg + e])
                              : ((const float*)g)[(int64_t)t * ldg + e];
      m = fmaxf(m, gv[j]);
    }
  }
  m = wave_fmax(m);
  uint32_t key[EPL];
  int s_all = 0;
#pragma unroll
  for (int j = 0; j < EPL; ++j) {
    const int e = lane + 64 * j;
    key[j] = 0;
    if (e < E) {
      const float v = rintf(f32_mul(m - gv[j], kRouterC));
      int sc = 0;
      if (v < 1073741824.0f) {  // d < 16 << 26 (also false for NaN / inf)
        const int d = v > 0.0f ? (int)v : 0;
        sc = tab[(d >> 13) & 8191] >> (d >> 26);
      }
      s_all += sc;
      key[j] = ((uint32_t)sc << 16) | (uint32_t)(0xffff - e);
    }
  }
  s_all = wave_sum_i32(s_all);
  s_mine = 0;
  e_mine = 0;
  int s_sum = 0;
  for (int r = 0; r < k; ++r) {
    uint32_t best = 0;
#pragma unroll
    for (int j = 0; j < EPL; ++j) best = key[j] > best ? key[j] : best;
    best = wave_max_u32(best);
    const int e = 0xffff - (int)(best & 0xffffu);
    const int sc = (int)(best >> 16);
    s_sum += sc;
    if (lane == r) {
      s_mine = sc;
      e_mine = e;
    }
#pragma unroll
    for (int j = 0; j < EPL; ++j)
      if (lane + 64 * j == e) key[j] = 0;
  }
  S = renorm ? s_sum : s_all;
  S = S < 1 ? 1 : S;
}

}  // namespace lsk
