// Grouped MX main loop for gfx950 (the MoE MXFP4 expert GEMMs): 128 x 128 tiles, four waves of
// 64 x 64, K staged 64 elements (two MX blocks) at a time through a ring of two (three blocks
// per CU, the default: measured faster) or three LDS stages.
//
// The exact block update (see mx_tile.h) costs one binary32 FMA per output per 32-wide block on
// the VALU, as many VALU cycles as the bf16 MFMAs that produce the block sums take on the matrix
// core; the loop is built so that little else runs on the VALU and several waves share each SIMD
// (three blocks per CU with the two-stage ring), letting one wave's FMAs run beside another's
// MFMAs:
//   - activations (bf16 rows) and the packed E2M1 codes go global -> LDS by direct buffer loads
//     (no staging registers, no LDS write instructions); the codes stay 4-bit in LDS (4 KB per
//     stage) and each wave converts only the fragments it multiplies (v_cvt_scalef32_pk_bf16_fp4
//     with scale 2 gives the doubled mantissas exactly);
//   - the E8M0 bytes ride one byte load per thread per stage, become 2^(e-128) once and are
//     stored to LDS as binary32;
//   - every load is a buffer load with a precomputed row offset (rows past the expert's run and
//     bytes past K read zero), so the loop has no branches around loads and its waits are
//     exact counts.
// LDS slots are XOR-swizzled so that the 16 lanes reading one logical chunk of 16 consecutive
// rows hit distinct bank groups (activations: chunk c of row r at c ^ ((r >> 1) & 7); codes:
// chunk c of row r at c ^ ((r >> 3) & 1)).
#pragma once
#include <type_traits>

#include "mx_tile.h"
#include "pp_tile.h"

namespace lsk {

template <int RING>
struct MxPPCfg {
  static_assert(RING == 2 || RING == 3, "two or three ring stages");
  static constexpr int BM = 128, BN = 128, kThreads = 256;
  static constexpr int WTM = 64, WTN = 64, TM = 4, TN = 4;
  static constexpr int kRing = RING;
  static constexpr int kStageA = BM * 128;   // bf16 [128 rows][64 k]
  static constexpr int kStageB = BN * 32;    // E2M1 codes [128 rows][64 k] (4 bits each)
  static constexpr int kStageS = BN * 2 * 4; // binary32 2^(e-128) [128 rows][2 blocks]
  static constexpr int kStage = kStageA + kStageB + kStageS;
  static constexpr int kRingBytes = kRing * kStage;
  static constexpr int kLoads = 6;           // VMEM operations per thread per stage (4 A, 1 B, 1 scale)
  typedef v4f Acc[TM][TN];
};

// Per-thread load plan of one tile, fixed before the K loop.
struct MxPPRows {
  uint32_t a[4];  // byte offset of the activation row of each A load slot (kOob: no row)
  uint32_t b;     // byte offset of the code row of this thread's B slot
  uint32_t s;     // byte offset of the exponent row of this thread's scale slot
  int ka[4];      // byte offset of each A slot's logical chunk within a stage's 128-byte row segment
  int kb;         // byte offset of the B slot's logical chunk within a stage's 32-byte row segment
};

// rowA(r): byte offset of tile row r's activation row in `ra` or kOob; rowB(r) / rowS(r): byte
// offsets of tile row r's code row in `rb` and exponent row in `rs`, or kOob.
template <class FA, class FB, class FS>
LSK_DEV MxPPRows mx_pp_rows(FA rowA, FB rowB, FS rowS) {
  const int tid = threadIdx.x;
  MxPPRows p;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int slot = j * 256 + tid;
    const int row = slot >> 3;
    p.a[j] = rowA(row);
    p.ka[j] = 16 * ((slot & 7) ^ ((row >> 1) & 7));
  }
  const int brow = tid >> 1;
  p.b = rowB(brow);
  p.kb = 16 * ((tid & 1) ^ ((brow >> 3) & 1));
  p.s = rowS(brow);
  return p;
}

template <bool SAFE, int RING>
LSK_DEV void mx_pp_mainloop(typename MxPPCfg<RING>::Acc& acc, __amdgpu_buffer_rsrc_t ra, __amdgpu_buffer_rsrc_t rb,
                            __amdgpu_buffer_rsrc_t rs, const MxPPRows& rows, int K, char* smem) {
  using C = MxPPCfg<RING>;
  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
  const int wm = wave >> 1, wn = wave & 1;
  const int nk = (K + 63) / 64;

  // the stage's loads into ring slot s % kRing (the scale byte into a register)
  auto issue = [&](int s, uint32_t& sreg) {
    char* st = smem + (s % C::kRing) * C::kStage;
    const int k0 = s * 64;
    const bool tail = k0 + 64 > K;  // only a last half stage reaches past K
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int kk = k0 * 2 + rows.ka[j];
      const uint32_t off = (tail && kk >= 2 * K) ? kOob : rows.a[j] + (uint32_t)kk;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (lds_void_t)(st + (j * C::kThreads + wave * 64) * 16), 16, off, 0,
                                               0, 0);
    }
    {
      const int kk = k0 / 2 + rows.kb;
      const uint32_t off = (tail && 2 * kk >= K) ? kOob : rows.b + (uint32_t)kk;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rb, (lds_void_t)(st + C::kStageA + wave * 64 * 16), 16, off, 0, 0, 0);
    }
    const int kb = k0 / 32 + (tid & 1);
    sreg = __builtin_amdgcn_raw_buffer_load_b8(rs, (tail && 32 * kb >= K) ? (int)kOob : (int)(rows.s + (uint32_t)kb),
                                               0, 0);
  };
  // the scale byte of stage s, as binary32 2^(e-128), into its ring slot
  auto put_scale = [&](int s, uint32_t sreg) {
    float* ss = (float*)(smem + (s % C::kRing) * C::kStage + C::kStageA + C::kStageB);
    ss[tid] = pow2f((int)(sreg & 0xffu) - 128);
  };

  // fragment addresses: A row wm*64 + 16i + (lane & 15), logical chunk 4b + (lane >> 4);
  // B row wn*64 + 16j + (lane & 15), bytes 16b + 4 (lane >> 4) of its 32-byte segment
  const int r16 = lane & 15, g = lane >> 4;
  const int swzA = r16 >> 1, swzB = (r16 >> 3) & 1;
  const int offA = (wm * 64 + r16) * 128;
  const int offB = C::kStageA + (wn * 64 + r16) * 32 + 4 * g;
  const int offS = C::kStageA + C::kStageB + (wn * 64 + r16) * 8;

  // The FMAs of each block result run three MFMAs after it (a rolling window of four results),
  // so the VALU works on earlier results while the matrix core computes later ones, and no
  // FMA waits for the MFMA it depends on except at the end of a block.
  auto fma4 = [&](v4f& a, const v4f& d, float sc) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      if (SAFE) a[r] = f32_add(a[r], f32_mul(d[r], sc));
      else a[r] = __builtin_fmaf(d[r], sc, a[r]);
    }
  };
  auto block = [&](const char* st, int b, const float (&sc)[C::TN]) {
    v4i af[C::TM], bf[C::TN];
#pragma unroll
    for (int i = 0; i < C::TM; ++i) af[i] = *(const v4i*)(st + offA + i * 16 * 128 + 16 * ((4 * b + g) ^ swzA));
#pragma unroll
    for (int j = 0; j < C::TN; ++j) {
      const uint32_t q = *(const uint32_t*)(st + offB + j * 16 * 32 + 16 * (b ^ swzB));
      bf[j] = v4i{(int)__builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(q, 2.0f, 0)),
                  (int)__builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(q, 2.0f, 1)),
                  (int)__builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(q, 2.0f, 2)),
                  (int)__builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(q, 2.0f, 3))};
    }
    constexpr int kN = C::TM * C::TN, kLag = 3;
    v4f d[kLag + 1];
#pragma unroll
    for (int t = 0; t < kN + kLag; ++t) {
      if (t < kN) d[t % (kLag + 1)] = mfma_bf16(af[t / C::TN], bf[t % C::TN]);
      if (t >= kLag) {
        const int u = t - kLag;
        fma4(acc[u / C::TN][u % C::TN], d[u % (kLag + 1)], sc[u % C::TN]);
      }
    }
  };
  auto compute = [&](int s, bool two) {
    const char* st = smem + (s % C::kRing) * C::kStage;
    float s0[C::TN], s1[C::TN];
#pragma unroll
    for (int j = 0; j < C::TN; ++j) {
      const v2f_t v = *(const v2f_t*)(st + offS + j * 16 * 8);
      s0[j] = v[0];
      s1[j] = v[1];
    }
    block(st, 0, s0);
    if (two) block(st, 1, s1);
  };

  if constexpr (RING == 2) {
    // one stage ahead: step kt issues stage kt+1, multiplies stage kt, waits for kt+1
    uint32_t sr = 0;
    issue(0, sr);
    compiler_fence();
    wait_vm<0>();
    put_scale(0, sr);
    __syncthreads();
    for (int kt = 0; kt < nk; ++kt) {
      const bool more = kt + 1 < nk;
      if (more) issue(kt + 1, sr);
      compute(kt, kt * 64 + 32 < K);
      if (more) {
        compiler_fence();
        wait_vm<0>();
        put_scale(kt + 1, sr);
        __syncthreads();
      }
    }
  } else {
    // step kt: issue stage kt+2 (its scale byte into `rn`, the register stage kt's byte used);
    // multiply stage kt; wait for stage kt+1 and store its scales (byte in `rp`); barrier.
    // Stage kt+1 is the only one a step waits for: the loads of stage kt+2 stay in flight.
    auto step = [&](int kt, uint32_t& rn, uint32_t& rp) {
      const bool more = kt + 2 < nk;
      if (more) issue(kt + 2, rn);
      compute(kt, kt * 64 + 32 < K);
      if (kt + 1 < nk) {
        compiler_fence();
        if (more) wait_vm<C::kLoads>();
        else wait_vm<0>();
        put_scale(kt + 1, rp);
        __syncthreads();
      }
    };
    // prologue: stages 0 and 1 in flight, stage 0 complete
    uint32_t s0 = 0, s1 = 0;
    issue(0, s0);
    if (nk > 1) issue(1, s1);
    compiler_fence();
    if (nk > 1) wait_vm<C::kLoads>();
    else wait_vm<0>();
    put_scale(0, s0);
    __syncthreads();
    for (int kt = 0; kt < nk; kt += 2) {
      step(kt, s0, s1);  // even stages' bytes live in s0, odd stages' in s1
      if (kt + 1 < nk) step(kt + 1, s1, s0);
    }
  }
  __syncthreads();  // every wave is past its last LDS read of the ring (the epilogue reuses it)
}

}  // namespace lsk
