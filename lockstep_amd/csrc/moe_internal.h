// Internal interface between the MoE layer driver (moe.hip) and the MXFP4 grouped GEMMs (mx.hip).
#pragma once
#include "lsk_common.h"

namespace lsk {

constexpr int kMoeBM = 128;  // rows per expert tile (the dispatch's tile table granularity)

// Arguments of one grouped expert GEMM (gate/up with the activation, or down with the weight).
struct MoeGemmArgs {
  const void* A;            // int8 (int8 experts) or bf16 (MXFP4 experts) activation rows
  int64_t lda;              // elements
  int64_t a_bytes;          // bytes of A (its buffer resource range)
  int64_t w_bytes;          // bytes of one expert's weight (its buffer resource range)
  const float* a_scale;     // per A row
  const int32_t* row_tok;   // gate/up: permuted row -> token (A row); down: unused
  const int32_t* offs;      // [E + 1]
  const int32_t* tiles;     // [0] count, then (expert, first row) pairs
  const int64_t* w_ptrs;    // [E]: int8 [N_w, K] or packed E2M1 [N_w, K / 2]
  int64_t ldw;              // weight row stride in bytes
  const int64_t* ws_ptrs;   // [E]: f32 scales [N_w] (int8) or E8M0 bytes [N_w, K / 32] (MXFP4)
  int64_t lds;              // E8M0 row stride in bytes (MXFP4)
  const int64_t* b_ptrs;    // [E] or null
  int K;
  int N;                    // gate/up: I (h columns); down: H
  int act;
  const int32_t* frac;
  const float* act_tab;     // the activation's gate table (65536 entries) or null
  uint16_t* h;              // gate/up out [R, I] bf16
  uint32_t* h_amax;         // [R]
  const float* row_w;       // down: routing weight per row
  const int32_t* row_dst;   // down: destination slot row
  uint16_t* y;              // down out [T * k, N] bf16
  // block-scaled activations (MXFP4 experts, moe_forward_mx2): 0 off; 1 the fused-update kernel
  // over tiles without a flagged row; 2 the general kernel over tiles with one
  int mx2;
  const int32_t* row_flag;  // per A row (gate/up: per token)
  const int32_t* any_flag;  // nonzero when some row is flagged
  const int32_t* a_ka;      // block exponents of the A rows [rows, K/32]
  int64_t ldka;
  // bit 0: the A rows (down projection, rows p) in the row-pair layout -- rows 2i and 2i+1
  // interleaved by 64-byte K chunks, byte (p >> 1) * 2 lda + (k >> 6) * 128 + (p & 1) * 64 +
  // (k & 63), lda % 64 == 0; bit 1: the weights (w_ptrs) in that layout, ldw % 64 == 0
  // (ping-pong tiles only)
  int pairs;
  // ping-pong tiles of at most this many rows take the skinny path (0: none)
  int skinny_rows;
};

// The calling thread's grouped MX main-loop choice (lsk_moe_mx_select).
int mx_variant();

// MXFP4 grouped GEMMs (mode 0: gate/up + activation; 1: down + routing weight).
int launch_moe_mx_gemm(int mode, const MoeGemmArgs& ga, int64_t max_tiles, int safe, hipStream_t s);

// Decode-sized MX expert GEMV over int8 activation rows (mode 0: bias-added gate / up values into
// gu [R, 2N] bf16; mode 1: the routing-weighted slot rows), for token counts up to 64.
int launch_moe_mx_gemv(int mode, const MoeGemmArgs& ga, int64_t max_tiles, int64_t T, int safe, uint16_t* gu,
                       hipStream_t s);

// One token routed from its logits inside the skinny MX gate/up launch: the router's inputs, the
// token's row of x, and the routing outputs and one-token dispatch its block 0 writes.
struct MxRouteArgs {
  const void* g;  // logits [E] (f32 or bf16)
  int gdt;
  int64_t ldg;
  int E, k, renorm;
  const int32_t* rtab;
  const uint16_t* x;  // [K] bf16, 16-byte aligned
  int64_t* idx_out;
  uint16_t* w_out;
  int32_t *offs, *tiles, *row_tok, *row_dst, *tok_cnt;
  float *row_w, *ascx;
};
int launch_moe_mx_route_skinny1(const MoeGemmArgs& ga, const MxRouteArgs& ra, int safe, uint16_t* gu, hipStream_t s);

// One token of MXFP4 experts (per-row scales, at most four): the down GEMV of every slot and the
// ordered combine (+ bfr(shared)) in one launch, writing the token's row of y.
int launch_moe_mx_down_combine1(const MoeGemmArgs& ga, int safe, const float* shared, uint16_t* y, hipStream_t s);

// Skinny grouped MX GEMM (experts with few rows; per-row activation scales): the chunk's rows in
// LDS, the codes streamed into the bf16 MFMA (mode 0: gate / up values into gu; mode 1: slot rows).
// rows: at least the most rows any expert holds (the layer's T; the grouped linear's R).
int launch_moe_mx_skinny(int mode, const MoeGemmArgs& ga, int64_t max_tiles, int64_t rows, int safe, uint16_t* gu,
                         hipStream_t s);
int moe_mx_skinny_lds(int64_t K, int64_t lds);
int64_t mx_skinny_bytes(int64_t rows, int64_t K);

// Row quant emitting the int8 values as bf16 (the MX GEMM's operand form).
int launch_rowquant_bf16(const uint16_t* x, int64_t T, int64_t H, uint16_t* q, float* asc, hipStream_t s);

// Block quant of bf16 rows for block-scaled activations: dequantised bf16 values (integer values
// on flagged rows), exponents [R, K/32] and row flags (exponent outside [lo, hi]); *any is raised
// (integer atomic OR) when some row is flagged.
int launch_blockquant_mx2(const uint16_t* x, int64_t ldx, int64_t R, const int32_t* nrows, int K, uint16_t* q,
                          int32_t* ka, int32_t* flag, int32_t* any, int lo, int hi, hipStream_t s);

// Requant of h (bf16 values) with per-row maxima, emitting bf16 int8 values.
int launch_requant_bf16(const uint16_t* h, const uint32_t* amax, const int32_t* nrows, int64_t R, int I, uint16_t* q,
                        float* asc, hipStream_t s);

}  // namespace lsk
