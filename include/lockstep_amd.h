/* lockstep_amd: the Lockstep contract matrix-multiply path on MI355X (gfx950).
 *
 * A plain C ABI over hand-written HIP kernels.  Every pointer is a device pointer unless
 * stated otherwise; sizes and leading dimensions are in elements; `stream` is a hipStream_t
 * (NULL = the legacy default stream).  Every entry point is stream-ordered, returns 0 on
 * success or an LSK_ERR_* code, and leaves a message for lsk_last_error() on failure.
 * Nothing here allocates device memory unless its comment says so; workspace comes from
 * the caller.  Results are bit-identical to the reference functions cited on each entry
 * point, for every input, on every launch (no floating-point atomics, no split-K of
 * anything but exact integer sums).
 */
#ifndef LOCKSTEP_AMD_H
#define LOCKSTEP_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* status codes */
#define LSK_OK 0
#define LSK_ERR_ARG 1          /* bad shape, stride, alignment or dtype */
#define LSK_ERR_HIP 2          /* a HIP launch or runtime call failed */
#define LSK_ERR_UNSUPPORTED 3  /* valid input this build does not handle */

/* element types */
typedef enum {
  LSK_F32 = 0,
  LSK_BF16 = 1,
  LSK_F16 = 2,
  LSK_I32 = 3,
  LSK_I8 = 4,
  LSK_BF16_AS_F32 = 5 /* binary32 storage holding bf16-rounded values (moe_ref's bfr) */
} lsk_dtype;

/* epilogue orders applied to the exact int32 accumulator */
typedef enum {
  LSK_EPI_V21 = 0,  /* out(fl32(fl32(acc)*ws[n])*asc[m]); bias: out(fl32(out) + b[n]) */
  LSK_EPI_V2 = 1,   /* out(fl32(fl32(fl32(acc)*asc[m])*ws[n]) + b[n]) (legacy order) */
  LSK_EPI_POW2 = 2, /* fl32(acc) * 2^-(shift + erow[m] + ecol[n]) (exact scaling) */
  LSK_EPI_RAW = 3,  /* the int32 accumulator itself */
  LSK_EPI_V25 = 4   /* v2.5 outlier side path: y8 = bf16(fl32(fl32(acc)*ws[n])*asc[m]);
                       y = bf16(fl32(y8) + side[m,n]), side[m,n] = sum_j fl32(ho[m,j]*wo[n,j]) in
                       ascending j from +0; bias: bf16(fl32(y) + b[n]); then out(y) */
} lsk_epilogue;

/* The last error message of the calling thread ("" if none). */
const char* lsk_last_error(void);

/* Library version string. */
const char* lsk_version(void);

/* Per-row int8 quantisation.
 * Replaces moe_ref.rowquant (reference/moe_ref.py:27-37), lockstep_fullstack.quantize_rows_int8
 * (reference/lockstep_fullstack.py:476-481) and the inline quant of contract_common.w8a8_linear
 * (reference/contract_common.py:168-169):
 *   asc[m] = fl32(max(max_k |x[m,k]|, fl32(1e-8)) / 127)       (true division)
 *   q[m,k] = clamp(rint_even(fl32(x[m,k] / asc[m])), -127, 127)
 * x: [M, K] of x_dtype (LSK_F32 / LSK_BF16 / LSK_F16), row stride ldx; q: [M, K] int8, row
 * stride ldq; asc: [M] float. */
int lsk_rowquant(const void* x, int x_dtype, int64_t M, int64_t K, int64_t ldx,
                 int8_t* q, int64_t ldq, float* asc, void* stream);

/* Exact int8 x int8 -> int32 GEMM with a contract epilogue, c[m, n] = sum_k a[m,k] * w[n,k].
 * Replaces moe_ref.int_mm + lin_epilogue / lin_epilogue_b (reference/moe_ref.py:40-55,164-169),
 * lockstep_fullstack._int_mm_exact + the w8a8_matmul epilogue (reference/lockstep_fullstack.py:484-527),
 * the _int_mm + epilogue of contract_common.w8a8_linear (reference/contract_common.py:170-174)
 * and ref_block_v1.gemm_int + its pow2 dequant (reference/ref_block_v1.py:132-133,167,193,198,218).
 * a: [M, K] int8 (row stride lda); w: [N, K] int8 (row stride ldw; the reference's b8 = W8.t());
 * out: [M, N] of out_dtype (row stride ldo).  `order` is an lsk_epilogue; asc/ws are used by
 * V21/V2, bias is optional (NULL), erow/ecol/shift by POW2, out_dtype must be LSK_I32 for RAW.
 * M may be 0.  K is bounded by 133144 (|acc| <= K * 127^2 < 2^31). */
int lsk_gemm_w8a8(const int8_t* a, int64_t lda, const int8_t* w, int64_t ldw,
                  int64_t M, int64_t N, int64_t K, int order,
                  const float* asc, const float* ws, const float* bias,
                  const int32_t* erow, const int32_t* ecol, int shift,
                  void* out, int out_dtype, int64_t ldo, void* stream);

/* The contract epilogue alone, over an existing int32 accumulator acc [M, N] (row stride ldc).
 * Replaces moe_ref.lin_epilogue / lin_epilogue_b (reference/moe_ref.py:40-42,164-169) when the
 * caller keeps the reference's separate int_mm and epilogue calls.  Same parameters as
 * lsk_gemm_w8a8; RAW is not accepted. */
int lsk_epilogue_apply(const int32_t* acc, int64_t ldc, int64_t M, int64_t N, int order,
                       const float* asc, const float* ws, const float* bias,
                       const int32_t* erow, const int32_t* ecol, int shift,
                       void* out, int out_dtype, int64_t ldo, void* stream);

/* Bytes of caller workspace lsk_w8a8_matmul needs for M rows of width K. */
int64_t lsk_w8a8_matmul_workspace(int64_t M, int64_t K);

/* The whole dense contract linear: row quant of x, exact GEMM, epilogue `order` (V21 or V2).
 * Replaces lockstep_fullstack.w8a8_matmul (reference/lockstep_fullstack.py:503-530; order V21)
 * and the forward of contract_common.w8a8_linear (reference/contract_common.py:166-174; order V2).
 * x: [M, K] of x_dtype (row stride ldx); w: [N, K] int8; ws: [N]; bias: [N] or NULL;
 * out: [M, N] of out_dtype.  workspace: device memory of lsk_w8a8_matmul_workspace(M, K) bytes,
 * 256-byte aligned. */
int lsk_w8a8_matmul(const void* x, int x_dtype, int64_t ldx, int64_t M, int64_t K,
                    const int8_t* w, int64_t ldw, int64_t N, const float* ws, const float* bias,
                    int order, void* out, int out_dtype, int64_t ldo,
                    void* workspace, int64_t workspace_bytes, void* stream);

/* lsk_w8a8_matmul with w_pairs: NULL, or the same weight in the row-pair layout
 * (lsk_pack_row_pairs), which the GEMM reads when its tiles take the quantised rows in that layout
 * (no reference counterpart as an argument: a prepared copy of W8; the same results). */
int lsk_w8a8_matmul_pairs(const void* x, int x_dtype, int64_t ldx, int64_t M, int64_t K, const int8_t* w,
                          int64_t ldw, const int8_t* w_pairs, int64_t N, const float* ws, const float* bias,
                          int order, void* out, int out_dtype, int64_t ldo, void* workspace, int64_t workspace_bytes,
                          void* stream);

/* lsk_w8a8_matmul without a workspace argument and without allocating: no counterpart in the
 * reference.  For callers that cannot allocate device memory (code under graph capture, tight
 * serving loops, harnesses that forbid hipMalloc).  The quantised rows and their scales go to a
 * fixed 16 MiB array of this library on each GPU (held until the process ends), so M rows of width
 * K are accepted only while lsk_w8a8_matmul_workspace(M, K) <= 16 MiB (e.g. M = 2048 at K = 4096);
 * larger sizes return LSK_ERR_ARG with a message.  Every call on one GPU uses that GPU's array:
 * calls that overlap on one GPU (other streams, other threads) race.  Same results and the same
 * other arguments as lsk_w8a8_matmul. */
int lsk_w8a8_matmul_noalloc(const void* x, int x_dtype, int64_t ldx, int64_t M, int64_t K,
                            const int8_t* w, int64_t ldw, int64_t N, const float* ws, const float* bias,
                            int order, void* out, int out_dtype, int64_t ldo, void* stream);

/* ---------------------------------------------------------------- the v2.5 outlier side path */

/* The side term alone (replaces lockstep_fullstack.outlier_side, reference/lockstep_fullstack.py:549-557):
 *   side[m, n] = sum_j fl32(ho[m, j]) * fl32(wo[n, j]), sequential in ascending j from +0, binary32.
 * ho: [M, ko] of ho_dtype, wo: [N, ko] of wo_dtype (each LSK_F32 / LSK_BF16 / LSK_F16, contiguous);
 * side: [M, N] binary32 contiguous.  ko = 0 gives +0 everywhere. */
int lsk_outlier_side(const void* ho, int ho_dtype, int64_t M, int64_t ko, const void* wo, int wo_dtype, int64_t N,
                     float* side, void* stream);

/* The outlier split of w8a8_outlier_linear (reference/lockstep_fullstack.py:566-569):
 * xm = binary32 copy of x [M, K] (row stride ldx, LSK_F32 / LSK_BF16 / LSK_F16) with the declared
 * channels oidx [ko] (int32; negative values count from the end, as torch indexing does) set to
 * +0; ho [M, ko] binary32 = x[:, oidx] (exact).  xm may be NULL (gather only).  A channel
 * outside [-K, K) masks nothing and gathers NaN.  ko <= 4096. */
int lsk_outlier_split(const void* x, int x_dtype, int64_t ldx, int64_t M, int64_t K, const int32_t* oidx, int64_t ko,
                      float* xm, int64_t ldm, float* ho, void* stream);

/* Exact GEMM with the V25 epilogue (lsk_epilogue) over pre-quantised rows: replaces the GEMM and
 * epilogue lines of lockstep_fullstack.w8a8_outlier_linear (reference/lockstep_fullstack.py:571-577).
 * a: [M, K] int8; w: [N, K] int8; asc [M], ws [N], bias [N] or NULL; ho: [M, ko] binary32;
 * wo: [N, ko] of wo_dtype (LSK_BF16 or LSK_F32); out: [M, N] of out_dtype (f32 / bf16 / f16 /
 * bf16-as-f32: the bf16 result cast like the reference's final `.to(out_dtype)`). */
int lsk_gemm_w8a8_outlier(const int8_t* a, int64_t lda, const int8_t* w, int64_t ldw, int64_t M, int64_t N, int64_t K,
                          const float* asc, const float* ws, const float* bias, const float* ho, int64_t ko,
                          const void* wo, int wo_dtype, void* out, int out_dtype, int64_t ldo, void* stream);

/* Bytes of caller workspace lsk_w8a8_outlier_linear needs (M rows of width K, ko channels). */
int64_t lsk_w8a8_outlier_linear_workspace(int64_t M, int64_t K, int64_t ko);

/* The whole v2.5 norm-fed linear (replaces lockstep_fullstack.w8a8_outlier_linear,
 * reference/lockstep_fullstack.py:560-578): split (lsk_outlier_split), the 256-block butterfly / 16
 * when rot (v2.5; rot = 0 is the v2.5.1 o_proj form), row quant, exact GEMM, V25 epilogue.
 * x: [M, K] (row stride ldx); oidx [ko] int32; wo [N, ko] (LSK_BF16 or LSK_F32); w [N, K] int8;
 * ws [N]; bias [N] or NULL; out [M, N] of out_dtype.  rot needs K % 256 == 0.  workspace:
 * lsk_w8a8_outlier_linear_workspace(M, K, ko) bytes, 256-byte aligned. */
int lsk_w8a8_outlier_linear(const void* x, int x_dtype, int64_t ldx, int64_t M, int64_t K, const int32_t* oidx,
                            int64_t ko, const void* wo, int wo_dtype, const int8_t* w, int64_t ldw, int64_t N,
                            const float* ws, const float* bias, int rot, void* out, int out_dtype, int64_t ldo,
                            void* workspace, int64_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------- two-plane wide-integer linears */

/* Per-row quant to `bits` (8, 11 or 15) and its int8 planes (replaces t16h_lmvariants._quant_rows +
 * _planes, reference/t16h_lmvariants.py:71-84, and quantize_weight :95-103 for weight rows):
 *   v = x, or fl32(x / sdiv[k]) (sdiv_op 1, the runtime SmoothQuant divide, :154), or
 *   fl32(x * sdiv[k]) (sdiv_op 2, the prepare-time fold, :145);
 *   asc[m] = fl32(max(max_k |v|, fl32(1e-8)) / (2^(bits-1) - 1)) (true division);
 *   a = clamp(rint_even(fl32(v / asc[m])), +-(2^(bits-1) - 1));
 * then q32 [M, K] int32 = a when q32 is not NULL, else the planes into q (row stride ldq): bits 8
 * one plane (q[m] = a); else hi = a >> (bits - 8) at row m and lo = a - (hi << (bits - 8)) at
 * row M + m.  x: [M, K] of x_dtype (LSK_F32 / LSK_BF16 / LSK_F16), row stride ldx. */
int lsk_quant_planes(const void* x, int x_dtype, int64_t ldx, int64_t M, int64_t K, int bits, const float* sdiv,
                     int sdiv_op, int8_t* q, int64_t ldq, int32_t* q32, float* asc, void* stream);

/* The plane split of int32 values (replaces t16h_lmvariants._planes, reference/t16h_lmvariants.py:71-77):
 * hi = a >> sh (floor), lo = a - (hi << sh); sh = 0 writes hi = a only.  a, hi, lo: n elements. */
int lsk_split_planes(const int32_t* a, int64_t n, int sh, int8_t* hi, int8_t* lo, void* stream);

/* The exact int64 plane combine and the logits epilogue (t16h_lmvariants.py:115-125):
 * c [Pa * M, Pw * N] int32 (row stride ldc) holds the plane products, block (i, j) = activation
 * plane i x weight plane j (plane 0 = hi when the width is above 8);
 * s = sum acc_ij << (shift_i + shift_j) in int64; y = fl32(fl32(fl32(s) * asc[m]) * ws[n]),
 * fl32(s) round-to-nearest-even from int64; with a bias y = fl32(y + bias[n]); out(y). */
int lsk_planes_combine(const int32_t* c, int64_t ldc, int64_t M, int64_t N, int abits, int wbits, const float* asc,
                       const float* ws, const float* bias, void* out, int out_dtype, int64_t ldo, void* stream);

/* Bytes of caller workspace lsk_planes_linear needs. */
int64_t lsk_planes_linear_workspace(int64_t M, int64_t K, int64_t N, int abits, int wbits);

/* The whole a<abits>w<wbits> linear / lm_head (replaces t16h_lmvariants._mm_planes and
 * Variant.logits, reference/t16h_lmvariants.py:115-125,150-155, with the bias add and cast of
 * lockstep_fullstack.get_logits_contract, reference/lockstep_fullstack.py:849-860):
 * rows quantised to abits (divided by sdiv first when sdiv is not NULL), one exact GEMM of the
 * stacked activation planes against the weight planes w [Pw * N, K] (row stride ldw; hi plane
 * rows first, from lsk_quant_planes of the weight rows), then lsk_planes_combine.  Rows are
 * processed in chunks whose plane products fit the workspace (lsk_planes_linear_workspace). */
int lsk_planes_linear(const void* x, int x_dtype, int64_t ldx, int64_t M, int64_t K, int abits, const float* sdiv,
                      const int8_t* w, int64_t ldw, int64_t N, int wbits, const float* ws, const float* bias, void* out,
                      int out_dtype, int64_t ldo, void* workspace, int64_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------- the contract 2.6 float norm */

/* The float RMSNorm (replaces t16n_ref.rmsnorm_float / row_sum_float, reference/t16n_ref.py:53-92),
 * optionally fused with the contract row quant of its bf16 output (what lockstep_fullstack.w8a8_matmul
 * applies to the norm output, reference/lockstep_fullstack.py:476-481):
 *   S = the pinned tree sum of fl32(x^2) (chains of 8, then the adjacent-pairs tree);
 *   S = fl32(S + fl32(fl64(N) * eps)) when eps != 0; S = max(S, 2^-126);
 *   rs = fl32(sN / fl32(sqrt S)) (sN <= 0 selects the width constant fl32(sqrt N));
 *   out = bf16(fl32(fl32(x * rs) * g)) (no gain when g is NULL), stored as out_dtype (bf16, or the
 *   bf16 value widened / narrowed to f32 / f16);
 *   q, asc (when q is not NULL) = the row quant of the bf16 out values.
 * x: [R, N] of x_dtype (row stride ldx), N % 8 == 0, N <= 65536; S (optional): the row sums before
 * eps, binary32 [R]; out / q may each be NULL. */
int lsk_rmsnorm_float(const void* x, int x_dtype, int64_t ldx, int64_t R, int64_t N, const void* g, int g_dtype,
                      float sN, double eps, void* out, int out_dtype, int64_t ldo, int8_t* q, int64_t ldq,
                      float* asc, float* S, void* stream);

/* The pinned tree over given leaves (replaces t16n_ref.tree_sum, reference/t16n_ref.py:42-50):
 * T(v) = fl32(T(v[:P]) + T(v[P:])), P the largest power of two below n.  v: [R, n] binary32
 * (row stride ldv), 1 <= n <= 65536; out: [R]. */
int lsk_tree_sum(const float* v, int64_t ldv, int64_t R, int64_t n, float* out, void* stream);

/* Tuning control with no counterpart in the reference: force the dense kernel
 * (0: 128x128 register-staged tile, 4 waves of 64x64; 1: ping-pong 256x256, 8 waves of 64x128;
 * 2: ping-pong 256x256, 8 waves of 128x64; 3: ping-pong 256x128, 8 waves of 64x64;
 * 4: ping-pong 128x256, 8 waves of 64x64; 5: the decode GEMV when M <= 32, else tile 0;
 * 6, 7: for M <= 4 the 8-row register-buffered / LDS-ring GEMV instead of the whole-row GEMV;
 * 8..11: the whole-row GEMV with 1 / 2 / 4 / 8 rows per wave; 12, 13: tiles 3, 4 with a
 * three-stage LDS ring, two blocks per CU; 14 / 15: for 4 < M <= 32 the GEMV reading 64-byte row
 * pieces straight into registers / for M <= 16 whole rows through LDS; 17: four-wave 256x128,
 * one wave per SIMD with 128x64 wave tiles (16, its 256x256 form, spilled registers and is
 * refused); 18: ping-pong 256x128 with 128-byte K stages
 * in a three-stage ring, the shape's default; 19: for every M <= 32 whose activation rows fit in
 * LDS (M * (ceil(K / 1024) * 1024 + 16) <= 160 KB) the skinny GEMV -- A staged in LDS once per
 * block, weight rows streamed into the MFMA operand, the default for 4 < M <= 32 -- other M as 5)
 * or -1 to choose by shape (the default).  Results are identical for every choice; only speed differs.
 * The choice applies to the calling host thread's later launches only (thread-local). */
int lsk_gemm_select(int tile_id);

/* Tuning control with no counterpart in the reference: the launch shape of the skinny decode GEMV
 * (lsk_gemm_select 19): gpb groups of 16 weight rows per block, kw waves per group splitting K,
 * depth weight steps in flight per wave (4 or 8); 0 leaves a parameter to the shape rule.
 * gpb * kw <= 16.  Results are identical.  Thread-local. */
int lsk_gemm_skinny_shape(int gpb, int kw, int depth);

/* Tuning control with no counterpart in the reference: 1 (the default) runs lsk_w8a8_matmul /
 * lsk_w8a8_matmul_pairs with one activation row and K <= 16384 as a single launch, the row quant
 * fused into the whole-row decode GEMV (each block quantises the row itself into LDS); 0 runs the
 * row quant and the GEMV as two launches.  Results are identical.  Thread-local, like
 * lsk_gemm_select. */
int lsk_gemm_fuse_rowquant(int on);

/* Tuning control with no counterpart in the reference: 1 lets lsk_linear_dyn run its quant8_dyn in
 * one pass when the activation fits on chip (a cooperative launch of four blocks per CU holding x
 * in registers and LDS across one grid-wide barrier: M K <= 29,360,128 elements on a 256-CU part,
 * ldx == K, K % 64 == 0, M even, the stream not being captured); 0 (the default: measured about 3x
 * slower than the two passes on MI355X, the cooperative launch costing more than the second read
 * of x saves) always uses the two passes (maxima, then quantise).  Results are identical.
 * Thread-local. */
int lsk_quant8_dyn_single_pass(int on);

/* Tuning control with no counterpart in the reference: the quantise pass of lsk_linear_dyn's
 * quant8_dyn (0: row pairs per block; 1, the default: a contiguous tensor with K % 64 == 0 and M
 * even walked in the order of q, a wave's stores covering two whole 128-byte lines of q, 0
 * otherwise; 2: as 1 with ordinary rather than non-temporal loads in both passes).  The same
 * exponent and q.  Thread-local. */
int lsk_quant8_dyn_variant(int v);

/* Tuning control with no counterpart in the reference: the persistent form of the 256x256
 * ping-pong kernel, taken for whole tiles under the POW2 epilogue with binary32 output (the
 * ref_block_v1 GEMMs): 1 one block per compute unit (the default), 0 off (one tile per block),
 * blocks > 1 that many blocks.  Results are identical for every choice; only speed differs.
 * Thread-local, like lsk_gemm_select. */
int lsk_gemm_persist(int blocks);

/* Power-of-two int8 quantisation of ref_block_v1 (reference/ref_block_v1.py:56-72,122-130).
 * mode 0 = per tensor (quant8_dyn: one exponent e_out[0]); 1 = per row (quant8_rows: e_out[M]);
 * 2 = per column (quant8_cols: e_out[K]).  e = 6 - (biased_exp(m) - 127), minus 1 when
 * fl32(m * 2^e) > 127, clipped to [-32, 40] (per tensor: 0 and q = 0 when m == 0);
 * q = clamp(rint_even(fl32(x * 2^e)), -127, 127).  x: [M, K] binary32 (row stride ldx);
 * q: [M, K] int8 (row stride ldq); e_out: int32.  workspace: 4 * (M + K + 64) bytes. */
int lsk_quant8_pow2(const float* x, int64_t M, int64_t K, int64_t ldx, int mode,
                    int8_t* q, int64_t ldq, int32_t* e_out, void* workspace, void* stream);

/* quant8_dyn of the golden block (reference/ref_block_v1.py:122-130), the quantiser in front of each
 * of its GEMM sites (:166-167 qkv, :191-193 o, :196-198 up, :216-218 down): one exponent for the
 * whole x [M, K] binary32 (row stride ldx), the same rule and q as lsk_quant8_pow2 mode 0.  Writes
 * e_out[0] and, when erow_out is not null, erow_out[0..M) = e, the per-row exponent vector that
 * lsk_gemm_w8a8's POW2 epilogue takes, so the exponent never leaves the device.  Two launches and
 * nothing to clear beforehand (graph-capturable).  workspace: lsk_quant8_dyn_workspace() bytes. */
int64_t lsk_quant8_dyn_workspace(void);
int lsk_quant8_dyn(const float* x, int64_t M, int64_t K, int64_t ldx, int8_t* q, int64_t ldq,
                   int32_t* e_out, int32_t* erow_out, void* workspace, int64_t workspace_bytes, void* stream);

/* One GEMM site of the golden block whole (reference/ref_block_v1.py:166-167 qkv, :191-193 o,
 * :196-198 up, :216-218 down, each `q8, ex = quant8_dyn(x); y = gemm_int(q8, W8) * 2^-(ex + ew)`):
 * (q, ex) = quant8_dyn(x) as lsk_quant8_dyn, then y[m, n] = fl32(fl32(acc[m, n]) * 2^-(ex + ew))
 * with acc = q @ w^T exact -- the same y as lsk_quant8_dyn followed by lsk_gemm_w8a8 (POW2,
 * erow, shift = ew, binary32 out), bit for bit.  x [M, K] binary32 (row stride ldx); w [N, K] int8
 * (row stride ldw); y [M, N] binary32 (row stride ldy); ex_out[0] = ex.  q stays in the workspace
 * (lsk_linear_dyn_workspace(M, K) bytes, 256-byte aligned), written in the layout the GEMM tiles
 * read fastest (rows paired by 64-byte K chunks when every tile is a ping-pong tile).  Three
 * launches, nothing to clear beforehand (graph-capturable).  w_pairs: null, or the same weight in
 * the row-pair layout (lsk_pack_row_pairs), which the GEMM then reads when q takes that layout.
 * stages: 3 the whole site; 1 only the quant (q and the exponents into the workspace, ex_out), 2
 * only the GEMM from a workspace that a stage-1 call with the same arguments filled (to time the
 * GEMM alone). */
int64_t lsk_linear_dyn_workspace(int64_t M, int64_t K);
int lsk_linear_dyn(const float* x, int64_t M, int64_t K, int64_t ldx, const int8_t* w, int64_t ldw,
                   const int8_t* w_pairs, int64_t N, int ew, float* y, int64_t ldy, int32_t* ex_out, int stages,
                   void* workspace, int64_t workspace_bytes, void* stream);

/* No counterpart in the reference: a weight w [N, K] int8 (row stride ldw; K and ldw multiples of
 * 16, 16-byte aligned) copied into the row-pair layout the GEMM tiles read whole 128-byte lines
 * of -- rows 2i and 2i+1 interleaved by 64-byte K chunks, element (n, k) at byte (n >> 1) * 2 kp
 * + (k >> 6) * 128 + (n & 1) * 64 + (k & 63) with kp = (K + 63) / 64 * 64 -- into out
 * (lsk_row_pairs_bytes(N, K) bytes; padding bytes 0), for lsk_linear_dyn's w_pairs.  Made once per
 * weight (a prepared weight, like the reference's arm-time weight quant). */
int64_t lsk_row_pairs_bytes(int64_t N, int64_t K);
int lsk_pack_row_pairs(const int8_t* w, int64_t N, int64_t K, int64_t ldw, int8_t* out, void* stream);

/* No counterpart in the reference: 1 when lsk_w8a8_matmul / lsk_linear_dyn with M rows, N output
 * channels and depth K (K % 16 == 0) run every tile of the GEMM on the tiles that read a w_pairs
 * copy, under the calling thread's lsk_gemm_select; 0 otherwise (no device work, callable without
 * a GPU).  A caller makes the copy only when this says it will be read. */
int lsk_gemm_reads_row_pairs(int64_t M, int64_t N, int64_t K);

/* ---------------------------------------------------------------- the MXFP4 operand */

/* The MXFP4-consuming GEMM (contract addendum item 5).  Replaces moe_ref.int_mm_mx and,
 * with epilogue = 1, lin_epilogue_mx (reference/moe_ref.py:243-261):
 *   for each 32-wide K block b, ascending: s = sum_{j in b} a[m, j] * m2[n, j] (exact);
 *   acc = fl32(acc + fl32(s) * 2^(kexp[n, b] - 128)), from +0;
 *   epilogue 0: out = acc (binary32); 1: out = bfr(acc * asc[m]), then bfr(out + bias[n]).
 * a: [M, K] int8 (row stride lda); weights either m2 int8 [N, K] (b_fmt 0, the reference's
 * doubled mantissas in {0, +-1, +-2, +-3, +-4, +-6, +-8, +-12}) or packed E2M1 codes
 * [N, K/2] (b_fmt 1, low nibble first), row stride ldb bytes; kexp: E8M0 bytes [N, K/32],
 * row stride lds; out: [M, N] binary32 (row stride ldo).  K % 32 == 0. */
int lsk_gemm_mx(const int8_t* a, int64_t lda, const void* b, int b_fmt, int64_t ldb, const uint8_t* kexp,
                int64_t lds, int64_t M, int64_t N, int64_t K, int epilogue, const float* asc, const float* bias,
                float* out, int64_t ldo, void* stream);

/* Block quant of activations (block-scaled activations, contract addendum item 5b).  Replaces
 * moe_ref.blockquant (reference/moe_ref.py:299-314): per 32-wide block of each row,
 * ka = the least k with 127 * 2^k >= max |x| (the reference's ceil(log2(max / 127)) with its
 * rounding guard), clamped to [-126, 127], -126 for an all-zero block; q = clamp(rint(x / 2^ka),
 * +-127).  x: [M, K] bf16 or f32 (x_dtype, row stride ldx, rows 16-byte aligned); q: [M, K] int8
 * (row stride ldq, a multiple of 8); ka: [M, K/32] int32 (row stride ldka).  K % 32 == 0.
 * Infinite inputs give ka = 127, q = +-127; NaN inputs are not supported (the reference's int8
 * conversion of NaN is undefined). */
int lsk_blockquant(const void* x, int x_dtype, int64_t ldx, int64_t M, int64_t K, int8_t* q, int64_t ldq, int32_t* ka,
                   int64_t ldka, void* stream);

/* The MX operand with block-scaled activations.  Replaces moe_ref.int_mm_mx2 and, with
 * epilogue = 1, its bfr epilogue (reference/moe_ref.py:317-339):
 *   for each 32-wide K block b, ascending: s = sum_{j in b} q[m, j] * m2[n, j] (exact);
 *   p = fl32(2^(ka[m, b] + kexp[n, b] - 128)) (0 below 2^-149, inf from 2^128);
 *   acc = fl32(acc + fl32(s * p)), from +0;
 *   epilogue 0: out = acc; 1: out = bfr(acc), then bfr(out + bias[n]) when bias is given.
 * q: [M, K] int8 (row stride ldq, 16-byte aligned rows); ka: [M, K/32] int32 (row stride ldka);
 * weights and kexp as lsk_gemm_mx; out: [M, N] binary32 (row stride ldo).  K % 32 == 0. */
int lsk_gemm_mx2(const int8_t* q, int64_t ldq, const int32_t* ka, int64_t ldka, const void* b, int b_fmt, int64_t ldb,
                 const uint8_t* kexp, int64_t lds, int64_t M, int64_t N, int64_t K, int epilogue, const float* bias,
                 float* out, int64_t ldo, void* stream);

/* The MX epilogue alone (replaces moe_ref.lin_epilogue_mx, reference/moe_ref.py:258-261):
 * out = bfr(acc[m, n] * asc[m]), then bfr(out + bias[n]) when bias is given.  acc, out:
 * [M, N] binary32 contiguous (out may equal acc). */
int lsk_mx_epilogue(const float* acc, int64_t M, int64_t N, const float* asc, const float* bias, float* out,
                    void* stream);

/* Exact MXFP4 dequant (replaces moe_mxfp4.dequant_mxfp4, reference/moe_mxfp4.py:26-35):
 * out[r, k] = fp4(code[r, k]) * 2^(scale[r, k / block] - 127), rounded to out_dtype (exact for
 * every finite result; scale 255 gives 2^128 = inf as the reference's ldexp does).
 * packed: [rows, K/2] uint8 (low nibble = even element); scale: [rows, K/block] uint8;
 * out: [rows, K] of out_dtype (LSK_BF16 or LSK_F32), contiguous. */
int lsk_dequant_mxfp4(const uint8_t* packed, const uint8_t* scale, int64_t rows, int64_t K, int block, void* out,
                      int out_dtype, void* stream);

/* Pack doubled mantissas m2 (int8 [n]) into E2M1 codes (uint8 [n / 2], low nibble first);
 * *bad (device int32, caller-zeroed) receives 1 if some m2 is not 2 * an E2M1 value. */
int lsk_mx_pack_m2(const int8_t* m2, int64_t n, uint8_t* packed, int32_t* bad, void* stream);

/* A prepared copy of MXFP4 expert codes with no counterpart in the reference (the same weights; the
 * skinny grouped MX GEMM of lsk_moe_forward reads it instead of the [rows, K/2] codes, one whole
 * kilobyte per wave load): for each group g of 16 rows, each step s of four 32-blocks and each row
 * c of the group, 64 bytes = the four blocks' 16 code bytes, block by block (rows past `rows` and
 * blocks past K/32 are zero).  codes: [rows, K/2] uint8 (row stride ldw bytes, 4-byte aligned,
 * ldw % 4 == 0); out: lsk_mx_skinny_bytes(rows, K) bytes, 16-byte aligned.  K % 32 == 0.  Made
 * once per weight, like the row-pair copies of the int8 experts. */
int64_t lsk_mx_skinny_bytes(int64_t rows, int64_t K);
int lsk_mx_skinny_pack(const uint8_t* codes, int64_t ldw, int64_t rows, int64_t K, uint8_t* out, void* stream);

/* ---------------------------------------------------------------- mixture of experts (v3) */

/* Activation of the gate/up pair in the expert block. */
typedef enum {
  LSK_ACT_SILU = 0,      /* moe_ref.act_silu: bfr(silu_contract(g) * u) (reference/moe_ref.py:183-186) */
  LSK_ACT_SWIGLUOAI = 1  /* moe_ref.act_swigluoai (reference/moe_ref.py:172-180) */
} lsk_act;

/* Router scores and top-k from gate logits.
 * Replaces moe_ref.router_from_logits + table_scores (reference/moe_ref.py:64-74,85-97):
 *   d = max(rint(fl32(fl32(max_e g - g) * fl32(2^26 / ln 2))), 0);
 *   s = tab[(d >> 13) & 8191] >> min(d >> 26, 63), 0 when d >= 16 << 26;
 *   top-k by s * E + (E - 1 - e) (ties to the lower index), in rank order;
 *   w = bf16(fl32(s_sel) / fl32(S)), S = sum of the selected (renormalize) or of all scores, >= 1.
 * g: [T, E] of g_dtype (LSK_F32 holding bf16 values, or LSK_BF16), row stride ldg;
 * tab: [8192] int32 (the FRAC table); idx: [T, k] int64; w_bf16: [T, k] bf16 bits.
 * E <= 1024, k <= min(E, 32). */
int lsk_router_topk(const void* g, int g_dtype, int64_t ldg, int64_t T, int64_t E, int k, int renormalize,
                    const int32_t* tab, int64_t* idx, uint16_t* w_bf16, void* stream);

/* Elementwise table activations over n binary32 elements (no libm; one IEEE operation per
 * declared step).  op LSK_OP_SILU: lockstep_fullstack.silu_contract(g)
 * (reference/lockstep_fullstack.py:590-604); LSK_OP_SIGMOID: moe_ref.sigmoid_contract(g)
 * (reference/moe_ref.py:150-161); LSK_OP_ACT_SILU: moe_ref.act_silu(g, u) (:183-186);
 * LSK_OP_ACT_SWIGLUOAI: moe_ref.act_swigluoai(g, u) (:172-180).  frac: the [8192] int32
 * FRAC table.  u is unused (may be NULL) for the one-input ops. */
#define LSK_OP_SILU 0
#define LSK_OP_SIGMOID 1
#define LSK_OP_ACT_SILU 2
#define LSK_OP_ACT_SWIGLUOAI 3
int lsk_act_elementwise(const float* g, const float* u, int64_t n, int op, const int32_t* frac, float* out,
                        void* stream);

/* Router table scores of n gaps (replaces moe_ref.table_scores, reference/moe_ref.py:64-74):
 * out = tab[(d >> 13) & 8191] >> min(d >> 26, 63) for d = max(rint(fl32(dgap * C)), 0) below
 * 16 << 26, else 0.  dgap: binary32; tab: [8192] int32; out: int64. */
int lsk_table_scores(const float* dgap, int64_t n, const int32_t* tab, int64_t* out, void* stream);

/* The R1 / R4 block butterfly (replaces lockstep_fullstack.fwht_blocks,
 * reference/lockstep_fullstack.py:533-546): on every blk-wide block of each row, pairs (i, i+h)
 * -> (a+b, a-b) for h = 1, 2, ..., blk/2 in binary32, then one multiply by `scale`.
 * x, y: [rows, D] binary32 (row strides ldx, ldy; y may equal x); blk a power of two <= 1024
 * dividing D. */
int lsk_fwht_blocks(const float* x, int64_t rows, int64_t D, int64_t ldx, int blk, float scale, float* y,
                    int64_t ldy, void* stream);

/* The whole contract v3 MoE layer with int8 or MXFP4 experts and injected routing.
 * Replaces moe_ref.moe_forward / moe_forward_b / moe_forward_mx / moe_forward_mx2 with
 * routing=(idx, w) (reference/moe_ref.py:117-140, 189-200, 213-230, 264-290, 329-352):
 *   for each expert e ascending and the tokens that chose it: rowquant(x) -> exact GEMM with
 *   w13[e] -> bfr(V21 epilogue) (+ bfr(+ b13)) -> act(gate, up) -> rowquant -> exact GEMM with
 *   w2[e] -> bfr(V21) (+ bfr(+ b2)); y[t] = bf16(sum over t's experts ascending of
 *   bfr(w * out), binary32 adds from +0) (+ bfr(shared[t]) last).  With MXFP4 experts each
 *   GEMM is the MX operand (ordered binary32 block updates, see lsk_gemm_mx) and its epilogue
 *   bfr(acc * asc[m]) (+ bfr(+ b)); no rotation.
 * Expert weights are given as device tables of E device addresses (int64): w13_ptrs -> int8
 * [2I, H] (row stride ldw13), ws13_ptrs -> f32 [2I], w2_ptrs -> int8 [H, I] (row stride ldw2),
 * ws2_ptrs -> f32 [H], b13_ptrs / b2_ptrs -> f32 [2I] / [H] (the tables may be NULL for no
 * bias).  x: [T, H] bf16; idx: [T, k] int64 (experts outside [0, E) are skipped, as the
 * reference's loop over range(E) skips them; a token's experts must be distinct);
 * w: [T, k] bf16 bits; shared: [T, H] f32 or NULL; y: [T, H] bf16.
 * frac: the [8192] int32 FRAC table of the activation.  rot_blk > 0 applies the block
 * rotation of moe_ref's rot / rot_blk options (H and I multiples of rot_blk, I <= 16384).
 * workspace: lsk_moe_workspace bytes, 256-byte aligned.  H % 16 == 0 and I % 16 == 0. */
typedef struct {
  int64_t T, H, I, E;
  int k;
  int act;                       /* lsk_act */
  int wfmt;                      /* 0: int8 experts; 1: MXFP4 experts (moe_forward_mx): w13/w2 tables
                                    point at packed E2M1 codes [N, K/2] (low nibble first, row stride
                                    ldw* bytes) and ws13/ws2 tables at their E8M0 bytes [N, K/32]
                                    (row stride lds* bytes); K % 32 == 0; 2: MXFP4 experts with
                                    block-scaled activations (moe_forward_mx2: blockquant instead of
                                    rowquant, lsk_gemm_mx2's update, epilogues bfr(acc) (+ bias)) */
  int mx_safe;                   /* MXFP4: 1 when some E8M0 byte is >= 240 (exact multiply-then-add
                                    block update instead of the fused one) */
  int64_t lds13, lds2;           /* MXFP4: E8M0 row strides */
  const uint16_t* x;             /* [T, H] bf16 */
  const int64_t* idx;            /* [T, k] */
  const uint16_t* w;             /* [T, k] bf16 */
  const int64_t* w13_ptrs;       /* [E] */
  int64_t ldw13;
  const int64_t* ws13_ptrs;      /* [E] */
  const int64_t* b13_ptrs;       /* [E] or NULL */
  const int64_t* w2_ptrs;        /* [E] */
  int64_t ldw2;
  const int64_t* ws2_ptrs;       /* [E] */
  const int64_t* b2_ptrs;        /* [E] or NULL */
  const int32_t* frac;           /* [8192] */
  int rot_blk;                   /* 0: no rotation; else the R1 / R4 block (fwht_blocks) applied to
                                    x before its row quant and to h before its requant */
  float rot_scale;               /* the butterfly's final scale (1 / sqrt(rot_blk)) */
  const float* shared;           /* [T, H] or NULL */
  uint16_t* y;                   /* [T, H] bf16 */
  void* workspace;
  int64_t workspace_bytes;
  int kw13_min, kw13_max;        /* wfmt 2: bounds of the E8M0 bytes of all w13 / w2 weights (any */
  int kw2_min, kw2_max;          /* bounds that contain them keep results exact; tighter bounds let
                                    more rows take the fused block update) */
  const float* act_tab;          /* NULL, or lsk_act_table's table for `act` built from `frac`: the
                                    same results, the activation read per gate value */
  /* Routing from logits inside the layer (no reference counterpart as one call: the same as
   * moe_ref.router_from_logits, i.e. lsk_router_topk, followed by the layer with routing=(idx, w)).
   * When logits is not NULL, idx and w are not read: the layer writes the routing to idx_out
   * [T, k] int64 and w_out [T, k] bf16 and uses it (for up to 4 tokens inside the layer's first
   * launch).  k <= E. */
  const void* logits;            /* [T, E] f32 or bf16 (row stride ld_logits), or NULL */
  int logits_dtype;              /* LSK_F32 or LSK_BF16 */
  int renormalize;               /* as lsk_router_topk */
  int64_t ld_logits;
  const int32_t* router_tab;     /* the [8192] FRAC table, as lsk_router_topk */
  int64_t* idx_out;              /* [T, k] */
  uint16_t* w_out;               /* [T, k] bf16 */
  /* Kernel choice for this call only (no reference counterpart; results are the same bits either
   * way): 0 keeps the calling thread's lsk_moe_select / lsk_moe_mx_select settings; select = v + 2
   * applies lsk_moe_select(v) (v in [-1, 7]) and mx_select = v + 1 applies lsk_moe_mx_select(v)
   * (v in [0, 3]) to this call, leaving the thread's settings as they were. */
  int select;
  int mx_select;
  /* NULL, or per expert the same int8 weights in the row-pair layout (lsk_pack_row_pairs of the
   * [2I, H] and [H, I] matrices; row stride (K + 63) / 64 * 64), which the ping-pong expert tiles
   * read instead (int8 experts; the same results).  MXFP4 experts (wfmt 1 and 2): NULL, or per
   * expert the codes' skinny-layout copies (lsk_mx_skinny_pack), read by the skinny grouped MX
   * GEMM. */
  const int64_t* w13_pair_ptrs;
  const int64_t* w2_pair_ptrs;
} lsk_moe_args;

int64_t lsk_moe_workspace(int64_t T, int k, int64_t E, int64_t H, int64_t I, int rot_blk, int wfmt);

/* The activation's gate part over all 65536 bf16 bit patterns g, for lsk_moe_args.act_tab (no
 * reference counterpart as a table; the values are moe_ref's): act = LSK_ACT_SILU:
 * table[g] = silu_contract(g) (binary32, lockstep_fullstack.py:590-604); LSK_ACT_SWIGLUOAI:
 * table[g] = bfr(gc * sigmoid_contract(bfr(gc * 1.702))), gc = min(g, 7) (moe_ref.py:172-180).
 * In the MoE epilogues the gate value is always bf16-valued, so act(g, u) = bfr(table[g] * u)
 * (SiLU) or bfr((clamp(u, -7, 7) + 1) * table[g]) (SwiGLU-OAI), the same bits as step by step.
 * frac: the [8192] FRAC table; table: [65536] binary32 on the device. */
int lsk_act_table(const int32_t* frac, int act, float* table, void* stream);

int lsk_moe_forward(const lsk_moe_args* args, void* stream);

/* No counterpart in the reference: 1 when lsk_moe_forward on int8 experts with T tokens, top-k over
 * E experts, hidden H, intermediate I and rotation block rot_blk, under the per-call kernel choice
 * select (lsk_moe_args.select) and the calling thread's settings, reads the experts' row-pair weight
 * copies (w13_pair_ptrs / w2_pair_ptrs); 0 otherwise.  No device work, callable without a GPU: a
 * caller makes the copies only when a call will read them. */
int lsk_moe_reads_row_pairs(int64_t T, int k, int64_t E, int64_t H, int64_t I, int rot_blk, int select);

/* No counterpart in the reference: 1 when lsk_moe_forward on MXFP4 experts (wfmt 1, or 2 with
 * block-scaled activations), T tokens, top-k over E experts, hidden H, intermediate I and E8M0 row strides
 * lds13 / lds2, under the per-call choices select / mx_select (lsk_moe_args) and the calling
 * thread's settings, reads the experts' skinny-layout code copies (lsk_mx_skinny_pack of the
 * [2I, H/2] and [H, I/2] codes, passed as w13_pair_ptrs / w2_pair_ptrs); 0 otherwise.  No device
 * work, callable without a GPU. */
int lsk_moe_mx_reads_skinny(int64_t T, int k, int64_t E, int64_t H, int64_t I, int64_t lds13, int64_t lds2,
                            int select, int mx_select);

/* One grouped expert linear over rows already sorted by expert: expert e owns rows
 * offs[e] .. offs[e + 1] - 1 (offs [E + 1] int32 on the device, nondecreasing) of a, and
 *   out[p, n] = bfr(fl32(fl32(acc[p, n]) * ws_e[n]) * asc[p]), then bfr(out + b_e[n]) with a bias,
 *   acc[p, n] = sum_k a[p, k] * w_e[n, k] exact,
 * bf16 out [R, N] (row stride N).  The grouped form of the per-expert int_mm + lin_epilogue /
 * lin_epilogue_b that moe_ref.expert_block runs for each expert (reference/moe_ref.py:40-55,
 * 164-169, 189-200) -- the grouped-GEMM stage of lsk_moe_forward without the routing weight.
 * a: [R, K] int8 (row stride lda); asc: [R]; w_ptrs[e]: int8 [N, K] (row stride ldw, the
 * reference's W.t() of w_col [K, N]); ws_ptrs[e]: f32 [N]; b_ptrs: null or [E] of f32 [N].
 * workspace: lsk_grouped_gemm_workspace(R, E) bytes, 256-byte aligned (the tile table and a clamped
 * copy of offs).  Offsets that decrease or leave [0, R] are made monotone and clamped on the device
 * (offs'[j] = min(R, max(0, offs[0..j]))) before any tile reads them: such experts come out empty or
 * shortened, and no row outside [0, R) is read or written. */
int64_t lsk_grouped_gemm_workspace(int64_t R, int64_t E);
int lsk_grouped_gemm_w8a8(const int8_t* a, int64_t lda, const float* asc, const int32_t* offs, int64_t E, int64_t R,
                          const int64_t* w_ptrs, int64_t ldw, const int64_t* ws_ptrs, const int64_t* b_ptrs,
                          int64_t N, int64_t K, uint16_t* out, void* workspace, int64_t workspace_bytes,
                          void* stream);
/* The same with w_pair_ptrs: NULL, or per expert the weight in the row-pair layout
 * (lsk_pack_row_pairs; row stride (K + 63) / 64 * 64), read by the ping-pong tiles (R >= 16 E)
 * instead of w_ptrs (no reference counterpart as an argument: prepared weight copies; the same
 * results). */
int lsk_grouped_gemm_w8a8_pairs(const int8_t* a, int64_t lda, const float* asc, const int32_t* offs, int64_t E,
                                int64_t R, const int64_t* w_ptrs, int64_t ldw, const int64_t* w_pair_ptrs,
                                const int64_t* ws_ptrs, const int64_t* b_ptrs, int64_t N, int64_t K, uint16_t* out,
                                void* workspace, int64_t workspace_bytes, void* stream);

/* The MXFP4 form: per expert e, int_mm_mx then lin_epilogue_mx (reference/moe_ref.py:243-261, run
 * per expert by expert_block_mx :264-271): acc = the ordered block accumulation of int_mm_mx,
 * out = bfr(fl32(acc * asc[p])), then bfr(out + b_e[n]).  a: the int8 row values held as bf16
 * [R, K] (row stride lda elements, the MX kernels' operand form); w_ptrs[e]: packed E2M1 codes
 * [N, K / 2] (row stride ldw bytes); kx_ptrs[e]: E8M0 bytes [N, K / 32] (row stride lds); safe as
 * lsk_moe_args.mx_safe.  Same offsets, output and workspace as lsk_grouped_gemm_w8a8. */
int lsk_grouped_gemm_mx(const uint16_t* a, int64_t lda, const float* asc, const int32_t* offs, int64_t E, int64_t R,
                        const int64_t* w_ptrs, int64_t ldw, const int64_t* kx_ptrs, int64_t lds, const int64_t* b_ptrs,
                        int64_t N, int64_t K, int safe, uint16_t* out, void* workspace, int64_t workspace_bytes,
                        void* stream);
/* The same with w_skinny_ptrs: NULL, or per expert the codes' skinny-layout copy
 * (lsk_mx_skinny_pack of the [N, K/2] codes), read by the skinny grouped MX GEMM where
 * lsk_grouped_mx_reads_skinny says so (experts averaging at most 32 rows) instead of w_ptrs (no
 * reference counterpart as an argument: prepared weight copies; the same results). */
int lsk_grouped_gemm_mx_skinny(const uint16_t* a, int64_t lda, const float* asc, const int32_t* offs, int64_t E,
                               int64_t R, const int64_t* w_ptrs, int64_t ldw, const int64_t* w_skinny_ptrs,
                               const int64_t* kx_ptrs, int64_t lds, const int64_t* b_ptrs, int64_t N, int64_t K,
                               int safe, uint16_t* out, void* workspace, int64_t workspace_bytes, void* stream);
/* No counterpart in the reference: 1 when lsk_grouped_gemm_mx_skinny over R rows, E experts, depth K
 * and E8M0 row stride lds reads the skinny-layout copies under the calling thread's
 * lsk_moe_mx_select setting; 0 otherwise.  No device work. */
int lsk_grouped_mx_reads_skinny(int64_t R, int64_t E, int64_t K, int64_t lds);

/* Tuning control with no counterpart in the reference: 1 (the default) runs a one-token int8 layer
 * routed from its logits (lsk_moe_args.logits, the grouped GEMV path, k <= 8) with the router, the
 * row quant of x and the gate/up GEMV in one launch, every wave routing the token and quantising x
 * itself, and likewise a one-token MXFP4 layer on the skinny grouped MX GEMM (k <= 8, H <= 8192)
 * with the router and the row quant inside its gate/up launch; 0 runs them as the prep launch and
 * the GEMV or GEMM.  Also (1) int8 layers of more than 256
 * tokens routed from logits (E <= 256, H <= 4096, no rotation) route and quantise x in one launch,
 * a wave per token; 0 runs the router and lsk_rowquant.  Results are identical.  Thread-local. */
int lsk_moe_fuse_route(int on);

/* Tuning control with no counterpart in the reference: the int8 grouped expert GEMMs of
 * lsk_moe_forward on the 128x128 register-staged tile (0), on the eight-wave ping-pong
 * 128x256 tile (1), on the grouped GEMV (2: whole weight rows streamed once against up to 8
 * rows per expert at a time; taken only for int8 experts without rotation, T <= 64 and
 * H, I <= 4096, the tiles otherwise), on the 128x256 tile with the four-wave main loop (3: one wave
 * per SIMD per block, 64x128 wave tiles), or chosen by size (-1, the default: the GEMV for one
 * token, the skinny grouped GEMM (7) from 2 tokens, the ping-pong tile once the routed rows reach
 * 16 E; the register-staged tile where neither applies).  MXFP4 experts (H, I <= 8192, no
 * rotation) take the MX GEMV under 2 for T <= 64 and by default for T <= 24 (T <= 16 with
 * block-scaled activations), the MX grouped tiles otherwise.  Results are identical for every
 * choice.  4: the ping-pong tile with 128-byte K stages (one block per CU).  5: the 256x256 ping-pong
 * tile (the dense kernel's tile: eight waves of 64x128, a four-stage ring, one block per CU, its own
 * 256-row tile table) in a persistent kernel, one block per CU walking the tiles, the next tile's
 * first stages loaded under the current tile's epilogue (K >= 384; 6 below otherwise).  6: the same
 * tile, one block per tile.  7: the skinny grouped GEMM (a block stages up to 32 of an expert's
 * activation rows in LDS and streams its weight rows into the MFMA operand; int8 experts without
 * rotation, T <= 256, H, I <= 4096; the default from 2 tokens while the routed rows stay under
 * 16 E).  The choice applies to the
 * calling host thread's later launches only (thread-local). */
int lsk_moe_select(int variant);

/* Tuning control with no counterpart in the reference: the skinny grouped GEMM's launch shape --
 * gpb groups of 16 weight rows per block, kw waves per group splitting K (gpb * kw <= 16); 0 leaves
 * a parameter to the size rule.  Results are identical.  Thread-local. */
int lsk_moe_skinny_shape(int gpb, int kw);

/* Tuning control with no counterpart in the reference: the int8 ping-pong expert tiles (and the
 * grouped linear's) that hold at most `rows` routed rows (0..32; 32 the default, 0 none) run on the
 * skinny path -- the tile's rows staged in LDS once, its weight rows streamed into the MFMA
 * operand -- instead of the main loop; the epilogue is the tile's.  Results are identical.
 * Thread-local. */
int lsk_moe_pp_skinny_rows(int rows);

/* Tuning control with no counterpart in the reference: the main loop of the grouped MXFP4
 * expert GEMMs (0: direct-to-LDS operand staging with fp4 fragments converted per wave, a
 * two-stage ring, three blocks per CU, the default; 1: register-staged operands converted to bf16
 * before LDS; 2: as 0 with a three-stage ring and two blocks per CU; 3: as 0, with the skinny
 * grouped MX GEMM -- an expert's rows 16 at a time in LDS, the codes streamed into the bf16 MFMA --
 * wherever the layer can take it, which 0 does by size: MXFP4 layers with per-row activation
 * scales from 2 to 256 tokens, whose callers pass the codes' skinny-layout copies, and one token
 * when k * 2I / 64 >= 320; 0 keeps the decode GEMV for other single tokens).  Results are
 * identical; only speed differs.  The choice applies to the calling host thread's later launches
 * only (thread-local). */
int lsk_moe_mx_select(int variant);

/* ---------------------------------------------------------------- diagnostics */

/* The part's int8 MFMA ceiling, no counterpart in the reference: `blocks` x 256 threads each run
 * iters x 16 v_mfma_i32_32x32x32_i8 on operands read once from ops (nops 16-byte values, reused
 * modulo nops), registers only, and write one checksum each to sink [blocks * 256].  Timed by the
 * caller; 65536 int8 ops per MFMA.  Constant versus uniformly random operands shows the power cost
 * of toggling operands. */
int lsk_mfma_probe(const void* ops, int64_t nops, int64_t blocks, int iters, int32_t* sink, void* stream);

/* Diagnostic with no counterpart in the reference: one v_mfma_f32_16x16x32_bf16 per case with the
 * caller's accumulator input, D = A B^T + C over K = 32.  Case c: a, b [16][32] bf16 (rows M / N,
 * K contiguous, 16-byte aligned), cin, d [16][16] binary32 (row M, column N), ncases cases back to
 * back.  It measures how the matrix core rounds the addition of C to an exact block sum. */
int lsk_mfma_bf16_acc_probe(const uint16_t* a, const uint16_t* b, const float* cin, float* d, int ncases,
                            void* stream);

/* The library's bf16 conversion check, no counterpart in the reference: over the binary32
 * patterns start .. start + count - 1 (start + count <= 2^32), gfx950's packed v_cvt_pk_bf16_f32
 * (patterns that are not NaN) and the library's binary32 -> bf16 conversion (every pattern; the
 * instruction with NaN mapped to 0x7FC0) against the round-to-nearest-even bit method torch's
 * .to(bfloat16) uses; adds the number of disagreements to *mismatches and lowers *first to the
 * smallest disagreeing pattern (initialise them to 0 and 0xFFFFFFFF). */
int lsk_bf16_cvt_check(uint64_t start, uint64_t count, uint32_t* mismatches, uint32_t* first, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* LOCKSTEP_AMD_H */
