// Contract v3 mixture-of-experts layer on gfx950, int8 experts (reference/moe_ref.py:117-230).
//
// Stages, all stream-ordered with no host synchronisation:
//   1. row quant of x once per token (an expert's rows are a subset of tokens; the per-row
//      quant does not depend on which other rows an expert sees);
//   2. dispatch: per-expert row counts, offsets and an M-tile table built on the device; rows
//      placed expert-major and token-ascending inside each expert (a counting sort whose
//      in-chunk ranks come from per-expert token bitmasks: deterministic);
//   3. grouped gate/up GEMM over variable-size expert tiles (token rows gathered), v2.1 epilogue
//      (+ bias) and the activation fused; each row's |h| maximum gathered by integer atomics on
//      the non-negative float bits (exact and order-free);
//   4. row requant of h;
//   5. grouped down GEMM, v2.1 epilogue (+ bias), times the routing weight, bf16 into a
//      token-major slot r = rank of the expert among the token's experts;
//   6. combine: per token, binary32 adds of its slots in ascending expert order from +0.
#include <atomic>

#include "contract_act.h"
#include "mfma_tile.h"
#include "moe_internal.h"
#include "moe_route.h"
#include "pp_tile.h"
#include "w4_tile.h"

namespace {

constexpr float kAmaxFloor = 0x1.5798eep-27f;  // fl32(1e-8)
constexpr int kBM = lsk::kMoeBM;
constexpr int kBM2 = 256;  // rows per tile of the 256 x 256 expert tiles (their own tile table)
thread_local int g_moe_force = -1;  // tuning control: -1 by size, 0 register-staged tile, 1 ping-pong tile, 2 GEMV,
                       // 3 the 128x256 tile on the four-wave main loop, 7 the skinny grouped GEMM
thread_local int g_rowq1 = 1;       // one-token layers from logits: router + row quant + gate/up GEMV in one launch
thread_local int g_msk_gpb = 0, g_msk_kw = 0;  // the skinny grouped GEMM's launch shape (0: by size)
// ping-pong expert tiles of at most this many rows take the skinny path (Qwen3-30B-A3B layer on
// MI355X, graph replays, T = 256 / 2048 / 4096: 167 / 294 / 418 us without, 153 / 284 / 412 at 16
// rows, 155 / 280 / 420 at 32)
thread_local int g_pp_skinny = 32;
thread_local int g_moe_w4 = 0;      // the ping-pong tile: 0 128x256 eight-wave ping-pong, 1 128x256 four waves,
                                    // 2 128x256 with 128-byte K stages, 3 256x256 (eight waves, four-stage ring)

// ---------------------------------------------------------------- router
// (route_select: moe_route.h)
using lsk::route_select;

template <int EPL>
LSK_DEV void route_token(const void* __restrict__ g, int gdt, int64_t ldg, int t, int E, int k, int renorm,
                         const int32_t* __restrict__ tab, int64_t* __restrict__ idx_out, uint16_t* __restrict__ w_out) {
  const int lane = threadIdx.x & 63;
  int e_mine, s_mine, S;
  route_select<EPL>(g, gdt, ldg, t, E, k, renorm, tab, e_mine, s_mine, S);
  if (lane < k) {
    idx_out[(int64_t)t * k + lane] = e_mine;
    w_out[(int64_t)t * k + lane] = f32_to_bf16(f32_div((float)s_mine, (float)S));
  }
}

template <int EPL>
__global__ __launch_bounds__(256) void router_topk_kernel(const void* __restrict__ g, int gdt, int64_t ldg, int T,
                                                          int E, int k, int renorm, const int32_t* __restrict__ tab,
                                                          int64_t* __restrict__ idx_out, uint16_t* __restrict__ w_out) {
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  route_token<EPL>(g, gdt, ldg, t, E, k, renorm, tab, idx_out, w_out);
}

// Layers of more than 256 tokens routed from logits: the router and the row quant of x in one launch
// (router_topk_kernel's and lsk_rowquant's values).  One wave per token: its row of x (bf16, H % 8
// == 0, H <= 512 NXC, 16-byte aligned) is requested first, the wave routes the token
// (route_token), takes the row's maximum over the wave and writes asc[t] = fl32(max(amax, 1e-8) /
// 127) and the row's int8 values (quant8_pack, row-major, row stride H).
template <int EPL, int NXC>
__global__ __launch_bounds__(256) void moe_route_rowq_kernel(const void* __restrict__ g, int gdt, int64_t ldg, int T,
                                                             int E, int k, int renorm, const int32_t* __restrict__ tab,
                                                             int64_t* __restrict__ idx_out, uint16_t* __restrict__ w_out,
                                                             const uint16_t* __restrict__ x, int H,
                                                             int8_t* __restrict__ q, float* __restrict__ asc) {
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;  // whole waves; no barrier follows
  const int lane = threadIdx.x & 63;
  const int H8 = H >> 3;
  const uint4* xr = (const uint4*)(x + (int64_t)t * H);
  uint4 u[NXC];
#pragma unroll
  for (int j = 0; j < NXC; ++j) {
    const int c = lane + 64 * j;
    u[j] = c < H8 ? xr[c] : make_uint4(0, 0, 0, 0);
  }
  route_token<EPL>(g, gdt, ldg, t, E, k, renorm, tab, idx_out, w_out);
  float v[NXC][8];
  float am = 0.0f;
#pragma unroll
  for (int j = 0; j < NXC; ++j) {
    const uint32_t wd[4] = {u[j].x, u[j].y, u[j].z, u[j].w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      v[j][2 * e] = bf16_to_f32((uint16_t)(wd[e] & 0xffff));
      v[j][2 * e + 1] = bf16_to_f32((uint16_t)(wd[e] >> 16));
      am = fmaxf(am, fmaxf(fabsf(v[j][2 * e]), fabsf(v[j][2 * e + 1])));
    }
  }
  am = wave_fmax(am);
  const float sc = f32_div(fmaxf(am, kAmaxFloor), 127.0f), rs = f32_div(1.0f, sc);
  if (lane == 0) asc[t] = sc;
  uint2* qr = (uint2*)(q + (int64_t)t * H);
#pragma unroll
  for (int j = 0; j < NXC; ++j) {
    const int c = lane + 64 * j;
    if (c < H8) qr[c] = quant8_pack(v[j], sc, rs);
  }
}

// ---------------------------------------------------------------- dispatch
// Rows are placed expert-major, token-ascending inside each expert: a counting sort over
// chunks of 256 tokens whose in-chunk ranks come from per-expert token bitmasks (no atomics
// decide a position, so the placement is deterministic).

// Exclusive scan of one int per thread across a block of THREADS threads; `total` gets the sum.
template <int THREADS>
LSK_DEV int block_excl_scan(int v, int* tmp, int& total) {
  const int lane = threadIdx.x & 63, wave = wave_id();
  int x = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(x, o, 64);
    if (lane >= o) x += y;
  }
  if (lane == 63) tmp[wave] = x;
  __syncthreads();
  int base = 0, tot = 0;
#pragma unroll
  for (int w2 = 0; w2 < THREADS / 64; ++w2) {
    const int t = tmp[w2];
    if (w2 < wave) base += t;
    tot += t;
  }
  __syncthreads();
  total = tot;
  return base + x - v;
}

// Expert offsets and the M-tile tables from per-expert row counts cnt[E] (any memory the block
// reads): offs[e] = rows of experts < e, offs[E] = all rows; tiles[0] = number of kBM-row tiles,
// then (expert, first row) per tile, experts ascending; tiles2 (if not null) the same in
// kBM2-row tiles (the 256 x 256 expert tiles).  Each thread owns a contiguous run of experts.
template <int THREADS>
LSK_DEV void expert_offsets_and_tiles(const int32_t* cnt, int E, int32_t* offs, int32_t* tiles, int* tmp,
                                      int32_t* tiles2 = nullptr) {
  const int per = (E + THREADS - 1) / THREADS;
  const int e0 = threadIdx.x * per;
  int rows = 0, ntl = 0, ntl2 = 0;
  for (int e = e0; e < e0 + per && e < E; ++e) {
    rows += cnt[e];
    ntl += (cnt[e] + kBM - 1) / kBM;
    ntl2 += (cnt[e] + kBM2 - 1) / kBM2;
  }
  int rows_all, tiles_all, tiles2_all;
  int rbase = block_excl_scan<THREADS>(rows, tmp, rows_all);
  int tbase = block_excl_scan<THREADS>(ntl, tmp, tiles_all);
  int tbase2 = block_excl_scan<THREADS>(ntl2, tmp, tiles2_all);
  for (int e = e0; e < e0 + per && e < E; ++e) {
    offs[e] = rbase;
    const int c = cnt[e];
    if (tiles)
      for (int r0 = 0; r0 < c; r0 += kBM, ++tbase) {
        tiles[1 + 2 * tbase] = e;
        tiles[2 + 2 * tbase] = rbase + r0;
      }
    if (tiles2)
      for (int r0 = 0; r0 < c; r0 += kBM2, ++tbase2) {
        tiles2[1 + 2 * tbase2] = e;
        tiles2[2 + 2 * tbase2] = rbase + r0;
      }
    rbase += c;
  }
  if (threadIdx.x == 0) {
    offs[E] = rows_all;
    if (tiles) tiles[0] = tiles_all;
    if (tiles2) tiles2[0] = tiles2_all;
  }
}

// The routing entries of the 256-token chunk c0 .. c0+255 as expert ids in LDS (-1 outside
// [0, E)), and their bf16 weights: one coalesced pass, so the steps below read LDS only.
LSK_DEV void load_chunk_routes(const int64_t* __restrict__ idx, const uint16_t* __restrict__ w, int T, int k, int E,
                               int c0, int32_t* ids, uint16_t* wts) {
  const int n = (T - c0 < 256 ? T - c0 : 256) * k;
  const int64_t* src = idx + (int64_t)c0 * k;
  for (int i = threadIdx.x; i < n; i += 256) {
    const int64_t e = src[i];
    ids[i] = (e >= 0 && e < E) ? (int)e : -1;
    if (wts) wts[i] = w[(int64_t)c0 * k + i];
  }
  __syncthreads();
}

// Place the rows of the 256-token chunk c0 .. c0+255 (its routes in ids / wts, as
// load_chunk_routes leaves them): p = base[e] + (rank of the token among the chunk's tokens
// routed to e); base (LDS or global) is advanced by the caller.  mask: E x 8 words.
LSK_DEV void place_chunk(const int32_t* ids, const uint16_t* wts, int T, int k, int E, int c0, const int32_t* base,
                         uint32_t* mask, int32_t* __restrict__ row_tok, int32_t* __restrict__ row_dst,
                         float* __restrict__ row_w, int wlo = 0, int whi = 256) {
  const int tid = threadIdx.x;
  for (int i = tid; i < E * 8; i += 256) mask[i] = 0;
  __syncthreads();
  const int t = c0 + tid;
  const int32_t* my = ids + tid * k;
  if (t < T) {
    for (int j = 0; j < k; ++j) {
      const int e = my[j];
      if (e >= 0) atomicOr(&mask[e * 8 + (tid >> 5)], 1u << (tid & 31));
    }
  }
  __syncthreads();
  if (t < T && tid >= wlo && tid < whi) {  // (the rows of tokens wlo .. whi-1 of the chunk)
    for (int j = 0; j < k; ++j) {
      const int e = my[j];
      if (e < 0) continue;
      int rank = __popc(mask[e * 8 + (tid >> 5)] & ((1u << (tid & 31)) - 1u));
      for (int wd = 0; wd < (tid >> 5); ++wd) rank += __popc(mask[e * 8 + wd]);
      const int p = base[e] + rank;
      int slot = 0;  // rank of e among the token's experts, ascending
      for (int j2 = 0; j2 < k; ++j2) {
        const int e2 = my[j2];
        if (e2 >= 0 && e2 < e) ++slot;
      }
      row_tok[p] = t;
      row_dst[p] = t * k + slot;
      row_w[p] = bf16_to_f32(wts[tid * k + j]);
    }
  }
  __syncthreads();
}

// Tokens routed to each expert in a 256-token chunk (LDS cnt[E]), and each token's number of
// valid routes; also zeroes zero_n words of zero_buf (the per-row |h| maxima) grid-wide.
LSK_DEV void count_chunk(const int32_t* ids, int T, int k, int c0, int32_t* cnt, int32_t* __restrict__ tok_cnt) {
  const int tid = threadIdx.x;
  const int t = c0 + tid;
  if (t < T) {
    int nv = 0;
    for (int j = 0; j < k; ++j) {
      const int e = ids[tid * k + j];
      if (e >= 0) {
        atomicAdd(&cnt[e], 1);
        ++nv;
      }
    }
    tok_cnt[t] = nv;
  }
}

// T <= 256: the whole dispatch in one block (dynamic LDS: cnt [E], base [E + 1], mask [8 E],
// ids [256 k], wts [256 k] u16).
LSK_DEV void dispatch_small_block(const int64_t* __restrict__ idx, const uint16_t* __restrict__ w, int T, int k, int E,
                                  int32_t* __restrict__ offs, int32_t* __restrict__ tiles,
                                  int32_t* __restrict__ row_tok, int32_t* __restrict__ row_dst,
                                  float* __restrict__ row_w, int32_t* __restrict__ tok_cnt,
                                  uint32_t* __restrict__ zero_buf, int64_t zero_n, int32_t* dsm,
                                  int32_t* __restrict__ tiles2) {
  __shared__ int tmp[4];
  int32_t* cnt = dsm;
  int32_t* base = dsm + E;
  uint32_t* mask = (uint32_t*)(dsm + 2 * E + 1);
  int32_t* ids = dsm + 10 * E + 1;
  uint16_t* wts = (uint16_t*)(ids + 256 * k);
  const int tid = threadIdx.x;
  for (int64_t i = tid; i < zero_n; i += 256) zero_buf[i] = 0u;
  for (int e = tid; e < E; e += 256) cnt[e] = 0;
  load_chunk_routes(idx, w, T, k, E, 0, ids, wts);  // ends with a barrier
  count_chunk(ids, T, k, 0, cnt, tok_cnt);
  __syncthreads();
  expert_offsets_and_tiles<256>(cnt, E, base, tiles, tmp, tiles2);
  __syncthreads();
  for (int e = tid; e <= E; e += 256) offs[e] = base[e];  // base[E] = all rows
  __syncthreads();
  place_chunk(ids, wts, T, k, E, 0, base, mask, row_tok, row_dst, row_w);
}

__global__ __launch_bounds__(256) void moe_dispatch_small_kernel(const int64_t* __restrict__ idx,
                                                                 const uint16_t* __restrict__ w, int T, int k, int E,
                                                                 int32_t* __restrict__ offs, int32_t* __restrict__ tiles,
                                                                 int32_t* __restrict__ row_tok,
                                                                 int32_t* __restrict__ row_dst,
                                                                 float* __restrict__ row_w,
                                                                 int32_t* __restrict__ tok_cnt,
                                                                 uint32_t* __restrict__ zero_buf, int64_t zero_n,
                                                                 int32_t* __restrict__ tiles2) {
  extern __shared__ int32_t dsm[];
  dispatch_small_block(idx, w, T, k, E, offs, tiles, row_tok, row_dst, row_w, tok_cnt, zero_buf, zero_n, dsm, tiles2);
}

// Decode-sized layers (the grouped GEMV path) start with one launch: block 0 runs the dispatch
// (clearing the per-row |h| maxima, zero_buf), block 1 + t the row quant of token t -- int8 rows, or their values as bf16 for MXFP4 experts -- with the
// scale and rounding of lsk_rowquant.
__global__ __launch_bounds__(256) void moe_decode_prep_kernel(const int64_t* __restrict__ idx,
                                                              const uint16_t* __restrict__ w, int T, int k, int E,
                                                              int32_t* __restrict__ offs, int32_t* __restrict__ tiles,
                                                              int32_t* __restrict__ row_tok,
                                                              int32_t* __restrict__ row_dst, float* __restrict__ row_w,
                                                              int32_t* __restrict__ tok_cnt,
                                                              uint32_t* __restrict__ zero_buf, int64_t zero_n,
                                                              const uint16_t* __restrict__ x, int H,
                                                              void* __restrict__ qx, float* __restrict__ ascx,
                                                              int q_bf16, const void* __restrict__ logits, int gdt,
                                                              int64_t ldg, const int32_t* __restrict__ rtab,
                                                              int renorm, int64_t* __restrict__ idx_out,
                                                              uint16_t* __restrict__ w_out, int32_t* __restrict__ tiles2) {
  extern __shared__ int32_t dsm[];
  if (blockIdx.x == 0) {
    if (logits) {
      // the routing first (T <= 4, E <= 256: a wave per token), then the dispatch reads it back
      for (int t = threadIdx.x >> 6; t < T; t += 4)
        route_token<4>(logits, gdt, ldg, t, E, k, renorm, rtab, idx_out, w_out);
      __threadfence_block();
      __syncthreads();
      idx = idx_out;
      w = w_out;
    }
    dispatch_small_block(idx, w, T, k, E, offs, tiles, row_tok, row_dst, row_w, tok_cnt, zero_buf, zero_n, dsm,
                         tiles2);
    return;
  }
  __shared__ float red[4];
  const int64_t t = blockIdx.x - 1;
  const uint16_t* row = x + t * H;
  const int tid = threadIdx.x;
  if ((H & 7) == 0 && H <= 8192 && ((uintptr_t)x & 15) == 0) {
    // the row in registers: thread tid holds elements 8 tid + 2048 j .. + 7 (16-byte loads, all
    // issued before the maximum)
    constexpr int NJ = 4;
    uint4 v[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int c = 8 * tid + 2048 * j;
      v[j] = c < H ? *(const uint4*)(row + c) : make_uint4(0, 0, 0, 0);
    }
    float am = 0.0f;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const uint32_t wd[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
#pragma unroll
      for (int e = 0; e < 4; ++e)
        am = fmaxf(am, fmaxf(fabsf(bf16_to_f32((uint16_t)(wd[e] & 0xffff))), fabsf(bf16_to_f32((uint16_t)(wd[e] >> 16)))));
    }
    am = wave_fmax(am);
    if ((tid & 63) == 0) red[tid >> 6] = am;
    __syncthreads();
    am = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    const float sc = f32_div(fmaxf(am, kAmaxFloor), 127.0f), rs = f32_div(1.0f, sc);
    if (tid == 0) ascx[t] = sc;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int c = 8 * tid + 2048 * j;
      if (c >= H) break;
      const uint32_t wd[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
      float qv[8];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        qv[2 * e] = fminf(fmaxf(rint_div8(bf16_to_f32((uint16_t)(wd[e] & 0xffff)), sc, rs), -127.0f), 127.0f);
        qv[2 * e + 1] = fminf(fmaxf(rint_div8(bf16_to_f32((uint16_t)(wd[e] >> 16)), sc, rs), -127.0f), 127.0f);
      }
      if (q_bf16) {
        uint32_t o[4];
#pragma unroll
        for (int e = 0; e < 4; ++e)
          o[e] = (__float_as_uint(qv[2 * e]) >> 16) | (__float_as_uint(qv[2 * e + 1]) & 0xffff0000u);
        store16_split((uint16_t*)qx + t * H + c, o[0], o[1], o[2], o[3]);
      } else {
        uint32_t o[2] = {0, 0};
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e >> 2] |= (uint32_t)(uint8_t)(int8_t)(int)qv[e] << (8 * (e & 3));
        *(v2u32*)((int8_t*)qx + t * H + c) = v2u32{o[0], o[1]};
      }
    }
    return;
  }
  float am = 0.0f;
  for (int i = tid; i < H; i += 256) am = fmaxf(am, fabsf(bf16_to_f32(row[i])));
  am = wave_fmax(am);
  if ((tid & 63) == 0) red[tid >> 6] = am;
  __syncthreads();
  am = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  const float sc = f32_div(fmaxf(am, kAmaxFloor), 127.0f), rs = f32_div(1.0f, sc);
  if (tid == 0) ascx[t] = sc;
  for (int i = tid; i < H; i += 256) {
    const float qv = fminf(fmaxf(rint_div8(bf16_to_f32(row[i]), sc, rs), -127.0f), 127.0f);
    if (q_bf16) ((uint16_t*)qx)[t * H + i] = (uint16_t)(__float_as_uint(qv) >> 16);  // exact in bf16
    else ((int8_t*)qx)[t * H + i] = (int8_t)(int)qv;
  }
}

// Large T, step 1: per-chunk expert counts ccnt[chunk][E].
__global__ __launch_bounds__(256) void moe_count_kernel(const int64_t* __restrict__ idx, int T, int k, int E,
                                                        int32_t* __restrict__ ccnt, int32_t* __restrict__ tok_cnt,
                                                        uint32_t* __restrict__ zero_buf, int64_t zero_n) {
  extern __shared__ int32_t cnt[];  // [E], then the chunk's ids [256 k]
  int32_t* ids = cnt + E;
  const int tid = threadIdx.x;
  for (int64_t i = (int64_t)blockIdx.x * 256 + tid; i < zero_n; i += (int64_t)gridDim.x * 256) zero_buf[i] = 0u;
  for (int e = tid; e < E; e += 256) cnt[e] = 0;
  load_chunk_routes(idx, nullptr, T, k, E, blockIdx.x * 256, ids, nullptr);  // ends with a barrier
  count_chunk(ids, T, k, blockIdx.x * 256, cnt, tok_cnt);
  __syncthreads();
  for (int e = tid; e < E; e += 256) ccnt[(int64_t)blockIdx.x * E + e] = cnt[e];
}

// Large T, step 2: each block sums the per-chunk counts itself (totals per expert and the
// counts of the chunks before its own), derives the expert offsets, and places a quarter of its
// chunk's rows (block b: chunk b / 4, tokens 64 (b % 4) .. +63; chunks ascending inside each
// expert: token order; four blocks per chunk spread the scattered row writes over more CUs);
// block 0 also writes the offsets and the M-tile table.  LDS: tot / pre / offs [E, E, E + 1], the placement mask [E][8], the chunk's ids
// [256 k] and weights [256 k] u16.
__global__ __launch_bounds__(256) void moe_place_kernel(const int64_t* __restrict__ idx, const uint16_t* __restrict__ w,
                                                        int T, int k, int E, const int32_t* __restrict__ ccnt,
                                                        int nchunks, int32_t* __restrict__ offs,
                                                        int32_t* __restrict__ tiles, int32_t* __restrict__ row_tok,
                                                        int32_t* __restrict__ row_dst, float* __restrict__ row_w,
                                                        int32_t* __restrict__ tiles2) {
  extern __shared__ int32_t sm_place[];
  int32_t* tot = sm_place;
  int32_t* pre = tot + E;
  int32_t* offl = pre + E;
  uint32_t* mask = (uint32_t*)(offl + E + 1);
  int32_t* ids = (int32_t*)(mask + 8 * E);
  uint16_t* wts = (uint16_t*)(ids + 256 * k);
  __shared__ int tmp[4];
  const int c0 = blockIdx.x >> 2, qr = blockIdx.x & 3;
  for (int e = threadIdx.x; e < E; e += 256) {
    int all = 0, before = 0;
    // the chunks' counts eight at a time, their loads issued together (one latency per eight)
    for (int cb = 0; cb < nchunks; cb += 8) {
      int v[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) v[j] = cb + j < nchunks ? ccnt[(int64_t)(cb + j) * E + e] : 0;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        all += v[j];
        before += cb + j < c0 ? v[j] : 0;
      }
    }
    tot[e] = all;
    pre[e] = before;
  }
  __syncthreads();
  expert_offsets_and_tiles<256>(tot, E, offl, blockIdx.x == 0 ? tiles : nullptr, tmp,
                                blockIdx.x == 0 ? tiles2 : nullptr);
  __syncthreads();
  for (int e = threadIdx.x; e <= E; e += 256) {
    if (blockIdx.x == 0) offs[e] = offl[e];
    if (e < E) offl[e] += pre[e];  // this chunk's first row per expert
  }
  load_chunk_routes(idx, w, T, k, E, c0 * 256, ids, wts);  // ends with a barrier
  place_chunk(ids, wts, T, k, E, c0 * 256, offl, mask, row_tok, row_dst, row_w, qr * 64, qr * 64 + 64);
}

__global__ __launch_bounds__(256) void widen_bf16_kernel(const uint16_t* __restrict__ x, int64_t n, float* __restrict__ y) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) y[i] = bf16_to_f32(x[i]);
}


// ---------------------------------------------------------------- grouped GEMM
using lsk::MoeGemmArgs;

// MODE 0: gate/up + activation; MODE 1: down + routing weight.
template <int MODE>
__global__ __launch_bounds__(256) void moe_gemm_kernel(MoeGemmArgs a) {
  using C = lsk::TileCfg<128, 128, 2, 2>;
  extern __shared__ v4i smem[];
  const int ntiles = MODE == 0 ? (a.N + 63) / 64 : (a.N + 127) / 128;
  const int L = lsk::xcd_logical_id(blockIdx.x, gridDim.x);
  const int mt = L / ntiles, nt = L - (L / ntiles) * ntiles;
  if (mt >= a.tiles[0]) return;
  const int e = a.tiles[1 + 2 * mt];
  const int p0 = a.tiles[2 + 2 * mt];
  const int p1 = min(a.offs[e + 1], p0 + kBM);
  const int8_t* wb = (const int8_t*)a.w_ptrs[e];
  const float* ws = (const float*)a.ws_ptrs[e];
  const float* bias = a.b_ptrs ? (const float*)a.b_ptrs[e] : nullptr;

  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
  const int wm = wave / 2, wn = wave % 2;
  // one resource over the whole activation matrix (gathered rows) and one over this expert's
  // weight; the host guarantees both spans fit 31-bit offsets
  const __amdgpu_buffer_rsrc_t ra_res = lsk::make_rsrc(a.A, a.a_bytes);
  const __amdgpu_buffer_rsrc_t rb_res = lsk::make_rsrc(wb, a.w_bytes);
  typename C::RowsA pa;
  typename C::RowsB pb;
#pragma unroll
  for (int j = 0; j < C::kAPer; ++j) {
    int row, c;
    lsk::chunk_of<C::kThreads>(tid, j, row, c);
    const int p = p0 + row;
    const int src = p < p1 ? (MODE == 0 ? a.row_tok[p] : p) : -1;
    pa[j] = src >= 0 ? (uint32_t)(src * a.lda) : lsk::kOob;
  }
#pragma unroll
  for (int j = 0; j < C::kBPer; ++j) {
    int row, c;
    lsk::chunk_of<C::kThreads>(tid, j, row, c);
    if (MODE == 0) {
      const int blk = row >> 5;  // 32-row blocks alternate gate / up weight rows
      const int hc = nt * 64 + (blk >> 1) * 32 + (row & 31);
      pb[j] = hc < a.N ? (uint32_t)(((blk & 1) ? a.N + hc : hc) * a.ldw) : lsk::kOob;
    } else {
      const int n = nt * 128 + row;
      pb[j] = n < a.N ? (uint32_t)(n * a.ldw) : lsk::kOob;
    }
  }
  typename C::Acc acc;
#pragma unroll
  for (int i = 0; i < C::TM; ++i)
#pragma unroll
    for (int j = 0; j < C::TN; ++j) acc[i][j] = lsk::zero16();

  lsk::mfma_mainloop<128, 128, 2, 2>(acc, ra_res, pa, rb_res, pb, a.K, smem);

  int32_t* region = (int32_t*)smem + wave * C::kStripInts;
#pragma unroll
  for (int i = 0; i < C::TM; ++i)
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      lsk::stage_half<C::TN, C::kLdc>(acc[i], hh, region);
      __syncthreads();
      const int rbase = p0 + wm * 64 + i * 32 + hh * 16;
      if (MODE == 0) {
        // half-strip columns: [gate 32 | up 32] for h columns nt*64 + wn*32 + [0, 32)
#pragma unroll
        for (int pass = 0; pass < 2; ++pass) {
          const int q = pass * 64 + lane;
          const int row = q >> 3, c4 = (q & 7) * 4;
          const v4i vg = *(const v4i*)(region + row * C::kLdc + c4);
          const v4i vu = *(const v4i*)(region + row * C::kLdc + 32 + c4);
          const int p = rbase + row;
          const int hc0 = nt * 64 + wn * 32 + c4;
          float am = 0.0f;
          if (p < p1) {
            const float asc = a.a_scale[a.row_tok[p]];
            uint16_t hb[4];
#pragma unroll
            for (int t = 0; t < 4; ++t) {
              const int hc = hc0 + t;
              hb[t] = 0;
              if (hc < a.N) {
                float yg = bfr(f32_mul(f32_mul((float)vg[t], ws[hc]), asc));
                float yu = bfr(f32_mul(f32_mul((float)vu[t], ws[a.N + hc]), asc));
                if (bias) {
                  yg = bfr(f32_add(yg, bias[hc]));
                  yu = bfr(f32_add(yu, bias[a.N + hc]));
                }
                const float hv =
                    lsk::act_eval(a.act, yg, yu, a.frac, a.act_tab);
                hb[t] = f32_to_bf16(hv);
                am = fmaxf(am, fabsf(hv));
              }
            }
            uint16_t* dst = a.h + (int64_t)p * a.N + hc0;
            if (hc0 + 4 <= a.N) {
              *(uint2*)dst =
                  make_uint2((uint32_t)hb[0] | ((uint32_t)hb[1] << 16), (uint32_t)hb[2] | ((uint32_t)hb[3] << 16));
            } else {
              for (int t = 0; t < 4; ++t)
                if (hc0 + t < a.N) dst[t] = hb[t];
            }
          }
          am = fmaxf(am, __shfl_xor(am, 1, 64));
          am = fmaxf(am, __shfl_xor(am, 2, 64));
          am = fmaxf(am, __shfl_xor(am, 4, 64));
          if ((lane & 7) == 0 && p < p1) atomicMax(&a.h_amax[p], __float_as_uint(am));
        }
      } else {
#pragma unroll
        for (int pass = 0; pass < 4; ++pass) {
          const int q = pass * 64 + lane;
          const int row = q >> 4, c4 = (q & 15) * 4;
          const v4i v = *(const v4i*)(region + row * C::kLdc + c4);
          const int p = rbase + row;
          const int n0 = nt * 128 + wn * 64 + c4;
          if (p < p1 && n0 < a.N) {
            const float asc = a.a_scale[p];
            const float wt = a.row_w ? a.row_w[p] : 1.0f;  // none: a plain grouped linear
            uint16_t ob[4];
#pragma unroll
            for (int t = 0; t < 4; ++t) {
              const int n = n0 + t;
              ob[t] = 0;
              if (n < a.N) {
                float yv = bfr(f32_mul(f32_mul((float)v[t], ws[n]), asc));
                if (bias) yv = bfr(f32_add(yv, bias[n]));
                ob[t] = f32_to_bf16(f32_mul(wt, yv));
              }
            }
            uint16_t* dst = a.y + (int64_t)(a.row_dst ? a.row_dst[p] : p) * a.N + n0;
            if (n0 + 4 <= a.N) {
              *(uint2*)dst =
                  make_uint2((uint32_t)ob[0] | ((uint32_t)ob[1] << 16), (uint32_t)ob[2] | ((uint32_t)ob[3] << 16));
            } else {
              for (int t = 0; t < 4; ++t)
                if (n0 + t < a.N) dst[t] = ob[t];
            }
          }
        }
      }
      __syncthreads();
    }
}

// Grouped GEMM tile: a 128-row expert tile (the dispatch's tile granularity) by 256 weight rows,
// on the eight-wave ping-pong main loop (PPM: waves of 64 x 64) or the four-wave one (W4M: waves of
// 64 x 128, one barrier per 16 MFMAs instead of two per 8); both rings take three stages, so two
// blocks share a CU and one's epilogue overlaps the other's main loop.  MODE 0 (gate/up): the 256
// weight rows are 128 h-columns' gate and up rows interleaved per 32, so a wave's strip holds
// [gate 32 | up 32] pairs and the activation is thread-local; MODE 1 (down): 256 output columns.
// The epilogue operands of the tile (row scales, routing weights and slots, column scales and
// biases) are loaded before the main loop and parked in LDS after it.
using PPM = lsk::PPCfg<128, 256, 2, 4, 3>;
using PPM128 = lsk::PPCfg<128, 256, 2, 4, 3, 128>;  // 128-byte K stages, one block per CU
using W4M = lsk::W4Cfg<128, 256, 3>;
// 256 x 256 expert tiles (the dense kernel's tile and wave shape, four-stage ring, one block per
// CU) over the 256-row tile table: half the operand bytes per MFMA of the 128-row tiles
using PPM256 = lsk::PPCfg<256, 256, 4, 2, 4>;
// LDS of a MoE tile: the ring / strip staging, then the tile's row operands (scale, weight, slot)
// and column operands (scale, bias)
template <class C>
constexpr int moe_smem_bytes() {
  return C::kSmemBytes > C::kScaleOff + (3 * C::kBM + 2 * C::kBN) * 4 ? C::kSmemBytes
                                                                    : C::kScaleOff + (3 * C::kBM + 2 * C::kBN) * 4;
}
static_assert(moe_smem_bytes<PPM128>() <= 160 * 1024 && moe_smem_bytes<PPM256>() <= 160 * 1024, "one block per CU");
static_assert(2 * moe_smem_bytes<W4M>() <= 160 * 1024 && 2 * moe_smem_bytes<PPM>() <= 160 * 1024, "two blocks per CU");

// A ping-pong tile of at most 32 rows on the skinny path: the main loop's LDS stages would move a
// 128-row activation panel for a few rows while the weight panel, the whole cost of such a tile,
// streams through a three-stage ring.  Instead the block copies the tile's rows into LDS once
// (direct loads, 1 KB of a row per instruction, row stride ldsk = a multiple of 1 KB plus 16 bytes;
// the down projection's rows from their row-pair layout when a.pairs & 1), and each wave streams the
// weight rows of two groups of 16 of the tile's columns (local columns 32 w .. 32 w + 31, weight rows
// wrow_of(c), the row-pair copy when a.pairs & 2) into the v_mfma_i32_16x16x64_i8 B operand, D steps
// per group in flight, the A fragments from LDS.  The exact sums go to the strip regions in the layout
// pp_stage_strip leaves them (row m, column c at region(c / WTN)[m * kLdc + c % WTN]), so the tile's
// epilogue runs unchanged on the waves of the first row of waves.
template <class C, int MODE, class WROW>
__device__ __forceinline__ void moe_tile_skinny(const MoeGemmArgs& a, char* smem, int p0, int p1, const int8_t* wb,
                                                WROW wrow_of) {
  constexpr int D = 4;
  static_assert(C::kThreads == 512 && C::kBN == 256, "eight waves of two 16-column groups");
  const int lane = threadIdx.x & 63, wave = wave_id();
  const int nr = p1 - p0;
  const int K = a.K, steps = (K + 63) >> 6;
  const int ldsk = (K + 1023) / 1024 * 1024 + 16;
  const int col = lane & 15, kg = lane >> 4;
  const bool pa = (a.pairs & 1) != 0, pw = (a.pairs & 2) != 0;
  // the tile's rows into LDS: their sources read once per wave (lane r holds row r's), then taken
  // by readlane, so no load sits between the direct loads
  const __amdgpu_buffer_rsrc_t ra = lsk::make_rsrc(a.A, a.a_bytes);
  const int cpr = (K + 1023) >> 10;
  int srcv = p0 + lane;
  if (MODE == 0) {
    const __amdgpu_buffer_rsrc_t rt = lsk::make_rsrc(a.row_tok + p0, 4 * (int64_t)nr);
    srcv = (int)__builtin_amdgcn_raw_buffer_load_b32(rt, lane < nr ? (uint32_t)(4 * lane) : lsk::kOob, 0, 0);
  }
  for (int c = wave; c < nr * cpr; c += 8) {
    const int r = c / cpr, j = c - (c / cpr) * cpr;
    const int src = __builtin_amdgcn_readlane(srcv, r);
    const int kk = j * 1024 + lane * 16;
    const uint32_t rowoff = (MODE == 1 && pa) ? (uint32_t)((src >> 1) * 2 * a.lda + (src & 1) * 64) : (uint32_t)(src * a.lda);
    const uint32_t koff = (MODE == 1 && pa) ? (uint32_t)((kk >> 6) * 128 + (kk & 63)) : (uint32_t)kk;
    const uint32_t off = kk < K ? rowoff + koff : lsk::kOob;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (lsk::lds_void_t)(smem + r * ldsk + j * 1024), 16, off, 0, 0, 0);
  }
  // this wave's two groups of weight rows, their first D steps
  const __amdgpu_buffer_rsrc_t rw = lsk::make_rsrc(wb, a.w_bytes);
  const uint32_t kstep = pw ? 128 : 64;
  uint32_t wbase[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    int hc;
    const int wr = wrow_of(32 * wave + 16 * h + col, hc);
    wbase[h] = hc < a.N ? (uint32_t)(pw ? (wr >> 1) * 2 * a.ldw + (wr & 1) * 64 : wr * a.ldw) + kg * 16 : lsk::kOob;
  }
  v4i w[2][D];
#pragma unroll
  for (int u = 0; u < D; ++u)
#pragma unroll
    for (int h = 0; h < 2; ++h)
      w[h][u] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(
                                            rw, (u < steps && wbase[h] != lsk::kOob) ? wbase[h] + u * kstep : lsk::kOob,
                                            0, 2 /* non-temporal */));
  lsk::compiler_fence();
  lsk::wait_vm<2 * D>();  // the rows (and the tile's operands requested before them)
  __syncthreads();
  v4i acc[2][2];
#pragma unroll
  for (int h = 0; h < 2; ++h) acc[h][0] = acc[h][1] = lsk::zero4();
  const char* arow[2];
  bool alive[2];
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int r = t * 16 + col;
    alive[t] = r < nr;
    arow[t] = smem + (r < nr ? r : nr - 1) * ldsk + kg * 16;
  }
  for (int s = 0; s < steps; s += D) {
#pragma unroll
    for (int u = 0; u < D; ++u) {
      const int st = s + u < steps ? s + u : 0;
      v4i af[2];
#pragma unroll
      for (int t = 0; t < 2; ++t) af[t] = alive[t] ? *(const v4i*)(arow[t] + st * 64) : lsk::zero4();
      const int nx = s + u + D;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        acc[h][0] = lsk::mfma_i8(af[0], w[h][u], acc[h][0]);
        acc[h][1] = lsk::mfma_i8(af[1], w[h][u], acc[h][1]);
        w[h][u] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(
                                              rw, (nx < steps && wbase[h] != lsk::kOob) ? wbase[h] + nx * kstep : lsk::kOob,
                                              0, 2 /* non-temporal */));
      }
    }
  }
  __syncthreads();  // every wave is past its last read of the rows: the strip regions reuse the LDS
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int c = 32 * wave + 16 * h + col;
    int32_t* region = (int32_t*)(smem + (c / C::WTN) * C::kStripBytes) + (c % C::WTN);
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) region[(t * 16 + kg * 4 + r) * C::kLdc] = acc[h][t][r];
  }
}

template <class C, int MODE, class MAIN>
__device__ __forceinline__ void moe_tile(const MoeGemmArgs& a, char* smem_moe, MAIN main) {
  static_assert((C::kBM == 128 || C::kBM == 256) && C::kBN == 256 && C::TM == 2,
                "128 or 256 x 256 tiles, two 32-row strips per wave");
  // a.tiles: the tile table in C::kBM-row tiles
  const int ntiles = MODE == 0 ? (a.N + 127) / 128 : (a.N + 255) / 256;
  const int L = lsk::xcd_logical_id(blockIdx.x, gridDim.x);
  const int mt = L / ntiles, nt = L - (L / ntiles) * ntiles;
  if (mt >= a.tiles[0]) return;  // the whole block leaves: no barrier is left waiting
  const int e = a.tiles[1 + 2 * mt];
  const int p0 = a.tiles[2 + 2 * mt];
  const int p1 = min(a.offs[e + 1], p0 + C::kBM);
  const int8_t* wb = (const int8_t*)a.w_ptrs[e];
  const float* ws = (const float*)a.ws_ptrs[e];
  const float* bias = a.b_ptrs ? (const float*)a.b_ptrs[e] : nullptr;
  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
  const int wm = wave / C::kWN, wn = wave % C::kWN;

  // weight row of local column c (gate/up interleave) and whether it exists
  auto wrow_of = [&](int c, int& hc) {
    if (MODE == 0) {
      const int blk = c >> 5;
      hc = nt * 128 + (blk >> 1) * 32 + (c & 31);
      return (blk & 1) ? a.N + hc : hc;
    }
    hc = nt * 256 + c;
    return hc;
  };

  // epilogue operands, held in registers across the main loop
  float r_asc = 0.0f, r_w = 0.0f, c_ws = 0.0f, c_b = 0.0f;
  int r_dst = 0;
  if (tid < C::kBM && p0 + tid < p1) {
    const int p = p0 + tid;
    if (MODE == 0) {
      r_asc = a.a_scale[a.row_tok[p]];
    } else {
      r_asc = a.a_scale[p];
      r_w = a.row_w ? a.row_w[p] : 1.0f;  // none: a plain grouped linear (weight 1, row p out)
      r_dst = a.row_dst ? a.row_dst[p] : p;
    }
  }
  if (tid < 256) {
    int hc;
    const int wr = wrow_of(tid, hc);
    if (hc < a.N) {
      c_ws = ws[wr];
      if (bias) c_b = bias[wr];
    }
  }

  const __amdgpu_buffer_rsrc_t ra_res = lsk::make_rsrc(a.A, a.a_bytes);
  const __amdgpu_buffer_rsrc_t rb_res = lsk::make_rsrc(wb, a.w_bytes);
  typename C::RowsA pa;
  typename C::RowsB pb;
#pragma unroll
  for (int j = 0; j < C::kLA; ++j) {
    int row, kb;
    lsk::pp_slot<C::kThreads, C::kChunks>(tid, j, row, kb);
    const int p = p0 + row;
    const int src = p < p1 ? (MODE == 0 ? a.row_tok[p] : p) : -1;
    const uint32_t ro = (MODE == 1 && (a.pairs & 1)) ? (uint32_t)((src >> 1) * 2 * a.lda + (src & 1) * 64)
                                                      : (uint32_t)(src * a.lda);
    pa[j] = src >= 0 ? ro : lsk::kOob;
  }
#pragma unroll
  for (int j = 0; j < C::kLB; ++j) {
    int row, kb, hc;
    lsk::pp_slot<C::kThreads, C::kChunks>(tid, j, row, kb);
    const int wr = wrow_of(row, hc);
    const uint32_t ro = (a.pairs & 2) ? (uint32_t)((wr >> 1) * 2 * a.ldw + (wr & 1) * 64) : (uint32_t)(wr * a.ldw);
    pb[j] = hc < a.N ? ro : lsk::kOob;
  }
  typename C::Acc acc;
#pragma unroll
  for (int i = 0; i < C::TM; ++i)
#pragma unroll
    for (int j = 0; j < C::TN; ++j) acc[i][j] = lsk::zero16();

  // the wave's 32-row strips that hold rows of the tile (the others are neither multiplied nor stored)
  const int na = max(0, min(C::TM, (p1 - p0 - wm * C::WTM + 31) / 32));
  // a tile of few rows: the skinny path, its sums left in the strip regions
  bool skinny = false;
  if constexpr (C::kThreads == 512 && C::kBN == 256) {
    skinny = p1 - p0 <= a.skinny_rows && p1 - p0 <= 32 && 32 * ((a.K + 1023) / 1024 * 1024 + 16) <= C::kScaleOff;
    if (skinny) moe_tile_skinny<C, MODE>(a, smem_moe, p0, p1, wb, wrow_of);
  }
  if (!skinny)
    main(acc, ra_res, pa, rb_res, pb, a.K, smem_moe, na, (MODE == 1 ? (a.pairs & 1) : 0) | (a.pairs & 2));

  // park the operands in LDS (past every wave's last ring read)
  float* sc_asc = (float*)(smem_moe + C::kScaleOff);
  float* sc_w = sc_asc + C::kBM;
  int* sc_dst = (int*)(sc_w + C::kBM);
  float* sc_ws = (float*)(sc_dst + C::kBM);
  float* sc_b = sc_ws + 256;
  if (tid < C::kBM) {
    sc_asc[tid] = r_asc;
    sc_w[tid] = r_w;
    sc_dst[tid] = r_dst;
  }
  if (tid < 256) {
    sc_ws[tid] = c_ws;
    sc_b[tid] = c_b;
  }
  __syncthreads();

  int32_t* region = (int32_t*)(smem_moe + wave * C::kStripBytes);
  auto strip = [&](int i) {
    if (MODE == 0) {
      // a wave strip is 32 rows x P [gate 32 | up 32] pairs; 8 lanes cover a pair's 32 columns
      // by quads, LPR lanes a row.  First every pass's gate / up values (and, with the table, all
      // their table entries, gathered together so that one latency covers the strip), then the
      // activations, the stores and the row maxima.
      constexpr int P = C::WTN / 64, LPR = 8 * P, RPP = 64 / LPR, NP = 32 / RPP;
      const int pr = (lane >> 3) % P;
      const int c4 = (lane & 7) * 4;
      const int hc0 = nt * 128 + wn * (32 * P) + pr * 32 + c4;
      // this lane's four gate and four up columns: the same in every pass
      const int cg0 = wn * C::WTN + pr * 64 + c4;
      const v4f wsg = *(const v4f*)(sc_ws + cg0), wsu = *(const v4f*)(sc_ws + cg0 + 32);
      const v4f bg = *(const v4f*)(sc_b + cg0), bu = *(const v4f*)(sc_b + cg0 + 32);
      float gv[NP][4], uv[NP][4];
#pragma unroll
      for (int t = 0; t < NP; ++t) {
        const int row = lane / LPR + RPP * t;
        const int ml = wm * C::WTM + i * 32 + row;
        const v4i vg = *(const v4i*)(region + row * C::kLdc + pr * 64 + c4);
        const v4i vu = *(const v4i*)(region + row * C::kLdc + pr * 64 + 32 + c4);
        const float asc = sc_asc[ml];  // 0 past the tile's rows
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          float yg = bfr(f32_mul(f32_mul((float)vg[q], wsg[q]), asc));
          float yu = bfr(f32_mul(f32_mul((float)vu[q], wsu[q]), asc));
          if (bias) {
            yg = bfr(f32_add(yg, bg[q]));
            yu = bfr(f32_add(yu, bu[q]));
          }
          gv[t][q] = yg;
          uv[t][q] = yu;
        }
      }
      if (a.act_tab) {
#pragma unroll
        for (int t = 0; t < NP; ++t)
#pragma unroll
          for (int q = 0; q < 4; ++q) gv[t][q] = a.act_tab[__float_as_uint(gv[t][q]) >> 16];
      }
#pragma unroll
      for (int t = 0; t < NP; ++t) {
        const int row = lane / LPR + RPP * t;
        const int ml = wm * C::WTM + i * 32 + row;
        const int p = p0 + ml;
        float am = 0.0f;
        if (p < p1 && hc0 + 4 <= a.N) {
          // a whole quad: no column tests
          float hv[4];
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            hv[q] = a.act_tab ? lsk::act_from_entry(a.act, gv[t][q], uv[t][q])
                              : lsk::act_eval(a.act, gv[t][q], uv[t][q], a.frac, nullptr);
            am = fmaxf(am, fabsf(hv[q]));
          }
          *(uint2*)(a.h + (int64_t)p * a.N + hc0) = make_uint2(pack_bf16x2(hv[0], hv[1]), pack_bf16x2(hv[2], hv[3]));
        } else if (p < p1) {
          uint16_t hb[4];
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            hb[q] = 0;
            if (hc0 + q < a.N) {
              const float hv = a.act_tab ? lsk::act_from_entry(a.act, gv[t][q], uv[t][q])
                                         : lsk::act_eval(a.act, gv[t][q], uv[t][q], a.frac, nullptr);
              hb[q] = f32_to_bf16(hv);
              am = fmaxf(am, fabsf(hv));
            }
          }
          uint16_t* dst = a.h + (int64_t)p * a.N + hc0;
          if (hc0 + 4 <= a.N) {
            *(uint2*)dst =
                make_uint2((uint32_t)hb[0] | ((uint32_t)hb[1] << 16), (uint32_t)hb[2] | ((uint32_t)hb[3] << 16));
          } else {
            for (int q = 0; q < 4; ++q)
              if (hc0 + q < a.N) dst[q] = hb[q];
          }
        }
#pragma unroll
        for (int o = 1; o < LPR; o <<= 1) am = fmaxf(am, __shfl_xor(am, o, 64));
        if (lane % LPR == 0 && p < p1) atomicMax(&a.h_amax[p], __float_as_uint(am));
      }
    } else {
      // 32 rows x QPR column quads; a lane keeps one quad
      constexpr int QPR = C::WTN / 4, RPP = 64 / QPR;
      const int c4 = (lane % QPR) * 4;
      const int n0 = nt * 256 + wn * C::WTN + c4;
      // this lane's four columns: the same in every pass
      const int cl0 = wn * C::WTN + c4;
      const v4f wsq = *(const v4f*)(sc_ws + cl0), bq = *(const v4f*)(sc_b + cl0);
#pragma unroll
      for (int t = 0; t < 32 / RPP; ++t) {
        const int row = lane / QPR + RPP * t;
        const int ml = wm * C::WTM + i * 32 + row;
        const int p = p0 + ml;
        const v4i v = *(const v4i*)(region + row * C::kLdc + c4);
        if (p < p1 && n0 + 4 <= a.N) {
          // a whole quad: no column tests
          const float asc = sc_asc[ml];
          const float wt = sc_w[ml];
          float o[4];
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            float yv = bfr(f32_mul(f32_mul((float)v[q], wsq[q]), asc));
            if (bias) yv = bfr(f32_add(yv, bq[q]));
            o[q] = f32_mul(wt, yv);
          }
          *(uint2*)(a.y + (int64_t)sc_dst[ml] * a.N + n0) = make_uint2(pack_bf16x2(o[0], o[1]), pack_bf16x2(o[2], o[3]));
        } else if (p < p1 && n0 < a.N) {
          const float asc = sc_asc[ml];
          const float wt = sc_w[ml];
          uint16_t ob[4];
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const int cl = wn * C::WTN + c4 + q;
            ob[q] = 0;
            if (n0 + q < a.N) {
              float yv = bfr(f32_mul(f32_mul((float)v[q], sc_ws[cl]), asc));
              if (bias) yv = bfr(f32_add(yv, sc_b[cl]));
              ob[q] = f32_to_bf16(f32_mul(wt, yv));
            }
          }
          uint16_t* dst = a.y + (int64_t)sc_dst[ml] * a.N + n0;
          if (n0 + 4 <= a.N) {
            *(uint2*)dst =
                make_uint2((uint32_t)ob[0] | ((uint32_t)ob[1] << 16), (uint32_t)ob[2] | ((uint32_t)ob[3] << 16));
          } else {
            for (int q = 0; q < 4; ++q)
              if (n0 + q < a.N) dst[q] = ob[q];
          }
        }
      }
    }
  };
  if (na > 0) {
    if (!skinny) lsk::pp_stage_strip<C::TN, C::kLdc>(acc[0], region);
    strip(0);
  }
  if (na > 1) {
    lsk::pp_stage_strip<C::TN, C::kLdc>(acc[1], region);
    strip(1);
  }
}

template <int MODE>
__global__ __launch_bounds__(512, 2) void moe_pp_kernel(MoeGemmArgs a) {
  extern __shared__ __attribute__((aligned(16))) char smem_moe[];
  moe_tile<PPM, MODE>(a, smem_moe,
                      [](PPM::Acc& acc, __amdgpu_buffer_rsrc_t ra, const PPM::RowsA& pa, __amdgpu_buffer_rsrc_t rb,
                         const PPM::RowsB& pb, int K, char* sm, int na, int pairs) {
                        lsk::pp_mainloop<128, 256, 2, 4, 3, 64, false, true>(acc, ra, pa, rb, pb, K, sm, na, pairs);
                      });
}

template <int MODE>
__global__ __launch_bounds__(512, 1) void moe_pp256_kernel(MoeGemmArgs a) {
  extern __shared__ __attribute__((aligned(16))) char smem_moe[];
  moe_tile<PPM256, MODE>(a, smem_moe,
                         [](PPM256::Acc& acc, __amdgpu_buffer_rsrc_t ra, const PPM256::RowsA& pa,
                            __amdgpu_buffer_rsrc_t rb, const PPM256::RowsB& pb, int K, char* sm, int na, int pairs) {
                           lsk::pp_mainloop<256, 256, 4, 2, 4, 64, false, true>(acc, ra, pa, rb, pb, K, sm, na, pairs);
                         });
}

// Persistent form of the 256 x 256 expert tiles (lsk_moe_select(5)): one block per CU walks the
// (256-row tile, N-tile) pairs v = blockIdx.x, blockIdx.x + gridDim.x, ... in moe_tile's logical order
// (xcd_logical_id over the pair count, read from the tile table).  After a tile's main loop the block
// parks the tile's epilogue operands in LDS past the ring, fills the whole ring with the next tile's
// first stages, and only then applies the epilogue straight from the accumulators (no LDS staging:
// the ring is being refilled), so the next tile's first loads run under the epilogue.  Register r of
// lane l of a 32 x 32 block is row 8 (r / 4) + 4 (l / 32) + r % 4, column l % 32, so lanes l and
// l ^ 1 hold neighbouring columns of the same rows: one exchange per register pair gives each lane
// two neighbouring bf16 values of one row, stored with one 4-byte store.  MODE 0: the gate and up
// values of an h-column sit in blocks 2t and 2t + 1 of the wave (the 32-interleave), so the
// activation is thread-local; each row's |h| maximum is reduced over its 32 lanes by shuffles and
// raised with one integer atomic per row and wave.  The arithmetic is moe_tile's.
constexpr int kP256pSmem = PPM256::kMainBytes + (3 * 256 + 2 * 256) * 4;
static_assert(kP256pSmem <= 160 * 1024, "one block per CU");

// Issue this thread's direct-to-LDS loads of the first kRing stages of a 256 x 256 expert tile into
// ring slots 0 .. kRing - 1 (pa / pb: the tile's load-slot row offsets; chunks past K read zeros).
__device__ __forceinline__ void moe256_issue_ring(__amdgpu_buffer_rsrc_t ra, const uint32_t* pa,
                                                  __amdgpu_buffer_rsrc_t rb, const uint32_t* pb, int K, char* smem,
                                                  int pairs) {
  using C = PPM256;
  const int tid = threadIdx.x, wave = wave_id();
  const int nk = (K + C::kBK - 1) / C::kBK;
#pragma unroll
  for (int st = 0; st < C::kRing; ++st) {
    if (st >= nk) break;
    char* base = smem + st * C::kStage;
#pragma unroll
    for (int j = 0; j < C::kLA; ++j) {
      int row, kbyte;
      lsk::pp_slot<C::kThreads, C::kChunks>(tid, j, row, kbyte);
      const int kk = st * C::kBK + kbyte;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (lsk::lds_void_t)(base + (j * C::kThreads + wave * 64) * 16), 16,
                                               kk < K ? pa[j] + lsk::pair_koff(kk, pairs & 1) : lsk::kOob, 0, 0, 0);
    }
#pragma unroll
    for (int j = 0; j < C::kLB; ++j) {
      int row, kbyte;
      lsk::pp_slot<C::kThreads, C::kChunks>(tid, j, row, kbyte);
      const int kk = st * C::kBK + kbyte;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rb, (lsk::lds_void_t)(base + C::kStageA + (j * C::kThreads + wave * 64) * 16), 16,
          kk < K ? pb[j] + lsk::pair_koff(kk, pairs & 2) : lsk::kOob, 0, 0, 0);
    }
  }
}

template <int MODE>
__global__ __launch_bounds__(512, 1) void moe_pp256p_kernel(MoeGemmArgs a) {
  using C = PPM256;
  extern __shared__ __attribute__((aligned(16))) char smem_moe[];
  const int ntiles = MODE == 0 ? (a.N + 127) / 128 : (a.N + 255) / 256;
  const int total = a.tiles[0] * ntiles;
  if ((int)blockIdx.x >= total) return;  // the whole block leaves: no barrier is left waiting
  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
  const int wm = wave / C::kWN, wn = wave % C::kWN;
  float* sc_asc = (float*)(smem_moe + C::kMainBytes);
  float* sc_w = sc_asc + 256;
  int* sc_dst = (int*)(sc_w + 256);
  float* sc_ws = (float*)(sc_dst + 256);
  float* sc_b = sc_ws + 256;
  const int apairs = (MODE == 1 ? (a.pairs & 1) : 0) | (a.pairs & 2);
  __amdgpu_buffer_rsrc_t ra = lsk::make_rsrc(a.A, a.a_bytes);

  struct Tile {
    int p0, p1, nt;
    const int8_t* wb;
    typename C::RowsA pa;
    typename C::RowsB pb;
    float r_asc, r_w, c_ws, c_b;
    int r_dst;
  };
  auto setup = [&](int v, Tile& t) {
    const int L = lsk::xcd_logical_id(v, total);
    const int mt = L / ntiles;
    t.nt = L - mt * ntiles;
    const int e = a.tiles[1 + 2 * mt];
    t.p0 = a.tiles[2 + 2 * mt];
    t.p1 = min(a.offs[e + 1], t.p0 + 256);
    t.wb = (const int8_t*)a.w_ptrs[e];
    const float* ws = (const float*)a.ws_ptrs[e];
    const float* bias = a.b_ptrs ? (const float*)a.b_ptrs[e] : nullptr;
    // weight row of local column c (gate/up interleave) and its h- or output column
    auto wrow_of = [&](int c, int& hc) {
      if (MODE == 0) {
        const int blk = c >> 5;
        hc = t.nt * 128 + (blk >> 1) * 32 + (c & 31);
        return (blk & 1) ? a.N + hc : hc;
      }
      hc = t.nt * 256 + c;
      return hc;
    };
    t.r_asc = t.r_w = t.c_ws = t.c_b = 0.0f;
    t.r_dst = 0;
    if (tid < 256) {
      const int p = t.p0 + tid;
      if (p < t.p1) {
        if (MODE == 0) {
          t.r_asc = a.a_scale[a.row_tok[p]];
        } else {
          t.r_asc = a.a_scale[p];
          t.r_w = a.row_w ? a.row_w[p] : 1.0f;
          t.r_dst = a.row_dst ? a.row_dst[p] : p;
        }
      }
      int hc;
      const int wr = wrow_of(tid, hc);
      if (hc < a.N) {
        t.c_ws = ws[wr];
        if (bias) t.c_b = bias[wr];
      }
    }
#pragma unroll
    for (int j = 0; j < C::kLA; ++j) {
      int row, kb;
      lsk::pp_slot<C::kThreads, C::kChunks>(tid, j, row, kb);
      const int p = t.p0 + row;
      const int src = p < t.p1 ? (MODE == 0 ? a.row_tok[p] : p) : -1;
      const uint32_t ro = (MODE == 1 && (a.pairs & 1)) ? (uint32_t)((src >> 1) * 2 * a.lda + (src & 1) * 64)
                                                        : (uint32_t)(src * a.lda);
      t.pa[j] = src >= 0 ? ro : lsk::kOob;
    }
#pragma unroll
    for (int j = 0; j < C::kLB; ++j) {
      int row, kb, hc;
      lsk::pp_slot<C::kThreads, C::kChunks>(tid, j, row, kb);
      const int wr = wrow_of(row, hc);
      const uint32_t ro = (a.pairs & 2) ? (uint32_t)((wr >> 1) * 2 * a.ldw + (wr & 1) * 64) : (uint32_t)(wr * a.ldw);
      t.pb[j] = hc < a.N ? ro : lsk::kOob;
    }
  };

  // ring slots 0 .. kRing - 1 take the first tile's first stages; later tiles' are issued under the
  // previous tile's epilogue (no wave reads the ring any more by then)
  Tile cur;
  setup(blockIdx.x, cur);
  moe256_issue_ring(ra, cur.pa, lsk::make_rsrc(cur.wb, a.w_bytes), cur.pb, a.K, smem_moe, apairs);
  for (int v = blockIdx.x; v < total; v += gridDim.x) {
    typename C::Acc acc;
#pragma unroll
    for (int i = 0; i < C::TM; ++i)
#pragma unroll
      for (int j = 0; j < C::TN; ++j) acc[i][j] = lsk::zero16();
    const int na = max(0, min(C::TM, (cur.p1 - cur.p0 - wm * C::WTM + 31) / 32));
    lsk::pp_mainloop<256, 256, 4, 2, 4, 64, true, true, true>(acc, ra, cur.pa, lsk::make_rsrc(cur.wb, a.w_bytes),
                                                              cur.pb, a.K, smem_moe, na, apairs);
    // every wave is past its last ring read; the previous tile's epilogue (the last reader of the
    // parked operands) ended before this tile's first barrier
    if (tid < 256) {
      sc_asc[tid] = cur.r_asc;
      sc_w[tid] = cur.r_w;
      sc_dst[tid] = cur.r_dst;
      sc_ws[tid] = cur.c_ws;
      sc_b[tid] = cur.c_b;
    }
    const int p0 = cur.p0, p1 = cur.p1, nt = cur.nt;
    if (v + (int)gridDim.x < total) {
      setup(v + gridDim.x, cur);
      moe256_issue_ring(ra, cur.pa, lsk::make_rsrc(cur.wb, a.w_bytes), cur.pb, a.K, smem_moe, apairs);
    }
    __syncthreads();

    // the lane's epilogue indices, derived afresh per tile (not kept live through the main loop)
    int tid_e = tid;
    asm volatile("" : "+v"(tid_e));
    const int lane_e = tid_e & 63, half = lane_e >> 5, col = lane_e & 31, odd = lane_e & 1;
    const bool bias = a.b_ptrs != nullptr;
    // rows outermost (register pairs r, r + 1), columns innermost: a row's parked operands are read
    // once and only two rows' worth are live next to the accumulators
#pragma unroll
    for (int i = 0; i < C::TM; ++i) {
      if (i >= na) break;
      const int rbase = wm * C::WTM + i * 32 + 4 * half;  // tile row of register 0
      if (MODE == 1) {
#pragma unroll
        for (int r = 0; r < 16; r += 2) {
          const int ml0 = rbase + 8 * (r >> 2) + (r & 3);  // rows of registers r and r + 1
          const int ml = ml0 + odd;                         // the row this lane stores
          const float asc0 = sc_asc[ml0], asc1 = sc_asc[ml0 + 1];
          const float w0 = sc_w[ml0], w1 = sc_w[ml0 + 1];
          const bool live = p0 + ml < p1;
          uint16_t* yrow = a.y + (int64_t)sc_dst[ml] * a.N;
#pragma unroll
          for (int j = 0; j < C::TN; ++j) {
            const int cl = wn * C::WTN + j * 32 + col;
            const int n2 = (nt * 256 + cl) & ~1;  // the even column of this lane's pair
            const float ws = sc_ws[cl], b = sc_b[cl];
            float y0 = bfr(f32_mul(f32_mul((float)acc[i][j][r], ws), asc0));
            float y1 = bfr(f32_mul(f32_mul((float)acc[i][j][r + 1], ws), asc1));
            if (bias) {
              y0 = bfr(f32_add(y0, b));
              y1 = bfr(f32_add(y1, b));
            }
            const float o0 = f32_mul(w0, y0), o1 = f32_mul(w1, y1);
            // even lanes keep register r's row, odd lanes register r + 1's
            const float got = __shfl_xor(odd ? o0 : o1, 1, 64);
            const float lo = odd ? got : o0, hi = odd ? o1 : got;
            if (live && n2 < a.N) {
              uint16_t* dst = yrow + n2;
              if (n2 + 1 < a.N) *(uint32_t*)dst = pack_bf16x2(lo, hi);
              else dst[0] = f32_to_bf16(lo);
            }
          }
        }
      } else {
        float am[16];
#pragma unroll
        for (int r = 0; r < 16; r += 2) {
          const int ml0 = rbase + 8 * (r >> 2) + (r & 3);
          const int ml = ml0 + odd;
          const float asc0 = sc_asc[ml0], asc1 = sc_asc[ml0 + 1];
          const bool live = p0 + ml < p1;
          uint16_t* hrow = a.h + (int64_t)(p0 + ml) * a.N;
          am[r] = am[r + 1] = 0.0f;
#pragma unroll
          for (int t = 0; t < 2; ++t) {
            const int cg = wn * C::WTN + 2 * t * 32 + col;  // gate column in the tile; up at + 32
            const int hc = nt * 128 + wn * 64 + t * 32 + col;
            const int h2 = hc & ~1;
            const float wsg = sc_ws[cg], wsu = sc_ws[cg + 32];
            float hv[2];
#pragma unroll
            for (int h = 0; h < 2; ++h) {
              const float asc = h ? asc1 : asc0;
              float yg = bfr(f32_mul(f32_mul((float)acc[i][2 * t][r + h], wsg), asc));
              float yu = bfr(f32_mul(f32_mul((float)acc[i][2 * t + 1][r + h], wsu), asc));
              if (bias) {
                yg = bfr(f32_add(yg, sc_b[cg]));
                yu = bfr(f32_add(yu, sc_b[cg + 32]));
              }
              hv[h] = a.act_tab ? lsk::act_from_entry(a.act, a.act_tab[__float_as_uint(yg) >> 16], yu)
                                : lsk::act_eval(a.act, yg, yu, a.frac, nullptr);
              if (hc < a.N) am[r + h] = fmaxf(am[r + h], fabsf(hv[h]));
            }
            const float got = __shfl_xor(odd ? hv[0] : hv[1], 1, 64);
            const float lo = odd ? got : hv[0], hi = odd ? hv[1] : got;
            if (live && h2 < a.N) {
              uint16_t* dst = hrow + h2;
              if (h2 + 1 < a.N) *(uint32_t*)dst = pack_bf16x2(lo, hi);
              else dst[0] = f32_to_bf16(lo);
            }
          }
        }
        // each row's maximum over the 32 lanes holding it (this wave's 64 h-columns of the row; the
        // maximum is order-free)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
#pragma unroll
          for (int o = 1; o < 32; o <<= 1) am[r] = fmaxf(am[r], __shfl_xor(am[r], o, 64));
          const int ml = rbase + 8 * (r >> 2) + (r & 3);
          if (col == 0 && p0 + ml < p1) atomicMax(&a.h_amax[p0 + ml], __float_as_uint(am[r]));
        }
      }
    }
  }
}

template <int MODE>
__global__ __launch_bounds__(512, 1) void moe_pp128_kernel(MoeGemmArgs a) {
  extern __shared__ __attribute__((aligned(16))) char smem_moe[];
  moe_tile<PPM128, MODE>(a, smem_moe,
                         [](PPM128::Acc& acc, __amdgpu_buffer_rsrc_t ra, const PPM128::RowsA& pa,
                            __amdgpu_buffer_rsrc_t rb, const PPM128::RowsB& pb, int K, char* sm, int na, int pairs) {
                           lsk::pp_mainloop<128, 256, 2, 4, 3, 128, false, true>(acc, ra, pa, rb, pb, K, sm, na, pairs);
                         });
}

template <int MODE>
__global__ __launch_bounds__(256, 2) void moe_w4_kernel(MoeGemmArgs a) {
  extern __shared__ __attribute__((aligned(16))) char smem_moe[];
  moe_tile<W4M, MODE>(a, smem_moe,
                      [](W4M::Acc& acc, __amdgpu_buffer_rsrc_t ra, const W4M::RowsA& pa, __amdgpu_buffer_rsrc_t rb,
                         const W4M::RowsB& pb, int K, char* sm, int, int) {
                        lsk::w4_mainloop<W4M>(acc, ra, pa, rb, pb, K, sm);  // row-major A only
                      });
}

// ---------------------------------------------------------------- decode-sized grouped GEMV
// One step of the transposing butterfly per level, sizes compile-time so the values stay in
// registers: with N values left, a lane with bit O set keeps the upper half and adds the
// partner's (lane ^ O) upper half; the other lane the lower halves.
template <int N, int O>
LSK_DEV void wave_xchg_sum(int* v, int lane) {
  if constexpr (N > 1) {
    const bool upper = (lane & O) != 0;
#pragma unroll
    for (int q = 0; q < N / 2; ++q) {
      const int send = upper ? v[q] : v[q + N / 2];
      const int keep = upper ? v[q + N / 2] : v[q];
      v[q] = keep + __shfl_xor(send, O, 64);
    }
    wave_xchg_sum<N / 2, O / 2>(v, lane);
  }
}

// Few rows per expert (decode token counts).  A wave owns RPW columns of one expert tile and
// loads their weight rows whole, once (non-temporal 16-byte loads, all in flight together; MODE
// 0 reads gate row c and up row N + c of h-column c), then multiplies them with the tile's
// activation rows MR at a time (v_dot4 into exact int32; the weights stay in registers).  The
// V = RPW x rows x MR partial sums of a lane are summed over the wave by a transposing
// butterfly: at offset o a lane keeps half of its values and adds the partner's other half, so
// after log2(V) steps lane l holds value l / (64 / V) (then plain steps over the rest).  Owner
// lanes apply the tiled kernels' epilogue steps: MODE 0 writes the bias-added gate and up values
// (bf16) for the activation-and-requant kernel; MODE 1 the routing-weighted output slot rows.
template <int MODE, int MR, int NC, int RPW>
__global__ __launch_bounds__(256) void moe_gemv_kernel(MoeGemmArgs a, uint16_t* __restrict__ gu) {
  constexpr int kRows = MODE == 0 ? 2 : 1;  // weight rows per column
  constexpr int V = RPW * kRows * MR;       // value index v = (i * MR + m) * kRows + r
  static_assert(V >= 2 && V <= 64 && (V & (V - 1)) == 0, "a power of two of at most 64 values");
  constexpr int kRep = 64 / V;  // lanes holding each value after the exchange steps
  const int cols_blk = 4 * RPW;
  const int nchunk = (a.N + cols_blk - 1) / cols_blk;
  const int mt = blockIdx.x / nchunk, ch = blockIdx.x - mt * nchunk;
  if (mt >= a.tiles[0]) return;
  const int e = a.tiles[1 + 2 * mt];
  const int p0 = a.tiles[2 + 2 * mt];
  const int p1 = min(a.offs[e + 1], p0 + kBM);
  const int lane = threadIdx.x & 63, wave = wave_id();
  const int c0 = ch * cols_blk + wave * RPW;
  const __amdgpu_buffer_rsrc_t rw = lsk::make_rsrc((const void*)a.w_ptrs[e], a.w_bytes);
  const __amdgpu_buffer_rsrc_t ra = lsk::make_rsrc(a.A, a.a_bytes);
  uint32_t koff[NC];
#pragma unroll
  for (int j = 0; j < NC; ++j) {
    const int kk = j * 1024 + lane * 16;
    koff[j] = kk < a.K ? (uint32_t)kk : lsk::kOob;
  }
  v4i w[RPW][kRows][NC];
#pragma unroll
  for (int i = 0; i < RPW; ++i)
#pragma unroll
    for (int r = 0; r < kRows; ++r) {
      const int c = c0 + i;
      const uint32_t ro = c < a.N ? (uint32_t)((MODE == 0 && r ? a.N + c : c) * a.ldw) : lsk::kOob;
#pragma unroll
      for (int j = 0; j < NC; ++j)
        w[i][r][j] = __builtin_bit_cast(
            v4i, __builtin_amdgcn_raw_buffer_load_b128(rw, (ro == lsk::kOob || koff[j] == lsk::kOob) ? lsk::kOob
                                                                                                   : ro + koff[j],
                                                       0, 2 /* non-temporal */));
    }
  // the value this lane ends with: column vi_i, row vi_m of the chunk, gate (0) or up (1)
  const int vi = lane / kRep;
  const int vi_i = vi / (MR * kRows), vi_m = (vi / kRows) % MR, vi_r = vi % kRows;
  const int c = c0 + vi_i;
  const bool owner = (lane % kRep) == 0 && vi_r == 0 && c < a.N;
  const float* ws = (const float*)a.ws_ptrs[e];
  const float* bias = a.b_ptrs ? (const float*)a.b_ptrs[e] : nullptr;
  float ws0 = 0.0f, ws1 = 0.0f, b0 = 0.0f, b1 = 0.0f;
  if (owner) {
    ws0 = ws[c];
    if (bias) b0 = bias[c];
    if (MODE == 0) {
      ws1 = ws[a.N + c];
      if (bias) b1 = bias[a.N + c];
    }
  }
  for (int rb = p0; rb < p1; rb += MR) {
    v4i act[MR][NC];
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      const int p = rb + m;
      const int src = p < p1 ? (MODE == 0 ? a.row_tok[p] : p) : -1;
#pragma unroll
      for (int j = 0; j < NC; ++j)
        act[m][j] = lsk::buf_load16(ra, (src >= 0 && koff[j] != lsk::kOob) ? (uint32_t)(src * a.lda) + koff[j]
                                                                           : lsk::kOob);
    }
    const int p = rb + vi_m;
    const bool rowok = owner && p < p1;
    float asc = 0.0f, wt = 0.0f;
    int dst = 0;
    if (rowok) {
      asc = a.a_scale[MODE == 0 ? a.row_tok[p] : p];
      if (MODE == 1) {
        wt = a.row_w ? a.row_w[p] : 1.0f;
        dst = a.row_dst ? a.row_dst[p] : p;
      }
    }
    int v[V];
#pragma unroll
    for (int i = 0; i < RPW; ++i)
#pragma unroll
      for (int m = 0; m < MR; ++m)
#pragma unroll
        for (int r = 0; r < kRows; ++r) {
          int t = 0;
#pragma unroll
          for (int j = 0; j < NC; ++j) {
            t = __builtin_amdgcn_sdot4(act[m][j][0], w[i][r][j][0], t, false);
            t = __builtin_amdgcn_sdot4(act[m][j][1], w[i][r][j][1], t, false);
            t = __builtin_amdgcn_sdot4(act[m][j][2], w[i][r][j][2], t, false);
            t = __builtin_amdgcn_sdot4(act[m][j][3], w[i][r][j][3], t, false);
          }
          v[(i * MR + m) * kRows + r] = t;
        }
    wave_xchg_sum<V, 32>(v, lane);
    int tot = v[0];
#pragma unroll
    for (int o = kRep / 2; o > 0; o >>= 1) tot += __shfl_xor(tot, o, 64);
    const int upv = MODE == 0 ? __shfl_xor(tot, kRep, 64) : 0;
    if (rowok) {
      if (MODE == 0) {
        float yg = bfr(f32_mul(f32_mul((float)tot, ws0), asc));
        float yu = bfr(f32_mul(f32_mul((float)upv, ws1), asc));
        if (bias) {
          yg = bfr(f32_add(yg, b0));
          yu = bfr(f32_add(yu, b1));
        }
        uint16_t* row = gu + (int64_t)p * 2 * a.N;
        row[c] = f32_to_bf16(yg);
        row[a.N + c] = f32_to_bf16(yu);
      } else {
        float yv = bfr(f32_mul(f32_mul((float)tot, ws0), asc));
        if (bias) yv = bfr(f32_add(yv, b0));
        a.y[(int64_t)dst * a.N + c] = f32_to_bf16(f32_mul(wt, yv));
      }
    }
  }
}

// Few rows per expert (decode token counts), the weights streamed by the MFMA: a block takes
// GPB groups of 16 weight rows of one expert tile (MODE 0: rows 0 .. 2N-1, gate rows then up
// rows, so gu column = weight row; MODE 1: the N output columns); the KW waves of a group split
// its K steps.  Per chunk of up to MT x 16 of the tile's rows: each wave first issues its first D
// weight steps (they depend on nothing), the chunk's row sources go to LDS (MODE 0: the token
// rows; the wait counts only those, the weights stay in flight), then the A rows are copied into
// LDS by direct loads (1 KB of a row per instruction, zeros past K, row stride ldsk = a multiple
// of 1 KB plus 16 bytes) with the rows' scales, routing weights and slots behind them.  Lane l
// streams 16 bytes of weight row g * 16 + l % 16 at K-group l / 16 of every 64-byte step (PAIRS:
// the expert's row-pair copy, whole 128-byte lines per instruction) into the
// v_mfma_i32_16x16x64_i8 B operand, D steps in flight, the A fragments read from LDS one step
// ahead.  The K-slices' exact int32 sums are added in LDS; the group's first wave applies the
// epilogue of moe_gemv_kernel element by element: MODE 0 the bias-added gate / up values into
// gu, MODE 1 the routing-weighted slot rows.  Rows past the chunk read a clamped staged row and
// multiply zeros.
template <int MODE, int MT, int D, bool PAIRS>
__global__ __launch_bounds__(1024) void moe_skinny_kernel(MoeGemmArgs a, uint16_t* __restrict__ gu, int gpb, int kw,
                                                          int sets, int ldsk) {
  extern __shared__ __attribute__((aligned(16))) char smem_sk[];
  constexpr int CR = MT * 16;  // rows per chunk
  const int lane = threadIdx.x & 63, wave = wave_id(), nw = blockDim.x >> 6, tid = threadIdx.x;
  const int mt = blockIdx.x / sets, gs = blockIdx.x - (blockIdx.x / sets) * sets;
  if (mt >= a.tiles[0]) return;  // the whole block leaves
  const int e = a.tiles[1 + 2 * mt];
  const int p0 = a.tiles[2 + 2 * mt];
  const int p1 = min(a.offs[e + 1], p0 + kBM);
  const int K = a.K, steps = (K + 63) >> 6;
  const int NWR = MODE == 0 ? 2 * a.N : a.N;  // weight rows
  const int G = (NWR + 15) >> 4;
  const int g = gs * gpb + wave / kw;
  const int ks = wave - (wave / kw) * kw;
  const int sps = (steps + kw - 1) / kw;
  const int s0 = ks * sps;
  const int nst = g < G ? max(0, min(steps, s0 + sps) - s0) : 0;
  const int col = lane & 15, kg = lane >> 4;
  const int n = g * 16 + col;
  const bool mine = ks == 0 && g < G && n < NWR;
  // this lane's column operands
  const float* wsp = (const float*)a.ws_ptrs[e];
  const float* bp = a.b_ptrs ? (const float*)a.b_ptrs[e] : nullptr;
  const __amdgpu_buffer_rsrc_t rcs = lsk::make_rsrc(wsp, 4 * (int64_t)NWR);
  const __amdgpu_buffer_rsrc_t rcb = lsk::make_rsrc(bp, bp ? 4 * (int64_t)NWR : 0);
  const float c_ws = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rcs, mine ? (uint32_t)(4 * n) : lsk::kOob, 0, 0));
  const float c_b = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rcb, mine ? (uint32_t)(4 * n) : lsk::kOob, 0, 0));
  // the chunk's row sources and operands in LDS past the A rows (and past the reduction area)
  const int arows = CR * ldsk;
  int* r_src = (int*)(smem_sk + max(arows, nw * MT * 1024));
  float* r_asc = (float*)(r_src + CR);
  float* r_w = r_asc + CR;
  int* r_dst = (int*)(r_w + CR);
  const __amdgpu_buffer_rsrc_t rw = lsk::make_rsrc((const void*)a.w_ptrs[e], a.w_bytes);
  const uint32_t wrow = n < NWR ? (uint32_t)(PAIRS ? (n >> 1) * 2 * a.ldw + (n & 1) * 64 : n * a.ldw) : lsk::kOob;
  const uint32_t wbase = (g < G && n < NWR) ? wrow + (uint32_t)(PAIRS ? s0 * 128 + kg * 16 : s0 * 64 + kg * 16)
                                            : lsk::kOob;
  constexpr uint32_t kStep = PAIRS ? 128 : 64;
  const __amdgpu_buffer_rsrc_t ra = lsk::make_rsrc(a.A, a.a_bytes);
  const int cpr = (K + 1023) >> 10;
  lsk::compiler_fence();
  for (int q0 = p0; q0 < p1; q0 += CR) {
    const int nr = min(CR, p1 - q0);
    if (q0 > p0) __syncthreads();  // the previous chunk's LDS reads are done
    v4i w[D];
#pragma unroll
    for (int u = 0; u < D; ++u)
      w[u] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(rw, u < nst ? wbase + u * kStep : lsk::kOob,
                                                                           0, 2 /* non-temporal */));
    if (MODE == 0) {
      // the token rows of the chunk: loaded behind the weight steps, waited for alone
      const int src = tid < nr ? a.row_tok[q0 + tid] : 0;
      lsk::compiler_fence();
      if (tid < nr) r_src[tid] = src;
      __syncthreads();
    }
    // A rows into LDS, then the rows' operands (needed only by the epilogue)
    for (int c = wave; c < nr * cpr; c += nw) {
      const int r = c / cpr, j = c - (c / cpr) * cpr;
      const int kb = j * 1024 + lane * 16;
      const int src = MODE == 0 ? r_src[r] : q0 + r;
      const uint32_t off = kb < K ? (uint32_t)(src * a.lda + kb) : lsk::kOob;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (lsk::lds_void_t)(smem_sk + r * ldsk + j * 1024), 16, off, 0, 0, 0);
    }
    float o_asc = 0.0f, o_w = 1.0f;
    int o_dst = 0;
    if (tid < nr) {
      const int p = q0 + tid;
      o_asc = a.a_scale[MODE == 0 ? r_src[tid] : p];
      if (MODE == 1) {
        o_w = a.row_w ? a.row_w[p] : 1.0f;
        o_dst = a.row_dst ? a.row_dst[p] : p;
      }
    }
    lsk::compiler_fence();
    lsk::wait_vm<0>();  // A, the rows' operands and the first weight steps
    if (tid < nr) {
      r_asc[tid] = o_asc;
      r_w[tid] = o_w;
      r_dst[tid] = o_dst;
    }
    __syncthreads();
    v4i acc[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) acc[t] = lsk::zero4();
    if (nst > 0) {
      const char* arow[MT];
      bool alive[MT];
#pragma unroll
      for (int t = 0; t < MT; ++t) {
        const int r = t * 16 + col;
        alive[t] = r < nr;
        arow[t] = smem_sk + (r < nr ? r : nr - 1) * ldsk + s0 * 64 + kg * 16;
      }
      for (int s = 0; s < nst; s += D) {
        v4i af[2][MT];
#pragma unroll
        for (int t = 0; t < MT; ++t) af[0][t] = *(const v4i*)(arow[t] + s * 64);
#pragma unroll
        for (int u = 0; u < D; ++u) {
          if (u + 1 < D) {
            const int st = s + u + 1 < nst ? s + u + 1 : 0;
#pragma unroll
            for (int t = 0; t < MT; ++t) af[(u + 1) & 1][t] = *(const v4i*)(arow[t] + st * 64);
          }
#pragma unroll
          for (int t = 0; t < MT; ++t)
            acc[t] = lsk::mfma_i8(alive[t] ? af[u & 1][t] : lsk::zero4(), w[u], acc[t]);
          const int nx = s + u + D;
          w[u] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(
                                             rw, nx < nst ? wbase + nx * kStep : lsk::kOob, 0, 2 /* non-temporal */));
        }
      }
    }
    if (kw > 1) {
      __syncthreads();  // every wave is past its last A read: the partial sums reuse the LDS
      v4i* red = (v4i*)smem_sk;
#pragma unroll
      for (int t = 0; t < MT; ++t) red[(wave * MT + t) * 64 + lane] = acc[t];
      __syncthreads();
      if (ks == 0)
        for (int j = 1; j < kw; ++j)
#pragma unroll
          for (int t = 0; t < MT; ++t) acc[t] += red[((wave + j) * MT + t) * 64 + lane];
    }
    if (mine) {
#pragma unroll
      for (int t = 0; t < MT; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int m = t * 16 + kg * 4 + r;
          if (m < nr) {
            float yv = bfr(f32_mul(f32_mul((float)acc[t][r], c_ws), r_asc[m]));
            if (bp) yv = bfr(f32_add(yv, c_b));
            if (MODE == 0) gu[(int64_t)(q0 + m) * NWR + n] = f32_to_bf16(yv);
            else a.y[(int64_t)r_dst[m] * a.N + n] = f32_to_bf16(f32_mul(r_w[m], yv));
          }
        }
    }
  }
}

// The first launch of a one-token int8 layer routed from its logits: the router, the row quant of x
// and the gate/up GEMV in one kernel.  Every wave routes the token itself (route_select: the same
// arithmetic as router_topk_kernel) and quantises the whole row of x in registers (its lanes hold
// the row's 16-element K chunks; the maximum is a wave reduction; rowquant's arithmetic), so no wave
// waits on another; block (s, chunk) then takes the expert in slot s (the k experts ascending),
// streams its RPW columns' gate and up weight rows and writes the bias-added gate and up values, as
// moe_gemv_kernel's MODE 0 does for one row.  Block 0's first wave also writes the routing outputs
// (idx_out / w_out in rank order) and the token's dispatch: offs, the tile table (slot s = the s-th
// expert ascending, row s), row_tok / row_dst / row_w, tok_cnt and ascx, which the act + requant and
// the down + combine launches read.  H = a.K, H % 16 == 0, H <= 1024 NC; k <= 8; E <= 64 EPL.
template <int NC, int RPW, int EPL>
__global__ __launch_bounds__(256) void moe_route_gemv1_kernel(MoeGemmArgs a, uint16_t* __restrict__ gu,
                                                              const uint16_t* __restrict__ x, const void* __restrict__ g,
                                                              int gdt, int E, int k, int renorm,
                                                              const int32_t* __restrict__ rtab,
                                                              int64_t* __restrict__ idx_out,
                                                              uint16_t* __restrict__ w_out, int32_t* __restrict__ offs,
                                                              int32_t* __restrict__ tiles, int32_t* __restrict__ row_tok,
                                                              int32_t* __restrict__ row_dst, float* __restrict__ row_w,
                                                              int32_t* __restrict__ tok_cnt, float* __restrict__ ascx) {
  const int cols_blk = 4 * RPW;
  const int nchunk = (a.N + cols_blk - 1) / cols_blk;
  const int mt = blockIdx.x / nchunk, ch = blockIdx.x - mt * nchunk;
  if (mt >= k) return;  // whole blocks; no barrier follows
  const int lane = threadIdx.x & 63, wave = wave_id();
  const int H = a.K;
  uint32_t koff[NC];
#pragma unroll
  for (int j = 0; j < NC; ++j) {
    const int kk = j * 1024 + lane * 16;
    koff[j] = kk < H ? (uint32_t)kk : lsk::kOob;
  }
  // the row of x (bf16): this lane's K chunks, requested before the routing
  uint4 xr[NC][2];
#pragma unroll
  for (int j = 0; j < NC; ++j) {
    xr[j][0] = xr[j][1] = make_uint4(0, 0, 0, 0);
    if (koff[j] != lsk::kOob) {
      xr[j][0] = *(const uint4*)(x + koff[j]);
      xr[j][1] = *(const uint4*)(x + koff[j] + 8);
    }
  }
  // the routing: lane r < k holds the rank-r expert; pos = its slot among the k experts ascending
  int e_r, s_r, S;
  route_select<EPL>(g, gdt, E, 0, E, k, renorm, rtab, e_r, s_r, S);
  int ek[8];  // the k experts in rank order, in every lane (gathered with the whole wave active)
#pragma unroll
  for (int j = 0; j < 8; ++j) ek[j] = __shfl(e_r, j < k ? j : 0, 64);
  int pos = 0;
#pragma unroll
  for (int j = 0; j < 8; ++j) pos += (j < k && ek[j] < e_r) ? 1 : 0;
  const uint64_t sel = __builtin_amdgcn_ballot_w64(lane < k && pos == mt);
  const int e = __shfl(e_r, (int)__builtin_ctzll(sel), 64);

  // this wave's weight rows: gate c and up N + c of columns c0 .. c0 + RPW - 1
  const int c0 = ch * cols_blk + wave * RPW;
  const __amdgpu_buffer_rsrc_t rw = lsk::make_rsrc((const void*)a.w_ptrs[e], a.w_bytes);
  v4i w[RPW][2][NC];
#pragma unroll
  for (int i = 0; i < RPW; ++i)
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const int c = c0 + i;
      const uint32_t ro = c < a.N ? (uint32_t)((r ? a.N + c : c) * a.ldw) : lsk::kOob;
#pragma unroll
      for (int j = 0; j < NC; ++j)
        w[i][r][j] = __builtin_bit_cast(
            v4i, __builtin_amdgcn_raw_buffer_load_b128(rw, (ro == lsk::kOob || koff[j] == lsk::kOob) ? lsk::kOob
                                                                                                   : ro + koff[j],
                                                       0, 2 /* non-temporal */));
    }
  // the row quant of x (every wave holds the whole row)
  float xv[NC][16];
  float am = 0.0f;
#pragma unroll
  for (int j = 0; j < NC; ++j) {
    const uint32_t wd[8] = {xr[j][0].x, xr[j][0].y, xr[j][0].z, xr[j][0].w,
                            xr[j][1].x, xr[j][1].y, xr[j][1].z, xr[j][1].w};
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      xv[j][2 * q] = bf16_to_f32((uint16_t)(wd[q] & 0xffff));
      xv[j][2 * q + 1] = bf16_to_f32((uint16_t)(wd[q] >> 16));
      am = fmaxf(am, fmaxf(fabsf(xv[j][2 * q]), fabsf(xv[j][2 * q + 1])));
    }
  }
  am = wave_fmax(am);
  const float sc = f32_div(fmaxf(am, kAmaxFloor), 127.0f), rs = f32_div(1.0f, sc);
  v4i act[NC];
#pragma unroll
  for (int j = 0; j < NC; ++j) {
    float lo8[8], hi8[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      lo8[q] = xv[j][q];
      hi8[q] = xv[j][8 + q];
    }
    const uint2 p0 = quant8_pack(lo8, sc, rs), p1 = quant8_pack(hi8, sc, rs);
    act[j] = v4i{(int)p0.x, (int)p0.y, (int)p1.x, (int)p1.y};
  }

  // block 0's first wave: the routing outputs and the one-token dispatch
  if (blockIdx.x == 0 && wave == 0) {
    if (lane < k) {
      const uint16_t wb = f32_to_bf16(f32_div((float)s_r, (float)S));
      idx_out[lane] = e_r;
      w_out[lane] = wb;
      tiles[1 + 2 * pos] = e_r;
      tiles[2 + 2 * pos] = pos;
      row_tok[pos] = 0;
      row_dst[pos] = pos;
      row_w[pos] = bf16_to_f32(wb);
    }
    for (int ee = lane; ee <= E; ee += 64) {
      int before = 0;
#pragma unroll
      for (int j = 0; j < 8; ++j) before += (j < k && ek[j] < ee) ? 1 : 0;
      offs[ee] = before;
    }
    if (lane == 0) {
      tiles[0] = k;
      tok_cnt[0] = k;
      ascx[0] = sc;
    }
  }

  // the gate / up dot products, reduced over the wave, and the epilogue of each column
  constexpr int V = RPW * 2;
  constexpr int kRep = 64 / V;
  const int vi = lane / kRep;
  const int vi_i = vi / 2, vi_r = vi % 2;
  const int c = c0 + vi_i;
  const bool owner = (lane % kRep) == 0 && vi_r == 0 && c < a.N;
  const float* ws = (const float*)a.ws_ptrs[e];
  const float* bias = a.b_ptrs ? (const float*)a.b_ptrs[e] : nullptr;
  float ws0 = 0.0f, ws1 = 0.0f, b0 = 0.0f, b1 = 0.0f;
  if (owner) {
    ws0 = ws[c];
    ws1 = ws[a.N + c];
    if (bias) {
      b0 = bias[c];
      b1 = bias[a.N + c];
    }
  }
  int v[V];
#pragma unroll
  for (int i = 0; i < RPW; ++i)
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      int t = 0;
#pragma unroll
      for (int j = 0; j < NC; ++j) {
        t = __builtin_amdgcn_sdot4(act[j][0], w[i][r][j][0], t, false);
        t = __builtin_amdgcn_sdot4(act[j][1], w[i][r][j][1], t, false);
        t = __builtin_amdgcn_sdot4(act[j][2], w[i][r][j][2], t, false);
        t = __builtin_amdgcn_sdot4(act[j][3], w[i][r][j][3], t, false);
      }
      v[i * 2 + r] = t;
    }
  wave_xchg_sum<V, 32>(v, lane);
  int tot = v[0];
#pragma unroll
  for (int o = kRep / 2; o > 0; o >>= 1) tot += __shfl_xor(tot, o, 64);
  const int upv = __shfl_xor(tot, kRep, 64);
  if (owner) {
    float yg = bfr(f32_mul(f32_mul((float)tot, ws0), sc));
    float yu = bfr(f32_mul(f32_mul((float)upv, ws1), sc));
    if (bias) {
      yg = bfr(f32_add(yg, b0));
      yu = bfr(f32_add(yu, b1));
    }
    uint16_t* row = gu + (int64_t)mt * 2 * a.N;
    row[c] = f32_to_bf16(yg);
    row[a.N + c] = f32_to_bf16(yu);
  }
}

// The down projection and the combine of a one-token layer in one launch (the decode GEMV path at
// T = 1).  The token's routed rows are its experts in ascending order, one row each (row s = slot
// s, expert tiles[1 + 2 s]), so a wave owning RPW output columns computes every slot's value for
// them -- moe_gemv_kernel's MODE 1 value bfr(w * bfr(fl32(fl32(acc) * ws[c]) * asc)) (with a bias
// bfr(... + b[c]) first) -- and adds the slots in order from +0 as moe_combine_kernel does (then
// bfr(shared[c])), writing y directly: no slot rows and no combine launch.  All weight and
// activation loads of a wave are issued together; the KMAX x RPW exact int32 sums are reduced by
// the transposing butterfly, and the column's owner lane gathers the slot values by shuffles.
template <int NC, int RPW, int KMAX>
__global__ __launch_bounds__(256) void moe_down_combine1_kernel(MoeGemmArgs a, const float* __restrict__ shared,
                                                               uint16_t* __restrict__ out) {
  constexpr int V = KMAX * RPW;
  static_assert(V >= 2 && V <= 64 && (V & (V - 1)) == 0, "a power of two of at most 64 values");
  constexpr int kRep = 64 / V;
  const int lane = threadIdx.x & 63, wave = wave_id();
  const int c0 = (blockIdx.x * 4 + wave) * RPW;
  if (c0 >= a.N) return;  // whole waves; no barrier follows
  const int n = a.tiles[0];  // routed rows (the host checks k <= KMAX)
  uint32_t koff[NC];
#pragma unroll
  for (int j = 0; j < NC; ++j) {
    const int kk = j * 1024 + lane * 16;
    koff[j] = kk < a.K ? (uint32_t)kk : lsk::kOob;
  }
  const __amdgpu_buffer_rsrc_t ra = lsk::make_rsrc(a.A, a.a_bytes);
  int es[KMAX];
  v4i wv[KMAX][RPW][NC], xv[KMAX][NC];
#pragma unroll
  for (int s = 0; s < KMAX; ++s) {
    es[s] = s < n ? a.tiles[1 + 2 * s] : 0;
    const __amdgpu_buffer_rsrc_t rw = lsk::make_rsrc((const void*)a.w_ptrs[es[s]], s < n ? a.w_bytes : 0);
#pragma unroll
    for (int i = 0; i < RPW; ++i) {
      const uint32_t ro = c0 + i < a.N ? (uint32_t)((c0 + i) * a.ldw) : lsk::kOob;
#pragma unroll
      for (int j = 0; j < NC; ++j)
        wv[s][i][j] = __builtin_bit_cast(
            v4i, __builtin_amdgcn_raw_buffer_load_b128(rw, (ro == lsk::kOob || koff[j] == lsk::kOob) ? lsk::kOob
                                                                                                    : ro + koff[j],
                                                       0, 2 /* non-temporal */));
    }
#pragma unroll
    for (int j = 0; j < NC; ++j)
      xv[s][j] = lsk::buf_load16(ra, (s < n && koff[j] != lsk::kOob) ? (uint32_t)(s * a.lda) + koff[j] : lsk::kOob);
  }
  // this lane's value after the exchange: slot vs, column c0 + vc; its epilogue operands
  const int vi = lane / kRep, vs = vi / RPW, vc = vi % RPW;
  const int c = c0 + vc;
  const bool live = vs < n && c < a.N;
  float ws = 0.0f, b = 0.0f, asc = 0.0f, wt = 0.0f;
  if (live) {
    ws = ((const float*)a.ws_ptrs[es[vs]])[c];
    if (a.b_ptrs) b = ((const float*)a.b_ptrs[es[vs]])[c];
    asc = a.a_scale[vs];
    wt = a.row_w[vs];
  }
  const float sh = (shared && vs == 0 && c < a.N) ? bfr(shared[c]) : 0.0f;
  int v[V];
#pragma unroll
  for (int s = 0; s < KMAX; ++s)
#pragma unroll
    for (int i = 0; i < RPW; ++i) {
      int t = 0;
#pragma unroll
      for (int j = 0; j < NC; ++j) {
        t = __builtin_amdgcn_sdot4(xv[s][j][0], wv[s][i][j][0], t, false);
        t = __builtin_amdgcn_sdot4(xv[s][j][1], wv[s][i][j][1], t, false);
        t = __builtin_amdgcn_sdot4(xv[s][j][2], wv[s][i][j][2], t, false);
        t = __builtin_amdgcn_sdot4(xv[s][j][3], wv[s][i][j][3], t, false);
      }
      v[s * RPW + i] = t;
    }
  wave_xchg_sum<V, 32>(v, lane);
  int tot = v[0];
#pragma unroll
  for (int o = kRep / 2; o > 0; o >>= 1) tot += __shfl_xor(tot, o, 64);
  float f = 0.0f;
  if (live) {
    float yv = bfr(f32_mul(f32_mul((float)tot, ws), asc));
    if (a.b_ptrs) yv = bfr(f32_add(yv, b));
    f = bfr(f32_mul(wt, yv));
  }
  // the column's slots in order from +0 (the combine), gathered from the lanes holding them
  float acc = 0.0f;
#pragma unroll
  for (int s = 0; s < KMAX; ++s) {
    const float g = __shfl(f, (s * RPW + vc) * kRep, 64);
    if (s < n) acc = f32_add(acc, g);
  }
  if (vs == 0 && (lane % kRep) == 0 && c < a.N) {
    if (shared) acc = f32_add(acc, sh);
    out[c] = f32_to_bf16(acc);
  }
}

// Decode path after the gate/up GEMV: per row, h = act(gate, up) (the values the tiled kernels
// store), its |h| maximum (fmaxf from +0, so a NaN is passed over as there), and the row quant
// of h exactly as moe_requant_kernel does it (int8, or its values as bf16 for the MX GEMV).
// One block of 1024 threads per row; I <= 1024 * PER.
template <int PER, bool OUT_BF16>
__global__ __launch_bounds__(1024) void moe_act_requant_kernel(const uint16_t* __restrict__ gu,
                                                              const int32_t* __restrict__ nrows, int I, int act,
                                                              const int32_t* __restrict__ frac,
                                                              const float* __restrict__ tab,
                                                              void* __restrict__ q, float* __restrict__ asc) {
  __shared__ float red[16];
  const int p = blockIdx.x;
  if (p >= *nrows) return;
  const int tid = threadIdx.x;
  const uint16_t* g = gu + (int64_t)p * 2 * I;
  const uint16_t* u = g + I;
  float hv[PER];
  float am = 0.0f;
#pragma unroll
  for (int t = 0; t < PER; ++t) {
    const int c = tid + 1024 * t;
    hv[t] = 0.0f;
    if (c < I) {
      const float yg = bf16_to_f32(g[c]), yu = bf16_to_f32(u[c]);
      hv[t] = lsk::act_eval(act, yg, yu, frac, tab);
      am = fmaxf(am, fabsf(hv[t]));
    }
  }
  am = wave_fmax(am);
  if ((tid & 63) == 0) red[tid >> 6] = am;
  __syncthreads();
  am = red[0];
#pragma unroll
  for (int w2 = 1; w2 < 16; ++w2) am = fmaxf(am, red[w2]);
  const float s = f32_div(fmaxf(am, kAmaxFloor), 127.0f), rs = f32_div(1.0f, s);
  if (tid == 0) asc[p] = s;
#pragma unroll
  for (int t = 0; t < PER; ++t) {
    const int c = tid + 1024 * t;
    if (c < I) {
      const float hb = bf16_to_f32(f32_to_bf16(hv[t]));  // h as the tiled kernels store it
      const float qv = fminf(fmaxf(rint_div8(hb, s, rs), -127.0f), 127.0f);
      if (OUT_BF16) ((uint16_t*)q)[(int64_t)p * I + c] = (uint16_t)(__float_as_uint(qv) >> 16);  // exact
      else ((int8_t*)q)[(int64_t)p * I + c] = (int8_t)(int)qv;
    }
  }
}

// Block-scaled activations after the skinny gate/up GEMM: h = act(gate, up) [R, I] bf16 from its
// bias-added values gu [R, 2I] (the values the tiled kernels store into h), unless a row of x was
// flagged (*any != 0: the general tile kernel then wrote h itself).  Grid-stride over R x I.
__global__ __launch_bounds__(256) void moe_act_h_kernel(const uint16_t* __restrict__ gu,
                                                        const int32_t* __restrict__ nrows, int I, int act,
                                                        const int32_t* __restrict__ frac,
                                                        const float* __restrict__ tab,
                                                        const int32_t* __restrict__ any, uint16_t* __restrict__ h) {
  if (*any != 0) return;
  const int64_t n = (int64_t)(*nrows) * I;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
    const int64_t p = i / I;
    const int64_t c = i - p * I;
    const uint16_t* g = gu + p * 2 * I;
    h[i] = f32_to_bf16(lsk::act_eval(act, bf16_to_f32(g[c]), bf16_to_f32(g[I + c]), frac, tab));
  }
}

// ---------------------------------------------------------------- requant and combine
// rowquant of the activation output h (bf16 values), with the row maxima from the GEMM; q row-major
// [R, I], or with pair in the row-pair layout the down tiles read (I % 64 == 0).  One wave per
// row (the row's scale and its reciprocal computed once), 8 elements per lane and step, two steps'
// loads in flight; rows w, w + (waves in the grid), ...
__global__ __launch_bounds__(256) void moe_requant_kernel(const uint16_t* __restrict__ h, const uint32_t* __restrict__ amax,
                                                          const int32_t* __restrict__ nrows, int I,
                                                          int8_t* __restrict__ q, float* __restrict__ asc, int pair) {
  const int R = *nrows;
  const int chunks = I / 8;
  const int lane = threadIdx.x & 63;
  const int nwaves = gridDim.x * 4;
  for (int p = blockIdx.x * 4 + wave_id(); p < R; p += nwaves) {
    const float s = f32_div(fmaxf(__uint_as_float(amax[p]), kAmaxFloor), 127.0f), rs = f32_div(1.0f, s);
    if (lane == 0) asc[p] = s;
    const uint16_t* hr = h + (int64_t)p * I;
    int8_t* qr = pair ? q + (int64_t)(p >> 1) * 2 * I + (p & 1) * 64 : q + (int64_t)p * I;
    for (int c0 = lane; c0 < chunks; c0 += 128) {
      uint4 u[2];
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const int c = c0 + 64 * t;
        u[t] = *(const uint4*)(hr + (c < chunks ? c : c0) * 8);
      }
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const int c = c0 + 64 * t;
        if (c >= chunks) continue;
        const uint32_t wd[4] = {u[t].x, u[t].y, u[t].z, u[t].w};
        uint32_t lo = 0, hi = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float v0 = bf16_to_f32((uint16_t)(wd[j] & 0xffff));
          const float v1 = bf16_to_f32((uint16_t)(wd[j] >> 16));
          float q0 = fminf(fmaxf(rint_div8(v0, s, rs), -127.0f), 127.0f);
          float q1 = fminf(fmaxf(rint_div8(v1, s, rs), -127.0f), 127.0f);
          const uint32_t b = ((uint32_t)(uint8_t)(int8_t)(int)q0) | (((uint32_t)(uint8_t)(int8_t)(int)q1) << 8);
          if (j < 2) lo |= b << (16 * j);
          else hi |= b << (16 * (j - 2));
        }
        const int k = c * 8;
        *(uint2*)(qr + (pair ? (k >> 6) * 128 + (k & 63) : k)) = make_uint2(lo, hi);
      }
    }
  }
}

// The R4 rotation of h followed by its row quant (moe_ref.py:112-113, 195-199 with rotation):
// one block per row; the row's bf16 values are widened into LDS, butterflied per blk-wide
// block in binary32, scaled, and quantised with the row's own maximum.
__global__ __launch_bounds__(256) void moe_rot_requant_kernel(const uint16_t* __restrict__ h,
                                                              const int32_t* __restrict__ nrows, int I, int blk,
                                                              float scale, int8_t* __restrict__ q,
                                                              float* __restrict__ asc) {
  extern __shared__ float rv[];
  __shared__ float red[4];
  const int64_t p = blockIdx.x;
  if (p >= *nrows) return;
  const int tid = threadIdx.x;
  for (int i = tid; i < I; i += 256) rv[i] = bf16_to_f32(h[p * I + i]);
  __syncthreads();
  const int half = blk / 2;
  for (int hh = 1; hh < blk; hh <<= 1) {
    for (int i = tid; i < I / 2; i += 256) {
      const int b = i / half, w = i - b * half;
      const int grp = w / hh, off = w - grp * hh;
      const int i0 = b * blk + grp * 2 * hh + off, i1 = i0 + hh;
      const float x0 = rv[i0], x1 = rv[i1];
      rv[i0] = f32_add(x0, x1);
      rv[i1] = x0 - x1;
    }
    __syncthreads();
  }
  float am = 0.0f;
  for (int i = tid; i < I; i += 256) {
    const float v = f32_mul(rv[i], scale);
    rv[i] = v;
    am = fmaxf(am, fabsf(v));
  }
  am = wave_fmax(am);
  if ((tid & 63) == 0) red[tid >> 6] = am;
  __syncthreads();
  am = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  const float s = f32_div(fmaxf(am, kAmaxFloor), 127.0f), rs = f32_div(1.0f, s);
  if (tid == 0) asc[p] = s;
  for (int i = tid; i < I; i += 256) {
    const float t = fminf(fmaxf(rint_div8(rv[i], s, rs), -127.0f), 127.0f);
    q[p * I + i] = (int8_t)(int)t;
  }
}

// y[t] = bf16( sum_r fl32(slot r of t) in ascending expert order, from +0 ) (+ bfr(shared[t]) last)
__global__ __launch_bounds__(256) void moe_combine_kernel(const uint16_t* __restrict__ slots, int64_t H, int k,
                                                          const int32_t* __restrict__ tok_cnt,
                                                          const float* __restrict__ shared, int64_t T,
                                                          uint16_t* __restrict__ out) {
  const int64_t chunks = H / 8;
  const int64_t total = T * chunks;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
    const int64_t t = i / chunks;
    const int64_t c = (i - t * chunks) * 8;
    float acc[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] = 0.0f;
    const int n = tok_cnt[t];
    // the token's slots four at a time, their loads issued together before the ordered adds
    for (int r0 = 0; r0 < n; r0 += 4) {
      uint4 u[4];
#pragma unroll
      for (int j = 0; j < 4; ++j)
        u[j] = r0 + j < n ? *(const uint4*)(slots + (t * k + r0 + j) * H + c) : make_uint4(0, 0, 0, 0);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if (r0 + j >= n) break;
        const uint32_t wd[4] = {u[j].x, u[j].y, u[j].z, u[j].w};
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          acc[2 * q] = f32_add(acc[2 * q], bf16_to_f32((uint16_t)(wd[q] & 0xffff)));
          acc[2 * q + 1] = f32_add(acc[2 * q + 1], bf16_to_f32((uint16_t)(wd[q] >> 16)));
        }
      }
    }
    if (shared) {
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[j] = f32_add(acc[j], bfr(shared[t * H + c + j]));
    }
    uint4 o;
    o.x = (uint32_t)f32_to_bf16(acc[0]) | ((uint32_t)f32_to_bf16(acc[1]) << 16);
    o.y = (uint32_t)f32_to_bf16(acc[2]) | ((uint32_t)f32_to_bf16(acc[3]) << 16);
    o.z = (uint32_t)f32_to_bf16(acc[4]) | ((uint32_t)f32_to_bf16(acc[5]) << 16);
    o.w = (uint32_t)f32_to_bf16(acc[6]) | ((uint32_t)f32_to_bf16(acc[7]) << 16);
    store16_split(out + t * H + c, o.x, o.y, o.z, o.w);
  }
}

// ---------------------------------------------------------------- workspace layout
struct MoeWs {
  int8_t* qx;
  float* ascx;
  int32_t* offs;
  int32_t* tiles;
  int32_t* row_tok;
  int32_t* row_dst;
  float* row_w;
  int32_t* tok_cnt;
  int32_t* ccnt;   // [chunks][E] per-chunk expert counts (T > 256)
  uint16_t* h;
  uint32_t* h_amax;
  int8_t* qh;
  float* asch;
  uint16_t* slots;
  float* xrot;
  uint16_t* gu;  // decode path: bias-added gate and up values [R, 2I] bf16 (T <= kGemvMaxT)
  int32_t* kax;    // block-scaled activations: block exponents of x [T, H/32] and of h [R, I/32],
  int32_t* flagx;  // and the row flags of each
  int32_t* kah;
  int32_t* flagh;
  int64_t bytes;
  int64_t max_tiles;
  int32_t* tiles2;     // the tile table in kBM2-row tiles
  int64_t max_tiles2;
};

inline int64_t up256(int64_t v) { return (v + 255) / 256 * 256; }

constexpr int64_t kGemvMaxT = 64;  // token counts the grouped GEMV may take
constexpr int64_t kSkinnyMaxT = 256;  // ... the skinny grouped GEMM

// Whether the ping-pong grouped GEMM runs on the 256 x 256 tiles: only when chosen
// (lsk_moe_select(5)).  One block per CU there leaves the load latency and the epilogue of a tile
// unhidden, which the two resident 128 x 256 blocks overlap: measured on MI355X, Qwen3-30B-A3B
// layer at 256 / 2048 / 4096 tokens 222 / 358 / 520 us against 169 / 299 / 425 us, the grouped
// gate/up and down stages at 16384 rows 179 / 137 us against 143 / 101 us, despite a third fewer
// operand bytes per MFMA.
static bool moe_uses_pp256(int64_t, int64_t) { return g_moe_w4 == 3 || g_moe_w4 == 4; }

// Whether the int8 grouped GEMMs of a layer run on moe_skinny_kernel: by size from 2 tokens up to
// where the ping-pong tiles take over (16 routed rows per expert) -- Qwen3-30B-A3B on MI355X, graph
// replays, us at T = 8 / 32 / 64 / 96 / 128 / 192: 51.3 / 65.0 / 85.4 / 113 / 143 / 149 against
// 56.2 / 94.0 / 129.6 on the grouped GEMV and 196 / 183 / 205 on the register-staged tile; at 256
// tokens the ping-pong tile 155 against 182 -- or whenever chosen (lsk_moe_select(7)); int8
// experts without rotation, T <= kSkinnyMaxT, H, I <= 4096 (a chunk of 32 rows in LDS).
static bool moe_takes_skinny(int64_t T, int k, int64_t E, int rb, int mx, int64_t H, int64_t I) {
  if (rb != 0 || mx || T > kSkinnyMaxT || H > 4096 || I > 4096) return false;
  return g_moe_force == 7 || (g_moe_force < 0 && T >= 2 && T * k < 16 * E);
}

constexpr int64_t kMxGemvMaxT = 24;   // ... with MXFP4 experts
constexpr int64_t kMx2GemvMaxT = 16;  // ... with MXFP4 experts and block-scaled activations

MoeWs moe_layout(char* base, int64_t T, int k, int64_t E, int64_t H, int64_t I, int rot_blk, int wfmt) {
  const int64_t qb = wfmt >= 1 ? 2 : 1;  // bytes per quantised activation element
  MoeWs w{};
  const int64_t R = T * k;
  w.max_tiles = R / kBM + (E < R ? E : R);
  w.max_tiles2 = R / kBM2 + (E < R ? E : R);
  int64_t off = 0;
  auto take = [&](int64_t nbytes) {
    char* p = base ? base + off : nullptr;
    off += up256(nbytes);
    return p;
  };
  w.qx = (int8_t*)take(T * H * qb);
  w.ascx = (float*)take(T * 4);
  w.offs = (int32_t*)take((E + 1) * 4);
  w.tiles = (int32_t*)take((1 + 2 * w.max_tiles) * 4);
  w.tiles2 = (int32_t*)take((1 + 2 * w.max_tiles2) * 4);
  w.row_tok = (int32_t*)take(R * 4);
  w.row_dst = (int32_t*)take(R * 4);
  w.row_w = (float*)take(R * 4);
  w.tok_cnt = (int32_t*)take(T * 4);
  const int64_t nchunks = (T + 255) / 256;
  w.ccnt = (int32_t*)take(nchunks * E * 4);
  w.h = (uint16_t*)take(R * I * 2);
  w.h_amax = (uint32_t*)take((R + 2) * 4);  // + the two "some row flagged" words of block-scaled activations
  w.qh = (int8_t*)take(((R + 1) & ~(int64_t)1) * I * qb);  // (room for a last row pair)
  w.asch = (float*)take(R * 4);
  w.slots = (uint16_t*)take(R * H * 2);
  w.xrot = rot_blk > 0 ? (float*)take(T * H * 4) : nullptr;
  w.gu = T <= std::max(kGemvMaxT, kSkinnyMaxT) ? (uint16_t*)take(R * 2 * I * 2) : nullptr;
  if (wfmt == 2) {
    w.kax = (int32_t*)take(T * (H / 32) * 4);
    w.flagx = (int32_t*)take(T * 4);
    w.kah = (int32_t*)take(R * (I / 32) * 4);
    w.flagh = (int32_t*)take(R * 4);
  }
  w.bytes = off;
  return w;
}

template <int MODE>
int launch_moe_pp(const MoeGemmArgs& ga, int64_t max_tiles, hipStream_t s, const char* name) {
  const int ntiles = MODE == 0 ? (ga.N + 127) / 128 : (ga.N + 255) / 256;
  const int64_t blocks = max_tiles * ntiles;
  if (blocks == 0) return LSK_OK;
  LSK_REQUIRE(blocks <= 0x7fffffff, "%s: grid too large", name);
  if (g_moe_w4 == 2) {
    static std::atomic<bool> attr_128{false};
    if (!attr_128) {
      if (hipFuncSetAttribute((const void*)moe_pp128_kernel<MODE>, hipFuncAttributeMaxDynamicSharedMemorySize,
                              moe_smem_bytes<PPM128>()) != hipSuccess) {
        lsk::set_error("%s: cannot reserve %d bytes of LDS", name, moe_smem_bytes<PPM128>());
        return LSK_ERR_HIP;
      }
      attr_128 = true;
    }
    hipLaunchKernelGGL(moe_pp128_kernel<MODE>, dim3((unsigned)blocks), dim3(512), moe_smem_bytes<PPM128>(), s, ga);
    return lsk::check_launch(name);
  }
  if (g_moe_w4) {
    static std::atomic<bool> attr_w4{false};
    if (!attr_w4) {
      if (hipFuncSetAttribute((const void*)moe_w4_kernel<MODE>, hipFuncAttributeMaxDynamicSharedMemorySize,
                              moe_smem_bytes<W4M>()) != hipSuccess) {
        lsk::set_error("%s: cannot reserve %d bytes of LDS", name, moe_smem_bytes<W4M>());
        return LSK_ERR_HIP;
      }
      attr_w4 = true;
    }
    hipLaunchKernelGGL(moe_w4_kernel<MODE>, dim3((unsigned)blocks), dim3(256), moe_smem_bytes<W4M>(), s, ga);
    return lsk::check_launch(name);
  }
  static std::atomic<bool> attr_set{false};
  if (!attr_set) {
    if (hipFuncSetAttribute((const void*)moe_pp_kernel<MODE>, hipFuncAttributeMaxDynamicSharedMemorySize,
                            moe_smem_bytes<PPM>()) != hipSuccess) {
      lsk::set_error("%s: cannot reserve %d bytes of LDS", name, moe_smem_bytes<PPM>());
      return LSK_ERR_HIP;
    }
    attr_set = true;
  }
  hipLaunchKernelGGL(moe_pp_kernel<MODE>, dim3((unsigned)blocks), dim3(512), moe_smem_bytes<PPM>(), s, ga);
  return lsk::check_launch(name);
}

// Compute units of the current device (the persistent grid), cached per device.
static int moe_cu_count() {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
  int n = cache[dev].load(std::memory_order_relaxed);
  if (n <= 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cache[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

// The 256 x 256 expert tiles: ga.tiles is the kBM2-row tile table, max_tiles its bound.  g_moe_w4
// == 3: the persistent kernel (one block per CU); 4: one tile per block.
template <int MODE>
int launch_moe_pp256(const MoeGemmArgs& ga, int64_t max_tiles, hipStream_t s, const char* name) {
  const int ntiles = MODE == 0 ? (ga.N + 127) / 128 : (ga.N + 255) / 256;
  const int64_t blocks = max_tiles * ntiles;
  if (blocks == 0) return LSK_OK;
  LSK_REQUIRE(blocks <= 0x7fffffff, "%s: grid too large", name);
  if (g_moe_w4 == 3 && ga.K >= (PPM256::kRing + 2) * PPM256::kBK) {  // the persistent loop's first steps
    static std::atomic<bool> attr_p{false};
    if (!attr_p) {
      if (hipFuncSetAttribute((const void*)moe_pp256p_kernel<MODE>, hipFuncAttributeMaxDynamicSharedMemorySize,
                              kP256pSmem) != hipSuccess) {
        lsk::set_error("%s: cannot reserve %d bytes of LDS", name, kP256pSmem);
        return LSK_ERR_HIP;
      }
      attr_p = true;
    }
    const int64_t grid = blocks < moe_cu_count() ? blocks : moe_cu_count();
    hipLaunchKernelGGL(moe_pp256p_kernel<MODE>, dim3((unsigned)grid), dim3(512), kP256pSmem, s, ga);
    return lsk::check_launch(name);
  }
  constexpr int kSmem = moe_smem_bytes<PPM256>();
  static std::atomic<bool> attr_set{false};
  if (!attr_set) {
    if (hipFuncSetAttribute((const void*)moe_pp256_kernel<MODE>, hipFuncAttributeMaxDynamicSharedMemorySize, kSmem) !=
        hipSuccess) {
      lsk::set_error("%s: cannot reserve %d bytes of LDS", name, kSmem);
      return LSK_ERR_HIP;
    }
    attr_set = true;
  }
  hipLaunchKernelGGL(moe_pp256_kernel<MODE>, dim3((unsigned)blocks), dim3(512), kSmem, s, ga);
  return lsk::check_launch(name);
}

// The grouped GEMV for decode token counts: MR = rows multiplied at once (a power of two >= the
// token count, at most 8; 4 when K needs four 1 KB sweeps), RPW columns per wave.
template <int MODE, int MR, int NC>
int launch_moe_gemv_k(const MoeGemmArgs& ga, int64_t max_tiles, uint16_t* gu, hipStream_t s, const char* name) {
  constexpr int RPW = MODE == 0 ? 2 : 4;
  const int nchunk = (ga.N + 4 * RPW - 1) / (4 * RPW);
  const int64_t blocks = max_tiles * nchunk;
  if (blocks == 0) return LSK_OK;
  LSK_REQUIRE(blocks <= 0x7fffffff, "%s: grid too large", name);
  hipLaunchKernelGGL((moe_gemv_kernel<MODE, MR, NC, RPW>), dim3((unsigned)blocks), dim3(256), 0, s, ga, gu);
  return lsk::check_launch(name);
}

template <int MODE, int MR>
int launch_moe_gemv_mr(const MoeGemmArgs& ga, int64_t max_tiles, uint16_t* gu, hipStream_t s, const char* name) {
  const int nc = (ga.K + 1023) / 1024;
  if (nc <= 1) return launch_moe_gemv_k<MODE, MR, 1>(ga, max_tiles, gu, s, name);
  if (nc <= 2) return launch_moe_gemv_k<MODE, MR, 2>(ga, max_tiles, gu, s, name);
  return launch_moe_gemv_k<MODE, (MR > 4 ? 4 : MR), 4>(ga, max_tiles, gu, s, name);
}

template <int MODE>
int launch_moe_gemv(const MoeGemmArgs& ga, int64_t max_tiles, int64_t T, uint16_t* gu, hipStream_t s,
                    const char* name) {
  if (T <= 1) return launch_moe_gemv_mr<MODE, 1>(ga, max_tiles, gu, s, name);
  if (T <= 2) return launch_moe_gemv_mr<MODE, 2>(ga, max_tiles, gu, s, name);
  if (T <= 4) return launch_moe_gemv_mr<MODE, 4>(ga, max_tiles, gu, s, name);
  return launch_moe_gemv_mr<MODE, 8>(ga, max_tiles, gu, s, name);
}

// moe_skinny_kernel's launch: chunks of 16 rows up to 16 tokens (no expert gets more rows than
// there are tokens), else 32; up to 64 tokens eight groups of 16 weight rows per block, one wave
// per group over the whole K, above that four groups of two waves.  (Qwen3-30B-A3B int8 layer on
// MI355X, graph replays, us at T = 8 / 32 / 64 for gpb x kw reading the row-pair copies: 8 x 1
// 51.3 / 65.0 / 85.4, 16 x 1 50.2 / 69.2 / 94.5, 4 x 2 50.6 / 67.2 / 87.3, 8 x 2 56.9 / 71.1 /
// 96.3, 4 x 4 64.2 / 90.0 / 112.6; at T = 96 / 128 / 192: 8 x 1 124.5 / 148.5 / 157.0, 4 x 2
// 113.3 / 142.8 / 149.5; row-major weights 8-15% slower.)  A (a chunk's rows) and the reduction
// share the LDS, the rows' operands follow.
template <int MODE>
int launch_moe_skinny(const MoeGemmArgs& ga, int64_t max_tiles, int64_t T, uint16_t* gu, hipStream_t s,
                      const char* name) {
  const int K = ga.K, steps = (K + 63) / 64;
  const int MT = T <= 16 ? 1 : 2, CR = 16 * MT;
  const int ldsk = (K + 1023) / 1024 * 1024 + 16;
  const int NWR = MODE == 0 ? 2 * ga.N : ga.N;
  const int G = (NWR + 15) / 16;
  int kw = T > 64 ? 2 : 1, gpb = T > 64 ? 4 : 8;
  if (g_msk_kw > 0) kw = g_msk_kw;
  if (g_msk_gpb > 0) gpb = g_msk_gpb;
  LSK_REQUIRE(gpb * kw <= 16, "%s: %d x %d waves", name, gpb, kw);
  const int nw = gpb * kw;
  const int sets = (G + gpb - 1) / gpb;
  const size_t smem = (size_t)std::max(CR * ldsk, nw * MT * 1024) + (size_t)CR * 16;
  LSK_REQUIRE(smem <= 160 * 1024, "%s: K=%d too long for the skinny grouped GEMM", name, K);
  const int64_t blocks = max_tiles * sets;
  if (blocks == 0) return LSK_OK;
  LSK_REQUIRE(blocks <= 0x7fffffff, "%s: grid too large", name);
  const bool pairs = (ga.pairs & 2) != 0;
#define LSK_MSK(MTV, PV)                                                                                        \
  {                                                                                                             \
    auto kern = moe_skinny_kernel<MODE, MTV, 8, PV>;                                                            \
    if (smem > 65536 &&                                                                                         \
        hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024) != hipSuccess) \
      return lsk::set_error("%s: cannot reserve LDS", name), LSK_ERR_HIP;                                      \
    hipLaunchKernelGGL(kern, dim3((unsigned)blocks), dim3(64 * nw), smem, s, ga, gu, gpb, kw, sets, ldsk);      \
    return lsk::check_launch(name);                                                                            \
  }
  if (MT == 1) {
    if (pairs) LSK_MSK(1, true) else LSK_MSK(1, false)
  } else {
    if (pairs) LSK_MSK(2, true) else LSK_MSK(2, false)
  }
#undef LSK_MSK
}

template <int MODE>
int launch_moe_gemm(const MoeGemmArgs& ga, int64_t max_tiles, int ntiles, hipStream_t s, const char* name) {
  using C = lsk::TileCfg<128, 128, 2, 2>;
  const int64_t blocks = max_tiles * ntiles;
  if (blocks == 0) return LSK_OK;
  LSK_REQUIRE(blocks <= 0x7fffffff, "%s: grid too large", name);
  hipLaunchKernelGGL(moe_gemm_kernel<MODE>, dim3((unsigned)blocks), dim3(256), C::kSmemBytes, s, ga);
  return lsk::check_launch(name);
}

}  // namespace

extern "C" int lsk_router_topk(const void* g, int g_dtype, int64_t ldg, int64_t T, int64_t E, int k, int renormalize,
                               const int32_t* tab, int64_t* idx, uint16_t* w_bf16, void* stream) {
  LSK_REQUIRE(T >= 0 && E >= 1 && E <= 1024, "lsk_router_topk: E=%lld not in [1, 1024]", (long long)E);
  LSK_REQUIRE(k >= 1 && k <= 32 && k <= E, "lsk_router_topk: k=%d not in [1, min(E, 32)]", k);
  LSK_REQUIRE(g_dtype == LSK_F32 || g_dtype == LSK_BF16, "lsk_router_topk: g_dtype must be f32 or bf16");
  LSK_REQUIRE(ldg >= E, "lsk_router_topk: ldg below E");
  if (T == 0) return LSK_OK;
  LSK_REQUIRE(g && tab && idx && w_bf16, "lsk_router_topk: null pointer");
  LSK_REQUIRE(T <= 0x7fffffffLL * 4, "lsk_router_topk: T too large");
  const dim3 grid((unsigned)((T + 3) / 4)), blk(256);
  hipStream_t s = (hipStream_t)stream;
  if (E <= 64) hipLaunchKernelGGL(router_topk_kernel<1>, grid, blk, 0, s, g, g_dtype, ldg, (int)T, (int)E, k,
                                  renormalize, tab, idx, w_bf16);
  else if (E <= 128) hipLaunchKernelGGL(router_topk_kernel<2>, grid, blk, 0, s, g, g_dtype, ldg, (int)T, (int)E, k,
                                        renormalize, tab, idx, w_bf16);
  else if (E <= 256) hipLaunchKernelGGL(router_topk_kernel<4>, grid, blk, 0, s, g, g_dtype, ldg, (int)T, (int)E, k,
                                        renormalize, tab, idx, w_bf16);
  else hipLaunchKernelGGL(router_topk_kernel<16>, grid, blk, 0, s, g, g_dtype, ldg, (int)T, (int)E, k, renormalize,
                          tab, idx, w_bf16);
  return lsk::check_launch("router_topk_kernel");
}

// ---------------------------------------------------------------- the grouped expert linear alone
// Tile table of expert-sorted rows from the caller's offsets (one block).  The offsets are first
// made monotone and clamped to [0, R] (coffs[j] = min(R, max(0, offs[0..j]))), so offsets that
// decrease or run past R give empty or shortened experts, never rows outside [0, R) nor more tiles
// than grouped_max_tiles(R, E); the tiles read coffs.  tiles[0] = number of bm-row tiles (bm = kBM
// or kBM2), then (expert, first row) per tile, experts ascending.
__global__ __launch_bounds__(256) void grouped_tiles_kernel(const int32_t* __restrict__ offs, int E, int R, int bm,
                                                            int32_t* __restrict__ tiles, int32_t* __restrict__ coffs) {
  __shared__ int tmp[4];
  __shared__ int run_max[256];
  __shared__ int co[1025];
  const int per = (E + 1 + 255) / 256;  // offsets 0..E, a contiguous run per thread
  const int j0 = threadIdx.x * per;
  int m = 0;
  for (int j = j0; j < j0 + per && j <= E; ++j) m = max(m, min(max(offs[j], 0), R));
  run_max[threadIdx.x] = m;
  __syncthreads();
  int run = 0;
  for (int t = 0; t < (int)threadIdx.x; ++t) run = max(run, run_max[t]);
  for (int j = j0; j < j0 + per && j <= E; ++j) {
    run = max(run, min(max(offs[j], 0), R));
    co[j] = run;
    coffs[j] = run;
  }
  __syncthreads();
  const int pe = (E + 255) / 256;
  const int e0 = threadIdx.x * pe;
  int ntl = 0;
  for (int e = e0; e < e0 + pe && e < E; ++e) ntl += (co[e + 1] - co[e] + bm - 1) / bm;
  int total;
  int tbase = block_excl_scan<256>(ntl, tmp, total);
  for (int e = e0; e < e0 + pe && e < E; ++e)
    for (int r0 = co[e]; r0 < co[e + 1]; r0 += bm, ++tbase) {
      tiles[1 + 2 * tbase] = e;
      tiles[2 + 2 * tbase] = r0;
    }
  if (threadIdx.x == 0) tiles[0] = total;
}

static int64_t grouped_max_tiles(int64_t R, int64_t E) { return R / kBM + (E < R ? E : R); }

static int64_t grouped_tiles_bytes(int64_t R, int64_t E) { return up256((1 + 2 * grouped_max_tiles(R, E)) * 4); }

extern "C" int64_t lsk_grouped_gemm_workspace(int64_t R, int64_t E) {
  return grouped_tiles_bytes(R, E) + up256((E + 1) * 4);
}

// The clamped offsets grouped_tiles_kernel leaves in the workspace, which the tiles read.
static const int32_t* grouped_offs(void* workspace, int64_t R, int64_t E) {
  return (const int32_t*)((char*)workspace + grouped_tiles_bytes(R, E));
}

// Shared checks and the tile table of the two grouped entry points.
static int grouped_setup(const char* who, const void* a, const float* asc, const int32_t* offs, int64_t E, int64_t R,
                         const int64_t* w_ptrs, const int64_t* ws_ptrs, int64_t N, int64_t K, const void* out,
                         void* workspace, int64_t workspace_bytes, hipStream_t s, int bm = kBM) {
  LSK_REQUIRE(R >= 0 && N > 0 && K > 0 && E >= 1 && E <= 1024, "%s: bad sizes R=%lld N=%lld K=%lld E=%lld", who,
              (long long)R, (long long)N, (long long)K, (long long)E);
  LSK_REQUIRE(K <= 133144, "%s: K above the int32-exact bound", who);
  LSK_REQUIRE(R <= 0x7fffffff && N <= 0x7fffffff, "%s: sizes beyond 31 bits", who);
  if (R == 0) return LSK_OK;
  LSK_REQUIRE(a && asc && offs && w_ptrs && ws_ptrs && out, "%s: null pointer", who);
  LSK_REQUIRE(workspace && workspace_bytes >= lsk_grouped_gemm_workspace(R, E) && ((uintptr_t)workspace & 255) == 0,
              "%s: workspace of %lld bytes (256-byte aligned) needed", who, (long long)lsk_grouped_gemm_workspace(R, E));
  hipLaunchKernelGGL(grouped_tiles_kernel, dim3(1), dim3(256), 0, s, offs, (int)E, (int)R, bm, (int32_t*)workspace,
                     (int32_t*)grouped_offs(workspace, R, E));
  return lsk::check_launch("grouped_tiles_kernel");
}

extern "C" int lsk_grouped_gemm_w8a8_pairs(const int8_t* a, int64_t lda, const float* asc, const int32_t* offs,
                                           int64_t E, int64_t R, const int64_t* w_ptrs, int64_t ldw,
                                           const int64_t* w_pair_ptrs, const int64_t* ws_ptrs, const int64_t* b_ptrs,
                                           int64_t N, int64_t K, uint16_t* out, void* workspace,
                                           int64_t workspace_bytes, void* stream);

extern "C" int lsk_grouped_gemm_w8a8(const int8_t* a, int64_t lda, const float* asc, const int32_t* offs, int64_t E,
                                     int64_t R, const int64_t* w_ptrs, int64_t ldw, const int64_t* ws_ptrs,
                                     const int64_t* b_ptrs, int64_t N, int64_t K, uint16_t* out, void* workspace,
                                     int64_t workspace_bytes, void* stream) {
  return lsk_grouped_gemm_w8a8_pairs(a, lda, asc, offs, E, R, w_ptrs, ldw, nullptr, ws_ptrs, b_ptrs, N, K, out,
                                     workspace, workspace_bytes, stream);
}

extern "C" int lsk_grouped_gemm_w8a8_pairs(const int8_t* a, int64_t lda, const float* asc, const int32_t* offs,
                                           int64_t E, int64_t R, const int64_t* w_ptrs, int64_t ldw,
                                           const int64_t* w_pair_ptrs, const int64_t* ws_ptrs, const int64_t* b_ptrs,
                                           int64_t N, int64_t K, uint16_t* out, void* workspace,
                                           int64_t workspace_bytes, void* stream) {
  hipStream_t s = (hipStream_t)stream;
  // the ping-pong tiles once experts average 16 rows (the 256 x 256 ones when chosen); the
  // register-staged tile (lsk_moe_select(0)) or the skinny grouped GEMM (7) when chosen
  const bool pp = g_moe_force != 0 && g_moe_force != 7 && (g_moe_force == 1 || g_moe_force == 3 || R >= 16 * E);
  const bool pp256 = pp && moe_uses_pp256(R, E);
  int rc = grouped_setup("lsk_grouped_gemm_w8a8", a, asc, offs, E, R, w_ptrs, ws_ptrs, N, K, out, workspace,
                         workspace_bytes, s, pp256 ? kBM2 : kBM);
  if (rc || R == 0) return rc;
  LSK_REQUIRE(lda >= K && lda % 16 == 0 && ldw >= K && ldw % 16 == 0 && N * ldw < 0x7fffffff &&
                  R * lda < 0x7fffffff,
              "lsk_grouped_gemm_w8a8: row strides must cover K and be multiples of 16 (31-bit buffer offsets)");
  MoeGemmArgs g{};
  g.skinny_rows = g_pp_skinny;
  g.A = a;
  g.lda = lda;
  g.a_bytes = R * lda;
  g.w_bytes = N * ldw;
  g.a_scale = asc;
  g.offs = grouped_offs(workspace, R, E);
  g.tiles = (const int32_t*)workspace;
  g.w_ptrs = w_ptrs;
  g.ldw = ldw;
  g.ws_ptrs = ws_ptrs;
  g.b_ptrs = b_ptrs;
  g.K = (int)K;
  g.N = (int)N;
  g.y = out;  // row_w / row_dst null: weight 1, row p of the output
  const int64_t mt = grouped_max_tiles(R, E);
  if (pp) {
    if (w_pair_ptrs && (g_moe_w4 == 0 || g_moe_w4 == 3 || g_moe_w4 == 4)) {  // the row-pair copies, ping-pong tiles
      g.w_ptrs = w_pair_ptrs;
      g.ldw = (K + 63) / 64 * 64;
      g.w_bytes = ((N + 1) & ~(int64_t)1) * g.ldw;
      g.pairs = 2;
    }
    if (pp256) return launch_moe_pp256<1>(g, R / kBM2 + (E < R ? E : R), s, "moe_pp256_kernel<grouped>");
    return launch_moe_pp<1>(g, mt, s, "moe_pp_kernel<grouped>");
  }
  // few rows per expert: the skinny grouped GEMM (chunks of 32 of an expert's rows in LDS) while
  // they fit, the register-staged tile otherwise or when chosen
  if (K <= 4096 && g_moe_force != 0) {
    if (w_pair_ptrs) {
      g.w_ptrs = w_pair_ptrs;
      g.ldw = (K + 63) / 64 * 64;
      g.w_bytes = ((N + 1) & ~(int64_t)1) * g.ldw;
      g.pairs = 2;
    }
    // (the launch shape by rows per expert: twice the average, the skew a Zipf routing leaves)
    const int64_t rpe = std::min<int64_t>(kSkinnyMaxT, std::max<int64_t>(1, 2 * ((R + E - 1) / E)));
    return launch_moe_skinny<1>(g, mt, rpe, nullptr, s, "moe_skinny_kernel<grouped>");
  }
  return launch_moe_gemm<1>(g, mt, (int)((N + 127) / 128), s, "moe_gemm_kernel<grouped>");
}

// Whether the grouped MX linear takes the skinny grouped MX GEMM when the caller passes the weights'
// skinny-layout copies: experts averaging at most 32 rows (R <= 32 E) under lsk_moe_mx_select(0),
// any row count under (3); its LDS within 160 KB.  (The layer's measurements: GPT-OSS-20B shapes on
// MI355X, 32 rows per expert 118.7 against 137.6 us on the tiles, 64 level, 181.9 / 183.5.)
static bool grouped_mx_takes_skinny(int64_t R, int64_t E, int64_t K, int64_t lds) {
  if (R < 1 || E < 1 || K <= 0 || K % 32 != 0 || lds < K / 32 || lsk::moe_mx_skinny_lds(K, lds) > 160 * 1024)
    return false;
  const int v = lsk::mx_variant();
  return v == 3 || (v == 0 && R <= 32 * E);
}

static int grouped_mx(const uint16_t* a, int64_t lda, const float* asc, const int32_t* offs, int64_t E, int64_t R,
                      const int64_t* w_ptrs, int64_t ldw, const int64_t* w_skinny_ptrs, const int64_t* kx_ptrs,
                      int64_t lds, const int64_t* b_ptrs, int64_t N, int64_t K, int safe, uint16_t* out,
                      void* workspace, int64_t workspace_bytes, hipStream_t s) {
  int rc = grouped_setup("lsk_grouped_gemm_mx", a, asc, offs, E, R, w_ptrs, kx_ptrs, N, K, out, workspace,
                         workspace_bytes, s);
  if (rc || R == 0) return rc;
  LSK_REQUIRE(K % 32 == 0 && lda >= K && lda % 8 == 0 && ldw >= K / 2 && ldw % 16 == 0 && lds >= K / 32 &&
                  N * ldw < 0x7fffffff && R * lda * 2 < 0x7fffffff,
              "lsk_grouped_gemm_mx: K %% 32 == 0; row strides must cover K (bf16 rows, multiples of 8), K/2 (code "
              "bytes, multiples of 16) and K/32 (31-bit buffer offsets)");
  MoeGemmArgs g{};
  g.skinny_rows = g_pp_skinny;
  g.A = a;
  g.lda = lda;
  g.a_bytes = R * lda * 2;
  g.w_bytes = N * ldw;
  g.a_scale = asc;
  g.offs = grouped_offs(workspace, R, E);
  g.tiles = (const int32_t*)workspace;
  g.w_ptrs = w_ptrs;
  g.ldw = ldw;
  g.ws_ptrs = kx_ptrs;
  g.lds = lds;
  g.b_ptrs = b_ptrs;
  g.K = (int)K;
  g.N = (int)N;
  g.y = out;
  if (w_skinny_ptrs && grouped_mx_takes_skinny(R, E, K, lds)) {
    LSK_REQUIRE(lsk::mx_skinny_bytes(N, K) < 0x7fffffff, "lsk_grouped_gemm_mx_skinny: a copy beyond 2 GB");
    g.w_ptrs = w_skinny_ptrs;
    g.w_bytes = lsk::mx_skinny_bytes(N, K);
    // no routing weights or slot rows: row p of out, bfr(fl32(acc * asc[p])) (+ b) as the tiles write it
    return lsk::launch_moe_mx_skinny(1, g, grouped_max_tiles(R, E), R, safe, nullptr, s);
  }
  return lsk::launch_moe_mx_gemm(1, g, grouped_max_tiles(R, E), safe, s);
}

extern "C" int lsk_grouped_gemm_mx(const uint16_t* a, int64_t lda, const float* asc, const int32_t* offs, int64_t E,
                                   int64_t R, const int64_t* w_ptrs, int64_t ldw, const int64_t* kx_ptrs, int64_t lds,
                                   const int64_t* b_ptrs, int64_t N, int64_t K, int safe, uint16_t* out,
                                   void* workspace, int64_t workspace_bytes, void* stream) {
  return grouped_mx(a, lda, asc, offs, E, R, w_ptrs, ldw, nullptr, kx_ptrs, lds, b_ptrs, N, K, safe, out, workspace,
                    workspace_bytes, (hipStream_t)stream);
}

extern "C" int lsk_grouped_gemm_mx_skinny(const uint16_t* a, int64_t lda, const float* asc, const int32_t* offs,
                                          int64_t E, int64_t R, const int64_t* w_ptrs, int64_t ldw,
                                          const int64_t* w_skinny_ptrs, const int64_t* kx_ptrs, int64_t lds,
                                          const int64_t* b_ptrs, int64_t N, int64_t K, int safe, uint16_t* out,
                                          void* workspace, int64_t workspace_bytes, void* stream) {
  return grouped_mx(a, lda, asc, offs, E, R, w_ptrs, ldw, w_skinny_ptrs, kx_ptrs, lds, b_ptrs, N, K, safe, out,
                    workspace, workspace_bytes, (hipStream_t)stream);
}

extern "C" int lsk_grouped_mx_reads_skinny(int64_t R, int64_t E, int64_t K, int64_t lds) {
  return grouped_mx_takes_skinny(R, E, K, lds) ? 1 : 0;
}

extern "C" int lsk_moe_fuse_route(int on) {
  LSK_REQUIRE(on == 0 || on == 1, "lsk_moe_fuse_route: %d not 0 or 1", on);
  g_rowq1 = on;
  return LSK_OK;
}

extern "C" int lsk_moe_pp_skinny_rows(int rows) {
  LSK_REQUIRE(rows >= 0 && rows <= 32, "lsk_moe_pp_skinny_rows: %d not in [0, 32]", rows);
  g_pp_skinny = rows;
  return LSK_OK;
}

extern "C" int lsk_moe_skinny_shape(int gpb, int kw) {
  LSK_REQUIRE(gpb >= 0 && kw >= 0 && gpb <= 16 && kw <= 16 && (gpb == 0 || kw == 0 || gpb * kw <= 16),
              "lsk_moe_skinny_shape: gpb=%d kw=%d (gpb * kw <= 16)", gpb, kw);
  g_msk_gpb = gpb;
  g_msk_kw = kw;
  return LSK_OK;
}

extern "C" int lsk_moe_select(int variant) {
  LSK_REQUIRE(variant >= -1 && variant <= 7, "lsk_moe_select: variant %d not in [-1, 7]", variant);
  g_moe_force = (variant >= 4 && variant <= 6) ? 1 : variant;
  g_moe_w4 = variant == 3 ? 1 : (variant == 4 ? 2 : (variant == 5 ? 3 : (variant == 6 ? 4 : 0)));
  return LSK_OK;
}

extern "C" int64_t lsk_moe_workspace(int64_t T, int k, int64_t E, int64_t H, int64_t I, int rot_blk, int wfmt) {
  return moe_layout(nullptr, T, k, E, H, I, rot_blk, wfmt).bytes;
}

static int moe_forward_call(const lsk_moe_args* a, void* stream);

// Whether an int8 layer of T tokens, top-k over E experts, runs its grouped GEMMs on the ping-pong
// tiles that read the experts' row-pair weight copies (w13_pair_ptrs / w2_pair_ptrs), under the
// calling thread's kernel selection: the rule moe_forward_call applies.
static bool moe_reads_pair_weights(int64_t T, int k, int64_t E, int64_t H, int64_t I, int rb) {
  const int64_t R = T * k;
  const bool use_pp = g_moe_force >= 0 ? (g_moe_force == 1 || g_moe_force == 3) : R >= 16 * E;
  const bool gemv_ok = rb == 0 && T <= kGemvMaxT && (g_moe_force >= 0 ? g_moe_force == 2 : true);
  const bool skinny = moe_takes_skinny(T, k, E, rb, 0, H, I);
  const bool use_gemv = gemv_ok && H <= 4096 && I <= 4096 && !skinny;
  return skinny || (use_pp && !use_gemv && (g_moe_w4 == 0 || g_moe_w4 == 3 || g_moe_w4 == 4));
}

extern "C" int lsk_moe_reads_row_pairs(int64_t T, int k, int64_t E, int64_t H, int64_t I, int rot_blk, int select) {
  if (T <= 0 || k < 1 || E < 1 || H <= 0 || I <= 0 || select < 0 || select > 9) return 0;
  const int force = g_moe_force, w4 = g_moe_w4;
  if (select) lsk_moe_select(select - 2);
  const bool r = moe_reads_pair_weights(T, k, E, H, I, rot_blk);
  g_moe_force = force;
  g_moe_w4 = w4;
  return r ? 1 : 0;
}

// Whether an MXFP4 layer (per-row activation scales) takes the skinny grouped MX GEMM when the caller
// has the skinny-layout code copies: by size from 2 tokens under lsk_moe_mx_select(0), and for one
// token when its gate/up launch has at least 320 four-wave blocks (k * 2I / 64; fewer leave CUs
// idle and the MX GEMV keeps the token); from 1 under (3); up to 256 tokens; its LDS (the chunk's
// bf16 rows and the E8M0 rows) within 160 KB; no rotation.  A forced GEMV (lsk_moe_select(2)) or
// forced tiles take none unless (3) asks for it.  GPT-OSS-20B on MI355X (E 32, top 4, H = I =
// 2880), us: T = 1 41.0 against 43.7 (GEMV), T = 2 47.7 / 64, T = 16 124 / 193, T = 32 129 / 262
// (tiles), T = 128 177 / 330, T = 256 267 / 390; at 64 rows per expert (E 8, top 2, T = 256) level
// with the tiles, 182 / 184; one token of E 8, top 2 35.4 against 34.4 on the GEMV.
static bool mx_takes_skinny(int64_t T, int k, int64_t E, int64_t H, int64_t I, int64_t lds13, int64_t lds2, int rb) {
  (void)E;
  if (rb != 0 || T < 1 || T > kSkinnyMaxT || H % 32 != 0 || I % 32 != 0) return false;
  if (lsk::moe_mx_skinny_lds(H, lds13) > 160 * 1024 || lsk::moe_mx_skinny_lds(I, lds2) > 160 * 1024) return false;
  const int v = lsk::mx_variant();
  if (g_moe_force == 2) return false;
  if (v == 3) return true;
  return v == 0 && g_moe_force < 0 && (T >= 2 || (int64_t)k * ((2 * I + 63) / 64) >= 320);
}

extern "C" int lsk_moe_mx_reads_skinny(int64_t T, int k, int64_t E, int64_t H, int64_t I, int64_t lds13, int64_t lds2,
                                       int select, int mx_select) {
  if (T <= 0 || k < 1 || E < 1 || H <= 0 || I <= 0 || select < 0 || select > 9 || mx_select < 0 || mx_select > 4)
    return 0;
  const int force = g_moe_force, w4 = g_moe_w4, mxv = lsk::mx_variant();
  if (select) lsk_moe_select(select - 2);
  if (mx_select) lsk_moe_mx_select(mx_select - 1);
  const bool r = mx_takes_skinny(T, k, E, H, I, lds13, lds2, 0);
  g_moe_force = force;
  g_moe_w4 = w4;
  lsk_moe_mx_select(mxv);
  return r ? 1 : 0;
}

extern "C" int lsk_moe_forward(const lsk_moe_args* a, void* stream) {
  LSK_REQUIRE(a, "lsk_moe_forward: null args");
  LSK_REQUIRE(a->select >= 0 && a->select <= 9 && a->mx_select >= 0 && a->mx_select <= 4,
              "lsk_moe_forward: select=%d / mx_select=%d outside [0, 9] / [0, 4]", a->select, a->mx_select);
  if (a->select == 0 && a->mx_select == 0) return moe_forward_call(a, stream);
  // this call's kernel choice, the thread's own restored afterwards
  const int force = g_moe_force, w4 = g_moe_w4, mxv = lsk::mx_variant();
  if (a->select) lsk_moe_select(a->select - 2);
  if (a->mx_select) lsk_moe_mx_select(a->mx_select - 1);
  const int rc = moe_forward_call(a, stream);
  g_moe_force = force;
  g_moe_w4 = w4;
  lsk_moe_mx_select(mxv);
  return rc;
}

static int moe_forward_call(const lsk_moe_args* a, void* stream) {
  const int64_t T = a->T, H = a->H, I = a->I, E = a->E;
  const int k = a->k;
  LSK_REQUIRE(T >= 0 && H > 0 && I > 0 && E >= 1 && E <= 1024, "lsk_moe_forward: bad sizes T=%lld H=%lld I=%lld E=%lld",
              (long long)T, (long long)H, (long long)I, (long long)E);
  LSK_REQUIRE(k >= 1 && k <= 32, "lsk_moe_forward: k=%d not in [1, 32]", k);
  LSK_REQUIRE(H % 16 == 0 && I % 16 == 0, "lsk_moe_forward: H and I must be multiples of 16");
  LSK_REQUIRE(H <= 133144 && I <= 133144, "lsk_moe_forward: K above the int32-exact bound");
  LSK_REQUIRE(a->act == LSK_ACT_SILU || a->act == LSK_ACT_SWIGLUOAI, "lsk_moe_forward: unknown act %d", a->act);
  LSK_REQUIRE(T * k <= 0x7fffffff && T * H * 2 < 0x7fffffff && T * k * I * 2 < 0x7fffffff,
              "lsk_moe_forward: activations beyond 2 GB (31-bit buffer offsets)");
  if (T == 0) return LSK_OK;
  LSK_REQUIRE(a->x && a->w13_ptrs && a->ws13_ptrs && a->w2_ptrs && a->ws2_ptrs && a->frac && a->y,
              "lsk_moe_forward: null pointer");
  // the routing: given (idx, w), or computed here from the logits into (idx_out, w_out)
  const int64_t* ridx = a->idx;
  const uint16_t* rwt = a->w;
  if (a->logits) {
    LSK_REQUIRE(a->idx_out && a->w_out && a->router_tab, "lsk_moe_forward: logits need idx_out, w_out and router_tab");
    LSK_REQUIRE(a->logits_dtype == LSK_F32 || a->logits_dtype == LSK_BF16, "lsk_moe_forward: logits must be f32 or bf16");
    LSK_REQUIRE(a->ld_logits >= E, "lsk_moe_forward: ld_logits below E");
    LSK_REQUIRE(k <= E, "lsk_moe_forward: k=%d above E=%lld", k, (long long)E);
    ridx = a->idx_out;
    rwt = a->w_out;
  } else {
    LSK_REQUIRE(a->idx && a->w, "lsk_moe_forward: null routing");
  }
  if (a->wfmt >= 1) {
    LSK_REQUIRE(a->ldw13 >= H / 2 && a->ldw13 % 16 == 0 && a->ldw2 >= I / 2 && a->ldw2 % 16 == 0 &&
                    a->lds13 >= H / 32 && a->lds2 >= I / 32,
                "lsk_moe_forward: MXFP4 row strides must cover K/2 (multiples of 16) and K/32");
  } else {
    LSK_REQUIRE(a->ldw13 >= H && a->ldw13 % 16 == 0 && a->ldw2 >= I && a->ldw2 % 16 == 0,
                "lsk_moe_forward: weight row strides must cover K and be multiples of 16");
    LSK_REQUIRE(2 * I * a->ldw13 < 0x7fffffff && H * a->ldw2 < 0x7fffffff,
                "lsk_moe_forward: an expert's weight beyond 2 GB (31-bit buffer offsets)");
  }
  const int rb = a->rot_blk;
  LSK_REQUIRE(rb == 0 || (rb >= 2 && rb <= 1024 && (rb & (rb - 1)) == 0 && H % rb == 0 && I % rb == 0 && I <= 16384),
              "lsk_moe_forward: rot_blk=%d must be 0 or a power of two dividing H and I (I <= 16384)", rb);
  const int mx = a->wfmt;
  LSK_REQUIRE(mx == 0 || mx == 1 || mx == 2, "lsk_moe_forward: unknown weight format %d", mx);
  LSK_REQUIRE(mx != 2 || (0 <= a->kw13_min && a->kw13_min <= a->kw13_max && a->kw13_max <= 255 && 0 <= a->kw2_min &&
                          a->kw2_min <= a->kw2_max && a->kw2_max <= 255),
              "lsk_moe_forward: E8M0 bounds must satisfy 0 <= min <= max <= 255");
  // block-scaled activations: the fused update on the dequantised values q * 2^ka is exact while
  // 2^ka stays in range for the MFMA block sums (ka <= 111) and every exponent ka + kexp - 128 of
  // a nonzero block lies in [-149, 111] (239 - kexp with the fused FMA, 255 - kexp with the
  // multiply-then-add update): no product underflows, overflows or rounds
  const int lo13 = -21 - a->kw13_min, lo2 = -21 - a->kw2_min;
  const int top = a->mx_safe ? 255 : 239;
  const int hi13 = std::min(111, top - a->kw13_max), hi2 = std::min(111, top - a->kw2_max);
  LSK_REQUIRE(!mx || (rb == 0 && H % 32 == 0 && I % 32 == 0), "lsk_moe_forward: MXFP4 experts need K %% 32 == 0 "
              "and no rotation");
  const MoeWs w = moe_layout((char*)a->workspace, T, k, E, H, I, rb, mx);
  LSK_REQUIRE(a->workspace && a->workspace_bytes >= w.bytes && ((uintptr_t)a->workspace & 255) == 0,
              "lsk_moe_forward: workspace of %lld bytes (256-byte aligned) needed", (long long)w.bytes);
  hipStream_t s = (hipStream_t)stream;
  const int64_t R = T * k;
  // the ping-pong grouped GEMM once experts average 16 routed rows (Qwen3-30B-A3B on MI355X: 256
  // tokens, 16 rows per expert, 187 us against 225 us on the 128x128 register-staged tile, level at
  // 2048 tokens); the register-staged tile below that
  const bool use_pp = g_moe_force >= 0 ? (g_moe_force == 1 || g_moe_force == 3) : R >= 16 * E;
  // decode token counts: the skinny grouped GEMM (activation rows in LDS, weight rows streamed into
  // the MFMA) from 2 tokens, the grouped GEMV (whole weight rows streamed once per tile, v_dot4)
  // for one token or when chosen
  const bool gemv_ok = rb == 0 && T <= kGemvMaxT && (g_moe_force >= 0 ? g_moe_force == 2 : true);
  const bool use_skinny = moe_takes_skinny(T, k, E, rb, mx, H, I);
  const bool use_gemv = gemv_ok && !mx && H <= 4096 && I <= 4096 && !use_skinny;
  // MXFP4 experts (per-row scales) past one token: the skinny grouped MX GEMM on the experts'
  // skinny-layout copies (w13_pair_ptrs / w2_pair_ptrs for MXFP4 experts), when the caller has them;
  // else the MX GEMV, which re-streams each expert's weights per 4-row pass, so past about 24 tokens
  // the tiled kernels win (GPT-OSS-20B on MI355X, T = 24 242 vs 276 us, T = 48 368 vs 278 us)
  const bool use_mx_skinny =
      mx == 1 && a->w13_pair_ptrs && a->w2_pair_ptrs && mx_takes_skinny(T, k, E, H, I, a->lds13, a->lds2, rb);
  const bool use_mx_gemv = gemv_ok && mx == 1 && !use_mx_skinny && (g_moe_force == 2 || T <= kMxGemvMaxT) &&
                           H <= 8192 && I <= 8192;
  // block-scaled activations at decode sizes: the same GEMV over integer-valued rows (every row
  // quantised in the general form) with the block exponents (T = 1 50 vs 116 us, T = 16 221 vs
  // 278 us, T = 24 281 vs 277 us)
  // and the skinny grouped MX GEMM where the MX layer would take it (the rows' dequantised bf16
  // values, no row scale; a flagged row sends the projection to the general tile kernel instead)
  const bool use_mx2_skinny =
      mx == 2 && a->w13_pair_ptrs && a->w2_pair_ptrs && mx_takes_skinny(T, k, E, H, I, a->lds13, a->lds2, rb);
  const bool use_mx2_gemv = gemv_ok && mx == 2 && !use_mx2_skinny && (g_moe_force == 2 || T <= kMx2GemvMaxT) &&
                            H <= 8192 && I <= 8192;
  // the down projection's quantised rows in the row-pair layout when the ping-pong tiles read them
  // (int8 experts, no rotation): its load instructions then read whole 128-byte lines
  const bool pair_down = use_pp && !mx && rb == 0 && !use_gemv && !use_skinny && I % 64 == 0 &&
                         (g_moe_w4 == 0 || g_moe_w4 == 3 || g_moe_w4 == 4);
  // the 256 x 256 expert tiles (their own tile table) for the ping-pong GEMMs
  const bool pp256 = use_pp && !mx && !use_gemv && !use_skinny && moe_uses_pp256(R, E);
  // the experts' row-pair weight copies on the same tiles, when the caller has them
  const bool pair_w = !mx && moe_reads_pair_weights(T, k, E, H, I, rb) && a->w13_pair_ptrs && a->w2_pair_ptrs;

  // up to 256 tokens: the dispatch and the row quant of x in one launch
  const bool prep_decode = T <= 256 && rb == 0 && mx != 2;
  // routing from logits: inside that launch for up to 4 tokens (a wave per token in its
  // dispatch block; with more, the waves' serial tokens cost more than the router launch they
  // save: Qwen3-30B-A3B on MI355X, T = 1 32.0 -> 31.4 us, T = 8 59.0 -> 63.4 us), else the
  // router kernel first
  const bool route_in_prep = a->logits && prep_decode && T <= 4 && E <= 256;
  // one token routed from its logits on the int8 GEMV path: the router, the row quant of x and the
  // gate/up GEMV in one launch (moe_route_gemv1_kernel; no prep launch)
  const bool route_gemv1 = route_in_prep && T == 1 && use_gemv && !mx && k <= 8 && H % 16 == 0 && H <= 4096 &&
                           I <= 2048 && ((uintptr_t)a->x & 15) == 0 && g_rowq1;
  // one MXFP4 token routed from its logits on the skinny path: the router and the row quant of x
  // inside the gate/up launch (no prep launch)
  const bool route_skinny1 = route_in_prep && T == 1 && use_mx_skinny && k <= 8 && H <= 8192 &&
                             ((uintptr_t)a->x & 15) == 0 && g_rowq1;
  // above 256 tokens (int8 experts, no rotation): the router and the row quant of x in one launch
  const bool route_rowq = a->logits && !route_in_prep && !prep_decode && rb == 0 && !mx && H % 8 == 0 &&
                          H <= 4096 && E <= 256 && ((uintptr_t)a->x & 15) == 0 && g_rowq1;
  int rc;
  if (route_rowq) {
    const dim3 grid((unsigned)((T + 3) / 4)), blk(256);
#define LSK_RRQ(EPLV, NXCV)                                                                                  \
  hipLaunchKernelGGL((moe_route_rowq_kernel<EPLV, NXCV>), grid, blk, 0, s, a->logits, a->logits_dtype,       \
                     a->ld_logits, (int)T, (int)E, k, a->renormalize, a->router_tab, a->idx_out, a->w_out, a->x, \
                     (int)H, w.qx, w.ascx)
#define LSK_RRQ_E(NXCV) \
  if (E <= 64) LSK_RRQ(1, NXCV); else if (E <= 128) LSK_RRQ(2, NXCV); else LSK_RRQ(4, NXCV);
    if (H <= 512) LSK_RRQ_E(1) else if (H <= 1024) LSK_RRQ_E(2) else if (H <= 2048) LSK_RRQ_E(4) else LSK_RRQ_E(8)
#undef LSK_RRQ_E
#undef LSK_RRQ
    if ((rc = lsk::check_launch("moe_route_rowq_kernel"))) return rc;
  } else if (a->logits && !route_in_prep) {
    const int rrc = lsk_router_topk(a->logits, a->logits_dtype, a->ld_logits, T, E, k, a->renormalize, a->router_tab,
                                    a->idx_out, a->w_out, stream);
    if (rrc) return rrc;
  }
  if (route_rowq) {
    rc = LSK_OK;  // x quantised above
  } else if (prep_decode) {
    rc = LSK_OK;  // the prep kernel below quantises x
  } else if (rb > 0) {
    // xrot = fwht_blocks(fl32(x)): widen, then butterfly in place
    int64_t blocks = (T * H + 255) / 256;
    blocks = blocks > 8192 ? 8192 : blocks;
    hipLaunchKernelGGL(widen_bf16_kernel, dim3((unsigned)blocks), dim3(256), 0, s, a->x, T * H, w.xrot);
    if ((rc = lsk::check_launch("widen_bf16_kernel"))) return rc;
    if ((rc = lsk_fwht_blocks(w.xrot, T, H, H, rb, a->rot_scale, w.xrot, H, stream))) return rc;
    rc = lsk_rowquant(w.xrot, LSK_F32, T, H, H, w.qx, H, w.ascx, stream);
  } else if (mx == 2) {
    rc = LSK_OK;  // after the dispatch, which clears the flag words it raises
  } else if (mx) {
    rc = lsk::launch_rowquant_bf16(a->x, T, H, (uint16_t*)w.qx, w.ascx, s);
  } else {
    rc = lsk_rowquant(a->x, LSK_BF16, T, H, H, w.qx, H, w.ascx, stream);
  }
  if (rc) return rc;
  // dispatch (and the zeroing of the per-row |h| maxima, which the gate/up GEMM raises); the
  // routes of a 256-token chunk are staged in LDS (up to 92 KB at E = 1024, k = 32)
  static std::atomic<bool> dispatch_lds{false};
  if (!dispatch_lds) {
    for (const void* f : {(const void*)moe_dispatch_small_kernel, (const void*)moe_count_kernel,
                          (const void*)moe_place_kernel, (const void*)moe_decode_prep_kernel})
      if (hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, 96 * 1024) != hipSuccess) {
        lsk::set_error("lsk_moe_forward: cannot reserve LDS for the dispatch");
        return LSK_ERR_HIP;
      }
    dispatch_lds = true;
  }
  // the dispatch also clears the per-row |h| maxima and, for block-scaled activations, the words
  // anyf[0] / anyf[1] that the block quants of x / h raise when they flag a row
  const int64_t nzero = mx == 2 ? R + 2 : R;
  int32_t* anyf = (int32_t*)(w.h_amax + R);
  const int64_t nchunks = (T + 255) / 256;
  if (route_gemv1 || route_skinny1) {
    // (the dispatch is written by the first launch below)
  } else if (prep_decode) {
    const size_t dsm = (size_t)(10 * E + 1) * 4 + (size_t)256 * k * 6;
    hipLaunchKernelGGL(moe_decode_prep_kernel, dim3((unsigned)(T + 1)), dim3(256), dsm, s, ridx, rwt, (int)T, k,
                       (int)E, w.offs, w.tiles, w.row_tok, w.row_dst, w.row_w, w.tok_cnt, w.h_amax, nzero,
                       a->x, (int)H, (void*)w.qx, w.ascx, mx ? 1 : 0, route_in_prep ? a->logits : nullptr,
                       a->logits_dtype, a->ld_logits, a->router_tab, a->renormalize, a->idx_out, a->w_out, w.tiles2);
    if ((rc = lsk::check_launch("moe_decode_prep_kernel"))) return rc;
  } else if (nchunks == 1) {
    const size_t dsm = (size_t)(10 * E + 1) * 4 + (size_t)256 * k * 6;
    hipLaunchKernelGGL(moe_dispatch_small_kernel, dim3(1), dim3(256), dsm, s, ridx, rwt, (int)T, k, (int)E, w.offs,
                       w.tiles, w.row_tok, w.row_dst, w.row_w, w.tok_cnt, w.h_amax, nzero, w.tiles2);
    if ((rc = lsk::check_launch("moe_dispatch_small_kernel"))) return rc;
  } else {
    hipLaunchKernelGGL(moe_count_kernel, dim3((unsigned)nchunks), dim3(256), (size_t)E * 4 + (size_t)256 * k * 4, s,
                       ridx, (int)T, k,
                       (int)E, w.ccnt, w.tok_cnt, w.h_amax, nzero);
    if ((rc = lsk::check_launch("moe_count_kernel"))) return rc;
    hipLaunchKernelGGL(moe_place_kernel, dim3((unsigned)(4 * nchunks)), dim3(256),
                       (size_t)(11 * E + 1) * 4 + (size_t)256 * k * 6, s, ridx, rwt, (int)T, k, (int)E, w.ccnt,
                       (int)nchunks, w.offs, w.tiles, w.row_tok, w.row_dst, w.row_w, w.tiles2);
    if ((rc = lsk::check_launch("moe_place_kernel"))) return rc;
  }
  if (mx == 2 &&
      (rc = lsk::launch_blockquant_mx2(a->x, H, T, nullptr, (int)H, (uint16_t*)w.qx, w.kax, w.flagx, anyf,
                                       use_mx2_gemv ? 1 : lo13, use_mx2_gemv ? 0 : hi13, s)))
    return rc;
  MoeGemmArgs g1{};
  g1.skinny_rows = g_pp_skinny;
  g1.A = w.qx;
  g1.lda = H;
  g1.a_bytes = T * H * (mx ? 2 : 1);
  g1.w_bytes = 2 * I * a->ldw13;
  g1.a_scale = w.ascx;
  g1.row_tok = w.row_tok;
  g1.offs = w.offs;
  g1.tiles = w.tiles;
  g1.w_ptrs = a->w13_ptrs;
  g1.ldw = a->ldw13;
  g1.ws_ptrs = a->ws13_ptrs;
  g1.b_ptrs = a->b13_ptrs;
  g1.K = (int)H;
  g1.N = (int)I;
  g1.act = a->act;
  g1.frac = a->frac;
  g1.act_tab = a->act_tab;
  g1.h = w.h;
  g1.h_amax = w.h_amax;
  g1.lds = a->lds13;
  if (mx == 2) {
    g1.a_scale = nullptr;
    g1.row_flag = w.flagx;
    g1.any_flag = anyf;
    g1.a_ka = w.kax;
    g1.ldka = H / 32;
  }
  if (use_mx_gemv || use_mx2_gemv) {
    if ((rc = lsk::launch_moe_mx_gemv(0, g1, w.max_tiles, T, a->mx_safe, use_mx2_gemv ? nullptr : w.gu, s))) return rc;
  } else if (use_mx2_skinny) {
    // the skinny GEMM when no row of x is flagged (gate / up values into gu), else the general tile
    // kernel over every tile (h itself)
    MoeGemmArgs gs = g1;
    gs.w_ptrs = a->w13_pair_ptrs;
    gs.w_bytes = lsk::mx_skinny_bytes(2 * I, H);
    gs.mx2 = 1;
    if ((rc = lsk::launch_moe_mx_skinny(0, gs, w.max_tiles, T, a->mx_safe, w.gu, s))) return rc;
    g1.mx2 = 3;
    if ((rc = lsk::launch_moe_mx_gemm(0, g1, w.max_tiles, a->mx_safe, s))) return rc;
  } else if (mx == 2) {
    g1.mx2 = 1;
    if ((rc = lsk::launch_moe_mx_gemm(0, g1, w.max_tiles, a->mx_safe, s))) return rc;
    g1.mx2 = 2;
    if ((rc = lsk::launch_moe_mx_gemm(0, g1, w.max_tiles, a->mx_safe, s))) return rc;
  } else if (use_mx_skinny) {
    g1.w_ptrs = a->w13_pair_ptrs;
    g1.w_bytes = lsk::mx_skinny_bytes(2 * I, H);
    if (route_skinny1) {
      lsk::MxRouteArgs ra{};
      ra.g = a->logits;
      ra.gdt = a->logits_dtype;
      ra.ldg = a->ld_logits;
      ra.E = (int)E;
      ra.k = k;
      ra.renorm = a->renormalize;
      ra.rtab = a->router_tab;
      ra.x = a->x;
      ra.idx_out = a->idx_out;
      ra.w_out = a->w_out;
      ra.offs = w.offs;
      ra.tiles = w.tiles;
      ra.row_tok = w.row_tok;
      ra.row_dst = w.row_dst;
      ra.tok_cnt = w.tok_cnt;
      ra.row_w = w.row_w;
      ra.ascx = w.ascx;
      if ((rc = lsk::launch_moe_mx_route_skinny1(g1, ra, a->mx_safe, w.gu, s))) return rc;
    } else if ((rc = lsk::launch_moe_mx_skinny(0, g1, w.max_tiles, T, a->mx_safe, w.gu, s))) {
      return rc;
    }
  } else if (mx) {
    if ((rc = lsk::launch_moe_mx_gemm(0, g1, w.max_tiles, a->mx_safe, s))) return rc;
  } else if (route_gemv1) {
    const int nchunk = (int)((I + 7) / 8);  // 4 waves x 2 columns per block
    const dim3 grid((unsigned)(k * nchunk));
#define LSK_RG1(NCV, EPLV)                                                                                     \
  hipLaunchKernelGGL((moe_route_gemv1_kernel<NCV, 2, EPLV>), grid, dim3(256), 0, s, g1, w.gu, a->x, a->logits, \
                     a->logits_dtype, (int)E, k, a->renormalize, a->router_tab, a->idx_out, a->w_out, w.offs,    \
                     w.tiles, w.row_tok, w.row_dst, w.row_w, w.tok_cnt, w.ascx)
    const int nc = (int)((H + 1023) / 1024);
    if (E <= 128) {
      if (nc <= 1) LSK_RG1(1, 2); else if (nc <= 2) LSK_RG1(2, 2); else LSK_RG1(4, 2);
    } else {
      if (nc <= 1) LSK_RG1(1, 4); else if (nc <= 2) LSK_RG1(2, 4); else LSK_RG1(4, 4);
    }
#undef LSK_RG1
    if ((rc = lsk::check_launch("moe_route_gemv1_kernel"))) return rc;
  } else if (use_skinny) {
    if (pair_w) {
      g1.w_ptrs = a->w13_pair_ptrs;
      g1.ldw = (H + 63) / 64 * 64;
      g1.w_bytes = 2 * I * g1.ldw;
      g1.pairs |= 2;
    }
    if ((rc = launch_moe_skinny<0>(g1, w.max_tiles, T, w.gu, s, "moe_skinny_kernel<gate_up>"))) return rc;
  } else if (use_gemv) {
    if ((rc = launch_moe_gemv<0>(g1, w.max_tiles, T, w.gu, s, "moe_gemv_kernel<gate_up>"))) return rc;
  } else if (use_pp) {
    if (pair_w) {
      g1.w_ptrs = a->w13_pair_ptrs;
      g1.ldw = (H + 63) / 64 * 64;
      g1.w_bytes = 2 * I * g1.ldw;
      g1.pairs |= 2;
    }
    if (pp256) {
      g1.tiles = w.tiles2;
      if ((rc = launch_moe_pp256<0>(g1, w.max_tiles2, s, "moe_pp256_kernel<gate_up>"))) return rc;
    } else if ((rc = launch_moe_pp<0>(g1, w.max_tiles, s, "moe_pp_kernel<gate_up>"))) {
      return rc;
    }
  } else if ((rc = launch_moe_gemm<0>(g1, w.max_tiles, (int)((I + 63) / 64), s, "moe_gemm_kernel<gate_up>"))) {
    return rc;
  }
  if (use_gemv || use_skinny || use_mx_gemv || use_mx_skinny) {
    const int per = (int)((I + 1023) / 1024);
    const dim3 grid((unsigned)R), blk(1024);
#define LSK_ACTQ(P)                                                                                             \
  {                                                                                                             \
    if (mx) hipLaunchKernelGGL((moe_act_requant_kernel<P, true>), grid, blk, 0, s, w.gu, w.offs + E, (int)I,    \
                               a->act, a->frac, a->act_tab, (void*)w.qh, w.asch);                               \
    else hipLaunchKernelGGL((moe_act_requant_kernel<P, false>), grid, blk, 0, s, w.gu, w.offs + E, (int)I,      \
                            a->act, a->frac, a->act_tab, (void*)w.qh, w.asch);                                  \
  }
    if (per <= 1) LSK_ACTQ(1) else if (per <= 2) LSK_ACTQ(2) else if (per <= 4) LSK_ACTQ(4) else LSK_ACTQ(8)
#undef LSK_ACTQ
    if ((rc = lsk::check_launch("moe_act_requant_kernel"))) return rc;
  } else if (rb > 0) {
    hipLaunchKernelGGL(moe_rot_requant_kernel, dim3((unsigned)R), dim3(256), (size_t)I * 4, s, w.h, w.offs + E, (int)I,
                       rb, a->rot_scale, w.qh, w.asch);
    if ((rc = lsk::check_launch("moe_rot_requant_kernel"))) return rc;
  } else if (mx == 2) {
    if (use_mx2_skinny) {
      const int64_t blocks = std::min<int64_t>(4096, std::max<int64_t>(1, (R * I + 255) / 256));
      hipLaunchKernelGGL(moe_act_h_kernel, dim3((unsigned)blocks), dim3(256), 0, s, w.gu, w.offs + E, (int)I, a->act,
                         a->frac, a->act_tab, anyf, w.h);
      if ((rc = lsk::check_launch("moe_act_h_kernel"))) return rc;
    }
    if ((rc = lsk::launch_blockquant_mx2(w.h, I, R, w.offs + E, (int)I, (uint16_t*)w.qh, w.kah, w.flagh, anyf + 1,
                                         use_mx2_gemv ? 1 : lo2, use_mx2_gemv ? 0 : hi2, s)))
      return rc;
  } else if (mx) {
    if ((rc = lsk::launch_requant_bf16(w.h, w.h_amax, w.offs + E, R, (int)I, (uint16_t*)w.qh, w.asch, s))) return rc;
  } else {
    int64_t blocks = (R + 3) / 4;  // a wave per row
    blocks = blocks > 8192 ? 8192 : (blocks < 1 ? 1 : blocks);
    hipLaunchKernelGGL(moe_requant_kernel, dim3((unsigned)blocks), dim3(256), 0, s, w.h, w.h_amax, w.offs + E, (int)I,
                       w.qh, w.asch, pair_down ? 1 : 0);
    if ((rc = lsk::check_launch("moe_requant_kernel"))) return rc;
  }
  MoeGemmArgs g2{};
  g2.skinny_rows = g_pp_skinny;
  g2.A = w.qh;
  g2.lda = I;
  g2.a_bytes = pair_down ? ((R + 1) & ~(int64_t)1) * I : R * I * (mx ? 2 : 1);
  g2.pairs = pair_down ? 1 : 0;
  g2.w_bytes = H * a->ldw2;
  g2.a_scale = w.asch;
  g2.offs = w.offs;
  g2.tiles = w.tiles;
  g2.w_ptrs = a->w2_ptrs;
  g2.ldw = a->ldw2;
  g2.ws_ptrs = a->ws2_ptrs;
  g2.b_ptrs = a->b2_ptrs;
  g2.K = (int)I;
  g2.N = (int)H;
  g2.row_w = w.row_w;
  g2.row_dst = w.row_dst;
  g2.y = w.slots;
  g2.lds = a->lds2;
  if (mx == 2) {
    g2.a_scale = nullptr;
    g2.row_flag = w.flagh;
    g2.any_flag = anyf + 1;
    g2.a_ka = w.kah;
    g2.ldka = I / 32;
  }
  if (mx == 1 && T == 1 && k <= 4 && (use_mx_gemv || use_mx_skinny) && lsk::mx_variant() == 0 && H <= 8192 &&
      I <= 8192) {
    // one token: the down GEMV of its (at most four) experts and the combine in one launch
    return lsk::launch_moe_mx_down_combine1(g2, a->mx_safe, a->shared, a->y, s);
  } else if (use_mx_gemv || use_mx2_gemv) {
    if ((rc = lsk::launch_moe_mx_gemv(1, g2, w.max_tiles, T, a->mx_safe, nullptr, s))) return rc;
  } else if (use_mx2_skinny) {
    MoeGemmArgs gs = g2;
    gs.w_ptrs = a->w2_pair_ptrs;
    gs.w_bytes = lsk::mx_skinny_bytes(H, I);
    gs.mx2 = 1;
    if ((rc = lsk::launch_moe_mx_skinny(1, gs, w.max_tiles, T, a->mx_safe, nullptr, s))) return rc;
    g2.mx2 = 3;
    if ((rc = lsk::launch_moe_mx_gemm(1, g2, w.max_tiles, a->mx_safe, s))) return rc;
  } else if (mx == 2) {
    g2.mx2 = 1;
    if ((rc = lsk::launch_moe_mx_gemm(1, g2, w.max_tiles, a->mx_safe, s))) return rc;
    g2.mx2 = 2;
    if ((rc = lsk::launch_moe_mx_gemm(1, g2, w.max_tiles, a->mx_safe, s))) return rc;
  } else if (use_mx_skinny) {
    g2.w_ptrs = a->w2_pair_ptrs;
    g2.w_bytes = lsk::mx_skinny_bytes(H, I);
    if ((rc = lsk::launch_moe_mx_skinny(1, g2, w.max_tiles, T, a->mx_safe, nullptr, s))) return rc;
  } else if (mx) {
    if ((rc = lsk::launch_moe_mx_gemm(1, g2, w.max_tiles, a->mx_safe, s))) return rc;
  } else if (use_gemv && T == 1 && k <= 8 && I <= 2048) {
    // one token: the down GEMV and the combine in one launch (writes y itself)
    const int64_t blocks = (H + 4 * 2 - 1) / (4 * 2);
#define LSK_DC(NCV)                                                                                    \
  hipLaunchKernelGGL((moe_down_combine1_kernel<NCV, 2, 8>), dim3((unsigned)blocks), dim3(256), 0, s, g2, \
                     a->shared, a->y)
    if (I <= 1024) LSK_DC(1);
    else LSK_DC(2);
#undef LSK_DC
    return lsk::check_launch("moe_down_combine1_kernel");
  } else if (use_skinny) {
    if (pair_w) {
      g2.w_ptrs = a->w2_pair_ptrs;
      g2.ldw = (I + 63) / 64 * 64;
      g2.w_bytes = H * g2.ldw;
      g2.pairs |= 2;
    }
    if ((rc = launch_moe_skinny<1>(g2, w.max_tiles, T, nullptr, s, "moe_skinny_kernel<down>"))) return rc;
  } else if (use_gemv) {
    if ((rc = launch_moe_gemv<1>(g2, w.max_tiles, T, nullptr, s, "moe_gemv_kernel<down>"))) return rc;
  } else if (use_pp) {
    if (pair_w) {
      g2.w_ptrs = a->w2_pair_ptrs;
      g2.ldw = (I + 63) / 64 * 64;
      g2.w_bytes = H * g2.ldw;
      g2.pairs |= 2;
    }
    if (pp256) {
      g2.tiles = w.tiles2;
      if ((rc = launch_moe_pp256<1>(g2, w.max_tiles2, s, "moe_pp256_kernel<down>"))) return rc;
    } else if ((rc = launch_moe_pp<1>(g2, w.max_tiles, s, "moe_pp_kernel<down>"))) {
      return rc;
    }
  } else if ((rc = launch_moe_gemm<1>(g2, w.max_tiles, (int)((H + 127) / 128), s, "moe_gemm_kernel<down>"))) {
    return rc;
  }
  {
    int64_t blocks = (T * (H / 8) + 255) / 256;
    blocks = blocks > 8192 ? 8192 : (blocks < 1 ? 1 : blocks);
    hipLaunchKernelGGL(moe_combine_kernel, dim3((unsigned)blocks), dim3(256), 0, s, w.slots, H, k, w.tok_cnt, a->shared,
                       T, a->y);
    if ((rc = lsk::check_launch("moe_combine_kernel"))) return rc;
  }
  return LSK_OK;
}
