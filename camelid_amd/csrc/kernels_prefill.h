// kernels_prefill.h -- HIP/CDNA4 kernels of the batched prefill (gfx950, wave64).
//
// Prefill runs every layer over a chunk of T prompt tokens at once.  Each token's arithmetic
// is the decode step's, in the same order (so the KV cache and the hidden states are
// bit-identical to T single-token steps, and to the CPU path, inference.rs:4411-4425):
//   RMSNorm rows     k_rmsnorm_quant with gridDim.y = T (one workgroup per token)
//   projections      k_gemm_q8: int8 matrix cores for the per-block dots, f32 folds in block order
//   QK-norm/RoPE/KV  k_rope_kv with gridDim.y = T
//   attention        k_attn_prefill: one workgroup per (head, token), causal over [0, pos]
//   SwiGLU           k_silu_rows
#pragma once
#include "kernels_decode.h"

namespace cm {

typedef int v4i_t __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------------------
// Q8_0 GEMM (q8_gemm_batched, cuda_resident.rs:1494; CPU: the row dot of
// inference.rs:19871-19905 per token):
//   y[t][n] = (resid ? resid[t][n] : 0) + fold_b (float(dot_b(W[n], X[t])) * wd[n][b]) * xs[t][b]
// with dot_b the exact int32 dot of one 32-value block and the fold in block order from 0.
// The block dots run on the matrix cores: one v_mfma_i32_16x16x32_i8 per 16x16 (rows x
// tokens) fragment and block; its K = 32 is exactly one Q8_0 block, so every block's int32
// dot comes out separately (any assignment of the 32 byte positions to lanes gives the same
// integer, as long as the weight and activation operands use the same one).
// Workgroup: 4 waves over a (32 NF)-row x 64-token tile, each wave 16 NF x 32 (NF x 2 fragments).
// Lane l of a fragment supplies row / token l % 16, bytes 8*(l/16) .. +7 of the block, and
// receives the outputs of rows 4*(l/16) + i (i = 0..3) for token l % 16.
// Operands move in steps of 4 blocks (128 bytes of every row and token): coalesced 16-byte
// global loads into registers one step ahead, then into a double-buffered LDS tile laid out
// [block][8-byte piece][row] (a fragment read is 16 consecutive 8-byte pieces per piece
// index: no bank conflicts).  Scales are staged in LDS 8 blocks at a time (transposed:
// [block][row], [block][token]), the next group's held in registers meanwhile.
// Tiles are dealt so that each XCD (workgroup id mod 8) runs a contiguous range of tiles,
// token tiles innermost: the row tile's weights are read once per XCD and re-read from its L2.
// N % 4 == 0 (16-byte output stores); K % 32 == 0; y may alias resid.
constexpr int GM_NT = 256;
constexpr int GM_RT = 64;  // tokens per workgroup tile
constexpr int GM_BG = 8;   // blocks per scale-staging group
constexpr int GM_SB = 4;   // blocks per operand step
// Rows per workgroup tile: 32 * NF, NF = 2 (64) or 1 (32, for small grids: a [3072 x 3072] x 511
// product has 384 tiles of 64 x 64, one or two 4-wave workgroups per CU, and a single wave
// issues one VALU instruction per ~7 clocks, so each SIMD then idles half the time).
__host__ __device__ constexpr int gm_rows(int NF) { return 32 * NF; }
// 8-byte pieces per [block][piece] row of an LDS operand tile: rows + 1 pad, so that the
// planes start 2 banks apart (2 * rows + 2 dwords) and the 8 pieces a row's 16-byte chunks
// scatter to land in different banks (the tile writes are otherwise 8-way bank conflicts)
__host__ __device__ constexpr int gm_ps(int rows) { return rows + 1; }
// The block dots start from the bit pattern of 1.5 * 2^23 instead of 0: |dot| <= 32 * 128^2
// = 2^19 < 2^22, so the int32 sum's bits are those of the f32 value 1.5 * 2^23 + dot (ulp 1
// in [2^23, 2^24)), and fma(f, w, -(1.5 * 2^23) w) = round(f w - 1.5 * 2^23 w) = round(dot w)
// exactly (the FMA rounds once, -(1.5 * 2^23) w is exact for every f16 w: 13 significant
// bits, no overflow).  That is float(dot) * w in one mixed-precision FMA, in place of a
// conversion and a multiply.  An infinite w (dot * w = +-inf, or NaN at dot = 0) is the one
// value it does not give: a matrix whose weight scales hold one runs k_gemm_q8<true, NF>, the
// plain form (the host decides per matrix).
constexpr int32_t GM_MAGIC = 0x4B400000;
constexpr float GM_MAGIC_F = 12582912.0f;

// a * f32(lo / hi half of w) + c, rounded once: one v_fma_mix_f32.  Written as an fma of the
// widened half (not inline assembly): the operand a comes straight from a matrix-core result,
// and only compiler-visible reads get the wait states the hardware needs after an MFMA write.
__device__ __forceinline__ float fma_f16_lo(float a, uint32_t w, float c) {
  _Float16 h[2];
  __builtin_memcpy(h, &w, 4);
  return __builtin_fmaf(a, (float)h[0], c);
}
__device__ __forceinline__ float fma_f16_hi(float a, uint32_t w, float c) {
  _Float16 h[2];
  __builtin_memcpy(h, &w, 4);
  return __builtin_fmaf(a, (float)h[1], c);
}

template <typename V, V X>
struct gm_const {
  static constexpr V value = X;
};

__host__ __device__ inline int gemm_tiles(int N, int T, int NF = 2) {
  return ((N + gm_rows(NF) - 1) / gm_rows(NF)) * ((T + GM_RT - 1) / GM_RT);
}
__host__ __device__ inline int gemm_grid(int N, int T, int NF = 2) { return ((gemm_tiles(N, T, NF) + 7) / 8) * 8; }

// PLAIN: the dots from 0, converted and multiplied by the weight scale (two VALU operations);
// else from the 1.5 * 2^23 pattern, one FMA (GM_MAGIC).  Both give float(dot) * w rounded
// once, then * xs, then + in block order.
// Waves: 2 (rows) x 2 (tokens), each 16 NF rows x 32 tokens (NF x 2 fragments).
// (at most 128 VGPRs and, with 8-block scale groups, under 40 KB of LDS: four workgroups per CU)
template <bool PLAIN, int NF>
__global__ __launch_bounds__(GM_NT, 4) void k_gemm_q8(const int8_t* __restrict__ wq, const uint16_t* __restrict__ wd,
                                                   int N, int K, const int8_t* __restrict__ xq,
                                                   const float* __restrict__ xs, int T, float* y,
                                                   const float* resid) {
  constexpr int RN = gm_rows(NF), PSA = gm_ps(RN), PSB = gm_ps(GM_RT);
  constexpr int AJ = RN / 32, BJ = GM_RT / 32;  // 16-byte global loads per thread and step
  static_assert((NF == 1 || NF == 2) && GM_RT == 64 && GM_NT == 256 && GM_SB == 4 && GM_BG % GM_SB == 0 &&
                    GM_NT % GM_BG == 0, "tile layout");
  __shared__ __align__(16) uint2 sa[2][GM_SB][4][PSA];
  __shared__ __align__(16) uint2 sb[2][GM_SB][4][PSB];
  __shared__ __align__(16) uint16_t swd[GM_BG][RN + 4];
  __shared__ __align__(16) float snb[GM_BG][RN + 4];  // -(1.5 * 2^23) * f32(wd)
  __shared__ __align__(16) float sxs[GM_BG][GM_RT + 1];
  const int NB = K >> 5;
  const int nsteps = (NB + GM_SB - 1) / GM_SB;
  const int ntt = (T + GM_RT - 1) / GM_RT;
  const int tiles = gemm_tiles(N, T, NF);
  const int per = (tiles + 7) >> 3;
  const int L = (int)(blockIdx.x & 7) * per + (int)(blockIdx.x >> 3);
  if (L >= tiles) return;
  const int n_base = (L / ntt) * RN, t_base = (L % ntt) * GM_RT;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int r = lane & 15, g = lane >> 4;
  const int wn = (wave & 1) * 16 * NF, wt = (wave >> 1) * 32;

  // global -> register loads of one step: chunk j of thread tid is 16 bytes of row / token
  // (tid + 256 j) / 8 at byte (tid % 8) * 16 of the step's 128
  const int crow = tid >> 3, cc = tid & 7;
  const int8_t* ga[AJ];
  const int8_t* gb[BJ];
#pragma unroll
  for (int j = 0; j < AJ; ++j) ga[j] = wq + (size_t)min(n_base + crow + 32 * j, N - 1) * K;
#pragma unroll
  for (int j = 0; j < BJ; ++j) gb[j] = xq + (size_t)min(t_base + crow + 32 * j, T - 1) * K;
  uint4 ra[AJ], rb[BJ];
  auto gload = [&](int step) __attribute__((always_inline)) {
    const int off = min(step * 128 + cc * 16, K - 16);
#pragma unroll
    for (int j = 0; j < AJ; ++j) ra[j] = *reinterpret_cast<const uint4*>(ga[j] + off);
#pragma unroll
    for (int j = 0; j < BJ; ++j) rb[j] = *reinterpret_cast<const uint4*>(gb[j] + off);
  };
  auto lds_put = [&](int buf) __attribute__((always_inline)) {  // bytes 0..7 -> piece 2(cc%2), 8..15 -> piece 2(cc%2)+1
    const int bl = cc >> 1, pc = (cc & 1) * 2;
#pragma unroll
    for (int j = 0; j < AJ; ++j) {
      sa[buf][bl][pc][crow + 32 * j] = make_uint2(ra[j].x, ra[j].y);
      sa[buf][bl][pc + 1][crow + 32 * j] = make_uint2(ra[j].z, ra[j].w);
    }
#pragma unroll
    for (int j = 0; j < BJ; ++j) {
      sb[buf][bl][pc][crow + 32 * j] = make_uint2(rb[j].x, rb[j].y);
      sb[buf][bl][pc + 1][crow + 32 * j] = make_uint2(rb[j].z, rb[j].w);
    }
  };

  // scale staging: thread tid carries block tid % GM_BG of rows / tokens tid / GM_BG + 16 i
  constexpr int SPW = GM_BG * RN / GM_NT, SPX = GM_BG * GM_RT / GM_NT, SRS = GM_NT / GM_BG;
  uint32_t pw[SPW];
  float px[SPX];
  auto stage_load = [&](int g0) __attribute__((always_inline)) {
    const int blk = min(g0 + (tid % GM_BG), NB - 1);
#pragma unroll
    for (int i = 0; i < SPW; ++i) pw[i] = wd[(size_t)min(n_base + tid / GM_BG + SRS * i, N - 1) * NB + blk];
#pragma unroll
    for (int i = 0; i < SPX; ++i) px[i] = xs[(size_t)min(t_base + tid / GM_BG + SRS * i, T - 1) * NB + blk];
  };
  auto stage_store = [&]() __attribute__((always_inline)) {
    const int bb = tid % GM_BG;
#pragma unroll
    for (int i = 0; i < SPW; ++i) {
      const int row = tid / GM_BG + SRS * i;
      swd[bb][row] = (uint16_t)pw[i];
      if (!PLAIN) snb[bb][row] = -GM_MAGIC_F * half_bits_to_float((uint16_t)pw[i]);
    }
#pragma unroll
    for (int i = 0; i < SPX; ++i) sxs[bb][tid / GM_BG + SRS * i] = px[i];
  };

  float acc[NF][2][4];
#pragma unroll
  for (int nf = 0; nf < NF; ++nf)
#pragma unroll
    for (int tf = 0; tf < 2; ++tf)
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[nf][tf][i] = 0.0f;

  // block b = step block bl, from LDS buffer buf
  auto block = [&](int buf, int bl, int b) __attribute__((always_inline)) {
    constexpr bool plain = PLAIN;
    long av[NF], bv[2];
#pragma unroll
    for (int f = 0; f < NF; ++f) av[f] = *reinterpret_cast<const long*>(&sa[buf][bl][g][wn + 16 * f + r]);
#pragma unroll
    for (int f = 0; f < 2; ++f) bv[f] = *reinterpret_cast<const long*>(&sb[buf][bl][g][wt + 16 * f + r]);
    const int32_t c0 = plain ? 0 : GM_MAGIC;
    v4i_t c[NF][2];
#pragma unroll
    for (int nf = 0; nf < NF; ++nf)
#pragma unroll
      for (int tf = 0; tf < 2; ++tf)
        c[nf][tf] = __builtin_amdgcn_mfma_i32_16x16x32_i8(av[nf], bv[tf], v4i_t{c0, c0, c0, c0}, 0, 0, 0);
    const int sl = b & (GM_BG - 1);
    uint2 w2[NF];
    float4 nb[NF];
    float xv[2];
#pragma unroll
    for (int nf = 0; nf < NF; ++nf) {
      w2[nf] = *reinterpret_cast<const uint2*>(&swd[sl][wn + 16 * nf + 4 * g]);
      if (!plain) nb[nf] = *reinterpret_cast<const float4*>(&snb[sl][wn + 16 * nf + 4 * g]);
    }
#pragma unroll
    for (int tf = 0; tf < 2; ++tf) xv[tf] = sxs[sl][wt + 16 * tf + r];
#pragma unroll
    for (int nf = 0; nf < NF; ++nf)
#pragma unroll
      for (int tf = 0; tf < 2; ++tf) {
        if (plain) {
          acc[nf][tf][0] += mul_f16_lo((float)c[nf][tf][0], w2[nf].x) * xv[tf];
          acc[nf][tf][1] += mul_f16_hi((float)c[nf][tf][1], w2[nf].x) * xv[tf];
          acc[nf][tf][2] += mul_f16_lo((float)c[nf][tf][2], w2[nf].y) * xv[tf];
          acc[nf][tf][3] += mul_f16_hi((float)c[nf][tf][3], w2[nf].y) * xv[tf];
        } else {
          acc[nf][tf][0] += fma_f16_lo(__int_as_float(c[nf][tf][0]), w2[nf].x, nb[nf].x) * xv[tf];
          acc[nf][tf][1] += fma_f16_hi(__int_as_float(c[nf][tf][1]), w2[nf].x, nb[nf].y) * xv[tf];
          acc[nf][tf][2] += fma_f16_lo(__int_as_float(c[nf][tf][2]), w2[nf].y, nb[nf].z) * xv[tf];
          acc[nf][tf][3] += fma_f16_hi(__int_as_float(c[nf][tf][3]), w2[nf].y, nb[nf].w) * xv[tf];
        }
      }
    // the folds stay in this block (not sunk past the staging branch with the dots held live)
#pragma unroll
    for (int nf = 0; nf < NF; ++nf)
#pragma unroll
      for (int tf = 0; tf < 2; ++tf)
#pragma unroll
        for (int i = 0; i < 4; ++i) asm volatile("" : "+v"(acc[nf][tf][i]));
  };
  // operand step s from LDS buffer s % 2, GM_SB blocks (FULL) or the NB % GM_SB of the last
  // step; then the next step's operands into the other buffer
  auto run_step = [&](int s, auto fullc) __attribute__((always_inline)) {
    constexpr bool full = decltype(fullc)::value;
    const int buf = s & 1, b0 = s * GM_SB;
    if (s + 1 < nsteps) gload(s + 1);
    if (full) {
      block(buf, 0, b0);
      block(buf, 1, b0 + 1);
      block(buf, 2, b0 + 2);
      block(buf, 3, b0 + 3);
    } else {
      for (int bl = 0; bl < NB - b0; ++bl) block(buf, bl, b0 + bl);
    }
    if (s + 1 < nsteps && ((s + 1) * GM_SB) % GM_BG == 0) {  // next step opens a new scale group
      lds_put(buf ^ 1);
      __syncthreads();  // every wave is done with this group's scales
      stage_store();
      const int g_next = (s + 1) * GM_SB + GM_BG;
      if (g_next < NB) stage_load(g_next);
      __syncthreads();
    } else {
      if (s + 1 < nsteps) lds_put(buf ^ 1);
      __syncthreads();
    }
  };

  stage_load(0);
  gload(0);
  stage_store();
  if (GM_BG < NB) stage_load(GM_BG);
  lds_put(0);
  __syncthreads();
  const int nfull = NB / GM_SB;
  for (int s = 0; s < nfull; ++s) run_step(s, gm_const<bool, true>{});
  if (nfull < nsteps) run_step(nfull, gm_const<bool, false>{});  // the partial last step
#pragma unroll
  for (int nf = 0; nf < NF; ++nf)
#pragma unroll
    for (int tf = 0; tf < 2; ++tf) {
      const int t = t_base + wt + 16 * tf + r, n = n_base + wn + 16 * nf + 4 * g;
      if (t < T && n < N) {
        const size_t o = (size_t)t * N + n;
        float4 v = make_float4(acc[nf][tf][0], acc[nf][tf][1], acc[nf][tf][2], acc[nf][tf][3]);
        if (resid) {
          const float4 rr = *reinterpret_cast<const float4*>(resid + o);
          v = make_float4(rr.x + v.x, rr.y + v.y, rr.z + v.z, rr.w + v.w);
        }
        *reinterpret_cast<float4*>(y + o) = v;
      }
    }
}

// Sets *flag (cleared by the caller) when one of the n f16 values is +-inf: which fold form a
// matrix of device-resident weight scales needs (k_gemm_q8<true> if set).
__global__ __launch_bounds__(256) void k_f16_any_inf(const uint16_t* __restrict__ h, size_t n, uint32_t* flag) {
  bool inf = false;
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256)
    inf |= (h[i] & 0x7fffu) == 0x7c00u;
  if (inf) *flag = 1u;  // every writer stores the same value
}

// ---------------------------------------------------------------------------
// Greedy argmax (inference.rs:5912-5925: first index of the max, strict '>') of T rows of n
// logits: workgroup (p, t) reduces slice p of row t to a (value, index) pair, then one
// wave per row reduces the AMR_PARTS pairs; a row with no value above -inf gives 0.
constexpr int AMR_PARTS = 64;
__global__ __launch_bounds__(256) void k_argmax_rows_part(const float* __restrict__ x, int n,
                                                          float* __restrict__ pv, uint32_t* __restrict__ pi) {
  __shared__ float rv[4];
  __shared__ uint32_t ri[4];
  const int t = blockIdx.y, p = blockIdx.x, tid = threadIdx.x;
  const int per = (n + AMR_PARTS - 1) / AMR_PARTS;
  const int lo = p * per, hi = min(n, lo + per);
  const float* row = x + (size_t)t * n;
  float bv = -INFINITY;
  uint32_t bi = 0xffffffffu;
  for (int i = lo + tid; i < hi; i += 256) {
    const float v = row[i];
    if (v > bv) {
      bv = v;
      bi = (uint32_t)i;
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) argmax_pair(bv, bi, __shfl_xor(bv, o), __shfl_xor(bi, o));
  if ((tid & 63) == 0) {
    rv[tid >> 6] = bv;
    ri[tid >> 6] = bi;
  }
  __syncthreads();
  if (tid == 0) {
    for (int w = 1; w < 4; ++w) argmax_pair(bv, bi, rv[w], ri[w]);
    pv[t * AMR_PARTS + p] = bv;
    pi[t * AMR_PARTS + p] = bi;
  }
}

__global__ __launch_bounds__(64) void k_argmax_rows_finish(const float* __restrict__ pv,
                                                           const uint32_t* __restrict__ pi,
                                                           uint32_t* __restrict__ out) {
  const int t = blockIdx.x, lane = threadIdx.x;
  float bv = pv[t * AMR_PARTS + lane];
  uint32_t bi = pi[t * AMR_PARTS + lane];
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) argmax_pair(bv, bi, __shfl_xor(bv, o), __shfl_xor(bi, o));
  if (lane == 0) out[t] = bi == 0xffffffffu ? 0u : bi;
}

// ---------------------------------------------------------------------------
// Y[t] = W . X[t] (+ resid[t]) for 1 <= T <= GMT_MAX tokens (speculative verify, short
// prefill chunks): the single-token GEMV's arithmetic for every (row, token) -- exact int32
// block dots, terms ((float)dot * d_w) * d_x, the in-order fold over blocks -- with each
// weight chunk loaded once and dotted with all T activations (a 64-token matrix-core tile
// would leave most CUs idle at this size).  4 waves x GMT_RPW rows per workgroup.
// Dynamic LDS: gemv_multi_lds_bytes(K, T).
constexpr int GMT_MAX = 8;
constexpr int GMT_RPW = 1;
constexpr int GMT_ROWS = 4 * GMT_RPW;
// LDS: the activations [T][K] i8 and their scales [T][K/32] f32, each rounded up to whole
// 1 KB wave loads (a direct load writes all 64 lanes' 16 bytes, the last one past the data),
// then per wave the terms of one 32-block slice [GMT_RPW][T][32] f32
__host__ __device__ inline size_t gemv_multi_xq_bytes(int K, int T) {
  return (((size_t)T * K + 1023) / 1024) * 1024;
}
__host__ __device__ inline size_t gemv_multi_xs_bytes(int K, int T) {
  return (((size_t)T * (K / 32) * 4 + 1023) / 1024) * 1024;
}
__host__ __device__ inline size_t gemv_multi_lds_bytes(int K, int T) {
  return gemv_multi_xq_bytes(K, T) + gemv_multi_xs_bytes(K, T) + (size_t)GMT_ROWS * T * 32 * 4;
}

template <int K>
__global__ __launch_bounds__(256) void k_gemv_multi(const int8_t* __restrict__ wq, const uint16_t* __restrict__ wd,
                                                    int rows, const int8_t* __restrict__ xq,
                                                    const float* __restrict__ xs, int T, float* y,
                                                    const float* resid) {
  constexpr int NB = K / 32, CPR = K / 16, IT = (CPR + 63) / 64;
  static_assert(NB % 4 == 0, "compile-time GEMV widths are multiples of 128");
  extern __shared__ __align__(16) unsigned char gmt_lds[];
  int8_t* xl = reinterpret_cast<int8_t*>(gmt_lds);                    // [T][K]
  float* xsl = reinterpret_cast<float*>(gmt_lds + gemv_multi_xq_bytes(K, T));  // [T][NB]
  // this wave's slice terms [GMT_RPW][T][32]
  float* tw = reinterpret_cast<float*>(gmt_lds + gemv_multi_xq_bytes(K, T) + gemv_multi_xs_bytes(K, T)) +
              (size_t)(threadIdx.x >> 6) * GMT_RPW * T * 32;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int row0 = blockIdx.x * GMT_ROWS;
  // the activations and their scales go to LDS by direct loads (1 KB per wave load; a last
  // load may overrun into its region's rounded-up pad, re-reading the last piece)
  {
    const uint4* sx = reinterpret_cast<const uint4*>(xq);
    const uint4* ss = reinterpret_cast<const uint4*>(xs);
    uint4* dx = reinterpret_cast<uint4*>(xl);
    uint4* ds = reinterpret_cast<uint4*>(xsl);
    const int nx = T * CPR, ns = (T * NB * 4 + 15) / 16;
    for (int b = wave * 64; b < nx; b += 256)
      __builtin_amdgcn_global_load_lds(reinterpret_cast<const void*>(sx + min(b + lane, nx - 1)),
                                       (__attribute__((address_space(3))) void*)(dx + b), 16, 0, 0);
    for (int b = wave * 64; b < ns; b += 256)
      __builtin_amdgcn_global_load_lds(reinterpret_cast<const void*>(ss + min(b + lane, ns - 1)),
                                       (__attribute__((address_space(3))) void*)(ds + b), 16, 0, 0);
  }
  int4 wv[GMT_RPW][IT];
  uint16_t dv[GMT_RPW][IT];
#pragma unroll
  for (int k = 0; k < GMT_RPW; ++k) {
    const int row = min(row0 + wave * GMT_RPW + k, rows - 1);
    const int4* w4 = reinterpret_cast<const int4*>(wq + (size_t)row * K);
    const uint16_t* d = wd + (size_t)row * NB;
#pragma unroll
    for (int i = 0; i < IT; ++i) {
      const int c = min(lane + 64 * i, CPR - 1);
      wv[k][i] = ld_stream(w4 + c);
      dv[k][i] = ld_stream(d + (c >> 1));
    }
  }
  __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8));  // vmcnt(0): this wave's direct loads have landed
  __syncthreads();
  // slice i = blocks 32 i .. 32 i + 31 of every (row, token): lane pairs form the block terms
  // into LDS, then lane f (< GMT_RPW * T) continues the in-order fold of (row f / T, token
  // f % T) over them (wave-level ordering only: the slice buffer is this wave's)
  auto wave_sync = [] {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  };
  float acc = 0.0f;
#pragma unroll
  for (int i = 0; i < IT; ++i) {
    const int c = lane + 64 * i;
    const int cc = min(c, CPR - 1);
#pragma unroll
    for (int k = 0; k < GMT_RPW; ++k) {
      const float dw = half_bits_to_float(dv[k][i]);
      for (int tk = 0; tk < T; ++tk) {
        int sacc = dot4x4(wv[k][i], reinterpret_cast<const int4*>(xl + (size_t)tk * K)[cc], 0);
        sacc += dpp_xor1(sacc);
        if ((lane & 1) == 0 && c < CPR)
          tw[(k * T + tk) * 32 + (lane >> 1)] = ((float)sacc * dw) * xsl[tk * NB + (c >> 1)];
      }
    }
    wave_sync();
    if (lane < GMT_RPW * T) {
      const int nb = min(32, NB - 32 * i);
      acc = fold_lds(tw + (size_t)lane * 32, nb, acc);
    }
    wave_sync();
  }
  if (lane < GMT_RPW * T) {
    const int lr = wave * GMT_RPW + lane / T, tk = lane - (lane / T) * T;
    const int row = row0 + lr;
    if (row < rows) {
      const size_t o = (size_t)tk * rows + row;
      y[o] = resid ? resid[o] + acc : acc;
    }
  }
}

// ---------------------------------------------------------------------------
// Causal attention of a prefill chunk (attention_batched, cuda_resident.rs:1994; CPU
// inference.rs:23945-24025 per token): one workgroup per (query head, token); token t of
// the chunk sits at position pos0 + t and attends positions [0, pos0 + t], all already in
// the cache.  The arithmetic is the decode kernel's: scores one lane per position with d in
// order, exact max, glibc expf, a serial fold of the exponentials, normalisation by the
// reciprocal, and out_d folded over positions in order (one lane per d).  A single position
// copies the V row (inference.rs:23564-23575).  The output row is quantized to Q8_0.
// Rows are dealt longest first.  Dynamic LDS: align4(pos0 + T) floats.
constexpr int AP_NT = 256;

template <int HD>
__global__ __launch_bounds__(AP_NT) void k_attn_prefill(const float* __restrict__ qrot, int n_heads, int n_kv,
                                                        const uint16_t* __restrict__ kc, const uint16_t* __restrict__ vc,
                                                        int layer, int kvs, int pos0, float scale,
                                                        float* __restrict__ att_out, int8_t* __restrict__ xq,
                                                        float* __restrict__ xs) {
  static_assert(HD % 64 == 0 && HD <= AP_NT, "head_dim must be 64, 128 or 256");
  constexpr int R8 = HD / 8;
  extern __shared__ __align__(16) float sc[];
  __shared__ __align__(16) float qs[HD];
  __shared__ float red[AP_NT / 64];
  __shared__ float s_inv;
  const int tid = threadIdx.x;
  const int h = blockIdx.x;
  const int t = (int)gridDim.y - 1 - (int)blockIdx.y;
  const int pos = pos0 + t, P = pos + 1;
  const int kvh = h / (n_heads / n_kv);
  const size_t hbase = kv_head_base(layer, n_kv, kvh, HD, kvs);
  const uint4* kg = reinterpret_cast<const uint4*>(kc + hbase);
  const uint4* vg = reinterpret_cast<const uint4*>(vc + hbase);
  const size_t row = (size_t)t * n_heads * HD + (size_t)h * HD;
  if (tid < HD) qs[tid] = qrot[row + tid];
  __syncthreads();
  float o = 0.0f;
  if (P == 1) {
    if (tid < HD) o = half_bits_to_float(vc[hbase + kv_v_index(HD, 0, tid)]);
  } else {
    float lmax = -INFINITY;
    for (int p = tid; p < P; p += AP_NT) {
      uint4 rk[R8];
#pragma unroll
      for (int u = 0; u < R8; ++u) rk[u] = kg[(size_t)u * kvs + p];
      float a = 0.0f;
#pragma unroll
      for (int u = 0; u < R8; ++u) {
        __builtin_amdgcn_sched_barrier(0);
        const float4 qa = reinterpret_cast<const float4*>(qs)[2 * u];
        const float4 qb = reinterpret_cast<const float4*>(qs)[2 * u + 1];
        a += mul_f16_lo(qa.x, rk[u].x);
        a += mul_f16_hi(qa.y, rk[u].x);
        a += mul_f16_lo(qa.z, rk[u].y);
        a += mul_f16_hi(qa.w, rk[u].y);
        a += mul_f16_lo(qb.x, rk[u].z);
        a += mul_f16_hi(qb.y, rk[u].z);
        a += mul_f16_lo(qb.z, rk[u].w);
        a += mul_f16_hi(qb.w, rk[u].w);
      }
      const float sv = a * scale;
      sc[p] = sv;
      lmax = fmaxf(lmax, sv);
    }
    const float mx = block_max(lmax, red);
    for (int p = tid; p < P; p += AP_NT) sc[p] = glibc_expf(sc[p] - mx);
    __syncthreads();
    if (tid == 0) s_inv = 1.0f / fold_lds(sc, P);
    __syncthreads();
    const float inv = s_inv;
    for (int p = tid; p < P; p += AP_NT) sc[p] = sc[p] * inv;
    __syncthreads();
    if (tid < HD) {
      const int ng = P >> 3;  // full granules of 8 positions (f16 V, one FMA-mix product each)
      const float4* pr4 = reinterpret_cast<const float4*>(sc);
      float a = 0.0f;
      auto granule = [&](const uint4& g, int j) {
        const float4 p0 = pr4[2 * j], p1 = pr4[2 * j + 1];
        const float r0 = mul_f16_lo(p0.x, g.x), r1 = mul_f16_hi(p0.y, g.x);
        const float r2 = mul_f16_lo(p0.z, g.y), r3 = mul_f16_hi(p0.w, g.y);
        const float r4 = mul_f16_lo(p1.x, g.z), r5 = mul_f16_hi(p1.y, g.z);
        const float r6 = mul_f16_lo(p1.z, g.w), r7 = mul_f16_hi(p1.w, g.w);
        a += r0;
        a += r1;
        a += r2;
        a += r3;
        a += r4;
        a += r5;
        a += r6;
        a += r7;
      };
      int j = 0;
      for (; j + 4 <= ng; j += 4) {
        uint4 v[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) v[u] = vg[(size_t)(j + u) * HD + tid];
#pragma unroll
        for (int u = 0; u < 4; ++u) granule(v[u], j + u);
      }
      for (; j < ng; ++j) granule(vg[(size_t)j * HD + tid], j);
      for (int p = ng * 8; p < P; ++p) a += sc[p] * half_bits_to_float(vc[hbase + kv_v_index(HD, p, tid)]);
      o = a;
    }
  }
  if (tid < HD) {
    if (att_out) att_out[row + tid] = o;
    int8_t q;
    const float dd = quantize_lane32(o, &q);
    xq[row + tid] = q;
    if ((tid & 31) == 0) xs[(row + tid) >> 5] = dd;
  }
}

// ---------------------------------------------------------------------------
// Causal attention of a prefill chunk, tiled over query tokens (attention_batched and the
// flash prefill of cuda_resident.rs:1994, :2523-2757; CPU inference.rs:23945-24025 per token).
// One workgroup per (KV head g, tile of TQ consecutive tokens).  Its rows are the (query head
// g*rep + i, token t0 + j) pairs, row r = i*TQ + j, at most 64 of them, so each K and V row of
// the cache is loaded once per tile and used by every row of it (k_attn_prefill loads it once
// per (head, token)).  Each row's arithmetic is k_attn_prefill's, in the same order:
//   A  scores s_p = (sum_d q_d * k_pd, d in order) * scale over 128-position blocks of K
//      granules in LDS, 4 rows x 4 positions per thread (16 independent chains); the scores go
//      to the scratch rows sc[r][p]; the row maximum (exact, any order);
//   B  e_p = expf(s_p - m_r), written back over the score, and folded into the row's sum in
//      position order by one lane per row (wave 0); inv_r = 1 / sum;
//   C  prob_p = e_p * inv_r, out_rd = fold_p prob_p * v_pd in position order: the block's V
//      granules in LDS, 4 rows x DB dims per thread.
// Every thread reads back only the scratch words it wrote itself (phases A, B and C share one
// (rows, positions) assignment), so no cache line of another thread's is ever stale.  The next
// block's global loads (K and V granules, scratch words) go out before the current block is
// computed.  A row's positions p >= P_r = pos0 + t + 1 contribute e = 0 to its sum and nothing
// to its outputs (masked adds in the blocks that reach past the tile's first row); a sum that
// starts at +0 and adds non-negative terms is never -0, so adding +0 leaves it unchanged.  A
// row with P_r = 1 copies the V row (inference.rs:23564-23575).  Outputs as k_attn_prefill:
// f32 rows (optional) and Q8_0 per 32-value block.  Scratch: sc + tile_index * 64 * pitch
// floats, pitch >= P_max rounded up to 128.  Dynamic LDS: apt_lds_bytes(HD).
constexpr int APT_NT = 1024;  // threads (the kernel is also instantiated at 512)
constexpr int APT_R = 64;    // rows per tile
constexpr int APT_PB = 128;  // positions per block
constexpr int APT_ES = APT_PB + 4;  // row stride of the exponential / probability block
__host__ __device__ constexpr int apt_tq(int rep) { return rep >= APT_R ? 1 : APT_R / rep; }
__host__ __device__ constexpr size_t apt_pitch(size_t pmax) { return (pmax + APT_PB - 1) / APT_PB * APT_PB; }
__host__ __device__ constexpr size_t apt_lds_bytes(int hd) {
  return (size_t)hd * APT_R * 4 + (size_t)(hd / 8) * APT_PB * 16 + (size_t)APT_R * APT_ES * 4;
}
__host__ __device__ constexpr bool apt_hd_ok(int hd) { return hd == 64 || hd == 128; }

// the f16 value e of the 8 in a 16-byte granule times x, rounded once (v_fma_mix)
__device__ __forceinline__ float mul_gran(float x, const uint4& g, int e) {
  const uint32_t w = e < 2 ? g.x : e < 4 ? g.y : e < 6 ? g.z : g.w;
  return (e & 1) ? mul_f16_hi(x, w) : mul_f16_lo(x, w);
}

template <int HD, int NT = APT_NT>
__global__ __launch_bounds__(NT) void k_attn_prefill_tile(
    const float* __restrict__ qrot, int n_heads, int n_kv, const uint16_t* __restrict__ kc,
    const uint16_t* __restrict__ vc, int layer, int kvs, int pos0, int T, float scale, float* __restrict__ scg,
    size_t pitch, float* __restrict__ att_out, int8_t* __restrict__ xq, float* __restrict__ xs) {
  static_assert(apt_hd_ok(HD), "tiled prefill attention: head_dim 64 or 128");
  constexpr int R8 = HD / 8;            // K granules per position
  constexpr int DB = HD / 32;           // output dims per thread in phase C (32 dim groups)
  constexpr int KG = R8 * APT_PB;       // K granules of a block (as many V granules: APT_PB/8 x HD)
  constexpr int GPT = KG / NT;          // of them per thread
  constexpr int NRG = NT / 32;          // row groups: 32 threads each (4 positions / DB dims a thread)
  constexpr int RPT = APT_R / NRG;      // rows per thread: 4 at 512 threads, 2 at 1024
  static_assert(KG == (APT_PB / 8) * HD && KG % NT == 0 && (RPT == 2 || RPT == 4), "block staging");
  extern __shared__ __align__(16) float4 dyn[];
  float* qs = reinterpret_cast<float*>(dyn);              // [HD][64] q tile; later out rows [64][HD]
  uint4* kb = reinterpret_cast<uint4*>(qs + HD * APT_R);  // K granules [R8][PB], then V [PB/8][HD]
  float* eb = reinterpret_cast<float*>(kb + KG);          // [64][APT_ES] exponentials / probabilities
  __shared__ float mrow[APT_R], irow[APT_R];
  __shared__ int prow[APT_R];  // P_r (0: no row in this slot)
  const int tid = threadIdx.x;
  const int rep = n_heads / n_kv, TQ = apt_tq(rep);
  const int g = blockIdx.x, ntile = gridDim.y, tile = ntile - 1 - (int)blockIdx.y;  // longest first
  const int t0 = tile * TQ;
  const size_t hbase = kv_head_base(layer, n_kv, g, HD, kvs);
  const uint4* kg = reinterpret_cast<const uint4*>(kc + hbase);
  const uint4* vg = reinterpret_cast<const uint4*>(vc + hbase);
  float* sc = scg + ((size_t)g * ntile + tile) * APT_R * pitch;
  auto row_head = [&](int r) { return g * rep + r / TQ; };
  auto row_tok = [&](int r) { return t0 + r % TQ; };
  if (tid < APT_R) {
    const int i = tid / TQ, t = t0 + tid % TQ;
    prow[tid] = (i < rep && t < T) ? pos0 + t + 1 : 0;
  }
  const int pmax = pos0 + min(t0 + TQ, T);  // the tile's longest row
  const int pmin = pos0 + t0 + 1;           // its shortest
  const int nblk = (pmax + APT_PB - 1) / APT_PB;
  // staging of block b through registers: K granule (u, p) or V granule (group, d) number
  // i = tid + NT * k (GPT = 1, 2 or 4 named registers: an array here went to scratch memory)
  const int glast = (pmax - 1) >> 3;
  uint4 stg0, stg1, stg2, stg3;
  auto kgran = [&](int b, int k) {
    const int i = tid + NT * k, u = i / APT_PB, p = i % APT_PB;
    return kg[(size_t)u * kvs + min(b * APT_PB + p, pmax - 1)];
  };
  auto vgran = [&](int b, int k) {
    const int i = tid + NT * k, gq = i / HD, d = i % HD;
    return vg[(size_t)min(b * (APT_PB / 8) + gq, glast) * HD + d];
  };
#define APT_LOAD_K(b)                                       \
  stg0 = kgran((b), 0);                                     \
  if (GPT > 1) stg1 = kgran((b), 1);                        \
  if (GPT > 2) {                                            \
    stg2 = kgran((b), 2);                                   \
    stg3 = kgran((b), 3);                                   \
  }
#define APT_LOAD_V(b)                                       \
  stg0 = vgran((b), 0);                                     \
  if (GPT > 1) stg1 = vgran((b), 1);                        \
  if (GPT > 2) {                                            \
    stg2 = vgran((b), 2);                                   \
    stg3 = vgran((b), 3);                                   \
  }
#define APT_PUT()                                           \
  kb[tid] = stg0;                                           \
  if (GPT > 1) kb[tid + NT] = stg1;                         \
  if (GPT > 2) {                                            \
    kb[tid + 2 * NT] = stg2;                                \
    kb[tid + 3 * NT] = stg3;                                \
  }
  static_assert(GPT == 1 || GPT == 2 || GPT == 4, "staging registers");
  APT_LOAD_K(0)
  // the q tile, transposed: qs[d][r]
  for (int i = tid; i < APT_R * HD; i += NT) {
    const int r = i / HD, d = i % HD;
    const int t = row_tok(r);
    const bool ok = r / TQ < rep && t < T;
    qs[d * APT_R + r] = ok ? qrot[(size_t)t * n_heads * HD + (size_t)row_head(r) * HD + d] : 0.0f;
  }
  APT_PUT()
  __syncthreads();
  const int rg = tid >> 5, pg = tid & 31;  // rows RPT rg .. +RPT-1, block positions 4pg .. 4pg+3
  int pr[RPT];
#pragma unroll
  for (int i = 0; i < RPT; ++i) pr[i] = prow[RPT * rg + i];
  auto scw = [&](int i, int b) { return reinterpret_cast<float4*>(sc + (size_t)(RPT * rg + i) * pitch + b * APT_PB) + pg; };
  // the q values of this thread's RPT rows for dim d (one LDS read)
  auto qrows = [&](int d, float (&qv)[RPT]) {
    if constexpr (RPT == 4) {
      const float4 q4 = reinterpret_cast<const float4*>(qs + d * APT_R)[rg];
      qv[0] = q4.x;
      qv[1] = q4.y;
      qv[2] = q4.z;
      qv[3] = q4.w;
    } else {
      const float2 q2 = reinterpret_cast<const float2*>(qs + d * APT_R)[rg];
      qv[0] = q2.x;
      qv[1] = q2.y;
    }
  };
  // ---- A: scores and row maxima
  float rmax[RPT];
#pragma unroll
  for (int i = 0; i < RPT; ++i) rmax[i] = -INFINITY;
  for (int b = 0; b < nblk; ++b) {
    if (b + 1 < nblk) {
      APT_LOAD_K(b + 1)
    }
    float acc[RPT][4];
#pragma unroll
    for (int i = 0; i < RPT; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = 0.0f;
    for (int u = 0; u < R8; ++u) {
      uint4 k4[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) k4[j] = kb[u * APT_PB + 4 * pg + j];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        float qv[RPT];
        qrows(8 * u + e, qv);
#pragma unroll
        for (int i = 0; i < RPT; ++i)
#pragma unroll
          for (int j = 0; j < 4; ++j) acc[i][j] += mul_gran(qv[i], k4[j], e);
      }
    }
    const int p0 = b * APT_PB + 4 * pg;
#pragma unroll
    for (int i = 0; i < RPT; ++i) {
      float sv[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        sv[j] = acc[i][j] * scale;
        if (p0 + j < pr[i]) rmax[i] = fmaxf(rmax[i], sv[j]);
      }
      if (pr[i] > p0) *scw(i, b) = make_float4(sv[0], sv[1], sv[2], sv[3]);
    }
    __syncthreads();  // every wave is done with this block's K
    if (b + 1 < nblk) {
      APT_PUT()
    }
    __syncthreads();
  }
  APT_LOAD_V(0)  // (the first V block streams during the softmax)
  // row maxima over the 32 threads of a row group (lanes 32 rg' .. 32 rg' + 31 of a wave)
#pragma unroll
  for (int i = 0; i < RPT; ++i) {
#pragma unroll
    for (int o = 16; o >= 1; o >>= 1) rmax[i] = fmaxf(rmax[i], __shfl_xor(rmax[i], o));
    if (pg == 0) mrow[RPT * rg + i] = rmax[i];
  }
  __syncthreads();
  float m[RPT];
#pragma unroll
  for (int i = 0; i < RPT; ++i) m[i] = mrow[RPT * rg + i];
  // ---- B: exponentials (over the scores in the scratch), each row's sum in position order
  float sum = 0.0f;
  float4 snext[RPT];
#pragma unroll
  for (int i = 0; i < RPT; ++i) snext[i] = pr[i] > 4 * pg ? *scw(i, 0) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  for (int b = 0; b < nblk; ++b) {
    const int p0 = b * APT_PB + 4 * pg;
    float4 scur[RPT];
#pragma unroll
    for (int i = 0; i < RPT; ++i) scur[i] = snext[i];
    if (b + 1 < nblk) {
#pragma unroll
      for (int i = 0; i < RPT; ++i) snext[i] = pr[i] > p0 + APT_PB ? *scw(i, b + 1) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
#pragma unroll
    for (int i = 0; i < RPT; ++i) {
      const float sv[4] = {scur[i].x, scur[i].y, scur[i].z, scur[i].w};
      float ev[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) ev[j] = p0 + j < pr[i] ? glibc_expf(sv[j] - m[i]) : 0.0f;
      const float4 e4 = make_float4(ev[0], ev[1], ev[2], ev[3]);
      reinterpret_cast<float4*>(eb + (RPT * rg + i) * APT_ES)[pg] = e4;
      if (pr[i] > p0) *scw(i, b) = e4;
    }
    __syncthreads();
    if (tid < APT_R) {
      const float* er = eb + tid * APT_ES;
#pragma unroll 8
      for (int p = 0; p < APT_PB; ++p) sum += er[p];
    }
    __syncthreads();
  }
  if (tid < APT_R) irow[tid] = 1.0f / sum;
  APT_PUT()  // the first V block
  __syncthreads();
  float inv[RPT];
#pragma unroll
  for (int i = 0; i < RPT; ++i) inv[i] = irow[RPT * rg + i];
  // ---- C: output sums
  const int dgi = tid & 31;  // dims DB*dgi .. +DB-1 of rows RPT rg ..
  float o[RPT][DB];
#pragma unroll
  for (int i = 0; i < RPT; ++i)
#pragma unroll
    for (int k = 0; k < DB; ++k) o[i][k] = 0.0f;
#pragma unroll
  for (int i = 0; i < RPT; ++i) snext[i] = pr[i] > 4 * pg ? *scw(i, 0) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  for (int b = 0; b < nblk; ++b) {
    const int pb = b * APT_PB, p0 = pb + 4 * pg;
    if (b + 1 < nblk) {
      APT_LOAD_V(b + 1)
    }
    float4 ecur[RPT];
#pragma unroll
    for (int i = 0; i < RPT; ++i) ecur[i] = snext[i];
    if (b + 1 < nblk) {
#pragma unroll
      for (int i = 0; i < RPT; ++i) snext[i] = pr[i] > p0 + APT_PB ? *scw(i, b + 1) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
#pragma unroll
    for (int i = 0; i < RPT; ++i) {
      const float ev[4] = {ecur[i].x, ecur[i].y, ecur[i].z, ecur[i].w};
      float pv[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) pv[j] = p0 + j < pr[i] ? ev[j] * inv[i] : 0.0f;
      reinterpret_cast<float4*>(eb + (RPT * rg + i) * APT_ES)[pg] = make_float4(pv[0], pv[1], pv[2], pv[3]);
    }
    __syncthreads();
    const bool masked = pb + APT_PB > pmin;  // a row of the tile ends inside this block
#pragma unroll 1
    for (int gq = 0; gq < APT_PB / 8; ++gq) {
      uint4 v[DB];
#pragma unroll
      for (int k = 0; k < DB; ++k) v[k] = kb[gq * HD + DB * dgi + k];
      float pp[RPT][8];
#pragma unroll
      for (int i = 0; i < RPT; ++i) {
        const float4 a = reinterpret_cast<const float4*>(eb + (RPT * rg + i) * APT_ES + 8 * gq)[0];
        const float4 c = reinterpret_cast<const float4*>(eb + (RPT * rg + i) * APT_ES + 8 * gq)[1];
        pp[i][0] = a.x; pp[i][1] = a.y; pp[i][2] = a.z; pp[i][3] = a.w;
        pp[i][4] = c.x; pp[i][5] = c.y; pp[i][6] = c.z; pp[i][7] = c.w;
      }
      if (!masked) {
#pragma unroll
        for (int e = 0; e < 8; ++e)
#pragma unroll
          for (int i = 0; i < RPT; ++i)
#pragma unroll
            for (int k = 0; k < DB; ++k) o[i][k] += mul_gran(pp[i][e], v[k], e);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int p = pb + 8 * gq + e;
#pragma unroll
          for (int i = 0; i < RPT; ++i)
#pragma unroll
            for (int k = 0; k < DB; ++k) {
              const float t = mul_gran(pp[i][e], v[k], e);
              if (p < pr[i]) o[i][k] += t;
            }
        }
      }
    }
    __syncthreads();  // every wave is done with this block's V and probabilities
    if (b + 1 < nblk) {
      APT_PUT()
    }
    // (the next block's probabilities are written after this barrier's successor)
  }
  __syncthreads();
  // ---- outputs: rows to LDS (reusing the q tile), then one (row, 32-value block) per thread
  float* os = qs;  // [64][HD]
#pragma unroll
  for (int i = 0; i < RPT; ++i) {
    const int r = RPT * rg + i;
#pragma unroll
    for (int k = 0; k < DB; ++k) {
      const int d = DB * dgi + k;
      // a single position copies the V row (its bits, -0 included)
      os[r * HD + d] = pr[i] == 1 ? half_bits_to_float(vc[hbase + kv_v_index(HD, 0, d)]) : o[i][k];
    }
  }
  __syncthreads();
  for (int i = tid; i < APT_R * (HD / 32); i += NT) {
    const int r = i / (HD / 32), blk = i % (HD / 32);
    if (prow[r] == 0) continue;
    float y[32];
#pragma unroll
    for (int e = 0; e < 32; ++e) y[e] = os[r * HD + 32 * blk + e];
    const size_t o0 = (size_t)row_tok(r) * n_heads * HD + (size_t)row_head(r) * HD + 32 * blk;
    if (att_out) {
#pragma unroll
      for (int e = 0; e < 32; e += 4)
        *reinterpret_cast<float4*>(att_out + o0 + e) = make_float4(y[e], y[e + 1], y[e + 2], y[e + 3]);
    }
    uint32_t packed[8];
    xs[o0 >> 5] = quantize_block_regs(y, packed);
    uint4* qp = reinterpret_cast<uint4*>(xq + o0);
    qp[0] = make_uint4(packed[0], packed[1], packed[2], packed[3]);
    qp[1] = make_uint4(packed[4], packed[5], packed[6], packed[7]);
  }
#undef APT_LOAD_K
#undef APT_LOAD_V
#undef APT_PUT
}

// ---------------------------------------------------------------------------
// SwiGLU + Q8_0 quantization of T rows (silu_mul_quantize, cuda_resident.rs:1315; CPU
// tensor/mod.rs:1943-1967).  Row t of gu holds 2F values: [gate | up], or, interleaved,
// groups of 32 gate values followed by the matching 32 up values.  grid (ceil(F/256), T).
__global__ __launch_bounds__(256) void k_silu_rows(const float* __restrict__ gu, int F, int interleaved,
                                                   int8_t* __restrict__ xq, float* __restrict__ xs) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i >= F) return;  // uniform per 32-lane group (F % 32 == 0)
  const size_t t = blockIdx.y;
  const float* r = gu + t * 2 * (size_t)F;
  const int gi = interleaved ? (i >> 5) * 64 + (i & 31) : i;
  const int ui = interleaved ? gi + 32 : F + i;
  const float a = silu_mul1(r[gi], r[ui]);
  int8_t q;
  const float d = quantize_lane32(a, &q);
  xq[t * F + i] = q;
  if ((i & 31) == 0) xs[(t * F + i) >> 5] = d;
}

}  // namespace cm
