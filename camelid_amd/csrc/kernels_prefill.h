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
// Workgroup: 4 waves over a 64-row x 64-token tile, each wave 32 x 32 (2 x 2 fragments).
// Lane l of a fragment supplies row / token l % 16, bytes 8*(l/16) .. +7 of the block, and
// receives the outputs of rows 4*(l/16) + i (i = 0..3) for token l % 16.
// Scales are staged in LDS for 32 blocks at a time (transposed: [block][row], [block][token]).
// Tiles are dealt so that each XCD (workgroup id mod 8) runs a contiguous range of tiles,
// token tiles innermost: the row tile's weights are read once per XCD and re-read from its L2.
// N % 4 == 0 (16-byte output stores); y may alias resid.
constexpr int GM_NT = 256;
constexpr int GM_RN = 64;  // rows per workgroup tile
constexpr int GM_RT = 64;  // tokens per workgroup tile
constexpr int GM_BG = 32;  // blocks per scale-staging group
constexpr int GM_PD = 4;   // operand prefetch distance, blocks

__host__ __device__ inline int gemm_tiles(int N, int T) {
  return ((N + GM_RN - 1) / GM_RN) * ((T + GM_RT - 1) / GM_RT);
}
__host__ __device__ inline int gemm_grid(int N, int T) { return ((gemm_tiles(N, T) + 7) / 8) * 8; }

__global__ __launch_bounds__(GM_NT) void k_gemm_q8(const int8_t* __restrict__ wq, const uint16_t* __restrict__ wd,
                                                   int N, int K, const int8_t* __restrict__ xq,
                                                   const float* __restrict__ xs, int T, float* y,
                                                   const float* resid) {
  __shared__ __align__(16) uint16_t swd[GM_BG][GM_RN + 4];
  __shared__ __align__(16) float sxs[GM_BG][GM_RT + 1];
  const int NB = K >> 5;
  const int ntt = (T + GM_RT - 1) / GM_RT;
  const int tiles = gemm_tiles(N, T);
  const int per = (tiles + 7) >> 3;
  const int L = (int)(blockIdx.x & 7) * per + (int)(blockIdx.x >> 3);
  if (L >= tiles) return;
  const int n_base = (L / ntt) * GM_RN, t_base = (L % ntt) * GM_RT;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int r = lane & 15, g = lane >> 4;
  const int wn = (wave & 1) * 32, wt = (wave >> 1) * 32;
  const int8_t* ap[2];
  const int8_t* bp[2];
#pragma unroll
  for (int f = 0; f < 2; ++f) {
    ap[f] = wq + (size_t)min(n_base + wn + 16 * f + r, N - 1) * K + 8 * g;
    bp[f] = xq + (size_t)min(t_base + wt + 16 * f + r, T - 1) * K + 8 * g;
  }
  float acc[2][2][4];
#pragma unroll
  for (int nf = 0; nf < 2; ++nf)
#pragma unroll
    for (int tf = 0; tf < 2; ++tf)
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[nf][tf][i] = 0.0f;
  long av[GM_PD][2], bv[GM_PD][2];
  auto load = [&](int s, int b) {  // operands of block b (clamped) into slot s
    const int bb = min(b, NB - 1) * 32;
#pragma unroll
    for (int f = 0; f < 2; ++f) {
      av[s][f] = *reinterpret_cast<const long*>(ap[f] + bb);
      bv[s][f] = *reinterpret_cast<const long*>(bp[f] + bb);
    }
  };
#pragma unroll
  for (int s = 0; s < GM_PD; ++s) load(s, s);
  for (int b0 = 0; b0 < NB; b0 += GM_PD) {
    if (b0 % GM_BG == 0) {
      __syncthreads();  // the previous group's scales are consumed
      for (int e = tid; e < GM_BG * GM_RN; e += GM_NT) {
        const int row = e / GM_BG, bb = e % GM_BG;
        const int blk = min(b0 + bb, NB - 1);
        swd[bb][row] = wd[(size_t)min(n_base + row, N - 1) * NB + blk];
      }
      for (int e = tid; e < GM_BG * GM_RT; e += GM_NT) {
        const int tok = e / GM_BG, bb = e % GM_BG;
        const int blk = min(b0 + bb, NB - 1);
        sxs[bb][tok] = xs[(size_t)min(t_base + tok, T - 1) * NB + blk];
      }
      __syncthreads();
    }
#pragma unroll
    for (int s = 0; s < GM_PD; ++s) {
      const int b = b0 + s;
      if (b < NB) {
        v4i_t c[2][2];
#pragma unroll
        for (int nf = 0; nf < 2; ++nf)
#pragma unroll
          for (int tf = 0; tf < 2; ++tf)
            c[nf][tf] = __builtin_amdgcn_mfma_i32_16x16x32_i8(av[s][nf], bv[s][tf], v4i_t{0, 0, 0, 0}, 0, 0, 0);
        load(s, b + GM_PD);
        const int bl = b % GM_BG;
        uint2 w2[2];
        float xv[2];
#pragma unroll
        for (int nf = 0; nf < 2; ++nf) w2[nf] = *reinterpret_cast<const uint2*>(&swd[bl][wn + 16 * nf + 4 * g]);
#pragma unroll
        for (int tf = 0; tf < 2; ++tf) xv[tf] = sxs[bl][wt + 16 * tf + r];
#pragma unroll
        for (int nf = 0; nf < 2; ++nf)
#pragma unroll
          for (int tf = 0; tf < 2; ++tf) {
            acc[nf][tf][0] += mul_f16_lo((float)c[nf][tf][0], w2[nf].x) * xv[tf];
            acc[nf][tf][1] += mul_f16_hi((float)c[nf][tf][1], w2[nf].x) * xv[tf];
            acc[nf][tf][2] += mul_f16_lo((float)c[nf][tf][2], w2[nf].y) * xv[tf];
            acc[nf][tf][3] += mul_f16_hi((float)c[nf][tf][3], w2[nf].y) * xv[tf];
          }
      }
    }
  }
#pragma unroll
  for (int nf = 0; nf < 2; ++nf)
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
                                                        const uint16_t* __restrict__ kc, const float* __restrict__ vc,
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
  const float4* vg = reinterpret_cast<const float4*>(vc + hbase);
  const size_t row = (size_t)t * n_heads * HD + (size_t)h * HD;
  if (tid < HD) qs[tid] = qrot[row + tid];
  __syncthreads();
  float o = 0.0f;
  if (P == 1) {
    if (tid < HD) o = vc[hbase + kv_v_index(HD, 0, tid)];
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
      const int ng = P >> 2;
      const float4* pr4 = reinterpret_cast<const float4*>(sc);
      float a = 0.0f;
      int j = 0;
      for (; j + 8 <= ng; j += 8) {
        float4 v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) v[u] = vg[(size_t)(j + u) * HD + tid];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const float4 pr = pr4[j + u];
          a += pr.x * v[u].x;
          a += pr.y * v[u].y;
          a += pr.z * v[u].z;
          a += pr.w * v[u].w;
        }
      }
      for (; j < ng; ++j) {
        const float4 v = vg[(size_t)j * HD + tid];
        const float4 pr = pr4[j];
        a += pr.x * v.x;
        a += pr.y * v.y;
        a += pr.z * v.z;
        a += pr.w * v.w;
      }
      for (int p = ng * 4; p < P; ++p) a += sc[p] * vc[hbase + kv_v_index(HD, p, tid)];
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
