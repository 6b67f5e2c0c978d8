// kernels_decode.h -- HIP/CDNA4 kernels of the resident decode step (gfx950, wave64).
//
// Bit-exactness contract: every f32 value that reaches a Q8_0 quantizer, the KV
// cache or the argmax is produced by the same sequence of IEEE f32 operations as
// Camelid's CPU path.  Integer work (int8 dot4) is reassociated freely (exact);
// f32 reductions are folded in the CPU's order by one lane per output.
//
// Weight layout in HBM ("Q8R", repacked from the 34-byte GGUF Q8_0 wire blocks):
//   quants: int8 [rows][K] row-major, 16-byte aligned rows (K % 32 == 0)
//   scales: f16 bits [rows][K/32]
// Total bytes = rows*K*34/32, the same as the wire format; the split keeps every
// wavefront load a 16-byte-aligned, fully coalesced dwordx4.
#pragma once
#include <hip/hip_runtime.h>
#include "device_math.h"

namespace cm {

__device__ __forceinline__ float half_bits_to_float(uint16_t b) {
  _Float16 h;
  __builtin_memcpy(&h, &b, 2);
  return (float)h;  // v_cvt_f32_f16: exact widening (f16 denormals are enabled on gfx9)
}

__device__ __forceinline__ int dot4x4(int4 w, int4 x, int acc) {
  acc = __builtin_amdgcn_sdot4(w.x, x.x, acc, false);
  acc = __builtin_amdgcn_sdot4(w.y, x.y, acc, false);
  acc = __builtin_amdgcn_sdot4(w.z, x.z, acc, false);
  acc = __builtin_amdgcn_sdot4(w.w, x.w, acc, false);
  return acc;
}

// Exact int32 dot of one 32-value block, split over a lane pair: each lane of the pair
// holds one 16-byte half (chunk c = 2*block + (lane & 1)); the pair sum is returned to both.
__device__ __forceinline__ int pair_block_dot(const int4* w4, const int4* x4, int c) {
  int s = dot4x4(w4[c], x4[c], 0);
  return s + __shfl_xor(s, 1);
}

// Per-(row, block) int32 dots through the GEMV's own dot path (test hook).
// grid = rows, block = 64.
__global__ __launch_bounds__(64) void k_q8_block_dots(const int8_t* __restrict__ wq, int K,
                                                      const int8_t* __restrict__ xq, int32_t* __restrict__ out) {
  const int row = blockIdx.x, lane = threadIdx.x;
  const int4* w4 = reinterpret_cast<const int4*>(wq + (size_t)row * K);
  const int4* x4 = reinterpret_cast<const int4*>(xq);
  for (int c = lane; c < (K >> 4); c += 64) {
    const int s = pair_block_dot(w4, x4, c);
    if ((lane & 1) == 0) out[(size_t)row * (K >> 5) + (c >> 1)] = s;
  }
}

// ---------------------------------------------------------------------------
// Q8_0 GEMV, faithful.  y[row] = (resid ? resid[row] : 0) + fold_b term(row, b),
//   term = (float(int_dot(w_b, x_b)) * w_scale_b) * x_scale_b   (inference.rs:19871-19905)
// Each wave owns RW rows.  Lanes stream a row's quants as 16-byte chunks (two lanes per
// 32-value block, combined with a lane-pair shuffle: integer, exact), write the per-block
// f32 terms to LDS, then lane r folds row r's terms in block order.
// grid = ceil(rows / (4*RW)), block = 256, dynamic LDS = 4*RW*(nb+1)*4 bytes.
template <int RW>
__global__ __launch_bounds__(256) void k_q8_gemv(const int8_t* __restrict__ wq,
                                                 const uint16_t* __restrict__ wd, int rows, int K,
                                                 const int8_t* __restrict__ xq,
                                                 const float* __restrict__ xs,
                                                 float* y, const float* resid) {
  extern __shared__ float lds[];
  const int nb = K >> 5;
  const int nchunk = K >> 4;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int row0 = (blockIdx.x * 4 + wave) * RW;
  float* t = lds + wave * RW * (nb + 1);
  const int4* x4 = reinterpret_cast<const int4*>(xq);
#pragma unroll
  for (int r = 0; r < RW; ++r) {
    const int row = min(row0 + r, rows - 1);  // clamped: uniform control flow, result discarded
    const int4* w4 = reinterpret_cast<const int4*>(wq + (size_t)row * K);
    const uint16_t* d = wd + (size_t)row * nb;
    for (int c = lane; c < nchunk; c += 64) {
      const int s = pair_block_dot(w4, x4, c);
      if ((lane & 1) == 0) {
        const int b = c >> 1;
        t[r * (nb + 1) + b] = ((float)s * half_bits_to_float(d[b])) * xs[b];
      }
    }
  }
  __syncthreads();
  if (lane < RW) {
    const int row = row0 + lane;
    if (row < rows) {
      const float* tr = t + lane * (nb + 1);
      float acc = 0.0f;
      for (int b = 0; b < nb; ++b) acc += tr[b];
      y[row] = resid ? resid[row] + acc : acc;
    }
  }
}

// ---------------------------------------------------------------------------
// Block reductions (exact: max / argmax only).
__device__ __forceinline__ float block_max(float v, float* red) {
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, nw = blockDim.x >> 6;
  __syncthreads();
  if (lane == 0) red[wave] = v;
  __syncthreads();
  float m = red[0];
  for (int i = 1; i < nw; ++i) m = fmaxf(m, red[i]);
  return m;
}

// Quantize `n` (multiple of 32) f32 values in LDS to Q8_0, one thread per block.
__device__ __forceinline__ void quantize_blocks_from_lds(const float* v, int n, int8_t* xq, float* xs) {
  for (int b = threadIdx.x; b < (n >> 5); b += blockDim.x) {
    int8_t q[32];
    xs[b] = quantize_q8_0_block(v + b * 32, q);
    int4* dst = reinterpret_cast<int4*>(xq + b * 32);
    const int4* src = reinterpret_cast<const int4*>(q);
    dst[0] = src[0];
    dst[1] = src[1];
  }
}

// Sequential f32 sum of LDS values 0..n-1 (one thread), the CPU's fold order.
__device__ __forceinline__ float serial_sum_lds(const float* v, int n) {
  float acc = 0.0f;
  int i = 0;
  for (; i + 8 <= n; i += 8) {
    const float4 a = *reinterpret_cast<const float4*>(v + i);
    const float4 b = *reinterpret_cast<const float4*>(v + i + 4);
    acc += a.x; acc += a.y; acc += a.z; acc += a.w;
    acc += b.x; acc += b.y; acc += b.z; acc += b.w;
  }
  for (; i < n; ++i) acc += v[i];
  return acc;
}

// ---------------------------------------------------------------------------
// RMSNorm (tensor/mod.rs:2083-2106) fused with Q8_0 quantization of the result.
// One workgroup; squares in parallel, the sum of squares folded serially by thread 0.
// Dynamic LDS = n*4 bytes (n % 32 == 0).
__global__ __launch_bounds__(1024) void k_rmsnorm_quant(const float* __restrict__ x,
                                                        const float* __restrict__ w, int n, float eps,
                                                        int8_t* __restrict__ xq, float* __restrict__ xs,
                                                        float* __restrict__ y_out) {
  extern __shared__ float s[];
  __shared__ float s_scale;
  for (int i = threadIdx.x; i < n; i += blockDim.x) {
    const float v = x[i];
    s[i] = v * v;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    const float ms = serial_sum_lds(s, n) / (float)n;
    s_scale = 1.0f / sqrtf(ms + eps);
  }
  __syncthreads();
  const float scale = s_scale;
  for (int i = threadIdx.x; i < n; i += blockDim.x) {
    const float yv = (x[i] * scale) * w[i];
    s[i] = yv;
    if (y_out) y_out[i] = yv;
  }
  __syncthreads();
  quantize_blocks_from_lds(s, n, xq, xs);
}

// Plain Q8_0 quantization of an f32 vector, one thread per block.
__global__ void k_quantize_q8_0(const float* __restrict__ x, int n, int8_t* __restrict__ xq,
                                float* __restrict__ xs) {
  const int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= (n >> 5)) return;
  float v[32];
  for (int i = 0; i < 32; ++i) v[i] = x[b * 32 + i];
  int8_t q[32];
  xs[b] = quantize_q8_0_block(v, q);
  int4* dst = reinterpret_cast<int4*>(xq + b * 32);
  const int4* src = reinterpret_cast<const int4*>(q);
  dst[0] = src[0];
  dst[1] = src[1];
}

// SwiGLU + Q8_0 quantization.  gate = gu[0..n), up = gu[n..2n); one thread per block.
__global__ void k_silu_mul_quant(const float* __restrict__ gu, int n, int8_t* __restrict__ xq,
                                 float* __restrict__ xs, float* __restrict__ act_out) {
  const int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= (n >> 5)) return;
  float v[32];
  for (int i = 0; i < 32; ++i) {
    v[i] = silu_mul1(gu[b * 32 + i], gu[n + b * 32 + i]);
    if (act_out) act_out[b * 32 + i] = v[i];
  }
  int8_t q[32];
  xs[b] = quantize_q8_0_block(v, q);
  int4* dst = reinterpret_cast<int4*>(xq + b * 32);
  const int4* src = reinterpret_cast<const int4*>(q);
  dst[0] = src[0];
  dst[1] = src[1];
}

// ---------------------------------------------------------------------------
// Per-head QK RMSNorm (optional) + RoPE + f16 KV store for the token at *d_pos.
// One workgroup per head: blocks [0, n_heads) are Q heads, [n_heads, n_heads+n_kv) K heads
// (which also store that head's V row).  qkv = [q | k | v] rows of the fused projection.
// RoPE math: rope.rs:489-524; f16 store: kv_cache.rs:573-600 (layout [L][n_kv][max_pos][hd]).
__global__ __launch_bounds__(128) void k_rope_kv(const float* __restrict__ qkv, int n_heads, int n_kv,
                                                 int hd, int rope_dim, int split_half,
                                                 const float* __restrict__ cosv,
                                                 const float* __restrict__ sinv,
                                                 const float* __restrict__ q_norm,
                                                 const float* __restrict__ k_norm, float eps,
                                                 float* __restrict__ qrot, uint16_t* __restrict__ kc,
                                                 uint16_t* __restrict__ vc, int layer, int max_pos,
                                                 const uint32_t* __restrict__ d_pos) {
  __shared__ float buf[512];
  __shared__ float sq[512];
  __shared__ float s_scale;
  const int h = blockIdx.x;
  const bool isq = h < n_heads;
  const float* src = isq ? qkv + (size_t)h * hd : qkv + (size_t)n_heads * hd + (size_t)(h - n_heads) * hd;
  for (int d = threadIdx.x; d < hd; d += blockDim.x) buf[d] = src[d];
  const float* nw = isq ? q_norm : k_norm;
  if (nw) {
    __syncthreads();
    for (int d = threadIdx.x; d < hd; d += blockDim.x) sq[d] = buf[d] * buf[d];
    __syncthreads();
    if (threadIdx.x == 0) {
      const float ms = serial_sum_lds(sq, hd) / (float)hd;
      s_scale = 1.0f / sqrtf(ms + eps);
    }
    __syncthreads();
    for (int d = threadIdx.x; d < hd; d += blockDim.x) buf[d] = (buf[d] * s_scale) * nw[d];
  }
  __syncthreads();
  const int half = rope_dim >> 1;
  for (int p = threadIdx.x; p < half; p += blockDim.x) {
    const int d0 = split_half ? p : 2 * p;
    const int d1 = split_half ? p + half : 2 * p + 1;
    const float c = cosv[p], s = sinv[p];
    const float x0 = buf[d0], x1 = buf[d1];
    buf[d0] = (x0 * c) - (x1 * s);
    buf[d1] = (x0 * s) + (x1 * c);
  }
  __syncthreads();
  if (isq) {
    for (int d = threadIdx.x; d < hd; d += blockDim.x) qrot[(size_t)h * hd + d] = buf[d];
  } else {
    const int kvh = h - n_heads;
    const size_t dst = (((size_t)layer * n_kv + kvh) * max_pos + *d_pos) * hd;
    const float* vsrc = qkv + (size_t)(n_heads + n_kv) * hd + (size_t)kvh * hd;
    for (int d = threadIdx.x; d < hd; d += blockDim.x) {
      kc[dst + d] = f32_to_f16_bits(buf[d]);
      vc[dst + d] = f32_to_f16_bits(vsrc[d]);
    }
  }
}

// ---------------------------------------------------------------------------
// Decode attention, faithful (inference.rs:23945-24025), one workgroup per query head:
//   score_p = dot_seq(q, k_p) * scale           (one thread per position, d in order)
//   m = max_p score_p                           (exact)
//   e_p = expf(score_p - m); sum = fold_p e_p   (serial fold by thread 0)
//   out_d = fold_p (e_p * (1/sum)) * v_pd       (one thread per d, p in order)
// The head's output is then quantized to Q8_0 (hd % 32 == 0: blocks never straddle heads).
// Dynamic LDS = (max_pos + hd) * 4 bytes.
__global__ __launch_bounds__(256) void k_attn_decode(const float* __restrict__ qrot,
                                                     const uint16_t* __restrict__ kc,
                                                     const uint16_t* __restrict__ vc, int layer,
                                                     int n_heads, int n_kv, int hd, int max_pos,
                                                     const uint32_t* __restrict__ d_pos, float scale,
                                                     float* __restrict__ att_out,
                                                     int8_t* __restrict__ xq, float* __restrict__ xs) {
  extern __shared__ float sm[];
  __shared__ float qs[512];
  __shared__ float red[16];
  __shared__ float s_inv;
  float* out = sm;        // [hd]
  float* sc = sm + hd;    // [P]
  const int h = blockIdx.x;
  const int kvh = h / (n_heads / n_kv);
  const int P = (int)*d_pos + 1;
  const size_t base = (((size_t)layer * n_kv + kvh) * max_pos) * hd;
  for (int d = threadIdx.x; d < hd; d += blockDim.x) qs[d] = qrot[(size_t)h * hd + d];
  __syncthreads();
  if (P == 1) {
    // inference.rs:23564-23575: a single position copies the V row.
    for (int d = threadIdx.x; d < hd; d += blockDim.x) out[d] = half_bits_to_float(vc[base + d]);
  } else {
    float lmax = -INFINITY;
    for (int p = threadIdx.x; p < P; p += blockDim.x) {
      const uint16_t* kr = kc + base + (size_t)p * hd;
      float acc = 0.0f;
      for (int d = 0; d < hd; d += 8) {
        const uint4 raw = *reinterpret_cast<const uint4*>(kr + d);
        const uint32_t wv[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          acc += qs[d + 2 * j] * half_bits_to_float((uint16_t)(wv[j] & 0xffffu));
          acc += qs[d + 2 * j + 1] * half_bits_to_float((uint16_t)(wv[j] >> 16));
        }
      }
      const float s = acc * scale;
      sc[p] = s;
      lmax = fmaxf(lmax, s);
    }
    const float mx = block_max(lmax, red);
    for (int p = threadIdx.x; p < P; p += blockDim.x) sc[p] = glibc_expf(sc[p] - mx);
    __syncthreads();
    if (threadIdx.x == 0) s_inv = 1.0f / serial_sum_lds(sc, P);
    __syncthreads();
    const float inv = s_inv;
    for (int p = threadIdx.x; p < P; p += blockDim.x) sc[p] = sc[p] * inv;
    __syncthreads();
    for (int d = threadIdx.x; d < hd; d += blockDim.x) {
      const uint16_t* vcol = vc + base + d;
      float acc = 0.0f;
      for (int p = 0; p < P; ++p) acc += sc[p] * half_bits_to_float(vcol[(size_t)p * hd]);
      out[d] = acc;
    }
  }
  __syncthreads();
  for (int d = threadIdx.x; d < hd; d += blockDim.x) att_out[(size_t)h * hd + d] = out[d];
  quantize_blocks_from_lds(out, hd, xq + (size_t)h * hd, xs + (size_t)h * (hd >> 5));
}

// ---------------------------------------------------------------------------
// Greedy argmax (inference.rs:5912-5925): first index of the maximum, strict '>'.
__global__ __launch_bounds__(1024) void k_argmax(const float* __restrict__ x, int n,
                                                 uint32_t* __restrict__ out) {
  __shared__ float bv_s[16];
  __shared__ uint32_t bi_s[16];
  float bv = -INFINITY;
  uint32_t bi = 0xffffffffu;
  for (int i = threadIdx.x; i < n; i += blockDim.x) {
    const float v = x[i];
    if (v > bv) { bv = v; bi = (uint32_t)i; }
  }
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(bv, o);
    const uint32_t oi = __shfl_xor(bi, o);
    if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
  }
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  if (lane == 0) { bv_s[wave] = bv; bi_s[wave] = bi; }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < (int)(blockDim.x >> 6); ++w) {
      if (bv_s[w] > bv || (bv_s[w] == bv && bi_s[w] < bi)) { bv = bv_s[w]; bi = bi_s[w]; }
    }
    *out = bi == 0xffffffffu ? 0u : bi;
  }
}

// On-device Q8R embedding row gather: h[i] = scale_b * q_i (exact; tensor/mod.rs:2329-2398).
__global__ void k_embed_q8(const int8_t* __restrict__ eq, const uint16_t* __restrict__ ed, int H,
                           const uint32_t* __restrict__ tok, float* __restrict__ h) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= H) return;
  const size_t t = *tok;
  h[i] = half_bits_to_float(ed[t * (H >> 5) + (i >> 5)]) * (float)eq[t * H + i];
}

// glibc-identical expf over a vector (test hook).
__global__ void k_expf(const float* __restrict__ x, float* __restrict__ y, size_t n) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) y[i] = glibc_expf(x[i]);
}

}  // namespace cm
