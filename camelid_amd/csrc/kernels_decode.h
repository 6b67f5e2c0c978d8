// kernels_decode.h -- HIP/CDNA4 kernels of the resident decode step (gfx950, wave64).
//
// Bit-exactness contract: every f32 value that reaches a Q8_0 quantizer, the KV cache or
// the argmax is produced by the same sequence of IEEE f32 operations as Camelid's CPU
// path.  Integer work (int8 dot4) and max/argmax are reassociated freely (exact); every
// f32 sum is folded in the CPU's order by one lane per output.
//
// Weight layout in HBM ("Q8R", repacked from the 34-byte GGUF Q8_0 wire blocks):
//   quants: int8 [rows][K] row-major (K % 32 == 0), so R consecutive rows are one
//           contiguous R*K-byte slab
//   scales: f16 bits [rows][K/32]
// Total bytes = rows*K*34/32, the same as the wire format; the split makes every
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

// ---------------------------------------------------------------------------
// Serial f32 fold of n LDS floats in index order (one lane), the CPU's summation order.
// LDS reads run W float4 groups ahead of the dependent add chain so the chain issues
// back to back.  p must be 16-byte aligned.
template <int W = 8>
__device__ __forceinline__ float fold_lds(const float* p, int n, float acc = 0.0f) {
  const float4* q = reinterpret_cast<const float4*>(p);
  const int g = n >> 2;
  float4 buf[W];
#pragma unroll
  for (int i = 0; i < W; ++i)
    if (i < g) buf[i] = q[i];
  for (int base = 0; base < g; base += W) {
#pragma unroll
    for (int i = 0; i < W; ++i) {
      if (base + i < g) {
        const float4 v = buf[i];
        if (base + i + W < g) buf[i] = q[base + i + W];
        acc += v.x;
        acc += v.y;
        acc += v.z;
        acc += v.w;
      }
    }
  }
  for (int i = g << 2; i < n; ++i) acc += p[i];
  return acc;
}

// Q8_0 quantization of one 32-value block held one value per lane by a 32-lane group
// (lanes 0-31 or 32-63 of a wave).  Returns the block's f16-valued scale (same in every
// lane); *q receives this lane's quant.  inference.rs:16953-16971.
__device__ __forceinline__ float quantize_lane32(float v, int8_t* q) {
  float amax = fabsf(v);
#pragma unroll
  for (int o = 16; o > 0; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o));
  const float unrounded = amax / 127.0f;
  const float scale = f16_bits_to_f32(f32_to_f16_bits(unrounded));
  const float inv = unrounded == 0.0f ? 0.0f : 1.0f / unrounded;
  float r = roundf(v * inv);
  r = fminf(fmaxf(r, -128.0f), 127.0f);
  *q = (int8_t)r;
  return scale;
}

__device__ __forceinline__ float block_max(float v, float* red) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, nw = blockDim.x >> 6;
  __syncthreads();
  if (lane == 0) red[wave] = v;
  __syncthreads();
  float m = red[0];
  for (int i = 1; i < nw; ++i) m = fmaxf(m, red[i]);
  return m;
}

// ---------------------------------------------------------------------------
// Per-(row, block) int32 dots (test hook for the bit-exact block-dot contract): the
// same lane-pair dot4 path as the GEMV.  grid = rows, block = 64.
__global__ __launch_bounds__(64) void k_q8_block_dots(const int8_t* __restrict__ wq, int K,
                                                      const int8_t* __restrict__ xq, int32_t* __restrict__ out) {
  const int row = blockIdx.x, lane = threadIdx.x;
  const int4* w4 = reinterpret_cast<const int4*>(wq + (size_t)row * K);
  const int4* x4 = reinterpret_cast<const int4*>(xq);
  for (int c = lane; c < (K >> 4); c += 64) {
    int s = dot4x4(w4[c], x4[c], 0);
    s += __shfl_xor(s, 1);
    if ((lane & 1) == 0) out[(size_t)row * (K >> 5) + (c >> 1)] = s;
  }
}

// ---------------------------------------------------------------------------
// Q8_0 GEMV, faithful:  y[row] = (resid ? resid[row] : 0) + fold_b term(row, b),
//   term = (float(int_dot(w_b, x_b)) * w_scale_b) * x_scale_b  (inference.rs:19871-19905).
// A workgroup of 256 threads owns GEMV_R consecutive rows = one contiguous slab of
// GEMV_R*K quant bytes.  The slab's 16-byte chunks are dealt round-robin (thread t takes
// chunks t, t+256, ...), so each workgroup-wide load is 4 KB contiguous.  Lane pairs
// (2j, 2j+1) always hold the two halves of one 32-value block (chunks per row is even),
// combined with one integer shuffle.  Even lanes turn the block dot into its f32 term in
// LDS; then lane r of wave 0 folds row r's terms in block order.
// Dynamic LDS: K bytes (x quants) + nb*4 (x scales) + GEMV_R*(nb+4)*4 (terms).
constexpr int GEMV_R = 8;
constexpr int GEMV_NT = 256;

__host__ __device__ inline int gemv_term_stride(int nb) { return ((nb + 3) & ~3) + 4; }
__host__ __device__ inline size_t gemv_term_offset(int K) { return ((size_t)K + (size_t)(K >> 5) * 4 + 15) & ~(size_t)15; }
__host__ __device__ inline size_t gemv_lds_bytes(int K) {
  return gemv_term_offset(K) + (size_t)GEMV_R * gemv_term_stride(K >> 5) * 4;
}

// Shared body; returns (in lanes 0..GEMV_R-1 of wave 0) the folded sum of row row0+lane.
__device__ __forceinline__ float gemv_rows(const int8_t* __restrict__ wq, const uint16_t* __restrict__ wd, int rows,
                                           int K, const int8_t* __restrict__ xq, const float* __restrict__ xs,
                                           int row0, unsigned char* smem) {
  const int nb = K >> 5;
  const int cpr = K >> 4;  // 16-byte chunks per row
  int8_t* xl = reinterpret_cast<int8_t*>(smem);
  float* xsl = reinterpret_cast<float*>(smem + K);
  float* t = reinterpret_cast<float*>(smem + gemv_term_offset(K));  // [GEMV_R][stride], 16-byte aligned rows
  const int tid = threadIdx.x;
  // stage the activation (K quants + nb scales) in LDS
  for (int c = tid; c < cpr; c += GEMV_NT)
    reinterpret_cast<int4*>(xl)[c] = reinterpret_cast<const int4*>(xq)[c];
  for (int b = tid; b < nb; b += GEMV_NT) xsl[b] = xs[b];
  __syncthreads();
  const int nrows = min(GEMV_R, rows - row0);
  const int total = nrows * cpr;
  const int4* slab = reinterpret_cast<const int4*>(wq + (size_t)row0 * K);
  const uint16_t* dslab = wd + (size_t)row0 * nb;
  const int stride = gemv_term_stride(nb);
  // (r, c) of chunk f tracked incrementally (no integer division in the stream loop)
  int r = tid / cpr;
  int c = tid - r * cpr;
#pragma unroll 4
  for (int f = tid; f < total; f += GEMV_NT) {
    int s = dot4x4(slab[f], reinterpret_cast<const int4*>(xl)[c], 0);
    s += __shfl_xor(s, 1);
    if ((tid & 1) == 0) {
      const int b = c >> 1;
      t[r * stride + b] = ((float)s * half_bits_to_float(dslab[r * nb + b])) * xsl[b];
    }
    c += GEMV_NT;
    while (c >= cpr) {
      c -= cpr;
      ++r;
    }
  }
  __syncthreads();
  float acc = 0.0f;
  if (tid < nrows) acc = fold_lds(t + tid * stride, nb);
  return acc;
}

__global__ __launch_bounds__(GEMV_NT) void k_gemv(const int8_t* __restrict__ wq, const uint16_t* __restrict__ wd,
                                                  int rows, int K, const int8_t* __restrict__ xq,
                                                  const float* __restrict__ xs, float* y, const float* resid) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int row0 = blockIdx.x * GEMV_R;
  const float acc = gemv_rows(wq, wd, rows, K, xq, xs, row0, smem);
  const int tid = threadIdx.x;
  if (tid < GEMV_R && row0 + tid < rows) {
    const int row = row0 + tid;
    y[row] = resid ? resid[row] + acc : acc;
  }
}

// Decode-loop state shared by the step's kernels (device memory).
struct StepState {
  uint32_t pos;      // position of the token being computed
  uint32_t tok;      // current token (input of the next step)
  uint32_t step;     // index into the generated-token ring
  uint32_t counter;  // last-workgroup counter of the lm_head GEMV (always returns to 0)
};

// lm_head GEMV fused with greedy argmax (inference.rs:5912-5925: first index of the max,
// strict '>').  Each workgroup reduces its rows to (value, index) with ties to the lower
// index; the last workgroup to finish (atomic ticket) reduces the partials in the same
// way, writes the token, appends it to tokens[step] and advances the position.
__global__ __launch_bounds__(GEMV_NT) void k_gemv_argmax(const int8_t* __restrict__ wq,
                                                         const uint16_t* __restrict__ wd, int rows, int K,
                                                         const int8_t* __restrict__ xq, const float* __restrict__ xs,
                                                         float* __restrict__ logits, float* __restrict__ part_v,
                                                         uint32_t* __restrict__ part_i, StepState* st,
                                                         uint32_t* __restrict__ tokens, uint32_t tokens_cap) {
  extern __shared__ __align__(16) unsigned char smem[];
  __shared__ int s_last;
  __shared__ float rv[GEMV_NT / 64];
  __shared__ uint32_t ri[GEMV_NT / 64];
  const int row0 = blockIdx.x * GEMV_R;
  const float acc = gemv_rows(wq, wd, rows, K, xq, xs, row0, smem);
  const int tid = threadIdx.x;
  if (tid < 64) {
    float bv = -INFINITY;
    uint32_t bi = 0xffffffffu;
    if (tid < GEMV_R && row0 + tid < rows) {
      logits[row0 + tid] = acc;
      if (acc > bv) { bv = acc; bi = (uint32_t)(row0 + tid); }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      const float ov = __shfl_xor(bv, o);
      const uint32_t oi = __shfl_xor(bi, o);
      if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
    }
    if (tid == 0) {
      part_v[blockIdx.x] = bv;
      part_i[blockIdx.x] = bi;
      __threadfence();
      const uint32_t ticket = atomicAdd(&st->counter, 1u);
      s_last = ticket == gridDim.x - 1;
    }
  }
  __syncthreads();
  if (!s_last) return;
  __threadfence();
  float bv = -INFINITY;
  uint32_t bi = 0xffffffffu;
  for (int i = tid; i < (int)gridDim.x; i += GEMV_NT) {
    const float v = part_v[i];
    const uint32_t ix = part_i[i];
    if (v > bv || (v == bv && ix < bi)) { bv = v; bi = ix; }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(bv, o);
    const uint32_t oi = __shfl_xor(bi, o);
    if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
  }
  if ((tid & 63) == 0) { rv[tid >> 6] = bv; ri[tid >> 6] = bi; }
  __syncthreads();
  if (tid == 0) {
    for (int w = 1; w < GEMV_NT / 64; ++w)
      if (rv[w] > bv || (rv[w] == bv && ri[w] < bi)) { bv = rv[w]; bi = ri[w]; }
    const uint32_t tok = bi == 0xffffffffu ? 0u : bi;  // all -inf: index 0, as the CPU loop
    st->tok = tok;
    const uint32_t s = st->step;
    if (tokens && s < tokens_cap) tokens[s] = tok;
    st->step = s + 1;
    st->pos = st->pos + 1;
    st->counter = 0;
  }
}

// ---------------------------------------------------------------------------
// RMSNorm (tensor/mod.rs:2083-2106) fused with Q8_0 quantization of the result.
// One workgroup of 1024 threads; thread t holds x[t + 1024 j] in registers; squares go to
// LDS and thread 0 folds them in order; each 32-lane group then quantizes one block.
// Dynamic LDS = n*4 bytes.  n % 32 == 0, n <= 1024 * RMS_MAXJ.
constexpr int RMS_NT = 1024;
constexpr int RMS_MAXJ = 16;

__global__ __launch_bounds__(RMS_NT) void k_rmsnorm_quant(const float* __restrict__ x, const float* __restrict__ w,
                                                          int n, float eps, int8_t* __restrict__ xq,
                                                          float* __restrict__ xs, float* __restrict__ y_out) {
  extern __shared__ __align__(16) float sq[];
  __shared__ float s_scale;
  const int tid = threadIdx.x;
  float xv[RMS_MAXJ];
#pragma unroll
  for (int j = 0; j < RMS_MAXJ; ++j) {
    const int i = tid + j * RMS_NT;
    if (i < n) {
      xv[j] = x[i];
      sq[i] = xv[j] * xv[j];
    }
  }
  __syncthreads();
  if (tid == 0) {
    const float ms = fold_lds(sq, n) / (float)n;
    s_scale = 1.0f / sqrtf(ms + eps);
  }
  __syncthreads();
  const float scale = s_scale;
#pragma unroll
  for (int j = 0; j < RMS_MAXJ; ++j) {
    const int i = tid + j * RMS_NT;
    if (i < n) {  // uniform per 32-lane group (n % 32 == 0, RMS_NT % 32 == 0)
      const float yv = (xv[j] * scale) * w[i];
      if (y_out) y_out[i] = yv;
      int8_t q;
      const float d = quantize_lane32(yv, &q);
      xq[i] = q;
      if ((tid & 31) == 0) xs[i >> 5] = d;
    }
  }
}

// Plain Q8_0 quantization of an f32 vector: one element per lane, one block per 32 lanes.
__global__ __launch_bounds__(256) void k_quantize_q8_0(const float* __restrict__ x, int n, int8_t* __restrict__ xq,
                                                       float* __restrict__ xs) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;  // uniform per 32-lane group
  int8_t q;
  const float d = quantize_lane32(x[i], &q);
  xq[i] = q;
  if ((i & 31) == 0) xs[i >> 5] = d;
}

// SwiGLU (tensor/mod.rs:1943-1967) + Q8_0 quantization.  gu = [gate(n) | up(n)].
__global__ __launch_bounds__(256) void k_silu_mul_quant(const float* __restrict__ gu, int n, int8_t* __restrict__ xq,
                                                        float* __restrict__ xs, float* __restrict__ act_out) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;  // uniform per 32-lane group
  const float a = silu_mul1(gu[i], gu[n + i]);
  if (act_out) act_out[i] = a;
  int8_t q;
  const float d = quantize_lane32(a, &q);
  xq[i] = q;
  if ((i & 31) == 0) xs[i >> 5] = d;
}

// ---------------------------------------------------------------------------
// Per-head QK RMSNorm (optional) + RoPE + f16 KV store for the token at st->pos (test
// entry point; the engine fuses this into the attention kernel).  One workgroup per head:
// blocks [0, n_heads) are Q heads, [n_heads, n_heads + n_kv) K heads (which also store the
// head's V row).  RoPE: rope.rs:489-524; f16 store: kv_cache.rs:573-600.
__global__ __launch_bounds__(64) void k_rope_kv(const float* __restrict__ qkv, int n_heads, int n_kv, int hd,
                                                int rope_dim, int split_half, const float* __restrict__ cosv,
                                                const float* __restrict__ sinv, const float* __restrict__ q_norm,
                                                const float* __restrict__ k_norm, float eps, float* __restrict__ qrot,
                                                uint16_t* __restrict__ kc, uint16_t* __restrict__ vc, int layer,
                                                int max_pos, const uint32_t* __restrict__ d_pos) {
  __shared__ __align__(16) float buf[512];
  __shared__ __align__(16) float sq[512];
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
    if (threadIdx.x == 0) s_scale = 1.0f / sqrtf(fold_lds(sq, hd) / (float)hd + eps);
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
// Decode attention, faithful (inference.rs:23945-24025), one workgroup per query head.
//   score_p = dot_seq(q, k_p) * scale         one lane per position, d in order
//   m = max_p score_p                          exact
//   e_p = expf(score_p - m); sum = fold_p e_p  serial fold by one lane
//   out_d = fold_p (e_p * (1/sum)) * v_pd      one lane per d, p in order
// FUSED (the engine's path): the kernel first builds this token's q (and the kv head's k
// and v) from the fused QKV projection: optional per-head QK RMSNorm (tensor/mod.rs:2112),
// RoPE (rope.rs:489-524) with the tables at cos_base + pos*rope_stride, f16 rounding of k
// and v (kv_cache.rs:573-600).  The first q head of each GQA group stores the new K/V row;
// every head of the group uses its own LDS copy of that row for position pos.
// Not FUSED (test entry point): q is taken from qsrc and K/V entirely from the cache.
// The head's output is quantized to Q8_0 (hd % 32 == 0: blocks never straddle heads).
// Dynamic LDS = align16(max_pos) * 4 bytes.
constexpr int ATT_NT = 256;

template <bool FUSED>
__global__ __launch_bounds__(ATT_NT) void k_attention(
    const float* __restrict__ qsrc, int n_heads, int n_kv, int hd, int rope_dim, int split_half,
    const float* __restrict__ cos_base, const float* __restrict__ sin_base, int rope_stride,
    const float* __restrict__ q_norm, const float* __restrict__ k_norm, float eps, uint16_t* __restrict__ kc,
    uint16_t* __restrict__ vc, int layer, int max_pos, const uint32_t* __restrict__ d_pos, float scale,
    float* __restrict__ att_out, int8_t* __restrict__ xq, float* __restrict__ xs) {
  extern __shared__ __align__(16) float sc[];
  __shared__ __align__(16) float qs[512];
  __shared__ __align__(16) float kn[512];  // this position's k (f16-rounded), then scratch
  __shared__ __align__(16) float vn[512];  // this position's v (f16-rounded)
  __shared__ __align__(16) float out[512];
  __shared__ __align__(16) float sq[1024];
  __shared__ float red[ATT_NT / 64];
  __shared__ float s_qscale, s_kscale, s_inv;
  const int tid = threadIdx.x;
  const int h = blockIdx.x;
  const int rep = n_heads / n_kv;
  const int kvh = h / rep;
  const int pos = (int)*d_pos;
  const int P = pos + 1;
  const size_t base = (((size_t)layer * n_kv + kvh) * max_pos) * hd;

  if (FUSED) {
    const float* q = qsrc + (size_t)h * hd;
    const float* k = qsrc + (size_t)n_heads * hd + (size_t)kvh * hd;
    const float* v = qsrc + (size_t)(n_heads + n_kv) * hd + (size_t)kvh * hd;
    for (int d = tid; d < hd; d += ATT_NT) {
      qs[d] = q[d];
      kn[d] = k[d];
      vn[d] = half_bits_to_float(f32_to_f16_bits(v[d]));
    }
    if (q_norm) {  // per-head RMSNorm of q and k (two serial folds by two lanes)
      __syncthreads();
      for (int d = tid; d < hd; d += ATT_NT) {
        sq[d] = qs[d] * qs[d];
        sq[512 + d] = kn[d] * kn[d];
      }
      __syncthreads();
      if (tid == 0) s_qscale = 1.0f / sqrtf(fold_lds(sq, hd) / (float)hd + eps);
      if (tid == 64) s_kscale = 1.0f / sqrtf(fold_lds(sq + 512, hd) / (float)hd + eps);
      __syncthreads();
      for (int d = tid; d < hd; d += ATT_NT) {
        qs[d] = (qs[d] * s_qscale) * q_norm[d];
        kn[d] = (kn[d] * s_kscale) * k_norm[d];
      }
    }
    __syncthreads();
    const float* cosv = cos_base + (size_t)pos * rope_stride;
    const float* sinv = sin_base + (size_t)pos * rope_stride;
    const int half = rope_dim >> 1;
    for (int p = tid; p < half; p += ATT_NT) {
      const int d0 = split_half ? p : 2 * p;
      const int d1 = split_half ? p + half : 2 * p + 1;
      const float c = cosv[p], s = sinv[p];
      float x0 = qs[d0], x1 = qs[d1];
      qs[d0] = (x0 * c) - (x1 * s);
      qs[d1] = (x0 * s) + (x1 * c);
      x0 = kn[d0];
      x1 = kn[d1];
      kn[d0] = (x0 * c) - (x1 * s);
      kn[d1] = (x0 * s) + (x1 * c);
    }
    __syncthreads();
    const bool store = (h % rep) == 0;
    for (int d = tid; d < hd; d += ATT_NT) {
      const uint16_t kb = f32_to_f16_bits(kn[d]);
      kn[d] = half_bits_to_float(kb);
      if (store) {
        kc[base + (size_t)pos * hd + d] = kb;
        vc[base + (size_t)pos * hd + d] = f32_to_f16_bits(vn[d]);
      }
    }
  } else {
    for (int d = tid; d < hd; d += ATT_NT) {
      qs[d] = qsrc[(size_t)h * hd + d];
      kn[d] = half_bits_to_float(kc[base + (size_t)pos * hd + d]);
      vn[d] = half_bits_to_float(vc[base + (size_t)pos * hd + d]);
    }
  }
  __syncthreads();

  if (P == 1) {
    // inference.rs:23564-23575: a single position copies the V row.
    for (int d = tid; d < hd; d += ATT_NT) out[d] = vn[d];
  } else {
    // scores
    float lmax = -INFINITY;
    for (int p = tid; p < P; p += ATT_NT) {
      float acc = 0.0f;
      if (p == pos) {
        for (int d = 0; d < hd; ++d) acc += qs[d] * kn[d];
      } else {
        const uint4* kr = reinterpret_cast<const uint4*>(kc + base + (size_t)p * hd);
        for (int d8 = 0; d8 < (hd >> 3); d8 += 4) {
          uint4 raw[4];
#pragma unroll
          for (int u = 0; u < 4; ++u) raw[u] = kr[d8 + u];
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            const uint32_t wv[4] = {raw[u].x, raw[u].y, raw[u].z, raw[u].w};
            const int d = (d8 + u) * 8;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              acc += qs[d + 2 * j] * half_bits_to_float((uint16_t)(wv[j] & 0xffffu));
              acc += qs[d + 2 * j + 1] * half_bits_to_float((uint16_t)(wv[j] >> 16));
            }
          }
        }
      }
      const float s = acc * scale;
      sc[p] = s;
      lmax = fmaxf(lmax, s);
    }
    const float mx = block_max(lmax, red);
    for (int p = tid; p < P; p += ATT_NT) sc[p] = glibc_expf(sc[p] - mx);
    __syncthreads();
    if (tid == 0) s_inv = 1.0f / fold_lds(sc, P);
    __syncthreads();
    const float inv = s_inv;
    for (int p = tid; p < P; p += ATT_NT) sc[p] = sc[p] * inv;
    __syncthreads();
    if (tid < hd) {
      // out_d = fold over p of prob_p * v_pd; V loads run one group of 8 positions ahead.
      const uint16_t* vcol = vc + base + tid;
      float acc = 0.0f;
      const int npre = pos;  // positions read from the cache
      uint16_t cur[8], nxt[8];
      int p = 0;
#pragma unroll
      for (int u = 0; u < 8; ++u) cur[u] = (u < npre) ? vcol[(size_t)u * hd] : 0;
      for (; p + 8 <= npre; p += 8) {
#pragma unroll
        for (int u = 0; u < 8; ++u) nxt[u] = (p + 8 + u < npre) ? vcol[(size_t)(p + 8 + u) * hd] : 0;
#pragma unroll
        for (int u = 0; u < 8; ++u) acc += sc[p + u] * half_bits_to_float(cur[u]);
#pragma unroll
        for (int u = 0; u < 8; ++u) cur[u] = nxt[u];
      }
      for (int u = 0; p < npre; ++p, ++u) acc += sc[p] * half_bits_to_float(cur[u]);
      acc += sc[pos] * vn[tid];
      out[tid] = acc;
    }
  }
  __syncthreads();
  for (int d = tid; d < hd; d += ATT_NT) {
    att_out[(size_t)h * hd + d] = out[d];
    int8_t q;
    const float dd = quantize_lane32(out[d], &q);
    xq[(size_t)h * hd + d] = q;
    if ((d & 31) == 0) xs[((size_t)h * hd + d) >> 5] = dd;
  }
}

// ---------------------------------------------------------------------------
// Greedy argmax (inference.rs:5912-5925) over a vector: one workgroup (test entry point).
__global__ __launch_bounds__(1024) void k_argmax(const float* __restrict__ x, int n, uint32_t* __restrict__ out) {
  __shared__ float bv_s[16];
  __shared__ uint32_t bi_s[16];
  float bv = -INFINITY;
  uint32_t bi = 0xffffffffu;
  for (int i = threadIdx.x; i < n; i += blockDim.x) {
    const float v = x[i];
    if (v > bv) { bv = v; bi = (uint32_t)i; }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(bv, o);
    const uint32_t oi = __shfl_xor(bi, o);
    if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
  }
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  if (lane == 0) { bv_s[wave] = bv; bi_s[wave] = bi; }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < (int)(blockDim.x >> 6); ++w)
      if (bv_s[w] > bv || (bv_s[w] == bv && bi_s[w] < bi)) { bv = bv_s[w]; bi = bi_s[w]; }
    *out = bi == 0xffffffffu ? 0u : bi;
  }
}

// On-device Q8R embedding row gather of st->tok: h[i] = scale_b * q_i (exact;
// tensor/mod.rs:2329-2398).
__global__ __launch_bounds__(256) void k_embed_q8(const int8_t* __restrict__ eq, const uint16_t* __restrict__ ed,
                                                  int H, const StepState* __restrict__ st, float* __restrict__ h) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= H) return;
  const size_t t = st->tok;
  h[i] = half_bits_to_float(ed[t * (H >> 5) + (i >> 5)]) * (float)eq[t * H + i];
}

// glibc-identical expf over a vector (test hook).
__global__ void k_expf(const float* __restrict__ x, float* __restrict__ y, size_t n) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) y[i] = glibc_expf(x[i]);
}

}  // namespace cm
