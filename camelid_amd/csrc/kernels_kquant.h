// kernels_kquant.h -- HIP/CDNA4 kernels of the K-quant decode path (Q4_K / Q6_K weights,
// Q8_K activations; gfx950, wave64).
//
// Weights are kept in HBM as planes split out of the GGUF superblocks (same bytes, so the
// algorithmic bytes stay 144 B / 256 for Q4_K and 210 B / 256 for Q6_K):
//   Q4_K: nibbles [rows][K/2], header [rows][K/256][16] = (f16 d, f16 dmin, 12 scale bytes)
//   Q6_K: ql [rows][K/2], qh [rows][K/4], scales [rows][K/256][16] (i8), d [rows][K/256] (f16)
// so that a lane streams 16-byte pieces of one plane and the headers arrive once per
// superblock.  The activation is quantized to Q8_K by k_quantize_q8k and staged in LDS.
#pragma once
#include "kernels_decode.h"
#include "kernels_prefill.h"

namespace cm {

// ---------------------------------------------------------------------------
// Q8_K quantization of n values (quantize_q8k, cuda_resident.rs:1416-1490), one workgroup per
// 256-value block (quantize_q8k_wg256: inference.rs:17564-17599), with the per-32 quant sums
// the Q4_K mins side reads.
__global__ __launch_bounds__(256) void k_quantize_q8k(const float* __restrict__ x, float* __restrict__ yd,
                                                      int8_t* __restrict__ yq, int32_t* __restrict__ ybs) {
  const size_t s = blockIdx.x;
  quantize_q8k_wg256(x[s * 256 + threadIdx.x], yq + s * 256, ybs + s * 8, yd + s);
}

// Integer sums over lane groups (exact in any order), by DPP lane exchanges inside each row
// of 16 lanes: one VALU add per step, where a __shfl_xor is an LDS permute round trip.
//   quad_sum: every lane of each aligned quad gets the quad's sum (xor-1 then xor-2 partners).
//   group8_sum_lead: lane 8g (the first of each aligned group of 8) gets the group's sum: the
//   quad sums, then lane 8g adds lane 8g + 4's (row_ror:12: lane i reads lane i - 12 mod 16 of
//   its row); the other lanes hold partials.
#define CM_DPP_ADD(v, ctrl) ((v) + __builtin_amdgcn_update_dpp(0, (v), (ctrl), 0xf, 0xf, false))
__device__ __forceinline__ int quad_sum(int v) {
  v = CM_DPP_ADD(v, 0xB1);  // quad_perm [1,0,3,2]
  v = CM_DPP_ADD(v, 0x4E);  // quad_perm [2,3,0,1]
  return v;
}
__device__ __forceinline__ int group8_sum_lead(int v) {
  v = quad_sum(v);
  return CM_DPP_ADD(v, 0x12C);  // row_ror:12
}
#undef CM_DPP_ADD

// Q8_K quantization of one 256-value block by one wave (lane l holds values 4l..4l+3) into
// LDS: quants, per-32 sums and the scale (inference.rs:17564-17599, as quantize_q8k_wg256).
// The block's (|max|, first index) pick needs only |max| and the sign of the value at its
// first occurrence: a wave max, then a wave min over (index << 1 | sign) of the lanes holding it.
__device__ __forceinline__ void quantize_q8k_wave_vals(const float4 v4, int8_t* q, int* bs, float* d) {
  const int lane = threadIdx.x & 63;
  const float vals[4] = {v4.x, v4.y, v4.z, v4.w};
  float a = 0.0f;
#pragma unroll
  for (int e = 0; e < 4; ++e) a = fabsf(vals[e]) > a ? fabsf(vals[e]) : a;
  a = max_wave(a);
  uint32_t key = 0xffffffffu;
#pragma unroll
  for (int e = 3; e >= 0; --e)
    key = fabsf(vals[e]) == a ? ((uint32_t)(4 * lane + e) << 1) | (__float_as_uint(vals[e]) >> 31) : key;
  key = min_wave(key);
  const float v = (key & 1u) ? -a : a;  // the value at the first index of the maximum (a > 0)
  const float iscale = a > 0.0f ? -127.0f / v : 0.0f;
  uint32_t word = 0;
  int sum = 0;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int qv = a > 0.0f ? min(nearest_int_ref(iscale * vals[e]), 127) : 0;
    sum += (int8_t)qv;
    word |= ((uint32_t)qv & 0xffu) << (8 * e);
  }
  reinterpret_cast<uint32_t*>(q)[lane] = word;
  sum = group8_sum_lead(sum);
  if ((lane & 7) == 0) bs[lane >> 3] = sum;
  if (lane == 0) *d = a > 0.0f ? 1.0f / iscale : 0.0f;
}

constexpr int KQ_NT = 256;  // 4 waves
__host__ __device__ inline int kq_rows_per_wg(int rpw) { return 4 * rpw; }

// ---------------------------------------------------------------------------
// In-launch handoff of a norm-fused K-quant GEMV: workgroup 0 computes the RMSNorm and its
// Q8_K quantization and publishes it with agent-scope (XCD-coherent) stores, waits for them
// to complete, then sets a flag word (one copy per XCD, 128 bytes apart); every other
// workgroup issues its weight loads, waits for the copy of its own XCD (workgroup b runs on
// XCD b % 8) and reads the activation with agent-scope loads.  Two flag slots, one per norm
// of a layer: a launch resets the other slot (whose launch has completed: the launches of the
// two kinds strictly alternate) and uses its own, which the previous launch reset.  The wait
// is bounded (about a second): past it the workgroup sets g_handoff_error and goes on.
constexpr int NF_XCD = 8, NF_STRIDE = 32;  // flag copies per slot, words between copies
constexpr int NF_WORDS = 2 * NF_XCD * NF_STRIDE;

// The waiting side: thread 0 polls its XCD's copy of the slot, then the workgroup barrier.
__device__ __forceinline__ void handoff_wait(const uint32_t* slot) {
  if (threadIdx.x == 0) {
    const uint32_t* f = slot + (blockIdx.x % NF_XCD) * NF_STRIDE;
    uint32_t polls = 0;
    while (ld_agent32(f) == 0u) {
      __builtin_amdgcn_s_sleep(2);
      if (++polls == (1u << 20)) {
        g_handoff_error = 1u;
        break;
      }
    }
  }
  __syncthreads();
}

// ---------------------------------------------------------------------------
// Q4_K GEMV (q4k_gemv, cuda_resident.rs:601; CPU: q4_k_dot_arm, refmath.rs:424-561, the
// Q4_K decode dot of inference.rs:17906-17965), faithful:
//   per superblock s: prod = sum_g bsum32_g * min_g, sumi = sum_j (lo_j*sc_2j + hi_j*sc_2j+1)
//   (exact integers), then  sumf = fma(-(y.d*dmin), prod, sumf); sumf = fma(y.d*d, sumi, sumf)
//   in superblock order from 0;  y[row] = (resid ? resid[row] : 0) + sumf.
// Lane work unit: one 16-byte nibble piece (32 weights: piece j of superblock s pairs its low
// nibbles with q8[64(j/2) + 16(j%2) ..] and its high nibbles 32 values further); IT pieces
// per lane and row, every load of a wave issued before the first dot; the 8 lanes of a
// superblock reduce their integers with butterflies, the first writes the superblock's four
// fold operands to LDS, and one lane per row folds them in order.
// xf (optional): the activation in f32, quantized to Q8_K by the workgroup itself (one wave
// per 256-value block) instead of read from yd/yq/ybs: a K-quant projection of the attention
// output needs no separate quantizer launch.
// Dynamic LDS: K quants + K/256 scales + K/32 sums + rows * K/256 * 16 bytes.
__host__ __device__ inline size_t kq4_terms_offset(int K) {
  return ((size_t)K + (size_t)(K / 256) * 4 + (size_t)(K / 32) * 4 + 15) & ~(size_t)15;
}
__host__ __device__ inline size_t kq4_lds_bytes(int K, int R) {
  return kq4_terms_offset(K) + (size_t)R * (K / 256) * 16;
}

// TAGF (with XF): the f32 activation arrives as [K] tagged words from other workgroups of the
// launch (xf_t, ao_tag in the high half, agent-scope): the waves wait for their blocks' words
// instead of loading xf, then quantize as with XF.
// HQ: lane j of a superblock's 8 lanes loads only dword j % 4 of the 16-byte header, and each
// 4-lane quad rebuilds the whole header with DPP broadcasts where it is used (5 instead of 8
// registers per row and piece).
template <int IT, int RPW, int NT = KQ_NT, bool XF = false, bool TAGF = false, bool HQ = false>
__device__ __forceinline__ void gemv_q4k_body(const int bid, const uint8_t* __restrict__ nib, const uint8_t* __restrict__ hdr,
                                                    int rows, int K, const float* __restrict__ yd,
                                                    const int8_t* __restrict__ yq, const int32_t* __restrict__ ybs,
                                                    float* y, const float* resid, float* __restrict__ part_v,
                                                    uint32_t* __restrict__ part_i, const float* __restrict__ xf,
                                                    const uint32_t* ready = nullptr, int sk = -1,
                                                    const uint64_t* xf_t = nullptr, uint32_t tag = 0,
                                                    int ao_layer = -1) {
  static_assert(!TAGF || XF, "tagged f32 words are an f32 activation");
  (void)ao_layer;  // (the measurement build: TAGF phase stamps of the first and last workgroup, g_ao_stamps)
#ifdef CM_STAMPS
#define CM_AOQ_STAMP(i)                                                                                        \
  if (TAGF && threadIdx.x == 0 && ao_layer >= 0 && ao_layer < 64 &&                                           \
      (bid == 0 || bid == (int)gridDim.x - 1 - ((int)blockIdx.x - bid)))                                      \
    g_ao_stamps[((size_t)ao_layer * 2 + (bid != 0)) * AO_NSTAMP + (i)] = __builtin_amdgcn_s_memrealtime();
#else
#define CM_AOQ_STAMP(i)
#endif
  CM_AOQ_STAMP(0)
  (void)sk;  // (the measurement build's stamp kind)
  constexpr int R = (NT / 64) * RPW;
  static_assert(R <= 64, "one lane per row folds the terms");
  extern __shared__ __align__(16) unsigned char smem[];
  const int NSB = K >> 8, NC = K >> 5;
  int8_t* xq = reinterpret_cast<int8_t*>(smem);
  float* xd = reinterpret_cast<float*>(smem + K);
  int* xbs = reinterpret_cast<int*>(smem + K + NSB * 4);
  float4* terms = reinterpret_cast<float4*>(smem + kq4_terms_offset(K));
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int row0 = bid * R;
  // XF: the loads of this wave's first four 256-value blocks of the f32 activation go out
  // first (from L2), so that its Q8_K quantization waits for them only, not for the weight
  // loads behind them (loads complete in issue order for the wait counter)
  constexpr int NW = NT / 64, PB = 4;
  float4 pre[XF ? PB : 1];
  if constexpr (XF && !TAGF) {
#pragma unroll
    for (int u = 0; u < PB; ++u) {
      const int b = wave + NW * u;
      if (b < NSB) pre[u] = reinterpret_cast<const float4*>(xf + 256 * b)[lane];
    }
  }
  // every weight and header load of this wave next (pieces lane + 64 i of each row; past
  // NC clamped, their results never stored)
  uint4 wv[RPW][IT], hv[HQ ? 1 : RPW][HQ ? 1 : IT];
  uint32_t hw[HQ ? RPW : 1][HQ ? IT : 1];
#pragma unroll
  for (int k = 0; k < RPW; ++k) {
    const int row = min(row0 + wave * RPW + k, rows - 1);
    const uint4* np = reinterpret_cast<const uint4*>(nib + (size_t)row * (K >> 1));
    const uint4* hp = reinterpret_cast<const uint4*>(hdr + (size_t)row * NSB * 16);
#pragma unroll
    for (int i = 0; i < IT; ++i) {
      const int cc = min(lane + 64 * i, NC - 1);
      wv[k][i] = ld_stream(np + cc);
      if constexpr (HQ)
        hw[k][i] = ld_stream(reinterpret_cast<const uint32_t*>(hp + (cc >> 3)) + (lane & 3));
      else
        hv[k][i] = ld_stream(hp + (cc >> 3));
    }
  }
  if (ready) {  // the activation published by workgroup 0 of this launch (agent-scope loads)
    handoff_wait(ready);
    for (int c = tid; c < (K >> 3); c += NT) reinterpret_cast<uint64_t*>(xq)[c] = ld_agent64(yq + 8 * c);
    for (int i = tid; i < NSB; i += NT) xd[i] = __uint_as_float(ld_agent32(yd + i));
    for (int i = tid; i < NC; i += NT) xbs[i] = (int)ld_agent32(ybs + i);
    if (sk >= 0) {
      CM_GEMV_STAMP_SAMPLED(sk, 3, 0)
    }
  } else if constexpr (TAGF) {  // the f32 activation as tagged words: one watcher, then every lane its own
    if (threadIdx.x == 0) (void)ao_wait_word(xf_t + (blockIdx.x * 97u) % (uint32_t)K, tag);
    __syncthreads();
    CM_AOQ_STAMP(1)
    for (int b = wave; b < NSB; b += NW) {
      // the lane's four words in one round trip (issued together), then a poll of any whose
      // tag is not there yet
      const uint64_t* wp = xf_t + 256 * b + 4 * lane;
      uint64_t v[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) v[u] = ld_agent64(wp + u);
#pragma unroll
      for (int u = 0; u < 4; ++u)
        if ((uint32_t)(v[u] >> 32) != tag) v[u] = ao_wait_word(wp + u, tag);
      const float4 f = make_float4(__uint_as_float((uint32_t)v[0]), __uint_as_float((uint32_t)v[1]),
                                   __uint_as_float((uint32_t)v[2]), __uint_as_float((uint32_t)v[3]));
      quantize_q8k_wave_vals(f, xq + 256 * b, xbs + 8 * b, xd + b);
    }
  } else if constexpr (XF) {  // the activation given in f32: each wave quantizes blocks wave, wave + NW, ... to Q8_K
#pragma unroll
    for (int u = 0; u < PB; ++u) {
      const int b = wave + NW * u;
      if (b < NSB) quantize_q8k_wave_vals(pre[u], xq + 256 * b, xbs + 8 * b, xd + b);
    }
    for (int b = wave + NW * PB; b < NSB; b += NW)
      quantize_q8k_wave_vals(reinterpret_cast<const float4*>(xf + 256 * b)[lane], xq + 256 * b, xbs + 8 * b, xd + b);
  } else {
    for (int c = tid; c < (K >> 4); c += NT) reinterpret_cast<int4*>(xq)[c] = reinterpret_cast<const int4*>(yq)[c];
    for (int i = tid; i < NSB; i += NT) xd[i] = yd[i];
    for (int i = tid; i < NC; i += NT) xbs[i] = ybs[i];
  }
  __syncthreads();
  CM_AOQ_STAMP(2)
  const uint32_t K1 = 0x3f3f3f3fu, K2 = 0x0f0f0f0fu, K3 = 0x03030303u;
#pragma unroll
  for (int k = 0; k < RPW; ++k) {
    const int rl = wave * RPW + k;
#pragma unroll
    for (int i = 0; i < IT; ++i) {
      __builtin_amdgcn_sched_barrier(0);
      const int c = lane + 64 * i;
      const bool valid = c < NC;  // uniform per 8-lane superblock group (NC % 8 == 0)
      const int cc = min(c, NC - 1);
      const uint4 w = wv[k][i];
      uint4 hd;
      if constexpr (HQ) {  // quad_perm broadcasts of lanes 0..3 of this lane's quad (whole quads clamp alike)
        const int hq = (int)hw[k][i];
        hd = make_uint4((uint32_t)__builtin_amdgcn_update_dpp(0, hq, 0x00, 0xf, 0xf, false),
                        (uint32_t)__builtin_amdgcn_update_dpp(0, hq, 0x55, 0xf, 0xf, false),
                        (uint32_t)__builtin_amdgcn_update_dpp(0, hq, 0xaa, 0xf, 0xf, false),
                        (uint32_t)__builtin_amdgcn_update_dpp(0, hq, 0xff, 0xf, 0xf, false));
      } else {
        hd = hv[k][i];
      }
      const int s = cc >> 3, j = cc & 7, c4 = j >> 1, h = j & 1;
      const uint32_t scw = (c4 < 2) ? (hd.y & K1) : ((hd.w & K2) | (((hd.y >> 6) & K3) << 4));
      const uint32_t mnw = (j < 4) ? (hd.z & K1) : (((hd.w >> 4) & K2) | (((hd.z >> 6) & K3) << 4));
      const int sc_lo = (scw >> (8 * ((2 * c4) & 3))) & 0xff;
      const int sc_hi = (scw >> (8 * ((2 * c4 + 1) & 3))) & 0xff;
      const int mn = (mnw >> (8 * (j & 3))) & 0xff;
      const int base = (s << 8) + 64 * c4 + 16 * h;
      const int4 qa = *reinterpret_cast<const int4*>(xq + base);
      const int4 qb = *reinterpret_cast<const int4*>(xq + base + 32);
      int lo = 0, hi = 0;
      lo = __builtin_amdgcn_sdot4((int)(w.x & K2), qa.x, lo, false);
      lo = __builtin_amdgcn_sdot4((int)(w.y & K2), qa.y, lo, false);
      lo = __builtin_amdgcn_sdot4((int)(w.z & K2), qa.z, lo, false);
      lo = __builtin_amdgcn_sdot4((int)(w.w & K2), qa.w, lo, false);
      hi = __builtin_amdgcn_sdot4((int)((w.x >> 4) & K2), qb.x, hi, false);
      hi = __builtin_amdgcn_sdot4((int)((w.y >> 4) & K2), qb.y, hi, false);
      hi = __builtin_amdgcn_sdot4((int)((w.z >> 4) & K2), qb.z, hi, false);
      hi = __builtin_amdgcn_sdot4((int)((w.w >> 4) & K2), qb.w, hi, false);
      const int sumi = group8_sum_lead(lo * sc_lo + hi * sc_hi);
      const int prod = group8_sum_lead(xbs[s * 8 + j] * mn);
      if (valid && j == 0) {
        const float ydv = xd[s];
        const float dw = half_bits_to_float((uint16_t)(hd.x & 0xffffu));
        const float dmw = half_bits_to_float((uint16_t)(hd.x >> 16));
        terms[s * R + rl] = make_float4(-(ydv * dmw), (float)prod, ydv * dw, (float)sumi);
      }
    }
  }
  __syncthreads();
  if (tid < 64) {
    float acc = 0.0f;
    if (tid < R) {
      const float4* t = terms + tid;  // superblock-major: the fold lanes read consecutive entries
      for (int s = 0; s < NSB; ++s) {
        const float4 v = t[s * R];
        acc = fmaf(v.x, v.y, acc);
        acc = fmaf(v.z, v.w, acc);
      }
    }
    const int row = row0 + tid;
    const bool live = tid < R && row < rows;
    if (live) y[row] = resid ? resid[row] + acc : acc;
    CM_AOQ_STAMP(3)
    if (part_v) {  // lm_head: this workgroup's argmax partial (first index of the max)
      float bv = live ? acc : -INFINITY;
      uint32_t bi = live ? (uint32_t)row : 0xffffffffu;
      argmax_wave(bv, bi);
      if (tid == 0) {
        part_v[bid] = bv;
        part_i[bid] = bi;
      }
    }
  }
  if (sk >= 0) {
    CM_GEMV_STAMP_SAMPLED(sk, 5, 0)
  }
}
#undef CM_AOQ_STAMP

// XF: the activation comes as f32 in xf (quantized by the workgroup), else as Q8_K in yd/yq/ybs
// (a separate instantiation: the f32 path's registers would lower every launch's occupancy).
template <int IT, int RPW, bool XF = false>
__global__ __launch_bounds__(KQ_NT) void k_gemv_q4k(const uint8_t* __restrict__ nib, const uint8_t* __restrict__ hdr,
                                                    int rows, int K, const float* __restrict__ yd,
                                                    const int8_t* __restrict__ yq, const int32_t* __restrict__ ybs,
                                                    float* y, const float* resid, float* __restrict__ part_v,
                                                    uint32_t* __restrict__ part_i, const float* __restrict__ xf) {
  gemv_q4k_body<IT, RPW, KQ_NT, XF>((int)blockIdx.x, nib, hdr, rows, K, yd, yq, ybs, y, resid, part_v, part_i, xf);
}

// ---------------------------------------------------------------------------
// Q6_K GEMV (q6k_gemv, cuda_resident.rs:925; CPU: q6_k_wire_row_dot, inference.rs:19240-19295,
// the Q6_K decode dot of inference.rs:19148-19195), faithful:
//   per superblock s: aux[l] = sum over positions p = l (mod 8) of sc[p/16] * q8[p] * w[p]
//   (exact integers); sums[l] += (f16(d_w) * y.d) * aux[l] in superblock order;
//   result = left fold of sums[0..8] from -0.0;  y[row] = (resid ? resid[row] : 0) + result.
// Lane work unit: 64 weights that share 16 bytes of qh (half n, offset q0 in {0, 16}): the
// 16-value groups q0 + 32k (k = 0..3) of the half, rebuilt from two 16-byte ql pieces.
// For each group the 8 position classes are separated with byte permutes: class l takes
// the group's values l and 8 + l, paired with the activation dword (q_l, q_8+l, q_l, q_8+l)
// prepared once per workgroup in LDS, and bytes 2-3 of the weight dword set to -32, so one
// dot4 gives sum (w - 32) * q over the class.  The 4 lanes of a superblock reduce their 8
// class sums with butterflies; the superblock's 8 products d * aux go to LDS; then 8 lanes
// per row run the 8 class chains and the first folds them.
// Dynamic LDS: K/256 * 512 bytes of activation pairs + K/256 scales + rows * K/256 * 32 bytes.
__host__ __device__ inline size_t kq6_terms_offset(int K) {
  return ((size_t)(K / 256) * 516 + 15) & ~(size_t)15;
}
__host__ __device__ inline size_t kq6_lds_bytes(int K, int R) {
  return kq6_terms_offset(K) + (size_t)R * (K / 256) * 32;
}

template <int RPW, int NT = KQ_NT, bool PRE = false>
__device__ __forceinline__ void gemv_q6k_body(const int bid, const uint8_t* __restrict__ ql, const uint8_t* __restrict__ qh,
                                                    const int8_t* __restrict__ scl, const uint16_t* __restrict__ dw,
                                                    int rows, int K, const float* __restrict__ yd,
                                                    const int8_t* __restrict__ yq, float* y, const float* resid,
                                                    float* __restrict__ part_v, uint32_t* __restrict__ part_i,
                                                    const uint32_t* ready = nullptr, int sk = -1) {
  (void)sk;  // (the measurement build's stamp kind)
  constexpr int R = (NT / 64) * RPW;
  static_assert(R <= 8, "eight lanes per row run the class chains");
  extern __shared__ __align__(16) unsigned char smem[];
  const int NSB = K >> 8, NU = K >> 6;
  uint32_t* xp = reinterpret_cast<uint32_t*>(smem);  // [s][group j][class l] activation pairs
  float* xd = reinterpret_cast<float*>(smem + NSB * 512);
  float* terms = reinterpret_cast<float*>(smem + kq6_terms_offset(K));  // [row][s][l]
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int row0 = bid * R;
  // the weight pieces of one lane work unit (row rl of this workgroup, unit u0 + lane)
  struct Unit6 {
    uint4 l0, l1, hh, sc;
    uint32_t d;  // the superblock's f16 scale bits
  };
  auto load_unit = [&](int rl, int u0) {
    const int row = min(row0 + rl, rows - 1);
    const int uu = min(u0 + lane, NU - 1);
    const int s = uu >> 2, n = (uu >> 1) & 1, q0 = (uu & 1) * 16;
    const uint8_t* qlr = ql + (size_t)row * (K >> 1);
    Unit6 w;
    w.l0 = ld_stream(reinterpret_cast<const uint4*>(qlr + s * 128 + n * 64 + q0));
    w.l1 = ld_stream(reinterpret_cast<const uint4*>(qlr + s * 128 + n * 64 + 32 + q0));
    w.hh = ld_stream(reinterpret_cast<const uint4*>(qh + (size_t)row * (K >> 2) + s * 64 + n * 32 + q0));
    w.sc = ld_stream(reinterpret_cast<const uint4*>(scl + ((size_t)row * NSB + s) * 16));
    w.d = dw[(size_t)row * NSB + s];
    return w;
  };
  // PRE (the norm-fused launch): the first unit's loads go out before the wait for the
  // activation (16 more registers live across it, which the plain launches do not spend)
  Unit6 first;
  if (PRE) first = load_unit(wave * RPW, 0);
  // activation pairs: entry (s, j, l) = bytes (q[16j+l], q[16j+8+l], q[16j+l], q[16j+8+l])
  // (published by workgroup 0 of this launch: agent-scope loads after the handoff)
  if (ready) handoff_wait(ready);
  for (int e = tid; e < NSB * 128; e += NT) {
    const int l = e & 7, g = e >> 3;  // g = s * 16 + j
    const uint32_t* src = reinterpret_cast<const uint32_t*>(yq + (size_t)g * 16);
    const uint32_t a = ready ? ld_agent32(src + (l >> 2)) : src[l >> 2];
    const uint32_t b = ready ? ld_agent32(src + (l >> 2) + 2) : src[(l >> 2) + 2];
    const uint32_t bl = l & 3;
    // bytes: 0 <- a.byte(bl), 1 <- b.byte(bl), 2 <- a.byte(bl), 3 <- b.byte(bl)
    const uint32_t sel = bl | ((4 + bl) << 8) | (bl << 16) | ((4 + bl) << 24);
    xp[e] = __builtin_amdgcn_perm(b, a, sel);
  }
  for (int i = tid; i < NSB; i += NT) xd[i] = ready ? __uint_as_float(ld_agent32(yd + i)) : yd[i];
  if (sk >= 0) {
    CM_GEMV_STAMP_SAMPLED(sk, 3, 0)
  }
  __syncthreads();
  const uint32_t M4 = 0x0f0f0f0fu, M2 = 0x03030303u;
  auto unit = [&](int rl, int u0, const Unit6& w) {
    const int u = u0 + lane;
    const bool valid = u < NU;  // uniform per 4-lane superblock group (NU % 4 == 0)
    const int uu = min(u, NU - 1);
    const int s = uu >> 2, n = (uu >> 1) & 1, q0 = (uu & 1) * 16;
    const uint32_t L0[4] = {w.l0.x, w.l0.y, w.l0.z, w.l0.w}, L1[4] = {w.l1.x, w.l1.y, w.l1.z, w.l1.w};
    const uint32_t HH[4] = {w.hh.x, w.hh.y, w.hh.z, w.hh.w};
    int aux[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const int j = n * 8 + (q0 >> 4) + 2 * kk;  // the group's index (scale index)
      // scale word j / 4 = 2n + kk / 2 (a select, not an indexed register array)
      const uint32_t scw = n ? (kk < 2 ? w.sc.z : w.sc.w) : (kk < 2 ? w.sc.x : w.sc.y);
      const int sc = (int)(int8_t)((scw >> (8 * (j & 3))) & 0xff);
      uint32_t v[4];
#pragma unroll
      for (int t4 = 0; t4 < 4; ++t4) {
        const uint32_t lq = (kk & 1) ? L1[t4] : L0[t4];
        const uint32_t lo = (kk < 2) ? (lq & M4) : ((lq >> 4) & M4);
        v[t4] = lo | (((HH[t4] >> (2 * kk)) & M2) << 4);
      }
      const uint32_t* xg = xp + (size_t)(s * 16 + j) * 8;
#pragma unroll
      for (int l = 0; l < 8; ++l) {
        const uint32_t bl = l & 3;
        const uint32_t a = v[l >> 2], b = v[(l >> 2) + 2];
        const uint32_t wpair = __builtin_amdgcn_perm(b, a, bl | ((4 + bl) << 8) | (0x0c << 16) | (0x0cu << 24)) |
                               0xe0e00000u;
        aux[l] += sc * __builtin_amdgcn_sdot4((int)wpair, (int)xg[l], 0, false);
      }
    }
#pragma unroll
    for (int l = 0; l < 8; ++l) aux[l] = quad_sum(aux[l]);
    if (valid && (uu & 3) == 0) {
      const float d = half_bits_to_float((uint16_t)w.d) * xd[s];
      float* tp = terms + ((size_t)rl * NSB + s) * 8;
      *reinterpret_cast<float4*>(tp) = make_float4(d * (float)aux[0], d * (float)aux[1], d * (float)aux[2],
                                                   d * (float)aux[3]);
      *reinterpret_cast<float4*>(tp + 4) = make_float4(d * (float)aux[4], d * (float)aux[5], d * (float)aux[6],
                                                       d * (float)aux[7]);
    }
  };
  if constexpr (PRE) {  // (one unit per lane: K <= 4096, as the norm-fused launch's callers check)
    static_assert(RPW == 1, "the preloaded unit is the wave's only one");
    unit(wave, 0, first);
  } else {
#pragma unroll
    for (int k = 0; k < RPW; ++k) {
      const int rl = wave * RPW + k;
      for (int u0 = 0; u0 < NU; u0 += 64) unit(rl, u0, load_unit(rl, u0));
    }
  }
  __syncthreads();
  if (tid < 64) {
    // lanes 8r .. 8r+7: the 8 class chains of row r (R <= 8)
    const int r = tid >> 3, l = tid & 7;
    float sl = 0.0f;
    if (r < R) {
      const float* t = terms + (size_t)r * NSB * 8 + l;
      for (int s = 0; s < NSB; ++s) sl += t[s * 8];
    }
    float acc = -0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) acc += __shfl(sl, (tid & ~7) + i);
    const int row = row0 + r;
    const bool live = l == 0 && r < R && row < rows;
    if (live) y[row] = resid ? resid[row] + acc : acc;
    if (part_v) {  // lm_head: this workgroup's argmax partial (first index of the max)
      float bv = live ? acc : -INFINITY;
      uint32_t bi = live ? (uint32_t)row : 0xffffffffu;
      argmax_wave(bv, bi);
      if (tid == 0) {
        part_v[bid] = bv;
        part_i[bid] = bi;
      }
    }
  }
  if (sk >= 0) {
    CM_GEMV_STAMP_SAMPLED(sk, 5, 0)
  }
}

// The Q4_K output projection inside the split decode attention launch (k_att_fused): 32 rows
// per 1024-thread workgroup (2 per wave), their weight loads issued as the workgroup starts (at
// the launch's start on the CUs the attention leaves free, the rest as the score slices retire);
// the attention output is read as tagged f32 words as the output workgroups store them,
// quantized to Q8_K by the workgroup (one wave per 256-value block) and dotted exactly as by
// k_gemv_q4k<IT, RPW, true> on the f32 activation: the same bits.  y = resid + W_o att.
constexpr int AOQ_RPW = 2;
constexpr int AOQ_ROWS = AOQ_RPW * 16;  // rows per projection workgroup
__host__ __device__ constexpr bool aoq_width_ok(int K) { return K == 4096; }
template <int NT>
__device__ __forceinline__ void att_oproj_q4k(const OProj& op, int wg, uint32_t tag) {
  static_assert(NT == 1024, "sixteen waves, AOQ_RPW rows each");
  gemv_q4k_body<2, AOQ_RPW, NT, true, true, true>(wg, op.k4nib, op.k4hdr, op.rows, op.K, nullptr, nullptr, nullptr,
                                                  op.y, op.resid, nullptr, nullptr, nullptr, nullptr, -1, op.xf_t,
                                                  tag, op.layer);
}

template <int RPW>
__global__ __launch_bounds__(KQ_NT) void k_gemv_q6k(const uint8_t* __restrict__ ql, const uint8_t* __restrict__ qh,
                                                    const int8_t* __restrict__ scl, const uint16_t* __restrict__ dw,
                                                    int rows, int K, const float* __restrict__ yd,
                                                    const int8_t* __restrict__ yq, float* y, const float* resid,
                                                    float* __restrict__ part_v, uint32_t* __restrict__ part_i) {
  gemv_q6k_body<RPW>((int)blockIdx.x, ql, qh, scl, dw, rows, K, yd, yq, y, resid, part_v, part_i);
}

// ---------------------------------------------------------------------------
// The q|k (Q4_K, stacked) and v (Q6_K) projections of a Q4_K_M layer in one launch: both
// read the same Q8_K activation, so workgroups [0, g4) run the Q4_K GEMV over the q|k rows
// and workgroups [g4, gridDim.x) the Q6_K GEMV over the v rows (one row per wave each, no
// residual).  Each output row is computed exactly as by k_gemv_q4k / k_gemv_q6k; the launch
// saves the v projection's own dispatch.  Dynamic LDS: the larger of the two kernels' needs.
template <int IT>
__global__ __launch_bounds__(KQ_NT) void k_gemv_qk4_v6(const uint8_t* __restrict__ nib, const uint8_t* __restrict__ hdr,
                                                       int rows4, float* y4, int g4, const uint8_t* __restrict__ ql,
                                                       const uint8_t* __restrict__ qh, const int8_t* __restrict__ scl,
                                                       const uint16_t* __restrict__ dw, int rows6, float* y6, int K,
                                                       const float* __restrict__ yd, const int8_t* __restrict__ yq,
                                                       const int32_t* __restrict__ ybs) {
  if ((int)blockIdx.x < g4)
    gemv_q4k_body<IT, 1>((int)blockIdx.x, nib, hdr, rows4, K, yd, yq, ybs, y4, nullptr, nullptr, nullptr, nullptr);
  else
    gemv_q6k_body<1>((int)blockIdx.x - g4, ql, qh, scl, dw, rows6, K, yd, yq, y6, nullptr, nullptr, nullptr);
}

// ---------------------------------------------------------------------------
// Norm-fused K-quant decode GEMVs (hidden 4096 = 512 threads x 8 values).  Workgroup 0 of
// the launch computes the layer's RMSNorm (tensor/mod.rs:2083-2106: the in-order sum of
// squares, scale = 1/sqrt(ss/n + eps), y = (x * scale) * w) and its Q8_K quantization
// (inference.rs:17564-17599, as k_rmsnorm_quant: the same operations, so the same bits) and
// publishes the activation (see handoff_wait); the other workgroups run the GEMV bodies with
// eight waves, whose weight loads go out before they wait for it.  The RMSNorm launch of the
// unfused layer and its dependency gap disappear; its latency overlaps the weight stream.
// Eight waves per workgroup (where the plain K-quant GEMVs run four): the norm workgroup's
// eight values per thread keep the kernel within 64 VGPRs, so as many GEMV waves stay
// resident as in the plain launches, and the one-pass sum is shorter at 512 threads.
constexpr int NF_NT = 512;  // threads of a norm-fused launch's workgroups
constexpr int NQ_C = 8;     // values per thread of the norm workgroup
__host__ __device__ inline size_t norm_q8k_lds_bytes(int n) { return (size_t)n * 4 + sizeof(FsLds<NF_NT>); }

// Q8_K quantization of one 256-value block held 8 values per lane by a half wave (lane l of
// the half: values 8l..8l+7; inference.rs:17564-17599, as k_rmsnorm_quant), stored with
// agent-scope (XCD-coherent) stores for a reader in the same launch: this lane's 8 quants to
// q8 (8 bytes), the per-32 sums to bs (by lanes l % 4 == 0), the scale to d (by lane l == 0).
// The block's (|max|, first index) pick needs only |max| and the sign of its first
// occurrence: a max, then a min over (index << 1 | sign) of the lanes holding |max|.
__device__ __forceinline__ void q8k_half_wave_block(const float (&y)[8], int l, int8_t* q8, int32_t* bs, float* d,
                                                    int kind = -1) {
  (void)kind;  // (the measurement build's stamp kind)
  constexpr int C = 8;
  float a = 0.0f;
#pragma unroll
  for (int e = 0; e < C; ++e) a = fabsf(y[e]) > a ? fabsf(y[e]) : a;
  a = max_half_wave(a);
  uint32_t key = 0xffffffffu;
#pragma unroll
  for (int e = C - 1; e >= 0; --e)
    key = fabsf(y[e]) == a ? ((uint32_t)(C * l + e) << 1) | (__float_as_uint(y[e]) >> 31) : key;
  key = min_half_wave(key);
  const float v = (key & 1u) ? -a : a;  // y at the first index of the maximum (a > 0)
  if (kind >= 0) {
    CM_GEMV_STAMP(kind, 3, 0)
  }
  const float iscale = a > 0.0f ? -127.0f / v : 0.0f;
  uint32_t words[C / 4];
  int sum = 0;
#pragma unroll
  for (int w4 = 0; w4 < C / 4; ++w4) {
    uint32_t word = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int q = a > 0.0f ? min(nearest_int_ref(iscale * y[w4 * 4 + e]), 127) : 0;
      sum += (int8_t)q;
      word |= ((uint32_t)q & 0xffu) << (8 * e);
    }
    words[w4] = word;
  }
  // the lanes of a quad hold 32 consecutive values: the per-32 sum
  const int s4 = quad_sum(sum);
  if (kind >= 0) {
    CM_GEMV_STAMP(kind, 4, 0)
  }
  st_agent64(q8, (uint64_t)words[0] | ((uint64_t)words[1] << 32));
  if ((l & 3) == 0) st_agent32(bs, (uint32_t)s4);
  if (l == 0) st_agent32(d, __float_as_uint(a > 0.0f ? 1.0f / iscale : 0.0f));
}

// Thread t holds values 8t..8t+7 (the one-pass sum's layout); a Q8_K block is one half wave
// (block position 8 l + e for lane l of the half).  smem: the n squares (the sum's fallback)
// + FsLds<512>.  n == 8 * 512.
// (measurement build: stamps of workgroup 0 in g_gemv_stamps[kind][0]: 0 start, 6 squares
// stored, 7 sum of squares, 2 y, 3 block maxima, 4 quants, 5 stores completed, 1 published; of a sample of the other workgroups (every
// ceil(grid / 256)-th): 0 start, 3 flag seen and activation staged, 5 end)
__device__ __forceinline__ void norm_q8k_publish(const float* __restrict__ x, const float* __restrict__ w, int n,
                                                 float eps, float* __restrict__ kd, int8_t* __restrict__ kq,
                                                 int32_t* __restrict__ kbs, uint32_t* slot_set,
                                                 uint32_t* slot_reset, unsigned char* smem, int kind) {
  (void)kind;
  constexpr int C = NQ_C;
  CM_GEMV_STAMP(kind, 0, 0)
  const int tid = threadIdx.x, l = tid & 31;
  float* sq = reinterpret_cast<float*>(smem);
  FsLds<NF_NT>& fs = *reinterpret_cast<FsLds<NF_NT>*>(smem + (size_t)n * 4);
  if (tid == 0) {  // the other kind's slot: its launch has completed
#pragma unroll
    for (int c = 0; c < NF_XCD; ++c) st_agent32(slot_reset + c * NF_STRIDE, 0u);
  }
  // (x and w are read again after the sum, not held across it: the kernel's register count
  // is this workgroup's, and it sets how many GEMV workgroups are resident)
  float tv[C];
#pragma unroll
  for (int u = 0; u < C / 4; ++u) {
    const float4 a = reinterpret_cast<const float4*>(x + tid * C)[u];
    tv[4 * u] = a.x * a.x, tv[4 * u + 1] = a.y * a.y, tv[4 * u + 2] = a.z * a.z, tv[4 * u + 3] = a.w * a.w;
  }
#pragma unroll
  for (int u = 0; u < C / 4; ++u)
    reinterpret_cast<float4*>(sq + tid * C)[u] = make_float4(tv[4 * u], tv[4 * u + 1], tv[4 * u + 2], tv[4 * u + 3]);
  CM_GEMV_STAMP(kind, 6, 0)
  __syncthreads();
  const float ss = inorder_sum_onepass<NF_NT, C>(tv, sq, n, fs, WgBar{}, kind);
  CM_GEMV_STAMP(kind, 7, 0)
  const float scale = 1.0f / sqrtf(ss / (float)n + eps);
  float y[C];
#pragma unroll
  for (int u = 0; u < C / 4; ++u) {
    const float4 a = reinterpret_cast<const float4*>(x + tid * C)[u];
    const float4 b = reinterpret_cast<const float4*>(w + tid * C)[u];
    y[4 * u] = (a.x * scale) * b.x;
    y[4 * u + 1] = (a.y * scale) * b.y;
    y[4 * u + 2] = (a.z * scale) * b.z;
    y[4 * u + 3] = (a.w * scale) * b.w;
  }
  CM_GEMV_STAMP(kind, 2, 0)
  q8k_half_wave_block(y, l, kq + tid * C, kbs + (tid >> 2), kd + (tid >> 5), kind);
  __builtin_amdgcn_s_waitcnt(0);  // this wave's stores have completed
  CM_GEMV_STAMP(kind, 5, 0)
  __syncthreads();
  if (tid == 0) {
#pragma unroll
    for (int c = 0; c < NF_XCD; ++c) st_agent32(slot_set + c * NF_STRIDE, 1u);
  }
  CM_GEMV_STAMP(kind, 1, 0)
}

// q|k (Q4_K) + v (Q6_K) with the attention RMSNorm: grid 1 + g4 + g6 (eight rows per
// workgroup, one per wave, as k_gemv_qk4_v6's workgroups with twice the waves) after the norm
// workgroup; slot `kind` of the flag words (slots: 2 x NF_XCD x NF_STRIDE words).
template <int IT>
__global__ __launch_bounds__(NF_NT, 8) void k_norm_qk4_v6(const float* __restrict__ x, const float* __restrict__ nw,
                                                       float eps, uint32_t* slots, int kind, float* __restrict__ kd,
                                                       int8_t* __restrict__ kq, int32_t* __restrict__ kbs,
                                                       const uint8_t* __restrict__ nib, const uint8_t* __restrict__ hdr,
                                                       int rows4, float* y4, int g4, const uint8_t* __restrict__ ql,
                                                       const uint8_t* __restrict__ qh, const int8_t* __restrict__ scl,
                                                       const uint16_t* __restrict__ dw, int rows6, float* y6, int K) {
  extern __shared__ __align__(16) unsigned char smem[];
  uint32_t* mine = slots + kind * NF_XCD * NF_STRIDE;
  if (blockIdx.x == 0) {
    norm_q8k_publish(x, nw, K, eps, kd, kq, kbs, mine, slots + (1 - kind) * NF_XCD * NF_STRIDE, smem, kind);
    return;
  }
  CM_GEMV_STAMP_SAMPLED(kind, 0, 0)
  const int b = (int)blockIdx.x - 1;
  if (b < g4)
    gemv_q4k_body<IT, 1, NF_NT>(b, nib, hdr, rows4, K, kd, kq, kbs, y4, nullptr, nullptr, nullptr, nullptr, mine,
                                kind);
  else
    gemv_q6k_body<1, NF_NT, true>(b - g4, ql, qh, scl, dw, rows6, K, kd, kq, y6, nullptr, nullptr, nullptr, mine,
                                  kind);
}

// A Q4_K projection (gate|up stacked) with the FFN RMSNorm: grid 1 + the GEMV's workgroups
// (8 RPW rows each).
template <int IT, int RPW>
__global__ __launch_bounds__(NF_NT, 8) void k_norm_gemv_q4k(const float* __restrict__ x, const float* __restrict__ nw,
                                                         float eps, uint32_t* slots, int kind, float* __restrict__ kd,
                                                         int8_t* __restrict__ kq, int32_t* __restrict__ kbs,
                                                         const uint8_t* __restrict__ nib,
                                                         const uint8_t* __restrict__ hdr, int rows, int K, float* y) {
  extern __shared__ __align__(16) unsigned char smem[];
  uint32_t* mine = slots + kind * NF_XCD * NF_STRIDE;
  if (blockIdx.x == 0) {
    norm_q8k_publish(x, nw, K, eps, kd, kq, kbs, mine, slots + (1 - kind) * NF_XCD * NF_STRIDE, smem, kind);
    return;
  }
  CM_GEMV_STAMP_SAMPLED(kind, 0, 0)
  gemv_q4k_body<IT, RPW, NF_NT>((int)blockIdx.x - 1, nib, hdr, rows, K, kd, kq, kbs, y, nullptr, nullptr, nullptr,
                                nullptr, mine, kind);
}

// ---------------------------------------------------------------------------
// Embedding row of a K-quant token table (the block dequantizers of tensor/mod.rs:4682-4703
// Q4_K: (d*sc)*q - dmin*m; :4818-4845 Q6_K: (d*sc)*q), for the token in StepState.
// One thread per value, grid H/256.
__global__ __launch_bounds__(256) void k_embed_q4k(const uint8_t* __restrict__ nib, const uint8_t* __restrict__ hdr,
                                                   int H, const StepState* __restrict__ st, float* __restrict__ out) {
  const int s = blockIdx.x, i = threadIdx.x;
  const int NSB = H >> 8;
  const size_t tok = st->tok;
  const uint8_t* hp = hdr + (tok * NSB + s) * 16;
  const uint8_t* sc = hp + 4;
  const int pair = i >> 6, hi = (i >> 5) & 1, l = i & 31;
  const int idx = 2 * pair + hi;
  int scale, mn;
  if (idx < 4) {
    scale = sc[idx] & 63;
    mn = sc[idx + 4] & 63;
  } else {
    scale = (sc[idx + 4] & 0x0f) | ((sc[idx - 4] >> 6) << 4);
    mn = (sc[idx + 4] >> 4) | ((sc[idx] >> 6) << 4);
  }
  const float d = half_bits_to_float((uint16_t)(hp[0] | (hp[1] << 8)));
  const float dmin = half_bits_to_float((uint16_t)(hp[2] | (hp[3] << 8)));
  const uint8_t byte = nib[(tok * NSB + s) * 128 + pair * 32 + l];
  const int q = hi ? (byte >> 4) : (byte & 0x0f);
  out[s * 256 + i] = (d * (float)scale) * (float)q - dmin * (float)mn;
}

__global__ __launch_bounds__(256) void k_embed_q6k(const uint8_t* __restrict__ ql, const uint8_t* __restrict__ qh,
                                                   const int8_t* __restrict__ scl, const uint16_t* __restrict__ dw,
                                                   int H, const StepState* __restrict__ st, float* __restrict__ out) {
  const int s = blockIdx.x, i = threadIdx.x;
  const int NSB = H >> 8;
  const size_t tok = st->tok;
  const size_t sb = tok * NSB + s;
  const int n = i >> 7, r = i & 127, k = r >> 5, l = r & 31;
  const uint8_t lq = ql[sb * 128 + n * 64 + (k & 1) * 32 + l];
  const uint8_t hq = qh[sb * 64 + n * 32 + l];
  const int lo = (k < 2) ? (lq & 0xf) : (lq >> 4);
  const int q = (lo | (((hq >> (2 * k)) & 3) << 4)) - 32;
  const float d = half_bits_to_float(dw[sb]);
  out[s * 256 + i] = d * (float)scl[sb * 16 + i / 16] * (float)q;
}

// ---------------------------------------------------------------------------
// Q4_K GEMM for prefill chunks and batched verify.  The reference has none: its CPU path
// (and its CUDA path for K-quant layers) prefills one token at a time through the row dot
// (inference.rs:2462-2473); this kernel gives every (token, row) exactly that dot's result:
//   per superblock s: sumi = sum_j sc_j * D_j,  D_j = sum over sub-block j of q4 * q8,
//                     prod = sum_j mn_j * bsum_j   (exact integers)
//   acc = fma(-(y.d * dmin), prod, acc); acc = fma(y.d * d, sumi, acc), s = 0, 1, ...
//   y[t][n] = (resid ? resid[t][n] : 0) + acc
// The integer parts run on the matrix cores: per sub-block (32 values) one
// v_mfma_i32_16x16x32_i8 gives D_j for a 16-token x 16-row fragment (the activation is the A
// operand, so a lane's 4 outputs are 4 tokens of one row and need that row's scales only),
// scaled by sc_j on the vector ALUs; prod comes from a second MFMA per sub-block whose row
// operand is mn_j repeated (sum_k q8[k] * mn_j = mn_j * bsum_j), accumulated over the
// superblock.  Lane l of a fragment supplies token / row l % 16, values 8*(l/16) .. +7 of
// the sub-block; 8 nibble bytes of a row give the row operands of both sub-blocks of a
// 64-value chunk (low nibbles: sub-block 2c, high: 2c + 1).
// Workgroup: 8 waves over a 64-row x 64-token tile, each wave 16 rows x 32 tokens (1 x 2
// fragments: a row's nibbles are unpacked once per 32 tokens; 24 accumulators per lane, so
// two workgroups share a CU at four waves per SIMD).
// One superblock per step: 128 nibble bytes of every row and 256 activation bytes of every
// token, loaded one step ahead into registers, then into a double-buffered LDS tile
// [chunk or sub-block][8-byte piece][row or token] (65-entry planes: no bank conflicts);
// headers and activation scales go the same way one step ahead.
// Tiles are dealt so that each XCD runs a contiguous range, token tiles innermost.
// K % 256 == 0; y may alias resid (same row stride ldy).
typedef uint16_t u16x2_t __attribute__((ext_vector_type(2)));
constexpr int G4_NT = 512;
constexpr int G4_RN = 64;
constexpr int G4_RT = 64;
constexpr int G4_PS = 65;
__host__ __device__ inline int gemm_q4k_tiles(int N, int T) {
  return ((N + G4_RN - 1) / G4_RN) * ((T + G4_RT - 1) / G4_RT);
}
__host__ __device__ inline int gemm_q4k_grid(int N, int T) { return ((gemm_q4k_tiles(N, T) + 7) / 8) * 8; }

__global__ __launch_bounds__(G4_NT, 4) void k_gemm_q4k(const uint8_t* __restrict__ nib,
                                                       const uint8_t* __restrict__ hdr, int N, int K,
                                                       const float* __restrict__ xd,
                                                       const int8_t* __restrict__ xq, int T, float* y, int ldy,
                                                       const float* resid) {
  // 16-byte units: weights [buf][64-value chunk][half][row] (chunk bytes 16 h .. 16 h + 15),
  // activations [buf][sub-block][half][token] (positions 16 h .. 16 h + 15); 65-unit planes
  __shared__ __align__(16) uint4 sw[2][4][2][G4_PS];
  __shared__ __align__(16) uint4 sx[2][8][2][G4_PS];
  __shared__ __align__(16) float sxd[2][G4_RT];       // activation scales: [buf][token]
  const int NSB = K >> 8;
  const int ntt = (T + G4_RT - 1) / G4_RT;
  const int tiles = gemm_q4k_tiles(N, T);
  const int per = (tiles + 7) >> 3;
  const int L = (int)(blockIdx.x & 7) * per + (int)(blockIdx.x >> 3);
  if (L >= tiles) return;
  const int n_base = (L / ntt) * G4_RN, t_base = (L % ntt) * G4_RT;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int r = lane & 15, g = lane >> 4;
  const int wn = (wave & 3) * 16, wt = (wave >> 2) * 32;

  // global -> register loads of one superblock step (32-bit offsets from the matrix bases)
  const int wrow = tid >> 3, wc = tid & 7;   // weights: row wrow, 16 bytes at wc * 16
  const int xrow = tid >> 4, xc = tid & 15;  // activations: tokens xrow + 32 j, 16 bytes at xc * 16
  const uint32_t ow = (uint32_t)min(n_base + wrow, N - 1) * (uint32_t)(K >> 1) + wc * 16;
  uint32_t ox[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) ox[j] = (uint32_t)min(t_base + xrow + 32 * j, T - 1) * (uint32_t)K + xc * 16;
  const uint32_t oh = (uint32_t)min(n_base + wn + r, N - 1) * (uint32_t)NSB;
  const float* gxd = xd + (size_t)min(t_base + (tid & (G4_RT - 1)), T - 1) * NSB;  // (threads < 64)
  uint4 rw, rx0, rx1, rh;
  float rxd = 0.0f;
  auto gload = [&](int s) {
    if (tid < G4_RT) rxd = gxd[s];
    rw = *reinterpret_cast<const uint4*>(nib + (ow + (uint32_t)s * 128u));
    rx0 = *reinterpret_cast<const uint4*>(xq + (ox[0] + (uint32_t)s * 256u));
    rx1 = *reinterpret_cast<const uint4*>(xq + (ox[1] + (uint32_t)s * 256u));
    rh = reinterpret_cast<const uint4*>(hdr)[oh + (uint32_t)s];
  };
  auto lds_put = [&](int buf) {
    sw[buf][wc >> 1][wc & 1][wrow] = make_uint4(rw.x, rw.y, rw.z, rw.w);
    sx[buf][xc >> 1][xc & 1][xrow] = make_uint4(rx0.x, rx0.y, rx0.z, rx0.w);
    sx[buf][xc >> 1][xc & 1][xrow + 32] = make_uint4(rx1.x, rx1.y, rx1.z, rx1.w);
    if (tid < G4_RT) sxd[buf][tid] = rxd;
  };

  float acc[2][4];  // [token fragment][token 4g + i]
#pragma unroll
  for (int tf = 0; tf < 2; ++tf)
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[tf][i] = 0.0f;

  const uint32_t K1 = 0x3f3f3f3fu, K2 = 0x0f0f0f0fu, K3 = 0x03030303u;
  auto step = [&](int buf, const uint4& hd) {
    // the row's 6-bit scales and mins, 4 per dword (sub-blocks 0-3, 4-7)
    uint32_t scp[2], mnp[2];
    scp[0] = hd.y & K1;
    scp[1] = (hd.w & K2) | (((hd.y >> 6) & K3) << 4);
    mnp[0] = hd.z & K1;
    mnp[1] = ((hd.w >> 4) & K2) | (((hd.z >> 6) & K3) << 4);
    // sumi = sum_j sc_j D_j as one K = 256 integer dot per plane: sc_j = 8 sh_j + sl_j (3 bits
    // each), so sh_j * q and sl_j * q (<= 105) are int8 weights: sumi = 8 (H . x) + (L . x);
    // prod = sum_k mn_j(k) x_k.  Per 64-value chunk one v_mfma_i32_16x16x64_i8 per plane and
    // token fragment; lane (r, g) supplies positions 16 (g % 2) .. +15 of sub-block
    // 2 chunk + g / 2 (the high nibbles for odd sub-blocks), the same positions of x.
    const int gb = g >> 1, gh = g & 1;
    v4i_t ch[2], cl[2], cm[2];
#pragma unroll
    for (int tf = 0; tf < 2; ++tf) ch[tf] = cl[tf] = cm[tf] = v4i_t{0, 0, 0, 0};
#pragma unroll
    for (int c4 = 0; c4 < 4; ++c4) {
      __builtin_amdgcn_sched_barrier(0);  // one 64-value chunk at a time (register pressure)
      const int sh8 = 16 * (c4 & 1) + 8 * gb;  // byte of sub-block 2 c4 + gb in scp / mnp[c4 / 2]
      const uint32_t sc = (scp[c4 >> 1] >> sh8) & 0xffu, mn = (mnp[c4 >> 1] >> sh8) & 0xffu;
      const u16x2_t shp = {(uint16_t)(sc >> 3), (uint16_t)(sc >> 3)}, slp = {(uint16_t)(sc & 7u), (uint16_t)(sc & 7u)};
      const uint32_t mrep = __builtin_amdgcn_perm(0u, mn, 0u);  // mn's byte 0 (selector 0: second operand) x 4
      const uint4 w = sw[buf][c4][gh][wn + r];
      const uint32_t ns = 4 * gb;
      const uint32_t nb[4] = {(w.x >> ns) & K2, (w.y >> ns) & K2, (w.z >> ns) & K2, (w.w >> ns) & K2};
      v4i_t wh, wl;
#pragma unroll
      for (int u = 0; u < 4; ++u) {  // bytes <= 15 times <= 7: no carry between the bytes of a half
        const u16x2_t q = __builtin_bit_cast(u16x2_t, nb[u]);
        wh[u] = __builtin_bit_cast(int, q * shp);
        wl[u] = __builtin_bit_cast(int, q * slp);
      }
      const v4i_t wm = v4i_t{(int)mrep, (int)mrep, (int)mrep, (int)mrep};
#pragma unroll
      for (int tf = 0; tf < 2; ++tf) {
        const v4i_t xa = __builtin_bit_cast(v4i_t, sx[buf][2 * c4 + gb][gh][wt + 16 * tf + r]);
        ch[tf] = __builtin_amdgcn_mfma_i32_16x16x64_i8(xa, wh, ch[tf], 0, 0, 0);
        cl[tf] = __builtin_amdgcn_mfma_i32_16x16x64_i8(xa, wl, cl[tf], 0, 0, 0);
        cm[tf] = __builtin_amdgcn_mfma_i32_16x16x64_i8(xa, wm, cm[tf], 0, 0, 0);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    const float dw = half_bits_to_float((uint16_t)(hd.x & 0xffffu));
    const float dmw = half_bits_to_float((uint16_t)(hd.x >> 16));
#pragma unroll
    for (int tf = 0; tf < 2; ++tf) {
      const float4 y4 = *reinterpret_cast<const float4*>(&sxd[buf][wt + 16 * tf + 4 * g]);
      const float ydv[4] = {y4.x, y4.y, y4.z, y4.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        acc[tf][i] = fmaf(-(ydv[i] * dmw), (float)cm[tf][i], acc[tf][i]);
        acc[tf][i] = fmaf(ydv[i] * dw, (float)(ch[tf][i] * 8 + cl[tf][i]), acc[tf][i]);
      }
    }
  };

  gload(0);
  lds_put(0);
  __syncthreads();
  for (int sb = 0; sb < NSB; ++sb) {
    const int buf = sb & 1;
    const uint4 hd = rh;
    if (sb + 1 < NSB) gload(sb + 1);
    step(buf, hd);
    if (sb + 1 < NSB) lds_put(buf ^ 1);
    __syncthreads();
  }
  const int n = n_base + wn + r;
#pragma unroll
  for (int tf = 0; tf < 2; ++tf)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int t = t_base + wt + 16 * tf + 4 * g + i;
      if (t < T && n < N) {
        const size_t o = (size_t)t * ldy + n;
        y[o] = resid ? resid[o] + acc[tf][i] : acc[tf][i];
      }
    }
}

// ---------------------------------------------------------------------------
// Q6_K GEMV over T tokens at once (speculative verify, prefill chunks): each token's result
// is k_gemv_q6k's, in the same order (the Q6_K decode dot of inference.rs:19148-19195); the
// weights of a lane's 64-value unit are loaded and split into their 8 position classes once
// and used for every token.  The activations stay in LDS as raw Q8_K quants (the class
// pairs are formed per use).  y[t * ldy + row] (+ resid, same stride).
// Dynamic LDS: gemv_q6k_multi_lds_bytes(K, T).
constexpr int Q6M_MAX = 8;
constexpr int Q6M_RPW = 1;
constexpr int Q6M_ROWS = 4 * Q6M_RPW;
__host__ __device__ inline size_t q6m_terms_offset(int K, int T) {
  return ((size_t)T * K + (size_t)T * (K / 256) * 4 + 15) & ~(size_t)15;
}
__host__ __device__ inline size_t gemv_q6k_multi_lds_bytes(int K, int T) {
  return q6m_terms_offset(K, T) + (size_t)Q6M_ROWS * T * (K / 256) * 32;
}

__global__ __launch_bounds__(KQ_NT) void k_gemv_q6k_multi(const uint8_t* __restrict__ ql,
                                                          const uint8_t* __restrict__ qh,
                                                          const int8_t* __restrict__ scl,
                                                          const uint16_t* __restrict__ dw, int rows, int K,
                                                          const float* __restrict__ yd,
                                                          const int8_t* __restrict__ yq, int T, float* y, int ldy,
                                                          const float* resid) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int NSB = K >> 8, NU = K >> 6;
  int8_t* xq = reinterpret_cast<int8_t*>(smem);                  // [T][K]
  float* xd = reinterpret_cast<float*>(smem + (size_t)T * K);    // [T][NSB]
  float* terms = reinterpret_cast<float*>(smem + q6m_terms_offset(K, T));  // [row][t][s][class]
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int row0 = blockIdx.x * Q6M_ROWS;
  for (int c = tid; c < (T * K) >> 4; c += KQ_NT) reinterpret_cast<int4*>(xq)[c] = reinterpret_cast<const int4*>(yq)[c];
  for (int i = tid; i < T * NSB; i += KQ_NT) xd[i] = yd[i];
  __syncthreads();
  const uint32_t M4 = 0x0f0f0f0fu, M2 = 0x03030303u;
#pragma unroll
  for (int k = 0; k < Q6M_RPW; ++k) {
    const int rl = wave * Q6M_RPW + k;
    const int row = min(row0 + rl, rows - 1);
    const uint8_t* qlr = ql + (size_t)row * (K >> 1);
    const uint8_t* qhr = qh + (size_t)row * (K >> 2);
    const int8_t* scr = scl + (size_t)row * NSB * 16;
    for (int u0 = 0; u0 < NU; u0 += 64) {
      const int u = u0 + lane;
      const bool valid = u < NU;  // uniform per 4-lane superblock group (NU % 4 == 0)
      const int uu = min(u, NU - 1);
      const int s = uu >> 2, n = (uu >> 1) & 1, q0 = (uu & 1) * 16;
      const uint4 l0 = ld_stream(reinterpret_cast<const uint4*>(qlr + s * 128 + n * 64 + q0));
      const uint4 l1 = ld_stream(reinterpret_cast<const uint4*>(qlr + s * 128 + n * 64 + 32 + q0));
      const uint4 hh = ld_stream(reinterpret_cast<const uint4*>(qhr + s * 64 + n * 32 + q0));
      const uint4 scv = ld_stream(reinterpret_cast<const uint4*>(scr + s * 16));
      const float dsb = half_bits_to_float(dw[(size_t)row * NSB + s]);
      const uint32_t L0[4] = {l0.x, l0.y, l0.z, l0.w}, L1[4] = {l1.x, l1.y, l1.z, l1.w};
      const uint32_t HH[4] = {hh.x, hh.y, hh.z, hh.w};
      const uint32_t SC[4] = {scv.x, scv.y, scv.z, scv.w};
      // the unit's weights as class pairs (bytes 2-3 = -32: one dot4 gives sum (w - 32) * q)
      uint32_t wp[4][8];
      int scg[4];
      int jg[4];
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        const int j = n * 8 + (q0 >> 4) + 2 * kk;
        jg[kk] = j;
        scg[kk] = (int)(int8_t)((SC[j >> 2] >> (8 * (j & 3))) & 0xff);
        uint32_t v[4];
#pragma unroll
        for (int t4 = 0; t4 < 4; ++t4) {
          const uint32_t lq = (kk & 1) ? L1[t4] : L0[t4];
          const uint32_t lo = (kk < 2) ? (lq & M4) : ((lq >> 4) & M4);
          v[t4] = lo | (((HH[t4] >> (2 * kk)) & M2) << 4);
        }
#pragma unroll
        for (int l = 0; l < 8; ++l) {
          const uint32_t bl = l & 3;
          wp[kk][l] = __builtin_amdgcn_perm(v[(l >> 2) + 2], v[l >> 2], bl | ((4 + bl) << 8) | (0x0c << 16) | (0x0cu << 24)) |
                      0xe0e00000u;
        }
      }
      for (int t = 0; t < T; ++t) {
        int aux[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
          const uint4 xg = *reinterpret_cast<const uint4*>(xq + (size_t)t * K + s * 256 + 16 * jg[kk]);
          const uint32_t X[4] = {xg.x, xg.y, xg.z, xg.w};
#pragma unroll
          for (int l = 0; l < 8; ++l) {
            const uint32_t bl = l & 3;
            // bytes (q[l], q[8 + l], q[l], q[8 + l]) of the 16-value group
            const uint32_t xpair = __builtin_amdgcn_perm(X[(l >> 2) + 2], X[l >> 2], bl | ((4 + bl) << 8) | (bl << 16) | ((4 + bl) << 24));
            aux[l] += scg[kk] * __builtin_amdgcn_sdot4((int)wp[kk][l], (int)xpair, 0, false);
          }
        }
#pragma unroll
        for (int l = 0; l < 8; ++l) aux[l] = quad_sum(aux[l]);
        if (valid && (uu & 3) == 0) {
          const float d = dsb * xd[t * NSB + s];
          float* tp = terms + (((size_t)rl * T + t) * NSB + s) * 8;
          *reinterpret_cast<float4*>(tp) = make_float4(d * (float)aux[0], d * (float)aux[1], d * (float)aux[2],
                                                       d * (float)aux[3]);
          *reinterpret_cast<float4*>(tp + 4) = make_float4(d * (float)aux[4], d * (float)aux[5], d * (float)aux[6],
                                                           d * (float)aux[7]);
        }
      }
    }
  }
  __syncthreads();
  // 8 lanes per (row, token): the 8 class chains, then the left fold by the first
  for (int base = 0; base < Q6M_ROWS * T * 8; base += KQ_NT) {
    const int id = base + tid;
    const int pair = id >> 3, l = id & 7;
    const int rl = pair / T, t = pair - rl * T;
    float sl = 0.0f;
    if (pair < Q6M_ROWS * T) {
      const float* tp = terms + ((size_t)rl * T + t) * NSB * 8 + l;
      for (int s = 0; s < NSB; ++s) sl += tp[s * 8];
    }
    float acc = -0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) acc += __shfl(sl, (lane & ~7) + i);
    const int row = row0 + rl;
    if (l == 0 && pair < Q6M_ROWS * T && row < rows) {
      const size_t o = (size_t)t * ldy + row;
      y[o] = resid ? resid[o] + acc : acc;
    }
  }
}

// ---------------------------------------------------------------------------
// Q6_K GEMM for prefill chunks: each (token, row) is k_gemv_q6k's result (the Q6_K decode dot
// of inference.rs:19148-19195):  aux[l] = sum over positions p = l (mod 8) of
// sc[p/16] * q8[p] * w[p] per superblock (exact integers), sums[l] += (f16(d) * y.d) * aux[l]
// in superblock order, result = left fold of sums[0..8] from -0.0.
// On the matrix cores, per 16-value scale group and token pair: one v_mfma_i32_16x16x32_i8
// whose K holds the group's 16 positions (the other 16 are zero) and whose 16 columns are
// (token, class) pairs -- column (t, l) carries q8[t][p] only at the group's two positions
// of class l -- so each output is one (group, class) partial sum w[l] q[l] + w[8+l] q[8+l],
// scaled by that group's sc on the vector ALUs and accumulated into aux.
// Workgroup: 4 waves x 16 rows, 16 tokens; one superblock of the 64 rows' ql/qh/scales and
// the 16 tokens' quants staged in LDS per step.  K % 256 == 0; y may alias resid.
constexpr int G6_NT = 256;
constexpr int G6_RN = 64;
constexpr int G6_RT = 16;

__global__ __launch_bounds__(G6_NT) void k_gemm_q6k(const uint8_t* __restrict__ ql, const uint8_t* __restrict__ qh,
                                                    const int8_t* __restrict__ scl, const uint16_t* __restrict__ dw,
                                                    int N, int K, const float* __restrict__ xd,
                                                    const int8_t* __restrict__ xq, int T, float* y, int ldy,
                                                    const float* resid) {
  __shared__ __align__(16) uint8_t sql[G6_RN][128];
  __shared__ __align__(16) uint8_t sqh[G6_RN][64];
  __shared__ __align__(16) int8_t ssc[G6_RN][16];
  __shared__ __align__(16) int8_t sxq[G6_RT][256];
  __shared__ float sd[G6_RN], sxd[G6_RT];
  const int NSB = K >> 8;
  const int n_base = blockIdx.x * G6_RN, t_base = blockIdx.y * G6_RT;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int r = lane & 15, k8 = lane >> 4;  // operand row / column, 8-position slice of K
  const int tl = r >> 3, cls = r & 7;       // this lane's output column: token of the pair, class
  int aux[8][4];
  float sums[8][4];
#pragma unroll
  for (int tp = 0; tp < 8; ++tp)
#pragma unroll
    for (int i = 0; i < 4; ++i) sums[tp][i] = 0.0f;
  const uint32_t M4 = 0x0f0f0f0fu, M2 = 0x03030303u;
  for (int s = 0; s < NSB; ++s) {
    __syncthreads();  // the previous superblock's tile is consumed
    {  // stage: 64 rows x (128 + 64 + 16) bytes, 16 tokens x 256 bytes, scales
      const int row = tid >> 2, part = tid & 3;  // 4 threads per row
      const size_t gr = (size_t)min(n_base + row, N - 1);
      const uint4* qlp = reinterpret_cast<const uint4*>(ql + gr * (K >> 1) + (size_t)s * 128);
      const uint4* qhp = reinterpret_cast<const uint4*>(qh + gr * (K >> 2) + (size_t)s * 64);
      reinterpret_cast<uint4*>(sql[row])[part * 2] = qlp[part * 2];
      reinterpret_cast<uint4*>(sql[row])[part * 2 + 1] = qlp[part * 2 + 1];
      reinterpret_cast<uint4*>(sqh[row])[part] = qhp[part];
      if (part == 0) {
        reinterpret_cast<uint4*>(ssc[row])[0] = *reinterpret_cast<const uint4*>(scl + (gr * NSB + s) * 16);
        sd[row] = half_bits_to_float(dw[gr * NSB + s]);
      }
      const int tok = tid >> 4, piece = tid & 15;  // 16 threads per token
      const size_t gt = (size_t)min(t_base + tok, T - 1);
      reinterpret_cast<uint4*>(sxq[tok])[piece] =
          *reinterpret_cast<const uint4*>(xq + gt * K + (size_t)s * 256 + piece * 16);
      if (piece == 0) sxd[tok] = xd[gt * NSB + s];
    }
    __syncthreads();
#pragma unroll
    for (int tp = 0; tp < 8; ++tp)
#pragma unroll
      for (int i = 0; i < 4; ++i) aux[tp][i] = 0;
    const int arow = wave * 16 + r;
#pragma unroll 2
    for (int g = 0; g < 16; ++g) {
      const int n = g >> 3, kk = (g & 7) >> 1, q0 = (g & 1) * 16;
      // A: the row's weights at positions 16 g + 8 k8 .. +7 (k8 < 2), as int8 (q - 32)
      long av = 0;
      if (k8 < 2) {
        const uint2 lq = *reinterpret_cast<const uint2*>(&sql[arow][n * 64 + (kk & 1) * 32 + q0 + 8 * k8]);
        const uint2 hq = *reinterpret_cast<const uint2*>(&sqh[arow][n * 32 + q0 + 8 * k8]);
        uint32_t w[2];
        const uint32_t L[2] = {lq.x, lq.y}, H[2] = {hq.x, hq.y};
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const uint32_t lo = (kk < 2) ? (L[h] & M4) : ((L[h] >> 4) & M4);
          const uint32_t v = lo | (((H[h] >> (2 * kk)) & M2) << 4);  // 0..63 per byte
          w[h] = (v & 0x1f1f1f1fu) | ((~v & 0x20202020u) * 7u);      // v - 32 per byte
        }
        av = (long)(((uint64_t)w[1] << 32) | w[0]);
      }
      int scr[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) scr[i] = ssc[wave * 16 + 4 * k8 + i][g];
#pragma unroll
      for (int tp = 0; tp < 8; ++tp) {
        // B: column (token 2 tp + tl, class cls): its quant at position 16 g + 8 k8 + cls only
        long bv = 0;
        if (k8 < 2) {
          const uint32_t q = (uint8_t)sxq[2 * tp + tl][16 * g + 8 * k8 + cls];
          bv = (long)((uint64_t)q << (8 * cls));
        }
        const v4i_t c = __builtin_amdgcn_mfma_i32_16x16x32_i8(av, bv, v4i_t{0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
        for (int i = 0; i < 4; ++i) aux[tp][i] += scr[i] * c[i];
      }
    }
#pragma unroll
    for (int tp = 0; tp < 8; ++tp) {
      const float ydv = sxd[2 * tp + tl];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float d = sd[wave * 16 + 4 * k8 + i] * ydv;
        sums[tp][i] += d * (float)aux[tp][i];
      }
    }
  }
  // left fold of the 8 class chains (lanes 8 (lane / 8) .. +7), from -0.0
#pragma unroll
  for (int tp = 0; tp < 8; ++tp)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float acc = -0.0f;
#pragma unroll
      for (int c = 0; c < 8; ++c) acc += __shfl(sums[tp][i], (lane & ~7) + c);
      const int row = n_base + wave * 16 + 4 * k8 + i, t = t_base + 2 * tp + tl;
      if (cls == 0 && row < N && t < T) {
        const size_t o = (size_t)t * ldy + row;
        y[o] = resid ? resid[o] + acc : acc;
      }
    }
}

// ---------------------------------------------------------------------------
// Q6_K GEMM, class-major form (prefill chunks).  The Q6_K dot's integer part per superblock,
// aux[l] = sum over the 32 positions p = 8 j + l (j = 0..31) of sc[p/16] * w[p] * q8[p]
// (inference.rs:19148-19195; exact, so any summation order gives it), is a K = 32 dot once
// the weights carry their scale: w'[p] = sc[p/16] * w[p] lies in [-4096, 4096], so it is stored
// as two int8 planes w' = 128 h + lo (h in [-32, 32], lo in [-64, 63]) and aux[l] =
// 128 (h . q8) + (lo . q8): two v_mfma_i32_16x16x32_i8 per class, K = j.  Then per class and
// output sums[l] += (f16(d) * y.d) * float(aux[l]) in superblock order, and the result is the
// left fold of sums[0..8] from -0.0 -- k_gemv_q6k's arithmetic, in its order.
// The eight class chains are independent, so wave l of a workgroup folds class l of its
// 32-row x 32-token tile (2 x 2 MFMA fragments, 16 chains per lane) and the class sums meet in
// LDS for the final fold: 8 waves per tile where one wave per tile holding all classes would
// leave the SIMDs issue-bound at one wave each.
// Both operands sit in HBM in the order the waves read them from LDS, so a superblock step
// stages each tile with one straight 16-byte copy per thread:
//   weights (k_q6k_w2, once per matrix): [32-row tile][superblock] blocks of 16 KB, each
//     [class l][plane h | lo][row half][k group g][row r][j % 8] (rows padded to 32 with zeros);
//   activations (k_q8k_classmajor, once per call): [32-token tile][superblock] blocks of 8 KB,
//     [class l][token half][k group g][token r][j % 8], j = 8 g + (j % 8).
constexpr int Q6G_NT = 512;   // 8 waves, wave l folds position class l
constexpr int Q6G_R = 32;     // rows and tokens per tile
constexpr int Q6G_WB = 16384; // weight-plane bytes per (32-row tile, superblock)
constexpr int Q6G_XB = 8192;  // activation bytes per (32-token tile, superblock)
constexpr int Q6G_DP = 36;    // floats per token row of the LDS scale-product and class-sum tables
constexpr int Q6G_LDS = 2 * (Q6G_WB + Q6G_XB) + 2 * Q6G_R * Q6G_DP * 4;
static_assert(8 * Q6G_R * Q6G_DP * 4 <= Q6G_LDS, "class sums fit the staging LDS");
__host__ __device__ inline size_t q6g_planes_bytes(int N, int K) {
  return (size_t)((N + Q6G_R - 1) / Q6G_R) * (K / 256) * Q6G_WB;
}
__host__ __device__ inline size_t q6g_act_bytes(int T, int K) {
  return (size_t)((T + Q6G_R - 1) / Q6G_R) * (K / 256) * Q6G_XB;
}
__host__ __device__ inline int gemm_q6k2_tiles(int N, int T) {
  return ((N + Q6G_R - 1) / Q6G_R) * ((T + Q6G_R - 1) / Q6G_R);
}
__host__ __device__ inline int gemm_q6k2_grid(int N, int T) { return ((gemm_q6k2_tiles(N, T) + 7) / 8) * 8; }

// grid (N rounded up to 32, K / 256), 256 threads: thread p of workgroup (row, s) writes
// position p's h and lo (zeros for the padding rows >= N).
__global__ __launch_bounds__(256) void k_q6k_w2(const uint8_t* __restrict__ ql, const uint8_t* __restrict__ qh,
                                                const int8_t* __restrict__ scl, int N, int K,
                                                int8_t* __restrict__ w2) {
  const int s = blockIdx.y, p = threadIdx.x, NSB = K >> 8;
  const int row = blockIdx.x;
  int h = 0, lo = 0;
  if (row < N) {
    const uint8_t* l8 = ql + (size_t)row * (K >> 1) + (size_t)s * 128;
    const uint8_t* h8 = qh + (size_t)row * (K >> 2) + (size_t)s * 64;
    const int n = p >> 7, q = p & 127, l32 = q & 31, quarter = q >> 5;  // (q6_k_values' order)
    const uint8_t lq = l8[64 * n + l32 + (quarter & 1) * 32];
    const int lo4 = (quarter < 2) ? (lq & 0xf) : (lq >> 4);
    const int hi2 = (h8[32 * n + l32] >> (2 * quarter)) & 3;
    const int w = (lo4 | (hi2 << 4)) - 32;
    const int wp = (int)scl[((size_t)row * NSB + s) * 16 + (p >> 4)] * w;
    h = (wp + 64) >> 7;  // floor((w' + 64) / 128): w' = 128 h + lo, lo in [-64, 63]
    lo = wp - 128 * h;
  }
  const int cls = p & 7, j = p >> 3, g = j >> 3, b = j & 7, rf = (row >> 4) & 1, r = row & 15;
  int8_t* o = w2 + ((size_t)(row / Q6G_R) * NSB + s) * Q6G_WB;
  o[(((cls * 2 + 0) * 2 + rf) * 4 + g) * 128 + r * 8 + b] = (int8_t)h;
  o[(((cls * 2 + 1) * 2 + rf) * 4 + g) * 128 + r * 8 + b] = (int8_t)lo;
}

// bytes b of a0..a3 as one dword (a0's in byte 0)
template <int B>
__device__ __forceinline__ uint32_t byte_col4(uint32_t a0, uint32_t a1, uint32_t a2, uint32_t a3) {
  constexpr uint32_t s01 = (uint32_t)B | ((4u + B) << 8) | (0x0cu << 16) | (0x0cu << 24);
  constexpr uint32_t s23 = 0x0cu | (0x0cu << 8) | ((uint32_t)B << 16) | ((4u + B) << 24);
  return __builtin_amdgcn_perm(a1, a0, s01) | __builtin_amdgcn_perm(a3, a2, s23);
}

// Q8_K quants [T][K] -> the class-major blocks above (zeros for the padding tokens >= T):
// thread (tile, superblock, g, token of the tile) moves positions 64 g .. 64 g + 63 of one
// token, an 8 x 8 byte transpose (position 64 g + 8 i + l is class l's j = 8 g + i).
__global__ __launch_bounds__(256) void k_q8k_classmajor(const int8_t* __restrict__ xq, int T, int K,
                                                        int8_t* __restrict__ xt) {
  const int NSB = K >> 8;
  const size_t id = (size_t)blockIdx.x * 256 + threadIdx.x;
  const size_t total = (size_t)((T + Q6G_R - 1) / Q6G_R) * NSB * 128;
  if (id >= total) return;
  const int rr = (int)(id & 31), g = (int)((id >> 5) & 3);
  const size_t rest = id >> 7;
  const int s = (int)(rest % NSB), tt = (int)(rest / NSB);
  const int tok = tt * Q6G_R + rr;
  uint4 v[4] = {};
  if (tok < T) {
    const uint4* src = reinterpret_cast<const uint4*>(xq + (size_t)tok * K + (size_t)s * 256 + 64 * g);
#pragma unroll
    for (int u = 0; u < 4; ++u) v[u] = src[u];
  }
  // d[2 i] = positions 64 g + 8 i .. +3, d[2 i + 1] = +4 .. +7
  const uint32_t d[16] = {v[0].x, v[0].y, v[0].z, v[0].w, v[1].x, v[1].y, v[1].z, v[1].w,
                          v[2].x, v[2].y, v[2].z, v[2].w, v[3].x, v[3].y, v[3].z, v[3].w};
  uint2* o = reinterpret_cast<uint2*>(xt + ((size_t)tt * NSB + s) * Q6G_XB) + (rr >> 4) * 64 + g * 16 + (rr & 15);
#define CM_Q6T(C)                                                                                               \
  o[(C) * 128] = make_uint2(byte_col4<(C) & 3>(d[(C) >> 2], d[2 + ((C) >> 2)], d[4 + ((C) >> 2)], d[6 + ((C) >> 2)]), \
                            byte_col4<(C) & 3>(d[8 + ((C) >> 2)], d[10 + ((C) >> 2)], d[12 + ((C) >> 2)],           \
                                               d[14 + ((C) >> 2)]));
  CM_Q6T(0) CM_Q6T(1) CM_Q6T(2) CM_Q6T(3) CM_Q6T(4) CM_Q6T(5) CM_Q6T(6) CM_Q6T(7)
#undef CM_Q6T
}

// y[t * ldy + n] (+ resid, same stride) for N % 4 == 0, ldy % 4 == 0; w2 and xt in the
// layouts above; grid gemm_q6k2_grid(N, T), Q6G_NT threads.
__global__ __launch_bounds__(Q6G_NT, 4) void k_gemm_q6k2(const int8_t* __restrict__ w2,
                                                         const uint16_t* __restrict__ dw, int N, int K,
                                                         const float* __restrict__ xd,
                                                         const int8_t* __restrict__ xt, int T, float* y, int ldy,
                                                         const float* resid) {
  // buffer b: weights at b * WB, activations at 2 WB + b * XB, scale products (f16(d) * y.d,
  // [token][row]) after both; the class sums [class][token][row] reuse it all at the end
  __shared__ __align__(16) unsigned char smem[Q6G_LDS];
  const int NSB = K >> 8;
  const int ntt = (T + Q6G_R - 1) / Q6G_R;
  const int tiles = gemm_q6k2_tiles(N, T);
  const int per = (tiles + 7) >> 3;
  const int L = (int)(blockIdx.x & 7) * per + (int)(blockIdx.x >> 3);  // contiguous tiles per XCD
  if (L >= tiles) return;
  const int rt = L / ntt, tt = L % ntt;
  const int tid = threadIdx.x, cls = tid >> 6, lane = tid & 63, r = lane & 15, g = lane >> 4;
  const uint4* gw = reinterpret_cast<const uint4*>(w2 + (size_t)rt * NSB * Q6G_WB);
  const uint4* gx = reinterpret_cast<const uint4*>(xt + (size_t)tt * NSB * Q6G_XB);
  // thread tid forms the scale products of token tid / 16, rows 2 (tid % 16) and + 1
  const int dtok = tid >> 4, drow = 2 * (tid & 15);
  const uint16_t* gd0 = dw + (size_t)min(rt * Q6G_R + drow, N - 1) * NSB;
  const uint16_t* gd1 = dw + (size_t)min(rt * Q6G_R + drow + 1, N - 1) * NSB;
  const float* gyd = xd + (size_t)min(tt * Q6G_R + dtok, T - 1) * NSB;
  // the tiles of the next two steps, held raw in registers (set j % 2 for step j) until they
  // are stored: a step's loads are issued two steps before its tile is folded, and the f16
  // scales are converted only at the store, so no use of a load waits inside its own step
  uint4 rw0_0, rw1_0, rx_0, rw0_1, rw1_1, rx_1;
  uint16_t rh0_0, rh1_0, rh0_1, rh1_1;
  float ryd_0, ryd_1;
#define CM_Q6G_LOAD(S, P)                                  \
  rw0_##P = gw[(size_t)(S) * (Q6G_WB / 16) + tid];         \
  rw1_##P = gw[(size_t)(S) * (Q6G_WB / 16) + Q6G_NT + tid]; \
  rx_##P = gx[(size_t)(S) * (Q6G_XB / 16) + tid];          \
  rh0_##P = gd0[S];                                        \
  rh1_##P = gd1[S];                                        \
  ryd_##P = gyd[S];
#define CM_Q6G_STORE(P)                                                                                     \
  {                                                                                                         \
    uint4* sw_ = reinterpret_cast<uint4*>(smem + (P) * Q6G_WB);                                           \
    sw_[tid] = rw0_##P;                                                                                     \
    sw_[Q6G_NT + tid] = rw1_##P;                                                                            \
    reinterpret_cast<uint4*>(smem + 2 * Q6G_WB + (P) * Q6G_XB)[tid] = rx_##P;                             \
    float* sdd_ = reinterpret_cast<float*>(smem + 2 * (Q6G_WB + Q6G_XB)) + (P) * Q6G_R * Q6G_DP;          \
    *reinterpret_cast<float2*>(sdd_ + dtok * Q6G_DP + drow) = make_float2(                                 \
        half_bits_to_float(rh0_##P) * ryd_##P, half_bits_to_float(rh1_##P) * ryd_##P);                     \
  }

  float sums[2][2][4];  // [row half][token half][i]: rows 16 rf + 4 g + i, token 16 tf + r
#pragma unroll
  for (int rf = 0; rf < 2; ++rf)
#pragma unroll
    for (int tf = 0; tf < 2; ++tf)
#pragma unroll
      for (int i = 0; i < 4; ++i) sums[rf][tf][i] = 0.0f;

  // fold of LDS buffer p: 8 MFMAs, then the 16 chains in superblock order
  auto fold = [&](int p) __attribute__((always_inline)) {
    const uint2* sw = reinterpret_cast<const uint2*>(smem + p * Q6G_WB) + cls * 256 + g * 16 + r;
    const uint2* sx = reinterpret_cast<const uint2*>(smem + 2 * Q6G_WB + p * Q6G_XB) + cls * 128 + g * 16 + r;
    const float* sdd = reinterpret_cast<const float*>(smem + 2 * (Q6G_WB + Q6G_XB)) + p * Q6G_R * Q6G_DP;
    long ah[2], al[2], bx[2];
#pragma unroll
    for (int f = 0; f < 2; ++f) {
      ah[f] = *reinterpret_cast<const long*>(sw + f * 64);        // plane h, row half f
      al[f] = *reinterpret_cast<const long*>(sw + 128 + f * 64);  // plane lo
      bx[f] = *reinterpret_cast<const long*>(sx + f * 64);        // token half f
    }
#pragma unroll
    for (int rf = 0; rf < 2; ++rf)
#pragma unroll
      for (int tf = 0; tf < 2; ++tf) {
        const v4i_t ch = __builtin_amdgcn_mfma_i32_16x16x32_i8(ah[rf], bx[tf], v4i_t{0, 0, 0, 0}, 0, 0, 0);
        const v4i_t cl = __builtin_amdgcn_mfma_i32_16x16x32_i8(al[rf], bx[tf], v4i_t{0, 0, 0, 0}, 0, 0, 0);
        const float4 dd = *reinterpret_cast<const float4*>(sdd + (16 * tf + r) * Q6G_DP + 16 * rf + 4 * g);
        sums[rf][tf][0] += dd.x * (float)(ch[0] * 128 + cl[0]);
        sums[rf][tf][1] += dd.y * (float)(ch[1] * 128 + cl[1]);
        sums[rf][tf][2] += dd.z * (float)(ch[2] * 128 + cl[2]);
        sums[rf][tf][3] += dd.w * (float)(ch[3] * 128 + cl[3]);
      }
    // the fold before the next tile's LDS stores (which wait for its global loads)
#pragma unroll
    for (int rf = 0; rf < 2; ++rf)
#pragma unroll
      for (int tf = 0; tf < 2; ++tf)
#pragma unroll
        for (int i = 0; i < 4; ++i) asm volatile("" : "+v"(sums[rf][tf][i]));
    __builtin_amdgcn_sched_barrier(0);
  };

  // step s (LDS buffer and register set s % 2): issue step s + 2's loads into that set (its
  // tile went to LDS at step s - 1 or before the loop), fold the buffer, store the other set
  // (step s + 1's tile, loaded at step s - 1) into the other buffer.  The loop body is two
  // whole steps with no branch: loads past the end re-read the last superblock and their
  // stores fill a buffer no step folds, so the loads in flight at each store are the same on
  // every path and a store waits only for its own set; an odd last step runs after the loop.
  const int last = NSB - 1;
  CM_Q6G_LOAD(0, 0)
  CM_Q6G_LOAD(min(1, last), 1)
  CM_Q6G_STORE(0)
  __syncthreads();
  int s = 0;
  for (; s + 1 < NSB; s += 2) {
    CM_Q6G_LOAD(min(s + 2, last), 0)
    fold(0);
    CM_Q6G_STORE(1)
    __syncthreads();
    CM_Q6G_LOAD(min(s + 3, last), 1)
    fold(1);
    CM_Q6G_STORE(0)  // step s + 2's tile (unused when s + 2 == NSB)
    __syncthreads();
  }
  if (s < NSB) {  // odd NSB: the last step, in buffer 0
    fold(0);
    __syncthreads();
  }
#undef CM_Q6G_LOAD
#undef CM_Q6G_STORE
  float* sf = reinterpret_cast<float*>(smem);  // [class][token][row]
#pragma unroll
  for (int rf = 0; rf < 2; ++rf)
#pragma unroll
    for (int tf = 0; tf < 2; ++tf)
      *reinterpret_cast<float4*>(sf + (cls * Q6G_R + 16 * tf + r) * Q6G_DP + 16 * rf + 4 * g) =
          make_float4(sums[rf][tf][0], sums[rf][tf][1], sums[rf][tf][2], sums[rf][tf][3]);
  __syncthreads();
  float a0 = -0.0f, a1 = -0.0f;
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    const float2 v = *reinterpret_cast<const float2*>(sf + (c * Q6G_R + dtok) * Q6G_DP + drow);
    a0 += v.x;
    a1 += v.y;
  }
  const int t = tt * Q6G_R + dtok, n = rt * Q6G_R + drow;
  if (t < T && n < N) {  // N even: n + 1 < N too
    const size_t o = (size_t)t * ldy + n;
    float2 out = make_float2(a0, a1);
    if (resid) {
      const float2 rr = *reinterpret_cast<const float2*>(resid + o);
      out = make_float2(rr.x + a0, rr.y + a1);
    }
    *reinterpret_cast<float2*>(y + o) = out;
  }
}

// ---------------------------------------------------------------------------
// Q4_K GEMV over T tokens at once (speculative verify): each token's result is k_gemv_q4k's,
// in the same order; a lane's weight pieces and their headers are loaded once and dotted with
// every token's Q8_K activation, staged in LDS ([T][K] quants, [T][K/256] scales, and the
// [T][K/32] quant sums formed there).  4 rows per workgroup; y[t * ldy + row] (+ resid, same stride).
// Dynamic LDS: gemv_q4k_multi_lds_bytes(K, T).
constexpr int Q4M_MAX = 8;
__host__ __device__ inline size_t q4m_terms_offset(int K, int T) {
  return ((size_t)T * (K + (K / 256) * 4 + (K / 32) * 4) + 15) & ~(size_t)15;
}
__host__ __device__ inline size_t gemv_q4k_multi_lds_bytes(int K, int T) {
  return q4m_terms_offset(K, T) + (size_t)4 * T * (K / 256) * 16;
}

template <int IT>
__global__ __launch_bounds__(KQ_NT) void k_gemv_q4k_multi(const uint8_t* __restrict__ nib,
                                                          const uint8_t* __restrict__ hdr, int rows, int K,
                                                          const float* __restrict__ yd,
                                                          const int8_t* __restrict__ yq, int T, float* y, int ldy,
                                                          const float* resid) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int NSB = K >> 8, NC = K >> 5;
  int8_t* xq = reinterpret_cast<int8_t*>(smem);                                          // [T][K]
  float* xd = reinterpret_cast<float*>(smem + (size_t)T * K);                           // [T][NSB]
  int* xbs = reinterpret_cast<int*>(smem + (size_t)T * K + (size_t)T * NSB * 4);        // [T][NC]
  float4* terms = reinterpret_cast<float4*>(smem + q4m_terms_offset(K, T));             // [row][t][s]
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int row = min((int)blockIdx.x * 4 + wave, rows - 1);
  uint4 wv[IT], hv[IT];
  {
    const uint4* np = reinterpret_cast<const uint4*>(nib + (size_t)row * (K >> 1));
    const uint4* hp = reinterpret_cast<const uint4*>(hdr + (size_t)row * NSB * 16);
#pragma unroll
    for (int i = 0; i < IT; ++i) {
      const int cc = min(lane + 64 * i, NC - 1);
      wv[i] = ld_stream(np + cc);
      hv[i] = ld_stream(hp + (cc >> 3));
    }
  }
  for (int c = tid; c < (T * K) >> 4; c += KQ_NT) reinterpret_cast<int4*>(xq)[c] = reinterpret_cast<const int4*>(yq)[c];
  for (int i = tid; i < T * NSB; i += KQ_NT) xd[i] = yd[i];
  __syncthreads();
  for (int i = tid; i < T * NC; i += KQ_NT) {  // the per-32 quant sums (exact), from LDS
    const int4* q = reinterpret_cast<const int4*>(xq + (size_t)i * 32);
    int sum = 0;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int4 v = q[u];
      sum = __builtin_amdgcn_sdot4(v.x, 0x01010101, sum, false);
      sum = __builtin_amdgcn_sdot4(v.y, 0x01010101, sum, false);
      sum = __builtin_amdgcn_sdot4(v.z, 0x01010101, sum, false);
      sum = __builtin_amdgcn_sdot4(v.w, 0x01010101, sum, false);
    }
    xbs[i] = sum;
  }
  __syncthreads();
  const uint32_t K1 = 0x3f3f3f3fu, K2 = 0x0f0f0f0fu, K3 = 0x03030303u;
#pragma unroll
  for (int i = 0; i < IT; ++i) {
    const int c = lane + 64 * i;
    const bool valid = c < NC;  // uniform per 8-lane superblock group (NC % 8 == 0)
    const int cc = min(c, NC - 1);
    const uint4 w = wv[i], hd = hv[i];
    const int s = cc >> 3, j = cc & 7, c4 = j >> 1, h = j & 1;
    const uint32_t scw = (c4 < 2) ? (hd.y & K1) : ((hd.w & K2) | (((hd.y >> 6) & K3) << 4));
    const uint32_t mnw = (j < 4) ? (hd.z & K1) : (((hd.w >> 4) & K2) | (((hd.z >> 6) & K3) << 4));
    const int sc_lo = (scw >> (8 * ((2 * c4) & 3))) & 0xff;
    const int sc_hi = (scw >> (8 * ((2 * c4 + 1) & 3))) & 0xff;
    const int mn = (mnw >> (8 * (j & 3))) & 0xff;
    const int base = (s << 8) + 64 * c4 + 16 * h;
    const int wl[4] = {(int)(w.x & K2), (int)(w.y & K2), (int)(w.z & K2), (int)(w.w & K2)};
    const int wh[4] = {(int)((w.x >> 4) & K2), (int)((w.y >> 4) & K2), (int)((w.z >> 4) & K2),
                       (int)((w.w >> 4) & K2)};
    const float dw = half_bits_to_float((uint16_t)(hd.x & 0xffffu));
    const float dmw = half_bits_to_float((uint16_t)(hd.x >> 16));
    for (int t = 0; t < T; ++t) {
      const int8_t* xt = xq + (size_t)t * K;
      const int4 qa = *reinterpret_cast<const int4*>(xt + base);
      const int4 qb = *reinterpret_cast<const int4*>(xt + base + 32);
      int lo = 0, hi = 0;
      lo = __builtin_amdgcn_sdot4(wl[0], qa.x, lo, false);
      lo = __builtin_amdgcn_sdot4(wl[1], qa.y, lo, false);
      lo = __builtin_amdgcn_sdot4(wl[2], qa.z, lo, false);
      lo = __builtin_amdgcn_sdot4(wl[3], qa.w, lo, false);
      hi = __builtin_amdgcn_sdot4(wh[0], qb.x, hi, false);
      hi = __builtin_amdgcn_sdot4(wh[1], qb.y, hi, false);
      hi = __builtin_amdgcn_sdot4(wh[2], qb.z, hi, false);
      hi = __builtin_amdgcn_sdot4(wh[3], qb.w, hi, false);
      const int sumi = group8_sum_lead(lo * sc_lo + hi * sc_hi);
      const int prod = group8_sum_lead(xbs[t * NC + s * 8 + j] * mn);
      if (valid && j == 0) {
        const float ydv = xd[t * NSB + s];
        terms[((size_t)wave * T + t) * NSB + s] = make_float4(-(ydv * dmw), (float)prod, ydv * dw, (float)sumi);
      }
    }
  }
  __syncthreads();
  for (int f = tid; f < 4 * T; f += KQ_NT) {  // one lane per (row, token): the in-order fold
    const int rl = f / T, t = f - rl * T;
    const int r = blockIdx.x * 4 + rl;
    if (r < rows) {
      const float4* tp = terms + (size_t)f * NSB;
      float acc = 0.0f;
      for (int s = 0; s < NSB; ++s) {
        const float4 v = tp[s];
        acc = fmaf(v.x, v.y, acc);
        acc = fmaf(v.z, v.w, acc);
      }
      const size_t o = (size_t)t * ldy + r;
      y[o] = resid ? resid[o] + acc : acc;
    }
  }
}

}  // namespace cm
