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
#include <type_traits>

namespace cm {

__device__ __forceinline__ float half_bits_to_float(uint16_t b) {
  _Float16 h;
  __builtin_memcpy(&h, &b, 2);
  return (float)h;  // v_cvt_f32_f16: exact widening (f16 denormals are enabled on gfx9)
}

// q * f32(h) for the f16 h in the low / high half of w, rounded once to f32: one
// mixed-precision FMA with a -0 addend (exactly the f32 product, signed zeros included),
// in place of a conversion and a multiply.
__device__ __forceinline__ float mul_f16_lo(float q, uint32_t w) {
  float r;
  asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel_hi:[0,1,0]" : "=v"(r) : "v"(q), "v"(w), "v"(-0.0f));
  return r;
}
__device__ __forceinline__ float mul_f16_hi(float q, uint32_t w) {
  float r;
  asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel:[0,1,0] op_sel_hi:[0,1,0]" : "=v"(r) : "v"(q), "v"(w), "v"(-0.0f));
  return r;
}

// Weight streams are read once per token: nontemporal (streaming) loads, which measured
// about 10 % faster than plain loads for reads far beyond the caches on MI355X.
#ifndef CM_STREAM_LOADS
#define CM_STREAM_LOADS 1
#endif
typedef int stream_v4i __attribute__((ext_vector_type(4)));
__device__ __forceinline__ int4 ld_stream(const int4* p) {
#if CM_STREAM_LOADS
  const stream_v4i v = __builtin_nontemporal_load(reinterpret_cast<const stream_v4i*>(p));
  return make_int4(v.x, v.y, v.z, v.w);
#else
  return *p;
#endif
}
__device__ __forceinline__ uint4 ld_stream(const uint4* p) {
#if CM_STREAM_LOADS
  const stream_v4i v = __builtin_nontemporal_load(reinterpret_cast<const stream_v4i*>(p));
  return make_uint4((uint32_t)v.x, (uint32_t)v.y, (uint32_t)v.z, (uint32_t)v.w);
#else
  return *p;
#endif
}
__device__ __forceinline__ uint16_t ld_stream(const uint16_t* p) {
#if CM_STREAM_LOADS
  return __builtin_nontemporal_load(p);
#else
  return *p;
#endif
}
__device__ __forceinline__ uint32_t ld_stream(const uint32_t* p) {
#if CM_STREAM_LOADS
  return __builtin_nontemporal_load(p);
#else
  return *p;
#endif
}

// Agent-scope (device-coherent across XCDs) loads and stores for data handed between the
// workgroups of one launch: they bypass the XCD-private L2 copies that plain accesses may hit.
__device__ __forceinline__ uint64_t ld_agent64(const void* p) {
  return __hip_atomic_load(reinterpret_cast<const uint64_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t ld_agent32(const void* p) {
  return __hip_atomic_load(reinterpret_cast<const uint32_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_agent64(void* p, uint64_t v) {
  __hip_atomic_store(reinterpret_cast<uint64_t*>(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_agent32(void* p, uint32_t v) {
  __hip_atomic_store(reinterpret_cast<uint32_t*>(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Set by a workgroup whose bounded wait for another workgroup of its launch ran out (the
// in-launch handoffs of the norm-fused K-quant GEMVs and of the attention's output
// projection); the engine clears it before a call's decode steps and reads it after them.
__device__ uint32_t g_handoff_error;

__device__ __forceinline__ int dot4x4(int4 w, int4 x, int acc) {
  acc = __builtin_amdgcn_sdot4(w.x, x.x, acc, false);
  acc = __builtin_amdgcn_sdot4(w.y, x.y, acc, false);
  acc = __builtin_amdgcn_sdot4(w.z, x.z, acc, false);
  acc = __builtin_amdgcn_sdot4(w.w, x.w, acc, false);
  return acc;
}

// ---------------------------------------------------------------------------
// Serial f32 folds in index order (one lane): the CPU's summation order.  LDS reads run
// 8 float4 groups (32 floats) ahead of the dependent add chain, with clamped (always in
// bounds) addresses so the main loop is straight-line code.  p must be 16-byte aligned.
__device__ __forceinline__ void add4(float& acc, const float4 v) {
  acc += v.x;
  acc += v.y;
  acc += v.z;
  acc += v.w;
}

__device__ __forceinline__ void load8(float4 (&r)[8], const float4* q) {
#pragma unroll
  for (int i = 0; i < 8; ++i) r[i] = q[i];
}
__device__ __forceinline__ void add8(float& acc, const float4 (&r)[8]) {
#pragma unroll
  for (int i = 0; i < 8; ++i) add4(acc, r[i]);
}

__device__ __forceinline__ float fold_lds(const float* p, int n, float acc = 0.0f) {
  const float4* q = reinterpret_cast<const float4*>(p);
  const int g = n >> 2;
  int base = 0;
  if (g >= 8) {
    // ping-pong between two register sets: the next 8 groups are always in flight
    float4 a[8], b[8];
    load8(a, q);
    base = 8;
    // not unrolled: a fully unrolled fold would hold every term in registers at once
#pragma unroll 1
    for (; base + 16 <= g; base += 16) {
      load8(b, q + base);
      __builtin_amdgcn_sched_barrier(0);
      add8(acc, a);
      load8(a, q + base + 8);
      __builtin_amdgcn_sched_barrier(0);
      add8(acc, b);
    }
    if (base + 8 <= g) {
      load8(b, q + base);
      __builtin_amdgcn_sched_barrier(0);
      add8(acc, a);
      add8(acc, b);
      base += 8;
    } else {
      add8(acc, a);
    }
  }
  for (; base < g; ++base) add4(acc, q[base]);
  for (int i = g << 2; i < n; ++i) acc += p[i];
  return acc;
}

// The same sequential fold with a small register footprint (two groups of 4 float4 in
// flight): the fallback of inorder_sum_onepass, which runs inside kernels whose registers
// are already committed.  p must be 16-byte aligned.
__device__ __forceinline__ float fold_lds_lean(const float* p, int n) {
  const float4* q = reinterpret_cast<const float4*>(p);
  const int g = n >> 2;
  float acc = 0.0f;
  int base = 0;
  if (g >= 4) {
    float4 a[4], b[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) a[u] = q[u];
    base = 4;
#pragma unroll 1
    for (; base + 4 <= g; base += 4) {
#pragma unroll
      for (int u = 0; u < 4; ++u) b[u] = q[base + u];
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        add4(acc, a[u]);
        a[u] = b[u];
      }
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) add4(acc, a[u]);
  }
  for (; base < g; ++base) add4(acc, q[base]);
  for (int i = g << 2; i < n; ++i) acc += p[i];
  return acc;
}

// ---------------------------------------------------------------------------
// Exact in-order sum of n f32 values (non-negative in the intended use), evaluated by a
// whole workgroup; bit-identical to the sequential fold s_i = RNE(s_{i-1} + t_i).
//
// While the running sum stays in one binade [2^e, 2^(e+1)) (or in [0, 2^-125), where
// the ulp is 2^-149 throughout), its ulp u is fixed and s_{i-1} is a multiple of u, so a
// step adds exactly the integer d_i = RNE(t_i / u) ulps -- unless t_i / u is an exact half
// (round-half-even then depends on the running parity), t_i >= 2^e, t_i is negative or
// not finite, or the step leaves the binade.
//   pass  (all threads): for each of seg_binades(C) consecutive binades from the current
//         one, d_i for every remaining term, with the exceptional terms ("flagged") given
//         d = 2^25, larger than any in-binade step; a saturating workgroup prefix sum of d
//         per binade goes to LDS.  A new pass is needed only past the last of them.
//   round (wave 0, per stop): in the running sum's binade, from the mantissa N (in ulps)
//         at term k, the first index i >= k whose step reaches 2^24 ulps or is flagged is
//         the first p with ps[p] >= 2^24 - N + ps[k] (ps is monotone), minus one; found by
//         a 64-way ballot search.  Terms k..i-1 are summed exactly by the integer
//         difference; term i is applied as a real f32 add (flag or binade change), or --
//         when it rounds up onto exactly 2^(e+1) -- written directly.
// The first m_seq terms, where binade changes are frequent, are folded sequentially.
// Negative or huge (>= 2^126) running sums take plain sequential steps.  Every thread
// of the workgroup must call; v (n floats) and ps (seg_binades(C) * (NT * C + 4) words) are
// in LDS; NT * C >= n.
constexpr uint32_t SEG_LIM = 1u << 24;   // ulps in a binade
constexpr uint32_t SEG_FLAG = 1u << 25;  // step given to a flagged term
constexpr uint32_t SEG_GUARD = 0xffffffffu - 2u * SEG_FLAG;  // prefix values the rounds accept

__device__ __forceinline__ uint32_t sat_add(uint32_t a, uint32_t b) { return __builtin_elementwise_add_sat(a, b); }

// Step (in ulps of the binade with exponent field Ep >= 1, u = 2^(Ep - 150)) of term t;
// SEG_FLAG when t / u is a tie, >= 2^23, negative (-0 included), or not finite.
__device__ __forceinline__ uint32_t seg_d(float t, int Ep, float* q_out = nullptr) {
  const float q = ldexpf(t, 150 - Ep);  // t / u, exact whenever it is >= 2^-126
  const float r = rintf(q);
  if (q_out) *q_out = q;
  const bool ok = __float_as_uint(q) < 0x4b000000u && fabsf(q - r) != 0.5f;
  return ok ? (uint32_t)r : SEG_FLAG;
}

// f32 with value Nv ulps in the binade Ep (Nv < 2^24; Nv == 2^24 gives 2^(e+1)).
__device__ __forceinline__ float seg_value(int Ep, uint32_t Nv) {
  return __uint_as_float(((uint32_t)(Ep - 1) << 23) + Nv);
}

// Saturating wave-wide inclusive scan: DPP row shifts within each 16-lane row, then row
// broadcasts across rows.
#define CM_DPP(x, ctrl, rmask) ((uint32_t)__builtin_amdgcn_update_dpp(0, (int)(x), ctrl, rmask, 0xf, false))
__device__ __forceinline__ uint32_t wave_scan_incl_sat(uint32_t x) {
  x = sat_add(x, CM_DPP(x, 0x111, 0xf));  // row_shr:1
  x = sat_add(x, CM_DPP(x, 0x112, 0xf));  // row_shr:2
  x = sat_add(x, CM_DPP(x, 0x114, 0xf));  // row_shr:4
  x = sat_add(x, CM_DPP(x, 0x118, 0xf));  // row_shr:8
  x = sat_add(x, CM_DPP(x, 0x142, 0xa));  // row_bcast:15 -> rows 1, 3
  x = sat_add(x, CM_DPP(x, 0x143, 0xc));  // row_bcast:31 -> rows 2, 3
  return x;
}

// Binades covered by one pass (prefix arrays of n + 4 words each in LDS), by chunk size.
// (measured: at 16 terms per thread three binades beat four, 14.0 vs 15.8 us for n = 4096)
__host__ __device__ constexpr int seg_binades(int C) { return C <= 12 ? 4 : C <= 32 ? 3 : 1; }

template <int NT, int C, int NBV = seg_binades(C)>
__device__ __forceinline__ float inorder_sum_nonneg(const float* v, uint32_t* ps, int n, int m_seq) {
  constexpr int NW = NT / 64;
  constexpr int NB = NBV;  // consecutive binades per pass
  constexpr int PSTRIDE = NT * C + 4;  // words per prefix array
  static_assert(NT % 64 == 0 && NW <= 16, "the cross-wave scan runs in one 16-lane DPP row");
  __shared__ float sh_s;
  __shared__ int sh_k;
  __shared__ uint32_t sh_tot[NB][NW];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int i0 = tid * C;  // this thread's contiguous chunk
  float t[C];
#pragma unroll
  for (int c = 0; c < C; ++c) t[c] = i0 + c < n ? v[i0 + c] : 0.0f;
  if (tid == 0) {
    const int m = min(n, m_seq);
    sh_s = fold_lds_lean(v, m);  // (the chunk's terms are held in registers meanwhile)
    sh_k = m;
  }
  __syncthreads();
  while (true) {
    float s = sh_s;
    int k = sh_k;
    if (k >= n) break;
    const uint32_t sb0 = __float_as_uint(s);
    const int E0 = (int)((sb0 >> 23) & 0xffu);
    const int Eb = max(E0, 1);  // first binade of this pass
    const bool plain = (sb0 >> 31) != 0u || E0 >= 254;
    if (!plain) {  // pass for binades Eb .. Eb+NB-1 over the terms k..n-1 (terms before k count 0)
      uint32_t dv[NB][C];
      uint32_t T[NB];
#pragma unroll
      for (int b = 0; b < NB; ++b) T[b] = 0;
      if (i0 + C > k) {
#pragma unroll
        for (int c = 0; c < C; ++c)
#pragma unroll
          for (int b = 0; b < NB; ++b) dv[b][c] = seg_d(t[c], Eb + b);
        if (i0 < k) {
#pragma unroll
          for (int c = 0; c < C; ++c)
#pragma unroll
            for (int b = 0; b < NB; ++b) dv[b][c] = i0 + c < k ? 0u : dv[b][c];
        }
      } else {
#pragma unroll
        for (int c = 0; c < C; ++c)
#pragma unroll
          for (int b = 0; b < NB; ++b) dv[b][c] = 0u;
      }
#pragma unroll
      for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int c = 0; c < C; ++c) T[b] = sat_add(T[b], dv[b][c]);
      uint32_t incl[NB];
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        incl[b] = wave_scan_incl_sat(T[b]);
        if (lane == 63) sh_tot[b][wave] = incl[b];
      }
      __syncthreads();
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        uint32_t wt = lane < NW ? sh_tot[b][lane] : 0u;
        wt = sat_add(wt, CM_DPP(wt, 0x111, 0xf));
        wt = sat_add(wt, CM_DPP(wt, 0x112, 0xf));
        wt = sat_add(wt, CM_DPP(wt, 0x114, 0xf));
        wt = sat_add(wt, CM_DPP(wt, 0x118, 0xf));
        const uint32_t wpre = (uint32_t)__builtin_amdgcn_readlane((int)CM_DPP(wt, 0x111, 0xf), wave);
        uint32_t P = sat_add(wpre, CM_DPP(incl[b], 0x138, 0xf));  // wave_shr:1 -> exclusive prefix
        uint32_t* psb = ps + b * PSTRIDE;
        uint32_t pv[C];
#pragma unroll
        for (int c = 0; c < C; ++c) {
          pv[c] = P;
          P = sat_add(P, dv[b][c]);
        }
        if constexpr (C % 4 == 0) {
          if (i0 + C <= n) {
#pragma unroll
            for (int c = 0; c < C; c += 4)
              *reinterpret_cast<uint4*>(psb + i0 + c) = make_uint4(pv[c], pv[c + 1], pv[c + 2], pv[c + 3]);
          } else {
#pragma unroll
            for (int c = 0; c < C; ++c)
              if (i0 + c < n) psb[i0 + c] = pv[c];
          }
        } else {
#pragma unroll
          for (int c = 0; c < C; ++c)
            if (i0 + c < n) psb[i0 + c] = pv[c];
        }
        if (i0 <= n - 1 && n - 1 < i0 + C) psb[n] = P;
      }
    }
    __syncthreads();
    if (wave == 0) {  // rounds: uniform control flow over the wave
      int cur = -1;            // prefix array in use (binade Eb + cur)
      uint32_t base = 0, tot = 0;  // its values at k and at n
      while (k < n) {
        const uint32_t sb = __float_as_uint(s);
        const int E = (int)((sb >> 23) & 0xffu);
        if ((sb >> 31) != 0u || E >= 254) {  // negative or huge running sum: plain step
          s = s + v[k];
          ++k;
          cur = -1;
          continue;
        }
        const int Ep = max(E, 1);
        const int b = Ep - Eb;
        if (plain || b < 0 || b >= NB) break;  // outside this pass's binades: new pass
        const uint32_t* psb = ps + b * PSTRIDE;
        if (b != cur) {
          base = psb[k];
          tot = psb[n];
          cur = b;
        }
        if (base > SEG_GUARD) break;  // keep the prefix sums unsaturated
        const uint32_t N = sb - ((uint32_t)(Ep - 1) << 23);
        const uint32_t X = SEG_LIM - N + base;
        if (tot < X) {  // no stop: the rest sums exactly in this binade
          s = seg_value(Ep, N + (tot - base));
          k = n;
          break;
        }
        // first p in [k + 1, n] with psb[p] >= X (psb[n] >= X)
        int lo = k + 1, hi = n;
        while (hi - lo >= 63) {
          const int stride = (hi - lo + 64) >> 6;
          const int p = min(lo + lane * stride + stride - 1, hi);
          const unsigned long long bm = __ballot(psb[p] >= X);
          const int nlo = lo + (__ffsll((long long)bm) - 1) * stride;
          hi = min(nlo + stride - 1, hi);
          lo = nlo;
        }
        // lane l holds position lo - 1 + l (lane 0: the term before the range)
        const int q = min(lo - 1 + lane, hi);
        const uint32_t pq = psb[q];
        const float tq = v[min(q, n - 1)];
        const unsigned long long bm = __ballot(lane >= 1 && lo - 1 + lane <= hi && pq >= X);
        const int li = __ffsll((long long)bm) - 2;  // lane holding the stopping term i = p - 1
        const int i = lo - 1 + li;
        const uint32_t pi = (uint32_t)__builtin_amdgcn_readlane((int)pq, li);
        const float ti = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(tq), li));
        float qi;
        const uint32_t di = seg_d(ti, Ep, &qi);
        const uint32_t Ni = N + (pi - base);  // running sum before term i, exact
        if (di == SEG_FLAG || Ni + (uint32_t)floorf(qi) >= SEG_LIM) {
          s = seg_value(Ep, Ni) + ti;  // flagged term or a binade change: real add
        } else {
          s = seg_value(Ep, SEG_LIM);  // rounds up onto exactly 2^(e+1)
        }
        base = sat_add(pi, di);  // psb[i + 1]
        k = i + 1;
      }
      if (lane == 0) {
        sh_s = s;
        sh_k = k;
      }
    }
    __syncthreads();
  }
  return sh_s;
}

// ---------------------------------------------------------------------------
// One-pass exact in-order sum of n f32 values held C per thread (thread t: terms t*C ..
// t*C+C-1, zero past n), bit-identical to the sequential fold s_i = RNE(s_{i-1} + t_i).
//
// The binade of every running sum s_i is predicted from an f64 prefix sum R_i of the terms:
// for non-negative terms each step rounds by at most 2^-24 of the new sum, so
// |s_i - R_i| <= i * 2^-24 * s_i, and R_i's binade is s_i's unless R_i lies within about
// (i+1) * 2^-23 (relative) of a binade boundary ("uncertain").  A step whose running sum is
// predicted to stay in one certain binade adds exactly d_i = RNE(t_i / u) ulps (seg_d:
// ties, terms of 2^23 ulps or more, negative and non-finite terms are excluded); every other
// step is "special".  Between two special steps the sum moves by the integer total of the
// d_i (a segmented scan over the workgroup).  Wave 0 then replays the special steps in order
// as real f32 adds, applying each run's integer total first -- after checking that the run
// starts in its predicted binade and ends below the binade's top: the d_i are
// non-negative, so the run then stayed in that binade and every step rounded as assumed.
// A failed check, or more than FS_CAP special steps, falls back to the sequential fold of v
// (the same n terms, in LDS): the result never depends on the prediction being right.
// Every thread of the workgroup must call; NT * C >= n; fs: the caller's LDS workspace (one
// per kernel, shared by every chunk size the kernel instantiates).
// Phase timestamps of the two norm-fused GEMVs (measurement build only, as g_att_stamps):
// kind 0 k_gemv_norm, 1 k_gemv_gu_silu; per workgroup (< 256; the last launch overwrites):
// 0 start (thread 0), 1 norm done (thread 0), 2 a weight wave's loads issued (thread 256),
// 3 past the workgroup barrier after the norm, 4 block dots done, 5 end.
constexpr int GEMV_NSTAMP = 13, GEMV_STAMP_WGS = 256;
#ifdef CM_STAMPS
__device__ uint64_t g_gemv_stamps[2 * GEMV_STAMP_WGS * GEMV_NSTAMP];
#define CM_GEMV_STAMP(kind, i, t)                                                                        \
  if (threadIdx.x == (t) && blockIdx.x < GEMV_STAMP_WGS)                                                 \
    g_gemv_stamps[((kind) * GEMV_STAMP_WGS + blockIdx.x) * GEMV_NSTAMP + (i)] = __builtin_amdgcn_s_memrealtime();
// (workgroups spread over the whole grid: every ceil(grid / 256)-th, in slot blockIdx / that)
#define CM_GEMV_STAMP_SAMPLED(kind, i, t)                                                                \
  if (threadIdx.x == (t) && blockIdx.x % ((gridDim.x + GEMV_STAMP_WGS - 1) / GEMV_STAMP_WGS) == 0)       \
    g_gemv_stamps[((kind) * GEMV_STAMP_WGS + blockIdx.x / ((gridDim.x + GEMV_STAMP_WGS - 1) / GEMV_STAMP_WGS)) * \
                      GEMV_NSTAMP + (i)] = __builtin_amdgcn_s_memrealtime();
#else
#define CM_GEMV_STAMP(kind, i, t)
#define CM_GEMV_STAMP_SAMPLED(kind, i, t)
#endif

constexpr int FS_CAP = 128;  // special steps the replay takes before falling back
template <int NT>
struct FsLds {
  uint4 ent[FS_CAP];                   // the special steps: (run before it, its check lo, lim, term bits)
  double r[NT / 64];                   // wave totals of the f64 prefix
  uint32_t rs[NT / 64], b[NT / 64], c[NT / 64];  // wave totals of the segmented scan
  uint32_t end[3];                     // the final run and its check
  float sum;
};

// Predicted binade (f32 exponent field, at least 1) of a running sum estimated as R after b
// terms; 0 when the sum may lie in a neighbouring binade (or R is negative or huge).  Written
// without branches (bitwise tests, one select): it runs C times per thread in the
// classification pass, whose length is set by each wave's instruction issue.
__device__ __forceinline__ int fs_binade(double R, int b) {
  const uint32_t hi = (uint32_t)__double2hiint(R);
  const int field = (int)(hi >> 20) - 896;  // f64 exponent rebased to f32's
  const uint32_t m20 = hi & 0xfffffu;       // leading 20 mantissa bits
  const uint32_t slack = ((uint32_t)(b + 1) >> 3) + 2;  // (b+1) * 2^-23 relative, in 2^-20 units
  const bool unsure = (field >= 254) | (m20 >= 0xfffffu - slack) | ((field >= 2) & (m20 < slack));
  // below 2^-126 (field <= 0): one binade (ulp 2^-149) down to zero
  return field <= 0 ? 1 : (unsure ? 0 : field);
}

// A special step's replay data: the run of V ulps before it is valid iff the running sum's
// bits sb satisfy (sb - lo) < lim (unsigned), i.e. sb lies in the run's predicted binade
// E and sb + V stays below its top; the run then moves the sum to the bits sb + V.
// (Selects, no branches: it runs for every term of the entries pass.)
__device__ __forceinline__ void fs_entry(uint32_t V, int E, uint32_t& lo, uint32_t& lim) {
  const uint32_t lo0 = E <= 1 ? 0u : (uint32_t)E << 23;    // lowest bits of the binade (E = 0: invalid)
  const uint32_t span = ((uint32_t)(E + 1) << 23) - lo0;  // bits in the binade
  const uint32_t lim0 = ((E >= 1) & (V < span)) ? span - V : 0u;
  // V == 0: nothing to apply, nothing to check
  lo = V == 0u ? 0u : lo0;
  lim = V == 0u ? 0xffffffffu : lim0;
}

template <int CTRL, int RMASK>
__device__ __forceinline__ double dpp_f64(double x) {
  const int lo = __builtin_amdgcn_update_dpp(0, __double2loint(x), CTRL, RMASK, 0xf, false);
  const int hi = __builtin_amdgcn_update_dpp(0, __double2hiint(x), CTRL, RMASK, 0xf, false);
  return __hiloint2double(hi, lo);
}

// Segmented-scan step: (rs, b) absorbs the earlier element (rp, bp): b restarts after a
// special step (rs set), else accumulates; cnt is a plain sum.
#define CM_FS_STEP(ctrl, rmask)                                                                            \
  {                                                                                                         \
    const uint32_t rp = CM_DPP(rs, ctrl, rmask), bp = CM_DPP(b, ctrl, rmask), cp = CM_DPP(cnt, ctrl, rmask); \
    b = rs ? b : sat_add(bp, b);                                                                            \
    rs |= rp;                                                                                               \
    cnt += cp;                                                                                              \
  }

// Barrier policies of the one-pass sum and the in-kernel norm: the whole workgroup
// (__syncthreads), or a team of the workgroup's first waves synchronising through an LDS
// counter (TeamBar), so that the other waves can stream weights meanwhile without taking part.
struct WgBar {
  __device__ __forceinline__ void operator()() const { __syncthreads(); }
};

// Software barrier of waves 0 .. nw-1 (threads 0 .. 64*nw-1) of a workgroup.  `ctr` is a
// zeroed LDS word (zeroed before a workgroup barrier that precedes the first use); each call
// adds one per wave and waits, with the team's LDS writes made visible first, until every
// team wave has arrived.  The wait is bounded: past about 2^22 polls (far beyond any
// schedule) the call returns with *bad set, so a broken schedule cannot hang the device; the
// caller then takes its fallback.
struct TeamBar {
  uint32_t* ctr;
  uint32_t* bad;
  uint32_t nw;
  uint32_t target;
  __device__ __forceinline__ void operator()() {
    target += nw;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    if ((threadIdx.x & 63) == 0) __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    uint32_t polls = 0;
    while (__hip_atomic_load(ctr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) < target) {
      __builtin_amdgcn_s_sleep(1);
      if (++polls == (1u << 22)) {
        *bad = 1u;
        break;
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
  }
};

template <int NT, int C, bool LINE = false, typename Bar = WgBar>
__device__ __forceinline__ float inorder_sum_onepass(const float (&t)[C], const float* v, int n, FsLds<NT>& fs,
                                                     Bar&& bar = Bar{}, int stamp_kind = -1) {
  (void)stamp_kind;  // (the measurement build: stamps 8..11 of the norm-fused GEMVs after each barrier)
  constexpr int NW = NT / 64;
  static_assert(NT % 64 == 0 && NW <= 16 && C <= 32, "one 16-lane row holds the wave totals");
  double* sh_r = fs.r;
  uint32_t *sh_rs = fs.rs, *sh_b = fs.b, *sh_c = fs.c;
  uint4* sh_ent = fs.ent;
  uint32_t* sh_end = fs.end;
  float& sh_sum = fs.sum;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform per wave: a scalar lane index
  const int i0 = tid * C;
  // f64 prefix of the terms before this thread's chunk: wave scan, then the wave totals
  // scanned in one 16-lane row
  double r = 0.0;
#pragma unroll
  for (int c = 0; c < C; ++c) r += (double)t[c];
  double incl = r;
  incl += dpp_f64<0x111, 0xf>(incl);  // row_shr:1
  incl += dpp_f64<0x112, 0xf>(incl);  // row_shr:2
  incl += dpp_f64<0x114, 0xf>(incl);  // row_shr:4
  incl += dpp_f64<0x118, 0xf>(incl);  // row_shr:8
  incl += dpp_f64<0x142, 0xa>(incl);  // row_bcast:15
  incl += dpp_f64<0x143, 0xc>(incl);  // row_bcast:31
  if (lane == 63) sh_r[wave] = incl;
  double R = dpp_f64<0x138, 0xf>(incl);  // wave_shr:1 -> exclusive
  bar();
  if (stamp_kind >= 0) {
    CM_GEMV_STAMP(stamp_kind, 8, 0)
  }
  if (NW > 1) {
    double wt = lane < NW ? sh_r[lane] : 0.0;
    wt += dpp_f64<0x111, 0xf>(wt);
    wt += dpp_f64<0x112, 0xf>(wt);
    wt += dpp_f64<0x114, 0xf>(wt);
    wt += dpp_f64<0x118, 0xf>(wt);
    const double wx = dpp_f64<0x111, 0xf>(wt);  // exclusive over the waves
    R += __hiloint2double(__builtin_amdgcn_readlane(__double2hiint(wx), wave),
                          __builtin_amdgcn_readlane(__double2loint(wx), wave));
  }
  // classify the steps; d = ulps of an in-binade step, 0 for a special one
  uint32_t d[C];
  uint32_t ebp[(C + 3) / 4];  // the predicted binade before each step (an exponent field: a byte each)
#pragma unroll
  for (int c = 0; c < (C + 3) / 4; ++c) ebp[c] = 0u;
  uint32_t spm = 0;
  int eb = fs_binade(R, i0), e_end = 1;
#pragma unroll
  for (int c = 0; c < C; ++c) {
    const int i = i0 + c;
    const double Ra = R + (double)t[c];
    const int ea = fs_binade(Ra, i + 1);
    // (seg_d unconditionally, then a select: no branch per term)
    const uint32_t sd = seg_d(t[c], eb > 0 ? eb : 1);
    const uint32_t dc = ((eb != 0) & (eb == ea)) ? sd : SEG_FLAG;
    const bool special = i < n && dc == SEG_FLAG;
    d[c] = (i < n && !special) ? dc : 0u;
    spm |= (uint32_t)special << c;
    ebp[c >> 2] |= (uint32_t)eb << (8 * (c & 3));
    if (i == n - 1) e_end = ea;
    eb = ea;
    R = Ra;
  }
  // segmented scan: the run total entering each chunk (a special step resets it), and the
  // count of special steps before it
  uint32_t b = 0;
#pragma unroll
  for (int c = 0; c < C; ++c) b = ((spm >> c) & 1u) ? 0u : sat_add(b, d[c]);
  uint32_t rs = spm != 0u, cnt = (uint32_t)__builtin_popcount(spm);
  CM_FS_STEP(0x111, 0xf)
  CM_FS_STEP(0x112, 0xf)
  CM_FS_STEP(0x114, 0xf)
  CM_FS_STEP(0x118, 0xf)
  CM_FS_STEP(0x142, 0xa)
  CM_FS_STEP(0x143, 0xc)
  if (lane == 63) {
    sh_rs[wave] = rs;
    sh_b[wave] = b;
    sh_c[wave] = cnt;
  }
  uint32_t run = CM_DPP(b, 0x138, 0xf), pos = CM_DPP(cnt, 0x138, 0xf);
  const uint32_t rs_x = CM_DPP(rs, 0x138, 0xf);
  bar();
  if (stamp_kind >= 0) {
    CM_GEMV_STAMP(stamp_kind, 9, 0)
  }
  uint32_t total;
  {
    const uint32_t wr = lane < NW ? sh_rs[lane] : 0u, wbv = lane < NW ? sh_b[lane] : 0u,
                   wc = lane < NW ? sh_c[lane] : 0u;
    {  // the wave totals' segmented scan in row 0
      uint32_t rs = wr, b = wbv, cnt = wc;
      CM_FS_STEP(0x111, 0xf)
      CM_FS_STEP(0x112, 0xf)
      CM_FS_STEP(0x114, 0xf)
      CM_FS_STEP(0x118, 0xf)
      total = (uint32_t)__builtin_amdgcn_readlane((int)cnt, NW - 1);
      const uint32_t bx = CM_DPP(b, 0x111, 0xf), cx = CM_DPP(cnt, 0x111, 0xf);
      const uint32_t bw = (uint32_t)__builtin_amdgcn_readlane((int)bx, wave);
      pos += (uint32_t)__builtin_amdgcn_readlane((int)cx, wave);
      run = rs_x ? run : sat_add(bw, run);
    }
  }
  // the special steps, in order: the term, and the run before it with its check (the entry
  // formed for every term, one guarded store: no nested branches per term)
#pragma unroll
  for (int c = 0; c < C; ++c) {
    const bool sp = (spm >> c) & 1u;
    uint32_t lo, lim;
    fs_entry(run, (int)((ebp[c >> 2] >> (8 * (c & 3))) & 0xffu), lo, lim);
    if (sp & (pos < (uint32_t)FS_CAP)) sh_ent[pos] = make_uint4(run, lo, lim, __float_as_uint(t[c]));
    pos += (uint32_t)sp;
    run = sp ? 0u : sat_add(run, d[c]);
  }
  if (i0 <= n - 1 && n - 1 < i0 + C) {
    uint32_t lo, lim;
    fs_entry(run, e_end, lo, lim);
    sh_end[0] = run;
    sh_end[1] = lo;
    sh_end[2] = lim;
  }
  if (tid < 3) {  // the entries padded to a multiple of 4 with steps that change nothing
    const uint32_t p = total + (uint32_t)tid;
    if (p < ((total + 3u) & ~3u) && p < (uint32_t)FS_CAP) sh_ent[p] = make_uint4(0u, 0u, 0xffffffffu, 0u);
  }
  bar();
  if (stamp_kind >= 0) {
    CM_GEMV_STAMP(stamp_kind, 10, 0)
  }
  if (wave == 0) {
    // replay: the sum's chain is one integer and one f32 add per special step.  Every lane
    // of wave 0 runs the same chain on the same entries: broadcast LDS reads of 4 entries, the
    // next 4 read while these are applied (two register sets, no moves; no step is skipped:
    // the padding steps add 0 ulps and +0.0, which leave a sum >= +0 unchanged)
    const int tot = __builtin_amdgcn_readfirstlane((int)total);
#ifdef CM_STAMPS
    if (stamp_kind >= 0 && threadIdx.x == 0 && blockIdx.x < GEMV_STAMP_WGS)  // (a count, not a time)
      g_gemv_stamps[(stamp_kind * GEMV_STAMP_WGS + blockIdx.x) * GEMV_NSTAMP + 12] = (uint64_t)tot;
#endif
    float s = 0.0f;
    // (a mask flag for the straight-line replay; a 0/1 word for the loop, as that form measured
    // faster in the attention and K-quant norm sums)
    typename std::conditional<LINE, bool, uint32_t>::type bad = tot > FS_CAP;
    if (!bad && tot > 0) {
      auto step = [&](const uint4& q) {
        const uint32_t sb = __float_as_uint(s);
        bad |= sb - q.y >= q.z;
        s = __uint_as_float(sb + q.x) + __uint_as_float(q.w);
      };
      const int nb = (tot + 3) >> 2;  // blocks of 4 entries (nb <= FS_CAP / 4)
      uint4 A[4], B[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) A[u] = sh_ent[u];
      // two blocks: A's steps while B's entries are read, B's while the next A's are; false
      // once the last block is applied
      auto pair = [&](int k) -> bool {
        if (k + 1 < nb) {
#pragma unroll
          for (int u = 0; u < 4; ++u) B[u] = sh_ent[4 * (k + 1) + u];
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int u = 0; u < 4; ++u) step(A[u]);
        if (k + 1 >= nb) return false;
        if (k + 2 < nb) {
#pragma unroll
          for (int u = 0; u < 4; ++u) A[u] = sh_ent[4 * (k + 2) + u];
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int u = 0; u < 4; ++u) step(B[u]);
        return k + 2 < nb;
      };
      // LINE: the first 32 entries as straight-line code (the two register sets alternate
      // without copies), any beyond as a loop; else all as a loop (less code where the sum is
      // not on the launch's critical path)
      bool more = true;
      int k0 = 0;
      if constexpr (LINE) {
#pragma unroll
        for (int k = 0; k < 8; k += 2)
          if (more) more = pair(k);
        k0 = 8;
      }
      if (more)
        for (int k = k0; k < nb && pair(k); k += 2) {
        }
    }
    {
      const uint32_t sb = __float_as_uint(s);
      bad |= sb - sh_end[1] >= sh_end[2];
      s = __uint_as_float(sb + sh_end[0]);
    }
    if (bad) s = fold_lds_lean(v, n);
    if (lane == 0) sh_sum = s;
  }
  bar();
  if (stamp_kind >= 0) {
    CM_GEMV_STAMP(stamp_kind, 11, 0)
  }
  return sh_sum;
}
#undef CM_FS_STEP

// Compile-time length variant (N % 4 == 0), same order.  The length is hidden from the
// optimiser (an empty asm statement) so that the fold stays a loop instead of straight-line
// code that hoists every term into registers (register count sets the workgroups per CU).
template <int N>
__device__ __forceinline__ float fold_lds_n(const float* p, float acc = 0.0f) {
  static_assert(N % 4 == 0, "fold length must be a multiple of 4");
  int n = N;
  asm volatile("" : "+s"(n));
  return fold_lds(p, n, acc);
}

// Lane-pair exchange (xor 1) through DPP quad_perm [1,0,3,2]; all lanes must be active.
__device__ __forceinline__ int dpp_xor1(int v) { return __builtin_amdgcn_mov_dpp(v, 0xB1, 0xF, 0xF, false); }

// Maximum over each aligned 32-lane half of the wave, in every lane of the half (fmaxf: order
// independent): quad and row exchanges by DPP (lane i then holds quads i, i - 4, i - 8, i - 12
// of its row), then the half's two rows from lanes 0/16 or 32/48.  Whole halves must be active.
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xf, 0xf, false));
}
__device__ __forceinline__ float max_half_wave(float a) {
  a = fmaxf(a, dpp_f32<0xB1>(a));   // quad_perm [1,0,3,2]
  a = fmaxf(a, dpp_f32<0x4E>(a));   // quad_perm [2,3,0,1]
  a = fmaxf(a, dpp_f32<0x124>(a));  // row_ror:4
  a = fmaxf(a, dpp_f32<0x128>(a));  // row_ror:8
  const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(a), 0));
  const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(a), 16));
  const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(a), 32));
  const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(a), 48));
  return (threadIdx.x & 32) ? fmaxf(r2, r3) : fmaxf(r0, r1);
}
// maximum over the whole wave, in every lane (as max_half_wave; the whole wave active)
__device__ __forceinline__ float max_wave(float a) {
  a = fmaxf(a, dpp_f32<0xB1>(a));
  a = fmaxf(a, dpp_f32<0x4E>(a));
  a = fmaxf(a, dpp_f32<0x124>(a));
  a = fmaxf(a, dpp_f32<0x128>(a));
  const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(a), 0));
  const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(a), 16));
  const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(a), 32));
  const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(a), 48));
  return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}
// unsigned minimum over the whole wave, in every lane (the whole wave active)
__device__ __forceinline__ uint32_t min_wave(uint32_t v) {
  v = min(v, (uint32_t)__builtin_amdgcn_update_dpp(-1, (int)v, 0xB1, 0xf, 0xf, false));
  v = min(v, (uint32_t)__builtin_amdgcn_update_dpp(-1, (int)v, 0x4E, 0xf, 0xf, false));
  v = min(v, (uint32_t)__builtin_amdgcn_update_dpp(-1, (int)v, 0x124, 0xf, 0xf, false));
  v = min(v, (uint32_t)__builtin_amdgcn_update_dpp(-1, (int)v, 0x128, 0xf, 0xf, false));
  const uint32_t lo = min((uint32_t)__builtin_amdgcn_readlane((int)v, 0), (uint32_t)__builtin_amdgcn_readlane((int)v, 16));
  const uint32_t hi = min((uint32_t)__builtin_amdgcn_readlane((int)v, 32), (uint32_t)__builtin_amdgcn_readlane((int)v, 48));
  return min(lo, hi);
}
// unsigned minimum over each aligned 32-lane half, in every lane of the half
__device__ __forceinline__ uint32_t min_half_wave(uint32_t v) {
  v = min(v, (uint32_t)__builtin_amdgcn_update_dpp(-1, (int)v, 0xB1, 0xf, 0xf, false));
  v = min(v, (uint32_t)__builtin_amdgcn_update_dpp(-1, (int)v, 0x4E, 0xf, 0xf, false));
  v = min(v, (uint32_t)__builtin_amdgcn_update_dpp(-1, (int)v, 0x124, 0xf, 0xf, false));
  v = min(v, (uint32_t)__builtin_amdgcn_update_dpp(-1, (int)v, 0x128, 0xf, 0xf, false));
  const uint32_t lo = min((uint32_t)__builtin_amdgcn_readlane((int)v, 0), (uint32_t)__builtin_amdgcn_readlane((int)v, 16));
  const uint32_t hi = min((uint32_t)__builtin_amdgcn_readlane((int)v, 32), (uint32_t)__builtin_amdgcn_readlane((int)v, 48));
  return (threadIdx.x & 32) ? hi : lo;
}
// integer sum over each aligned 32-lane half, in every lane of the half (exact)
__device__ __forceinline__ int sum_half_wave(int v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xf, 0xf, false);
  v += __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xf, 0xf, false);
  v += __builtin_amdgcn_update_dpp(0, v, 0x124, 0xf, 0xf, false);
  v += __builtin_amdgcn_update_dpp(0, v, 0x128, 0xf, 0xf, false);
  const int lo = __builtin_amdgcn_readlane(v, 0) + __builtin_amdgcn_readlane(v, 16);
  const int hi = __builtin_amdgcn_readlane(v, 32) + __builtin_amdgcn_readlane(v, 48);
  return (threadIdx.x & 32) ? hi : lo;
}

// Q8_0 quantization of one 32-value block held one value per lane by a 32-lane group
// (lanes 0-31 or 32-63 of a wave).  Returns the block's f16-valued scale (same in every
// lane); *q receives this lane's quant.  inference.rs:16953-16971.
__device__ __forceinline__ float quantize_lane32(float v, int8_t* q) {
  const float amax = max_half_wave(fabsf(v));
  const float unrounded = amax / 127.0f;
  const float scale = f16_bits_to_f32(f32_to_f16_bits(unrounded));
  const float inv = unrounded == 0.0f ? 0.0f : 1.0f / unrounded;
  float r = roundf(v * inv);
  r = fminf(fmaxf(r, -128.0f), 127.0f);
  *q = (int8_t)r;
  return scale;
}

// Q8_0 quantization of one 32-value block held 8 values per lane by a quad of lanes (lanes
// 4b..4b+3, values 8j..8j+7 in lane 4b+j; all four lanes active): the block's absolute
// maximum by two quad exchanges (exact), then each lane quantizes its 8 values; returns the
// f16-valued scale (every lane of the quad), packs the 8 quants into q[0..1].
// inference.rs:16953-16971.
__device__ __forceinline__ float quantize_quad8(const float (&y)[8], uint32_t (&q)[2]) {
  float amax = 0.0f;
#pragma unroll
  for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf(y[e]));
  amax = fmaxf(amax, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(amax), 0xB1, 0xF, 0xF, false)));  // xor 1
  amax = fmaxf(amax, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(amax), 0x4E, 0xF, 0xF, false)));  // xor 2
  const float unrounded = amax / 127.0f;
  const float scale = f16_bits_to_f32(f32_to_f16_bits(unrounded));
  const float inv = unrounded == 0.0f ? 0.0f : 1.0f / unrounded;
#pragma unroll
  for (int w = 0; w < 2; ++w) {
    uint32_t word = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float r = roundf(y[w * 4 + e] * inv);
      r = fminf(fmaxf(r, -128.0f), 127.0f);
      word |= ((uint32_t)(int32_t)r & 0xffu) << (8 * e);
    }
    q[w] = word;
  }
  return scale;
}

// Q8_0 quantization of one 32-element block held by one lane (inference.rs:16953-16971):
// returns the f16-rounded scale, writes the 32 quants as 8 packed words.
__device__ __forceinline__ float quantize_block_regs(const float (&y)[32], uint32_t (&packed)[8]) {
  float amax = 0.0f;
#pragma unroll
  for (int e = 0; e < 32; ++e) amax = fmaxf(amax, fabsf(y[e]));
  const float unrounded = amax / 127.0f;
  const float scale = f16_bits_to_f32(f32_to_f16_bits(unrounded));
  const float inv = unrounded == 0.0f ? 0.0f : 1.0f / unrounded;
#pragma unroll
  for (int w4 = 0; w4 < 8; ++w4) {
    uint32_t word = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float r = roundf(y[w4 * 4 + e] * inv);
      r = fminf(fmaxf(r, -128.0f), 127.0f);
      word |= ((uint32_t)(int32_t)r & 0xffu) << (8 * e);
    }
    packed[w4] = word;
  }
  return scale;
}

// ---------------------------------------------------------------------------
// Q8_K quantization (inference.rs:17564-17599 quantize_q8_k_blocks): per 256-value block,
// max = the signed value of the first largest |x| (a strict '>' scan from 0), iscale =
// -127/max, q = min(nearest_int(iscale*x), 127), d = 1/iscale; a block whose |x| never
// exceeds 0 gives d = 0 and zero quants.  nearest_int: inference.rs:17555-17561.
__device__ __forceinline__ int nearest_int_ref(float f) {
  const float v = f + 12582912.0f;
  return (int)(__float_as_uint(v) & 0x007fffffu) - 0x00400000;
}

// (|x|, index, x) of the first largest |x|: keep the incumbent unless the challenger is
// larger, or equal with a smaller index.
__device__ __forceinline__ void amax_pick(float& a, int& i, float& v, float oa, int oi, float ov) {
  if (oa > a || (oa == a && oi < i)) {
    a = oa;
    i = oi;
    v = ov;
  }
}

// The (|max|, first index) reduction across lanes by DPP exchanges (one VALU move per value,
// where a __shfl_xor is an LDS permute round trip).  amax_pick is a total order on (a, -i) for
// the non-NaN a the quantizers produce (a starts at 0 and only grows through '>'), so every
// reduction tree gives the same pick.
template <int CTRL>
__device__ __forceinline__ void amax_dpp(float& a, int& i, float& v, float& oa, int& oi, float& ov) {
  oa = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(a), CTRL, 0xf, 0xf, false));
  oi = __builtin_amdgcn_update_dpp(0, i, CTRL, 0xf, 0xf, false);
  ov = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}
template <int CTRL>
__device__ __forceinline__ void amax_pick_dpp(float& a, int& i, float& v) {
  float oa, ov;
  int oi;
  amax_dpp<CTRL>(a, i, v, oa, oi, ov);
  amax_pick(a, i, v, oa, oi, ov);
}
// every lane of each aligned quad: the quad's pick (xor-1, then xor-2 partners)
__device__ __forceinline__ void amax_pick_quad(float& a, int& i, float& v) {
  amax_pick_dpp<0xB1>(a, i, v);  // quad_perm [1,0,3,2]
  amax_pick_dpp<0x4E>(a, i, v);  // quad_perm [2,3,0,1]
}
// every lane of each aligned group of 8: the quads, then the other quad of the group (lane
// i ^ 4: row_ror:4 reads lane i - 4, row_ror:12 lane i + 4, within the row of 16)
__device__ __forceinline__ void amax_pick_group8(float& a, int& i, float& v) {
  amax_pick_quad(a, i, v);
  float oa4, ov4, oa12, ov12;
  int oi4, oi12;
  amax_dpp<0x124>(a, i, v, oa4, oi4, ov4);
  amax_dpp<0x12C>(a, i, v, oa12, oi12, ov12);
  const bool upper = (threadIdx.x & 4) != 0;
  amax_pick(a, i, v, upper ? oa4 : oa12, upper ? oi4 : oi12, upper ? ov4 : ov12);
}
// every lane of the wave: the quads, the row's four quads by rotations (lane i then holds
// quads i, i - 4, i - 8, i - 12 of its row), then the four rows' picks from lanes 0, 16, 32, 48
__device__ __forceinline__ void amax_pick_wave(float& a, int& i, float& v) {
  amax_pick_quad(a, i, v);
  amax_pick_dpp<0x124>(a, i, v);  // row_ror:4
  amax_pick_dpp<0x128>(a, i, v);  // row_ror:8
  float ra[4], rv[4];
  int ri[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    ra[r] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(a), 16 * r));
    ri[r] = __builtin_amdgcn_readlane(i, 16 * r);
    rv[r] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16 * r));
  }
  a = ra[0];
  i = ri[0];
  v = rv[0];
#pragma unroll
  for (int r = 1; r < 4; ++r) amax_pick(a, i, v, ra[r], ri[r], rv[r]);
}

// Q8_K block held as eight 32-value pieces by eight consecutive lanes (piece j = values
// 32j..32j+31 of the block, in lane j of the group): each lane writes its 32 quants and their
// sum; the group's first lane writes the block scale.
__device__ __forceinline__ void quantize_q8k_lanes8(const float (&y)[32], int8_t* __restrict__ q32,
                                                    int32_t* __restrict__ bsum, float* __restrict__ d_out) {
  const int j = threadIdx.x & 7;
  float a = 0.0f, v = 0.0f;
  int idx = 0x7fffffff;
#pragma unroll
  for (int e = 0; e < 32; ++e)
    if (fabsf(y[e]) > a) {
      a = fabsf(y[e]);
      v = y[e];
      idx = 32 * j + e;
    }
  amax_pick_group8(a, idx, v);
  const float iscale = a > 0.0f ? -127.0f / v : 0.0f;
  int sum = 0;
#pragma unroll
  for (int w4 = 0; w4 < 8; ++w4) {
    uint32_t word = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int q = a > 0.0f ? min(nearest_int_ref(iscale * y[w4 * 4 + e]), 127) : 0;
      sum += (int8_t)q;
      word |= ((uint32_t)q & 0xffu) << (8 * e);
    }
    reinterpret_cast<uint32_t*>(q32)[w4] = word;
  }
  *bsum = sum;
  if (j == 0) *d_out = a > 0.0f ? 1.0f / iscale : 0.0f;
}

// Q8_K block of a 256-thread workgroup, one value per thread (thread t = value t): writes
// the quants, the per-32 sums and the scale.  Every thread of the workgroup must call it.
__device__ __forceinline__ void quantize_q8k_wg256(float x, int8_t* __restrict__ yq, int32_t* __restrict__ ybs,
                                                   float* __restrict__ yd) {
  __shared__ float s_a[4], s_v[4];
  __shared__ int s_i[4];
  const int tid = threadIdx.x;
  float a = fabsf(x), v = x;
  int idx = tid;
  if (!(a > 0.0f)) a = 0.0f;  // zeros and NaN never win against the scan's initial 0
  amax_pick_wave(a, idx, v);
  if ((tid & 63) == 0) {
    s_a[tid >> 6] = a;
    s_i[tid >> 6] = idx;
    s_v[tid >> 6] = v;
  }
  __syncthreads();
  a = s_a[0];
  idx = s_i[0];
  v = s_v[0];
  for (int w = 1; w < 4; ++w) amax_pick(a, idx, v, s_a[w], s_i[w], s_v[w]);
  const float iscale = a > 0.0f ? -127.0f / v : 0.0f;
  const int q = a > 0.0f ? min(nearest_int_ref(iscale * x), 127) : 0;
  const int8_t q8 = (int8_t)q;
  yq[tid] = q8;
  const int bs = sum_half_wave(q8);
  if ((tid & 31) == 0) ybs[tid >> 5] = bs;
  if (tid == 0) *yd = a > 0.0f ? 1.0f / iscale : 0.0f;
}

__device__ __forceinline__ float block_max(float v, float* red) {
  v = max_wave(v);
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
// A workgroup of 4 waves owns 4*RPW consecutive rows; wave w owns rows RPW*w .. RPW*w+RPW-1.
// Lane l streams 16-byte chunks l, l+64, ... of each of its wave's rows (a wave load is
// 1 KB contiguous), so lane pairs (2j, 2j+1) hold the two halves of one 32-value block,
// combined by a DPP exchange (integer, exact).  Every weight and scale load of a wave is
// issued before the first dot.  Even lanes write the block's f32 term to LDS; then lane r
// of wave 0 folds row r's terms in block order.
constexpr int GEMV_R = 8;     // rows per workgroup of the runtime-width fallback
constexpr int GEMV_NT = 256;  // 4 waves

__host__ __device__ constexpr int gemv_term_stride(int nb) { return ((nb + 3) & ~3) + 4; }

// Shared body for a compile-time row width K and RPW rows per wave; returns (in lanes
// 0..4*RPW-1 of wave 0) the folded sum of row row0 + lane.
template <int K, int RPW>
__device__ __forceinline__ float gemv_rows_k(const int8_t* __restrict__ wq, const uint16_t* __restrict__ wd, int rows,
                                             const int8_t* __restrict__ xq, const float* __restrict__ xs, int row0) {
  constexpr int NB = K / 32, CPR = K / 16, IT = (CPR + 63) / 64, STRIDE = gemv_term_stride(NB);
  constexpr int R = 4 * RPW;
  static_assert(NB % 4 == 0, "compile-time GEMV widths are multiples of 128");
  __shared__ __align__(16) int8_t xl[K];
  __shared__ __align__(16) float xsl[NB];
  __shared__ __align__(16) float t[R * STRIDE];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  // issue this wave's weight and scale loads first (rows clamped: results of rows past the
  // end are computed but never stored)
  int4 wv[RPW][IT];
  uint16_t dv[RPW][IT];
#pragma unroll
  for (int k = 0; k < RPW; ++k) {
    const int row = min(row0 + wave * RPW + k, rows - 1);
    const int4* w4 = reinterpret_cast<const int4*>(wq + (size_t)row * K);
    const uint16_t* d = wd + (size_t)row * NB;
#pragma unroll
    for (int i = 0; i < IT; ++i) {
      const int c = min(lane + 64 * i, CPR - 1);
      wv[k][i] = ld_stream(w4 + c);
      dv[k][i] = ld_stream(d + (c >> 1));
    }
  }
  // stage the activation (K quants + NB scales) in LDS
  for (int c = tid; c < CPR; c += GEMV_NT) reinterpret_cast<int4*>(xl)[c] = reinterpret_cast<const int4*>(xq)[c];
  for (int b = tid; b < NB; b += GEMV_NT) xsl[b] = xs[b];
  __syncthreads();
#pragma unroll
  for (int k = 0; k < RPW; ++k) {
    float* tr = t + (wave * RPW + k) * STRIDE;
#pragma unroll
    for (int i = 0; i < IT; ++i) {
      // one chunk at a time: keeps the activation reads from being hoisted into registers
      // next to the in-flight weights (register count sets the workgroups per CU)
      __builtin_amdgcn_sched_barrier(0);
      const int c = lane + 64 * i;
      const int cc = min(c, CPR - 1);
      int s = dot4x4(wv[k][i], reinterpret_cast<const int4*>(xl)[cc], 0);
      s += dpp_xor1(s);
      if ((lane & 1) == 0 && c < CPR) tr[c >> 1] = ((float)s * half_bits_to_float(dv[k][i])) * xsl[c >> 1];
    }
  }
  __syncthreads();
  float acc = 0.0f;
  if (tid < R) acc = fold_lds_n<NB>(t + tid * STRIDE);
  return acc;
}

// Runtime-K fallback (any K % 32 == 0 whose LDS stage fits): same arithmetic, chunks dealt
// round-robin over the workgroup.
__host__ __device__ inline size_t gemv_term_offset(int K) { return ((size_t)K + (size_t)(K >> 5) * 4 + 15) & ~(size_t)15; }
__host__ __device__ inline size_t gemv_lds_bytes(int K) {
  return gemv_term_offset(K) + (size_t)GEMV_R * gemv_term_stride(K >> 5) * 4;
}

__device__ __forceinline__ float gemv_rows_rt(const int8_t* __restrict__ wq, const uint16_t* __restrict__ wd, int rows,
                                              int K, const int8_t* __restrict__ xq, const float* __restrict__ xs,
                                              int row0, unsigned char* smem) {
  const int nb = K >> 5;
  const int cpr = K >> 4;
  int8_t* xl = reinterpret_cast<int8_t*>(smem);
  float* xsl = reinterpret_cast<float*>(smem + K);
  float* t = reinterpret_cast<float*>(smem + gemv_term_offset(K));
  const int tid = threadIdx.x;
  for (int c = tid; c < cpr; c += GEMV_NT) reinterpret_cast<int4*>(xl)[c] = reinterpret_cast<const int4*>(xq)[c];
  for (int b = tid; b < nb; b += GEMV_NT) xsl[b] = xs[b];
  __syncthreads();
  const int nrows = min(GEMV_R, rows - row0);
  const int total = nrows * cpr;
  const int4* slab = reinterpret_cast<const int4*>(wq + (size_t)row0 * K);
  const uint16_t* dslab = wd + (size_t)row0 * nb;
  const int stride = gemv_term_stride(nb);
  const int iters = (GEMV_R * cpr + GEMV_NT - 1) / GEMV_NT;
  for (int it = 0; it < iters; ++it) {
    const int f = tid + it * GEMV_NT;
    const int fc = min(f, total - 1);
    const int r = fc / cpr;
    const int c = fc - r * cpr;
    int s = dot4x4(slab[fc], reinterpret_cast<const int4*>(xl)[c], 0);
    s += dpp_xor1(s);
    if ((tid & 1) == 0 && f < total) {
      const int b = c >> 1;
      t[r * stride + b] = ((float)s * half_bits_to_float(dslab[r * nb + b])) * xsl[b];
    }
  }
  __syncthreads();
  float acc = 0.0f;
  if (tid < nrows) acc = fold_lds(t + tid * stride, nb);
  return acc;
}

// K values with a compile-time specialisation (the configured model widths), and the
// rows per wave used for each: one row per wave keeps >= ~4 workgroups per CU on the
// smaller projections; two rows per wave halve the workgroup count of the large ones.
#define CM_GEMV_KS(X) X(2048) X(3072) X(4096) X(5632) X(8192) X(12288) X(14336)
__host__ __device__ constexpr int gemv_rpw(int K, int rows) { return (rows >= 16384 && K <= 4096) ? 2 : 1; }

template <int K, int RPW>
__global__ __launch_bounds__(GEMV_NT) void k_gemv_k(const int8_t* __restrict__ wq, const uint16_t* __restrict__ wd,
                                                    int rows, const int8_t* __restrict__ xq,
                                                    const float* __restrict__ xs, float* y, const float* resid) {
  const int row0 = blockIdx.x * (4 * RPW);
  const float acc = gemv_rows_k<K, RPW>(wq, wd, rows, xq, xs, row0);
  const int tid = threadIdx.x;
  if (tid < 4 * RPW && row0 + tid < rows) {
    const int row = row0 + tid;
    y[row] = resid ? resid[row] + acc : acc;
  }
}

__global__ __launch_bounds__(GEMV_NT) void k_gemv(const int8_t* __restrict__ wq, const uint16_t* __restrict__ wd,
                                                  int rows, int K, const int8_t* __restrict__ xq,
                                                  const float* __restrict__ xs, float* y, const float* resid) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int row0 = blockIdx.x * GEMV_R;
  const float acc = gemv_rows_rt(wq, wd, rows, K, xq, xs, row0, smem);
  const int tid = threadIdx.x;
  if (tid < GEMV_R && row0 + tid < rows) {
    const int row = row0 + tid;
    y[row] = resid ? resid[row] + acc : acc;
  }
}

// Serial fold in index order of N terms spaced `stride` floats apart in LDS (one lane; a
// block-major term layout [block][row], whose fold lanes - one per row - then read consecutive
// words), one 4-byte read per term, 8 terms ahead of the dependent add chain: 16 registers
// where the 16-byte reads of fold_lds take 64 (the looping gate/up GEMV folds with the next
// group's weights in flight).
template <int N>
__device__ __forceinline__ float fold_lds_strided(const float* p, int stride) {
  static_assert(N % 8 == 0 && N >= 8, "strided fold length must be a multiple of 8");
  float a[8], b[8];
#pragma unroll
  for (int u = 0; u < 8; ++u) a[u] = p[u * stride];
  float acc = 0.0f;
  int n = N;
  asm volatile("" : "+s"(n));  // keep the fold a loop (registers set the occupancy)
#pragma unroll 1
  for (int base = 8; base < n; base += 8) {
#pragma unroll
    for (int u = 0; u < 8; ++u) b[u] = p[(base + u) * stride];
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      acc += a[u];
      a[u] = b[u];
    }
    __builtin_amdgcn_sched_barrier(0);
  }
#pragma unroll
  for (int u = 0; u < 8; ++u) acc += a[u];
  return acc;
}

// ---------------------------------------------------------------------------
// RMSNorm fused into the GEMV that consumes it: every workgroup normalises the activation
// itself (the arithmetic of k_rmsnorm_quant) into LDS, so the norm needs no launch of its own.
// The workgroup splits into two teams.  The norm team (waves 0..GN_TEAM/64-1) loads x and the
// norm weights first, computes the norm with team-only synchronisation (TeamBar) and only
// then loads its own weight rows; the other waves issue all their weight loads at once.  The
// CU's share of HBM bandwidth, not the norm, then sets the kernel's time: a wave that issues
// into a full memory queue stalls, but no norm barrier waits for the weight waves.
constexpr int GN_NT = 1024;
constexpr int GN_TEAM = 256;      // threads of the gate/up kernel's norm team
constexpr int GN_TEAM_QKV = 512;  // threads of the qkv kernel's norm team (its weight waves hold every row)


// The norm team's share of x and w: thread t holds the C consecutive values t*C.. (the layout
// of inorder_sum_onepass).
template <int C>
__device__ __forceinline__ void norm_load_team(const float* __restrict__ x, const float* __restrict__ w, int n,
                                               float (&xv)[C], float (&wv)[C]) {
  const int i0 = threadIdx.x * C;
#pragma unroll
  for (int c = 0; c < C; ++c) {
    const bool in = i0 + c < n;
    xv[c] = in ? x[i0 + c] : 0.0f;
    wv[c] = in ? w[i0 + c] : 0.0f;
  }
}

// The RMSNorm's scale (tensor/mod.rs:2083-2106): the in-order sum of the squares of the n
// values xv (thread t holds t*C..), scale = 1/sqrt(ss/n + eps), written to *s_scale by thread
// 0.  Called by the NT threads that hold the values, synchronised by `bar` (the whole
// workgroup or a TeamBar; no bar() after the sum: the caller's workgroup barrier publishes
// the scale).  x and w are also copied to the LDS arrays xf and wf for norm_quantize_all; yl
// (NT*C floats) holds the squares for the sum's fallback.
template <int NT, int C, typename Bar = WgBar>
__device__ __forceinline__ void norm_scale(const float (&xv)[C], const float (&wv)[C], int n, float eps, float* xf,
                                           float* wf, float* yl, FsLds<NT>& fs, float* s_scale, Bar&& bar = Bar{},
                                           int stamp_kind = -1) {
  const int tid = threadIdx.x, i0 = tid * C;
  (void)stamp_kind;
  float t[C];
#pragma unroll
  for (int c = 0; c < C; ++c) {
    t[c] = xv[c] * xv[c];
    if (i0 + c < n) {
      yl[i0 + c] = t[c];  // the sum's fallback reads the squares here
      xf[i0 + c] = xv[c];
      wf[i0 + c] = wv[c];
    }
  }
  if (stamp_kind >= 0) {
    CM_GEMV_STAMP(stamp_kind, 6, 0)  // (the measurement build: x and w have arrived)
  }
  const float ss = inorder_sum_onepass<NT, C, true>(t, yl, n, fs, bar, stamp_kind);
  if (tid == 0) *s_scale = 1.0f / sqrtf(ss / (float)n + eps);
  if (stamp_kind >= 0) {
    CM_GEMV_STAMP(stamp_kind, 7, 0)  // the sum of squares is known
  }
}

// The normalised values y = (x * scale) * w of xf/wf (LDS, 16-byte aligned, n % 32 == 0),
// Q8_0-quantized into LDS (xl: n quants, xsl: n/32 scales) by the whole workgroup (NTALL
// threads, a multiple of 64): each quad of lanes quantizes one 32-value block, 8 values per
// lane (quantize_quad8).  The caller synchronises before (scale, xf, wf written) and after
// (xl, xsl read).
template <int NTALL>
__device__ __forceinline__ void norm_quantize_all(const float* xf, const float* wf, int n, float scale, int8_t* xl,
                                                  float* xsl) {
  for (int p = threadIdx.x; p < (n >> 3); p += NTALL) {  // (uniform per quad: n % 32 == 0)
    const float4* xp = reinterpret_cast<const float4*>(xf) + 2 * p;
    const float4* wp = reinterpret_cast<const float4*>(wf) + 2 * p;
    const float4 x0 = xp[0], x1 = xp[1], w0 = wp[0], w1 = wp[1];
    const float y[8] = {(x0.x * scale) * w0.x, (x0.y * scale) * w0.y, (x0.z * scale) * w0.z, (x0.w * scale) * w0.w,
                        (x1.x * scale) * w1.x, (x1.y * scale) * w1.y, (x1.z * scale) * w1.z, (x1.w * scale) * w1.w};
    uint32_t q[2];
    const float d = quantize_quad8(y, q);
    reinterpret_cast<uint2*>(xl)[p] = make_uint2(q[0], q[1]);
    if ((p & 3) == 0) xsl[p >> 2] = d;
  }
}

// The norm team's LDS: its counter and failure word (TeamBar), its one-pass-sum workspace.
template <int NTEAM>
struct NormTeamLds {
  uint32_t ctr;
  uint32_t bad;
  float scale;
  FsLds<NTEAM> fs;
};

// ---------------------------------------------------------------------------
// KV cache layout.  Per layer and kv head a region of hd * kvs elements (kvs: the position
// stride, a multiple of 8) at kv_head_base; inside it, f16 bits,
//   K: [hd/8][kvs][8]  -- 16-byte granule = 8 dims of one position,
//   V: [kvs/8][hd][8]  -- 16-byte granule = 8 positions of one dim,
// so that lanes over consecutive positions (scores) or consecutive dims (the output sum)
// read consecutive granules.  Both products (q * k, p * v) are one mixed-precision FMA on
// the f16 value, so each position costs the serial add chain two VALU operations.
__host__ __device__ __forceinline__ size_t kv_head_base(int layer, int n_kv, int kvh, int hd, int kvs) {
  return ((size_t)layer * n_kv + kvh) * (size_t)hd * kvs;
}
__host__ __device__ __forceinline__ size_t kv_k_index(int kvs, int p, int d) {
  return ((size_t)(d >> 3) * kvs + p) * 8 + (d & 7);
}
__host__ __device__ __forceinline__ size_t kv_v_index(int hd, int p, int d) {
  return ((size_t)(p >> 3) * hd + d) * 8 + (p & 7);
}

// Read-ahead of one layer's KV cache into the L2 of the XCD whose attention workgroups will
// read it.  Workgroup b of a launch runs on XCD b % 8, each XCD has an L2 of its own, and an
// L2 line stays valid across kernel boundaries (measured on MI355X: a line read by one kernel
// is hit at ~93 ns by the next kernel's workgroups on the same XCD, ~235 ns from other XCDs,
// ~370 ns cold).  The single-workgroup decode attention maps its workgroup b to head
// xcd_member(b, n_kv, rep); the read-ahead workgroups on XCD x touch one word of every
// 128-byte line of the K and V rows [0, pos) of the KV heads that those heads read, so that
// the attention's K-row loads and V staging hit the L2 instead of HBM.  Loads only; pos (the
// row the attention kernel itself writes) and beyond are not touched.  nwg % 8 == 0 workgroups
// after the owning kernel's own; a position outside the cache reads nothing.
// Workgroups are dealt to the 8 XCDs round-robin (workgroup b runs on XCD b % 8), and each
// XCD has an L2 of its own.  The attention workgroups that read the same KV rows (the query
// heads of one KV head; with `parts` workgroups per head, the same part of them) are mapped
// to one XCD, so that the rows come from HBM once and from that L2 for the rest.  Workgroup b
// of n_kv * parts * rep returns its (kv unit, member) as kv_unit * rep + member, where kv unit
// u = kv_head * parts + part; the identity when the units do not divide over the XCDs.
constexpr int N_XCD = 8;
__device__ __forceinline__ int xcd_member(int b, int n_units, int rep) {
  if (n_units % N_XCD != 0) return b;
  const int x = b % N_XCD, i = b / N_XCD;
  return (x + N_XCD * (i / rep)) * rep + i % rep;
}

struct KvAhead {
  const uint16_t* kc;
  const uint16_t* vc;
  const uint32_t* d_pos;
  int layer, n_heads, n_kv, hd, kvs;
  int on;  // 0: no read-ahead
};

// The read-ahead share of lane `lane` of `nlanes` in workgroup b of a grid of `nwg`
// workgroups (b runs on XCD b % 8; the workgroups of one XCD split its lines).
__device__ __forceinline__ void kv_ahead(const KvAhead& a, int b, int nwg, int lane, int nlanes) {
  const int x = b % N_XCD, member = b / N_XCD, members = (nwg - x + N_XCD - 1) / N_XCD;
  const int pos = (int)*a.d_pos;
  if (pos <= 0 || pos >= a.kvs) return;
  const int rep = a.n_heads / a.n_kv;
  const size_t kstripe = (size_t)((pos + 7) / 8);         // lines of one K stripe (8 dims, positions [0, pos))
  const size_t lines_per_head = (size_t)(a.hd / 8) * kstripe;  // of K, and of V
  const size_t stride = (size_t)members * nlanes;
  uint32_t acc = 0;
  int last = -1;
  for (int w = x; w < a.n_heads; w += N_XCD) {
    const int kvh = xcd_member(w, a.n_kv, rep) / rep;
    if (kvh == last) continue;  // (consecutive heads of one group share their rows)
    last = kvh;
    const size_t base = kv_head_base(a.layer, a.n_kv, kvh, a.hd, a.kvs);
    const uint32_t* k32 = reinterpret_cast<const uint32_t*>(a.kc + base);
    const uint32_t* v32 = reinterpret_cast<const uint32_t*>(a.vc + base);
    for (size_t l = (size_t)member * nlanes + lane; l < 2 * lines_per_head; l += stride) {
      if (l < lines_per_head) {
        const size_t u = l / kstripe, r = l - u * kstripe;  // stripe u (dims 8u..8u+7), line r
        acc ^= k32[(u * (size_t)a.kvs * 16 + r * 128) / 4];
      } else {
        acc ^= v32[(l - lines_per_head) * 32];
      }
    }
  }
  asm volatile("" ::"v"(acc));  // keeps the loads
}

// Row stride of a block-major term layout [block][row]: an odd word count, so that the lanes
// writing one row's terms (one block each) and the lanes folding the rows (one row each) both
// touch distinct LDS banks.
__host__ __device__ constexpr int gemv_row_stride(int rows) { return rows | 1; }

// y = W · rmsnorm(x) for a Q8_0 W [rows][K]: workgroup b takes rows b*rows_per_wg .. (at most
// 8 * RPW, all held by the 8 weight waves): the norm team (8 waves) computes the norm while
// the weight waves' loads stream, then the same per-row block dots and in-order folds as
// k_gemv_k.
template <int K, int RPW>
__global__ __launch_bounds__(GN_NT) void k_gemv_norm(const int8_t* __restrict__ wq, const uint16_t* __restrict__ wd,
                                                     int rows, int rows_per_wg, const float* __restrict__ x,
                                                     const float* __restrict__ nw, float eps, float* __restrict__ y,
                                                     KvAhead kva) {
  constexpr int NB = K / 32, CPR = K / 16, IT = (CPR + 63) / 64;
  constexpr int NT = GN_TEAM_QKV;  // the norm team: waves 0..TW-1; waves TW.. hold the rows
  constexpr int NWV = GN_NT / 64, R = NWV * RPW, C = (K + NT - 1) / NT, TW = NT / 64;
  constexpr int ST = gemv_term_stride(NB);  // terms row-major: t[slot * ST + block]
  __shared__ __align__(16) int8_t xl[K];
  __shared__ __align__(16) float xsl[NB];
  __shared__ __align__(16) float t[R * ST];
  __shared__ __align__(16) float yl[NT * C];
  __shared__ __align__(16) float xf[NT * C];
  __shared__ __align__(16) float wf[NT * C];
  __shared__ NormTeamLds<NT> team;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const bool in_team = wave < TW;  // (wave-uniform)
  const int row0 = blockIdx.x * rows_per_wg;
  const int nrows = min(rows_per_wg, rows - row0);
  CM_GEMV_STAMP(0, 0, 0)
  float nxv[C], nwv[C];
  if (in_team) norm_load_team<C>(x, nw, K, nxv, nwv);
  if (tid == 0) {
    team.ctr = 0u;
    team.bad = 0u;
  }
  // the norm's loads are issued ahead of every weight load; the team counter is zeroed
  __syncthreads();
  // local row slots: the weight waves' first (slot (wave - TW) + k (NWV - TW)), the norm
  // team's last, so that rows_per_wg <= (NWV - TW) * RPW rows all stream during the norm;
  // slots past nrows load nothing and store nothing
  auto slot_of = [&](int k) {
    return in_team ? (NWV - TW) * RPW + wave + TW * k : (wave - TW) + (NWV - TW) * k;
  };
  int4 wv[RPW][IT];
  uint16_t dv[RPW][IT];
  auto load_row = [&](int k) {
    const int sl = slot_of(k);
    if (sl >= nrows) return;  // (wave-uniform)
    const int4* w4 = reinterpret_cast<const int4*>(wq + (size_t)(row0 + sl) * K);
    const uint16_t* d = wd + (size_t)(row0 + sl) * NB;
#pragma unroll
    for (int i = 0; i < IT; ++i) {
      const int c = min(lane + 64 * i, CPR - 1);
      wv[k][i] = ld_stream(w4 + c);
      dv[k][i] = ld_stream(d + (c >> 1));
    }
  };
  if (in_team) {
    norm_scale<NT, C>(nxv, nwv, K, eps, xf, wf, yl, team.fs, &team.scale, TeamBar{&team.ctr, &team.bad, TW, 0u}, 0);
    CM_GEMV_STAMP(0, 1, 0)
  }
#pragma unroll
  for (int k = 0; k < RPW; ++k) load_row(k);
  CM_GEMV_STAMP(0, 2, NT)
  __syncthreads();  // the scale and x, w are in LDS for every wave
  norm_quantize_all<GN_NT>(xf, wf, K, team.scale, xl, xsl);
  __syncthreads();  // the normalised activation (Q8_0) is in LDS
  CM_GEMV_STAMP(0, 3, 0)
  // (the weight scale enters as the raw f16 operand of a mixed-precision multiply, exactly
  // float(sacc) * f32(scale) rounded once: a separate f16->f32 conversion was placed by the
  // compiler right behind each row's loads inside the conditional load block, which made the
  // wave wait for every row before issuing the next one)
#pragma unroll
  for (int k = 0; k < RPW; ++k) {
    const int sl = slot_of(k);
    if (sl >= nrows) continue;  // (wave-uniform)
#pragma unroll
    for (int i = 0; i < IT; ++i) {
      __builtin_amdgcn_sched_barrier(0);
      const int c = lane + 64 * i;
      const int cc = min(c, CPR - 1);
      int sacc = dot4x4(wv[k][i], reinterpret_cast<const int4*>(xl)[cc], 0);
      sacc += dpp_xor1(sacc);
      if ((lane & 1) == 0 && c < CPR)
        t[sl * ST + (c >> 1)] = mul_f16_lo((float)sacc, dv[k][i]) * xsl[c >> 1];
    }
  }
  CM_GEMV_STAMP(0, 4, 0)
  __syncthreads();
  if (tid < nrows) y[row0 + tid] = team.bad ? __builtin_nanf("") : fold_lds_n<NB>(t + tid * ST);
  // the norm team's other waves, idle from here on: the KV rows of the attention that follows
  // into their XCD's L2 (nothing waits on these loads but the end of the kernel, which the
  // folds of wave 0 hold up longer)
  if (kva.on && wave >= 1 && wave < TW) kv_ahead(kva, blockIdx.x, gridDim.x, tid - 64, NT - 64);
  CM_GEMV_STAMP(0, 5, 0)
}

// Gate/up projection fused with SwiGLU (tensor/mod.rs:1943-1967) and the Q8_0 quantization
// of the activation.  The matrix rows are interleaved in groups of 32: group g holds gate
// rows 32g..32g+31 followed by up rows 32g..32g+31, so one workgroup (8 waves, 8 rows each)
// computes both halves of one 32-value block of the activation: the same per-row block
// dots and in-order folds as k_gemv_k, then silu(gate) * up and the block's quantization.
constexpr int GU_NT = 512;
constexpr int GU_ROWS = 64;  // rows per workgroup: 32 gate + 32 up
__host__ __device__ constexpr bool gu_fused_k(int K) { return K == 2048 || K == 3072 || K == 4096; }
// widths whose gate/up kernel also takes the RMSNorm
__host__ __device__ constexpr bool gu_norm_k(int K) { return K == 2048 || K == 3072 || K == 4096; }

// NORM: the activation is the RMSNorm of x (weights nw), computed by every workgroup in its
// prologue (norm_scale by the norm team, norm_quantize_all) instead of read quantized from
// xq/xs.
// groups: the 64-row groups of the matrix (ffn / 32), one per workgroup.  LOOP: workgroup b takes
// groups b, b + grid, ... (a grid of fewer workgroups than groups, where the groups do not all
// fit the CUs at once): each workgroup forms the activation once and issues the next group's
// weight loads as soon as the current group's block dots have consumed its registers, so that
// they stream while the current group's rows are folded, instead of a second round of
// workgroups starting behind the first one's fold tails.  (Its own instantiation: the loop's
// live state costs registers that the one-group launches do not pay.)
template <int K, int NT, bool NORM, bool LOOP = false>
__global__ __launch_bounds__(NT) void k_gemv_gu_silu(const int8_t* __restrict__ wq, const uint16_t* __restrict__ wd,
                                                    const int8_t* __restrict__ xq, const float* __restrict__ xs,
                                                    const float* __restrict__ x, const float* __restrict__ nw,
                                                    float eps, int8_t* __restrict__ aq, float* __restrict__ as,
                                                    int groups) {
  constexpr int NB = K / 32, CPR = K / 16, IT = (CPR + 63) / 64;
  // terms row-major, t[row * ST + block], folded with 16-byte reads (fold_lds_n: 1.25
  // instructions per term); LOOP: block-major, t[block * ST + row], folded with 4-byte reads
  // (fold_lds_strided: 16 registers, where the next group's weights are in flight)
  constexpr int ST = LOOP ? gemv_row_stride(GU_ROWS) : gemv_term_stride(NB);
  // row slots per wave: 8 at 512 threads; with NORM the weight waves' slots come first (up to
  // K = 3072 six each: all 64 rows stream during the norm; at 4096, where six rows of
  // registers do not fit, four each and the norm team's slots take the last 16 rows)
  constexpr int TW = NORM ? GN_TEAM / 64 : 0;  // norm-team waves
  constexpr int NWW = NT / 64 - TW;           // weight waves
  constexpr int RPW = NORM ? (K <= 3072 ? 6 : 4) : GU_ROWS / (NT / 64);
  constexpr int CT = (K + GN_TEAM - 1) / GN_TEAM;  // norm values per norm-team thread
  static_assert(NB % 4 == 0 && (NORM || GU_ROWS % (NT / 64) == 0), "compile-time GEMV widths are multiples of 128");
  __shared__ __align__(16) int8_t xl[K];
  __shared__ __align__(16) float xsl[NB];
  __shared__ __align__(16) float t[LOOP ? NB * ST : GU_ROWS * ST];
  __shared__ __align__(16) float vals[GU_ROWS];
  __shared__ __align__(16) float yl[NORM ? GN_TEAM * CT : 4];
  __shared__ __align__(16) float xf[NORM ? GN_TEAM * CT : 4];
  __shared__ __align__(16) float wf[NORM ? GN_TEAM * CT : 4];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const bool in_team = NORM && wave < GN_TEAM / 64;  // (wave-uniform) the norm team, as in k_gemv_norm
  uint32_t g = blockIdx.x;  // this workgroup's current group
  if constexpr (LOOP) {
    if (g >= (uint32_t)groups) return;  // (uniform; the engine's grid has none such)
  }
  size_t row0 = (size_t)g * GU_ROWS;
  float nxv[NORM ? CT : 1], nwv[NORM ? CT : 1];
  __shared__ NormTeamLds<GN_TEAM> team;
  CM_GEMV_STAMP(1, 0, 0)
  if constexpr (NORM) {
    if (in_team) norm_load_team<CT>(x, nw, K, nxv, nwv);
    if (tid == 0) {
      team.ctr = 0u;
      team.bad = 0u;
    }
    __syncthreads();  // the norm's loads ahead of every weight load; the team counter zeroed
  }
  // the wave's weight and scale loads: all up front; the norm team's after its norm
  int4 wv[RPW][IT];
  uint16_t dv[RPW][IT];
  // local row of slot k of this wave (-1: none): rows wave*RPW + k without NORM; with NORM the
  // weight waves' slots (wave - TW) + NWW k, then the norm team's NWW RPW + wave + TW k
  auto row_of = [&](int k) {
    const int r = NORM ? (in_team ? NWW * RPW + wave + TW * k : (wave - TW) + NWW * k) : wave * RPW + k;
    return r < GU_ROWS ? r : -1;
  };
  auto load_row = [&](int k) {
    const int lr = row_of(k);
    if (lr < 0) return;  // (wave-uniform)
    const size_t row = row0 + lr;
    const int4* w4 = reinterpret_cast<const int4*>(wq + row * K);
    const uint16_t* d = wd + row * NB;
#pragma unroll
    for (int i = 0; i < IT; ++i) {
      const int c = min(lane + 64 * i, CPR - 1);
      wv[k][i] = ld_stream(w4 + c);
      dv[k][i] = ld_stream(d + (c >> 1));
    }
  };
  if constexpr (NORM) {
    if (in_team) {
      norm_scale<GN_TEAM, CT>(nxv, nwv, K, eps, xf, wf, yl, team.fs, &team.scale,
                              TeamBar{&team.ctr, &team.bad, GN_TEAM / 64, 0u}, 1);
      CM_GEMV_STAMP(1, 1, 0)
    }
#pragma unroll
    for (int k = 0; k < RPW; ++k) load_row(k);
    CM_GEMV_STAMP(1, 2, GN_TEAM)
    __syncthreads();  // the scale and x, w are in LDS for every wave
    norm_quantize_all<NT>(xf, wf, K, team.scale, xl, xsl);
    __syncthreads();  // the normalised activation (Q8_0) is in LDS
    CM_GEMV_STAMP(1, 3, 0)
  } else {
#pragma unroll
    for (int k = 0; k < RPW; ++k) load_row(k);
    for (int c = tid; c < CPR; c += NT) reinterpret_cast<int4*>(xl)[c] = reinterpret_cast<const int4*>(xq)[c];
    for (int b = tid; b < NB; b += NT) xsl[b] = xs[b];
    __syncthreads();
  }
  for (;;) {
#pragma unroll
    for (int k = 0; k < RPW; ++k) {
      const int lr = row_of(k);
      if (lr < 0) continue;  // (wave-uniform)
#pragma unroll
      for (int i = 0; i < IT; ++i) {
        __builtin_amdgcn_sched_barrier(0);
        const int c = lane + 64 * i;
        const int cc = min(c, CPR - 1);
        int sacc = dot4x4(wv[k][i], reinterpret_cast<const int4*>(xl)[cc], 0);
        sacc += dpp_xor1(sacc);
        if ((lane & 1) == 0 && c < CPR)
          t[LOOP ? (c >> 1) * ST + lr : lr * ST + (c >> 1)] = mul_f16_lo((float)sacc, dv[k][i]) * xsl[c >> 1];
      }
    }
    CM_GEMV_STAMP(1, 4, 0)
    // the next group's weights (every wave's slots, the team's included) go out now
    const uint32_t gn = g + gridDim.x;
    if (LOOP && gn < (uint32_t)groups) {
      row0 = (size_t)gn * GU_ROWS;
#pragma unroll
      for (int k = 0; k < RPW; ++k) load_row(k);
    }
    __syncthreads();
    if (tid < GU_ROWS)  // one lane per row
      vals[tid] = NORM && team.bad ? __builtin_nanf("")
                                   : (LOOP ? fold_lds_strided<NB>(t + tid, ST) : fold_lds_n<NB>(t + tid * ST));
    __syncthreads();  // (also: every fold has read t, which the next group's dots rewrite)
    if (tid < 32) {  // SwiGLU and the block's Q8_0 quantization, one value per lane
      int8_t q;
      const float d = quantize_lane32(silu_mul1(vals[tid], vals[32 + tid]), &q);
      aq[(size_t)g * 32 + tid] = q;
      if (tid == 0) as[g] = d;
    }
    CM_GEMV_STAMP(1, 5, 0)
    if (!LOOP || gn >= (uint32_t)groups) break;
    g = gn;
  }
}

// Decode-loop state shared by the step's kernels (device memory).
struct StepState {
  uint32_t pos;      // position of the token being computed
  uint32_t tok;      // current token (input of the next step)
  uint32_t step;     // index into the generated-token ring
  uint32_t pad;
};

// lm_head GEMV fused with greedy argmax (inference.rs:5912-5925: first index of the max,
// strict '>').  Each workgroup reduces its rows to (value, index) with ties to the lower
// index; the last workgroup to finish (atomic ticket) reduces the partials in the same
// way, writes the token, appends it to tokens[step] and advances the position.
// K = 0 selects the runtime-width body.
__device__ __forceinline__ void argmax_pair(float& bv, uint32_t& bi, float ov, uint32_t oi) {
  if (ov > bv || (ov == bv && oi < bi)) {
    bv = ov;
    bi = oi;
  }
}
// argmax_pair over the whole wave, in every lane: a total order on (value, -index) for the
// non-NaN values it admits (NaN never replaces the running pair), so any reduction tree gives
// the first index of the maximum; DPP quad and row exchanges, then the four rows' pairs
template <int CTRL>
__device__ __forceinline__ void argmax_dpp(float& bv, uint32_t& bi) {
  argmax_pair(bv, bi, dpp_f32<CTRL>(bv), (uint32_t)__builtin_amdgcn_update_dpp(0, (int)bi, CTRL, 0xf, 0xf, false));
}
__device__ __forceinline__ void argmax_wave(float& bv, uint32_t& bi) {
  argmax_dpp<0xB1>(bv, bi);
  argmax_dpp<0x4E>(bv, bi);
  argmax_dpp<0x124>(bv, bi);
  argmax_dpp<0x128>(bv, bi);
  float rv[4];
  uint32_t ri[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    rv[r] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(bv), 16 * r));
    ri[r] = (uint32_t)__builtin_amdgcn_readlane((int)bi, 16 * r);
  }
  bv = rv[0];
  bi = ri[0];
#pragma unroll
  for (int r = 1; r < 4; ++r) argmax_pair(bv, bi, rv[r], ri[r]);
}

// lm_head: the GEMV writes the logits and, per workgroup, its (value, index) argmax
// partial; k_argmax_finish (one workgroup, the next launch) reduces the partials, writes
// the token, appends it to tokens[step] and advances the position.  K = 0 selects the
// runtime-width body.
template <int K, int RPW>
__global__ __launch_bounds__(GEMV_NT) void k_gemv_argmax(const int8_t* __restrict__ wq,
                                                         const uint16_t* __restrict__ wd, int rows, int k_rt,
                                                         const int8_t* __restrict__ xq, const float* __restrict__ xs,
                                                         float* __restrict__ logits, float* __restrict__ part_v,
                                                         uint32_t* __restrict__ part_i) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int R = K > 0 ? 4 * RPW : GEMV_R;
  const int row0 = blockIdx.x * R;
  float acc;
  if constexpr (K > 0) {
    acc = gemv_rows_k<K, RPW>(wq, wd, rows, xq, xs, row0);
  } else {
    acc = gemv_rows_rt(wq, wd, rows, k_rt, xq, xs, row0, smem);
  }
  const int tid = threadIdx.x;
  if (tid < 64) {
    float bv = -INFINITY;
    uint32_t bi = 0xffffffffu;
    if (tid < R && row0 + tid < rows) {
      logits[row0 + tid] = acc;
      argmax_pair(bv, bi, acc, (uint32_t)(row0 + tid));
    }
    argmax_wave(bv, bi);
    if (tid == 0) {
      part_v[blockIdx.x] = bv;
      part_i[blockIdx.x] = bi;
    }
  }
}

__global__ __launch_bounds__(1024) void k_argmax_finish(const float* __restrict__ part_v,
                                                        const uint32_t* __restrict__ part_i, int nparts, StepState* st,
                                                        uint32_t* __restrict__ tokens, uint32_t tokens_cap) {
  __shared__ float rv[16];
  __shared__ uint32_t ri[16];
  const int tid = threadIdx.x;
  float bv = -INFINITY;
  uint32_t bi = 0xffffffffu;
  for (int base = 0; base < nparts; base += 1024 * 8) {  // 8 pairs per lane in flight
    float v[8];
    uint32_t ix[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int i = base + tid + u * 1024;
      v[u] = i < nparts ? part_v[i] : -INFINITY;
      ix[u] = i < nparts ? part_i[i] : 0xffffffffu;
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) argmax_pair(bv, bi, v[u], ix[u]);
  }
  argmax_wave(bv, bi);
  if ((tid & 63) == 0) {
    rv[tid >> 6] = bv;
    ri[tid >> 6] = bi;
  }
  __syncthreads();
  if (tid == 0) {
    for (int w = 1; w < 16; ++w) argmax_pair(bv, bi, rv[w], ri[w]);
    const uint32_t tok = bi == 0xffffffffu ? 0u : bi;  // all -inf: index 0, as the CPU loop
    st->tok = tok;
    const uint32_t s = st->step;
    if (tokens && s < tokens_cap) tokens[s] = tok;
    st->step = s + 1;
    st->pos = st->pos + 1;
  }
}

// ---------------------------------------------------------------------------
// Read-ahead of the next projection's weights by the spare workgroups of a latency-bound
// kernel (the RMSNorm and attention kernels use one or a few CUs for several
// microseconds): one 4-byte load per 128-byte line pulls the lines into the L2 / MALL
// caches, so that the GEMV that follows streams them from cache.  Two regions (the int8
// quants and the f16 scales of a Q8R matrix); worker `wg` of `nwg`.  Loads only.
struct Prefetch {
  const uint32_t* a;
  size_t a_lines;
  const uint32_t* b;
  size_t b_lines;
};

__device__ __forceinline__ uint32_t prefetch_line(const Prefetch& pf, size_t l) {
  return l < pf.a_lines ? pf.a[l * 32] : pf.b[(l - pf.a_lines) * 32];
}

__device__ __forceinline__ void prefetch_lines(const Prefetch& pf, int wg, int nwg, float* sink_lds) {
  const size_t stride = (size_t)nwg * blockDim.x;
  uint32_t acc = 0;
  const size_t total = pf.a_lines + pf.b_lines;
  size_t i = (size_t)wg * blockDim.x + threadIdx.x;
  for (; i + 7 * stride < total; i += 8 * stride) {
    uint32_t v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = prefetch_line(pf, i + u * stride);
#pragma unroll
    for (int u = 0; u < 8; ++u) acc ^= v[u];
  }
  for (; i < total; i += stride) acc ^= prefetch_line(pf, i);
  if (acc == 0x9e3779b9u && pf.a_lines == 1) sink_lds[0] = 0.0f;  // keeps the loads
}

// ---------------------------------------------------------------------------
// RMSNorm (tensor/mod.rs:2083-2106) fused with Q8_0 quantization of the result.
// Workgroup 0 (RMS_NT threads) computes it; any further workgroups read ahead `pf`.  Thread t
// owns the 32-element blocks t + RMS_NT b: it loads their x and w values up front (16-byte
// loads, all in flight together), writes the squares to LDS for the in-order sum
// (inorder_sum_onepass, C consecutive terms per thread: bit-identical to the sequential
// fold), then normalises and quantizes its blocks from registers, with no cross-lane
// traffic.  1024 threads: the sum's per-thread work is short and four waves per SIMD hide
// each other's latencies.  n % 32 == 0, n <= RMS_NT * C.
constexpr int RMS_NT = 1024;
#define CM_RMS_CHUNKS(X) X(1) X(2) X(3) X(4) X(5) X(6) X(8) X(12) X(16)
__host__ __device__ constexpr int rms_chunk(int n) {
  return n <= 1024 ? 1 : n <= 2048 ? 2 : n <= 3072 ? 3 : n <= 4096 ? 4 : n <= 5120 ? 5 : n <= 6144 ? 6
       : n <= 8192 ? 8 : n <= 12288 ? 12 : 16;
}

__device__ __forceinline__ float4 mul4(const float4 a, const float4 b) {
  return make_float4(a.x * b.x, a.y * b.y, a.z * b.z, a.w * b.w);
}

template <int C>
__global__ __launch_bounds__(RMS_NT) void k_rmsnorm_quant(const float* __restrict__ x, const float* __restrict__ w,
                                                          int n, float eps, int8_t* __restrict__ xq,
                                                          float* __restrict__ xs, float* __restrict__ y_out,
                                                          Prefetch pf, float* __restrict__ kd,
                                                          int8_t* __restrict__ kq, int32_t* __restrict__ kbs) {
  constexpr int BPT = (C + 31) / 32;  // blocks per thread
  __shared__ __align__(16) float sq[RMS_NT * C];
  __shared__ __align__(16) float wl[RMS_NT * C];  // w waits here during the sum (registers are short)
  if (blockIdx.x > 0) {  // spare workgroups: read ahead the next projection's weights
    prefetch_lines(pf, blockIdx.x - 1, gridDim.x - 1, sq);
    return;
  }
  {  // row blockIdx.y of a [rows][n] batch (prefill); row 0 in the decode step
    const size_t row = blockIdx.y;
    x += row * n;
    xq += row * n;
    xs += row * (n >> 5);
    if (y_out) y_out += row * n;
    if (kd) {
      kd += row * (n >> 8);
      kq += row * n;
      kbs += row * (n >> 5);
    }
  }
  const int tid = threadIdx.x;
  const int nb = n >> 5;
  float4 xv[BPT][8], wv[BPT][8];
#pragma unroll
  for (int b = 0; b < BPT; ++b) {
    const int blk = tid + b * RMS_NT;
    if (blk < nb) {
      const float4* xp = reinterpret_cast<const float4*>(x + blk * 32);
      const float4* wp = reinterpret_cast<const float4*>(w + blk * 32);
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        xv[b][u] = xp[u];
        wv[b][u] = wp[u];
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        reinterpret_cast<float4*>(sq + blk * 32)[u] = mul4(xv[b][u], xv[b][u]);
        reinterpret_cast<float4*>(wl + blk * 32)[u] = wv[b][u];
      }
    }
  }
  __syncthreads();
  __shared__ FsLds<RMS_NT> fs;
  float tv[C];
#pragma unroll
  for (int c = 0; c < C; ++c) tv[c] = tid * C + c < n ? sq[tid * C + c] : 0.0f;
  const float ss = inorder_sum_onepass<RMS_NT, C>(tv, sq, n, fs);
  const float scale = 1.0f / sqrtf(ss / (float)n + eps);
#pragma unroll
  for (int b = 0; b < BPT; ++b) {
    const int blk = tid + b * RMS_NT;
    if (blk < nb) {
#pragma unroll
      for (int u = 0; u < 8; ++u) wv[b][u] = reinterpret_cast<const float4*>(wl + blk * 32)[u];
      float y[32];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        y[u * 4 + 0] = (xv[b][u].x * scale) * wv[b][u].x;
        y[u * 4 + 1] = (xv[b][u].y * scale) * wv[b][u].y;
        y[u * 4 + 2] = (xv[b][u].z * scale) * wv[b][u].z;
        y[u * 4 + 3] = (xv[b][u].w * scale) * wv[b][u].w;
      }
      if (y_out) {
#pragma unroll
        for (int u = 0; u < 8; ++u)
          reinterpret_cast<float4*>(y_out + blk * 32)[u] = make_float4(y[u * 4], y[u * 4 + 1], y[u * 4 + 2], y[u * 4 + 3]);
      }
      uint32_t packed[8];
      xs[blk] = quantize_block_regs(y, packed);
      uint4* qp = reinterpret_cast<uint4*>(xq + blk * 32);
      qp[0] = make_uint4(packed[0], packed[1], packed[2], packed[3]);
      qp[1] = make_uint4(packed[4], packed[5], packed[6], packed[7]);
      // Q8_K for K-quant consumers (n % 256 == 0: a 256-block is 8 consecutive lanes' blocks)
      if (kd) quantize_q8k_lanes8(y, kq + blk * 32, kbs + blk, kd + (blk >> 3));
    }
  }
}

// Chunk sizes instantiated for the 256-thread segmented sum (n <= 256 * C).
#define CM_SEG_CHUNKS(X) X(1) X(2) X(4) X(8) X(12) X(16) X(20) X(24) X(32) X(48) X(64)
constexpr int SEG_MAX_N = 256 * 64;
__host__ __device__ constexpr int seg_chunk(int n) {
  return n <= 256 ? 1 : n <= 512 ? 2 : n <= 1024 ? 4 : n <= 2048 ? 8 : n <= 3072 ? 12 : n <= 4096 ? 16
       : n <= 5120 ? 20 : n <= 6144 ? 24 : n <= 8192 ? 32 : n <= 12288 ? 48 : 64;
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

// SwiGLU (tensor/mod.rs:1943-1967) + Q8_0 quantization (skipped with xq null).  gu = [gate(n) | up(n)].
// kd (optional, n % 256 == 0): also the Q8_K quantization of the activation, one block per
// workgroup.  gridDim.y rows (prefill chunks): row y at gu + y * 2n, outputs likewise.
__global__ __launch_bounds__(256) void k_silu_mul_quant(const float* __restrict__ gu, int n, int8_t* __restrict__ xq,
                                                        float* __restrict__ xs, float* __restrict__ act_out,
                                                        Prefetch pf, float* __restrict__ kd,
                                                        int8_t* __restrict__ kq, int32_t* __restrict__ kbs) {
  const int nwork = (n + 255) / 256;
  if ((int)blockIdx.x >= nwork) {  // spare workgroups: read ahead the down projection
    __shared__ float sink[1];
    prefetch_lines(pf, blockIdx.x - nwork, gridDim.x - nwork, sink);
    return;
  }
  {  // row blockIdx.y of a [rows][2n] batch (prefill); row 0 in the decode step
    const size_t row = blockIdx.y;
    gu += row * 2 * n;
    xq += row * n;
    xs += row * (n >> 5);
    if (act_out) act_out += row * n;
    if (kd) {
      kd += row * (n >> 8);
      kq += row * n;
      kbs += row * (n >> 5);
    }
  }
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;  // uniform per 32-lane group
  const float a = silu_mul1(gu[i], gu[n + i]);
  if (act_out) act_out[i] = a;
  if (xq) {  // (null: only the Q8_K activation is read next)
    int8_t q;
    const float d = quantize_lane32(a, &q);
    xq[i] = q;
    if ((i & 31) == 0) xs[i >> 5] = d;
  }
  if (kd) quantize_q8k_wg256(a, kq + (size_t)blockIdx.x * 256, kbs + (size_t)blockIdx.x * 8, kd + blockIdx.x);
}

// Position guard of the decode kernels that read their position from device memory: a
// position outside the KV cache (pos >= kvs) makes the kernel touch no cache entry and write
// no output; it sets this word to 1 instead.  The kernel-level entry points clear and read it
// (the engine validates every position on the host before it is written to device memory).
__device__ uint32_t g_kv_pos_error;
__device__ __forceinline__ bool kv_pos_bad(int pos, int kvs) {
  if ((unsigned)pos < (unsigned)kvs) return false;
  if (threadIdx.x == 0) g_kv_pos_error = 1u;
  return true;
}

// ---------------------------------------------------------------------------
// Per-head QK RMSNorm (optional) + RoPE + f16 KV store for the token at *d_pos (or pos0
// when d_pos is null).  The decode step fuses this into the attention kernel; prefill runs
// it over a chunk of tokens, token blockIdx.y at position pos + blockIdx.y with its RoPE
// row at cos/sin + blockIdx.y * rope_stride.  One workgroup per head:
// blocks [0, n_heads) are Q heads, [n_heads, n_heads + n_kv) K heads (which also store the
// head's V entries).  Cache layout: kv_k_index / kv_v_index.  RoPE: rope.rs:489-524; f16
// store: kv_cache.rs:573-600.
__global__ __launch_bounds__(64) void k_rope_kv(const float* __restrict__ qkv, int n_heads, int n_kv, int hd,
                                                int rope_dim, int split_half, const float* __restrict__ cosv,
                                                const float* __restrict__ sinv, const float* __restrict__ q_norm,
                                                const float* __restrict__ k_norm, float eps, float* __restrict__ qrot,
                                                uint16_t* __restrict__ kc, uint16_t* __restrict__ vc, int layer,
                                                int kvs, const uint32_t* __restrict__ d_pos, int pos0,
                                                int rope_stride) {
  __shared__ __align__(16) float buf[512];
  __shared__ __align__(16) float sq[512];
  __shared__ float s_scale;
  const int h = blockIdx.x;
  const bool isq = h < n_heads;
  {  // token blockIdx.y of a prefill chunk: its QKV row, q row, RoPE row and position
    const size_t t = blockIdx.y;
    qkv += t * (size_t)(n_heads + 2 * n_kv) * hd;
    qrot += t * (size_t)n_heads * hd;
    cosv += t * (size_t)rope_stride;
    sinv += t * (size_t)rope_stride;
  }
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
    const int pos = (d_pos ? (int)*d_pos : pos0) + (int)blockIdx.y;
    if (kv_pos_bad(pos, kvs)) return;
    const size_t hbase = kv_head_base(layer, n_kv, kvh, hd, kvs);
    const float* vsrc = qkv + (size_t)(n_heads + n_kv) * hd + (size_t)kvh * hd;
    for (int d = threadIdx.x; d < hd; d += blockDim.x) {
      kc[hbase + kv_k_index(kvs, pos, d)] = f32_to_f16_bits(buf[d]);
      vc[hbase + kv_v_index(hd, pos, d)] = f32_to_f16_bits(vsrc[d]);
    }
  }
}

// ---------------------------------------------------------------------------
// Phase timestamps of the decode attention, compiled only into the measurement build
// (-DCM_STAMPS, libcamelid_hip_stamps.so): thread 0 of head h's workgroup in layer l records
// the 100 MHz real-time counter at each phase boundary into g_att_stamps[l][h][i]
// (camelid_hip_phase_stamps reads them).  Phases: 0 start, 1 q/k/v built and K/V stored,
// 2 scores and their maximum, 3 exponentials, 4 denominator, 5 output sums, 6 end; 7 the first
// row wave's K-row loads issued, 8 its scores done (before the maximum's barrier).
constexpr int ATT_NSTAMP = 9;
constexpr int ATT_STAMP_LAYERS = 64, ATT_STAMP_HEADS = 64;
#ifdef CM_STAMPS
__device__ uint64_t g_att_stamps[ATT_STAMP_LAYERS * ATT_STAMP_HEADS * ATT_NSTAMP];
#endif
// The split attention's workgroups (measurement build): kind 0 k_att_scores (workgroup index
// head * slices + slice), 1 k_att_out (head * dim groups + group); per workgroup < 1024 of the
// last layer: k_att_scores 0 start, 1 q built, 2 scores done, 3 end; k_att_out 0 start,
// 1 scores loaded and maximum, 2 exponentials, 3 denominator, 4 output sums, 5 end, and the
// output chain's time summed over its product blocks: 6 in its adds, 7 at the block barriers.
constexpr int SPLIT_NSTAMP = 8, SPLIT_STAMP_WGS = 1024;
#ifdef CM_STAMPS
__device__ uint64_t g_split_stamps[2 * SPLIT_STAMP_WGS * SPLIT_NSTAMP];
#define CM_SPLIT_STAMP(kind, wg, i)                                                                        \
  if (threadIdx.x == 0 && (wg) < SPLIT_STAMP_WGS)                                                         \
    g_split_stamps[((kind) * SPLIT_STAMP_WGS + (wg)) * SPLIT_NSTAMP + (i)] = __builtin_amdgcn_s_memrealtime();
#else
#define CM_SPLIT_STAMP(kind, wg, i)
#endif
#ifdef CM_STAMPS
#define CM_ATT_STAMP_T(i, t)                                                                            \
  if (tid == (t) && layer < ATT_STAMP_LAYERS && h < ATT_STAMP_HEADS)                                    \
    g_att_stamps[((size_t)layer * ATT_STAMP_HEADS + h) * ATT_NSTAMP + (i)] = __builtin_amdgcn_s_memrealtime();
#else
#define CM_ATT_STAMP_T(i, t)
#endif
#define CM_ATT_STAMP(i) CM_ATT_STAMP_T(i, 0)

// ---------------------------------------------------------------------------
// Decode attention, faithful (inference.rs:23945-24025), one workgroup per query head.
//   score_p = dot_seq(q, k_p) * scale         one lane per position, d in order
//   m = max_p score_p                          exact
//   e_p = expf(score_p - m); sum = fold_p e_p  serial fold by one lane
//   out_d = fold_p (e_p * (1/sum)) * v_pd      one lane per d, p in order
// KV cache layout: kv_k_index / kv_v_index (16-byte granules; a wave's loads are contiguous
// both for the score lanes, one position each, and for the output lanes, one d each).
// V for the output sum goes through an LDS ring (ring_slots chunks of 32 KB, filled by
// staging waves with direct global->LDS loads, the first ring_slots-1 chunks issued before
// the softmax); the output lanes read granules from LDS, two VALU operations per position.
// FUSED (the engine's path): the kernel first builds this token's q (and the kv head's k
// and v) from the fused QKV projection: optional per-head QK RMSNorm (tensor/mod.rs:2112),
// RoPE (rope.rs:489-524) with the tables at cos_base + pos*rope_stride, f16 rounding of k
// and v (kv_cache.rs:573-600).  The first q head of each GQA group stores the new K/V
// entries; every head of the group uses its own LDS copy of them for position pos.
// Not FUSED (test entry point): q is taken from qsrc and K/V entirely from the cache.
// The head's output is quantized to Q8_0 (HD % 32 == 0: blocks never straddle heads).
// kvs (the position stride) % 8 == 0.  Dynamic LDS = ring_slots * 32 KB + align4(kvs) * 4 bytes,
// ring_slots >= 2.
// Threads per workgroup: 1024 (16 waves) up to head_dim 128; 512 for head_dim 256, whose
// 512-byte K rows need twice the registers.
__host__ __device__ constexpr int att_nt(int hd) { return hd <= 128 ? 1024 : 512; }

// V staging ring: chunks of 32 KB (2048 16-byte granules), 32 wave-loads of 1 KB each.
constexpr int ATT_RING_GRANULES = 2048;
constexpr int ATT_RING_LOADS = 32;
// The split output workgroups' V ring: chunks of 16 KB (1024 granules, 16 wave-loads), three
// of them, so that 256-position product blocks (one workgroup barrier per block) fit beside
// the scores at 8K positions, where 32 KB chunks left room for 128-position blocks only.
constexpr int AO_RING_GRANULES = 1024;
constexpr int AO_RING_LOADS = 16;

// Waits until at most n of this wave's vector memory operations are outstanding (gfx9
// s_waitcnt encoding: vmcnt in bits 3:0 and 15:14; expcnt and lgkmcnt left at their maxima).
__device__ __forceinline__ void wait_vmcnt(int n) {
#define CM_VMW(N)                                                                          \
  case N:                                                                                  \
    __builtin_amdgcn_s_waitcnt(((N) & 15) | (((N) >> 4) << 14) | (7 << 4) | (15 << 8)); \
    break;
  switch (n) {
    CM_VMW(0) CM_VMW(1) CM_VMW(2) CM_VMW(3) CM_VMW(4) CM_VMW(5) CM_VMW(6) CM_VMW(7)
    CM_VMW(8) CM_VMW(9) CM_VMW(10) CM_VMW(11) CM_VMW(12) CM_VMW(13) CM_VMW(14) CM_VMW(15)
    CM_VMW(16) CM_VMW(17) CM_VMW(18) CM_VMW(19) CM_VMW(20) CM_VMW(21) CM_VMW(22) CM_VMW(23)
    CM_VMW(24)
    default:
      __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8));  // vmcnt(0)
  }
#undef CM_VMW
}

// Segmented softmax denominator: positions per thread (0: fold serially instead) and the
// prefix array's bytes, for P positions over NT threads.
constexpr int ATT_SEG_MIN = 2048;
template <int NT>
__host__ __device__ constexpr int att_seg_chunk(int P) {
  return P <= ATT_SEG_MIN ? 0 : P <= NT * 4 ? 4 : P <= NT * 8 ? 8 : P <= NT * 12 ? 12 : P <= NT * 16 ? 16 : 0;
}
template <int NT>
__host__ __device__ constexpr size_t att_seg_bytes(int P) {
  return ((size_t)NT * att_seg_chunk<NT>(P) + 4) * 4;
}
template <int NT>
__device__ __forceinline__ float att_seg_sum(const float* v, uint32_t* ps, int P) {
  switch (att_seg_chunk<NT>(P)) {
    case 4:
      return inorder_sum_nonneg<NT, 4, 1>(v, ps, P, 128);
    case 8:
      return inorder_sum_nonneg<NT, 8, 1>(v, ps, P, 128);
    case 12:
      return inorder_sum_nonneg<NT, 12, 1>(v, ps, P, 128);
    default:
      return inorder_sum_nonneg<NT, 16, 1>(v, ps, P, 128);
  }
}

// Softmax denominator by the one-pass exact in-order sum for ATT_FOLD_MAX <= P <= NT *
// ATT_ONEPASS_C positions (C = P / NT rounded up to the next of 1, 2, 3, 4, 6, 8, 9, 12, 16
// positions per thread, 16384 at 1024 threads: the classification pass costs C steps per
// thread, so a context just past a power-of-two multiple of NT does not pay for twice its
// terms); below, a serial fold
// by one lane is faster (measured: 2.0 us fold vs 2.9 us one-pass at P = 560).
constexpr int ATT_ONEPASS_C = 16;
constexpr int ATT_FOLD_MAX = 1024;
template <int NT>
__device__ __forceinline__ float att_onepass_sum(const float* v, int P, FsLds<NT>& fs) {
  const int tid = threadIdx.x;
#define CM_AOP(C)                                                               \
  {                                                                             \
    float t[C];                                                                 \
    _Pragma("unroll") for (int c = 0; c < C; ++c) t[c] = tid * C + c < P ? v[tid * C + c] : 0.0f; \
    return inorder_sum_onepass<NT, C>(t, v, P, fs);                             \
  }
  if (P <= NT) CM_AOP(1)
  if (P <= NT * 2) CM_AOP(2)
  if (P <= NT * 3) CM_AOP(3)
  if (P <= NT * 4) CM_AOP(4)
  if (P <= NT * 6) CM_AOP(6)
  if (P <= NT * 8) CM_AOP(8)
  if (P <= NT * 9) CM_AOP(9)
  if (P <= NT * 12) CM_AOP(12)
  CM_AOP(16)
#undef CM_AOP
}


// ---------------------------------------------------------------------------
// The output projection inside the decode attention launch (att . W_o^T + residual, the
// Q8_0 GEMV k_gemv_k computes after the attention: q8_gemv with the residual add,
// cuda_resident.rs:230; CPU inference.rs:19871-19905).  The attention occupies one CU per
// workgroup for its whole duration while the HBM stream idles, so the launch carries
// ceil(rows / 16) more workgroups that load their W_o rows (one per wave) at once and then
// read the Q8_0 activation as the attention workgroups publish it, and run k_gemv_k's dots
// and block-ordered folds: the same terms in the same order, so the same bits.
// Handoff: the attention workgroups store their quants (four to a word) and block scales as
// 8-byte words whose high half is a tag, ao_tag(pos, layer), with agent-scope (cross-XCD
// coherent) stores; a projection workgroup's thread 0 first watches one scale word, then every
// thread reads its words with agent-scope loads until each carries the tag.  One tag per
// (position, layer): the engine clears the words before a call's decode steps, and within a
// call every (position, layer) is computed once.  The wait is bounded: past about 2^18 polls
// per word the workgroup sets g_handoff_error and computes from whatever it read.
constexpr int AO_ROWS = 16;  // rows per projection workgroup (one per wave)
// rows per wave of the projection workgroups in the split output launch (k_att_out), which
// take the CUs its 32-dim output workgroups leave free: 2, so that a [4096 x 4096] W_o fits
// 128 workgroups beside the 128 output workgroups of 32 heads of 128
constexpr int AO_SPLIT_RPW = 2;
// (measurement build: thread 0 of the first and the last projection workgroup of layer l
// records 0 start, 1 watched word tagged, 2 activation staged, 3 end into g_ao_stamps[l][0|1])
constexpr int AO_NSTAMP = 4;
#ifdef CM_STAMPS
__device__ uint64_t g_ao_stamps[64 * 2 * AO_NSTAMP];
#define CM_AO_STAMP(i)                                                                                  \
  if (threadIdx.x == 0 && op.layer < 64 && (wg == 0 || wg == (int)gridDim.x - 1 - (int)(blockIdx.x - wg))) \
    g_ao_stamps[((size_t)op.layer * 2 + (wg != 0)) * AO_NSTAMP + (i)] = __builtin_amdgcn_s_memrealtime();
#else
#define CM_AO_STAMP(i)
#endif
struct OProj {
  const int8_t* q;      // W_o quants [rows][K] (null: no Q8_0 projection in this launch)
  const uint16_t* d;    // W_o f16 block scales [rows][K / 32]
  int rows, K;          // K = n_heads * head_dim
  float* y;             // y[r] = resid[r] + (W_o att)[r]
  const float* resid;
  uint64_t* xq_t;       // [K / 4] tagged quant words
  uint64_t* xs_t;       // [K / 32] tagged block scales
  int layer;
  // a Q4_K W_o instead (k_att_fused only; q null): its nibble and header planes, and the
  // attention output as [K] tagged f32 words, quantized to Q8_K by the projection workgroups
  const uint8_t* k4nib = nullptr;
  const uint8_t* k4hdr = nullptr;
  uint64_t* xf_t = nullptr;
};
__host__ __device__ constexpr uint32_t ao_tag(uint32_t pos, uint32_t layer) { return ((pos + 1u) << 8) | layer; }
__host__ __device__ constexpr size_t ao_lds_bytes(int K, int rows = AO_ROWS) {
  return (size_t)K + (size_t)(K / 32) * 4 + (size_t)rows * gemv_term_stride(K / 32) * 4;
}

__device__ __forceinline__ uint64_t ao_wait_word(const uint64_t* p, uint32_t tag) {
  uint64_t v = ld_agent64(p);
  uint32_t polls = 0;
  while ((uint32_t)(v >> 32) != tag) {
    __builtin_amdgcn_s_sleep(1);
    if (++polls == (1u << 18)) {
      g_handoff_error = 1u;
      break;
    }
    v = ld_agent64(p);
  }
  return v;
}

// RPW rows per wave (AO_ROWS * RPW per workgroup).
template <int K, int NT, int RPW = 1>
__device__ __forceinline__ void att_oproj_rows(const OProj& op, int wg, uint32_t tag, unsigned char* smem) {
  constexpr int NB = K / 32, CPR = K / 16, IT = (CPR + 63) / 64, STRIDE = gemv_term_stride(NB);
  constexpr int R = AO_ROWS * RPW;
  static_assert(NT / 64 == AO_ROWS && K % 128 == 0, "sixteen waves, whole 128-value groups");
  uint32_t* xl = reinterpret_cast<uint32_t*>(smem);
  float* xsl = reinterpret_cast<float*>(smem + K);
  float* t = xsl + NB;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int row0 = wg * R;
  CM_AO_STAMP(0)
  // this wave's rows: every weight and scale load first (rows past the end clamped; their
  // results are never stored)
  int4 wv[RPW][IT];
  uint16_t dv[RPW][IT];
#pragma unroll
  for (int k = 0; k < RPW; ++k) {
    const int row = min(row0 + wave * RPW + k, op.rows - 1);
    const int4* w4 = reinterpret_cast<const int4*>(op.q + (size_t)row * K);
    const uint16_t* dp = op.d + (size_t)row * NB;
#pragma unroll
    for (int i = 0; i < IT; ++i) {
      const int c = min(lane + 64 * i, CPR - 1);
      wv[k][i] = ld_stream(w4 + c);
      dv[k][i] = ld_stream(dp + (c >> 1));
    }
  }
  // one watcher until a scale word carries the tag (the heads finish together), then every
  // word by its own thread
  if (tid == 0) (void)ao_wait_word(op.xs_t + (blockIdx.x % NB), tag);
  CM_AO_STAMP(1)
  __syncthreads();
  for (int c = tid; c < K / 4 + NB; c += NT) {
    if (c < K / 4)
      xl[c] = (uint32_t)ao_wait_word(op.xq_t + c, tag);
    else
      xsl[c - K / 4] = __uint_as_float((uint32_t)ao_wait_word(op.xs_t + (c - K / 4), tag));
  }
  __syncthreads();
  CM_AO_STAMP(2)
#pragma unroll
  for (int k = 0; k < RPW; ++k) {
    float* tr = t + (wave * RPW + k) * STRIDE;
#pragma unroll
    for (int i = 0; i < IT; ++i) {
      __builtin_amdgcn_sched_barrier(0);
      const int c = lane + 64 * i;
      const int cc = min(c, CPR - 1);
      int s = dot4x4(wv[k][i], reinterpret_cast<const int4*>(xl)[cc], 0);
      s += dpp_xor1(s);
      if ((lane & 1) == 0 && c < CPR) tr[c >> 1] = ((float)s * half_bits_to_float(dv[k][i])) * xsl[c >> 1];
    }
  }
  __syncthreads();
  if (tid < R && row0 + tid < op.rows) {
    const float acc = fold_lds_n<NB>(t + tid * STRIDE);
    op.y[row0 + tid] = op.resid[row0 + tid] + acc;
  }
  CM_AO_STAMP(3)
}

// The attention's widths n_heads * head_dim with an instantiated projection body.
__host__ __device__ constexpr bool ao_width_ok(int K) { return K == 2048 || K == 3072 || K == 4096; }

template <int NT, int RPW = 1>
__device__ __forceinline__ void att_oproj(const OProj& op, int wg, uint32_t tag, unsigned char* smem) {
  switch (op.K) {
    case 2048:
      att_oproj_rows<2048, NT, RPW>(op, wg, tag, smem);
      break;
    case 3072:
      att_oproj_rows<3072, NT, RPW>(op, wg, tag, smem);
      break;
    case 4096:
      att_oproj_rows<4096, NT, RPW>(op, wg, tag, smem);
      break;
    default:
      break;
  }
}

// DG workgroups per query head (the grid is n_heads * DG): each computes the head's scores,
// softmax and denominator (the same bits in every one of them) and the output sums of its
// HD / DG dims, so that a CU stages 1/DG of the head's V rows; one of them stores the K/V row.
// With op.q set, ceil(op.rows / 16) more workgroups compute the output projection (att_oproj).
template <int HD, bool FUSED, int DG = 1>
__global__ __launch_bounds__(att_nt(HD)) void k_attention(
    const float* __restrict__ qsrc, int n_heads, int n_kv, int rope_dim, int split_half,
    const float* __restrict__ cos_base, const float* __restrict__ sin_base, int rope_stride,
    const float* __restrict__ q_norm, const float* __restrict__ k_norm, float eps, uint16_t* __restrict__ kc,
    uint16_t* __restrict__ vc, int layer, int kvs, const uint32_t* __restrict__ d_pos, float scale,
    float* __restrict__ att_out, int8_t* __restrict__ xq, float* __restrict__ xs, int ring_slots, Prefetch pf,
    OProj op) {
  constexpr int ATT_NT = att_nt(HD);
  static_assert(HD % 64 == 0 && HD <= 256, "head_dim must be 64, 128 or 256");
  constexpr int R8 = HD / 8;  // 16-byte granules per K row
  constexpr int NW = ATT_NT / 64;
  constexpr int CW = HD / 64;                        // output waves: one lane per dim
  constexpr int NH = (NW - CW) >= 8 ? 8 : 4;         // V-staging waves (divides the 32 loads)
  constexpr int LH = ATT_RING_LOADS / NH;            // 1 KB wave loads per staging wave per chunk
  constexpr int OD = HD / DG;                        // output dims of this workgroup: [d0, d0 + OD)
  static_assert(OD % 32 == 0 && OD <= 64 * CW, "whole Q8_0 blocks of output per workgroup");
  constexpr int CG = ATT_RING_GRANULES / OD;         // 8-position groups per ring chunk
  extern __shared__ __align__(16) float4 dyn[];
  float4* ring = dyn;  // ring_slots chunks of ATT_RING_GRANULES V granules
  float* sc = reinterpret_cast<float*>(dyn + (size_t)ring_slots * ATT_RING_GRANULES);
  if ((int)blockIdx.x >= n_heads * DG) {
    if constexpr (ATT_NT == AO_ROWS * 64) {
      if (op.q) {  // the output projection's workgroups
        const int pos = (int)*d_pos;
        if (kv_pos_bad(pos, kvs)) return;
        att_oproj<ATT_NT>(op, (int)blockIdx.x - n_heads * DG, ao_tag((uint32_t)pos, (uint32_t)op.layer),
                          reinterpret_cast<unsigned char*>(dyn));
        return;
      }
    }
    // spare workgroups: read ahead the output projection
    prefetch_lines(pf, blockIdx.x - n_heads * DG, gridDim.x - n_heads * DG, sc);
    return;
  }
  __shared__ __align__(16) float qs[HD];
  __shared__ __align__(16) float kn[HD];  // this position's k (f16-rounded)
  __shared__ __align__(16) float vn[HD];  // this position's v (f16-rounded)
  __shared__ __align__(16) float sq[2 * HD];
  __shared__ float red[ATT_NT / 64];
  __shared__ float s_qscale, s_kscale, s_inv;
  __shared__ uint64_t etab[32];  // the expf table, read from LDS by the exponentials
  __shared__ FsLds<ATT_NT> fs;
  __shared__ uint32_t team_ctr, team_bad;  // the head team's LDS barrier
  const int tid = threadIdx.x;
  const int rep = n_heads / n_kv;
  // workgroup (h, dg): the head's DG workgroups and those of the other query heads of its KV
  // head on one XCD
  const int hm = xcd_member(blockIdx.x, n_kv, rep * DG);
  const int h = hm / DG, dg = hm % DG, d0 = dg * OD;
  const int kvh = h / rep;
  const size_t hbase = kv_head_base(layer, n_kv, kvh, HD, kvs);
  const uint4* kg = reinterpret_cast<const uint4*>(kc + hbase);  // K granule (u, p): u * kvs + p
  const uint4* vg = reinterpret_cast<const uint4*>(vc + hbase);  // V granule (g, d): g * HD + d
  const int pos = (int)*d_pos;
  if (kv_pos_bad(pos, kvs)) return;  // (uniform, before any barrier)
  CM_ATT_STAMP(0)
  const int P = pos + 1;
  const int ncache = pos;
  // Loads in the order they are needed (a wave's loads complete in order): this token's q, k
  // and v and the expf table first.
  float qv = 0.0f, kv = 0.0f, vv = 0.0f;
  uint64_t et = 0;
  if (tid < HD) {
    if (FUSED) {
      qv = qsrc[(size_t)h * HD + tid];
      kv = qsrc[(size_t)n_heads * HD + (size_t)kvh * HD + tid];
      vv = qsrc[(size_t)(n_heads + n_kv) * HD + (size_t)kvh * HD + tid];
    } else {
      qv = qsrc[(size_t)h * HD + tid];
      kv = half_bits_to_float(kc[hbase + kv_k_index(kvs, pos, tid)]);
      vv = half_bits_to_float(vc[hbase + kv_v_index(HD, pos, tid)]);
    }
  }
  if (tid < 32) et = kExp2Tab[tid];
  // The output lanes also load now the (up to 7) V values of the positions past the last
  // full 8-position granule, which their output chain adds from registers at the end, and
  // the RoPE table entries and QK-norm weights of this head.
  uint16_t vtail[7];
  const int half = rope_dim >> 1;
  float rc = 0.0f, rs = 0.0f, qnw = 0.0f, knw = 0.0f;
  if (tid < HD) {
    const int tail0 = (pos >> 3) << 3;  // first position past the full granules of [0, pos)
    if (tid < OD) {
#pragma unroll
      for (int u = 0; u < 7; ++u)
        vtail[u] = tail0 + u < pos ? vc[hbase + kv_v_index(HD, tail0 + u, d0 + tid)] : (uint16_t)0;
    }
    if (FUSED) {
      if (tid < half) {
        rc = cos_base[(size_t)pos * rope_stride + tid];
        rs = sin_base[(size_t)pos * rope_stride + tid];
      }
      if (q_norm) {
        qnw = q_norm[tid];
        knw = k_norm[tid];
      }
    }
  }
  if (tid == 0) {
    team_ctr = 0u;
    team_bad = 0u;
  }
  // Waves 0..CW-1 (the head team) build q and this position's k and v; the other waves hold
  // the cache rows of the first score pass (score lane lt = tid - HD, positions lt, lt + NT,
  // ...; the team's lanes take lt = NT - HD + tid).  This barrier puts the team's loads at the
  // head of the CU's memory queue; then the row waves issue their K rows, which stream while
  // the team works (it synchronises through an LDS counter, so a row wave stalled issuing
  // its loads holds up nobody) and are in registers when the score phase starts.
  __syncthreads();
  const int lt = tid >= HD ? tid - HD : tid + ATT_NT - HD;
  uint4 row0[R8];
  if (tid >= HD && lt < ncache) {
#pragma unroll
    for (int u = 0; u < R8; ++u) row0[u] = kg[(size_t)u * kvs + lt];
    if (lt == 0) {
      CM_ATT_STAMP_T(7, HD)
    }
  }
  // V staging: the cache positions' V granules (full 8-position groups) of this workgroup's
  // dims are copied into an LDS ring of ring_slots chunks by NH staging waves with direct
  // global->LDS loads; the output lanes read them from LDS.  A chunk holds CG groups of OD
  // granules (contiguous in the cache layout when DG = 1, else OD-granule runs).  The first
  // chunks go out after the exponentials (longer contexts with the segmented denominator use
  // the ring for its prefix arrays first).
  const int ng = ncache >> 3;  // full groups of 8 cache positions
  const int nchunks = (ng + CG - 1) / CG;
  const int R = ring_slots;
  const int hw = (tid >> 6) - CW;
  const bool stager = hw >= 0 && hw < NH;
  const size_t last_group = (size_t)max(ng, 1) - 1;
  auto stage = [&](int c) {  // chunk c into slot c % R
    float4* slot = ring + (size_t)(c % R) * ATT_RING_GRANULES;
#pragma unroll
    for (int j = 0; j < LH; ++j) {
      const int i = hw + NH * j;  // 1 KB piece of the chunk
      const int q = i * 64 + (tid & 63);  // granule q of the chunk: group q / OD, dim d0 + q % OD
      const size_t gsrc = min((size_t)c * CG + (size_t)(q / OD), last_group) * HD + d0 + q % OD;
      __builtin_amdgcn_global_load_lds(reinterpret_cast<const void*>(vg + gsrc),
                                       (__attribute__((address_space(3))) void*)(slot + i * 64), 16, 0, 0);
    }
  };
  // the denominator: a serial fold below ATT_FOLD_MAX positions, the one-pass exact sum up
  // to ATT_NT * ATT_ONEPASS_C, the segmented passes beyond (which use the ring first)
  const bool onepass = P >= ATT_FOLD_MAX && P <= ATT_NT * ATT_ONEPASS_C;
  const bool early = P > 1 && P <= ATT_NT * ATT_ONEPASS_C;
  if (tid < HD) {  // (the head team: whole waves)
    TeamBar tb{&team_ctr, &team_bad, (uint32_t)CW, 0u};
    if (tid < 32) etab[tid] = et;
    qs[tid] = qv;
    kn[tid] = kv;
    vn[tid] = vv;
    if (FUSED) {
      if (q_norm) {  // per-head RMSNorm of q and k (two serial folds by two lanes)
        tb();
        sq[tid] = qs[tid] * qs[tid];
        sq[HD + tid] = kn[tid] * kn[tid];
        tb();
        constexpr int KT = HD >= 128 ? 64 : 32;  // the k fold's lane (another wave when there is one)
        if (tid == 0 || tid == KT) {
          const float r = 1.0f / sqrtf(fold_lds_lean(tid == 0 ? sq : sq + HD, HD) / (float)HD + eps);
          if (tid == 0) s_qscale = r;
          else s_kscale = r;
        }
        tb();
        qs[tid] = (qs[tid] * s_qscale) * qnw;
        kn[tid] = (kn[tid] * s_kscale) * knw;
      }
      tb();
      if (tid < half) {
        const int d0 = split_half ? tid : 2 * tid;
        const int d1 = split_half ? tid + half : 2 * tid + 1;
        float x0 = qs[d0], x1 = qs[d1];
        qs[d0] = (x0 * rc) - (x1 * rs);
        qs[d1] = (x0 * rs) + (x1 * rc);
        x0 = kn[d0];
        x1 = kn[d1];
        kn[d0] = (x0 * rc) - (x1 * rs);
        kn[d1] = (x0 * rs) + (x1 * rc);
      }
      tb();
      const uint16_t kb = f32_to_f16_bits(kn[tid]);
      const uint16_t vb = f32_to_f16_bits(vn[tid]);
      kn[tid] = half_bits_to_float(kb);
      vn[tid] = half_bits_to_float(vb);
      if ((h % rep) == 0 && dg == 0) {
        kc[hbase + kv_k_index(kvs, pos, tid)] = kb;
        vc[hbase + kv_v_index(HD, pos, tid)] = vb;
      }
    }
  }
  __syncthreads();
  CM_ATT_STAMP(1)

  float res = 0.0f;  // this output lane's value (tid < HD)
  if (P == 1) {
    // inference.rs:23564-23575: a single position copies the V row.
    if (tid < OD) res = vn[d0 + tid];
  } else {
    // ---- scores: cache positions 0..pos-1, one lane each
    float lmax = -INFINITY;
    auto score = [&](const uint4(&row)[R8], int p) {
      float acc = 0.0f;
      // q is read from LDS 8 values at a time (fencing the schedule keeps the whole of q from
      // being hoisted into registers next to the in-flight row): the next granule's q goes out
      // after this granule's 8 products and before its 8 dependent adds, so the read latency
      // overlaps the adds, and no add waits on its product
      const float4* q4 = reinterpret_cast<const float4*>(qs);
      float4 qa = q4[0], qb = q4[1];
#pragma unroll
      for (int u = 0; u < R8; ++u) {
        __builtin_amdgcn_sched_barrier(0);
        const float p0 = mul_f16_lo(qa.x, row[u].x), p1 = mul_f16_hi(qa.y, row[u].x);
        const float p2 = mul_f16_lo(qa.z, row[u].y), p3 = mul_f16_hi(qa.w, row[u].y);
        const float p4 = mul_f16_lo(qb.x, row[u].z), p5 = mul_f16_hi(qb.y, row[u].z);
        const float p6 = mul_f16_lo(qb.z, row[u].w), p7 = mul_f16_hi(qb.w, row[u].w);
        __builtin_amdgcn_sched_barrier(0);
        if (u + 1 < R8) {
          qa = q4[2 * u + 2];
          qb = q4[2 * u + 3];
        }
        __builtin_amdgcn_sched_barrier(0);
        acc += p0;
        acc += p1;
        acc += p2;
        acc += p3;
        acc += p4;
        acc += p5;
        acc += p6;
        acc += p7;
        asm volatile("" : "+v"(acc));  // this granule's adds stay ahead of the next reads
      }
      const float sv = acc * scale;
      sc[p] = sv;
      lmax = fmaxf(lmax, sv);
    };
    if (lt < ncache) {
      if (tid >= HD) {
        score(row0, lt);
      } else {  // (the team's lanes: positions NT - HD + tid, reached from NT - HD + 1 positions)
        uint4 row[R8];
#pragma unroll
        for (int u = 0; u < R8; ++u) row[u] = kg[(size_t)u * kvs + lt];
        score(row, lt);
      }
    }
    if (lt == 0) {
      CM_ATT_STAMP_T(8, HD)
    }
    for (int p = lt + ATT_NT; p < ncache; p += ATT_NT) {
      uint4 row[R8];
#pragma unroll
      for (int u = 0; u < R8; ++u) row[u] = kg[(size_t)u * kvs + p];
      score(row, p);
    }
    // this token's own key (from LDS) by the team's last lane, which has no cache row below
    // NT positions (its chain then runs beside the row waves' instead of after one of them);
    // 8 products ahead of their 8 dependent adds
    if (tid == HD - 1) {
      float acc = 0.0f;
      const float4* q4 = reinterpret_cast<const float4*>(qs);
      const float4* k4 = reinterpret_cast<const float4*>(kn);
#pragma unroll
      for (int u = 0; u < HD / 8; ++u) {
        const float4 qa = q4[2 * u], qb = q4[2 * u + 1], ka = k4[2 * u], kb = k4[2 * u + 1];
        const float p0 = qa.x * ka.x, p1 = qa.y * ka.y, p2 = qa.z * ka.z, p3 = qa.w * ka.w;
        const float p4 = qb.x * kb.x, p5 = qb.y * kb.y, p6 = qb.z * kb.z, p7 = qb.w * kb.w;
        acc += p0;
        acc += p1;
        acc += p2;
        acc += p3;
        acc += p4;
        acc += p5;
        acc += p6;
        acc += p7;
      }
      const float sv = acc * scale;
      sc[pos] = sv;
      lmax = fmaxf(lmax, sv);
    }
    const float mx = block_max(lmax, red);
    CM_ATT_STAMP(2)
    for (int p = tid; p < P; p += ATT_NT) sc[p] = glibc_expf_t(sc[p] - mx, etab);
    // The denominator: the one-pass exact in-order sum; beyond its limit the exact segmented
    // sum (one binade per pass) with its prefix array in the V ring, staged only afterwards,
    // or (when even that does not fit) a serial fold by one lane.
    const bool seg = !early && att_seg_chunk<ATT_NT>(P) > 0 &&
                     att_seg_bytes<ATT_NT>(P) <= (size_t)R * ATT_RING_GRANULES * 16;
    __syncthreads();
    CM_ATT_STAMP(3)
    // the first V chunks go out now: the staging waves' issue (a wave stalls while the CU's
    // memory queue is full) overlaps the denominator's serial fold by one lane, and no
    // barrier waits on it before that
    if (stager && !seg) {
      for (int c = 0; c < min(R - 1, nchunks); ++c) stage(c);
    }
    float inv;
    if (onepass) {
      inv = 1.0f / att_onepass_sum<ATT_NT>(sc, P, fs);
    } else {
      if (seg) {
        const float ssum = att_seg_sum<ATT_NT>(sc, reinterpret_cast<uint32_t*>(ring), P);
        if (tid == 0) s_inv = 1.0f / ssum;
        if (stager) {
          for (int c = 0; c < min(R - 1, nchunks); ++c) stage(c);
        }
      } else if (tid == 0) {
        s_inv = 1.0f / fold_lds(sc, P);
      }
      __syncthreads();
      inv = s_inv;
    }
    CM_ATT_STAMP(4)
    for (int p = tid; p < P; p += ATT_NT) sc[p] = sc[p] * inv;
    // ---- out_d = fold_p prob_p * v_pd: lane d walks the ring chunk by chunk (granules of
    // 8 positions; each product is one mixed-precision FMA on the f16 value).
    float acc = 0.0f;
    for (int c = 0; c < nchunks; ++c) {
      if (stager) wait_vmcnt(LH * (min(c + R - 2, nchunks - 1) - c));  // chunk c has landed
      __syncthreads();  // chunk c visible; the slot of chunk c - 1 is free
      if (stager && c + R - 1 < nchunks) stage(c + R - 1);
      if (tid < OD) {
        const uint4* slot = reinterpret_cast<const uint4*>(ring + (size_t)(c % R) * ATT_RING_GRANULES) + tid;
        const float4* pr4 = reinterpret_cast<const float4*>(sc) + (size_t)c * CG * 2;
        const int gn = min(CG, ng - c * CG);
        // granule g (8 positions) with its probabilities p0 (positions 0-3), p1 (4-7): the 8
        // products, then the 8 dependent adds (no add waits on its own product)
        auto granule = [&](const uint4& g, const float4& p0, const float4& p1, float (&pr)[8]) {
          pr[0] = mul_f16_lo(p0.x, g.x);
          pr[1] = mul_f16_hi(p0.y, g.x);
          pr[2] = mul_f16_lo(p0.z, g.y);
          pr[3] = mul_f16_hi(p0.w, g.y);
          pr[4] = mul_f16_lo(p1.x, g.z);
          pr[5] = mul_f16_hi(p1.y, g.z);
          pr[6] = mul_f16_lo(p1.z, g.w);
          pr[7] = mul_f16_hi(p1.w, g.w);
        };
        // LDS reads ping-pong between two batches of 2 granules (16 positions) so that the
        // add chain never waits on LDS latency
        static_assert(CG % 4 == 0, "ring chunks hold a multiple of 4 granule groups");
        uint4 va[2], vb[2];
        float4 pa[4], pb[4];
        auto ld = [&](uint4(&v)[2], float4(&pq)[4], int j0) {
#pragma unroll
          for (int u = 0; u < 2; ++u) {
            v[u] = slot[(j0 + u) * OD];
            pq[2 * u] = pr4[2 * (j0 + u)];
            pq[2 * u + 1] = pr4[2 * (j0 + u) + 1];
          }
        };
        auto mac = [&](const uint4(&v)[2], const float4(&pq)[4]) {
          float pr[2][8];
          granule(v[0], pq[0], pq[1], pr[0]);
          granule(v[1], pq[2], pq[3], pr[1]);
          __builtin_amdgcn_sched_barrier(0);
#pragma unroll
          for (int u = 0; u < 2; ++u)
#pragma unroll
            for (int e = 0; e < 8; ++e) acc += pr[u][e];
        };
        if (gn == CG) {
          ld(va, pa, 0);
#pragma unroll
          for (int j = 0; j < CG; j += 4) {
            ld(vb, pb, j + 2);
            __builtin_amdgcn_sched_barrier(0);
            mac(va, pa);
            if (j + 4 < CG) ld(va, pa, j + 4);
            __builtin_amdgcn_sched_barrier(0);
            mac(vb, pb);
          }
        } else {
          // the last chunk: its whole batches of 4 granules as above, then one at a time
          const int g4 = gn & ~3;
          if (g4 > 0) ld(va, pa, 0);
          for (int j = 0; j < g4; j += 4) {
            ld(vb, pb, j + 2);
            __builtin_amdgcn_sched_barrier(0);
            mac(va, pa);
            if (j + 4 < g4) ld(va, pa, j + 4);
            __builtin_amdgcn_sched_barrier(0);
            mac(vb, pb);
          }
          for (int j = g4; j < gn; ++j) {
            float pr[8];
            granule(slot[j * OD], pr4[2 * j], pr4[2 * j + 1], pr);
#pragma unroll
            for (int e = 0; e < 8; ++e) acc += pr[e];
          }
        }
      }
    }
    CM_ATT_STAMP(5)
    // the normalised probabilities past the ring were published by the ring loop's first
    // barrier; with no chunks at all, by this one (uniform)
    if (nchunks == 0) __syncthreads();
    if (tid < OD) {
#pragma unroll
      for (int u = 0; u < 7; ++u)
        if (ng * 8 + u < ncache) acc += sc[ng * 8 + u] * half_bits_to_float(vtail[u]);
      acc += sc[pos] * vn[d0 + tid];
      res = acc;
    }
  }
  // (each output lane stores and quantizes its own value: no barrier; the Q8_0 block's
  // scale is formed by lane shuffles within the 32-lane group)
  const bool publish = ATT_NT == AO_ROWS * 64 && op.q != nullptr;
  if (tid < OD) {
    if (team_bad) res = __builtin_nanf("");  // (the team barrier's bound was reached: no result)
    const size_t o = (size_t)h * HD + d0 + tid;
    att_out[o] = res;
    int8_t q;
    const float dd = quantize_lane32(res, &q);
    if (publish) {
      // for the projection workgroups of this launch: four lanes' quants in one word, and the
      // block scale, each with the tag in its high half, by agent-scope stores
      const uint64_t tg = (uint64_t)ao_tag((uint32_t)pos, (uint32_t)op.layer) << 32;
      const uint32_t b = (uint32_t)(uint8_t)q;
      const uint32_t w = b | ((uint32_t)__shfl_down((int)b, 1) << 8) | ((uint32_t)__shfl_down((int)b, 2) << 16) |
                         ((uint32_t)__shfl_down((int)b, 3) << 24);
      if ((tid & 3) == 0) st_agent64(op.xq_t + (o >> 2), tg | w);
      if ((tid & 31) == 0) st_agent64(op.xs_t + (o >> 5), tg | __float_as_uint(dd));
    } else {
      xq[o] = q;
      if ((tid & 31) == 0) xs[o >> 5] = dd;
    }
  }
  CM_ATT_STAMP(6)
}

// ---------------------------------------------------------------------------
// Decode attention split over workgroups: k_attention's arithmetic, in the same order, with
// a head's K and V streamed through many CUs instead of one (one CU's loads in flight, not the
// arithmetic, bound the single-workgroup kernel: about 30 GB/s per CU).
//   k_att_scores  grid (heads, ceil(kvs / NT)): workgroup (h, s) builds q (and, for s = 0
//                 of a group's first head, stores this position's K/V, as k_attention does),
//                 then the scores of positions [s NT, (s + 1) NT) ∩ [0, pos] into g_sc[h][p]
//                 and their max into g_max[h][s]; slices past pos exit at once.  Each thread's
//                 K row is issued with the q/k/v loads, so the slice streams while q is built.
//   k_att_out     grid (heads * HD / 32 [+ read-ahead workgroups]): workgroup (h, w) reads the
//                 head's scores, softmax as k_attention (max, expf, the in-order denominator,
//                 normalise), then out_d for d in [32 w, 32 w + 32) through a V ring whose 32 KB
//                 chunks hold 512 positions of those 32 dims (its first chunks issued behind
//                 the scores loads), and quantizes them (one Q8_0 block).  Every position's V
//                 comes from the cache (k_att_scores stored pos).
// Score slice s of head h: positions [s SL, (s + 1) SL) by threads 0 .. SL - 1 of the NT
// threads.  TAG: each score goes out as soon as it is formed, as a tagged word (sc_t[h][p]:
// the value's bits, tag << 32) by an agent-scope store, for the output workgroups of the same
// launch (k_att_fused), which take the maximum themselves; else the scores and the slice
// maximum as plain floats (g_sc, g_max).
template <int HD, bool FUSED, int NT, int SL, bool TAG>
__device__ __forceinline__ void att_scores_body(
    int h, int s, int n_slices, const float* __restrict__ qsrc, int n_heads, int n_kv, int rope_dim, int split_half,
    const float* __restrict__ cos_base, const float* __restrict__ sin_base, int rope_stride,
    const float* __restrict__ q_norm, const float* __restrict__ k_norm, float eps, uint16_t* __restrict__ kc,
    uint16_t* __restrict__ vc, int layer, int kvs, const uint32_t* __restrict__ d_pos, float scale,
    float* __restrict__ g_sc, float* __restrict__ g_max, uint64_t* __restrict__ sc_t) {
  constexpr int ATT_NT = NT;
  static_assert(HD % 64 == 0 && HD <= 256 && NT >= HD && NT % 64 == 0 && SL <= NT, "head_dim must be 64, 128 or 256");
  constexpr int R8 = HD / 8;
  __shared__ __align__(16) float qs[HD];
  __shared__ __align__(16) float kn[HD];
  __shared__ __align__(16) float vn[HD];
  __shared__ __align__(16) float sq[2 * HD];
  __shared__ float red[ATT_NT / 64];
  __shared__ float s_qscale, s_kscale;
  const int tid = threadIdx.x;
  const int pos = (int)*d_pos;
  if (kv_pos_bad(pos, kvs)) return;  // (uniform, before any barrier)
  const int p0 = s * SL;
  if (p0 > pos) return;  // (uniform) a slice past the current position
  const uint64_t tg = TAG ? (uint64_t)ao_tag((uint32_t)pos, (uint32_t)layer) << 32 : 0;
  const int rep = n_heads / n_kv;
  const int kvh = h / rep;
  const size_t hbase = kv_head_base(layer, n_kv, kvh, HD, kvs);
  const uint4* kg = reinterpret_cast<const uint4*>(kc + hbase);
  const int wg = h * n_slices + s;
  (void)wg;
  CM_SPLIT_STAMP(0, wg, 0)
  if (tid < HD) {
    qs[tid] = qsrc[(size_t)h * HD + tid];
    if (FUSED) {
      kn[tid] = qsrc[(size_t)n_heads * HD + (size_t)kvh * HD + tid];
      vn[tid] = qsrc[(size_t)(n_heads + n_kv) * HD + (size_t)kvh * HD + tid];
    } else {
      kn[tid] = half_bits_to_float(kc[hbase + kv_k_index(kvs, pos, tid)]);
    }
  }
  // this thread's cache position's K row: issued now (behind q/k/v in their waves), so that
  // the slice's K streams while q is built
  const int p = tid < SL ? p0 + tid : 0x7fffffff;
  uint4 row[R8];
  if (p < pos) {
#pragma unroll
    for (int u = 0; u < R8; ++u) row[u] = kg[(size_t)u * kvs + p];
  }
  if (FUSED) {
    if (q_norm) {  // per-head RMSNorm of q and k (serial folds, as k_attention)
      __syncthreads();
      if (tid < HD) {
        sq[tid] = qs[tid] * qs[tid];
        sq[HD + tid] = kn[tid] * kn[tid];
      }
      __syncthreads();
      if (tid == 0) s_qscale = 1.0f / sqrtf(fold_lds_lean(sq, HD) / (float)HD + eps);
      if (tid == 64) s_kscale = 1.0f / sqrtf(fold_lds_lean(sq + HD, HD) / (float)HD + eps);
      __syncthreads();
      if (tid < HD) {
        qs[tid] = (qs[tid] * s_qscale) * q_norm[tid];
        kn[tid] = (kn[tid] * s_kscale) * k_norm[tid];
      }
    }
    __syncthreads();
    const float* cosv = cos_base + (size_t)pos * rope_stride;
    const float* sinv = sin_base + (size_t)pos * rope_stride;
    const int half = rope_dim >> 1;
    if (tid < half) {
      const int d0 = split_half ? tid : 2 * tid;
      const int d1 = split_half ? tid + half : 2 * tid + 1;
      const float c = cosv[tid], sn = sinv[tid];
      float x0 = qs[d0], x1 = qs[d1];
      qs[d0] = (x0 * c) - (x1 * sn);
      qs[d1] = (x0 * sn) + (x1 * c);
      x0 = kn[d0];
      x1 = kn[d1];
      kn[d0] = (x0 * c) - (x1 * sn);
      kn[d1] = (x0 * sn) + (x1 * c);
    }
    __syncthreads();
    if (tid < HD) {
      const uint16_t kb = f32_to_f16_bits(kn[tid]);
      kn[tid] = half_bits_to_float(kb);
      if ((h % rep) == 0 && s == 0) {
        kc[hbase + kv_k_index(kvs, pos, tid)] = kb;
        vc[hbase + kv_v_index(HD, pos, tid)] = f32_to_f16_bits(vn[tid]);
      }
    }
  }
  __syncthreads();
  CM_SPLIT_STAMP(0, wg, 1)
  float lmax = -INFINITY;
  if (p < pos) {
    float acc = 0.0f;
#pragma unroll
    for (int u = 0; u < R8; ++u) {
      __builtin_amdgcn_sched_barrier(0);
      const float4 qa = reinterpret_cast<const float4*>(qs)[2 * u];
      const float4 qb = reinterpret_cast<const float4*>(qs)[2 * u + 1];
      const float e0 = mul_f16_lo(qa.x, row[u].x), e1 = mul_f16_hi(qa.y, row[u].x);
      const float e2 = mul_f16_lo(qa.z, row[u].y), e3 = mul_f16_hi(qa.w, row[u].y);
      const float e4 = mul_f16_lo(qb.x, row[u].z), e5 = mul_f16_hi(qb.y, row[u].z);
      const float e6 = mul_f16_lo(qb.z, row[u].w), e7 = mul_f16_hi(qb.w, row[u].w);
      acc += e0;
      acc += e1;
      acc += e2;
      acc += e3;
      acc += e4;
      acc += e5;
      acc += e6;
      acc += e7;
    }
    const float sv = acc * scale;
    if (TAG)
      st_agent64(sc_t + (size_t)h * kvs + p, tg | __float_as_uint(sv));
    else
      g_sc[(size_t)h * kvs + p] = sv;
    lmax = sv;
  } else if (p == pos) {  // this token's own key, from LDS (16-byte reads, 8 products ahead of their adds)
    float acc = 0.0f;
    const float4* q4 = reinterpret_cast<const float4*>(qs);
    const float4* k4 = reinterpret_cast<const float4*>(kn);
#pragma unroll
    for (int u = 0; u < HD / 8; ++u) {
      const float4 qa = q4[2 * u], qb = q4[2 * u + 1], ka = k4[2 * u], kb = k4[2 * u + 1];
      const float p0 = qa.x * ka.x, p1 = qa.y * ka.y, p2 = qa.z * ka.z, p3 = qa.w * ka.w;
      const float p4 = qb.x * kb.x, p5 = qb.y * kb.y, p6 = qb.z * kb.z, p7 = qb.w * kb.w;
      acc += p0;
      acc += p1;
      acc += p2;
      acc += p3;
      acc += p4;
      acc += p5;
      acc += p6;
      acc += p7;
    }
    const float sv = acc * scale;
    if (TAG)
      st_agent64(sc_t + (size_t)h * kvs + p, tg | __float_as_uint(sv));
    else
      g_sc[(size_t)h * kvs + p] = sv;
    lmax = sv;
  }
  CM_SPLIT_STAMP(0, wg, 2)
  if (!TAG) {
    const float mx = block_max(lmax, red);
    if (tid == 0) g_max[(size_t)h * n_slices + s] = mx;
  }
  CM_SPLIT_STAMP(0, wg, 3)
}

template <int HD, bool FUSED, int NT>
__global__ __launch_bounds__(NT) void k_att_scores(
    const float* __restrict__ qsrc, int n_heads, int n_kv, int rope_dim, int split_half,
    const float* __restrict__ cos_base, const float* __restrict__ sin_base, int rope_stride,
    const float* __restrict__ q_norm, const float* __restrict__ k_norm, float eps, uint16_t* __restrict__ kc,
    uint16_t* __restrict__ vc, int layer, int kvs, const uint32_t* __restrict__ d_pos, float scale,
    float* __restrict__ g_sc, float* __restrict__ g_max) {
  const int h = gridDim.x % N_XCD == 0 ? xcd_member(blockIdx.x, n_kv, n_heads / n_kv) : (int)blockIdx.x;
  att_scores_body<HD, FUSED, NT, NT, false>(h, (int)blockIdx.y, (int)gridDim.y, qsrc, n_heads, n_kv, rope_dim,
                                            split_half, cos_base, sin_base, rope_stride, q_norm, k_norm, eps, kc, vc,
                                            layer, kvs, d_pos, scale, g_sc, g_max, nullptr);
}

// The split output kernel's products: two buffers of [32 dims][PB positions + 4] f32 (the
// row pad keeps the 16-byte LDS reads and writes of consecutive dims on distinct banks),
// placed after the scores in dynamic LDS.  Larger blocks pay the per-block barrier fewer
// times; the launch takes the largest of 256, 128, 64 that leaves three 16 KB V ring chunks.
__host__ __device__ constexpr size_t avp_bytes(int pb) { return (size_t)2 * 32 * (pb + 4) * 4; }

// Output workgroup `bid` (32 dims of one head).  TAG (k_att_fused): the head's scores are read
// as tagged words (sc_t) once the score workgroups of the same launch have stored them, and
// their maximum is taken here; this position's V row comes from qsrc (the cache row is stored
// by a score workgroup of the same launch); with op.q the Q8_0 output goes out as tagged words
// for the output projection's workgroups (att_oproj).
template <int HD, int PB, bool TAG>
__device__ __forceinline__ void att_out_body(
    int bid, const uint16_t* __restrict__ vc, int n_heads, int n_kv, int layer, int kvs,
    const uint32_t* __restrict__ d_pos, const float* __restrict__ g_sc, const float* __restrict__ g_max,
    int n_slices, int n_slices_pos, float* __restrict__ att_out, int8_t* __restrict__ xq, float* __restrict__ xs,
    int ring_slots, const uint64_t* __restrict__ sc_t, const float* __restrict__ qsrc, const OProj& op) {
  constexpr int ATT_NT = att_nt(HD);
  constexpr int NW = ATT_NT / 64;
  constexpr int DW = 32;                       // output dims per workgroup: one Q8_0 block
  constexpr int NDW = HD / DW;
  constexpr int NH = (NW - 1) >= 8 ? 8 : 4;    // V-staging waves 1..NH
  constexpr int LH = AO_RING_LOADS / NH;      // 1 KB wave loads per staging wave per chunk
  constexpr int CG = AO_RING_GRANULES / DW;   // 8-position groups per ring chunk
  static_assert(CG % 4 == 0, "ring chunks hold a multiple of 4 granule groups");
  constexpr int BG = PB / 8;  // groups per product block
  constexpr int AVP_RS = PB + 4;
  static_assert(CG % BG == 0, "product blocks tile the ring chunks");
  extern __shared__ __align__(16) float4 dyn[];
  float4* ring = dyn;
  float* sc = reinterpret_cast<float*>(dyn + (size_t)ring_slots * AO_RING_GRANULES);
  float* pbuf = sc + ((kvs + 3) & ~3);  // (16-byte aligned)
  __shared__ float red[NW];
  __shared__ float s_inv;
  __shared__ uint64_t etab[32];
  __shared__ FsLds<ATT_NT> fs;
  const int tid = threadIdx.x;
  const int rep = n_heads / n_kv;
  // (head, part): unit u = kv head * NDW + w, shared by the group's rep heads
  const int m = xcd_member(bid, n_kv * NDW, rep);
  const int w = (m / rep) % NDW, h = (m / rep / NDW) * rep + m % rep;
  const size_t hbase = kv_head_base(layer, n_kv, h / rep, HD, kvs);
  const uint4* vg = reinterpret_cast<const uint4*>(vc + hbase);  // V granule (g, d): g * HD + d
  const int pos = (int)*d_pos;
  if (kv_pos_bad(pos, kvs)) return;  // (uniform, before any barrier)
  const int P = pos + 1;
  const int d = w * DW + tid;  // output lanes: tid < DW
  const uint32_t tag = (TAG || op.q) ? ao_tag((uint32_t)pos, (uint32_t)layer) : 0u;
  // this position's V value of output lane d (TAG: from the projection's output, rounded to
  // f16 as the cache row that a score workgroup of this launch stores)
  auto v_pos = [&]() -> uint16_t {
    if (TAG) return f32_to_f16_bits(qsrc[(size_t)(n_heads + n_kv) * HD + (size_t)(h / rep) * HD + d]);
    return vc[hbase + kv_v_index(HD, pos, d)];
  };
  float acc = 0.0f;
  CM_SPLIT_STAMP(1, bid, 0)
  if (P == 1) {
    // inference.rs:23564-23575: a single position copies the V row
    if (tid < DW) acc = half_bits_to_float(v_pos());
  } else {
    const int ng = pos >> 3;  // full groups of 8 positions before pos
    // the output lanes' V values past the full groups (positions ng*8 .. pos, at most 8), loaded
    // now: the output chain adds them from registers at the end
    uint16_t vtail[8];
    if (tid < DW) {
#pragma unroll
      for (int u = 0; u < 8; ++u)
        vtail[u] = ng * 8 + u < pos ? vc[hbase + kv_v_index(HD, ng * 8 + u, d)]
                                    : (ng * 8 + u == pos ? v_pos() : (uint16_t)0);
    }
    if (tid < 32) etab[tid] = kExp2Tab[tid];
    const int R = ring_slots;
    const int nchunks = (ng + CG - 1) / CG;
    const int hw = (tid >> 6) - 1;
    const bool stager = hw >= 0 && hw < NH;
    const size_t last_group = (size_t)max(ng, 1) - 1;
    auto stage = [&](int c) {  // chunk c into slot c % R: 1 KB wave load i = groups 2i, 2i+1
      float4* slot = ring + (size_t)(c % R) * AO_RING_GRANULES;
#pragma unroll
      for (int j = 0; j < LH; ++j) {
        const int i = hw + NH * j;
        const int lane = tid & 63;
        const size_t grp = min((size_t)c * CG + 2 * i + (lane >> 5), last_group);
        __builtin_amdgcn_global_load_lds(reinterpret_cast<const void*>(vg + grp * HD + w * DW + (lane & 31)),
                                         (__attribute__((address_space(3))) void*)(slot + i * 64), 16, 0, 0);
      }
    };
    const bool onepass = P >= ATT_FOLD_MAX && P <= ATT_NT * ATT_ONEPASS_C;
    const bool early = P <= ATT_NT * ATT_ONEPASS_C;
    const bool seg = !early && att_seg_chunk<ATT_NT>(P) > 0 &&
                     att_seg_bytes<ATT_NT>(P) <= (size_t)R * AO_RING_GRANULES * 16;
    float lm = -INFINITY;
    const int nsl = (P + n_slices_pos - 1) / n_slices_pos;
    if (TAG) {
      // the first V chunks go out first (the scores are not there yet); then one watcher until
      // this position's score carries the tag, then every score word, read by the waves that
      // stage no V (a wave's loads complete in order: behind its V loads a score word would
      // wait for them).  (Measured at C3: watching each slice's last cache position instead
      // starts the reads 0.8 us later.)
      (void)nsl;
      if (stager && !seg) {
        for (int c = 0; c < min(R - 1, nchunks); ++c) stage(c);
      }
      const uint64_t* gs = sc_t + (size_t)h * kvs;
      if (tid == 0) (void)ao_wait_word(gs + pos, tag);
      __syncthreads();
      // (with the segmented denominator no V is staged yet: every wave reads)
      if (!stager || seg) {
        const int i0 = seg || tid < 64 ? tid : tid - 64 * NH;  // wave 0, then waves NH + 1 ..
        const int ns = seg ? ATT_NT : ATT_NT - 64 * NH;
        // eight words in flight per thread; a word not yet tagged is polled on its own
        for (int b0 = i0; b0 < P; b0 += 8 * ns) {
          uint64_t v[8];
#pragma unroll
          for (int u = 0; u < 8; ++u) v[u] = b0 + u * ns < P ? ld_agent64(gs + b0 + u * ns) : 0;
#pragma unroll
          for (int u = 0; u < 8; ++u) {
            const int p = b0 + u * ns;
            if (p < P) {
              if ((uint32_t)(v[u] >> 32) != tag) v[u] = ao_wait_word(gs + p, tag);
              const float f = __uint_as_float((uint32_t)v[u]);
              sc[p] = f;
              lm = fmaxf(lm, f);
            }
          }
        }
      }
    } else {
      const float* gs = g_sc + (size_t)h * kvs;
      for (int p = tid; p < P; p += ATT_NT) sc[p] = gs[p];
      for (int i = tid; i < nsl; i += ATT_NT) lm = fmaxf(lm, g_max[(size_t)h * n_slices + i]);
      // the first V chunks go out behind the scores loads (nothing waits on them before the
      // output sum; the segmented denominator uses the ring first and stages afterwards)
      if (stager && !seg) {
        for (int c = 0; c < min(R - 1, nchunks); ++c) stage(c);
      }
    }
    const float mx = block_max(lm, red);  // (its barriers also publish sc and etab)
    CM_SPLIT_STAMP(1, bid, 1)
    for (int p = tid; p < P; p += ATT_NT) sc[p] = glibc_expf_t(sc[p] - mx, etab);
    __syncthreads();
    CM_SPLIT_STAMP(1, bid, 2)
    float inv;
    if (onepass) {
      inv = 1.0f / att_onepass_sum<ATT_NT>(sc, P, fs);
    } else {
      if (seg) {
        const float ssum = att_seg_sum<ATT_NT>(sc, reinterpret_cast<uint32_t*>(ring), P);
        if (tid == 0) s_inv = 1.0f / ssum;
        if (stager) {
          for (int c = 0; c < min(R - 1, nchunks); ++c) stage(c);
        }
      } else if (tid == 0) {
        s_inv = 1.0f / fold_lds(sc, P);
      }
      __syncthreads();
      inv = s_inv;
    }
    CM_SPLIT_STAMP(1, bid, 3)
    for (int p = tid; p < P; p += ATT_NT) sc[p] = sc[p] * inv;
    // ---- out_d = fold_p prob_p * v_pd over the full 8-position groups: the products of a
    // block of BG groups are formed by all waves but wave 0 (the rounded f32 product of the
    // probability and the f16 value, as the chain would form it) into one of two LDS buffers,
    // while wave 0's output lanes (lane d = dim d) add the previous block's in position
    // order: the chain then only adds.  One barrier per block; the staging waves keep V
    // chunks landing in the ring on a fixed schedule (chunk c's slot is refilled once the
    // products of its last block have been formed).
    constexpr int BPC = CG / BG;  // product blocks per ring chunk
    const int nb = (ng + BG - 1) / BG;
    int issued = min(R - 1, nchunks);  // ring chunks issued so far (staging waves)
    auto products = [&](int b) {
      const int c = b / BPC;
      const uint4* slot = reinterpret_cast<const uint4*>(ring + (size_t)(c % R) * AO_RING_GRANULES);
      float* dst0 = pbuf + (size_t)(b & 1) * DW * AVP_RS;
      for (int gi = tid - 64; gi < BG * DW; gi += ATT_NT - 64) {
        const int gl = gi / DW, dd = gi % DW, g = b * BG + gl;
        if (g < ng) {
          const uint4 v = slot[(g - c * CG) * DW + dd];
          const float4 q0 = reinterpret_cast<const float4*>(sc)[2 * g];
          const float4 q1 = reinterpret_cast<const float4*>(sc)[2 * g + 1];
          float4* dst = reinterpret_cast<float4*>(dst0 + (size_t)dd * AVP_RS + gl * 8);
          dst[0] = make_float4(mul_f16_lo(q0.x, v.x), mul_f16_hi(q0.y, v.x), mul_f16_lo(q0.z, v.y),
                               mul_f16_hi(q0.w, v.y));
          dst[1] = make_float4(mul_f16_lo(q1.x, v.z), mul_f16_hi(q1.y, v.z), mul_f16_lo(q1.z, v.w),
                               mul_f16_hi(q1.w, v.w));
        }
      }
    };
    if (nb > 0) {
      if (stager) {
        if (issued < min(R, nchunks)) stage(issued++);  // chunk R - 1 into the unused slot
        // chunk 0 has landed, and the chunk of block 1 (chunk 1 when a chunk holds one block):
        // block 1's products are formed in the loop's first iteration, before its first wait
        const int q1 = min(nchunks - 1, 1 / BPC);
        wait_vmcnt(LH * (issued - 1 - q1));
      }
      __syncthreads();  // chunk 0 and the normalised probabilities
      if (tid >= 64) products(0);
      __syncthreads();
    }
#ifdef CM_STAMPS
    uint64_t t_adds = 0, t_wait = 0, t_mark = 0;  // (thread 0: time in the adds, at the barriers)
#endif
    for (int b = 0; b < nb; ++b) {
#ifdef CM_STAMPS
      if (tid == 0) t_mark = __builtin_amdgcn_s_memrealtime();
#endif
      if (tid < DW) {
        const float4* row = reinterpret_cast<const float4*>(pbuf + ((size_t)(b & 1) * DW + tid) * AVP_RS);
        const int n4 = min(BG, ng - b * BG) * 2;  // 4-position pieces of this block
        if (n4 == BG * 2) {
          // 8 pieces in flight ahead of the adds (ping-pong), as in fold_lds
          float4 x[8], y[8];
#pragma unroll
          for (int i = 0; i < 8; ++i) x[i] = row[i];
#pragma unroll
          for (int j = 8; j < BG * 2; j += 16) {
#pragma unroll
            for (int i = 0; i < 8; ++i) y[i] = row[j + i];
            __builtin_amdgcn_sched_barrier(0);
            add8(acc, x);
            if (j + 8 < BG * 2) {
#pragma unroll
              for (int i = 0; i < 8; ++i) x[i] = row[j + 8 + i];
            }
            __builtin_amdgcn_sched_barrier(0);
            add8(acc, y);
          }
        } else {
          for (int i = 0; i < n4; ++i) add4(acc, row[i]);
        }
      } else if (tid >= 64) {
        if (b + 1 < nb) products(b + 1);
        if (stager) {
          // chunk c's last block was formed in the previous iteration: refill its slot
          if (b % BPC == BPC - 1) {
            const int c = (b - (BPC - 1)) / BPC;
            if (c + R < nchunks && c + R >= issued) stage(issued++);
          }
          // the products of the next iteration read a new chunk: it must have landed
          const int q = (b + 2) / BPC;
          if ((b + 2) % BPC == 0 && q < nchunks) wait_vmcnt(LH * (issued - 1 - q));
        }
      }
#ifdef CM_STAMPS
      if (tid == 0) {
        const uint64_t t1 = __builtin_amdgcn_s_memrealtime();
        t_adds += t1 - t_mark;
        t_mark = t1;
      }
#endif
      __syncthreads();  // wave 0 is done with buffer b & 1; block b + 1's products are visible
#ifdef CM_STAMPS
      if (tid == 0) t_wait += __builtin_amdgcn_s_memrealtime() - t_mark;
#endif
    }
#ifdef CM_STAMPS
    if (tid == 0 && bid < SPLIT_STAMP_WGS) {  // slots 6, 7: sums over the blocks, not times
      g_split_stamps[(SPLIT_STAMP_WGS + bid) * SPLIT_NSTAMP + 6] = t_adds;
      g_split_stamps[(SPLIT_STAMP_WGS + bid) * SPLIT_NSTAMP + 7] = t_wait;
    }
#endif
    CM_SPLIT_STAMP(1, bid, 4)
    if (tid < DW) {
#pragma unroll
      for (int u = 0; u < 8; ++u)
        if (ng * 8 + u < P) acc += sc[ng * 8 + u] * half_bits_to_float(vtail[u]);
    }
  }
  if (tid < DW) {
    const size_t o = (size_t)h * HD + d;
    att_out[o] = acc;
    if (TAG && op.xf_t)  // the f32 value, tagged, for the Q4_K projection's workgroups of this launch
      st_agent64(op.xf_t + o, ((uint64_t)tag << 32) | __float_as_uint(acc));
    int8_t q;
    const float dd = quantize_lane32(acc, &q);
    if (op.q) {  // for the output projection's workgroups of this launch (as k_attention)
      const uint64_t tg = (uint64_t)tag << 32;
      const uint32_t b = (uint32_t)(uint8_t)q;
      const uint32_t wq = b | ((uint32_t)__shfl_down((int)b, 1) << 8) | ((uint32_t)__shfl_down((int)b, 2) << 16) |
                          ((uint32_t)__shfl_down((int)b, 3) << 24);
      if ((tid & 3) == 0) st_agent64(op.xq_t + (o >> 2), tg | wq);
      if (tid == 0) st_agent64(op.xs_t + (o >> 5), tg | __float_as_uint(dd));
    } else {
      xq[o] = q;
      if (tid == 0) xs[o >> 5] = dd;
    }
  }
  CM_SPLIT_STAMP(1, bid, 5)
}

template <int HD, int PB>
__global__ __launch_bounds__(att_nt(HD)) void k_att_out(
    const uint16_t* __restrict__ vc, int n_heads, int n_kv, int layer, int kvs, const uint32_t* __restrict__ d_pos,
    const float* __restrict__ g_sc, const float* __restrict__ g_max, int n_slices, int n_slices_pos,
    float* __restrict__ att_out,
    int8_t* __restrict__ xq, float* __restrict__ xs, int ring_slots, Prefetch pf, OProj op) {
  const int nwork = n_heads * (HD / 32);
  if ((int)blockIdx.x >= nwork) {
    extern __shared__ __align__(16) float4 dyn[];
    if constexpr (att_nt(HD) == AO_ROWS * 64) {
      if (op.q) {  // the output projection's workgroups (AO_SPLIT_RPW rows per wave)
        const int pos = (int)*d_pos;
        if (kv_pos_bad(pos, kvs)) return;
        att_oproj<att_nt(HD), AO_SPLIT_RPW>(op, (int)blockIdx.x - nwork, ao_tag((uint32_t)pos, (uint32_t)layer),
                                            reinterpret_cast<unsigned char*>(dyn));
        return;
      }
    }
    // spare workgroups: read ahead the output projection
    prefetch_lines(pf, blockIdx.x - nwork, gridDim.x - nwork,
                   reinterpret_cast<float*>(dyn + (size_t)ring_slots * AO_RING_GRANULES));
    return;
  }
  att_out_body<HD, PB, false>((int)blockIdx.x, vc, n_heads, n_kv, layer, kvs, d_pos, g_sc, g_max, n_slices,
                              n_slices_pos, att_out, xq, xs, ring_slots, nullptr, nullptr, op);
}

// The Q4_K output projection's workgroups of k_att_fused (defined with the K-quant kernels).
template <int NT>
__device__ __forceinline__ void att_oproj_q4k(const OProj& op, int wg, uint32_t tag);

// ---------------------------------------------------------------------------
// The split decode attention in one launch (no round trip of the scores through a launch
// boundary): workgroups [0, n_heads * n_slices) are score slices of SL positions (slice s of
// head h at s * n_heads + h: every head's first slices are dispatched first), then n_heads *
// HD / 32 output workgroups, then (op.q set) the output projection's workgroups.  Every
// workgroup waits only for workgroups of lower index, which the dispatcher has started
// before it, so the waits end whatever the number of CUs.  Same arithmetic and order as
// k_att_scores + k_att_out + k_gemv_k.
template <int HD, int PB, int SL>
__global__ __launch_bounds__(att_nt(HD)) void k_att_fused(
    const float* __restrict__ qsrc, int n_heads, int n_kv, int rope_dim, int split_half,
    const float* __restrict__ cos_base, const float* __restrict__ sin_base, int rope_stride,
    const float* __restrict__ q_norm, const float* __restrict__ k_norm, float eps, uint16_t* __restrict__ kc,
    uint16_t* __restrict__ vc, int layer, int kvs, const uint32_t* __restrict__ d_pos, float scale,
    uint64_t* __restrict__ sc_t, int n_slices, float* __restrict__ att_out,
    int8_t* __restrict__ xq, float* __restrict__ xs, int ring_slots, OProj op) {
  constexpr int NT = att_nt(HD);
  const int nsw = n_heads * n_slices, now = n_heads * (HD / 32);
  const int b = (int)blockIdx.x;
  if (b < nsw) {
    att_scores_body<HD, true, NT, SL, true>(b % n_heads, b / n_heads, n_slices, qsrc, n_heads, n_kv, rope_dim,
                                            split_half, cos_base, sin_base, rope_stride, q_norm, k_norm, eps, kc, vc,
                                            layer, kvs, d_pos, scale, nullptr, nullptr, sc_t);
  } else if (b < nsw + now) {
    att_out_body<HD, PB, true>(b - nsw, vc, n_heads, n_kv, layer, kvs, d_pos, nullptr, nullptr, n_slices, SL,
                               att_out, xq, xs, ring_slots, sc_t, qsrc, op);
  } else if constexpr (NT == AO_ROWS * 64) {
    if (op.q) {
      extern __shared__ __align__(16) float4 dyn[];
      const int pos = (int)*d_pos;
      if (kv_pos_bad(pos, kvs)) return;
      att_oproj<NT>(op, b - nsw - now, ao_tag((uint32_t)pos, (uint32_t)layer), reinterpret_cast<unsigned char*>(dyn));
    } else if (op.k4nib) {
      const int pos = (int)*d_pos;
      if (kv_pos_bad(pos, kvs)) return;
      att_oproj_q4k<NT>(op, b - nsw - now, ao_tag((uint32_t)pos, (uint32_t)layer));
    }
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

// In-order sums of rows (test hooks): one workgroup per row of n values.  k_inorder_sum_rows:
// the segmented passes (256 threads, n <= 256 * C), the first m_seq terms folded
// sequentially; k_inorder_sum_rows_onepass: the one-pass method as the RMSNorm runs it
// (RMS_NT threads, n <= RMS_NT * C).
template <int C>
__global__ __launch_bounds__(256) void k_inorder_sum_rows(const float* __restrict__ x, int n, int m_seq,
                                                          float* __restrict__ out) {
  __shared__ __align__(16) float v[256 * C];
  __shared__ __align__(16) uint32_t ps[seg_binades(C) * (256 * C + 4)];
  const float* row = x + (size_t)blockIdx.x * n;
  for (int i = threadIdx.x; i < n; i += 256) v[i] = row[i];
  __syncthreads();
  const float sum = inorder_sum_nonneg<256, C>(v, ps, n, m_seq);
  if (threadIdx.x == 0) out[blockIdx.x] = sum;
}

template <int C>
__global__ __launch_bounds__(RMS_NT) void k_inorder_sum_rows_onepass(const float* __restrict__ x, int n,
                                                                     float* __restrict__ out) {
  __shared__ __align__(16) float v[RMS_NT * C];
  const float* row = x + (size_t)blockIdx.x * n;
  for (int i = threadIdx.x; i < n; i += RMS_NT) v[i] = row[i];
  __syncthreads();
  __shared__ FsLds<RMS_NT> fs;
  float t[C];
#pragma unroll
  for (int c = 0; c < C; ++c) t[c] = (int)threadIdx.x * C + c < n ? v[threadIdx.x * C + c] : 0.0f;
  const float sum = inorder_sum_onepass<RMS_NT, C>(t, v, n, fs);
  if (threadIdx.x == 0) out[blockIdx.x] = sum;
}

// glibc-identical expf over a vector (test hook).
__global__ void k_expf(const float* __restrict__ x, float* __restrict__ y, size_t n) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) y[i] = glibc_expf(x[i]);
}

}  // namespace cm
