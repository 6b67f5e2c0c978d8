// camelid_oracle.cpp -- CPU ORACLE (test infrastructure only).
//
// A scalar C++ restatement of Camelid's CPU forward path for the resident
// decode/prefill hot path.  It is the checker for the HIP backend: only the
// tests, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it.
// The product (camelid_amd/) never links or calls it.
//
// Build: g++ -O3 -ffp-contract=off -fopenmp -shared -fPIC (oracle/Makefile).
// -ffp-contract=off is the analogue of Rust never contracting a*b+c into an
// FMA; math functions (expf, sinf, cosf, powf, sqrtf) are glibc's, exactly as
// Rust's f32::{exp,sin,cos,powf,sqrt} resolve on Linux.
//
// Every function cites the reference file:line it restates (paths relative to
// the Camelid source tree).  Parallelism is over independent output rows only
// (each output owns its serial reduction, as rayon's row split does), so the
// thread count never changes a result bit.
//
// Parity pins (what checks each function; see tests/test_oracle_*.py):
//   f16 conversions        - exhaustive vs F16C semantics + reference fixtures F16.json
//   Q8_0 dequant           - reference fixtures Q8_0.json (gguf==0.19.0)
//   quantize_q8_0          - reference KAT q8_0_input_quantization_uses_unrounded_scale
//                            + brute-force properties (round-half-away, clamp); scale and
//                            x * inv expression known answers
//   block int dot          - brute force int64 sums
//   Q8_0 row fold          - exact integer case; order/FMA/association known answers
//   rms_norm               - closed form on constant rows; float64 bound; sum-order and
//                            rounded-square known answers; scale / (x*scale)*w known answer
//   rope                   - pos 0 identity, norm preservation, llama3 KAT; rotation (no
//                            FMA), powf frequency and llama3 association known answers
//   attention              - single-position copy, uniform keys -> mean of V; score-dot,
//                            softmax-sum and AV order / rounded-product known answers;
//                            score scale and e * (1/sum) known answers
//   silu_mul / argmax      - expression known answer / brute force incl. ties
//   quantize_q8_k          - properties; iscale product and d = 1/iscale known answers
//   Q4_K / Q6_K row dots   - fixture-pinned dequant sums; FMA chain and class-chain
//                            left-fold known answers
// tests/test_oracle_mutants.py rebuilds this file with 21 single-expression rewrites and
// requires each to fail one of these pins.
#include <cmath>
#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <vector>
#include <algorithm>
#include <omp.h>

#define OX extern "C" __attribute__((visibility("default")))

namespace {

inline uint32_t f2u(float f) { uint32_t u; std::memcpy(&u, &f, 4); return u; }
inline float u2f(uint32_t u) { float f; std::memcpy(&f, &u, 4); return f; }

// inference.rs:20767-20801 f32_to_f16_bits (round-to-nearest-even, NaN -> 0x7e00).
uint16_t f32_to_f16_bits(float value) {
  uint32_t bits = f2u(value);
  uint16_t sign = (uint16_t)((bits >> 16) & 0x8000);
  int32_t exp = (int32_t)((bits >> 23) & 0xff);
  uint32_t mant = bits & 0x007fffff;
  if (exp == 0xff) return sign | (mant == 0 ? 0x7c00 : 0x7e00);
  int32_t half_exp = exp - 127 + 15;
  if (half_exp >= 0x1f) return sign | 0x7c00;
  if (half_exp <= 0) {
    if (half_exp < -10) return sign;
    uint32_t mantissa = mant | 0x00800000u;
    uint32_t shift = (uint32_t)(14 - half_exp);
    uint16_t half_mant = (uint16_t)(mantissa >> shift);
    uint32_t round_bit = 1u << (shift - 1);
    if ((mantissa & round_bit) != 0 && ((mantissa & (round_bit - 1)) != 0 || (half_mant & 1) != 0))
      half_mant = (uint16_t)(half_mant + 1);
    return sign | half_mant;
  }
  uint16_t half = (uint16_t)(sign | ((uint16_t)half_exp << 10) | (uint16_t)(mant >> 13));
  if ((mant & 0x00001000u) != 0 && ((mant & 0x00000fffu) != 0 || (half & 1) != 0))
    half = (uint16_t)(half + 1);
  return half;
}

// inference.rs:20803-20830 f16_bits_to_f32 (exact widening).
float f16_bits_to_f32(uint16_t bits) {
  uint32_t sign = ((uint32_t)(bits & 0x8000)) << 16;
  uint32_t exp = (bits & 0x7c00) >> 10;
  uint32_t frac = bits & 0x03ff;
  uint32_t out;
  if (exp == 0) {
    if (frac == 0) {
      out = sign;
    } else {
      uint32_t mant = frac;
      int32_t e = -14;
      while ((mant & 0x0400) == 0) { mant <<= 1; e -= 1; }
      mant &= 0x03ff;
      out = sign | ((uint32_t)(e + 127) << 23) | (mant << 13);
    }
  } else if (exp == 0x1f) {
    out = sign | 0x7f800000u | (frac << 13);
  } else {
    out = sign | ((exp + (127 - 15)) << 23) | (frac << 13);
  }
  return u2f(out);
}

// inference.rs:16953-16971 quantize_q8_0_block: fold max|x|, scale = f16(amax/127),
// quants use the UNROUNDED inverse, round half away from zero, clamp [-128,127].
void quantize_q8_0_block(const float* block, float* scale_out, int8_t* quants) {
  float max_abs = 0.0f;
  for (int i = 0; i < 32; ++i) max_abs = std::fmax(max_abs, std::fabs(block[i]));
  float unrounded = max_abs / 127.0f;
  *scale_out = f16_bits_to_f32(f32_to_f16_bits(unrounded));
  float inv = (unrounded == 0.0f) ? 0.0f : 1.0f / unrounded;
  for (int i = 0; i < 32; ++i) {
    float r = std::round(block[i] * inv);
    r = std::fmin(std::fmax(r, -128.0f), 127.0f);
    quants[i] = (int8_t)r;
  }
}

// inference.rs:20539-20566 q8_0_block_int_dot_horizontal_sum_scalar (exact int32).
int32_t q8_block_dot(const int8_t* w, const int8_t* x) {
  int32_t lanes[4] = {0, 0, 0, 0};
  for (int g = 0; g < 4; ++g) {
    int32_t a = 0, b = 0;
    for (int j = 0; j < 4; ++j) {
      a += (int32_t)w[4 * g + j] * (int32_t)x[4 * g + j];
      b += (int32_t)w[16 + 4 * g + j] * (int32_t)x[16 + 4 * g + j];
    }
    lanes[g] = a + b;
  }
  return (lanes[0] + lanes[1]) + (lanes[2] + lanes[3]);
}

// inference.rs:20421-20443 dot_q8_0_encoded_row_with_scales / :19871-19905 q8_0_dot_rows:
// per block  term = (float(int_dot) * w_scale) * x_scale ; sum += term in block order.
float q8_0_row_dot_wire(const uint8_t* row, const float* xs, const int8_t* xq, size_t nb) {
  float sum = 0.0f;
  for (size_t b = 0; b < nb; ++b) {
    const uint8_t* blk = row + b * 34;
    float ws = f16_bits_to_f32((uint16_t)(blk[0] | (blk[1] << 8)));
    int32_t d = q8_block_dot((const int8_t*)(blk + 2), xq + b * 32);
    sum += ((float)d * ws) * xs[b];
  }
  return sum;
}

// ---------------------------------------------------------------- K-quants
// Projection formats (the C ABI's ProjQuant codes).
enum { Q_Q8_0 = 0, Q_Q4_K = 1, Q_Q6_K = 2 };
inline uint32_t le32(const uint8_t* p) { return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24); }
inline uint16_t le16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }

// inference.rs:17555-17561 nearest_int_reference: adding 1.5*2^23 rounds to nearest even
// into the mantissa.
int32_t nearest_int(float fval) {
  const float val = fval + 12582912.0f;
  return (int32_t)(f2u(val) & 0x007fffffu) - 0x00400000;
}

// inference.rs:17564-17599 quantize_q8_k_blocks, one 256-value block: max = the signed
// value of the first largest |x| (strict >), iscale = -127/max, q = min(nearest_int(iscale*x),
// 127) (wrapped to i8), d = 1/iscale; an all-zero block gives d = 0, q = 0.
void quantize_q8_k_block(const float* x, float* d, int8_t* qs) {
  float amax = 0.0f, mx = 0.0f;
  for (int i = 0; i < 256; ++i)
    if (std::fabs(x[i]) > amax) { amax = std::fabs(x[i]); mx = x[i]; }
  if (amax == 0.0f) {
    *d = 0.0f;
    std::memset(qs, 0, 256);
    return;
  }
  const float iscale = -127.0f / mx;
  for (int i = 0; i < 256; ++i) qs[i] = (int8_t)std::min(nearest_int(iscale * x[i]), 127);
  *d = 1.0f / iscale;
}

// tensor/mod.rs:4776-4785 q4_k_scale_min: 6-bit (scale, min) of sub-block idx.
void q4_k_scale_min(int idx, const uint8_t* sc, uint8_t* scale, uint8_t* mn) {
  if (idx < 4) {
    *scale = sc[idx] & 63;
    *mn = sc[idx + 4] & 63;
  } else {
    *scale = (uint8_t)((sc[idx + 4] & 0x0f) | ((sc[idx - 4] >> 6) << 4));
    *mn = (uint8_t)((sc[idx + 4] >> 4) | ((sc[idx] >> 6) << 4));
  }
}

// tensor/mod.rs:4682-4703 Q4KBlock::dequantize (144-byte superblock: f16 d, f16 dmin,
// 12 packed scale/min bytes, 128 nibble bytes): out = (d*sc)*q - dmin*m.
void dequant_q4_k_block(const uint8_t* b, float* out) {
  const float d = f16_bits_to_f32(le16(b)), dmin = f16_bits_to_f32(le16(b + 2));
  for (int pair = 0; pair < 4; ++pair) {
    uint8_t ls, lm, hs, hm;
    q4_k_scale_min(2 * pair, b + 4, &ls, &lm);
    q4_k_scale_min(2 * pair + 1, b + 4, &hs, &hm);
    const float lo_s = d * (float)ls, hi_s = d * (float)hs, lo_m = dmin * (float)lm, hi_m = dmin * (float)hm;
    for (int l = 0; l < 32; ++l) {
      const uint8_t byte = b[16 + pair * 32 + l];
      out[pair * 64 + l] = lo_s * (float)(byte & 0x0f) - lo_m;
      out[pair * 64 + 32 + l] = hi_s * (float)(byte >> 4) - hi_m;
    }
  }
}

// The signed 6-bit weights of a Q6_K superblock (210 bytes: ql[128], qh[64], i8 scales[16],
// f16 d), in value order (inference.rs:19256-19276; tensor/mod.rs:4818-4845).
void q6_k_values(const uint8_t* b, int8_t* a) {
  for (int n = 0; n < 2; ++n) {
    const uint8_t* ql = b + 64 * n;
    const uint8_t* qh = b + 128 + 32 * n;
    int8_t* w = a + 128 * n;
    for (int l = 0; l < 32; ++l) {
      w[l] = (int8_t)(((ql[l] & 0xF) | ((qh[l] & 3) << 4)) - 32);
      w[l + 32] = (int8_t)(((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32);
      w[l + 64] = (int8_t)(((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32);
      w[l + 96] = (int8_t)(((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32);
    }
  }
}

// tensor/mod.rs:4818-4845 Q6KBlock::dequantize: out = (d*sc)*q.
void dequant_q6_k_block(const uint8_t* b, float* out) {
  const float d = f16_bits_to_f32(le16(b + 208));
  int8_t a[256];
  q6_k_values(b, a);
  for (int i = 0; i < 256; ++i) out[i] = d * (float)(int8_t)b[192 + i / 16] * (float)a[i];
}

// refmath.rs:503-561 q4_k_dot_scalar (= q4_k_dot_arm, the CPU decode's Q4_K dot via
// inference.rs:17906-17965): per superblock exact integer mins product and scaled nibble
// dots, then sumf = fma(-dmin, prod, sumf); sumf = fma(d, sumi1 + sumi2, sumf), with
// d = y.d * f16(d_w), dmin = y.d * f16(dmin_w).
float q4_k_row_dot(const uint8_t* row, const float* yd, const int8_t* yqs, size_t nsb) {
  const uint32_t K1 = 0x3f3f3f3f, K2 = 0x0f0f0f0f, K3 = 0x03030303;
  float sumf = 0.0f;
  for (size_t s = 0; s < nsb; ++s) {
    const uint8_t* b = row + s * 144;
    const float d = yd[s] * f16_bits_to_f32(le16(b));
    const float dmin = yd[s] * f16_bits_to_f32(le16(b + 2));
    const uint32_t u0 = le32(b + 4), u1 = le32(b + 8), u2 = le32(b + 12);
    const uint32_t mins8[2] = {u1 & K1, ((u2 >> 4) & K2) | (((u1 >> 6) & K3) << 4)};
    const uint32_t scw[2] = {u0 & K1, (u2 & K2) | (((u0 >> 6) & K3) << 4)};
    auto scale_at = [&](int g) { return (int64_t)((scw[g / 4] >> (8 * (g % 4))) & 0xff); };
    auto min_at = [&](int g) { return (int64_t)((mins8[g / 4] >> (8 * (g % 4))) & 0xff); };
    const int8_t* q8 = yqs + s * 256;
    int64_t prod = 0;
    for (int g = 0; g < 8; ++g) {
      int64_t bs = 0;
      for (int t = 0; t < 32; ++t) bs += q8[32 * g + t];
      prod += bs * min_at(g);
    }
    sumf = std::fma(-dmin, (float)prod, sumf);
    int64_t sumi1 = 0, sumi2 = 0;
    for (int j = 0; j < 4; ++j) {
      const uint8_t* q4 = b + 16 + 32 * j;
      int64_t lo = 0, hi = 0;
      for (int t = 0; t < 32; ++t) {
        lo += (int64_t)(q4[t] & 0xf) * q8[64 * j + t];
        hi += (int64_t)(q4[t] >> 4) * q8[64 * j + 32 + t];
      }
      sumi1 += lo * scale_at(2 * j);
      sumi2 += hi * scale_at(2 * j + 1);
    }
    sumf = std::fma(d, (float)(sumi1 + sumi2), sumf);
  }
  return sumf;
}

// inference.rs:19240-19295 q6_k_wire_row_dot (the CPU decode's Q6_K dot via
// inference.rs:19148-19195): per superblock 8 integer lanes aux[l] (l = position mod 8)
// += scale_j * q8 * a; sums[l] += (f16(d_w) * y.d) * aux[l]; the result is the left fold of
// sums[0..8] (Rust's f32 Sum, whose initial value is -0.0).
float q6_k_row_dot(const uint8_t* row, const float* yd, const int8_t* yqs, size_t nsb) {
  float sums[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  int8_t a[256];
  for (size_t s = 0; s < nsb; ++s) {
    const uint8_t* b = row + s * 210;
    const float d = f16_bits_to_f32(le16(b + 208)) * yd[s];
    q6_k_values(b, a);
    const int8_t* q8 = yqs + s * 256;
    int32_t aux[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int j = 0; j < 16; ++j) {
      const int32_t scale = (int8_t)b[192 + j];
      const int off = j * 16;
      for (int l = 0; l < 8; ++l) aux[l] += scale * (int32_t)q8[off + l] * (int32_t)a[off + l];
      for (int l = 0; l < 8; ++l) aux[l] += scale * (int32_t)q8[off + 8 + l] * (int32_t)a[off + 8 + l];
    }
    for (int l = 0; l < 8; ++l) sums[l] += d * (float)aux[l];
  }
  float r = -0.0f;
  for (int l = 0; l < 8; ++l) r += sums[l];
  return r;
}

size_t quant_row_bytes(int quant, size_t k) {
  return quant == Q_Q8_0 ? k / 32 * 34 : quant == Q_Q4_K ? k / 256 * 144 : k / 256 * 210;
}

// tensor/mod.rs:2083-2106 rms_norm_into (scalar branch): sequential sum of squares,
// /n, scale = 1/sqrt(ms+eps), out = (x*scale)*w.
void rms_norm_row(const float* x, const float* w, size_t n, float eps, float* out) {
  float ss = 0.0f;
  for (size_t i = 0; i < n; ++i) ss += x[i] * x[i];
  float ms = ss / (float)n;
  float scale = 1.0f / std::sqrt(ms + eps);
  for (size_t i = 0; i < n; ++i) out[i] = (x[i] * scale) * w[i];
}

// tensor/mod.rs:2632-2648 dot_product (sequential; the 4-way unroll keeps order).
float dot_product(const float* a, const float* b, size_t n) {
  float sum = 0.0f;
  for (size_t i = 0; i < n; ++i) sum += a[i] * b[i];
  return sum;
}

// ---------------------------------------------------------------- RoPE
// rope.rs:526-560 rope_pair_frequency, :687-711 llama3_scaled_rope_frequency,
// :568-627 resident_decode_rope_tables.
struct RopeCfg {
  uint32_t rope_dim;
  float freq_base;
  int scaling_kind;        // 0 none, 1 linear, 2 llama3
  float factor;
  float orig_ctx;          // llama3 original_context_length (as f32)
  float low_freq_factor;
  float high_freq_factor;
  const float* rope_freqs; // optional per-pair divisors (rope_freqs.weight)
};

float llama3_scaled(float frequency, const RopeCfg& c) {
  const float PI_F = 3.14159265358979323846f;
  float wavelength = (2.0f * PI_F) / frequency;
  float low_wl = c.orig_ctx / c.low_freq_factor;
  float high_wl = c.orig_ctx / c.high_freq_factor;
  if (wavelength < high_wl) return frequency;
  if (wavelength > low_wl) return frequency / c.factor;
  float smooth = (c.orig_ctx / wavelength - c.low_freq_factor) / (c.high_freq_factor - c.low_freq_factor);
  return ((1.0f - smooth) * frequency / c.factor) + (smooth * frequency);
}

float rope_pair_frequency(uint32_t pair, const RopeCfg& c) {
  float base = std::pow(c.freq_base, -((float)pair * 2.0f) / (float)c.rope_dim);
  float eff = c.rope_freqs ? base / c.rope_freqs[pair] : base;
  switch (c.scaling_kind) {
    case 1: return eff / c.factor;
    case 2: return llama3_scaled(eff, c);
    default: return eff;
  }
}

void rope_tables(const RopeCfg& c, uint32_t pos0, uint32_t n_pos, float* cos_out, float* sin_out) {
  uint32_t half = c.rope_dim / 2;
  std::vector<float> f(half);
  for (uint32_t p = 0; p < half; ++p) f[p] = rope_pair_frequency(p, c);
  for (uint32_t i = 0; i < n_pos; ++i) {
    float eff = (float)(pos0 + i);
    for (uint32_t p = 0; p < half; ++p) {
      float a = eff * f[p];
      // mscale is exactly 1.0 for none/linear/llama3 (rope.rs:370-375).
      cos_out[(size_t)i * half + p] = std::cos(a);
      sin_out[(size_t)i * half + p] = std::sin(a);
    }
  }
}

// rope.rs:489-524 apply_rope_to_row (forward direction), pairing 0 adjacent / 1 split-half.
void apply_rope(float* data, uint32_t heads, uint32_t hd, uint32_t rope_dim, const float* cosv,
                const float* sinv, int split_half) {
  uint32_t half = rope_dim / 2;
  for (uint32_t p = 0; p < half; ++p) {
    float c = cosv[p], s = sinv[p];
    for (uint32_t h = 0; h < heads; ++h) {
      size_t base = (size_t)h * hd;
      size_t d0 = split_half ? base + p : base + 2 * p;
      size_t d1 = split_half ? base + p + half : d0 + 1;
      float x0 = data[d0], x1 = data[d1];
      data[d0] = (x0 * c) - (x1 * s);
      data[d1] = (x0 * s) + (x1 * c);
    }
  }
}

// tensor/mod.rs:1943-1967 silu_mul: (g / (1 + exp(-g))) * u.
inline float silu_mul1(float g, float u) { return (g / (1.0f + std::exp(-g))) * u; }

// ---------------------------------------------------------------- Model
struct Model {
  uint32_t L, n_heads, n_kv, hd, H, F, V, max_pos;
  float eps;
  int split_half;
  // per layer wire pointers (Q8_0 34 B blocks, Q4_K 144 B or Q6_K 210 B superblocks),
  // borrowed from the caller; qt[l*7 + proj] = the projection's format (q,k,v,o,gate,up,down)
  std::vector<const uint8_t*> wq, wk, wv, wo, wg, wu, wd;
  std::vector<uint8_t> qt;
  int out_quant = Q_Q8_0, embd_quant = Q_Q8_0;
  std::vector<const float*> attn_norm, ffn_norm, q_norm, k_norm;
  const float* out_norm = nullptr;
  const uint8_t* out_w = nullptr;   // lm_head (may equal token_embd when tied)
  const uint8_t* embd = nullptr;    // token_embd Q8_0 wire [V][H]
  // KV cache: f32 holding f16-rounded values, [L][n_kv][max_pos][hd]
  std::vector<float> kc, vc;
  // scratch
  std::vector<float> h, xn, q, k, v, ctx, tmp, g, u, act, logits;
  std::vector<float> xs; std::vector<int8_t> xq;
  std::vector<float> kd; std::vector<int8_t> kq;  // Q8_K activation
};

void quantize_row(const float* x, size_t n, std::vector<float>& xs, std::vector<int8_t>& xq) {
  size_t nb = n / 32;
  xs.resize(nb); xq.resize(n);
  for (size_t b = 0; b < nb; ++b) quantize_q8_0_block(x + b * 32, &xs[b], &xq[b * 32]);
}

// Q8_0 linear (inference.rs:16766-16803): quantize input once, each output row a serial block fold.
void linear_q8(const uint8_t* w, size_t rows, size_t k, const float* x, float* out,
               std::vector<float>& xs, std::vector<int8_t>& xq) {
  quantize_row(x, k, xs, xq);
  size_t nb = k / 32;
  const float* xsp = xs.data();
  const int8_t* xqp = xq.data();
#pragma omp parallel for schedule(static)
  for (long r = 0; r < (long)rows; ++r)
    out[r] = q8_0_row_dot_wire(w + (size_t)r * nb * 34, xsp, xqp, nb);
}

// A linear layer in the projection's format: Q8_0 as above; K-quants quantize the input
// row to Q8_K once, then dot every wire row (inference.rs:17906-17965 Q4_K,
// :19148-19195 Q6_K).
void linear(Model& m, const uint8_t* w, int quant, size_t rows, size_t k, const float* x, float* out) {
  if (quant == Q_Q8_0) {
    linear_q8(w, rows, k, x, out, m.xs, m.xq);
    return;
  }
  const size_t nsb = k / 256, rb = quant_row_bytes(quant, k);
  m.kd.resize(nsb);
  m.kq.resize(k);
  for (size_t sb = 0; sb < nsb; ++sb) quantize_q8_k_block(x + 256 * sb, &m.kd[sb], &m.kq[256 * sb]);
  const float* kd = m.kd.data();
  const int8_t* kq = m.kq.data();
#pragma omp parallel for schedule(static)
  for (long r = 0; r < (long)rows; ++r)
    out[r] = quant == Q_Q4_K ? q4_k_row_dot(w + (size_t)r * rb, kd, kq, nsb) : q6_k_row_dot(w + (size_t)r * rb, kd, kq, nsb);
}

// inference.rs:23945-24025 attention_context_for_head_into_with_kernels (F32 KV dtype,
// legacy dot_product lane), :23564-23575 single-position copy.
void attention_head(const Model& m, uint32_t layer, uint32_t kvh, const float* qh, uint32_t n_pos,
                    float scale, float* out, std::vector<float>& sc) {
  size_t base = (((size_t)layer * m.n_kv + kvh) * m.max_pos) * m.hd;
  if (n_pos == 1) {
    std::memcpy(out, &m.vc[base], m.hd * sizeof(float));
    return;
  }
  sc.resize(n_pos);
  for (uint32_t p = 0; p < n_pos; ++p) sc[p] = dot_product(qh, &m.kc[base + (size_t)p * m.hd], m.hd) * scale;
  float mx = -INFINITY;
  for (uint32_t p = 0; p < n_pos; ++p) mx = std::fmax(mx, sc[p]);
  float sum = 0.0f;
  for (uint32_t p = 0; p < n_pos; ++p) { sc[p] = std::exp(sc[p] - mx); sum += sc[p]; }
  float inv = 1.0f / sum;
  for (uint32_t d = 0; d < m.hd; ++d) out[d] = 0.0f;
  for (uint32_t p = 0; p < n_pos; ++p) {
    float prob = sc[p] * inv;
    const float* vr = &m.vc[base + (size_t)p * m.hd];
    for (uint32_t d = 0; d < m.hd; ++d) out[d] += prob * vr[d];
  }
}

// inference.rs:6228-6807 forward_layer_timed (Q8_0 llama/qwen3 dense layer).
void forward_layer(Model& m, uint32_t l, uint32_t pos, const float* cosv, const float* sinv,
                   float* capture_q /*nullable*/) {
  const uint32_t H = m.H, hd = m.hd, nq = m.n_heads * hd, nkv = m.n_kv * hd;
  rms_norm_row(m.h.data(), m.attn_norm[l], H, m.eps, m.xn.data());
  // Q/K/V share one quantized input (the row is quantized identically for each linear).
  const uint8_t* qt = &m.qt[(size_t)l * 7];
  linear(m, m.wq[l], qt[0], nq, H, m.xn.data(), m.q.data());
  linear(m, m.wk[l], qt[1], nkv, H, m.xn.data(), m.k.data());
  linear(m, m.wv[l], qt[2], nkv, H, m.xn.data(), m.v.data());
  // per-head QK RMSNorm (tensor/mod.rs:2112-2136) before RoPE (inference.rs:6369-6386).
  if (m.q_norm[l]) for (uint32_t h = 0; h < m.n_heads; ++h) rms_norm_row(&m.q[h * hd], m.q_norm[l], hd, m.eps, &m.q[h * hd]);
  if (m.k_norm[l]) for (uint32_t h = 0; h < m.n_kv; ++h) rms_norm_row(&m.k[h * hd], m.k_norm[l], hd, m.eps, &m.k[h * hd]);
  apply_rope(m.q.data(), m.n_heads, hd, hd, cosv, sinv, m.split_half);
  apply_rope(m.k.data(), m.n_kv, hd, hd, cosv, sinv, m.split_half);
  if (capture_q) std::memcpy(capture_q, m.q.data(), nq * sizeof(float));
  // kv_cache.rs:573-600 store_kv_head_row: round through f16.
  for (uint32_t h = 0; h < m.n_kv; ++h) {
    size_t dst = (((size_t)l * m.n_kv + h) * m.max_pos + pos) * hd;
    for (uint32_t d = 0; d < hd; ++d) {
      m.kc[dst + d] = f16_bits_to_f32(f32_to_f16_bits(m.k[h * hd + d]));
      m.vc[dst + d] = f16_bits_to_f32(f32_to_f16_bits(m.v[h * hd + d]));
    }
  }
  // attention (diagnostic_config.rs:300-305 scale; grouped GQA mapping head/repeats)
  const float scale = 1.0f / std::sqrt((float)hd);
  const uint32_t rep = m.n_heads / m.n_kv;
#pragma omp parallel
  {
    std::vector<float> sc;
#pragma omp for schedule(static)
    for (long h = 0; h < (long)m.n_heads; ++h)
      attention_head(m, l, (uint32_t)h / rep, &m.q[h * hd], pos + 1, scale, &m.ctx[h * hd], sc);
  }
  linear(m, m.wo[l], qt[3], H, nq, m.ctx.data(), m.tmp.data());
  for (uint32_t i = 0; i < H; ++i) m.h[i] = m.h[i] + m.tmp[i];   // pooled_add residual
  rms_norm_row(m.h.data(), m.ffn_norm[l], H, m.eps, m.xn.data());
  linear(m, m.wg[l], qt[4], m.F, H, m.xn.data(), m.g.data());
  linear(m, m.wu[l], qt[5], m.F, H, m.xn.data(), m.u.data());
  for (uint32_t i = 0; i < m.F; ++i) m.act[i] = silu_mul1(m.g[i], m.u[i]);
  linear(m, m.wd[l], qt[6], H, m.F, m.act.data(), m.tmp.data());
  for (uint32_t i = 0; i < H; ++i) m.h[i] = m.h[i] + m.tmp[i];
}

}  // namespace

// ============================================================== C ABI (ctypes)
OX uint16_t oracle_f32_to_f16(float v) { return f32_to_f16_bits(v); }
OX float oracle_f16_to_f32(uint16_t b) { return f16_bits_to_f32(b); }
OX void oracle_f32_to_f16_n(const float* x, uint16_t* out, size_t n) {
  for (size_t i = 0; i < n; ++i) out[i] = f32_to_f16_bits(x[i]);
}
OX void oracle_f16_to_f32_n(const uint16_t* x, float* out, size_t n) {
  for (size_t i = 0; i < n; ++i) out[i] = f16_bits_to_f32(x[i]);
}
OX void oracle_expf_n(const float* x, float* out, size_t n) {
#pragma omp parallel for schedule(static)
  for (long i = 0; i < (long)n; ++i) out[i] = std::exp(x[i]);
}
OX void oracle_quantize_q8_0(const float* x, size_t n, float* scales, int8_t* quants) {
  for (size_t b = 0; b < n / 32; ++b) quantize_q8_0_block(x + b * 32, &scales[b], &quants[b * 32]);
}
// Encode f32 rows to Q8_0 wire (34 B blocks: f16 LE scale + 32 i8), as a GGUF writer does.
OX void oracle_quantize_q8_0_wire(const float* x, size_t n, uint8_t* wire) {
  for (size_t b = 0; b < n / 32; ++b) {
    float s; int8_t q[32];
    quantize_q8_0_block(x + b * 32, &s, q);
    uint16_t bits = f32_to_f16_bits(s);
    wire[b * 34] = (uint8_t)(bits & 0xff);
    wire[b * 34 + 1] = (uint8_t)(bits >> 8);
    std::memcpy(wire + b * 34 + 2, q, 32);
  }
}
// tensor/mod.rs:4159-4189 Q8_0 wire decode: value = f16(d) * q.
OX void oracle_dequant_q8_0_wire(const uint8_t* wire, size_t nblocks, float* out) {
  for (size_t b = 0; b < nblocks; ++b) {
    float d = f16_bits_to_f32((uint16_t)(wire[b * 34] | (wire[b * 34 + 1] << 8)));
    for (int i = 0; i < 32; ++i) out[b * 32 + i] = d * (float)(int8_t)wire[b * 34 + 2 + i];
  }
}
OX int32_t oracle_q8_block_dot(const int8_t* w, const int8_t* x) { return q8_block_dot(w, x); }
// Per-(row, block) int32 dots of a Q8_0 wire matrix against a quantized row.
OX void oracle_q8_0_block_dots(const uint8_t* wire, size_t rows, size_t k, const int8_t* xq, int32_t* out) {
  size_t nb = k / 32;
#pragma omp parallel for schedule(static)
  for (long r = 0; r < (long)rows; ++r)
    for (size_t b = 0; b < nb; ++b)
      out[r * nb + b] = q8_block_dot((const int8_t*)(wire + (r * nb + b) * 34 + 2), xq + b * 32);
}
// Q8_0 GEMV with an already-quantized activation row (the exact linear inner loop).
OX void oracle_q8_0_gemv(const uint8_t* wire, size_t rows, size_t k, const float* xs, const int8_t* xq, float* out) {
  size_t nb = k / 32;
#pragma omp parallel for schedule(static)
  for (long r = 0; r < (long)rows; ++r) out[r] = q8_0_row_dot_wire(wire + (size_t)r * nb * 34, xs, xq, nb);
}
// Batched (prefill) form: T quantized rows.
OX void oracle_q8_0_gemm(const uint8_t* wire, size_t rows, size_t k, size_t T, const float* xs,
                         const int8_t* xq, float* out /*[T][rows]*/) {
  size_t nb = k / 32;
#pragma omp parallel for schedule(static)
  for (long r = 0; r < (long)rows; ++r)
    for (size_t t = 0; t < T; ++t)
      out[t * rows + r] = q8_0_row_dot_wire(wire + (size_t)r * nb * 34, xs + t * nb, xq + t * k, nb);
}
// K-quant kernels: Q8_K activation quantizer, wire dequantizers, row dots.
OX void oracle_quantize_q8_k(const float* x, size_t n, float* d, int8_t* qs) {
  for (size_t b = 0; b < n / 256; ++b) quantize_q8_k_block(x + 256 * b, &d[b], &qs[256 * b]);
}
OX int32_t oracle_nearest_int(float x) { return nearest_int(x); }
OX void oracle_dequant_q4_k(const uint8_t* wire, size_t nsb, float* out) {
  for (size_t b = 0; b < nsb; ++b) dequant_q4_k_block(wire + b * 144, out + b * 256);
}
OX void oracle_dequant_q6_k(const uint8_t* wire, size_t nsb, float* out) {
  for (size_t b = 0; b < nsb; ++b) dequant_q6_k_block(wire + b * 210, out + b * 256);
}
// rows x k K-quant GEMV (quant 1 Q4_K, 2 Q6_K) against a Q8_K activation row.
OX void oracle_kquant_gemv(int quant, const uint8_t* wire, size_t rows, size_t k, const float* yd, const int8_t* yqs,
                           float* out) {
  const size_t nsb = k / 256, rb = quant_row_bytes(quant, k);
#pragma omp parallel for schedule(static)
  for (long r = 0; r < (long)rows; ++r)
    out[r] = quant == Q_Q4_K ? q4_k_row_dot(wire + (size_t)r * rb, yd, yqs, nsb)
                             : q6_k_row_dot(wire + (size_t)r * rb, yd, yqs, nsb);
}
OX void oracle_rms_norm(const float* x, const float* w, size_t rows, size_t n, float eps, float* out) {
  for (size_t r = 0; r < rows; ++r) rms_norm_row(x + r * n, w, n, eps, out + r * n);
}
OX void oracle_rope_tables(uint32_t rope_dim, float freq_base, int scaling_kind, float factor, float orig_ctx,
                           float low, float high, const float* rope_freqs, uint32_t pos0, uint32_t n_pos,
                           float* cos_out, float* sin_out) {
  RopeCfg c{rope_dim, freq_base, scaling_kind, factor, orig_ctx, low, high, rope_freqs};
  rope_tables(c, pos0, n_pos, cos_out, sin_out);
}
// The per-pair frequencies theta_i (rope_pair_frequency, rope.rs:526-560) the tables are built from.
OX void oracle_rope_frequencies(uint32_t rope_dim, float freq_base, int scaling_kind, float factor, float orig_ctx,
                                float low, float high, const float* rope_freqs, float* theta_out) {
  RopeCfg c{rope_dim, freq_base, scaling_kind, factor, orig_ctx, low, high, rope_freqs};
  for (uint32_t p = 0; p < rope_dim / 2; ++p) theta_out[p] = rope_pair_frequency(p, c);
}
OX void oracle_apply_rope(float* data, uint32_t heads, uint32_t hd, uint32_t rope_dim, const float* cosv,
                          const float* sinv, int split_half) {
  apply_rope(data, heads, hd, rope_dim, cosv, sinv, split_half);
}
OX void oracle_silu_mul(const float* g, const float* u, size_t n, float* out) {
  for (size_t i = 0; i < n; ++i) out[i] = silu_mul1(g[i], u[i]);
}
// inference.rs:5912-5925 greedy_sample: first index of the max, strict '>'.
OX uint32_t oracle_argmax(const float* x, size_t n) {
  size_t best = 0;
  float bv = -INFINITY;
  for (size_t i = 0; i < n; ++i) if (x[i] > bv) { best = i; bv = x[i]; }
  return (uint32_t)best;
}
// Attention for one query row against an f32 KV slab [n_kv][max_pos][hd] (f16-rounded values).
OX void oracle_attention(const float* q, const float* kc, const float* vc, uint32_t n_heads, uint32_t n_kv,
                         uint32_t hd, uint32_t max_pos, uint32_t n_pos, float* out) {
  Model m{};
  m.n_kv = n_kv; m.hd = hd; m.max_pos = max_pos;
  m.kc.assign(kc, kc + (size_t)n_kv * max_pos * hd);
  m.vc.assign(vc, vc + (size_t)n_kv * max_pos * hd);
  std::vector<float> sc;
  const float scale = 1.0f / std::sqrt((float)hd);
  uint32_t rep = n_heads / n_kv;
  for (uint32_t h = 0; h < n_heads; ++h) attention_head(m, 0, h / rep, q + (size_t)h * hd, n_pos, scale, out + (size_t)h * hd, sc);
}

// ---- model
OX void* oracle_model_new(uint32_t L, uint32_t n_heads, uint32_t n_kv, uint32_t hd, uint32_t H, uint32_t F,
                          uint32_t V, uint32_t max_pos, float eps, int split_half) {
  Model* m = new Model();
  m->L = L; m->n_heads = n_heads; m->n_kv = n_kv; m->hd = hd; m->H = H; m->F = F; m->V = V;
  m->max_pos = max_pos; m->eps = eps; m->split_half = split_half;
  m->qt.assign((size_t)L * 7, (uint8_t)Q_Q8_0);
  m->wq.assign(L, nullptr); m->wk = m->wq; m->wv = m->wq; m->wo = m->wq; m->wg = m->wq; m->wu = m->wq; m->wd = m->wq;
  m->attn_norm.assign(L, nullptr); m->ffn_norm = m->attn_norm; m->q_norm = m->attn_norm; m->k_norm = m->attn_norm;
  m->kc.assign((size_t)L * n_kv * max_pos * hd, 0.0f);
  m->vc.assign((size_t)L * n_kv * max_pos * hd, 0.0f);
  m->h.assign(H, 0); m->xn.assign(H, 0); m->q.assign((size_t)n_heads * hd, 0); m->k.assign((size_t)n_kv * hd, 0);
  m->v = m->k; m->ctx = m->q; m->tmp.assign(H, 0); m->g.assign(F, 0); m->u = m->g; m->act = m->g;
  m->logits.assign(V, 0);
  return m;
}
OX void oracle_model_free(void* p) { delete (Model*)p; }
OX void oracle_model_set_layer(void* p, uint32_t l, const uint8_t* wq, const uint8_t* wk, const uint8_t* wv,
                               const uint8_t* wo, const uint8_t* wg, const uint8_t* wu, const uint8_t* wd,
                               const float* attn_norm, const float* ffn_norm, const float* q_norm,
                               const float* k_norm) {
  Model* m = (Model*)p;
  m->wq[l] = wq; m->wk[l] = wk; m->wv[l] = wv; m->wo[l] = wo; m->wg[l] = wg; m->wu[l] = wu; m->wd[l] = wd;
  m->attn_norm[l] = attn_norm; m->ffn_norm[l] = ffn_norm; m->q_norm[l] = q_norm; m->k_norm[l] = k_norm;
}
OX void oracle_model_set_output(void* p, const float* out_norm, const uint8_t* out_w, const uint8_t* embd) {
  Model* m = (Model*)p;
  m->out_norm = out_norm; m->out_w = out_w; m->embd = embd;
}
// Formats of one layer's seven projections (q, k, v, o, gate, up, down), of the output
// projection and of the token embedding (0 Q8_0, 1 Q4_K, 2 Q6_K).
OX void oracle_model_set_quant(void* p, uint32_t l, const uint8_t* quant7) {
  Model* m = (Model*)p;
  std::memcpy(&m->qt[(size_t)l * 7], quant7, 7);
}
OX void oracle_model_set_output_quant(void* p, int out_quant, int embd_quant) {
  Model* m = (Model*)p;
  m->out_quant = out_quant;
  m->embd_quant = embd_quant;
}
// Embedding row (tensor/mod.rs:2329-2398 Q8_0: scale * q, exact; K-quant rows through the
// block dequantizers).
OX void oracle_model_embed(void* p, uint32_t token, float* out) {
  Model* m = (Model*)p;
  const size_t rb = quant_row_bytes(m->embd_quant, m->H);
  const uint8_t* row = m->embd + (size_t)token * rb;
  if (m->embd_quant == Q_Q8_0) {
    oracle_dequant_q8_0_wire(row, m->H / 32, out);
  } else {
    for (size_t sb = 0; sb < m->H / 256; ++sb) {
      if (m->embd_quant == Q_Q4_K) dequant_q4_k_block(row + sb * 144, out + sb * 256);
      else dequant_q6_k_block(row + sb * 210, out + sb * 256);
    }
  }
}
// One forward step at `pos` from an embedding row.  Optional captures:
//   hidden_out [L+1][H]: the residual stream entering each layer and after the last;
//   logits_out [V]: the output projection (computed only when logits_out or tok_out is set).
// Returns 0, or -1 when pos is out of range.
OX int oracle_model_forward(void* p, const float* emb, uint32_t pos, const float* cosv, const float* sinv,
                            float* hidden_out, float* logits_out, uint32_t* tok_out) {
  Model* m = (Model*)p;
  if (pos >= m->max_pos) return -1;
  std::memcpy(m->h.data(), emb, m->H * sizeof(float));
  for (uint32_t l = 0; l < m->L; ++l) {
    if (hidden_out) std::memcpy(hidden_out + (size_t)l * m->H, m->h.data(), m->H * sizeof(float));
    forward_layer(*m, l, pos, cosv, sinv, nullptr);
  }
  if (hidden_out) std::memcpy(hidden_out + (size_t)m->L * m->H, m->h.data(), m->H * sizeof(float));
  if (logits_out || tok_out) {
    rms_norm_row(m->h.data(), m->out_norm, m->H, m->eps, m->xn.data());
    linear(*m, m->out_w, m->out_quant, m->V, m->H, m->xn.data(), m->logits.data());
    if (logits_out) std::memcpy(logits_out, m->logits.data(), m->V * sizeof(float));
    if (tok_out) *tok_out = oracle_argmax(m->logits.data(), m->V);
  }
  return 0;
}
// Copy out the KV rows of one layer for positions [0, n): [n_kv][n][hd].
OX void oracle_model_read_kv(void* p, uint32_t l, uint32_t n, float* k_out, float* v_out) {
  Model* m = (Model*)p;
  for (uint32_t h = 0; h < m->n_kv; ++h)
    for (uint32_t t = 0; t < n; ++t) {
      size_t src = (((size_t)l * m->n_kv + h) * m->max_pos + t) * m->hd;
      size_t dst = ((size_t)h * n + t) * m->hd;
      std::memcpy(k_out + dst, &m->kc[src], m->hd * sizeof(float));
      std::memcpy(v_out + dst, &m->vc[src], m->hd * sizeof(float));
    }
}

// Seed one layer's KV for positions [0, n) from [n_kv][n][hd] f32 (rounded through f16, as
// kv_cache.rs:573-600 stores every row).
OX void oracle_model_seed_kv(void* p, uint32_t l, uint32_t n, const float* k_in, const float* v_in) {
  Model* m = (Model*)p;
  for (uint32_t h = 0; h < m->n_kv; ++h)
    for (uint32_t t = 0; t < n; ++t) {
      size_t dst = (((size_t)l * m->n_kv + h) * m->max_pos + t) * m->hd;
      size_t src = ((size_t)h * n + t) * m->hd;
      for (uint32_t d = 0; d < m->hd; ++d) {
        m->kc[dst + d] = f16_bits_to_f32(f32_to_f16_bits(k_in[src + d]));
        m->vc[dst + d] = f16_bits_to_f32(f32_to_f16_bits(v_in[src + d]));
      }
    }
}

// Sequential f32 fold of each row, sum = 0; sum += x[i] (the `.sum::<f32>()` order of
// tensor/mod.rs:2083-2106 and the softmax denominator of inference.rs:23990-23994).
OX void oracle_serial_sum_rows(const float* x, size_t rows, size_t n, float* out) {
  for (size_t r = 0; r < rows; ++r) {
    float acc = 0.0f;
    for (size_t i = 0; i < n; ++i) acc += x[r * n + i];
    out[r] = acc;
  }
}

// OpenMP threads of the row-parallel loops (the baseline timing runs at several counts;
// the results do not depend on it: every output row is computed by one thread).
OX void oracle_set_threads(int n) { omp_set_num_threads(n > 0 ? n : 1); }
