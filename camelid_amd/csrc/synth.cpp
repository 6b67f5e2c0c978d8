// synth.cpp -- seeded synthetic GGUF-style weights for the benchmark configurations.
//
// Generator (portable, counter-based so it splits across threads):
//   stream seed  s = seed XOR fnv1a64(tensor name)
//   uniform u_i  = (splitmix64(s + (i+1)*0x9E3779B97F4A7C15) >> 11) * 2^-53      in [0, 1)
//   normal pair  (z_2j, z_2j+1) = sqrt(-2 ln(1-u_2j)) * (cos, sin)(2*pi*u_2j+1)  (Box-Muller, binary64)
//   value        = (float)(std * z)
// Q8_0 tensors are quantized per 32-block exactly as Camelid quantizes (fp16 scale =
// amax/127, round half away from zero) and written as 34-byte GGUF wire blocks.
#include <cmath>
#include <cstdint>
#include <cstring>
#include <thread>
#include <vector>
#include <algorithm>

#include "device_math.h"

#define CX extern "C" __attribute__((visibility("default")))

namespace {

uint64_t fnv1a64(const char* s) {
  uint64_t h = 0xcbf29ce484222325ull;
  for (; *s; ++s) {
    h ^= (uint8_t)*s;
    h *= 0x100000001b3ull;
  }
  return h;
}

inline uint64_t splitmix(uint64_t x) {
  x = (x ^ (x >> 30)) * 0xbf58476d1ce4e5b9ull;
  x = (x ^ (x >> 27)) * 0x94d049bb133111ebull;
  return x ^ (x >> 31);
}

inline double uniform(uint64_t s, uint64_t i) {
  return (double)(splitmix(s + (i + 1) * 0x9E3779B97F4A7C15ull) >> 11) * 0x1.0p-53;
}

// Values [i0, i1) of the stream (i0 even).
void normals(uint64_t s, double stdv, uint64_t i0, uint64_t i1, float* out) {
  const double two_pi = 6.283185307179586476925286766559;
  for (uint64_t i = i0; i < i1; i += 2) {
    const double u1 = 1.0 - uniform(s, i);
    const double u2 = uniform(s, i + 1);
    const double r = std::sqrt(-2.0 * std::log(u1));
    const double th = two_pi * u2;
    out[i - i0] = (float)(stdv * (r * std::cos(th)));
    if (i + 1 < i1) out[i + 1 - i0] = (float)(stdv * (r * std::sin(th)));
  }
}

template <typename F>
void parallel_chunks(uint64_t n, uint64_t align, F fn) {
  unsigned nt = std::max(1u, std::min(16u, std::thread::hardware_concurrency()));
  if (n < (1u << 16)) nt = 1;
  std::vector<std::thread> th;
  for (unsigned t = 0; t < nt; ++t) {
    uint64_t a = (n * t / nt) / align * align;
    uint64_t b = t + 1 == nt ? n : (n * (t + 1) / nt) / align * align;
    if (b > a) th.emplace_back(fn, a, b);
  }
  for (auto& x : th) x.join();
}

}  // namespace

// n values of N(0, std^2) for tensor `name`.
CX void camelid_synth_normal_f32(const char* name, uint64_t seed, float stdv, float* out, uint64_t n) {
  const uint64_t s = seed ^ fnv1a64(name);
  parallel_chunks(n, 2, [&](uint64_t a, uint64_t b) { normals(s, stdv, a, b, out + a); });
}

// n (multiple of 32) values of N(0, std^2) for tensor `name`, quantized to Q8_0 wire blocks.
CX int camelid_synth_q8_0_wire(const char* name, uint64_t seed, float stdv, uint64_t n, uint8_t* out) {
  if (n % 32) return 1;
  const uint64_t s = seed ^ fnv1a64(name);
  parallel_chunks(n, 32, [&](uint64_t a, uint64_t b) {
    float v[32];
    int8_t q[32];
    for (uint64_t i = a; i < b; i += 32) {
      normals(s, stdv, i, i + 32, v);
      const float d = cm::quantize_q8_0_block(v, q);
      const uint16_t bits = cm::f32_to_f16_bits(d);
      uint8_t* blk = out + (i / 32) * 34;
      blk[0] = (uint8_t)(bits & 0xff);
      blk[1] = (uint8_t)(bits >> 8);
      std::memcpy(blk + 2, q, 32);
    }
  });
  return 0;
}

namespace {

inline void put_f16(uint8_t* p, float v) {
  const uint16_t b = cm::f32_to_f16_bits(v);
  p[0] = (uint8_t)(b & 0xff);
  p[1] = (uint8_t)(b >> 8);
}
inline float f16r(float v) { return cm::f16_bits_to_f32(cm::f32_to_f16_bits(v)); }

// A GGUF Q4_K superblock (144 bytes) for 256 values: per 32-value sub-block an affine
// 4-bit code (x ~ d*sc*q - dmin*m), 6-bit sub-block scales/mins under f16 d/dmin, packed
// with the layout tensor/mod.rs:4776-4785 decodes.  (A plain min/max fit, not llama.cpp's
// search: any valid superblock serves as synthetic weights.)
void encode_q4_k(const float* x, uint8_t* out) {
  float sc_r[8], mn_r[8];
  float max_sc = 0.0f, max_mn = 0.0f;
  for (int g = 0; g < 8; ++g) {
    float lo = x[32 * g], hi = x[32 * g];
    for (int i = 1; i < 32; ++i) {
      lo = std::min(lo, x[32 * g + i]);
      hi = std::max(hi, x[32 * g + i]);
    }
    lo = std::min(lo, 0.0f);
    sc_r[g] = (hi - lo) / 15.0f;
    mn_r[g] = -lo;
    max_sc = std::max(max_sc, sc_r[g]);
    max_mn = std::max(max_mn, mn_r[g]);
  }
  const float d = f16r(max_sc / 63.0f), dmin = f16r(max_mn / 63.0f);
  uint8_t sc[8], mn[8];
  for (int g = 0; g < 8; ++g) {
    sc[g] = d > 0.0f ? (uint8_t)std::min(63.0f, std::nearbyint(sc_r[g] / d)) : 0;
    mn[g] = dmin > 0.0f ? (uint8_t)std::min(63.0f, std::nearbyint(mn_r[g] / dmin)) : 0;
  }
  put_f16(out, d);
  put_f16(out + 2, dmin);
  uint8_t* s = out + 4;
  for (int i = 0; i < 4; ++i) {
    s[i] = (uint8_t)((sc[i] & 63) | ((sc[i + 4] >> 4) << 6));
    s[i + 4] = (uint8_t)((mn[i] & 63) | ((mn[i + 4] >> 4) << 6));
    s[i + 8] = (uint8_t)((sc[i + 4] & 15) | ((mn[i + 4] & 15) << 4));
  }
  uint8_t q[256];
  for (int g = 0; g < 8; ++g) {
    const float rs = d * (float)sc[g], rm = dmin * (float)mn[g];
    for (int i = 0; i < 32; ++i) {
      const float v = rs > 0.0f ? std::nearbyint((x[32 * g + i] + rm) / rs) : 0.0f;
      q[32 * g + i] = (uint8_t)std::min(15.0f, std::max(0.0f, v));
    }
  }
  for (int pair = 0; pair < 4; ++pair)
    for (int l = 0; l < 32; ++l) out[16 + 32 * pair + l] = (uint8_t)(q[64 * pair + l] | (q[64 * pair + 32 + l] << 4));
}

// A GGUF Q6_K superblock (210 bytes: ql[128], qh[64], i8 scales[16], f16 d) for 256 values:
// per 16-value group a symmetric 6-bit code (x ~ d*sc*q, q in [-32, 31]), stored with the
// layout inference.rs:19201-19232 decodes.
void encode_q6_k(const float* x, uint8_t* out) {
  float gs[16], max_s = 0.0f;
  for (int g = 0; g < 16; ++g) {
    float a = 0.0f;
    for (int i = 0; i < 16; ++i) a = std::max(a, std::fabs(x[16 * g + i]));
    gs[g] = a / 31.0f;
    max_s = std::max(max_s, gs[g]);
  }
  const float d = f16r(max_s / 127.0f);
  int8_t sc[16];
  for (int g = 0; g < 16; ++g)
    sc[g] = d > 0.0f ? (int8_t)std::min(127.0f, std::max(-128.0f, std::nearbyint(gs[g] / d))) : 0;
  std::memset(out, 0, 210);
  for (int p = 0; p < 256; ++p) {
    const float r = d * (float)sc[p / 16];
    const float v = r > 0.0f ? std::nearbyint(x[p] / r) : 0.0f;
    const int q = (int)std::min(31.0f, std::max(-32.0f, v)) + 32;
    const int n = p / 128, k = (p % 128) / 32, l = p % 32;
    uint8_t& lq = out[n * 64 + (k & 1) * 32 + l];
    lq |= (uint8_t)((q & 15) << (k < 2 ? 0 : 4));
    out[128 + n * 32 + l] |= (uint8_t)((q >> 4) << (2 * k));
  }
  for (int g = 0; g < 16; ++g) out[192 + g] = (uint8_t)sc[g];
  put_f16(out + 208, d);
}

}  // namespace

// n (multiple of 256) values of N(0, std^2) for tensor `name`, as Q4_K (quant 1, 144-byte
// superblocks) or Q6_K (quant 2, 210-byte superblocks) wire bytes.
CX int camelid_synth_kquant_wire(const char* name, uint64_t seed, float stdv, uint64_t n, int quant, uint8_t* out) {
  if (n % 256 || (quant != 1 && quant != 2)) return 1;
  const uint64_t s = seed ^ fnv1a64(name);
  const size_t bytes = quant == 1 ? 144 : 210;
  parallel_chunks(n, 256, [&](uint64_t a, uint64_t b) {
    float v[256];
    for (uint64_t i = a; i < b; i += 256) {
      normals(s, stdv, i, i + 256, v);
      if (quant == 1) encode_q4_k(v, out + (i / 256) * bytes);
      else encode_q6_k(v, out + (i / 256) * bytes);
    }
  });
  return 0;
}

// n token ids uniform in [0, vocab) from `seed`.
CX void camelid_synth_tokens(uint64_t seed, uint32_t vocab, uint32_t n, uint32_t* out) {
  for (uint32_t i = 0; i < n; ++i) out[i] = (uint32_t)(splitmix(seed + (uint64_t)(i + 1) * 0x9E3779B97F4A7C15ull) % vocab);
}
