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

// n token ids uniform in [0, vocab) from `seed`.
CX void camelid_synth_tokens(uint64_t seed, uint32_t vocab, uint32_t n, uint32_t* out) {
  for (uint32_t i = 0; i < n; ++i) out[i] = (uint32_t)(splitmix(seed + (uint64_t)(i + 1) * 0x9E3779B97F4A7C15ull) % vocab);
}
