// seam.cpp -- host-side half of the resident seam (the inference.rs side of the
// engine boundary): per-position RoPE cos/sin tables and the Q8_0 embedding row
// lookup that the caller hands to forward_token/prefill.  Compiled with
// -ffp-contract=off against glibc libm, as Rust's f32::{powf,sin,cos} resolve.
#include <cmath>
#include <cstdint>
#include <cstring>
#include <vector>

#include "device_math.h"

#define CX extern "C" __attribute__((visibility("default")))

namespace {

struct Rope {
  uint32_t rope_dim;
  float base;
  int kind;  // 0 none, 1 linear, 2 llama3
  float factor, orig_ctx, low, high;
  const float* freqs;
};

// rope.rs:687-711 llama3_scaled_rope_frequency.
float llama3(float f, const Rope& r) {
  const float two_pi = 2.0f * 3.14159265358979323846f;
  const float wavelength = two_pi / f;
  const float low_wl = r.orig_ctx / r.low;
  const float high_wl = r.orig_ctx / r.high;
  if (wavelength < high_wl) return f;
  if (wavelength > low_wl) return f / r.factor;
  const float smooth = (r.orig_ctx / wavelength - r.low) / (r.high - r.low);
  return ((1.0f - smooth) * f / r.factor) + (smooth * f);
}

// rope.rs:526-560 rope_pair_frequency.
float pair_frequency(uint32_t i, const Rope& r) {
  float f = std::pow(r.base, -((float)i * 2.0f) / (float)r.rope_dim);
  if (r.freqs) f = f / r.freqs[i];
  if (r.kind == 1) return f / r.factor;
  if (r.kind == 2) return llama3(f, r);
  return f;
}

}  // namespace

// rope.rs:568-627 resident_decode_rope_tables / :629-685 resident_prefill_rope_tables:
// cos/sin [n_pos][rope_dim/2] for positions pos0 .. pos0+n_pos-1 (zero-based positions,
// magnitude scale 1 for none/linear/llama3).  Returns 0, or 1 on invalid metadata.
CX int camelid_rope_tables(uint32_t rope_dim, float freq_base, int scaling_kind, float factor, float orig_ctx,
                           float low, float high, const float* rope_freqs, uint32_t pos0, uint32_t n_pos,
                           float* cos_out, float* sin_out) {
  if (rope_dim == 0 || rope_dim % 2 || !(freq_base > 0.0f) || !std::isfinite(freq_base)) return 1;
  if (scaling_kind < 0 || scaling_kind > 2 || !(factor > 0.0f)) return 1;
  if (scaling_kind == 2 && !(orig_ctx > 0.0f && low > 0.0f && high > low)) return 1;
  const Rope r{rope_dim, freq_base, scaling_kind, factor, orig_ctx, low, high, rope_freqs};
  const uint32_t half = rope_dim / 2;
  std::vector<float> f(half);
  for (uint32_t i = 0; i < half; ++i) f[i] = pair_frequency(i, r);
  for (uint32_t t = 0; t < n_pos; ++t) {
    const float pos = (float)(pos0 + t);
    for (uint32_t i = 0; i < half; ++i) {
      const float a = pos * f[i];
      cos_out[(size_t)t * half + i] = std::cos(a);
      sin_out[(size_t)t * half + i] = std::sin(a);
    }
  }
  return 0;
}

// tensor/mod.rs:2329-2398 Q8_0 embedding rows from wire bytes: value = f16(d) * q (exact).
CX int camelid_embed_q8_0(const uint8_t* wire, uint32_t vocab, uint32_t hidden, const uint32_t* tokens, uint32_t n,
                          float* out) {
  if (hidden % 32) return 1;
  const size_t nb = hidden / 32;
  for (uint32_t t = 0; t < n; ++t) {
    if (tokens[t] >= vocab) return 1;
    const uint8_t* row = wire + (size_t)tokens[t] * nb * 34;
    for (size_t b = 0; b < nb; ++b) {
      const float d = cm::f16_bits_to_f32((uint16_t)(row[b * 34] | (row[b * 34 + 1] << 8)));
      for (int i = 0; i < 32; ++i) out[(size_t)t * hidden + b * 32 + i] = d * (float)(int8_t)row[b * 34 + 2 + i];
    }
  }
  return 0;
}

// K-quant embedding rows (the block dequantizers: tensor/mod.rs:4682-4703 Q4_K,
// (d*sc)*q - dmin*m; :4818-4845 Q6_K, (d*sc)*q).  quant 1 = Q4_K, 2 = Q6_K.
CX int camelid_embed_kquant(int quant, const uint8_t* wire, uint32_t vocab, uint32_t hidden, const uint32_t* tokens,
                            uint32_t n, float* out) {
  if (hidden % 256 || (quant != 1 && quant != 2)) return 1;
  const size_t nsb = hidden / 256, bb = quant == 1 ? 144 : 210;
  for (uint32_t t = 0; t < n; ++t) {
    if (tokens[t] >= vocab) return 1;
    for (size_t s = 0; s < nsb; ++s) {
      const uint8_t* b = wire + ((size_t)tokens[t] * nsb + s) * bb;
      float* o = out + (size_t)t * hidden + s * 256;
      if (quant == 1) {
        const float d = cm::f16_bits_to_f32((uint16_t)(b[0] | (b[1] << 8)));
        const float dmin = cm::f16_bits_to_f32((uint16_t)(b[2] | (b[3] << 8)));
        const uint8_t* sc = b + 4;
        for (int idx = 0; idx < 8; ++idx) {
          int scale, mn;
          if (idx < 4) {
            scale = sc[idx] & 63;
            mn = sc[idx + 4] & 63;
          } else {
            scale = (sc[idx + 4] & 0x0f) | ((sc[idx - 4] >> 6) << 4);
            mn = (sc[idx + 4] >> 4) | ((sc[idx] >> 6) << 4);
          }
          const float ds = d * (float)scale, dm = dmin * (float)mn;
          const int pair = idx / 2, hi = idx % 2;
          for (int l = 0; l < 32; ++l) {
            const uint8_t byte = b[16 + pair * 32 + l];
            o[pair * 64 + hi * 32 + l] = ds * (float)(hi ? (byte >> 4) : (byte & 0x0f)) - dm;
          }
        }
      } else {
        const float d = cm::f16_bits_to_f32((uint16_t)(b[208] | (b[209] << 8)));
        for (int p = 0; p < 256; ++p) {
          const int nn = p / 128, k = (p % 128) / 32, l = p % 32;
          const uint8_t lq = b[nn * 64 + (k & 1) * 32 + l];
          const int lo = k < 2 ? (lq & 0x0f) : (lq >> 4);
          const int q = (lo | (((b[128 + nn * 32 + l] >> (2 * k)) & 3) << 4)) - 32;
          o[p] = d * (float)(int8_t)b[192 + p / 16] * (float)q;
        }
      }
    }
  }
  return 0;
}
