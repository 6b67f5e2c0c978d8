// gguf.cpp -- read-only memory map of a GGUF model file, its metadata and tensor directory,
// and the loader that hands the mapped weight bytes to the resident engine (host C++).
//
// The parse follows Camelid's reader (src/gguf/reader.rs:346-470 read_metadata_with_len):
// magic "GGUF", version 2 or 3, i64 tensor and metadata counts, typed metadata values
// (nested arrays refused, strings <= 16 MiB, arrays <= 1e6 elements), general.alignment
// (default 32, a power of two), tensor infos (name < 64 bytes, 1-4 dims, GGML type id, offset),
// data start = header end aligned up, offsets contiguous at the alignment, every tensor's byte
// range inside the file.  The mapping is read-only and shared (src/wire_mmap.rs:78-130
// GgufWireMmap::map), so the engine reads the weights straight from the page cache: no host
// copy of the model is made before the upload.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <cmath>
#include <cstring>
#include <map>
#include <string>
#include <vector>

#include "../../include/camelid_gguf.h"

#define CX extern "C" __attribute__((visibility("default")))

namespace {

thread_local std::string g_err;

int gfail(const std::string& m) {
  g_err = m;
  return 1;
}

// IEEE binary16 -> binary32 (exact; subnormal halves normalised), and bfloat16 (the top half
// of a binary32).
float camelid_f16_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1fu, man = h & 0x3ffu, bits;
  if (exp == 0x1fu) {
    bits = sign | 0x7f800000u | (man << 13);
  } else if (exp != 0) {
    bits = sign | ((exp + 112u) << 23) | (man << 13);
  } else if (man == 0) {
    bits = sign;
  } else {
    int e = 113;
    while (!(man & 0x400u)) { man <<= 1; --e; }
    bits = sign | ((uint32_t)e << 23) | ((man & 0x3ffu) << 13);
  }
  float f;
  std::memcpy(&f, &bits, 4);
  return f;
}

float bf16_to_f32(uint16_t b) {
  const uint32_t bits = (uint32_t)b << 16;
  float f;
  std::memcpy(&f, &bits, 4);
  return f;
}

// GGML type id -> (values per block, bytes per block) (reader.rs:101-133).
bool ggml_layout(int32_t t, uint64_t* bs, uint64_t* ts) {
  struct L {
    int32_t id;
    uint64_t b, s;
  };
  static const L tab[] = {{0, 1, 4},      {1, 1, 2},      {2, 32, 18},    {3, 32, 20},   {6, 32, 22},
                          {7, 32, 22},    {8, 32, 34},    {9, 32, 36},    {10, 256, 84}, {11, 256, 110},
                          {12, 256, 144}, {13, 256, 176}, {14, 256, 210}, {15, 256, 292}, {20, 32, 18},
                          {23, 256, 136}, {34, 256, 54},  {35, 256, 66},  {40, 64, 36},  {24, 1, 1},
                          {25, 1, 2},     {30, 1, 2},     {26, 1, 4},     {27, 1, 8},    {28, 1, 8}};
  for (const L& l : tab)
    if (l.id == t) {
      *bs = l.b;
      *ts = l.s;
      return true;
    }
  return false;
}

struct Meta {
  int32_t type = -1;  // GGUF value type; 9 = array
  uint64_t u = 0;     // unsigned integers and bools
  int64_t i = 0;      // signed integers
  double f = 0.0;     // floats
  std::string s;
  int32_t elem = -1;  // array element type
  uint64_t count = 0;
};

struct Cursor {
  const uint8_t* p;
  uint64_t len, pos = 0;
  bool ok = true;
  bool take(void* out, uint64_t n) {
    if (!ok || n > len - pos) {
      ok = false;
      return false;
    }
    std::memcpy(out, p + pos, n);
    pos += n;
    return true;
  }
  template <typename T>
  T get() {
    T v{};
    take(&v, sizeof(T));
    return v;
  }
  bool str(std::string* out) {
    const uint64_t n = get<uint64_t>();
    if (!ok) return false;
    if (n > 16u * 1024 * 1024) return false;
    if (n > len - pos) {
      ok = false;
      return false;
    }
    out->assign(reinterpret_cast<const char*>(p + pos), n);
    pos += n;
    return true;
  }
};

uint64_t align_up(uint64_t v, uint64_t a) { return (v + a - 1) & ~(a - 1); }

}  // namespace

struct camelid_gguf {
  int fd = -1;
  const uint8_t* base = nullptr;
  uint64_t len = 0;
  uint32_t version = 0;
  uint64_t alignment = 32, data_start = 0;
  std::map<std::string, Meta> meta;
  std::vector<std::string> names;
  std::map<std::string, camelid_gguf_tensor> tensors;
  // rope_freqs.weight widened to f32 when the file stores it as F16 or BF16; the pointer that
  // camelid_gguf_model hands out stays valid until camelid_gguf_close
  mutable std::vector<float> rope_freqs_f32;
};

namespace {

// One metadata value of type ty (reader.rs:484-536 read_value_of_type).
bool read_value(Cursor& c, int32_t ty, Meta* m, std::string* why) {
  m->type = ty;
  switch (ty) {
    case 0: m->u = c.get<uint8_t>(); break;
    case 1: m->i = c.get<int8_t>(); break;
    case 2: m->u = c.get<uint16_t>(); break;
    case 3: m->i = c.get<int16_t>(); break;
    case 4: m->u = c.get<uint32_t>(); break;
    case 5: m->i = c.get<int32_t>(); break;
    case 6: m->f = c.get<float>(); break;
    case 7: m->u = c.get<uint8_t>() != 0; break;
    case 8:
      if (!c.str(&m->s)) {
        *why = c.ok ? "string too large" : "unexpected end of file";
        return false;
      }
      break;
    case 9: {
      const int32_t et = c.get<int32_t>();
      if (et == 9) {
        *why = "nested metadata arrays are not supported";
        return false;
      }
      const uint64_t n = c.get<uint64_t>();
      if (!c.ok) break;
      if (n > 1000000) {
        *why = "metadata array too large: " + std::to_string(n);
        return false;
      }
      m->elem = et;
      m->count = n;
      Meta e;
      for (uint64_t k = 0; k < n; ++k)
        if (!read_value(c, et, &e, why)) return false;
      break;
    }
    case 10: m->u = c.get<uint64_t>(); break;
    case 11: m->i = c.get<int64_t>(); break;
    case 12: m->f = c.get<double>(); break;
    default:
      *why = "unsupported metadata value type " + std::to_string(ty);
      return false;
  }
  if (!c.ok) {
    *why = "unexpected end of file";
    return false;
  }
  return true;
}

// Parse the header of a mapped file into g (reader.rs:346-470).
bool parse(camelid_gguf* g, std::string* why) {
  Cursor c{g->base, g->len};
  char magic[4];
  if (!c.take(magic, 4) || std::memcmp(magic, "GGUF", 4) != 0) {
    *why = "bad magic; expected GGUF";
    return false;
  }
  g->version = c.get<uint32_t>();
  if (!c.ok || g->version < 2 || g->version > 3) {
    *why = "version " + std::to_string(g->version) + "; expected v2 or v3";
    return false;
  }
  const int64_t n_tensors = c.get<int64_t>(), n_meta = c.get<int64_t>();
  if (!c.ok || n_tensors < 0 || n_meta < 0) {
    *why = c.ok ? "negative tensor or metadata count" : "unexpected end of file";
    return false;
  }
  for (int64_t k = 0; k < n_meta; ++k) {
    std::string key;
    if (!c.str(&key)) {
      *why = c.ok ? "string too large" : "unexpected end of file";
      return false;
    }
    Meta m;
    if (!read_value(c, c.get<int32_t>(), &m, why)) return false;
    if (!g->meta.emplace(key, m).second) {
      *why = "duplicate metadata key " + key;
      return false;
    }
  }
  auto al = g->meta.find("general.alignment");
  if (al != g->meta.end()) {
    if (al->second.type != 4 && al->second.type != 10) {
      *why = "general.alignment has non-integer type";
      return false;
    }
    g->alignment = al->second.u;
  }
  if (g->alignment == 0 || (g->alignment & (g->alignment - 1))) {
    *why = "invalid alignment " + std::to_string(g->alignment);
    return false;
  }
  struct Raw {
    std::string name;
    std::vector<uint64_t> dims;
    int32_t type;
    uint64_t off;
  };
  std::vector<Raw> raw;
  for (int64_t k = 0; k < n_tensors; ++k) {
    Raw r;
    if (!c.str(&r.name)) {
      *why = c.ok ? "string too large" : "unexpected end of file";
      return false;
    }
    if (r.name.size() >= 64) {
      *why = "tensor name " + r.name + " exceeds GGML_MAX_NAME";
      return false;
    }
    const uint32_t nd = c.get<uint32_t>();
    if (c.ok && (nd == 0 || nd > 4)) {
      *why = "tensor " + r.name + " has invalid dimension count " + std::to_string(nd);
      return false;
    }
    for (uint32_t d = 0; c.ok && d < nd; ++d) {
      const int64_t v = c.get<int64_t>();
      if (v < 0) {
        *why = "tensor " + r.name + " has negative dimension";
        return false;
      }
      r.dims.push_back((uint64_t)v);
    }
    r.type = c.get<int32_t>();
    r.off = c.get<uint64_t>();
    if (!c.ok) {
      *why = "unexpected end of file";
      return false;
    }
    raw.push_back(std::move(r));
  }
  g->data_start = align_up(c.pos, g->alignment);
  if (g->data_start > g->len) {
    *why = "aligned tensor data start is beyond end of file";
    return false;
  }
  uint64_t expected = 0;
  for (const Raw& r : raw) {
    if (g->tensors.count(r.name)) {
      *why = "duplicate tensor name " + r.name;
      return false;
    }
    if (r.off != expected) {
      *why = "tensor " + r.name + " offset " + std::to_string(r.off) + " is not contiguous; expected " +
             std::to_string(expected);
      return false;
    }
    uint64_t bs = 0, ts = 0;
    if (!ggml_layout(r.type, &bs, &ts)) {
      *why = "tensor " + r.name + " has unknown GGML type " + std::to_string(r.type);
      return false;
    }
    if (r.dims[0] % bs) {
      *why = "tensor " + r.name + " first dimension " + std::to_string(r.dims[0]) +
             " is not divisible by block size " + std::to_string(bs);
      return false;
    }
    // element count with a per-dimension overflow check past 2^64 (reader.rs:553-557 checked_mul)
    unsigned __int128 elems = 1;
    bool overflow = false;
    for (uint64_t d : r.dims) {
      elems *= d;
      if (elems >> 64) {
        overflow = true;
        break;
      }
    }
    if (overflow) {
      *why = "tensor " + r.name + " element count overflows";
      return false;
    }
    const unsigned __int128 nb = elems / bs * ts;
    const unsigned __int128 end = (unsigned __int128)g->data_start + r.off + nb;
    if (nb >> 64 || end > g->len) {
      *why = "tensor " + r.name + " data extends beyond end of file";
      return false;
    }
    camelid_gguf_tensor t{};
    t.data = g->base + g->data_start + r.off;
    t.n_bytes = (uint64_t)nb;
    t.offset = g->data_start + r.off;
    t.n_dims = (uint32_t)r.dims.size();
    for (uint32_t d = 0; d < 4; ++d) t.dims[d] = d < t.n_dims ? r.dims[d] : 1;
    t.type = r.type;
    g->tensors.emplace(r.name, t);
    g->names.push_back(r.name);
    expected = align_up(r.off + (uint64_t)nb, g->alignment);
  }
  return true;
}

const Meta* find_meta(const camelid_gguf* g, const std::string& key) {
  auto it = g->meta.find(key);
  return it == g->meta.end() ? nullptr : &it->second;
}

// metadata_u32 (reader.rs:182-188): u32, or a u64 that fits.
bool meta_u32(const camelid_gguf* g, const std::string& key, uint32_t* out) {
  const Meta* m = find_meta(g, key);
  if (!m || (m->type != 4 && m->type != 10) || m->u > 0xffffffffull) return false;
  *out = (uint32_t)m->u;
  return true;
}

// metadata_f32 (reader.rs:190-196): f32, or an f64 narrowed.
bool meta_f32(const camelid_gguf* g, const std::string& key, float* out) {
  const Meta* m = find_meta(g, key);
  if (!m || (m->type != 6 && m->type != 12)) return false;
  *out = (float)m->f;
  return true;
}

const camelid_gguf_tensor* tensor(const camelid_gguf* g, const std::string& name) {
  auto it = g->tensors.find(name);
  return it == g->tensors.end() ? nullptr : &it->second;
}

// GGML type -> engine weight format (the formats the resident path runs: ProjQuant,
// cuda_resident.rs:5262).
int engine_quant(int32_t ggml) {
  switch (ggml) {
    case 8: return CAMELID_Q8_0;
    case 12: return CAMELID_Q4_K;
    case 14: return CAMELID_Q6_K;
    default: return -1;
  }
}

}  // namespace

CX const char* camelid_gguf_last_error(void) { return g_err.c_str(); }

CX int camelid_gguf_open(const char* path, camelid_gguf** out) {
  if (!path || !out) return gfail("null argument");
  *out = nullptr;
  const int fd = ::open(path, O_RDONLY | O_CLOEXEC);
  if (fd < 0) return gfail(std::string("wire mmap open failed for ") + path + ": " + std::strerror(errno));
  struct stat st;
  if (fstat(fd, &st) != 0) {
    const int e = errno;
    ::close(fd);
    return gfail(std::string("wire mmap metadata failed for ") + path + ": " + std::strerror(e));
  }
  if (st.st_size == 0) {
    ::close(fd);
    return gfail(std::string("wire mmap refused for empty file ") + path);
  }
  void* p = mmap(nullptr, (size_t)st.st_size, PROT_READ, MAP_SHARED, fd, 0);
  if (p == MAP_FAILED) {
    const int e = errno;
    ::close(fd);
    return gfail(std::string("wire mmap failed for ") + path + ": " + std::strerror(e));
  }
  auto* g = new camelid_gguf;
  g->fd = fd;
  g->base = static_cast<const uint8_t*>(p);
  g->len = (uint64_t)st.st_size;
  std::string why;
  if (!parse(g, &why)) {
    camelid_gguf_close(g);
    return gfail(why);
  }
  // the weights are read front to back once (wire_mmap.rs:132 advise_sequential)
  (void)madvise(const_cast<uint8_t*>(g->base), (size_t)g->len, MADV_SEQUENTIAL);
  *out = g;
  return 0;
}

CX void camelid_gguf_close(camelid_gguf* g) {
  if (!g) return;
  if (g->base) munmap(const_cast<uint8_t*>(g->base), (size_t)g->len);
  if (g->fd >= 0) ::close(g->fd);
  delete g;
}

CX uint32_t camelid_gguf_version(const camelid_gguf* g) { return g ? g->version : 0; }
CX uint64_t camelid_gguf_alignment(const camelid_gguf* g) { return g ? g->alignment : 0; }
CX uint64_t camelid_gguf_tensor_count(const camelid_gguf* g) { return g ? g->names.size() : 0; }

CX const char* camelid_gguf_tensor_name(const camelid_gguf* g, uint64_t i) {
  return g && i < g->names.size() ? g->names[i].c_str() : nullptr;
}

CX int camelid_gguf_find(const camelid_gguf* g, const char* name, camelid_gguf_tensor* out) {
  if (!g || !name || !out) return gfail("null argument");
  const camelid_gguf_tensor* t = tensor(g, name);
  if (!t) return gfail(std::string("tensor ") + name + " not found");
  *out = *t;
  return 0;
}

CX int camelid_gguf_meta_u32(const camelid_gguf* g, const char* key, uint32_t* out) {
  if (!g || !key || !out) return gfail("null argument");
  return meta_u32(g, key, out) ? 0 : gfail(std::string("metadata ") + key + " missing or not u32");
}

CX int camelid_gguf_meta_f32(const camelid_gguf* g, const char* key, float* out) {
  if (!g || !key || !out) return gfail("null argument");
  return meta_f32(g, key, out) ? 0 : gfail(std::string("metadata ") + key + " missing or not f32");
}

CX const char* camelid_gguf_meta_str(const camelid_gguf* g, const char* key) {
  if (!g || !key) return nullptr;
  const Meta* m = find_meta(g, key);
  return m && m->type == 8 ? m->s.c_str() : nullptr;
}

// The engine dimensions and RoPE parameters of a mapped model (model.rs:137-230
// ModelConfig::from_gguf for the dense architectures the resident path runs).
CX int camelid_gguf_model(const camelid_gguf* g, uint32_t max_pos, camelid_hip_dims* dims, camelid_gguf_rope* rope) {
  if (!g || !dims || !rope) return gfail("null argument");
  const char* arch = camelid_gguf_meta_str(g, "general.architecture");
  if (!arch) return gfail("required metadata general.architecture is missing");
  const std::string a(arch);
  if (a != "llama" && a != "mistral" && a != "qwen3" && a != "qwen2")
    return gfail("architecture " + a + " is not on the resident decode path");
  auto key = [&](const char* s) { return a + "." + s; };
  camelid_hip_dims d{};
  uint32_t v = 0;
  if (!meta_u32(g, key("block_count"), &d.n_layers) || !meta_u32(g, key("embedding_length"), &d.hidden) ||
      !meta_u32(g, key("feed_forward_length"), &d.ffn_dim) || !meta_u32(g, key("attention.head_count"), &d.n_heads))
    return gfail("required " + a + " dimension metadata missing");
  d.n_kv_heads = meta_u32(g, key("attention.head_count_kv"), &v) ? v : d.n_heads;
  if (d.n_heads == 0) return gfail("attention.head_count is zero");
  d.head_dim = meta_u32(g, key("attention.key_length"), &v) ? v : d.hidden / d.n_heads;
  d.rope_dim = meta_u32(g, key("rope.dimension_count"), &v) ? v : d.head_dim;
  const camelid_gguf_tensor* emb = tensor(g, "token_embd.weight");
  if (meta_u32(g, key("vocab_size"), &v)) {
    d.vocab = v;
  } else if (emb && emb->n_dims == 2 && emb->dims[0] == d.hidden) {
    d.vocab = (uint32_t)emb->dims[1];
  } else {
    return gfail("vocab size unknown (no vocab_size and no token_embd.weight [hidden, vocab])");
  }
  float f = 0.0f;
  d.eps = meta_f32(g, key("attention.layer_norm_rms_epsilon"), &f) ? f : 1e-5f;
  d.split_half_pairing = (a == "qwen3" || a == "qwen2") ? 1u : 0u;  // model.rs:690-692 (unpermuted GGUFs)
  d.max_pos = max_pos;
  camelid_gguf_rope r{};
  r.freq_base = meta_f32(g, key("rope.freq_base"), &f) ? f : 10000.0f;
  r.scaling_kind = 0;
  r.factor = 1.0f;
  if (const char* st = camelid_gguf_meta_str(g, key("rope.scaling.type").c_str())) {
    const std::string s(st);
    if (s == "linear") r.scaling_kind = 1;
    else if (s == "llama3") r.scaling_kind = 2;
    else if (s != "none") return gfail("rope scaling " + s + " is not supported");
  }
  if (meta_f32(g, key("rope.scaling.factor"), &f)) r.factor = f;
  r.orig_ctx = meta_u32(g, key("rope.scaling.original_context_length"), &v) ? (float)v : 8192.0f;
  r.low = meta_f32(g, key("rope.scaling.low_freq_factor"), &f) ? f : 1.0f;
  r.high = meta_f32(g, key("rope.scaling.high_freq_factor"), &f) ? f : 4.0f;
  r.freqs = nullptr;
  if (const camelid_gguf_tensor* rf = tensor(g, "rope_freqs.weight")) {
    // model.rs:938-944: the RoPE dimension count must be even and within the head dimension,
    // and the tensor's descriptor shape exactly [rope_dim / 2]
    if (d.rope_dim == 0 || d.rope_dim > d.head_dim || d.rope_dim % 2 != 0)
      return gfail("RoPE dimension count " + std::to_string(d.rope_dim) + " must be even and within head dimension " +
                   std::to_string(d.head_dim));
    const uint32_t half = d.rope_dim / 2;
    if (rf->n_dims != 1 || rf->dims[0] != half) {
      std::string got = "[";
      for (uint32_t i = 0; i < rf->n_dims; ++i) got += (i ? ", " : "") + std::to_string(rf->dims[i]);
      return gfail("rope frequencies tensor rope_freqs.weight expected descriptor shape [" + std::to_string(half) +
                   "], got " + got + "]");
    }
    // tensor/mod.rs:3943-3946 load_cpu_f32: F32 as stored, F16 and BF16 widened
    const uint8_t* p = rf->data;
    if (rf->type == 0) {
      r.freqs = reinterpret_cast<const float*>(p);
    } else if (rf->type == 1 || rf->type == 30) {
      g->rope_freqs_f32.resize(half);
      for (uint32_t i = 0; i < half; ++i) {
        const uint16_t b = (uint16_t)(p[2 * i] | (p[2 * i + 1] << 8));
        g->rope_freqs_f32[i] = rf->type == 1 ? camelid_f16_to_f32(b) : bf16_to_f32(b);
      }
      r.freqs = g->rope_freqs_f32.data();
    } else {
      return gfail("rope_freqs.weight of GGML type " + std::to_string(rf->type) +
                   " is not read by this loader (F32, F16 or BF16 only)");
    }
    // rope.rs:303-312 validate_rope_frequency_tensor
    for (uint32_t i = 0; i < half; ++i)
      if (!(r.freqs[i] > 0.0f) || !std::isfinite(r.freqs[i]))
        return gfail("rope_freqs.weight[" + std::to_string(i) + "] frequency factor " + std::to_string(r.freqs[i]) +
                     " must be finite and positive");
  }
  *dims = d;
  *rope = r;
  return 0;
}

// Every layer, the output and (optionally) the token table of a mapped model into the engine:
// the seam's upload (inference.rs:11245 build_resident_cuda_engine) with the tensors read
// straight from the mapping.  Tensor names are the GGUF ones (model.rs:770-900); the lm_head
// falls back to token_embd.weight when output.weight is absent (tied embeddings).
CX int camelid_hip_load_gguf(camelid_hip_engine* e, const camelid_gguf* g, int with_embedding) {
  if (!e || !g) return gfail("null argument");
  static const char* proj[7] = {"attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_up", "ffn_down"};
  const uint32_t L = camelid_hip_n_layers(e);
  auto f32 = [&](const std::string& name, bool required, const float** out) -> bool {
    *out = nullptr;
    const camelid_gguf_tensor* t = tensor(g, name);
    if (!t) return !required || !gfail("tensor " + name + " not found");
    if (t->type != 0) return !gfail("tensor " + name + " must be F32");
    *out = reinterpret_cast<const float*>(t->data);
    return true;
  };
  for (uint32_t l = 0; l < L; ++l) {
    const uint8_t* w[7];
    size_t len[7];
    uint8_t quant[7];
    for (int i = 0; i < 7; ++i) {
      const std::string name = "blk." + std::to_string(l) + "." + proj[i] + ".weight";
      const camelid_gguf_tensor* t = tensor(g, name);
      if (!t) return gfail("tensor " + name + " not found");
      const int q = engine_quant(t->type);
      if (q < 0) return gfail("tensor " + name + " has GGML type " + std::to_string(t->type) +
                              " (the resident path runs Q8_0, Q4_K and Q6_K)");
      w[i] = t->data;
      len[i] = (size_t)t->n_bytes;
      quant[i] = (uint8_t)q;
    }
    const std::string pre = "blk." + std::to_string(l) + ".";
    const float *an, *fn, *qn, *kn;
    if (!f32(pre + "attn_norm.weight", true, &an) || !f32(pre + "ffn_norm.weight", true, &fn) ||
        !f32(pre + "attn_q_norm.weight", false, &qn) || !f32(pre + "attn_k_norm.weight", false, &kn))
      return 1;
    if (camelid_hip_set_layer(e, l, w, len, quant, CAMELID_Q8_WIRE34, an, fn, qn, kn))
      return gfail(camelid_hip_last_error(e));
  }
  const float* on;
  if (!f32("output_norm.weight", true, &on)) return 1;
  const camelid_gguf_tensor* out = tensor(g, "output.weight");
  if (!out) out = tensor(g, "token_embd.weight");
  if (!out) return gfail("neither output.weight nor token_embd.weight is present");
  const int oq = engine_quant(out->type);
  if (oq < 0) return gfail("output projection GGML type " + std::to_string(out->type) + " is not supported");
  if (camelid_hip_set_output(e, on, out->data, (size_t)out->n_bytes, (uint8_t)oq, CAMELID_Q8_WIRE34))
    return gfail(camelid_hip_last_error(e));
  if (with_embedding) {
    const camelid_gguf_tensor* emb = tensor(g, "token_embd.weight");
    if (!emb) return gfail("tensor token_embd.weight not found");
    const int eq = engine_quant(emb->type);
    if (eq < 0) return gfail("token_embd GGML type " + std::to_string(emb->type) + " is not supported");
    if (camelid_hip_set_embedding(e, emb->data, (size_t)emb->n_bytes, (uint8_t)eq, CAMELID_Q8_WIRE34))
      return gfail(camelid_hip_last_error(e));
  }
  return 0;
}
