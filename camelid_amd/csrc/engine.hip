// engine.hip -- resident decode engine for MI355X (gfx950) behind the C ABI of
// include/camelid_hip.h.  Mirrors CudaResidentDecode (src/cuda_resident.rs:5398-8857):
// weights and the f16 KV cache stay in HBM; one HIP stream; one host sync per call.
//
// Device memory layout (all resident for the engine's lifetime):
//   per layer: Wqkv (Q8R, rows nq+2*nkv), Wo (Q8R), Wgate|up (Q8R, rows 2F), Wdown (Q8R),
//              attn/ffn norm [H], optional q/k norm [hd]
//   lm_head Q8R [V][H], final norm [H], optional token_embd Q8R [V][H]
//   KV cache: per (layer, kv head) regions of hd * kvs f16 elements, K as [hd/8][kvs][8] and
//   V as [kvs/8][hd][8] (cm::kv_k_index / cm::kv_v_index), kvs = max_pos rounded up to a
//   multiple of 8
//   activations: h [H] (residual stream), qkv, att [nq], gu [2F], logits [V], one Q8_0
//                activation buffer (quants + f32 scales) reused by every GEMV
//   StepState {pos, tok, step}: the decode loop's device-side state
//
// Per decode step (launch order on the one stream):
//   [embed]  rmsnorm_quant -> gemv(QKV) -> attention(+QK-norm, RoPE, KV store) ->
//   gemv(O, +residual) -> rmsnorm_quant -> gemv(gate|up) -> silu_quant ->
//   gemv(down, +residual)   x L,   then rmsnorm_quant -> gemv_argmax(lm_head)
// The device-side loop captures one step in a HIP graph and replays it; the step reads
// the token and position from StepState and the argmax advances them.
#include <hip/hip_runtime.h>
#include <hip/hip_ext.h>
#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <thread>
#include <vector>

#include "../../include/camelid_hip.h"
#include "kernels_decode.h"
#include "kernels_prefill.h"
#include "kernels_kquant.h"

namespace {

thread_local std::string g_last_error;

struct Q8Mat {
  int8_t* q = nullptr;
  uint16_t* d = nullptr;
  uint32_t rows = 0, k = 0;
  // a weight scale is +-inf (or not known not to be): the prefill GEMM folds with the plain
  // conversion and product (cm::k_gemm_q8<true, NF>), which gives dot * inf; else with one FMA
  bool inf_scale = true;
};

// Whether any of the n f16 values is +-inf.
bool f16_any_inf(const uint16_t* h, size_t n) {
  for (size_t i = 0; i < n; ++i)
    if ((h[i] & 0x7fffu) == 0x7c00u) return true;
  return false;
}

// A K-quant matrix as planes split out of its GGUF superblocks (kernels_kquant.h):
// Q4_K: a = nibbles [rows][k/2], b = headers [rows][k/256][16];
// Q6_K: a = ql [rows][k/2], b = qh [rows][k/4], sc = scales [rows][k/256][16], d = f16 [rows][k/256].
struct KMat {
  uint8_t quant = 0;
  uint8_t* a = nullptr;
  uint8_t* b = nullptr;
  int8_t* sc = nullptr;
  uint16_t* d = nullptr;
  uint32_t rows = 0, k = 0;
  // Q6_K projections: the scaled weights as class-major int8 planes for the prefill GEMM
  // (cm::k_gemm_q6k2; cm::q6g_planes_bytes, built by cm::k_q6k_w2); null: the sparse-MFMA GEMM
  int8_t* w2 = nullptr;
};

// One projection in its own format (the layers with any K-quant projection keep all seven
// separately; all-Q8_0 layers use the fused QKV / gate|up matrices below).
struct Proj {
  uint8_t quant = CAMELID_Q8_0;
  Q8Mat q8;
  KMat kq;
};

struct LayerW {
  Q8Mat qkv, o, gu, down;
  bool generic = false;  // some projection is a K-quant: seven separate projections in p
  Proj p[7];
  bool qk_stacked = false;  // generic layer: p[0] holds q|k stacked (same K-quant format)
  bool gu_stacked = false;  // generic layer: p[4] holds gate|up stacked
  float* attn_norm = nullptr;
  float* ffn_norm = nullptr;
  float* q_norm = nullptr;
  float* k_norm = nullptr;
  bool set = false;
};

// Profiling categories (camelid_hip_profile_end).
enum { P_GEMV = 0, P_NORM, P_ATTN, P_SILU, P_HEAD, P_EMBED, P_GEMM, P_NCAT };

}  // namespace

struct camelid_hip_engine {
  camelid_hip_dims d{};
  int device = 0;
  hipStream_t stream = nullptr;
  std::vector<LayerW> layers;
  Q8Mat out;
  KMat out_k;                 // K-quant lm_head (out_quant != Q8_0)
  uint8_t out_quant = CAMELID_Q8_0;
  float* out_norm = nullptr;
  bool out_set = false;
  Q8Mat embd;
  KMat embd_k;                // K-quant token table (embd_quant != Q8_0)
  uint8_t embd_quant = CAMELID_Q8_0;
  bool embd_set = false;
  bool any_kquant = false;
  // K-quant activations: the f32 input of the next projection and its Q8_K quantization
  float* xn = nullptr;        // [max(H, F, nq)]
  float* actf = nullptr;      // SwiGLU output [F]
  float* kd = nullptr;        // Q8_K block scales
  int8_t* kq = nullptr;       // Q8_K quants
  int32_t* kbs = nullptr;     // per-32 quant sums
  uint16_t* kc = nullptr;  // K, granules of 8 dims per position (cm::kv_k_index)
  uint16_t* vc = nullptr;  // V, granules of 8 positions per dim (cm::kv_v_index)
  uint32_t kvs = 0;        // KV position stride: max_pos rounded up to a multiple of 8
  int att_slots = 0;       // V ring chunks of the attention kernel
  // long contexts: the split attention (k_att_scores + k_att_out) from att_split_min positions
  // on (CAMELID_HIP_ATT_SPLIT; 0 = never); its scores [n_heads][kvs] and slice maxima.
  // Measured on MI355X: at ~550 positions the single-workgroup kernel is faster (C3 657 vs
  // 638 tok/s with the split everywhere); from ~1024 on the split is (C5 299.5 vs 293.4 tok/s)
  uint32_t att_split_min = 1024;
  float* att_sc = nullptr;
  float* att_mx = nullptr;
  // the split attention as one launch (cm::k_att_fused: score slices, output workgroups and,
  // for Q8_0 layers, the output projection, handing over through tagged words;
  // CAMELID_HIP_ATT_FUSED_SPLIT=0: the two launches) and its tagged scores [n_heads][kvs]
  bool att_fsplit = true;
  uint64_t* att_sct = nullptr;
  uint32_t n_cus = 256;  // compute units of the device (read at creation)
  int att_mode = -1;       // -1: by position; 0 / 1: single / split (graph capture)
  // Read-ahead (off by default): spare workgroups of the norm and attention kernels read the
  // next projection's weights towards the caches; the qkv GEMV's idle norm waves read the
  // layer's KV rows.  Measured on the three big configs with the current kernels: no gain
  // (C3 663.5 -> 664.8, C4 213.0 -> 214.2, C5 355.7 -> 359.7 tok/s with it off), and the
  // counters show attention fetching its K/V rows again either way, so it is opt-in.
  bool read_ahead = false;
  bool kv_ahead = false;
  // workgroups per query head of the decode attention (CAMELID_HIP_ATT_DG; 0: 64 output dims
  // per workgroup): each stages only its dims' V rows
  int att_dg = 0;
  bool gu_fused = false;   // gate/up rows interleaved by 32, SwiGLU fused into their GEMV
  bool norm_fused = true;  // RMSNorms computed inside the qkv and gate/up GEMVs (Q8_0 layers)
  bool qkv_merged = true;  // Q4_K q|k and Q6_K v projections in one launch (k_gemv_qk4_v6)
  // K-quant layers with the RMSNorm inside the q|k+v and gate|up launches (cm::k_norm_qk4_v6,
  // cm::k_norm_gemv_q4k; CAMELID_HIP_KQ_NORM_FUSED): on when every layer has that shape
  bool kq_norm_fused = true;
  bool q6_gemm2 = true;  // Q6_K projections get the class-major prefill GEMM's planes (CAMELID_HIP_Q6K_GEMM2)
  bool gu_loop = true;   // norm-fused Q8_0 gate/up: workgroups loop over row groups (CAMELID_HIP_GU_LOOP)
  int nf_state = -1;              // -1 unknown, 0 off, 1 on (every layer fusable)
  uint32_t* nf_slots = nullptr;   // the launches' flag words (cm::NF_WORDS)
  // Q8_0 layers: the output projection inside the single-workgroup attention launch
  // (cm::att_oproj; CAMELID_HIP_ATT_O).  Measured on MI355X: see the layer loop.
  bool att_o_fused = true;
  int ao_state = -1;              // -1 unknown, 0 off, 1 on
  int ao4_state = -1;             // the Q4_K output projection in the split attention launch (ao4_enabled)
  uint64_t* ao_words = nullptr;   // the tagged activation words (ao_words())
  uint32_t* p_err = nullptr;      // host copy of the handoff error word
  bool err_pending = false;       // nf_end enqueued its copy in the current call
  float *h = nullptr, *qkv = nullptr, *att = nullptr, *gu = nullptr;
  float *logits = nullptr, *hidden_cap = nullptr, *xs = nullptr;
  float *cos_cur = nullptr, *sin_cur = nullptr, *rope_cos = nullptr, *rope_sin = nullptr;
  uint32_t rope_rows = 0;
  int8_t* xq = nullptr;
  int8_t* aq = nullptr;      // SwiGLU activation quants (fused gate/up path), [ffn]
  float* as = nullptr;       // its block scales, [ffn / 32]
  float* part_v = nullptr;
  uint32_t* part_i = nullptr;
  cm::StepState* st = nullptr;
  uint32_t* tokens = nullptr;  // device ring of generated tokens (device-side loop)
  uint32_t tokens_cap = 0;
  // pinned host staging
  float *p_emb = nullptr, *p_cos = nullptr, *p_sin = nullptr, *p_logits = nullptr;
  cm::StepState* p_st = nullptr;
  // batched prefill: per-chunk activations of up to PREFILL_CHUNK tokens (allocated on the
  // first prefill): residual rows, QKV rows, rotated q rows, gate|up rows, Q8_0 activations
  bool prefill_batched = true;
  float *pf_h = nullptr, *pf_qkv = nullptr, *pf_q = nullptr, *pf_gu = nullptr, *pf_xs = nullptr;
  int8_t* pf_xq = nullptr;
  // layers with K-quant projections: Q8_K activation rows, f32 attention rows, and the rows of
  // a Q8_0 projection before they are scattered into the QKV / gate|up rows
  float *pf_kd = nullptr, *pf_att = nullptr, *pf_tmp = nullptr;
  int8_t* pf_kq = nullptr;
  int8_t* pf_kqt = nullptr;  // the chunk's Q8_K quants in the class-major order of the Q6_K GEMM
  int32_t* pf_kbs = nullptr;
  // score rows of the tiled prefill attention (cm::k_attn_prefill_tile; CAMELID_HIP_ATT_TILE=0:
  // one workgroup per (head, token) instead), sized for a chunk ending at max_pos
  bool att_tile = true;
  uint32_t att_tile_pos = 1024;  // chunks ending below this position: per-token kernel (CAMELID_HIP_ATT_TILE_POS)
  float* pf_sc = nullptr;
  // verify scratch (allocated on first use): inputs of up to CAMELID_MAX_VERIFY_K tokens,
  // their logits and greedy tokens
  float *v_embs = nullptr, *v_cos = nullptr, *v_sin = nullptr, *v_logits = nullptr, *v_pv = nullptr;
  uint32_t *v_tok = nullptr, *v_pi = nullptr;
  uint32_t filled = 0;
  uint32_t cur_pos = 0;  // host copy of the position being computed (profiling byte counts)
  bool capture = false;
  // device-side loop graph (one decode step)
  hipGraph_t graph[2] = {nullptr, nullptr};  // [0]: single-workgroup attention, [1]: split
  hipGraphExec_t graph_exec[2] = {nullptr, nullptr};
  float graph_scale[2] = {0.0f, 0.0f};
  bool use_graph = true;
  // optional per-launch HIP-event timing (camelid_hip_profile_*)
  bool profiling = false;
  struct Rec {
    int cat;
    double bytes;
    hipEvent_t a, b;
  };
  std::vector<Rec> recs;
  std::vector<hipEvent_t> event_pool;
  size_t pool_next = 0;
  std::string err;
  std::vector<void*> dev_allocs;
  std::vector<void*> host_allocs;
};

namespace {

int fail(camelid_hip_engine* e, const std::string& msg) {
  if (e) e->err = msg;
  g_last_error = msg;
  return 1;
}

#define HIP_TRY(eng, expr)                                                           \
  do {                                                                               \
    hipError_t _st = (expr);                                                         \
    if (_st != hipSuccess)                                                           \
      return fail((eng), std::string(#expr) + " failed: " + hipGetErrorString(_st)); \
  } while (0)

template <typename T>
int dev_alloc(camelid_hip_engine* e, T** p, size_t count) {
  void* v = nullptr;
  size_t bytes = std::max<size_t>(count * sizeof(T), 256);
  hipError_t st = hipMalloc(&v, bytes);
  if (st != hipSuccess)
    return fail(e, std::string("hipMalloc(") + std::to_string(bytes) + ") failed: " + hipGetErrorString(st));
  e->dev_allocs.push_back(v);
  *p = static_cast<T*>(v);
  return 0;
}

template <typename T>
int host_alloc(camelid_hip_engine* e, T** p, size_t count) {
  void* v = nullptr;
  const size_t bytes = std::max<size_t>(count * sizeof(T), 64);
  hipError_t st = hipHostMalloc(&v, bytes, hipHostMallocDefault);
  if (st != hipSuccess) return fail(e, std::string("hipHostMalloc failed: ") + hipGetErrorString(st));
  std::memset(v, 0, bytes);  // (pinned pages may be reused from an earlier allocation)
  e->host_allocs.push_back(v);
  *p = static_cast<T*>(v);
  return 0;
}

uint16_t read_le16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }

// Repack rows [r0, r1) of a 34/36-byte-block Q8_0 matrix into the Q8R planes.
void repack_rows(const uint8_t* src, size_t r0, size_t r1, size_t k, uint8_t layout, int8_t* q, uint16_t* d) {
  const size_t nb = k / 32;
  for (size_t r = r0; r < r1; ++r) {
    for (size_t b = 0; b < nb; ++b) {
      const uint8_t* blk = src + (r * nb + b) * layout;
      uint16_t bits;
      if (layout == 34) {
        bits = read_le16(blk);
      } else {
        float f;
        std::memcpy(&f, blk, 4);
        bits = cm::f32_to_f16_bits(f);  // exact: the f32 scale was decoded from an f16
      }
      d[r * nb + b] = bits;
      std::memcpy(q + r * k + b * 32, blk + (layout == 34 ? 2 : 4), 32);
    }
  }
}

void repack_parallel(const uint8_t* src, size_t rows, size_t k, uint8_t layout, int8_t* q, uint16_t* d) {
  unsigned nt = std::max(1u, std::min(16u, std::thread::hardware_concurrency()));
  if (rows < 4096) nt = 1;
  std::vector<std::thread> th;
  for (unsigned t = 0; t < nt; ++t) {
    size_t r0 = rows * t / nt, r1 = rows * (t + 1) / nt;
    th.emplace_back(repack_rows, src, r0, r1, k, layout, q, d);
  }
  for (auto& x : th) x.join();
}

struct Part {
  const uint8_t* src;
  size_t len;
  uint32_t rows;
};

// Upload `parts` (stacked row-wise) as one Q8R matrix.
// group > 0 (two parts of equal rows): interleave them in groups of `group` rows, part 0's
// group first (the fused gate/up layout).
int upload_q8(camelid_hip_engine* e, Q8Mat* m, const std::vector<Part>& parts, uint32_t k, uint8_t layout,
              uint32_t group = 0) {
  if (layout != 34 && layout != 36) return fail(e, "q8_layout must be 34 or 36");
  if (k % 32 != 0) return fail(e, "Q8_0 row width must be a multiple of 32");
  uint32_t rows = 0;
  for (const Part& p : parts) {
    if (!p.src) return fail(e, "missing projection bytes");
    size_t want = (size_t)p.rows * (k / 32) * layout;
    if (p.len != want)
      return fail(e, "projection byte length " + std::to_string(p.len) + " != expected " + std::to_string(want));
    rows += p.rows;
  }
  const size_t nb = k / 32;
  std::vector<int8_t> q((size_t)rows * k);
  std::vector<uint16_t> d((size_t)rows * nb);
  size_t r = 0;
  for (const Part& p : parts) {
    repack_parallel(p.src, p.rows, k, layout, q.data() + r * k, d.data() + r * nb);
    r += p.rows;
  }
  if (group) {
    if (parts.size() != 2 || parts[0].rows != parts[1].rows || parts[0].rows % group)
      return fail(e, "interleaved upload needs two parts of equal rows, a multiple of the group");
    const size_t half = parts[0].rows;
    std::vector<int8_t> q2(q.size());
    std::vector<uint16_t> d2(d.size());
    for (size_t g = 0; g < half / group; ++g)
      for (size_t h = 0; h < 2; ++h) {
        const size_t src = h * half + g * group, dst = (2 * g + h) * group;
        std::memcpy(q2.data() + dst * k, q.data() + src * k, group * k);
        std::memcpy(d2.data() + dst * nb, d.data() + src * nb, group * nb * 2);
      }
    q.swap(q2);
    d.swap(d2);
  }
  if (!m->q) {
    if (dev_alloc(e, &m->q, q.size()) || dev_alloc(e, &m->d, d.size())) return 1;
  } else if (m->rows != rows || m->k != k) {
    return fail(e, "matrix shape changed on re-upload");
  }
  m->rows = rows;
  m->k = k;
  m->inf_scale = f16_any_inf(d.data(), d.size());
  HIP_TRY(e, hipMemcpy(m->q, q.data(), q.size(), hipMemcpyHostToDevice));
  HIP_TRY(e, hipMemcpy(m->d, d.data(), d.size() * 2, hipMemcpyHostToDevice));
  return 0;
}

// Split rows of K-quant wire superblocks into the KMat planes (host).
void kq_split_rows(uint8_t quant, const uint8_t* src, size_t r0, size_t r1, size_t k, uint8_t* a, uint8_t* b,
                   int8_t* sc, uint16_t* d) {
  const size_t nsb = k / 256, bb = quant == CAMELID_Q4_K ? 144 : 210;
  for (size_t r = r0; r < r1; ++r)
    for (size_t s = 0; s < nsb; ++s) {
      const uint8_t* blk = src + (r * nsb + s) * bb;
      const size_t sb = r * nsb + s;
      if (quant == CAMELID_Q4_K) {
        std::memcpy(b + sb * 16, blk, 16);
        std::memcpy(a + sb * 128, blk + 16, 128);
      } else {
        std::memcpy(a + sb * 128, blk, 128);
        std::memcpy(b + sb * 64, blk + 128, 64);
        std::memcpy(sc + sb * 16, blk + 192, 16);
        d[sb] = read_le16(blk + 208);
      }
    }
}

size_t kq_block_bytes(uint8_t quant) { return quant == CAMELID_Q4_K ? 144 : 210; }

// Widest K-quant row the GEMV/GEMM kernels take (k_gemv_q4k<IT> is instantiated for IT <= 8
// 16-byte pieces per lane: (k / 32 + 63) / 64 <= 8).
constexpr uint32_t KQ_MAX_K = 16384;

// A launch the host could not map to a kernel instantiation (reported by check_launch; set
// by launch helpers that have no engine to fail on).
thread_local std::string g_launch_error;

int upload_kq(camelid_hip_engine* e, KMat* m, const uint8_t* src, size_t len, uint32_t rows, uint32_t k,
              uint8_t quant, bool gemm_planes = false) {
  if (quant != CAMELID_Q4_K && quant != CAMELID_Q6_K) return fail(e, "unknown weight format");
  if (!src) return fail(e, "missing projection bytes");
  if (k % 256) return fail(e, "K-quant row width must be a multiple of 256");
  // the K-quant GEMVs hold a row's activation in LDS and instantiate up to 8 pieces per lane
  if (k > (uint32_t)KQ_MAX_K)
    return fail(e, "K-quant row width " + std::to_string(k) + " > " + std::to_string(KQ_MAX_K) + " is not supported");
  const size_t nsb = k / 256, want = (size_t)rows * nsb * kq_block_bytes(quant);
  if (len != want) return fail(e, "K-quant byte length " + std::to_string(len) + " != expected " + std::to_string(want));
  std::vector<uint8_t> a((size_t)rows * k / 2), b((size_t)rows * nsb * (quant == CAMELID_Q4_K ? 16 : 64));
  std::vector<int8_t> sc(quant == CAMELID_Q6_K ? (size_t)rows * nsb * 16 : 0);
  std::vector<uint16_t> d(quant == CAMELID_Q6_K ? (size_t)rows * nsb : 0);
  {
    unsigned nt = std::max(1u, std::min(16u, std::thread::hardware_concurrency()));
    if (rows < 4096) nt = 1;
    std::vector<std::thread> th;
    for (unsigned t = 0; t < nt; ++t)
      th.emplace_back(kq_split_rows, quant, src, (size_t)rows * t / nt, (size_t)rows * (t + 1) / nt, (size_t)k,
                      a.data(), b.data(), sc.data(), d.data());
    for (auto& x : th) x.join();
  }
  if (!m->a) {
    if (dev_alloc(e, &m->a, a.size()) || dev_alloc(e, &m->b, b.size())) return 1;
    if (quant == CAMELID_Q6_K && (dev_alloc(e, &m->sc, sc.size()) || dev_alloc(e, &m->d, d.size()))) return 1;
  } else if (m->rows != rows || m->k != k || m->quant != quant) {
    return fail(e, "matrix shape changed on re-upload");
  }
  m->quant = quant;
  m->rows = rows;
  m->k = k;
  HIP_TRY(e, hipMemcpy(m->a, a.data(), a.size(), hipMemcpyHostToDevice));
  HIP_TRY(e, hipMemcpy(m->b, b.data(), b.size(), hipMemcpyHostToDevice));
  if (quant == CAMELID_Q6_K) {
    HIP_TRY(e, hipMemcpy(m->sc, sc.data(), sc.size(), hipMemcpyHostToDevice));
    HIP_TRY(e, hipMemcpy(m->d, d.data(), d.size() * 2, hipMemcpyHostToDevice));
    if (gemm_planes && e->q6_gemm2) {  // the prefill GEMM's weight planes, built on the device
      if (!m->w2 && dev_alloc(e, &m->w2, cm::q6g_planes_bytes((int)rows, (int)k))) return 1;
      hipLaunchKernelGGL(cm::k_q6k_w2, dim3((rows + cm::Q6G_R - 1) / cm::Q6G_R * cm::Q6G_R, (uint32_t)nsb), dim3(256),
                         0, e->stream, m->a, m->b, m->sc, (int)rows, (int)k, m->w2);
      HIP_TRY(e, hipGetLastError());
      HIP_TRY(e, hipStreamSynchronize(e->stream));
    }
  }
  return 0;
}

int upload_f32(camelid_hip_engine* e, float** dst, const float* src, size_t n) {
  if (!*dst && dev_alloc(e, dst, n)) return 1;
  HIP_TRY(e, hipMemcpy(*dst, src, n * 4, hipMemcpyHostToDevice));
  return 0;
}

// ---------------------------------------------------------------- profiling
hipEvent_t next_event(camelid_hip_engine* e) {
  if (e->pool_next == e->event_pool.size()) {
    hipEvent_t ev;
    if (hipEventCreate(&ev) != hipSuccess) return nullptr;
    e->event_pool.push_back(ev);
  }
  return e->event_pool[e->pool_next++];
}

// Profiling: while a ProfScope is open on the calling thread, each engine launch goes out
// through hipExtLaunchKernelGGL with a start/stop event pair, which the runtime stamps at
// the dispatch's own begin and end (the kernel's duration, as a kernel trace reports it).
// The scope's algorithmic bytes are credited to its first launch.
struct ProfScope;
thread_local ProfScope* g_prof = nullptr;

struct ProfScope {
  camelid_hip_engine* e;
  int cat;
  double bytes;
  bool first = true;
  ProfScope(camelid_hip_engine* eng, int c, double b) : e(eng), cat(c), bytes(b) {
    if (e->profiling) g_prof = this;
  }
  ~ProfScope() {
    if (g_prof == this) g_prof = nullptr;
  }
  // Event pair for the next launch of this scope (false when none can be created).
  bool take(hipEvent_t* a, hipEvent_t* b) {
    *a = next_event(e);
    *b = *a ? next_event(e) : nullptr;
    if (!*b) return false;
    e->recs.push_back({cat, first ? bytes : 0.0, *a, *b});
    first = false;
    return true;
  }
};

// Launch through the profiler when a scope is open, plainly otherwise.
#define CM_LAUNCH(K, G, B, S, STREAM, ...)                                                 \
  do {                                                                                    \
    hipEvent_t cm_a_, cm_b_;                                                              \
    if (g_prof && g_prof->take(&cm_a_, &cm_b_))                                           \
      hipExtLaunchKernelGGL(K, G, B, S, STREAM, cm_a_, cm_b_, 0, __VA_ARGS__);            \
    else                                                                                  \
      hipLaunchKernelGGL(K, G, B, S, STREAM, __VA_ARGS__);                        \
  } while (0)

// Algorithmic bytes of one Q8_0 GEMV launch: weights (34 B per 32 values), the quantized
// activation, the f32 output (+ the residual read when fused).
double q8_bytes(const Q8Mat& m, bool resid) {
  return (double)m.rows * m.k * 34.0 / 32.0 + m.k * 34.0 / 32.0 + m.rows * (resid ? 8.0 : 4.0);
}

// ---------------------------------------------------------------- launches
uint32_t gemv_rows_per_wg(const Q8Mat& m) {
  switch (m.k) {
#define CM_GEMV_CASE(K) \
  case K:               \
    return 4 * cm::gemv_rpw(K, (int)m.rows);
    CM_GEMV_KS(CM_GEMV_CASE)
#undef CM_GEMV_CASE
    default:
      return cm::GEMV_R;
  }
}

void launch_gemv(const Q8Mat& m, const int8_t* xq, const float* xs, float* y, const float* resid, hipStream_t s) {
  const uint32_t grid = (m.rows + gemv_rows_per_wg(m) - 1) / gemv_rows_per_wg(m);
  switch (m.k) {
#define CM_GEMV_CASE(K)                                                                                             \
  case K:                                                                                                           \
    if (cm::gemv_rpw(K, (int)m.rows) == 2)                                                                          \
      CM_LAUNCH((cm::k_gemv_k<K, 2>), dim3(grid), dim3(cm::GEMV_NT), 0, s, m.q, m.d, (int)m.rows, xq, xs, y, \
                         resid);                                                                                    \
    else                                                                                                            \
      CM_LAUNCH((cm::k_gemv_k<K, 1>), dim3(grid), dim3(cm::GEMV_NT), 0, s, m.q, m.d, (int)m.rows, xq, xs, y, \
                         resid);                                                                                    \
    return;
    CM_GEMV_KS(CM_GEMV_CASE)
#undef CM_GEMV_CASE
    default:
      CM_LAUNCH(cm::k_gemv, dim3(grid), dim3(cm::GEMV_NT), cm::gemv_lds_bytes((int)m.k), s, m.q, m.d,
                         (int)m.rows, (int)m.k, xq, xs, y, resid);
  }
}

// y = W · rmsnorm(x; nw) for a Q8_0 W whose width is a fused-norm width (2048, 3072, 4096):
// at most 32 rows per workgroup, spread over up to 256 workgroups; the 8 weight waves hold
// ceil(rows per workgroup / 8) rows each.
void launch_gemv_norm(const Q8Mat& m, const float* x, const float* nw, float eps, float* y, hipStream_t s,
                      cm::KvAhead kva = cm::KvAhead{}) {
  const uint32_t per = std::min(32u, std::max(1u, (m.rows + 255u) / 256u));
  const uint32_t grid = (m.rows + per - 1) / per;
  const uint32_t rpw = (per + 7) / 8;
  switch (m.k * 8 + rpw) {
#define CM_GN(K, RPW)                                                                                                 \
  case K * 8 + RPW:                                                                                                   \
    CM_LAUNCH((cm::k_gemv_norm<K, RPW>), dim3(grid), dim3(cm::GN_NT), 0, s, m.q, m.d, (int)m.rows, (int)per, x, nw, \
              eps, y, kva);                                                                                           \
    return;
    CM_GN(2048, 1) CM_GN(2048, 2) CM_GN(2048, 3) CM_GN(2048, 4)
    CM_GN(3072, 1) CM_GN(3072, 2) CM_GN(3072, 3) CM_GN(3072, 4)
    CM_GN(4096, 1) CM_GN(4096, 2) CM_GN(4096, 3) CM_GN(4096, 4)
#undef CM_GN
    default:  // not reached: callers admit only these widths (cm::gu_fused_k), per <= 32
      g_launch_error = "qkv GEMV: no kernel for row width " + std::to_string(m.k);
      break;
  }
}

// lm_head GEMV with per-workgroup argmax partials; returns the number of partials.
uint32_t launch_gemv_argmax(const Q8Mat& m, const int8_t* xq, const float* xs, float* logits, float* part_v,
                            uint32_t* part_i, hipStream_t s) {
  const uint32_t R = gemv_rows_per_wg(m);
  const uint32_t grid = (m.rows + R - 1) / R;
  switch (m.k) {
#define CM_GEMV_CASE(K)                                                                                               \
  case K:                                                                                                             \
    if (cm::gemv_rpw(K, (int)m.rows) == 2)                                                                            \
      CM_LAUNCH((cm::k_gemv_argmax<K, 2>), dim3(grid), dim3(cm::GEMV_NT), 0, s, m.q, m.d, (int)m.rows, K, xq, \
                         xs, logits, part_v, part_i);                                                                 \
    else                                                                                                              \
      CM_LAUNCH((cm::k_gemv_argmax<K, 1>), dim3(grid), dim3(cm::GEMV_NT), 0, s, m.q, m.d, (int)m.rows, K, xq, \
                         xs, logits, part_v, part_i);                                                                 \
    return grid;
    CM_GEMV_KS(CM_GEMV_CASE)
#undef CM_GEMV_CASE
    default:
      CM_LAUNCH((cm::k_gemv_argmax<0, 1>), dim3(grid), dim3(cm::GEMV_NT), cm::gemv_lds_bytes((int)m.k), s,
                         m.q, m.d, (int)m.rows, (int)m.k, xq, xs, logits, part_v, part_i);
      return grid;
  }
}

// Attention launch for the supported head widths.
bool attention_hd_supported(uint32_t hd) { return hd == 64 || hd == 128 || hd == 256; }

constexpr uint32_t PREFETCH_WGS = 256;  // spare workgroups added to a kernel that reads ahead
// Largest matrix worth reading ahead: beyond a fraction of the 256 MB last-level cache the
// lines are evicted before their GEMV reads them and the read-ahead only adds HBM traffic and
// launch time (measured: reading the 510 MB Q6_K lm_head ahead made the final RMSNorm launch
// 77 us instead of ~10 us, with no gain in the lm_head GEMV).
constexpr size_t PREFETCH_MAX_BYTES = (size_t)128 << 20;

// Read-ahead descriptor of a Q8R matrix (quants and scales, in 128-byte lines).
cm::Prefetch prefetch_of(const Q8Mat* m) {
  cm::Prefetch pf{nullptr, 0, nullptr, 0};
  if (m && m->q && (size_t)m->rows * m->k * 34 / 32 <= PREFETCH_MAX_BYTES) {
    pf.a = reinterpret_cast<const uint32_t*>(m->q);
    pf.a_lines = (size_t)m->rows * m->k / 128;
    pf.b = reinterpret_cast<const uint32_t*>(m->d);
    pf.b_lines = (size_t)m->rows * (m->k / 32) * 2 / 128;
  }
  return pf;
}
cm::Prefetch prefetch_of(const KMat* m) {
  cm::Prefetch pf{nullptr, 0, nullptr, 0};
  if (m && m->a && (size_t)m->rows * (m->k / 256) * kq_block_bytes(m->quant) <= PREFETCH_MAX_BYTES) {
    pf.a = reinterpret_cast<const uint32_t*>(m->a);
    pf.a_lines = (size_t)m->rows * m->k / 2 / 128;
    pf.b = reinterpret_cast<const uint32_t*>(m->b);
    pf.b_lines = (size_t)m->rows * (m->k / 256) * (m->quant == CAMELID_Q4_K ? 16 : 64) / 128;
  }
  return pf;
}

size_t attn_sc_bytes(uint32_t kvs) { return (((size_t)kvs + 3) & ~(size_t)3) * 4; }
int attn_ring_slots(uint32_t kvs, bool host_only = false);
int attn_out_slots(uint32_t kvs, int slots, int* pb);

// dg: workgroups per query head (k_attention's DG: 1, 2 or 4, at most hd / 32); 0 takes the
// default, 64 output dims per workgroup (C3 decode: 671.0 / 675.6 / 668.0 tok/s at 1 / 2 / 4
// workgroups per head of 128 dims).
template <bool FUSED>
void launch_attention(uint32_t hd, uint32_t n_heads, int slots, hipStream_t s, const float* qsrc, int nh, int nkv,
                      int rope_dim, int split_half, const float* cb, const float* sb, int rs, const float* qn,
                      const float* kn, float eps, uint16_t* kc, uint16_t* vc, int layer, int kvs, const uint32_t* pos,
                      float scale, float* att, int8_t* xq, float* xs, cm::Prefetch pf, int dg = 1,
                      cm::OProj op = cm::OProj{}) {
  size_t lds = (size_t)slots * cm::ATT_RING_GRANULES * 16 + attn_sc_bytes((uint32_t)kvs);
  if (dg <= 0) dg = (int)std::max<uint32_t>(1, hd / 64);
  if (dg > 4 || (dg & (dg - 1)) || hd / (uint32_t)dg < 32) {
    g_launch_error = "attention: " + std::to_string(dg) + " workgroups per head of " + std::to_string(hd) +
                     " dims has no instantiation";
    return;
  }
  uint32_t grid = n_heads * (uint32_t)dg + (pf.a_lines ? PREFETCH_WGS : 0);
  if (op.q) {  // the output projection's workgroups instead of read-ahead ones
    if (cm::att_nt((int)hd) != cm::AO_ROWS * 64 || !cm::ao_width_ok(op.K) || op.K != (int)(n_heads * hd)) {
      g_launch_error = "attention: no output projection body for this shape";
      return;
    }
    grid = n_heads * (uint32_t)dg + (uint32_t)(op.rows + cm::AO_ROWS - 1) / cm::AO_ROWS;
    lds = std::max(lds, cm::ao_lds_bytes(op.K));
  }
#define CM_ATT(HD, DG)                                                                                         \
  CM_LAUNCH((cm::k_attention<HD, FUSED, DG>), dim3(grid), dim3(cm::att_nt(HD)), lds, s, qsrc, nh, nkv, rope_dim, \
            split_half, cb, sb, rs, qn, kn, eps, kc, vc, layer, kvs, pos, scale, att, xq, xs, slots, pf, op)
  if (hd == 64) {
    if (dg == 1) CM_ATT(64, 1);
    else CM_ATT(64, 2);
  } else if (hd == 128) {
    if (dg == 1) CM_ATT(128, 1);
    else if (dg == 2) CM_ATT(128, 2);
    else CM_ATT(128, 4);
  } else {
    if (dg == 1) CM_ATT(256, 1);
    else if (dg == 2) CM_ATT(256, 2);
    else CM_ATT(256, 4);
  }
#undef CM_ATT
}

// The split attention (k_att_scores + k_att_out): score slices of ATT_SLICE positions (grid
// sized for kvs; slices past the position exit), 32-dim output workgroups (+ read-ahead
// workgroups) for the softmax and output sum.
constexpr int ATT_SLICE = 256;
template <bool FUSED>
void launch_attention_split(uint32_t hd, uint32_t n_heads, int slots, hipStream_t s, const float* qsrc, int nh,
                            int nkv, int rope_dim, int split_half, const float* cb, const float* sb, int rs,
                            const float* qn, const float* kn, float eps, uint16_t* kc, uint16_t* vc, int layer,
                            int kvs, const uint32_t* pos, float scale, float* g_sc, float* g_mx, float* att,
                            int8_t* xq, float* xs, cm::Prefetch pf, cm::OProj op = cm::OProj{}) {
  const size_t lds = (size_t)slots * cm::ATT_RING_GRANULES * 16 + attn_sc_bytes((uint32_t)kvs);
  const int nsl = (kvs + ATT_SLICE - 1) / ATT_SLICE;
  constexpr int AOR = cm::AO_ROWS * cm::AO_SPLIT_RPW;  // rows per projection workgroup
  if (op.q && (cm::att_nt((int)hd) != cm::AO_ROWS * 64 || !cm::ao_width_ok(op.K) || op.K != (int)(n_heads * hd))) {
    g_launch_error = "split attention: no output projection body for this shape";
    return;
  }
#define CM_ATTS(HD)                                                                                                \
  {                                                                                                                \
    CM_LAUNCH((cm::k_att_scores<HD, FUSED, (HD > ATT_SLICE ? HD : ATT_SLICE)>), dim3(n_heads, nsl),               \
              dim3(HD > ATT_SLICE ? HD : ATT_SLICE), 0, s, qsrc, nh, nkv, rope_dim, split_half, cb, sb, rs, qn, kn, \
              eps, kc, vc, layer, kvs, pos, scale, g_sc, g_mx);                                                   \
    const uint32_t grid = n_heads * (HD / 32) +                                                                    \
                          (op.q ? (uint32_t)(op.rows + AOR - 1) / AOR : (pf.a_lines ? PREFETCH_WGS : 0));           \
    int pb = 0;                                                                                                    \
    const int so = attn_out_slots((uint32_t)kvs, slots, &pb);                                                      \
    size_t lds_o = (size_t)so * cm::AO_RING_GRANULES * 16 + attn_sc_bytes((uint32_t)kvs) + cm::avp_bytes(pb);     \
    if (op.q) lds_o = std::max(lds_o, cm::ao_lds_bytes(op.K, AOR));                                               \
    if (pb == 256)                                                                                                 \
      CM_LAUNCH((cm::k_att_out<HD, 256>), dim3(grid), dim3(cm::att_nt(HD)), lds_o, s, vc, nh, nkv, layer, kvs, pos, \
                g_sc, g_mx, nsl, (HD > ATT_SLICE ? HD : ATT_SLICE), att, xq, xs, so, pf, op);                      \
    else if (pb == 128)                                                                                            \
      CM_LAUNCH((cm::k_att_out<HD, 128>), dim3(grid), dim3(cm::att_nt(HD)), lds_o, s, vc, nh, nkv, layer, kvs, pos, \
                g_sc, g_mx, nsl, (HD > ATT_SLICE ? HD : ATT_SLICE), att, xq, xs, so, pf, op);                      \
    else                                                                                                           \
      CM_LAUNCH((cm::k_att_out<HD, 64>), dim3(grid), dim3(cm::att_nt(HD)), lds_o, s, vc, nh, nkv, layer, kvs, pos,  \
                g_sc, g_mx, nsl, (HD > ATT_SLICE ? HD : ATT_SLICE), att, xq, xs, so, pf, op);                      \
  }
  if (hd == 64) CM_ATTS(64)
  else if (hd == 128) CM_ATTS(128)
  else CM_ATTS(256)
#undef CM_ATTS
}

// The one-launch split attention (cm::k_att_fused): score slices of 128 positions up to 1024
// cache positions (more CUs stream a head's K), of one workgroup's threads beyond; output
// workgroups as k_att_out's; the output projection's workgroups when op.q is set.
int fsplit_sl(uint32_t kvs, uint32_t hd) { return kvs <= 1024 ? 128 : cm::att_nt((int)hd); }
bool fsplit_supported(uint32_t hd) { return hd == 64 || hd == 128; }
void launch_attention_fused(uint32_t hd, uint32_t n_heads, int slots, hipStream_t s, const float* qsrc, int nh,
                            int nkv, int rope_dim, int split_half, const float* cb, const float* sb, int rs,
                            const float* qn, const float* kn, float eps, uint16_t* kc, uint16_t* vc, int layer,
                            int kvs, const uint32_t* pos, float scale, uint64_t* sct, float* att,
                            int8_t* xq, float* xs, cm::OProj op) {
  if (!fsplit_supported(hd)) {
    g_launch_error = "fused split attention: head_dim " + std::to_string(hd) + " has no instantiation";
    return;
  }
  const int sl = fsplit_sl((uint32_t)kvs, hd);
  const int nsl = (kvs + sl - 1) / sl;
  int pb = 0;
  const int so = attn_out_slots((uint32_t)kvs, slots, &pb);
  size_t lds = (size_t)so * cm::AO_RING_GRANULES * 16 + attn_sc_bytes((uint32_t)kvs) + cm::avp_bytes(pb);
  uint32_t grid = n_heads * (uint32_t)nsl + n_heads * (hd / 32);
  if (op.q) {
    if (cm::att_nt((int)hd) != cm::AO_ROWS * 64 || !cm::ao_width_ok(op.K) || op.K != (int)(n_heads * hd)) {
      g_launch_error = "attention: no output projection body for this shape";
      return;
    }
    grid += (uint32_t)(op.rows + cm::AO_ROWS - 1) / cm::AO_ROWS;
    lds = std::max(lds, cm::ao_lds_bytes(op.K));
  } else if (op.k4nib) {
    if (cm::att_nt((int)hd) != cm::AO_ROWS * 64 || !cm::aoq_width_ok(op.K) || op.K != (int)(n_heads * hd)) {
      g_launch_error = "attention: no Q4_K output projection body for this shape";
      return;
    }
    grid += (uint32_t)(op.rows + cm::AOQ_ROWS - 1) / cm::AOQ_ROWS;
    lds = std::max(lds, cm::kq4_lds_bytes(op.K, cm::AOQ_ROWS));
  }
#define CM_ATTF(HD, PB, SL)                                                                                    \
  CM_LAUNCH((cm::k_att_fused<HD, PB, SL>), dim3(grid), dim3(cm::att_nt(HD)), lds, s, qsrc, nh, nkv, rope_dim,    \
            split_half, cb, sb, rs, qn, kn, eps, kc, vc, layer, kvs, pos, scale, sct, nsl, att, xq, xs, so, op)
#define CM_ATTF_PB(HD, SL)           \
  if (pb == 256) CM_ATTF(HD, 256, SL); \
  else if (pb == 128) CM_ATTF(HD, 128, SL); \
  else CM_ATTF(HD, 64, SL);
  if (hd == 64) {
    if (sl == 128) { CM_ATTF_PB(64, 128) } else { CM_ATTF_PB(64, 1024) }
  } else {
    if (sl == 128) { CM_ATTF_PB(128, 128) } else { CM_ATTF_PB(128, 1024) }
  }
#undef CM_ATTF_PB
#undef CM_ATTF
}

// The attention of this step: the split kernels from att_split_min positions on.
bool att_split(const camelid_hip_engine* e) {
  if (e->att_mode >= 0) return e->att_mode == 1;
  return e->att_split_min && (uint64_t)e->cur_pos + 1 >= e->att_split_min;
}

// rows > 1: a [rows][n] batch, one workgroup per row (no read-ahead).
// kd/kq/kbs (optional, n % 256 == 0): also the Q8_K quantization of the normalized rows.
void launch_rmsnorm_quant(const float* x, const float* w, uint32_t n, float eps, int8_t* xq, float* xs, float* y,
                          hipStream_t s, cm::Prefetch pf = cm::Prefetch{nullptr, 0, nullptr, 0}, uint32_t rows = 1,
                          float* kd = nullptr,
                          int8_t* kq = nullptr, int32_t* kbs = nullptr) {
  if (rows != 1) pf = cm::Prefetch{nullptr, 0, nullptr, 0};
  const uint32_t grid = 1 + (pf.a_lines ? PREFETCH_WGS : 0);
  switch (cm::rms_chunk((int)n)) {
#define CM_RMS(C)                                                                                                   \
  case C:                                                                                                           \
    CM_LAUNCH(cm::k_rmsnorm_quant<C>, dim3(grid, rows), dim3(cm::RMS_NT), 0, s, x, w, (int)n, eps, xq, xs, y, pf, \
              kd, kq, kbs);                                                                                         \
    break;
    CM_RMS_CHUNKS(CM_RMS)
#undef CM_RMS
  }
}

// LDS of the attention kernel: the score vector (align4(kvs) floats) plus a V ring of 2..4
// chunks of 32 KB; 0 when even two chunks do not fit beside the scores.
// The largest static LDS of the decode attention kernels (the dynamic ring and score vector
// come on top of it), read from the compiled kernels.
// Without a device (the host-only preflight), the static LDS of the attention kernels is taken
// as this bound (the compiled kernels use at most 8832 bytes) and the LDS of a workgroup as
// gfx950's 160 KB.
constexpr long ATT_STATIC_LDS_BOUND = 16384;
constexpr int GFX950_LDS_PER_WORKGROUP = 160 * 1024;
long attn_static_lds() {
  static long bytes = -1;
  if (bytes < 0) {
    long m = 0;
    hipFuncAttributes a;
#define CM_ATT_LDS(HD, F)                                                                          \
  if (hipFuncGetAttributes(&a, reinterpret_cast<const void*>(&cm::k_attention<HD, F>)) == hipSuccess) \
    m = std::max<long>(m, (long)a.sharedSizeBytes);                                                 \
  else                                                                                              \
    m = std::max<long>(m, ATT_STATIC_LDS_BOUND);
    CM_ATT_LDS(64, true) CM_ATT_LDS(64, false) CM_ATT_LDS(128, true) CM_ATT_LDS(128, false)
    CM_ATT_LDS(256, true) CM_ATT_LDS(256, false)
#undef CM_ATT_LDS
#define CM_ATTO_LDS(HD)                                                                      \
  if (hipFuncGetAttributes(&a, reinterpret_cast<const void*>(&cm::k_att_out<HD, 128>)) == hipSuccess) \
    m = std::max<long>(m, (long)a.sharedSizeBytes);                                           \
  else                                                                                        \
    m = std::max<long>(m, ATT_STATIC_LDS_BOUND);
    CM_ATTO_LDS(64) CM_ATTO_LDS(128) CM_ATTO_LDS(256)
#undef CM_ATTO_LDS
#define CM_ATTF_LDS(HD, SL)                                                                                 \
  if (hipFuncGetAttributes(&a, reinterpret_cast<const void*>(&cm::k_att_fused<HD, 64, SL>)) == hipSuccess) \
    m = std::max<long>(m, (long)a.sharedSizeBytes);                                                         \
  else                                                                                                      \
    m = std::max<long>(m, ATT_STATIC_LDS_BOUND);
    CM_ATTF_LDS(64, 128) CM_ATTF_LDS(64, 1024) CM_ATTF_LDS(128, 128) CM_ATTF_LDS(128, 1024)
#undef CM_ATTF_LDS
    bytes = m;
  }
  return bytes;
}

// LDS per workgroup of the device (read once; the gfx950 figure without a device).
long attn_lds_limit() {
  static int limit = -1;
  if (limit < 0) {
    int dev = 0, v = 0;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess)
      v = GFX950_LDS_PER_WORKGROUP;
    limit = v;
  }
  return limit;
}

// host_only: the figures of the device-free preflight (gfx950's LDS per workgroup and the
// bound on the kernels' static LDS), with no HIP call.
int attn_ring_slots(uint32_t kvs, bool host_only) {
  const long room = (host_only ? (long)GFX950_LDS_PER_WORKGROUP - ATT_STATIC_LDS_BOUND
                               : attn_lds_limit() - attn_static_lds()) -
                    (long)attn_sc_bytes(kvs);
  const long slots = std::min<long>(4, room / (cm::ATT_RING_GRANULES * 16));
  // the split output kernel also holds its product buffers (64-position blocks at least),
  // and two ring chunks beside them
  const long out_slots = (room - (long)cm::avp_bytes(64)) / (cm::ATT_RING_GRANULES * 16);
  return slots >= 2 && out_slots >= 2 ? (int)slots : 0;
}

// Ring slots and product block of the split output kernel, whose product buffers take LDS
// beside the V ring: three 16 KB chunks (more chunks in flight measured slower) beside the
// largest product block of 256, 128, 64 positions that leaves room for them; the block size
// sets the number of workgroup barriers of the output chain (C4, 8K positions: 128 -> 256
// positions per block, 225.8 -> 239.6 tok/s).  attn_ring_slots admitted kvs only with room
// for two 32 KB chunks beside 64-position blocks, so at least three 16 KB chunks fit.
int attn_out_slots(uint32_t kvs, int slots, int* pb) {
  (void)slots;
  const long room = (long)attn_lds_limit() - attn_static_lds() - (long)attn_sc_bytes(kvs);
  constexpr long chunk = (long)cm::AO_RING_GRANULES * 16;
  *pb = 64;
  for (int b : {256, 128})
    if ((room - (long)cm::avp_bytes(b)) / chunk >= 3) {
      *pb = b;
      break;
    }
  return (int)std::min<long>(3, (room - (long)cm::avp_bytes(*pb)) / chunk);
}

// Algorithmic bytes of one K-quant GEMV launch: superblocks (144 or 210 B per 256 values),
// the Q8_K activation (K + K/256 * 4 + K/32 * 4 bytes), the output (+ residual).
double kq_bytes(const KMat& m, bool resid) {
  return (double)m.rows * (m.k / 256) * kq_block_bytes(m.quant) + m.k * (1.0 + 4.0 / 256 + 4.0 / 32) +
         m.rows * (resid ? 8.0 : 4.0);
}

// K-quant GEMV (+ residual, + per-workgroup argmax partials when part_v is set); returns
// the number of workgroups.
// xf (Q4_K only): the activation in f32, quantized to Q8_K inside the GEMV.
uint32_t launch_kgemv(const KMat& m, const float* yd, const int8_t* yq, const int32_t* ybs, float* y,
                      const float* resid, float* part_v, uint32_t* part_i, hipStream_t s,
                      const float* xf = nullptr) {
  const int rpw = m.rows >= 16384 ? 2 : 1;
  const uint32_t R = 4 * rpw, grid = (m.rows + R - 1) / R;
  if (m.quant == CAMELID_Q4_K) {
    const size_t lds = cm::kq4_lds_bytes((int)m.k, (int)R);
    const int it = (int)(m.k / 32 + 63) / 64;  // 16-byte pieces per lane and row (k <= 16384: <= 8)
    if (xf) {  // (f32 activation: one row per wave)
      switch (rpw == 1 ? it : 0) {
#define CM_Q4X(IT)                                                                                               \
  case IT:                                                                                                       \
    CM_LAUNCH((cm::k_gemv_q4k<IT, 1, true>), dim3(grid), dim3(cm::KQ_NT), lds, s, m.a, m.b, (int)m.rows, (int)m.k, \
              yd, yq, ybs, y, resid, part_v, part_i, xf);                                                        \
    break;
        CM_Q4X(1) CM_Q4X(2) CM_Q4X(3) CM_Q4X(4) CM_Q4X(5) CM_Q4X(6) CM_Q4X(7) CM_Q4X(8)
#undef CM_Q4X
        default:
          g_launch_error = "Q4_K GEMV of an f32 activation: " + std::to_string(m.rows) + " x " + std::to_string(m.k) +
                           " has no kernel instantiation";
          return 0;
      }
      return grid;
    }
    switch (it * 2 + (rpw == 2)) {
#define CM_Q4(IT, RPW)                                                                                           \
  case IT * 2 + (RPW == 2):                                                                                      \
    CM_LAUNCH((cm::k_gemv_q4k<IT, RPW>), dim3(grid), dim3(cm::KQ_NT), lds, s, m.a, m.b, (int)m.rows, (int)m.k, yd, \
              yq, ybs, y, resid, part_v, part_i, nullptr);                                                       \
    break;
      CM_Q4(1, 1) CM_Q4(1, 2) CM_Q4(2, 1) CM_Q4(2, 2) CM_Q4(3, 1) CM_Q4(3, 2) CM_Q4(4, 1) CM_Q4(4, 2)
      CM_Q4(5, 1) CM_Q4(6, 1) CM_Q4(7, 1) CM_Q4(8, 1)
      CM_Q4(5, 2) CM_Q4(6, 2) CM_Q4(7, 2) CM_Q4(8, 2)
#undef CM_Q4
      default:
        g_launch_error = "Q4_K GEMV: row width " + std::to_string(m.k) + " has no kernel instantiation";
        return 0;
    }
  } else {
    const size_t lds = cm::kq6_lds_bytes((int)m.k, (int)R);
    if (rpw == 2)
      CM_LAUNCH(cm::k_gemv_q6k<2>, dim3(grid), dim3(cm::KQ_NT), lds, s, m.a, m.b, m.sc, m.d, (int)m.rows, (int)m.k,
                yd, yq, y, resid, part_v, part_i);
    else
      CM_LAUNCH(cm::k_gemv_q6k<1>, dim3(grid), dim3(cm::KQ_NT), lds, s, m.a, m.b, m.sc, m.d, (int)m.rows, (int)m.k,
                yd, yq, y, resid, part_v, part_i);
  }
  return grid;
}

void gemv(camelid_hip_engine* e, const Q8Mat& m, float* y, const float* resid, const int8_t* xq = nullptr,
          const float* xs = nullptr) {
  ProfScope ps(e, P_GEMV, q8_bytes(m, resid != nullptr));
  launch_gemv(m, xq ? xq : e->xq, xs ? xs : e->xs, y, resid, e->stream);
}

void rmsnorm(camelid_hip_engine* e, const float* w, const Q8Mat* next) {
  const uint32_t n = e->d.hidden;
  ProfScope ps(e, P_NORM, n * 8.0 + n * 34.0 / 32.0);
  launch_rmsnorm_quant(e->h, w, n, e->d.eps, e->xq, e->xs, nullptr, e->stream,
                       prefetch_of(e->read_ahead ? next : nullptr));
}

// Q8_K quantization of n values (the K-quant projections' activation).
void quant_q8k(camelid_hip_engine* e, const float* x, uint32_t n) {
  ProfScope ps(e, P_NORM, n * 4.0 + n * (1.0 + 4.0 / 256 + 4.0 / 32));
  CM_LAUNCH(cm::k_quantize_q8k, dim3(n / 256), dim3(256), 0, e->stream, x, e->kd, e->kq, e->kbs);
}

// One projection in its own format: Q8_0 from the Q8_0 activation, K-quants from the Q8_K
// one, or (xf given) from the f32 activation, which a Q4_K GEMV of one row per wave (rows <
// 16384) quantizes itself.
void proj(camelid_hip_engine* e, const Proj& p, float* y, const float* resid, const float* xf = nullptr) {
  if (p.quant == CAMELID_Q8_0) {
    gemv(e, p.q8, y, resid);
    return;
  }
  if (xf && (p.quant == CAMELID_Q6_K || p.kq.rows >= 16384)) {
    quant_q8k(e, xf, p.kq.k);
    xf = nullptr;
  }
  ProfScope ps(e, P_GEMV, kq_bytes(p.kq, resid != nullptr));
  launch_kgemv(p.kq, e->kd, e->kq, e->kbs, y, resid, nullptr, nullptr, e->stream, xf);
}

// Whether the split attention runs as one launch (k_att_fused): on by default where it is
// instantiated, and only with the read-ahead off (the two-launch path keeps its read-ahead).
// The launch's score and output workgroups must also fit on the device's CUs at once (one
// workgroup per CU): with more score slices than that (C4's 8K context: 288 score + 128 output
// workgroups) the output workgroups start only as score workgroups retire, and the two launches
// measured faster (212.1 vs 204.1 tok/s); within it the one launch is (C5 372.0 vs 365.3).
// The count includes the output projection's workgroups when the Q8_0 O projection rides in
// the launch.  The score words are tagged with (position + 1, layer) in 24 + 8 bits, so the
// layer count and the cache length must fit those fields, as for the projection's words.
bool ao_enabled(camelid_hip_engine* e);
bool att_fused_split(camelid_hip_engine* e) {
  if (!(e->att_fsplit && fsplit_supported(e->d.head_dim) && !e->read_ahead && e->att_sct)) return false;
  if (e->d.n_layers > 255 || e->kvs >= (1u << 24) - 1) return false;
  const uint32_t sl = (uint32_t)fsplit_sl(e->kvs, e->d.head_dim);
  uint32_t wgs = e->d.n_heads * ((e->kvs + sl - 1) / sl) + e->d.n_heads * (e->d.head_dim / 32);
  if (ao_enabled(e)) wgs += (e->d.hidden + cm::AO_ROWS - 1) / cm::AO_ROWS;
  return wgs <= e->n_cus;
}

// The decode attention of layer l for the token at StepState.pos (QK-norm, RoPE and the K/V
// store fused): one workgroup per head, or the split kernels for long contexts.
void decode_attention(camelid_hip_engine* e, uint32_t l, const float* cos_base, const float* sin_base,
                      int rope_stride, float scale, cm::Prefetch pf, cm::OProj op = cm::OProj{}) {
  const camelid_hip_dims& d = e->d;
  const LayerW& L = e->layers[l];
  if (att_split(e) && att_fused_split(e))
    launch_attention_fused(d.head_dim, d.n_heads, e->att_slots, e->stream, e->qkv, (int)d.n_heads, (int)d.n_kv_heads,
                           (int)d.rope_dim, (int)d.split_half_pairing, cos_base, sin_base, rope_stride, L.q_norm,
                           L.k_norm, d.eps, e->kc, e->vc, (int)l, (int)e->kvs, &e->st->pos, scale, e->att_sct,
                           e->att, e->xq, e->xs, op);
  else if (att_split(e))
    launch_attention_split<true>(d.head_dim, d.n_heads, e->att_slots, e->stream, e->qkv, (int)d.n_heads,
                                 (int)d.n_kv_heads, (int)d.rope_dim, (int)d.split_half_pairing, cos_base, sin_base,
                                 rope_stride, L.q_norm, L.k_norm, d.eps, e->kc, e->vc, (int)l, (int)e->kvs,
                                 &e->st->pos, scale, e->att_sc, e->att_mx, e->att, e->xq, e->xs, pf, op);
  else
    launch_attention<true>(d.head_dim, d.n_heads, e->att_slots, e->stream, e->qkv, (int)d.n_heads,
                           (int)d.n_kv_heads, (int)d.rope_dim, (int)d.split_half_pairing, cos_base, sin_base,
                           rope_stride, L.q_norm, L.k_norm, d.eps, e->kc, e->vc, (int)l, (int)e->kvs, &e->st->pos,
                           scale, e->att, e->xq, e->xs, pf, e->att_dg, op);
}

// Tagged activation words of the attention's output projection: K / 4 quant words and K / 32
// scales (Q8_0 W_o), or K f32 values (Q4_K W_o).
size_t ao_words(const camelid_hip_engine* e) {
  const size_t nq = (size_t)e->d.n_heads * e->d.head_dim;
  return std::max(nq / 4 + nq / 32 + 1, nq);
}

// Whether the Q8_0 decode layers compute the output projection inside the single-workgroup
// attention launch (cm::att_oproj; CAMELID_HIP_ATT_O=0 turns it off): every layer must be a
// Q8_0 layer whose W_o width has a projection body, with the read-ahead off (its workgroups
// take the same place in the grid).
bool ao_enabled(camelid_hip_engine* e) {
  if (e->ao_state < 0) {
    const camelid_hip_dims& d = e->d;
    // (tags: the layer in 8 bits, position + 1 in 24)
    bool ok = e->att_o_fused && !e->read_ahead && d.n_layers <= 255 && e->kvs < (1u << 24) - 1 &&
              cm::att_nt((int)d.head_dim) == cm::AO_ROWS * 64 && cm::ao_width_ok((int)(d.n_heads * d.head_dim)) &&
              e->ao_words != nullptr;
    for (uint32_t l = 0; ok && l < d.n_layers; ++l) {
      const LayerW& L = e->layers[l];
      ok = L.set && !L.generic && L.o.k == d.n_heads * d.head_dim && L.o.rows == d.hidden;
    }
    e->ao_state = ok ? 1 : 0;
  }
  return e->ao_state == 1;
}

// The two-launch split attention takes the Q8_0 output projection's workgroups in its output
// launch where they fit beside the output workgroups (cm::k_att_out, AO_SPLIT_RPW rows per wave).
bool ao_split_fits(camelid_hip_engine* e) {
  const uint32_t aor = (uint32_t)(cm::AO_ROWS * cm::AO_SPLIT_RPW);
  return ao_enabled(e) && e->d.n_heads * (e->d.head_dim / 32) + (e->d.hidden + aor - 1) / aor <= e->n_cus;
}

// Whether the K-quant decode layers compute a Q4_K output projection inside the one-launch
// split attention (cm::att_oproj_q4k; CAMELID_HIP_ATT_O=0 turns it off): every layer must be a
// K-quant layer whose W_o is Q4_K of width n_heads * head_dim = 4096 and hidden rows, with the
// read-ahead off.  It rides only in launches where it fits the CUs (ao4_rides).
bool ao4_enabled(camelid_hip_engine* e) {
  if (e->ao4_state < 0) {
    const camelid_hip_dims& d = e->d;
    bool ok = e->att_o_fused && !e->read_ahead && d.n_layers <= 255 && e->kvs < (1u << 24) - 1 &&
              cm::att_nt((int)d.head_dim) == cm::AO_ROWS * 64 && cm::aoq_width_ok((int)(d.n_heads * d.head_dim)) &&
              e->ao_words != nullptr && d.n_layers > 0;
    for (uint32_t l = 0; ok && l < d.n_layers; ++l) {
      const LayerW& L = e->layers[l];
      ok = L.set && L.generic && L.p[3].quant == CAMELID_Q4_K && L.p[3].kq.k == d.n_heads * d.head_dim &&
           L.p[3].kq.rows == d.hidden;
    }
    e->ao4_state = ok ? 1 : 0;
  }
  return e->ao4_state == 1;
}
// The one-launch split attention takes the Q4_K projection's workgroups where they fit the CUs
// once the score slices retire (those come first and finish long before the output sums: the
// projection workgroups that find no free CU start then, and still have their weights in
// registers before the attention output is ready).
bool ao4_rides(camelid_hip_engine* e) {
  if (!ao4_enabled(e) || !att_fused_split(e)) return false;
  const uint32_t sl = (uint32_t)fsplit_sl(e->kvs, e->d.head_dim);
  const uint32_t outs = e->d.n_heads * (e->d.head_dim / 32);
  const uint32_t wgs = outs + (e->d.hidden + cm::AOQ_ROWS - 1) / cm::AOQ_ROWS;
  (void)sl;
  return wgs <= e->n_cus;
}

// The K-quant layer shape the norm-fused launches take: hidden 4096 (the norm workgroup's 512 x
// 8 values), q|k stacked Q4_K + v Q6_K as k_gemv_qk4_v6 takes them, gate|up stacked Q4_K.
bool nf_layer_ok(const camelid_hip_engine* e, const LayerW& L) {
  const camelid_hip_dims& d = e->d;
  if (!L.generic || d.hidden != (uint32_t)cm::NF_NT * cm::NQ_C) return false;
  const KMat& qk = L.p[0].kq;
  const KMat& v6 = L.p[2].kq;
  const KMat& gu = L.p[4].kq;
  return e->qkv_merged && L.qk_stacked && L.p[0].quant == CAMELID_Q4_K && L.p[2].quant == CAMELID_Q6_K &&
         qk.rows < 16384 && v6.rows < 16384 && qk.k == d.hidden && v6.k == d.hidden && L.gu_stacked &&
         L.p[4].quant == CAMELID_Q4_K && gu.k == d.hidden;
}

// Whether the decode layers run the norm-fused launches: every layer must (their two flag
// slots rely on the launches of the two kinds strictly alternating).
bool nf_enabled(camelid_hip_engine* e) {
  if (e->nf_state < 0) {
    bool ok = e->kq_norm_fused && e->d.n_layers > 0;
    for (uint32_t l = 0; ok && l < e->d.n_layers; ++l) ok = e->layers[l].set && nf_layer_ok(e, e->layers[l]);
    e->nf_state = ok ? 1 : 0;
  }
  return e->nf_state == 1;
}

// Before a call's decode steps (not inside a captured graph): the flag slots start cleared (a
// step cut short by an error leaves one set) and the handoff error word is cleared.
// The same for the attention's output-projection counters (one per layer).
int nf_begin(camelid_hip_engine* e) {
  const bool nf = nf_enabled(e), ao = ao_enabled(e), fs = att_fused_split(e), ao4 = ao4_rides(e);
  if (fs) HIP_TRY(e, hipMemsetAsync(e->att_sct, 0, (size_t)e->d.n_heads * e->kvs * 8, e->stream));
  if (!nf && !ao && !fs) return 0;
  static const uint32_t zero = 0;
  if (nf) HIP_TRY(e, hipMemsetAsync(e->nf_slots, 0, cm::NF_WORDS * 4, e->stream));
  if (ao || ao4) HIP_TRY(e, hipMemsetAsync(e->ao_words, 0, ao_words(e) * 8, e->stream));
  HIP_TRY(e, hipMemcpyToSymbolAsync(HIP_SYMBOL(cm::g_handoff_error), &zero, 4, 0, hipMemcpyHostToDevice, e->stream));
  return 0;
}
// After the call's work is enqueued: the error word comes back with the call's own sync.
int nf_end(camelid_hip_engine* e) {
  if (e->nf_state != 1 && e->ao_state != 1 && !att_fused_split(e)) return 0;
  HIP_TRY(e, hipMemcpyFromSymbolAsync(e->p_err, HIP_SYMBOL(cm::g_handoff_error), 4, 0, hipMemcpyDeviceToHost,
                                      e->stream));
  e->err_pending = true;
  return 0;
}
// After the call's sync: only a word that nf_end asked for in this call is read.
int nf_failed(camelid_hip_engine* e) {
  const bool pending = e->err_pending;
  e->err_pending = false;
  if (pending && *e->p_err) {
    e->filled = 0;
    return fail(e, "in-launch handoff: a workgroup's wait for another workgroup of its launch timed out");
  }
  return 0;
}

// A layer with K-quant projections (forward_layer_timed, inference.rs:6228-6807): the same
// order as run_layer, with each projection in its own format; the RMSNorm kernel also writes
// the normalized row, which is quantized to Q8_K when a K-quant projection reads it.
void run_layer_generic(camelid_hip_engine* e, uint32_t l, const float* cos_base, const float* sin_base,
                       int rope_stride, float scale) {
  const camelid_hip_dims& d = e->d;
  const LayerW& L = e->layers[l];
  hipStream_t s = e->stream;
  const uint32_t nq = d.n_heads * d.head_dim, nkv = d.n_kv_heads * d.head_dim;
  auto is_k = [&](int i) { return L.p[i].quant != CAMELID_Q8_0; };
  // the RMSNorm kernel writes the Q8_K activation itself when a K-quant projection reads it
  // read-ahead of the projection that runs next, in its own format
  auto ahead = [&](const Proj& p) {
    if (!e->read_ahead) return prefetch_of((const Q8Mat*)nullptr);
    return p.quant == CAMELID_Q8_0 ? prefetch_of(&p.q8) : prefetch_of(&p.kq);
  };
  auto norm = [&](const float* w, bool k8, cm::Prefetch pf) {
    ProfScope ps(e, P_NORM, d.hidden * 8.0 + d.hidden * 34.0 / 32.0 + (k8 ? d.hidden * (1.0 + 4.0 / 256 + 4.0 / 32) : 0.0));
    launch_rmsnorm_quant(e->h, w, d.hidden, d.eps, e->xq, e->xs, nullptr, s, pf, 1, k8 ? e->kd : nullptr,
                         k8 ? e->kq : nullptr, k8 ? e->kbs : nullptr);
  };
  const bool nf = e->nf_state == 1;  // (decided by nf_begin before the call's steps)
  const KMat& qk = L.p[0].kq;
  const KMat& v6 = L.p[2].kq;
  if (nf) {
    // the attention RMSNorm inside the q|k + v launch (workgroup 0), flag slot 0
    ProfScope ps(e, P_GEMV, kq_bytes(qk, false) + kq_bytes(v6, false) - qk.k * (1.0 + 4.0 / 256 + 4.0 / 32) +
                                d.hidden * 8.0);
    constexpr uint32_t R = cm::NF_NT / 64;  // rows per workgroup: one per wave
    const uint32_t g4 = (qk.rows + R - 1) / R, g6 = (v6.rows + R - 1) / R;
    const size_t lds = std::max({cm::kq4_lds_bytes((int)qk.k, R), cm::kq6_lds_bytes((int)qk.k, R),
                                 cm::norm_q8k_lds_bytes((int)qk.k)});
    const int it = (int)(qk.k / 32 + 63) / 64;
    if (it == 2)
      CM_LAUNCH(cm::k_norm_qk4_v6<2>, dim3(1 + g4 + g6), dim3(cm::NF_NT), lds, s, e->h, L.attn_norm, d.eps,
                e->nf_slots, 0, e->kd, e->kq, e->kbs, qk.a, qk.b, (int)qk.rows, e->qkv, (int)g4, v6.a, v6.b, v6.sc,
                v6.d, (int)v6.rows, e->qkv + nq + nkv, (int)qk.k);
    else
      g_launch_error = "norm-fused q|k+v GEMV: row width " + std::to_string(qk.k) + " has no instantiation";
  } else {
  norm(L.attn_norm, is_k(0) || is_k(1) || is_k(2), ahead(L.p[0]));
  if (e->qkv_merged && L.qk_stacked && L.p[0].quant == CAMELID_Q4_K && L.p[2].quant == CAMELID_Q6_K &&
      qk.rows < 16384 && v6.rows < 16384 && qk.k == v6.k && qk.k / 32 <= 8 * 64) {
    // q|k and v in one launch (both from the Q8_K activation the norm wrote)
    ProfScope ps(e, P_GEMV, kq_bytes(qk, false) + kq_bytes(v6, false) - qk.k * (1.0 + 4.0 / 256 + 4.0 / 32));
    const uint32_t g4 = (qk.rows + 3) / 4, g6 = (v6.rows + 3) / 4;
    const size_t lds = std::max(cm::kq4_lds_bytes((int)qk.k, 4), cm::kq6_lds_bytes((int)qk.k, 4));
    const int it = (int)(qk.k / 32 + 63) / 64;
    switch (it) {
#define CM_QKV(IT)                                                                                            \
  case IT:                                                                                                    \
    CM_LAUNCH(cm::k_gemv_qk4_v6<IT>, dim3(g4 + g6), dim3(cm::KQ_NT), lds, s, qk.a, qk.b, (int)qk.rows, e->qkv, \
              (int)g4, v6.a, v6.b, v6.sc, v6.d, (int)v6.rows, e->qkv + nq + nkv, (int)qk.k, e->kd, e->kq, e->kbs); \
    break;
      CM_QKV(1) CM_QKV(2) CM_QKV(3) CM_QKV(4) CM_QKV(5) CM_QKV(6) CM_QKV(7) CM_QKV(8)
#undef CM_QKV
      default:
        g_launch_error = "Q4_K|Q6_K qkv GEMV: row width " + std::to_string(qk.k) + " has no kernel instantiation";
        break;
    }
  } else {
    proj(e, L.p[0], e->qkv, nullptr);  // q, or q|k stacked
    if (!L.qk_stacked) proj(e, L.p[1], e->qkv + nq, nullptr);
    proj(e, L.p[2], e->qkv + nq + nkv, nullptr);
  }
  }
  const double att_bytes = (nq + 2.0 * nkv) * 4 + 2.0 * nkv * 2 * (e->cur_pos + 1) + nq * (4 + 34.0 / 32.0);
  if (att_split(e) && ao4_rides(e)) {
    // the Q4_K output projection's workgroups ride in the split attention launch
    ProfScope ps(e, P_ATTN, att_bytes + kq_bytes(L.p[3].kq, true));
    cm::OProj op{nullptr, nullptr, (int)L.p[3].kq.rows, (int)L.p[3].kq.k, e->h, e->h, nullptr, nullptr, (int)l};
    op.k4nib = L.p[3].kq.a;
    op.k4hdr = L.p[3].kq.b;
    op.xf_t = e->ao_words;
    decode_attention(e, l, cos_base, sin_base, rope_stride, scale, cm::Prefetch{nullptr, 0, nullptr, 0}, op);
  } else {
    {
      ProfScope ps(e, P_ATTN, att_bytes);
      decode_attention(e, l, cos_base, sin_base, rope_stride, scale, ahead(L.p[3]));
    }
    proj(e, L.p[3], e->h, e->h, is_k(3) ? e->att : nullptr);
  }
  if (nf) {
    // the FFN RMSNorm inside the gate|up launch (workgroup 0), flag slot 1
    const KMat& gu = L.p[4].kq;
    ProfScope ps(e, P_GEMV, kq_bytes(gu, false) - gu.k * (1.0 + 4.0 / 256 + 4.0 / 32) + d.hidden * 8.0);
    const int rpw = gu.rows >= 16384 ? 2 : 1;
    const uint32_t R = (cm::NF_NT / 64) * rpw, grid = (gu.rows + R - 1) / R;
    const size_t lds = std::max(cm::kq4_lds_bytes((int)gu.k, (int)R), cm::norm_q8k_lds_bytes((int)gu.k));
    const int it = (int)(gu.k / 32 + 63) / 64;
    if (it == 2 && rpw == 2)
      CM_LAUNCH((cm::k_norm_gemv_q4k<2, 2>), dim3(1 + grid), dim3(cm::NF_NT), lds, s, e->h, L.ffn_norm, d.eps,
                e->nf_slots, 1, e->kd, e->kq, e->kbs, gu.a, gu.b, (int)gu.rows, (int)gu.k, e->gu);
    else if (it == 2)
      CM_LAUNCH((cm::k_norm_gemv_q4k<2, 1>), dim3(1 + grid), dim3(cm::NF_NT), lds, s, e->h, L.ffn_norm, d.eps,
                e->nf_slots, 1, e->kd, e->kq, e->kbs, gu.a, gu.b, (int)gu.rows, (int)gu.k, e->gu);
    else
      g_launch_error = "norm-fused gate|up GEMV: row width " + std::to_string(gu.k) + " has no instantiation";
  } else {
    norm(L.ffn_norm, is_k(4) || is_k(5), ahead(L.p[4]));
    proj(e, L.p[4], e->gu, nullptr);  // gate, or gate|up stacked
    if (!L.gu_stacked) proj(e, L.p[5], e->gu + d.ffn_dim, nullptr);
  }
  {
    ProfScope ps(e, P_SILU, d.ffn_dim * 12.0 + d.ffn_dim * 34.0 / 32.0);
    const cm::Prefetch pf = ahead(L.p[6]);
    const bool k8 = is_k(6);
    CM_LAUNCH(cm::k_silu_mul_quant, dim3((d.ffn_dim + 255) / 256 + (pf.a_lines ? PREFETCH_WGS : 0)), dim3(256), 0, s,
              e->gu, (int)d.ffn_dim, k8 ? (int8_t*)nullptr : e->xq, k8 ? (float*)nullptr : e->xs, (float*)nullptr,
              pf, k8 ? e->kd : nullptr, k8 ? e->kq : nullptr, k8 ? e->kbs : nullptr);
  }
  proj(e, L.p[6], e->h, e->h);
}

// One transformer layer at StepState.pos; RoPE tables at cos_base + pos*rope_stride.
void run_layer(camelid_hip_engine* e, uint32_t l, const float* cos_base, const float* sin_base, int rope_stride,
               float scale) {
  const camelid_hip_dims& d = e->d;
  const LayerW& L = e->layers[l];
  if (L.generic) {
    run_layer_generic(e, l, cos_base, sin_base, rope_stride, scale);
    return;
  }
  hipStream_t s = e->stream;
  const double nq = (double)d.n_heads * d.head_dim, nkv = (double)d.n_kv_heads * d.head_dim;
  // the RMSNorms inside the qkv and gate/up GEMVs (norm_q8_lds) for the widths instantiated
  const bool norm_fused = e->norm_fused && cm::gu_fused_k((int)d.hidden);
  const bool gu_norm = norm_fused && e->gu_fused && cm::gu_norm_k((int)d.hidden);
  if (norm_fused) {
    ProfScope ps(e, P_GEMV, q8_bytes(L.qkv, false) + d.hidden * 8.0);
    // the attention that follows reads this layer's K/V rows from its XCDs' L2
    cm::KvAhead kva{};
    if (e->kv_ahead && !att_split(e))
      kva = cm::KvAhead{e->kc, e->vc, &e->st->pos, (int)l, (int)d.n_heads, (int)d.n_kv_heads, (int)d.head_dim,
                        (int)e->kvs, 1};
    launch_gemv_norm(L.qkv, e->h, L.attn_norm, d.eps, e->qkv, s, kva);
  } else {
    rmsnorm(e, L.attn_norm, &L.qkv);
    gemv(e, L.qkv, e->qkv, nullptr);
  }
  const double att_bytes = (nq + 2 * nkv) * 4 + 2.0 * nkv * 2 * (e->cur_pos + 1) + nq * (4 + 34.0 / 32.0);
  if (ao_enabled(e) && (!att_split(e) || att_fused_split(e) || ao_split_fits(e))) {
    // the output projection's workgroups ride in the attention launch (attention + W_o bytes)
    ProfScope ps(e, P_ATTN, att_bytes + q8_bytes(L.o, true));
    const size_t nqw = (size_t)d.n_heads * d.head_dim / 4;
    const cm::OProj op{L.o.q, L.o.d, (int)L.o.rows, (int)L.o.k, e->h, e->h, e->ao_words, e->ao_words + nqw, (int)l};
    decode_attention(e, l, cos_base, sin_base, rope_stride, scale, cm::Prefetch{nullptr, 0, nullptr, 0}, op);
  } else {
    {
      ProfScope ps(e, P_ATTN, att_bytes);
      decode_attention(e, l, cos_base, sin_base, rope_stride, scale, prefetch_of(e->read_ahead ? &L.o : nullptr));
    }
    gemv(e, L.o, e->h, e->h);
  }
  if (!gu_norm) rmsnorm(e, L.ffn_norm, &L.gu);
  if (e->gu_fused) {
    ProfScope ps(e, P_GEMV, q8_bytes(L.gu, false) - L.gu.rows * 4.0 + d.ffn_dim * 34.0 / 32.0 +
                                (gu_norm ? d.hidden * 8.0 - d.hidden * 34.0 / 32.0 : 0.0));
    const uint32_t groups = d.ffn_dim / 32;
    // norm-fused: one 1024-thread workgroup fits a CU, so where the groups exceed the CUs one
    // workgroup per CU takes groups b, b + CUs, ... in turn (the next group's weights streaming
    // during the current one's fold; CAMELID_HIP_GU_LOOP=0: one group per workgroup, in rounds).
    // Measured on the Mistral-7B shape (448 groups): 256 workgroups 253.1, 224 of two groups each
    // 252.0, two rounds 250.8 tok/s.
    const uint32_t ngrid = (e->gu_loop && groups > e->n_cus) ? e->n_cus : groups;
    const bool loop = ngrid < groups;  // (the looping instantiation)
    switch (d.hidden) {
#define CM_GU(K)                                                                                                 \
  case K:                                                                                                        \
    if (cm::gu_norm_k(K) && gu_norm && loop)                                                                    \
      CM_LAUNCH((cm::k_gemv_gu_silu<K, cm::GN_NT, cm::gu_norm_k(K), true>), dim3(ngrid), dim3(cm::GN_NT), 0, s,  \
                L.gu.q, L.gu.d, (const int8_t*)nullptr, (const float*)nullptr, e->h, L.ffn_norm, d.eps, e->aq,  \
                e->as, (int)groups);                                                                           \
    else if (cm::gu_norm_k(K) && gu_norm)                                                                      \
      CM_LAUNCH((cm::k_gemv_gu_silu<K, cm::GN_NT, cm::gu_norm_k(K)>), dim3(groups), dim3(cm::GN_NT), 0, s,       \
                L.gu.q, L.gu.d, (const int8_t*)nullptr, (const float*)nullptr, e->h, L.ffn_norm, d.eps, e->aq,  \
                e->as, (int)groups);                                                                           \
    else                                                                                                       \
      CM_LAUNCH((cm::k_gemv_gu_silu<K, cm::GU_NT, false>), dim3(groups), dim3(cm::GU_NT), 0, s, L.gu.q, L.gu.d,  \
                e->xq, e->xs, (const float*)nullptr, (const float*)nullptr, 0.0f, e->aq, e->as, (int)groups);  \
    break;
      CM_GU(2048) CM_GU(3072) CM_GU(4096)
#undef CM_GU
    }
  } else {
    gemv(e, L.gu, e->gu, nullptr);
    ProfScope ps(e, P_SILU, d.ffn_dim * 8.0 + d.ffn_dim * 34.0 / 32.0);
    const cm::Prefetch pf = prefetch_of(e->read_ahead ? &L.down : nullptr);
    const uint32_t grid = (d.ffn_dim + 255) / 256 + (pf.a_lines ? PREFETCH_WGS : 0);
    CM_LAUNCH(cm::k_silu_mul_quant, dim3(grid), dim3(256), 0, s, e->gu, (int)d.ffn_dim, e->xq, e->xs, nullptr, pf,
              (float*)nullptr, (int8_t*)nullptr, (int32_t*)nullptr);
  }
  if (e->gu_fused)
    gemv(e, L.down, e->h, e->h, e->aq, e->as);  // the activation quantized by the fused gate/up kernel
  else
    gemv(e, L.down, e->h, e->h);
}

void run_stack(camelid_hip_engine* e, const float* cos_base, const float* sin_base, int rope_stride, float scale) {
  const camelid_hip_dims& d = e->d;
  for (uint32_t l = 0; l < d.n_layers; ++l) {
    if (e->capture)
      (void)hipMemcpyAsync(e->hidden_cap + (size_t)l * d.hidden, e->h, d.hidden * 4, hipMemcpyDeviceToDevice,
                           e->stream);
    run_layer(e, l, cos_base, sin_base, rope_stride, scale);
  }
  if (e->capture)
    (void)hipMemcpyAsync(e->hidden_cap + (size_t)d.n_layers * d.hidden, e->h, d.hidden * 4, hipMemcpyDeviceToDevice,
                         e->stream);
}

// Final norm, lm_head and greedy argmax; advances StepState (pos+1, tok, tokens[step]).
void run_head(camelid_hip_engine* e, uint32_t* tokens, uint32_t cap) {
  uint32_t nparts;
  if (e->out_quant == CAMELID_Q8_0) {
    rmsnorm(e, e->out_norm, nullptr);
    const Q8Mat& m = e->out;
    ProfScope ps(e, P_GEMV, q8_bytes(m, false));
    nparts = launch_gemv_argmax(m, e->xq, e->xs, e->logits, e->part_v, e->part_i, e->stream);
  } else {
    {
      const double H = e->d.hidden;
      ProfScope ps(e, P_NORM, H * 8.0 + H * 34.0 / 32.0 + H * (1.0 + 4.0 / 256 + 4.0 / 32));
      launch_rmsnorm_quant(e->h, e->out_norm, e->d.hidden, e->d.eps, e->xq, e->xs, nullptr, e->stream,
                           prefetch_of(e->read_ahead ? &e->out_k : nullptr), 1,
                           e->kd, e->kq, e->kbs);
    }
    ProfScope ps(e, P_GEMV, kq_bytes(e->out_k, false));
    nparts = launch_kgemv(e->out_k, e->kd, e->kq, e->kbs, e->logits, nullptr, e->part_v, e->part_i, e->stream);
  }
  ProfScope ps(e, P_HEAD, 0.0);
  CM_LAUNCH(cm::k_argmax_finish, dim3(1), dim3(1024), 0, e->stream, e->part_v, e->part_i, (int)nparts, e->st,
                     tokens, cap);
}

void run_embed(camelid_hip_engine* e) {
  const camelid_hip_dims& d = e->d;
  ProfScope ps(e, P_EMBED, d.hidden * (34.0 / 32.0 + 4.0));
  if (e->embd_quant == CAMELID_Q4_K)
    CM_LAUNCH(cm::k_embed_q4k, dim3(d.hidden / 256), dim3(256), 0, e->stream, e->embd_k.a, e->embd_k.b,
              (int)d.hidden, e->st, e->h);
  else if (e->embd_quant == CAMELID_Q6_K)
    CM_LAUNCH(cm::k_embed_q6k, dim3(d.hidden / 256), dim3(256), 0, e->stream, e->embd_k.a, e->embd_k.b,
              e->embd_k.sc, e->embd_k.d, (int)d.hidden, e->st, e->h);
  else
    CM_LAUNCH(cm::k_embed_q8, dim3((d.hidden + 255) / 256), dim3(256), 0, e->stream, e->embd.q, e->embd.d,
              (int)d.hidden, e->st, e->h);
}

// ---------------------------------------------------------------- batched prefill
constexpr uint32_t PREFILL_CHUNK = 512;  // tokens per pass over the layers

// Scratch floats the tiled prefill attention needs for T tokens up to position pos0 + T - 1
// (its score rows: 64 per tile, one tile per TQ tokens of each KV head).
size_t attn_prefill_scratch(uint32_t n_heads, uint32_t n_kv, uint32_t T, uint32_t pos_end) {
  const uint32_t tq = (uint32_t)cm::apt_tq((int)(n_heads / n_kv));
  return (size_t)n_kv * ((T + tq - 1) / tq) * cm::APT_R * cm::apt_pitch(pos_end);
}

int ensure_prefill_buffers(camelid_hip_engine* e) {
  if (e->pf_h) return 0;
  const camelid_hip_dims& d = e->d;
  const size_t tc = PREFILL_CHUNK;
  const size_t nq = (size_t)d.n_heads * d.head_dim, nkv = (size_t)d.n_kv_heads * d.head_dim;
  const size_t act = std::max<size_t>({(size_t)d.hidden, (size_t)d.ffn_dim, nq});
  if (dev_alloc(e, &e->pf_h, tc * d.hidden) || dev_alloc(e, &e->pf_qkv, tc * (nq + 2 * nkv)) ||
      dev_alloc(e, &e->pf_q, tc * nq) || dev_alloc(e, &e->pf_gu, tc * 2 * d.ffn_dim) ||
      dev_alloc(e, &e->pf_xq, tc * act) || dev_alloc(e, &e->pf_xs, tc * act / 32))
    return 1;
  if (e->att_tile && cm::apt_hd_ok((int)d.head_dim) && d.n_heads / d.n_kv_heads <= (uint32_t)cm::APT_R &&
      dev_alloc(e, &e->pf_sc, attn_prefill_scratch(d.n_heads, d.n_kv_heads, PREFILL_CHUNK, e->kvs)))
    return 1;
  if (!e->any_kquant) return 0;
  return dev_alloc(e, &e->pf_kd, tc * act / 256) || dev_alloc(e, &e->pf_kq, tc * act) ||
         dev_alloc(e, &e->pf_kbs, tc * act / 32) || dev_alloc(e, &e->pf_att, tc * nq) ||
         dev_alloc(e, &e->pf_tmp, tc * act) || dev_alloc(e, &e->pf_kqt, cm::q6g_act_bytes((int)tc, (int)act));
}

// Tokens per launch of the multi-token Q6_K GEMV at width K (its activations and terms
// within 64 KB of LDS).
uint32_t q6m_tokens(uint32_t K) {
  uint32_t t = cm::Q6M_MAX;
  while (t > 1 && cm::gemv_q6k_multi_lds_bytes((int)K, (int)t) > 65536) --t;
  return t;
}

// A K-quant projection over T tokens with Q8_K activation rows (kd [T][k/256], kq [T][k]):
// y[t * ldy + row] (+ resid, same stride).  Q4_K: the matrix-core GEMM; Q6_K: for more than
// Q6M_MAX tokens the class-major GEMM (needs m.w2 and xt, cm::q6g_act_bytes(T, k) bytes for
// the class-major copy of kq) or else the sparse-MFMA GEMM, for fewer the multi-token GEMV.
void launch_kgemm(const KMat& m, uint32_t T, const float* kd, const int8_t* kq, float* y, uint32_t ldy,
                  const float* resid, hipStream_t s, int8_t* xt) {
  if (m.quant == CAMELID_Q4_K && T <= (uint32_t)cm::Q4M_MAX) {  // a few tokens (verify)
    uint32_t tt = T;
    while (tt > 1 && cm::gemv_q4k_multi_lds_bytes((int)m.k, (int)tt) > 65536) --tt;
    const uint32_t nsb = m.k / 256, it = (m.k / 32 + 63) / 64;
    for (uint32_t t0 = 0; t0 < T; t0 += tt) {
      const uint32_t n = std::min(tt, T - t0);
      const size_t lds = cm::gemv_q4k_multi_lds_bytes((int)m.k, (int)n);
      switch (it) {
#define CM_Q4M(IT)                                                                                                \
  case IT:                                                                                                        \
    CM_LAUNCH(cm::k_gemv_q4k_multi<IT>, dim3((m.rows + 3) / 4), dim3(cm::KQ_NT), lds, s, m.a, m.b, (int)m.rows,   \
              (int)m.k, kd + (size_t)t0 * nsb, kq + (size_t)t0 * m.k, (int)n,                                     \
              y + (size_t)t0 * ldy, (int)ldy, resid ? resid + (size_t)t0 * ldy : nullptr);                        \
    break;
        CM_Q4M(1) CM_Q4M(2) CM_Q4M(3) CM_Q4M(4) CM_Q4M(5) CM_Q4M(6) CM_Q4M(7) CM_Q4M(8)
#undef CM_Q4M
        default:
          g_launch_error = "Q4_K multi-token GEMV: row width " + std::to_string(m.k) + " has no kernel instantiation";
          return;
      }
    }
    return;
  }
  if (m.quant == CAMELID_Q4_K) {
    CM_LAUNCH(cm::k_gemm_q4k, dim3(cm::gemm_q4k_grid((int)m.rows, (int)T)), dim3(cm::G4_NT), 0, s, m.a, m.b,
              (int)m.rows, (int)m.k, kd, kq, (int)T, y, (int)ldy, resid);
    return;
  }
  if (T > (uint32_t)cm::Q6M_MAX && m.w2 && xt && m.rows % 4 == 0 && ldy % 4 == 0) {  // a chunk: class-major GEMM
    const size_t threads = cm::q6g_act_bytes((int)T, (int)m.k) / 64;
    CM_LAUNCH(cm::k_q8k_classmajor, dim3((uint32_t)((threads + 255) / 256)), dim3(256), 0, s, kq, (int)T, (int)m.k,
              xt);
    CM_LAUNCH(cm::k_gemm_q6k2, dim3(cm::gemm_q6k2_grid((int)m.rows, (int)T)), dim3(cm::Q6G_NT), 0, s, m.w2, m.d,
              (int)m.rows, (int)m.k, kd, xt, (int)T, y, (int)ldy, resid);
    return;
  }
  if (T > (uint32_t)cm::Q6M_MAX) {  // a chunk: the sparse-MFMA GEMM
    CM_LAUNCH(cm::k_gemm_q6k, dim3((m.rows + cm::G6_RN - 1) / cm::G6_RN, (T + cm::G6_RT - 1) / cm::G6_RT),
              dim3(cm::G6_NT), 0, s, m.a, m.b, m.sc, m.d, (int)m.rows, (int)m.k, kd, kq, (int)T, y, (int)ldy, resid);
    return;
  }
  const uint32_t tt = q6m_tokens(m.k), nsb = m.k / 256;
  for (uint32_t t0 = 0; t0 < T; t0 += tt) {
    const uint32_t n = std::min(tt, T - t0);
    CM_LAUNCH(cm::k_gemv_q6k_multi, dim3((m.rows + cm::Q6M_ROWS - 1) / cm::Q6M_ROWS), dim3(cm::KQ_NT),
              cm::gemv_q6k_multi_lds_bytes((int)m.k, (int)n), s, m.a, m.b, m.sc, m.d, (int)m.rows, (int)m.k,
              kd + (size_t)t0 * nsb, kq + (size_t)t0 * m.k, (int)n, y + (size_t)t0 * ldy, (int)ldy,
              resid ? resid + (size_t)t0 * ldy : nullptr);
  }
}

constexpr int GEMM_NF1_BELOW = 512;
void launch_gemm(const Q8Mat& m, uint32_t T, const int8_t* xq, const float* xs, float* y, const float* resid,
                 hipStream_t s) {
  if (T <= (uint32_t)cm::GMT_MAX && m.k <= 8192) {  // a few tokens: weights streamed once by GEMV-shaped workgroups
    const uint32_t grid = (m.rows + cm::GMT_ROWS - 1) / cm::GMT_ROWS;
    const size_t lds = cm::gemv_multi_lds_bytes((int)m.k, (int)T);
    switch (m.k) {
#define CM_GMT(K)                                                                                                  \
  case K:                                                                                                          \
    CM_LAUNCH(cm::k_gemv_multi<K>, dim3(grid), dim3(256), lds, s, m.q, m.d, (int)m.rows, xq, xs, (int)T, y, resid); \
    return;
      CM_GMT(2048) CM_GMT(3072) CM_GMT(4096) CM_GMT(5632) CM_GMT(8192)
#undef CM_GMT
      default:
        break;
    }
  }
  // 32-row tiles when 64-row ones give fewer than two workgroups per CU of the 256 (measured
  // at 512 tokens: [2048 x 2048] 20.5 -> 18.1 us, [2048 x 5632] 52.8 -> 46.2 us with them; at
  // 704 tiles, [5632 x 2048], 36.3 -> 40.4 us, so not there).  CAMELID_HIP_GEMM_NF=1 / 2
  // forces either tile height.
  int nf = cm::gemm_tiles((int)m.rows, (int)T, 2) < GEMM_NF1_BELOW ? 1 : 2;
  if (const char* f = std::getenv("CAMELID_HIP_GEMM_NF")) {
    if (f[0] == '1') nf = 1;
    if (f[0] == '2') nf = 2;
  }
#define CM_GEMM(PLAIN, NF)                                                                                      \
  CM_LAUNCH((cm::k_gemm_q8<PLAIN, NF>), dim3(cm::gemm_grid((int)m.rows, (int)T, NF)), dim3(cm::GM_NT), 0, s, m.q, \
            m.d, (int)m.rows, (int)m.k, xq, xs, (int)T, y, resid)
  if (m.inf_scale) {
    if (nf == 1) CM_GEMM(true, 1);
    else CM_GEMM(true, 2);
  } else {
    if (nf == 1) CM_GEMM(false, 1);
    else CM_GEMM(false, 2);
  }
#undef CM_GEMM
}

// Q8Mat::inf_scale of weight scales already on the device (the entry points that take device
// pointers): a scan on the stream, its flag read back (synchronizes the stream).
int q8_scan_inf_scales(Q8Mat* m, hipStream_t s) {
  const size_t n = (size_t)m->rows * (m->k / 32);
  uint32_t* flag = nullptr;
  uint32_t h = 1;
  if (hipMalloc(&flag, 4) != hipSuccess) return fail(nullptr, "scale scan: device allocation failed");
  const uint32_t grid = (uint32_t)std::min<size_t>((n + 255) / 256, 1024);
  bool ok = hipMemsetAsync(flag, 0, 4, s) == hipSuccess;
  if (ok) hipLaunchKernelGGL(cm::k_f16_any_inf, dim3(grid), dim3(256), 0, s, m->d, n, flag);
  ok = ok && hipGetLastError() == hipSuccess && hipMemcpyAsync(&h, flag, 4, hipMemcpyDeviceToHost, s) == hipSuccess &&
       hipStreamSynchronize(s) == hipSuccess;
  (void)hipFree(flag);
  if (!ok) return fail(nullptr, "scale scan failed");
  m->inf_scale = h != 0;
  return 0;
}

// Causal attention of a prefill chunk: the tiled kernel (K/V rows shared by a tile of query
// tokens and the heads of their KV group) when scratch is given, the geometry has it and the
// chunk has at least tile_min tokens and reaches position tile_pos, else one workgroup per
// (head, token): a verify batch of a few tokens spreads wider that way, and below ~1K positions
// the per-token kernel measured faster (C5 1023-token prefill 0.072 vs 0.076 s, C3 511 tokens
// 0.016 vs 0.018 s; C4 8191 tokens 1.52 -> 1.03 s tiled).
constexpr uint32_t APT_TILE_MIN = 32;
constexpr uint32_t APT_TILE_POS = 1024;
void launch_attn_prefill(uint32_t hd, uint32_t n_heads, uint32_t n_kv, uint32_t T, const float* q, const uint16_t* kc,
                         const uint16_t* vc, int layer, int kvs, int pos0, float scale, float* att, int8_t* xq, float* xs,
                         hipStream_t s, float* scratch = nullptr, uint32_t tile_min = APT_TILE_MIN,
                         uint32_t tile_pos = APT_TILE_POS) {
  if (scratch && cm::apt_hd_ok((int)hd) && n_heads / n_kv <= (uint32_t)cm::APT_R && T >= tile_min &&
      (uint32_t)pos0 + T >= tile_pos) {
    const uint32_t tq = (uint32_t)cm::apt_tq((int)(n_heads / n_kv));
    const size_t pitch = cm::apt_pitch((size_t)pos0 + T);
    const dim3 grid(n_kv, (T + tq - 1) / tq);
    // 1024 threads (2 rows per thread, 110 VGPRs: four waves per SIMD) by default; 512 (4 rows
    // per thread, 155 VGPRs, two waves per SIMD) with CAMELID_HIP_APT_NT=512.  C4's 8191-token
    // prefill: 1.004 s at 512, 0.915 s at 1024 (a single wave issues one VALU instruction per
    // ~7 clocks, so two waves leave a SIMD idle between their issues)
    const char* nt = std::getenv("CAMELID_HIP_APT_NT");
    const bool wide = !(nt && std::atoi(nt) == 512);
#define CM_APT(HD, NT)                                                                                        \
  CM_LAUNCH((cm::k_attn_prefill_tile<HD, NT>), grid, dim3(NT), cm::apt_lds_bytes(HD), s, q, (int)n_heads,     \
            (int)n_kv, kc, vc, layer, kvs, pos0, (int)T, scale, scratch, pitch, att, xq, xs)
    if (hd == 64) {
      if (wide) CM_APT(64, 1024);
      else CM_APT(64, 512);
    } else {
      if (wide) CM_APT(128, 1024);
      else CM_APT(128, 512);
    }
#undef CM_APT
    return;
  }
  const size_t lds = (((size_t)pos0 + T + 3) & ~(size_t)3) * 4;
#define CM_AP(HD)                                                                                                  \
  CM_LAUNCH(cm::k_attn_prefill<HD>, dim3(n_heads, T), dim3(cm::AP_NT), lds, s, q, (int)n_heads, (int)n_kv, kc, vc, \
            layer, kvs, pos0, scale, att, xq, xs)
  if (hd == 64) CM_AP(64);
  else if (hd == 128) CM_AP(128);
  else CM_AP(256);
#undef CM_AP
}

// One chunk of T prompt tokens at positions pos0.. through every layer; the residual rows
// are in e->pf_h, the RoPE rows of the chunk at cosv / sinv.
// A layer with K-quant projections over the chunk (the order of run_layer_generic per token):
// RMSNorm rows to Q8_0 and Q8_K, each projection in its own format (Q4_K: k_gemm_q4k, Q6_K:
// k_gemv_q6k_multi, Q8_0: launch_gemm), the attention rows also in f32 for a K-quant O.
void prefill_layer_generic(camelid_hip_engine* e, uint32_t l, const float* cosv, const float* sinv, uint32_t T,
                           uint32_t pos0, float scale) {
  const camelid_hip_dims& d = e->d;
  const LayerW& L = e->layers[l];
  hipStream_t s = e->stream;
  const uint32_t half = d.rope_dim / 2;
  const uint32_t nq = d.n_heads * d.head_dim, nkv = d.n_kv_heads * d.head_dim, F = d.ffn_dim, H = d.hidden;
  // projection i into rows [T][ldy] at y (+ resid)
  auto proj_rows = [&](const Proj& p, float* y, uint32_t ldy, const float* resid) {
    ProfScope ps(e, P_GEMM, 2.0 * (p.quant != CAMELID_Q8_0 ? p.kq.rows : p.q8.rows) *
                                (p.quant != CAMELID_Q8_0 ? p.kq.k : p.q8.k) * T);
    if (p.quant != CAMELID_Q8_0) {
      launch_kgemm(p.kq, T, e->pf_kd, e->pf_kq, y, ldy, resid, s, e->pf_kqt);
    } else if (ldy == p.q8.rows) {
      launch_gemm(p.q8, T, e->pf_xq, e->pf_xs, y, resid, s);
    } else {  // (no residual on the strided projections)
      launch_gemm(p.q8, T, e->pf_xq, e->pf_xs, e->pf_tmp, nullptr, s);
      (void)hipMemcpy2DAsync(y, (size_t)ldy * 4, e->pf_tmp, (size_t)p.q8.rows * 4, (size_t)p.q8.rows * 4, T,
                             hipMemcpyDeviceToDevice, s);
    }
  };
  const uint32_t W = nq + 2 * nkv;
  launch_rmsnorm_quant(e->pf_h, L.attn_norm, H, d.eps, e->pf_xq, e->pf_xs, nullptr, s, cm::Prefetch{}, T, e->pf_kd,
                       e->pf_kq, e->pf_kbs);
  proj_rows(L.p[0], e->pf_qkv, W, nullptr);
  if (!L.qk_stacked) proj_rows(L.p[1], e->pf_qkv + nq, W, nullptr);
  proj_rows(L.p[2], e->pf_qkv + nq + nkv, W, nullptr);
  CM_LAUNCH(cm::k_rope_kv, dim3(d.n_heads + d.n_kv_heads, T), dim3(64), 0, s, e->pf_qkv, (int)d.n_heads,
            (int)d.n_kv_heads, (int)d.head_dim, (int)d.rope_dim, (int)d.split_half_pairing, cosv, sinv, L.q_norm,
            L.k_norm, d.eps, e->pf_q, e->kc, e->vc, (int)l, (int)e->kvs, (const uint32_t*)nullptr, (int)pos0,
            (int)half);
  launch_attn_prefill(d.head_dim, d.n_heads, d.n_kv_heads, T, e->pf_q, e->kc, e->vc, (int)l, (int)e->kvs, (int)pos0,
                      scale, e->pf_att, e->pf_xq, e->pf_xs, s, e->pf_sc, APT_TILE_MIN, e->att_tile_pos);
  if (L.p[3].quant != CAMELID_Q8_0)
    CM_LAUNCH(cm::k_quantize_q8k, dim3(T * nq / 256), dim3(256), 0, s, e->pf_att, e->pf_kd, e->pf_kq,
              e->pf_kbs);
  proj_rows(L.p[3], e->pf_h, H, e->pf_h);
  launch_rmsnorm_quant(e->pf_h, L.ffn_norm, H, d.eps, e->pf_xq, e->pf_xs, nullptr, s, cm::Prefetch{}, T, e->pf_kd,
                       e->pf_kq, e->pf_kbs);
  proj_rows(L.p[4], e->pf_gu, 2 * F, nullptr);
  if (!L.gu_stacked) proj_rows(L.p[5], e->pf_gu + F, 2 * F, nullptr);
  const bool k8 = L.p[6].quant != CAMELID_Q8_0;
  CM_LAUNCH(cm::k_silu_mul_quant, dim3((F + 255) / 256, T), dim3(256), 0, s, e->pf_gu, (int)F,
            k8 ? (int8_t*)nullptr : e->pf_xq, k8 ? (float*)nullptr : e->pf_xs, (float*)nullptr, cm::Prefetch{},
            k8 ? e->pf_kd : nullptr, k8 ? e->pf_kq : nullptr, k8 ? e->pf_kbs : nullptr);
  proj_rows(L.p[6], e->pf_h, H, e->pf_h);
}

void prefill_chunk(camelid_hip_engine* e, const float* cosv, const float* sinv, uint32_t T, uint32_t pos0,
                   float scale) {
  const camelid_hip_dims& d = e->d;
  hipStream_t s = e->stream;
  const uint32_t half = d.rope_dim / 2;
  // a Q8_0 projection of the chunk; int8 ops (2 per weight and token) credited to the profile
  auto gemm = [&](const Q8Mat& m, float* y, const float* resid) {
    ProfScope ps(e, P_GEMM, 2.0 * m.rows * m.k * T);
    launch_gemm(m, T, e->pf_xq, e->pf_xs, y, resid, s);
  };
  for (uint32_t l = 0; l < d.n_layers; ++l) {
    const LayerW& L = e->layers[l];
    if (L.generic) {
      prefill_layer_generic(e, l, cosv, sinv, T, pos0, scale);
      continue;
    }
    launch_rmsnorm_quant(e->pf_h, L.attn_norm, d.hidden, d.eps, e->pf_xq, e->pf_xs, nullptr, s, cm::Prefetch{}, T);
    gemm(L.qkv, e->pf_qkv, nullptr);
    CM_LAUNCH(cm::k_rope_kv, dim3(d.n_heads + d.n_kv_heads, T), dim3(64), 0, s, e->pf_qkv, (int)d.n_heads,
              (int)d.n_kv_heads, (int)d.head_dim, (int)d.rope_dim, (int)d.split_half_pairing, cosv, sinv, L.q_norm,
              L.k_norm, d.eps, e->pf_q, e->kc, e->vc, (int)l, (int)e->kvs, (const uint32_t*)nullptr, (int)pos0,
              (int)half);
    launch_attn_prefill(d.head_dim, d.n_heads, d.n_kv_heads, T, e->pf_q, e->kc, e->vc, (int)l, (int)e->kvs,
                        (int)pos0, scale, nullptr, e->pf_xq, e->pf_xs, s, e->pf_sc, APT_TILE_MIN, e->att_tile_pos);
    gemm(L.o, e->pf_h, e->pf_h);
    launch_rmsnorm_quant(e->pf_h, L.ffn_norm, d.hidden, d.eps, e->pf_xq, e->pf_xs, nullptr, s, cm::Prefetch{}, T);
    gemm(L.gu, e->pf_gu, nullptr);
    CM_LAUNCH(cm::k_silu_rows, dim3((d.ffn_dim + 255) / 256, T), dim3(256), 0, s, e->pf_gu, (int)d.ffn_dim,
              (int)e->gu_fused, e->pf_xq, e->pf_xs);
    gemm(L.down, e->pf_h, e->pf_h);
  }
}

bool ready(const camelid_hip_engine* e) {
  if (!e->out_set) return false;
  for (const LayerW& L : e->layers)
    if (!L.set) return false;
  return true;
}

int check_launch(camelid_hip_engine* e) {
  hipError_t st = hipGetLastError();
  if (st != hipSuccess) return fail(e, std::string("kernel launch failed: ") + hipGetErrorString(st));
  if (!g_launch_error.empty()) {
    const std::string m = g_launch_error;
    g_launch_error.clear();
    return fail(e, m);
  }
  return 0;
}

void drop_graph(camelid_hip_engine* e) {
  for (int m = 0; m < 2; ++m) {
    if (e->graph_exec[m]) (void)hipGraphExecDestroy(e->graph_exec[m]);
    if (e->graph[m]) (void)hipGraphDestroy(e->graph[m]);
    e->graph_exec[m] = nullptr;
    e->graph[m] = nullptr;
  }
}

// Device-side decode step (embed -> layers -> head) as launched work on e->stream.
void enqueue_device_step(camelid_hip_engine* e, float scale) {
  run_embed(e);
  run_stack(e, e->rope_cos, e->rope_sin, (int)(e->d.rope_dim / 2), scale);
  run_head(e, e->tokens, e->tokens_cap);
}

// Captures one device-side step into a graph (once per scale and attention mode: the
// position is read on the device, so the graph for the split attention is a second graph).
int ensure_graph(camelid_hip_engine* e, float scale, int mode) {
  if (e->graph_exec[mode] && e->graph_scale[mode] == scale) return 0;
  if (e->graph_exec[mode]) (void)hipGraphExecDestroy(e->graph_exec[mode]);
  if (e->graph[mode]) (void)hipGraphDestroy(e->graph[mode]);
  e->graph_exec[mode] = nullptr;
  e->graph[mode] = nullptr;
  HIP_TRY(e, hipStreamBeginCapture(e->stream, hipStreamCaptureModeThreadLocal));
  e->att_mode = mode;
  enqueue_device_step(e, scale);
  e->att_mode = -1;
  hipGraph_t g = nullptr;
  hipError_t st = hipStreamEndCapture(e->stream, &g);
  if (st != hipSuccess) return fail(e, std::string("graph capture failed: ") + hipGetErrorString(st));
  e->graph[mode] = g;
  st = hipGraphInstantiate(&e->graph_exec[mode], g, nullptr, nullptr, 0);
  if (st != hipSuccess) {
    drop_graph(e);
    return fail(e, std::string("graph instantiate failed: ") + hipGetErrorString(st));
  }
  e->graph_scale[mode] = scale;
  return 0;
}

// Why the engine would refuse these dimensions ("" when it takes them).  host_only (the
// preflight camelid_hip_check_model): no HIP call; the attention's LDS room is judged with the
// device-free bounds, which decline a max_pos within a few hundred positions of the device's
// own limit that engine_new would still take.
std::string dims_problem(const camelid_hip_dims& d, bool host_only) {
  if (!d.n_layers || !d.n_heads || !d.n_kv_heads || !d.head_dim || !d.hidden || !d.ffn_dim || !d.vocab || !d.max_pos)
    return "all dimensions must be nonzero";
  if (d.n_heads % d.n_kv_heads) return "n_heads must be a multiple of n_kv_heads";
  if (d.hidden % 32 || d.ffn_dim % 32 || d.head_dim % 32) return "hidden, ffn_dim and head_dim must be multiples of 32";
  if (!attention_hd_supported(d.head_dim)) return "head_dim must be 64, 128 or 256";
  if (d.hidden > (uint32_t)cm::SEG_MAX_N) return "hidden > 16384 is not supported by the RMSNorm kernel";
  if (d.rope_dim == 0 || d.rope_dim > d.head_dim || d.rope_dim % 2) return "rope_dim must be even and within head_dim";
  if (attn_ring_slots((d.max_pos + 7u) & ~7u, host_only) == 0) return "max_pos too large for the decode attention";
  if (cm::gemv_lds_bytes((int)std::max(d.ffn_dim, d.n_heads * d.head_dim)) > 64 * 1024)
    return "row width too large for the GEMV";
  return "";
}

// Why set_layer / set_output would refuse a projection of `quant` with row width k ("" when
// they take it).  The byte length is checked at upload.
std::string proj_problem(uint8_t quant, uint32_t k) {
  if (quant == CAMELID_Q8_0) return k % 32 ? "Q8_0 row width must be a multiple of 32" : "";
  if (quant != CAMELID_Q4_K && quant != CAMELID_Q6_K) return "unknown weight format";
  if (k % 256) return "K-quant row width must be a multiple of 256";
  if (k > KQ_MAX_K)
    return "K-quant row width " + std::to_string(k) + " > " + std::to_string(KQ_MAX_K) + " is not supported";
  return "";
}

}  // namespace

// ====================================================================== C ABI
extern "C" {

const char* camelid_hip_last_error(const camelid_hip_engine* e) { return e ? e->err.c_str() : g_last_error.c_str(); }

int camelid_hip_check_model(const camelid_hip_dims* dims, const uint8_t layer_quant[7], uint8_t out_quant) {
  if (!dims) return fail(nullptr, "null argument");
  const camelid_hip_dims& d = *dims;
  std::string bad = dims_problem(d, true);
  if (!bad.empty()) return fail(nullptr, bad);
  const uint32_t nq = d.n_heads * d.head_dim;
  const uint32_t ks[7] = {d.hidden, d.hidden, d.hidden, nq, d.hidden, d.hidden, d.ffn_dim};
  static const char* names[7] = {"q", "k", "v", "o", "gate", "up", "down"};
  if (layer_quant)
    for (int i = 0; i < 7; ++i) {
      bad = proj_problem(layer_quant[i], ks[i]);
      if (!bad.empty()) return fail(nullptr, std::string(names[i]) + " projection: " + bad);
    }
  bad = proj_problem(out_quant, d.hidden);
  if (!bad.empty()) return fail(nullptr, "output projection: " + bad);
  return 0;
}

int camelid_hip_engine_new(const camelid_hip_dims* dims, camelid_hip_engine** out) {
  if (!dims || !out) return fail(nullptr, "null argument");
  *out = nullptr;
  const camelid_hip_dims& d = *dims;
  const std::string bad = dims_problem(d, false);
  if (!bad.empty()) return fail(nullptr, bad);
  auto* e = new camelid_hip_engine();
  e->d = d;
  if (const char* dev = std::getenv("CAMELID_HIP_DEVICE")) e->device = std::atoi(dev);
  if (const char* g = std::getenv("CAMELID_HIP_GRAPHS")) e->use_graph = std::atoi(g) != 0;
  if (const char* r = std::getenv("CAMELID_HIP_READ_AHEAD")) e->read_ahead = e->kv_ahead = std::atoi(r) != 0;
  if (const char* r = std::getenv("CAMELID_HIP_KV_AHEAD")) e->kv_ahead = std::atoi(r) != 0;
  if (const char* p = std::getenv("CAMELID_HIP_PREFILL")) e->prefill_batched = std::strcmp(p, "token") != 0;
  hipError_t st = hipSetDevice(e->device);
  if (st != hipSuccess) {
    fail(nullptr, std::string("hipSetDevice failed: ") + hipGetErrorString(st));
    delete e;
    return 1;
  }
  st = hipStreamCreateWithFlags(&e->stream, hipStreamNonBlocking);
  if (st != hipSuccess) {
    fail(nullptr, std::string("hipStreamCreate failed: ") + hipGetErrorString(st));
    delete e;
    return 1;
  }
  e->layers.resize(d.n_layers);
  e->kvs = (d.max_pos + 7u) & ~7u;
  e->gu_fused = cm::gu_fused_k((int)d.hidden);
  if (const char* f = std::getenv("CAMELID_HIP_FUSED_GU")) e->gu_fused = e->gu_fused && std::atoi(f) != 0;
  if (const char* f = std::getenv("CAMELID_HIP_FUSED_NORM")) e->norm_fused = std::atoi(f) != 0;
  if (const char* f = std::getenv("CAMELID_HIP_QKV_MERGED")) e->qkv_merged = std::atoi(f) != 0;
  if (const char* f = std::getenv("CAMELID_HIP_KQ_NORM_FUSED")) e->kq_norm_fused = std::atoi(f) != 0;
  if (const char* f = std::getenv("CAMELID_HIP_Q6K_GEMM2")) e->q6_gemm2 = std::atoi(f) != 0;
  if (const char* f = std::getenv("CAMELID_HIP_GU_LOOP")) e->gu_loop = std::atoi(f) != 0;
  e->att_slots = attn_ring_slots(e->kvs);
  if (const char* f = std::getenv("CAMELID_HIP_ATT_SPLIT")) e->att_split_min = (uint32_t)std::strtoul(f, nullptr, 10);
  if (const char* f = std::getenv("CAMELID_HIP_ATT_DG")) e->att_dg = std::atoi(f);
  if (const char* f = std::getenv("CAMELID_HIP_ATT_O")) e->att_o_fused = std::atoi(f) != 0;
  if (const char* f = std::getenv("CAMELID_HIP_ATT_TILE")) e->att_tile = std::atoi(f) != 0;
  if (const char* f = std::getenv("CAMELID_HIP_ATT_TILE_POS")) e->att_tile_pos = (uint32_t)std::max(0, std::atoi(f));
  if (const char* f = std::getenv("CAMELID_HIP_ATT_FUSED_SPLIT")) e->att_fsplit = std::atoi(f) != 0;
  {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, e->device) == hipSuccess && cus > 0)
      e->n_cus = (uint32_t)cus;
  }
  const size_t nq = (size_t)d.n_heads * d.head_dim, nkv = (size_t)d.n_kv_heads * d.head_dim;
  const size_t kv_elems = (size_t)d.n_layers * d.n_kv_heads * e->kvs * d.head_dim;
  const size_t act = std::max<size_t>({(size_t)d.hidden, (size_t)d.ffn_dim, nq});
  const uint32_t half = d.rope_dim / 2;
  const size_t nparts = (d.vocab + 3) / 4;  // at least 4 rows per lm_head workgroup
  e->tokens_cap = d.max_pos;
  int rc = dev_alloc(e, &e->kc, kv_elems) || dev_alloc(e, &e->vc, kv_elems) || dev_alloc(e, &e->h, d.hidden) ||
           dev_alloc(e, &e->qkv, nq + 2 * nkv) || dev_alloc(e, &e->att, nq) ||
           dev_alloc(e, &e->gu, 2 * (size_t)d.ffn_dim) || dev_alloc(e, &e->logits, d.vocab) ||
           dev_alloc(e, &e->aq, d.ffn_dim) || dev_alloc(e, &e->as, d.ffn_dim / 32) ||
           dev_alloc(e, &e->hidden_cap, (size_t)(d.n_layers + 1) * d.hidden) || dev_alloc(e, &e->xq, act) ||
           dev_alloc(e, &e->xs, act / 32) || dev_alloc(e, &e->cos_cur, half) || dev_alloc(e, &e->sin_cur, half) ||
           dev_alloc(e, &e->part_v, nparts) || dev_alloc(e, &e->part_i, nparts) || dev_alloc(e, &e->st, 1) ||
           dev_alloc(e, &e->tokens, e->tokens_cap) || dev_alloc(e, &e->xn, act) || dev_alloc(e, &e->actf, d.ffn_dim) ||
           dev_alloc(e, &e->kd, act / 256 + 1) || dev_alloc(e, &e->kq, act) || dev_alloc(e, &e->kbs, act / 32) ||
           dev_alloc(e, &e->att_sc, (size_t)d.n_heads * e->kvs) ||
           dev_alloc(e, &e->att_mx, (size_t)d.n_heads * ((e->kvs + 255) / 256)) ||
           dev_alloc(e, &e->att_sct, (size_t)d.n_heads * e->kvs) ||
           host_alloc(e, &e->p_emb, d.hidden) ||
           host_alloc(e, &e->p_cos, half) || host_alloc(e, &e->p_sin, half) || host_alloc(e, &e->p_logits, d.vocab) ||
           host_alloc(e, &e->p_st, 1) || host_alloc(e, &e->p_err, 1) ||
           dev_alloc(e, &e->nf_slots, (size_t)cm::NF_WORDS) || dev_alloc(e, &e->ao_words, ao_words(e));
  if (rc) {
    std::string m = e->err;
    camelid_hip_engine_free(e);
    return fail(nullptr, m);
  }
  // A fresh cache reads as zeros (K/V past `filled` are never read); StepState starts at 0.
  if (hipMemset(e->kc, 0, kv_elems * 2) != hipSuccess || hipMemset(e->vc, 0, kv_elems * 2) != hipSuccess ||
      hipMemset(e->st, 0, sizeof(cm::StepState)) != hipSuccess ||
      hipMemset(e->nf_slots, 0, cm::NF_WORDS * 4) != hipSuccess || hipMemset(e->ao_words, 0, ao_words(e) * 8) != hipSuccess ||
      hipDeviceSynchronize() != hipSuccess) {
    camelid_hip_engine_free(e);
    return fail(nullptr, "initial device memset failed");
  }
  *out = e;
  return 0;
}

void camelid_hip_engine_free(camelid_hip_engine* e) {
  if (!e) return;
  (void)hipSetDevice(e->device);
  if (e->stream) (void)hipStreamSynchronize(e->stream);
  drop_graph(e);
  for (hipEvent_t ev : e->event_pool) (void)hipEventDestroy(ev);
  for (void* p : e->dev_allocs) (void)hipFree(p);
  for (void* p : e->host_allocs) (void)hipHostFree(p);
  if (e->stream) (void)hipStreamDestroy(e->stream);
  delete e;
}

int camelid_hip_set_layer(camelid_hip_engine* e, uint32_t layer, const uint8_t* const w[7], const size_t len[7],
                          const uint8_t quant[7], uint8_t q8_layout, const float* attn_norm, const float* ffn_norm,
                          const float* q_norm, const float* k_norm) {
  if (e) e->nf_state = e->ao_state = e->ao4_state = -1;  // (the fused-launch decisions are taken again for the new weights)
  if (!e) return fail(nullptr, "null engine");
  if (layer >= e->d.n_layers) return fail(e, "layer index out of range");
  if (!w || !len || !quant || !attn_norm || !ffn_norm) return fail(e, "null argument");
  if ((q_norm == nullptr) != (k_norm == nullptr)) return fail(e, "q_norm and k_norm must be given together");
  bool all_q8 = true;
  {
    const uint32_t nq0 = e->d.n_heads * e->d.head_dim;
    const uint32_t ks0[7] = {e->d.hidden, e->d.hidden, e->d.hidden, nq0, e->d.hidden, e->d.hidden, e->d.ffn_dim};
    for (int i = 0; i < 7; ++i) {
      const std::string bad = proj_problem(quant[i], ks0[i]);
      if (!bad.empty()) return fail(e, bad);
      all_q8 = all_q8 && quant[i] == CAMELID_Q8_0;
    }
  }
  HIP_TRY(e, hipSetDevice(e->device));
  const camelid_hip_dims& d = e->d;
  const uint32_t nq = d.n_heads * d.head_dim, nkv = d.n_kv_heads * d.head_dim;
  LayerW& L = e->layers[layer];
  if (L.set && L.generic == all_q8) return fail(e, "a layer's formats cannot change after upload");
  if (!all_q8) {
    // seven separate projections, each in its own format
    const uint32_t rows[7] = {nq, nkv, nkv, d.hidden, d.ffn_dim, d.ffn_dim, d.hidden};
    const uint32_t ks[7] = {d.hidden, d.hidden, d.hidden, nq, d.hidden, d.hidden, d.ffn_dim};
    // q|k and gate|up of one K-quant format go up as one stacked matrix (one launch each)
    const bool qk = quant[0] == quant[1] && quant[0] != CAMELID_Q8_0;
    const bool gu = quant[4] == quant[5] && quant[4] != CAMELID_Q8_0;
    if (L.set && (qk != L.qk_stacked || gu != L.gu_stacked)) return fail(e, "a layer's formats cannot change after upload");
    for (int i = 0; i < 7; ++i) {
      Proj& P = L.p[i];
      if (L.set && P.quant != quant[i]) return fail(e, "a layer's formats cannot change after upload");
      P.quant = quant[i];
      if ((i == 1 && qk) || (i == 5 && gu)) continue;  // uploaded with its partner
      int rc;
      if ((i == 0 && qk) || (i == 4 && gu)) {
        if (!w[i] || !w[i + 1]) return fail(e, "missing projection bytes");
        std::vector<uint8_t> both(len[i] + len[i + 1]);
        std::memcpy(both.data(), w[i], len[i]);
        std::memcpy(both.data() + len[i], w[i + 1], len[i + 1]);
        const size_t per_row = (size_t)(ks[i] / 256) * kq_block_bytes(quant[i]);
        if (len[i] != (size_t)rows[i] * per_row || len[i + 1] != (size_t)rows[i + 1] * per_row)
          return fail(e, "K-quant byte length does not match the projection shape");
        rc = upload_kq(e, &P.kq, both.data(), both.size(), rows[i] + rows[i + 1], ks[i], quant[i], true);
      } else {
        rc = quant[i] == CAMELID_Q8_0 ? upload_q8(e, &P.q8, {{w[i], len[i], rows[i]}}, ks[i], q8_layout)
                                      : upload_kq(e, &P.kq, w[i], len[i], rows[i], ks[i], quant[i], true);
      }
      if (rc) return 1;
    }
    L.qk_stacked = qk;
    L.gu_stacked = gu;
    if (upload_f32(e, &L.attn_norm, attn_norm, d.hidden) || upload_f32(e, &L.ffn_norm, ffn_norm, d.hidden)) return 1;
    if (q_norm && (upload_f32(e, &L.q_norm, q_norm, d.head_dim) || upload_f32(e, &L.k_norm, k_norm, d.head_dim)))
      return 1;
    L.generic = true;
    L.set = true;
    e->any_kquant = true;
    drop_graph(e);
    return 0;
  }
  if (upload_q8(e, &L.qkv, {{w[0], len[0], nq}, {w[1], len[1], nkv}, {w[2], len[2], nkv}}, d.hidden, q8_layout) ||
      upload_q8(e, &L.o, {{w[3], len[3], d.hidden}}, nq, q8_layout) ||
      upload_q8(e, &L.gu, {{w[4], len[4], d.ffn_dim}, {w[5], len[5], d.ffn_dim}}, d.hidden, q8_layout,
                e->gu_fused ? 32u : 0u) ||
      upload_q8(e, &L.down, {{w[6], len[6], d.hidden}}, d.ffn_dim, q8_layout) ||
      upload_f32(e, &L.attn_norm, attn_norm, d.hidden) || upload_f32(e, &L.ffn_norm, ffn_norm, d.hidden))
    return 1;
  if (q_norm && (upload_f32(e, &L.q_norm, q_norm, d.head_dim) || upload_f32(e, &L.k_norm, k_norm, d.head_dim)))
    return 1;
  L.set = true;
  drop_graph(e);
  return 0;
}

int camelid_hip_set_output(camelid_hip_engine* e, const float* final_norm, const uint8_t* w, size_t len, uint8_t quant,
                           uint8_t q8_layout) {
  if (!e) return fail(nullptr, "null engine");
  if (!final_norm || !w) return fail(e, "null argument");
  if (quant != CAMELID_Q8_0 && quant != CAMELID_Q4_K && quant != CAMELID_Q6_K)
    return fail(e, "unknown output projection format");
  {
    const std::string bad = proj_problem(quant, e->d.hidden);
    if (!bad.empty()) return fail(e, "output projection: " + bad);
  }
  if (e->out_set && quant != e->out_quant) return fail(e, "the output format cannot change after upload");
  HIP_TRY(e, hipSetDevice(e->device));
  const int rc = quant == CAMELID_Q8_0 ? upload_q8(e, &e->out, {{w, len, e->d.vocab}}, e->d.hidden, q8_layout)
                                       : upload_kq(e, &e->out_k, w, len, e->d.vocab, e->d.hidden, quant);
  if (rc || upload_f32(e, &e->out_norm, final_norm, e->d.hidden)) return 1;
  e->out_quant = quant;
  if (quant != CAMELID_Q8_0) e->any_kquant = true;
  e->out_set = true;
  drop_graph(e);
  return 0;
}

int camelid_hip_set_embedding(camelid_hip_engine* e, const uint8_t* w, size_t len, uint8_t quant, uint8_t q8_layout) {
  if (!e) return fail(nullptr, "null engine");
  if (!w) return fail(e, "null argument");
  if (quant != CAMELID_Q8_0 && quant != CAMELID_Q4_K && quant != CAMELID_Q6_K)
    return fail(e, "unknown embedding format");
  if (e->embd_set && quant != e->embd_quant) return fail(e, "the embedding format cannot change after upload");
  HIP_TRY(e, hipSetDevice(e->device));
  const int rc = quant == CAMELID_Q8_0 ? upload_q8(e, &e->embd, {{w, len, e->d.vocab}}, e->d.hidden, q8_layout)
                                       : upload_kq(e, &e->embd_k, w, len, e->d.vocab, e->d.hidden, quant);
  if (rc) return 1;
  e->embd_quant = quant;
  e->embd_set = true;
  drop_graph(e);
  return 0;
}

int camelid_hip_set_rope_table(camelid_hip_engine* e, const float* cos_all, const float* sin_all, uint32_t n_pos) {
  if (!e) return fail(nullptr, "null engine");
  if (!cos_all || !sin_all) return fail(e, "null argument");
  if (n_pos > e->d.max_pos) return fail(e, "rope table longer than max_pos");
  HIP_TRY(e, hipSetDevice(e->device));
  const size_t half = e->d.rope_dim / 2;
  if (!e->rope_cos && (dev_alloc(e, &e->rope_cos, (size_t)e->d.max_pos * half) ||
                       dev_alloc(e, &e->rope_sin, (size_t)e->d.max_pos * half)))
    return 1;
  HIP_TRY(e, hipMemcpy(e->rope_cos, cos_all, (size_t)n_pos * half * 4, hipMemcpyHostToDevice));
  HIP_TRY(e, hipMemcpy(e->rope_sin, sin_all, (size_t)n_pos * half * 4, hipMemcpyHostToDevice));
  e->rope_rows = n_pos;
  drop_graph(e);
  return 0;
}

int camelid_hip_weights_ready(const camelid_hip_engine* e) { return e && ready(e) ? 1 : 0; }
uint32_t camelid_hip_filled(const camelid_hip_engine* e) { return e ? e->filled : 0; }
int camelid_hip_set_filled(camelid_hip_engine* e, uint32_t filled) {
  if (!e) return fail(nullptr, "null engine");
  if (filled > e->d.max_pos) return fail(e, "filled beyond max_pos");
  e->filled = filled;
  return 0;
}
uint32_t camelid_hip_max_pos(const camelid_hip_engine* e) { return e ? e->d.max_pos : 0; }
uint32_t camelid_hip_n_layers(const camelid_hip_engine* e) { return e ? e->d.n_layers : 0; }
int camelid_hip_uses_kquant(const camelid_hip_engine* e) { return e && e->any_kquant ? 1 : 0; }

int camelid_hip_seed_layer(camelid_hip_engine* e, uint32_t layer, const float* ck, const float* cv, uint32_t n_pos) {
  if (!e) return fail(nullptr, "null engine");
  if (layer >= e->d.n_layers || n_pos > e->d.max_pos) return fail(e, "seed_layer out of range");
  if (!ck || !cv) return fail(e, "null argument");
  HIP_TRY(e, hipSetDevice(e->device));
  HIP_TRY(e, hipStreamSynchronize(e->stream));
  const camelid_hip_dims& d = e->d;
  const int hd = (int)d.head_dim, kvs = (int)e->kvs;
  std::vector<uint16_t> hk((size_t)hd * kvs), hv((size_t)hd * kvs);
  for (uint32_t h = 0; h < d.n_kv_heads; ++h) {
    const size_t src = (size_t)h * n_pos * hd;
    const size_t base = cm::kv_head_base((int)layer, (int)d.n_kv_heads, (int)h, hd, kvs);
    HIP_TRY(e, hipMemcpy(hk.data(), e->kc + base, hk.size() * 2, hipMemcpyDeviceToHost));
    HIP_TRY(e, hipMemcpy(hv.data(), e->vc + base, hv.size() * 2, hipMemcpyDeviceToHost));
    for (int t = 0; t < (int)n_pos; ++t)
      for (int j = 0; j < hd; ++j) {
        hk[cm::kv_k_index(kvs, t, j)] = cm::f32_to_f16_bits(ck[src + (size_t)t * hd + j]);
        hv[cm::kv_v_index(hd, t, j)] = cm::f32_to_f16_bits(cv[src + (size_t)t * hd + j]);
      }
    HIP_TRY(e, hipMemcpy(e->kc + base, hk.data(), hk.size() * 2, hipMemcpyHostToDevice));
    HIP_TRY(e, hipMemcpy(e->vc + base, hv.data(), hv.size() * 2, hipMemcpyHostToDevice));
  }
  return 0;
}

int camelid_hip_read_kv_layer(camelid_hip_engine* e, uint32_t layer, uint32_t n, float* ck, float* cv) {
  if (!e) return fail(nullptr, "null engine");
  if (layer >= e->d.n_layers || n > e->d.max_pos) return fail(e, "read_kv_layer out of range");
  if (!ck || !cv) return fail(e, "null argument");
  HIP_TRY(e, hipSetDevice(e->device));
  HIP_TRY(e, hipStreamSynchronize(e->stream));
  const camelid_hip_dims& d = e->d;
  const int hd = (int)d.head_dim, kvs = (int)e->kvs;
  std::vector<uint16_t> hk((size_t)hd * kvs), hv((size_t)hd * kvs);
  for (uint32_t h = 0; h < d.n_kv_heads; ++h) {
    const size_t base = cm::kv_head_base((int)layer, (int)d.n_kv_heads, (int)h, hd, kvs);
    HIP_TRY(e, hipMemcpy(hk.data(), e->kc + base, hk.size() * 2, hipMemcpyDeviceToHost));
    HIP_TRY(e, hipMemcpy(hv.data(), e->vc + base, hv.size() * 2, hipMemcpyDeviceToHost));
    const size_t dst = (size_t)h * n * hd;
    for (int t = 0; t < (int)n; ++t)
      for (int j = 0; j < hd; ++j) {
        ck[dst + (size_t)t * hd + j] = cm::f16_bits_to_f32(hk[cm::kv_k_index(kvs, t, j)]);
        cv[dst + (size_t)t * hd + j] = cm::f16_bits_to_f32(hv[cm::kv_v_index(hd, t, j)]);
      }
  }
  return 0;
}

int camelid_hip_forward_token(camelid_hip_engine* e, const float* emb, const float* cos_tab, const float* sin_tab,
                              uint32_t position, float scale, int want_logits, uint32_t* tok_out, float* logits_out) {
  if (!e) return fail(nullptr, "null engine");
  if (!ready(e)) return fail(e, "weights not ready");
  if (!emb || !cos_tab || !sin_tab) return fail(e, "null argument");
  if (position >= e->d.max_pos) return fail(e, "position beyond max_pos");
  if (!std::isfinite(scale)) return fail(e, "attention score scale must be finite");
  HIP_TRY(e, hipSetDevice(e->device));
  const camelid_hip_dims& d = e->d;
  const size_t half = d.rope_dim / 2;
  std::memcpy(e->p_emb, emb, d.hidden * 4);
  std::memcpy(e->p_cos, cos_tab, half * 4);
  std::memcpy(e->p_sin, sin_tab, half * 4);
  *e->p_st = cm::StepState{position, 0u, 0u, 0u};
  e->cur_pos = position;
  HIP_TRY(e, hipMemcpyAsync(e->h, e->p_emb, d.hidden * 4, hipMemcpyHostToDevice, e->stream));
  HIP_TRY(e, hipMemcpyAsync(e->cos_cur, e->p_cos, half * 4, hipMemcpyHostToDevice, e->stream));
  HIP_TRY(e, hipMemcpyAsync(e->sin_cur, e->p_sin, half * 4, hipMemcpyHostToDevice, e->stream));
  HIP_TRY(e, hipMemcpyAsync(e->st, e->p_st, sizeof(cm::StepState), hipMemcpyHostToDevice, e->stream));
  if (nf_begin(e)) return 1;
  run_stack(e, e->cos_cur, e->sin_cur, 0, scale);
  run_head(e, nullptr, 0);
  if (check_launch(e)) {
    e->filled = 0;
    return 1;
  }
  if (nf_end(e)) return 1;
  HIP_TRY(e, hipMemcpyAsync(e->p_st, e->st, sizeof(cm::StepState), hipMemcpyDeviceToHost, e->stream));
  if (want_logits && logits_out)
    HIP_TRY(e, hipMemcpyAsync(e->p_logits, e->logits, (size_t)d.vocab * 4, hipMemcpyDeviceToHost, e->stream));
  hipError_t st = hipStreamSynchronize(e->stream);
  if (st != hipSuccess) {
    e->filled = 0;
    return fail(e, std::string("forward_token: ") + hipGetErrorString(st));
  }
  if (nf_failed(e)) return 1;
  if (tok_out) *tok_out = e->p_st->tok;
  if (want_logits && logits_out) std::memcpy(logits_out, e->p_logits, (size_t)d.vocab * 4);
  e->filled = position + 1;
  return 0;
}

int camelid_hip_prefill(camelid_hip_engine* e, const float* embs, const float* cos_all, const float* sin_all,
                        uint32_t n, float scale) {
  if (!e) return fail(nullptr, "null engine");
  if (!ready(e)) return fail(e, "weights not ready");
  if (!embs || !cos_all || !sin_all) return fail(e, "null argument");
  const camelid_hip_dims& d = e->d;
  if ((size_t)e->filled + n > d.max_pos) return fail(e, "prefill beyond max_pos");
  if (!std::isfinite(scale)) return fail(e, "attention score scale must be finite");
  if (n == 0) return 0;
  HIP_TRY(e, hipSetDevice(e->device));
  const size_t half = d.rope_dim / 2;
  float *d_embs = nullptr, *d_cos = nullptr, *d_sin = nullptr;
  cm::StepState* d_sts = nullptr;
  HIP_TRY(e, hipMalloc(&d_embs, (size_t)n * d.hidden * 4));
  HIP_TRY(e, hipMalloc(&d_cos, (size_t)n * half * 4));
  HIP_TRY(e, hipMalloc(&d_sin, (size_t)n * half * 4));
  HIP_TRY(e, hipMalloc(&d_sts, (size_t)n * sizeof(cm::StepState)));
  std::vector<cm::StepState> sv(n);
  for (uint32_t t = 0; t < n; ++t) sv[t] = cm::StepState{e->filled + t, 0u, 0u, 0u};
  int rc = 0;
  do {
    if (hipMemcpy(d_embs, embs, (size_t)n * d.hidden * 4, hipMemcpyHostToDevice) != hipSuccess ||
        hipMemcpy(d_cos, cos_all, (size_t)n * half * 4, hipMemcpyHostToDevice) != hipSuccess ||
        hipMemcpy(d_sin, sin_all, (size_t)n * half * 4, hipMemcpyHostToDevice) != hipSuccess ||
        hipMemcpy(d_sts, sv.data(), (size_t)n * sizeof(cm::StepState), hipMemcpyHostToDevice) != hipSuccess) {
      rc = fail(e, "prefill staging copy failed");
      break;
    }
    if (e->prefill_batched) {
      // chunks of PREFILL_CHUNK tokens, every layer over the whole chunk
      if (ensure_prefill_buffers(e)) {
        rc = 1;
        break;
      }
      for (uint32_t c0 = 0; c0 < n; c0 += PREFILL_CHUNK) {
        const uint32_t T = std::min(PREFILL_CHUNK, n - c0);
        (void)hipMemcpyAsync(e->pf_h, d_embs + (size_t)c0 * d.hidden, (size_t)T * d.hidden * 4,
                             hipMemcpyDeviceToDevice, e->stream);
        prefill_chunk(e, d_cos + (size_t)c0 * half, d_sin + (size_t)c0 * half, T, e->filled + c0, scale);
      }
    } else {
      // one decode step per token (CAMELID_HIP_PREFILL=token; the reference's CPU prefill of
      // K-quant layers is likewise a per-token loop of row dots, inference.rs:2462-2473)
      if (nf_begin(e)) {
        rc = 1;
        break;
      }
      for (uint32_t t = 0; t < n; ++t) {
        (void)hipMemcpyAsync(e->h, d_embs + (size_t)t * d.hidden, d.hidden * 4, hipMemcpyDeviceToDevice, e->stream);
        (void)hipMemcpyAsync(e->st, d_sts + t, sizeof(cm::StepState), hipMemcpyDeviceToDevice, e->stream);
        e->cur_pos = sv[t].pos;
        run_stack(e, d_cos + (size_t)t * half, d_sin + (size_t)t * half, 0, scale);
      }
      if (nf_end(e)) {
        rc = 1;
        break;
      }
    }
    if (check_launch(e)) {
      rc = 1;
      break;
    }
    hipError_t st = hipStreamSynchronize(e->stream);
    if (st != hipSuccess) {
      rc = fail(e, std::string("prefill: ") + hipGetErrorString(st));
      break;
    }
    if (nf_failed(e)) {
      rc = 1;
      break;
    }
  } while (0);
  (void)hipFree(d_embs);
  (void)hipFree(d_cos);
  (void)hipFree(d_sin);
  (void)hipFree(d_sts);
  if (rc) {
    e->filled = 0;
    return rc;
  }
  e->filled += n;
  return 0;
}

int camelid_hip_verify(camelid_hip_engine* e, const float* embs, const float* cos_all, const float* sin_all,
                       uint32_t base_position, uint32_t k, float scale, uint32_t* tokens_out) {
  if (!e) return fail(nullptr, "null engine");
  if (!ready(e)) return fail(e, "weights not ready");
  if (!embs || !cos_all || !sin_all || !tokens_out) return fail(e, "null argument");
  const camelid_hip_dims& d = e->d;
  if (k == 0 || k > CAMELID_MAX_VERIFY_K) return fail(e, "verify: k out of 1..=8");
  if ((size_t)base_position + k > d.max_pos) return fail(e, "verify beyond max_pos");
  if (base_position > e->filled) return fail(e, "verify: base_position past the filled cache");
  if (!std::isfinite(scale)) return fail(e, "attention score scale must be finite");
  HIP_TRY(e, hipSetDevice(e->device));
  const size_t half = d.rope_dim / 2, K = CAMELID_MAX_VERIFY_K;
  if (!e->v_embs && (dev_alloc(e, &e->v_embs, K * d.hidden) || dev_alloc(e, &e->v_cos, K * half) ||
                     dev_alloc(e, &e->v_sin, K * half) || dev_alloc(e, &e->v_logits, K * (size_t)d.vocab) ||
                     dev_alloc(e, &e->v_tok, K) || dev_alloc(e, &e->v_pv, K * cm::AMR_PARTS) ||
                     dev_alloc(e, &e->v_pi, K * cm::AMR_PARTS)))
    return 1;
  HIP_TRY(e, hipMemcpy(e->v_embs, embs, (size_t)k * d.hidden * 4, hipMemcpyHostToDevice));
  HIP_TRY(e, hipMemcpy(e->v_cos, cos_all, (size_t)k * half * 4, hipMemcpyHostToDevice));
  HIP_TRY(e, hipMemcpy(e->v_sin, sin_all, (size_t)k * half * 4, hipMemcpyHostToDevice));
  const bool batched = e->prefill_batched && (e->out_quant != CAMELID_Q8_0 || e->out.rows % 4 == 0);
  if (batched) {
    // one batched forward (the prefill chunk path: bit-identical to token steps), then the
    // final norm, lm_head GEMM and one argmax per token
    if (ensure_prefill_buffers(e)) return 1;
    HIP_TRY(e, hipMemcpyAsync(e->pf_h, e->v_embs, (size_t)k * d.hidden * 4, hipMemcpyDeviceToDevice, e->stream));
    prefill_chunk(e, e->v_cos, e->v_sin, k, base_position, scale);
    const bool kout = e->out_quant != CAMELID_Q8_0;
    launch_rmsnorm_quant(e->pf_h, e->out_norm, d.hidden, d.eps, e->pf_xq, e->pf_xs, nullptr, e->stream,
                         cm::Prefetch{}, k, kout ? e->pf_kd : nullptr, kout ? e->pf_kq : nullptr,
                         kout ? e->pf_kbs : nullptr);
    if (kout)
      launch_kgemm(e->out_k, k, e->pf_kd, e->pf_kq, e->v_logits, d.vocab, nullptr, e->stream, e->pf_kqt);
    else
      launch_gemm(e->out, k, e->pf_xq, e->pf_xs, e->v_logits, nullptr, e->stream);
    CM_LAUNCH(cm::k_argmax_rows_part, dim3(cm::AMR_PARTS, k), dim3(256), 0, e->stream, e->v_logits, (int)d.vocab,
              e->v_pv, e->v_pi);
    CM_LAUNCH(cm::k_argmax_rows_finish, dim3(k), dim3(64), 0, e->stream, e->v_pv, e->v_pi, e->v_tok);
  } else {
    // k single-token steps; the head writes each greedy token to v_tok[step]
    *e->p_st = cm::StepState{base_position, 0u, 0u, 0u};
    HIP_TRY(e, hipMemcpyAsync(e->st, e->p_st, sizeof(cm::StepState), hipMemcpyHostToDevice, e->stream));
    if (nf_begin(e)) return 1;
    for (uint32_t t = 0; t < k; ++t) {
      HIP_TRY(e, hipMemcpyAsync(e->h, e->v_embs + (size_t)t * d.hidden, d.hidden * 4, hipMemcpyDeviceToDevice,
                                e->stream));
      e->cur_pos = base_position + t;
      run_stack(e, e->v_cos + (size_t)t * half, e->v_sin + (size_t)t * half, 0, scale);
      run_head(e, e->v_tok, k);
    }
    if (nf_end(e)) return 1;
  }
  if (check_launch(e)) {
    e->filled = 0;
    return 1;
  }
  hipError_t st = hipStreamSynchronize(e->stream);
  if (st != hipSuccess) {
    e->filled = 0;
    return fail(e, std::string("verify: ") + hipGetErrorString(st));
  }
  if (nf_failed(e)) return 1;
  HIP_TRY(e, hipMemcpy(tokens_out, e->v_tok, (size_t)k * 4, hipMemcpyDeviceToHost));
  return 0;
}

int camelid_hip_generate(camelid_hip_engine* e, uint32_t token, uint32_t position, uint32_t n_steps, float scale,
                         uint32_t* tokens_out) {
  if (!e) return fail(nullptr, "null engine");
  if (!ready(e) || !e->embd_set) return fail(e, "weights or embedding not ready");
  if (!tokens_out) return fail(e, "null argument");
  const camelid_hip_dims& d = e->d;
  if ((size_t)position + n_steps > e->rope_rows) return fail(e, "rope table does not cover the requested steps");
  if (n_steps > e->tokens_cap) return fail(e, "more steps than the token ring holds");
  if (token >= d.vocab) return fail(e, "token id out of range");
  if (!std::isfinite(scale)) return fail(e, "attention score scale must be finite");
  if (n_steps == 0) return 0;
  HIP_TRY(e, hipSetDevice(e->device));
  const bool graph = e->use_graph && !e->profiling && !e->capture;
  *e->p_st = cm::StepState{position, token, 0u, 0u};
  HIP_TRY(e, hipMemcpyAsync(e->st, e->p_st, sizeof(cm::StepState), hipMemcpyHostToDevice, e->stream));
  if (nf_begin(e)) return 1;
  if (graph) {  // the graphs this call's positions need (the split attention from att_split_min on)
    const uint64_t first = (uint64_t)position + 1, last = (uint64_t)position + n_steps;
    const bool split_used = e->att_split_min && last >= e->att_split_min;
    const bool single_used = !e->att_split_min || first < e->att_split_min;
    if ((single_used && ensure_graph(e, scale, 0)) || (split_used && ensure_graph(e, scale, 1))) return 1;
  }
  for (uint32_t t = 0; t < n_steps; ++t) {
    e->cur_pos = position + t;
    if (graph) {
      const int mode = att_split(e) ? 1 : 0;
      hipError_t st = hipGraphLaunch(e->graph_exec[mode], e->stream);
      if (st != hipSuccess) {
        e->filled = 0;
        return fail(e, std::string("graph launch failed: ") + hipGetErrorString(st));
      }
    } else {
      enqueue_device_step(e, scale);
    }
  }
  if (check_launch(e)) {
    e->filled = 0;
    return 1;
  }
  if (nf_end(e)) return 1;
  hipError_t st = hipStreamSynchronize(e->stream);
  if (st != hipSuccess) {
    e->filled = 0;
    return fail(e, std::string("generate: ") + hipGetErrorString(st));
  }
  if (nf_failed(e)) return 1;
  HIP_TRY(e, hipMemcpy(tokens_out, e->tokens, (size_t)n_steps * 4, hipMemcpyDeviceToHost));
  e->filled = position + n_steps;
  return 0;
}

int camelid_hip_capture_hidden(camelid_hip_engine* e, int enable) {
  if (!e) return fail(nullptr, "null engine");
  e->capture = enable != 0;
  return 0;
}

int camelid_hip_read_hidden(camelid_hip_engine* e, float* out) {
  if (!e || !out) return fail(e, "null argument");
  HIP_TRY(e, hipSetDevice(e->device));
  HIP_TRY(e, hipStreamSynchronize(e->stream));
  HIP_TRY(e, hipMemcpy(out, e->hidden_cap, (size_t)(e->d.n_layers + 1) * e->d.hidden * 4, hipMemcpyDeviceToHost));
  return 0;
}

int camelid_hip_profile_begin(camelid_hip_engine* e) {
  if (!e) return fail(nullptr, "null engine");
  e->recs.clear();
  e->pool_next = 0;
  e->profiling = true;
  return 0;
}

int camelid_hip_profile_end(camelid_hip_engine* e, double* ms, double* bytes, uint64_t* launches, uint32_t n_cat) {
  if (!e) return fail(nullptr, "null engine");
  e->profiling = false;
  HIP_TRY(e, hipStreamSynchronize(e->stream));
  for (uint32_t c = 0; c < n_cat; ++c) {
    if (ms) ms[c] = 0;
    if (bytes) bytes[c] = 0;
    if (launches) launches[c] = 0;
  }
  for (const auto& r : e->recs) {
    if ((uint32_t)r.cat >= n_cat) continue;
    float t = 0.0f;
    HIP_TRY(e, hipEventElapsedTime(&t, r.a, r.b));
    if (ms) ms[r.cat] += t;
    if (bytes) bytes[r.cat] += r.bytes;
    if (launches) launches[r.cat] += 1;
  }
  e->recs.clear();
  e->pool_next = 0;
  return 0;
}

#define G_TRY(expr)                                                                                    \
  do {                                                                                                 \
    hipError_t _st = (expr);                                                                           \
    if (_st != hipSuccess) return fail(nullptr, std::string(#expr) + ": " + hipGetErrorString(_st)); \
  } while (0)

int camelid_hip_phase_stamps(uint64_t* out, size_t n, size_t* n_out) {
  if (!out || !n_out) return fail(nullptr, "null argument");
  const size_t na = (size_t)cm::ATT_STAMP_LAYERS * cm::ATT_STAMP_HEADS * cm::ATT_NSTAMP;
  const size_t ng = (size_t)2 * cm::GEMV_STAMP_WGS * cm::GEMV_NSTAMP;
  const size_t nsp = (size_t)2 * cm::SPLIT_STAMP_WGS * cm::SPLIT_NSTAMP;
  const size_t nao = (size_t)cm::ATT_STAMP_LAYERS * 2 * cm::AO_NSTAMP;
  const size_t total = na + ng + nsp + nao;
#ifdef CM_STAMPS
  G_TRY(hipDeviceSynchronize());
  const size_t m1 = std::min(n, na), m2 = std::min(n - m1, ng), m3 = std::min(n - m1 - m2, nsp),
               m4 = std::min(n - m1 - m2 - m3, nao);
  G_TRY(hipMemcpyFromSymbol(out, HIP_SYMBOL(cm::g_att_stamps), m1 * sizeof(uint64_t), 0, hipMemcpyDeviceToHost));
  if (m2)
    G_TRY(hipMemcpyFromSymbol(out + m1, HIP_SYMBOL(cm::g_gemv_stamps), m2 * sizeof(uint64_t), 0,
                              hipMemcpyDeviceToHost));
  if (m3)
    G_TRY(hipMemcpyFromSymbol(out + m1 + m2, HIP_SYMBOL(cm::g_split_stamps), m3 * sizeof(uint64_t), 0,
                              hipMemcpyDeviceToHost));
  if (m4)
    G_TRY(hipMemcpyFromSymbol(out + m1 + m2 + m3, HIP_SYMBOL(cm::g_ao_stamps), m4 * sizeof(uint64_t), 0,
                              hipMemcpyDeviceToHost));
  *n_out = m1 + m2 + m3 + m4;
  return 0;
#else
  (void)n;
  (void)total;
  *n_out = 0;
  return fail(nullptr, "phase stamps are recorded only by the measurement build (libcamelid_hip_stamps.so)");
#endif
}

int camelid_hip_device_info(char* name, size_t name_len, int* n_cu) {
  int dev = 0;
  if (const char* s = std::getenv("CAMELID_HIP_DEVICE")) dev = std::atoi(s);
  hipDeviceProp_t p;
  hipError_t st = hipGetDeviceProperties(&p, dev);
  if (st != hipSuccess) return fail(nullptr, std::string("hipGetDeviceProperties: ") + hipGetErrorString(st));
  if (name && name_len) std::snprintf(name, name_len, "%s%s%s", p.name, p.name[0] ? " " : "", p.gcnArchName);
  if (n_cu) *n_cu = p.multiProcessorCount;
  return 0;
}

// HBM bandwidth probe: STREAM's triad a = b + s*c and a read-only pass over one array, each
// workgroup on a contiguous span, with nontemporal (streaming) loads and stores, the fastest
// of the forms measured on MI355X for arrays far beyond the caches.
typedef float bw_v4 __attribute__((ext_vector_type(4)));
constexpr int BW_TRIAD_U = 4, BW_TRIAD_NT = 256;  // 16-byte elements per thread, threads
constexpr int BW_READ_U = 16, BW_READ_NT = 512;
constexpr size_t BW_GRAIN = (size_t)BW_READ_U * BW_READ_NT * 16;  // bytes; a multiple of the triad span
__global__ __launch_bounds__(BW_TRIAD_NT) void k_bw_triad(bw_v4* __restrict__ a, const bw_v4* __restrict__ b,
                                                          const bw_v4* __restrict__ c, float sc) {
  const size_t base = (size_t)blockIdx.x * BW_TRIAD_NT * BW_TRIAD_U + threadIdx.x;
  bw_v4 x[BW_TRIAD_U], y[BW_TRIAD_U];
#pragma unroll
  for (int u = 0; u < BW_TRIAD_U; ++u) {
    x[u] = __builtin_nontemporal_load(b + base + u * BW_TRIAD_NT);
    y[u] = __builtin_nontemporal_load(c + base + u * BW_TRIAD_NT);
  }
#pragma unroll
  for (int u = 0; u < BW_TRIAD_U; ++u) __builtin_nontemporal_store(x[u] + sc * y[u], a + base + u * BW_TRIAD_NT);
}
__global__ __launch_bounds__(BW_READ_NT) void k_bw_read(const bw_v4* __restrict__ b, float* __restrict__ sink) {
  const size_t base = (size_t)blockIdx.x * BW_READ_NT * BW_READ_U + threadIdx.x;
  bw_v4 x[BW_READ_U];
#pragma unroll
  for (int u = 0; u < BW_READ_U; ++u) x[u] = __builtin_nontemporal_load(b + base + u * BW_READ_NT);
  float acc = 0.0f;
#pragma unroll
  for (int u = 0; u < BW_READ_U; ++u) acc += (x[u].x + x[u].y) + (x[u].z + x[u].w);
  if (acc == -1.0f) sink[threadIdx.x] = acc;  // (the arrays hold zeros: never taken, but not provable)
}

int camelid_hip_hbm_bandwidth(size_t bytes_per_array, uint32_t reps, double* triad_gbs, double* read_gbs) {
  if (!triad_gbs || !read_gbs || reps == 0) return fail(nullptr, "null argument");
  if (bytes_per_array == 0 || bytes_per_array % BW_GRAIN)
    return fail(nullptr, "bytes_per_array must be a positive multiple of " + std::to_string(BW_GRAIN));
  const size_t n4 = bytes_per_array / 16;
  bw_v4 *a = nullptr, *b = nullptr, *c = nullptr;
  float* sink = nullptr;
  hipEvent_t e0 = nullptr, e1 = nullptr;
  int rc = 0;
  if (hipMalloc(&a, bytes_per_array) != hipSuccess || hipMalloc(&b, bytes_per_array) != hipSuccess ||
      hipMalloc(&c, bytes_per_array) != hipSuccess || hipMalloc(&sink, BW_READ_NT * 4) != hipSuccess) {
    rc = fail(nullptr, "hbm_bandwidth: allocation failed");
  } else if (hipMemset(a, 0, bytes_per_array) != hipSuccess || hipMemset(b, 0, bytes_per_array) != hipSuccess ||
             hipMemset(c, 0, bytes_per_array) != hipSuccess || hipEventCreate(&e0) != hipSuccess ||
             hipEventCreate(&e1) != hipSuccess || hipDeviceSynchronize() != hipSuccess) {
    rc = fail(nullptr, "hbm_bandwidth: set-up failed");
  } else {
    // best of `reps` timed passes after one warm-up pass, the triads first, then the reads
    auto best_of = [&](auto launch, double moved, double* out) {
      double best = 0.0;
      for (uint32_t i = 0; i <= reps; ++i) {
        float ms = 0.0f;
        (void)hipEventRecord(e0, nullptr);
        launch();
        (void)hipEventRecord(e1, nullptr);
        if (hipEventSynchronize(e1) != hipSuccess || hipEventElapsedTime(&ms, e0, e1) != hipSuccess)
          return fail(nullptr, "hbm_bandwidth: timing failed");
        if (i > 0 && ms > 0.0f) best = std::max(best, moved / (ms * 1e-3) / 1e9);
      }
      *out = best;
      return 0;
    };
    rc = best_of([&] { hipLaunchKernelGGL(k_bw_triad, dim3((uint32_t)(n4 / (BW_TRIAD_NT * BW_TRIAD_U))),
                                          dim3(BW_TRIAD_NT), 0, nullptr, a, b, c, 3.0f); },
                 3.0 * bytes_per_array, triad_gbs);
    if (!rc)
      rc = best_of([&] { hipLaunchKernelGGL(k_bw_read, dim3((uint32_t)(n4 / (BW_READ_NT * BW_READ_U))),
                                            dim3(BW_READ_NT), 0, nullptr, b, sink); },
                   1.0 * bytes_per_array, read_gbs);
    if (!rc && hipGetLastError() != hipSuccess) rc = fail(nullptr, "hbm_bandwidth: launch failed");
  }
  if (e0) (void)hipEventDestroy(e0);
  if (e1) (void)hipEventDestroy(e1);
  (void)hipFree(a);
  (void)hipFree(b);
  (void)hipFree(c);
  (void)hipFree(sink);
  return rc;
}

// ------------------------------------------------------------------ kernel-level ABI

int camelid_hip_malloc(void** ptr, size_t bytes) {
  if (!ptr) return fail(nullptr, "null argument");
  G_TRY(hipMalloc(ptr, std::max<size_t>(bytes, 256)));
  return 0;
}
int camelid_hip_free(void* ptr) {
  G_TRY(hipFree(ptr));
  return 0;
}
int camelid_hip_memcpy_htod(void* dst, const void* src, size_t bytes) {
  G_TRY(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice));
  return 0;
}
int camelid_hip_memcpy_dtoh(void* dst, const void* src, size_t bytes) {
  G_TRY(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost));
  return 0;
}
int camelid_hip_synchronize(void) {
  G_TRY(hipDeviceSynchronize());
  return 0;
}

int camelid_q8_0_repack(const uint8_t* src, size_t rows, size_t k, uint8_t layout, int8_t* quants_out,
                        uint16_t* scales_out) {
  if (!src || !quants_out || !scales_out) return fail(nullptr, "null argument");
  if (layout != 34 && layout != 36) return fail(nullptr, "layout must be 34 or 36");
  if (k % 32) return fail(nullptr, "k must be a multiple of 32");
  repack_parallel(src, rows, k, layout, quants_out, scales_out);
  return 0;
}

static int launch_status(const char* what) {
  hipError_t st = hipGetLastError();
  if (st != hipSuccess) return fail(nullptr, std::string(what) + ": " + hipGetErrorString(st));
  if (!g_launch_error.empty()) {
    const std::string m = g_launch_error;
    g_launch_error.clear();
    return fail(nullptr, std::string(what) + ": " + m);
  }
  return 0;
}

int camelid_hip_q8_0_gemv(const int8_t* wq, const uint16_t* wd, uint32_t rows, uint32_t k, const int8_t* xq,
                          const float* xs, float* y, const float* resid, void* stream) {
  if (!wq || !wd || !xq || !xs || !y) return fail(nullptr, "null argument");
  if (k % 32 || k == 0 || rows == 0) return fail(nullptr, "k must be a nonzero multiple of 32 and rows > 0");
  if (cm::gemv_lds_bytes((int)k) > 64 * 1024) return fail(nullptr, "k too large for the GEMV LDS stage");
  Q8Mat m;
  m.q = const_cast<int8_t*>(wq);
  m.d = const_cast<uint16_t*>(wd);
  m.rows = rows;
  m.k = k;
  launch_gemv(m, xq, xs, y, resid, (hipStream_t)stream);
  return launch_status("q8_0_gemv");
}

int camelid_hip_q8_0_block_dots(const int8_t* wq, uint32_t rows, uint32_t k, const int8_t* xq, int32_t* out,
                                void* stream) {
  if (!wq || !xq || !out) return fail(nullptr, "null argument");
  if (k % 32 || k == 0 || rows == 0) return fail(nullptr, "k must be a nonzero multiple of 32 and rows > 0");
  hipLaunchKernelGGL(cm::k_q8_block_dots, dim3(rows), dim3(64), 0, (hipStream_t)stream, wq, (int)k, xq, out);
  return launch_status("q8_0_block_dots");
}

int camelid_hip_rmsnorm_quantize(const float* x, const float* w, uint32_t n, float eps, int8_t* xq, float* xs, float* y,
                                 void* stream) {
  if (!x || !w || !xq || !xs) return fail(nullptr, "null argument");
  if (n == 0 || n % 32 || n > (uint32_t)cm::SEG_MAX_N) return fail(nullptr, "n must be a multiple of 32 in (0, 16384]");
  if (((uintptr_t)x | (uintptr_t)w | (uintptr_t)xq | (uintptr_t)y) & 15u)
    return fail(nullptr, "x, w, xq and y must be 16-byte aligned");
  launch_rmsnorm_quant(x, w, n, eps, xq, xs, y, (hipStream_t)stream);
  return launch_status("rmsnorm_quantize");
}

int camelid_hip_quantize_q8_0(const float* x, uint32_t n, int8_t* xq, float* xs, void* stream) {
  if (!x || !xq || !xs) return fail(nullptr, "null argument");
  if (n % 32) return fail(nullptr, "n must be a multiple of 32");
  if (n == 0) return 0;
  hipLaunchKernelGGL(cm::k_quantize_q8_0, dim3((n + 255) / 256), dim3(256), 0, (hipStream_t)stream, x, (int)n, xq,
                     xs);
  return launch_status("quantize_q8_0");
}

int camelid_hip_silu_mul_quantize(const float* gu, uint32_t n, int8_t* xq, float* xs, float* act, void* stream) {
  if (!gu || !xq || !xs) return fail(nullptr, "null argument");
  if (n % 32) return fail(nullptr, "n must be a multiple of 32");
  if (n == 0) return 0;
  hipLaunchKernelGGL(cm::k_silu_mul_quant, dim3((n + 255) / 256), dim3(256), 0, (hipStream_t)stream, gu, (int)n, xq,
                     xs, act, prefetch_of((const Q8Mat*)nullptr), (float*)nullptr, (int8_t*)nullptr, (int32_t*)nullptr);
  return launch_status("silu_mul_quantize");
}

int camelid_hip_rmsnorm_q8_k(const float* x, const float* w, uint32_t n, float eps, float* yd, int8_t* yq,
                             int32_t* ybs, void* stream) {
  if (!x || !w || !yd || !yq || !ybs) return fail(nullptr, "null argument");
  if (n == 0 || n % 256 || n > (uint32_t)cm::SEG_MAX_N) return fail(nullptr, "n must be a multiple of 256, <= 16384");
  if ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(w)) & 15)
    return fail(nullptr, "x and w must be 16-byte aligned");
  int8_t* xq = nullptr;
  float* xs = nullptr;
  if (hipMalloc(&xq, n) != hipSuccess || hipMalloc(&xs, n / 32 * 4) != hipSuccess) {
    (void)hipFree(xq);
    return fail(nullptr, "scratch allocation failed");
  }
  launch_rmsnorm_quant(x, w, n, eps, xq, xs, nullptr, (hipStream_t)stream, cm::Prefetch{}, 1, yd, yq, ybs);
  const int rc = launch_status("rmsnorm_q8_k");
  (void)hipStreamSynchronize((hipStream_t)stream);
  (void)hipFree(xq);
  (void)hipFree(xs);
  return rc;
}

int camelid_hip_silu_mul_q8_k(const float* gu, uint32_t n, float* yd, int8_t* yq, int32_t* ybs, void* stream) {
  if (!gu || !yd || !yq || !ybs) return fail(nullptr, "null argument");
  if (n == 0 || n % 256) return fail(nullptr, "n must be a multiple of 256");
  hipLaunchKernelGGL(cm::k_silu_mul_quant, dim3(n / 256), dim3(256), 0, (hipStream_t)stream, gu, (int)n,
                     (int8_t*)nullptr, (float*)nullptr, (float*)nullptr, prefetch_of((const Q8Mat*)nullptr), yd, yq,
                     ybs);
  return launch_status("silu_mul_q8_k");
}

// The kernel-level entry points that read the position from device memory (d_pos): the
// position is read on the host first and refused unless it lies inside the cache (pos <
// max_pos); the kernels' own guard (cm::kv_pos_bad) is cleared before the launch and read
// after it, so a position changed on the device in between is reported, not used.
static int kv_pos_check(const uint32_t* d_pos, uint32_t max_pos, hipStream_t s, const char* what) {
  uint32_t pos = 0;
  G_TRY(hipStreamSynchronize(s));
  G_TRY(hipMemcpy(&pos, d_pos, 4, hipMemcpyDeviceToHost));
  if (pos >= max_pos)
    return fail(nullptr, std::string(what) + ": position " + std::to_string(pos) + " is outside the KV cache (" +
                             std::to_string(max_pos) + " positions)");
  const uint32_t zero = 0;
  G_TRY(hipMemcpyToSymbol(HIP_SYMBOL(cm::g_kv_pos_error), &zero, 4, 0, hipMemcpyHostToDevice));
  return 0;
}
static int kv_pos_result(hipStream_t s, const char* what) {
  uint32_t bad = 0;
  G_TRY(hipStreamSynchronize(s));
  G_TRY(hipMemcpyFromSymbol(&bad, HIP_SYMBOL(cm::g_kv_pos_error), 4, 0, hipMemcpyDeviceToHost));
  if (bad) return fail(nullptr, std::string(what) + ": the device-side position is outside the KV cache");
  return 0;
}

int camelid_hip_rope_kv(const float* qkv, uint32_t n_heads, uint32_t n_kv, uint32_t hd, uint32_t rope_dim,
                        uint32_t split_half, const float* cos_tab, const float* sin_tab, const float* q_norm,
                        const float* k_norm, float eps, float* qrot, uint16_t* kc, uint16_t* vc, uint32_t layer,
                        uint32_t max_pos, const uint32_t* d_pos, void* stream) {
  if (!qkv || !cos_tab || !sin_tab || !qrot || !kc || !vc || !d_pos) return fail(nullptr, "null argument");
  if (!n_heads || !n_kv || n_heads % n_kv || hd == 0 || hd > 512 || rope_dim > hd || rope_dim % 2)
    return fail(nullptr, "invalid head geometry");
  if (max_pos % 8) return fail(nullptr, "the KV position stride (max_pos) must be a multiple of 8");
  if (kv_pos_check(d_pos, max_pos, (hipStream_t)stream, "rope_kv")) return 1;
  hipLaunchKernelGGL(cm::k_rope_kv, dim3(n_heads + n_kv), dim3(64), 0, (hipStream_t)stream, qkv, (int)n_heads,
                     (int)n_kv, (int)hd, (int)rope_dim, (int)split_half, cos_tab, sin_tab, q_norm, k_norm, eps, qrot,
                     kc, vc, (int)layer, (int)max_pos, d_pos, 0, 0);
  if (launch_status("rope_kv")) return 1;
  return kv_pos_result((hipStream_t)stream, "rope_kv");
}

int camelid_hip_attention_decode(const float* qrot, const uint16_t* kc, const uint16_t* vc, uint32_t layer,
                                 uint32_t n_heads, uint32_t n_kv, uint32_t hd, uint32_t max_pos, const uint32_t* d_pos,
                                 float scale, float* att_out, int8_t* xq, float* xs, void* stream) {
  if (!qrot || !kc || !vc || !d_pos || !att_out || !xq || !xs) return fail(nullptr, "null argument");
  if (!n_heads || !n_kv || n_heads % n_kv || !attention_hd_supported(hd)) return fail(nullptr, "invalid head geometry");
  if (max_pos % 8) return fail(nullptr, "the KV position stride (max_pos) must be a multiple of 8");
  const int slots = attn_ring_slots(max_pos);
  if (slots == 0) return fail(nullptr, "max_pos too large for the decode attention");
  if (kv_pos_check(d_pos, max_pos, (hipStream_t)stream, "attention_decode")) return 1;
  launch_attention<false>(hd, n_heads, slots, (hipStream_t)stream, qrot, (int)n_heads, (int)n_kv,
                          (int)hd, 0, nullptr, nullptr, 0, nullptr, nullptr, 0.0f, const_cast<uint16_t*>(kc),
                          const_cast<uint16_t*>(vc), (int)layer, (int)max_pos, d_pos, scale, att_out, xq, xs,
                          prefetch_of((const Q8Mat*)nullptr));
  if (launch_status("attention_decode")) return 1;
  return kv_pos_result((hipStream_t)stream, "attention_decode");
}

int camelid_hip_attention_decode_split(const float* qrot, const uint16_t* kc, const uint16_t* vc, uint32_t layer,
                                       uint32_t n_heads, uint32_t n_kv, uint32_t hd, uint32_t max_pos,
                                       const uint32_t* d_pos, float scale, float* att_out, int8_t* xq, float* xs,
                                       void* stream) {
  if (!qrot || !kc || !vc || !d_pos || !att_out || !xq || !xs) return fail(nullptr, "null argument");
  if (!n_heads || !n_kv || n_heads % n_kv || !attention_hd_supported(hd)) return fail(nullptr, "invalid head geometry");
  if (max_pos % 8) return fail(nullptr, "the KV position stride (max_pos) must be a multiple of 8");
  const int slots = attn_ring_slots(max_pos);
  if (slots == 0) return fail(nullptr, "max_pos too large for the decode attention");
  if (kv_pos_check(d_pos, max_pos, (hipStream_t)stream, "attention_decode_split")) return 1;
  float *g_sc = nullptr, *g_mx = nullptr;
  if (hipMalloc(&g_sc, (size_t)n_heads * max_pos * 4) != hipSuccess ||
      hipMalloc(&g_mx, (size_t)n_heads * ((max_pos + 255) / 256) * 4) != hipSuccess) {
    (void)hipFree(g_sc);
    return fail(nullptr, "attention_decode_split: scratch allocation failed");
  }
  launch_attention_split<false>(hd, n_heads, slots, (hipStream_t)stream, qrot, (int)n_heads, (int)n_kv, (int)hd, 0,
                                nullptr, nullptr, 0, nullptr, nullptr, 0.0f, const_cast<uint16_t*>(kc),
                                const_cast<uint16_t*>(vc), (int)layer, (int)max_pos, d_pos, scale, g_sc, g_mx, att_out,
                                xq, xs, prefetch_of((const Q8Mat*)nullptr));
  const int rc = launch_status("attention_decode_split");
  const hipError_t st = hipStreamSynchronize((hipStream_t)stream);
  (void)hipFree(g_sc);
  (void)hipFree(g_mx);
  if (!rc && st != hipSuccess) return fail(nullptr, std::string("attention_decode_split: ") + hipGetErrorString(st));
  return rc ? rc : kv_pos_result((hipStream_t)stream, "attention_decode_split");
}

// ---- the split attention without allocation (camelid_hip_attention_decode_split_noalloc)
// Its score scratch: a file-scope device array, one copy per GPU, held until the process
// ends.  Host code never passes the array's name to a kernel (on the host it is a stand-in,
// not a device address): the first call on each device looks up that device's copy with
// hipGetSymbolAddress and keeps the address per device.
constexpr size_t NOALLOC_SCORE_FLOATS = (size_t)1 << 20;  // n_heads * max_pos score words (4 MiB)
constexpr size_t NOALLOC_MAX_FLOATS = (size_t)1 << 14;    // n_heads * ceil(max_pos / 256) slice maxima
static __device__ __align__(256) float scratch[NOALLOC_SCORE_FLOATS + NOALLOC_MAX_FLOATS];
constexpr int NOALLOC_MAX_DEVICES = 64;
static std::atomic<float*> g_scratch_ptr[NOALLOC_MAX_DEVICES];

// This device's copy of `scratch` (looked up once per device, with that device current).
static int scratch_for_current_device(float** out) {
  int dev = 0;
  G_TRY(hipGetDevice(&dev));
  if (dev < 0 || dev >= NOALLOC_MAX_DEVICES) return fail(nullptr, "attention_decode_split_noalloc: device index out of range");
  float* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (!p) {
    void* sym = nullptr;
    const hipError_t st = hipGetSymbolAddress(&sym, HIP_SYMBOL(scratch));
    if (st != hipSuccess || !sym)
      return fail(nullptr, std::string("attention_decode_split_noalloc: hipGetSymbolAddress(scratch): ") +
                               hipGetErrorString(st));
    p = static_cast<float*>(sym);
    g_scratch_ptr[dev].store(p, std::memory_order_release);
  }
  *out = p;
  return 0;
}

int camelid_hip_attention_decode_split_noalloc(const float* qrot, const uint16_t* kc, const uint16_t* vc,
                                               uint32_t layer, uint32_t n_heads, uint32_t n_kv, uint32_t hd,
                                               uint32_t max_pos, const uint32_t* d_pos, float scale, float* att_out,
                                               int8_t* xq, float* xs, void* stream) {
  if (!qrot || !kc || !vc || !d_pos || !att_out || !xq || !xs) return fail(nullptr, "null argument");
  if (!n_heads || !n_kv || n_heads % n_kv || !attention_hd_supported(hd)) return fail(nullptr, "invalid head geometry");
  if (max_pos % 8) return fail(nullptr, "the KV position stride (max_pos) must be a multiple of 8");
  const size_t n_scores = (size_t)n_heads * max_pos;
  const size_t n_max = (size_t)n_heads * ((max_pos + ATT_SLICE - 1) / ATT_SLICE);
  if (n_scores > NOALLOC_SCORE_FLOATS || n_max > NOALLOC_MAX_FLOATS)
    return fail(nullptr, "attention_decode_split_noalloc: n_heads * max_pos = " + std::to_string(n_scores) +
                             " exceeds the static scratch (" + std::to_string(NOALLOC_SCORE_FLOATS) + " scores)");
  const int slots = attn_ring_slots(max_pos);
  if (slots == 0) return fail(nullptr, "max_pos too large for the decode attention");
  float* base = nullptr;
  if (scratch_for_current_device(&base)) return 1;
  if (kv_pos_check(d_pos, max_pos, (hipStream_t)stream, "attention_decode_split_noalloc")) return 1;
  // every scratch word the output kernel reads is written by the scores kernel of this call
  launch_attention_split<false>(hd, n_heads, slots, (hipStream_t)stream, qrot, (int)n_heads, (int)n_kv, (int)hd, 0,
                                nullptr, nullptr, 0, nullptr, nullptr, 0.0f, const_cast<uint16_t*>(kc),
                                const_cast<uint16_t*>(vc), (int)layer, (int)max_pos, d_pos, scale, base,
                                base + NOALLOC_SCORE_FLOATS, att_out, xq, xs, prefetch_of((const Q8Mat*)nullptr));
  if (launch_status("attention_decode_split_noalloc")) return 1;
  return kv_pos_result((hipStream_t)stream, "attention_decode_split_noalloc");
}

int camelid_hip_rmsnorm_q8_0_gemv(const int8_t* wq, const uint16_t* wd, uint32_t rows, uint32_t k, const float* x,
                                  const float* nw, float eps, float* y, void* stream) {
  if (!wq || !wd || !x || !nw || !y) return fail(nullptr, "null argument");
  if (!cm::gu_fused_k((int)k) || rows == 0) return fail(nullptr, "k must be 2048, 3072 or 4096 and rows > 0");
  Q8Mat m;
  m.q = const_cast<int8_t*>(wq);
  m.d = const_cast<uint16_t*>(wd);
  m.rows = rows;
  m.k = k;
  launch_gemv_norm(m, x, nw, eps, y, (hipStream_t)stream);
  return launch_status("rmsnorm_q8_0_gemv");
}

int camelid_hip_gate_up_silu(const int8_t* wq, const uint16_t* wd, uint32_t ffn, uint32_t k, const int8_t* xq,
                             const float* xs, const float* x, const float* nw, float eps, int8_t* aq, float* as,
                             void* stream) {
  if (!wq || !wd || !aq || !as || (x ? !nw : (!xq || !xs))) return fail(nullptr, "null argument");
  if (!cm::gu_fused_k((int)k) || ffn == 0 || ffn % 32) return fail(nullptr, "k must be 2048, 3072 or 4096; ffn a nonzero multiple of 32");
  if (x && !cm::gu_norm_k((int)k)) return fail(nullptr, "the in-kernel RMSNorm takes k = 2048, 3072 or 4096");
  const hipStream_t s = (hipStream_t)stream;
  switch (k) {
#define CM_GU(K)                                                                                                   \
  case K:                                                                                                          \
    if (x && cm::gu_norm_k(K))                                                                                     \
      hipLaunchKernelGGL((cm::k_gemv_gu_silu<K, cm::GN_NT, cm::gu_norm_k(K)>), dim3(ffn / 32), dim3(cm::GN_NT), 0, \
                         s, wq, wd, (const int8_t*)nullptr, (const float*)nullptr, x, nw, eps, aq, as,             \
                         (int)(ffn / 32));                                                                         \
    else                                                                                                           \
      hipLaunchKernelGGL((cm::k_gemv_gu_silu<K, cm::GU_NT, false>), dim3(ffn / 32), dim3(cm::GU_NT), 0, s, wq, wd, \
                         xq, xs, (const float*)nullptr, (const float*)nullptr, 0.0f, aq, as, (int)(ffn / 32));     \
    break;
    CM_GU(2048) CM_GU(3072) CM_GU(4096)
#undef CM_GU
  }
  return launch_status("gate_up_silu");
}

int camelid_hip_q8_0_gemm(const int8_t* wq, const uint16_t* wd, uint32_t rows, uint32_t k, const int8_t* xq,
                          const float* xs, uint32_t tokens, float* y, const float* resid, void* stream) {
  if (!wq || !wd || !xq || !xs || !y) return fail(nullptr, "null argument");
  if (k % 32 || k == 0 || rows == 0 || tokens == 0) return fail(nullptr, "k must be a nonzero multiple of 32, rows and tokens > 0");
  if (rows % 4) return fail(nullptr, "rows must be a multiple of 4");
  Q8Mat m;
  m.q = const_cast<int8_t*>(wq);
  m.d = const_cast<uint16_t*>(wd);
  m.rows = rows;
  m.k = k;
  if (q8_scan_inf_scales(&m, (hipStream_t)stream)) return 1;
  launch_gemm(m, tokens, xq, xs, y, resid, (hipStream_t)stream);
  return launch_status("q8_0_gemm");
}

int camelid_hip_attention_prefill(const float* qrot, const uint16_t* kc, const uint16_t* vc, uint32_t layer,
                                  uint32_t n_heads, uint32_t n_kv, uint32_t hd, uint32_t max_pos, uint32_t pos0,
                                  uint32_t tokens, float scale, float* att_out, int8_t* xq, float* xs, void* stream) {
  if (!qrot || !kc || !vc || !xq || !xs) return fail(nullptr, "null argument");
  if (!n_heads || !n_kv || n_heads % n_kv || !attention_hd_supported(hd)) return fail(nullptr, "invalid head geometry");
  if (max_pos % 8) return fail(nullptr, "the KV position stride (max_pos) must be a multiple of 8");
  if (tokens == 0 || (size_t)pos0 + tokens > max_pos) return fail(nullptr, "positions beyond max_pos");
  if (((size_t)pos0 + tokens) * 4 > 64 * 1024) return fail(nullptr, "more than 16384 positions");
  // the tiled kernel whenever it applies (any token count), unless CAMELID_HIP_ATT_TILE=0;
  // its score scratch is allocated for the call
  const char* te = std::getenv("CAMELID_HIP_ATT_TILE");
  const bool tiled = !(te && std::atoi(te) == 0) && cm::apt_hd_ok((int)hd) && n_heads / n_kv <= (uint32_t)cm::APT_R;
  float* scratch = nullptr;
  if (tiled && hipMalloc(&scratch, attn_prefill_scratch(n_heads, n_kv, tokens, pos0 + tokens) * 4) != hipSuccess)
    return fail(nullptr, "scratch allocation failed");
  launch_attn_prefill(hd, n_heads, n_kv, tokens, qrot, kc, vc, (int)layer, (int)max_pos, (int)pos0, scale, att_out,
                      xq, xs, (hipStream_t)stream, scratch, 1, 0);
  if (scratch) {
    const hipError_t st = hipStreamSynchronize((hipStream_t)stream);
    (void)hipFree(scratch);
    if (st != hipSuccess) return fail(nullptr, std::string("attention_prefill: ") + hipGetErrorString(st));
  }
  return launch_status("attention_prefill");
}

int camelid_hip_quantize_q8_k(const float* x, uint32_t n, float* yd, int8_t* yq, int32_t* ybs, void* stream) {
  if (!x || !yd || !yq || !ybs) return fail(nullptr, "null argument");
  if (n == 0 || n % 256) return fail(nullptr, "n must be a nonzero multiple of 256");
  hipLaunchKernelGGL(cm::k_quantize_q8k, dim3(n / 256), dim3(256), 0, (hipStream_t)stream, x, yd, yq, ybs);
  return launch_status("quantize_q8_k");
}

int camelid_kquant_repack(uint8_t quant, const uint8_t* src, size_t rows, size_t k, uint8_t* a, uint8_t* b,
                          int8_t* sc, uint16_t* d) {
  if (!src || !a || !b) return fail(nullptr, "null argument");
  if (quant != CAMELID_Q4_K && quant != CAMELID_Q6_K) return fail(nullptr, "quant must be Q4_K or Q6_K");
  if (quant == CAMELID_Q6_K && (!sc || !d)) return fail(nullptr, "null argument");
  if (k % 256) return fail(nullptr, "k must be a multiple of 256");
  kq_split_rows(quant, src, 0, rows, k, a, b, sc, d);
  return 0;
}

int camelid_hip_kquant_gemv(uint8_t quant, const uint8_t* a, const uint8_t* b, const int8_t* sc, const uint16_t* d,
                            uint32_t rows, uint32_t k, const float* yd, const int8_t* yq, const int32_t* ybs,
                            float* y, const float* resid, void* stream) {
  if (!a || !b || !yd || !yq || !ybs || !y) return fail(nullptr, "null argument");
  if (quant != CAMELID_Q4_K && quant != CAMELID_Q6_K) return fail(nullptr, "quant must be Q4_K or Q6_K");
  if (quant == CAMELID_Q6_K && (!sc || !d)) return fail(nullptr, "null argument");
  if (rows == 0 || k == 0 || k % 256 || k > 16384) return fail(nullptr, "k must be a multiple of 256, at most 16384");
  KMat m;
  m.quant = quant;
  m.a = const_cast<uint8_t*>(a);
  m.b = const_cast<uint8_t*>(b);
  m.sc = const_cast<int8_t*>(sc);
  m.d = const_cast<uint16_t*>(d);
  m.rows = rows;
  m.k = k;
  launch_kgemv(m, yd, yq, ybs, y, resid, nullptr, nullptr, (hipStream_t)stream);
  return launch_status("kquant_gemv");
}

int camelid_hip_kquant_gemm(uint8_t quant, const uint8_t* a, const uint8_t* b, const int8_t* sc, const uint16_t* d,
                            uint32_t rows, uint32_t k, uint32_t tokens, const float* yd, const int8_t* yq, float* y,
                            uint32_t ldy, const float* resid, void* stream) {
  if (!a || !b || !yd || !yq || !y) return fail(nullptr, "null argument");
  if (quant != CAMELID_Q4_K && quant != CAMELID_Q6_K) return fail(nullptr, "quant must be Q4_K or Q6_K");
  if (quant == CAMELID_Q6_K && (!sc || !d)) return fail(nullptr, "null argument");
  if (rows == 0 || k == 0 || k % 256 || k > 16384) return fail(nullptr, "k must be a multiple of 256, at most 16384");
  if (tokens == 0 || ldy < rows) return fail(nullptr, "tokens must be nonzero and ldy >= rows");
  if ((uint64_t)tokens * k >= (1ull << 31) || (uint64_t)rows * k >= (1ull << 32))
    return fail(nullptr, "kquant_gemm: tokens * k must be below 2^31 and rows * k below 2^32 (32-bit GEMM offsets)");
  KMat m;
  m.quant = quant;
  m.a = const_cast<uint8_t*>(a);
  m.b = const_cast<uint8_t*>(b);
  m.sc = const_cast<int8_t*>(sc);
  m.d = const_cast<uint16_t*>(d);
  m.rows = rows;
  m.k = k;
  // Q6_K chunks: the class-major GEMM with its weight planes and activation copy in temporary
  // allocations for this call (the stream is synchronized before they are freed) unless
  // CAMELID_HIP_Q6K_GEMM2=0
  const char* g2 = std::getenv("CAMELID_HIP_Q6K_GEMM2");
  const bool planes = quant == CAMELID_Q6_K && tokens > (uint32_t)cm::Q6M_MAX && rows % 4 == 0 && ldy % 4 == 0 &&
                      !(g2 && std::atoi(g2) == 0);
  int8_t* xt = nullptr;
  if (planes) {
    if (hipMalloc(&m.w2, cm::q6g_planes_bytes((int)rows, (int)k)) != hipSuccess) {
      m.w2 = nullptr;
      return fail(nullptr, "kquant_gemm: weight plane allocation failed");
    }
    if (hipMalloc(&xt, cm::q6g_act_bytes((int)tokens, (int)k)) != hipSuccess) {
      (void)hipFree(m.w2);
      return fail(nullptr, "kquant_gemm: activation copy allocation failed");
    }
    hipLaunchKernelGGL(cm::k_q6k_w2, dim3((rows + cm::Q6G_R - 1) / cm::Q6G_R * cm::Q6G_R, k / 256), dim3(256), 0,
                       (hipStream_t)stream, m.a, m.b, m.sc, (int)rows, (int)k, m.w2);
  }
  launch_kgemm(m, tokens, yd, yq, y, ldy, resid, (hipStream_t)stream, xt);
  const int rc = launch_status("kquant_gemm");
  if (planes) {
    const bool synced = hipStreamSynchronize((hipStream_t)stream) == hipSuccess;
    (void)hipFree(m.w2);
    (void)hipFree(xt);
    if (!synced && !rc) return fail(nullptr, "kquant_gemm: stream synchronization failed");
  }
  return rc;
}

int camelid_hip_time_q8_0(int batched, const int8_t* const* wq, const uint16_t* const* wd, uint32_t copies,
                          uint32_t rows, uint32_t k, const int8_t* xq, const float* xs, uint32_t tokens, float* y,
                          uint32_t iters, float* ms_out) {
  if (!wq || !wd || !xq || !xs || !y || !ms_out || copies == 0 || iters == 0) return fail(nullptr, "null argument");
  if (k % 32 || k == 0 || rows == 0 || (batched && (tokens == 0 || rows % 4)))
    return fail(nullptr, "invalid shape");
  hipStream_t s = nullptr;
  if (hipStreamCreateWithFlags(&s, hipStreamNonBlocking) != hipSuccess) return fail(nullptr, "stream create failed");
  hipEvent_t a = nullptr, b = nullptr;
  int rc = 0;
  if (hipEventCreate(&a) != hipSuccess || hipEventCreate(&b) != hipSuccess) {
    rc = fail(nullptr, "event create failed");
  } else {
    std::vector<Q8Mat> mats(copies);
    for (uint32_t c = 0; c < copies && !rc; ++c) {
      mats[c].q = const_cast<int8_t*>(wq[c]);
      mats[c].d = const_cast<uint16_t*>(wd[c]);
      mats[c].rows = rows;
      mats[c].k = k;
      if (batched) rc = q8_scan_inf_scales(&mats[c], s);
    }
    auto launch = [&](uint32_t i) {
      const Q8Mat& m = mats[i % copies];
      if (batched)
        launch_gemm(m, tokens, xq, xs, y, nullptr, s);
      else
        launch_gemv(m, xq, xs, y, nullptr, s);
    };
    if (!rc) {
      for (uint32_t i = 0; i < std::min(copies, 4u); ++i) launch(i);  // warm-up
      (void)hipEventRecord(a, s);
      for (uint32_t i = 0; i < iters; ++i) launch(i);
      (void)hipEventRecord(b, s);
      if (hipEventSynchronize(b) != hipSuccess || hipEventElapsedTime(ms_out, a, b) != hipSuccess)
        rc = fail(nullptr, "timing failed");
      if (!rc && hipGetLastError() != hipSuccess) rc = fail(nullptr, "launch failed");
    }
  }
  if (a) (void)hipEventDestroy(a);
  if (b) (void)hipEventDestroy(b);
  (void)hipStreamDestroy(s);
  return rc;
}

int camelid_hip_time_kquant(uint8_t quant, const uint8_t* a, const uint8_t* b, const int8_t* sc, const uint16_t* d,
                            uint32_t rows, uint32_t k, uint32_t tokens, const float* yd, const int8_t* yq, float* y,
                            uint32_t iters, float* ms_out) {
  if (!a || !b || !yd || !yq || !y || !ms_out || iters == 0) return fail(nullptr, "null argument");
  if (quant != CAMELID_Q4_K && quant != CAMELID_Q6_K) return fail(nullptr, "quant must be Q4_K or Q6_K");
  if (quant == CAMELID_Q6_K && (!sc || !d)) return fail(nullptr, "null argument");
  if (rows == 0 || k == 0 || k % 256 || k > 16384 || tokens == 0) return fail(nullptr, "invalid shape");
  hipStream_t s = nullptr;
  if (hipStreamCreateWithFlags(&s, hipStreamNonBlocking) != hipSuccess) return fail(nullptr, "stream create failed");
  hipEvent_t ea = nullptr, eb = nullptr;
  KMat m;
  m.quant = quant;
  m.a = const_cast<uint8_t*>(a);
  m.b = const_cast<uint8_t*>(b);
  m.sc = const_cast<int8_t*>(sc);
  m.d = const_cast<uint16_t*>(d);
  m.rows = rows;
  m.k = k;
  int rc = 0;
  // the Q6_K weight planes are built once, outside the timed launches (as at model upload);
  // each timed launch includes the activations' class-major copy (as in a prefill chunk)
  const char* g2 = std::getenv("CAMELID_HIP_Q6K_GEMM2");
  int8_t* xt = nullptr;
  if (quant == CAMELID_Q6_K && tokens > (uint32_t)cm::Q6M_MAX && rows % 4 == 0 && !(g2 && std::atoi(g2) == 0)) {
    if (hipMalloc(&m.w2, cm::q6g_planes_bytes((int)rows, (int)k)) != hipSuccess) {
      m.w2 = nullptr;
      rc = fail(nullptr, "time_kquant: weight plane allocation failed");
    } else if (hipMalloc(&xt, cm::q6g_act_bytes((int)tokens, (int)k)) != hipSuccess) {
      xt = nullptr;
      rc = fail(nullptr, "time_kquant: activation copy allocation failed");
    } else {
      hipLaunchKernelGGL(cm::k_q6k_w2, dim3((rows + cm::Q6G_R - 1) / cm::Q6G_R * cm::Q6G_R, k / 256), dim3(256), 0,
                         s, m.a, m.b, m.sc, (int)rows, (int)k, m.w2);
    }
  }
  if (!rc && (hipEventCreate(&ea) != hipSuccess || hipEventCreate(&eb) != hipSuccess))
    rc = fail(nullptr, "event create failed");
  if (!rc) {
    launch_kgemm(m, tokens, yd, yq, y, rows, nullptr, s, xt);  // warm-up
    (void)hipEventRecord(ea, s);
    for (uint32_t i = 0; i < iters; ++i) launch_kgemm(m, tokens, yd, yq, y, rows, nullptr, s, xt);
    (void)hipEventRecord(eb, s);
    if (hipEventSynchronize(eb) != hipSuccess || hipEventElapsedTime(ms_out, ea, eb) != hipSuccess)
      rc = fail(nullptr, "timing failed");
    if (!rc && hipGetLastError() != hipSuccess) rc = fail(nullptr, "launch failed");
  }
  (void)hipStreamSynchronize(s);
  if (m.w2) (void)hipFree(m.w2);
  if (xt) (void)hipFree(xt);
  if (ea) (void)hipEventDestroy(ea);
  if (eb) (void)hipEventDestroy(eb);
  (void)hipStreamDestroy(s);
  return rc;
}

int camelid_hip_argmax(const float* x, uint32_t n, uint32_t* out, void* stream) {
  if (!x || !out) return fail(nullptr, "null argument");
  hipLaunchKernelGGL(cm::k_argmax, dim3(1), dim3(1024), 0, (hipStream_t)stream, x, (int)n, out);
  return launch_status("argmax");
}

int camelid_hip_inorder_sum_rows(const float* x, uint32_t rows, uint32_t n, uint32_t m_seq, uint32_t method,
                                 float* out, void* stream) {
  if (!x || !out) return fail(nullptr, "null argument");
  if (n == 0 || n > (uint32_t)cm::SEG_MAX_N || rows == 0) return fail(nullptr, "n must be in (0, 16384] and rows > 0");
  if (method > 1) return fail(nullptr, "method must be 0 (segmented passes) or 1 (one pass)");
  if (method == 1) {
    switch (cm::rms_chunk((int)n)) {
#define CM_SUM(C)                                                                                                  \
  case C:                                                                                                          \
    hipLaunchKernelGGL(cm::k_inorder_sum_rows_onepass<C>, dim3(rows), dim3(cm::RMS_NT), 0, (hipStream_t)stream, x, \
                       (int)n, out);                                                                               \
    break;
      CM_RMS_CHUNKS(CM_SUM)
#undef CM_SUM
    }
    return launch_status("inorder_sum_rows");
  }
  switch (cm::seg_chunk((int)n)) {
#define CM_SUM(C)                                                                                                \
  case C:                                                                                                        \
    hipLaunchKernelGGL(cm::k_inorder_sum_rows<C>, dim3(rows), dim3(256), 0, (hipStream_t)stream, x, (int)n,      \
                       (int)m_seq, out);                                                                         \
    break;
    CM_SEG_CHUNKS(CM_SUM)
#undef CM_SUM
  }
  return launch_status("inorder_sum_rows");
}

int camelid_hip_expf(const float* x, float* y, size_t n, void* stream) {
  if (!x || !y) return fail(nullptr, "null argument");
  if (n == 0) return 0;
  hipLaunchKernelGGL(cm::k_expf, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream, x, y, n);
  return launch_status("expf");
}

void camelid_expf_host(const float* x, float* y, size_t n) {
  for (size_t i = 0; i < n; ++i) y[i] = cm::glibc_expf(x[i]);
}

}  // extern "C"
