/* camelid_hip.h -- C ABI of the MI355X (gfx950) resident decode/prefill backend.
 *
 * Drop-in boundary for Camelid's CUDA resident engine: every engine entry point
 * mirrors one method of `CudaResidentDecode` (src/cuda_resident.rs) with the same
 * argument meaning.  Conventions (mirroring the reference):
 *   - every call returns 0 on success, nonzero on error; the message is available
 *     from camelid_hip_last_error(engine) (engine-owned string).  A caller treats
 *     any error as "decline -> CPU fallback" (inference.rs:3316-3371); after an
 *     error in prefill/forward the engine sets filled = 0 (inference.rs:2484);
 *   - inputs are borrowed for the call and copied to device memory; the engine owns
 *     every device buffer (cuda_resident.rs:5601-5762);
 *   - the engine is not internally synchronised: one caller at a time
 *     (inference.rs:10952 single-slot mutex);
 *   - one HIP stream, one host synchronisation per forward call
 *     (cuda_resident.rs:7475-7476).
 * Plain pointers and sizes only; no HIP or torch types cross this boundary.
 */
#ifndef CAMELID_HIP_H
#define CAMELID_HIP_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct camelid_hip_engine camelid_hip_engine;

/* Model dimensions: the arguments of CudaResidentDecode::new (cuda_resident.rs:5601). */
typedef struct camelid_hip_dims {
  uint32_t n_layers;
  uint32_t n_heads;
  uint32_t n_kv_heads;
  uint32_t head_dim;
  uint32_t hidden;
  uint32_t ffn_dim;
  uint32_t rope_dim;
  uint32_t max_pos;
  uint32_t vocab;
  float eps;
  uint32_t split_half_pairing; /* 0: adjacent pairs (llama), 1: split-half (qwen3) */
} camelid_hip_dims;

/* Weight formats: ProjQuant (cuda_resident.rs:5262). */
enum { CAMELID_Q8_0 = 0, CAMELID_Q4_K = 1, CAMELID_Q6_K = 2 };
/* Q8_0 byte layouts accepted by set_layer/set_output: 34 = GGUF wire block (f16 scale LE +
 * 32 i8); 36 = Camelid's in-memory Q8_0Block (f32 scale + 32 i8, inference.rs:19992). */
enum { CAMELID_Q8_WIRE34 = 34, CAMELID_Q8_BLOCK36 = 36 };
/* Projection order inside set_layer's arrays: q, k, v, o, gate, up, down. */
enum { CAMELID_PROJ_Q = 0, CAMELID_PROJ_K, CAMELID_PROJ_V, CAMELID_PROJ_O,
       CAMELID_PROJ_GATE, CAMELID_PROJ_UP, CAMELID_PROJ_DOWN, CAMELID_N_PROJ };

/* CudaResidentDecode::new (cuda_resident.rs:5601): allocates the f16 KV cache (per layer and
 * kv head, K in granules of 8 dims of one position, V in granules of 8 positions of one dim,
 * as camelid_hip_rope_kv documents; position stride kvs = max_pos rounded up to 8) and all
 * scratch on device 0 (or CAMELID_HIP_DEVICE).  head_dim must be 64, 128 or 256. */
int camelid_hip_engine_new(const camelid_hip_dims* dims, camelid_hip_engine** out);
/* Host-only preflight of build_resident_cuda_engine's decline (inference.rs:11245-11678 returns
 * None, and the caller runs the model on the CPU path, for a model the resident engine cannot
 * take): 0 when engine_new would accept `dims` and set_layer / set_output would accept a layer
 * whose projections have the formats layer_quant[7] (CAMELID_PROJ_* order; NULL: no layer
 * check) and an lm_head of format out_quant; nonzero otherwise, with the reason in
 * camelid_hip_last_error(NULL).  Makes no HIP call: the decode attention's LDS room is judged
 * with gfx950's 160 KB per workgroup and a bound on the kernels' static LDS, so a max_pos within
 * a few hundred positions of the device's own limit may be declined here and still be taken
 * by engine_new. */
int camelid_hip_check_model(const camelid_hip_dims* dims, const uint8_t layer_quant[7], uint8_t out_quant);
/* Drop (cuda_resident.rs:5398 Drop + cuda.rs:485 release_async_pool). */
void camelid_hip_engine_free(camelid_hip_engine* e);
/* Last error message of this engine ("" if none); NULL engine -> last global error. */
const char* camelid_hip_last_error(const camelid_hip_engine* e);

/* CudaResidentDecode::set_layer_located (cuda_resident.rs:5801). w[i]/len[i]: projection
 * bytes in CAMELID_PROJ_* order; quant[i]: CAMELID_Q8_0, CAMELID_Q4_K or CAMELID_Q6_K (K-quants
 * as GGUF wire superblocks); q8_layout: 34 or 36 (Q8_0 projections).  q_norm/k_norm may be
 * NULL (no QK-norm). */
int camelid_hip_set_layer(camelid_hip_engine* e, uint32_t layer, const uint8_t* const w[7],
                          const size_t len[7], const uint8_t quant[7], uint8_t q8_layout,
                          const float* attn_norm, const float* ffn_norm, const float* q_norm,
                          const float* k_norm);
/* CudaResidentDecode::set_output (cuda_resident.rs:6008): final norm [H] + lm_head [V][H]. */
int camelid_hip_set_output(camelid_hip_engine* e, const float* final_norm, const uint8_t* w,
                           size_t len, uint8_t quant, uint8_t q8_layout);
/* weights_ready (cuda_resident.rs:6261): 1 when every layer and the output are set. */
int camelid_hip_weights_ready(const camelid_hip_engine* e);
/* filled / set_filled (cuda_resident.rs:6265-6271): positions of valid KV. */
uint32_t camelid_hip_filled(const camelid_hip_engine* e);
int camelid_hip_set_filled(camelid_hip_engine* e, uint32_t filled);
/* max_pos / n_layers / uses_kquant (cuda_resident.rs:6285, :6292, :6220). */
uint32_t camelid_hip_max_pos(const camelid_hip_engine* e);
uint32_t camelid_hip_n_layers(const camelid_hip_engine* e);
int camelid_hip_uses_kquant(const camelid_hip_engine* e);

/* seed_layer (cuda_resident.rs:6305): upload CPU KV history of one layer, f32 values laid
 * out [kv_head][pos][hd] for positions [0, n_pos) (rounded to f16 on upload). */
int camelid_hip_seed_layer(camelid_hip_engine* e, uint32_t layer, const float* ck, const float* cv,
                           uint32_t n_pos);
/* read_kv_layer (cuda_resident.rs:6348): download positions [0, n) of one layer as f32,
 * [kv_head][pos][hd]. */
int camelid_hip_read_kv_layer(camelid_hip_engine* e, uint32_t layer, uint32_t n, float* ck,
                              float* cv);

/* forward_token (cuda_resident.rs:7430) / forward_token_logits (:7724): one decode step at
 * `position` from the embedding row emb[H] with that position's RoPE tables cos/sin
 * [rope_dim/2].  `scale` is the attention score scale (1/sqrt(hd)).  want_logits != 0
 * copies the logits row to logits_out [vocab].  *tok_out receives the greedy token. */
int camelid_hip_forward_token(camelid_hip_engine* e, const float* emb, const float* cos_tab,
                              const float* sin_tab, uint32_t position, float scale,
                              int want_logits, uint32_t* tok_out, float* logits_out);
/* prefill / prefill_batched (cuda_resident.rs:7785, :8797): positions
 * [filled, filled + n) from embs [n][H], cos_all/sin_all [n][rope_dim/2]. */
int camelid_hip_prefill(camelid_hip_engine* e, const float* embs, const float* cos_all,
                        const float* sin_all, uint32_t n, float scale);
/* verify_batch (cuda_resident.rs:7821; MAX_VERIFY_K :5524; seam inference.rs:2752-2876):
 * the k tokens of embs [k][H] at positions [base_position, base_position + k) in one batched
 * forward (their K/V are written), tokens_out[k] = the greedy token after each, bit-identical
 * to k single-token steps.  1 <= k <= CAMELID_MAX_VERIFY_K; base_position <= filled.
 * filled is not changed: the caller sets it to base_position + the accepted length
 * (inference.rs:2873). */
#define CAMELID_MAX_VERIFY_K 8
int camelid_hip_verify(camelid_hip_engine* e, const float* embs, const float* cos_all, const float* sin_all,
                       uint32_t base_position, uint32_t k, float scale, uint32_t* tokens_out);

/* Device-side token loop (forward_token_device, cuda_resident.rs:7529; embed_gather_q8_0
 * :2995; rope_select :3012).  set_embedding uploads token_embd (Q8_0); set_rope_table
 * uploads cos/sin for positions [0, n_pos).  generate runs n_steps greedy steps starting
 * with `token` at `position`, feeding each argmax back on the device; tokens_out[n_steps]. */
int camelid_hip_set_embedding(camelid_hip_engine* e, const uint8_t* w, size_t len, uint8_t quant,
                              uint8_t q8_layout);
int camelid_hip_set_rope_table(camelid_hip_engine* e, const float* cos_all, const float* sin_all,
                               uint32_t n_pos);
int camelid_hip_generate(camelid_hip_engine* e, uint32_t token, uint32_t position, uint32_t n_steps,
                         float scale, uint32_t* tokens_out);

/* Test hooks.  capture_hidden: 1 enables recording the residual stream entering each layer
 * and after the last ([L+1][H] f32) on every forward; read_hidden copies the last one. */
int camelid_hip_capture_hidden(camelid_hip_engine* e, int enable);
int camelid_hip_read_hidden(camelid_hip_engine* e, float* out);
/* Per-launch HIP-event timing on the engine's stream (measurement hook).  Between begin and
 * end every kernel launch is bracketed by events (the device-side loop then runs without
 * its graph); end synchronises and returns, per category (0 Q8_0 GEMV incl. the lm_head +
 * argmax launch, 1 RMSNorm+quantize, 2 attention incl. QK-norm/RoPE/KV store, 3 SwiGLU +
 * quantize, 4 argmax finish, 5 embedding gather, 6 the prefill projections: matrix-core GEMMs
 * and multi-token GEMVs, whose "bytes" are int8 operations, 2 per weight and token), the
 * summed kernel milliseconds, algorithmic bytes and launch count. */
int camelid_hip_profile_begin(camelid_hip_engine* e);
int camelid_hip_profile_end(camelid_hip_engine* e, double* ms, double* bytes, uint64_t* launches,
                            uint32_t n_cat);
/* Measurement hook (no reference counterpart): in-kernel phase timestamps (100 MHz counter) of
 * the last decode step, recorded only by the measurement build of this library
 * (libcamelid_hip_stamps.so, compiled with -DCM_STAMPS); the product build returns an error.
 * Layout: the decode attention [layer < 64][head < 64][9] (start, q/k/v built, scores,
 * exponentials, denominator, output sums, end, a row wave's K-row loads issued, its scores
 * done), then the norm-fused GEMVs of the last layer [kind 0 qkv, 1 gate/up][workgroup <
 * 256][13] (start, norm done, a weight wave's loads issued, past the post-norm barrier, block
 * dots done, end, the norm inputs arrived, the sum of squares known, the one-pass sum's four
 * phases, its special-step count), then the split attention of the last layer [kind 0 scores,
 * 1 output][workgroup < 1024][8] (scores: start, q built, scores done, end; output: start,
 * scores and maximum, exponentials, denominator, output sums, end), then the output-projection
 * workgroups of the attention launch [layer < 64][first, last workgroup][4] (start, watched
 * word tagged, activation staged, end).  Copies min(n, 64*64*9 + 2*256*13 + 2*1024*8 + 64*2*4)
 * words; *n_out receives the count. */
int camelid_hip_phase_stamps(uint64_t* out, size_t n, size_t* n_out);
/* Measurement hook (no reference counterpart): HBM bandwidth of this device, best of `reps`
 * passes over three device arrays of bytes_per_array each (a multiple of 128 KiB; allocated
 * and freed here): STREAM's triad a = b + 3c (3 x bytes_per_array moved per pass) and a
 * read-only pass over b, both with nontemporal loads and stores.  GB/s = 1e9 bytes per second. */
int camelid_hip_hbm_bandwidth(size_t bytes_per_array, uint32_t reps, double* triad_gbs, double* read_gbs);
/* Device name and compute units. */
int camelid_hip_device_info(char* name, size_t name_len, int* n_cu);

/* ---------------------------------------------------------------------------------------
 * Kernel-level entry points (device pointers; `stream` is a hipStream_t or NULL for the
 * default stream).  They are the units the engine composes; exported for parity tests and
 * the isolated kernel sweep.  Weight matrices use the "Q8R" split layout produced by
 * camelid_q8_0_repack: int8 quants [rows][K] + f16 scale bits [rows][K/32].
 * Global errors are read with camelid_hip_last_error(NULL). */
int camelid_hip_malloc(void** ptr, size_t bytes);
int camelid_hip_free(void* ptr);
int camelid_hip_memcpy_htod(void* dst, const void* src, size_t bytes);
int camelid_hip_memcpy_dtoh(void* dst, const void* src, size_t bytes);
int camelid_hip_synchronize(void);

/* Host repack of a Q8_0 matrix [rows][k] from 34- or 36-byte blocks into Q8R. */
int camelid_q8_0_repack(const uint8_t* src, size_t rows, size_t k, uint8_t layout,
                        int8_t* quants_out, uint16_t* scales_out);
/* q8_gemv (cuda_resident.rs:230; CPU inference.rs:19871-19905): y = resid + W.x, faithful
 * block-ordered fold.  resid may be NULL; y may alias resid. */
int camelid_hip_q8_0_gemv(const int8_t* wq, const uint16_t* wd, uint32_t rows, uint32_t k,
                          const int8_t* xq, const float* xs, float* y, const float* resid,
                          void* stream);
/* Per-(row, block) int32 dots [rows][k/32] through the GEMV's dot path (test hook for the
 * bit-exact block-dot contract, CPU inference.rs:20539-20566). */
int camelid_hip_q8_0_block_dots(const int8_t* wq, uint32_t rows, uint32_t k, const int8_t* xq, int32_t* out,
                                void* stream);
/* rms_norm_quantize followed by q8_gemv (cuda_resident.rs:177 + :230; CPU tensor/mod.rs:2083-2106,
 * inference.rs:16953, 19871-19905), with the norm computed inside the GEMV: y = W.Q8_0(rmsnorm(x; nw)),
 * bit-identical to camelid_hip_rmsnorm_quantize + camelid_hip_q8_0_gemv (the decode step's qkv
 * projection).  k (the hidden width) in {2048, 3072, 4096}. */
int camelid_hip_rmsnorm_q8_0_gemv(const int8_t* wq, const uint16_t* wd, uint32_t rows, uint32_t k, const float* x,
                                  const float* nw, float eps, float* y, void* stream);
/* Gate/up projection + SwiGLU + Q8_0 quantization of the activation (CPU tensor/mod.rs:1943-1967,
 * inference.rs:16953): W holds gate and up rows interleaved in groups of 32 (group g: gate rows
 * 32g..32g+31, then up rows 32g..32g+31; ffn groups), aq/as = Q8_0(silu(gate.x) * up.x).  The
 * activation is Q8_0(rmsnorm(x; nw)) computed in-kernel when x is given,
 * else xq/xs.  k in {2048, 3072, 4096}; ffn % 32 == 0. */
int camelid_hip_gate_up_silu(const int8_t* wq, const uint16_t* wd, uint32_t ffn, uint32_t k, const int8_t* xq,
                             const float* xs, const float* x, const float* nw, float eps, int8_t* aq, float* as,
                             void* stream);
/* rms_norm_quantize (cuda_resident.rs:177; CPU tensor/mod.rs:2083-2106 + inference.rs:16953).
 * n % 32 == 0, n <= 16384; x, w, xq and y (when given) 16-byte aligned. */
int camelid_hip_rmsnorm_quantize(const float* x, const float* w, uint32_t n, float eps, int8_t* xq,
                                 float* xs, float* y, void* stream);
/* quantize_q8_0 (cuda_resident.rs:151; CPU inference.rs:16953-16971). */
int camelid_hip_quantize_q8_0(const float* x, uint32_t n, int8_t* xq, float* xs, void* stream);
/* silu_mul_quantize (cuda_resident.rs:1315; CPU tensor/mod.rs:1943-1967). gu = [gate|up]. */
int camelid_hip_silu_mul_quantize(const float* gu, uint32_t n, int8_t* xq, float* xs, float* act,
                                  void* stream);
/* rope_rotate + kv_scatter (cuda_resident.rs:1545, :1569; CPU rope.rs:489-524,
 * kv_cache.rs:573-600), with optional per-head QK RMSNorm (cuda_resident.rs:122).  Cache
 * layout: per (layer, kv head) a region of hd * max_pos f16 elements at element offset
 * (layer * n_kv + kv_head) * hd * max_pos; K element (p, d) at ((d / 8) * max_pos + p) * 8
 * + d % 8; V element (p, d) at ((p / 8) * hd + d) * 8 + p % 8 (16-byte granules: 8 dims of
 * one position for K, 8 positions of one dim for V).  max_pos (the position stride) % 8 == 0.
 * Position contract (the engine's filled/max_pos, cuda_resident.rs:6265-6292): *d_pos is read
 * on the host and refused unless *d_pos < max_pos; the kernel also skips every cache access
 * for a position outside the cache and the call then returns an error.  Synchronizes the
 * stream. */
int camelid_hip_rope_kv(const float* qkv, uint32_t n_heads, uint32_t n_kv, uint32_t hd,
                        uint32_t rope_dim, uint32_t split_half, const float* cos_tab,
                        const float* sin_tab, const float* q_norm, const float* k_norm, float eps,
                        float* qrot, uint16_t* kc, uint16_t* vc, uint32_t layer, uint32_t max_pos,
                        const uint32_t* d_pos, void* stream);
/* attention_decode (cuda_resident.rs:1587; CPU inference.rs:23945-24025), faithful order.
 * Cache layout and position contract as camelid_hip_rope_kv (synchronizes the stream);
 * max_pos (the position stride) % 8 == 0; hd in {64,128,256}. */
int camelid_hip_attention_decode(const float* qrot, const uint16_t* kc, const uint16_t* vc,
                                 uint32_t layer, uint32_t n_heads, uint32_t n_kv, uint32_t hd,
                                 uint32_t max_pos, const uint32_t* d_pos, float scale,
                                 float* att_out, int8_t* xq, float* xs, void* stream);
/* The same attention split over workgroups for long contexts (the engine's path from
 * CAMELID_HIP_ATT_SPLIT positions on, default 2048): scores by slices of positions, softmax and
 * output sum by 32-dim slices; bit-identical to camelid_hip_attention_decode.  Allocates its
 * score scratch and synchronizes the stream (test entry point). */
int camelid_hip_attention_decode_split(const float* qrot, const uint16_t* kc, const uint16_t* vc,
                                       uint32_t layer, uint32_t n_heads, uint32_t n_kv, uint32_t hd,
                                       uint32_t max_pos, const uint32_t* d_pos, float scale,
                                       float* att_out, int8_t* xq, float* xs, void* stream);
/* No counterpart in the reference: camelid_hip_attention_decode_split for callers that cannot
 * allocate (tight serving loops, harnesses that forbid hipMalloc).  It is not for code under
 * stream capture: like the allocating entry it reads the position back to the host and
 * synchronizes the stream.  The same kernels and bits as camelid_hip_attention_decode_split, but the score
 * scratch is a static device array of the library (4 MiB + 64 KiB per GPU, held until the
 * process ends) instead of a per-call allocation; no hipMalloc or hipFree is called.  Limit:
 * n_heads * max_pos <= 2^20 and n_heads * ceil(max_pos / 256) <= 2^14, else an error.  Every
 * call on one GPU shares that GPU's scratch (it keeps no state between calls: each word read
 * is written earlier in the same call), so calls that overlap on one GPU (other streams or
 * threads) race.  Position contract as camelid_hip_rope_kv; synchronizes the stream. */
int camelid_hip_attention_decode_split_noalloc(const float* qrot, const uint16_t* kc, const uint16_t* vc,
                                               uint32_t layer, uint32_t n_heads, uint32_t n_kv, uint32_t hd,
                                               uint32_t max_pos, const uint32_t* d_pos, float scale,
                                               float* att_out, int8_t* xq, float* xs, void* stream);
/* q8_gemm_batched (cuda_resident.rs:1494; CPU: the row dot of inference.rs:19871-19905 for
 * each token): y[t][n] = resid[t][n] + W[n].X[t] for T = tokens activation rows X [tokens][k]
 * (Q8_0 quants, f32 block scales [tokens][k/32]); output [tokens][rows]; the same
 * block-ordered fold as the GEMV.  rows % 4 == 0; resid may be NULL; y may alias resid. */
int camelid_hip_q8_0_gemm(const int8_t* wq, const uint16_t* wd, uint32_t rows, uint32_t k,
                          const int8_t* xq, const float* xs, uint32_t tokens, float* y,
                          const float* resid, void* stream);
/* attention_batched (cuda_resident.rs:1994; CPU inference.rs:23945-24025 per token): causal
 * attention of `tokens` query rows qrot [tokens][n_heads*hd], row t at position pos0 + t,
 * over the cache positions [0, pos0 + t] (already stored).  Cache layout as
 * camelid_hip_rope_kv.  Outputs [tokens][n_heads*hd] (att_out may be NULL) and their Q8_0
 * quantization.  pos0 + tokens <= max_pos, <= 16384. */
int camelid_hip_attention_prefill(const float* qrot, const uint16_t* kc, const uint16_t* vc,
                                  uint32_t layer, uint32_t n_heads, uint32_t n_kv, uint32_t hd,
                                  uint32_t max_pos, uint32_t pos0, uint32_t tokens, float scale,
                                  float* att_out, int8_t* xq, float* xs, void* stream);
/* quantize_q8k (cuda_resident.rs:1416-1490; CPU inference.rs:17564-17599): n (multiple of 256)
 * f32 values -> Q8_K blocks: scales yd [n/256], quants yq [n], per-32 quant sums ybs [n/32]. */
int camelid_hip_quantize_q8_k(const float* x, uint32_t n, float* yd, int8_t* yq, int32_t* ybs,
                              void* stream);
/* rms_norm + quantize_q8k (CPU tensor/mod.rs:2083-2106 then inference.rs:17564-17599): the
 * RMSNorm kernel writing the Q8_K activation of a K-quant projection.  n % 256 == 0,
 * n <= 16384; x, w 16-byte aligned.  (Test hook; allocates its own Q8_0 scratch.) */
int camelid_hip_rmsnorm_q8_k(const float* x, const float* w, uint32_t n, float eps, float* yd,
                             int8_t* yq, int32_t* ybs, void* stream);
/* silu_mul + quantize_q8k (CPU tensor/mod.rs:1943-1967 then inference.rs:17564-17599), gu =
 * [gate|up], n % 256 == 0.  (Test hook; asynchronous on stream, allocates nothing.) */
int camelid_hip_silu_mul_q8_k(const float* gu, uint32_t n, float* yd, int8_t* yq, int32_t* ybs,
                              void* stream);
/* Host split of K-quant wire rows [rows][k/256 superblocks] into the device planes the
 * K-quant GEMV reads: Q4_K (quant 1): a = nibbles [rows][k/2], b = superblock headers
 * [rows][k/256][16] (sc, d unused); Q6_K (quant 2): a = ql [rows][k/2], b = qh [rows][k/4],
 * sc = scales [rows][k/256][16], d = f16 scales [rows][k/256]. */
int camelid_kquant_repack(uint8_t quant, const uint8_t* src, size_t rows, size_t k, uint8_t* a,
                          uint8_t* b, int8_t* sc, uint16_t* d);
/* q4k_gemv / q6k_gemv (cuda_resident.rs:601, :925; CPU q4_k_dot_arm refmath.rs:424-561 via
 * inference.rs:17906-17965, q6_k_wire_row_dot inference.rs:19240-19295 via :19148-19195):
 * y = resid + W.x for a Q8_K activation (camelid_hip_quantize_q8_k) and planes from
 * camelid_kquant_repack; faithful per-row order.  k % 256 == 0, k <= 16384; resid may be
 * NULL; y may alias resid. */
int camelid_hip_kquant_gemv(uint8_t quant, const uint8_t* a, const uint8_t* b, const int8_t* sc,
                            const uint16_t* d, uint32_t rows, uint32_t k, const float* yd,
                            const int8_t* yq, const int32_t* ybs, float* y, const float* resid,
                            void* stream);
/* K-quant projection over `tokens` Q8_K activation rows (yd [tokens][k/256], yq [tokens][k]):
 * y[t * ldy + r] = resid[t * ldy + r] + W[r].x[t], each (token, row) bit-identical to
 * camelid_hip_kquant_gemv on that token.  Replaces the reference's per-token K-quant prefill
 * loop (inference.rs:2462-2473; the reference has no K-quant GEMM), on the int8 matrix cores.
 * Q6_K over more than 8 tokens with rows % 4 == 0 and ldy % 4 == 0 builds the matrix's
 * class-major weight planes and a class-major copy of yq for the call (temporary device
 * allocations, freed after the stream is synchronized; the engine builds the planes once at
 * upload).  k % 256 == 0,
 * k <= 16384, ldy >= rows, tokens * k < 2^31, rows * k < 2^32; resid may be NULL; y may
 * alias resid. */
int camelid_hip_kquant_gemm(uint8_t quant, const uint8_t* a, const uint8_t* b, const int8_t* sc,
                            const uint16_t* d, uint32_t rows, uint32_t k, uint32_t tokens,
                            const float* yd, const int8_t* yq, float* y, uint32_t ldy,
                            const float* resid, void* stream);
/* Measurement hook (no reference counterpart; the kernel sweep of the benchmark): `iters`
 * launches of the Q8_0 GEMV (batched = 0) or of the prefill GEMM over `tokens` activation
 * rows (batched = 1), rotating over `copies` weight matrices, timed with HIP events on a
 * stream of its own; *ms_out = total milliseconds. */
int camelid_hip_time_q8_0(int batched, const int8_t* const* wq, const uint16_t* const* wd,
                          uint32_t copies, uint32_t rows, uint32_t k, const int8_t* xq,
                          const float* xs, uint32_t tokens, float* y, uint32_t iters,
                          float* ms_out);
/* Measurement hook (no reference counterpart; the kernel sweep of the benchmark): `iters`
 * launches of the K-quant prefill GEMM over `tokens` Q8_K activation rows (ldy = rows), timed
 * with HIP events on a stream of its own; Q6_K's weight planes are built once before the
 * timed launches, each of which includes the activations' class-major copy; *ms_out = total
 * milliseconds. */
int camelid_hip_time_kquant(uint8_t quant, const uint8_t* a, const uint8_t* b, const int8_t* sc,
                            const uint16_t* d, uint32_t rows, uint32_t k, uint32_t tokens,
                            const float* yd, const int8_t* yq, float* y, uint32_t iters,
                            float* ms_out);
/* argmax_f32 (cuda_resident.rs:1847; CPU inference.rs:5912). */
int camelid_hip_argmax(const float* x, uint32_t n, uint32_t* out, void* stream);
/* Sequential-order f32 sums of rows [rows][n] (n <= 16384), evaluated by a workgroup-parallel
 * exact method (test hook; CPU order: the Σx² fold of tensor/mod.rs:2083-2106).  method 0:
 * segmented passes (the long-context softmax denominator), m_seq leading terms folded
 * sequentially; method 1: the one-pass binade-prediction method the RMSNorm uses (m_seq
 * unused). */
int camelid_hip_inorder_sum_rows(const float* x, uint32_t rows, uint32_t n, uint32_t m_seq, uint32_t method,
                                 float* out, void* stream);
/* glibc-identical expf on the device (test hook for the softmax/SiLU exponential). */
int camelid_hip_expf(const float* x, float* y, size_t n, void* stream);
/* The same expf restatement evaluated on the host (test hook). */
void camelid_expf_host(const float* x, float* y, size_t n);

#ifdef __cplusplus
}
#endif
#endif /* CAMELID_HIP_H */
