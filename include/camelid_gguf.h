/* camelid_gguf.h -- C ABI of the host side around the resident engine: GGUF model files
 * mapped read-only (src/wire_mmap.rs, src/gguf/reader.rs), the loader that uploads a mapped
 * model into the engine, and the seam's host helpers (RoPE tables, embedding rows).
 *
 * Conventions: 0 on success, nonzero on error; camelid_gguf_last_error() gives the message
 * of the calling thread's last GGUF error.  Tensor data pointers point into the mapping and
 * stay valid until camelid_gguf_close.
 */
#ifndef CAMELID_GGUF_H
#define CAMELID_GGUF_H
#include <stddef.h>
#include <stdint.h>

#include "camelid_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct camelid_gguf camelid_gguf;

/* One tensor of the directory (GgufTensorDescriptor, src/gguf/reader.rs:455-462 plus the
 * mapped range of WireMmapTensor, src/wire_mmap.rs:397-422).  dims[0] is the contiguous
 * dimension (for a weight: the input width k; dims[1] = output rows); unused dims are 1.
 * type: GGML type id (0 F32, 8 Q8_0, 12 Q4_K, 14 Q6_K, ...). */
typedef struct camelid_gguf_tensor {
  const uint8_t* data;
  uint64_t n_bytes;
  uint64_t offset; /* absolute file offset of the data */
  uint64_t dims[4];
  uint32_t n_dims;
  int32_t type;
} camelid_gguf_tensor;

/* RoPE parameters of a model (ModelConfig rope fields, src/model.rs:164-186), in the
 * argument form of camelid_rope_tables.  freqs: the F32 rope_freqs.weight tensor [rope_dim/2]
 * inside the mapping, or NULL. */
typedef struct camelid_gguf_rope {
  float freq_base;
  int32_t scaling_kind; /* 0 none, 1 linear, 2 llama3 */
  float factor, orig_ctx, low, high;
  const float* freqs;
} camelid_gguf_rope;

/* GgufWireMmap::map (src/wire_mmap.rs:78) + read_metadata_with_len (src/gguf/reader.rs:346):
 * maps the whole file read-only (MAP_SHARED) and validates header, metadata and tensor
 * directory with the reference's rules (v2/v3, alignment, contiguous offsets, ranges). */
int camelid_gguf_open(const char* path, camelid_gguf** out);
/* Drop of GgufWireMmap (src/wire_mmap.rs:66): unmaps. */
void camelid_gguf_close(camelid_gguf* g);
const char* camelid_gguf_last_error(void);
/* GgufFile fields version / alignment / tensors.len() (src/gguf/reader.rs:148-158). */
uint32_t camelid_gguf_version(const camelid_gguf* g);
uint64_t camelid_gguf_alignment(const camelid_gguf* g);
uint64_t camelid_gguf_tensor_count(const camelid_gguf* g);
/* Name of tensor i in file order, NULL past the end. */
const char* camelid_gguf_tensor_name(const camelid_gguf* g, uint64_t i);
/* Tensor lookup by name (wire_mmap_tensors, src/wire_mmap.rs:426); 1 when absent. */
int camelid_gguf_find(const camelid_gguf* g, const char* name, camelid_gguf_tensor* out);
/* metadata_u32 / metadata_f32 / metadata_string (src/gguf/reader.rs:168-196): u32 also
 * accepts a u64 that fits, f32 also an f64; the string is owned by g (NULL if absent). */
int camelid_gguf_meta_u32(const camelid_gguf* g, const char* key, uint32_t* out);
int camelid_gguf_meta_f32(const camelid_gguf* g, const char* key, float* out);
const char* camelid_gguf_meta_str(const camelid_gguf* g, const char* key);
/* ModelConfig::from_gguf (src/model.rs:137-230) for the dense architectures of the resident
 * path (llama, mistral, qwen2, qwen3): engine dimensions for a KV cache of max_pos positions
 * (split-half RoPE pairing for qwen, src/model.rs:690) and the RoPE parameters. */
int camelid_gguf_model(const camelid_gguf* g, uint32_t max_pos, camelid_hip_dims* dims,
                       camelid_gguf_rope* rope);
/* The seam's upload of a model into the resident engine (build_resident_cuda_engine,
 * src/inference.rs:11245): set_layer for every layer, set_output (output.weight, or
 * token_embd.weight when tied) and, if with_embedding, set_embedding -- every tensor read
 * straight from the mapping (Q8_0 as 34-byte wire blocks, Q4_K / Q6_K as wire superblocks). */
int camelid_hip_load_gguf(camelid_hip_engine* e, const camelid_gguf* g, int with_embedding);

/* Seam host helpers.
 * resident_decode_rope_tables / resident_prefill_rope_tables (src/rope.rs:568-685): cos/sin
 * [n_pos][rope_dim/2] for positions pos0 .. pos0+n_pos-1; 1 on invalid parameters. */
int camelid_rope_tables(uint32_t rope_dim, float freq_base, int scaling_kind, float factor,
                        float orig_ctx, float low, float high, const float* rope_freqs,
                        uint32_t pos0, uint32_t n_pos, float* cos_out, float* sin_out);
/* Embedding rows of n tokens from a Q8_0 (34-byte wire) or K-quant token table
 * (src/tensor/mod.rs:2329-2398, :4682-4703, :4818-4845); 1 on a token out of range. */
int camelid_embed_q8_0(const uint8_t* wire, uint32_t vocab, uint32_t hidden, const uint32_t* tokens,
                       uint32_t n, float* out);
int camelid_embed_kquant(int quant, const uint8_t* wire, uint32_t vocab, uint32_t hidden,
                         const uint32_t* tokens, uint32_t n, float* out);

#ifdef __cplusplus
}
#endif
#endif
