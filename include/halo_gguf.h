/* GGUF checkpoints: a bounds-checked, zero-copy reader and the load of Q8_0 weights into the device layout.
 *
 * Replaces the reference's halo::core::GgufReader (src/core/gguf.hpp:146-245, src/core/gguf.cpp) for the loading
 * path and FlashNextGpu::Upload / RepackQ8 (src/engine/flash_next_gpu.cpp:90-123, 414-432). The reader maps the
 * file (or takes a caller's buffer), validates every header field against the file size (untrusted bytes: counts,
 * string lengths, array lengths, tensor extents and alignment), and indexes metadata and tensors by name; tensor
 * data stays in the mapping. Files split as <name>-00001-of-0000N.gguf open as one model when the first shard is
 * given. Functions return 0 / -1 with a message in err (halo_rt.h convention) unless stated. */
#ifndef HALO_GGUF_H_
#define HALO_GGUF_H_

#include <stddef.h>
#include <stdint.h>

#include "halo_model.h"
#include "halo_ops.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct halo_gguf halo_gguf;

/* GGML storage types (the values of the format; GgmlType, src/core/gguf.hpp:19-40). */
enum {
  HALO_GGML_F32 = 0, HALO_GGML_F16 = 1, HALO_GGML_Q4_0 = 2, HALO_GGML_Q4_1 = 3, HALO_GGML_Q5_0 = 6,
  HALO_GGML_Q5_1 = 7, HALO_GGML_Q8_0 = 8, HALO_GGML_Q8_1 = 9, HALO_GGML_Q2_K = 10, HALO_GGML_Q3_K = 11,
  HALO_GGML_Q4_K = 12, HALO_GGML_Q5_K = 13, HALO_GGML_Q6_K = 14, HALO_GGML_Q8_K = 15, HALO_GGML_IQ2_XXS = 16,
  HALO_GGML_IQ4_NL = 20, HALO_GGML_IQ3_S = 21, HALO_GGML_IQ4_XS = 23, HALO_GGML_I32 = 26, HALO_GGML_BF16 = 30
};
/* GGUF metadata value types (GgufValueType, src/core/gguf.hpp:94-108). */
enum {
  HALO_GGUF_U8 = 0, HALO_GGUF_I8 = 1, HALO_GGUF_U16 = 2, HALO_GGUF_I16 = 3, HALO_GGUF_U32 = 4, HALO_GGUF_I32 = 5,
  HALO_GGUF_F32 = 6, HALO_GGUF_BOOL = 7, HALO_GGUF_STRING = 8, HALO_GGUF_ARRAY = 9, HALO_GGUF_U64 = 10,
  HALO_GGUF_I64 = 11, HALO_GGUF_F64 = 12
};

/* One tensor (GgufTensorInfo, src/core/gguf.hpp:118-140): dims[0] is the fastest-varying extent. */
typedef struct halo_gguf_tensor {
  const char* name; /* not NUL-terminated: name_len bytes */
  size_t name_len;
  uint32_t type, n_dims;
  uint64_t dims[8];
  uint64_t offset; /* from the start of the data section */
  const void* data;
  uint64_t size_bytes;
} halo_gguf_tensor;

/* GgufReader::OpenFile / OpenMemory (src/core/gguf.cpp:170-356). The memory variant borrows `data` (it must outlive
 * the reader). */
int halo_gguf_open_file(const char* path, halo_gguf** out, char* err, size_t errlen);
int halo_gguf_open_memory(const void* data, size_t size, halo_gguf** out, char* err, size_t errlen);
void halo_gguf_close(halo_gguf* g);

uint32_t halo_gguf_version(const halo_gguf* g);
uint64_t halo_gguf_alignment(const halo_gguf* g);
uint64_t halo_gguf_tensor_count(const halo_gguf* g);
uint64_t halo_gguf_metadata_count(const halo_gguf* g);
/* Tensor i in file order (shard order for split files); FindTensor by name. Return 0, or -1 when absent. */
int halo_gguf_tensor_at(const halo_gguf* g, uint64_t i, halo_gguf_tensor* out);
int halo_gguf_find_tensor(const halo_gguf* g, const char* name, halo_gguf_tensor* out);

/* Metadata (GetMetadata*, src/core/gguf.cpp:763-850): the value type of a key or -1; typed getters return 0 when
 * the key holds a value of a compatible kind in range (unsigned / signed integers for the integer getters, f32 / f64
 * for the float getter), -1 otherwise. Strings are not NUL-terminated. Arrays: element type, length, and element i
 * of integer, float and string arrays. */
int halo_gguf_metadata_type(const halo_gguf* g, const char* key);
/* Key i of the metadata (0 <= i < halo_gguf_metadata_count; an unspecified but fixed order). */
int halo_gguf_metadata_key_at(const halo_gguf* g, uint64_t i, const char** key, size_t* len);
int halo_gguf_get_u32(const halo_gguf* g, const char* key, uint32_t* out);
int halo_gguf_get_u64(const halo_gguf* g, const char* key, uint64_t* out);
int halo_gguf_get_f32(const halo_gguf* g, const char* key, float* out);
int halo_gguf_get_bool(const halo_gguf* g, const char* key, int* out);
int halo_gguf_get_i64(const halo_gguf* g, const char* key, int64_t* out); /* signed integer scalars */
int halo_gguf_get_f64(const halo_gguf* g, const char* key, double* out);  /* f32 / f64 scalars */
int halo_gguf_get_string(const halo_gguf* g, const char* key, const char** data, size_t* len);
int halo_gguf_get_array_info(const halo_gguf* g, const char* key, uint32_t* elem_type, uint64_t* length);
int halo_gguf_get_array_u64(const halo_gguf* g, const char* key, uint64_t i, uint64_t* out);
int halo_gguf_get_array_i64(const halo_gguf* g, const char* key, uint64_t i, int64_t* out);
int halo_gguf_get_array_f64(const halo_gguf* g, const char* key, uint64_t i, double* out);
int halo_gguf_get_array_string(const halo_gguf* g, const char* key, uint64_t i, const char** data, size_t* len);
/* GetQuantizationLabel (src/core/gguf.cpp:868-898): the storage type holding the most elements, " mixed" appended
 * below four fifths of all elements, "unknown" without tensors. Writes a NUL-terminated label; returns its length. */
size_t halo_gguf_quantization_label(const halo_gguf* g, char* out, size_t len);
/* Encoded bytes of `elements` values of a storage type (quant::EncodedSizeBytes, src/core/quant.cpp:160-258);
 * 0 for an unknown type, a count that is not a whole number of blocks, or an overflow. */
uint64_t halo_ggml_encoded_bytes(uint32_t type, uint64_t elements);

/* Q8_0 load (FlashNextGpu::Upload + RepackQ8): the rows [row0, row0 + rows) of a Q8_0 tensor (dims[0] = cols,
 * rows counted over dims[1..]) go to the repacked device layout qs [rows][qstride] int8 + d [rows][cols / 32] fp16
 * through `staging` (device memory of at least one row's 34-byte blocks; larger staging moves more rows per copy).
 * Synchronous. */
int halo_gguf_upload_q8_0(halo_engine* eng, const halo_gguf_tensor* t, uint64_t row0, uint32_t rows, int8_t* qs,
                          uint16_t* d, uint32_t qstride, void* staging, size_t staging_bytes, char* err,
                          size_t errlen);

/* The model's configuration from GGUF metadata under "<general.architecture>." (the keys of Config::FromGguf,
 * src/model/config.cpp:77-160: block_count, embedding_length, full_attention_interval, attention.head_count,
 * attention.head_count_kv, attention.key_length, rope.dimension_count, rope.freq_base,
 * attention.layer_norm_rms_epsilon, ssm.conv_kernel, ssm.state_size, ssm.group_count, ssm.time_step_rank,
 * expert_count, expert_used_count, expert_feed_forward_length, expert_shared_feed_forward_length) and the vocabulary
 * from token_embd.weight. Session fields (max_sessions, max_context, prefix_tokens) are left as given in *cfg. */
int halo_model_config_from_gguf(const halo_gguf* g, halo_model_config* cfg, char* err, size_t errlen);
/* Loads every weight of the model from the checkpoint, by the reference's tensor names (src/model/weights.cpp:
 * 137-290): blk.N.{attn_norm, post_attention_norm}.weight; DeltaNet layers attn_qkv, attn_gate, ssm_alpha +
 * ssm_beta (the two halves of the model's alpha | beta rows), ssm_conv1d, ssm_a, ssm_dt.bias, ssm_norm, ssm_out;
 * attention layers attn_q (per head q | gate), attn_k, attn_v, attn_output, attn_q_norm, attn_k_norm; every layer
 * ffn_gate_inp, ffn_gate_exps, ffn_up_exps, ffn_down_exps, ffn_gate_inp_shexp, ffn_gate_shexp, ffn_up_shexp,
 * ffn_down_shexp; token_embd, output, output_norm. Q8_0 matrices are repacked on the device; fp32 tensors are
 * copied. Every tensor's type and shape is checked against the model before anything is copied. */
int halo_model_load_gguf(halo_model* m, const halo_gguf* g, char* err, size_t errlen);

#ifdef __cplusplus
}
#endif

#endif /* HALO_GGUF_H_ */
