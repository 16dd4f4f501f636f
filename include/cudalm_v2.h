/*
 * cudalm_v2 -- reader for the `.cudalm` v2 weight container (magic
 * "CUDLMW02") with repack-at-load into the engine's W4A16 layout.
 *
 * Replaces, for the projection engine's tensors, the reference's
 * WeightFileV2 (include/cudalm/weight_loader_v2.h, src/runtime/
 * weight_loader_v2.cpp:48-240) and the upload step of
 * Qwen35LayerWeights::load (weight_loader_v2.cpp:416-500). The on-disk
 * format is unchanged (include/cudalm/weight_format_v2.h:31-100):
 *
 *   header (88 B): magic[8] "CUDLMW02", version u32 = 2, flags u32 = 0,
 *     num_tensors u32, num_metadata u16, pad u16 = 0, then u64 pairs
 *     (offset, size) of the config blob (88 B), metadata, tensor table and
 *     payload (payload offset 16 B aligned); sections must not overlap.
 *   config blob: 21 little-endian i32/f32 fields + a reserved u32 = 0.
 *   metadata: num_metadata x (key_len u8, key, value_len u16 <= 4096, value).
 *   table entry: name_len u8 (1..255), name [A-Za-z0-9._-], dtype u8,
 *     ndim u8 (1..8), pad u16 = 0, dims i64[8] (unused = 0, used in
 *     1..1e8), offset u64 (from payload start), byte_size u64, align u8
 *     (1,2,4,8,16; the file offset must honour it), pad u8 = 0.
 *
 * The file is memory-mapped read-only; tensor views point into the mapping
 * and stay valid until cudalm_v2_close. Every structural rule of the
 * reference reader is enforced, and a rejected file leaves nothing open.
 * Error codes: the CUDALM_W4A16_E* set plus the CUDALM_V2_E* below.
 */
#ifndef CUDALM_V2_H
#define CUDALM_V2_H

#include <stddef.h>
#include <stdint.h>

#include <hip/hip_runtime_api.h>

#include "cudalm_w4a16.h"

#ifdef __cplusplus
extern "C" {
#endif

#define CUDALM_V2_EFORMAT (-7)   /* the file breaks a container rule */
#define CUDALM_V2_EIO (-8)       /* open / stat / map failed */
#define CUDALM_V2_ENOTFOUND (-9) /* no tensor of that name, or wrong dtype/shape */

/* cudalm::Dtype (include/cudalm/tensor.h:18-24) */
#define CUDALM_V2_DTYPE_FP16 1
#define CUDALM_V2_DTYPE_INT4_PACKED 2 /* dims in packed bytes: [N, K/2] */
#define CUDALM_V2_DTYPE_FP16_SCALE 3
#define CUDALM_V2_DTYPE_FP32 4
#define CUDALM_V2_DTYPE_BF16 5

typedef struct cudalm_v2_file cudalm_v2_file;

typedef struct cudalm_v2_tensor {
  const char* name; /* NUL-terminated, owned by the file */
  int dtype;
  int ndim;
  int64_t dims[8];
  uint64_t offset;    /* from the payload start */
  uint64_t byte_size;
  int align;
  const void* host;   /* bytes inside the mapping */
} cudalm_v2_tensor;

/* Qwen35Config, the 88-byte blob's field order (weight_format_v2.h:129-151). */
typedef struct cudalm_v2_config {
  int32_t hidden_size, num_hidden_layers, intermediate_size, vocab_size;
  int32_t n_heads, n_kv_heads, head_dim;
  int32_t lin_num_k_heads, lin_num_v_heads, lin_key_head_dim, lin_value_head_dim;
  int32_t lin_conv_kernel_dim, full_attention_interval, group_size, max_seq_len;
  float eps, rope_theta, partial_rotary_factor;
  int32_t mrope_section[3];
} cudalm_v2_config;

/* Open and validate. On failure *out is NULL and, if err is non-NULL, a
 * NUL-terminated reason is written to err[0 .. errlen). */
int cudalm_v2_open(const char* path, cudalm_v2_file** out, char* err, size_t errlen);
void cudalm_v2_close(cudalm_v2_file* f);

int cudalm_v2_num_tensors(const cudalm_v2_file* f);
int cudalm_v2_tensor_at(const cudalm_v2_file* f, int index, cudalm_v2_tensor* out);
int cudalm_v2_find(const cudalm_v2_file* f, const char* name, cudalm_v2_tensor* out);
/* Metadata value for key (NUL-terminated, owned by the file) or NULL. */
const char* cudalm_v2_meta(const cudalm_v2_file* f, const char* key);
int cudalm_v2_get_config(const cudalm_v2_file* f, cudalm_v2_config* out);

/* The per-layer tensor set of the Qwen3.5 hybrid stack for layer_idx
 * (weight_loader_v2.cpp:263-376): names, dtypes and shapes. */
int cudalm_v2_validate_layer(const cudalm_v2_file* f, int layer_idx, char* err, size_t errlen);

/* Shape of the W4A16 projection `prefix` ("layers.0.mlp.gate_proj"):
 * prefix.weight int4 [N, K/2] and prefix.scale fp16 [N, K/128], K % 128 == 0. */
int cudalm_v2_w4a16_shape(const cudalm_v2_file* f, const char* prefix, int* N, int* K);

/* Repack-at-load: the projection's file bytes, repacked on the host into
 * the prepacked layout (cudalm_w4a16_repack_host), copied to `packed_dev`
 * (>= cudalm_w4a16_packed_bytes(N, K) bytes, 16 B aligned) on `stream`.
 * Returns once the copy has completed. */
int cudalm_v2_upload_w4a16_packed(const cudalm_v2_file* f, const char* prefix, void* packed_dev,
                                  size_t bytes, hipStream_t stream);

/* A tensor's file bytes, unchanged, to device memory (dst_bytes >= its
 * byte_size), completed before return. */
int cudalm_v2_upload(const cudalm_v2_file* f, const char* name, void* dst_dev, size_t dst_bytes,
                     hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif
