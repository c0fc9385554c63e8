/* rdl_gguf.h -- GGUF reader of librdlquant.so: parses a GGUF v2/v3 file in
 * place (memory-mapped, nothing copied to host RAM) and streams tensor blocks
 * straight into device memory.
 *
 * Reference interface replaced (paths relative to the rust-deeplearning
 * repository root):
 *   GGUFFile::parse_header / parse_bytes   rustml/gguf/main/src/core/parser.rs:143-211
 *   Cursor::read_value (metadata values)   rustml/gguf/main/src/core/parser.rs:109-131
 *   GGUFFile::to_model_config              rustml/gguf/main/src/core/parser.rs:214-289
 *   GGUFFile::load_tensors                 rustml/gguf/main/src/core/parser.rs:292-351
 *   GGMLType (ids, block geometry)         rustml/gguf/main/src/api/types.rs:4-78
 *   GGUFValue::as_u32 / as_f32 / as_string rustml/gguf/main/src/api/types.rs:97-121
 *   GgufError                              rustml/gguf/main/src/api/error.rs:5-21
 *
 * The reference reads the whole file into a Vec twice (parse_header and
 * load_tensors) and copies every tensor into its own Vec.  Here the file is
 * mapped read-only once; header, metadata and tensor infos point into the
 * mapping, and rdl_gguf_upload_tensor copies a tensor's bytes to HBM through
 * two pinned staging buffers (file read of one chunk overlapped with the DMA
 * of the previous one).
 *
 * All entry points return an rdl_status (rdl_quant.h) and set
 * rdl_last_error() on failure, with the reference's error text where it has
 * one.  Strings returned by a handle live as long as the handle.
 */
#ifndef RDL_GGUF_H
#define RDL_GGUF_H

#include <stddef.h>
#include <stdint.h>

#include "rdl_quant.h"

#ifdef __cplusplus
extern "C" {
#endif

/* GgufError variants (error.rs:5-21) as status codes, after rdl_quant.h's. */
enum {
    RDL_ERR_GGUF_IO = 9,                /* GgufError::Io: file errors, unexpected EOF, invalid UTF-8 */
    RDL_ERR_GGUF_INVALID_FORMAT = 10,   /* GgufError::InvalidFormat: bad magic, unsupported version */
    RDL_ERR_GGUF_UNSUPPORTED_TYPE = 11, /* GgufError::UnsupportedType: unknown GGML or value type */
    RDL_ERR_GGUF_MISSING_METADATA = 12, /* GgufError::MissingMetadata */
    RDL_ERR_NOT_FOUND = 13              /* a tensor or metadata key that is not in the file */
};

/* GGUF metadata value type ids (the match in parser.rs:110-130). */
enum {
    RDL_GGUF_U8 = 0, RDL_GGUF_I8 = 1, RDL_GGUF_U16 = 2, RDL_GGUF_I16 = 3,
    RDL_GGUF_U32 = 4, RDL_GGUF_I32 = 5, RDL_GGUF_F32 = 6, RDL_GGUF_BOOL = 7,
    RDL_GGUF_STRING = 8, RDL_GGUF_ARRAY = 9, RDL_GGUF_U64 = 10, RDL_GGUF_I64 = 11,
    RDL_GGUF_F64 = 12
};

typedef struct rdl_gguf rdl_gguf;

/* A metadata value as it lies in the file.  For scalars `raw` points at the
 * little-endian value (raw_len bytes) and count = 1; for a string at its
 * UTF-8 bytes (raw_len = length, no terminator); for an array at its first
 * element, with elem_type and count set (raw_len covers every element). */
typedef struct rdl_gguf_value {
    int32_t type;
    int32_t elem_type; /* arrays only; -1 otherwise */
    uint64_t count;
    const void* raw;
    uint64_t raw_len;
} rdl_gguf_value;

/* GGUFTensorInfo (types.rs:123-130) plus its byte size. */
typedef struct rdl_gguf_tensor_info {
    const char* name;      /* NUL-terminated (a name may itself hold NUL bytes: name_len counts them) */
    uint64_t name_len;
    uint32_t n_dims;
    const uint64_t* dims;  /* GGUF order: innermost (row length) first */
    int32_t ggml_type;     /* GGMLType id */
    uint64_t offset;       /* relative to the data section */
    uint64_t n_bytes;      /* (product(dims) / block_size) * block_bytes, as load_tensors sizes it
                              (UINT64_MAX when that overflows 64 bits) */
} rdl_gguf_tensor_info;

/* GGUFFile::parse_header: maps `path` read-only and parses it. */
rdl_status rdl_gguf_open(const char* path, rdl_gguf** out);
/* GGUFFile::parse_bytes over a caller buffer, which must outlive the handle
 * (nothing is copied). */
rdl_status rdl_gguf_open_bytes(const void* data, size_t len, rdl_gguf** out);
rdl_status rdl_gguf_close(rdl_gguf* g);

/* GGUFFile fields: version, data_offset, tensor_infos.len(), metadata.len()
 * (distinct keys: a repeated key keeps its last value, as HashMap::insert). */
rdl_status rdl_gguf_version(const rdl_gguf* g, uint32_t* out);
rdl_status rdl_gguf_data_offset(const rdl_gguf* g, uint64_t* out);
rdl_status rdl_gguf_file_size(const rdl_gguf* g, uint64_t* out);
rdl_status rdl_gguf_tensor_count(const rdl_gguf* g, size_t* out);
rdl_status rdl_gguf_metadata_count(const rdl_gguf* g, size_t* out);

/* Metadata entry i (file order of first appearance; key NUL-terminated,
 * key_len bytes long) and lookup by a NUL-terminated key. */
rdl_status rdl_gguf_metadata_at(const rdl_gguf* g, size_t i, const char** key, size_t* key_len,
                                rdl_gguf_value* value);
rdl_status rdl_gguf_metadata_find(const rdl_gguf* g, const char* key, rdl_gguf_value* value);
/* Element i of an array value (for arrays of strings or arrays, located
 * through an index built while parsing). */
rdl_status rdl_gguf_array_element(const rdl_gguf* g, const rdl_gguf_value* array, uint64_t i,
                                  rdl_gguf_value* elem);

/* Typed getters with GGUFValue's conversion rules (types.rs:97-121):
 * u32 from U32, I32 or U64 (truncating casts); f32 from F32 or F64; string
 * from String.  A missing key or another type gives
 * RDL_ERR_GGUF_MISSING_METADATA (the reference's `ok_or_else` path). */
rdl_status rdl_gguf_get_u32(const rdl_gguf* g, const char* key, uint32_t* out);
rdl_status rdl_gguf_get_f32(const rdl_gguf* g, const char* key, float* out);
rdl_status rdl_gguf_get_string(const rdl_gguf* g, const char* key, const char** out, size_t* len);

/* Tensor info i (file order) and lookup by name. */
rdl_status rdl_gguf_tensor_info_at(const rdl_gguf* g, size_t i, rdl_gguf_tensor_info* out);
rdl_status rdl_gguf_find_tensor(const rdl_gguf* g, const char* name, size_t* index);

/* Host view of tensor i's bytes inside the mapping (zero-copy).  Fails with
 * RDL_ERR_GGUF_IO "Tensor '<name>' data exceeds file bounds" as
 * load_tensors does (parser.rs:307-312). */
rdl_status rdl_gguf_tensor_data(const rdl_gguf* g, size_t i, const void** data, uint64_t* len);

/* load_tensors for one tensor, into device memory: copies tensor i's raw
 * GGUF bytes (no dequantization, no repacking) to dst_dev, which must hold
 * dst_len >= n_bytes bytes.  Synchronous: returns once the bytes are in HBM.
 * `stream` is a hipStream_t (NULL: the null stream). */
rdl_status rdl_gguf_upload_tensor(const rdl_gguf* g, size_t i, void* dst_dev, uint64_t dst_len, void* stream);

/* load_tensors' F32 expansion for one tensor, on the device: tensor i's
 * blocks are uploaded to device scratch and expanded into dst_dev (f32,
 * 16-byte aligned, dst_len >= the tensor's element count) exactly as the
 * reference dequantizes at load (parser.rs:321-346, 371-776: K-quants,
 * Q4_1, Q5_0, Q5_1, Q8_1) or Tensor::to_f32 expands it at model build
 * (tensor.rs:535-639: F16, Q4_0, Q8_0); F32 is copied.  Only whole blocks
 * are expanded, the elements after them are zero (the reference's
 * n_elements / block_size).  Synchronous. */
rdl_status rdl_gguf_upload_tensor_f32(const rdl_gguf* g, size_t i, float* dst_dev, uint64_t dst_len, void* stream);

/* The same expansion of n_elements of GGML type ggml_type already in device
 * memory (src_dev: GGUF blocks, src_len bytes) into dst_dev; stream-ordered.
 * Unknown type ids give RDL_ERR_GGUF_UNSUPPORTED_TYPE. */
rdl_status rdl_dequantize_gguf_dev(int32_t ggml_type, const void* src_dev, size_t src_len, size_t n_elements,
                                   float* dst_dev, void* stream);

/* GgufModelConfig (types.rs:165-186) as filled by to_model_config
 * (parser.rs:214-289).  Optional fields the file lacks are 0, or -1 for the
 * token ids; has_* flags say which were present. */
typedef struct rdl_gguf_model_config {
    char architecture[64]; /* general.architecture, or "llama" (truncated to 63 bytes) */
    uint32_t dim;          /* {arch}.embedding_length (required) */
    uint32_t hidden_dim;   /* {arch}.feed_forward_length, else 4 * dim */
    uint32_t n_layers;     /* {arch}.block_count (required) */
    uint32_t n_heads;      /* {arch}.attention.head_count (required) */
    uint32_t n_kv_heads;   /* {arch}.attention.head_count_kv, else 0 */
    uint32_t vocab_size;   /* {arch}.vocab_size, tokenizer.ggml.tokens_count, len(tokenizer.ggml.tokens), else 32000 */
    float norm_eps;        /* {arch}.attention.layer_norm_rms_epsilon, else 1e-5 */
    uint32_t max_seq_len;  /* {arch}.context_length, else 2048 */
    float rope_theta;      /* {arch}.rope.freq_base, else 10000 */
    int64_t bos_token_id;  /* tokenizer.ggml.bos_token_id, else -1 */
    int64_t eos_token_id;  /* tokenizer.ggml.eos_token_id, else -1 */
    uint32_t head_dim;     /* {arch}.attention.key_length, else 0 */
    uint32_t sliding_window; /* {arch}.attention.sliding_window, else 0 */
    int32_t has_n_kv_heads, has_head_dim, has_sliding_window, has_chat_template;
} rdl_gguf_model_config;

rdl_status rdl_gguf_model_config_get(const rdl_gguf* g, rdl_gguf_model_config* out);

#ifdef __cplusplus
}
#endif

#endif
