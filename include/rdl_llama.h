/* rdl_llama.h -- batch-1 Llama-style decoder on one MI355X, built on the
 * quantized Linear path of rdl_quant.h (librdlquant.so).
 *
 * It replaces, for GGUF models (Q4_0, Q8_0, Q4_1, Q4_K, Q6_K matrices) with
 * RMSNorm, RoPE, grouped-query attention and SwiGLU, the rustml decode loop:
 *   LlmModel::forward_with_cache_pass   rustml/nlp/main/src/core/model.rs:890-937
 *   TransformerBlock::forward_with_cache rustml/nn/main/src/core/transformer_block.rs:297-356
 *   MultiHeadAttention::forward_with_cache rustml/nn/main/src/core/attention.rs:353-449
 *   FeedForward::forward (SwiGLU)       rustml/nn/main/src/core/feed_forward.rs:138-150
 *   RoPEFreqs::new / apply              rustml/nn/main/src/core/rope.rs:93-200
 *   KVCache                             rustml/nn/main/src/core/kv_cache.rs:10-114
 *   Generator::prefill / decode_step    rustml/nlp/main/src/core/generator.rs:212-240
 *   sampling::argmax                    rustml/nlp/main/src/core/sampling.rs:8-18
 * Activations, the KV cache and the sampled tokens stay on the device; a
 * greedy decode step is one replay of a captured HIP graph.
 *
 * Divergences from the reference, by design: the KV cache may be held in
 * f16 (kv_f16 = 1; the reference keeps f32), and the last row's logits are
 * the only ones computed (the reference computes every row and keeps the
 * last). */
#ifndef RDL_LLAMA_H
#define RDL_LLAMA_H

#include <stddef.h>
#include <stdint.h>

#include "rdl_gguf.h"
#include "rdl_quant.h"

#ifdef __cplusplus
extern "C" {
#endif

/* ModelConfig fields used by the Llama path (rustml/nlp/main/src/api/types.rs:186). */
typedef struct rdl_llama_config {
    int32_t dim;         /* hidden size */
    int32_t n_layers;
    int32_t n_heads;     /* query heads */
    int32_t n_kv_heads;  /* key/value heads (n_heads % n_kv_heads == 0) */
    int32_t head_dim;    /* dim == n_heads * head_dim; even */
    int32_t ffn_dim;     /* SwiGLU hidden size */
    int32_t vocab;
    int32_t max_seq;     /* KV cache capacity (max_seq_len) */
    float norm_eps;
    float rope_theta;
    int32_t kv_f16;      /* 1: f16 KV cache, 0: f32 (the reference's) */
    int32_t max_batch;   /* most rows one forward call takes (prefill chunk) */
    int32_t output_dtype; /* GGML type of the output matrix: RDL_DTYPE_Q4_0 (also
                             when 0), _Q8_0, _Q4_1, _Q4_K or _Q6_K (K-quants:
                             dim % 256 == 0) */
} rdl_llama_config;

typedef struct rdl_llama rdl_llama;

/* Weight slots.  GGUF block bytes for the matrices (row-major [out, in]
 * blocks, as Linear::from_weights receives them) and the embedding, in the
 * slot's type (Q4_0 unless rdl_llama_create_typed says otherwise); f32 for
 * the norm weights.  `layer` is ignored for the model-level slots. */
enum {
    RDL_LLAMA_TOKEN_EMBEDDING = 0, /* [vocab, dim] (dequantized per row like Tensor::to_f32) */
    RDL_LLAMA_ATTN_NORM = 1,       /* [dim] f32 */
    RDL_LLAMA_WQ = 2,              /* [n_heads*head_dim, dim] */
    RDL_LLAMA_WK = 3,              /* [n_kv_heads*head_dim, dim] */
    RDL_LLAMA_WV = 4,              /* [n_kv_heads*head_dim, dim] */
    RDL_LLAMA_WO = 5,              /* [dim, n_heads*head_dim] */
    RDL_LLAMA_FFN_NORM = 6,        /* [dim] f32 */
    RDL_LLAMA_W_GATE = 7,          /* [ffn_dim, dim] */
    RDL_LLAMA_W_UP = 8,            /* [ffn_dim, dim] */
    RDL_LLAMA_W_DOWN = 9,          /* [dim, ffn_dim] */
    RDL_LLAMA_FINAL_NORM = 10,     /* [dim] f32 */
    RDL_LLAMA_OUTPUT = 11,         /* [vocab, dim] in output_dtype's GGUF blocks */
    RDL_LLAMA_SLOTS = 12
};

/* Allocates weights, KV cache and activations on the current device; every
 * matrix and the embedding Q4_0, the output matrix in cfg->output_dtype. */
rdl_status rdl_llama_create(const rdl_llama_config* cfg, rdl_llama** out);

/* The same with a GGUF type per matrix (as llama.cpp's mixed files hold
 * them, e.g. Q4_K with Q6_K attn_v / ffn_down layers): types[layer *
 * RDL_LLAMA_SLOTS + slot] for the per-layer matrix slots, layer 0's row for
 * the embedding and output slots; norm slots are ignored; 0 means Q4_0 (the
 * output: cfg->output_dtype).  Types: Q4_0, Q8_0, Q4_1, Q4_K, Q6_K (K-quants
 * need in_features % 256 == 0).  A layer whose matrices are all Q4_0 runs
 * the fused launches; other layers run their GEMVs by type with separate
 * norm / RoPE / SwiGLU / add launches (q, k, v and gate, up as separate
 * matrices when their types differ).  types may be NULL (rdl_llama_create). */
rdl_status rdl_llama_create_typed(const rdl_llama_config* cfg, const int32_t* types, rdl_llama** out);
rdl_status rdl_llama_free(rdl_llama* model);

/* Copies one weight from host memory (len must equal the slot's size). */
rdl_status rdl_llama_set_weight(rdl_llama* model, int32_t slot, int32_t layer, const void* bytes,
                                size_t len);

/* Seeded synthetic weights on the device, all slots: Q4_0 blocks with
 * nibbles uniform in [0, 15] and d = f16(|N(0, 0.02)| / 8), norm weights 1.0.
 * All-Q4_0 models only (RDL_ERR_UNSUPPORTED otherwise). */
rdl_status rdl_llama_init_random(rdl_llama* model, uint64_t seed);

/* Empties the KV cache (KVCache::new state, current_len = 0). */
rdl_status rdl_llama_reset(rdl_llama* model);

/* Number of cached positions (KVCache::current_len). */
rdl_status rdl_llama_position(const rdl_llama* model, size_t* out);

/* The KV cache is paged (the decode-loop extension of KVCache, kv_cache.rs:
 * 23-114, whose cache is one contiguous [n_kv][max_seq][hd] buffer per layer):
 * positions live in pages of page_positions (64) positions, each page holding
 * every KV head's rows of one layer, and a device table maps logical page
 * pos / page_positions to a physical page of the pool.  The table starts as
 * the identity (the contiguous layout).  rdl_llama_kv_pages reports the page
 * size and the number of pages (ceil(max_seq / page_positions)). */
rdl_status rdl_llama_kv_pages(const rdl_llama* model, size_t* page_positions, size_t* n_pages);
/* Installs a page table: table[logical page] = physical page, a permutation
 * of 0 .. n_pages - 1 (RDL_ERR_INVALID_DATA otherwise, RDL_ERR_SHAPE_MISMATCH
 * for another length).  Only on an empty cache (position 0, after create or
 * rdl_llama_reset; RDL_ERR_INVALID_DATA otherwise); it then holds for every
 * write and read of the cache, captured decode graphs included. */
rdl_status rdl_llama_set_kv_page_table(rdl_llama* model, const int32_t* table, size_t n);

/* Decode steps (one row) of layers whose matrices are all Q4_0 run the
 * q/k/v projection, the attention and the o projection in one launch when
 * the cache layout allows (f16 cache with head_dim 64 or 128, f32 cache with
 * head_dim 64); with enable = 2 that launch also runs the previous such
 * layer's down projection (a decode step then takes two launches a layer);
 * enable = 1 runs the down projection on its own, enable = 0 the q/k/v
 * projection, the attention and the o projection as three launches.  Every
 * level does the same arithmetic with the same results.  The default is 1
 * (on the 7B shape level 2 measured 788 against 824 tokens/s).  No
 * reference counterpart: a tuning and testing switch. */
rdl_status rdl_llama_set_fused_attention(rdl_llama* model, int32_t enable);

/* Linear::set_native_q4_matmul for every Linear of one layer
 * (TransformerBlock::set_native_q4_matmul, transformer_block.rs:248-255;
 * layer = -1: every layer, as gemma3_gguf.rs:126-128 does): the layer's
 * Q4_0 and Q4_1 products quantize their activation rows to Q8_0
 * (quantize_row_q8_0) and sum int32 block dots (matmul_f32_q4_native /
 * matmul_f32_q4_1_native, quantize.rs:326-394, 501-572); other types keep
 * their one path (linear.rs:119-177).  Such layers run their RMSNorm, RoPE,
 * SwiGLU and adds as separate launches.  The output matrix is not a layer's
 * and keeps the float path, as in the reference.  Default: off. */
rdl_status rdl_llama_set_native_q4(rdl_llama* model, int32_t layer, int32_t enable);

/* Kernel launches the model has enqueued since create, by attention path:
 * host-side counts (a captured decode graph counts its launches once, at
 * capture, however often it is replayed).  No reference counterpart: it lets
 * tests assert which kernels a configuration reaches. */
typedef struct rdl_llama_path_counts {
    uint64_t fused_decode;  /* q/k/v projection + attention + o projection in one launch */
    uint64_t prefill_mfma;  /* prompt-chunk attention on the matrix cores (f16 cache, 32+ rows) */
    uint64_t prefill_rows;  /* prompt-chunk attention, a wave a row over LDS-staged pages */
    uint64_t attention;     /* the per-row attention launch (span workgroups) */
    uint64_t fused_down;    /* of fused_decode: led by the previous layer's down projection */
} rdl_llama_path_counts;
rdl_status rdl_llama_get_path_counts(const rdl_llama* model, rdl_llama_path_counts* out);

/* forward_with_cache_pass over n tokens followed by cache.advance(n): the
 * logits of the last row, copied to host memory (vocab floats).  Token ids
 * must be < vocab; n <= max_batch; position + n <= max_seq.  Synchronous.
 * After an RDL_ERR_HIP from this call or rdl_llama_generate_greedy the cache
 * contents are undefined: rdl_llama_reset before the next call. */
rdl_status rdl_llama_forward(rdl_llama* model, const int32_t* tokens, size_t n, float* logits,
                             size_t logits_len);

/* Greedy generation (Generator::generate with argmax sampling): prefill of
 * the prompt (in chunks of max_batch), then n_gen - 1 decode steps, each one
 * replay of a captured graph; out_tokens receives the n_gen sampled ids.
 * Continues from the current cache position.  Synchronous. */
rdl_status rdl_llama_generate_greedy(rdl_llama* model, const int32_t* prompt, size_t n_prompt,
                                     size_t n_gen, int32_t* out_tokens);

/* Device time, in milliseconds, of the last rdl_llama_generate_greedy call:
 * its prefill and its decode steps (HIP events on the model's stream). */
rdl_status rdl_llama_last_timing(const rdl_llama* model, float* prefill_ms, float* decode_ms);

/* The model's RoPE tables (RoPEFreqs::new: [max_seq, head_dim/2] f32 each),
 * copied to host memory. */
rdl_status rdl_llama_rope_tables(const rdl_llama* model, float* cos_out, float* sin_out, size_t len);

/* The config a model was created with (for a GGUF load: as resolved from
 * the file's metadata and tensor shapes). */
rdl_status rdl_llama_get_config(const rdl_llama* model, rdl_llama_config* out);

/* Options of rdl_llama_load_gguf. */
typedef struct rdl_llama_gguf_options {
    int32_t max_seq;   /* KV cache capacity; 0: the file's context_length (2048 if absent) */
    int32_t max_batch; /* rows per forward call; 0: 32 */
    int32_t kv_f16;    /* 1: f16 KV cache, 0: f32 */
} rdl_llama_gguf_options;

/* LlmModel::from_pretrained over GGUFFile::load_and_remap, the Llama branch
 * of rustml/nlp/main/src/bin/infer.rs:80-120:
 *   config   to_model_config (parser.rs:214-289) -> gguf_config_to_model_config
 *            (gguf_bridge.rs:46-84) -> ModelConfig::validate (types.rs:794-826)
 *   names    gguf_llama_weight_map (weight_map.rs:26-73)
 *   weights  from_pretrained (nlp/main/src/core/model.rs:81-232)
 * head_dim = dim / n_heads, the FFN width and the vocabulary come from the
 * ffn_up and output matrices.  Every mapped tensor's type, shape and file
 * bounds are checked before anything is allocated; the bytes then go from the
 * file mapping to HBM through pinned staging buffers, without a host copy of
 * the file.  Tensors the map does not name are ignored.  Errors: a missing
 * weight gives RDL_ERR_NOT_FOUND "Missing weight: <internal name>" (the
 * reference's ModelError text); a matrix or embedding that is not Q4_0 /
 * Q8_0 / Q4_1 / Q4_K / Q6_K (each keeps its own type, as in
 * rdl_llama_create_typed), norm weights that are not F32/F16, a model
 * without ffn_gate or a gemma3 file give
 * RDL_ERR_UNSUPPORTED; dims that differ from the config give
 * RDL_ERR_SHAPE_MISMATCH.  opt may be NULL (all defaults). */
rdl_status rdl_llama_load_gguf(const rdl_gguf* gguf, const rdl_llama_gguf_options* opt, rdl_llama** out);

#ifdef __cplusplus
}
#endif

#endif
