/*
 * air_oracle_qwen2.h -- CPU oracle for one Qwen2 decode step.
 *
 * TEST INFRASTRUCTURE ONLY.  Plain-C restatement of AIR's
 * ReferenceExecutor::step_impl (src/reference/reference_executor.cpp:325-428)
 * with its helpers rms_norm (:17-27), silu (:33-35), apply_rope (:37-72) and
 * attention (:74-138), over the linears of air_oracle.h.  Arithmetic follows
 * the reference operation by operation: double sums for the norm and the
 * attention scores, double RoPE angles rounded to float, a double softmax
 * whose probabilities are rounded to float, float accumulation of the
 * attention output in token order, float SiLU.  The greedy choice is
 * Sampler::sample at temperature 0 (src/runtime/sampling.cpp:13-16): the
 * first maximum.
 */
#ifndef AIR_ORACLE_QWEN2_H
#define AIR_ORACLE_QWEN2_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* One tensor: GGML type id, bytes, GGML dims (dims[0] contiguous). bytes ==
 * NULL means the tensor is absent (optional biases, untied output). */
typedef struct oracle_tensor {
    int type;
    const uint8_t* bytes;
    uint64_t nbytes;
    uint64_t dims[2];
    uint32_t rank;
} oracle_tensor;

typedef struct oracle_qwen2_layer {
    oracle_tensor attn_norm, q, k, v, q_bias, k_bias, v_bias, o;
    oracle_tensor ffn_norm, gate, up, down;
} oracle_qwen2_layer;

typedef struct oracle_qwen2_model {
    uint32_t layers, embedding, ffn, heads, kv_heads, rope_dims;
    uint64_t context, vocab;
    double rope_base, eps;
    oracle_tensor token_embd, output_norm, output, output_bias;  /* output absent: tied to token_embd */
    const oracle_qwen2_layer* layer;                              /* [layers] */
} oracle_qwen2_model;

/* Contiguous fp32 K and V: [layers][capacity][kv_heads * head_dim]. */
typedef struct oracle_qwen2_cache {
    float* k;
    float* v;
    uint64_t tokens;
    uint64_t capacity;
} oracle_qwen2_cache;

int oracle_qwen2_cache_init(const oracle_qwen2_model* model, oracle_qwen2_cache* cache, uint64_t capacity);
void oracle_qwen2_cache_free(oracle_qwen2_cache* cache);

/* Appends `token` at position cache->tokens and writes the vocabulary logits.
 * logits == NULL skips the final norm and the lm_head (a prompt token whose
 * logits nobody reads); the cache advances exactly as with logits.  The
 * linears run on oracle_set_threads() threads (bit-identical results). */
int oracle_qwen2_step(const oracle_qwen2_model* model, oracle_qwen2_cache* cache, int32_t token, float* logits);

/* Index of the first maximum (std::max_element). */
uint64_t oracle_greedy(const float* logits, uint64_t n);

#ifdef __cplusplus
}
#endif

#endif /* AIR_ORACLE_QWEN2_H */
