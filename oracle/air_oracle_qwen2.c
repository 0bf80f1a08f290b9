/*
 * air_oracle_qwen2.c -- CPU oracle for one Qwen2 decode step.
 *
 * TEST INFRASTRUCTURE ONLY (see air_oracle_qwen2.h).  Each helper names the
 * reference function it restates; the order of every floating-point
 * operation is the reference's, so the same compiler settings give the same
 * bits.
 */
#include "air_oracle_qwen2.h"

#include "air_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

enum { Q_OK = 0, Q_INVALID_ARGUMENT = 1, Q_INVALID_STATE = 2, Q_DATA_ERROR = 5, Q_INTERNAL = 7 };

static uint64_t head_dim(const oracle_qwen2_model* m) { return m->embedding / m->heads; }
static uint64_t kv_width(const oracle_qwen2_model* m) { return (uint64_t)m->kv_heads * head_dim(m); }

/* ReferenceTensorReader::vector over a rank-1 tensor. */
static int vector_of(const oracle_tensor* t, uint64_t n, float* out) {
    if (!t->bytes) return Q_DATA_ERROR;
    return oracle_decode(t->type, t->bytes, t->nbytes, n, out);
}

/* ReferenceTensorReader::row: row `r` of a {K, N} matrix (tensor_reader.cpp:347-367). */
static int row_of(const oracle_tensor* t, uint64_t r, float* out) {
    const uint64_t k = t->dims[0];
    const uint32_t be = oracle_block_elements(t->type), bb = oracle_block_bytes(t->type);
    if (!be || k % be) return Q_DATA_ERROR;
    const uint64_t row_bytes = (k / be) * bb;
    if ((r + 1) * row_bytes > t->nbytes) return Q_INVALID_ARGUMENT;
    return oracle_decode(t->type, t->bytes + r * row_bytes, row_bytes, k, out);
}

/* matvec + add_optional_bias (reference_executor.cpp:314-323). */
static int linear_of(const oracle_tensor* w, const oracle_tensor* bias, const float* x, float* y) {
    float* b = NULL;
    int rc;
    if (bias && bias->bytes) {
        b = (float*)malloc(w->dims[1] * sizeof(float));
        if (!b) return Q_INTERNAL;
        rc = vector_of(bias, w->dims[1], b);
        if (rc) { free(b); return rc; }
    }
    rc = oracle_linear(w->type, w->bytes, w->nbytes, w->dims[0], w->dims[1], 1, x, b, y);
    free(b);
    return rc;
}

/* rms_norm (reference_executor.cpp:17-27). */
static void rms_norm(const float* in, const float* weight, uint64_t n, double eps, float* out) {
    double square_sum = 0.0;
    for (uint64_t i = 0; i < n; ++i) square_sum += (double)in[i] * in[i];
    const double mean = square_sum / (double)n;
    const float scale = (float)(1.0 / sqrt(mean + eps));
    for (uint64_t i = 0; i < n; ++i) out[i] = in[i] * scale * weight[i];
}

/* silu (reference_executor.cpp:33-35). */
static float silu(float v) { return v / (1.0f + expf(-v)); }

/* apply_rope's rotate_heads (reference_executor.cpp:51-66). */
static void rotate_heads(float* values, uint32_t heads, uint32_t hd, uint32_t rope_dims, uint64_t position,
                         double base) {
    const uint32_t half = rope_dims / 2u;
    for (uint32_t h = 0; h < heads; ++h) {
        const uint64_t b = (uint64_t)h * hd;
        for (uint32_t i = 0; i < half; ++i) {
            const double exponent = (2.0 * (double)i) / (double)rope_dims;
            const double inverse_frequency = 1.0 / pow(base, exponent);
            const double angle = (double)position * inverse_frequency;
            const float c = (float)cos(angle);
            const float s = (float)sin(angle);
            const float first = values[b + i];
            const float second = values[b + i + half];
            values[b + i] = first * c - second * s;
            values[b + i + half] = first * s + second * c;
        }
    }
}

/* attention (reference_executor.cpp:74-138) over the cache, whose last slot
 * already holds the current token's k and v. */
static int attention(const oracle_qwen2_model* m, const oracle_qwen2_cache* cache, uint32_t layer, const float* q,
                     uint64_t total, float* out) {
    const uint64_t hd = head_dim(m), kvw = kv_width(m);
    double* scores = (double*)malloc(total * sizeof(double));
    if (!scores) return Q_INTERNAL;
    const double scale = 1.0 / sqrt((double)hd);
    memset(out, 0, (uint64_t)m->heads * hd * sizeof(float));
    const float* kl = cache->k + (uint64_t)layer * cache->capacity * kvw;
    const float* vl = cache->v + (uint64_t)layer * cache->capacity * kvw;
    for (uint32_t qh = 0; qh < m->heads; ++qh) {
        const uint32_t kvh = (uint32_t)(((uint64_t)qh * m->kv_heads) / m->heads);
        const uint64_t qb = (uint64_t)qh * hd, kb = (uint64_t)kvh * hd;
        double maximum = -INFINITY;
        for (uint64_t t = 0; t < total; ++t) {
            const float* key = kl + t * kvw + kb;
            double score = 0.0;
            for (uint64_t d = 0; d < hd; ++d) score += (double)q[qb + d] * (double)key[d];
            score *= scale;
            scores[t] = score;
            if (score > maximum) maximum = score;
        }
        double denominator = 0.0;
        for (uint64_t t = 0; t < total; ++t) {
            scores[t] = exp(scores[t] - maximum);
            denominator += scores[t];
        }
        if (!(denominator > 0.0) || !isfinite(denominator)) { free(scores); return Q_INTERNAL; }
        for (uint64_t t = 0; t < total; ++t) {
            const float* value = vl + t * kvw + kb;
            const float p = (float)(scores[t] / denominator);
            for (uint64_t d = 0; d < hd; ++d) out[qb + d] += p * value[d];
        }
    }
    free(scores);
    return Q_OK;
}

int oracle_qwen2_cache_init(const oracle_qwen2_model* m, oracle_qwen2_cache* c, uint64_t capacity) {
    const uint64_t n = (uint64_t)m->layers * capacity * kv_width(m);
    c->k = (float*)calloc(n ? n : 1, sizeof(float));
    c->v = (float*)calloc(n ? n : 1, sizeof(float));
    c->tokens = 0;
    c->capacity = capacity;
    return c->k && c->v ? Q_OK : Q_INTERNAL;
}

void oracle_qwen2_cache_free(oracle_qwen2_cache* c) {
    free(c->k);
    free(c->v);
    c->k = c->v = NULL;
    c->tokens = c->capacity = 0;
}

uint64_t oracle_greedy(const float* logits, uint64_t n) {
    uint64_t best = 0;
    for (uint64_t i = 1; i < n; ++i)
        if (logits[best] < logits[i]) best = i;
    return best;
}

/* ReferenceExecutor::step_impl (reference_executor.cpp:325-428). */
int oracle_qwen2_step(const oracle_qwen2_model* m, oracle_qwen2_cache* c, int32_t token, float* logits) {
    if (token < 0 || (uint64_t)token >= m->vocab) return Q_INVALID_ARGUMENT;
    if (c->tokens >= m->context || c->tokens >= c->capacity) return Q_INVALID_STATE;
    const uint64_t e = m->embedding, hd = head_dim(m), kvw = kv_width(m), ffn = m->ffn;
    const uint64_t qw = (uint64_t)m->heads * hd;
    const uint64_t pos = c->tokens;
    int rc = Q_INTERNAL;
    float* hidden = (float*)malloc(e * sizeof(float));
    float* normed = (float*)malloc(e * sizeof(float));
    float* wbuf = (float*)malloc(e * sizeof(float));
    float* q = (float*)malloc(qw * sizeof(float));
    float* k = (float*)malloc(kvw * sizeof(float));
    float* v = (float*)malloc(kvw * sizeof(float));
    float* att = (float*)malloc(qw * sizeof(float));
    float* proj = (float*)malloc(e * sizeof(float));
    float* gate = (float*)malloc(ffn * sizeof(float));
    float* up = (float*)malloc(ffn * sizeof(float));
    if (!hidden || !normed || !wbuf || !q || !k || !v || !att || !proj || !gate || !up) goto done;

    if ((rc = row_of(&m->token_embd, (uint64_t)token, hidden))) goto done;
    for (uint32_t l = 0; l < m->layers; ++l) {
        const oracle_qwen2_layer* L = &m->layer[l];
        if ((rc = vector_of(&L->attn_norm, e, wbuf))) goto done;
        rms_norm(hidden, wbuf, e, m->eps, normed);
        if ((rc = linear_of(&L->q, &L->q_bias, normed, q))) goto done;
        if ((rc = linear_of(&L->k, &L->k_bias, normed, k))) goto done;
        if ((rc = linear_of(&L->v, &L->v_bias, normed, v))) goto done;
        rotate_heads(q, m->heads, (uint32_t)hd, m->rope_dims, pos, m->rope_base);
        rotate_heads(k, m->kv_heads, (uint32_t)hd, m->rope_dims, pos, m->rope_base);
        memcpy(c->k + ((uint64_t)l * c->capacity + pos) * kvw, k, kvw * sizeof(float));
        memcpy(c->v + ((uint64_t)l * c->capacity + pos) * kvw, v, kvw * sizeof(float));
        if ((rc = attention(m, c, l, q, pos + 1, att))) goto done;
        if ((rc = linear_of(&L->o, NULL, att, proj))) goto done;
        for (uint64_t i = 0; i < e; ++i) hidden[i] += proj[i];
        if ((rc = vector_of(&L->ffn_norm, e, wbuf))) goto done;
        rms_norm(hidden, wbuf, e, m->eps, normed);
        if ((rc = linear_of(&L->gate, NULL, normed, gate))) goto done;
        if ((rc = linear_of(&L->up, NULL, normed, up))) goto done;
        for (uint64_t i = 0; i < ffn; ++i) gate[i] = silu(gate[i]) * up[i];
        if ((rc = linear_of(&L->down, NULL, gate, proj))) goto done;
        for (uint64_t i = 0; i < e; ++i) hidden[i] += proj[i];
    }
    if (logits) {
        if ((rc = vector_of(&m->output_norm, e, wbuf))) goto done;
        rms_norm(hidden, wbuf, e, m->eps, normed);
        rc = linear_of(m->output.bytes ? &m->output : &m->token_embd, &m->output_bias, normed, logits);
    }
    if (rc == Q_OK) c->tokens = pos + 1;
done:
    free(hidden); free(normed); free(wbuf); free(q); free(k); free(v);
    free(att); free(proj); free(gate); free(up);
    return rc;
}
