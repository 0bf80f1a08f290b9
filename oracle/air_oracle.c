/*
 * air_oracle.c -- CPU oracle for the quantized linear path.
 *
 * TEST INFRASTRUCTURE ONLY (see air_oracle.h).  A plain-C restatement of the
 * reference CPU executor's block decoders and double-accumulating matvec,
 * written from the reference's documented behaviour; the citations name the
 * reference lines each function follows.
 */
#include "air_oracle.h"

#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* src/reference/tensor_reader.cpp:11-36: exact half -> single, including
 * subnormals (renormalised), signed zero, infinities and NaN payloads. */
float oracle_f16_to_f32(uint16_t value) {
    uint32_t sign = (uint32_t)(value & 0x8000u) << 16;
    uint32_t exponent = (value >> 10) & 0x1fu;
    uint32_t mantissa = value & 0x03ffu;
    uint32_t bits;
    if (exponent == 0) {
        if (mantissa == 0) {
            bits = sign;
        } else {
            /* value = mantissa * 2^-24; shift until the implicit bit appears */
            uint32_t e = 127u - 15u + 1u;
            while ((mantissa & 0x0400u) == 0) {
                mantissa <<= 1;
                --e;
            }
            bits = sign | (e << 23) | ((mantissa & 0x03ffu) << 13);
        }
    } else if (exponent == 0x1fu) {
        bits = sign | 0x7f800000u | (mantissa << 13);
    } else {
        bits = sign | ((exponent + 112u) << 23) | (mantissa << 13);
    }
    float out;
    memcpy(&out, &bits, sizeof out);
    return out;
}

static uint16_t rd16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }

uint32_t oracle_block_elements(int type) {
    switch (type) {
    case ORACLE_TYPE_F32: case ORACLE_TYPE_F16: case ORACLE_TYPE_BF16: return 1;
    case ORACLE_TYPE_Q4_0: case ORACLE_TYPE_Q5_0: case ORACLE_TYPE_Q8_0: return 32;
    case ORACLE_TYPE_Q4_K: case ORACLE_TYPE_Q6_K: return 256;
    default: return 0;
    }
}

uint32_t oracle_block_bytes(int type) {
    switch (type) {
    case ORACLE_TYPE_F32: return 4;
    case ORACLE_TYPE_F16: case ORACLE_TYPE_BF16: return 2;
    case ORACLE_TYPE_Q4_0: return 18;
    case ORACLE_TYPE_Q5_0: return 22;
    case ORACLE_TYPE_Q8_0: return 34;
    case ORACLE_TYPE_Q4_K: return 144;
    case ORACLE_TYPE_Q6_K: return 210;
    default: return 0;
    }
}

/* Q4_K 6-bit scale/min unpack for sub-block j of 8
 * (src/reference/tensor_reader.cpp:153-165). */
static void q4k_scale_min(uint32_t j, const uint8_t* s, uint8_t* sc, uint8_t* mn) {
    if (j < 4) {
        *sc = s[j] & 63u;
        *mn = s[j + 4] & 63u;
    } else {
        *sc = (uint8_t)((s[j + 4] & 0x0fu) | ((s[j - 4] >> 6) << 4));
        *mn = (uint8_t)((s[j + 4] >> 4) | ((s[j] >> 6) << 4));
    }
}

/* decode_all, src/reference/tensor_reader.cpp:51-247. */
int oracle_decode(int type, const uint8_t* bytes, uint64_t nbytes,
                  uint64_t elements, float* out) {
    const uint32_t be = oracle_block_elements(type);
    const uint32_t bb = oracle_block_bytes(type);
    if (be == 0) return ORACLE_UNSUPPORTED;
    if (elements % be != 0 || nbytes != (elements / be) * bb) return ORACLE_DATA_ERROR;
    const uint64_t blocks = elements / be;

    switch (type) {
    case ORACLE_TYPE_F32: /* :60-67 */
        for (uint64_t i = 0; i < elements; ++i) {
            uint32_t b = (uint32_t)bytes[4 * i] | ((uint32_t)bytes[4 * i + 1] << 8) |
                         ((uint32_t)bytes[4 * i + 2] << 16) | ((uint32_t)bytes[4 * i + 3] << 24);
            memcpy(&out[i], &b, 4);
        }
        return ORACLE_OK;
    case ORACLE_TYPE_F16: /* :68-75 */
        for (uint64_t i = 0; i < elements; ++i) out[i] = oracle_f16_to_f32(rd16(bytes + 2 * i));
        return ORACLE_OK;
    case ORACLE_TYPE_BF16: /* :76-84 */
        for (uint64_t i = 0; i < elements; ++i) {
            uint32_t b = (uint32_t)rd16(bytes + 2 * i) << 16;
            memcpy(&out[i], &b, 4);
        }
        return ORACLE_OK;
    case ORACLE_TYPE_Q4_0: /* :85-103  [d:f16][16 bytes: lo nibble = elem i, hi = elem i+16] */
        for (uint64_t b = 0; b < blocks; ++b) {
            const uint8_t* src = bytes + b * 18;
            const float d = oracle_f16_to_f32(rd16(src));
            float* dst = out + b * 32;
            for (int i = 0; i < 16; ++i) {
                const uint8_t p = src[2 + i];
                dst[i] = d * (float)((int)(p & 0x0f) - 8);
                dst[i + 16] = d * (float)((int)(p >> 4) - 8);
            }
        }
        return ORACLE_OK;
    case ORACLE_TYPE_Q5_0: /* :104-130  [d:f16][qh:4][qs:16] */
        for (uint64_t b = 0; b < blocks; ++b) {
            const uint8_t* src = bytes + b * 22;
            const float d = oracle_f16_to_f32(rd16(src));
            const uint8_t* qh = src + 2;
            const uint8_t* qs = src + 6;
            float* dst = out + b * 32;
            for (uint32_t i = 0; i < 16; ++i) {
                const uint32_t j = i + 16;
                const int h0 = ((qh[i / 8] >> (i % 8)) & 1) << 4;
                const int h1 = ((qh[j / 8] >> (j % 8)) & 1) << 4;
                dst[i] = d * (float)(((qs[i] & 0x0f) | h0) - 16);
                dst[j] = d * (float)(((qs[i] >> 4) | h1) - 16);
            }
        }
        return ORACLE_OK;
    case ORACLE_TYPE_Q8_0: /* :131-146  [d:f16][32 x int8] */
        for (uint64_t b = 0; b < blocks; ++b) {
            const uint8_t* src = bytes + b * 34;
            const float d = oracle_f16_to_f32(rd16(src));
            float* dst = out + b * 32;
            for (int i = 0; i < 32; ++i) dst[i] = d * (float)(int8_t)src[2 + i];
        }
        return ORACLE_OK;
    case ORACLE_TYPE_Q4_K: /* :147-196  [d:f16][dmin:f16][scales:12][qs:128] */
        for (uint64_t b = 0; b < blocks; ++b) {
            const uint8_t* src = bytes + b * 144;
            const float d = oracle_f16_to_f32(rd16(src));
            const float dmin = oracle_f16_to_f32(rd16(src + 2));
            const uint8_t* scales = src + 4;
            const uint8_t* qs = src + 16;
            float* dst = out + b * 256;
            for (uint32_t g = 0; g < 4; ++g) {
                uint8_t s0, m0, s1, m1;
                q4k_scale_min(2 * g, scales, &s0, &m0);
                q4k_scale_min(2 * g + 1, scales, &s1, &m1);
                const float d0 = d * (float)s0, mm0 = dmin * (float)m0;
                const float d1 = d * (float)s1, mm1 = dmin * (float)m1;
                for (uint32_t i = 0; i < 32; ++i) {
                    const uint8_t p = qs[g * 32 + i];
                    dst[g * 64 + i] = d0 * (float)(p & 0x0f) - mm0;
                    dst[g * 64 + 32 + i] = d1 * (float)(p >> 4) - mm1;
                }
            }
        }
        return ORACLE_OK;
    case ORACLE_TYPE_Q6_K: /* :197-242  [ql:128][qh:64][scales:16 x int8][d:f16] */
        for (uint64_t b = 0; b < blocks; ++b) {
            const uint8_t* src = bytes + b * 210;
            const float d = oracle_f16_to_f32(rd16(src + 208));
            float* dst = out + b * 256;
            for (uint32_t half = 0; half < 2; ++half) {
                const uint8_t* lo = src + half * 64;
                const uint8_t* hi = src + 128 + half * 32;
                const int8_t* sc = (const int8_t*)(src + 192 + half * 8);
                float* h = dst + half * 128;
                for (uint32_t i = 0; i < 32; ++i) {
                    const uint32_t pair = i / 16;
                    const int q0 = ((lo[i] & 0x0f) | (((hi[i] >> 0) & 3) << 4)) - 32;
                    const int q1 = ((lo[i + 32] & 0x0f) | (((hi[i] >> 2) & 3) << 4)) - 32;
                    const int q2 = ((lo[i] >> 4) | (((hi[i] >> 4) & 3) << 4)) - 32;
                    const int q3 = ((lo[i + 32] >> 4) | (((hi[i] >> 6) & 3) << 4)) - 32;
                    h[i] = d * (float)sc[pair + 0] * (float)q0;
                    h[i + 32] = d * (float)sc[pair + 2] * (float)q1;
                    h[i + 64] = d * (float)sc[pair + 4] * (float)q2;
                    h[i + 96] = d * (float)sc[pair + 6] * (float)q3;
                }
            }
        }
        return ORACLE_OK;
    default:
        return ORACLE_UNSUPPORTED;
    }
}

static int row_geometry(int type, uint64_t K, uint64_t N, uint64_t nbytes, uint64_t* row_bytes) {
    const uint32_t be = oracle_block_elements(type);
    const uint32_t bb = oracle_block_bytes(type);
    if (be == 0) return ORACLE_UNSUPPORTED;
    /* decode_range requires block-aligned rows (:297-331) */
    if (K == 0 || K % be != 0) return ORACLE_UNSUPPORTED;
    *row_bytes = (K / be) * bb;
    if (nbytes != *row_bytes * N) return ORACLE_DATA_ERROR;
    return ORACLE_OK;
}

static uint32_t g_threads = 1;

void oracle_set_threads(uint32_t threads) { g_threads = threads == 0 ? 1 : (threads > 64 ? 64 : threads); }
uint32_t oracle_threads(void) { return g_threads; }

/* One output row r of every input row (ReferenceTensorReader::matvec,
 * src/reference/tensor_reader.cpp:369-394, plus add_optional_bias):
 * y[m * y_stride + col] = float(sum_k double(w[r,k]) * double(x[m,k])) (+ bias[r]). */
static int linear_one_row(int type, const uint8_t* bytes, uint64_t row_bytes, uint64_t K, uint32_t M,
                          const float* x, const float* bias, uint64_t r, float* w, float* y, uint64_t y_stride,
                          uint64_t col) {
    int rc = oracle_decode(type, bytes + r * row_bytes, row_bytes, K, w);
    if (rc != ORACLE_OK) return rc;
    for (uint32_t m = 0; m < M; ++m) {
        const float* xm = x + (uint64_t)m * K;
        double sum = 0.0;
        for (uint64_t k = 0; k < K; ++k) sum += (double)w[k] * (double)xm[k];
        float out = (float)sum;
        if (bias) out += bias[r]; /* add_in_place after the matvec, f32 */
        y[(uint64_t)m * y_stride + col] = out;
    }
    return ORACLE_OK;
}

/* A slice of the output rows: either the range [begin, end) (rows == NULL,
 * output column = row) or the listed rows rows[begin..end) (column = index). */
typedef struct linear_job {
    int type;
    const uint8_t* bytes;
    uint64_t row_bytes, K, y_stride;
    uint32_t M;
    const float* x;
    const float* bias;
    const uint64_t* rows;
    uint64_t begin, end;
    float* y;
    int rc;
} linear_job;

static void* linear_job_run(void* arg) {
    linear_job* j = (linear_job*)arg;
    /* the reference decodes each row into a fresh heap vector (:384); one
       buffer per job computes the same values */
    float* w = (float*)malloc(j->K * sizeof(float));
    j->rc = w ? ORACLE_OK : ORACLE_DATA_ERROR;
    for (uint64_t i = j->begin; w && i < j->end && j->rc == ORACLE_OK; ++i) {
        const uint64_t r = j->rows ? j->rows[i] : i;
        j->rc = linear_one_row(j->type, j->bytes, j->row_bytes, j->K, j->M, j->x, j->bias, r, w, j->y, j->y_stride,
                               j->rows ? i : r);
    }
    free(w);
    return NULL;
}

/* Runs `job` over [begin, end) on up to g_threads threads (contiguous
 * slices; every row is computed by exactly one thread). */
static int run_linear_jobs(linear_job job, uint64_t begin, uint64_t end) {
    const uint64_t count = end - begin;
    uint64_t threads = g_threads;
    /* below ~1M multiply-adds a thread costs more than it saves */
    if (count * job.K * job.M < (1u << 20)) threads = 1;
    if (threads > count) threads = count ? count : 1;
    linear_job jobs[64];
    pthread_t tids[64];
    int started[64] = {0};
    for (uint64_t t = 0; t < threads; ++t) {
        jobs[t] = job;
        jobs[t].begin = begin + count * t / threads;
        jobs[t].end = begin + count * (t + 1) / threads;
        if (t + 1 < threads && pthread_create(&tids[t], NULL, linear_job_run, &jobs[t]) == 0) {
            started[t] = 1;
        } else {
            linear_job_run(&jobs[t]);   /* the last slice (or a failed spawn) on this thread */
        }
    }
    int rc = ORACLE_OK;
    for (uint64_t t = 0; t < threads; ++t) {
        if (started[t]) pthread_join(tids[t], NULL);
        if (rc == ORACLE_OK && jobs[t].rc != ORACLE_OK) rc = jobs[t].rc;
    }
    return rc;
}

/* ReferenceTensorReader::matvec, src/reference/tensor_reader.cpp:369-394. */
int oracle_linear_rows(int type, const uint8_t* bytes, uint64_t nbytes,
                       uint64_t K, uint64_t N, uint32_t M,
                       const float* x, const float* bias, float* y,
                       uint64_t row_begin, uint64_t row_end) {
    uint64_t row_bytes = 0;
    int rc = row_geometry(type, K, N, nbytes, &row_bytes);
    if (rc != ORACLE_OK) return rc;
    if (row_begin > row_end || row_end > N) return ORACLE_INVALID_ARGUMENT;
    const linear_job job = {type, bytes, row_bytes, K, N, M, x, bias, NULL, 0, 0, y, ORACLE_OK};
    return run_linear_jobs(job, row_begin, row_end);
}

int oracle_linear_row_list(int type, const uint8_t* bytes, uint64_t nbytes,
                           uint64_t K, uint64_t N, uint32_t M,
                           const float* x, const float* bias,
                           const uint64_t* rows, uint64_t count, float* y) {
    uint64_t row_bytes = 0;
    int rc = row_geometry(type, K, N, nbytes, &row_bytes);
    if (rc != ORACLE_OK) return rc;
    if (count && !rows) return ORACLE_INVALID_ARGUMENT;
    for (uint64_t i = 0; i < count; ++i) {
        if (rows[i] >= N) return ORACLE_INVALID_ARGUMENT;
    }
    const linear_job job = {type, bytes, row_bytes, K, count, M, x, bias, rows, 0, 0, y, ORACLE_OK};
    return run_linear_jobs(job, 0, count);
}

int oracle_linear(int type, const uint8_t* bytes, uint64_t nbytes,
                  uint64_t K, uint64_t N, uint32_t M,
                  const float* x, const float* bias, float* y) {
    return oracle_linear_rows(type, bytes, nbytes, K, N, M, x, bias, y, 0, N);
}

int oracle_matvec(int type, const uint8_t* bytes, uint64_t nbytes,
                  uint64_t K, uint64_t N, const float* x, float* y) {
    return oracle_linear(type, bytes, nbytes, K, N, 1, x, NULL, y);
}
