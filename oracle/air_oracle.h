/*
 * air_oracle.h -- CPU oracle for the quantized linear path.
 *
 * TEST INFRASTRUCTURE ONLY.  This is a clean-room plain-C restatement of
 * AIR's reference CPU executor for GGUF block decode and the
 * double-accumulating matrix-vector product.  Only tests/, the smoke entry
 * point and the CPU-baseline leg of bench.py may load it, and only as the
 * checker: no product code path calls it.
 *
 * Every function cites the reference function it restates
 * (paths relative to the AIR 0.9.12 checkout).
 *
 * Type ids are GGML/GGUF on-disk type ids (the `format_type` field of the
 * reference TensorDescriptor, src/formats/gguf/gguf_format.cpp:24-63).
 */
#ifndef AIR_ORACLE_H
#define AIR_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    ORACLE_TYPE_F32 = 0,
    ORACLE_TYPE_F16 = 1,
    ORACLE_TYPE_Q4_0 = 2,
    ORACLE_TYPE_Q5_0 = 6,
    ORACLE_TYPE_Q8_0 = 8,
    ORACLE_TYPE_Q4_K = 12,
    ORACLE_TYPE_Q6_K = 14,
    ORACLE_TYPE_BF16 = 30
};

/* Return codes mirror air::ErrorCode (include/air/status.hpp:8-17). */
enum {
    ORACLE_OK = 0,
    ORACLE_INVALID_ARGUMENT = 1,
    ORACLE_DATA_ERROR = 5,
    ORACLE_UNSUPPORTED = 6
};

/* Exact IEEE half -> single (src/reference/tensor_reader.cpp:11-36). */
float oracle_f16_to_f32(uint16_t bits);

/* Elements per block and bytes per block of a type; 0 for unknown types
 * (block geometry of src/reference/tensor_reader.cpp:59-242). */
uint32_t oracle_block_elements(int type);
uint32_t oracle_block_bytes(int type);

/* Decode `elements` values from canonical GGUF bytes
 * (decode_all, src/reference/tensor_reader.cpp:51-247).  `nbytes` must be
 * exactly the storage size of `elements` values. */
int oracle_decode(int type, const uint8_t* bytes, uint64_t nbytes,
                  uint64_t elements, float* out);

/* y[r] = float(sum_k double(w[r,k]) * double(x[k])), k ascending, for a GGML
 * row-major matrix with dims {K, N} (ReferenceTensorReader::matvec,
 * src/reference/tensor_reader.cpp:369-394).  Rows are decoded one at a time
 * (decode_range, :270-345). */
int oracle_matvec(int type, const uint8_t* bytes, uint64_t nbytes,
                  uint64_t K, uint64_t N, const float* x, float* y);

/* M independent matvecs over rows of x [M x K] into y [M x N], each followed
 * by the optional f32 bias add of ReferenceExecutor::add_optional_bias
 * (src/reference/reference_executor.cpp:29-31,315-323).  `bias` may be NULL.
 * This is the per-item semantics every GPU batch row must reproduce. */
int oracle_linear(int type, const uint8_t* bytes, uint64_t nbytes,
                  uint64_t K, uint64_t N, uint32_t M,
                  const float* x, const float* bias, float* y);

/* Same as oracle_linear but rows [row_begin, row_end) of the output only
 * (for timing bounded samples of very large matrices). */
int oracle_linear_rows(int type, const uint8_t* bytes, uint64_t nbytes,
                       uint64_t K, uint64_t N, uint32_t M,
                       const float* x, const float* bias, float* y,
                       uint64_t row_begin, uint64_t row_end);

/* Rows rows[0..count) of the linear: y[m][j] is output row rows[j] of input
 * row m (y is [M x count]), computed exactly as oracle_linear computes that
 * row.  For parity checks of very large matrices on a seeded sample of
 * rows. */
int oracle_linear_row_list(int type, const uint8_t* bytes, uint64_t nbytes,
                           uint64_t K, uint64_t N, uint32_t M,
                           const float* x, const float* bias,
                           const uint64_t* rows, uint64_t count, float* y);

/* Worker threads the linears above may split their output rows over (default
 * 1, at most 64).  Each output row is still one sequential double sum in k
 * order, computed by one thread, so the results are bit-identical for every
 * thread count; the reference itself is single-threaded
 * (tensor_reader.cpp:383-393). */
void oracle_set_threads(uint32_t threads);
uint32_t oracle_threads(void);

#ifdef __cplusplus
}
#endif

#endif /* AIR_ORACLE_H */
