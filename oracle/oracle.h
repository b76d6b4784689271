/*
 * ORACLE -- test infrastructure, not product code.
 *
 * A from-scratch CPU restatement, in plain C, of the reference engine's quantized-weight
 * matrix path (GGML block decode + scalar F32 dot/matvec), extended with the GGML formats
 * the reference only registers (Q4_K decode, Q8_K activation quantization, Q x Q8_K integer
 * dots).  It exists to check the HIP library; only tests, the smoke check and the CPU
 * baseline leg of the benchmark may load it.  Nothing on the product path calls it.
 *
 * Every function names the reference file:line it follows.  Functions whose behaviour the
 * reference does not contain (Q4_K decode, Q8_K quantize, integer Q x Q8_K dots) restate
 * GGML's published format algorithms; how each is pinned is written above its definition.
 *
 * Build with -ffp-contract=off and no -march (the reference's own flags add only warnings,
 * CMakeLists.txt:52-56): the reference's F32 arithmetic is a separate multiply and add.
 */
#ifndef ORACLE_ORACLE_H
#define ORACLE_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* status codes: the reference throws; the restatement returns the exception kind */
enum {
    ORC_OK = 0,
    ORC_INVALID_ARGUMENT = -1, /* std::invalid_argument */
    ORC_OUT_OF_RANGE = -2,     /* std::out_of_range */
    ORC_OVERFLOW = -3,         /* std::overflow_error */
    ORC_RUNTIME_ERROR = -4,    /* std::runtime_error (unsupported / unregistered type) */
    ORC_LOGIC_ERROR = -5       /* std::logic_error */
};

/* GGML type ids (ggml_type.cpp:12-54) */
enum {
    ORC_TYPE_F32 = 0,
    ORC_TYPE_F16 = 1,
    ORC_TYPE_Q8_0 = 8,
    ORC_TYPE_Q4_K = 12,
    ORC_TYPE_Q5_K = 13,
    ORC_TYPE_Q6_K = 14,
    ORC_TYPE_Q8_K = 15,
    ORC_TYPE_BF16 = 30
};

#define ORC_QK_K 256
#define ORC_Q4_K_BYTES 144
#define ORC_Q5_K_BYTES 176
#define ORC_Q6_K_BYTES 210
#define ORC_Q8_0_BYTES 34
#define ORC_Q8_K_BYTES 292

const char* orc_last_error(void);

/* registry: ggml_type.cpp:62-118 */
int orc_type_layout(uint32_t type, uint64_t* block_elements, uint64_t* bytes_per_block,
                    int* quantized, const char** name);
int orc_row_byte_size(uint64_t row_elements, uint32_t type, uint64_t* out);

/* scalar conversions: storage_decode.cpp:150-180 */
float orc_f16_to_f32(uint16_t bits);
float orc_bf16_to_f32(uint16_t bits);

/* block codecs: storage_decode.cpp:44-139 (+ GGML Q4_K) */
void orc_unpack_scale_min_k4(int index, const uint8_t* packed12, uint8_t* scale, uint8_t* minimum);
void orc_decode_q4_k_block(const uint8_t* block, float* out256);
void orc_decode_q5_k_block(const uint8_t* block, float* out256);
void orc_decode_q6_k_block(const uint8_t* block, float* out256);
void orc_decode_q8_0_block(const uint8_t* block, float* out32);

/* storage_decode.cpp:182-198 with the decoder whitelist extended by Q4_K */
int orc_check_row(uint32_t type, uint64_t row_elements, uint64_t nbytes);
/* storage_decode.cpp:244-294 */
int orc_decode_row(uint32_t type, uint64_t row_elements, const uint8_t* bytes, uint64_t nbytes,
                   float* out);

/* quantized_reference.cpp:24-82: one F32 accumulator, sequential, multiply then add */
int orc_storage_dot(uint32_t type, uint64_t row_elements, const uint8_t* bytes, uint64_t nbytes,
                    const float* x, float* out);
/* quantized_reference.cpp:128-162 */
int orc_storage_matvec(uint32_t type, uint64_t rows, uint64_t cols, const uint8_t* matrix,
                       uint64_t nbytes, const float* x, float* y);
/* same arithmetic per row, rows split over `threads` POSIX threads (CPU baseline timing) */
int orc_storage_matvec_mt(uint32_t type, uint64_t rows, uint64_t cols, const uint8_t* matrix,
                          uint64_t nbytes, const float* x, float* y, int threads);
/* M independent matvecs (the reference's multi-token semantics, qwen35_target_multi.cpp:14-25);
   x is [m][cols], y is [m][rows] */
int orc_storage_matmul_mt(uint32_t type, uint64_t rows, uint64_t cols, const uint8_t* matrix,
                          uint64_t nbytes, uint64_t m, const float* x, float* y, int threads);

/* tolerance companions: double-precision dot and the normaliser sum_k |w_k * x_k| */
int orc_storage_dot_stats(uint32_t type, uint64_t row_elements, const uint8_t* bytes,
                          uint64_t nbytes, const float* x, double* dot_f64, double* abs_sum);
int orc_storage_matvec_stats(uint32_t type, uint64_t rows, uint64_t cols, const uint8_t* matrix,
                             uint64_t nbytes, const float* x, double* dot_f64, double* abs_sum,
                             int threads);

/* GGML block_q8_K: { f32 d; i8 qs[256]; i16 bsums[16] } = 292 bytes */
int orc_quantize_row_q8_k(const float* x, uint64_t k, uint8_t* out);
int orc_dequantize_row_q8_k(const uint8_t* blocks, uint64_t k, float* out);

/* GGML integer dots of a weight row against a Q8_K row */
int orc_vec_dot_q8_k(uint32_t type, uint64_t k, const uint8_t* wrow, const uint8_t* q8k, float* out);

/* FNV-1a 64 over raw bytes (the reference fingerprints F32 bit patterns the same way,
   qwen35_block.cpp:354-364) */
uint64_t orc_fnv1a64(const void* data, uint64_t nbytes);

#ifdef __cplusplus
}
#endif

#endif
