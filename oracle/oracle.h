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

/* ---------------------------------------------------------------- Gated DeltaNet decode block
 * Restatement of the reference's recurrent (linear-attention) block at batch 1:
 *   orc_sigmoid / orc_softplus / orc_silu    qwen35_block.cpp:138-159
 *   orc_rms_norm_rows                        qwen35_block.cpp:161-186 (double sum of squares)
 *   orc_l2_inverse (inside the delta step)   reference_kernels.cpp:283-292
 *   orc_conv_step                            reference_kernels.cpp:197-225
 *   orc_gated_delta_step                     reference_kernels.cpp:227-335 (state [head][key][value])
 *   orc_deltanet_step                        qwen35_block.cpp:406-605 + finish_block :326-352 +
 *                                            execute_mlp :296-324
 * The block's projections use the device path's product semantics: a K-quant weight row is
 * dotted (quantized_reference.cpp:24-82 arithmetic) with the activation after Q8_K
 * quantization and dequantization; other types with the F32 activation.
 */
float orc_sigmoid(float v);
float orc_softplus(float v);
float orc_silu(float v);
/* out[r][c] = in[r][c] * inverse_rms(r) * weight[c]; rows = n / width */
int orc_rms_norm_rows(const float* in, const float* weight, uint64_t n, uint64_t width, float eps,
                      float* out);
/* history [channels][kernel] is shifted and receives input; out = sum(history * weights) */
int orc_conv_step(const float* input, const float* weights, uint64_t channels, uint64_t kernel,
                  float* history, float* out, int apply_silu);
/* q, k [heads][dk]; v, out [heads][dv]; beta, log_decay [heads]; state [heads][dk][dv] */
int orc_gated_delta_step(const float* q, const float* k, const float* v, const float* beta,
                         const float* log_decay, uint64_t heads, uint64_t dk, uint64_t dv,
                         float eps, float* state, float* out);

typedef struct orc_deltanet_block {
    uint64_t embedding, key_heads, value_heads, key_dim, value_dim, conv_kernel, ffn;
    float eps;
    /* GGML weights, rows x cols row-major GGML rows (dimensions[1] x dimensions[0]) */
    uint32_t qkv_type, z_type, beta_type, alpha_type, out_type, gate_type, up_type, down_type;
    const uint8_t *qkv, *z, *beta, *alpha, *out, *gate, *up, *down;
    /* F32 vectors: input_norm[E], conv_weight[C][kernel], dt_bias[Hv], decay[Hv],
       out_norm[dv], post_norm[E] */
    const float *input_norm, *conv_weight, *dt_bias, *decay, *out_norm, *post_norm;
} orc_deltanet_block;

/* intermediates, in order (NULL to skip); sizes: C = 2*Hk*dk + Hv*dv, V = Hv*dv, F = ffn */
enum { ORC_DN_TRACE_FIELDS = 16 };
/* trace layout: qkv[C] z[V] beta[Hv] alpha[Hv] conv[C] rec[V] gated[V] branch[E] resid[E]
   post[E] gate[F] up[F] act[F] ffn[E] beta_s[Hv] log_decay[Hv]  (beta_s = sigmoid(beta),
   log_decay = softplus(alpha + dt_bias) * decay: the reference's "beta_sigmoid" and "gate") */
uint64_t orc_deltanet_trace_size(const orc_deltanet_block* b);
int orc_deltanet_step(const orc_deltanet_block* b, float* conv_history, float* state,
                      const float* x, float* y, float* trace, int threads);

/* ---------------------------------------------------------------- full-attention decode
 * Restatement of the reference's attention block at batch 1:
 *   orc_rope                  reference_kernels.cpp:77-125 (+ position_for_frequency :28-40):
 *                             angles in double (base^(2f/R), coordinate * 1/that), cos and sin
 *                             rounded to F32, pairs (f, R/2 + f) rotated with separate F32
 *                             multiplies and adds
 *   orc_kv_cache              KvCache (hybrid_cache.cpp:131-207): keys [capacity][kv_heads][key_dim],
 *                             values [capacity][kv_heads][value_dim], F32, caller-owned arrays
 *   orc_attention_step        reference_kernels.cpp:127-195: append, then per query head
 *                             (kv head = head / (q_heads / kv_heads)) double-accumulated dots
 *                             times 1/sqrt(key_dim) in F32, max, expf, double denominator,
 *                             F32 probabilities, F32 weighted sum in token order
 *   orc_attention_block_step  qwen35_block.cpp:607-756 + finish_block :326-352 + execute_mlp
 *                             :296-324, projections with orc_deltanet_step's semantics
 */
typedef struct orc_kv_cache {
    uint64_t capacity, kv_heads, key_dim, value_dim, length;
    float *keys, *values;
} orc_kv_cache;
/* heads [n_heads][head_dim] rotated in place; position = {temporal, height, width} */
int orc_rope(float* heads, uint64_t n_heads, uint64_t head_dim, uint64_t rotary_dim, const int32_t sections[4],
             float base, const uint64_t position[3]);
/* q [q_heads][key_dim], k [kv_heads][key_dim], v [kv_heads][value_dim] -> out [q_heads][value_dim] */
int orc_attention_step(const float* q, uint64_t q_heads, const float* k, const float* v, orc_kv_cache* cache,
                       float* out);

typedef struct orc_attention_block {
    uint64_t embedding, q_heads, kv_heads, head_dim, ffn, rope_dim;
    int32_t rope_sections[4];
    float rope_base, eps;
    /* GGML weights: q [E -> 2*Hq*D] (per head: D query values then D gate values),
       k [E -> Hkv*D], v [E -> Hkv*D], out [Hq*D -> E], gate/up [E -> F], down [F -> E] */
    uint32_t q_type, k_type, v_type, out_type, gate_type, up_type, down_type;
    const uint8_t *q, *k, *v, *out, *gate, *up, *down;
    /* F32 vectors: input_norm[E], q_norm[D], k_norm[D], post_norm[E] */
    const float *input_norm, *q_norm, *k_norm, *post_norm;
} orc_attention_block;

/* trace layout (Q = Hq*D, KV = Hkv*D): qfull[2Q] k[KV] v[KV] qcur[Q] kcur[KV] pregate[Q]
   gate_s[Q] gated[Q] branch[E] resid[E] post[E] gate[F] up[F] act[F] ffn[E]  -- the reference's
   Qcur_full Kcur_projected Vcur_projected Qcur Kcur attn_pregate gate_sigmoid attn_gated
   attn_output attn_residual attn_post_norm ffn_gate ffn_up ffn_swiglu ffn_out */
enum { ORC_ATTN_TRACE_FIELDS = 15 };
uint64_t orc_attention_trace_size(const orc_attention_block* b);
int orc_attention_block_step(const orc_attention_block* b, orc_kv_cache* cache, const uint64_t position[3],
                             const float* x, float* y, float* trace, int threads);

/* FNV-1a 64 over raw bytes (the reference fingerprints F32 bit patterns the same way,
   qwen35_block.cpp:354-364) */
uint64_t orc_fnv1a64(const void* data, uint64_t nbytes);

#ifdef __cplusplus
}
#endif

#endif
