/*
 * oq.h -- C ABI of the MI355X (gfx950) quantized-weight matrix library (liboq.so).
 *
 * Plain pointers and sizes only.  "dev" pointers are device (HBM) addresses; "host" pointers
 * are ordinary host memory (an mmap'd GGUF payload is fine).  Every entry point returns an
 * oq_status; the text of the last failure on a context is available from oq_last_error().
 *
 * Each declaration names the reference interface it replaces (paths are relative to the
 * reference engine's source tree).  The reference's quantized path is a set of free
 * functions in oracle::backend::cpu (include/oracle/backend/cpu/quantized_reference.hpp:10-27)
 * over oracle::model::GgufTensorView (include/oracle/model/mapped_gguf.hpp:18-41) and the
 * GGML layout registry (include/oracle/model/ggml_type.hpp:9-24).  The C++ adapter in
 * oracle_amd/host/ maps those signatures, and their exceptions, onto this ABI.
 *
 * Threading: one oq_context owns one HIP stream on one device and is not thread-safe.
 * Weights are immutable after upload and may be used from any context on the same device.
 * All compute entry points are asynchronous on the context's stream; oq_synchronize() waits.
 */
#ifndef OQ_H
#define OQ_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum oq_status {
    OQ_OK = 0,
    OQ_INVALID_ARGUMENT = -1, /* reference: std::invalid_argument */
    OQ_OUT_OF_RANGE = -2,     /* reference: std::out_of_range */
    OQ_OVERFLOW = -3,         /* reference: std::overflow_error */
    OQ_UNSUPPORTED_TYPE = -4, /* reference: std::runtime_error("unsupported GGML tensor type") */
    OQ_DEVICE_ERROR = -5,     /* HIP runtime failure */
    OQ_OUT_OF_MEMORY = -6,    /* device allocation failure */
    OQ_LOGIC_ERROR = -7,      /* reference: std::logic_error (bad row geometry) */
    OQ_RUNTIME_ERROR = -8     /* reference: std::runtime_error (malformed model payload) */
} oq_status;

/* GGML type ids, as registered in the reference (src/model/ggml_type.cpp:12-54) */
enum {
    OQ_TYPE_F32 = 0,
    OQ_TYPE_F16 = 1,
    OQ_TYPE_Q8_0 = 8,
    OQ_TYPE_Q4_K = 12,
    OQ_TYPE_Q5_K = 13,
    OQ_TYPE_Q6_K = 14,
    OQ_TYPE_Q8_K = 15,
    OQ_TYPE_BF16 = 30
};

typedef struct oq_context oq_context;
typedef struct oq_weight oq_weight;
typedef struct oq_graph oq_graph;

/* ------------------------------------------------------------------ registry */

/* Replaces oracle::model::ggml_type_layout (src/model/ggml_type.cpp:62-75).  Returns
   OQ_UNSUPPORTED_TYPE for unknown, deprecated and removed ids (the reference returns nullptr).
   Any output pointer may be NULL.  *name points at static storage. */
int oq_type_layout(uint32_t type, uint64_t* block_elements, uint64_t* bytes_per_block,
                   int* quantized, const char** name);

/* Replaces oracle::model::ggml_row_byte_size (src/model/ggml_type.cpp:77-94): unknown type ->
   OQ_UNSUPPORTED_TYPE, zero elements -> OQ_INVALID_ARGUMENT, ragged row -> OQ_UNSUPPORTED_TYPE
   (the reference throws std::runtime_error for both), overflow -> OQ_OVERFLOW. */
int oq_row_byte_size(uint64_t row_elements, uint32_t type, uint64_t* out);

/* 1 if the device path decodes/multiplies this type: f32, f16, bf16, q8_0, q4_K, q5_K, q6_K.
   This is the reference decoder whitelist (src/model/storage_decode.cpp:192-193) plus q4_K. */
int oq_type_supported(uint32_t type);

/* ------------------------------------------------------------------ context */

/* No reference counterpart (the reference is CPU-only; backend choice by name happens in
   src/runtime/engine.cpp:62-72).  Creates a context on HIP device `device` with its own stream. */
int oq_context_create(int device, oq_context** out);
void oq_context_destroy(oq_context* ctx);
/* Text of the last failure on ctx (or of the last failed oq_context_create when ctx is NULL). */
const char* oq_last_error(const oq_context* ctx);
int oq_synchronize(oq_context* ctx);
/* The context's hipStream_t, for callers that interleave their own work. */
void* oq_context_stream(oq_context* ctx);
/* Launch-shape options (environment variables OQ_GEMV_*, OQ_GEMM_*, OQ_BLOCK_*, ... selecting
   alternative kernel schedules for measurement) are read once, when the first context is
   created; this re-reads them.  No reference counterpart.  The option table is replaced
   atomically, so launches on other threads read either the old or the new one. */
void oq_reload_options(void);

/* Device memory helpers (so callers need no other GPU runtime). */
int oq_device_alloc(oq_context* ctx, uint64_t bytes, void** out_dev);
int oq_device_free(oq_context* ctx, void* dev);
int oq_copy_to_device(oq_context* ctx, void* dst_dev, const void* src_host, uint64_t bytes);
int oq_copy_to_host(oq_context* ctx, void* dst_host, const void* src_dev, uint64_t bytes);
int oq_copy_device(oq_context* ctx, void* dst_dev, const void* src_dev, uint64_t bytes);

/* ------------------------------------------------------------------ weights */

/* One-time upload of a rank-2 GGML tensor: ne0 = K (contiguous, GGUF dimensions[0]),
   ne1 = N rows (dimensions[1]), `host_bytes` = GgufTensorView::bytes() (zero-copy: the mmap
   pointer is copied straight to HBM).  Validates exactly what reference_storage_matvec
   validates before its loop (src/backend/cpu/quantized_reference.cpp:134-153) plus the decoder
   whitelist (src/model/storage_decode.cpp:192-193, extended by q4_K).  Quantized rows (q8_0,
   q4_K, q5_K, q6_K) are re-laid out on the device into aligned planes; the values they decode to
   are unchanged. */
int oq_weight_upload(oq_context* ctx, uint32_t type, uint64_t ne0, uint64_t ne1,
                     const void* host_bytes, uint64_t nbytes, oq_weight** out);
/* Same, from bytes already in device memory (e.g. a whole GGUF payload uploaded once). */
int oq_weight_upload_device(oq_context* ctx, uint32_t type, uint64_t ne0, uint64_t ne1,
                            const void* dev_bytes, uint64_t nbytes, oq_weight** out);
void oq_weight_release(oq_weight* w);
int oq_weight_info(const oq_weight* w, uint32_t* type, uint64_t* ne0, uint64_t* ne1,
                   uint64_t* device_bytes);

/* ------------------------------------------------------------------ whole-model upload */

/* One tensor of a GGUF payload: GgufTensorInfo (include/oracle/model/gguf.hpp:77-82) with its
   byte offset in the payload passed to oq_model_upload (GgufTensorView::absolute_offset when the
   payload is the whole mapped file, MappedGgufModel::mapping()). */
typedef struct oq_tensor_desc {
    const char* name;
    uint32_t type;     /* GGML type id */
    uint32_t n_dims;   /* 1..4 */
    uint64_t dims[4];  /* dims[0] contiguous (GGUF dimensions) */
    uint64_t offset;   /* byte offset in the payload */
} oq_tensor_desc;

typedef struct oq_model oq_model;

/* Checks a tensor table against a payload of payload_bytes the way the reference's GGUF reader
   and MappedGgufModel do (src/model/gguf.cpp:457-497, src/model/mapped_gguf.cpp:124-203), in
   their order: unique names, dimension count and non-zero dimensions, offsets inside the payload
   (OQ_RUNTIME_ERROR); then per tensor its registered type (OQ_UNSUPPORTED_TYPE), byte size
   (ggml_tensor_byte_size, src/model/ggml_type.cpp:96-118: ragged rows, overflow) and payload
   end (OQ_RUNTIME_ERROR); then overlapping payloads (OQ_RUNTIME_ERROR).  Tensors of more than
   four dimensions are refused (OQ_INVALID_ARGUMENT).  Host only, needs no device. */
int oq_model_validate(uint64_t payload_bytes, const oq_tensor_desc* tensors, uint64_t count);

/* Replaces the per-call use of mapped tensor views with one upload of the whole model: validates
   as oq_model_validate, then copies the payload to HBM once (in payload order, through a staging
   buffer of max(256 MiB, largest tensor)).  Rank-2 tensors of a type oq_type_supported accepts
   become weights (as oq_weight_upload: device row layout, ready for oq_matvec / oq_matmul);
   every other tensor keeps its GGML bytes in HBM.  The host payload may be released afterwards. */
int oq_model_upload(oq_context* ctx, const void* payload, uint64_t payload_bytes, const oq_tensor_desc* tensors,
                    uint64_t count, oq_model** out);
void oq_model_release(oq_model* m);
uint64_t oq_model_tensor_count(const oq_model* m);
/* MappedGgufModel::find_tensor / tensor (src/model/mapped_gguf.cpp:211-222): index of the tensor
   called `name`; OQ_OUT_OF_RANGE ("GGUF tensor not found") if there is none. */
int oq_model_find(const oq_model* m, const char* name, uint64_t* index);
typedef struct oq_model_tensor_info {
    const char* name;        /* valid while the model lives */
    uint32_t type, n_dims;
    uint64_t dims[4];
    uint64_t nbytes;          /* GGML bytes */
    const oq_weight* weight;  /* the uploaded weight, or NULL */
    const void* data_dev;     /* the GGML bytes in HBM when weight is NULL, else NULL */
} oq_model_tensor_info;
int oq_model_tensor(const oq_model* m, uint64_t index, oq_model_tensor_info* info);
/* HBM held by the model (weights in device layout plus raw tensors). */
uint64_t oq_model_device_bytes(const oq_model* m);

/* ------------------------------------------------------------------ decode */

/* Replaces oracle::backend::cpu::reference_decode_mapped_tensor
   (src/backend/cpu/quantized_reference.cpp:85-105) and, row by row, oracle::model::
   decode_storage_row (src/model/storage_decode.cpp:244-294): rows [row0, row0+nrows) of w
   decoded to F32 into out_dev[nrows][ne0].  Bit-identical to the reference's decode.
   row0 + nrows > ne1 -> OQ_OUT_OF_RANGE (make_storage_row_view(tensor,row),
   src/model/storage_decode.cpp:223-225). */
int oq_dequantize_rows(oq_context* ctx, const oq_weight* w, uint64_t row0, uint64_t nrows,
                       float* out_dev);

/* ------------------------------------------------------------------ activations */

/* F32 -> GGML block_q8_K {f32 d; i8 qs[256]; i16 bsums[16]} (292 B per 256 values).  The
   reference registers the layout only (src/model/ggml_type.cpp:28); this is GGML's
   quantize_row_q8_K: bit-identical to it for finite inputs (an all-zero block gets d = 0 and
   zero bsums).  x_dev is [m][k], q8k_dev receives m*k/256 blocks.  k % 256 != 0 ->
   OQ_INVALID_ARGUMENT. */
int oq_quantize_q8k(oq_context* ctx, const float* x_dev, uint64_t m, uint64_t k, void* q8k_dev);

/* Replaces the greedy choice over a logits vector, Sampler::sample at temperature 0
   (src/runtime/sampler.cpp:22-41) and the MTP argmax (src/runtime/qwen35_mtp.cpp:300-308), on
   logits left in device memory by the head's oq_matvec: *token_dev = the first index of the
   maximum of logits_dev[0..n), *value_dev = that maximum.  A NaN anywhere gives *token_dev =
   0xFFFFFFFF (the reference rejects NaN logits); all -inf gives token 0 with value -inf (the
   sampler rejects that, the MTP argmax returns 0).  Asynchronous on the context's stream,
   graph-capturable.  Errors: OQ_INVALID_ARGUMENT for n == 0, n > 2^32 - 1, null or misaligned
   buffers. */
int oq_argmax(oq_context* ctx, const float* logits_dev, uint64_t n, uint32_t* token_dev, float* value_dev);

/* The output head and its greedy token in one call: oq_matvec(w, x) into logits y_dev (ne1
   values), then oq_argmax over them -- the head matvec and sampler of the reference's decode step
   (src/runtime/qwen35_forward.cpp:450-465 with Sampler::sample at temperature 0,
   src/runtime/sampler.cpp:22-44; MTP: src/runtime/qwen35_mtp.cpp:292-308).  For K-quant weights the
   decode GEMV reduces the logits it writes to one partial per workgroup and a single small kernel
   combines them (no pass over the logits); other types run the two calls.  Same results as the
   two calls: token = first index of the maximum, 0xFFFFFFFF if a logit is NaN. */
int oq_matvec_argmax(oq_context* ctx, const oq_weight* w, const float* x_dev, float* y_dev, uint32_t* token_dev,
                     float* value_dev);

/* ------------------------------------------------------------------ products */

/* Replaces oracle::backend::cpu::reference_mapped_tensor_matvec / reference_storage_matvec
   (src/backend/cpu/quantized_reference.cpp:107-162): y_dev[n] = row_n(w) . x for n < ne1.
   x_dev holds ne0 F32 values, y_dev ne1.  q4_K / q5_K / q6_K weights quantize x to Q8_K on the
   device and use integer dots (GGML vec_dot_qX_K_q8_K semantics); q8_0 and plain types use the
   F32 activation directly.  Result within 1e-4 * sum_k |w_k x_k| of the reference's F32 dot. */
int oq_matvec(oq_context* ctx, const oq_weight* w, const float* x_dev, float* y_dev);

/* As oq_matvec for K-quant weights, with activations already in Q8_K blocks (ne0/256 blocks). */
int oq_matvec_q8k(oq_context* ctx, const oq_weight* w, const void* q8k_dev, float* y_dev);

/* M activation rows: x_dev [m][ne0] -> y_dev [m][ne1].  The reference has no M>1 kernel; its
   multi-token evaluation is M independent matvecs (src/runtime/qwen35_target_multi.cpp:14-25),
   which is the semantics here.  Small m streams the weights once with register reuse;
   m >= 16 on q4_K, q5_K and q6_K with K >= 4096 uses matrix cores: both operands rounded once
   to f16 (each weight the reference's F32 decoded value, Q8_K activations dequantized), F32
   accumulation.  Each product is then off by at most about 2^-10 of itself (a weight below
   2^-14 in magnitude, binary16's subnormal range, by at most 2^-25 absolute), so an output is
   within about 2^-10 of sum |w * xhat| (plus F32 summation) whatever the data, and within the
   product bar (1e-4 of it) when the sum spreads over many products (N(0,1)-like rows: 2.4e-5 to
   4.3e-5 measured); a row led by a few products exceeds 1e-4 (up to 7e-4 measured on saturated
   SwiGLU outputs).  OQ_GEMM_MFMA=0 (read by oq_reload_options) sends every m to the integer-dot
   path instead (exact products, F32 scales).  OQ_GEMM_FAST_DEQUANT=1 (measurement only) rounds
   the scales and mins to f16 first, which voids the per-product bound for q4_K / q5_K.  Each activation row is scaled by
   a power of two into binary16's range before the rounding and scaled back in the output, so any
   finite activation magnitude is accepted.  Weights must decode inside binary16's range
   (|(d sc) q - dmin m| <= 65504, i.e. d <= 69 for q4_K / q5_K; GGUF checkpoints store d as f16 and
   hold values many orders below that); a weight outside it makes that output non-finite. */
int oq_matmul(oq_context* ctx, const oq_weight* w, uint64_t m, const float* x_dev, float* y_dev);
int oq_matmul_q8k(oq_context* ctx, const oq_weight* w, uint64_t m, const void* q8k_dev,
                  float* y_dev);

/* ------------------------------------------------------------------ Gated DeltaNet block */
/* One Qwen3.5 recurrent (Gated DeltaNet) decoder block at batch 1, chained on the device.
   Replaces oracle::runtime::execute_qwen35_recurrent_block_reference
   (src/runtime/qwen35_block.cpp:406-605, with finish_block :326-352 and execute_mlp :296-324):
     normed = RMSNorm(x) * input_norm
     qkv, z, beta, alpha = projections of normed          (qkv: [2*Hk*dk + Hv*dv] rows)
     conv = SiLU(causal depthwise conv step of qkv)       (reference_kernels.cpp:197-225)
     out  = gated delta rule step over Hv heads            (reference_kernels.cpp:227-335)
            with q, k of key head h % Hk, beta = sigmoid(beta),
            log_decay = softplus(alpha + dt_bias) * decay
     gated = RMSNorm_head(out) * out_norm * SiLU(z);  branch = out_proj(gated)
     resid = x + branch;  post = RMSNorm(resid) * post_norm
     y = resid + down(SiLU(gate(post)) * up(post))
   The projections run on the library's matvec path (K-quant weights: activations quantized to
   Q8_K, as oq_matvec).  conv_history_dev [C][conv_kernel] and state_dev [Hv][dk][dv] (the
   reference's SsmState buffers, hybrid_cache.hpp:76-120) are updated in place.  trace_dev, if
   not NULL, receives the intermediates in this order (F32, packed):
     qkv[C] z[Hv*dv] beta[Hv] alpha[Hv] conv[C] out[Hv*dv] gated[Hv*dv] branch[E] resid[E]
     post[E] gate[F] up[F] act[F] ffn[E] beta_s[Hv] log_decay[Hv]      with C = 2*Hk*dk + Hv*dv,
     beta_s = sigmoid(beta), log_decay = softplus(alpha + dt_bias) * decay.
   Shapes: dk in {32, 64, 128}, dv in {64, 128, 192, 256} and conv_kernel <= 16 take the fused
   launches; any other shape (dk <= 4096; wider keys -> OQ_INVALID_ARGUMENT) runs one launch per
   stage with the delta rule's state in HBM, in the same arithmetic order (the register-resident
   kernel's bits where both apply).  Weight shape mismatches -> OQ_INVALID_ARGUMENT. */
typedef struct oq_deltanet_block {
    uint64_t embedding;   /* E */
    uint64_t key_heads;   /* Hk */
    uint64_t value_heads; /* Hv, a multiple of Hk */
    uint64_t key_dim;     /* dk */
    uint64_t value_dim;   /* dv */
    uint64_t conv_kernel; /* taps of the causal convolution */
    uint64_t ffn;         /* F */
    float eps;            /* RMSNorm / L2-norm epsilon (manifest attention_rms_epsilon) */
    const oq_weight *qkv, *z, *beta, *alpha, *out, *gate, *up, *down;
    /* F32 device vectors: input_norm[E], conv_weight[C][conv_kernel], dt_bias[Hv], decay[Hv],
       out_norm[dv], post_norm[E] */
    const float *input_norm, *conv_weight, *dt_bias, *decay, *out_norm, *post_norm;
} oq_deltanet_block;
int oq_deltanet_step(oq_context* ctx, const oq_deltanet_block* block, float* conv_history_dev,
                     float* state_dev, const float* x_dev, float* y_dev, float* trace_dev);

/* m consecutive tokens through the block: the same results as m oq_deltanet_step calls on the rows
   of x_dev [m][E] in order (token t sees the convolution history and state that token t - 1 left),
   y_dev [m][E].  Replaces the per-token loop of the reference's multi-token evaluation
   (src/runtime/qwen35_target_multi.cpp:14-25, one execute_qwen35_recurrent_block_reference per
   token per block; MTP verification, src/runtime/qwen35_mtp_chain_verify_batched.cpp:38-158).  Each
   projection streams its weights once for all m tokens (m >= 16: the matrix-core path of
   oq_matmul, with its precision contract, except the out projection, whose heavy-tailed gated
   input keeps the integer-dot products; below 16: the small-batch integer-dot products); the
   convolution and the delta rule run the tokens in order inside one launch each, the state read
   and written once, every token's arithmetic that of the single step.  trace_dev, if not NULL,
   receives m traces of oq_deltanet_step's layout, one after the other.  Checks as
   oq_deltanet_step, plus m in 1..65535 and x_dev 16-byte aligned. */
int oq_deltanet_steps(oq_context* ctx, const oq_deltanet_block* block, uint64_t m, float* conv_history_dev,
                      float* state_dev, const float* x_dev, float* y_dev, float* trace_dev);

/* ------------------------------------------------------------------ full attention (decode) */
/* A device KV cache in the reference's layout and semantics (oracle::runtime::KvCache,
   include/oracle/runtime/hybrid_cache.hpp:37-74, src/runtime/hybrid_cache.cpp:131-207): keys
   [capacity][kv_heads][key_dim] and values [capacity][kv_heads][value_dim], F32, in HBM; `size`
   tokens are stored, appends write row `size`.  The length is kept on the host: a step enqueued
   on a context counts as appended when it returns OQ_OK.
   Create: zero capacity / heads / dimensions -> OQ_INVALID_ARGUMENT ("KV cache capacity must be
   non-zero", "KV head count ...", "KV key dimension ...", "KV value dimension ...", :139-142);
   the arrays are allocated and zeroed.  The cache belongs to the creating context. */
typedef struct oq_kv_cache oq_kv_cache;
int oq_kv_cache_create(oq_context* ctx, uint64_t capacity, uint64_t kv_heads, uint64_t key_dim,
                       uint64_t value_dim, oq_kv_cache** out);
/* No counterpart in the reference (its cache is F32): a cache whose key and value elements are of
   `type`, OQ_TYPE_F32 (as oq_kv_cache_create) or OQ_TYPE_F16 (binary16: half the bytes that every
   attention step reads).  An F16 cache stores each appended or loaded F32 element rounded to
   nearest even, and attention steps read what is stored, the new token's row included: their
   outputs are attention over the rounded rows, within the same bound as over an F32 cache, and
   differ from an F32 cache's by that rounding (relative 2^-11 per element).  Other types ->
   OQ_INVALID_ARGUMENT ("KV cache element type must be F32 or F16"); then as oq_kv_cache_create. */
int oq_kv_cache_create_typed(oq_context* ctx, uint64_t capacity, uint64_t kv_heads, uint64_t key_dim,
                             uint64_t value_dim, uint32_t type, oq_kv_cache** out);
uint32_t oq_kv_cache_type(const oq_kv_cache* cache);  /* OQ_TYPE_F32 or OQ_TYPE_F16; 0 for NULL */
void oq_kv_cache_release(oq_kv_cache* cache);
uint64_t oq_kv_cache_size(const oq_kv_cache* cache);      /* KvCache::size */
uint64_t oq_kv_cache_capacity(const oq_kv_cache* cache);  /* KvCache::capacity */
/* KvCache::reset (hybrid_cache.cpp:171-175): length 0, arrays zeroed (on the context's stream) */
int oq_kv_cache_reset(oq_kv_cache* cache);
/* KvCache::truncate (:177-182): new_length > size -> OQ_INVALID_ARGUMENT ("KV cache truncate
   must not grow state") */
int oq_kv_cache_truncate(oq_kv_cache* cache, uint64_t new_length);
/* No counterpart in the reference (its cache only grows by append): stores `length` token rows
   [length][kv_heads][dim] from host memory and sets the length, e.g. to resume from keys and
   values computed elsewhere.  length > capacity -> OQ_OVERFLOW ("KV cache capacity exceeded").
   The rows are F32 for either element type; an F16 cache rounds them on the device (through a
   staging buffer of at most 64 MiB, allocated for the call). */
int oq_kv_cache_load(oq_kv_cache* cache, const float* keys_host, const float* values_host, uint64_t length);
/* the device arrays (row t, head h of keys at element (t * kv_heads + h) * key_dim), of the
   cache's element type: F32, or binary16 for an F16 cache (the pointers then address 2-byte
   elements) */
int oq_kv_cache_arrays(const oq_kv_cache* cache, float** keys_dev, float** values_dev);

/* oracle::runtime::apply_qwen35_rope (src/runtime/reference_kernels.cpp:77-125) on
   heads_dev [n_heads][head_dim] in place: frequency f < rotary_dim/2 turns the pair
   (f, rotary_dim/2 + f) by coordinate * base^(-2f/rotary_dim), the coordinate being
   position[1] (height) when f % 3 == 1 and f / 3 < sections[1], position[2] (width) when
   f % 3 == 2 and f / 3 < sections[2], else position[0] (temporal).  Angles in double, cos and
   sin rounded to F32, separate F32 multiplies and adds, as the reference.  The reference's checks
   and messages (OQ_INVALID_ARGUMENT): rotary_dim non-zero, even, <= head_dim; base positive and
   finite; sections non-negative and summing to rotary_dim / 2.  position: 3 values. */
int oq_rope(oq_context* ctx, float* heads_dev, uint64_t n_heads, uint64_t head_dim, uint64_t rotary_dim,
            const int32_t sections[4], float base, const uint64_t position[3]);

/* oracle::runtime::causal_attention_step (src/runtime/reference_kernels.cpp:127-195): appends
   k_dev [kv_heads][key_dim] and v_dev [kv_heads][value_dim] to the cache, then for every query
   head h of q_dev [q_heads][key_dim] (KV head h / (q_heads / kv_heads)) writes to
   out_dev [q_heads][value_dim] the softmax(q . k_t / sqrt(key_dim)) weighted sum of the cached
   values, t over every stored token.  Checks as the reference: dimensions ("causal_attention_step
   dimensions are incompatible", OQ_INVALID_ARGUMENT), then capacity ("KV cache capacity
   exceeded", OQ_OVERFLOW), both before any device work.  F32 arithmetic split over token chunks
   and merged with the usual max rescaling: outputs agree with the reference within 1e-4 of
   sum_t p_t |v_t| (the reference sums doubles for the dot products and the denominator).  A
   non-finite score yields non-finite outputs where the reference throws.  key_dim == value_dim in
   {64, 128, 256} with q_heads / kv_heads <= 256 takes the chunked kernels: up to 8 query heads per
   KV head read each cached row once per step; a larger group runs as equal subgroups of at most 8
   heads (16: two of 8), each reading the group's rows.  Any other shape (key_dim <= 8192; wider
   keys -> OQ_INVALID_ARGUMENT) runs one workgroup per query head in the reference's order (double
   dot products and denominator, F32 value sums in token order), the cached rows read once per
   query head.
   The cache must belong to ctx, and the step is refused while ctx's stream is being captured
   (OQ_INVALID_ARGUMENT; both apply to oq_attention_block_step too). */
int oq_attention_step(oq_context* ctx, const float* q_dev, uint64_t q_heads, const float* k_dev,
                      const float* v_dev, oq_kv_cache* cache, float* out_dev);

/* One Qwen3.5 full-attention decoder block at batch 1, chained on the device.  Replaces
   oracle::runtime::execute_qwen35_attention_block_reference (src/runtime/qwen35_block.cpp:607-756,
   with finish_block :326-352 and execute_mlp :296-324):
     normed = RMSNorm(x) * input_norm
     qfull, k, v = projections of normed        (qfull: per head D query values, D gate values)
     q = rope(RMSNorm_head(query) * q_norm),  k = rope(RMSNorm_head(k) * k_norm)
     pregate = causal attention step of (q, k, v) over the cache (appends k, v)
     gated = pregate * sigmoid(gate);  branch = out_proj(gated);  resid = x + branch
     y = resid + down(SiLU(gate(post)) * up(post)),  post = RMSNorm(resid) * post_norm
   Projections as oq_deltanet_step's.  trace_dev, if not NULL, receives (F32, packed; Q = Hq*D,
   KV = Hkv*D): qfull[2Q] k[KV] v[KV] qcur[Q] kcur[KV] pregate[Q] gate_s[Q] gated[Q] branch[E]
   resid[E] post[E] gate[F] up[F] act[F] ffn[E] -- the reference's trace tensors Qcur_full,
   Kcur_projected, Vcur_projected, Qcur, Kcur, attn_pregate, gate_sigmoid, attn_gated,
   attn_output, attn_residual, attn_post_norm, ffn_gate, ffn_up, ffn_swiglu, ffn_out.
   Checks: dimensions, cache geometry ("Qwen3.5 attention cache dimensions do not match the
   manifest"), the RoPE checks above, weight shapes, capacity -- before any device work. */
typedef struct oq_attention_block {
    uint64_t embedding; /* E */
    uint64_t q_heads;   /* Hq, a multiple of kv_heads */
    uint64_t kv_heads;  /* Hkv */
    uint64_t head_dim;  /* D = key_length = value_length */
    uint64_t ffn;       /* F */
    uint64_t rope_dim;  /* rotary dimension (<= D) */
    int32_t rope_sections[4];
    float rope_base;
    float eps;          /* manifest attention_rms_epsilon */
    const oq_weight *q, *k, *v, *out, *gate, *up, *down;
    /* F32 device vectors: input_norm[E], q_norm[D], k_norm[D], post_norm[E] */
    const float *input_norm, *q_norm, *k_norm, *post_norm;
} oq_attention_block;
int oq_attention_block_step(oq_context* ctx, const oq_attention_block* block, oq_kv_cache* cache,
                            const uint64_t position[3], const float* x_dev, float* y_dev, float* trace_dev);

/* m consecutive tokens through the block: the same results as m oq_attention_block_step calls on
   the rows of x_dev [m][E] in order, token t at positions[3 t .. 3 t + 2] (host array), appending
   m rows to the cache; y_dev [m][E].  Replaces the per-token loop of the reference's multi-token
   evaluation (src/runtime/qwen35_target_multi.cpp:14-25).  The projections stream their weights
   once for all m tokens (m >= 16: the matrix-core path of oq_matmul, with its precision contract;
   below 16: the small-batch integer-dot products).  Every token's heads are prepared in one launch
   with the single step's arithmetic (token t's key and value appended at row size + t, bit for bit
   the single step's), then one attention launch over all tokens, token t attending over every row
   up to its own; its chunks are laid out for the last token, so attention outputs agree with m
   single steps within the attention bound, not bit for bit.  trace_dev,
   if not NULL, receives m traces of oq_attention_block_step's layout, one after the other.
   Checks as oq_attention_block_step, every position, m in 1..65535, and size + m <= capacity
   (OQ_OVERFLOW, "KV cache capacity exceeded"), all before any device work. */
int oq_attention_block_steps(oq_context* ctx, const oq_attention_block* block, oq_kv_cache* cache, uint64_t m,
                             const uint64_t* positions, const float* x_dev, float* y_dev, float* trace_dev);

/* No counterpart in the reference.  oq_deltanet_step for callers that cannot allocate device
   memory (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc):
   same arguments, checks, kernels and results, but it allocates nothing -- the block's
   workspace is a fixed per-GPU device array of oq_deltanet_noalloc_capacity() bytes (4 MiB;
   a hidden-4096, FFN-12288 block needs about 440 KiB), held for the life of the process.  A
   block whose workspace would exceed it gets OQ_INVALID_ARGUMENT.  Every call on one GPU
   shares that array: calls that overlap on one GPU (several streams or threads) race. */
int oq_deltanet_step_noalloc(oq_context* ctx, const oq_deltanet_block* block, float* conv_history_dev,
                             float* state_dev, const float* x_dev, float* y_dev, float* trace_dev);
uint64_t oq_deltanet_noalloc_capacity(void);

/* ------------------------------------------------------------------ timing / graphs */

/* HIP events on the context's stream, for timing the kernels launched there.  They are recorded
   without a system-scope fence (hipEventDisableSystemFence: no cache write-back inside the timed
   interval); oq_timer_stop then synchronizes the stream, so the timed work is complete and visible
   to the host when it returns. */
int oq_timer_start(oq_context* ctx);
int oq_timer_stop(oq_context* ctx, float* elapsed_ms); /* waits for the stop event and the stream */

/* Capture every oq_* launch on ctx between begin and end into a replayable HIP graph.  Run each
   captured call once eagerly first: a call that would have to grow the context's workspace
   during capture fails with OQ_INVALID_ARGUMENT.  A graph keeps the workspace it captured: when
   a later eager call grows it, the old allocation is kept until the context's last graph is
   destroyed.  Destroy a context's graphs before the context.  Refused during any capture of the
   context's stream (this one, or the caller's own hipStreamBeginCapture on oq_context_stream()):
   weight and model uploads, KV cache create / reset / load, workspace growth, and the attention
   steps (oq_attention_step, oq_attention_block_step), whose cache length advances on the host
   when the step is issued -- OQ_INVALID_ARGUMENT. */
int oq_capture_begin(oq_context* ctx);
int oq_capture_end(oq_context* ctx, oq_graph** out);
int oq_graph_launch(oq_context* ctx, oq_graph* g);
void oq_graph_destroy(oq_graph* g);

#ifdef __cplusplus
}
#endif

#endif
