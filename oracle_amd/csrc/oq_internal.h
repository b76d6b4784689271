// Internal interfaces between the C ABI (oq_api.cpp) and the kernel translation units.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

struct oq_context;
struct oq_deltanet_block;

namespace oq {

constexpr int kQK = 256;          // K-quant super-block
constexpr int kQ4KBytes = 144;    // {f16 d, f16 dmin, u8 scales[12], u8 qs[128]}
constexpr int kQ5KBytes = 176;    // {d, dmin, scales[12], qh[32], qs[128]}
constexpr int kQ6KBytes = 210;    // {ql[128], qh[64], i8 sc[16], f16 d}
constexpr int kQ80Bytes = 34;     // {f16 d, i8 qs[32]}
constexpr int kQ8KBytes = 292;    // {f32 d, i8 qs[256], i16 bsums[16]}

// How a weight's rows sit in HBM.  Every row starts at a multiple of `pitch` bytes from
// `base`, and `pitch` is a multiple of 16 so rows can be streamed with 128-bit loads.
//   q4_K       : per-row planes  qs[nsb][128] | hdr[nsb][16]   (hdr = f16 d, f16 dmin, scales[12])
//   q5_K       : per-row planes  qs[nsb][128] | qh[nsb][32] | hdr[nsb][16]
//   q6_K       : per-row planes  ql[nsb][128] | qh[nsb][64] | sc[nsb][16] | d[nsb] (f16)
//   q8_0       : per-row planes  qs[nb][32] | d[nb] (f16)
//   f32/f16/bf16: native
struct DeviceMatrix {
    uint32_t type;
    uint64_t k;      // elements per row (GGUF dimensions[0])
    uint64_t n;      // rows (GGUF dimensions[1])
    uint64_t pitch;  // device bytes per row
    const uint8_t* base;
};

uint64_t device_pitch(uint32_t type, uint64_t k);

struct ArgmaxPart;  // one slice's greedy-token result (below)

// ---- oq_api.cpp
// Launch options (OQ_* environment variables), read once when the first context is created and
// again by oq_reload_options(); never per launch.
enum Knob : int {
    kGemmSplits,  // OQ_GEMM_SPLITS
    kGemmFastDequant,  // OQ_GEMM_FAST_DEQUANT: 1 rounds the q4_K / q5_K / q6_K scales and mins to f16 before the weights (K >= 8192; measurement only, outside the precision contract)
    kGemmWs,  // OQ_GEMM_WS: 1 (default) weights converted in the MFMA waves (q4_K, q5_K), 0 the four-wave kernel (q4_K), 2 converted by the load waves (every type; q6_K always)
    kGemvMaxWg,  // OQ_GEMV_MAX_WG
    kQ80Rows,  // OQ_Q8_0_ROWS
    kGemvWgPerCu,  // OQ_GEMV_WG_PER_CU
    kStreamWgPerCu,  // OQ_STREAM_WG_PER_CU
    kGemvStream,  // OQ_GEMV_STREAM
    kStreamWaves,  // OQ_STREAM_WAVES
    kGemvStreamMt,  // OQ_GEMV_STREAM_MT
    kGemvRows,  // OQ_GEMV_ROWS
    kGemvWaves,  // OQ_GEMV_WAVES
    kGemvRowsMt,  // OQ_GEMV_ROWS_MT
    kBlockStream,  // OQ_BLOCK_STREAM
    kBlockFused,  // OQ_BLOCK_FUSED
    kGemmMfma,  // OQ_GEMM_MFMA
    kFusedQuant,  // OQ_FUSED_QUANT
    kGemmInt8,  // OQ_GEMM_INT8
    kAttnWgPerCu,  // OQ_ATTN_WG_PER_CU
    kAttnMinChunk,  // OQ_ATTN_MIN_CHUNK
    kGemmMinK,  // OQ_GEMM_MIN_K: shortest rows (K) of the matrix-core path (default 4096; measurement only)
    kAttnShareMin,  // OQ_ATTN_SHARE_MIN: cached rows from which a multi-token attention workgroup serves several tokens
    kAnyShape,  // OQ_ANY_SHAPE: 1 runs the delta rule and attention on the any-shape kernels at every shape (testing)
    kKnobCount
};
int knob(Knob k, int fallback);  // the option's value, or fallback when it is unset
void load_knobs();    // (re)reads every OQ_* option from the environment
void ensure_knobs();  // load_knobs() once, unless a table is already in force
int cu_count();                               // compute units of the current device (cached)

// ---- oq_decode.hip
hipError_t launch_relayout(uint32_t type, uint64_t k, uint64_t n, const uint8_t* src,
                           uint8_t* dst, uint64_t pitch, hipStream_t s);
hipError_t launch_dequantize(const DeviceMatrix& w, uint64_t row0, uint64_t nrows, float* out,
                             hipStream_t s);
hipError_t launch_quantize_q8k(const float* x, uint64_t m, uint64_t k, uint8_t* q8k,
                               hipStream_t s);

// ---- oq_gemv_kq.hip  (K-quant weights, m <= 8 activation rows per launch, weights streamed once)
// Q8_K activations given as blocks (q8k) or as F32 (x, quantized by every workgroup into LDS;
// bit-identical to launch_quantize_q8k).
bool gemv_kquant_supported(const DeviceMatrix& w);
// Up to four matrices of one type, K and pitch multiplied by the same activation rows in one launch
// of the small-batch kernel: their rows concatenated (matrix i holds rows [row_end[i - 1],
// row_end[i])), matrix i's outputs at y[i][mi * rows_i + local row].  nmat == 0: a single matrix.
// The Gated DeltaNet in-projection's epilogue over several tokens (conv_gates_tokens_kernel's
// results): matrix 0's rows are the channels of the causal convolution (history [C][kernel],
// weights, outputs [tokens][C]), matrix 2's rows the beta gates (beta_s [tokens][Hv]), matrix 3's
// the alpha gates (log_decay [tokens][Hv], with dt_bias and decay)
struct MtConv {
    const float* conv_w;
    float* history;
    float* conv_out;
    uint32_t kernel;
    float *beta_s, *log_decay;
    const float *dt_bias, *decay;
};
constexpr uint32_t kMtConvTaps = 16;  // the longest convolution the epilogue takes
// RMSNorm of the activation rows in the small-batch kernel's staging (rmsnorm_kernel's values):
// rows x [+ b] (F32, K each), weights w; workgroup 0 stores x + b to sum_out and the normalised
// rows to norm_out when given
struct MtNorm {
    const float *b, *w;
    float eps;
    float *sum_out, *norm_out;
};
constexpr int kMtNormBlocks = 4;  // 256-blocks per wave the normalising staging holds (2 rows of 8192)
struct MtSet {
    const uint8_t* base[4];
    float* y[4];
    const float* add[4];  // null, or rows laid out like y's: y = add + the product
    uint32_t row_end[4];
    uint32_t nmat;
    MtConv conv;          // conv.conv_w null: no epilogue
    MtNorm norm;          // norm.w null: the activations are Q8_K blocks
};
// mats[0 .. nmat) from m (2 .. 15) rows of Q8_K blocks, in one launch per 8 activation rows:
// hipErrorNotSupported when the streamed small-batch kernel does not apply (the caller multiplies
// the matrices one by one; each row's bits are the same either way).  With adds, matrix i's
// outputs are adds[i] + its product (adds[i] null: the product), each sum rounded once.
// With conv (nmat 4: q/k/v channels, z, beta, alpha) the launches also run the DeltaNet epilogue
// over the m tokens in order, or nothing is launched (hipErrorNotSupported: a convolution longer
// than kMtConvTaps, or a wave with 64 rows or more).
hipError_t launch_gemv_kquant_set(const DeviceMatrix* mats, uint32_t nmat, int m, const uint8_t* q8k, float* const* ys,
                                  hipStream_t s, const float* const* adds = nullptr, const MtConv* conv = nullptr);
// The same from two F32 rows x [+ norm.b] normalised in the kernel's staging (one launch, K <=
// 8192), or hipErrorNotSupported with nothing launched
hipError_t launch_gemv_kquant_set_norm(const DeviceMatrix* mats, uint32_t nmat, int m, const float* x, const MtNorm& norm,
                                       float* const* ys, hipStream_t s, const MtConv* conv = nullptr);
hipError_t launch_gemv_kquant(const DeviceMatrix& w, int m, const float* x, const uint8_t* q8k,
                              float* y, hipStream_t s);
int gemv_max_m();
// passes per launch of the windowed long-row kernel for m activation rows (0: the row fits the
// compile-time kernels)
uint32_t gemv_window_passes(const DeviceMatrix& w, int m);
// m = 1 decode GEMV that also reduces its outputs to one greedy-token partial per workgroup
// (parts[0..*nparts)); hipErrorNotSupported when the row does not fit the streamed kernel or the
// grid would exceed max_parts workgroups
hipError_t launch_gemv_kquant_argmax(const DeviceMatrix& w, const float* x, const uint8_t* q8k, float* y,
                                     ArgmaxPart* parts, uint32_t max_parts, uint32_t* nparts, hipStream_t s);

// ---- oq_gemv_inst.hip  (one instantiation set per weight type and activation form)
template <uint32_t TYPE, bool FUSED>
hipError_t launch_kq(const DeviceMatrix& w, int m, const float* x, const uint8_t* q8k, float* y, hipStream_t s);
template <uint32_t TYPE, bool FUSED>
hipError_t launch_kq_argmax(const DeviceMatrix& w, const float* x, const uint8_t* q8k, float* y, ArgmaxPart* parts,
                            uint32_t max_parts, uint32_t* nparts, hipStream_t s);
template <uint32_t TYPE, bool FUSED>
hipError_t launch_kq_window(const DeviceMatrix& w, int m, const float* x, const uint8_t* q8k, float* y,
                            uint32_t pass0, uint32_t npass, int accumulate, hipStream_t s);

// ---- oq_gemv.hip  (q8_0 / f32 / f16 / bf16 weights against F32 activations)
hipError_t launch_gemv_f32act(const DeviceMatrix& w, int m, const float* x, float* y,
                              hipStream_t s);

// greedy token: first index of the maximum of logits[0..n) (n >= 1), its value; 0xFFFFFFFF on NaN.
// partials: kArgmaxParts ArgmaxPart of device memory (per-slice results; no initial contents)
struct ArgmaxPart {
    float value;
    uint32_t index;  // 0xFFFFFFFF: no element
    uint32_t nan;
};
constexpr uint32_t kArgmaxParts = 1024;
hipError_t launch_argmax(const float* logits, uint64_t n, uint32_t* token, float* value, void* partials,
                         hipStream_t s);
// the combination of nparts slice results (from launch_argmax's first kernel or a GEMV epilogue)
hipError_t launch_argmax_final(const ArgmaxPart* parts, uint32_t nparts, uint32_t* token, float* value,
                               hipStream_t s);

// ---- oq_gemm.hip  (m >= 16, q4_K / q5_K / q6_K, K >= 4096: F16 matrix cores on F16-rounded operands)
// Activations are given either as F32 (x; quantized to Q8_K inside, bit-identical to
// launch_quantize_q8k) or as Q8_K blocks (q8k); exactly one of the two is non-null.
bool gemm_mfma_supported(const DeviceMatrix& w, int m);
uint64_t gemm_scratch_bytes(const DeviceMatrix& w, int m);  // planar Q8_K image + split partials
hipError_t launch_gemm_mfma(const DeviceMatrix& w, int m, const float* x, const uint8_t* q8k, float* y,
                                void* scratch, hipStream_t s);

// ---- oq_gemm_i8.hip  (m >= 16, q4_K: int8 matrix cores on Q8_K x nibbles, per-sub-block integer
// rescale; the alternative to the f16 kernel, selected with OQ_GEMM_INT8=1)
bool gemm_i8_supported(const DeviceMatrix& w, int m);
uint64_t gemm_i8_scratch_bytes(const DeviceMatrix& w, int m);  // int8 image, scales, f16 partial sums
hipError_t launch_gemm_q4k_i8(const DeviceMatrix& w, int m, const float* x, const uint8_t* q8k, float* y,
                              void* scratch, hipStream_t s);

// ---- oq_deltanet.hip  (Gated DeltaNet decode block: kernels between the projections)
// the shapes of the fused block launches and the register-resident delta rule; every other shape
// takes the per-stage launches with the any-shape delta rule (deltanet_dims_any)
bool deltanet_dims_supported(uint64_t key_dim, uint64_t value_dim, uint64_t conv_kernel);
constexpr uint64_t kDeltaMaxKeyDim = 4096;  // the any-shape delta rule's normalised q / k in LDS
bool deltanet_dims_any(uint64_t key_dim, uint64_t value_dim, uint64_t conv_kernel);
// rows consecutive rows of n values (one workgroup each)
// q8, when not null, also receives the rows' Q8_K blocks (n a multiple of 256)
hipError_t launch_rmsnorm(const float* a, const float* b, const float* w, uint64_t n, float eps, float* sum_out,
                          float* out, hipStream_t s, uint64_t rows = 1, uint8_t* q8 = nullptr);
hipError_t launch_conv_gates(const float* qkv, const float* conv_w, float* history, uint64_t channels,
                             uint64_t kernel, const float* beta, const float* alpha, const float* dt_bias,
                             const float* decay, uint64_t heads, float* conv_out, float* beta_s, float* log_decay,
                             hipStream_t s);
// tokens consecutive tokens: qkv / conv_out [tokens][channels], beta / alpha / beta_s / log_decay [tokens][heads]
hipError_t launch_conv_gates_tokens(const float* qkv, const float* conv_w, float* history, uint64_t channels,
                                    uint64_t kernel, const float* beta, const float* alpha, const float* dt_bias,
                                    const float* decay, uint64_t heads, uint64_t tokens, float* conv_out,
                                    float* beta_s, float* log_decay, hipStream_t s);
// the delta rule over Hv * ceil(dv/32) workgroups: rec_out[Hv][dv] and head_ss[Hv][delta_chunks(dv)], the
// per-chunk double sums of rec_out^2 that the head's gated RMSNorm takes (launch_gated_norm, or the out
// projection's staging).  Key widths 32, 64, 128 with dv a multiple of 32 keep the state in registers; any
// other shape (or OQ_ANY_SHAPE=1) runs the any-shape kernel.
// z / z_silu: when not null (register-resident shapes only), the launch also stores SiLU(z) of the
// block's gate row (the value heads' columns, [Hv][dv]) for the out projection's staging
hipError_t launch_delta(const float* conv, uint64_t key_heads, uint64_t value_heads, uint64_t dk, uint64_t dv,
                        const float* beta_s, const float* log_decay, float eps, float* state, float* rec_out,
                        double* head_ss, const float* z, float* z_silu, hipStream_t s, uint64_t tokens = 1);
// q8, when not null, also receives each token's gated row as Q8_K blocks (heads * dv a multiple of 256)
hipError_t launch_gated_norm(const float* rec, const double* head_ss, const float* z, const float* out_norm,
                             uint64_t heads, uint64_t dv, float eps, float* gated, hipStream_t s, uint64_t tokens = 1,
                             uint8_t* q8 = nullptr);
uint64_t delta_chunks(uint64_t dv);  // head_ss entries per head
// q8, when not null, also receives act's Q8_K blocks (n a multiple of 256)
hipError_t launch_swiglu(const float* gate, const float* up, uint64_t n, float* act, hipStream_t s, uint8_t* q8 = nullptr);
hipError_t launch_add(const float* a, const float* b, uint64_t n, float* out, hipStream_t s);

// ---- oq_attention.hip  (full-attention decode: RoPE, the block's head preparation, attention)
struct RopeParams {
    uint32_t rotary_dim, sec1, sec2;  // sections[1] (height) and sections[2] (width)
    float base;
    uint64_t pos[3];  // temporal, height, width
};
// cos and sin of each frequency's angle at one position, computed on the host exactly as
// apply_qwen35_rope does (reference_kernels.cpp:105-115: double pow, cos and sin of the host's
// libm, rounded to F32), so a single-position rotation uses the reference's own values; pairs = 0
// when absent (rotary_dim / 2 above kRopeTablePairs, or positions that differ per token): then the
// device computes them in double (rope_cs)
constexpr uint32_t kRopeTablePairs = 128;
struct RopeTable {
    uint32_t pairs;
    float cs[2][kRopeTablePairs];
};
void rope_table(const RopeParams& p, RopeTable& t);
// The decoder block's per-head preparation (qwen35_block.cpp:671-711), done by the attention
// chunk kernel: RMSNorm of the query heads (q_norm) and of the new key (k_norm), rotation, the
// append of the new key and value rows, and the trace's copies qcur / kcur.
struct AttnPrep {
    const float *qfull, *kp, *vp;  // projections: [Hq][2D], [Hkv][D], [Hkv][D]
    const float *q_norm, *k_norm;
    float eps;
    RopeParams rope;
    RopeTable table;              // the any-shape preparation's cos / sin at rope.pos (pairs = 0: computed on the device)
    float *qcur, *kcur;           // [Hq][D], [Hkv][D], or null (not stored)
    bool v_stored;                // an F16 cache's new value row already stored (by the projection)
};
struct AttnLaunch {
    const float* q;            // [Hkv * rep][D]
    void* keys;                // cache [capacity][Hkv][D] of F32, or of binary16 when f16
    void* values;
    bool f16;
    const float* new_k;        // token T-1's key/value rows [Hkv][D], stored into the cache; or null
    const float* new_v;        //   when the cache already holds them
    uint32_t T, Hkv, rep, D, chunk, nchunks;
    float scale;               // 1 / sqrt(D)
    float* part;               // attention_partial_floats(Hkv, rep, D, nchunks) floats
    float* out;                // [Hkv * rep][D]; with a gate, may be null (not stored)
    const float* gate;         // raw output gate of head h at gate + h * gate_stride, or null
    uint32_t gate_stride;
    float* gate_s;             // sigmoid(gate) [Hq][D] (or null: not stored) and out * sigmoid(gate), when gate is given
    float* gated;
    const AttnPrep* prep;      // or null; when given, q and new_k / new_v are not read
    // the any-shape kernels (widths outside {64, 128, 256}, key width != value width, or
    // OQ_ANY_SHAPE=1): D is the key width, Dv the value width (out / gate_s / gated rows of Dv),
    // chunk / nchunks unused, part holds attention_any_floats(Hkv * rep, T) floats; with a prep,
    // prep->qcur must be given (the rotated queries the attention reads)
    bool any;
    uint32_t Dv;
};
constexpr uint64_t kAttnMaxRep = 256;  // query heads per KV head
bool attention_dims_supported(uint64_t head_dim, uint64_t rep);
constexpr uint64_t kAttnAnyMaxDim = 8192;  // the any-shape kernels' widest key / head row (LDS)
uint64_t attention_any_floats(uint64_t q_heads, uint64_t T);
uint32_t attention_subgroups(uint32_t rep);  // chunk workgroups per (KV head, chunk): rep / subgroups <= 8 heads each
// token_groups: launches of that many tokens' workgroups share the grid (several tokens per call)
void attention_plan(uint64_t T, uint64_t Hkv, uint64_t rep, uint32_t& chunk, uint32_t& nchunks,
                    uint64_t token_groups = 1);
// tokens each chunk workgroup of a several-token launch serves (over long caches, as many as its 8
// query rows hold; otherwise one)
uint32_t attention_tokens_per_workgroup(uint64_t T, uint64_t rep, uint64_t tokens);
uint64_t attention_partial_floats(uint64_t Hkv, uint64_t rep, uint64_t head_dim, uint32_t nchunks);
constexpr uint32_t kAttnMaxChunks = 8192;
hipError_t launch_attention(const AttnLaunch& a, hipStream_t s);
// Several consecutive tokens of the decoder block (L shaped for the last token: T = its rows, the
// partials `tokens` times attention_partial_floats(...) floats, out / gate / gate_s / gated for
// token 0).  Three launches: the per-head preparation of every token (queries to qcur, keys and
// values into cache rows T - tokens .. T - 1, kcur when given), one chunk launch and one merge
// launch over all tokens; token i attends over the rows up to its own.
struct AttnTokens {
    uint32_t tokens;
    const float *qfull, *kp, *vp;  // [tokens][Hq][2D], [tokens][Hkv][D], [tokens][Hkv][D]
    const float *q_norm, *k_norm;
    float eps;
    RopeParams rope;               // rotary_dim, sections and base (positions from `positions`)
    const uint64_t* positions;     // device [tokens][3]; or null with positions_host and at most
    const uint64_t* positions_host;  // kInlineTokenPositions tokens: passed as launch arguments
    float* qcur;                   // [tokens][Hq][D]: the prepared queries
    float* kcur;                   // [tokens][Hkv][D] or null
    uint64_t gate_tok_stride;      // floats between the tokens' output gates
};
constexpr uint32_t kInlineTokenPositions = 32;
hipError_t launch_attention_tokens(const AttnLaunch& L, const AttnTokens& tk, hipStream_t s);
hipError_t launch_f32_to_f16(const float* src, void* dst, uint64_t n, hipStream_t s);  // round to nearest even
hipError_t launch_rope(float* heads, uint64_t n_heads, uint64_t head_dim, const RopeParams& p, const RopeTable& t,
                       hipStream_t s);

// ---- oq_gemv_block.hip  (fused m = 1 GEMV of the DeltaNet decode block; see the kernel comment)
enum : int { kBlockIn = 0, kBlockAdd = 1, kBlockFfn = 2 };
struct BlockGemv {
    DeviceMatrix mat[4];   // same type, K and pitch
    uint32_t row_end[4];   // IN / ADD: cumulative row counts of mat[0..nmat)
    uint32_t nmat;
    const float* x;        // F32 activation, K values
    const float* norm_w;   // RMSNorm weight (K values) or null
    float eps;
    float* norm_out;       // the normalised activation (written by workgroup 0) or null
    float* raw[4];         // per-matrix outputs (or null: not stored; the attention block's IN needs them)
    _Float16* v16;         // IN: when not null, matrix 2's outputs also stored rounded to binary16 here
                           // (the new value row of an F16 KV cache)
    const float* conv_w;   // IN: convolution taps [rows of mat[0]][conv_kernel]
    float* history;        // IN: convolution history, same shape, updated in place
    uint32_t conv_kernel;
    float* conv_out;       // IN: SiLU(conv) per channel of mat[0]
    const float* dt_bias;  // IN: per row of mat[3]
    const float* decay;
    float* beta_s;         // IN: sigmoid of mat[2]'s outputs
    float* log_decay;      // IN: softplus(mat[3] + dt_bias) * decay
    const float* add;      // ADD: sum_out = add + y
    float* sum_out;
    float* act;            // FFN: SiLU(gate) * up
    // ADD, streamed: when rec is not null the activation is the recurrent block's gated output,
    // formed in the staging from the delta rule's output: x = RMSNorm_head(rec) * out_norm *
    // SiLU(z) with each head's sum of squares from head_ss[h * dchunks ...] (eps as above) and
    // z_silu = SiLU(z) as the delta rule's launch stores it; workgroup 0 stores x to gated_out
    const float* rec;
    const double* head_ss;
    const float* z;        // SiLU(z), [Hv][dv]
    const float* out_norm;
    uint32_t dv, dchunks;
    float* gated_out;
};
bool gemv_block_supported(const BlockGemv& a);
// whether launch_gemv_block(kBlockAdd, a) runs the streamed kernel (the one that can form the
// gated activation itself)
bool gemv_block_add_streams(const BlockGemv& a);
// whether launch_gemv_block(kBlockIn, a) runs the streamed kernel (normalised, raw outputs only)
bool gemv_block_in_streams(const BlockGemv& a);
hipError_t launch_gemv_block(int mode, const BlockGemv& a, hipStream_t s);

// ---- oq_api.cpp: the block step on a caller-provided workspace (validation, capacity check, launches)
int deltanet_step_into(oq_context* ctx, const oq_deltanet_block* b, float* hist, float* state, const float* x,
                       float* y, float* trace, float* ws, uint64_t ws_bytes);
int context_device(const oq_context* ctx);
int set_error(oq_context* ctx, int code, const char* msg);

// ---- oq_noalloc.hip: the allocation-free entry point's per-device workspace
void noalloc_setup(int device);  // device must be current; once per device

}  // namespace oq
