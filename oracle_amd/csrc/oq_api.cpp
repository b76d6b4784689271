// C ABI of liboq.so (declared in include/oq.h): contexts, one-time weight upload, argument
// validation with the reference's error kinds, and dispatch to the gfx950 kernels.
//
// Validation mirrors what the reference checks before it writes anything
// (src/backend/cpu/quantized_reference.cpp:134-153, src/model/ggml_type.cpp:77-94,
// src/model/storage_decode.cpp:182-198): the first failing check decides the status.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <cmath>
#include <algorithm>
#include <atomic>
#include <initializer_list>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/oq.h"
#include "oq_internal.h"
#include "oq_workspace.h"

namespace oq {

namespace {

constexpr const char* kKnobNames[kKnobCount] = {
    "OQ_GEMM_SPLITS",   "OQ_GEMM_FAST_DEQUANT",  "OQ_GEMM_WS",     "OQ_GEMV_MAX_WG",   "OQ_Q8_0_ROWS",
    "OQ_GEMV_WG_PER_CU", "OQ_STREAM_WG_PER_CU",  "OQ_GEMV_STREAM", "OQ_STREAM_WAVES",  "OQ_GEMV_STREAM_MT",
    "OQ_GEMV_ROWS",     "OQ_GEMV_WAVES",         "OQ_GEMV_ROWS_MT", "OQ_BLOCK_STREAM", "OQ_BLOCK_FUSED",
    "OQ_GEMM_MFMA",     "OQ_FUSED_QUANT",        "OQ_GEMM_INT8",   "OQ_ATTN_WG_PER_CU", "OQ_ATTN_MIN_CHUNK",
    "OQ_GEMM_MIN_K",    "OQ_ATTN_SHARE_MIN",     "OQ_ANY_SHAPE",
};

struct KnobTable {
    int value[kKnobCount] = {};
    bool set[kKnobCount] = {};
};
// The table in force is published through an atomic pointer, so a launch on one thread may read
// it while another thread creates a context or reloads the options.  Replaced tables are kept
// (a reader may still hold one) and freed at exit.
std::atomic<const KnobTable*> g_knobs{nullptr};
std::mutex g_knob_mutex;
std::vector<std::unique_ptr<KnobTable>> g_knob_tables;

}  // namespace

void load_knobs() {
    auto t = std::make_unique<KnobTable>();
    for (int i = 0; i < kKnobCount; ++i) {
        const char* v = getenv(kKnobNames[i]);
        t->set[i] = v != nullptr;
        t->value[i] = v ? atoi(v) : 0;
    }
    std::lock_guard<std::mutex> lock(g_knob_mutex);
    g_knobs.store(t.get(), std::memory_order_release);
    g_knob_tables.push_back(std::move(t));
}

void ensure_knobs() {
    if (g_knobs.load(std::memory_order_acquire) != nullptr) return;
    {
        std::lock_guard<std::mutex> lock(g_knob_mutex);
        if (g_knobs.load(std::memory_order_relaxed) != nullptr) return;
    }
    load_knobs();
}

int knob(Knob k, int fallback) {
    const KnobTable* t = g_knobs.load(std::memory_order_acquire);
    return (t && t->set[k]) ? t->value[k] : fallback;
}

int cu_count() {
    static std::atomic<int> cus{0};
    int v = cus.load(std::memory_order_relaxed);
    if (v == 0) {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0) {
            v = 256;
        }
        cus.store(v, std::memory_order_relaxed);
    }
    return v;
}

}  // namespace oq

struct oq_context {
    int device = 0;
    hipStream_t stream = nullptr;
    hipEvent_t t0 = nullptr, t1 = nullptr;
    std::string error;
    bool capturing = false;
    oq::Workspace scratch;  // Q8_K staging (small batches) or the GEMM's activation image + split partials
    oq::Workspace work;     // intermediates of the DeltaNet block step
    void* argmax_parts = nullptr;  // per-slice results of oq_argmax (kArgmaxParts ArgmaxPart)
    std::vector<oq_graph*> graphs;  // live graphs captured on this context
};

struct oq_weight {
    oq::DeviceMatrix m{};
    void* owned = nullptr;
    uint64_t device_bytes = 0;
    int device = 0;
};

struct oq_graph {
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    oq_context* ctx = nullptr;  // the context it was captured on (null once that is destroyed)
};

namespace {

thread_local std::string g_error;

struct Layout {
    const char* name;
    uint32_t block_elements;
    uint32_t bytes_per_block;
    int quantized;
};

// GGML on-disk layouts by type id (the reference keeps the same table, src/model/ggml_type.cpp
// :12-54; ids with zero geometry are deprecated or removed and count as unregistered).
constexpr Layout kLayouts[] = {
    {"f32", 1, 4, 0},          {"f16", 1, 2, 0},           {"q4_0", 32, 18, 1},
    {"q4_1", 32, 20, 1},       {"deprecated_q4_2", 0, 0, 0}, {"deprecated_q4_3", 0, 0, 0},
    {"q5_0", 32, 22, 1},       {"q5_1", 32, 24, 1},        {"q8_0", 32, 34, 1},
    {"q8_1", 32, 36, 1},       {"q2_K", 256, 84, 1},       {"q3_K", 256, 110, 1},
    {"q4_K", 256, 144, 1},     {"q5_K", 256, 176, 1},      {"q6_K", 256, 210, 1},
    {"q8_K", 256, 292, 1},     {"iq2_xxs", 256, 66, 1},    {"iq2_xs", 256, 74, 1},
    {"iq3_xxs", 256, 98, 1},   {"iq1_s", 256, 50, 1},      {"iq4_nl", 32, 18, 1},
    {"iq3_s", 256, 110, 1},    {"iq2_s", 256, 82, 1},      {"iq4_xs", 256, 136, 1},
    {"i8", 1, 1, 0},           {"i16", 1, 2, 0},           {"i32", 1, 4, 0},
    {"i64", 1, 8, 0},          {"f64", 1, 8, 0},           {"iq1_m", 256, 56, 1},
    {"bf16", 1, 2, 0},         {"removed_q4_0_4_4", 0, 0, 0}, {"removed_q4_0_4_8", 0, 0, 0},
    {"removed_q4_0_8_8", 0, 0, 0}, {"tq1_0", 256, 54, 1},  {"tq2_0", 256, 66, 1},
    {"removed_iq4_nl_4_4", 0, 0, 0}, {"removed_iq4_nl_4_8", 0, 0, 0},
    {"removed_iq4_nl_8_8", 0, 0, 0}, {"mxfp4", 32, 17, 1}, {"nvfp4", 64, 36, 1},
    {"q1_0", 128, 18, 1},      {"q2_0", 64, 18, 1},
};
constexpr uint32_t kLayoutCount = sizeof(kLayouts) / sizeof(kLayouts[0]);

const Layout* layout_of(uint32_t type) {
    if (type >= kLayoutCount) return nullptr;
    const Layout& l = kLayouts[type];
    return (l.block_elements == 0 || l.bytes_per_block == 0) ? nullptr : &l;
}

bool is_kquant(uint32_t t) { return t == OQ_TYPE_Q4_K || t == OQ_TYPE_Q5_K || t == OQ_TYPE_Q6_K; }

int fail(oq_context* ctx, int code, const std::string& msg) {
    if (ctx) ctx->error = msg;
    else g_error = msg;
    return code;
}

int hip_fail(oq_context* ctx, hipError_t e, const char* what) {
    const int code = e == hipErrorOutOfMemory ? OQ_OUT_OF_MEMORY : OQ_DEVICE_ERROR;
    return fail(ctx, code, std::string(what) + ": " + hipGetErrorString(e));
}

#define OQ_HIP(ctx, expr, what)                         \
    do {                                                \
        hipError_t e_ = (expr);                         \
        if (e_ != hipSuccess) return hip_fail(ctx, e_, what); \
    } while (0)

// ggml_row_byte_size (src/model/ggml_type.cpp:77-94)
int row_bytes(oq_context* ctx, uint64_t k, uint32_t type, uint64_t* out) {
    const Layout* l = layout_of(type);
    if (!l) return fail(ctx, OQ_UNSUPPORTED_TYPE, "unsupported GGML tensor type: " + std::to_string(type));
    if (k == 0) return fail(ctx, OQ_INVALID_ARGUMENT, "GGML tensor row must contain at least one element");
    if (k % l->block_elements != 0) {
        return fail(ctx, OQ_UNSUPPORTED_TYPE,
                    "GGML tensor row length " + std::to_string(k) + " is not divisible by block size " +
                        std::to_string(l->block_elements) + " for type " + l->name);
    }
    const uint64_t blocks = k / l->block_elements;
    if (blocks != 0 && l->bytes_per_block > UINT64_MAX / blocks) {
        return fail(ctx, OQ_OVERFLOW, "GGML row byte size overflow");
    }
    *out = blocks * l->bytes_per_block;
    return OQ_OK;
}

bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

int check_weight(oq_context* ctx, const oq_weight* w) {
    if (!w || !w->m.base) return fail(ctx, OQ_INVALID_ARGUMENT, "null weight");
    if (w->device != ctx->device) return fail(ctx, OQ_INVALID_ARGUMENT, "weight lives on another device");
    return OQ_OK;
}

void device_free(void* p) { (void)hipFree(p); }

// The context's stream is being captured, by oq_capture_begin or by the caller's own
// hipStreamBeginCapture on oq_context_stream().
bool capturing_now(oq_context* ctx) {
    hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
    const hipError_t e = hipStreamIsCapturing(ctx->stream, &st);
    oq::StreamCapture q = oq::StreamCapture::kNone;
    if (e != hipSuccess) q = oq::StreamCapture::kQueryFailed;
    else if (st == hipStreamCaptureStatusActive) q = oq::StreamCapture::kActive;
    else if (st == hipStreamCaptureStatusInvalidated) q = oq::StreamCapture::kInvalidated;
    return oq::capture_in_progress(ctx->capturing, q);
}

// Grows a context workspace; allocations that a live graph may still replay are kept until the
// context's last graph is destroyed (oq_workspace.h).
int ensure_workspace(oq_context* ctx, oq::Workspace& ws, uint64_t bytes, const char* what) {
    if (ws.bytes >= bytes) return OQ_OK;
    hipError_t err = hipSuccess;
    const oq::GrowResult r = ws.ensure(
        bytes, capturing_now(ctx), (int)ctx->graphs.size(),
        [&](uint64_t n) -> void* {
            void* p = nullptr;
            err = hipMalloc(&p, n);
            return err == hipSuccess ? p : nullptr;
        },
        device_free, [&] { return (err = hipStreamSynchronize(ctx->stream)) == hipSuccess; });
    switch (r) {
        case oq::GrowResult::kOk: return OQ_OK;
        case oq::GrowResult::kCapturing:
            return fail(ctx, OQ_INVALID_ARGUMENT,
                        std::string(what) + " must be sized before graph capture (run the call once first)");
        default: return hip_fail(ctx, err, what);
    }
}

int ensure_scratch(oq_context* ctx, uint64_t bytes) {
    return ensure_workspace(ctx, ctx->scratch, bytes, "activation staging buffer");
}

int ensure_work(oq_context* ctx, uint64_t bytes) { return ensure_workspace(ctx, ctx->work, bytes, "block workspace"); }

bool knob_flag(oq::Knob k, bool fallback) { return oq::knob(k, fallback ? 1 : 0) != 0; }

int upload_common(oq_context* ctx, uint32_t type, uint64_t ne0, uint64_t ne1, const void* bytes,
                  uint64_t nbytes, bool from_device, oq_weight** out) {
    if (!ctx) return fail(nullptr, OQ_INVALID_ARGUMENT, "null context");
    if (!out) return fail(ctx, OQ_INVALID_ARGUMENT, "null output handle");
    *out = nullptr;
    if (ne0 == 0 || ne1 == 0) return fail(ctx, OQ_INVALID_ARGUMENT, "reference matvec dimensions must be non-zero");
    uint64_t rb = 0;
    if (int rc = row_bytes(ctx, ne0, type, &rb)) return rc;
    if (rb > UINT64_MAX / ne1) return fail(ctx, OQ_OVERFLOW, "reference matvec matrix size overflow");
    if (nbytes != rb * ne1) return fail(ctx, OQ_INVALID_ARGUMENT, "reference matvec matrix byte size mismatch");
    if (!oq_type_supported(type)) {
        return fail(ctx, OQ_INVALID_ARGUMENT, "storage decoder does not support GGML type " + std::to_string(type));
    }
    if (!bytes) return fail(ctx, OQ_INVALID_ARGUMENT, "null tensor bytes");
    if (capturing_now(ctx)) return fail(ctx, OQ_INVALID_ARGUMENT, "weights cannot be uploaded during graph capture");

    const uint64_t pitch = oq::device_pitch(type, ne0);
    if (pitch != 0 && ne1 > UINT64_MAX / pitch) return fail(ctx, OQ_OVERFLOW, "device matrix size overflow");
    const uint64_t dbytes = pitch * ne1;
    OQ_HIP(ctx, hipSetDevice(ctx->device), "hipSetDevice");
    void* dst = nullptr;
    OQ_HIP(ctx, hipMalloc(&dst, dbytes), "hipMalloc(weight)");
    auto cleanup = [&](int rc) {
        (void)hipFree(dst);
        return rc;
    };
    const bool identity = pitch == rb && (type == OQ_TYPE_F32 || type == OQ_TYPE_F16 || type == OQ_TYPE_BF16);
    hipError_t e = hipSuccess;
    if (identity) {
        e = hipMemcpyAsync(dst, bytes, nbytes, from_device ? hipMemcpyDeviceToDevice : hipMemcpyHostToDevice,
                           ctx->stream);
    } else {
        const void* src = bytes;
        void* staging = nullptr;
        // the relayout reads 16-byte pieces of q4_K / q5_K blocks: device sources off that
        // alignment are copied to an aligned buffer first
        if (!from_device || !aligned(bytes, 16)) {
            e = hipMalloc(&staging, nbytes);
            if (e == hipSuccess)
                e = hipMemcpyAsync(staging, bytes, nbytes, from_device ? hipMemcpyDeviceToDevice : hipMemcpyHostToDevice,
                                   ctx->stream);
            src = staging;
        }
        if (e == hipSuccess && dbytes != nbytes) e = hipMemsetAsync(dst, 0, dbytes, ctx->stream);
        if (e == hipSuccess)
            e = oq::launch_relayout(type, ne0, ne1, static_cast<const uint8_t*>(src),
                                    static_cast<uint8_t*>(dst), pitch, ctx->stream);
        if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
        if (staging) (void)hipFree(staging);
    }
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) return cleanup(hip_fail(ctx, e, "weight upload"));
    oq_weight* w = new oq_weight;
    w->m.type = type;
    w->m.k = ne0;
    w->m.n = ne1;
    w->m.pitch = pitch;
    w->m.base = static_cast<const uint8_t*>(dst);
    w->owned = dst;
    w->device_bytes = dbytes;
    w->device = ctx->device;
    *out = w;
    return OQ_OK;
}

int launch_rc(oq_context* ctx, hipError_t e, const char* what) {
    return e == hipSuccess ? OQ_OK : hip_fail(ctx, e, what);
}

// One projection of the DeltaNet block (batch 1): the matvec path of oq_matvec with the F32
// activation quantized inside the K-quant GEMV.
hipError_t block_project(const oq_weight* w, const float* x, float* y, hipStream_t s) {
    if (is_kquant(w->m.type)) return oq::launch_gemv_kquant(w->m, 1, x, nullptr, y, s);
    return oq::launch_gemv_f32act(w->m, 1, x, y, s);
}

int check_block_weight(oq_context* ctx, const oq_weight* w, uint64_t ne0, uint64_t ne1, const char* name) {
    if (int rc = check_weight(ctx, w)) return fail(ctx, rc, std::string("DeltaNet block weight ") + name + ": " + ctx->error);
    if (w->m.k != ne0 || w->m.n != ne1) {
        return fail(ctx, OQ_INVALID_ARGUMENT,
                    std::string("DeltaNet block weight ") + name + " has shape [" + std::to_string(w->m.k) + ", " +
                        std::to_string(w->m.n) + "], expected [" + std::to_string(ne0) + ", " + std::to_string(ne1) + "]");
    }
    return OQ_OK;
}

// Workspace of one block step: the trace fields, then beta_s, log_decay, the normalised input, the
// delta rule's per-chunk sums of squares and SiLU(z), each padded to 64 floats so every projection
// input is 256-byte aligned.
struct BlockLayout {
    uint64_t sizes[19];
    uint64_t off[19];
    uint64_t total_floats;
};

BlockLayout block_layout(const oq_deltanet_block* b) {
    const uint64_t E = b->embedding, Hk = b->key_heads, Hv = b->value_heads, dk = b->key_dim, dv = b->value_dim,
                   F = b->ffn;
    const uint64_t V = Hv * dv, C = 2 * Hk * dk + V;
    // the last field: the delta rule's per-chunk double sums of squares (2 floats each)
    BlockLayout l{{C, V, Hv, Hv, C, V, V, E, E, E, F, F, F, E, Hv, Hv, E, 2 * Hv * oq::delta_chunks(dv), V}, {}, 0};
    for (int i = 0; i < 19; ++i) {
        l.off[i] = l.total_floats;
        l.total_floats += (l.sizes[i] + 63) & ~uint64_t(63);
    }
    return l;
}

// The block step's checks and launches.  ws: caller-provided workspace of ws_bytes, or null to
// use (and grow) the context's own.
int deltanet_step(oq_context* ctx, const oq_deltanet_block* b, float* hist, float* state, const float* x, float* y,
                  float* trace, float* ext_ws, uint64_t ext_ws_bytes) {
    if (!ctx) return fail(nullptr, OQ_INVALID_ARGUMENT, "null context");
    if (!b || !hist || !state || !x || !y) return fail(ctx, OQ_INVALID_ARGUMENT, "null argument");
    const uint64_t E = b->embedding, Hk = b->key_heads, Hv = b->value_heads, dk = b->key_dim, dv = b->value_dim,
                   K = b->conv_kernel, F = b->ffn;
    if (E == 0 || Hk == 0 || Hv == 0 || dk == 0 || dv == 0 || K == 0 || F == 0 || Hv % Hk != 0) {
        return fail(ctx, OQ_INVALID_ARGUMENT, "Qwen3.5 recurrent block dimensions are incompatible");
    }
    if (!(b->eps > 0.0f) || !std::isfinite(b->eps)) {
        return fail(ctx, OQ_INVALID_ARGUMENT, "Qwen3.5 RMSNorm epsilon must be positive and finite");
    }
    if (!oq::deltanet_dims_any(dk, dv, K)) {
        return fail(ctx, OQ_INVALID_ARGUMENT, "DeltaNet block device path needs key_dim <= 4096");
    }
    if (E > 0x7FFFFFFF || F > 0x7FFFFFFF || Hv * dv > 0x7FFFFFFF || 2 * Hk * dk + Hv * dv > 0x7FFFFFFF ||
        Hv * oq::delta_chunks(dv) > 0x7FFFFFFF) {
        return fail(ctx, OQ_OVERFLOW, "block too large");
    }
    const uint64_t V = Hv * dv, C = 2 * Hk * dk + V;
    const BlockLayout lay = block_layout(b);
    if (ext_ws != nullptr && lay.total_floats * sizeof(float) > ext_ws_bytes) {
        return fail(ctx, OQ_INVALID_ARGUMENT,
                    "DeltaNet block workspace of " + std::to_string(lay.total_floats * sizeof(float)) +
                        " bytes exceeds the allocation-free entry point's fixed " + std::to_string(ext_ws_bytes) +
                        " bytes");
    }
    if (int rc = check_block_weight(ctx, b->qkv, E, C, "qkv")) return rc;
    if (int rc = check_block_weight(ctx, b->z, E, V, "z")) return rc;
    if (int rc = check_block_weight(ctx, b->beta, E, Hv, "beta")) return rc;
    if (int rc = check_block_weight(ctx, b->alpha, E, Hv, "alpha")) return rc;
    if (int rc = check_block_weight(ctx, b->out, V, E, "out")) return rc;
    if (int rc = check_block_weight(ctx, b->gate, E, F, "gate")) return rc;
    if (int rc = check_block_weight(ctx, b->up, E, F, "up")) return rc;
    if (int rc = check_block_weight(ctx, b->down, F, E, "down")) return rc;
    if (!b->input_norm || !b->conv_weight || !b->dt_bias || !b->decay || !b->out_norm || !b->post_norm) {
        return fail(ctx, OQ_INVALID_ARGUMENT, "null block vector");
    }
    if (!aligned(x, 4) || !aligned(y, 4) || !aligned(hist, 4) || !aligned(state, 4)) {
        return fail(ctx, OQ_INVALID_ARGUMENT, "misaligned buffer");
    }
    const uint64_t* sizes = lay.sizes;
    const uint64_t* off = lay.off;
    float* ws = ext_ws;
    if (ws == nullptr) {
        if (int rc = ensure_work(ctx, lay.total_floats * sizeof(float))) return rc;
        ws = static_cast<float*>(ctx->work.ptr);
    }
    float *qkv = ws + off[0], *z = ws + off[1], *beta = ws + off[2], *alpha = ws + off[3], *conv = ws + off[4],
          *rec = ws + off[5], *gated = ws + off[6], *branch = ws + off[7], *resid = ws + off[8], *post = ws + off[9],
          *gate = ws + off[10], *up = ws + off[11], *act = ws + off[12], *ffn = ws + off[13], *beta_s = ws + off[14],
          *log_decay = ws + off[15], *normed = ws + off[16];
    double* head_ss = reinterpret_cast<double*>(ws + off[17]);
    float* z_silu = ws + off[18];
    hipStream_t s = ctx->stream;
    hipError_t e = hipSuccess;
    // Fused path: five launches (normed in-projections with the convolution and gates, the delta
    // rule, the out projection with the residual, normed gate/up with SwiGLU, down with the
    // residual) when every projection is a K-quant GEMV of the supported shapes.
    oq::BlockGemv in{}, outp{}, ffn_in{}, down{};
    in.nmat = 4;
    in.mat[0] = b->qkv->m;
    in.mat[1] = b->z->m;
    in.mat[2] = b->beta->m;
    in.mat[3] = b->alpha->m;
    in.row_end[0] = (uint32_t)C;
    in.row_end[1] = (uint32_t)(C + V);
    in.row_end[2] = (uint32_t)(C + V + Hv);
    in.row_end[3] = (uint32_t)(C + V + 2 * Hv);
    in.x = x;
    in.norm_w = b->input_norm;
    in.eps = b->eps;
    // the raw q/k/v, beta and alpha rows feed only the trace (the delta rule reads the
    // convolution's output and the gates): without a trace they are not stored
    in.raw[0] = trace ? qkv : nullptr;
    in.raw[1] = z;
    in.raw[2] = trace ? beta : nullptr;
    in.raw[3] = trace ? alpha : nullptr;
    in.conv_w = b->conv_weight;
    in.history = hist;
    in.conv_kernel = (uint32_t)K;
    in.conv_out = conv;
    in.dt_bias = b->dt_bias;
    in.decay = b->decay;
    in.beta_s = beta_s;
    in.log_decay = log_decay;
    outp.nmat = 1;
    outp.mat[0] = b->out->m;
    outp.row_end[0] = (uint32_t)E;
    outp.x = gated;
    outp.raw[0] = trace ? branch : nullptr;  // raw outputs and staged rows: only the trace reads them
    outp.add = x;
    outp.sum_out = resid;
    outp.eps = b->eps;
    if (oq::gemv_block_add_streams(outp)) {
        // the out projection forms the gated activation in its staging (and stores it), from
        // SiLU(z) formed by the delta rule's launch
        outp.rec = rec;
        outp.head_ss = head_ss;
        outp.z = z_silu;
        outp.out_norm = b->out_norm;
        outp.dv = (uint32_t)dv;
        outp.dchunks = (uint32_t)oq::delta_chunks(dv);
        outp.gated_out = trace ? gated : nullptr;
    }
    ffn_in.nmat = 2;
    ffn_in.mat[0] = b->gate->m;
    ffn_in.mat[1] = b->up->m;
    ffn_in.row_end[0] = (uint32_t)F;
    ffn_in.row_end[1] = (uint32_t)(2 * F);
    ffn_in.x = resid;
    ffn_in.norm_w = b->post_norm;
    ffn_in.eps = b->eps;
    ffn_in.norm_out = trace ? post : nullptr;
    ffn_in.raw[0] = trace ? gate : nullptr;
    ffn_in.raw[1] = trace ? up : nullptr;
    ffn_in.act = act;
    down.nmat = 1;
    down.mat[0] = b->down->m;
    down.row_end[0] = (uint32_t)E;
    down.x = act;
    down.raw[0] = trace ? ffn : nullptr;
    down.add = resid;
    down.sum_out = y;
    const bool even = C % 2 == 0 && V % 2 == 0 && Hv % 2 == 0 && E % 2 == 0;
    // other shapes: one launch per stage, the delta rule on its any-shape kernel
    const bool fused = knob_flag(oq::kBlockFused, true) && even && aligned(x, 16) &&
                       oq::deltanet_dims_supported(dk, dv, K) && oq::gemv_block_supported(in) &&
                       oq::gemv_block_supported(outp) && oq::gemv_block_supported(ffn_in) &&
                       oq::gemv_block_supported(down);
    if (fused) {
        e = oq::launch_gemv_block(oq::kBlockIn, in, s);
        if (e == hipSuccess)
            e = oq::launch_delta(conv, Hk, Hv, dk, dv, beta_s, log_decay, b->eps, state, rec, head_ss,
                                 outp.rec != nullptr ? z : nullptr, outp.rec != nullptr ? z_silu : nullptr, s);
        if (e == hipSuccess && outp.rec == nullptr)
            e = oq::launch_gated_norm(rec, head_ss, z, b->out_norm, Hv, dv, b->eps, gated, s);
        if (e == hipSuccess) e = oq::launch_gemv_block(oq::kBlockAdd, outp, s);
        if (e == hipSuccess) e = oq::launch_gemv_block(oq::kBlockFfn, ffn_in, s);
        if (e == hipSuccess) e = oq::launch_gemv_block(oq::kBlockAdd, down, s);
    } else {
        e = oq::launch_rmsnorm(x, nullptr, b->input_norm, E, b->eps, nullptr, normed, s);
        if (e == hipSuccess) e = block_project(b->qkv, normed, qkv, s);
        if (e == hipSuccess) e = block_project(b->z, normed, z, s);
        if (e == hipSuccess) e = block_project(b->beta, normed, beta, s);
        if (e == hipSuccess) e = block_project(b->alpha, normed, alpha, s);
        if (e == hipSuccess)
            e = oq::launch_conv_gates(qkv, b->conv_weight, hist, C, K, beta, alpha, b->dt_bias, b->decay, Hv, conv, beta_s,
                                      log_decay, s);
        if (e == hipSuccess)
            e = oq::launch_delta(conv, Hk, Hv, dk, dv, beta_s, log_decay, b->eps, state, rec, head_ss, nullptr, nullptr,
                                 s);
        if (e == hipSuccess) e = oq::launch_gated_norm(rec, head_ss, z, b->out_norm, Hv, dv, b->eps, gated, s);
        if (e == hipSuccess) e = block_project(b->out, gated, branch, s);
        if (e == hipSuccess) e = oq::launch_rmsnorm(x, branch, b->post_norm, E, b->eps, resid, post, s);
        if (e == hipSuccess) e = block_project(b->gate, post, gate, s);
        if (e == hipSuccess) e = block_project(b->up, post, up, s);
        if (e == hipSuccess) e = oq::launch_swiglu(gate, up, F, act, s);
        if (e == hipSuccess) e = block_project(b->down, act, ffn, s);
        if (e == hipSuccess) e = oq::launch_add(resid, ffn, E, y, s);
    }
    if (e == hipSuccess && trace) {
        uint64_t t = 0;
        for (int i = 0; i < 16 && e == hipSuccess; ++i) {
            e = hipMemcpyAsync(trace + t, ws + off[i], sizes[i] * sizeof(float), hipMemcpyDeviceToDevice, s);
            t += sizes[i];
        }
    }
    return launch_rc(ctx, e, "deltanet_step");
}

// ---------------------------------------------------------------- m consecutive tokens

// Workspace of an m-token block step: every field of block_layout with m rows (a field's rows
// consecutive, each padded to 64 floats), then the Q8_K image of one projection input (m rows of
// the widest input).
struct StepsLayout {
    uint64_t row[19];   // floats per row of each field
    uint64_t off[19];
    uint64_t q8_off, total_floats;
};

StepsLayout steps_layout(const oq_deltanet_block* b, uint64_t m) {
    const BlockLayout one = block_layout(b);
    StepsLayout l{};
    for (int i = 0; i < 19; ++i) {
        l.row[i] = one.sizes[i];
        l.off[i] = l.total_floats;
        l.total_floats += (m * one.sizes[i] + 63) & ~uint64_t(63);
    }
    const uint64_t kmax = std::max({b->embedding, b->value_heads * b->value_dim, b->ffn});
    l.q8_off = l.total_floats;
    l.total_floats += (m * (kmax / oq::kQK) * oq::kQ8KBytes / sizeof(float) + 64) & ~uint64_t(63);
    return l;
}

// m activation rows through one block projection, with the path oq_matmul takes: matrix cores for
// m >= 16 (where `mfma` allows), else the K-quant small-batch GEMV from the Q8_K image q8
// (quantized once per input by the caller) or the F32-activation GEMV.
bool on_matrix_cores(const oq_weight* w, uint64_t m, bool mfma) {
    return mfma && oq::gemm_mfma_supported(w->m, (int)m) && knob_flag(oq::kGemmMfma, true);
}

hipError_t project_rows(oq_context* ctx, const oq_weight* w, uint64_t m, const float* x, const uint8_t* q8, float* y,
                        bool mfma = true) {
    if (on_matrix_cores(w, m, mfma)) return oq::launch_gemm_mfma(w->m, (int)m, x, nullptr, y, ctx->scratch.ptr, ctx->stream);
    if (is_kquant(w->m.type)) return oq::launch_gemv_kquant(w->m, (int)m, nullptr, q8, y, ctx->stream);
    return oq::launch_gemv_f32act(w->m, (int)m, x, y, ctx->stream);
}

// The same m rows through several matrices: one small-batch launch for matrices it can take
// together (K-quant, one type, K and pitch, none on matrix cores; 2 <= m <= 15), else one product
// each.  Each output row has the same bits either way.  With conv (the DeltaNet in-projection's
// four matrices) *conv_done tells whether the launch also ran the convolution and gates.
hipError_t project_set(oq_context* ctx, std::initializer_list<std::pair<const oq_weight*, float*>> ps, uint64_t m,
                       const float* x, const uint8_t* q8, const oq::MtConv* conv = nullptr, bool* conv_done = nullptr) {
    if (conv_done != nullptr) *conv_done = false;
    if (m >= 2 && m <= 15 && ps.size() >= 2 && ps.size() <= 4 && knob_flag(oq::kBlockFused, true)) {
        oq::DeviceMatrix mats[4];
        float* ys[4];
        uint32_t n = 0;
        bool together = true;
        for (const auto& p : ps) {
            together = together && is_kquant(p.first->m.type) && !on_matrix_cores(p.first, m, true);
            mats[n] = p.first->m;
            ys[n] = p.second;
            ++n;
        }
        if (together) {
            hipError_t e = hipErrorNotSupported;
            if (conv != nullptr && knob_flag(oq::kBlockFused, true)) {
                e = oq::launch_gemv_kquant_set(mats, n, (int)m, q8, ys, ctx->stream, nullptr, conv);
                if (e == hipSuccess && conv_done != nullptr) *conv_done = true;
            }
            if (e == hipErrorNotSupported) e = oq::launch_gemv_kquant_set(mats, n, (int)m, q8, ys, ctx->stream);
            if (e != hipErrorNotSupported) return e;
        }
    }
    for (const auto& p : ps) {
        const hipError_t e = project_rows(ctx, p.first, m, x, q8, p.second);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

// y = add + w x over m rows: the residual added in the small-batch launch's stores where it takes
// w (the same bits as a separate sum), else the product into `product` and one add launch
hipError_t project_add(oq_context* ctx, const oq_weight* w, uint64_t m, const float* x, const uint8_t* q8,
                       const float* add, float* product, float* y) {
    if (m >= 2 && m <= 15 && is_kquant(w->m.type) && !on_matrix_cores(w, m, true) && knob_flag(oq::kBlockFused, true)) {
        const hipError_t e = oq::launch_gemv_kquant_set(&w->m, 1, (int)m, q8, &y, ctx->stream, &add);
        if (e != hipErrorNotSupported) return e;
    }
    hipError_t e = project_rows(ctx, w, m, x, q8, product);
    if (e == hipSuccess) e = oq::launch_add(add, product, m * w->m.n, y, ctx->stream);
    return e;
}

bool needs_q8(const oq_weight* w, uint64_t m, bool mfma = true) {
    return is_kquant(w->m.type) && !on_matrix_cores(w, m, mfma);
}

// RMSNorm of m rows a [+ b] (n values each) feeding a set of projections.  Where the set's
// small-batch launch takes the matrices together and its staging holds the rows (m = 2,
// n <= 8192) the launch normalises them itself (sum_out and, with keep_normed, normed stored by
// its first workgroup); else the RMSNorm launch (sum_out, normed and the Q8_K image when a
// projection takes it) and project_set.  Each output has the same value either way (the
// same formula; the double sums of squares are added in another order, which changes the F32
// inverse RMS only when the sums fall within about 1e-16 of a rounding boundary).
hipError_t norm_project_set(oq_context* ctx, std::initializer_list<std::pair<const oq_weight*, float*>> ps, uint64_t m,
                            const float* a, const float* b, const float* w, float eps, uint64_t n, float* sum_out,
                            float* normed, bool keep_normed, uint8_t* q8, const oq::MtConv* conv = nullptr,
                            bool* conv_done = nullptr) {
    if (conv_done != nullptr) *conv_done = false;
    if (m == 2 && ps.size() >= 2 && ps.size() <= 4 && knob_flag(oq::kBlockFused, true)) {
        oq::DeviceMatrix mats[4];
        float* ys[4];
        uint32_t cnt = 0;
        bool together = true;
        for (const auto& p : ps) {
            together = together && is_kquant(p.first->m.type) && !on_matrix_cores(p.first, m, true);
            mats[cnt] = p.first->m;
            ys[cnt] = p.second;
            ++cnt;
        }
        if (together) {
            const oq::MtNorm nm{b, w, eps, sum_out, keep_normed ? normed : nullptr};
            hipError_t e = hipErrorNotSupported;
            if (conv != nullptr) {
                e = oq::launch_gemv_kquant_set_norm(mats, cnt, (int)m, a, nm, ys, ctx->stream, conv);
                if (e == hipSuccess && conv_done != nullptr) *conv_done = true;
            }
            if (e == hipErrorNotSupported) e = oq::launch_gemv_kquant_set_norm(mats, cnt, (int)m, a, nm, ys, ctx->stream);
            if (e != hipErrorNotSupported) return e;
        }
    }
    bool q8_needed = false;
    for (const auto& p : ps) q8_needed = q8_needed || needs_q8(p.first, m);
    hipError_t e = oq::launch_rmsnorm(a, b, w, n, eps, sum_out, normed, ctx->stream, m, q8_needed ? q8 : nullptr);
    if (e == hipSuccess) e = project_set(ctx, ps, m, normed, q8, conv, conv_done);
    return e;
}

int deltanet_steps(oq_context* ctx, const oq_deltanet_block* b, uint64_t m, float* hist, float* state, const float* x,
                   float* y, float* trace) {
    if (!ctx) return fail(nullptr, OQ_INVALID_ARGUMENT, "null context");
    if (!b || !hist || !state || !x || !y) return fail(ctx, OQ_INVALID_ARGUMENT, "null argument");
    if (m == 0) return fail(ctx, OQ_INVALID_ARGUMENT, "token count must be non-zero");
    if (m > 0xFFFF) return fail(ctx, OQ_INVALID_ARGUMENT, "at most 65535 tokens per call");
    const uint64_t E = b->embedding, Hk = b->key_heads, Hv = b->value_heads, dk = b->key_dim, dv = b->value_dim,
                   K = b->conv_kernel, F = b->ffn;
    if (E == 0 || Hk == 0 || Hv == 0 || dk == 0 || dv == 0 || K == 0 || F == 0 || Hv % Hk != 0) {
        return fail(ctx, OQ_INVALID_ARGUMENT, "Qwen3.5 recurrent block dimensions are incompatible");
    }
    if (!(b->eps > 0.0f) || !std::isfinite(b->eps)) {
        return fail(ctx, OQ_INVALID_ARGUMENT, "Qwen3.5 RMSNorm epsilon must be positive and finite");
    }
    if (!oq::deltanet_dims_any(dk, dv, K)) {
        return fail(ctx, OQ_INVALID_ARGUMENT, "DeltaNet block device path needs key_dim <= 4096");
    }
    const uint64_t V = Hv * dv, C = 2 * Hk * dk + V;
    if (m * std::max({E, F, C}) > 0x7FFFFFFF || Hv * oq::delta_chunks(dv) > 0x7FFFFFFF) {
        return fail(ctx, OQ_OVERFLOW, "block too large");
    }
    if (int rc = check_block_weight(ctx, b->qkv, E, C, "qkv")) return rc;
    if (int rc = check_block_weight(ctx, b->z, E, V, "z")) return rc;
    if (int rc = check_block_weight(ctx, b->beta, E, Hv, "beta")) return rc;
    if (int rc = check_block_weight(ctx, b->alpha, E, Hv, "alpha")) return rc;
    if (int rc = check_block_weight(ctx, b->out, V, E, "out")) return rc;
    if (int rc = check_block_weight(ctx, b->gate, E, F, "gate")) return rc;
    if (int rc = check_block_weight(ctx, b->up, E, F, "up")) return rc;
    if (int rc = check_block_weight(ctx, b->down, F, E, "down")) return rc;
    if (!b->input_norm || !b->conv_weight || !b->dt_bias || !b->decay || !b->out_norm || !b->post_norm) {
        return fail(ctx, OQ_INVALID_ARGUMENT, "null block vector");
    }
    if (!aligned(x, 16) || !aligned(y, 4) || !aligned(hist, 4) || !aligned(state, 4) || (trace && !aligned(trace, 4))) {
        return fail(ctx, OQ_INVALID_ARGUMENT, "misaligned buffer (x 16-byte, others 4-byte)");
    }
    if (!oq::deltanet_dims_supported(dk, dv, K)) {
        // shapes outside the token-batched kernels: the single step's per-stage launches, token by
        // token (token t's trace at trace + t * the single step's trace size, as below)
        const BlockLayout one = block_layout(b);
        uint64_t per_token = 0;
        for (int i = 0; i < 16; ++i) per_token += one.sizes[i];
        for (uint64_t t = 0; t < m; ++t) {
            if (int rc = deltanet_step(ctx, b, hist, state, x + t * E, y + t * E, trace ? trace + t * per_token : nullptr,
                                       nullptr, 0))
                return rc;
        }
        return OQ_OK;
    }
    const StepsLayout lay = steps_layout(b, m);
    if (int rc = ensure_work(ctx, lay.total_floats * sizeof(float))) return rc;
    uint64_t scratch = 0;
    for (const oq_weight* w : {b->qkv, b->z, b->beta, b->alpha, b->gate, b->up, b->down}) {
        if (oq::gemm_mfma_supported(w->m, (int)m) && knob_flag(oq::kGemmMfma, true))
            scratch = std::max(scratch, oq::gemm_scratch_bytes(w->m, (int)m));
    }
    if (scratch > 0) {
        if (int rc = ensure_scratch(ctx, scratch)) return rc;
    }
    float* ws = static_cast<float*>(ctx->work.ptr);
    const uint64_t* off = lay.off;
    float *qkv = ws + off[0], *z = ws + off[1], *beta = ws + off[2], *alpha = ws + off[3], *conv = ws + off[4],
          *rec = ws + off[5], *gated = ws + off[6], *branch = ws + off[7], *resid = ws + off[8], *post = ws + off[9],
          *gate = ws + off[10], *up = ws + off[11], *act = ws + off[12], *ffn = ws + off[13], *beta_s = ws + off[14],
          *log_decay = ws + off[15], *normed = ws + off[16];
    double* head_ss = reinterpret_cast<double*>(ws + off[17]);
    uint8_t* q8 = reinterpret_cast<uint8_t*>(ws + lay.q8_off);
    hipStream_t s = ctx->stream;
    // the Q8_K image an input's producer writes beside it, when a projection of it takes the
    // small-batch GEMV (null: none does)
    auto q8_for = [&](std::initializer_list<const oq_weight*> consumers) -> uint8_t* {
        for (const oq_weight* w : consumers)
            if (needs_q8(w, m)) return q8;
        return nullptr;
    };
    hipError_t e = hipSuccess;
    // the convolution and gates in the in-projection's launch where it takes the four matrices
    // together, else their own launch
    oq::MtConv epi{b->conv_weight, hist, conv, (uint32_t)K, beta_s, log_decay, b->dt_bias, b->decay};
    bool conv_done = false;
    if (e == hipSuccess)
        e = norm_project_set(ctx, {{b->qkv, qkv}, {b->z, z}, {b->beta, beta}, {b->alpha, alpha}}, m, x, nullptr,
                             b->input_norm, b->eps, E, nullptr, normed, false, q8, &epi, &conv_done);
    if (e == hipSuccess && !conv_done)
        e = oq::launch_conv_gates_tokens(qkv, b->conv_weight, hist, C, K, beta, alpha, b->dt_bias, b->decay, Hv, m,
                                         conv, beta_s, log_decay, s);
    if (e == hipSuccess)
        e = oq::launch_delta(conv, Hk, Hv, dk, dv, beta_s, log_decay, b->eps, state, rec, head_ss, nullptr, nullptr, s,
                             m);
    // the out projection's input (RMSNorm(rec) * out_norm * SiLU(z), a product of two near-Gaussian
    // rows) is heavy-tailed -- kurtosis 68 on the hidden-4096 block, one product up to 13 % of
    // sum |w xhat| -- so f16 operands would reach the product bar (2.3e-4 measured at 16 tokens):
    // it keeps the integer-dot products at every m, from the Q8_K blocks the gated norm writes
    if (e == hipSuccess)
        e = oq::launch_gated_norm(rec, head_ss, z, b->out_norm, Hv, dv, b->eps, gated, s, m,
                                  is_kquant(b->out->m.type) ? q8 : nullptr);
    if (e == hipSuccess) e = project_rows(ctx, b->out, m, gated, q8, branch, false);
    if (e == hipSuccess)
        e = norm_project_set(ctx, {{b->gate, gate}, {b->up, up}}, m, x, branch, b->post_norm, b->eps, E, resid, post,
                             trace != nullptr, q8);
    if (e == hipSuccess) e = oq::launch_swiglu(gate, up, m * F, act, s, q8_for({b->down}));
    if (e == hipSuccess && trace) {
        e = project_rows(ctx, b->down, m, act, q8, ffn);  // the trace keeps the down projection
        if (e == hipSuccess) e = oq::launch_add(resid, ffn, m * E, y, s);
    } else if (e == hipSuccess) {
        e = project_add(ctx, b->down, m, act, q8, resid, ffn, y);
    }
    if (e == hipSuccess && trace) {
        // token t's trace (the 16 fields of oq_deltanet_step's trace, in order) at trace + t * size
        uint64_t per_token = 0;
        for (int i = 0; i < 16; ++i) per_token += lay.row[i];
        uint64_t t = 0;
        for (int i = 0; i < 16 && e == hipSuccess; ++i) {
            e = hipMemcpy2DAsync(trace + t, per_token * sizeof(float), ws + off[i], lay.row[i] * sizeof(float),
                                 lay.row[i] * sizeof(float), m, hipMemcpyDeviceToDevice, s);
            t += lay.row[i];
        }
    }
    return launch_rc(ctx, e, "deltanet_steps");
}

}  // namespace

namespace oq {

int deltanet_step_into(oq_context* ctx, const oq_deltanet_block* b, float* hist, float* state, const float* x,
                       float* y, float* trace, float* ws, uint64_t ws_bytes) {
    if (ws == nullptr) return fail(ctx, OQ_DEVICE_ERROR, "allocation-free workspace is not set up on this device");
    return deltanet_step(ctx, b, hist, state, x, y, trace, ws, ws_bytes);
}

int context_device(const oq_context* ctx) { return ctx->device; }

int set_error(oq_context* ctx, int code, const char* msg) { return fail(ctx, code, msg); }

}  // namespace oq

extern "C" {

int oq_deltanet_step(oq_context* ctx, const oq_deltanet_block* b, float* hist, float* state, const float* x,
                     float* y, float* trace) {
    return deltanet_step(ctx, b, hist, state, x, y, trace, nullptr, 0);
}

int oq_deltanet_steps(oq_context* ctx, const oq_deltanet_block* b, uint64_t m, float* hist, float* state,
                      const float* x, float* y, float* trace) {
    return deltanet_steps(ctx, b, m, hist, state, x, y, trace);
}

}  // extern "C"

namespace {

}  // namespace

extern "C" {

int oq_type_layout(uint32_t type, uint64_t* block_elements, uint64_t* bytes_per_block, int* quantized,
                   const char** name) {
    const Layout* l = layout_of(type);
    if (!l) return fail(nullptr, OQ_UNSUPPORTED_TYPE, "unsupported GGML tensor type: " + std::to_string(type));
    if (block_elements) *block_elements = l->block_elements;
    if (bytes_per_block) *bytes_per_block = l->bytes_per_block;
    if (quantized) *quantized = l->quantized;
    if (name) *name = l->name;
    return OQ_OK;
}

int oq_row_byte_size(uint64_t row_elements, uint32_t type, uint64_t* out) {
    if (!out) return fail(nullptr, OQ_INVALID_ARGUMENT, "null output");
    return row_bytes(nullptr, row_elements, type, out);
}

int oq_type_supported(uint32_t t) {
    return t == OQ_TYPE_F32 || t == OQ_TYPE_F16 || t == OQ_TYPE_BF16 || t == OQ_TYPE_Q8_0 ||
           t == OQ_TYPE_Q4_K || t == OQ_TYPE_Q5_K || t == OQ_TYPE_Q6_K;
}

int oq_context_create(int device, oq_context** out) {
    if (!out) return fail(nullptr, OQ_INVALID_ARGUMENT, "null output handle");
    *out = nullptr;
    int count = 0;
    hipError_t e = hipGetDeviceCount(&count);
    if (e != hipSuccess) return hip_fail(nullptr, e, "hipGetDeviceCount");
    if (device < 0 || device >= count) {
        return fail(nullptr, OQ_OUT_OF_RANGE, "device ordinal " + std::to_string(device) + " out of range");
    }
    e = hipSetDevice(device);
    if (e != hipSuccess) return hip_fail(nullptr, e, "hipSetDevice");
    oq::ensure_knobs();
    oq::noalloc_setup(device);  // its failure is reported by the allocation-free entry point
    oq_context* ctx = new oq_context;
    ctx->device = device;
    e = hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking);
    if (e == hipSuccess) e = hipEventCreateWithFlags(&ctx->t0, hipEventDisableSystemFence);
    if (e == hipSuccess) e = hipEventCreateWithFlags(&ctx->t1, hipEventDisableSystemFence);
    if (e == hipSuccess) e = hipMalloc(&ctx->argmax_parts, oq::kArgmaxParts * sizeof(oq::ArgmaxPart));
    if (e != hipSuccess) {
        const int rc = hip_fail(nullptr, e, "context creation");
        oq_context_destroy(ctx);
        return rc;
    }
    *out = ctx;
    return OQ_OK;
}

void oq_context_destroy(oq_context* ctx) {
    if (!ctx) return;
    (void)hipSetDevice(ctx->device);
    if (ctx->stream) (void)hipStreamSynchronize(ctx->stream);
    for (oq_graph* g : ctx->graphs) g->ctx = nullptr;
    ctx->scratch.release_all(device_free);
    ctx->work.release_all(device_free);
    if (ctx->argmax_parts) (void)hipFree(ctx->argmax_parts);
    if (ctx->t0) (void)hipEventDestroy(ctx->t0);
    if (ctx->t1) (void)hipEventDestroy(ctx->t1);
    if (ctx->stream) (void)hipStreamDestroy(ctx->stream);
    delete ctx;
}

const char* oq_last_error(const oq_context* ctx) { return ctx ? ctx->error.c_str() : g_error.c_str(); }

void oq_reload_options(void) { oq::load_knobs(); }

int oq_synchronize(oq_context* ctx) {
    if (!ctx) return fail(nullptr, OQ_INVALID_ARGUMENT, "null context");
    OQ_HIP(ctx, hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
    return OQ_OK;
}

void* oq_context_stream(oq_context* ctx) { return ctx ? ctx->stream : nullptr; }

int oq_device_alloc(oq_context* ctx, uint64_t bytes, void** out) {
    if (!ctx || !out) return fail(ctx, OQ_INVALID_ARGUMENT, "null argument");
    *out = nullptr;
    OQ_HIP(ctx, hipSetDevice(ctx->device), "hipSetDevice");
    OQ_HIP(ctx, hipMalloc(out, bytes ? bytes : 1), "hipMalloc");
    return OQ_OK;
}

int oq_device_free(oq_context* ctx, void* p) {
    if (!ctx) return fail(nullptr, OQ_INVALID_ARGUMENT, "null context");
    if (p) {
        OQ_HIP(ctx, hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
        OQ_HIP(ctx, hipFree(p), "hipFree");
    }
    return OQ_OK;
}

int oq_copy_to_device(oq_context* ctx, void* dst, const void* src, uint64_t bytes) {
    if (!ctx || (bytes && (!dst || !src))) return fail(ctx, OQ_INVALID_ARGUMENT, "null argument");
    OQ_HIP(ctx, hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, ctx->stream), "hipMemcpy H2D");
    OQ_HIP(ctx, hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
    return OQ_OK;
}

int oq_copy_to_host(oq_context* ctx, void* dst, const void* src, uint64_t bytes) {
    if (!ctx || (bytes && (!dst || !src))) return fail(ctx, OQ_INVALID_ARGUMENT, "null argument");
    OQ_HIP(ctx, hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, ctx->stream), "hipMemcpy D2H");
    OQ_HIP(ctx, hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
    return OQ_OK;
}

int oq_copy_device(oq_context* ctx, void* dst, const void* src, uint64_t bytes) {
    if (!ctx || (bytes && (!dst || !src))) return fail(ctx, OQ_INVALID_ARGUMENT, "null argument");
    OQ_HIP(ctx, hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, ctx->stream), "hipMemcpy D2D");
    return OQ_OK;
}

int oq_weight_upload(oq_context* ctx, uint32_t type, uint64_t ne0, uint64_t ne1, const void* host_bytes,
                     uint64_t nbytes, oq_weight** out) {
    return upload_common(ctx, type, ne0, ne1, host_bytes, nbytes, false, out);
}

int oq_weight_upload_device(oq_context* ctx, uint32_t type, uint64_t ne0, uint64_t ne1, const void* dev_bytes,
                            uint64_t nbytes, oq_weight** out) {
    return upload_common(ctx, type, ne0, ne1, dev_bytes, nbytes, true, out);
}

void oq_weight_release(oq_weight* w) {
    if (!w) return;
    if (w->owned) {
        (void)hipSetDevice(w->device);
        (void)hipDeviceSynchronize();
        (void)hipFree(w->owned);
    }
    delete w;
}

int oq_weight_info(const oq_weight* w, uint32_t* type, uint64_t* ne0, uint64_t* ne1, uint64_t* device_bytes) {
    if (!w) return fail(nullptr, OQ_INVALID_ARGUMENT, "null weight");
    if (type) *type = w->m.type;
    if (ne0) *ne0 = w->m.k;
    if (ne1) *ne1 = w->m.n;
    if (device_bytes) *device_bytes = w->device_bytes;
    return OQ_OK;
}

int oq_dequantize_rows(oq_context* ctx, const oq_weight* w, uint64_t row0, uint64_t nrows, float* out) {
    if (!ctx) return fail(nullptr, OQ_INVALID_ARGUMENT, "null context");
    if (int rc = check_weight(ctx, w)) return rc;
    if (row0 > w->m.n || nrows > w->m.n - row0) {
        return fail(ctx, OQ_OUT_OF_RANGE, "GGUF tensor row index exceeds row count");
    }
    if (nrows == 0) return OQ_OK;
    if (!out) return fail(ctx, OQ_INVALID_ARGUMENT, "null output");
    return launch_rc(ctx, oq::launch_dequantize(w->m, row0, nrows, out, ctx->stream), "dequantize");
}

int oq_quantize_q8k(oq_context* ctx, const float* x, uint64_t m, uint64_t k, void* q8k) {
    if (!ctx) return fail(nullptr, OQ_INVALID_ARGUMENT, "null context");
    if (m == 0 || k == 0 || k % oq::kQK != 0) {
        return fail(ctx, OQ_INVALID_ARGUMENT, "Q8_K quantization needs m > 0 rows of a multiple of 256 values");
    }
    if (!x || !q8k) return fail(ctx, OQ_INVALID_ARGUMENT, "null buffer");
    if (!aligned(x, 16) || !aligned(q8k, 4)) {
        return fail(ctx, OQ_INVALID_ARGUMENT, "activations must be 16-byte aligned and Q8_K blocks 4-byte aligned");
    }
    return launch_rc(ctx, oq::launch_quantize_q8k(x, m, k, static_cast<uint8_t*>(q8k), ctx->stream),
                     "quantize_q8k");
}

int oq_argmax(oq_context* ctx, const float* logits, uint64_t n, uint32_t* token, float* value) {
    if (!ctx) return fail(nullptr, OQ_INVALID_ARGUMENT, "null context");
    // checks in the order of Sampler::sample (src/runtime/sampler.cpp:22-28)
    if (n == 0) return fail(ctx, OQ_INVALID_ARGUMENT, "cannot sample an empty logits vector");
    if (n > 0xFFFFFFFFull) return fail(ctx, OQ_INVALID_ARGUMENT, "logits vector exceeds token-id range");
    if (!logits || !token || !value) return fail(ctx, OQ_INVALID_ARGUMENT, "null buffer");
    if (!aligned(logits, 4) || !aligned(token, 4) || !aligned(value, 4)) {
        return fail(ctx, OQ_INVALID_ARGUMENT, "argmax buffers must be 4-byte aligned");
    }
    return launch_rc(ctx, oq::launch_argmax(logits, n, token, value, ctx->argmax_parts, ctx->stream), "argmax");
}

int oq_matmul(oq_context* ctx, const oq_weight* w, uint64_t m, const float* x, float* y) {
    if (!ctx) return fail(nullptr, OQ_INVALID_ARGUMENT, "null context");
    if (int rc = check_weight(ctx, w)) return rc;
    if (m == 0) return fail(ctx, OQ_INVALID_ARGUMENT, "matmul batch must be non-zero");
    if (m > 0x7FFFFFFF) return fail(ctx, OQ_OVERFLOW, "matmul batch too large");
    if (!x || !y) return fail(ctx, OQ_INVALID_ARGUMENT, "null buffer");
    const uint32_t t = w->m.type;
    const bool vec_loads = is_kquant(t) || t == OQ_TYPE_Q8_0;
    if ((vec_loads && !aligned(x, 16)) || !aligned(x, 4) || !aligned(y, 4)) {
        return fail(ctx, OQ_INVALID_ARGUMENT, "activation / output buffers are misaligned");
    }
    if (is_kquant(t)) {
        if (oq::gemm_i8_supported(w->m, (int)m) && knob_flag(oq::kGemmInt8, false)) {
            if (int rc = ensure_scratch(ctx, oq::gemm_i8_scratch_bytes(w->m, (int)m))) return rc;
            return launch_rc(ctx, oq::launch_gemm_q4k_i8(w->m, (int)m, x, nullptr, y, ctx->scratch.ptr, ctx->stream),
                             "matmul");
        }
        if (oq::gemm_mfma_supported(w->m, (int)m) && knob_flag(oq::kGemmMfma, true)) {
            if (int rc = ensure_scratch(ctx, oq::gemm_scratch_bytes(w->m, (int)m))) return rc;
            return launch_rc(ctx, oq::launch_gemm_mfma(w->m, (int)m, x, nullptr, y, ctx->scratch.ptr, ctx->stream),
                             "matmul");
        }
        // one row: every workgroup quantizes x itself (saves a launch); several rows: quantize
        // once and let the workgroups copy the Q8_K blocks
        if (!knob_flag(oq::kFusedQuant, m == 1)) {
            const uint64_t q8bytes = (m * (w->m.k / oq::kQK) * oq::kQ8KBytes + 255) & ~uint64_t(255);
            if (int rc = ensure_scratch(ctx, q8bytes)) return rc;
            uint8_t* q8 = static_cast<uint8_t*>(ctx->scratch.ptr);
            hipError_t e = oq::launch_quantize_q8k(x, m, w->m.k, q8, ctx->stream);
            if (e == hipSuccess) e = oq::launch_gemv_kquant(w->m, (int)m, nullptr, q8, y, ctx->stream);
            return launch_rc(ctx, e, "matmul");
        }
        return launch_rc(ctx, oq::launch_gemv_kquant(w->m, (int)m, x, nullptr, y, ctx->stream), "matmul");
    }
    if (t == OQ_TYPE_Q8_0 && oq::gemm_mfma_supported(w->m, (int)m) && knob_flag(oq::kGemmMfma, true)) {
        if (int rc = ensure_scratch(ctx, oq::gemm_scratch_bytes(w->m, (int)m))) return rc;
        return launch_rc(ctx, oq::launch_gemm_mfma(w->m, (int)m, x, nullptr, y, ctx->scratch.ptr, ctx->stream),
                         "matmul");
    }
    return launch_rc(ctx, oq::launch_gemv_f32act(w->m, (int)m, x, y, ctx->stream), "matmul");
}

int oq_matvec(oq_context* ctx, const oq_weight* w, const float* x, float* y) {
    return oq_matmul(ctx, w, 1, x, y);
}

int oq_matvec_argmax(oq_context* ctx, const oq_weight* w, const float* x, float* y, uint32_t* token, float* value) {
    if (!ctx) return fail(nullptr, OQ_INVALID_ARGUMENT, "null context");
    if (int rc = check_weight(ctx, w)) return rc;
    if (!x || !y || !token || !value) return fail(ctx, OQ_INVALID_ARGUMENT, "null buffer");
    if (w->m.n > 0xFFFFFFFEull) return fail(ctx, OQ_OVERFLOW, "argmax over more than 2^32 - 1 logits");
    if (!aligned(token, 4) || !aligned(value, 4)) {
        return fail(ctx, OQ_INVALID_ARGUMENT, "argmax buffers must be 4-byte aligned");
    }
    if (is_kquant(w->m.type) && aligned(x, 16) && aligned(y, 4)) {
        // the decode GEMV reduces its own outputs: one partial per workgroup, then one small
        // kernel combines them
        uint32_t nparts = 0;
        auto* parts = static_cast<oq::ArgmaxPart*>(ctx->argmax_parts);
        hipError_t e = oq::launch_gemv_kquant_argmax(w->m, x, nullptr, y, parts, oq::kArgmaxParts, &nparts, ctx->stream);
        if (e == hipSuccess) {
            return launch_rc(ctx, oq::launch_argmax_final(parts, nparts, token, value, ctx->stream), "matvec_argmax");
        }
        if (e != hipErrorNotSupported) return launch_rc(ctx, e, "matvec_argmax");
        (void)hipGetLastError();
    }
    if (int rc = oq_matmul(ctx, w, 1, x, y)) return rc;
    return oq_argmax(ctx, y, w->m.n, token, value);
}

int oq_matmul_q8k(oq_context* ctx, const oq_weight* w, uint64_t m, const void* q8k, float* y) {
    if (!ctx) return fail(nullptr, OQ_INVALID_ARGUMENT, "null context");
    if (int rc = check_weight(ctx, w)) return rc;
    if (!is_kquant(w->m.type)) {
        return fail(ctx, OQ_INVALID_ARGUMENT, "Q8_K activations need a q4_K, q5_K or q6_K weight");
    }
    if (m == 0) return fail(ctx, OQ_INVALID_ARGUMENT, "matmul batch must be non-zero");
    if (m > 0x7FFFFFFF) return fail(ctx, OQ_OVERFLOW, "matmul batch too large");
    if (!q8k || !y) return fail(ctx, OQ_INVALID_ARGUMENT, "null buffer");
    if (!aligned(q8k, 4) || !aligned(y, 4)) return fail(ctx, OQ_INVALID_ARGUMENT, "misaligned buffer");
    const uint8_t* q8 = static_cast<const uint8_t*>(q8k);
    if (oq::gemm_i8_supported(w->m, (int)m) && knob_flag(oq::kGemmInt8, false)) {
        if (int rc = ensure_scratch(ctx, oq::gemm_i8_scratch_bytes(w->m, (int)m))) return rc;
        return launch_rc(ctx, oq::launch_gemm_q4k_i8(w->m, (int)m, nullptr, q8, y, ctx->scratch.ptr, ctx->stream),
                         "matmul_q8k");
    }
    if (oq::gemm_mfma_supported(w->m, (int)m) && knob_flag(oq::kGemmMfma, true)) {
        if (int rc = ensure_scratch(ctx, oq::gemm_scratch_bytes(w->m, (int)m))) return rc;
        return launch_rc(ctx, oq::launch_gemm_mfma(w->m, (int)m, nullptr, q8, y, ctx->scratch.ptr, ctx->stream),
                         "matmul_q8k");
    }
    return launch_rc(ctx, oq::launch_gemv_kquant(w->m, (int)m, nullptr, q8, y, ctx->stream), "matmul_q8k");
}

int oq_matvec_q8k(oq_context* ctx, const oq_weight* w, const void* q8k, float* y) {
    return oq_matmul_q8k(ctx, w, 1, q8k, y);
}

int oq_timer_start(oq_context* ctx) {
    if (!ctx) return fail(nullptr, OQ_INVALID_ARGUMENT, "null context");
    OQ_HIP(ctx, hipEventRecord(ctx->t0, ctx->stream), "hipEventRecord");
    return OQ_OK;
}

int oq_timer_stop(oq_context* ctx, float* ms) {
    if (!ctx || !ms) return fail(ctx, OQ_INVALID_ARGUMENT, "null argument");
    OQ_HIP(ctx, hipEventRecord(ctx->t1, ctx->stream), "hipEventRecord");
    OQ_HIP(ctx, hipEventSynchronize(ctx->t1), "hipEventSynchronize");
    OQ_HIP(ctx, hipEventElapsedTime(ms, ctx->t0, ctx->t1), "hipEventElapsedTime");
    OQ_HIP(ctx, hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
    return OQ_OK;
}

int oq_capture_begin(oq_context* ctx) {
    if (!ctx) return fail(nullptr, OQ_INVALID_ARGUMENT, "null context");
    if (ctx->capturing) return fail(ctx, OQ_INVALID_ARGUMENT, "capture already active");
    OQ_HIP(ctx, hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
    ctx->capturing = true;
    return OQ_OK;
}

int oq_capture_end(oq_context* ctx, oq_graph** out) {
    if (!ctx || !out) return fail(ctx, OQ_INVALID_ARGUMENT, "null argument");
    *out = nullptr;
    if (!ctx->capturing) return fail(ctx, OQ_INVALID_ARGUMENT, "no capture active");
    ctx->capturing = false;
    hipGraph_t g = nullptr;
    OQ_HIP(ctx, hipStreamEndCapture(ctx->stream, &g), "hipStreamEndCapture");
    hipGraphExec_t ex = nullptr;
    hipError_t e = hipGraphInstantiate(&ex, g, nullptr, nullptr, 0);
    // upload the executable graph now, so that its first launch does not pay for it
    if (e == hipSuccess) e = hipGraphUpload(ex, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) {
        if (ex) (void)hipGraphExecDestroy(ex);
        (void)hipGraphDestroy(g);
        return hip_fail(ctx, e, "hipGraphInstantiate");
    }
    oq_graph* gr = new oq_graph;
    gr->graph = g;
    gr->exec = ex;
    gr->ctx = ctx;
    ctx->graphs.push_back(gr);
    *out = gr;
    return OQ_OK;
}

int oq_graph_launch(oq_context* ctx, oq_graph* g) {
    if (!ctx || !g) return fail(ctx, OQ_INVALID_ARGUMENT, "null argument");
    OQ_HIP(ctx, hipGraphLaunch(g->exec, ctx->stream), "hipGraphLaunch");
    return OQ_OK;
}

void oq_graph_destroy(oq_graph* g) {
    if (!g) return;
    if (oq_context* ctx = g->ctx) {
        // a replay may still be running on the context's stream
        (void)hipStreamSynchronize(ctx->stream);
        ctx->graphs.erase(std::remove(ctx->graphs.begin(), ctx->graphs.end(), g), ctx->graphs.end());
        if (ctx->graphs.empty()) {
            ctx->scratch.release_retired(device_free);
            ctx->work.release_retired(device_free);
        }
    }
    if (g->exec) (void)hipGraphExecDestroy(g->exec);
    if (g->graph) (void)hipGraphDestroy(g->graph);
    delete g;
}

}  // extern "C"

// ---------------------------------------------------------------- full attention (decode)

struct oq_kv_cache {
    oq_context* ctx = nullptr;
    int device = 0;
    uint32_t type = OQ_TYPE_F32;  // element type: OQ_TYPE_F32 or OQ_TYPE_F16
    uint64_t capacity = 0, kv_heads = 0, key_dim = 0, value_dim = 0, length = 0;
    void* keys = nullptr;
    void* values = nullptr;
    uint64_t element_bytes() const { return type == OQ_TYPE_F16 ? 2 : 4; }
};

namespace {

// apply_qwen35_rope's checks (reference_kernels.cpp:80-99), in its order
int rope_params(oq_context* ctx, uint64_t head_dim, uint64_t rotary_dim, const int32_t* sections, float base,
                const uint64_t* position, oq::RopeParams& p) {
    if (!sections || !position) return fail(ctx, OQ_INVALID_ARGUMENT, "null RoPE sections or position");
    if (rotary_dim == 0 || rotary_dim % 2 != 0 || rotary_dim > head_dim) {
        return fail(ctx, OQ_INVALID_ARGUMENT, "RoPE dimension must be non-zero, even, and within head width");
    }
    if (!(base > 0.0f) || !std::isfinite(base)) {
        return fail(ctx, OQ_INVALID_ARGUMENT, "RoPE frequency base must be positive and finite");
    }
    int64_t sum = 0;
    for (int i = 0; i < 4; ++i) {
        if (sections[i] < 0) return fail(ctx, OQ_INVALID_ARGUMENT, "RoPE dimension sections must be non-negative");
        sum += sections[i];
    }
    if (sum != (int64_t)(rotary_dim / 2)) {
        return fail(ctx, OQ_INVALID_ARGUMENT, "RoPE dimension sections must sum to half the rotary dimension");
    }
    if (rotary_dim > 0xFFFFFFFFull) return fail(ctx, OQ_OVERFLOW, "RoPE dimension too large");
    p.rotary_dim = (uint32_t)rotary_dim;
    p.sec1 = (uint32_t)sections[1];
    p.sec2 = (uint32_t)sections[2];
    p.base = base;
    p.pos[0] = position[0];
    p.pos[1] = position[1];
    p.pos[2] = position[2];
    return OQ_OK;
}

}  // namespace

// apply_qwen35_rope's angles (reference_kernels.cpp:105-115), frequency by frequency, in the same
// double operations on the host's libm
void oq::rope_table(const RopeParams& p, RopeTable& t) {
    const uint32_t half = p.rotary_dim / 2;
    t.pairs = 0;
    if (half == 0 || half > kRopeTablePairs) return;
    for (uint32_t f = 0; f < half; ++f) {
        const double exponent = (2.0 * (double)f) / (double)p.rotary_dim;
        const double inverse_frequency = 1.0 / std::pow((double)p.base, exponent);
        // position_for_frequency (reference_kernels.cpp:28-40)
        uint64_t coordinate = p.pos[0];
        if (f % 3u == 1u && f / 3u < p.sec1) {
            coordinate = p.pos[1];
        } else if (f % 3u == 2u && f / 3u < p.sec2) {
            coordinate = p.pos[2];
        }
        const double angle = (double)coordinate * inverse_frequency;
        t.cs[0][f] = (float)std::cos(angle);
        t.cs[1][f] = (float)std::sin(angle);
    }
    t.pairs = half;
}

namespace {

// A step runs on the cache's own context: its stream orders the step after the cache's reset and
// load.  The token count lives on the host and advances when the step is issued, so a step cannot
// be recorded into a graph (a replay would attend over the recorded length and rewrite the same
// row).
int check_cache(oq_context* ctx, const oq_kv_cache* c) {
    if (!c) return fail(ctx, OQ_INVALID_ARGUMENT, "null KV cache");
    if (c->device != ctx->device) return fail(ctx, OQ_INVALID_ARGUMENT, "KV cache lives on another device");
    if (c->ctx != ctx) return fail(ctx, OQ_INVALID_ARGUMENT, "KV cache belongs to another context");
    if (capturing_now(ctx)) {
        return fail(ctx, OQ_INVALID_ARGUMENT,
                    "an attention step cannot be captured into a graph (the KV cache length advances on the host)");
    }
    return OQ_OK;
}

// the attention launch over a cache whose new token (index T - 1 = cache->length) is given by
// new_k / new_v, or already stored (both null); the partials go to `part`
// the chunked kernels' shapes; every other one takes the any-shape kernels
bool attention_fast(const oq_kv_cache* c, uint64_t q_heads) {
    return c->key_dim == c->value_dim && oq::attention_dims_supported(c->key_dim, q_heads / c->kv_heads) &&
           !knob_flag(oq::kAnyShape, false);
}

int attention_shape(oq_context* ctx, const oq_kv_cache* c, uint64_t q_heads, oq::AttnLaunch& L, uint64_t ahead = 0,
                    uint64_t token_groups = 1) {
    const uint64_t rep = q_heads / c->kv_heads;
    const uint64_t T = c->length + 1 + ahead;  // the token `ahead` places after the next one to append
    if (!attention_fast(c, q_heads)) {
        if (c->key_dim > oq::kAttnAnyMaxDim) {
            return fail(ctx, OQ_INVALID_ARGUMENT, "attention device path needs key_dim <= 8192");
        }
        if (T > 0xFFFFFFFFull || c->kv_heads > 0xFFFF || q_heads > 0x7FFFFFFF || c->value_dim > 0xFFFFFFFFull) {
            return fail(ctx, OQ_INVALID_ARGUMENT, "attention device path supports at most 4294967295 cached tokens");
        }
        L.any = true;
        L.T = (uint32_t)T;
        L.Hkv = (uint32_t)c->kv_heads;
        L.rep = (uint32_t)rep;
        L.D = (uint32_t)c->key_dim;
        L.Dv = (uint32_t)c->value_dim;
        L.scale = 1.0f / std::sqrt((float)c->key_dim);  // reference_kernels.cpp:158
        L.keys = c->keys;
        L.values = c->values;
        L.f16 = c->type == OQ_TYPE_F16;
        return OQ_OK;
    }
    uint32_t chunk = 0, nchunks = 0;
    oq::attention_plan(T, c->kv_heads, rep, chunk, nchunks, token_groups);
    if (nchunks > oq::kAttnMaxChunks || T > 0xFFFFFFFFull || c->kv_heads > 0xFFFF) {
        return fail(ctx, OQ_INVALID_ARGUMENT, "attention device path supports at most 8388608 cached tokens");
    }
    L.T = (uint32_t)T;
    L.Hkv = (uint32_t)c->kv_heads;
    L.rep = (uint32_t)rep;
    L.D = (uint32_t)c->key_dim;
    L.chunk = chunk;
    L.nchunks = nchunks;
    L.scale = 1.0f / std::sqrt((float)c->key_dim);  // reference_kernels.cpp:158
    L.keys = c->keys;
    L.values = c->values;
    L.f16 = c->type == OQ_TYPE_F16;
    return OQ_OK;
}

// The attention launch's scratch: the chunks' partial sums, or the any-shape kernels' scores
uint64_t attention_scratch_floats(const oq::AttnLaunch& L) {
    return L.any ? oq::attention_any_floats((uint64_t)L.Hkv * L.rep, L.T)
                 : oq::attention_partial_floats(L.Hkv, L.rep, L.D, L.nchunks);
}

// Workspace of one attention block step: the 15 trace fields, the normalised input and the
// attention scratch (P floats), each padded to 64 floats.
struct AttnLayout {
    uint64_t sizes[17];
    uint64_t off[17];
    uint64_t total_floats;
};

AttnLayout attn_layout(const oq_attention_block* b, uint64_t P) {
    const uint64_t E = b->embedding, D = b->head_dim, F = b->ffn, Q = b->q_heads * D, KV = b->kv_heads * D;
    AttnLayout l{{2 * Q, KV, KV, Q, KV, Q, Q, Q, E, E, E, F, F, F, E, E, P}, {}, 0};
    for (int i = 0; i < 17; ++i) {
        l.off[i] = l.total_floats;
        l.total_floats += (l.sizes[i] + 63) & ~uint64_t(63);
    }
    return l;
}

int check_attn_weight(oq_context* ctx, const oq_weight* w, uint64_t ne0, uint64_t ne1, const char* name) {
    if (int rc = check_weight(ctx, w)) return fail(ctx, rc, std::string("attention block weight ") + name + ": " + ctx->error);
    if (w->m.k != ne0 || w->m.n != ne1) {
        return fail(ctx, OQ_INVALID_ARGUMENT,
                    std::string("attention block weight ") + name + " has shape [" + std::to_string(w->m.k) + ", " +
                        std::to_string(w->m.n) + "], expected [" + std::to_string(ne0) + ", " + std::to_string(ne1) + "]");
    }
    return OQ_OK;
}

}  // namespace

extern "C" {

int oq_kv_cache_create(oq_context* ctx, uint64_t capacity, uint64_t kv_heads, uint64_t key_dim, uint64_t value_dim,
                       oq_kv_cache** out) {
    return oq_kv_cache_create_typed(ctx, capacity, kv_heads, key_dim, value_dim, OQ_TYPE_F32, out);
}

int oq_kv_cache_create_typed(oq_context* ctx, uint64_t capacity, uint64_t kv_heads, uint64_t key_dim,
                             uint64_t value_dim, uint32_t type, oq_kv_cache** out) {
    if (!ctx) return fail(nullptr, OQ_INVALID_ARGUMENT, "null context");
    if (!out) return fail(ctx, OQ_INVALID_ARGUMENT, "null output handle");
    *out = nullptr;
    // KvCache::KvCache (hybrid_cache.cpp:131-152)
    if (capacity == 0) return fail(ctx, OQ_INVALID_ARGUMENT, "KV cache capacity must be non-zero");
    if (kv_heads == 0) return fail(ctx, OQ_INVALID_ARGUMENT, "KV head count must be non-zero");
    if (key_dim == 0) return fail(ctx, OQ_INVALID_ARGUMENT, "KV key dimension must be non-zero");
    if (value_dim == 0) return fail(ctx, OQ_INVALID_ARGUMENT, "KV value dimension must be non-zero");
    if (type != OQ_TYPE_F32 && type != OQ_TYPE_F16) {
        return fail(ctx, OQ_INVALID_ARGUMENT, "KV cache element type must be F32 or F16");
    }
    const uint64_t es = type == OQ_TYPE_F16 ? 2 : 4;
    const uint64_t lim = UINT64_MAX / es;
    if (kv_heads > lim / capacity || key_dim > lim / (capacity * kv_heads) ||
        value_dim > lim / (capacity * kv_heads)) {
        return fail(ctx, OQ_OVERFLOW, "KV cache size overflow");
    }
    if (capturing_now(ctx)) return fail(ctx, OQ_INVALID_ARGUMENT, "a KV cache cannot be created during graph capture");
    const uint64_t kb = capacity * kv_heads * key_dim * es;
    const uint64_t vb = capacity * kv_heads * value_dim * es;
    OQ_HIP(ctx, hipSetDevice(ctx->device), "hipSetDevice");
    oq_kv_cache* c = new oq_kv_cache;
    c->ctx = ctx;
    c->device = ctx->device;
    c->type = type;
    c->capacity = capacity;
    c->kv_heads = kv_heads;
    c->key_dim = key_dim;
    c->value_dim = value_dim;
    hipError_t e = hipMalloc(&c->keys, kb);
    if (e == hipSuccess) e = hipMalloc(&c->values, vb);
    if (e == hipSuccess) e = hipMemsetAsync(c->keys, 0, kb, ctx->stream);
    if (e == hipSuccess) e = hipMemsetAsync(c->values, 0, vb, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) {
        const int rc = hip_fail(ctx, e, "KV cache allocation");
        oq_kv_cache_release(c);
        return rc;
    }
    *out = c;
    return OQ_OK;
}

void oq_kv_cache_release(oq_kv_cache* c) {
    if (!c) return;
    (void)hipSetDevice(c->device);
    if (c->ctx && c->ctx->stream) (void)hipStreamSynchronize(c->ctx->stream);
    if (c->keys) (void)hipFree(c->keys);
    if (c->values) (void)hipFree(c->values);
    delete c;
}

uint64_t oq_kv_cache_size(const oq_kv_cache* c) { return c ? c->length : 0; }
uint64_t oq_kv_cache_capacity(const oq_kv_cache* c) { return c ? c->capacity : 0; }

int oq_kv_cache_reset(oq_kv_cache* c) {
    if (!c) return fail(nullptr, OQ_INVALID_ARGUMENT, "null KV cache");
    oq_context* ctx = c->ctx;
    if (capturing_now(ctx)) return fail(ctx, OQ_INVALID_ARGUMENT, "a KV cache cannot be reset during graph capture");
    c->length = 0;
    OQ_HIP(ctx, hipMemsetAsync(c->keys, 0, c->capacity * c->kv_heads * c->key_dim * c->element_bytes(), ctx->stream),
           "KV cache reset");
    OQ_HIP(ctx, hipMemsetAsync(c->values, 0, c->capacity * c->kv_heads * c->value_dim * c->element_bytes(), ctx->stream),
           "KV cache reset");
    return OQ_OK;
}

int oq_kv_cache_truncate(oq_kv_cache* c, uint64_t new_length) {
    if (!c) return fail(nullptr, OQ_INVALID_ARGUMENT, "null KV cache");
    if (new_length > c->length) return fail(c->ctx, OQ_INVALID_ARGUMENT, "KV cache truncate must not grow state");
    c->length = new_length;
    return OQ_OK;
}

int oq_kv_cache_load(oq_kv_cache* c, const float* keys, const float* values, uint64_t length) {
    if (!c) return fail(nullptr, OQ_INVALID_ARGUMENT, "null KV cache");
    oq_context* ctx = c->ctx;
    if (length > c->capacity) return fail(ctx, OQ_OVERFLOW, "KV cache capacity exceeded");
    if (length > 0 && (!keys || !values)) return fail(ctx, OQ_INVALID_ARGUMENT, "null cache rows");
    if (capturing_now(ctx)) return fail(ctx, OQ_INVALID_ARGUMENT, "a KV cache cannot be loaded during graph capture");
    if (length > 0 && c->type == OQ_TYPE_F32) {
        OQ_HIP(ctx, hipMemcpyAsync(c->keys, keys, length * c->kv_heads * c->key_dim * sizeof(float),
                                   hipMemcpyHostToDevice, ctx->stream), "KV cache load");
        OQ_HIP(ctx, hipMemcpyAsync(c->values, values, length * c->kv_heads * c->value_dim * sizeof(float),
                                   hipMemcpyHostToDevice, ctx->stream), "KV cache load");
        OQ_HIP(ctx, hipStreamSynchronize(ctx->stream), "KV cache load");
    } else if (length > 0) {
        // F16: the F32 rows go through a bounded device staging buffer and are rounded on the device
        // (the rounding of the attention steps' appends)
        const uint64_t total[2] = {length * c->kv_heads * c->key_dim, length * c->kv_heads * c->value_dim};
        const float* src[2] = {keys, values};
        _Float16* dst[2] = {static_cast<_Float16*>(c->keys), static_cast<_Float16*>(c->values)};
        const uint64_t chunk = std::min<uint64_t>(std::max(total[0], total[1]), uint64_t(16) << 20);  // floats
        void* staging = nullptr;
        OQ_HIP(ctx, hipMalloc(&staging, chunk * sizeof(float)), "KV cache load staging");
        hipError_t e = hipSuccess;
        for (int a = 0; a < 2 && e == hipSuccess; ++a) {
            for (uint64_t off = 0; off < total[a] && e == hipSuccess; off += chunk) {
                const uint64_t n = std::min(chunk, total[a] - off);
                e = hipMemcpyAsync(staging, src[a] + off, n * sizeof(float), hipMemcpyHostToDevice, ctx->stream);
                if (e == hipSuccess) e = oq::launch_f32_to_f16(static_cast<const float*>(staging), dst[a] + off, n, ctx->stream);
            }
        }
        if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
        (void)hipFree(staging);
        if (e != hipSuccess) return hip_fail(ctx, e, "KV cache load");
    }
    c->length = length;
    return OQ_OK;
}

int oq_kv_cache_arrays(const oq_kv_cache* c, float** keys_dev, float** values_dev) {
    if (!c) return fail(nullptr, OQ_INVALID_ARGUMENT, "null KV cache");
    if (keys_dev) *keys_dev = static_cast<float*>(c->keys);
    if (values_dev) *values_dev = static_cast<float*>(c->values);
    return OQ_OK;
}

uint32_t oq_kv_cache_type(const oq_kv_cache* c) { return c ? c->type : 0; }

int oq_rope(oq_context* ctx, float* heads, uint64_t n_heads, uint64_t head_dim, uint64_t rotary_dim,
            const int32_t sections[4], float base, const uint64_t position[3]) {
    if (!ctx) return fail(nullptr, OQ_INVALID_ARGUMENT, "null context");
    oq::RopeParams p{};
    if (int rc = rope_params(ctx, head_dim, rotary_dim, sections, base, position, p)) return rc;
    if (n_heads == 0) return OQ_OK;
    if (!heads) return fail(ctx, OQ_INVALID_ARGUMENT, "null heads");
    if (!aligned(heads, 4)) return fail(ctx, OQ_INVALID_ARGUMENT, "misaligned buffer");
    if (n_heads > 0x7FFFFFFF || head_dim > 0xFFFFFFFFull) return fail(ctx, OQ_OVERFLOW, "RoPE tensor too large");
    oq::RopeTable t;
    oq::rope_table(p, t);
    return launch_rc(ctx, oq::launch_rope(heads, n_heads, head_dim, p, t, ctx->stream), "rope");
}

int oq_attention_step(oq_context* ctx, const float* q, uint64_t q_heads, const float* k, const float* v,
                      oq_kv_cache* cache, float* out) {
    if (!ctx) return fail(nullptr, OQ_INVALID_ARGUMENT, "null context");
    if (int rc = check_cache(ctx, cache)) return rc;
    if (!q || !k || !v || !out) return fail(ctx, OQ_INVALID_ARGUMENT, "null argument");
    // causal_attention_step (reference_kernels.cpp:139-150), then KvCache::append's capacity check
    if (q_heads == 0 || q_heads % cache->kv_heads != 0) {
        return fail(ctx, OQ_INVALID_ARGUMENT, "causal_attention_step dimensions are incompatible");
    }
    if (cache->length >= cache->capacity) return fail(ctx, OQ_OVERFLOW, "KV cache capacity exceeded");
    oq::AttnLaunch L{};
    if (int rc = attention_shape(ctx, cache, q_heads, L)) return rc;
    if (!aligned(q, 16) || !aligned(k, 16) || !aligned(v, 16) || !aligned(out, 16)) {
        return fail(ctx, OQ_INVALID_ARGUMENT, "attention buffers must be 16-byte aligned");
    }
    const uint64_t pf = attention_scratch_floats(L);
    if (int rc = ensure_scratch(ctx, pf * sizeof(float))) return rc;
    L.q = q;
    L.new_k = k;
    L.new_v = v;
    L.part = static_cast<float*>(ctx->scratch.ptr);
    L.out = out;
    const int rc = launch_rc(ctx, oq::launch_attention(L, ctx->stream), "attention_step");
    if (rc == OQ_OK) cache->length += 1;
    return rc;
}

// oq_attention_block_step with x aligned to x_align bytes (16 through the C ABI; 4 for the token rows
// of a several-token call on the any-shape kernels, whose embedding need not be a multiple of 4)
static int attention_block_step_core(oq_context* ctx, const oq_attention_block* b, oq_kv_cache* cache,
                                     const uint64_t position[3], const float* x, float* y, float* trace,
                                     uint64_t x_align) {
    if (!ctx) return fail(nullptr, OQ_INVALID_ARGUMENT, "null context");
    if (!b || !x || !y) return fail(ctx, OQ_INVALID_ARGUMENT, "null argument");
    if (int rc = check_cache(ctx, cache)) return rc;
    const uint64_t E = b->embedding, Hq = b->q_heads, Hkv = b->kv_heads, D = b->head_dim, F = b->ffn;
    if (E == 0 || Hq == 0 || Hkv == 0 || D == 0 || F == 0 || Hq % Hkv != 0) {
        return fail(ctx, OQ_INVALID_ARGUMENT, "Qwen3.5 attention block dimensions are incompatible");
    }
    // execute_qwen35_attention_block_reference (qwen35_block.cpp:621-625)
    if (cache->kv_heads != Hkv || cache->key_dim != D || cache->value_dim != D) {
        return fail(ctx, OQ_INVALID_ARGUMENT, "Qwen3.5 attention cache dimensions do not match the manifest");
    }
    if (!(b->eps > 0.0f) || !std::isfinite(b->eps)) {
        return fail(ctx, OQ_INVALID_ARGUMENT, "Qwen3.5 RMSNorm epsilon must be positive and finite");
    }
    oq::RopeParams rp{};
    if (int rc = rope_params(ctx, D, b->rope_dim, b->rope_sections, b->rope_base, position, rp)) return rc;
    if (E > 0x7FFFFFFF || F > 0x7FFFFFFF || Hq * D > 0x7FFFFFFF) return fail(ctx, OQ_OVERFLOW, "block too large");
    const uint64_t Q = Hq * D, KV = Hkv * D;
    if (int rc = check_attn_weight(ctx, b->q, E, 2 * Q, "q")) return rc;
    if (int rc = check_attn_weight(ctx, b->k, E, KV, "k")) return rc;
    if (int rc = check_attn_weight(ctx, b->v, E, KV, "v")) return rc;
    if (int rc = check_attn_weight(ctx, b->out, Q, E, "out")) return rc;
    if (int rc = check_attn_weight(ctx, b->gate, E, F, "gate")) return rc;
    if (int rc = check_attn_weight(ctx, b->up, E, F, "up")) return rc;
    if (int rc = check_attn_weight(ctx, b->down, F, E, "down")) return rc;
    if (!b->input_norm || !b->q_norm || !b->k_norm || !b->post_norm) {
        return fail(ctx, OQ_INVALID_ARGUMENT, "null block vector");
    }
    if (!aligned(x, x_align) || !aligned(y, 4)) return fail(ctx, OQ_INVALID_ARGUMENT, "misaligned buffer");
    if (cache->length >= cache->capacity) return fail(ctx, OQ_OVERFLOW, "KV cache capacity exceeded");
    oq::AttnLaunch L{};
    if (int rc = attention_shape(ctx, cache, Hq, L)) return rc;
    const AttnLayout lay = attn_layout(b, attention_scratch_floats(L));
    if (int rc = ensure_work(ctx, lay.total_floats * sizeof(float))) return rc;
    float* ws = static_cast<float*>(ctx->work.ptr);
    const uint64_t* off = lay.off;
    float *qfull = ws + off[0], *kp = ws + off[1], *vp = ws + off[2], *qcur = ws + off[3], *kcur = ws + off[4],
          *pregate = ws + off[5], *gate_s = ws + off[6], *gated = ws + off[7], *branch = ws + off[8],
          *resid = ws + off[9], *post = ws + off[10], *gate = ws + off[11], *up = ws + off[12], *act = ws + off[13],
          *ffn = ws + off[14], *normed = ws + off[15], *part = ws + off[16];
    hipStream_t s = ctx->stream;
    hipError_t e = hipSuccess;

    oq::BlockGemv in{}, outp{}, ffn_in{}, down{};
    in.nmat = 3;
    in.mat[0] = b->q->m;
    in.mat[1] = b->k->m;
    in.mat[2] = b->v->m;
    in.row_end[0] = (uint32_t)(2 * Q);
    in.row_end[1] = (uint32_t)(2 * Q + KV);
    in.row_end[2] = (uint32_t)(2 * Q + 2 * KV);
    in.x = x;
    in.norm_w = b->input_norm;
    in.eps = b->eps;
    in.raw[0] = qfull;
    in.raw[1] = kp;
    in.raw[2] = vp;
    outp.nmat = 1;
    outp.mat[0] = b->out->m;
    outp.row_end[0] = (uint32_t)E;
    outp.x = gated;
    outp.raw[0] = trace ? branch : nullptr;  // raw outputs and per-head copies: only the trace reads them
    outp.add = x;
    outp.sum_out = resid;
    ffn_in.nmat = 2;
    ffn_in.mat[0] = b->gate->m;
    ffn_in.mat[1] = b->up->m;
    ffn_in.row_end[0] = (uint32_t)F;
    ffn_in.row_end[1] = (uint32_t)(2 * F);
    ffn_in.x = resid;
    ffn_in.norm_w = b->post_norm;
    ffn_in.eps = b->eps;
    ffn_in.norm_out = trace ? post : nullptr;
    ffn_in.raw[0] = trace ? gate : nullptr;
    ffn_in.raw[1] = trace ? up : nullptr;
    ffn_in.act = act;
    down.nmat = 1;
    down.mat[0] = b->down->m;
    down.row_end[0] = (uint32_t)E;
    down.x = act;
    down.raw[0] = trace ? ffn : nullptr;
    down.add = resid;
    down.sum_out = y;

    oq::AttnPrep prep{};
    prep.qfull = qfull;
    prep.kp = kp;
    prep.vp = vp;
    prep.q_norm = b->q_norm;
    prep.k_norm = b->k_norm;
    prep.eps = b->eps;
    prep.rope = rp;
    // the any-shape preparation rotates by the host's table; the chunk kernel computes its angles
    // itself (a table in its arguments measured slower: 52.5 against 51.8 us per block)
    if (L.any) oq::rope_table(rp, prep.table);
    prep.qcur = trace || L.any ? qcur : nullptr;  // the any-shape attention reads the rotated queries from there
    prep.kcur = trace ? kcur : nullptr;
    L.prep = &prep;
    L.part = part;
    L.out = trace ? pregate : nullptr;
    L.gate = qfull + D;
    L.gate_stride = (uint32_t)(2 * D);
    L.gate_s = trace ? gate_s : nullptr;
    L.gated = gated;

    const bool even = E % 2 == 0 && F % 2 == 0;
    const bool fused_in = knob_flag(oq::kBlockFused, true) && even && aligned(x, 16) && oq::gemv_block_supported(in);
    const bool fused_tail = knob_flag(oq::kBlockFused, true) && even && oq::gemv_block_supported(outp) &&
                            oq::gemv_block_supported(ffn_in) && oq::gemv_block_supported(down);
    if (fused_in) {
        if (cache->type == OQ_TYPE_F16) {
            // the projection stores the new value row of an F16 cache itself (no append launch)
            in.v16 = static_cast<_Float16*>(cache->values) + cache->length * Hkv * D;
            prep.v_stored = true;
        }
        e = oq::launch_gemv_block(oq::kBlockIn, in, s);
    } else {
        e = oq::launch_rmsnorm(x, nullptr, b->input_norm, E, b->eps, nullptr, normed, s);
        if (e == hipSuccess) e = block_project(b->q, normed, qfull, s);
        if (e == hipSuccess) e = block_project(b->k, normed, kp, s);
        if (e == hipSuccess) e = block_project(b->v, normed, vp, s);
    }
    if (e == hipSuccess) e = oq::launch_attention(L, s);
    if (fused_tail) {
        if (e == hipSuccess) e = oq::launch_gemv_block(oq::kBlockAdd, outp, s);
        if (e == hipSuccess) e = oq::launch_gemv_block(oq::kBlockFfn, ffn_in, s);
        if (e == hipSuccess) e = oq::launch_gemv_block(oq::kBlockAdd, down, s);
    } else {
        if (e == hipSuccess) e = block_project(b->out, gated, branch, s);
        if (e == hipSuccess) e = oq::launch_rmsnorm(x, branch, b->post_norm, E, b->eps, resid, post, s);
        if (e == hipSuccess) e = block_project(b->gate, post, gate, s);
        if (e == hipSuccess) e = block_project(b->up, post, up, s);
        if (e == hipSuccess) e = oq::launch_swiglu(gate, up, F, act, s);
        if (e == hipSuccess) e = block_project(b->down, act, ffn, s);
        if (e == hipSuccess) e = oq::launch_add(resid, ffn, E, y, s);
    }
    if (e == hipSuccess && trace) {
        uint64_t t = 0;
        for (int i = 0; i < 15 && e == hipSuccess; ++i) {
            e = hipMemcpyAsync(trace + t, ws + off[i], lay.sizes[i] * sizeof(float), hipMemcpyDeviceToDevice, s);
            t += lay.sizes[i];
        }
    }
    const int rc = launch_rc(ctx, e, "attention_block_step");
    if (rc == OQ_OK) cache->length += 1;
    return rc;
}

int oq_attention_block_step(oq_context* ctx, const oq_attention_block* b, oq_kv_cache* cache,
                            const uint64_t position[3], const float* x, float* y, float* trace) {
    return attention_block_step_core(ctx, b, cache, position, x, y, trace, 16);
}

int oq_attention_block_steps(oq_context* ctx, const oq_attention_block* b, oq_kv_cache* cache, uint64_t m,
                             const uint64_t* positions, const float* x, float* y, float* trace) {
    if (!ctx) return fail(nullptr, OQ_INVALID_ARGUMENT, "null context");
    if (!b || !x || !y || !positions) return fail(ctx, OQ_INVALID_ARGUMENT, "null argument");
    if (int rc = check_cache(ctx, cache)) return rc;
    if (m == 0) return fail(ctx, OQ_INVALID_ARGUMENT, "token count must be non-zero");
    if (m > 0xFFFF) return fail(ctx, OQ_INVALID_ARGUMENT, "at most 65535 tokens per call");
    const uint64_t E = b->embedding, Hq = b->q_heads, Hkv = b->kv_heads, D = b->head_dim, F = b->ffn;
    if (E == 0 || Hq == 0 || Hkv == 0 || D == 0 || F == 0 || Hq % Hkv != 0) {
        return fail(ctx, OQ_INVALID_ARGUMENT, "Qwen3.5 attention block dimensions are incompatible");
    }
    if (cache->kv_heads != Hkv || cache->key_dim != D || cache->value_dim != D) {
        return fail(ctx, OQ_INVALID_ARGUMENT, "Qwen3.5 attention cache dimensions do not match the manifest");
    }
    if (!(b->eps > 0.0f) || !std::isfinite(b->eps)) {
        return fail(ctx, OQ_INVALID_ARGUMENT, "Qwen3.5 RMSNorm epsilon must be positive and finite");
    }
    std::vector<oq::RopeParams> rps(m);
    for (uint64_t t = 0; t < m; ++t) {
        if (int rc = rope_params(ctx, D, b->rope_dim, b->rope_sections, b->rope_base, positions + 3 * t, rps[t])) return rc;
    }
    const uint64_t Q = Hq * D, KV = Hkv * D;
    if (m * std::max({E, F, 2 * Q}) > 0x7FFFFFFF) return fail(ctx, OQ_OVERFLOW, "block too large");
    if (int rc = check_attn_weight(ctx, b->q, E, 2 * Q, "q")) return rc;
    if (int rc = check_attn_weight(ctx, b->k, E, KV, "k")) return rc;
    if (int rc = check_attn_weight(ctx, b->v, E, KV, "v")) return rc;
    if (int rc = check_attn_weight(ctx, b->out, Q, E, "out")) return rc;
    if (int rc = check_attn_weight(ctx, b->gate, E, F, "gate")) return rc;
    if (int rc = check_attn_weight(ctx, b->up, E, F, "up")) return rc;
    if (int rc = check_attn_weight(ctx, b->down, F, E, "down")) return rc;
    if (!b->input_norm || !b->q_norm || !b->k_norm || !b->post_norm) {
        return fail(ctx, OQ_INVALID_ARGUMENT, "null block vector");
    }
    if (!aligned(x, 16) || !aligned(y, 4) || (trace && !aligned(trace, 4))) {
        return fail(ctx, OQ_INVALID_ARGUMENT, "misaligned buffer (x 16-byte, others 4-byte)");
    }
    if (cache->capacity - cache->length < m) return fail(ctx, OQ_OVERFLOW, "KV cache capacity exceeded");
    if (!attention_fast(cache, Hq)) {
        // shapes outside the chunked kernels: the single step token by token (token t's trace at
        // trace + t * the single step's trace size, as below)
        const uint64_t per_token = 2 * Q + KV + KV + Q + KV + Q + Q + Q + E + E + E + F + F + F + E;
        for (uint64_t t = 0; t < m; ++t) {
            if (int rc = attention_block_step_core(ctx, b, cache, positions + 3 * t, x + t * E, y + t * E,
                                                   trace ? trace + t * per_token : nullptr, 4))
                return rc;
        }
        return OQ_OK;
    }
    // the attention of all m tokens in one chunk launch, shaped for the last token (its chunks lay
    // out every token's partials); a grid too large for one launch runs the tokens one by one
    // the chunks sized so that the launch's workgroups over all token groups fill the GPU about as
    // one token's do
    oq::AttnLaunch last{};
    const uint64_t tpw = oq::attention_tokens_per_workgroup(cache->length + m, Hq / Hkv, m);
    if (int rc = attention_shape(ctx, cache, Hq, last, m - 1, (m + tpw - 1) / tpw)) return rc;
    const uint64_t part_last = oq::attention_partial_floats(Hkv, Hq / Hkv, D, last.nchunks);
    const bool batched = m * Hkv * oq::attention_subgroups((uint32_t)(Hq / Hkv)) * last.nchunks <= 0x7FFFFFFFull;
    std::vector<oq::AttnLaunch> Ls;
    uint64_t part_floats = batched ? m * part_last : 0;
    if (!batched) {
        Ls.resize(m);
        for (uint64_t t = 0; t < m; ++t) {
            if (int rc = attention_shape(ctx, cache, Hq, Ls[t], t)) return rc;
            part_floats = std::max(part_floats, oq::attention_partial_floats(Hkv, Hq / Hkv, D, Ls[t].nchunks));
        }
    }
    // workspace: the 15 trace fields with m rows each, the normalised input, the partial sums, one
    // Q8_K image (m rows of the widest projection input) and the tokens' positions
    const uint64_t row[16] = {2 * Q, KV, KV, Q, KV, Q, Q, Q, E, E, E, F, F, F, E, E};
    uint64_t off[19], total = 0;
    for (int i = 0; i < 16; ++i) {
        off[i] = total;
        total += (m * row[i] + 63) & ~uint64_t(63);
    }
    off[16] = total;
    total += (part_floats + 63) & ~uint64_t(63);
    off[17] = total;
    total += (m * (std::max({E, Q, F}) / oq::kQK) * oq::kQ8KBytes / sizeof(float) + 64) & ~uint64_t(63);
    off[18] = total;
    total += (m * 3 * sizeof(uint64_t) / sizeof(float) + 63) & ~uint64_t(63);
    if (int rc = ensure_work(ctx, total * sizeof(float))) return rc;
    uint64_t scratch = 0;
    for (const oq_weight* w : {b->q, b->k, b->v, b->out, b->gate, b->up, b->down}) {
        if (on_matrix_cores(w, m, true)) scratch = std::max(scratch, oq::gemm_scratch_bytes(w->m, (int)m));
    }
    if (scratch > 0) {
        if (int rc = ensure_scratch(ctx, scratch)) return rc;
    }
    float* ws = static_cast<float*>(ctx->work.ptr);
    float *qfull = ws + off[0], *kp = ws + off[1], *vp = ws + off[2], *qcur = ws + off[3], *kcur = ws + off[4],
          *pregate = ws + off[5], *gate_s = ws + off[6], *gated = ws + off[7], *branch = ws + off[8],
          *resid = ws + off[9], *post = ws + off[10], *gate = ws + off[11], *up = ws + off[12], *act = ws + off[13],
          *ffn = ws + off[14], *normed = ws + off[15], *part = ws + off[16];
    uint8_t* q8 = reinterpret_cast<uint8_t*>(ws + off[17]);
    uint64_t* pos_dev = reinterpret_cast<uint64_t*>(ws + off[18]);
    hipStream_t s = ctx->stream;
    auto quantize = [&](const float* in, uint64_t k, std::initializer_list<const oq_weight*> consumers) {
        for (const oq_weight* w : consumers)
            if (needs_q8(w, m)) return oq::launch_quantize_q8k(in, m, k, q8, s);
        return hipSuccess;
    };
    // the Q8_K image an input's producer writes beside it, when a projection of it takes the
    // small-batch GEMV (null: none does)
    auto q8_for = [&](std::initializer_list<const oq_weight*> consumers) -> uint8_t* {
        for (const oq_weight* w : consumers)
            if (needs_q8(w, m)) return q8;
        return nullptr;
    };
    hipError_t e = hipSuccess;
    // the tokens' positions: launch arguments for a few tokens, else a copy to the device
    const bool pos_inline = m <= oq::kInlineTokenPositions;
    if (batched && !pos_inline) e = hipMemcpyAsync(pos_dev, positions, m * 3 * sizeof(uint64_t), hipMemcpyHostToDevice, s);
    if (e == hipSuccess)
        e = norm_project_set(ctx, {{b->q, qfull}, {b->k, kp}, {b->v, vp}}, m, x, nullptr, b->input_norm, b->eps, E,
                             nullptr, normed, false, q8);
    // the tokens' heads prepared together (token t's key and value appended at row length + t),
    // then token t attending over the rows up to its own, all tokens in one chunk and one merge
    // launch; or, when that grid is too large, the single step's launch token by token
    if (batched && e == hipSuccess) {
        oq::AttnTokens tk{};
        tk.tokens = (uint32_t)m;
        tk.qfull = qfull;
        tk.kp = kp;
        tk.vp = vp;
        tk.q_norm = b->q_norm;
        tk.k_norm = b->k_norm;
        tk.eps = b->eps;
        tk.rope = rps[0];
        tk.positions = pos_inline ? nullptr : pos_dev;
        tk.positions_host = pos_inline ? positions : nullptr;
        tk.qcur = qcur;
        tk.kcur = trace ? kcur : nullptr;
        tk.gate_tok_stride = 2 * Q;
        last.part = part;
        last.out = trace ? pregate : nullptr;
        last.gate = qfull + D;
        last.gate_stride = (uint32_t)(2 * D);
        last.gate_s = trace ? gate_s : nullptr;
        last.gated = gated;
        e = oq::launch_attention_tokens(last, tk, s);
    }
    for (uint64_t t = 0; !batched && t < m && e == hipSuccess; ++t) {
        oq::AttnPrep prep{};
        prep.qfull = qfull + t * 2 * Q;
        prep.kp = kp + t * KV;
        prep.vp = vp + t * KV;
        prep.q_norm = b->q_norm;
        prep.k_norm = b->k_norm;
        prep.eps = b->eps;
        prep.rope = rps[t];
        prep.qcur = trace ? qcur + t * Q : nullptr;
        prep.kcur = trace ? kcur + t * KV : nullptr;
        oq::AttnLaunch& L = Ls[t];
        L.prep = &prep;
        L.part = part;
        L.out = trace ? pregate + t * Q : nullptr;
        L.gate = qfull + t * 2 * Q + D;
        L.gate_stride = (uint32_t)(2 * D);
        L.gate_s = trace ? gate_s + t * Q : nullptr;
        L.gated = gated + t * Q;
        e = oq::launch_attention(L, s);
    }
    // the out projection: at two tokens its staging quantizes the gated rows itself (each
    // workgroup, 32 KB of rows), cheaper than the quantization launch it replaces; same bits
    if (e == hipSuccess && m == 2 && needs_q8(b->out, m) && knob_flag(oq::kBlockFused, true)) {
        e = oq::launch_gemv_kquant(b->out->m, (int)m, gated, nullptr, branch, s);
    } else {
        if (e == hipSuccess) e = quantize(gated, Q, {b->out});
        if (e == hipSuccess) e = project_rows(ctx, b->out, m, gated, q8, branch);
    }
    if (e == hipSuccess)
        e = norm_project_set(ctx, {{b->gate, gate}, {b->up, up}}, m, x, branch, b->post_norm, b->eps, E, resid, post,
                             trace != nullptr, q8);
    if (e == hipSuccess) e = oq::launch_swiglu(gate, up, m * F, act, s, q8_for({b->down}));
    if (e == hipSuccess && trace) {
        e = project_rows(ctx, b->down, m, act, q8, ffn);  // the trace keeps the down projection
        if (e == hipSuccess) e = oq::launch_add(resid, ffn, m * E, y, s);
    } else if (e == hipSuccess) {
        e = project_add(ctx, b->down, m, act, q8, resid, ffn, y);
    }
    if (e == hipSuccess && trace) {
        // token t's trace (oq_attention_block_step's 15 fields, in order) at trace + t * size
        uint64_t per_token = 0;
        for (int i = 0; i < 15; ++i) per_token += row[i];
        uint64_t t = 0;
        for (int i = 0; i < 15 && e == hipSuccess; ++i) {
            e = hipMemcpy2DAsync(trace + t, per_token * sizeof(float), ws + off[i], row[i] * sizeof(float),
                                 row[i] * sizeof(float), m, hipMemcpyDeviceToDevice, s);
            t += row[i];
        }
    }
    const int rc = launch_rc(ctx, e, "attention_block_steps");
    if (rc == OQ_OK) cache->length += m;
    return rc;
}

}  // extern "C"
