// ORACLE -- test infrastructure, not product code.
//
// A C-callable shim over the reference engine's own quantized path and Qwen3.5 block kernels,
// compiled together with the reference's sources (ggml_type.cpp, storage_decode.cpp,
// quantized_reference.cpp, the GgufTensorView they take, reference_kernels.cpp, qwen35_block.cpp
// and what they link) into oracle/_ref/libref.so by oracle/Makefile.  It lets the tests
// compare the C restatement (oracle.c) with the reference itself, bit for bit, and lets the
// benchmark time the reference's CPU path.  Exceptions are caught and returned as the same
// status codes the restatement uses.
#include "oracle/backend/cpu/quantized_reference.hpp"
#include "oracle/model/ggml_type.hpp"
#include "oracle/model/gguf.hpp"
#include "oracle/model/mapped_gguf.hpp"
#include "oracle/model/storage_decode.hpp"
#include "oracle/core/tensor.hpp"
#include "oracle/runtime/hybrid_cache.hpp"
#include "oracle/runtime/reference_kernels.hpp"
#include "oracle/runtime/qwen35_block.hpp"
#include "oracle/model/qwen35_weights.hpp"

#include <cstdio>
#include <cstring>
#include <exception>
#include <span>
#include <stdexcept>
#include <string>
#include <vector>

namespace {

thread_local std::string g_error;

template <typename F>
int guarded(F&& f) {
    try {
        f();
        return 0;
    } catch (const std::out_of_range& e) {
        g_error = e.what();
        return -2;
    } catch (const std::overflow_error& e) {
        g_error = e.what();
        return -3;
    } catch (const std::invalid_argument& e) {
        g_error = e.what();
        return -1;
    } catch (const std::logic_error& e) {
        g_error = e.what();
        return -5;
    } catch (const std::runtime_error& e) {
        g_error = e.what();
        return -4;
    } catch (const std::exception& e) {
        g_error = e.what();
        return -6;
    }
}

std::span<const std::byte> as_bytes(const void* p, std::uint64_t n) {
    return {static_cast<const std::byte*>(p), static_cast<std::size_t>(n)};
}

}  // namespace

extern "C" {

const char* ref_last_error() { return g_error.c_str(); }

float ref_f16_to_f32(std::uint16_t bits) { return oracle::model::f16_to_f32(bits); }
float ref_bf16_to_f32(std::uint16_t bits) { return oracle::model::bf16_to_f32(bits); }

int ref_type_layout(std::uint32_t type, std::uint64_t* block_elements,
                    std::uint64_t* bytes_per_block, int* quantized, char* name, int name_cap) {
    const auto* layout = oracle::model::ggml_type_layout(type);
    if (layout == nullptr) {
        g_error = "unregistered";
        return -4;
    }
    *block_elements = layout->block_elements;
    *bytes_per_block = layout->bytes_per_block;
    *quantized = layout->quantized ? 1 : 0;
    std::snprintf(name, static_cast<std::size_t>(name_cap), "%.*s",
                  static_cast<int>(layout->name.size()), layout->name.data());
    return 0;
}

int ref_row_byte_size(std::uint64_t row_elements, std::uint32_t type, std::uint64_t* out) {
    return guarded([&] { *out = oracle::model::ggml_row_byte_size(row_elements, type); });
}

int ref_decode_row(std::uint32_t type, std::uint64_t n, const void* bytes, std::uint64_t nbytes,
                   float* out, std::uint64_t out_len) {
    return guarded([&] {
        oracle::model::decode_storage_row(
            oracle::model::make_storage_row_view(type, static_cast<std::size_t>(n),
                                                 as_bytes(bytes, nbytes)),
            std::span<float>(out, static_cast<std::size_t>(out_len)));
    });
}

int ref_storage_dot(std::uint32_t type, std::uint64_t n, const void* bytes, std::uint64_t nbytes,
                    const float* x, std::uint64_t x_len, float* out) {
    return guarded([&] {
        *out = oracle::backend::cpu::reference_storage_dot(
            oracle::model::make_storage_row_view(type, static_cast<std::size_t>(n),
                                                 as_bytes(bytes, nbytes)),
            std::span<const float>(x, static_cast<std::size_t>(x_len)));
    });
}

int ref_storage_matvec(std::uint32_t type, std::uint64_t rows, std::uint64_t cols,
                       const void* matrix, std::uint64_t nbytes, const float* x,
                       std::uint64_t x_len, float* y, std::uint64_t y_len) {
    return guarded([&] {
        oracle::backend::cpu::reference_storage_matvec(
            type, static_cast<std::size_t>(rows), static_cast<std::size_t>(cols),
            as_bytes(matrix, nbytes), std::span<const float>(x, static_cast<std::size_t>(x_len)),
            std::span<float>(y, static_cast<std::size_t>(y_len)));
    });
}

// reference_mapped_tensor_matvec over an in-memory GgufTensorView (the reference's own tests
// build views the same way, tests/test_phase2a.cpp:301-306)
int ref_mapped_tensor_matvec(std::uint32_t type, std::uint64_t ne0, std::uint64_t ne1,
                             const void* matrix, std::uint64_t nbytes, const float* x,
                             std::uint64_t x_len, float* y, std::uint64_t y_len) {
    return guarded([&] {
        const auto* layout = oracle::model::ggml_type_layout(type);
        if (layout == nullptr) throw std::runtime_error("unregistered type");
        oracle::model::GgufTensorInfo info{"shim.weight", {ne0, ne1}, type, 0};
        const oracle::model::GgufTensorView view(
            &info, layout, static_cast<const std::byte*>(matrix),
            static_cast<std::size_t>(nbytes), 0);
        oracle::backend::cpu::reference_mapped_tensor_matvec(
            view, std::span<const float>(x, static_cast<std::size_t>(x_len)),
            std::span<float>(y, static_cast<std::size_t>(y_len)));
    });
}

// rows [row_begin, row_end) of a matvec, for a row-parallel timing of the reference's dot
int ref_storage_matvec_rows(std::uint32_t type, std::uint64_t cols, const void* matrix,
                            std::uint64_t row_bytes, std::uint64_t row_begin,
                            std::uint64_t row_end, const float* x, float* y) {
    return guarded([&] {
        const auto* base = static_cast<const std::byte*>(matrix);
        for (std::uint64_t r = row_begin; r < row_end; ++r) {
            y[r] = oracle::backend::cpu::reference_storage_dot(
                oracle::model::make_storage_row_view(
                    type, static_cast<std::size_t>(cols),
                    std::span<const std::byte>(base + r * row_bytes,
                                               static_cast<std::size_t>(row_bytes))),
                std::span<const float>(x, static_cast<std::size_t>(cols)));
        }
    });
}


// The reference's causal depthwise convolution step (src/runtime/reference_kernels.cpp:197-225)
// on an SsmState whose history is loaded from and stored back to `history` [channels][kernel].
int ref_conv_step(std::uint64_t channels, std::uint64_t kernel, float* history, const float* weights,
                  const float* input, float* out, int apply_silu) {
    return guarded([&] {
        oracle::runtime::SsmState st(static_cast<std::size_t>(channels), static_cast<std::size_t>(kernel), 1, 1, 1);
        auto h = st.convolution_history();
        std::copy(history, history + channels * kernel, h.begin());
        oracle::runtime::causal_depthwise_convolution_step(
            std::span<const float>(input, static_cast<std::size_t>(channels)),
            std::span<const float>(weights, static_cast<std::size_t>(channels * kernel)), st,
            std::span<float>(out, static_cast<std::size_t>(channels)), apply_silu != 0);
        std::copy(h.begin(), h.end(), history);
    });
}

// The reference's gated delta rule step (src/runtime/reference_kernels.cpp:227-335) with the
// recurrent state [heads][dk][dv] loaded from and stored back to `state`.
int ref_gated_delta_step(std::uint64_t heads, std::uint64_t dk, std::uint64_t dv, const float* q,
                         const float* k, const float* v, const float* beta, const float* log_decay,
                         float eps, float* state, float* out) {
    return guarded([&] {
        const auto H = static_cast<std::size_t>(heads), K = static_cast<std::size_t>(dk),
                   D = static_cast<std::size_t>(dv);
        oracle::runtime::SsmState st(1, 1, H, K, D);
        auto r = st.recurrent();
        std::copy(state, state + H * K * D, r.begin());
        oracle::core::Tensor tq({H, K}), tk({H, K}), tv({H, D}), to({H, D});
        std::copy(q, q + H * K, tq.data().begin());
        std::copy(k, k + H * K, tk.data().begin());
        std::copy(v, v + H * D, tv.data().begin());
        oracle::runtime::gated_delta_step(tq, tk, tv, std::span<const float>(beta, H),
                                          std::span<const float>(log_decay, H), st, to, eps);
        std::copy(r.begin(), r.end(), state);
        std::copy(to.data().begin(), to.data().end(), out);
    });
}
}  // extern "C"

// ---------------------------------------------------------------- the reference's recurrent block
//
// execute_qwen35_recurrent_block_reference (src/runtime/qwen35_block.cpp:406-605) driven on
// in-memory GgufTensorViews, as the reference's own block test builds them
// (tests/test_phase2c.cpp:72-213).  The block description has the layout of the oracle's
// orc_deltanet_block; projection weights may be any type the reference decodes (or q4_K when
// that projection is overridden).  `overrides`, if not NULL, holds 8 pointers in the order
// qkv, z, beta, alpha, out, gate, up, down; a non-NULL entry replaces that projection's output
// through the reference's Qwen35MatvecOverrides.  `trace`, if not NULL, receives the oracle's 16
// trace fields (qkv z beta alpha conv rec gated branch resid post gate up act ffn beta_s
// log_decay) taken from the
// reference's named trace; every named trace tensor of the last call stays readable through
// ref_block_trace_value.
struct RefDeltaNetBlock {
    std::uint64_t embedding, key_heads, value_heads, key_dim, value_dim, conv_kernel, ffn;
    float eps;
    std::uint32_t types[8];
    const std::uint8_t* weights[8];
    const float *input_norm, *conv_weight, *dt_bias, *decay, *out_norm, *post_norm;
};

namespace {

std::vector<oracle::runtime::Qwen35TraceTensor> g_trace;

struct ViewStore {
    std::vector<oracle::model::GgufTensorInfo> infos;
    std::vector<oracle::model::GgufTensorView> views;
    ViewStore() {
        infos.reserve(32);
        views.reserve(32);
    }
    const oracle::model::GgufTensorView* add(std::string name, std::vector<std::uint64_t> dims, std::uint32_t type,
                                             const void* data) {
        const auto* layout = oracle::model::ggml_type_layout(type);
        if (layout == nullptr) throw std::runtime_error("unregistered type");
        std::uint64_t elements = 1;
        for (auto d : dims) elements *= d;
        const std::uint64_t bytes = elements / layout->block_elements * layout->bytes_per_block;
        infos.push_back({std::move(name), std::move(dims), type, 0});
        views.emplace_back(&infos.back(), layout, static_cast<const std::byte*>(data),
                           static_cast<std::size_t>(bytes), 0);
        return &views.back();
    }
};

}  // namespace

extern "C" {

int ref_recurrent_block(const RefDeltaNetBlock* b, float* conv_history, float* state, const float* x, float* y,
                        float* trace, const float* const* overrides) {
    return guarded([&] {
        const std::uint64_t E = b->embedding, Hk = b->key_heads, Hv = b->value_heads, dk = b->key_dim,
                            dv = b->value_dim, K = b->conv_kernel, F = b->ffn;
        const std::uint64_t V = Hv * dv, C = 2 * Hk * dk + V;
        oracle::model::Qwen35Manifest m;
        m.architecture = "qwen35";
        m.embedding_length = static_cast<std::uint32_t>(E);
        m.feed_forward_length = static_cast<std::uint32_t>(F);
        m.attention_rms_epsilon = b->eps;
        m.ssm_convolution_kernel = static_cast<std::uint32_t>(K);
        m.ssm_state_size = static_cast<std::uint32_t>(dk);
        m.ssm_group_count = static_cast<std::uint32_t>(Hk);
        m.ssm_time_step_rank = static_cast<std::uint32_t>(Hv);
        m.ssm_inner_size = static_cast<std::uint32_t>(V);
        ViewStore vs;
        // {dimensions[0] = columns, dimensions[1] = rows}, as GGUF stores a matrix
        const std::uint64_t cols[8] = {E, E, E, E, V, E, E, F};
        const std::uint64_t rows[8] = {C, V, Hv, Hv, E, F, F, E};
        const char* names[8] = {"qkv", "z", "beta", "alpha", "out", "gate", "up", "down"};
        const oracle::model::GgufTensorView* w[8];
        for (int i = 0; i < 8; ++i) w[i] = vs.add(names[i], {cols[i], rows[i]}, b->types[i], b->weights[i]);
        oracle::model::Qwen35BackboneBlockWeights blk;
        blk.index = 0;
        blk.kind = oracle::model::Qwen35BlockKind::recurrent;
        blk.input_norm = vs.add("input_norm", {E}, 0, b->input_norm);
        blk.post_attention_norm = vs.add("post_norm", {E}, 0, b->post_norm);
        blk.mlp.gate = w[5];
        blk.mlp.up = w[6];
        blk.mlp.down = w[7];
        oracle::model::Qwen35RecurrentWeights rw;
        rw.qkv = w[0];
        rw.gate = w[1];
        rw.beta = w[2];
        rw.alpha = w[3];
        rw.output = w[4];
        rw.convolution = vs.add("conv", {K, C}, 0, b->conv_weight);
        rw.time_step_bias = vs.add("dt_bias", {Hv}, 0, b->dt_bias);
        rw.decay = vs.add("decay", {Hv}, 0, b->decay);
        rw.norm = vs.add("norm", {dv}, 0, b->out_norm);
        blk.recurrent = rw;

        oracle::runtime::SsmState st(static_cast<std::size_t>(C), static_cast<std::size_t>(K),
                                     static_cast<std::size_t>(Hv), static_cast<std::size_t>(dk),
                                     static_cast<std::size_t>(dv));
        auto h = st.convolution_history();
        std::copy(conv_history, conv_history + C * K, h.begin());
        auto r = st.recurrent();
        std::copy(state, state + Hv * dk * dv, r.begin());

        oracle::runtime::Qwen35MatvecOverrides ov;
        if (overrides != nullptr) {
            const char* trace_names[8] = {"linear_attn_qkv_mixed", "z", "beta", "alpha",
                                          "linear_attn_out", "ffn_gate", "ffn_up", "ffn_out"};
            for (int i = 0; i < 8; ++i) {
                if (overrides[i] == nullptr) continue;
                ov.tensors.push_back({trace_names[i], std::vector<float>(overrides[i], overrides[i] + rows[i])});
            }
        }
        auto res = oracle::runtime::execute_qwen35_recurrent_block_reference(
            m, blk, std::span<const float>(x, static_cast<std::size_t>(E)), st, true,
            overrides != nullptr ? &ov : nullptr);
        std::copy(res.output.begin(), res.output.end(), y);
        std::copy(h.begin(), h.end(), conv_history);
        std::copy(r.begin(), r.end(), state);
        g_trace = res.trace.tensors;
        if (trace != nullptr) {
            const char* fields[16] = {"linear_attn_qkv_mixed", "z", "beta", "alpha", "conv_output_silu",
                                      "recurrent_output", "attn_out_norm", "linear_attn_out", "attn_residual",
                                      "attn_post_norm", "ffn_gate", "ffn_up", "ffn_swiglu", "ffn_out",
                                      "beta_sigmoid", "gate"};
            std::uint64_t off = 0;
            for (const char* f : fields) {
                const auto* t = res.trace.find(f);
                if (t == nullptr) throw std::runtime_error(std::string("reference trace lacks ") + f);
                std::copy(t->values.begin(), t->values.end(), trace + off);
                off += t->values.size();
            }
        }
    });
}

// Named trace tensor of the last ref_recurrent_block call: copies up to cap values, returns the
// tensor's length (or -1 when the name is absent).
std::int64_t ref_block_trace_value(const char* name, float* out, std::uint64_t cap) {
    for (const auto& t : g_trace) {
        if (t.name == name) {
            const std::uint64_t n = t.values.size() < cap ? t.values.size() : cap;
            std::copy(t.values.begin(), t.values.begin() + static_cast<std::ptrdiff_t>(n), out);
            return static_cast<std::int64_t>(t.values.size());
        }
    }
    return -1;
}
}  // extern "C"

// ---------------------------------------------------------------- the reference's GGUF mapping
//
// MappedGgufModel (src/model/mapped_gguf.cpp:124-203) over a file: ref_gguf_open maps it (or
// returns the reference's error), ref_gguf_tensor reads entry `index` of its tensor table.
#include <memory>

namespace {
std::unique_ptr<oracle::model::MappedGgufModel> g_model;
}

extern "C" {

int ref_gguf_open(const char* path, std::uint64_t* count) {
    return guarded([&] {
        g_model.reset();
        g_model = std::make_unique<oracle::model::MappedGgufModel>(path);
        *count = g_model->tensors().size();
    });
}

int ref_gguf_tensor(std::uint64_t index, char* name, int name_cap, std::uint32_t* type, std::uint32_t* n_dims,
                    std::uint64_t* dims, std::uint64_t* absolute_offset, std::uint64_t* nbytes) {
    return guarded([&] {
        if (!g_model || index >= g_model->tensors().size()) throw std::out_of_range("tensor index");
        const auto& t = g_model->tensors()[static_cast<std::size_t>(index)];
        std::snprintf(name, static_cast<std::size_t>(name_cap), "%.*s", static_cast<int>(t.name().size()),
                      t.name().data());
        *type = t.layout().type;
        const auto d = t.dimensions();
        *n_dims = static_cast<std::uint32_t>(d.size());
        for (std::size_t i = 0; i < d.size() && i < 4; ++i) dims[i] = d[i];
        *absolute_offset = t.absolute_offset();
        *nbytes = t.bytes().size();
    });
}

}  // extern "C"

// ---------------------------------------------------------------- the reference's attention path
//
// apply_qwen35_rope (src/runtime/reference_kernels.cpp:77-125), causal_attention_step (:127-195)
// and execute_qwen35_attention_block_reference (src/runtime/qwen35_block.cpp:607-756) on the
// caller's arrays.  The KV cache crosses the boundary as the oracle's orc_kv_cache arrays: a
// KvCache of the same capacity is rebuilt by appending the `length` stored tokens in order
// (KvCache::append copies, so the rebuilt cache holds the same bits), the call runs, and the
// cache's rows are copied back.
struct RefKvCache {
    std::uint64_t capacity, kv_heads, key_dim, value_dim, length;
    float *keys, *values;
};

struct RefAttentionBlock {
    std::uint64_t embedding, q_heads, kv_heads, head_dim, ffn, rope_dim;
    std::int32_t rope_sections[4];
    float rope_base, eps;
    std::uint32_t types[7];  // q k v out gate up down
    const std::uint8_t* weights[7];
    const float *input_norm, *q_norm, *k_norm, *post_norm;
};

namespace {

oracle::runtime::KvCache rebuild(const RefKvCache& c) {
    oracle::runtime::KvCache cache(static_cast<std::size_t>(c.capacity), static_cast<std::size_t>(c.kv_heads),
                                   static_cast<std::size_t>(c.key_dim), static_cast<std::size_t>(c.value_dim));
    const std::size_t kw = static_cast<std::size_t>(c.kv_heads * c.key_dim);
    const std::size_t vw = static_cast<std::size_t>(c.kv_heads * c.value_dim);
    for (std::uint64_t t = 0; t < c.length; ++t) {
        cache.append(std::span<const float>(c.keys + t * kw, kw), std::span<const float>(c.values + t * vw, vw));
    }
    return cache;
}

void store(const oracle::runtime::KvCache& cache, RefKvCache& c) {
    c.length = cache.size();
    for (std::size_t t = 0; t < cache.size(); ++t) {
        for (std::size_t h = 0; h < cache.key_value_heads(); ++h) {
            const auto k = cache.key(t, h);
            const auto v = cache.value(t, h);
            std::copy(k.begin(), k.end(), c.keys + (t * cache.key_value_heads() + h) * cache.key_dimension());
            std::copy(v.begin(), v.end(), c.values + (t * cache.key_value_heads() + h) * cache.value_dimension());
        }
    }
}

}  // namespace

extern "C" {

int ref_rope(float* heads, std::uint64_t n_heads, std::uint64_t head_dim, std::uint64_t rotary_dim,
             const std::int32_t* sections, float base, const std::uint64_t* position) {
    return guarded([&] {
        oracle::core::Tensor t({static_cast<std::size_t>(n_heads), static_cast<std::size_t>(head_dim)});
        std::copy(heads, heads + n_heads * head_dim, t.data().begin());
        oracle::runtime::apply_qwen35_rope(t, {position[0], position[1], position[2]},
                                           static_cast<std::size_t>(rotary_dim),
                                           {sections[0], sections[1], sections[2], sections[3]}, base);
        std::copy(t.data().begin(), t.data().end(), heads);
    });
}

int ref_attention_step(const float* q, std::uint64_t q_heads, const float* k, const float* v, RefKvCache* c,
                       float* out) {
    return guarded([&] {
        auto cache = rebuild(*c);
        const auto Hq = static_cast<std::size_t>(q_heads), Hkv = static_cast<std::size_t>(c->kv_heads),
                   dk = static_cast<std::size_t>(c->key_dim), dv = static_cast<std::size_t>(c->value_dim);
        oracle::core::Tensor tq({Hq, dk}), tk({Hkv, dk}), tv({Hkv, dv}), to({Hq, dv});
        std::copy(q, q + Hq * dk, tq.data().begin());
        std::copy(k, k + Hkv * dk, tk.data().begin());
        std::copy(v, v + Hkv * dv, tv.data().begin());
        oracle::runtime::causal_attention_step(tq, tk, tv, cache, to);
        std::copy(to.data().begin(), to.data().end(), out);
        store(cache, *c);
    });
}

int ref_attention_block(const RefAttentionBlock* b, RefKvCache* c, const std::uint64_t* position, const float* x,
                        float* y, float* trace, const float* const* overrides) {
    return guarded([&] {
        const std::uint64_t E = b->embedding, Hq = b->q_heads, Hkv = b->kv_heads, D = b->head_dim, F = b->ffn;
        const std::uint64_t Q = Hq * D, KV = Hkv * D;
        oracle::model::Qwen35Manifest m;
        m.architecture = "qwen35";
        m.embedding_length = static_cast<std::uint32_t>(E);
        m.feed_forward_length = static_cast<std::uint32_t>(F);
        m.attention_rms_epsilon = b->eps;
        m.attention_head_count = static_cast<std::uint32_t>(Hq);
        m.attention_head_count_kv = static_cast<std::uint32_t>(Hkv);
        m.attention_key_length = static_cast<std::uint32_t>(D);
        m.attention_value_length = static_cast<std::uint32_t>(D);
        m.rope_dimension_count = static_cast<std::uint32_t>(b->rope_dim);
        m.rope_dimension_sections = {b->rope_sections[0], b->rope_sections[1], b->rope_sections[2],
                                     b->rope_sections[3]};
        m.rope_frequency_base = b->rope_base;
        ViewStore vs;
        const std::uint64_t cols[7] = {E, E, E, Q, E, E, F};
        const std::uint64_t rows[7] = {2 * Q, KV, KV, E, F, F, E};
        const char* names[7] = {"attn_q", "attn_k", "attn_v", "attn_output", "gate", "up", "down"};
        const oracle::model::GgufTensorView* w[7];
        for (int i = 0; i < 7; ++i) w[i] = vs.add(names[i], {cols[i], rows[i]}, b->types[i], b->weights[i]);
        oracle::model::Qwen35BackboneBlockWeights blk;
        blk.index = 3;
        blk.kind = oracle::model::Qwen35BlockKind::full_attention;
        blk.input_norm = vs.add("input_norm", {E}, 0, b->input_norm);
        blk.post_attention_norm = vs.add("post_norm", {E}, 0, b->post_norm);
        blk.mlp.gate = w[4];
        blk.mlp.up = w[5];
        blk.mlp.down = w[6];
        oracle::model::Qwen35AttentionWeights aw;
        aw.query = w[0];
        aw.key = w[1];
        aw.value = w[2];
        aw.output = w[3];
        aw.query_norm = vs.add("attn_q_norm", {D}, 0, b->q_norm);
        aw.key_norm = vs.add("attn_k_norm", {D}, 0, b->k_norm);
        blk.attention = aw;

        auto cache = rebuild(*c);
        oracle::runtime::Qwen35MatvecOverrides ov;
        if (overrides != nullptr) {
            const char* trace_names[7] = {"Qcur_full", "Kcur_projected", "Vcur_projected", "attn_output",
                                          "ffn_gate", "ffn_up", "ffn_out"};
            for (int i = 0; i < 7; ++i) {
                if (overrides[i] == nullptr) continue;
                ov.tensors.push_back({trace_names[i], std::vector<float>(overrides[i], overrides[i] + rows[i])});
            }
        }
        auto res = oracle::runtime::execute_qwen35_attention_block_reference(
            m, blk, std::span<const float>(x, static_cast<std::size_t>(E)), cache,
            {position[0], position[1], position[2]}, true, overrides != nullptr ? &ov : nullptr);
        std::copy(res.output.begin(), res.output.end(), y);
        store(cache, *c);
        g_trace = res.trace.tensors;
        if (trace != nullptr) {
            const char* fields[15] = {"Qcur_full", "Kcur_projected", "Vcur_projected", "Qcur", "Kcur",
                                      "attn_pregate", "gate_sigmoid", "attn_gated", "attn_output", "attn_residual",
                                      "attn_post_norm", "ffn_gate", "ffn_up", "ffn_swiglu", "ffn_out"};
            std::uint64_t off = 0;
            for (const char* f : fields) {
                const auto* t = res.trace.find(f);
                if (t == nullptr) throw std::runtime_error(std::string("reference trace lacks ") + f);
                std::copy(t->values.begin(), t->values.end(), trace + off);
                off += t->values.size();
            }
        }
    });
}

}  // extern "C"
