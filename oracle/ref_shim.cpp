// ORACLE -- test infrastructure, not product code.
//
// A C-callable shim over the reference engine's own quantized path, compiled together with
// the reference's sources (ggml_type.cpp, storage_decode.cpp, quantized_reference.cpp and the
// GgufTensorView they take) into oracle/_ref/libref.so by oracle/Makefile.  It lets the tests
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
