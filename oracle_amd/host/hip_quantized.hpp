// C++20 host adapter: the reference engine's quantized matrix functions on an MI355X.
//
// oracle::backend::hip::QuantizedDevice offers the signatures of oracle::backend::cpu's
// reference_storage_dot / reference_storage_matvec / reference_mapped_tensor_matvec /
// reference_decode_mapped_tensor (include/oracle/backend/cpu/quantized_reference.hpp:10-27 of
// the reference) and throws the same exception types for the same conditions, in the same order
// (src/backend/cpu/quantized_reference.cpp:107-153, src/model/ggml_type.cpp:77-94,
// src/model/storage_decode.cpp:182-198).  The difference is where the arithmetic runs: weights
// are uploaded once to HBM through liboq.so's C ABI (include/oq.h) and stay resident, keyed by
// the address and geometry of the mapped bytes, so a GgufTensorView's mmap'd payload is copied
// straight to the device the first time it is used and never again.
//
// Tensor views are taken generically: anything with dimensions() (a range of uint64_t),
// bytes() (std::span<const std::byte>) and layout().type works, which includes
// oracle::model::GgufTensorView (include/oracle/model/mapped_gguf.hpp:18-41).
//
// Threading: one QuantizedDevice owns one oq_context (one HIP stream) and is not thread-safe,
// matching the reference's single-threaded use.  Validation runs before any device work, so
// argument errors are reported even on a machine without a GPU.
#pragma once

#include <cstddef>
#include <cstdint>
#include <limits>
#include <map>
#include <span>
#include <stdexcept>
#include <string>
#include <tuple>

#include "oq.h"

namespace oracle::backend::hip {

// Throw the reference's exception kind for an oq_status (OQ_OK returns).
void throw_on_status(int status, const std::string& message);

// Mirror of oracle::model::StorageRowView (include/oracle/model/storage_decode.hpp:24-28).
struct StorageRowView {
    std::uint32_t type{0};
    std::size_t element_count{0};
    std::span<const std::byte> bytes;
};

class QuantizedDevice {
public:
    explicit QuantizedDevice(int device = 0);
    ~QuantizedDevice();
    QuantizedDevice(const QuantizedDevice&) = delete;
    QuantizedDevice& operator=(const QuantizedDevice&) = delete;

    // reference_storage_matvec (src/backend/cpu/quantized_reference.cpp:128-162)
    void storage_matvec(std::uint32_t type, std::size_t row_count, std::size_t column_count,
                        std::span<const std::byte> matrix_bytes, std::span<const float> vector,
                        std::span<float> output);

    // M activation rows at once: vectors [m][column_count] -> outputs [m][row_count].  The
    // reference evaluates M tokens as M independent matvecs (src/runtime/qwen35_target_multi.cpp
    // :14-25); this streams the weights once for all of them.
    void storage_matmul(std::uint32_t type, std::size_t row_count, std::size_t column_count,
                        std::span<const std::byte> matrix_bytes, std::size_t m,
                        std::span<const float> vectors, std::span<float> outputs);

    // reference_storage_dot (src/backend/cpu/quantized_reference.cpp:24-82): one row.
    [[nodiscard]] float storage_dot(StorageRowView row, std::span<const float> vector);

    // reference_mapped_tensor_matvec (src/backend/cpu/quantized_reference.cpp:107-126)
    template <typename TensorView>
    void mapped_tensor_matvec(const TensorView& tensor, std::span<const float> vector,
                              std::span<float> output) {
        const auto [rows, cols] = rank2(tensor);
        storage_matvec(tensor.layout().type, rows, cols, tensor.bytes(), vector, output);
    }

    template <typename TensorView>
    void mapped_tensor_matmul(const TensorView& tensor, std::size_t m,
                              std::span<const float> vectors, std::span<float> outputs) {
        const auto [rows, cols] = rank2(tensor);
        storage_matmul(tensor.layout().type, rows, cols, tensor.bytes(), m, vectors, outputs);
    }

    // reference_decode_mapped_tensor (src/backend/cpu/quantized_reference.cpp:85-105): every row
    // of the tensor decoded to F32, bit-identical to the reference's decoders.
    template <typename TensorView>
    void decode_mapped_tensor(const TensorView& tensor, std::span<float> output) {
        const auto dims = tensor.dimensions();
        if (dims.size() == 0) throw std::invalid_argument("GGUF tensor must have at least one dimension");
        std::uint64_t total = 1;
        for (const std::uint64_t d : dims) {
            if (d == 0) throw std::invalid_argument("GGML tensor dimensions must be non-zero");
            if (total > std::numeric_limits<std::uint64_t>::max() / d) {
                throw std::overflow_error("GGML tensor element count overflow");
            }
            total *= d;
        }
        const std::uint64_t width = *dims.begin();
        if (total % width != 0) throw std::logic_error("GGUF tensor has invalid row geometry");
        decode_rows(tensor.layout().type, static_cast<std::size_t>(total / width),
                    static_cast<std::size_t>(width), tensor.bytes(), output);
    }

    void decode_rows(std::uint32_t type, std::size_t row_count, std::size_t column_count,
                     std::span<const std::byte> matrix_bytes, std::span<float> output);

    // Greedy token of Sampler::sample at temperature 0 (src/runtime/sampler.cpp:22-44): the
    // first index of the maximum, std::invalid_argument for an empty vector, a NaN or no finite
    // candidate.  Computed on the device by oq_argmax (on a model path the logits stay in HBM and
    // oq_argmax is called on them directly).
    [[nodiscard]] std::uint32_t greedy_token(std::span<const float> logits);

    // Device-resident access for callers that keep activations in HBM (chained layers).
    const oq_weight* resident(std::uint32_t type, std::size_t row_count, std::size_t column_count,
                              std::span<const std::byte> matrix_bytes);
    [[nodiscard]] std::size_t resident_count() const noexcept { return weights_.size(); }
    void evict_all() noexcept;
    oq_context* context();  // created on first use
    [[nodiscard]] std::string_view name() const noexcept { return "hip"; }

private:
    template <typename TensorView>
    static std::pair<std::size_t, std::size_t> rank2(const TensorView& tensor) {
        const auto dims = tensor.dimensions();
        if (dims.size() != 2) throw std::invalid_argument("mapped tensor matvec requires a rank-2 tensor");
        const std::uint64_t d0 = *dims.begin(), d1 = *(dims.begin() + 1);
        if (d0 > std::numeric_limits<std::size_t>::max() || d1 > std::numeric_limits<std::size_t>::max()) {
            throw std::overflow_error("mapped tensor matvec dimensions exceed addressable size");
        }
        return {static_cast<std::size_t>(d1), static_cast<std::size_t>(d0)};
    }

    void validate(std::uint32_t type, std::size_t rows, std::size_t cols,
                  std::span<const std::byte> matrix_bytes, std::size_t m, std::size_t vector_len,
                  std::size_t output_len);
    float* device_floats(void*& buffer, std::size_t& capacity, std::size_t count);

    using Key = std::tuple<const std::byte*, std::size_t, std::uint32_t, std::size_t>;
    int device_;
    oq_context* ctx_ = nullptr;
    std::map<Key, oq_weight*> weights_;
    void* x_dev_ = nullptr;
    std::size_t x_cap_ = 0;
    void* y_dev_ = nullptr;
    std::size_t y_cap_ = 0;
    void* t_dev_ = nullptr;  // greedy token and its value
    std::size_t t_cap_ = 0;
};

}  // namespace oracle::backend::hip
