// C++20 host adapter: the reference engine's quantized matrix functions on an MI355X.
//
// oracle::backend::hip::QuantizedDevice offers the signatures of oracle::backend::cpu's
// reference_storage_dot / reference_storage_matvec / reference_mapped_tensor_matvec /
// reference_decode_mapped_tensor (include/oracle/backend/cpu/quantized_reference.hpp:10-27 of
// the reference) and throws the same exception types for the same conditions, in the same order
// (src/backend/cpu/quantized_reference.cpp:107-153, src/model/ggml_type.cpp:77-94,
// src/model/storage_decode.cpp:182-198).  The difference is where the arithmetic runs: weights
// live in HBM, uploaded through liboq.so's C ABI (include/oq.h):
//   - upload_model(model) takes a whole MappedGgufModel once (oq_model_upload) and serves every
//     later mapped_tensor_* call on one of its tensors from HBM, looked up by name;
//   - a mapped tensor outside such a model is uploaded on first use and stays resident, keyed by
//     the address and geometry of its (immutable, mmap'd) bytes;
//   - raw spans (storage_matvec, storage_matmul, storage_dot, decode_rows) are uploaded for the
//     call only: their memory belongs to the caller and may change between calls.
//
// Tensor views are taken generically: anything with dimensions() (a range of uint64_t),
// bytes() (std::span<const std::byte>), layout().type and name() works, which includes
// oracle::model::GgufTensorView (include/oracle/model/mapped_gguf.hpp:18-41); a model is anything
// with tensors() (such views, each with absolute_offset()) and mapping() (data(), size()), which
// includes oracle::model::MappedGgufModel (:53-78).  Row views: any type with the fields of
// oracle::model::StorageRowView (include/oracle/model/storage_decode.hpp:24-28).
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
#include <string_view>
#include <tuple>
#include <vector>

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

    // reference_storage_dot (src/backend/cpu/quantized_reference.cpp:24-82): one row, given as
    // oracle::model::StorageRowView (or the mirror above, or any type with its three fields).
    template <typename RowView>
    [[nodiscard]] float storage_dot(const RowView& row, std::span<const float> vector) {
        return row_dot(row.type, row.element_count, row.bytes, vector);
    }
    [[nodiscard]] float storage_dot(const StorageRowView& row, std::span<const float> vector) {
        return row_dot(row.type, row.element_count, row.bytes, vector);
    }

    // reference_mapped_tensor_matvec (src/backend/cpu/quantized_reference.cpp:107-126)
    template <typename TensorView>
    void mapped_tensor_matvec(const TensorView& tensor, std::span<const float> vector,
                              std::span<float> output) {
        mapped_tensor_matmul(tensor, 1, vector, output);
    }

    template <typename TensorView>
    void mapped_tensor_matmul(const TensorView& tensor, std::size_t m,
                              std::span<const float> vectors, std::span<float> outputs) {
        const auto [rows, cols] = rank2(tensor);
        const std::uint32_t type = tensor.layout().type;
        validate(type, rows, cols, tensor.bytes(), m, vectors.size(), outputs.size());
        run_matmul(mapped_weight(tensor, type, rows, cols), m, vectors, outputs);
    }

    // The same products with activations and outputs already in device memory (x_dev [m][cols],
    // y_dev [m][rows], F32): for callers that chain projections in HBM (mapped_matvec,
    // src/runtime/qwen35_block.cpp:108-119, without a host round trip per projection).
    // Asynchronous on the device's stream (context()); synchronize() waits.
    template <typename TensorView>
    void mapped_tensor_matmul_device(const TensorView& tensor, std::size_t m, const float* x_dev, float* y_dev) {
        (void)context();
        const auto [rows, cols] = rank2(tensor);
        const std::uint32_t type = tensor.layout().type;
        validate(type, rows, cols, tensor.bytes(), m, cols * m, rows * m);
        const oq_weight* w = mapped_weight(tensor, type, rows, cols);
        check_status(m == 1 ? oq_matvec(ctx_, w, x_dev, y_dev) : oq_matmul(ctx_, w, m, x_dev, y_dev));
    }
    void synchronize();

    // One-time upload of a whole mapped model (oq_model_upload): every tensor validated as
    // MappedGgufModel does, copied to HBM once; its rank-2 tensors of the supported types become
    // resident weights, found by name by the mapped_tensor_* calls.  Replaces a previous model.
    template <typename Model>
    void upload_model(const Model& model) {
        std::vector<std::string> names;
        std::vector<oq_tensor_desc> descs;
        names.reserve(model.tensors().size());
        descs.reserve(model.tensors().size());
        for (const auto& t : model.tensors()) {
            names.emplace_back(t.name());
            oq_tensor_desc d{};
            d.type = t.layout().type;
            const auto dims = t.dimensions();
            if (dims.size() > 4) throw std::invalid_argument("tensors of more than four dimensions are not supported");
            d.n_dims = static_cast<std::uint32_t>(dims.size());
            std::uint32_t i = 0;
            for (const std::uint64_t v : dims) d.dims[i++] = v;
            d.offset = t.absolute_offset();
            descs.push_back(d);
        }
        for (std::size_t i = 0; i < descs.size(); ++i) descs[i].name = names[i].c_str();
        const auto& map = model.mapping();
        load_model(map.data(), map.size(), descs);
    }
    void load_model(const void* payload, std::size_t payload_bytes, const std::vector<oq_tensor_desc>& tensors);
    [[nodiscard]] const oq_model* model() const noexcept { return model_; }

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

    // The resident weight of a mapped tensor's bytes (immutable for the model's lifetime),
    // uploaded on first use.
    const oq_weight* resident(std::uint32_t type, std::size_t row_count, std::size_t column_count,
                              std::span<const std::byte> matrix_bytes);
    [[nodiscard]] std::size_t resident_count() const noexcept { return weights_.size(); }
    void evict_all() noexcept;  // also releases an uploaded model
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

    // the model's weight for a tensor of this name and geometry whose bytes lie in the model's
    // payload, else the address-keyed resident upload
    template <typename TensorView>
    const oq_weight* mapped_weight(const TensorView& tensor, std::uint32_t type, std::size_t rows, std::size_t cols) {
        if (model_ != nullptr) {
            const std::byte* p = tensor.bytes().data();
            if (p >= model_base_ && p < model_base_ + model_bytes_) {
                if (const oq_weight* w = model_weight(std::string(tensor.name()), type, rows, cols)) return w;
            }
        }
        return resident(type, rows, cols, tensor.bytes());
    }
    const oq_weight* model_weight(const std::string& name, std::uint32_t type, std::size_t rows, std::size_t cols);

    void validate(std::uint32_t type, std::size_t rows, std::size_t cols,
                  std::span<const std::byte> matrix_bytes, std::size_t m, std::size_t vector_len,
                  std::size_t output_len);
    float row_dot(std::uint32_t type, std::size_t element_count, std::span<const std::byte> bytes,
                  std::span<const float> vector);
    void run_matmul(const oq_weight* w, std::size_t m, std::span<const float> vectors, std::span<float> outputs);
    void check_status(int status);
    float* device_floats(void*& buffer, std::size_t& capacity, std::size_t count);

    // a weight uploaded for one call (raw caller-owned bytes), released by the destructor
    struct Transient {
        oq_weight* w = nullptr;
        ~Transient() { oq_weight_release(w); }
    };

    using Key = std::tuple<const std::byte*, std::size_t, std::uint32_t, std::size_t>;
    int device_;
    oq_context* ctx_ = nullptr;
    std::map<Key, oq_weight*> weights_;
    oq_model* model_ = nullptr;
    const std::byte* model_base_ = nullptr;
    std::size_t model_bytes_ = 0;
    void* x_dev_ = nullptr;
    std::size_t x_cap_ = 0;
    void* y_dev_ = nullptr;
    std::size_t y_cap_ = 0;
    void* t_dev_ = nullptr;  // greedy token and its value
    std::size_t t_cap_ = 0;
};

}  // namespace oracle::backend::hip
