// Implementation of the C++20 host adapter over liboq.so (see hip_quantized.hpp).
#include "hip_quantized.hpp"

#include <cmath>
#include <cstring>
#include <string>

namespace oracle::backend::hip {

void throw_on_status(int status, const std::string& message) {
    switch (status) {
        case OQ_OK: return;
        case OQ_INVALID_ARGUMENT: throw std::invalid_argument(message);
        case OQ_OUT_OF_RANGE: throw std::out_of_range(message);
        case OQ_OVERFLOW: throw std::overflow_error(message);
        case OQ_UNSUPPORTED_TYPE: throw std::runtime_error(message);
        case OQ_LOGIC_ERROR: throw std::logic_error(message);
        case OQ_RUNTIME_ERROR: throw std::runtime_error(message);
        default: throw std::runtime_error("HIP device failure: " + message);
    }
}

namespace {

void check(int status, const oq_context* ctx) {
    if (status != OQ_OK) throw_on_status(status, oq_last_error(ctx));
}

}  // namespace

QuantizedDevice::QuantizedDevice(int device) : device_(device) {}

QuantizedDevice::~QuantizedDevice() {
    evict_all();
    if (ctx_) {
        if (x_dev_) (void)oq_device_free(ctx_, x_dev_);
        if (y_dev_) (void)oq_device_free(ctx_, y_dev_);
        if (t_dev_) (void)oq_device_free(ctx_, t_dev_);
        oq_context_destroy(ctx_);
    }
}

oq_context* QuantizedDevice::context() {
    if (!ctx_) check(oq_context_create(device_, &ctx_), nullptr);
    return ctx_;
}

void QuantizedDevice::evict_all() noexcept {
    for (auto& kv : weights_) oq_weight_release(kv.second);
    weights_.clear();
    oq_model_release(model_);
    model_ = nullptr;
    model_base_ = nullptr;
    model_bytes_ = 0;
}

void QuantizedDevice::check_status(int status) { check(status, ctx_); }

void QuantizedDevice::synchronize() { check(oq_synchronize(context()), ctx_); }

void QuantizedDevice::load_model(const void* payload, std::size_t payload_bytes,
                                 const std::vector<oq_tensor_desc>& tensors) {
    check(oq_model_validate(payload_bytes, tensors.data(), tensors.size()), nullptr);
    oq_model* m = nullptr;
    check(oq_model_upload(context(), payload, payload_bytes, tensors.data(), tensors.size(), &m), ctx_);
    oq_model_release(model_);
    model_ = m;
    model_base_ = static_cast<const std::byte*>(payload);
    model_bytes_ = payload_bytes;
}

const oq_weight* QuantizedDevice::model_weight(const std::string& name, std::uint32_t type, std::size_t rows,
                                               std::size_t cols) {
    std::uint64_t index = 0;
    if (oq_model_find(model_, name.c_str(), &index) != OQ_OK) return nullptr;
    oq_model_tensor_info info{};
    check(oq_model_tensor(model_, index, &info), nullptr);
    if (info.weight == nullptr || info.type != type || info.n_dims != 2 || info.dims[0] != cols ||
        info.dims[1] != rows) {
        return nullptr;
    }
    return info.weight;
}

// The checks reference_storage_matvec makes before its row loop, in its order
// (src/backend/cpu/quantized_reference.cpp:134-153), then the decoder whitelist that
// make_storage_row_view applies to the first row (src/model/storage_decode.cpp:192-193,
// here extended by q4_K).
void QuantizedDevice::validate(std::uint32_t type, std::size_t rows, std::size_t cols,
                               std::span<const std::byte> matrix_bytes, std::size_t m,
                               std::size_t vector_len, std::size_t output_len) {
    if (rows == 0 || cols == 0) throw std::invalid_argument("reference matvec dimensions must be non-zero");
    if (m == 0) throw std::invalid_argument("matmul batch must be non-zero");
    if (cols > std::numeric_limits<std::size_t>::max() / m || vector_len != cols * m) {
        throw std::invalid_argument("reference matvec vector length mismatch");
    }
    if (rows > std::numeric_limits<std::size_t>::max() / m || output_len != rows * m) {
        throw std::invalid_argument("reference matvec output length mismatch");
    }
    std::uint64_t row_bytes = 0;
    check(oq_row_byte_size(cols, type, &row_bytes), nullptr);
    if (row_bytes > std::numeric_limits<std::size_t>::max() ||
        (rows != 0 && row_bytes > std::numeric_limits<std::size_t>::max() / rows)) {
        throw std::overflow_error("reference matvec matrix size overflow");
    }
    if (matrix_bytes.size() != row_bytes * rows) {
        throw std::invalid_argument("reference matvec matrix byte size mismatch");
    }
    if (!oq_type_supported(type)) {
        throw std::invalid_argument("storage decoder does not support GGML type " + std::to_string(type));
    }
}

const oq_weight* QuantizedDevice::resident(std::uint32_t type, std::size_t rows, std::size_t cols,
                                           std::span<const std::byte> matrix_bytes) {
    const Key key{matrix_bytes.data(), matrix_bytes.size(), type, cols};
    if (auto it = weights_.find(key); it != weights_.end()) return it->second;
    oq_weight* w = nullptr;
    check(oq_weight_upload(context(), type, cols, rows, matrix_bytes.data(), matrix_bytes.size(), &w),
          context());
    weights_.emplace(key, w);
    return w;
}

float* QuantizedDevice::device_floats(void*& buffer, std::size_t& capacity, std::size_t count) {
    const std::size_t bytes = count * sizeof(float);
    if (capacity < bytes) {
        if (buffer) check(oq_device_free(context(), buffer), ctx_);
        buffer = nullptr;
        capacity = 0;
        check(oq_device_alloc(context(), bytes, &buffer), ctx_);
        capacity = bytes;
    }
    return static_cast<float*>(buffer);
}

void QuantizedDevice::run_matmul(const oq_weight* w, std::size_t m, std::span<const float> vectors,
                                 std::span<float> outputs) {
    float* x = device_floats(x_dev_, x_cap_, vectors.size());
    float* y = device_floats(y_dev_, y_cap_, outputs.size());
    check(oq_copy_to_device(ctx_, x, vectors.data(), vectors.size_bytes()), ctx_);
    check(m == 1 ? oq_matvec(ctx_, w, x, y) : oq_matmul(ctx_, w, m, x, y), ctx_);
    check(oq_copy_to_host(ctx_, outputs.data(), y, outputs.size_bytes()), ctx_);
}

void QuantizedDevice::storage_matmul(std::uint32_t type, std::size_t rows, std::size_t cols,
                                     std::span<const std::byte> matrix_bytes, std::size_t m,
                                     std::span<const float> vectors, std::span<float> outputs) {
    validate(type, rows, cols, matrix_bytes, m, vectors.size(), outputs.size());
    // caller-owned bytes: uploaded for this call only
    Transient t;
    check(oq_weight_upload(context(), type, cols, rows, matrix_bytes.data(), matrix_bytes.size(), &t.w), ctx_);
    run_matmul(t.w, m, vectors, outputs);
}

void QuantizedDevice::storage_matvec(std::uint32_t type, std::size_t rows, std::size_t cols,
                                     std::span<const std::byte> matrix_bytes,
                                     std::span<const float> vector, std::span<float> output) {
    storage_matmul(type, rows, cols, matrix_bytes, 1, vector, output);
}

float QuantizedDevice::row_dot(std::uint32_t type, std::size_t element_count, std::span<const std::byte> bytes,
                               std::span<const float> vector) {
    // make_storage_row_view's checks (byte size, then whitelist), then the vector length
    // (src/backend/cpu/quantized_reference.cpp:25-29)
    std::uint64_t expected = 0;
    check(oq_row_byte_size(element_count, type, &expected), nullptr);
    if (bytes.size() != expected) {
        throw std::invalid_argument("storage row byte size mismatch: expected " + std::to_string(expected) +
                                    ", received " + std::to_string(bytes.size()));
    }
    if (!oq_type_supported(type)) {
        throw std::invalid_argument("storage decoder does not support GGML type " + std::to_string(type));
    }
    if (vector.size() != element_count) throw std::invalid_argument("reference dot vector length mismatch");
    float out = 0.0F;
    storage_matvec(type, 1, element_count, bytes, vector, std::span<float>(&out, 1));
    return out;
}

std::uint32_t QuantizedDevice::greedy_token(std::span<const float> logits) {
    // the sampler's argument checks, in its order (src/runtime/sampler.cpp:23-28)
    if (logits.empty()) throw std::invalid_argument("cannot sample an empty logits vector");
    if (logits.size() > std::numeric_limits<std::uint32_t>::max()) {
        throw std::invalid_argument("logits vector exceeds token-id range");
    }
    float* x = device_floats(x_dev_, x_cap_, logits.size());
    float* t = device_floats(t_dev_, t_cap_, 2);  // [0]: token bits, [1]: value
    check(oq_copy_to_device(ctx_, x, logits.data(), logits.size_bytes()), ctx_);
    check(oq_argmax(ctx_, x, logits.size(), reinterpret_cast<std::uint32_t*>(t), t + 1), ctx_);
    std::uint32_t token = 0;
    float value = 0.0F;
    check(oq_copy_to_host(ctx_, &token, t, sizeof(token)), ctx_);
    check(oq_copy_to_host(ctx_, &value, t + 1, sizeof(value)), ctx_);
    if (token == 0xFFFFFFFFu) throw std::invalid_argument("logits contain NaN");
    if (!std::isfinite(value)) throw std::invalid_argument("logits contain no finite candidates");
    return token;
}

void QuantizedDevice::decode_rows(std::uint32_t type, std::size_t rows, std::size_t cols,
                                  std::span<const std::byte> matrix_bytes, std::span<float> output) {
    std::uint64_t row_bytes = 0;
    check(oq_row_byte_size(cols, type, &row_bytes), nullptr);
    if (rows != 0 && row_bytes > std::numeric_limits<std::size_t>::max() / rows) {
        throw std::overflow_error("GGUF tensor byte size exceeds addressable size");
    }
    if (matrix_bytes.size() != row_bytes * rows) {
        throw std::invalid_argument("GGUF tensor byte size does not match row geometry");
    }
    if (!oq_type_supported(type)) {
        throw std::invalid_argument("storage decoder does not support GGML type " + std::to_string(type));
    }
    if (cols != 0 && rows > std::numeric_limits<std::size_t>::max() / cols) {
        throw std::overflow_error("mapped tensor element count overflow");
    }
    if (output.size() != rows * cols) throw std::invalid_argument("mapped tensor decode output length mismatch");
    Transient t;
    check(oq_weight_upload(context(), type, cols, rows, matrix_bytes.data(), matrix_bytes.size(), &t.w), ctx_);
    float* out = device_floats(y_dev_, y_cap_, output.size());
    check(oq_dequantize_rows(ctx_, t.w, 0, rows, out), ctx_);
    check(oq_copy_to_host(ctx_, output.data(), out, output.size_bytes()), ctx_);
}

}  // namespace oracle::backend::hip
