// Tests of the C++ host adapter (hip_quantized.hpp), in the reference's own test style: known
// answers from the reference's quantized-path fixtures, exception kinds for malformed input, and
// (with "gpu") device results checked against the CPU oracle (oracle/oracle.h, test-only).
//
//   adapter_test cpu   -- validation and exception kinds only; never touches a GPU
//   adapter_test gpu   -- everything, on device 0
#include <algorithm>
#include <array>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <exception>
#include <iostream>
#include <span>
#include <stdexcept>
#include <string>
#include <vector>

#include "../../oracle/oracle.h"
#include "hip_quantized.hpp"

namespace {

using oracle::backend::hip::QuantizedDevice;

void require(bool ok, const std::string& what) {
    if (!ok) throw std::runtime_error(what);
}

template <typename E, typename F>
void require_throws(F&& f, const std::string& what) {
    try {
        f();
    } catch (const E&) {
        return;
    } catch (const std::exception& e) {
        throw std::runtime_error(what + ": wrong exception kind: " + e.what());
    }
    throw std::runtime_error(what + ": nothing thrown");
}

// A tensor view with GgufTensorView's accessors (dimensions(), bytes(), layout().type).
struct Layout {
    std::uint32_t type;
};
struct View {
    std::vector<std::uint64_t> dims;
    std::span<const std::byte> data;
    Layout lay;
    std::string nm = "fixture.weight";
    std::span<const std::uint64_t> dimensions() const { return dims; }
    std::span<const std::byte> bytes() const { return data; }
    const Layout& layout() const { return lay; }
    std::string_view name() const { return nm; }
};

std::span<const std::byte> as_bytes(const std::vector<std::uint8_t>& v) {
    return {reinterpret_cast<const std::byte*>(v.data()), v.size()};
}

void put16(std::vector<std::uint8_t>& b, std::size_t at, std::uint16_t v) {
    b[at] = static_cast<std::uint8_t>(v & 0xFF);
    b[at + 1] = static_cast<std::uint8_t>(v >> 8);
}

// The reference's quantized-path fixtures (tests/test_phase2a.cpp of the reference), as bytes.
std::vector<std::uint8_t> q5_block() {
    std::vector<std::uint8_t> b(176, 0x21);
    put16(b, 0, 0x3800);
    put16(b, 2, 0x3400);
    const std::uint8_t sc[12] = {2, 2, 2, 2, 3, 3, 3, 3, 0x32, 0x32, 0x32, 0x32};
    std::copy(sc, sc + 12, b.begin() + 4);
    std::fill(b.begin() + 16, b.begin() + 48, 0xFF);
    return b;
}
std::vector<std::uint8_t> q6_block() {
    std::vector<std::uint8_t> b(210, 0x21);
    std::fill(b.begin() + 128, b.begin() + 192, 0xFF);
    std::fill(b.begin() + 192, b.begin() + 208, 0x02);
    put16(b, 208, 0x3800);
    return b;
}
std::vector<std::uint8_t> q8_0_block(bool ramp) {
    std::vector<std::uint8_t> b(34, 4);
    if (ramp) {
        const std::int8_t q[32] = {0, 1, -1, 127, -128, 2, -2, 3, -3, 4, -4, 5, -5, 6, -6, 7,
                                   -7, 8, -8, 9, -9, 10, -10, 11, -11, 12, -12, 13, -13, 14, -14, 15};
        for (int i = 0; i < 32; ++i) b[2 + i] = static_cast<std::uint8_t>(q[i]);
        put16(b, 0, 0x3C00);
    } else {
        put16(b, 0, 0x3800);
    }
    return b;
}

void test_validation_kinds() {
    QuantizedDevice dev;  // no context is created by argument errors
    std::vector<std::uint8_t> q4(2 * 144, 0);
    std::vector<float> x(256, 1.0F), y(2, 0.0F);
    const auto m = as_bytes(q4);
    require_throws<std::invalid_argument>([&] { dev.storage_matvec(12, 0, 256, m, x, y); }, "zero rows");
    require_throws<std::invalid_argument>(
        [&] { dev.storage_matvec(12, 2, 256, m, std::span<const float>(x).first(255), y); }, "vector length");
    require_throws<std::invalid_argument>(
        [&] { dev.storage_matvec(12, 2, 256, m, x, std::span<float>(y).first(1)); }, "output length");
    require_throws<std::runtime_error>([&] { dev.storage_matvec(99, 2, 256, m, x, y); }, "unregistered type");
    std::vector<float> x250(250, 1.0F);
    require_throws<std::runtime_error>([&] { dev.storage_matvec(12, 2, 250, m, x250, y); }, "ragged row");
    require_throws<std::invalid_argument>(
        [&] { dev.storage_matvec(12, 2, 256, m.first(m.size() - 1), x, y); }, "matrix byte size");
    std::vector<std::uint8_t> q40(2 * 8 * 18, 0);
    require_throws<std::invalid_argument>(
        [&] { dev.storage_matvec(2, 2, 256, as_bytes(q40), x, y); }, "q4_0 is not decodable");
    View rank3{{256, 1, 2}, m, {12}};
    require_throws<std::invalid_argument>([&] { dev.mapped_tensor_matvec(rank3, x, y); }, "rank-3 view");
    require_throws<std::invalid_argument>(
        [&] { (void)dev.storage_dot({12, 256, m.first(143)}, x); }, "truncated row");
    require_throws<std::invalid_argument>(
        [&] { (void)dev.storage_dot({12, 256, m.first(144)}, std::span<const float>(x).first(10)); },
        "dot vector length");
    std::vector<float> out(3);
    View v{{256, 2}, m, {12}};
    require_throws<std::invalid_argument>([&] { dev.decode_mapped_tensor(v, out); }, "decode output length");
    require(dev.resident_count() == 0, "argument errors must not upload anything");
}

void test_reference_known_answers(QuantizedDevice& dev) {
    // Q5_K: 16.25 / 17.25 per 64-group, dot(ones) = 4288; second row (qh, qs cleared) = -192
    auto q5 = q5_block();
    std::vector<float> dec(256);
    View v5{{256, 1}, as_bytes(q5), {13}};
    dev.decode_mapped_tensor(v5, dec);
    for (int g = 0; g < 4; ++g)
        for (int l = 0; l < 32; ++l) {
            require(dec[g * 64 + l] == 16.25F, "Q5_K low-half known answer");
            require(dec[g * 64 + 32 + l] == 17.25F, "Q5_K high-half known answer");
        }
    std::vector<float> ones(256, 1.0F);
    auto two = q5;
    auto second = q5;
    std::fill(second.begin() + 16, second.end(), 0);
    two.insert(two.end(), second.begin(), second.end());
    std::vector<float> y(2);
    View vm{{256, 2}, as_bytes(two), {13}};
    dev.mapped_tensor_matvec(vm, ones, y);
    // Q8_K activations: 1.0 quantizes exactly (d = -1/127, q = -127), so these stay exact up to
    // the F32 rounding of d
    require(std::fabs(y[0] - 4288.0F) <= 4288.0F * 1e-6F, "Q5_K matvec first row");
    require(std::fabs(y[1] + 192.0F) <= 192.0F * 1e-6F, "Q5_K matvec second row");
    // Q6_K: 17 / 18, dot(ones) = 4480
    auto q6 = q6_block();
    View v6{{256, 1}, as_bytes(q6), {14}};
    dev.decode_mapped_tensor(v6, dec);
    for (int h = 0; h < 2; ++h)
        for (int l = 0; l < 64; ++l) {
            require(dec[h * 128 + l] == 17.0F, "Q6_K lower known answer");
            require(dec[h * 128 + 64 + l] == 18.0F, "Q6_K upper known answer");
        }
    const float d6 = dev.storage_dot({14, 256, as_bytes(q6)}, ones);
    require(std::fabs(d6 - 4480.0F) <= 4480.0F * 1e-6F, "Q6_K dot");
    // Q8_0 (F32 activations, exact): dot(ones) = 14 and 64
    auto q8 = q8_0_block(true);
    auto q8b = q8_0_block(false);
    q8.insert(q8.end(), q8b.begin(), q8b.end());
    std::vector<float> ones32(32, 1.0F);
    View v8{{32, 2}, as_bytes(q8), {8}};
    dev.mapped_tensor_matvec(v8, ones32, y);
    require(y[0] == 14.0F && y[1] == 64.0F, "Q8_0 matvec known answers");
}

std::uint64_t g_state = 0x243F6A8885A308D3ull;
std::uint64_t next_u64() {
    g_state ^= g_state << 13;
    g_state ^= g_state >> 7;
    g_state ^= g_state << 17;
    return g_state;
}

void test_against_oracle(QuantizedDevice& dev, std::uint32_t type, std::size_t rows, std::size_t cols) {
    std::uint64_t rb = 0;
    require(orc_row_byte_size(cols, type, &rb) == 0, "row bytes");
    std::vector<std::uint8_t> data(rows * rb);
    for (auto& b : data) b = static_cast<std::uint8_t>(next_u64());
    // finite, moderate f16 scales
    const std::size_t blk = type == 8 ? 34 : (type == 14 ? 210 : 144);
    for (std::size_t off = 0; off < data.size(); off += blk) {
        const std::uint16_t s = static_cast<std::uint16_t>(0x1000 + (next_u64() % 0x1800));
        if (type == 14) put16(data, off + 208, s);
        else put16(data, off, s);
        if (type == 12) put16(data, off + 2, static_cast<std::uint16_t>(0x1000 + (next_u64() % 0x1800)));
    }
    std::vector<float> x(cols);
    for (auto& v : x) v = static_cast<float>(static_cast<std::int64_t>(next_u64() % 2001) - 1000) / 250.0F;
    std::vector<float> y(rows);
    View view{{cols, rows}, as_bytes(data), {type}};
    dev.mapped_tensor_matvec(view, x, y);
    dev.mapped_tensor_matvec(view, x, y);  // resident: no second upload
    std::vector<float> xhat = x;
    if (type != 8) {
        std::vector<std::uint8_t> q8(cols / 256 * 292);
        orc_quantize_row_q8_k(x.data(), cols, q8.data());
        orc_dequantize_row_q8_k(q8.data(), cols, xhat.data());
    }
    for (std::size_t r = 0; r < rows; ++r) {
        double dot = 0, ab = 0;
        require(orc_storage_dot_stats(type, cols, data.data() + r * rb, rb, xhat.data(), &dot, &ab) == 0, "stats");
        float ref = 0;
        orc_storage_dot(type, cols, data.data() + r * rb, rb, xhat.data(), &ref);
        require(std::fabs(static_cast<double>(y[r]) - ref) <= 1e-4 * ab,
                "matvec tolerance, type " + std::to_string(type) + " row " + std::to_string(r));
    }
    // bit-exact decode
    std::vector<float> dec(rows * cols), want(cols);
    dev.decode_mapped_tensor(view, dec);
    for (std::size_t r = 0; r < rows; ++r) {
        orc_decode_row(type, cols, data.data() + r * rb, rb, want.data());
        require(std::memcmp(want.data(), dec.data() + r * cols, cols * 4) == 0, "decode bit-exact");
    }
    // M = 3 through the matmul form
    std::vector<float> x3(3 * cols), y3(3 * rows);
    for (int m = 0; m < 3; ++m) std::copy(x.begin(), x.end(), x3.begin() + m * cols);
    dev.mapped_tensor_matmul(view, 3, x3, y3);
    // the batched kernel sums in another order than the batch-1 kernel: same tolerance bar
    for (int m = 0; m < 3; ++m)
        for (std::size_t r = 0; r < rows; ++r) {
            double dot = 0, ab = 0;
            orc_storage_dot_stats(type, cols, data.data() + r * rb, rb, xhat.data(), &dot, &ab);
            require(std::fabs(static_cast<double>(y3[m * rows + r]) - y[r]) <= 2e-4 * ab, "matmul rows match matvec");
        }
}

// greedy token against the reference's loop (first index of the strict maximum) and the
// sampler's errors
void test_greedy_token(QuantizedDevice& dev) {
    require(dev.greedy_token(std::vector<float>{1.0F, 5.0F, 5.0F, 2.0F}) == 1, "ties: the first index");
    require(dev.greedy_token(std::vector<float>{-3.0F}) == 0, "one logit");
    const float inf = std::numeric_limits<float>::infinity();
    require_throws<std::invalid_argument>([&] { (void)dev.greedy_token(std::vector<float>{}); }, "empty logits");
    require_throws<std::invalid_argument>(
        [&] { (void)dev.greedy_token(std::vector<float>{1.0F, std::nanf("")}); }, "NaN logits");
    require_throws<std::invalid_argument>([&] { (void)dev.greedy_token(std::vector<float>{-inf, -inf}); },
                                          "no finite candidate");
    std::vector<float> v(151936);
    std::uint64_t s = 0x9E3779B97F4A7C15ull;
    for (float& e : v) {
        s ^= s << 13;
        s ^= s >> 7;
        s ^= s << 17;
        e = static_cast<float>(static_cast<int>(s % 2001) - 1000);  // many ties
    }
    std::size_t best = 0;
    for (std::size_t i = 1; i < v.size(); ++i)
        if (v[i] > v[best]) best = i;
    require(dev.greedy_token(v) == best, "greedy token matches the reference loop");
}

// raw caller-owned bytes are not cached: a buffer reused with new contents gives new results
void test_raw_spans_follow_their_bytes(QuantizedDevice& dev) {
    const std::size_t rows = 8, cols = 256;
    std::vector<std::uint8_t> data(rows * 144);
    std::vector<float> x(cols, 1.0F), y(rows);
    for (int round = 0; round < 2; ++round) {
        for (auto& b : data) b = static_cast<std::uint8_t>(next_u64());
        for (std::size_t r = 0; r < rows; ++r) {
            put16(data, r * 144, 0x2000);
            put16(data, r * 144 + 2, 0x1800);
        }
        const std::size_t before = dev.resident_count();
        dev.storage_matvec(12, rows, cols, as_bytes(data), x, y);
        require(dev.resident_count() == before, "raw spans are not kept resident");
        std::vector<float> xhat(cols);
        std::vector<std::uint8_t> q8(292);
        orc_quantize_row_q8_k(x.data(), cols, q8.data());
        orc_dequantize_row_q8_k(q8.data(), cols, xhat.data());
        for (std::size_t r = 0; r < rows; ++r) {
            double dot = 0, ab = 0;
            orc_storage_dot_stats(12, cols, data.data() + r * 144, 144, xhat.data(), &dot, &ab);
            require(std::fabs(static_cast<double>(y[r]) - dot) <= 1e-4 * ab, "reused buffer: new contents multiplied");
        }
    }
}

// A model with MappedGgufModel's accessors: tensors() of views with name() and
// absolute_offset(), mapping() with data() and size().
struct ModelView {
    std::string nm;
    std::vector<std::uint64_t> dims;
    std::span<const std::byte> data;
    Layout lay;
    std::uint64_t abs;
    std::string_view name() const { return nm; }
    std::span<const std::uint64_t> dimensions() const { return dims; }
    std::span<const std::byte> bytes() const { return data; }
    const Layout& layout() const { return lay; }
    std::uint64_t absolute_offset() const { return abs; }
};
struct Mapping {
    const std::byte* p;
    std::size_t n;
    const std::byte* data() const { return p; }
    std::size_t size() const { return n; }
};
struct FakeModel {
    std::vector<ModelView> views;
    Mapping map;
    const std::vector<ModelView>& tensors() const { return views; }
    const Mapping& mapping() const { return map; }
};

void test_model_upload(QuantizedDevice& dev) {
    // payload: a 64-byte header, then a q4_K matrix (40 x 512), a q6_K matrix (12 x 256), an F32 vector
    const std::size_t r1 = 40, c1 = 512, r2 = 12, c2 = 256;
    std::vector<std::uint8_t> payload(64 + r1 * 2 * 144 + r2 * 210 + 64 + 256 * 4, 0);
    for (std::size_t i = 64; i < payload.size(); ++i) payload[i] = static_cast<std::uint8_t>(next_u64());
    const std::size_t o1 = 64, o2 = o1 + r1 * 2 * 144, o3 = (o2 + r2 * 210 + 63) / 64 * 64;
    for (std::size_t b = 0; b < r1 * 2; ++b) {
        put16(payload, o1 + b * 144, 0x2000);
        put16(payload, o1 + b * 144 + 2, 0x1800);
    }
    for (std::size_t b = 0; b < r2; ++b) put16(payload, o2 + b * 210 + 208, 0x2000);
    const std::byte* base = reinterpret_cast<const std::byte*>(payload.data());
    FakeModel m{{{"blk.0.ffn_up.weight", {c1, r1}, {base + o1, r1 * 2 * 144}, {12}, o1},
                 {"blk.0.attn_output.weight", {c2, r2}, {base + o2, r2 * 210}, {14}, o2},
                 {"blk.0.attn_norm.weight", {256}, {base + o3, 1024}, {0}, o3}},
                {base, payload.size()}};
    const std::size_t resident_before = dev.resident_count();
    dev.upload_model(m);
    require(dev.model() != nullptr && oq_model_tensor_count(dev.model()) == 3, "model registered");
    for (int t = 0; t < 2; ++t) {
        const ModelView& v = m.views[t];
        const std::size_t rows = v.dims[1], cols = v.dims[0];
        const std::uint64_t rb = v.data.size() / rows;
        std::vector<float> x(cols), y(rows);
        for (auto& e : x) e = static_cast<float>(static_cast<std::int64_t>(next_u64() % 2001) - 1000) / 500.0F;
        dev.mapped_tensor_matvec(v, x, y);
        std::vector<float> xhat(cols);
        std::vector<std::uint8_t> q8(cols / 256 * 292);
        orc_quantize_row_q8_k(x.data(), cols, q8.data());
        orc_dequantize_row_q8_k(q8.data(), cols, xhat.data());
        const auto* raw = reinterpret_cast<const std::uint8_t*>(v.data.data());
        for (std::size_t r = 0; r < rows; ++r) {
            double dot = 0, ab = 0;
            orc_storage_dot_stats(v.lay.type, cols, raw + r * rb, rb, xhat.data(), &dot, &ab);
            require(std::fabs(static_cast<double>(y[r]) - dot) <= 1e-4 * ab, "model weight multiplies like the oracle");
        }
        // the same product with activations and outputs in device memory
        void *xd = nullptr, *yd = nullptr;
        require(oq_device_alloc(dev.context(), cols * 4, &xd) == 0 && oq_device_alloc(dev.context(), rows * 4, &yd) == 0,
                "device buffers");
        require(oq_copy_to_device(dev.context(), xd, x.data(), cols * 4) == 0, "upload x");
        dev.mapped_tensor_matmul_device(v, 1, static_cast<const float*>(xd), static_cast<float*>(yd));
        dev.synchronize();
        std::vector<float> yd_host(rows);
        require(oq_copy_to_host(dev.context(), yd_host.data(), yd, rows * 4) == 0, "download y");
        require(std::memcmp(yd_host.data(), y.data(), rows * 4) == 0, "device-pointer product equals the host form");
        oq_device_free(dev.context(), xd);
        oq_device_free(dev.context(), yd);
    }
    require(dev.resident_count() == resident_before, "model tensors are served from the model, not uploaded again");
    // a malformed model fails like MappedGgufModel: overlapping payloads
    FakeModel bad{{m.views[0], m.views[1]}, m.map};
    bad.views[1].abs = o1 + 16;
    require_throws<std::runtime_error>([&] { dev.upload_model(bad); }, "overlapping payloads");
}

}  // namespace

int main(int argc, char** argv) {
    const bool gpu = argc > 1 && std::string(argv[1]) == "gpu";
    try {
        test_validation_kinds();
        if (gpu) {
            QuantizedDevice dev(0);
            test_reference_known_answers(dev);
            test_against_oracle(dev, 12, 300, 4096);
            test_against_oracle(dev, 14, 130, 2048);
            test_against_oracle(dev, 8, 200, 4096);
            test_greedy_token(dev);
            require(dev.resident_count() == 2 + 3, "one resident copy per distinct mapped tensor");
            test_raw_spans_follow_their_bytes(dev);
            test_model_upload(dev);
        }
        std::cout << "host adapter tests passed (" << (gpu ? "gpu" : "cpu") << ")\n";
    } catch (const std::exception& e) {
        std::cerr << "host adapter test failure: " << e.what() << '\n';
        return 1;
    }
    return 0;
}
