// Whole-model one-time upload into a name-keyed device registry (oq_model_* in include/oq.h).
//
// The reference maps a GGUF file once and hands out zero-copy tensor views
// (MappedGgufModel, src/model/mapped_gguf.cpp:124-203); every projection then runs on its view.
// Here the mapped payload goes to HBM once: tensors are validated with the reference's checks
// and in its order (registered type, byte size from the dimensions, payload bounds, unique
// names, no overlapping payloads), then streamed through a bounded staging buffer in payload
// order.  Rank-2 tensors of a type the device path multiplies become weights in the device row
// layout (one relayout kernel each); every other tensor keeps its GGML bytes in one HBM region.
// Lookups are by name, as MappedGgufModel::find_tensor / tensor (:211-222).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <cstring>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/oq.h"
#include "oq_internal.h"

namespace {

constexpr uint64_t kStagingBytes = 256ull << 20;

uint64_t up256(uint64_t v) { return (v + 255) & ~uint64_t(255); }

struct Entry {
    std::string name;
    uint32_t type = 0;
    uint32_t n_dims = 0;
    uint64_t dims[4] = {0, 0, 0, 0};
    uint64_t offset = 0;   // in the caller's payload
    uint64_t nbytes = 0;   // GGML bytes
    oq_weight* weight = nullptr;
    uint64_t raw_off = UINT64_MAX;  // offset in the raw region (tensors without a weight)
};

// checked a * b (GGML byte-size arithmetic, src/model/ggml_type.cpp:56-64)
bool mul_ok(uint64_t a, uint64_t b, uint64_t* out) {
    if (a != 0 && b > UINT64_MAX / a) return false;
    *out = a * b;
    return true;
}

// Validation of a tensor table in the reference's order; fills entries.  First the container
// checks of its GGUF reader over the whole table (src/model/gguf.cpp:457-497: unique names,
// dimension count, non-zero dimensions, offsets inside the payload), then the mapping checks per
// tensor (src/model/mapped_gguf.cpp:139-157: registered type, byte size from the dimensions,
// payload end inside the payload), then overlaps (:177-189).
int validate(uint64_t payload_bytes, const oq_tensor_desc* t, uint64_t count, std::vector<Entry>& entries,
             std::string& msg) {
    if (count != 0 && t == nullptr) {
        msg = "null tensor table";
        return OQ_INVALID_ARGUMENT;
    }
    entries.clear();
    entries.reserve(count);
    std::unordered_map<std::string, uint64_t> names;
    for (uint64_t i = 0; i < count; ++i) {
        const oq_tensor_desc& d = t[i];
        if (d.name == nullptr) {
            msg = "null tensor name";
            return OQ_INVALID_ARGUMENT;
        }
        if (!names.emplace(d.name, i).second) {
            msg = std::string("duplicate GGUF tensor name: ") + d.name;
            return OQ_RUNTIME_ERROR;
        }
        if (d.n_dims == 0 || d.n_dims > 64) {
            msg = "GGUF tensor dimension count is invalid";
            return OQ_RUNTIME_ERROR;
        }
        if (d.n_dims > 4) {
            msg = std::string("tensors of more than four dimensions are not supported: ") + d.name;
            return OQ_INVALID_ARGUMENT;
        }
        for (uint32_t k = 0; k < d.n_dims; ++k) {
            if (d.dims[k] == 0) {
                msg = "GGUF tensor dimensions must be non-zero";
                return OQ_RUNTIME_ERROR;
            }
        }
    }
    for (uint64_t i = 0; i < count; ++i) {
        if (t[i].offset > payload_bytes) {
            msg = std::string("GGUF tensor offset exceeds file size: ") + t[i].name;
            return OQ_RUNTIME_ERROR;
        }
    }
    for (uint64_t i = 0; i < count; ++i) {
        const oq_tensor_desc& d = t[i];
        Entry e;
        e.name = d.name;
        e.type = d.type;
        const char* lname = nullptr;
        uint64_t be = 0, bpb = 0;
        if (oq_type_layout(d.type, &be, &bpb, nullptr, &lname) != OQ_OK) {
            msg = "unsupported GGML tensor type " + std::to_string(d.type) + " for tensor " + e.name;
            return OQ_UNSUPPORTED_TYPE;
        }
        // ggml_tensor_byte_size (src/model/ggml_type.cpp:96-118)
        uint64_t elements = 1;
        for (uint32_t k = 0; k < d.n_dims; ++k) {
            if (!mul_ok(elements, d.dims[k], &elements)) {
                msg = "GGML tensor element count overflow";
                return OQ_OVERFLOW;
            }
        }
        uint64_t bytes = 0;
        const int rc = oq_row_byte_size(d.dims[0], d.type, &bytes);
        if (rc != OQ_OK) {
            msg = oq_last_error(nullptr);
            return rc;
        }
        for (uint32_t k = 1; k < d.n_dims; ++k) {
            if (!mul_ok(bytes, d.dims[k], &bytes)) {
                msg = "GGML tensor byte size overflow";
                return OQ_OVERFLOW;
            }
        }
        if (bytes > payload_bytes - d.offset) {
            msg = "GGUF tensor payload exceeds file size: " + e.name;
            return OQ_RUNTIME_ERROR;
        }
        e.n_dims = d.n_dims;
        for (uint32_t k = 0; k < d.n_dims; ++k) e.dims[k] = d.dims[k];
        e.offset = d.offset;
        e.nbytes = bytes;
        entries.push_back(e);
    }
    // payloads sorted by (begin, end) must not overlap
    std::vector<uint64_t> order(entries.size());
    for (uint64_t i = 0; i < order.size(); ++i) order[i] = i;
    std::sort(order.begin(), order.end(), [&](uint64_t a, uint64_t b) {
        const Entry &x = entries[a], &y = entries[b];
        return x.offset != y.offset ? x.offset < y.offset : x.offset + x.nbytes < y.offset + y.nbytes;
    });
    for (uint64_t i = 1; i < order.size(); ++i) {
        const Entry &prev = entries[order[i - 1]], &cur = entries[order[i]];
        if (cur.offset < prev.offset + prev.nbytes) {
            msg = "GGUF tensor payloads overlap: " + prev.name + " and " + cur.name;
            return OQ_RUNTIME_ERROR;
        }
    }
    return OQ_OK;
}

bool becomes_weight(const Entry& e) { return e.n_dims == 2 && oq_type_supported(e.type); }

}  // namespace

struct oq_model {
    std::vector<Entry> entries;
    std::unordered_map<std::string, uint64_t> index;
    void* raw = nullptr;
    uint64_t raw_bytes = 0;
    int device = 0;

    ~oq_model() {
        for (Entry& e : entries) oq_weight_release(e.weight);
        if (raw) {
            (void)hipSetDevice(device);
            (void)hipFree(raw);
        }
    }
};

extern "C" {

int oq_model_validate(uint64_t payload_bytes, const oq_tensor_desc* tensors, uint64_t count) {
    std::vector<Entry> entries;
    std::string msg;
    const int rc = validate(payload_bytes, tensors, count, entries, msg);
    if (rc != OQ_OK) oq::set_error(nullptr, rc, msg.c_str());
    return rc;
}

int oq_model_upload(oq_context* ctx, const void* payload, uint64_t payload_bytes, const oq_tensor_desc* tensors,
                    uint64_t count, oq_model** out) {
    if (!ctx) return oq::set_error(nullptr, OQ_INVALID_ARGUMENT, "null context");
    if (!out) return oq::set_error(ctx, OQ_INVALID_ARGUMENT, "null output handle");
    *out = nullptr;
    if (!payload && payload_bytes != 0) return oq::set_error(ctx, OQ_INVALID_ARGUMENT, "null payload");
    oq_model* m = new oq_model;
    m->device = oq::context_device(ctx);
    std::string msg;
    int rc = validate(payload_bytes, tensors, count, m->entries, msg);
    if (rc != OQ_OK) {
        delete m;
        return oq::set_error(ctx, rc, msg.c_str());
    }
    auto fail = [&](int code, const std::string& what) {
        delete m;
        return oq::set_error(ctx, code, what.c_str());
    };
    // the raw region: every tensor that does not become a weight, 256-byte aligned each
    for (Entry& e : m->entries) {
        if (becomes_weight(e)) continue;
        e.raw_off = m->raw_bytes;
        m->raw_bytes += up256(e.nbytes);
    }
    hipStream_t s = static_cast<hipStream_t>(oq_context_stream(ctx));
    if (hipSetDevice(m->device) != hipSuccess) return fail(OQ_DEVICE_ERROR, "hipSetDevice");
    if (m->raw_bytes && hipMalloc(&m->raw, m->raw_bytes) != hipSuccess) {
        return fail(OQ_OUT_OF_MEMORY, "hipMalloc(model raw tensors)");
    }
    // staging: whole tensors in payload order, at most max(kStagingBytes, largest tensor)
    std::vector<uint64_t> order(m->entries.size());
    for (uint64_t i = 0; i < order.size(); ++i) order[i] = i;
    std::sort(order.begin(), order.end(), [&](uint64_t a, uint64_t b) { return m->entries[a].offset < m->entries[b].offset; });
    uint64_t largest = 0;
    for (const Entry& e : m->entries) largest = std::max(largest, e.nbytes);
    const uint64_t cap = std::max(kStagingBytes, up256(largest));
    void* staging = nullptr;
    if (!m->entries.empty() && hipMalloc(&staging, std::min(cap, up256(payload_bytes) + 256)) != hipSuccess) {
        return fail(OQ_OUT_OF_MEMORY, "hipMalloc(model staging)");
    }
    const uint8_t* host = static_cast<const uint8_t*>(payload);
    uint64_t i = 0;
    while (i < order.size()) {
        // a batch of consecutive tensors whose payload span fits the staging buffer
        const uint64_t first = m->entries[order[i]].offset;
        uint64_t j = i, end = first;
        while (j < order.size()) {
            const Entry& e = m->entries[order[j]];
            const uint64_t e_end = e.offset + e.nbytes;
            if (e_end - first > cap) break;
            end = std::max(end, e_end);
            ++j;
        }
        hipError_t he = hipMemcpyAsync(staging, host + first, end - first, hipMemcpyHostToDevice, s);
        if (he == hipSuccess) he = hipStreamSynchronize(s);
        if (he != hipSuccess) {
            (void)hipFree(staging);
            return fail(OQ_DEVICE_ERROR, std::string("model upload: ") + hipGetErrorString(he));
        }
        for (uint64_t k = i; k < j; ++k) {
            Entry& e = m->entries[order[k]];
            const uint8_t* src = static_cast<const uint8_t*>(staging) + (e.offset - first);
            if (becomes_weight(e)) {
                rc = oq_weight_upload_device(ctx, e.type, e.dims[0], e.dims[1], src, e.nbytes, &e.weight);
                if (rc != OQ_OK) {
                    const std::string why = std::string("tensor ") + e.name + ": " + oq_last_error(ctx);
                    (void)hipFree(staging);
                    return fail(rc, why);
                }
            } else {
                he = hipMemcpyAsync(static_cast<uint8_t*>(m->raw) + e.raw_off, src, e.nbytes, hipMemcpyDeviceToDevice, s);
                if (he != hipSuccess) {
                    (void)hipFree(staging);
                    return fail(OQ_DEVICE_ERROR, std::string("model upload: ") + hipGetErrorString(he));
                }
            }
        }
        if (hipStreamSynchronize(s) != hipSuccess) {
            (void)hipFree(staging);
            return fail(OQ_DEVICE_ERROR, "model upload: stream synchronization");
        }
        i = j;
    }
    if (staging) (void)hipFree(staging);
    for (uint64_t k = 0; k < m->entries.size(); ++k) m->index.emplace(m->entries[k].name, k);
    *out = m;
    return OQ_OK;
}

void oq_model_release(oq_model* m) { delete m; }

uint64_t oq_model_tensor_count(const oq_model* m) { return m ? m->entries.size() : 0; }

int oq_model_find(const oq_model* m, const char* name, uint64_t* index) {
    if (!m || !name || !index) return oq::set_error(nullptr, OQ_INVALID_ARGUMENT, "null argument");
    const auto it = m->index.find(name);
    if (it == m->index.end()) {
        return oq::set_error(nullptr, OQ_OUT_OF_RANGE, (std::string("GGUF tensor not found: ") + name).c_str());
    }
    *index = it->second;
    return OQ_OK;
}

int oq_model_tensor(const oq_model* m, uint64_t index, oq_model_tensor_info* info) {
    if (!m || !info) return oq::set_error(nullptr, OQ_INVALID_ARGUMENT, "null argument");
    if (index >= m->entries.size()) return oq::set_error(nullptr, OQ_OUT_OF_RANGE, "model tensor index out of range");
    const Entry& e = m->entries[index];
    info->name = e.name.c_str();
    info->type = e.type;
    info->n_dims = e.n_dims;
    for (int k = 0; k < 4; ++k) info->dims[k] = e.dims[k];
    info->nbytes = e.nbytes;
    info->weight = e.weight;
    info->data_dev = e.weight ? nullptr : static_cast<const uint8_t*>(m->raw) + e.raw_off;
    return OQ_OK;
}

uint64_t oq_model_device_bytes(const oq_model* m) {
    if (!m) return 0;
    uint64_t total = m->raw_bytes;
    for (const Entry& e : m->entries) {
        uint64_t b = 0;
        if (e.weight) (void)oq_weight_info(e.weight, nullptr, nullptr, nullptr, &b);
        total += b;
    }
    return total;
}

}  // extern "C"
