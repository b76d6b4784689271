// Dispatch of the K-quant (q4_K, q5_K, q6_K) decode GEMV and small-batch products
// (oq_gemv_kq.h; instantiated per type and activation form in oq_gemv_inst.hip).
//
// Rows of up to 16384 elements whose Q8_K image fits the LDS budget run the compile-time kernels
// (activation slices in registers, every pass unrolled), at most 8 activation rows per launch.
// Longer rows run the windowed kernel: consecutive launches over windows of passes, each adding
// its partial sums to y, at most two activation rows per launch.
#include "oq_gemv_kq.h"

namespace oq {

namespace {

template <bool FUSED>
hipError_t launch_type(const DeviceMatrix& w, int m, const float* x, const uint8_t* q8k, float* y, hipStream_t s) {
    switch (w.type) {
        case 12: return launch_kq<12, FUSED>(w, m, x, q8k, y, s);
        case 13: return launch_kq<13, FUSED>(w, m, x, q8k, y, s);
        case 14: return launch_kq<14, FUSED>(w, m, x, q8k, y, s);
        default: return hipErrorInvalidValue;
    }
}

template <bool FUSED>
hipError_t launch_type_window(const DeviceMatrix& w, int m, const float* x, const uint8_t* q8k, float* y,
                              uint32_t pass0, uint32_t npass, int accumulate, hipStream_t s) {
    switch (w.type) {
        case 12: return launch_kq_window<12, FUSED>(w, m, x, q8k, y, pass0, npass, accumulate, s);
        case 13: return launch_kq_window<13, FUSED>(w, m, x, q8k, y, pass0, npass, accumulate, s);
        case 14: return launch_kq_window<14, FUSED>(w, m, x, q8k, y, pass0, npass, accumulate, s);
        default: return hipErrorInvalidValue;
    }
}

bool short_rows(const DeviceMatrix& w) {
    return (w.k / kQK + 15) / 16 <= (uint64_t)kq::kMaxIters && kq::act_lds_bytes(w.k, 1) <= kq::kLdsBudget;
}

}  // namespace

int gemv_max_m() { return 8; }

bool gemv_kquant_supported(const DeviceMatrix& w) {
    return (w.type == 12 || w.type == 13 || w.type == 14) && w.k > 0 && w.k % kQK == 0;
}

uint32_t gemv_window_passes(const DeviceMatrix& w, int m) {
    if (short_rows(w)) return 0;
    const int rows = m >= 2 ? 2 : 1;
    const uint64_t per_pass = kq::act_lds_bytes(16 * kQK, rows);  // LDS image of one pass of `rows` rows
    const uint64_t win = kq::kLdsBudget / per_pass;
    return (uint32_t)(win < 1 ? 1 : win);
}

hipError_t launch_gemv_kquant_argmax(const DeviceMatrix& w, const float* x, const uint8_t* q8k, float* y,
                                     ArgmaxPart* parts, uint32_t max_parts, uint32_t* nparts, hipStream_t s) {
    if (!gemv_kquant_supported(w) || !short_rows(w)) return hipErrorNotSupported;
    const bool fused = x != nullptr;
    switch (w.type) {
        case 12: return fused ? launch_kq_argmax<12, true>(w, x, q8k, y, parts, max_parts, nparts, s)
                              : launch_kq_argmax<12, false>(w, x, q8k, y, parts, max_parts, nparts, s);
        case 13: return fused ? launch_kq_argmax<13, true>(w, x, q8k, y, parts, max_parts, nparts, s)
                              : launch_kq_argmax<13, false>(w, x, q8k, y, parts, max_parts, nparts, s);
        case 14: return fused ? launch_kq_argmax<14, true>(w, x, q8k, y, parts, max_parts, nparts, s)
                              : launch_kq_argmax<14, false>(w, x, q8k, y, parts, max_parts, nparts, s);
        default: return hipErrorNotSupported;
    }
}

hipError_t launch_gemv_kquant_set(const DeviceMatrix* mats, uint32_t nmat, int m, const uint8_t* q8k, float* const* ys,
                                  hipStream_t s, const float* const* adds, const MtConv* conv) {
    if (nmat < 1 || nmat > 4 || m < 2 || m > 15) return hipErrorNotSupported;
    if (conv != nullptr && (nmat != 4 || conv->kernel < 1 || conv->kernel > kMtConvTaps ||
                            mats[2].n != mats[3].n)) {
        return hipErrorNotSupported;
    }
    const DeviceMatrix& w = mats[0];
    if (!gemv_kquant_supported(w) || !short_rows(w)) return hipErrorNotSupported;
    uint64_t rows = 0;
    for (uint32_t i = 0; i < nmat; ++i) {
        if (mats[i].type != w.type || mats[i].k != w.k || mats[i].pitch != w.pitch) return hipErrorNotSupported;
        rows += mats[i].n;
    }
    if (rows > 0xFFFFFFFFull) return hipErrorNotSupported;
    const uint64_t nsb = w.k / kQK;
    // activation rows per launch, as launch_gemv_kquant: what fits the LDS budget, at most 8
    int chunk = 8;
    while (chunk > 1 && kq::act_lds_bytes(w.k, chunk) > kq::mt_lds_budget(w.type)) chunk >>= 1;
    for (int m0 = 0; m0 < m; m0 += chunk) {
        const int mc = m - m0 < chunk ? m - m0 : chunk;
        MtSet set{};
        set.nmat = nmat;
        uint32_t end = 0;
        for (uint32_t i = 0; i < nmat; ++i) {
            set.base[i] = mats[i].base;
            set.y[i] = ys[i] + (uint64_t)m0 * mats[i].n;
            set.add[i] = adds != nullptr && adds[i] != nullptr ? adds[i] + (uint64_t)m0 * mats[i].n : nullptr;
            end += (uint32_t)mats[i].n;
            set.row_end[i] = end;
        }
        if (conv != nullptr) {
            set.conv = *conv;
            set.conv.conv_out = conv->conv_out + (uint64_t)m0 * mats[0].n;
            set.conv.beta_s = conv->beta_s + (uint64_t)m0 * mats[2].n;
            set.conv.log_decay = conv->log_decay + (uint64_t)m0 * mats[3].n;
        }
        const uint8_t* q = q8k + (uint64_t)m0 * nsb * kQ8KBytes;
        hipError_t e;
        switch (w.type) {
            case 12: e = kq::launch_set_m<12>(w, mc, q, set, s); break;
            case 13: e = kq::launch_set_m<13>(w, mc, q, set, s); break;
            case 14: e = kq::launch_set_m<14>(w, mc, q, set, s); break;
            default: e = hipErrorNotSupported;
        }
        // the first chunk refused: nothing launched, the caller multiplies the matrices one by one;
        // a later chunk the set kernel does not cover (one row left) runs matrix by matrix here
        if (e == hipErrorNotSupported && m0 > 0) {
            for (uint32_t i = 0; i < nmat; ++i) {
                float* yi = ys[i] + (uint64_t)m0 * mats[i].n;
                e = launch_gemv_kquant(mats[i], mc, nullptr, q, yi, s);
                if (e == hipSuccess && set.add[i] != nullptr) e = launch_add(set.add[i], yi, (uint64_t)mc * mats[i].n, yi, s);
                if (e != hipSuccess) return e;
            }
            if (conv != nullptr) {
                // this chunk's tokens through the separate epilogue launch, in token order after the
                // earlier chunks'
                e = launch_conv_gates_tokens(ys[0] + (uint64_t)m0 * mats[0].n, conv->conv_w, conv->history, mats[0].n,
                                             conv->kernel, ys[2] + (uint64_t)m0 * mats[2].n,
                                             ys[3] + (uint64_t)m0 * mats[3].n, conv->dt_bias, conv->decay, mats[2].n,
                                             (uint64_t)mc, set.conv.conv_out, set.conv.beta_s, set.conv.log_decay, s);
                if (e != hipSuccess) return e;
            }
            continue;
        }
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

hipError_t launch_gemv_kquant_set_norm(const DeviceMatrix* mats, uint32_t nmat, int m, const float* x, const MtNorm& norm,
                                       float* const* ys, hipStream_t s, const MtConv* conv) {
    if (nmat < 1 || nmat > 4 || m != 2 || norm.w == nullptr) return hipErrorNotSupported;
    if (conv != nullptr && (nmat != 4 || conv->kernel < 1 || conv->kernel > kMtConvTaps || mats[2].n != mats[3].n)) {
        return hipErrorNotSupported;
    }
    const DeviceMatrix& w = mats[0];
    if (!gemv_kquant_supported(w) || !short_rows(w)) return hipErrorNotSupported;
    uint64_t rows = 0;
    MtSet set{};
    set.nmat = nmat;
    for (uint32_t i = 0; i < nmat; ++i) {
        if (mats[i].type != w.type || mats[i].k != w.k || mats[i].pitch != w.pitch) return hipErrorNotSupported;
        rows += mats[i].n;
        set.base[i] = mats[i].base;
        set.y[i] = ys[i];
        set.row_end[i] = (uint32_t)rows;
    }
    if (rows > 0xFFFFFFFFull) return hipErrorNotSupported;
    if (conv != nullptr) set.conv = *conv;
    set.norm = norm;
    switch (w.type) {
        case 12: return kq::launch_set_norm_m<12>(w, m, x, set, s);
        case 13: return kq::launch_set_norm_m<13>(w, m, x, set, s);
        case 14: return kq::launch_set_norm_m<14>(w, m, x, set, s);
        default: return hipErrorNotSupported;
    }
}

hipError_t launch_gemv_kquant(const DeviceMatrix& w, int m, const float* x, const uint8_t* q8k, float* y,
                              hipStream_t s) {
    if (!gemv_kquant_supported(w)) return hipErrorNotSupported;
    const uint64_t nsb = w.k / kQK;
    if (short_rows(w)) {
        // activation rows per launch: what fits the LDS budget, at most 8
        int chunk = 8;
        while (chunk > 1 && kq::act_lds_bytes(w.k, chunk) > kq::mt_lds_budget(w.type)) chunk >>= 1;
        for (int m0 = 0; m0 < m; m0 += chunk) {
            const int mc = m - m0 < chunk ? m - m0 : chunk;
            hipError_t e;
            if (x != nullptr) {
                e = launch_type<true>(w, mc, x + (uint64_t)m0 * w.k, nullptr, y + (uint64_t)m0 * w.n, s);
            } else {
                e = launch_type<false>(w, mc, nullptr, q8k + (uint64_t)m0 * nsb * kQ8KBytes, y + (uint64_t)m0 * w.n,
                                       s);
            }
            if (e != hipSuccess) return e;
        }
        return hipSuccess;
    }
    const uint32_t passes = (uint32_t)((nsb + 15) / 16);
    const uint32_t win = gemv_window_passes(w, m);
    const int chunk = 2;
    for (int m0 = 0; m0 < m; m0 += chunk) {
        const int mc = m - m0 < chunk ? m - m0 : chunk;
        for (uint32_t p0 = 0; p0 < passes; p0 += win) {
            const uint32_t np = passes - p0 < win ? passes - p0 : win;
            hipError_t e;
            if (x != nullptr) {
                e = launch_type_window<true>(w, mc, x + (uint64_t)m0 * w.k, nullptr, y + (uint64_t)m0 * w.n, p0, np,
                                             p0 > 0, s);
            } else {
                e = launch_type_window<false>(w, mc, nullptr, q8k + (uint64_t)m0 * nsb * kQ8KBytes,
                                              y + (uint64_t)m0 * w.n, p0, np, p0 > 0, s);
            }
            if (e != hipSuccess) return e;
        }
    }
    return hipSuccess;
}

}  // namespace oq
