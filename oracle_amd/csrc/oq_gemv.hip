// Decode GEMV / small-batch kernels for weights multiplied against F32 activations (gfx950):
// q8_0 (the reference's Q8_0 path: decoded d*q times F32 x, src/backend/cpu/
// quantized_reference.cpp:50-64) and plain f32 / f16 / bf16 rows.  One wave owns a row, lanes
// stream its 16-byte chunks, and the row sum is reduced across the wave (no atomics).
#include "oq_common.h"

namespace oq {

namespace {

constexpr int kWaves = 4;  // waves per workgroup
constexpr int kThreads = 64 * kWaves;
constexpr uint64_t kLdsBudget = 64 * 1024;

OQ_DEVICE uint4 ldg128(const uint8_t* p) { return *reinterpret_cast<const uint4*>(p); }


// ---------------------------------------------------------------- F32-activation kernels

// q8_0 (plane layout qs[K] | d[K/32]) against F32 activations held in LDS [MT][K] (or read
// from global memory when they do not fit).  Lane l of the row's wave takes 16-byte chunks
// l, l+64, ... of the row's quants (half a block each): sum q*x in F32, then scale by d.
template <int MT, bool XLDS>
__global__ __launch_bounds__(kThreads) void gemv_q8_0_kernel(DeviceMatrix w, int m,
                                                             const float* __restrict__ x,
                                                             float* __restrict__ y) {
    extern __shared__ __align__(16) uint8_t smem[];
    float* xs = reinterpret_cast<float*>(smem);
    const uint64_t k = w.k, n = w.n;
    if constexpr (XLDS) {
        const uint64_t total4 = (uint64_t)m * k / 4;
        for (uint64_t i = threadIdx.x; i < total4; i += kThreads)
            reinterpret_cast<float4*>(xs)[i] = reinterpret_cast<const float4*>(x)[i];
        __syncthreads();
    }
    const float* xa = XLDS ? xs : x;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint64_t chunks = k / 16;
    for (uint64_t row = (uint64_t)blockIdx.x * kWaves + wave; row < n;
         row += (uint64_t)gridDim.x * kWaves) {
        const uint8_t* base = w.base + row * w.pitch;
        float acc[MT];
#pragma unroll
        for (int mi = 0; mi < MT; ++mi) acc[mi] = 0.0f;
        for (uint64_t c = lane; c < chunks; c += 64) {
            const uint4 raw = ldg128(base + 16 * c);
            const float scale = f16_bits_to_f32(*reinterpret_cast<const uint16_t*>(base + k + 2 * (c >> 1)));
            const uint32_t words[4] = {raw.x, raw.y, raw.z, raw.w};
            float wv[16];
#pragma unroll
            for (int i = 0; i < 16; ++i) wv[i] = (float)(int8_t)(words[i >> 2] >> (8 * (i & 3)));
#pragma unroll
            for (int mi = 0; mi < MT; ++mi) {
                if (mi < m) {
                    const float4* xp = reinterpret_cast<const float4*>(xa + mi * k + c * 16);
                    float part = 0.0f;
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const float4 xv = xp[q];
                        part += wv[4 * q] * xv.x;
                        part += wv[4 * q + 1] * xv.y;
                        part += wv[4 * q + 2] * xv.z;
                        part += wv[4 * q + 3] * xv.w;
                    }
                    acc[mi] += scale * part;
                }
            }
        }
#pragma unroll
        for (int mi = 0; mi < MT; ++mi) {
            const float v = wave_sum(acc[mi]);
            if (lane == 0 && mi < m) y[(uint64_t)mi * n + row] = v;
        }
    }
}

// f32 / f16 / bf16 rows of any length: one wave per row, lanes stride over elements.  These
// types carry norm and gate vectors in the reference (src/model/qwen35_weights.cpp:49-59), not
// the bandwidth-heavy projections.
template <uint32_t TYPE, int MT>
__global__ __launch_bounds__(kThreads) void gemv_plain_kernel(DeviceMatrix w, int m,
                                                              const float* __restrict__ x,
                                                              float* __restrict__ y) {
    const uint64_t k = w.k, n = w.n;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    for (uint64_t row = (uint64_t)blockIdx.x * kWaves + wave; row < n;
         row += (uint64_t)gridDim.x * kWaves) {
        const uint8_t* base = w.base + row * w.pitch;
        float acc[MT];
#pragma unroll
        for (int mi = 0; mi < MT; ++mi) acc[mi] = 0.0f;
        for (uint64_t i = lane; i < k; i += 64) {
            float wv;
            if constexpr (TYPE == 0) wv = reinterpret_cast<const float*>(base)[i];
            else if constexpr (TYPE == 1) wv = f16_bits_to_f32(reinterpret_cast<const uint16_t*>(base)[i]);
            else wv = bf16_bits_to_f32(reinterpret_cast<const uint16_t*>(base)[i]);
#pragma unroll
            for (int mi = 0; mi < MT; ++mi)
                if (mi < m) acc[mi] += wv * x[mi * k + i];
        }
#pragma unroll
        for (int mi = 0; mi < MT; ++mi) {
            const float v = wave_sum(acc[mi]);
            if (lane == 0 && mi < m) y[(uint64_t)mi * n + row] = v;
        }
    }
}

// ---------------------------------------------------------------- launch configuration

unsigned grid_for(uint64_t work_items, int per_wg_items) {
    const uint64_t want = (work_items + per_wg_items - 1) / per_wg_items;
    const uint64_t cap = (uint64_t)env_int("OQ_GEMV_MAX_WG", 1 << 20);
    return (unsigned)(want < cap ? (want ? want : 1) : cap);
}

template <int MT>
hipError_t launch_q8_0_mt(const DeviceMatrix& w, int m, const float* x, float* y, hipStream_t s) {
    const uint64_t lds = (uint64_t)MT * w.k * 4;
    const unsigned grid = grid_for(w.n, kWaves);
    if (lds <= kLdsBudget) {
        hipLaunchKernelGGL((gemv_q8_0_kernel<MT, true>), dim3(grid), dim3(kThreads), lds, s, w, m, x, y);
    } else {
        hipLaunchKernelGGL((gemv_q8_0_kernel<MT, false>), dim3(grid), dim3(kThreads), 0, s, w, m, x, y);
    }
    return hipGetLastError();
}

template <uint32_t TYPE, int MT>
hipError_t launch_plain_mt(const DeviceMatrix& w, int m, const float* x, float* y, hipStream_t s) {
    const unsigned grid = grid_for(w.n, kWaves);
    hipLaunchKernelGGL((gemv_plain_kernel<TYPE, MT>), dim3(grid), dim3(kThreads), 0, s, w, m, x, y);
    return hipGetLastError();
}

template <int MT>
hipError_t launch_f32_mt(const DeviceMatrix& w, int m, const float* x, float* y, hipStream_t s) {
    switch (w.type) {
        case 0: return launch_plain_mt<0, MT>(w, m, x, y, s);
        case 1: return launch_plain_mt<1, MT>(w, m, x, y, s);
        case 30: return launch_plain_mt<30, MT>(w, m, x, y, s);
        case 8: return launch_q8_0_mt<MT>(w, m, x, y, s);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace

hipError_t launch_gemv_f32act(const DeviceMatrix& w, int m, const float* x, float* y,
                              hipStream_t s) {
    for (int m0 = 0; m0 < m; m0 += 8) {
        const int mc = m - m0 < 8 ? m - m0 : 8;
        const float* xc = x + (uint64_t)m0 * w.k;
        float* yc = y + (uint64_t)m0 * w.n;
        hipError_t e;
        if (mc <= 1) e = launch_f32_mt<1>(w, mc, xc, yc, s);
        else if (mc <= 2) e = launch_f32_mt<2>(w, mc, xc, yc, s);
        else if (mc <= 4) e = launch_f32_mt<4>(w, mc, xc, yc, s);
        else e = launch_f32_mt<8>(w, mc, xc, yc, s);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

}  // namespace oq
