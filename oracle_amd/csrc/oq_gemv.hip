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

// q8_0 weight chunks: read once per launch (non-temporal, see load_stream)
OQ_DEVICE uint4 ldg128(const uint8_t* p) { return load_stream(reinterpret_cast<const uint4*>(p)); }


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

// Decode GEMV for q8_0 (one activation row; K = 1024, 2048 or 4096, ITERS = K / 1024).
// Wave i of workgroup b owns rows b * kRowWaves + i + j * (waves in the grid).  A lane takes the
// 16-byte quant chunks lane + 64 j (every load instruction of the wave reads 1 KiB of consecutive
// bytes) and their f16 scales.  Each workgroup copies x into LDS once: the x loads are issued
// first, then the first row's weight loads, so the copy waits only for x while the weights stream.
// In LDS the four 16-byte pieces of each 64-byte x chunk are rotated by the chunk index, so the
// lanes of one ds_read_b128 read distinct banks.  Arithmetic per chunk as gemv_q8_0_kernel.
constexpr int kRowWaves = 16;

template <int ITERS>
OQ_DEVICE void load_q8_0_row(uint4 (&q)[ITERS], uint32_t (&d)[ITERS], const DeviceMatrix& w, uint32_t row, int lane) {
    const uint32_t n = (uint32_t)w.n;
    row = row < n ? row : n - 1;
    const uint8_t* base = w.base + (uint64_t)__builtin_amdgcn_readfirstlane(row) * w.pitch;
#pragma unroll
    for (int j = 0; j < ITERS; ++j) {
        const uint32_t c = (uint32_t)lane + 64u * j;
        q[j] = ldg128(base + 16u * c);
        d[j] = *reinterpret_cast<const uint16_t*>(base + (uint32_t)w.k + 2u * (c >> 1));
    }
}

template <int ITERS>
__global__ __launch_bounds__(64 * kRowWaves) void gemv_q8_0_rows_kernel(DeviceMatrix w, const float* x,
                                                                        float* __restrict__ y) {
    extern __shared__ __align__(16) uint8_t smem[];
    float4* xs = reinterpret_cast<float4*>(smem);
    constexpr int XPT = (ITERS + 3) / 4;  // float4 of x per thread
    const int lane = threadIdx.x & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t n = (uint32_t)w.n, k4 = (uint32_t)(w.k / 4);
    const uint32_t nw = gridDim.x * kRowWaves;
    uint32_t row = blockIdx.x * kRowWaves + wave;

    float4 xv[XPT];
#pragma unroll
    for (int t = 0; t < XPT; ++t) {
        uint32_t f = threadIdx.x + 64u * kRowWaves * t;
        f = f < k4 ? f : k4 - 1;
        xv[t] = reinterpret_cast<const float4*>(x)[f];
    }
    asm volatile("" ::: "memory");  // x is not __restrict__: its loads stay ahead of the weights'
    uint4 q[ITERS];
    uint32_t d[ITERS];
    load_q8_0_row<ITERS>(q, d, w, row, lane);
#pragma unroll
    for (int t = 0; t < XPT; ++t) {
        const uint32_t f = threadIdx.x + 64u * kRowWaves * t;
        const uint32_t c = f >> 2, i = f & 3;
        if (f < k4) xs[4u * c + ((i + c) & 3u)] = xv[t];
    }
    __syncthreads();
    while (row < n) {
        float acc = 0.0f;
#pragma unroll
        for (int j = 0; j < ITERS; ++j) {
            const uint32_t c = (uint32_t)lane + 64u * j;
            const float scale = f16_bits_to_f32((uint16_t)d[j]);
            const uint32_t words[4] = {q[j].x, q[j].y, q[j].z, q[j].w};
            float part = 0.0f;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float4 xp = xs[4u * c + ((i + c) & 3u)];
                const uint32_t wd = words[i];
                part += (float)(int8_t)(wd) * xp.x;
                part += (float)(int8_t)(wd >> 8) * xp.y;
                part += (float)(int8_t)(wd >> 16) * xp.z;
                part += (float)(int8_t)(wd >> 24) * xp.w;
            }
            acc += scale * part;
        }
        const float v = wave_sum_uniform(acc);
        if (lane == 0) y[row] = v;
        row += nw;
        if (row < n) load_q8_0_row<ITERS>(q, d, w, row, lane);
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
    const uint64_t cap = (uint64_t)knob(kGemvMaxWg, 1 << 20);
    return (unsigned)(want < cap ? (want ? want : 1) : cap);
}

template <int ITERS>
hipError_t launch_q8_0_rows(const DeviceMatrix& w, const float* x, float* y, hipStream_t s) {
    uint64_t wgs = (w.n + kRowWaves - 1) / kRowWaves;
    const uint64_t cap = (uint64_t)cu_count() * (ITERS <= 2 ? 2u : 1u);  // workgroups resident per CU
    if (wgs > cap) wgs = cap;
    hipLaunchKernelGGL((gemv_q8_0_rows_kernel<ITERS>), dim3((unsigned)wgs), dim3(64 * kRowWaves), w.k * 4, s, w, x, y);
    return hipGetLastError();
}

template <int MT>
hipError_t launch_q8_0_mt(const DeviceMatrix& w, int m, const float* x, float* y, hipStream_t s) {
    if (MT == 1 && w.k % 1024 == 0 && knob(kQ80Rows, 1) != 0) {
        switch (w.k / 1024) {
            case 1: return launch_q8_0_rows<1>(w, x, y, s);
            case 2: return launch_q8_0_rows<2>(w, x, y, s);
            case 4: return launch_q8_0_rows<4>(w, x, y, s);
            default: break;  // longer rows would not fit the registers of 16-wave workgroups
        }
    }
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
