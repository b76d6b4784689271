// Decode GEMV / small-batch kernels (gfx950, wave64).
//
// y[m][n] = sum_k W[n][k] * x[m][k] for a handful of activation rows m, weights streamed from
// HBM exactly once.  The same (GGML) arithmetic as vec_dot_qX_K_q8_K: integer dot products of
// the weight quants with Q8_K activation quants per 16/32-element group, then the block scales
// in F32.  Reference semantics: reference_storage_matvec (src/backend/cpu/quantized_reference.cpp
// :128-162), one output per weight row.
//
// Work split (K-quants): one wave owns a weight row; within the row, lane l handles super-block
// (l/4) + 16*i and its 64-element group g = l%4, i.e. 32 bytes of 4-bit quants (two 128-bit
// loads) plus the 16-byte block header.  A wave therefore streams 16 contiguous super-blocks per
// pass.  The activation rows sit in LDS as Q8_K: int8 quants [m][K], F32 block scales [m][K/256],
// int16 16-element sums [m][K/16].  Each workgroup (4 waves) either copies them from Q8_K blocks
// in global memory or quantizes F32 activations itself (bit-identical to quantize_q8k_kernel).
// Row sums are reduced across the wave with cross-lane shuffles; no atomics, deterministic.
#include "oq_common.h"

namespace oq {

namespace {

constexpr int kWaves = 4;  // waves per workgroup
constexpr int kThreads = 64 * kWaves;
constexpr uint64_t kLdsBudget = 64 * 1024;

OQ_DEVICE uint4 ldg128(const uint8_t* p) { return *reinterpret_cast<const uint4*>(p); }
OQ_DEVICE uint4 lds128(const int8_t* p) { return *reinterpret_cast<const uint4*>(p); }

OQ_DEVICE int dot4(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

// LDS image of MT activation rows in Q8_K form
struct Q8Lds {
    int8_t* q;       // [MT][K]
    float* d;        // [MT][K/256]
    int16_t* bsum;   // [MT][K/16]
};

OQ_DEVICE Q8Lds carve_lds(uint8_t* smem, int mt, uint64_t k) {
    Q8Lds s;
    s.q = reinterpret_cast<int8_t*>(smem);
    s.d = reinterpret_cast<float*>(smem + mt * k);
    s.bsum = reinterpret_cast<int16_t*>(smem + mt * k + mt * (k / kQK) * 4);
    return s;
}

// Stage m activation rows into LDS: quantize F32 `x` (fused) or copy Q8_K blocks `q8k`.
template <bool FUSED>
OQ_DEVICE void stage_q8k(const Q8Lds& s, int m, uint64_t k, const float* x, const uint8_t* q8k) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint64_t nsb = k / kQK;
    const uint64_t nblk = (uint64_t)m * nsb;
    for (uint64_t b = wave; b < nblk; b += kWaves) {
        const uint64_t mi = b / nsb, sb = b % nsb;
        uint32_t qword;
        int bsum16 = 0;
        float d = 0.0f;
        if constexpr (FUSED) {
            const float4 v = reinterpret_cast<const float4*>(x + mi * k + sb * kQK)[lane];
            const Q8KLane r = quantize_q8k_block_wave(v, lane);
            qword = r.qword;
            bsum16 = r.quad_bsum;
            d = r.d;
        } else {
            const uint8_t* blk = q8k + b * kQ8KBytes;
            qword = *reinterpret_cast<const uint32_t*>(blk + 4 + 4 * lane);
            if ((lane & 3) == 0) bsum16 = *reinterpret_cast<const int16_t*>(blk + 260 + 2 * (lane >> 2));
            d = *reinterpret_cast<const float*>(blk);
        }
        *reinterpret_cast<uint32_t*>(s.q + mi * k + sb * kQK + 4 * lane) = qword;
        if ((lane & 3) == 0) s.bsum[mi * (k / 16) + sb * 16 + (lane >> 2)] = (int16_t)bsum16;
        if (lane == 0) s.d[mi * nsb + sb] = d;
    }
}

// ---------------------------------------------------------------- per-lane block math

// q4_K / q5_K: lane group g of one super-block.  qs holds the group's 32 quant bytes (low
// nibbles = sub-block 2g, high nibbles = sub-block 2g+1); hbits (q5_K only) holds the
// fifth bits already moved to bit 4 of each byte for both sub-blocks.
template <int MT, bool Q5>
OQ_DEVICE void kq45_lane(const uint4 hdr, const uint32_t (&qs)[8], const uint32_t (&hb_lo)[8],
                         const uint32_t (&hb_hi)[8], int g, uint64_t sb, uint64_t k, int m,
                         const Q8Lds& s, float (&acc)[MT]) {
    const float d = f16_bits_to_f32(hdr.x & 0xFFFFu);
    const float dmin = f16_bits_to_f32(hdr.x >> 16);
    uint32_t sc0, mn0, sc1, mn1;
    scale_min_k4(2 * g, hdr.y, hdr.z, hdr.w, sc0, mn0);
    scale_min_k4(2 * g + 1, hdr.y, hdr.z, hdr.w, sc1, mn1);
    uint32_t lo[8], hi[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        lo[i] = qs[i] & 0x0F0F0F0Fu;
        hi[i] = (qs[i] >> 4) & 0x0F0F0F0Fu;
        if constexpr (Q5) {
            lo[i] |= hb_lo[i];
            hi[i] |= hb_hi[i];
        }
    }
    const uint64_t nsb = k / kQK;
#pragma unroll
    for (int mi = 0; mi < MT; ++mi) {
        if (mi < m) {
            const int8_t* q8 = s.q + mi * k + sb * kQK + 64 * g;
            const uint4 x0 = lds128(q8), x1 = lds128(q8 + 16), x2 = lds128(q8 + 32),
                        x3 = lds128(q8 + 48);
            int slo = 0, shi = 0;
            slo = dot4(lo[0], x0.x, slo); slo = dot4(lo[1], x0.y, slo);
            slo = dot4(lo[2], x0.z, slo); slo = dot4(lo[3], x0.w, slo);
            slo = dot4(lo[4], x1.x, slo); slo = dot4(lo[5], x1.y, slo);
            slo = dot4(lo[6], x1.z, slo); slo = dot4(lo[7], x1.w, slo);
            shi = dot4(hi[0], x2.x, shi); shi = dot4(hi[1], x2.y, shi);
            shi = dot4(hi[2], x2.z, shi); shi = dot4(hi[3], x2.w, shi);
            shi = dot4(hi[4], x3.x, shi); shi = dot4(hi[5], x3.y, shi);
            shi = dot4(hi[6], x3.z, shi); shi = dot4(hi[7], x3.w, shi);
            const int16_t* bs = s.bsum + mi * (k / 16) + sb * 16 + 4 * g;
            const int b0 = bs[0] + bs[1], b1 = bs[2] + bs[3];
            const int isum = (int)sc0 * slo + (int)sc1 * shi;
            const int imin = (int)mn0 * b0 + (int)mn1 * b1;
            const float dx = s.d[mi * nsb + sb];
            acc[mi] += dx * (d * (float)isum - dmin * (float)imin);
        }
    }
}

// q6_K (plane layout): lane group g -> half h = g/2, segments s0 = g%2 and s0+2; 32 ql bytes
// [32g, 32g+32), 32 qh bytes [32h, 32h+32), scales sc[8h + 2*s0 + {0,1,4,5}].
template <int MT>
OQ_DEVICE void kq6_lane(const uint32_t (&ql)[8], const uint32_t (&qh)[8], uint64_t sc8, float d,
                        int g, uint64_t sb, uint64_t k, int m, const Q8Lds& s,
                        float (&acc)[MT]) {
    const int h = g >> 1, s0 = g & 1;
    const int sh0 = 2 * s0, sh1 = 2 * s0 + 4;
    uint32_t qa[8], qb[8];  // 6-bit unsigned quants for segment s0 and s0+2
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        qa[i] = (ql[i] & 0x0F0F0F0Fu) | (((qh[i] >> sh0) & 0x03030303u) << 4);
        qb[i] = ((ql[i] >> 4) & 0x0F0F0F0Fu) | (((qh[i] >> sh1) & 0x03030303u) << 4);
    }
    const int c0 = (int)(int8_t)(sc8 >> (8 * (2 * s0)));
    const int c1 = (int)(int8_t)(sc8 >> (8 * (2 * s0 + 1)));
    const int c2 = (int)(int8_t)(sc8 >> (8 * (2 * s0 + 4)));
    const int c3 = (int)(int8_t)(sc8 >> (8 * (2 * s0 + 5)));
    const uint64_t nsb = k / kQK;
    const int e0 = 128 * h + 32 * s0;
#pragma unroll
    for (int mi = 0; mi < MT; ++mi) {
        if (mi < m) {
            const int8_t* q8 = s.q + mi * k + sb * kQK + e0;
            const uint4 x0 = lds128(q8), x1 = lds128(q8 + 16), x2 = lds128(q8 + 64),
                        x3 = lds128(q8 + 80);
            int p0 = 0, p1 = 0, p2 = 0, p3 = 0;
            p0 = dot4(qa[0], x0.x, p0); p0 = dot4(qa[1], x0.y, p0);
            p0 = dot4(qa[2], x0.z, p0); p0 = dot4(qa[3], x0.w, p0);
            p1 = dot4(qa[4], x1.x, p1); p1 = dot4(qa[5], x1.y, p1);
            p1 = dot4(qa[6], x1.z, p1); p1 = dot4(qa[7], x1.w, p1);
            p2 = dot4(qb[0], x2.x, p2); p2 = dot4(qb[1], x2.y, p2);
            p2 = dot4(qb[2], x2.z, p2); p2 = dot4(qb[3], x2.w, p2);
            p3 = dot4(qb[4], x3.x, p3); p3 = dot4(qb[5], x3.y, p3);
            p3 = dot4(qb[6], x3.z, p3); p3 = dot4(qb[7], x3.w, p3);
            const int16_t* bs = s.bsum + mi * (k / 16) + sb * 16 + e0 / 16;
            const int isum = c0 * (p0 - 32 * bs[0]) + c1 * (p1 - 32 * bs[1]) +
                             c2 * (p2 - 32 * bs[4]) + c3 * (p3 - 32 * bs[5]);
            acc[mi] += s.d[mi * nsb + sb] * (d * (float)isum);
        }
    }
}

// ---------------------------------------------------------------- K-quant GEMV kernel

template <uint32_t TYPE, int MT, int ROWS, bool FUSED>
__global__ __launch_bounds__(kThreads) void gemv_kquant_kernel(DeviceMatrix w, int m,
                                                               const float* __restrict__ x,
                                                               const uint8_t* __restrict__ q8k,
                                                               float* __restrict__ y) {
    extern __shared__ __align__(16) uint8_t smem[];
    const uint64_t k = w.k, n = w.n, nsb = k / kQK;
    const Q8Lds s = carve_lds(smem, MT, k);
    stage_q8k<FUSED>(s, m, k, x, q8k);
    __syncthreads();

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int sbi = lane >> 2, g = lane & 3;
    const uint64_t groups = (n + ROWS - 1) / ROWS;
    for (uint64_t grp = (uint64_t)blockIdx.x * kWaves + wave; grp < groups;
         grp += (uint64_t)gridDim.x * kWaves) {
        float acc[ROWS][MT];
#pragma unroll
        for (int r = 0; r < ROWS; ++r)
#pragma unroll
            for (int mi = 0; mi < MT; ++mi) acc[r][mi] = 0.0f;

        for (uint64_t sb = sbi; sb < nsb; sb += 16) {
            if constexpr (TYPE == 14) {
                uint32_t ql[ROWS][8], qh[ROWS][8];
                uint64_t sc8[ROWS];
                float dd[ROWS];
#pragma unroll
                for (int r = 0; r < ROWS; ++r) {
                    const uint64_t row = grp * ROWS + r < n ? grp * ROWS + r : n - 1;
                    const uint8_t* base = w.base + row * w.pitch;
                    const uint4 a = ldg128(base + sb * 128 + 32 * g);
                    const uint4 b = ldg128(base + sb * 128 + 32 * g + 16);
                    const uint4 c = ldg128(base + 128 * nsb + sb * 64 + 32 * (g >> 1));
                    const uint4 e = ldg128(base + 128 * nsb + sb * 64 + 32 * (g >> 1) + 16);
                    ql[r][0] = a.x; ql[r][1] = a.y; ql[r][2] = a.z; ql[r][3] = a.w;
                    ql[r][4] = b.x; ql[r][5] = b.y; ql[r][6] = b.z; ql[r][7] = b.w;
                    qh[r][0] = c.x; qh[r][1] = c.y; qh[r][2] = c.z; qh[r][3] = c.w;
                    qh[r][4] = e.x; qh[r][5] = e.y; qh[r][6] = e.z; qh[r][7] = e.w;
                    sc8[r] = *reinterpret_cast<const uint64_t*>(base + 192 * nsb + sb * 16 + 8 * (g >> 1));
                    dd[r] = f16_bits_to_f32(*reinterpret_cast<const uint16_t*>(base + 208 * nsb + sb * 2));
                }
#pragma unroll
                for (int r = 0; r < ROWS; ++r) kq6_lane<MT>(ql[r], qh[r], sc8[r], dd[r], g, sb, k, m, s, acc[r]);
            } else {
                constexpr bool Q5 = TYPE == 13;
                constexpr int BB = Q5 ? kQ5KBytes : kQ4KBytes;
                constexpr int QOFF = Q5 ? 48 : 16;
                uint4 hdr[ROWS];
                uint32_t qs[ROWS][8];
                uint32_t hl[ROWS][8], hh[ROWS][8];
#pragma unroll
                for (int r = 0; r < ROWS; ++r) {
                    const uint64_t row = grp * ROWS + r < n ? grp * ROWS + r : n - 1;
                    const uint8_t* blk = w.base + row * w.pitch + sb * BB;
                    hdr[r] = ldg128(blk);
                    const uint4 a = ldg128(blk + QOFF + 32 * g);
                    const uint4 b = ldg128(blk + QOFF + 32 * g + 16);
                    qs[r][0] = a.x; qs[r][1] = a.y; qs[r][2] = a.z; qs[r][3] = a.w;
                    qs[r][4] = b.x; qs[r][5] = b.y; qs[r][6] = b.z; qs[r][7] = b.w;
                    if constexpr (Q5) {
                        // fifth bits: qh[l] bit (2g) -> low-nibble quant, bit (2g+1) -> high
                        const uint4 c = ldg128(blk + 16);
                        const uint4 e = ldg128(blk + 32);
                        const uint32_t hw[8] = {c.x, c.y, c.z, c.w, e.x, e.y, e.z, e.w};
#pragma unroll
                        for (int i = 0; i < 8; ++i) {
                            hl[r][i] = ((hw[i] >> (2 * g)) & 0x01010101u) << 4;
                            hh[r][i] = ((hw[i] >> (2 * g + 1)) & 0x01010101u) << 4;
                        }
                    }
                }
#pragma unroll
                for (int r = 0; r < ROWS; ++r)
                    kq45_lane<MT, Q5>(hdr[r], qs[r], hl[r], hh[r], g, sb, k, m, s, acc[r]);
            }
        }
#pragma unroll
        for (int r = 0; r < ROWS; ++r) {
#pragma unroll
            for (int mi = 0; mi < MT; ++mi) {
                const float v = wave_sum(acc[r][mi]);
                const uint64_t row = grp * ROWS + r;
                if (lane == 0 && mi < m && row < n) y[(uint64_t)mi * n + row] = v;
            }
        }
    }
}

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

int env_int(const char* name, int fallback) {
    const char* v = getenv(name);
    return v ? atoi(v) : fallback;
}

uint64_t q8_lds_bytes(int mt, uint64_t k) { return (uint64_t)mt * (k + k / kQK * 4 + k / 16 * 2); }

unsigned grid_for(uint64_t work_items, int per_wg_items) {
    const uint64_t want = (work_items + per_wg_items - 1) / per_wg_items;
    const uint64_t cap = (uint64_t)env_int("OQ_GEMV_MAX_WG", 1 << 20);
    return (unsigned)(want < cap ? (want ? want : 1) : cap);
}

template <uint32_t TYPE, int MT, bool FUSED>
hipError_t launch_kq_mt(const DeviceMatrix& w, int m, const float* x, const uint8_t* q8k, float* y,
                        hipStream_t s) {
    const int rows = env_int("OQ_GEMV_ROWS", 1);
    const size_t lds = q8_lds_bytes(MT, w.k);
    if (rows >= 2) {
        const unsigned grid = grid_for((w.n + 1) / 2, kWaves);
        hipLaunchKernelGGL((gemv_kquant_kernel<TYPE, MT, 2, FUSED>), dim3(grid), dim3(kThreads), lds,
                           s, w, m, x, q8k, y);
    } else {
        const unsigned grid = grid_for(w.n, kWaves);
        hipLaunchKernelGGL((gemv_kquant_kernel<TYPE, MT, 1, FUSED>), dim3(grid), dim3(kThreads), lds,
                           s, w, m, x, q8k, y);
    }
    return hipGetLastError();
}

template <uint32_t TYPE, bool FUSED>
hipError_t launch_kq_type(const DeviceMatrix& w, int m, const float* x, const uint8_t* q8k, float* y,
                          hipStream_t s) {
    if (m <= 1) return launch_kq_mt<TYPE, 1, FUSED>(w, m, x, q8k, y, s);
    if (m <= 2) return launch_kq_mt<TYPE, 2, FUSED>(w, m, x, q8k, y, s);
    if (m <= 4) return launch_kq_mt<TYPE, 4, FUSED>(w, m, x, q8k, y, s);
    return launch_kq_mt<TYPE, 8, FUSED>(w, m, x, q8k, y, s);
}

template <bool FUSED>
hipError_t launch_kq_fused(const DeviceMatrix& w, int m, const float* x, const uint8_t* q8k,
                           float* y, hipStream_t s) {
    switch (w.type) {
        case 12: return launch_kq_type<12, FUSED>(w, m, x, q8k, y, s);
        case 13: return launch_kq_type<13, FUSED>(w, m, x, q8k, y, s);
        case 14: return launch_kq_type<14, FUSED>(w, m, x, q8k, y, s);
        default: return hipErrorInvalidValue;
    }
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

int gemv_max_m() { return 8; }

hipError_t launch_gemv_kquant(const DeviceMatrix& w, int m, const float* x, const uint8_t* q8k,
                              float* y, hipStream_t s) {
    // split the activation rows so each launch's LDS image fits the budget
    int chunk = 8;
    while (chunk > 1 && q8_lds_bytes(chunk, w.k) > kLdsBudget) chunk >>= 1;
    if (q8_lds_bytes(1, w.k) > kLdsBudget) return hipErrorInvalidValue;
    for (int m0 = 0; m0 < m; m0 += chunk) {
        const int mc = m - m0 < chunk ? m - m0 : chunk;
        hipError_t e;
        if (x != nullptr) {
            e = launch_kq_fused<true>(w, mc, x + (uint64_t)m0 * w.k, nullptr, y + (uint64_t)m0 * w.n, s);
        } else {
            e = launch_kq_fused<false>(w, mc, nullptr, q8k + (uint64_t)m0 * (w.k / kQK) * kQ8KBytes,
                                       y + (uint64_t)m0 * w.n, s);
        }
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

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
