// Prefill / verify GEMM for q4_K weights on gfx950 int8 matrix cores (m >= 16 activation rows),
// the alternative to the f16 kernel of oq_gemm.hip (selected with OQ_GEMM_INT8=1).
//
// Y[m][n] = sum over super-blocks sb of dx[m][sb] * (d[n][sb] * I[m][n][sb] - dmin[n][sb] * M[m][n][sb])
//   I = sum_j sc[n][j] * sum_{k in sub-block j} q8[m][k] * q4[n][k]     (exact int32)
//   M = sum_j mn[n][j] * (bsum[m][2j] + bsum[m][2j+1])                  (exact, via f16 MFMA)
// -- GGML's vec_dot_q4_K_q8_K per activation row (the reference's multi-token evaluation is one
// matvec per row, src/runtime/qwen35_target_multi.cpp:14-25), with the K-quant dot semantics of
// src/backend/cpu/quantized_reference.cpp:67-81 up to F32 rounding.
//
// Each 32-element sub-block is one v_mfma_i32_32x32x32_i8 (Q8_K quants x nibbles widened to
// bytes); its 32 x 32 int32 result is scaled by the sub-block's 6-bit scale into an int32
// accumulator with one 24-bit multiply-add per value (the scale differs per output column and
// sub-block, so it cannot enter the MFMA).  The min term is one v_mfma_f32_32x32x16_f16 per
// super-block: the 16 partial sums of 16 quants (|b| <= 2032) times the mins, all exact in f16.
// At the end of a super-block the int32 and min sums are scaled in F32.  The per-sub-block
// rescale is vector work of one multiply-add per output per 32 k, which bounds this kernel.
//
// Layout: one workgroup of 4 waves per (128-row m-tile, 64-column n-tile); wave w owns rows
// m0 + 32 w .. + 31 and the tile's 64 columns (two 32 x 32 fragments).  No LDS: the activation
// image rows a wave reads are its own, the weight rows are shared by the 4 waves through L1.
// Every load of super-block i + 1 is issued before super-block i is multiplied.
#include "oq_common.h"
#include "oq_layout.h"

namespace oq {

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef _Float16 half8 __attribute__((ext_vector_type(8)));

constexpr int kI8BM = 128, kI8BN = 64;

// ---------------------------------------------------------------- activation image
//
// q[m][K] int8 (the Q8_K quants), d[sb][mp] F32 (block scales, rows contiguous per super-block,
// mp = m rounded up to 4 so that four consecutive rows are one aligned 16-byte load),
// b16[m][sb][16] f16 (the 16-element quant sums, exact in f16).
struct I8Image {
    int8_t* q;
    float* d;
    _Float16* b16;
    uint64_t mp;
};

__global__ __launch_bounds__(256) void quantize_i8_kernel(const float* __restrict__ x, uint64_t m, uint64_t nsb,
                                                          I8Image img) {
    const int lane = threadIdx.x & 63;
    const uint64_t blk = blockIdx.x * 4ull + (threadIdx.x >> 6);
    if (blk >= m * nsb) return;
    const uint64_t row = blk / nsb, sb = blk % nsb;
    const float4 v = reinterpret_cast<const float4*>(x + blk * kQK)[lane];
    const Q8KLane r = quantize_q8k_block_wave(v, lane);
    *reinterpret_cast<uint32_t*>(img.q + blk * kQK + 4 * lane) = r.qword;
    if (lane == 0) img.d[sb * img.mp + row] = r.d;
    if ((lane & 3) == 0) img.b16[blk * 16 + (lane >> 2)] = (_Float16)r.quad_bsum;
}

__global__ __launch_bounds__(256) void q8k_to_i8_kernel(const uint8_t* __restrict__ q8k, uint64_t m, uint64_t nsb,
                                                        I8Image img) {
    const int lane = threadIdx.x & 63;
    const uint64_t blk = blockIdx.x * 4ull + (threadIdx.x >> 6);
    if (blk >= m * nsb) return;
    const uint64_t row = blk / nsb, sb = blk % nsb;
    const uint8_t* b = q8k + blk * kQ8KBytes;
    *reinterpret_cast<uint32_t*>(img.q + blk * kQK + 4 * lane) = *reinterpret_cast<const uint32_t*>(b + 4 + 4 * lane);
    if (lane == 0) img.d[sb * img.mp + row] = *reinterpret_cast<const float*>(b);
    if (lane < 16) img.b16[blk * 16 + lane] = (_Float16)(float)*reinterpret_cast<const int16_t*>(b + 260 + 2 * lane);
}

// ---------------------------------------------------------------- GEMM

struct SbLoads {
    uint4 a[8];     // activation quants of the lane's row: sub-block j, k = 32 j + 16 h .. + 15
    uint4 bs;       // the row's 16-element sums 8 h .. 8 h + 7 (f16)
    float4 dx[4];   // activation scales of rows 8 t + 4 h + 0..3 of the wave's fragment
    uint4 wq[2][4]; // weight chunk (group g, half h) of fragment columns: nibbles of sub-blocks 2g, 2g+1
    uint4 hdr[2];   // weight header of the fragment columns (f16 d, f16 dmin, scales[12])
};

OQ_DEVICE void load_sb(SbLoads& L, const DeviceMatrix& w, const I8Image& img, uint64_t m, uint32_t sb, uint32_t nsb,
                       uint32_t row_a, const uint32_t (&wrow_off)[2], uint32_t m0w, int h) {
    const int8_t* qa = img.q + (uint64_t)row_a * w.k + (uint64_t)sb * kQK + 16 * h;
#pragma unroll
    for (int j = 0; j < 8; ++j) L.a[j] = *reinterpret_cast<const uint4*>(qa + 32 * j);
    L.bs = *reinterpret_cast<const uint4*>(img.b16 + ((uint64_t)row_a * nsb + sb) * 16 + 8 * h);
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        // rows 8 t + 4 h + 0..3 of the wave's 32 (clamped to m - 1 by the caller's tile layout)
        const uint64_t r = (uint64_t)m0w + 8 * t + 4 * h;
        const float* dp = img.d + (uint64_t)sb * img.mp;
        if (r + 3 < m) {
            L.dx[t] = *reinterpret_cast<const float4*>(dp + r);
        } else {
            L.dx[t].x = dp[r < m ? r : m - 1];
            L.dx[t].y = dp[r + 1 < m ? r + 1 : m - 1];
            L.dx[t].z = dp[r + 2 < m ? r + 2 : m - 1];
            L.dx[t].w = dp[r + 3 < m ? r + 3 : m - 1];
        }
    }
    const uint32_t pass = sb / 16u, s16 = sb % 16u;
    const uint32_t mp = nsb - 16u * pass < 16u ? nsb - 16u * pass : 16u;
#pragma unroll
    for (int f = 0; f < 2; ++f) {
        const uint8_t* row = w.base + wrow_off[f];
#pragma unroll
        for (int g = 0; g < 4; ++g)
            L.wq[f][g] = *reinterpret_cast<const uint4*>(row + 16u * (128u * pass + (uint32_t)h * 4u * mp + 4u * s16 + g));
        L.hdr[f] = *reinterpret_cast<const uint4*>(row + 128u * nsb + 16u * sb);
    }
}

template <bool FULL_M>
__global__ __launch_bounds__(256) void gemm_q4k_i8_kernel(DeviceMatrix w, int m_, I8Image img, uint32_t tiles_m,
                                                          float* __restrict__ y) {
    const uint64_t m = (uint64_t)m_;
    const int lane = threadIdx.x & 63, h = lane >> 5, l32 = lane & 31;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t mt = blockIdx.x % tiles_m, nt = blockIdx.x / tiles_m;
    const uint32_t nsb = (uint32_t)(w.k / kQK);
    const uint32_t m0w = mt * kI8BM + 32u * wave;            // first row of the wave's fragment
    const uint64_t row_l = m0w + l32;                          // the lane's A row
    const uint32_t row_a = (uint32_t)(row_l < m ? row_l : m - 1);
    uint32_t wrow_off[2];
#pragma unroll
    for (int f = 0; f < 2; ++f) {
        uint64_t n = (uint64_t)nt * kI8BN + 32u * f + l32;
        n = n < w.n ? n : w.n - 1;
        wrow_off[f] = (uint32_t)(n * w.pitch);
    }
    v16f out[2];
#pragma unroll
    for (int f = 0; f < 2; ++f)
#pragma unroll
        for (int r = 0; r < 16; ++r) out[f][r] = 0.0f;
    const v16i zero_i = {};
    const v16f zero_f = {};

    SbLoads cur, nxt;
    load_sb(cur, w, img, m, 0, nsb, row_a, wrow_off, m0w, h);
    for (uint32_t sb = 0; sb < nsb; ++sb) {
        load_sb(nxt, w, img, m, sb + 1 < nsb ? sb + 1 : sb, nsb, row_a, wrow_off, m0w, h);
#pragma unroll
        for (int f = 0; f < 2; ++f) {
            const uint4 hd = cur.hdr[f];
            // 6-bit scales and mins of the column's 8 sub-blocks (src/model/storage_decode.cpp:44-61)
            const uint32_t sc_lo = hd.y & 0x3F3F3F3Fu, mn_lo = hd.z & 0x3F3F3F3Fu;
            const uint32_t sc_hi = (hd.w & 0x0F0F0F0Fu) | ((hd.y >> 2) & 0x30303030u);
            const uint32_t mn_hi = ((hd.w >> 4) & 0x0F0F0F0Fu) | ((hd.z >> 2) & 0x30303030u);
            v16i acc = zero_i;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const uint4 q = cur.wq[f][j >> 1];
                const int sh = (j & 1) ? 4 : 0;
                const v4i b = {(int)((q.x >> sh) & 0x0F0F0F0Fu), (int)((q.y >> sh) & 0x0F0F0F0Fu),
                               (int)((q.z >> sh) & 0x0F0F0F0Fu), (int)((q.w >> sh) & 0x0F0F0F0Fu)};
                const v4i a = {(int)cur.a[j].x, (int)cur.a[j].y, (int)cur.a[j].z, (int)cur.a[j].w};
                const v16i p = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, zero_i, 0, 0, 0);
                const int sc = (int)(((j < 4 ? sc_lo : sc_hi) >> (8 * (j & 3))) & 0xFFu);
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[r] = __mul24(sc, p[r]) + acc[r];
            }
            // min term: sum_i b16[i] * mn[i / 2] over the 16 partial sums, one f16 MFMA
            half8 mb;
#pragma unroll
            for (int t = 0; t < 8; ++t) {
                const int jm = 4 * h + t / 2;  // sub-block of partial sum 8 h + t
                mb[t] = (_Float16)(float)(((jm < 4 ? mn_lo : mn_hi) >> (8 * (jm & 3))) & 0xFFu);
            }
            const half8 ab = __builtin_bit_cast(half8, cur.bs);
            const v16f mins = __builtin_amdgcn_mfma_f32_32x32x16_f16(ab, mb, zero_f, 0, 0, 0);
            const float d = (float)__builtin_bit_cast(_Float16, (uint16_t)(hd.x & 0xFFFFu));
            const float dmin = (float)__builtin_bit_cast(_Float16, (uint16_t)(hd.x >> 16));
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const float4 dx4 = cur.dx[r / 4];
                const float dx = (r & 3) == 0 ? dx4.x : ((r & 3) == 1 ? dx4.y : ((r & 3) == 2 ? dx4.z : dx4.w));
                out[f][r] += dx * (d * (float)acc[r] - dmin * mins[r]);
            }
        }
        cur = nxt;
    }
    // result register r of lane l: row 8 (r / 4) + 4 h + r % 4 of the fragment, column l % 32
#pragma unroll
    for (int f = 0; f < 2; ++f) {
        const uint64_t col = (uint64_t)nt * kI8BN + 32u * f + l32;
        if (col >= w.n) continue;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const uint64_t row = (uint64_t)m0w + 8 * (r / 4) + 4 * h + (r % 4);
            if (FULL_M || row < m) y[row * w.n + col] = out[f][r];
        }
    }
}

uint64_t round256(uint64_t v) { return (v + 255) & ~uint64_t(255); }

I8Image image_at(void* scratch, uint64_t m, uint64_t k) {
    uint8_t* base = static_cast<uint8_t*>(scratch);
    const uint64_t nsb = k / kQK;
    I8Image img;
    img.mp = (m + 3) & ~uint64_t(3);
    img.q = reinterpret_cast<int8_t*>(base);
    img.d = reinterpret_cast<float*>(base + round256(m * k));
    img.b16 = reinterpret_cast<_Float16*>(base + round256(m * k) + round256(nsb * img.mp * 4));
    return img;
}

}  // namespace

bool gemm_i8_supported(const DeviceMatrix& w, int m) { return w.type == 12 && m >= 16 && w.k % kQK == 0; }

uint64_t gemm_i8_scratch_bytes(const DeviceMatrix& w, int m) {
    const uint64_t nsb = w.k / kQK;
    const uint64_t mp = ((uint64_t)m + 3) & ~uint64_t(3);
    return round256((uint64_t)m * w.k) + round256(nsb * mp * 4) + round256((uint64_t)m * nsb * 32);
}

hipError_t launch_gemm_q4k_i8(const DeviceMatrix& w, int m, const float* x, const uint8_t* q8k, float* y, void* scratch,
                              hipStream_t s) {
    if (!gemm_i8_supported(w, m) || (x == nullptr) == (q8k == nullptr)) return hipErrorNotSupported;
    const uint64_t nsb = w.k / kQK;
    const I8Image img = image_at(scratch, (uint64_t)m, w.k);
    const unsigned qgrid = (unsigned)(((uint64_t)m * nsb + 3) / 4);
    if (x) hipLaunchKernelGGL(quantize_i8_kernel, dim3(qgrid), dim3(256), 0, s, x, (uint64_t)m, nsb, img);
    else hipLaunchKernelGGL(q8k_to_i8_kernel, dim3(qgrid), dim3(256), 0, s, q8k, (uint64_t)m, nsb, img);
    const uint32_t tiles_m = (uint32_t)((m + kI8BM - 1) / kI8BM);
    const uint32_t tiles_n = (uint32_t)((w.n + kI8BN - 1) / kI8BN);
    const dim3 grid(tiles_m * tiles_n);
    if (m % kI8BM == 0) hipLaunchKernelGGL(gemm_q4k_i8_kernel<true>, grid, dim3(256), 0, s, w, m, img, tiles_m, y);
    else hipLaunchKernelGGL(gemm_q4k_i8_kernel<false>, grid, dim3(256), 0, s, w, m, img, tiles_m, y);
    return hipGetLastError();
}

}  // namespace oq
