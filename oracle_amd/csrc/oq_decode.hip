// Upload relayout, bit-exact dequantization and F32 -> Q8_K activation quantization (gfx950).
//
// Dequantization follows the reference's block decoders value for value
// (src/model/storage_decode.cpp:63-139; q4_K is GGML's format on the same template): every
// F32 it writes has the bits the reference's scalar decoder produces, because the arithmetic
// is the same sequence of correctly rounded operations with contraction off.
#include "oq_common.h"
#include "oq_layout.h"

namespace oq {

uint64_t device_pitch(uint32_t type, uint64_t k) {
    auto up16 = [](uint64_t b) { return (b + 15u) & ~uint64_t(15); };
    switch (type) {
        case 0: return up16(k * 4);
        case 1:
        case 30: return up16(k * 2);
        case 8: return up16(k / 32 * kQ80Bytes);
        case 12: return k / kQK * kQ4KBytes;
        case 13: return k / kQK * kQ5KBytes;
        case 14: return up16(k / kQK * kQ6KBytes);
        default: return 0;
    }
}

// ------------------------------------------------------------------ relayout (upload)

// GGML rows (contiguous, row_bytes each) -> device rows at `pitch`.  Plain types keep their
// bytes; quantized blocks are split into per-row planes, so that every plane starts 16-byte
// aligned (210- and 34-byte blocks are not) and a wave streaming a row reads contiguous bytes.
__global__ void relayout_kernel(uint32_t type, uint64_t k, uint64_t n, const uint8_t* __restrict__ src,
                                uint8_t* __restrict__ dst, uint64_t row_bytes, uint64_t pitch) {
    const uint64_t total = n * row_bytes;
    for (uint64_t t = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; t < total;
         t += (uint64_t)gridDim.x * blockDim.x) {
        const uint64_t r = t / row_bytes, off = t % row_bytes;
        uint64_t o;
        if (type == 14) {
            const uint64_t nsb = k / kQK, sb = off / kQ6KBytes;
            const uint32_t b = (uint32_t)(off % kQ6KBytes);
            if (b < 128) o = q6_ql_offset(nsb, sb, b);
            else if (b < 192) o = 128 * nsb + sb * 64 + (b - 128);
            else if (b < 208) o = 192 * nsb + sb * 16 + q6_sc_offset(b - 192);
            else o = 208 * nsb + sb * 2 + (b - 208);
        } else if (type == 8) {
            const uint64_t nb = k / 32, blk = off / kQ80Bytes, b = off % kQ80Bytes;
            o = b < 2 ? 32 * nb + blk * 2 + b : blk * 32 + (b - 2);
        } else if (type == 12) {
            const uint64_t nsb = k / kQK, sb = off / kQ4KBytes;
            const uint32_t b = (uint32_t)(off % kQ4KBytes);
            o = b < 16 ? 128 * nsb + sb * 16 + b : q45_qs_offset(nsb, sb, b - 16);
        } else if (type == 13) {
            const uint64_t nsb = k / kQK, sb = off / kQ5KBytes;
            const uint32_t b = (uint32_t)(off % kQ5KBytes);
            if (b < 16) o = 160 * nsb + sb * 16 + b;
            else if (b < 48) o = 128 * nsb + sb * 32 + (b - 16);
            else o = q45_qs_offset(nsb, sb, b - 48);
        } else {
            o = off;
        }
        dst[r * pitch + o] = src[t];
    }
}

hipError_t launch_relayout(uint32_t type, uint64_t k, uint64_t n, const uint8_t* src,
                           uint8_t* dst, uint64_t pitch, hipStream_t s) {
    uint64_t row_bytes = 0;
    switch (type) {
        case 0: row_bytes = k * 4; break;
        case 1:
        case 30: row_bytes = k * 2; break;
        case 8: row_bytes = k / 32 * kQ80Bytes; break;
        case 12: row_bytes = k / kQK * kQ4KBytes; break;
        case 13: row_bytes = k / kQK * kQ5KBytes; break;
        case 14: row_bytes = k / kQK * kQ6KBytes; break;
        default: return hipErrorInvalidValue;
    }
    const uint64_t total = n * row_bytes;
    uint64_t blocks = (total + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    if (blocks == 0) return hipSuccess;
    hipLaunchKernelGGL(relayout_kernel, dim3((unsigned)blocks), dim3(256), 0, s, type, k, n, src,
                       dst, row_bytes, pitch);
    return hipGetLastError();
}

// ------------------------------------------------------------------ dequantize

OQ_DEVICE uint32_t ld_u16(const uint8_t* p) { return (uint32_t)p[0] | ((uint32_t)p[1] << 8); }
OQ_DEVICE uint32_t ld_u32(const uint8_t* p) {
    return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}

// one element of a q4_K / q5_K super-block (storage_decode.cpp:63-94 element map), given the
// row, the block's 16-byte header {d, dmin, scales[12]} and (q5_K) its 32 fifth-bit bytes
OQ_DEVICE float decode_q45k_elem(const uint8_t* row, uint64_t nsb, uint64_t sb, const uint8_t* hdr,
                                 const uint8_t* qh, uint32_t ii) {
#pragma clang fp contract(off)
    const float d = f16_bits_to_f32(ld_u16(hdr));
    const float dmin = f16_bits_to_f32(ld_u16(hdr + 2));
    const uint32_t g = ii / 64, hi = (ii % 64) / 32, l = ii % 32;
    uint32_t sc, mn;
    scale_min_k4(2 * g + hi, ld_u32(hdr + 4), ld_u32(hdr + 8), ld_u32(hdr + 12), sc, mn);
    const uint32_t byte = row[q45_qs_offset(nsb, sb, g * 32 + l)];
    uint32_t q = hi ? (byte >> 4) : (byte & 15u);
    if (qh && ((qh[l] >> (2 * g + hi)) & 1u)) q += 16u;
    const float ds = d * (float)sc;
    const float mm = dmin * (float)mn;
    return ds * (float)q - mm;
}

__global__ void dequantize_kernel(DeviceMatrix w, uint64_t row0, uint64_t nrows,
                                  float* __restrict__ out) {
#pragma clang fp contract(off)
    const uint64_t total = nrows * w.k;
    for (uint64_t e = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; e < total;
         e += (uint64_t)gridDim.x * blockDim.x) {
        const uint64_t r = row0 + e / w.k, i = e % w.k;
        const uint8_t* row = w.base + r * w.pitch;
        float v;
        switch (w.type) {
            case 0: v = bits_f32(ld_u32(row + 4 * i)); break;
            case 1: v = f16_bits_to_f32(ld_u16(row + 2 * i)); break;
            case 30: v = bf16_bits_to_f32(ld_u16(row + 2 * i)); break;
            case 8: {
                const uint64_t nb = w.k / 32, b = i / 32;
                const float d = f16_bits_to_f32(ld_u16(row + 32 * nb + 2 * b));
                v = d * (float)(int8_t)row[i];
                break;
            }
            case 12: {  // planes qs | hdr[nsb][16]
                const uint64_t nsb = w.k / kQK, sb = i / kQK;
                v = decode_q45k_elem(row, nsb, sb, row + 128 * nsb + sb * 16, nullptr, (uint32_t)(i % kQK));
                break;
            }
            case 13: {  // planes qs | qh[nsb][32] | hdr[nsb][16]
                const uint64_t nsb = w.k / kQK, sb = i / kQK;
                v = decode_q45k_elem(row, nsb, sb, row + 160 * nsb + sb * 16, row + 128 * nsb + sb * 32,
                                     (uint32_t)(i % kQK));
                break;
            }
            case 14: {
                // storage_decode.cpp:96-125 element map over the plane layout
                const uint64_t nsb = w.k / kQK, sb = i / kQK;
                const uint32_t ii = (uint32_t)(i % kQK);
                const uint32_t h = ii / 128, sg = (ii % 128) / 32, l = ii % 32;
                const uint8_t* qh = row + 128 * nsb + sb * 64;
                const int8_t* sc = (const int8_t*)(row + 192 * nsb + sb * 16);
                const float d = f16_bits_to_f32(ld_u16(row + 208 * nsb + sb * 2));
                const uint32_t lb = row[q6_ql_offset(nsb, sb, 64 * h + l + 32 * (sg & 1))];
                const uint32_t low = sg >= 2 ? (lb >> 4) : (lb & 15u);
                const uint32_t high = (qh[32 * h + l] >> (2 * sg)) & 3u;
                const int q = (int)(low | (high << 4)) - 32;
                const int scale = sc[q6_sc_offset(8 * h + l / 16 + 2 * sg)];
                const float ds = d * (float)scale;
                v = ds * (float)q;
                break;
            }
            default: v = 0.0f;
        }
        out[e] = v;
    }
}

hipError_t launch_dequantize(const DeviceMatrix& w, uint64_t row0, uint64_t nrows, float* out,
                             hipStream_t s) {
    const uint64_t total = nrows * w.k;
    uint64_t blocks = (total + 255) / 256;
    if (blocks > 131072) blocks = 131072;
    if (blocks == 0) return hipSuccess;
    hipLaunchKernelGGL(dequantize_kernel, dim3((unsigned)blocks), dim3(256), 0, s, w, row0, nrows,
                       out);
    return hipGetLastError();
}

// ------------------------------------------------------------------ Q8_K quantize

// One wave per 256-value block; a 256-thread workgroup quantizes four blocks.
__global__ __launch_bounds__(256) void quantize_q8k_kernel(const float* __restrict__ x,
                                                           uint64_t nblocks,
                                                           uint8_t* __restrict__ q8k) {
    const int lane = threadIdx.x & 63;
    const uint64_t blk = blockIdx.x * 4ull + (threadIdx.x >> 6);
    if (blk >= nblocks) return;
    const float4 v = reinterpret_cast<const float4*>(x + blk * kQK)[lane];
    const Q8KLane r = quantize_q8k_block_wave(v, lane);
    uint8_t* ob = q8k + blk * kQ8KBytes;
    *reinterpret_cast<uint32_t*>(ob + 4 + 4 * lane) = r.qword;
    if ((lane & 3) == 0) *reinterpret_cast<int16_t*>(ob + 260 + 2 * (lane >> 2)) = (int16_t)r.quad_bsum;
    if (lane == 0) *reinterpret_cast<float*>(ob) = r.d;
}

hipError_t launch_quantize_q8k(const float* x, uint64_t m, uint64_t k, uint8_t* q8k,
                               hipStream_t s) {
    const uint64_t nblocks = m * (k / kQK);
    const uint64_t wgs = (nblocks + 3) / 4;
    if (wgs == 0) return hipSuccess;
    hipLaunchKernelGGL(quantize_q8k_kernel, dim3((unsigned)wgs), dim3(256), 0, s, x, nblocks, q8k);
    return hipGetLastError();
}

}  // namespace oq
