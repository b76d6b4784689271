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

// ---------------------------------------------------------------- greedy token (argmax)
//
// The reference's greedy choice over a logits vector (src/runtime/sampler.cpp:30-41,
// src/runtime/qwen35_mtp.cpp:300-308): the first index holding the maximum (strict '>' in index
// order).  Two launches: workgroup g scans its contiguous slice (thread t visits t, t + 256, ...
// in increasing order and keeps its first maximum) and writes (value, index, NaN seen) to
// part[g]; one workgroup then combines the slices.  Every combination keeps the larger value and,
// on equal values, the smaller index, so the result is the first index of the maximum whatever
// the order of combination.  A NaN anywhere (the sampler rejects it) makes the token 0xFFFFFFFF.
namespace {

constexpr int kArgmaxThreads = 256;

struct ArgmaxPart {
    float value;
    uint32_t index;  // 0xFFFFFFFF: no element
    uint32_t nan;
};

OQ_DEVICE void argmax_take(float& best, uint32_t& bi, float ov, uint32_t oi) {
    const bool take = oi != 0xFFFFFFFFu && (bi == 0xFFFFFFFFu || ov > best || (ov == best && oi < bi));
    best = take ? ov : best;
    bi = take ? oi : bi;
}

// workgroup reduction of (best, bi, nan); the result is valid in thread 0
OQ_DEVICE void argmax_block(float& best, uint32_t& bi, uint32_t& nan) {
    __shared__ float sv[kArgmaxThreads / 64];
    __shared__ uint32_t si[kArgmaxThreads / 64];
    __shared__ uint32_t sn[kArgmaxThreads / 64];
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const float ov = __shfl_xor(best, off, 64);
        const uint32_t oi = __shfl_xor(bi, off, 64);
        nan |= __shfl_xor(nan, off, 64);
        argmax_take(best, bi, ov, oi);
    }
    const uint32_t t = threadIdx.x;
    if ((t & 63) == 0) {
        sv[t >> 6] = best;
        si[t >> 6] = bi;
        sn[t >> 6] = nan;
    }
    __syncthreads();
    if (t == 0) {
        for (int w = 1; w < kArgmaxThreads / 64; ++w) {
            nan |= sn[w];
            argmax_take(best, bi, sv[w], si[w]);
        }
    }
}

__global__ __launch_bounds__(kArgmaxThreads) void argmax_slice_kernel(const float* __restrict__ logits, uint32_t n,
                                                                      uint32_t slice, ArgmaxPart* __restrict__ part) {
    const uint64_t lo = (uint64_t)blockIdx.x * slice;
    const uint64_t hi = lo + slice < n ? lo + slice : n;
    float best = -__builtin_inff();
    uint32_t bi = 0xFFFFFFFFu, nan = 0;
    for (uint64_t i = lo + threadIdx.x; i < hi; i += kArgmaxThreads) {
        const float v = logits[i];
        nan |= v != v ? 1u : 0u;
        // the first visited element is taken as is (the reference starts from logits[0]), later
        // ones only when strictly larger
        if (bi == 0xFFFFFFFFu || v > best) {
            best = v;
            bi = (uint32_t)i;
        }
    }
    argmax_block(best, bi, nan);
    if (threadIdx.x == 0) part[blockIdx.x] = ArgmaxPart{best, bi, nan};
}

__global__ __launch_bounds__(kArgmaxThreads) void argmax_final_kernel(const ArgmaxPart* __restrict__ part, uint32_t parts,
                                                                      uint32_t* __restrict__ token, float* __restrict__ value) {
    float best = -__builtin_inff();
    uint32_t bi = 0xFFFFFFFFu, nan = 0;
    for (uint32_t g = threadIdx.x; g < parts; g += kArgmaxThreads) {
        const ArgmaxPart p = part[g];
        nan |= p.nan;
        argmax_take(best, bi, p.value, p.index);
    }
    argmax_block(best, bi, nan);
    if (threadIdx.x == 0) {
        *token = nan ? 0xFFFFFFFFu : bi;
        *value = best;
    }
}

}  // namespace

hipError_t launch_argmax(const float* logits, uint64_t n, uint32_t* token, float* value, void* partials,
                         hipStream_t s) {
    // slices of at least 1024 elements, at most kArgmaxParts of them
    uint64_t parts = (n + 1023) / 1024;
    if (parts > kArgmaxParts) parts = kArgmaxParts;
    const uint64_t slice = (n + parts - 1) / parts;
    auto* part = static_cast<ArgmaxPart*>(partials);
    hipLaunchKernelGGL(argmax_slice_kernel, dim3((unsigned)parts), dim3(kArgmaxThreads), 0, s, logits, (uint32_t)n,
                       (uint32_t)slice, part);
    hipLaunchKernelGGL(argmax_final_kernel, dim3(1), dim3(kArgmaxThreads), 0, s, part, (uint32_t)parts, token, value);
    return hipGetLastError();
}

}  // namespace oq
