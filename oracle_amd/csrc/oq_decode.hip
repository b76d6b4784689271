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
//
// One thread per 16-byte piece of the destination row (a header, a quant chunk, a high-bit
// chunk, regrouped q6_K scales) or per 2-byte q6_K / q8_0 scale: the piece's source bytes are
// contiguous in the GGML block (q6_K scales: a permutation of 16 contiguous bytes), read with
// the widest loads their alignment allows.  Row and block indices are 32-bit.
OQ_DEVICE uint32_t ld_u16a(const uint8_t* p) { return *reinterpret_cast<const uint16_t*>(p); }

// 16 source bytes at a 2-byte aligned address
OQ_DEVICE uint4 ld16_a2(const uint8_t* p) {
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) w[i] = ld_u16a(p + 4 * i) | (ld_u16a(p + 4 * i + 2) << 16);
    return make_uint4(w[0], w[1], w[2], w[3]);
}

template <uint32_t TYPE>
__global__ __launch_bounds__(256) void relayout_kernel(uint32_t nsb, uint32_t n, const uint8_t* __restrict__ src,
                                                       uint8_t* __restrict__ dst, uint64_t row_bytes, uint64_t pitch) {
    // pieces per block: q4_K 9 (header, 8 quant chunks); q5_K 11 (header, 2 fifth-bit chunks, 8
    // quant chunks); q6_K 14 (8 ql chunks, 4 qh chunks, scales, d); q8_0 3 (2 quant halves, d)
    constexpr uint32_t P = TYPE == 12 ? 9 : (TYPE == 13 ? 11 : (TYPE == 14 ? 14 : 3));
    constexpr uint32_t BB = TYPE == 12 ? kQ4KBytes : (TYPE == 13 ? kQ5KBytes : (TYPE == 14 ? kQ6KBytes : kQ80Bytes));
    const uint64_t per_row = (uint64_t)nsb * P;
    const uint64_t total = per_row * n;
    for (uint64_t t = blockIdx.x * 256ull + threadIdx.x; t < total; t += (uint64_t)gridDim.x * 256u) {
        const uint32_t r = (uint32_t)(t / per_row);
        const uint32_t rem = (uint32_t)(t - (uint64_t)r * per_row);
        const uint32_t sb = rem / P, piece = rem % P;
        const uint8_t* blk = src + (uint64_t)r * row_bytes + (uint64_t)sb * BB;
        uint8_t* row = dst + (uint64_t)r * pitch;
        if constexpr (TYPE == 12) {
            // 144-byte blocks: 16-byte aligned when the tensor is
            const uint4 v = reinterpret_cast<const uint4*>(blk)[piece];
            const uint64_t o = piece == 0 ? 128ull * nsb + 16ull * sb : 16ull * perm_chunk(nsb, sb, (piece - 1) / 2, (piece - 1) % 2);
            *reinterpret_cast<uint4*>(row + o) = v;
        } else if constexpr (TYPE == 13) {
            const uint4 v = reinterpret_cast<const uint4*>(blk)[piece];
            uint64_t o;
            if (piece == 0) o = 160ull * nsb + 16ull * sb;
            else if (piece < 3) o = 128ull * nsb + 32ull * sb + 16ull * (piece - 1);
            else o = 16ull * perm_chunk(nsb, sb, (piece - 3) / 2, (piece - 3) % 2);
            *reinterpret_cast<uint4*>(row + o) = v;
        } else if constexpr (TYPE == 14) {
            // 210-byte blocks: 2-byte aligned
            if (piece < 8) {
                const uint32_t c = piece, h = c / 4, p2 = (c / 2) % 2, hf = c % 2;
                *reinterpret_cast<uint4*>(row + 16ull * perm_chunk(nsb, sb, 2 * h + hf, p2)) = ld16_a2(blk + 16 * c);
            } else if (piece < 12) {
                *reinterpret_cast<uint4*>(row + 128ull * nsb + 64ull * sb + 16ull * (piece - 8)) =
                    ld16_a2(blk + 128 + 16 * (piece - 8));
            } else if (piece == 12) {
                const uint4 v = ld16_a2(blk + 192);
                const uint32_t in[4] = {v.x, v.y, v.z, v.w};
                uint32_t out[4] = {0, 0, 0, 0};
#pragma unroll
                for (uint32_t j = 0; j < 16; ++j) {
                    const uint32_t byte = (in[j / 4] >> (8 * (j % 4))) & 0xFFu;
                    const uint32_t o = q6_sc_offset(j);
                    out[o / 4] |= byte << (8 * (o % 4));
                }
                *reinterpret_cast<uint4*>(row + 192ull * nsb + 16ull * sb) = make_uint4(out[0], out[1], out[2], out[3]);
            } else {
                *reinterpret_cast<uint16_t*>(row + 208ull * nsb + 2ull * sb) = (uint16_t)ld_u16a(blk + 208);
            }
        } else {
            // q8_0, 34-byte blocks (nsb = blocks of 32 per row): 2-byte aligned
            if (piece < 2) *reinterpret_cast<uint4*>(row + 32ull * sb + 16ull * piece) = ld16_a2(blk + 2 + 16 * piece);
            else *reinterpret_cast<uint16_t*>(row + 32ull * nsb + 2ull * sb) = (uint16_t)ld_u16a(blk);
        }
    }
}

// plain rows: bytes copied to the pitched rows, 4 bytes per thread (row_bytes is even; f16/bf16
// rows of odd length end in a 2-byte tail)
__global__ __launch_bounds__(256) void relayout_plain_kernel(uint32_t n, const uint8_t* __restrict__ src,
                                                             uint8_t* __restrict__ dst, uint64_t row_bytes,
                                                             uint64_t pitch) {
    const uint64_t per_row = (row_bytes + 3) / 4;
    const uint64_t total = per_row * n;
    for (uint64_t t = blockIdx.x * 256ull + threadIdx.x; t < total; t += (uint64_t)gridDim.x * 256u) {
        const uint64_t r = t / per_row, w = t - r * per_row;
        const uint8_t* s = src + r * row_bytes + 4 * w;
        uint8_t* d = dst + r * pitch + 4 * w;
        if (4 * w + 4 <= row_bytes) {
            *reinterpret_cast<uint32_t*>(d) = ld_u16a(s) | (ld_u16a(s + 2) << 16);
        } else {
            *reinterpret_cast<uint16_t*>(d) = (uint16_t)ld_u16a(s);
        }
    }
}

hipError_t launch_relayout(uint32_t type, uint64_t k, uint64_t n, const uint8_t* src,
                           uint8_t* dst, uint64_t pitch, hipStream_t s) {
    uint64_t row_bytes = 0, pieces = 0, nblk = 0;
    switch (type) {
        case 0: row_bytes = k * 4; break;
        case 1:
        case 30: row_bytes = k * 2; break;
        case 8: row_bytes = k / 32 * kQ80Bytes; nblk = k / 32; pieces = 3; break;
        case 12: row_bytes = k / kQK * kQ4KBytes; nblk = k / kQK; pieces = 9; break;
        case 13: row_bytes = k / kQK * kQ5KBytes; nblk = k / kQK; pieces = 11; break;
        case 14: row_bytes = k / kQK * kQ6KBytes; nblk = k / kQK; pieces = 14; break;
        default: return hipErrorInvalidValue;
    }
    if (n == 0 || row_bytes == 0) return hipSuccess;
    if (n > 0xFFFFFFFFull || nblk > 0xFFFFFFFFull) return hipErrorInvalidValue;
    const uint64_t total = pieces ? n * nblk * pieces : n * ((row_bytes + 3) / 4);
    uint64_t blocks = (total + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    const dim3 grid((unsigned)blocks), block(256);
    switch (type) {
        case 8: hipLaunchKernelGGL(relayout_kernel<8>, grid, block, 0, s, (uint32_t)nblk, (uint32_t)n, src, dst, row_bytes, pitch); break;
        case 12: hipLaunchKernelGGL(relayout_kernel<12>, grid, block, 0, s, (uint32_t)nblk, (uint32_t)n, src, dst, row_bytes, pitch); break;
        case 13: hipLaunchKernelGGL(relayout_kernel<13>, grid, block, 0, s, (uint32_t)nblk, (uint32_t)n, src, dst, row_bytes, pitch); break;
        case 14: hipLaunchKernelGGL(relayout_kernel<14>, grid, block, 0, s, (uint32_t)nblk, (uint32_t)n, src, dst, row_bytes, pitch); break;
        default: hipLaunchKernelGGL(relayout_plain_kernel, grid, block, 0, s, (uint32_t)n, src, dst, row_bytes, pitch); break;
    }
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
    store_q8k_block(q8k + blk * kQ8KBytes, quantize_q8k_block_wave(v, lane), lane);
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

// workgroup reduction of (best, bi, nan); the result is valid in thread 0
OQ_DEVICE void argmax_block(float& best, uint32_t& bi, uint32_t& nan) {
    __shared__ float sv[kArgmaxThreads / 64];
    __shared__ uint32_t si[kArgmaxThreads / 64];
    __shared__ uint32_t sn[kArgmaxThreads / 64];
    argmax_wave(best, bi, nan);
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

hipError_t launch_argmax_final(const ArgmaxPart* parts, uint32_t nparts, uint32_t* token, float* value,
                               hipStream_t s) {
    hipLaunchKernelGGL(argmax_final_kernel, dim3(1), dim3(kArgmaxThreads), 0, s, parts, nparts, token, value);
    return hipGetLastError();
}

}  // namespace oq
