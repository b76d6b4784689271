// Device helpers shared by the gfx950 kernels: exact GGML scalar decodes, the K-quant
// scale/min unpack, wave64 reductions and the Q8_K block quantizer.
//
// Everything here that feeds a bit-exact output (dequantized rows, Q8_K blocks) is compiled
// with FP contraction off, so a*b - c*d stays two roundings as in the reference's scalar C++.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "oq_internal.h"

#define OQ_DEVICE __device__ __forceinline__

namespace oq {

// ------------------------------------------------------------------ scalars

OQ_DEVICE float bits_f32(uint32_t u) { return __uint_as_float(u); }

// Loads of data read once per launch (weights, cached keys and values), marked non-temporal:
// streamed through the caches at the lowest retention, they do not evict the activation rows that
// every workgroup reads (measured: 12288 x 4096 q4_K GEMV 7.23 -> 7.07 us, 151936 x 4096 q6_K
// head 87.7 -> 79.5 us).
OQ_DEVICE uint32_t load_stream(const uint32_t* p) { return __builtin_nontemporal_load(p); }
OQ_DEVICE float load_stream(const float* p) { return __builtin_nontemporal_load(p); }
OQ_DEVICE float2 load_stream(const float2* p) {
    typedef float v2 __attribute__((ext_vector_type(2)));
    const v2 v = __builtin_nontemporal_load(reinterpret_cast<const v2*>(p));
    return make_float2(v.x, v.y);
}
OQ_DEVICE float4 load_stream(const float4* p) {
    typedef float v4 __attribute__((ext_vector_type(4)));
    const v4 v = __builtin_nontemporal_load(reinterpret_cast<const v4*>(p));
    return make_float4(v.x, v.y, v.z, v.w);
}
OQ_DEVICE uint4 load_stream(const uint4* p) {
    typedef unsigned v4 __attribute__((ext_vector_type(4)));
    const v4 v = __builtin_nontemporal_load(reinterpret_cast<const v4*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}
OQ_DEVICE uint2 load_stream(const uint2* p) {
    typedef unsigned v2 __attribute__((ext_vector_type(2)));
    const v2 v = __builtin_nontemporal_load(reinterpret_cast<const v2*>(p));
    return make_uint2(v.x, v.y);
}
OQ_DEVICE uint16_t load_stream(const uint16_t* p) { return __builtin_nontemporal_load(p); }

// Exact binary16 -> binary32 that keeps NaN payloads bit for bit (the hardware conversion
// quiets signalling NaNs; the reference's f16_to_f32, src/model/storage_decode.cpp:150-176,
// does not).  Subnormals: value = mantissa * 2^-24, exact in F32.
OQ_DEVICE float f16_bits_to_f32(uint32_t h) {
    const uint32_t sign = (h & 0x8000u) << 16;
    const uint32_t em = h & 0x7FFFu;
    if (em >= 0x7C00u) return bits_f32(sign | 0x7F800000u | ((em & 0x3FFu) << 13));
    if (em >= 0x0400u) return bits_f32(sign | ((em << 13) + (112u << 23)));
    return bits_f32(sign | __float_as_uint((float)em * 5.9604644775390625e-08f));
}

OQ_DEVICE float bf16_bits_to_f32(uint32_t h) { return bits_f32(h << 16); }

// byte `idx` (0..11) of the 12-byte K-quant scale array held in three dwords
OQ_DEVICE uint32_t byte_of3(uint32_t p0, uint32_t p1, uint32_t p2, uint32_t idx) {
    const uint32_t w = idx < 4 ? p0 : (idx < 8 ? p1 : p2);
    return (w >> (8u * (idx & 3u))) & 0xFFu;
}

// K-quant 6-bit (scale, min) pair j of 8 (src/model/storage_decode.cpp:44-61): pairs 0..3 are
// the low six bits of bytes j and j+4; pairs 4..7 take a low nibble from byte j+4 and their two
// high bits from bits 6..7 of bytes j-4 (scale) and j (min).
OQ_DEVICE void scale_min_k4(uint32_t j, uint32_t p0, uint32_t p1, uint32_t p2, uint32_t& sc,
                            uint32_t& mn) {
    if (j < 4) {
        sc = byte_of3(p0, p1, p2, j) & 63u;
        mn = byte_of3(p0, p1, p2, j + 4) & 63u;
    } else {
        const uint32_t b4 = byte_of3(p0, p1, p2, j + 4);
        sc = (b4 & 15u) | ((byte_of3(p0, p1, p2, j - 4) >> 6) << 4);
        mn = (b4 >> 4) | ((byte_of3(p0, p1, p2, j) >> 6) << 4);
    }
}

// ------------------------------------------------------------------ wave64 reductions

OQ_DEVICE float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

OQ_DEVICE float wave_max(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
    return v;
}

OQ_DEVICE int wave_min_int(int v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v = min(v, __shfl_xor(v, off, 64));
    return v;
}

// sum over aligned groups of 4 lanes
OQ_DEVICE int quad_sum_int(int v) {
    v += __shfl_xor(v, 1, 64);
    v += __shfl_xor(v, 2, 64);
    return v;
}

// DPP lane exchanges (GFX9 encodings): quad_perm [1,0,3,2] = lane^1, [2,3,0,1] = lane^2,
// row_half_mirror = 7-i within 8 lanes, row_mirror = 15-i within 16 lanes.
constexpr int kDppQuadXor1 = 0xB1;
constexpr int kDppQuadXor2 = 0x4E;
constexpr int kDppRowHalfMirror = 0x141;
constexpr int kDppRowMirror = 0x140;

template <int CTRL>
OQ_DEVICE int dpp_i(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, true);
}
template <int CTRL>
OQ_DEVICE float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, true));
}

// Sum over each row of 16 lanes, left in every lane of the row.
OQ_DEVICE float row16_sum(float v) {
    v += dpp_f<kDppQuadXor1>(v);
    v += dpp_f<kDppQuadXor2>(v);
    v += dpp_f<kDppRowHalfMirror>(v);
    v += dpp_f<kDppRowMirror>(v);
    return v;
}

// Greedy-token combination: keeps the larger value and, on equal values, the smaller index, so
// any order of combination yields the first index of the maximum; index 0xFFFFFFFF: no element;
// NaN values are never taken (the caller records them separately).
OQ_DEVICE void argmax_take(float& best, uint32_t& bi, float ov, uint32_t oi) {
    const bool take = oi != 0xFFFFFFFFu && (bi == 0xFFFFFFFFu || ov > best || (ov == best && oi < bi));
    best = take ? ov : best;
    bi = take ? oi : bi;
}

OQ_DEVICE void argmax_wave(float& best, uint32_t& bi, uint32_t& nan) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const float ov = __shfl_xor(best, off, 64);
        const uint32_t oi = __shfl_xor(bi, off, 64);
        nan |= __shfl_xor(nan, off, 64);
        argmax_take(best, bi, ov, oi);
    }
}

OQ_DEVICE float readlane_f(float v, int lane) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

// Sum over the 64 lanes of a wave; the result is wave-uniform.  Fixed association order, so
// results are deterministic run to run.
OQ_DEVICE float wave_sum_uniform(float v) {
    v = row16_sum(v);
    return (readlane_f(v, 0) + readlane_f(v, 16)) + (readlane_f(v, 32) + readlane_f(v, 48));
}

// ------------------------------------------------------------------ Q8_K

// Result of quantizing one 256-value block with one wave: lane l owns values 4l..4l+3.
struct Q8KLane {
    uint32_t qword;  // the lane's four int8 quants, little-endian
    int quad_bsum;   // sum of the 16 quants of bsums group l/4 (same in the 4 lanes of a quad)
    float d;         // block scale (wave-uniform)
};

// Wave-uniform maximum of a 32-bit unsigned key: DPP maxima within rows of 16 lanes, then the
// four row results through scalar registers.
OQ_DEVICE uint32_t wave_max_u32(uint32_t v) {
    v = max(v, (uint32_t)dpp_i<kDppQuadXor1>((int)v));
    v = max(v, (uint32_t)dpp_i<kDppQuadXor2>((int)v));
    v = max(v, (uint32_t)dpp_i<kDppRowHalfMirror>((int)v));
    v = max(v, (uint32_t)dpp_i<kDppRowMirror>((int)v));
    const uint32_t r0 = (uint32_t)__builtin_amdgcn_readlane((int)v, 0);
    const uint32_t r1 = (uint32_t)__builtin_amdgcn_readlane((int)v, 16);
    const uint32_t r2 = (uint32_t)__builtin_amdgcn_readlane((int)v, 32);
    const uint32_t r3 = (uint32_t)__builtin_amdgcn_readlane((int)v, 48);
    return max(max(r0, r1), max(r2, r3));
}

// GGML quantize_row_q8_K on one block, wave-parallel.  amax = max |x|; `max` is x at the
// FIRST index reaching amax (a strict > scan keeps the first); amax == 0 gives d = 0, q = 0.
// iscale = -127/max (correctly rounded division), q = min(127, rne(iscale*x)), d = 1/iscale.
// Identical bits to the sequential algorithm for finite x:
//  - |x| is compared through its bit pattern (non-negative floats order like unsigned ints);
//  - the first index: the lowest lane holding a value of magnitude amax (ballot + find-first),
//    and within that lane its lowest element;
//  - rne(t) for |t| < 2^22 is read from the bits of t + 1.5*2^23 (the product rounded first,
//    as GGML's nearest_int does): the low byte is q's two's-complement byte and bits - 0x4B400000
//    is q.  |iscale*x| <= 127*(1+2^-24)^2 < 127.5, so the min(127, .) clamp never binds.
OQ_DEVICE Q8KLane quantize_q8k_block_wave(float4 v, int lane) {
#pragma clang fp contract(off)
    (void)lane;
    const uint32_t b0 = __float_as_uint(v.x) & 0x7FFFFFFFu, b1 = __float_as_uint(v.y) & 0x7FFFFFFFu;
    const uint32_t b2 = __float_as_uint(v.z) & 0x7FFFFFFFu, b3 = __float_as_uint(v.w) & 0x7FFFFFFFu;
    const uint32_t amax = wave_max_u32(max(max(b0, b1), max(b2, b3)));
    Q8KLane r;
    if (amax == 0u) {
        r.qword = 0u;
        r.quad_bsum = 0;
        r.d = 0.0f;
        return r;
    }
    const bool h0 = b0 == amax, h1 = b1 == amax, h2 = b2 == amax, h3 = b3 == amax;
    // one compare mask per element, combined in scalar registers
    const uint64_t owners = __builtin_amdgcn_ballot_w64(h0) | __builtin_amdgcn_ballot_w64(h1) |
                            __builtin_amdgcn_ballot_w64(h2) | __builtin_amdgcn_ballot_w64(h3);
    const float mine = h0 ? v.x : (h1 ? v.y : (h2 ? v.z : v.w));
    const float maxv = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(mine), (int)__builtin_ctzll(owners)));
    const float iscale = -127.0f / maxv;
    constexpr float kMagic = 12582912.0f;  // 1.5 * 2^23
    const uint32_t t0 = __float_as_uint(iscale * v.x + kMagic), t1 = __float_as_uint(iscale * v.y + kMagic);
    const uint32_t t2 = __float_as_uint(iscale * v.z + kMagic), t3 = __float_as_uint(iscale * v.w + kMagic);
    // bytes 0 of t0..t3, little-endian
    r.qword = __builtin_amdgcn_perm(__builtin_amdgcn_perm(t3, t2, 0x0C0C0400u), __builtin_amdgcn_perm(t1, t0, 0x0C0C0400u),
                                    0x05040100u);
    const int s = (int)(t0 + t1 + t2 + t3 - 4u * 0x4B400000u);
    r.quad_bsum = s + dpp_i<kDppQuadXor1>(s);
    r.quad_bsum += dpp_i<kDppQuadXor2>(r.quad_bsum);
    r.d = 1.0f / iscale;
    return r;
}

// sum over the wave, butterfly order (every lane gets it)
OQ_DEVICE double wave_sum_f64(double v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

// The block's scalar activations as the reference evaluates them in F32 (qwen35_block.cpp:138-155):
// sigmoid from exp of the non-positive argument, softplus with its +-20 cut-offs, SiLU = v * sigmoid(v).
OQ_DEVICE float sigmoid_ref(float v) {
#pragma clang fp contract(off)
    if (v >= 0.0f) {
        const float e = expf(-v);
        return 1.0f / (1.0f + e);
    }
    const float e = expf(v);
    return e / (1.0f + e);
}

OQ_DEVICE float softplus_ref(float v) {
    if (v > 20.0f) return v;
    if (v < -20.0f) return expf(v);
    return log1pf(expf(v));
}

OQ_DEVICE float silu_ref(float v) {
#pragma clang fp contract(off)
    return v * sigmoid_ref(v);
}

// One quantized block stored in GGML's block_q8_K layout (f32 d, 256 int8 quants, 16 int16 bsums)
// by the wave that quantized it
OQ_DEVICE void store_q8k_block(uint8_t* ob, const Q8KLane& r, int lane) {
    *reinterpret_cast<uint32_t*>(ob + 4 + 4 * lane) = r.qword;
    if ((lane & 3) == 0) *reinterpret_cast<int16_t*>(ob + 260 + 2 * (lane >> 2)) = (int16_t)r.quad_bsum;
    if (lane == 0) *reinterpret_cast<float*>(ob) = r.d;
}

}  // namespace oq
