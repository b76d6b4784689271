// Prefill / verify GEMM for K-quant weights (m >= 16 activation rows) on gfx950 matrix cores.
//
// Y[m][n] = sum_k Xhat[m][k] * W[n][k] with Xhat the dequantized Q8_K activations (d*q) and W
// the reference's decoded weights ((d*sc)*q - dmin*m for q4_K / q5_K, src/model/storage_decode.cpp
// :63-94; (d*sc)*q for q6_K, :96-125).  q4_K and q5_K run gemm_ws_kernel, q6_K gemm_ws6_kernel:
// MFMA waves convert the weights in registers while load waves stage every tile in LDS (q4_K
// 64.7 us at M = 512, 4096 x 12288).  gemm_kq_kernel, whose load waves convert each step's weights
// into an f16 B tile in LDS, stays selectable (q4_K through it: 80.6 us).  Both operands are
// rounded once to binary16 and multiplied on v_mfma_f32_32x32x16_f16 with F32 accumulation.  The
// rounding is relative 2^-11 per operand, so each product is within about 2^-10 of itself and an
// output within 2^-10 * sum_k |w_k * xhat_k| (plus F32 summation) whatever the data; over
// K >= 4096 terms that spread over many products the effect stays below 1e-4 of that sum with a
// wide margin (checked by the parity tests), so the path is enabled only for K >= 4096.
// Every kernel of a weight type forms the same f16 operands and adds the products in the same
// order, so they agree bit for bit.
//
// Data flow (one call):
//   1. activations -> F16 image Xhat[m][K] in scratch.  From F32 x the Q8_K quantization is
//      the one of quantize_q8k (bit-identical q and d) and Xhat = f16(2^e_r * d*q); caller-supplied
//      Q8_K blocks are converted the same way.  e_r is one power-of-two exponent per row (below).
//   2. GEMM: a 128 (m) x 256 (n) output tile per workgroup over one K-split of whole
//      super-blocks, in steps of 64 k.  MFMA wave w owns all 128 rows and 64 columns (4 x 2
//      accumulators of 32 x 32).
//   3. with more than one K-split, partial tiles go to scratch and a reduction kernel adds
//      them in split order (deterministic).
//
// Weight dequantization: a quant pair becomes exact f16 integers (a nibble read as fp8 e4m3 and
// converted with scale 2^9; a 5- or 6-bit value by a byte permute under the f16 exponent of 1024,
// minus 1024), and each weight is the F32 (d*sc)*q - dmin*m of the reference's F32 scale and min
// rounded once to f16 (v_fma_mixlo_f16 / v_fma_mixhi_f16, two per pair).  OQ_GEMM_FAST_DEQUANT=1
// (K >= 8192, measurement only) applies f16-rounded scale and min with one packed f16 fma per
// pair instead: about 5% faster on q4_K, but a weight that is the small difference of its scale
// and min terms then carries an error relative to those terms, not to itself, which breaks the
// bound above (9e-3 of sum |w * xhat| measured on a row dominated by a few products).  The
// conversion instructions are interleaved with the MFMAs, which execute asynchronously.
#include <algorithm>
#include <type_traits>

#include "oq_common.h"
#include "oq_layout.h"

namespace oq {

namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float float2v __attribute__((ext_vector_type(2)));
typedef float float16v __attribute__((ext_vector_type(16)));

constexpr int kBM = 128, kBN = 256, kBK = 64;
constexpr int kThreads = 256;       // 4 waves, one per SIMD
constexpr uint64_t kMinK = 4096;
// OQ_GEMM_FAST_DEQUANT=1 applies from this K on (scale and min rounded to f16 per sub-block).
constexpr uint64_t kFastMinK = 8192;
constexpr int kMaxSplits = 8;

// ---------------------------------------------------------------- activation image

OQ_DEVICE uint32_t pack_f16(float a, float b) {
    const float2v v = {a, b};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, half2v));
}

// Row exponents.  Row r of the image holds f16(2^e_r * d * q), e_r chosen so that the row's
// largest value, 127 * max |d| over its blocks, lands in [2^14, 2^15): every finite activation then
// fits binary16's range (|d q| alone can exceed 65504), and a row of small values keeps binary16's
// full relative precision instead of falling into its subnormals.  Every GEMM epilogue multiplies
// row r's outputs by 2^-e_r.  Scaling by a power of two commutes with each rounding on the way (the
// f16 operands, their exact products, the F32 sums) while values stay in the normal range, so a row
// whose values are normal with and without the scaling gives bit-identical outputs either way.
// The exponents sit in scratch right after the image (row_exponents), padded to whole m-tiles.
OQ_DEVICE int row_exponent(float amax) {
    if (!(amax > 0.0f) || !__builtin_isfinite(amax)) return 0;  // zero or non-finite rows stay as they are
    int x = 0;
    (void)frexpf(amax, &x);  // amax = f * 2^x, f in [0.5, 1)
    return 15 - x;
}

OQ_DEVICE uint64_t image_bytes(uint64_t m, uint64_t k) { return (m * k * 2 + 255) & ~uint64_t(255); }

OQ_DEVICE const int* row_exponents(const _Float16* a16, uint64_t m, uint64_t k) {
    return reinterpret_cast<const int*>(reinterpret_cast<const uint8_t*>(a16) + image_bytes(m, k));
}

// A row's workgroup: 16 waves, block b of the row on wave b % 16.  Blocks per wave whose Q8_K
// words stay in registers between the two passes: 4 (rows of up to 64 blocks, K <= 16384); the
// blocks of longer rows are quantized again in the second pass.
constexpr int kRowWaves = 16;
constexpr int kRowCache = 4;

OQ_DEVICE float row_max_of_waves(const float* wmax) {
    float v = wmax[0];
#pragma unroll
    for (int i = 1; i < kRowWaves; ++i) v = fmaxf(v, wmax[i]);
    return v;
}

// F32 x [m][K] -> the image, one workgroup per row.  Pass 1 quantizes every block of the row (the
// Q8_K quantization of quantize_q8k, bit-identical q and d; all of a wave's loads issued together)
// and reduces max |d| over the row; pass 2 writes f16(2^e d * q).
__global__ __launch_bounds__(1024) void quantize_f16_kernel(const float* __restrict__ x, uint32_t nb,
                                                            _Float16* __restrict__ out, int* __restrict__ rexp) {
    __shared__ float wmax[kRowWaves];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint64_t row = blockIdx.x;
    const float* xr = x + row * nb * (uint64_t)kQK;
    _Float16* orow = out + row * nb * (uint64_t)kQK;
    float4 v[kRowCache];
#pragma unroll
    for (int t = 0; t < kRowCache; ++t) {
        const uint32_t b = (uint32_t)wave + kRowWaves * t;
        if (b < nb) v[t] = reinterpret_cast<const float4*>(xr + (uint64_t)b * kQK)[lane];
    }
    uint32_t qw[kRowCache];
    float dv[kRowCache];
    float dmax = 0.0f;
#pragma unroll
    for (int t = 0; t < kRowCache; ++t) {
        const uint32_t b = (uint32_t)wave + kRowWaves * t;
        if (b < nb) {
            const Q8KLane r = quantize_q8k_block_wave(v[t], lane);
            qw[t] = r.qword;
            dv[t] = r.d;
            dmax = fmaxf(dmax, fabsf(r.d));
        }
    }
    for (uint32_t b = (uint32_t)wave + kRowWaves * kRowCache; b < nb; b += kRowWaves) {
        const Q8KLane r = quantize_q8k_block_wave(reinterpret_cast<const float4*>(xr + (uint64_t)b * kQK)[lane], lane);
        dmax = fmaxf(dmax, fabsf(r.d));
    }
    if (lane == 0) wmax[wave] = dmax;  // d is uniform across the wave
    __syncthreads();
    const int e = row_exponent(127.0f * row_max_of_waves(wmax));
    if (threadIdx.x == 0) rexp[row] = e;
    auto put = [&](uint32_t b, uint32_t q, float d) {
        const float ds = ldexpf(d, e);
        float f[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) f[i] = ds * (float)(int8_t)(q >> (8 * i));
        *reinterpret_cast<uint2*>(orow + (uint64_t)b * kQK + 4 * lane) = make_uint2(pack_f16(f[0], f[1]), pack_f16(f[2], f[3]));
    };
#pragma unroll
    for (int t = 0; t < kRowCache; ++t) {
        const uint32_t b = (uint32_t)wave + kRowWaves * t;
        if (b < nb) put(b, qw[t], dv[t]);
    }
    for (uint32_t b = (uint32_t)wave + kRowWaves * kRowCache; b < nb; b += kRowWaves) {
        const Q8KLane r = quantize_q8k_block_wave(reinterpret_cast<const float4*>(xr + (uint64_t)b * kQK)[lane], lane);
        put(b, r.qword, r.d);
    }
}

// Q8_K blocks [m][nb] -> the image, one workgroup per row: max |d| over the row's blocks, then
// f16(2^e d * q) as quantize_f16_kernel.
__global__ __launch_bounds__(1024) void q8k_to_f16_kernel(const uint8_t* __restrict__ q8k, uint32_t nb,
                                                          _Float16* __restrict__ out, int* __restrict__ rexp) {
    __shared__ float wmax[kRowWaves];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint64_t row = blockIdx.x;
    const uint8_t* qr = q8k + row * nb * (uint64_t)kQ8KBytes;
    _Float16* orow = out + row * nb * (uint64_t)kQK;
    float dmax = 0.0f;
    for (uint32_t b = threadIdx.x; b < nb; b += 64 * kRowWaves)
        dmax = fmaxf(dmax, fabsf(*reinterpret_cast<const float*>(qr + (uint64_t)b * kQ8KBytes)));
    dmax = __int_as_float((int)wave_max_u32((uint32_t)__float_as_int(dmax)));  // non-negative: integer order
    if (lane == 0) wmax[wave] = dmax;
    __syncthreads();
    const int e = row_exponent(127.0f * row_max_of_waves(wmax));
    if (threadIdx.x == 0) rexp[row] = e;
    for (uint32_t b = (uint32_t)wave; b < nb; b += kRowWaves) {
        const uint8_t* blk = qr + (uint64_t)b * kQ8KBytes;
        const float ds = ldexpf(*reinterpret_cast<const float*>(blk), e);
        const uint32_t q = *reinterpret_cast<const uint32_t*>(blk + 4 + 4 * lane);
        float f[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) f[i] = ds * (float)(int8_t)(q >> (8 * i));
        *reinterpret_cast<uint2*>(orow + (uint64_t)b * kQK + 4 * lane) = make_uint2(pack_f16(f[0], f[1]), pack_f16(f[2], f[3]));
    }
}

// F32 x [m][K] -> f16(2^e x), one workgroup per row (K a multiple of 256): the image of q8_0
// weights, whose products take the activations as they are (the reference multiplies q8_0 rows by
// the F32 activation, src/backend/cpu/quantized_reference.cpp:50-64).  Pass 1 reduces max |x|
// over the row, pass 2 writes; e as for the Q8_K images.
__global__ __launch_bounds__(1024) void scale_f16_kernel(const float* __restrict__ x, uint32_t nb,
                                                         _Float16* __restrict__ out, int* __restrict__ rexp) {
    __shared__ float wmax[kRowWaves];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint64_t row = blockIdx.x;
    const float* xr = x + row * nb * (uint64_t)kQK;
    _Float16* orow = out + row * nb * (uint64_t)kQK;
    float4 v[kRowCache];
    float amax = 0.0f;
#pragma unroll
    for (int t = 0; t < kRowCache; ++t) {
        const uint32_t b = (uint32_t)wave + kRowWaves * t;
        if (b < nb) {
            v[t] = reinterpret_cast<const float4*>(xr + (uint64_t)b * kQK)[lane];
            amax = fmaxf(amax, fmaxf(fmaxf(fabsf(v[t].x), fabsf(v[t].y)), fmaxf(fabsf(v[t].z), fabsf(v[t].w))));
        }
    }
    for (uint32_t b = (uint32_t)wave + kRowWaves * kRowCache; b < nb; b += kRowWaves) {
        const float4 u = reinterpret_cast<const float4*>(xr + (uint64_t)b * kQK)[lane];
        amax = fmaxf(amax, fmaxf(fmaxf(fabsf(u.x), fabsf(u.y)), fmaxf(fabsf(u.z), fabsf(u.w))));
    }
    amax = __int_as_float((int)wave_max_u32((uint32_t)__float_as_int(amax)));  // non-negative: integer order
    if (lane == 0) wmax[wave] = amax;
    __syncthreads();
    const int e = row_exponent(row_max_of_waves(wmax));
    if (threadIdx.x == 0) rexp[row] = e;
    auto put = [&](uint32_t b, float4 u) {
        *reinterpret_cast<uint2*>(orow + (uint64_t)b * kQK + 4 * lane) =
            make_uint2(pack_f16(ldexpf(u.x, e), ldexpf(u.y, e)), pack_f16(ldexpf(u.z, e), ldexpf(u.w, e)));
    };
#pragma unroll
    for (int t = 0; t < kRowCache; ++t) {
        const uint32_t b = (uint32_t)wave + kRowWaves * t;
        if (b < nb) put(b, v[t]);
    }
    for (uint32_t b = (uint32_t)wave + kRowWaves * kRowCache; b < nb; b += kRowWaves)
        put(b, reinterpret_cast<const float4*>(xr + (uint64_t)b * kQK)[lane]);
}

// One wave's 128 x 64 output tile (accumulators acc[i][j]: m-subtile i, n-subtile j, 32 x 32 each;
// result register r of lane l: row 8 (r / 4) + 4 (l / 32) + r % 4, column l % 32), stored to o
// (m x n, row-major).  col0: the wave's first column.  With rexp (the last writer of the outputs:
// a single K-split) each row is scaled back by 2^-e_row; a split's partial tile is stored as it
// is and the split reduction scales the sums back.
OQ_DEVICE void store_wave_tile(float* __restrict__ o, const int* __restrict__ rexp, uint64_t m0, uint64_t m,
                               uint64_t n, uint64_t col0, int h, int r0, const float16v (&acc)[4][2]) {
    int e[4][16] = {};
    if (rexp != nullptr) {
        // rows 8 g + 4 h + 0..3 of m-subtile i: four consecutive exponents per load, all 16 loads
        // issued before the first use (the array is padded to whole m-tiles: reads stay inside it)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int4 ev = *reinterpret_cast<const int4*>(rexp + m0 + 32 * i + 8 * g + 4 * h);
                e[i][4 * g] = ev.x;
                e[i][4 * g + 1] = ev.y;
                e[i][4 * g + 2] = ev.z;
                e[i][4 * g + 3] = ev.w;
            }
        }
    }
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const uint64_t col = col0 + 32 * j + r0;
        if (col >= n) continue;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
#pragma unroll
            for (int rr = 0; rr < 16; ++rr) {
                const uint64_t row = m0 + 32 * i + 8 * (rr / 4) + 4 * h + (rr % 4);
                if (row < m) o[row * n + col] = rexp != nullptr ? ldexpf(acc[i][j][rr], -e[i][rr]) : acc[i][j][rr];
            }
        }
    }
}

// ---------------------------------------------------------------- tiles and addressing
//
// One workgroup: a 128 (m) x 256 (n) output tile over one K-split, in steps of 64 k (a quarter
// super-block, "group" G = 0..3: sub-blocks 2G and 2G+1).  Wave w owns all 128 rows and columns
// n0 + 64 w .. n0 + 64 w + 63 (4 x 2 accumulators of 32 x 32).
//
// Activation tiles (F16, 128 rows x 64 k = 16 KB) pass through a ring of four LDS buffers; the
// tile of step s sits in buffer s % 4, so inside the four-step loop body every LDS address is a
// per-lane constant plus an immediate.  Row r holds eight 16-byte chunks; logical chunk c sits at
// physical chunk c ^ ((r / 2) % 8), which keeps the operand reads and the tile writes free of
// bank conflicts without padding.
//
// k order inside one group (the same for both operands, so the product is unchanged): MFMA
// k-slice ks (16 k), lane half h, operand element i covers k = 32 (ks & 1) + 16 h + 8 (ks >> 1) + i.
//   A: 8 consecutive k = logical chunk 4 (ks & 1) + 2 h + (ks >> 1) of a tile row;
//   B: bytes 16 h + 8 (ks >> 1) + i of the weight row's 32-byte group chunk pair, low nibbles for
//      even ks, high nibbles for odd ks: lane half h reads only chunk e = h of the group (see
//      oq_layout.h), and slice ks lies inside sub-block 2G + (ks & 1).
OQ_DEVICE int a_chunk(int ks, int h) { return 4 * (ks & 1) + 2 * h + (ks >> 1); }

constexpr uint32_t kTileBytes = kBM * kBK * 2;  // 16 KB

// ---------------------------------------------------------------- per-sub-block scales
//
// Scale state of one (weight row, sub-block):
//   FAST : one dword = f16 pair {d*sc, -(dmin*m)}, each the exact product rounded once to f16;
//   exact: F32 {d*sc, dmin*m} as the reference computes them (two F32 products, no contraction).
// Pairs for sub-blocks 2G, 2G+1 of a header (f16 d, f16 dmin, 12 packed 6-bit scale/min bytes):
// the four 6-bit values of a half super-block are unpacked bytewise in one go, the same unpack
// as scale_min_k4 (src/model/storage_decode.cpp:44-61).
template <int G>
OQ_DEVICE void unpack_scale_bytes(uint4 hdr, uint32_t& scb, uint32_t& mnb) {
    if (G < 2) {
        scb = hdr.y & 0x3F3F3F3Fu;
        mnb = hdr.z & 0x3F3F3F3Fu;
    } else {
        scb = (hdr.w & 0x0F0F0F0Fu) | ((hdr.y >> 2) & 0x30303030u);
        mnb = ((hdr.w >> 4) & 0x0F0F0F0Fu) | ((hdr.z >> 2) & 0x30303030u);
    }
}

template <bool FAST>
struct ScaleT;
template <>
struct ScaleT<true> {
    uint32_t v;
};
template <>
struct ScaleT<false> {
    float ds, dm;
};

template <bool FAST, int G>
OQ_DEVICE void scale_pairs(uint4 hdr, ScaleT<FAST> (&out)[2]) {
    uint32_t scb, mnb;
    unpack_scale_bytes<G>(hdr, scb, mnb);
#pragma unroll
    for (int par = 0; par < 2; ++par) {
        const uint32_t b = (2 * G + par) & 3;
        if constexpr (FAST) {
            // {sc, mn} as the f16 values 1024 + sc, 1024 + mn (exact), minus 1024, times {d, -dmin}
            const half2v k1024 = {(_Float16)1024.0f, (_Float16)1024.0f};
            const uint32_t sel = b | (0x0Cu << 8) | ((4u + b) << 16) | (0x0Cu << 24);
            const uint32_t v = __builtin_amdgcn_perm(mnb, scb, sel) | 0x64006400u;
            const half2v dd = __builtin_bit_cast(half2v, hdr.x ^ 0x80000000u);
            half2v x = __builtin_bit_cast(half2v, v) - k1024;
            out[par].v = __builtin_bit_cast(uint32_t, x * dd);
        } else {
            // hardware f16 -> f32 (exact for every finite value; NaN payloads do not matter here)
            const float d = (float)__builtin_bit_cast(_Float16, (uint16_t)(hdr.x & 0xFFFFu));
            const float dmin = (float)__builtin_bit_cast(_Float16, (uint16_t)(hdr.x >> 16));
            const float sc = (float)((scb >> (8 * b)) & 0xFFu);
            const float mn = (float)((mnb >> (8 * b)) & 0xFFu);
            {
#pragma clang fp contract(off)
                out[par].ds = d * sc;
                out[par].dm = dmin * mn;
            }
        }
    }
}

// ---------------------------------------------------------------- weight conversion
//
// Nibble word of slice ks (4 weights, one per byte, values 0..15) from a lane's 16-byte group
// chunk: dwords x, y for ks < 2, z, w for ks >= 2; low nibbles for even ks, high for odd.
template <int KS>
OQ_DEVICE uint32_t nib_word(uint4 q, int half) {
    const uint32_t d = (KS >> 1) == 0 ? (half == 0 ? q.x : q.y) : (half == 0 ? q.z : q.w);
    return (KS & 1) ? (d >> 4) & 0x0F0F0F0Fu : d & 0x0F0F0F0Fu;
}

// f16(fma(x_i, a, c)) for both halves of x (exact f16 integers): the F32 fma of an f16 operand
// converted to f16, which is one v_fma_mixlo_f16 / v_fma_mixhi_f16 each (x stays packed, no
// widening instructions).
OQ_DEVICE uint32_t mix_pair(half2v x, float a, float c) {
    const half2v r = {(_Float16)__builtin_fmaf((float)x[0], a, c), (_Float16)__builtin_fmaf((float)x[1], a, c)};
    return __builtin_bit_cast(uint32_t, r);
}

// Two weights of a B operand from bytes 2p, 2p+1 of a nibble word.  A byte q in 0..15 read as
// an fp8 e4m3 pattern is q * 2^-9 (subnormal or the first binade), so the scaled fp8 conversion
// with scale 2^9 yields q exactly, two per instruction.
//   FAST : one v_pk_fma_f16 with {d*sc, -(dmin*m)}: f16(d*sc*q - dmin*m) from the f16-rounded
//          scale and min, one rounding;
//   exact: the F32 fma with the reference's F32 scale and min, rounded to f16 (mix_pair).
template <bool FAST, int P>
OQ_DEVICE uint32_t weight_pair(uint32_t nib, const ScaleT<FAST>& s) {
    const half2v x = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(nib, 512.0f, P != 0);
    if constexpr (FAST) {
        const half2v sv = __builtin_bit_cast(half2v, s.v);
        const half2v r = __builtin_elementwise_fma(x, __builtin_shufflevector(sv, sv, 0, 0),
                                                   __builtin_shufflevector(sv, sv, 1, 1));
        return __builtin_bit_cast(uint32_t, r);
    } else {
        return mix_pair(x, s.ds, -s.dm);
    }
}

OQ_DEVICE uint32_t dword_of(uint4 v, int i) { return i == 0 ? v.x : (i == 1 ? v.y : (i == 2 ? v.z : v.w)); }

// Bytes (2P, 2P+1) of a word of quant values (below 256) as the f16 pair {1024 + q0, 1024 + q1}:
// one byte permute that puts 0x64 (the high byte of f16 1024) above each quant byte.
template <int P>
OQ_DEVICE half2v f16_1024_pair(uint32_t v) {
    const uint32_t sel = P ? 0x04030402u : 0x04010400u;
    return __builtin_bit_cast(half2v, __builtin_amdgcn_perm(0x64646464u, v, sel));
}

// Two weights (bytes 2P, 2P+1 of the word of 5-bit quants q) of a q5_K sub-block: (d sc) q - dmin m,
// with the same scale state and rounding as weight_pair.
template <bool FAST, int P>
OQ_DEVICE uint32_t q5_pair(uint32_t q, const ScaleT<FAST>& s) {
    if constexpr (FAST) {
        const half2v k1024 = {(_Float16)1024.0f, (_Float16)1024.0f};
        const half2v x = f16_1024_pair<P>(q) - k1024;  // exact integers 0..31
        const half2v sv = __builtin_bit_cast(half2v, s.v);
        const half2v r = __builtin_elementwise_fma(x, __builtin_shufflevector(sv, sv, 0, 0),
                                                   __builtin_shufflevector(sv, sv, 1, 1));
        return __builtin_bit_cast(uint32_t, r);
    } else {
        const half2v k1024 = {(_Float16)1024.0f, (_Float16)1024.0f};
        return mix_pair(f16_1024_pair<P>(q) - k1024, s.ds, -s.dm);
    }
}

// Two weights of a q6_K sub-block from the word of 6-bit codes u (q = u - 32): (d sc) q.
//   FAST : ds = f16(d * sc) (d * sc is exact in F32), x = q exactly, one v_pk_mul_f16;
//   exact: F32 (d * sc) * q as the reference (exact in F32), rounded to f16; the F32 product is
//          formed as fma(q, d * sc, +0), so a zero weight is +0 whatever the sign of the scale.
template <bool FAST, int P>
OQ_DEVICE uint32_t q6_pair(uint32_t u, float ds) {
    const half2v k1056 = {(_Float16)1056.0f, (_Float16)1056.0f};
    const half2v x = f16_1024_pair<P>(u) - k1056;  // exact integers -32..31
    if constexpr (FAST) {
        const _Float16 h = (_Float16)ds;
        const half2v dv = {h, h};
        return __builtin_bit_cast(uint32_t, x * dv);
    } else {
        return mix_pair(x, ds, 0.0f);
    }
}

// Two weights of a q8_0 block from bytes (2P, 2P+1) of a word of int8 quants: the bytes offset to
// unsigned (q + 128) become the exact f16 integers 1024 + q + 128, minus 1152 gives q, and one
// v_pk_mul_f16 by the block's f16 d rounds d * q (exact in F32) once: f16(d * q).
template <int P>
OQ_DEVICE uint32_t q8_pair(uint32_t v, uint32_t dbits) {
    const half2v k1152 = {(_Float16)1152.0f, (_Float16)1152.0f};
    const half2v x = f16_1024_pair<P>(v ^ 0x80808080u) - k1152;
    const _Float16 dh = __builtin_bit_cast(_Float16, (uint16_t)dbits);
    const half2v dv = {dh, dh};
    return __builtin_bit_cast(uint32_t, x * dv);
}

// q4_K (TYPE 12) or q5_K (13) weight pair from a word of quant bytes (nibbles, or 5-bit values)
template <uint32_t TYPE, bool FAST, int P>
OQ_DEVICE uint32_t k_pair(uint32_t q, const ScaleT<FAST>& s) {
    if constexpr (TYPE == 13) return q5_pair<FAST, P>(q, s);
    else return weight_pair<FAST, P>(q, s);
}

// The fifth bits of q5_K slice ks of group g for bytes 4e .. 4e + 3 of a lane's chunk half, moved
// to bit 4 of each byte: byte l of the lane's 16-byte high-bit half holds bit 2g + (ks & 1) for
// element l of that half (GGML block_q5_K qh, src/model/storage_decode.cpp:63-94).
OQ_DEVICE uint32_t q5_high(uint4 qh, int ks, int g, int e) {
    return ((dword_of(qh, 2 * (ks >> 1) + e) >> (2 * g + (ks & 1))) & 0x01010101u) << 4;
}

// ---------------------------------------------------------------- wave state
//
// Per lane, fixed for the whole workgroup:
//   act_off[j]  byte offset of activation chunk c = tid + 256 j (row c / 8 of the m-tile, chunk
//               c % 8) within a 64-k column block of the F16 image (rows clamped to m - 1);
//   st_off      LDS byte offset of the tile stores (buffer 0, j = 0; +4096 per j);
//   rd_off[ks]  LDS byte offset of the A operand read of slice ks (buffer 0, m-subtile 0);
//   row_off[j]  byte offset of weight row n0 + 64 w + 32 j + lane % 32 (clamped to n - 1).
// Global addresses are a uniform (scalar) base plus these 32-bit lane offsets.
struct WaveState {
    uint32_t act_off[4];
    uint32_t st_off;
    uint32_t rd_off[4];
    uint32_t row_off[2];
};

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

OQ_DEVICE half8 lds_read(const uint8_t* lds, uint32_t off) {
    return *reinterpret_cast<const half8*>(lds + off);
}

OQ_DEVICE half8 as_b_operand(const uint32_t (&b)[4]) {
    const u32x4 v = {b[0], b[1], b[2], b[3]};
    return __builtin_bit_cast(half8, v);
}

// Workgroup barrier after this wave's LDS operations have completed.  Unlike __syncthreads() it
// does not wait for outstanding global loads (the prefetches in flight across the barrier).
OQ_DEVICE void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// Work units (n-tile, m-tile, K-split) are numbered so that the workgroups one XCD receives
// (workgroup ids are dealt to the eight XCDs in turn) share a K-split and a band of n-tiles:
// each XCD then reads its activation rows once and its weight rows once.
struct Unit {
    uint32_t nt, mt, z;
};

OQ_DEVICE Unit unit_of(uint32_t id, uint32_t tiles_n, uint32_t tiles_m, uint32_t splits) {
    const uint32_t total = tiles_n * tiles_m * splits;
    uint32_t u = id;
    if (total % 8 == 0) u = (id % 8) * (total / 8) + id / 8;
    Unit r;
    r.mt = u % tiles_m;
    r.nt = (u / tiles_m) % tiles_n;
    r.z = u / (tiles_m * tiles_n);
    return r;
}

// Uniform addressing of one K-split: super-block i (0-based within the split, clamped to the
// last one) and activation step s (clamped to the last step).
struct Split {
    const uint8_t* wbase;   // weight matrix base
    const uint8_t* a16;     // F16 image, column of the split's first super-block
    uint32_t sb0, nsbu, nsb, last_step, hdr_base;
};

OQ_DEVICE uint32_t split_sb(const Split& sp, uint32_t i) { return sp.sb0 + (i < sp.nsbu ? i : sp.nsbu - 1); }

// quant chunk (group g, lane half h) of super-block sb: uniform part, and the lane part that
// depends on the pass length of that super-block
OQ_DEVICE const uint8_t* quant_base(const Split& sp, uint32_t sb, int g) {
    return sp.wbase + 16u * (128u * (sb / 16u) + 4u * (sb % 16u) + (uint32_t)g);
}

OQ_DEVICE uint32_t quant_lane(const Split& sp, uint32_t sb, uint32_t hmask) {
    const uint32_t pass = sb / 16u;
    const uint32_t mp = sp.nsb - 16u * pass < 16u ? sp.nsb - 16u * pass : 16u;
    return hmask & (64u * mp);
}

OQ_DEVICE uint4 load_u4(const uint8_t* base, uint32_t off) {
    return *reinterpret_cast<const uint4*>(base + off);
}

// ---------------------------------------------------------------- one step of one wave
//
// Multiplies group G of the current super-block (activation tile in buffer G) and meanwhile:
//   - reads the A operands of the next k-slice (the last slice reads slice 0 of the next step
//     from buffer (G + 1) % 4) and converts the B operands of the next k-slice (the last slice
//     converts slice 0 of the next step from wq[(G + 1) % 4], holding the next super-block's
//     group 0 when G = 3);
//   - stores the activation tile of step s + 3 (loaded two steps earlier, register set
//     (G + 1) % 2) into buffer (G + 3) % 4, whose last reader was step s - 1, and loads the
//     tile of step s + 5 into the same register set;
//   - computes the scale state of the next step (from hdr, or from hdrn when G = 3);
//   - when G = 0 loads the next super-block's headers; after its last use of wq[G] loads the
//     next super-block's group G into it.
// MFMAs execute asynchronously; every MFMA is followed by a small piece of the conversion and
// pinned there with sched_barrier, since a wave issues in order and MFMAs grouped together
// would hold the conversion back.
template <bool FAST, int G>
OQ_DEVICE void wave_step(const uint8_t* lds, uint8_t* lds_w, const WaveState& ws, const Split& sp,
                         uint32_t i_sb, uint32_t s, uint32_t hmask, float16v (&acc)[4][2], half8 (&a)[4],
                         uint32_t (&b)[2][4], uint4 (&wq)[4][2], uint4 (&hdr)[2], uint4 (&hdrn)[2],
                         ScaleT<FAST> (&sc)[2][2][2], uint4 (&act)[2][4]) {
    constexpr int G1 = (G + 1) & 3;
    constexpr int P = G & 1;       // scale set of this step
    constexpr int AS = (G + 1) & 1;  // activation register set stored and reloaded by this step
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
        const int nks = (ks + 1) & 3;
        const uint32_t nbuf = ks < 3 ? (uint32_t)G : (uint32_t)G1;
        half8 an[4];
        uint32_t bn[2][4];
        uint32_t nw[2][2];
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            const int i = q >> 1, j = q & 1;
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[i], as_b_operand(b[j]), acc[i][j], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
            if (q == 0) {
#pragma unroll
                for (int ii = 0; ii < 4; ++ii) an[ii] = lds_read(lds, nbuf * kTileBytes + 4096u * ii + ws.rd_off[nks]);
            }
            // B operand of the next slice: MFMA q converts pair q % 4 of n-tile q / 4
            const int jj = q >> 2, pp = q & 3;
            const uint4 src = ks < 3 ? wq[G][jj] : wq[G1][jj];
            const ScaleT<FAST>& scl = ks < 3 ? sc[P][jj][nks & 1] : sc[P ^ 1][jj][0];
            if (pp == 0) {
                if (nks == 0) {
                    nw[jj][0] = nib_word<0>(src, 0);
                    nw[jj][1] = nib_word<0>(src, 1);
                } else if (nks == 1) {
                    nw[jj][0] = nib_word<1>(src, 0);
                    nw[jj][1] = nib_word<1>(src, 1);
                } else if (nks == 2) {
                    nw[jj][0] = nib_word<2>(src, 0);
                    nw[jj][1] = nib_word<2>(src, 1);
                } else {
                    nw[jj][0] = nib_word<3>(src, 0);
                    nw[jj][1] = nib_word<3>(src, 1);
                }
            }
            bn[jj][pp] = (pp & 1) ? weight_pair<FAST, 1>(nw[jj][pp >> 1], scl) : weight_pair<FAST, 0>(nw[jj][pp >> 1], scl);
            // side work
            if (ks == 0 && q >= 1 && q <= 4) {
                const int jt = q - 1;
                *reinterpret_cast<uint4*>(lds_w + ((G + 3) & 3) * kTileBytes + 4096u * jt + ws.st_off) = act[AS][jt];
            }
            if (ks == 1 && q < 4) {
                const uint32_t st = s + 5 < sp.last_step ? s + 5 : sp.last_step;
                act[AS][q] = load_u4(sp.a16 + 128u * st, ws.act_off[q]);
            }
            if (ks == 1 && q == 4) {
                if (G < 3) scale_pairs<FAST, G1>(hdr[0], sc[P ^ 1][0]);
                else scale_pairs<FAST, 0>(hdrn[0], sc[P ^ 1][0]);
            }
            if (ks == 1 && q == 6) {
                if (G < 3) scale_pairs<FAST, G1>(hdr[1], sc[P ^ 1][1]);
                else scale_pairs<FAST, 0>(hdrn[1], sc[P ^ 1][1]);
            }
            if (G == 0 && ks == 2 && q < 2) {
                const uint32_t sbn = split_sb(sp, i_sb + 1);
                hdrn[q] = load_u4(sp.wbase + sp.hdr_base + 16u * sbn, ws.row_off[q]);
            }
            if (ks == 3 && q < 2) {
                const uint32_t sbn = split_sb(sp, i_sb + 1);
                wq[G][q] = load_u4(quant_base(sp, sbn, G), ws.row_off[q] + quant_lane(sp, sbn, hmask));
            }
            __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int ii = 0; ii < 4; ++ii) a[ii] = an[ii];
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int e = 0; e < 4; ++e) b[j][e] = bn[j][e];
    }
}

// grid: tiles_n * tiles_m * splits workgroups of 4 waves.  Output: y (one split) or
// partial[z][m][n].
template <bool FAST>
__global__ __launch_bounds__(kThreads) void gemm_q4k_f16_kernel(DeviceMatrix w, int m, const _Float16* a16,
                                                               uint32_t tiles_n, uint32_t tiles_m, uint32_t splits,
                                                               float* __restrict__ out) {
    __shared__ __align__(16) uint8_t lds[4 * kTileBytes];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int h = lane >> 5, r0 = lane & 31;
    const uint32_t hmask = h ? 0xFFFFFFFFu : 0u;
    const uint32_t nsb = (uint32_t)(w.k / kQK);
    const Unit un = unit_of(blockIdx.x, tiles_n, tiles_m, splits);
    const uint32_t z = un.z;
    const uint64_t n0 = (uint64_t)un.nt * kBN, m0 = (uint64_t)un.mt * kBM;
    Split sp;
    sp.sb0 = (uint32_t)((uint64_t)z * nsb / splits);
    const uint32_t sb1 = (uint32_t)((uint64_t)(z + 1) * nsb / splits);
    sp.nsbu = sb1 - sp.sb0;  // >= 1: splits <= nsb
    sp.nsb = nsb;
    sp.last_step = 4 * sp.nsbu - 1;
    sp.hdr_base = 128u * nsb;
    sp.wbase = w.base;
    sp.a16 = reinterpret_cast<const uint8_t*>(a16) + 2ull * kQK * sp.sb0;

    WaveState ws;
    const uint32_t krow = (uint32_t)(w.k * 2);  // bytes per F16 image row
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        uint64_t row = m0 + (uint32_t)(tid >> 3) + 32u * j;
        row = row < (uint64_t)m ? row : (uint64_t)m - 1;
        ws.act_off[j] = (uint32_t)row * krow + 16u * (uint32_t)(tid & 7);
    }
    ws.st_off = 128u * (uint32_t)(tid >> 3) + 16u * (uint32_t)((tid & 7) ^ ((tid >> 4) & 7));
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) ws.rd_off[ks] = 128u * (uint32_t)r0 + 16u * (uint32_t)(a_chunk(ks, h) ^ ((r0 >> 1) & 7));
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        uint64_t n = n0 + 64 * wave + 32 * j + r0;
        n = n < w.n ? n : w.n - 1;
        ws.row_off[j] = (uint32_t)(n * w.pitch);
    }

    float16v acc[4][2] = {};
    // prologue: activation tiles 0..2 into buffers 0..2, tiles 3 and 4 in flight (sets 1, 0)
    uint4 act[2][4];
    for (uint32_t t = 0; t < 3; ++t) {
        const uint32_t st = t < sp.last_step ? t : sp.last_step;
        uint4 v[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] = load_u4(sp.a16 + 128u * st, ws.act_off[j]);
#pragma unroll
        for (int j = 0; j < 4; ++j) *reinterpret_cast<uint4*>(lds + t * kTileBytes + 4096u * j + ws.st_off) = v[j];
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        act[1][j] = load_u4(sp.a16 + 128u * (3 < sp.last_step ? 3 : sp.last_step), ws.act_off[j]);
        act[0][j] = load_u4(sp.a16 + 128u * (4 < sp.last_step ? 4 : sp.last_step), ws.act_off[j]);
    }
    // weights of the first super-block: headers and the four groups
    uint4 hdr[2], hdrn[2], wq[4][2];
    {
        const uint32_t sb = sp.sb0;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            hdr[j] = load_u4(sp.wbase + sp.hdr_base + 16u * sb, ws.row_off[j]);
            hdrn[j] = hdr[j];
#pragma unroll
            for (int g = 0; g < 4; ++g) wq[g][j] = load_u4(quant_base(sp, sb, g), ws.row_off[j] + quant_lane(sp, sb, hmask));
        }
    }
    ScaleT<FAST> sc[2][2][2];
    scale_pairs<FAST, 0>(hdr[0], sc[0][0]);
    scale_pairs<FAST, 0>(hdr[1], sc[0][1]);
    lds_barrier();
    half8 a[4];
    uint32_t b[2][4];
#pragma unroll
    for (int i = 0; i < 4; ++i) a[i] = lds_read(lds, 4096u * i + ws.rd_off[0]);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const uint32_t w0 = nib_word<0>(wq[0][j], 0), w1 = nib_word<0>(wq[0][j], 1);
        b[j][0] = weight_pair<FAST, 0>(w0, sc[0][j][0]);
        b[j][1] = weight_pair<FAST, 1>(w0, sc[0][j][0]);
        b[j][2] = weight_pair<FAST, 0>(w1, sc[0][j][0]);
        b[j][3] = weight_pair<FAST, 1>(w1, sc[0][j][0]);
    }
    for (uint32_t i = 0; i < sp.nsbu; ++i) {
        const uint32_t s = 4 * i;
        wave_step<FAST, 0>(lds, lds, ws, sp, i, s, hmask, acc, a, b, wq, hdr, hdrn, sc, act);
        lds_barrier();
        wave_step<FAST, 1>(lds, lds, ws, sp, i, s + 1, hmask, acc, a, b, wq, hdr, hdrn, sc, act);
        lds_barrier();
        wave_step<FAST, 2>(lds, lds, ws, sp, i, s + 2, hmask, acc, a, b, wq, hdr, hdrn, sc, act);
        lds_barrier();
        wave_step<FAST, 3>(lds, lds, ws, sp, i, s + 3, hmask, acc, a, b, wq, hdr, hdrn, sc, act);
        lds_barrier();
        hdr[0] = hdrn[0];
        hdr[1] = hdrn[1];
    }
    store_wave_tile(out + (uint64_t)z * (uint64_t)m * w.n, splits > 1 ? nullptr : row_exponents(a16, (uint64_t)m, w.k),
                    m0, (uint64_t)m, w.n, n0 + 64 * wave, h, r0, acc);
}

// ---------------------------------------------------------------- producer / consumer variant
//
// 8 waves per workgroup, two per SIMD: consumer waves 0..3 (the MFMA waves above: all 128 rows,
// columns 64 c .. 64 c + 63, B converted in registers) and producer waves 4..7, which do every
// global load of the workgroup and stage it in LDS.  An MFMA on one wave and vector work on the
// other wave of its SIMD run side by side, and the consumers' own instruction stream holds only
// LDS reads, conversions and MFMAs: no global load latency reaches them through the in-order
// load counter.
//
// LDS (dynamic, 136 KB; 152 KB for q5_K):
//   A ring   4 x 16 KB  activation tile of step s in buffer s % 4 (layout as above)
//   W ring   2 x 32 KB  the quant chunks of super-block i in slot i % 2: group g, row n, half e
//                       at g * 8 KB + ((32 n + 16 e) ^ (64 g))
//   H ring   2 x  4 KB  the headers of super-block i in slot i % 2: row n at 16 n
//   Q ring   2 x  8 KB  q5_K only: the 32-byte high-bit planes of super-block i in slot i % 2,
//                       half e of row n at 4096 e + 16 n (a half-wave reads 512 contiguous bytes)
// Producer p: activation rows 32 p .. 32 p + 31 of each tile (four 16-byte chunks per lane, eight
// rows of 128 bytes per load instruction) and weight rows 64 p .. 64 p + 63: per super-block 8 KB
// of quants, loaded as 16 row pieces of 64 contiguous bytes per instruction (four lanes per
// piece), one 16-byte header per lane and, for q5_K, the lane row's 32-byte high-bit plane.
// Timing, step s = 4 i + g of the split:
//   producer: stores tile s + 3 (loaded at step s - 2) into buffer (s + 3) % 4 and loads tile
//             s + 5; at g = 0 stores super-block i + 1 (loaded during super-block i - 1) into W/H
//             slot (i + 1) % 2, whose last reader was super-block i - 1, and loads super-block i + 2;
//   consumer: multiplies step s; during it reads the next step's quant chunks (and at g = 3 the
//             next super-block's headers and high-bit halves) from LDS;
//   all 8 waves: one barrier per step.
constexpr uint32_t kWsThreads = 512;
constexpr uint32_t kWsA = 4 * kTileBytes;   // 64 KB
constexpr uint32_t kWsWSlot = 32768;
constexpr uint32_t kWsHSlot = 4096;
constexpr uint32_t kWsQSlot = 8192;
constexpr uint32_t kWsLds = kWsA + 2 * kWsWSlot + 2 * kWsHSlot;
template <uint32_t TYPE>
constexpr uint32_t ws_lds_bytes() { return kWsLds + (TYPE == 13 ? 2 * kWsQSlot : 0u); }

OQ_DEVICE uint32_t ws_w_off(uint32_t slot, uint32_t g, uint32_t n, uint32_t e) {
    return kWsA + slot * kWsWSlot + g * 8192u + ((32u * n + 16u * e) ^ (64u * g));
}
OQ_DEVICE uint32_t ws_h_off(uint32_t slot, uint32_t n) { return kWsA + 2 * kWsWSlot + slot * kWsHSlot + 16u * n; }
OQ_DEVICE uint32_t ws_q_off(uint32_t slot, uint32_t n, uint32_t e) {
    return kWsLds + slot * kWsQSlot + 4096u * e + 16u * n;
}

// consumer: one step (see wave_step); W chunks of this step in wc[j], of the next step in wn[j]
// (read here from LDS at slice 1), scale state as there; headers of this super-block in hdr,
// of the next one in hdrn (read at g = 3); for q5_K the lane's high-bit halves of this
// super-block in qh, of the next one in qhn (read at g = 3).
template <uint32_t TYPE, bool FAST, int G>
OQ_DEVICE void ws_consumer_step(const uint8_t* lds, const uint32_t (&rd_off)[4], uint32_t wslot, uint32_t wslot_next,
                                uint32_t hslot_next, uint32_t n_lane0, uint32_t h, float16v (&acc)[4][2],
                                half8 (&a)[4], uint32_t (&b)[2][4], const uint4 (&wc)[2], uint4 (&wn)[2],
                                const uint4 (&hdr)[2], uint4 (&hdrn)[2], const uint4 (&qh)[2], uint4 (&qhn)[2],
                                ScaleT<FAST> (&sc)[2][2][2]) {
    constexpr int G1 = (G + 1) & 3;
    constexpr int P = G & 1;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
        const int nks = (ks + 1) & 3;
        const uint32_t nbuf = ks < 3 ? (uint32_t)G : (uint32_t)G1;
        half8 an[4];
        uint32_t bn[2][4];
        uint32_t nw[2][2];
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            const int i = q >> 1, j = q & 1;
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[i], as_b_operand(b[j]), acc[i][j], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
            if (q == 0) {
#pragma unroll
                for (int ii = 0; ii < 4; ++ii) an[ii] = lds_read(lds, nbuf * kTileBytes + 4096u * ii + rd_off[nks]);
            }
            const int jj = q >> 2, pp = q & 3;
            const uint4 src = ks < 3 ? wc[jj] : wn[jj];
            const ScaleT<FAST>& scl = ks < 3 ? sc[P][jj][nks & 1] : sc[P ^ 1][jj][0];
            if (pp == 0) {
                if (nks == 0) {
                    nw[jj][0] = nib_word<0>(src, 0);
                    nw[jj][1] = nib_word<0>(src, 1);
                } else if (nks == 1) {
                    nw[jj][0] = nib_word<1>(src, 0);
                    nw[jj][1] = nib_word<1>(src, 1);
                } else if (nks == 2) {
                    nw[jj][0] = nib_word<2>(src, 0);
                    nw[jj][1] = nib_word<2>(src, 1);
                } else {
                    nw[jj][0] = nib_word<3>(src, 0);
                    nw[jj][1] = nib_word<3>(src, 1);
                }
                if constexpr (TYPE == 13) {
                    // the next slice's group: G, or G + 1 (of the next super-block when G = 3)
                    const uint4 qsrc = ks < 3 || G < 3 ? qh[jj] : qhn[jj];
                    const int grp = ks < 3 ? G : G1;
                    nw[jj][0] |= q5_high(qsrc, nks, grp, 0);
                    nw[jj][1] |= q5_high(qsrc, nks, grp, 1);
                }
            }
            bn[jj][pp] = (pp & 1) ? k_pair<TYPE, FAST, 1>(nw[jj][pp >> 1], scl) : k_pair<TYPE, FAST, 0>(nw[jj][pp >> 1], scl);
            if (ks == 0 && q < 2) {
                // quant chunks of the next step: group G + 1 of this super-block, or group 0 of the next
                const uint32_t slot = G < 3 ? wslot : wslot_next;
                wn[q] = *reinterpret_cast<const uint4*>(lds + ws_w_off(slot, (uint32_t)G1, n_lane0 + 32u * q, h));
            }
            if (G == 3 && ks == 0 && (q == 2 || q == 3)) {
                hdrn[q - 2] = *reinterpret_cast<const uint4*>(lds + ws_h_off(hslot_next, n_lane0 + 32u * (q - 2)));
            }
            if (TYPE == 13 && G == 3 && ks == 0 && (q == 4 || q == 5)) {
                qhn[q - 4] = *reinterpret_cast<const uint4*>(lds + ws_q_off(hslot_next, n_lane0 + 32u * (q - 4), h));
            }
            if (ks == 1 && q == 4) {
                if (G < 3) scale_pairs<FAST, G1>(hdr[0], sc[P ^ 1][0]);
                else scale_pairs<FAST, 0>(hdrn[0], sc[P ^ 1][0]);
            }
            if (ks == 1 && q == 6) {
                if (G < 3) scale_pairs<FAST, G1>(hdr[1], sc[P ^ 1][1]);
                else scale_pairs<FAST, 0>(hdrn[1], sc[P ^ 1][1]);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int ii = 0; ii < 4; ++ii) a[ii] = an[ii];
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int e = 0; e < 4; ++e) b[j][e] = bn[j][e];
    }
}

// producer state: activation chunk offsets (4 per lane) and LDS store offset; weight piece
// offsets (8 per lane, one per load instruction) and LDS store offsets; header row offset
struct Producer {
    uint32_t act_off[4];
    uint32_t act_st;
    uint32_t wrow_off[8];  // row * pitch of the piece's row
    uint32_t w_e[8];       // half e of the piece
    uint32_t w_st[8];      // LDS offset of the chunk within a slot
    uint32_t hrow_off;     // row * pitch of the lane's header row
};

template <uint32_t TYPE>
OQ_DEVICE void ws_load_sb(const Split& sp, const Producer& pr, uint32_t sb, int lane, uint4 (&wq)[8], uint4& hq,
                          uint4 (&qq)[2]) {
    const uint32_t pass = sb / 16u, s16 = sb % 16u;
    const uint32_t mp = sp.nsb - 16u * pass < 16u ? sp.nsb - 16u * pass : 16u;
    const uint8_t* qbase = sp.wbase + 16u * (128u * pass + 4u * s16 + (uint32_t)(lane & 3));
#pragma unroll
    for (int t = 0; t < 8; ++t) wq[t] = load_u4(qbase, pr.wrow_off[t] + pr.w_e[t] * 64u * mp);
    hq = load_u4(sp.wbase + sp.hdr_base + 16u * sb, pr.hrow_off);
    if constexpr (TYPE == 13) {
        // the high-bit plane: 32 bytes per super-block after the 128 * nsb quant bytes of the row
        const uint8_t* qh = sp.wbase + 128u * sp.nsb + 32u * sb;
        qq[0] = load_u4(qh, pr.hrow_off);
        qq[1] = load_u4(qh + 16, pr.hrow_off);
    }
}

template <uint32_t TYPE>
OQ_DEVICE void ws_store_sb(uint8_t* lds, const Producer& pr, uint32_t slot, const uint4 (&wq)[8], uint4 hq,
                           const uint4 (&qq)[2], int pw, int lane) {
#pragma unroll
    for (int t = 0; t < 8; ++t) *reinterpret_cast<uint4*>(lds + kWsA + slot * kWsWSlot + pr.w_st[t]) = wq[t];
    const uint32_t n = 64u * (uint32_t)pw + (uint32_t)lane;
    *reinterpret_cast<uint4*>(lds + ws_h_off(slot, n)) = hq;
    if constexpr (TYPE == 13) {
        *reinterpret_cast<uint4*>(lds + ws_q_off(slot, n, 0)) = qq[0];
        *reinterpret_cast<uint4*>(lds + ws_q_off(slot, n, 1)) = qq[1];
    }
}

// q4_K (TYPE 12) and q5_K (13): the same tiles, steps and k order; q5_K adds the high-bit plane
// (staged beside the headers) to each nibble word before the conversion.
template <uint32_t TYPE, bool FAST>
__global__ __launch_bounds__(kWsThreads) void gemm_ws_kernel(DeviceMatrix w, int m, const _Float16* a16,
                                                             uint32_t tiles_n, uint32_t tiles_m, uint32_t splits,
                                                             float* __restrict__ out) {
    static_assert(TYPE == 12 || TYPE == 13, "q4_K or q5_K");
    extern __shared__ __align__(16) uint8_t lds[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t nsb = (uint32_t)(w.k / kQK);
    const Unit un = unit_of(blockIdx.x, tiles_n, tiles_m, splits);
    const uint32_t z = un.z;
    const uint64_t n0 = (uint64_t)un.nt * kBN, m0 = (uint64_t)un.mt * kBM;
    Split sp;
    sp.sb0 = (uint32_t)((uint64_t)z * nsb / splits);
    const uint32_t sb1 = (uint32_t)((uint64_t)(z + 1) * nsb / splits);
    sp.nsbu = sb1 - sp.sb0;  // >= 1: splits <= nsb
    sp.nsb = nsb;
    sp.last_step = 4 * sp.nsbu - 1;
    sp.hdr_base = (TYPE == 13 ? 160u : 128u) * nsb;
    sp.wbase = w.base;
    sp.a16 = reinterpret_cast<const uint8_t*>(a16) + 2ull * kQK * sp.sb0;
    const uint32_t nsteps = 4 * sp.nsbu;

    if (wave >= 4) {
        // ------------------------------------------------------------ producer
        const int pw = wave - 4;
        Producer pr;
        const uint32_t krow = (uint32_t)(w.k * 2);
        // lane: chunk lane % 8 of rows rb + {0, 1, 16, 17} (rb even), so the four rows share the
        // tile swizzle and the four stores differ by immediates
        const uint32_t rb = 32u * pw + 2u * ((uint32_t)lane >> 3), c8 = (uint32_t)lane & 7;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            uint64_t row = m0 + rb + (uint32_t)(j & 1) + 16u * (uint32_t)(j >> 1);
            row = row < (uint64_t)m ? row : (uint64_t)m - 1;
            pr.act_off[j] = (uint32_t)row * krow + 16u * c8;
        }
        pr.act_st = 128u * rb + 16u * (c8 ^ ((rb >> 1) & 7));
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            const uint32_t piece = 16u * t + ((uint32_t)lane >> 2);  // 0..127: (row n', half e)
            const uint32_t nl = 64u * pw + (piece >> 1), e = piece & 1, g = (uint32_t)lane & 3;
            uint64_t n = n0 + nl;
            n = n < w.n ? n : w.n - 1;
            pr.wrow_off[t] = (uint32_t)(n * w.pitch);
            pr.w_e[t] = e;
            pr.w_st[t] = g * 8192u + ((32u * nl + 16u * e) ^ (64u * g));
        }
        {
            uint64_t n = n0 + 64u * pw + lane;
            n = n < w.n ? n : w.n - 1;
            pr.hrow_off = (uint32_t)(n * w.pitch);
        }
        auto act_load = [&](uint32_t t, uint4 (&v)[4]) {
            const uint32_t st = t < sp.last_step ? t : sp.last_step;
#pragma unroll
            for (int j = 0; j < 4; ++j) v[j] = load_u4(sp.a16 + 128u * st, pr.act_off[j]);
        };
        auto act_store = [&](uint32_t buf, const uint4 (&v)[4]) {
#pragma unroll
            for (int j = 0; j < 4; ++j)
                *reinterpret_cast<uint4*>(lds + buf * kTileBytes + pr.act_st + 128u * (j & 1) + 2048u * (j >> 1)) = v[j];
        };
        uint4 av[2][4], wq[8], hq, qq[2];
        // prologue: tiles 0..2, super-block 0 into slot 0; tiles 3, 4 and super-block 1 in flight
        {
            uint4 t0[4], t1[4], t2[4];
            act_load(0, t0);
            act_load(1, t1);
            act_load(2, t2);
            ws_load_sb<TYPE>(sp, pr, split_sb(sp, 0), lane, wq, hq, qq);
            act_store(0, t0);
            act_store(1, t1);
            act_store(2, t2);
            ws_store_sb<TYPE>(lds, pr, 0, wq, hq, qq, pw, lane);
        }
        // Issued in the order of a loop trip (tile of set 1, then of set 0), each group whole: the
        // compiler's wait counts at the loop head merge this path with the loop's back edge, and
        // interleaved prologue loads would leave a tile with fewer younger loads here than in the
        // loop, so that every trip would wait for the loads of the step before.
        ws_load_sb<TYPE>(sp, pr, split_sb(sp, 1), lane, wq, hq, qq);
        asm volatile("" ::: "memory");
        act_load(3, av[1]);
        asm volatile("" ::: "memory");
        act_load(4, av[0]);
        lds_barrier();
        for (uint32_t s = 0; s < nsteps; s += 4) {
            const uint32_t i = s / 4;
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int as = (g + 1) & 1;  // register set of tiles s + 3 (stored) and s + 5 (loaded)
                act_store((uint32_t)((g + 3) & 3), av[as]);
                act_load(s + g + 5, av[as]);
                if (g == 0) {
                    ws_store_sb<TYPE>(lds, pr, (i + 1) & 1, wq, hq, qq, pw, lane);
                    ws_load_sb<TYPE>(sp, pr, split_sb(sp, i + 2), lane, wq, hq, qq);
                }
                lds_barrier();
            }
        }
        return;
    }

    // ---------------------------------------------------------------- consumer
    const int h = lane >> 5, r0 = lane & 31;
    uint32_t rd_off[4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) rd_off[ks] = 128u * (uint32_t)r0 + 16u * (uint32_t)(a_chunk(ks, h) ^ ((r0 >> 1) & 7));
    const uint32_t n_lane0 = 64u * (uint32_t)wave + (uint32_t)r0;  // row of n-subtile j: + 32 j

    float16v acc[4][2] = {};
    lds_barrier();  // the producers' prologue
    uint4 wcur[2], wnext[2], hdr[2], hdrn[2], qh[2], qhn[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        wcur[j] = *reinterpret_cast<const uint4*>(lds + ws_w_off(0, 0, n_lane0 + 32u * j, h));
        hdr[j] = *reinterpret_cast<const uint4*>(lds + ws_h_off(0, n_lane0 + 32u * j));
        hdrn[j] = hdr[j];
        wnext[j] = wcur[j];
        if constexpr (TYPE == 13) qh[j] = *reinterpret_cast<const uint4*>(lds + ws_q_off(0, n_lane0 + 32u * j, h));
        else qh[j] = make_uint4(0u, 0u, 0u, 0u);
        qhn[j] = qh[j];
    }
    ScaleT<FAST> sc[2][2][2];
    scale_pairs<FAST, 0>(hdr[0], sc[0][0]);
    scale_pairs<FAST, 0>(hdr[1], sc[0][1]);
    half8 a[4];
    uint32_t b[2][4];
#pragma unroll
    for (int i = 0; i < 4; ++i) a[i] = lds_read(lds, 4096u * i + rd_off[0]);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        uint32_t w0 = nib_word<0>(wcur[j], 0), w1 = nib_word<0>(wcur[j], 1);
        if constexpr (TYPE == 13) {
            w0 |= q5_high(qh[j], 0, 0, 0);
            w1 |= q5_high(qh[j], 0, 0, 1);
        }
        b[j][0] = k_pair<TYPE, FAST, 0>(w0, sc[0][j][0]);
        b[j][1] = k_pair<TYPE, FAST, 1>(w0, sc[0][j][0]);
        b[j][2] = k_pair<TYPE, FAST, 0>(w1, sc[0][j][0]);
        b[j][3] = k_pair<TYPE, FAST, 1>(w1, sc[0][j][0]);
    }
    for (uint32_t s = 0; s < nsteps; s += 4) {
        const uint32_t i = s / 4, slot = i & 1, slot1 = (i + 1) & 1;
        ws_consumer_step<TYPE, FAST, 0>(lds, rd_off, slot, slot1, slot1, n_lane0, h, acc, a, b, wcur, wnext, hdr, hdrn,
                                        qh, qhn, sc);
        lds_barrier();
        ws_consumer_step<TYPE, FAST, 1>(lds, rd_off, slot, slot1, slot1, n_lane0, h, acc, a, b, wnext, wcur, hdr, hdrn,
                                        qh, qhn, sc);
        lds_barrier();
        ws_consumer_step<TYPE, FAST, 2>(lds, rd_off, slot, slot1, slot1, n_lane0, h, acc, a, b, wcur, wnext, hdr, hdrn,
                                        qh, qhn, sc);
        lds_barrier();
        ws_consumer_step<TYPE, FAST, 3>(lds, rd_off, slot, slot1, slot1, n_lane0, h, acc, a, b, wnext, wcur, hdr, hdrn,
                                        qh, qhn, sc);
        lds_barrier();
        hdr[0] = hdrn[0];
        hdr[1] = hdrn[1];
        qh[0] = qhn[0];
        qh[1] = qhn[1];
    }
    store_wave_tile(out + (uint64_t)z * (uint64_t)m * w.n, splits > 1 ? nullptr : row_exponents(a16, (uint64_t)m, w.k),
                    m0, (uint64_t)m, w.n, n0 + 64 * wave, h, r0, acc);
}

// ---------------------------------------------------------------- q6_K with weights in registers
//
// gemm_ws_kernel's tiles, steps, wave roles and k order for q6_K, with gemm_kq_kernel's element
// map (so the two kernels form the same operands): step G of a super-block is half G / 2 of it
// (low nibbles of the 6-bit codes for even G, high for odd), slice ks of step G is segment
// 2 (G & 1) + (ks & 1), and lane half h takes group g = 2 (G / 2) + h: both halves of its quant
// chunk, its high-bit chunk, its scale word (segments 0..3) and the block's d.  Both steps of a
// half use the same data, so the load waves stage half a super-block at a time ("half-unit" u:
// super-block u / 2, half u % 2) in a two-slot ring, and each MFMA wave reads a half-unit once,
// during the step before the half-unit's first step.
//
// LDS (dynamic, 117 KB):
//   A ring    4 x 16 KB    as gemm_ws_kernel
//   Q6 ring   2 x 26.5 KB  half-unit u in slot u % 2: quant chunk (group 2 (u % 2) + gl, half e)
//                          of row n at 4096 c + 16 ((n + 4 c) % 256), c = 2 gl + e; high-bit
//                          chunk gl at 16 KB + 4096 gl + 16 ((n + 8 gl) % 256); the two scale
//                          words at 24 KB + 8 n; d at 26 KB + 2 n (a half-wave reads 512 bytes,
//                          contiguous modulo 4 KB, of each array)
// Timing, step t = 2 u + b (b = 0, 1) of the split:
//   load waves: the activation tiles as gemm_ws_kernel; at b = 0 store half-unit u + 1 (loaded
//               at step t - 4) into slot (u + 1) % 2, whose last reader was step t - 1, and load
//               half-unit u + 3 into the same registers;
//   MFMA waves: multiply step t; at b = 1 read half-unit u + 1 from its slot (chunk half 1 at the
//               last slice, when half-unit u's chunks are no longer read).
constexpr uint32_t kQ6Slot = 27136;
constexpr uint32_t kQ6Lds = kWsA + 2 * kQ6Slot;

// chunk array c = 2 gl + e holds row n at position (n + 4 c) % 256: the load waves' stores (lanes
// 4 r + c of a 16-lane pass: rows r, arrays c) then fall on 16 distinct bank groups, and a
// half-wave's reads (32 consecutive rows of one array) stay contiguous modulo 4 KB
OQ_DEVICE uint32_t q6_ql_off(uint32_t slot, uint32_t gl, uint32_t e, uint32_t n) {
    const uint32_t c = 2u * gl + e;
    return kWsA + slot * kQ6Slot + 4096u * c + 16u * ((n + 4u * c) & 255u);
}
// (high-bit chunk array gl holds row n at (n + 8 gl) % 256, for the same reason)
OQ_DEVICE uint32_t q6_qh_off(uint32_t slot, uint32_t gl, uint32_t n) {
    return kWsA + slot * kQ6Slot + 16384u + 4096u * gl + 16u * ((n + 8u * gl) & 255u);
}
OQ_DEVICE uint32_t q6_sc_off(uint32_t slot, uint32_t n) { return kWsA + slot * kQ6Slot + 24576u + 8u * n; }
OQ_DEVICE uint32_t q6_d_off(uint32_t slot, uint32_t n) { return kWsA + slot * kQ6Slot + 26624u + 2u * n; }

// one half-unit of one weight row, as an MFMA lane holds it
struct Q6Half {
    uint4 ql[2];  // quant chunk halves e = 0, 1 of the lane's group
    uint4 qh;     // high-bit chunk of the group
    uint32_t sc;  // int8 scales of segments 0..3
    uint32_t d;   // f16 bits of the block's d
};

// what slice 0 of a half-unit needs (quant chunk half 0, high bits, scales, d), and chunk half 1
OQ_DEVICE void q6_read_head(const uint8_t* lds, uint32_t slot, uint32_t n, uint32_t h, Q6Half& r) {
    r.ql[0] = *reinterpret_cast<const uint4*>(lds + q6_ql_off(slot, h, 0, n));
    r.qh = *reinterpret_cast<const uint4*>(lds + q6_qh_off(slot, h, n));
    r.sc = *reinterpret_cast<const uint32_t*>(lds + q6_sc_off(slot, n) + 4u * h);
    r.d = *reinterpret_cast<const uint16_t*>(lds + q6_d_off(slot, n));
}
OQ_DEVICE void q6_read_ql1(const uint8_t* lds, uint32_t slot, uint32_t n, uint32_t h, Q6Half& r) {
    r.ql[1] = *reinterpret_cast<const uint4*>(lds + q6_ql_off(slot, h, 1, n));
}

// The two 4-code words and the scale of slice ks (of a step with half-parity par = G & 1) of a
// lane's half-unit: codes u = low nibble | high bits << 4 (0..63, q = u - 32), ds = d * sc as F32
OQ_DEVICE void q6_words(const Q6Half& r, int ks, int par, uint32_t (&u)[2], float& ds) {
    const int e = ks & 1, seg = 2 * par + e;
    const float d = (float)__builtin_bit_cast(_Float16, (uint16_t)(r.d & 0xFFFFu));
    ds = d * (float)(int8_t)((r.sc >> (8 * seg)) & 0xFFu);
#pragma unroll
    for (int wd = 0; wd < 2; ++wd) {
        const uint32_t lo = (dword_of(r.ql[e], 2 * (ks >> 1) + wd) >> (4 * par)) & 0x0F0F0F0Fu;
        const uint32_t hi = (dword_of(r.qh, 2 * (ks >> 1) + wd) >> (2 * seg)) & 0x03030303u;
        u[wd] = lo | (hi << 4);
    }
}

// MFMA wave, one step G: multiplies it (A of slice ks in a, B in b) while converting the next
// slice's B operands, one weight pair after each MFMA (from cur, or at the last slice of an odd
// step from nxt, the next half-unit) and, at odd G, reading the next half-unit from slot nslot
// into nxt.
template <bool FAST, int G>
OQ_DEVICE void ws6_consumer_step(const uint8_t* lds, const uint32_t (&rd_off)[4], uint32_t nslot, uint32_t n_lane0,
                                 uint32_t h, float16v (&acc)[4][2], half8 (&a)[4], uint32_t (&b)[2][4],
                                 const Q6Half (&cur)[2], Q6Half (&nxt)[2]) {
    constexpr int G1 = (G + 1) & 3;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
        const int nks = (ks + 1) & 3;
        const uint32_t nbuf = ks < 3 ? (uint32_t)G : (uint32_t)G1;
        const int npar = ks < 3 ? (G & 1) : (G1 & 1);  // half-parity of the next slice's step
        half8 an[4];
        uint32_t bn[2][4];
        uint32_t uw[2][2];
        float ds[2];
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            const int i = q >> 1, j = q & 1;
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[i], as_b_operand(b[j]), acc[i][j], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
            if (q == 0) {
#pragma unroll
                for (int ii = 0; ii < 4; ++ii) an[ii] = lds_read(lds, nbuf * kTileBytes + 4096u * ii + rd_off[nks]);
            }
            // the next half-unit: what its first slice needs at slice 0, chunk half 1 (first used
            // by the next step's slice 1) at slice 3, once this half-unit's chunks are dead
            if ((G & 1) && ks == 0 && (q == 2 || q == 3)) q6_read_head(lds, nslot, n_lane0 + 32u * (q - 2), h, nxt[q - 2]);
            if ((G & 1) && ks == 3 && (q == 1 || q == 2)) q6_read_ql1(lds, nslot, n_lane0 + 32u * (q - 1), h, nxt[q - 1]);
            const int jj = q >> 2, pp = q & 3;
            if (pp == 0) q6_words(ks == 3 && (G & 1) ? nxt[jj] : cur[jj], nks, npar, uw[jj], ds[jj]);
            bn[jj][pp] = (pp & 1) ? q6_pair<FAST, 1>(uw[jj][pp >> 1], ds[jj]) : q6_pair<FAST, 0>(uw[jj][pp >> 1], ds[jj]);
            __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int ii = 0; ii < 4; ++ii) a[ii] = an[ii];
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int e = 0; e < 4; ++e) b[j][e] = bn[j][e];
    }
}

// load waves' registers for one half-unit: quant pieces (see ws6 producer), the lane row's
// high-bit chunks, scale words and d
struct Q6Raw {
    uint4 ql[4], qh[2];  // qh[t]: chunk (lane % 2) of row 32 t + lane / 2
    uint2 sc;
    uint32_t d;
};

template <bool FAST>
__global__ __launch_bounds__(kWsThreads) void gemm_ws6_kernel(DeviceMatrix w, int m, const _Float16* a16,
                                                              uint32_t tiles_n, uint32_t tiles_m, uint32_t splits,
                                                              float* __restrict__ out) {
    extern __shared__ __align__(16) uint8_t lds[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t nsb = (uint32_t)(w.k / kQK);
    const Unit un = unit_of(blockIdx.x, tiles_n, tiles_m, splits);
    const uint32_t z = un.z;
    const uint64_t n0 = (uint64_t)un.nt * kBN, m0 = (uint64_t)un.mt * kBM;
    Split sp;
    sp.sb0 = (uint32_t)((uint64_t)z * nsb / splits);
    const uint32_t sb1 = (uint32_t)((uint64_t)(z + 1) * nsb / splits);
    sp.nsbu = sb1 - sp.sb0;  // >= 1: splits <= nsb
    sp.nsb = nsb;
    sp.last_step = 4 * sp.nsbu - 1;
    sp.hdr_base = 0;
    sp.wbase = w.base;
    sp.a16 = reinterpret_cast<const uint8_t*>(a16) + 2ull * kQK * sp.sb0;
    const uint32_t nsteps = 4 * sp.nsbu;

    if (wave >= 4) {
        // ------------------------------------------------------------ load waves
        const int pw = wave - 4;
        const uint32_t krow = (uint32_t)(w.k * 2);
        uint32_t act_off[4];
        const uint32_t rb = 32u * pw + 2u * ((uint32_t)lane >> 3), c8 = (uint32_t)lane & 7;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            uint64_t row = m0 + rb + (uint32_t)(j & 1) + 16u * (uint32_t)(j >> 1);
            row = row < (uint64_t)m ? row : (uint64_t)m - 1;
            act_off[j] = (uint32_t)row * krow + 16u * c8;
        }
        const uint32_t act_st = 128u * rb + 16u * (c8 ^ ((rb >> 1) & 7));
        auto act_load = [&](uint32_t t, uint4 (&v)[4]) {
            const uint32_t st = t < sp.last_step ? t : sp.last_step;
#pragma unroll
            for (int j = 0; j < 4; ++j) v[j] = load_u4(sp.a16 + 128u * st, act_off[j]);
        };
        auto act_store = [&](uint32_t buf, const uint4 (&v)[4]) {
#pragma unroll
            for (int j = 0; j < 4; ++j)
                *reinterpret_cast<uint4*>(lds + buf * kTileBytes + act_st + 128u * (j & 1) + 2048u * (j >> 1)) = v[j];
        };
        // quant pieces: load t takes piece 32 t + lane / 2 = (row 16 t + lane / 4, half e = lane / 2 % 2)
        // and chunk gl = lane % 2 of the half-unit's two groups: each lane pair reads 32 bytes
        uint32_t prow_off[4], pst[4], pe[4];
        const uint32_t gl = (uint32_t)lane & 1;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const uint32_t piece = 32u * t + ((uint32_t)lane >> 1);
            const uint32_t nl = 64u * pw + (piece >> 1), e = piece & 1;
            uint64_t n = n0 + nl;
            n = n < w.n ? n : w.n - 1;
            prow_off[t] = (uint32_t)(n * w.pitch);
            pe[t] = e;
            pst[t] = q6_ql_off(0, gl, e, nl) - kWsA;
        }
        const uint32_t nrow = 64u * pw + (uint32_t)lane;  // the lane's row for scales and d
        uint32_t hrow_off, qrow_off[2];
        {
            uint64_t n = n0 + nrow;
            n = n < w.n ? n : w.n - 1;
            hrow_off = (uint32_t)(n * w.pitch);
        }
        // high bits: lane pairs read a row's 32 contiguous bytes, rows 32 t + lane / 2
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            uint64_t n = n0 + 64u * pw + 32u * t + ((uint32_t)lane >> 1);
            n = n < w.n ? n : w.n - 1;
            qrow_off[t] = (uint32_t)(n * w.pitch) + 16u * gl;
        }
        auto half_load = [&](uint32_t u, Q6Raw& r) {
            const uint32_t sb = split_sb(sp, u / 2), hf = u & 1;
            const uint32_t pass = sb / 16u, s16 = sb % 16u;
            const uint32_t mp = nsb - 16u * pass < 16u ? nsb - 16u * pass : 16u;
            const uint8_t* qb = w.base + 16u * (128u * pass + 4u * s16 + 2u * hf + gl);
#pragma unroll
            for (int t = 0; t < 4; ++t) r.ql[t] = load_u4(qb, prow_off[t] + pe[t] * 64u * mp);
            const uint8_t* hb = w.base + 128u * nsb + 64u * sb + 32u * hf;
            r.qh[0] = load_u4(hb, qrow_off[0]);
            r.qh[1] = load_u4(hb, qrow_off[1]);
            r.sc = *reinterpret_cast<const uint2*>(w.base + 192u * nsb + 16u * sb + 8u * hf + hrow_off);
            r.d = *reinterpret_cast<const uint16_t*>(w.base + 208u * nsb + 2u * sb + hrow_off);
        };
        auto half_store = [&](uint32_t slot, const Q6Raw& r) {
            uint8_t* base = lds + kWsA + slot * kQ6Slot;
#pragma unroll
            for (int t = 0; t < 4; ++t) *reinterpret_cast<uint4*>(base + pst[t]) = r.ql[t];
#pragma unroll
            for (int t = 0; t < 2; ++t)
                *reinterpret_cast<uint4*>(lds + q6_qh_off(slot, gl, 64u * pw + 32u * t + ((uint32_t)lane >> 1))) = r.qh[t];
            *reinterpret_cast<uint2*>(lds + q6_sc_off(slot, nrow)) = r.sc;
            *reinterpret_cast<uint16_t*>(lds + q6_d_off(slot, nrow)) = (uint16_t)r.d;
        };
        uint4 av[2][4];
        Q6Raw hr[2];
        // prologue: tiles 0..2 and half-unit 0 stored; half-units 1 (set 1) and 2 (set 0), tiles
        // 3 and 4 in flight
        {
            uint4 t0[4], t1[4], t2[4];
            Q6Raw h0;
            act_load(0, t0);
            act_load(1, t1);
            act_load(2, t2);
            half_load(0, h0);
            act_store(0, t0);
            act_store(1, t1);
            act_store(2, t2);
            half_store(0, h0);
        }
        // (the order keeps as many younger loads behind each set as a loop trip does, so that the
        // wait counts the compiler merges at the loop head are the loop's own)
        half_load(1, hr[1]);
        asm volatile("" ::: "memory");
        act_load(3, av[1]);
        asm volatile("" ::: "memory");
        act_load(4, av[0]);
        asm volatile("" ::: "memory");
        half_load(2, hr[0]);
        lds_barrier();
        for (uint32_t s = 0; s < nsteps; s += 4) {
            const uint32_t i = s / 4;
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int as = (g + 1) & 1;
                act_store((uint32_t)((g + 3) & 3), av[as]);
                act_load(s + g + 5, av[as]);
                if (g == 0) {
                    half_store(1, hr[1]);
                    half_load(2 * i + 3, hr[1]);
                } else if (g == 2) {
                    half_store(0, hr[0]);
                    half_load(2 * i + 4, hr[0]);
                }
                lds_barrier();
            }
        }
        return;
    }

    // ---------------------------------------------------------------- MFMA waves
    const int h = lane >> 5, r0 = lane & 31;
    uint32_t rd_off[4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) rd_off[ks] = 128u * (uint32_t)r0 + 16u * (uint32_t)(a_chunk(ks, h) ^ ((r0 >> 1) & 7));
    const uint32_t n_lane0 = 64u * (uint32_t)wave + (uint32_t)r0;  // row of n-subtile j: + 32 j

    float16v acc[4][2] = {};
    lds_barrier();  // the load waves' prologue
    Q6Half cur[2], nxt[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        q6_read_head(lds, 0, n_lane0 + 32u * j, (uint32_t)h, cur[j]);
        q6_read_ql1(lds, 0, n_lane0 + 32u * j, (uint32_t)h, cur[j]);
        nxt[j] = cur[j];
    }
    half8 a[4];
    uint32_t b[2][4];
#pragma unroll
    for (int i = 0; i < 4; ++i) a[i] = lds_read(lds, 4096u * i + rd_off[0]);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        uint32_t uw[2];
        float ds;
        q6_words(cur[j], 0, 0, uw, ds);
        b[j][0] = q6_pair<FAST, 0>(uw[0], ds);
        b[j][1] = q6_pair<FAST, 1>(uw[0], ds);
        b[j][2] = q6_pair<FAST, 0>(uw[1], ds);
        b[j][3] = q6_pair<FAST, 1>(uw[1], ds);
    }
    for (uint32_t s = 0; s < nsteps; s += 4) {
        ws6_consumer_step<FAST, 0>(lds, rd_off, 1, n_lane0, h, acc, a, b, cur, nxt);
        lds_barrier();
        ws6_consumer_step<FAST, 1>(lds, rd_off, 1, n_lane0, h, acc, a, b, cur, nxt);
        lds_barrier();
        cur[0] = nxt[0];
        cur[1] = nxt[1];
        ws6_consumer_step<FAST, 2>(lds, rd_off, 0, n_lane0, h, acc, a, b, cur, nxt);
        lds_barrier();
        ws6_consumer_step<FAST, 3>(lds, rd_off, 0, n_lane0, h, acc, a, b, cur, nxt);
        lds_barrier();
        cur[0] = nxt[0];
        cur[1] = nxt[1];
    }
    store_wave_tile(out + (uint64_t)z * (uint64_t)m * w.n, splits > 1 ? nullptr : row_exponents(a16, (uint64_t)m, w.k),
                    m0, (uint64_t)m, w.n, n0 + 64 * wave, h, r0, acc);
}

// ---------------------------------------------------------------- B tiles converted by the load waves
//
// The producer/consumer workgroup with the weights converted by the load waves: every 64-k step
// the producers turn the step's quants into the f16 B tile of the MFMAs in LDS, so the MFMA waves
// only read LDS and multiply, whatever the weight type (q4_K, q5_K, q6_K).
//
// LDS (dynamic, 144 KB):
//   A ring  3 x 16 KB  activation tile of step s in buffer s % 3 (layout as above)
//   B ring  3 x 32 KB  weight tile of step s in buffer s % 3: slice ks, row n (0..255), lane half
//                      hb: the 8 f16 of the MFMA B operand at 8192 ks + 32 n + 16 hb
// Producer p: activation rows 32 p .. 32 p + 31 of each tile (four 16-byte chunks per lane) and
// weight rows 64 p .. 64 p + 63 in two passes of 32 rows; lane = 2 r + hb works on row 32 pass + r,
// operand half hb, so its four 16-byte stores per pass (one per slice) are contiguous over the
// wave.  During step s it stores activation tile s + 2 (loaded at step s - 2) and converts the
// quants of step s + 2 (loaded at step s - 2; two register sets, alternating by step) into B
// buffer (s + 2) % 3, both buffers last read at step s - 1.  The MFMA waves read the
// operands of step s + 1 during the last slice of step s (both tiles complete since the barrier
// ending step s - 1), so no LDS latency is exposed at a step boundary.  One barrier per step.
//
// Which quants make the B operand of slice ks, half hb, element i at step G of a super-block
// (k = 32 (ks & 1) + 16 hb + 8 (ks >> 1) + i within the step, the k order of a_chunk):
//   q4_K / q5_K: chunk (group G, half hb), byte 8 (ks >> 1) + i, low nibble for even ks (sub-block
//                2G), high for odd (2G + 1); q5_K's fifth bit is bit 2G + (ks & 1) of qh byte
//                16 hb + 8 (ks >> 1) + i;
//   q6_K      : chunk (group 2 (G / 2) + hb, half ks & 1), byte 8 (ks >> 1) + i, low nibble for
//                even G, high for odd; high bits from qh byte 32 (G / 2) + 16 hb + 8 (ks >> 1) + i
//                shifted by 2 seg, seg = 2 (G % 2) + (ks & 1); scale sc[8 (G / 2) + hb + 2 seg]
//                (src/model/storage_decode.cpp:96-125: element 128 half + 32 seg + lane).
constexpr uint32_t kKqThreads = 512;
constexpr uint32_t kKqBTile = 32768;
constexpr uint32_t kKqLds = 3 * kTileBytes + 3 * kKqBTile;

template <uint32_t TYPE>
struct KqRaw;
template <>
struct KqRaw<8> {
    uint4 q0[2], q1[2];  // bytes 16 hb .. 16 hb + 15 of the step's two blocks
    uint32_t d[2];       // their f16 scales
};
template <>
struct KqRaw<12> {
    uint4 q[2], hdr[2];
};
template <>
struct KqRaw<13> {
    uint4 q[2], hdr[2], qh[2];
};
template <>
struct KqRaw<14> {
    uint4 q0[2], q1[2], qh[2];
    uint32_t sc[2], d[2];
};

// quant chunk (group g, half e) of super-block sb: offset within the row
OQ_DEVICE uint32_t kq_chunk_off(uint32_t nsb, uint32_t sb, uint32_t g, uint32_t e) {
    const uint32_t pass = sb / 16u;
    const uint32_t mp = nsb - 16u * pass < 16u ? nsb - 16u * pass : 16u;
    return 16u * (128u * pass + e * 4u * mp + 4u * (sb % 16u) + g);
}

template <uint32_t TYPE, int G>
OQ_DEVICE void kq_load(KqRaw<TYPE>& r, const uint8_t* wb, const uint32_t (&row_off)[2], uint32_t nsb, uint32_t sb,
                       uint32_t hb) {
#pragma unroll
    for (int pp = 0; pp < 2; ++pp) {
        const uint8_t* row = wb + row_off[pp];
        if constexpr (TYPE == 8) {
            // step G of super-block sb: q8_0 blocks 8 sb + 2 G and 8 sb + 2 G + 1 (qs[nb][32] | d[nb])
            const uint32_t blk = 8u * sb + 2u * (uint32_t)G;
            r.q0[pp] = *reinterpret_cast<const uint4*>(row + 32u * blk + 16u * hb);
            r.q1[pp] = *reinterpret_cast<const uint4*>(row + 32u * blk + 32u + 16u * hb);
            r.d[pp] = *reinterpret_cast<const uint32_t*>(row + 256u * nsb + 2u * blk);
        } else if constexpr (TYPE == 14) {
            const uint32_t g = 2u * (G / 2) + hb;
            r.q0[pp] = *reinterpret_cast<const uint4*>(row + kq_chunk_off(nsb, sb, g, 0));
            r.q1[pp] = *reinterpret_cast<const uint4*>(row + kq_chunk_off(nsb, sb, g, 1));
            r.qh[pp] = *reinterpret_cast<const uint4*>(row + 128u * nsb + 64u * sb + 16u * g);
            r.sc[pp] = *reinterpret_cast<const uint32_t*>(row + 192u * nsb + 16u * sb + 4u * g);
            r.d[pp] = *reinterpret_cast<const uint16_t*>(row + 208u * nsb + 2u * sb);
        } else {
            r.q[pp] = *reinterpret_cast<const uint4*>(row + kq_chunk_off(nsb, sb, (uint32_t)G, hb));
            r.hdr[pp] = *reinterpret_cast<const uint4*>(row + (TYPE == 13 ? 160u : 128u) * nsb + 16u * sb);
            if constexpr (TYPE == 13) r.qh[pp] = *reinterpret_cast<const uint4*>(row + 128u * nsb + 32u * sb + 16u * hb);
        }
    }
}

// Converts the quants of one step (G) of a super-block into the four 16-byte B operand pieces of
// each pass and stores them.
template <uint32_t TYPE, bool FAST, int G>
OQ_DEVICE void kq_convert(const KqRaw<TYPE>& r, uint8_t* bdst, const uint32_t (&wr_off)[2]) {
#pragma unroll
    for (int pp = 0; pp < 2; ++pp) {
        uint32_t out[4][4];
        if constexpr (TYPE == 8) {
            // slice ks takes block ks & 1, bytes 8 (ks >> 1) .. + 7 of the lane's half
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) {
                const uint4 src = (ks & 1) ? r.q1[pp] : r.q0[pp];
                const uint32_t dh = (ks & 1) ? r.d[pp] >> 16 : r.d[pp] & 0xFFFFu;
#pragma unroll
                for (int wd = 0; wd < 2; ++wd) {
                    const uint32_t v = dword_of(src, 2 * (ks >> 1) + wd);
                    out[ks][2 * wd] = q8_pair<0>(v, dh);
                    out[ks][2 * wd + 1] = q8_pair<1>(v, dh);
                }
            }
        } else if constexpr (TYPE == 14) {
            const float d = (float)__builtin_bit_cast(_Float16, (uint16_t)(r.d[pp] & 0xFFFFu));
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) {
                const int e = ks & 1, seg = 2 * (G & 1) + e;
                const uint4 src = e ? r.q1[pp] : r.q0[pp];
                const float ds = d * (float)(int8_t)((r.sc[pp] >> (8 * seg)) & 0xFFu);
#pragma unroll
                for (int wd = 0; wd < 2; ++wd) {
                    const uint32_t lo = (dword_of(src, 2 * (ks >> 1) + wd) >> (4 * (G & 1))) & 0x0F0F0F0Fu;
                    const uint32_t hi = (dword_of(r.qh[pp], 2 * (ks >> 1) + wd) >> (2 * seg)) & 0x03030303u;
                    const uint32_t u = lo | (hi << 4);
                    out[ks][2 * wd] = q6_pair<FAST, 0>(u, ds);
                    out[ks][2 * wd + 1] = q6_pair<FAST, 1>(u, ds);
                }
            }
        } else {
            ScaleT<FAST> sc[2];
            scale_pairs<FAST, G>(r.hdr[pp], sc);
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) {
#pragma unroll
                for (int wd = 0; wd < 2; ++wd) {
                    const uint32_t dw = dword_of(r.q[pp], 2 * (ks >> 1) + wd);
                    const uint32_t nib = (ks & 1) ? (dw >> 4) & 0x0F0F0F0Fu : dw & 0x0F0F0F0Fu;
                    if constexpr (TYPE == 13) {
                        const uint32_t q = nib | q5_high(r.qh[pp], ks, G, wd);
                        out[ks][2 * wd] = q5_pair<FAST, 0>(q, sc[ks & 1]);
                        out[ks][2 * wd + 1] = q5_pair<FAST, 1>(q, sc[ks & 1]);
                    } else {
                        out[ks][2 * wd] = weight_pair<FAST, 0>(nib, sc[ks & 1]);
                        out[ks][2 * wd + 1] = weight_pair<FAST, 1>(nib, sc[ks & 1]);
                    }
                }
            }
        }
#pragma unroll
        for (int ks = 0; ks < 4; ++ks)
            *reinterpret_cast<uint4*>(bdst + 8192u * ks + wr_off[pp]) = make_uint4(out[ks][0], out[ks][1], out[ks][2], out[ks][3]);
    }
}

template <uint32_t TYPE, bool FAST>
__global__ __launch_bounds__(kKqThreads) void gemm_kq_kernel(DeviceMatrix w, int m, const _Float16* a16,
                                                             uint32_t tiles_n, uint32_t tiles_m, uint32_t splits,
                                                             float* __restrict__ out) {
    extern __shared__ __align__(16) uint8_t lds[];
    uint8_t* const bring = lds + 3 * kTileBytes;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t nsb = (uint32_t)(w.k / kQK);
    const Unit un = unit_of(blockIdx.x, tiles_n, tiles_m, splits);
    const uint32_t z = un.z;
    const uint64_t n0 = (uint64_t)un.nt * kBN, m0 = (uint64_t)un.mt * kBM;
    Split sp;
    sp.sb0 = (uint32_t)((uint64_t)z * nsb / splits);
    const uint32_t sb1 = (uint32_t)((uint64_t)(z + 1) * nsb / splits);
    sp.nsbu = sb1 - sp.sb0;  // >= 1: splits <= nsb
    sp.nsb = nsb;
    sp.last_step = 4 * sp.nsbu - 1;
    sp.hdr_base = 0;
    sp.wbase = w.base;
    sp.a16 = reinterpret_cast<const uint8_t*>(a16) + 2ull * kQK * sp.sb0;
    const uint32_t nsteps = 4 * sp.nsbu;

    if (wave >= 4) {
        // ------------------------------------------------------------ producer
        const int pw = wave - 4;
        uint32_t act_off[4];
        const uint32_t krow = (uint32_t)(w.k * 2);
        const uint32_t rb = 32u * pw + 2u * ((uint32_t)lane >> 3), c8 = (uint32_t)lane & 7;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            uint64_t row = m0 + rb + (uint32_t)(j & 1) + 16u * (uint32_t)(j >> 1);
            row = row < (uint64_t)m ? row : (uint64_t)m - 1;
            act_off[j] = (uint32_t)row * krow + 16u * c8;
        }
        const uint32_t act_st = 128u * rb + 16u * (c8 ^ ((rb >> 1) & 7));
        auto act_load = [&](uint32_t t, uint4 (&v)[4]) {
            const uint32_t st = t < sp.last_step ? t : sp.last_step;
#pragma unroll
            for (int j = 0; j < 4; ++j) v[j] = load_u4(sp.a16 + 128u * st, act_off[j]);
        };
        auto act_store = [&](uint32_t buf, const uint4 (&v)[4]) {
#pragma unroll
            for (int j = 0; j < 4; ++j)
                *reinterpret_cast<uint4*>(lds + buf * kTileBytes + act_st + 128u * (j & 1) + 2048u * (j >> 1)) = v[j];
        };
        // weight rows of the two passes, B store offsets
        const uint32_t r = (uint32_t)lane >> 1, hb = (uint32_t)lane & 1;
        uint32_t row_off[2], wr_off[2];
#pragma unroll
        for (int pp = 0; pp < 2; ++pp) {
            const uint32_t nl = 64u * pw + 32u * pp + r;
            uint64_t n = n0 + nl;
            n = n < w.n ? n : w.n - 1;
            row_off[pp] = (uint32_t)(n * w.pitch);
            wr_off[pp] = 32u * nl + 16u * hb;
        }
        KqRaw<TYPE> raw[2];
        uint4 av[2][4];
        // prologue: activation tiles 0, 1 stored, 2 and 3 in flight (sets 0, 1); quants of steps 0
        // and 1 converted into B buffers 0 and 1, those of steps 2 and 3 in flight (sets 0, 1)
        {
            uint4 t0[4], t1[4];
            act_load(0, t0);
            act_load(1, t1);
            const uint32_t sb = split_sb(sp, 0);
            kq_load<TYPE, 0>(raw[0], sp.wbase, row_off, nsb, sb, hb);
            kq_load<TYPE, 1>(raw[1], sp.wbase, row_off, nsb, sb, hb);
            act_load(2, av[0]);
            act_load(3, av[1]);
            act_store(0, t0);
            act_store(1, t1);
            kq_convert<TYPE, FAST, 0>(raw[0], bring, wr_off);
            kq_load<TYPE, 2>(raw[0], sp.wbase, row_off, nsb, sb, hb);
            kq_convert<TYPE, FAST, 1>(raw[1], bring + kKqBTile, wr_off);
            kq_load<TYPE, 3>(raw[1], sp.wbase, row_off, nsb, sb, hb);
        }
        lds_barrier();
        uint32_t buf2 = 2;  // (s + 2) % 3
        for (uint32_t s = 0; s < nsteps; s += 4) {
            const uint32_t i = s / 4;
            const uint32_t sbn = split_sb(sp, i + 1);
            // step s + g: store tile s + g + 2 (set g % 2) into buffer (s + g + 2) % 3 and load tile
            // s + g + 4 into the set; convert the quants of step s + g + 2 (set g % 2) into B
            // buffer (s + g + 2) % 3 and reload the set with step s + g + 4
            auto next_buf = [&] { buf2 = buf2 == 2 ? 0 : buf2 + 1; };
            act_store(buf2, av[0]);
            act_load(s + 4, av[0]);
            kq_convert<TYPE, FAST, 2>(raw[0], bring + buf2 * kKqBTile, wr_off);
            kq_load<TYPE, 0>(raw[0], sp.wbase, row_off, nsb, sbn, hb);
            next_buf();
            lds_barrier();
            act_store(buf2, av[1]);
            act_load(s + 5, av[1]);
            kq_convert<TYPE, FAST, 3>(raw[1], bring + buf2 * kKqBTile, wr_off);
            kq_load<TYPE, 1>(raw[1], sp.wbase, row_off, nsb, sbn, hb);
            next_buf();
            lds_barrier();
            act_store(buf2, av[0]);
            act_load(s + 6, av[0]);
            kq_convert<TYPE, FAST, 0>(raw[0], bring + buf2 * kKqBTile, wr_off);
            kq_load<TYPE, 2>(raw[0], sp.wbase, row_off, nsb, sbn, hb);
            next_buf();
            lds_barrier();
            act_store(buf2, av[1]);
            act_load(s + 7, av[1]);
            kq_convert<TYPE, FAST, 1>(raw[1], bring + buf2 * kKqBTile, wr_off);
            kq_load<TYPE, 3>(raw[1], sp.wbase, row_off, nsb, sbn, hb);
            next_buf();
            lds_barrier();
        }
        return;
    }

    // ---------------------------------------------------------------- consumer
    const int h = lane >> 5, r0 = lane & 31;
    uint32_t rd_off[4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) rd_off[ks] = 128u * (uint32_t)r0 + 16u * (uint32_t)(a_chunk(ks, h) ^ ((r0 >> 1) & 7));
    // B operand of n-subtile j: row 64 wave + 32 j + r0, half h
    const uint32_t b_off = 32u * (64u * (uint32_t)wave + (uint32_t)r0) + 16u * (uint32_t)h;
    float16v acc[4][2] = {};
    __builtin_amdgcn_s_waitcnt(0xC07F);
    __builtin_amdgcn_s_barrier();  // the producers' prologue
    half8 a[4], b[2];
#pragma unroll
    for (int i = 0; i < 4; ++i) a[i] = lds_read(lds, 4096u * i + rd_off[0]);
#pragma unroll
    for (int j = 0; j < 2; ++j) b[j] = lds_read(bring, 1024u * j + b_off);
    uint32_t buf = 0;  // s % 3
    for (uint32_t s = 0; s < nsteps; ++s) {
        const uint32_t nbuf = buf == 2 ? 0 : buf + 1;
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            // the next slice's operands (of the next step after slice 3) are requested before this
            // slice's MFMAs, which then cover their latency
            half8 an[4], bn[2];
            const uint32_t ab = (ks < 3 ? buf : nbuf) * kTileBytes, bb = (ks < 3 ? buf : nbuf) * kKqBTile;
            const int nks = (ks + 1) & 3;
#pragma unroll
            for (int i = 0; i < 4; ++i) an[i] = lds_read(lds, ab + 4096u * i + rd_off[nks]);
#pragma unroll
            for (int j = 0; j < 2; ++j) bn[j] = lds_read(bring, bb + 8192u * nks + 1024u * j + b_off);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                const int i = q >> 1, j = q & 1;
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[i], b[j], acc[i][j], 0, 0, 0);
            }
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int i = 0; i < 4; ++i) a[i] = an[i];
#pragma unroll
            for (int j = 0; j < 2; ++j) b[j] = bn[j];
        }
        // the barrier with a wait the compiler sees (the inline-asm one is opaque to its wait
        // counting, which then waits for the next step's fresh reads before its first MFMA)
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
        __builtin_amdgcn_s_barrier();
        buf = nbuf;
    }
    store_wave_tile(out + (uint64_t)z * (uint64_t)m * w.n, splits > 1 ? nullptr : row_exponents(a16, (uint64_t)m, w.k),
                    m0, (uint64_t)m, w.n, n0 + 64 * wave, h, r0, acc);
}

// y[i] = 2^-e_row * (sum over splits s, in order, of partial[s][i]); count4 = outputs / 4, n = row
// length (a multiple of 4, so the four outputs of an index share their row)
__global__ __launch_bounds__(256) void reduce_splits_kernel(const float4* __restrict__ part, uint64_t count4,
                                                            uint32_t splits, uint64_t n, const int* __restrict__ rexp,
                                                            float4* __restrict__ y) {
    const uint64_t stride = (uint64_t)gridDim.x * 256;
    for (uint64_t i = blockIdx.x * 256ull + threadIdx.x; i < count4; i += stride) {
        const int e = -rexp[4 * i / n];
        float4 s = part[i];
        for (uint32_t z = 1; z < splits; ++z) {
            const float4 p = part[(uint64_t)z * count4 + i];
            s.x += p.x;
            s.y += p.y;
            s.z += p.z;
            s.w += p.w;
        }
        y[i] = make_float4(ldexpf(s.x, e), ldexpf(s.y, e), ldexpf(s.z, e), ldexpf(s.w, e));
    }
}

// the same for rows whose length is not a multiple of 4
__global__ __launch_bounds__(256) void reduce_splits_scalar_kernel(const float* __restrict__ part, uint64_t count,
                                                                   uint32_t splits, uint64_t n,
                                                                   const int* __restrict__ rexp, float* __restrict__ y) {
    const uint64_t stride = (uint64_t)gridDim.x * 256;
    for (uint64_t i = blockIdx.x * 256ull + threadIdx.x; i < count; i += stride) {
        float s = part[i];
        for (uint32_t z = 1; z < splits; ++z) s += part[(uint64_t)z * count + i];
        y[i] = ldexpf(s, -rexp[i / n]);
    }
}

// Scratch of one call: the F16 image [m][K] (image_bytes), the row exponents [tiles_m * kBM] (int),
// then the split partials [splits][m][n] (F32) when splits > 1.
struct Plan {
    uint32_t tiles_n, tiles_m, splits;
    uint64_t a16_bytes, rexp_bytes, part_bytes;
};

uint64_t round256(uint64_t v) { return (v + 255) & ~uint64_t(255); }

Plan make_plan(const DeviceMatrix& w, int m) {
    Plan p;
    p.tiles_n = (uint32_t)((w.n + kBN - 1) / kBN);
    p.tiles_m = (uint32_t)((m + kBM - 1) / kBM);
    const uint64_t tiles = (uint64_t)p.tiles_n * p.tiles_m;
    const uint32_t nsb = (uint32_t)(w.k / kQK);
    uint64_t s = ((uint64_t)cu_count() + tiles / 2) / tiles;
    int forced = knob(kGemmSplits, 0);
    if (forced > 0) s = (uint64_t)forced;
    if (s < 1) s = 1;
    if (s > kMaxSplits) s = kMaxSplits;
    if (s > nsb) s = nsb;
    p.splits = (uint32_t)s;
    p.a16_bytes = round256((uint64_t)m * w.k * 2);
    p.rexp_bytes = round256((uint64_t)p.tiles_m * kBM * 4);
    p.part_bytes = p.splits > 1 ? (uint64_t)p.splits * m * w.n * 4 : 0;
    return p;
}

}  // namespace

bool gemm_mfma_supported(const DeviceMatrix& w, int m) {
    // rows shorter than kMinK stay on the integer paths: their f16 rounding errors average over fewer
    // products (OQ_GEMM_MIN_K lowers the limit for measurement)
    const uint64_t min_k = (uint64_t)std::max(knob(kGemmMinK, (int)kMinK), (int)kQK);
    return (w.type == 8 || w.type == 12 || w.type == 13 || w.type == 14) && m >= 16 && w.k >= min_k && w.k % kQK == 0;
}

uint64_t gemm_scratch_bytes(const DeviceMatrix& w, int m) {
    const Plan p = make_plan(w, m);
    return p.a16_bytes + p.rexp_bytes + p.part_bytes;
}

template <uint32_t TYPE, bool FAST>
void launch_kq(const DeviceMatrix& w, int m, const _Float16* a16, const Plan& p, float* dst, hipStream_t s) {
    // once per process (a function-local static: thread-safe)
    static const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void*>(gemm_kq_kernel<TYPE, FAST>),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, (int)kKqLds);
    (void)attr;
    hipLaunchKernelGGL((gemm_kq_kernel<TYPE, FAST>), dim3(p.tiles_n * p.tiles_m * p.splits), dim3(kKqThreads), kKqLds, s,
                       w, m, a16, p.tiles_n, p.tiles_m, p.splits, dst);
}

template <uint32_t TYPE, bool FAST>
void launch_ws(const DeviceMatrix& w, int m, const _Float16* a16, const Plan& p, float* dst, hipStream_t s) {
    // once per process (a function-local static: thread-safe)
    static const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void*>(gemm_ws_kernel<TYPE, FAST>),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, (int)ws_lds_bytes<TYPE>());
    (void)attr;
    hipLaunchKernelGGL((gemm_ws_kernel<TYPE, FAST>), dim3(p.tiles_n * p.tiles_m * p.splits), dim3(kWsThreads),
                       ws_lds_bytes<TYPE>(), s, w, m, a16, p.tiles_n, p.tiles_m, p.splits, dst);
}

template <bool FAST>
void launch_ws6(const DeviceMatrix& w, int m, const _Float16* a16, const Plan& p, float* dst, hipStream_t s) {
    // once per process (a function-local static: thread-safe)
    static const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void*>(gemm_ws6_kernel<FAST>),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, (int)kQ6Lds);
    (void)attr;
    hipLaunchKernelGGL((gemm_ws6_kernel<FAST>), dim3(p.tiles_n * p.tiles_m * p.splits), dim3(kWsThreads), kQ6Lds, s,
                       w, m, a16, p.tiles_n, p.tiles_m, p.splits, dst);
}

hipError_t launch_gemm_mfma(const DeviceMatrix& w, int m, const float* x, const uint8_t* q8k, float* y,
                                void* scratch, hipStream_t s) {
    if (!gemm_mfma_supported(w, m) || (x == nullptr) == (q8k == nullptr)) return hipErrorNotSupported;
    const Plan p = make_plan(w, m);
    uint8_t* base = static_cast<uint8_t*>(scratch);
    _Float16* a16 = reinterpret_cast<_Float16*>(base);
    int* rexp = reinterpret_cast<int*>(base + p.a16_bytes);  // = row_exponents(a16, m, K)
    float* part = reinterpret_cast<float*>(base + p.a16_bytes + p.rexp_bytes);
    const uint32_t nb = (uint32_t)(w.k / kQK);
    if (w.type == 8) {
        // q8_0: the F32 activations themselves (no Q8_K), weights converted by the load waves
        if (!x) return hipErrorNotSupported;
        hipLaunchKernelGGL(scale_f16_kernel, dim3((unsigned)m), dim3(64 * kRowWaves), 0, s, x, nb, a16, rexp);
        launch_kq<8, true>(w, m, a16, p, p.splits > 1 ? part : y, s);
    } else if (x) {
        hipLaunchKernelGGL(quantize_f16_kernel, dim3((unsigned)m), dim3(64 * kRowWaves), 0, s, x, nb, a16, rexp);
    } else {
        hipLaunchKernelGGL(q8k_to_f16_kernel, dim3((unsigned)m), dim3(64 * kRowWaves), 0, s, q8k, nb, a16, rexp);
    }
    const unsigned wgs = p.tiles_n * p.tiles_m * p.splits;
    const bool fast = w.k >= kFastMinK && knob(kGemmFastDequant, 0) != 0;
    if (w.type == 8) {
        // launched above
    } else if (knob(kGemmWs, 1) == 2) {
        // the weights converted by the load waves (every type with OQ_GEMM_WS=2)
        float* dst = p.splits > 1 ? part : y;
        if (w.type == 12) fast ? launch_kq<12, true>(w, m, a16, p, dst, s) : launch_kq<12, false>(w, m, a16, p, dst, s);
        else if (w.type == 13) fast ? launch_kq<13, true>(w, m, a16, p, dst, s) : launch_kq<13, false>(w, m, a16, p, dst, s);
        else fast ? launch_kq<14, true>(w, m, a16, p, dst, s) : launch_kq<14, false>(w, m, a16, p, dst, s);
    } else if (w.type == 14) {
        float* dst = p.splits > 1 ? part : y;
        fast ? launch_ws6<true>(w, m, a16, p, dst, s) : launch_ws6<false>(w, m, a16, p, dst, s);
    } else if (knob(kGemmWs, 1) != 0 || w.type == 13) {
        float* dst = p.splits > 1 ? part : y;
        if (w.type == 13) fast ? launch_ws<13, true>(w, m, a16, p, dst, s) : launch_ws<13, false>(w, m, a16, p, dst, s);
        else fast ? launch_ws<12, true>(w, m, a16, p, dst, s) : launch_ws<12, false>(w, m, a16, p, dst, s);
    } else if (fast) {
        hipLaunchKernelGGL(gemm_q4k_f16_kernel<true>, dim3(wgs), dim3(kThreads), 0, s, w, m, a16, p.tiles_n,
                           p.tiles_m, p.splits, p.splits > 1 ? part : y);
    } else {
        hipLaunchKernelGGL(gemm_q4k_f16_kernel<false>, dim3(wgs), dim3(kThreads), 0, s, w, m, a16, p.tiles_n,
                           p.tiles_m, p.splits, p.splits > 1 ? part : y);
    }
    if (p.splits > 1) {
        const uint64_t count = (uint64_t)m * w.n;
        if (w.n % 4 == 0) {
            uint64_t blocks = (count / 4 + 255) / 256;
            if (blocks > 8192) blocks = 8192;
            hipLaunchKernelGGL(reduce_splits_kernel, dim3((unsigned)blocks), dim3(256), 0, s,
                               reinterpret_cast<const float4*>(part), count / 4, p.splits, w.n, rexp,
                               reinterpret_cast<float4*>(y));
        } else {
            uint64_t blocks = (count + 255) / 256;
            if (blocks > 8192) blocks = 8192;
            hipLaunchKernelGGL(reduce_splits_scalar_kernel, dim3((unsigned)blocks), dim3(256), 0, s, part, count,
                               p.splits, w.n, rexp, y);
        }
    }
    return hipGetLastError();
}

}  // namespace oq
