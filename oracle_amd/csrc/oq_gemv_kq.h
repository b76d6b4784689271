// Decode GEMV and small-batch products (m <= 8) for K-quant weights (q4_K, q5_K, q6_K) against
// Q8_K activations.
//
// y[m][n] = sum_k W[n][k] * x[m][k]; arithmetic as GGML's vec_dot_qX_K_q8_K: int8 dot products of
// the weight quants with the Q8_K activation quants, block scales applied in F32 (reference
// semantics: reference_storage_matvec, src/backend/cpu/quantized_reference.cpp:128-162, applied to
// each activation row as the reference's multi-token evaluation does).
//
// Weights stream from the permuted row planes of oq_layout.h: in pass P (16 super-blocks) lane
// l = 4*s + q loads chunks 128P + l and 128P + 4m + l -- every load instruction of the wave reads
// 1 KiB of consecutive bytes -- and gets, for q4_K/q5_K, both halves of 64-element group q of
// super-block s (one header / scale unpack per 64 weights), for q6_K the low and high segments
// sharing one 16-byte high-bit chunk and four scales.
//
// Activations: each workgroup stages the Q8_K form of its m rows once in LDS, quantizing F32 x
// itself (one wave per 256-block, DPP reductions; bit-identical to quantize_q8k_kernel) or copying
// Q8_K blocks.  For m = 1 every lane then keeps its 64 quants, scale and 16-element sums in
// registers (its slot is the same in every row); for m > 1 they are read from LDS per use, so each
// weight byte is decoded once for all m rows.  Weight loads for the first rows are issued before
// the staging completes.  Row sums: DPP row reductions + readlane in a fixed order.
//
// This header holds the kernels and their launch templates; oq_gemv_inst.hip instantiates them
// once per (weight type, activation form), oq_gemv_block.hip builds the DeltaNet block kernels
// on them and oq_gemv_kq.hip dispatches.
#pragma once

#include "oq_common.h"
#include "oq_layout.h"

namespace oq {

namespace kq {

// Internal linkage: every translation unit that includes this header gets its own copies of the
// instantiations it uses.
namespace {

constexpr int kMaxIters = 4;  // passes of 16 super-blocks held by the compile-time kernels (K <= 16384)
constexpr uint64_t kLdsBudget = 64 * 1024;
// The small-batch streamed kernel runs one 16-wave workgroup per CU, so its activation image may
// take most of the CU's 160 KB: eight rows of 12288 (124 KB) in one launch.  q5_K, and every type
// with OQ_GEMV_STREAM_MT=0, keep the general budget (those rows run the batched kernel, whose
// workgroups share a CU).
constexpr uint64_t kMtLdsBudget = 128 * 1024;
uint64_t mt_lds_budget(uint32_t type) {
    return type == 13 || knob(kGemvStreamMt, 1) == 0 ? kLdsBudget : kMtLdsBudget;
}

OQ_DEVICE uint4 ldg128(const uint8_t* p) { return *reinterpret_cast<const uint4*>(p); }
OQ_DEVICE uint32_t ldg32(const uint8_t* p) { return *reinterpret_cast<const uint32_t*>(p); }
// weight loads (read once per launch: non-temporal, see load_stream)
OQ_DEVICE uint4 ldg128_stream(const uint8_t* p) { return load_stream(reinterpret_cast<const uint4*>(p)); }
OQ_DEVICE uint32_t ldg32_stream(const uint8_t* p) { return load_stream(reinterpret_cast<const uint32_t*>(p)); }
OQ_DEVICE int dot4(uint32_t a, uint32_t b, int c) { return __builtin_amdgcn_sdot4((int)a, (int)b, c, false); }
OQ_DEVICE float h2f(uint32_t bits16) { return (float)__builtin_bit_cast(_Float16, (uint16_t)bits16); }


// ---------------------------------------------------------------- LDS image of activation rows

// per row: q8[K] | d[K/256] | bsum[K/16] (int32)
struct ActLds {
    uint8_t* base;
    uint64_t k;
    OQ_DEVICE uint64_t stride() const { return k + (k / kQK) * 4 + (k / 16) * 4; }
    OQ_DEVICE int8_t* q(int mi) const { return reinterpret_cast<int8_t*>(base + mi * stride()); }
    OQ_DEVICE float* d(int mi) const { return reinterpret_cast<float*>(base + mi * stride() + k); }
    OQ_DEVICE int* bsum(int mi) const {
        return reinterpret_cast<int*>(base + mi * stride() + k + (k / kQK) * 4);
    }
};
uint64_t act_lds_bytes(uint64_t k, int m) { return (uint64_t)m * (k + (k / kQK) * 4 + (k / 16) * 4); }

// GGML quantize_row_q8_K of one 256-block held by a wave (lane: values 4l..4l+3): the lane's 4
// quants, the 16-element sum of its quad (valid in every lane of the quad) and d.
OQ_DEVICE void quantize_block(const float4 v, int lane, uint32_t& qword, int& bsum, float& d) {
    const Q8KLane r = quantize_q8k_block_wave(v, lane);
    qword = r.qword;
    bsum = r.quad_bsum;
    d = r.d;
}

// The 16 sixteen-byte chunks of a staged 256-block are stored in permuted order: chunk c of
// block b sits at c ^ swz(b).  The lanes that read one piece each (4 per block, 16 blocks per
// wave) then hit 16 different chunk positions in every group of 16 lanes instead of 4 (the
// pieces of one lane slot are 64 bytes apart for q4_K/q5_K, 128 + 16 for q6_K): no bank
// conflicts when the small-batch kernels re-read the slices for every activation row.
template <uint32_t TYPE>
OQ_DEVICE uint32_t swz(uint64_t b) {
    return TYPE == 14 ? ((uint32_t)b & 3u) << 1 : ((uint32_t)b & 3u);
}

template <uint32_t TYPE>
OQ_DEVICE uint32_t stage_off(uint64_t b, int lane) {
    return 16u * (((uint32_t)lane >> 2) ^ swz<TYPE>(b)) + 4u * ((uint32_t)lane & 3u);
}

template <uint32_t TYPE>
OQ_DEVICE void store_block(const ActLds& s, int mi, uint64_t b, int lane, uint32_t qword, int bsum16_quad,
                           float d) {
    *reinterpret_cast<uint32_t*>(s.q(mi) + b * kQK + stage_off<TYPE>(b, lane)) = qword;
    if ((lane & 3) == 0) s.bsum(mi)[b * 16 + (lane >> 2)] = bsum16_quad;
    if (lane == 0) s.d(mi)[b] = d;
}

// Q8_K block copy: lane's quant dword, d, and bsums 2*(lane%8), +1 in one dword
template <uint32_t TYPE>
OQ_DEVICE void copy_block_store(const ActLds& s, int mi, uint64_t b, int lane, uint32_t qword, uint32_t bsdw,
                                float d) {
    *reinterpret_cast<uint32_t*>(s.q(mi) + b * kQK + stage_off<TYPE>(b, lane)) = qword;
    if (lane < 8) {
        s.bsum(mi)[b * 16 + 2 * lane] = (int)(int16_t)(bsdw & 0xFFFFu);
        s.bsum(mi)[b * 16 + 2 * lane + 1] = (int)(int16_t)(bsdw >> 16);
    }
    if (lane == 0) s.d(mi)[b] = d;
}

// ---------------------------------------------------------------- per-lane activation slice

struct Act {
    uint4 x0, x1, x2, x3;  // 64 quants (4 pieces of 16; see piece offsets)
    float d;
    int b[4];              // 16-element sums of the 4 pieces
};

// element offset (within the 256-block) of piece i of lane slot q
template <uint32_t TYPE>
OQ_DEVICE int piece(int q, int i) {
    if constexpr (TYPE == 14) return 128 * (q >> 1) + 16 * (q & 1) + 32 * i;
    else return 64 * q + 16 * i;
}

template <uint32_t TYPE>
OQ_DEVICE void slice_from_lds(Act& a, const ActLds& s, int mi, uint64_t sb, int q) {
    const int8_t* qb = s.q(mi) + sb * kQK;
    const uint32_t z = swz<TYPE>(sb);
    a.x0 = *reinterpret_cast<const uint4*>(qb + 16 * ((piece<TYPE>(q, 0) / 16) ^ z));
    a.x1 = *reinterpret_cast<const uint4*>(qb + 16 * ((piece<TYPE>(q, 1) / 16) ^ z));
    a.x2 = *reinterpret_cast<const uint4*>(qb + 16 * ((piece<TYPE>(q, 2) / 16) ^ z));
    a.x3 = *reinterpret_cast<const uint4*>(qb + 16 * ((piece<TYPE>(q, 3) / 16) ^ z));
    a.d = s.d(mi)[sb];
    const int* bs = s.bsum(mi) + sb * 16;
#pragma unroll
    for (int i = 0; i < 4; ++i) a.b[i] = bs[piece<TYPE>(q, i) / 16];
}

// ---------------------------------------------------------------- weights

struct W45 {
    uint4 c0, c1, hdr;  // quant chunks e = 0, 1 of the lane's 64-element group; block header
    uint4 h0, h1;       // q5_K: fifth-bit bytes l = 0..15, 16..31
};
struct W6 {
    uint4 c0, c1, qh;  // ql chunks (segment parity 0, 1), high-bit chunk
    uint32_t sc;       // four scales (segments 0..3)
    uint32_t d;
};
template <uint32_t TYPE>
struct WRegs {
    using type = W45;
};
template <>
struct WRegs<14> {
    using type = W6;
};

// Offsets are 32-bit (a row is far below 4 GiB) so the loads use a scalar row base plus a
// per-lane 32-bit offset.
template <uint32_t TYPE>
OQ_DEVICE void load_w(typename WRegs<TYPE>::type& r, const uint8_t* row, uint32_t nsb, int it, int lane) {
    const uint32_t m = nsb - 16u * it < 16u ? nsb - 16u * it : 16u;
    const uint32_t l = (uint32_t)lane < 4 * m ? (uint32_t)lane : 4 * m - 1;  // surplus lanes re-read
    const uint32_t sb = 16u * it + (l >> 2);
    const uint32_t q = l & 3;
    r.c0 = ldg128_stream(row + 16u * (128u * it + l));
    r.c1 = ldg128_stream(row + 16u * (128u * it + 4u * m + l));
    if constexpr (TYPE == 14) {
        r.qh = ldg128_stream(row + (128u * nsb + 64u * sb + 16u * q));
        r.sc = ldg32_stream(row + (192u * nsb + 16u * sb + 4u * q));
        r.d = *reinterpret_cast<const uint16_t*>(row + (208u * nsb + 2u * sb));
    } else {
        r.hdr = ldg128_stream(row + ((TYPE == 13 ? 160u : 128u) * nsb + 16u * sb));
        if constexpr (TYPE == 13) {
            r.h0 = ldg128_stream(row + (128u * nsb + 32u * sb));
            r.h1 = ldg128_stream(row + (128u * nsb + 32u * sb + 16u));
        }
    }
}

// decoded, m-independent part of a lane's 64 weights
struct Dec45 {
    uint32_t lo[8], hi[8];  // 4-bit (5-bit) quants: lo pairs with pieces 0,1; hi with 2,3
    float d, dmin;
    int sc0, sc1, mn0, mn1;
};
struct Dec6 {
    uint32_t s[4][4];  // 6-bit unsigned quants of segments 0..3
    float d;
    int sc[4];
};

// Lane-constant masks and shifts that pick, without branches, the (scale, min) byte-vector
// holding the lane's sub-blocks 2q, 2q+1 out of GGML's 12-byte K-quant packing:
//   pairs 0..3: scales = p0 & 0x3f.., mins = p1 & 0x3f..
//   pairs 4..7: scales = (p2 & 0x0f..) | ((p0 >> 2) & 0x30..), mins = ((p2 >> 4) & 0x0f..) | ((p1 >> 2) & 0x30..)
struct ScaleSel {
    uint32_t mask_a, mask_b;  // applied to p0/p1 (shifted) and to p2 (shifted)
    int sh_a, sh_b, sh_pair;  // p0/p1 shift, p2 shift for the mins, byte offset of the pair
};
OQ_DEVICE ScaleSel scale_sel(int q) {
    const bool low = q < 2;
    return {low ? 0x3F3F3F3Fu : 0x30303030u, low ? 0u : 0x0F0F0F0Fu, low ? 0 : 2, low ? 0 : 4, 16 * (q & 1)};
}

template <uint32_t TYPE>
OQ_DEVICE Dec45 decode_w(const W45& r, const ScaleSel& ss, int q) {
    Dec45 o;
    o.d = h2f(r.hdr.x & 0xFFFFu);
    o.dmin = h2f(r.hdr.x >> 16);
    const uint32_t p0 = r.hdr.y, p1 = r.hdr.z, p2 = r.hdr.w;
    const uint32_t scw = ((p0 >> ss.sh_a) & ss.mask_a) | (p2 & ss.mask_b);
    const uint32_t mnw = ((p1 >> ss.sh_a) & ss.mask_a) | ((p2 >> ss.sh_b) & ss.mask_b);
    const int sh = ss.sh_pair;
    o.sc0 = (int)((scw >> sh) & 0xFFu);
    o.sc1 = (int)((scw >> (sh + 8)) & 0xFFu);
    o.mn0 = (int)((mnw >> sh) & 0xFFu);
    o.mn1 = (int)((mnw >> (sh + 8)) & 0xFFu);
    const uint32_t w[8] = {r.c0.x, r.c0.y, r.c0.z, r.c0.w, r.c1.x, r.c1.y, r.c1.z, r.c1.w};
    const uint32_t hb[8] = {r.h0.x, r.h0.y, r.h0.z, r.h0.w, r.h1.x, r.h1.y, r.h1.z, r.h1.w};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        o.lo[i] = w[i] & 0x0F0F0F0Fu;
        o.hi[i] = (w[i] >> 4) & 0x0F0F0F0Fu;
        if constexpr (TYPE == 13) {
            o.lo[i] |= ((hb[i] >> (2 * q)) & 0x01010101u) << 4;
            o.hi[i] |= ((hb[i] >> (2 * q + 1)) & 0x01010101u) << 4;
        }
    }
    return o;
}

template <uint32_t TYPE>
OQ_DEVICE Dec6 decode_w(const W6& r, const ScaleSel&, int) {
    Dec6 o;
    o.d = h2f(r.d);
    const uint32_t c0[4] = {r.c0.x, r.c0.y, r.c0.z, r.c0.w};
    const uint32_t c1[4] = {r.c1.x, r.c1.y, r.c1.z, r.c1.w};
    const uint32_t h[4] = {r.qh.x, r.qh.y, r.qh.z, r.qh.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        o.s[0][i] = (c0[i] & 0x0F0F0F0Fu) | ((h[i] << 4) & 0x30303030u);
        o.s[1][i] = (c1[i] & 0x0F0F0F0Fu) | ((h[i] << 2) & 0x30303030u);
        o.s[2][i] = ((c0[i] >> 4) & 0x0F0F0F0Fu) | (h[i] & 0x30303030u);
        o.s[3][i] = ((c1[i] >> 4) & 0x0F0F0F0Fu) | ((h[i] >> 2) & 0x30303030u);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) o.sc[i] = (int)(int8_t)(r.sc >> (8 * i));
    return o;
}

OQ_DEVICE int dot16(const uint32_t* w, const uint4 x, int acc) {
    acc = dot4(w[0], x.x, acc);
    acc = dot4(w[1], x.y, acc);
    acc = dot4(w[2], x.z, acc);
    acc = dot4(w[3], x.w, acc);
    return acc;
}

// A lane's share of one pass: the activation block's scale times lane_inner, accumulated as one
// fused multiply-add (lane_fma) in every kernel, so that kernels splitting the passes of a row
// differently give the same bits.
OQ_DEVICE float lane_inner(const Dec45& w, const Act& a) {
    int slo = dot16(w.lo, a.x0, 0);
    slo = dot16(w.lo + 4, a.x1, slo);
    int shi = dot16(w.hi, a.x2, 0);
    shi = dot16(w.hi + 4, a.x3, shi);
    // all factors fit in 24 bits (|slo| <= 32*31*127, scales <= 63, |bsum| <= 16*127): full-rate
    // 24-bit multiplies are exact here
    const int isum = __mul24(w.sc0, slo) + __mul24(w.sc1, shi);
    const int imin = __mul24(w.mn0, a.b[0] + a.b[1]) + __mul24(w.mn1, a.b[2] + a.b[3]);
    return w.d * (float)isum - w.dmin * (float)imin;
}

OQ_DEVICE float lane_inner(const Dec6& w, const Act& a) {
    const int p0 = dot16(w.s[0], a.x0, 0) - 32 * a.b[0];
    const int p1 = dot16(w.s[1], a.x1, 0) - 32 * a.b[1];
    const int p2 = dot16(w.s[2], a.x2, 0) - 32 * a.b[2];
    const int p3 = dot16(w.s[3], a.x3, 0) - 32 * a.b[3];
    // |p_i| <= 16*63*127 + 32*16*127, |sc| <= 128: exact in 24-bit multiplies
    const int isum = __mul24(w.sc[0], p0) + __mul24(w.sc[1], p1) + __mul24(w.sc[2], p2) + __mul24(w.sc[3], p3);
    return w.d * (float)isum;
}

template <typename Dec>
OQ_DEVICE float lane_fma(const Dec& w, const Act& a, float acc) {
    return __builtin_fmaf(a.d, lane_inner(w, a), acc);
}

// ---------------------------------------------------------------- kernel

template <uint32_t TYPE, int ITERS, int R>
OQ_DEVICE void load_group(typename WRegs<TYPE>::type (&W)[R][ITERS], const DeviceMatrix& w, uint64_t grp,
                          int lane) {
    const uint32_t nsb = (uint32_t)(w.k / kQK);
#pragma unroll
    for (int r = 0; r < R; ++r) {
        uint64_t row = grp * R + r;
        row = row < w.n ? row : w.n - 1;
        // the row index is wave-uniform: keep it (and the row address) in scalar registers
        const uint32_t row_s = __builtin_amdgcn_readfirstlane((uint32_t)row);
        const uint8_t* base = w.base + (uint64_t)row_s * w.pitch;
#pragma unroll
        for (int it = 0; it < ITERS; ++it) load_w<TYPE>(W[r][it], base, nsb, it, lane);
    }
}

template <uint32_t TYPE, int ITERS, int R, int MT, bool FULL>
OQ_DEVICE void finish_group(const typename WRegs<TYPE>::type (&W)[R][ITERS], const Act (&act)[ITERS],
                            const ActLds& s, int m, const DeviceMatrix& w, uint64_t grp, int lane, float* y) {
    const uint64_t nsb = w.k / kQK;
    const int q = lane & 3;
    const ScaleSel ss = scale_sel(q);
    float acc[R][MT];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int mi = 0; mi < MT; ++mi) acc[r][mi] = 0.0f;
#pragma unroll
    for (int it = 0; it < ITERS; ++it) {
        const uint64_t sb = 16u * it + (lane >> 2);
        if (!FULL && sb >= nsb) continue;  // FULL: K is a multiple of 4096, every lane has a slot
        if constexpr (MT == 1) {
#pragma unroll
            for (int r = 0; r < R; ++r) acc[r][0] = lane_fma(decode_w<TYPE>(W[r][it], ss, q), act[it], acc[r][0]);
        } else {
            // each activation slice is read from LDS once for the R rows
            decltype(decode_w<TYPE>(W[0][it], ss, q)) dec[R];
#pragma unroll
            for (int r = 0; r < R; ++r) dec[r] = decode_w<TYPE>(W[r][it], ss, q);
#pragma unroll
            for (int mi = 0; mi < MT; ++mi) {
                if (mi < m) {
                    Act a;
                    slice_from_lds<TYPE>(a, s, mi, sb, q);
#pragma unroll
                    for (int r = 0; r < R; ++r) acc[r][mi] = lane_fma(dec[r], a, acc[r][mi]);
                }
            }
        }
    }
#pragma unroll
    for (int mi = 0; mi < MT; ++mi) {
        if (mi >= m) break;
        float out = 0.0f;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const float v = wave_sum_uniform(acc[r][mi]);
            out = lane == r ? v : out;
        }
        const uint64_t row = grp * R + lane;
        if (lane < R && row < w.n) y[(uint64_t)mi * w.n + row] = out;
    }
}

// Stages the Q8_K form of one activation row in LDS (quantizing F32 x, or copying Q8_K blocks),
// wave w taking blocks w, w + WAVES, ...  The activation loads go out first (unconditional,
// clamped) so that the waits before quantizing count only them; x and q8k are deliberately not
// __restrict__, so the fence keeps them ahead of the weight loads that issue() starts, which then
// stay in flight through the staging.
template <uint32_t TYPE, int ITERS, bool FUSED, int WAVES, typename Issue>
OQ_DEVICE void stage_one_row(const ActLds& s, const float* x, const uint8_t* q8k, uint64_t nsb, int wave_in_wg,
                             int lane, Issue&& issue) {
    constexpr int SBW = (ITERS * 16 + WAVES - 1) / WAVES;
    float4 xv[SBW];
    uint32_t qv[SBW], bv[SBW];
    float dv[SBW];
#pragma unroll
    for (int j = 0; j < SBW; ++j) {
        uint64_t b = (uint64_t)wave_in_wg + (uint64_t)WAVES * j;
        b = b < nsb ? b : nsb - 1;
        if constexpr (FUSED) {
            xv[j] = reinterpret_cast<const float4*>(x + b * kQK)[lane];
        } else {
            const uint8_t* blk = q8k + b * kQ8KBytes;
            qv[j] = ldg32(blk + 4 + 4 * lane);
            bv[j] = ldg32(blk + 260 + 4 * (lane & 7));
            dv[j] = __uint_as_float(ldg32(blk));
        }
    }
    asm volatile("" ::: "memory");
    issue();
#pragma unroll
    for (int j = 0; j < SBW; ++j) {
        const uint64_t b = (uint64_t)wave_in_wg + (uint64_t)WAVES * j;
        if (b >= nsb) break;
        if constexpr (FUSED) {
            uint32_t qw;
            int bs;
            float d;
            quantize_block(xv[j], lane, qw, bs, d);
            store_block<TYPE>(s, 0, b, lane, qw, bs, d);
        } else {
            copy_block_store<TYPE>(s, 0, b, lane, qv[j], bv[j], dv[j]);
        }
    }
}

template <uint32_t TYPE, int ITERS, int R, int MT, bool FUSED, int WAVES, bool FULL>
__global__ __launch_bounds__(64 * WAVES) void gemv_kq_kernel(DeviceMatrix w, int m, const float* x,
                                                             const uint8_t* q8k, float* __restrict__ y) {
    using WR = typename WRegs<TYPE>::type;
    extern __shared__ __align__(16) uint8_t smem[];
    const int lane = threadIdx.x & 63;
    const int wave_in_wg = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform (scalar)
    const uint64_t wave = (uint64_t)blockIdx.x * WAVES + wave_in_wg;
    const uint64_t nw = (uint64_t)gridDim.x * WAVES;
    const uint64_t nsb = w.k / kQK;
    const uint64_t groups = (w.n + R - 1) / R;
    const ActLds s{smem, w.k};
    const bool active = wave < groups;
    WR A[R][ITERS];

    if constexpr (MT == 1) {
        stage_one_row<TYPE, ITERS, FUSED, WAVES>(s, x, q8k, nsb, wave_in_wg, lane,
                                                 [&] { load_group<TYPE, ITERS, R>(A, w, active ? wave : groups - 1, lane); });
    } else {
        // m rows: the wave's blocks are staged U at a time (their loads issued together); the
        // first batch goes out before the weight loads so that its wait does not include them
        constexpr int U = 4;
        const uint64_t nblk = (uint64_t)m * nsb;
        float4 xv[U];
        uint32_t qv[U], bv[U];
        float dv[U];
        auto load_batch = [&](uint64_t b0) {
#pragma unroll
            for (int u = 0; u < U; ++u) {
                uint64_t b = b0 + (uint64_t)WAVES * u;
                b = b < nblk ? b : nblk - 1;
                if constexpr (FUSED) {
                    const uint64_t mi = b / nsb, sb = b % nsb;
                    xv[u] = reinterpret_cast<const float4*>(x + mi * w.k + sb * kQK)[lane];
                } else {
                    const uint8_t* blk = q8k + b * kQ8KBytes;
                    qv[u] = ldg32(blk + 4 + 4 * lane);
                    bv[u] = ldg32(blk + 260 + 4 * (lane & 7));
                    dv[u] = __uint_as_float(ldg32(blk));
                }
            }
        };
        auto store_batch = [&](uint64_t b0) {
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const uint64_t b = b0 + (uint64_t)WAVES * u;
                if (b >= nblk) break;
                const int mi = (int)(b / nsb);
                const uint64_t sb = b % nsb;
                if constexpr (FUSED) {
                    uint32_t qw;
                    int bs;
                    float d;
                    quantize_block(xv[u], lane, qw, bs, d);
                    store_block<TYPE>(s, mi, sb, lane, qw, bs, d);
                } else {
                    copy_block_store<TYPE>(s, mi, sb, lane, qv[u], bv[u], dv[u]);
                }
            }
        };
        uint64_t b0 = (uint64_t)wave_in_wg;
        load_batch(b0);
        asm volatile("" ::: "memory");
        load_group<TYPE, ITERS, R>(A, w, active ? wave : groups - 1, lane);
        while (true) {
            store_batch(b0);
            b0 += (uint64_t)WAVES * U;
            if (b0 >= nblk) break;
            load_batch(b0);
        }
    }
    __syncthreads();
    if (!active) return;

    Act act[ITERS];
    if constexpr (MT == 1) {
#pragma unroll
        for (int it = 0; it < ITERS; ++it) {
            const uint64_t sb = 16u * it + (lane >> 2);
            if (sb < nsb) slice_from_lds<TYPE>(act[it], s, 0, sb, lane & 3);
        }
    }
    uint64_t grp = wave;
    while (true) {
        finish_group<TYPE, ITERS, R, MT, FULL>(A, act, s, m, w, grp, lane, y);
        grp += nw;
        if (grp >= groups) break;
        load_group<TYPE, ITERS, R>(A, w, grp, lane);
    }
}

// Marks the registers of a loaded pass as redefined here, after every memory operation above
// (memory clobber): their decode cannot be scheduled earlier.
OQ_DEVICE void hold4(uint4& v) { asm volatile("" : "+v"(v.x), "+v"(v.y), "+v"(v.z), "+v"(v.w)::"memory"); }
template <uint32_t TYPE>
OQ_DEVICE void hold(W45& r) {
    hold4(r.c0);
    hold4(r.c1);
    hold4(r.hdr);
    if constexpr (TYPE == 13) {
        hold4(r.h0);
        hold4(r.h1);
    }
}
template <uint32_t TYPE>
OQ_DEVICE void hold(W6& r) {
    hold4(r.c0);
    hold4(r.c1);
    hold4(r.qh);
    asm volatile("" : "+v"(r.sc), "+v"(r.d)::"memory");
}

// Decode GEMV (one activation row), streamed.  Wave i of workgroup b owns the rows
// b*WAVES + i + k*nw (k >= 0, nw = waves in the grid) and walks their passes (16 super-blocks:
// 2 KiB of quants plus headers per wave) in order, holding exactly one pass in flight while it
// computes the previous one: the loads of pass u + 1 are issued once pass u has arrived.  The
// chip then keeps about one pass per resident wave in flight, enough to keep HBM streaming, while
// the memory queues stay short.  Per-lane partial sums and the row reduction are those of
// gemv_kq_kernel, so both kernels give the same bits.
template <uint32_t TYPE, int ITERS, bool FUSED, int WAVES, bool FULL>
__global__ __launch_bounds__(64 * WAVES) void gemv_stream_kernel(DeviceMatrix w, const float* x, const uint8_t* q8k,
                                                                 float* __restrict__ y, ArgmaxPart* amax) {
    using WR = typename WRegs<TYPE>::type;
    extern __shared__ __align__(16) uint8_t smem[];
    const int lane = threadIdx.x & 63;
    const int wave_in_wg = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t nw = gridDim.x * WAVES;
    const uint32_t n = (uint32_t)w.n;
    const uint32_t nsb = (uint32_t)(w.k / kQK);
    const ActLds s{smem, w.k};
    const uint32_t first = blockIdx.x * WAVES + (uint32_t)wave_in_wg;
    auto row_base = [&](uint32_t row) {
        row = row < n ? row : n - 1;  // a wave without rows reads row n-1 once
        return w.base + (uint64_t)__builtin_amdgcn_readfirstlane(row) * w.pitch;
    };

    // The first pass is requested once the activation row is staged: weight requests in flight
    // delay the activation loads of the workgroups that start later, which all wait on them.
    WR buf[2];
    stage_one_row<TYPE, ITERS, FUSED, WAVES>(s, x, q8k, nsb, wave_in_wg, lane, [] {});
    load_w<TYPE>(buf[0], row_base(first), nsb, 0, lane);
    __syncthreads();
    // greedy-token epilogue (amax set): the lane's first maximum over the rows it stores
    float best = -__builtin_inff();
    uint32_t bi = 0xFFFFFFFFu, nan = 0;
    if (first < n) {
    const int q = lane & 3;
    const ScaleSel ss = scale_sel(q);
    // up to two passes the lane's activation slices stay in registers; longer rows read the
    // slice of each pass from LDS when it is used
    constexpr bool kActRegs = ITERS <= 2;
    Act act[kActRegs ? ITERS : 1];
    if constexpr (kActRegs) {
#pragma unroll
        for (int it = 0; it < ITERS; ++it) {
            const uint32_t sb = 16u * it + (lane >> 2);
            if (sb < nsb) slice_from_lds<TYPE>(act[it], s, 0, sb, q);
        }
    }

    // Finished rows: lane (done % 64) keeps the sum and the row index of the done-th row; 64 at
    // a time are stored together.
    float acc = 0.0f, out = 0.0f;
    uint32_t out_row = 0, done = 0;
    uint32_t row = first, it = 0;  // the unit whose loads are in flight
    bool more = true;
    while (more) {
        // two units per trip, so that the buffer of every unit is a compile-time index (rows have
        // ITERS units: for ITERS <= 2 the pass of unit j is a compile-time index too)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int its = ITERS == 1 ? 0 : (ITERS == 2 ? j : (int)it);
            // Wait for unit (row, it), the only memory operation outstanding.  acc ties the wait
            // to the previous unit's arithmetic, which therefore stays ahead of it instead of
            // being deferred while the loads of further units are issued.
            asm volatile("s_waitcnt vmcnt(0)" : "+v"(acc), "+v"(out) :: "memory");
            // The wave whose data has arrived requests its next unit ahead of the other waves'
            // arithmetic on the SIMD: raised priority from the wait until those loads are issued
            // (the same bits; 12288 x 4096 6.95 -> 6.86 us, the 151936 x 4096 head 82.8 -> 80.8 us;
            // slower in the small-batch kernels and no faster in the block kernels, so not there).
            __builtin_amdgcn_s_setprio(2);
            uint32_t nrow = row, nit = it + 1;
            if (nit == ITERS) {
                nrow = row + nw < row ? n : row + nw;  // (no wrap-around)
                nit = 0;
            }
            more = nrow < n;
            // past the wave's last row: rows of one unit request nothing (the wait above covers
            // whatever is outstanding), measured 7.05 -> 6.91 us at 12288 x 4096; rows of several
            // units re-read the current pass (a cache hit), slower without it at 4096 x 12288
            // (7.81 -> 8.1 us)
            if (ITERS != 1 || more) load_w<TYPE>(buf[(j + 1) & 1], row_base(more ? nrow : row), nsb, (int)(more ? nit : it), lane);
            __builtin_amdgcn_s_setprio(0);
            hold<TYPE>(buf[j & 1]);  // the arithmetic below follows those loads
            const uint32_t sb = 16u * (uint32_t)its + (lane >> 2);
            if (FULL || sb < nsb) {
                if constexpr (kActRegs) {
                    acc = lane_fma(decode_w<TYPE>(buf[j & 1], ss, q), act[its], acc);
                } else {
                    Act a;
                    slice_from_lds<TYPE>(a, s, 0, sb, q);
                    acc = lane_fma(decode_w<TYPE>(buf[j & 1], ss, q), a, acc);
                }
            }
            if (it == ITERS - 1) {
                const float v = wave_sum_uniform(acc);
                const bool mine = lane == (int)(done & 63u);
                out = mine ? v : out;
                out_row = mine ? row : out_row;
                acc = 0.0f;
                ++done;
                if ((done & 63u) == 0u) {
                    y[out_row] = out;
                    if (amax != nullptr) {
                        nan |= out != out ? 1u : 0u;
                        argmax_take(best, bi, out, out_row);
                    }
                }
            }
            row = nrow;
            it = nit;
            if (!more) break;
        }
    }
    if ((uint32_t)lane < (done & 63u)) {
        y[out_row] = out;
        if (amax != nullptr) {
            nan |= out != out ? 1u : 0u;
            argmax_take(best, bi, out, out_row);
        }
    }
    }  // first < n
    if (amax != nullptr) {
        __shared__ float sv[WAVES];
        __shared__ uint32_t si[WAVES], sn[WAVES];
        argmax_wave(best, bi, nan);
        if (lane == 0) {
            sv[wave_in_wg] = best;
            si[wave_in_wg] = bi;
            sn[wave_in_wg] = nan;
        }
        __syncthreads();
        if (threadIdx.x == 0) {
            for (int i = 1; i < WAVES; ++i) {
                nan |= sn[i];
                argmax_take(best, bi, sv[i], si[i]);
            }
            amax[blockIdx.x] = ArgmaxPart{best, bi, nan};
        }
    }
}

// Stages the Q8_K form of m activation rows in LDS (row mi at s.q(mi)...), wave w taking the
// blocks w, w + WAVES, ... of the m * nsb blocks, four at a time with their loads issued together.
template <uint32_t TYPE, bool FUSED, int WAVES>
OQ_DEVICE void stage_rows(const ActLds& s, int m, const float* x, const uint8_t* q8k, uint64_t nsb, uint64_t k,
                          int wave_in_wg, int lane) {
    constexpr int U = 4;
    const uint64_t nblk = (uint64_t)m * nsb;
    for (uint64_t b0 = (uint64_t)wave_in_wg; b0 < nblk; b0 += (uint64_t)WAVES * U) {
        float4 xv[U];
        uint32_t qv[U], bv[U];
        float dv[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            uint64_t b = b0 + (uint64_t)WAVES * u;
            b = b < nblk ? b : nblk - 1;
            if constexpr (FUSED) {
                const uint64_t mi = b / nsb, sb = b % nsb;
                xv[u] = reinterpret_cast<const float4*>(x + mi * k + sb * kQK)[lane];
            } else {
                const uint8_t* blk = q8k + b * kQ8KBytes;
                qv[u] = ldg32(blk + 4 + 4 * lane);
                bv[u] = ldg32(blk + 260 + 4 * (lane & 7));
                dv[u] = __uint_as_float(ldg32(blk));
            }
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const uint64_t b = b0 + (uint64_t)WAVES * u;
            if (b >= nblk) break;
            const int mi = (int)(b / nsb);
            const uint64_t sb = b % nsb;
            if constexpr (FUSED) {
                uint32_t qw;
                int bs;
                float d;
                quantize_block(xv[u], lane, qw, bs, d);
                store_block<TYPE>(s, mi, sb, lane, qw, bs, d);
            } else {
                copy_block_store<TYPE>(s, mi, sb, lane, qv[u], bv[u], dv[u]);
            }
        }
    }
}

// The m F32 rows x [+ b] of K values, RMS-normalised and staged as Q8_K in one round (every
// block of a wave requested before the first store, then `issue`): per block the wave's double sum
// of squares (each lane's four squares in order, then the butterfly), per row the blocks' sums in
// block order, inv = 1 / sqrt(sum / K + eps) rounded to F32, values (v * inv) * w
// (rmsnorm_kernel's formula); workgroup 0 also stores the sums and the normalised rows.
template <uint32_t TYPE, int SBW, int WAVES, typename Issue>
OQ_DEVICE void stage_rows_norm(const ActLds& s, int m, const float* x, const MtNorm& nm, uint64_t nsb, uint64_t k,
                               int wave_in_wg, int lane, Issue&& issue) {
#pragma clang fp contract(off)
    __shared__ double red[kMtNormBlocks * WAVES];
    const uint64_t nblk = (uint64_t)m * nsb;
    float4 xv[SBW], bv[SBW], wv[SBW];
#pragma unroll
    for (int j = 0; j < SBW; ++j) {
        uint64_t b = (uint64_t)wave_in_wg + (uint64_t)WAVES * j;
        b = b < nblk ? b : nblk - 1;
        const uint64_t mi = b / nsb, sb = b % nsb;
        xv[j] = reinterpret_cast<const float4*>(x + mi * k + sb * kQK)[lane];
        if (nm.b != nullptr) bv[j] = reinterpret_cast<const float4*>(nm.b + mi * k + sb * kQK)[lane];
        wv[j] = reinterpret_cast<const float4*>(nm.w + sb * kQK)[lane];
    }
    asm volatile("" ::: "memory");
    issue();
#pragma unroll
    for (int j = 0; j < SBW; ++j) {
        const uint64_t b = (uint64_t)wave_in_wg + (uint64_t)WAVES * j;
        if (b >= nblk) break;
        if (nm.b != nullptr) {
            xv[j].x = xv[j].x + bv[j].x;
            xv[j].y = xv[j].y + bv[j].y;
            xv[j].z = xv[j].z + bv[j].z;
            xv[j].w = xv[j].w + bv[j].w;
        }
        const double sq = (double)xv[j].x * (double)xv[j].x + (double)xv[j].y * (double)xv[j].y +
                          (double)xv[j].z * (double)xv[j].z + (double)xv[j].w * (double)xv[j].w;
        const double bs = wave_sum_f64(sq);
        if (lane == 0) red[b] = bs;
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < SBW; ++j) {
        const uint64_t b = (uint64_t)wave_in_wg + (uint64_t)WAVES * j;
        if (b >= nblk) break;
        const uint64_t mi = b / nsb, sb = b % nsb;
        double tot = 0.0;
        for (uint64_t c = 0; c < nsb; ++c) tot += red[mi * nsb + c];
        const float inv = (float)(1.0 / sqrt(tot / (double)k + (double)nm.eps));
        float4 v;
        v.x = xv[j].x * inv * wv[j].x;
        v.y = xv[j].y * inv * wv[j].y;
        v.z = xv[j].z * inv * wv[j].z;
        v.w = xv[j].w * inv * wv[j].w;
        if (blockIdx.x == 0) {
            if (nm.sum_out != nullptr) reinterpret_cast<float4*>(nm.sum_out + mi * k + sb * kQK)[lane] = xv[j];
            if (nm.norm_out != nullptr) reinterpret_cast<float4*>(nm.norm_out + mi * k + sb * kQK)[lane] = v;
        }
        uint32_t qw;
        int bsum;
        float d;
        quantize_block(v, lane, qw, bsum, d);
        store_block<TYPE>(s, (int)mi, sb, lane, qw, bsum, d);
    }
}

// The m activation rows staged in one round: every block a wave stages (at most MT * ITERS * 16 /
// WAVES of them) is requested before the first store, then `issue` (the first weight loads), then
// the stores.  (A loop over rounds of a few blocks costs one memory round trip per round.)
template <uint32_t TYPE, int ITERS, int MT, bool FUSED, int WAVES, typename Issue>
OQ_DEVICE void stage_rows_once(const ActLds& s, int m, const float* x, const uint8_t* q8k, uint64_t nsb, uint64_t k,
                               int wave_in_wg, int lane, Issue&& issue) {
    constexpr int SBW = (MT * ITERS * 16 + WAVES - 1) / WAVES;
    const uint64_t nblk = (uint64_t)m * nsb;
    float4 xv[FUSED ? SBW : 1];
    uint32_t qv[FUSED ? 1 : SBW], bv[FUSED ? 1 : SBW];
    float dv[FUSED ? 1 : SBW];
#pragma unroll
    for (int j = 0; j < SBW; ++j) {
        uint64_t b = (uint64_t)wave_in_wg + (uint64_t)WAVES * j;
        b = b < nblk ? b : nblk - 1;
        if constexpr (FUSED) {
            const uint64_t mi = b / nsb, sb = b % nsb;
            xv[j] = reinterpret_cast<const float4*>(x + mi * k + sb * kQK)[lane];
        } else {
            const uint8_t* blk = q8k + b * kQ8KBytes;
            qv[j] = ldg32(blk + 4 + 4 * lane);
            bv[j] = ldg32(blk + 260 + 4 * (lane & 7));
            dv[j] = __uint_as_float(ldg32(blk));
        }
    }
    asm volatile("" ::: "memory");
    issue();
#pragma unroll
    for (int j = 0; j < SBW; ++j) {
        const uint64_t b = (uint64_t)wave_in_wg + (uint64_t)WAVES * j;
        if (b >= nblk) break;
        const int mi = (int)(b / nsb);
        const uint64_t sb = b % nsb;
        if constexpr (FUSED) {
            uint32_t qw;
            int bs;
            float d;
            quantize_block(xv[j], lane, qw, bs, d);
            store_block<TYPE>(s, mi, sb, lane, qw, bs, d);
        } else {
            copy_block_store<TYPE>(s, mi, sb, lane, qv[j], bv[j], dv[j]);
        }
    }
}

// Small-batch product (2 <= m <= MT activation rows), streamed like gemv_stream_kernel: 16-wave
// workgroups stage the m rows' Q8_K blocks in LDS once, a wave walks its weight rows one pass at
// a time with one pass in flight, decodes each pass once and multiplies it with the m activation
// slices read from LDS.  Per-lane sums in the order of gemv_kq_kernel (pass, then row mi) and the
// same row reductions: the same bits.  With set.nmat > 0 the rows are those of up to four
// matrices of w's type, K and pitch, concatenated (MtSet), each writing its own outputs: the same
// bits per row as one launch per matrix.  With set.conv the lane that stores a row of the DeltaNet
// in-projection also runs its epilogue over the m tokens (every wave then has fewer than 64 rows,
// so each row's outputs are still in the lane's registers at the end): the arithmetic of
// conv_gates_tokens_kernel, the same bits.
template <uint32_t TYPE, int ITERS, int MT, bool FUSED, bool FULL>
__global__ __launch_bounds__(1024) void gemv_stream_mt_kernel(DeviceMatrix w, int m, const float* x, const uint8_t* q8k,
                                                              float* __restrict__ y, MtSet set) {
    constexpr int WAVES = 16;
    using WR = typename WRegs<TYPE>::type;
    extern __shared__ __align__(16) uint8_t smem[];
    const int lane = threadIdx.x & 63;
    const int wave_in_wg = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t nw = gridDim.x * WAVES;
    const uint32_t n = set.nmat > 0 ? set.row_end[set.nmat - 1] : (uint32_t)w.n;
    const uint32_t nsb = (uint32_t)(w.k / kQK);
    const ActLds s{smem, w.k};
    const uint32_t first = blockIdx.x * WAVES + (uint32_t)wave_in_wg;
    // matrix of row r in a set (selects, not an indexed kernel-argument array)
    auto set_mat = [&](uint32_t r) {
        uint32_t i = 0;
#pragma unroll
        for (int j = 0; j < 3; ++j)
            if ((uint32_t)j + 1 < set.nmat && r >= set.row_end[j]) i = (uint32_t)j + 1;
        return i;
    };
    auto set_start = [&](uint32_t i) { return i == 0 ? 0u : i == 1 ? set.row_end[0] : i == 2 ? set.row_end[1] : set.row_end[2]; };
    auto row_base = [&](uint32_t row) {
        row = row < n ? row : n - 1;
        row = __builtin_amdgcn_readfirstlane(row);
        if (set.nmat == 0) return w.base + (uint64_t)row * w.pitch;
        const uint32_t i = set_mat(row);
        const uint8_t* b = i == 0 ? set.base[0] : i == 1 ? set.base[1] : i == 2 ? set.base[2] : set.base[3];
        return b + (uint64_t)(row - set_start(i)) * w.pitch;
    };
    auto store = [&](uint32_t r, int mi, float v) {
        if (set.nmat == 0) {
            y[(uint64_t)mi * n + r] = v;
            return;
        }
        const uint32_t i = set_mat(r), start = set_start(i);
        const uint32_t rows = (i == 0 ? set.row_end[0] : i == 1 ? set.row_end[1] : i == 2 ? set.row_end[2] : set.row_end[3]) - start;
        float* yi = i == 0 ? set.y[0] : i == 1 ? set.y[1] : i == 2 ? set.y[2] : set.y[3];
        const float* ai = i == 0 ? set.add[0] : i == 1 ? set.add[1] : i == 2 ? set.add[2] : set.add[3];
        const uint64_t at = (uint64_t)mi * rows + (r - start);
        yi[at] = ai != nullptr ? ai[at] + v : v;
    };
    // The DeltaNet in-projection epilogue, run by the whole wave after its last row: lane j < done
    // holds the m outputs of the wave's j-th row (row first + j * nw).  Every (row, token) pair gets
    // a lane: a channel row's token t sums the taps i in tap order in double (exact products) over
    // the values the history holds after t + 1 shifts -- history[t + 1 + i] while inside it, else
    // output t + 1 + i - K -- then SiLU; beta rows take the sigmoid, alpha rows softplus(a +
    // dt_bias) * decay.  Then each channel row's new history: its last K values of (history,
    // outputs).
    auto conv_epilogue = [&](uint32_t done, const float (&out)[MT]) {
        const MtConv& c = set.conv;
        const uint32_t K = c.kernel, C = set.row_end[0], H = set.row_end[2] - set.row_end[1];
        const uint32_t um = (uint32_t)m, pairs = done * um;
        auto pick = [&](const float (&v)[MT], uint32_t idx) {
            float r = 0.0f;
#pragma unroll
            for (int q = 0; q < MT; ++q) r = idx == (uint32_t)q ? v[q] : r;
            return r;
        };
        for (uint32_t p0 = 0; p0 < pairs; p0 += 64) {
            const uint32_t p = p0 + (uint32_t)lane;
            const uint32_t j = p < pairs ? p / um : 0, t = p < pairs ? p % um : 0;
            float xs[MT];  // row j's outputs, from lane j
#pragma unroll
            for (int q = 0; q < MT; ++q) xs[q] = __shfl(out[q], (int)j, 64);
            if (p >= pairs) continue;
            const uint32_t r = first + j * nw, i = set_mat(r), local = r - set_start(i);
            if (i == 0) {
                const float* hst = c.history + (uint64_t)local * K;
                const float* wc = c.conv_w + (uint64_t)local * K;
                double sum = 0.0;
                for (uint32_t tap = 0; tap < K; ++tap) {
                    const uint32_t u = t + 1 + tap;
                    const float v = u < K ? hst[u] : pick(xs, u - K);
                    sum += (double)v * (double)wc[tap];
                }
                c.conv_out[(uint64_t)t * C + local] = silu_ref((float)sum);
            } else if (i == 2) {
                c.beta_s[(uint64_t)t * H + local] = sigmoid_ref(pick(xs, t));
            } else if (i == 3) {
#pragma clang fp contract(off)
                c.log_decay[(uint64_t)t * H + local] = softplus_ref(pick(xs, t) + c.dt_bias[local]) * c.decay[local];
            }
        }
        // the new history, once every read of the old one above has returned
        if ((uint32_t)lane < done) {
            const uint32_t r = first + (uint32_t)lane * nw;  // matrix 0 starts the set: local row r
            if (set_mat(r) == 0) {
                float* hst = c.history + (uint64_t)r * K;
                float nv[kMtConvTaps];
#pragma unroll
                for (uint32_t tap = 0; tap < kMtConvTaps; ++tap) {
                    const uint32_t u = um + tap;
                    nv[tap] = tap < K ? (u < K ? hst[u] : pick(out, u - K)) : 0.0f;
                }
#pragma unroll
                for (uint32_t tap = 0; tap < kMtConvTaps; ++tap)
                    if (tap < K) hst[tap] = nv[tap];
            }
        }
    };

    WR buf[2];
    // one staging round (the first pass's weights requested between its loads and its stores)
    // while the per-wave block count stays small; several rounds beyond
    constexpr bool kOnce = (MT * ITERS * 16 + WAVES - 1) / WAVES <= (FUSED ? 8 : 12);
    constexpr int kSbw = (MT * ITERS * 16 + WAVES - 1) / WAVES;
    if constexpr (FUSED && kSbw <= kMtNormBlocks) {
        if (set.norm.w != nullptr) {
            stage_rows_norm<TYPE, kSbw, WAVES>(s, m, x, set.norm, nsb, w.k, wave_in_wg, lane,
                                               [&] { load_w<TYPE>(buf[0], row_base(first), nsb, 0, lane); });
        } else {
            stage_rows_once<TYPE, ITERS, MT, FUSED, WAVES>(s, m, x, q8k, nsb, w.k, wave_in_wg, lane,
                                                           [&] { load_w<TYPE>(buf[0], row_base(first), nsb, 0, lane); });
        }
    } else if constexpr (kOnce) {
        stage_rows_once<TYPE, ITERS, MT, FUSED, WAVES>(s, m, x, q8k, nsb, w.k, wave_in_wg, lane,
                                                       [&] { load_w<TYPE>(buf[0], row_base(first), nsb, 0, lane); });
    } else {
        stage_rows<TYPE, FUSED, WAVES>(s, m, x, q8k, nsb, w.k, wave_in_wg, lane);
        load_w<TYPE>(buf[0], row_base(first), nsb, 0, lane);
    }
    __syncthreads();
    if (first >= n) return;

    const int q = lane & 3;
    const ScaleSel ss = scale_sel(q);
    float acc[MT], out[MT];
#pragma unroll
    for (int mi = 0; mi < MT; ++mi) acc[mi] = out[mi] = 0.0f;
    uint32_t out_row = 0, done = 0;
    uint32_t row = first, it = 0;  // the unit whose loads are in flight
    bool more = true;
    while (more) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            uint32_t nrow = row, nit = it + 1;
            if (nit == ITERS) {
                nrow = row + nw < row ? n : row + nw;
                nit = 0;
            }
            more = nrow < n;
            load_w<TYPE>(buf[(j + 1) & 1], row_base(more ? nrow : row), nsb, (int)(more ? nit : it), lane);
            hold<TYPE>(buf[j & 1]);
            const uint32_t sb = 16u * it + (lane >> 2);
            if (FULL || sb < nsb) {
                const auto dec = decode_w<TYPE>(buf[j & 1], ss, q);
#pragma unroll
                for (int mi = 0; mi < MT; ++mi) {
                    if (mi < m) {
                        Act a;
                        slice_from_lds<TYPE>(a, s, mi, sb, q);
                        acc[mi] = lane_fma(dec, a, acc[mi]);
                    }
                }
            }
            if (it == ITERS - 1) {
                const bool mine = lane == (int)(done & 63u);
#pragma unroll
                for (int mi = 0; mi < MT; ++mi) {
                    const float v = wave_sum_uniform(acc[mi]);
                    out[mi] = mine ? v : out[mi];
                    acc[mi] = 0.0f;
                }
                out_row = mine ? row : out_row;
                ++done;
                if ((done & 63u) == 0u) {
#pragma unroll
                    for (int mi = 0; mi < MT; ++mi)
                        if (mi < m) store(out_row, mi, out[mi]);
                }
            }
            row = nrow;
            it = nit;
            if (!more) break;
        }
    }
    if ((uint32_t)lane < (done & 63u)) {
#pragma unroll
        for (int mi = 0; mi < MT; ++mi)
            if (mi < m) store(out_row, mi, out[mi]);
    }
    if (set.conv.conv_w != nullptr) conv_epilogue(done, out);
}

// Long rows (K beyond the compile-time kernels), any m <= MT: a window of passes
// [pass0, pass0 + npass) of every row, streamed like gemv_stream_mt_kernel (16-wave workgroups,
// the m rows' Q8_K blocks of the window staged in LDS once, one pass in flight per wave).  With
// `accumulate` the window's partial sums are added to y, so a row longer than one window's LDS
// image is multiplied by consecutive launches over its windows (the reference's dot has no
// length limit, src/backend/cpu/quantized_reference.cpp:128-162).  Activation rows are
// x + mi * w.k (F32, quantized in the staging) or Q8_K blocks q8k + mi * (w.k / 256).
template <uint32_t TYPE, bool FUSED>
OQ_DEVICE void stage_window(const ActLds& s, int m, const float* x, const uint8_t* q8k, uint64_t k_total,
                            uint32_t sb0, uint32_t nsbw, int wave_in_wg, int lane) {
    constexpr int WAVES = 16, U = 4;
    const uint64_t nblk = (uint64_t)m * nsbw;
    const uint64_t nsb_total = k_total / kQK;
    for (uint64_t b0 = (uint64_t)wave_in_wg; b0 < nblk; b0 += (uint64_t)WAVES * U) {
        float4 xv[U];
        uint32_t qv[U], bv[U];
        float dv[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            uint64_t b = b0 + (uint64_t)WAVES * u;
            b = b < nblk ? b : nblk - 1;
            const uint64_t mi = b / nsbw, sb = sb0 + b % nsbw;
            if constexpr (FUSED) {
                xv[u] = reinterpret_cast<const float4*>(x + mi * k_total + sb * kQK)[lane];
            } else {
                const uint8_t* blk = q8k + (mi * nsb_total + sb) * kQ8KBytes;
                qv[u] = ldg32(blk + 4 + 4 * lane);
                bv[u] = ldg32(blk + 260 + 4 * (lane & 7));
                dv[u] = __uint_as_float(ldg32(blk));
            }
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const uint64_t b = b0 + (uint64_t)WAVES * u;
            if (b >= nblk) break;
            const int mi = (int)(b / nsbw);
            const uint64_t sb = b % nsbw;  // block index within the window image
            if constexpr (FUSED) {
                uint32_t qw;
                int bs;
                float d;
                quantize_block(xv[u], lane, qw, bs, d);
                store_block<TYPE>(s, mi, sb, lane, qw, bs, d);
            } else {
                copy_block_store<TYPE>(s, mi, sb, lane, qv[u], bv[u], dv[u]);
            }
        }
    }
}

template <uint32_t TYPE, int MT, bool FUSED>
__global__ __launch_bounds__(1024) void gemv_stream_win_kernel(DeviceMatrix w, int m, const float* x,
                                                               const uint8_t* q8k, float* __restrict__ y,
                                                               uint32_t pass0, uint32_t npass, int accumulate) {
    constexpr int WAVES = 16;
    using WR = typename WRegs<TYPE>::type;
    extern __shared__ __align__(16) uint8_t smem[];
    const int lane = threadIdx.x & 63;
    const int wave_in_wg = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t nw = gridDim.x * WAVES;
    const uint32_t n = (uint32_t)w.n;
    const uint32_t nsb = (uint32_t)(w.k / kQK);
    const uint32_t sb0 = 16u * pass0;
    const uint32_t sb_end = 16u * (pass0 + npass) < nsb ? 16u * (pass0 + npass) : nsb;
    const uint32_t nsbw = sb_end - sb0;
    const uint32_t pass_end = pass0 + npass;
    const ActLds s{smem, (uint64_t)nsbw * kQK};
    const uint32_t first = blockIdx.x * WAVES + (uint32_t)wave_in_wg;
    auto row_base = [&](uint32_t row) {
        row = row < n ? row : n - 1;
        return w.base + (uint64_t)__builtin_amdgcn_readfirstlane(row) * w.pitch;
    };

    WR buf[2];
    stage_window<TYPE, FUSED>(s, m, x, q8k, w.k, sb0, nsbw, wave_in_wg, lane);
    load_w<TYPE>(buf[0], row_base(first), nsb, (int)pass0, lane);
    __syncthreads();
    if (first >= n) return;

    const int q = lane & 3;
    const ScaleSel ss = scale_sel(q);
    float acc[MT], out[MT];
#pragma unroll
    for (int mi = 0; mi < MT; ++mi) acc[mi] = out[mi] = 0.0f;
    uint32_t out_row = 0, done = 0;
    uint32_t row = first, it = pass0;  // the unit whose loads are in flight
    bool more = true;
    auto flush = [&](bool all) {
        // lane (done % 64) holds the sum of the done-th finished row
        if (all || (uint32_t)lane < (done & 63u)) {
#pragma unroll
            for (int mi = 0; mi < MT; ++mi) {
                if (mi < m) {
                    float* dst = y + (uint64_t)mi * n + out_row;
                    *dst = accumulate ? *dst + out[mi] : out[mi];
                }
            }
        }
    };
    while (more) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            uint32_t nrow = row, nit = it + 1;
            if (nit == pass_end) {
                nrow = row + nw < row ? n : row + nw;
                nit = pass0;
            }
            more = nrow < n;
            load_w<TYPE>(buf[(j + 1) & 1], row_base(more ? nrow : row), nsb, (int)(more ? nit : it), lane);
            hold<TYPE>(buf[j & 1]);
            const uint32_t sb = 16u * it + (lane >> 2);
            if (sb < nsb) {
                const auto dec = decode_w<TYPE>(buf[j & 1], ss, q);
#pragma unroll
                for (int mi = 0; mi < MT; ++mi) {
                    if (mi < m) {
                        Act a;
                        slice_from_lds<TYPE>(a, s, mi, sb - sb0, q);
                        acc[mi] = lane_fma(dec, a, acc[mi]);
                    }
                }
            }
            if (it == pass_end - 1) {
                const bool mine = lane == (int)(done & 63u);
#pragma unroll
                for (int mi = 0; mi < MT; ++mi) {
                    const float v = wave_sum_uniform(acc[mi]);
                    out[mi] = mine ? v : out[mi];
                    acc[mi] = 0.0f;
                }
                out_row = mine ? row : out_row;
                ++done;
                if ((done & 63u) == 0u) flush(true);
            }
            row = nrow;
            it = nit;
            if (!more) break;
        }
    }
    flush(false);
}

template <uint32_t TYPE, int MT, bool FUSED>
hipError_t launch_window(const DeviceMatrix& w, int m, const float* x, const uint8_t* q8k, float* y, uint32_t pass0,
                         uint32_t npass, int accumulate, hipStream_t s) {
    const uint64_t nsb = w.k / kQK;
    const uint64_t sb_end = 16ull * (pass0 + npass) < nsb ? 16ull * (pass0 + npass) : nsb;
    const uint64_t lds = act_lds_bytes((sb_end - 16ull * pass0) * kQK, MT);
    uint64_t wgs = (uint64_t)cu_count();
    const uint64_t need = (w.n + 15) / 16;
    if (wgs > need) wgs = need;
    hipLaunchKernelGGL((gemv_stream_win_kernel<TYPE, MT, FUSED>), dim3((unsigned)wgs), dim3(1024), lds, s, w, m, x,
                       q8k, y, pass0, npass, accumulate);
    return hipGetLastError();
}

// ---------------------------------------------------------------- launch

// Workgroups resident per CU for this instantiation (register and LDS limits), from the first
// call's LDS size (a function-local static: initialised once, thread-safe)
template <uint32_t TYPE, int ITERS, int R, int MT, bool FUSED, int WAVES, bool FULL>
int resident_per_cu(uint64_t lds_bytes) {
    static const int cached = [lds_bytes] {
        int n = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, gemv_kq_kernel<TYPE, ITERS, R, MT, FUSED, WAVES, FULL>,
                                                         64 * WAVES, lds_bytes) != hipSuccess || n < 1) {
            n = 1;
        }
        return n;
    }();
    return cached;
}

template <uint32_t TYPE, int ITERS, int R, int MT, bool FUSED, int WAVES, bool FULL>
hipError_t launch_full(const DeviceMatrix& w, int m, const float* x, const uint8_t* q8k, float* y, hipStream_t s) {
    const uint64_t groups = (w.n + R - 1) / R;
    const uint64_t lds = act_lds_bytes(w.k, MT);
    // two workgroups per CU where both fit (more would only repeat the activation staging)
    int wg_per_cu = knob(kGemvWgPerCu, 2);
    if (wg_per_cu < 1) wg_per_cu = 1;
    const int resident = resident_per_cu<TYPE, ITERS, R, MT, FUSED, WAVES, FULL>(lds);
    if (wg_per_cu > resident) wg_per_cu = resident;
    uint64_t wgs = (uint64_t)cu_count() * (uint64_t)wg_per_cu;
    const uint64_t need = (groups + WAVES - 1) / WAVES;
    if (wgs > need) wgs = need;
    hipLaunchKernelGGL((gemv_kq_kernel<TYPE, ITERS, R, MT, FUSED, WAVES, FULL>), dim3((unsigned)wgs), dim3(64 * WAVES),
                       lds, s, w, m, x, q8k, y);
    return hipGetLastError();
}

template <uint32_t TYPE, int ITERS, int R, int MT, bool FUSED, int WAVES>
hipError_t launch_one(const DeviceMatrix& w, int m, const float* x, const uint8_t* q8k, float* y, hipStream_t s) {
    if ((w.k / kQK) % 16 == 0) return launch_full<TYPE, ITERS, R, MT, FUSED, WAVES, true>(w, m, x, q8k, y, s);
    return launch_full<TYPE, ITERS, R, MT, FUSED, WAVES, false>(w, m, x, q8k, y, s);
}

template <uint32_t TYPE, int ITERS, bool FUSED, int WAVES, bool FULL>
hipError_t launch_stream(const DeviceMatrix& w, const float* x, const uint8_t* q8k, float* y, hipStream_t s,
                         ArgmaxPart* amax = nullptr, uint32_t max_parts = 0, uint32_t* nparts = nullptr) {
    const uint64_t lds = act_lds_bytes(w.k, 1);
    static const int resident = [lds] {
        int n = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, gemv_stream_kernel<TYPE, ITERS, FUSED, WAVES, FULL>,
                                                         64 * WAVES, lds) != hipSuccess || n < 1) {
            n = 1;
        }
        return n;
    }();
    // sixteen waves per CU: ~37 KiB of weights in flight per CU, and each CU stages the
    // activation row once per sixteen waves
    int wg_per_cu = knob(kStreamWgPerCu, 16 / WAVES);
    wg_per_cu = wg_per_cu < 1 ? 1 : (wg_per_cu > resident ? resident : wg_per_cu);
    uint64_t wgs = (uint64_t)cu_count() * (uint64_t)wg_per_cu;
    const uint64_t need = (w.n + WAVES - 1) / WAVES;
    if (wgs > need) wgs = need;
    if (amax != nullptr) {
        if (wgs > max_parts) return hipErrorNotSupported;
        *nparts = (uint32_t)wgs;
    }
    hipLaunchKernelGGL((gemv_stream_kernel<TYPE, ITERS, FUSED, WAVES, FULL>), dim3((unsigned)wgs), dim3(64 * WAVES),
                       lds, s, w, x, q8k, y, amax);
    return hipGetLastError();
}

// the m = 1 streamed GEMV with the greedy-token epilogue (16-wave workgroups)
template <uint32_t TYPE, bool FUSED>
hipError_t launch_argmax_iters(const DeviceMatrix& w, const float* x, const uint8_t* q8k, float* y, ArgmaxPart* amax,
                               uint32_t max_parts, uint32_t* nparts, hipStream_t s) {
    const bool full = (w.k / kQK) % 16 == 0;
    switch ((w.k / kQK + 15) / 16) {
#define OQ_ARGMAX_CASE(IT)                                                                                        \
    case IT:                                                                                                      \
        return full ? launch_stream<TYPE, IT, FUSED, 16, true>(w, x, q8k, y, s, amax, max_parts, nparts)          \
                    : launch_stream<TYPE, IT, FUSED, 16, false>(w, x, q8k, y, s, amax, max_parts, nparts);
        OQ_ARGMAX_CASE(1)
        OQ_ARGMAX_CASE(2)
        OQ_ARGMAX_CASE(3)
        OQ_ARGMAX_CASE(4)
#undef OQ_ARGMAX_CASE
        default: return hipErrorNotSupported;
    }
}

template <uint32_t TYPE, int ITERS, int MT, bool FUSED, bool FULL>
hipError_t launch_stream_mt(const DeviceMatrix& w, int m, const float* x, const uint8_t* q8k, float* y, hipStream_t s,
                            const MtSet& set = MtSet{}) {
    const uint64_t lds = act_lds_bytes(w.k, MT);
    if (lds > kLdsBudget) {
        // beyond the default dynamic LDS limit (once per instantiation; a function-local static)
        static const hipError_t attr = hipFuncSetAttribute(
            reinterpret_cast<const void*>(gemv_stream_mt_kernel<TYPE, ITERS, MT, FUSED, FULL>),
            hipFuncAttributeMaxDynamicSharedMemorySize, (int)kMtLdsBudget);
        if (attr != hipSuccess) return attr;
    }
    uint64_t wgs = (uint64_t)cu_count();
    const uint64_t rows = set.nmat > 0 ? set.row_end[set.nmat - 1] : w.n;
    const uint64_t need = (rows + 15) / 16;
    if (wgs > need) wgs = need;
    // the epilogue runs at the end, on the rows still held: fewer than 64 per wave
    if (set.conv.conv_w != nullptr && (rows + wgs * 16 - 1) / (wgs * 16) >= 64) return hipErrorNotSupported;
    hipLaunchKernelGGL((gemv_stream_mt_kernel<TYPE, ITERS, MT, FUSED, FULL>), dim3((unsigned)wgs), dim3(1024), lds, s,
                       w, m, x, q8k, y, set);
    return hipGetLastError();
}

// A set of matrices through the streamed small-batch kernel (Q8_K activations): hipErrorNotSupported
// where that kernel is not the one launch_rows would choose for this m, K and type
template <uint32_t TYPE, int ITERS, int MT>
hipError_t launch_set_rows(const DeviceMatrix& w, int m, const uint8_t* q8k, const MtSet& set, hipStream_t s) {
    if constexpr (MT > 1 && !(TYPE == 13 && MT == 8)) {
        if (act_lds_bytes(w.k, MT) <= mt_lds_budget(TYPE) && knob(kGemvStreamMt, 1) != 0) {
            return (w.k / kQK) % 16 == 0 ? launch_stream_mt<TYPE, ITERS, MT, false, true>(w, m, nullptr, q8k, nullptr, s, set)
                                         : launch_stream_mt<TYPE, ITERS, MT, false, false>(w, m, nullptr, q8k, nullptr, s, set);
        }
    }
    return hipErrorNotSupported;
}

template <uint32_t TYPE, int MT>
hipError_t launch_set_iters(const DeviceMatrix& w, int m, const uint8_t* q8k, const MtSet& set, hipStream_t s) {
    switch ((w.k / kQK + 15) / 16) {
        case 1: return launch_set_rows<TYPE, 1, MT>(w, m, q8k, set, s);
        case 2: return launch_set_rows<TYPE, 2, MT>(w, m, q8k, set, s);
        case 3: return launch_set_rows<TYPE, 3, MT>(w, m, q8k, set, s);
        case 4: return launch_set_rows<TYPE, 4, MT>(w, m, q8k, set, s);
        default: return hipErrorNotSupported;
    }
}

// The normalising set launch (F32 rows x, set.norm): the kernels whose staging holds a wave's
// blocks in one round, m * K <= kMtNormBlocks * 4096; hipErrorNotSupported otherwise
template <uint32_t TYPE, int ITERS, int MT>
hipError_t launch_set_norm_rows(const DeviceMatrix& w, int m, const float* x, const MtSet& set, hipStream_t s) {
    if constexpr (MT > 1 && !(TYPE == 13 && MT == 8) && MT * ITERS <= kMtNormBlocks) {
        if (act_lds_bytes(w.k, MT) <= mt_lds_budget(TYPE) && knob(kGemvStreamMt, 1) != 0) {
            return (w.k / kQK) % 16 == 0 ? launch_stream_mt<TYPE, ITERS, MT, true, true>(w, m, x, nullptr, nullptr, s, set)
                                         : launch_stream_mt<TYPE, ITERS, MT, true, false>(w, m, x, nullptr, nullptr, s, set);
        }
    }
    return hipErrorNotSupported;
}

// Two rows only: every workgroup normalises the rows itself, which at four rows of 4096 (and the
// post-attention norm's addend rows) cost more than the separate RMSNorm launch it saves
// (DeltaNet block 90.2 -> 93.4 us, attention block 108.6 -> 113.8 us at 4 tokens; 2 tokens
// 67.3 -> 63.9 and 80.8 -> 77.6 us)
template <uint32_t TYPE>
hipError_t launch_set_norm_m(const DeviceMatrix& w, int m, const float* x, const MtSet& set, hipStream_t s) {
    const uint64_t iters = (w.k / kQK + 15) / 16;
    if (m != 2) return hipErrorNotSupported;
    if (iters == 1) return launch_set_norm_rows<TYPE, 1, 2>(w, m, x, set, s);
    if (iters == 2) return launch_set_norm_rows<TYPE, 2, 2>(w, m, x, set, s);
    return hipErrorNotSupported;
}

template <uint32_t TYPE>
hipError_t launch_set_m(const DeviceMatrix& w, int m, const uint8_t* q8k, const MtSet& set, hipStream_t s) {
    if (m <= 1) return hipErrorNotSupported;
    if (m <= 2) return launch_set_iters<TYPE, 2>(w, m, q8k, set, s);
    if (m <= 4) return launch_set_iters<TYPE, 4>(w, m, q8k, set, s);
    return launch_set_iters<TYPE, 8>(w, m, q8k, set, s);
}

template <uint32_t TYPE, int ITERS, int MT, bool FUSED>
hipError_t launch_rows(const DeviceMatrix& w, int m, const float* x, const uint8_t* q8k, float* y, hipStream_t s) {
    if constexpr (MT == 1) {
        // Streamed kernel: measured faster than issuing every row of a wave at once (below) for
        // 2048 to 151936 rows of 2048 to 12288 columns (0.8 to 1.2 us less on 2048 to 12288 q4_K
        // rows of 4096); the batched kernel stays selectable with OQ_GEMV_STREAM=0.
        if (knob(kGemvStream, 1) != 0) {
            const bool full = (w.k / kQK) % 16 == 0;
            if (knob(kStreamWaves, 16) >= 16) {
                return full ? launch_stream<TYPE, ITERS, FUSED, 16, true>(w, x, q8k, y, s)
                            : launch_stream<TYPE, ITERS, FUSED, 16, false>(w, x, q8k, y, s);
            }
            return full ? launch_stream<TYPE, ITERS, FUSED, 8, true>(w, x, q8k, y, s)
                        : launch_stream<TYPE, ITERS, FUSED, 8, false>(w, x, q8k, y, s);
        }
    }
    if constexpr (MT > 1 && !(TYPE == 13 && MT == 8)) {
        // small batches (from Q8_K blocks, or F32 rows quantized in the staging): streamed, one
        // pass in flight
        // (q5_K with eight rows would spill within the 128 registers of a 16-wave workgroup)
        if (act_lds_bytes(w.k, MT) <= mt_lds_budget(TYPE) && knob(kGemvStreamMt, 1) != 0) {
            return (w.k / kQK) % 16 == 0 ? launch_stream_mt<TYPE, ITERS, MT, FUSED, true>(w, m, x, q8k, y, s)
                                         : launch_stream_mt<TYPE, ITERS, MT, FUSED, false>(w, m, x, q8k, y, s);
        }
    }
    const int rows = knob(kGemvRows, MT == 1 && ITERS <= 2 ? 2 : 1);
    const int waves = knob(kGemvWaves, 8);
    if constexpr (MT == 1 && ITERS <= 3) {  // two rows per wave would spill beyond 3 passes
        if (rows >= 2) {
            if constexpr (ITERS == 1) {
                if (waves >= 16) return launch_one<TYPE, ITERS, 2, MT, FUSED, 16>(w, m, x, q8k, y, s);
            }
            return launch_one<TYPE, ITERS, 2, MT, FUSED, 8>(w, m, x, q8k, y, s);
        }
    }
    // small batches: two rows per wave use every activation slice read from LDS twice (Q5_K's
    // extra high-bit words do not fit two rows of three slots for eight columns without spilling)
    if constexpr (MT > 1 && ITERS <= 3 && !(TYPE == 13 && ITERS * MT > 16)) {
        if (knob(kGemvRowsMt, 2) >= 2) return launch_one<TYPE, ITERS, 2, MT, FUSED, 8>(w, m, x, q8k, y, s);
    }
    return launch_one<TYPE, ITERS, 1, MT, FUSED, 8>(w, m, x, q8k, y, s);
}

template <uint32_t TYPE, int MT, bool FUSED>
hipError_t launch_iters(const DeviceMatrix& w, int m, const float* x, const uint8_t* q8k, float* y, hipStream_t s) {
    switch ((w.k / kQK + 15) / 16) {
        case 1: return launch_rows<TYPE, 1, MT, FUSED>(w, m, x, q8k, y, s);
        case 2: return launch_rows<TYPE, 2, MT, FUSED>(w, m, x, q8k, y, s);
        case 3: return launch_rows<TYPE, 3, MT, FUSED>(w, m, x, q8k, y, s);
        case 4: return launch_rows<TYPE, 4, MT, FUSED>(w, m, x, q8k, y, s);
        default: return hipErrorNotSupported;
    }
}

template <uint32_t TYPE, bool FUSED>
hipError_t launch_m(const DeviceMatrix& w, int m, const float* x, const uint8_t* q8k, float* y, hipStream_t s) {
    if (m <= 1) return launch_iters<TYPE, 1, FUSED>(w, m, x, q8k, y, s);
    if (m <= 2) return launch_iters<TYPE, 2, FUSED>(w, m, x, q8k, y, s);
    if (m <= 4) return launch_iters<TYPE, 4, FUSED>(w, m, x, q8k, y, s);
    return launch_iters<TYPE, 8, FUSED>(w, m, x, q8k, y, s);
}

}  // namespace

}  // namespace kq

}  // namespace oq
