// Prefill / verify GEMM for q4_K weights (m >= 16 activation rows) on gfx950 matrix cores.
//
// Y[m][n] = sum_k Xhat[m][k] * W[n][k] with Xhat the dequantized Q8_K activations (d*q) and W
// the reference's decoded weights ((d*sc)*q - dmin*m, src/model/storage_decode.cpp:63-94 applied
// to GGML q4_K).  Both operands are rounded once to binary16 and multiplied on
// v_mfma_f32_32x32x16_f16 with F32 accumulation.  The rounding is relative 2^-11 per operand;
// over K >= 4096 terms its effect on an output stays below 1e-4 * sum_k |w_k * xhat_k| with a
// wide margin (checked by the parity tests), so the path is enabled only for K >= 4096.
//
// Data flow (one call):
//   1. activations -> F16 image Xhat[m][K] in scratch.  From F32 x the Q8_K quantization is
//      the one of quantize_q8k (bit-identical q and d) and Xhat = f16(d*q); caller-supplied
//      Q8_K blocks are converted the same way.
//   2. GEMM: a 128 (m) x 256 (n) output tile per 256-thread workgroup (one wave per SIMD)
//      over one K-split of whole super-blocks, in steps of 64 k.  Wave w owns all 128 rows and
//      64 columns (4 x 2 accumulators of 32 x 32).  It dequantizes its own weight columns
//      straight into MFMA B operands in registers (no LDS), while the activation tiles are
//      shared through a ring of three LDS buffers.  A wave can retire only about one 1 KB LDS
//      read per 50 cycles, so the LDS traffic is what limits a GEMM with one wave per SIMD;
//      keeping the weights out of LDS leaves 16 operand reads + 4 stores per wave per step.
//   3. with more than one K-split, partial tiles go to scratch and a reduction kernel adds
//      them in split order (deterministic).
//
// Weight dequantization: a nibble goes to F32 exactly (v_cvt_f32_ubyte), one F32 fma applies
// the scale and the min, and v_cvt_pk_f16_f32 rounds two weights to f16 (nearest even); the
// conversion instructions are interleaved with the MFMAs, which execute asynchronously.
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
// From this K on, weights are dequantized with packed f16 arithmetic (scale and min rounded to
// f16 per sub-block); below it, from F32.  The extra rounding roughly 1.3x the output error,
// which the longer sums absorb: worst normalised errors measured 3.7e-5 at K = 8192 and 3.3e-5
// at K = 12288 against the 1e-4 bar.
constexpr uint64_t kFastMinK = 8192;
constexpr int kMaxSplits = 8;
constexpr int kLdsA = kBM * kBK;    // f16 elements per A tile buffer

// F16 tiles: row r holds 64 k as eight 16-byte chunks; logical chunk c sits at physical chunk
// c ^ ((r / 2) % 8), which keeps the MFMA operand reads and the tile writes free of LDS bank
// conflicts without padding.
OQ_DEVICE int tile_off(int r, int c) { return r * kBK + 8 * (c ^ ((r >> 1) & 7)); }

// ---------------------------------------------------------------- activation image

OQ_DEVICE uint32_t pack_f16(float a, float b) {
    const float2v v = {a, b};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, half2v));
}

// F32 x [m][K] -> f16(d * q) with the Q8_K quantization of quantize_q8k (one wave per block)
__global__ __launch_bounds__(256) void quantize_f16_kernel(const float* __restrict__ x, uint64_t nblocks,
                                                           _Float16* __restrict__ out) {
    const int lane = threadIdx.x & 63;
    const uint64_t blk = blockIdx.x * 4ull + (threadIdx.x >> 6);
    if (blk >= nblocks) return;
    const float4 v = reinterpret_cast<const float4*>(x + blk * kQK)[lane];
    const Q8KLane r = quantize_q8k_block_wave(v, lane);
    float f[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) f[i] = r.d * (float)(int8_t)(r.qword >> (8 * i));
    *reinterpret_cast<uint2*>(out + blk * kQK + 4 * lane) = make_uint2(pack_f16(f[0], f[1]), pack_f16(f[2], f[3]));
}

// Q8_K blocks -> f16(d * q)
__global__ __launch_bounds__(256) void q8k_to_f16_kernel(const uint8_t* __restrict__ q8k, uint64_t nblocks,
                                                         _Float16* __restrict__ out) {
    const int lane = threadIdx.x & 63;
    const uint64_t blk = blockIdx.x * 4ull + (threadIdx.x >> 6);
    if (blk >= nblocks) return;
    const uint8_t* b = q8k + blk * kQ8KBytes;
    const float d = *reinterpret_cast<const float*>(b);
    const uint32_t q = *reinterpret_cast<const uint32_t*>(b + 4 + 4 * lane);
    float f[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) f[i] = d * (float)(int8_t)(q >> (8 * i));
    *reinterpret_cast<uint2*>(out + blk * kQK + 4 * lane) = make_uint2(pack_f16(f[0], f[1]), pack_f16(f[2], f[3]));
}

// ---------------------------------------------------------------- tiles

struct Tile {
    uint64_t m0, n0;
    uint32_t sb0;  // first super-block of this split
};

// k order inside one 64-element group (the same for both operands, so the product is
// unchanged): MFMA k-slice ks (16 k), lane half h, operand element i covers
//   k = 32 (ks & 1) + 16 h + 8 (ks >> 1) + i.
// A: 8 consecutive k = chunk 4 (ks & 1) + 2 h + (ks >> 1) of an F16 tile row.
// B: bytes 16 h + 8 (ks >> 1) + i of the weight row's 32-byte group, low nibbles for even ks,
//    high nibbles for odd ks: lane half h reads exactly 16-byte chunk e = h of the group (see
//    oq_layout.h), and the slices alternate between the group's two sub-blocks.
OQ_DEVICE int a_chunk(int ks, int h) { return 4 * (ks & 1) + 2 * h + (ks >> 1); }

// ---------------------------------------------------------------- activations
//
// All 256 threads copy the step's 128 x 64 F16 tile: 16-byte chunks c = tid + 256 j (j = 0..3),
// row c / 8, chunk c % 8.

struct Act {
    uint4 c[4];
};

OQ_DEVICE Act load_act(const _Float16* a16, const DeviceMatrix& w, int m, const Tile& t, uint32_t step, int tid) {
    Act a;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t c = tid + 256 * j;
        uint64_t row = t.m0 + (c >> 3);
        row = row < (uint64_t)m ? row : (uint64_t)m - 1;
        a.c[j] = *reinterpret_cast<const uint4*>(a16 + row * w.k + (uint64_t)t.sb0 * kQK + (uint64_t)step * kBK +
                                                 8 * (c & 7));
    }
    return a;
}

OQ_DEVICE void store_act(const Act& a, _Float16* As, int tid) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int c = tid + 256 * j;
        *reinterpret_cast<uint4*>(As + tile_off(c >> 3, c & 7)) = a.c[j];
    }
}

// ---------------------------------------------------------------- weights
//
// Wave w owns weight rows n0 + 64 w + 32 j + (lane % 32), j = 0, 1 (two 32-column MFMA tiles);
// lane half h = lane / 32 reads chunk e = h of every group.  Per super-block a lane loads the
// four chunks (one per group, adjacent in the row layout) of both its rows and the two rows'
// headers; the weights never pass through LDS.

struct WData {
    uint4 q[2][4];  // [j][group]
    uint4 hdr[2];   // [j]
};

OQ_DEVICE WData load_wdata(const DeviceMatrix& w, const Tile& t, uint64_t sb, int wave, int lane) {
    const uint64_t nsb = w.k / kQK;
    WData d;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        uint64_t n = t.n0 + 64 * wave + 32 * j + (lane & 31);
        n = n < w.n ? n : w.n - 1;
        const uint8_t* row = w.base + n * w.pitch;
        const uint4* q = reinterpret_cast<const uint4*>(row + 16 * perm_chunk(nsb, sb, 0, (uint32_t)(lane >> 5)));
#pragma unroll
        for (int g = 0; g < 4; ++g) d.q[j][g] = q[g];
        d.hdr[j] = *reinterpret_cast<const uint4*>(row + 128 * nsb + 16 * sb);
    }
    return d;
}

// d*sc and dmin*m of sub-block `sub` of a header, in the reference's F32 arithmetic, and (for
// the packed path) as f16 pairs {ds, ds}, {-dm, -dm}
struct Scale {
    float ds, dm;
    uint32_t ds2, ndm2;
};

template <bool FAST>
OQ_DEVICE Scale scale_of(uint4 hdr, uint32_t sub) {
    // hardware f16 -> f32 (exact for every finite value; NaN payloads do not matter here)
    const float d = (float)__builtin_bit_cast(_Float16, (uint16_t)(hdr.x & 0xFFFFu));
    const float dmin = (float)__builtin_bit_cast(_Float16, (uint16_t)(hdr.x >> 16));
    uint32_t sc, mn;
    scale_min_k4(sub, hdr.y, hdr.z, hdr.w, sc, mn);
    Scale s;
    {
#pragma clang fp contract(off)
        s.ds = d * (float)sc;
        s.dm = dmin * (float)mn;
    }
    if (FAST) {
        s.ds2 = pack_f16(s.ds, s.ds);
        s.ndm2 = pack_f16(-s.dm, -s.dm);
    } else {
        s.ds2 = s.ndm2 = 0;
    }
    return s;
}

// Identity byte permutation (one v_perm_b32): keeps the optimizer from merging a byte mask into
// the extractions below, so that they map onto v_cvt_f32_ubyte<i>, while remaining an ordinary
// vector instruction.
OQ_DEVICE uint32_t opaque(uint32_t v) { return __builtin_amdgcn_perm(0u, v, 0x03020100u); }

template <int I>
OQ_DEVICE float ubyte(uint32_t u) {
    return (float)((u >> (8 * I)) & 0xFFu);
}

// Two weights of a B operand from the nibbles of bytes 2p, 2p+1 of `nib` (already masked).
//   exact: f16(ds*q - dm) from F32 (one rounding);
//   FAST:  the nibbles become the f16 values 1024 + q (bit pattern 0x6400 | q, placed by one
//          v_perm_b32), minus 1024 (exact), then one v_pk_fma_f16 with ds and -dm rounded to f16:
//          three instructions per pair instead of five, at the price of the f16 rounding of
//          the sub-block's scale and min.
template <bool FAST>
OQ_DEVICE uint32_t weight_pair(uint32_t nib, int p, const Scale& s) {
    if (FAST) {
        const half2v k1024 = {(_Float16)1024.0f, (_Float16)1024.0f};
        half2v x = __builtin_bit_cast(half2v, __builtin_amdgcn_perm(0x64646464u, nib, p == 0 ? 0x04010400u : 0x04030402u));
        x = x - k1024;
        x = __builtin_elementwise_fma(x, __builtin_bit_cast(half2v, s.ds2), __builtin_bit_cast(half2v, s.ndm2));
        return __builtin_bit_cast(uint32_t, x);
    }
    const float a = p == 0 ? ubyte<0>(nib) : ubyte<2>(nib);
    const float b = p == 0 ? ubyte<1>(nib) : ubyte<3>(nib);
    return pack_f16(__builtin_fmaf(a, s.ds, -s.dm), __builtin_fmaf(b, s.ds, -s.dm));
}

// nibble word (masked, one per quant dword) of slice ks from a lane's 16-byte group chunk
template <bool FAST>
OQ_DEVICE uint32_t nib_word(uint4 q, int ks, int half) {
    const uint32_t d = (ks >> 1) == 0 ? (half == 0 ? q.x : q.y) : (half == 0 ? q.z : q.w);
    const uint32_t v = (ks & 1) ? (d >> 4) & 0x0F0F0F0Fu : d & 0x0F0F0F0Fu;
    return FAST ? v : opaque(v);
}

// ---------------------------------------------------------------- one step of one wave
//
// Multiplies step s (group G) from A buffer Ac, with B operands converted in registers, and
// meanwhile: reads the A operands of its next k-slice; converts the B operands of its next
// k-slice; during the last slice, reads the first A operands of step s+1 (buffer An1, filled at
// step s-1) and converts the first B operands of step s+1 (group G1 of `wn`, scales sn0 of
// sub-block 2 G1); at the end stores the activation tile of step s+2 (loaded two steps
// earlier) into buffer An2.
//
// The MFMAs alternate with small pieces of the conversion (a wave issues in order; MFMAs
// grouped together would hold the conversion back), fixed by sched_barrier.
template <bool FAST, int G, int G1>
OQ_DEVICE void wave_step(const _Float16* Ac, const _Float16* An1, _Float16* An2, float16v (&acc)[4][2],
                         half8 (&a)[4], uint32_t (&b)[2][4], const WData& wc, const WData& wn, Scale sn0_0,
                         Scale sn0_1, const Act& act2, int lane, int tid) {
    const int h = lane >> 5, r0 = lane & 31;
    const Scale s0[2] = {scale_of<FAST>(wc.hdr[0], 2 * G), scale_of<FAST>(wc.hdr[1], 2 * G)};
    const Scale s1[2] = {scale_of<FAST>(wc.hdr[0], 2 * G + 1), scale_of<FAST>(wc.hdr[1], 2 * G + 1)};
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
        // operands of the next slice (of this step, or slice 0 of step s+1)
        const _Float16* As = ks < 3 ? Ac : An1;
        const int nks = (ks + 1) & 3;
        half8 an[4];
        uint32_t bn[2][4];
#pragma unroll
        for (int i = 0; i < 4; ++i) an[i] = *reinterpret_cast<const half8*>(As + tile_off(32 * i + r0, a_chunk(nks, h)));
        uint32_t nw[2][2];
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            const int i = q >> 1, j = q & 1;
            half8 bj;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const uint32_t v = b[j][e];
                bj[2 * e] = __builtin_bit_cast(half2v, v)[0];
                bj[2 * e + 1] = __builtin_bit_cast(half2v, v)[1];
            }
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[i], bj, acc[i][j], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
            // B operand of the next slice: MFMA q converts pair q % 4 of n-tile q / 4
            const int jj = q >> 2, pp = q & 3;
            const uint4 src = ks < 3 ? wc.q[jj][G] : wn.q[jj][G1];
            const Scale sc = ks < 3 ? ((nks & 1) ? s1[jj] : s0[jj]) : (jj == 0 ? sn0_0 : sn0_1);
            if (pp == 0) {
                nw[jj][0] = nib_word<FAST>(src, nks, 0);
                nw[jj][1] = nib_word<FAST>(src, nks, 1);
            }
            bn[jj][pp] = weight_pair<FAST>(nw[jj][pp >> 1], pp & 1, sc);
            __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) a[i] = an[i];
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int e = 0; e < 4; ++e) b[j][e] = bn[j][e];
    }
    store_act(act2, An2, tid);
}

// Workgroup barrier after this wave's LDS writes have completed.  Unlike __syncthreads() it does
// not wait for outstanding global loads (the prefetches in flight across the barrier).
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

// grid: tiles_n * tiles_m * splits workgroups of 4 waves.  Output: y (one split) or
// partial[z][m][n].  Wave w computes rows m0..m0+127 x columns n0+64w..n0+64w+63 (4 x 2
// accumulators of 32 x 32).  Activation tiles go through a ring of three LDS buffers: step s
// reads buffer s%3, stores step s+2 into buffer (s+2)%3 (last read at step s-1), and reads the
// first operands of step s+1 from buffer (s+1)%3 (stored at step s-1); one barrier per step.
template <bool FAST>
__global__ __launch_bounds__(kThreads) void gemm_q4k_f16_kernel(DeviceMatrix w, int m, const _Float16* a16,
                                                               uint32_t tiles_n, uint32_t tiles_m, uint32_t splits,
                                                               float* __restrict__ out) {
    __shared__ __align__(16) _Float16 ring[3 * kLdsA];
    _Float16* const A0 = ring;
    _Float16* const A1 = ring + kLdsA;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t nsb = (uint32_t)(w.k / kQK);
    const Unit un = unit_of(blockIdx.x, tiles_n, tiles_m, splits);
    const uint32_t z = un.z;
    Tile t;
    t.n0 = (uint64_t)un.nt * kBN;
    t.m0 = (uint64_t)un.mt * kBM;
    t.sb0 = (uint32_t)((uint64_t)z * nsb / splits);
    const uint32_t sb1 = (uint32_t)((uint64_t)(z + 1) * nsb / splits);
    const uint32_t nsbu = sb1 - t.sb0;   // >= 1: splits <= nsb
    const uint32_t last = 4 * nsbu - 1;  // last step
    auto step_of = [last](uint32_t s) { return s <= last ? s : last; };
    auto sb_of = [&](uint32_t i) { return (uint64_t)t.sb0 + (i < nsbu ? i : nsbu - 1); };
    const int h = lane >> 5, r0 = lane & 31;

    float16v acc[4][2] = {};
    // prologue: activation tiles of steps 0 and 1, the operands of step 0's first slice
    Act act = load_act(a16, w, m, t, 0, tid);
    store_act(act, A0, tid);
    act = load_act(a16, w, m, t, step_of(1), tid);
    store_act(act, A1, tid);
    // activation tiles in flight: actA for steps 2, 4, ..., actB for steps 3, 5, ...
    Act actA = load_act(a16, w, m, t, step_of(2), tid);
    Act actB = load_act(a16, w, m, t, step_of(3), tid);
    WData cur = load_wdata(w, t, sb_of(0), wave, lane), nxt = cur;
    lds_barrier();
    half8 a[4];
    uint32_t b[2][4];
#pragma unroll
    for (int i = 0; i < 4; ++i) a[i] = *reinterpret_cast<const half8*>(A0 + tile_off(32 * i + r0, a_chunk(0, h)));
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const Scale sc = scale_of<FAST>(cur.hdr[j], 0);
        const uint32_t n0w = nib_word<FAST>(cur.q[j][0], 0, 0), n1w = nib_word<FAST>(cur.q[j][0], 0, 1);
        b[j][0] = weight_pair<FAST>(n0w, 0, sc);
        b[j][1] = weight_pair<FAST>(n0w, 1, sc);
        b[j][2] = weight_pair<FAST>(n1w, 0, sc);
        b[j][3] = weight_pair<FAST>(n1w, 1, sc);
    }
    // Each step: wave_step, then the activation load of step s+4, then the barrier.
    auto step = [&](auto G_, auto G1_, const _Float16* Ac, const _Float16* An1, _Float16* An2, uint32_t s,
                    const WData& wc, const WData& wn, Act& act2) {
        constexpr int G = decltype(G_)::value, G1 = decltype(G1_)::value;
        const Scale sn0_0 = scale_of<FAST>(wn.hdr[0], 2 * G1), sn0_1 = scale_of<FAST>(wn.hdr[1], 2 * G1);
        wave_step<FAST, G, G1>(Ac, An1, An2, acc, a, b, wc, wn, sn0_0, sn0_1, act2, lane, tid);
        act2 = load_act(a16, w, m, t, step_of(s + 4), tid);
        lds_barrier();
    };
    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    using I2 = std::integral_constant<int, 2>;
    using I3 = std::integral_constant<int, 3>;
    auto buf = [&](uint32_t k) { return ring + kLdsA * (k % 3); };  // tile buffer of step k
    for (uint32_t i = 0; i < nsbu; ++i) {
        const uint32_t s = 4 * i;
        nxt = load_wdata(w, t, sb_of(i + 1), wave, lane);
        step(I0{}, I1{}, buf(s), buf(s + 1), buf(s + 2), s, cur, cur, actA);
        step(I1{}, I2{}, buf(s + 1), buf(s + 2), buf(s + 3), s + 1, cur, cur, actB);
        step(I2{}, I3{}, buf(s + 2), buf(s + 3), buf(s + 4), s + 2, cur, cur, actA);
        step(I3{}, I0{}, buf(s + 3), buf(s + 4), buf(s + 5), s + 3, cur, nxt, actB);
        cur = nxt;
    }
    // result register r of lane l: row 8*(r/4) + 4*(l/32) + r%4, column l%32
    float* o = out + (uint64_t)z * (uint64_t)m * w.n;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const uint64_t col = t.n0 + 64 * wave + 32 * j + (lane & 31);
        if (col >= w.n) continue;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
#pragma unroll
            for (int rr = 0; rr < 16; ++rr) {
                const uint64_t row = t.m0 + 32 * i + 8 * (rr / 4) + 4 * (lane >> 5) + (rr % 4);
                if (row < (uint64_t)m) o[row * w.n + col] = acc[i][j][rr];
            }
        }
    }
}

// y[i] = sum over splits s (in order) of partial[s][i]; count4 = outputs / 4
__global__ __launch_bounds__(256) void reduce_splits_kernel(const float4* __restrict__ part, uint64_t count4,
                                                            uint32_t splits, float4* __restrict__ y) {
    const uint64_t stride = (uint64_t)gridDim.x * 256;
    for (uint64_t i = blockIdx.x * 256ull + threadIdx.x; i < count4; i += stride) {
        float4 s = part[i];
        for (uint32_t z = 1; z < splits; ++z) {
            const float4 p = part[(uint64_t)z * count4 + i];
            s.x += p.x;
            s.y += p.y;
            s.z += p.z;
            s.w += p.w;
        }
        y[i] = s;
    }
}

// the same for outputs whose count is not a multiple of 4
__global__ __launch_bounds__(256) void reduce_splits_scalar_kernel(const float* __restrict__ part, uint64_t count,
                                                                   uint32_t splits, float* __restrict__ y) {
    const uint64_t stride = (uint64_t)gridDim.x * 256;
    for (uint64_t i = blockIdx.x * 256ull + threadIdx.x; i < count; i += stride) {
        float s = part[i];
        for (uint32_t z = 1; z < splits; ++z) s += part[(uint64_t)z * count + i];
        y[i] = s;
    }
}

struct Plan {
    uint32_t tiles_n, tiles_m, splits;
    uint64_t a16_bytes, part_bytes;
};

uint64_t round256(uint64_t v) { return (v + 255) & ~uint64_t(255); }

Plan make_plan(const DeviceMatrix& w, int m) {
    Plan p;
    p.tiles_n = (uint32_t)((w.n + kBN - 1) / kBN);
    p.tiles_m = (uint32_t)((m + kBM - 1) / kBM);
    const uint64_t tiles = (uint64_t)p.tiles_n * p.tiles_m;
    const uint32_t nsb = (uint32_t)(w.k / kQK);
    uint64_t s = ((uint64_t)cu_count() + tiles / 2) / tiles;
    int forced = env_int("OQ_GEMM_SPLITS", 0);
    if (forced > 0) s = (uint64_t)forced;
    if (s < 1) s = 1;
    if (s > kMaxSplits) s = kMaxSplits;
    if (s > nsb) s = nsb;
    p.splits = (uint32_t)s;
    p.a16_bytes = round256((uint64_t)m * w.k * 2);
    p.part_bytes = p.splits > 1 ? (uint64_t)p.splits * m * w.n * 4 : 0;
    return p;
}

}  // namespace

bool gemm_mfma_supported(const DeviceMatrix& w, int m) {
    return w.type == 12 && m >= 16 && w.k >= kMinK && w.k % kQK == 0;
}

uint64_t gemm_scratch_bytes(const DeviceMatrix& w, int m) {
    const Plan p = make_plan(w, m);
    return p.a16_bytes + p.part_bytes;
}

hipError_t launch_gemm_q4k_mfma(const DeviceMatrix& w, int m, const float* x, const uint8_t* q8k, float* y,
                                void* scratch, hipStream_t s) {
    if (!gemm_mfma_supported(w, m) || (x == nullptr) == (q8k == nullptr)) return hipErrorNotSupported;
    const Plan p = make_plan(w, m);
    uint8_t* base = static_cast<uint8_t*>(scratch);
    _Float16* a16 = reinterpret_cast<_Float16*>(base);
    float* part = reinterpret_cast<float*>(base + p.a16_bytes);
    const uint64_t nblocks = (uint64_t)m * (w.k / kQK);
    const unsigned qgrid = (unsigned)((nblocks + 3) / 4);
    if (x) {
        hipLaunchKernelGGL(quantize_f16_kernel, dim3(qgrid), dim3(256), 0, s, x, nblocks, a16);
    } else {
        hipLaunchKernelGGL(q8k_to_f16_kernel, dim3(qgrid), dim3(256), 0, s, q8k, nblocks, a16);
    }
    const unsigned wgs = p.tiles_n * p.tiles_m * p.splits;
    if (w.k >= kFastMinK && env_int("OQ_GEMM_EXACT_DEQUANT", 0) == 0) {
        hipLaunchKernelGGL(gemm_q4k_f16_kernel<true>, dim3(wgs), dim3(kThreads), 0, s, w, m, a16, p.tiles_n,
                           p.tiles_m, p.splits, p.splits > 1 ? part : y);
    } else {
        hipLaunchKernelGGL(gemm_q4k_f16_kernel<false>, dim3(wgs), dim3(kThreads), 0, s, w, m, a16, p.tiles_n,
                           p.tiles_m, p.splits, p.splits > 1 ? part : y);
    }
    if (p.splits > 1) {
        const uint64_t count = (uint64_t)m * w.n;
        if (count % 4 == 0) {
            uint64_t blocks = (count / 4 + 255) / 256;
            if (blocks > 8192) blocks = 8192;
            hipLaunchKernelGGL(reduce_splits_kernel, dim3((unsigned)blocks), dim3(256), 0, s,
                               reinterpret_cast<const float4*>(part), count / 4, p.splits,
                               reinterpret_cast<float4*>(y));
        } else {
            uint64_t blocks = (count + 255) / 256;
            if (blocks > 8192) blocks = 8192;
            hipLaunchKernelGGL(reduce_splits_scalar_kernel, dim3((unsigned)blocks), dim3(256), 0, s, part, count,
                               p.splits, y);
        }
    }
    return hipGetLastError();
}

}  // namespace oq
