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
//      over one K-split of whole super-blocks, in steps of 64 k, double-buffered in LDS.  Each
//      wave issues the MFMAs of its 64 x 128 sub-tile (eight 32 x 32 accumulators) from one
//      pair of F16 tiles and, while they run, copies its share of the next step's activations
//      into the other pair and dequantizes its share of the next step's 4-bit weights into it.
//      Large sub-tiles keep the LDS operand traffic near 96 KB per step.
//   3. with more than one K-split, partial tiles go to scratch and a reduction kernel adds
//      them in split order (deterministic).
//
// Weight dequantization: a nibble goes to F32 exactly (v_cvt_f32_ubyte), one F32 fma applies
// the scale and the min, and v_cvt_pk_f16_f32 rounds two weights to f16 (nearest even).
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
constexpr int kMaxSplits = 8;
constexpr int kLdsA = kBM * kBK;    // f16 elements per A tile buffer
constexpr int kLdsB = kBN * kBK;    // f16 elements per B tile buffer

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

// ---------------------------------------------------------------- conversion share
//
// Thread u = tid (0..255) of the workgroup:
//   activations: 16-byte chunks u + 256 j (j = 0..3) of the step's 128 x 64 F16 tile (row c/8,
//                chunk c%8), copied from the F16 image;
//   weights:     row u of the tile: per super-block the thread loads both 64-byte lines of the
//                row (piece 0 and 1: four 16-byte chunks each, one per 64-group, adjacent in
//                the row layout of oq_layout.h) and dequantizes one chunk of each (64 weights)
//                per step.

struct Lines {
    uint4 p0[4], p1[4];  // piece 0 / piece 1 chunk of group 0..3
};

OQ_DEVICE Lines load_lines(const DeviceMatrix& w, const Tile& t, uint64_t sb, int u) {
    const uint64_t nsb = w.k / kQK;
    uint64_t n = t.n0 + u;
    n = n < w.n ? n : w.n - 1;
    const uint8_t* row = w.base + n * w.pitch;
    const uint4* q0 = reinterpret_cast<const uint4*>(row + 16 * perm_chunk(nsb, sb, 0, 0));
    const uint4* q1 = reinterpret_cast<const uint4*>(row + 16 * perm_chunk(nsb, sb, 0, 1));
    Lines l;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        l.p0[g] = q0[g];
        l.p1[g] = q1[g];
    }
    return l;
}

OQ_DEVICE uint4 load_header(const DeviceMatrix& w, const Tile& t, uint64_t sb, int u) {
    uint64_t n = t.n0 + u;
    n = n < w.n ? n : w.n - 1;
    return *reinterpret_cast<const uint4*>(w.base + n * w.pitch + 128 * (w.k / kQK) + 16 * sb);
}

struct Act {
    uint4 c[4];  // chunks u + 256 j of one step's activation tile
};

OQ_DEVICE Act load_act(const _Float16* a16, const DeviceMatrix& w, int m, const Tile& t, uint32_t step, int u) {
    Act a;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t c = u + 256 * j;
        uint64_t row = t.m0 + (c >> 3);
        row = row < (uint64_t)m ? row : (uint64_t)m - 1;
        a.c[j] = *reinterpret_cast<const uint4*>(a16 + row * w.k + (uint64_t)t.sb0 * kQK + (uint64_t)step * kBK +
                                                 8 * (c & 7));
    }
    return a;
}

OQ_DEVICE void store_act(const Act& a, _Float16* As, int u) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int c = u + 256 * j;
        *reinterpret_cast<uint4*>(As + tile_off(c >> 3, c & 7)) = a.c[j];
    }
}

// Identity byte permutation (one v_perm_b32): keeps the optimizer from merging a byte mask into
// the extractions below, so that they map onto v_cvt_f32_ubyte<i>, while remaining an ordinary
// vector instruction the scheduler can move.
OQ_DEVICE uint32_t opaque(uint32_t v) { return __builtin_amdgcn_perm(0u, v, 0x03020100u); }

template <int I>
OQ_DEVICE float ubyte(uint32_t u) {
    return (float)((u >> (8 * I)) & 0xFFu);
}

// bytes b_0..b_3 of u -> f16(s * b_i + c), as two dwords (b_0, b_1), (b_2, b_3)
OQ_DEVICE uint2 convert4(uint32_t u, float s, float c) {
    uint2 r;
    r.x = pack_f16(__builtin_fmaf(ubyte<0>(u), s, c), __builtin_fmaf(ubyte<1>(u), s, c));
    r.y = pack_f16(__builtin_fmaf(ubyte<2>(u), s, c), __builtin_fmaf(ubyte<3>(u), s, c));
    return r;
}

// f16((d*sc)*q - dmin*m) for the 32 weights of one chunk of group G of weight row r:
// low nibbles -> k = 16P + i (sub-block 2G), high nibbles -> k = 32 + 16P + i (sub-block 2G+1)
OQ_DEVICE void convert_chunk(uint4 qv, float ds0, float dm0, float ds1, float dm1, _Float16* Bs, int r, int piece) {
    const uint32_t words[4] = {qv.x, qv.y, qv.z, qv.w};
    uint32_t lo[8], hi[8];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t l4 = opaque(words[j] & 0x0F0F0F0Fu), h4 = opaque((words[j] >> 4) & 0x0F0F0F0Fu);
        const uint2 a = convert4(l4, ds0, -dm0), b = convert4(h4, ds1, -dm1);
        lo[2 * j] = a.x;
        lo[2 * j + 1] = a.y;
        hi[2 * j] = b.x;
        hi[2 * j + 1] = b.y;
    }
    const int c = 2 * piece;
    *reinterpret_cast<uint4*>(Bs + tile_off(r, c)) = make_uint4(lo[0], lo[1], lo[2], lo[3]);
    *reinterpret_cast<uint4*>(Bs + tile_off(r, c + 1)) = make_uint4(lo[4], lo[5], lo[6], lo[7]);
    *reinterpret_cast<uint4*>(Bs + tile_off(r, c + 4)) = make_uint4(hi[0], hi[1], hi[2], hi[3]);
    *reinterpret_cast<uint4*>(Bs + tile_off(r, c + 5)) = make_uint4(hi[4], hi[5], hi[6], hi[7]);
}

// both chunks (pieces) of group G of weight row u
template <int G>
OQ_DEVICE void convert_weights(uint4 hdr, const Lines& l, _Float16* Bs, int u) {
    // hardware f16 -> f32 (exact for every finite value; NaN payloads do not matter here)
    const float d = (float)__builtin_bit_cast(_Float16, (uint16_t)(hdr.x & 0xFFFFu));
    const float dmin = (float)__builtin_bit_cast(_Float16, (uint16_t)(hdr.x >> 16));
    uint32_t sc0, mn0, sc1, mn1;
    scale_min_k4(2 * G, hdr.y, hdr.z, hdr.w, sc0, mn0);
    scale_min_k4(2 * G + 1, hdr.y, hdr.z, hdr.w, sc1, mn1);
    float ds0, dm0, ds1, dm1;
    {
#pragma clang fp contract(off)
        ds0 = d * (float)sc0;
        dm0 = dmin * (float)mn0;
        ds1 = d * (float)sc1;
        dm1 = dmin * (float)mn1;
    }
    convert_chunk(l.p0[G], ds0, dm0, ds1, dm1, Bs, u, 0);
    convert_chunk(l.p1[G], ds0, dm0, ds1, dm1, Bs, u, 1);
}

// ---------------------------------------------------------------- MFMA waves
//
// Wave w in a 2 (m) x 2 (n) grid: a 64 x 128 sub-tile, 2 x 4 accumulators of 32 x 32.
OQ_DEVICE void mma_step(const _Float16* As, const _Float16* Bs, int wm, int wn, int lane, float16v (&acc)[2][4]) {
    const int ra = 64 * wm + (lane & 31), rb = 128 * wn + (lane & 31), h = lane >> 5;
#pragma unroll
    for (int ks = 0; ks < kBK / 16; ++ks) {
        half8 a[2], b[4];
#pragma unroll
        for (int i = 0; i < 2; ++i) a[i] = *reinterpret_cast<const half8*>(As + tile_off(ra + 32 * i, 2 * ks + h));
#pragma unroll
        for (int j = 0; j < 4; ++j) b[j] = *reinterpret_cast<const half8*>(Bs + tile_off(rb + 32 * j, 2 * ks + h));
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[i], b[j], acc[i][j], 0, 0, 0);
    }
}

// One step of one wave, in an explicit instruction order: the MFMAs of this step's tiles (64 x
// 128 sub-tile, four k-slices of 16) with, after every fourth MFMA, one unit of the conversion
// of the next step (four weight nibble-words -> 32 f16, i.e. one 16-byte quant dword pair of
// lanes) and the operand reads of the next k-slice issued one slice ahead.  A wave issues in
// order, so MFMAs grouped together would hold the conversion back until the last one issued;
// interleaved, the vector ALU works while the matrix core executes.  sched_barrier keeps the
// compiler from regrouping them.
template <int G>
OQ_DEVICE void fused_step(const _Float16* Ac, const _Float16* Bc, _Float16* An, _Float16* Bn, int wm, int wn,
                          int lane, float16v (&acc)[2][4], const Act& act, uint4 hdr, const Lines& l, int u) {
    const int ra = 64 * wm + (lane & 31), rb = 128 * wn + (lane & 31), h = lane >> 5;
    half8 a[2], b[4];
#pragma unroll
    for (int i = 0; i < 2; ++i) a[i] = *reinterpret_cast<const half8*>(Ac + tile_off(ra + 32 * i, h));
#pragma unroll
    for (int j = 0; j < 4; ++j) b[j] = *reinterpret_cast<const half8*>(Bc + tile_off(rb + 32 * j, h));
    store_act(act, An, u);
    // scales of sub-blocks 2G, 2G+1 of weight row u
    const float d = (float)__builtin_bit_cast(_Float16, (uint16_t)(hdr.x & 0xFFFFu));
    const float dmin = (float)__builtin_bit_cast(_Float16, (uint16_t)(hdr.x >> 16));
    uint32_t sc0, mn0, sc1, mn1;
    scale_min_k4(2 * G, hdr.y, hdr.z, hdr.w, sc0, mn0);
    scale_min_k4(2 * G + 1, hdr.y, hdr.z, hdr.w, sc1, mn1);
    float ds0, dm0, ds1, dm1;
    {
#pragma clang fp contract(off)
        ds0 = d * (float)sc0;
        dm0 = dmin * (float)mn0;
        ds1 = d * (float)sc1;
        dm1 = dmin * (float)mn1;
    }
    const uint32_t words[8] = {l.p0[G].x, l.p0[G].y, l.p0[G].z, l.p0[G].w,
                               l.p1[G].x, l.p1[G].y, l.p1[G].z, l.p1[G].w};
    uint32_t lo[8], hi[8], l4 = 0, h4 = 0;
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
        half8 an[2], bn[4];
        if (ks < 3) {
#pragma unroll
            for (int i = 0; i < 2; ++i) an[i] = *reinterpret_cast<const half8*>(Ac + tile_off(ra + 32 * i, 2 * (ks + 1) + h));
#pragma unroll
            for (int j = 0; j < 4; ++j) bn[j] = *reinterpret_cast<const half8*>(Bc + tile_off(rb + 32 * j, 2 * (ks + 1) + h));
        }
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            const int i = q >> 2, j = q & 3;
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[i], b[j], acc[i][j], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
            // weight pair p = 8 ks + q of the 32 this thread converts: quant word p/4, pair p%4
            // (0, 1: low nibbles of bytes 0-1 / 2-3; 2, 3: high nibbles)
            const int p = 8 * ks + q, wd = p >> 2, pp = p & 3, wi = wd & 3;
            if (pp == 0) {
                l4 = opaque(words[wd] & 0x0F0F0F0Fu);
                h4 = opaque((words[wd] >> 4) & 0x0F0F0F0Fu);
            }
            if (pp == 0) lo[2 * wi] = pack_f16(__builtin_fmaf(ubyte<0>(l4), ds0, -dm0), __builtin_fmaf(ubyte<1>(l4), ds0, -dm0));
            if (pp == 1) lo[2 * wi + 1] = pack_f16(__builtin_fmaf(ubyte<2>(l4), ds0, -dm0), __builtin_fmaf(ubyte<3>(l4), ds0, -dm0));
            if (pp == 2) hi[2 * wi] = pack_f16(__builtin_fmaf(ubyte<0>(h4), ds1, -dm1), __builtin_fmaf(ubyte<1>(h4), ds1, -dm1));
            if (pp == 3) {
                hi[2 * wi + 1] = pack_f16(__builtin_fmaf(ubyte<2>(h4), ds1, -dm1), __builtin_fmaf(ubyte<3>(h4), ds1, -dm1));
                if (wi == 3) {  // a whole 16-byte chunk (32 weights) of piece wd/4 is ready
                    const int c = 2 * (wd >> 2);
                    *reinterpret_cast<uint4*>(Bn + tile_off(u, c)) = make_uint4(lo[0], lo[1], lo[2], lo[3]);
                    *reinterpret_cast<uint4*>(Bn + tile_off(u, c + 1)) = make_uint4(lo[4], lo[5], lo[6], lo[7]);
                    *reinterpret_cast<uint4*>(Bn + tile_off(u, c + 4)) = make_uint4(hi[0], hi[1], hi[2], hi[3]);
                    *reinterpret_cast<uint4*>(Bn + tile_off(u, c + 5)) = make_uint4(hi[4], hi[5], hi[6], hi[7]);
                }
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        if (ks < 3) {
#pragma unroll
            for (int i = 0; i < 2; ++i) a[i] = an[i];
#pragma unroll
            for (int j = 0; j < 4; ++j) b[j] = bn[j];
        }
    }
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

// grid: tiles_n * tiles_m * splits workgroups.  Output: y (one split) or partial[z][m][n].
//
// Each of the four waves (one per SIMD) multiplies its 64 x 128 sub-tile of step s from tile
// buffer s%2 while it converts its share of step s+1 (weight row u = tid, activation chunks
// u + 256 j) into buffer (s+1)%2: the MFMAs run asynchronously in the matrix core while the
// same wave's conversion instructions issue on the vector ALU.  One barrier per step.
// Activations are loaded two steps ahead, the weight lines and headers of super-block i+1 at
// the first step of super-block i.
__global__ __launch_bounds__(kThreads) void gemm_q4k_f16_kernel(DeviceMatrix w, int m, const _Float16* a16,
                                                               uint32_t tiles_n, uint32_t tiles_m, uint32_t splits,
                                                               float* __restrict__ out) {
    // separate objects per buffer, so that the compiler may interleave the conversion's stores
    // to one buffer with the operand loads from the other
    __shared__ __align__(16) _Float16 As0[kLdsA], Bs0[kLdsB];
    __shared__ __align__(16) _Float16 As1[kLdsA], Bs1[kLdsB];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1, u = tid;
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

    float16v acc[2][4] = {};
    Lines cur = load_lines(w, t, sb_of(0), u), nxt;
    uint4 hdr = load_header(w, t, sb_of(0), u), hdr_next;
    Act a0 = load_act(a16, w, m, t, 0, u);
    Act a1 = load_act(a16, w, m, t, step_of(1), u);
    store_act(a0, As0, u);
    convert_weights<0>(hdr, cur, Bs0, u);
    a0 = load_act(a16, w, m, t, step_of(2), u);
    lds_barrier();  // step 0 converted
    for (uint32_t i = 0; i < nsbu; ++i) {
        const uint32_t s = 4 * i;
        // step s: multiply s, convert s+1
        nxt = load_lines(w, t, sb_of(i + 1), u);
        hdr_next = load_header(w, t, sb_of(i + 1), u);
        fused_step<1>(As0, Bs0, As1, Bs1, wm, wn, lane, acc, a1, hdr, cur, u);
        a1 = load_act(a16, w, m, t, step_of(s + 3), u);
        lds_barrier();
        // step s+1
        fused_step<2>(As1, Bs1, As0, Bs0, wm, wn, lane, acc, a0, hdr, cur, u);
        a0 = load_act(a16, w, m, t, step_of(s + 4), u);
        lds_barrier();
        // step s+2
        fused_step<3>(As0, Bs0, As1, Bs1, wm, wn, lane, acc, a1, hdr, cur, u);
        a1 = load_act(a16, w, m, t, step_of(s + 5), u);
        lds_barrier();
        // step s+3: convert the first group of super-block i+1
        cur = nxt;
        hdr = hdr_next;
        fused_step<0>(As1, Bs1, As0, Bs0, wm, wn, lane, acc, a0, hdr, cur, u);
        a0 = load_act(a16, w, m, t, step_of(s + 6), u);
        lds_barrier();
    }
    // result register r of lane l: row 8*(r/4) + 4*(l/32) + r%4, column l%32
    float* o = out + (uint64_t)z * (uint64_t)m * w.n;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint64_t col = t.n0 + 128 * wn + 32 * j + (lane & 31);
        if (col >= w.n) continue;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const uint64_t row = t.m0 + 64 * wm + 32 * i + 8 * (r / 4) + 4 * (lane >> 5) + (r % 4);
                if (row < (uint64_t)m) o[row * w.n + col] = acc[i][j][r];
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
    hipLaunchKernelGGL(gemm_q4k_f16_kernel, dim3(wgs), dim3(kThreads), 0, s, w, m, a16, p.tiles_n, p.tiles_m,
                       p.splits, p.splits > 1 ? part : y);
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
