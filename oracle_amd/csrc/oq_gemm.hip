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
//   2. GEMM: a 128 (m) x 256 (n) output tile per 1024-thread workgroup over one K-split of
//      whole super-blocks, in steps of 64 k, double-buffered in LDS.  Eight waves issue the
//      MFMAs (each a 64 x 64 sub-tile, four 32 x 32 accumulators) from one pair of F16 tiles
//      while the other eight copy the next step's activations into the other pair and
//      dequantize the next step's 4-bit weights into it.  Two VALU-issuing waves per SIMD keep
//      the vector ALU at full rate (one wave alone issues at about half rate) and the matrix
//      cores run beside them.
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
constexpr int kThreads = 1024;
constexpr uint64_t kMinK = 4096;
constexpr int kMaxSplits = 8;
constexpr int kLdsA = kBM * kBK;    // f16 elements per A tile buffer
constexpr int kLdsB = kBN * kBK;    // f16 elements per B tile buffer
constexpr int kRawB = kBN * 128;    // q4_K quants of one super-block for the tile's 256 weight rows

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

// Raw quant slot c (16 bytes) of a super-block holds chunk (row c/8, piece ((c/4)%2) ^ h(row),
// group (c%4) ^ f(row)) with h(row) = (row/2)%2, f(row) = (row/4)%4.  Four consecutive slots
// are one 64-byte line of one weight row (the chunks of one piece, see oq_layout.h), so the
// global loads that fill the slots are fully coalesced; the swizzle makes the per-row
// read-back free of LDS bank conflicts.
OQ_DEVICE uint32_t raw_slot(uint32_t row, uint32_t piece, uint32_t g) {
    return 8 * row + 4 * (piece ^ ((row >> 1) & 1)) + (g ^ ((row >> 2) & 3));
}

// ---------------------------------------------------------------- converter waves
//
// Waves 8..15 (thread index u = tid - 512, 0..511):
//   activations: 16-byte chunks u and u + 512 of the step's 128 x 64 F16 tile (row c/8,
//                chunk c%8), copied from the F16 image;
//   weights:     row u % 256, piece u / 256 (32 weights) of the step's 64-group, dequantized
//                from the raw quants in LDS.
// The raw quants of super-block i+1 are loaded while super-block i is converted: slots
// 512 j + u (j = 0..3), in two halves of two.

struct QuantHalf {
    uint4 q0, q1;
};

OQ_DEVICE uint4 load_quant_slot(const DeviceMatrix& w, const Tile& t, uint64_t sb, uint32_t c) {
    const uint64_t nsb = w.k / kQK;
    const uint32_t row = c >> 3;
    const uint32_t piece = ((c >> 2) & 1) ^ ((row >> 1) & 1), g = (c & 3) ^ ((row >> 2) & 3);
    uint64_t n = t.n0 + row;
    n = n < w.n ? n : w.n - 1;
    return *reinterpret_cast<const uint4*>(w.base + n * w.pitch + 16 * perm_chunk(nsb, sb, g, piece));
}

OQ_DEVICE void load_quant_half(QuantHalf& l, const DeviceMatrix& w, const Tile& t, uint64_t sb, int h, int u) {
    l.q0 = load_quant_slot(w, t, sb, 512u * (2 * h) + u);
    l.q1 = load_quant_slot(w, t, sb, 512u * (2 * h + 1) + u);
}

OQ_DEVICE void store_quant_half(const QuantHalf& l, uint8_t* raw, int h, int u) {
    *reinterpret_cast<uint4*>(raw + 16 * (512 * (2 * h) + u)) = l.q0;
    *reinterpret_cast<uint4*>(raw + 16 * (512 * (2 * h + 1) + u)) = l.q1;
}

OQ_DEVICE uint4 load_header(const DeviceMatrix& w, const Tile& t, uint64_t sb, int u) {
    uint64_t n = t.n0 + (u & 255);
    n = n < w.n ? n : w.n - 1;
    return *reinterpret_cast<const uint4*>(w.base + n * w.pitch + 128 * (w.k / kQK) + 16 * sb);
}

struct Act {
    uint4 c0, c1;  // chunks u and u + 512 of one step's activation tile
};

OQ_DEVICE uint4 load_act_chunk(const _Float16* a16, const DeviceMatrix& w, int m, const Tile& t, uint32_t step,
                               uint32_t c) {
    uint64_t row = t.m0 + (c >> 3);
    row = row < (uint64_t)m ? row : (uint64_t)m - 1;
    return *reinterpret_cast<const uint4*>(a16 + row * w.k + (uint64_t)t.sb0 * kQK + (uint64_t)step * kBK +
                                           8 * (c & 7));
}

OQ_DEVICE Act load_act(const _Float16* a16, const DeviceMatrix& w, int m, const Tile& t, uint32_t step, int u) {
    Act a;
    a.c0 = load_act_chunk(a16, w, m, t, step, u);
    a.c1 = load_act_chunk(a16, w, m, t, step, u + 512);
    return a;
}

OQ_DEVICE void store_act(const Act& a, _Float16* As, int u) {
    *reinterpret_cast<uint4*>(As + tile_off(u >> 3, u & 7)) = a.c0;
    *reinterpret_cast<uint4*>(As + tile_off((u + 512) >> 3, u & 7)) = a.c1;
}

// Hides a value from the optimizer, so that the byte extractions below map onto
// v_cvt_f32_ubyte<i>.
OQ_DEVICE uint32_t opaque(uint32_t v) {
    asm volatile("" : "+v"(v));
    return v;
}

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

// f16((d*sc)*q - dmin*m) for the 32 weights of group G, piece P of this thread's weight row:
// low nibbles -> k = 16P + i (sub-block 2G), high nibbles -> k = 32 + 16P + i (sub-block 2G+1)
template <int G>
OQ_DEVICE void convert_weights(uint4 hdr, const uint8_t* raw, _Float16* Bs, int u) {
    const int row = u & 255, piece = u >> 8;
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
    const uint4 qv = *reinterpret_cast<const uint4*>(raw + 16 * raw_slot(row, piece, G));
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
    *reinterpret_cast<uint4*>(Bs + tile_off(row, c)) = make_uint4(lo[0], lo[1], lo[2], lo[3]);
    *reinterpret_cast<uint4*>(Bs + tile_off(row, c + 1)) = make_uint4(lo[4], lo[5], lo[6], lo[7]);
    *reinterpret_cast<uint4*>(Bs + tile_off(row, c + 4)) = make_uint4(hi[0], hi[1], hi[2], hi[3]);
    *reinterpret_cast<uint4*>(Bs + tile_off(row, c + 5)) = make_uint4(hi[4], hi[5], hi[6], hi[7]);
}

// ---------------------------------------------------------------- MFMA waves
//
// Waves 0..7 in a 2 (m) x 4 (n) grid, each a 64 x 64 sub-tile: 2 x 2 accumulators of 32 x 32.
OQ_DEVICE void mma_step(const _Float16* As, const _Float16* Bs, int wm, int wn, int lane, float16v (&acc)[2][2]) {
    const int ra = 64 * wm + (lane & 31), rb = 64 * wn + (lane & 31), h = lane >> 5;
#pragma unroll
    for (int ks = 0; ks < kBK / 16; ++ks) {
        half8 a[2], b[2];
#pragma unroll
        for (int i = 0; i < 2; ++i) a[i] = *reinterpret_cast<const half8*>(As + tile_off(ra + 32 * i, 2 * ks + h));
#pragma unroll
        for (int j = 0; j < 2; ++j) b[j] = *reinterpret_cast<const half8*>(Bs + tile_off(rb + 32 * j, 2 * ks + h));
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[i], b[j], acc[i][j], 0, 0, 0);
    }
}

// Workgroup barrier after this wave's LDS writes have completed.  Unlike __syncthreads() it does
// not wait for outstanding global loads (the prefetches in flight across the barrier).
OQ_DEVICE void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// grid: x = n-tile, y = m-tile, z = K-split.  Output: y (one split) or partial[z][m][n].
//
// Step s (64 k) is multiplied from tile buffer s%2 while buffer (s+1)%2 receives step s+1;
// all waves meet at one barrier per step (and two in the prologue), so every wave passes the
// same number of barriers.  Converter pipeline: activations two steps ahead; for super-block
// i (steps 4i..4i+3) the raw quants of super-block i+1 are loaded at steps 4i-2 / 4i-1 and
// stored to the other raw buffer at steps 4i / 4i+1 (read from step 4i+3 on), and its headers
// are loaded at step 4i.
__global__ __launch_bounds__(kThreads) void gemm_q4k_f16_kernel(DeviceMatrix w, int m, const _Float16* a16,
                                                               uint32_t splits, float* __restrict__ out) {
    __shared__ __align__(16) _Float16 tiles[2 * (kLdsA + kLdsB)];
    __shared__ __align__(16) uint8_t raw[2][kRawB];
    _Float16* const As[2] = {tiles, tiles + kLdsA};
    _Float16* const Bs[2] = {tiles + 2 * kLdsA, tiles + 2 * kLdsA + kLdsB};
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t nsb = (uint32_t)(w.k / kQK);
    const uint32_t z = blockIdx.z;
    Tile t;
    t.n0 = (uint64_t)blockIdx.x * kBN;
    t.m0 = (uint64_t)blockIdx.y * kBM;
    t.sb0 = (uint32_t)((uint64_t)z * nsb / splits);
    const uint32_t sb1 = (uint32_t)((uint64_t)(z + 1) * nsb / splits);
    const uint32_t nsbu = sb1 - t.sb0;  // >= 1: splits <= nsb

    if (wave < 8) {
        const int wm = wave >> 2, wn = wave & 3;
        float16v acc[2][2] = {};
        lds_barrier();  // raw quants of super-block 0 stored
        lds_barrier();  // step 0 converted
        for (uint32_t i = 0; i < nsbu; ++i) {
            mma_step(As[0], Bs[0], wm, wn, lane, acc);
            lds_barrier();
            mma_step(As[1], Bs[1], wm, wn, lane, acc);
            lds_barrier();
            mma_step(As[0], Bs[0], wm, wn, lane, acc);
            lds_barrier();
            mma_step(As[1], Bs[1], wm, wn, lane, acc);
            lds_barrier();
        }
        // result register r of lane l: row 8*(r/4) + 4*(l/32) + r%4, column l%32
        float* o = out + (uint64_t)z * (uint64_t)m * w.n;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const uint64_t col = t.n0 + 64 * wn + 32 * j + (lane & 31);
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
        return;
    }

    const int u = tid - 512;
    const uint32_t last = 4 * nsbu - 1;  // last step
    auto step_of = [last](uint32_t s) { return s <= last ? s : last; };
    auto sb_of = [&](uint32_t i) { return (uint64_t)t.sb0 + (i < nsbu ? i : nsbu - 1); };
    QuantHalf qa, qb;  // halves 0 and 1 of the next super-block's raw quants
    load_quant_half(qa, w, t, sb_of(0), 0, u);
    load_quant_half(qb, w, t, sb_of(0), 1, u);
    uint4 hdr = load_header(w, t, sb_of(0), u), hdr_next;
    Act a0 = load_act(a16, w, m, t, 0, u);
    Act a1 = load_act(a16, w, m, t, step_of(1), u);
    store_quant_half(qa, raw[0], 0, u);
    store_quant_half(qb, raw[0], 1, u);
    lds_barrier();  // raw quants of super-block 0 stored
    store_act(a0, As[0], u);
    convert_weights<0>(hdr, raw[0], Bs[0], u);
    a0 = load_act(a16, w, m, t, step_of(2), u);
    load_quant_half(qa, w, t, sb_of(1), 0, u);
    load_quant_half(qb, w, t, sb_of(1), 1, u);
    lds_barrier();  // step 0 converted
    // Every iteration passes four barriers, as every MFMA-wave iteration does.
    for (uint32_t i = 0; i < nsbu; ++i) {
        const uint32_t s = 4 * i;
        const uint8_t* rc = raw[i & 1];
        uint8_t* rn = raw[(i + 1) & 1];
        // step s: convert s+1
        store_quant_half(qa, rn, 0, u);
        hdr_next = load_header(w, t, sb_of(i + 1), u);
        store_act(a1, As[1], u);
        convert_weights<1>(hdr, rc, Bs[1], u);
        a1 = load_act(a16, w, m, t, step_of(s + 3), u);
        lds_barrier();
        // step s+1: convert s+2
        store_quant_half(qb, rn, 1, u);
        store_act(a0, As[0], u);
        convert_weights<2>(hdr, rc, Bs[0], u);
        a0 = load_act(a16, w, m, t, step_of(s + 4), u);
        lds_barrier();
        // step s+2: convert s+3
        store_act(a1, As[1], u);
        convert_weights<3>(hdr, rc, Bs[1], u);
        a1 = load_act(a16, w, m, t, step_of(s + 5), u);
        load_quant_half(qa, w, t, sb_of(i + 2), 0, u);
        lds_barrier();
        // step s+3: convert s+4 (first group of super-block i+1)
        hdr = hdr_next;
        store_act(a0, As[0], u);
        convert_weights<0>(hdr, rn, Bs[0], u);
        a0 = load_act(a16, w, m, t, step_of(s + 6), u);
        load_quant_half(qb, w, t, sb_of(i + 2), 1, u);
        lds_barrier();
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
    const dim3 grid(p.tiles_n, p.tiles_m, p.splits);
    hipLaunchKernelGGL(gemm_q4k_f16_kernel, grid, dim3(kThreads), 0, s, w, m, a16, p.splits,
                       p.splits > 1 ? part : y);
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
