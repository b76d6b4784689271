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
//   1. activations -> planar Q8_K image in scratch: q8[m][K] (int8) and d[m][K/256] (f32).
//      From F32 x this is the same quantization as quantize_q8k (bit-identical q and d); from
//      caller-supplied Q8_K blocks it is a repack.
//   2. GEMM: a 128 (m) x 256 (n) output tile per 512-thread workgroup over one K-split of whole
//      super-blocks, in steps of 64 k.  Four waves issue the MFMAs (each a 64 x 128 sub-tile,
//      eight 32 x 32 accumulators) from one pair of F16 LDS tiles and, between them, convert
//      the next step's int8 activations into the other pair; the other four waves dequantize
//      the next step's 4-bit weights into it.  Activations travel as int8 (1 byte/element) and
//      are converted in the workgroup, because the L2 -> CU path, not the matrix cores, is the
//      scarce resource: each activation element is re-read by every n-tile.
//   3. with more than one K-split, partial tiles go to scratch and a reduction kernel adds
//      them in split order (deterministic).
//
// Conversions: a byte or nibble goes to F32 exactly (v_cvt_f32_ubyte), one F32 fma applies
// the scale (and the min), and v_cvt_pk_f16_f32 rounds two values to f16 (nearest even).
#include "oq_common.h"
#include "oq_layout.h"

namespace oq {

namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float float16v __attribute__((ext_vector_type(16)));

constexpr int kBM = 128, kBN = 256, kBK = 64;
constexpr int kThreads = 512;
constexpr uint64_t kMinK = 4096;
constexpr int kMaxSplits = 8;
constexpr int kLdsA = kBM * kBK;        // f16 elements per A tile buffer
constexpr int kLdsB = kBN * kBK;        // f16 elements per B tile buffer

// F16 tiles: row r holds 64 k as eight 16-byte chunks; logical chunk c sits at physical chunk
// c ^ ((r / 2) % 8), which keeps the MFMA operand reads and the conversion writes free of LDS
// bank conflicts without padding.
OQ_DEVICE int tile_off(int r, int c) { return r * kBK + 8 * (c ^ ((r >> 1) & 7)); }

// ---------------------------------------------------------------- activation images

// F32 x [m][K] -> planar Q8_K (one wave per 256-block; same arithmetic as quantize_q8k)
__global__ __launch_bounds__(256) void quantize_planar_kernel(const float* __restrict__ x, uint64_t nblocks,
                                                              uint64_t k, int8_t* __restrict__ q8,
                                                              float* __restrict__ dplane) {
    const int lane = threadIdx.x & 63;
    const uint64_t blk = blockIdx.x * 4ull + (threadIdx.x >> 6);
    if (blk >= nblocks) return;
    const float4 v = reinterpret_cast<const float4*>(x + blk * kQK)[lane];
    const Q8KLane r = quantize_q8k_block_wave(v, lane);
    *reinterpret_cast<uint32_t*>(q8 + blk * kQK + 4 * lane) = r.qword;
    if (lane == 0) dplane[blk] = r.d;
    (void)k;
}

// Q8_K blocks -> planar image (q and d copied unchanged)
__global__ __launch_bounds__(256) void repack_planar_kernel(const uint8_t* __restrict__ q8k, uint64_t nblocks,
                                                            int8_t* __restrict__ q8, float* __restrict__ dplane) {
    const int lane = threadIdx.x & 63;
    const uint64_t blk = blockIdx.x * 4ull + (threadIdx.x >> 6);
    if (blk >= nblocks) return;
    const uint8_t* b = q8k + blk * kQ8KBytes;
    *reinterpret_cast<uint32_t*>(q8 + blk * kQK + 4 * lane) = *reinterpret_cast<const uint32_t*>(b + 4 + 4 * lane);
    if (lane == 0) dplane[blk] = *reinterpret_cast<const float*>(b);
}

// ---------------------------------------------------------------- conversions

typedef float float2v __attribute__((ext_vector_type(2)));

// Hides a value from the optimizer, so that byte extractions below map onto v_cvt_f32_ubyte<i>.
OQ_DEVICE uint32_t opaque(uint32_t v) {
    asm volatile("" : "+v"(v));
    return v;
}

// two floats -> one dword of two f16 (round to nearest even, v_cvt_pk_f16_f32)
OQ_DEVICE uint32_t pack_f16(float a, float b) {
    const float2v v = {a, b};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, half2v));
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

constexpr int kRawB = kBN * 128;  // q4_K quants of one super-block for the tile's 256 weight rows

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

// ---------------------------------------------------------------- weight conversion
//
// Waves 4..7 (thread index u = tid - 256, 0..255) dequantize weight row u of each step (both
// 32-byte pieces of the step's 64-group).  The raw quants of super-block i+1 are loaded while
// super-block i is converted: slots 256 j + u (j = 0..7), in two halves of four.

struct QuantHalf {
    uint4 q[4];
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
#pragma unroll
    for (int j = 0; j < 4; ++j) l.q[j] = load_quant_slot(w, t, sb, 256u * (4 * h + j) + u);
}

OQ_DEVICE void store_quant_half(const QuantHalf& l, uint8_t* raw, int h, int u) {
#pragma unroll
    for (int j = 0; j < 4; ++j) *reinterpret_cast<uint4*>(raw + 16 * (256 * (4 * h + j) + u)) = l.q[j];
}

OQ_DEVICE uint4 load_header(const DeviceMatrix& w, const Tile& t, uint64_t sb, int u) {
    uint64_t n = t.n0 + u;
    n = n < w.n ? n : w.n - 1;
    return *reinterpret_cast<const uint4*>(w.base + n * w.pitch + 128 * (w.k / kQK) + 16 * sb);
}

// f16((d*sc)*q - dmin*m) for the 32 weights of one 16-byte chunk (piece P of group G of row r):
// low nibbles -> k = 16P + i (sub-block 2G), high nibbles -> k = 32 + 16P + i (sub-block 2G+1)
OQ_DEVICE void convert_quant_chunk(uint4 qv, float ds0, float dm0, float ds1, float dm1, _Float16* Bs, int r,
                                   int piece) {
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

template <int G>
OQ_DEVICE void convert_weights(uint4 hdr, const uint8_t* raw, _Float16* Bs, int u) {
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
#pragma unroll
    for (int p = 0; p < 2; ++p) {
        const uint4 qv = *reinterpret_cast<const uint4*>(raw + 16 * raw_slot(u, p, G));
        convert_quant_chunk(qv, ds0, dm0, ds1, dm1, Bs, u, p);
    }
}

// ---------------------------------------------------------------- MFMA waves
//
// Waves 0..3 (thread index v = tid, 0..255) each own a 64 (m) x 128 (n) sub-tile (2 x 4
// accumulators of 32 x 32) and convert activation row v/2, 32 k at 32 * (v%2), of each step.

struct Act32 {
    uint4 lo, hi;
};

OQ_DEVICE Act32 load_act(const int8_t* q8, const DeviceMatrix& w, int m, const Tile& t, uint32_t step, int v) {
    uint64_t row = t.m0 + (v >> 1);
    row = row < (uint64_t)m ? row : (uint64_t)m - 1;
    const int8_t* p = q8 + row * w.k + (uint64_t)t.sb0 * kQK + (uint64_t)step * kBK + 32 * (v & 1);
    Act32 a;
    a.lo = *reinterpret_cast<const uint4*>(p);
    a.hi = *reinterpret_cast<const uint4*>(p + 16);
    return a;
}

OQ_DEVICE float load_dx(const float* dplane, const DeviceMatrix& w, int m, const Tile& t, uint64_t sb, int v) {
    uint64_t row = t.m0 + (v >> 1);
    row = row < (uint64_t)m ? row : (uint64_t)m - 1;
    return dplane[row * (w.k / kQK) + sb];
}

// f16(d * q) of 32 int8 activations into the A tile
OQ_DEVICE void convert_act(const Act32& a, float dx, _Float16* As, int v) {
    const float c = -128.0f * dx;
    const uint32_t words[8] = {a.lo.x, a.lo.y, a.lo.z, a.lo.w, a.hi.x, a.hi.y, a.hi.z, a.hi.w};
    uint32_t h[16];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const uint2 r = convert4(opaque(words[j] ^ 0x80808080u), dx, c);  // bytes q + 128
        h[2 * j] = r.x;
        h[2 * j + 1] = r.y;
    }
    const int r = v >> 1, c0 = 4 * (v & 1);
#pragma unroll
    for (int j = 0; j < 4; ++j)
        *reinterpret_cast<uint4*>(As + tile_off(r, c0 + j)) = make_uint4(h[4 * j], h[4 * j + 1], h[4 * j + 2], h[4 * j + 3]);
}

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

// Workgroup barrier after this wave's LDS writes have completed.  Unlike __syncthreads() it does
// not wait for outstanding global loads (the prefetches in flight across the barrier).
OQ_DEVICE void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// grid: x = n-tile, y = m-tile, z = K-split.  Output: y (one split) or partial[z][m][n].
//
// Step s (64 k) is multiplied from tile buffer s%2 while buffer (s+1)%2 receives step s+1;
// all waves meet at one barrier per step (and two in the prologue), so every wave passes the
// same number of barriers.  Activations are loaded two steps ahead.  Weight pipeline for
// super-block i (steps 4i..4i+3): the raw quants of super-block i+1 are loaded at steps
// 4i-2 / 4i-1 and stored to the other raw buffer at steps 4i / 4i+1 (read from step 4i+3 on);
// headers and activation scales of super-block i+1 are loaded at step 4i.
__global__ __launch_bounds__(kThreads) void gemm_q4k_f16_kernel(DeviceMatrix w, int m, const int8_t* q8,
                                                               const float* dplane, uint32_t splits,
                                                               float* __restrict__ out) {
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
    const uint32_t nsbu = sb1 - t.sb0;   // >= 1: splits <= nsb
    const uint32_t last = 4 * nsbu - 1;  // last step
    auto step_of = [last](uint32_t s) { return s <= last ? s : last; };
    auto sb_of = [&](uint32_t i) { return (uint64_t)t.sb0 + (i < nsbu ? i : nsbu - 1); };

    if (wave < 4) {
        const int v = tid, wm = wave >> 1, wn = wave & 1;
        float16v acc[2][4] = {};
        float dx = load_dx(dplane, w, m, t, sb_of(0), v), dx_next;
        Act32 a0 = load_act(q8, w, m, t, 0, v);
        Act32 a1 = load_act(q8, w, m, t, step_of(1), v);
        lds_barrier();  // raw quants of super-block 0 stored
        convert_act(a0, dx, As[0], v);
        a0 = load_act(q8, w, m, t, step_of(2), v);
        lds_barrier();  // step 0 converted
        for (uint32_t i = 0; i < nsbu; ++i) {
            const uint32_t s = 4 * i;
            dx_next = load_dx(dplane, w, m, t, sb_of(i + 1), v);
            mma_step(As[0], Bs[0], wm, wn, lane, acc);
            convert_act(a1, dx, As[1], v);
            a1 = load_act(q8, w, m, t, step_of(s + 3), v);
            lds_barrier();
            mma_step(As[1], Bs[1], wm, wn, lane, acc);
            convert_act(a0, dx, As[0], v);
            a0 = load_act(q8, w, m, t, step_of(s + 4), v);
            lds_barrier();
            mma_step(As[0], Bs[0], wm, wn, lane, acc);
            convert_act(a1, dx, As[1], v);
            a1 = load_act(q8, w, m, t, step_of(s + 5), v);
            lds_barrier();
            dx = dx_next;
            mma_step(As[1], Bs[1], wm, wn, lane, acc);
            convert_act(a0, dx, As[0], v);
            a0 = load_act(q8, w, m, t, step_of(s + 6), v);
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
        return;
    }

    const int u = tid - 256;
    QuantHalf qa, qb;  // halves 0 and 1 of the next super-block's raw quants
    load_quant_half(qa, w, t, sb_of(0), 0, u);
    load_quant_half(qb, w, t, sb_of(0), 1, u);
    store_quant_half(qa, raw[0], 0, u);
    store_quant_half(qb, raw[0], 1, u);
    uint4 hdr = load_header(w, t, sb_of(0), u), hdr_next;
    lds_barrier();  // raw quants of super-block 0 stored
    convert_weights<0>(hdr, raw[0], Bs[0], u);
    load_quant_half(qa, w, t, sb_of(1), 0, u);
    load_quant_half(qb, w, t, sb_of(1), 1, u);
    lds_barrier();  // step 0 converted
    // Every iteration passes four barriers, as every MFMA-wave iteration does.
    for (uint32_t i = 0; i < nsbu; ++i) {
        const uint8_t* rc = raw[i & 1];
        uint8_t* rn = raw[(i + 1) & 1];
        // step 4i: convert 4i+1
        store_quant_half(qa, rn, 0, u);
        hdr_next = load_header(w, t, sb_of(i + 1), u);
        convert_weights<1>(hdr, rc, Bs[1], u);
        lds_barrier();
        // step 4i+1: convert 4i+2
        store_quant_half(qb, rn, 1, u);
        convert_weights<2>(hdr, rc, Bs[0], u);
        lds_barrier();
        // step 4i+2: convert 4i+3
        convert_weights<3>(hdr, rc, Bs[1], u);
        load_quant_half(qa, w, t, sb_of(i + 2), 0, u);
        lds_barrier();
        // step 4i+3: convert 4i+4 (first group of super-block i+1)
        hdr = hdr_next;
        convert_weights<0>(hdr, rn, Bs[0], u);
        load_quant_half(qb, w, t, sb_of(i + 2), 1, u);
        lds_barrier();
    }
}

// y[i] = sum over splits s (in order) of partial[s][i]
__global__ __launch_bounds__(256) void reduce_splits_kernel(const float* __restrict__ part, uint64_t count,
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
    uint64_t q8_bytes, d_bytes, part_bytes;
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
    p.q8_bytes = round256((uint64_t)m * w.k);
    p.d_bytes = round256((uint64_t)m * nsb * 4);
    p.part_bytes = p.splits > 1 ? (uint64_t)p.splits * m * w.n * 4 : 0;
    return p;
}

}  // namespace

bool gemm_mfma_supported(const DeviceMatrix& w, int m) {
    return w.type == 12 && m >= 16 && w.k >= kMinK && w.k % kQK == 0;
}

uint64_t gemm_scratch_bytes(const DeviceMatrix& w, int m) {
    const Plan p = make_plan(w, m);
    return p.q8_bytes + p.d_bytes + p.part_bytes;
}

hipError_t launch_gemm_q4k_mfma(const DeviceMatrix& w, int m, const float* x, const uint8_t* q8k, float* y,
                                void* scratch, hipStream_t s) {
    if (!gemm_mfma_supported(w, m) || (x == nullptr) == (q8k == nullptr)) return hipErrorNotSupported;
    const Plan p = make_plan(w, m);
    uint8_t* base = static_cast<uint8_t*>(scratch);
    int8_t* q8 = reinterpret_cast<int8_t*>(base);
    float* dplane = reinterpret_cast<float*>(base + p.q8_bytes);
    float* part = reinterpret_cast<float*>(base + p.q8_bytes + p.d_bytes);
    const uint64_t nblocks = (uint64_t)m * (w.k / kQK);
    const unsigned qgrid = (unsigned)((nblocks + 3) / 4);
    if (x) {
        hipLaunchKernelGGL(quantize_planar_kernel, dim3(qgrid), dim3(256), 0, s, x, nblocks, w.k, q8, dplane);
    } else {
        hipLaunchKernelGGL(repack_planar_kernel, dim3(qgrid), dim3(256), 0, s, q8k, nblocks, q8, dplane);
    }
    const dim3 grid(p.tiles_n, p.tiles_m, p.splits);
    hipLaunchKernelGGL(gemm_q4k_f16_kernel, grid, dim3(kThreads), 0, s, w, m, q8, dplane, p.splits,
                       p.splits > 1 ? part : y);
    if (p.splits > 1) {
        const uint64_t count = (uint64_t)m * w.n;
        uint64_t blocks = (count + 255) / 256;
        if (blocks > 4096) blocks = 4096;
        hipLaunchKernelGGL(reduce_splits_kernel, dim3((unsigned)blocks), dim3(256), 0, s, part, count, p.splits, y);
    }
    return hipGetLastError();
}

}  // namespace oq
