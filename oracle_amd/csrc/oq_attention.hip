// Full-attention decode for gfx950: RoPE / MRoPE, the attention block's per-head preparation and
// single-token GQA attention over an F32 KV cache in HBM.
//
// Attention (reference_kernels.cpp:127-195) is split over the token axis, flash-decoding style:
//   chunk kernel   one workgroup per (KV head g, subgroup, chunk of tokens), 4 waves.  The
//                  query heads of g (q_heads / kv_heads of them) share each key and value row; up
//                  to 8 of them are one subgroup, whose workgroups hold every head's query slices
//                  in registers, so K and V are read from HBM once per step for groups of up to
//                  8 heads.  A larger group is split into equal subgroups of at most 8 heads
//                  (16 heads: two of 8; 12: two of 6), each reading the group's rows again.
//                  scores: 16 lanes per token, each lane holding D/16 key values (four 16-lane
//                    groups per wave, 256 contiguous bytes per group and load); the rep query
//                    heads' matching slices sit in registers; F32 products reduced over the 16
//                    lanes; s = dot * 1/sqrt(D) kept in LDS
//                  softmax: per head the chunk's max m_c, p = exp(s - m_c) in place, l_c = sum p
//                  values: each wave takes every fourth token, lane i owning D/64 value columns,
//                    o[h] += p[h][t] * v_t for the rep heads; the four waves' sums are added in LDS
//                  -> o_c [rep][D], (m_c, l_c) [rep] for the chunk
//   merge kernel   one workgroup per (query head, 64 output columns), 16 chunk groups x 16 float4
//                  columns, every load issued before the first use: the largest chunk maximum M
//                  (over the groups through LDS), then each chunk weighted on its own,
//                  out = sum_c e^(m_c - M) o_c / sum_c e^(m_c - M) l_c, the groups' sums added in
//                  LDS (no running rescale: one exp per chunk and no chain of them).  For the
//                  decoder block also the output gate (gate_s = sigmoid(gate), gated = out * gate_s,
//                  qwen35_block.cpp:734-741)
// The reference sums the dot products and the softmax denominator in double and the weighted
// values in F32 in token order; here everything is F32 in the order above, so results agree
// within a small multiple of F32 rounding (tested against 1e-4 of sum_t p_t |v_t|).
//
// The append (KvCache::append, hybrid_cache.cpp:154-169) is folded in: when new_k / new_v are
// given, the workgroup whose chunk holds the new token reads it from there and stores it into
// cache row T - 1; nothing else reads that row during the step.
//
// A cache of binary16 elements (no counterpart in the reference, whose cache is F32) halves the
// bytes every step reads.  Its rows are the F32 rows rounded to nearest even on append, and
// attention reads what is stored, the new token's row included: a small launch stores the new
// row rounded before the chunk kernel (which then reads every row from the cache), and with the
// block's preparation folded in, the new key is scored rounded and stored rounded by the
// workgroup that prepares it.  Each lane loads the same elements as from an F32 cache (4 of a key
// row, D / 64 of a value row), half the bytes, kept raw in registers until used.
//
// For the decoder block the per-head preparation (qwen35_block.cpp:671-711: RMSNorm of each query
// head with q_norm and of each key head with k_norm, then the rotation) is folded in as well, so
// the block has no separate preparation launch: every chunk workgroup of KV head g normalises and
// rotates g's rep query heads itself, in LDS, while its first key rows are in flight, and the
// workgroup whose chunk holds the new token also prepares the new key, scores that token from LDS
// (the key loads issued before it was ready skip it) and stores it into the cache.
#include <type_traits>

#include "oq_common.h"

namespace oq {

namespace {

constexpr int kAttnWaves = 4;
constexpr int kAttnThreads = kAttnWaves * 64;
constexpr uint32_t kTokStep = kAttnWaves * 4;  // tokens per workgroup pass in the score phase
constexpr uint32_t kMaxChunk = 1024;
constexpr int kMergeGroups = 16;  // chunk groups of the merge kernel

struct ChunkArgs {
    const float* q;       // [Hq][D]
    void* keys;           // [capacity][Hkv][D] of the cache's element type
    void* values;         // [capacity][Hkv][D]
    const float* new_k;   // [Hkv][D] or null
    const float* new_v;
    uint32_t T, Hkv, rep, chunk, nchunks;
    uint32_t rep_all;     // query heads per KV head
    uint32_t nsub;        // subgroups per KV head, of rep = rep_all / nsub query heads each
    // consecutive tokens of one launch: token i attends over T + i rows, its queries at q + i *
    // q_tok_stride and its partials at part_o / part_ml + i * part_tok_stride (one token: 1, 0, 0)
    uint32_t tokens;
    uint64_t q_tok_stride, part_tok_stride;
    // a workgroup serves tpw consecutive tokens with `heads` query heads each: its query rows are
    // (token i, head j) in order, row i * heads + j, rep = tpw * heads of them (one token: 1, rep)
    uint32_t tpw, heads;
    float scale;
    float* part_o;        // [Hq][D/64][nchunks][64]: one head slice's chunks contiguous
    float* part_ml;       // [Hq][nchunks][2]
    // the block's preparation (PREP kernels); new_k is null and new_v the value projection
    const float* qfull;   // [Hq][2D]: query values, then the output gate
    const float* kp;      // [Hkv][D] key projection
    const float* q_norm;  // [D]
    const float* k_norm;  // [D]
    float eps;
    RopeParams rope;
    float* qcur;          // [Hq][D], written by each subgroup's chunk 0
    float* kcur;          // [Hkv][D], written by subgroup 0's chunk holding the new token
    uint32_t stage;       // float offset of the preparation's LDS: [rep + 1][D] rows, cos/sin [2][128]
};

struct MergeArgs {
    const float* part_o;
    const float* part_ml;
    uint32_t nchunks;     // chunks of the partials' layout (the last token's)
    // consecutive tokens (as ChunkArgs): token i's T0 + i rows in chunks of `chunk`, its partials at
    // + i * part_tok_stride, out / gate_s / gated at + i * out_tok_stride, gate at + i * gate_tok_stride
    uint32_t tokens, T0, chunk;
    uint64_t part_tok_stride, out_tok_stride, gate_tok_stride;
    float* out;           // [Hq][D]
    const float* gate;    // gate of head h at gate + h * gate_stride, or null
    uint32_t gate_stride;
    float* gate_s;        // [Hq][D]
    float* gated;         // [Hq][D]
};

template <int N>
struct Vec;
template <>
struct Vec<1> {
    using type = float;
    OQ_DEVICE static void unpack(type v, float* o) { o[0] = v; }
};
template <>
struct Vec<2> {
    using type = float2;
    OQ_DEVICE static void unpack(type v, float* o) {
        o[0] = v.x;
        o[1] = v.y;
    }
};
template <>
struct Vec<4> {
    using type = float4;
    OQ_DEVICE static void unpack(type v, float* o) {
        o[0] = v.x;
        o[1] = v.y;
        o[2] = v.z;
        o[3] = v.w;
    }
};

// Binary16 values of a value row per lane (VW of them) as raw bits, and their F32 values
template <int N>
struct HalfVec;
template <>
struct HalfVec<1> {
    using type = uint16_t;
    OQ_DEVICE static void unpack(type v, float* o) { o[0] = (float)__builtin_bit_cast(_Float16, v); }
};
template <>
struct HalfVec<2> {
    using type = uint32_t;
    OQ_DEVICE static void unpack(type v, float* o) {
        o[0] = (float)__builtin_bit_cast(_Float16, (uint16_t)(v & 0xFFFFu));
        o[1] = (float)__builtin_bit_cast(_Float16, (uint16_t)(v >> 16));
    }
};
template <>
struct HalfVec<4> {
    using type = uint2;
    OQ_DEVICE static void unpack(type v, float* o) {
        HalfVec<2>::unpack(v.x, o);
        HalfVec<2>::unpack(v.y, o + 2);
    }
};

// Loads of cache rows of element type KT.  A lane of a 16-lane key group holds NV = D / 64 pieces
// of 4 key elements, piece j being the row's 4-element piece q_index(j, l16) (the query slices
// in registers follow the same map); the pieces arrive in NK loads of type K, kept raw until
// unpack_k converts them.  V holds a lane's VW value elements as loaded, unpack_v converts them.
// round gives the value a cache element holds for an F32 value, store the element itself.
template <typename KT, int VW>
struct KvIo;
template <int VW>
struct KvIo<float, VW> {
    static constexpr int NV = VW, NK = VW;  // one 16-byte load per piece
    using K = float4;
    using V = typename Vec<VW>::type;
    OQ_DEVICE static uint32_t q_index(int j, int l16) { return 16u * (uint32_t)j + (uint32_t)l16; }
    OQ_DEVICE static K load_k(const float* row, int j, int l16) {
        return load_stream(reinterpret_cast<const float4*>(row) + q_index(j, l16));
    }
    OQ_DEVICE static void unpack_k(const K (&k)[NK], float4 (&f)[NV]) {
#pragma unroll
        for (int j = 0; j < NK; ++j) f[j] = k[j];
    }
    OQ_DEVICE static V load_v(const float* row, int lane) { return load_stream(reinterpret_cast<const V*>(row) + lane); }
    OQ_DEVICE static void unpack_v(V v, float* o) { Vec<VW>::unpack(v, o); }
    OQ_DEVICE static float round(float x) { return x; }
    OQ_DEVICE static float store(float x) { return x; }
};
// binary16: rows of 128 elements or more load 8 halves (16 bytes) per lane, two pieces per load
// (pieces 2i and 2i + 1 = 4-element pieces 2 (16 i + l16) and + 1); rows of 64, 4 halves
template <int VW>
struct KvIo<_Float16, VW> {
    static constexpr bool kWide = VW >= 2;
    static constexpr int NV = VW, NK = kWide ? VW / 2 : VW;
    using K = std::conditional_t<kWide, uint4, uint2>;
    using V = typename HalfVec<VW>::type;
    OQ_DEVICE static uint32_t q_index(int j, int l16) {
        return kWide ? 2u * (16u * (uint32_t)(j >> 1) + (uint32_t)l16) + (uint32_t)(j & 1) : 16u * (uint32_t)j + (uint32_t)l16;
    }
    OQ_DEVICE static K load_k(const _Float16* row, int i, int l16) {
        return load_stream(reinterpret_cast<const K*>(row) + 16 * i + l16);
    }
    OQ_DEVICE static void unpack_k(const K (&k)[NK], float4 (&f)[NV]) {
#pragma unroll
        for (int i = 0; i < NK; ++i) {
            float o[8];
            if constexpr (kWide) {
                HalfVec<4>::unpack(make_uint2(k[i].x, k[i].y), o);
                HalfVec<4>::unpack(make_uint2(k[i].z, k[i].w), o + 4);
                f[2 * i] = make_float4(o[0], o[1], o[2], o[3]);
                f[2 * i + 1] = make_float4(o[4], o[5], o[6], o[7]);
            } else {
                HalfVec<4>::unpack(k[i], o);
                f[i] = make_float4(o[0], o[1], o[2], o[3]);
            }
        }
    }
    OQ_DEVICE static V load_v(const _Float16* row, int lane) { return load_stream(reinterpret_cast<const V*>(row) + lane); }
    OQ_DEVICE static void unpack_v(V v, float* o) { HalfVec<VW>::unpack(v, o); }
    OQ_DEVICE static float round(float x) { return (float)(_Float16)x; }
    OQ_DEVICE static _Float16 store(float x) { return (_Float16)x; }
};

// The new token's key and value rows [Hkv * D] stored into an F16 cache (rounded to nearest even)
// before an attention launch over it; either source may be null (not stored).
__global__ __launch_bounds__(256) void kv_append_f16_kernel(const float* __restrict__ k, const float* __restrict__ v,
                                                            _Float16* __restrict__ kd, _Float16* __restrict__ vd,
                                                            uint32_t n) {
    const uint32_t i = blockIdx.x * 256u + threadIdx.x;
    if (i >= n) return;
    if (k != nullptr) kd[i] = (_Float16)k[i];
    if (v != nullptr) vd[i] = (_Float16)v[i];
}

// F32 rows -> an F16 cache's elements, rounded to nearest even (oq_kv_cache_load)
__global__ __launch_bounds__(256) void f32_to_f16_kernel(const float* __restrict__ src, _Float16* __restrict__ dst,
                                                         uint64_t n) {
    const uint64_t stride = (uint64_t)gridDim.x * 256u;
    for (uint64_t i = (uint64_t)blockIdx.x * 256u + threadIdx.x; i < n; i += stride) dst[i] = (_Float16)src[i];
}

// cos and sin of frequency f's angle, as apply_qwen35_rope (reference_kernels.cpp:105-115):
// base^(2f/R) and the angle in double, the coordinate chosen as position_for_frequency (:28-40)
OQ_DEVICE void rope_cs(uint32_t f, const RopeParams& p, float& c, float& s) {
    const double exponent = (2.0 * (double)f) / (double)p.rotary_dim;
    const double inv_freq = 1.0 / pow((double)p.base, exponent);
    uint64_t coord = p.pos[0];
    if (f % 3u == 1u && f / 3u < p.sec1) coord = p.pos[1];
    else if (f % 3u == 2u && f / 3u < p.sec2) coord = p.pos[2];
    const double angle = (double)coord * inv_freq;
    c = (float)cos(angle);
    s = (float)sin(angle);
}

OQ_DEVICE void rotate_pair(float* x, uint32_t f, uint32_t half, float c, float s) {
#pragma clang fp contract(off)
    const float a = x[f], b = x[half + f];
    x[f] = a * c - b * s;
    x[half + f] = b * c + a * s;
}

// One row of the block's preparation in wave registers (lane i holding elements i*VW ..): the
// RMSNorm of rms_norm_rows (qwen35_block.cpp:161-189, sum of squares in double; called at :691-698)
// with weight w, written to LDS row y for the rotation
template <int D>
OQ_DEVICE void prep_row_norm(const float* x, const float* w, float eps, int lane, float* y) {
#pragma clang fp contract(off)
    constexpr int VW = D / 64;
    double ss = 0.0;
#pragma unroll
    for (int e = 0; e < VW; ++e) ss += (double)x[e] * (double)x[e];
    ss = wave_sum_f64(ss);
    const float inv = (float)(1.0 / sqrt(ss / (double)D + (double)eps));
#pragma unroll
    for (int e = 0; e < VW; ++e) y[lane * VW + e] = x[e] * inv * w[e];
}

// Both phases run in blocks of NB passes (keys) or NB groups (values); every block but the last
// requests the next block's rows as it consumes its own, and the last requests nothing.  ONE: the
// chunk fits the NB passes in flight (chunk <= 16 NB tokens), so the last block is the only one.
template <typename KT, int D, int REP, int NB, bool PREP, bool ONE>
__global__ __launch_bounds__(kAttnThreads) void attention_chunk_kernel(ChunkArgs a) {
    constexpr int NV = D / 64;  // 4-element pieces of one key row per lane (16 lanes per row)
    constexpr int VW = D / 64;  // value columns per lane (64 lanes per row)
    using IO = KvIo<KT, VW>;
    using VT = typename IO::V;
    KT* const keys = static_cast<KT*>(a.keys);
    KT* const values = static_cast<KT*>(a.values);
    extern __shared__ __align__(16) float lds[];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t tpw = a.tpw > 0 ? a.tpw : 1u;
    const uint32_t heads = a.tpw > 0 ? a.heads : a.rep;
    const uint32_t per_tg = a.Hkv * a.nsub * a.nchunks;
    const uint32_t tg = blockIdx.x / per_tg;  // the workgroup's group of tokens
    const uint32_t bid = blockIdx.x - tg * per_tg;
    const uint32_t grp = bid / a.nchunks;  // (KV head, subgroup)
    const uint32_t c = bid - grp * a.nchunks;
    const uint32_t g = grp / a.nsub, sub = grp - g * a.nsub;
    const uint64_t h0 = (uint64_t)g * a.rep_all + (uint64_t)sub * heads;  // the subgroup's first query head
    const uint32_t t0 = tg * tpw;                                        // the group's first token
    const uint32_t ntok = min(tpw, max(a.tokens, 1u) - t0);
    const uint32_t T = a.T + t0 + ntok - 1;  // the rows of the group's last token
    const uint32_t c0 = c * a.chunk;
    if (c0 >= T) return;  // a chunk past every token's rows (the whole workgroup)
    const uint32_t c1 = min(c0 + a.chunk, T);
    const uint32_t n = c1 - c0;
    const uint32_t rep = ntok * heads;  // query rows
    const uint32_t last = T - 1;
    // row r: token t0 + r / heads (rows a.T + that token), query head h0 + r % heads.  A row whose
    // token's rows end before c1 scores -inf past them; a chunk past them all yields partials its
    // token's merge never reads (it reads the chunks up to its rows only).
    auto row_tok = [&](uint32_t r) { return t0 + r / heads; };
    auto row_head = [&](uint32_t r) { return h0 + (r % heads); };
    float* sc = lds;  // [rep][chunk] scores, then probabilities

    // rows t of the cache; the new token's rows from new_k / new_v when given (an F32 cache only:
    // an F16 cache holds them before the launch)
    auto key_row = [&](uint32_t t) -> const KT* {
        if constexpr (std::is_same_v<KT, float>) {
            if (a.new_k != nullptr && t == last) return a.new_k + (uint64_t)g * D;
        }
        return keys + ((uint64_t)t * a.Hkv + g) * D;
    };
    auto value_row = [&](uint32_t t) -> const KT* {
        if constexpr (std::is_same_v<KT, float>) {
            if (a.new_v != nullptr && t == last) return a.new_v + (uint64_t)g * D;
        }
        return values + ((uint64_t)t * a.Hkv + g) * D;
    };

    // the append: subgroup 0's chunk holding the new token stores its key and value row
    if (a.new_k != nullptr && c1 == T && sub == 0) {
        for (uint32_t i = threadIdx.x; i < (uint32_t)D; i += kAttnThreads) {
            keys[((uint64_t)last * a.Hkv + g) * D + i] = IO::store(a.new_k[(uint64_t)g * D + i]);
            values[((uint64_t)last * a.Hkv + g) * D + i] = IO::store(a.new_v[(uint64_t)g * D + i]);
        }
    }

    // ---- scores: NB passes of 16 tokens in flight per wave, buffers rotated by unrolling (a copy
    // between buffers would wait for the loads it copies)
    const int l16 = lane & 15;
    float4 qr[REP][NV];
    // the preparation's rows: query heads of g as rows 0 .. rep-1, the new key as row rep; wave w
    // takes rows w, w + 4, ..  Their loads go out before the key rows, so waiting for them does not
    // wait for the keys.
    constexpr int kPrepRows = PREP ? (REP + kAttnWaves) / kAttnWaves : 1;
    const bool holds_new = c1 == T;
    const uint32_t prep_rows = rep + (holds_new ? 1u : 0u);
    float px[kPrepRows][VW], pw[kPrepRows][VW];
    if constexpr (PREP) {
#pragma unroll
        for (int r = 0; r < kPrepRows; ++r) {
            const uint32_t row = (uint32_t)wave + (uint32_t)r * kAttnWaves;
            if (row < prep_rows) {
                const bool is_q = row < rep;
                const float* src = is_q ? a.qfull + (h0 + row) * 2 * D : a.kp + (uint64_t)g * D;
                const float* w = is_q ? a.q_norm : a.k_norm;
                Vec<VW>::unpack(*reinterpret_cast<const typename Vec<VW>::type*>(src + lane * VW), px[r]);
#pragma unroll
                for (int e = 0; e < VW; ++e) pw[r][e] = w[lane * VW + e];
            }
        }
    } else {
#pragma unroll
        for (int h = 0; h < REP; ++h) {
            const uint32_t hh = (uint32_t)h < rep ? (uint32_t)h : 0u;
            const float4* qp = reinterpret_cast<const float4*>(a.q + (uint64_t)row_tok(hh) * a.q_tok_stride + row_head(hh) * D);
#pragma unroll
            for (int j = 0; j < NV; ++j) qr[h][j] = qp[IO::q_index(j, l16)];
        }
    }
    const uint32_t first = c0 + (uint32_t)wave * 4u;  // this wave's first pass (wave-uniform)
    auto load_keys = [&](typename IO::K (&dst)[IO::NK], uint32_t pass_base) {
        const uint32_t t = pass_base + (uint32_t)(lane >> 4);
        const KT* kp = key_row(t < c1 ? t : c1 - 1);
#pragma unroll
        for (int j = 0; j < IO::NK; ++j) dst[j] = IO::load_k(kp, j, l16);
    };
    {
        typename IO::K kb[NB][IO::NK];
#pragma unroll
        for (int b = 0; b < NB; ++b) load_keys(kb[b], first + (uint32_t)b * kTokStep);
        if constexpr (PREP) {
            // normalise (each wave its rows), then rotate (the workgroup over every row's frequency
            // pairs), while the key rows arrive
            float* stage = lds + a.stage;
            float* rc = stage + (rep + 1) * D;  // cos [128], sin [128]
            const uint32_t half = a.rope.rotary_dim / 2;
            if (threadIdx.x < half) rope_cs(threadIdx.x, a.rope, rc[threadIdx.x], rc[128 + threadIdx.x]);
#pragma unroll
            for (int r = 0; r < kPrepRows; ++r) {
                const uint32_t row = (uint32_t)wave + (uint32_t)r * kAttnWaves;
                if (row < prep_rows) prep_row_norm<D>(px[r], pw[r], a.eps, lane, stage + row * D);
            }
            __syncthreads();
            for (uint32_t i = threadIdx.x; i < prep_rows * half; i += kAttnThreads) {
                const uint32_t row = i / half, f = i - row * half;
                rotate_pair(stage + row * D, f, half, rc[f], rc[128 + f]);
            }
            __syncthreads();
#pragma unroll
            for (int h = 0; h < REP; ++h) {
                const uint32_t hh = (uint32_t)h < rep ? (uint32_t)h : 0u;
#pragma unroll
                for (int j = 0; j < NV; ++j) qr[h][j] = *reinterpret_cast<const float4*>(stage + hh * D + 4 * IO::q_index(j, l16));
            }
            // the trace's copies, and the append of the new key and value rows
            if (c == 0 && a.qcur != nullptr) {
                for (uint32_t i = threadIdx.x; i < rep * D; i += kAttnThreads) a.qcur[h0 * D + i] = stage[i];
            }
            if (holds_new && sub == 0) {
                for (uint32_t i = threadIdx.x; i < (uint32_t)D; i += kAttnThreads) {
                    const float k = stage[rep * D + i];
                    if (a.kcur != nullptr) a.kcur[(uint64_t)g * D + i] = k;
                    keys[((uint64_t)last * a.Hkv + g) * D + i] = IO::store(k);
                    // (an F16 cache's value row was stored before the launch: new_v is null)
                    if (a.new_v != nullptr) values[((uint64_t)last * a.Hkv + g) * D + i] = IO::store(a.new_v[(uint64_t)g * D + i]);
                }
            }
        }
        auto score_block = [&](uint32_t base, auto reload) {
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                const uint32_t pb = base + (uint32_t)b * kTokStep;
                const uint32_t t = pb + (uint32_t)(lane >> 4);
                float acc[REP];
                float4 kf[NV];
                IO::unpack_k(kb[b], kf);
#pragma unroll
                for (int h = 0; h < REP; ++h) {
                    float sum = 0.0f;
#pragma unroll
                    for (int j = 0; j < NV; ++j) {
                        sum += qr[h][j].x * kf[j].x;
                        sum += qr[h][j].y * kf[j].y;
                        sum += qr[h][j].z * kf[j].z;
                        sum += qr[h][j].w * kf[j].w;
                    }
                    acc[h] = row16_sum(sum);
                }
                // (with the preparation folded in, the new token's cache row was loaded before
                // it was written: its score comes from LDS below)
                if (t < c1 && (uint32_t)l16 < rep && !(PREP && t == last)) {
                    float v = acc[0];
#pragma unroll
                    for (int h = 1; h < REP; ++h) v = l16 == h ? acc[h] : v;
                    const uint32_t lim = a.T + row_tok((uint32_t)l16);  // rows of the row's token
                    sc[(uint32_t)l16 * a.chunk + (t - c0)] = t < lim ? v * a.scale : -INFINITY;
                }
                if constexpr (decltype(reload)::value) load_keys(kb[b], pb + NB * kTokStep);
            }
        };
        uint32_t base = first;
        if constexpr (!ONE) {
            for (; base + NB * kTokStep < c1; base += NB * kTokStep) score_block(base, std::true_type{});
        }
        if (base < c1) score_block(base, std::false_type{});
    }
    if constexpr (PREP) {
        if (holds_new) {
            const float* stage = lds + a.stage;
            const float* kn = stage + rep * D;
            for (uint32_t h = (uint32_t)wave; h < rep; h += kAttnWaves) {
                float s = 0.0f;
#pragma unroll
                for (int e = 0; e < VW; ++e) s += stage[h * D + (uint32_t)lane * VW + e] * IO::round(kn[(uint32_t)lane * VW + e]);
                s = wave_sum(s);
                if (lane == 0) sc[h * a.chunk + (last - c0)] = s * a.scale;
            }
        }
    }
    // this wave's first value rows go out before the softmax (they do not depend on it): NB groups
    // of four rows, rotated like the keys.  Over chunks longer than the passes in flight, a binary16
    // row of 128 or 256 values is loaded 8 values (16 bytes) per lane: D / 8 lanes per row,
    // TPI = 512 / D of the group's rows per load (lane slot s takes row 4 (v TPI + s) of the group
    // in load v), the slots' sums added at the end (32768 cached rows: 36.5 -> 31.8 us per step);
    // other rows one per load, VW values per lane (short chunks measured 0.25 us faster so).
    constexpr bool kWideV = std::is_same_v<KT, _Float16> && D >= 128 && !ONE;
    constexpr int TPI = kWideV ? 512 / D : 1;  // rows per value load
    constexpr int VL = 4 / TPI;                // value loads per group of four rows
    constexpr int VE = kWideV ? 8 : VW;        // value columns per lane
    using VLT = std::conditional_t<kWideV, uint4, VT>;
    const uint32_t vslot = kWideV ? (uint32_t)lane / (uint32_t)(D / 8) : 0u;
    const uint32_t vcol = kWideV ? ((uint32_t)lane % (uint32_t)(D / 8)) * 8u : (uint32_t)lane * VW;
    VLT vb[NB][VL];
    auto load_values = [&](VLT (&dst)[VL], uint32_t i0) {
#pragma unroll
        for (int v = 0; v < VL; ++v) {
            const uint32_t i = i0 + ((uint32_t)v * TPI + vslot) * kAttnWaves;
            const KT* row = value_row(c0 + (i < n ? i : n - 1));
            if constexpr (kWideV) {
                dst[v] = load_stream(reinterpret_cast<const uint4*>(row + vcol));
            } else {
                dst[v] = IO::load_v(row, lane);
            }
        }
    };
    constexpr uint32_t kGroup = 4u * kAttnWaves;  // tokens per value group of the workgroup
#pragma unroll
    for (int b = 0; b < NB; ++b) load_values(vb[b], (uint32_t)wave + (uint32_t)b * kGroup);
    __syncthreads();

    // ---- softmax over the chunk, one wave per head
    for (uint32_t h = (uint32_t)wave; h < rep; h += kAttnWaves) {
        float* sh = sc + h * a.chunk;
        float m = -INFINITY;
        for (uint32_t i = (uint32_t)lane; i < n; i += 64) m = fmaxf(m, sh[i]);
        m = wave_max(m);
        float l = 0.0f;
        for (uint32_t i = (uint32_t)lane; i < n; i += 64) {
            const float p = expf(sh[i] - m);
            sh[i] = p;
            l += p;
        }
        l = wave_sum(l);
        if (lane == 0) {
            float* ml = a.part_ml + (uint64_t)row_tok(h) * a.part_tok_stride + (row_head(h) * a.nchunks + c) * 2;
            ml[0] = m;
            ml[1] = l;
        }
    }
    __syncthreads();

    // ---- weighted values: wave w takes tokens c0 + w, c0 + w + 4, ...
    float o[REP][VE];
#pragma unroll
    for (int h = 0; h < REP; ++h)
#pragma unroll
        for (int e = 0; e < VE; ++e) o[h][e] = 0.0f;
    auto value_block = [&](uint32_t i0, auto reload) {
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            const uint32_t ib = i0 + (uint32_t)b * kGroup;
#pragma unroll
            for (int u = 0; u < VL; ++u) {
                const uint32_t i = ib + ((uint32_t)u * TPI + vslot) * kAttnWaves;
                // rows past the chunk are clamped loads with weight 0
                const uint32_t ic = i < n ? i : n - 1;
                float v[VE];
                if constexpr (kWideV) {
                    HalfVec<4>::unpack(make_uint2(vb[b][u].x, vb[b][u].y), v);
                    HalfVec<4>::unpack(make_uint2(vb[b][u].z, vb[b][u].w), v + 4);
                } else {
                    IO::unpack_v(vb[b][u], v);
                }
#pragma unroll
                for (int h = 0; h < REP; ++h) {
                    if ((uint32_t)h >= rep) break;
                    const float p = i < n ? sc[(uint32_t)h * a.chunk + ic] : 0.0f;
#pragma unroll
                    for (int e = 0; e < VE; ++e) o[h][e] += p * v[e];
                }
            }
            if constexpr (decltype(reload)::value) load_values(vb[b], ib + NB * kGroup);
        }
    };
    uint32_t i0 = (uint32_t)wave;
    if constexpr (!ONE) {
        for (; i0 + NB * kGroup < n; i0 += NB * kGroup) value_block(i0, std::true_type{});
    }
    if (i0 < n) value_block(i0, std::false_type{});
    if constexpr (kWideV) {
        // the slots' sums of each column, added across the lanes D / 8 apart
#pragma unroll
        for (int h = 0; h < REP; ++h)
#pragma unroll
            for (int e = 0; e < VE; ++e)
#pragma unroll
                for (int off = D / 8; off < 64; off <<= 1) o[h][e] += __shfl_xor(o[h][e], off, 64);
    }
    __syncthreads();  // the probabilities are no longer read: reuse the LDS for the wave sums
    float* red = lds;  // [wave][rep][D]
#pragma unroll
    for (int h = 0; h < REP; ++h) {
        if ((uint32_t)h >= rep) break;
        if (vslot != 0) break;
#pragma unroll
        for (int e = 0; e < VE; ++e) red[((uint32_t)wave * rep + (uint32_t)h) * D + vcol + e] = o[h][e];
    }
    __syncthreads();
    for (uint32_t i = threadIdx.x; i < rep * (uint32_t)D; i += kAttnThreads) {
        float s = red[i];
#pragma unroll
        for (int w = 1; w < kAttnWaves; ++w) s += red[(uint32_t)w * rep * D + i];
        const uint32_t h = i / D, slice = (i % D) / 64;
        a.part_o[(uint64_t)row_tok(h) * a.part_tok_stride + ((row_head(h) * (D / 64) + slice) * a.nchunks + c) * 64 +
                 (i % 64)] = s;
    }
}

template <int D, int kMergeUnroll>
__global__ __launch_bounds__(256) void attention_merge_kernel(MergeArgs a) {
    constexpr int SLICES = D / 64;
    __shared__ float4 s_o[kMergeGroups][16];
    __shared__ float s_m[kMergeGroups], s_l[kMergeGroups];
    const uint32_t tok = blockIdx.y;
    const uint32_t h = blockIdx.x / SLICES, slice = blockIdx.x - h * SLICES;
    const int col = threadIdx.x & 15, grp = threadIdx.x >> 4;
    // this token's chunks (its rows T0 + tok in chunks of `chunk`; one token: the layout's)
    const uint32_t nch = a.tokens > 1 ? (a.T0 + tok + a.chunk - 1) / a.chunk : a.nchunks;
    const uint64_t ptok = (uint64_t)tok * a.part_tok_stride;
    const float* mlp = a.part_ml + ptok + (uint64_t)h * a.nchunks * 2;                     // [nchunks][2]
    const float* op = a.part_o + ptok + ((uint64_t)h * SLICES + slice) * a.nchunks * 64;  // [nchunks][64]
    constexpr uint32_t kPass = kMergeGroups * kMergeUnroll;  // chunks per pass of the workgroup
    const uint64_t base = (uint64_t)tok * a.out_tok_stride + (uint64_t)h * D + slice * 64 + (uint64_t)col * 4;
    // the block's output gate, needed last, requested first
    float4 gv = {0.0f, 0.0f, 0.0f, 0.0f};
    if (a.gate != nullptr && grp == 0)
        gv = *reinterpret_cast<const float4*>(a.gate + (uint64_t)tok * a.gate_tok_stride + (uint64_t)h * a.gate_stride +
                                              slice * 64 + col * 4);
    // the first pass's chunk maxima and sums, then its value slices, all requested before any
    // use (loads complete in order: M waits only for the maxima)
    float2 ml[kMergeUnroll];
    float4 oc[kMergeUnroll];
#pragma unroll
    for (int u = 0; u < kMergeUnroll; ++u) {
        uint32_t c = (uint32_t)grp + (uint32_t)u * kMergeGroups;
        c = c < nch ? c : nch - 1;
        ml[u] = *reinterpret_cast<const float2*>(mlp + (uint64_t)c * 2);
    }
#pragma unroll
    for (int u = 0; u < kMergeUnroll; ++u) {
        uint32_t c = (uint32_t)grp + (uint32_t)u * kMergeGroups;
        c = c < nch ? c : nch - 1;
        oc[u] = reinterpret_cast<const float4*>(op + (uint64_t)c * 64)[col];
    }
    // 1. M = the largest chunk maximum (every chunk holds at least one token: m_c is finite);
    //    clamped repeats of the last chunk do not change a maximum
    float m = ml[0].x;
#pragma unroll
    for (int u = 1; u < kMergeUnroll; ++u) m = fmaxf(m, ml[u].x);
    for (uint32_t c = (uint32_t)grp + kPass; c < nch; c += kMergeGroups)
        m = fmaxf(m, mlp[(uint64_t)c * 2]);
    if (col == 0) s_m[grp] = m;
    __syncthreads();
    float M = s_m[0];
#pragma unroll
    for (int i = 1; i < kMergeGroups; ++i) M = fmaxf(M, s_m[i]);
    // 2. out = sum_c e^(m_c - M) o_c / sum_c e^(m_c - M) l_c: each chunk's weight on its own, the
    //    sums in chunk order within a group, then over the groups in group order
    float l = 0.0f;
    float4 o = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int u = 0; u < kMergeUnroll; ++u) {
        const bool in = (uint32_t)grp + (uint32_t)u * kMergeGroups < nch;
        const float wgt = in ? expf(ml[u].x - M) : 0.0f;
        l = fmaf(wgt, ml[u].y, l);
        o.x = fmaf(wgt, oc[u].x, o.x);
        o.y = fmaf(wgt, oc[u].y, o.y);
        o.z = fmaf(wgt, oc[u].z, o.z);
        o.w = fmaf(wgt, oc[u].w, o.w);
    }
    for (uint32_t c = (uint32_t)grp + kPass; c < nch; c += kMergeGroups) {
        const float2 v = *reinterpret_cast<const float2*>(mlp + (uint64_t)c * 2);
        const float4 ov = reinterpret_cast<const float4*>(op + (uint64_t)c * 64)[col];
        const float wgt = expf(v.x - M);
        l = fmaf(wgt, v.y, l);
        o.x = fmaf(wgt, ov.x, o.x);
        o.y = fmaf(wgt, ov.y, o.y);
        o.z = fmaf(wgt, ov.z, o.z);
        o.w = fmaf(wgt, ov.w, o.w);
    }
    s_o[grp][col] = o;
    if (col == 0) s_l[grp] = l;
    __syncthreads();
    if (grp != 0) return;
    float L = s_l[0];
    float4 O = s_o[0][col];
#pragma unroll
    for (int i = 1; i < kMergeGroups; ++i) {
        L += s_l[i];
        const float4 v = s_o[i][col];
        O.x += v.x;
        O.y += v.y;
        O.z += v.z;
        O.w += v.w;
    }
    const float out[4] = {O.x / L, O.y / L, O.z / L, O.w / L};
    if (a.out != nullptr) *reinterpret_cast<float4*>(a.out + base) = make_float4(out[0], out[1], out[2], out[3]);
    if (a.gate != nullptr) {
        const float gs[4] = {sigmoid_ref(gv.x), sigmoid_ref(gv.y), sigmoid_ref(gv.z), sigmoid_ref(gv.w)};
        if (a.gate_s != nullptr) *reinterpret_cast<float4*>(a.gate_s + base) = make_float4(gs[0], gs[1], gs[2], gs[3]);
        *reinterpret_cast<float4*>(a.gated + base) = make_float4(out[0] * gs[0], out[1] * gs[1], out[2] * gs[2],
                                                                 out[3] * gs[3]);
    }
}

// ---------------------------------------------------------------- several tokens
//
// The per-head preparation of consecutive tokens in one launch, one wave per (token, row): row r <
// Hq is query head r, the rest key head r - Hq.  The arithmetic is the chunk kernel's preparation
// (prep_row_norm, the rotation with rope_cs), so each row gets the same bits; queries go to qcur,
// keys (and their tokens' value rows) into cache row row0 + token, kcur when given.
struct TokPrepArgs {
    const float *qfull, *kp, *vp;
    uint64_t qfull_tok_stride, kv_tok_stride;
    const float *q_norm, *k_norm;
    float eps;
    RopeParams rope;
    const uint64_t* positions;  // [tokens][3] in device memory, or null: pos below
    uint32_t Hq, Hkv;
    uint64_t row0;
    void *keys, *values;
    float *qcur, *kcur;
    uint64_t pos[3 * kInlineTokenPositions];  // up to kInlineTokenPositions tokens' positions, by value
};

template <typename KT, int D>
__global__ __launch_bounds__(64) void attention_prep_tokens_kernel(TokPrepArgs a) {
    constexpr int VW = D / 64;
    __shared__ float row[D];
    __shared__ float rc[256];
    const int lane = threadIdx.x;
    const uint32_t t = blockIdx.y, r = blockIdx.x;
    const bool is_q = r < a.Hq;
    const uint32_t h = is_q ? r : r - a.Hq;
    const float* src = is_q ? a.qfull + (uint64_t)t * a.qfull_tok_stride + (uint64_t)h * 2 * D
                            : a.kp + (uint64_t)t * a.kv_tok_stride + (uint64_t)h * D;
    const float* w = is_q ? a.q_norm : a.k_norm;
    float px[VW], pw[VW];
    Vec<VW>::unpack(*reinterpret_cast<const typename Vec<VW>::type*>(src + lane * VW), px);
#pragma unroll
    for (int e = 0; e < VW; ++e) pw[e] = w[lane * VW + e];
    RopeParams p = a.rope;
    const uint64_t* tp = a.positions != nullptr ? a.positions + 3 * (uint64_t)t : a.pos + 3 * t;
    p.pos[0] = tp[0];
    p.pos[1] = tp[1];
    p.pos[2] = tp[2];
    const uint32_t half = p.rotary_dim / 2;
    for (uint32_t f = (uint32_t)lane; f < half; f += 64) rope_cs(f, p, rc[f], rc[128 + f]);
    prep_row_norm<D>(px, pw, a.eps, lane, row);
    __syncthreads();
    for (uint32_t f = (uint32_t)lane; f < half; f += 64) rotate_pair(row, f, half, rc[f], rc[128 + f]);
    __syncthreads();
    if (is_q) {
        float* dst = a.qcur + ((uint64_t)t * a.Hq + h) * D;
#pragma unroll
        for (int e = 0; e < VW; ++e) dst[lane * VW + e] = row[lane * VW + e];
        return;
    }
    using IO = KvIo<KT, VW>;
    KT* krow = static_cast<KT*>(a.keys) + ((a.row0 + t) * a.Hkv + h) * D;
    KT* vrow = static_cast<KT*>(a.values) + ((a.row0 + t) * a.Hkv + h) * D;
    const float* vsrc = a.vp + (uint64_t)t * a.kv_tok_stride + (uint64_t)h * D;
#pragma unroll
    for (int e = 0; e < VW; ++e) {
        const uint32_t i = (uint32_t)lane * VW + e;
        if (a.kcur != nullptr) a.kcur[((uint64_t)t * a.Hkv + h) * D + i] = row[i];
        krow[i] = IO::store(row[i]);
        vrow[i] = IO::store(vsrc[i]);
    }
}

// ---------------------------------------------------------------- RoPE

// frequency f's cos / sin: from the host's table when it has one, else computed here
OQ_DEVICE void rope_cs_at(uint32_t f, const RopeParams& p, const RopeTable& t, float& c, float& s) {
    if (t.pairs != 0) {
        c = t.cs[0][f];
        s = t.cs[1][f];
    } else {
        rope_cs(f, p, c, s);
    }
}

__global__ __launch_bounds__(256) void rope_kernel(float* heads, uint32_t head_dim, RopeParams p, RopeTable t) {
    float* x = heads + (uint64_t)blockIdx.x * head_dim;
    const uint32_t half = p.rotary_dim / 2;
    for (uint32_t f = threadIdx.x; f < half; f += blockDim.x) {
        float c, s;
        rope_cs_at(f, p, t, c, s);
        rotate_pair(x, f, half, c, s);
    }
}

template <typename KT, int D, int REP, int NB, bool ONE>
hipError_t launch_nb(const ChunkArgs& a, uint64_t lds, hipStream_t s) {
    const uint32_t tpw = std::max(a.tpw, 1u);
    const uint32_t groups = (std::max(a.tokens, 1u) + tpw - 1) / tpw;  // token groups
    const dim3 grid(groups * a.Hkv * a.nsub * a.nchunks);
    if (a.qfull != nullptr) {
        hipLaunchKernelGGL((attention_chunk_kernel<KT, D, REP, NB, true, ONE>), grid, dim3(kAttnThreads), lds, s, a);
    } else {
        hipLaunchKernelGGL((attention_chunk_kernel<KT, D, REP, NB, false, ONE>), grid, dim3(kAttnThreads), lds, s, a);
    }
    return hipGetLastError();
}

template <typename KT, int D, int REP>
hipError_t launch_chunks(const ChunkArgs& a, uint64_t lds, hipStream_t s) {
    // passes in flight per wave.  Long chunks: two, measured 56.1 us per step (chunk + merge, 16
    // query heads over 4 KV heads of 256, 32768 tokens) against 57.2 with one and 62.4 with three;
    // four for 64-token chunks took 24.3 against 19.9 us at 8192 tokens.  A chunk of one, two or
    // three passes keeps exactly that many in flight, so keys and values each need one round
    // trip and no pass is a clamped copy of the chunk's last row: attention at 1024 / 2048 / 4096
    // tokens 12.1 / 15.5 / 17.8 us with three passes in flight -> 9.45 / 12.3 / 15.6; the attention
    // block at 4097 tokens (48-token chunks) 54.3-55.2 us with two -> 52.9-53.3 with three.
    if (a.chunk <= kTokStep) return launch_nb<KT, D, REP, 1, true>(a, lds, s);
    if (a.chunk <= 2 * kTokStep) return launch_nb<KT, D, REP, 2, true>(a, lds, s);
    if (a.chunk <= 3 * kTokStep) return launch_nb<KT, D, REP, 3, true>(a, lds, s);
    return launch_nb<KT, D, REP, 2, false>(a, lds, s);
}

template <typename KT, int D>
hipError_t launch_reps(const ChunkArgs& a, uint64_t lds, hipStream_t s) {
    if (a.rep == 1) return launch_chunks<KT, D, 1>(a, lds, s);
    if (a.rep == 2) return launch_chunks<KT, D, 2>(a, lds, s);
    if (a.rep <= 4) return launch_chunks<KT, D, 4>(a, lds, s);
    return launch_chunks<KT, D, 8>(a, lds, s);
}

template <int D>
hipError_t launch_d(const AttnLaunch& L, hipStream_t s) {
    ChunkArgs a{};
    a.q = L.q;
    a.keys = L.keys;
    a.values = L.values;
    a.new_k = L.new_k;
    a.new_v = L.new_v;
    a.T = L.T;
    a.Hkv = L.Hkv;
    a.rep_all = L.rep;
    a.nsub = attention_subgroups(L.rep);
    a.rep = L.rep / a.nsub;
    a.tpw = 1;
    a.heads = a.rep;
    a.chunk = L.chunk;
    a.nchunks = L.nchunks;
    a.scale = L.scale;
    a.part_o = L.part;
    a.part_ml = L.part + (uint64_t)L.Hkv * L.nchunks * L.rep * D;
    a.stage = std::max(a.rep * L.chunk, (uint32_t)kAttnWaves * a.rep * D);
    uint64_t lds = a.stage;
    if (L.prep != nullptr) {
        const AttnPrep& p = *L.prep;
        a.q = nullptr;
        a.new_k = nullptr;
        a.new_v = p.vp;
        a.qfull = p.qfull;
        a.kp = p.kp;
        a.q_norm = p.q_norm;
        a.k_norm = p.k_norm;
        a.eps = p.eps;
        a.rope = p.rope;
        a.qcur = p.qcur;
        a.kcur = p.kcur;
        lds += (uint64_t)(a.rep + 1) * D + 256;  // the preparation's rows and cos / sin
    }
    lds *= sizeof(float);
    hipError_t e;
    if (L.f16) {
        // the new token's rows (with the preparation folded in, its value row only: the key is
        // prepared and stored by the chunk kernel) rounded into the cache before the chunk kernel
        const float* nv = L.prep != nullptr && L.prep->v_stored ? nullptr : a.new_v;  // stored by the projection
        if (a.new_k != nullptr || nv != nullptr) {
            const uint32_t n = L.Hkv * (uint32_t)D;
            const uint64_t row = (uint64_t)(L.T - 1) * L.Hkv * D;
            hipLaunchKernelGGL(kv_append_f16_kernel, dim3((n + 255) / 256), dim3(256), 0, s, a.new_k, nv,
                               static_cast<_Float16*>(L.keys) + row, static_cast<_Float16*>(L.values) + row, n);
            if ((e = hipGetLastError()) != hipSuccess) return e;
        }
        a.new_k = nullptr;
        a.new_v = nullptr;
        e = launch_reps<_Float16, D>(a, lds, s);
    } else {
        e = launch_reps<float, D>(a, lds, s);
    }
    if (e != hipSuccess) return e;
    MergeArgs m{};
    m.part_o = a.part_o;
    m.part_ml = a.part_ml;
    m.nchunks = L.nchunks;
    m.out = L.out;
    m.gate = L.gate;
    m.gate_stride = L.gate_stride;
    m.gate_s = L.gate_s;
    m.gated = L.gated;
    // chunks in flight per merge thread: as many as the chunks need, up to 8 (no clamped repeats
    // of the last chunk): 256 / 512 / 1024 tokens 8.87 / 8.98 / 9.34 -> 8.43 / 8.52 / 9.05 us
    const dim3 mgrid(L.Hkv * L.rep * (D / 64));
    if (L.nchunks <= 2 * kMergeGroups) hipLaunchKernelGGL((attention_merge_kernel<D, 2>), mgrid, dim3(256), 0, s, m);
    else if (L.nchunks <= 4 * kMergeGroups) hipLaunchKernelGGL((attention_merge_kernel<D, 4>), mgrid, dim3(256), 0, s, m);
    else hipLaunchKernelGGL((attention_merge_kernel<D, 8>), mgrid, dim3(256), 0, s, m);
    return hipGetLastError();
}

template <int D>
hipError_t launch_tokens_d(const AttnLaunch& L, const AttnTokens& tk, hipStream_t s) {
    const uint32_t T0 = L.T - (tk.tokens - 1);  // rows of the first token
    TokPrepArgs pa{};
    pa.qfull = tk.qfull;
    pa.kp = tk.kp;
    pa.vp = tk.vp;
    pa.qfull_tok_stride = (uint64_t)L.Hkv * L.rep * 2 * D;
    pa.kv_tok_stride = (uint64_t)L.Hkv * D;
    pa.q_norm = tk.q_norm;
    pa.k_norm = tk.k_norm;
    pa.eps = tk.eps;
    pa.rope = tk.rope;
    if (tk.positions_host != nullptr && tk.tokens <= kInlineTokenPositions) {
        for (uint32_t i = 0; i < 3 * tk.tokens; ++i) pa.pos[i] = tk.positions_host[i];
        pa.positions = nullptr;
    } else {
        if (tk.positions == nullptr) return hipErrorInvalidValue;
        pa.positions = tk.positions;
    }
    pa.Hq = L.Hkv * L.rep;
    pa.Hkv = L.Hkv;
    pa.row0 = T0 - 1;
    pa.keys = L.keys;
    pa.values = L.values;
    pa.qcur = tk.qcur;
    pa.kcur = tk.kcur;
    const dim3 pgrid(pa.Hq + pa.Hkv, tk.tokens);
    if (L.f16) hipLaunchKernelGGL((attention_prep_tokens_kernel<_Float16, D>), pgrid, dim3(64), 0, s, pa);
    else hipLaunchKernelGGL((attention_prep_tokens_kernel<float, D>), pgrid, dim3(64), 0, s, pa);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;

    ChunkArgs a{};
    a.q = tk.qcur;
    a.keys = L.keys;
    a.values = L.values;
    a.T = T0;
    a.Hkv = L.Hkv;
    a.rep_all = L.rep;
    a.nsub = attention_subgroups(L.rep);
    // over long caches, as many tokens per workgroup as its 8 query rows hold: each key and value row
    // read once for them (shorter caches keep one token per workgroup: twice the workgroups)
    a.heads = L.rep / a.nsub;
    a.tpw = attention_tokens_per_workgroup(L.T, L.rep, tk.tokens);
    a.rep = a.tpw * a.heads;
    a.chunk = L.chunk;
    a.nchunks = L.nchunks;
    a.scale = L.scale;
    a.tokens = tk.tokens;
    a.q_tok_stride = (uint64_t)L.Hkv * L.rep * D;
    a.part_tok_stride = attention_partial_floats(L.Hkv, L.rep, D, L.nchunks);
    a.part_o = L.part;
    a.part_ml = L.part + (uint64_t)L.Hkv * L.nchunks * L.rep * D;
    a.stage = std::max(a.rep * L.chunk, (uint32_t)kAttnWaves * a.rep * D);
    const uint64_t lds = (uint64_t)a.stage * sizeof(float);
    e = L.f16 ? launch_reps<_Float16, D>(a, lds, s) : launch_reps<float, D>(a, lds, s);
    if (e != hipSuccess) return e;

    MergeArgs m{};
    m.part_o = a.part_o;
    m.part_ml = a.part_ml;
    m.nchunks = L.nchunks;
    m.tokens = tk.tokens;
    m.T0 = T0;
    m.chunk = L.chunk;
    m.part_tok_stride = a.part_tok_stride;
    m.out_tok_stride = (uint64_t)L.Hkv * L.rep * D;
    m.gate_tok_stride = tk.gate_tok_stride;
    m.out = L.out;
    m.gate = L.gate;
    m.gate_stride = L.gate_stride;
    m.gate_s = L.gate_s;
    m.gated = L.gated;
    const dim3 mgrid(L.Hkv * L.rep * (D / 64), tk.tokens);
    if (L.nchunks <= 2 * kMergeGroups) hipLaunchKernelGGL((attention_merge_kernel<D, 2>), mgrid, dim3(256), 0, s, m);
    else if (L.nchunks <= 4 * kMergeGroups) hipLaunchKernelGGL((attention_merge_kernel<D, 4>), mgrid, dim3(256), 0, s, m);
    else hipLaunchKernelGGL((attention_merge_kernel<D, 8>), mgrid, dim3(256), 0, s, m);
    return hipGetLastError();
}

// ---------------------------------------------------------------- any shape
//
// Key and value widths outside {64, 128, 256}, a key width different from the value width, or more
// than 256 query heads per KV head (the reference's causal_attention_step and block take any
// shape): plain kernels in the reference's order, one workgroup per head.

// The block's per-head preparation for one token: workgroup r < Hq normalises query head r with
// q_norm and rotates it into qcur; workgroup Hq + g normalises key head g with k_norm, rotates it
// into cache row `row` (and kcur when given) and stores value head g beside it (unless an F16
// cache's value row is already stored).  The row sits in dynamic LDS (D floats); its sum of squares
// is in double (rms_norm_rows, qwen35_block.cpp:161-189), the rotation rope_cs / rotate_pair's.
template <typename KT>
__global__ __launch_bounds__(256) void attention_prep_any_kernel(AttnPrep p, uint32_t Hq, uint32_t Hkv, uint32_t D,
                                                                 uint64_t row, KT* __restrict__ keys,
                                                                 KT* __restrict__ values) {
#pragma clang fp contract(off)
    extern __shared__ __align__(16) float xrow[];  // [D]
    __shared__ double red[4];
    const uint32_t r = blockIdx.x;
    const bool is_q = r < Hq;
    const uint32_t h = is_q ? r : r - Hq;
    const float* src = is_q ? p.qfull + (uint64_t)h * 2 * D : p.kp + (uint64_t)h * D;
    const float* w = is_q ? p.q_norm : p.k_norm;
    double ss = 0.0;
    for (uint32_t i = threadIdx.x; i < D; i += 256) {
        const float v = src[i];
        xrow[i] = v;
        ss += (double)v * (double)v;
    }
    ss = wave_sum_f64(ss);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
    __syncthreads();
    ss = red[0] + red[1] + red[2] + red[3];
    const float inv = (float)(1.0 / sqrt(ss / (double)D + (double)p.eps));
    for (uint32_t i = threadIdx.x; i < D; i += 256) xrow[i] = xrow[i] * inv * w[i];
    __syncthreads();
    const uint32_t half = p.rope.rotary_dim / 2;
    for (uint32_t f = threadIdx.x; f < half; f += 256) {
        float c, sn;
        rope_cs_at(f, p.rope, p.table, c, sn);
        rotate_pair(xrow, f, half, c, sn);
    }
    __syncthreads();
    if (is_q) {
        float* dst = p.qcur + (uint64_t)h * D;
        for (uint32_t i = threadIdx.x; i < D; i += 256) dst[i] = xrow[i];
        return;
    }
    KT* krow = keys + (row * Hkv + h) * D;
    KT* vrow = values + (row * Hkv + h) * D;
    const float* vsrc = p.vp + (uint64_t)h * D;
    for (uint32_t i = threadIdx.x; i < D; i += 256) {
        if (p.kcur != nullptr) p.kcur[(uint64_t)h * D + i] = xrow[i];
        krow[i] = (KT)xrow[i];
        if (!p.v_stored) vrow[i] = (KT)vsrc[i];
    }
}

// The new token's key rows [Hkv][Dk] and value rows [Hkv][Dv] stored into cache row `row`
// (KvCache::append, hybrid_cache.cpp:154-169; an F16 cache rounds to nearest even)
template <typename KT>
__global__ __launch_bounds__(256) void kv_append_any_kernel(const float* __restrict__ k, const float* __restrict__ v,
                                                            KT* __restrict__ keys, KT* __restrict__ values, uint64_t row,
                                                            uint64_t nk, uint64_t nv) {
    const uint64_t i = (uint64_t)blockIdx.x * 256u + threadIdx.x;
    if (k != nullptr && i < nk) keys[row * nk + i] = (KT)k[i];
    if (v != nullptr && i < nv) values[row * nv + i] = (KT)v[i];
}

// Query head h over the T cached rows of KV head h / rep (causal_attention_step,
// reference_kernels.cpp:152-193): each score a double dot product in dimension order, rounded to
// F32 and scaled; p = exp(s - max) in F32, the denominator in double (per thread over its tokens,
// then over the threads), p / denominator in double rounded to F32; each output column the F32 sum
// of p_t * v_t in token order, as the reference adds it.  Scores and then probabilities are kept
// in scores [T]; the query in dynamic LDS (Dk floats).  With a gate: gate_s = sigmoid(gate),
// gated = out * gate_s (qwen35_block.cpp:734-741).
template <typename KT>
__global__ __launch_bounds__(256) void attention_any_kernel(const float* __restrict__ q, const KT* __restrict__ keys,
                                                            const KT* __restrict__ values, uint32_t T, uint32_t Hkv,
                                                            uint32_t rep, uint32_t Dk, uint32_t Dv, float scale,
                                                            float* __restrict__ scores, float* __restrict__ out,
                                                            const float* __restrict__ gate, uint32_t gate_stride,
                                                            float* __restrict__ gate_s, float* __restrict__ gated) {
#pragma clang fp contract(off)
    extern __shared__ __align__(16) float qs[];  // [Dk]
    __shared__ float redf[4];
    __shared__ double redd[4];
    const uint32_t h = blockIdx.x, g = h / rep;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    for (uint32_t i = threadIdx.x; i < Dk; i += 256) qs[i] = q[(uint64_t)h * Dk + i];
    __syncthreads();
    float* sc = scores + (uint64_t)h * T;
    float mx = -INFINITY;
    for (uint32_t t = threadIdx.x; t < T; t += 256) {
        const KT* k = keys + ((uint64_t)t * Hkv + g) * Dk;
        double dot = 0.0;
        for (uint32_t d = 0; d < Dk; ++d) dot += (double)qs[d] * (double)(float)k[d];
        const float s = (float)dot * scale;
        sc[t] = s;
        mx = fmaxf(mx, s);
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
    if (lane == 0) redf[wave] = mx;
    __syncthreads();
    const float M = fmaxf(fmaxf(redf[0], redf[1]), fmaxf(redf[2], redf[3]));
    double l = 0.0;
    for (uint32_t t = threadIdx.x; t < T; t += 256) {
        const float e = expf(sc[t] - M);
        sc[t] = e;
        l += (double)e;
    }
    l = wave_sum_f64(l);
    if (lane == 0) redd[wave] = l;
    __syncthreads();
    const double den = redd[0] + redd[1] + redd[2] + redd[3];
    for (uint32_t t = threadIdx.x; t < T; t += 256) sc[t] = (float)((double)sc[t] / den);
    __syncthreads();  // every probability stored before any column reads them
    for (uint32_t d = threadIdx.x; d < Dv; d += 256) {
        float acc = 0.0f;
        for (uint32_t t = 0; t < T; ++t) acc += sc[t] * (float)values[((uint64_t)t * Hkv + g) * Dv + d];
        const uint64_t o = (uint64_t)h * Dv + d;
        if (out != nullptr) out[o] = acc;
        if (gate != nullptr) {
            const float gs = sigmoid_ref(gate[(uint64_t)h * gate_stride + d]);
            if (gate_s != nullptr) gate_s[o] = gs;
            gated[o] = acc * gs;
        }
    }
}

template <typename KT>
hipError_t launch_any(const AttnLaunch& L, hipStream_t s) {
    const uint32_t Hq = L.Hkv * L.rep;
    KT* keys = static_cast<KT*>(L.keys);
    KT* values = static_cast<KT*>(L.values);
    const uint64_t row = (uint64_t)L.T - 1;
    const float* q = L.q;
    if (L.prep != nullptr) {
        const AttnPrep& p = *L.prep;
        if (p.qcur == nullptr || L.D != L.Dv) return hipErrorInvalidValue;
        hipLaunchKernelGGL(attention_prep_any_kernel<KT>, dim3(Hq + L.Hkv), dim3(256), (uint64_t)L.D * sizeof(float), s,
                           p, Hq, L.Hkv, L.D, row, keys, values);
        q = p.qcur;
    } else if (L.new_k != nullptr || L.new_v != nullptr) {
        const uint64_t nk = (uint64_t)L.Hkv * L.D, nv = (uint64_t)L.Hkv * L.Dv;
        const uint64_t n = nk > nv ? nk : nv;
        hipLaunchKernelGGL(kv_append_any_kernel<KT>, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, L.new_k, L.new_v,
                           keys, values, row, nk, nv);
    }
    if (L.gate != nullptr && L.gated == nullptr) return hipErrorInvalidValue;
    hipLaunchKernelGGL(attention_any_kernel<KT>, dim3(Hq), dim3(256), (uint64_t)L.D * sizeof(float), s, q, keys, values,
                       L.T, L.Hkv, L.rep, L.D, L.Dv, L.scale, L.part, L.out, L.gate, L.gate_stride, L.gate_s, L.gated);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_attention_tokens(const AttnLaunch& L, const AttnTokens& tk, hipStream_t s) {
    if (tk.tokens == 0 || tk.tokens > L.T) return hipErrorInvalidValue;
    switch (L.D) {
        case 64: return launch_tokens_d<64>(L, tk, s);
        case 128: return launch_tokens_d<128>(L, tk, s);
        case 256: return launch_tokens_d<256>(L, tk, s);
        default: return hipErrorInvalidValue;
    }
}

bool attention_dims_supported(uint64_t head_dim, uint64_t rep) {
    return (head_dim == 64 || head_dim == 128 || head_dim == 256) && rep >= 1 && rep <= kAttnMaxRep;
}

uint32_t attention_tokens_per_workgroup(uint64_t T, uint64_t rep, uint64_t tokens) {
    const bool share = T >= (uint64_t)std::max(0, knob(kAttnShareMin, 8192));
    const uint32_t heads = (uint32_t)rep / attention_subgroups((uint32_t)rep);
    return share ? (uint32_t)std::min<uint64_t>(tokens, std::max<uint32_t>(1, 8 / heads)) : 1u;
}

uint32_t attention_subgroups(uint32_t rep) {
    // the fewest equal subgroups of at most 8 query heads (a prime group above 8 becomes single heads)
    for (uint32_t n = (rep + 7) / 8; n < rep; ++n)
        if (rep % n == 0) return n;
    return rep;
}

void attention_plan(uint64_t T, uint64_t Hkv, uint64_t rep, uint32_t& chunk, uint32_t& nchunks, uint64_t token_groups) {
    // about two chunk workgroups per compute unit (OQ_ATTN_WG_PER_CU) over the (KV head, subgroup)
    // pairs and the token groups, chunks a multiple of the score pass
    const uint64_t per_cu = (uint64_t)std::max(1, knob(kAttnWgPerCu, 2));
    const uint64_t groups = std::max<uint64_t>(Hkv, 1) * attention_subgroups((uint32_t)std::max<uint64_t>(rep, 1)) *
                            std::max<uint64_t>(token_groups, 1);
    const uint64_t target = std::max<uint64_t>(1, (per_cu * (uint64_t)cu_count()) / groups);
    uint64_t c = (T + target - 1) / target;
    const uint64_t min_chunk = (uint64_t)std::max(1, knob(kAttnMinChunk, (int)kTokStep));
    c = std::max<uint64_t>(c, min_chunk);
    c = (c + kTokStep - 1) / kTokStep * kTokStep;
    c = std::min<uint64_t>(std::max<uint64_t>(c, kTokStep), kMaxChunk);
    chunk = (uint32_t)c;
    nchunks = (uint32_t)((T + c - 1) / c);
}

uint64_t attention_partial_floats(uint64_t Hkv, uint64_t rep, uint64_t head_dim, uint32_t nchunks) {
    return Hkv * (uint64_t)nchunks * rep * (head_dim + 2);
}

hipError_t launch_f32_to_f16(const float* src, void* dst, uint64_t n, hipStream_t s) {
    if (n == 0) return hipSuccess;
    const uint64_t blocks = std::min<uint64_t>((n + 255) / 256, 65536);
    hipLaunchKernelGGL(f32_to_f16_kernel, dim3((unsigned)blocks), dim3(256), 0, s, src, static_cast<_Float16*>(dst), n);
    return hipGetLastError();
}

uint64_t attention_any_floats(uint64_t q_heads, uint64_t T) { return q_heads * T; }

hipError_t launch_attention(const AttnLaunch& L, hipStream_t s) {
    if (L.any) {
        if (L.T == 0 || L.D == 0 || L.Dv == 0 || L.D > kAttnAnyMaxDim || L.Hkv == 0 || L.rep == 0 ||
            (uint64_t)L.Hkv * L.rep > 0x7FFFFFFFull)
            return hipErrorInvalidValue;
        return L.f16 ? launch_any<_Float16>(L, s) : launch_any<float>(L, s);
    }
    switch (L.D) {
        case 64: return launch_d<64>(L, s);
        case 128: return launch_d<128>(L, s);
        case 256: return launch_d<256>(L, s);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_rope(float* heads, uint64_t n_heads, uint64_t head_dim, const RopeParams& p, const RopeTable& t,
                       hipStream_t s) {
    if (n_heads == 0) return hipSuccess;
    hipLaunchKernelGGL(rope_kernel, dim3((unsigned)n_heads), dim3(std::min<uint32_t>(256u, std::max(64u, p.rotary_dim / 2))),
                       0, s, heads, (uint32_t)head_dim, p, t);
    return hipGetLastError();
}

}  // namespace oq
