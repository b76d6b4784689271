// The m = 1 decode GEMV of oq_gemv_kq.h with the small operations of a Gated DeltaNet decode
// block folded into its prologue and epilogue (see the comment below and oq_deltanet.hip).
#include "oq_gemv_kq.h"

namespace oq {

namespace {

using namespace kq;

// ---------------------------------------------------------------- fused decode-block GEMV
//
// The m = 1 kernel above with the small operations of a Gated DeltaNet block folded in (see
// oq_deltanet.hip for the block order), two rows per wave, 8 waves per workgroup:
//   prologue  (IN, FFN): x' = (x * inverse_rms(x)) * norm_w before the Q8_K staging; every
//             workgroup reduces sum x^2 over the whole row itself (double), workgroup 0 also
//             stores x' (norm_out)
//   rows      IN: the concatenation of up to four matrices sharing K and type (row pairs never
//             straddle two); FFN: pair g = (row g of mat[0], row g of mat[1]); ADD: one matrix
//   epilogue  IN: raw outputs (of the matrices whose raw[i] is given); rows of mat[0] (qkv) run
//             their channel's causal convolution step and SiLU, rows of mat[2] (beta) the
//             sigmoid, rows of mat[3] (alpha) softplus(a + dt_bias) * decay -- each only when its
//             output is given (the attention block's q / k / v projections take raw outputs
//             only); ADD: sum_out[n] = add[n] + y[n]; FFN: act[g] = SiLU(gate) * up.

// IN: matrix index and local row of row `row` of the concatenation (wave-uniform)
OQ_DEVICE void blk_in_row(const BlockGemv& a, uint32_t row, uint32_t& mi, uint32_t& local) {
    mi = 0;
#pragma unroll
    for (int i = 0; i < 3; ++i)
        if ((uint32_t)i + 1 < a.nmat && row >= a.row_end[i]) mi = (uint32_t)i + 1;
    local = row - (mi ? a.row_end[mi - 1] : 0u);
    mi = __builtin_amdgcn_readfirstlane(mi);
    local = __builtin_amdgcn_readfirstlane(local);
}

// IN: the epilogue's operands of a group, requested with its weights (behind them: they are
// needed only after the weights): lane 16 r + i of a convolution row r holds the channel's history
// value i + 1 (v[0]; unused for the last tap) and tap i (v[1]); lane 16 r of an alpha row holds
// dt_bias (v[0]) and decay (v[1]).  Loaded in the epilogue instead, they would cost the last group
// of every wave one dependent round trip per tap.
struct EpiPf {
    float v[2];
};

template <uint32_t TYPE, int ITERS, int MODE, bool FULL>
OQ_DEVICE void blk_load_group(typename WRegs<TYPE>::type (&W)[2][ITERS], EpiPf& pf, const BlockGemv& a, uint64_t grp,
                              int lane) {
    const uint32_t nsb = (uint32_t)(a.mat[0].k / kQK);
    uint32_t mis[2], locals[2];
#pragma unroll
    for (int r = 0; r < 2; ++r) {
        uint32_t mi, local;
        if constexpr (MODE == kBlockFfn) {
            mi = (uint32_t)r;
            local = (uint32_t)grp;
        } else {
            blk_in_row(a, (uint32_t)grp * 2u + (uint32_t)r, mi, local);
        }
        mis[r] = mi;
        locals[r] = local;
        const DeviceMatrix& w = a.mat[mi];
        const uint32_t lrow = local < (uint32_t)w.n ? local : (uint32_t)w.n - 1;
        const uint8_t* base = w.base + (uint64_t)lrow * w.pitch;
#pragma unroll
        for (int it = 0; it < ITERS; ++it) load_w<TYPE>(W[r][it], base, nsb, it, lane);
    }
    if constexpr (MODE == kBlockIn) {
        const uint32_t nrows = a.row_end[a.nmat - 1];
        const uint32_t r = (uint32_t)lane >> 4, i = (uint32_t)lane & 15u;
        const uint32_t mi = r == 0 ? mis[0] : mis[1], l = r == 0 ? locals[0] : locals[1];
        const bool row_ok = lane < 32 && (uint32_t)grp * 2u + r < nrows;
        const uint32_t K = a.conv_kernel;
        // one load per register, its address chosen per lane: two loads into one register on
        // paths of different lanes would make the second wait for every load in flight (the
        // group's weights included)
        const bool conv = row_ok && mi == 0 && a.conv_w != nullptr && i < K;
        const bool alpha = row_ok && mi == 3 && a.log_decay != nullptr && i == 0;
        const float* p0 = conv ? a.history + (uint64_t)l * K + i + 1 : a.dt_bias + l;
        const float* p1 = conv ? a.conv_w + (uint64_t)l * K + i : a.decay + l;
        if ((conv && i + 1 < K) || alpha) pf.v[0] = *p0;
        if (conv || alpha) pf.v[1] = *p1;
    }
}

OQ_DEVICE double readlane_f64(double v, int src) {
    const uint64_t b = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)b, src);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(b >> 32), src);
    return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}

// v0, v1: the group's two row outputs (wave-uniform); pf: its prefetched epilogue operands
template <int MODE>
OQ_DEVICE void blk_epilogue(const BlockGemv& a, uint64_t grp, int lane, float v0, float v1, const EpiPf& pf) {
    if constexpr (MODE == kBlockFfn) {
        // lane 0: gate row grp, lane 1: up row grp
        if (lane == 0) {
#pragma clang fp contract(off)
            if (a.raw[0] != nullptr) a.raw[0][grp] = v0;
            a.act[grp] = silu_ref(v0) * v1;
        } else if (lane == 1 && a.raw[1] != nullptr) {
            a.raw[1][grp] = v1;
        }
    } else if constexpr (MODE == kBlockAdd) {
        const uint64_t row = grp * 2 + lane;
        if (lane < 2 && row < a.mat[0].n) {
            const float v = lane == 0 ? v0 : v1;
            if (a.raw[0] != nullptr) a.raw[0][row] = v;
            a.sum_out[row] = a.add[row] + v;
        }
    } else {
        const uint32_t nrows = a.row_end[a.nmat - 1];
#pragma unroll
        for (int r = 0; r < 2; ++r) {
            const uint32_t row = (uint32_t)grp * 2u + (uint32_t)r;
            if (row >= nrows) break;
            uint32_t mi, l;
            blk_in_row(a, row, mi, l);
            const float v = r == 0 ? v0 : v1;
            if (lane == r && a.raw[mi] != nullptr) a.raw[mi][l] = v;
            if (lane == r && mi == 2 && a.v16 != nullptr) a.v16[l] = (_Float16)v;
            if (mi == 0 && a.conv_w != nullptr) {
                // causal depthwise convolution step of channel l (reference_kernels.cpp:197-225) +
                // SiLU: the history shifts by one (tap i takes value i + 1, the last tap the new
                // output), then the taps are summed in tap order, in double, as the reference does
                const uint32_t K = a.conv_kernel, i = (uint32_t)lane - 16u * (uint32_t)r;
                const bool mine = i < K;  // lanes 16 r .. 16 r + K - 1
                const float t = i + 1 < K ? pf.v[0] : v;
                double p = 0.0;
                if (mine) {
                    a.history[(uint64_t)l * K + i] = t;
                    p = (double)t * (double)pf.v[1];
                }
                double sum = 0.0;
                for (uint32_t j = 0; j < K; ++j) {
#pragma clang fp contract(off)
                    sum += readlane_f64(p, 16 * r + (int)j);
                }
                if (lane == r) a.conv_out[l] = silu_ref((float)sum);
            } else if (mi == 2 && a.beta_s != nullptr) {
                if (lane == r) a.beta_s[l] = sigmoid_ref(v);
            } else if (mi == 3 && a.log_decay != nullptr) {
                if (lane == 16 * r) {
#pragma clang fp contract(off)
                    a.log_decay[l] = softplus_ref(v + pf.v[0]) * pf.v[1];
                }
            }
        }
    }
}

template <uint32_t TYPE, int ITERS, int MODE, bool FULL>
__global__ __launch_bounds__(512) void gemv_block_kernel(BlockGemv a) {
    using WR = typename WRegs<TYPE>::type;
    constexpr int WAVES = 8, R = 2;
    extern __shared__ __align__(16) uint8_t smem[];
    __shared__ double red[WAVES];
    const int lane = threadIdx.x & 63;
    const int wave_in_wg = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint64_t wave = (uint64_t)blockIdx.x * WAVES + wave_in_wg;
    const uint64_t nw = (uint64_t)gridDim.x * WAVES;
    const uint64_t k = a.mat[0].k;
    const uint64_t nsb = k / kQK;
    const uint64_t groups = MODE == kBlockFfn ? a.mat[0].n : ((uint64_t)a.row_end[a.nmat - 1] + 1) / 2;
    const ActLds s{smem, k};
    const bool active = wave < groups;
    WR A[R][ITERS];

    constexpr int SBW = (ITERS * 16 + WAVES - 1) / WAVES;
    // the norm weights are requested with x (up to two blocks per wave): otherwise their load is
    // one more round trip after the sum-of-squares barrier
    constexpr bool kNormEarly = SBW <= 2;
    float4 xv[SBW], nv[kNormEarly ? SBW : 1];
#pragma unroll
    for (int j = 0; j < SBW; ++j) {
        uint64_t b = (uint64_t)wave_in_wg + (uint64_t)WAVES * j;
        b = b < nsb ? b : nsb - 1;
        xv[j] = reinterpret_cast<const float4*>(a.x + b * kQK)[lane];
        if constexpr (kNormEarly) {
            if (a.norm_w) nv[j] = reinterpret_cast<const float4*>(a.norm_w + b * kQK)[lane];
        }
    }
    asm volatile("" ::: "memory");
    EpiPf pf[2] = {};
    blk_load_group<TYPE, ITERS, MODE, FULL>(A, pf[0], a, active ? wave : groups - 1, lane);
    if (a.norm_w) {
        // RMSNorm (qwen35_block.cpp:161-186): sum of squares in double over the whole row
        double ss = 0.0;
#pragma unroll
        for (int j = 0; j < SBW; ++j) {
            const uint64_t b = (uint64_t)wave_in_wg + (uint64_t)WAVES * j;
            if (b < nsb) {
                ss += (double)xv[j].x * (double)xv[j].x + (double)xv[j].y * (double)xv[j].y +
                      (double)xv[j].z * (double)xv[j].z + (double)xv[j].w * (double)xv[j].w;
            }
        }
        ss = wave_sum_f64(ss);
        if (lane == 0) red[wave_in_wg] = ss;
        __syncthreads();
        double tot = 0.0;
#pragma unroll
        for (int i = 0; i < WAVES; ++i) tot += red[i];
        const float inv = (float)(1.0 / sqrt(tot / (double)k + (double)a.eps));
#pragma unroll
        for (int j = 0; j < SBW; ++j) {
            const uint64_t b = (uint64_t)wave_in_wg + (uint64_t)WAVES * j;
            if (b >= nsb) break;
            float4 w4;
            if constexpr (kNormEarly) w4 = nv[j];
            else w4 = reinterpret_cast<const float4*>(a.norm_w + b * kQK)[lane];
            {
#pragma clang fp contract(off)
                xv[j].x = xv[j].x * inv * w4.x;
                xv[j].y = xv[j].y * inv * w4.y;
                xv[j].z = xv[j].z * inv * w4.z;
                xv[j].w = xv[j].w * inv * w4.w;
            }
            if (blockIdx.x == 0 && a.norm_out) reinterpret_cast<float4*>(a.norm_out + b * kQK)[lane] = xv[j];
        }
    }
#pragma unroll
    for (int j = 0; j < SBW; ++j) {
        const uint64_t b = (uint64_t)wave_in_wg + (uint64_t)WAVES * j;
        if (b >= nsb) break;
        uint32_t qw;
        int bs;
        float d;
        quantize_block(xv[j], lane, qw, bs, d);
        store_block<TYPE>(s, 0, b, lane, qw, bs, d);
    }
    __syncthreads();
    if (!active) return;

    Act act[ITERS];
#pragma unroll
    for (int it = 0; it < ITERS; ++it) {
        const uint64_t sb = 16u * it + (lane >> 2);
        if (sb < nsb) slice_from_lds<TYPE>(act[it], s, 0, sb, lane & 3);
    }
    const int q = lane & 3;
    const ScaleSel ss = scale_sel(q);
    uint64_t grp = wave;
    while (true) {
        float acc[R] = {0.0f, 0.0f};
#pragma unroll
        for (int it = 0; it < ITERS; ++it) {
            const uint64_t sb = 16u * it + (lane >> 2);
            if (!FULL && sb >= nsb) continue;
#pragma unroll
            for (int r = 0; r < R; ++r) acc[r] = lane_fma(decode_w<TYPE>(A[r][it], ss, q), act[it], acc[r]);
        }
        const float v0 = wave_sum_uniform(acc[0]), v1 = wave_sum_uniform(acc[1]);
        // the next group's weights and epilogue operands go out before this group's epilogue
        const uint64_t next = grp + nw;
        pf[1] = pf[0];
        if (next < groups) blk_load_group<TYPE, ITERS, MODE, FULL>(A, pf[0], a, next, lane);
        blk_epilogue<MODE>(a, grp, lane, v0, v1, pf[1]);
        grp = next;
        if (grp >= groups) break;
    }
}

// The residual (ADD) projections of the block -- out projection and FFN down, one matrix each --
// streamed: x staged as Q8_K in LDS by 16-wave workgroups, then the rows walked as in
// gemv_stream_kernel (wave i of workgroup b owns rows b * 16 + i + j * (waves in the grid), one
// pass of one row in flight).  Lane (done % 64) keeps the done-th finished row; every 64 rows, and
// at the end, each lane writes its row's raw output and residual sum.  Per-lane sums and row
// reductions as gemv_block_kernel: the same bits.
// Stages the recurrent block's gated output as the activation row (Q8_K in LDS): value i of head
// h = i / dv is ((rec[i] * inv_rms(h)) * out_norm[i % dv]) * SiLU(z[i]) (qwen35_block.cpp:579-588),
// inv_rms(h) = 1 / sqrt(ss_h / dv + eps) with ss_h the delta rule's per-chunk sums of squares
// added in chunk order, SiLU(z[i]) as the delta rule's launch stored it (a.z).  dv is a multiple of
// 32, so a lane's four values share one head.
constexpr uint32_t kMaxHeadChunks = 8;  // value_dim <= 256 in chunks of 32 columns
template <uint32_t TYPE, int ITERS, int WAVES>
OQ_DEVICE void stage_gated_row(const ActLds& s, const BlockGemv& a, uint64_t nsb, int wave_in_wg, int lane) {
#pragma clang fp contract(off)
    constexpr int SBW = (ITERS * 16 + WAVES - 1) / WAVES;
    float4 rv[SBW], zv[SBW], wv[SBW];
    double ssv[SBW];
#pragma unroll
    for (int j = 0; j < SBW; ++j) {
        uint64_t b = (uint64_t)wave_in_wg + (uint64_t)WAVES * j;
        b = b < nsb ? b : nsb - 1;
        const uint64_t i = b * kQK + 4u * (uint32_t)lane;
        rv[j] = *reinterpret_cast<const float4*>(a.rec + i);
        zv[j] = *reinterpret_cast<const float4*>(a.z + i);
        wv[j] = *reinterpret_cast<const float4*>(a.out_norm + i % a.dv);
        // the head's chunk sums, requested together (at most kMaxHeadChunks), then added in order
        const double* hs = a.head_ss + (i / a.dv) * a.dchunks;
        double hv[kMaxHeadChunks];
#pragma unroll
        for (uint32_t c = 0; c < kMaxHeadChunks; ++c) hv[c] = c < a.dchunks ? hs[c] : 0.0;
        double ss = 0.0;
#pragma unroll
        for (uint32_t c = 0; c < kMaxHeadChunks; ++c)
            if (c < a.dchunks) ss += hv[c];
        ssv[j] = ss;
    }
#pragma unroll
    for (int j = 0; j < SBW; ++j) {
        const uint64_t b = (uint64_t)wave_in_wg + (uint64_t)WAVES * j;
        if (b >= nsb) break;
        const float inv = (float)(1.0 / sqrt(ssv[j] / (double)a.dv + (double)a.eps));
        float4 g;
        g.x = rv[j].x * inv * wv[j].x * zv[j].x;
        g.y = rv[j].y * inv * wv[j].y * zv[j].y;
        g.z = rv[j].z * inv * wv[j].z * zv[j].z;
        g.w = rv[j].w * inv * wv[j].w * zv[j].w;
        if (blockIdx.x == 0 && a.gated_out != nullptr) reinterpret_cast<float4*>(a.gated_out + b * kQK)[lane] = g;
        uint32_t qw;
        int bs;
        float d;
        quantize_block(g, lane, qw, bs, d);
        store_block<TYPE>(s, 0, b, lane, qw, bs, d);
    }
}

template <uint32_t TYPE, int ITERS, bool FULL>
__global__ __launch_bounds__(1024) void gemv_block_add_stream_kernel(BlockGemv a) {
    constexpr int WAVES = 16;
    using WR = typename WRegs<TYPE>::type;
    extern __shared__ __align__(16) uint8_t smem[];
    const int lane = threadIdx.x & 63;
    const int wave_in_wg = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t nw = gridDim.x * WAVES;
    const DeviceMatrix& w = a.mat[0];
    const uint32_t nsb = (uint32_t)(w.k / kQK);
    const uint32_t n = (uint32_t)w.n;
    const ActLds s{smem, w.k};
    const uint32_t first = blockIdx.x * WAVES + (uint32_t)wave_in_wg;
    auto row_base = [&](uint32_t row) {
        row = row < n ? row : n - 1;  // a wave without rows reads row n-1
        return w.base + (uint64_t)__builtin_amdgcn_readfirstlane(row) * w.pitch;
    };

    WR buf[2];
    if (a.rec != nullptr) {
        stage_gated_row<TYPE, ITERS, WAVES>(s, a, nsb, wave_in_wg, lane);
    } else {
        stage_one_row<TYPE, ITERS, true, WAVES>(s, a.x, nullptr, nsb, wave_in_wg, lane, [] {});
    }
    load_w<TYPE>(buf[0], row_base(first), nsb, 0, lane);
    __syncthreads();
    if (first >= n) return;

    const int q = lane & 3;
    const ScaleSel ss = scale_sel(q);
    constexpr bool kActRegs = ITERS <= 2;
    Act act[kActRegs ? ITERS : 1];
    if constexpr (kActRegs) {
#pragma unroll
        for (int it = 0; it < ITERS; ++it) {
            const uint32_t sb = 16u * it + (lane >> 2);
            if (sb < nsb) slice_from_lds<TYPE>(act[it], s, 0, sb, q);
        }
    }
    float acc = 0.0f, out = 0.0f;
    uint32_t out_row = 0, done = 0;
    uint32_t row = first, it = 0;  // the unit whose loads are in flight
    bool more = true;
    while (more) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int its = ITERS == 1 ? 0 : (ITERS == 2 ? j : (int)it);
            asm volatile("s_waitcnt vmcnt(0)" : "+v"(acc), "+v"(out)::"memory");
            uint32_t nrow = row, nit = it + 1;
            if (nit == ITERS) {
                nrow = row + nw < row ? n : row + nw;
                nit = 0;
            }
            more = nrow < n;
            // as gemv_stream_kernel: rows of one unit request nothing past the wave's last row
            if (ITERS != 1 || more) load_w<TYPE>(buf[(j + 1) & 1], row_base(more ? nrow : row), nsb, (int)(more ? nit : it), lane);
            hold<TYPE>(buf[j & 1]);
            const uint32_t sb = 16u * (uint32_t)its + (lane >> 2);
            if (FULL || sb < nsb) {
                if constexpr (kActRegs) {
                    acc = lane_fma(decode_w<TYPE>(buf[j & 1], ss, q), act[its], acc);
                } else {
                    Act av;
                    slice_from_lds<TYPE>(av, s, 0, sb, q);
                    acc = lane_fma(decode_w<TYPE>(buf[j & 1], ss, q), av, acc);
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
                    if (a.raw[0] != nullptr) a.raw[0][out_row] = out;
                    a.sum_out[out_row] = a.add[out_row] + out;
                }
            }
            row = nrow;
            it = nit;
            if (!more) break;
        }
    }
    if ((uint32_t)lane < (done & 63u)) {
        if (a.raw[0] != nullptr) a.raw[0][out_row] = out;
        a.sum_out[out_row] = a.add[out_row] + out;
    }
}

// The normalised in-projection without per-row epilogue (the attention block's q / k / v: raw
// outputs only) streamed like the residual projections.  Staging: each wave requests its x
// blocks and their norm weights, then its first row's weights; RMSNorm (qwen35_block.cpp:161-189,
// sum of squares in double, the 16 waves' sums added in wave order); x' quantized to Q8_K in LDS.
// Rows of the concatenation mat[0] | mat[1] | .. are walked as in gemv_block_add_stream_kernel.
template <uint32_t TYPE, int ITERS, bool FULL>
__global__ __launch_bounds__(1024) void gemv_block_in_stream_kernel(BlockGemv a) {
    constexpr int WAVES = 16;
    constexpr int SBW = (ITERS * 16 + WAVES - 1) / WAVES;
    using WR = typename WRegs<TYPE>::type;
    extern __shared__ __align__(16) uint8_t smem[];
    __shared__ double red[WAVES];
    const int lane = threadIdx.x & 63;
    const int wave_in_wg = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t nw = gridDim.x * WAVES;
    const uint64_t k = a.mat[0].k;
    const uint32_t nsb = (uint32_t)(k / kQK);
    const uint32_t n = a.row_end[a.nmat - 1];
    const ActLds s{smem, k};
    const uint32_t first = blockIdx.x * WAVES + (uint32_t)wave_in_wg;
    auto row_base = [&](uint32_t row) {
        row = row < n ? row : n - 1;  // a wave without rows reads row n-1
        uint32_t mi, local;
        blk_in_row(a, row, mi, local);
        return a.mat[mi].base + (uint64_t)local * a.mat[mi].pitch;
    };

    float4 xv[SBW], nv[SBW];
#pragma unroll
    for (int j = 0; j < SBW; ++j) {
        uint64_t b = (uint64_t)wave_in_wg + (uint64_t)WAVES * j;
        b = b < nsb ? b : nsb - 1;
        xv[j] = reinterpret_cast<const float4*>(a.x + b * kQK)[lane];
        nv[j] = reinterpret_cast<const float4*>(a.norm_w + b * kQK)[lane];
    }
    asm volatile("" ::: "memory");
    WR buf[2];
    load_w<TYPE>(buf[0], row_base(first), nsb, 0, lane);
    {
        double ss = 0.0;
#pragma unroll
        for (int j = 0; j < SBW; ++j) {
            const uint64_t b = (uint64_t)wave_in_wg + (uint64_t)WAVES * j;
            if (b < nsb) {
                ss += (double)xv[j].x * (double)xv[j].x + (double)xv[j].y * (double)xv[j].y +
                      (double)xv[j].z * (double)xv[j].z + (double)xv[j].w * (double)xv[j].w;
            }
        }
        ss = wave_sum_f64(ss);
        if (lane == 0) red[wave_in_wg] = ss;
    }
    __syncthreads();
    double tot = 0.0;
#pragma unroll
    for (int i = 0; i < WAVES; ++i) tot += red[i];
    const float inv = (float)(1.0 / sqrt(tot / (double)k + (double)a.eps));
#pragma unroll
    for (int j = 0; j < SBW; ++j) {
        const uint64_t b = (uint64_t)wave_in_wg + (uint64_t)WAVES * j;
        if (b >= nsb) break;
        float4 v;
        {
#pragma clang fp contract(off)
            v.x = xv[j].x * inv * nv[j].x;
            v.y = xv[j].y * inv * nv[j].y;
            v.z = xv[j].z * inv * nv[j].z;
            v.w = xv[j].w * inv * nv[j].w;
        }
        if (blockIdx.x == 0 && a.norm_out) reinterpret_cast<float4*>(a.norm_out + b * kQK)[lane] = v;
        uint32_t qw;
        int bs;
        float d;
        quantize_block(v, lane, qw, bs, d);
        store_block<TYPE>(s, 0, b, lane, qw, bs, d);
    }
    __syncthreads();
    if (first >= n) return;

    // row -> (matrix, local row) per lane, for the deferred stores
    auto store_row = [&](uint32_t row, float v) {
        uint32_t mi = 0;
#pragma unroll
        for (int i = 0; i < 3; ++i)
            if ((uint32_t)i + 1 < a.nmat && row >= a.row_end[i]) mi = (uint32_t)i + 1;
        const uint32_t local = row - (mi ? a.row_end[mi - 1] : 0u);
        float* dst = mi == 0 ? a.raw[0] : mi == 1 ? a.raw[1] : mi == 2 ? a.raw[2] : a.raw[3];
        dst[local] = v;
        if (mi == 2 && a.v16 != nullptr) a.v16[local] = (_Float16)v;
    };
    const int q = lane & 3;
    const ScaleSel ss = scale_sel(q);
    constexpr bool kActRegs = ITERS <= 2;
    Act act[kActRegs ? ITERS : 1];
    if constexpr (kActRegs) {
#pragma unroll
        for (int it = 0; it < ITERS; ++it) {
            const uint32_t sb = 16u * it + (lane >> 2);
            if (sb < nsb) slice_from_lds<TYPE>(act[it], s, 0, sb, q);
        }
    }
    float acc = 0.0f, out = 0.0f;
    uint32_t out_row = 0, done = 0;
    uint32_t row = first, it = 0;  // the unit whose loads are in flight
    bool more = true;
    while (more) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int its = ITERS == 1 ? 0 : (ITERS == 2 ? j : (int)it);
            asm volatile("s_waitcnt vmcnt(0)" : "+v"(acc), "+v"(out)::"memory");
            uint32_t nrow = row, nit = it + 1;
            if (nit == ITERS) {
                nrow = row + nw < row ? n : row + nw;
                nit = 0;
            }
            more = nrow < n;
            // as gemv_stream_kernel: rows of one unit request nothing past the wave's last row
            if (ITERS != 1 || more) load_w<TYPE>(buf[(j + 1) & 1], row_base(more ? nrow : row), nsb, (int)(more ? nit : it), lane);
            hold<TYPE>(buf[j & 1]);
            const uint32_t sb = 16u * (uint32_t)its + (lane >> 2);
            if (FULL || sb < nsb) {
                if constexpr (kActRegs) {
                    acc = lane_fma(decode_w<TYPE>(buf[j & 1], ss, q), act[its], acc);
                } else {
                    Act av;
                    slice_from_lds<TYPE>(av, s, 0, sb, q);
                    acc = lane_fma(decode_w<TYPE>(buf[j & 1], ss, q), av, acc);
                }
            }
            if (it == ITERS - 1) {
                const float v = wave_sum_uniform(acc);
                const bool mine = lane == (int)(done & 63u);
                out = mine ? v : out;
                out_row = mine ? row : out_row;
                acc = 0.0f;
                ++done;
                if ((done & 63u) == 0u) store_row(out_row, out);
            }
            row = nrow;
            it = nit;
            if (!more) break;
        }
    }
    if ((uint32_t)lane < (done & 63u)) store_row(out_row, out);
}

template <uint32_t TYPE, int ITERS, bool FULL>
hipError_t launch_block_in_stream(const BlockGemv& a, hipStream_t s) {
    const uint64_t lds = act_lds_bytes(a.mat[0].k, 1);
    uint64_t wgs = (uint64_t)cu_count();
    const uint64_t need = ((uint64_t)a.row_end[a.nmat - 1] + 15) / 16;
    if (wgs > need) wgs = need;
    hipLaunchKernelGGL((gemv_block_in_stream_kernel<TYPE, ITERS, FULL>), dim3((unsigned)wgs), dim3(1024), lds, s, a);
    return hipGetLastError();
}

template <uint32_t TYPE, int ITERS, bool FULL>
hipError_t launch_block_add_stream(const BlockGemv& a, hipStream_t s) {
    const uint64_t lds = act_lds_bytes(a.mat[0].k, 1);
    uint64_t wgs = (uint64_t)cu_count();
    const uint64_t need = (a.mat[0].n + 15) / 16;
    if (wgs > need) wgs = need;
    hipLaunchKernelGGL((gemv_block_add_stream_kernel<TYPE, ITERS, FULL>), dim3((unsigned)wgs), dim3(1024), lds, s, a);
    return hipGetLastError();
}

template <uint32_t TYPE, int ITERS, int MODE, bool FULL>
hipError_t launch_block_full(const BlockGemv& a, hipStream_t s) {
    if constexpr (MODE == kBlockAdd) {
        // the residual projections without a normalising prologue stream like the plain decode
        // GEMV (FFN down 4096 x 12288: 9.3 us against 11.1 us in the structure below)
        if (gemv_block_add_streams(a)) return launch_block_add_stream<TYPE, ITERS, FULL>(a, s);
        if (a.rec != nullptr) return hipErrorInvalidValue;  // only the streamed kernel forms the gated row
    }
    if constexpr (MODE == kBlockIn) {
        if (gemv_block_in_streams(a)) return launch_block_in_stream<TYPE, ITERS, FULL>(a, s);
    }
    const uint64_t groups = MODE == kBlockFfn ? a.mat[0].n : ((uint64_t)a.row_end[a.nmat - 1] + 1) / 2;
    const uint64_t lds = act_lds_bytes(a.mat[0].k, 1);
    static const int resident = [lds] {
        int n = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, gemv_block_kernel<TYPE, ITERS, MODE, FULL>, 512, lds) !=
                hipSuccess || n < 1) {
            n = 1;
        }
        return n;
    }();
    uint64_t wgs = (uint64_t)cu_count() * (uint64_t)(resident < 2 ? resident : 2);
    const uint64_t need = (groups + 7) / 8;
    if (wgs > need) wgs = need;
    hipLaunchKernelGGL((gemv_block_kernel<TYPE, ITERS, MODE, FULL>), dim3((unsigned)wgs), dim3(512), lds, s, a);
    return hipGetLastError();
}

template <uint32_t TYPE, int MODE>
hipError_t launch_block_type(const BlockGemv& a, hipStream_t s) {
    const uint64_t nsb = a.mat[0].k / kQK;
    const bool full = nsb % 16 == 0;
    switch ((nsb + 15) / 16) {
        case 1: return full ? launch_block_full<TYPE, 1, MODE, true>(a, s) : launch_block_full<TYPE, 1, MODE, false>(a, s);
        case 2: return full ? launch_block_full<TYPE, 2, MODE, true>(a, s) : launch_block_full<TYPE, 2, MODE, false>(a, s);
        case 3: return full ? launch_block_full<TYPE, 3, MODE, true>(a, s) : launch_block_full<TYPE, 3, MODE, false>(a, s);
        default: return hipErrorNotSupported;
    }
}

template <int MODE>
hipError_t launch_block_mode(const BlockGemv& a, hipStream_t s) {
    switch (a.mat[0].type) {
        case 12: return launch_block_type<12, MODE>(a, s);
        case 14: return launch_block_type<14, MODE>(a, s);
        default: return hipErrorNotSupported;
    }
}

}  // namespace

bool gemv_block_add_streams(const BlockGemv& a) { return a.norm_w == nullptr && knob(kBlockStream, 1) != 0; }

bool gemv_block_in_streams(const BlockGemv& a) {
    return a.norm_w != nullptr && a.conv_w == nullptr && a.beta_s == nullptr && a.log_decay == nullptr &&
           knob(kBlockStream, 1) != 0;
}

bool gemv_block_supported(const BlockGemv& a) {
    if (a.nmat < 1 || a.nmat > 4) return false;
    const DeviceMatrix& w0 = a.mat[0];
    if ((w0.type != 12 && w0.type != 14) || w0.k % kQK != 0 || (w0.k / kQK + 15) / 16 > 3) return false;
    if (act_lds_bytes(w0.k, 1) > kLdsBudget) return false;
    for (uint32_t i = 1; i < a.nmat; ++i) {
        if (a.mat[i].type != w0.type || a.mat[i].k != w0.k || a.mat[i].pitch != w0.pitch) return false;
    }
    return true;
}

hipError_t launch_gemv_block(int mode, const BlockGemv& a, hipStream_t s) {
    if (!gemv_block_supported(a)) return hipErrorNotSupported;
    switch (mode) {
        case kBlockIn: return launch_block_mode<kBlockIn>(a, s);
        case kBlockAdd: return launch_block_mode<kBlockAdd>(a, s);
        case kBlockFfn: return launch_block_mode<kBlockFfn>(a, s);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace oq
