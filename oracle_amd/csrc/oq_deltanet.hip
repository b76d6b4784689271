// Gated DeltaNet (linear-attention) decode block at batch 1 on gfx950: the elementwise and
// per-head kernels between the block's quantized projections.
//
// The block order is the reference's execute_qwen35_recurrent_block_reference
// (src/runtime/qwen35_block.cpp:406-605) followed by finish_block (:326-352) and execute_mlp
// (:296-324); the projections are launched by the C ABI (oq_api.cpp) on the GEMV kernels.
// Arithmetic follows the reference's: F32 values, double sums of squares, the gated delta
// rule's memory in F32 key order and its output in double (reference_kernels.cpp:227-335), and
// no fused multiply-add where the reference multiplies and adds separately.
#include "oq_common.h"

// The reference multiplies and adds separately (no contraction) everywhere on this path.
#pragma clang fp contract(off)

namespace oq {

namespace {

constexpr int kNormThreads = 1024;
constexpr int kMaxConvKernel = 16;

// sum over the workgroup (blockDim.x a multiple of 64, at most 1024); every thread gets it
OQ_DEVICE double block_sum_f64(double v, double* lds) {
    v = wave_sum_f64(v);
    const int wave = threadIdx.x >> 6, waves = blockDim.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) lds[wave] = v;
    __syncthreads();
    double s = 0.0;
    for (int i = 0; i < waves; ++i) s += lds[i];
    return s;
}

// out = rms_norm(a [+ b]) * w over one row of n values (qwen35_block.cpp:161-186); with b the
// sum a + b is also stored to sum_out (the block's residual, qwen35_block.cpp:334).
__global__ __launch_bounds__(kNormThreads) void rmsnorm_kernel(const float* __restrict__ a, const float* __restrict__ b,
                                                               const float* __restrict__ w, uint32_t n, float eps,
                                                               float* __restrict__ sum_out, float* __restrict__ out,
                                                               uint8_t* __restrict__ q8) {
    __shared__ double red[16];
    // workgroup r normalises row r (rows of n values, consecutive)
    const uint64_t row = (uint64_t)blockIdx.x * n;
    a += row;
    if (b) {
        b += row;
        sum_out += row;
    }
    out += row;
    double ss = 0.0;
    for (uint32_t i = threadIdx.x; i < n; i += blockDim.x) {
        float v = a[i];
        if (b) {
            v = v + b[i];
            sum_out[i] = v;
        }
        ss += (double)v * (double)v;
    }
    ss = block_sum_f64(ss, red);
    const float inv = (float)(1.0 / sqrt(ss / (double)n + (double)eps));
    for (uint32_t i = threadIdx.x; i < n; i += blockDim.x) {
        const float v = b ? sum_out[i] : a[i];
        out[i] = v * inv * w[i];
    }
    if (q8 != nullptr) {
        // the row's Q8_K blocks (n a multiple of 256), one wave per block, from the values just
        // stored: quantize_q8k_kernel's quantization of the same values
        __syncthreads();
        const int lane = threadIdx.x & 63;
        const uint32_t nb = n / kQK;
        for (uint32_t blk = threadIdx.x >> 6; blk < nb; blk += kNormThreads / 64) {
            const float4 v = reinterpret_cast<const float4*>(out + (uint64_t)blk * kQK)[lane];
            store_q8k_block(q8 + ((uint64_t)blockIdx.x * nb + blk) * kQ8KBytes, quantize_q8k_block_wave(v, lane), lane);
        }
    }
}

// rmsnorm_kernel's values for rows of n = 256 * nb values (nb <= kNormWaves * NBW), one workgroup
// per row with every value in registers: wave w holds the 256-blocks w, w + kNormWaves, ... (lane
// l: values 4l..4l+3 of each), so the row is read once and its Q8_K blocks come from the same
// registers.  The sum of squares is the small-batch kernels' staging order (each lane's four
// squares in order, the wave's butterfly per block, the blocks' sums in block order), so a row
// normalised here and one normalised in that staging have the same bits.
constexpr int kNormWaves = 8;
template <int NBW>
__global__ __launch_bounds__(64 * kNormWaves) void rmsnorm_blocks_kernel(
    const float* __restrict__ a, const float* __restrict__ b, const float* __restrict__ w, uint32_t nb, float eps,
    float* __restrict__ sum_out, float* __restrict__ out, uint8_t* __restrict__ q8) {
#pragma clang fp contract(off)
    __shared__ double red[kNormWaves * NBW];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint64_t n = (uint64_t)nb * kQK, row = (uint64_t)blockIdx.x * n;
    float4 v[NBW], wv[NBW];
#pragma unroll
    for (int j = 0; j < NBW; ++j) {
        uint32_t blk = (uint32_t)wave + kNormWaves * j;
        blk = blk < nb ? blk : nb - 1;
        const uint64_t i = row + (uint64_t)blk * kQK + 4u * (uint32_t)lane;
        v[j] = *reinterpret_cast<const float4*>(a + i);
        if (b != nullptr) {
            const float4 u = *reinterpret_cast<const float4*>(b + i);
            v[j] = make_float4(v[j].x + u.x, v[j].y + u.y, v[j].z + u.z, v[j].w + u.w);
        }
        wv[j] = *reinterpret_cast<const float4*>(w + (uint64_t)blk * kQK + 4u * (uint32_t)lane);
    }
#pragma unroll
    for (int j = 0; j < NBW; ++j) {
        const uint32_t blk = (uint32_t)wave + kNormWaves * j;
        if (blk >= nb) break;
        if (b != nullptr) *reinterpret_cast<float4*>(sum_out + row + (uint64_t)blk * kQK + 4u * (uint32_t)lane) = v[j];
        const double sq = (double)v[j].x * (double)v[j].x + (double)v[j].y * (double)v[j].y +
                          (double)v[j].z * (double)v[j].z + (double)v[j].w * (double)v[j].w;
        const double bs = wave_sum_f64(sq);
        if (lane == 0) red[blk] = bs;
    }
    __syncthreads();
    double tot = 0.0;
    for (uint32_t c = 0; c < nb; ++c) tot += red[c];
    const float inv = (float)(1.0 / sqrt(tot / (double)n + (double)eps));
#pragma unroll
    for (int j = 0; j < NBW; ++j) {
        const uint32_t blk = (uint32_t)wave + kNormWaves * j;
        if (blk >= nb) break;
        const float4 o = make_float4(v[j].x * inv * wv[j].x, v[j].y * inv * wv[j].y, v[j].z * inv * wv[j].z,
                                     v[j].w * inv * wv[j].w);
        *reinterpret_cast<float4*>(out + row + (uint64_t)blk * kQK + 4u * (uint32_t)lane) = o;
        if (q8 != nullptr)
            store_q8k_block(q8 + ((uint64_t)blockIdx.x * nb + blk) * kQ8KBytes, quantize_q8k_block_wave(o, lane), lane);
    }
}

// Causal depthwise convolution step with SiLU (reference_kernels.cpp:197-225 with
// qwen35_block.cpp:500-503) over `channels` channels of `kernel` taps; the first workgroup
// also forms the per-head gates: beta_s = sigmoid(beta), log_decay = softplus(alpha + dt_bias)
// * decay (qwen35_block.cpp:464-494).
__global__ __launch_bounds__(256) void conv_gates_kernel(const float* __restrict__ qkv, const float* __restrict__ conv_w,
                                                         float* __restrict__ history, uint32_t channels, uint32_t kernel,
                                                         const float* __restrict__ beta, const float* __restrict__ alpha,
                                                         const float* __restrict__ dt_bias,
                                                         const float* __restrict__ decay, uint32_t heads,
                                                         float* __restrict__ conv_out, float* __restrict__ beta_s,
                                                         float* __restrict__ log_decay) {
    const uint32_t c = blockIdx.x * 256 + threadIdx.x;
    if (blockIdx.x == 0) {
        for (uint32_t h = threadIdx.x; h < heads; h += 256) {
            beta_s[h] = sigmoid_ref(beta[h]);
            log_decay[h] = softplus_ref(alpha[h] + dt_bias[h]) * decay[h];
        }
    }
    if (c >= channels) return;
    float* hst = history + (uint64_t)c * kernel;
    const float* wc = conv_w + (uint64_t)c * kernel;
    double sum = 0.0;
    for (uint32_t i = 0; i < kernel; ++i) {
        // shift left in place (tap i + 1 is read before it is overwritten), append the input
        const float t = i + 1 < kernel ? hst[i + 1] : qkv[c];
        hst[i] = t;
        sum += (double)t * (double)wc[i];
    }
    conv_out[c] = silu_ref((float)sum);
}

// The same for `tokens` consecutive tokens: qkv [tokens][channels] -> conv_out [tokens][channels],
// the history advanced once per token in token order (as `tokens` calls of the step), the gates
// per (token, head).
__global__ __launch_bounds__(256) void conv_gates_tokens_kernel(
    const float* __restrict__ qkv, const float* __restrict__ conv_w, float* __restrict__ history, uint32_t channels,
    uint32_t kernel, const float* __restrict__ beta, const float* __restrict__ alpha,
    const float* __restrict__ dt_bias, const float* __restrict__ decay, uint32_t heads, uint32_t tokens,
    float* __restrict__ conv_out, float* __restrict__ beta_s, float* __restrict__ log_decay) {
    const uint32_t c = blockIdx.x * 256 + threadIdx.x;
    if (blockIdx.x == 0) {
        for (uint32_t i = threadIdx.x; i < heads * tokens; i += 256) {
            const uint32_t h = i % heads;
            beta_s[i] = sigmoid_ref(beta[i]);
            log_decay[i] = softplus_ref(alpha[i] + dt_bias[h]) * decay[h];
        }
    }
    if (c >= channels) return;
    float* hst = history + (uint64_t)c * kernel;
    const float* wc = conv_w + (uint64_t)c * kernel;
    for (uint32_t t = 0; t < tokens; ++t) {
        double sum = 0.0;
        for (uint32_t i = 0; i < kernel; ++i) {
            const float v = i + 1 < kernel ? hst[i + 1] : qkv[(uint64_t)t * channels + c];
            hst[i] = v;
            sum += (double)v * (double)wc[i];
        }
        conv_out[(uint64_t)t * channels + c] = silu_ref((float)sum);
    }
}

// The gated delta rule step (reference_kernels.cpp:227-335) on the state [head][key][value],
// one workgroup per (value head h, chunk of 32 value columns), 256 threads = 8 key slices x 32
// columns: thread (slice, column) keeps the DK/8 state values of its column and key slice in
// registers, so the head's state is read once and written once by DK/8-deep chains spread over
// Hv * dv/32 workgroups.  The head's query/key come from key head h % Hk (repeat_heads_tiled,
// qwen35_block.cpp:233-251), L2-normalised by the first wave (double sums of squares, the scale
// 1/max(norm, eps) rounded to F32, q also by 1/sqrt(DK)).  Per column: the decayed state's memory
// sum_k S k is formed in F32 per key slice in key order, then over the slices in key order;
// delta = (v - memory) * beta; the updated column's output sum_k S q in double the same way.
// Outputs: rec_out[h][v] and, per (head, chunk), the double sum of the chunk's rec_out^2 in
// head_ss[h * chunks + chunk] -- the head's gated RMSNorm (qwen35_block.cpp:579-588) is applied
// where rec_out is consumed (gated_norm_kernel, or the out projection's activation staging).  With
// z_silu set, the chunk's columns of the gate row z also leave as SiLU(z) (z requested with the
// state), so that the out projection's staging reads a row this launch has just written instead of
// z, written three launches earlier (measured: out projection 8.5 -> 7.3 us without the z loads).
// value columns per workgroup of the delta rule and per head_ss entry (16 measured slower:
// more workgroups, each with a shorter chain, 49.9 against 48.6 us per block)
constexpr int kDeltaCols = 32;

//
// With tokens > 1 the launch runs `tokens` consecutive steps (token t's conv row at conv + t * C,
// its gates at beta_s / log_decay + t * Hv, its outputs at rec_out + t * Hv * dv and head_ss +
// t * Hv * chunks): each thread keeps its state values in registers from the first token to the
// last, and every token's arithmetic is that of a single step, so the results equal `tokens`
// launches bit for bit while the state is read and written once.
template <int DK, int COLS>
__global__ __launch_bounds__(256) void delta_kernel(const float* __restrict__ conv, uint32_t key_heads, uint32_t dv,
                                                    const float* __restrict__ beta_s, const float* __restrict__ log_decay,
                                                    float eps, float* __restrict__ state, float* __restrict__ rec_out,
                                                    double* __restrict__ head_ss, const float* __restrict__ z,
                                                    float* __restrict__ z_silu, uint32_t tokens, uint32_t value_heads) {
    constexpr int SLICES = 256 / COLS;
    constexpr int KS = DK / SLICES;  // keys per thread
    __shared__ __align__(16) float nq[DK];
    __shared__ __align__(16) float nk[DK];
    __shared__ float mem_part[SLICES][COLS];
    __shared__ double out_part[SLICES][COLS];
    const uint32_t chunks = dv / COLS;
    const uint32_t h = blockIdx.x / chunks, chunk = blockIdx.x % chunks;
    const uint32_t col = threadIdx.x % COLS, slice = threadIdx.x / COLS;
    const uint32_t v = chunk * COLS + col;
    const uint32_t d0 = slice * KS;
    float* scol = state + ((uint64_t)h * DK + d0) * dv + v;
    const uint32_t kw = key_heads * DK;
    const uint64_t cstride = 2ull * kw + (uint64_t)value_heads * dv;  // one token's conv row
    // every input is requested before the first barrier
    float s[KS];
#pragma unroll
    for (int i = 0; i < KS; ++i) s[i] = scol[(uint64_t)i * dv];
    for (uint32_t t = 0; t < tokens; ++t) {
    if (t > 0) __syncthreads();  // the previous token's reads of nq / nk and the partial sums are done
    const float* q = conv + t * cstride + (uint64_t)(h % key_heads) * DK;
    const float* k = conv + t * cstride + kw + (uint64_t)(h % key_heads) * DK;
    const float vv = conv[t * cstride + 2u * kw + (uint64_t)h * dv + v];
    const float zv = z_silu != nullptr && slice == 0 ? z[(uint64_t)h * dv + v] : 0.0f;
    const float ldh = log_decay[(uint64_t)t * value_heads + h];
    const float beta = beta_s[(uint64_t)t * value_heads + h];
    if (threadIdx.x < 64) {
        // the first wave: L2 norms of the head's query and key (DK <= 128: two values per lane)
        const int lane = threadIdx.x;
        const float q0 = lane < DK ? q[lane] : 0.0f, k0 = lane < DK ? k[lane] : 0.0f;
        const float q1 = lane + 64 < DK ? q[lane + 64] : 0.0f, k1 = lane + 64 < DK ? k[lane + 64] : 0.0f;
        const double qs = wave_sum_f64((double)q0 * (double)q0 + (double)q1 * (double)q1);
        const double ks = wave_sum_f64((double)k0 * (double)k0 + (double)k1 * (double)k1);
        const double ql = sqrt(qs), kl = sqrt(ks);
        const float iq = (float)(1.0 / (ql > (double)eps ? ql : (double)eps));
        const float ik = (float)(1.0 / (kl > (double)eps ? kl : (double)eps));
        const float query_scale = 1.0f / sqrtf((float)DK);
        if (lane < DK) {
            nq[lane] = q0 * iq * query_scale;
            nk[lane] = k0 * ik;
        }
        if (lane + 64 < DK) {
            nq[lane + 64] = q1 * iq * query_scale;
            nk[lane + 64] = k1 * ik;
        }
    }
    __syncthreads();

    const float decay = expf(ldh);
    float mem = 0.0f;
#pragma unroll
    for (int i = 0; i < KS; ++i) {
        s[i] = s[i] * decay;
        mem = mem + s[i] * nk[d0 + i];
    }
    mem_part[slice][col] = mem;
    __syncthreads();
    float memory = 0.0f;
#pragma unroll
    for (int j = 0; j < SLICES; ++j) memory = memory + mem_part[j][col];
    const float delta = (vv - memory) * beta;
    double o = 0.0;
#pragma unroll
    for (int i = 0; i < KS; ++i) {
        s[i] = s[i] + nk[d0 + i] * delta;
        o = o + (double)s[i] * (double)nq[d0 + i];
    }
    out_part[slice][col] = o;
    __syncthreads();
    if (slice == 0) {
        double out = 0.0;
#pragma unroll
        for (int j = 0; j < SLICES; ++j) out = out + out_part[j][col];
        const float of = (float)out;
        const uint64_t vt = (uint64_t)t * value_heads * dv;
        rec_out[vt + (uint64_t)h * dv + v] = of;
        // the chunk's sum of squares over its COLS columns (the first COLS lanes of wave 0)
        double sq = (double)of * (double)of;
#pragma unroll
        for (int off = COLS / 2; off >= 1; off >>= 1) sq += __shfl_xor(sq, off, 64);
        if (col == 0) head_ss[(uint64_t)t * value_heads * chunks + (uint64_t)h * chunks + chunk] = sq;
        if (z_silu != nullptr) z_silu[(uint64_t)h * dv + v] = silu_ref(zv);
    }
    }
#pragma unroll
    for (int i = 0; i < KS; ++i) scol[(uint64_t)i * dv] = s[i];
}

// Any key and value width (the reference's gated_delta_step, reference_kernels.cpp:227-335, takes any
// shape): delta_kernel's workgroups (one per (value head, chunk of COLS value columns), the last chunk
// of a head possibly partial; 256 threads = 8 key slices x 32 columns, slice j owning keys
// [j ks, min(dk, (j + 1) ks)) with ks = ceil(dk / 8)) and its arithmetic in the same order, with the
// state in HBM instead of registers: a thread reads its entries for the memory sum and rewrites them
// with the update, every token.  At the widths delta_kernel takes, the two give the same bits.  The
// normalised query and key sit in dynamic LDS (2 dk floats).  query_scale = 1/sqrt(dk), rounded on
// the host as the register kernel's compile-time constant is.
__global__ __launch_bounds__(256) void delta_any_kernel(const float* __restrict__ conv, uint32_t key_heads, uint32_t dk,
                                                        uint32_t dv, const float* __restrict__ beta_s,
                                                        const float* __restrict__ log_decay, float eps, float query_scale,
                                                        float* __restrict__ state, float* __restrict__ rec_out,
                                                        double* __restrict__ head_ss, uint32_t tokens,
                                                        uint32_t value_heads) {
    constexpr int COLS = kDeltaCols, SLICES = 256 / COLS;
    extern __shared__ __align__(16) float nqk[];  // nq[dk], then nk[dk]
    float* nq = nqk;
    float* nk = nqk + dk;
    __shared__ float mem_part[SLICES][COLS];
    __shared__ double out_part[SLICES][COLS];
    const uint32_t chunks = (dv + COLS - 1) / COLS;
    const uint32_t h = blockIdx.x / chunks, chunk = blockIdx.x % chunks;
    const uint32_t col = threadIdx.x % COLS, slice = threadIdx.x / COLS;
    const uint32_t v = chunk * COLS + col;
    const bool vok = v < dv;
    const uint32_t ks = (dk + SLICES - 1) / SLICES;
    const uint32_t d0 = min(dk, slice * ks), d1 = min(dk, d0 + ks);
    float* scol = state + (uint64_t)h * dk * dv + v;  // key d's entry at scol[d * dv]
    const uint32_t kw = key_heads * dk;
    const uint64_t cstride = 2ull * kw + (uint64_t)value_heads * dv;  // one token's conv row
    for (uint32_t t = 0; t < tokens; ++t) {
        if (t > 0) __syncthreads();  // the previous token's reads of nq / nk and the partial sums are done
        const float* q = conv + t * cstride + (uint64_t)(h % key_heads) * dk;
        const float* k = conv + t * cstride + kw + (uint64_t)(h % key_heads) * dk;
        const float vv = vok ? conv[t * cstride + 2ull * kw + (uint64_t)h * dv + v] : 0.0f;
        const float ldh = log_decay[(uint64_t)t * value_heads + h];
        const float beta = beta_s[(uint64_t)t * value_heads + h];
        if (threadIdx.x < 64) {
            // the first wave: L2 norms of the head's query and key, lane i summing elements i, i + 64, ...
            const uint32_t lane = threadIdx.x;
            double qs = 0.0, kss = 0.0;
            for (uint32_t e = lane; e < dk; e += 64) {
                qs = qs + (double)q[e] * (double)q[e];
                kss = kss + (double)k[e] * (double)k[e];
            }
            qs = wave_sum_f64(qs);
            kss = wave_sum_f64(kss);
            const double ql = sqrt(qs), kl = sqrt(kss);
            const float iq = (float)(1.0 / (ql > (double)eps ? ql : (double)eps));
            const float ik = (float)(1.0 / (kl > (double)eps ? kl : (double)eps));
            for (uint32_t e = lane; e < dk; e += 64) {
                nq[e] = q[e] * iq * query_scale;
                nk[e] = k[e] * ik;
            }
        }
        __syncthreads();
        const float decay = expf(ldh);
        float mem = 0.0f;
        if (vok) {
            for (uint32_t d = d0; d < d1; ++d) mem = mem + (scol[(uint64_t)d * dv] * decay) * nk[d];
        }
        mem_part[slice][col] = mem;
        __syncthreads();
        float memory = 0.0f;
#pragma unroll
        for (int j = 0; j < SLICES; ++j) memory = memory + mem_part[j][col];
        const float delta = (vv - memory) * beta;
        double o = 0.0;
        if (vok) {
            for (uint32_t d = d0; d < d1; ++d) {
                float sv = scol[(uint64_t)d * dv] * decay;
                sv = sv + nk[d] * delta;
                scol[(uint64_t)d * dv] = sv;
                o = o + (double)sv * (double)nq[d];
            }
        }
        out_part[slice][col] = o;
        __syncthreads();
        if (slice == 0) {
            double out = 0.0;
#pragma unroll
            for (int j = 0; j < SLICES; ++j) out = out + out_part[j][col];
            const float of = (float)out;
            if (vok) rec_out[(uint64_t)t * value_heads * dv + (uint64_t)h * dv + v] = of;
            double sq = vok ? (double)of * (double)of : 0.0;
#pragma unroll
            for (int off = COLS / 2; off >= 1; off >>= 1) sq += __shfl_xor(sq, off, 64);
            if (col == 0) head_ss[(uint64_t)t * value_heads * chunks + (uint64_t)h * chunks + chunk] = sq;
        }
    }
}

// gated[h][v] = RMSNorm(rec[h])[v] * out_norm[v] * SiLU(z[h][v]) (qwen35_block.cpp:579-588), the
// head's sum of squares taken from the delta kernel's per-chunk partials (added in chunk order).
__global__ __launch_bounds__(256) void gated_norm_kernel(const float* __restrict__ rec, const double* __restrict__ head_ss,
                                                         const float* __restrict__ z, const float* __restrict__ out_norm,
                                                         uint32_t total, uint32_t dv, uint32_t chunks, float eps,
                                                         float* __restrict__ gated) {
    // i over tokens x heads x dv: token rows of rec / z / gated are consecutive, as are the
    // tokens' head_ss rows
    const uint32_t i = blockIdx.x * 256 + threadIdx.x;
    if (i >= total) return;
    const uint32_t hv = i / dv, v = i % dv;  // hv = token * heads + head
    double ss = 0.0;
    for (uint32_t c = 0; c < chunks; ++c) ss += head_ss[(uint64_t)hv * chunks + c];
    const float inv = (float)(1.0 / sqrt(ss / (double)dv + (double)eps));
    gated[i] = rec[i] * inv * out_norm[v] * silu_ref(z[i]);
}

// gated_norm_kernel's values and their Q8_K blocks (quantize_q8k_kernel's layout; dv a multiple of
// 64, so a lane's four values lie in one head): one wave per 256 values
__global__ __launch_bounds__(256) void gated_norm_q8k_kernel(const float* __restrict__ rec, const double* __restrict__ head_ss,
                                                             const float* __restrict__ z, const float* __restrict__ out_norm,
                                                             uint64_t nblocks, uint32_t dv, uint32_t chunks, float eps,
                                                             float* __restrict__ gated, uint8_t* __restrict__ q8) {
    const int lane = threadIdx.x & 63;
    const uint64_t blk = blockIdx.x * 4ull + (threadIdx.x >> 6);
    if (blk >= nblocks) return;
    const uint64_t i = blk * kQK + 4u * (uint32_t)lane;
    const uint64_t hv = i / dv;
    const uint32_t v = (uint32_t)(i % dv);
    double ss = 0.0;
    for (uint32_t c = 0; c < chunks; ++c) ss += head_ss[hv * chunks + c];
    const float inv = (float)(1.0 / sqrt(ss / (double)dv + (double)eps));
    const float4 r = *reinterpret_cast<const float4*>(rec + i), zz = *reinterpret_cast<const float4*>(z + i);
    const float* w = out_norm + v;  // a caller's vector: 4-byte alignment only
    const float4 g = make_float4(r.x * inv * w[0] * silu_ref(zz.x), r.y * inv * w[1] * silu_ref(zz.y),
                                 r.z * inv * w[2] * silu_ref(zz.z), r.w * inv * w[3] * silu_ref(zz.w));
    *reinterpret_cast<float4*>(gated + i) = g;
    store_q8k_block(q8 + blk * kQ8KBytes, quantize_q8k_block_wave(g, lane), lane);
}

// act = silu(gate) * up (qwen35_block.cpp:313-316)
__global__ __launch_bounds__(256) void swiglu_kernel(const float* __restrict__ gate, const float* __restrict__ up,
                                                     uint32_t n, float* __restrict__ act) {
    const uint32_t i = blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    act[i] = silu_ref(gate[i]) * up[i];
}

// swiglu_kernel's values, and their Q8_K blocks (quantize_q8k_kernel's layout over the n values,
// n a multiple of 256): one wave per block
__global__ __launch_bounds__(256) void swiglu_q8k_kernel(const float* __restrict__ gate, const float* __restrict__ up,
                                                         uint64_t nblocks, float* __restrict__ act, uint8_t* __restrict__ q8) {
    const int lane = threadIdx.x & 63;
    const uint64_t blk = blockIdx.x * 4ull + (threadIdx.x >> 6);
    if (blk >= nblocks) return;
    const uint64_t i = blk * kQK + 4u * (uint32_t)lane;
    const float4 g = *reinterpret_cast<const float4*>(gate + i), u = *reinterpret_cast<const float4*>(up + i);
    const float4 v = make_float4(silu_ref(g.x) * u.x, silu_ref(g.y) * u.y, silu_ref(g.z) * u.z, silu_ref(g.w) * u.w);
    *reinterpret_cast<float4*>(act + i) = v;
    store_q8k_block(q8 + blk * kQ8KBytes, quantize_q8k_block_wave(v, lane), lane);
}

// out = a + b (qwen35_block.cpp:188-198)
__global__ __launch_bounds__(256) void add_kernel(const float* __restrict__ a, const float* __restrict__ b, uint32_t n,
                                                  float* __restrict__ out) {
    const uint32_t i = blockIdx.x * 256 + threadIdx.x;
    if (i < n) out[i] = a[i] + b[i];
}

unsigned blocks_of(uint64_t n, unsigned t) { return (unsigned)((n + t - 1) / t); }

}  // namespace

bool deltanet_dims_supported(uint64_t key_dim, uint64_t value_dim, uint64_t conv_kernel) {
    return (key_dim == 32 || key_dim == 64 || key_dim == 128) && value_dim >= 64 && value_dim <= 256 &&
           value_dim % 64 == 0 && conv_kernel >= 1 && conv_kernel <= kMaxConvKernel && knob(kAnyShape, 0) == 0;
}

bool deltanet_dims_any(uint64_t key_dim, uint64_t value_dim, uint64_t conv_kernel) {
    return key_dim >= 1 && key_dim <= kDeltaMaxKeyDim && value_dim >= 1 && value_dim <= 0xFFFFFFFFull &&
           conv_kernel >= 1 && conv_kernel <= 0xFFFFFFFFull;
}

hipError_t launch_rmsnorm(const float* a, const float* b, const float* w, uint64_t n, float eps, float* sum_out,
                          float* out, hipStream_t s, uint64_t rows, uint8_t* q8) {
    if (q8 != nullptr && n % kQK != 0) return hipErrorInvalidValue;
    // rows of whole 256-blocks, up to 16384 values: every value in registers, read once
    const uint64_t nb = n / kQK;
    if (n % kQK == 0 && nb >= 1 && nb <= (uint64_t)kNormWaves * 8) {
        const bool aligned16 = ((reinterpret_cast<uintptr_t>(a) | reinterpret_cast<uintptr_t>(b) |
                                 reinterpret_cast<uintptr_t>(w) | reinterpret_cast<uintptr_t>(sum_out) |
                                 reinterpret_cast<uintptr_t>(out)) & 15u) == 0;
        if (aligned16) {
            if (nb <= (uint64_t)kNormWaves * 2) {
                hipLaunchKernelGGL(rmsnorm_blocks_kernel<2>, dim3((unsigned)rows), dim3(64 * kNormWaves), 0, s, a, b, w,
                                   (uint32_t)nb, eps, sum_out, out, q8);
            } else {
                hipLaunchKernelGGL(rmsnorm_blocks_kernel<8>, dim3((unsigned)rows), dim3(64 * kNormWaves), 0, s, a, b, w,
                                   (uint32_t)nb, eps, sum_out, out, q8);
            }
            return hipGetLastError();
        }
    }
    hipLaunchKernelGGL(rmsnorm_kernel, dim3((unsigned)rows), dim3(kNormThreads), 0, s, a, b, w, (uint32_t)n, eps, sum_out,
                       out, q8);
    return hipGetLastError();
}

hipError_t launch_conv_gates_tokens(const float* qkv, const float* conv_w, float* history, uint64_t channels,
                                    uint64_t kernel, const float* beta, const float* alpha, const float* dt_bias,
                                    const float* decay, uint64_t heads, uint64_t tokens, float* conv_out,
                                    float* beta_s, float* log_decay, hipStream_t s) {
    hipLaunchKernelGGL(conv_gates_tokens_kernel, dim3(blocks_of(channels, 256)), dim3(256), 0, s, qkv, conv_w, history,
                       (uint32_t)channels, (uint32_t)kernel, beta, alpha, dt_bias, decay, (uint32_t)heads,
                       (uint32_t)tokens, conv_out, beta_s, log_decay);
    return hipGetLastError();
}

hipError_t launch_conv_gates(const float* qkv, const float* conv_w, float* history, uint64_t channels,
                             uint64_t kernel, const float* beta, const float* alpha, const float* dt_bias,
                             const float* decay, uint64_t heads, float* conv_out, float* beta_s, float* log_decay,
                             hipStream_t s) {
    hipLaunchKernelGGL(conv_gates_kernel, dim3(blocks_of(channels, 256)), dim3(256), 0, s, qkv, conv_w, history,
                       (uint32_t)channels, (uint32_t)kernel, beta, alpha, dt_bias, decay, (uint32_t)heads, conv_out,
                       beta_s, log_decay);
    return hipGetLastError();
}

hipError_t launch_delta(const float* conv, uint64_t key_heads, uint64_t value_heads, uint64_t dk, uint64_t dv,
                        const float* beta_s, const float* log_decay, float eps, float* state, float* rec_out,
                        double* head_ss, const float* z, float* z_silu, hipStream_t s, uint64_t tokens) {
    if (tokens > 1 && z_silu != nullptr) return hipErrorInvalidValue;  // SiLU(z) is a single-token epilogue
    if ((z == nullptr) != (z_silu == nullptr)) return hipErrorInvalidValue;
    const bool regs = (dk == 32 || dk == 64 || dk == 128) && dv % kDeltaCols == 0 && knob(kAnyShape, 0) == 0;
    if (!regs) {
        if (z_silu != nullptr || dk == 0 || dk > kDeltaMaxKeyDim || dv == 0 || value_heads == 0 || key_heads == 0)
            return hipErrorInvalidValue;
        const uint64_t grid = value_heads * delta_chunks(dv);
        if (grid > 0x7FFFFFFFull) return hipErrorInvalidValue;
        const float query_scale = 1.0f / std::sqrt((float)dk);
        hipLaunchKernelGGL(delta_any_kernel, dim3((unsigned)grid), dim3(256), 2 * dk * sizeof(float), s, conv,
                           (uint32_t)key_heads, (uint32_t)dk, (uint32_t)dv, beta_s, log_decay, eps, query_scale, state,
                           rec_out, head_ss, (uint32_t)tokens, (uint32_t)value_heads);
        return hipGetLastError();
    }
    const dim3 grid((unsigned)(value_heads * (dv / kDeltaCols))), block(256);
    switch (dk) {
        case 32:
            hipLaunchKernelGGL((delta_kernel<32, kDeltaCols>), grid, block, 0, s, conv, (uint32_t)key_heads,
                               (uint32_t)dv, beta_s, log_decay, eps, state, rec_out, head_ss, z, z_silu, (uint32_t)tokens,
                               (uint32_t)value_heads);
            break;
        case 64:
            hipLaunchKernelGGL((delta_kernel<64, kDeltaCols>), grid, block, 0, s, conv, (uint32_t)key_heads,
                               (uint32_t)dv, beta_s, log_decay, eps, state, rec_out, head_ss, z, z_silu, (uint32_t)tokens,
                               (uint32_t)value_heads);
            break;
        case 128:
            hipLaunchKernelGGL((delta_kernel<128, kDeltaCols>), grid, block, 0, s, conv, (uint32_t)key_heads,
                               (uint32_t)dv, beta_s, log_decay, eps, state, rec_out, head_ss, z, z_silu, (uint32_t)tokens,
                               (uint32_t)value_heads);
            break;
        default:
            return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_gated_norm(const float* rec, const double* head_ss, const float* z, const float* out_norm,
                             uint64_t heads, uint64_t dv, float eps, float* gated, hipStream_t s, uint64_t tokens,
                             uint8_t* q8) {
    const uint64_t total = tokens * heads * dv;
    if (q8 != nullptr) {
        if ((heads * dv) % kQK != 0 || dv % 64 != 0) return hipErrorInvalidValue;
        const uint64_t nblocks = total / kQK;
        hipLaunchKernelGGL(gated_norm_q8k_kernel, dim3(blocks_of(nblocks, 4)), dim3(256), 0, s, rec, head_ss, z,
                           out_norm, nblocks, (uint32_t)dv, (uint32_t)delta_chunks(dv), eps, gated, q8);
        return hipGetLastError();
    }
    hipLaunchKernelGGL(gated_norm_kernel, dim3(blocks_of(total, 256)), dim3(256), 0, s, rec, head_ss, z, out_norm,
                       (uint32_t)total, (uint32_t)dv, (uint32_t)delta_chunks(dv), eps, gated);
    return hipGetLastError();
}

uint64_t delta_chunks(uint64_t dv) { return (dv + kDeltaCols - 1) / kDeltaCols; }

hipError_t launch_swiglu(const float* gate, const float* up, uint64_t n, float* act, hipStream_t s, uint8_t* q8) {
    if (q8 != nullptr) {
        if (n % kQK != 0) return hipErrorInvalidValue;
        const uint64_t nblocks = n / kQK;
        hipLaunchKernelGGL(swiglu_q8k_kernel, dim3(blocks_of(nblocks, 4)), dim3(256), 0, s, gate, up, nblocks, act, q8);
        return hipGetLastError();
    }
    hipLaunchKernelGGL(swiglu_kernel, dim3(blocks_of(n, 256)), dim3(256), 0, s, gate, up, (uint32_t)n, act);
    return hipGetLastError();
}

hipError_t launch_add(const float* a, const float* b, uint64_t n, float* out, hipStream_t s) {
    hipLaunchKernelGGL(add_kernel, dim3(blocks_of(n, 256)), dim3(256), 0, s, a, b, (uint32_t)n, out);
    return hipGetLastError();
}

}  // namespace oq
