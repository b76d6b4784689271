// Prefill / verify GEMM for q4_K weights (m >= 16 activation rows) on gfx950 matrix cores.
//
// Y[m][n] = sum_k Xhat[m][k] * W[n][k] with Xhat the dequantized Q8_K activations (d*q) and W
// the reference's decoded weights ((d*sc)*q - dmin*m, src/model/storage_decode.cpp:63-94 applied
// to GGML q4_K).  Both operands are rounded to binary16 and multiplied on
// v_mfma_f32_32x32x16_f16 with F32 accumulation.  The rounding is relative 2^-11 per operand;
// over K >= 4096 terms its effect on an output stays below 1e-4 * sum_k |w_k * xhat_k| with a
// wide margin (checked by the parity tests), so the path is enabled only for K >= 4096.
//
// Structure: a 64 (m) x 128 (n) output tile per 256-thread workgroup, K in steps of 64 (one
// 64-element group of a q4_K super-block).  Each step stages the activation tile (already F16,
// produced once per call by act_to_f16_kernel) and the weight tile (dequantized from the row
// planes by the workgroup, once per tile) in LDS, double-buffered; four waves in a 2 x 2 grid
// each own a 32 x 64 sub-tile (two 32 x 32 MFMA accumulators).
#include "oq_common.h"
#include "oq_layout.h"

namespace oq {

namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float float16v __attribute__((ext_vector_type(16)));

constexpr int kBM = 64, kBN = 128, kBK = 64;
constexpr int kPad = 8;                 // f16 elements of padding per LDS row
constexpr int kLdsRow = kBK + kPad;     // 72 f16 = 144 bytes
constexpr int kThreads = 256;
constexpr uint64_t kMinK = 4096;

// Q8_K blocks [m][K/256] -> F16 activations [m][K] (d*q rounded to nearest even)
__global__ __launch_bounds__(256) void act_to_f16_kernel(const uint8_t* __restrict__ q8k, uint64_t total,
                                                          _Float16* __restrict__ out) {
    for (uint64_t i = blockIdx.x * 256ull + threadIdx.x; i * 4 < total; i += (uint64_t)gridDim.x * 256) {
        const uint64_t e = i * 4, blk = e / kQK, off = e % kQK;
        const uint8_t* b = q8k + blk * kQ8KBytes;
        const float d = *reinterpret_cast<const float*>(b);
        const uint32_t q = *reinterpret_cast<const uint32_t*>(b + 4 + off);
#pragma unroll
        for (int j = 0; j < 4; ++j) out[e + j] = (_Float16)(d * (float)(int8_t)(q >> (8 * j)));
    }
}

struct StageRegs {
    uint4 a0, a1;  // 16 activations (F16) of one row of the A tile
    uint4 qs;      // 16 quant bytes of one weight row (chunk e of the step's 64-group)
    uint4 hdr;     // that row's super-block header
};

OQ_DEVICE void stage_load(StageRegs& r, const _Float16* a16, const DeviceMatrix& w, int m, uint64_t m0,
                          uint64_t n0, uint64_t kt, int tid) {
    const uint64_t k = w.k, nsb = k / kQK;
    // A: 64 rows x 64 k, thread -> row tid/4, 16 k at 16*(tid%4)
    uint64_t row = m0 + (tid >> 2);
    row = row < (uint64_t)m ? row : (uint64_t)m - 1;
    const _Float16* ap = a16 + row * k + kt * kBK + 16 * (tid & 3);
    r.a0 = *reinterpret_cast<const uint4*>(ap);
    r.a1 = *reinterpret_cast<const uint4*>(ap + 8);
    // B: 128 weight rows, thread -> row tid/2, chunk e = tid%2 of group g of super-block sb
    uint64_t n = n0 + (tid >> 1);
    n = n < w.n ? n : w.n - 1;
    const uint64_t sb = kt / 4, g = kt % 4;
    const uint8_t* rowp = w.base + n * w.pitch;
    r.qs = *reinterpret_cast<const uint4*>(rowp + 16 * perm_chunk(nsb, sb, (uint32_t)g, (uint32_t)(tid & 1)));
    r.hdr = *reinterpret_cast<const uint4*>(rowp + 128 * nsb + 16 * sb);
}

OQ_DEVICE void stage_store(const StageRegs& r, _Float16* As, _Float16* Bs, uint64_t kt, int tid) {
    // A
    _Float16* ad = As + (tid >> 2) * kLdsRow + 16 * (tid & 3);
    *reinterpret_cast<uint4*>(ad) = r.a0;
    *reinterpret_cast<uint4*>(ad + 8) = r.a1;
    // B: decode 32 weights exactly in F32 (as the reference does), round once to F16
    const uint32_t g = (uint32_t)(kt % 4), e = (uint32_t)(tid & 1);
    const float d = f16_bits_to_f32(r.hdr.x & 0xFFFFu);
    const float dmin = f16_bits_to_f32(r.hdr.x >> 16);
    uint32_t sc0, mn0, sc1, mn1;
    scale_min_k4(2 * g, r.hdr.y, r.hdr.z, r.hdr.w, sc0, mn0);
    scale_min_k4(2 * g + 1, r.hdr.y, r.hdr.z, r.hdr.w, sc1, mn1);
    const float ds0 = d * (float)sc0, dm0 = dmin * (float)mn0;
    const float ds1 = d * (float)sc1, dm1 = dmin * (float)mn1;
    const uint32_t words[4] = {r.qs.x, r.qs.y, r.qs.z, r.qs.w};
    _Float16 lo[16], hi[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const uint32_t byte = (words[i >> 2] >> (8 * (i & 3))) & 0xFFu;
        lo[i] = (_Float16)(ds0 * (float)(byte & 15u) - dm0);
        hi[i] = (_Float16)(ds1 * (float)(byte >> 4) - dm1);
    }
    _Float16* bd = Bs + (tid >> 1) * kLdsRow;
#pragma unroll
    for (int i = 0; i < 16; i += 8) {
        half8 vlo, vhi;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            vlo[j] = lo[i + j];
            vhi[j] = hi[i + j];
        }
        *reinterpret_cast<half8*>(bd + 16 * e + i) = vlo;       // k = 16e + i (sub-block 2g)
        *reinterpret_cast<half8*>(bd + 32 + 16 * e + i) = vhi;  // k = 32 + 16e + i (sub-block 2g+1)
    }
}

__global__ __launch_bounds__(kThreads) void gemm_q4k_f16_kernel(DeviceMatrix w, int m, const _Float16* a16,
                                                               float* __restrict__ y) {
    __shared__ __align__(16) _Float16 As[2][kBM * kLdsRow];
    __shared__ __align__(16) _Float16 Bs[2][kBN * kLdsRow];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    const uint64_t n0 = (uint64_t)blockIdx.x * kBN, m0 = (uint64_t)blockIdx.y * kBM;
    const uint64_t ksteps = w.k / kBK;

    float16v acc0 = {}, acc1 = {};
    StageRegs st;
    stage_load(st, a16, w, m, m0, n0, 0, tid);
    stage_store(st, As[0], Bs[0], 0, tid);
    __syncthreads();
    for (uint64_t kt = 0; kt < ksteps; ++kt) {
        const int buf = (int)(kt & 1);
        const bool more = kt + 1 < ksteps;
        if (more) stage_load(st, a16, w, m, m0, n0, kt + 1, tid);
        const _Float16* as = As[buf] + (32 * wm + (lane & 31)) * kLdsRow + 8 * (lane >> 5);
        const _Float16* bs0 = Bs[buf] + (64 * wn + (lane & 31)) * kLdsRow + 8 * (lane >> 5);
        const _Float16* bs1 = bs0 + 32 * kLdsRow;
#pragma unroll
        for (int ks = 0; ks < kBK / 16; ++ks) {
            const half8 a = *reinterpret_cast<const half8*>(as + 16 * ks);
            const half8 b0 = *reinterpret_cast<const half8*>(bs0 + 16 * ks);
            const half8 b1 = *reinterpret_cast<const half8*>(bs1 + 16 * ks);
            acc0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b0, acc0, 0, 0, 0);
            acc1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b1, acc1, 0, 0, 0);
        }
        if (more) stage_store(st, As[buf ^ 1], Bs[buf ^ 1], kt + 1, tid);
        __syncthreads();
    }
    // result register r of lane l: row 8*(r/4) + 4*(l/32) + r%4, column l%32
    const uint64_t col0 = n0 + 64 * wn + (lane & 31);
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const uint64_t row = m0 + 32 * wm + 8 * (r / 4) + 4 * (lane >> 5) + (r % 4);
        if (row < (uint64_t)m) {
            if (col0 < w.n) y[row * w.n + col0] = acc0[r];
            if (col0 + 32 < w.n) y[row * w.n + col0 + 32] = acc1[r];
        }
    }
}

}  // namespace

bool gemm_mfma_supported(const DeviceMatrix& w, int m) {
    return w.type == 12 && m >= 16 && w.k >= kMinK && w.k % kBK == 0;
}

uint64_t gemm_scratch_bytes(const DeviceMatrix& w, int m) { return (uint64_t)m * w.k * 2; }

hipError_t launch_gemm_q4k_mfma(const DeviceMatrix& w, int m, const uint8_t* q8k, float* y, void* scratch,
                                hipStream_t s) {
    if (!gemm_mfma_supported(w, m)) return hipErrorNotSupported;
    _Float16* a16 = static_cast<_Float16*>(scratch);
    const uint64_t total = (uint64_t)m * w.k;
    uint64_t blocks = (total / 4 + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    hipLaunchKernelGGL(act_to_f16_kernel, dim3((unsigned)blocks), dim3(256), 0, s, q8k, total, a16);
    const dim3 grid((unsigned)((w.n + kBN - 1) / kBN), (unsigned)((m + kBM - 1) / kBM));
    hipLaunchKernelGGL(gemm_q4k_f16_kernel, grid, dim3(kThreads), 0, s, w, m, a16, y);
    return hipGetLastError();
}

}  // namespace oq
