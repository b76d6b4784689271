// HBM read floor on this GPU: how long a kernel that only reads N bytes (and XORs them) takes,
// for sizes from 7 MB to 510 MB and several launch shapes, with ordinary and with non-temporal
// loads ("_nt": the form the library's weight and KV loads take), as steady-state back-to-back launches
// (200 launches captured in a HIP graph over distinct copies that together exceed the 256 MB
// Infinity Cache; best of three replays after a first one).  It bounds every bandwidth-bound kernel of this library: a
// decode GEMV over a weight of N bytes cannot take less than the read of N bytes.  Then the launch
// floor: the time per launch of a dependent chain of eager launches that do no memory work to speak
// of, by launch shape (waves in the grid), the fixed cost of each launch of a chained block step.
//
//   build: oracle_amd/build.py (calibration/read_floor)   run: oracle_amd/calibration/read_floor
#include <hip/hip_runtime.h>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>
#define CK(x) do { hipError_t e = (x); if (e != hipSuccess) { printf("err %s line %d\n", hipGetErrorString(e), __LINE__); exit(1);} } while (0)

typedef unsigned u32x4v __attribute__((ext_vector_type(4)));
template <bool NT>
__device__ __forceinline__ uint4 ld(const uint4* p) {
    if constexpr (NT) {
        const u32x4v v = __builtin_nontemporal_load(reinterpret_cast<const u32x4v*>(p));
        return make_uint4(v.x, v.y, v.z, v.w);
    } else {
        return *p;
    }
}

// grid-stride: each thread loads UNR uint4 per trip
template <int UNR, bool NT>
__global__ __launch_bounds__(1024) void read_gs(const uint4* __restrict__ p, uint64_t n16, unsigned* out) {
    uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    unsigned acc = 0;
    for (; i + (UNR - 1) * stride < n16; i += UNR * stride) {
        uint4 v[UNR];
#pragma unroll
        for (int u = 0; u < UNR; ++u) v[u] = ld<NT>(p + i + u * stride);
#pragma unroll
        for (int u = 0; u < UNR; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    }
    for (; i < n16; i += stride) { uint4 v = ld<NT>(p + i); acc ^= v.x ^ v.y ^ v.z ^ v.w; }
    if (acc == 0x12345678u) out[0] = acc;
}
// one-shot: each wave reads a contiguous chunk of CH uint4 per lane
template <int CH, bool NT>
__global__ __launch_bounds__(256) void read_chunk(const uint4* __restrict__ p, uint64_t n16, unsigned* out) {
    const uint64_t wave = ((uint64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    const int lane = threadIdx.x & 63;
    const uint64_t base = wave * 64 * CH;
    unsigned acc = 0;
    uint4 v[CH];
#pragma unroll
    for (int c = 0; c < CH; ++c) { uint64_t i = base + c * 64 + lane; v[c] = i < n16 ? ld<NT>(p + i) : make_uint4(0,0,0,0); }
#pragma unroll
    for (int c = 0; c < CH; ++c) acc ^= v[c].x ^ v[c].y ^ v[c].z ^ v[c].w;
    if (acc == 0x12345678u) out[0] = acc;
}

// one element per thread from the previous launch's output: a dependent chain of launches that do
// (almost) no memory work
__global__ __launch_bounds__(1024) void chain_step(const unsigned* __restrict__ in, unsigned* __restrict__ out, unsigned n) {
    const unsigned i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = in[(i * 7u) % n] + 1u;
}

int main() {
    int cus = 0; CK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, 0));
    hipStream_t s; CK(hipStreamCreate(&s));
    unsigned* out; CK(hipMalloc(&out, 4));
    const uint64_t total = 1200ull << 20;
    uint8_t* big; CK(hipMalloc(&big, total));
    CK(hipMemset(big, 1, total));
    hipEvent_t e0, e1; CK(hipEventCreate(&e0)); CK(hipEventCreate(&e1));
    const uint64_t sizes[] = {7077888, 14155776, 28311552, 56623104, 113246208, 226492416, 510504960};
    struct Best { double us = 1e30; char name[64] = ""; };
    std::vector<Best> best_any(7), best_plain(7);
    int si = -1;
    for (uint64_t S : sizes) {
        ++si;
        const uint64_t n16 = S / 16;
        const int ncopies = (int)((total / S) < 40 ? total / S : 40);
        auto run = [&](const char* name, auto launch) {
            const int steps = 200;
            for (int w = 0; w < 20; ++w) launch((const uint4*)(big + (w % ncopies) * S));
            hipGraph_t g; hipGraphExec_t ge;
            CK(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
            for (int i = 0; i < steps; ++i) launch((const uint4*)(big + (i % ncopies) * S));
            CK(hipStreamEndCapture(s, &g));
            CK(hipGraphInstantiate(&ge, g, nullptr, nullptr, 0));
            CK(hipGraphLaunch(ge, s)); CK(hipStreamSynchronize(s));
            float best = 1e9;
            for (int r = 0; r < 3; ++r) {
                CK(hipEventRecord(e0, s)); CK(hipGraphLaunch(ge, s)); CK(hipEventRecord(e1, s)); CK(hipEventSynchronize(e1));
                float ms; CK(hipEventElapsedTime(&ms, e0, e1)); if (ms < best) best = ms;
            }
            const double us = best * 1e3 / steps;
            printf("{\"size\": %llu, \"kernel\": \"%s\", \"us\": %.3f, \"tbs\": %.3f}\n", (unsigned long long)S, name, us, S / us / 1e6);
            if (us < best_any[si].us) { best_any[si].us = us; snprintf(best_any[si].name, 64, "%s", name); }
            if (!strstr(name, "_nt") && us < best_plain[si].us) { best_plain[si].us = us; snprintf(best_plain[si].name, 64, "%s", name); }
            fflush(stdout);
            CK(hipGraphExecDestroy(ge)); CK(hipGraphDestroy(g));
        };
        for (int nt = 0; nt < 2; ++nt) {
            const char* sfx = nt ? "_nt" : "";
            char nm[64];
            for (int wpc : {1, 2}) {
                snprintf(nm, 64, "gs4_1024x%d%s", wpc, sfx);
                if (nt) run(nm, [&](const uint4* p) { hipLaunchKernelGGL((read_gs<4, true>), dim3(cus * wpc), dim3(1024), 0, s, p, n16, out); });
                else run(nm, [&](const uint4* p) { hipLaunchKernelGGL((read_gs<4, false>), dim3(cus * wpc), dim3(1024), 0, s, p, n16, out); });
            }
            snprintf(nm, 64, "gs8_1024x1%s", sfx);
            if (nt) run(nm, [&](const uint4* p) { hipLaunchKernelGGL((read_gs<8, true>), dim3(cus), dim3(1024), 0, s, p, n16, out); });
            else run(nm, [&](const uint4* p) { hipLaunchKernelGGL((read_gs<8, false>), dim3(cus), dim3(1024), 0, s, p, n16, out); });
            snprintf(nm, 64, "gs2_1024x2%s", sfx);
            if (nt) run(nm, [&](const uint4* p) { hipLaunchKernelGGL((read_gs<2, true>), dim3(cus * 2), dim3(1024), 0, s, p, n16, out); });
            else run(nm, [&](const uint4* p) { hipLaunchKernelGGL((read_gs<2, false>), dim3(cus * 2), dim3(1024), 0, s, p, n16, out); });
            for (int ch : {4, 8, 16}) {
                snprintf(nm, 64, "chunk%d%s", ch, sfx);
                const uint64_t waves = (n16 + 64 * ch - 1) / (64 * ch);
                const unsigned wgs = (unsigned)((waves + 3) / 4);
                if (ch == 4 && nt) run(nm, [&](const uint4* p) { hipLaunchKernelGGL((read_chunk<4, true>), dim3(wgs), dim3(256), 0, s, p, n16, out); });
                if (ch == 4 && !nt) run(nm, [&](const uint4* p) { hipLaunchKernelGGL((read_chunk<4, false>), dim3(wgs), dim3(256), 0, s, p, n16, out); });
                if (ch == 8 && nt) run(nm, [&](const uint4* p) { hipLaunchKernelGGL((read_chunk<8, true>), dim3(wgs), dim3(256), 0, s, p, n16, out); });
                if (ch == 8 && !nt) run(nm, [&](const uint4* p) { hipLaunchKernelGGL((read_chunk<8, false>), dim3(wgs), dim3(256), 0, s, p, n16, out); });
                if (ch == 16 && nt) run(nm, [&](const uint4* p) { hipLaunchKernelGGL((read_chunk<16, true>), dim3(wgs), dim3(256), 0, s, p, n16, out); });
                if (ch == 16 && !nt) run(nm, [&](const uint4* p) { hipLaunchKernelGGL((read_chunk<16, false>), dim3(wgs), dim3(256), 0, s, p, n16, out); });
            }
        }
    }
    // an empty kernel: the per-launch floor of a graph
    {
        const int steps = 200;
        hipGraph_t g; hipGraphExec_t ge;
        CK(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
        for (int i = 0; i < steps; ++i) hipLaunchKernelGGL((read_chunk<1, false>), dim3(cus), dim3(256), 0, s, (const uint4*)big, 0, out);
        CK(hipStreamEndCapture(s, &g)); CK(hipGraphInstantiate(&ge, g, nullptr, nullptr, 0));
        CK(hipGraphLaunch(ge, s)); CK(hipStreamSynchronize(s));
        CK(hipEventRecord(e0, s)); CK(hipGraphLaunch(ge, s)); CK(hipEventRecord(e1, s)); CK(hipEventSynchronize(e1));
        float ms; CK(hipEventElapsedTime(&ms, e0, e1));
        printf("{\"kernel\": \"empty_256wg\", \"us\": %.3f}\n", ms * 1e3 / steps);
    }
    // Launch floor: 200 dependent launches issued eagerly on one stream (the library's calls), each
    // workgroup shape with no memory work to speak of; per launch, best of three
    {
        const unsigned shapes[][2] = {{1, 64}, {256, 256}, {256, 1024}, {512, 512}, {1024, 256}, {4096, 64},
                                      {512, 1024}, {2048, 256}};
        unsigned *a, *b;
        const unsigned nmax = 512u * 1024u;
        CK(hipMalloc(&a, nmax * 4)); CK(hipMalloc(&b, nmax * 4));
        CK(hipMemset(a, 0, nmax * 4)); CK(hipMemset(b, 0, nmax * 4));
        for (auto& sh : shapes) {
            const unsigned wgs = sh[0], th = sh[1], n = wgs * th;
            float best = 1e9;
            for (int r = 0; r < 3; ++r) {
                CK(hipStreamSynchronize(s));
                CK(hipEventRecord(e0, s));
                for (int i = 0; i < 200; ++i)
                    hipLaunchKernelGGL(chain_step, dim3(wgs), dim3(th), 0, s, (i & 1) ? b : a, (i & 1) ? a : b, n);
                CK(hipEventRecord(e1, s)); CK(hipEventSynchronize(e1));
                float ms; CK(hipEventElapsedTime(&ms, e0, e1)); if (ms < best) best = ms;
            }
            CK(hipGetLastError());
            printf("{\"kernel\": \"chain_%ux%u\", \"waves\": %u, \"us\": %.3f}\n", wgs, th, wgs * ((th + 63) / 64),
                   best * 1e3 / 200);
            fflush(stdout);
        }
        CK(hipFree(a)); CK(hipFree(b));
    }
    printf("# best per size, any load form | ordinary loads only (%% of 8 TB/s)\n");
    for (int i = 0; i < 7; ++i) {
        const double a = sizes[i] / best_any[i].us / 1e6, b = sizes[i] / best_plain[i].us / 1e6;
        printf("#  %10llu B  %-14s %7.3f us %6.3f TB/s (%4.1f %%) | %-12s %7.3f us %6.3f TB/s (%4.1f %%)\n",
               (unsigned long long)sizes[i], best_any[i].name, best_any[i].us, a, a / 8.0 * 100.0, best_plain[i].name,
               best_plain[i].us, b, b / 8.0 * 100.0);
    }
    return 0;
}
