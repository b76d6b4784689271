// The allocation-free entry point oq_deltanet_step_noalloc (declared in include/oq.h).
//
// For callers that cannot allocate device memory (code under HIP graph capture, tight serving
// loops, harnesses that forbid hipMalloc): the block step's workspace is a file-scope device
// array of kNoAllocScratchBytes instead of the context's growable buffer.  Each GPU the library
// runs on holds its own copy for the life of the process; its address on a device is taken once,
// with hipGetSymbolAddress, when the first context on that device is created, and only that
// address is ever handed to kernels (the array's name is not a device address in host code).
// Every call on one GPU shares that GPU's array: calls that overlap on one GPU (two streams, two
// threads) race.  The step writes every workspace value before it reads it, so the contents a
// previous call left need no clearing.
#include <hip/hip_runtime.h>

#include <mutex>

#include "../../include/oq.h"
#include "oq_internal.h"

namespace {

constexpr uint64_t kNoAllocScratchBytes = 4ull << 20;  // a hidden-4096 block step needs ~440 KiB
constexpr int kMaxDevices = 64;

static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

std::once_flag g_once[kMaxDevices];
void* g_scratch_dev[kMaxDevices] = {};  // per-device address of `scratch` (null until set up)

}  // namespace

namespace oq {

void noalloc_setup(int device) {
    if (device < 0 || device >= kMaxDevices) return;
    std::call_once(g_once[device], [device] {
        void* p = nullptr;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) == hipSuccess) g_scratch_dev[device] = p;
    });
}

}  // namespace oq

extern "C" {

uint64_t oq_deltanet_noalloc_capacity(void) { return kNoAllocScratchBytes; }

int oq_deltanet_step_noalloc(oq_context* ctx, const oq_deltanet_block* block, float* conv_history_dev,
                             float* state_dev, const float* x_dev, float* y_dev, float* trace_dev) {
    if (!ctx) return oq::set_error(nullptr, OQ_INVALID_ARGUMENT, "null context");
    const int dev = oq::context_device(ctx);
    void* ws = (dev >= 0 && dev < kMaxDevices) ? g_scratch_dev[dev] : nullptr;
    return oq::deltanet_step_into(ctx, block, conv_history_dev, state_dev, x_dev, y_dev, trace_dev,
                                  static_cast<float*>(ws), kNoAllocScratchBytes);
}

}  // extern "C"
