// A growable device workspace shared between eager calls and captured HIP graphs (host code only).
//
// A graph captured on a context records the workspace address it saw.  When a later eager call
// needs a larger workspace, the old allocation must outlive every graph that may still replay
// it: with live graphs it is retired (kept) instead of freed, and the retired allocations are
// freed once the last graph of the context is destroyed.  Growing during a capture is refused:
// the capture would record an allocation the graph cannot own.
#pragma once

#include <cstdint>
#include <vector>

namespace oq {

enum class GrowResult { kOk, kCapturing, kAllocFailed, kSyncFailed };

// What a query of the context's stream (hipStreamIsCapturing) reported.
enum class StreamCapture { kNone, kActive, kInvalidated, kQueryFailed };

// Whether a call must treat the context's stream as being captured: the library's own capture
// (oq_capture_begin) or a caller's hipStreamBeginCapture on the same stream.  An invalidated
// capture is still a capture, and a failed query is treated as one, so that nothing which would
// record memsets, allocations or host-side state changes into a graph slips through.
inline bool capture_in_progress(bool library_capture, StreamCapture stream) {
    return library_capture || stream != StreamCapture::kNone;
}

struct Workspace {
    void* ptr = nullptr;
    uint64_t bytes = 0;
    std::vector<void*> retired;

    // Makes ptr hold at least `need` bytes.  alloc(bytes) -> pointer or nullptr; free(pointer);
    // sync() -> bool waits for work that may still use the old allocation.
    template <typename Alloc, typename Free, typename Sync>
    GrowResult ensure(uint64_t need, bool capturing, int live_graphs, Alloc alloc, Free free, Sync sync) {
        if (bytes >= need) return GrowResult::kOk;
        if (capturing) return GrowResult::kCapturing;
        if (ptr != nullptr) {
            if (live_graphs > 0) {
                retired.push_back(ptr);
            } else {
                if (!sync()) return GrowResult::kSyncFailed;
                free(ptr);
            }
            ptr = nullptr;
            bytes = 0;
        }
        ptr = alloc(need);
        if (ptr == nullptr) return GrowResult::kAllocFailed;
        bytes = need;
        return GrowResult::kOk;
    }

    // Frees the retired allocations (call when no graph can replay them any more).
    template <typename Free>
    void release_retired(Free free) {
        for (void* p : retired) free(p);
        retired.clear();
    }

    template <typename Free>
    void release_all(Free free) {
        release_retired(free);
        if (ptr != nullptr) free(ptr);
        ptr = nullptr;
        bytes = 0;
    }
};

}  // namespace oq
