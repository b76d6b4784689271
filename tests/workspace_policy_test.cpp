// Host-only check of the context workspace growth policy (oracle_amd/csrc/oq_workspace.h) with a
// counting allocator: no device needed.  Exits non-zero on the first failed expectation.
#include <cstdio>
#include <cstdlib>
#include <set>

#include "oq_workspace.h"

namespace {
std::set<void*> live;
int syncs = 0;
bool fail_alloc = false;

void* alloc(uint64_t n) {
    if (fail_alloc) return nullptr;
    void* p = std::malloc(n);
    live.insert(p);
    return p;
}
void release(void* p) {
    if (!live.erase(p)) {
        std::printf("free of an unknown pointer\n");
        std::exit(3);
    }
    std::free(p);
}
bool sync() {
    ++syncs;
    return true;
}
#define EXPECT(c)                                                   \
    do {                                                            \
        if (!(c)) {                                             \
            std::printf("line %d: expectation failed: %s\n", __LINE__, #c); \
            return 1;                                               \
        }                                                           \
    } while (0)
}  // namespace

int main() {
    oq::Workspace ws;
    EXPECT(ws.ensure(100, false, 0, alloc, release, sync) == oq::GrowResult::kOk);
    void* first = ws.ptr;
    EXPECT(first != nullptr && ws.bytes == 100 && live.size() == 1);
    // big enough already: nothing changes
    EXPECT(ws.ensure(50, true, 3, alloc, release, sync) == oq::GrowResult::kOk && ws.ptr == first);
    // growing while capturing is refused and leaves the buffer alone
    EXPECT(ws.ensure(200, true, 0, alloc, release, sync) == oq::GrowResult::kCapturing && ws.ptr == first);
    // growing with a live graph keeps the old allocation (the graph replays it)
    EXPECT(ws.ensure(200, false, 1, alloc, release, sync) == oq::GrowResult::kOk);
    EXPECT(ws.ptr != first && ws.bytes == 200 && live.count(first) == 1 && ws.retired.size() == 1);
    void* second = ws.ptr;
    // with no graph left, growth waits for the stream, then frees the old allocation at once
    const int s0 = syncs;
    EXPECT(ws.ensure(400, false, 0, alloc, release, sync) == oq::GrowResult::kOk);
    EXPECT(live.count(second) == 0 && syncs == s0 + 1 && ws.retired.size() == 1);
    // the last graph's destruction frees what was retired
    ws.release_retired(release);
    EXPECT(live.count(first) == 0 && ws.retired.empty() && live.size() == 1);
    // an allocation failure reports and leaves no buffer
    fail_alloc = true;
    EXPECT(ws.ensure(800, false, 0, alloc, release, sync) == oq::GrowResult::kAllocFailed);
    EXPECT(ws.ptr == nullptr && ws.bytes == 0 && live.empty());
    fail_alloc = false;
    EXPECT(ws.ensure(16, false, 0, alloc, release, sync) == oq::GrowResult::kOk);
    ws.release_all(release);
    EXPECT(live.empty() && ws.ptr == nullptr);
    // capture refusal: the library's own capture, or any capture state the stream query reports
    // (a caller's hipStreamBeginCapture on the context's stream), or a failed query
    using SC = oq::StreamCapture;
    EXPECT(!oq::capture_in_progress(false, SC::kNone));
    EXPECT(oq::capture_in_progress(true, SC::kNone));
    EXPECT(oq::capture_in_progress(false, SC::kActive));
    EXPECT(oq::capture_in_progress(false, SC::kInvalidated));
    EXPECT(oq::capture_in_progress(false, SC::kQueryFailed));
    EXPECT(oq::capture_in_progress(true, SC::kActive));
    std::printf("workspace policy ok\n");
    return 0;
}
