// Stand-in for the part of genie-ai-runtime's src/engine/model.cpp that stays
// compiled in the engine when the kernel translation units are replaced by
// libjllm_hip.so: the mapped-weight registry (model.cpp:39-66).  One region
// per host base; a pointer inside [host, host + bytes) maps to the device
// alias at the same offset.  Test infrastructure: it lets the link test show
// that these three symbols are defined once (here, not by the library) and
// that the library's weak reference finds them at run time.
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <cstdint>
#include <mutex>
#include <vector>
#include "jllm_kernels.h"

namespace {
struct Region { const char* host; const char* dev; int64_t bytes; };
std::mutex mu;
std::vector<Region> regions;
}  // namespace

namespace jllm {

void register_mapped_weight_region(const void* host_base, const void* device_base, int64_t bytes) {
    std::lock_guard<std::mutex> lk(mu);
    regions.push_back({(const char*)host_base, (const char*)device_base, bytes});
}

void clear_mapped_weight_region(const void* host_base) {
    std::lock_guard<std::mutex> lk(mu);
    for (size_t i = 0; i < regions.size(); i++)
        if (regions[i].host == (const char*)host_base) { regions.erase(regions.begin() + i); return; }
}

const void* resolve_mapped_weight_device_ptr(const void* host_ptr) {
    const char* p = (const char*)host_ptr;
    std::lock_guard<std::mutex> lk(mu);
    for (const auto& r : regions)
        if (p >= r.host && p < r.host + r.bytes) return r.dev + (p - r.host);
    return nullptr;
}

}  // namespace jllm
