// Status strings, HIP error capture and the per-device workspace behind the C ABI.
#include "kdq_common.hpp"

#include <mutex>
#include <string>
#include <vector>

namespace kdq {
namespace {
thread_local std::string last_hip_error;

struct Workspace {
    void* ptr = nullptr;
    size_t bytes = 0;
};

std::mutex workspace_mutex;
std::vector<Workspace> workspaces;  // indexed by device
}  // namespace

int hip_failure(hipError_t error) {
    last_hip_error = hipGetErrorString(error);
    return KDQ_ERR_HIP;
}

void* workspace(size_t bytes, int* status) {
    int device = 0;
    if (hipGetDevice(&device) != hipSuccess) {
        *status = KDQ_ERR_HIP;
        return nullptr;
    }
    std::lock_guard<std::mutex> lock(workspace_mutex);
    if (workspaces.size() <= size_t(device))
        workspaces.resize(size_t(device) + 1);
    Workspace& w = workspaces[size_t(device)];
    if (w.bytes < bytes) {
        // Growing frees the old buffer: wait for work that may still use it.
        if (w.ptr) {
            if (hipDeviceSynchronize() != hipSuccess || hipFree(w.ptr) != hipSuccess) {
                *status = KDQ_ERR_HIP;
                return nullptr;
            }
            w.ptr = nullptr;
            w.bytes = 0;
        }
        size_t grown = bytes < (size_t(1) << 20) ? (size_t(1) << 20) : bytes;
        if (hipMalloc(&w.ptr, grown) != hipSuccess) {
            w.ptr = nullptr;
            *status = KDQ_ERR_SCRATCH;
            return nullptr;
        }
        w.bytes = grown;
    }
    *status = KDQ_OK;
    return w.ptr;
}

unsigned compute_units() {
    static std::mutex mutex;
    static std::vector<unsigned> cached;
    int device = 0;
    if (hipGetDevice(&device) != hipSuccess)
        return 256;
    std::lock_guard<std::mutex> lock(mutex);
    if (cached.size() <= size_t(device))
        cached.resize(size_t(device) + 1, 0);
    if (!cached[size_t(device)]) {
        int count = 0;
        cached[size_t(device)] =
            hipDeviceGetAttribute(&count, hipDeviceAttributeMultiprocessorCount, device) ==
                        hipSuccess && count > 0
                ? unsigned(count)
                : 256u;
    }
    return cached[size_t(device)];
}
}  // namespace kdq

extern "C" const char* kdq_status_string(int status) {
    switch (status) {
    case KDQ_OK:
        return "ok";
    case KDQ_ERR_ARGUMENT:
        return "kdq_argument";
    case KDQ_ERR_SHAPE:
        return "kdq_projection_shape";
    case KDQ_ERR_UNSUPPORTED:
        return "kdq_unsupported";
    case KDQ_ERR_ALIAS:
        return "kdq_alias";
    case KDQ_ERR_HIP:
        return "kdq_hip";
    case KDQ_ERR_SCRATCH:
        return "kdq_projection_scratch";
    case KDQ_ERR_ALIGNMENT:
        return "kdq_alignment";
    default:
        return "kdq_unknown_status";
    }
}

extern "C" const char* kdq_last_hip_error(void) {
    return kdq::last_hip_error.c_str();
}

extern "C" size_t kdq_block_values(int encoding) {
    return kdq::block_values(encoding);
}

extern "C" size_t kdq_block_bytes(int encoding) {
    return kdq::block_bytes(encoding);
}

extern "C" size_t kdq_row_bytes(int encoding, size_t in) {
    const size_t values = kdq::block_values(encoding);
    if (!values || in % values)
        return 0;
    return in / values * kdq::block_bytes(encoding);
}

extern "C" int kdq_release_scratch(void) {
    int device = 0;
    KDQ_HIP(hipGetDevice(&device));
    std::lock_guard<std::mutex> lock(kdq::workspace_mutex);
    if (kdq::workspaces.size() > size_t(device) && kdq::workspaces[size_t(device)].ptr) {
        KDQ_HIP(hipDeviceSynchronize());
        KDQ_HIP(hipFree(kdq::workspaces[size_t(device)].ptr));
        kdq::workspaces[size_t(device)] = {};
    }
    return KDQ_OK;
}
