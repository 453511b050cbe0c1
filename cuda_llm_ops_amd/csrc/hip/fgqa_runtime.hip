// Host runtime pieces of libfgqa: status strings, the cached device
// properties and the library-owned decode workspace.
#include <mutex>
#include <vector>

#include "fgqa_internal.h"

namespace fgqa {

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_mutex;      // device properties and kernel attributes
std::mutex g_ws_mutex;   // the library-owned workspaces
int g_cu_count[kMaxDevices] = {0};
constexpr int kMaxKernelSlots = 32;
bool g_smem_set[kMaxDevices][kMaxKernelSlots] = {};
void* g_ws_ptr[kMaxDevices] = {nullptr};
size_t g_ws_bytes[kMaxDevices] = {0};
}  // namespace

int device_cu_count() {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 0;
    std::lock_guard<std::mutex> lock(g_mutex);
    if (g_cu_count[dev] == 0) {
        int cus = 0;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
        g_cu_count[dev] = cus;
    }
    return g_cu_count[dev];
}

int set_kernel_smem_once(int slot, const void* fn, int bytes) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return FGQA_ERR_HIP;
    if (dev < 0 || dev >= kMaxDevices || slot < 0 || slot >= kMaxKernelSlots) return FGQA_ERR_UNSUPPORTED;
    std::lock_guard<std::mutex> lock(g_mutex);
    if (!g_smem_set[dev][slot]) {
        if (hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, bytes) != hipSuccess)
            return FGQA_ERR_HIP;
        g_smem_set[dev][slot] = true;
    }
    return FGQA_OK;
}

std::unique_lock<std::mutex> workspace_lock() { return std::unique_lock<std::mutex>(g_ws_mutex); }

void* internal_workspace(size_t bytes, int* status) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
        *status = FGQA_ERR_HIP;
        return nullptr;
    }
    if (g_ws_bytes[dev] < bytes) {
        // Work already queued on any stream may still read the old buffer, so
        // drain the device before releasing it.
        if (g_ws_ptr[dev] != nullptr) {
            if (hipDeviceSynchronize() != hipSuccess || hipFree(g_ws_ptr[dev]) != hipSuccess) {
                *status = FGQA_ERR_HIP;
                return nullptr;
            }
            g_ws_ptr[dev] = nullptr;
            g_ws_bytes[dev] = 0;
        }
        const size_t rounded = (bytes + (1u << 20) - 1) & ~static_cast<size_t>((1u << 20) - 1);
        void* p = nullptr;
        if (hipMalloc(&p, rounded) != hipSuccess) {
            *status = FGQA_ERR_HIP;
            return nullptr;
        }
        g_ws_ptr[dev] = p;
        g_ws_bytes[dev] = rounded;
    }
    *status = FGQA_OK;
    return g_ws_ptr[dev];
}

// Workgroup w's first thread reads its CU's shader-clock counter
// (s_memtime), the 100 MHz real-time counter (s_memrealtime) and where it
// runs (XCD number, and the SE / SH / CU fields of HW_ID), and stores them
// at out[3w .. 3w+2].
__global__ __launch_bounds__(64) void clock_sample_kernel(unsigned long long* out) {
    if (threadIdx.x != 0) return;
    const unsigned long long t = __builtin_amdgcn_s_memtime();
    const unsigned long long r = __builtin_amdgcn_s_memrealtime();
    unsigned xcc, hw;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_HW_ID)" : "=s"(hw));
    unsigned long long* o = out + 3 * (size_t)blockIdx.x;
    o[0] = t;
    o[1] = r;
    o[2] = ((unsigned long long)(xcc & 15u) << 8) | ((hw >> 8) & 0xffu);
}

}  // namespace fgqa

extern "C" int fgqa_clock_sample(unsigned long long* out, int samples, void* stream) {
    if (out == nullptr || (reinterpret_cast<uintptr_t>(out) & 7u) != 0 || samples < 1 || samples > 65536)
        return FGQA_ERR_INVALID_ARGUMENT;
    hipLaunchKernelGGL(fgqa::clock_sample_kernel, dim3((unsigned)samples), dim3(64), 0,
                       static_cast<hipStream_t>(stream), out);
    return hipGetLastError() == hipSuccess ? FGQA_OK : FGQA_ERR_HIP;
}

extern "C" const char* fgqa_status_string(int status) {
    switch (status) {
        case FGQA_OK: return "ok";
        case FGQA_ERR_INVALID_ARGUMENT: return "invalid argument";
        case FGQA_ERR_UNSUPPORTED: return "unsupported shape, layout or alignment";
        case FGQA_ERR_WORKSPACE: return "workspace too small";
        case FGQA_ERR_HIP: return "HIP runtime error";
        default: return "unknown status";
    }
}

extern "C" int fgqa_version(void) { return 201; }
