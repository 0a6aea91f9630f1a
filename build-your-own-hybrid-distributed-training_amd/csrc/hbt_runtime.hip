// Error state, device queries and ABI metadata for libhbt.so.
#include <cstdarg>
#include <mutex>

#include "hbt_common.hpp"

namespace hbt {

namespace {
thread_local std::string g_last_error;

constexpr int kMaxDevices = 64;
int g_cu_count[kMaxDevices] = {0};
std::mutex g_device_mutex;
}  // namespace

void set_error(const char* fmt, ...) {
    char buffer[1024];
    va_list args;
    va_start(args, fmt);
    vsnprintf(buffer, sizeof(buffer), fmt, args);
    va_end(args);
    g_last_error = buffer;
}

void clear_error() { g_last_error.clear(); }

int32_t check_hip(hipError_t status, const char* what) {
    if (status == hipSuccess) return HBT_OK;
    set_error("%s: HIP error %d (%s)", what, static_cast<int>(status), hipGetErrorString(status));
    return HBT_ERR_HIP;
}

int32_t check_launch(const char* what) { return check_hip(hipGetLastError(), what); }

int device_cu_count() {
    int device = 0;
    if (hipGetDevice(&device) != hipSuccess || device < 0 || device >= kMaxDevices) return 256;
    std::lock_guard<std::mutex> lock(g_device_mutex);
    if (g_cu_count[device] == 0) {
        int cus = 0;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) !=
                hipSuccess ||
            cus <= 0) {
            cus = 256;
        }
        g_cu_count[device] = cus;
    }
    return g_cu_count[device];
}

}  // namespace hbt

extern "C" {

const char* hbt_last_error(void) { return hbt::g_last_error.c_str(); }

// Bumped whenever an exported signature or a table layout changes.
int32_t hbt_abi_version(void) { return 18; }

// Entry points declared in include/hbt.h (hbt_last_error .. hbt_scale_inplace_f64).
int32_t hbt_symbol_count(void) { return 34; }

int64_t hbt_grid_slices(int64_t blocks, int32_t threads, int64_t* first, int64_t* count, int64_t capacity) {
    if (threads <= 0) return -1;
    const int64_t slices = hbt::grid_slice_count(blocks, threads);
    const int64_t per = hbt::grid_max_blocks(threads);
    for (int64_t k = 0; k < slices && k < capacity; ++k) {
        const int64_t start = k * per;
        if (first != nullptr) first[k] = start;
        if (count != nullptr) count[k] = blocks - start < per ? blocks - start : per;
    }
    return slices;
}

}  // extern "C"
