// launch_once.h -- one-time, per-device launch set-up that is safe when several
// host threads launch at once: the first caller on a device runs the set-up
// under std::call_once and every caller sees its result.
#pragma once
#include <hip/hip_runtime.h>
#include <mutex>

namespace vai_dev {

constexpr int kMaxDevices = 64;

struct PerDevice {
    std::once_flag flag[kMaxDevices];
    hipError_t err[kMaxDevices] = {};
    template <class F>
    hipError_t run(F&& f)
    {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
        std::call_once(flag[dev], [&] { err[dev] = f(dev); });
        return err[dev];
    }
};

// Raises a kernel's dynamic LDS limit once per device (needed above 64 KB).
inline hipError_t set_max_lds(PerDevice& once, const void* kern, int bytes)
{
    return once.run([&](int) { return hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, bytes); });
}

// The current device's CU count, read once per device.
inline hipError_t device_cus(int* cus)
{
    static PerDevice once;
    static int count[kMaxDevices] = {};
    int dev = 0;
    hipError_t e = once.run([&](int d) { return hipDeviceGetAttribute(&count[d], hipDeviceAttributeMultiprocessorCount, d); });
    if (e != hipSuccess) return e;
    if (hipGetDevice(&dev) != hipSuccess) return hipErrorInvalidDevice;
    *cus = count[dev];
    return hipSuccess;
}

}   // namespace vai_dev
