// Shared helpers for the gfx950 kernels and the C ABI of libkitty_hip.so.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string>

#include "kitty_hip.h"

namespace kitty {

// Thread-local message behind kitty_last_error().
void set_error(const std::string &msg);
const char *get_error();

inline int fail(int code, const std::string &msg)
{
    set_error(msg);
    return code;
}

// Launch-error check shared by the entry points.
inline int check_launch(const char *what)
{
    hipError_t e = hipGetLastError();
    if (e != hipSuccess)
        return fail(KITTY_E_HIP, std::string(what) + ": " + hipGetErrorString(e));
    return KITTY_OK;
}

__device__ __forceinline__ float h2f(uint16_t b)
{
    return (float)__builtin_bit_cast(_Float16, b);
}

// fp32 -> fp16 with round-to-nearest-even (v_cvt_f16_f32 in the default mode),
// the same rounding as torch's .to(torch.float16).
__device__ __forceinline__ uint16_t f2h(float f)
{
    return __builtin_bit_cast(uint16_t, (_Float16)f);
}

constexpr float kLog2e = 1.4426950408889634f;

} // namespace kitty
