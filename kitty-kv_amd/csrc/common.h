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

// bf16 -> fp32 (exact) and a 16-bit value of either type -> fp32.
__device__ __forceinline__ float bf2f(uint16_t b)
{
    return __builtin_bit_cast(float, (uint32_t)b << 16);
}

__device__ __forceinline__ float x2f(uint16_t b, bool bf16)
{
    return bf16 ? bf2f(b) : h2f(b);
}

// fp32 -> bf16 with round-to-nearest-even, NaN -> 0x7FC0: torch's
// .to(torch.bfloat16).
__device__ __forceinline__ uint16_t f2bf(float f)
{
    uint32_t u = __builtin_bit_cast(uint32_t, f);
    if ((u & 0x7fffffffu) > 0x7f800000u)
        return 0x7fc0;
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

// fp32 -> a 16-bit value of either type, rounded to nearest even.
__device__ __forceinline__ uint16_t f2x(float f, bool bf16)
{
    return bf16 ? f2bf(f) : f2h(f);
}

// A scale or zero point as a metadata pool stores it: the reference computes
// it as fp16 (quantize_key.py:121-122, quantize_value.py:90) and copies that
// into the pool's dtype, so a bf16 pool holds bf16(fp16(x)).
__device__ __forceinline__ uint16_t meta_store(float f, bool bf16)
{
    const uint16_t h = f2h(f);
    return bf16 ? f2bf(h2f(h)) : h;
}

constexpr float kLog2e = 1.4426950408889634f;

} // namespace kitty
