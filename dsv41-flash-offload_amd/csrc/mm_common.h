// Shared device helpers for the MI355X (gfx950) routed-expert MoE kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/mi355moe.h"

namespace mm {

// EXL3 "mul1" codebook constants (kernels/cpu_avx2/ft_core.h:28-40): state * MUL1 (mod 2^32), byte sum s,
// weight = fp16(fma(1024 + s, KINV, KBIAS)) with KINV = fp16 0x1eee, KBIAS = fp16 0xc931.
constexpr uint32_t MUL1 = 0x83DCD12Du;
constexpr uint16_t KINV_BITS = 0x1eee;
constexpr uint16_t KBIAS_BITS = 0xc931;
// 1/sqrt(128) as the reference spells it (ft_core.h:29); the same literal gives the same fp32 value.
constexpr float HAD = 0.088388347648f;

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float h2f(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }
__device__ __forceinline__ uint16_t f2h(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }   // RNE
__device__ __forceinline__ float r16(float f) { return (float)(_Float16)f; }

// fp32 -> bf16 bits, round to nearest even; NaN stays a (quiet) NaN.
__device__ __forceinline__ uint16_t f2bf(float f)
{
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}
__device__ __forceinline__ float bf16_value(float f) { return __uint_as_float((uint32_t)f2bf(f) << 16); }

// 128-point fast Walsh-Hadamard transform held by one wave64: lane L owns elements L (a) and L + 64 (b).
// Stages run with strides 1, 2, ..., 64 and write (lo + hi, lo - hi), exactly the reference butterfly
// (ft_core.h:89-94), so the fp32 results are bit-identical.
__device__ __forceinline__ void fwht128_wave(float& a, float& b)
{
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int w = 1; w < 64; w <<= 1)
    {
        const float oa = __shfl_xor(a, w, 64);
        const float ob = __shfl_xor(b, w, 64);
        const bool up = (lane & w) != 0;
        a = up ? (oa - a) : (a + oa);
        b = up ? (ob - b) : (b + ob);
    }
    const float lo = a, hi = b;
    a = lo + hi;
    b = lo - hi;
}

// Input transform of one 128-block (ft_core.h:96-102): xt = r16(FWHT(x * suh) * HAD).
__device__ __forceinline__ void prep_block_wave(float& a, float& b, float suh_a, float suh_b)
{
    a = a * suh_a;
    b = b * suh_b;
    fwht128_wave(a, b);
    a = r16(a * HAD);
    b = r16(b * HAD);
}

// Output transform of one 128-block (ft_core.h:104-110): y = r16(FWHT(r16(y)) * HAD * svh).
__device__ __forceinline__ void out_block_wave(float& a, float& b, float svh_a, float svh_b)
{
    a = r16(a);
    b = r16(b);
    fwht128_wave(a, b);
    a = r16((a * HAD) * svh_a);
    b = r16((b * HAD) * svh_b);
}

// SwiGLU with the exllamav3 clamp (ft_core.h:123-133).
__device__ __forceinline__ float act_gu(float g, float u, float limit)
{
    float x = g / (1.0f + expf(-g));
    if (limit != 0.0f)
    {
        u = fminf(fmaxf(u, -limit), limit);
        x = fminf(x, limit);
    }
    return x * u;
}

// Host-side error reporting shared by every translation unit of the library.
int set_error(int code, const char* fmt, ...);
int check_launch(const char* what);

}  // namespace mm

#define MM_CHECK_ARG(cond, ...) \
    do { if (!(cond)) return ::mm::set_error(MM_ERR_ARG, __VA_ARGS__); } while (0)
