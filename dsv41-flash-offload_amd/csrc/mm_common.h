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
// fp32 -> fp16 rounds the fp32 value it is given (RNE). The empty asm hides where the value came from: otherwise
// the compiler folds a multiply and the rounding after it into one v_fma_mix*_f16, which rounds the exact product
// to fp16 once, where the reference rounds the fp32 product first (1 ulp apart on rare inputs).
__device__ __forceinline__ float fp32_operand(float f)
{
    asm("" : "+v"(f));
    return f;
}
__device__ __forceinline__ uint16_t f2h(float f) { return __builtin_bit_cast(uint16_t, (_Float16)fp32_operand(f)); }
__device__ __forceinline__ float r16(float f) { return (float)(_Float16)fp32_operand(f); }

// fp32 -> bf16 bits, round to nearest even; NaN stays a (quiet) NaN.
__device__ __forceinline__ uint16_t f2bf(float f)
{
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}
__device__ __forceinline__ float bf16_value(float f) { return __uint_as_float((uint32_t)f2bf(f) << 16); }

// Value of lane (lane ^ D) of the wave, D in {1, 2, 4, 8, 16, 32}, through DPP moves (xor 4 = the 8-lane mirror
// then the reversed quad) and the gfx950 lane-swap instructions, so no exchange goes through the LDS crossbar.
// Every lane of the wave must be active.
template <int D>
__device__ __forceinline__ int xor_lane_i(int v)
{
    static_assert(D == 1 || D == 2 || D == 4 || D == 8 || D == 16 || D == 32, "xor distance");
    if constexpr (D == 1) return __builtin_amdgcn_mov_dpp(v, 0xB1, 0xF, 0xF, false);          // quad_perm 1,0,3,2
    if constexpr (D == 2) return __builtin_amdgcn_mov_dpp(v, 0x4E, 0xF, 0xF, false);          // quad_perm 2,3,0,1
    if constexpr (D == 4)                                                                       // half mirror, 3,2,1,0
        return __builtin_amdgcn_mov_dpp(__builtin_amdgcn_mov_dpp(v, 0x141, 0xF, 0xF, false), 0x1B, 0xF, 0xF, false);
    if constexpr (D == 8) return __builtin_amdgcn_mov_dpp(v, 0x128, 0xF, 0xF, false);         // row_ror 8
    const int lane = threadIdx.x & 63;
    if constexpr (D == 16)
    {
        // swapping the odd 16-lane rows of one copy with the even rows of another leaves the partner row in the
        // first copy for odd rows and in the second for even rows
        const auto r = __builtin_amdgcn_permlane16_swap((unsigned)v, (unsigned)v, false, false);
        return (lane & 16) ? (int)r[0] : (int)r[1];
    }
    const auto r = __builtin_amdgcn_permlane32_swap((unsigned)v, (unsigned)v, false, false);
    return (lane & 32) ? (int)r[0] : (int)r[1];
}
template <int D>
__device__ __forceinline__ float xor_lane(float v)
{
    return __int_as_float(xor_lane_i<D>(__float_as_int(v)));
}

// Inclusive prefix sum over the 64 lanes: shifts within each 16-lane row (DPP row_shr with zero fill), then the
// totals of the rows below, read as scalars. Every lane of the wave must be active.
__device__ __forceinline__ int wave_incl_scan(int v)
{
    v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xF, 0xF, true);    // row_shr 1
    v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xF, 0xF, true);    // row_shr 2
    v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xF, 0xF, true);    // row_shr 4
    v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xF, 0xF, true);    // row_shr 8
    const int lane = threadIdx.x & 63;
    const int r0 = __builtin_amdgcn_readlane(v, 15), r1 = __builtin_amdgcn_readlane(v, 31);
    const int r2 = __builtin_amdgcn_readlane(v, 47);
    return v + (lane >= 16 ? r0 : 0) + (lane >= 32 ? r1 : 0) + (lane >= 48 ? r2 : 0);
}

// 128-point fast Walsh-Hadamard transform held by one wave64: lane L owns elements L (a) and L + 64 (b).
// Stages run with strides 1, 2, ..., 64 and write (lo + hi, lo - hi), exactly the reference butterfly
// (ft_core.h:89-94), so the fp32 results are bit-identical.
template <int W>
__device__ __forceinline__ void fwht_stage(float& a, float& b)
{
    const bool up = (threadIdx.x & W) != 0;
    const float oa = xor_lane<W>(a), ob = xor_lane<W>(b);
    a = up ? (oa - a) : (a + oa);
    b = up ? (ob - b) : (b + ob);
}
__device__ __forceinline__ void fwht128_wave(float& a, float& b)
{
    fwht_stage<1>(a, b);
    fwht_stage<2>(a, b);
    fwht_stage<4>(a, b);
    fwht_stage<8>(a, b);
    fwht_stage<16>(a, b);
    fwht_stage<32>(a, b);
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

// The permutation behind mm_permute; e_sorted (optional, [n]) receives the expert bin of each sorted position.
int permute_launch(const int64_t* ids, const float* w, int n, int topk, int E, int32_t* counts, int32_t* offsets,
                   int32_t* order, int32_t* token_sorted, float* weight_sorted, int32_t* inv_order, int32_t* active,
                   int32_t* nactive, int32_t* e_sorted, void* workspace, size_t workspace_bytes, mm_stream_t stream);

}  // namespace mm

#define MM_CHECK_ARG(cond, ...) \
    do { if (!(cond)) return ::mm::set_error(MM_ERR_ARG, __VA_ARGS__); } while (0)
