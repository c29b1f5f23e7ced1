// Device code shared by the decode path (mm_gemv.hip) and the fat-expert path (mm_fat.hip): the EXL3 tile
// decode in MFMA operand layout, the input operand order, wait helpers and the route-prep launcher.
#pragma once
#include "mm_common.h"

namespace mm {

typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));

// One active expert of a call: its id, route count, first sorted position and matrix addresses.
struct ExpertRec
{
    int32_t e, cnt, first, pad;
    int64_t w[3];             // gate, up, down trellis
    int64_t pad2;
};

__device__ __forceinline__ float kinv_f() { return h2f(KINV_BITS); }
__device__ __forceinline__ float kbias_f() { return h2f(KBIAS_BITS); }

// ------------------------------------------------------------------------------------------------ decode

// The multiply-accumulate runs on v_mfma_f32_16x16x32_f16 over two tile rows at a time: A = transformed inputs
// [16 routes][32 rows], B = two decoded 16x16 tiles stacked along k, D = [16 routes][16 columns]. Lane l of B
// holds column n = l & 15 and MFMA k-group g = l >> 4 (8 values). A dot product does not depend on the order of
// its terms, so the k-group need not be adjacent rows: k-group g is rows (2g, 2g+1, 2g+8, 2g+9) of the first tile
// and the same rows of the second, which in column n are the 4 consecutive trellis states i0 .. i0+3 of each
// tile with i0 = 32 (n & 7) + 8 g + 4 (n >> 3) (PERM, ft_core.h:48-61). A carries the same rows of the inputs,
// so each lane decodes 4 adjacent states per tile and nothing moves between lanes.
//
// The 4 states span 25 stream bits ending at e = 3 i0 + 11, which lie in tile dwords b - 1 and b (b = e >> 5;
// dword -1 is dword 23: the stream wraps). One v_alignbit puts state i0 + 3 - j at bits 3j .. 3j + 15.
// The (1024 + bytesum) fp16 codes of a state pair come out packed from v_sad_u8 / v_sad_hi_u8 with 0x6400 in
// both accumulator halves; EXACT applies KINV, KBIAS with one v_pk_fma_f16 (a single rounding).
template <bool EXACT>
__device__ __forceinline__ half4_t decode4(uint32_t hi, uint32_t lo, uint32_t sh)
{
    const uint32_t X = __builtin_amdgcn_alignbit(hi, lo, sh);
    const uint32_t p0 = __builtin_amdgcn_ubfe(X, 9, 16) * MUL1;
    const uint32_t p1 = __builtin_amdgcn_ubfe(X, 6, 16) * MUL1;
    const uint32_t p2 = __builtin_amdgcn_ubfe(X, 3, 16) * MUL1;
    const uint32_t p3 = (X & 0xffffu) * MUL1;
    const uint32_t v01 = __builtin_amdgcn_sad_hi_u8(p1, 0u, __builtin_amdgcn_sad_u8(p0, 0u, 0x64006400u));
    const uint32_t v23 = __builtin_amdgcn_sad_hi_u8(p3, 0u, __builtin_amdgcn_sad_u8(p2, 0u, 0x64006400u));
    half2_t w01 = __builtin_bit_cast(half2_t, v01), w23 = __builtin_bit_cast(half2_t, v23);
    if constexpr (EXACT)
    {
        const half2_t kinv = { __builtin_bit_cast(_Float16, KINV_BITS), __builtin_bit_cast(_Float16, KINV_BITS) };
        const half2_t kbias = { __builtin_bit_cast(_Float16, KBIAS_BITS), __builtin_bit_cast(_Float16, KBIAS_BITS) };
        w01 = __builtin_elementwise_fma(w01, kinv, kbias);
        w23 = __builtin_elementwise_fma(w23, kinv, kbias);
    }
    return half4_t{ w01[0], w01[1], w23[0], w23[1] };
}

// MFMA operand order of an input row, in 32-row groups (two tile rows t = 0, 1): element 16 t + r of a group,
// r = 2 d + (r & 1) with d = 4 h + g, sits at 8 g + 4 t + 2 h + (r & 1). The lane of k-group g then finds its
// four rows (2g, 2g+1, 2g+8, 2g+9) of tile row t as 8 contiguous bytes, and those of both tile rows as 16.
__device__ __forceinline__ int operand_index(int k)
{
    const int r = k & 15, d = r >> 1;
    return (k & ~31) + 8 * (d & 3) + 4 * ((k >> 4) & 1) + 2 * (d >> 2) + (r & 1);
}

// Waits written as inline asm with a memory clobber, so the compiler neither moves LDS accesses across them
// nor drops them: buffer-to-LDS loads are counted by vmcnt but their LDS writes are invisible to the compiler.
template <int N>
__device__ __forceinline__ void wait_vmcnt()
{
    static_assert(N >= 0 && N < 64, "vmcnt range");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
__device__ __forceinline__ void wait_lgkm0() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }
// Workgroup barrier for LDS written with ds stores: the stores are complete first; loads still in flight (vmcnt)
// are not waited for, unlike __syncthreads, whose fence waits for every outstanding memory operation.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

__device__ __forceinline__ float wave_sum(float v)
{
    v += xor_lane<32>(v);
    v += xor_lane<16>(v);
    v += xor_lane<8>(v);
    v += xor_lane<4>(v);
    v += xor_lane<2>(v);
    v += xor_lane<1>(v);
    return v;
}

struct PrepArgs
{
    const void* x;            // [T][H], element type x_dtype
    const int64_t* ids;       // [n]
    const int32_t* offsets;   // permutation (null: routing found here from ids)
    const int32_t* order;
    const int32_t* active;
    const int32_t* nactive_in;
    const int64_t* wtab0;     // gate, up, down pointer tables
    const int64_t* wtab1;
    const int64_t* wtab2;
    const uint16_t* suh13;    // [E][2][H]
    ExpertRec* rec;           // [max_active]
    int32_t* counts;          // [2]: active experts, routed (valid) routes
    int32_t* pos_of;          // [n] sorted position of each route, -1 if its id is outside [0, E)
    int32_t* route_at;        // [n] route at each sorted position
    int32_t* e_at;            // [n] expert at each sorted position
    int32_t* ai_at;           // [n] active index (record) of the expert at each sorted position
    int32_t* ai_of;           // [n] active index of each route's expert
    uint16_t* xa;             // [n][2][H] fp16 in operand order
    float* xsum;              // [n][2][nb] sums of xa over each workgroup's rows
    int n, topk, E, H, nb, x_dtype, rescale;
    int cap;                  // experts with more than cap routes are left out (no record work, no outputs)
    int npos;                 // sorted positions visited (n with in-kernel routing; the permutation's valid
                              // positions must lie below it)
};

__device__ __forceinline__ int wave_sum_int(int v)
{
    v += xor_lane_i<32>(v);
    v += xor_lane_i<16>(v);
    v += xor_lane_i<8>(v);
    v += xor_lane_i<4>(v);
    v += xor_lane_i<2>(v);
    v += xor_lane_i<1>(v);
    return v;
}

// Route prep (kernel k_route_prep in mm_gemv.hip): positions, expert records and transformed inputs of n
// routes, from the ids (offsets == nullptr) or from a permutation. nb = input-row blocks per route and matrix.
int prep_blocks(int H);
void launch_route_prep(const PrepArgs& p, hipStream_t s);

// The launches of mm_moe_decode on a given workspace (argument checks included); `who` names the caller in errors.
// accumulate: out += the layer sum instead of out = the layer sum.
int moe_decode_launch(const mm_layer_t* L, const void* x, int x_dtype, int rescale, int T, int topk, const int64_t* ids,
                      const float* w, int max_rows, float* out, void* workspace, size_t workspace_bytes,
                      mm_stream_t stream, const char* who, int accumulate = 0);

// Decode workspace of n routes whose sorted positions lie below npos, and the decode path over such a
// permutation (routes of experts above cap left out) added to / written into out; no argument checks.
size_t decode_ws_bytes(int n, int npos, int E, int H, int I);
int decode_perm_launch(const mm_layer_t* L, const void* x, int x_dtype, int T, int topk, const int64_t* ids,
                       const float* w, const int32_t* offsets, const int32_t* order, const int32_t* active,
                       const int32_t* nactive, int npos, int cap, float* out, int accumulate, void* workspace,
                       hipStream_t s);

}  // namespace mm
