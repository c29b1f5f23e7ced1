// Fat-expert path (prefill): per-expert grouped GEMM with the EXL3 weights decoded into LDS and multiplied on
// MFMA, for experts that receive many routes (the reference's apply_exl3_batched_fat / run_batch,
// patches/vllm-exl3-host-dma.patch:182-201, runtime/dma_gemm.py:5-26, which reconstruct fp16 weights and run a
// 128x128 GEMM).
//
// Launches: mm_permute (sorted positions) -> k_fat_prep (transformed inputs per sorted position) -> k_fat_plan
// (expert records and the two tile lists) -> k_fat<0, 8>, k_fat16<0, 2> (gate/up) -> k_fat16<1, 4>, k_fat16<1, 2>
// (down) -> k_fat_combine.
//
// A workgroup (k_fat: 8 waves, two per SIMD; k_fat16: 16 waves, four per SIMD) owns a tile of 256 routes (sorted
// positions of one expert; 128 for an expert's last <= 128 routes) x 256 output columns:
//   gate/up (MODE 0): gate columns 128 c .. 128 c + 127 and the same up columns, so the epilogue holds both and
//                     applies the output transforms, SwiGLU and the down-input transform of that 128-block (the
//                     transforms act within 128-blocks);
//   down    (MODE 1): two 128-blocks of H; the epilogue applies the output transform and writes per-route rows.
// Per 32-row step (two tile rows) the inputs (buffer-to-LDS, FT_PA - 1 steps ahead) and the 32 trellis tiles of
// the columns (768-byte rows, buffer-to-LDS, FT_PT steps ahead) are staged in LDS by loader waves; every wave
// decodes 4 tiles of the next step into the MFMA B layout (fp16 weights, rounded as the reconstruct does) in
// between its v_mfma_f32_16x16x32_f16 over a (BM / 2) x 64 sub-tile (128 accumulators per lane), so one wave's
// decode runs while the other wave of its SIMD multiplies. The weights are decoded once per tile.
#include <algorithm>
#include <type_traits>

#include "mm_decode.h"

namespace mm {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int FT_BIG = 256;         // routes per tile (8 row blocks per row-wave)
constexpr int FT_SMALL = 128;       // routes per tile for an expert's remainder of at most 128 routes
constexpr int FT_BN = 256;          // output columns per tile
constexpr int FT_WAVES = 8;
constexpr int FT_THREADS = 64 * FT_WAVES;
constexpr int FT16_THREADS = 1024;   // the sixteen-wave form
constexpr int FT_PA = 3;            // input ring stages (loads run FT_PA - 1 steps ahead)
constexpr int FT_PT = 5;            // trellis steps in flight
constexpr int FT_TS = FT_PT + 1;    // trellis ring slots
constexpr int FT_PLAN_MAX = 1024;   // active experts the plan kernel handles

struct FatArgs
{
    const ExpertRec* rec;         // [max_active] active experts (permutation order)
    const int32_t* nactive;       // [1]
    const int32_t* tile_off;      // [max_active + 1] first tile of each active expert in this launch's list
    const int32_t* big_off;       // [max_active + 1] 256-route tiles (a 128-route tile follows them)
    const uint16_t* xa;           // mode 0: [n][H/32][gate 32, up 32]; mode 1: [n][I] (operand order)
    const uint16_t* svh13;        // [E][2][I]
    const uint16_t* suh2;         // [E][I]
    const uint16_t* svh2;         // [E][H]
    const int32_t* route_at;      // [n] flat route index of each sorted position
    uint16_t* xd;                 // mode 0 output [n][I] (operand order)
    float* Y;                     // mode 1 output [n_routes][H] (per route), fp32 or (YH) fp16 bits
    int H, I, K, N, nunits, max_active;
    float limit;
};

// Transformed inputs of every fat route, one workgroup per sorted position: r16(FWHT(x16 * suh_m) * HAD) per
// 128-block (ft_core.h:96-102), where x16 is fp16 input as is, or bf16 / fp32 input rounded through bf16. Row pos
// of xa holds, per 32-element step, the gate step then the up step in operand order (128 bytes: one cache line
// per step, which the gate/up kernel loads whole).
//
// Wave w transforms matrix w >> 1, blocks (w & 1) * nb / 2 .. , four blocks at a time, 16 lanes per block and
// 8 elements per lane: lane 4 q + g of a block holds the elements k = 32 q + 2 g + j + 8 h + 16 t (j, h, t in
// {0, 1}) as v[4 t + 2 h + j], exactly the 8 operand-order positions 8 g .. 8 g + 7 of step q, so it stores them
// with one 16-byte write. The butterflies keep the reference's order and arithmetic (strides 1, 2, 4, ..., 64,
// (a, b) -> (a + b, a - b), ft_core.h:89-94): strides 1, 8, 16 pair elements within a lane; strides 2 and 4 pair
// lanes 4 q + g and 4 q + (g ^ 1 or 2), strides 32 and 64 lanes q ^ 1 and q ^ 2 of the block (DPP moves, all
// within the block's 16 lanes). The lane holding the upper element of a cross-lane pair forms partner - self as
// fma(-1, self, partner), the same single rounding.
__device__ __forceinline__ float xlane(float v, int pattern)
{
    if (pattern == 1) return xor_lane<1>(v);
    if (pattern == 2) return xor_lane<2>(v);
    if (pattern == 4) return xor_lane<4>(v);
    return xor_lane<8>(v);
}

// The 128-point transform of a block held by 16 lanes (lane 4 q + g of the block) with 8 elements each,
// v[4 t + 2 h + j] = element 32 q + 2 g + j + 8 h + 16 t. sgn = (g & 1, g & 2, q & 1, q & 2 ? -1 : 1).
struct Lane8Signs
{
    float s2, s4, s32, s64;
};
__device__ __forceinline__ Lane8Signs lane8_signs(int lane)
{
    const int g = lane & 3, q = (lane >> 2) & 3;
    return { (g & 1) ? -1.0f : 1.0f, (g & 2) ? -1.0f : 1.0f, (q & 1) ? -1.0f : 1.0f, (q & 2) ? -1.0f : 1.0f };
}
__device__ __forceinline__ void fwht128_lane8(float (&v)[8], const Lane8Signs& sg)
{
    // stride 1 (j)
#pragma unroll
    for (int i = 0; i < 8; i += 2)
    {
        const float a0 = v[i], a1 = v[i + 1];
        v[i] = a0 + a1;
        v[i + 1] = a0 - a1;
    }
    // strides 2, 4 (lanes g ^ 1, g ^ 2)
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = __builtin_fmaf(sg.s2, v[i], xlane(v[i], 1));
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = __builtin_fmaf(sg.s4, v[i], xlane(v[i], 2));
    // strides 8 (h), 16 (t)
#pragma unroll
    for (int i = 0; i < 8; ++i)
        if ((i & 2) == 0)
        {
            const float a0 = v[i], a1 = v[i + 2];
            v[i] = a0 + a1;
            v[i + 2] = a0 - a1;
        }
#pragma unroll
    for (int i = 0; i < 4; ++i)
    {
        const float a0 = v[i], a1 = v[i + 4];
        v[i] = a0 + a1;
        v[i + 4] = a0 - a1;
    }
    // strides 32, 64 (lanes q ^ 1, q ^ 2)
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = __builtin_fmaf(sg.s32, v[i], xlane(v[i], 4));
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = __builtin_fmaf(sg.s64, v[i], xlane(v[i], 8));
}
// element index of v[i] in its 128-block for the lane (q, g) of the block
__device__ __forceinline__ int lane8_k(int lane, int i)
{
    return 32 * ((lane >> 2) & 3) + 2 * (lane & 3) + (i & 1) + 8 * ((i >> 1) & 1) + 16 * (i >> 2);
}

template <int XD>
// cnt_e (optional): the expert's route count, read with the row and compared only before the stores (rows of
// experts with cnt_e[0] <= cap are not stored), so it costs no round trip of its own.
__device__ __forceinline__ void fat_prep_row_t(const void* x, size_t row, int e, int pos, const uint16_t* suh13,
                                               uint16_t* xa, int H, const int32_t* cnt_e, int cap)
{
    int ce = cnt_e ? cnt_e[0] : cap + 1;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int g = lane & 3, q = (lane >> 2) & 3, bl = lane >> 4;
    const int nb = H / 128;
    const Lane8Signs sg = lane8_signs(lane);
    const uint16_t* su0 = suh13 + (size_t)e * 2 * H;       // gate; up follows
    uint16_t* dst = xa + (size_t)pos * 2 * H + 8 * g;
    // raw words of element pair (t, h): fp16 / bf16 input as one dword, fp32 as two
    using Raw = typename std::conditional<XD == MM_DTYPE_F32, uint2, uint32_t>::type;
    // lane group bl of wave w takes blocks w + 4 bl + 16 i of the row, both matrices (the input is read once): two
    // blocks per pass, all loaded before any is used (blocks past the row reload its last block and are not stored)
    for (int f0 = wave + 4 * bl; f0 < nb; f0 += 32)
    {
        Raw xr[2][4];
        uint32_t sr[2][2][4];
#pragma unroll
        for (int it = 0; it < 2; ++it)
        {
            const int k0 = min(f0 + 16 * it, nb - 1) * 128 + 32 * q + 2 * g;
#pragma unroll
            for (int th = 0; th < 4; ++th)
            {
                const int k = k0 + 8 * (th & 1) + 16 * (th >> 1);
                if constexpr (XD == MM_DTYPE_F32)
                    xr[it][th] = *reinterpret_cast<const uint2*>(static_cast<const float*>(x) + row + k);
                else
                    xr[it][th] = *reinterpret_cast<const uint32_t*>(static_cast<const uint16_t*>(x) + row + k);
                sr[it][0][th] = *reinterpret_cast<const uint32_t*>(su0 + k);
                sr[it][1][th] = *reinterpret_cast<const uint32_t*>(su0 + H + k);
            }
        }
        asm volatile("" : "+v"(ce));       // the count is first used here, after the row's loads
        if (ce <= cap) return;
#pragma unroll
        for (int it = 0; it < 2; ++it)
        {
            const int b = f0 + 16 * it;
            if (b >= nb) break;
            // th = 2 t + h: elements 8 h + 16 t (+ 0, 1) of the lane's column pair go to xv[4 t + 2 h + j]
            float xv[8];
#pragma unroll
            for (int th = 0; th < 4; ++th)
            {
                const int i = 4 * (th >> 1) + 2 * (th & 1);
                if constexpr (XD == MM_DTYPE_F16)
                {
                    xv[i] = h2f((uint16_t)(xr[it][th] & 0xffffu));
                    xv[i + 1] = h2f((uint16_t)(xr[it][th] >> 16));
                }
                else if constexpr (XD == MM_DTYPE_BF16)
                {
                    xv[i] = r16(__uint_as_float(xr[it][th] << 16));
                    xv[i + 1] = r16(__uint_as_float(xr[it][th] & 0xffff0000u));
                }
                else
                {
                    xv[i] = r16(bf16_value(__uint_as_float(xr[it][th].x)));
                    xv[i + 1] = r16(bf16_value(__uint_as_float(xr[it][th].y)));
                }
            }
#pragma unroll
            for (int m = 0; m < 2; ++m)
            {
                float v[8];
#pragma unroll
                for (int th = 0; th < 4; ++th)
                {
                    const int i = 4 * (th >> 1) + 2 * (th & 1);
                    v[i] = xv[i] * h2f((uint16_t)(sr[it][m][th] & 0xffffu));
                    v[i + 1] = xv[i + 1] * h2f((uint16_t)(sr[it][m][th] >> 16));
                }
                fwht128_lane8(v, sg);
                uint4 o;
                o.x = (uint32_t)f2h(v[0] * HAD) | ((uint32_t)f2h(v[1] * HAD) << 16);
                o.y = (uint32_t)f2h(v[2] * HAD) | ((uint32_t)f2h(v[3] * HAD) << 16);
                o.z = (uint32_t)f2h(v[4] * HAD) | ((uint32_t)f2h(v[5] * HAD) << 16);
                o.w = (uint32_t)f2h(v[6] * HAD) | ((uint32_t)f2h(v[7] * HAD) << 16);
                // a nontemporal store: the 16 KB per route (2 GB at 16k tokens) stream past the caches, which
                // their readers' tiles would otherwise lose to them (16k layer 9.67-9.79 -> 9.50-9.52 ms)
                __builtin_nontemporal_store(u32x4{ o.x, o.y, o.z, o.w },
                                            reinterpret_cast<u32x4*>(dst + (size_t)(4 * b + q) * 64 + m * 32));
            }
        }
    }
}

__device__ __forceinline__ void fat_prep_row(const void* x, int x_dtype, size_t row, int e, int pos,
                                             const uint16_t* suh13, uint16_t* xa, int H, const int32_t* cnt_e, int cap)
{
    if (x_dtype == MM_DTYPE_F16)
        fat_prep_row_t<MM_DTYPE_F16>(x, row, e, pos, suh13, xa, H, cnt_e, cap);
    else if (x_dtype == MM_DTYPE_BF16)
        fat_prep_row_t<MM_DTYPE_BF16>(x, row, e, pos, suh13, xa, H, cnt_e, cap);
    else
        fat_prep_row_t<MM_DTYPE_F32>(x, row, e, pos, suh13, xa, H, cnt_e, cap);
}

__global__ __launch_bounds__(256) void k_fat_prep(const void* x, int x_dtype, const int32_t* e_sorted,
                                                  const int32_t* counts, const int32_t* offsets, const int32_t* order,
                                                  const uint16_t* suh13, uint16_t* xa, int topk, int E, int H, int cap)
{
    const int pos = blockIdx.x;
    // round trip 1: the routed count, the route and its expert (pos < n: in range past the routed count too)
    const int nvalid = offsets[E];
    const int s = order[pos], e = e_sorted[pos];
    if (pos >= nvalid || (s | e) < 0) return;        // s, e >= 0: the test only keeps their loads before the branch
    // round trip 2: the expert's route count with the row's loads; rows of experts at or below cap are not stored
    fat_prep_row(x, x_dtype, (size_t)(s / topk) * H, e, pos, suh13, xa, H, counts + e, cap);
}

// Sorted-route form: position pos belongs to the expert e with offsets[e] <= pos < offsets[e + 1] (binary search
// over the E + 1 offsets) and to token token_sorted[pos]; only positions of experts with counts[e] > 0 (the
// selected fat experts) are transformed.
__global__ __launch_bounds__(256) void k_fatb_prep(const void* x, int x_dtype, const int64_t* token_sorted,
                                                   const int32_t* counts, const int32_t* offsets,
                                                   const uint16_t* suh13, uint16_t* xa, int T, int E, int H)
{
    const int pos = blockIdx.x;
    if (pos >= offsets[E]) return;
    int lo = 0, hi = E;                 // largest e with offsets[e] <= pos
    while (hi - lo > 1)
    {
        const int mid = (lo + hi) >> 1;
        if (offsets[mid] <= pos) lo = mid; else hi = mid;
    }
    const int e = lo;
    if (counts[e] <= 0 || pos >= offsets[e] + counts[e]) return;
    const int64_t t = token_sorted[pos];
    if (t < 0 || t >= T) return;
    fat_prep_row(x, x_dtype, (size_t)t * H, e, pos, suh13, xa, H, nullptr, 0);
}

// Expert records and the tile lists of the experts with more than cap routes. An expert of c routes gets
// c / 256 tiles of 256 routes; a remainder r = c % 256 takes one more 256-route tile if r > 128 (a 256-route step
// costs less than two 128-route steps), else one 128-route tile. off_big / off_small = tiles of active experts
// 0 .. a-1 in each list.
__global__ __launch_bounds__(FT_PLAN_MAX) void k_fat_plan(const int32_t* counts, const int32_t* offsets,
                                                         const int32_t* active, const int32_t* nactive,
                                                         const int64_t* gate, const int64_t* up, const int64_t* down,
                                                         ExpertRec* rec, int32_t* off_big, int32_t* off_small,
                                                         int max_active, int cap)
{
    __shared__ int s_w[2][FT_PLAN_MAX / 64];
    const int a = threadIdx.x, lane = a & 63, wave = a >> 6;
    const int nact = min(nactive[0], max_active);
    int c = 0;
    if (a < nact)
    {
        const int e = active[a];
        c = counts[e];
        ExpertRec r{ e, c, offsets[e], 0, { gate[e], up[e], down[e] }, 0 };
        rec[a] = r;
    }
    int tb = 0, ts = 0;
    if (c > cap)
    {
        const int r = c % FT_BIG;
        tb = c / FT_BIG + (r > FT_SMALL ? 1 : 0);
        ts = (r > 0 && r <= FT_SMALL) ? 1 : 0;
    }
    const int ib = wave_incl_scan(tb), is = wave_incl_scan(ts);
    if (lane == 63)
    {
        s_w[0][wave] = ib;
        s_w[1][wave] = is;
    }
    __syncthreads();
    int bb = 0, bs = 0, nb = 0, ns = 0;
    for (int w = 0; w < FT_PLAN_MAX / 64; ++w)
    {
        if (w < wave)
        {
            bb += s_w[0][w];
            bs += s_w[1][w];
        }
        nb += s_w[0][w];
        ns += s_w[1][w];
    }
    if (a < max_active)
    {
        off_big[a] = bb + ib - tb;
        off_small[a] = bs + is - ts;
    }
    if (a == 0)
    {
        off_big[max_active] = nb;
        off_small[max_active] = ns;
    }
}

// LDS slot of 16-byte chunk q of row r of an input stage whose rows hold NA x 64 bytes (NA = 2: gate chunks 0 .. 3,
// up chunks 4 .. 7): the 16 rows one MFMA operand read covers fall in distinct 16-byte bank groups both for 8
// lanes over 32 banks and for 16 lanes over 64 banks.
template <int NA>
__device__ __forceinline__ int chunk_slot(int q, int r)
{
    if constexpr (NA == 2) return q ^ (((r >> 1) & 7) ^ ((r & 1) << 2));
    else return q ^ (((r >> 1) ^ (r >> 2)) & 3);
}

// Epilogue of a fat tile from the transposed fp16 C tile in LDS (column c at c * CS halves, the raw GEMM outputs
// rounded to fp16): gate/up (MODE 0) applies the output transforms, SwiGLU and the down-input transform of the
// tile's 128-block and writes the down input in operand order; down (MODE 1) applies the output transform of its
// two 128-blocks and writes per-route rows. The C tile is complete (the caller's barrier) when this runs.
template <int MODE, int CS, bool YH, int NW = FT_WAVES>
__device__ __forceinline__ void fat_tile_epilogue(const FatArgs& a, const uint16_t* C, int rows, int pos0, int e,
                                                  int nu, int wave, int lane)
{
    // Transforms in the layout of fwht128_lane8: per pass a wave takes 8 rows; lane (rpair, q, g) = (lane >> 4,
    // (lane >> 2) & 3, lane & 3) holds rows r0 + 2 rpair and r0 + 2 rpair + 1 (one dword of the transposed tile per
    // column) of the 8 columns lane8_k(lane, i) of each 128-block, so each butterfly stage is in-lane or a DPP
    // exchange within 16 lanes.
    const Lane8Signs sg = lane8_signs(lane);
    const int rpair = lane >> 4;
    int kk[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) kk[i] = lane8_k(lane, i);
    // column c at rows r, r + 1 (r even)
    auto rows2 = [&](int c, int r, float& v0, float& v1) {
        const uint32_t d = *reinterpret_cast<const uint32_t*>(C + (size_t)c * CS + r);
        v0 = h2f((uint16_t)(d & 0xffffu));
        v1 = h2f((uint16_t)(d >> 16));
    };
    if constexpr (MODE == 0)
    {
        const int c0 = nu * 128;
        const uint16_t* svg = a.svh13 + ((size_t)e * 2 + 0) * a.I + c0;
        const uint16_t* svu = a.svh13 + ((size_t)e * 2 + 1) * a.I + c0;
        const uint16_t* sd = a.suh2 + (size_t)e * a.I + c0;
        float sgv[8], suv[8], sdv[8];
#pragma unroll
        for (int i = 0; i < 8; ++i)
        {
            sgv[i] = h2f(svg[kk[i]]);
            suv[i] = h2f(svu[kk[i]]);
            sdv[i] = h2f(sd[kk[i]]);
        }
        // operand order: the lane's 8 elements are positions 32 q + 8 g .. + 7 of the block, v[i] at + i
        const int od = c0 + 32 * ((lane >> 2) & 3) + 8 * (lane & 3);
        for (int r0 = 8 * wave; r0 < rows; r0 += 8 * NW)
        {
            const int r = r0 + 2 * rpair;
            float gv[2][8], uv[2][8];
#pragma unroll
            for (int i = 0; i < 8; ++i)
            {
                rows2(kk[i], r, gv[0][i], gv[1][i]);
                rows2(128 + kk[i], r, uv[0][i], uv[1][i]);
            }
#pragma unroll
            for (int h2 = 0; h2 < 2; ++h2)
            {
                // the tile holds fp16 values, so the output transform's first rounding is exact
                fwht128_lane8(gv[h2], sg);
                fwht128_lane8(uv[h2], sg);
                float xv[8];
#pragma unroll
                for (int i = 0; i < 8; ++i)
                {
                    const float gg = r16((gv[h2][i] * HAD) * sgv[i]);
                    const float uu = r16((uv[h2][i] * HAD) * suv[i]);
                    xv[i] = r16(act_gu(gg, uu, a.limit)) * sdv[i];
                }
                fwht128_lane8(xv, sg);
                if (r + h2 < rows)
                {
                    uint4 o;
                    o.x = (uint32_t)f2h(xv[0] * HAD) | ((uint32_t)f2h(xv[1] * HAD) << 16);
                    o.y = (uint32_t)f2h(xv[2] * HAD) | ((uint32_t)f2h(xv[3] * HAD) << 16);
                    o.z = (uint32_t)f2h(xv[4] * HAD) | ((uint32_t)f2h(xv[5] * HAD) << 16);
                    o.w = (uint32_t)f2h(xv[6] * HAD) | ((uint32_t)f2h(xv[7] * HAD) << 16);
                    *reinterpret_cast<uint4*>(a.xd + (size_t)(pos0 + r + h2) * a.I + od) = o;
                }
            }
        }
    }
    else
    {
        float svv[2][8];
#pragma unroll
        for (int hb = 0; hb < 2; ++hb)
        {
            const uint16_t* sv = a.svh2 + (size_t)e * a.H + (2 * nu + hb) * 128;
#pragma unroll
            for (int i = 0; i < 8; ++i) svv[hb][i] = h2f(sv[kk[i]]);
        }
        for (int r0 = 8 * wave; r0 < rows; r0 += 8 * NW)
        {
            const int r = r0 + 2 * rpair;
            // output rows of the lane's two routes (a row past the tile's routes is not stored)
            const int y0 = r < rows ? a.route_at[pos0 + r] : 0;
            const int y1 = r + 1 < rows ? a.route_at[pos0 + r + 1] : 0;
#pragma unroll
            for (int hb = 0; hb < 2; ++hb)
            {
                const int c0 = (2 * nu + hb) * 128;
                float yv[2][8];
#pragma unroll
                for (int i = 0; i < 8; ++i) rows2(hb * 128 + kk[i], r, yv[0][i], yv[1][i]);
#pragma unroll
                for (int h2 = 0; h2 < 2; ++h2)
                {
                    fwht128_lane8(yv[h2], sg);
#pragma unroll
                    for (int i = 0; i < 8; ++i) yv[h2][i] = r16((yv[h2][i] * HAD) * svv[hb][i]);
                    if (r + h2 < rows)
                    {
                        const size_t yo = (size_t)(h2 ? y1 : y0) * a.H + c0;
                        // elements 2 p, 2 p + 1 are adjacent columns kk[2 p], kk[2 p] + 1
#pragma unroll
                        for (int p2 = 0; p2 < 4; ++p2)
                        {
                            if constexpr (YH)
                            {
                                // the output transform rounded y to fp16: the half stores are exact
                                const uint32_t w2 = (uint32_t)f2h(yv[h2][2 * p2]) | ((uint32_t)f2h(yv[h2][2 * p2 + 1]) << 16);
                                *reinterpret_cast<uint32_t*>(reinterpret_cast<uint16_t*>(a.Y) + yo + kk[2 * p2]) = w2;
                            }
                            else
                            {
                                *reinterpret_cast<float2*>(a.Y + yo + kk[2 * p2]) =
                                    make_float2(yv[h2][2 * p2], yv[h2][2 * p2 + 1]);
                            }
                        }
                    }
                }
            }
        }
    }
}

// MB = 16-row blocks per row-wave: tiles of BM = 32 MB routes (256 or 128). 8 waves: wave (wm, wn) = (w >> 2,
// w & 3) multiplies row blocks wm, wm + 2, wm + 4, ... (rows 16 (2 i + wm) .. + 15) by column tiles 4 wn .. 4 wn + 3
// of 16, so in a tile with fewer routes the two waves of a SIMD keep about the same number of row blocks
// (0.7 % off the 16k layer against contiguous halves); every wave loads an
// eighth of the inputs and waves 0 .. 3 also the trellis (chunk w: tile row w >> 1 of matrix / block w & 1),
// which runs further ahead; wave w decodes column tiles 2 (w & 3), 2 (w & 3) + 1 of sub-block w >> 2 in both tile
// rows (chunks w >> 2 and 2 + (w >> 2)). Rows past the tile's routes read zero inputs.
template <int MODE, int MB, bool YH = false>
__global__ __launch_bounds__(FT_THREADS, 1) void k_fat(FatArgs a)
{
    constexpr int BM = 32 * MB;
    constexpr int NA = MODE == 0 ? 2 : 1;                        // input matrices (gate, up share the tile)
    constexpr int SEG = NA * 64;                                 // bytes of one route's step (gate, up)
    constexpr int A_STAGE = BM * SEG;                            // one step's inputs
    constexpr int LA = A_STAGE / 1024 / FT_WAVES;                // input loads (1 KB each) per wave and step
    constexpr int T_SLOT = 4 * 1024;                             // one step's trellis: 4 chunks of 8 tiles
    constexpr int B_BUF = 16 * 64 * 16;                          // decoded B of one step: 16 tiles x 64 lanes
    constexpr int A_BYTES = FT_PA * A_STAGE, T_BYTES = FT_TS * T_SLOT;
    constexpr int MAIN = A_BYTES + T_BYTES + 2 * B_BUF;
    constexpr int CS = BM + 2;                                   // transposed C tile: column stride in halves
    constexpr int SMEM = MAIN > FT_BN * CS * 2 ? MAIN : FT_BN * CS * 2;
    static_assert(SMEM <= 160 * 1024, "LDS");
    static_assert(((CS / 2) & 1) == 1, "odd dword stride: conflict-free column reads");
    static_assert(MB % 2 == 0, "one decoded tile per two row blocks");
    __shared__ __align__(16) uint8_t smem[SMEM];
    uint8_t* Aring = smem;
    uint8_t* Tring = smem + A_BYTES;
    uint8_t* Bdec = smem + A_BYTES + T_BYTES;

    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    // ---- tile. The grid is sized for the most tiles a call can have; the work = tiles x column blocks of this
    // call is spread evenly over the 8 XCDs (workgroup b runs on XCD b % 8), and consecutive work items (the
    // column blocks of one route block, then the next block of the same expert) stay on one XCD, so they share
    // its L2 for the inputs and the trellis.
    const int nact = min(a.nactive[0], a.max_active);
    const int total = a.tile_off[nact];
    const int work = total * a.nunits, per_xcd = (work + 7) >> 3;
    const int L = (int)(blockIdx.x & 7) * per_xcd + (int)(blockIdx.x >> 3);
    if ((int)(blockIdx.x >> 3) >= per_xcd || L >= work) return;
    const int mt = L / a.nunits, nu = L % a.nunits;
    int lo = 0, hi = nact - 1;
    while (lo < hi)
    {
        const int mid = (lo + hi + 1) >> 1;
        if (a.tile_off[mid] <= mt) lo = mid; else hi = mid - 1;
    }
    const ExpertRec* rp = a.rec + lo;
    // an expert's 256-route tiles come first; its 128-route tile (if any) follows them
    const int row0 = BM == FT_BIG ? (mt - a.tile_off[lo]) * BM : (a.big_off[lo + 1] - a.big_off[lo]) * FT_BIG;
    const int rows = __builtin_amdgcn_readfirstlane(min(BM, rp->cnt - row0));
    const int pos0 = __builtin_amdgcn_readfirstlane(rp->first + row0);
    const int e = __builtin_amdgcn_readfirstlane(rp->e);
    const int S = a.K / 32;

    // ---- buffer descriptors (wave-uniform bases through readfirstlane, each half widened as uint32_t)
    auto uniform_ptr = [](const void* p) {
        const uint64_t v = (uint64_t)(uintptr_t)p;
        const uint32_t l = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)v);
        const uint32_t h = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(v >> 32));
        return reinterpret_cast<void*>((uintptr_t)((uint64_t)l | ((uint64_t)h << 32)));
    };
    const bool tloader = wave < 4;
    // trellis loader (waves 0 .. 3): chunk q = wave of step s is tile row 2 s + (q >> 1) of matrix q & 1 (gate/up)
    // or of column block 2 nu + (q & 1) (down), 8 tiles = 768 bytes, 12 bytes per lane stored 16 bytes apart.
    // Steps past the end reload the last row into the free slot, so every step issues one load.
    const int tq = wave & 3;
    const uint32_t row_bytes = (uint32_t)(a.N / 16) * 96, wbytes = (uint32_t)(a.K / 16) * row_bytes;
    const void* wbase = (const void*)(uintptr_t)(MODE == 0 ? ((tq & 1) ? rp->w[1] : rp->w[0]) : rp->w[2]);
    const __amdgpu_buffer_rsrc_t wres = __builtin_amdgcn_make_buffer_rsrc(uniform_ptr(wbase), (short)0, (int)wbytes,
                                                                          0x00020000);
    const uint32_t wcol = MODE == 0 ? (uint32_t)nu * 768 : (uint32_t)(2 * nu + (tq & 1)) * 768;
    auto load_trellis = [&](int s) {
        const uint32_t tr = (uint32_t)(2 * min(s, S - 1) + (tq >> 1));
        __builtin_amdgcn_raw_ptr_buffer_load_lds(wres, Tring + (size_t)(s % FT_TS) * T_SLOT + (size_t)tq * 1024, 12,
                                                 tr * row_bytes + wcol + (uint32_t)lane * 12, 0, 0, 0);
    };
    // inputs (every wave): LA loads of 1 KB = 1024 / SEG rows each (SEG / 16 lanes per row step); chunk q of row r
    // goes to slot chunk_slot(q, r). Rows past the tile's routes and steps past the end read out of range (zero,
    // no memory access).
    const uint32_t a_row = (uint32_t)NA * a.K * 2;                       // bytes per route of the inputs
    const __amdgpu_buffer_rsrc_t ares = __builtin_amdgcn_make_buffer_rsrc(
        uniform_ptr(a.xa + (size_t)pos0 * NA * a.K), (short)0, (int)((uint32_t)rows * a_row), 0x00020000);
    auto load_input = [&](int s, int u) {
        const int st = s % FT_PA;
        const uint32_t ks = s < S ? (uint32_t)s * SEG : 0x40000000u; // the range is below 2^30
        const int li = wave * LA + u;                                  // 0 .. A_STAGE / 1024 - 1
        const int r = li * (1024 / SEG) + lane / (SEG / 16), slot = lane % (SEG / 16);
        const uint32_t voff = (uint32_t)r * a_row + (uint32_t)chunk_slot<NA>(slot, r) * 16 + ks;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(ares, Aring + (size_t)st * A_STAGE + (size_t)li * 1024, 16, voff, 0, 0, 0);
    };

    // ---- decode: lane (col, g) decodes states i0 .. i0+3 of column col in a tile
    const int col = lane & 15, g = lane >> 4;
    const int i0 = 32 * (col & 7) + 8 * g + 4 * (col >> 3);
    const int eb = 3 * i0 + 11;
    const int blo = eb >> 5, bhi = (blo + 23) % 24;
    const int llo = 4 * (blo / 3) + blo % 3, lhi = 4 * (bhi / 3) + bhi % 3;
    const uint32_t sh = 31u - (uint32_t)(eb & 31);
    // Wave w decodes column tiles 2 (w & 3) and 2 (w & 3) + 1 of sub-block w >> 2 (chunks w >> 2 and 2 + (w >> 2):
    // tile rows 0 and 1 of the step) and stores each column tile's 8 k-values per lane, tile row 0 in the low 8
    // bytes and row 1 in the high 8, as one 16-byte write (lane-contiguous: no LDS bank conflicts). Decoded tile k
    // of the wave (k = 0 .. 3) is tile row k & 1 of column tile 2 (w & 3) + (k >> 1): trellis words at
    // tword + (k & 1) * 512 + (k >> 1) * 32.
    const int db = wave >> 2, dc = 2 * (wave & 3);
    const uint32_t* tword = reinterpret_cast<const uint32_t*>(Tring + (size_t)db * 1024 + (size_t)dc * 128);
    uint8_t* bdst = Bdec + ((size_t)(db * 8 + dc) * 64 + lane) * 16;
    // ---- MFMA: rows 16 (2 i + wm) + col of input matrix wn >> 1 (gate/up), B tiles 4 wn .. + 3
    const int wm = wave >> 2, wn = wave & 3;
    const uint8_t* bsrc = Bdec + ((size_t)(wn * 4) * 64 + lane) * 16;
    int aoff[MB];
#pragma unroll
    for (int i = 0; i < MB; ++i)
    {
        const int r = 16 * (2 * i + wm) + col;
        aoff[i] = r * SEG + chunk_slot<NA>((MODE == 0 ? (wn >> 1) : 0) * 4 + g, r) * 16;
    }
    float4_t acc[MB][4];
#pragma unroll
    for (int i = 0; i < MB; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = float4_t{ 0.f, 0.f, 0.f, 0.f };

    // Loads in issue order, per wave: inputs of step 0, [trellis of steps 0 .. FT_PT - 1], inputs of step 1, then
    // in step s [the trellis of step s + FT_PT] and the inputs of step s + 2 (LA loads, in between the MFMAs);
    // [..] = waves 0 .. 3 only. At the top of step s the inputs of step s (issued in step s - 2, or before the loop)
    // are complete once at most LA (+ 1 trellis load for waves 0 .. 3) loads are outstanding: that is exactly what
    // step s - 1 issued after them (step 0: more than that came after). The trellis of step s + 1 is older than
    // the inputs of step s (FT_PT - 1 > 2 steps earlier, or before them in the prologue, with more than LA + 1 loads
    // after it), so it is complete too. One barrier per step then publishes the loads and the tiles decoded in step
    // s - 1.
    static_assert(FT_PA == 3 && FT_PT >= 4, "issue order above");
#pragma unroll
    for (int u = 0; u < LA; ++u) load_input(0, u);
    asm volatile("" ::: "memory");                                // keep the issue order
    if (tloader)
        for (int s = 0; s < FT_PT; ++s) load_trellis(s);
    asm volatile("" ::: "memory");
#pragma unroll
    for (int u = 0; u < LA; ++u) load_input(1, u);
    if (tloader) wait_vmcnt<LA + FT_PT - 1>(); else wait_vmcnt<LA>();          // trellis of step 0
    lds_barrier();
#pragma unroll
    for (int v = 0; v < 2; ++v)
    {
        const half4_t r0 = decode4<true>(tword[v * 32 + lhi], tword[v * 32 + llo], sh);
        const half4_t r1 = decode4<true>(tword[512 + v * 32 + lhi], tword[512 + v * 32 + llo], sh);
        *reinterpret_cast<half8_t*>(bdst + v * 1024) = half8_t{ r0[0], r0[1], r0[2], r0[3], r1[0], r1[1], r1[2], r1[3] };
    }
    // Row blocks of this wave that hold routes of the tile (uniform; blocks i < nvb): in a partial tile a wave skips
    // the MFMAs and input reads of its empty row blocks (their accumulators stay zero and are never stored); loads
    // and decode, which serve the whole workgroup, run either way. Full waves take the scheduled variant.
    const int nvb = max(0, min(MB, ((rows + 15) / 16 - wm + 1) / 2));
    auto main_loop = [&](auto part_tag) {
        constexpr bool PART = decltype(part_tag)::value;
        for (int s = 0; s < S; ++s)
        {
            if (tloader) wait_vmcnt<LA + 1>(); else wait_vmcnt<LA>();
            lds_barrier();
            if (tloader) load_trellis(s + FT_PT);
            // one step: the trellis words of step s + 1 and the operands of step s first, then per row block its 4
            // MFMAs, one tile of step s + 1 decoded after every MB / 4 blocks
            // slot offset as one scalar, so each read is a per-lane base plus an immediate
            const uint32_t toff = (uint32_t)__builtin_amdgcn_readfirstlane(((s + 1) % FT_TS) * T_SLOT);
            const uint8_t* thp = reinterpret_cast<const uint8_t*>(tword + lhi) + toff;
            const uint8_t* tlp = reinterpret_cast<const uint8_t*>(tword + llo) + toff;
            uint32_t th[4], tl[4];
    #pragma unroll
            for (int u = 0; u < 4; ++u)
            {
                th[u] = *reinterpret_cast<const uint32_t*>(thp + (u & 1) * 2048 + (u >> 1) * 128);
                tl[u] = *reinterpret_cast<const uint32_t*>(tlp + (u & 1) * 2048 + (u >> 1) * 128);
            }
            const uint8_t* as = Aring + (size_t)(s % FT_PA) * A_STAGE;
            const uint8_t* bs = bsrc + (size_t)(s & 1) * B_BUF;
            uint8_t* bd = bdst + (size_t)((s + 1) & 1) * B_BUF;
            // every operand of the step is read before the step's LDS writes (input loads, decoded tiles): the
            // compiler keeps LDS accesses that may alias in program order, so reads placed after a write would each
            // wait a full LDS round trip
            half8_t B[4], A[MB];
    #pragma unroll
            for (int j = 0; j < 4; ++j) B[j] = *reinterpret_cast<const half8_t*>(bs + j * 1024);
    #pragma unroll
            for (int i = 0; i < MB; ++i)
                if (!PART || i < nvb) A[i] = *reinterpret_cast<const half8_t*>(as + aoff[i]);
            // tile 0 is decoded before the first MFMA: the decode runs while the workgroup's operand reads of the
            // step are still being served (about 2 % off the layer against decoding it after the MFMAs of row
            // blocks 0 .. MB / 4 - 1); tiles 1 .. 3 follow row blocks MB / 4 - 1, MB / 2 - 1, 3 MB / 4 - 1, and
            // each column tile is stored once both of its tile rows are decoded
            half4_t d0 = decode4<true>(th[0], tl[0], sh);
    #pragma unroll
            for (int i = 0; i < MB; ++i)
            {
                if (!PART || i < nvb)
    #pragma unroll
                    for (int j = 0; j < 4; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[i], B[j], acc[i][j], 0, 0, 0);
                if (i % (MB / LA) == 0) load_input(s + FT_PA - 1, i / (MB / LA));
                if (i % (MB / 4) == MB / 4 - 1 && i / (MB / 4) < 3)
                {
                    const int u = i / (MB / 4) + 1;
                    const half4_t d = decode4<true>(th[u], tl[u], sh);
                    if (u & 1)
                        *reinterpret_cast<half8_t*>(bd + (u >> 1) * 1024) =
                            half8_t{ d0[0], d0[1], d0[2], d0[3], d[0], d[1], d[2], d[3] };
                    else
                        d0 = d;
                }
            }
            // schedule: the LDS reads first, the decode of tile 0, then one MFMA followed by two VALU
            // instructions (the rest of the decode, which needs about that many per MFMA), so a wave keeps its MFMA
            // pipe busy between its own decode instructions
            if constexpr (!PART)
            {
                __builtin_amdgcn_sched_group_barrier(0x0100, 4 + MB + 8, 0);
                __builtin_amdgcn_sched_group_barrier(0x0002, 16, 0);
    #pragma unroll
                for (int k = 0; k < 4 * MB; ++k)
                {
                    __builtin_amdgcn_sched_group_barrier(0x0008, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(0x0002, 2, 0);
                }
            }
        }
    };
    if (nvb == MB)
        main_loop(std::false_type{});
    else
        main_loop(std::true_type{});
    wait_vmcnt<0>();
    lds_barrier();

    // ---- epilogue through a transposed fp16 C tile in LDS (column c at c * CS halves; the output transforms
    // round y to fp16 first)
    uint16_t* C = reinterpret_cast<uint16_t*>(smem);
#pragma unroll
    for (int i = 0; i < MB; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
        {
            const int c = (wn * 4 + j) * 16 + col, r = 16 * (2 * i + wm) + 4 * g;
            uint32_t* d = reinterpret_cast<uint32_t*>(C + (size_t)c * CS + r);
            d[0] = (uint32_t)f2h(acc[i][j][0]) | ((uint32_t)f2h(acc[i][j][1]) << 16);
            d[1] = (uint32_t)f2h(acc[i][j][2]) | ((uint32_t)f2h(acc[i][j][3]) << 16);
        }
    __syncthreads();
    fat_tile_epilogue<MODE, CS, YH>(a, C, rows, pos0, e, nu, wave, lane);
}

// Sixteen-wave form of the tile (four waves per SIMD, 64 accumulators per lane): MBW = row blocks per wave, BM =
// 64 MBW routes (256 or 128). Wave (wm, wn) = (w >> 2, w & 3) multiplies row blocks wm, wm + 4, ... (rows
// 16 (4 i + wm) .. + 15) by column tiles 4 wn .. 4 wn + 3, so each SIMD (waves w, w + 4, w + 8, w + 12) holds
// one column group over every row block of the tile. Inputs: buffer-to-LDS, two steps ahead in a three-stage ring,
// input load li of a step (1 KB) issued by wave li % 16; trellis as k_fat (waves 0 .. 3); wave w decodes column
// tile w & 7 of sub-block w >> 3 in both tile rows (one 16-byte store per lane and step).
template <int MODE, int MBW, bool YH = false>
__global__ __launch_bounds__(FT16_THREADS, 1) void k_fat16(FatArgs a)
{
    constexpr int NW = 16;
    constexpr int BM = 64 * MBW;
    constexpr int NA = MODE == 0 ? 2 : 1;
    constexpr int SEG = NA * 64;
    constexpr int A_STAGE = BM * SEG;
    constexpr int NL = A_STAGE / 1024;                           // input loads of a step
    constexpr int T_SLOT = 4 * 1024;
    constexpr int B_BUF = 16 * 64 * 16;
    constexpr int A_BYTES = FT_PA * A_STAGE, T_BYTES = FT_TS * T_SLOT;
    constexpr int MAIN = A_BYTES + T_BYTES + 2 * B_BUF;
    constexpr int CS = BM + 2;
    constexpr int SMEM = MAIN > FT_BN * CS * 2 ? MAIN : FT_BN * CS * 2;
    static_assert(SMEM <= 160 * 1024, "LDS");
    static_assert(((CS / 2) & 1) == 1, "odd dword stride: conflict-free column reads");
    static_assert(NL >= 4 && NL <= 2 * NW, "the trellis loaders also load inputs; at most two input loads per wave");
    __shared__ __align__(16) uint8_t smem[SMEM];
    uint8_t* Aring = smem;
    uint8_t* Tring = smem + A_BYTES;
    uint8_t* Bdec = smem + A_BYTES + T_BYTES;

    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int nact = min(a.nactive[0], a.max_active);
    const int total = a.tile_off[nact];
    const int work = total * a.nunits, per_xcd = (work + 7) >> 3;
    const int L = (int)(blockIdx.x & 7) * per_xcd + (int)(blockIdx.x >> 3);
    if ((int)(blockIdx.x >> 3) >= per_xcd || L >= work) return;
    const int mt = L / a.nunits, nu = L % a.nunits;
    int lo = 0, hi = nact - 1;
    while (lo < hi)
    {
        const int mid = (lo + hi + 1) >> 1;
        if (a.tile_off[mid] <= mt) lo = mid; else hi = mid - 1;
    }
    const ExpertRec* rp = a.rec + lo;
    const int row0 = BM == FT_BIG ? (mt - a.tile_off[lo]) * BM : (a.big_off[lo + 1] - a.big_off[lo]) * FT_BIG;
    const int rows = __builtin_amdgcn_readfirstlane(min(BM, rp->cnt - row0));
    const int pos0 = __builtin_amdgcn_readfirstlane(rp->first + row0);
    const int e = __builtin_amdgcn_readfirstlane(rp->e);
    const int S = a.K / 32;

    auto uniform_ptr = [](const void* p) {
        const uint64_t v = (uint64_t)(uintptr_t)p;
        const uint32_t l = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)v);
        const uint32_t h = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(v >> 32));
        return reinterpret_cast<void*>((uintptr_t)((uint64_t)l | ((uint64_t)h << 32)));
    };
    const bool tloader = wave < 4;
    const int tq = wave & 3;
    const uint32_t row_bytes = (uint32_t)(a.N / 16) * 96, wbytes = (uint32_t)(a.K / 16) * row_bytes;
    const void* wbase = (const void*)(uintptr_t)(MODE == 0 ? ((tq & 1) ? rp->w[1] : rp->w[0]) : rp->w[2]);
    const __amdgpu_buffer_rsrc_t wres = __builtin_amdgcn_make_buffer_rsrc(uniform_ptr(wbase), (short)0, (int)wbytes,
                                                                          0x00020000);
    const uint32_t wcol = MODE == 0 ? (uint32_t)nu * 768 : (uint32_t)(2 * nu + (tq & 1)) * 768;
    auto load_trellis = [&](int s) {
        const uint32_t tr = (uint32_t)(2 * min(s, S - 1) + (tq >> 1));
        __builtin_amdgcn_raw_ptr_buffer_load_lds(wres, Tring + (size_t)(s % FT_TS) * T_SLOT + (size_t)tq * 1024, 12,
                                                 tr * row_bytes + wcol + (uint32_t)lane * 12, 0, 0, 0);
    };
    const uint32_t a_row = (uint32_t)NA * a.K * 2;
    const __amdgpu_buffer_rsrc_t ares = __builtin_amdgcn_make_buffer_rsrc(
        uniform_ptr(a.xa + (size_t)pos0 * NA * a.K), (short)0, (int)((uint32_t)rows * a_row), 0x00020000);
    // input load li = wave + 16 u of a step; this wave issues na of them (uniform)
    const int na = wave < NL ? (wave + NW < NL ? 2 : 1) : 0;
    auto load_input = [&](int s, int u) {
        const int st = s % FT_PA;
        const uint32_t ks = s < S ? (uint32_t)s * SEG : 0x40000000u;
        const int li = wave + NW * u;
        const int r = li * (1024 / SEG) + lane / (SEG / 16), slot = lane % (SEG / 16);
        const uint32_t voff = (uint32_t)r * a_row + (uint32_t)chunk_slot<NA>(slot, r) * 16 + ks;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(ares, Aring + (size_t)st * A_STAGE + (size_t)li * 1024, 16, voff, 0, 0, 0);
    };
    auto load_inputs = [&](int s) {
        if (na > 0) load_input(s, 0);
        if (na > 1) load_input(s, 1);
    };

    const int col = lane & 15, g = lane >> 4;
    const int i0 = 32 * (col & 7) + 8 * g + 4 * (col >> 3);
    const int eb = 3 * i0 + 11;
    const int blo = eb >> 5, bhi = (blo + 23) % 24;
    const int llo = 4 * (blo / 3) + blo % 3, lhi = 4 * (bhi / 3) + bhi % 3;
    const uint32_t sh = 31u - (uint32_t)(eb & 31);
    const int db = wave >> 3, dc = wave & 7;
    const uint32_t* tword = reinterpret_cast<const uint32_t*>(Tring + (size_t)db * 1024 + (size_t)dc * 128);
    uint8_t* bdst = Bdec + ((size_t)(db * 8 + dc) * 64 + lane) * 16;
    const int wm = wave >> 2, wn = wave & 3;
    const uint8_t* bsrc = Bdec + ((size_t)(wn * 4) * 64 + lane) * 16;
    int aoff[MBW];
#pragma unroll
    for (int i = 0; i < MBW; ++i)
    {
        const int r = 16 * (4 * i + wm) + col;
        aoff[i] = r * SEG + chunk_slot<NA>((MODE == 0 ? (wn >> 1) : 0) * 4 + g, r) * 16;
    }
    float4_t acc[MBW][4];
#pragma unroll
    for (int i = 0; i < MBW; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = float4_t{ 0.f, 0.f, 0.f, 0.f };

    // Issue order per wave: inputs of step 0, [trellis of steps 0 .. FT_PT - 1], inputs of step 1, then in step s
    // [the trellis of step s + FT_PT] and the inputs of step s + 2 ([..] = waves 0 .. 3). At the top of step s the
    // wave's inputs of step s are complete once at most na (+ 1) loads are outstanding (what step s - 1 issued
    // after them; step 0: more came after); the trellis of step s + 1 was issued before them.
    auto wait_step = [&]() {
        const int k = na + (tloader ? 1 : 0);
        if (k >= 3) wait_vmcnt<3>();
        else if (k == 2) wait_vmcnt<2>();
        else if (k == 1) wait_vmcnt<1>();
        else if (na == 0 && tloader) wait_vmcnt<FT_PT - 2>();
    };
    load_inputs(0);
    asm volatile("" ::: "memory");
    if (tloader)
        for (int s = 0; s < FT_PT; ++s) load_trellis(s);
    asm volatile("" ::: "memory");
    load_inputs(1);
    if (tloader)
    {
        if (na == 2) wait_vmcnt<2 + FT_PT - 1>();
        else wait_vmcnt<1 + FT_PT - 1>();
    }
    lds_barrier();
    {
        const half4_t r0 = decode4<true>(tword[lhi], tword[llo], sh);
        const half4_t r1 = decode4<true>(tword[512 + lhi], tword[512 + llo], sh);
        *reinterpret_cast<half8_t*>(bdst) = half8_t{ r0[0], r0[1], r0[2], r0[3], r1[0], r1[1], r1[2], r1[3] };
    }
    const int nb16 = (rows + 15) >> 4;
    const int nvb = max(0, min(MBW, (nb16 - wm + 3) >> 2));
    auto main_loop = [&](auto part_tag) {
        constexpr bool PART = decltype(part_tag)::value;
        for (int s = 0; s < S; ++s)
        {
            wait_step();
            lds_barrier();
            if (tloader) load_trellis(s + FT_PT);
            const uint32_t toff = (uint32_t)__builtin_amdgcn_readfirstlane(((s + 1) % FT_TS) * T_SLOT);
            const uint8_t* thp = reinterpret_cast<const uint8_t*>(tword + lhi) + toff;
            const uint8_t* tlp = reinterpret_cast<const uint8_t*>(tword + llo) + toff;
            const uint32_t th0 = *reinterpret_cast<const uint32_t*>(thp), tl0 = *reinterpret_cast<const uint32_t*>(tlp);
            const uint32_t th1 = *reinterpret_cast<const uint32_t*>(thp + 2048);
            const uint32_t tl1 = *reinterpret_cast<const uint32_t*>(tlp + 2048);
            const uint8_t* as = Aring + (size_t)(s % FT_PA) * A_STAGE;
            const uint8_t* bs = bsrc + (size_t)(s & 1) * B_BUF;
            uint8_t* bd = bdst + (size_t)((s + 1) & 1) * B_BUF;
            half8_t B[4], A[MBW];
#pragma unroll
            for (int j = 0; j < 4; ++j) B[j] = *reinterpret_cast<const half8_t*>(bs + j * 1024);
#pragma unroll
            for (int i = 0; i < MBW; ++i)
                if (!PART || i < nvb) A[i] = *reinterpret_cast<const half8_t*>(as + aoff[i]);
            const half4_t d0 = decode4<true>(th0, tl0, sh);
#pragma unroll
            for (int i = 0; i < MBW; ++i)
            {
                if (!PART || i < nvb)
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[i], B[j], acc[i][j], 0, 0, 0);
                if (i == 0) load_inputs(s + FT_PA - 1);
                if (i == MBW / 2 - 1)
                {
                    const half4_t d1 = decode4<true>(th1, tl1, sh);
                    *reinterpret_cast<half8_t*>(bd) = half8_t{ d0[0], d0[1], d0[2], d0[3], d1[0], d1[1], d1[2], d1[3] };
                }
            }
            if constexpr (!PART)
            {
                __builtin_amdgcn_sched_group_barrier(0x0100, 4 + MBW + 4, 0);
                __builtin_amdgcn_sched_group_barrier(0x0002, 8, 0);
#pragma unroll
                for (int k = 0; k < 4 * MBW; ++k)
                {
                    __builtin_amdgcn_sched_group_barrier(0x0008, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(0x0002, 1, 0);
                }
            }
        }
    };
    if (nvb == MBW)
        main_loop(std::false_type{});
    else
        main_loop(std::true_type{});
    wait_vmcnt<0>();
    lds_barrier();

    uint16_t* C = reinterpret_cast<uint16_t*>(smem);
#pragma unroll
    for (int i = 0; i < MBW; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
        {
            const int c = (wn * 4 + j) * 16 + col, r = 16 * (4 * i + wm) + 4 * g;
            uint32_t* d = reinterpret_cast<uint32_t*>(C + (size_t)c * CS + r);
            d[0] = (uint32_t)f2h(acc[i][j][0]) | ((uint32_t)f2h(acc[i][j][1]) << 16);
            d[1] = (uint32_t)f2h(acc[i][j][2]) | ((uint32_t)f2h(acc[i][j][3]) << 16);
        }
    __syncthreads();
    fat_tile_epilogue<MODE, CS, YH, NW>(a, C, rows, pos0, e, nu, wave, lane);
}

// Weighted combine of the fat routes: out[t] = (accumulate ? out[t] : 0) + sum_j w_j y_j over the routes j of
// token t whose expert has more than cap routes, fp32 fma in ascending j (with cap 0 this is mm_combine). The
// per-route rows y_j are fp16 (the down GEMM writes them so: its output transform rounds every value to fp16).
__global__ __launch_bounds__(256) void k_fat_combine(float* __restrict__ out, const uint16_t* __restrict__ Y,
                                                     const int64_t* __restrict__ ids, const float* __restrict__ w,
                                                     const int32_t* __restrict__ counts, int T, int k, int H, int E,
                                                     int cap, int accumulate)
{
    const int t = blockIdx.y;
    const int h = (blockIdx.x * blockDim.x + threadIdx.x) * 4;
    if (t >= T || h >= H) return;
    float4 acc = accumulate ? *reinterpret_cast<const float4*>(out + (size_t)t * H + h) : make_float4(0.f, 0.f, 0.f, 0.f);
    for (int j = 0; j < k; ++j)
    {
        const int s = t * k + j;
        const int64_t e = ids[s];
        if (e < 0 || e >= E || counts[e] <= cap) continue;
        const float wj = w[s];
        const uint2 yb = *reinterpret_cast<const uint2*>(Y + (size_t)s * H + h);
        const float4 y = make_float4(h2f((uint16_t)(yb.x & 0xffffu)), h2f((uint16_t)(yb.x >> 16)),
                                     h2f((uint16_t)(yb.y & 0xffffu)), h2f((uint16_t)(yb.y >> 16)));
        acc.x = fmaf(wj, y.x, acc.x);
        acc.y = fmaf(wj, y.y, acc.y);
        acc.z = fmaf(wj, y.z, acc.z);
        acc.w = fmaf(wj, y.w, acc.w);
    }
    *reinterpret_cast<float4*>(out + (size_t)t * H + h) = acc;
}

// ------------------------------------------------------------------------------- sorted-route form
// The reference's fat entry takes the routes already sorted by expert (token_sorted, weight_sorted and per-expert
// counts, patches/vllm-exl3-host-dma.patch:182-201). Selection, token lists and the combine of that form:

// One block: counts (effective) = counts_in[e] for experts with more than cap routes that are not skipped and whose
// range lies within the n positions, else 0; offsets = exclusive sums of counts_in (clamped to n), offsets[E] =
// the routed positions, offsets[E + 1] = n; active = the selected experts in ascending id, nactive their number.
__global__ __launch_bounds__(FT_PLAN_MAX) void k_fatb_setup(const int32_t* counts_in, const uint8_t* skip, int E, int n,
                                                           int cap, int32_t* counts, int32_t* offsets, int32_t* active,
                                                           int32_t* nactive)
{
    __shared__ int s_w[2][FT_PLAN_MAX / 64];
    const int e = threadIdx.x, lane = e & 63, wave = e >> 6;
    const int c = e < E ? max(counts_in[e], 0) : 0;
    const int ic = wave_incl_scan(c);
    if (lane == 63) s_w[0][wave] = ic;
    __syncthreads();
    int base = 0, total = 0;
    for (int w = 0; w < FT_PLAN_MAX / 64; ++w)
    {
        if (w < wave) base += s_w[0][w];
        total += s_w[0][w];
    }
    const long long off = (long long)base + ic - c;
    const bool sel = e < E && c > cap && !(skip && skip[e]) && off + c <= n;
    const int f = wave_incl_scan(sel ? 1 : 0);
    if (lane == 63) s_w[1][wave] = f;
    __syncthreads();
    int fb = 0, nf = 0;
    for (int w = 0; w < FT_PLAN_MAX / 64; ++w)
    {
        if (w < wave) fb += s_w[1][w];
        nf += s_w[1][w];
    }
    if (e < E)
    {
        offsets[e] = (int)min(off, (long long)n);
        counts[e] = sel ? c : 0;
        if (sel) active[fb + f - 1] = e;
    }
    if (e == 0)
    {
        const int routed = min(total, n);
        offsets[E] = routed;
        offsets[E + 1] = n;
        counts[E] = n - routed;
        nactive[0] = nf;
    }
}

__device__ __forceinline__ int fatb_expert(const int32_t* offsets, int E, int pos)
{
    int lo = 0, hi = E;
    while (hi - lo > 1)
    {
        const int mid = (lo + hi) >> 1;
        if (offsets[mid] <= pos) lo = mid; else hi = mid;
    }
    return lo;
}

__global__ __launch_bounds__(256) void k_fill_i32(int32_t* p, int n, int v)
{
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) p[i] = v;
}

// Per position of a selected expert: FILL = 0 counts the position's token (tcount[t]++) and writes order[pos] =
// pos (the grouped GEMM's output row); FILL = 1 appends the position to its token's list (any order within a
// token: the combine visits a list in ascending position).
template <int FILL>
__global__ __launch_bounds__(256) void k_fatb_tokens(const int64_t* token_sorted, const int32_t* counts,
                                                     const int32_t* offsets, int32_t* order, int32_t* tcount,
                                                     const int32_t* toff, int32_t* tpos, int T, int E, int n)
{
    for (int pos = blockIdx.x * blockDim.x + threadIdx.x; pos < n; pos += gridDim.x * blockDim.x)
    {
        if (FILL == 0) order[pos] = pos;
        if (pos >= offsets[E]) continue;
        const int e = fatb_expert(offsets, E, pos);
        if (counts[e] <= 0 || pos >= offsets[e] + counts[e]) continue;
        const int64_t t = token_sorted[pos];
        if (t < 0 || t >= T) continue;
        if (FILL == 0)
            atomicAdd(&tcount[t], 1);
        else
            tpos[toff[t] + atomicAdd(&tcount[t], 1)] = pos;
    }
}

// One block: toff[0 .. T] = exclusive sums of tcount[0 .. T-1] (each thread sums a contiguous chunk).
__global__ __launch_bounds__(1024) void k_scan_i32(const int32_t* tcount, int32_t* toff, int T)
{
    __shared__ int s_w[16];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int per = (T + 1023) / 1024, i0 = min(tid * per, T), i1 = min(i0 + per, T);
    int sum = 0;
    for (int i = i0; i < i1; ++i) sum += tcount[i];
    const int inc = wave_incl_scan(sum);
    if (lane == 63) s_w[wave] = inc;
    __syncthreads();
    int base = 0, total = 0;
    for (int w = 0; w < 16; ++w)
    {
        if (w < wave) base += s_w[w];
        total += s_w[w];
    }
    int run = base + inc - sum;
    for (int i = i0; i < i1; ++i)
    {
        toff[i] = run;
        run += tcount[i];
    }
    if (tid == 0) toff[T] = total;
}

// out[t] += sum over the token's selected positions p, in ascending p, of fp32(weight_sorted[p]) * Y[p] (fp32 fma).
__global__ __launch_bounds__(256) void k_fatb_combine(float* __restrict__ out, const uint16_t* __restrict__ Y,
                                                      const uint16_t* __restrict__ wsorted, const int32_t* __restrict__ toff,
                                                      const int32_t* __restrict__ tpos, int T, int H)
{
    const int t = blockIdx.y;
    const int h = (blockIdx.x * blockDim.x + threadIdx.x) * 4;
    if (t >= T || h >= H) return;
    const int b = toff[t], m = toff[t + 1] - b;
    if (m <= 0) return;
    float4 acc = *reinterpret_cast<const float4*>(out + (size_t)t * H + h);
    int prev = -1;
    for (int i = 0; i < m; ++i)
    {
        int p = 0x7fffffff;
        for (int j = 0; j < m; ++j)
        {
            const int q = tpos[b + j];
            if (q > prev && q < p) p = q;
        }
        prev = p;
        const float wj = h2f(wsorted[p]);
        const uint2 yb = *reinterpret_cast<const uint2*>(Y + (size_t)p * H + h);
        const float4 y = make_float4(h2f((uint16_t)(yb.x & 0xffffu)), h2f((uint16_t)(yb.x >> 16)),
                                     h2f((uint16_t)(yb.y & 0xffffu)), h2f((uint16_t)(yb.y >> 16)));
        acc.x = fmaf(wj, y.x, acc.x);
        acc.y = fmaf(wj, y.y, acc.y);
        acc.z = fmaf(wj, y.z, acc.z);
        acc.w = fmaf(wj, y.w, acc.w);
    }
    *reinterpret_cast<float4*>(out + (size_t)t * H + h) = acc;
}

// ------------------------------------------------------------------------------------------------- host

struct FatWs
{
    int32_t* counts;      // [E + 1]   permutation
    int32_t* offsets;     // [E + 2]
    int32_t* order;       // [n]
    int32_t* active;      // [E]
    int32_t* nactive;     // [1]
    void* pws;            // permutation workspace
    size_t pws_bytes;
    ExpertRec* rec;       // [min(n, E)]
    int32_t* off_big;     // [min(n, E) + 1]
    int32_t* off_small;   // [min(n, E) + 1]
    uint16_t* xa;         // [n][2][H]
    uint16_t* xd;         // [n][I]
    float* Y;             // [n][H]
    int32_t* e_sorted;    // [n] expert bin of each sorted position
    size_t bytes;
};

static FatWs fat_carve(void* base, int n, int E, int H, int I)
{
    auto al = [](size_t x) { return (x + 255) & ~(size_t)255; };
    const size_t na = (size_t)(n < E ? n : E);
    const size_t pwsb = mm_permute_workspace(n, E);
    constexpr int NS = 13;
    const size_t sizes[NS] = { al((size_t)(E + 1) * 4), al((size_t)(E + 2) * 4), al((size_t)n * 4), al((size_t)E * 4),
                               al(4), al(pwsb), al(na * sizeof(ExpertRec)), al((na + 1) * 4), al((na + 1) * 4),
                               al((size_t)n * 2 * H * 2), al((size_t)n * I * 2), al((size_t)n * H * 4),
                               al((size_t)n * 4) };
    char* p = static_cast<char*>(base);
    char* at[NS];
    size_t off = 0;
    for (int i = 0; i < NS; ++i)
    {
        at[i] = p ? p + off : nullptr;
        off += sizes[i];
    }
    FatWs w;
    w.counts = (int32_t*)at[0]; w.offsets = (int32_t*)at[1]; w.order = (int32_t*)at[2]; w.active = (int32_t*)at[3];
    w.nactive = (int32_t*)at[4]; w.pws = at[5]; w.pws_bytes = pwsb; w.rec = (ExpertRec*)at[6];
    w.off_big = (int32_t*)at[7]; w.off_small = (int32_t*)at[8]; w.xa = (uint16_t*)at[9]; w.xd = (uint16_t*)at[10];
    w.Y = (float*)at[11]; w.e_sorted = (int32_t*)at[12];
    w.bytes = off;
    return w;
}

static int fat_check(const mm_layer_t* L, const void* x, int x_dtype, int T, int topk, const int64_t* ids, void* ws,
                     size_t ws_bytes, const char* who, bool check_ws = true)
{
    MM_CHECK_ARG(L && L->gate_ptr && L->up_ptr && L->down_ptr && L->suh13 && L->svh13 && L->suh2 && L->svh2,
                 "%s: incomplete layer", who);
    MM_CHECK_ARG(L->E > 0 && L->E <= FT_PLAN_MAX && L->H % 256 == 0 && L->I % 128 == 0 && L->H > 0 && L->I > 0,
                 "%s: need 0 < E <= %d, H a multiple of 256 and I of 128", who, FT_PLAN_MAX);
    MM_CHECK_ARG((size_t)(L->H / 16) * (L->I / 16) * 96 < ((size_t)1 << 31), "%s: matrix larger than 2 GiB", who);
    MM_CHECK_ARG((size_t)FT_BIG * 2 * L->H * 2 < ((size_t)1 << 30), "%s: H too large", who);
    MM_CHECK_ARG(x && ids, "%s: null pointer", who);
    MM_CHECK_ARG(x_dtype == MM_DTYPE_F16 || x_dtype == MM_DTYPE_BF16 || x_dtype == MM_DTYPE_F32,
                 "%s: x_dtype must be MM_DTYPE_F16, MM_DTYPE_BF16 or MM_DTYPE_F32", who);
    MM_CHECK_ARG(T > 0 && topk > 0 && (size_t)T * topk < ((size_t)1 << 30), "%s: bad T/topk", who);
    if (!check_ws) return MM_OK;
    const size_t need = fat_carve(nullptr, T * topk, L->E, L->H, L->I).bytes;
    MM_CHECK_ARG(ws && ws_bytes >= need, "%s: workspace too small (%zu < %zu)", who, ws_bytes, need);
    return MM_OK;
}

// Plan and both GEMMs over the sorted positions in ws (counts, offsets, order, active, nactive filled): Y rows of
// every position of an active expert with more than cap routes.
static int fat_gemms(const mm_layer_t* L, int n, int cap, const FatWs& ws, hipStream_t s, bool yh)
{
    const int E = L->E, na = n < E ? n : E;
    hipLaunchKernelGGL(k_fat_plan, dim3(1), dim3(FT_PLAN_MAX), 0, s, ws.counts, ws.offsets, ws.active, ws.nactive,
                       L->gate_ptr, L->up_ptr, L->down_ptr, ws.rec, ws.off_big, ws.off_small, na, cap);
    // a 256-route tile holds more than 128 routes: at most n / 129 of them; one 128-route tile per active expert
    const int max_big = n / (FT_SMALL + 1), max_small = na;
    auto grid = [](int tiles, int units) { return dim3((unsigned)(((size_t)tiles * units + 7) & ~(size_t)7)); };    // >= 8 per_xcd
    FatArgs g{ ws.rec, ws.nactive, ws.off_big, ws.off_big, ws.xa, L->svh13, L->suh2, L->svh2, ws.order, ws.xd, ws.Y,
               L->H, L->I, L->H, L->I, L->I / 128, na, L->limit };
    FatArgs gs = g;
    gs.tile_off = ws.off_small;
    FatArgs d = g;
    d.xa = ws.xd; d.K = L->I; d.N = L->H; d.nunits = L->H / 256;
    FatArgs ds = d;
    ds.tile_off = ws.off_small;
    // gate/up: 256-route tiles on the 8-wave kernel, 128-route tiles and the down GEMM on the 16-wave kernel (same
    // bits; measured on the 16k layer: gate/up 256-route tiles equal, 128-route tiles 97 against 111 us, down
    // 2.76-2.85 against 2.92-2.94 ms)
    if (max_big > 0) hipLaunchKernelGGL((k_fat<0, FT_BIG / 32>), grid(max_big, g.nunits), dim3(FT_THREADS), 0, s, g);
    hipLaunchKernelGGL((k_fat16<0, FT_SMALL / 64>), grid(max_small, g.nunits), dim3(FT16_THREADS), 0, s, gs);
    if (yh)
    {
        if (max_big > 0)
            hipLaunchKernelGGL((k_fat16<1, FT_BIG / 64, true>), grid(max_big, d.nunits), dim3(FT16_THREADS), 0, s, d);
        hipLaunchKernelGGL((k_fat16<1, FT_SMALL / 64, true>), grid(max_small, d.nunits), dim3(FT16_THREADS), 0, s, ds);
    }
    else
    {
        if (max_big > 0)
            hipLaunchKernelGGL((k_fat16<1, FT_BIG / 64>), grid(max_big, d.nunits), dim3(FT16_THREADS), 0, s, d);
        hipLaunchKernelGGL((k_fat16<1, FT_SMALL / 64>), grid(max_small, d.nunits), dim3(FT16_THREADS), 0, s, ds);
    }
    return check_launch("fat path");
}

// Permutation, input prep, plan and both GEMMs: Y rows of every route whose expert has more than cap routes.
static int fat_run(const mm_layer_t* L, const void* x, int x_dtype, int T, int topk, const int64_t* ids, int cap,
                   const FatWs& ws, hipStream_t s, bool yh)
{
    const int n = T * topk, E = L->E;
    int rc = permute_launch(ids, nullptr, n, topk, E, ws.counts, ws.offsets, ws.order, nullptr, nullptr, nullptr,
                            ws.active, ws.nactive, ws.e_sorted, ws.pws, ws.pws_bytes, s);
    if (rc) return rc;
    hipLaunchKernelGGL(k_fat_prep, dim3(n), dim3(256), 0, s, x, x_dtype, ws.e_sorted, ws.counts, ws.offsets, ws.order,
                       L->suh13, ws.xa, topk, E, L->H, cap);
    return fat_gemms(L, n, cap, ws, s, yh);
}

// Workspace of the sorted-route form: the fat sections for n positions, then the token lists.
struct FatbWs
{
    FatWs f;
    int32_t* tcount;     // [T]
    int32_t* toff;       // [T + 1]
    int32_t* tpos;       // [n]
    size_t bytes;
};

static FatbWs fatb_carve(void* base, int n, int T, int E, int H, int I)
{
    auto al = [](size_t x) { return (x + 255) & ~(size_t)255; };
    FatbWs w;
    w.f = fat_carve(base, n, E, H, I);
    char* p = base ? static_cast<char*>(base) + w.f.bytes : nullptr;
    const size_t s0 = al((size_t)T * 4), s1 = al((size_t)(T + 1) * 4), s2 = al((size_t)n * 4);
    w.tcount = (int32_t*)p;
    w.toff = p ? (int32_t*)(p + s0) : nullptr;
    w.tpos = p ? (int32_t*)(p + s0 + s1) : nullptr;
    w.bytes = w.f.bytes + s0 + s1 + s2;
    return w;
}

// ------------------------------------------------------------------------------------ the fused-MoE call

// ids_small[s] = ids[s] when its expert has at most cap routes in the call (counts from the fat pass's
// permutation), else -1: the routes the decode path takes.
__global__ __launch_bounds__(256) void k_small_ids(const int64_t* __restrict__ ids, const int32_t* __restrict__ counts,
                                                   int n, int E, int cap, int64_t* __restrict__ ids_small)
{
    for (int s = blockIdx.x * blockDim.x + threadIdx.x; s < n; s += gridDim.x * blockDim.x)
    {
        const int64_t e = ids[s];
        ids_small[s] = (e >= 0 && e < E && counts[e] <= cap) ? e : -1;
    }
}

// Workspace of mm_fused_moe: the fat pass over all n routes, the decode path's ids and permutation, then the
// decode workspace with positions bounded by npos.
struct FusedWs
{
    FatWs fat;
    int64_t* ids_small;   // [n]
    int32_t* counts;      // [E + 1]  permutation of ids_small
    int32_t* offsets;     // [E + 2]
    int32_t* order;       // [n]
    int32_t* active;      // [E]
    int32_t* nactive;     // [1]
    void* pws;
    size_t pws_bytes;
    void* dws;            // decode workspace
    int npos;
    bool in_kernel;       // decode routing found in-kernel (n <= 1024, topk <= 16)
    size_t bytes;
};

static FusedWs fused_carve(void* base, int T, int topk, int E, int H, int I, int cap)
{
    auto al = [](size_t x) { return (x + 255) & ~(size_t)255; };
    const int n = T * topk;
    FusedWs w;
    w.fat = fat_carve(base, n, E, H, I);
    w.in_kernel = n <= 1024 && topk <= 16;
    // every decode-path expert has at most cap routes, so their positions lie below E x cap
    w.npos = w.in_kernel ? n : (int)std::min<int64_t>(n, (int64_t)E * std::max(cap, 1));
    w.pws_bytes = mm_permute_workspace(n, E);
    const size_t sizes[8] = { al((size_t)n * 8), al((size_t)(E + 1) * 4), al((size_t)(E + 2) * 4), al((size_t)n * 4),
                              al((size_t)E * 4), al(4), al(w.pws_bytes), decode_ws_bytes(n, w.npos, E, H, I) };
    char* p = base ? static_cast<char*>(base) + w.fat.bytes : nullptr;
    char* at[8];
    size_t off = 0;
    for (int i = 0; i < 8; ++i)
    {
        at[i] = p ? p + off : nullptr;
        off += sizes[i];
    }
    w.ids_small = (int64_t*)at[0]; w.counts = (int32_t*)at[1]; w.offsets = (int32_t*)at[2]; w.order = (int32_t*)at[3];
    w.active = (int32_t*)at[4]; w.nactive = (int32_t*)at[5]; w.pws = at[6]; w.dws = at[7];
    w.bytes = w.fat.bytes + off;
    return w;
}

}  // namespace mm

using namespace mm;

extern "C" {

size_t mm_fused_moe_workspace(int T, int topk, int E, int H, int I, int cap)
{
    if (T <= 0 || topk <= 0 || E <= 0 || H <= 0 || I <= 0 || cap < 0) return 0;
    return fused_carve(nullptr, T, topk, E, H, I, cap).bytes;
}

int mm_fused_moe(const mm_layer_t* L, const void* x, int x_dtype, int T, int topk, const int64_t* ids, const float* w,
                 int cap, float* out, void* workspace, size_t workspace_bytes, mm_stream_t stream)
{
    const int rc = fat_check(L, x, x_dtype, T, topk, ids, workspace, 0, "mm_fused_moe", false);
    if (rc) return rc;
    MM_CHECK_ARG(w && out && cap >= 1, "mm_fused_moe: null pointer or cap < 1");
    MM_CHECK_ARG(topk <= 16, "mm_fused_moe: topk must be at most 16");
    const int n = T * topk, E = L->E;
    const FusedWs ws = fused_carve(workspace, T, topk, E, L->H, L->I, cap);
    // the decode path's per-position inputs are addressed with 32-bit buffer offsets
    MM_CHECK_ARG((size_t)ws.npos * 2 * std::max(L->H, L->I) * 2 < ((size_t)1 << 31),
                 "mm_fused_moe: too many decode-path positions (%d)", ws.npos);
    MM_CHECK_ARG(workspace && workspace_bytes >= ws.bytes, "mm_fused_moe: workspace too small (%zu < %zu)",
                 workspace_bytes, ws.bytes);
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    // 1. experts above cap on the grouped GEMM: out = their weighted sum (every token written)
    int r = fat_run(L, x, x_dtype, T, topk, ids, cap, ws.fat, s, true);
    if (r) return r;
    const dim3 cgrid((unsigned)((L->H / 4 + 255) / 256), (unsigned)T);
    hipLaunchKernelGGL(k_fat_combine, cgrid, dim3(256), 0, s, out, reinterpret_cast<const uint16_t*>(ws.fat.Y), ids, w,
                       ws.fat.counts, T, topk, L->H, E, cap, 0);
    // 2. the others on the decode path, added per token in ascending route order
    hipLaunchKernelGGL(k_small_ids, dim3((unsigned)std::min((n + 255) / 256, 1024)), dim3(256), 0, s, ids,
                       ws.fat.counts, n, E, cap, ws.ids_small);
    if (ws.in_kernel)
        return moe_decode_launch(L, x, x_dtype, 0, T, topk, ws.ids_small, w, cap, out, ws.dws,
                                 decode_ws_bytes(n, n, E, L->H, L->I), stream, "mm_fused_moe", 1);
    r = permute_launch(ws.ids_small, nullptr, n, topk, E, ws.counts, ws.offsets, ws.order, nullptr, nullptr, nullptr,
                       ws.active, ws.nactive, nullptr, ws.pws, ws.pws_bytes, s);
    if (r) return r;
    return decode_perm_launch(L, x, x_dtype, T, topk, ws.ids_small, w, ws.offsets, ws.order, ws.active, ws.nactive,
                              ws.npos, cap, out, 1, ws.dws, s);
}

size_t mm_prefill_workspace(int n, int E, int H, int I)
{
    if (n <= 0 || E <= 0 || H <= 0 || I <= 0) return 0;
    return fat_carve(nullptr, n, E, H, I).bytes;
}

int mm_grouped_gemm(const mm_layer_t* L, const void* x, int x_dtype, int T, int topk, const int64_t* ids, int cap,
                    float* Y, void* workspace, size_t workspace_bytes, mm_stream_t stream)
{
    const int rc = fat_check(L, x, x_dtype, T, topk, ids, workspace, workspace_bytes, "mm_grouped_gemm");
    if (rc) return rc;
    MM_CHECK_ARG(Y && cap >= 0, "mm_grouped_gemm: null Y or negative cap");
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    FatWs ws = fat_carve(workspace, T * topk, L->E, L->H, L->I);
    ws.Y = Y;
    return fat_run(L, x, x_dtype, T, topk, ids, cap, ws, s, false);
}

int mm_moe_prefill(const mm_layer_t* L, const void* x, int x_dtype, int T, int topk, const int64_t* ids, const float* w,
                   int cap, int accumulate, float* out, void* workspace, size_t workspace_bytes, mm_stream_t stream)
{
    const int rc = fat_check(L, x, x_dtype, T, topk, ids, workspace, workspace_bytes, "mm_moe_prefill");
    if (rc) return rc;
    MM_CHECK_ARG(w && out && cap >= 0, "mm_moe_prefill: null pointer or negative cap");
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    const FatWs ws = fat_carve(workspace, T * topk, L->E, L->H, L->I);
    const int r = fat_run(L, x, x_dtype, T, topk, ids, cap, ws, s, true);
    if (r) return r;
    const dim3 grid((unsigned)((L->H / 4 + 255) / 256), (unsigned)T);
    hipLaunchKernelGGL(k_fat_combine, grid, dim3(256), 0, s, out, reinterpret_cast<const uint16_t*>(ws.Y), ids, w,
                       ws.counts, T, topk, L->H, L->E, cap,
                       accumulate);
    return check_launch("mm_moe_prefill");
}

size_t mm_fat_batched_workspace(int n, int T, int E, int H, int I)
{
    if (n <= 0 || T <= 0 || E <= 0 || H <= 0 || I <= 0) return 0;
    return fatb_carve(nullptr, n, T, E, H, I).bytes;
}

int mm_fat_batched(const mm_layer_t* L, const void* x, int x_dtype, int T, int n, const int64_t* token_sorted,
                   const uint16_t* weight_sorted, const int32_t* counts, const uint8_t* skip, int cap, float* out,
                   void* workspace, size_t workspace_bytes, mm_stream_t stream)
{
    MM_CHECK_ARG(n > 0, "mm_fat_batched: need n > 0 sorted positions");
    MM_CHECK_ARG(L && L->gate_ptr && L->up_ptr && L->down_ptr && L->suh13 && L->svh13 && L->suh2 && L->svh2,
                 "mm_fat_batched: incomplete layer");
    MM_CHECK_ARG(L->E > 0 && L->E <= FT_PLAN_MAX && L->H % 256 == 0 && L->I % 128 == 0 && L->H > 0 && L->I > 0,
                 "mm_fat_batched: need 0 < E <= %d, H a multiple of 256 and I of 128", FT_PLAN_MAX);
    MM_CHECK_ARG((size_t)(L->H / 16) * (L->I / 16) * 96 < ((size_t)1 << 31), "mm_fat_batched: matrix larger than 2 GiB");
    MM_CHECK_ARG(x_dtype == MM_DTYPE_F16 || x_dtype == MM_DTYPE_BF16 || x_dtype == MM_DTYPE_F32,
                 "mm_fat_batched: x_dtype must be MM_DTYPE_F16, MM_DTYPE_BF16 or MM_DTYPE_F32");
    MM_CHECK_ARG(x && token_sorted && weight_sorted && counts && out && cap >= 0, "mm_fat_batched: null pointer or negative cap");
    MM_CHECK_ARG(T > 0 && n < (1 << 30) && T < (1 << 30), "mm_fat_batched: bad T/n");
    const FatbWs ws = fatb_carve(workspace, n, T, L->E, L->H, L->I);
    MM_CHECK_ARG(workspace && workspace_bytes >= ws.bytes, "mm_fat_batched: workspace too small (%zu < %zu)",
                 workspace_bytes, ws.bytes);
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    const int E = L->E;
    const unsigned pg = (unsigned)std::min((n + 255) / 256, 4096);
    hipLaunchKernelGGL(k_fatb_setup, dim3(1), dim3(FT_PLAN_MAX), 0, s, counts, skip, E, n, cap, ws.f.counts,
                       ws.f.offsets, ws.f.active, ws.f.nactive);
    hipLaunchKernelGGL(k_fill_i32, dim3((unsigned)std::min((T + 255) / 256, 1024)), dim3(256), 0, s, ws.tcount, T, 0);
    hipLaunchKernelGGL(k_fatb_tokens<0>, dim3(pg), dim3(256), 0, s, token_sorted, ws.f.counts, ws.f.offsets, ws.f.order,
                       ws.tcount, ws.toff, ws.tpos, T, E, n);
    hipLaunchKernelGGL(k_scan_i32, dim3(1), dim3(1024), 0, s, ws.tcount, ws.toff, T);
    hipLaunchKernelGGL(k_fill_i32, dim3((unsigned)std::min((T + 255) / 256, 1024)), dim3(256), 0, s, ws.tcount, T, 0);
    hipLaunchKernelGGL(k_fatb_tokens<1>, dim3(pg), dim3(256), 0, s, token_sorted, ws.f.counts, ws.f.offsets, ws.f.order,
                       ws.tcount, ws.toff, ws.tpos, T, E, n);
    hipLaunchKernelGGL(k_fatb_prep, dim3(n), dim3(256), 0, s, x, x_dtype, token_sorted, ws.f.counts, ws.f.offsets,
                       L->suh13, ws.f.xa, T, E, L->H);
    int r = fat_gemms(L, n, cap, ws.f, s, true);
    if (r) return r;
    const dim3 grid((unsigned)((L->H / 4 + 255) / 256), (unsigned)T);
    hipLaunchKernelGGL(k_fatb_combine, grid, dim3(256), 0, s, out, reinterpret_cast<const uint16_t*>(ws.f.Y),
                       weight_sorted, ws.toff, ws.tpos, T, L->H);
    return check_launch("mm_fat_batched");
}

}  // extern "C"
