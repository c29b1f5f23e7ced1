// Routing kernels for the MI355X routed-expert MoE layer: router top-k, the decode-tier split, the host-partial
// combine, the deterministic token->expert permutation and the fixed-order weighted combine.
#include <stdarg.h>
#include <stdio.h>

#include "mm_common.h"

namespace mm {

static thread_local char g_err[512] = "";

int set_error(int code, const char* fmt, ...)
{
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return code;
}

int check_launch(const char* what)
{
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return set_error(MM_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
    return MM_OK;
}

// ---------------------------------------------------------------------------------------------------------
// Wave / block helpers
// ---------------------------------------------------------------------------------------------------------
__device__ __forceinline__ uint64_t lanemask_lt() { return (1ull << (threadIdx.x & 63)) - 1ull; }

// Lanes of this wave holding the same key (only lanes with valid set take part).
__device__ __forceinline__ uint64_t peer_mask(int key, bool valid)
{
    uint64_t todo = __ballot(valid);
    uint64_t mine = 0;
    while (todo)
    {
        const int leader = __ffsll((unsigned long long)todo) - 1;
        const int k0 = __builtin_amdgcn_readlane(key, leader);
        const uint64_t m = __ballot(valid && key == k0);
        if (valid && key == k0) mine = m;
        todo &= ~m;
    }
    return mine;
}

// Exclusive prefix sum over the threads of a block (blockDim.x a multiple of 64, <= 1024). Returns this
// thread's exclusive prefix; *total gets the block sum. Uses `scratch` (>= 16 ints of LDS).
__device__ int block_scan_excl(int v, int* scratch, int* total)
{
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    const int incl = wave_incl_scan(v);
    __syncthreads();
    if (lane == 63) scratch[wave] = incl;
    __syncthreads();
    int before = 0, all = 0;
    for (int w = 0; w < nw; ++w)
    {
        const int s = scratch[w];
        if (w < wave) before += s;
        all += s;
    }
    *total = all;
    return before + incl - v;
}

// ---------------------------------------------------------------------------------------------------------
// Router: logits = x . G^T in fp32 (64x64 tiles, fp32 FMA), then one wave per token picks the top k.
// ---------------------------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_router_logits(const uint16_t* __restrict__ x, const float* __restrict__ G,
                                                       float* __restrict__ logits, int T, int H, int E)
{
    __shared__ float As[16][64 + 1];
    __shared__ float Bs[16][64 + 1];
    const int t0 = blockIdx.y * 64, e0 = blockIdx.x * 64;
    const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
    float acc[4][4] = {};
    for (int k0 = 0; k0 < H; k0 += 16)
    {
        for (int i = threadIdx.x; i < 16 * 64; i += 256)
        {
            const int r = i / 16, kk = i % 16;
            const int tr = t0 + r, er = e0 + r;
            As[kk][r] = tr < T ? __builtin_bit_cast(float, (uint32_t)x[(size_t)tr * H + k0 + kk] << 16) : 0.0f;
            Bs[kk][r] = er < E ? G[(size_t)er * H + k0 + kk] : 0.0f;
        }
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < 16; ++kk)
        {
            float a[4], b[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) { a[i] = As[kk][ty * 4 + i]; b[i] = Bs[kk][tx * 4 + i]; }
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][j] = fmaf(a[i], b[j], acc[i][j]);
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
        {
            const int tr = t0 + ty * 4 + i, er = e0 + tx * 4 + j;
            if (tr < T && er < E) logits[(size_t)tr * E + er] = acc[i][j];
        }
}

// Decode-sized router logits: one workgroup per expert (and TB tokens), its 4 waves take interleaved 256-element
// chunks of the gate row (16-byte loads; chunk c by wave c % 4), four chunks' loads issued before any is used, the
// x rows (8-byte bf16 loads of TB tokens; they stay in L2 for every expert) with them; lane partials in fp32, a
// wave sum per token, then the 4 waves' sums added in wave order. A launch of 64 x 64 tiles would give a 4-token
// call only E / 64 workgroups, and one wave per expert walking its row chunk by chunk waits a memory round trip per
// chunk.
constexpr int RT_MAX_T = 64;

template <int TB>
__global__ __launch_bounds__(256) void k_router_gemv(const uint16_t* __restrict__ x, const float* __restrict__ G,
                                                     float* __restrict__ logits, int T, int H, int E)
{
    __shared__ float part[4][TB];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int e = blockIdx.x;
    const int t0 = blockIdx.y * TB;
    const int nt = min(TB, T - t0);
    const int nch = H / 256;
    float acc[TB];
#pragma unroll
    for (int t = 0; t < TB; ++t) acc[t] = 0.0f;
    const float4* g = reinterpret_cast<const float4*>(G + (size_t)e * H);
    auto bf = [](uint32_t b) { return __builtin_bit_cast(float, b << 16); };
    // tokens past nt read the last valid row (never stored), chunks past the row reload the last chunk (not added)
    auto xrow = [&](int t, int c) {
        return *reinterpret_cast<const uint2*>(x + (size_t)(t0 + min(t, nt - 1)) * H + (size_t)c * 256 + lane * 4);
    };
    for (int c0 = wv; c0 < nch; c0 += 16)
    {
        float4 gv[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) gv[u] = g[(size_t)min(c0 + 4 * u, nch - 1) * 64 + lane];
        if constexpr (TB <= 4)
        {
            uint2 xr[4][TB];
#pragma unroll
            for (int u = 0; u < 4; ++u)
#pragma unroll
                for (int t = 0; t < TB; ++t) xr[u][t] = xrow(t, min(c0 + 4 * u, nch - 1));
#pragma unroll
            for (int u = 0; u < 4; ++u)
                if (c0 + 4 * u < nch)
#pragma unroll
                    for (int t = 0; t < TB; ++t)
                    {
                        acc[t] = fmaf(bf(xr[u][t].x & 0xffffu), gv[u].x, acc[t]);
                        acc[t] = fmaf(bf(xr[u][t].x >> 16), gv[u].y, acc[t]);
                        acc[t] = fmaf(bf(xr[u][t].y & 0xffffu), gv[u].z, acc[t]);
                        acc[t] = fmaf(bf(xr[u][t].y >> 16), gv[u].w, acc[t]);
                    }
        }
        else
        {
#pragma unroll
            for (int u = 0; u < 4; ++u)
            {
                uint2 xr[TB];
#pragma unroll
                for (int t = 0; t < TB; ++t) xr[t] = xrow(t, min(c0 + 4 * u, nch - 1));
                if (c0 + 4 * u < nch)
#pragma unroll
                    for (int t = 0; t < TB; ++t)
                    {
                        acc[t] = fmaf(bf(xr[t].x & 0xffffu), gv[u].x, acc[t]);
                        acc[t] = fmaf(bf(xr[t].x >> 16), gv[u].y, acc[t]);
                        acc[t] = fmaf(bf(xr[t].y & 0xffffu), gv[u].z, acc[t]);
                        acc[t] = fmaf(bf(xr[t].y >> 16), gv[u].w, acc[t]);
                    }
            }
        }
    }
#pragma unroll
    for (int t = 0; t < TB; ++t)
    {
        float v = acc[t];
        v += xor_lane<32>(v);
        v += xor_lane<16>(v);
        v += xor_lane<8>(v);
        v += xor_lane<4>(v);
        v += xor_lane<2>(v);
        v += xor_lane<1>(v);
        if (lane == 0) part[wv][t] = v;
    }
    __syncthreads();
    if (wv == 0 && lane < nt)
        logits[(size_t)(t0 + lane) * E + e] = ((part[0][lane] + part[1][lane]) + part[2][lane]) + part[3][lane];
}

// Prefill-sized router logits on MFMA (v_mfma_f32_16x16x32_bf16). The fp32 gate is split exactly into three bf16
// parts, g = g1 + g2 + g3: g1 is g with its low 16 bits cleared (its top 8 significant bits), g2 the same of the
// exact remainder g - g1, and g3 = g - g1 - g2, which has at most 8 significant bits; each product of a bf16 input
// with a part is exact in fp32, so the MFMA's fp32 accumulation is the only rounding, as in an fp32 dot product
// (in another order). A workgroup of WM x WN waves computes TM tokens x TN experts: per 32-row step the input tile
// and the gate tile (split into the three bf16 planes on the way into LDS) are staged, the next step's loads are in
// flight during the multiplies; wave (wm, wn) takes tokens TM / WM wm .. and experts TN / WN wn ... The launch uses
// 128 tokens x 192 experts on 8 waves (2 x 6 tiles x 3 parts per wave): each gate element is split once per 128
// tokens, and 16,384 tokens x 384 experts are 256 workgroups, one per CU (router call at that size: 64 x 128 on 4
// waves 233-242 us, this shape 201-210 us; two LDS stages with one barrier per step 220-222 us).
constexpr int RM_TM = 128, RM_TN = 192, RM_WM = 4, RM_WN = 2, RM_K = 32;
constexpr int RM_ROW = 32;            // LDS row: 32 bf16 = four 16-byte chunks, chunk q of row r stored at q ^ ((r >> 2) & 3)
// The swizzle puts the 16 rows of an operand read (one chunk each) and the 16 chunks of four rows that 16 lanes
// write in 16 distinct 16-byte bank groups (the padded 80-byte rows read conflict-free but wrote with conflicts:
// 36 % of the kernel's LDS cycles).
__device__ __forceinline__ int rm_at(int r, int q) { return r * RM_ROW + 8 * (q ^ ((r >> 2) & 3)); }
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float rm_f4_t __attribute__((ext_vector_type(4)));

template <int TM, int TN, int WM, int WN>
__global__ __launch_bounds__(64 * WM * WN) void k_router_mfma(const uint16_t* __restrict__ x, const float* __restrict__ G,
                                                              float* __restrict__ logits, int T, int H, int E)
{
    constexpr int NT = 64 * WM * WN;                        // threads
    constexpr int MI = TM / WM / 16, NJ = TN / WN / 16;      // 16 x 16 tiles per wave
    constexpr int XL = 4 * TM / NT, GL = 8 * TN / NT;        // 16-byte loads per thread and step
    static_assert(MI * WM * 16 == TM && NJ * WN * 16 == TN && XL * NT == 4 * TM && GL * NT == 8 * TN, "tile shape");
    __shared__ __align__(16) uint16_t xs[TM * RM_ROW];
    __shared__ __align__(16) uint16_t gs[3][TN * RM_ROW];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int t0 = blockIdx.y * TM, e0 = blockIdx.x * TN;
    const int wm = wave / WN, wn = wave % WN;
    // this thread's loads of a step: XL 16-byte chunks of the input tile (TM rows x 4 chunks), GL of the gate tile
    // (TN rows x 8 chunks of 4 floats); rows past T or E load zeros
    int xr[XL], xq[XL];
    bool xin[XL];
    const uint16_t* xp[XL];
#pragma unroll
    for (int j = 0; j < XL; ++j)
    {
        const int c = tid + NT * j;
        xr[j] = c >> 2;
        xq[j] = c & 3;
        xin[j] = t0 + xr[j] < T;
        xp[j] = x + (size_t)min(t0 + xr[j], T - 1) * H + 8 * xq[j];
    }
    int gr[GL], gq[GL];
    bool gin[GL];
    const float* gp[GL];
#pragma unroll
    for (int j = 0; j < GL; ++j)
    {
        const int c = tid + NT * j;
        gr[j] = c >> 3;
        gq[j] = c & 7;
        gin[j] = e0 + gr[j] < E;
        gp[j] = G + (size_t)min(e0 + gr[j], E - 1) * H + 4 * gq[j];
    }
    uint4 xv[XL];
    float4 gv[GL];
    auto load = [&](int k0) {
#pragma unroll
        for (int j = 0; j < XL; ++j) xv[j] = xin[j] ? *reinterpret_cast<const uint4*>(xp[j] + k0) : make_uint4(0, 0, 0, 0);
#pragma unroll
        for (int j = 0; j < GL; ++j) gv[j] = gin[j] ? *reinterpret_cast<const float4*>(gp[j] + k0) : make_float4(0, 0, 0, 0);
    };
    auto split = [](float g, uint32_t& a, uint32_t& b, uint32_t& c) {
        const uint32_t h1 = __float_as_uint(g) & 0xffff0000u;
        const float r1 = g - __uint_as_float(h1);
        const uint32_t h2 = __float_as_uint(r1) & 0xffff0000u;
        const float r2 = r1 - __uint_as_float(h2);
        a = h1 >> 16;
        b = h2 >> 16;
        c = __float_as_uint(r2) >> 16;
    };
    rm_f4_t acc[MI][NJ];
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < NJ; ++j) acc[i][j] = rm_f4_t{ 0.f, 0.f, 0.f, 0.f };
    const int S = H / RM_K;
    load(0);
    for (int s = 0; s < S; ++s)
    {
        __syncthreads();                                       // the previous step's operand reads are done
#pragma unroll
        for (int j = 0; j < XL; ++j) *reinterpret_cast<uint4*>(&xs[rm_at(xr[j], xq[j])]) = xv[j];
#pragma unroll
        for (int j = 0; j < GL; ++j)
        {
            uint32_t a[4], b[4], c[4];
            split(gv[j].x, a[0], b[0], c[0]);
            split(gv[j].y, a[1], b[1], c[1]);
            split(gv[j].z, a[2], b[2], c[2]);
            split(gv[j].w, a[3], b[3], c[3]);
            const int o = rm_at(gr[j], gq[j] >> 1) + 4 * (gq[j] & 1);
            *reinterpret_cast<uint2*>(&gs[0][o]) = make_uint2(a[0] | (a[1] << 16), a[2] | (a[3] << 16));
            *reinterpret_cast<uint2*>(&gs[1][o]) = make_uint2(b[0] | (b[1] << 16), b[2] | (b[3] << 16));
            *reinterpret_cast<uint2*>(&gs[2][o]) = make_uint2(c[0] | (c[1] << 16), c[2] | (c[3] << 16));
        }
        __syncthreads();
        if (s + 1 < S) load((s + 1) * RM_K);
        bf16x8_t A[MI], B[3][NJ];
#pragma unroll
        for (int i = 0; i < MI; ++i)
            A[i] = *reinterpret_cast<const bf16x8_t*>(&xs[rm_at(16 * (MI * wm + i) + (lane & 15), lane >> 4)]);
#pragma unroll
        for (int p = 0; p < 3; ++p)
#pragma unroll
            for (int j = 0; j < NJ; ++j)
                B[p][j] = *reinterpret_cast<const bf16x8_t*>(&gs[p][rm_at(16 * (NJ * wn + j) + (lane & 15), lane >> 4)]);
#pragma unroll
        for (int p = 0; p < 3; ++p)
#pragma unroll
            for (int i = 0; i < MI; ++i)
#pragma unroll
                for (int j = 0; j < NJ; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[i], B[p][j], acc[i][j], 0, 0, 0);
    }
    // D: lane (column l & 15, group l >> 4) holds rows 4 g .. 4 g + 3 of its column of each tile
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < NJ; ++j)
        {
            const int e = e0 + 16 * (NJ * wn + j) + (lane & 15);
#pragma unroll
            for (int r = 0; r < 4; ++r)
            {
                const int t = t0 + 16 * (MI * wm + i) + 4 * (lane >> 4) + r;
                if (t < T && e < E) logits[(size_t)t * E + e] = acc[i][j][r];
            }
        }
}

// One wave per token: k rounds of a wave-wide argmax (ties to the lower index), then softmax over the picks.
__global__ __launch_bounds__(256) void k_router_topk(const float* __restrict__ logits, int T, int E, int k,
                                                     int64_t* __restrict__ ids, float* __restrict__ w)
{
    const int lane = threadIdx.x & 63;
    const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (t >= T) return;
    float v[16];
    uint32_t taken = 0;
    const float* row = logits + (size_t)t * E;
#pragma unroll
    for (int i = 0; i < 16; ++i)
    {
        const int e = lane + 64 * i;
        v[i] = e < E ? row[e] : -INFINITY;
        if (e >= E) taken |= 1u << i;
    }
    float sel_v[32];
    int sel_e[32];
    for (int r = 0; r < k; ++r)
    {
        float bv = -INFINITY;
        int be = 0x7fffffff;
#pragma unroll
        for (int i = 0; i < 16; ++i)
            if (!(taken & (1u << i)) && (v[i] > bv || (v[i] == bv && lane + 64 * i < be))) { bv = v[i]; be = lane + 64 * i; }
        // max (value, then lower index) over the wave, distances 32, 16, ..., 1
        auto pick = [&](float ov, int oe) {
            if (ov > bv || (ov == bv && oe < be)) { bv = ov; be = oe; }
        };
        pick(xor_lane<32>(bv), xor_lane_i<32>(be));
        pick(xor_lane<16>(bv), xor_lane_i<16>(be));
        pick(xor_lane<8>(bv), xor_lane_i<8>(be));
        pick(xor_lane<4>(bv), xor_lane_i<4>(be));
        pick(xor_lane<2>(bv), xor_lane_i<2>(be));
        pick(xor_lane<1>(bv), xor_lane_i<1>(be));
        if ((be & 63) == lane) taken |= 1u << (be >> 6);
        sel_v[r] = bv;
        sel_e[r] = be;
    }
    if (lane == 0)
    {
        const float m = sel_v[0];
        float den = 0.0f;
        for (int r = 0; r < k; ++r) den += expf(sel_v[r] - m);
        for (int r = 0; r < k; ++r)
        {
            ids[(size_t)t * k + r] = sel_e[r];
            w[(size_t)t * k + r] = expf(sel_v[r] - m) / den;
        }
    }
}

// Top-k for E <= 64 NV: each lane sorts its NV logits (experts lane + 64 i) once, descending by (value, lower
// index), and keeps them as a queue; a round is a wave-wide max of the lanes' queue heads (6 exchange stages, ties
// to the lower index) and the winning lane pops its head. Round r's pick is kept by lane r, so the softmax runs
// on k lanes at once: exp(v - max) per lane, a wave sum, and each lane writes its id and weight. Same picks, order
// and weights as k_router_topk.
template <int NV>
__global__ __launch_bounds__(256) void k_router_topk_q(const float* __restrict__ logits, int T, int E, int k,
                                                       int64_t* __restrict__ ids, float* __restrict__ w)
{
    const int lane = threadIdx.x & 63;
    const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (t >= T) return;
    const float* row = logits + (size_t)t * E;
    float qv[NV];
    int qe[NV];
#pragma unroll
    for (int i = 0; i < NV; ++i)
    {
        const int e = lane + 64 * i;
        qv[i] = e < E ? row[e] : -INFINITY;
        qe[i] = e < E ? e : 0x7fffffff;
    }
    // insertion sort of the lane's NV entries: (a before b) iff a.v > b.v or (equal and a.e < b.e)
#pragma unroll
    for (int i = 1; i < NV; ++i)
#pragma unroll
        for (int j = i; j > 0; --j)
        {
            const bool sw = qv[j] > qv[j - 1] || (qv[j] == qv[j - 1] && qe[j] < qe[j - 1]);
            const float tv = qv[j];
            const int te = qe[j];
            qv[j] = sw ? qv[j - 1] : tv;
            qe[j] = sw ? qe[j - 1] : te;
            qv[j - 1] = sw ? tv : qv[j - 1];
            qe[j - 1] = sw ? te : qe[j - 1];
        }
    float myv = -INFINITY;
    int mye = 0;
    for (int r = 0; r < k; ++r)
    {
        float bv = qv[0];
        int be = qe[0];
        auto pick = [&](float ov, int oe) {
            if (ov > bv || (ov == bv && oe < be)) { bv = ov; be = oe; }
        };
        pick(xor_lane<32>(bv), xor_lane_i<32>(be));
        pick(xor_lane<16>(bv), xor_lane_i<16>(be));
        pick(xor_lane<8>(bv), xor_lane_i<8>(be));
        pick(xor_lane<4>(bv), xor_lane_i<4>(be));
        pick(xor_lane<2>(bv), xor_lane_i<2>(be));
        pick(xor_lane<1>(bv), xor_lane_i<1>(be));
        if (be == qe[0])                                  // this lane's head won: pop it
        {
#pragma unroll
            for (int i = 0; i + 1 < NV; ++i)
            {
                qv[i] = qv[i + 1];
                qe[i] = qe[i + 1];
            }
            qv[NV - 1] = -INFINITY;
            qe[NV - 1] = 0x7fffffff;
        }
        if (lane == r)
        {
            myv = bv;
            mye = be;
        }
    }
    // the first pick is the row's maximum; lanes k .. 63 contribute 0 to the sum
    const float m = __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, myv)));
    const float z = lane < k ? expf(myv - m) : 0.0f;
    // den = ((0 + z_0) + z_1) + ... in pick order, on every lane
    float den = 0.0f;
    for (int r = 0; r < k; ++r) den += __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, z), r));
    if (lane < k)
    {
        ids[(size_t)t * k + lane] = mye;
        w[(size_t)t * k + lane] = z / den;
    }
}

// ---------------------------------------------------------------------------------------------------------
// Decode-tier split (ct/ft_tier_cu_v.cu:16-101). One block of 256 threads: LDS histogram, ballot/scan for
// the hit and miss lists and the CPU pick list, stable rank sort of misses by score, serial cost model in
// lane 0 with the reference's operation order.
// ---------------------------------------------------------------------------------------------------------
struct SplitArgs
{
    const int64_t* sel; const float* w; const uint16_t* z; int n, bsz, topk, H, E;
    const int32_t* slotof; const float* score; const float* p;
    int64_t* ctrl; uint16_t* hx; int32_t* hpicks; int64_t* seqc; int li;
    int64_t* sel_out; float* w_out; int64_t* dflag; int64_t* stats; int32_t* counts;
    int32_t* hits; int32_t* misses; int32_t* nhnm;
};

__global__ __launch_bounds__(256) void k_split(SplitArgs a)
{
    __shared__ int cnt[1024];
    __shared__ int missA[1024];   // misses in ascending id
    __shared__ int miss[1024];    // misses stable-sorted by score
    __shared__ float mkey[1024];  // score of missA[i]
    __shared__ int s_slot[1024];  // slotof[e] >= 0
    __shared__ float s_score[1024];
    __shared__ unsigned char cpu[1024];
    __shared__ int scan_tmp[16];
    __shared__ int s_nh, s_nm, s_best, s_publish, s_npk;
    __shared__ long long s_seq;
    const int t = threadIdx.x, E = a.E;
    // every global input is loaded up front (one round trip): the slot table and scores into LDS, this thread's
    // routes t + 256 k (the first SPT of them kept in registers), and the policy words and counters thread 0 uses
    for (int e = t; e < E; e += blockDim.x)
    {
        cnt[e] = 0;
        cpu[e] = 0;
        s_slot[e] = a.slotof[e] >= 0 ? 1 : 0;
        s_score[e] = a.score[e];
    }
    constexpr int SPT = 4;
    int64_t re[SPT];
    float rw[SPT];
#pragma unroll
    for (int k = 0; k < SPT; ++k)
    {
        re[k] = -1;
        rw[k] = 0.0f;
    }
    if (a.n > 0)
#pragma unroll
        for (int k = 0; k < SPT; ++k)
        {
            const int s = min(t + 256 * k, a.n - 1);        // routes past n reload route n - 1 (not used)
            re[k] = a.sel[s];
            rw[k] = a.w[s];
        }
    float pol[9] = {};
    int64_t st[4] = {}, sq = 0;
    if (t == 0)
    {
#pragma unroll
        for (int i = 0; i < 9; ++i) pol[i] = a.p[i];
#pragma unroll
        for (int i = 0; i < 4; ++i) st[i] = a.stats[i];
        sq = a.seqc[0];
    }
    __syncthreads();
    auto count_route = [&](int64_t e, float wt) {
        if (wt != 0.0f && e >= 0 && e < E)
        {
            atomicAdd(&cnt[e], 1);
            if (a.counts) atomicAdd(&a.counts[e], 1);
        }
    };
#pragma unroll
    for (int k = 0; k < SPT; ++k)
        if (t + 256 * k < a.n) count_route(re[k], rw[k]);
    for (int s = t + 256 * SPT; s < a.n; s += 256) count_route(a.sel[s], a.w[s]);
    __syncthreads();
    // hit list and miss list in ascending expert id
    int nh = 0, nm = 0;
    for (int base = 0; base < E; base += blockDim.x)
    {
        const int e = base + t;
        const bool touched = e < E && cnt[e] > 0;
        const bool hit = touched && s_slot[e] != 0, mis = touched && !hit;
        int th, tm;
        const int ph = block_scan_excl(hit ? 1 : 0, scan_tmp, &th);
        const int pm = block_scan_excl(mis ? 1 : 0, scan_tmp + 0, &tm);
        if (hit && a.hits) a.hits[nh + ph] = e;
        if (mis) missA[nm + pm] = e;
        nh += th;
        nm += tm;
    }
    __syncthreads();
    // stable sort of misses by score: rank = #smaller + #equal earlier (keys staged in LDS with one load each)
    for (int i = t; i < nm; i += blockDim.x) mkey[i] = s_score[missA[i]];
    __syncthreads();
    for (int i = t; i < nm; i += blockDim.x)
    {
        const float key = mkey[i];
        int r = 0;
        for (int m = 0; m < nm; ++m)
        {
            const float km = mkey[m];
            r += (km < key) || (km == key && m < i);
        }
        miss[r] = missA[i];
    }
    __syncthreads();
    if (t == 0)
    {
        const float* p = pol;
        int best = 0;
        const int force = (int)p[6];
        const int maxc = min((int)p[5], nm);
        if (force >= 0) best = min(force, nm);
        else
        {
            float bt = 1e30f, c = 0.0f;
            for (int k = 0; k <= maxc; ++k)
            {
                if (k) c = fmaf(p[3], fmaf(p[4], (float)(cnt[miss[k - 1]] - 1), 1.0f), c);
                const float gpu = fmaf(p[1], (float)(nh + nm - k), p[0] * (float)(nm - k));
                const float tt = fmaxf(gpu, k ? p[2] + c : 0.0f);
                if (tt < bt - 1e-6f) { bt = tt; best = k; }
            }
        }
        for (int k = 0; k < best; ++k) cpu[miss[k]] = 1;
        const int publish = best > 0 || p[7] > 0.5f;
        a.stats[0] = st[0] + nh;
        a.stats[1] = st[1] + nm;
        a.stats[2] = st[2] + best;
        a.stats[3] = st[3] + 1;
        if (publish) a.seqc[0] = sq + 1;
        s_seq = publish ? sq + 1 : 0;
        s_best = best;
        s_publish = publish;
        s_nh = nh;
        s_nm = nm;
        if (a.nhnm) { a.nhnm[0] = nh; a.nhnm[1] = nm; }
    }
    __syncthreads();
    for (int i = t; i < nm; i += blockDim.x)
        if (a.misses) a.misses[i] = miss[i];
    const int publish = s_publish;
    // CPU picks in ascending route index, then the masked selection
    int npk = 0;
    auto pick_pass = [&](int base, int64_t e, float wt) {
        const int s = base + t;
        const bool in = s < a.n;
        const bool pick = in && e >= 0 && e < E && cpu[e] && wt != 0.0f;
        int tot;
        const int pos = block_scan_excl(pick ? 1 : 0, scan_tmp, &tot);
        if (publish && pick)
        {
            int32_t* hp = a.hpicks + (size_t)(npk + pos) * 3;
            __hip_atomic_store(hp + 0, s / a.topk, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
            __hip_atomic_store(hp + 1, (int32_t)e, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
            __hip_atomic_store(hp + 2, __float_as_int(wt), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        }
        npk += tot;
        if (in)
        {
            const bool c = e >= 0 && e < E && cpu[e];
            a.sel_out[s] = c ? -1 : e;
            a.w_out[s] = c ? 0.0f : wt;
        }
    };
#pragma unroll
    for (int k = 0; k < SPT; ++k)
        if (256 * k < a.n) pick_pass(256 * k, re[k], rw[k]);
    for (int base = 256 * SPT; base < a.n; base += 256)
    {
        const int s = base + t;
        pick_pass(base, s < a.n ? a.sel[s] : -1, s < a.n ? a.w[s] : 0.0f);
    }
    if (publish)
    {
        // the payload (x rows, picks, job words), one system fence per thread, then the sequence word: the host
        // sees ctrl[0] = seq only after everything it describes (ct/ft_tier_cu_v.cu:85-98)
        const int nx = a.p[8] > 0.5f ? 0 : a.bsz * a.H / 8;
        const int4* src = reinterpret_cast<const int4*>(a.z);
        int4* dst = reinterpret_cast<int4*>(a.hx);
        for (int i = t; i < nx; i += blockDim.x) dst[i] = src[i];
        if (t == 0)
        {
            __hip_atomic_store(&a.ctrl[2], (int64_t)a.li, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
            __hip_atomic_store(&a.ctrl[3], (int64_t)a.bsz, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
            __hip_atomic_store(&a.ctrl[4], (int64_t)npk, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        }
        __threadfence_system();
        __syncthreads();
        if (t == 0)
        {
            __hip_atomic_store(&a.ctrl[0], (int64_t)s_seq, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
            a.dflag[0] = s_seq;
        }
    }
    else if (t == 0)
        a.dflag[0] = 0;
}

// ---------------------------------------------------------------------------------------------------------
// Host-partial add (ct/ft_tier_cu_v.cu:103-127): bounded wait on the host's done word, then out += hout.
// The decision is taken once, by the one-lane wait kernel: on a timeout it clears dflag[0], so the add kernel
// (every workgroup of it) either adds the whole partial or none of it. The reference lets each of its 16
// workgroups wait and decide on its own, which can add part of a partial that lands near the deadline.
// ---------------------------------------------------------------------------------------------------------
__global__ __launch_bounds__(64) void k_host_wait(int64_t* __restrict__ dflag, int64_t* ctrl, int64_t* stats,
                                                  uint64_t timeout_ticks, double ns_per_tick)
{
    if (threadIdx.x != 0) return;
    const int64_t s = dflag[0];
    if (s == 0) return;
    const uint64_t t0 = wall_clock64();
    uint64_t t1 = t0;
    while (__hip_atomic_load(&ctrl[1], __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_SYSTEM) < s)
    {
        t1 = wall_clock64();
        if (t1 - t0 > timeout_ticks)
        {
            dflag[0] = 0;                     // the partial is dropped
            atomicAdd((unsigned long long*)&stats[6], 1ull);
            break;
        }
        __builtin_amdgcn_s_sleep(2);
    }
    atomicAdd((unsigned long long*)&stats[4], (unsigned long long)((double)(t1 - t0) * ns_per_tick));
    atomicAdd((unsigned long long*)&stats[5], 1ull);
}

__global__ __launch_bounds__(256) void k_host_add(float* __restrict__ out, int n, const int64_t* __restrict__ dflag,
                                                  const float* hout)
{
    if (dflag[0] == 0) return;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x)
        out[i] += __hip_atomic_load(hout + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

// ---------------------------------------------------------------------------------------------------------
// Permutation: stable counting sort of routes by expert (sentinel E last).
// ---------------------------------------------------------------------------------------------------------
constexpr int PERM_THREADS = 1024;
constexpr int PERM_SINGLE_MAX = 8192;      // one-block path up to this many routes
constexpr int PERM_CHUNK = 4096;           // routes per block on the multi-block path

__device__ __forceinline__ int route_bin(const int64_t* ids, int s, int E)
{
    const int64_t e = ids[s];
    return (e >= 0 && e < E) ? (int)e : E;
}

// Scatter routes [lo, hi) in order; fill[] (LDS) holds the next free sorted position of every bin.
__device__ void scatter_chunk(const int64_t* ids, const float* w, int lo, int hi, int topk, int E, int* fill,
                              int32_t* order, int32_t* token_sorted, float* weight_sorted, int32_t* inv_order,
                              int32_t* e_sorted)
{
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    for (int base = lo; base < hi; base += blockDim.x)
    {
        const int s = base + threadIdx.x;
        const bool valid = s < hi;
        const int e = valid ? route_bin(ids, s, E) : -1;
        const uint64_t peers = peer_mask(e, valid);
        const int rank = __popcll(peers & lanemask_lt());
        const int grp = __popcll(peers);
        int pos = 0;
        const int waves_here = min(nw, (hi - base + 63) / 64);
        for (int w = 0; w < waves_here; ++w)
        {
            if (wave == w && valid)
            {
                const int b = fill[e];
                pos = b + rank;
                if (rank == 0) fill[e] = b + grp;
            }
            __syncthreads();
        }
        if (valid)
        {
            order[pos] = s;
            if (token_sorted) token_sorted[pos] = s / topk;
            if (weight_sorted && w) weight_sorted[pos] = w[s];
            if (inv_order) inv_order[s] = pos;
            if (e_sorted) e_sorted[pos] = e;
        }
        (void)lane;
    }
}

// Active expert list (count > 0, ascending id, sentinel excluded).
__device__ void write_active(const int* cnt, int E, int32_t* active, int32_t* nactive, int* scan_tmp)
{
    int na = 0;
    for (int base = 0; base < E; base += blockDim.x)
    {
        const int e = base + threadIdx.x;
        const bool on = e < E && cnt[e] > 0;
        int tot;
        const int pos = block_scan_excl(on ? 1 : 0, scan_tmp, &tot);
        if (on && active) active[na + pos] = e;
        na += tot;
    }
    if (threadIdx.x == 0 && nactive) nactive[0] = na;
}

__global__ __launch_bounds__(PERM_THREADS) void k_permute_single(const int64_t* __restrict__ ids, const float* __restrict__ w,
    int n, int topk, int E, int32_t* counts, int32_t* offsets, int32_t* order, int32_t* token_sorted,
    float* weight_sorted, int32_t* inv_order, int32_t* active, int32_t* nactive, int32_t* e_sorted)
{
    __shared__ int cnt[1025 + 1];
    __shared__ int fill[1025 + 1];
    __shared__ int scan_tmp[16];
    const int nb = E + 1;
    for (int e = threadIdx.x; e < nb; e += blockDim.x) cnt[e] = 0;
    __syncthreads();
    for (int s = threadIdx.x; s < n; s += blockDim.x) atomicAdd(&cnt[route_bin(ids, s, E)], 1);
    __syncthreads();
    int run = 0;
    for (int base = 0; base < nb; base += blockDim.x)
    {
        const int e = base + threadIdx.x;
        const int c = e < nb ? cnt[e] : 0;
        int tot;
        const int pre = block_scan_excl(c, scan_tmp, &tot);
        if (e < nb)
        {
            fill[e] = run + pre;
            counts[e] = c;
            offsets[e] = run + pre;
        }
        run += tot;
    }
    if (threadIdx.x == 0) offsets[nb] = run;
    write_active(cnt, E, active, nactive, scan_tmp);
    __syncthreads();
    scatter_chunk(ids, w, 0, n, topk, E, fill, order, token_sorted, weight_sorted, inv_order, e_sorted);
}

// Multi-block path: per-block bin histograms (bin-major), one-block scan, then per-block stable scatter.
__global__ __launch_bounds__(PERM_THREADS) void k_permute_hist(const int64_t* __restrict__ ids, int n, int E, int chunk,
                                                               int32_t* __restrict__ hist)
{
    __shared__ int cnt[1025 + 1];
    const int nb = E + 1, B = gridDim.x, b = blockIdx.x;
    for (int e = threadIdx.x; e < nb; e += blockDim.x) cnt[e] = 0;
    __syncthreads();
    const int lo = b * chunk, hi = min(n, lo + chunk);
    for (int s = lo + threadIdx.x; s < hi; s += blockDim.x) atomicAdd(&cnt[route_bin(ids, s, E)], 1);
    __syncthreads();
    for (int e = threadIdx.x; e < nb; e += blockDim.x) hist[(size_t)e * B + b] = cnt[e];
}

__global__ __launch_bounds__(PERM_THREADS) void k_permute_scan(int32_t* hist, int B, int n, int E, int32_t* counts,
    int32_t* offsets, int32_t* active, int32_t* nactive)
{
    __shared__ int scan_tmp[16];
    __shared__ int cnt[1025 + 1];
    const int nb = E + 1;
    const long long M = (long long)nb * B;
    const long long per = (M + blockDim.x - 1) / blockDim.x;
    const long long lo = per * threadIdx.x, hi = min(M, lo + per);
    int sum = 0;
    for (long long i = lo; i < hi; ++i) sum += hist[i];
    int tot;
    int run = block_scan_excl(sum, scan_tmp, &tot);
    for (long long i = lo; i < hi; ++i)
    {
        const int c = hist[i];
        hist[i] = run;
        run += c;
    }
    __syncthreads();
    for (int e = threadIdx.x; e < nb; e += blockDim.x)
    {
        const int start = hist[(size_t)e * B];
        const int end = e + 1 < nb ? hist[(size_t)(e + 1) * B] : n;
        counts[e] = end - start;
        offsets[e] = start;
        cnt[e] = end - start;
    }
    if (threadIdx.x == 0) offsets[nb] = n;
    __syncthreads();
    write_active(cnt, E, active, nactive, scan_tmp);
}

__global__ __launch_bounds__(PERM_THREADS) void k_permute_scatter(const int64_t* __restrict__ ids, const float* __restrict__ w,
    int n, int topk, int E, int chunk, const int32_t* __restrict__ hist, int32_t* order, int32_t* token_sorted,
    float* weight_sorted, int32_t* inv_order, int32_t* e_sorted)
{
    __shared__ int fill[1025 + 1];
    const int nb = E + 1, B = gridDim.x, b = blockIdx.x;
    for (int e = threadIdx.x; e < nb; e += blockDim.x) fill[e] = hist[(size_t)e * B + b];
    __syncthreads();
    const int lo = b * chunk, hi = min(n, lo + chunk);
    scatter_chunk(ids, w, lo, hi, topk, E, fill, order, token_sorted, weight_sorted, inv_order, e_sorted);
}

// ---------------------------------------------------------------------------------------------------------
// Fixed-order weighted combine: out[t] (+)= sum_j w[t,j] * Y[t*k+j], fp32 fma in ascending j.
// ---------------------------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_combine(float* __restrict__ out, const float* __restrict__ Y,
                                                 const int64_t* __restrict__ ids, const float* __restrict__ w, int T,
                                                 int k, int H, int E, int accumulate)
{
    const int t = blockIdx.y;
    const int h = (blockIdx.x * blockDim.x + threadIdx.x) * 4;
    if (t >= T || h >= H) return;
    float4 acc = accumulate ? *reinterpret_cast<const float4*>(out + (size_t)t * H + h) : make_float4(0.f, 0.f, 0.f, 0.f);
    for (int j = 0; j < k; ++j)
    {
        const int s = t * k + j;
        const int64_t e = ids[s];
        if (e < 0 || e >= E) continue;
        const float wj = w[s];
        const float4 y = *reinterpret_cast<const float4*>(Y + (size_t)s * H + h);
        acc.x = fmaf(wj, y.x, acc.x);
        acc.y = fmaf(wj, y.y, acc.y);
        acc.z = fmaf(wj, y.z, acc.z);
        acc.w = fmaf(wj, y.w, acc.w);
    }
    *reinterpret_cast<float4*>(out + (size_t)t * H + h) = acc;
}

// ---------------------------------------------------------------------------------------------------------
// Expert input: fp32 -> (optional unit-RMS rescale) -> bf16 (RNE) -> fp16.
// ---------------------------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_prepare_input(const float* __restrict__ x, int H, int rescale,
                                                       uint16_t* __restrict__ xb, uint16_t* __restrict__ xh)
{
    __shared__ float red[4];
    const int t = blockIdx.x;
    const float* row = x + (size_t)t * H;
    float scale = 1.0f;
    if (rescale)
    {
        // h = thread, + blockDim, ... in order; eight loads in flight before they are used
        float ss = 0.0f;
        for (int hb = threadIdx.x; hb < H; hb += blockDim.x * 8)
        {
            float v[8];
#pragma unroll
            for (int k = 0; k < 8; ++k) v[k] = row[min(hb + (int)blockDim.x * k, H - 1)];
#pragma unroll
            for (int k = 0; k < 8; ++k)
                if (hb + (int)blockDim.x * k < H) ss = fmaf(v[k], v[k], ss);
        }
        ss += xor_lane<32>(ss);
        ss += xor_lane<16>(ss);
        ss += xor_lane<8>(ss);
        ss += xor_lane<4>(ss);
        ss += xor_lane<2>(ss);
        ss += xor_lane<1>(ss);
        if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
        __syncthreads();
        const float tot = (red[0] + red[1]) + (red[2] + red[3]);
        scale = tot > 0.0f ? 1.0f / sqrtf(tot / (float)H) : 1.0f;
    }
    for (int h = threadIdx.x; h < H; h += blockDim.x)
    {
        const uint16_t b = f2bf(row[h] * scale);
        if (xb) xb[(size_t)t * H + h] = b;
        xh[(size_t)t * H + h] = f2h(__uint_as_float((uint32_t)b << 16));
    }
}

// ---------------------------------------------------------------------------------------------------------
// Synthetic trellis (counter-based splitmix64; the oracle computes the same integers).
// ---------------------------------------------------------------------------------------------------------
__host__ __device__ __forceinline__ uint64_t mix64(uint64_t z)
{
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

__device__ __forceinline__ uint16_t synth_word(uint64_t seed, uint64_t i)
{
    return (uint16_t)(mix64(seed + ((i >> 2) + 1) * 0x9E3779B97F4A7C15ull) >> (16 * (i & 3)));
}

__global__ __launch_bounds__(256) void k_synth_u16(uint16_t* __restrict__ dst, uint64_t n, uint64_t seed, uint64_t start)
{
    const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t j = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; j < n; j += stride) dst[j] = synth_word(seed, start + j);
}

// One expert per blockIdx.y; four words (one hash) per thread and step, 8-byte stores.
__global__ __launch_bounds__(256) void k_synth_layer(const int64_t* __restrict__ gp, const int64_t* __restrict__ up,
                                                     const int64_t* __restrict__ dp, uint64_t n1, uint64_t layer_seed)
{
    const int e = blockIdx.y;
    const uint64_t seed = mix64(layer_seed * 0x100000001B3ull + (uint64_t)e);
    uint16_t* base[3] = { reinterpret_cast<uint16_t*>(gp[e]), reinterpret_cast<uint16_t*>(up[e]),
                          reinterpret_cast<uint16_t*>(dp[e]) };
    const uint64_t nq = 3 * n1 / 4;   // n1 is a multiple of 4
    const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t q = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; q < nq; q += stride)
    {
        const uint64_t h = mix64(seed + (q + 1) * 0x9E3779B97F4A7C15ull);
        const uint64_t i = q * 4;
        const int m = (int)(i / n1);
        *reinterpret_cast<uint64_t*>(base[m] + (i - (uint64_t)m * n1)) = h;
    }
}

// mm_permute's launches; e_sorted (optional, [n]) receives the expert bin of each sorted position.
int permute_launch(const int64_t* ids, const float* w, int n, int topk, int E, int32_t* counts, int32_t* offsets,
                   int32_t* order, int32_t* token_sorted, float* weight_sorted, int32_t* inv_order, int32_t* active,
                   int32_t* nactive, int32_t* e_sorted, void* workspace, size_t workspace_bytes, mm_stream_t stream)
{
    MM_CHECK_ARG(E > 0 && E <= 1024, "mm_permute: E must be in [1, 1024] (E=%d)", E);
    MM_CHECK_ARG(n >= 0 && topk > 0, "mm_permute: bad n/topk");
    MM_CHECK_ARG(counts && offsets && (n == 0 || (ids && order)), "mm_permute: null pointer");
    const size_t need = mm_permute_workspace(n, E);
    MM_CHECK_ARG(workspace_bytes >= need && (need == 0 || workspace), "mm_permute: workspace too small (%zu < %zu)",
                 workspace_bytes, need);
    const hipStream_t hs = reinterpret_cast<hipStream_t>(stream);
    if (n <= PERM_SINGLE_MAX)
    {
        hipLaunchKernelGGL(k_permute_single, dim3(1), dim3(PERM_THREADS), 0, hs, ids, w, n, topk, E, counts, offsets,
                           order, token_sorted, weight_sorted, inv_order, active, nactive, e_sorted);
    }
    else
    {
        const int B = (n + PERM_CHUNK - 1) / PERM_CHUNK;
        int32_t* hist = (int32_t*)workspace;
        hipLaunchKernelGGL(k_permute_hist, dim3(B), dim3(PERM_THREADS), 0, hs, ids, n, E, PERM_CHUNK, hist);
        hipLaunchKernelGGL(k_permute_scan, dim3(1), dim3(PERM_THREADS), 0, hs, hist, B, n, E, counts, offsets, active,
                           nactive);
        hipLaunchKernelGGL(k_permute_scatter, dim3(B), dim3(PERM_THREADS), 0, hs, ids, w, n, topk, E, PERM_CHUNK, hist,
                           order, token_sorted, weight_sorted, inv_order, e_sorted);
    }
    return check_launch("mm_permute");
}

}  // namespace mm

using namespace mm;

static inline hipStream_t S(mm_stream_t s) { return reinterpret_cast<hipStream_t>(s); }

extern "C" {

int mm_version(void) { return 100; }

const char* mm_last_error(void) { return mm::g_err; }

int mm_host_alloc(void** ptr, size_t bytes)
{
    MM_CHECK_ARG(ptr != nullptr, "mm_host_alloc: null out pointer");
    const hipError_t e = hipHostMalloc(ptr, bytes ? bytes : 1, hipHostMallocMapped | hipHostMallocPortable | hipHostMallocCoherent);
    if (e != hipSuccess) return set_error(MM_ERR_HIP, "mm_host_alloc(%zu): %s", bytes, hipGetErrorString(e));
    return MM_OK;
}

int mm_host_free(void* ptr)
{
    if (!ptr) return MM_OK;
    const hipError_t e = hipHostFree(ptr);
    if (e != hipSuccess) return set_error(MM_ERR_HIP, "mm_host_free: %s", hipGetErrorString(e));
    return MM_OK;
}

int mm_router_topk(const void* x_bf16, int T, int H, const float* gate, int E, int k, float* logits, int64_t* ids,
                   float* w, mm_stream_t stream)
{
    MM_CHECK_ARG(T >= 0 && H > 0 && H % 16 == 0, "mm_router_topk: need H > 0, H %% 16 == 0 (H=%d)", H);
    MM_CHECK_ARG(E > 0 && E <= 1024 && k > 0 && k <= 32 && k <= E, "mm_router_topk: need 0 < k <= 32, k <= E <= 1024");
    MM_CHECK_ARG(x_bf16 && gate && ids && w && logits, "mm_router_topk: null pointer (logits workspace is required)");
    if (T == 0) return MM_OK;
    if (T <= 4 && H % 256 == 0 && ((uintptr_t)x_bf16 & 7) == 0 && ((uintptr_t)gate & 15) == 0)
        hipLaunchKernelGGL(k_router_gemv<4>, dim3(E, 1), dim3(256), 0, S(stream), (const uint16_t*)x_bf16, gate,
                           logits, T, H, E);
    else if (T <= RT_MAX_T && H % 256 == 0 && ((uintptr_t)x_bf16 & 7) == 0 && ((uintptr_t)gate & 15) == 0)
        hipLaunchKernelGGL(k_router_gemv<16>, dim3(E, (T + 15) / 16), dim3(256), 0, S(stream), (const uint16_t*)x_bf16,
                           gate, logits, T, H, E);
    else if (H % RM_K == 0 && ((uintptr_t)x_bf16 & 15) == 0 && ((uintptr_t)gate & 15) == 0)
        hipLaunchKernelGGL((k_router_mfma<RM_TM, RM_TN, RM_WM, RM_WN>), dim3((E + RM_TN - 1) / RM_TN,
                           (T + RM_TM - 1) / RM_TM), dim3(64 * RM_WM * RM_WN), 0, S(stream),
                           (const uint16_t*)x_bf16, gate, logits, T, H, E);
    else
        hipLaunchKernelGGL(k_router_logits, dim3((E + 63) / 64, (T + 63) / 64), dim3(256), 0, S(stream),
                           (const uint16_t*)x_bf16, gate, logits, T, H, E);
    if (E <= 384)
        hipLaunchKernelGGL(k_router_topk_q<6>, dim3((T + 3) / 4), dim3(256), 0, S(stream), logits, T, E, k, ids, w);
    else if (E <= 512)
        hipLaunchKernelGGL(k_router_topk_q<8>, dim3((T + 3) / 4), dim3(256), 0, S(stream), logits, T, E, k, ids, w);
    else
        hipLaunchKernelGGL(k_router_topk, dim3((T + 3) / 4), dim3(256), 0, S(stream), logits, T, E, k, ids, w);
    return check_launch("mm_router_topk");
}

int mm_split(const int64_t* sel, const float* w, const void* z_fp16, int n, int bsz, int H, int E, const int32_t* slotof,
             const float* score, const float* pol, int64_t* ctrl, void* hx, int32_t* hpicks, int64_t* seqc, int li,
             int64_t* sel_out, float* w_out, int64_t* dflag, int64_t* stats, int32_t* counts, int32_t* hits,
             int32_t* misses, int32_t* nhnm, mm_stream_t stream)
{
    MM_CHECK_ARG(E > 0 && E <= 1024, "mm_split: E <= 1024 (E=%d)", E);
    MM_CHECK_ARG(H % 8 == 0 && bsz > 0 && n >= 0 && n % bsz == 0, "mm_split: need H %% 8 == 0 and n a multiple of bsz");
    MM_CHECK_ARG(sel && w && z_fp16 && slotof && score && pol && ctrl && hx && hpicks && seqc && sel_out && w_out && dflag && stats,
                 "mm_split: null pointer");
    SplitArgs a{ sel, w, (const uint16_t*)z_fp16, n, bsz, n / bsz, H, E, slotof, score, pol, ctrl, (uint16_t*)hx, hpicks,
                 seqc, li, sel_out, w_out, dflag, stats, counts, hits, misses, nhnm };
    hipLaunchKernelGGL(k_split, dim3(1), dim3(256), 0, S(stream), a);
    return check_launch("mm_split");
}

int mm_combine_host(float* out, int n, int64_t* dflag, const int64_t* ctrl, const float* hout, int64_t* stats,
                    int64_t timeout_ns, mm_stream_t stream)
{
    MM_CHECK_ARG(out && dflag && ctrl && hout && stats && n >= 0, "mm_combine_host: bad argument");
    int dev = 0, khz = 0;
    (void)hipGetDevice(&dev);
    if (hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, dev) != hipSuccess || khz <= 0) khz = 100000;
    const double ns_per_tick = 1e6 / (double)khz;
    const uint64_t ticks = timeout_ns <= 0 ? 0 : (uint64_t)((double)timeout_ns / ns_per_tick);
    const int blocks = n <= 16 * 256 * 16 ? 16 : min(256, (n + 256 * 16 - 1) / (256 * 16));
    hipLaunchKernelGGL(k_host_wait, dim3(1), dim3(64), 0, S(stream), dflag,
                       const_cast<int64_t*>(ctrl), stats, ticks, ns_per_tick);
    hipLaunchKernelGGL(k_host_add, dim3(blocks), dim3(256), 0, S(stream), out, n, dflag, hout);
    return check_launch("mm_combine_host");
}

size_t mm_permute_workspace(int n, int E)
{
    if (n <= PERM_SINGLE_MAX) return 0;
    const int B = (n + PERM_CHUNK - 1) / PERM_CHUNK;
    return (size_t)(E + 1) * B * sizeof(int32_t);
}

int mm_permute(const int64_t* ids, const float* w, int n, int topk, int E, int32_t* counts, int32_t* offsets,
               int32_t* order, int32_t* token_sorted, float* weight_sorted, int32_t* inv_order, int32_t* active,
               int32_t* nactive, void* workspace, size_t workspace_bytes, mm_stream_t stream)
{
    return mm::permute_launch(ids, w, n, topk, E, counts, offsets, order, token_sorted, weight_sorted, inv_order, active,
                              nactive, nullptr, workspace, workspace_bytes, stream);
}

int mm_combine(float* out, const float* Y, const int64_t* ids, const float* w, int T, int k, int H, int E, int accumulate,
               mm_stream_t stream)
{
    MM_CHECK_ARG(out && Y && ids && w, "mm_combine: null pointer");
    MM_CHECK_ARG(T >= 0 && k > 0 && H > 0 && H % 4 == 0, "mm_combine: need H %% 4 == 0");
    if (T == 0) return MM_OK;
    dim3 grid((H / 4 + 255) / 256, T);
    hipLaunchKernelGGL(k_combine, grid, dim3(256), 0, S(stream), out, Y, ids, w, T, k, H, E, accumulate);
    return check_launch("mm_combine");
}

int mm_prepare_input(const float* x, int T, int H, int rescale, void* x_bf16, void* x_fp16, mm_stream_t stream)
{
    MM_CHECK_ARG(x && x_fp16 && T >= 0 && H > 0, "mm_prepare_input: bad argument");
    if (T == 0) return MM_OK;
    hipLaunchKernelGGL(k_prepare_input, dim3(T), dim3(256), 0, S(stream), x, H, rescale, (uint16_t*)x_bf16, (uint16_t*)x_fp16);
    return check_launch("mm_prepare_input");
}

uint64_t mm_expert_seed(uint64_t layer_seed, uint64_t expert) { return mix64(layer_seed * 0x100000001B3ull + expert); }

int mm_synth_u16(uint16_t* dst, uint64_t n, uint64_t seed, uint64_t start, mm_stream_t stream)
{
    MM_CHECK_ARG(dst || n == 0, "mm_synth_u16: null pointer");
    if (n == 0) return MM_OK;
    const uint64_t blocks = (n + 255) / 256;
    hipLaunchKernelGGL(k_synth_u16, dim3((unsigned)(blocks < 65536 ? blocks : 65536)), dim3(256), 0, S(stream), dst, n, seed, start);
    return check_launch("mm_synth_u16");
}

int mm_synth_layer(const mm_layer_t* L, uint64_t layer_seed, mm_stream_t stream)
{
    MM_CHECK_ARG(L && L->gate_ptr && L->up_ptr && L->down_ptr, "mm_synth_layer: null layer");
    MM_CHECK_ARG(L->E > 0 && L->H % 128 == 0 && L->I % 128 == 0, "mm_synth_layer: bad shape");
    const uint64_t n1 = (uint64_t)(L->H / 16) * (L->I / 16) * 48;
    hipLaunchKernelGGL(k_synth_layer, dim3(256, L->E), dim3(256), 0, S(stream), L->gate_ptr, L->up_ptr, L->down_ptr, n1,
                       layer_seed);
    return check_launch("mm_synth_layer");
}

}  // extern "C"
