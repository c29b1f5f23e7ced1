// Decode expert path: EXL3 3-bpw trellis decode fused into a multi-token GEMV on gfx950.
//
// Work unit = (active expert, 128-column output block, 1024-row K part). Each workgroup of 4 waves streams
// its unit's tiles straight from HBM with coalesced 12-byte loads: a wave covers one tile row of the
// block (8 tiles x 96 B = 768 B contiguous), 8 lanes per tile, and each lane decodes 32 consecutive trellis
// states = 16 rows x 2 columns of its tile. The input Hadamard transform of the unit's K part is computed
// in the prologue into LDS; partial sums of the K parts go to a workspace and the last workgroup of a unit
// (atomic ticket) adds them in fixed order and runs the epilogue (output transform, SwiGLU, down-input
// transform / output transform). Results are deterministic.
//
// Numerics follow the reference's EXACT expert (kernels/cpu_avx2/ft_core.h:977-1011): fp16 weights
// fp16(fma(1024 + bytesum, KINV, KBIAS)) (one rounding, v_pk_fma_f16), fp16 transformed activations,
// fp32 accumulation (v_dot2_f32_f16), fp16 rounding at the same points.
#include "mm_common.h"

namespace mm {

constexpr int GV_WAVES = 4;
constexpr int GV_THREADS = 64 * GV_WAVES;
constexpr int GV_COLS = 128;         // output columns per unit (8 tiles)
constexpr int GV_KPART = 1024;       // input rows per unit (64 tile rows)
constexpr int GV_MAX_ROWS = 256;     // routes per expert on this path

// Trellis words are read through the global address space (global_load, not flat_load): the pointer tables
// hold plain device addresses.
typedef const __attribute__((address_space(1))) uint32_t gu32;

struct GemvArgs
{
    const int64_t* wptr0;     // gate (mode 0) or down (mode 1) pointer table
    const int64_t* wptr1;     // up (mode 0)
    const uint16_t* suh13;    // [E][2][H]
    const uint16_t* svh13;    // [E][2][I]
    const uint16_t* suh2;     // [E][I]
    const uint16_t* svh2;     // [E][H]
    const uint16_t* xin;      // mode 0: x fp16 [T][H]; mode 1: xd fp16 [n][I]
    const int32_t* offsets;   // [E+2]
    const int32_t* order;     // [n]
    const int32_t* active;    // [E]
    const int32_t* nactive;   // [1]
    float* part;              // [kparts][n][nmat][N]
    int32_t* tickets;         // [max_active * ncb * maxchunk]
    uint16_t* xd;             // mode 0 output: [n][I] fp16
    float* Y;                 // mode 1 output: [n][H] fp32 at flat route index
    int H, I, E, n, topk;
    int K, N, ncb, kparts, maxchunk, max_active;
    float limit;
};

__device__ __forceinline__ uint32_t wbits(uint32_t v)
{
    // (1024 + bytesum(state * MUL1)) as fp16 bits: 1024 is 0x6400 and the byte sum (<= 1020) fills the
    // mantissa exactly, so v_sad_u8 with 0x6400 as accumulator yields the fp16 operand of the hfma.
    const uint32_t p = (v & 0xffffu) * MUL1;
    return __builtin_amdgcn_sad_u8(p, 0u, 0x6400u);
}

// Decode one lane's 32 states of a tile from the 128-bit window d0:d1:d2:d3 (d0 most significant: tile
// dwords 3c-1 .. 3c+2). State m has its LSB at bit 93 - 3m of the window. Returns 16 packed fp16 weight
// pairs: w[4q + 0] rows (2q, 2q+1) col c; w[4q + 1] rows (2q+8, 2q+9) col c; w[4q + 2], w[4q + 3] the
// same rows for col c + 8.
__device__ __forceinline__ void decode_lane(uint32_t d0, uint32_t d1, uint32_t d2, uint32_t d3, half2_t* w)
{
    const half2_t kinv = { __builtin_bit_cast(_Float16, KINV_BITS), __builtin_bit_cast(_Float16, KINV_BITS) };
    const half2_t kbias = { __builtin_bit_cast(_Float16, KBIAS_BITS), __builtin_bit_cast(_Float16, KBIAS_BITS) };
    uint32_t h[32];
#pragma unroll
    for (int m = 0; m < 32; ++m)
    {
        const int s = 93 - 3 * m;
        const int q = s >> 5, r = s & 31;
        const uint32_t lo = q == 0 ? d3 : (q == 1 ? d2 : d1);
        const uint32_t hi = q == 0 ? d2 : (q == 1 ? d1 : d0);
        const uint32_t v = r == 0 ? lo : __builtin_amdgcn_alignbit(hi, lo, r);
        h[m] = wbits(v);
    }
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int j = 0; j < 4; ++j)
        {
            const uint32_t pk = h[8 * q + 2 * j] | (h[8 * q + 2 * j + 1] << 16);
            // j = 0: states 8q+0,1 (col c, rows 2q, 2q+1); j = 1: 8q+2,3 (col c, rows 2q+8, 2q+9);
            // j = 2: 8q+4,5 (col c+8, rows 2q, 2q+1); j = 3: 8q+6,7 (col c+8, rows 2q+8, 2q+9)
            w[4 * q + j] = __builtin_elementwise_fma(__builtin_bit_cast(half2_t, pk), kinv, kbias);
        }
}

template <int MODE, int MT>
__global__ __launch_bounds__(GV_THREADS) void k_expert_gemv(GemvArgs a)
{
    constexpr int NMAT = MODE == 0 ? 2 : 1;
    // LDS: transformed inputs [NMAT][MT][KPART] fp16, reused as the cross-wave reduction buffer
    // [GV_WAVES][NMAT][MT][GV_COLS] fp32 (same size: KPART * 2 B = GV_WAVES * GV_COLS * 4 B).
    __shared__ __align__(16) uint32_t lds[NMAT * MT * GV_KPART / 2];
    __shared__ int s_last;
    static_assert(GV_KPART * 2 == GV_WAVES * GV_COLS * 4, "LDS reuse");

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int b = blockIdx.x;
    const int xcd = b & 7, slot = b >> 3;
    const int kq = slot % a.kparts;
    const int g = (slot / a.kparts) * 8 + xcd;          // all K parts of a unit on one XCD
    const int a_idx = g / a.ncb, cb = g % a.ncb;
    if (a_idx >= a.max_active || a_idx >= a.nactive[0]) return;
    const int e = a.active[a_idx];
    const int row0 = a.offsets[e];
    const int cnt = a.offsets[e + 1] - row0;
    const int k0 = kq * GV_KPART;
    const int klen = min(GV_KPART, a.K - k0);
    const int ntr = klen / 16;                           // tile rows in this K part
    const int NT = a.N / 16;                             // tiles per tile row
    const int tau = lane >> 3, cp = lane & 7;
    const int src_lane = cp == 0 ? lane + 7 : lane - 1;

    gu32* wbase[NMAT];
    wbase[0] = reinterpret_cast<gu32*>((uintptr_t)a.wptr0[e]);
    if constexpr (NMAT == 2) wbase[NMAT - 1] = reinterpret_cast<gu32*>((uintptr_t)a.wptr1[e]);

    for (int chunk = 0; chunk * MT < cnt && chunk < a.maxchunk; ++chunk)
    {
        const int r0 = chunk * MT, nr = min(MT, cnt - r0);
        __syncthreads();   // LDS reuse across chunks
        // ---- prologue: transformed inputs of this K part
        uint16_t* xt = reinterpret_cast<uint16_t*>(lds);
        if constexpr (MODE == 0)
        {
            const int nblk = klen / 128;
            for (int item = wave; item < NMAT * MT * nblk; item += GV_WAVES)
            {
                const int m = item / (MT * nblk), r = (item / nblk) % MT, blk = item % nblk;
                uint16_t* dst = xt + ((size_t)m * MT + r) * GV_KPART + blk * 128;
                if (r < nr)
                {
                    const int p = row0 + r0 + r;
                    const int tok = a.order[p] / a.topk;
                    const int k = k0 + blk * 128;
                    const uint16_t* xr = a.xin + (size_t)tok * a.H + k;
                    const uint16_t* su = a.suh13 + ((size_t)e * 2 + m) * a.H + k;
                    float va = h2f(xr[lane]), vb = h2f(xr[lane + 64]);
                    prep_block_wave(va, vb, h2f(su[lane]), h2f(su[lane + 64]));
                    dst[lane] = f2h(va);
                    dst[lane + 64] = f2h(vb);
                }
                else
                {
                    dst[lane] = 0;
                    dst[lane + 64] = 0;
                }
            }
        }
        else
        {
            for (int i = threadIdx.x; i < MT * klen / 2; i += GV_THREADS)
            {
                const int r = i / (klen / 2), c = i % (klen / 2);
                uint32_t v = 0;
                if (r < nr)
                {
                    const int p = row0 + r0 + r;
                    v = reinterpret_cast<const uint32_t*>(a.xin + (size_t)p * a.I + k0)[c];
                }
                lds[r * (GV_KPART / 2) + c] = v;
            }
        }
        __syncthreads();

        // ---- main loop: decode + dot2 over this wave's tile rows
        float acc[NMAT][2][MT];
#pragma unroll
        for (int m = 0; m < NMAT; ++m)
#pragma unroll
            for (int c = 0; c < 2; ++c)
#pragma unroll
                for (int r = 0; r < MT; ++r) acc[m][c][r] = 0.0f;

#pragma unroll
        for (int m = 0; m < NMAT; ++m)
        {
            gu32* wb = wbase[m] + ((size_t)(k0 / 16) * NT + cb * 8 + tau) * 24 + 3 * cp;
            const uint32_t* xm = lds + (size_t)m * MT * (GV_KPART / 2);
            // software pipeline: the next tile row's 12 bytes are in flight while the current one decodes
            int tr = wave;
            uint32_t n1 = 0, n2 = 0, n3 = 0;
            if (tr < ntr)
            {
                gu32* src = wb + (size_t)tr * NT * 24;
                n1 = __builtin_nontemporal_load(src);
                n2 = __builtin_nontemporal_load(src + 1);
                n3 = __builtin_nontemporal_load(src + 2);
            }
            for (; tr < ntr; tr += GV_WAVES)
            {
                const uint32_t d1 = n1, d2 = n2, d3 = n3;
                const int nx = tr + GV_WAVES;
                if (nx < ntr)
                {
                    gu32* src = wb + (size_t)nx * NT * 24;
                    n1 = __builtin_nontemporal_load(src);
                    n2 = __builtin_nontemporal_load(src + 1);
                    n3 = __builtin_nontemporal_load(src + 2);
                }
                const uint32_t d0 = __shfl(d3, src_lane, 64);
                half2_t wv[16];
                decode_lane(d0, d1, d2, d3, wv);
#pragma unroll
                for (int r = 0; r < MT; ++r)
                {
                    const uint4 xa = *reinterpret_cast<const uint4*>(xm + (size_t)r * (GV_KPART / 2) + tr * 8);
                    const uint4 xb = *reinterpret_cast<const uint4*>(xm + (size_t)r * (GV_KPART / 2) + tr * 8 + 4);
                    const uint32_t X[8] = { xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w };
                    float c0 = acc[m][0][r], c1 = acc[m][1][r];
#pragma unroll
                    for (int q = 0; q < 4; ++q)
                    {
                        c0 = __builtin_amdgcn_fdot2(wv[4 * q + 0], __builtin_bit_cast(half2_t, X[q]), c0, false);
                        c0 = __builtin_amdgcn_fdot2(wv[4 * q + 1], __builtin_bit_cast(half2_t, X[4 + q]), c0, false);
                        c1 = __builtin_amdgcn_fdot2(wv[4 * q + 2], __builtin_bit_cast(half2_t, X[q]), c1, false);
                        c1 = __builtin_amdgcn_fdot2(wv[4 * q + 3], __builtin_bit_cast(half2_t, X[4 + q]), c1, false);
                    }
                    acc[m][0][r] = c0;
                    acc[m][1][r] = c1;
                }
            }
        }

        // ---- cross-wave reduction (fixed wave order) and partial store
        __syncthreads();
        float* red = reinterpret_cast<float*>(lds);
        const int col0 = tau * 16 + cp;
#pragma unroll
        for (int m = 0; m < NMAT; ++m)
#pragma unroll
            for (int r = 0; r < MT; ++r)
            {
                float* rr = red + (((size_t)wave * NMAT + m) * MT + r) * GV_COLS;
                rr[col0] = acc[m][0][r];
                rr[col0 + 8] = acc[m][1][r];
            }
        __syncthreads();
        for (int i = threadIdx.x; i < NMAT * MT * GV_COLS; i += GV_THREADS)
        {
            const int m = i / (MT * GV_COLS), r = (i / GV_COLS) % MT, c = i % GV_COLS;
            if (r >= nr) continue;
            float s = 0.0f;
#pragma unroll
            for (int w = 0; w < GV_WAVES; ++w) s += red[(((size_t)w * NMAT + m) * MT + r) * GV_COLS + c];
            const int p = row0 + r0 + r;
            a.part[(((size_t)kq * a.n + p) * NMAT + m) * a.N + cb * GV_COLS + c] = s;
        }

        // ---- ticket: the last K part of this unit runs the epilogue
        __threadfence();
        __syncthreads();
        if (threadIdx.x == 0)
        {
            int32_t* tk = a.tickets + ((size_t)g * a.maxchunk + chunk);
            const int old = atomicAdd(tk, 1);
            s_last = old == a.kparts - 1;
            if (s_last) *tk = 0;
        }
        __syncthreads();
        if (!s_last) continue;
        __threadfence();

        for (int r = wave; r < nr; r += GV_WAVES)
        {
            const int p = row0 + r0 + r;
            const int c = cb * GV_COLS;
            float v[NMAT][2];
#pragma unroll
            for (int m = 0; m < NMAT; ++m)
            {
                float sa = 0.0f, sb = 0.0f;
                for (int q = 0; q < a.kparts; ++q)
                {
                    const float* pp = a.part + (((size_t)q * a.n + p) * NMAT + m) * a.N + c;
                    sa += __builtin_nontemporal_load(pp + lane);
                    sb += __builtin_nontemporal_load(pp + lane + 64);
                }
                v[m][0] = sa;
                v[m][1] = sb;
            }
            if constexpr (MODE == 0)
            {
                const uint16_t* svg = a.svh13 + ((size_t)e * 2 + 0) * a.I + c;
                const uint16_t* svu = a.svh13 + ((size_t)e * 2 + 1) * a.I + c;
                out_block_wave(v[0][0], v[0][1], h2f(svg[lane]), h2f(svg[lane + 64]));
                out_block_wave(v[1][0], v[1][1], h2f(svu[lane]), h2f(svu[lane + 64]));
                float xa = r16(act_gu(v[0][0], v[1][0], a.limit));
                float xb = r16(act_gu(v[0][1], v[1][1], a.limit));
                const uint16_t* sd = a.suh2 + (size_t)e * a.I + c;
                prep_block_wave(xa, xb, h2f(sd[lane]), h2f(sd[lane + 64]));
                a.xd[(size_t)p * a.I + c + lane] = f2h(xa);
                a.xd[(size_t)p * a.I + c + lane + 64] = f2h(xb);
            }
            else
            {
                const uint16_t* sv = a.svh2 + (size_t)e * a.H + c;
                out_block_wave(v[0][0], v[0][1], h2f(sv[lane]), h2f(sv[lane + 64]));
                const int s = a.order[p];
                a.Y[(size_t)s * a.H + c + lane] = v[0][0];
                a.Y[(size_t)s * a.H + c + lane + 64] = v[0][1];
            }
        }
    }
}

struct GemvPlan
{
    int max_active, maxchunk, mt;
    size_t part_gu, part_d, xd, tickets_gu, tickets_d;
};

static int pick_mt(int max_rows) { return max_rows <= 1 ? 1 : max_rows <= 2 ? 2 : max_rows <= 4 ? 4 : 8; }

static GemvPlan plan(int n, int E, int H, int I, int max_rows)
{
    GemvPlan p;
    p.max_active = n < E ? n : E;
    p.mt = pick_mt(max_rows);
    p.maxchunk = (GV_MAX_ROWS + 1 - 1) / 1;   // tickets sized for the largest chunk count (MT = 1)
    const int kp_gu = (H + GV_KPART - 1) / GV_KPART, kp_d = (I + GV_KPART - 1) / GV_KPART;
    auto al = [](size_t x) { return (x + 255) & ~(size_t)255; };
    p.tickets_gu = al((size_t)p.max_active * (I / GV_COLS) * p.maxchunk * 4);
    p.tickets_d = al((size_t)p.max_active * (H / GV_COLS) * p.maxchunk * 4);
    p.part_gu = al((size_t)kp_gu * n * 2 * I * 4);
    p.part_d = al((size_t)kp_d * n * H * 4);
    p.xd = al((size_t)n * I * 2);
    return p;
}

template <int MODE>
static void launch_gemv(const GemvArgs& a, int mt, int blocks, hipStream_t s)
{
    switch (mt)
    {
        case 1: hipLaunchKernelGGL((k_expert_gemv<MODE, 1>), dim3(blocks), dim3(GV_THREADS), 0, s, a); break;
        case 2: hipLaunchKernelGGL((k_expert_gemv<MODE, 2>), dim3(blocks), dim3(GV_THREADS), 0, s, a); break;
        case 4: hipLaunchKernelGGL((k_expert_gemv<MODE, 4>), dim3(blocks), dim3(GV_THREADS), 0, s, a); break;
        default: hipLaunchKernelGGL((k_expert_gemv<MODE, 8>), dim3(blocks), dim3(GV_THREADS), 0, s, a); break;
    }
}

}  // namespace mm

using namespace mm;

extern "C" {

size_t mm_gemv_counter_bytes(int n, int E, int H, int I)
{
    const GemvPlan p = plan(n, E, H, I, 1);
    return p.tickets_gu + p.tickets_d;
}

size_t mm_gemv_workspace(int n, int E, int H, int I)
{
    const GemvPlan p = plan(n, E, H, I, 1);
    return p.tickets_gu + p.tickets_d + p.part_gu + p.part_d + p.xd;
}

int mm_expert_gemv(const mm_layer_t* L, const void* x_fp16, int T, int n, int topk, const int32_t* offsets,
                   const int32_t* order, const int32_t* active, const int32_t* nactive, int max_rows, float* Y,
                   void* workspace, size_t workspace_bytes, mm_stream_t stream)
{
    MM_CHECK_ARG(L && L->gate_ptr && L->up_ptr && L->down_ptr && L->suh13 && L->svh13 && L->suh2 && L->svh2,
                 "mm_expert_gemv: incomplete layer");
    MM_CHECK_ARG(L->E > 0 && L->H > 0 && L->I > 0 && L->H % 128 == 0 && L->I % 128 == 0,
                 "mm_expert_gemv: H and I must be positive multiples of 128 (H=%d I=%d)", L->H, L->I);
    MM_CHECK_ARG(x_fp16 && offsets && order && active && nactive && Y, "mm_expert_gemv: null pointer");
    MM_CHECK_ARG(T > 0 && n > 0 && topk > 0 && n <= T * topk, "mm_expert_gemv: bad T/n/topk");
    MM_CHECK_ARG(max_rows > 0 && max_rows <= GV_MAX_ROWS, "mm_expert_gemv: max_rows must be in [1, %d]", GV_MAX_ROWS);
    const size_t need = mm_gemv_workspace(n, L->E, L->H, L->I);
    MM_CHECK_ARG(workspace && workspace_bytes >= need, "mm_expert_gemv: workspace too small (%zu < %zu)", workspace_bytes, need);
    const GemvPlan p = plan(n, L->E, L->H, L->I, max_rows);
    char* ws = static_cast<char*>(workspace);
    int32_t* tk_gu = reinterpret_cast<int32_t*>(ws);
    int32_t* tk_d = reinterpret_cast<int32_t*>(ws + p.tickets_gu);
    float* part_gu = reinterpret_cast<float*>(ws + p.tickets_gu + p.tickets_d);
    float* part_d = reinterpret_cast<float*>(ws + p.tickets_gu + p.tickets_d + p.part_gu);
    uint16_t* xd = reinterpret_cast<uint16_t*>(ws + p.tickets_gu + p.tickets_d + p.part_gu + p.part_d);
    const int maxchunk = (max_rows + p.mt - 1) / p.mt;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);

    GemvArgs a{};
    a.suh13 = L->suh13; a.svh13 = L->svh13; a.suh2 = L->suh2; a.svh2 = L->svh2;
    a.offsets = offsets; a.order = order; a.active = active; a.nactive = nactive;
    a.H = L->H; a.I = L->I; a.E = L->E; a.n = n; a.topk = topk; a.limit = L->limit;
    a.max_active = p.max_active; a.maxchunk = maxchunk;
    // gate + up
    a.wptr0 = L->gate_ptr; a.wptr1 = L->up_ptr; a.xin = (const uint16_t*)x_fp16;
    a.part = part_gu; a.tickets = tk_gu; a.xd = xd; a.Y = nullptr;
    a.K = L->H; a.N = L->I; a.ncb = L->I / GV_COLS; a.kparts = (L->H + GV_KPART - 1) / GV_KPART;
    {
        const int groups = (p.max_active * a.ncb + 7) / 8 * 8;
        launch_gemv<0>(a, p.mt, groups * a.kparts, s);
    }
    // down
    a.wptr0 = L->down_ptr; a.wptr1 = nullptr; a.xin = xd;
    a.part = part_d; a.tickets = tk_d; a.xd = nullptr; a.Y = Y;
    a.K = L->I; a.N = L->H; a.ncb = L->H / GV_COLS; a.kparts = (L->I + GV_KPART - 1) / GV_KPART;
    {
        const int groups = (p.max_active * a.ncb + 7) / 8 * 8;
        launch_gemv<1>(a, p.mt, groups * a.kparts, s);
    }
    return check_launch("mm_expert_gemv");
}

}  // extern "C"
