// Decode expert path: EXL3 3-bpw trellis decode fused into a multi-token GEMV on gfx950.
//
// Work unit = (active expert, 128-column output block), full K. A workgroup of 8 waves streams its unit's tiles
// straight from HBM: a wave covers one tile row of the block per step (8 tiles x 96 B = 768 B contiguous, one
// 12-byte load per lane, 4 tile rows in flight), 8 lanes per tile, each lane decoding 32 consecutive trellis
// states = 16 input rows x 2 output columns of its tile. Waves split K; their partial sums meet in LDS in fixed
// order and the same workgroup runs the epilogue (output Hadamard transform, SwiGLU, down-input transform or
// the down output transform). No cross-workgroup communication: every launch is self-contained and the
// results are deterministic.
//
// Routing: for decode-sized calls the workgroup finds its expert and that expert's routes directly from the
// route ids (n <= 1024): the a-th active expert in ascending id, its routes in ascending route index -- the
// same stable order as the permutation. Larger calls pass the permutation (offsets/order/active).
//
// Numerics follow the reference's EXACT expert (kernels/cpu_avx2/ft_core.h:977-1011): fp16 weights
// fp16(fma(1024 + bytesum, KINV, KBIAS)) (one rounding, v_pk_fma_f16), fp16 transformed activations,
// fp32 accumulation (v_dot2_f32_f16), fp16 rounding at the same points.
#include "mm_common.h"

namespace mm {

constexpr int GV_WAVES = 8;
constexpr int GV_THREADS = 64 * GV_WAVES;
constexpr int GV_COLS = 128;         // output columns per unit (8 tiles)
constexpr int GV_MAX_ROWS = 256;     // routes per expert on this path
constexpr int GV_ROUTE_MAX = 1024;   // in-kernel routing limit (routes per call)
constexpr int GV_PF = 4;             // tile rows in flight per wave

typedef const __attribute__((address_space(1))) uint32_t gu32;

struct GemvArgs
{
    const int64_t* wptr0;     // gate (mode 0) or down (mode 1) pointer table
    const int64_t* wptr1;     // up (mode 0)
    const uint16_t* suh13;    // [E][2][H]
    const uint16_t* svh13;    // [E][2][I]
    const uint16_t* suh2;     // [E][I]
    const uint16_t* svh2;     // [E][H]
    const uint16_t* xin;      // mode 0: x fp16 [T][H]; mode 1: xd fp16 [n][I] (flat route order)
    const int64_t* ids;       // [n] route expert ids (in-kernel routing)
    const int32_t* offsets;   // [E+2] or null (then in-kernel routing)
    const int32_t* order;     // [n]
    const int32_t* active;    // [E]
    const int32_t* nactive;   // [1]
    uint16_t* xd;             // mode 0 output: [n][I] fp16, flat route order
    float* Y;                 // mode 1 output: [n][H] fp32, flat route order
    int H, I, E, n, topk;
    int K, N, ncb, max_active;
    float limit;
};

// One lane's share of a tile row: 32 trellis states -> 32 fp16 weights -> dot products with the transformed
// inputs of nr routes.
// Window d0:d1:d2:d3 = tile dwords 3c-1 .. 3c+2 (d0 most significant); state m (stream index 32c + m) has its
// LSB at bit 93 - 3m. Every 16-bit field lies inside one of d1..d3 or one of the dwords straddling their
// boundaries (bits 16..47, 48..79, 80..111 of the window), so each state is one v_bfe_u32.
// The (1024 + bytesum) fp16 operands of a pair are produced packed by v_sad_u8 / v_sad_hi_u8 with 0x6400 in
// both halves of the accumulator, then one v_pk_fma_f16 applies KINV, KBIAS with a single rounding.
// States 8q+2j, 8q+2j+1 (j = 0..3) hold rows (2q, 2q+1) for j even and (2q+8, 2q+9) for j odd, of column c
// (j < 2) or c + 8 (j >= 2) (PERM, ft_core.h:48-61); X[r][d] is the fp16 input pair of rows (2d, 2d+1) of
// route r, so pair j meets X[r][q + 4 * (j & 1)] and accumulates into column j >> 1.
template <int MT>
__device__ __forceinline__ void decode_dot(uint32_t d0, uint32_t d1, uint32_t d2, uint32_t d3,
                                          const uint32_t (*X)[8], int nr, float (*acc)[MT])
{
    const half2_t kinv = { __builtin_bit_cast(_Float16, KINV_BITS), __builtin_bit_cast(_Float16, KINV_BITS) };
    const half2_t kbias = { __builtin_bit_cast(_Float16, KBIAS_BITS), __builtin_bit_cast(_Float16, KBIAS_BITS) };
    const uint32_t mid[3] = { __builtin_amdgcn_alignbit(d2, d3, 16), __builtin_amdgcn_alignbit(d1, d2, 16),
                              __builtin_amdgcn_alignbit(d0, d1, 16) };   // window bits 16.., 48.., 80..
    const uint32_t dw[3] = { d3, d2, d1 };                              // window bits 0.., 32.., 64..
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int j = 0; j < 4; ++j)
        {
            uint32_t p[2];
#pragma unroll
            for (int h = 0; h < 2; ++h)
            {
                const int m = 8 * q + 2 * j + h;
                const int sft = 93 - 3 * m;
                const uint32_t st = (sft & 31) <= 16 ? __builtin_amdgcn_ubfe(dw[sft >> 5], sft & 31, 16)
                                                     : __builtin_amdgcn_ubfe(mid[(sft - 16) >> 5], (sft - 16) & 31, 16);
                p[h] = st * MUL1;
            }
            const uint32_t lo = __builtin_amdgcn_sad_u8(p[0], 0u, 0x64006400u);
            const uint32_t pk = __builtin_amdgcn_sad_hi_u8(p[1], 0u, lo);
            const half2_t wv = __builtin_elementwise_fma(__builtin_bit_cast(half2_t, pk), kinv, kbias);
#pragma unroll
            for (int r = 0; r < MT; ++r)
            {
                if (r >= nr) break;
                acc[j >> 1][r] = __builtin_amdgcn_fdot2(wv, __builtin_bit_cast(half2_t, X[r][q + 4 * (j & 1)]), acc[j >> 1][r], false);
            }
        }
}

__device__ __forceinline__ int block_excl_scan(int v, int* tmp, int* total)
{
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    int incl = v;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1)
    {
        const int o = __shfl_up(incl, d, 64);
        if (lane >= d) incl += o;
    }
    __syncthreads();
    if (lane == 63) tmp[wave] = incl;
    __syncthreads();
    int before = 0, all = 0;
    for (int w = 0; w < nw; ++w)
    {
        const int s = tmp[w];
        if (w < wave) before += s;
        all += s;
    }
    *total = all;
    return before + incl - v;
}

template <int MODE, int MT>
__global__ __launch_bounds__(GV_THREADS, MT >= 8 ? 2 : 4) void k_expert_gemv(GemvArgs a)
{
    constexpr int NMAT = MODE == 0 ? 2 : 1;
    constexpr int WPM = GV_WAVES / NMAT;          // waves per matrix: gate on waves 0..3, up on 4..7
    extern __shared__ __align__(16) uint32_t lds[];   // transformed inputs, then the cross-wave reduction
    __shared__ uint32_t s_bm[32];
    __shared__ int s_tmp[16];
    __shared__ int s_e, s_cnt;
    __shared__ int s_rows[GV_MAX_ROWS];

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int a_idx = blockIdx.x / a.ncb, cb = blockIdx.x % a.ncb;
    if (a_idx >= a.max_active) return;

    // ---- routing: this unit's expert and its routes (flat route indices, ascending)
    if (a.offsets)
    {
        if (threadIdx.x == 0)
        {
            const int na = a.nactive[0];
            s_e = a_idx < na ? a.active[a_idx] : -1;
            s_cnt = s_e >= 0 ? min(GV_MAX_ROWS, a.offsets[s_e + 1] - a.offsets[s_e]) : 0;
        }
        __syncthreads();
        if (s_e < 0) return;
        for (int r = threadIdx.x; r < s_cnt; r += GV_THREADS) s_rows[r] = a.order[a.offsets[s_e] + r];
    }
    else
    {
        if (threadIdx.x < 32) s_bm[threadIdx.x] = 0;
        __syncthreads();
        for (int s = threadIdx.x; s < a.n; s += GV_THREADS)
        {
            const int64_t e = a.ids[s];
            if (e >= 0 && e < a.E) atomicOr(&s_bm[e >> 5], 1u << (e & 31));
        }
        __syncthreads();
        if (wave == 0)
        {
            const int c = lane < 32 ? __popc(s_bm[lane]) : 0;
            int incl = c;
#pragma unroll
            for (int d = 1; d < 32; d <<= 1)
            {
                const int o = __shfl_up(incl, d, 64);
                if (lane >= d) incl += o;
            }
            // the word holding the a_idx-th set bit (0-based)
            const bool here = lane < 32 && a_idx >= incl - c && a_idx < incl;
            if (lane == 0) s_e = -1;
            if (here)
            {
                uint32_t bits = s_bm[lane];
                for (int k = a_idx - (incl - c); k > 0; --k) bits &= bits - 1;
                s_e = lane * 32 + __ffs(bits) - 1;
            }
        }
        __syncthreads();
        if (s_e < 0) return;
        const int e = s_e;
        int base = 0;
        for (int s0 = 0; s0 < a.n; s0 += GV_THREADS)
        {
            const int s = s0 + threadIdx.x;
            const bool f = s < a.n && a.ids[s] == e;
            int tot;
            const int pos = block_excl_scan(f ? 1 : 0, s_tmp, &tot);
            if (f && base + pos < GV_MAX_ROWS) s_rows[base + pos] = s;
            base += tot;
        }
        if (threadIdx.x == 0) s_cnt = min(base, GV_MAX_ROWS);
    }
    __syncthreads();
    const int e = s_e, cnt = s_cnt;

    const int K = a.K, KT = K / 16, NT = a.N / 16;
    const int tau = lane >> 3, cp = lane & 7;
    const int src_lane = cp == 0 ? lane + 7 : lane - 1;
    const int mw = wave / WPM, kw = wave % WPM;   // this wave's matrix and its K slot
    const int64_t* wtab = (NMAT == 2 && mw == 1) ? a.wptr1 : a.wptr0;
    gu32* wbase = reinterpret_cast<gu32*>((uintptr_t)wtab[e]) + (size_t)(cb * 8 + tau) * 24 + 3 * cp;
    const size_t row_stride = (size_t)NT * 24;   // dwords between tile rows
    const int xrow = K / 2;                       // dwords per transformed input row in LDS

    for (int r0 = 0; r0 < cnt; r0 += MT)
    {
        const int nr = min(MT, cnt - r0);
        __syncthreads();
        // ---- prologue: transformed inputs (fp16) for all K, rows r0 .. r0+nr-1
        uint16_t* xt = reinterpret_cast<uint16_t*>(lds);
        if constexpr (MODE == 0)
        {
            const int nblk = K / 128;
            const int items = NMAT * nr * nblk;
            for (int it0 = wave; it0 < items; it0 += 4 * GV_WAVES)
            {
                float va[4], vb[4], sa[4], sb[4];
#pragma unroll
                for (int u = 0; u < 4; ++u)
                {
                    const int it = it0 + u * GV_WAVES;
                    if (it < items)
                    {
                        const int m = it / (nr * nblk), r = (it / nblk) % nr, blk = it % nblk;
                        const int tok = s_rows[r0 + r] / a.topk;
                        const uint16_t* xr = a.xin + (size_t)tok * a.H + blk * 128;
                        const uint16_t* su = a.suh13 + ((size_t)e * 2 + m) * a.H + blk * 128;
                        va[u] = h2f(xr[lane]); vb[u] = h2f(xr[lane + 64]);
                        sa[u] = h2f(su[lane]); sb[u] = h2f(su[lane + 64]);
                    }
                }
#pragma unroll
                for (int u = 0; u < 4; ++u)
                {
                    const int it = it0 + u * GV_WAVES;
                    if (it < items)
                    {
                        const int m = it / (nr * nblk), r = (it / nblk) % nr, blk = it % nblk;
                        prep_block_wave(va[u], vb[u], sa[u], sb[u]);
                        uint16_t* dst = xt + ((size_t)m * MT + r) * K + blk * 128;
                        dst[lane] = f2h(va[u]);
                        dst[lane + 64] = f2h(vb[u]);
                    }
                }
            }
        }
        else
        {
            for (int i = threadIdx.x; i < nr * xrow; i += GV_THREADS)
            {
                const int r = i / xrow, c = i % xrow;
                lds[r * xrow + c] = reinterpret_cast<const uint32_t*>(a.xin + (size_t)s_rows[r0 + r] * a.I)[c];
            }
        }
        __syncthreads();

        // ---- main loop: decode + dot2, GV_PF tile rows in flight per wave
        float acc[2][MT];
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
            for (int r = 0; r < MT; ++r) acc[c][r] = 0.0f;

        const int nit = (KT - kw + WPM - 1) / WPM;   // tile rows of this wave
        {
            gu32* wb = wbase + (size_t)kw * row_stride;
            const uint32_t* xm = lds + (size_t)mw * MT * xrow;
            uint32_t buf[GV_PF][3];
#pragma unroll
            for (int j = 0; j < GV_PF; ++j)
                if (j < nit)
                {
                    gu32* src = wb + (size_t)j * WPM * row_stride;
                    buf[j][0] = __builtin_nontemporal_load(src);
                    buf[j][1] = __builtin_nontemporal_load(src + 1);
                    buf[j][2] = __builtin_nontemporal_load(src + 2);
                }
            for (int g = 0; g < nit; g += GV_PF)
            {
#pragma unroll
                for (int j = 0; j < GV_PF; ++j)
                {
                    if (g + j >= nit) break;
                    const uint32_t d1 = buf[j][0], d2 = buf[j][1], d3 = buf[j][2];
                    if (g + GV_PF + j < nit)      // refill this slot: GV_PF tile rows stay in flight
                    {
                        gu32* src = wb + (size_t)(g + GV_PF + j) * WPM * row_stride;
                        buf[j][0] = __builtin_nontemporal_load(src);
                        buf[j][1] = __builtin_nontemporal_load(src + 1);
                        buf[j][2] = __builtin_nontemporal_load(src + 2);
                    }
                    const int tr = kw + (g + j) * WPM;
                    const uint32_t d0 = __shfl(d3, src_lane, 64);
                    uint32_t X[MT][8];
#pragma unroll
                    for (int r = 0; r < MT; ++r)
                    {
                        if (r >= nr) break;
                        const uint4 xa = *reinterpret_cast<const uint4*>(xm + (size_t)r * xrow + tr * 8);
                        const uint4 xb = *reinterpret_cast<const uint4*>(xm + (size_t)r * xrow + tr * 8 + 4);
                        X[r][0] = xa.x; X[r][1] = xa.y; X[r][2] = xa.z; X[r][3] = xa.w;
                        X[r][4] = xb.x; X[r][5] = xb.y; X[r][6] = xb.z; X[r][7] = xb.w;
                    }
                    decode_dot<MT>(d0, d1, d2, d3, X, nr, acc);
                    // keep each tile row's decode within its step: bounds the live registers while the
                    // GV_PF loads stay in flight
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
        }

        // ---- cross-wave reduction in fixed wave order (waves of one matrix are consecutive)
        __syncthreads();
        float* red = reinterpret_cast<float*>(lds);
        const int col0 = tau * 16 + cp;
#pragma unroll
        for (int r = 0; r < MT; ++r)
        {
            if (r >= nr) break;
            float* rr = red + ((size_t)wave * MT + r) * GV_COLS;
            rr[col0] = acc[0][r];
            rr[col0 + 8] = acc[1][r];
        }
        __syncthreads();
        float* sum = red + (size_t)GV_WAVES * MT * GV_COLS;
        for (int i = threadIdx.x; i < NMAT * nr * GV_COLS; i += GV_THREADS)
        {
            const int m = i / (nr * GV_COLS), r = (i / GV_COLS) % nr, c = i % GV_COLS;
            float s = 0.0f;
#pragma unroll
            for (int w = 0; w < WPM; ++w) s += red[((size_t)(m * WPM + w) * MT + r) * GV_COLS + c];
            sum[((size_t)m * MT + r) * GV_COLS + c] = s;
        }
        __syncthreads();

        // ---- epilogue (one wave per route row)
        for (int r = wave; r < nr; r += GV_WAVES)
        {
            const int s = s_rows[r0 + r];
            const int c = cb * GV_COLS;
            if constexpr (MODE == 0)
            {
                float ga = sum[(0 * MT + r) * GV_COLS + lane], gb = sum[(0 * MT + r) * GV_COLS + lane + 64];
                float ua = sum[(1 * MT + r) * GV_COLS + lane], ub = sum[(1 * MT + r) * GV_COLS + lane + 64];
                const uint16_t* svg = a.svh13 + ((size_t)e * 2 + 0) * a.I + c;
                const uint16_t* svu = a.svh13 + ((size_t)e * 2 + 1) * a.I + c;
                out_block_wave(ga, gb, h2f(svg[lane]), h2f(svg[lane + 64]));
                out_block_wave(ua, ub, h2f(svu[lane]), h2f(svu[lane + 64]));
                float xa = r16(act_gu(ga, ua, a.limit));
                float xb = r16(act_gu(gb, ub, a.limit));
                const uint16_t* sd = a.suh2 + (size_t)e * a.I + c;
                prep_block_wave(xa, xb, h2f(sd[lane]), h2f(sd[lane + 64]));
                a.xd[(size_t)s * a.I + c + lane] = f2h(xa);
                a.xd[(size_t)s * a.I + c + lane + 64] = f2h(xb);
            }
            else
            {
                float ya = sum[r * GV_COLS + lane], yb = sum[r * GV_COLS + lane + 64];
                const uint16_t* sv = a.svh2 + (size_t)e * a.H + c;
                out_block_wave(ya, yb, h2f(sv[lane]), h2f(sv[lane + 64]));
                a.Y[(size_t)s * a.H + c + lane] = ya;
                a.Y[(size_t)s * a.H + c + lane + 64] = yb;
            }
        }
    }
}

static int pick_mt(int max_rows) { return max_rows <= 1 ? 1 : max_rows <= 2 ? 2 : max_rows <= 4 ? 4 : 8; }

static size_t lds_bytes(int nmat, int mt, int K)
{
    const size_t xt = (size_t)nmat * mt * K * 2;
    const size_t red = ((size_t)GV_WAVES + nmat) * mt * GV_COLS * 4;
    return xt > red ? xt : red;
}

template <int MODE>
static void launch_gemv(const GemvArgs& a, int mt, int blocks, hipStream_t s)
{
    const int nmat = MODE == 0 ? 2 : 1;
    const size_t sh = lds_bytes(nmat, mt, a.K);
    switch (mt)
    {
        case 1: hipLaunchKernelGGL((k_expert_gemv<MODE, 1>), dim3(blocks), dim3(GV_THREADS), sh, s, a); break;
        case 2: hipLaunchKernelGGL((k_expert_gemv<MODE, 2>), dim3(blocks), dim3(GV_THREADS), sh, s, a); break;
        case 4: hipLaunchKernelGGL((k_expert_gemv<MODE, 4>), dim3(blocks), dim3(GV_THREADS), sh, s, a); break;
        default: hipLaunchKernelGGL((k_expert_gemv<MODE, 8>), dim3(blocks), dim3(GV_THREADS), sh, s, a); break;
    }
}

static bool g_attr_done = false;
static int g_max_dyn_lds = 64 * 1024;

template <typename F>
static void allow_dynamic_lds(F* kernel, int max_block)
{
    hipFuncAttributes fa{};
    if (hipFuncGetAttributes(&fa, (const void*)kernel) != hipSuccess) return;
    const int dyn = max_block - (int)fa.sharedSizeBytes;
    if (dyn > 0) (void)hipFuncSetAttribute((const void*)kernel, hipFuncAttributeMaxDynamicSharedMemorySize, dyn);
}

// Lets the kernels use the whole LDS of a workgroup (160 KB on gfx950) for their dynamic part; clears any
// error these queries leave behind so it is not reported by a later launch check.
static int set_lds_limits()
{
    if (g_attr_done) return MM_OK;
    int dev = 0, max_block = 0;
    (void)hipGetDevice(&dev);
    if (hipDeviceGetAttribute(&max_block, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess || max_block <= 0)
        max_block = 64 * 1024;
    allow_dynamic_lds(k_expert_gemv<0, 1>, max_block);
    allow_dynamic_lds(k_expert_gemv<0, 2>, max_block);
    allow_dynamic_lds(k_expert_gemv<0, 4>, max_block);
    allow_dynamic_lds(k_expert_gemv<0, 8>, max_block);
    allow_dynamic_lds(k_expert_gemv<1, 1>, max_block);
    allow_dynamic_lds(k_expert_gemv<1, 2>, max_block);
    allow_dynamic_lds(k_expert_gemv<1, 4>, max_block);
    allow_dynamic_lds(k_expert_gemv<1, 8>, max_block);
    (void)hipGetLastError();
    g_max_dyn_lds = max_block - 2048;   // static LDS of the kernels is < 2 KB
    g_attr_done = true;
    return MM_OK;
}

}  // namespace mm

using namespace mm;

extern "C" {

size_t mm_gemv_workspace(int n, int E, int H, int I)
{
    (void)E; (void)H;
    return ((size_t)n * I * 2 + 255) & ~(size_t)255;   // xd: transformed down-projection inputs, fp16 [n][I]
}

int mm_expert_gemv(const mm_layer_t* L, const void* x_fp16, int T, int n, int topk, const int64_t* ids,
                   const int32_t* offsets, const int32_t* order, const int32_t* active, const int32_t* nactive,
                   int max_rows, float* Y, void* workspace, size_t workspace_bytes, int phases, mm_stream_t stream)
{
    MM_CHECK_ARG(L && L->gate_ptr && L->up_ptr && L->down_ptr && L->suh13 && L->svh13 && L->suh2 && L->svh2,
                 "mm_expert_gemv: incomplete layer");
    MM_CHECK_ARG(phases >= 1 && phases <= 3, "mm_expert_gemv: phases must be 1, 2 or 3");
    MM_CHECK_ARG(L->E > 0 && L->E <= 1024 && L->H > 0 && L->I > 0 && L->H % 128 == 0 && L->I % 128 == 0,
                 "mm_expert_gemv: need 0 < E <= 1024 and H, I positive multiples of 128 (E=%d H=%d I=%d)", L->E, L->H, L->I);
    MM_CHECK_ARG(x_fp16 && Y, "mm_expert_gemv: null pointer");
    MM_CHECK_ARG(T > 0 && n > 0 && topk > 0 && n <= T * topk, "mm_expert_gemv: bad T/n/topk");
    MM_CHECK_ARG(max_rows > 0 && max_rows <= GV_MAX_ROWS, "mm_expert_gemv: max_rows must be in [1, %d]", GV_MAX_ROWS);
    const bool perm = offsets != nullptr;
    MM_CHECK_ARG(perm ? (order && active && nactive) : (ids != nullptr && n <= GV_ROUTE_MAX),
                 "mm_expert_gemv: pass ids (n <= %d) or the permutation (offsets, order, active, nactive)", GV_ROUTE_MAX);
    const size_t need = mm_gemv_workspace(n, L->E, L->H, L->I);
    MM_CHECK_ARG(workspace && workspace_bytes >= need, "mm_expert_gemv: workspace too small (%zu < %zu)", workspace_bytes, need);
    const int mt = pick_mt(max_rows);
    set_lds_limits();
    MM_CHECK_ARG(lds_bytes(2, mt, L->H) <= (size_t)g_max_dyn_lds && lds_bytes(1, mt, L->I) <= (size_t)g_max_dyn_lds,
                 "mm_expert_gemv: H or I too large for the LDS budget at %d rows", mt);
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);

    GemvArgs a{};
    a.suh13 = L->suh13; a.svh13 = L->svh13; a.suh2 = L->suh2; a.svh2 = L->svh2;
    a.ids = ids; a.offsets = offsets; a.order = order; a.active = active; a.nactive = nactive;
    a.H = L->H; a.I = L->I; a.E = L->E; a.n = n; a.topk = topk; a.limit = L->limit;
    a.max_active = n < L->E ? n : L->E;
    uint16_t* xd = static_cast<uint16_t*>(workspace);
    if (phases & 1)
    {
        a.wptr0 = L->gate_ptr; a.wptr1 = L->up_ptr; a.xin = (const uint16_t*)x_fp16; a.xd = xd; a.Y = nullptr;
        a.K = L->H; a.N = L->I; a.ncb = L->I / GV_COLS;
        launch_gemv<0>(a, mt, a.max_active * a.ncb, s);
    }
    if (phases & 2)
    {
        a.wptr0 = L->down_ptr; a.wptr1 = nullptr; a.xin = xd; a.xd = nullptr; a.Y = Y;
        a.K = L->I; a.N = L->H; a.ncb = L->H / GV_COLS;
        launch_gemv<1>(a, mt, a.max_active * a.ncb, s);
    }
    return check_launch("mm_expert_gemv");
}

}  // extern "C"
