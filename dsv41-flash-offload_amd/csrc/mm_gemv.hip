// Decode expert path: EXL3 3-bpw trellis decode fused into a multi-token GEMV on gfx950.
//
// Each projection runs as two launches. The partial kernel's work unit is (active expert, 128-column output
// block, 1024-row K part): a 4-wave workgroup streams the unit's tiles straight from HBM -- a wave covers one
// tile row of the block per step (8 tiles x 96 B = 768 B contiguous, one 12-byte load per lane, two register
// sets of 4 tile rows in flight), 8 lanes per tile, each lane decoding 32 consecutive trellis states = 16 input
// rows x 2 output columns -- and writes the unit's partial sums. The epilogue kernel adds the K parts in fixed
// order and applies the output Hadamard transform, SwiGLU and the down-input transform (gate/up) or the down
// output transform. Stream order alone makes the partials visible to the epilogue: the kernels never fence or
// wait on each other, and every result is deterministic. Splitting K gives ~1600 units per projection at the
// decode shapes, which keeps all 256 CUs evenly busy.
//
// Routing: for decode-sized calls (n <= 1024 routes) a workgroup finds its expert and that expert's routes from
// the route ids -- the a-th active expert in ascending id, its routes in ascending route index, the same stable
// order as the permutation. Larger calls pass the permutation (offsets/order/active).
//
// Numerics follow the reference's EXACT expert (kernels/cpu_avx2/ft_core.h:977-1011): fp16 weights
// fp16(fma(1024 + bytesum, KINV, KBIAS)) (one rounding, v_pk_fma_f16), fp16 transformed activations,
// fp32 accumulation (v_dot2_f32_f16), fp16 rounding at the same points.
#include "mm_common.h"

namespace mm {

constexpr int GV_WAVES = 4;
constexpr int GV_THREADS = 64 * GV_WAVES;
constexpr int GV_COLS = 128;         // output columns per unit (8 tiles)
constexpr int GV_KPART = 1024;       // input rows per unit
constexpr int GV_MAX_ROWS = 256;     // routes per expert on this path
constexpr int GV_ROUTE_MAX = 1024;   // in-kernel routing limit (routes per call)
constexpr int GV_PF = 4;             // tile rows per register set (two sets in flight)

typedef uint32_t u32x3 __attribute__((ext_vector_type(3)));

// Trellis rows are read with raw buffer loads: a per-matrix resource descriptor in SGPRs (bounds-checked to the
// matrix), one per-lane 32-bit byte offset and a wave-uniform row offset, so the in-flight loads cost no VGPRs
// for addresses. aux = 2 marks the loads non-temporal (each byte is read once per call).
constexpr int BUF_DWORD3 = 0x00020000;
__device__ __forceinline__ u32x3 load_row(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff)
{
    return __builtin_amdgcn_raw_buffer_load_b96(r, voff, soff, 2);
}

struct GemvArgs
{
    const int64_t* wptr0;     // gate (mode 0) or down (mode 1) pointer table
    const int64_t* wptr1;     // up (mode 0)
    const uint16_t* suh13;    // [E][2][H]
    const uint16_t* xin;      // mode 0: x fp16 [T][H]; mode 1: xd fp16 [n][I] (flat route order)
    const int64_t* ids;       // [n] route expert ids
    const int32_t* offsets;   // [E+2] or null (then in-kernel routing)
    const int32_t* order;     // [n]
    const int32_t* active;    // [E]
    const int32_t* nactive;   // [1]
    float* part;              // [kparts][n][nmat][N] partial sums
    int H, I, E, n, topk;
    int K, N, ncb, kparts, max_active;
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

// The same decode without the dot products: 16 packed fp16 weight pairs in the order of decode_dot's pairs
// (pair 4q + j = states 8q + 2j, 8q + 2j + 1).
__device__ __forceinline__ void decode_pairs(uint32_t d0, uint32_t d1, uint32_t d2, uint32_t d3, half2_t* wv)
{
    const half2_t kinv = { __builtin_bit_cast(_Float16, KINV_BITS), __builtin_bit_cast(_Float16, KINV_BITS) };
    const half2_t kbias = { __builtin_bit_cast(_Float16, KBIAS_BITS), __builtin_bit_cast(_Float16, KBIAS_BITS) };
    const uint32_t mid[3] = { __builtin_amdgcn_alignbit(d2, d3, 16), __builtin_amdgcn_alignbit(d1, d2, 16),
                              __builtin_amdgcn_alignbit(d0, d1, 16) };
    const uint32_t dw[3] = { d3, d2, d1 };
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
            wv[4 * q + j] = __builtin_elementwise_fma(__builtin_bit_cast(half2_t, pk), kinv, kbias);
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

// Main loop for exactly NR routes (a compile-time count: no per-route branches inside the unrolled loop, which
// keeps the register allocation tight). Decodes this wave's tile rows of the K part and leaves the wave's partial
// sums for its 128 columns in red[wave][r][col].
template <int NR>
__device__ __forceinline__ void gemv_rows(__amdgpu_buffer_rsrc_t wres, uint32_t voff, uint32_t row0, uint32_t row_bytes,
                                          int nit, int wpm, int kw, int src_lane, const uint32_t* xm, int xrow,
                                          float* red, int wave, int col0, int mt)
{
    float acc[2][NR];
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int r = 0; r < NR; ++r) acc[c][r] = 0.0f;
    auto step = [&](uint32_t d1, uint32_t d2, uint32_t d3, int t) {
        const int tr = kw + t * wpm;
        const uint32_t d0 = __shfl(d3, src_lane, 64);
        if constexpr (NR == 1)
        {
            // one route: the pairs feed the dot products as they are decoded
            uint32_t X[1][8];
            const uint4 xa = *reinterpret_cast<const uint4*>(xm + tr * 8);
            const uint4 xb = *reinterpret_cast<const uint4*>(xm + tr * 8 + 4);
            X[0][0] = xa.x; X[0][1] = xa.y; X[0][2] = xa.z; X[0][3] = xa.w;
            X[0][4] = xb.x; X[0][5] = xb.y; X[0][6] = xb.z; X[0][7] = xb.w;
            decode_dot<1>(d0, d1, d2, d3, X, 1, acc);
        }
        else
        {
            // several routes: decode once, then one route at a time (its inputs loaded just in time)
            half2_t wv[16];
            decode_pairs(d0, d1, d2, d3, wv);
#pragma unroll
            for (int r = 0; r < NR; ++r)
            {
                const uint4 xa = *reinterpret_cast<const uint4*>(xm + (size_t)r * xrow + tr * 8);
                const uint4 xb = *reinterpret_cast<const uint4*>(xm + (size_t)r * xrow + tr * 8 + 4);
                const uint32_t X[8] = { xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w };
                float c0 = acc[0][r], c1 = acc[1][r];
#pragma unroll
                for (int q = 0; q < 4; ++q)
                {
                    c0 = __builtin_amdgcn_fdot2(wv[4 * q + 0], __builtin_bit_cast(half2_t, X[q]), c0, false);
                    c0 = __builtin_amdgcn_fdot2(wv[4 * q + 1], __builtin_bit_cast(half2_t, X[q + 4]), c0, false);
                    c1 = __builtin_amdgcn_fdot2(wv[4 * q + 2], __builtin_bit_cast(half2_t, X[q]), c1, false);
                    c1 = __builtin_amdgcn_fdot2(wv[4 * q + 3], __builtin_bit_cast(half2_t, X[q + 4]), c1, false);
                }
                acc[0][r] = c0;
                acc[1][r] = c1;
            }
        }
    };
    // Two register sets of GV_PF rows alternate: while one set is decoded the other set's loads are in flight, and
    // a set is refilled only after it has been consumed, so no register copy (and no drain of the load queue) is
    // needed at the loop back-edge. The refill past this wave's last row re-reads an in-range row; the remaining
    // nit % (2 GV_PF) rows run unpipelined.
    const int ngroups = (nit / (2 * GV_PF)) * 2;
    u32x3 ra[GV_PF], rb[GV_PF];
    auto load_set = [&](u32x3* rg, int g) {
#pragma unroll
        for (int j = 0; j < GV_PF; ++j)
            rg[j] = load_row(wres, voff, (row0 + (uint32_t)(min(g * GV_PF + j, nit - 1) * wpm)) * row_bytes);
    };
    auto run_set = [&](u32x3* rg, int g) {
#pragma unroll
        for (int j = 0; j < GV_PF; ++j)
        {
            step(rg[j].x, rg[j].y, rg[j].z, g * GV_PF + j);
            // keep each tile row's decode within its step: bounds the live registers
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    if (ngroups > 0) load_set(ra, 0);
    for (int g = 0; g < ngroups; g += 2)
    {
        load_set(rb, g + 1);
        run_set(ra, g);
        load_set(ra, g + 2);
        run_set(rb, g + 1);
    }
    for (int t = ngroups * GV_PF; t < nit; ++t)
    {
        const u32x3 v = load_row(wres, voff, (row0 + (uint32_t)(t * wpm)) * row_bytes);
        step(v.x, v.y, v.z, t);
    }
    __syncthreads();      // every wave is done reading the LDS inputs before they are overwritten
#pragma unroll
    for (int r = 0; r < NR; ++r)
    {
        float* rr = red + ((size_t)wave * mt + r) * GV_COLS;
        rr[col0] = acc[0][r];
        rr[col0 + 8] = acc[1][r];
    }
}

template <int MODE, int MT>
__global__ __launch_bounds__(GV_THREADS, MT == 1 ? 8 : 4) void k_expert_partial(GemvArgs a)
{
    constexpr int NMAT = MODE == 0 ? 2 : 1;
    constexpr int WPM = GV_WAVES / NMAT;          // waves per matrix (gate on the first half, up on the second)
    __shared__ __align__(16) uint32_t lds[NMAT * MT * GV_KPART / 2];   // transformed inputs, then the reduction
    __shared__ uint32_t s_bm[32];
    __shared__ int s_tmp[16];
    __shared__ int s_e, s_cnt;
    __shared__ int s_rows[GV_MAX_ROWS];
    static_assert(NMAT * MT * GV_KPART * 2 >= GV_WAVES * MT * GV_COLS * 4, "LDS reuse");

    // the wave index is uniform across the wave: readfirstlane keeps the loop bounds in SGPRs, so the K loop
    // branches on scalars and the in-flight loads are not drained at every step
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int kq = blockIdx.x % a.kparts;
    const int unit = blockIdx.x / a.kparts;
    const int a_idx = unit / a.ncb, cb = unit % a.ncb;
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
    const int e = __builtin_amdgcn_readfirstlane(s_e), cnt = __builtin_amdgcn_readfirstlane(s_cnt);

    const int k0 = kq * GV_KPART, klen = min(GV_KPART, a.K - k0);
    const int KTp = klen / 16, NT = a.N / 16;
    const int tau = lane >> 3, cp = lane & 7;
    const int src_lane = cp == 0 ? lane + 7 : lane - 1;
    const int mw = wave / WPM, kw = wave % WPM;   // this wave's matrix and its K slot
    const int64_t* wtab = (NMAT == 2 && mw == 1) ? a.wptr1 : a.wptr0;
    const size_t row_stride = (size_t)NT * 24;   // dwords between tile rows
    // the matrix base is wave-uniform; readfirstlane puts it (and so the descriptor) in SGPRs. readfirstlane
    // returns int: each half goes through uint32_t before widening, or a low word >= 2^31 would sign-extend
    // into the high word and the descriptor would point at a wild address.
    const uint64_t wp = (uint64_t)wtab[e];
    const uint32_t wlo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)wp);
    const uint32_t whi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(wp >> 32));
    const uint64_t wpu = (uint64_t)wlo | ((uint64_t)whi << 32);
    const __amdgpu_buffer_rsrc_t wres = __builtin_amdgcn_make_buffer_rsrc(
        reinterpret_cast<void*>((uintptr_t)wpu), (short)0, (int)((size_t)(a.K / 16) * row_stride * 4), BUF_DWORD3);
    const uint32_t voff = (uint32_t)(((cb * 8 + tau) * 24 + 3 * cp) * 4);      // bytes within a tile row
    const uint32_t row_bytes = (uint32_t)(row_stride * 4);
    constexpr int xrow = GV_KPART / 2;            // dwords per transformed input row in LDS

    for (int r0 = 0; r0 < cnt; r0 += MT)
    {
        const int nr = min(MT, cnt - r0);
        __syncthreads();
        // ---- prologue: transformed inputs (fp16) of this K part, rows r0 .. r0+nr-1
        uint16_t* xt = reinterpret_cast<uint16_t*>(lds);
        if constexpr (MODE == 0)
        {
            const int nblk = klen / 128;
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
                        const uint16_t* xr = a.xin + (size_t)tok * a.H + k0 + blk * 128;
                        const uint16_t* su = a.suh13 + ((size_t)e * 2 + m) * a.H + k0 + blk * 128;
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
                        uint16_t* dst = xt + ((size_t)m * MT + r) * GV_KPART + blk * 128;
                        dst[lane] = f2h(va[u]);
                        dst[lane + 64] = f2h(vb[u]);
                    }
                }
            }
        }
        else
        {
            const int nd = klen / 2;
            for (int i = threadIdx.x; i < nr * nd; i += GV_THREADS)
            {
                const int r = i / nd, c = i % nd;
                lds[r * xrow + c] = reinterpret_cast<const uint32_t*>(a.xin + (size_t)s_rows[r0 + r] * a.I + k0)[c];
            }
        }
        __syncthreads();

        // ---- main loop (specialised for the route count) and the waves' partial sums into LDS
        {
            const int nit = (KTp - kw + WPM - 1) / WPM;   // tile rows of this wave
            const uint32_t row0 = (uint32_t)(k0 / 16 + kw);
            const uint32_t* xm = lds + (size_t)mw * MT * xrow;
            float* red = reinterpret_cast<float*>(lds);
            const int col0 = tau * 16 + cp;
#define MM_ROWS_CASE(R) case R: if constexpr (R <= MT) gemv_rows<R>(wres, voff, row0, row_bytes, nit, WPM, kw, src_lane, xm, xrow, red, wave, col0, MT); break;
            switch (nr)
            {
                MM_ROWS_CASE(1)
                MM_ROWS_CASE(2)
                MM_ROWS_CASE(3)
                MM_ROWS_CASE(4)
                MM_ROWS_CASE(5)
                MM_ROWS_CASE(6)
                MM_ROWS_CASE(7)
                default: gemv_rows<MT>(wres, voff, row0, row_bytes, nit, WPM, kw, src_lane, xm, xrow, red, wave, col0, MT); break;
            }
#undef MM_ROWS_CASE
        }
        __syncthreads();
        const float* red = reinterpret_cast<const float*>(lds);
        for (int i = threadIdx.x; i < NMAT * nr * GV_COLS; i += GV_THREADS)
        {
            const int m = i / (nr * GV_COLS), r = (i / GV_COLS) % nr, c = i % GV_COLS;
            float sum = 0.0f;
#pragma unroll
            for (int w = 0; w < WPM; ++w) sum += red[((size_t)(m * WPM + w) * MT + r) * GV_COLS + c];
            const int s = s_rows[r0 + r];
            a.part[(((size_t)kq * a.n + s) * NMAT + m) * a.N + cb * GV_COLS + c] = sum;
        }
    }
}

// Gate/up epilogue, one wave per (route, 128-column block of I): K parts added in order, output transforms,
// SwiGLU, down-input transform -> xd fp16 [n][I].
struct GuEpiArgs
{
    const float* part;        // [kparts][n][2][I]
    const int64_t* ids;
    const uint16_t* svh13;    // [E][2][I]
    const uint16_t* suh2;     // [E][I]
    uint16_t* xd;
    int n, E, I, kparts;
    float limit;
};

__global__ __launch_bounds__(256) void k_gu_epilogue(GuEpiArgs a)
{
    const int lane = threadIdx.x & 63;
    const int item = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int ncb = a.I / GV_COLS;
    const int s = item / ncb, cb = item % ncb;
    if (s >= a.n) return;
    const int64_t e = a.ids[s];
    if (e < 0 || e >= a.E) return;
    const int c = cb * GV_COLS;
    float ga = 0.f, gb = 0.f, ua = 0.f, ub = 0.f;
    for (int q = 0; q < a.kparts; ++q)
    {
        const float* pg = a.part + (((size_t)q * a.n + s) * 2 + 0) * a.I + c;
        const float* pu = a.part + (((size_t)q * a.n + s) * 2 + 1) * a.I + c;
        ga += pg[lane]; gb += pg[lane + 64];
        ua += pu[lane]; ub += pu[lane + 64];
    }
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

// Down epilogue of one (route, 128-column block of H): K parts added in order, then the output transform.
__device__ __forceinline__ void down_block(const float* part, int kparts, int n, int H, int s, int c, const uint16_t* sv,
                                           int lane, float& ya, float& yb)
{
    ya = 0.f;
    yb = 0.f;
    for (int q = 0; q < kparts; ++q)
    {
        const float* pd = part + ((size_t)q * n + s) * H + c;
        ya += pd[lane];
        yb += pd[lane + 64];
    }
    out_block_wave(ya, yb, h2f(sv[lane]), h2f(sv[lane + 64]));
}

struct DEpiArgs
{
    const float* part;        // [kparts][n][H]
    const int64_t* ids;
    const float* w;           // route weights (combine kernel)
    const uint16_t* svh2;     // [E][H]
    float* Y;                 // [n][H]
    float* out;               // [T][H] (combine kernel)
    uint16_t* xnext;          // [T][H] fp16 or null (combine kernel)
    int n, E, H, kparts, topk, rescale;
};

__global__ __launch_bounds__(256) void k_d_epilogue(DEpiArgs a)
{
    const int lane = threadIdx.x & 63;
    const int item = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int ncb = a.H / GV_COLS;
    const int s = item / ncb, cb = item % ncb;
    if (s >= a.n) return;
    const int64_t e = a.ids[s];
    if (e < 0 || e >= a.E) return;
    const int c = cb * GV_COLS;
    float ya, yb;
    down_block(a.part, a.kparts, a.n, a.H, s, c, a.svh2 + (size_t)e * a.H + c, lane, ya, yb);
    a.Y[(size_t)s * a.H + c + lane] = ya;
    a.Y[(size_t)s * a.H + c + lane + 64] = yb;
}

// Down epilogue fused with the weighted combine and the next layer's input: one workgroup per token; a wave owns
// a 128-column block and adds the routes in ascending j with fp32 fma (the order of k_combine), so out equals
// the unfused path bit for bit.
__global__ __launch_bounds__(1024) void k_d_epilogue_combine(DEpiArgs a)
{
    __shared__ float red[16];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    const int t = blockIdx.x;
    const int ncb = a.H / GV_COLS;
    float ss = 0.0f;
    for (int cb = wave; cb < ncb; cb += nw)
    {
        const int c = cb * GV_COLS;
        float oa = 0.f, ob = 0.f;
        for (int j = 0; j < a.topk; ++j)
        {
            const int s = t * a.topk + j;
            const int64_t e = a.ids[s];
            if (e < 0 || e >= a.E) continue;
            float ya, yb;
            down_block(a.part, a.kparts, a.n, a.H, s, c, a.svh2 + (size_t)e * a.H + c, lane, ya, yb);
            const float wj = a.w[s];
            oa = fmaf(wj, ya, oa);
            ob = fmaf(wj, yb, ob);
        }
        a.out[(size_t)t * a.H + c + lane] = oa;
        a.out[(size_t)t * a.H + c + lane + 64] = ob;
        ss = fmaf(oa, oa, ss);
        ss = fmaf(ob, ob, ss);
    }
    if (!a.xnext) return;
    float scale = 1.0f;
    if (a.rescale)
    {
        for (int d = 32; d >= 1; d >>= 1) ss += __shfl_xor(ss, d, 64);
        if (lane == 0) red[wave] = ss;
        __syncthreads();
        float tot = 0.0f;
        for (int i = 0; i < nw; ++i) tot += red[i];
        scale = tot > 0.0f ? 1.0f / sqrtf(tot / (float)a.H) : 1.0f;
    }
    else
        __syncthreads();
    __syncthreads();   // every wave's out columns are written before they are re-read below
    for (int h = threadIdx.x; h < a.H; h += blockDim.x)
    {
        uint32_t u = __float_as_uint(a.out[(size_t)t * a.H + h] * scale);
        if ((u & 0x7fffffffu) > 0x7f800000u) u |= 0x400000u;
        else u += 0x7fffu + ((u >> 16) & 1u);
        a.xnext[(size_t)t * a.H + h] = f2h(__uint_as_float(u & 0xffff0000u));
    }
}

static int pick_mt(int max_rows) { return max_rows <= 1 ? 1 : max_rows <= 2 ? 2 : max_rows <= 4 ? 4 : 8; }

template <int MODE>
static void launch_partial(const GemvArgs& a, int mt, hipStream_t s)
{
    const int blocks = a.max_active * a.ncb * a.kparts;
    switch (mt)
    {
        case 1: hipLaunchKernelGGL((k_expert_partial<MODE, 1>), dim3(blocks), dim3(GV_THREADS), 0, s, a); break;
        case 2: hipLaunchKernelGGL((k_expert_partial<MODE, 2>), dim3(blocks), dim3(GV_THREADS), 0, s, a); break;
        case 4: hipLaunchKernelGGL((k_expert_partial<MODE, 4>), dim3(blocks), dim3(GV_THREADS), 0, s, a); break;
        default: hipLaunchKernelGGL((k_expert_partial<MODE, 8>), dim3(blocks), dim3(GV_THREADS), 0, s, a); break;
    }
}

struct Ws
{
    float* part_gu;
    float* part_d;
    uint16_t* xd;
    size_t bytes;
};

static Ws carve(void* base, int n, int H, int I)
{
    auto al = [](size_t x) { return (x + 255) & ~(size_t)255; };
    const size_t kq = (H + GV_KPART - 1) / GV_KPART, kh = (I + GV_KPART - 1) / GV_KPART;
    const size_t b_gu = al(kq * n * 2 * I * 4), b_d = al(kh * n * H * 4), b_xd = al((size_t)n * I * 2);
    char* p = static_cast<char*>(base);
    return { reinterpret_cast<float*>(p), reinterpret_cast<float*>(p + b_gu), reinterpret_cast<uint16_t*>(p + b_gu + b_d),
             b_gu + b_d + b_xd };
}

static int check_common(const mm_layer_t* L, const void* x, int T, int n, int topk, const int64_t* ids,
                        const int32_t* offsets, const int32_t* order, const int32_t* active, const int32_t* nactive,
                        int max_rows, void* ws, size_t ws_bytes, const char* who)
{
    MM_CHECK_ARG(L && L->gate_ptr && L->up_ptr && L->down_ptr && L->suh13 && L->svh13 && L->suh2 && L->svh2,
                 "%s: incomplete layer", who);
    MM_CHECK_ARG(L->E > 0 && L->E <= 1024 && L->H > 0 && L->I > 0 && L->H % 128 == 0 && L->I % 128 == 0,
                 "%s: need 0 < E <= 1024 and H, I positive multiples of 128 (E=%d H=%d I=%d)", who, L->E, L->H, L->I);
    MM_CHECK_ARG(x && ids, "%s: null pointer", who);
    MM_CHECK_ARG(T > 0 && n > 0 && topk > 0 && n <= T * topk, "%s: bad T/n/topk", who);
    MM_CHECK_ARG(max_rows > 0 && max_rows <= GV_MAX_ROWS, "%s: max_rows must be in [1, %d]", who, GV_MAX_ROWS);
    const bool perm = offsets != nullptr;
    MM_CHECK_ARG(perm ? (order && active && nactive) : n <= GV_ROUTE_MAX,
                 "%s: more than %d routes need the permutation (offsets, order, active, nactive)", who, GV_ROUTE_MAX);
    MM_CHECK_ARG(ws && ws_bytes >= carve(nullptr, n, L->H, L->I).bytes, "%s: workspace too small (%zu < %zu)", who, ws_bytes,
                 carve(nullptr, n, L->H, L->I).bytes);
    return MM_OK;
}

static GemvArgs base_args(const mm_layer_t* L, int n, int topk, const int64_t* ids, const int32_t* offsets,
                          const int32_t* order, const int32_t* active, const int32_t* nactive)
{
    GemvArgs a{};
    a.suh13 = L->suh13;
    a.ids = ids; a.offsets = offsets; a.order = order; a.active = active; a.nactive = nactive;
    a.H = L->H; a.I = L->I; a.E = L->E; a.n = n; a.topk = topk;
    a.max_active = n < L->E ? n : L->E;
    return a;
}

static void run_gate_up(const mm_layer_t* L, GemvArgs a, const void* x, const Ws& w, int mt, hipStream_t s, int parts)
{
    a.wptr0 = L->gate_ptr; a.wptr1 = L->up_ptr; a.xin = (const uint16_t*)x; a.part = w.part_gu;
    a.K = L->H; a.N = L->I; a.ncb = L->I / GV_COLS; a.kparts = (L->H + GV_KPART - 1) / GV_KPART;
    if (parts & 1) launch_partial<0>(a, mt, s);
    GuEpiArgs g{ w.part_gu, a.ids, L->svh13, L->suh2, w.xd, a.n, L->E, L->I, a.kparts, L->limit };
    if (parts & 2) hipLaunchKernelGGL(k_gu_epilogue, dim3((a.n * (L->I / GV_COLS) + 3) / 4), dim3(256), 0, s, g);
}

static int run_down_partial(const mm_layer_t* L, GemvArgs a, const Ws& w, int mt, hipStream_t s, bool launch)
{
    a.wptr0 = L->down_ptr; a.wptr1 = nullptr; a.xin = w.xd; a.part = w.part_d;
    a.K = L->I; a.N = L->H; a.ncb = L->H / GV_COLS; a.kparts = (L->I + GV_KPART - 1) / GV_KPART;
    if (launch) launch_partial<1>(a, mt, s);
    return a.kparts;
}

}  // namespace mm

using namespace mm;

extern "C" {

size_t mm_gemv_workspace(int n, int E, int H, int I)
{
    (void)E;
    return carve(nullptr, n, H, I).bytes;
}

int mm_expert_gemv(const mm_layer_t* L, const void* x_fp16, int T, int n, int topk, const int64_t* ids,
                   const int32_t* offsets, const int32_t* order, const int32_t* active, const int32_t* nactive,
                   int max_rows, float* Y, void* workspace, size_t workspace_bytes, int phases, mm_stream_t stream)
{
    MM_CHECK_ARG(phases >= 1 && phases <= 15, "mm_expert_gemv: phases is a mask of 1, 2, 4, 8");
    const int rc = check_common(L, x_fp16, T, n, topk, ids, offsets, order, active, nactive, max_rows, workspace,
                                workspace_bytes, "mm_expert_gemv");
    if (rc) return rc;
    MM_CHECK_ARG(Y, "mm_expert_gemv: null Y");
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    const Ws w = carve(workspace, n, L->H, L->I);
    const int mt = pick_mt(max_rows);
    const GemvArgs a = base_args(L, n, topk, ids, offsets, order, active, nactive);
    if (phases & 3) run_gate_up(L, a, x_fp16, w, mt, s, phases & 3);
    if (phases & 12)
    {
        const int kh = run_down_partial(L, a, w, mt, s, (phases & 4) != 0);
        DEpiArgs d{ w.part_d, ids, nullptr, L->svh2, Y, nullptr, nullptr, n, L->E, L->H, kh, topk, 0 };
        if (phases & 8) hipLaunchKernelGGL(k_d_epilogue, dim3((n * (L->H / GV_COLS) + 3) / 4), dim3(256), 0, s, d);
    }
    return check_launch("mm_expert_gemv");
}

int mm_moe_decode(const mm_layer_t* L, const void* x_fp16, int T, int topk, const int64_t* ids, const float* w, int max_rows,
                  float* out, void* x_next_fp16, int rescale, void* workspace, size_t workspace_bytes, mm_stream_t stream)
{
    const int n = T * topk;
    const int rc = check_common(L, x_fp16, T, n, topk, ids, nullptr, nullptr, nullptr, nullptr, max_rows, workspace,
                                workspace_bytes, "mm_moe_decode");
    if (rc) return rc;
    MM_CHECK_ARG(w && out, "mm_moe_decode: null pointer");
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    const Ws ws = carve(workspace, n, L->H, L->I);
    const int mt = pick_mt(max_rows);
    const GemvArgs a = base_args(L, n, topk, ids, nullptr, nullptr, nullptr, nullptr);
    run_gate_up(L, a, x_fp16, ws, mt, s, 3);
    const int kh = run_down_partial(L, a, ws, mt, s, true);
    DEpiArgs d{ ws.part_d, ids, w, L->svh2, nullptr, out, (uint16_t*)x_next_fp16, n, L->E, L->H, kh, topk, rescale };
    hipLaunchKernelGGL(k_d_epilogue_combine, dim3(T), dim3(1024), 0, s, d);
    return check_launch("mm_moe_decode");
}

}  // extern "C"
