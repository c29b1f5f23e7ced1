// Fat-expert path (prefill): per-expert grouped GEMM with the EXL3 weights decoded into LDS and multiplied on
// MFMA, for experts that receive many routes (the reference's apply_exl3_batched_fat / run_batch,
// patches/vllm-exl3-host-dma.patch:182-201, runtime/dma_gemm.py:5-26, which reconstruct fp16 weights and run a
// 128x128 GEMM).
//
// A workgroup (8 waves) owns a tile of 128 routes (sorted positions of one expert) x 256 output columns:
//   gate/up (k_fat<0>): gate columns 128 c .. 128 c + 127 and the same up columns, so the epilogue holds both and
//                       applies the output transforms, SwiGLU and the down-input transform of that 128-block
//                       (the transforms act within 128-blocks);
//   down    (k_fat<1>): two 128-blocks of H; the epilogue applies the output transform and writes per-route rows.
// Per 32-row step (two tile rows) the workgroup loads the routes' transformed inputs (buffer-to-LDS, 4 steps
// ahead) and the 32 trellis tiles of its columns (768-byte rows, buffer-to-LDS, 12 steps ahead), every wave
// decodes 4 tiles into the MFMA B layout (fp16 weights rounded as the reference's EXACT expert), and each wave
// multiplies a 64 x 64 sub-tile on v_mfma_f32_16x16x32_f16. The weights are decoded once per 128 routes.
#include "mm_decode.h"

namespace mm {

constexpr int FT_BM = 128;          // routes per tile
constexpr int FT_BN = 256;          // output columns per tile
constexpr int FT_WAVES = 8;
constexpr int FT_THREADS = 64 * FT_WAVES;
constexpr int FT_PA = 4;            // input steps in flight
constexpr int FT_PT = 12;           // trellis steps in flight
constexpr int FT_TS = FT_PT + 1;    // trellis ring slots
constexpr int FT_PLAN_MAX = 1024;   // active experts the plan kernel handles

struct FatArgs
{
    const ExpertRec* rec;
    const int32_t* counts;        // [0] active experts
    const int32_t* tile_off;      // [max_active + 1] first tile of each active expert (exclusive prefix)
    const uint16_t* xa;           // mode 0: [n][2][H]; mode 1: [n][I] (operand order)
    const uint16_t* svh13;        // [E][2][I]
    const uint16_t* suh2;         // [E][I]
    const uint16_t* svh2;         // [E][H]
    const int32_t* route_at;      // [n]
    uint16_t* xd;                 // mode 0 output [n][I] (operand order)
    float* Y;                     // mode 1 output [n_routes][H] (per route)
    int H, I, K, N, nunits, max_active;
    float limit;
};

// Tiles of each active expert with more than cap routes: tile_off[a] = tiles of experts 0 .. a-1.
__global__ __launch_bounds__(FT_PLAN_MAX) void k_fat_plan(const ExpertRec* rec, const int32_t* counts, int32_t* tile_off,
                                                         int max_active, int cap)
{
    __shared__ int s_w[FT_PLAN_MAX / 64];
    const int a = threadIdx.x, lane = a & 63, wave = a >> 6;
    const int nact = counts[0];
    const int c = (a < nact && a < max_active) ? rec[a].cnt : 0;
    const int tiles = c > cap ? (c + FT_BM - 1) / FT_BM : 0;
    int incl = tiles;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1)
    {
        const int o = __shfl_up(incl, d, 64);
        if (lane >= d) incl += o;
    }
    if (lane == 63) s_w[wave] = incl;
    __syncthreads();
    int before = 0, total = 0;
    for (int w = 0; w < FT_PLAN_MAX / 64; ++w)
    {
        if (w < wave) before += s_w[w];
        total += s_w[w];
    }
    if (a < max_active) tile_off[a] = before + incl - tiles;
    if (a == 0) tile_off[max_active] = total;
}

template <int MODE>
__global__ __launch_bounds__(FT_THREADS, 1) void k_fat(FatArgs a)
{
    constexpr int NA = MODE == 0 ? 2 : 1;                        // input matrices (gate, up share the tile)
    constexpr int LA = 2 * NA;                                   // input loads per loader wave and step
    constexpr int A_STAGE = NA * FT_BM * 64;                     // bytes of one step's inputs
    constexpr int T_SLOT = 4 * 1024;                             // one step's trellis: 4 chunks of 8 tiles
    constexpr int B_BUF = 16 * 64 * 16;                          // decoded B of one step
    constexpr int A_BYTES = FT_PA * A_STAGE, T_BYTES = FT_TS * T_SLOT, B_BYTES = 2 * B_BUF;
    constexpr int C_STRIDE = FT_BN * 2 + 16;                     // epilogue tile row (fp16), padded
    constexpr int MAIN = A_BYTES + T_BYTES + B_BYTES;
    constexpr int SMEM = MAIN > FT_BM * C_STRIDE ? MAIN : FT_BM * C_STRIDE;
    static_assert(SMEM <= 160 * 1024, "LDS");
    __shared__ __align__(16) uint8_t smem[SMEM];
    uint8_t* Aring = smem;
    uint8_t* Tring = smem + A_BYTES;
    uint8_t* Bdec = smem + A_BYTES + T_BYTES;

    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    // ---- tile. Consecutive tiles (the column blocks of one 128-route block, then the next block of the same
    // expert) go to one XCD, so they share its L2 for the inputs and the trellis.
    const int nblk = gridDim.x;                                  // a multiple of 8
    const int L = (int)(blockIdx.x & 7) * (nblk >> 3) + (int)(blockIdx.x >> 3);
    const int nact = min(a.counts[0], a.max_active);
    const int total = a.tile_off[nact];
    const int mt = L / a.nunits, nu = L % a.nunits;
    if (mt >= total) return;
    int lo = 0, hi = nact - 1;
    while (lo < hi)
    {
        const int mid = (lo + hi + 1) >> 1;
        if (a.tile_off[mid] <= mt) lo = mid; else hi = mid - 1;
    }
    const ExpertRec* rp = a.rec + lo;
    const int row0 = (mt - a.tile_off[lo]) * FT_BM;
    const int rows = __builtin_amdgcn_readfirstlane(min(FT_BM, rp->cnt - row0));
    const int pos0 = __builtin_amdgcn_readfirstlane(rp->first + row0);
    const int e = __builtin_amdgcn_readfirstlane(rp->e);

    // ---- buffer descriptors (wave-uniform bases through readfirstlane, each half widened as uint32_t)
    auto uniform_ptr = [](const void* p) {
        const uint64_t v = (uint64_t)(uintptr_t)p;
        const uint32_t l = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)v);
        const uint32_t h = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(v >> 32));
        return reinterpret_cast<void*>((uintptr_t)((uint64_t)l | ((uint64_t)h << 32)));
    };
    const uint32_t a_row = (uint32_t)NA * a.K * 2;                       // bytes per route of the inputs
    const __amdgpu_buffer_rsrc_t ares = __builtin_amdgcn_make_buffer_rsrc(
        uniform_ptr(a.xa + (size_t)pos0 * NA * a.K), (short)0, (int)((uint32_t)rows * a_row), 0x00020000);
    const uint32_t row_bytes = (uint32_t)(a.N / 16) * 96, wbytes = (uint32_t)(a.K / 16) * row_bytes;
    // trellis loader waves 0 .. 3 move chunk q = wave of every step: tile row 2 s + (q >> 1) of matrix q & 1
    // (gate/up) or of column block 2 nu + (q & 1) (down), 8 tiles = 768 bytes
    const int tb = wave & 1, tt = (wave >> 1) & 1;
    const void* wbase = (const void*)(uintptr_t)(MODE == 0 ? (tb ? rp->w[1] : rp->w[0]) : rp->w[2]);
    const __amdgpu_buffer_rsrc_t wres = __builtin_amdgcn_make_buffer_rsrc(uniform_ptr(wbase), (short)0, (int)wbytes,
                                                                          0x00020000);
    const uint32_t wcol = MODE == 0 ? (uint32_t)nu * 768 : (uint32_t)(2 * nu + tb) * 768;
    auto load_trellis = [&](int s) {       // 12 bytes per lane, stored 16 bytes apart
        const uint32_t tr = (uint32_t)(2 * s + tt);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(wres, Tring + (size_t)(s % FT_TS) * T_SLOT + (size_t)wave * 1024, 12,
                                                 tr * row_bytes + wcol + (uint32_t)lane * 12, 0, 0, 0);
    };
    // input loader waves 4 .. 7: LA loads of 16 rows each (4 lanes per 64-byte row step). The 16-byte chunks of
    // row r sit at chunk ^ ((r >> 2) & 3) so the MFMA operand reads spread over the LDS banks. Rows past the
    // tile's routes are out of the descriptor's range and read as zero.
    auto load_inputs = [&](int s) {
        const int st = s % FT_PA;
#pragma unroll
        for (int u = 0; u < LA; ++u)
        {
            const int li = (wave - 4) * LA + u;                        // 0 .. 8 NA - 1
            const int am = li >> 3, rb = li & 7;
            const int r = rb * 16 + (lane >> 2), p = lane & 3;
            const uint32_t voff = (uint32_t)r * a_row + (uint32_t)am * a.K * 2 + (uint32_t)s * 64 +
                                  (uint32_t)(p ^ ((r >> 2) & 3)) * 16;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(ares, Aring + (size_t)st * A_STAGE + ((size_t)am * FT_BM + rb * 16) * 64,
                                                     16, voff, 0, 0, 0);
        }
    };

    // ---- decode: wave w owns chunk w >> 1 (tile row t, matrix or block b), tiles 4 (w & 1) .. + 3
    const int col = lane & 15, g = lane >> 4;
    const int i0 = 32 * (col & 7) + 8 * g + 4 * (col >> 3);
    const int eb = 3 * i0 + 11;
    const int blo = eb >> 5, bhi = (blo + 23) % 24;
    const int llo = 4 * (blo / 3) + blo % 3, lhi = 4 * (bhi / 3) + bhi % 3;
    const uint32_t sh = 31u - (uint32_t)(eb & 31);
    auto decode = [&](int s) {
        const int q = wave >> 1, t = q >> 1, b = q & 1;
        const uint32_t* slot = reinterpret_cast<const uint32_t*>(Tring + (size_t)(s % FT_TS) * T_SLOT + (size_t)q * 1024);
        uint8_t* bd = Bdec + (size_t)(s & 1) * B_BUF;
#pragma unroll
        for (int u = 0; u < 4; ++u)
        {
            const int c = (wave & 1) * 4 + u;
            const half4_t wv = decode4<true>(slot[c * 32 + lhi], slot[c * 32 + llo], sh);
            *reinterpret_cast<half4_t*>(bd + ((size_t)(b * 8 + c) * 64 + lane) * 16 + t * 8) = wv;
        }
    };
    // ---- MFMA sub-tile of wave w: rows 64 (w >> 2) .. + 63, column tiles 4 (w & 3) .. + 3 of the 16
    const int wm = wave >> 2, wn = wave & 3;
    const int am_mfma = MODE == 0 ? (wn >> 1) : 0;
    float4_t acc[4][4];
#pragma unroll
    for (int mb = 0; mb < 4; ++mb)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[mb][i] = float4_t{ 0.f, 0.f, 0.f, 0.f };
    auto mfma = [&](int s) {
        const uint8_t* as = Aring + (size_t)(s % FT_PA) * A_STAGE + (size_t)am_mfma * FT_BM * 64;
        const uint8_t* bs = Bdec + (size_t)(s & 1) * B_BUF;
        half8_t A[4], B[4];
#pragma unroll
        for (int mb = 0; mb < 4; ++mb)
        {
            const int r = wm * 64 + mb * 16 + col;
            A[mb] = *reinterpret_cast<const half8_t*>(as + (size_t)r * 64 + ((g ^ ((r >> 2) & 3)) * 16));
        }
#pragma unroll
        for (int i = 0; i < 4; ++i)
            B[i] = *reinterpret_cast<const half8_t*>(bs + ((size_t)(wn * 4 + i) * 64 + lane) * 16);
#pragma unroll
        for (int mb = 0; mb < 4; ++mb)
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[mb][i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[mb], B[i], acc[mb][i], 0, 0, 0);
    };

    // ---- main loop over 32-row steps. Loads run ahead: inputs of step s + FT_PA - 1 and trellis of step
    // s + FT_PT are issued in iteration s, into the ring slots that iteration s - 1 finished with. Iteration s
    // waits for its own loads (vmcnt counts in issue order), meets the other waves at the one barrier, multiplies
    // step s and decodes step s + 1 into the other B buffer.
    const int S = a.K / 32;
    if (wave < 4)
    {
        for (int s = 0; s < FT_PT && s < S; ++s) load_trellis(s);
        if (S >= FT_PT) wait_vmcnt<FT_PT - 1>(); else wait_vmcnt<0>();     // step 0 arrived
    }
    else
        for (int s = 0; s < FT_PA - 1 && s < S; ++s) load_inputs(s);
    __syncthreads();
    decode(0);
    for (int s = 0; s < S; ++s)
    {
        if (wave < 4)
        {
            if (s + FT_PT - 1 < S) wait_vmcnt<FT_PT - 2>(); else wait_vmcnt<0>();    // trellis of step s + 1
        }
        else
        {
            if (s + 2 < S) wait_vmcnt<(FT_PA - 2) * LA>();                           // inputs of step s
            else if (s + 1 < S) wait_vmcnt<LA>();
            else wait_vmcnt<0>();
        }
        __syncthreads();
        if (wave < 4)
        {
            if (s + FT_PT < S) load_trellis(s + FT_PT);
        }
        else if (s + FT_PA - 1 < S)
            load_inputs(s + FT_PA - 1);
        mfma(s);
        if (s + 1 < S) decode(s + 1);
    }
    __syncthreads();

    // ---- epilogue through an fp16 tile in LDS (the output transforms round y to fp16 first)
    uint8_t* C = smem;
#pragma unroll
    for (int mb = 0; mb < 4; ++mb)
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int v = 0; v < 4; ++v)
            {
                const int r = wm * 64 + mb * 16 + 4 * g + v, cc = (wn * 4 + i) * 16 + col;
                *reinterpret_cast<uint16_t*>(C + (size_t)r * C_STRIDE + cc * 2) = f2h(acc[mb][i][v]);
            }
    __syncthreads();
    for (int r = wave; r < rows; r += FT_WAVES)
    {
        const uint16_t* cr = reinterpret_cast<const uint16_t*>(C + (size_t)r * C_STRIDE);
        const int pos = pos0 + r;
        if constexpr (MODE == 0)
        {
            const int c0 = nu * 128;
            float ga = h2f(cr[lane]), gb = h2f(cr[lane + 64]);
            float ua = h2f(cr[128 + lane]), ub = h2f(cr[128 + lane + 64]);
            const uint16_t* svg = a.svh13 + ((size_t)e * 2 + 0) * a.I + c0;
            const uint16_t* svu = a.svh13 + ((size_t)e * 2 + 1) * a.I + c0;
            out_block_wave(ga, gb, h2f(svg[lane]), h2f(svg[lane + 64]));
            out_block_wave(ua, ub, h2f(svu[lane]), h2f(svu[lane + 64]));
            float xa = r16(act_gu(ga, ua, a.limit));
            float xb = r16(act_gu(gb, ub, a.limit));
            const uint16_t* sd = a.suh2 + (size_t)e * a.I + c0;
            prep_block_wave(xa, xb, h2f(sd[lane]), h2f(sd[lane + 64]));
            uint16_t* dst = a.xd + (size_t)pos * a.I;
            dst[operand_index(c0 + lane)] = f2h(xa);
            dst[operand_index(c0 + lane + 64)] = f2h(xb);
        }
        else
        {
            float* yr = a.Y + (size_t)a.route_at[pos] * a.H;
#pragma unroll
            for (int hb = 0; hb < 2; ++hb)
            {
                const int c0 = (2 * nu + hb) * 128;
                float ya = h2f(cr[hb * 128 + lane]), yb = h2f(cr[hb * 128 + lane + 64]);
                const uint16_t* sv = a.svh2 + (size_t)e * a.H + c0;
                out_block_wave(ya, yb, h2f(sv[lane]), h2f(sv[lane + 64]));
                yr[c0 + lane] = ya;
                yr[c0 + lane + 64] = yb;
            }
        }
    }
}

// Weighted combine of the fat routes: out[t] = (accumulate ? out[t] : 0) + sum_j w_j y_j over the routes j of
// token t whose expert has more than cap routes, fp32 fma in ascending j (with cap 0 this is mm_combine).
__global__ __launch_bounds__(256) void k_fat_combine(float* __restrict__ out, const float* __restrict__ Y,
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
        const float4 y = *reinterpret_cast<const float4*>(Y + (size_t)s * H + h);
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
    int32_t* pcounts;     // [2]  route prep
    int32_t* pos_of;      // [n]
    int32_t* route_at;    // [n]
    int32_t* e_at;        // [n]
    uint16_t* xa;         // [n][2][H]
    float* xsum;          // [n][2][nb]
    int32_t* tile_off;    // [min(n, E) + 1]
    uint16_t* xd;         // [n][I]
    float* Y;             // [n][H]
    size_t bytes;
};

static FatWs fat_carve(void* base, int n, int E, int H, int I)
{
    auto al = [](size_t x) { return (x + 255) & ~(size_t)255; };
    const size_t na = (size_t)(n < E ? n : E);
    const size_t pwsb = mm_permute_workspace(n, E);
    const size_t sizes[17] = { al((size_t)(E + 1) * 4), al((size_t)(E + 2) * 4), al((size_t)n * 4), al((size_t)E * 4), al(4),
                               al(pwsb), al(na * sizeof(ExpertRec)), al(2 * 4), al((size_t)n * 4), al((size_t)n * 4),
                               al((size_t)n * 4), al((size_t)n * 2 * H * 2), al((size_t)n * 2 * prep_blocks(H) * 4),
                               al((na + 1) * 4), al((size_t)n * I * 2), al((size_t)n * H * 4), 0 };
    char* p = static_cast<char*>(base);
    char* at[17];
    size_t off = 0;
    for (int i = 0; i < 17; ++i)
    {
        at[i] = p ? p + off : nullptr;
        off += sizes[i];
    }
    FatWs w;
    w.counts = (int32_t*)at[0]; w.offsets = (int32_t*)at[1]; w.order = (int32_t*)at[2]; w.active = (int32_t*)at[3];
    w.nactive = (int32_t*)at[4]; w.pws = at[5]; w.pws_bytes = pwsb; w.rec = (ExpertRec*)at[6]; w.pcounts = (int32_t*)at[7];
    w.pos_of = (int32_t*)at[8]; w.route_at = (int32_t*)at[9]; w.e_at = (int32_t*)at[10]; w.xa = (uint16_t*)at[11];
    w.xsum = (float*)at[12]; w.tile_off = (int32_t*)at[13]; w.xd = (uint16_t*)at[14]; w.Y = (float*)at[15];
    w.bytes = off;
    return w;
}

static int fat_check(const mm_layer_t* L, const void* x, int x_dtype, int T, int topk, const int64_t* ids, void* ws,
                     size_t ws_bytes, const char* who)
{
    MM_CHECK_ARG(L && L->gate_ptr && L->up_ptr && L->down_ptr && L->suh13 && L->svh13 && L->suh2 && L->svh2,
                 "%s: incomplete layer", who);
    MM_CHECK_ARG(L->E > 0 && L->E <= FT_PLAN_MAX && L->H % 256 == 0 && L->I % 128 == 0 && L->H > 0 && L->I > 0,
                 "%s: need 0 < E <= %d, H a multiple of 256 and I of 128", who, FT_PLAN_MAX);
    MM_CHECK_ARG((size_t)(L->H / 16) * (L->I / 16) * 96 < ((size_t)1 << 31), "%s: matrix larger than 2 GiB", who);
    MM_CHECK_ARG(x && ids, "%s: null pointer", who);
    MM_CHECK_ARG(x_dtype == MM_DTYPE_F16 || x_dtype == MM_DTYPE_BF16 || x_dtype == MM_DTYPE_F32,
                 "%s: x_dtype must be MM_DTYPE_F16, MM_DTYPE_BF16 or MM_DTYPE_F32", who);
    MM_CHECK_ARG(T > 0 && topk > 0 && (size_t)T * topk < ((size_t)1 << 30), "%s: bad T/topk", who);
    const size_t need = fat_carve(nullptr, T * topk, L->E, L->H, L->I).bytes;
    MM_CHECK_ARG(ws && ws_bytes >= need, "%s: workspace too small (%zu < %zu)", who, ws_bytes, need);
    return MM_OK;
}

// Permutation, route prep, plan and both GEMMs: Y rows of every route whose expert has more than cap routes.
static int fat_run(const mm_layer_t* L, const void* x, int x_dtype, int T, int topk, const int64_t* ids, int cap,
                   const FatWs& ws, hipStream_t s)
{
    const int n = T * topk, E = L->E, na = n < E ? n : E;
    int rc = mm_permute(ids, nullptr, n, topk, E, ws.counts, ws.offsets, ws.order, nullptr, nullptr, nullptr, ws.active,
                        ws.nactive, ws.pws, ws.pws_bytes, s);
    if (rc) return rc;
    PrepArgs p{ x, ids, ws.offsets, ws.order, ws.active, ws.nactive, L->gate_ptr, L->up_ptr, L->down_ptr, L->suh13,
                ws.rec, ws.pcounts, ws.pos_of, ws.route_at, ws.e_at, ws.xa, ws.xsum, n, topk, E, L->H, prep_blocks(L->H),
                x_dtype, 0 };
    launch_route_prep(p, s);
    hipLaunchKernelGGL(k_fat_plan, dim3(1), dim3(FT_PLAN_MAX), 0, s, ws.rec, ws.pcounts, ws.tile_off, na, cap);
    // tiles: at most one partial tile per active expert beyond the full ones
    const int tiles_max = (n + FT_BM - 1) / FT_BM + na;
    FatArgs g{ ws.rec, ws.pcounts, ws.tile_off, ws.xa, L->svh13, L->suh2, L->svh2, ws.route_at, ws.xd, ws.Y,
               L->H, L->I, L->H, L->I, L->I / 128, na, L->limit };
    auto grid = [&](int units) { return dim3((unsigned)(((size_t)tiles_max * units + 7) & ~(size_t)7)); };
    hipLaunchKernelGGL(k_fat<0>, grid(g.nunits), dim3(FT_THREADS), 0, s, g);
    FatArgs d = g;
    d.xa = ws.xd; d.K = L->I; d.N = L->H; d.nunits = L->H / 256;
    hipLaunchKernelGGL(k_fat<1>, grid(d.nunits), dim3(FT_THREADS), 0, s, d);
    return check_launch("fat path");
}

}  // namespace mm

using namespace mm;

extern "C" {

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
    return fat_run(L, x, x_dtype, T, topk, ids, cap, ws, s);
}

int mm_moe_prefill(const mm_layer_t* L, const void* x, int x_dtype, int T, int topk, const int64_t* ids, const float* w,
                   int cap, int accumulate, float* out, void* workspace, size_t workspace_bytes, mm_stream_t stream)
{
    const int rc = fat_check(L, x, x_dtype, T, topk, ids, workspace, workspace_bytes, "mm_moe_prefill");
    if (rc) return rc;
    MM_CHECK_ARG(w && out && cap >= 0, "mm_moe_prefill: null pointer or negative cap");
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    const FatWs ws = fat_carve(workspace, T * topk, L->E, L->H, L->I);
    const int r = fat_run(L, x, x_dtype, T, topk, ids, cap, ws, s);
    if (r) return r;
    const dim3 grid((unsigned)((L->H / 4 + 255) / 256), (unsigned)T);
    hipLaunchKernelGGL(k_fat_combine, grid, dim3(256), 0, s, out, ws.Y, ids, w, ws.counts, T, topk, L->H, L->E, cap,
                       accumulate);
    return check_launch("mm_moe_prefill");
}

}  // extern "C"
