// Decode expert path: EXL3 3-bpw trellis decode fused into a multi-token GEMV on gfx950, multiply-accumulate
// on MFMA.
//
// A layer runs as five launches on the caller's stream. Stream order is the only synchronisation (no fences,
// no atomics between workgroups), so every result is deterministic:
//   1. k_route_prep    one workgroup per (route, gate|up, 512 input rows): the route's sorted position (stable
//                      by expert, then route index), one record per active expert, and the route's transformed
//                      input xt = r16(FWHT128(x * suh) * HAD) in MFMA operand order, with its sums (the input
//                      conversion and the optional unit-RMS rescale happen here too).
//   2. k_partial<0>    gate/up partial sums, one launch that fills the GPU once: the work -- every
//                      (active expert, matrix, 128 output columns) segment of 256 tile rows -- is cut into
//                      equal runs of rows, one per wave, from the active-expert count on the device. A wave
//                      streams its rows (8 tiles = 768 contiguous bytes each) from HBM into a 4-deep
//                      wave-private LDS ring with buffer-to-LDS loads, decodes each tile in registers and
//                      multiplies two tile rows at a time on v_mfma_f32_16x16x32_f16 against the inputs of up
//                      to 16 routes (L2 reads, prefetched with the same depth).
//   3. k_gu_epilogue   per (route, 128 columns of I): the pieces added in order, output transforms, SwiGLU, the
//                      down-input transform (MFMA operand order) and its sums.
//   4. k_partial<1>    down partial sums, as 2.
//   5. k_down_combine  per (token, 128 columns of H): the pieces, output transform, weighted sum of the token's
//                      routes in ascending order; or k_down_y: per-route rows.
//
// Codebook (kernels/cpu_avx2/ft_core.h:75-83): w = fp16(fma(1024 + bytesum, KINV, KBIAS)). By default the
// weights are evaluated as the reference's AFFINE expert does (ft_core.h:267-293): MFMA accumulates
// S = sum x (1024 + bytesum) on the exact fp16 codes and the epilogue forms KINV * S + KBIAS * sum x, so no
// per-weight rounding is spent. With MM_LAYER_EXACT every weight is rounded to fp16 first (v_pk_fma_f16), the
// reference's EXACT expert (ft_core.h:977-1011). fp16 activations, fp32 accumulation, fp16 rounding at the
// reference's points in both.
#include "mm_decode.h"

namespace mm {

constexpr int GV_WAVES = 4;
constexpr int GV_THREADS = 64 * GV_WAVES;
constexpr int GV_COLS = 128;          // output columns per segment (8 tiles)
constexpr int GV_ROUTE_MAX = 1024;    // in-kernel routing limit (routes per call)
constexpr int GV_RING = 4;            // tile rows in flight per wave (even: rows go through MFMA in pairs)
static_assert(GV_RING % 2 == 0, "row pairs");
constexpr int ROW_BYTES = 8 * 96;     // one tile row of a segment
constexpr int WAVES_PER_CU = 24;      // partial kernels: 6 workgroups of 4 waves per CU (<= 80 VGPRs, 16 KB LDS)
constexpr int PREP_ROWS = 512;        // input rows per route-prep workgroup
constexpr int SS_LOADS = 16;          // route prep: row elements per thread loaded at once for the rescale
constexpr int MAX_TOPK = 16;

// Rows of a partial launch: nseg segments of KT tile rows each (KT a multiple of 8), in segment order, cut into
// nw runs of equal length (within 4 rows) that start and end on multiples of 4 rows, one per wave, so every wave
// streams as many rows as every other. A run that reaches the end of a segment goes on in the next one; the wave
// then computes one piece of each, and a segment's pieces are the runs that meet it, numbered from 0 in row
// order. nw is the launch's wave count, lowered where runs that short would cut a segment into more than cap
// pieces (the partial sums hold cap per segment): nw runs over Q quads of rows start in any K consecutive quads
// at most ceil(K nw / Q) times, so with nw <= (cap - 1) Q / K a segment of K quads meets at most cap runs.
// Kernels 2-5 derive the split from the same inputs, so they agree on the layout of the partial sums.
struct RowSplit
{
    int64_t quads;
    int nw;
};
__device__ __forceinline__ RowSplit row_split(int nwaves, int nseg, int KT, int cap)
{
    const int64_t quads = (int64_t)nseg * (KT / 4);
    const int64_t most = (int64_t)(cap - 1) * nseg;      // (cap - 1) quads / (KT / 4)
    int64_t nw = nwaves;
    nw = nw < quads ? nw : quads;
    nw = nw < most ? nw : most;
    return { quads, (int)nw };
}
// floor(x / d) for 0 <= x < 2^53 and 0 < d < 2^31, in fp64: both operands convert exactly and the division
// rounds correctly, and a quotient below an integer k falls short of it by at least 1 / d, far more than half an
// ulp of k, so the rounded quotient never reaches k (a few fp64 instructions where an int64 division takes about
// a hundred)
__device__ __forceinline__ int floor_div(int64_t x, int64_t d) { return (int)floor((double)x / (double)d); }
// first quad of wave w's run (w <= nw)
__device__ __forceinline__ int run_start(const RowSplit& s, int w) { return floor_div((int64_t)w * s.quads, s.nw); }
// the wave whose run holds quad q
__device__ __forceinline__ int run_of(const RowSplit& s, int64_t q) { return floor_div((q + 1) * s.nw - 1, s.quads); }
// (a wave-uniform count: computed on the vector unit, returned as a scalar so the branches on it stay scalar)
__device__ __forceinline__ int seg_pieces(const RowSplit& s, int seg, int KT)
{
    if (s.nw <= 0) return 1;      // no rows: the one piece a caller may read is left out by it
    return __builtin_amdgcn_readfirstlane(run_of(s, (int64_t)(seg + 1) * (KT / 4) - 1) -
                                          run_of(s, (int64_t)seg * (KT / 4)) + 1);
}

// ------------------------------------------------------------------------------------------ 1. route prep

// Every load that does not depend on another is issued before the first barrier, with no branch in between (the
// route's id, all ids for the position, the token row for the rescale, this wave's block of it; the loads that need
// the expert follow with clamped indices, before the row's sum of squares is formed), and the routing counts and
// the row's sum of squares share one reduction, so the kernel costs about two memory round trips. XD = the input's element type.
template <int XD>
__device__ __forceinline__ float load_x_t(const void* x, size_t i)
{
    if constexpr (XD == MM_DTYPE_F16) return h2f(static_cast<const uint16_t*>(x)[i]);
    if constexpr (XD == MM_DTYPE_BF16) return __uint_as_float((uint32_t) static_cast<const uint16_t*>(x)[i] << 16);
    return static_cast<const float*>(x)[i];
}

template <int XD>
__global__ __launch_bounds__(256) void k_route_prep(PrepArgs a)
{
    __shared__ uint32_t s_bm[32];
    __shared__ int s_cnt[4][4];
    __shared__ float s_ss[4];
    __shared__ int s_ai;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int blk = blockIdx.x % a.nb, m = (blockIdx.x / a.nb) & 1, idx = blockIdx.x / (2 * a.nb);
    const bool writer = m == 0 && blk == 0;      // the one workgroup of a route that writes its routing data
    const bool perm = a.offsets != nullptr;
    // routing from the permutation: the workgroups of index idx own sorted position idx
    const int nvalid_perm = perm ? a.offsets[a.E] : 0;
    const int s = perm ? a.order[idx] : idx;
    const int64_t e64 = a.ids[s];
    const int t = s / a.topk;
    const size_t row = (size_t)t * a.H;
    const int h0 = blk * PREP_ROWS + wave * 128;
    const int hc = h0 < a.H ? h0 : 0;           // a block in range for the loads (h0 is wave-uniform)
    float va = load_x_t<XD>(a.x, row + hc + lane), vb = load_x_t<XD>(a.x, row + hc + lane + 64), ss = 0.f;
    // the ids for the in-kernel routing (at most GV_ROUTE_MAX = 4 x 256 routes; indices past n reload id n - 1)
    int64_t rid[GV_ROUTE_MAX / 256];
#pragma unroll
    for (int k = 0; k < GV_ROUTE_MAX / 256; ++k) rid[k] = a.ids[min(tid + 256 * k, a.n - 1)];
    // with a permutation: the active experts (ascending, at most E <= 4 x 256), searched for the route's expert
    int32_t act[4] = { -1, -1, -1, -1 };
    int nact_perm = 0;
    if (perm && writer)
    {
        nact_perm = a.nactive_in[0];
#pragma unroll
        for (int k = 0; k < 4; ++k) act[k] = a.active[min(tid + 256 * k, a.E - 1)];
    }
    // the row for its sum of squares: h = tid + 256 j, the first SS_LOADS of them issued here with the other first
    // loads (rows up to 256 SS_LOADS elements in one round trip), summed below in the same order
    float xr[SS_LOADS];
    if (a.rescale)
#pragma unroll
        for (int j = 0; j < SS_LOADS; ++j) xr[j] = load_x_t<XD>(a.x, row + min(tid + 256 * j, a.H - 1));
    const bool valid = perm ? idx < nvalid_perm : (e64 >= 0 && e64 < a.E);
    const int e = valid ? (int)e64 : -1;
    const int ec = valid ? e : 0;               // an expert in range for the loads
    const uint16_t* su = a.suh13 + ((size_t)ec * 2 + m) * a.H;
    const float sa = h2f(su[hc + lane]), sb = h2f(su[hc + lane + 64]);
    // the expert's route count from the permutation (the in-kernel routing counts it below)
    const int pcnt = perm ? a.offsets[ec + 1] - a.offsets[ec] : 0;
    // the record's matrix addresses, loaded by the thread that may write it
    int64_t wt0 = 0, wt1 = 0, wt2 = 0;
    if (tid == 0 && writer && valid)
    {
        wt0 = a.wtab0[e];
        wt1 = a.wtab1[e];
        wt2 = a.wtab2[e];
    }
    if (a.rescale)
    {
#pragma unroll
        for (int j = 0; j < SS_LOADS; ++j)
            if (tid + 256 * j < a.H) ss = fmaf(xr[j], xr[j], ss);
        for (int h = tid + 256 * SS_LOADS; h < a.H; h += 256)
        {
            const float v = load_x_t<XD>(a.x, row + h);
            ss = fmaf(v, v, ss);
        }
    }
    if (tid < 32) s_bm[tid] = 0;
    if (tid == 0) s_ai = -1;
    __syncthreads();
#pragma unroll
    for (int k = 0; k < 4; ++k)
        if (tid + 256 * k < nact_perm && act[k] == e) s_ai = tid + 256 * k;     // one match at most
    // in-kernel routing: position = routes of lower experts + earlier routes of the same expert
    int less = 0, same = 0, rank = 0, nv = 0;
#pragma unroll
    for (int k = 0; k < GV_ROUTE_MAX / 256; ++k)
    {
        const int64_t v = rid[k];
        const int i = tid + 256 * k;
        if (perm || i >= a.n || v < 0 || v >= a.E) continue;
        atomicOr(&s_bm[v >> 5], 1u << (v & 31));
        nv += 1;
        less += v < e;
        same += v == e;
        rank += (v == e) && (i < s);
    }
    less = wave_sum_int(less);
    same = wave_sum_int(same);
    rank = wave_sum_int(rank);
    nv = wave_sum_int(nv);
    ss = wave_sum(ss);
    if (lane == 0)
    {
        s_cnt[wave][0] = less;
        s_cnt[wave][1] = same;
        s_cnt[wave][2] = rank;
        s_cnt[wave][3] = nv;
        s_ss[wave] = ss;
    }
    __syncthreads();
    less = s_cnt[0][0] + s_cnt[1][0] + s_cnt[2][0] + s_cnt[3][0];
    same = s_cnt[0][1] + s_cnt[1][1] + s_cnt[2][1] + s_cnt[3][1];
    rank = s_cnt[0][2] + s_cnt[1][2] + s_cnt[2][2] + s_cnt[3][2];
    nv = s_cnt[0][3] + s_cnt[1][3] + s_cnt[2][3] + s_cnt[3][3];
    const int pos = perm ? idx : less + rank;
    // an expert with more than cap routes belongs to the fat-expert path: its positions stay reserved, but it gets
    // an empty record and its routes no transformed inputs and no outputs
    const bool fat = valid && (perm ? pcnt : same) > a.cap;
    // in-kernel routing: the experts present below the route's expert (its record index) and in all, from the
    // bitmap by one reduction over the first wave
    int below = 0, present = 0;
    if (!perm && wave == 0 && (writer || blockIdx.x == 0))
    {
        const uint32_t wd = lane < 32 ? s_bm[lane] : 0u;
        const int eb = valid ? (e >> 5) : -1;
        below = wave_sum_int(lane < eb ? __popc(wd) : (lane == eb ? __popc(wd & ((1u << (e & 31)) - 1u)) : 0));
        present = wave_sum_int(__popc(wd));
    }
    if (tid == 0 && (writer || blockIdx.x == 0))
    {
        if (blockIdx.x == 0)
        {
            a.counts[0] = perm ? a.nactive_in[0] : present;
            a.counts[1] = perm ? nvalid_perm : nv;
        }
        if (writer)
        {
            // the expert's active index: experts present below it (in-kernel routing), or its place in the
            // permutation's active list (-1 if absent there)
            const int ai = !valid ? -1 : (perm ? s_ai : below);
            a.pos_of[s] = valid && !fat ? pos : -1;
            a.ai_of[s] = valid && !fat ? ai : -1;
            if (valid)
            {
                a.route_at[pos] = s;
                a.e_at[pos] = fat ? -1 : e;
                a.ai_at[pos] = fat ? -1 : ai;
                // the expert's first route writes its record
                const bool first_route = perm ? pos == a.offsets[e] : rank == 0;
                if (first_route && ai >= 0)
                {
                    const int cnt = perm ? a.offsets[e + 1] - pos : same;
                    ExpertRec r{ e, fat ? 0 : cnt, pos, 0, { wt0, wt1, wt2 }, 0 };
                    a.rec[ai] = r;
                }
            }
        }
    }
    if (!valid || fat) return;

    // the route's expert input: x16 = fp16(bf16(x_t * s_t)) (fp16 input without rescale is taken as is);
    // s_t = 1 / RMS(x_t), the per-wave sums added as mm_prepare_input adds them
    float scale = 1.0f;
    if (a.rescale)
    {
        const float tot = (s_ss[0] + s_ss[1]) + (s_ss[2] + s_ss[3]);
        scale = tot > 0.0f ? 1.0f / sqrtf(tot / (float)a.H) : 1.0f;
    }
    __syncthreads();      // s_ss is reused below
    float bsum = 0.0f;
    if (h0 < a.H)
    {
        if (!(XD == MM_DTYPE_F16 && !a.rescale))
        {
            va = r16(bf16_value(va * scale));
            vb = r16(bf16_value(vb * scale));
        }
        prep_block_wave(va, vb, sa, sb);
        uint16_t* dst = a.xa + ((size_t)pos * 2 + m) * a.H;
        dst[operand_index(h0 + lane)] = f2h(va);
        dst[operand_index(h0 + lane + 64)] = f2h(vb);
        bsum = wave_sum(va + vb);
    }
    if (lane == 0) s_ss[wave] = bsum;
    __syncthreads();
    if (tid == 0) a.xsum[((size_t)pos * 2 + m) * a.nb + blk] = (s_ss[0] + s_ss[1]) + (s_ss[2] + s_ss[3]);
}

// ------------------------------------------------------------------------------------ 2/4. partial sums

struct PartArgs
{
    const ExpertRec* rec;
    const int32_t* counts;
    const uint16_t* xa;       // mode 0: [n][2][K]; mode 1: [n][K] (operand order)
    float* part;              // [pieces][npos][nmat][N]
    int npos, K, N, ncb, cap; // npos: sorted positions the workspace holds
};

// One pass of a partial-sum wave (k_partial): r0 of the run's rows [tr0, tr0 + nrow) of segment seg.
struct Pass
{
    __amdgpu_buffer_rsrc_t wres;     // the pass's matrix
    uint32_t wcol;                   // byte offset of the segment's 768-byte column chunk in a tile row
    int seg, piece, tr0, nrow, r0, nr, first, cnt, m, cb;
};

template <int MODE, bool EXACT>
__global__ __launch_bounds__(GV_THREADS, 6) void k_partial(PartArgs a)
{
    constexpr int NMAT = MODE == 0 ? 2 : 1;
    // A 12-byte buffer-to-LDS load writes lane i's bytes at slot + 16 i (the fourth dword of each lane's 16 is
    // left untouched), so a tile row occupies 1024 bytes: tile c's dword w sits at dword 32 c + 4 (w / 3) + w % 3.
    constexpr int SLOT = 256;                     // dwords per ring slot
    __shared__ __align__(16) uint32_t ring[GV_WAVES * GV_RING * SLOT];

    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    // consecutive runs (the pieces of one segment, then adjacent 768-byte column chunks: the same inputs) go to
    // one XCD; workgroups are dealt to the 8 XCDs round-robin
    const int nb = gridDim.x;
    const int b = (nb & 7) == 0 ? (int)(blockIdx.x & 7) * (nb >> 3) + (int)(blockIdx.x >> 3) : (int)blockIdx.x;
    const int nwaves = nb * GV_WAVES;
    const int KT = a.K / 16, NT = a.N / 16;
    const RowSplit split = row_split(nwaves, a.counts[0] * NMAT * a.ncb, KT, a.cap);
    const int w = b * GV_WAVES + wave;
    if (w >= split.nw) return;
    const uint32_t row_bytes = (uint32_t)NT * 96;
    const uint32_t wbytes = (uint32_t)KT * row_bytes;                   // one matrix
    const uint32_t xbytes = (uint32_t)((size_t)a.npos * NMAT * a.K * 2);   // the input array
    const __amdgpu_buffer_rsrc_t xres = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(a.xa), (short)0,
                                                                          (int)xbytes, 0x00020000);
    // lane constants of the decode
    const int col = lane & 15, g = lane >> 4;
    const int i0 = 32 * (col & 7) + 8 * g + 4 * (col >> 3);
    const int eb = 3 * i0 + 11;
    const int blo = eb >> 5, bhi = (blo + 23) % 24;
    const int llo = 4 * (blo / 3) + blo % 3, lhi = 4 * (bhi / 3) + bhi % 3;     // their places in a staged tile
    const uint32_t sh = 31u - (uint32_t)(eb & 31);

    // The run's passes, in row order: for each segment the run meets, one pass per 16 routes of the segment's
    // expert over the run's rows of that segment (its piece). The ring's loads run GV_RING rows ahead of the
    // multiplies and, past the end of a pass, fetch the next pass's first rows: pieces start and end on multiples
    // of 4 rows, so row i of the next pass lands in ring slot i % GV_RING as its own first loads would put it,
    // and a wave streams its whole run without a pause between passes.

    // This lane's input row of pass P (route position, matrix) and k-group: routes past nr repeat a valid one
    // and their outputs are never stored. Computed from an opaque copy of the lane index, so none of it is
    // computed ahead and held across the loop.
    auto xoff_of = [&](const Pass& P) {
        int l = lane;
        asm volatile("" : "+v"(l));
        const int pos = P.first + P.r0 + max(0, min(l & 15, P.nr - 1));
        return (uint32_t)(((size_t)pos * NMAT + P.m) * a.K * 2) + (uint32_t)(l >> 4) * 16;
    };
    const int end = 4 * (int)run_start(split, w + 1);
    // the run's first segment and this wave's piece of it; every later segment the run meets starts inside the
    // run, so the wave computes its piece 0
    const int seg0 = 4 * run_start(split, w) / KT, piece0 = w - run_of(split, (int64_t)seg0 * (KT / 4));
    // pass r0 of the run's rows [tr0, tr0 + nrow) of segment seg; nr = 0 if its expert has no routes past r0
    auto load_pass = [&](int seg, int tr0, int nrow, int r0) {
        Pass P;
        P.seg = seg;
        P.tr0 = tr0;
        P.nrow = nrow;
        P.r0 = r0;
        P.piece = seg == seg0 ? piece0 : 0;
        P.cb = seg % a.ncb;
        const int r = seg / a.ncb;
        P.m = r % NMAT;
        const int ai = r / NMAT;
        // fields read through the pointer (a local copy indexed by the runtime matrix would live in scratch), in
        // the constant address space: the records do not change during the launch, so the reads are scalar loads,
        // which the ring's vector-load waits do not count
        typedef __attribute__((address_space(4))) const ExpertRec ConstRec;
        ConstRec* rc = (ConstRec*)(a.rec + ai);
        P.cnt = rc->cnt;
        P.first = rc->first;
        // per-matrix buffer descriptor in SGPRs. readfirstlane returns int: each half goes through uint32_t
        // before widening, or a low word >= 2^31 would sign-extend into the high word.
        const uint64_t wp = (uint64_t)rc->w[MODE == 0 ? P.m : 2];
        const uint32_t wlo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)wp);
        const uint32_t whi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(wp >> 32));
        P.wres = __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void*>((uintptr_t)((uint64_t)wlo | ((uint64_t)whi << 32))),
                                                   (short)0, (int)wbytes, 0x00020000);
        P.wcol = (uint32_t)P.cb * ROW_BYTES;
        P.nr = max(0, min(16, P.cnt - r0));
        return P;
    };
    // the pass after P in this run, skipping segments of experts without routes; none: nr = nrow = 0 (its loads
    // are then the empty ones, on P's matrix)
    auto next_pass = [&](const Pass& P) {
        if (P.r0 + 16 < P.cnt) return load_pass(P.seg, P.tr0, P.nrow, P.r0 + 16);
        Pass Q = P;
        Q.nr = 0;
        for (int seg = P.seg + 1, row = seg * KT; row < end; ++seg, row += KT)
        {
            Q = load_pass(seg, 0, min(KT, end - row), 0);
            if (Q.nr > 0) break;
        }
        if (Q.nr == 0) Q.nrow = 0;
        return Q;
    };
    // the current pass, carried from one pass to the next as four plain integers (its segment, first row, row
    // count and first route) and rebuilt from them, so the loop carries nothing else
    int cseg, ctr0, cnrow, cr0;
    {
        const int row = 4 * (int)run_start(split, w), seg = row / KT, tr0 = row - seg * KT;
        Pass P = load_pass(seg, tr0, min(KT - tr0, end - row), 0);
        if (P.nr == 0) P = next_pass(P);
        if (P.nr == 0) return;
        cseg = P.seg;
        ctr0 = P.tr0;
        cnrow = P.nrow;
        cr0 = P.r0;
    }

    uint2 areg[GV_RING];
    // row t of pass P: one 768-byte trellis load into ring slot j and the lane's 8 input bytes (xo = xoff_of(P)).
    // Rows past the pass are issued with offsets beyond the buffers, which the buffer unit answers with zeros and
    // no memory access, so every row keeps the same two loads and the waits stay uniform.
    auto issue = [&](const Pass& P, uint32_t xo, int j, int t) {
        const bool in = t < P.nrow;
        const uint32_t tr = (uint32_t)(P.tr0 + t);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(P.wres, &ring[(wave * GV_RING + j) * SLOT], 12, (uint32_t)lane * 12,
                                                 in ? tr * row_bytes + P.wcol : wbytes, 0, 0);
        // operand order: tile row tr's 4 inputs of k-group g at byte 64 (tr / 2) + 16 g + 8 (tr % 2)
        const uint32_t xrow = (tr >> 1) * 64 + (tr & 1) * 8;
        areg[j] = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(xres, xo, in ? xrow : xbytes, 0));
    };
    {
        const Pass P = load_pass(cseg, ctr0, cnrow, cr0);
        const uint32_t xo = xoff_of(P);
#pragma unroll
        for (int j = 0; j < GV_RING; ++j) issue(P, xo, j, j);
    }
    for (;;)
    {
        const Pass cur = load_pass(__builtin_amdgcn_readfirstlane(cseg), __builtin_amdgcn_readfirstlane(ctr0),
                                   __builtin_amdgcn_readfirstlane(cnrow), __builtin_amdgcn_readfirstlane(cr0));
        const uint32_t xoff = xoff_of(cur);
        float4_t acc[8];
#pragma unroll
        for (int c = 0; c < 8; ++c) acc[c] = float4_t{ 0.f, 0.f, 0.f, 0.f };
        // rows j and j + 1 (ring slots) through one MFMA per tile
        auto pair_mma = [&](int j) {
            const uint32_t* s0 = &ring[(wave * GV_RING + j) * SLOT];
            const uint32_t* s1 = s0 + SLOT;
            const half4_t a0 = __builtin_bit_cast(half4_t, areg[j]), a1 = __builtin_bit_cast(half4_t, areg[j + 1]);
            const half8_t A = { a0[0], a0[1], a0[2], a0[3], a1[0], a1[1], a1[2], a1[3] };
#pragma unroll
            for (int c = 0; c < 8; ++c)
            {
                const half4_t b0 = decode4<EXACT>(s0[c * 32 + lhi], s0[c * 32 + llo], sh);
                const half4_t b1 = decode4<EXACT>(s1[c * 32 + lhi], s1[c * 32 + llo], sh);
                const half8_t B = { b0[0], b0[1], b0[2], b0[3], b1[0], b1[1], b1[2], b1[3] };
                acc[c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, B, acc[c], 0, 0, 0);
            }
        };
        // rows t and t + 1 hold the oldest 4 of the 2 GV_RING loads in flight; their slots are refilled with
        // rows t + GV_RING and t + GV_RING + 1 once the slots' LDS reads have returned. Pass lengths are multiples
        // of GV_RING, so the last GV_RING rows refill their slots with the next pass's first rows, each in the
        // slot its own first loads would use.
        for (int t0 = 0; t0 + GV_RING < cur.nrow; t0 += GV_RING)
        {
#pragma unroll
            for (int j = 0; j < GV_RING; j += 2)
            {
                wait_vmcnt<2 * (GV_RING - 2)>();
                pair_mma(j);
                wait_lgkm0();
                issue(cur, xoff, j, t0 + j + GV_RING);
                issue(cur, xoff, j + 1, t0 + j + 1 + GV_RING);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        // the next pass, looked up here: its record's load is waited for with the first pair's LDS reads
        const Pass nxt = next_pass(cur);
        {
            const uint32_t nxo = xoff_of(nxt);
#pragma unroll
            for (int j = 0; j < GV_RING; j += 2)
            {
                wait_vmcnt<2 * (GV_RING - 2)>();
                pair_mma(j);
                wait_lgkm0();
                issue(nxt, nxo, j, j);
                issue(nxt, nxo, j + 1, j + 1);
                __builtin_amdgcn_sched_barrier(0);
            }
        }

        // D layout: lane (column col, group g) holds routes 4g .. 4g+3 of column col of each tile; each store
        // writes 4 runs of 16 columns (64 bytes). The ring keeps streaming meanwhile. (Staging the rows through
        // LDS for 16-byte stores of whole rows was measured slower.)
        {
            // lane indices from an opaque copy, so nothing of this block is held across the loop
            int l = lane;
            asm volatile("" : "+v"(l));
            const int sg = l >> 4;
            float* dst = a.part + ((size_t)(cur.piece * a.npos + cur.first + cur.r0 + 4 * sg) * NMAT + cur.m) * a.N +
                         cur.cb * GV_COLS + (l & 15);
#pragma unroll
            for (int v = 0; v < 4; ++v)
                if (4 * sg + v < cur.nr)
#pragma unroll
                    for (int c = 0; c < 8; ++c) dst[(size_t)v * NMAT * a.N + 16 * c] = acc[c][v];
        }
        if (nxt.nr == 0) break;
        cseg = nxt.seg;
        ctr0 = nxt.tr0;
        cnrow = nxt.nrow;
        cr0 = nxt.r0;
    }
    wait_vmcnt<0>();      // the trailing (empty) loads, so the ring is quiet when the wave leaves
}

// ------------------------------------------------------------------------------------ 3. gate/up epilogue

// For each of NS streams i: a[i] += p[i][q * stride + lane], b[i] += p[i][q * stride + lane + 64] for
// q = 0 .. np[i] - 1 in ascending q. BATCH pieces of every stream are loaded before any is added (pieces past
// np[i] reload piece np[i] - 1 and are not added), so counts up to BATCH cost one memory round trip.
template <int NS, int BATCH>
__device__ __forceinline__ void sum_pieces_batched(const float* const (&p)[NS], size_t stride, const int (&np)[NS],
                                                   int most, int lane, float (&a)[NS], float (&b)[NS])
{
    for (int q0 = 0; q0 < most; q0 += BATCH)
    {
        float va[NS][BATCH], vb[NS][BATCH];
#pragma unroll
        for (int k = 0; k < BATCH; ++k)
#pragma unroll
            for (int i = 0; i < NS; ++i)
            {
                const float* pk = p[i] + (size_t)min(q0 + k, np[i] - 1) * stride;
                va[i][k] = pk[lane];
                vb[i][k] = pk[lane + 64];
            }
#pragma unroll
        for (int k = 0; k < BATCH; ++k)
#pragma unroll
            for (int i = 0; i < NS; ++i)
                if (q0 + k < np[i])
                {
                    a[i] += va[i][k];
                    b[i] += vb[i][k];
                }
    }
}

// Up to 8 pieces per stream (a call with at least 4 tokens at top-8 cuts segments into 8 or 9) in one round
// trip of 8 loads per stream, up to 12 in one of 12, more (calls of 1-3 tokens, up to 32 pieces) in round trips
// of 24.
template <int NS>
__device__ __forceinline__ void sum_pieces(const float* const (&p)[NS], size_t stride, const int (&np)[NS], int lane,
                                           float (&a)[NS], float (&b)[NS])
{
    int most = np[0];
#pragma unroll
    for (int i = 1; i < NS; ++i) most = max(most, np[i]);
    if (most <= 8)
        sum_pieces_batched<NS, 8>(p, stride, np, most, lane, a, b);
    else if (most <= 12)
        sum_pieces_batched<NS, 12>(p, stride, np, most, lane, a, b);
    else
        sum_pieces_batched<NS, 24>(p, stride, np, most, lane, a, b);
}

// Sum of p[0 .. count) by one wave, split so its first load shares a round trip with the loads after it:
// wave_sum_first loads lane's first element (0 past count) without using it; wave_sum_rest adds the lane's
// elements lane + 64, lane + 128, ... and reduces over the wave in a fixed order.
__device__ __forceinline__ float wave_sum_first(const float* p, int count, int lane)
{
    return p[min(lane, count - 1)];      // count >= 1; lanes past count are zeroed by wave_sum_rest
}
__device__ __forceinline__ float wave_sum_rest(const float* p, int count, int lane, float first)
{
    asm volatile("" : "+v"(first));      // first used here, not where it was loaded
    float v = lane < count ? 0.0f + first : 0.0f;
    for (int i = lane + 64; i < count; i += 64) v += p[i];
    return wave_sum(v);
}

struct GuEpiArgs
{
    const float* part;        // [pieces][n][2][I]
    const float* xsum;        // [n][2][nb]
    const int32_t* counts;
    const int32_t* e_at;
    const int32_t* ai_at;
    const uint16_t* svh13;    // [E][2][I]
    const uint16_t* suh2;     // [E][I]
    uint16_t* xd;             // [n][I] fp16 in operand order
    float* xdsum;             // [n][I / 128] sums of xd over each 128-column block
    int npos, H, I, nb, nwaves, cap, affine;
    float limit;
};

// One wave per (sorted position, 128-column block of I): pieces added in order (then the AFFINE fixup),
// output transforms, SwiGLU, the down-input transform.
__global__ __launch_bounds__(256) void k_gu_epilogue(GuEpiArgs a)
{
    const int lane = threadIdx.x & 63;
    const int item = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int ncb = a.I / GV_COLS;
    const int pos = item / ncb, cb = item % ncb;
    // round trip 1: the counts and the position's expert (read before the range check: only the last
    // workgroup's spare waves are past n, and they read position n - 1)
    const int nvalid = a.counts[1], nact = a.counts[0];
    // (the wave's position is one, so e and ai are too: read as scalars, the piece counts and the branches on
    // them below stay scalar)
    const int e = __builtin_amdgcn_readfirstlane(a.e_at[min(pos, a.npos - 1)]);
    const int ai = __builtin_amdgcn_readfirstlane(a.ai_at[min(pos, a.npos - 1)]);
    asm volatile("" ::"s"(nact), "s"(e), "s"(ai));      // one round trip, not the count after the branch below
    if (pos >= nvalid || e < 0 || ai < 0) return;      // past the routes, or a route of an expert above the cap
    const int KT = a.H / 16;
    const RowSplit split = row_split(a.nwaves, nact * 2 * ncb, KT, a.cap);
    const int np[2] = { seg_pieces(split, (ai * 2 + 0) * ncb + cb, KT), seg_pieces(split, (ai * 2 + 1) * ncb + cb, KT) };
    const int c = cb * GV_COLS;
    // round trip 2: scales, input sums and partial sums
    const uint16_t* svg = a.svh13 + ((size_t)e * 2 + 0) * a.I + c;
    const uint16_t* svu = a.svh13 + ((size_t)e * 2 + 1) * a.I + c;
    const uint16_t* sd = a.suh2 + (size_t)e * a.I + c;
    const float sga = h2f(svg[lane]), sgb = h2f(svg[lane + 64]), sua = h2f(svu[lane]), sub = h2f(svu[lane + 64]);
    const float sda = h2f(sd[lane]), sdb = h2f(sd[lane + 64]);
    const float* xsg = a.xsum + ((size_t)pos * 2 + 0) * a.nb;
    const float* xsu = a.xsum + ((size_t)pos * 2 + 1) * a.nb;
    float sg = 0.f, su = 0.f;
    if (a.affine)
    {
        sg = wave_sum_first(xsg, a.nb, lane);
        su = wave_sum_first(xsu, a.nb, lane);
    }
    const float* const pgu[2] = { a.part + ((size_t)pos * 2 + 0) * a.I + c, a.part + ((size_t)pos * 2 + 1) * a.I + c };
    float s0[2] = { 0.f, 0.f }, s1[2] = { 0.f, 0.f };
    sum_pieces<2>(pgu, (size_t)a.npos * 2 * a.I, np, lane, s0, s1);
    float ga = s0[0], gb = s1[0], ua = s0[1], ub = s1[1];
    if (a.affine)
    {
        sg = wave_sum_rest(xsg, a.nb, lane, sg);
        su = wave_sum_rest(xsu, a.nb, lane, su);
        const float ki = kinv_f(), kb = kbias_f();
        ga = fmaf(ki, ga, kb * sg);
        gb = fmaf(ki, gb, kb * sg);
        ua = fmaf(ki, ua, kb * su);
        ub = fmaf(ki, ub, kb * su);
    }
    out_block_wave(ga, gb, sga, sgb);
    out_block_wave(ua, ub, sua, sub);
    float xa = r16(act_gu(ga, ua, a.limit));
    float xb = r16(act_gu(gb, ub, a.limit));
    prep_block_wave(xa, xb, sda, sdb);
    uint16_t* dst = a.xd + (size_t)pos * a.I;
    dst[operand_index(c + lane)] = f2h(xa);
    dst[operand_index(c + lane + 64)] = f2h(xb);
    const float bs = wave_sum(xa + xb);
    if (lane == 0) a.xdsum[(size_t)pos * ncb + cb] = bs;
}

// ------------------------------------------------------------------------------------ 5. down epilogues

struct DEpiArgs
{
    const float* part;        // [pieces][n][H]
    const float* xdsum;       // [n][I / 128]
    const int32_t* counts;
    const int32_t* pos_of;
    const int32_t* route_at;
    const int32_t* e_at;
    const int32_t* ai_at;
    const int32_t* ai_of;
    const int64_t* ids;
    const float* w;           // route weights (combine)
    const uint16_t* svh2;     // [E][H]
    float* Y;                 // [n][H] (per-route rows)
    float* out;               // [T][H] (combine)
    int npos, H, I, topk, nwaves, cap, affine;
    int accumulate;           // combine: out += the sum instead of out = the sum
};

// Down output of one (sorted position, 128-column block of H): pieces added in order (then the AFFINE
// fixup), output transform.
// nact = active experts (counts[0]), read by the caller with its other first loads; the scales, input sums and
// partial sums then share one round trip.
__device__ __forceinline__ void down_block(const DEpiArgs& a, int nact, int ai, int pos, int c, int64_t e, int lane,
                                           float& ya, float& yb)
{
    const int KT = a.I / 16, ncb = a.H / GV_COLS;
    const RowSplit split = row_split(a.nwaves, nact * ncb, KT, a.cap);
    const int np[1] = { seg_pieces(split, ai * ncb + c / GV_COLS, KT) };
    const uint16_t* sv = a.svh2 + (size_t)e * a.H + c;
    const float sva = h2f(sv[lane]), svb = h2f(sv[lane + 64]);
    const float* xs = a.xdsum + (size_t)pos * (a.I / GV_COLS);
    float sx = a.affine ? wave_sum_first(xs, a.I / GV_COLS, lane) : 0.f;
    const float* const pd[1] = { a.part + (size_t)pos * a.H + c };
    float s0[1] = { 0.f }, s1[1] = { 0.f };
    sum_pieces<1>(pd, (size_t)a.npos * a.H, np, lane, s0, s1);
    ya = s0[0];
    yb = s1[0];
    if (a.affine)
    {
        sx = wave_sum_rest(xs, a.I / GV_COLS, lane, sx);
        const float ki = kinv_f(), kb = kbias_f();
        ya = fmaf(ki, ya, kb * sx);
        yb = fmaf(ki, yb, kb * sx);
    }
    out_block_wave(ya, yb, sva, svb);
}

// Per-route rows: Y[s] for every routed s.
__global__ __launch_bounds__(256) void k_down_y(DEpiArgs a)
{
    const int lane = threadIdx.x & 63;
    const int item = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int ncb = a.H / GV_COLS;
    const int pos = item / ncb, cb = item % ncb;
    const int nvalid = a.counts[1], nact = a.counts[0];
    const int pc = min(pos, a.npos - 1);
    // one position per wave: read as scalars
    const int s = __builtin_amdgcn_readfirstlane(a.route_at[pc]), e = __builtin_amdgcn_readfirstlane(a.e_at[pc]);
    const int ai = __builtin_amdgcn_readfirstlane(a.ai_at[pc]);
    asm volatile("" ::"s"(nact), "s"(s), "s"(e), "s"(ai));      // one round trip, not the count after the branch
    if (pos >= nvalid || e < 0 || ai < 0) return;
    const int c = cb * GV_COLS;
    float ya, yb;
    down_block(a, nact, ai, pos, c, e, lane, ya, yb);
    a.Y[(size_t)s * a.H + c + lane] = ya;
    a.Y[(size_t)s * a.H + c + lane + 64] = yb;
}

// Weighted combine: one workgroup per (token, 128-column block of H), wave j computes route j's output block,
// then out = sum_j w_j y_j with fp32 fma in ascending j over the routed j (the order of mm_combine, so the
// result equals mm_combine over the per-route rows bit for bit).
__global__ __launch_bounds__(1024) void k_down_combine(DEpiArgs a)
{
    __shared__ float ys[MAX_TOPK][GV_COLS];
    __shared__ float wj[MAX_TOPK];
    __shared__ int ok[MAX_TOPK];
    const int lane = threadIdx.x & 63, j = threadIdx.x >> 6;
    const int ncb = a.H / GV_COLS;
    const int t = blockIdx.x / ncb, c = (blockIdx.x % ncb) * GV_COLS;
    if (j < a.topk)
    {
        // round trip 1: the route's position, expert, active index and weight and the active-expert count. A pick
        // outside [0, E) (position -1) is computed on position 0 and expert 0 and left out of the sum, so no branch
        // keeps the expert's load from being issued with the others.
        const int s = t * a.topk + j;     // one route per wave: its fields are read as scalars
        const int pos = __builtin_amdgcn_readfirstlane(a.pos_of[s]), ai = __builtin_amdgcn_readfirstlane(a.ai_of[s]);
        const int64_t e = a.ids[s];
        const float wt = a.w[s];
        const int nact = a.counts[0];
        asm volatile("" ::"s"(nact), "s"(pos), "s"(ai), "v"(e), "v"(wt));     // all in one round trip
        float ya, yb;
        down_block(a, nact, pos >= 0 ? ai : 0, max(pos, 0), c, pos >= 0 ? e : 0, lane, ya, yb);
        ys[j][lane] = ya;
        ys[j][lane + 64] = yb;
        if (lane == 0)
        {
            ok[j] = pos >= 0;
            wj[j] = wt;
        }
    }
    __syncthreads();
    for (int h = threadIdx.x; h < GV_COLS; h += blockDim.x)
    {
        float* dst = a.out + (size_t)t * a.H + c + h;
        float o = a.accumulate ? *dst : 0.0f;
        for (int jj = 0; jj < a.topk; ++jj)
            if (ok[jj]) o = fmaf(wj[jj], ys[jj][h], o);
        *dst = o;
    }
}

// ------------------------------------------------------------------------------------------------- host

struct Ws
{
    ExpertRec* rec;
    int32_t* counts;
    int32_t* pos_of;
    int32_t* route_at;
    int32_t* e_at;
    uint16_t* xa;
    float* xsum;
    float* part_gu;
    uint16_t* xd;
    float* xdsum;
    float* part_d;
    int32_t* ai_at;
    int32_t* ai_of;
    size_t bytes;
};

int prep_blocks(int H) { return (H + PREP_ROWS - 1) / PREP_ROWS; }

void launch_route_prep(const PrepArgs& p, hipStream_t s)
{
    const dim3 grid(2 * p.npos * p.nb), block(256);
    if (p.x_dtype == MM_DTYPE_F16)
        hipLaunchKernelGGL(k_route_prep<MM_DTYPE_F16>, grid, block, 0, s, p);
    else if (p.x_dtype == MM_DTYPE_BF16)
        hipLaunchKernelGGL(k_route_prep<MM_DTYPE_BF16>, grid, block, 0, s, p);
    else
        hipLaunchKernelGGL(k_route_prep<MM_DTYPE_F32>, grid, block, 0, s, p);
}

// Most pieces per segment a partial launch may use: bounded so the partial sums stay a few MB.
static int piece_cap(int n)
{
    const int c = n > 0 ? 8192 / n : 32;
    return c > 32 ? 32 : (c < 4 ? 4 : c);
}

// Workspace of n routes whose sorted positions lie below npos (npos = n unless a caller bounds the positions).
static Ws carve(void* base, int n, int npos, int E, int H, int I)
{
    auto al = [](size_t x) { return (x + 255) & ~(size_t)255; };
    const size_t m = (size_t)npos;
    const size_t na = (size_t)(npos < E ? npos : E), cap = (size_t)piece_cap(npos);
    // the small routing arrays first and together (records, counts, pos_of, route_at, e_at, ai_at, ai_of), so the
    // epilogues' first loads fall in the same few pages
    const size_t sizes[13] = { al(na * sizeof(ExpertRec)), al(2 * 4), al((size_t)n * 4), al(m * 4),
                               al(m * 4), al(m * 4), al((size_t)n * 4), al(m * 2 * H * 2),
                               al(m * 2 * prep_blocks(H) * 4), al(cap * m * 2 * I * 4), al(m * I * 2),
                               al(m * (I / GV_COLS) * 4), al(cap * m * H * 4) };
    char* p = static_cast<char*>(base);
    char* at[13];
    size_t off = 0;
    for (int i = 0; i < 13; ++i)
    {
        at[i] = p ? p + off : nullptr;
        off += sizes[i];
    }
    Ws w;
    w.rec = reinterpret_cast<ExpertRec*>(at[0]);
    w.counts = reinterpret_cast<int32_t*>(at[1]);
    w.pos_of = reinterpret_cast<int32_t*>(at[2]);
    w.route_at = reinterpret_cast<int32_t*>(at[3]);
    w.e_at = reinterpret_cast<int32_t*>(at[4]);
    w.ai_at = reinterpret_cast<int32_t*>(at[5]);
    w.ai_of = reinterpret_cast<int32_t*>(at[6]);
    w.xa = reinterpret_cast<uint16_t*>(at[7]);
    w.xsum = reinterpret_cast<float*>(at[8]);
    w.part_gu = reinterpret_cast<float*>(at[9]);
    w.xd = reinterpret_cast<uint16_t*>(at[10]);
    w.xdsum = reinterpret_cast<float*>(at[11]);
    w.part_d = reinterpret_cast<float*>(at[12]);
    w.bytes = off;
    return w;
}

// Waves of one partial launch: the whole GPU once (WAVES_PER_CU per CU, a multiple of 8 workgroups), or half of
// that (three waves per SIMD) when the call's segments would otherwise be cut into more than 12 pieces each
// even with every route on an expert of its own (nseg_max = min(n, E) x matrices x column blocks): at one token
// and top-8 + 1 the 288 segments of a launch would take 21 pieces each, which the epilogues add in round trips
// of 24 loads; with half the waves they take 10-11, added in one round trip of 12, and the partial kernels run
// as fast with three waves per SIMD on runs twice as long (one-token step 4 % shorter). The partial kernel
// finds its wave count from its grid, and the epilogues are given the same value.
static int partial_waves(int64_t nseg_max)
{
    static int full = 0;
    if (!full)
    {
        int dev = 0, cus = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
            cus = 256;
        const int blocks = ((cus * WAVES_PER_CU / GV_WAVES) + 7) & ~7;
        full = blocks * GV_WAVES;
    }
    if ((int64_t)full > 12 * nseg_max)
        return (((full / GV_WAVES) / 2 + 7) & ~7) * GV_WAVES;
    return full;
}
// the segment bound of a partial launch of mode 0 (gate/up) or 1 (down) over n routes
static int64_t seg_max(const mm_layer_t* L, int n, int mode)
{
    const int64_t na = n < L->E ? n : L->E;
    return mode == 0 ? na * 2 * (L->I / GV_COLS) : na * (L->H / GV_COLS);
}

static int check_common(const mm_layer_t* L, const void* x, int x_dtype, int T, int n, int topk, const int64_t* ids,
                        const int32_t* offsets, const int32_t* order, const int32_t* active, const int32_t* nactive,
                        int max_rows, void* ws, size_t ws_bytes, const char* who)
{
    MM_CHECK_ARG(L && L->gate_ptr && L->up_ptr && L->down_ptr && L->suh13 && L->svh13 && L->suh2 && L->svh2,
                 "%s: incomplete layer", who);
    MM_CHECK_ARG(L->E > 0 && L->E <= 1024 && L->H > 0 && L->I > 0 && L->H % 128 == 0 && L->I % 128 == 0,
                 "%s: need 0 < E <= 1024 and H, I positive multiples of 128 (E=%d H=%d I=%d)", who, L->E, L->H, L->I);
    MM_CHECK_ARG((size_t)(L->H / 16) * (L->I / 16) * 96 < ((size_t)1 << 31), "%s: matrix larger than 2 GiB", who);
    MM_CHECK_ARG(x && ids, "%s: null pointer", who);
    MM_CHECK_ARG(x_dtype == MM_DTYPE_F16 || x_dtype == MM_DTYPE_BF16 || x_dtype == MM_DTYPE_F32,
                 "%s: x_dtype must be MM_DTYPE_F16, MM_DTYPE_BF16 or MM_DTYPE_F32", who);
    MM_CHECK_ARG(T > 0 && n > 0 && topk > 0 && n <= T * topk, "%s: bad T/n/topk", who);
    MM_CHECK_ARG((size_t)n * 2 * (L->H > L->I ? L->H : L->I) * 2 < ((size_t)1 << 31), "%s: too many routes", who);
    // tile rows of a partial launch (active experts x 2 matrices x column blocks x tile rows) count in int
    MM_CHECK_ARG((size_t)(n < L->E ? n : L->E) * L->H / 1024 * L->I < ((size_t)1 << 31), "%s: too many routes", who);
    MM_CHECK_ARG(max_rows > 0, "%s: max_rows must be at least 1", who);
    const bool perm = offsets != nullptr;
    MM_CHECK_ARG(perm ? (order && active && nactive) : n <= GV_ROUTE_MAX,
                 "%s: more than %d routes need the permutation (offsets, order, active, nactive)", who, GV_ROUTE_MAX);
    const size_t need = carve(nullptr, n, n, L->E, L->H, L->I).bytes;
    MM_CHECK_ARG(ws && ws_bytes >= need, "%s: workspace too small (%zu < %zu)", who, ws_bytes, need);
    return MM_OK;
}

__global__ __launch_bounds__(256) void k_fill_pos(int32_t* p, int n)
{
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) p[i] = -1;
}

static void launch_prep(const mm_layer_t* L, const Ws& w, const void* x, int x_dtype, int rescale, int n, int npos,
                        int topk, const int64_t* ids, const int32_t* offsets, const int32_t* order,
                        const int32_t* active, const int32_t* nactive, int cap, hipStream_t s)
{
    const int nb = prep_blocks(L->H);
    // positions past npos are not visited: their routes' pos_of must read "no position"
    if (npos < n) hipLaunchKernelGGL(k_fill_pos, dim3((unsigned)min((n + 255) / 256, 1024)), dim3(256), 0, s, w.pos_of, n);
    PrepArgs p{ x, ids, offsets, order, active, nactive, L->gate_ptr, L->up_ptr, L->down_ptr, L->suh13,
                w.rec, w.counts, w.pos_of, w.route_at, w.e_at, w.ai_at, w.ai_of, w.xa, w.xsum, n, topk, L->E, L->H, nb,
                x_dtype, rescale, cap, npos };
    launch_route_prep(p, s);
}

template <int MODE>
static void launch_partial(const mm_layer_t* L, const Ws& w, int npos, hipStream_t s)
{
    const int K = MODE == 0 ? L->H : L->I, N = MODE == 0 ? L->I : L->H;
    PartArgs p{ w.rec, w.counts, MODE == 0 ? w.xa : w.xd, MODE == 0 ? w.part_gu : w.part_d, npos, K, N, N / GV_COLS,
                piece_cap(npos) };
    const dim3 grid(partial_waves(seg_max(L, npos, MODE)) / GV_WAVES), block(GV_THREADS);
    if (L->flags & MM_LAYER_EXACT)
        hipLaunchKernelGGL((k_partial<MODE, true>), grid, block, 0, s, p);
    else
        hipLaunchKernelGGL((k_partial<MODE, false>), grid, block, 0, s, p);
}

static void launch_gu_epilogue(const mm_layer_t* L, const Ws& w, int npos, hipStream_t s)
{
    GuEpiArgs g{ w.part_gu, w.xsum, w.counts, w.e_at, w.ai_at, L->svh13, L->suh2, w.xd, w.xdsum, npos, L->H, L->I,
                 prep_blocks(L->H), partial_waves(seg_max(L, npos, 0)), piece_cap(npos), (L->flags & MM_LAYER_EXACT) ? 0 : 1, L->limit };
    hipLaunchKernelGGL(k_gu_epilogue, dim3((npos * (L->I / GV_COLS) + 3) / 4), dim3(256), 0, s, g);
}

static DEpiArgs down_args(const mm_layer_t* L, const Ws& w, int npos, int topk, const int64_t* ids, const float* wt,
                          float* Y, float* out, int accumulate)
{
    return DEpiArgs{ w.part_d, w.xdsum, w.counts, w.pos_of, w.route_at, w.e_at, w.ai_at, w.ai_of, ids, wt, L->svh2, Y, out, npos, L->H,
                     L->I, topk, partial_waves(seg_max(L, npos, 1)), piece_cap(npos), (L->flags & MM_LAYER_EXACT) ? 0 : 1, accumulate };
}

// One decode layer (mm_moe_decode) on a caller-provided workspace; `who` names the entry point in errors.
int moe_decode_launch(const mm_layer_t* L, const void* x, int x_dtype, int rescale, int T, int topk, const int64_t* ids,
                      const float* w, int max_rows, float* out, void* workspace, size_t workspace_bytes,
                      mm_stream_t stream, const char* who, int accumulate)
{
    MM_CHECK_ARG(topk > 0 && topk <= MAX_TOPK, "%s: topk must be in [1, %d]", who, MAX_TOPK);
    const int n = T * topk;
    const int rc = check_common(L, x, x_dtype, T, n, topk, ids, nullptr, nullptr, nullptr, nullptr, max_rows, workspace,
                                workspace_bytes, who);
    if (rc) return rc;
    MM_CHECK_ARG(w && out, "%s: null pointer", who);
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    const Ws ws = carve(workspace, n, n, L->E, L->H, L->I);
    launch_prep(L, ws, x, x_dtype, rescale, n, n, topk, ids, nullptr, nullptr, nullptr, nullptr, max_rows, s);
    launch_partial<0>(L, ws, n, s);
    launch_gu_epilogue(L, ws, n, s);
    launch_partial<1>(L, ws, n, s);
    const int threads = 64 * (topk < 2 ? 2 : topk);
    hipLaunchKernelGGL(k_down_combine, dim3(T * (L->H / GV_COLS)), dim3(threads), 0, s,
                       down_args(L, ws, n, topk, ids, w, nullptr, out, accumulate));
    return check_launch(who);
}

size_t decode_ws_bytes(int n, int npos, int E, int H, int I) { return carve(nullptr, n, npos, E, H, I).bytes; }

// The decode path of a call on a permutation whose valid positions lie below npos (every expert <= cap routes
// there), summed per token into out (out += with accumulate). Arguments are checked by the caller.
int decode_perm_launch(const mm_layer_t* L, const void* x, int x_dtype, int T, int topk, const int64_t* ids,
                       const float* w, const int32_t* offsets, const int32_t* order, const int32_t* active,
                       const int32_t* nactive, int npos, int cap, float* out, int accumulate, void* workspace,
                       hipStream_t s)
{
    const int n = T * topk;
    const Ws ws = carve(workspace, n, npos, L->E, L->H, L->I);
    launch_prep(L, ws, x, x_dtype, 0, n, npos, topk, ids, offsets, order, active, nactive, cap, s);
    launch_partial<0>(L, ws, npos, s);
    launch_gu_epilogue(L, ws, npos, s);
    launch_partial<1>(L, ws, npos, s);
    const int threads = 64 * (topk < 2 ? 2 : topk);
    hipLaunchKernelGGL(k_down_combine, dim3(T * (L->H / GV_COLS)), dim3(threads), 0, s,
                       down_args(L, ws, npos, topk, ids, w, nullptr, out, accumulate));
    return check_launch("decode path");
}

}  // namespace mm

using namespace mm;

extern "C" {

size_t mm_gemv_workspace(int n, int E, int H, int I)
{
    if (n <= 0 || E <= 0 || H <= 0 || I <= 0) return 0;
    return carve(nullptr, n, n, E, H, I).bytes;
}

int mm_expert_gemv(const mm_layer_t* L, const void* x, int x_dtype, int rescale, int T, int n, int topk,
                   const int64_t* ids, const int32_t* offsets, const int32_t* order, const int32_t* active,
                   const int32_t* nactive, int max_rows, float* Y, void* workspace, size_t workspace_bytes, int phases,
                   mm_stream_t stream)
{
    MM_CHECK_ARG(phases >= 1 && phases <= 31, "mm_expert_gemv: phases is a mask of 1, 2, 4, 8, 16");
    const int rc = check_common(L, x, x_dtype, T, n, topk, ids, offsets, order, active, nactive, max_rows, workspace,
                                workspace_bytes, "mm_expert_gemv");
    if (rc) return rc;
    MM_CHECK_ARG(Y || !(phases & 16), "mm_expert_gemv: null Y");
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    const Ws w = carve(workspace, n, n, L->E, L->H, L->I);
    if (phases & 1) launch_prep(L, w, x, x_dtype, rescale, n, n, topk, ids, offsets, order, active, nactive, max_rows, s);
    if (phases & 2) launch_partial<0>(L, w, n, s);
    if (phases & 4) launch_gu_epilogue(L, w, n, s);
    if (phases & 8) launch_partial<1>(L, w, n, s);
    if (phases & 16)
        hipLaunchKernelGGL(k_down_y, dim3((n * (L->H / GV_COLS) + 3) / 4), dim3(256), 0, s,
                           down_args(L, w, n, topk, ids, nullptr, Y, nullptr, 0));
    return check_launch("mm_expert_gemv");
}

int mm_moe_decode(const mm_layer_t* L, const void* x, int x_dtype, int rescale, int T, int topk, const int64_t* ids,
                  const float* w, int max_rows, float* out, void* workspace, size_t workspace_bytes, mm_stream_t stream)
{
    return mm::moe_decode_launch(L, x, x_dtype, rescale, T, topk, ids, w, max_rows, out, workspace, workspace_bytes,
                                 stream, "mm_moe_decode", 0);
}

}  // extern "C"
