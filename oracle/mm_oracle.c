/*
 * CPU ORACLE for the routed-expert MoE path. TEST INFRASTRUCTURE ONLY.
 *
 * This file restates, in plain C, the arithmetic of the reference's routed-expert path so that the
 * HIP kernels can be checked against it. It is never linked into, loaded by, or called from the product
 * library: only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may use it, and only as
 * the expected result that GPU outputs are compared against.
 *
 * Every function names the reference lines it follows (paths relative to the reference checkout).
 * How each function is pinned (golden vectors from the compiled reference, closed forms, brute force):
 * see the header of oracle/oracle.py, which wraps this file.
 *
 * Build: oracle/Makefile (gcc -O2 -fopenmp -ffp-contract=off). The contraction switch matters: the
 * reference computes the transforms with separate fp32 multiplies and adds, and so does this file.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define MMO_EXPORT __attribute__((visibility("default")))

/* ---------------------------------------------------------------------------------------------
 * fp16 <-> fp32 (IEEE binary16, round to nearest even), written out so the oracle does not depend on
 * F16C. Pinned in tests against numpy's float16 conversion over every fp16 bit pattern and a sweep of
 * fp32 values (ties, subnormals, overflow).
 * ------------------------------------------------------------------------------------------- */
MMO_EXPORT float mmo_h2f(uint16_t h)
{
    const uint32_t s = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
    uint32_t bits;
    float f;
    if (e == 0) {
        f = (float)m * 0x1p-24f;
        memcpy(&bits, &f, 4);
        bits |= s;
    } else if (e == 31) {
        bits = s | 0x7f800000u | (m << 13);
    } else {
        bits = s | ((e + 112u) << 23) | (m << 13);
    }
    memcpy(&f, &bits, 4);
    return f;
}

MMO_EXPORT uint16_t mmo_f2h(float f)
{
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint16_t s = (uint16_t)((x >> 16) & 0x8000u);
    x &= 0x7fffffffu;
    if (x >= 0x7f800000u) return (uint16_t)(s | 0x7c00u | (x > 0x7f800000u ? 0x200u : 0u));
    if (x >= 0x477ff000u) return (uint16_t)(s | 0x7c00u);          /* >= 65520 rounds to inf */
    if (x < 0x38800000u) {                                          /* below 2^-14: subnormal */
        float a;
        memcpy(&a, &x, 4);
        return (uint16_t)(s | (uint16_t)rintf(a * 0x1p24f));       /* exact scaling, RNE */
    }
    const uint32_t e = x - 0x38000000u;                             /* rebias 127 -> 15 */
    uint32_t r = e >> 13;
    const uint32_t rem = e & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (r & 1u))) r++;
    return (uint16_t)(s | r);
}

static inline float r16(float f) { return mmo_h2f(mmo_f2h(f)); }

/* ---------------------------------------------------------------------------------------------
 * EXL3 3-bpw trellis format, "mul1" codebook.  kernels/cpu_avx2/ft_core.h:28-83
 * ------------------------------------------------------------------------------------------- */
#define MMO_MUL1 0x83DCD12Du          /* ft_core.h:28 */
static const float MMO_HAD = 0.088388347648f;   /* ft_core.h:29 (same literal -> same fp32 value) */

/* stream index i (0..255) -> r*16 + c within a 16x16 tile.  ft_core.h:48-61 */
MMO_EXPORT void mmo_perm(int* perm)
{
    for (int t = 0; t < 32; ++t) {
        const int rb = (t & 3) * 2, col = t >> 2;
        static const int dr[4] = { 0, 1, 8, 9 };
        for (int j = 0; j < 8; ++j) {
            const int r = rb + dr[j & 3];
            const int c = col + ((j >> 2) << 3);
            perm[t * 8 + j] = r * 16 + c;
        }
    }
}

/* 16-bit trellis state of stream index i: the 16 stream bits ending at bit 3i+2 (mod 768), MSB-first
 * over the tile's 24 little-endian 32-bit words.  ft_core.h:63-73 */
MMO_EXPORT uint16_t mmo_state(const uint16_t* tile, int i)
{
    uint32_t w[24];
    memcpy(w, tile, 96);
    const int last = (3 * i + 2) % 768;                 /* position of the state's LSB */
    uint32_t st = 0;
    for (int b = 15; b >= 0; --b) {
        const int pos = (last - b + 768) % 768;          /* MSB first */
        const uint32_t bit = (w[pos >> 5] >> (31 - (pos & 31))) & 1u;
        st = (st << 1) | bit;
    }
    return (uint16_t)st;
}

/* byte sum of st * MUL1 (mod 2^32).  ft_core.h:75-79 */
MMO_EXPORT int mmo_bytesum(uint16_t st)
{
    const uint32_t x = (uint32_t)st * MMO_MUL1;
    return (int)((x & 0xffu) + ((x >> 8) & 0xffu) + ((x >> 16) & 0xffu) + (x >> 24));
}

/* weight = fp16(fma(1024 + bytesum, KINV, KBIAS)) with one fp16 rounding; KINV = fp16 0x1eee,
 * KBIAS = fp16 0xc931.  ft_core.h:38-39,81-83. The fp32 fma is exact here (|numerator| < 2^22 in units
 * of 2^-18), so this equals a single fp16 rounding of the exact value. Returns fp16 bits. */
MMO_EXPORT uint16_t mmo_weight_h(uint16_t st)
{
    const float kinv = mmo_h2f(0x1eee), kbias = mmo_h2f(0xc931);
    return mmo_f2h(fmaf((float)(1024 + mmo_bytesum(st)), kinv, kbias));
}

/* Dense K x N weights (fp32 holding fp16 values) of one matrix stored as tiles [K/16][N/16][48 int16].
 * ft_core.h:977-992 */
MMO_EXPORT void mmo_dense(const uint16_t* trellis, int K, int N, float* W)
{
    int perm[256];
    mmo_perm(perm);
    float lut[1021];
    const float kinv = mmo_h2f(0x1eee), kbias = mmo_h2f(0xc931);
    for (int s = 0; s <= 1020; ++s) lut[s] = r16(fmaf((float)(1024 + s), kinv, kbias));
    const int tn = N / 16, tk_n = K / 16;
#pragma omp parallel for schedule(static)
    for (int tk = 0; tk < tk_n; ++tk)
        for (int t = 0; t < tn; ++t) {
            const uint16_t* tile = trellis + ((size_t)tk * tn + t) * 48;
            for (int i = 0; i < 256; ++i) {
                const int rc = perm[i];
                W[(size_t)(tk * 16 + rc / 16) * N + t * 16 + rc % 16] = lut[mmo_bytesum(mmo_state(tile, i))];
            }
        }
}

/* ---------------------------------------------------------------------------------------------
 * Hadamard transforms, fp32 math with fp16 rounding points.  ft_core.h:89-110
 * ------------------------------------------------------------------------------------------- */
MMO_EXPORT void mmo_had128(float* v)
{
    for (int w = 1; w < 128; w *= 2)
        for (int b = 0; b < 128; b += 2 * w)
            for (int i = 0; i < w; ++i) {
                const float a = v[b + i], c = v[b + w + i];
                v[b + i] = a + c;
                v[b + w + i] = a - c;
            }
}

/* xt = r16(FWHT(x * suh) * HAD) on one 128-block; x holds fp16 values.  ft_core.h:96-102 */
MMO_EXPORT void mmo_prep_block(const float* x, const uint16_t* suh, float* xt)
{
    for (int i = 0; i < 128; ++i) xt[i] = x[i] * mmo_h2f(suh[i]);
    mmo_had128(xt);
    for (int i = 0; i < 128; ++i) xt[i] = r16(xt[i] * MMO_HAD);
}

/* y = r16(FWHT(r16(y)) * HAD * svh), two fp32 multiplies left to right.  ft_core.h:104-110 */
MMO_EXPORT void mmo_out_block(float* y, const uint16_t* svh)
{
    for (int i = 0; i < 128; ++i) y[i] = r16(y[i]);
    mmo_had128(y);
    for (int i = 0; i < 128; ++i) y[i] = r16((y[i] * MMO_HAD) * mmo_h2f(svh[i]));
}

/* silu(g) = g / (1 + exp(-g)); act = min(silu(g), L) * clamp(u, -L, L) when L != 0.  ft_core.h:123-133 */
MMO_EXPORT float mmo_act(float g, float u, float limit)
{
    float x = g / (1.0f + expf(-g));
    if (limit != 0.0f) {
        u = fminf(fmaxf(u, -limit), limit);
        x = fminf(x, limit);
    }
    return x * u;
}

/* ---------------------------------------------------------------------------------------------
 * Reference linear and expert: double accumulation over GPU-exact fp16 weights, same fp16 rounding
 * points.  ft_core.h:994-1011
 * ------------------------------------------------------------------------------------------- */
/* ntok rows of x [ntok][K] (fp16 values) -> y [ntok][N]. W: dense [K][N] from mmo_dense. */
MMO_EXPORT void mmo_linear_dense(const float* W, const uint16_t* suh, const uint16_t* svh, int K, int N, int ntok,
                                 const float* x, float* y)
{
    float* xt = (float*)malloc(sizeof(float) * (size_t)ntok * K);
    for (int t = 0; t < ntok; ++t)
        for (int b = 0; b < K / 128; ++b) mmo_prep_block(x + (size_t)t * K + b * 128, suh + b * 128, xt + (size_t)t * K + b * 128);
    const int chunk = 64;
#pragma omp parallel for schedule(static)
    for (int n0 = 0; n0 < N; n0 += chunk) {
        double acc[64];
        for (int t = 0; t < ntok; ++t) {
            for (int n = 0; n < chunk; ++n) acc[n] = 0.0;
            const float* xr = xt + (size_t)t * K;
            for (int k = 0; k < K; ++k) {
                const double xv = xr[k];
                const float* wr = W + (size_t)k * N + n0;
                for (int n = 0; n < chunk; ++n) acc[n] += xv * (double)wr[n];
            }
            for (int n = 0; n < chunk; ++n) y[(size_t)t * N + n0 + n] = (float)acc[n];
        }
    }
    for (int t = 0; t < ntok; ++t)
        for (int b = 0; b < N / 128; ++b) mmo_out_block(y + (size_t)t * N + b * 128, svh + b * 128);
    free(xt);
}

/* One expert over ntok tokens: g = Lg(x), u = Lu(x), a = r16(act(g, u)), y = Ld(a).
 * Wg, Wu: dense [H][I]; Wd: dense [I][H].  ft_core.h:1004-1011 (act limit: ct/ct_vllm.py:83-85) */
MMO_EXPORT void mmo_expert_dense(const float* Wg, const float* Wu, const float* Wd, const uint16_t* suh_g,
                                 const uint16_t* svh_g, const uint16_t* suh_u, const uint16_t* svh_u,
                                 const uint16_t* suh_d, const uint16_t* svh_d, int H, int I, float limit, int ntok,
                                 const float* x, float* y)
{
    float* g = (float*)malloc(sizeof(float) * (size_t)ntok * I);
    float* u = (float*)malloc(sizeof(float) * (size_t)ntok * I);
    mmo_linear_dense(Wg, suh_g, svh_g, H, I, ntok, x, g);
    mmo_linear_dense(Wu, suh_u, svh_u, H, I, ntok, x, u);
    for (size_t i = 0; i < (size_t)ntok * I; ++i) g[i] = r16(mmo_act(g[i], u[i], limit));
    mmo_linear_dense(Wd, suh_d, svh_d, I, H, ntok, g, y);
    free(g);
    free(u);
}

/* ---------------------------------------------------------------------------------------------
 * Synthetic trellis words: counter-based splitmix64. Word i of a stream with seed s is bits
 * 16*(i%4) .. 16*(i%4)+15 of mix64(s + (i/4 + 1) * 0x9E3779B97F4A7C15). The GPU fill kernel computes
 * the same integers, so any expert of a large synthetic store can be regenerated here.
 * ------------------------------------------------------------------------------------------- */
static inline uint64_t mix64(uint64_t z)
{
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

MMO_EXPORT uint64_t mmo_expert_seed(uint64_t layer_seed, uint64_t expert)
{
    return mix64(layer_seed * 0x100000001B3ull + expert);
}

MMO_EXPORT void mmo_synth_u16(uint64_t seed, uint64_t start, uint64_t n, uint16_t* out)
{
#pragma omp parallel for schedule(static)
    for (long long j = 0; j < (long long)n; ++j) {
        const uint64_t i = start + (uint64_t)j;
        const uint64_t h = mix64(seed + ((i >> 2) + 1) * 0x9E3779B97F4A7C15ull);
        out[j] = (uint16_t)(h >> (16 * (i & 3)));
    }
}

/* ---------------------------------------------------------------------------------------------
 * Router: logits = x . G^T (fp32 result of a double sum), top-k by descending logit with ties to the
 * lower expert index, weights = softmax over the selected logits. The reference takes topk_ids /
 * topk_weights from vLLM's FusedMoE router (patches/vllm-exl3-host-dma.patch:496-507); this is the
 * build's fixed definition of it.
 * ------------------------------------------------------------------------------------------- */
MMO_EXPORT void mmo_router(const float* x, const float* G, int T, int H, int E, int k, float* logits, int64_t* ids,
                           float* w)
{
#pragma omp parallel for schedule(static)
    for (int t = 0; t < T; ++t) {
        float* lg = logits + (size_t)t * E;
        for (int e = 0; e < E; ++e) {
            double s = 0.0;
            for (int h = 0; h < H; ++h) s += (double)x[(size_t)t * H + h] * (double)G[(size_t)e * H + h];
            lg[e] = (float)s;
        }
        unsigned char* used = (unsigned char*)calloc((size_t)E, 1);
        for (int j = 0; j < k; ++j) {
            int best = -1;
            for (int e = 0; e < E; ++e)
                if (!used[e] && (best < 0 || lg[e] > lg[best])) best = e;
            used[best] = 1;
            ids[(size_t)t * k + j] = best;
        }
        free(used);
        const double m = lg[ids[(size_t)t * k]];
        double den = 0.0;
        for (int j = 0; j < k; ++j) den += exp((double)lg[ids[(size_t)t * k + j]] - m);
        for (int j = 0; j < k; ++j) w[(size_t)t * k + j] = (float)(exp((double)lg[ids[(size_t)t * k + j]] - m) / den);
    }
}

/* ---------------------------------------------------------------------------------------------
 * Split (the decode tier's cost-model split).  ct/ft_tier_cu_v.cu:16-101
 * Policy p[9]: 0 t_zc, 1 t_hit, 2 cpu_a, 3 cpu_b, 4 cpu_tok, 5 max_cpu, 6 force_n, 7 handshake, 8 x-in-hx.
 * Host-side ctrl/hx/hpicks are plain arrays here. Extra outputs (hit and miss lists) are what the reference
 * keeps in shared memory; they are returned so the tests can compare them.
 * The cost model is evaluated in fp32 with the multiply-add pairs fused (fmaf), the form nvcc's default
 * contraction gives the reference source; tie-free policies make the argmin independent of that choice.
 * ------------------------------------------------------------------------------------------- */
MMO_EXPORT void mmo_split(const int64_t* sel, const float* w, const uint16_t* z, int n, int bsz, int H, int E,
                          const int32_t* slotof, const float* score, const float* p, int64_t* ctrl, uint16_t* hx,
                          int32_t* hpicks, int64_t* seqc, int li, int64_t* sel_out, float* w_out, int64_t* dflag,
                          int64_t* stats, int32_t* counts, int32_t* hits, int32_t* misses, int32_t* nhnm)
{
    const int topk = n / bsz;
    int* cnt = (int*)calloc((size_t)E, sizeof(int));
    unsigned char* cpu = (unsigned char*)calloc((size_t)E, 1);
    int* miss = (int*)malloc(sizeof(int) * (size_t)(E > 0 ? E : 1));
    for (int s = 0; s < n; ++s) {                                   /* :29-33 */
        const int64_t e = sel[s];
        if (w[s] != 0.0f && e >= 0 && e < E) {
            cnt[e]++;
            if (counts) counts[e]++;
        }
    }
    int nm = 0, nh = 0;
    for (int e = 0; e < E; ++e) {                                   /* :37-46 */
        if (!cnt[e]) continue;
        if (slotof[e] >= 0) {
            if (hits) hits[nh] = e;
            ++nh;
            continue;
        }
        int b = nm++;
        while (b > 0 && score[miss[b - 1]] > score[e]) { miss[b] = miss[b - 1]; --b; }
        miss[b] = e;
    }
    if (misses) for (int i = 0; i < nm; ++i) misses[i] = miss[i];
    if (nhnm) { nhnm[0] = nh; nhnm[1] = nm; }
    int best = 0;                                                   /* :47-60 */
    const int force = (int)p[6];
    const int maxc = (int)p[5] < nm ? (int)p[5] : nm;
    if (force >= 0) best = force < nm ? force : nm;
    else {
        float bt = 1e30f, c = 0.0f;
        for (int k = 0; k <= maxc; ++k) {
            if (k) c = fmaf(p[3], fmaf(p[4], (float)(cnt[miss[k - 1]] - 1), 1.0f), c);
            const float gpu = fmaf(p[1], (float)(nh + nm - k), p[0] * (float)(nm - k));
            const float tt = fmaxf(gpu, k ? p[2] + c : 0.0f);
            if (tt < bt - 1e-6f) { bt = tt; best = k; }
        }
    }
    for (int k = 0; k < best; ++k) cpu[miss[k]] = 1;                 /* :61 */
    const int publish = best > 0 || p[7] > 0.5f;
    stats[0] += nh; stats[1] += nm; stats[2] += best; stats[3] += 1;
    int npk = 0;
    int64_t seq = 0;
    if (publish) {                                                  /* :65-75 */
        seq = ++seqc[0];
        for (int s = 0; s < n; ++s) {
            const int64_t e = sel[s];
            if (e < 0 || e >= E || !cpu[e] || w[s] == 0.0f) continue;
            hpicks[npk * 3] = s / topk;
            hpicks[npk * 3 + 1] = (int32_t)e;
            memcpy(&hpicks[npk * 3 + 2], &w[s], 4);
            ++npk;
        }
    }
    for (int s = 0; s < n; ++s) {                                   /* :78-84 */
        const int64_t e = sel[s];
        const int c = e >= 0 && e < E && cpu[e];
        sel_out[s] = c ? -1 : e;
        w_out[s] = c ? 0.0f : w[s];
    }
    if (publish) {                                                  /* :85-98 */
        if (!(p[8] > 0.5f)) memcpy(hx, z, sizeof(uint16_t) * (size_t)bsz * H);
        ctrl[2] = li; ctrl[3] = bsz; ctrl[4] = npk;
        ctrl[0] = seq;
        dflag[0] = seq;
    } else
        dflag[0] = 0;                                               /* :100 */
    free(cnt); free(cpu); free(miss);
}

/* ---------------------------------------------------------------------------------------------
 * Routing prep: map out-of-range ids to the sentinel E, count per expert (E+1 bins), stable order by
 * (expert, flat index), token index = flat index / topk, per-expert exclusive offsets.
 * patches/vllm-exl3-host-dma.patch:204-236,296-312 (argsort stability is unspecified there; the order here
 * is stable by definition).
 * ------------------------------------------------------------------------------------------- */
MMO_EXPORT void mmo_permute(const int64_t* ids, const float* w, int n, int topk, int E, int32_t* counts,
                            int32_t* offsets, int32_t* order, int32_t* token_sorted, float* weight_sorted)
{
    for (int e = 0; e <= E; ++e) counts[e] = 0;
    for (int s = 0; s < n; ++s) {
        const int64_t e = ids[s];
        counts[(e >= 0 && e < E) ? e : E]++;
    }
    offsets[0] = 0;
    for (int e = 0; e <= E; ++e) offsets[e + 1] = offsets[e] + counts[e];
    int32_t* fill = (int32_t*)malloc(sizeof(int32_t) * (size_t)(E + 1));
    for (int e = 0; e <= E; ++e) fill[e] = offsets[e];
    for (int s = 0; s < n; ++s) {
        const int64_t e0 = ids[s];
        const int e = (e0 >= 0 && e0 < E) ? (int)e0 : E;
        const int pos = fill[e]++;
        order[pos] = s;
        if (token_sorted) token_sorted[pos] = s / topk;
        if (weight_sorted) weight_sorted[pos] = w ? w[s] : 0.0f;
    }
    free(fill);
}

/* ---------------------------------------------------------------------------------------------
 * Combine: out[t] += sum_j w[t,j] * Y[t*k + j] in fixed j order (fp32 fma), then the optional host
 * partial: out += hout once ctrl[1] >= dflag (here the wait is resolved by the caller).
 * The routed sum replaces the atomics of the fused kernel (patches/vllm-exl3-host-dma.patch:327-342);
 * the host-partial add follows ct/ft_tier_cu_v.cu:103-127.
 * ------------------------------------------------------------------------------------------- */
MMO_EXPORT void mmo_combine(float* out, const float* Y, const float* w, int T, int k, int H, const float* hout,
                            int add_hout)
{
    for (int t = 0; t < T; ++t)
        for (int h = 0; h < H; ++h) {
            float acc = out[(size_t)t * H + h];
            for (int j = 0; j < k; ++j) acc = fmaf(w[(size_t)t * k + j], Y[((size_t)t * k + j) * H + h], acc);
            if (add_hout) acc += hout[(size_t)t * H + h];
            out[(size_t)t * H + h] = acc;
        }
}

/* ---------------------------------------------------------------------------------------------
 * The decode chain's step between layers (a definition of the benchmark workload; the reference has no
 * counterpart): fp16(bf16(x * s)) per row, s = 1 / sqrt(ss / H) in fp32 (correctly rounded divide and
 * square root), s = 1 for rescale == 0 or ss == 0. ss is accumulated in fp32 in one fixed order, the one
 * the device kernels use: 256 partial sums, partial j takes h = j, j + 256, j + 512, ... through fused
 * multiply-adds; each group of 64 partials is combined by exchange at distances 32, 16, 8, 4, 2, 1 (every
 * partial adds the one at its index xor the distance); the four group sums add as (g0 + g1) + (g2 + g3).
 * bf16 rounds to nearest even (a NaN stays a quiet NaN), then fp16 rounds to nearest even.
 * xb (optional) receives the bf16 bits, xh the fp16 bits, both [T, H].
 * ------------------------------------------------------------------------------------------- */
static uint16_t f2bf_rne(float f)
{
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

MMO_EXPORT float mmo_row_sumsq(const float* row, int H)
{
    float p[256], q[64];
    for (int j = 0; j < 256; ++j) {
        float ss = 0.0f;
        for (int h = j; h < H; h += 256) ss = fmaf(row[h], row[h], ss);
        p[j] = ss;
    }
    float g[4];
    for (int w = 0; w < 4; ++w) {
        float* v = p + 64 * w;
        for (int d = 32; d >= 1; d >>= 1) {
            for (int l = 0; l < 64; ++l) q[l] = v[l] + v[l ^ d];
            memcpy(v, q, sizeof q);
        }
        g[w] = v[0];
    }
    return (g[0] + g[1]) + (g[2] + g[3]);
}

MMO_EXPORT float mmo_row_scale(const float* row, int H)
{
    const float tot = mmo_row_sumsq(row, H);
    return tot > 0.0f ? 1.0f / sqrtf(tot / (float)H) : 1.0f;
}

MMO_EXPORT void mmo_prepare_input(const float* x, int T, int H, int rescale, uint16_t* xb, uint16_t* xh)
{
    for (int t = 0; t < T; ++t) {
        const float* row = x + (size_t)t * H;
        const float s = rescale ? mmo_row_scale(row, H) : 1.0f;
        for (int h = 0; h < H; ++h) {
            const uint16_t b = f2bf_rne(row[h] * s);
            const uint32_t bits = (uint32_t)b << 16;
            float v;
            memcpy(&v, &bits, 4);
            if (xb) xb[(size_t)t * H + h] = b;
            xh[(size_t)t * H + h] = mmo_f2h(v);
        }
    }
}
