// Host expert tier: routed experts computed on the host cores, straight from their pinned home copies, for the
// picks the decode split sends to the host (the reference's CPU tier, kernels/cpu_avx2/ft_tier_ext.cpp:36-231 and
// ft_core.h:573-727, rebuilt for AVX-512 hosts). Three parts:
//
//   Pool      N threads pinned to the given CPUs (the caller is thread 0); a phase is a list of work units taken
//             from an atomic counter. Idle threads spin on a generation word, then nap.
//   kernel    the EXL3 3-bpw expert MLP for a group of tokens: input transform, gate/up GEMV, SwiGLU, down-input
//             transform, down GEMV, output transforms, weighted sum per token.
//   worker    a thread that serves the mailbox the GPU split kernel publishes (ctrl words, fp16 x rows, picks) and
//             answers with an fp32 partial in host-mapped memory and the done word.
//
// Trellis decode, 16 weights per AVX-512 operation: a 16x16 tile is 24 dwords (held in two zmm registers); the
// 16 weights of tile row r, columns 0..15, are the trellis states i(r, c) = 32 (c & 7) + 8 ((r & 7) >> 1) + (r & 1)
// + 2 (r >> 3) + 4 (c >> 3) (the inverse of the stream order PERM, ft_core.h:48-61). State i is the 16-bit window
// ending at stream bit 3 i + 2 (mod 768, MSB first over the tile's little-endian dwords, ft_core.h:63-73): two
// lane permutes fetch the two dwords holding it, one double shift (VBMI2) extracts it. The code is
// 1024 + bytesum(state * 0x83DCD12D) (ft_core.h:75-83): one 32-bit multiply, one byte dot product against ones
// (VNNI) that adds the four bytes onto the constant. EXACT rounds KINV * code + KBIAS to fp16 per weight (the
// reference's EXACT expert and the GPU's fp16 weights); AFFINE (the default) accumulates sum_k x_k (code_k - 1534)
// per column and forms KINV * S + (KBIAS + 1534 KINV) * sum_k x_k once per output (ft_core.h:267-293's AFFINE
// evaluation; the codes are centred so the fp32 sum carries less of the common offset). I16 (ft_core.h:315-415)
// quantises each 128-block of transformed inputs to int16 (|x| <= 16383 with one fp32 scale per block) and sums
// bytesum * x exactly in int32 per block (VNNI vpdpwssd over row pairs), scaled into fp32 once per block; the
// output is KINV * S + (1024 KINV + KBIAS) * sum of the dequantised inputs. The automatic mode takes I16 for jobs
// whose experts have at most two rows each and AFFINE otherwise, as the reference's tier does.
#include <immintrin.h>
#include <pthread.h>
#include <sched.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>
#include <time.h>
#include <unistd.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <thread>
#include <vector>

#include "host_tier.h"

namespace tier {

using mm::set_error;

constexpr uint32_t MUL1 = 0x83DCD12Du;
constexpr float HAD = 0.088388347648f;           // 1/sqrt(128), the reference's literal (ft_core.h:29)
constexpr int TILE_BYTES = 96;
constexpr int MAX_MT = 3;                        // tokens per pass of the GEMV (accumulators in registers)
constexpr int CENTER = 1534;                     // AFFINE: codes 1024 + bytesum (1024 .. 2044) centred on 1534

static inline float h2f(uint16_t h) { return _cvtsh_ss(h); }
static inline uint16_t f2h(float f) { return _cvtss_sh(f, _MM_FROUND_TO_NEAREST_INT | _MM_FROUND_NO_EXC); }
static inline float r16(float f) { return h2f(f2h(f)); }
static inline float kinv() { return h2f(0x1eee); }
static inline float kbias() { return h2f(0xc931); }

static double now_s()
{
    timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (double)ts.tv_sec + 1e-9 * (double)ts.tv_nsec;
}

// ------------------------------------------------------------------------------------------------ pool

class Pool
{
public:
    typedef void (*Fn)(void* ctx, int unit);

    void start(const std::vector<int>& cpus, int n)
    {
        n_ = n < 1 ? 1 : n;
        cpus_ = cpus;
        quit_.store(false);
        // the generation the threads start from is read here, before any run() or stop() can move it
        const uint64_t g0 = gen_.load(std::memory_order_acquire);
        for (int w = 1; w < n_; ++w) th_.emplace_back([this, w, g0] { loop(w, g0); });
    }
    void stop()
    {
        quit_.store(true);
        gen_.fetch_add(1, std::memory_order_release);
        for (auto& t : th_) t.join();
        th_.clear();
    }
    int size() const { return n_; }
    int cpu_of(int w) const { return cpus_.empty() ? -1 : cpus_[(size_t)w % cpus_.size()]; }

    // Runs fn(ctx, u) for u in [0, units) on every thread (the caller included); returns when all are done.
    void run(Fn fn, void* ctx, int units)
    {
        if (units <= 0) return;
        fn_ = fn;
        ctx_ = ctx;
        units_ = units;
        next_.store(0, std::memory_order_relaxed);
        done_.store(0, std::memory_order_relaxed);
        gen_.fetch_add(1, std::memory_order_release);
        work();
        while (done_.load(std::memory_order_acquire) < n_ - 1) _mm_pause();
    }

    static void pin(int cpu)
    {
        if (cpu < 0) return;
        cpu_set_t s;
        CPU_ZERO(&s);
        CPU_SET(cpu, &s);
        pthread_setaffinity_np(pthread_self(), sizeof(s), &s);
    }

private:
    void work()
    {
        for (;;)
        {
            const int u = next_.fetch_add(1, std::memory_order_relaxed);
            if (u >= units_) break;
            fn_(ctx_, u);
        }
    }
    void loop(int w, uint64_t seen)
    {
        pin(cpu_of(w));
        for (;;)
        {
            long spins = 0;
            uint64_t g;
            while ((g = gen_.load(std::memory_order_acquire)) == seen)
            {
                if (++spins < 200000) _mm_pause();
                else usleep(20);
            }
            seen = g;
            if (quit_.load()) return;
            work();
            done_.fetch_add(1, std::memory_order_acq_rel);
        }
    }

    int n_ = 1;
    std::vector<int> cpus_;
    std::vector<std::thread> th_;
    std::atomic<uint64_t> gen_{ 0 };
    std::atomic<int> next_{ 0 }, done_{ 0 };
    std::atomic<bool> quit_{ false };
    Fn fn_ = nullptr;
    void* ctx_ = nullptr;
    int units_ = 0;
};

// ------------------------------------------------------------------------------------------------ model

struct Mat
{
    const uint8_t* tr = nullptr;     // tiles [K/16][N/16][96 B]
    const uint16_t* suh = nullptr;   // fp16 [K]
    const uint16_t* svh = nullptr;   // fp16 [N]
    int K = 0, N = 0;
};
struct Expert { Mat g, u, d; };
struct Layer { int E = 0; std::vector<Expert> ex; };

// Per tile row r (16) and lane c (16): the dword holding the state's last bit, the one before it (circularly)
// and the right shift that leaves the 16-bit state in the low half of the pair.
struct Tables
{
    alignas(64) int32_t lo[16][16];
    alignas(64) int32_t hi[16][16];
    alignas(64) int32_t sh[16][16];
    Tables()
    {
        for (int r = 0; r < 16; ++r)
            for (int c = 0; c < 16; ++c)
            {
                const int i = 32 * (c & 7) + 8 * ((r & 7) >> 1) + (r & 1) + 2 * (r >> 3) + 4 * (c >> 3);
                const int last = (3 * i + 2) % 768;
                lo[r][c] = last >> 5;
                hi[r][c] = ((last >> 5) + 23) % 24;
                sh[r][c] = 31 - (last & 31);
            }
    }
};
// Built on first use (this file is compiled for AVX-512; nothing of it runs before the CPU check).
static const Tables& tab()
{
    static const Tables t;
    return t;
}

// ------------------------------------------------------------------------------------------------ transforms

// 128-point Walsh-Hadamard transform with the reference's butterfly (strides 1 .. 64, (a + b, a - b),
// ft_core.h:89-94), so every fp32 result is the reference's.
static void fwht128(float* v)
{
    for (int h = 1; h < 128; h <<= 1)
        for (int i = 0; i < 128; i += 2 * h)
            for (int j = i; j < i + h; ++j)
            {
                const float a = v[j], b = v[j + h];
                v[j] = a + b;
                v[j + h] = a - b;
            }
}

// xt = r16(FWHT(x * suh) * HAD) per 128-block (ft_core.h:96-102); returns the sum of xt.
static float prep_input(const float* x, const uint16_t* suh, int K, float* xt)
{
    float s = 0.0f;
    for (int b = 0; b < K; b += 128)
    {
        float v[128];
        for (int i = 0; i < 128; ++i) v[i] = x[b + i] * h2f(suh[b + i]);
        fwht128(v);
        for (int i = 0; i < 128; ++i)
        {
            xt[b + i] = r16(v[i] * HAD);
            s += xt[b + i];
        }
    }
    return s;
}

// I16 inputs (ft_core.h:393-411): each 128-block of xt as int16 with scale amax / 16383 (1 for an all-zero block),
// rounded to nearest even after a multiply by the reciprocal; returns the sum of the dequantised values, block by
// block in fp32 (the fix-up's input sum).
static float quant_i16(const float* xt, int K, int16_t* xq, float* qs)
{
    float s = 0.0f;
    for (int b = 0; b < K; b += 128)
    {
        float amax = 0.0f;
        for (int i = 0; i < 128; ++i) amax = std::max(amax, std::fabs(xt[b + i]));
        const float sc = amax > 0.0f ? amax / 16383.0f : 1.0f, rs = 1.0f / sc;
        long si = 0;
        for (int i = 0; i < 128; ++i)
        {
            const int v = (int)std::nearbyint(xt[b + i] * rs);
            xq[b + i] = (int16_t)v;
            si += v;
        }
        qs[b / 128] = sc;
        s += (float)si * sc;
    }
    return s;
}

// y = r16(FWHT(r16(y)) * HAD * svh) on one 128-block in place (ft_core.h:104-110).
static void out_block(float* y, const uint16_t* svh)
{
    for (int i = 0; i < 128; ++i) y[i] = r16(y[i]);
    fwht128(y);
    for (int i = 0; i < 128; ++i) y[i] = r16((y[i] * HAD) * h2f(svh[i]));
}

static inline float act_gu(float g, float u, float limit)
{
    float x = g / (1.0f + std::exp(-g));
    if (limit != 0.0f)
    {
        u = std::fmin(std::fmax(u, -limit), limit);
        x = std::fmin(x, limit);
    }
    return x * u;
}

// ------------------------------------------------------------------------------------------------ GEMV

// The rows of a group of tokens: token t's transformed input is xt + t * xstride (K values), its input sum
// xs[t * sstride], its output row y + t * ystride (128 values of the column block).
struct Rows
{
    const float* xt;
    size_t xstride;
    const float* xs;
    size_t sstride;
    float* y;
    size_t ystride;
    Rows at(int t) const { return { xt + t * xstride, xstride, xs + t * sstride, sstride, y + t * ystride, ystride }; }
};

// The decode constants of one GEMV.
struct DecodeConsts
{
    __m512i vmask, vmul, vones, vbase;
    __m512 vkinv, vkbias;
    template <bool EXACT>
    static DecodeConsts make()
    {
        return { _mm512_set1_epi32(0xffff), _mm512_set1_epi32((int)MUL1), _mm512_set1_epi8(1),
                 _mm512_set1_epi32(EXACT ? 1024 : 1024 - CENTER), _mm512_set1_ps(kinv()), _mm512_set1_ps(kbias()) };
    }
};

// Weights of row r, columns 0 .. 15 of the tile held in wa (dwords 0 .. 15) and wb (dwords 16 .. 23). EXACT:
// fp16-rounded weights; else the centred AFFINE codes.
template <bool EXACT>
static inline __m512 decode_row(__m512i wa, __m512i wb, int r, const Tables& TAB, const DecodeConsts& C)
{
    const __m512i lo = _mm512_permutex2var_epi32(wa, _mm512_load_si512(TAB.lo[r]), wb);
    const __m512i hi = _mm512_permutex2var_epi32(wa, _mm512_load_si512(TAB.hi[r]), wb);
    const __m512i st = _mm512_and_si512(_mm512_shrdv_epi32(lo, hi, _mm512_load_si512(TAB.sh[r])), C.vmask);
    const __m512i p = _mm512_mullo_epi32(st, C.vmul);
    const __m512i code = _mm512_dpbusd_epi32(C.vbase, p, C.vones);
    __m512 w = _mm512_cvtepi32_ps(code);
    if constexpr (EXACT)
        w = _mm512_cvtph_ps(_mm512_cvtps_ph(_mm512_fmadd_ps(w, C.vkinv, C.vkbias),
                                            _MM_FROUND_TO_NEAREST_INT | _MM_FROUND_NO_EXC));
    return w;
}

// Byte sums (code - 1024) of row r, columns 0 .. 15, as int32.
static inline __m512i byte_sums(__m512i wa, __m512i wb, int r, const Tables& TAB, const DecodeConsts& C)
{
    const __m512i lo = _mm512_permutex2var_epi32(wa, _mm512_load_si512(TAB.lo[r]), wb);
    const __m512i hi = _mm512_permutex2var_epi32(wa, _mm512_load_si512(TAB.hi[r]), wb);
    const __m512i st = _mm512_and_si512(_mm512_shrdv_epi32(lo, hi, _mm512_load_si512(TAB.sh[r])), C.vmask);
    return _mm512_dpbusd_epi32(_mm512_setzero_si512(), _mm512_mullo_epi32(st, C.vmul), C.vones);
}

static inline void prefetch_rows(const uint8_t* row)
{
    for (int o = 0; o < 8 * TILE_BYTES; o += 64) _mm_prefetch((const char*)(row + o), _MM_HINT_T0);
}

// The raw sums of MT tokens (in registers) -> y rows: EXACT as they are, AFFINE fixed up per output.
template <int MT, bool EXACT>
static inline void store_rows(__m512 (&acc)[MT][8], const Rows& R)
{
    const __m512 vkinv = _mm512_set1_ps(kinv());
    for (int t = 0; t < MT; ++t)
    {
        if constexpr (EXACT)
        {
            for (int j = 0; j < 8; ++j) _mm512_storeu_ps(R.y + t * R.ystride + 16 * j, acc[t][j]);
        }
        else
        {
            const __m512 off = _mm512_set1_ps((float)((double)kbias() + CENTER * (double)kinv()) * R.xs[t * R.sstride]);
            for (int j = 0; j < 8; ++j) _mm512_storeu_ps(R.y + t * R.ystride + 16 * j, _mm512_fmadd_ps(vkinv, acc[t][j], off));
        }
    }
}

// y[t][0..127] (raw sums, before the output transform) of column block cb of matrix m for MT tokens, each
// weight decoded in registers and used at once.
template <int MT, bool EXACT>
static void gemv_block(const Mat& m, int cb, const Rows& R)
{
    const int NT = m.N / 16, KT = m.K / 16;
    const DecodeConsts C = DecodeConsts::make<EXACT>();
    __m512 acc[MT][8];
    for (int t = 0; t < MT; ++t)
        for (int j = 0; j < 8; ++j) acc[t][j] = _mm512_setzero_ps();
    const uint8_t* base = m.tr + (size_t)cb * 8 * TILE_BYTES;
    const Tables& TAB = tab();
    for (int tk = 0; tk < KT; ++tk)
    {
        const uint8_t* row = base + (size_t)tk * NT * TILE_BYTES;
        if (tk + 4 < KT) prefetch_rows(row + (size_t)4 * NT * TILE_BYTES);
        for (int j = 0; j < 8; ++j)
        {
            const uint8_t* tile = row + j * TILE_BYTES;
            const __m512i wa = _mm512_loadu_si512(tile);
            const __m512i wb = _mm512_castsi256_si512(_mm256_loadu_si256((const __m256i*)(tile + 64)));
            for (int r = 0; r < 16; ++r)
            {
                const __m512 w = decode_row<EXACT>(wa, wb, r, TAB, C);
                const int k = tk * 16 + r;
                for (int t = 0; t < MT; ++t) acc[t][j] = _mm512_fmadd_ps(_mm512_set1_ps(R.xt[t * R.xstride + k]), w, acc[t][j]);
            }
        }
    }
    store_rows<MT, EXACT>(acc, R);
}

// The same sums for any number of tokens (an expert with many rows, as a prefill tail job has): the weights of
// CHUNK_TR tile rows are decoded once into an L1 buffer, then every group of up to MAX_MT tokens runs over the
// chunk with its sums in registers, kept between chunks in a per-thread buffer. Each output's fma chain runs in
// ascending k as in gemv_block, so the results are bit-identical to it.
constexpr int CHUNK_TR = 2;

template <int MT, bool EXACT>
static inline void chunk_pass(const float* W, int k0, float* accbuf, const Rows& R)
{
    __m512 acc[MT][8];
    for (int t = 0; t < MT; ++t)
        for (int j = 0; j < 8; ++j) acc[t][j] = _mm512_load_ps(accbuf + t * 128 + 16 * j);
    for (int k = 0; k < CHUNK_TR * 16; ++k)
    {
        __m512 xb[MT];
        for (int t = 0; t < MT; ++t) xb[t] = _mm512_set1_ps(R.xt[t * R.xstride + k0 + k]);
        for (int j = 0; j < 8; ++j)
        {
            const __m512 w = _mm512_load_ps(W + k * 128 + 16 * j);
            for (int t = 0; t < MT; ++t) acc[t][j] = _mm512_fmadd_ps(xb[t], w, acc[t][j]);
        }
    }
    for (int t = 0; t < MT; ++t)
        for (int j = 0; j < 8; ++j) _mm512_store_ps(accbuf + t * 128 + 16 * j, acc[t][j]);
}

template <bool EXACT>
static void gemv_many(const Mat& m, int cb, int nt, const Rows& R)
{
    thread_local std::vector<float> accv;
    alignas(64) static thread_local float W[CHUNK_TR * 16 * 128];
    const size_t need = (size_t)((nt + MAX_MT - 1) / MAX_MT) * MAX_MT * 128;
    if (accv.size() < need + 16) accv.resize(need + 16);
    float* accbuf = reinterpret_cast<float*>(((uintptr_t)accv.data() + 63) & ~(uintptr_t)63);
    memset(accbuf, 0, need * sizeof(float));
    const int NT = m.N / 16, KT = m.K / 16;
    const DecodeConsts C = DecodeConsts::make<EXACT>();
    const uint8_t* base = m.tr + (size_t)cb * 8 * TILE_BYTES;
    const Tables& TAB = tab();
    for (int tk0 = 0; tk0 < KT; tk0 += CHUNK_TR)
    {
        for (int q = 0; q < CHUNK_TR; ++q)
        {
            const uint8_t* row = base + (size_t)(tk0 + q) * NT * TILE_BYTES;
            if (tk0 + q + 4 < KT) prefetch_rows(row + (size_t)4 * NT * TILE_BYTES);
            for (int j = 0; j < 8; ++j)
            {
                const uint8_t* tile = row + j * TILE_BYTES;
                const __m512i wa = _mm512_loadu_si512(tile);
                const __m512i wb = _mm512_castsi256_si512(_mm256_loadu_si256((const __m256i*)(tile + 64)));
                for (int r = 0; r < 16; ++r) _mm512_store_ps(W + (q * 16 + r) * 128 + 16 * j, decode_row<EXACT>(wa, wb, r, TAB, C));
            }
        }
        const int k0 = tk0 * 16;
        for (int t0 = 0; t0 < nt; t0 += MAX_MT)
        {
            const int mt = nt - t0 < MAX_MT ? nt - t0 : MAX_MT;
            float* ab = accbuf + (size_t)t0 * 128;
            if (mt == 3) chunk_pass<3, EXACT>(W, k0, ab, R.at(t0));
            else if (mt == 2) chunk_pass<2, EXACT>(W, k0, ab, R.at(t0));
            else chunk_pass<1, EXACT>(W, k0, ab, R.at(t0));
        }
    }
    for (int t0 = 0; t0 < nt; t0 += MAX_MT)
    {
        const int mt = nt - t0 < MAX_MT ? nt - t0 : MAX_MT;
        __m512 acc[MAX_MT][8];
        for (int t = 0; t < mt; ++t)
            for (int j = 0; j < 8; ++j) acc[t][j] = _mm512_load_ps(accbuf + (size_t)(t0 + t) * 128 + 16 * j);
        if (mt == 3) store_rows<3, EXACT>(acc, R.at(t0));
        else if (mt == 2) store_rows<2, EXACT>(reinterpret_cast<__m512(&)[2][8]>(acc), R.at(t0));
        else store_rows<1, EXACT>(reinterpret_cast<__m512(&)[1][8]>(acc), R.at(t0));
    }
}

// Tokens past MANY_MIN take the chunked path (one decode for all of them); fewer run gemv_block, decoding per
// group of MAX_MT.
constexpr int MANY_MIN = 4;

template <bool EXACT>
static void gemv_tokens(const Mat& m, int cb, int nt, const Rows& R)
{
    if (nt >= MANY_MIN)
    {
        gemv_many<EXACT>(m, cb, nt, R);
        return;
    }
    for (int t0 = 0; t0 < nt; t0 += MAX_MT)
    {
        const int mt = nt - t0 < MAX_MT ? nt - t0 : MAX_MT;
        if (mt == 3) gemv_block<3, EXACT>(m, cb, R.at(t0));
        else if (mt == 2) gemv_block<2, EXACT>(m, cb, R.at(t0));
        else gemv_block<1, EXACT>(m, cb, R.at(t0));
    }
}

// I16 sums of column block cb for MT tokens: int16 inputs xq[t] (row pairs read as one dword), block scales
// qs[t], input sums xs[t]; per tile row pair the two rows' byte sums are packed into the halves of each dword and
// one vpdpwssd per token adds both products; every 8 tile rows (one 128-block) the int32 sums are scaled into fp32.
struct RowsI16
{
    const int16_t* xq;
    size_t xstride;
    const float* qs;
    size_t qstride;
    const float* xs;
    size_t sstride;
    float* y;
    size_t ystride;
    RowsI16 at(int t) const
    {
        return { xq + t * xstride, xstride, qs + t * qstride, qstride, xs + t * sstride, sstride, y + t * ystride, ystride };
    }
};

template <int MT>
static void gemv_block_i16(const Mat& m, int cb, const RowsI16& R)
{
    const int NT = m.N / 16, KT = m.K / 16;
    const DecodeConsts C = DecodeConsts::make<false>();
    const __m512i zero = _mm512_setzero_si512();
    __m512i acc[MT][8];
    alignas(64) float accf[MT][8][16];
    for (int t = 0; t < MT; ++t)
        for (int j = 0; j < 8; ++j)
        {
            acc[t][j] = zero;
            _mm512_store_ps(accf[t][j], _mm512_setzero_ps());
        }
    const uint8_t* base = m.tr + (size_t)cb * 8 * TILE_BYTES;
    const Tables& TAB = tab();
    for (int tk = 0; tk < KT; ++tk)
    {
        const uint8_t* row = base + (size_t)tk * NT * TILE_BYTES;
        if (tk + 4 < KT) prefetch_rows(row + (size_t)4 * NT * TILE_BYTES);
        for (int j = 0; j < 8; ++j)
        {
            const uint8_t* tile = row + j * TILE_BYTES;
            const __m512i wa = _mm512_loadu_si512(tile);
            const __m512i wb = _mm512_castsi256_si512(_mm256_loadu_si256((const __m256i*)(tile + 64)));
            for (int r = 0; r < 16; r += 2)
            {
                const __m512i b0 = byte_sums(wa, wb, r, TAB, C), b1 = byte_sums(wa, wb, r + 1, TAB, C);
                const __m512i pair = _mm512_or_si512(b0, _mm512_slli_epi32(b1, 16));
                const int k = tk * 16 + r;
                for (int t = 0; t < MT; ++t)
                {
                    int32_t xp;
                    memcpy(&xp, R.xq + t * R.xstride + k, 4);
                    acc[t][j] = _mm512_dpwssd_epi32(acc[t][j], pair, _mm512_set1_epi32(xp));
                }
            }
        }
        if ((tk & 7) == 7)
            for (int t = 0; t < MT; ++t)
            {
                const __m512 sc = _mm512_set1_ps(R.qs[t * R.qstride + (tk >> 3)]);
                for (int j = 0; j < 8; ++j)
                {
                    _mm512_store_ps(accf[t][j], _mm512_fmadd_ps(_mm512_cvtepi32_ps(acc[t][j]), sc, _mm512_load_ps(accf[t][j])));
                    acc[t][j] = zero;
                }
            }
    }
    const __m512 vkinv = _mm512_set1_ps(kinv());
    const float caff = (float)(1024.0 * (double)kinv() + (double)kbias());       // -3.453125, exact
    for (int t = 0; t < MT; ++t)
    {
        const __m512 off = _mm512_set1_ps(caff * R.xs[t * R.sstride]);
        for (int j = 0; j < 8; ++j)
            _mm512_storeu_ps(R.y + t * R.ystride + 16 * j, _mm512_fmadd_ps(vkinv, _mm512_load_ps(accf[t][j]), off));
    }
}

static void gemv_tokens_i16(const Mat& m, int cb, int nt, const RowsI16& R)
{
    for (int t0 = 0; t0 < nt; t0 += MAX_MT)
    {
        const int mt = nt - t0 < MAX_MT ? nt - t0 : MAX_MT;
        if (mt == 3) gemv_block_i16<3>(m, cb, R.at(t0));
        else if (mt == 2) gemv_block_i16<2>(m, cb, R.at(t0));
        else gemv_block_i16<1>(m, cb, R.at(t0));
    }
}

// ------------------------------------------------------------------------------------------------ a job

// The picks of one call grouped by expert: expert g's tokens are tok[first[g] .. first[g + 1]) (pick order).
// Every buffer lives here and keeps its capacity from job to job, so serving a job allocates only when it is
// larger than every job before it.
struct Job
{
    const Layer* L = nullptr;
    int H = 0, I = 0, T = 0, mode = 0;
    float limit = 0.0f;
    const float* x = nullptr;               // [T][H] fp32
    std::vector<int> gexp, first, tok;      // experts, token groups
    std::vector<float> wt;                  // weight of each group entry
    std::vector<int> pick_of;               // group entry of pick p (the combine's order)
    std::vector<int> tok_pick_start, tok_picks;   // picks of token t in pick order
    std::vector<int> cnt, slot, fill, tfill;      // grouping scratch
    // per group entry (expert e, token t): transformed inputs and intermediate rows
    std::vector<float> xt, xs, gu, xd, xds, yd;
    // I16 mode: int16 inputs and block scales of the gate/up inputs and of the down inputs
    std::vector<int16_t> xq, xdq;
    std::vector<float> qs, qds;
    float* out = nullptr;                   // [T][H]
};

static int group_of(const Job& J, int u)
{
    return (int)(std::upper_bound(J.first.begin(), J.first.end(), u) - J.first.begin()) - 1;
}

static void ph_input(void* c, int u)          // u = group entry
{
    Job& J = *static_cast<Job*>(c);
    const Expert& E = J.L->ex[J.gexp[group_of(J, u)]];
    const float* x = J.x + (size_t)J.tok[u] * J.H;
    float* xt = J.xt.data() + (size_t)u * 2 * J.H;
    J.xs[2 * u + 0] = prep_input(x, E.g.suh, J.H, xt);
    J.xs[2 * u + 1] = prep_input(x, E.u.suh, J.H, xt + J.H);
    if (J.mode == 2)
    {
        const int nb = J.H / 128;
        int16_t* xq = J.xq.data() + (size_t)u * 2 * J.H;
        float* qs = J.qs.data() + (size_t)u * 2 * nb;
        J.xs[2 * u + 0] = quant_i16(xt, J.H, xq, qs);
        J.xs[2 * u + 1] = quant_i16(xt + J.H, J.H, xq + J.H, qs + nb);
    }
}

static void ph_gateup(void* c, int u)         // u = (group, matrix, column block of I)
{
    Job& J = *static_cast<Job*>(c);
    const int ncb = J.I / 128;
    const int cb = u % ncb, mm = (u / ncb) % 2, g = u / (2 * ncb);
    const Expert& E = J.L->ex[J.gexp[g]];
    const Mat& M = mm == 0 ? E.g : E.u;
    const int f = J.first[g], nt = J.first[g + 1] - f;
    const Rows R = { J.xt.data() + (size_t)f * 2 * J.H + (size_t)mm * J.H, (size_t)2 * J.H,
                     J.xs.data() + 2 * (size_t)f + mm, 2,
                     J.gu.data() + (size_t)f * 2 * J.I + (size_t)mm * J.I + cb * 128, (size_t)2 * J.I };
    if (J.mode == 2)
    {
        const int nb = J.H / 128;
        const RowsI16 Q = { J.xq.data() + (size_t)f * 2 * J.H + (size_t)mm * J.H, (size_t)2 * J.H,
                            J.qs.data() + (size_t)f * 2 * nb + (size_t)mm * nb, (size_t)2 * nb, R.xs, R.sstride, R.y,
                            R.ystride };
        gemv_tokens_i16(M, cb, nt, Q);
    }
    else if (J.mode == 1) gemv_tokens<true>(M, cb, nt, R);
    else gemv_tokens<false>(M, cb, nt, R);
    for (int t = 0; t < nt; ++t) out_block(R.y + t * R.ystride, M.svh + cb * 128);
}

static void ph_act(void* c, int u)            // u = group entry: SwiGLU (in place of the gate row), down input
{
    Job& J = *static_cast<Job*>(c);
    const Expert& E = J.L->ex[J.gexp[group_of(J, u)]];
    float* gg = J.gu.data() + (size_t)u * 2 * J.I;
    const float* uu = gg + J.I;
    for (int i = 0; i < J.I; ++i) gg[i] = r16(act_gu(gg[i], uu[i], J.limit));
    J.xds[u] = prep_input(gg, E.d.suh, J.I, J.xd.data() + (size_t)u * J.I);
    if (J.mode == 2)
        J.xds[u] = quant_i16(J.xd.data() + (size_t)u * J.I, J.I, J.xdq.data() + (size_t)u * J.I,
                             J.qds.data() + (size_t)u * (J.I / 128));
}

static void ph_down(void* c, int u)           // u = (group, column block of H)
{
    Job& J = *static_cast<Job*>(c);
    const int ncb = J.H / 128;
    const int cb = u % ncb, g = u / ncb;
    const Mat& M = J.L->ex[J.gexp[g]].d;
    const int f = J.first[g], nt = J.first[g + 1] - f;
    const Rows R = { J.xd.data() + (size_t)f * J.I, (size_t)J.I, J.xds.data() + f, 1,
                     J.yd.data() + (size_t)f * J.H + cb * 128, (size_t)J.H };
    if (J.mode == 2)
    {
        const int nb = J.I / 128;
        const RowsI16 Q = { J.xdq.data() + (size_t)f * J.I, (size_t)J.I, J.qds.data() + (size_t)f * nb, (size_t)nb,
                            R.xs, R.sstride, R.y, R.ystride };
        gemv_tokens_i16(M, cb, nt, Q);
    }
    else if (J.mode == 1) gemv_tokens<true>(M, cb, nt, R);
    else gemv_tokens<false>(M, cb, nt, R);
    for (int t = 0; t < nt; ++t) out_block(R.y + t * R.ystride, M.svh + cb * 128);
}

static void ph_combine(void* c, int u)        // u = (token, 512-column chunk): out = sum of w * y in pick order
{
    Job& J = *static_cast<Job*>(c);
    const int nch = J.H / 512 > 0 ? J.H / 512 : 1;
    const int t = u / nch, ch = u % nch;
    const int h0 = ch * (J.H / nch), h1 = ch == nch - 1 ? J.H : h0 + J.H / nch;
    float* o = J.out + (size_t)t * J.H;
    for (int h = h0; h < h1; ++h) o[h] = 0.0f;
    for (int q = J.tok_pick_start[t]; q < J.tok_pick_start[t + 1]; ++q)
    {
        const int ge = J.pick_of[J.tok_picks[q]];
        const float w = J.wt[ge];
        const float* y = J.yd.data() + (size_t)ge * J.H;
        for (int h = h0; h < h1; ++h) o[h] = std::fma(w, y[h], o[h]);
    }
}

// Runs the picks (token, expert, weight) of one layer: out [T][H] (every token row written). The picks must name
// tokens in [0, T) and experts in [0, L.E).
static void run_picks(Pool& pool, const Layer& L, int H, int I, const float* x, int T, const int32_t* pt,
                      const int32_t* pe, const float* pw, int np, int mode, float limit, float* out, Job& J)
{
    J.L = &L;
    J.H = H;
    J.I = I;
    J.T = T;
    J.limit = limit;
    J.x = x;
    J.out = out;
    // group the picks by expert (ascending id), tokens in pick order
    J.cnt.assign(L.E, 0);
    for (int p = 0; p < np; ++p) J.cnt[pe[p]]++;
    J.gexp.clear();
    J.first.assign(1, 0);
    J.slot.assign(L.E, -1);
    for (int e = 0; e < L.E; ++e)
        if (J.cnt[e])
        {
            J.slot[e] = (int)J.gexp.size();
            J.gexp.push_back(e);
            J.first.push_back(J.first.back() + J.cnt[e]);
        }
    const int ng = (int)J.gexp.size();
    // mode: 0 AFFINE, 1 EXACT, 2 I16; automatic (-1): I16 if no expert has more than two rows, else AFFINE
    // (ft_tier_ext.cpp:130-132)
    int maxm = 0;
    for (int e : J.gexp) maxm = std::max(maxm, J.cnt[e]);
    J.mode = mode >= 0 ? mode : (maxm <= 2 ? 2 : 0);
    J.tok.assign(np, 0);
    J.wt.assign(np, 0.0f);
    J.pick_of.assign(np, 0);
    J.fill.assign(J.first.begin(), J.first.end() - 1);
    for (int p = 0; p < np; ++p)
    {
        const int ge = J.fill[J.slot[pe[p]]]++;
        J.tok[ge] = pt[p];
        J.wt[ge] = pw[p];
        J.pick_of[p] = ge;
    }
    J.tok_pick_start.assign(T + 1, 0);
    for (int p = 0; p < np; ++p) J.tok_pick_start[pt[p] + 1]++;
    for (int t = 0; t < T; ++t) J.tok_pick_start[t + 1] += J.tok_pick_start[t];
    J.tok_picks.assign(np, 0);
    J.tfill.assign(J.tok_pick_start.begin(), J.tok_pick_start.end() - 1);
    for (int p = 0; p < np; ++p) J.tok_picks[J.tfill[pt[p]]++] = p;
    J.xt.resize((size_t)np * 2 * H);
    J.xs.resize((size_t)np * 2);
    J.gu.resize((size_t)np * 2 * I);
    J.xd.resize((size_t)np * I);
    J.xds.resize((size_t)np);
    J.yd.resize((size_t)np * H);
    if (J.mode == 2)
    {
        J.xq.resize((size_t)np * 2 * H);
        J.qs.resize((size_t)np * 2 * (H / 128));
        J.xdq.resize((size_t)np * I);
        J.qds.resize((size_t)np * (I / 128));
    }
    if (np)
    {
        pool.run(ph_input, &J, np);
        pool.run(ph_gateup, &J, ng * 2 * (I / 128));
        pool.run(ph_act, &J, np);
        pool.run(ph_down, &J, ng * (H / 128));
    }
    pool.run(ph_combine, &J, T * (H / 512 > 0 ? H / 512 : 1));
}

// ------------------------------------------------------------------------------------------------ the tier

struct Tier
{
    Pool pool;
    std::vector<int> cpus;
    std::vector<Layer> layers;
    // the mailbox and its capacity: hx [maxtok][H] fp16, picks [maxpicks][3], hout [maxtok][H] fp32
    int64_t* ctrl = nullptr;
    const uint16_t* hx = nullptr;
    const int32_t* picks = nullptr;
    float* hout = nullptr;
    int maxtok = 0, maxpicks = 0;
    int H = 0, I = 0;
    // set at any time (mm_tier_set_mode / mm_tier_set_limit), read by the worker at each job
    std::atomic<int> mode{ -1 };
    std::atomic<float> limit{ 0.0f };
    std::thread th;
    std::atomic<bool> quit{ false }, running{ false };
    std::atomic<int64_t> jobs{ 0 }, experts{ 0 }, tokens{ 0 }, empty{ 0 }, busy_ns{ 0 }, rejected{ 0 }, stale{ 0 };
    std::vector<float> xf;
    std::vector<int32_t> pt, pe;
    std::vector<float> pw;
    Job job;
    void (*hook)(void*, int, int64_t) = nullptr;   // test hook (impl_set_test_hook)
    void* hook_arg = nullptr;
};

static Tier* g_tier = nullptr;

// mode: 0 AFFINE, 1 EXACT, 2 I16, -1 automatic (resolved per job in run_picks); anything else is automatic
static int eff_mode(int m) { return m >= 0 && m <= 2 ? m : -1; }

// The mailbox's x rows fp16 -> fp32. The words are read as relaxed atomics: the publisher may rewrite them while
// they are read (after a timed-out job), which the sequence check after the copy detects.
struct Convert
{
    const uint16_t* h;
    float* f;
    size_t n;
};
constexpr size_t CONVERT_UNIT = (size_t)1 << 15;     // halves per pool unit of a large job's conversion

static void convert_range(const uint16_t* h, float* f, size_t lo, size_t hi)
{
    size_t i = lo;
    if (((uintptr_t)(h + i) & 7) == 0)
        for (; i + 8 <= hi; i += 8)
        {
            const uint64_t a = __atomic_load_n(reinterpret_cast<const uint64_t*>(h + i), __ATOMIC_RELAXED);
            const uint64_t b = __atomic_load_n(reinterpret_cast<const uint64_t*>(h + i + 4), __ATOMIC_RELAXED);
            _mm256_storeu_ps(f + i, _mm256_cvtph_ps(_mm_set_epi64x((long long)b, (long long)a)));
        }
    for (; i < hi; ++i) f[i] = h2f(__atomic_load_n(h + i, __ATOMIC_RELAXED));
}

static void ph_convert(void* c, int u)
{
    const Convert& C = *static_cast<const Convert*>(c);
    const size_t lo = (size_t)u * CONVERT_UNIT, hi = std::min(C.n, lo + CONVERT_UNIT);
    convert_range(C.h, C.f, lo, hi);
}

// One published job, sequence s. The sizes come from the mailbox: a job larger than the mailbox, or naming a
// layer that was never added, is not computed (the rows of hout that exist are zeroed, so the combine adds
// nothing) and counted as rejected. The x rows and the picks are copied out first; if the sequence moved on
// meanwhile, the publisher (the GPU split, after the combine gave up waiting for this job) has been rewriting
// them, the copy may be torn, and the job is dropped and counted as stale: nobody waits for its partial any more.
static void serve_job(Tier& Tr, int64_t s, int64_t li, int64_t bsz, int64_t np)
{
    const int H = Tr.H;
    if (li < 0 || li >= (int64_t)Tr.layers.size() || Tr.layers[(size_t)li].E <= 0 || bsz < 0 || np < 0 ||
        bsz > Tr.maxtok || np > Tr.maxpicks)
    {
        const int64_t rows = bsz < 0 ? 0 : (bsz > Tr.maxtok ? Tr.maxtok : bsz);
        memset(Tr.hout, 0, (size_t)rows * H * sizeof(float));
        Tr.rejected++;
        return;
    }
    const size_t nx = (size_t)bsz * H;
    Tr.xf.resize(nx > 0 ? nx : 1);
    if (nx > CONVERT_UNIT)
    {
        Convert C = { Tr.hx, Tr.xf.data(), nx };
        Tr.pool.run(ph_convert, &C, (int)((nx + CONVERT_UNIT - 1) / CONVERT_UNIT));
    }
    else
        convert_range(Tr.hx, Tr.xf.data(), 0, nx);
    // picks whose token or expert is out of range are left out (as mm_tier_forward leaves them out), so a
    // malformed job cannot index past the layer's experts or the job's rows
    const Layer& L = Tr.layers[(size_t)li];
    Tr.pt.resize((size_t)np);
    Tr.pe.resize((size_t)np);
    Tr.pw.resize((size_t)np);
    int nk = 0;
    for (int64_t p = 0; p < np; ++p)
    {
        const int32_t t = __atomic_load_n(Tr.picks + 3 * p, __ATOMIC_RELAXED);
        const int32_t e = __atomic_load_n(Tr.picks + 3 * p + 1, __ATOMIC_RELAXED);
        const int32_t wb = __atomic_load_n(Tr.picks + 3 * p + 2, __ATOMIC_RELAXED);
        if (t < 0 || t >= bsz || e < 0 || e >= L.E) continue;
        Tr.pt[nk] = t;
        Tr.pe[nk] = e;
        memcpy(&Tr.pw[nk], &wb, 4);
        ++nk;
    }
    if (Tr.hook) Tr.hook(Tr.hook_arg, 0, s);
    // every read of the copy above happens before the sequence is read again
    std::atomic_thread_fence(std::memory_order_acquire);
    if (__atomic_load_n(Tr.ctrl, __ATOMIC_RELAXED) != s)
    {
        Tr.stale++;
        return;
    }
    run_picks(Tr.pool, L, H, Tr.I, Tr.xf.data(), (int)bsz, Tr.pt.data(), Tr.pe.data(), Tr.pw.data(), nk,
              eff_mode(Tr.mode.load()), Tr.limit.load(), Tr.hout, Tr.job);
    if (Tr.hook) Tr.hook(Tr.hook_arg, 1, s);
    if (np == 0) Tr.empty++;
    Tr.experts += nk;
    Tr.tokens += bsz;
}

// `last` is the job sequence when the tier started: read by the starting thread, so a job published right after
// mm_tier_start returns is not mistaken for an old one. Every job seen is answered with ctrl[1] = its sequence,
// computed or not; the combine waits for its own sequence only, so an answer to an older job is never taken for
// a newer one.
static void worker_main(Tier* Tr, int cpu0, int64_t last)
{
    Pool::pin(cpu0);
    long idle = 0;
    while (!Tr->quit.load(std::memory_order_relaxed))
    {
        const int64_t s = __atomic_load_n(Tr->ctrl, __ATOMIC_ACQUIRE);
        if (s == last)
        {
            if (++idle < 400000) _mm_pause();
            else usleep(20);
            continue;
        }
        idle = 0;
        const double t0 = now_s();
        serve_job(*Tr, s, __atomic_load_n(Tr->ctrl + 2, __ATOMIC_RELAXED), __atomic_load_n(Tr->ctrl + 3, __ATOMIC_RELAXED),
                  __atomic_load_n(Tr->ctrl + 4, __ATOMIC_RELAXED));
        Tr->busy_ns += (int64_t)((now_s() - t0) * 1e9);
        Tr->jobs++;
        last = s;
        __atomic_store_n(Tr->ctrl + 1, s, __ATOMIC_RELEASE);
    }
}

}  // namespace tier

namespace tier {

// At process exit the worker and the pool must be gone before the memory they read (the pinned mailbox and the
// expert homes, which the GPU runtime releases at its own teardown) is: exit handlers run in the reverse order of
// their registration, and this one is registered after the runtime and the caller's buffers exist.
static void at_exit()
{
    impl_shutdown();
}

int impl_init(int threads, const int* cpus, int ncpus, int64_t* ctrl, const void* hx, const int32_t* picks,
              float* hout, int maxtok, int maxpicks, int mode, int H, int I, int nlayers)
{
    static bool exit_hook = false;
    if (g_tier) return set_error(MM_ERR_ARG, "mm_tier_init: the tier is already initialised");
    if (threads < 1 || H <= 0 || I <= 0 || H % 512 || I % 128 || nlayers <= 0 || (ncpus > 0 && !cpus))
        return set_error(MM_ERR_ARG, "mm_tier_init: need threads >= 1, H a multiple of 512, I of 128, nlayers > 0");
    const bool mailbox = ctrl || hx || picks || hout;
    if (mailbox && (!ctrl || !hx || !picks || !hout || maxtok <= 0 || maxpicks <= 0))
        return set_error(MM_ERR_ARG, "mm_tier_init: a mailbox needs ctrl, hx, picks and hout and capacities maxtok > 0, "
                                     "maxpicks > 0 (got %d, %d)", maxtok, maxpicks);
    if (!exit_hook)
    {
        if (atexit(at_exit) != 0) return set_error(MM_ERR_ARG, "mm_tier_init: atexit failed");
        exit_hook = true;
    }
    Tier* T = new Tier();
    if (ncpus > 0) T->cpus.assign(cpus, cpus + ncpus);
    T->ctrl = ctrl;
    T->hx = static_cast<const uint16_t*>(hx);
    T->picks = picks;
    T->hout = hout;
    T->maxtok = mailbox ? maxtok : 0;
    T->maxpicks = mailbox ? maxpicks : 0;
    T->mode.store(mode);
    T->H = H;
    T->I = I;
    T->layers.resize(nlayers);
    T->pool.start(T->cpus, threads);
    g_tier = T;
    return MM_OK;
}

int impl_add_layer(int li, int E, const int64_t* ptrs, const void* suh_g, const void* svh_g, const void* suh_u,
                      const void* svh_u, const void* suh_d, const void* svh_d)
{
    Tier* T = g_tier;
    if (!T) return set_error(MM_ERR_ARG, "mm_tier_add_layer: mm_tier_init first");
    if (li < 0 || li >= (int)T->layers.size() || E <= 0 || !ptrs || !suh_g || !svh_g || !suh_u || !svh_u || !suh_d || !svh_d)
        return set_error(MM_ERR_ARG, "mm_tier_add_layer: bad layer index, expert count or null pointer");
    if (T->running.load()) return set_error(MM_ERR_ARG, "mm_tier_add_layer: the worker is running");
    const int H = T->H, I = T->I;
    auto u16 = [](const void* p, size_t off) { return static_cast<const uint16_t*>(p) + off; };
    Layer& L = T->layers[li];
    L.E = E;
    L.ex.assign(E, Expert());
    for (int e = 0; e < E; ++e)
    {
        Expert& X = L.ex[e];
        X.g = { reinterpret_cast<const uint8_t*>(ptrs[3 * e]), u16(suh_g, (size_t)e * H), u16(svh_g, (size_t)e * I), H, I };
        X.u = { reinterpret_cast<const uint8_t*>(ptrs[3 * e + 1]), u16(suh_u, (size_t)e * H), u16(svh_u, (size_t)e * I), H, I };
        X.d = { reinterpret_cast<const uint8_t*>(ptrs[3 * e + 2]), u16(suh_d, (size_t)e * I), u16(svh_d, (size_t)e * H), I, H };
    }
    return MM_OK;
}

int impl_set_limit(float limit)
{
    if (!g_tier) return set_error(MM_ERR_ARG, "mm_tier_set_limit: mm_tier_init first");
    g_tier->limit.store(limit);
    return MM_OK;
}

int impl_set_mode(int mode)
{
    if (!g_tier) return set_error(MM_ERR_ARG, "mm_tier_set_mode: mm_tier_init first");
    g_tier->mode.store(mode);
    return MM_OK;
}

int impl_start(int cpu0)
{
    Tier* T = g_tier;
    if (!T || T->running.load()) return set_error(MM_ERR_ARG, "mm_tier_start: not initialised or already running");
    if (!T->ctrl || !T->hx || !T->picks || !T->hout)
        return set_error(MM_ERR_ARG, "mm_tier_start: the mailbox (ctrl, hx, picks, hout) was not given to mm_tier_init");
    T->quit.store(false);
    T->running.store(true);
    T->th = std::thread(worker_main, T, cpu0, __atomic_load_n(T->ctrl, __ATOMIC_ACQUIRE));
    return MM_OK;
}

int impl_stop()
{
    Tier* T = g_tier;
    if (!T) return MM_OK;
    if (T->running.load())
    {
        T->quit.store(true);
        if (T->th.joinable()) T->th.join();
        T->running.store(false);
    }
    return MM_OK;
}

int impl_shutdown()
{
    Tier* T = g_tier;
    if (!T) return MM_OK;
    impl_stop();
    T->pool.stop();
    delete T;
    g_tier = nullptr;
    return MM_OK;
}

int impl_forward(int li, const float* x, int m, const int32_t* sel, const float* w, int k, float* out, int mode)
{
    Tier* T = g_tier;
    if (!T) return set_error(MM_ERR_ARG, "mm_tier_forward: mm_tier_init first");
    if (T->running.load()) return set_error(MM_ERR_ARG, "mm_tier_forward: the worker is running");
    if (li < 0 || li >= (int)T->layers.size() || T->layers[li].E <= 0 || m < 0 || k <= 0 || !x || !sel || !w || !out)
        return set_error(MM_ERR_ARG, "mm_tier_forward: bad layer or argument");
    const int E = T->layers[li].E;
    T->pt.clear();
    T->pe.clear();
    T->pw.clear();
    for (int t = 0; t < m; ++t)
        for (int j = 0; j < k; ++j)
        {
            const int e = sel[(size_t)t * k + j];
            if (e < 0 || e >= E) continue;
            T->pt.push_back(t);
            T->pe.push_back(e);
            T->pw.push_back(w[(size_t)t * k + j]);
        }
    run_picks(T->pool, T->layers[li], T->H, T->I, x, m, T->pt.data(), T->pe.data(), T->pw.data(), (int)T->pt.size(),
              eff_mode(mode >= 0 ? mode : T->mode.load()), T->limit.load(), out, T->job);
    return MM_OK;
}

int impl_stats(int64_t* out)
{
    Tier* T = g_tier;
    if (!out) return set_error(MM_ERR_ARG, "mm_tier_stats: null pointer");
    if (!T)
    {
        for (int i = 0; i < MM_TIER_NSTATS; ++i) out[i] = 0;
        return MM_OK;
    }
    out[0] = T->jobs.load();
    out[1] = T->experts.load();
    out[2] = T->tokens.load();
    out[3] = T->empty.load();
    out[4] = T->busy_ns.load();
    out[5] = T->rejected.load();
    out[6] = T->stale.load();
    return MM_OK;
}

int impl_set_test_hook(void (*fn)(void*, int, int64_t), void* arg)
{
    Tier* T = g_tier;
    if (!T) return set_error(MM_ERR_ARG, "impl_set_test_hook: mm_tier_init first");
    if (T->running.load()) return set_error(MM_ERR_ARG, "impl_set_test_hook: the worker is running");
    T->hook = fn;
    T->hook_arg = arg;
    return MM_OK;
}

}  // namespace tier
