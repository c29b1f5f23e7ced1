// ThreadSanitizer driver of the host expert tier (host code only, built by tsan_check.sh with g++): a layer of
// random experts, the mailbox worker serving jobs published the way the decode split publishes them, a second
// thread changing the mode and the SwiGLU limit and reading the statistics meanwhile, then the synchronous forward
// on the pool. Every job's partial must equal the synchronous forward of the same picks bit for bit. Exits 0 when
// every check passes (a race is reported by the sanitizer, which then fails the run).
#include <atomic>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <immintrin.h>
#include <random>
#include <thread>
#include <vector>

#include "../../include/mi355moe.h"

namespace mm {
// the library's error slot (defined in the HIP sources of the full build)
thread_local char g_err[512];
int set_error(int code, const char* fmt, ...)
{
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return code;
}
}  // namespace mm

extern "C" const char* mm_last_error(void) { return mm::g_err; }

#define CHECK(c, ...)                                                                                                \
    do {                                                                                                             \
        if (!(c)) {                                                                                                  \
            fprintf(stderr, "host_tier_tsan: " __VA_ARGS__);                                                         \
            fprintf(stderr, " (%s)\n", mm_last_error());                                                             \
            return 1;                                                                                                \
        }                                                                                                            \
    } while (0)

int main()
{
    const int H = 512, I = 256, E = 8, T = 4, K = 3, JOBS = 24;
    std::mt19937 rng(7);
    auto tiles = [](int k, int n) { return (size_t)(k / 16) * (n / 16) * 48; };
    // expert rows (gate, up, down trellis) and scales: suh = +-1, svh small positive
    std::vector<std::vector<uint16_t>> mats;
    std::vector<int64_t> ptrs(3 * E);
    for (int e = 0; e < E; ++e)
        for (int m = 0; m < 3; ++m)
        {
            std::vector<uint16_t> t(m < 2 ? tiles(H, I) : tiles(I, H));
            for (auto& v : t) v = (uint16_t)rng();
            mats.push_back(std::move(t));
            ptrs[3 * e + m] = (int64_t)(uintptr_t)mats.back().data();
        }
    auto signs = [&](size_t n) {
        std::vector<uint16_t> v(n);
        for (auto& x : v) x = (rng() & 1) ? 0x3C00 : 0xBC00;
        return v;
    };
    auto small = [&](size_t n) {
        std::vector<uint16_t> v(n);
        for (auto& x : v) x = (uint16_t)(0x2000 + (rng() & 0x3FF));
        return v;
    };
    std::vector<uint16_t> suh_g = signs((size_t)E * H), svh_g = small((size_t)E * I), suh_u = signs((size_t)E * H),
                          svh_u = small((size_t)E * I), suh_d = signs((size_t)E * I), svh_d = small((size_t)E * H);

    // the mailbox: ctrl [16], hx fp16 [T][H], picks [T*K][3], hout fp32 [T][H]
    std::vector<int64_t> ctrl(16, 0);
    std::vector<uint16_t> hx((size_t)T * H);
    std::vector<int32_t> picks((size_t)T * K * 3);
    std::vector<float> hout((size_t)T * H);
    std::vector<int> cpus;
    CHECK(mm_tier_init(3, cpus.data(), 0, ctrl.data(), hx.data(), picks.data(), hout.data(), 0, H, I, 1) == MM_OK,
          "init");
    CHECK(mm_tier_add_layer(0, E, ptrs.data(), suh_g.data(), svh_g.data(), suh_u.data(), svh_u.data(), suh_d.data(),
                            svh_d.data()) == MM_OK, "add_layer");
    CHECK(mm_tier_set_limit(10.0f) == MM_OK, "set_limit");

    // the jobs and their expected partials (synchronous forward before the worker starts)
    struct JobData
    {
        std::vector<float> x;
        std::vector<int32_t> sel;
        std::vector<float> w, want;
    };
    std::vector<JobData> jobs(JOBS);
    std::normal_distribution<float> nd(0.f, 1.f);
    std::uniform_real_distribution<float> ud(0.1f, 1.f);
    for (auto& j : jobs)
    {
        j.x.resize((size_t)T * H);
        for (auto& v : j.x) v = _cvtsh_ss(_cvtss_sh(nd(rng), 0));       // fp16 values, as the mailbox carries them
        j.sel.resize((size_t)T * K);
        for (int t = 0; t < T; ++t)
            for (int k = 0; k < K; ++k) j.sel[(size_t)t * K + k] = (int32_t)((t + 3 * k + (int)(rng() % 2)) % E);
        j.w.resize((size_t)T * K);
        for (auto& v : j.w) v = ud(rng);
        j.want.assign((size_t)T * H, 0.f);
        CHECK(mm_tier_forward(0, j.x.data(), T, j.sel.data(), j.w.data(), K, j.want.data(), 0) == MM_OK, "forward");
    }

    CHECK(mm_tier_start(-1) == MM_OK, "start");
    std::atomic<bool> stop{ false };
    std::thread poker([&] {           // setters and statistics while the worker serves jobs
        int64_t st[5];
        while (!stop.load())
        {
            mm_tier_set_mode(0);
            mm_tier_set_limit(10.0f);
            mm_tier_stats(st);
            std::this_thread::yield();
        }
    });
    int bad = 0;
    for (int n = 0; n < JOBS; ++n)
    {
        const JobData& j = jobs[(size_t)n];
        for (size_t i = 0; i < hx.size(); ++i) hx[i] = _cvtss_sh(j.x[i], 0);
        int np = 0;
        for (int t = 0; t < T; ++t)
            for (int k = 0; k < K; ++k)
            {
                picks[3 * np] = t;
                picks[3 * np + 1] = j.sel[(size_t)t * K + k];
                memcpy(&picks[3 * np + 2], &j.w[(size_t)t * K + k], 4);
                ++np;
            }
        __atomic_store_n(&ctrl[2], (int64_t)0, __ATOMIC_RELAXED);
        __atomic_store_n(&ctrl[3], (int64_t)T, __ATOMIC_RELAXED);
        __atomic_store_n(&ctrl[4], (int64_t)np, __ATOMIC_RELAXED);
        __atomic_store_n(&ctrl[0], (int64_t)(n + 1), __ATOMIC_RELEASE);     // the payload before the sequence
        long spins = 0;
        while (__atomic_load_n(&ctrl[1], __ATOMIC_ACQUIRE) != n + 1)
        {
            CHECK(++spins < 200000000L, "job %d not answered", n);
            std::this_thread::yield();
        }
        if (memcmp(hout.data(), j.want.data(), hout.size() * 4) != 0) ++bad;
    }
    stop.store(true);
    poker.join();
    CHECK(mm_tier_stop() == MM_OK, "stop");
    CHECK(bad == 0, "%d of %d job partials differ from the synchronous forward", bad, JOBS);
    int64_t st[5];
    CHECK(mm_tier_stats(st) == MM_OK && st[0] == JOBS, "stats: %lld jobs", (long long)st[0]);
    // the pool again, synchronously, after the worker stopped
    std::vector<float> again((size_t)T * H);
    CHECK(mm_tier_forward(0, jobs[0].x.data(), T, jobs[0].sel.data(), jobs[0].w.data(), K, again.data(), 0) == MM_OK &&
              memcmp(again.data(), jobs[0].want.data(), again.size() * 4) == 0, "forward after stop");
    CHECK(mm_tier_shutdown() == MM_OK, "shutdown");
    printf("host_tier_tsan: %d jobs served, partials bit-identical to the synchronous forward\n", JOBS);
    return 0;
}
