// Sanitizer driver of the host expert tier (host code only, built by sanitize_check.sh with g++ under
// ThreadSanitizer and under AddressSanitizer + UBSan). A layer of random experts and a mailbox allocated at exactly
// its stated capacity (so a read or write past it is reported), served by the tier's worker the way the decode
// split publishes jobs (the payload, then the sequence with release ordering; every mailbox word written as a
// relaxed atomic, as the GPU's stores are to the worker). Cases:
//   serve     24 jobs while another thread sets the mode and the SwiGLU limit and reads the statistics; every
//             partial equals the synchronous forward of the same picks bit for bit
//   oversize  jobs with more tokens or picks than the mailbox holds, and one naming a layer never added: each is
//             answered, counted as rejected, and zeroes the hout rows that exist
//   republish the next job is published while the worker is still copying the current one (the combine gave up
//             on it): that job is dropped as stale and the next one is served from its own payload
//   late      the next job is published after the worker copied the current one but before it answered (a
//             worker that finishes after the combine's timeout): the answer to the next job carries the next
//             job's partial only
//   exit      (separate run, argument "exit") the process exits while the worker is inside a job; the mailbox is
//             freed by an exit handler registered before the tier's, as the GPU runtime releases pinned memory at
//             its own teardown; the tier's handler must stop the worker first
// Exits 0 when every check passes; a race or an invalid access is reported by the sanitizer, which fails the run.
#include <atomic>
#include <chrono>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <immintrin.h>
#include <random>
#include <thread>
#include <vector>

#include "host_tier.h"

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
            fprintf(stderr, "host_tier_check: " __VA_ARGS__);                                                        \
            fprintf(stderr, " (%s)\n", mm_last_error());                                                             \
            return 1;                                                                                                \
        }                                                                                                            \
    } while (0)

namespace {

constexpr int H = 512, I = 256, E = 8, T = 4, K = 3;
constexpr int MAXTOK = T, MAXPICKS = T * K;

struct Layer
{
    std::vector<std::vector<uint16_t>> mats;
    std::vector<int64_t> ptrs;
    std::vector<uint16_t> suh_g, svh_g, suh_u, svh_u, suh_d, svh_d;
};

// expert rows (gate, up, down trellis) and scales: suh = +-1, svh small positive
void make_layer(Layer& L, std::mt19937& rng)
{
    auto tiles = [](int k, int n) { return (size_t)(k / 16) * (n / 16) * 48; };
    L.mats.clear();
    L.mats.reserve(3 * E);
    L.ptrs.assign(3 * E, 0);
    for (int e = 0; e < E; ++e)
        for (int m = 0; m < 3; ++m)
        {
            std::vector<uint16_t> t(m < 2 ? tiles(H, I) : tiles(I, H));
            for (auto& v : t) v = (uint16_t)rng();
            L.mats.push_back(std::move(t));
            L.ptrs[3 * e + m] = (int64_t)(uintptr_t)L.mats.back().data();
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
    L.suh_g = signs((size_t)E * H);
    L.svh_g = small((size_t)E * I);
    L.suh_u = signs((size_t)E * H);
    L.svh_u = small((size_t)E * I);
    L.suh_d = signs((size_t)E * I);
    L.svh_d = small((size_t)E * H);
}

// The mailbox at exactly its capacity, on the heap.
struct Mailbox
{
    int64_t* ctrl;
    uint16_t* hx;
    int32_t* picks;
    float* hout;
    Mailbox()
    {
        ctrl = new int64_t[16]();
        hx = new uint16_t[(size_t)MAXTOK * H]();
        picks = new int32_t[(size_t)MAXPICKS * 3]();
        hout = new float[(size_t)MAXTOK * H]();
    }
    void free_all()
    {
        delete[] ctrl;
        delete[] hx;
        delete[] picks;
        delete[] hout;
        ctrl = nullptr;
    }
};

struct JobData
{
    std::vector<float> x;
    std::vector<int32_t> sel;
    std::vector<float> w, want;
};

std::vector<JobData> make_jobs(int n, std::mt19937& rng)
{
    std::vector<JobData> jobs((size_t)n);
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
    }
    return jobs;
}

// Publishes a job the way the split does: payload words (relaxed atomics), sizes, then the sequence (release).
void publish(Mailbox& M, const JobData& j, int64_t seq, int64_t li = 0, int64_t bsz = T, int64_t np_override = -1)
{
    for (size_t i = 0; i + 4 <= (size_t)T * H; i += 4)
    {
        uint64_t v = 0;
        for (int q = 0; q < 4; ++q) v |= (uint64_t)_cvtss_sh(j.x[i + q], 0) << (16 * q);
        __atomic_store_n(reinterpret_cast<uint64_t*>(M.hx + i), v, __ATOMIC_RELAXED);
    }
    int np = 0;
    for (int t = 0; t < T; ++t)
        for (int k = 0; k < K; ++k)
        {
            int32_t wb;
            memcpy(&wb, &j.w[(size_t)t * K + k], 4);
            __atomic_store_n(&M.picks[3 * np], (int32_t)t, __ATOMIC_RELAXED);
            __atomic_store_n(&M.picks[3 * np + 1], j.sel[(size_t)t * K + k], __ATOMIC_RELAXED);
            __atomic_store_n(&M.picks[3 * np + 2], wb, __ATOMIC_RELAXED);
            ++np;
        }
    __atomic_store_n(&M.ctrl[2], li, __ATOMIC_RELAXED);
    __atomic_store_n(&M.ctrl[3], bsz, __ATOMIC_RELAXED);
    __atomic_store_n(&M.ctrl[4], np_override >= 0 ? np_override : (int64_t)np, __ATOMIC_RELAXED);
    __atomic_store_n(&M.ctrl[0], seq, __ATOMIC_RELEASE);
}

bool wait_done(const Mailbox& M, int64_t seq)
{
    const auto t0 = std::chrono::steady_clock::now();
    while (__atomic_load_n(&M.ctrl[1], __ATOMIC_ACQUIRE) != seq)
    {
        if (std::chrono::steady_clock::now() - t0 > std::chrono::seconds(60)) return false;
        std::this_thread::yield();
    }
    return true;
}

// hout against an expected partial (read after the answer: the worker's stores happen before its release of ctrl[1])
bool hout_equals(const Mailbox& M, const std::vector<float>& want)
{
    return memcmp(M.hout, want.data(), want.size() * sizeof(float)) == 0;
}

// The test hook: when the worker reaches `stage` of job `seq`, it asks the main thread to publish the next job
// and waits until it has.
struct Hook
{
    std::atomic<int> stage{ -1 };
    std::atomic<int64_t> seq{ -1 }, asked{ -1 }, answered{ -1 };
    std::atomic<int> sleep_ms{ 0 };
};

void hook_fn(void* arg, int stage, int64_t s)
{
    Hook& h = *static_cast<Hook*>(arg);
    if (h.sleep_ms.load() > 0 && stage == 1) std::this_thread::sleep_for(std::chrono::milliseconds(h.sleep_ms.load()));
    if (stage != h.stage.load() || s != h.seq.load()) return;
    h.asked.store(s);
    while (h.answered.load() != s) std::this_thread::yield();
}

int64_t stat(int i)
{
    int64_t st[MM_TIER_NSTATS];
    tier::impl_stats(st);
    return st[i];
}

int setup(Layer& L, Mailbox& M, Hook& hook, std::mt19937& rng)
{
    make_layer(L, rng);
    std::vector<int> cpus;
    CHECK(mm_tier_init(3, cpus.data(), 0, M.ctrl, M.hx, M.picks, M.hout, MAXTOK, MAXPICKS, 0, H, I, 2) == MM_OK,
          "init");
    CHECK(mm_tier_add_layer(0, E, L.ptrs.data(), L.suh_g.data(), L.svh_g.data(), L.suh_u.data(), L.svh_u.data(),
                            L.suh_d.data(), L.svh_d.data()) == MM_OK, "add_layer");
    CHECK(mm_tier_set_limit(10.0f) == MM_OK, "set_limit");
    CHECK(tier::impl_set_test_hook(hook_fn, &hook) == MM_OK, "hook");
    return 0;
}

int run_serve()
{
    std::mt19937 rng(7);
    Layer L;
    Mailbox M;
    Hook hook;
    if (setup(L, M, hook, rng)) return 1;
    const int JOBS = 24;
    std::vector<JobData> jobs = make_jobs(JOBS + 4, rng);
    for (auto& j : jobs)           // expected partials (synchronous forward before the worker starts)
        CHECK(mm_tier_forward(0, j.x.data(), T, j.sel.data(), j.w.data(), K, j.want.data(), 0) == MM_OK, "forward");

    CHECK(mm_tier_start(-1) == MM_OK, "start");
    std::atomic<bool> stop{ false };
    std::thread poker([&] {           // setters and statistics while the worker serves jobs
        int64_t st[MM_TIER_NSTATS];
        while (!stop.load())
        {
            mm_tier_set_mode(0);
            mm_tier_set_limit(10.0f);
            mm_tier_stats(st);
            std::this_thread::yield();
        }
    });
    int64_t seq = 0;
    // serve
    int bad = 0;
    for (int n = 0; n < JOBS; ++n)
    {
        publish(M, jobs[(size_t)n], ++seq);
        CHECK(wait_done(M, seq), "job %d not answered", n);
        if (!hout_equals(M, jobs[(size_t)n].want)) ++bad;
    }
    CHECK(bad == 0, "serve: %d of %d job partials differ from the synchronous forward", bad, JOBS);
    CHECK(stat(0) == JOBS && stat(5) == 0 && stat(6) == 0, "serve: stats %lld jobs", (long long)stat(0));

    // oversize: too many tokens, too many picks, an unknown layer (the hout rows that exist are zeroed)
    const int64_t oversize[3][3] = { { 0, MAXTOK + 1, MAXPICKS }, { 0, T, MAXPICKS + 1 }, { 1, T, MAXPICKS } };
    for (int c = 0; c < 3; ++c)
    {
        for (size_t i = 0; i < (size_t)MAXTOK * H; ++i) M.hout[i] = 1.0f;
        publish(M, jobs[0], ++seq, oversize[c][0], oversize[c][1], oversize[c][2]);
        CHECK(wait_done(M, seq), "oversize job %d not answered", c);
        CHECK(hout_equals(M, std::vector<float>((size_t)MAXTOK * H, 0.0f)), "oversize job %d: hout not zeroed", c);
    }
    CHECK(stat(5) == 3, "oversize: %lld rejected, expected 3", (long long)stat(5));

    // republish: job A is rewritten by job B while the worker copies A
    {
        const int64_t a = ++seq, b = ++seq;
        hook.seq.store(a);
        hook.stage.store(0);
        publish(M, jobs[(size_t)JOBS], a);
        while (hook.asked.load() != a) std::this_thread::yield();
        publish(M, jobs[(size_t)JOBS + 1], b);
        hook.answered.store(a);
        CHECK(wait_done(M, b), "republish: job B not answered");
        CHECK(hout_equals(M, jobs[(size_t)JOBS + 1].want), "republish: job B's partial differs");
        CHECK(stat(6) == 1, "republish: %lld stale jobs, expected 1", (long long)stat(6));
    }

    // late: job D is published after the worker copied job C, before it answered C
    {
        const int64_t c = ++seq, d = ++seq;
        hook.seq.store(c);
        hook.stage.store(1);
        publish(M, jobs[(size_t)JOBS + 2], c);
        while (hook.asked.load() != c) std::this_thread::yield();
        publish(M, jobs[(size_t)JOBS + 3], d);
        hook.answered.store(c);
        CHECK(wait_done(M, d), "late: job D not answered");
        CHECK(hout_equals(M, jobs[(size_t)JOBS + 3].want), "late: job D's partial differs");
        CHECK(stat(6) == 1, "late: %lld stale jobs, expected 1", (long long)stat(6));
    }
    stop.store(true);
    poker.join();
    CHECK(mm_tier_stop() == MM_OK, "stop");
    // the pool again, synchronously, after the worker stopped
    std::vector<float> again((size_t)T * H);
    CHECK(mm_tier_forward(0, jobs[0].x.data(), T, jobs[0].sel.data(), jobs[0].w.data(), K, again.data(), 0) == MM_OK &&
              memcmp(again.data(), jobs[0].want.data(), again.size() * 4) == 0, "forward after stop");
    CHECK(mm_tier_shutdown() == MM_OK, "shutdown");
    M.free_all();
    printf("host_tier_check: %d jobs served bit-identical to the synchronous forward; 3 oversize jobs rejected; "
           "a republished job dropped as stale; a late answer not taken for the next job\n", JOBS);
    return 0;
}

// exit: the process ends while the worker is inside a job. The mailbox is released by an exit handler registered
// before mm_tier_init, so it runs after the tier's own handler.
Mailbox* g_exit_mailbox = nullptr;

void free_exit_mailbox()
{
    if (!g_exit_mailbox) return;
    g_exit_mailbox->free_all();
    // teardown goes on after the release: a worker still running would now touch the freed mailbox
    std::this_thread::sleep_for(std::chrono::milliseconds(200));
}

int run_exit()
{
    std::mt19937 rng(11);
    static Layer L;              // outlives main: the worker may read it until the tier's exit handler ran
    static Mailbox M;
    static Hook hook;
    g_exit_mailbox = &M;
    atexit(free_exit_mailbox);
    if (setup(L, M, hook, rng)) return 1;
    std::vector<JobData> jobs = make_jobs(1, rng);
    hook.sleep_ms.store(50);
    CHECK(mm_tier_start(-1) == MM_OK, "start");
    publish(M, jobs[0], 1);
    std::this_thread::sleep_for(std::chrono::milliseconds(10));
    printf("host_tier_check: exiting with the worker inside a job\n");
    fflush(stdout);
    exit(0);
}

}  // namespace

int main(int argc, char** argv)
{
    if (argc > 1 && strcmp(argv[1], "exit") == 0) return run_exit();
    return run_serve();
}
