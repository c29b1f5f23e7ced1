// C ABI of the host expert tier. Compiled for the baseline x86-64 target: the implementation (host_tier.cpp) uses
// AVX-512 throughout, so nothing of it may run before mm_tier_init has checked that the host supports it.
#include "host_tier.h"

namespace {

bool cpu_ok()
{
    __builtin_cpu_init();
    return __builtin_cpu_supports("avx512f") && __builtin_cpu_supports("avx512bw") &&
           __builtin_cpu_supports("avx512vl") && __builtin_cpu_supports("avx512vbmi2") &&
           __builtin_cpu_supports("avx512vnni") && __builtin_cpu_supports("f16c") && __builtin_cpu_supports("fma");
}

bool g_ok = false;     // the CPU passed the check in mm_tier_init

}  // namespace

extern "C" {

int mm_tier_init(int threads, const int* cpus, int ncpus, int64_t* ctrl, const void* hx, const int32_t* picks,
                 float* hout, int maxtok, int maxpicks, int mode, int H, int I, int nlayers)
{
    if (!cpu_ok())
        return mm::set_error(MM_ERR_UNSUP, "mm_tier_init: the host tier needs AVX-512 (F, BW, VL, VBMI2, VNNI), F16C and FMA");
    g_ok = true;
    return tier::impl_init(threads, cpus, ncpus, ctrl, hx, picks, hout, maxtok, maxpicks, mode, H, I, nlayers);
}

#define NEED_INIT(who) \
    do { if (!g_ok) return mm::set_error(MM_ERR_ARG, who ": mm_tier_init first"); } while (0)

int mm_tier_add_layer(int li, int E, const int64_t* ptrs, const void* suh_g, const void* svh_g, const void* suh_u,
                      const void* svh_u, const void* suh_d, const void* svh_d)
{
    NEED_INIT("mm_tier_add_layer");
    return tier::impl_add_layer(li, E, ptrs, suh_g, svh_g, suh_u, svh_u, suh_d, svh_d);
}

int mm_tier_set_limit(float limit)
{
    NEED_INIT("mm_tier_set_limit");
    return tier::impl_set_limit(limit);
}

int mm_tier_set_mode(int mode)
{
    NEED_INIT("mm_tier_set_mode");
    return tier::impl_set_mode(mode);
}

int mm_tier_start(int cpu0)
{
    NEED_INIT("mm_tier_start");
    return tier::impl_start(cpu0);
}

int mm_tier_stop(void)
{
    if (!g_ok) return MM_OK;
    return tier::impl_stop();
}

int mm_tier_shutdown(void)
{
    if (!g_ok) return MM_OK;
    return tier::impl_shutdown();
}

int mm_tier_forward(int li, const float* x, int m, const int32_t* sel, const float* w, int k, float* out, int mode)
{
    NEED_INIT("mm_tier_forward");
    return tier::impl_forward(li, x, m, sel, w, k, out, mode);
}

int mm_tier_stats(int64_t* out)
{
    if (!out) return mm::set_error(MM_ERR_ARG, "mm_tier_stats: null pointer");
    if (!g_ok)
    {
        for (int i = 0; i < MM_TIER_NSTATS; ++i) out[i] = 0;
        return MM_OK;
    }
    return tier::impl_stats(out);
}

}  // extern "C"
