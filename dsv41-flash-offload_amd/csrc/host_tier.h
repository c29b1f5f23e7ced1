// The host expert tier's implementation (host_tier.cpp, compiled for AVX-512) as the C ABI's wrappers
// (host_tier_abi.cpp, compiled for the baseline x86-64 target) call it, after checking the CPU.
#pragma once
#include <stdint.h>

#include "../../include/mi355moe.h"

namespace mm {
int set_error(int code, const char* fmt, ...);
}

namespace tier {
int impl_init(int threads, const int* cpus, int ncpus, int64_t* ctrl, const void* hx, const int32_t* picks,
              float* hout, int maxtok, int maxpicks, int mode, int H, int I, int nlayers);
int impl_add_layer(int li, int E, const int64_t* ptrs, const void* suh_g, const void* svh_g, const void* suh_u,
                   const void* svh_u, const void* suh_d, const void* svh_d);
int impl_set_limit(float limit);
int impl_set_mode(int mode);
int impl_start(int cpu0);
int impl_stop();
int impl_shutdown();
int impl_forward(int li, const float* x, int m, const int32_t* sel, const float* w, int k, float* out, int mode);
int impl_stats(int64_t* out);
// Sanitizer drivers only (not part of the C ABI): fn(arg, stage, seq) runs on the serving thread after a job's
// copy, before its sequence is checked again (stage 0), and after its partial is written, before the answer
// (stage 1). Set while the worker is stopped.
int impl_set_test_hook(void (*fn)(void*, int, int64_t), void* arg);
}  // namespace tier
