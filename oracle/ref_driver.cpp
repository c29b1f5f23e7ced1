// C-ABI driver around the reference's own CPU expert kernel (kernels/cpu_avx2/ft_core.h), compiled from
// the reference checkout in place by oracle/Makefile into oracle/_ref/libftref.so. TEST INFRASTRUCTURE:
// used to write golden vectors that pin the oracle, and as the timed CPU baseline. Nothing of the
// reference is copied here; the header is included from where it lies.
#include "ft_core.h"

#include <vector>

namespace {

struct RefState
{
    Pool pool;
    bool started = false;
    std::vector<Layer> layers;
};

RefState* g_ref = nullptr;

RefState& st()
{
    if (!g_ref) { init_perm(); init_tables(); g_ref = new RefState(); }
    return *g_ref;
}

}  // namespace

extern "C" {

// Dense K x N weights of one matrix (ft_core.h:977-992).
__attribute__((visibility("default"))) void ref_dense(const uint8_t* tr, int k, int n, float* W)
{
    st();
    Mat m{ tr, nullptr, nullptr, k, n };
    std::vector<float> d = dense_weights(m);
    std::memcpy(W, d.data(), d.size() * sizeof(float));
}

// Double-accumulation expert (ft_core.h:1004-1011); I must be 2048 (the reference fixes it there).
__attribute__((visibility("default"))) void ref_expert_fwd(const uint8_t* tg, const uint8_t* tu, const uint8_t* td,
    const uint16_t* suh_g, const uint16_t* svh_g, const uint16_t* suh_u, const uint16_t* svh_u, const uint16_t* suh_d,
    const uint16_t* svh_d, int H, int I, float limit, const float* x, float* y)
{
    st();
    g_act_limit = limit;
    Expert E;
    E.g = { tg, suh_g, svh_g, H, I };
    E.u = { tu, suh_u, svh_u, H, I };
    E.d = { td, suh_d, svh_d, I, H };
    std::vector<float> W[3] = { dense_weights(E.g), dense_weights(E.u), dense_weights(E.d) };
    ref_expert(E, W, x, y);
}

// Start the reference's pinned spinning pool (ft_core.h:421-465) on the given CPUs.
__attribute__((visibility("default"))) void ref_pool_start(int threads, const int* cpus, int ncpus)
{
    RefState& s = st();
    if (s.started) return;
    std::vector<int> c(cpus, cpus + ncpus);
    cpu_set_t saved;
    sched_getaffinity(0, sizeof(saved), &saved);
    s.pool.start(threads, c);
    sched_setaffinity(0, sizeof(saved), &saved);
    s.started = true;
}

__attribute__((visibility("default"))) void ref_set_limit(float limit) { st(); g_act_limit = limit; }

// Register a layer: per expert e, trellis pointers ptrs[e*3 + {0,1,2}] (native tile layout) and fp16
// scales [E][H] / [E][I] (same layout as ft_tier_ext.cpp:56-73).
__attribute__((visibility("default"))) void ref_add_layer(int li, int E, int H, int I, const int64_t* ptrs,
    const uint16_t* suh_g, const uint16_t* svh_g, const uint16_t* suh_u, const uint16_t* svh_u,
    const uint16_t* suh_d, const uint16_t* svh_d)
{
    RefState& s = st();
    if ((int)s.layers.size() <= li) s.layers.resize(li + 1);
    Layer& L = s.layers[li];
    L.H = H; L.I = I; L.ex.resize(E);
    for (int e = 0; e < E; ++e)
    {
        L.ex[e].g = { reinterpret_cast<const uint8_t*>(ptrs[e * 3 + 0]), suh_g + size_t(e) * H, svh_g + size_t(e) * I, H, I };
        L.ex[e].u = { reinterpret_cast<const uint8_t*>(ptrs[e * 3 + 1]), suh_u + size_t(e) * H, svh_u + size_t(e) * I, H, I };
        L.ex[e].d = { reinterpret_cast<const uint8_t*>(ptrs[e * 3 + 2]), suh_d + size_t(e) * I, svh_d + size_t(e) * H, I, H };
    }
}

// The CPU tier's MoE forward (ft_core.h:703-727): x fp32 [ntok][H] (fp16 values), routes as flat
// (token, expert, weight) triples, out fp32 [ntok][H]. mode: 0 AFFINE, 1 EXACT, 2 I16, -1 auto
// (ft_tier_ext.cpp:130-132).
__attribute__((visibility("default"))) int ref_moe_forward(int li, const float* x, int ntok, const int* tok,
    const int* exp, const float* w, int npicks, float* out, int mode)
{
    RefState& s = st();
    if (!s.started || li >= (int)s.layers.size()) return -1;
    std::vector<std::vector<std::pair<int, float>>> route(ntok);
    for (int i = 0; i < npicks; ++i) route[tok[i]].push_back({ exp[i], w[i] });
    int maxm = 0;
    {
        std::vector<int> cnt(s.layers[li].ex.size(), 0);
        for (auto& r : route) for (auto& pr : r) maxm = std::max(maxm, ++cnt[pr.first]);
    }
    const int md = mode >= 0 ? mode : (maxm <= 2 ? 2 : 0);
    moe_forward(s.pool, s.layers[li], x, ntok, route, out, md);
    return md;
}

}  // extern "C"
