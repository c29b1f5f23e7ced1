// One decode MoE layer for callers that cannot allocate (code under HIP graph capture, tight serving loops,
// harnesses that forbid hipMalloc): mm_moe_decode's launches on a workspace that lives in a file-scope device
// array instead of caller-provided memory.
//
// The array is `scratch` below (MM_NOALLOC_SCRATCH_BYTES). In host code its name is only a stand-in for the
// device variable, so the entry point never passes it to a kernel or a copy: on the first call on a device (with
// that device current) it asks the runtime for the device's own address of the array with hipGetSymbolAddress
// and keeps it per device; every launch then gets that address. Each device that loads the library holds its own
// copy of the array until the process ends. That first call must therefore run outside graph capture; the
// calls after it only launch kernels and can be captured. Every call on one device shares that device's array, which keeps
// the previous call's contents: mm_moe_decode's launches write every workspace location before they read it,
// so nothing needs clearing, but calls that overlap on one device (two streams, two threads) race.
#include <mutex>

#include "mm_decode.h"

namespace mm {

constexpr size_t NOALLOC_BYTES = MM_NOALLOC_SCRATCH_BYTES;
constexpr int NOALLOC_MAX_DEVICES = 64;

static __device__ __align__(256) unsigned char scratch[NOALLOC_BYTES];

static std::mutex g_noalloc_mu;
static void* g_noalloc_ptr[NOALLOC_MAX_DEVICES] = {};

// The current device's address of `scratch`, looked up once per device.
static int noalloc_scratch(void** out)
{
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return set_error(MM_ERR_HIP, "mm_moe_decode_noalloc: hipGetDevice: %s", hipGetErrorString(e));
    if (dev < 0 || dev >= NOALLOC_MAX_DEVICES)
        return set_error(MM_ERR_UNSUP, "mm_moe_decode_noalloc: device %d beyond the %d supported", dev,
                         NOALLOC_MAX_DEVICES);
    std::lock_guard<std::mutex> lock(g_noalloc_mu);
    if (!g_noalloc_ptr[dev])
    {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p)
            return set_error(MM_ERR_HIP, "mm_moe_decode_noalloc: hipGetSymbolAddress(scratch) on device %d: %s", dev,
                             hipGetErrorString(e));
        g_noalloc_ptr[dev] = p;
    }
    *out = g_noalloc_ptr[dev];
    return MM_OK;
}

}  // namespace mm

using namespace mm;

extern "C" {

int mm_moe_decode_noalloc(const mm_layer_t* L, const void* x, int x_dtype, int rescale, int T, int topk,
                          const int64_t* ids, const float* w, int max_rows, float* out, mm_stream_t stream)
{
    MM_CHECK_ARG(L && T > 0 && topk > 0, "mm_moe_decode_noalloc: need a layer, T > 0 and topk > 0");
    MM_CHECK_ARG((size_t)T * topk < ((size_t)1 << 30), "mm_moe_decode_noalloc: too many routes");
    const size_t need = mm_gemv_workspace(T * topk, L->E, L->H, L->I);
    MM_CHECK_ARG(need <= NOALLOC_BYTES,
                 "mm_moe_decode_noalloc: %d routes at E=%d H=%d I=%d need %zu bytes of workspace, more than the %zu "
                 "bytes of the library's device scratch (use mm_moe_decode with a workspace)",
                 T * topk, L->E, L->H, L->I, need, NOALLOC_BYTES);
    void* ws = nullptr;
    const int rc = noalloc_scratch(&ws);
    if (rc) return rc;
    return moe_decode_launch(L, x, x_dtype, rescale, T, topk, ids, w, max_rows, out, ws, NOALLOC_BYTES, stream,
                             "mm_moe_decode_noalloc");
}

}  // extern "C"
