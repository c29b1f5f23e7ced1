// Expert placement: stream-ordered slot-table repoints and host -> HBM staging copies.
//
// Every kernel reads an expert's trellis through the layer's pointer tables (gate / up / down address per
// expert), so moving an expert between its home copy, a cache slot and a staging slot is a write of three table
// entries plus its slot number (the reference's _ec_point, ct/ct_vllm.py:268-279, which index_copy_'s them on the
// compute stream). The copies themselves go to the copy engines (hipMemcpyAsync on the caller's stream), the
// reference's copy_(non_blocking=True) of pinned host rows (ct/ct_vllm.py:399-405,416-421;
// patches/vllm-exl3-host-dma.patch:100-124).
#include "mm_common.h"

namespace mm {

// items [n][5] = (e, gate, up, down, slot). Item i is applied unless a later item names the same expert, so the
// last item of an expert wins whatever the thread order.
__global__ __launch_bounds__(256) void k_slot_point(int64_t* __restrict__ gp, int64_t* __restrict__ up,
                                                    int64_t* __restrict__ dp, int32_t* __restrict__ slotof, int E,
                                                    const int64_t* __restrict__ items, int n)
{
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const int64_t* it = items + (size_t)i * 5;
    const int64_t e = it[0];
    if (e < 0 || e >= E) return;
    for (int j = i + 1; j < n; ++j)
        if (items[(size_t)j * 5] == e) return;
    gp[e] = it[1];
    up[e] = it[2];
    dp[e] = it[3];
    if (slotof) slotof[e] = (int32_t)it[4];
}

// HBM read calibration: each thread streams 16-byte vectors (four in flight) over a grid-stride range; the xor of
// every word read is folded per workgroup and xor-ed into one word.
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(256) void k_read_probe(const u32x4* __restrict__ src, uint64_t n16, uint32_t* sink)
{
    const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    u32x4 acc = { 0u, 0u, 0u, 0u };
    for (; i + 3 * stride < n16; i += 4 * stride)
    {
        const u32x4 a = __builtin_nontemporal_load(src + i);
        const u32x4 b = __builtin_nontemporal_load(src + i + stride);
        const u32x4 c = __builtin_nontemporal_load(src + i + 2 * stride);
        const u32x4 d = __builtin_nontemporal_load(src + i + 3 * stride);
        acc ^= a ^ b ^ c ^ d;
    }
    for (; i < n16; i += stride) acc ^= __builtin_nontemporal_load(src + i);
    __shared__ uint32_t red[256];
    red[threadIdx.x] = acc.x ^ acc.y ^ acc.z ^ acc.w;
    __syncthreads();
    for (int s = 128; s > 0; s >>= 1)
    {
        if (threadIdx.x < s) red[threadIdx.x] ^= red[threadIdx.x + s];
        __syncthreads();
    }
    if (threadIdx.x == 0) atomicXor(sink, red[0]);
}

}  // namespace mm

using namespace mm;

extern "C" {

int mm_slot_point(int64_t* gate_ptr, int64_t* up_ptr, int64_t* down_ptr, int32_t* slotof, int E, const int64_t* items,
                  int n, mm_stream_t stream)
{
    MM_CHECK_ARG(E > 0 && n >= 0, "mm_slot_point: need E > 0 and n >= 0 (E=%d, n=%d)", E, n);
    MM_CHECK_ARG(gate_ptr && up_ptr && down_ptr && (n == 0 || items), "mm_slot_point: null pointer");
    MM_CHECK_ARG(n <= (1 << 16), "mm_slot_point: at most 65536 items per call (n=%d)", n);
    if (n == 0) return MM_OK;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    hipLaunchKernelGGL(k_slot_point, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, gate_ptr, up_ptr, down_ptr,
                       slotof, E, items, n);
    return check_launch("mm_slot_point");
}

int mm_read_probe(const void* src, uint64_t bytes, uint32_t* sink, int blocks, mm_stream_t stream)
{
    MM_CHECK_ARG(src && sink && bytes % 16 == 0 && ((uintptr_t)src & 15) == 0,
                 "mm_read_probe: need device src (16-byte aligned, bytes a multiple of 16) and sink");
    MM_CHECK_ARG(blocks >= 0 && blocks <= (1 << 20), "mm_read_probe: blocks must be in [0, 2^20]");
    if (bytes == 0) return MM_OK;
    if (blocks == 0)
    {
        int dev = 0, cus = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
            cus = 256;
        blocks = 8 * cus;
    }
    hipLaunchKernelGGL(k_read_probe, dim3((unsigned)blocks), dim3(256), 0, reinterpret_cast<hipStream_t>(stream),
                       reinterpret_cast<const u32x4*>(src), bytes / 16, sink);
    return check_launch("mm_read_probe");
}

int mm_stage_copy(const uint64_t* dst, const uint64_t* src, const uint64_t* bytes, int n, mm_stream_t stream)
{
    MM_CHECK_ARG(n >= 0 && (n == 0 || (dst && src && bytes)), "mm_stage_copy: bad argument");
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    int issued = 0;
    int i = 0;
    while (i < n)
    {
        MM_CHECK_ARG(bytes[i] == 0 || (dst[i] && src[i]), "mm_stage_copy: null address in copy %d", i);
        uint64_t d = dst[i], sr = src[i], b = bytes[i];
        int j = i + 1;
        // merge the following copies that continue both the destination and the source range
        while (j < n && bytes[j] && dst[j] == d + b && src[j] == sr + b)
        {
            b += bytes[j];
            ++j;
        }
        if (b)
        {
            const hipError_t e = hipMemcpyAsync(reinterpret_cast<void*>((uintptr_t)d),
                                                reinterpret_cast<const void*>((uintptr_t)sr), (size_t)b,
                                                hipMemcpyDefault, s);
            if (e != hipSuccess)
                return set_error(MM_ERR_HIP, "mm_stage_copy: hipMemcpyAsync(%llu bytes): %s", (unsigned long long)b,
                                 hipGetErrorString(e));
            ++issued;
        }
        i = j;
    }
    return issued;
}

}  // extern "C"
