// Expert placement: stream-ordered slot-table repoints and host -> HBM staging copies.
//
// Every kernel reads an expert's trellis through the layer's pointer tables (gate / up / down address per
// expert), so moving an expert between its home copy, a cache slot and a staging slot is a write of three table
// entries plus its slot number (the reference's _ec_point, ct/ct_vllm.py:268-279, which index_copy_'s them on the
// compute stream). The copies themselves go to the copy engines (hipMemcpyAsync on the caller's stream), the
// reference's copy_(non_blocking=True) of pinned host rows (ct/ct_vllm.py:399-405,416-421;
// patches/vllm-exl3-host-dma.patch:100-124).
#include <chrono>
#include <mutex>
#include <thread>
#include <utility>
#include <vector>

#include "mm_common.h"

namespace mm {

// Copy streams. HIP maps streams onto a pool of GPU_MAX_HW_QUEUES hardware queues (4 by default), each new
// stream taking the least used queue, so a side stream can land on the compute stream's queue; its transfers then
// wait for the compute kernels queued before them, and a staged prefill runs its copies and its GEMMs one after
// the other instead of side by side. (Which queue a stream gets depends on every stream the process made before:
// torch hands out its pool streams round robin.) The library therefore keeps its own non-blocking streams and
// checks, once per (device, compute stream), that a candidate runs while the compute stream is held: k_hold
// occupies the compute stream until the host releases it, and a candidate whose empty kernel completes meanwhile
// is on another queue. Candidates that fail are kept for other compute streams; new ones are made up to
// COPY_MAX_CANDIDATES per device.
constexpr int COPY_MAX_DEVICES = 64;
constexpr int COPY_MAX_CANDIDATES = 8;
constexpr int COPY_POLL_MS = 50;           // how long the host waits for a candidate's kernel
constexpr int COPY_HOLD_MS = 500;          // k_hold's own limit, far beyond the poll: the kernel always ends

struct CopyChoice
{
    hipStream_t compute;
    int index;
    hipStream_t stream;
    bool verified;
};

struct CopyDevice
{
    std::vector<hipStream_t> cands;
    std::vector<std::pair<hipStream_t, hipStream_t>> tested_ok, tested_bad;   // (compute, candidate)
    std::vector<CopyChoice> chosen;
    int* flag = nullptr;                   // host memory the hold kernel polls
    hipEvent_t ev = nullptr;
};

static std::mutex g_copy_mu;
static CopyDevice g_copy[COPY_MAX_DEVICES];

// One lane keeps the stream busy until *flag turns nonzero or max_ticks of the constant-rate wall clock have
// passed, whichever comes first.
__global__ __launch_bounds__(64) void k_hold(const int* flag, uint64_t max_ticks)
{
    if (threadIdx.x != 0) return;
    const uint64_t t0 = wall_clock64();
    while (__hip_atomic_load(flag, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_SYSTEM) == 0 &&
           wall_clock64() - t0 < max_ticks)
        __builtin_amdgcn_s_sleep(8);
}

__global__ __launch_bounds__(64) void k_nop() {}

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

namespace mm {

// Whether `cand` runs while `compute` is held. The device is current; both streams are idle on return.
static int copy_independent(CopyDevice& D, int device, hipStream_t compute, hipStream_t cand, bool* ok)
{
    int khz = 0;
    if (hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, device) != hipSuccess || khz <= 0) khz = 100000;
    hipError_t e = hipStreamSynchronize(compute);          // an idle device, so the candidate finds a free CU
    if (e == hipSuccess) e = hipStreamSynchronize(cand);
    if (e != hipSuccess) return set_error(MM_ERR_HIP, "mm_copy_stream: stream synchronize: %s", hipGetErrorString(e));
    __atomic_store_n(D.flag, 0, __ATOMIC_RELEASE);
    hipLaunchKernelGGL(k_hold, dim3(1), dim3(64), 0, compute, D.flag, (uint64_t)khz * COPY_HOLD_MS);
    e = hipGetLastError();
    if (e != hipSuccess)
    {
        __atomic_store_n(D.flag, 1, __ATOMIC_RELEASE);
        return set_error(MM_ERR_HIP, "mm_copy_stream: hold launch: %s", hipGetErrorString(e));
    }
    hipLaunchKernelGGL(k_nop, dim3(1), dim3(64), 0, cand);
    e = hipGetLastError();
    if (e == hipSuccess) e = hipEventRecord(D.ev, cand);
    bool done = false;
    if (e == hipSuccess)
    {
        const auto t0 = std::chrono::steady_clock::now();
        while (!done)
        {
            const hipError_t q = hipEventQuery(D.ev);
            if (q == hipSuccess) done = true;
            else if (q != hipErrorNotReady) { e = q; break; }
            else if (std::chrono::steady_clock::now() - t0 > std::chrono::milliseconds(COPY_POLL_MS)) break;
            else std::this_thread::sleep_for(std::chrono::microseconds(50));
        }
    }
    __atomic_store_n(D.flag, 1, __ATOMIC_RELEASE);        // release the hold on every path
    const hipError_t e2 = hipStreamSynchronize(compute);
    const hipError_t e3 = hipStreamSynchronize(cand);
    if (e == hipSuccess) e = e2 != hipSuccess ? e2 : e3;
    if (e != hipSuccess) return set_error(MM_ERR_HIP, "mm_copy_stream: queue check: %s", hipGetErrorString(e));
    *ok = done;
    return MM_OK;
}

static int copy_choose(CopyDevice& D, int device, int index, hipStream_t compute, hipStream_t* out, bool* verified)
{
    for (const CopyChoice& c : D.chosen)
        if (c.compute == compute && c.index == index)
        {
            *out = c.stream;
            *verified = c.verified;
            return MM_OK;
        }
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    hipError_t e = hipStreamIsCapturing(compute, &cap);
    if (e != hipSuccess) return set_error(MM_ERR_HIP, "mm_copy_stream: hipStreamIsCapturing: %s", hipGetErrorString(e));
    MM_CHECK_ARG(cap == hipStreamCaptureStatusNone, "mm_copy_stream: the compute stream is capturing a graph");
    if (compute)
    {
        hipDevice_t sd = -1;
        e = hipStreamGetDevice(compute, &sd);
        if (e != hipSuccess) return set_error(MM_ERR_HIP, "mm_copy_stream: hipStreamGetDevice: %s", hipGetErrorString(e));
        MM_CHECK_ARG(sd == device, "mm_copy_stream: the compute stream belongs to device %d, not %d", (int)sd, device);
    }
    if (!D.flag)
    {
        e = hipHostMalloc((void**)&D.flag, 64, hipHostMallocMapped | hipHostMallocPortable | hipHostMallocCoherent);
        if (e != hipSuccess) { D.flag = nullptr; return set_error(MM_ERR_HIP, "mm_copy_stream: flag: %s", hipGetErrorString(e)); }
        e = hipEventCreateWithFlags(&D.ev, hipEventDisableTiming);
        if (e != hipSuccess) { D.ev = nullptr; return set_error(MM_ERR_HIP, "mm_copy_stream: event: %s", hipGetErrorString(e)); }
    }
    auto taken = [&](hipStream_t s) {                        // already the copy stream of another index here
        for (const CopyChoice& c : D.chosen)
            if (c.compute == compute && c.stream == s) return true;
        return false;
    };
    auto known = [&](const std::vector<std::pair<hipStream_t, hipStream_t>>& v, hipStream_t s) {
        for (const auto& p : v)
            if (p.first == compute && p.second == s) return true;
        return false;
    };
    hipStream_t pick = nullptr, fallback = nullptr;
    // pass 0: streams no other index uses for this compute stream, new ones made as needed; pass 1: any
    for (int pass = 0; pass < 2 && !pick; ++pass)
        for (size_t i = 0; i <= D.cands.size() && !pick; ++i)
        {
            if (i == D.cands.size())
            {
                if (pass == 1 || (int)D.cands.size() >= COPY_MAX_CANDIDATES) break;
                hipStream_t s = nullptr;
                e = hipStreamCreateWithFlags(&s, hipStreamNonBlocking);
                if (e != hipSuccess) return set_error(MM_ERR_HIP, "mm_copy_stream: stream: %s", hipGetErrorString(e));
                D.cands.push_back(s);
            }
            hipStream_t s = D.cands[i];
            if (s == compute || (pass == 0 && taken(s)) || known(D.tested_bad, s)) continue;
            if (!fallback) fallback = s;
            bool ok = known(D.tested_ok, s);
            if (!ok)
            {
                const int rc = copy_independent(D, device, compute, s, &ok);
                if (rc != MM_OK) return rc;
                (ok ? D.tested_ok : D.tested_bad).push_back({compute, s});
            }
            if (ok) pick = s;
        }
    if (!pick && !fallback)
    {
        for (hipStream_t s : D.cands)
            if (s != compute) { fallback = s; break; }
        if (!fallback) return set_error(MM_ERR_HIP, "mm_copy_stream: no candidate stream on device %d", device);
    }
    D.chosen.push_back({compute, index, pick ? pick : fallback, pick != nullptr});
    *out = pick ? pick : fallback;
    *verified = pick != nullptr;
    return MM_OK;
}

}  // namespace mm

extern "C" {

int mm_copy_stream(int device, int index, mm_stream_t compute, mm_stream_t* out)
{
    MM_CHECK_ARG(out, "mm_copy_stream: null output");
    MM_CHECK_ARG(index >= 0 && index < MM_COPY_STREAMS, "mm_copy_stream: index %d outside [0, %d)", index,
                 MM_COPY_STREAMS);
    int ndev = 0;
    hipError_t e = hipGetDeviceCount(&ndev);
    if (e != hipSuccess) return set_error(MM_ERR_HIP, "mm_copy_stream: hipGetDeviceCount: %s", hipGetErrorString(e));
    MM_CHECK_ARG(device >= 0 && device < ndev && device < COPY_MAX_DEVICES,
                 "mm_copy_stream: device %d outside [0, %d)", device, ndev < COPY_MAX_DEVICES ? ndev : COPY_MAX_DEVICES);
    int cur = 0;
    e = hipGetDevice(&cur);
    if (e != hipSuccess) return set_error(MM_ERR_HIP, "mm_copy_stream: hipGetDevice: %s", hipGetErrorString(e));
    if (cur != device && (e = hipSetDevice(device)) != hipSuccess)
        return set_error(MM_ERR_HIP, "mm_copy_stream: hipSetDevice(%d): %s", device, hipGetErrorString(e));
    hipStream_t s = nullptr;
    bool verified = false;
    int rc;
    {
        std::lock_guard<std::mutex> lock(g_copy_mu);
        rc = copy_choose(g_copy[device], device, index, reinterpret_cast<hipStream_t>(compute), &s, &verified);
    }
    if (cur != device) (void)hipSetDevice(cur);
    if (rc != MM_OK) return rc;
    *out = reinterpret_cast<mm_stream_t>(s);
    return verified ? MM_OK : MM_COPY_UNVERIFIED;
}

}  // extern "C"
