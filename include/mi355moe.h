/*
 * mi355moe -- C ABI of the MI355X-native routed-expert MoE layer.
 *
 * Conventions for every entry point:
 *   - All pointers are caller-owned: device memory, or host memory allocated with mm_host_alloc (mapped,
 *     coherent) where a parameter says "host-mapped". The library allocates nothing per call.
 *   - `stream` is a hipStream_t (0 = the null stream). Work is enqueued on it; no entry point synchronises
 *     the host, so every call can be captured into a HIP graph (except mm_copy_stream, a set-up call whose first
 *     call for a compute stream synchronises it).
 *   - Return 0 on success or a negative MM_ERR_* code; mm_last_error() gives a thread-local message.
 *   - Calls on distinct streams with distinct buffers are independent; calls sharing a workspace race.
 *
 * Trellis layout (EXL3 3 bpw, identical to the reference's storage): a K x N matrix is tiles
 * [K/16][N/16] of 48 uint16 words (96 bytes); gate/up are K=H, N=I; down is K=I, N=H.
 * Scales (fp16): suh13 [E][2][H], svh13 [E][2][I], suh2 [E][I], svh2 [E][H] (reference parameter shapes,
 * patches/vllm-exl3-host-dma.patch:660-690).
 */
#ifndef MI355MOE_H
#define MI355MOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MM_OK 0
#define MM_ERR_ARG (-1)      /* invalid argument (shape, size, null pointer) */
#define MM_ERR_HIP (-2)      /* HIP runtime error (launch, copy, allocation of host memory) */
#define MM_ERR_UNSUP (-3)    /* unsupported configuration (e.g. codebook other than mul1) */

typedef void* mm_stream_t;

/* Element types of a layer input x [T][H]. */
#define MM_DTYPE_F16 0
#define MM_DTYPE_BF16 1
#define MM_DTYPE_F32 2

/* Library version (major*10000 + minor*100 + patch). */
int mm_version(void);

/* Thread-local message of the last failing call on this thread ("" if none). */
const char* mm_last_error(void);

/* Pinned, device-mapped, coherent host memory for the host mailbox and host-resident expert copies
 * (replaces the reference's torch pin_memory() mailbox, ct/ct_vllm.py:62-65, and the cudaHostRegister'd
 * home store, patches/vllm-exl3-host-dma.patch:609-617). */
int mm_host_alloc(void** ptr, size_t bytes);
int mm_host_free(void* ptr);

/* ----------------------------------------------------------------------------------------- routing */

/* Router top-k (vLLM FusedMoE semantics at the boundary patches/vllm-exl3-host-dma.patch:496-507):
 * logits[t][e] = sum_h x[t][h] * gate[e][h] (x bf16 [T][H], gate fp32 [E][H], fp32 sums);
 * ids[t][:k] = the k largest logits (ties -> lower expert id), w[t][:k] = softmax over those k logits.
 * logits fp32 [T][E] is written too (it is the kernels' workspace: required). Requires E <= 1024, k <= 32.
 * Up to 64 tokens (H a multiple of 256) one wave per expert sums lane partials; larger calls (H a multiple of 32)
 * run on bf16 MFMA with the fp32 gate split exactly into three bf16 parts, so every product is exact in fp32 and
 * the fp32 accumulation (in the matrix cores' order) is the only rounding; other shapes sum each logit in
 * ascending h. The last bits of a logit may differ between the paths. */
int mm_router_topk(const void* x_bf16, int T, int H, const float* gate, int E, int k, float* logits, int64_t* ids,
                   float* w, mm_stream_t stream);

/* Decode-tier split; replaces ft_split (ct/ft_tier_cu_v.cu:129-143), same buffers and semantics:
 * sel int64 [n], w fp32 [n], z fp16 [bsz][H] (n = bsz * topk), slotof int32 [E], score fp32 [E], pol fp32 [9];
 * ctrl int64 [16], hx fp16 [bsz*H] and hpicks int32 [n*3] are host-mapped; seqc, dflag int64 [1] and
 * stats int64 [8] are device counters; counts int32 [E] (may be NULL) accumulates routed counts.
 * Outputs sel_out int64 [n], w_out fp32 [n]. Extra optional outputs (NULL to skip): hits int32 [E] (resident
 * touched experts, ascending id), misses int32 [E] (non-resident, stable by score), nhnm int32 [2].
 * Requires E <= 1024, H % 8 == 0. Scores must not be NaN. */
int mm_split(const int64_t* sel, const float* w, const void* z_fp16, int n, int bsz, int H, int E, const int32_t* slotof,
             const float* score, const float* pol, int64_t* ctrl, void* hx, int32_t* hpicks, int64_t* seqc, int li,
             int64_t* sel_out, float* w_out, int64_t* dflag, int64_t* stats, int32_t* counts, int32_t* hits,
             int32_t* misses, int32_t* nhnm, mm_stream_t stream);

/* Host-partial add; replaces ft_combine (ct/ft_tier_cu_v.cu:145-153): if dflag[0] != 0, wait (bounded by
 * timeout_ns, measured on the GPU's constant-rate clock) until host-mapped ctrl[1] >= dflag[0], then
 * out[i] += hout[i] for i < n (hout host-mapped fp32, written by the host worker). On timeout the whole partial
 * is dropped, dflag[0] is cleared and stats[6]++; stats[4] += wait ns, stats[5]++ as in the reference. One wait
 * decides for the whole output (the reference's workgroups each wait and decide on their own). */
int mm_combine_host(float* out, int n, int64_t* dflag, const int64_t* ctrl, const float* hout, int64_t* stats,
                    int64_t timeout_ns, mm_stream_t stream);

/* Bytes of device workspace mm_permute needs for n routes over E experts. */
size_t mm_permute_workspace(int n, int E);

/* Routing prep (patches/vllm-exl3-host-dma.patch:204-236,296-312), made deterministic: ids int64 [n]
 * (ids outside [0, E) go to the sentinel bin E); counts int32 [E+1]; offsets int32 [E+2] (exclusive sums,
 * offsets[E+1] = n); order int32 [n] = flat route index at each sorted position, stable by (expert, index);
 * token_sorted int32 [n] = order / topk; weight_sorted fp32 [n] = w[order] (NULL w or NULL output skips it);
 * inv_order int32 [n] (may be NULL) = sorted position of each flat index; active int32 [E] (may be NULL) =
 * experts with count > 0 in ascending id and nactive int32 [1] their number. */
int mm_permute(const int64_t* ids, const float* w, int n, int topk, int E, int32_t* counts, int32_t* offsets,
               int32_t* order, int32_t* token_sorted, float* weight_sorted, int32_t* inv_order, int32_t* active,
               int32_t* nactive, void* workspace, size_t workspace_bytes, mm_stream_t stream);

/* Weighted combine of per-route expert outputs in a fixed order (replaces the fused kernel's atomic
 * accumulation, patches/vllm-exl3-host-dma.patch:327-342): for every token t and column h,
 * out[t][h] = (accumulate ? out[t][h] : 0) + sum_{j<k, 0<=ids[t*k+j]<E} w[t*k+j] * Y[t*k+j][h], fp32 fma in
 * ascending j. Y fp32 [T*k][H] in flat route order. */
int mm_combine(float* out, const float* Y, const int64_t* ids, const float* w, int T, int k, int H, int E,
               int accumulate, mm_stream_t stream);

/* ------------------------------------------------------------------------------------ expert layer */

/* Device-side description of one MoE layer's experts (the reference's per-layer pointer tables
 * layer._exl3_ptrs["gate_trellis"/"up_trellis"/"down_trellis"], patches/vllm-exl3-host-dma.patch:727-751,
 * and its stacked scale parameters). Every pointer is a device address. */
typedef struct mm_layer
{
    const int64_t* gate_ptr;    /* [E] address of expert e's gate trellis [H/16][I/16][48] */
    const int64_t* up_ptr;      /* [E] address of expert e's up trellis   [H/16][I/16][48] */
    const int64_t* down_ptr;    /* [E] address of expert e's down trellis [I/16][H/16][48] */
    const uint16_t* suh13;      /* fp16 [E][2][H] */
    const uint16_t* svh13;      /* fp16 [E][2][I] */
    const uint16_t* suh2;       /* fp16 [E][I] */
    const uint16_t* svh2;       /* fp16 [E][H] */
    int E, H, I;
    float limit;                /* SwiGLU clamp (0 = off); reference default 10 */
    int flags;                  /* MM_LAYER_* bits */
} mm_layer_t;

/* mm_layer_t.flags. Without MM_LAYER_EXACT the decode path evaluates the codebook as the reference's AFFINE
 * expert does (kernels/cpu_avx2/ft_core.h:267-293): unrounded w = KINV * (1024 + bytesum) + KBIAS, applied once
 * per output through the input sum (sum_k x_k w_k = KINV * sum_k x_k (1024 + s_k) + KBIAS * sum_k x_k). With it,
 * every weight is rounded to fp16 first, as the reference's EXACT expert and the exllamav3 kernel do
 * (ft_core.h:75-83); that costs two more VALU operations per 16x16 tile. */
#define MM_LAYER_EXACT 1

/* Bytes of device workspace mm_expert_gemv / mm_moe_decode need for n routes over E experts (per-expert
 * records, sorted positions, transformed inputs, K-part partial sums). */
size_t mm_gemv_workspace(int n, int E, int H, int I);

/* Decode expert path (replaces exllamav3 exl3_moe on the decode split, patches/vllm-exl3-host-dma.patch:323-445):
 * for every route s < n with 0 <= ids[s] < E (token s / topk), computes the expert SwiGLU MLP with fused EXL3
 * trellis decode and writes Y fp32 [n][H] row s (rows of other routes are left untouched).
 * The expert input of token t is x[t] (x_dtype MM_DTYPE_*) converted to fp16: fp16 input is used as is, other
 * types go through bf16 (RNE); with rescale != 0 the row is first scaled to unit RMS (any type), as
 * mm_prepare_input does. Routes are found in-kernel from ids when offsets is NULL (n <= 1024); otherwise
 * offsets/order/active/nactive from mm_permute over the same routes are used. max_rows (>= 1) is the fat-expert
 * threshold of the call: an expert with more than max_rows routes is left to the fat-expert path (its rows stay
 * untouched here), so a caller can split a call between both paths without reading the counts on the host;
 * max_rows >= n computes every route. Any number of routes per expert is supported (the trellis is streamed once
 * per 16 routes of an expert). phases is a mask of the five launches, run in this order on the same workspace:
 * 1 = route prep and input transform, 2 = gate/up partial sums, 4 = gate/up epilogue (output transforms, SwiGLU,
 * down-input transform), 8 = down partial sums, 16 = down epilogue into Y; 31 = the whole expert MLP. */
int mm_expert_gemv(const mm_layer_t* layer, const void* x, int x_dtype, int rescale, int T, int n, int topk,
                   const int64_t* ids, const int32_t* offsets, const int32_t* order, const int32_t* active,
                   const int32_t* nactive, int max_rows, float* Y, void* workspace, size_t workspace_bytes, int phases,
                   mm_stream_t stream);

/* One decode MoE layer (the fused-MoE call of the decode split, patches/vllm-exl3-host-dma.patch:315-449, with the
 * weighted combine of patches/vllm-exl3-host-dma.patch:327-342 made deterministic): routes ids int64 [T*topk]
 * with weights w fp32 [T*topk] (topk <= 16, T*topk <= 1024; ids outside [0, E) contribute nothing) ->
 * out fp32 [T][H] = sum_j w[t,j] * expert_{ids[t,j]}(x_t), summed in ascending j with fp32 fma (equal to
 * mm_combine over mm_expert_gemv's rows). x, x_dtype and rescale as for mm_expert_gemv: a chain of layers
 * passes the previous layer's out with MM_DTYPE_F32. max_rows as for mm_expert_gemv: routes of experts with more
 * than max_rows routes contribute nothing (mm_moe_prefill with cap = max_rows and accumulate = 1 adds them). */
int mm_moe_decode(const mm_layer_t* layer, const void* x, int x_dtype, int rescale, int T, int topk,
                  const int64_t* ids, const float* w, int max_rows, float* out, void* workspace, size_t workspace_bytes,
                  mm_stream_t stream);

/* Bytes of the library's device scratch array behind mm_moe_decode_noalloc (one array per device, held from the
 * library's load until the process ends). */
#define MM_NOALLOC_SCRATCH_BYTES ((size_t)64 << 20)

/* mm_moe_decode without a workspace argument. No counterpart in the reference: it is for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * Same arguments, kernels and results (bit for bit) as mm_moe_decode; the workspace is a file-scope device array
 * of MM_NOALLOC_SCRATCH_BYTES per device, and the call allocates nothing. A call whose workspace
 * (mm_gemv_workspace(T * topk, E, H, I)) exceeds that size fails with MM_ERR_ARG: at most 62 routes per call at
 * H 4096 / I 2048 (T = 6 at top-8 plus a shared expert), 52 at H 5120 / I 2304. All calls on one device
 * share its array: calls that overlap on one device (concurrent streams or threads) race. The first call on a
 * device looks up the array's device address (hipGetSymbolAddress) and must run outside graph capture; later
 * calls may be captured. */
int mm_moe_decode_noalloc(const mm_layer_t* layer, const void* x, int x_dtype, int rescale, int T, int topk,
                          const int64_t* ids, const float* w, int max_rows, float* out, mm_stream_t stream);

/* ------------------------------------------------------------------------------ fat experts (prefill) */

/* Bytes of device workspace mm_grouped_gemm / mm_moe_prefill need for n routes over E experts (permutation,
 * per-expert records, transformed inputs, the down input and per-route outputs). */
size_t mm_prefill_workspace(int n, int E, int H, int I);

/* Fat-expert grouped GEMM (replaces apply_exl3_batched_fat's per-expert reconstruct + 128x128 GEMM,
 * patches/vllm-exl3-host-dma.patch:182-201, and runtime/dma_gemm.py:5-26 run_batch, which feeds it): for every
 * route s < T*topk whose expert (0 <= ids[s] < E) has more than cap routes in the call, computes the expert
 * SwiGLU MLP and writes Y fp32 [T*topk][H] row s; other rows are left untouched. The weights are decoded into LDS
 * as fp16 (the reconstruct's rounding, ft_core.h:75-83) once per 128 routes and multiplied on MFMA; fp16
 * activations, fp32 accumulation, fp16 rounding at the reference's points. x, x_dtype as for mm_expert_gemv
 * (no rescale). Needs H a multiple of 256, I of 128, E <= 1024. */
int mm_grouped_gemm(const mm_layer_t* layer, const void* x, int x_dtype, int T, int topk, const int64_t* ids, int cap,
                    float* Y, void* workspace, size_t workspace_bytes, mm_stream_t stream);

/* Prefill MoE layer: mm_grouped_gemm, then out fp32 [T][H] = (accumulate ? out : 0) + sum_j w[t,j] * y_{t,j}
 * over the routes j whose expert has more than cap routes, fp32 fma in ascending j. cap = 0, accumulate = 0 is
 * the whole layer (equal to mm_combine over the routes' rows); cap = the fat threshold with accumulate = 1 adds the
 * fat experts to an out that already holds the other routes, as apply_exl3_batched_fat does. */
int mm_moe_prefill(const mm_layer_t* layer, const void* x, int x_dtype, int T, int topk, const int64_t* ids,
                   const float* w, int cap, int accumulate, float* out, void* workspace, size_t workspace_bytes,
                   mm_stream_t stream);

/* The fused-MoE call of a prefill-sized batch (patches/vllm-exl3-host-dma.patch:241-449: experts with more than
 * the fat threshold routes through the fat-expert GEMM, patch:286-291,450-460, the others through the fused
 * group kernel), with the split made on the device: out fp32 [T][H] = sum_j w[t,j] * expert_{ids[t,j]}(x_t) over
 * the valid routes, where experts with more than cap routes run on the grouped GEMM (fp16-rounded weights, as the
 * reference's reconstruct) and the others on the decode path (the layer's codebook evaluation), each token's
 * decode-path routes added in ascending j onto its fat-expert sum. No host synchronisation: the call can be
 * captured. ids int64 [T*topk], w fp32 [T*topk], topk <= 16, cap >= 1; x as for mm_moe_prefill. Workspace:
 * mm_fused_moe_workspace(T, topk, E, H, I, cap) bytes. */
size_t mm_fused_moe_workspace(int T, int topk, int E, int H, int I, int cap);
int mm_fused_moe(const mm_layer_t* layer, const void* x, int x_dtype, int T, int topk, const int64_t* ids,
                 const float* w, int cap, float* out, void* workspace, size_t workspace_bytes, mm_stream_t stream);

/* ----------------------------------------------------------------------------------------- utility */

/* Fat-expert path on routes already sorted by expert, with the argument meaning of the reference's
 * apply_exl3_batched_fat(xh, token_sorted, weight_sorted, counts_host, inners, limit, cap, out, use_kernel, skip)
 * (patches/vllm-exl3-host-dma.patch:182-201): positions offsets[e] .. offsets[e] + counts[e] - 1 (offsets =
 * exclusive sums of counts) are expert e's routes, position p belongs to token token_sorted[p] (int64 [n]) with
 * weight weight_sorted[p] (fp16 bits [n]). For every expert with counts[e] > cap and skip[e] == 0 (skip uint8 [E]
 * may be NULL), out[t] += sum over the expert's positions p of token t of w[p] * expert_e(x_t), added per token in
 * ascending p (fp32 fma). counts int32 [E] in device memory; the layer's pointer tables give each expert's trellis
 * (a staging slot, a cache slot or the home copy) and `layer->limit` is the SwiGLU clamp. Experts whose range
 * passes n are ignored. x [T][H] as for mm_moe_prefill. Requires E <= 1024, H % 256 == 0, I % 128 == 0. */
size_t mm_fat_batched_workspace(int n, int T, int E, int H, int I);
int mm_fat_batched(const mm_layer_t* layer, const void* x, int x_dtype, int T, int n, const int64_t* token_sorted,
                   const uint16_t* weight_sorted, const int32_t* counts, const uint8_t* skip, int cap, float* out,
                   void* workspace, size_t workspace_bytes, mm_stream_t stream);

/* ------------------------------------------------------------------------------------ expert placement */

/* Slot-table repoint; replaces _ec_point's index_copy_ writes (ct/ct_vllm.py:268-279): items int64 [n][5] =
 * (e, gate address, up address, down address, slot) in device or host-mapped memory; for each item
 * gate_ptr[e], up_ptr[e], down_ptr[e] = the addresses and slotof[e] = slot (slotof int32 [E], may be NULL).
 * Items with e outside [0, E) are skipped; of several items naming one expert the last wins. Stream-ordered:
 * kernels enqueued after it on `stream` read the new placement, kernels before it the old one. n <= 65536. */
int mm_slot_point(int64_t* gate_ptr, int64_t* up_ptr, int64_t* down_ptr, int32_t* slotof, int E, const int64_t* items,
                  int n, mm_stream_t stream);

/* Staging copies; replaces the reference's per-expert copy_(non_blocking=True) of pinned host rows into cache
 * and staging slots (ct/ct_vllm.py:399-405, patches/vllm-exl3-host-dma.patch:100-124): copy i moves bytes[i]
 * bytes from src[i] to dst[i] (host arrays of addresses: device memory, or host memory from mm_host_alloc), as
 * copy-engine transfers (hipMemcpyAsync) enqueued on `stream`. A copy whose source and destination both continue
 * the previous one is merged into it. Returns the number of transfers enqueued (>= 0) or a negative error. */
int mm_stage_copy(const uint64_t* dst, const uint64_t* src, const uint64_t* bytes, int n, mm_stream_t stream);

/* Copy stream `index` (0 .. MM_COPY_STREAMS - 1) of `device` for work that must overlap the kernels of `compute`
 * (a stream of that device, or NULL for its null stream); replaces the reference's side streams for staging and
 * cache copies (torch.cuda.Stream(dev) at ct/ct_vllm.py:358 and patches/vllm-exl3-host-dma.patch:99,116).
 * HIP spreads streams over a few shared hardware queues (GPU_MAX_HW_QUEUES, 4 by default), so an ordinary side
 * stream can share the compute stream's queue, and its transfers then wait for the compute kernels queued before
 * them. The library keeps its own non-blocking streams and, on the first call for a (device, compute stream),
 * checks that the one it returns runs while `compute` is held (it synchronises both streams, holds `compute` with
 * a one-lane kernel that ends when the host releases it, and waits up to 50 ms for an empty kernel on the
 * candidate), trying up to 8 streams; later calls return the same stream at once. Different indices get
 * different streams where one is free. Returns MM_OK with *out the hipStream_t, MM_COPY_UNVERIFIED (> 0) with
 * *out a usable stream that no check could clear, or a negative error (also when `compute` is capturing a
 * graph). Streams live until the process ends. */
#define MM_COPY_STREAMS 4
#define MM_COPY_UNVERIFIED 1
int mm_copy_stream(int device, int index, mm_stream_t compute, mm_stream_t* out);

/* Synthetic trellis words: word i of a stream with `seed` is bits 16*(i%4)..+15 of
 * splitmix64(seed + (i/4 + 1) * 0x9E3779B97F4A7C15). Fills dst[j] = word(start + j) for j < n. */
int mm_synth_u16(uint16_t* dst, uint64_t n, uint64_t seed, uint64_t start, mm_stream_t stream);

/* Expert-store fill: for experts e in [0, E) of one layer whose trellis lives at gate_ptr/up_ptr/down_ptr,
 * writes the synthetic words of stream mm_expert_seed(layer_seed, e) (gate, then up, then down). */
int mm_synth_layer(const mm_layer_t* layer, uint64_t layer_seed, mm_stream_t stream);
uint64_t mm_expert_seed(uint64_t layer_seed, uint64_t expert);

/* HBM read calibration (no counterpart in the reference; the benchmark's measured read roofline): every byte of
 * src [bytes] (device memory, 16-byte aligned, bytes a multiple of 16) is loaded once in 16-byte vector loads by a
 * grid of `blocks` x 256 threads (0: 8 workgroups per CU), and an xor of everything read is written to *sink
 * (device memory) so that no load can be dropped. */
int mm_read_probe(const void* src, uint64_t bytes, uint32_t* sink, int blocks, mm_stream_t stream);

/* Convert an fp32 [T][H] activation to the expert input fp16 [T][H] through bf16, optionally rescaling each
 * row to unit RMS first (the decode-chain workload's between-layer step): x16 = fp16(bf16(x * s_t)),
 * s_t = 1/sqrt(mean(x_t^2)) if rescale else 1. Also writes bf16 [T][H] if x_bf16 != NULL. */
int mm_prepare_input(const float* x, int T, int H, int rescale, void* x_bf16, void* x_fp16, mm_stream_t stream);

/* ----------------------------------------------------------------------------------------- host tier */

/* Host expert tier (replaces the reference's CPU tier extension, kernels/cpu_avx2/ft_tier_ext.cpp:36-231, and its
 * expert kernel, kernels/cpu_avx2/ft_core.h:573-727): experts computed on the host cores straight from their
 * pinned home rows, serving the mailbox mm_split publishes. One tier per process. Needs an AVX-512 host
 * (F, BW, VL, VBMI2, VNNI) with F16C and FMA; every entry fails with MM_ERR_UNSUP / MM_ERR_ARG otherwise.
 *
 * mm_tier_init (tier_init, ft_tier_ext.cpp:36-56): `threads` workers pinned to cpus[0 .. ncpus) (the serving thread
 * is worker 0 and runs on cpus[0]); the mailbox is the split's: ctrl int64 [16] (ctrl[0] job sequence, written by
 * the GPU last; ctrl[1] done sequence, written here last; ctrl[2] layer, ctrl[3] tokens, ctrl[4] picks), hx fp16
 * [maxtok][H], picks int32 [maxpicks][3] = (token, expert, weight fp32 bits), hout fp32 [maxtok][H] (all host
 * memory the GPU maps, e.g. mm_host_alloc); they may be NULL (and the capacities 0) when only mm_tier_forward is
 * used. A published job with more than maxtok tokens or maxpicks picks, or naming a layer never added, is not
 * computed: the serving thread zeroes the hout rows that exist, answers it, and counts it as rejected (the
 * reference's worker trusts ctrl[3] and ctrl[4]). mode: 1 EXACT (fp16-rounded weights), 0 AFFINE, 2 I16 (int16
 * inputs per 128-block, exact int32 block sums), -1 automatic (I16 for a job whose experts have at most two rows
 * each, else AFFINE: the reference's choice, ft_tier_ext.cpp:130-132). H a multiple of 512, I of 128.
 * The first call registers a process exit handler that stops the serving thread and the workers before memory
 * released at exit (the mailbox, the expert homes) can go away. */
int mm_tier_init(int threads, const int* cpus, int ncpus, int64_t* ctrl, const void* hx, const int32_t* picks,
                 float* hout, int maxtok, int maxpicks, int mode, int H, int I, int nlayers);
/* Layer li (tier_add_layer, ft_tier_ext.cpp:60-101): ptrs int64 [E][3] host addresses of each expert's gate, up and
 * down trellis (tiles [K/16][N/16][96 B], as the GPU reads them); scales fp16 in host memory, per expert:
 * suh_g [E][H], svh_g [E][I], suh_u [E][H], svh_u [E][I], suh_d [E][I], svh_d [E][H]. The memory stays the
 * caller's and must outlive the tier. */
int mm_tier_add_layer(int li, int E, const int64_t* ptrs, const void* suh_g, const void* svh_g, const void* suh_u,
                      const void* svh_u, const void* suh_d, const void* svh_d);
/* SwiGLU clamp (tier_set_limit; 0 = off) and mode (tier_set_mode). */
int mm_tier_set_limit(float limit);
int mm_tier_set_mode(int mode);
/* Start / stop the serving thread (tier_start, tier_stop, ft_tier_ext.cpp:161-175): it waits for ctrl[0] to move,
 * copies the job's x rows and picks, computes sum over the picks of token t of w * expert(x_t) into hout rows
 * 0 .. tokens-1 (every row written), then stores ctrl[1] = ctrl[0] with release ordering. If ctrl[0] moved on
 * while the job was being copied (the combine gave up on it and the split published the next job over it), the
 * job is dropped uncomputed (hout untouched) and counted as stale; it is still answered, and the next job is
 * served. mm_tier_shutdown also stops the workers and frees the tier (mm_tier_init may then be called again);
 * the mailbox and the expert homes must stay allocated until it returns. */
int mm_tier_start(int cpu0);
int mm_tier_stop(void);
int mm_tier_shutdown(void);
/* Synchronous forward (tier_forward, ft_tier_ext.cpp:177-191), refused while the serving thread runs: x fp32
 * [m][H] (fp16-valued), sel int32 [m][k] (entries outside [0, E) skipped), w fp32 [m][k] -> out fp32 [m][H];
 * mode as for mm_tier_init (-1: the tier's mode). */
int mm_tier_forward(int li, const float* x, int m, const int32_t* sel, const float* w, int k, float* out, int mode);
/* out int64 [MM_TIER_NSTATS]: jobs answered, picks computed, tokens, jobs without picks, busy nanoseconds
 * (tier_stats), jobs rejected (larger than the mailbox, or an unknown layer), stale jobs dropped. */
#define MM_TIER_NSTATS 7
int mm_tier_stats(int64_t* out);

#ifdef __cplusplus
}
#endif

#endif /* MI355MOE_H */
