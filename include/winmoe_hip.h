/*
 * winmoe_hip.h -- C-ABI of libwinmoe_hip.so, the MI355X (gfx950) MoE
 * expert-layer library.
 *
 * Two surfaces:
 *   1. wm_*   device-pointer, stream-ordered entry points.  Pointers are device
 *             (HBM) addresses, `stream` is a hipStream_t passed as void*
 *             (NULL = the null stream).  No call synchronises the host unless
 *             its comment says so.  The routing trace, per-expert hit counters
 *             and all scratch live in one caller-allocated workspace sized by
 *             wm_workspace_size().
 *   2. gpu_*  the expert subset of the reference's GPU offload ABI
 *             (engine/runtime/gpu_offload.h:15-100), same names, argument
 *             meaning and 0 / -1 / slot returns, caller-owned host buffers,
 *             blocking.  Any supported quant type may back a slot.
 *
 * Return codes: WM_OK (0) success, WM_ERR (-1) HIP runtime error (message on
 * stderr, as CHECK_CUDA does in gpu_offload.cu:23-29), WM_EINVAL (-2) bad
 * argument (unsupported type, misaligned pointer, shape outside the supported
 * set, undersized workspace).
 *
 * Threading: a workspace serves one stream at a time.  Calls on distinct
 * workspaces may come from several host threads and streams; the library
 * orders them where it must: the persistent decode kernel needs every CU at
 * once, so persistent launches never overlap.  On one stream, stream order
 * does it.  The first persistent launch on a second stream of a device waits
 * once for the device to drain (a host wait); after that every persistent
 * launch records an event and a launch on another stream than the last waits
 * for it on the device (no host wait).  Work of other libraries on other
 * streams only delays a step.  Under stream capture no ordering is added: do
 * not replay a captured decode step concurrently with other decode steps.
 * The gpu_* shims keep global state and are single-threaded like the
 * reference.
 */
#ifndef WINMOE_HIP_H
#define WINMOE_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define WM_OK 0
#define WM_ERR (-1)
#define WM_EINVAL (-2)

/* ggml tensor type ids (engine/runtime/gguf_parser.h:21-29; Q2_K = 10 and
 * Q3_K = 11 are the public ggml ids the reference table lacks). */
enum {
    WM_F32 = 0, WM_F16 = 1, WM_Q8_0 = 8, WM_Q2_K = 10, WM_Q3_K = 11,
    WM_Q4_K = 12, WM_Q5_K = 13, WM_Q6_K = 14
};

/* Workspace status bits (read back with wm_workspace_status). */
#define WM_STATUS_DEGENERATE_ROUTING 1   /* a top-K pass found no logit > -1e30 */
#define WM_STATUS_BAD_EXPERT_ID      2   /* forced routing named an id outside [0, E) */
#define WM_STATUS_NONFINITE_WEIGHT   4   /* a routing weight was NaN/Inf */
#define WM_STATUS_SPIN_TIMEOUT       8   /* a fused-step dependency wait hit its bound (results invalid;
                                            call wm_workspace_reset before the next call) */

/* wm_layer_desc.flags: run the decode step as a sequence of per-phase kernel
 * launches instead of the single fused launch (same results, bit for bit). */
#define WM_FLAG_MULTI_KERNEL 1
/* wm_layer_desc.flags: the fused step also records, per work item, its start,
 * dependency-satisfied and end times (device constant-rate clock) and its kind
 * into the workspace (diagnostics; see wm_workspace_timeline). */
#define WM_FLAG_TIMELINE 2
/* wm_layer_desc.flags: the fused decode step has two kernels with the same
 * results, bit for bit: the persistent kernel (one workgroup per CU; needs
 * every workgroup resident at once, every supported type pair, inter ==
 * inter_shared and the LDS budget of one workgroup per CU) and the
 * work-item-list kernel (one workgroup per work item, items wait only for
 * smaller ids).  By default the persistent kernel runs every layer that fits
 * it and the item-list kernel everything else; WM_FLAG_ITEM_KERNEL always
 * picks the item-list kernel.  WM_FLAG_PERSIST_KERNEL is the default choice,
 * stated explicitly. */
#define WM_FLAG_ITEM_KERNEL 4
#define WM_FLAG_PERSIST_KERNEL 8
/* wm_layer_desc.flags, test hook of the persistent kernel: every wait of the
 * step (on another workgroup's data or inside the workgroup) gives up at its
 * first unsuccessful poll instead of after ~0.1 s.  The step then ends at
 * once with WM_STATUS_SPIN_TIMEOUT set and invalid results;
 * wm_workspace_reset makes the workspace usable again.  Lets a test drive the
 * timeout path without anything waiting long. */
#define WM_FLAG_SPIN_PROBE 16
/* wm_layer_desc.flags, prefill only: the expert GEMMs take the batch's pairs
 * in passes of at most 16 (PASS16) or 32 (PASS32) pairs of one expert.  By
 * default a batch that averages at most 10 pairs per expert (T*K <= 10*E)
 * with Q8_0 gate/up, or at most 4 with K-quant gate/up, uses 16, any other
 * 32.  The results are the same bit for bit either way; only the speed
 * differs. */
#define WM_FLAG_PREFILL_PASS16 32
#define WM_FLAG_PREFILL_PASS32 64

/* One MoE layer.  Expert tensors are the raw GGUF blocks, stacked by expert:
 * gate/up expert e = [inter rows][hidden/QK blocks] at gate_exps + e*gate_stride,
 * down expert e = [hidden rows][inter/QK blocks] at down_exps + e*down_stride
 * (the per-expert slicing of winmoe_inference.c:467-489,1770-1775).  A stride
 * of 0 means densely packed.  Replaces the reference's LayerWeights expert
 * fields (engine/runtime/transformer.h:80-99). */
typedef struct wm_layer_desc {
    int32_t hidden;          /* H */
    int32_t inter;           /* I, routed expert intermediate */
    int32_t inter_shared;    /* I of the shared expert (0 = inter) */
    int32_t n_experts;       /* E */
    int32_t top_k;           /* K, 1..16 (no silent clamp, unlike winmoe_inference.c:812) */
    int32_t gate_type, up_type, down_type;
    int32_t sh_gate_type, sh_up_type, sh_down_type;
    int32_t flags;           /* WM_FLAG_* */
    const float* router;     /* [E][H] fp32, row-major; NULL only for forced routing */
    const void* gate_exps;
    const void* up_exps;
    const void* down_exps;
    int64_t gate_stride, up_stride, down_stride;
    const void* sh_gate;     /* shared expert [I_s][H/QK]; NULL = no shared expert */
    const void* sh_up;
    const void* sh_down;     /* [H][I_s/QK] */
    const float* sh_gate_inp;/* [H] fp32 sigmoid gate of the shared expert, or NULL */
    /* The step either side of the layer (fused decode step, persistent
     * kernel only; other paths return WM_EINVAL when norm_w is set): */
    const float* norm_w;     /* [H] fp32: the decode input is the residual stream h and the
                                layer's x = rmsnorm(h) (attention.h:29-44: fp64 sum of squares,
                                scale = 1/sqrtf(ss/H + norm_eps), (h*scale)*w); NULL: x is given */
    float norm_eps;          /* 1e-6 in the reference */
    int32_t add_residual;    /* with norm_w: out = h + moe_out (winmoe_inference.c:2041) */
} wm_layer_desc;

/* ---------------------------------------------------------------- library */

/* Selects the current HIP device and caches its properties.  Optional: every
 * entry point calls it on first use.  Returns WM_OK or WM_ERR. */
int wm_init(void);
const char* wm_version(void);
int wm_block_bytes(int qtype);          /* 0 if unsupported */
int wm_block_elems(int qtype);          /* 0 if unsupported */

/* -------------------------------------------------- device-pointer API */

/* Dequantise nblocks raw blocks to fp32 (bit-exact checking hook; the same
 * per-block decode the expert kernels use).  blocks must be 4-byte aligned. */
int wm_dequant(int qtype, const void* blocks, int64_t nblocks, float* out, void* stream);

/* Quantise n fp32 values (n a multiple of the block size) into qtype blocks.
 * Used to build synthetic expert tensors.  wm_quantize_host is the same
 * quantiser on host memory, bit-identical to the device one. */
int wm_quantize(int qtype, const float* x, int64_t n, void* blocks, void* stream);
int wm_quantize_host(int qtype, const float* x, int64_t n, void* blocks);

/* y[r] = sum_c W[r][c] x[c] for one raw quantised matrix [rows][in/QK]
 * (quant_matvec, engine/runtime/transformer.h:157-194, on the GPU). */
int wm_quant_matvec(int qtype, const void* W, const float* x, int rows, int in, float* y,
                    void* ws, int64_t ws_bytes, void* stream);

/* Router + top-K on the GPU: reference-order fp32 logits, K-pass arg-max with
 * ties to the lower index, softmax over the K picks
 * (router_topk, engine/runtime/transformer.h:107-152).  ids/w are device
 * arrays of length K.  Needs a workspace of wm_router_workspace_size(E). */
int64_t wm_router_workspace_size(int E);
/* Router logits only, fp32 [E], bit-identical to the reference's fp32 AVX-512
 * accumulation (quant_matvec default case, transformer.h:172-191; the device
 * counterpart of gpu_router, gpu_offload.h:66-67). */
int wm_router_logits(const float* x, const float* W_r, int H, int E, float* logits, void* stream);
int wm_router_topk(const float* x, const float* W_r, int H, int E, int K, int32_t* ids, float* w,
                   void* ws, int64_t ws_bytes, void* stream);

/* Bytes of the fixed HBM workspace for a layer: routing trace of max_tokens
 * entries, hit counters, activation scratch and the prefill buffers for up to
 * max_tokens tokens.  < 0 on bad descriptor. */
int64_t wm_workspace_size(const wm_layer_desc* d, int max_tokens);

/* Clears the trace, counters and status of a workspace (stream-ordered). */
int wm_workspace_reset(const wm_layer_desc* d, int max_tokens, void* ws, int64_t ws_bytes, void* stream);

/* Byte offset of the fused-step timeline in the workspace (valid when the
 * descriptor has WM_FLAG_TIMELINE): uint64 [capacity][8] = start, dependencies
 * met, main work done, end (device clock ticks, wm_device_clock_khz per ms),
 * kind | HW_ID << 8 | XCC_ID << 40, then for router items the time their
 * counter increment returned and, for the one that ran top-K, the time top-K
 * finished (0 otherwise), and the time its weight rows had landed in LDS
 * (router items only); kind 0 = shared gate / forced
 * routing, 1 = router, 2 = shared gate/up, 3 = routed gate/up, 4 = down (+8
 * when it also combined).
 * The persistent step (the default decode path) writes instead 32 words per
 * workgroup, [workgroup][32], device clock ticks (0: not reached): 0 start,
 * 1 x and the router rows in LDS, 2 its logits stored, 3 routing known,
 * 4 its last SwiGLU outputs published, 6 combine start, 7 end, 8 x operand
 * records built, 9 first streaming wave done, 11 every logit polled,
 * 16 + q its SwiGLU outputs of slot position q published (q < 12; position 0
 * is the shared expert when the layer has one). */
int wm_workspace_timeline(const wm_layer_desc* d, int max_tokens, int64_t* offset, int64_t* capacity);
int64_t wm_device_clock_khz(void);

/* Host-synchronous read of the workspace status bits (WM_STATUS_*). */
int wm_workspace_status(void* ws, int64_t ws_bytes, int32_t* status_out);

/* Device offsets (bytes from ws) of the routing trace: ids int32 [max_tokens][K],
 * weights fp32 [max_tokens][K], hit counters uint32 [E]. */
int wm_workspace_trace(const wm_layer_desc* d, int max_tokens, int64_t* ids_off, int64_t* w_off,
                       int64_t* hits_off);

/* One decode token through the MoE block (winmoe_inference.c:1684-2027):
 * router -> top-K -> K experts (gate/up -> SwiGLU -> down) -> weighted
 * combine -> shared expert with its sigmoid gate.  x fp32[H] in, out fp32[H]
 * = moe_out before the residual add.  step selects the trace entry
 * (step % max_tokens).  No host synchronisation. */
int wm_moe_decode(const wm_layer_desc* d, const float* x, float* out, void* ws, int64_t ws_bytes,
                  int max_tokens, int step, void* stream);

/* Same with routing supplied by the caller: ids int32[K], w fp32[K] (device).
 * Out-of-range ids set WM_STATUS_BAD_EXPERT_ID and contribute zero. */
int wm_moe_decode_forced(const wm_layer_desc* d, const float* x, const int32_t* ids, const float* w,
                         float* out, void* ws, int64_t ws_bytes, int max_tokens, int step, void* stream);

/* n_layers decode steps of one token chained as the reference chains its
 * layers (winmoe_inference.c:1659-1668: layer l's input is layer l-1's
 * output; with the RMSNorm and residual set on each descriptor that is
 * h_{l+1} = h_l + moe_l(rmsnorm(h_l))).  The reference has no such call: it
 * enters each layer on its own, as wm_moe_decode / wm_moe_decode_forced do
 * here, and the results are the same bit for bit.  Here up to 8 layers run in
 * one launch, each workgroup going on to the next layer as soon as it is done
 * with the previous one.  d, ws, ws_bytes: one entry per layer (each layer
 * its own workspace); every layer has the same hidden size; x fp32[H]; out
 * fp32[n_layers][H] receives every layer's output; ids, w: NULL (every layer
 * routed by its router) or one device pointer pair per layer (a NULL entry:
 * that layer uses its router).  Layers that the chained kernel does not take
 * (formats without an instance, LDS, workspaces that overlap another layer's
 * of the same launch) run one launch each, with the same results. */
int wm_moe_decode_stack(int n_layers, const wm_layer_desc* const* d, void* const* ws, const int64_t* ws_bytes,
                        const float* x, float* out, const int32_t* const* ids, const float* const* w,
                        int max_tokens, int step, void* stream);

/* Batched prefill of T tokens through the layer: x bf16 [T][H] -> out fp32
 * [T][H] (moe_out of every token).  The reference has no batched path: its
 * prompt tokens go one at a time through the decode loop
 * (winmoe_inference.c:1079,2286-2288), each with router_topk
 * (transformer.h:107-152) and the expert loop (:1684-2027); the result per
 * token is the same mathematics.  Here all T tokens are routed, the (token,
 * slot) pairs are grouped by expert in the workspace, each expert's matrices
 * are streamed once for all of its tokens on MFMA, and a weighted combine
 * gathers the outputs.  T <= max_tokens; the workspace (one per layer and
 * stream) holds wm_prefill_workspace_size(d, max_tokens) bytes, 256-byte
 * aligned.  x and out are 16-byte aligned.  Expert matrices (routed and
 * shared, each with its own formats): Q8_0 or Q2_K .. Q6_K, gate and up of
 * one format; 16-byte aligned with strides that are multiples of 16; H, I,
 * inter_shared multiples of 256; otherwise WM_EINVAL. */
int64_t wm_prefill_workspace_size(const wm_layer_desc* d, int max_tokens);
int wm_moe_prefill(const wm_layer_desc* d, const uint16_t* x_bf16, int T, float* out, void* ws,
                   int64_t ws_bytes, int max_tokens, void* stream);
/* Same with routing supplied by the caller: ids int32 [T][K], w fp32 [T][K]
 * (device).  Ids outside [0, E) are skipped and set WM_STATUS_BAD_EXPERT_ID. */
int wm_moe_prefill_forced(const wm_layer_desc* d, const uint16_t* x_bf16, int T, const int32_t* ids,
                          const float* w, float* out, void* ws, int64_t ws_bytes, int max_tokens, void* stream);
/* Byte offsets in a prefill workspace of the last call's routing: ids int32
 * [T][K], weights fp32 [T][K], per-expert pick counts uint32 [E] (cumulative
 * over calls until wm_workspace_reset-style clearing by the caller). */
int wm_prefill_workspace_routing(const wm_layer_desc* d, int max_tokens, int64_t* ids_off, int64_t* w_off,
                                 int64_t* hits_off);

/* One expert FFN: out = down(SwiGLU(gate x, up x)) (gpu_expert_ffn_fused's
 * maths on device pointers, any supported types). */
int wm_expert_ffn(const void* gate, int gate_type, const void* up, int up_type, const void* down,
                  int down_type, const float* x, int H, int I, float* out, void* ws, int64_t ws_bytes,
                  void* stream);
int64_t wm_expert_workspace_size(int H, int I);

/* ------------------------------------------------- decode without allocation */
/* No counterpart in the reference: for callers that cannot allocate device
 * memory (code under HIP graph capture, serving loops that forbid hipMalloc).
 * wm_moe_decode_noalloc is wm_moe_decode (routing by the router, one token)
 * with its workspace in a fixed device array the library holds on every
 * device it runs on until the process ends (WM_NOALLOC_SCRATCH_BYTES), so it
 * calls no hipMalloc / hipFree and creates nothing once wm_noalloc_init has
 * run on the device (it runs on the first call otherwise); the phase profiler
 * must be off.  x fp32[H] in, out fp32[H]; ids_out int32[K] / w_out fp32[K]
 * (device, may be NULL) receive the routing.  A layer whose decode workspace
 * (wm_workspace_size(d, 1)) exceeds the array returns WM_EINVAL.  Every call
 * on a device shares that device's array: calls that overlap on one device
 * (other streams, other threads) race and give wrong results.  Each call
 * clears the part it uses with a kernel before the step. */
#define WM_NOALLOC_SCRATCH_BYTES (3 * 1024 * 1024)
int wm_noalloc_init(void);
int64_t wm_noalloc_scratch_bytes(void);
int wm_moe_decode_noalloc(const wm_layer_desc* d, const float* x, float* out, int32_t* ids_out, float* w_out,
                          void* stream);
/* Host-synchronous read of the status bits of the last no-allocation call on
 * the current device. */
int wm_noalloc_status(int32_t* status_out);

/* ------------------------------------------- host -> HBM expert streaming */
/* For models whose experts do not all fit in HBM: a pool of n_slots expert
 * slots in HBM, each holding one expert's [gate | up | down] bytes (each part
 * 256-byte aligned), filled from host memory on demand.  Replaces the
 * reference's miss path -- asynchronous reads of every missing pick issued
 * before the first is computed, into [gate | up | down] slots
 * (winmoe_inference.c:1736-1789) -- and the per-slot upload of the GPU expert
 * cache (gpu_offload.cu:590-659).  A missing expert is copied with
 * asynchronous host-to-device copies on the pool's own stream; the step's
 * stream waits for those copies on the device, and a slot is rewritten only
 * after the steps that read it are over, so the host never waits for the
 * device (except when all 64 entries of the pool's slot-index ring are still
 * in flight).  Host memory should be pinned (hipHostMalloc) for the copies to
 * overlap compute.  One host thread drives a pool; its slot memory is the
 * caller's (n_slots * wm_pool_slot_bytes, 256-byte aligned, device memory). */
typedef struct wm_expert_pool wm_expert_pool;
int64_t wm_pool_slot_bytes(int64_t gate_bytes, int64_t up_bytes, int64_t down_bytes);
int wm_pool_create(void* slots, int64_t slots_bytes, int n_slots, int64_t gate_bytes, int64_t up_bytes,
                   int64_t down_bytes, wm_expert_pool** pool);
int wm_pool_destroy(wm_expert_pool* pool);
/* The pool as a layer's expert tensors: sets gate_exps / up_exps / down_exps
 * and their strides to the slots and n_experts to n_slots; a step on it takes
 * slot indices as expert ids (wm_moe_decode_forced). */
int wm_pool_layer(const wm_expert_pool* pool, wm_layer_desc* d);
/* Makes experts ids[0..n) of `layer` (n <= n_slots) resident for the next
 * steps on `stream`: a resident expert is a hit; a missing one goes to a free
 * slot, else to the least recently used slot that no unreleased acquire
 * holds, copied from gate_src + id * gate_stride (up, down alike).  Every id
 * must name one of the source's n_src experts (0 <= id < n_src).  Writes,
 * in stream order, the slot of each id to slots_dev (device int32 [n]): the
 * ids to pass to wm_moe_decode_forced on the pool's layer.  Returns the
 * number of misses; WM_EINVAL, before any state changes, for a bad argument
 * (an id outside [0, n_src) included) or when every slot is held by
 * unreleased acquires. */
int wm_pool_acquire(wm_expert_pool* pool, int layer, const int32_t* ids, int n, int n_src, const void* gate_src,
                    const void* up_src, const void* down_src, int64_t gate_stride, int64_t up_stride,
                    int64_t down_stride, int32_t* slots_dev, void* stream);
/* As wm_pool_acquire, from host memory that holds each expert as one image
 * in the slot layout -- gate at 0, up at ru(gate_bytes), down at
 * ru(gate_bytes) + ru(up_bytes), ru() rounding up to a multiple of 256 -- at
 * src + id * src_stride (src_stride >= wm_pool_slot_bytes): one copy per
 * missing expert instead of three.  When every part size is a multiple of
 * 256 bytes (every shape of the benchmarked layers) the image is the
 * reference's RAM cache slot, gate, up and down back to back
 * (winmoe_inference.c:1764-1786). */
int wm_pool_acquire_packed(wm_expert_pool* pool, int layer, const int32_t* ids, int n, int n_src, const void* src,
                           int64_t src_stride, int32_t* slots_dev, void* stream);
/* To be called once the steps that read the slots of the acquires since the
 * last release are enqueued on `stream`: those slots may then be recycled,
 * after those steps (the pool's stream waits for them on the device). */
int wm_pool_release(wm_expert_pool* pool, void* stream);
/* Hits, misses and bytes copied since the pool was created. */
int wm_pool_stats(const wm_expert_pool* pool, int64_t* hits, int64_t* misses, int64_t* bytes_copied);

/* ------------------------------------------------------------ profiling */
/* Per-phase device timers of wm_moe_decode / wm_moe_decode_forced /
 * wm_moe_prefill, the counterpart of the reference's per-phase
 * QueryPerformanceCounter accumulators (winmoe_inference.c:1031-1037,
 * 1685-1697, 1795-1806): when enabled, every phase launch is bracketed by HIP
 * events on the caller's stream.  wm_profile_read synchronises those events
 * and returns, per phase, the summed milliseconds and the launch count since
 * the last read (arrays of WM_PROF_NPHASE; names via wm_profile_phase_name). */
#define WM_PROF_NPHASE 8
int wm_profile_enable(int on);
int wm_profile_read(double* ms, int64_t* count, int nphase);
const char* wm_profile_phase_name(int phase);

/* ------------------------------- reference-compatible shims (host pointers) */
/* engine/runtime/gpu_offload.h:18-21 */
int gpu_init(void);
void gpu_shutdown(void);
int gpu_is_initialized(void);
float gpu_vram_used_mb(void);
/* engine/runtime/gpu_offload.h:66-67 */
int gpu_upload_router(int layer, const float* weights, int hidden_dim, int num_experts);
int gpu_router(int layer, const float* normed, int hidden_dim, float* logits_out, int num_experts);
/* engine/runtime/gpu_offload.h:70-74: copy one expert's raw [gate|up|down]
 * blocks into HBM; returns the slot or -1.  The quant types are inferred from
 * the byte sizes at compute time (every supported type has a distinct
 * bytes-per-weight ratio); gpu_cache_expert_typed records them explicitly. */
int gpu_cache_expert(int layer, int expert_id, const void* gate_data, int gate_size,
                     const void* up_data, int up_size, const void* down_data, int down_size);
int gpu_cache_expert_typed(int layer, int expert_id, const void* gate_data, int gate_size, int gate_type,
                           const void* up_data, int up_size, int up_type, const void* down_data,
                           int down_size, int down_type);
int gpu_find_cached_expert(int layer, int expert_id);                      /* gpu_offload.h:75 */
/* gpu_offload.h:76-80: gate/up outputs (pre-SwiGLU) and the expert output. */
int gpu_expert_ffn(int cache_idx, const float* input, int hidden_dim, int intermediate, float* gate_out,
                   float* up_out, float* expert_out, int gate_type, int down_type);
int gpu_expert_down(int cache_idx, const float* act, int intermediate, float* output, int hidden_dim);
/* gpu_offload.h:82-83: gate+up+SwiGLU+down on the GPU, blocking. */
int gpu_expert_ffn_fused(int cache_idx, const float* input, int hidden_dim, int intermediate,
                         float* expert_out);
/* gpu_offload.h:86-88 */
int gpu_expert_batch_start(const float* normed, int hidden_dim);
int gpu_expert_batch_add(int cache_idx, int hidden_dim, int intermediate, float weight);
int gpu_expert_batch_finish(float* moe_out, int hidden_dim);
int gpu_expert_cache_count(void);                                           /* gpu_offload.h:90 */
void gpu_set_expert_limit(int limit);                                       /* gpu_offload.h:93 */

#ifdef __cplusplus
}
#endif
#endif
