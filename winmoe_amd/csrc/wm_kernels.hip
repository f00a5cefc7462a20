// wm_kernels.hip -- CDNA4 (gfx950) kernels of the MoE expert-layer path and
// their launchers.  See wm_device.h for the segment / operand scheme.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "../../include/winmoe_hip.h"
#include "wm_device.h"
#include "wm_launch.h"
#include "wm_quant.h"
#include "wm_wave.h"

namespace wm {

// ------------------------------------------------------------------ router

// Logits in the reference order (transformer.h:172-191), rr rows per
// workgroup; see wg_router_rows.
__global__ __launch_bounds__(256) void k_router_logits(const float* __restrict__ x, const float* __restrict__ W, int H,
                                                       int E, int rr, int region, float* __restrict__ logits) {
    extern __shared__ __attribute__((aligned(16))) uint8_t s_dyn[];
    const int r0 = blockIdx.x * rr;
    wg_router_rows<false>(x, W, H, r0, min(rr, E - r0), region, (lds8_t*)s_dyn, logits);
}

int launch_router_logits(const float* x, const float* W, int H, int E, float* logits, hipStream_t s) {
    const bool aligned = (H % 4 == 0) && ((((uintptr_t)x) | ((uintptr_t)W)) & 15) == 0;
    const int rr = router_rows_per_wg(H, aligned), region = router_region(H, aligned);
    if (rr <= 0) return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL(k_router_logits, dim3((E + rr - 1) / rr), dim3(256), (size_t)ROUTER_LDS, s, x, W, H, E, rr,
                       region, logits);
    return (int)hipGetLastError();
}

// K-pass arg-max (transformer.h:117-139: strict '>' from -1e30, skip picked,
// equal values to the lower index, NaN never picked, nothing valid -> index 0)
// and softmax over the picks (:142-149).  One wave; E <= 1024.
__global__ __launch_bounds__(64) void k_topk(const float* __restrict__ logits, int E, int K, int32_t* __restrict__ ids,
                                             float* __restrict__ w, uint32_t* __restrict__ hits,
                                             int32_t* __restrict__ status) {
    wave_topk(logits, E, K, ids, w, hits, status, threadIdx.x);
}

int launch_topk(const float* logits, int E, int K, int32_t* ids, float* w, uint32_t* hits, int32_t* status,
                hipStream_t s) {
    hipLaunchKernelGGL(k_topk, dim3(1), dim3(64), 0, s, logits, E, K, ids, w, hits, status);
    return (int)hipGetLastError();
}

__global__ __launch_bounds__(256) void k_shgate(const float* __restrict__ x, const float* __restrict__ g, int H,
                                                float* __restrict__ out) {
    wg_shgate(x, g, H, out);
}

int launch_shgate(const float* x, const float* g, int H, float* out, hipStream_t s) {
    hipLaunchKernelGGL(k_shgate, dim3(1), dim3(256), 0, s, x, g, H, out);
    return (int)hipGetLastError();
}

// ------------------------------------------------------------------ SwiGLU

// act[slot][i] = silu(g[slot][i]) * u[slot][i] (gate and up of different
// types), rounded as every decode path hands it to the down projection.
__global__ __launch_bounds__(256) void k_swiglu(const float* __restrict__ g, const float* __restrict__ u,
                                                float* __restrict__ act, int n, int64_t stride) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    const int64_t o = (int64_t)blockIdx.y * stride + i;
    if (i < n) act[o] = act_round(silu_mul(g[o], u[o]));
}

int launch_swiglu(const float* g, const float* u, float* act, int n, int nslots, int64_t stride, hipStream_t s) {
    hipLaunchKernelGGL(k_swiglu, dim3((n + 255) / 256, nslots), dim3(256), 0, s, g, u, act, n, stride);
    return (int)hipGetLastError();
}

// ------------------------------------------------------------------ expert GEMV

// y[slot][row] = W_slot[row] . x_slot: workgroup = 4 waves x tiles_per_wave tiles.
template <int T>
__global__ __launch_bounds__(256) void k_gemv(GemvArgs a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t s_dyn[];
    const int slot = a.slot0 + blockIdx.y;
    const uint8_t* W = slot_matrix(a.m, slot, a.status);
    wg_gemv_item<T, false>(W, a.rows, a.in, blockIdx.x * WAVES * a.tiles_per_wave, a.tiles_per_wave,
                           a.x + slot * a.x_slot_stride, a.y + slot * a.y_slot_stride, s_dyn);
}

// act[slot][row] = silu(gate_row . x) * (up_row . x) for gate and up of the
// same type, sharing one activation operand: workgroup = 2 x tiles_per_wave tiles.
template <int T>
__global__ __launch_bounds__(256) void k_gateup(GateUpArgs a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t s_dyn[];
    const int slot = a.slot0 + blockIdx.y;
    const uint8_t* Wg = slot_matrix(a.gate, slot, a.status);
    const uint8_t* Wu = slot_matrix(a.up, slot, nullptr);
    wg_gateup_item<T, false>(Wg, Wu, a.rows, a.in, blockIdx.x * 2 * a.tiles_per_wave, a.tiles_per_wave, a.x,
                             a.act + slot * a.act_slot_stride, s_dyn);
}

static int tile_buf_rt(int t) {
    switch (t) {
    case Q8_0: return tile_buf<Q8_0>();
    case Q2_K: return tile_buf<Q2_K>();
    case Q3_K: return tile_buf<Q3_K>();
    case Q4_K: return tile_buf<Q4_K>();
    case Q5_K: return tile_buf<Q5_K>();
    case Q6_K: return tile_buf<Q6_K>();
    default: return 0;
    }
}

// Tiles per wave so a launch has about `target` workgroups (>= 1, <= cap).
static int pick_tpw(int64_t tiles_total, int tiles_per_wg_unit, int cap, int64_t target = 1024) {
    int64_t tpw = (tiles_total + target * tiles_per_wg_unit - 1) / (target * tiles_per_wg_unit);
    return (int)(tpw < 1 ? 1 : (tpw > cap ? cap : tpw));
}

#define WM_TYPE_SWITCH(t, KERNEL, ...)                                                                   \
    switch (t) {                                                                                         \
    case Q8_0: hipLaunchKernelGGL(KERNEL<Q8_0>, __VA_ARGS__); break;                                      \
    case Q2_K: hipLaunchKernelGGL(KERNEL<Q2_K>, __VA_ARGS__); break;                                      \
    case Q3_K: hipLaunchKernelGGL(KERNEL<Q3_K>, __VA_ARGS__); break;                                      \
    case Q4_K: hipLaunchKernelGGL(KERNEL<Q4_K>, __VA_ARGS__); break;                                      \
    case Q5_K: hipLaunchKernelGGL(KERNEL<Q5_K>, __VA_ARGS__); break;                                      \
    case Q6_K: hipLaunchKernelGGL(KERNEL<Q6_K>, __VA_ARGS__); break;                                      \
    default: return (int)hipErrorInvalidValue;                                                            \
    }

int launch_gemv(int t, const GemvArgs& a0, int nslots, hipStream_t s) {
    GemvArgs a = a0;
    Geo g = geometry(t, a.in);
    int ntiles = (a.rows + g.rpt - 1) / g.rpt;
    if (a.tiles_per_wave <= 0) a.tiles_per_wave = pick_tpw((int64_t)ntiles * nslots, WAVES, 64);
    int per_wg = WAVES * a.tiles_per_wave;
    dim3 grid((ntiles + per_wg - 1) / per_wg, nslots), block(64 * WAVES);
    size_t lds = wg_stream_lds_bytes(tile_buf_rt(t));
    WM_TYPE_SWITCH(t, k_gemv, grid, block, lds, s, a)
    return (int)hipGetLastError();
}

int launch_gateup(int t, const GateUpArgs& a0, int nslots, hipStream_t s) {
    GateUpArgs a = a0;
    Geo g = geometry(t, a.in);
    int ntiles = (a.rows + g.rpt - 1) / g.rpt;
    int cap = GU_ROWS_MAX / (2 * g.rpt);
    if (a.tiles_per_wave <= 0) a.tiles_per_wave = pick_tpw((int64_t)ntiles * nslots, 2, cap);
    if (a.tiles_per_wave > cap) a.tiles_per_wave = cap;
    int per_wg = 2 * a.tiles_per_wave;
    dim3 grid((ntiles + per_wg - 1) / per_wg, nslots), block(64 * WAVES);
    size_t lds = wg_stream_lds_bytes(tile_buf_rt(t));
    WM_TYPE_SWITCH(t, k_gateup, grid, block, lds, s, a)
    return (int)hipGetLastError();
}

// ------------------------------------------------------------------ combine

// moe_out = sum_k w_k * y_k in top-K order with single-rounding FMAs
// (winmoe_inference.c:1971-1980), then + sigmoid-gated shared output
// (:2021-2026).  Experts with an out-of-range id contribute nothing.
// out[h] = sum_k w_k y_k[h] (k order, invalid ids skipped) + gate * y_shared[h].
// Every load is unconditional (indices clamped) so they are in flight together.
__global__ __launch_bounds__(256) void k_combine(CombineArgs a) {
    constexpr int KMAX = 16;
    int h = blockIdx.x * 256 + threadIdx.x;
    if (h >= a.H) return;
    const int K1 = a.K + (a.has_shared ? 1 : 0);
    float yv[KMAX + 1], wv[KMAX];
    int ev[KMAX];
#pragma unroll
    for (int k = 0; k <= KMAX; k++) yv[k] = a.ypart[(int64_t)min(k, K1 - 1) * a.y_stride + h];
#pragma unroll
    for (int k = 0; k < KMAX; k++) {
        ev[k] = a.ids ? a.ids[min(k, a.K - 1)] : 0;
        wv[k] = a.w[min(k, a.K - 1)];
    }
    const float sg = a.sh_gate ? *a.sh_gate : 1.0f;
    float acc = 0.0f;
#pragma unroll
    for (int k = 0; k < KMAX; k++)
        if (k < a.K && ev[k] >= 0 && ev[k] < a.E) acc = fmaf(wv[k], yv[k], acc);
    if (a.has_shared) {
        float ys = yv[a.K];
        if (a.sh_gate) ys *= sg;
        acc = acc + ys;
    }
    a.out[h] = acc;
}

int launch_combine(const CombineArgs& a, hipStream_t s) {
    hipLaunchKernelGGL(k_combine, dim3((a.H + 255) / 256), dim3(256), 0, s, a);
    return (int)hipGetLastError();
}

// ------------------------------------------------------------------ dequant / quantise

// One wave per tile of 4096 weights (16 super-blocks or 128 Q8_0 blocks):
// the tile is staged in LDS exactly as in the GEMV, each lane decodes its
// segment with the same Seg<T>::load and writes the 64 dequantised weights.
template <int T>
__global__ __launch_bounds__(256) void k_dequant(const uint8_t* __restrict__ blocks, int64_t nblocks,
                                                 float* __restrict__ out) {
    __shared__ __attribute__((aligned(16))) uint8_t s_tile[WAVES][TILE_LDS];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    constexpr int BPT = (T == Q8_0) ? 128 : 16;      // blocks per tile
    const int64_t tile = (int64_t)blockIdx.x * WAVES + wave;
    const int64_t b0 = tile * BPT;
    if (b0 >= nblocks) return;
    const int64_t nb = min((int64_t)BPT, nblocks - b0);
    lds8_t* lt = (lds8_t*)&s_tile[wave][0];
    TileLoad tl;
    tile_issue(blocks, b0 * block_bytes(T), nb * block_bytes(T), lane, tl);
    tile_store(lt, tl, lane);
    wave_lds_sync();
    const int64_t lane_block = (T == Q8_0) ? 2 * lane : lane / 4;
    if (lane_block >= nb) return;
    Seg<T> sg;
    sg.load(lt + tl.shift, lane);
    float* o = out + tile * 4096;
#pragma unroll
    for (int j = 0; j < 64; j++) {
        int c = seg_col(T, lane, j);
        if (T != Q8_0 || (c >> 5) < nb) o[c] = seg_weight<T>(sg, j);
    }
}

int launch_dequant(int t, const void* blocks, int64_t nblocks, float* out, hipStream_t s) {
    int64_t bpt = (t == Q8_0) ? 128 : 16;
    int64_t tiles = (nblocks + bpt - 1) / bpt;
    dim3 grid((unsigned)((tiles + WAVES - 1) / WAVES)), block(64 * WAVES);
    const uint8_t* b = (const uint8_t*)blocks;
    switch (t) {
    case Q8_0: hipLaunchKernelGGL(k_dequant<Q8_0>, grid, block, 0, s, b, nblocks, out); break;
    case Q2_K: hipLaunchKernelGGL(k_dequant<Q2_K>, grid, block, 0, s, b, nblocks, out); break;
    case Q3_K: hipLaunchKernelGGL(k_dequant<Q3_K>, grid, block, 0, s, b, nblocks, out); break;
    case Q4_K: hipLaunchKernelGGL(k_dequant<Q4_K>, grid, block, 0, s, b, nblocks, out); break;
    case Q5_K: hipLaunchKernelGGL(k_dequant<Q5_K>, grid, block, 0, s, b, nblocks, out); break;
    case Q6_K: hipLaunchKernelGGL(k_dequant<Q6_K>, grid, block, 0, s, b, nblocks, out); break;
    default: return (int)hipErrorInvalidValue;
    }
    return (int)hipGetLastError();
}

__global__ __launch_bounds__(256) void k_quantize(int t, const float* __restrict__ x, int64_t nblocks,
                                                  uint8_t* __restrict__ out) {
    int64_t b = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (b >= nblocks) return;
    quant_block(t, x + b * block_elems(t), out + b * block_bytes(t));
}

int launch_quantize(int t, const float* x, int64_t nblocks, void* out, hipStream_t s) {
    hipLaunchKernelGGL(k_quantize, dim3((unsigned)((nblocks + 255) / 256)), dim3(256), 0, s, t, x, nblocks,
                       (uint8_t*)out);
    return (int)hipGetLastError();
}

// acc[i] = fma(w, y[i], acc[i]) (weighted_add_kernel, gpu_offload.cu:470-473).
__global__ void k_axpy(float* __restrict__ acc, const float* __restrict__ y, float w, int n) {
    int i = blockIdx.x * 256 + threadIdx.x;
    if (i < n) acc[i] = fmaf(w, y[i], acc[i]);
}

int launch_axpy(float* acc, const float* y, float w, int n, hipStream_t s) {
    hipLaunchKernelGGL(k_axpy, dim3((n + 255) / 256), dim3(256), 0, s, acc, y, w, n);
    return (int)hipGetLastError();
}

__global__ void k_fill_i32(int32_t* p, int32_t v, int64_t n) {
    int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) p[i] = v;
}

// Expert hit counters of caller-supplied routing (out-of-range ids flagged).
__global__ void k_count_hits(const int32_t* ids, int K, int E, uint32_t* hits, int32_t* status) {
    int k = threadIdx.x;
    if (k >= K) return;
    int e = ids[k];
    if (e >= 0 && e < E) atomicAdd(hits + e, 1u);
    else atomicOr(status, WM_STATUS_BAD_EXPERT_ID);
}

int launch_count_hits(const int32_t* ids, int K, int E, uint32_t* hits, int32_t* status, hipStream_t s) {
    hipLaunchKernelGGL(k_count_hits, dim3(1), dim3(64), 0, s, ids, K, E, hits, status);
    return (int)hipGetLastError();
}

int launch_fill_i32(int32_t* p, int32_t v, int64_t n, hipStream_t s) {
    if (n <= 0) return 0;
    hipLaunchKernelGGL(k_fill_i32, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, p, v, n);
    return (int)hipGetLastError();
}

}  // namespace wm
