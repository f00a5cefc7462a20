// wm_kernels.hip -- CDNA4 (gfx950) kernels of the MoE expert-layer path and
// their launchers.  See wm_device.h for the segment / operand scheme.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "../../include/winmoe_hip.h"
#include "wm_device.h"
#include "wm_launch.h"
#include "wm_quant.h"

namespace wm {

constexpr int WAVES = 4;               // waves per workgroup of the segment kernels
constexpr int TILE_LDS = 4416;         // max tile (64 x 68 B) + 16 B alignment shift + 48 B over-read pad

// ------------------------------------------------------------------ helpers

WM_DEV const uint8_t* slot_matrix(const MatSet& m, int slot, int32_t* status) {
    if (slot < m.n_routed) {
        int e = m.ids ? m.ids[slot] : slot;
        if (e < 0 || e >= m.E) {
            if (status) atomicOr(status, WM_STATUS_BAD_EXPERT_ID);
            return nullptr;
        }
        return m.base + (int64_t)e * m.stride;
    }
    return m.shared;
}

// Issue the coalesced 16-byte loads of one tile: bytes [off, off + nbytes) of
// W, read from the 16-byte aligned granules that contain them.
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

struct TileLoad {
    u32x4 r[5];
    uint32_t shift;
    int nch;
};
WM_DEV void tile_issue(const uint8_t* W, int64_t off, int64_t nbytes, int lane, TileLoad& tl) {
    uintptr_t G = (uintptr_t)(W + off);
    uintptr_t A = G & ~(uintptr_t)15;
    tl.shift = (uint32_t)(G - A);
    tl.nch = (int)((tl.shift + nbytes + 15) >> 4);
    const u32x4* p = (const u32x4*)A;
#pragma unroll
    for (int k = 0; k < 5; k++) {
        int i = lane + 64 * k;
        if (i < tl.nch) tl.r[k] = __builtin_nontemporal_load(p + i);
    }
}
WM_DEV void tile_store(lds8_t* lt, const TileLoad& tl, int lane) {
    lds32_t* d = (lds32_t*)lt;
#pragma unroll
    for (int k = 0; k < 5; k++) {
        int i = lane + 64 * k;
        if (i < tl.nch) {
            lds32_t* q = d + 4 * i;
            q[0] = tl.r[k].x; q[1] = tl.r[k].y; q[2] = tl.r[k].z; q[3] = tl.r[k].w;
        }
    }
}

WM_DEV float silu_mul(float g, float u) {
    // g * sigmoid(g) * u with the branch-stable sigmoid of deltanet_impl.h:108-115
    float sg;
    if (g >= 0.0f) sg = 1.0f / (1.0f + expf(-g));
    else { float z = expf(g); sg = z / (1.0f + z); }
    return g * sg * u;
}

// ------------------------------------------------------------------ router

// Logits in the reference order (transformer.h:172-191): per row 16 running
// fp32 FMA lanes over columns c = l, l+16, ..., a 16-lane xor tree
// (8, 4, 2, 1 = _mm512_reduce_add_ps), then the scalar tail.  A workgroup
// stages RR rows and x in LDS with coalesced loads, then 16*RR lanes run the
// chains.
template <int RR>
__global__ __launch_bounds__(256) void k_router_logits(const float* __restrict__ x, const float* __restrict__ W, int H,
                                                       int E, float* __restrict__ logits) {
    extern __shared__ float s_mem[];
    int r0 = blockIdx.x * RR;
    int nr = min(RR, E - r0);
    float* srow = s_mem;
    float* sx = s_mem + RR * H;
    const float* src = W + (int64_t)r0 * H;
    int n = nr * H;
    if ((H & 3) == 0 && (((uintptr_t)W | (uintptr_t)x) & 15) == 0) {
        const f32x4* s4 = (const f32x4*)src;
        f32x4* d4 = (f32x4*)srow;
        for (int i = threadIdx.x; i < n / 4; i += 256) d4[i] = __builtin_nontemporal_load(s4 + i);
        for (int i = threadIdx.x; i < H / 4; i += 256) ((f32x4*)sx)[i] = ((const f32x4*)x)[i];
    } else {
        for (int i = threadIdx.x; i < n; i += 256) srow[i] = src[i];
        for (int i = threadIdx.x; i < H; i += 256) sx[i] = x[i];
    }
    __syncthreads();
    if ((int)threadIdx.x < 16 * nr) {
        int r = threadIdx.x >> 4, l = threadIdx.x & 15;
        const float* row = srow + r * H;
        float acc = 0.0f;
        int c = 0;
        for (; c + 15 < H; c += 16) acc = fmaf(row[c + l], sx[c + l], acc);
        acc += __shfl_xor(acc, 8, 16);
        acc += __shfl_xor(acc, 4, 16);
        acc += __shfl_xor(acc, 2, 16);
        acc += __shfl_xor(acc, 1, 16);
        if (l == 0) {
            for (; c < H; c++) acc = fmaf(row[c], sx[c], acc);
            logits[r0 + r] = acc;
        }
    }
}

int launch_router_logits(const float* x, const float* W, int H, int E, float* logits, hipStream_t s) {
    if ((size_t)3 * H * sizeof(float) <= 65536) {
        hipLaunchKernelGGL(k_router_logits<2>, dim3((E + 1) / 2), dim3(256), 3 * H * sizeof(float), s, x, W, H, E,
                           logits);
    } else {
        hipLaunchKernelGGL(k_router_logits<1>, dim3(E), dim3(256), 2 * H * sizeof(float), s, x, W, H, E, logits);
    }
    return (int)hipGetLastError();
}

// K-pass arg-max (transformer.h:117-139: strict '>' from -1e30, skip picked,
// equal values to the lower index, NaN never picked, nothing valid -> index 0)
// and softmax over the picks (:142-149).  One wave; E <= 1024.
WM_DEV uint64_t topk_key(float v, int e) {
    if (!(v > -1e30f)) return 0ull;              // NaN / -inf / <= -1e30 never selected
    if (v == 0.0f) v = 0.0f;                     // -0 == +0 for the comparison
    uint32_t u = __builtin_bit_cast(uint32_t, v);
    u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((uint64_t)u << 32) | (uint64_t)(0xFFFFFFFFu - (uint32_t)e);
}

__global__ __launch_bounds__(64) void k_topk(const float* __restrict__ logits, int E, int K, int32_t* __restrict__ ids,
                                             float* __restrict__ w, uint32_t* __restrict__ hits,
                                             int32_t* __restrict__ status) {
    constexpr int MAXV = 16;
    int lane = threadIdx.x;
    uint64_t key[MAXV];
#pragma unroll
    for (int i = 0; i < MAXV; i++) {
        int e = lane + 64 * i;
        key[i] = e < E ? topk_key(logits[e], e) : 0ull;
    }
    uint32_t picked = 0;
    int my_id[16];
    bool degenerate = false;
    for (int k = 0; k < K; k++) {
        uint64_t best = 0ull;
#pragma unroll
        for (int i = 0; i < MAXV; i++)
            if (!((picked >> i) & 1u) && key[i] > best) best = key[i];
#pragma unroll
        for (int m = 32; m >= 1; m >>= 1) {
            uint32_t lo = __shfl_xor((uint32_t)best, m, 64), hi = __shfl_xor((uint32_t)(best >> 32), m, 64);
            uint64_t o = ((uint64_t)hi << 32) | lo;
            best = o > best ? o : best;
        }
        int e = 0;
        if (best == 0ull) degenerate = true;
        else {
            e = (int)(0xFFFFFFFFu - (uint32_t)best);
            if ((e & 63) == lane) picked |= 1u << (e >> 6);
        }
        my_id[k] = e;
    }
    if (lane == 0) {
        float wl[16];
        for (int k = 0; k < K; k++) wl[k] = logits[my_id[k]];
        float wmax = wl[0];
        for (int k = 1; k < K; k++) if (wl[k] > wmax) wmax = wl[k];
        float wsum = 0.0f;
        for (int k = 0; k < K; k++) { wl[k] = expf(wl[k] - wmax); wsum += wl[k]; }
        if (wsum > 0.0f) for (int k = 0; k < K; k++) wl[k] /= wsum;
        bool nonfinite = false;
        for (int k = 0; k < K; k++) {
            ids[k] = my_id[k];
            w[k] = wl[k];
            nonfinite = nonfinite || !isfinite(wl[k]);
            if (hits) atomicAdd(hits + my_id[k], 1u);
        }
        int st = (degenerate ? WM_STATUS_DEGENERATE_ROUTING : 0) | (nonfinite ? WM_STATUS_NONFINITE_WEIGHT : 0);
        if (st && status) atomicOr(status, st);
    }
}

int launch_topk(const float* logits, int E, int K, int32_t* ids, float* w, uint32_t* hits, int32_t* status,
                hipStream_t s) {
    hipLaunchKernelGGL(k_topk, dim3(1), dim3(64), 0, s, logits, E, K, ids, w, hits, status);
    return (int)hipGetLastError();
}

// Shared-expert gate: sigmoid_stable((float) sum_h g[h] * x[h]) with the dot
// in fp64 (winmoe_inference.c:2005-2009); fixed-order tree reduction.
__global__ __launch_bounds__(256) void k_shgate(const float* __restrict__ x, const float* __restrict__ g, int H,
                                                float* __restrict__ out) {
    __shared__ double s_part[256];
    double acc = 0.0;
    for (int h = threadIdx.x; h < H; h += 256) acc += (double)g[h] * (double)x[h];
    s_part[threadIdx.x] = acc;
    __syncthreads();
    for (int m = 128; m >= 1; m >>= 1) {
        if ((int)threadIdx.x < m) s_part[threadIdx.x] += s_part[threadIdx.x + m];
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        float v = (float)s_part[0], sg;
        if (v >= 0.0f) sg = 1.0f / (1.0f + expf(-v));
        else { float z = expf(v); sg = z / (1.0f + z); }
        *out = sg;
    }
}

int launch_shgate(const float* x, const float* g, int H, float* out, hipStream_t s) {
    hipLaunchKernelGGL(k_shgate, dim3(1), dim3(256), 0, s, x, g, H, out);
    return (int)hipGetLastError();
}

// ------------------------------------------------------------------ activation operands

template <int T>
__global__ __launch_bounds__(64) void k_xprep(XPrepArgs a) {
    int nseg = a.in / SEG;
    int gid = blockIdx.x * 64 + threadIdx.x;
    if (gid >= a.nslots * nseg) return;
    int slot = gid / nseg, seg = gid % nseg;
    const float* src = a.src + slot * a.src_stride;
    float v[64];
    if (a.mode == 0) {
#pragma unroll
        for (int j = 0; j < 64; j++) v[j] = src[seg_col(T, seg, j)];
    } else {
        const float* src2 = a.src2 + slot * a.src_stride;
        float* act = a.act_out ? a.act_out + slot * a.act_stride : nullptr;
#pragma unroll
        for (int j = 0; j < 64; j++) {
            int c = seg_col(T, seg, j);
            v[j] = silu_mul(src[c], src2[c]);
            if (act) act[c] = v[j];
        }
    }
    build_xop<T>(v, a.out + slot * a.out_stride + (int64_t)seg * XOP_DW);
}

int launch_xprep(int t, const XPrepArgs& a, hipStream_t s) {
    int n = a.nslots * (a.in / SEG);
    dim3 grid((n + 63) / 64), block(64);
    switch (t) {
    case Q8_0: hipLaunchKernelGGL(k_xprep<Q8_0>, grid, block, 0, s, a); break;
    case Q2_K: hipLaunchKernelGGL(k_xprep<Q2_K>, grid, block, 0, s, a); break;
    case Q3_K: hipLaunchKernelGGL(k_xprep<Q3_K>, grid, block, 0, s, a); break;
    case Q4_K: hipLaunchKernelGGL(k_xprep<Q4_K>, grid, block, 0, s, a); break;
    case Q5_K: hipLaunchKernelGGL(k_xprep<Q5_K>, grid, block, 0, s, a); break;
    case Q6_K: hipLaunchKernelGGL(k_xprep<Q6_K>, grid, block, 0, s, a); break;
    default: return (int)hipErrorInvalidValue;
    }
    return (int)hipGetLastError();
}

// ------------------------------------------------------------------ expert GEMV

// y[slot][row] = W_slot[row] . x_slot.  Each wave streams `tiles_per_wave`
// consecutive tiles of one slot's matrix through its LDS slice, prefetching
// tile t+1 into registers while tile t is decoded.
template <int T>
__global__ __launch_bounds__(256) void k_gemv(GemvArgs a) {
    __shared__ __attribute__((aligned(16))) uint8_t s_tile[WAVES][TILE_LDS];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int slot = a.slot0 + blockIdx.y;
    const Geo g = geometry(T, a.in);
    const int ntiles = (a.rows + g.rpt - 1) / g.rpt;
    const int t0 = (blockIdx.x * WAVES + wave) * a.tiles_per_wave;
    const int t1 = min(t0 + a.tiles_per_wave, ntiles);
    if (t0 >= t1) return;
    float* y = a.y + slot * a.y_slot_stride;
    const int rig = lane / g.lpr, sub = lane % g.lpr;
    const uint8_t* W = slot_matrix(a.m, slot, a.status);
    if (!W) {
        for (int t = t0; t < t1; t++) {
            int row = t * g.rpt + rig;
            if (sub == 0 && rig < g.rpt && row < a.rows) y[row] = 0.0f;
        }
        return;
    }
    XOp x;
    load_xop(a.xop + slot * a.xop_slot_stride + (int64_t)sub * XOP_DW, x);
    lds8_t* lt = (lds8_t*)&s_tile[wave][0];
    TileLoad tl;
    auto tile_bytes = [&](int t) -> int64_t {
        int64_t rows_left = a.rows - (int64_t)t * g.rpt;
        return (rows_left >= g.rpt ? g.rpt : rows_left) * g.row_bytes;
    };
    tile_issue(W, (int64_t)t0 * g.tile_bytes, tile_bytes(t0), lane, tl);
    for (int t = t0; t < t1; t++) {
        uint32_t shift = tl.shift;
        tile_store(lt, tl, lane);
        wave_lds_sync();
        if (t + 1 < t1) tile_issue(W, (int64_t)(t + 1) * g.tile_bytes, tile_bytes(t + 1), lane, tl);
        Seg<T> sg;
        sg.load(lt + shift, lane < g.active ? lane : 0);
        float p = lane < g.active ? seg_dot<T>(sg, x) : 0.0f;
        p = row_reduce(p, g.lpr);
        int row = t * g.rpt + rig;
        if (sub == 0 && rig < g.rpt && row < a.rows) y[row] = p;
        wave_lds_sync();
    }
}

// act[slot][row] = silu(gate_row . x) * (up_row . x) for gate and up of the
// same type, sharing one activation operand.
template <int T>
__global__ __launch_bounds__(256) void k_gateup(GateUpArgs a) {
    __shared__ __attribute__((aligned(16))) uint8_t s_tile[WAVES][2][TILE_LDS];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int slot = a.slot0 + blockIdx.y;
    const Geo g = geometry(T, a.in);
    const int ntiles = (a.rows + g.rpt - 1) / g.rpt;
    const int t0 = (blockIdx.x * WAVES + wave) * a.tiles_per_wave;
    const int t1 = min(t0 + a.tiles_per_wave, ntiles);
    if (t0 >= t1) return;
    float* act = a.act + slot * a.act_slot_stride;
    const int rig = lane / g.lpr, sub = lane % g.lpr;
    const uint8_t* Wg = slot_matrix(a.gate, slot, a.status);
    const uint8_t* Wu = slot_matrix(a.up, slot, nullptr);
    if (!Wg || !Wu) {
        for (int t = t0; t < t1; t++) {
            int row = t * g.rpt + rig;
            if (sub == 0 && rig < g.rpt && row < a.rows) act[row] = 0.0f;
        }
        return;
    }
    XOp x;
    load_xop(a.xop + (int64_t)sub * XOP_DW, x);
    lds8_t* lg = (lds8_t*)&s_tile[wave][0][0];
    lds8_t* lu = (lds8_t*)&s_tile[wave][1][0];
    TileLoad tg, tu;
    auto tile_bytes = [&](int t) -> int64_t {
        int64_t rows_left = a.rows - (int64_t)t * g.rpt;
        return (rows_left >= g.rpt ? g.rpt : rows_left) * g.row_bytes;
    };
    tile_issue(Wg, (int64_t)t0 * g.tile_bytes, tile_bytes(t0), lane, tg);
    tile_issue(Wu, (int64_t)t0 * g.tile_bytes, tile_bytes(t0), lane, tu);
    for (int t = t0; t < t1; t++) {
        uint32_t shg = tg.shift, shu = tu.shift;
        tile_store(lg, tg, lane);
        tile_store(lu, tu, lane);
        wave_lds_sync();
        if (t + 1 < t1) {
            int64_t off = (int64_t)(t + 1) * g.tile_bytes, nb = tile_bytes(t + 1);
            tile_issue(Wg, off, nb, lane, tg);
            tile_issue(Wu, off, nb, lane, tu);
        }
        const int sl = lane < g.active ? lane : 0;
        float pg, pu;
        {
            Seg<T> sg;
            sg.load(lg + shg, sl);
            pg = lane < g.active ? seg_dot<T>(sg, x) : 0.0f;
        }
        {
            Seg<T> su;
            su.load(lu + shu, sl);
            pu = lane < g.active ? seg_dot<T>(su, x) : 0.0f;
        }
        pg = row_reduce(pg, g.lpr);
        pu = row_reduce(pu, g.lpr);
        int row = t * g.rpt + rig;
        if (sub == 0 && rig < g.rpt && row < a.rows) act[row] = silu_mul(pg, pu);
        wave_lds_sync();
    }
}

static int waves_for(int ntiles, int tpw) { return (ntiles + tpw - 1) / tpw; }

// Tiles per wave: enough waves to fill 256 CUs several times over, at least 1.
static int pick_tpw(int64_t total_tiles) {
    int64_t target_waves = 4096;
    int64_t tpw = (total_tiles + target_waves - 1) / target_waves;
    return (int)(tpw < 1 ? 1 : (tpw > 64 ? 64 : tpw));
}

int launch_gemv(int t, const GemvArgs& a0, int nslots, hipStream_t s) {
    GemvArgs a = a0;
    Geo g = geometry(t, a.in);
    int ntiles = (a.rows + g.rpt - 1) / g.rpt;
    if (a.tiles_per_wave <= 0) a.tiles_per_wave = pick_tpw((int64_t)ntiles * nslots);
    int nw = waves_for(ntiles, a.tiles_per_wave);
    dim3 grid((nw + WAVES - 1) / WAVES, nslots), block(64 * WAVES);
    switch (t) {
    case Q8_0: hipLaunchKernelGGL(k_gemv<Q8_0>, grid, block, 0, s, a); break;
    case Q2_K: hipLaunchKernelGGL(k_gemv<Q2_K>, grid, block, 0, s, a); break;
    case Q3_K: hipLaunchKernelGGL(k_gemv<Q3_K>, grid, block, 0, s, a); break;
    case Q4_K: hipLaunchKernelGGL(k_gemv<Q4_K>, grid, block, 0, s, a); break;
    case Q5_K: hipLaunchKernelGGL(k_gemv<Q5_K>, grid, block, 0, s, a); break;
    case Q6_K: hipLaunchKernelGGL(k_gemv<Q6_K>, grid, block, 0, s, a); break;
    default: return (int)hipErrorInvalidValue;
    }
    return (int)hipGetLastError();
}

int launch_gateup(int t, const GateUpArgs& a0, int nslots, hipStream_t s) {
    GateUpArgs a = a0;
    Geo g = geometry(t, a.in);
    int ntiles = (a.rows + g.rpt - 1) / g.rpt;
    if (a.tiles_per_wave <= 0) a.tiles_per_wave = pick_tpw((int64_t)ntiles * nslots * 2);
    int nw = waves_for(ntiles, a.tiles_per_wave);
    dim3 grid((nw + WAVES - 1) / WAVES, nslots), block(64 * WAVES);
    switch (t) {
    case Q8_0: hipLaunchKernelGGL(k_gateup<Q8_0>, grid, block, 0, s, a); break;
    case Q2_K: hipLaunchKernelGGL(k_gateup<Q2_K>, grid, block, 0, s, a); break;
    case Q3_K: hipLaunchKernelGGL(k_gateup<Q3_K>, grid, block, 0, s, a); break;
    case Q4_K: hipLaunchKernelGGL(k_gateup<Q4_K>, grid, block, 0, s, a); break;
    case Q5_K: hipLaunchKernelGGL(k_gateup<Q5_K>, grid, block, 0, s, a); break;
    case Q6_K: hipLaunchKernelGGL(k_gateup<Q6_K>, grid, block, 0, s, a); break;
    default: return (int)hipErrorInvalidValue;
    }
    return (int)hipGetLastError();
}

// ------------------------------------------------------------------ combine

// moe_out = sum_k w_k * y_k in top-K order with single-rounding FMAs
// (winmoe_inference.c:1971-1980), then + sigmoid-gated shared output
// (:2021-2026).  Experts with an out-of-range id contribute nothing.
__global__ __launch_bounds__(256) void k_combine(CombineArgs a) {
    int h = blockIdx.x * 256 + threadIdx.x;
    if (h >= a.H) return;
    float acc = 0.0f;
    for (int k = 0; k < a.K; k++) {
        int e = a.ids ? a.ids[k] : 0;
        if (e < 0 || e >= a.E) continue;
        acc = fmaf(a.w[k], a.ypart[k * a.y_stride + h], acc);
    }
    if (a.has_shared) {
        float ys = a.ypart[a.K * a.y_stride + h];
        if (a.sh_gate) ys *= *a.sh_gate;
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

int launch_fill_i32(int32_t* p, int32_t v, int64_t n, hipStream_t s) {
    if (n <= 0) return 0;
    hipLaunchKernelGGL(k_fill_i32, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, p, v, n);
    return (int)hipGetLastError();
}

}  // namespace wm
