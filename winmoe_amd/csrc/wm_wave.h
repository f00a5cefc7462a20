// wm_wave.h -- wave- and workgroup-level building blocks shared by the
// standalone kernels (wm_kernels.hip) and the fused decode-step kernel
// (wm_decode.hip).  Workgroups are 256 threads (4 wave64s).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/winmoe_hip.h"
#include "wm_device.h"
#include "wm_launch.h"

namespace wm {

constexpr int WAVES = 4;               // waves per workgroup
constexpr int TILE_LDS = 4416;         // max tile (64 x 68 B) + 16 B alignment shift + 48 B over-read pad

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

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

// Coalesced 16-byte loads of one tile: bytes [off, off + nbytes) of W, read
// from the 16-byte aligned granules that contain them (a granule never
// crosses a page, so the over-read stays inside the allocation).
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

// e^x rounded to fp32 from the fp64 exponential: the correctly rounded value
// except when the fp64 result falls within an fp64 ulp of an fp32 rounding
// midpoint.  The routing softmax uses it so that its weights match a CPU
// expf of at most ~0.5 ulp error (the reference's, transformer.h:146) bit for
// bit in all but such corner cases.
WM_DEV float exp_rn(float x) { return (float)exp((double)x); }

WM_DEV float silu_mul(float g, float u) {
    // g * sigmoid(g) * u with the branch-stable sigmoid of deltanet_impl.h:108-115
    float sg;
    if (g >= 0.0f) sg = 1.0f / (1.0f + expf(-g));
    else { float z = expf(g); sg = z / (1.0f + z); }
    return g * sg * u;
}

// The SwiGLU output as the decode path's down projection takes it: fp32
// rounded to a 16-bit significand (the low 8 bits of the pattern, to nearest
// even: relative error <= 2^-17; an infinity stays, a NaN becomes a quiet
// NaN of the same sign), so that two of them and a 16-bit tag fit in one
// 64-bit hand-off word.  act24 is the 24-bit code, act_float its value.
WM_DEV uint32_t act24(float v) {
    const uint32_t u = __builtin_bit_cast(uint32_t, v);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (u >> 8) | 0x400000u;
    return (u + 0x7Fu + ((u >> 8) & 1u)) >> 8;
}
WM_DEV float act_float(uint32_t c) { return __builtin_bit_cast(float, c << 8); }
WM_DEV float act_round(float v) { return act_float(act24(v)); }

WM_DEV float sigmoid_stable(float v) {
    if (v >= 0.0f) return 1.0f / (1.0f + expf(-v));
    float z = expf(v);
    return z / (1.0f + z);
}

WM_DEV int64_t tile_nbytes(const Geo& g, int rows, int t) {
    int64_t rows_left = rows - (int64_t)t * g.rpt;
    return (rows_left >= g.rpt ? g.rpt : rows_left) * g.row_bytes;
}

// ---------------------------------------------------------------- tile streaming
// A wave streams its tiles through a ring of S LDS buffers filled by
// global_load_lds_dwordx4 (each instruction: 64 lanes x 16 B = 1 KB of
// consecutive bytes, written to LDS in lane order), so S tiles are in flight
// per wave with no register staging.  Every tile is exactly NI instructions
// (lanes past the tile end reload its last granule), so "tile t has landed"
// is s_waitcnt vmcnt(#instructions issued after it).

template <int T> WM_HD constexpr int tile_ni() {
    return T == Q8_0 ? 5 : (T == Q6_K ? 4 : ((T == Q4_K || T == Q5_K) ? 3 : 2));
}
template <int T> WM_HD constexpr int tile_buf() { return tile_ni<T>() * 1024; }

// Issue the NI DMA loads of bytes [off, off + nbytes) of W (16-byte granules
// containing them) into dst.  The weights are read once per step, so the
// loads carry the non-temporal policy (CPOL nt): streamed lines do not evict
// what other workgroups share (x, the router vector), and the stream runs
// ~14 % faster than with the default policy (6.9 vs 6.1 TB/s, 4352-byte tiles,
// 3 in flight per wave).
constexpr int CPOL_NT = 2;
// Agent-scope coherent read (the sc1 bit): past the XCD's L2, for data other
// XCDs write during the launch.
constexpr int CPOL_SC1 = 16;
template <int NI>
WM_DEV void tile_dma(const uint8_t* W, int64_t off, int64_t nbytes, int lane, lds8_t* dst) {
    const uintptr_t G = (uintptr_t)(W + off);
    const uintptr_t A = G & ~(uintptr_t)15;
    const int nch = (int)(((G - A) + (uintptr_t)nbytes + 15) >> 4);
#pragma unroll
    for (int k = 0; k < NI; k++) {
        int i = lane + 64 * k;
        i = i < nch ? i : nch - 1;
        __builtin_amdgcn_global_load_lds((const void*)(A + 16 * (uintptr_t)i),
                                         (__attribute__((address_space(3))) void*)(dst + 1024 * k), 16, 0, CPOL_NT);
    }
}

// s_waitcnt vmcnt(ahead * NI) for ahead in [0, S).
template <int NI, int S> WM_DEV void wait_tiles(int ahead) {
    static_assert((S - 1) * NI <= 63, "vmcnt range");
    if (ahead <= 0) WM_WAIT_VMCNT(0);
    else if (ahead == 1) WM_WAIT_VMCNT(NI);
    else if (S > 2 && ahead == 2) WM_WAIT_VMCNT(2 * NI);
    else WM_WAIT_VMCNT(3 * NI < 64 ? 3 * NI : 63);
}

// One wave: row sums W[row] . x over tiles [t0, t1) (t0 < t1) of a
// [rows][in] matrix.  x is the fp32 input vector (16-byte aligned); each
// lane builds the integer-dot operand of its segment in registers while the
// first S tiles are in flight.  Row results go to gout[row] (global,
// device-coherent when COH) and/or lout[row - lrow0] (LDS).  ring holds
// S * tile_buf<T>() bytes.
// The first S tiles of wave_stream's range (repeating the last one when the
// wave has fewer), issued ahead of the stream (PRE = true below).
template <int T, int S>
WM_DEV void wave_stream_prologue(const uint8_t* W, int rows, const Geo& g, int t0, int t1, lds8_t* ring, int lane) {
    constexpr int NI = tile_ni<T>(), BUF = tile_buf<T>();
#pragma unroll
    for (int s = 0; s < S; s++) {
        const int t = min(t0 + s, t1 - 1);
        tile_dma<NI>(W, (int64_t)t * g.tile_bytes, tile_nbytes(g, rows, t), lane, ring + s * BUF);
    }
}

// PRE: the prologue was issued earlier (wave_stream_prologue), before the
// input vector was ready; the operand fetch then waits for it as well.
template <int T, int S, bool COH, bool PRE = false>
WM_DEV void wave_stream(const uint8_t* W, int rows, const Geo& g, int t0, int t1, const float* xsrc, lds8_t* ring,
                        float* gout, __attribute__((address_space(3))) float* lout, int lrow0, int lane,
                        float gscale = 1.0f, bool scaled = false) {
    constexpr int NI = tile_ni<T>(), BUF = tile_buf<T>();
    const int rig = lane / g.lpr, sub = lane % g.lpr;
    f32x4 xr[16];
    xop_fetch<T>(xsrc, sub, xr);
    // The prologue always issues S tiles (repeating the last one when the
    // wave has fewer), so exactly S * NI loads follow the operand fetch.
    if constexpr (!PRE) wave_stream_prologue<T, S>(W, rows, g, t0, t1, ring, lane);
    // keep the operand arithmetic (which waits for the operand loads) after
    // the tile loads have been issued
    __builtin_amdgcn_sched_barrier(0);
    XOp x;
    xop_make<T>(xr, x);
    for (int t = t0; t < t1; t++) {
        const int s = (t - t0) % S;
        wait_tiles<NI, S>(min(S - 1, t1 - 1 - t));
        const uint32_t shift = (uint32_t)(((uintptr_t)W + (uintptr_t)((int64_t)t * g.tile_bytes)) & 15u);
        Seg<T> sg;
        sg.load(ring + s * BUF + shift, lane < g.active ? lane : 0);
        float p = lane < g.active ? seg_dot<T>(sg, x) : 0.0f;
        p = row_reduce(p, g.lpr);
        wave_lds_sync();           // every lane's reads of this buffer are done before it is refilled
        if (t + S < t1) tile_dma<NI>(W, (int64_t)(t + S) * g.tile_bytes, tile_nbytes(g, rows, t + S), lane, ring + s * BUF);
        const int row = t * g.rpt + rig;
        if (sub == g.lpr - 1 && rig < g.rpt && row < rows) {
            if (gout) gst<COH>(gout + row, scaled ? p * gscale : p);
            if (lout) lout[row - lrow0] = p;
        }
    }
}

// ---------------------------------------------------------------- workgroup items
// COH: the item's outputs are read by other workgroups of the same launch
// (device-coherent stores).  The input vector is always read with ordinary
// cached loads, even when another workgroup of the launch wrote it: its
// writer stores it device-coherently and raises a flag after the stores
// completed, nobody reads it before that flag, and caches hold nothing of it
// from earlier launches (each launch starts with invalidated caches), so no
// cache can return a stale copy.  Device-coherent loads would send every
// item's reads of the same few KB past L2 and congest the channels holding them.
constexpr int RING_S = 3;            // tiles in flight per wave
constexpr int GU_ROWS_MAX = 512;     // rows of one gate/up item (LDS row sums)

// Dynamic LDS of a 4-wave streaming workgroup: one ring per wave + gate/up row sums.
WM_HD constexpr int wg_stream_lds_bytes(int max_tile_buf) { return WAVES * RING_S * max_tile_buf + 2 * GU_ROWS_MAX * 4; }

// Gate/up + SwiGLU over tiles [tb, tb + 2*tpw) of one slot: waves 0-1 stream
// gate, waves 2-3 stream up (tpw tiles each), row sums meet in LDS, and
// act[row] = silu(g) * u.  A null matrix (bad expert id) yields zeros.
template <int T, bool COH>
WM_DEV void wg_gateup_item(const uint8_t* Wg, const uint8_t* Wu, int rows, int in, int tb, int tpw, const float* x,
                           float* act, uint8_t* lds) {
    typedef __attribute__((address_space(3))) float lf;
    constexpr int BUF = tile_buf<T>();
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const Geo g = geometry(T, in);
    const int ntiles = (rows + g.rpt - 1) / g.rpt;
    lf* garr = (lf*)(lds + WAVES * RING_S * BUF);
    lf* uarr = garr + GU_ROWS_MAX;
    const int r0 = tb * g.rpt;
    const int r1 = min(rows, (tb + 2 * tpw) * g.rpt);
    const int t0 = tb + (wave & 1) * tpw, t1 = min(t0 + tpw, ntiles);
    const uint8_t* W = wave < 2 ? Wg : Wu;
    if (Wg && Wu && t0 < t1)
        wave_stream<T, RING_S, COH>(W, rows, g, t0, t1, x, (lds8_t*)(lds + wave * RING_S * BUF), nullptr,
                                    wave < 2 ? garr : uarr, r0, lane);
    __syncthreads();
    for (int r = threadIdx.x; r < r1 - r0; r += 256)
        gst<COH>(act + r0 + r, (Wg && Wu) ? act_round(silu_mul(garr[r], uarr[r])) : 0.0f);
    __syncthreads();
}

// y[row] = W[row] . x over tiles [tb, tb + 4*tpw) (tpw per wave), times
// *scale when scale is not null.
template <int T, bool COH>
WM_DEV void wg_gemv_item(const uint8_t* W, int rows, int in, int tb, int tpw, const float* x, float* y, uint8_t* lds,
                         const float* scale = nullptr) {
    constexpr int BUF = tile_buf<T>();
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const Geo g = geometry(T, in);
    const int ntiles = (rows + g.rpt - 1) / g.rpt;
    const int t0 = tb + wave * tpw, t1 = min(t0 + tpw, ntiles);
    if (t0 >= t1) return;
    if (!W) {
        const int rig = lane / g.lpr, sub = lane % g.lpr;
        for (int t = t0; t < t1; t++) {
            int row = t * g.rpt + rig;
            if (sub == 0 && rig < g.rpt && row < rows) gst<COH>(y + row, 0.0f);
        }
        return;
    }
    wave_stream<T, RING_S, COH>(W, rows, g, t0, t1, x, (lds8_t*)(lds + wave * RING_S * BUF), y, nullptr, 0, lane,
                                scale ? *scale : 1.0f, scale != nullptr);
}

// wg_gemv_item for an input vector that is not ready yet: every wave issues
// its first RING_S weight tiles, then `wait()` (called by all threads of the
// workgroup) returns once x (and *scale) may be read, and the stream goes on
// with those tiles already on their way.
template <int T, bool COH, typename F>
WM_DEV void wg_gemv_item_prefetch(const uint8_t* W, int rows, int in, int tb, int tpw, const float* x, float* y,
                                  uint8_t* lds, const float* scale, F&& wait) {
    constexpr int BUF = tile_buf<T>();
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const Geo g = geometry(T, in);
    const int ntiles = (rows + g.rpt - 1) / g.rpt;
    const int t0 = tb + wave * tpw, t1 = min(t0 + tpw, ntiles);
    lds8_t* ring = (lds8_t*)(lds + wave * RING_S * BUF);
    if (W && t0 < t1) wave_stream_prologue<T, RING_S>(W, rows, g, t0, t1, ring, lane);
    wait();
    if (t0 >= t1) return;
    if (!W) {
        const int rig = lane / g.lpr, sub = lane % g.lpr;
        for (int t = t0; t < t1; t++) {
            int row = t * g.rpt + rig;
            if (sub == 0 && rig < g.rpt && row < rows) gst<COH>(y + row, 0.0f);
        }
        return;
    }
    wave_stream<T, RING_S, COH, true>(W, rows, g, t0, t1, x, ring, y, nullptr, 0, lane, scale ? *scale : 1.0f,
                                      scale != nullptr);
}

// ---------------------------------------------------------------- router
constexpr int ROUTER_LDS = 65536;    // LDS of a router workgroup (x + rows)

// LDS bytes of one router operand (x or one weight row): H floats plus the
// 16-byte alignment shift of an unaligned source, in whole 1 KB DMA units.
WM_HD int router_region(int H, bool aligned) { return ((H * 4 + (aligned ? 0 : 16) + 1023) / 1024) * 1024; }
// Rows per router workgroup (1..4), or 0 when x and one row do not fit.
WM_HD int router_rows_per_wg(int H, bool aligned) {
    int n = ROUTER_LDS / router_region(H, aligned) - 1;
    return n < 1 ? 0 : (n > 4 ? 4 : n);
}

// NB blocks of 8 reference-order FMA steps (block b: this lane's columns
// 128 b + 16 j from wp / xp, one base address per block and immediate
// offsets, the LDS reads paired two to an instruction, 8 per block).  The
// blocks are unrolled with three register sets in rotation: the reads of
// blocks b + 1 and b + 2 are in flight while block b's FMAs run, so those
// FMAs wait only for reads sent two blocks earlier.  (The LDS counter tracks
// 15 instructions: a loop over 16-step blocks in two sets waited for reads
// just sent, and a rolled loop's copies of carried registers waited for all.)
template <int NB> WM_DEV float rc_blocks(const lf32_t* wp, const lf32_t* xp) {
    float acc = 0.0f;
    float w[3][8], x[3][8];
#pragma unroll
    for (int b = 0; b < NB + 2; b++) {
        if (b < NB) {
            // block b's base addresses pass through an empty asm that takes
            // the running sum after block b - 3: no pass can hoist the reads
            // above those FMAs (a memory clobber or a scheduling barrier alone
            // does not hold LDS reads in straight-line code), and the
            // scheduling barrier below keeps them ahead of block b - 2's FMAs
            const lf32_t* wq = wp;
            const lf32_t* xq = xp;
            if (b >= 3) asm volatile("" : "+v"(wq), "+v"(xq) : "v"(acc));
#pragma unroll
            for (int j = 0; j < 8; j++) {
                w[b % 3][j] = wq[128 * b + 16 * j];
                x[b % 3][j] = xq[128 * b + 16 * j];
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        if (b >= 2) {
#pragma unroll
            for (int j = 0; j < 8; j++) acc = fmaf(w[(b - 2) % 3][j], x[(b - 2) % 3][j], acc);
        }
    }
    return acc;
}

// The steps of one chain in 8-step blocks for the step counts of
// H = 128 .. 4096 (H = 64 * 2^k): acc from them, the count done (the caller
// runs the rest, if any, one by one).
WM_DEV int rc_steps(const lf32_t* wp, const lf32_t* xp, int nsteps, float& acc) {
    switch (nsteps) {
    case 256: acc = rc_blocks<32>(wp, xp); return 256;
    case 128: acc = rc_blocks<16>(wp, xp); return 128;
    case 64: acc = rc_blocks<8>(wp, xp); return 64;
    case 32: acc = rc_blocks<4>(wp, xp); return 32;
    case 16: acc = rc_blocks<2>(wp, xp); return 16;
    case 8: acc = rc_blocks<1>(wp, xp); return 8;
    default: acc = 0.0f; return 0;
    }
}

// Router logits of rows [r0, r0 + nr), nr <= 4, in the reference order
// (transformer.h:172-191): lane l of a row keeps the running fp32 FMA over
// columns l, l+16, ...; the 16 lanes then reduce with the xor tree 8, 4, 2, 1
// (= _mm512_reduce_add_ps) and lane 0 adds the scalar tail.  x and the rows
// are pulled into LDS regions of `region` bytes at once (LDS-DMA, 1 KB per
// wave instruction, all in flight together); wave r then runs the 16 chains
// of row r.  Called by all 256 threads.
template <bool COH>
WM_DEV void wg_router_rows(const float* __restrict__ x, const float* __restrict__ W, int H, int r0, int nr, int region,
                           lds8_t* lds, float* __restrict__ logits, uint64_t* t_landed = nullptr) {
    typedef __attribute__((address_space(3))) float lf;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t nbytes = (int64_t)H * 4;
    // DMA units per operand: enough for H floats plus a possible 16 B shift,
    // never past the region (the host sizes the region for the actual shift)
    const int units = min((int)((nbytes + 16 + 1023) >> 10), region >> 10);
    // operand q: 0 = x, 1..nr = rows; its DMA units go round-robin over the waves
    for (int u = wave; u < (nr + 1) * units; u += WAVES) {
        const int q = u / units, k = u % units;
        const float* src = q == 0 ? x : W + (int64_t)(r0 + q - 1) * H;
        const uintptr_t G = (uintptr_t)src, A = G & ~(uintptr_t)15;
        const int nch = (int)(((G - A) + (uintptr_t)nbytes + 15) >> 4);
        int i = lane + 64 * k;
        i = i < nch ? i : nch - 1;
        // x is read by every router workgroup (default policy, stays in L2);
        // each weight row by one (non-temporal)
        if (q == 0)
            __builtin_amdgcn_global_load_lds((const void*)(A + 16 * (uintptr_t)i),
                                             (__attribute__((address_space(3))) void*)(lds + q * region + 1024 * k), 16,
                                             0, 0);
        else
            __builtin_amdgcn_global_load_lds((const void*)(A + 16 * (uintptr_t)i),
                                             (__attribute__((address_space(3))) void*)(lds + q * region + 1024 * k), 16,
                                             0, CPOL_NT);
    }
    WM_WAIT_VMCNT(0);
    __syncthreads();
    if (t_landed) *t_landed = __builtin_amdgcn_s_memrealtime();
    if (wave < nr && lane < 16) {
        const lf* xr = (const lf*)(lds + (((uintptr_t)x) & 15));
        const float* wsrc = W + (int64_t)(r0 + wave) * H;
        const lf* wr = (const lf*)(lds + (wave + 1) * region + (((uintptr_t)wsrc) & 15));
        const int H16 = H - (H & 15), nsteps = H16 / 16;
        float acc = 0.0f;
        int s = rc_steps(wr + lane, xr + lane, nsteps, acc);
        for (; s < nsteps; s++) acc = fmaf(wr[lane + 16 * s], xr[lane + 16 * s], acc);
        // xor tree 8, 4, 2, 1 over the 16 lanes as row rotations: after the
        // step of distance d the partial sums repeat with period d, so the
        // lane d places on is the xor partner up to that repetition
        acc += dpp_f32<DPP_ROR8>(acc);
        acc += dpp_f32<DPP_ROR4>(acc);
        acc += dpp_f32<DPP_ROR2>(acc);
        acc += dpp_f32<DPP_ROR1>(acc);
        if (lane == 0) {
            for (int c = H16; c < H; c++) acc = fmaf(wr[c], xr[c], acc);
            gst<COH>(logits + r0 + wave, acc);
        }
    }
    __syncthreads();
}

// K-pass arg-max (transformer.h:117-139: strict '>' from -1e30, skip picked,
// equal values to the lower index, NaN never picked, nothing valid -> index 0)
WM_DEV uint64_t topk_key(float v, int e) {
    if (!(v > -1e30f)) return 0ull;              // NaN / -inf / <= -1e30 never selected
    if (v == 0.0f) v = 0.0f;                     // -0 == +0 for the comparison
    uint32_t u = __builtin_bit_cast(uint32_t, v);
    u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((uint64_t)u << 32) | (uint64_t)(0xFFFFFFFFu - (uint32_t)e);
}

// Maximum of N keys of one lane (tree).
template <int N> WM_DEV uint64_t lane_max(const uint64_t (&k)[N]) {
    uint64_t m[N];
#pragma unroll
    for (int i = 0; i < N; i++) m[i] = k[i];
#pragma unroll
    for (int w = N / 2; w >= 1; w >>= 1)
#pragma unroll
        for (int i = 0; i < w; i++) m[i] = max_u64(m[i], m[i + w]);
    return m[0];
}

// K-pass arg-max state of one wave over E <= 64 * MAXV logits: every lane
// keeps the order keys of logits lane, lane + 64, ... and the maximum of
// them; a pick takes the wave maximum of those, and the lane that owned it
// clears it and recomputes its maximum.
template <int MAXV> struct Picker {
    uint64_t key[MAXV];
    uint64_t head;
    float v0;                                        // logits[0]: the value of a degenerate pick (index 0)

    template <bool COH> WM_DEV void init(const float* logits, int E, int lane) {
        float lv[MAXV];
        // all loads unconditional (index clamped) so they are in flight together
#pragma unroll
        for (int i = 0; i < MAXV; i++) lv[i] = gld<COH>(logits + min(lane + 64 * i, E - 1));
        v0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, lv[0]), 0));
#pragma unroll
        for (int i = 0; i < MAXV; i++) key[i] = (lane + 64 * i) < E ? topk_key(lv[i], lane + 64 * i) : 0ull;
        head = lane_max<MAXV>(key);
    }
    // As init, from values already in registers (lv[i] = logit lane + 64 i).
    WM_DEV void init_vals(const float (&lv)[MAXV], int E, int lane) {
        v0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, lv[0]), 0));
#pragma unroll
        for (int i = 0; i < MAXV; i++) key[i] = (lane + 64 * i) < E ? topk_key(lv[i], lane + 64 * i) : 0ull;
        head = lane_max<MAXV>(key);
    }
    // Next pick: its key (0 = degenerate, nothing valid left) in every lane.
    // The wave maximum of the 64-bit heads: the largest upper half; when one
    // lane alone holds it (the upper half is the logit's order bits, so
    // unless two logits are equal) that lane's head is the maximum, else a
    // second pass takes the largest lower half among the lanes holding it.
    WM_DEV uint64_t next() {
        const uint32_t hh = (uint32_t)(head >> 32);
        const uint32_t hi = wave_max_u32(hh);
        const uint64_t at_hi = __builtin_amdgcn_ballot_w64(hh == hi);
        uint32_t lo;
        if (__builtin_popcountll(at_hi) == 1) {
            const int wl = (int)__builtin_ctzll(at_hi);
            lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)head, wl);
        } else {
            lo = wave_max_u32(hh == hi ? (uint32_t)head : 0u);
        }
        const uint64_t best = ((uint64_t)hi << 32) | lo;
        if (best != 0ull && head == best) {
#pragma unroll
            for (int i = 0; i < MAXV; i++) key[i] = key[i] == best ? 0ull : key[i];
            head = lane_max<MAXV>(key);
        }
        return best;
    }
    WM_DEV static int id_of(uint64_t best) { return best ? (int)(0xFFFFFFFFu - (uint32_t)best) : 0; }
    // the value back from its order key (-0 comes back as +0, which changes
    // no difference or exponential of the softmax)
    WM_DEV float value_of(uint64_t best) const {
        if (!best) return v0;
        const uint32_t u = (uint32_t)(best >> 32);
        return __builtin_bit_cast(float, (u & 0x80000000u) ? (u & 0x7FFFFFFFu) : ~u);
    }
};

// One wave: top-K (K <= 16) of E <= 64 * MAXV logits and the softmax over
// the picks (transformer.h:142-149).  Lane k keeps pick k, writes ids[k] /
// w[k] and bumps the pick's hit counter; degenerate / non-finite routing is
// reported in *status.  The softmax matches the sequential form: wmax starts
// from pick 0 and takes later picks that compare greater, the exponentials
// are summed in k order.
template <int MAXV, bool COH>
WM_DEV void wave_topk_n(const float* logits, int E, int K, int32_t* ids, float* w, uint32_t* hits, int32_t* status,
                        int lane) {
    // the logits are read with ordinary loads also inside one launch: their
    // writers finish (device-coherent stores) before the flag that lets this
    // wave read them, and no cache holds an older copy (see wg_wait's users)
    Picker<MAXV> pk;
    pk.template init<false>(logits, E, lane);
    int my_e = 0;
    float my_v = 0.0f;
    bool degenerate = false;
    for (int k = 0; k < K; k++) {
        const uint64_t best = pk.next();
        degenerate = degenerate || best == 0ull;
        if (lane == k) { my_e = Picker<MAXV>::id_of(best); my_v = pk.value_of(best); }
    }
    const bool mine = lane < K;
    float wmax = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, my_v), 0));
    for (int k = 1; k < K; k++) {
        const float vk = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, my_v), k));
        if (vk > wmax) wmax = vk;
    }
    const float ex = mine ? exp_rn(my_v - wmax) : 0.0f;
    float wsum = 0.0f;
    for (int k = 0; k < K; k++) wsum += __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, ex), k));
    const float wk = wsum > 0.0f ? ex / wsum : ex;
    const bool nonfinite = __builtin_amdgcn_ballot_w64(mine && !isfinite(wk)) != 0ull;
    if (mine) {
        gst<COH>(ids + lane, (int32_t)my_e);
        gst<COH>(w + lane, wk);
        if (hits) atomicAdd(hits + my_e, 1u);
    }
    if (lane == 0) {
        int st = (degenerate ? WM_STATUS_DEGENERATE_ROUTING : 0) | (nonfinite ? WM_STATUS_NONFINITE_WEIGHT : 0);
        if (st && status) atomicOr(status, st);
    }
}

// Expert id and logit of routing slot `slot` (pick slot + 1 of the K-pass
// arg-max), computed by one wave from the logits (ordinary loads).
WM_DEV int wave_pick(const float* logits, int E, int slot, int lane, float& value) {
    uint64_t best = 0ull;
    if (E <= 512) {
        Picker<8> pk;
        pk.template init<false>(logits, E, lane);
        for (int k = 0; k <= slot; k++) best = pk.next();
        value = pk.value_of(best);
    } else {
        Picker<16> pk;
        pk.template init<false>(logits, E, lane);
        for (int k = 0; k <= slot; k++) best = pk.next();
        value = pk.value_of(best);
    }
    return Picker<8>::id_of(best);
}

// Softmax weight of pick k from the K pick logits, exactly as wave_topk_n
// computes it (wmax from pick 0 raised by later picks that compare greater,
// exponentials summed in k order).
WM_DEV float pick_weight(const float* v, int K, int k) {
    float wmax = v[0];
    for (int i = 1; i < K; i++) if (v[i] > wmax) wmax = v[i];
    float wsum = 0.0f;
    for (int i = 0; i < K; i++) wsum += exp_rn(v[i] - wmax);
    const float ex = exp_rn(v[k] - wmax);
    return wsum > 0.0f ? ex / wsum : ex;
}

template <bool COH = false>
WM_DEV void wave_topk(const float* logits, int E, int K, int32_t* ids, float* w, uint32_t* hits, int32_t* status,
                      int lane) {
    if (E <= 512) wave_topk_n<8, COH>(logits, E, K, ids, w, hits, status, lane);
    else wave_topk_n<16, COH>(logits, E, K, ids, w, hits, status, lane);
}

// Shared-expert gate: sigmoid_stable((float) sum_h g[h] * x[h]) with the dot
// in fp64 (winmoe_inference.c:2005-2009).  One wave: lane l accumulates
// h = l, l + 64, ... in order, then an xor tree over the 64 lanes (every lane
// ends with the same sum).  Every path (fused steps, per-phase kernels) uses
// this order, so they agree bit for bit.
WM_DEV float wave_shgate(const float* __restrict__ x, const float* __restrict__ g, int H, int lane) {
    double acc = 0.0;
    for (int base = 0; base < H; base += 64 * 16) {
        float gv[16], xv[16];
#pragma unroll
        for (int i = 0; i < 16; i++) {              // clamped, unconditional: all loads in flight together
            const int h = min(base + lane + 64 * i, H - 1);
            gv[i] = g[h];
            xv[i] = x[h];
        }
#pragma unroll
        for (int i = 0; i < 16; i++)
            if (base + lane + 64 * i < H) acc += (double)gv[i] * (double)xv[i];
    }
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) acc += __shfl_xor(acc, m);
    return sigmoid_stable((float)acc);
}

// wave_shgate with x in LDS (same order of operations).
WM_DEV float wave_shgate_lds(const lf32_t* x, const float* __restrict__ g, int H, int lane) {
    double acc = 0.0;
    for (int base = 0; base < H; base += 64 * 16) {
        float gv[16], xv[16];
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const int h = min(base + lane + 64 * i, H - 1);
            gv[i] = g[h];
            xv[i] = x[h];
        }
#pragma unroll
        for (int i = 0; i < 16; i++)
            if (base + lane + 64 * i < H) acc += (double)gv[i] * (double)xv[i];
    }
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) acc += __shfl_xor(acc, m);
    return sigmoid_stable((float)acc);
}

// wave_shgate for a whole workgroup (all threads call it; wave 0 computes,
// thread 0 writes *out).
template <bool COH = false>
WM_DEV void wg_shgate(const float* __restrict__ x, const float* __restrict__ g, int H, float* __restrict__ out) {
    if (threadIdx.x < 64) {
        const float r = wave_shgate(x, g, H, (int)threadIdx.x);
        if (threadIdx.x == 0) gst<COH>(out, r);
    }
    __syncthreads();
}

// ---------------------------------------------------------------- split operand build
// The integer-dot operand (xop_core) of one segment built by 8 lanes: lanes
// 8q .. 8q+7 of the wave share segment q, part p = lane % 8 holds weights
// j = 8p .. 8p+7 of it (v[i] = the input value of column seg_col(T, seg, 8p+i)).
// The record (XOP_DW dwords: hi bytes, lo bytes, run sums, scale) is written
// to LDS.  Same digits, sums and scale as xop_core: the maximum and the
// integer sums do not depend on the order, every digit is computed alone.
template <int T> WM_DEV void xop_part(const float (&v)[8], int part, lds32_t* rec) {
    constexpr bool Q8 = (T == Q8_0);
    constexpr int RUNLEN = (T == Q8_0 || T == Q4_K || T == Q5_K) ? 32 : 16;
    float amax = 0.0f;
    uint32_t fin = 1u;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        amax = fmaxf(amax, fabsf(v[i]));
        fin &= isfinite(v[i]) ? 1u : 0u;
    }
    // maximum / all-finite over the segment's 8 lanes (DPP within groups of
    // 8: xor 1, xor 2, then the mirror of the two quads)
    amax = fmaxf(amax, dpp_f32<DPP_XOR1>(amax));
    amax = fmaxf(amax, dpp_f32<DPP_XOR2>(amax));
    amax = fmaxf(amax, dpp_f32<DPP_HALF_MIRROR>(amax));
    fin = min(fin, dpp_u32<DPP_XOR1>(fin));
    fin = min(fin, dpp_u32<DPP_XOR2>(fin));
    fin = min(fin, dpp_u32<DPP_HALF_MIRROR>(fin));
    const bool finite = fin != 0u;
    const float inv = amax > 0.0f ? 32639.0f / amax : 0.0f;
    // the 8 hi and 8 lo digit bytes, packed little-endian in two dwords each
    uint32_t hb[2] = {0u, 0u}, lb[2] = {0u, 0u};
    int psum = 0;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        int xi = finite ? (int)rintf(v[i] * inv) : 0;
        xi = xi > 32639 ? 32639 : (xi < -32639 ? -32639 : xi);
        const int l = ((xi + 128) & 255) - 128;
        const int h = (xi - l) >> 8;
        hb[i >> 2] |= (uint32_t)(h & 0xFF) << (8 * (i & 3));
        lb[i >> 2] |= (uint32_t)(l & 0xFF) << (8 * (i & 3));
        psum += xi;
    }
    lds8_t* rb = (lds8_t*)rec;
    if (Q8) {
        // weights j = 8p .. 8p+7 sit at bytes j + 2 (+ 2 more from j = 32): a
        // 16-bit, a 32-bit and a 16-bit store per digit array
        const int p0 = 8 * part + 2 + (part >= 4 ? 2 : 0);
        typedef __attribute__((address_space(3))) uint16_t lds16_t;
        *(lds16_t*)(rb + 4 * XOP_HI + p0) = (uint16_t)hb[0];
        *(lds32_t*)(rb + 4 * XOP_HI + p0 + 2) = (hb[0] >> 16) | (hb[1] << 16);
        *(lds16_t*)(rb + 4 * XOP_HI + p0 + 6) = (uint16_t)(hb[1] >> 16);
        *(lds16_t*)(rb + 4 * XOP_LO + p0) = (uint16_t)lb[0];
        *(lds32_t*)(rb + 4 * XOP_LO + p0 + 2) = (lb[0] >> 16) | (lb[1] << 16);
        *(lds16_t*)(rb + 4 * XOP_LO + p0 + 6) = (uint16_t)(lb[1] >> 16);
    } else {
        rec[XOP_HI + 2 * part] = hb[0];
        rec[XOP_HI + 2 * part + 1] = hb[1];
        rec[XOP_LO + 2 * part] = lb[0];
        rec[XOP_LO + 2 * part + 1] = lb[1];
    }
    psum += (int)dpp_u32<DPP_XOR1>((uint32_t)psum);
    if (RUNLEN == 32) psum += (int)dpp_u32<DPP_XOR2>((uint32_t)psum);
    constexpr int LPR = RUNLEN / 8;                  // lanes per run
    if (part % LPR == 0) rec[XOP_SUM + part / LPR] = (uint32_t)psum;
    if (part == 0) {
        if (RUNLEN == 32) { rec[XOP_SUM + 2] = 0u; rec[XOP_SUM + 3] = 0u; }
        rec[XOP_S] = __builtin_bit_cast(uint32_t, finite ? amax / 32639.0f : __builtin_nanf(""));
        if (Q8) {
            rb[4 * XOP_HI + 0] = 0; rb[4 * XOP_HI + 1] = 0; rb[4 * XOP_HI + 34] = 0; rb[4 * XOP_HI + 35] = 0;
            rb[4 * XOP_LO + 0] = 0; rb[4 * XOP_LO + 1] = 0; rb[4 * XOP_LO + 34] = 0; rb[4 * XOP_LO + 35] = 0;
        } else {
            rec[XOP_HI + 16] = 0u;
            rec[XOP_LO + 16] = 0u;
        }
    }
}

// The 8 input values of part `part` of segment `seg` (16-byte aligned fp32 vector).
template <int T> WM_DEV void xop_part_fetch(const float* src, int seg, int part, float (&v)[8]) {
    const f32x4* p = (const f32x4*)(src + seg_col(T, seg, 8 * part));
    const f32x4 a = p[0], b = p[1];
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}

// As xop_part_fetch, from an fp32 vector in LDS.
template <int T> WM_DEV void xop_part_fetch_lds(const lf32_t* src, int seg, int part, float (&v)[8]) {
    const lf32_t* p = src + seg_col(T, seg, 8 * part);
#pragma unroll
    for (int i = 0; i < 8; i++) v[i] = p[i];
}

// An operand record from LDS into registers.
WM_DEV void xop_read(const lds32_t* rec, XOp& x) {
    typedef __attribute__((address_space(3))) const u32x4 lq;
    u32x4 r[10];
#pragma unroll
    for (int i = 0; i < 10; i++) r[i] = ((lq*)rec)[i];
    uint32_t d[40];
#pragma unroll
    for (int i = 0; i < 10; i++) { d[4 * i] = r[i].x; d[4 * i + 1] = r[i].y; d[4 * i + 2] = r[i].z; d[4 * i + 3] = r[i].w; }
#pragma unroll
    for (int i = 0; i < 17; i++) { x.hi[i] = d[XOP_HI + i]; x.lo[i] = d[XOP_LO + i]; }
#pragma unroll
    for (int i = 0; i < 4; i++) x.sum[i] = (int)d[XOP_SUM + i];
    x.s = __builtin_bit_cast(float, d[XOP_S]);
}

}  // namespace wm
