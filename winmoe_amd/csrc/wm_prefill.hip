// wm_prefill.hip -- batched prefill of T tokens through the MoE block.
//
// The reference has no batched path: prompt tokens go one at a time through
// the decode loop (winmoe_inference.c:1079,2286-2288).  Here the T x K
// (token, slot) pairs are grouped by expert and every expert's matrices are
// streamed once for all of its tokens:
//
//   k_pf_router    reference-order fp32 logits of all tokens (tiles of 16
//                  tokens x 16 experts, each lane one of the 16 FMA chains of
//                  4 x 4 (token, expert) pairs)
//   k_pf_topk      one wave per token: K-pass arg-max + softmax
//   k_pf_group     counting sort of the pairs by expert; passes of <= 16
//                  or 32 pairs of one expert (prefill_pass_size)
//   k_pf_xpack     x as fp16 times a power of two per token
//   k_pf_gemm      gate and up + SwiGLU on fp16 MFMA, persistent: one
//                  workgroup per CU streams (pass, 128-row block) items
//                  through an LDS-DMA ring; the SwiGLU output is stored as
//                  fp16 hi + lo times a power of two per (pair, 128 rows);
//                  then the down projection of the same form (hi and lo:
//                  two MFMAs) (both in wm_pf_gemm.h, one instance per weight
//                  format; routed and shared experts of different formats
//                  take a launch each)
//   k_pf_combine   per token: sum_k w_k y_k in k order + gate * y_shared
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "../../include/winmoe_hip.h"
#include "wm_device.h"
#include "wm_format.h"
#include "wm_pf_gemm.h"
#include "wm_prefill.h"
#include "wm_wave.h"

namespace wm {

WM_DEV float bf16f(uint16_t b) { return __builtin_bit_cast(float, (uint32_t)b << 16); }

// ------------------------------------------------------------------ router

constexpr int PR_T = 16, PR_E = 16, PR_CH = 256, PR_LD = PR_CH + 4;

// Logits[t][e] in the reference order (transformer.h:172-191): for each
// (t, e), lane l keeps the fp32 FMA chain over columns l, l+16, ...; the 16
// lanes reduce with the xor tree 8, 4, 2, 1, then lane 0 adds the tail.
// Thread (chain l, sub-block sb) runs the chains of tokens 4*(sb/4)+i and
// experts 4*(sb%4)+j of the tile.
__global__ __launch_bounds__(256) void k_pf_router(const uint16_t* __restrict__ x, const float* __restrict__ W, int H,
                                                   int T, int E, float* __restrict__ logits) {
    __shared__ float xs[PR_T * PR_LD];
    __shared__ float wsh[PR_E * PR_LD];
    const int t0 = blockIdx.x * PR_T, e0 = blockIdx.y * PR_E;
    const int tid = threadIdx.x, l = tid & 15, sb = tid >> 4, tq = sb >> 2, eq = sb & 3;
    const int H16 = H - (H & 15);
    float acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] = 0.0f;
    for (int c0 = 0; c0 < H16; c0 += PR_CH) {
        const int cn = min(PR_CH, H16 - c0);
        for (int i = tid; i < PR_T * PR_CH; i += 256) {
            const int r = i / PR_CH, c = i % PR_CH;
            xs[r * PR_LD + c] = (t0 + r < T && c < cn) ? bf16f(x[(int64_t)(t0 + r) * H + c0 + c]) : 0.0f;
        }
        for (int i = tid; i < PR_E * PR_CH; i += 256) {
            const int r = i / PR_CH, c = i % PR_CH;
            wsh[r * PR_LD + c] = (e0 + r < E && c < cn) ? W[(int64_t)(e0 + r) * H + c0 + c] : 0.0f;
        }
        __syncthreads();
        for (int s = 0; s < cn / 16; s++) {
            float xv[4], wv[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                xv[i] = xs[(4 * tq + i) * PR_LD + l + 16 * s];
                wv[i] = wsh[(4 * eq + i) * PR_LD + l + 16 * s];
            }
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int j = 0; j < 4; j++) acc[i][j] = fmaf(wv[j], xv[i], acc[i][j]);
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) {
            // xor tree 8, 4, 2, 1 as row rotations (the partial sums repeat
            // with the period of the finished step)
            float v = acc[i][j];
            v += dpp_f32<DPP_ROR8>(v);
            v += dpp_f32<DPP_ROR4>(v);
            v += dpp_f32<DPP_ROR2>(v);
            v += dpp_f32<DPP_ROR1>(v);
            const int t = t0 + 4 * tq + i, e = e0 + 4 * eq + j;
            if (l == 0 && t < T && e < E) {
                for (int c = H16; c < H; c++) v = fmaf(W[(int64_t)e * H + c], bf16f(x[(int64_t)t * H + c]), v);
                logits[(int64_t)t * E + e] = v;
            }
        }
}

// The same logits, for H a multiple of 128 and 16-byte aligned x rows and
// router rows: tiles of 16 tokens x 32 experts, each thread the chain of
// column residue l of 4 tokens x 8 experts (32 accumulators: 12 LDS reads per
// 32 FMAs), the columns in chunks of 128 staged in LDS twice over: the loads
// (16-byte vectors) of the next two chunks are in flight while the current
// one is summed.  Every chain adds its columns in the same order as above, so the
// logits are the same bit for bit.  LDS rows are 144 floats (16 mod 32 and
// mod 64 banks) and the router row of local expert 8q + j is kept at row
// q + 4j: the four expert groups of a wave (q = 0..3) read the same column of
// rows q + 4j, 16 banks apart, with no conflict; rows stay 16-byte aligned
// for the staging's 16-byte stores.
constexpr int PQ_T = 16, PQ_E = 32, PQ_CH = 128, PQ_LD = PQ_CH + 16;
WM_HD constexpr int pq_wrow(int e) { return (e >> 3) + 4 * (e & 7); }
__global__ __launch_bounds__(256) void k_pf_router_v(const uint16_t* __restrict__ x, const float* __restrict__ W, int H,
                                                     int T, int E, float* __restrict__ logits) {
    __shared__ __attribute__((aligned(16))) float xs[2][PQ_T * PQ_LD];
    __shared__ __attribute__((aligned(16))) float wsh[2][PQ_E * PQ_LD];
    const int t0 = blockIdx.x * PQ_T, e0 = blockIdx.y * PQ_E;
    const int tid = threadIdx.x, l = tid & 15, sb = tid >> 4, tq = sb >> 2, eq = sb & 3;
    // staging: x row tid / 16, columns 8 (tid % 16) .. + 8 (one 16-byte load
    // of bf16); W row tid / 8, columns 16 (tid % 8) .. + 16 (four)
    const int xr = tid >> 4, xc = 8 * (tid & 15), wr = tid >> 3, wc = 16 * (tid & 7);
    const bool xin = t0 + xr < T, win = e0 + wr < E;
    const uint4* xsrc = (const uint4*)(x + (int64_t)(xin ? t0 + xr : 0) * H + xc);
    const uint4* wsrc = (const uint4*)(W + (int64_t)(win ? e0 + wr : 0) * H + wc);
    uint4 xv, wv[4], xv2, wv2[4];
    auto gload = [&](int c0) {
        const uint4 z = {0u, 0u, 0u, 0u};
        xv = xin ? xsrc[c0 / 8] : z;
#pragma unroll
        for (int q = 0; q < 4; q++) wv[q] = win ? wsrc[c0 / 4 + q] : z;
    };
    auto gload2 = [&](int c0) {
        const uint4 z = {0u, 0u, 0u, 0u};
        xv2 = xin ? xsrc[c0 / 8] : z;
#pragma unroll
        for (int q = 0; q < 4; q++) wv2[q] = win ? wsrc[c0 / 4 + q] : z;
    };
    auto lstore = [&](int b) {
        f32x4* xd = (f32x4*)&xs[b][xr * PQ_LD + xc];
        xd[0] = (f32x4){bf16f((uint16_t)(xv.x & 0xFFFFu)), bf16f((uint16_t)(xv.x >> 16)),
                        bf16f((uint16_t)(xv.y & 0xFFFFu)), bf16f((uint16_t)(xv.y >> 16))};
        xd[1] = (f32x4){bf16f((uint16_t)(xv.z & 0xFFFFu)), bf16f((uint16_t)(xv.z >> 16)),
                        bf16f((uint16_t)(xv.w & 0xFFFFu)), bf16f((uint16_t)(xv.w >> 16))};
        f32x4* wd = (f32x4*)&wsh[b][pq_wrow(wr) * PQ_LD + wc];
#pragma unroll
        for (int q = 0; q < 4; q++) wd[q] = __builtin_bit_cast(f32x4, wv[q]);
    };
    float acc[4][8];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 8; j++) acc[i][j] = 0.0f;
    const int nch = H / PQ_CH;
    gload(0);
    lstore(0);
    if (nch > 1) gload2(PQ_CH);
    __syncthreads();
    for (int c = 0; c < nch; c++) {
        const int b = c & 1;
        // chunk c + 1 is in flight in (xv2, wv2); chunk c + 2 goes out now
        xv = xv2;
#pragma unroll
        for (int q = 0; q < 4; q++) wv[q] = wv2[q];
        if (c + 2 < nch) gload2((c + 2) * PQ_CH);
        const float* xb = &xs[b][(4 * tq) * PQ_LD + l];
        const float* wb = &wsh[b][eq * PQ_LD + l];
#pragma unroll 2
        for (int st = 0; st < PQ_CH / 16; st++) {
            float xq[4], wq[8];
#pragma unroll
            for (int i = 0; i < 4; i++) xq[i] = xb[i * PQ_LD + 16 * st];
#pragma unroll
            for (int j = 0; j < 8; j++) wq[j] = wb[4 * j * PQ_LD + 16 * st];
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int j = 0; j < 8; j++) acc[i][j] = fmaf(wq[j], xq[i], acc[i][j]);
        }
        // (the other buffer was last read before the previous barrier)
        if (c + 1 < nch) lstore(b ^ 1);     // chunk c + 1
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 8; j++) {
            float v = acc[i][j];
            v += dpp_f32<DPP_ROR8>(v);
            v += dpp_f32<DPP_ROR4>(v);
            v += dpp_f32<DPP_ROR2>(v);
            v += dpp_f32<DPP_ROR1>(v);
            const int t = t0 + 4 * tq + i, e = e0 + 8 * eq + j;
            if (l == 0 && t < T && e < E) logits[(int64_t)t * E + e] = v;
        }
}

// ------------------------------------------------------------------ top-K, forced routing, grouping

__global__ __launch_bounds__(256) void k_pf_topk(const float* __restrict__ logits, int T, int E, int K,
                                                 int32_t* __restrict__ ids, float* __restrict__ w,
                                                 uint32_t* __restrict__ hits, int32_t* __restrict__ status) {
    const int t = blockIdx.x * WAVES + (threadIdx.x >> 6);
    if (t >= T) return;                       // whole waves
    wave_topk<false>(logits + (int64_t)t * E, E, K, ids + (int64_t)t * K, w + (int64_t)t * K, hits, status,
                     threadIdx.x & 63);
}

__global__ __launch_bounds__(256) void k_pf_forced(const int32_t* __restrict__ fids, const float* __restrict__ fw,
                                                   int n, int E, int32_t* __restrict__ ids, float* __restrict__ w,
                                                   uint32_t* __restrict__ hits, int32_t* __restrict__ status) {
    const int p = blockIdx.x * 256 + threadIdx.x;
    if (p >= n) return;
    const int e = fids[p];
    ids[p] = e;
    w[p] = fw[p];
    if (e >= 0 && e < E) atomicAdd(hits + e, 1u);
    else atomicOr(status, WM_STATUS_BAD_EXPERT_ID);
}

// Exclusive prefix sums of (a, b) over the 1024 threads of a workgroup; the
// totals go to *tot.  wsum: 16 x 2 ints of LDS.
WM_DEV int2 block_excl_scan2(int2 v, int* wsum, int2* tot) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    int2 inc = v;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const int ux = __shfl_up(inc.x, d), uy = __shfl_up(inc.y, d);
        if (lane >= d) {
            inc.x += ux;
            inc.y += uy;
        }
    }
    if (lane == 63) {
        wsum[2 * wave] = inc.x;
        wsum[2 * wave + 1] = inc.y;
    }
    __syncthreads();
    int2 before = make_int2(0, 0), all = make_int2(0, 0);
    for (int w = 0; w < 16; w++) {
        const int2 ws = make_int2(wsum[2 * w], wsum[2 * w + 1]);
        if (w < wave) {
            before.x += ws.x;
            before.y += ws.y;
        }
        all.x += ws.x;
        all.y += ws.y;
    }
    __syncthreads();
    *tot = all;
    return make_int2(before.x + inc.x - v.x, before.y + inc.y - v.y);
}

// Sizes for which k_pf_group keeps its data on chip: the pairs' expert ids
// in registers (up to PG_REG per thread), the sorted pair list and the
// tokens' exponents in LDS; larger batches read them from global memory.
constexpr int PG_REG = 8, PG_SORT = 10240, PG_XEXP = 2048;

// One workgroup: pairs grouped by expert (order inside an expert is free:
// every pair's output row is computed independently of the others), then
// cut into pass records of at most pm pairs (16 or 32): routed passes first,
// in expert order, then the shared expert's; pass_count = {routed passes,
// shared passes}.  A record also carries the x scale of each pair's token.
__global__ __launch_bounds__(1024) void k_pf_group(const int32_t* __restrict__ ids, int T, int K, int E, int has_shared,
                                                   int pm,
                                                   int32_t* __restrict__ offsets, int32_t* __restrict__ sorted,
                                                   int32_t* __restrict__ passes, int32_t* __restrict__ pass_count,
                                                   const int32_t* __restrict__ xexp) {
    __shared__ int cnt[1025];
    __shared__ int off[1026];
    __shared__ int pbase[1026];
    __shared__ int wsum[32];
    __shared__ int srt[PG_SORT];
    __shared__ int xe[PG_XEXP];
    const int tid = threadIdx.x, P = T * K, G = E + 1;      // group E: the shared expert (empty without one)
    const bool reg = P <= 1024 * PG_REG, lsort = P + (has_shared ? T : 0) <= PG_SORT, lxe = T <= PG_XEXP;
    // the ids and exponents are read once, together
    int ev[PG_REG];
#pragma unroll
    for (int i = 0; i < PG_REG; i++) ev[i] = reg && tid + 1024 * i < P ? ids[tid + 1024 * i] : -1;
    if (lxe)
        for (int t = tid; t < T; t += 1024) xe[t] = xexp[t];
    for (int e = tid; e < E; e += 1024) cnt[e] = 0;
    if (tid == 0) cnt[E] = has_shared ? T : 0;
    __syncthreads();
    if (reg) {
#pragma unroll
        for (int i = 0; i < PG_REG; i++)
            if (ev[i] >= 0 && ev[i] < E) atomicAdd(&cnt[ev[i]], 1);
    } else {
        for (int p = tid; p < P; p += 1024) {
            const int e = ids[p];
            if (e >= 0 && e < E) atomicAdd(&cnt[e], 1);
        }
    }
    __syncthreads();
    // pair offsets and pass bases of the groups, 1024 groups per round
    int2 carry = make_int2(0, 0);
    for (int base = 0; base < G; base += 1024) {
        const int e = base + tid;
        const int n = e < G ? cnt[e] : 0;
        int2 tot;
        const int2 ex = block_excl_scan2(make_int2(n, (n + pm - 1) / pm), wsum, &tot);
        if (e < G) {
            off[e] = carry.x + ex.x;
            pbase[e] = carry.y + ex.y;
            cnt[e] = carry.x + ex.x;          // scatter cursor
        }
        carry.x += tot.x;
        carry.y += tot.y;
    }
    if (tid == 0) {
        off[G] = carry.x;
        pbase[G] = carry.y;
    }
    __syncthreads();
    for (int e = tid; e <= G; e += 1024) offsets[e] = off[e];
    if (tid == 0) {
        pass_count[0] = pbase[E];
        pass_count[1] = pbase[G] - pbase[E];
    }
    // the sorted list: in LDS when it fits, else in global memory
    if (reg) {
#pragma unroll
        for (int i = 0; i < PG_REG; i++) {
            const int e = ev[i], p = tid + 1024 * i;
            if (e >= 0 && e < E) {
                const int pos = atomicAdd(&cnt[e], 1);
                if (lsort) srt[pos] = p;
                else sorted[pos] = p;
            }
        }
    } else {
        for (int p = tid; p < P; p += 1024) {
            const int e = ids[p];
            if (e >= 0 && e < E) {
                const int pos = atomicAdd(&cnt[e], 1);
                if (lsort) srt[pos] = p;
                else sorted[pos] = p;
            }
        }
    }
    if (has_shared)
        for (int t = tid; t < T; t += 1024) {
            if (lsort) srt[off[E] + t] = P + t;
            else sorted[off[E] + t] = P + t;
        }
    __syncthreads();
    // one thread per pass: its group by binary search over the pass bases
    const int npass = pbase[G];
    for (int q = tid; q < npass; q += 1024) {
        int lo = 0, hi = G - 1;                  // largest e with pbase[e] <= q
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (pbase[mid] <= q) lo = mid;
            else hi = mid - 1;
        }
        const int e = lo, first = off[e] + (q - pbase[e]) * pm;
        const int mn = min(pm, off[e + 1] - first);
        int32_t* rec = passes + (int64_t)q * GM_REC;
        rec[0] = e;
        rec[1] = mn;
        rec[2] = 0;
        rec[3] = 0;
        int prs[GM_M];
#pragma unroll
        for (int m = 0; m < GM_M; m++) {
            const int at = first + min(m, mn - 1);
            prs[m] = lsort ? srt[at] : sorted[at];
        }
#pragma unroll
        for (int m4 = 0; m4 < GM_M / 4; m4++) {
            uint32_t ex = 0;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int pr = prs[4 * m4 + j], tok = pair_token(pr, T, K);
                rec[4 + 4 * m4 + j] = pr;
                ex |= (uint32_t)((lxe ? xe[tok] : xexp[tok]) & 0xFF) << (8 * j);
            }
            rec[4 + GM_M + m4] = (int32_t)ex;
        }
    }
}

// x bf16 [T][H] -> x16 = fp16(x * 2^-e) with e per token (pf_exp of the
// token's largest |x|), xexp[t] = e.  bf16 values are exact in fp16 at that
// scale (8 significant bits, normal range down to 2^-29 of the maximum).
__global__ __launch_bounds__(256) void k_pf_xpack(const uint16_t* __restrict__ x, int H, uint16_t* __restrict__ x16,
                                                  int32_t* __restrict__ xexp) {
    __shared__ float wmax[WAVES];
    const int t = blockIdx.x, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint16_t* xr = x + (int64_t)t * H;
    float m = 0.0f;
    for (int c0 = threadIdx.x * 8; c0 < H; c0 += 256 * 8) {
        const u32x4 v = *(const u32x4*)(xr + c0);
#pragma unroll
        for (int i = 0; i < 4; i++)
            m = fmaxf(m, fmaxf(fabsf(__builtin_bit_cast(float, v[i] << 16)),
                               fabsf(__builtin_bit_cast(float, v[i] & 0xFFFF0000u))));
    }
    m = fmaxf(m, dpp_f32<DPP_XOR1>(m));
    m = fmaxf(m, dpp_f32<DPP_XOR2>(m));
    m = fmaxf(m, dpp_f32<DPP_HALF_MIRROR>(m));
    m = fmaxf(m, dpp_f32<DPP_MIRROR>(m));       // max of the 16 lanes of each row
    float r = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, m), 0));
    r = fmaxf(r, __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, m), 16)));
    r = fmaxf(r, __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, m), 32)));
    r = fmaxf(r, __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, m), 48)));
    if (lane == 0) wmax[wave] = r;
    __syncthreads();
    const float M = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
    const int e = pf_exp(M);
    const float inv = ldexpf(1.0f, -e);
    for (int c0 = threadIdx.x * 8; c0 < H; c0 += 256 * 8) {
        const u32x4 v = *(const u32x4*)(xr + c0);
        u32x4 o;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t lo = __builtin_bit_cast(uint16_t, (_Float16)(__builtin_bit_cast(float, v[i] << 16) * inv));
            const uint32_t hi =
                __builtin_bit_cast(uint16_t, (_Float16)(__builtin_bit_cast(float, v[i] & 0xFFFF0000u) * inv));
            o[i] = lo | (hi << 16);
        }
        *(u32x4*)(x16 + (int64_t)t * H + c0) = o;
    }
    if (threadIdx.x == 0) xexp[t] = e;
}

// Shared-expert gate of every token: sigmoid_stable((float) sum_h g[h] x[h])
// with the dot in fp64 (winmoe_inference.c:2005-2009), fixed-order tree.
__global__ __launch_bounds__(256) void k_pf_shgate(const uint16_t* __restrict__ x, const float* __restrict__ g, int H,
                                                   float* __restrict__ sg) {
    __shared__ double part[256];
    const int t = blockIdx.x;
    const uint16_t* xr = x + (int64_t)t * H;
    double acc = 0.0;
    for (int base = 0; base < H; base += 256 * 16) {
        float gv[16], xv[16];
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const int h = min(base + (int)threadIdx.x + 256 * i, H - 1);
            gv[i] = g[h];
            xv[i] = bf16f(xr[h]);
        }
#pragma unroll
        for (int i = 0; i < 16; i++)
            if (base + (int)threadIdx.x + 256 * i < H) acc += (double)gv[i] * (double)xv[i];
    }
    part[threadIdx.x] = acc;
    __syncthreads();
    for (int m = 128; m >= 1; m >>= 1) {
        if ((int)threadIdx.x < m) part[threadIdx.x] += part[threadIdx.x + m];
        __syncthreads();
    }
    if (threadIdx.x == 0) sg[t] = sigmoid_stable((float)part[0]);
}



// out[t][h] = sum_k w[t][k] y[t*K + k][h] (k order, invalid ids skipped) + gate(t) * y_shared[t][h];
// 4 consecutive h per thread.
__global__ __launch_bounds__(256) void k_pf_combine(PrefillArgs a) {
    const int t = blockIdx.y, h4 = blockIdx.x * 256 + threadIdx.x;
    if (4 * h4 >= a.H) return;
    const int H4 = a.H / 4;
    const f32x4* y4 = (const f32x4*)a.y;
    f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int k = 0; k < a.K; k++) {
        const int e = a.ids[(int64_t)t * a.K + k];
        if (e < 0 || e >= a.E) continue;
        const float wk = a.w[(int64_t)t * a.K + k];
        const f32x4 v = y4[((int64_t)t * a.K + k) * H4 + h4];
#pragma unroll
        for (int i = 0; i < 4; i++) acc[i] = fmaf(wk, v[i], acc[i]);
    }
    if (a.has_shared) {
        f32x4 ys = y4[((int64_t)a.T * a.K + t) * H4 + h4];
        if (a.sh_gate_inp) {
            const float gt = a.sg[t];
#pragma unroll
            for (int i = 0; i < 4; i++) ys[i] *= gt;
        }
#pragma unroll
        for (int i = 0; i < 4; i++) acc[i] = acc[i] + ys[i];
    }
    ((f32x4*)a.out)[(int64_t)t * H4 + h4] = acc;
}

// ------------------------------------------------------------------ launcher

int launch_prefill_route(const PrefillArgs& a, const int32_t* forced_ids, const float* forced_w, hipStream_t s) {
    const int P = a.T * a.K;
    if (forced_ids) {
        hipLaunchKernelGGL(k_pf_forced, dim3((P + 255) / 256), dim3(256), 0, s, forced_ids, forced_w, P, a.E, a.ids, a.w,
                           a.hits, a.status);
    } else {
        if (a.H % PQ_CH == 0 && ((uintptr_t)a.x & 15) == 0 && ((uintptr_t)a.router & 15) == 0)
            hipLaunchKernelGGL(k_pf_router_v, dim3((a.T + PQ_T - 1) / PQ_T, (a.E + PQ_E - 1) / PQ_E), dim3(256), 0, s,
                               a.x, a.router, a.H, a.T, a.E, a.logits);
        else
            hipLaunchKernelGGL(k_pf_router, dim3((a.T + PR_T - 1) / PR_T, (a.E + PR_E - 1) / PR_E), dim3(256), 0, s, a.x,
                               a.router, a.H, a.T, a.E, a.logits);
        hipLaunchKernelGGL(k_pf_topk, dim3((a.T + WAVES - 1) / WAVES), dim3(256), 0, s, a.logits, a.T, a.E, a.K, a.ids,
                           a.w, a.hits, a.status);
    }
    hipLaunchKernelGGL(k_pf_xpack, dim3(a.T), dim3(256), 0, s, a.x, a.H, a.x16, a.xexp);
    hipLaunchKernelGGL(k_pf_group, dim3(1), dim3(1024), 0, s, a.ids, a.T, a.K, a.E, a.has_shared, a.pass_m, a.offsets,
                       a.sorted, a.passes, a.pass_count, a.xexp);
    if (a.has_shared && a.sh_gate_inp)
        hipLaunchKernelGGL(k_pf_shgate, dim3(a.T), dim3(256), 0, s, a.x, a.sh_gate_inp, a.H, a.sg);
    return (int)hipGetLastError();
}

// One gate/up or down GEMM launch of format wt over the passes sel selects,
// for passes of m pairs.
template <int M> static int launch_q8(int nmat, int nsub, const PfGemm& g, int n_wg, hipStream_t s) {
    if (nmat == 2) return launch_pf_gemm<1, 1, 2, Q8_0, M>(g, n_wg, s);     // gate and up in alternate stages
    return nsub == 4 ? launch_pf_gemm<1, 2, 4, Q8_0, M>(g, n_wg, s) : launch_pf_gemm<1, 2, 2, Q8_0, M>(g, n_wg, s);
}
static int launch_fmt(int m, int nmat, int nsub, int wt, const PfGemm& g, int n_wg, hipStream_t s) {
    if (wt != Q8_0) return launch_pf_gemm_kq(m, nmat, nsub, wt, g, n_wg, s);
    return m == 16 ? launch_q8<16>(nmat, nsub, g, n_wg, s) : launch_q8<32>(nmat, nsub, g, n_wg, s);
}

// Routed and shared passes in one launch when their formats agree, else in two.
static int launch_split(int m, int nmat, int nsub, int wt_r, int wt_s, bool has_shared, PfGemm& g, int n_wg,
                        hipStream_t s) {
    if (!has_shared || wt_r == wt_s) {
        g.sel = 0;
        return launch_fmt(m, nmat, nsub, wt_r, g, n_wg, s);
    }
    g.sel = 1;
    if (int rc = launch_fmt(m, nmat, nsub, wt_r, g, n_wg, s)) return rc;
    g.sel = 2;
    return launch_fmt(m, nmat, nsub, wt_s, g, n_wg, s);
}

int launch_prefill_gateup(const PrefillArgs& a, hipStream_t s) {
    PfGemm g = {};
    g.w0 = a.gate; g.w1 = a.up; g.st0 = a.gstride; g.st1 = a.ustride;
    g.s0 = a.sh_gate; g.s1 = a.sh_up;
    g.rb_r = matrix_bytes(a.gt, 1, a.H);
    g.rb_s = a.has_shared ? matrix_bytes(a.sgt, 1, a.H) : g.rb_r;
    g.mb_r = (int32_t)(g.rb_r * a.I);
    g.mb_s = a.has_shared ? (int32_t)(g.rb_s * a.Is) : g.mb_r;
    g.a_hi = a.x16; g.a_lo = a.x16; g.a_ld = a.H; g.a_sc = nullptr; g.sc_ld = 0;
    g.a_bytes = (int32_t)((int64_t)a.T * a.H * 2); g.sc_bytes = 0;
    g.T = a.T; g.K = a.K; g.E = a.E; g.by_token = 1;
    g.nrb_r = a.I / GM_ROWS; g.nrb_s = a.has_shared ? a.Is / GM_ROWS : 1;
    g.ncol_r = g.ncol_s = a.H;
    g.recs = a.passes; g.npass = a.pass_count;
    g.o_hi = a.act_hi; g.o_lo = a.act_lo; g.o_sc = a.act_sc; g.o_ld = a.act_stride; g.osc_ld = a.act_stride / 128;
    return launch_split(a.pass_m, 2, 1, a.gt, a.sgt, a.has_shared, g, a.n_wg, s);
}

int launch_prefill_down(const PrefillArgs& a, hipStream_t s) {
    PfGemm g = {};
    g.w0 = a.down; g.w1 = a.down; g.st0 = g.st1 = a.dstride;
    g.s0 = g.s1 = a.sh_down;
    g.rb_r = matrix_bytes(a.dt, 1, a.I);
    g.rb_s = a.has_shared ? matrix_bytes(a.sdt, 1, a.Is) : g.rb_r;
    g.mb_r = (int32_t)(g.rb_r * a.H); g.mb_s = (int32_t)(g.rb_s * a.H);
    g.a_hi = a.act_hi; g.a_lo = a.act_lo; g.a_ld = a.act_stride; g.a_sc = a.act_sc; g.sc_ld = a.act_stride / 128;
    const int64_t pairs = (int64_t)a.T * a.K + (a.has_shared ? a.T : 0);
    g.a_bytes = (int32_t)(pairs * a.act_stride * 2); g.sc_bytes = (int32_t)(pairs * (a.act_stride / 128) * 4);
    g.T = a.T; g.K = a.K; g.E = a.E; g.by_token = 0;
    g.ncol_r = a.I; g.ncol_s = a.has_shared ? a.Is : g.ncol_r;
    g.recs = a.passes; g.npass = a.pass_count;
    g.y = a.y; g.y_ld = a.H;
    // row groups of 4 blocks of 128 rows when H allows, else of 2 (H % 256
    // == 0).  Q8_0 down takes groups of 2 whatever H: twice the items, so the
    // last round of the persistent grid leaves less idle (C5: 1525 -> 1503 us
    // per batch); for the K-quant down formats the groups of 4 measured
    // faster (the Q4_K / Q6_K layer at 512 tokens: 1400 against 1404 us).
    const int nsub = a.H % (4 * GM_ROWS) == 0 && a.dt != Q8_0 ? 4 : 2;
    g.nrb_r = g.nrb_s = a.H / (nsub * GM_ROWS);
    return launch_split(a.pass_m, 1, nsub, a.dt, a.sdt, a.has_shared, g, a.n_wg, s);
}

int launch_prefill_combine(const PrefillArgs& a, hipStream_t s) {
    hipLaunchKernelGGL(k_pf_combine, dim3((a.H / 4 + 255) / 256, a.T), dim3(256), 0, s, a);
    return (int)hipGetLastError();
}

}  // namespace wm
