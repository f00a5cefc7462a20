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
//   k_pf_group     counting sort of the pairs by expert
//   k_pf_gateup    per (expert, 64 rows): gate and up on bf16 MFMA
//                  (v_mfma_f32_16x16x32_bf16, one Q8_0 block per MFMA: the
//                  int8 weights and the bf16 inputs are exact in bf16, the
//                  block's fp16 scale multiplies the fp32 partial), SwiGLU
//   k_pf_down      per (expert, 64 rows of H): down projection, the fp32
//                  SwiGLU output split into bf16 hi + lo (two MFMAs)
//   k_pf_combine   per token: sum_k w_k y_k in k order + gate * y_shared
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/winmoe_hip.h"
#include "wm_device.h"
#include "wm_format.h"
#include "wm_prefill.h"
#include "wm_wave.h"

namespace wm {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

WM_DEV float bf16f(uint16_t b) { return __builtin_bit_cast(float, (uint32_t)b << 16); }

WM_DEV int pair_token(int p, int T, int K) { return p < T * K ? p / K : p - T * K; }

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

// One workgroup: pairs grouped by expert (order inside an expert is free:
// every pair's output row is computed independently of the others).
__global__ __launch_bounds__(1024) void k_pf_group(const int32_t* __restrict__ ids, int T, int K, int E, int has_shared,
                                                   int32_t* __restrict__ offsets, int32_t* __restrict__ sorted) {
    __shared__ int cnt[1024];
    __shared__ int s_total;
    const int tid = threadIdx.x, P = T * K;
    for (int e = tid; e < E; e += 1024) cnt[e] = 0;
    __syncthreads();
    for (int p = tid; p < P; p += 1024) {
        const int e = ids[p];
        if (e >= 0 && e < E) atomicAdd(&cnt[e], 1);
    }
    __syncthreads();
    if (tid == 0) {
        int run = 0;
        for (int e = 0; e < E; e++) {
            const int c = cnt[e];
            cnt[e] = run;
            offsets[e] = run;
            run += c;
        }
        offsets[E] = run;
        offsets[E + 1] = run + (has_shared ? T : 0);
        s_total = run;
    }
    __syncthreads();
    for (int p = tid; p < P; p += 1024) {
        const int e = ids[p];
        if (e >= 0 && e < E) sorted[atomicAdd(&cnt[e], 1)] = p;
    }
    if (has_shared)
        for (int t = tid; t < T; t += 1024) sorted[s_total + t] = P + t;
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

// ------------------------------------------------------------------ grouped expert GEMMs (Q8_0)

constexpr int PG_N = 64;        // matrix rows per item (16 per wave)
constexpr int PG_M = 64;        // pairs per pass (4 MFMA row tiles)
constexpr int PG_SLOT = 160;    // LDS bytes per row chunk: 4 blocks (136 B) + alignment shift, whole granules
constexpr int PG_XLD = 136;     // LDS row of an activation chunk, bf16 elements (128 + 8 pad)

// 8 bytes at an arbitrary LDS byte offset.
WM_DEV void lds_u64u(const uint8_t* base, uint32_t off, uint32_t& lo, uint32_t& hi) {
    const uint32_t* p = (const uint32_t*)(base + (off & ~3u));
    const uint32_t s = off & 3u;
    const uint32_t w0 = p[0], w1 = p[1], w2 = p[2];
    lo = alignbyte(w1, w0, s);
    hi = alignbyte(w2, w1, s);
}

// 8 signed bytes -> 8 bf16 (exact).
WM_DEV bf16x8 q8_bf16x8(uint32_t lo, uint32_t hi) {
    bf16x8 r;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        r[j] = (__bf16)(float)(int8_t)(lo >> (8 * j));
        r[4 + j] = (__bf16)(float)(int8_t)(hi >> (8 * j));
    }
    return r;
}

// Address of the 16-byte granule j of the 4-block chunk kc of row `row` of a
// Q8_0 matrix, clamped to the chunk's last granule (no read past the chunk).
WM_DEV const u32x4* chunk_granule(const uint8_t* W, int64_t row_bytes, int row, int kc, int j) {
    const uintptr_t start = (uintptr_t)(W + (int64_t)row * row_bytes + (int64_t)kc * 136);
    const uintptr_t A = start & ~(uintptr_t)15;
    const int nch = (int)(((start - A) + 136 + 15) >> 4);
    return (const u32x4*)(A + 16 * (uintptr_t)min(j, nch - 1));
}
WM_DEV uint32_t chunk_shift(const uint8_t* W, int64_t row_bytes, int row, int kc) {
    return (uint32_t)(((uintptr_t)(W + (int64_t)row * row_bytes + (int64_t)kc * 136)) & 15u);
}

// Gate and up of one expert for rows [n0, n0 + 64) and all of its pairs:
// act[pair][row] = silu(g) * u.
__global__ __launch_bounds__(256) void k_pf_gateup(PrefillArgs a) {
    __shared__ __attribute__((aligned(16))) uint8_t wl[2 * PG_N * PG_SLOT];
    __shared__ __attribute__((aligned(16))) uint16_t xl[PG_M * PG_XLD];
    const int eg = blockIdx.y;
    const bool shared = eg == a.E;
    const int rows = shared ? a.Is : a.I;
    const int n0 = blockIdx.x * PG_N;
    const int p0 = a.offsets[eg], np = a.offsets[eg + 1] - p0;
    if (n0 >= rows || np <= 0) return;
    const uint8_t* Wg = shared ? a.sh_gate : a.gate + (int64_t)eg * a.gstride;
    const uint8_t* Wu = shared ? a.sh_up : a.up + (int64_t)eg * a.ustride;
    const int H = a.H;
    const int64_t row_bytes = (int64_t)(H / 32) * 34;
    const int nkc = H / 128;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, g = lane >> 4, c = lane & 15;
    const int rl = 16 * wave + c;                       // this lane's B row within the item
    const f32x4 zero = {0.0f, 0.0f, 0.0f, 0.0f};

    for (int mp = 0; mp < np; mp += PG_M) {
        const int mn = min(PG_M, np - mp);
        f32x4 acc[4][2];
#pragma unroll
        for (int mt = 0; mt < 4; mt++) acc[mt][0] = acc[mt][1] = zero;
        u32x4 rw[5], rx[4];
        // chunk loader: weights 2 x 64 rows x 10 granules, activations mn x 16 granules
        auto load = [&](int kc) {
#pragma unroll
            for (int q = 0; q < 5; q++) {
                const int i = tid + 256 * q;
                const int mat = i / (PG_N * 10), r = (i % (PG_N * 10)) / 10, j = i % 10;
                rw[q] = (u32x4){0u, 0u, 0u, 0u};
                if (i < 2 * PG_N * 10 && n0 + r < rows) rw[q] = *chunk_granule(mat ? Wu : Wg, row_bytes, n0 + r, kc, j);
            }
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const int i = tid + 256 * q, m = i >> 4, j = i & 15;
                rx[q] = (u32x4){0u, 0u, 0u, 0u};
                if (m < mn) {
                    const int tok = pair_token(a.sorted[p0 + mp + m], a.T, a.K);
                    rx[q] = *(const u32x4*)(a.x + (int64_t)tok * H + (int64_t)kc * 128 + 8 * j);
                }
            }
        };
        auto store = [&]() {
#pragma unroll
            for (int q = 0; q < 5; q++) {
                const int i = tid + 256 * q;
                if (i < 2 * PG_N * 10) *(u32x4*)(wl + 16 * i) = rw[q];
            }
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const int i = tid + 256 * q, m = i >> 4, j = i & 15;
                *(u32x4*)(xl + m * PG_XLD + 8 * j) = rx[q];
            }
        };
        load(0);
        store();
        __syncthreads();
        for (int kc = 0; kc < nkc; kc++) {
            if (kc + 1 < nkc) load(kc + 1);
#pragma unroll
            for (int mat = 0; mat < 2; mat++) {
                const uint32_t shift = n0 + rl < rows ? chunk_shift(mat ? Wu : Wg, row_bytes, n0 + rl, kc) : 0u;
                const uint8_t* slot = wl + (mat * PG_N + rl) * PG_SLOT;
#pragma unroll
                for (int b = 0; b < 4; b++) {
                    const uint32_t off = shift + 34 * b;
                    const float d = h2f(*(const uint16_t*)(slot + off));
                    uint32_t qlo, qhi;
                    lds_u64u(slot, off + 2 + 8 * g, qlo, qhi);
                    const bf16x8 B = q8_bf16x8(qlo, qhi);
#pragma unroll
                    for (int mt = 0; mt < 4; mt++) {
                        if (16 * mt < mn) {
                            const bf16x8 A = *(const bf16x8*)(xl + (16 * mt + c) * PG_XLD + 32 * b + 8 * g);
                            const f32x4 P = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A, B, zero, 0, 0, 0);
#pragma unroll
                            for (int i = 0; i < 4; i++) acc[mt][mat][i] = fmaf(d, P[i], acc[mt][mat][i]);
                        }
                    }
                }
            }
            __syncthreads();
            if (kc + 1 < nkc) {
                store();
                __syncthreads();
            }
        }
        // lane holds C[4g + i][c] of each row tile: pair 16mt + 4g + i, row n0 + rl
        const int row = n0 + rl;
#pragma unroll
        for (int mt = 0; mt < 4; mt++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int m = 16 * mt + 4 * g + i;
                if (m < mn && row < rows) {
                    const int pair = a.sorted[p0 + mp + m];
                    a.act[(int64_t)pair * a.act_stride + row] = silu_mul(acc[mt][0][i], acc[mt][1][i]);
                }
            }
        __syncthreads();
    }
}

// Down projection of one expert for output rows [n0, n0 + 64) and all of its
// pairs: y[pair][row] = W_down[row] . act[pair], the activation as bf16 hi + lo.
__global__ __launch_bounds__(256) void k_pf_down(PrefillArgs a) {
    __shared__ __attribute__((aligned(16))) uint8_t wl[PG_N * PG_SLOT];
    __shared__ __attribute__((aligned(16))) uint16_t ahl[PG_M * PG_XLD];
    __shared__ __attribute__((aligned(16))) uint16_t all_[PG_M * PG_XLD];
    const int eg = blockIdx.y;
    const bool shared = eg == a.E;
    const int Ie = shared ? a.Is : a.I;
    const int rows = a.H;
    const int n0 = blockIdx.x * PG_N;
    const int p0 = a.offsets[eg], np = a.offsets[eg + 1] - p0;
    if (n0 >= rows || np <= 0) return;
    const uint8_t* W = shared ? a.sh_down : a.down + (int64_t)eg * a.dstride;
    const int64_t row_bytes = (int64_t)(Ie / 32) * 34;
    const int nkc = Ie / 128;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, g = lane >> 4, c = lane & 15;
    const int rl = 16 * wave + c;
    const f32x4 zero = {0.0f, 0.0f, 0.0f, 0.0f};

    for (int mp = 0; mp < np; mp += PG_M) {
        const int mn = min(PG_M, np - mp);
        f32x4 acc[4];
#pragma unroll
        for (int mt = 0; mt < 4; mt++) acc[mt] = zero;
        u32x4 rw[3];
        f32x4 ra[8];
        auto load = [&](int kc) {
#pragma unroll
            for (int q = 0; q < 3; q++) {
                const int i = tid + 256 * q, r = i / 10, j = i % 10;
                rw[q] = (u32x4){0u, 0u, 0u, 0u};
                if (i < PG_N * 10 && n0 + r < rows) rw[q] = *chunk_granule(W, row_bytes, n0 + r, kc, j);
            }
#pragma unroll
            for (int q = 0; q < 8; q++) {
                const int i = tid + 256 * q, m = i >> 5, j = i & 31;     // 32 float4 per pair row chunk
                ra[q] = zero;
                if (m < mn) {
                    const int pair = a.sorted[p0 + mp + m];
                    ra[q] = *(const f32x4*)(a.act + (int64_t)pair * a.act_stride + (int64_t)kc * 128 + 4 * j);
                }
            }
        };
        auto store = [&]() {
#pragma unroll
            for (int q = 0; q < 3; q++) {
                const int i = tid + 256 * q;
                if (i < PG_N * 10) *(u32x4*)(wl + 16 * i) = rw[q];
            }
#pragma unroll
            for (int q = 0; q < 8; q++) {
                const int i = tid + 256 * q, m = i >> 5, j = i & 31;
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const __bf16 h = (__bf16)ra[q][e];
                    const __bf16 lo = (__bf16)(ra[q][e] - (float)h);
                    ahl[m * PG_XLD + 4 * j + e] = __builtin_bit_cast(uint16_t, h);
                    all_[m * PG_XLD + 4 * j + e] = __builtin_bit_cast(uint16_t, lo);
                }
            }
        };
        load(0);
        store();
        __syncthreads();
        for (int kc = 0; kc < nkc; kc++) {
            if (kc + 1 < nkc) load(kc + 1);
            const uint32_t shift = n0 + rl < rows ? chunk_shift(W, row_bytes, n0 + rl, kc) : 0u;
            const uint8_t* slot = wl + rl * PG_SLOT;
#pragma unroll
            for (int b = 0; b < 4; b++) {
                const uint32_t off = shift + 34 * b;
                const float d = h2f(*(const uint16_t*)(slot + off));
                uint32_t qlo, qhi;
                lds_u64u(slot, off + 2 + 8 * g, qlo, qhi);
                const bf16x8 B = q8_bf16x8(qlo, qhi);
#pragma unroll
                for (int mt = 0; mt < 4; mt++) {
                    if (16 * mt < mn) {
                        const bf16x8 Ah = *(const bf16x8*)(ahl + (16 * mt + c) * PG_XLD + 32 * b + 8 * g);
                        const bf16x8 Al = *(const bf16x8*)(all_ + (16 * mt + c) * PG_XLD + 32 * b + 8 * g);
                        f32x4 P = __builtin_amdgcn_mfma_f32_16x16x32_bf16(Ah, B, zero, 0, 0, 0);
                        P = __builtin_amdgcn_mfma_f32_16x16x32_bf16(Al, B, P, 0, 0, 0);
#pragma unroll
                        for (int i = 0; i < 4; i++) acc[mt][i] = fmaf(d, P[i], acc[mt][i]);
                    }
                }
            }
            __syncthreads();
            if (kc + 1 < nkc) {
                store();
                __syncthreads();
            }
        }
        const int row = n0 + rl;
#pragma unroll
        for (int mt = 0; mt < 4; mt++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int m = 16 * mt + 4 * g + i;
                if (m < mn && row < rows) {
                    const int pair = a.sorted[p0 + mp + m];
                    a.y[(int64_t)pair * rows + row] = acc[mt][i];
                }
            }
        __syncthreads();
    }
}

// out[t][h] = sum_k w[t][k] y[t*K + k][h] (k order, invalid ids skipped) + gate(t) * y_shared[t][h].
__global__ __launch_bounds__(256) void k_pf_combine(PrefillArgs a) {
    const int t = blockIdx.y, h = blockIdx.x * 256 + threadIdx.x;
    if (h >= a.H) return;
    float acc = 0.0f;
    for (int k = 0; k < a.K; k++) {
        const int e = a.ids[(int64_t)t * a.K + k];
        if (e < 0 || e >= a.E) continue;
        acc = fmaf(a.w[(int64_t)t * a.K + k], a.y[((int64_t)t * a.K + k) * a.H + h], acc);
    }
    if (a.has_shared) {
        float ys = a.y[((int64_t)a.T * a.K + t) * a.H + h];
        if (a.sh_gate_inp) ys *= a.sg[t];
        acc = acc + ys;
    }
    a.out[(int64_t)t * a.H + h] = acc;
}

// ------------------------------------------------------------------ launcher

int launch_prefill_route(const PrefillArgs& a, const int32_t* forced_ids, const float* forced_w, hipStream_t s) {
    const int P = a.T * a.K;
    if (forced_ids) {
        hipLaunchKernelGGL(k_pf_forced, dim3((P + 255) / 256), dim3(256), 0, s, forced_ids, forced_w, P, a.E, a.ids, a.w,
                           a.hits, a.status);
    } else {
        hipLaunchKernelGGL(k_pf_router, dim3((a.T + PR_T - 1) / PR_T, (a.E + PR_E - 1) / PR_E), dim3(256), 0, s, a.x,
                           a.router, a.H, a.T, a.E, a.logits);
        hipLaunchKernelGGL(k_pf_topk, dim3((a.T + WAVES - 1) / WAVES), dim3(256), 0, s, a.logits, a.T, a.E, a.K, a.ids,
                           a.w, a.hits, a.status);
    }
    hipLaunchKernelGGL(k_pf_group, dim3(1), dim3(1024), 0, s, a.ids, a.T, a.K, a.E, a.has_shared, a.offsets, a.sorted);
    if (a.has_shared && a.sh_gate_inp)
        hipLaunchKernelGGL(k_pf_shgate, dim3(a.T), dim3(256), 0, s, a.x, a.sh_gate_inp, a.H, a.sg);
    return (int)hipGetLastError();
}

int launch_prefill_gateup(const PrefillArgs& a, hipStream_t s) {
    const int ng = a.E + (a.has_shared ? 1 : 0);
    const int Imax = a.has_shared && a.Is > a.I ? a.Is : a.I;
    hipLaunchKernelGGL(k_pf_gateup, dim3((Imax + PG_N - 1) / PG_N, ng), dim3(256), 0, s, a);
    return (int)hipGetLastError();
}

int launch_prefill_down(const PrefillArgs& a, hipStream_t s) {
    const int ng = a.E + (a.has_shared ? 1 : 0);
    hipLaunchKernelGGL(k_pf_down, dim3((a.H + PG_N - 1) / PG_N, ng), dim3(256), 0, s, a);
    return (int)hipGetLastError();
}

int launch_prefill_combine(const PrefillArgs& a, hipStream_t s) {
    hipLaunchKernelGGL(k_pf_combine, dim3((a.H + 255) / 256, a.T), dim3(256), 0, s, a);
    return (int)hipGetLastError();
}

}  // namespace wm
