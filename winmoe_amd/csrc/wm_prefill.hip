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
//   k_pf_group     counting sort of the pairs by expert; passes of <= 32
//                  pairs of one expert
//   k_pf_xpack     x as fp16 times a power of two per token
//   k_pf_gemm<2,1> gate and up + SwiGLU on fp16 MFMA, persistent: one
//                  workgroup per CU streams (pass, 128-row block) items
//                  through an LDS-DMA ring; the SwiGLU output is stored as
//                  fp16 hi + lo times a power of two per (pair, 128 rows)
//   k_pf_gemm<1,2> down projection of the same form (hi and lo: two MFMAs)
//   k_pf_combine   per token: sum_k w_k y_k in k order + gate * y_shared
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "../../include/winmoe_hip.h"
#include "wm_device.h"
#include "wm_format.h"
#include "wm_prefill.h"
#include "wm_wave.h"

namespace wm {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

WM_DEV float bf16f(uint16_t b) { return __builtin_bit_cast(float, (uint32_t)b << 16); }

WM_DEV int pair_token(int p, int T, int K) { return p < T * K ? p / K : p - T * K; }

// Exponent e with m * 2^-e in [2^14, 2^15) for a finite m > 0 (clamped to
// e >= -126 so that 2^e and 2^-e are normal floats); 0 otherwise.  Values of
// a group scaled by 2^-e fit fp16 with its full 11-bit precision down to
// 2^-29 of the group maximum.
WM_DEV int pf_exp(float m) {
    if (!(m > 0.0f) || !(m <= 3.402823466e38f)) return 0;
    int E;
    frexpf(m, &E);                 // m in [2^(E-1), 2^E)
    return max(E - 15, -126);
}

// Expert passes: a pass is up to GM_M pairs of one expert, described by a
// record of GM_REC ints: expert (E = shared), pair count, 0, 0, GM_M pair ids
// (positions past the count repeat the last id), then the x scale exponents
// of the pairs' tokens, 4 signed bytes per int.
constexpr int GM_M = 32;
constexpr int GM_REC = 64;

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

// One workgroup: pairs grouped by expert (order inside an expert is free:
// every pair's output row is computed independently of the others), then
// cut into pass records: routed passes first, in expert order, then the
// shared expert's; pass_count = {routed passes, shared passes}.  A record
// also carries the x scale of each pair's token.
__global__ __launch_bounds__(1024) void k_pf_group(const int32_t* __restrict__ ids, int T, int K, int E, int has_shared,
                                                   int32_t* __restrict__ offsets, int32_t* __restrict__ sorted,
                                                   int32_t* __restrict__ passes, int32_t* __restrict__ pass_count,
                                                   const int32_t* __restrict__ xexp) {
    __shared__ int cnt[1025];
    __shared__ int off[1026];
    __shared__ int pbase[1026];
    __shared__ int wsum[32];
    const int tid = threadIdx.x, P = T * K, G = E + 1;      // group E: the shared expert (empty without one)
    for (int e = tid; e < E; e += 1024) cnt[e] = 0;
    if (tid == 0) cnt[E] = has_shared ? T : 0;
    __syncthreads();
    for (int p = tid; p < P; p += 1024) {
        const int e = ids[p];
        if (e >= 0 && e < E) atomicAdd(&cnt[e], 1);
    }
    __syncthreads();
    // pair offsets and pass bases of the groups, 1024 groups per round
    int2 carry = make_int2(0, 0);
    for (int base = 0; base < G; base += 1024) {
        const int e = base + tid;
        const int n = e < G ? cnt[e] : 0;
        int2 tot;
        const int2 ex = block_excl_scan2(make_int2(n, (n + GM_M - 1) / GM_M), wsum, &tot);
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
    for (int p = tid; p < P; p += 1024) {
        const int e = ids[p];
        if (e >= 0 && e < E) sorted[atomicAdd(&cnt[e], 1)] = p;
    }
    if (has_shared)
        for (int t = tid; t < T; t += 1024) sorted[off[E] + t] = P + t;
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
        const int e = lo, first = off[e] + (q - pbase[e]) * GM_M;
        const int mn = min(GM_M, off[e + 1] - first);
        int32_t* rec = passes + (int64_t)q * GM_REC;
        rec[0] = e;
        rec[1] = mn;
        rec[2] = 0;
        rec[3] = 0;
        int prs[GM_M];
#pragma unroll
        for (int m = 0; m < GM_M; m++) prs[m] = sorted[first + min(m, mn - 1)];
#pragma unroll
        for (int m4 = 0; m4 < GM_M / 4; m4++) {
            uint32_t ex = 0;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int pr = prs[4 * m4 + j];
                rec[4 + 4 * m4 + j] = pr;
                ex |= (uint32_t)(xexp[pair_token(pr, T, K)] & 0xFF) << (8 * j);
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

// ------------------------------------------------------------------ grouped expert GEMMs (Q8_0, fp16 MFMA)
//
// One workgroup per CU works through a static list of items: item j of a
// launch is (pass, block of 128 matrix rows), and workgroup b takes items
// b, b + grid, b + 2 grid, ...  For each item it streams the block's rows (of
// gate and up, or of down) through an S-stage LDS ring, 128 columns = 4 Q8_0
// blocks per stage, filled by global_load_lds:
//   * weights: each row's 136-byte stage chunk as 9 granules of 16 B from
//     the 16-byte boundary at or before it (the chunk starts 0 or 8 bytes
//     into its first granule; the 9 granules never leave the row when the
//     column count is a multiple of 256);
//   * activations: the pass's 32 rows x 128 fp16, rows 272 bytes apart (a
//     pad granule each), so the MFMA operand reads of 16 rows hit 16
//     different 16-byte slots of a 256-byte bank cycle;
//   * the activations' power-of-two scales of the stage (one dword each).
// The ring runs across item boundaries: the next item's first stages are in
// flight while the current one finishes.  Waves 0-7 issue the loads and do
// the maths (16 rows each); wave 8 only writes results, because vector
// stores count in vmcnt: issued by the compute waves they would hold up the
// "stage landed" waits.
//
// Per (row, block) the 32 int8 weights become fp16 exactly (byte ^ 0x80
// under the exponent byte 0x64 is 1152 + q; minus 1152), so
// v_mfma_f32_16x16x32_f16 gives the block's dot product with the scaled fp16
// activations; the block's fp16 scale d multiplies it, the activation scale
// multiplies the stage's sum.

constexpr int GM_ROWS = 128;          // matrix rows per item
constexpr int GM_RSLOT = 144;         // LDS bytes of a row's stage chunk (9 granules)
constexpr int GM_CW = 8;              // compute waves
constexpr int GM_THREADS = 64 * (GM_CW + 1);
constexpr int GM_DESC = 8;            // pass records held in LDS
constexpr int GM_ALD = 272;           // LDS bytes per activation row of a stage (256 + one pad granule)
constexpr int GM_APART = 9 * 1024;    // one activation array of a stage: 32 rows x 272 B in 9 DMA units
constexpr int GM_A16 = 5;             // DMA units holding rows 0-15 (16 x 272 B)

template <int NMAT, int AHL, int NSUB> struct GmGeo {
    static constexpr int S = NMAT == 2 ? 3 : 5;                        // weight ring stages
    static constexpr int W_BYTES = NMAT * GM_ROWS * GM_RSLOT;
    static constexpr int A_BYTES = AHL * GM_APART;
    static constexpr int A_SLOT = A_BYTES + 256;                        // + 64 scale dwords
    // activation slots: a slot is refilled S - 1 stages after its last use
    static constexpr int NAS = (S - 1 + NSUB - 1) / NSUB + 1;
    static constexpr int ABASE = S * W_BYTES;
    static constexpr int DESC = ABASE + NAS * A_SLOT;
    static constexpr int RED = DESC + GM_DESC * GM_REC * 4;             // [32 pairs][8 waves] maxima
    static constexpr int STG = RED + (NMAT == 2 ? GM_M * GM_CW * 4 : 0);
    // staging: gate/up 32 pairs x 128 rows of fp16 hi and lo + 32 scales;
    // down 16 pairs x 128 rows of fp32 (the halves of a pass pass through in turn)
    static constexpr int LDS = STG + (NMAT == 2 ? GM_M * GM_ROWS * 4 + GM_M * 4 : 16 * GM_ROWS * 4);
    static constexpr int NW = NMAT * GM_ROWS * 9 / 64;                // weight DMA instructions per stage
    static constexpr int NWT = (NW + GM_CW - 1) / GM_CW;
    static constexpr int NA = AHL * 9;                                // activation DMA instructions per column step
    static constexpr int NAT = (NA + GM_CW - 1) / GM_CW;
    static_assert(NAS * NSUB >= NSUB + S - 1, "activation slot reuse");
};
static_assert(GmGeo<2, 1, 1>::LDS <= 163840 && GmGeo<1, 2, 4>::LDS <= 163840 && GmGeo<1, 2, 2>::LDS <= 163840,
              "LDS per workgroup");
static_assert(4 + GM_M + GM_M / 4 <= GM_REC, "pass record");

struct PfGemm {
    const uint8_t* w0;                 // routed matrices (gate, up) or (down, -): expert e at + e * st
    const uint8_t* w1;
    int64_t st0, st1;
    const uint8_t* s0;                 // shared-expert matrices
    const uint8_t* s1;
    int64_t rb_r, rb_s;                // bytes per matrix row: routed, shared
    int32_t mb_r, mb_s;                // bytes per matrix: routed, shared
    const uint16_t* a_hi;              // activations, fp16 bits [rows][a_ld]
    const uint16_t* a_lo;
    int64_t a_ld;
    const float* a_sc;                 // activation scales [rows][sc_ld], one per 128 columns
    int64_t sc_ld;
    int32_t a_bytes, sc_bytes;         // sizes of the activation and scale arrays
    int32_t T, K, E, by_token;         // activation row: token of the pair (1) or the pair (0)
    int32_t nrb_r, nrb_s, nkc_r, nkc_s;    // row groups per pass and column steps per item: routed, shared
    const int32_t* recs;
    const int32_t* npass;              // {routed passes, shared passes}
    uint16_t* o_hi;                    // gate/up: SwiGLU output hi / lo [pair][o_ld], scales [pair][osc_ld]
    uint16_t* o_lo;
    float* o_sc;
    int64_t o_ld, osc_ld;
    float* y;                          // down: [pair][y_ld]
    int64_t y_ld;
};

typedef __attribute__((address_space(3))) void lds_void;

// Raw buffer resource over [p, p + bytes) (gfx9 word 3: 32-bit data format).
WM_DEV __amdgpu_buffer_rsrc_t gm_rsrc(const void* p, int bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, bytes, 0x00020000);
}

// All waves of the workgroup meet; this wave's LDS accesses are complete.
// (No fence: a fence would also wait for the ring's loads in flight.)
WM_DEV void gm_bar() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xC07F);          // lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// s_waitcnt vmcnt(n) for a wave-uniform n (values past 15 wait for all).
WM_DEV void gm_wait_vm(int n) {
    switch (n) {
#define WM_GM_CASE(k) \
    case k: WM_WAIT_VMCNT(k); break;
        WM_GM_CASE(1) WM_GM_CASE(2) WM_GM_CASE(3) WM_GM_CASE(4) WM_GM_CASE(5) WM_GM_CASE(6) WM_GM_CASE(7)
        WM_GM_CASE(8) WM_GM_CASE(9) WM_GM_CASE(10) WM_GM_CASE(11) WM_GM_CASE(12) WM_GM_CASE(13) WM_GM_CASE(14)
        WM_GM_CASE(15)
#undef WM_GM_CASE
        default: WM_WAIT_VMCNT(0); break;
    }
}

// The 8 int8 weights k = 8g .. 8g+7 of block B of a row chunk as fp16
// (exact).  rowp: the chunk's first byte in LDS (8-byte aligned).
template <int B> WM_DEV f16x8 q8_f16x8(const uint8_t* rowp, int g) {
    constexpr int off = 34 * B + 2;
    const uint32_t* p = (const uint32_t*)(rowp + (off & ~3) + 8 * g);
    const uint32_t K = 0x64646464u, X = 0x80808080u;
    uint32_t h0, h1, h2, h3;
    if constexpr ((off & 3) == 0) {
        const uint32_t d0 = p[0] ^ X, d1 = p[1] ^ X;
        h0 = __builtin_amdgcn_perm(K, d0, 0x04010400u);
        h1 = __builtin_amdgcn_perm(K, d0, 0x04030402u);
        h2 = __builtin_amdgcn_perm(K, d1, 0x04010400u);
        h3 = __builtin_amdgcn_perm(K, d1, 0x04030402u);
    } else {
        const uint32_t d0 = p[0] ^ X, d1 = p[1] ^ X, d2 = p[2] ^ X;
        h0 = __builtin_amdgcn_perm(K, d0, 0x04030402u);
        h1 = __builtin_amdgcn_perm(K, d1, 0x04010400u);
        h2 = __builtin_amdgcn_perm(K, d1, 0x04030402u);
        h3 = __builtin_amdgcn_perm(K, d2, 0x04010400u);
    }
    const f16x2 bias = {(_Float16)1152.0f, (_Float16)1152.0f};
    const f16x2 v0 = __builtin_bit_cast(f16x2, h0) - bias, v1 = __builtin_bit_cast(f16x2, h1) - bias;
    const f16x2 v2 = __builtin_bit_cast(f16x2, h2) - bias, v3 = __builtin_bit_cast(f16x2, h3) - bias;
    return (f16x8){v0[0], v0[1], v1[0], v1[1], v2[0], v2[1], v3[0], v3[1]};
}

// NMAT = 2: gate and up of a pass (activations: the tokens' x, AHL = 1),
// SwiGLU epilogue.  NMAT = 1: down (activations: the pairs' SwiGLU outputs as
// hi + lo, AHL = 2), fp32 epilogue.  An item covers NSUB blocks of 128 rows:
// each column step loads the activations once and the NSUB weight blocks in
// turn (one ring stage each).
template <int NMAT, int AHL, int NSUB>
__global__ __launch_bounds__(GM_THREADS) void k_pf_gemm(PfGemm a) {
#if defined(__HIP_DEVICE_COMPILE__)      // the host pass only needs the launch stub (buffer resources are device types)
    typedef GmGeo<NMAT, AHL, NSUB> G;
    constexpr int S = G::S;
    extern __shared__ __attribute__((aligned(16))) uint8_t gsm[];
    // the wave index is uniform: readfirstlane lets the compiler keep what depends on it in SGPRs
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), g = lane >> 4, c = lane & 15;
    const bool cw = wave < GM_CW;
    const int n_rp = a.npass[0], n_sp = a.npass[1];
    const int n_r = n_rp * a.nrb_r, n_items = n_r + n_sp * a.nrb_s;
    if ((int)blockIdx.x >= n_items) return;

    // item i of this workgroup: pass, row group, column steps
    auto item = [&](int i, int& pass, int& rg, int& nkc) __attribute__((always_inline)) -> bool {
        const int j = (int)blockIdx.x + i * (int)gridDim.x;
        if (j >= n_items) return false;
        if (j < n_r) {
            pass = j / a.nrb_r;
            rg = j - pass * a.nrb_r;
            nkc = a.nkc_r;
        } else {
            const int q = (j - n_r) / a.nrb_s;
            rg = (j - n_r) - q * a.nrb_s;
            pass = n_rp + q;
            nkc = a.nkc_s;
        }
        return true;
    };
    const int32_t* desc = (const int32_t*)(gsm + G::DESC);
    auto desc_dma = [&](int i, int pass) __attribute__((always_inline)) {
        __builtin_amdgcn_global_load_lds((const void*)(a.recs + (int64_t)pass * GM_REC + lane),
                                         (lds_void*)(gsm + G::DESC + (i % GM_DESC) * GM_REC * 4), 4, 0, 0);
    };

    // Down (NMAT = 1) activations carry a scale per (row, column step);
    // gate/up activations (x) one per token, applied in the epilogue.
    constexpr bool SCALED = NMAT == 1;
    // DMA instructions of this wave per weight stage, and per activation
    // column step (activations + scales; a pass of at most 16 pairs loads only
    // the first 5 units of each activation array: rows 0-15)
    int n_wt = 0, n_a = SCALED && wave == GM_CW - 1 ? 1 : 0;
#pragma unroll
    for (int t = 0; t < G::NWT; t++)
        if (wave + GM_CW * t < G::NW) n_wt++;
    int n_a16 = n_a;
#pragma unroll
    for (int t = 0; t < G::NAT; t++) {
        const int u = wave + GM_CW * t;
        if (u < G::NA) n_a++;
        if (u < G::NA && u % 9 < GM_A16) n_a16++;
    }
    const int m_s = lane & 31;        // this lane's pass row of the scale load

    // issue pointer: item ii, stage ist = NSUB * column step + row block; the
    // item's sources as uniform bases plus this lane's 32-bit byte offsets.
    // Weight instruction t of this wave covers granules p = 64 (wave + 8 t) +
    // lane of a stage: matrix p / (128 * 9) (uniform per instruction), row
    // (p % 1152) / 9, granule p % 9.
    int ii = 0, ist = 0, ip = 0, irg = 0, inkc = 0;
    bool iok = item(0, ip, irg, inkc);
    // Sources are bounds-checked buffer resources (a read past the
    // resource's size returns zeros instead of touching memory).
    const __amdgpu_buffer_rsrc_t rA0 = gm_rsrc(a.a_hi, a.a_bytes), rA1 = gm_rsrc(a.a_lo, a.a_bytes);
    const __amdgpu_buffer_rsrc_t rS = gm_rsrc(a.a_sc, a.sc_bytes);
    __amdgpu_buffer_rsrc_t rW0 = rA0, rW1 = rA0;
    uint32_t iwo[G::NWT], iao[G::NAT];
    uint32_t iso = 0, irowb = 0;
    bool itwo = true;                 // the issue item's pass uses rows 16-31
    auto setup_issue = [&]() __attribute__((always_inline)) {
        const int32_t* rec = desc + (ii % GM_DESC) * GM_REC;
        itwo = __builtin_amdgcn_readfirstlane(rec[1]) > 16;
        const int ge = __builtin_amdgcn_readfirstlane(rec[0]);
        const bool shared = ip >= n_rp;
        const int mb = shared ? a.mb_s : a.mb_r;
        rW0 = gm_rsrc(shared ? a.s0 : a.w0 + (int64_t)ge * a.st0, mb);
        rW1 = NMAT == 2 ? gm_rsrc(shared ? a.s1 : a.w1 + (int64_t)ge * a.st1, mb) : rW0;
        irowb = (uint32_t)(shared ? a.rb_s : a.rb_r);
#pragma unroll
        for (int t = 0; t < G::NWT; t++) {
            const int p = 64 * (wave + GM_CW * t) + lane, rem = p % (GM_ROWS * 9), r = rem / 9;
            iwo[t] = (uint32_t)(irg * NSUB * GM_ROWS + r) * irowb + 16u * (uint32_t)(rem - 9 * r);
        }
        // activation instruction u = wave + 8 t: array u / 9, LDS granules
        // 64 (u % 9) + lane = 17 m + jj of the array (jj = 16: pad; m >= 32:
        // slack), loaded from granule min(jj, 15) of pass row min(m, 31)
#pragma unroll
        for (int t = 0; t < G::NAT; t++) {
            const int p = 64 * ((wave + GM_CW * t) % 9) + lane, m = min(p / 17, GM_M - 1), jj = min(p % 17, 15);
            const int pa = rec[4 + m], ra = a.by_token ? pair_token(pa, a.T, a.K) : pa;
            iao[t] = (uint32_t)ra * (uint32_t)a.a_ld * 2u + 16u * (uint32_t)jj;
        }
        if constexpr (SCALED) iso = ((uint32_t)rec[4 + m_s] * (uint32_t)a.sc_ld) * 4u;
    };
    int issued = 0, a_issued = 0;
    // Per-wave DMA instruction counts of the issued stages not yet consumed,
    // 4 bits each, oldest in the low bits (at most S of them), and their sum:
    // "stage landed" is vmcnt(sum minus the oldest count).
    uint32_t qpack = 0;
    int qn = 0, qsum = 0;
    // Loads of stage (ii, ist): the weight block into ring slot issued % S;
    // at a column step's first block also the activations and scales into
    // activation slot a_issued % NAS; at an item's first stage wave 6 also
    // fetches the record of the item two ahead (after the stage's loads, so
    // "stage landed" implies "record landed").
    auto issue_next = [&](auto sw_tag) __attribute__((always_inline)) {
        constexpr bool SW = decltype(sw_tag)::value;
        const int kc = ist / NSUB, sub = ist - kc * NSUB;
        if constexpr (!SW) {
            const int n = n_wt + (sub == 0 ? (itwo ? n_a : n_a16) : 0);
            qpack |= (uint32_t)n << (4 * qn);
            ++qn;
            qsum += n;
            lds8_t* dst = (lds8_t*)(gsm + (issued % S) * G::W_BYTES);
            const uint32_t soff = (((uint32_t)kc * 136u) & ~15u) + (uint32_t)(sub * GM_ROWS) * irowb;
#pragma unroll
            for (int t = 0; t < G::NWT; t++) {
                const int q = wave + GM_CW * t;
                if (q < G::NW)
                    __builtin_amdgcn_raw_ptr_buffer_load_lds(q < GM_ROWS * 9 / 64 ? rW0 : rW1, (lds_void*)(dst + 1024 * q),
                                                             16, iwo[t], soff, 0, 0);
            }
            if (sub == 0) {
                lds8_t* adst = (lds8_t*)(gsm + G::ABASE + (a_issued % G::NAS) * G::A_SLOT);
#pragma unroll
                for (int t = 0; t < G::NAT; t++) {
                    const int u = wave + GM_CW * t;
                    if (u < G::NA && (itwo || u % 9 < GM_A16))
                        __builtin_amdgcn_raw_ptr_buffer_load_lds(u >= 9 ? rA1 : rA0,
                                                                 (lds_void*)(adst + GM_APART * (u / 9) + 1024 * (u % 9)),
                                                                 16, iao[t], 256u * (uint32_t)kc, 0, 0);
                }
                if (SCALED && wave == GM_CW - 1)
                    __builtin_amdgcn_raw_ptr_buffer_load_lds(rS, (lds_void*)(adst + G::A_BYTES), 4, iso,
                                                             4u * (uint32_t)kc, 0, 0);
            }
            if (ist == 0 && wave == 6) {
                int p2, r2, n2;
                if (item(ii + 2, p2, r2, n2)) desc_dma(ii + 2, p2);
            }
        }
        ++issued;
        if (sub == 0) ++a_issued;
        if (++ist == inkc * NSUB) {
            ist = 0;
            ++ii;
            iok = item(ii, ip, irg, inkc);
            if constexpr (!SW)
                if (iok) setup_issue();
        }
    };

    f32x4 acc[NSUB][NMAT][2];
    const f32x4 zero = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int u = 0; u < NSUB; u++)
#pragma unroll
        for (int mat = 0; mat < NMAT; mat++) acc[u][mat][0] = acc[u][mat][1] = zero;

    // The sums of one stage (column step kc of a weight block) from weight
    // slot ws and activation slot as, not yet scaled; TWO: pass rows 16-31
    // are in use (one straight-line body per case, for the scheduler; the
    // row tile 16-31 sums stay zero otherwise).
    struct Sums {
        f32x4 v[NMAT][2];
    };
    auto compute = [&](int ws, int as, int kc, auto two_tag) __attribute__((always_inline)) -> Sums {
        constexpr bool TWO = decltype(two_tag)::value;
        const uint8_t* wb = gsm + ws * G::W_BYTES;
        const uint8_t* ab = gsm + G::ABASE + as * G::A_SLOT;
        const int sh8 = (kc & 1) * 8;
        Sums t;
#pragma unroll
        for (int mat = 0; mat < NMAT; mat++) t.v[mat][0] = t.v[mat][1] = zero;
#pragma unroll
        for (int b = 0; b < 4; b++) {
            f16x8 A[AHL][2];
#pragma unroll
            for (int h = 0; h < AHL; h++)
#pragma unroll
                for (int mt = 0; mt < 2; mt++)
                    A[h][mt] = *(const f16x8*)(ab + GM_APART * h + (16 * mt + c) * GM_ALD + 16 * (4 * b + g));
#pragma unroll
            for (int mat = 0; mat < NMAT; mat++) {
                const uint8_t* rowp = wb + (mat * GM_ROWS + 16 * wave + c) * GM_RSLOT + sh8;
                const float d = (float)*(const _Float16*)(rowp + 34 * b);
                f16x8 B;
                if (b == 0) B = q8_f16x8<0>(rowp, g);
                else if (b == 1) B = q8_f16x8<1>(rowp, g);
                else if (b == 2) B = q8_f16x8<2>(rowp, g);
                else B = q8_f16x8<3>(rowp, g);
#pragma unroll
                for (int mt = 0; mt < 2; mt++) {
                    if (mt == 1 && !TWO) continue;
                    f32x4 P = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[0][mt], B, zero, 0, 0, 0);
                    if constexpr (AHL == 2) P = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[AHL - 1][mt], B, P, 0, 0, 0);
#pragma unroll
                    for (int i = 0; i < 4; i++) t.v[mat][mt][i] = fmaf(d, P[i], t.v[mat][mt][i]);
                }
            }
        }
        return t;
    };
    // acc[SUB] += the stage's sums (SCALED: times the column step's
    // activation scales of the pass rows 16 mt + 4 g + i)
    auto accumulate = [&](int as, const Sums& t, auto sub_tag) __attribute__((always_inline)) {
        constexpr int SUB = decltype(sub_tag)::value;
        const f32x4* scp = (const f32x4*)(gsm + G::ABASE + as * G::A_SLOT + G::A_BYTES);
#pragma unroll
        for (int mt = 0; mt < 2; mt++) {
            const f32x4 sc = SCALED ? scp[4 * mt + g] : (f32x4){1.0f, 1.0f, 1.0f, 1.0f};
#pragma unroll
            for (int mat = 0; mat < NMAT; mat++) {
                f32x4 r = acc[SUB][mat][mt];
#pragma unroll
                for (int i = 0; i < 4; i++) r[i] = SCALED ? fmaf(sc[i], t.v[mat][mt][i], r[i]) : r[i] + t.v[mat][mt][i];
                acc[SUB][mat][mt] = r;
            }
        }
    };

    // Down: 16 pairs (one row tile) of row block rb of item i, staged, to
    // registers and from registers to HBM (wave 8).
    auto load_half = [&](u32x4(&v)[8]) __attribute__((always_inline)) {
#pragma unroll
        for (int it = 0; it < 8; it++) v[it] = *(const u32x4*)(gsm + G::STG + (2 * it + (lane >> 5)) * 512 + 16 * (lane & 31));
    };
    auto store_half = [&](int i, int rb, int half, const u32x4(&v)[8]) __attribute__((always_inline)) {
        const int32_t* rec = desc + (i % GM_DESC) * GM_REC;
        const int mn = rec[1];
#pragma unroll
        for (int it = 0; it < 8; it++) {
            const int m = 16 * half + 2 * it + (lane >> 5);
            if (m < mn)
                *(u32x4*)((uint8_t*)(a.y + (int64_t)rec[4 + m] * a.y_ld + rb * GM_ROWS) + 16 * (lane & 31)) = v[it];
        }
    };
    // Gate/up: results of item i (row block rb) from the staging area to HBM (wave 8).
    auto store_gu = [&](int i, int rb) __attribute__((always_inline)) {
        const int32_t* rec = desc + (i % GM_DESC) * GM_REC;
        const int mn = rec[1];
        const uint8_t* sh = gsm + G::STG;
        const uint8_t* sl = sh + GM_M * GM_ROWS * 2;
        const float* ss = (const float*)(sl + GM_M * GM_ROWS * 2);
#pragma unroll
        for (int it = 0; it < GM_M / 4; it++) {
            const int m = 4 * it + (lane >> 4), seg = lane & 15;
            if (m < mn) {
                const int64_t o = (int64_t)rec[4 + m] * a.o_ld + rb * GM_ROWS;
                *(u32x4*)((uint8_t*)(a.o_hi + o) + 16 * seg) = *(const u32x4*)(sh + m * 256 + 16 * seg);
                *(u32x4*)((uint8_t*)(a.o_lo + o) + 16 * seg) = *(const u32x4*)(sl + m * 256 + 16 * seg);
            }
        }
        if (lane < mn) a.o_sc[(int64_t)rec[4 + lane] * a.osc_ld + rb] = ss[lane];
    };

    // The compute waves and the store wave run the same schedule (item and
    // stage pointers, barriers) in two separately compiled copies, so that
    // neither holds the other's registers.
    auto run = [&](auto sw_tag) __attribute__((always_inline)) {
        constexpr bool SW = decltype(sw_tag)::value;
        // prologue: records of the first two items, then S - 1 stages
        if constexpr (!SW) {
            int p1, r1, n1;
            if (wave == 6) {
                desc_dma(0, ip);
                if (item(1, p1, r1, n1)) desc_dma(1, p1);
            }
            WM_WAIT_VMCNT(0);
        }
        gm_bar();
        if constexpr (!SW) setup_issue();
        for (int s = 0; s < S - 1 && iok; s++) issue_next(sw_tag);

        int ci = 0, ckc = 0, cp = 0, crg = 0, cnkc = 0, sigma = 0, a_cons = 0;
        item(0, cp, crg, cnkc);
        bool two = false, pend = false;
        int pi = 0, prb = 0;
        // one stage: wait for it, meet, refill the ring, compute
        auto stage = [&](auto sub_tag) __attribute__((always_inline)) {
            if constexpr (!SW) {
                const int oldest = (int)(qpack & 15u);
                gm_wait_vm(qsum - oldest);
                qsum -= oldest;
                qpack >>= 4;
                --qn;
            }
            gm_bar();
            if constexpr (SW) {
                if (pend) {
                    store_gu(pi, prb);
                    pend = false;
                }
            }
            if (iok) issue_next(sw_tag);
            if constexpr (!SW) {
                const int as = a_cons % G::NAS;
                const Sums t = two ? compute(sigma % S, as, ckc, std::true_type{})
                                   : compute(sigma % S, as, ckc, std::false_type{});
                accumulate(as, t, sub_tag);
            }
            ++sigma;
        };
        for (;;) {
            if (ckc == 0) two = __builtin_amdgcn_readfirstlane(desc[(ci % GM_DESC) * GM_REC + 1]) > 16;
            stage(std::integral_constant<int, 0>{});
            if constexpr (NSUB > 1) stage(std::integral_constant<int, 1>{});
            if constexpr (NSUB > 2) stage(std::integral_constant<int, 2>{});
            if constexpr (NSUB > 3) stage(std::integral_constant<int, 3>{});
            ++a_cons;
            if (ckc < cnkc - 1) {
                ++ckc;
                continue;
            }
            // item done: epilogue into the staging area
            if constexpr (NMAT == 2) {
                // this lane's pass rows are 16 mt + 4 g + i: one base per
                // array plus constant offsets
                float av[2][4];
                float* red = (float*)(gsm + G::RED);
                if constexpr (!SW) {
                    const uint32_t xw = (uint32_t)desc[(ci % GM_DESC) * GM_REC + 4 + GM_M + g];   // rows 4g..4g+3
                    const uint32_t xw1 = (uint32_t)desc[(ci % GM_DESC) * GM_REC + 4 + GM_M + 4 + g];
                    float* redp = red + 4 * g * GM_CW + wave;
#pragma unroll
                    for (int mt = 0; mt < 2; mt++)
#pragma unroll
                        for (int i = 0; i < 4; i++) {
                            const int xe = (int)(int8_t)((mt ? xw1 : xw) >> (8 * i));
                            const float xs = ldexpf(1.0f, xe);
                            const float v = silu_mul(acc[0][0][mt][i] * xs, acc[0][1][mt][i] * xs);
                            av[mt][i] = v;
                            float mx = fabsf(v);
                            mx = fmaxf(mx, dpp_f32<DPP_ROR8>(mx));
                            mx = fmaxf(mx, dpp_f32<DPP_ROR4>(mx));
                            mx = fmaxf(mx, dpp_f32<DPP_ROR2>(mx));
                            mx = fmaxf(mx, dpp_f32<DPP_ROR1>(mx));
                            if (c == 0) redp[(16 * mt + i) * GM_CW] = mx;
                        }
                }
                gm_bar();
                if constexpr (!SW) {
                    uint16_t* shp = (uint16_t*)(gsm + G::STG) + 4 * g * GM_ROWS + 16 * wave + c;
                    uint16_t* slp = shp + GM_M * GM_ROWS;
                    float* ss = (float*)(gsm + G::STG + GM_M * GM_ROWS * 4);
                    const float* redr = red + 4 * g * GM_CW;
#pragma unroll
                    for (int mt = 0; mt < 2; mt++)
#pragma unroll
                        for (int i = 0; i < 4; i++) {
                            const int o = 16 * mt + i;
                            const f32x4 r0 = *(const f32x4*)(redr + o * GM_CW), r1 = *(const f32x4*)(redr + o * GM_CW + 4);
                            const float M = fmaxf(fmaxf(fmaxf(r0[0], r0[1]), fmaxf(r0[2], r0[3])),
                                                  fmaxf(fmaxf(r1[0], r1[1]), fmaxf(r1[2], r1[3])));
                            const int e = pf_exp(M);
                            const float v = av[mt][i] * ldexpf(1.0f, -e);
                            const _Float16 hv = (_Float16)v;
                            const _Float16 lv = (_Float16)(v - (float)hv);
                            shp[o * GM_ROWS] = __builtin_bit_cast(uint16_t, hv);
                            slp[o * GM_ROWS] = __builtin_bit_cast(uint16_t, lv);
                            if (wave == 0 && c == 0) ss[4 * g + o] = ldexpf(1.0f, e);
                        }
                }
                pend = true;
                pi = ci;
                prb = crg;
            } else {
                // each row block's two row tiles pass through the staging
                // area into wave 8's registers, which it then stores
                float* sy = (float*)(gsm + G::STG) + 4 * g * GM_ROWS + 16 * wave + c;
                auto half = [&](auto u_tag, auto mt_tag) __attribute__((always_inline)) {
                    constexpr int U = decltype(u_tag)::value, MT = decltype(mt_tag)::value;
                    if constexpr (!SW) {
                        const f32x4 r = acc[U][0][MT];
#pragma unroll
                        for (int i = 0; i < 4; i++) sy[i * GM_ROWS] = r[i];
                    }
                    gm_bar();
                    u32x4 v[8];
                    if constexpr (SW) load_half(v);
                    gm_bar();
                    if constexpr (SW) store_half(ci, crg * NSUB + U, MT, v);
                };
                auto block = [&](auto u_tag) __attribute__((always_inline)) {
                    half(u_tag, std::integral_constant<int, 0>{});
                    if (two) half(u_tag, std::integral_constant<int, 1>{});
                };
                block(std::integral_constant<int, 0>{});
                if constexpr (NSUB > 1) block(std::integral_constant<int, 1>{});
                if constexpr (NSUB > 2) block(std::integral_constant<int, 2>{});
                if constexpr (NSUB > 3) block(std::integral_constant<int, 3>{});
            }
            if constexpr (!SW) {
#pragma unroll
                for (int u = 0; u < NSUB; u++)
#pragma unroll
                    for (int mat = 0; mat < NMAT; mat++) acc[u][mat][0] = acc[u][mat][1] = zero;
            }
            ckc = 0;
            ++ci;
            if (!item(ci, cp, crg, cnkc)) break;
        }
        gm_bar();
        if constexpr (SW)
            if (pend) store_gu(pi, prb);
    };
    if (cw) run(std::false_type{});
    else run(std::true_type{});
#endif
}

template __global__ void k_pf_gemm<2, 1, 1>(PfGemm);
template __global__ void k_pf_gemm<1, 2, 4>(PfGemm);
template __global__ void k_pf_gemm<1, 2, 2>(PfGemm);


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
        hipLaunchKernelGGL(k_pf_router, dim3((a.T + PR_T - 1) / PR_T, (a.E + PR_E - 1) / PR_E), dim3(256), 0, s, a.x,
                           a.router, a.H, a.T, a.E, a.logits);
        hipLaunchKernelGGL(k_pf_topk, dim3((a.T + WAVES - 1) / WAVES), dim3(256), 0, s, a.logits, a.T, a.E, a.K, a.ids,
                           a.w, a.hits, a.status);
    }
    hipLaunchKernelGGL(k_pf_xpack, dim3(a.T), dim3(256), 0, s, a.x, a.H, a.x16, a.xexp);
    hipLaunchKernelGGL(k_pf_group, dim3(1), dim3(1024), 0, s, a.ids, a.T, a.K, a.E, a.has_shared, a.offsets, a.sorted,
                       a.passes, a.pass_count, a.xexp);
    if (a.has_shared && a.sh_gate_inp)
        hipLaunchKernelGGL(k_pf_shgate, dim3(a.T), dim3(256), 0, s, a.x, a.sh_gate_inp, a.H, a.sg);
    return (int)hipGetLastError();
}

template <int NMAT, int AHL, int NSUB> static int launch_gemm(const PfGemm& g, int n_wg, hipStream_t s) {
    typedef GmGeo<NMAT, AHL, NSUB> G;
    hipError_t e = hipFuncSetAttribute((const void*)k_pf_gemm<NMAT, AHL, NSUB>,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, G::LDS);
    if (e != hipSuccess) return (int)e;
    hipLaunchKernelGGL((k_pf_gemm<NMAT, AHL, NSUB>), dim3(n_wg), dim3(GM_THREADS), G::LDS, s, g);
    return (int)hipGetLastError();
}

int launch_prefill_gateup(const PrefillArgs& a, hipStream_t s) {
    PfGemm g = {};
    g.w0 = a.gate; g.w1 = a.up; g.st0 = a.gstride; g.st1 = a.ustride;
    g.s0 = a.sh_gate; g.s1 = a.sh_up;
    g.rb_r = g.rb_s = (int64_t)(a.H / 32) * 34;
    g.mb_r = (int32_t)(g.rb_r * a.I);
    g.mb_s = a.has_shared ? (int32_t)(g.rb_s * a.Is) : g.mb_r;
    g.a_hi = a.x16; g.a_lo = a.x16; g.a_ld = a.H; g.a_sc = nullptr; g.sc_ld = 0;
    g.a_bytes = (int32_t)((int64_t)a.T * a.H * 2); g.sc_bytes = 0;
    g.T = a.T; g.K = a.K; g.E = a.E; g.by_token = 1;
    g.nrb_r = a.I / GM_ROWS; g.nrb_s = a.has_shared ? a.Is / GM_ROWS : 1;
    g.nkc_r = g.nkc_s = a.H / 128;
    g.recs = a.passes; g.npass = a.pass_count;
    g.o_hi = a.act_hi; g.o_lo = a.act_lo; g.o_sc = a.act_sc; g.o_ld = a.act_stride; g.osc_ld = a.act_stride / 128;
    return launch_gemm<2, 1, 1>(g, a.n_wg, s);
}

int launch_prefill_down(const PrefillArgs& a, hipStream_t s) {
    PfGemm g = {};
    g.w0 = a.down; g.w1 = a.down; g.st0 = g.st1 = a.dstride;
    g.s0 = g.s1 = a.sh_down;
    g.rb_r = (int64_t)(a.I / 32) * 34; g.rb_s = a.has_shared ? (int64_t)(a.Is / 32) * 34 : g.rb_r;
    g.mb_r = (int32_t)(g.rb_r * a.H); g.mb_s = (int32_t)(g.rb_s * a.H);
    g.a_hi = a.act_hi; g.a_lo = a.act_lo; g.a_ld = a.act_stride; g.a_sc = a.act_sc; g.sc_ld = a.act_stride / 128;
    const int64_t pairs = (int64_t)a.T * a.K + (a.has_shared ? a.T : 0);
    g.a_bytes = (int32_t)(pairs * a.act_stride * 2); g.sc_bytes = (int32_t)(pairs * (a.act_stride / 128) * 4);
    g.T = a.T; g.K = a.K; g.E = a.E; g.by_token = 0;
    g.nkc_r = a.I / 128; g.nkc_s = a.has_shared ? a.Is / 128 : g.nkc_r;
    g.recs = a.passes; g.npass = a.pass_count;
    g.y = a.y; g.y_ld = a.H;
    // row groups of 4 blocks of 128 rows when H allows, else of 2 (H % 256 == 0)
    if (a.H % (4 * GM_ROWS) == 0) {
        g.nrb_r = g.nrb_s = a.H / (4 * GM_ROWS);
        return launch_gemm<1, 2, 4>(g, a.n_wg, s);
    }
    g.nrb_r = g.nrb_s = a.H / (2 * GM_ROWS);
    return launch_gemm<1, 2, 2>(g, a.n_wg, s);
}

int launch_prefill_combine(const PrefillArgs& a, hipStream_t s) {
    hipLaunchKernelGGL(k_pf_combine, dim3((a.H / 4 + 255) / 256, a.T), dim3(256), 0, s, a);
    return (int)hipGetLastError();
}

}  // namespace wm
