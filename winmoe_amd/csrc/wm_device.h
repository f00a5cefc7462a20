// wm_device.h -- device building blocks of the expert kernels (gfx950, wave64).
//
// Data flow of one expert matrix-vector product:
//   * a wave stages a tile of 4096 weights (floor(64 / (in/64)) whole rows) of
//     raw GGUF bytes from HBM into its private LDS slice with coalesced 16-byte
//     loads (no repacking of the block layout);
//   * lane l decodes segment l of the tile (Seg<T>::load): 64 quantised values
//     packed four per dword, plus one fp32 multiplier a[r] (and min b[r]) per
//     independently scaled run;
//   * the activation operand of the lane's columns is held as two signed 8-bit
//     digits per value (XOp), so each packed dword meets two v_dot4_i32_i8;
//     run sums are exact int32, scaled once per run in fp32;
//   * the lanes of a row reduce their partials with a fixed butterfly
//     (deterministic order).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "wm_format.h"

#define WM_DEV __device__ __forceinline__

namespace wm {

typedef __attribute__((address_space(3))) uint8_t lds8_t;
typedef __attribute__((address_space(3))) uint16_t lds16_t;
typedef __attribute__((address_space(3))) uint32_t lds32_t;
typedef __attribute__((address_space(3))) uint64_t lds64_t;
typedef __attribute__((address_space(3))) float lf32_t;

WM_DEV float h2f(uint32_t bits) { return (float)__builtin_bit_cast(_Float16, (uint16_t)(bits & 0xFFFFu)); }

WM_DEV uint32_t alignbyte(uint32_t hi, uint32_t lo, uint32_t sel) { return __builtin_amdgcn_alignbyte(hi, lo, sel); }

WM_DEV int dot4(uint32_t a, uint32_t b, int c) { return __builtin_amdgcn_sdot4((int)a, (int)b, c, false); }

// 4 dwords starting at any byte offset of an LDS buffer (reads 5 aligned dwords).
WM_DEV void lds_u32x4(const lds8_t* base, uint32_t off, uint32_t* o) {
    const lds32_t* p = (const lds32_t*)(base + (off & ~3u));
    uint32_t s = off & 3u;
    uint32_t w0 = p[0], w1 = p[1], w2 = p[2], w3 = p[3], w4 = p[4];
    o[0] = alignbyte(w1, w0, s);
    o[1] = alignbyte(w2, w1, s);
    o[2] = alignbyte(w3, w2, s);
    o[3] = alignbyte(w4, w3, s);
}
WM_DEV uint32_t lds_u32(const lds8_t* base, uint32_t off) {
    const lds32_t* p = (const lds32_t*)(base + (off & ~3u));
    return alignbyte(p[1], p[0], off & 3u);
}
WM_DEV uint32_t byte_of(uint32_t w, int k) { return (w >> (8 * k)) & 0xFFu; }

// ------------------------------------------------------------- segments
// Seg<T>: NDW packed dwords q[], NRUN runs of RUNDW dwords each (Q8_0: 9 + 8),
// per-run multiplier a[] and min b[], value bias BIAS (w = a*(q - BIAS) - b).

template <int T> struct Seg;

// Q8_0: lane l owns blocks 2l, 2l+1 of the tile = bytes [68l, 68l+68), read
// as 17 raw dwords.  The d bytes stay inside dwords 0 and 8; the activation
// operand carries zero digits at those byte positions.
template <> struct Seg<Q8_0> {
    static constexpr int NDW = 17, NRUN = 2, BIAS = 0;
    uint32_t q[17];
    float a[2], b[2];
    WM_DEV void load(const lds8_t* t, int lane) {
        const lds32_t* p = (const lds32_t*)(t + 68 * lane);
#pragma unroll
        for (int i = 0; i < 17; i++) q[i] = p[i];
        a[0] = h2f(q[0]);
        a[1] = h2f(q[8] >> 16);
        b[0] = b[1] = 0.0f;
    }
    WM_DEV int value(int j) const {          // signed q of weight j (0..63)
        int p = j + 2 + ((j >> 5) << 1);
        return (int)(int8_t)byte_of(q[p >> 2], p & 3);
    }
    WM_DEV int run_of(int j) const { return j >> 5; }
};

// Q4_K / Q5_K 6-bit scale and min of sub-block i (q4k_dequant.h:43-60), the
// 12 scale bytes being s0, s1, s2: i < 4 takes byte i of s0 (scale) and of
// s1 (min); i >= 4 takes byte j = i - 4 of s2 (low nibbles) and the top two
// bits of byte j of s0 and of s1.  Shifts and one select, so a lane-varying
// i indexes no register array.
WM_DEV void k45_scale_min(uint32_t s0, uint32_t s1, uint32_t s2, int i, int& sc, int& m) {
    const uint32_t sh = 8u * (uint32_t)(i & 3);
    const uint32_t b0 = (s0 >> sh) & 0xFFu, b1 = (s1 >> sh) & 0xFFu, b2 = (s2 >> sh) & 0xFFu;
    const bool lo = i < 4;
    sc = (int)(lo ? (b0 & 63u) : ((b2 & 0xFu) | ((b0 >> 6) << 4)));
    m = (int)(lo ? (b1 & 63u) : ((b2 >> 4) | ((b1 >> 6) << 4)));
}

// Q4_K: lane l -> block l/4, chunk c = l%4 (32 qs bytes): low nibbles are
// columns 64c+[0,32) (sub-block 2c), high nibbles 64c+32+[0,32) (2c+1).
template <> struct Seg<Q4_K> {
    static constexpr int NDW = 16, NRUN = 2, BIAS = 0;
    uint32_t q[16];
    float a[2], b[2];
    WM_DEV void load(const lds8_t* t, int lane) {
        const lds8_t* blk = t + 144 * (lane >> 2);
        int c = lane & 3;
        const lds32_t* h = (const lds32_t*)blk;
        uint32_t h0 = h[0], s0 = h[1], s1 = h[2], s2 = h[3];
        const lds32_t* qs = (const lds32_t*)(blk + 16 + 32 * c);
#pragma unroll
        for (int i = 0; i < 8; i++) {
            uint32_t w = qs[i];
            q[i] = w & 0x0F0F0F0Fu;
            q[8 + i] = (w >> 4) & 0x0F0F0F0Fu;
        }
        float d = h2f(h0), dmin = h2f(h0 >> 16);
        int sc0, m0, sc1, m1;
        k45_scale_min(s0, s1, s2, 2 * c, sc0, m0);
        k45_scale_min(s0, s1, s2, 2 * c + 1, sc1, m1);
        a[0] = d * (float)sc0; b[0] = dmin * (float)m0;
        a[1] = d * (float)sc1; b[1] = dmin * (float)m1;
    }
    WM_DEV int value(int j) const { return (int)byte_of(q[j >> 2], j & 3); }
    WM_DEV int run_of(int j) const { return j >> 5; }
};

// Q5_K: as Q4_K with bit (2c) / (2c+1) of qh[j] as the fifth bit (q5k_dequant.h:98-131).
template <> struct Seg<Q5_K> {
    static constexpr int NDW = 16, NRUN = 2, BIAS = 0;
    uint32_t q[16];
    float a[2], b[2];
    WM_DEV void load(const lds8_t* t, int lane) {
        const lds8_t* blk = t + 176 * (lane >> 2);
        int c = lane & 3;
        const lds32_t* h = (const lds32_t*)blk;
        uint32_t h0 = h[0], s0 = h[1], s1 = h[2], s2 = h[3];
        const lds32_t* qh = (const lds32_t*)(blk + 16);
        const lds32_t* qs = (const lds32_t*)(blk + 48 + 32 * c);
#pragma unroll
        for (int i = 0; i < 8; i++) {
            uint32_t w = qs[i], e = qh[i];
            q[i] = (w & 0x0F0F0F0Fu) | (((e >> (2 * c)) & 0x01010101u) << 4);
            q[8 + i] = ((w >> 4) & 0x0F0F0F0Fu) | (((e >> (2 * c + 1)) & 0x01010101u) << 4);
        }
        float d = h2f(h0), dmin = h2f(h0 >> 16);
        int sc0, m0, sc1, m1;
        k45_scale_min(s0, s1, s2, 2 * c, sc0, m0);
        k45_scale_min(s0, s1, s2, 2 * c + 1, sc1, m1);
        a[0] = d * (float)sc0; b[0] = dmin * (float)m0;
        a[1] = d * (float)sc1; b[1] = dmin * (float)m1;
    }
    WM_DEV int value(int j) const { return (int)byte_of(q[j >> 2], j & 3); }
    WM_DEV int run_of(int j) const { return j >> 5; }
};

// Q6_K: lane l -> block l/4, r = l%4: half h = r/2, sixteenth i = r%2.
// Run g (0..3) = columns 128h + 32g + 16i + [0,16), scale sc[8h + i + 2g]
// (q6k_dequant.h:112-141, is = n/16 + l/16), value q - 32.
template <> struct Seg<Q6_K> {
    static constexpr int NDW = 16, NRUN = 4, BIAS = 32;
    uint32_t q[16];
    float a[4], b[4];
    WM_DEV void load(const lds8_t* t, int lane) {
        uint32_t blk = 210u * (uint32_t)(lane >> 2);
        int r = lane & 3, h = r >> 1, i = r & 1;
        uint32_t la[4], lb[4], e[4];
        lds_u32x4(t, blk + 64 * h + 16 * i, la);
        lds_u32x4(t, blk + 64 * h + 32 + 16 * i, lb);
        lds_u32x4(t, blk + 128 + 32 * h + 16 * i, e);
#pragma unroll
        for (int k = 0; k < 4; k++) {
            q[k] = (la[k] & 0x0F0F0F0Fu) | ((e[k] & 0x03030303u) << 4);
            q[4 + k] = (lb[k] & 0x0F0F0F0Fu) | (((e[k] >> 2) & 0x03030303u) << 4);
            q[8 + k] = ((la[k] >> 4) & 0x0F0F0F0Fu) | (((e[k] >> 4) & 0x03030303u) << 4);
            q[12 + k] = ((lb[k] >> 4) & 0x0F0F0F0Fu) | (((e[k] >> 6) & 0x03030303u) << 4);
        }
        uint32_t s0 = lds_u32(t, blk + 192 + 8 * h), s1 = lds_u32(t, blk + 196 + 8 * h);
        float d = h2f(lds_u32(t, blk + 208));
        // scales[8h + i + 2g]: bytes i, i+2 of s0 and i, i+2 of s1
        a[0] = d * (float)(int8_t)byte_of(s0, i);
        a[1] = d * (float)(int8_t)byte_of(s0, i + 2);
        a[2] = d * (float)(int8_t)byte_of(s1, i);
        a[3] = d * (float)(int8_t)byte_of(s1, i + 2);
        b[0] = b[1] = b[2] = b[3] = 0.0f;
    }
    WM_DEV int value(int j) const { return (int)byte_of(q[j >> 2], j & 3); }
    WM_DEV int run_of(int j) const { return j >> 4; }
};

// Q2_K: lane l -> block l/4, half h, sixteenth i.  Run j (0..3) = columns
// 128h + 32j + 16i + [0,16) from bits 2j of qs[32h + 16i + 0..15], scale byte
// scales[8h + 2j + i]: multiplier d*(s & 15), min dmin*(s >> 4).
template <> struct Seg<Q2_K> {
    static constexpr int NDW = 16, NRUN = 4, BIAS = 0;
    uint32_t q[16];
    float a[4], b[4];
    WM_DEV void load(const lds8_t* t, int lane) {
        const lds8_t* blk = t + 84 * (lane >> 2);
        int r = lane & 3, h = r >> 1, i = r & 1;
        const lds32_t* qs = (const lds32_t*)(blk + 16 + 32 * h + 16 * i);
        uint32_t w[4] = {qs[0], qs[1], qs[2], qs[3]};
#pragma unroll
        for (int j = 0; j < 4; j++)
#pragma unroll
            for (int k = 0; k < 4; k++) q[4 * j + k] = (w[k] >> (2 * j)) & 0x03030303u;
        const lds32_t* sp = (const lds32_t*)(blk + 8 * h);
        uint32_t s0 = sp[0], s1 = sp[1];
        uint32_t dd = ((const lds32_t*)(blk + 80))[0];
        float d = h2f(dd), dmin = h2f(dd >> 16);
        uint32_t sc[4] = {byte_of(s0, i), byte_of(s0, i + 2), byte_of(s1, i), byte_of(s1, i + 2)};
#pragma unroll
        for (int j = 0; j < 4; j++) {
            a[j] = d * (float)(sc[j] & 0xF);
            b[j] = dmin * (float)(sc[j] >> 4);
        }
    }
    WM_DEV int value(int j) const { return (int)byte_of(q[j >> 2], j & 3); }
    WM_DEV int run_of(int j) const { return j >> 4; }
};

// Q3_K sixteen 6-bit scales: low nibble from byte k (k < 8) or the high nibble
// of byte k-8; high two bits from byte 8 + (k & 3) at shift 2*(k >> 2).
WM_DEV int q3k_scale(uint32_t s0, uint32_t s1, uint32_t s2, int k) {
    uint32_t lo = k < 8 ? byte_of(k < 4 ? s0 : s1, k & 3) & 0xF : byte_of(k < 12 ? s0 : s1, k & 3) >> 4;
    uint32_t hi = (byte_of(s2, k & 3) >> (2 * (k >> 2))) & 3;
    return (int)(lo | (hi << 4)) - 32;
}

// Q3_K: lane l -> block l/4, half h, sixteenth i.  Run j = columns
// 128h + 32j + 16i + [0,16): low two bits from qs[32h + 16i + ..] >> 2j, high
// bit (4h + j) of hmask[16i + ..] (clear = minus 4); stored here as the
// unsigned 3-bit value q + 4 with BIAS 4.
template <> struct Seg<Q3_K> {
    static constexpr int NDW = 16, NRUN = 4, BIAS = 4;
    uint32_t q[16];
    float a[4], b[4];
    WM_DEV void load(const lds8_t* t, int lane) {
        uint32_t blk = 110u * (uint32_t)(lane >> 2);
        int r = lane & 3, h = r >> 1, i = r & 1;
        uint32_t w[4], m[4];
        lds_u32x4(t, blk + 32 + 32 * h + 16 * i, w);
        lds_u32x4(t, blk + 16 * i, m);
#pragma unroll
        for (int j = 0; j < 4; j++)
#pragma unroll
            for (int k = 0; k < 4; k++)
                q[4 * j + k] = ((w[k] >> (2 * j)) & 0x03030303u) | (((m[k] >> (4 * h + j)) & 0x01010101u) << 2);
        uint32_t s0 = lds_u32(t, blk + 96), s1 = lds_u32(t, blk + 100), s2 = lds_u32(t, blk + 104);
        float d = h2f(lds_u32(t, blk + 108));
#pragma unroll
        for (int j = 0; j < 4; j++) {
            a[j] = d * (float)q3k_scale(s0, s1, s2, 8 * h + 2 * j + i);
            b[j] = 0.0f;
        }
    }
    WM_DEV int value(int j) const { return (int)byte_of(q[j >> 2], j & 3); }
    WM_DEV int run_of(int j) const { return j >> 4; }
};

// Exact dequantised weight j of a decoded segment (same float expression as
// the oracle: products are exact in fp32, one rounding at the subtraction).
template <int T> WM_DEV float seg_weight(const Seg<T>& s, int j) {
    int r = s.run_of(j);
    return s.a[r] * (float)(s.value(j) - Seg<T>::BIAS) - s.b[r];
}

// ------------------------------------------------------------- activation operand
struct XOp {
    uint32_t hi[17], lo[17];
    int sum[4];
    float s;
};

typedef float f32x4 __attribute__((ext_vector_type(4)));

// Operand of 64 values v[j] (segment order) for type T: two signed 8-bit
// digits per value, x_j ~= s * (256*hi + lo) with |256*hi + lo| <= 32639
// (round to nearest even), packed in the byte order of the segment's
// quantised values (Q8_0: after each block's 2-byte scale), the exact integer
// run sums, and s = amax / 32639 (NaN when a value is not finite, which makes
// every dot product with the segment NaN).
template <int T> WM_DEV void xop_core(const float* v, uint32_t* hi, uint32_t* lo, int* sum, float& s) {
    constexpr bool Q8 = (T == Q8_0);
    constexpr int RUNLEN = (T == Q8_0 || T == Q4_K || T == Q5_K) ? 32 : 16;
    float amax = 0.0f;
    bool finite = true;
#pragma unroll
    for (int j = 0; j < 64; j++) {
        amax = fmaxf(amax, fabsf(v[j]));
        finite = finite && isfinite(v[j]);
    }
    float inv = amax > 0.0f ? 32639.0f / amax : 0.0f;
#pragma unroll
    for (int k = 0; k < 17; k++) hi[k] = lo[k] = 0u;
#pragma unroll
    for (int r = 0; r < 4; r++) sum[r] = 0;
#pragma unroll
    for (int j = 0; j < 64; j++) {
        int xi = finite ? (int)rintf(v[j] * inv) : 0;
        xi = xi > 32639 ? 32639 : (xi < -32639 ? -32639 : xi);
        int l = ((xi + 128) & 255) - 128;
        int h = (xi - l) >> 8;
        int p = Q8 ? j + 2 + ((j >> 5) << 1) : j;
        hi[p >> 2] |= ((uint32_t)h & 0xFFu) << (8 * (p & 3));
        lo[p >> 2] |= ((uint32_t)l & 0xFFu) << (8 * (p & 3));
        sum[j / RUNLEN] += xi;
    }
    s = finite ? amax / 32639.0f : __builtin_nanf("");
}

// The 64 values of segment `seg` of a 16-byte aligned fp32 vector: four runs
// of 16 consecutive floats (seg_col), fetched as 16 b128 loads.
template <int T> WM_DEV void xop_fetch(const float* src, int seg, f32x4 (&r)[16]) {
#pragma unroll
    for (int g = 0; g < 4; g++) {
        const f32x4* p = (const f32x4*)(src + seg_col(T, seg, 16 * g));
#pragma unroll
        for (int q = 0; q < 4; q++) r[4 * g + q] = p[q];
    }
}

template <int T> WM_DEV void xop_make(const f32x4 (&r)[16], XOp& x) {
    float v[64];
#pragma unroll
    for (int i = 0; i < 16; i++) {
        v[4 * i] = r[i].x; v[4 * i + 1] = r[i].y; v[4 * i + 2] = r[i].z; v[4 * i + 3] = r[i].w;
    }
    xop_core<T>(v, x.hi, x.lo, x.sum, x.s);
}

// Device-coherent access for data handed between workgroups inside one
// launch (COH = true): relaxed agent-scope atomics, i.e. loads / stores with
// the device-scope cache policy (sc1), which bypass the per-XCD L2's
// non-coherent copies without whole-cache writeback or invalidation.
template <bool COH, typename V> WM_DEV void gst(V* p, V v) {
    if constexpr (COH) __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    else *p = v;
}
template <bool COH, typename V> WM_DEV V gld(const V* p) {
    if constexpr (COH) return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    else return *p;
}

// Segment partial dot product: sum_j w_j * x_j of the lane's 64 weights.
template <int T> WM_DEV float seg_dot(const Seg<T>& s, const XOp& x) {
    if constexpr (T == Q8_0) {
        int h0 = 0, l0 = 0, h1 = 0, l1 = 0;
#pragma unroll
        for (int i = 0; i < 9; i++) { h0 = dot4(s.q[i], x.hi[i], h0); l0 = dot4(s.q[i], x.lo[i], l0); }
#pragma unroll
        for (int i = 9; i < 17; i++) { h1 = dot4(s.q[i], x.hi[i], h1); l1 = dot4(s.q[i], x.lo[i], l1); }
        // explicit fused multiply-adds: every kernel computes the same value
        // whatever the compiler would otherwise contract (contraction is off)
        const float r = fmaf(s.a[0], (float)(h0 * 256 + l0), s.a[1] * (float)(h1 * 256 + l1));
        return r * x.s;
    } else {
        constexpr int NR = Seg<T>::NRUN, DPR = 16 / NR;
        float r = 0.0f;
#pragma unroll
        for (int run = 0; run < NR; run++) {
            int hs = 0, ls = 0;
#pragma unroll
            for (int i = run * DPR; i < (run + 1) * DPR; i++) { hs = dot4(s.q[i], x.hi[i], hs); ls = dot4(s.q[i], x.lo[i], ls); }
            int S = hs * 256 + ls - Seg<T>::BIAS * x.sum[run];
            r += fmaf(s.a[run], (float)S, -(s.b[run] * (float)x.sum[run]));
        }
        return r * x.s;
    }
}

// DPP lane moves (gfx9 encodings): quad permutes, mirrors within 8 and 16
// lanes, rotations within a row of 16, and the row broadcasts of lane 15 /
// lane 31.  A lane whose row is masked off, or whose source is off, gets 0.
constexpr int DPP_XOR1 = 0xB1, DPP_XOR2 = 0x4E, DPP_HALF_MIRROR = 0x141, DPP_MIRROR = 0x140;
constexpr int DPP_ROR1 = 0x121, DPP_ROR2 = 0x122, DPP_ROR4 = 0x124, DPP_ROR8 = 0x128;
constexpr int DPP_BCAST15 = 0x142, DPP_BCAST31 = 0x143;
template <int CTRL, int ROW_MASK = 0xF> WM_DEV uint32_t dpp_u32(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, ROW_MASK, 0xF, false);
}
template <int CTRL, int ROW_MASK = 0xF> WM_DEV float dpp_f32(float v) {
    return __builtin_bit_cast(float, dpp_u32<CTRL, ROW_MASK>(__builtin_bit_cast(uint32_t, v)));
}
template <int CTRL> WM_DEV uint64_t dpp_u64(uint64_t v) {
    return ((uint64_t)dpp_u32<CTRL>((uint32_t)(v >> 32)) << 32) | dpp_u32<CTRL>((uint32_t)v);
}

// Sum over groups of `lpr` consecutive lanes (lpr a power of two <= 64), with
// DPP moves; the sum is complete in the group's last lane (in every lane of
// the group when lpr <= 16).  Called with all 64 lanes active.
WM_DEV float row_reduce(float v, int lpr) {
    if (lpr >= 2) v += dpp_f32<DPP_XOR1>(v);
    if (lpr >= 4) v += dpp_f32<DPP_XOR2>(v);
    if (lpr >= 8) v += dpp_f32<DPP_HALF_MIRROR>(v);
    if (lpr >= 16) v += dpp_f32<DPP_MIRROR>(v);
    if (lpr >= 32) v += dpp_f32<DPP_BCAST15, 0xA>(v);
    if (lpr >= 64) v += dpp_f32<DPP_BCAST31, 0xC>(v);
    return v;
}

WM_DEV uint64_t max_u64(uint64_t a, uint64_t b) { return a > b ? a : b; }

// gfx950 cross-row lane swaps with both operands v: permlane16_swap pairs row
// r (16 lanes) with row r^1, permlane32_swap lane i with lane i^32; .first
// and .second of the result are the two members of each pair.
WM_DEV uint64_t swap_max_u64_rows(uint64_t v) {
    const uint32_t hi = (uint32_t)(v >> 32), lo = (uint32_t)v;
    const auto h = __builtin_amdgcn_permlane16_swap(hi, hi, false, false);
    const auto l = __builtin_amdgcn_permlane16_swap(lo, lo, false, false);
    return max_u64(((uint64_t)h[0] << 32) | l[0], ((uint64_t)h[1] << 32) | l[1]);
}
WM_DEV uint64_t swap_max_u64_halves(uint64_t v) {
    const uint32_t hi = (uint32_t)(v >> 32), lo = (uint32_t)v;
    const auto h = __builtin_amdgcn_permlane32_swap(hi, hi, false, false);
    const auto l = __builtin_amdgcn_permlane32_swap(lo, lo, false, false);
    return max_u64(((uint64_t)h[0] << 32) | l[0], ((uint64_t)h[1] << 32) | l[1]);
}

// Maximum of a 32-bit value over the wave (all 64 lanes active), in every lane.
WM_DEV uint32_t wave_max_u32(uint32_t v) {
    v = max(v, dpp_u32<DPP_XOR1>(v));
    v = max(v, dpp_u32<DPP_XOR2>(v));
    v = max(v, dpp_u32<DPP_HALF_MIRROR>(v));
    v = max(v, dpp_u32<DPP_MIRROR>(v));
    const auto a = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    v = max((uint32_t)a[0], (uint32_t)a[1]);
    const auto b = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    return max((uint32_t)b[0], (uint32_t)b[1]);
}

// Maximum of a 64-bit key over the wave (all 64 lanes active), in every lane:
// DPP within rows of 16, then the two cross-row swaps; no scalar round trips.
WM_DEV uint64_t wave_max_u64(uint64_t v) {
    v = max_u64(v, dpp_u64<DPP_XOR1>(v));
    v = max_u64(v, dpp_u64<DPP_XOR2>(v));
    v = max_u64(v, dpp_u64<DPP_HALF_MIRROR>(v));
    v = max_u64(v, dpp_u64<DPP_MIRROR>(v));
    v = swap_max_u64_rows(v);
    return swap_max_u64_halves(v);
}

// s_waitcnt with vmcnt only (gfx9 encoding: vmcnt[3:0] | vmcnt[5:4] << 14,
// expcnt and lgkmcnt left at their "don't wait" maxima).
#define WM_WAIT_VMCNT(n) __builtin_amdgcn_s_waitcnt(((n) & 0xF) | (((n) >> 4) << 14) | (0x7 << 4) | (0xF << 8))

WM_DEV void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

}  // namespace wm
