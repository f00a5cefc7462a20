// wm_quant.h -- block quantisers for building synthetic expert tensors.
//
// Compiled for both host and device; identical float operations (no FMA
// contraction, correctly rounded division, roundf, RNE fp16 conversion) make
// the host and device outputs bit-identical.  These are valid packings of the
// ggml block formats, not ggml's search-based quantisers: parity always
// compares the HIP path with the oracle on the same bytes, so any valid
// packing serves (the reference itself ships no weight quantiser).
#pragma once
#include <math.h>
#include <stdint.h>

#include "wm_format.h"

namespace wm {

WM_HD uint16_t f32_to_f16_bits(float x) {
    _Float16 h = (_Float16)x;
    return __builtin_bit_cast(uint16_t, h);
}
WM_HD float f16_bits_to_f32(uint16_t b) { return (float)__builtin_bit_cast(_Float16, b); }

WM_HD int q_round_clamp(float v, int lo, int hi) {
    if (!(v == v)) return 0;                     // NaN -> 0
    float r = roundf(v);
    if (r < (float)lo) return lo;
    if (r > (float)hi) return hi;
    return (int)r;
}

WM_HD void put16(uint8_t* p, uint16_t v) { p[0] = (uint8_t)(v & 0xFF); p[1] = (uint8_t)(v >> 8); }

// Q8_0: d = amax/127, q = round(x/d).
WM_HD void quant_block_q8_0(const float* x, uint8_t* b) {
#pragma clang fp contract(off)
    float amax = 0.0f;
    for (int j = 0; j < 32; j++) amax = fmaxf(amax, fabsf(x[j]));
    float d = amax / 127.0f;
    float id = d != 0.0f ? 1.0f / d : 0.0f;
    put16(b, f32_to_f16_bits(d));
    for (int j = 0; j < 32; j++) b[2 + j] = (uint8_t)(int8_t)q_round_clamp(x[j] * id, -127, 127);
}

// Q4_K (NMAX = 15) and Q5_K (NMAX = 31): per 32-weight sub-block an
// asymmetric range [mn, mx] with mn <= 0; 6-bit scales/mins relative to the
// super-block d / dmin.
template <int NMAX>
WM_HD void quant_k45_core(const float* x, uint16_t* dh, uint16_t* dmh, uint8_t* sc6, uint8_t* m6, uint8_t* q) {
#pragma clang fp contract(off)
    float scale[8], mins[8], maxs = 0.0f, maxm = 0.0f;
    for (int j = 0; j < 8; j++) {
        float mn = 0.0f, mx = 0.0f;
        for (int l = 0; l < 32; l++) {
            float v = x[32 * j + l];
            mn = fminf(mn, v);
            mx = fmaxf(mx, v);
        }
        scale[j] = (mx - mn) / (float)NMAX;
        mins[j] = mn < 0.0f ? -mn : 0.0f;   // never -0: fmaxf(+0, -0) differs between host and device
        maxs = fmaxf(maxs, scale[j]);
        maxm = fmaxf(maxm, mins[j]);
    }
    float d = maxs / 63.0f, dmin = maxm / 63.0f;
    *dh = f32_to_f16_bits(d);
    *dmh = f32_to_f16_bits(dmin);
    float df = f16_bits_to_f32(*dh), dmf = f16_bits_to_f32(*dmh);
    for (int j = 0; j < 8; j++) {
        sc6[j] = df > 0.0f ? (uint8_t)q_round_clamp(scale[j] / df, 0, 63) : 0;
        m6[j] = dmf > 0.0f ? (uint8_t)q_round_clamp(mins[j] / dmf, 0, 63) : 0;
        float ds = df * (float)sc6[j], dm = dmf * (float)m6[j];
        for (int l = 0; l < 32; l++)
            q[32 * j + l] = ds > 0.0f ? (uint8_t)q_round_clamp((x[32 * j + l] + dm) / ds, 0, NMAX) : 0;
    }
}

// Inverse of the 6-bit scale/min packing read by q4k_dequant.h:43-60.
WM_HD void pack_k45_scales(const uint8_t* sc6, const uint8_t* m6, uint8_t* s) {
    for (int j = 0; j < 4; j++) {
        s[j] = (uint8_t)((sc6[j] & 63) | ((sc6[j + 4] >> 4) << 6));
        s[j + 4] = (uint8_t)((m6[j] & 63) | ((m6[j + 4] >> 4) << 6));
        s[j + 8] = (uint8_t)((sc6[j + 4] & 0xF) | ((m6[j + 4] & 0xF) << 4));
    }
}

WM_HD void quant_block_q4_k(const float* x, uint8_t* b) {
    uint16_t dh, dmh;
    uint8_t sc6[8], m6[8], q[256];
    quant_k45_core<15>(x, &dh, &dmh, sc6, m6, q);
    put16(b, dh);
    put16(b + 2, dmh);
    pack_k45_scales(sc6, m6, b + 4);
    for (int c = 0; c < 4; c++)
        for (int l = 0; l < 32; l++) b[16 + 32 * c + l] = (uint8_t)(q[64 * c + l] | (q[64 * c + 32 + l] << 4));
}

WM_HD void quant_block_q5_k(const float* x, uint8_t* b) {
    uint16_t dh, dmh;
    uint8_t sc6[8], m6[8], q[256];
    quant_k45_core<31>(x, &dh, &dmh, sc6, m6, q);
    put16(b, dh);
    put16(b + 2, dmh);
    pack_k45_scales(sc6, m6, b + 4);
    for (int l = 0; l < 32; l++) {
        uint8_t h = 0;
        for (int c = 0; c < 4; c++) {
            h |= (uint8_t)(((q[64 * c + l] >> 4) & 1) << (2 * c));
            h |= (uint8_t)(((q[64 * c + 32 + l] >> 4) & 1) << (2 * c + 1));
        }
        b[16 + l] = h;
    }
    for (int c = 0; c < 4; c++)
        for (int l = 0; l < 32; l++)
            b[48 + 32 * c + l] = (uint8_t)((q[64 * c + l] & 0xF) | ((q[64 * c + 32 + l] & 0xF) << 4));
}

// Q6_K: symmetric 16-weight sub-blocks (scale index = weight / 16), q in [0,63].
WM_HD void quant_block_q6_k(const float* x, uint8_t* b) {
#pragma clang fp contract(off)
    float scale[16], maxs = 0.0f;
    for (int j = 0; j < 16; j++) {
        float amax = 0.0f;
        for (int l = 0; l < 16; l++) amax = fmaxf(amax, fabsf(x[16 * j + l]));
        scale[j] = amax / 31.0f;
        maxs = fmaxf(maxs, scale[j]);
    }
    float d = maxs / 127.0f;
    uint16_t dh = f32_to_f16_bits(d);
    float df = f16_bits_to_f32(dh);
    int8_t sc[16];
    uint8_t q[256];
    for (int j = 0; j < 16; j++) {
        sc[j] = df > 0.0f ? (int8_t)q_round_clamp(scale[j] / df, 0, 127) : 0;
        float s = df * (float)sc[j];
        for (int l = 0; l < 16; l++)
            q[16 * j + l] = (uint8_t)((s > 0.0f ? q_round_clamp(x[16 * j + l] / s, -32, 31) : 0) + 32);
    }
    for (int h = 0; h < 2; h++) {
        int n = 128 * h;
        for (int l = 0; l < 32; l++) {
            int q1 = q[n + l], q2 = q[n + l + 32], q3 = q[n + l + 64], q4 = q[n + l + 96];
            b[64 * h + l] = (uint8_t)((q1 & 0xF) | ((q3 & 0xF) << 4));
            b[64 * h + l + 32] = (uint8_t)((q2 & 0xF) | ((q4 & 0xF) << 4));
            b[128 + 32 * h + l] = (uint8_t)((q1 >> 4) | ((q2 >> 4) << 2) | ((q3 >> 4) << 4) | ((q4 >> 4) << 6));
        }
    }
    for (int j = 0; j < 16; j++) b[192 + j] = (uint8_t)sc[j];
    put16(b + 208, dh);
}

// Q2_K: asymmetric 16-weight sub-blocks (scale index = weight / 16), q in [0,3].
WM_HD void quant_block_q2_k(const float* x, uint8_t* b) {
#pragma clang fp contract(off)
    float scale[16], mins[16], maxs = 0.0f, maxm = 0.0f;
    for (int j = 0; j < 16; j++) {
        float mn = 0.0f, mx = 0.0f;
        for (int l = 0; l < 16; l++) {
            mn = fminf(mn, x[16 * j + l]);
            mx = fmaxf(mx, x[16 * j + l]);
        }
        scale[j] = (mx - mn) / 3.0f;
        mins[j] = mn < 0.0f ? -mn : 0.0f;   // never -0: fmaxf(+0, -0) differs between host and device
        maxs = fmaxf(maxs, scale[j]);
        maxm = fmaxf(maxm, mins[j]);
    }
    float d = maxs / 15.0f, dmin = maxm / 15.0f;
    uint16_t dh = f32_to_f16_bits(d), dmh = f32_to_f16_bits(dmin);
    float df = f16_bits_to_f32(dh), dmf = f16_bits_to_f32(dmh);
    for (int k = 0; k < 64; k++) b[16 + k] = 0;
    for (int j = 0; j < 16; j++) {
        int s4 = df > 0.0f ? q_round_clamp(scale[j] / df, 0, 15) : 0;
        int m4 = dmf > 0.0f ? q_round_clamp(mins[j] / dmf, 0, 15) : 0;
        b[j] = (uint8_t)(s4 | (m4 << 4));
        float ds = df * (float)s4, dm = dmf * (float)m4;
        for (int l = 0; l < 16; l++) {
            int w = 16 * j + l;
            int qv = ds > 0.0f ? q_round_clamp((x[w] + dm) / ds, 0, 3) : 0;
            int h = w >> 7, jj = (w >> 5) & 3, ll = w & 31;
            b[16 + 32 * h + ll] |= (uint8_t)(qv << (2 * jj));
        }
    }
    put16(b + 80, dh);
    put16(b + 82, dmh);
}

// Q3_K: symmetric 16-weight sub-blocks, signed 6-bit scales (stored +32),
// q in [-4,3] stored as two low bits in qs plus a high bit in hmask.
WM_HD void quant_block_q3_k(const float* x, uint8_t* b) {
#pragma clang fp contract(off)
    float scale[16], maxs = 0.0f;
    for (int j = 0; j < 16; j++) {
        float amax = 0.0f;
        for (int l = 0; l < 16; l++) amax = fmaxf(amax, fabsf(x[16 * j + l]));
        scale[j] = amax / 4.0f;
        maxs = fmaxf(maxs, scale[j]);
    }
    float d = maxs / 31.0f;
    uint16_t dh = f32_to_f16_bits(d);
    float df = f16_bits_to_f32(dh);
    uint8_t s6[16];
    for (int k = 0; k < 110; k++) b[k] = 0;
    for (int j = 0; j < 16; j++) {
        int sv = df > 0.0f ? q_round_clamp(scale[j] / df, 0, 31) : 0;
        s6[j] = (uint8_t)(sv + 32);
        float s = df * (float)sv;
        for (int l = 0; l < 16; l++) {
            int w = 16 * j + l;
            int u = (s > 0.0f ? q_round_clamp(x[w] / s, -4, 3) : 0) + 4;   // 0..7
            int h = w >> 7, jj = (w >> 5) & 3, ll = w & 31;
            b[32 + 32 * h + ll] |= (uint8_t)((u & 3) << (2 * jj));
            if (u >> 2) b[ll] |= (uint8_t)(1 << (4 * h + jj));
        }
    }
    for (int k = 0; k < 16; k++) {
        int lo = s6[k] & 0xF, hi = s6[k] >> 4;
        if (k < 8) b[96 + k] |= (uint8_t)lo;
        else b[96 + k - 8] |= (uint8_t)(lo << 4);
        b[96 + 8 + (k & 3)] |= (uint8_t)(hi << (2 * (k >> 2)));
    }
    put16(b + 108, dh);
}

WM_HD bool quant_block(int t, const float* x, uint8_t* b) {
    switch (t) {
    case Q8_0: quant_block_q8_0(x, b); return true;
    case Q2_K: quant_block_q2_k(x, b); return true;
    case Q3_K: quant_block_q3_k(x, b); return true;
    case Q4_K: quant_block_q4_k(x, b); return true;
    case Q5_K: quant_block_q5_k(x, b); return true;
    case Q6_K: quant_block_q6_k(x, b); return true;
    default: return false;
    }
}

}  // namespace wm
