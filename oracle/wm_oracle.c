/*
 * wm_oracle.c -- CPU oracle for the WinMoE MoE expert-layer hot path.
 *
 * TEST INFRASTRUCTURE ONLY (see wm_oracle.h): the parity reference the HIP
 * path is compared against, never the product.  Built with -ffp-contract=off so the
 * fp32 expressions below round exactly as written (the dequant products are
 * exact in fp32 either way; see the per-format notes).
 *
 * Pinning (tests/test_oracle.py):
 *   fp16          exhaustive over all 65536 patterns vs numpy, and vs the
 *                 reference's fp16_to_fp32 compiled from source (oracle/_ref)
 *   Q8_0          bit-exact vs reference q8_dequant_row (oracle/_ref)
 *   Q6_K          bit-exact vs reference q6k_dot_block with one-hot activations
 *   Q4_K / Q5_K   index map and values vs reference q4k_dot_q8k / q5k_dot_q8k
 *                 with exactly-representable one-hot activations; known answer
 *                 480 of test_q4k.c:21-40 in ggml layout
 *   Q2_K / Q3_K   parity unpinned against the reference (it has no code for
 *                 them); pinned by hand-built per-field blocks and quantise ->
 *                 dequantise round trips
 *   router        bit-exact vs reference router_topk (oracle/_ref), planted ties
 *   rmsnorm       closed forms (constant and one-hot rows: exact results) and
 *                 a sequential fp64 sum in numpy (the order matters only in
 *                 the last bits of ss); not compiled from the reference
 *                 (attention.h is an AVX2 header of the attention layer)
 *   expert / MoE  brute-force fp64 on tiny shapes vs an independent dense path
 */
#include "wm_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

int wmo_block_bytes(int t) {
    switch (t) {
    case WMO_F32: return 4;
    case WMO_F16: return 2;
    case WMO_Q8_0: return 34;
    case WMO_Q2_K: return 84;
    case WMO_Q3_K: return 110;
    case WMO_Q4_K: return 144;
    case WMO_Q5_K: return 176;
    case WMO_Q6_K: return 210;
    default: return 0;
    }
}

int wmo_block_elems(int t) {
    switch (t) {
    case WMO_F32: case WMO_F16: return 1;
    case WMO_Q8_0: return 32;
    case WMO_Q2_K: case WMO_Q3_K: case WMO_Q4_K: case WMO_Q5_K: case WMO_Q6_K: return 256;
    default: return 0;
    }
}

static uint16_t rd16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* engine/runtime/iq2_dequant.h:22-40: subnormals via ldexpf(mant, -24),
 * +-inf, any NaN -> NAN, normals ldexpf(mant + 1024, exp - 25). */
float wmo_fp16_to_fp32(uint16_t h) {
    uint32_t sign = (h >> 15) & 1u, ex = (h >> 10) & 0x1fu, mant = h & 0x3ffu;
    if (ex == 0) {
        if (mant == 0) return sign ? -0.0f : 0.0f;
        float v = ldexpf((float)mant, -24);
        return sign ? -v : v;
    }
    if (ex == 0x1f) {
        if (mant == 0) return sign ? -INFINITY : INFINITY;
        return NAN;
    }
    float v = ldexpf((float)(mant + 1024), (int)ex - 25);
    return sign ? -v : v;
}

/* Q4_K / Q5_K 6-bit scale and min of sub-block i (q4k_dequant.h:43-60). */
static void k4_scale_min(const uint8_t* s, int i, int* sc, int* m) {
    if (i < 4) {
        *sc = s[i] & 63;
        *m = s[i + 4] & 63;
    } else {
        *sc = (s[i + 4] & 0xF) | ((s[i - 4] >> 6) << 4);
        *m = (s[i + 4] >> 4) | ((s[i] >> 6) << 4);
    }
}

/* Q8_0: {u16 d; i8 qs[32]}, w = d * q (q8_dequant.h:15-18,116-126). */
static void dq_q8_0(const uint8_t* b, float* y) {
    float d = wmo_fp16_to_fp32(rd16(b));
    for (int j = 0; j < 32; j++) y[j] = d * (float)(int8_t)b[2 + j];
}

/* Q4_K: {u16 d; u16 dmin; u8 scales[12]; u8 qs[128]}.  Chunk c holds 32 bytes:
 * low nibble j -> weight 64c+j (sub-block 2c), high nibble -> 64c+32+j
 * (sub-block 2c+1) (q4k_dequant.h:129-155, gpu_offload.cu:373-389).
 * d*sc*q and dmin*m are exact in fp32; the subtraction rounds once. */
static void dq_q4_k(const uint8_t* b, float* y) {
    float d = wmo_fp16_to_fp32(rd16(b)), dmin = wmo_fp16_to_fp32(rd16(b + 2));
    const uint8_t* sc = b + 4; const uint8_t* qs = b + 16;
    for (int c = 0; c < 4; c++) {
        int s0, m0, s1, m1;
        k4_scale_min(sc, 2 * c, &s0, &m0);
        k4_scale_min(sc, 2 * c + 1, &s1, &m1);
        float a0 = d * (float)s0, b0 = dmin * (float)m0;
        float a1 = d * (float)s1, b1 = dmin * (float)m1;
        for (int j = 0; j < 32; j++) {
            uint8_t q = qs[32 * c + j];
            y[64 * c + j] = a0 * (float)(q & 0xF) - b0;
            y[64 * c + 32 + j] = a1 * (float)(q >> 4) - b1;
        }
    }
}

/* Q5_K: {u16 d; u16 dmin; u8 scales[12]; u8 qh[32]; u8 qs[128]}; as Q4_K plus
 * bit (2c) / (2c+1) of qh[j] as the fifth bit (q5k_dequant.h:98-131). */
static void dq_q5_k(const uint8_t* b, float* y) {
    float d = wmo_fp16_to_fp32(rd16(b)), dmin = wmo_fp16_to_fp32(rd16(b + 2));
    const uint8_t* sc = b + 4; const uint8_t* qh = b + 16; const uint8_t* qs = b + 48;
    for (int c = 0; c < 4; c++) {
        int s0, m0, s1, m1;
        k4_scale_min(sc, 2 * c, &s0, &m0);
        k4_scale_min(sc, 2 * c + 1, &s1, &m1);
        float a0 = d * (float)s0, b0 = dmin * (float)m0;
        float a1 = d * (float)s1, b1 = dmin * (float)m1;
        for (int j = 0; j < 32; j++) {
            uint8_t q = qs[32 * c + j];
            int lo = (q & 0xF) | (((qh[j] >> (2 * c)) & 1) << 4);
            int hi = (q >> 4) | (((qh[j] >> (2 * c + 1)) & 1) << 4);
            y[64 * c + j] = a0 * (float)lo - b0;
            y[64 * c + 32 + j] = a1 * (float)hi - b1;
        }
    }
}

/* Q6_K: {u8 ql[128]; u8 qh[64]; i8 scales[16]; u16 d} with d LAST
 * (q6k_dequant.h:20-25, scalar dot :112-141 with is = n/16 + l/16).
 * d*sc*(q-32) is exact in fp32 (|sc*(q-32)| <= 4096). */
static void dq_q6_k(const uint8_t* b, float* y) {
    const uint8_t* ql = b; const uint8_t* qh = b + 128; const int8_t* sc = (const int8_t*)(b + 192);
    float d = wmo_fp16_to_fp32(rd16(b + 208));
    for (int n = 0; n < 256; n += 128) {
        for (int l = 0; l < 32; l++) {
            int is = n / 16 + l / 16;
            int q1 = (ql[n / 2 + l] & 0xF) | (((qh[n / 4 + l] >> 0) & 3) << 4);
            int q2 = (ql[n / 2 + l + 32] & 0xF) | (((qh[n / 4 + l] >> 2) & 3) << 4);
            int q3 = (ql[n / 2 + l] >> 4) | (((qh[n / 4 + l] >> 4) & 3) << 4);
            int q4 = (ql[n / 2 + l + 32] >> 4) | (((qh[n / 4 + l] >> 6) & 3) << 4);
            y[n + l] = d * (float)sc[is + 0] * (float)(q1 - 32);
            y[n + l + 32] = d * (float)sc[is + 2] * (float)(q2 - 32);
            y[n + l + 64] = d * (float)sc[is + 4] * (float)(q3 - 32);
            y[n + l + 96] = d * (float)sc[is + 6] * (float)(q4 - 32);
        }
    }
}

/* Q2_K (public ggml format): {u8 scales[16]; u8 qs[64]; u16 d; u16 dmin}.
 * Half h, group j (shift 2j): weights 128h+32j+l, l<16 use scales[8h+2j],
 * l>=16 use scales[8h+2j+1]; 2-bit q = (qs[32h+l] >> 2j) & 3;
 * w = d*(sc & 15)*q - dmin*(sc >> 4). */
static void dq_q2_k(const uint8_t* b, float* y) {
    const uint8_t* scales = b; const uint8_t* qs = b + 16;
    float d = wmo_fp16_to_fp32(rd16(b + 80)), dmin = wmo_fp16_to_fp32(rd16(b + 82));
    for (int h = 0; h < 2; h++) {
        for (int j = 0; j < 4; j++) {
            for (int l = 0; l < 32; l++) {
                uint8_t s = scales[8 * h + 2 * j + (l >> 4)];
                float dl = d * (float)(s & 0xF), ml = dmin * (float)(s >> 4);
                int q = (qs[32 * h + l] >> (2 * j)) & 3;
                y[128 * h + 32 * j + l] = dl * (float)q - ml;
            }
        }
    }
}

/* Q3_K sixteen 6-bit scales from the 12 packed bytes: low nibble from byte k
 * (k < 8) or the high nibble of byte k-8, high two bits from byte 8 + (k & 3)
 * at shift 2*(k >> 2); value minus 32. */
static int q3_scale(const uint8_t* s, int k) {
    int lo = (k < 8) ? (s[k] & 0xF) : (s[k - 8] >> 4);
    int hi = (s[8 + (k & 3)] >> (2 * (k >> 2))) & 3;
    return (lo | (hi << 4)) - 32;
}

/* Q3_K (public ggml format): {u8 hmask[32]; u8 qs[64]; u8 scales[12]; u16 d}.
 * Half h, group j: weights 128h+32j+l; q = ((qs[32h+l] >> 2j) & 3) - 4 unless
 * bit (4h+j) of hmask[l] is set; scale index 8h+2j+(l >= 16). */
static void dq_q3_k(const uint8_t* b, float* y) {
    const uint8_t* hm = b; const uint8_t* qs = b + 32; const uint8_t* sc = b + 96;
    float d = wmo_fp16_to_fp32(rd16(b + 108));
    for (int h = 0; h < 2; h++) {
        for (int j = 0; j < 4; j++) {
            for (int l = 0; l < 32; l++) {
                float dl = d * (float)q3_scale(sc, 8 * h + 2 * j + (l >> 4));
                int q = ((qs[32 * h + l] >> (2 * j)) & 3) - ((hm[l] & (1 << (4 * h + j))) ? 0 : 4);
                y[128 * h + 32 * j + l] = dl * (float)q;
            }
        }
    }
}

int wmo_dequant(int qtype, const void* blocks, int64_t nblocks, float* out) {
    const uint8_t* p = (const uint8_t*)blocks;
    int bs = wmo_block_bytes(qtype), ne = wmo_block_elems(qtype);
    if (bs == 0 || nblocks < 0) return -2;
    for (int64_t i = 0; i < nblocks; i++) {
        const uint8_t* b = p + i * bs;
        float* y = out + i * ne;
        switch (qtype) {
        case WMO_F32: memcpy(y, b, 4); break;
        case WMO_F16: y[0] = wmo_fp16_to_fp32(rd16(b)); break;
        case WMO_Q8_0: dq_q8_0(b, y); break;
        case WMO_Q2_K: dq_q2_k(b, y); break;
        case WMO_Q3_K: dq_q3_k(b, y); break;
        case WMO_Q4_K: dq_q4_k(b, y); break;
        case WMO_Q5_K: dq_q5_k(b, y); break;
        case WMO_Q6_K: dq_q6_k(b, y); break;
        default: return -2;
        }
    }
    return 0;
}

/* Per-block checksums of the dequantised values, for comparing a whole
 * expert stack with a device dequantisation without moving the fp32 values:
 * s1[i] = sum of the 32-bit patterns of block i's values, s2[i] = sum of
 * (j + 1) * pattern of value j.  A value that differs changes s1. */
int wmo_dequant_block_sums(int qtype, const void* blocks, int64_t nblocks, int64_t* s1, int64_t* s2) {
    const int bs = wmo_block_bytes(qtype), ne = wmo_block_elems(qtype);
    if (bs == 0 || nblocks < 0 || ne > 256) return -2;
    float y[256];
    const uint8_t* p = (const uint8_t*)blocks;
    for (int64_t i = 0; i < nblocks; i++) {
        int rc = wmo_dequant(qtype, p + i * bs, 1, y);
        if (rc) return rc;
        int64_t a = 0, b = 0;
        for (int j = 0; j < ne; j++) {
            uint32_t u;
            memcpy(&u, &y[j], 4);
            a += (int64_t)u;
            b += (int64_t)(j + 1) * (int64_t)u;
        }
        s1[i] = a;
        s2[i] = b;
    }
    return 0;
}

/* transformer.h:172-191 default case: AVX-512 16-lane FMA accumulation, then
 * _mm512_reduce_add_ps (GCC avx512fintrin.h: halves, quarters, then lanes
 * {0,2},{1,3}, then 0+1), then the scalar tail `s += row[c] * x[c]`, which
 * GCC contracts to an FMA under -mfma (restated as fmaf). */
void wmo_router_logits(const float* x, const float* W, int H, int E, float* logits) {
    for (int r = 0; r < E; r++) {
        const float* row = W + (int64_t)r * H;
        float acc[16] = {0};
        int c;
        for (c = 0; c + 15 < H; c += 16)
            for (int l = 0; l < 16; l++) acc[l] = fmaf(row[c + l], x[c + l], acc[l]);
        float t3[8], t6[4];
        for (int i = 0; i < 8; i++) t3[i] = acc[i + 8] + acc[i];
        for (int i = 0; i < 4; i++) t6[i] = t3[i + 4] + t3[i];
        float t8_0 = t6[0] + t6[2], t8_1 = t6[1] + t6[3];
        float s = t8_0 + t8_1;
        for (; c < H; c++) s = fmaf(row[c], x[c], s);
        logits[r] = s;
    }
}

/* transformer.h:117-149. */
int wmo_topk_softmax(const float* logits, int E, int K, int32_t* ids, float* w) {
    int degenerate = 0;
    for (int k = 0; k < K; k++) {
        float best = -1e30f;
        int best_idx = 0, found = 0;
        for (int e = 0; e < E; e++) {
            int already = 0;
            for (int j = 0; j < k; j++) if (ids[j] == e) { already = 1; break; }
            if (!already && logits[e] > best) { best = logits[e]; best_idx = e; found = 1; }
        }
        if (!found) degenerate = 1;
        ids[k] = best_idx;
        w[k] = logits[best_idx];
    }
    float wmax = w[0];
    for (int k = 1; k < K; k++) if (w[k] > wmax) wmax = w[k];
    float wsum = 0.0f;
    for (int k = 0; k < K; k++) { w[k] = expf(w[k] - wmax); wsum += w[k]; }
    if (wsum > 0) for (int k = 0; k < K; k++) w[k] /= wsum;
    return degenerate;
}

/* deltanet_impl.h:108-115 in double precision. */
double wmo_sigmoid(double x) {
    if (x >= 0.0) return 1.0 / (1.0 + exp(-x));
    double z = exp(x);
    return z / (1.0 + z);
}

int wmo_matvec(int qtype, const void* W, const double* x, int rows, int in, double* y) {
    int bs = wmo_block_bytes(qtype), ne = wmo_block_elems(qtype);
    if (bs == 0 || rows < 0 || in <= 0 || in % ne) return -2;
    int64_t nb = in / ne, row_bytes = nb * bs;
    float* wrow = (float*)malloc(sizeof(float) * (size_t)in);
    if (!wrow) return -1;
    for (int r = 0; r < rows; r++) {
        wmo_dequant(qtype, (const uint8_t*)W + (int64_t)r * row_bytes, nb, wrow);
        double s = 0.0;
        for (int c = 0; c < in; c++) s += (double)wrow[c] * x[c];
        y[r] = s;
    }
    free(wrow);
    return 0;
}

/* winmoe_inference.c:1932-1966: gate, up, act = g * sigmoid(g) * u, down. */
int wmo_expert_ffn(const void* gate, int gt, const void* up, int ut, const void* down, int dt,
                   const double* x, int H, int I, double* y, double* act_out) {
    double* g = (double*)malloc(sizeof(double) * (size_t)I * 3);
    if (!g) return -1;
    double *u = g + I, *a = g + 2 * I;
    int rc = wmo_matvec(gt, gate, x, I, H, g);
    if (!rc) rc = wmo_matvec(ut, up, x, I, H, u);
    if (!rc) {
        for (int i = 0; i < I; i++) a[i] = g[i] * wmo_sigmoid(g[i]) * u[i];
        rc = wmo_matvec(dt, down, a, H, I, y);
        if (act_out) memcpy(act_out, a, sizeof(double) * (size_t)I);
    }
    free(g);
    return rc;
}

static int64_t mat_bytes(int qtype, int rows, int in) {
    return (int64_t)rows * (in / wmo_block_elems(qtype)) * wmo_block_bytes(qtype);
}

/* winmoe_inference.c:1684-2027 for one token. */
int wmo_moe_layer(const wmo_layer* L, const float* x, const int32_t* forced_ids,
                  const float* forced_w, int32_t* ids, float* w, double* out) {
    int H = L->H, I = L->I, K = L->K, E = L->E, degenerate = 0;
    if (H <= 0 || I <= 0 || K <= 0 || K > E) return -2;
    double* xd = (double*)malloc(sizeof(double) * (size_t)(H * 2));
    if (!xd) return -1;
    double* y = xd + H;
    for (int h = 0; h < H; h++) xd[h] = x[h];
    if (forced_ids) {
        for (int k = 0; k < K; k++) { ids[k] = forced_ids[k]; w[k] = forced_w[k]; }
    } else {
        float* logits = (float*)malloc(sizeof(float) * (size_t)E);
        if (!logits) { free(xd); return -1; }
        wmo_router_logits(x, L->router, H, E, logits);
        degenerate = wmo_topk_softmax(logits, E, K, ids, w);
        free(logits);
    }
    int64_t gs = L->gate_stride ? L->gate_stride : mat_bytes(L->gate_type, I, H);
    int64_t us = L->up_stride ? L->up_stride : mat_bytes(L->up_type, I, H);
    int64_t ds = L->down_stride ? L->down_stride : mat_bytes(L->down_type, H, I);
    for (int h = 0; h < H; h++) out[h] = 0.0;
    int rc = 0;
    for (int k = 0; k < K && !rc; k++) {
        int e = ids[k];
        rc = wmo_expert_ffn((const uint8_t*)L->gate_exps + e * gs, L->gate_type,
                            (const uint8_t*)L->up_exps + e * us, L->up_type,
                            (const uint8_t*)L->down_exps + e * ds, L->down_type,
                            xd, H, I, y, NULL);
        for (int h = 0; h < H; h++) out[h] += (double)w[k] * y[h];
    }
    if (!rc && L->sh_gate && L->sh_up && L->sh_down) {
        int Is = L->I_shared > 0 ? L->I_shared : I;
        rc = wmo_expert_ffn(L->sh_gate, L->sh_gate_type, L->sh_up, L->sh_up_type,
                            L->sh_down, L->sh_down_type, xd, H, Is, y, NULL);
        double gate = 1.0;
        if (L->sh_gate_inp) {
            double s = 0.0;
            for (int h = 0; h < H; h++) s += (double)L->sh_gate_inp[h] * xd[h];
            gate = wmo_sigmoid(s);
        }
        for (int h = 0; h < H; h++) out[h] += gate * y[h];
    }
    free(xd);
    return rc ? rc : degenerate;
}

void wmo_rmsnorm(float* out, const float* x, const float* w, int dim, float eps) {
    double ss = 0.0;
    for (int i = 0; i < dim; i++) ss += (double)x[i] * (double)x[i];
    const float scale = 1.0f / sqrtf((float)(ss / dim) + eps);
    for (int i = 0; i < dim; i++) out[i] = (x[i] * scale) * w[i];
}
