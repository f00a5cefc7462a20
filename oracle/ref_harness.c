/*
 * ref_harness.c -- exports the reference's own CPU hot-path kernels, compiled
 * from the reference sources where they lie (engine/runtime/*.h, included via
 * -I by oracle/Makefile), into oracle/_ref/libwmref.so.
 *
 * TEST INFRASTRUCTURE ONLY: used by tests/ to pin the oracle and by bench.py's
 * cpu_baseline leg as the timed reference CPU path.  Nothing here is copied
 * from the reference; the reference headers are #included unmodified.
 *
 * Buildability: the headers are MSVC-oriented.  The functions this file calls
 * compile with GCC as-is.  q8_matvec / q4k_matvec / q5k_matvec use the
 * MSVC-only _malloca/_freea and are never called (GCC only warns about the
 * implicit declaration and emits no code for the unused static inline
 * functions); oracle/Makefile fails the build if any such symbol is left
 * undefined in the library.  The loops that wrap the reference block kernels
 * below restate the reference's own loops (cited), because the wrappers that
 * contain them are among the uncallable functions.
 */
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "iq2xxs_grid_def.h"
#include "iq2_dequant.h"     /* fp16_to_fp32 :22-40 */
#include "q8k_quant.h"       /* block_q8_K, quantize_row_q8_K :32-104 */
#include "q8_dequant.h"      /* block_q8_0, q8_dot_block, q8_dot_q8k, q8_dequant_row */
#include "q4k_dequant.h"     /* block_q4_K, decode_q4k_scales, q4k_dot_q8k, q4k_matvec_q8k */
#include "q5k_dequant.h"     /* block_q5_K, q5k_dot_q8k, q5k_matvec_q8k */
#include "q6k_dequant.h"     /* block_q6_K, q6k_dot_block(_avx2) */
#include "gguf_parser.h"     /* GGML_TYPE_* ids used by transformer.h */
#include "transformer.h"     /* router_topk :107-152 */
#include "deltanet_impl.h"   /* sigmoid_stable :108-115 */
#include "attention.h"       /* rmsnorm :29-44 */

#include "wm_oracle.h"       /* wmo_layer descriptor, Q2_K/Q3_K dequant (port) */

#define REF_API __attribute__((visibility("default")))

REF_API float ref_fp16_to_fp32(uint16_t h) { return fp16_to_fp32(h); }

REF_API void ref_q8_dequant_row(const void* data, int n, float* out) { q8_dequant_row(out, data, n); }

REF_API float ref_q6k_dot_block(const void* blk, const float* y) { return q6k_dot_block((const block_q6_K*)blk, y); }

REF_API float ref_q6k_dot_block_avx2(const void* blk, const float* y) {
    return q6k_dot_block_avx2((const block_q6_K*)blk, y);
}

REF_API void ref_decode_q4k_scales(const uint8_t* q, uint8_t* scales, uint8_t* mins) {
    decode_q4k_scales(q, scales, mins);
}

REF_API void ref_quantize_row_q8_K(const float* x, int n, void* out) {
    quantize_row_q8_K((block_q8_K*)out, x, n);
}

REF_API int ref_sizeof_block_q8_K(void) { return (int)sizeof(block_q8_K); }

/* One 256-weight Q4_K block dotted with x (quantised to Q8_K first, as every
 * reference caller does: q4k_matvec q4k_dequant.h:197, winmoe_inference.c:1702). */
REF_API float ref_q4k_dot_q8k(const void* blk, const float* x256) {
    block_q8_K a;
    quantize_row_q8_K(&a, x256, 256);
    return q4k_dot_q8k((const block_q4_K*)blk, &a);
}

REF_API float ref_q5k_dot_q8k(const void* blk, const float* x256) {
    block_q8_K a;
    quantize_row_q8_K(&a, x256, 256);
    return q5k_dot_q8k((const block_q5_K*)blk, &a);
}

REF_API float ref_q8_dot_block(const void* blk, const float* y32) { return q8_dot_block((const block_q8_0*)blk, y32); }

REF_API float ref_sigmoid_stable(float x) { return sigmoid_stable(x); }

/* The reference router: fp32 logits (quant_matvec default case), K-pass
 * arg-max, softmax over the K picks.  Single call site, constant gate_type 0
 * (F32), so only the fp32 branch of quant_matvec is instantiated. */
REF_API void ref_router_topk(const float* x, const float* W, int H, int E, int K, int32_t* ids, float* w) {
    int tmp_ids[64];
    float tmp_w[64];
    router_topk(x, W, 0, H, E, K, tmp_ids, tmp_w);
    for (int k = 0; k < K; k++) { ids[k] = tmp_ids[k]; w[k] = tmp_w[k]; }
}

/* ---------------------------------------------------------------------- */
/* Reference CPU matvec dispatch (transformer.h:157-194).  The Q8_0 branch
 * restates q8_matvec (q8_dequant.h:63-113) around the reference q8_dot_q8k /
 * q8_dot_block; Q4_K / Q5_K quantise x to Q8_K then call the reference
 * q4k_matvec_q8k / q5k_matvec_q8k (= q4k_matvec / q5k_matvec :174-210);
 * Q6_K restates q6k_matvec (q6k_dequant.h:145-176) around
 * q6k_dot_block_avx2.  Q2_K / Q3_K have no reference kernel: the port
 * dequantises each row (oracle) and dots in fp32; *used_port is set. */
static int g_used_port = 0;

static void ref_matvec(float* out, const void* W, const float* x, int out_dim, int in_dim, int type) {
    switch (type) {
    case GGML_TYPE_Q8_0: {
        int blocks_per_row = in_dim / Q8_QK;
        const block_q8_0* blocks = (const block_q8_0*)W;
        int q8k_blocks = in_dim / Q8K_QK;
        block_q8_K* x_q8k = NULL;
        if (q8k_blocks > 0 && out_dim >= 128) {
            x_q8k = (block_q8_K*)malloc((size_t)q8k_blocks * sizeof(block_q8_K));
            if (x_q8k) quantize_row_q8_K(x_q8k, x, q8k_blocks * Q8K_QK);
        }
        int row;
        #pragma omp parallel for schedule(static) if(out_dim >= 128)
        for (row = 0; row < out_dim; row++) {
            float sum = 0.0f;
            const block_q8_0* row_blocks = &blocks[(int64_t)row * blocks_per_row];
            if (x_q8k) {
                for (int qb = 0; qb < q8k_blocks; qb++) {
                    for (int sb = 0; sb < 8; sb++) {
                        int bidx = qb * 8 + sb;
                        if (bidx < blocks_per_row) {
                            block_q8_K mini;
                            mini.d = x_q8k[qb].d;
                            memcpy(mini.qs, x_q8k[qb].qs + sb * 32, 32);
                            sum += q8_dot_q8k(&row_blocks[bidx], &mini);
                        }
                    }
                }
            } else {
                for (int b = 0; b < blocks_per_row; b++) sum += q8_dot_block(&row_blocks[b], &x[b * Q8_QK]);
            }
            out[row] = sum;
        }
        free(x_q8k);
        break;
    }
    case GGML_TYPE_Q4_K:
    case GGML_TYPE_Q5_K: {
        int nb = in_dim / Q8K_QK;
        block_q8_K* xq = (block_q8_K*)malloc((size_t)nb * sizeof(block_q8_K));
        quantize_row_q8_K(xq, x, in_dim);
        if (type == GGML_TYPE_Q4_K) q4k_matvec_q8k(out, W, xq, out_dim, in_dim);
        else q5k_matvec_q8k(out, W, xq, out_dim, in_dim);
        free(xq);
        break;
    }
    case GGML_TYPE_Q6_K: {
        int blocks_per_row = in_dim / Q6K_QK;
        const block_q6_K* blocks = (const block_q6_K*)W;
        int row;
        #pragma omp parallel for schedule(static) if(out_dim >= 128)
        for (row = 0; row < out_dim; row++) {
            float sum = 0.0f;
            const block_q6_K* row_blocks = &blocks[(int64_t)row * blocks_per_row];
            for (int b = 0; b < blocks_per_row; b++) sum += q6k_dot_block_avx2(&row_blocks[b], &x[b * Q6K_QK]);
            out[row] = sum;
        }
        break;
    }
    default: { /* WMO_Q2_K / WMO_Q3_K: port */
        int ne = wmo_block_elems(type), bs = wmo_block_bytes(type);
        int nb = in_dim / ne;
        g_used_port = 1;
        int row;
        #pragma omp parallel for schedule(static) if(out_dim >= 128)
        for (row = 0; row < out_dim; row++) {
            float wrow[4096 * 4];
            float sum = 0.0f;
            wmo_dequant(type, (const uint8_t*)W + (int64_t)row * nb * bs, nb, wrow);
            for (int c = 0; c < in_dim; c++) sum += wrow[c] * x[c];
            out[row] = sum;
        }
        break;
    }
    }
}

static int64_t ref_mat_bytes(int qtype, int rows, int in) {
    return (int64_t)rows * (in / wmo_block_elems(qtype)) * wmo_block_bytes(qtype);
}

/* The MoE block of winmoe_inference.c:1684-2027 for one token, with the cache
 * and I/O machinery removed (all experts resident in RAM): router_topk, the
 * fused Q4_K gate+up loop (:1907-1930) or quant_matvec, SwiGLU with
 * sigmoid_stable (:1936-1940), down (:1958-1966, Q5_K via Q8_K), the AVX2 FMA
 * accumulate (:1971-1980), and the shared expert with its fp64 gate dot
 * (:1990-2027).  out receives moe_out before the residual add.
 * Returns 1 if a Q2_K/Q3_K port kernel was used, 0 otherwise, -2 on bad args. */
REF_API int ref_moe_layer_cpu(const wmo_layer* L, const float* normed, const int32_t* forced_ids,
                              const float* forced_w, int32_t* ids_out, float* w_out, float* moe_out) {
    int H = L->H, I = L->I, K = L->K, E = L->E, i;
    if (H <= 0 || I <= 0 || K <= 0 || K > E || K > 64 || H > 16384 || I > 16384) return -2;
    g_used_port = 0;
    int32_t expert_ids[64];
    float expert_weights[64];
    if (forced_ids) {
        for (i = 0; i < K; i++) { expert_ids[i] = forced_ids[i]; expert_weights[i] = forced_w[i]; }
    } else {
        ref_router_topk(normed, L->router, H, E, K, expert_ids, expert_weights);
    }
    int q8k_blocks = H / Q8K_QK;
    block_q8_K* normed_q8k = (block_q8_K*)malloc((size_t)q8k_blocks * sizeof(block_q8_K));
    if (normed_q8k) quantize_row_q8_K(normed_q8k, normed, H);
    float* gate_buf = (float*)malloc(sizeof(float) * (size_t)(3 * I + H));
    float* up_buf = gate_buf + I;
    float* act_buf = up_buf + I;
    float* expert_out = act_buf + I;
    int64_t gs = L->gate_stride ? L->gate_stride : ref_mat_bytes(L->gate_type, I, H);
    int64_t us = L->up_stride ? L->up_stride : ref_mat_bytes(L->up_type, I, H);
    int64_t ds = L->down_stride ? L->down_stride : ref_mat_bytes(L->down_type, H, I);
    memset(moe_out, 0, (size_t)H * sizeof(float));
    for (int ek = 0; ek < K; ek++) {
        int eid = expert_ids[ek];
        const uint8_t* gate_data = (const uint8_t*)L->gate_exps + eid * gs;
        const uint8_t* up_data = (const uint8_t*)L->up_exps + eid * us;
        const uint8_t* down_data = (const uint8_t*)L->down_exps + eid * ds;
        if (normed_q8k && L->gate_type == GGML_TYPE_Q4_K && L->up_type == GGML_TYPE_Q4_K) {
            int bpr = H / Q4K_QK;
            const block_q4_K* gw = (const block_q4_K*)gate_data;
            const block_q4_K* uw = (const block_q4_K*)up_data;
            int frow;
            #pragma omp parallel for schedule(static)
            for (frow = 0; frow < I; frow++) {
                if (frow + 1 < I) {
                    _mm_prefetch((const char*)&gw[(frow + 1) * bpr], _MM_HINT_T0);
                    _mm_prefetch((const char*)&uw[(frow + 1) * bpr], _MM_HINT_T0);
                }
                float gsum = 0.0f, usum = 0.0f;
                for (int fb = 0; fb < bpr; fb++) {
                    gsum += q4k_dot_q8k(&gw[frow * bpr + fb], &normed_q8k[fb]);
                    usum += q4k_dot_q8k(&uw[frow * bpr + fb], &normed_q8k[fb]);
                }
                gate_buf[frow] = gsum;
                up_buf[frow] = usum;
            }
        } else {
            ref_matvec(gate_buf, gate_data, normed, I, H, L->gate_type);
            ref_matvec(up_buf, up_data, normed, I, H, L->up_type);
        }
        for (i = 0; i < I; i++) {
            float g = gate_buf[i];
            act_buf[i] = g * sigmoid_stable(g) * up_buf[i];
        }
        if (L->down_type == GGML_TYPE_Q5_K) {
            block_q8_K act_q8k[64];
            quantize_row_q8_K(act_q8k, act_buf, I);
            q5k_matvec_q8k(expert_out, down_data, act_q8k, H, I);
        } else {
            ref_matvec(expert_out, down_data, act_buf, H, I, L->down_type);
        }
        {
            __m256 vw = _mm256_set1_ps(expert_weights[ek]);
            for (i = 0; i + 7 < H; i += 8) {
                __m256 vm = _mm256_loadu_ps(moe_out + i);
                __m256 ve = _mm256_loadu_ps(expert_out + i);
                _mm256_storeu_ps(moe_out + i, _mm256_fmadd_ps(vw, ve, vm));
            }
            for (; i < H; i++) moe_out[i] += expert_weights[ek] * expert_out[i];
        }
    }
    if (L->sh_gate && L->sh_up && L->sh_down) {
        /* The reference sizes the shared expert with the routed I
         * (winmoe_inference.c:1992-1993, 2002); the configs here have
         * I_shared == I. */
        int Is = L->I_shared > 0 ? L->I_shared : I;
        ref_matvec(gate_buf, L->sh_gate, normed, Is, H, L->sh_gate_type);
        ref_matvec(up_buf, L->sh_up, normed, Is, H, L->sh_up_type);
        for (i = 0; i < Is; i++) {
            float g = gate_buf[i];
            act_buf[i] = g * sigmoid_stable(g) * up_buf[i];
        }
        ref_matvec(expert_out, L->sh_down, act_buf, H, Is, L->sh_down_type);
        if (L->sh_gate_inp) {
            double gate_scalar = 0.0;
            for (i = 0; i < H; i++) gate_scalar += (double)L->sh_gate_inp[i] * (double)normed[i];
            float sig_gate = sigmoid_stable((float)gate_scalar);
            for (i = 0; i < H; i++) expert_out[i] *= sig_gate;
        }
        for (i = 0; i + 7 < H; i += 8) {
            __m256 vm = _mm256_loadu_ps(moe_out + i);
            __m256 ve = _mm256_loadu_ps(expert_out + i);
            _mm256_storeu_ps(moe_out + i, _mm256_add_ps(vm, ve));
        }
        for (; i < H; i++) moe_out[i] += expert_out[i];
    }
    for (i = 0; i < K; i++) { ids_out[i] = expert_ids[i]; w_out[i] = expert_weights[i]; }
    free(gate_buf);
    free(normed_q8k);
    return g_used_port;
}

/* attention.h:29-44, as compiled from the reference (eps fixed at 1e-6 there). */
void wmref_rmsnorm(float* out, const float* x, const float* w, int dim) { rmsnorm(out, x, w, dim); }
