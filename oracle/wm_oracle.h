/*
 * wm_oracle.h -- CPU oracle for the WinMoE MoE expert-layer hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the parity
 * reference (or, for the baseline, as the timed CPU restatement).  The product path in
 * winmoe_amd/ never calls it.
 *
 * Plain C, scalar, single-threaded unless noted.  Each function cites the
 * reference file:line it restates (paths relative to the reference root).
 */
#ifndef WM_ORACLE_H
#define WM_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ggml type ids (engine/runtime/gguf_parser.h:21-29, plus the public ggml ids
 * 10 = Q2_K and 11 = Q3_K, which the reference's table lacks). */
enum {
    WMO_F32 = 0, WMO_F16 = 1, WMO_Q8_0 = 8, WMO_Q2_K = 10, WMO_Q3_K = 11,
    WMO_Q4_K = 12, WMO_Q5_K = 13, WMO_Q6_K = 14
};

int   wmo_block_bytes(int qtype);   /* bytes per block, 0 if unsupported */
int   wmo_block_elems(int qtype);   /* weights per block, 0 if unsupported */

/* Exact IEEE half -> float (engine/runtime/iq2_dequant.h:22-40). */
float wmo_fp16_to_fp32(uint16_t h);

/* Dequantise nblocks raw blocks of qtype to fp32.  Returns 0, or -2 for an
 * unsupported type.  Formats: Q8_0 q8_dequant.h:15-18,116-126; Q4_K
 * q4k_dequant.h:28-60,129-155; Q5_K q5k_dequant.h:19-25,103-131; Q6_K
 * q6k_dequant.h:20-25,112-141; Q2_K / Q3_K: public ggml block format (no
 * reference implementation exists). */
int   wmo_dequant(int qtype, const void* blocks, int64_t nblocks, float* out);
/* Per-block sums of the dequantised values' 32-bit patterns: s1[i] plain,
 * s2[i] weighted by (position in the block + 1). */
int   wmo_dequant_block_sums(int qtype, const void* blocks, int64_t nblocks, int64_t* s1, int64_t* s2);

/* Router logits in the reference's fp32 order (transformer.h:172-191, default
 * case of quant_matvec): per row, 16 running fp32 FMA lanes over columns
 * c = l, l+16, ..., then a pairwise tree (l, l^8), (l, l^4), (l, l^2), (0, 1)
 * as _mm512_reduce_add_ps, then a scalar tail for H % 16 columns. */
void  wmo_router_logits(const float* x, const float* W, int H, int E, float* logits);

/* K-pass arg-max + softmax over the K picks (transformer.h:117-149).
 * Returns 1 when a pass found no logit above -1e30 (the reference then
 * re-picks index 0), else 0. */
int   wmo_topk_softmax(const float* logits, int E, int K, int32_t* ids, float* w);

/* Branch-stable sigmoid of deltanet_impl.h:108-115, evaluated in double. */
/* RMSNorm (attention.h:29-44): ss = sum of (double)x[i]^2 in index order,
 * scale = 1 / sqrtf((float)(ss / dim) + eps), out[i] = (x[i] * scale) * w[i]. */
void  wmo_rmsnorm(float* out, const float* x, const float* w, int dim, float eps);
double wmo_sigmoid(double x);

/* y[r] = sum_c dequant(W)[r][c] * x[c]: fp32 dequantised weights, fp64
 * accumulate (the verify_*.py style "numpy fp64" expert maths). */
int   wmo_matvec(int qtype, const void* W, const double* x, int rows, int in, double* y);

/* One expert: gate/up -> SwiGLU -> down, fp64 after fp32 dequant
 * (winmoe_inference.c:1932-1966).  act (optional, length I) receives the
 * SwiGLU output. */
int   wmo_expert_ffn(const void* gate, int gate_type, const void* up, int up_type,
                     const void* down, int down_type, const double* x, int H, int I,
                     double* y, double* act);

typedef struct {
    int32_t H, I, I_shared, E, K;
    int32_t gate_type, up_type, down_type;
    int32_t sh_gate_type, sh_up_type, sh_down_type;
    const float* router;       /* [E][H] fp32, NULL when routing is forced */
    const void* gate_exps;     /* stacked [E] x [I rows][H/QK blocks] */
    const void* up_exps;
    const void* down_exps;     /* stacked [E] x [H rows][I/QK blocks] */
    int64_t gate_stride, up_stride, down_stride;   /* bytes per expert */
    const void* sh_gate;       /* NULL = no shared expert */
    const void* sh_up;
    const void* sh_down;
    const float* sh_gate_inp;  /* [H] fp32 or NULL */
} wmo_layer;

/* The MoE block of winmoe_inference.c:1684-2027 for one token: router (unless
 * forced_ids != NULL, then ids/weights are taken from forced_ids/forced_w),
 * K experts, weighted combine in top-K order, shared expert with its sigmoid
 * gate (fp64 dot, :2005-2008).  out = moe_out before the residual add.
 * ids_out / w_out (length K) receive the routing used.  Returns the
 * degenerate-routing flag of wmo_topk_softmax, or -2 on bad arguments. */
int   wmo_moe_layer(const wmo_layer* L, const float* x, const int32_t* forced_ids,
                    const float* forced_w, int32_t* ids_out, float* w_out, double* out);

#ifdef __cplusplus
}
#endif
#endif
