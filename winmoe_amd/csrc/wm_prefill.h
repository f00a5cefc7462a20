// wm_prefill.h -- arguments of the batched prefill kernels (wm_prefill.hip).
// Internal; not part of the public ABI.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "wm_format.h"

namespace wm {

// A (token, slot) pair p = t * K + k is one routed use of an expert; pair
// T * K + t is token t's use of the shared expert.
struct PrefillArgs {
    int32_t H, I, Is, E, K, T, has_shared;
    int32_t gt, dt, sgt, sdt;   // weight formats: routed gate = up, down; shared gate = up, down
    const uint16_t* x;          // bf16 [T][H]
    const float* router;        // fp32 [E][H]
    const uint8_t* gate;
    const uint8_t* up;
    const uint8_t* down;
    int64_t gstride, ustride, dstride;
    const uint8_t* sh_gate;
    const uint8_t* sh_up;
    const uint8_t* sh_down;
    const float* sh_gate_inp;   // fp32 [H] or NULL
    int32_t* ids;               // [T][K]
    float* w;                   // [T][K]
    float* logits;              // [T][E]
    uint32_t* hits;             // [E]
    int32_t* status;
    int32_t* offsets;           // [E + 2]: pairs of expert e are sorted[offsets[e] .. offsets[e + 1]); shared: [E] .. [E + 1]
    int32_t* sorted;            // [T * K + T] pair indices grouped by expert
    int32_t* passes;            // [prefill_max_passes][64] pass records (up to pass_m pairs of one expert)
    int32_t* pass_count;        // [2]: routed passes, shared passes
    uint16_t* x16;              // fp16 [T][H]: x * 2^-e per token
    int32_t* xexp;              // [T]: e
    uint16_t* act_hi;           // fp16 [pairs][act_stride]: SwiGLU output = (hi + lo) * 2^e per (pair, 128 rows)
    uint16_t* act_lo;
    float* act_sc;              // [pairs][act_stride / 128]: 2^e
    int64_t act_stride;
    float* y;                   // [pairs][H] expert outputs
    float* sg;                  // [T] shared-expert gate
    float* out;                 // [T][H]
    int32_t n_wg;               // workgroups of the persistent expert GEMMs (one per CU)
    int32_t pass_m;             // pairs per pass: 16 or 32 (prefill_pass_size)
};

// Pass records a prefill of T tokens may need (passes of 16 pairs or more).
inline int64_t prefill_max_passes(int64_t T, int64_t K, int64_t E) { return (T * K + 15) / 16 + E + (T + 15) / 16 + 1; }

// Pairs per pass: 16 when the batch averages at most 10 (Q8_0 gate/up) or 4
// (K-quant gate/up) pairs per routed expert, else 32.  Passes of 16 have
// smaller activation slots (LDS for a deeper weight ring) and a lighter
// stage; passes of 32 stream a busy expert's rows half as often.  Measured
// with Zipf routing over 512 experts (ms per batch, 16 / 32): Q8_0 at 10
// pairs per expert 1.54 / 1.56, at 20 2.16 / 1.80; Q4_K gate/up, Q6_K down
// at 3 pairs 1.45 / 1.54, at 12 2.14 / 1.95.
inline int prefill_pass_size(int64_t T, int64_t K, int64_t E, int gate_type) {
    return T * K <= (gate_type == Q8_0 ? 10 : 4) * E ? 16 : 32;
}

// Weight formats the expert GEMMs read: gate and up (one format for both) and down.
inline bool prefill_type(int t) { return t == Q8_0 || t == Q2_K || t == Q3_K || t == Q4_K || t == Q5_K || t == Q6_K; }

// The phases of a prefill, stream-ordered (the caller checks types: gate and
// up of one format, formats the GEMMs read, H, I, Is multiples of 256, expert
// strides multiples of 16):
//   routing: router + top-K, or the caller's ids / weights; grouping; shared
//   gate; fp16 copy of x
//   gate/up + SwiGLU, down projection, combine.
int launch_prefill_route(const PrefillArgs& a, const int32_t* forced_ids, const float* forced_w, hipStream_t s);
int launch_prefill_gateup(const PrefillArgs& a, hipStream_t s);
int launch_prefill_down(const PrefillArgs& a, hipStream_t s);
int launch_prefill_combine(const PrefillArgs& a, hipStream_t s);

}  // namespace wm
