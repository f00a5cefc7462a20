// wm_prefill.h -- arguments of the batched prefill kernels (wm_prefill.hip).
// Internal; not part of the public ABI.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace wm {

// A (token, slot) pair p = t * K + k is one routed use of an expert; pair
// T * K + t is token t's use of the shared expert.
struct PrefillArgs {
    int32_t H, I, Is, E, K, T, has_shared;
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
    float* act;                 // [pairs][act_stride] SwiGLU outputs
    int64_t act_stride;
    float* y;                   // [pairs][H] expert outputs
    float* sg;                  // [T] shared-expert gate
    float* out;                 // [T][H]
};

// The phases of a prefill, stream-ordered (the caller checks types: Q8_0
// expert matrices, H, I, Is multiples of 128):
//   routing: router + top-K, or the caller's ids / weights; grouping; shared gate
//   gate/up + SwiGLU, down projection, combine.
int launch_prefill_route(const PrefillArgs& a, const int32_t* forced_ids, const float* forced_w, hipStream_t s);
int launch_prefill_gateup(const PrefillArgs& a, hipStream_t s);
int launch_prefill_down(const PrefillArgs& a, hipStream_t s);
int launch_prefill_combine(const PrefillArgs& a, hipStream_t s);

}  // namespace wm
