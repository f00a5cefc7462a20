// wm_launch.h -- internal interface between the C-ABI layer (wm_capi.cpp) and
// the kernel launchers (wm_kernels.hip).  Not part of the public ABI.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "wm_format.h"

namespace wm {

// Where the matrix of slot s lives: routed slots s < n_routed use expert
// ids[s] (or s when ids == NULL) of a stacked tensor; slot n_routed is the
// shared expert.
struct MatSet {
    const uint8_t* base;
    int64_t stride;
    const int32_t* ids;
    int32_t n_routed;
    int32_t E;
    const uint8_t* shared;
};

struct GemvArgs {
    MatSet m;
    int32_t slot0;            // first slot handled by the launch (blockIdx.y offset)
    int32_t rows, in;
    int32_t tiles_per_wave;
    const float* x;           // input vectors [slot][x_slot_stride], 16-byte aligned
    int64_t x_slot_stride;    // floats between slots (0 = shared by all slots)
    float* y;                 // outputs [slot][rows]
    int64_t y_slot_stride;    // floats
    int32_t* status;
};

struct GateUpArgs {
    MatSet gate, up;
    int32_t slot0;
    int32_t rows, in;
    int32_t tiles_per_wave;
    const float* x;           // input vector shared by all slots, 16-byte aligned
    float* act;               // SwiGLU output [slot][act_slot_stride]
    int64_t act_slot_stride;
    int32_t* status;
};

struct CombineArgs {
    const float* ypart;       // [K(+1)][H]
    int64_t y_stride;
    const float* w;           // [K] routing weights
    const int32_t* ids;       // [K] (checked against E)
    int32_t K, E, H;
    int32_t has_shared;
    const float* sh_gate;     // scalar or NULL
    float* out;
};

// Launchers (return hipError_t as int; 0 = success).
int launch_router_logits(const float* x, const float* W, int H, int E, float* logits, hipStream_t s);
int launch_topk(const float* logits, int E, int K, int32_t* ids, float* w, uint32_t* hits, int32_t* status,
                hipStream_t s);
int launch_swiglu(const float* g, const float* u, float* act, int n, int nslots, int64_t stride, hipStream_t s);
int launch_gemv(int t, const GemvArgs& a, int nslots, hipStream_t s);
int launch_gateup(int t, const GateUpArgs& a, int nslots, hipStream_t s);
int launch_combine(const CombineArgs& a, hipStream_t s);
int launch_shgate(const float* x, const float* g, int H, float* out, hipStream_t s);
int launch_dequant(int t, const void* blocks, int64_t nblocks, float* out, hipStream_t s);
int launch_quantize(int t, const float* x, int64_t nblocks, void* out, hipStream_t s);
int launch_fill_i32(int32_t* p, int32_t v, int64_t n, hipStream_t s);
int launch_count_hits(const int32_t* ids, int K, int E, uint32_t* hits, int32_t* status, hipStream_t s);
int launch_axpy(float* acc, const float* y, float w, int n, hipStream_t s);

// Creates the current device's event that orders persistent decode launches
// across streams (otherwise made on first need).  WM_OK or WM_ERR.
int persist_order_prepare();

// Geometry of the segment mapping for a row of `in` weights.
struct Geo {
    int lpr, rpt, active;
    int64_t row_bytes, tile_bytes;
};
WM_HD Geo geometry(int t, int in) {
    Geo g;
    g.lpr = in / SEG;
    g.rpt = g.lpr > 0 ? SEG / g.lpr : 0;
    g.active = g.rpt * g.lpr;
    g.row_bytes = matrix_bytes(t, 1, in);
    g.tile_bytes = g.row_bytes * g.rpt;
    return g;
}
// Shapes the segment kernels accept: in a multiple of the block size and of
// 64, in/64 a power of two dividing 64 (in = 64 .. 4096).
WM_HD bool gemv_shape_ok(int t, int in) {
    if (!supported(t) || in <= 0 || in % block_elems(t) || in % SEG || in > 4096) return false;
    int lpr = in / SEG;
    return (lpr & (lpr - 1)) == 0;
}

}  // namespace wm
