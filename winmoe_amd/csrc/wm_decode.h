// wm_decode.h -- arguments and workspace counters of the fused decode-step
// kernel (wm_decode.hip).  Internal; not part of the public ABI.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace wm {

// Counters (uint32) inside the workspace, each alone in its own 256-byte line:
// device-scope atomics on one line are serialised where they are performed
// (about 11 ns each on MI355X), and reads of the line slow them further,
// while atomics on distinct lines proceed in parallel.  All zero between
// launches.
constexpr int CTR_STRIDE = 64;    // dwords between counters
constexpr int RGROUP = 16;        // router items per group counter
enum : int {
    C_RTOP = 0,        // router groups finished: every logit is written
    C_TOPK = 1,        // routing of this step is in the trace
    C_AUX = 2,         // shared-expert gate (and forced routing) written
    C_COMBINED = 3,    // row ranges combined
    C_SLOTEID = 4,     // not a counter: dword s = expert id of routed slot s
    C_GU = 5,          // + slot: gate/up items finished for the slot
    C_RGROUP = 37,     // + group: router items finished in the group
    C_MAX_RGROUPS = 64,
    C_RANGE = C_RGROUP + C_MAX_RGROUPS,   // + range: down items finished for the row range
    C_MAX_RANGES = 256,
    C_GO = C_RANGE + C_MAX_RANGES,        // + i: every logit is written (C_RTOP fanned out to C_NGO lines)
    C_NGO = 32,
    C_TOTAL = C_GO + C_NGO,               // counters (lines)
};

struct DecodeArgs {
    int32_t H, I, Is, E, K, has_shared, forced, rr;
    const float* x;
    float* out;
    const float* router;
    const uint8_t* gate;
    const uint8_t* up;
    const uint8_t* down;
    int64_t gstride, ustride, dstride;
    const uint8_t* sh_gate;
    const uint8_t* sh_up;
    const uint8_t* sh_down;
    const float* sh_gate_inp;
    const int32_t* forced_ids;
    const float* forced_w;
    float* logits;
    int32_t* ids;
    float* w;
    uint32_t* hits;
    int32_t* status;
    float* act;
    int64_t act_stride;
    float* ypart;
    float* shgate;
    uint32_t* ctr;
    int32_t n_items, it_router, n_router, n_rgroups, it_sgu, n_sgu, it_sdn, it_gu, n_gu_slot, it_dn, n_dn_slot;
    int32_t tpw_gu, tpw_sgu, rows_dn_item, router_region;
    uint64_t* timeline;    // NULL, or [n_items][8]: start, dependencies met, work done, end (device clock), kind | hw ids
    int32_t timeline_cap;
};

constexpr int TIMELINE_CAP = 16384;
constexpr int DECODE_LDS = 65536;   // dynamic LDS of a decode-step workgroup (2 per CU)

bool decode_step_supported(int gut, int dt, int sgut, int sdt);
int launch_decode_step(const DecodeArgs& a, int gut, int dt, int sgut, int sdt, hipStream_t s);

}  // namespace wm
