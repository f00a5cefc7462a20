// wm_decode.h -- arguments and workspace counters of the fused decode-step
// kernel (wm_decode.hip).  Internal; not part of the public ABI.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "wm_format.h"

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

// ------------------------------------------------------------------ persistent step
// One workgroup per CU: PW streaming waves + 3 helper waves (router rows,
// routing, operand staging, SwiGLU publishing, combine).  Internal.
namespace wm {

// Streaming waves per workgroup (each loads one tile at a time into its own
// LDS buffer and processes it; with the 3 helpers, 16 waves per CU).
constexpr int PW = 13;
constexpr int PRING = 1;                 // LDS buffers per streaming wave
constexpr int PSTAGE = 2;                // helper waves besides the publisher: the router wave and the x loader
constexpr int PTHREADS = 64 * (PW + 1 + PSTAGE);  // + publisher
constexpr int PMAXK = 16;
constexpr int PMAXACT = 16;              // act tiles of one slot (64-value segments of I / segments per act tile)
constexpr int P_TL = 32;                 // timeline words per workgroup
constexpr int P_MAX_WG = 1024;           // workgroups (CUs) the workspace has start-tag words for
constexpr int P_REP = 8;                 // replicas of the tagged logits (each read by 1/8 of the workgroups)
constexpr int P_AREP = 4;                // replicas of the tagged SwiGLU outputs
constexpr int P_XREP = 8;                // replicas of a chained layer's tagged output (read whole by every workgroup)
constexpr uint32_t PSPIN_G = 1u << 17;   // device-memory polls (~1 us each) before a wait gives up

// Ring buffer bytes of one tile of type T: NI DMA units of 1 KB, except Q8_0
// whose 5th unit is cut to the 4352-byte tile + 16 B of alignment shift (the
// lanes beyond it issue no load) + over-read pad.
template <int T> WM_HD constexpr int ring_tile_bytes() { return T == Q8_0 ? 4416 : (T == Q6_K ? 4096 : ((T == Q4_K || T == Q5_K) ? 3072 : 2048)); }
WM_HD int ring_tile_bytes_rt(int t) { return t == Q8_0 ? 4416 : (t == Q6_K ? 4096 : ((t == Q4_K || t == Q5_K) ? 3072 : 2048)); }

// LDS control block of one workgroup (zeroed at the start of every launch).
// The streaming waves use LDS atomics only while none of their LDS-DMA loads
// is in flight (the compiler makes every LDS atomic wait for all of them).
struct PersistCtl {
    uint32_t next;                 // next tile-list entry to claim
    uint32_t n_done;               // down tiles processed
    uint32_t gu_done[PMAXK + 1];   // gate/up tiles of the slot processed
    uint32_t xop_built[PW];        // streaming wave w wrote its part of the x operand records
    uint32_t routed;               // routing of this step is in ids / w / valid
    uint32_t sgate_ready;          // sgate holds the shared-expert gate
    uint32_t tag;                  // this launch's tag (epoch + 1)
    uint32_t abort;                // a wait of this workgroup gave up: every later wait ends at once
    uint32_t rows_in;              // x and the router rows are in LDS
    uint32_t router_done[2];       // helper h is done with the router rows (their ring space is free)
    uint32_t npicked;              // picks 0 .. npicked-1 of the routing are in ids / valid / rbase
    uint32_t act_done[PMAXK + 1][PMAXACT]; // the slot's SwiGLU operand records of act tile t are in LDS
    int32_t ids[PMAXK];
    float w[PMAXK];
    int32_t valid[PMAXK];
    float sgate;
    uint32_t x_in;                 // x is in LDS (the second staging wave loads it)
    uint32_t desc_built;           // the tile descriptor table is built
    uint32_t xpart[PW + 1];        // a chained layer's input: wave w's part of it is in x
    uint64_t rbase[PMAXK][3];      // routed slot k's gate / up / down bytes | 1 (1 alone: no weights), 0 until picked
    uint64_t t[P_TL];              // timeline (device clock)
};

struct PersistArgs {
    int32_t H, I, E, K, has_shared, forced, nwg, rr;
    int32_t gu_tiles, dn_tiles;        // tiles of one gate/up matrix (I rows) and of one down matrix (H rows)
    int32_t gu_step;                   // gate/up tiles are split among workgroups in units of gu_step (an even row count)
    int32_t n_rwaves;                  // streaming waves whose rings hold x and the router rows at the start
    int32_t o_ring, ring_buf, nstream; // LDS: the rings of the nstream streaming waves (PRING buffers of ring_buf bytes each)
    int32_t x_region;                  // bytes of x / of one router row in the router region
    int32_t o_router;                  // LDS: x and the router rows (the first rings, or a region of its own)
    int32_t o_reg;                     // LDS: SwiGLU operand records [K+1][I/64]
    int32_t o_norm;                    // LDS: the RMSNorm weights (x_region bytes, over the records until x is in)
    int32_t aseg, nact;                // act tiles: segments of the SwiGLU vector per tile, tiles per slot
    int32_t o_xop, o_xop2;             // LDS: x operand records of the routed / shared gate-up types
    int32_t o_gu, gu_cap;              // LDS: gate and up row sums [K+1][gu_cap] each
    int32_t o_y, y_cap;                // LDS: down row sums [K+1][y_cap]
    int32_t o_desc, n_desc;            // LDS: the tile list's descriptors (16 bytes per entry, n_desc at most)
    const float* x;                    // x, or the residual stream h when norm_w is set
    float* out;
    const float* router;
    const float* norm_w;               // RMSNorm weight [H] or null
    float norm_eps;
    int32_t add_res;                   // out = h + moe_out
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
    int32_t* ids;                      // trace slot of this step
    float* w;
    uint32_t* hits;
    int32_t* status;
    uint64_t* tlogits;                 // [P_REP][E] (tag << 32) | logit bits
    uint32_t* hello;                   // [nwg] tag of the launch each workgroup started in
    uint32_t* epoch;                   // launches completed since the workspace was reset
    uint64_t* tact;                    // [K+1][P_AREP][I/2] (tag16 << 48) | act24(v[2i+1]) << 24 | act24(v[2i])
    uint64_t* timeline;                // NULL or [nwg][P_TL]
    uint32_t probe;                    // nonzero: every wait of the step gives up at its first unsuccessful poll
    // layers chained in one launch (k_decode_stack): this layer's output
    // also as tagged words (tag << 32 | value bits) for the next layer, and
    // its input as the previous layer's tagged words (null: x), staged in
    // LDS at o_stage (8 bytes a value)
    uint64_t* tx_out;
    const uint64_t* tx_in;
    int32_t o_stage;
};

// Layers of one launch of the chained step (kernel arguments: at most 4 KB).
constexpr int P_STACK = 8;
struct StackArgs {
    PersistArgs L[P_STACK];
    int32_t n;
};
static_assert(sizeof(StackArgs) <= 4096, "kernel arguments");

bool persist_supported(int gut, int dt, int sgut, int sdt);
int launch_persist(const PersistArgs& a, size_t lds, int gut, int dt, int sgut, int sdt, hipStream_t s);
int launch_stack(const StackArgs& a, size_t lds, int gut, int dt, int sgut, int sdt, hipStream_t s);
bool stack_supported(int gut, int dt, int sgut, int sdt);     // the type sets with a chained-launch instance

}  // namespace wm
