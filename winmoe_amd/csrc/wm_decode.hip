// wm_decode.hip -- one decode token through the MoE block in ONE launch.
//
// The step is a list of work items, one per 256-thread workgroup (item =
// workgroup id).  Items only wait for items with smaller ids, which start
// first, so every wait ends (and each wait is bounded anyway):
//
//   item 0              shared-expert gate (+ forced routing)
//   router items        reference-order fp32 logits of rr rows each; the last
//                       one to finish runs top-K + softmax into the trace
//   shared gate/up      shared expert gate/up + SwiGLU, and then the
//   shared down         shared down projection: neither needs the routing, so
//                       they stream while the router finishes
//   routed gate/up      per routed slot, once the routing is in
//   routed down         per (slot, row range), once the slot's gate/up items
//                       are done; the last slot to finish a row range
//                       combines sum_k w_k y_k + gate * y_shared there
//
// Every item builds the integer-dot operand of its input vector (x, or the
// slot's SwiGLU output) itself, in registers, while its first weight tiles
// are in flight.  Counters live in the workspace and are returned to zero by
// the last combining item, so consecutive launches (and graph replays) need
// no host work in between.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/winmoe_hip.h"
#include "wm_decode.h"
#include "wm_device.h"
#include "wm_launch.h"
#include "wm_wave.h"

namespace wm {

constexpr int MAX_TOPK = 16;               // top_k limit of the layer descriptor
constexpr uint32_t SPIN_LIMIT = 1u << 20;   // polls before a wait gives up (~0.5 s)

// Hand-off protocol between workgroups.  Agent-scope fences would write back
// and invalidate a whole XCD L2 per call on this multi-XCD part, so instead
// every datum handed between workgroups is stored with device-scope (sc1)
// stores (gst<true>), a producer waits for its own stores to complete
// (s_waitcnt vmcnt(0)) before bumping a counter, and a consumer polls the
// counter before it reads (see wm_wave.h on why ordinary loads are safe for
// the vectors).  The counters themselves are device-scope atomics.
WM_DEV uint32_t ld_relaxed(const uint32_t* p) { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
WM_DEV void st_relaxed(uint32_t* p, uint32_t v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
WM_DEV uint32_t add_relaxed(uint32_t* p, uint32_t v) {
    return __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
WM_DEV uint64_t ld_relaxed64(const uint64_t* p) { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
WM_DEV void st_relaxed64(uint64_t* p, uint64_t v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }

// Dwords 2-3 of a slot's gate/up counter line: (expert id << 32) | 1 once the
// slot's first gate/up item knows the expert, 0 before.
WM_DEV uint64_t* slot_expert(uint32_t* gu_line) { return (uint64_t*)(gu_line + 2); }

// All of this workgroup's stores complete, then one thread bumps *ctr.
// Returns the counter value before the increment (to all threads).
WM_DEV uint32_t wg_signal(uint32_t* ctr) {
    __shared__ uint32_t s_old;
    WM_WAIT_VMCNT(0);
    __syncthreads();
    if (threadIdx.x == 0) s_old = add_relaxed(ctr, 1u);
    __syncthreads();
    return s_old;
}

// As wg_signal, without waiting for the increment to come back.
WM_DEV void wg_post(uint32_t* ctr) {
    WM_WAIT_VMCNT(0);
    __syncthreads();
    if (threadIdx.x == 0) (void)add_relaxed(ctr, 1u);
}

// The whole workgroup waits until *ctr >= target (bounded).  One thread
// polls, backing off to ~0.4 us between polls: hundreds of workgroups polling
// one device-coherent address back to back congest the memory system that
// the streaming workgroups depend on.
WM_DEV void wg_wait(const uint32_t* ctr, uint32_t target, int32_t* status) {
    if (threadIdx.x == 0) {
        uint32_t it = 0;
        int nap = 1;
        while (ld_relaxed(ctr) < target) {
            if (++it > SPIN_LIMIT) {
                atomicOr(status, WM_STATUS_SPIN_TIMEOUT);
                break;
            }
            for (int i = 0; i < nap; i++) __builtin_amdgcn_s_sleep(4);
            nap = nap < 4 ? 2 * nap : 4;
        }
    }
    __syncthreads();
}

// All of this workgroup's stores complete, then one thread sets *ctr = 1.
// The whole workgroup waits until *p != 0 (bounded) and gets the value.
WM_DEV uint64_t wg_wait_set64(const uint64_t* p, int32_t* status) {
    __shared__ uint64_t s_v;
    if (threadIdx.x == 0) {
        uint32_t it = 0;
        int nap = 1;
        uint64_t v;
        while ((v = ld_relaxed64(p)) == 0ull) {
            if (++it > SPIN_LIMIT) {
                atomicOr(status, WM_STATUS_SPIN_TIMEOUT);
                break;
            }
            for (int i = 0; i < nap; i++) __builtin_amdgcn_s_sleep(4);
            nap = nap < 4 ? 2 * nap : 4;
        }
        s_v = v;
    }
    __syncthreads();
    return s_v;
}

WM_DEV void wg_flag(uint32_t* ctr) {
    WM_WAIT_VMCNT(0);
    __syncthreads();
    if (threadIdx.x == 0) st_relaxed(ctr, 1u);
}

// Gate/up + SwiGLU item j of a slot: 2 * tpw tiles of gate and of up.
template <int T>
WM_DEV void item_gateup(const DecodeArgs& a, const uint8_t* Wg, const uint8_t* Wu, int rows, int j, int tpw,
                        float* act, uint8_t* smem) {
    wg_gateup_item<T, true>(Wg, Wu, rows, a.H, j * 2 * tpw, tpw, a.x, act, smem);
}

// Down-projection rows [range * rows_dn_item, ...) of one slot, 4 waves.
template <int T>
WM_DEV void item_down(const DecodeArgs& a, const uint8_t* W, int in, int range, const float* act, float* y,
                      uint8_t* smem, const float* scale = nullptr) {
    const Geo g = geometry(T, in);
    const int tpw = a.rows_dn_item / (WAVES * g.rpt);
    wg_gemv_item<T, true>(W, a.H, in, range * WAVES * tpw, tpw, act, y, smem, scale);
}

// item_down with the weights' first tiles issued before `wait` (the input is
// not ready yet).
template <int T, typename F>
WM_DEV void item_down_prefetch(const DecodeArgs& a, const uint8_t* W, int in, int range, const float* act, float* y,
                               uint8_t* smem, const float* scale, F&& wait) {
    const Geo g = geometry(T, in);
    const int tpw = a.rows_dn_item / (WAVES * g.rpt);
    wg_gemv_item_prefetch<T, true>(W, a.H, in, range * WAVES * tpw, tpw, act, y, smem, scale, wait);
}

WM_DEV uint32_t* ctr(const DecodeArgs& a, int i) { return a.ctr + (int64_t)i * CTR_STRIDE; }

WM_DEV const uint8_t* routed(const uint8_t* base, int64_t stride, int e, int E) {
    return (e >= 0 && e < E) ? base + (int64_t)e * stride : nullptr;
}

template <int GUT, int DT, int SGUT, int SDT>
__global__ __launch_bounds__(256) void k_decode_step(DecodeArgs a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    // Item = workgroup id.  Each XCD starts its workgroups in id order and
    // every wait below is for items with smaller ids, so the smallest
    // unfinished item is always running and can finish: the waits end (they
    // are bounded in any case).
    const int item = (int)blockIdx.x;
    const uint64_t t_start = __builtin_amdgcn_s_memrealtime();
    uint64_t t_ready = t_start, t_work = 0, t_x1 = 0, t_x2 = 0, t_x3 = 0;
    int kind = 0;
    const int K = a.K, K1 = a.K + (a.has_shared ? 1 : 0);

    if (item == 0) {
        // ---- shared-expert gate and forced routing
        if (a.has_shared && a.sh_gate_inp) wg_shgate<true>(a.x, a.sh_gate_inp, a.H, a.shgate);
        if (a.forced && (int)threadIdx.x < K) {
            int e = a.forced_ids[threadIdx.x];
            gst<true>(a.ids + threadIdx.x, (int32_t)e);
            gst<true>(a.w + threadIdx.x, a.forced_w[threadIdx.x]);
            if (e >= 0 && e < a.E) atomicAdd(a.hits + e, 1u);
            else atomicOr(a.status, WM_STATUS_BAD_EXPERT_ID);
        }
        t_work = __builtin_amdgcn_s_memrealtime();
        wg_flag(ctr(a, C_AUX));
        if (a.forced && threadIdx.x == 0) st_relaxed(ctr(a, C_TOPK), 1u);
    } else if (item < a.it_gu) {
        // ---- router rows.  The last item of each group of RGROUP bumps the
        // top counter (all logits are in once it reaches n_rgroups); the last
        // of those writes the trace: top-K, softmax weights, hit counts.
        const int j = item - a.it_router;
        const int r0 = j * a.rr, g = j / RGROUP;
        kind = 1;
        wg_router_rows<true>(a.x, a.router, a.H, r0, min(a.rr, a.E - r0), a.router_region, (lds8_t*)smem, a.logits,
                             &t_x3);
        t_work = __builtin_amdgcn_s_memrealtime();
        const uint32_t gsize = (uint32_t)min(RGROUP, a.n_router - g * RGROUP);
        if (wg_signal(ctr(a, C_RGROUP + g)) == gsize - 1) {
            t_x1 = __builtin_amdgcn_s_memrealtime();
            if (wg_signal(ctr(a, C_RTOP)) == (uint32_t)(a.n_rgroups - 1)) {
                // every logit is in: one flag line per group of routed items,
                // so that their polls spread over C_NGO lines
                if (threadIdx.x < C_NGO) st_relaxed(ctr(a, C_GO + threadIdx.x), 1u);
                if (threadIdx.x < 64) wave_topk<true>(a.logits, a.E, K, a.ids, a.w, a.hits, a.status, threadIdx.x);
                t_x2 = __builtin_amdgcn_s_memrealtime();
                wg_flag(ctr(a, C_TOPK));
            }
        }
    } else if (item >= a.it_sgu && item < a.it_sdn) {
        // ---- shared expert gate/up + SwiGLU (needs no routing)
        kind = 2;
        item_gateup<SGUT>(a, a.sh_gate, a.sh_up, a.Is, item - a.it_sgu, a.tpw_sgu, a.act + (int64_t)K * a.act_stride,
                          smem);
        t_work = __builtin_amdgcn_s_memrealtime();
        wg_post(ctr(a, C_GU + K));
    } else if (item < a.it_sgu) {
        // ---- routed gate/up + SwiGLU.  The item finds its slot's expert
        // itself (slot + 1 picks over the logits), so it does not wait for the
        // whole top-K; the slot's first item publishes the id for the down items.
        // (the last slot first: its pick takes the most passes)
        const int j = item - a.it_gu;
        const int slot = K - 1 - j / a.n_gu_slot, jj = j % a.n_gu_slot;
        int e;
        float v = 0.0f;
        if (a.forced) {
            wg_wait(ctr(a, C_TOPK), 1u, a.status);
            e = gld<true>(a.ids + slot);
        } else {
            wg_wait(ctr(a, C_GO + item % C_NGO), 1u, a.status);
            t_x1 = __builtin_amdgcn_s_memrealtime();
            e = wave_pick(a.logits, a.E, slot, threadIdx.x & 63, v);
        }
        t_ready = __builtin_amdgcn_s_memrealtime();
        kind = 3;
        if (jj == 0 && threadIdx.x == 0) {
            gst<true>((int32_t*)ctr(a, C_SLOTEID) + slot, (int32_t)e);
            gst<true>((float*)ctr(a, C_SLOTEID) + MAX_TOPK + slot, v);
            // the down items of the slot start loading its weights on this
            st_relaxed64(slot_expert(ctr(a, C_GU + slot)), ((uint64_t)(uint32_t)e << 32) | 1ull);
        }
        item_gateup<GUT>(a, routed(a.gate, a.gstride, e, a.E), routed(a.up, a.ustride, e, a.E), a.I, jj, a.tpw_gu,
                         a.act + (int64_t)slot * a.act_stride, smem);
        t_work = __builtin_amdgcn_s_memrealtime();
        wg_post(ctr(a, C_GU + slot));
    } else {
        // ---- down projection of one (slot, row range); the last slot of a range combines it
        int slot, range;
        if (item < a.it_dn) { slot = K; range = item - a.it_sdn; }
        else { slot = (item - a.it_dn) / a.n_dn_slot; range = (item - a.it_dn) % a.n_dn_slot; }
        kind = 4;
        const float* act = a.act + (int64_t)slot * a.act_stride;
        float* y = a.ypart + (int64_t)slot * a.H;
        const uint32_t n_need = (uint32_t)(slot == K ? a.n_sgu : a.n_gu_slot);
        // The weights' first tiles are loaded while the slot's gate/up items
        // finish (the expert is known before its SwiGLU output is).
        if (slot == K) {
            // the shared-expert gate multiplies the shared rows here (the
            // same product the combine would form)
            __shared__ float s_gate;
            const bool gated = a.sh_gate_inp != nullptr;
            item_down_prefetch<SDT>(a, a.sh_down, a.Is, range, act, y, smem, gated ? &s_gate : nullptr, [&]() {
                wg_wait(ctr(a, C_GU + K), n_need, a.status);
                if (gated) {
                    wg_wait(ctr(a, C_AUX), 1u, a.status);
                    if (threadIdx.x == 0) s_gate = gld<true>(a.shgate);
                    __syncthreads();
                }
                t_ready = __builtin_amdgcn_s_memrealtime();
            });
        } else {
            const uint64_t se = wg_wait_set64(slot_expert(ctr(a, C_GU + slot)), a.status);
            item_down_prefetch<DT>(a, routed(a.down, a.dstride, (int32_t)(se >> 32), a.E), a.I, range, act, y, smem,
                                   nullptr, [&]() {
                                       wg_wait(ctr(a, C_GU + slot), n_need, a.status);
                                       t_ready = __builtin_amdgcn_s_memrealtime();
                                   });
        }
        t_work = __builtin_amdgcn_s_memrealtime();
        uint32_t old = wg_signal(ctr(a, C_RANGE + range));
        if (old == (uint32_t)(K1 - 1)) {
            // out[h] = sum_k w_k y_k[h] (k order, invalid ids skipped) + gate * y_shared[h]
            kind |= 8;
            __shared__ float s_w[MAX_TOPK];
            __shared__ int s_valid[MAX_TOPK];
            if ((int)threadIdx.x < K) {
                const int k = threadIdx.x;
                const int e = gld<true>((const int32_t*)ctr(a, C_SLOTEID) + k);
                float wk;
                if (a.forced) wk = gld<true>(a.w + k);
                else {
                    // the softmax weight from the K published pick logits
                    float v[MAX_TOPK];
#pragma unroll
                    for (int i = 0; i < MAX_TOPK; i++)      // clamped, unconditional: loads in flight together
                        v[i] = gld<true>((const float*)ctr(a, C_SLOTEID) + MAX_TOPK + min(i, K - 1));
                    wk = pick_weight(v, K, k);
                }
                s_valid[k] = (e >= 0 && e < a.E) ? 1 : 0;
                s_w[k] = (e >= 0 && e < a.E) ? wk : 0.0f;
            }
            __syncthreads();
            const int h0 = range * a.rows_dn_item, h1 = min(a.H, h0 + a.rows_dn_item);
            for (int h = h0 + threadIdx.x; h < h1; h += 256) {
                float yv[MAX_TOPK + 1];
#pragma unroll
                for (int k = 0; k <= MAX_TOPK; k++)          // clamped, unconditional: loads in flight together
                    yv[k] = a.ypart[(int64_t)min(k, K1 - 1) * a.H + h];   // ordinary loads, as for the vectors
                float acc = 0.0f;
#pragma unroll
                for (int k = 0; k < MAX_TOPK; k++)
                    if (k < K && s_valid[k]) acc = fmaf(s_w[k], yv[k], acc);
                if (a.has_shared) acc = acc + yv[K];            // gate already applied
                a.out[h] = acc;
            }
            // The last combined range ends the step: every other item has
            // already made its last counter access (each one feeds a range,
            // and item 0 and the trace writer are awaited here), so the
            // counters go back to zero.
            uint32_t done = wg_signal(ctr(a, C_COMBINED));
            if (done == (uint32_t)(a.n_dn_slot - 1)) {
                wg_wait(ctr(a, C_TOPK), 1u, a.status);
                wg_wait(ctr(a, C_AUX), 1u, a.status);
                for (int i = threadIdx.x; i < C_TOTAL; i += 256) st_relaxed(a.ctr + (int64_t)i * CTR_STRIDE, 0u);
                if ((int)threadIdx.x < K) st_relaxed64(slot_expert(ctr(a, C_GU + threadIdx.x)), 0ull);
            }
        }
    }

    if (a.timeline && threadIdx.x == 0 && item < a.timeline_cap) {
        uint64_t* r = a.timeline + 8 * (int64_t)item;
        r[0] = t_start;
        r[1] = t_ready;
        r[2] = t_work;
        r[3] = __builtin_amdgcn_s_memrealtime();
        uint64_t hw = (uint32_t)__builtin_amdgcn_s_getreg((4) | (0 << 6) | (31 << 11));
        uint64_t xcc = (uint32_t)__builtin_amdgcn_s_getreg((20) | (0 << 6) | (31 << 11));
        r[4] = (uint64_t)kind | (hw << 8) | (xcc << 40);
        r[5] = t_x1;
        r[6] = t_x2;
        r[7] = t_x3;
    }
}

// ------------------------------------------------------------------ launcher

template <int GUT, int DT, int SGUT, int SDT>
static int launch_inst(const DecodeArgs& a, size_t lds, hipStream_t s) {
    hipLaunchKernelGGL((k_decode_step<GUT, DT, SGUT, SDT>), dim3(a.n_items), dim3(256), lds, s, a);
    return (int)hipGetLastError();
}

#define WM_DEC_CASE(g, d, sg, sd)                                                      \
    if (gut == g && dt == d && sgut == sg && sdt == sd) return launch_inst<g, d, sg, sd>(a, lds, s);

int launch_decode_step(const DecodeArgs& a, int gut, int dt, int sgut, int sdt, hipStream_t s) {

    const size_t lds = DECODE_LDS;
    WM_DEC_CASE(Q8_0, Q8_0, Q8_0, Q8_0)
    WM_DEC_CASE(Q2_K, Q2_K, Q2_K, Q2_K)
    WM_DEC_CASE(Q3_K, Q3_K, Q3_K, Q3_K)
    WM_DEC_CASE(Q4_K, Q4_K, Q4_K, Q4_K)
    WM_DEC_CASE(Q5_K, Q5_K, Q5_K, Q5_K)
    WM_DEC_CASE(Q6_K, Q6_K, Q6_K, Q6_K)
    WM_DEC_CASE(Q4_K, Q6_K, Q8_0, Q8_0)
    WM_DEC_CASE(Q4_K, Q6_K, Q4_K, Q6_K)
    WM_DEC_CASE(Q4_K, Q5_K, Q8_0, Q8_0)
    WM_DEC_CASE(Q4_K, Q5_K, Q4_K, Q5_K)
    WM_DEC_CASE(Q2_K, Q3_K, Q8_0, Q8_0)
    WM_DEC_CASE(Q2_K, Q3_K, Q2_K, Q3_K)
    return -1;   // combination without a fused instantiation
}

bool decode_step_supported(int gut, int dt, int sgut, int sdt) {
    const int c[12][4] = {{Q8_0, Q8_0, Q8_0, Q8_0}, {Q2_K, Q2_K, Q2_K, Q2_K}, {Q3_K, Q3_K, Q3_K, Q3_K},
                          {Q4_K, Q4_K, Q4_K, Q4_K}, {Q5_K, Q5_K, Q5_K, Q5_K}, {Q6_K, Q6_K, Q6_K, Q6_K},
                          {Q4_K, Q6_K, Q8_0, Q8_0}, {Q4_K, Q6_K, Q4_K, Q6_K}, {Q4_K, Q5_K, Q8_0, Q8_0},
                          {Q4_K, Q5_K, Q4_K, Q5_K}, {Q2_K, Q3_K, Q8_0, Q8_0}, {Q2_K, Q3_K, Q2_K, Q3_K}};
    for (auto& r : c)
        if (r[0] == gut && r[1] == dt && r[2] == sgut && r[3] == sdt) return true;
    return false;
}

}  // namespace wm
