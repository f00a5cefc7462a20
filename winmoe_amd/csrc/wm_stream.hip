// wm_stream.hip -- host -> HBM expert streaming: a pool of expert slots in
// HBM for models whose experts do not all fit there.  Host code only.
//
// The reference serves a missing expert from SSD into a RAM slot with
// asynchronous reads issued for all K picks before the first one is computed
// (winmoe_inference.c:1736-1789) and, with the GPU enabled, uploads the slot
// [gate | up | down] to the GPU expert cache (gpu_offload.cu:590-659).  Here
// the slots live in HBM and a step never waits on the host:
//   * a missing expert's three parts are copied from host memory with
//     asynchronous copies on the pool's own stream, then an event marks the
//     slot ready; the compute stream waits for that event on the device;
//   * a released slot carries an event recorded after the steps that read
//     it; before the pool's stream overwrites the slot it waits for that
//     event (again on the device), so a slot is never rewritten under a step;
//   * the slot indices go to the device through a ring of pinned host words
//     (an entry is reused only after its copy has run).
// With pinned host memory the copies overlap the compute of other experts and
// layers; with pageable memory they are still correct but the runtime stages
// them through the host.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>

#include <algorithm>
#include <unordered_map>
#include <vector>

#include "../../include/winmoe_hip.h"
#include "wm_host.h"

using wm::round_up256;

namespace {
constexpr int kRing = 64;      // entries of the pinned ring of slot indices
}

struct wm_expert_pool {
    int n_slots = 0;
    int64_t part[3] = {0, 0, 0};         // bytes of gate, up, down of one expert
    int64_t off[3] = {0, 0, 0};          // their offsets inside a slot (256-byte aligned)
    int64_t slot_bytes = 0;
    uint8_t* base = nullptr;             // caller's device memory: n_slots * slot_bytes
    hipStream_t copy = nullptr;          // the pool's copy stream
    std::vector<int64_t> key;            // per slot: (layer << 32 | expert) held, -1 when free
    std::vector<uint64_t> stamp;         // per slot: last use (LRU)
    std::vector<char> taken;             // per slot: used by an acquire not yet released
    std::vector<hipEvent_t> ready;       // per slot: its bytes have landed (pool's stream)
    std::vector<char> ready_set;
    std::vector<hipEvent_t> done;        // per slot: the released steps that read it are over
    std::vector<char> done_set;
    std::vector<int> pending;            // slots of the acquires since the last release
    std::unordered_map<int64_t, int> where;
    uint64_t clock = 0;
    int32_t* ring = nullptr;             // pinned [kRing][n_slots]
    hipEvent_t ring_ev[kRing] = {};
    char ring_set[kRing] = {};
    int ring_pos = 0;
    int64_t hits = 0, misses = 0, bytes = 0;
};

static void pool_free(wm_expert_pool* p) {
    if (!p) return;
    if (p->copy) (void)hipStreamSynchronize(p->copy);
    for (hipEvent_t e : p->ready) if (e) (void)hipEventDestroy(e);
    for (hipEvent_t e : p->done) if (e) (void)hipEventDestroy(e);
    for (hipEvent_t e : p->ring_ev) if (e) (void)hipEventDestroy(e);
    if (p->ring) (void)hipHostFree(p->ring);
    if (p->copy) (void)hipStreamDestroy(p->copy);
    delete p;
}

extern "C" int64_t wm_pool_slot_bytes(int64_t gate_bytes, int64_t up_bytes, int64_t down_bytes) {
    if (gate_bytes <= 0 || up_bytes <= 0 || down_bytes <= 0) return WM_EINVAL;
    return round_up256(gate_bytes) + round_up256(up_bytes) + round_up256(down_bytes);
}

extern "C" int wm_pool_create(void* slots, int64_t slots_bytes, int n_slots, int64_t gate_bytes, int64_t up_bytes,
                              int64_t down_bytes, wm_expert_pool** out) {
    WM_CHECK_ARG(out && slots && n_slots >= 1 && n_slots <= 1024);
    *out = nullptr;
    const int64_t sb = wm_pool_slot_bytes(gate_bytes, up_bytes, down_bytes);
    WM_CHECK_ARG(sb > 0 && ((uintptr_t)slots % 256) == 0 && slots_bytes >= sb * n_slots);
    if (wm_init()) return WM_ERR;
    wm_expert_pool* p = new wm_expert_pool();
    p->n_slots = n_slots;
    p->part[0] = gate_bytes; p->part[1] = up_bytes; p->part[2] = down_bytes;
    p->off[0] = 0;
    p->off[1] = round_up256(gate_bytes);
    p->off[2] = p->off[1] + round_up256(up_bytes);
    p->slot_bytes = sb;
    p->base = (uint8_t*)slots;
    p->key.assign(n_slots, -1);
    p->stamp.assign(n_slots, 0);
    p->taken.assign(n_slots, 0);
    p->ready.assign(n_slots, nullptr);
    p->ready_set.assign(n_slots, 0);
    p->done.assign(n_slots, nullptr);
    p->done_set.assign(n_slots, 0);
    auto fail = [&](hipError_t e) {
        fprintf(stderr, "winmoe_hip: expert pool: %s\n", hipGetErrorString(e));
        pool_free(p);
        return WM_ERR;
    };
    hipError_t e = hipStreamCreateWithFlags(&p->copy, hipStreamNonBlocking);
    if (e != hipSuccess) return fail(e);
    for (int s = 0; s < n_slots; s++) {
        if ((e = hipEventCreateWithFlags(&p->ready[s], hipEventDisableTiming)) != hipSuccess) return fail(e);
        if ((e = hipEventCreateWithFlags(&p->done[s], hipEventDisableTiming)) != hipSuccess) return fail(e);
    }
    for (int r = 0; r < kRing; r++)
        if ((e = hipEventCreateWithFlags(&p->ring_ev[r], hipEventDisableTiming)) != hipSuccess) return fail(e);
    if ((e = hipHostMalloc((void**)&p->ring, (size_t)kRing * n_slots * sizeof(int32_t), hipHostMallocDefault)) !=
        hipSuccess)
        return fail(e);
    *out = p;
    return WM_OK;
}

extern "C" int wm_pool_destroy(wm_expert_pool* pool) {
    pool_free(pool);
    return WM_OK;
}

extern "C" int wm_pool_layer(const wm_expert_pool* pool, wm_layer_desc* d) {
    WM_CHECK_ARG(pool && d);
    d->gate_exps = pool->base + pool->off[0];
    d->up_exps = pool->base + pool->off[1];
    d->down_exps = pool->base + pool->off[2];
    d->gate_stride = d->up_stride = d->down_stride = pool->slot_bytes;
    d->n_experts = pool->n_slots;
    return WM_OK;
}

// Makes ids[0..n) of `layer` resident; copy(i, slot) enqueues the copies of
// ids[i] into `slot` on the pool's stream and returns the bytes it copies (< 0
// on a HIP failure).  Shared by the per-part and the packed sources.
template <class Copy>
static int pool_acquire(wm_expert_pool* pool, int layer, const int32_t* ids, int n, int n_src, int32_t* slots_dev,
                        void* stream, Copy copy) {
    WM_CHECK_ARG(pool && ids && n >= 1 && n <= pool->n_slots && layer >= 0 && n_src >= 1);
    WM_CHECK_ARG(slots_dev && ((uintptr_t)slots_dev % 4) == 0);
    // every id names an expert of the source (checked before any state changes)
    for (int i = 0; i < n; i++) WM_CHECK_ARG(ids[i] >= 0 && ids[i] < n_src);
    wm_expert_pool& P = *pool;
    hipStream_t s = (hipStream_t)stream;
    // refuse up front (no state changes) when the misses would find no slot:
    // they need as many slots as are neither held by unreleased acquires nor
    // hit by this call
    {
        std::vector<char> busy(P.taken.begin(), P.taken.end());
        std::vector<int64_t> fresh;
        for (int i = 0; i < n; i++) {
            const int64_t k = ((int64_t)layer << 32) | (uint32_t)ids[i];
            auto it = P.where.find(k);
            if (it != P.where.end()) busy[it->second] = 1;
            else if (std::find(fresh.begin(), fresh.end(), k) == fresh.end()) fresh.push_back(k);
        }
        const int avail = (int)std::count(busy.begin(), busy.end(), 0);
        if ((int)fresh.size() > avail) {
            fprintf(stderr, "winmoe_hip: expert pool: %d experts to load, %d of %d slots not held by unreleased "
                            "steps\n", (int)fresh.size(), avail, P.n_slots);
            return WM_EINVAL;
        }
    }
    int32_t* entry = P.ring + (int64_t)P.ring_pos * P.n_slots;
    if (P.ring_set[P.ring_pos]) WM_FAIL_HIP(hipEventSynchronize(P.ring_ev[P.ring_pos]));
    // the call's resident experts are held first, so that no miss of the
    // call evicts an expert the call asks for
    auto hold = [&](int slot) {
        if (!P.taken[slot]) {
            P.taken[slot] = 1;
            P.pending.push_back(slot);
        }
    };
    for (int i = 0; i < n; i++) {
        auto it = P.where.find(((int64_t)layer << 32) | (uint32_t)ids[i]);
        entry[i] = it != P.where.end() ? it->second : -1;
        if (entry[i] >= 0) hold(entry[i]);
    }
    int nmiss = 0;
    for (int i = 0; i < n; i++) {
        const int64_t k = ((int64_t)layer << 32) | (uint32_t)ids[i];
        if (entry[i] < 0) {
            auto it = P.where.find(k);          // (loaded for an earlier copy of the id in this call)
            if (it != P.where.end()) {
                entry[i] = it->second;
            } else {
                // a free slot, else the least recently used one that no
                // unreleased step and no part of this call holds
                int slot = -1;
                for (int c = 0; c < P.n_slots && slot < 0; c++)
                    if (P.key[c] < 0 && !P.taken[c]) slot = c;
                for (int c = 0; c < P.n_slots; c++)
                    if (!P.taken[c] && P.key[c] >= 0 && (slot < 0 || (P.key[slot] >= 0 && P.stamp[c] < P.stamp[slot])))
                        slot = c;
                if (slot < 0) {     // (excluded by the check above)
                    fprintf(stderr, "winmoe_hip: expert pool: no slot free\n");
                    return WM_ERR;
                }
                if (P.key[slot] >= 0) P.where.erase(P.key[slot]);
                // the pool's stream rewrites the slot once the steps that read it are over
                if (P.done_set[slot]) WM_FAIL_HIP(hipStreamWaitEvent(P.copy, P.done[slot], 0));
                const int64_t nb = copy(i, slot);
                if (nb < 0) return WM_ERR;
                P.bytes += nb;
                WM_FAIL_HIP(hipEventRecord(P.ready[slot], P.copy));
                P.ready_set[slot] = 1;
                P.key[slot] = k;
                P.where[k] = slot;
                P.misses++;
                nmiss++;
                entry[i] = slot;
                hold(slot);
                P.stamp[slot] = ++P.clock;
                continue;
            }
        }
        P.hits++;
        P.stamp[entry[i]] = ++P.clock;
    }
    // the step waits for the copies of its slots (a finished event costs nothing)
    for (int i = 0; i < n; i++)
        if (P.ready_set[entry[i]]) WM_FAIL_HIP(hipStreamWaitEvent(s, P.ready[entry[i]], 0));
    WM_FAIL_HIP(hipMemcpyAsync(slots_dev, entry, (size_t)n * sizeof(int32_t), hipMemcpyHostToDevice, s));
    WM_FAIL_HIP(hipEventRecord(P.ring_ev[P.ring_pos], s));
    P.ring_set[P.ring_pos] = 1;
    P.ring_pos = (P.ring_pos + 1) % kRing;
    return nmiss;
}

extern "C" int wm_pool_acquire(wm_expert_pool* pool, int layer, const int32_t* ids, int n, int n_src,
                               const void* gate_src, const void* up_src, const void* down_src, int64_t gate_stride,
                               int64_t up_stride, int64_t down_stride, int32_t* slots_dev, void* stream) {
    WM_CHECK_ARG(pool && gate_src && up_src && down_src);
    WM_CHECK_ARG(gate_stride >= pool->part[0] && up_stride >= pool->part[1] && down_stride >= pool->part[2]);
    const void* src[3] = {gate_src, up_src, down_src};
    const int64_t sstride[3] = {gate_stride, up_stride, down_stride};
    wm_expert_pool& P = *pool;
    return pool_acquire(pool, layer, ids, n, n_src, slots_dev, stream, [&](int i, int slot) -> int64_t {
        int64_t nb = 0;
        for (int m = 0; m < 3; m++) {
            const uint8_t* from = (const uint8_t*)src[m] + (int64_t)ids[i] * sstride[m];
            if (hipMemcpyAsync(P.base + (int64_t)slot * P.slot_bytes + P.off[m], from, (size_t)P.part[m],
                               hipMemcpyHostToDevice, P.copy) != hipSuccess) {
                fprintf(stderr, "winmoe_hip: expert pool: host-to-device copy failed\n");
                return -1;
            }
            nb += P.part[m];
        }
        return nb;
    });
}

extern "C" int wm_pool_acquire_packed(wm_expert_pool* pool, int layer, const int32_t* ids, int n, int n_src,
                                      const void* src, int64_t src_stride, int32_t* slots_dev, void* stream) {
    WM_CHECK_ARG(pool && src && src_stride >= pool->slot_bytes);
    wm_expert_pool& P = *pool;
    return pool_acquire(pool, layer, ids, n, n_src, slots_dev, stream, [&](int i, int slot) -> int64_t {
        // one copy of the expert's whole image: [gate | up | down] at the
        // slot's own part offsets, up to the end of the down part
        const int64_t nb = P.off[2] + P.part[2];
        if (hipMemcpyAsync(P.base + (int64_t)slot * P.slot_bytes, (const uint8_t*)src + (int64_t)ids[i] * src_stride,
                           (size_t)nb, hipMemcpyHostToDevice, P.copy) != hipSuccess) {
            fprintf(stderr, "winmoe_hip: expert pool: host-to-device copy failed\n");
            return -1;
        }
        return P.part[0] + P.part[1] + P.part[2];
    });
}

extern "C" int wm_pool_release(wm_expert_pool* pool, void* stream) {
    WM_CHECK_ARG(pool);
    for (int slot : pool->pending) {
        WM_FAIL_HIP(hipEventRecord(pool->done[slot], (hipStream_t)stream));
        pool->done_set[slot] = 1;
        pool->taken[slot] = 0;
    }
    pool->pending.clear();
    return WM_OK;
}

extern "C" int wm_pool_stats(const wm_expert_pool* pool, int64_t* hits, int64_t* misses, int64_t* bytes_copied) {
    WM_CHECK_ARG(pool);
    if (hits) *hits = pool->hits;
    if (misses) *misses = pool->misses;
    if (bytes_copied) *bytes_copied = pool->bytes;
    return WM_OK;
}
