// wm_persist.hip -- one decode token through the MoE block in one launch of a
// persistent kernel: one workgroup per CU, and every workgroup takes an equal
// share of every phase of the step.
//
// Workgroup w of nwg (PW streaming waves, 3 helper waves):
//   * router rows [w*rr, (w+1)*rr): reference-order fp32 logits, stored with
//     this launch's tag in the upper 32 bits, in P_REP replicas;
//   * gate/up tiles [tw0, tw1) of the shared expert and of every routed slot
//     (the same row range in every slot);
//   * down rows of its own output range [d0, d1) for every slot, which it
//     then combines itself: out[h] = sum_k w_k y_k[h] + shared, in k order.
// The workgroup's tiles form one list (TileList) of blocks: gate/up of every
// slot, the act tiles of each slot (the slot's SwiGLU outputs, read back from
// the other workgroups into operand records) a few gate/up blocks later, and
// the down tiles.  The streaming waves claim the
// entries in list order from an LDS counter; each loads its entry into its
// own LDS buffer with LDS-DMA and processes it.
//
// Hand-offs between workgroups carry the launch tag in every 64-bit word, so
// a reader needs one read of the data itself and no counter: the routing
// (logits as tag << 32 | value; every workgroup reads one replica of them
// and runs the K-pass arg-max itself) and the SwiGLU outputs of each slot
// (two outputs rounded to 24 bits and the tag's low 16 bits per word; every
// workgroup writes its row pairs into P_AREP replicas and reads one replica
// back in act tiles).  A stale word carries an older tag,
// so a reader never takes it.  The tag is epoch + 1; workgroup 0 stores the
// new epoch once it has seen every workgroup's start tag (so no workgroup can
// still read the old one; the next launch begins after this one ends).
// Nothing is reset between launches; wm_workspace_reset zeroes the words.
//
// Helper 0: router DMA and rows 0/2, routing.  Helper 1: rows 1/3, SwiGLU
// publishing, combine.  Helper 2: x into LDS (and the RMSNorm when the layer
// has one), the shared-expert gate, and in workgroup 0 the epoch.
//
// Progress: every workgroup must be resident at once (the routing needs every
// workgroup's router rows).  The host launches one workgroup per CU with more
// than half the CU's LDS, so each CU holds exactly one; a workgroup delayed by
// other work on the device only delays the step.  Every wait is bounded and
// reports WM_STATUS_SPIN_TIMEOUT when it gives up.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "../../include/winmoe_hip.h"
#include "wm_decode.h"
#include "wm_device.h"
#include "wm_launch.h"
#include "wm_wave.h"

namespace wm {

static_assert(PRING >= 1 && PRING <= 8, "a streaming wave keeps at most PRING tiles in its ring");
static_assert(3 * (PMAXK + 1) <= 64, "a wave holds one tile-list block per lane");
static_assert(PSTAGE == 2, "two helper waves besides the publisher: the router wave and the x loader");

typedef __attribute__((address_space(3))) PersistCtl lctl_t;

constexpr uint32_t PSPIN = 1u << 20;    // LDS polls (~0.2 us each after the first few) before a wait gives up

#define WM_WAIT_LGKM0() __builtin_amdgcn_s_waitcnt(0xC07F)

WM_DEV uint32_t gld_agent(const uint32_t* p) { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
WM_DEV uint64_t gld_agent64(const uint64_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// The first read of a tagged hand-off vector: through the XCD's L2, so the
// workgroups of one XCD that read the same replica share one fetch.  A line
// the L2 got before all its words were written shows an older tag; the
// retries read with agent scope, past the L2.
WM_DEV uint64_t gld_first64(const uint64_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
WM_DEV void gst_agent(uint32_t* p, uint32_t v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
WM_DEV void gst_agent64(uint64_t* p, uint64_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
WM_DEV uint64_t tagged(uint32_t tag, float v) { return ((uint64_t)tag << 32) | (uint64_t)__builtin_bit_cast(uint32_t, v); }

// LDS flag / counter read.  A volatile load, not an atomic one: the compiler
// treats an atomic LDS load as possibly depending on the wave's LDS-DMA tile
// loads and waits for all of them first (vmcnt(0)), which would drain the
// weight stream at every flag check.
WM_DEV uint32_t lds_ld(const lds32_t* p) { return *(const volatile lds32_t*)p; }
WM_DEV uint64_t lds_ld64(const lds64_t* p) { return *(const volatile lds64_t*)p; }
WM_DEV lctl_t* ctl_of(uint8_t* smem) { return (lctl_t*)smem; }

// Every LDS write of this wave is complete, then lane 0 stores v to *p (a
// word with one writer; volatile, not atomic, for the reason above), then
// s_wakeup ends the s_sleep of every waiting wave of the workgroup, so a
// waiter polls again at once instead of after its pause.
WM_DEV void lds_set(lds32_t* p, uint32_t v, int lane) {
    WM_WAIT_LGKM0();
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    if (lane == 0) *(volatile lds32_t*)p = v;
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    asm volatile("s_wakeup" ::: "memory");
}

// A wait gave up: report it and make every later wait of the workgroup end
// at once (the step's results are invalid; the launch still finishes).
WM_DEV void give_up(lctl_t* ctl, int32_t* status, int lane) {
    if (lane == 0) {
        atomicOr(status, WM_STATUS_SPIN_TIMEOUT);
        *(volatile lds32_t*)&ctl->abort = 1u;
    }
}
WM_DEV bool aborted(lctl_t* ctl) { return lds_ld(&ctl->abort) != 0u; }

// Pause between polls: 64 clocks at first, doubling to 512.  Polling waves
// share their SIMD with the streaming waves; every poll costs issue slots.
WM_DEV void backoff(uint32_t it) {
    if (it < 2) __builtin_amdgcn_s_sleep(1);
    else if (it < 4) __builtin_amdgcn_s_sleep(2);
    else if (it < 8) __builtin_amdgcn_s_sleep(4);
    else __builtin_amdgcn_s_sleep(8);
}

// The wave waits until *p >= target (bounded).
WM_DEV void lds_wait(lctl_t* ctl, const lds32_t* p, uint32_t target, int32_t* status, int lane) {
    uint32_t it = 0;
    while (lds_ld(p) < target) {
        if (++it > PSPIN || aborted(ctl)) {
            give_up(ctl, status, lane);
            break;
        }
        backoff(it);
    }
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// As lds_wait with pauses of at most 128 clocks: the waits of the helper
// waves (x loader, router, publisher), whose ends are on the step's critical
// path (the SwiGLU hand-off after a slot's last gate/up tile, the combine
// after the last down tile, a chained layer's input) while only one wave of
// the SIMD polls.  Against the doubling pause: C4 134.1 -> 128.7 us per
// token, C2 35.56 -> 35.36, C1 14.80 -> 14.67, C3 21.52 -> 21.35 us per
// step; the streaming waves' waits keep it (with the short pause there C3
// lost 0.4 us: their polls take issue slots from the tiles beside them).
WM_DEV void lds_wait_f(lctl_t* ctl, const lds32_t* p, uint32_t target, int32_t* status, int lane) {
    uint32_t it = 0;
    while (lds_ld(p) < target) {
        if (++it > PSPIN || aborted(ctl)) {
            give_up(ctl, status, lane);
            break;
        }
        if (it < 2) __builtin_amdgcn_s_sleep(1);
        else __builtin_amdgcn_s_sleep(2);
    }
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}
WM_DEV void wait_all_f(lctl_t* ctl, const lds32_t* p, int n, int32_t* status, int lane) {
    for (int i = 0; i < n; i++) lds_wait_f(ctl, p + i, 1u, status, lane);
}

// The wave waits until all n words at p are nonzero (bounded).
WM_DEV void wait_all(lctl_t* ctl, const lds32_t* p, int n, int32_t* status, int lane) {
    for (int i = 0; i < n; i++) lds_wait(ctl, p + i, 1u, status, lane);
}

WM_DEV uint64_t now() { return __builtin_amdgcn_s_memrealtime(); }

// s_waitcnt vmcnt(n), n in [0, 63] (the instructions of the later tiles in
// flight).
WM_DEV void wait_vm(int n) {
#define WM_VM_CASE(k) case k: WM_WAIT_VMCNT(k); break;
#define WM_VM_CASE8(k) WM_VM_CASE(k) WM_VM_CASE(k + 1) WM_VM_CASE(k + 2) WM_VM_CASE(k + 3) \
    WM_VM_CASE(k + 4) WM_VM_CASE(k + 5) WM_VM_CASE(k + 6) WM_VM_CASE(k + 7)
    switch (n) {
        WM_VM_CASE8(0) WM_VM_CASE8(8) WM_VM_CASE8(16) WM_VM_CASE8(24)
        WM_VM_CASE8(32) WM_VM_CASE8(40) WM_VM_CASE8(48) WM_VM_CASE(56) WM_VM_CASE(57) WM_VM_CASE(58)
        WM_VM_CASE(59) WM_VM_CASE(60) WM_VM_CASE(61) WM_VM_CASE(62)
    default: WM_WAIT_VMCNT(63); break;
    }
#undef WM_VM_CASE8
#undef WM_VM_CASE
}

// The DMA loads of one tile of type T into a ring buffer (as tile_dma; for
// Q8_0 the lanes whose 16 bytes would fall past the buffer issue nothing, so
// a buffer holds 4416 bytes instead of 5 KB).  Returns the instruction count.
template <int T> WM_DEV int ring_dma(uint64_t G, int nbytes, int lane, lds8_t* dst) {
    constexpr int NI = tile_ni<T>(), CAP = ring_tile_bytes<T>() / 16;
    const uint64_t A = G & ~(uint64_t)15;
    const int nch = (int)(((G - A) + (uint64_t)nbytes + 15) >> 4);     // granules holding the tile's bytes
#pragma unroll
    for (int k = 0; k < NI; k++) {
        int i = lane + 64 * k;
        if (64 * k + 63 < CAP || i < CAP) {     // lane 0 always issues: every instruction counts
            i = i < nch ? i : nch - 1;
            __builtin_amdgcn_global_load_lds((const void*)(uintptr_t)(A + 16 * (uint64_t)i),
                                             (__attribute__((address_space(3))) void*)(dst + 1024 * k), 16, 0, CPOL_NT);
        }
    }
    return NI;
}

// The DMA loads of an act tile (nbytes of tagged words, 16-byte aligned, a
// multiple of 256) into a ring buffer: the first read through the L2 (the
// workgroups of an XCD reading one replica share its fetch), a re-read
// (cpol CPOL_SC1) past it.  Lanes past the tile's last 16 bytes read those
// again (the buffer holds whole kilobytes of the tile).  Returns the
// instruction count.
template <int CPOL> WM_DEV int act_dma(uint64_t G, int nbytes, int lane, lds8_t* dst) {
    const int nch = nbytes >> 4, ni = (nch + 63) >> 6;
    for (int k = 0; k < ni; k++)
        __builtin_amdgcn_global_load_lds((const void*)(uintptr_t)(G + 16u * (uint32_t)min(lane + 64 * k, nch - 1)),
                                         (__attribute__((address_space(3))) void*)(dst + 1024 * k), 16, 0, CPOL);
    return ni;
}

// ------------------------------------------------------------------ tile list
// Tile lists longer than this (entries per workgroup, at most) have their
// descriptor table built by the streaming waves, shorter ones by the x loader.
constexpr int P_TAB_SPLIT = 128;
enum : int { K_SG = 0, K_SU = 1, K_RG = 2, K_RU = 3, K_SD = 4, K_RD = 5, K_ACT = 6 };
struct TRef {
    int kind, slot, t;    // t: tile within the workgroup's range
};

struct Part {
    int w, tw0, ngu, d0, ndn;
};
// floor(x / d) for wave-uniform 0 <= x <= 2^22, 0 < d <= 2^12: the fp32 quotient from
// the hardware reciprocal is within 0.75 of x / d (relative error below
// 1.5 * 2^-23 on a value at most 2^22), so the truncated quotient is off by
// at most one, which the two corrections remove.  A few VALU operations where
// the compiler's integer division is a long dependent sequence (~150
// operations for a 64-bit one), which every wave ran at the start of a step.
WM_DEV int udiv22(int x, int d) {
    uint32_t q = (uint32_t)((float)x * __builtin_amdgcn_rcpf((float)d));
    if ((int)q * d > x) q--;
    if (((int)q + 1) * d <= x) q++;
    return __builtin_amdgcn_readfirstlane((int)q);     // (uniform: its inputs are)
}

// The workgroup's share of every phase (rows w * n / nwg .. (w + 1) * n / nwg
// of each split; nwg <= 1024 and n <= 4096, so every product is below 2^22).
WM_DEV Part partition(const PersistArgs& a) {
    Part p;
    p.w = (int)blockIdx.x;
    const int gs = a.gu_step, gu_units = gs == 2 ? a.gu_tiles >> 1 : a.gu_tiles;    // (gu_step is 1 or 2)
    p.tw0 = gs * udiv22(p.w * gu_units, a.nwg);
    p.ngu = gs * udiv22((p.w + 1) * gu_units, a.nwg) - p.tw0;
    p.d0 = udiv22(p.w * a.dn_tiles, a.nwg);
    p.ndn = udiv22((p.w + 1) * a.dn_tiles, a.nwg) - p.d0;
    return p;
}

// Slot at position q of the order shared, 0 .. K-1 (shared first when present).
WM_DEV int slot_at(int q, int K, int sh) { return sh ? (q == 0 ? K : q - 1) : q; }

// The workgroup's tile list: blocks of entries, G(q) = the gate/up tiles of
// the slot at position q of the order shared, 0 .. K-1 (gate and up of a row
// adjacent), A(q) = its act tiles (the slot's SwiGLU outputs from every
// workgroup, into operand records) and D(q) = its down tiles.  A slot's
// SwiGLU outputs are complete once every workgroup has processed its G(q), so
// A(q) comes P_ALAG gate/up blocks after G(q) (the other workgroups' share
// lands meanwhile); the down blocks follow every gate/up block, and each act
// block not placed by then comes P_ALEAD down blocks before its D(q).  Every
// A(q) is after G(q) and before D(q).  Lane b of the wave holds block b's
// code (kind | position << 2) and first entry, so an entry's block is the
// count of blocks that start at or before it, minus one.  The order is built
// in registers (uniform control flow), with no memory read.  init and at are
// called with all 64 lanes active.
constexpr int P_ALAG = 3, P_ALEAD = 1;
struct TileList {
    int K, sh, g, na, dn, n;
    int v_blk, v_start;
    WM_DEV void init(const PersistArgs& a, int ngu, int ndn, int lane) {
        K = a.K; sh = a.has_shared;
        g = 2 * ngu; dn = ndn;
        na = ndn > 0 ? a.nact : 0;       // (a workgroup without down rows needs no records)
        const int nq = K + sh;
        int code = 0, size = 0, b = 0;
        auto emit = [&](int kind, int q, int sz) {
            if (lane == b) {
                code = kind | (q << 2);
                size = sz;
            }
            b++;
        };
        for (int q = 0; q < nq; q++) {
            emit(0, q, g);
            if (q >= P_ALAG) emit(1, q - P_ALAG, na);
        }
        int next_a = max(0, nq - P_ALAG);
        for (int q = 0; q < nq; q++) {
            for (; next_a < nq && next_a <= q + P_ALEAD; next_a++) emit(1, next_a, na);
            emit(2, q, dn);
        }
        v_blk = code;
        int incl = size;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const int u = __shfl_up(incl, o);
            if (lane >= o) incl += u;
        }
        n = __shfl(incl, 63);
        v_start = lane < b ? incl - size : 0x7FFFFFFF;
    }
    WM_DEV TRef at(int j) const {
        const int b = __builtin_popcountll(__builtin_amdgcn_ballot_w64(v_start <= j)) - 1;
        const int code = __builtin_amdgcn_readlane(v_blk, b), t = j - __builtin_amdgcn_readlane(v_start, b);
        return decode(code, t);
    }
    // As at(j) for a lane-varying j in [0, n) (called with all 64 lanes
    // active): the block is the count of block starts at or before j, minus
    // one; its code and start come from the lane that holds them.
    WM_DEV TRef at_lane(int j) const {
        int b = -1;
        for (int bb = 0; bb < 64; bb++) b += __builtin_amdgcn_readlane(v_start, bb) <= j ? 1 : 0;
        const int code = __shfl(v_blk, b), t = j - __shfl(v_start, b);
        return decode(code, t);
    }
    WM_DEV TRef decode(int code, int t) const {
        const int q = code >> 2, c = code & 3;
        const bool shared = sh && q == 0;
        TRef r;
        r.slot = slot_at(q, K, sh);
        if (c == 0) {
            r.kind = (t & 1) ? (shared ? K_SU : K_RU) : (shared ? K_SG : K_RG);
            r.t = t >> 1;
        } else {
            r.kind = c == 1 ? K_ACT : (shared ? K_SD : K_RD);
            r.t = t;
        }
        return r;
    }
};

// Act tile `at` of `slot`, landed in `buf` (nb bytes loaded from G): segments
// [at*aseg, (at+1)*aseg) of the slot's tagged SwiGLU outputs, in rounds of 8
// segments, 8 lanes per segment, 8 values (4 words) per lane.  While a word
// still carries an older tag (its producer has not published it yet) the
// tile is loaded again past the L2; then each lane builds its part of the
// segment's operand record and the tile is marked done for the slot's down
// tiles.  Act tiles travel in the streaming waves' own lists: a CU's memory
// pipeline serves its waves in turn, so these 4 KB per slot move at the
// streaming waves' share instead of one helper wave's.
template <int DT, int SDT>
WM_DEV void act_tile(const PersistArgs& a, lctl_t* ctl, lds8_t* lds, lds8_t* buf, uint64_t G, int nb, int slot, int at,
                     int lane) {
    const int K = a.K, nseg = a.I / SEG, part = lane & 7;
    const int nround = (a.aseg + 7) >> 3;
    lds_wait(ctl, &ctl->rows_in, 1u, a.status, lane);        // the tag is set before rows_in
    const uint32_t tag16 = ctl->tag & 0xFFFFu;
    // segment of round rd for this lane (or -1) and its 4 words in the buffer
    auto seg_of = [&](int rd) -> int {
        const int s_in = 8 * rd + (lane >> 3), seg = at * a.aseg + s_in;
        return s_in < a.aseg && seg < nseg ? seg : -1;
    };
    auto words = [&](int seg) -> const lds64_t* {
        const int col = slot == K ? seg_col(SDT, seg, 8 * part) : seg_col(DT, seg, 8 * part);
        return (const lds64_t*)buf + (col - at * a.aseg * SEG) / 2;
    };
    uint32_t it = 0;
    while (true) {
        bool ok = true;
        for (int rd = 0; rd < nround; rd++) {
            const int seg = seg_of(rd);
            if (seg >= 0) {
                const lds64_t* w = words(seg);
#pragma unroll
                for (int j = 0; j < 4; j++) ok = ok && (uint32_t)(w[j] >> 48) == tag16;
            }
        }
        if (__builtin_amdgcn_ballot_w64(!ok) == 0ull) break;
        if (++it > PSPIN_G || aborted(ctl)) {
            give_up(ctl, a.status, lane);
            break;
        }
        __builtin_amdgcn_s_sleep(4);
        wave_lds_sync();      // every lane has read the buffer before it is loaded again
        act_dma<CPOL_SC1>(G, nb, lane, buf);
        WM_WAIT_VMCNT(0);
    }
    for (int rd = 0; rd < nround; rd++) {
        const int seg = seg_of(rd);
        if (seg >= 0) {
            const lds64_t* w = words(seg);
            float v[8];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const uint64_t x = w[j];
                v[2 * j] = act_float((uint32_t)x & 0xFFFFFFu);
                v[2 * j + 1] = act_float((uint32_t)(x >> 24) & 0xFFFFFFu);
            }
            lds32_t* rec = (lds32_t*)(lds + a.o_reg) + ((int64_t)slot * nseg + seg) * XOP_DW;
            if (slot == K) xop_part<SDT>(v, part, rec);
            else xop_part<DT>(v, part, rec);
        }
    }
    lds_set(&ctl->act_done[slot][at], 1u, lane);
}

// ------------------------------------------------------------------ streaming waves
// The streaming waves claim the list entries in order from one LDS counter
// (ctl->next): a wave that is free takes the next entry, loads it into its
// own LDS buffer with LDS-DMA and processes it.  Entries therefore start in
// list order whatever each wave waited for before (a pick, a hand-off), so
// the act tiles of a slot are always taken before the slot's down tiles.
// The LDS-DMA bandwidth of a CU grows with the number of waves that issue it
// (each wave's loads complete in order), so every streaming wave issues its
// own.  The first n_rwaves buffers hold x and the router rows at the start;
// those waves send nothing before the router helpers are done with them.
//
// A wave claims and counts only while none of its LDS-DMA loads is in flight
// (one buffer per wave): the compiler makes an LDS atomic wait for all of
// them.

// A pointer / 64-bit argument as an opaque scalar value.
WM_DEV uint64_t sval64(int64_t v) {
    uint64_t r = (uint64_t)v;
    asm volatile("" : "+s"(r));
    return r;
}
WM_DEV uint64_t sval(const void* p) { return sval64((int64_t)(uintptr_t)p); }

// A tile of the list: kind, slot, byte offset in its matrix, bytes, where its
// row sums go (float index into the gate / up / down sums) and its rows.
struct TileDesc {
    int kind, slot, nb, out, rows;
    int64_t off;
};
template <int GUT, int DT, int SGUT, int SDT>
WM_DEV TileDesc tile_desc(const PersistArgs& a, const Part& P, const TRef& r, int lg_gu, int lg_dn) {
    const int K = a.K, H = a.H, I = a.I;
    if (r.kind == K_ACT) {
        // segments [t*aseg, (t+1)*aseg) of the slot's tagged SwiGLU outputs in
        // replica w % P_AREP (byte offset from a.tact; a word holds two outputs)
        TileDesc d;
        const int seg0 = r.t * a.aseg;
        d.kind = K_ACT;
        d.slot = r.slot;
        d.rows = 0;
        d.out = r.t;
        d.off = ((int64_t)(r.slot * P_AREP + P.w % P_AREP) * (I / 2) + (int64_t)seg0 * (SEG / 2)) * 8;
        d.nb = min(a.aseg, I / SEG - seg0) * SEG * 4;
        return d;
    }
    const bool gu = r.kind <= K_RU;
    const int rpt_gu = SEG >> lg_gu, rpt_dn = SEG >> lg_dn;
    const int rpt = gu ? rpt_gu : rpt_dn, rows = gu ? I : H, abs_t = (gu ? P.tw0 : P.d0) + r.t;
    // (row bytes per instantiated type: divisions by constants)
    const int64_t rb = r.kind == K_SG || r.kind == K_SU ? matrix_bytes(SGUT, 1, H) : r.kind == K_SD ? matrix_bytes(SDT, 1, I)
                     : gu ? matrix_bytes(GUT, 1, H) : matrix_bytes(DT, 1, I);
    TileDesc d;
    d.rows = min(rpt, rows - abs_t * rpt);
    d.kind = r.kind;
    d.slot = r.slot;
    d.off = (int64_t)abs_t * rpt * rb;
    d.nb = (int)((int64_t)d.rows * rb);
    d.out = gu ? (r.kind == K_SG || r.kind == K_RG ? 0 : (K + 1) * a.gu_cap) + r.slot * a.gu_cap + r.t * rpt_gu
               : r.slot * a.y_cap + r.t * rpt_dn;
    return d;
}

// A tile descriptor as the LDS table holds it (16 bytes): kind | slot << 4 |
// rows << 12, the offset in its matrix (below 2^32 for every supported shape:
// a matrix of 4096 x 4096 Q8_0 weights is 17.8 MB), where its row sums go,
// its bytes.
typedef __attribute__((address_space(3))) u32x4 lq4_t;
WM_DEV u32x4 desc_pack(const TileDesc& d) {
    u32x4 e;
    e.x = (uint32_t)d.kind | ((uint32_t)d.slot << 4) | ((uint32_t)d.rows << 12);
    e.y = (uint32_t)d.off;
    e.z = (uint32_t)d.out;
    e.w = (uint32_t)d.nb;
    return e;
}
// (the entry is the same in every lane: read as wave-uniform values)
WM_DEV TileDesc desc_unpack(const u32x4& e) {
    const uint32_t w0 = (uint32_t)__builtin_amdgcn_readfirstlane((int)e.x);
    TileDesc d;
    d.kind = (int)(w0 & 15u);
    d.slot = (int)((w0 >> 4) & 255u);
    d.rows = (int)(w0 >> 12);
    d.off = (int64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)e.y);
    d.out = __builtin_amdgcn_readfirstlane((int)e.z);
    d.nb = __builtin_amdgcn_readfirstlane((int)e.w);
    return d;
}

WM_DEV int lg_tile_lanes(int n) { return 31 - __builtin_clz((unsigned)(n / SEG)); }
WM_DEV bool routed_kind(int k) { return k == K_RG || k == K_RU || k == K_RD; }

// A chained layer's input, part `part` of nparts: the previous layer's
// tagged words (tag << 32 | value bits, 8 bytes a value; P_XREP replicas,
// replica w % P_XREP read by workgroup w) come into LDS at o_stage with
// LDS-DMA, kilobytes part, part + nparts, ... of it, the first read through
// the L2 and the re-reads of a kilobyte that still holds an older tag past
// it, until every word carries the previous layer's tag (bounded); one pass
// over each kilobyte that came in checks its tags and writes its values into
// x.  The staged words stay for the residual add.  Every wave of the
// workgroup loads a part: lines just written by other workgroups come slowly
// (~6 us for 32 KB read by one wave), and fourteen waves read them side by
// side.
WM_DEV void x_tagged_part(const PersistArgs& a, uint8_t* smem, lds8_t* xl, uint32_t tag, int part, int nparts, int lane) {
    lctl_t* ctl = (lctl_t*)smem;
    lds8_t* st = (lds8_t*)smem + a.o_stage;
    typedef __attribute__((address_space(3))) const u32x4 lq4c_t;
    const int H = a.H, nch = H / 2, units = (nch + 63) >> 6;     // 16-byte granules (two values each), KB units
    const uint8_t* src = (const uint8_t*)(a.tx_in + (int64_t)((int)blockIdx.x % P_XREP) * H);
    uint32_t pend = 0u;                                            // this part's units still to (re)load
    for (int k = part; k < units; k += nparts) pend |= 1u << k;
    uint32_t it = 0;
    bool first = true;
    while (pend) {
        for (int k = part; k < units; k += nparts) {
            if (!((pend >> k) & 1u)) continue;
            const int i = min(lane + 64 * k, nch - 1);
            if (first)
                __builtin_amdgcn_global_load_lds((const void*)(src + 16 * i), (__attribute__((address_space(3))) void*)(st + 1024 * k), 16, 0, 0);
            else
                __builtin_amdgcn_global_load_lds((const void*)(src + 16 * i), (__attribute__((address_space(3))) void*)(st + 1024 * k), 16, 0, CPOL_SC1);
        }
        WM_WAIT_VMCNT(0);
        first = false;
        uint32_t bad = 0u;
        for (int k = part; k < units; k += nparts) {
            if (!((pend >> k) & 1u)) continue;
            const int i = lane + 64 * k;
            const u32x4 q = *(lq4c_t*)(st + 16 * min(i, nch - 1));        // words 2i, 2i + 1: lo, hi, lo, hi
            const bool ok = i >= nch || (q.y == tag && q.w == tag);
            if (i < nch) {
                // (one 64-bit store of the two value words: stored as two
                // 32-bit values, or as a float2, this ROCm's compiler merged
                // them into one store holding the first value twice)
                *(lds64_t*)(xl + 8 * i) = (uint64_t)q.x | ((uint64_t)q.z << 32);
            }
            if (__builtin_amdgcn_ballot_w64(!ok) != 0ull) bad |= 1u << k;
        }
        pend = bad;
        if (!pend) break;
        if (++it > PSPIN_G || aborted(ctl)) {
            give_up(ctl, a.status, lane);
            break;
        }
        __builtin_amdgcn_s_sleep(4);
    }
    lds_set(&ctl->xpart[part], 1u, lane);
}

template <int GUT, int DT, int SGUT, int SDT>
WM_DEV void stream_wave(const PersistArgs& a, uint8_t* smem, int wave_v, uint32_t prev_tag, int lane) {
    lctl_t* ctl = (lctl_t*)smem;
    lds8_t* lds = (lds8_t*)smem;
    const int wave = __builtin_amdgcn_readfirstlane(wave_v);
    // a chained layer: this wave's part of the input first (it is on every
    // path; sending the first tile before it made it later, 133.6 -> 145.5 us
    // for the 8 C4 layers)
    if (a.tx_in) x_tagged_part(a, smem, lds + a.o_router, prev_tag, wave, PW + 1, lane);
    const int K = a.K, sh = a.has_shared, H = a.H, I = a.I;
    const int nseg_dn = I / SEG;
    // geometry (lanes per row: powers of two; a tile is 64 segments, so every
    // lane holds one)
    const int lg_gu = lg_tile_lanes(H), lg_dn = lg_tile_lanes(I);
    const int sub_gu = lane & ((1 << lg_gu) - 1), rig_gu = lane >> lg_gu;
    const int sub_dn = lane & ((1 << lg_dn) - 1), rig_dn = lane >> lg_dn;
    const bool active = wave < a.nstream;
    lds8_t* const buf = lds + a.o_ring + wave * a.ring_buf;
    const Part P = partition(a);
    lq4_t* const tab = (lq4_t*)(lds + a.o_desc);
    TileList L;
    L.init(a, P.ngu, P.ndn, lane);
    // (the host sizes the descriptor table for the longest list; a longer one
    // would be an invalid step, reported as a wait that gave up)
    if (active && L.n > a.n_desc) give_up(ctl, a.status, lane);
    const int n = active ? min(L.n, a.n_desc) : 0;
    bool rfree = wave >= a.n_rwaves;     // this wave's buffer is free of the router rows
    bool tab_ready = false;

    // the claimed entry j: its tile, source address (0: no weights) and the
    // count of load instructions sent for it
    int j = n;
    TileDesc d = {};
    uint64_t G = 0ull;
    bool sent = false;
    // The next entry and its tile: from the descriptor table once it is
    // built (until then a claim computes its tile itself).
    // take(v): entry v (lane 0's value) becomes the claimed one
    auto take = [&](uint32_t v) {
        j = min(__builtin_amdgcn_readfirstlane((int)v), n);
        if (j < n) {
            if (!tab_ready) tab_ready = lds_ld(&ctl->desc_built) >= (uint32_t)a.nstream;
            if (tab_ready) {
                const u32x4 e = tab[j];
                d = desc_unpack(e);
            } else {
                d = tile_desc<GUT, DT, SGUT, SDT>(a, P, L.at(j), lg_gu, lg_dn);
            }
        }
        sent = false;
    };
    auto claim = [&]() {
        uint32_t v = 0u;
        if (lane == 0) v = __hip_atomic_fetch_add(&ctl->next, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        take(v);
    };
    // (the addresses of the shared expert's matrices and of the SwiGLU
    // hand-off words, read once)
    const uint64_t b_sg = sval(a.sh_gate), b_su = sval(a.sh_up), b_sd = sval(a.sh_down), b_act = sval(a.tact);
    // Send the claimed tile's loads; false (nothing sent) when it needs a pick
    // or its buffer that is not available yet and !block.
    auto send = [&](bool block) -> bool {
        uint64_t base;
        if (routed_kind(d.kind)) {
            // the slot's matrix address, published by the routing with the pick
            const lds64_t* rb = (const lds64_t*)&ctl->rbase[d.slot][d.kind == K_RG ? 0 : d.kind == K_RU ? 1 : 2];
            uint64_t b = lds_ld64(rb);
            if (!b) {
                if (!block) return false;
                uint32_t it = 0;
                while ((b = lds_ld64(rb)) == 0ull) {
                    if (++it > PSPIN || aborted(ctl)) {
                        give_up(ctl, a.status, lane);
                        b = 1ull;
                        break;
                    }
                    // (a short pause throughout: picks come ~0.5 us apart, and
                    // the growing pause of the other waits made the first
                    // routed tiles late, C3 22.2 -> 21.8 us per step)
                    __builtin_amdgcn_s_sleep(1);
                }
            }
            base = b & ~1ull;
        } else {
            base = d.kind == K_SG ? b_sg : d.kind == K_SU ? b_su : d.kind == K_ACT ? b_act : b_sd;
        }
        if (!rfree) {
            if (!block) return false;
            wait_all(ctl, ctl->router_done, 2, a.status, lane);
            rfree = true;
        }
        G = base ? base + (uint64_t)d.off : 0ull;
        if (G) {
            switch (d.kind) {
            case K_SG: case K_SU: ring_dma<SGUT>(G, d.nb, lane, buf); break;
            case K_RG: case K_RU: ring_dma<GUT>(G, d.nb, lane, buf); break;
            case K_SD: ring_dma<SDT>(G, d.nb, lane, buf); break;
            case K_ACT: act_dma<0>(G, d.nb, lane, buf); break;
            default: ring_dma<DT>(G, d.nb, lane, buf); break;
            }
        }
        sent = true;
        return true;
    };

    // operand in registers and what it is: 1000 + type (x) or the slot (act)
    XOp xo;
    int xkey = -1;
    float sgate = 1.0f;
    bool have_sgate = false;
    lf32_t* sums = (lf32_t*)(lds + a.o_gu);
    lf32_t* yarr = (lf32_t*)(lds + a.o_y);

    // Row sums of the claimed tile (landed in buf).
    auto process = [&]() {
        const int kind = d.kind, slot = d.slot, out = d.out, nrow = d.rows;
        const bool has_w = G != 0ull;
        const lds8_t* tb = buf + (uint32_t)(G & 15u);
        auto rowsum = [&](auto tag_t, int lpr) -> float {
            constexpr int T = decltype(tag_t)::value;
            if (!has_w) return 0.0f;
            Seg<T> sg;
            sg.load(tb, lane);
            return row_reduce(seg_dot<T>(sg, xo), lpr);
        };
        if (kind == K_ACT) {
            act_tile<DT, SDT>(a, ctl, lds, buf, G, d.nb, slot, out, lane);
        } else if (kind <= K_RU) {
            const bool shared = kind <= K_SU;
            const int key = 1000 + (shared ? SGUT : GUT);
            if (xkey != key) {
                const int o = (shared && SGUT != GUT) ? a.o_xop2 : a.o_xop;
                xop_read((const lds32_t*)(lds + o) + sub_gu * XOP_DW, xo);
                xkey = key;
            }
            float p;
            if (SGUT == GUT || !shared) p = rowsum(std::integral_constant<int, GUT>(), 1 << lg_gu);
            else p = rowsum(std::integral_constant<int, SGUT>(), 1 << lg_gu);
            if (sub_gu == (1 << lg_gu) - 1 && rig_gu < nrow) sums[out + rig_gu] = p;
        } else {
            const bool shared = kind == K_SD;
            if (xkey != slot) {
                for (int i = 0; i < a.nact; i++) lds_wait(ctl, &ctl->act_done[slot][i], 1u, a.status, lane);
                xop_read((const lds32_t*)(lds + a.o_reg) + ((int64_t)slot * nseg_dn + sub_dn) * XOP_DW, xo);
                xkey = slot;
            }
            float p;
            if (SDT == DT || !shared) p = rowsum(std::integral_constant<int, DT>(), 1 << lg_dn);
            else p = rowsum(std::integral_constant<int, SDT>(), 1 << lg_dn);
            if (shared && a.sh_gate_inp) {
                if (!have_sgate) {
                    lds_wait(ctl, &ctl->sgate_ready, 1u, a.status, lane);
                    sgate = ctl->sgate;
                    have_sgate = true;
                }
                p = p * sgate;
            }
            if (sub_dn == (1 << lg_dn) - 1 && rig_dn < nrow) yarr[out + rig_dn] = p;
        }
    };

    // ---- the first entry (sent when its buffer is free and it needs no
    // pick), then the x operand records (8 lanes per segment, 8 segments per
    // wave) while it flies
    if (active) {
        claim();
        if (j < n && rfree) send(false);
    }
    {
        const int nseg = H / SEG, part = lane & 7;
        const bool two = sh && SGUT != GUT;
        float v[8], v2[8];
        // the normalised x lives in LDS (the router's x region) until the
        // router helpers are done, which needs this wave's records first
        lds_wait(ctl, &ctl->x_in, 1u, a.status, lane);
        // With one record type (routed and shared gate/up of one format) the
        // records wait for the first router helper's FMA chains: the chains
        // then run without the records' LDS traffic beside them and the
        // routing is known sooner (C2: 39.6 -> 39.0 us).  With two types the
        // records take twice as long and the wait costs more than it saves
        // (C3: +0.9 us).
        if constexpr (SGUT == GUT) lds_wait(ctl, &ctl->router_done[0], 1u, a.status, lane);
        const lf32_t* xl = (const lf32_t*)(lds + a.o_router);
        for (int sg = wave * 8 + (lane >> 3); sg < nseg; sg += PW * 8) {
            xop_part_fetch_lds<GUT>(xl, sg, part, v);
            if (two) xop_part_fetch_lds<SGUT>(xl, sg, part, v2);
            xop_part<GUT>(v, part, (lds32_t*)(lds + a.o_xop) + sg * XOP_DW);
            if (two) xop_part<SGUT>(v2, part, (lds32_t*)(lds + a.o_xop2) + sg * XOP_DW);
        }
        lds_set(&ctl->xop_built[wave], 1u, lane);
    }
    // A long list's descriptor table is built by the streaming waves
    // themselves (entries 64 w + lane, every 64 nstream entries), after
    // their records: with many slots the routing leaves them time to spare
    // and the x loader alone would finish it after the first claims.  A
    // short one is the x loader's.
    if (active && a.n_desc > P_TAB_SPLIT) {
        for (int j0 = 64 * wave; j0 < n; j0 += 64 * a.nstream) {
            const int jl = min(j0 + lane, n - 1);
            const TileDesc e = tile_desc<GUT, DT, SGUT, SDT>(a, P, L.at_lane(jl), lg_gu, lg_dn);
            if (j0 + lane < n) tab[jl] = desc_pack(e);
        }
        WM_WAIT_LGKM0();
        if (lane == 0) __hip_atomic_fetch_add(&ctl->desc_built, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
    wait_all(ctl, ctl->xop_built, PW, a.status, lane);
    if (wave == 0 && lane == 0) ctl->t[8] = now();

    while (j < n) {
        if (!sent) send(true);
        WM_WAIT_VMCNT(0);         // (the claimed tile's loads are the only ones in flight)
        process();
        // counted after the row sums (LDS executes one wave's operations in
        // order): gate/up tiles for the SwiGLU publisher, down tiles for the
        // combine (an act tile sets its own flags)
        if (lane == 0) {
            if (d.kind <= K_RU)
                __hip_atomic_fetch_add(&ctl->gu_done[d.slot], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
            else if (d.kind != K_ACT)
                __hip_atomic_fetch_add(&ctl->n_done, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        }
        wave_lds_sync();          // every lane's reads of the buffer are done before it is refilled
        // (the next entry is claimed only now: one claimed while this tile is
        // processed would wait behind it, and an act tile held that way holds
        // back the slot's down tiles on the other waves)
        claim();
    }
    if (wave == 0 && lane == 0) ctl->t[9] = now();
}

// ------------------------------------------------------------------ helpers: router rows

// x and router rows [r0, r0 + nr) into LDS regions of `region` bytes (x
// first, then the rows; 16-byte aligned sources; x with the default policy,
// the rows non-temporal), all in flight together.
WM_DEV void router_dma(const float* x, const float* W, int H, int r0, int qa, int qb, lds8_t* dst0, int region,
                       int lane) {
    // x (when given) into region 0, rows r0 + qa and r0 + qb (when >= 0) into
    // regions 1 + qa and 1 + qb
    const int64_t nbytes = (int64_t)H * 4;
    const int units = (int)((nbytes + 1023) >> 10);
    const int nch = (int)((nbytes + 15) >> 4);
    for (int n = 0; n < 3; n++) {
        const int q = n == 0 ? (x ? -1 : -2) : (n == 1 ? qa : qb);
        if (q == -2 || (n > 0 && q < 0)) continue;
        const uint8_t* src = (const uint8_t*)(n == 0 ? x : W + (int64_t)(r0 + q) * H);
        lds8_t* dst = dst0 + (n == 0 ? 0 : 1 + q) * region;
        for (int k = 0; k < units; k++) {
            int i = lane + 64 * k;
            i = i < nch ? i : nch - 1;
            if (n == 0)
                __builtin_amdgcn_global_load_lds((const void*)(src + 16 * i),
                                                 (__attribute__((address_space(3))) void*)(dst + 1024 * k), 16, 0, 0);
            else
                __builtin_amdgcn_global_load_lds((const void*)(src + 16 * i),
                                                 (__attribute__((address_space(3))) void*)(dst + 1024 * k), 16, 0,
                                                 CPOL_NT);
        }
    }
    WM_WAIT_VMCNT(0);
}

// Router logits of up to two of the rows in LDS: lanes 16i .. 16i+15 take row
// rsel i (none when < 0), in the reference order (transformer.h:172-191; as
// wg_router_rows): lane c of a row keeps the running fp32 FMA over columns
// c, c+16, ...; xor tree 8, 4, 2, 1 over the 16 lanes; lane 0 of the row adds
// the scalar tail.  Each logit goes with the tag in its upper 32 bits into
// all P_REP replicas (lane r of the row stores replica r).
WM_DEV void router_chains(const lds8_t* lx, int region, int H, int r0, int ra, int rb, int E, uint32_t tag,
                          uint64_t* tlogits, int lane) {
    const int q = lane >> 4, c = lane & 15;
    const int row = q == 0 ? ra : (q == 1 ? rb : -1);
    if (row < 0) return;                            // (idle lanes take no LDS bandwidth)
    const lf32_t* xr = (const lf32_t*)lx;
    const lf32_t* wr = (const lf32_t*)(lx + (1 + (row >= 0 ? row : 0)) * region);
    const int H16 = H - (H & 15), nsteps = H16 / 16;
    float acc;
    const int done = rc_steps(wr + c, xr + c, nsteps, acc);
    for (int s = done; s < nsteps; s++) acc = fmaf(wr[c + 16 * s], xr[c + 16 * s], acc);
    acc += dpp_f32<DPP_ROR8>(acc);
    acc += dpp_f32<DPP_ROR4>(acc);
    acc += dpp_f32<DPP_ROR2>(acc);
    acc += dpp_f32<DPP_ROR1>(acc);
    if (c == 0)
        for (int col = H16; col < H; col++) acc = fmaf(wr[col], xr[col], acc);
    acc = __shfl(acc, lane & ~15);                  // the row's total (lane 0 of the row) in all its lanes
    if (c < P_REP) gst_agent64(tlogits + (int64_t)c * E + r0 + row, tagged(tag, acc));
}

// The byte addresses of expert e's gate, up and down matrices for routed
// slot k, each | 1 (bit 0 marks the slot as published; the matrices are
// 16-byte aligned), or 1 alone for a slot without an expert.
WM_DEV void publish_bases(const PersistArgs& a, lctl_t* ctl, int k, int e, bool valid) {
    typedef __attribute__((address_space(3))) uint64_t l64;
    l64* rb = (l64*)&ctl->rbase[k][0];
    rb[0] = valid ? ((uint64_t)(uintptr_t)a.gate + (uint64_t)e * (uint64_t)a.gstride) | 1ull : 1ull;
    rb[1] = valid ? ((uint64_t)(uintptr_t)a.up + (uint64_t)e * (uint64_t)a.ustride) | 1ull : 1ull;
    rb[2] = valid ? ((uint64_t)(uintptr_t)a.down + (uint64_t)e * (uint64_t)a.dstride) | 1ull : 1ull;
}

// Routing from replica `rep` of the tagged logits (polled until every one
// carries `tag`), then the K-pass arg-max and
// softmax of wave_topk_n.  Lanes k < K return their pick (id, weight).
template <int MAXV>
WM_DEV void route_tagged(const PersistArgs& a, lctl_t* ctl, int rep, uint32_t tag, int lane, int& my_e, float& wk,
                         bool& degenerate, bool& nonfinite) {
    const int E = a.E, K = a.K;
    // one lane address plus constant offsets (the loads then need no address
    // registers of their own, so nothing is spilled around them)
    const uint64_t* src = a.tlogits + (int64_t)rep * E + lane;
    const uint64_t pad = (uint64_t)tag << 32;     // words past E: taken as present (never picked)
    // the first read takes every logit; later polls re-read only the words
    // that still carry an older tag (a poll of the whole vector by every
    // workgroup would take bandwidth from the weight streams)
    uint64_t tv[MAXV];
#pragma unroll
    for (int i = 0; i < MAXV; i++) tv[i] = lane + 64 * i < E ? gld_first64(src + 64 * i) : pad;
    uint32_t it = 0;
    while (true) {
        bool ok = true;
#pragma unroll
        for (int i = 0; i < MAXV; i++) ok = ok && (uint32_t)(tv[i] >> 32) == tag;
        if (__builtin_amdgcn_ballot_w64(!ok) == 0ull) break;
        if (++it > PSPIN_G || aborted(ctl)) {
            give_up(ctl, a.status, lane);
            break;
        }
        // (no pause: every re-read is a memory round trip of ~1 us; a
        // 512-clock pause between them put the routing ~0.3 us later)
#pragma unroll
        for (int i = 0; i < MAXV; i++)
            if ((uint32_t)(tv[i] >> 32) != tag) tv[i] = gld_agent64(src + 64 * i);
    }
    if (lane == 0) ctl->t[11] = now();
    float lv[MAXV];
#pragma unroll
    for (int i = 0; i < MAXV; i++) lv[i] = __builtin_bit_cast(float, (uint32_t)tv[i]);
    // (keys unsorted: pick 0 is one lane maximum and one wave maximum away,
    // and a later pick recomputes only its winning lane's maximum)
    Picker<MAXV> pk;
    pk.init_vals(lv, E, lane);
    // lane k keeps pick k's key; ids and values are decoded after the loop
    uint64_t kb = 0ull;
    degenerate = false;
    for (int k = 0; k < K; k++) {
        const uint64_t best = pk.next();
        degenerate = degenerate || best == 0ull;
        kb = lane == k ? best : kb;
        // each pick goes out at once, with its expert's gate / up / down
        // addresses: its slot's weights can start streaming
        if (lane == 0) {
            const int e = Picker<MAXV>::id_of(best);
            ctl->ids[k] = e;
            ctl->valid[k] = 1;
            publish_bases(a, ctl, k, e, true);
        }
        lds_set(&ctl->npicked, (uint32_t)(k + 1), lane);
    }
    my_e = Picker<MAXV>::id_of(kb);
    const float my_v = pk.value_of(kb);
    const bool mine = lane < K;
    // the sequential maximum over the picks in k order is pick 0's value: the
    // picks come in descending order, and a degenerate pick's value
    // (logits[0], itself invalid or already picked) never compares greater
    const float wmax = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, my_v), 0));
    const float ex = mine ? exp_rn(my_v - wmax) : 0.0f;
    float wsum = 0.0f;
    for (int k = 0; k < K; k++) wsum += __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, ex), k));
    wk = wsum > 0.0f ? ex / wsum : ex;
    nonfinite = __builtin_amdgcn_ballot_w64(mine && !isfinite(wk)) != 0ull;
}

// RMSNorm of the residual stream h in LDS, in place (attention.h:29-44), for
// H <= 256 * NST: ss = sum of (double)h[i]^2 (each product exact in fp64),
// lane l keeping four sums s_c over its elements 4l + 256k + c (k in order),
// ss_l = (s_0 + s_1) + (s_2 + s_3), then an xor tree over the lanes (32, 16,
// ..., 1); the reference adds in index order, which can differ in the last
// bits of ss, so when the two could round (float)(ss / H) differently the sum
// is taken again in index order (the scale is then the reference's bit for
// bit); scale = 1 / sqrtf((float)(ss / H) + eps) correctly rounded,
// x[i] = (h[i] * scale) * w[i], w in LDS at wl.  Straight-line code: the
// reads of a batch are in flight together.  Each region holds at least 256
// floats, so every read is inside it.
template <int NST>
WM_DEV void rmsnorm_lds(lf32_t* xl, const lf32_t* wl, int H, float eps, int lane) {
    typedef __attribute__((address_space(3))) f32x4 lf32x4_t;
    lf32x4_t* p = (lf32x4_t*)(xl + 4 * lane);
    const lf32x4_t* q = (const lf32x4_t*)(wl + 4 * lane);
    const bool in = 4 * lane < H;        // (NST > 1: H >= 512, every lane is in)
    constexpr int B = NST < 4 ? NST : 4;     // strides per batch of reads
    double s0 = 0.0, s1 = 0.0, s2 = 0.0, s3 = 0.0;
#pragma unroll
    for (int k0 = 0; k0 < NST; k0 += B) {
        f32x4 v[B];
#pragma unroll
        for (int k = 0; k < B; k++) v[k] = p[64 * (k0 + k)];
#pragma unroll
        for (int k = 0; k < B; k++) {
            s0 = fma((double)v[k].x, (double)v[k].x, s0);
            s1 = fma((double)v[k].y, (double)v[k].y, s1);
            s2 = fma((double)v[k].z, (double)v[k].z, s2);
            s3 = fma((double)v[k].w, (double)v[k].w, s3);
        }
    }
    double ss = in ? (s0 + s1) + (s2 + s3) : 0.0;
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) ss += __shfl_xor(ss, m);       // (the same value in every lane)
    // The reference adds the squares in index order (attention.h:31-34).  The
    // terms are exact and non-negative, so any order of the H - 1 additions is
    // within (H - 1) * 2^-53 of the exact sum relative to it: this sum and the
    // reference's differ by less than 2H * 2^-53 * ss, and after the division
    // (each correctly rounded) qt = ss / H differs from the reference's by
    // less than dq.  Rounding to float is monotonic: when qt - dq and qt + dq
    // round to the same float, so does the reference's quotient.  Otherwise (a
    // float rounding boundary within dq of qt: about one vector in 10^5 at
    // H = 4096) the sum is taken again in index order.
    const double qt = ss / (double)H;
    const double dq = qt * ((double)(2 * H + 8) * 0x1p-53) * 1.0625;
    if ((float)(qt - dq) != (float)(qt + dq)) {
        const lf32_t* hx = xl;
        double s = 0.0;
        for (int i = 0; i < H; i++) {
            const double v = (double)hx[i];
            s += v * v;                      // (exact product, rounded sum: the reference's step)
        }
        ss = s;
    }
    const float scale = __fdiv_rn(1.0f, __fsqrt_rn((float)(ss / (double)H) + eps));
#pragma unroll
    for (int k0 = 0; k0 < NST; k0 += B) {
        f32x4 v[B], wv[B];
#pragma unroll
        for (int k = 0; k < B; k++) {
            v[k] = p[64 * (k0 + k)];
            wv[k] = q[64 * (k0 + k)];
        }
#pragma unroll
        for (int k = 0; k < B; k++) {
            f32x4 o;
            o.x = (v[k].x * scale) * wv[k].x;
            o.y = (v[k].y * scale) * wv[k].y;
            o.z = (v[k].z * scale) * wv[k].z;
            o.w = (v[k].w * scale) * wv[k].w;
            if (in) p[64 * (k0 + k)] = o;
        }
    }
    WM_WAIT_LGKM0();
}

// H floats (16-byte aligned) into LDS at dst with LDS-DMA, 1 KB per
// instruction (lanes past the end reload the last granule); no wait.
WM_DEV void vec_dma(const float* src, int H, lds8_t* dst, int lane) {
    const int units = (H * 4 + 1023) >> 10, nch = (H * 4 + 15) >> 4;
    for (int k = 0; k < units; k++) {
        const int i = min(lane + 64 * k, nch - 1);
        __builtin_amdgcn_global_load_lds((const void*)((const uint8_t*)src + 16 * i),
                                         (__attribute__((address_space(3))) void*)(dst + 1024 * k), 16, 0, 0);
    }
}

// A short tile list as descriptors in LDS (64 entries per pass), then
// desc_built: run by the x loader once x is in, so that no streaming wave
// spends its start on it (a streaming wave computes the descriptor of each
// entry it claims until the table is there).
template <int GUT, int DT, int SGUT, int SDT>
WM_DEV void desc_table(const PersistArgs& a, uint8_t* smem, int lane) {
    lctl_t* ctl = (lctl_t*)smem;
    if (a.n_desc > P_TAB_SPLIT) return;      // (the streaming waves build a long one)
    lq4_t* const tab = (lq4_t*)((lds8_t*)smem + a.o_desc);
    const Part P = partition(a);
    TileList L;
    L.init(a, P.ngu, P.ndn, lane);
    const int n = min(L.n, a.n_desc);
    const int lg_gu = lg_tile_lanes(a.H), lg_dn = lg_tile_lanes(a.I);
    for (int j0 = 0; j0 < n; j0 += 64) {
        const int jl = min(j0 + lane, n - 1);
        const TileDesc e = tile_desc<GUT, DT, SGUT, SDT>(a, P, L.at_lane(jl), lg_gu, lg_dn);
        if (j0 + lane < n) tab[jl] = desc_pack(e);
    }
    lds_set(&ctl->desc_built, (uint32_t)a.nstream, lane);
}

// x into the region at xl and the RMSNorm in place, for H <= 256 * NST; the
// norm weights land at o_norm (over the operand records, which are built
// only after x is in) with x.
template <int NST> WM_DEV void x_norm_in(const PersistArgs& a, uint8_t* smem, lds8_t* xl, uint32_t prev_tag, int lane) {
    lds8_t* wl = (lds8_t*)smem + a.o_norm;
    if (a.tx_in) {
        vec_dma(a.norm_w, a.H, wl, lane);
        x_tagged_part(a, smem, xl, prev_tag, PW, PW + 1, lane);
        wait_all_f(ctl_of(smem), ctl_of(smem)->xpart, PW + 1, a.status, lane);
    } else {
        vec_dma(a.x, a.H, xl, lane);
        vec_dma(a.norm_w, a.H, wl, lane);
    }
    WM_WAIT_VMCNT(0);
    rmsnorm_lds<NST>((lf32_t*)xl, (const lf32_t*)wl, a.H, a.norm_eps, lane);
}

// The x loader (the second helper wave): x into the router region (every
// wave's x operand records are built from there), the RMSNorm in place when
// the layer has one (its weights come in with x), the shared expert's gate,
// the tile descriptor table.
template <int GUT, int DT, int SGUT, int SDT>
WM_DEV void helper_xload(const PersistArgs& a, uint8_t* smem, uint32_t prev_tag, int lane) {
    lctl_t* ctl = (lctl_t*)smem;
    __builtin_amdgcn_s_setprio(3);
    lds8_t* xl = (lds8_t*)smem + a.o_router;
    if (a.norm_w) {
        switch ((a.H + 255) / 256) {
        case 1: x_norm_in<1>(a, smem, xl, prev_tag, lane); break;
        case 2: x_norm_in<2>(a, smem, xl, prev_tag, lane); break;
        case 4: x_norm_in<4>(a, smem, xl, prev_tag, lane); break;
        case 8: x_norm_in<8>(a, smem, xl, prev_tag, lane); break;
        default: x_norm_in<16>(a, smem, xl, prev_tag, lane); break;
        }
    } else if (a.tx_in) {
        x_tagged_part(a, smem, xl, prev_tag, PW, PW + 1, lane);
        wait_all_f(ctl, ctl->xpart, PW + 1, a.status, lane);
    } else {
        router_dma(a.x, nullptr, a.H, 0, -1, -1, xl, a.x_region, lane);
    }
    lds_set(&ctl->x_in, 1u, lane);
    __builtin_amdgcn_s_setprio(0);
    // the shared expert's sigmoid gate (fp64 dot with x, winmoe_inference.c:2005-2009)
    if (a.has_shared && a.sh_gate_inp) {
        const float g = wave_shgate_lds((const lf32_t*)xl, a.sh_gate_inp, a.H, lane);
        if (lane == 0) ctl->sgate = g;
    }
    lds_set(&ctl->sgate_ready, 1u, lane);
    desc_table<GUT, DT, SGUT, SDT>(a, smem, lane);
    // workgroup 0 advances the epoch once every workgroup has posted this
    // launch's tag (each has read the old epoch by then); the next launch
    // starts only after this one ends, so the new value is read only then
    if (blockIdx.x == 0) {
        lds_wait_f(ctl, &ctl->rows_in, 1u, a.status, lane);       // (the tag is set before rows_in)
        const uint32_t tag = ctl->tag;
        for (int i = lane; i < a.nwg; i += 64) {
            uint32_t it = 0;
            while (gld_agent(a.hello + i) != tag) {
                if (++it > PSPIN_G || aborted(ctl)) {
                    atomicOr(a.status, WM_STATUS_SPIN_TIMEOUT);
                    break;
                }
                __builtin_amdgcn_s_sleep(8);
            }
        }
        WM_WAIT_VMCNT(0);
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        if (lane == 0) gst_agent(a.epoch, tag);
    }
}

// ------------------------------------------------------------------ helper 0: router rows, routing, operand records

template <int GUT, int DT, int SGUT, int SDT>
WM_DEV void helper_router(const PersistArgs& a, uint8_t* smem, int lane) {
    lctl_t* ctl = (lctl_t*)smem;
    lds8_t* lds = (lds8_t*)smem;
    const Part P = partition(a);
    const int K = a.K, E = a.E;
    const uint64_t t0 = now();
    const uint32_t tag = gld_agent(a.epoch) + 1u;
    if (lane == 0) {
        ctl->t[0] = t0;
        ctl->tag = tag;
        gst_agent(a.hello + P.w, tag);
    }
    int my_e = 0;
    float wk = 0.0f;
    bool valid = false;
    if (!a.forced) {
        const int r0 = P.w * a.rr, nr = max(0, min(a.rr, E - r0));
        // rows 0 and 2 here, rows 1 and 3 on the publishing helper, x on the
        // second staging wave: three waves' loads land together
        if (nr > 0) router_dma(nullptr, a.router, a.H, r0, 0, nr > 2 ? 2 : -1, lds + a.o_router, a.x_region, lane);
        lds_wait_f(ctl, &ctl->x_in, 1u, a.status, lane);
        lds_set(&ctl->rows_in, 1u, lane);          // (also when this workgroup has no router rows)
        if (lane == 0) ctl->t[1] = now();
        if (nr > 0)   // rows 0 and 2 here, rows 1 and 3 on the other helper
            router_chains(lds + a.o_router, a.x_region, a.H, r0, 0, nr > 2 ? 2 : -1, E, tag, a.tlogits, lane);
        lds_set(&ctl->router_done[0], 1u, lane);
        if (lane == 0) ctl->t[2] = now();
        bool degenerate = false, nonfinite = false;
        if (E <= 64) route_tagged<1>(a, ctl, P.w % P_REP, tag, lane, my_e, wk, degenerate, nonfinite);
        else if (E <= 512) route_tagged<8>(a, ctl, P.w % P_REP, tag, lane, my_e, wk, degenerate, nonfinite);
        else route_tagged<16>(a, ctl, P.w % P_REP, tag, lane, my_e, wk, degenerate, nonfinite);
        valid = lane < K;
        if (P.w == 0) {
            if (lane < K) {
                a.ids[lane] = my_e;
                a.w[lane] = wk;
                if (a.hits) atomicAdd(a.hits + my_e, 1u);
            }
            const int st = (degenerate ? WM_STATUS_DEGENERATE_ROUTING : 0) | (nonfinite ? WM_STATUS_NONFINITE_WEIGHT : 0);
            if (lane == 0 && st) atomicOr(a.status, st);
        }
    } else {
        lds_set(&ctl->rows_in, 1u, lane);
        lds_set(&ctl->router_done[0], 1u, lane);
        if (lane < K) {
            my_e = a.forced_ids[lane];
            wk = a.forced_w[lane];
            valid = my_e >= 0 && my_e < E;
            if (P.w == 0) {
                a.ids[lane] = my_e;
                a.w[lane] = wk;
                if (valid) { if (a.hits) atomicAdd(a.hits + my_e, 1u); }
                else atomicOr(a.status, WM_STATUS_BAD_EXPERT_ID);
            }
        }
    }
    if (lane < K) {
        ctl->ids[lane] = my_e;
        ctl->w[lane] = valid ? wk : 0.0f;
        ctl->valid[lane] = valid ? 1 : 0;
        if (a.forced) publish_bases(a, ctl, lane, my_e, valid);     // (routed: with each pick)
    }
    lds_set(&ctl->npicked, (uint32_t)K, lane);     // (forced routing: all at once)
    lds_set(&ctl->routed, 1u, lane);
    __builtin_amdgcn_s_setprio(0);
    if (lane == 0) ctl->t[3] = now();
}

// ------------------------------------------------------------------ helper 1: router rows, shared gate, SwiGLU publisher, combine

template <int GUT, int DT, int SGUT, int SDT>
WM_DEV void helper_publish(const PersistArgs& a, uint8_t* smem, int lane) {
    lctl_t* ctl = (lctl_t*)smem;
    lds8_t* lds = (lds8_t*)smem;
    const Part P = partition(a);
    const int K = a.K, sh = a.has_shared, nq = K + sh;
    if (!a.forced) {
        const int r0 = P.w * a.rr, nr = max(0, min(a.rr, a.E - r0));
        if (nr > 1) router_dma(nullptr, a.router, a.H, r0, 1, nr > 3 ? 3 : -1, lds + a.o_router, a.x_region, lane);
    }
    lds_wait_f(ctl, &ctl->rows_in, 1u, a.status, lane);
    const uint32_t tag = ctl->tag;
    // The SwiGLU hand-off words carry the tag's low 16 bits: every launch of
    // the layer rewrites every word a launch can read (each slot's I
    // outputs in every replica, an invalid pick's as zeros), so a word is
    // at most one launch old and never carries the current 16 bits stale.
    const uint64_t tg16 = (uint64_t)(tag & 0xFFFFu) << 48;
    if (!a.forced) {
        const int r0 = P.w * a.rr, nr = max(0, min(a.rr, a.E - r0));
        if (nr > 1) router_chains(lds + a.o_router, a.x_region, a.H, r0, 1, nr > 3 ? 3 : -1, a.E, tag, a.tlogits, lane);
    }
    // the x loader computes the shared gate from x in the router region: that
    // region is given up (router_done) only after it is done
    if (sh && a.sh_gate_inp) lds_wait_f(ctl, &ctl->sgate_ready, 1u, a.status, lane);
    lds_set(&ctl->router_done[1], 1u, lane);
    __builtin_amdgcn_s_setprio(0);

    lf32_t* garr = (lf32_t*)(lds + a.o_gu);
    lf32_t* uarr = garr + (K + 1) * a.gu_cap;
    lf32_t* yarr = (lf32_t*)(lds + a.o_y);
    // the counts of this workgroup's list (TileList: per slot, 2 * ngu gate/up
    // tiles, nact act tiles when it has down rows, ndn down tiles); building
    // the list itself here took ~2 us of this wave's time
    const int n_gu = 2 * P.ngu, n_dn = nq * P.ndn;
    if (P.ngu > 0) {
        const int rpt = geometry(GUT, a.H).rpt;
        const int row0 = P.tw0 * rpt, nrows = min(a.I, (P.tw0 + P.ngu) * rpt) - row0;
        for (int q = 0; q < nq; q++) {
            const int slot = slot_at(q, K, sh);
            lds_wait_f(ctl, &ctl->gu_done[slot], (uint32_t)n_gu, a.status, lane);
            __builtin_amdgcn_s_setprio(2);
            if (lane == 0 && q < 12) ctl->t[16 + q] = now();
            const bool valid = slot == K || ctl->valid[slot] != 0;
            uint64_t* dst = a.tact + (int64_t)slot * P_AREP * (a.I / 2) + row0 / 2;
            // rows x replicas over the lanes (one output each); the lane of
            // an even row takes the next row's code from the lane P_AREP up
            // and stores the pair as one tagged word (row0 and nrows are
            // even, and 64 lanes hold whole pairs)
            for (int i0 = 0; i0 < nrows * P_AREP; i0 += 64) {
                const int i = i0 + lane, r = i / P_AREP, rp = i - r * P_AREP, o = slot * a.gu_cap + r;
                const bool in = i < nrows * P_AREP;
                const uint32_t c = act24(in && valid ? silu_mul(garr[o], uarr[o]) : 0.0f);
                const uint32_t c1 = (uint32_t)__shfl_down((int)c, P_AREP);
                if (in && !(r & 1)) gst_agent64(dst + (int64_t)rp * (a.I / 2) + r / 2, tg16 | ((uint64_t)c1 << 24) | c);
            }
            __builtin_amdgcn_s_setprio(0);
        }
    }
    if (lane == 0) ctl->t[4] = now();
    if (P.ndn > 0) {
        const int rpt = geometry(DT, a.I).rpt;
        const int h0 = P.d0 * rpt, nrows = min(a.H, (P.d0 + P.ndn) * rpt) - h0;
        // the routing weights into registers while the down tiles finish
        lds_wait_f(ctl, &ctl->routed, 1u, a.status, lane);     // the weights come after the last pick
        typedef __attribute__((address_space(3))) const uint64_t l64c_t;
        const l64c_t* stw = (const l64c_t*)(lds + a.o_stage);     // (a chained launch's staged input)
        const uint32_t otag = ctl->tag;
        bool vk[PMAXK];
        float wk[PMAXK];
#pragma unroll
        for (int k = 0; k < PMAXK; k++) {
            vk[k] = k < K && ctl->valid[k] != 0;
            wk[k] = k < K ? ctl->w[k] : 0.0f;
        }
        lds_wait_f(ctl, &ctl->n_done, (uint32_t)n_dn, a.status, lane);   // every down tile is processed
        if (lane == 0) ctl->t[6] = now();
        for (int r = lane; r < nrows; r += 64) {
            // out[h] = sum_k w_k y_k[h] (k order, invalid ids skipped) + gate * y_shared[h]
            float y[PMAXK];
#pragma unroll
            for (int k = 0; k < PMAXK; k++) y[k] = vk[k] ? yarr[k * a.y_cap + r] : 0.0f;
            const float ys = sh ? yarr[K * a.y_cap + r] : 0.0f;
            // (in a chained launch the input is the staged tagged words)
            const float xr = !a.add_res ? 0.0f
                           : a.tx_in ? __builtin_bit_cast(float, (uint32_t)stw[h0 + r]) : a.x[h0 + r];
            float acc = 0.0f;
#pragma unroll
            for (int k = 0; k < PMAXK; k++)
                if (vk[k]) acc = fmaf(wk[k], y[k], acc);
            if (sh) acc = acc + ys;
            if (a.add_res) acc = xr + acc;          // residual + moe_out
            a.out[h0 + r] = acc;
            if (a.tx_out) {
                const uint64_t tw = tagged(otag, acc);
#pragma unroll
                for (int q = 0; q < P_XREP; q++) gst_agent64(a.tx_out + (int64_t)q * a.H + h0 + r, tw);
            }
        }
    }

    if (lane == 0) ctl->t[7] = now();
    if (a.timeline && lane < P_TL) a.timeline[(int64_t)P.w * P_TL + lane] = ctl->t[lane];
}

// ------------------------------------------------------------------ kernel

template <int GUT, int DT, int SGUT, int SDT>
__global__ __launch_bounds__(PTHREADS) void k_decode_persist(PersistArgs a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    for (int i = threadIdx.x; i < (int)(sizeof(PersistCtl) / 4); i += PTHREADS)
        ((lds32_t*)(lds8_t*)smem)[i] = 0u;
    // the timeout test hook: every wait gives up at its first unsuccessful poll
    if (threadIdx.x == 0 && a.probe) ((PersistCtl*)smem)->abort = 1u;
    __syncthreads();
    // the arguments through a pointer the compiler cannot see through: each
    // role loads the words it needs after the barrier (loaded before it, they
    // came in several waited rounds, each one cold-cache latency, before any
    // wave could start)
    typedef const __attribute__((address_space(4))) PersistArgs kargs_t;
    kargs_t* ka = (kargs_t*)__builtin_amdgcn_kernarg_segment_ptr();      // (the only kernel argument)
    asm volatile("" : "+s"(ka));
    const PersistArgs* ap = (const PersistArgs*)ka;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    if (wave < PW) stream_wave<GUT, DT, SGUT, SDT>(*ap, smem, wave, 0u, lane);
    // the router rows and the routing are the critical path: the helper
    // waves win the issue arbitration against the streaming waves until the
    // routing is known (their later polling must not)
    else if (wave == PW) { __builtin_amdgcn_s_setprio(3); helper_router<GUT, DT, SGUT, SDT>(*ap, smem, lane); }
    else if (wave == PW + 1) { __builtin_amdgcn_s_setprio(3); helper_publish<GUT, DT, SGUT, SDT>(*ap, smem, lane); }
    else if (wave == PW + 2) helper_xload<GUT, DT, SGUT, SDT>(*ap, smem, 0u, lane);
}

// Layers chained in one launch: layer l's input is layer l-1's output, handed
// over in tagged words (PersistArgs::tx_out / tx_in) so that a workgroup
// starts a layer as soon as it is done with the previous one (its first
// weight tiles load while the previous layer's last outputs arrive) instead
// of after a kernel boundary.  Each layer runs the step above with its own
// arguments and workspace; the control block is cleared between layers.
template <int GUT, int DT, int SGUT, int SDT>
__global__ __launch_bounds__(PTHREADS) void k_decode_stack(StackArgs sa) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    typedef const __attribute__((address_space(4))) StackArgs kargs_t;
    kargs_t* ka = (kargs_t*)__builtin_amdgcn_kernarg_segment_ptr();      // (the only kernel argument)
    asm volatile("" : "+s"(ka));
    const StackArgs* sp = (const StackArgs*)ka;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int nl = sp->n;
    lctl_t* ctl = (lctl_t*)smem;
    // Every wave meets the same three barriers per layer: the control block
    // is clear (the x loader clears it), the layer is done, its tag is read.
    auto layer_end = [&](uint32_t& tag) {
        __builtin_amdgcn_s_setprio(0);
        __syncthreads();
        tag = *(const volatile lds32_t*)&ctl->tag;     // the tag this layer's outputs carry
        __syncthreads();
    };
    uint32_t prev_tag = 0u;
    if (wave < PW) {
        for (int l = 0; l < nl; l++) {
            __syncthreads();
            int ln = lane;
            asm volatile("" : "+v"(ln));      // (nothing derived from the lane is kept across layers)
            stream_wave<GUT, DT, SGUT, SDT>(sp->L[l], smem, wave, prev_tag, ln);
            layer_end(prev_tag);
        }
    } else if (wave == PW) {
        for (int l = 0; l < nl; l++) {
            __syncthreads();
            __builtin_amdgcn_s_setprio(3);
            int ln = lane;
            asm volatile("" : "+v"(ln));
            helper_router<GUT, DT, SGUT, SDT>(sp->L[l], smem, ln);
            layer_end(prev_tag);
        }
    } else if (wave == PW + 1) {
        for (int l = 0; l < nl; l++) {
            __syncthreads();
            __builtin_amdgcn_s_setprio(3);
            int ln = lane;
            asm volatile("" : "+v"(ln));
            helper_publish<GUT, DT, SGUT, SDT>(sp->L[l], smem, ln);
            layer_end(prev_tag);
        }
    } else {
        for (int l = 0; l < nl; l++) {
            for (int i = lane; i < (int)(sizeof(PersistCtl) / 4); i += 64) ((lds32_t*)(lds8_t*)smem)[i] = 0u;
            if (lane == 0 && sp->L[l].probe) ctl->abort = 1u;
            WM_WAIT_LGKM0();
            __syncthreads();
            int ln = lane;
            asm volatile("" : "+v"(ln));
            helper_xload<GUT, DT, SGUT, SDT>(sp->L[l], smem, prev_tag, ln);
            layer_end(prev_tag);
        }
    }
}

template <int GUT, int DT, int SGUT, int SDT>
static int launch_p(const PersistArgs& a, size_t lds, hipStream_t s) {
    static size_t configured = 0;
    if (configured < lds) {
        hipError_t e = hipFuncSetAttribute((const void*)k_decode_persist<GUT, DT, SGUT, SDT>,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return (int)e;
        configured = lds;
    }
    hipLaunchKernelGGL((k_decode_persist<GUT, DT, SGUT, SDT>), dim3(a.nwg), dim3(PTHREADS), lds, s, a);
    return (int)hipGetLastError();
}

template <int GUT, int DT, int SGUT, int SDT>
static int launch_st(const StackArgs& a, size_t lds, hipStream_t s) {
    static size_t configured = 0;
    if (configured < lds) {
        hipError_t e = hipFuncSetAttribute((const void*)k_decode_stack<GUT, DT, SGUT, SDT>,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return (int)e;
        configured = lds;
    }
    hipLaunchKernelGGL((k_decode_stack<GUT, DT, SGUT, SDT>), dim3(a.L[0].nwg), dim3(PTHREADS), lds, s, a);
    return (int)hipGetLastError();
}

#define WM_P_CASE(g, d, sg, sd) \
    if (gut == g && dt == d && sgut == sg && sdt == sd) return launch_p<g, d, sg, sd>(a, lds, s);

int launch_persist(const PersistArgs& a, size_t lds, int gut, int dt, int sgut, int sdt, hipStream_t s) {
    WM_P_CASE(Q8_0, Q8_0, Q8_0, Q8_0)
    WM_P_CASE(Q2_K, Q2_K, Q2_K, Q2_K)
    WM_P_CASE(Q3_K, Q3_K, Q3_K, Q3_K)
    WM_P_CASE(Q4_K, Q4_K, Q4_K, Q4_K)
    WM_P_CASE(Q5_K, Q5_K, Q5_K, Q5_K)
    WM_P_CASE(Q6_K, Q6_K, Q6_K, Q6_K)
    WM_P_CASE(Q4_K, Q6_K, Q8_0, Q8_0)
    WM_P_CASE(Q4_K, Q6_K, Q4_K, Q6_K)
    WM_P_CASE(Q4_K, Q5_K, Q8_0, Q8_0)
    WM_P_CASE(Q4_K, Q5_K, Q4_K, Q5_K)
    WM_P_CASE(Q2_K, Q3_K, Q8_0, Q8_0)
    WM_P_CASE(Q2_K, Q3_K, Q2_K, Q3_K)
    return -1;
}

#define WM_S_CASE(g, d, sg, sd) \
    if (gut == g && dt == d && sgut == sg && sdt == sd) return launch_st<g, d, sg, sd>(a, lds, s);

int launch_stack(const StackArgs& a, size_t lds, int gut, int dt, int sgut, int sdt, hipStream_t s) {
    WM_S_CASE(Q8_0, Q8_0, Q8_0, Q8_0)
    WM_S_CASE(Q2_K, Q3_K, Q2_K, Q3_K)
    WM_S_CASE(Q4_K, Q6_K, Q8_0, Q8_0)
    return -1;
}

bool stack_supported(int gut, int dt, int sgut, int sdt) {
    return (gut == Q8_0 && dt == Q8_0 && sgut == Q8_0 && sdt == Q8_0) || (gut == Q2_K && dt == Q3_K && sgut == Q2_K && sdt == Q3_K) ||
           (gut == Q4_K && dt == Q6_K && sgut == Q8_0 && sdt == Q8_0);
}

bool persist_supported(int gut, int dt, int sgut, int sdt) { return decode_step_supported(gut, dt, sgut, sdt); }

}  // namespace wm
