// wm_pf_gemm.h -- the grouped expert GEMMs of the batched prefill (fp16 MFMA),
// for every supported weight format.  Included by wm_prefill.hip (Q8_0
// instances, the prefill launcher) and wm_prefill_kq.hip (K-quant instances).
// Internal; not part of the public ABI.
//
// One workgroup per CU works through a static list of items: item j of a
// launch is (pass, block of 128 matrix rows), and workgroup b takes items
// k, k + grid, k + 2 grid, ... with k = pf_item_slot(b) (the row blocks of a
// pass on workgroups of one XCD).  For each item it streams the block's rows (of
// gate and up, or of down) through an S-stage LDS ring, 256 columns per
// stage (Q8_0: 8 blocks; K-quants: one super-block, or two when gate and up
// alternate with passes of 16 pairs: 512 columns), filled by global_load_lds:
//   * weights: each row's stage chunk as GR granules of 16 B from the
//     16-byte boundary at or before the row start plus the 16-byte boundary
//     at or before the chunk's offset in the row (Q8_0 272 B, Q4_K 144 B and
//     Q5_K 176 B start aligned: 17, 9 and 11 granules; Q2_K 84 B, Q3_K 110 B
//     and Q6_K 210 B start up to 24 or 28 bytes in: 7, 9 and 15; two Q2_K,
//     Q3_K or Q4_K super-blocks 13, 17 and 19, an odd count: gm_granules).
//     Longer runs per row stream faster: a probe of this
//     one-workgroup-per-CU ring reads 136-byte row pieces at 4.6 TB/s,
//     272-byte ones at 5.5;
//   * activations: the pass's M rows x KC fp16 (M = 16 or 32, the pass
//     size the launch was grouped with), rows one pad granule
//     longer than their data, so the MFMA operand reads of 16 rows hit 16
//     different 16-byte slots of a 256-byte bank cycle;
//   * the activations' power-of-two scales of the stage (one dword per row
//     and 128 columns).
// The ring runs across item boundaries: the next item's first stages are in
// flight while the current one finishes.  Waves 0-7 issue the loads and do
// the maths (16 rows each); wave 8 only writes results, because vector
// stores count in vmcnt: issued by the compute waves they would hold up the
// "stage landed" waits.
//
// Weights become fp16 exactly (small integers under the exponent byte 0x64
// are 1024 + q; minus 1024 + bias), so v_mfma_f32_16x16x32_f16 gives the dot
// product of 32 weights with the scaled fp16 activations:
//   * Q8_0 (q8_dequant.h:15-18): one MFMA per 32-weight block (byte ^ 0x80
//     is q + 128), times the block's fp16 scale d;
//   * Q4_K / Q5_K (q4k_dequant.h:112-168, q5k_dequant.h:98-131): one MFMA
//     per 32-weight sub-block, times d*sc; the min term dmin*m times the
//     sub-block's activation sum, an MFMA of the activations with ones;
//   * Q6_K / Q3_K / Q2_K (q6k_dequant.h:112-141 and the public ggml
//     layouts): 16-weight sub-blocks, so two MFMAs per 32 columns, each with
//     the other half of the weight operand zero (lanes 0-31 hold k 0-15,
//     lanes 32-63 k 16-31), times the sub-block's multiplier; Q2_K's mins
//     as above with half-masked ones.
// The activation scale multiplies the sum of each 128 columns.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "wm_device.h"
#include "wm_format.h"
#include "wm_wave.h"

namespace wm {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

WM_DEV int pair_token(int p, int T, int K) { return p < T * K ? p / K : p - T * K; }

// Exponent e with m * 2^-e in [2^14, 2^15) for a finite m > 0 (clamped to
// e >= -126 so that 2^e and 2^-e are normal floats); 0 otherwise.  Values of
// a group scaled by 2^-e fit fp16 with its full 11-bit precision down to
// 2^-29 of the group maximum.
WM_DEV int pf_exp(float m) {
    if (!(m > 0.0f) || !(m <= 3.402823466e38f)) return 0;
    int E;
    frexpf(m, &E);                 // m in [2^(E-1), 2^E)
    return max(E - 15, -126);
}

// Expert passes: a pass is up to M pairs of one expert (M = 16 or 32, one
// value per launch), described by a record of GM_REC ints: expert (E =
// shared), pair count, 0, 0, GM_M pair ids (positions past the count repeat
// the last id), then the x scale exponents of the pairs' tokens, 4 signed
// bytes per int, for GM_M pairs.  The record layout is the same for both pass
// sizes.
constexpr int GM_M = 32;
constexpr int GM_REC = 64;

constexpr int GM_ROWS = 128;          // matrix rows per item
constexpr int GM_CW = 8;              // compute waves
constexpr int GM_THREADS = 64 * (GM_CW + 1);
constexpr int GM_DESC = 8;            // pass records held in LDS

// Columns per super-block of a stage (a stage holds NSB of them; the column
// steps of an item are the matrix width over NSB x 256).
constexpr int GM_KC = 256;

// Granules of 16 B loaded per row and stage for format WT (nsb
// super-blocks; Q8_0: nsb x 8 blocks): enough to hold the chunk wherever it
// starts (the chunk plus the row start's and the chunk offset's distances
// past a 16-byte boundary: none for Q8_0, Q4_K and Q5_K, whose rows and
// chunks start aligned; up to 12 bytes each for Q2_K, 14 for Q3_K and Q6_K),
// rounded up to an odd count.  A row's LDS slot is then an odd multiple of
// 4 dwords long, so the slots of 16 consecutive rows start on 16 different
// groups of 4 banks (of 64) and the 8-byte reads of half a wave (16 rows x
// 2 lanes) hit 64 different banks; with an even count rows 8 apart, or
// closer, shared banks.
constexpr int gm_granules(int wt, int nsb) {
    const int bytes = wt == Q8_0 ? nsb * 272 : nsb * block_bytes(wt);
    const int mis = wt == Q2_K ? 12 : (wt == Q3_K || wt == Q6_K) ? 14 : 0;
    return ((bytes + 2 * mis + 15) / 16) | 1;
}

// LDS bytes of a GEMM's layout (GmGeo) with an s-stage weight ring, passes
// of m pairs and stages of nsb x 256 columns.
constexpr int gm_lds(int nmat, int ahl, int nsub, int wt, int m, int s, int nsb) {
    const bool gu = ahl == 1;
    const int w = nmat * GM_ROWS * 16 * gm_granules(wt, nsb);
    const int a_slot = ahl * ((m * (nsb * GM_KC / 8 + 1) + 63) / 64) * 1024 + 256;
    const int nas = (s - 1 + nsub - 1) / nsub + 1;
    return s * w + nas * a_slot + GM_DESC * GM_REC * 4 +
           (gu ? m * GM_CW * 4 + m * GM_ROWS * 4 + m * 4 : 16 * GM_ROWS * 4);
}

// NSB: 256-column super-blocks per stage (2: a K-quant row's chunk of two
// super-blocks, twice the run per row at the same stage size when gate and
// up alternate).
template <int NMAT, int AHL, int NSUB, int WT, int M, int NSB> struct GmGeo {
    static_assert(M == 16 || M == 32, "pass size");
    static_assert(NSB == 1 || NSB == 2, "super-blocks per stage");
    static constexpr int MT = M / 16;                                   // row tiles of 16 pairs
    static constexpr bool KQ = WT != Q8_0;
    static constexpr bool GU = AHL == 1;                                // gate/up (else down)
    static constexpr bool SPLIT = GU && NMAT == 1;                      // gate and up in alternate stages
    static constexpr int KC = GM_KC * NSB;                              // columns per stage
    static constexpr int CHUNK = KQ ? NSB * block_bytes(WT) : KC / 32 * 34;   // bytes of a row's stage chunk
    static constexpr int GR = gm_granules(WT, NSB);
    static constexpr int ROWS_ITEM = SPLIT ? GM_ROWS : NSUB * GM_ROWS;  // matrix rows per item
    static_assert(!SPLIT || NSUB == 2, "split gate/up stages");
    static_assert(KQ || GR * 16 == CHUNK, "Q8_0 chunks are whole granules");
    static constexpr int RSLOT = 16 * GR;                               // LDS bytes of a row's chunk
    static constexpr int GPR = KC / 8 + 1;                              // activation granules per row (+ pad)
    static constexpr int ALD = 16 * GPR;
    static constexpr int NAU = (M * GPR + 63) / 64;                     // DMA units per activation array
    static constexpr int APART = NAU * 1024;
    // weight ring stages: one more where 16-pair passes leave the LDS for it
    static constexpr int S0 = SPLIT ? 3 : 2;
    static constexpr int S = M == 16 && gm_lds(NMAT, AHL, NSUB, WT, M, S0 + 1, NSB) <= 163840 ? S0 + 1 : S0;
    static constexpr int W_BYTES = NMAT * GM_ROWS * RSLOT;
    static constexpr int A_BYTES = AHL * APART;
    static constexpr int A_SLOT = A_BYTES + 256;                        // + 64 scale dwords
    // activation slots: a slot is refilled S - 1 stages after its last use
    static constexpr int NAS = (S - 1 + NSUB - 1) / NSUB + 1;
    static constexpr int ABASE = S * W_BYTES;
    static constexpr int DESC = ABASE + NAS * A_SLOT;
    static constexpr int RED = DESC + GM_DESC * GM_REC * 4;             // [M pairs][8 waves] maxima
    static constexpr int STG = RED + (GU ? M * GM_CW * 4 : 0);
    // staging: gate/up M pairs x 128 rows of fp16 hi and lo + M scales;
    // down 16 pairs x 128 rows of fp32 (the halves of a pass pass through in turn)
    static constexpr int LDS = STG + (GU ? M * GM_ROWS * 4 + M * 4 : 16 * GM_ROWS * 4);
    static constexpr int NW = NMAT * GM_ROWS * GR / 64;                 // weight DMA instructions per stage
    static constexpr int NWT = (NW + GM_CW - 1) / GM_CW;
    static constexpr int NA = AHL * NAU;                                // activation DMA instructions per column step
    static constexpr int NAT = (NA + GM_CW - 1) / GM_CW;
    static_assert(NAS * NSUB >= NSUB + S - 1, "activation slot reuse");
    static_assert(GM_ROWS * GR % 64 == 0, "weight DMA units");
    static_assert(LDS <= 163840 && LDS == gm_lds(NMAT, AHL, NSUB, WT, M, S, NSB), "LDS");
    static_assert(GU || GM_M * (KC / 128) <= 64, "activation scale dwords");
};

static_assert(4 + GM_M + GM_M / 4 <= GM_REC, "pass record");

struct PfGemm {
    const uint8_t* w0;                 // routed matrices (gate, up) or (down, -): expert e at + e * st
    const uint8_t* w1;
    int64_t st0, st1;
    const uint8_t* s0;                 // shared-expert matrices
    const uint8_t* s1;
    int64_t rb_r, rb_s;                // bytes per matrix row: routed, shared
    int32_t mb_r, mb_s;                // bytes per matrix: routed, shared
    const uint16_t* a_hi;              // activations, fp16 bits [rows][a_ld]
    const uint16_t* a_lo;
    int64_t a_ld;
    const float* a_sc;                 // activation scales [rows][sc_ld], one per 128 columns
    int64_t sc_ld;
    int32_t a_bytes, sc_bytes;         // sizes of the activation and scale arrays
    int32_t T, K, E, by_token;         // activation row: token of the pair (1) or the pair (0)
    int32_t nrb_r, nrb_s;              // row groups per pass: routed, shared
    int32_t ncol_r, ncol_s;            // matrix columns: routed, shared
    int32_t nkc_r, nkc_s;              // column steps per item (launch_pf_gemm: columns / the instance's KC)
    int32_t sel;                       // passes of this launch: 0 all, 1 routed only, 2 shared only
    const int32_t* recs;
    const int32_t* npass;              // {routed passes, shared passes}
    uint16_t* o_hi;                    // gate/up: SwiGLU output hi / lo [pair][o_ld], scales [pair][osc_ld]
    uint16_t* o_lo;
    float* o_sc;
    int64_t o_ld, osc_ld;
    float* y;                          // down: [pair][y_ld]
    int64_t y_ld;
};

typedef __attribute__((address_space(3))) void lds_void;

// Workgroups are dispatched to the 8 XCDs in turn (workgroup b on XCD b % 8)
// and each XCD has its own L2.  Item j of round i goes to workgroup b with
// j - i * grid = slot(b): the R consecutive items of one pass (its row groups,
// which read the same activations) land on workgroups of one XCD, so the
// activations come from HBM once per pass rather than once per XCD.  A
// bijection of [0, grid) when grid is a multiple of 8 R; the identity
// otherwise.
constexpr int PF_XCDS = 8;
WM_HD int pf_item_slot(int b, int grid, int R) {
    if (R <= 0 || grid % (PF_XCDS * R)) return b;
    const int x = b % PF_XCDS, q = b / PF_XCDS;
    return ((q / R) * PF_XCDS + x) * R + q % R;
}

// Raw buffer resource over [p, p + bytes) (gfx9 word 3: 32-bit data format).
WM_DEV __amdgpu_buffer_rsrc_t gm_rsrc(const void* p, int bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, bytes, 0x00020000);
}

// All waves of the workgroup meet; this wave's LDS accesses are complete.
// (No fence: a fence would also wait for the ring's loads in flight.)
WM_DEV void gm_bar() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xC07F);          // lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// s_waitcnt vmcnt(n) for a wave-uniform n (values past 15 wait for all).
WM_DEV void gm_wait_vm(int n) {
    switch (n) {
#define WM_GM_CASE(k) \
    case k: WM_WAIT_VMCNT(k); break;
        WM_GM_CASE(1) WM_GM_CASE(2) WM_GM_CASE(3) WM_GM_CASE(4) WM_GM_CASE(5) WM_GM_CASE(6) WM_GM_CASE(7)
        WM_GM_CASE(8) WM_GM_CASE(9) WM_GM_CASE(10) WM_GM_CASE(11) WM_GM_CASE(12) WM_GM_CASE(13) WM_GM_CASE(14)
        WM_GM_CASE(15)
#undef WM_GM_CASE
        default: WM_WAIT_VMCNT(0); break;
    }
}

// The 8 int8 weights k = 8g .. 8g+7 of block B of a row chunk as fp16
// (exact).  rowp: the chunk's first byte in LDS (16-byte aligned).
template <int B> WM_DEV f16x8 q8_f16x8(const uint8_t* rowp, int g) {
    constexpr int off = 34 * B + 2;
    const uint32_t* p = (const uint32_t*)(rowp + (off & ~3) + 8 * g);
    const uint32_t K = 0x64646464u, X = 0x80808080u;
    uint32_t h0, h1, h2, h3;
    if constexpr ((off & 3) == 0) {
        const uint32_t d0 = p[0] ^ X, d1 = p[1] ^ X;
        h0 = __builtin_amdgcn_perm(K, d0, 0x04010400u);
        h1 = __builtin_amdgcn_perm(K, d0, 0x04030402u);
        h2 = __builtin_amdgcn_perm(K, d1, 0x04010400u);
        h3 = __builtin_amdgcn_perm(K, d1, 0x04030402u);
    } else {
        const uint32_t d0 = p[0] ^ X, d1 = p[1] ^ X, d2 = p[2] ^ X;
        h0 = __builtin_amdgcn_perm(K, d0, 0x04030402u);
        h1 = __builtin_amdgcn_perm(K, d1, 0x04010400u);
        h2 = __builtin_amdgcn_perm(K, d1, 0x04030402u);
        h3 = __builtin_amdgcn_perm(K, d2, 0x04010400u);
    }
    const f16x2 bias = {(_Float16)1152.0f, (_Float16)1152.0f};
    const f16x2 v0 = __builtin_bit_cast(f16x2, h0) - bias, v1 = __builtin_bit_cast(f16x2, h1) - bias;
    const f16x2 v2 = __builtin_bit_cast(f16x2, h2) - bias, v3 = __builtin_bit_cast(f16x2, h3) - bias;
    return (f16x8){v0[0], v0[1], v1[0], v1[1], v2[0], v2[1], v3[0], v3[1]};
}

// ------------------------------------------------------------------ K-quant row chunks in LDS

// 8 unsigned integers below 256, one per byte of (d0, d1), minus BIAS as fp16 (exact).
template <int BIAS> WM_DEV f16x8 u8_f16x8(uint32_t d0, uint32_t d1) {
    const uint32_t K = 0x64646464u;
    const uint32_t h0 = __builtin_amdgcn_perm(K, d0, 0x04010400u), h1 = __builtin_amdgcn_perm(K, d0, 0x04030402u);
    const uint32_t h2 = __builtin_amdgcn_perm(K, d1, 0x04010400u), h3 = __builtin_amdgcn_perm(K, d1, 0x04030402u);
    const f16x2 bias = {(_Float16)(1024.0f + BIAS), (_Float16)(1024.0f + BIAS)};
    const f16x2 v0 = __builtin_bit_cast(f16x2, h0) - bias, v1 = __builtin_bit_cast(f16x2, h1) - bias;
    const f16x2 v2 = __builtin_bit_cast(f16x2, h2) - bias, v3 = __builtin_bit_cast(f16x2, h3) - bias;
    return (f16x8){v0[0], v0[1], v1[0], v1[1], v2[0], v2[1], v3[0], v3[1]};
}

// Two dwords at byte offset o of an LDS row slot whose address is 16-byte
// aligned; AL: the alignment o is known to have (8, 4 or 2).
template <int AL> WM_DEV void ld_u32x2(const uint8_t* slot, int o, uint32_t& w0, uint32_t& w1) {
    if constexpr (AL >= 8) {
        const uint2 v = *(const uint2*)(slot + o);
        w0 = v.x;
        w1 = v.y;
    } else if constexpr (AL == 4) {
        const uint32_t* p = (const uint32_t*)(slot + o);
        w0 = p[0];
        w1 = p[1];
    } else {
        const uint32_t* p = (const uint32_t*)(slot + (o & ~3));
        const uint32_t s = (uint32_t)o & 3u, a0 = p[0], a1 = p[1], a2 = p[2];
        w0 = alignbyte(a1, a0, s);
        w1 = alignbyte(a2, a1, s);
    }
}
template <int AL> WM_DEV uint32_t ld_u32(const uint8_t* slot, int o) {
    if constexpr (AL >= 4) return *(const uint32_t*)(slot + o);
    const uint32_t* p = (const uint32_t*)(slot + (o & ~3));
    return alignbyte(p[1], p[0], (uint32_t)o & 3u);
}

// {s, s} as fp16 for the unsigned byte of w that perm selector sel picks
// (sel: the byte index in bytes 0 and 2, 4 in bytes 1 and 3), minus BIAS.
template <int BIAS> WM_DEV f16x2 byte_f16x2(uint32_t w, uint32_t sel) {
    const f16x2 bias = {(_Float16)(1024.0f + BIAS), (_Float16)(1024.0f + BIAS)};
    return __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(0x64646464u, w, sel)) - bias;
}
WM_HD constexpr uint32_t byte_sel(uint32_t p) { return p | (p << 16) | 0x04000400u; }

// fma(x, s, c) on four fp16 pairs (one rounding each)
WM_DEV f16x8 f16x8_fma(f16x8 x, f16x2 s, f16x2 c) {
    const f16x8 s8 = {s[0], s[1], s[0], s[1], s[0], s[1], s[0], s[1]};
    const f16x8 c8 = {c[0], c[1], c[0], c[1], c[0], c[1], c[0], c[1]};
    return __builtin_elementwise_fma(x, s8, c8);
}
WM_DEV f16x8 f16x8_rep(f16x2 v) { return (f16x8){v[0], v[1], v[0], v[1], v[0], v[1], v[0], v[1]}; }

// 8 unsigned integers below 256, one per byte of (d0, d1), as 1024 + value in fp16.
WM_DEV f16x8 u8_h1024(uint32_t d0, uint32_t d1) {
    const uint32_t K = 0x64646464u;
    return __builtin_bit_cast(f16x8, (u32x4){__builtin_amdgcn_perm(K, d0, 0x04010400u), __builtin_amdgcn_perm(K, d0, 0x04030402u),
                                             __builtin_amdgcn_perm(K, d1, 0x04010400u), __builtin_amdgcn_perm(K, d1, 0x04030402u)});
}

// A K-quant super-block of one weight row in LDS (slot + o: its first byte);
// unit b = columns 32b .. 32b + 31, of which this lane holds 32b + 8g .. + 7
// (one sub-block: the 32-weight sub-block b, or the 16-weight sub-block
// 2b + g / 2).  head() reads the block's scales once per stage.
//
// FOLD formats (q times its sub-block scale is an integer fp16 holds
// exactly: Q4_K <= 15*63, Q5_K <= 31*63, Q3_K <= 4*32, Q2_K <= 3*15):
// unit(b) gives Bq = q * sc and Bm = the sub-block min m, and the weight is
// d * Bq - dmin * Bm with the block's d, dmin.
// Q6_K (|q * sc| up to 32*128) unit(b) gives the values q and the
// multipliers am[h] = d * sc of the unit's two 16-weight sub-blocks (h = 0:
// columns 32b + [0,16)), applied after the MFMA.
template <int WT> struct KqRow;

template <> struct KqRow<Q4_K> {                 // q4k_dequant.h:28-33, 43-60, 112-168
    static constexpr int AL = 16;
    static constexpr bool FOLD = true, MINS = true;
    float d, dmin;
    uint32_t sc[2], mn[2];                       // 6-bit scales and mins of sub-blocks 0-3, 4-7 (a byte each)
    WM_DEV void head(const uint8_t* slot, int o) {
        const uint4 h = *(const uint4*)(slot + o);
        d = h2f(h.x);
        dmin = h2f(h.x >> 16);
        sc[0] = h.y & 0x3F3F3F3Fu;
        mn[0] = h.z & 0x3F3F3F3Fu;
        sc[1] = (h.w & 0x0F0F0F0Fu) | ((h.y >> 2) & 0x30303030u);
        mn[1] = ((h.w >> 4) & 0x0F0F0F0Fu) | ((h.z >> 2) & 0x30303030u);
    }
    // sub-block b: qs bytes 32 (b / 2) + l, low nibble for even b, high for odd
    WM_DEV void unit(const uint8_t* slot, int o, int b, int g, f16x8& Bq, f16x8& Bm) const {
        uint32_t w0, w1;
        ld_u32x2<AL>(slot, o + 16 + 32 * (b >> 1) + 8 * g, w0, w1);
        const int sh = 4 * (b & 1);
        const uint32_t scw = b >= 4 ? sc[1] : sc[0], mnw = b >= 4 ? mn[1] : mn[0];
        const f16x2 s2 = byte_f16x2<0>(scw, byte_sel(b & 3));
        const f16x2 c2 = s2 * (f16x2){(_Float16)-1024.0f, (_Float16)-1024.0f};
        // (1024 + q) * sc - 1024 * sc, one rounding of the exact integer q * sc
        Bq = f16x8_fma(u8_h1024((w0 >> sh) & 0x0F0F0F0Fu, (w1 >> sh) & 0x0F0F0F0Fu), s2, c2);
        Bm = f16x8_rep(byte_f16x2<0>(mnw, byte_sel(b & 3)));
    }
};

template <> struct KqRow<Q5_K> {                 // q5k_dequant.h:19-25, 98-131
    static constexpr int AL = 16;
    static constexpr bool FOLD = true, MINS = true;
    float d, dmin;
    uint32_t sc[2], mn[2];
    WM_DEV void head(const uint8_t* slot, int o) {
        const uint4 h = *(const uint4*)(slot + o);
        d = h2f(h.x);
        dmin = h2f(h.x >> 16);
        sc[0] = h.y & 0x3F3F3F3Fu;
        mn[0] = h.z & 0x3F3F3F3Fu;
        sc[1] = (h.w & 0x0F0F0F0Fu) | ((h.y >> 2) & 0x30303030u);
        mn[1] = ((h.w >> 4) & 0x0F0F0F0Fu) | ((h.z >> 2) & 0x30303030u);
    }
    // sub-block b: nibble as Q4_K (qs at 48), fifth bit = bit b of qh[l] (qh at 16)
    WM_DEV void unit(const uint8_t* slot, int o, int b, int g, f16x8& Bq, f16x8& Bm) const {
        uint32_t w0, w1, e0, e1;
        ld_u32x2<AL>(slot, o + 48 + 32 * (b >> 1) + 8 * g, w0, w1);
        ld_u32x2<AL>(slot, o + 16 + 8 * g, e0, e1);
        const int sh = 4 * (b & 1);
        const f16x2 s2 = byte_f16x2<0>(sc[b >> 2], byte_sel(b & 3));
        const f16x8 q = u8_f16x8<0>(((w0 >> sh) & 0x0F0F0F0Fu) | (((e0 >> b) & 0x01010101u) << 4),
                                    ((w1 >> sh) & 0x0F0F0F0Fu) | (((e1 >> b) & 0x01010101u) << 4));
        Bq = q * f16x8_rep(s2);                  // exact: q * sc <= 1953
        Bm = f16x8_rep(byte_f16x2<0>(mn[b >> 2], byte_sel(b & 3)));
    }
};

// Column 128 h + 32 j + l of the 16-weight sub-block formats: unit b = 4 h + j,
// sub-block 8 h + 2 j + l / 16 (l / 16 = g / 2 for this lane).
template <> struct KqRow<Q6_K> {                 // q6k_dequant.h:20-25, 112-141
    static constexpr int AL = 2;
    static constexpr bool FOLD = false, MINS = false;
    float d;
    uint32_t sc[4];                              // int8 scales[16]
    WM_DEV void head(const uint8_t* slot, int o) {
        ld_u32x2<AL>(slot, o + 192, sc[0], sc[1]);
        ld_u32x2<AL>(slot, o + 200, sc[2], sc[3]);
        d = h2f(*(const uint16_t*)(slot + o + 208));
    }
    // The bytes of half h this lane's units read: ql[64 h + 8g ..] (units
    // j = 0, 2: low, high nibble), ql[64 h + 32 + 8g ..] (j = 1, 3), qh[32 h + 8g ..]
    // (bits 2j, 2j+1 for unit j).
    uint32_t ql[2][2], qh[2];
    WM_DEV void half(const uint8_t* slot, int o, int h, int g) {
        ld_u32x2<AL>(slot, o + 64 * h + 8 * g, ql[0][0], ql[0][1]);
        ld_u32x2<AL>(slot, o + 64 * h + 32 + 8 * g, ql[1][0], ql[1][1]);
        ld_u32x2<AL>(slot, o + 128 + 32 * h + 8 * g, qh[0], qh[1]);
    }
    // unit 4 h + j of the loaded half: values q - 32, multipliers of
    // sub-blocks 8 h + 2 j and 8 h + 2 j + 1
    WM_DEV f16x8 unit(int h, int j, float* am) const {
        const int sh = 4 * (j >> 1);
        const int k = 8 * h + 2 * j;
        am[0] = d * (float)(int8_t)byte_of(sc[k >> 2], k & 3);
        am[1] = d * (float)(int8_t)byte_of(sc[(k + 1) >> 2], (k + 1) & 3);
        const uint32_t* w = ql[j & 1];
        return u8_f16x8<32>(((w[0] >> sh) & 0x0F0F0F0Fu) | (((qh[0] >> (2 * j)) & 0x03030303u) << 4),
                            ((w[1] >> sh) & 0x0F0F0F0Fu) | (((qh[1] >> (2 * j)) & 0x03030303u) << 4));
    }
};

template <> struct KqRow<Q3_K> {                 // hmask[32] qs[64] scales[12] d
    static constexpr int AL = 2;
    static constexpr bool FOLD = true, MINS = false;
    float d, dmin;
    uint32_t sc[4];                              // sub-blocks 4i .. 4i+3: the 6-bit scale + 32 (a byte each)
    WM_DEV void head(const uint8_t* slot, int o) {
        uint32_t s0, s1, s2;
        ld_u32x2<AL>(slot, o + 96, s0, s1);
        s2 = ld_u32<AL>(slot, o + 104);
        d = h2f(*(const uint16_t*)(slot + o + 108));
        dmin = 0.0f;
        // low 4 bits: bytes 0-7 of the scales (sub-blocks 0-7), their high
        // nibbles (8-15); high 2 bits: bits 2(k / 4) of byte 8 + k % 4
        sc[0] = (s0 & 0x0F0F0F0Fu) | ((s2 << 4) & 0x30303030u);
        sc[1] = (s1 & 0x0F0F0F0Fu) | ((s2 << 2) & 0x30303030u);
        sc[2] = ((s0 >> 4) & 0x0F0F0F0Fu) | (s2 & 0x30303030u);
        sc[3] = ((s1 >> 4) & 0x0F0F0F0Fu) | ((s2 >> 2) & 0x30303030u);
    }
    // low bits (qs[32 h + l] >> 2j) & 3, high bit (hmask[l] >> (4h + j)) & 1
    // (clear: minus 4), i.e. value u - 4
    WM_DEV void unit(const uint8_t* slot, int o, int b, int g, f16x8& Bq, f16x8& Bm) const {
        const int h = b >> 2, j = b & 3, hb = 4 * h + j;
        uint32_t w0, w1, e0, e1;
        ld_u32x2<AL>(slot, o + 32 + 32 * h + 8 * g, w0, w1);
        ld_u32x2<AL>(slot, o + 8 * g, e0, e1);
        const int k = 8 * h + 2 * j;             // + g / 2
        const f16x2 s2 = byte_f16x2<32>(sc[k >> 2], byte_sel((uint32_t)((k & 3) + (g >> 1))));
        const f16x8 q = u8_f16x8<4>(((w0 >> (2 * j)) & 0x03030303u) | (((e0 >> hb) & 0x01010101u) << 2),
                                    ((w1 >> (2 * j)) & 0x03030303u) | (((e1 >> hb) & 0x01010101u) << 2));
        Bq = q * f16x8_rep(s2);                  // exact: |q * sc| <= 128
        Bm = Bq;
    }
};

template <> struct KqRow<Q2_K> {                 // scales[16] qs[64] d dmin
    static constexpr int AL = 4;
    static constexpr bool FOLD = true, MINS = true;
    float d, dmin;
    uint32_t sb[4];                              // sub-blocks 4i .. 4i+3: scale (low nibble), min (high)
    WM_DEV void head(const uint8_t* slot, int o) {
        ld_u32x2<AL>(slot, o, sb[0], sb[1]);
        ld_u32x2<AL>(slot, o + 8, sb[2], sb[3]);
        const uint32_t dd = ld_u32<AL>(slot, o + 80);
        d = h2f(dd);
        dmin = h2f(dd >> 16);
    }
    // (qs[32 h + l] >> 2j) & 3
    WM_DEV void unit(const uint8_t* slot, int o, int b, int g, f16x8& Bq, f16x8& Bm) const {
        const int h = b >> 2, j = b & 3;
        uint32_t w0, w1;
        ld_u32x2<AL>(slot, o + 16 + 32 * h + 8 * g, w0, w1);
        const int k = 8 * h + 2 * j;             // + g / 2
        const uint32_t sel = byte_sel((uint32_t)((k & 3) + (g >> 1)));
        const f16x2 s2 = byte_f16x2<0>(sb[k >> 2] & 0x0F0F0F0Fu, sel);
        const f16x2 c2 = s2 * (f16x2){(_Float16)-1024.0f, (_Float16)-1024.0f};
        Bq = f16x8_fma(u8_h1024((w0 >> (2 * j)) & 0x03030303u, (w1 >> (2 * j)) & 0x03030303u), s2, c2);
        Bm = f16x8_rep(byte_f16x2<0>((sb[k >> 2] >> 4) & 0x0F0F0F0Fu, sel));
    }
};

// Q8_0 needs no K-quant row decoder; a placeholder keeps the kernel generic.
template <> struct KqRow<Q8_0> {
    static constexpr int AL = 16;
    static constexpr bool FOLD = false, MINS = false;
    WM_DEV void head(const uint8_t*, int) {}
    WM_DEV void half(const uint8_t*, int, int, int) {}
    WM_DEV f16x8 unit(int, int, float*) const { return (f16x8){}; }
};

// ------------------------------------------------------------------ the kernel

// AHL = 1: gate and up of a pass (activations: the tokens' x), SwiGLU
// epilogue; both matrices in each stage (NMAT = 2, NSUB = 1), or gate and up
// in alternate stages over one activation column step (NMAT = 1, NSUB = 2,
// Q8_0: 272-byte runs per row).  AHL = 2: down (activations: the pairs'
// SwiGLU outputs as hi + lo), fp32 epilogue; an item covers NSUB blocks of
// 128 rows: each column step loads the activations once and the NSUB weight
// blocks in turn (one ring stage each).  WT: the weight format of every matrix the
// launch reads (a.sel picks the routed or the shared passes when the two
// differ).
template <int NMAT, int AHL, int NSUB, int WT, int M, int NSB>
__global__ __launch_bounds__(GM_THREADS) void k_pf_gemm(PfGemm a) {
#if defined(__HIP_DEVICE_COMPILE__)      // the host pass only needs the launch stub (buffer resources are device types)
    typedef GmGeo<NMAT, AHL, NSUB, WT, M, NSB> G;
    typedef KqRow<WT> F;
    constexpr bool KQ = G::KQ;
    constexpr int S = G::S;
    extern __shared__ __attribute__((aligned(16))) uint8_t gsm[];
    // the wave index is uniform: readfirstlane lets the compiler keep what depends on it in SGPRs
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), g = lane >> 4, c = lane & 15;
    const bool cw = wave < GM_CW;
    const int n_rp = a.npass[0], n_sp = a.npass[1];
    const int n_r = a.sel == 2 ? 0 : n_rp * a.nrb_r, n_items = n_r + (a.sel == 1 ? 0 : n_sp * a.nrb_s);
    const int k0 = pf_item_slot((int)blockIdx.x, (int)gridDim.x, a.sel == 2 ? a.nrb_s : a.nrb_r);
    if (k0 >= n_items) return;

    // item i of this workgroup: pass, row group, column steps
    auto item = [&](int i, int& pass, int& rg, int& nkc) __attribute__((always_inline)) -> bool {
        const int j = k0 + i * (int)gridDim.x;
        if (j >= n_items) return false;
        if (j < n_r) {
            pass = j / a.nrb_r;
            rg = j - pass * a.nrb_r;
            nkc = a.nkc_r;
        } else {
            const int q = (j - n_r) / a.nrb_s;
            rg = (j - n_r) - q * a.nrb_s;
            pass = n_rp + q;
            nkc = a.nkc_s;
        }
        return true;
    };
    const int32_t* desc = (const int32_t*)(gsm + G::DESC);
    auto desc_dma = [&](int i, int pass) __attribute__((always_inline)) {
        __builtin_amdgcn_global_load_lds((const void*)(a.recs + (int64_t)pass * GM_REC + lane),
                                         (lds_void*)(gsm + G::DESC + (i % GM_DESC) * GM_REC * 4), 4, 0, 0);
    };

    // Down activations carry a scale per (row, 128 columns); gate/up
    // activations (x) one per token, applied in the epilogue.
    constexpr bool SCALED = !G::GU;
    // DMA instructions of this wave per weight stage
    int n_wt = 0;
#pragma unroll
    for (int t = 0; t < G::NWT; t++)
        if (wave + GM_CW * t < G::NW) n_wt++;
    const int m_s = lane & 31;        // this lane's pass row of the scale load

    // issue pointer: item ii, stage ist = NSUB * column step + row block; the
    // item's sources as uniform bases plus this lane's 32-bit byte offsets.
    // Weight instruction t of this wave covers granules p = 64 (wave + 8 t) +
    // lane of a stage: matrix p / (128 GR) (uniform per instruction), row
    // (p % 128 GR) / GR, granule p % GR.
    int ii = 0, ist = 0, ip = 0, irg = 0, inkc = 0;
    bool iok = item(0, ip, irg, inkc);
    // Sources are bounds-checked buffer resources (a read past the
    // resource's size returns zeros instead of touching memory).
    const __amdgpu_buffer_rsrc_t rA0 = gm_rsrc(a.a_hi, a.a_bytes), rA1 = gm_rsrc(a.a_lo, a.a_bytes);
    const __amdgpu_buffer_rsrc_t rS = gm_rsrc(a.a_sc, a.sc_bytes);
    __amdgpu_buffer_rsrc_t rW0 = rA0, rW1 = rA0;
    uint32_t iwo[G::NWT], iao[G::NAT];
    uint32_t iso = 0, irowb = 0;
    // The issue item's pass: DMA units of each activation array holding its
    // rows (the first ceil(pairs * GPR / 64); rows past the pair count feed
    // only output rows that are never stored) and this wave's activation DMA
    // instructions per column step (with the scales)
    int iau = G::NAU, n_a = 0;
    auto setup_issue = [&]() __attribute__((always_inline)) {
        const int32_t* rec = desc + (ii % GM_DESC) * GM_REC;
        iau = min((__builtin_amdgcn_readfirstlane(rec[1]) * G::GPR + 63) >> 6, G::NAU);
        n_a = SCALED && wave == GM_CW - 1 ? 1 : 0;
#pragma unroll
        for (int t = 0; t < G::NAT; t++) {
            const int u = wave + GM_CW * t;
            if (u < G::NA && u % G::NAU < iau) n_a++;
        }
        const int ge = __builtin_amdgcn_readfirstlane(rec[0]);
        const bool shared = ip >= n_rp;
        const int mb = shared ? a.mb_s : a.mb_r;
        rW0 = gm_rsrc(shared ? a.s0 : a.w0 + (int64_t)ge * a.st0, mb);
        rW1 = G::GU ? gm_rsrc(shared ? a.s1 : a.w1 + (int64_t)ge * a.st1, mb) : rW0;
        irowb = (uint32_t)(shared ? a.rb_s : a.rb_r);
#pragma unroll
        for (int t = 0; t < G::NWT; t++) {
            const int p = 64 * (wave + GM_CW * t) + lane, rem = p % (GM_ROWS * G::GR), r = rem / G::GR;
            iwo[t] = (((uint32_t)(irg * G::ROWS_ITEM + r) * irowb) & ~15u) + 16u * (uint32_t)(rem - G::GR * r);
        }
        // activation instruction u = wave + 8 t: array u / NAU, LDS granules
        // 64 (u % NAU) + lane = GPR m + jj of the array (jj = GPR - 1: pad;
        // m >= M: slack), loaded from granule min(jj, GPR - 2) of pass row
        // min(m, M - 1)
#pragma unroll
        for (int t = 0; t < G::NAT; t++) {
            const int p = 64 * ((wave + GM_CW * t) % G::NAU) + lane, m = min(p / G::GPR, M - 1),
                      jj = min(p % G::GPR, G::GPR - 2);
            const int pa = rec[4 + m], ra = a.by_token ? pair_token(pa, a.T, a.K) : pa;
            iao[t] = (uint32_t)ra * (uint32_t)a.a_ld * 2u + 16u * (uint32_t)jj;
        }
        // scale dword of lane l: pass row l % 32, the stage's 128-column half l / 32
        if constexpr (SCALED)
            iso = ((uint32_t)rec[4 + m_s] * (uint32_t)a.sc_ld + (G::KC > 128 ? (uint32_t)(lane >> 5) : 0u)) * 4u;
    };
    int issued = 0, a_issued = 0;
    // Per-wave DMA instruction counts of the issued stages not yet consumed,
    // 4 bits each, oldest in the low bits (at most S of them), and their sum:
    // "stage landed" is vmcnt(sum minus the oldest count).
    uint32_t qpack = 0;
    int qn = 0, qsum = 0;
    // Loads of stage (ii, ist): the weight block into ring slot issued % S;
    // at a column step's first block also the activations and scales into
    // activation slot a_issued % NAS; at an item's first stage wave 6 also
    // fetches the record of the item two ahead (after the stage's loads, so
    // "stage landed" implies "record landed").
    auto issue_next = [&](auto sw_tag) __attribute__((always_inline)) {
        constexpr bool SW = decltype(sw_tag)::value;
        const int kc = ist / NSUB, sub = ist - kc * NSUB;
        if constexpr (!SW) {
            const int n = n_wt + (sub == 0 ? n_a : 0);
            qpack |= (uint32_t)n << (4 * qn);
            ++qn;
            qsum += n;
            lds8_t* dst = (lds8_t*)(gsm + (issued % S) * G::W_BYTES);
            const uint32_t soff = (((uint32_t)kc * (uint32_t)G::CHUNK) & ~15u) +
                                  (G::SPLIT ? 0u : (uint32_t)(sub * GM_ROWS) * irowb);
#pragma unroll
            for (int t = 0; t < G::NWT; t++) {
                const int q = wave + GM_CW * t;
                if (q < G::NW)
                    __builtin_amdgcn_raw_ptr_buffer_load_lds((G::SPLIT ? sub != 0 : q >= GM_ROWS * G::GR / 64) ? rW1 : rW0,
                                                             (lds_void*)(dst + 1024 * q), 16, iwo[t], soff, 0, 0);
            }
            if (sub == 0) {
                lds8_t* adst = (lds8_t*)(gsm + G::ABASE + (a_issued % G::NAS) * G::A_SLOT);
#pragma unroll
                for (int t = 0; t < G::NAT; t++) {
                    const int u = wave + GM_CW * t;
                    if (u < G::NA && u % G::NAU < iau)
                        __builtin_amdgcn_raw_ptr_buffer_load_lds(u >= G::NAU ? rA1 : rA0,
                                                                 (lds_void*)(adst + G::APART * (u / G::NAU) + 1024 * (u % G::NAU)),
                                                                 16, iao[t], (uint32_t)(2 * G::KC) * (uint32_t)kc, 0, 0);
                }
                if (SCALED && wave == GM_CW - 1)
                    __builtin_amdgcn_raw_ptr_buffer_load_lds(rS, (lds_void*)(adst + G::A_BYTES), 4, iso,
                                                             (uint32_t)(4 * (G::KC / 128)) * (uint32_t)kc, 0, 0);
            }
            if (ist == 0 && wave == 6) {
                int p2, r2, n2;
                if (item(ii + 2, p2, r2, n2)) desc_dma(ii + 2, p2);
            }
        }
        ++issued;
        if (sub == 0) ++a_issued;
        if (++ist == inkc * NSUB) {
            ist = 0;
            ++ii;
            iok = item(ii, ip, irg, inkc);
            if constexpr (!SW)
                if (iok) setup_issue();
        }
    };

    f32x4 acc[NSUB][1][NMAT][2];
    const f32x4 zero = {0.0f, 0.0f, 0.0f, 0.0f};
    // Q6_K's 16-weight sub-blocks: the lanes of one half of an MFMA
    // operand's k range (lanes 0-31: k 0-15, lanes 32-63: k 16-31)
    const bool lo32 = lane < 32;
    auto half_of = [&](f16x8 v, int hv) __attribute__((always_inline)) -> f16x8 {
        const u32x4 u = __builtin_bit_cast(u32x4, v);
        const bool keep = hv == 0 ? lo32 : !lo32;
        return __builtin_bit_cast(f16x8, (u32x4){keep ? u[0] : 0u, keep ? u[1] : 0u, keep ? u[2] : 0u, keep ? u[3] : 0u});
    };
#pragma unroll
    for (int u = 0; u < NSUB; u++)
#pragma unroll
        for (int mat = 0; mat < NMAT; mat++) acc[u][0][mat][0] = acc[u][0][mat][1] = zero;

    // The sums of one stage (column step kc of a weight block) from weight
    // slot ws and activation slot as, not yet scaled; TWO: pass rows 16-31
    // are in use (one straight-line body per case, for the scheduler; the
    // row tile 16-31 sums stay zero otherwise).  NH: sums per 128 columns
    // of the stage that take their own activation scale.
    // K-quant gate/up stages add into the item's accumulators directly.
    constexpr int NH = SCALED ? G::KC / 128 : 1;
    constexpr bool DIRECT = KQ && !SCALED;
    struct Sums {
        f32x4 v[NH][NMAT][2];
    };
    auto compute = [&](int ws, int as, int kc, int lsh, auto two_tag, f32x4(&tv)[NH][NMAT][2])
                       __attribute__((always_inline)) {
        constexpr bool TWO = decltype(two_tag)::value;
        const uint8_t* wb = gsm + ws * G::W_BYTES;
        const uint8_t* ab = gsm + G::ABASE + as * G::A_SLOT;
        if constexpr (!DIRECT) {
#pragma unroll
            for (int h = 0; h < NH; h++)
#pragma unroll
                for (int mat = 0; mat < NMAT; mat++) tv[h][mat][0] = tv[h][mat][1] = zero;
        }
        if constexpr (!KQ) {
#pragma unroll
            for (int b = 0; b < G::KC / 32; b++) {
                const int hs = SCALED ? b / 4 : 0;          // the stage's 128-column half
                f16x8 A[AHL][2];
#pragma unroll
                for (int h = 0; h < AHL; h++)
#pragma unroll
                    for (int mt = 0; mt < 2; mt++)
                        A[h][mt] = *(const f16x8*)(ab + G::APART * h + (16 * mt + c) * G::ALD + 16 * (4 * b + g));
#pragma unroll
                for (int mat = 0; mat < NMAT; mat++) {
                    const uint8_t* rowp = wb + (mat * GM_ROWS + 16 * wave + c) * G::RSLOT;
                    const float d = (float)*(const _Float16*)(rowp + 34 * b);
                    f16x8 B;
                    if (b == 0) B = q8_f16x8<0>(rowp, g);
                    else if (b == 1) B = q8_f16x8<1>(rowp, g);
                    else if (b == 2) B = q8_f16x8<2>(rowp, g);
                    else if (b == 3) B = q8_f16x8<3>(rowp, g);
                    else if (b == 4) B = q8_f16x8<4>(rowp, g);
                    else if (b == 5) B = q8_f16x8<5>(rowp, g);
                    else if (b == 6) B = q8_f16x8<6>(rowp, g);
                    else B = q8_f16x8<7>(rowp, g);
#pragma unroll
                    for (int mt = 0; mt < 2; mt++) {
                        if (mt == 1 && !TWO) continue;
                        f32x4 P = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[0][mt], B, zero, 0, 0, 0);
                        if constexpr (AHL == 2) P = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[AHL - 1][mt], B, P, 0, 0, 0);
#pragma unroll
                        for (int i = 0; i < 4; i++) tv[hs][mat][mt][i] = fmaf(d, P[i], tv[hs][mat][mt][i]);
                    }
                }
            }
        } else {
#pragma unroll
            for (int sb = 0; sb < NSB; sb++) {
                // super-block sb of each row: its first byte is lsh (the row start's
                // offset past a 16-byte boundary) plus the chunk offset's into the
                // slot, plus sb super-blocks; its activations 512 sb bytes into
                // the rows
                const int o = lsh + ((kc * G::CHUNK) & 15) + sb * block_bytes(WT);
                const int cb = 512 * sb;
                const uint8_t* slot[NMAT];
                F row[NMAT];
    #pragma unroll
                for (int mat = 0; mat < NMAT; mat++) {
                    slot[mat] = wb + (mat * GM_ROWS + 16 * wave + c) * G::RSLOT;
                    row[mat].head(slot[mat], o);
                }
                if constexpr (F::FOLD) {
                    // the stage's sums of q * sc and of the mins, per 128-column
                    // half, in the MFMA accumulators; d and dmin once at the end
                    f32x4 sq[NH][NMAT][2], sm[NH][NMAT][2];
    #pragma unroll
                    for (int h = 0; h < NH; h++)
    #pragma unroll
                        for (int mat = 0; mat < NMAT; mat++) sq[h][mat][0] = sq[h][mat][1] = sm[h][mat][0] = sm[h][mat][1] = zero;
    #pragma unroll
                    for (int b = 0; b < 8; b++) {
                        const int hs = SCALED ? 2 * sb + b / 4 : 0;
                        f16x8 A[AHL][2];
    #pragma unroll
                        for (int h = 0; h < AHL; h++)
    #pragma unroll
                            for (int mt = 0; mt < 2; mt++)
                                A[h][mt] = *(const f16x8*)(ab + G::APART * h + (16 * mt + c) * G::ALD + cb + 16 * (4 * b + g));
    #pragma unroll
                        for (int mat = 0; mat < NMAT; mat++) {
                            f16x8 Bq, Bm;
                            row[mat].unit(slot[mat], o, b, g, Bq, Bm);
    #pragma unroll
                            for (int mt = 0; mt < 2; mt++) {
                                if (mt == 1 && !TWO) continue;
    #pragma unroll
                                for (int h = 0; h < AHL; h++)
                                    sq[hs][mat][mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[h][mt], Bq, sq[hs][mat][mt], 0, 0, 0);
                                if constexpr (F::MINS) {
    #pragma unroll
                                    for (int h = 0; h < AHL; h++)
                                        sm[hs][mat][mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[h][mt], Bm, sm[hs][mat][mt], 0, 0, 0);
                                }
                            }
                        }
                    }
    #pragma unroll
                    for (int h = 0; h < NH; h++)
    #pragma unroll
                        for (int mat = 0; mat < NMAT; mat++)
    #pragma unroll
                            for (int mt = 0; mt < 2; mt++) {
                                if (mt == 1 && !TWO) continue;
                                f32x4 r = tv[h][mat][mt];
    #pragma unroll
                                for (int i = 0; i < 4; i++) r[i] = fmaf(row[mat].d, sq[h][mat][mt][i], r[i]);
                                if constexpr (F::MINS) {
    #pragma unroll
                                    for (int i = 0; i < 4; i++) r[i] = fmaf(-row[mat].dmin, sm[h][mat][mt][i], r[i]);
                                }
                                tv[h][mat][mt] = r;
                            }
                } else {
                    // Q6_K: two MFMAs per unit, each over one 16-weight sub-block
                    // (the other half of the weight operand zero), times d * sc;
                    // the quantised bytes of a 128-column half are read once
    #pragma unroll
                    for (int b = 0; b < 8; b++) {
                        const int hs = SCALED ? 2 * sb + b / 4 : 0;
                        if ((b & 3) == 0) {
    #pragma unroll
                            for (int mat = 0; mat < NMAT; mat++) row[mat].half(slot[mat], o, b >> 2, g);
                        }
                        f16x8 A[AHL][2];
    #pragma unroll
                        for (int h = 0; h < AHL; h++)
    #pragma unroll
                            for (int mt = 0; mt < 2; mt++)
                                A[h][mt] = *(const f16x8*)(ab + G::APART * h + (16 * mt + c) * G::ALD + cb + 16 * (4 * b + g));
    #pragma unroll
                        for (int mat = 0; mat < NMAT; mat++) {
                            float am[2];
                            const f16x8 Bv = row[mat].unit(b >> 2, b & 3, am);
                            const f16x8 B[2] = {half_of(Bv, 0), half_of(Bv, 1)};
    #pragma unroll
                            for (int mt = 0; mt < 2; mt++) {
                                if (mt == 1 && !TWO) continue;
                                f32x4 r = tv[hs][mat][mt];
    #pragma unroll
                                for (int hv = 0; hv < 2; hv++) {
                                    f32x4 P = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[0][mt], B[hv], zero, 0, 0, 0);
                                    if constexpr (AHL == 2) P = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[1][mt], B[hv], P, 0, 0, 0);
    #pragma unroll
                                    for (int i = 0; i < 4; i++) r[i] = fmaf(am[hv], P[i], r[i]);
                                }
                                tv[hs][mat][mt] = r;
                            }
                        }
                        // one unit's operands live at a time (fewer registers than
                        // letting the scheduler hoist the next units' LDS reads)
                        __builtin_amdgcn_sched_barrier(0);
                    }
                }
            }
        }
    };
    // acc[SUB] += the stage's sums (SCALED: times the activation scales of
    // the pass rows 16 mt + 4 g + i, one per 128 columns)
    auto accumulate = [&](int as, const Sums& t, auto sub_tag) __attribute__((always_inline)) {
        constexpr int SUB = decltype(sub_tag)::value;
        const f32x4* scp = (const f32x4*)(gsm + G::ABASE + as * G::A_SLOT + G::A_BYTES);
#pragma unroll
        for (int mt = 0; mt < G::MT; mt++) {
#pragma unroll
            for (int mat = 0; mat < NMAT; mat++) {
                f32x4 r = acc[SUB][0][mat][mt];
#pragma unroll
                for (int h = 0; h < NH; h++) {
                    const f32x4 sc = SCALED ? scp[8 * h + 4 * mt + g] : (f32x4){1.0f, 1.0f, 1.0f, 1.0f};
#pragma unroll
                    for (int i = 0; i < 4; i++) r[i] = SCALED ? fmaf(sc[i], t.v[h][mat][mt][i], r[i]) : r[i] + t.v[h][mat][mt][i];
                }
                acc[SUB][0][mat][mt] = r;
            }
        }
    };

    // Down: 16 pairs (one row tile) of row block rb of item i, staged, to
    // registers and from registers to HBM (wave 8).
    auto load_half = [&](u32x4(&v)[8]) __attribute__((always_inline)) {
#pragma unroll
        for (int it = 0; it < 8; it++) v[it] = *(const u32x4*)(gsm + G::STG + (2 * it + (lane >> 5)) * 512 + 16 * (lane & 31));
    };
    auto store_half = [&](int i, int rb, int half, const u32x4(&v)[8]) __attribute__((always_inline)) {
        const int32_t* rec = desc + (i % GM_DESC) * GM_REC;
        const int mn = rec[1];
#pragma unroll
        for (int it = 0; it < 8; it++) {
            const int m = 16 * half + 2 * it + (lane >> 5);
            if (m < mn)
                *(u32x4*)((uint8_t*)(a.y + (int64_t)rec[4 + m] * a.y_ld + rb * GM_ROWS) + 16 * (lane & 31)) = v[it];
        }
    };
    // Gate/up: results of item i (row block rb) from the staging area to HBM (wave 8).
    auto store_gu = [&](int i, int rb) __attribute__((always_inline)) {
        const int32_t* rec = desc + (i % GM_DESC) * GM_REC;
        const int mn = rec[1];
        const uint8_t* sh = gsm + G::STG;
        const uint8_t* sl = sh + M * GM_ROWS * 2;
        const float* ss = (const float*)(sl + M * GM_ROWS * 2);
#pragma unroll
        for (int it = 0; it < M / 4; it++) {
            const int m = 4 * it + (lane >> 4), seg = lane & 15;
            if (m < mn) {
                const int64_t o = (int64_t)rec[4 + m] * a.o_ld + rb * GM_ROWS;
                *(u32x4*)((uint8_t*)(a.o_hi + o) + 16 * seg) = *(const u32x4*)(sh + m * 256 + 16 * seg);
                *(u32x4*)((uint8_t*)(a.o_lo + o) + 16 * seg) = *(const u32x4*)(sl + m * 256 + 16 * seg);
            }
        }
        if (lane < mn) a.o_sc[(int64_t)rec[4 + lane] * a.osc_ld + rb] = ss[lane];
    };

    // The compute waves and the store wave run the same schedule (item and
    // stage pointers, barriers) in two separately compiled copies, so that
    // neither holds the other's registers.
    auto run = [&](auto sw_tag) __attribute__((always_inline)) {
        constexpr bool SW = decltype(sw_tag)::value;
        // prologue: records of the first two items, then S - 1 stages
        if constexpr (!SW) {
            int p1, r1, n1;
            if (wave == 6) {
                desc_dma(0, ip);
                if (item(1, p1, r1, n1)) desc_dma(1, p1);
            }
            WM_WAIT_VMCNT(0);
        }
        gm_bar();
        if constexpr (!SW) setup_issue();
        for (int s = 0; s < S - 1 && iok; s++) issue_next(sw_tag);

        int ci = 0, ckc = 0, cp = 0, crg = 0, cnkc = 0, sigma = 0, a_cons = 0;
        item(0, cp, crg, cnkc);
        // byte offset past a 16-byte boundary of this lane's row start in the
        // current item's matrix (unaligned K-quant rows only)
        auto row_shift = [&]() __attribute__((always_inline)) -> int {
            if constexpr (F::AL >= 16) return 0;
            const uint32_t rb = (uint32_t)(cp >= n_rp ? a.rb_s : a.rb_r);
            return (int)(((uint32_t)(crg * G::ROWS_ITEM + 16 * wave + c) * rb) & 15u);
        };
        int clsh = row_shift();
        bool two = false, pend = false;
        int pi = 0, prb = 0;
        // one stage: wait for it, meet, refill the ring, compute
        auto stage = [&](auto sub_tag) __attribute__((always_inline)) {
            if constexpr (!SW) {
                const int oldest = (int)(qpack & 15u);
                gm_wait_vm(qsum - oldest);
                qsum -= oldest;
                qpack >>= 4;
                --qn;
            }
            gm_bar();
            if constexpr (SW) {
                if (pend) {
                    store_gu(pi, prb);
                    pend = false;
                }
            }
            if (iok) issue_next(sw_tag);
            if constexpr (!SW) {
                const int as = a_cons % G::NAS;
                constexpr int SUB = decltype(sub_tag)::value;
                if constexpr (DIRECT) {
                    if (two) compute(sigma % S, as, ckc, clsh, std::true_type{}, acc[SUB]);
                    else compute(sigma % S, as, ckc, clsh, std::false_type{}, acc[SUB]);
                } else {
                    Sums t;
                    if (two) compute(sigma % S, as, ckc, clsh, std::true_type{}, t.v);
                    else compute(sigma % S, as, ckc, clsh, std::false_type{}, t.v);
                    accumulate(as, t, sub_tag);
                }
            }
            ++sigma;
        };
        for (;;) {
            if (ckc == 0) two = M > 16 && __builtin_amdgcn_readfirstlane(desc[(ci % GM_DESC) * GM_REC + 1]) > 16;
            stage(std::integral_constant<int, 0>{});
            if constexpr (NSUB > 1) stage(std::integral_constant<int, 1>{});
            if constexpr (NSUB > 2) stage(std::integral_constant<int, 2>{});
            if constexpr (NSUB > 3) stage(std::integral_constant<int, 3>{});
            ++a_cons;
            if (ckc < cnkc - 1) {
                ++ckc;
                continue;
            }
            // item done: epilogue into the staging area
            if constexpr (G::GU) {
                // this lane's pass rows are 16 mt + 4 g + i: one base per
                // array plus constant offsets
                float av[2][4];
                float* red = (float*)(gsm + G::RED);
                if constexpr (!SW) {
                    const uint32_t xw = (uint32_t)desc[(ci % GM_DESC) * GM_REC + 4 + GM_M + g];   // rows 4g..4g+3
                    const uint32_t xw1 = M > 16 ? (uint32_t)desc[(ci % GM_DESC) * GM_REC + 4 + GM_M + 4 + g] : 0u;
                    float* redp = red + 4 * g * GM_CW + wave;
#pragma unroll
                    for (int mt = 0; mt < G::MT; mt++)
#pragma unroll
                        for (int i = 0; i < 4; i++) {
                            const int xe = (int)(int8_t)((mt ? xw1 : xw) >> (8 * i));
                            const float xs = ldexpf(1.0f, xe);
                            const float gv = acc[0][0][0][mt][i], uv = G::SPLIT ? acc[NSUB - 1][0][0][mt][i]
                                                                                 : acc[0][0][NMAT - 1][mt][i];
                            const float v = silu_mul(gv * xs, uv * xs);
                            av[mt][i] = v;
                            float mx = fabsf(v);
                            mx = fmaxf(mx, dpp_f32<DPP_ROR8>(mx));
                            mx = fmaxf(mx, dpp_f32<DPP_ROR4>(mx));
                            mx = fmaxf(mx, dpp_f32<DPP_ROR2>(mx));
                            mx = fmaxf(mx, dpp_f32<DPP_ROR1>(mx));
                            if (c == 0) redp[(16 * mt + i) * GM_CW] = mx;
                        }
                }
                gm_bar();
                if constexpr (!SW) {
                    uint16_t* shp = (uint16_t*)(gsm + G::STG) + 4 * g * GM_ROWS + 16 * wave + c;
                    uint16_t* slp = shp + M * GM_ROWS;
                    float* ss = (float*)(gsm + G::STG + M * GM_ROWS * 4);
                    const float* redr = red + 4 * g * GM_CW;
#pragma unroll
                    for (int mt = 0; mt < G::MT; mt++)
#pragma unroll
                        for (int i = 0; i < 4; i++) {
                            const int o = 16 * mt + i;
                            const f32x4 r0 = *(const f32x4*)(redr + o * GM_CW), r1 = *(const f32x4*)(redr + o * GM_CW + 4);
                            const float mx = fmaxf(fmaxf(fmaxf(r0[0], r0[1]), fmaxf(r0[2], r0[3])),
                                                   fmaxf(fmaxf(r1[0], r1[1]), fmaxf(r1[2], r1[3])));
                            const int e = pf_exp(mx);
                            const float v = av[mt][i] * ldexpf(1.0f, -e);
                            const _Float16 hv = (_Float16)v;
                            const _Float16 lv = (_Float16)(v - (float)hv);
                            shp[o * GM_ROWS] = __builtin_bit_cast(uint16_t, hv);
                            slp[o * GM_ROWS] = __builtin_bit_cast(uint16_t, lv);
                            if (wave == 0 && c == 0) ss[4 * g + o] = ldexpf(1.0f, e);
                        }
                }
                pend = true;
                pi = ci;
                prb = crg;
            } else {
                // each row block's two row tiles pass through the staging
                // area into wave 8's registers, which it then stores
                float* sy = (float*)(gsm + G::STG) + 4 * g * GM_ROWS + 16 * wave + c;
                auto half = [&](auto u_tag, auto mt_tag) __attribute__((always_inline)) {
                    constexpr int U = decltype(u_tag)::value, MT = decltype(mt_tag)::value;
                    if constexpr (!SW) {
                        const f32x4 r = acc[U][0][0][MT];
#pragma unroll
                        for (int i = 0; i < 4; i++) sy[i * GM_ROWS] = r[i];
                    }
                    gm_bar();
                    u32x4 v[8];
                    if constexpr (SW) load_half(v);
                    gm_bar();
                    if constexpr (SW) store_half(ci, crg * NSUB + U, MT, v);
                };
                auto block = [&](auto u_tag) __attribute__((always_inline)) {
                    half(u_tag, std::integral_constant<int, 0>{});
                    if (two) half(u_tag, std::integral_constant<int, 1>{});
                };
                block(std::integral_constant<int, 0>{});
                if constexpr (NSUB > 1) block(std::integral_constant<int, 1>{});
                if constexpr (NSUB > 2) block(std::integral_constant<int, 2>{});
                if constexpr (NSUB > 3) block(std::integral_constant<int, 3>{});
            }
            if constexpr (!SW) {
#pragma unroll
                for (int u = 0; u < NSUB; u++)
#pragma unroll
                    for (int mat = 0; mat < NMAT; mat++) acc[u][0][mat][0] = acc[u][0][mat][1] = zero;
            }
            ckc = 0;
            ++ci;
            if (!item(ci, cp, crg, cnkc)) break;
            clsh = row_shift();
        }
        gm_bar();
        if constexpr (SW)
            if (pend) store_gu(pi, prb);
    };
    if (cw) run(std::false_type{});
    else run(std::true_type{});
#endif
}


template <int NMAT, int AHL, int NSUB, int WT, int M, int NSB = 1>
int launch_pf_gemm(const PfGemm& g, int n_wg, hipStream_t s) {
    typedef GmGeo<NMAT, AHL, NSUB, WT, M, NSB> G;
    if (g.ncol_r % G::KC || g.ncol_s % G::KC) return (int)hipErrorInvalidValue;
    PfGemm h = g;
    h.nkc_r = g.ncol_r / G::KC;
    h.nkc_s = g.ncol_s / G::KC;
    hipError_t e = hipFuncSetAttribute((const void*)k_pf_gemm<NMAT, AHL, NSUB, WT, M, NSB>,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, G::LDS);
    if (e != hipSuccess) return (int)e;
    hipLaunchKernelGGL((k_pf_gemm<NMAT, AHL, NSUB, WT, M, NSB>), dim3(n_wg), dim3(GM_THREADS), G::LDS, s, h);
    return (int)hipGetLastError();
}

// The K-quant instances (wm_prefill_kq.hip): gate/up (nmat = 2) and down
// (nmat = 1, nsub = 2 or 4) of Q2_K .. Q6_K, for passes of m = 16 or 32
// pairs.  Returns hipErrorInvalidValue for another combination.
int launch_pf_gemm_kq(int m, int nmat, int nsub, int wt, const PfGemm& g, int n_wg, hipStream_t s);

}  // namespace wm
