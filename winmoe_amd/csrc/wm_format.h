// wm_format.h -- GGUF block formats shared by host and device code.
//
// Block layouts (little-endian, packed):
//   Q8_0  {u16 d; i8 qs[32]}                              34 B / 32 w   (q8_dequant.h:15-18)
//   Q4_K  {u16 d; u16 dmin; u8 scales[12]; u8 qs[128]}    144 B / 256 w (q4k_dequant.h:28-33)
//   Q5_K  {u16 d; u16 dmin; u8 scales[12]; u8 qh[32]; u8 qs[128]}  176 B (q5k_dequant.h:19-25)
//   Q6_K  {u8 ql[128]; u8 qh[64]; i8 scales[16]; u16 d}   210 B / 256 w (q6k_dequant.h:20-25)
//   Q2_K  {u8 scales[16]; u8 qs[64]; u16 d; u16 dmin}     84 B / 256 w  (public ggml format)
//   Q3_K  {u8 hmask[32]; u8 qs[64]; u8 scales[12]; u16 d} 110 B / 256 w (public ggml format)
#pragma once
#include <stdint.h>

#if defined(__HIPCC__)
#define WM_HD __host__ __device__ inline
#else
#define WM_HD inline
#endif

namespace wm {

enum QType : int { F32 = 0, F16 = 1, Q8_0 = 8, Q2_K = 10, Q3_K = 11, Q4_K = 12, Q5_K = 13, Q6_K = 14 };

WM_HD constexpr int block_bytes(int t) {
    switch (t) {
    case Q8_0: return 34;
    case Q2_K: return 84;
    case Q3_K: return 110;
    case Q4_K: return 144;
    case Q5_K: return 176;
    case Q6_K: return 210;
    default: return 0;
    }
}

WM_HD constexpr int block_elems(int t) {
    switch (t) {
    case Q8_0: return 32;
    case Q2_K: case Q3_K: case Q4_K: case Q5_K: case Q6_K: return 256;
    default: return 0;
    }
}

WM_HD bool supported(int t) { return block_bytes(t) != 0; }

WM_HD int64_t matrix_bytes(int t, int64_t rows, int64_t in) {
    return rows * (in / block_elems(t)) * block_bytes(t);
}

// Every lane of a 64-wide wave owns one 64-weight "segment" of a row: for
// Q8_0 a pair of consecutive blocks, for the K-quants a quarter of a
// 256-weight super-block.  A row of `in` weights therefore has in/64
// segments; a wave covers floor(64 / (in/64)) rows per pass.
constexpr int SEG = 64;

// Column (within the row) of the j-th weight (0..63) of segment `seg`, in the
// order the expert kernels pack quantised values into dwords.
//   Q8_0 / Q4_K / Q5_K: the segment is 64 contiguous columns.
//   Q6_K / Q2_K / Q3_K: segment (block b, half h, sixteenth i) covers four runs
//   of 16 columns at 256b + 128h + 32g + 16i (g = 0..3).
WM_HD int seg_col(int t, int seg, int j) {
    if (t == Q8_0 || t == Q4_K || t == Q5_K) return seg * 64 + j;
    int b = seg >> 2, r = seg & 3, h = r >> 1, i = r & 1, g = j >> 4;
    return 256 * b + 128 * h + 32 * g + 16 * i + (j & 15);
}

// Number of packed dwords per segment and of independently scaled runs.
WM_HD int seg_ndw(int t) { return t == Q8_0 ? 17 : 16; }
WM_HD int seg_nrun(int t) { return (t == Q8_0 || t == Q4_K || t == Q5_K) ? 2 : 4; }

// Activation operand of one segment in the integer-dot layout: two signed
// 8-bit digits per value (x ~= s * (256*hi + lo), |256*hi + lo| <= 32639),
// packed in the same byte order as the segment's quantised values, the exact
// integer sums of 256*hi+lo over each run, and the scale s.
constexpr int XOP_DW = 40;     // dwords per segment operand (hi[17] lo[17] sum[4] s pad)
constexpr int XOP_HI = 0, XOP_LO = 17, XOP_SUM = 34, XOP_S = 38;

}  // namespace wm
