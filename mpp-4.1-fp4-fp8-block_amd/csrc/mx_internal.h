// mx_internal.h - launcher declarations shared between the kernel files and
// the C-ABI layer (mx_api.cpp).  Host-only types; no torch anywhere.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/mxfp4hip.h"

namespace mx {

// ---- codecs / elementwise (mx_codecs.hip) --------------------------------
hipError_t launch_pack(int fmt, const float* in, uint8_t* out, size_t n, hipStream_t st);
hipError_t launch_unpack(int fmt, const uint8_t* in, float* out, size_t n, hipStream_t st);
hipError_t launch_mxfp4_quantize(const void* src, int src_dtype, uint8_t* packed, uint8_t* scales,
                                 size_t rows, size_t k, hipStream_t st);
hipError_t launch_mxfp4_dequant_f16(const uint8_t* packed, const uint8_t* scales, uint16_t* out,
                                    size_t rows, size_t depth, hipStream_t st);
hipError_t launch_swiglu(int variant, const void* gate, const void* up, void* mid, size_t count,
                         hipStream_t st);
hipError_t launch_quant_rowwise(int fmt, const float* w, int rows, int k, uint8_t* q, float* scale,
                                hipStream_t st);
hipError_t launch_quant_int4_g32(const float* w, size_t rows, size_t k, uint8_t* q,
                                 uint16_t* scales, hipStream_t st);
hipError_t launch_quant_act_int8(const void* x, int x_dtype, int rows, int k, int8_t* q,
                                 float* scale, hipStream_t st);
hipError_t launch_fill_normal(void* dst, int dtype, size_t n, uint64_t seed, float mean,
                              float stddev, hipStream_t st);

// ---- half-activation GEMM family (mx_gemm_h.hip) --------------------------
// B operand encodings of the tiled fp16-MFMA GEMM.
enum BKind : int {
  BK_F16 = 0,      // f16 [N][K]
  BK_MXFP4 = 1,    // E2M1 [N][K/2] + E8M0 [N][K/32]
  BK_E4M3 = 2,     // FP8 E4M3 [N][K] + f32 row scale [N]
  BK_E5M2 = 3,     // FP8 E5M2 [N][K] + f32 row scale [N]
  BK_INT8 = 4,     // int8 [N][K] + f32 row scale [N]
  BK_INT4G32 = 5,  // int4 [N][K/2] + f16 scale [N][K/32]
  BK_I8 = 6,       // int8 [N][K] + f32 row scale [N], int8 activations (W8A8)
};

// Activation encodings of the small-M GEMM family (mx_gemm_q.hip).
enum AKind : int {
  AK_F16 = 0,      // f16 [M][K]
  AK_F32 = 1,      // f32 [M][K] (rounded to f16 for the MFMA)
  AK_I8 = 2,       // int8 [M][K] + f32 per-row (token) scale [M]
  AK_F8X2 = 3,     // two FP8 E4M3 terms + E8M0 scales per 64 K (the F8X2 layout below)
};

// F8X2: an activation matrix [M][K] (K % 64 == 0) as two FP8 E4M3 terms,
// v ~= t1 * 2^(e1-127) + t2 * 2^(e2-127), with one E8M0 pair (e1, e2) per
// row and 64-K group.  data [M][K/64][2 terms][64 bytes]: within a term the
// group's values sit in the order k 0-15, 32-47, 16-31, 48-63 (lane half h
// of a v_mfma_scale 32x32x64 FP8 operand holds k [16h, 16h+16) and
// [32+16h, 32+16h+16)); e8 [K/64][M] dwords, bytes 0 / 1 = e1 / e2.
inline size_t f8x2_data_bytes(size_t m, size_t k) { return 2 * m * k; }
inline size_t f8x2_e8_bytes(size_t m, size_t k) { return m * (k / 64) * 4; }
// f16 [M][K] -> F8X2 (mx_codecs.hip)
hipError_t launch_split_f8x2(const uint16_t* x, int m, int k, uint8_t* data, uint32_t* e8, hipStream_t st);

// Epilogues.
enum Epi : int {
  EPI_STORE_F32 = 0,     // C f32 [M][N]
  EPI_STORE_F16 = 1,     // C f16 [M][N]
  EPI_SWIGLU_F16 = 2,    // dual B: mid f16 = silu(g) * u              (swiglu_float)
  EPI_SWIGLU_HALF = 3,   // dual B: mid f16 = silu(clamp(g/16)) * u/16  (swiglu_half)
  EPI_SWIGLU_F32 = 4,    // dual B: mid f32 = silu(g) * u               (W8A8 mid)
  EPI_STORE_I32 = 5,     // C i32 [M][N], raw integer sums (AK_I8 x BK_I8, no scales)
  EPI_SWIGLU_F8X2 = 6,   // dual B: mid = silu(g) * u in f32, stored as F8X2 (c data, c_e8 scales)
};

struct GemmArgs {
  const void* a;  int a_dtype;            // f16 or f32 [M][K]
  const void* b0; const void* s0;         // weights + scales (matrix 0)
  const void* b1; const void* s1;         // second matrix for dual epilogues
  void* c;                                // output
  int m, n, k;                            // n = columns of each B matrix
};

hipError_t launch_gemm_h(int bkind, int epi, const GemmArgs& g, hipStream_t st);

// Grouped (MoE) launches: group e owns token rows [off[e], off[e+1]) of the
// activations / outputs, and its weights (scales) sit e * b_stride
// (e * s_stride) bytes after group 0's.  Passed by value as a kernel argument.
constexpr int kMaxGroups = 256;
struct GroupTable {
  int off[kMaxGroups + 1];
  size_t b_stride, s_stride;
};
// Small / medium-M GEMM family (mx_gemm_q.hip): 128 x 128 tiles, 64-K
// stages (128 for W8A8), split K with an ordered reduction for few tiles.
struct QGemmArgs {
  const void* a;                          // activations (AKind)
  const float* a_scale;                   // per-row scale for AK_I8
  const void* b0; const void* s0;         // weights + scales (matrix 0)
  const void* b1; const void* s1;         // second matrix for dual epilogues
  void* c;                                // output
  void* ws;                               // split-K partials (gemm_q_ws_bytes)
  int m, n, k;                            // n = rows of each weight matrix
  int tiles_m;                            // set by the launcher
  const uint32_t* a_e8;                   // AK_F8X2: E8M0 pairs [K/64][M]
  uint32_t* c_e8;                         // EPI_SWIGLU_F8X2: mid E8M0 pairs [N/64][M]
  const uint16_t* a_f16;                  // EPI_SWIGLU_F8X2: the f16 activations the F8X2
                                          // ones were split from (exact fix-up of NaN outputs)
  // Few-tile gate/up kernel only: weights of the GEMM that follows
  // (pf_rows rows of pf_row_bytes), pulled into each XCD's L2 for the
  // workgroups that will read them there (a hint; null for none).
  const void* pf = nullptr;
  int pf_rows = 0, pf_row_bytes = 0;
};
bool gemm_q_ok(int akind, int bkind, int epi, int m, int n, int k);
size_t gemm_q_ws_bytes(int akind, int bkind, int epi, int m, int n, int k);
int gemm_q_splits(int akind, int bkind, int epi, int m, int n, int k);
hipError_t launch_gemm_q(int akind, int bkind, int epi, const QGemmArgs& g, hipStream_t st);
// Few-tile MXFP4 GEMMs (mx_gemm_small.hip): f16 activations, at most 128
// rows; the dual gate/up + SwiGLU at K = 1024, or a plain GEMM with
// K % 1024 == 0 (<= 4096) and N % 32 == 0 (<= 2048).  launch_gemm_q takes
// this path for AK_F16 x BK_MXFP4 shapes it accepts.
bool small_gemm_ok(int epi, int m, int n, int k);
hipError_t launch_small_gemm(int epi, const QGemmArgs& g, hipStream_t st);
// K-split-in-workgroup MXFP4 gate/up + SwiGLU (mx_gemm_kq.hip): f16
// activations (SwiGLU to f16) or F8X2 ones (SwiGLU to F8X2), 64 x 64-channel
// tiles, 192 to 256 of them, K % 256 == 0 and K >= 1024 (BASELINE
// configs[2]).  launch_gemm_q takes this path for the BK_MXFP4 shapes it
// accepts.
bool kq_gemm_ok(int ak, int epi, int m, int n, int k);
hipError_t launch_kq_gemm(int ak, int epi, const QGemmArgs& g, hipStream_t st);
// Grouped (MoE) form, MXFP4 weights and f16 activations only; g.m = the
// largest group's rows, epi EPI_SWIGLU_F16 or EPI_STORE_F16, no split K.
hipError_t launch_gemm_q_grouped(int epi, const QGemmArgs& g, const GroupTable& gt, int groups, hipStream_t st);

// Decode-shaped (tokens <= 16) GEMV (mx_gemv.hip): one workgroup per 16
// weight rows, K split across its waves and reduced in LDS.
struct GemvArgs {
  const uint16_t* x;                      // f16 [T][K]
  const uint8_t* b0; const uint8_t* s0;   // MXFP4 weights (matrix 0)
  const uint8_t* b1; const uint8_t* s1;   // second matrix (dual / SwiGLU)
  uint16_t* out;                          // f16 [T][N] (out or mid)
  int t, n, k;
};
hipError_t launch_gemv_mxfp4(int dual_swiglu, const GemvArgs& g, hipStream_t st);

hipError_t launch_gemv_mxfp4_grouped(int dual_swiglu, const GemvArgs& g, const GroupTable& gt, int groups,
                                     hipStream_t st);

// Unscaled FP4 x FP4 / FP8 E4M3 x FP8 E4M3 GEMM for the accumulator probe
// (mx_accum.hip): C f32 or f16 [m][n] = A [m][k] . B [n][k]^T.
bool gemm_f8f6f4_unit_ok(int m, int n, int k);
// Rows of rb bytes -> rows of rbp >= rb bytes, zero-filled (mx_accum.hip).
hipError_t launch_pad_rows(const uint8_t* src, size_t rows, size_t rb, uint8_t* dst, size_t rbp, hipStream_t st);
// INT4 (src_int4) or INT8 rows of k values -> zero-padded rows of kp values
// as f16 (dst_f16) or int8, exactly (mx_accum.hip).
hipError_t launch_widen_rows(int src_int4, int dst_f16, const uint8_t* src, size_t rows, size_t k, void* dst,
                             size_t kp, hipStream_t st);
hipError_t launch_fill_u16(uint16_t* dst, size_t n, uint16_t value, hipStream_t st);
// dst[0, n) = value by a kernel (dst 4-byte aligned).
hipError_t launch_fill_u8(uint8_t* dst, size_t n, uint8_t value, hipStream_t st);
hipError_t launch_gemm_f8f6f4_unit(int fp4, int out_f32, const uint8_t* a, const uint8_t* b, void* c, int m,
                                   int n, int k, hipStream_t st);
size_t gemv_lds_need(int t, int k);  // dynamic LDS of one workgroup (<= 160 KB to run)

// W4A4 FP4 x FP4 scaled-MFMA GEMM (mx_gemm_fp4.hip).
// Scale planes come in two layouts:
//   reference    [rows][K/32] bytes (GUIDE:48-50)
//   stage-major  [K/128][rows_pad] dwords: the 4 E8M0 bytes of one 128-K
//                stage of a row in one dword, all rows of a stage contiguous
//                (rows_pad = rows rounded up to 256), so a 256-row tile's
//                scales for one stage are one contiguous 1 KB.
struct Fp4GemmArgs {
  const uint8_t* a; const uint8_t* as;    // activations MXFP4 [M][K/2] + scales
  const uint8_t* b0; const uint8_t* s0;   // weights MXFP4 [N][K/2] + scales
  const uint8_t* b1; const uint8_t* s1;   // up weights (dual epilogue)
  void* c;                                // f16 [M][N] or mid MXFP4 [M][N/2]
  uint8_t* cs;                            // mid scales (dual epilogue)
  int m, n, k;
  int stage_major;                        // 1: all scale planes stage-major; 2: also the
                                          // activations and the dual epilogue's mid,
                                          // [K/128][rows rounded up to 256][64 B] (v6)
  float* ws;                              // split-K partials (splits > 1)
  int splits;                             // K splits, from gemm_fp4_splits (0 or 1: none)
};
hipError_t launch_gemm_fp4(int dual_requant, const Fp4GemmArgs& g, hipStream_t st);
// K splits for the W4A4 GEMM of this shape (stage-major scales) and the
// bytes of f32 partials they need (0 without a split).
int gemm_fp4_splits(int dual_requant, int m, int n, int k);
size_t gemm_fp4_ws_bytes(int dual_requant, int m, int n, int k);
// 256x256-tile kernel for stage-major scales (mx_gemm_fp4_v3.hip).
hipError_t launch_gemm_fp4_v3(int dual_requant, const Fp4GemmArgs& g, hipStream_t st);
// Full-cache-line DMA, K stage 256 (mx_gemm_fp4_v5.hip), for K % 512 == 0.
hipError_t launch_gemm_fp4_v5(int dual_requant, const Fp4GemmArgs& g, hipStream_t st);
bool gemm_fp4_v5_ok(int k);
// 128-K stages in a four-slot ring, stage-major activations
// (mx_gemm_fp4_v6.hip), for whole-tile grids with K % 512 == 0.
hipError_t launch_gemm_fp4_v6(int dual_requant, const Fp4GemmArgs& g, hipStream_t st);
bool gemm_fp4_v6_ok(int dual_requant, int n, int k);
// True when a W4A4 MLP (T x H x I) runs both GEMMs on v6, so that the
// prologue writes x, and the gate/up GEMM the mid, stage-major.
bool w4a4_act_stage_major(int t, int hidden, int inter);
// True when the stage-major 256x256 kernel takes this MLP (T x H x I).
bool w4a4_stage_major_ok(int hidden, int inter);
__host__ __device__ inline size_t stage_major_rows(size_t rows) { return (rows + 255) / 256 * 256; }
// W4A4 prologue, one launch: x f16 [T][H] -> MXFP4 [T][H/2] + stage-major
// scales, and the three weight scale planes -> stage-major copies.
struct W4A4Prologue {
  const uint16_t* x; uint8_t* xq; uint8_t* xs;
  const uint8_t* sg; const uint8_t* su; const uint8_t* sd;   // reference layout
  uint8_t* sg2; uint8_t* su2; uint8_t* sd2;                  // stage-major
  int t, h, i;
  int xq_sm;  // 1: x codes stage-major [H/128][Tpad][64 B], else [T][H/2]
};
hipError_t launch_w4a4_prologue(const W4A4Prologue& p, hipStream_t st);
// After the W4A4 down GEMM: outputs of rows whose down scales hold byte 255
// rewritten to the reference's +-inf where its semantics give infinity
// (mid codes mq [T][I/2], mid scales stage-major or [T][I/32]).
hipError_t launch_w4a4_down_inf(const uint8_t* wd, const uint8_t* sd, const uint8_t* mq, const uint8_t* ms,
                                int ms_stage_major, int t, int h, int i, uint16_t* out, hipStream_t st);

}  // namespace mx
