/*
 * mx_oracle.h - CPU restatement of the reference's MXFP4 MLP arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the checker
 * (or the timed CPU baseline), never as the product path.  The product is
 * libmxfp4hip (HIP kernels for gfx950); it has no CPU fallback.
 *
 * Every function cites the reference file:line it restates.  Paths are
 * relative to the reference root (Anemll/MPP-4.1-FP4-FP8-block):
 *   MX = Sources/MetalFP41Probe/Shaders/MXFP4Kernels.metal
 *   MP = Sources/MetalFP41Probe/Shaders/MPPMLPKernels.metal
 *   PN = Sources/MetalFP41Probe/Shaders/PackedNumericKernels.metal
 *   MS = Sources/MetalFP41Probe/main.swift
 */
#ifndef MX_ORACLE_H
#define MX_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- scalar codecs ---------------------------------------------------- */
uint16_t orc_f32_to_f16(float f);            /* IEEE binary16, RNE, subnormals */
float orc_f16_to_f32(uint16_t h);
void orc_f32_to_f16_bulk(const float *in, size_t n, uint16_t *out);
float orc_e8m0_to_float(uint8_t b);          /* MX:26-29  bits<<23           */
float orc_fp4_decode(uint8_t nibble);        /* MX:33-36  LUT                */
uint8_t orc_fp4_encode(float x);             /* MS:112-115 KAT; RNE, sat ±6  */
float orc_fp8_e4m3_decode(uint8_t b);
uint8_t orc_fp8_e4m3_encode(float x);        /* MS:118-124 KAT; RNE, sat ±448 */
float orc_fp8_e5m2_decode(uint8_t b);
uint8_t orc_fp8_e5m2_encode(float x);        /* MS:125-131 KAT; RNE, sat ±57344 */

/* ---- bulk roundtrip (PN:35-96) ---------------------------------------- */
/* fmt: 0 = FP4 E2M1 (2 per byte, low nibble = even index), 1 = FP8 E4M3,
 * 2 = FP8 E5M2.  packed must hold n/2 (fp4) or n (fp8) bytes. */
void orc_pack(int fmt, const float *in, size_t n, uint8_t *packed);
void orc_unpack(int fmt, const uint8_t *packed, size_t n, float *out);

/* ---- MXFP4 block quantizer (BASELINE-defined) -------------------------- */
/* scale byte = floor(log2(amax)) - 2 + 127 per 32 K-elements; elements RNE,
 * saturating to E2M1.  src row-major [rows][k] (f32 or f16 bits). */
uint8_t orc_mxfp4_scale_byte(float amax);
void orc_mxfp4_quantize_f32(const float *src, int rows, int k, uint8_t *packed, uint8_t *scales);
void orc_mxfp4_quantize_f16(const uint16_t *src, int rows, int k, uint8_t *packed, uint8_t *scales);

/* ---- dequant to half (MX:509-538, MX:543-564) -------------------------- */
void orc_mxfp4_dequant_f16(const uint8_t *packed, const uint8_t *scales, int rows, int depth,
                           uint16_t *out);

/* ---- MXFP4 matmul (MX:138-173) ----------------------------------------- */
/* c[m][n] = sum_k a[m][k] * fp4(b[n][k]) * 2^(s[n][k/32]-127).
 * a_kind 0: a is f16 bits [m][k]; 1: a is f32 [m][k].  Accumulates in double. */
void orc_mxfp4_matmul(const void *a, int a_kind, const uint8_t *b, const uint8_t *s, int m, int n,
                      int k, float *c);

/* ---- SwiGLU (MP:186-257) ----------------------------------------------- */
float orc_silu(float g);
void orc_swiglu_float(const float *gate, const float *up, size_t count, float *mid);   /* MP:186-202 */
void orc_swiglu_half(const float *gate, const float *up, size_t count, uint16_t *mid); /* MP:204-220 */
void orc_swiglu_i8(const int32_t *gate, const int32_t *up, size_t count, int8_t *mid);  /* MP:240-257 */

/* ---- full MXFP4 MLP ----------------------------------------------------- */
/* mode 0: f16 activations, dequantize-then-FP32(here: double)-accumulate,
 *         mid = silu(g)*u (float), f16 out.
 * mode 1: W4A4: x and mid re-quantized to MXFP4 along K, f16 out.
 * mode 2: reference checksum row: swiglu_half (x1/16, clamp +-20, mid half),
 *         f32 out (MS:1953-2135 with MP:204-220).
 * rows_sel: token indices to evaluate (NULL = all tokens); out has
 * n_sel x hidden entries (f16 bits for modes 0/1, f32 for mode 2).
 * threads: worker threads (>=1). */
/* Dot products of orc_mlp_mxfp4 / orc_mlp_format (except W8A8, which is
 * integer) accumulate in float64 by default; on != 0 switches to float32 in
 * K order, BASELINE's CPU-baseline semantics (bench.py's cpu_baseline leg
 * only; the tests keep float64).  Process-wide. */
void orc_set_accum_f32(int on);

void orc_mlp_mxfp4(int mode, int tokens, int hidden, int inter, const uint16_t *x,
                   const uint8_t *wg, const uint8_t *sg, const uint8_t *wu, const uint8_t *su,
                   const uint8_t *wd, const uint8_t *sd, const int *rows_sel, int n_sel,
                   void *out, int threads);

/* ---- weight-format rows (MP:50-125, PN:25-33) ------- */
/* fmt: 1 = FP8 E4M3 per-row f32 scale (amax/448), 2 = FP8 E5M2 per-row
 * (amax/57344), 3 = INT8 per-row (amax/127), 4 = INT4 two per byte,
 * f16 scale per 32 K-elements (amax/7). */
void orc_quant_rowwise(int fmt, const float *w, int rows, int k, uint8_t *q, float *row_scale);
void orc_quant_int4_g32(const float *w, int rows, int k, uint8_t *q, uint16_t *scale_f16);
/* W8A8 activations: int8 per-token, scale = amax/127. */
void orc_quant_int8_per_token(const float *x, int tokens, int k, int8_t *q, float *scale);
/* Format MLP (f16 activations for fmt 1..4; fmt 5 = W8A8 with int8 weights
 * per-row, int8 activations per-token, int32 accumulate, per-token requant
 * of mid).  Weight args: q + row_scale (fmt 1,2,3,5) or q + g32 scales (fmt 4). */
void orc_mlp_format(int fmt, int tokens, int hidden, int inter, const uint16_t *x,
                    const uint8_t *qg, const void *sg, const uint8_t *qu, const void *su,
                    const uint8_t *qd, const void *sd, const int *rows_sel, int n_sel,
                    uint16_t *out, int threads);

/* ---- reference data generators (MS:2785-2842) --------------------------
 * lcg_bytes, lcg_pattern and lcg_half are pinned end to end by the
 * reference's published checksum 403573 (README.md:292-294), which is
 * computed over data made by all three.  lcg_int8 (makeInt8MatrixValues,
 * MS:2833-2842) has no published output of its own; it is makeHalfMatrixValues
 * before the Float16 scale, and is pinned by equality with lcg_half at
 * scale 1 (tests/test_oracle_mlp.py). */
void orc_lcg_bytes(uint32_t seed, size_t count, uint8_t *out);
void orc_lcg_pattern(uint32_t seed, size_t count, const uint8_t *pattern, int pattern_count,
                     uint8_t *out);
void orc_lcg_half(uint32_t seed, size_t count, float scale, uint16_t *out);
void orc_lcg_int8(uint32_t seed, size_t count, int8_t *out);

/* ---- checksums (MS:2844-2884) ------------------------------------------
 * checksum_f32 is pinned by 403573.  checksum_i32 and checksum_f16raw
 * (sampleIntChecksum / sampleHalfRawChecksum) have no published value; they
 * sample like checksum_f32 and are pinned by equality with it on integer
 * data and by the closed form on index ramps (tests/test_oracle_mlp.py). */
double orc_checksum_f32(const float *p, size_t count, int *samples);
int64_t orc_checksum_i32(const int32_t *p, size_t count, int *samples);
uint64_t orc_checksum_f16raw(const uint16_t *p, size_t count, int *samples);

#ifdef __cplusplus
}
#endif
#endif
