/*
 * mx_oracle.c - CPU restatement of the reference's MXFP4 MLP arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY (see mx_oracle.h).  The reference is Swift +
 * Metal (Apple only) and cannot be built or run here, so this file restates
 * its algorithm from the sources it cites.  Where the reference leaves a
 * case open (ties, NaN/Inf, E8M0 endpoints) the choice made here is stated
 * at the function and pinned by a test in tests/.
 *
 * Citations (reference root = Anemll/MPP-4.1-FP4-FP8-block):
 *   MX = Sources/MetalFP41Probe/Shaders/MXFP4Kernels.metal
 *   MP = Sources/MetalFP41Probe/Shaders/MPPMLPKernels.metal
 *   PN = Sources/MetalFP41Probe/Shaders/PackedNumericKernels.metal
 *   MS = Sources/MetalFP41Probe/main.swift
 *   GUIDE = docs/MXFP4-MPP41-GUIDE.md
 */
#include "mx_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* ------------------------------------------------------------------------ */
/* IEEE binary16 <-> binary32.  Round-to-nearest-even with subnormals; this
 * is the rounding of Metal's half(float) conversion used throughout the
 * reference (e.g. MX:536, MP:219).  Pinned exhaustively against numpy's
 * float16 cast in tests/test_oracle_codecs.py. */
uint16_t orc_f32_to_f16(float f)
{
    uint32_t x = f2u(f);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t a = x & 0x7fffffffu;
    if (a >= 0x7f800000u) {                 /* inf / nan */
        if (a > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((a >> 13) & 0x3ffu));
        return (uint16_t)(sign | 0x7c00u);
    }
    if (a >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* >= 65520 -> inf */
    if (a < 0x38800000u) {                  /* result subnormal or zero */
        uint32_t e = a >> 23;
        if (e < 102) return (uint16_t)sign;
        uint32_t m = (a & 0x7fffffu) | 0x800000u;
        uint32_t shift = 126 - e;           /* 14..24 */
        uint32_t q = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (q & 1u))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t r = a - 0x38000000u;           /* rebias 127 -> 15 */
    uint32_t q = r >> 13;
    uint32_t rem = r & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q++;
    return (uint16_t)(sign | q);
}

float orc_f16_to_f32(uint16_t h)
{
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu;
    uint32_t m = h & 0x3ffu;
    if (e == 0x1f) return u2f(sign | 0x7f800000u | (m << 13));
    if (e == 0) {
        float v = (float)m * 5.9604644775390625e-08f; /* 2^-24, exact */
        return sign ? -v : v;
    }
    return u2f(sign | ((e + 112u) << 23) | (m << 13));
}

void orc_f32_to_f16_bulk(const float *in, size_t n, uint16_t *out)
{
    for (size_t i = 0; i < n; i++) out[i] = orc_f32_to_f16(in[i]);
}

/* ------------------------------------------------------------------------ */
/* E8M0 decode: as_type<float>(uint(bits) << 23) (MX:26-29, GUIDE:398-399).
 * Byte 0 -> 0.0 and byte 255 -> +inf, as in the reference (OCP/gfx950 read
 * them as 2^-127 and NaN; that divergence is documented, not hidden). */
float orc_e8m0_to_float(uint8_t b) { return u2f((uint32_t)b << 23); }

/* FP4 E2M1 value table (MX:33-36, GUIDE:57-62). */
static const float kFP4[16] = {0.0f,  0.5f,  1.0f,  1.5f,  2.0f,  3.0f,  4.0f,  6.0f,
                               -0.0f, -0.5f, -1.0f, -1.5f, -2.0f, -3.0f, -4.0f, -6.0f};
float orc_fp4_decode(uint8_t nibble) { return kFP4[nibble & 15u]; }

/* Round a finite, non-negative float to a minifloat with `mbits` mantissa
 * bits and exponent bias `bias`, RNE, returning the magnitude code; codes
 * above max_code saturate to max_code.  Ties go to the even code, which is
 * the even mantissa.  Used for E2M1, E4M3 and E5M2 (all sign-magnitude). */
static uint32_t round_minifloat(uint32_t a /* |x| bits */, int mbits, int bias, uint32_t max_code)
{
    if (a == 0) return 0;
    int ex = (int)(a >> 23) - 127;
    uint32_t mm = (a & 0x7fffffu) | 0x800000u;
    if ((a >> 23) == 0) return 0;           /* f32 subnormal: far below every target */
    int emin = 1 - bias;
    uint32_t code;
    if (ex >= emin) {
        int shift = 23 - mbits;
        uint32_t q = mm >> shift;
        uint32_t rem = mm & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1);
        if (rem > half || (rem == half && (q & 1u))) q++;
        if (q == (2u << mbits)) { q >>= 1; ex++; }
        int be = ex + bias;
        if (be > 64) return max_code;       /* far beyond any target range */
        code = ((uint32_t)be << mbits) | (q & ((1u << mbits) - 1u));
    } else {
        int shift = 23 + emin - mbits - ex;
        if (shift >= 32) return 0;
        uint32_t q = mm >> shift;
        uint32_t rem = mm & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1);
        if (rem > half || (rem == half && (q & 1u))) q++;
        code = q;
    }
    return code > max_code ? max_code : code;
}

/* FP4 E2M1 encode.  Pinned by the reference KAT (MS:112-115): -8 -> -6,
 * 8 -> 6 (saturating), every table value round-trips.  Ties: RNE (OCP MX).
 * NaN -> sign|7 (max magnitude), Inf -> saturate: not pinned by the
 * reference; matches the gfx950 conversion and is pinned by a GPU test. */
uint8_t orc_fp4_encode(float x)
{
    uint32_t u = f2u(x);
    uint8_t sign = (uint8_t)((u >> 28) & 8u);
    uint32_t a = u & 0x7fffffffu;
    if (a >= 0x7f800000u) return (uint8_t)(sign | 7u);
    return (uint8_t)(sign | round_minifloat(a, 1, 1, 7u));
}

/* FP8 E4M3 (OCP "fn": no inf, NaN = S.1111.111, max 448).
 * Pinned by the KAT at MS:118-124: +-512 -> +-448 (saturating).  Inf
 * saturates, NaN -> sign|0x7f. */
float orc_fp8_e4m3_decode(uint8_t b)
{
    uint32_t s = b >> 7, e = (b >> 3) & 15u, m = b & 7u;
    float v;
    if (e == 15 && m == 7) v = NAN;
    else if (e == 0) v = ldexpf((float)m, -9);
    else v = ldexpf((float)(8u + m), (int)e - 10);
    return s ? -v : v;
}

uint8_t orc_fp8_e4m3_encode(float x)
{
    uint32_t u = f2u(x);
    uint8_t sign = (uint8_t)((u >> 24) & 0x80u);
    uint32_t a = u & 0x7fffffffu;
    if (a > 0x7f800000u) return (uint8_t)(sign | 0x7fu);
    if (a == 0x7f800000u) return (uint8_t)(sign | 0x7eu);
    return (uint8_t)(sign | round_minifloat(a, 3, 7, 0x7eu));
}

/* FP8 E5M2 (IEEE-like: inf = S.11111.00, NaN mantissa != 0, max 57344).
 * Pinned by the KAT at MS:125-131 (57344 round-trips).  Finite overflow and
 * Inf saturate to +-57344 (consistent with E4M3); NaN -> sign|0x7e. */
float orc_fp8_e5m2_decode(uint8_t b)
{
    uint32_t s = b >> 7, e = (b >> 2) & 31u, m = b & 3u;
    float v;
    if (e == 31) v = m ? NAN : INFINITY;
    else if (e == 0) v = ldexpf((float)m, -16);
    else v = ldexpf((float)(4u + m), (int)e - 17);
    return s ? -v : v;
}

uint8_t orc_fp8_e5m2_encode(float x)
{
    uint32_t u = f2u(x);
    uint8_t sign = (uint8_t)((u >> 24) & 0x80u);
    uint32_t a = u & 0x7fffffffu;
    if (a > 0x7f800000u) return (uint8_t)(sign | 0x7eu);
    if (a == 0x7f800000u) return (uint8_t)(sign | 0x7bu);
    return (uint8_t)(sign | round_minifloat(a, 2, 15, 0x7bu));
}

/* Bulk pack / unpack: the roundtrip kernels at PN:35-96 (pack<fmt>(vec),
 * then unpack<float>).  FP4 storage: low nibble = even index (MX:345,
 * MX:562-563). */
void orc_pack(int fmt, const float *in, size_t n, uint8_t *packed)
{
    if (fmt == 0) {
        for (size_t i = 0; i + 1 < n; i += 2)
            packed[i / 2] = (uint8_t)(orc_fp4_encode(in[i]) | (orc_fp4_encode(in[i + 1]) << 4));
        if (n & 1) packed[n / 2] = orc_fp4_encode(in[n - 1]);
    } else if (fmt == 1) {
        for (size_t i = 0; i < n; i++) packed[i] = orc_fp8_e4m3_encode(in[i]);
    } else {
        for (size_t i = 0; i < n; i++) packed[i] = orc_fp8_e5m2_encode(in[i]);
    }
}

void orc_unpack(int fmt, const uint8_t *packed, size_t n, float *out)
{
    for (size_t i = 0; i < n; i++) {
        if (fmt == 0) out[i] = orc_fp4_decode((uint8_t)(packed[i / 2] >> ((i & 1) * 4)));
        else if (fmt == 1) out[i] = orc_fp8_e4m3_decode(packed[i]);
        else out[i] = orc_fp8_e5m2_decode(packed[i]);
    }
}

/* ------------------------------------------------------------------------ */
/* MXFP4 block quantizer ("E8M0 scale =
 * 2^(floor(log2(amax))-2); elements rounded to nearest even, saturating to
 * E2M1"; OCP MX v1.0 with emax(E2M1) = 2).  floor(log2) is taken from the
 * float's exponent bits, exactly.  Special cases (not in the reference):
 *   amax == 0          -> byte 127 (scale 1.0), codes encode(+-0)
 *   amax inf/NaN       -> byte 255, codes 0
 *   exponent < -127    -> byte 0 (only for subnormal amax)
 * Elements: code = encode(x * 2^-e) (exact scaling, then RNE). */
uint8_t orc_mxfp4_scale_byte(float amax)
{
    uint32_t a = f2u(amax) & 0x7fffffffu;
    if (a >= 0x7f800000u) return 255;
    if (a == 0) return 127;
    int fl;
    if ((a >> 23) == 0) {                   /* subnormal: MSB position */
        int msb = 31 - __builtin_clz(a);
        fl = msb - 149;
    } else {
        fl = (int)(a >> 23) - 127;
    }
    int e = fl - 2;
    if (e < -127) e = -127;
    return (uint8_t)(e + 127);
}

static void quantize_block(const float *v, uint8_t *packed_row, int k0, uint8_t *scale_out)
{
    float amax = 0.0f;
    int nonfinite = 0;
    for (int j = 0; j < 32; j++) {
        float a = fabsf(v[j]);
        if (!(a <= 3.4028234663852886e38f)) nonfinite = 1;
        else if (a > amax) amax = a;
    }
    uint8_t sb = nonfinite ? 255 : orc_mxfp4_scale_byte(amax);
    *scale_out = sb;
    for (int j = 0; j < 32; j += 2) {
        uint8_t c0, c1;
        if (sb == 255) {
            c0 = c1 = 0;
        } else {
            int e = (int)sb - 127;
            c0 = orc_fp4_encode(ldexpf(v[j], -e));
            c1 = orc_fp4_encode(ldexpf(v[j + 1], -e));
        }
        packed_row[(k0 + j) / 2] = (uint8_t)(c0 | (c1 << 4));
    }
}

void orc_mxfp4_quantize_f32(const float *src, int rows, int k, uint8_t *packed, uint8_t *scales)
{
    int kb = k / 32;
    for (int r = 0; r < rows; r++)
        for (int b = 0; b < kb; b++)
            quantize_block(src + (size_t)r * k + b * 32, packed + (size_t)r * (k / 2), b * 32,
                           scales + (size_t)r * kb + b);
}

void orc_mxfp4_quantize_f16(const uint16_t *src, int rows, int k, uint8_t *packed, uint8_t *scales)
{
    int kb = k / 32;
    float tmp[32];
    for (int r = 0; r < rows; r++)
        for (int b = 0; b < kb; b++) {
            for (int j = 0; j < 32; j++) tmp[j] = orc_f16_to_f32(src[(size_t)r * k + b * 32 + j]);
            quantize_block(tmp, packed + (size_t)r * (k / 2), b * 32, scales + (size_t)r * kb + b);
        }
}

/* Dequant to half: out[r][k] = half(fp4(packed) * e8m0(scale[r][k/32]))
 * (MX:509-538 native unpack; MX:543-564 LUT; both give the same bits,
 * README.md:240-242).  The product is exact in f32; one RNE to half. */
void orc_mxfp4_dequant_f16(const uint8_t *packed, const uint8_t *scales, int rows, int depth,
                           uint16_t *out)
{
    int kb = depth / 32;
    for (int r = 0; r < rows; r++)
        for (int k = 0; k < depth; k++) {
            uint8_t byte = packed[(size_t)r * (depth / 2) + k / 2];
            float v = orc_fp4_decode((uint8_t)(byte >> ((k & 1) * 4)));
            float s = orc_e8m0_to_float(scales[(size_t)r * kb + k / 32]);
            out[(size_t)r * depth + k] = orc_f32_to_f16(v * s);
        }
}

/* Dequantize one weight row to f32 (exact). */
static void deq_row(const uint8_t *packed, const uint8_t *scales, int row, int k, float *dst)
{
    const uint8_t *p = packed + (size_t)row * (k / 2);
    const uint8_t *s = scales + (size_t)row * (k / 32);
    for (int b = 0; b < k / 32; b++) {
        float sc = orc_e8m0_to_float(s[b]);
        for (int j = 0; j < 32; j += 2) {
            uint8_t byte = p[(b * 32 + j) / 2];
            dst[b * 32 + j] = kFP4[byte & 15u] * sc;
            dst[b * 32 + j + 1] = kFP4[byte >> 4] * sc;
        }
    }
}

/* c[m][n] = sum_k a[m][k] * fp4(b[n][k]) * 2^(s[n][k/32]-127): the native
 * scale-plane matmul (MX:138-173; identical math to the per-block fused
 * form MX:42-130).  Accumulated in double; this is the "truth" the GPU's
 * FP32 accumulation is compared against within tolerance. */
void orc_mxfp4_matmul(const void *a, int a_kind, const uint8_t *b, const uint8_t *s, int m, int n,
                      int k, float *c)
{
    float *w = (float *)malloc(sizeof(float) * (size_t)k);
    float *arow = (float *)malloc(sizeof(float) * (size_t)k);
    for (int j = 0; j < n; j++) {
        deq_row(b, s, j, k, w);
        for (int i = 0; i < m; i++) {
            if (a_kind == 0) {
                const uint16_t *ah = (const uint16_t *)a + (size_t)i * k;
                for (int t = 0; t < k; t++) arow[t] = orc_f16_to_f32(ah[t]);
            } else {
                memcpy(arow, (const float *)a + (size_t)i * k, sizeof(float) * (size_t)k);
            }
            double acc = 0.0;
            for (int t = 0; t < k; t++) acc += (double)arow[t] * (double)w[t];
            c[(size_t)i * n + j] = (float)acc;
        }
    }
    free(w);
    free(arow);
}

/* ------------------------------------------------------------------------ */
/* SwiGLU.  silu(g) = g / (1 + exp(-g)) (MP:201, PN:19-23). */
float orc_silu(float g) { return g / (1.0f + expf(-g)); }

/* mpp_mlp_swiglu_float (MP:186-202): mid = silu(g) * u, f32. */
void orc_swiglu_float(const float *gate, const float *up, size_t count, float *mid)
{
    for (size_t i = 0; i < count; i++) mid[i] = orc_silu(gate[i]) * up[i];
}

/* mpp_mlp_swiglu_half (MP:204-220): g' = clamp(g/16, +-20), u' = u/16,
 * mid = half(silu(g') * u'). */
void orc_swiglu_half(const float *gate, const float *up, size_t count, uint16_t *mid)
{
    for (size_t i = 0; i < count; i++) {
        float g = gate[i] * 0.0625f;
        g = g < -20.0f ? -20.0f : (g > 20.0f ? 20.0f : g);
        float u = up[i] * 0.0625f;
        mid[i] = orc_f32_to_f16(orc_silu(g) * u);
    }
}

/* mpp_mlp_swiglu_i8 (MP:240-257): g = clamp(gate * 2^-12, +-20),
 * u = up * 2^-12 (not clamped), v = silu(g) * u * 32, mid = int8(rint(clamp(v,
 * -128, 127))).  rintf rounds half to even, as Metal's rint does. */
void orc_swiglu_i8(const int32_t *gate, const int32_t *up, size_t count, int8_t *mid)
{
    for (size_t i = 0; i < count; i++) {
        float g = (float)gate[i] * 0.000244140625f;
        g = g < -20.0f ? -20.0f : (g > 20.0f ? 20.0f : g);
        float u = (float)up[i] * 0.000244140625f;
        float v = orc_silu(g) * u * 32.0f;
        v = v < -128.0f ? -128.0f : (v > 127.0f ? 127.0f : v);
        mid[i] = (int8_t)(int)rintf(v);
    }
}

/* ------------------------------------------------------------------------ */
/* Threaded row loops.  Work is split over weight rows; each worker decodes a
 * row once and dots it with every selected token. */
typedef struct {
    int mode;           /* MLP mode (see header) or format id + 16 */
    int n_rows, k;      /* weight rows / reduction depth */
    int n_tok;
    const float *act;   /* [n_tok][k] f32 activations */
    const uint8_t *q;   /* weight data */
    const void *s;      /* weight scales */
    int fmt;            /* 0 = mxfp4, 1..4 = formats */
    float *out;         /* [n_tok][n_rows] */
    int r0, r1;
} rowjob_t;

static void deq_row_fmt(int fmt, const uint8_t *q, const void *s, int row, int k, float *dst)
{
    if (fmt == 0) { deq_row(q, (const uint8_t *)s, row, k, dst); return; }
    const uint8_t *p = q + (size_t)row * (fmt == 4 ? k / 2 : k);
    if (fmt == 4) {
        const uint16_t *sc = (const uint16_t *)s + (size_t)row * (k / 32);
        for (int t = 0; t < k; t++) {
            uint8_t byte = p[t / 2];
            int v = (((byte >> ((t & 1) * 4)) & 15) ^ 8) - 8;   /* PN:30-33 */
            dst[t] = (float)v * orc_f16_to_f32(sc[t / 32]);
        }
        return;
    }
    float rs = ((const float *)s)[row];
    for (int t = 0; t < k; t++) {
        float v = fmt == 1 ? orc_fp8_e4m3_decode(p[t])
                           : fmt == 2 ? orc_fp8_e5m2_decode(p[t]) : (float)(int8_t)p[t];
        dst[t] = v * rs;
    }
}

/* Accumulation of the dequantized dot products: float64 (the oracle, the
 * default) or float32 in K order (BASELINE's CPU-baseline semantics, used
 * only to time that baseline).  Process-wide; set before a call. */
static int g_accum_f32 = 0;

void orc_set_accum_f32(int on) { g_accum_f32 = on != 0; }

static void *rowjob_run(void *arg)
{
    rowjob_t *j = (rowjob_t *)arg;
    float *w = (float *)malloc(sizeof(float) * (size_t)j->k);
    const int f32 = g_accum_f32;
    for (int r = j->r0; r < j->r1; r++) {
        deq_row_fmt(j->fmt, j->q, j->s, r, j->k, w);
        for (int t = 0; t < j->n_tok; t++) {
            const float *a = j->act + (size_t)t * j->k;
            if (f32) {
                float acc = 0.0f;
                for (int i = 0; i < j->k; i++) acc += a[i] * w[i];
                j->out[(size_t)t * j->n_rows + r] = acc;
            } else {
                double acc = 0.0;
                for (int i = 0; i < j->k; i++) acc += (double)a[i] * (double)w[i];
                j->out[(size_t)t * j->n_rows + r] = (float)acc;
            }
        }
    }
    free(w);
    return NULL;
}

/* out[t][r] = sum_i act[t][i] * W[r][i] for every weight row r. */
static void rows_gemm(int fmt, const uint8_t *q, const void *s, int n_rows, int k,
                      const float *act, int n_tok, float *out, int threads)
{
    if (threads < 1) threads = 1;
    if (threads > 256) threads = 256;
    pthread_t th[256];
    rowjob_t jobs[256];
    int per = (n_rows + threads - 1) / threads;
    int started = 0;
    for (int t = 0; t < threads; t++) {
        rowjob_t *j = &jobs[t];
        j->fmt = fmt; j->q = q; j->s = s; j->n_rows = n_rows; j->k = k;
        j->act = act; j->n_tok = n_tok; j->out = out;
        j->r0 = t * per; j->r1 = (t + 1) * per > n_rows ? n_rows : (t + 1) * per;
        if (j->r0 >= j->r1) break;
        if (threads == 1) { rowjob_run(j); started = 0; break; }
        pthread_create(&th[t], NULL, rowjob_run, j);
        started++;
    }
    for (int t = 0; t < started; t++) pthread_join(th[t], NULL);
}

static void requant_mxfp4_rows(float *v, int rows, int k)
{
    uint8_t *p = (uint8_t *)malloc((size_t)k / 2);
    uint8_t *s = (uint8_t *)malloc((size_t)k / 32);
    for (int r = 0; r < rows; r++) {
        orc_mxfp4_quantize_f32(v + (size_t)r * k, 1, k, p, s);
        deq_row(p, s, 0, k, v + (size_t)r * k);
    }
    free(p);
    free(s);
}

/* Full MXFP4 MLP down(silu(gate(x)) * up(x)) (MS:607; composition as in
 * encodeMXFP4FusedMLP MS:2033-2135 and encodeMXFP4DequantMLP MS:2426-2538),
 * with BASELINE's dequantize-then-FP32-accumulate semantics (modes 0/1) or
 * the reference's fused-row epilogue (mode 2). */
void orc_mlp_mxfp4(int mode, int tokens, int hidden, int inter, const uint16_t *x,
                   const uint8_t *wg, const uint8_t *sg, const uint8_t *wu, const uint8_t *su,
                   const uint8_t *wd, const uint8_t *sd, const int *rows_sel, int n_sel,
                   void *out, int threads)
{
    if (!rows_sel) n_sel = tokens;
    float *xa = (float *)malloc(sizeof(float) * (size_t)n_sel * hidden);
    float *g = (float *)malloc(sizeof(float) * (size_t)n_sel * inter);
    float *u = (float *)malloc(sizeof(float) * (size_t)n_sel * inter);
    float *mid = (float *)malloc(sizeof(float) * (size_t)n_sel * inter);
    float *o = (float *)malloc(sizeof(float) * (size_t)n_sel * hidden);
    for (int t = 0; t < n_sel; t++) {
        int src = rows_sel ? rows_sel[t] : t;
        for (int i = 0; i < hidden; i++)
            xa[(size_t)t * hidden + i] = orc_f16_to_f32(x[(size_t)src * hidden + i]);
    }
    if (mode == 1) requant_mxfp4_rows(xa, n_sel, hidden);
    rows_gemm(0, wg, sg, inter, hidden, xa, n_sel, g, threads);
    rows_gemm(0, wu, su, inter, hidden, xa, n_sel, u, threads);
    size_t cnt = (size_t)n_sel * inter;
    if (mode == 2) {
        uint16_t *mh = (uint16_t *)malloc(sizeof(uint16_t) * cnt);
        orc_swiglu_half(g, u, cnt, mh);
        for (size_t i = 0; i < cnt; i++) mid[i] = orc_f16_to_f32(mh[i]);
        free(mh);
    } else {
        orc_swiglu_float(g, u, cnt, mid);
    }
    if (mode == 1) requant_mxfp4_rows(mid, n_sel, inter);
    rows_gemm(0, wd, sd, hidden, inter, mid, n_sel, o, threads);
    size_t ocnt = (size_t)n_sel * hidden;
    if (mode == 2) memcpy(out, o, sizeof(float) * ocnt);
    else for (size_t i = 0; i < ocnt; i++) ((uint16_t *)out)[i] = orc_f32_to_f16(o[i]);
    free(xa); free(g); free(u); free(mid); free(o);
}

/* ------------------------------------------------------------------------ */
/* Weight-format quantizers.  The reference's
 * format rows are unscaled (MP:50-125); BASELINE adds the scales below.
 * Division (not reciprocal multiply) in f32, so the GPU can match bit for
 * bit. */
void orc_quant_rowwise(int fmt, const float *w, int rows, int k, uint8_t *q, float *row_scale)
{
    float qmax = fmt == 1 ? 448.0f : fmt == 2 ? 57344.0f : 127.0f;
    for (int r = 0; r < rows; r++) {
        const float *src = w + (size_t)r * k;
        float amax = 0.0f;
        for (int i = 0; i < k; i++) { float a = fabsf(src[i]); if (a > amax) amax = a; }
        float sc = amax > 0.0f ? amax / qmax : 1.0f;
        row_scale[r] = sc;
        for (int i = 0; i < k; i++) {
            float v = src[i] / sc;
            uint8_t c;
            if (fmt == 1) c = orc_fp8_e4m3_encode(v);
            else if (fmt == 2) c = orc_fp8_e5m2_encode(v);
            else {
                float rv = rintf(v);
                rv = rv > 127.0f ? 127.0f : (rv < -127.0f ? -127.0f : rv);
                c = (uint8_t)(int8_t)rv;
            }
            q[(size_t)r * k + i] = c;
        }
    }
}

void orc_quant_int4_g32(const float *w, int rows, int k, uint8_t *q, uint16_t *scale_f16)
{
    for (int r = 0; r < rows; r++)
        for (int b = 0; b < k / 32; b++) {
            const float *src = w + (size_t)r * k + b * 32;
            float amax = 0.0f;
            for (int i = 0; i < 32; i++) { float a = fabsf(src[i]); if (a > amax) amax = a; }
            uint16_t sh = amax > 0.0f ? orc_f32_to_f16(amax / 7.0f) : (uint16_t)0x3c00u;
            float s = orc_f16_to_f32(sh);
            if (s == 0.0f) { sh = 0x3c00u; s = 1.0f; }
            scale_f16[(size_t)r * (k / 32) + b] = sh;
            for (int i = 0; i < 32; i += 2) {
                int c[2];
                for (int h = 0; h < 2; h++) {
                    float rv = rintf(src[i + h] / s);
                    rv = rv > 7.0f ? 7.0f : (rv < -8.0f ? -8.0f : rv);
                    c[h] = ((int)rv) & 15;
                }
                q[(size_t)r * (k / 2) + (b * 32 + i) / 2] = (uint8_t)(c[0] | (c[1] << 4));
            }
        }
}

void orc_quant_int8_per_token(const float *x, int tokens, int k, int8_t *q, float *scale)
{
    orc_quant_rowwise(3, x, tokens, k, (uint8_t *)q, scale);
}

/* W8A8 rows: out[t][r] = (sum_i qx[t][i] * qw[r][i]) * sx[t] * sw[r], the
 * int32-accumulate row of MP:61-70 with per-token/per-row scales.  Exact
 * integer sums, so the split of the rows over threads changes nothing. */
typedef struct {
    const int8_t *qx; const float *sx; int n_tok;
    const uint8_t *qw; const float *sw; int n_rows, k;
    float *out;
    int r0, r1;
} w8a8job_t;

static void *w8a8_run(void *arg)
{
    const w8a8job_t *j = (const w8a8job_t *)arg;
    for (int r = j->r0; r < j->r1; r++) {
        const int8_t *wr = (const int8_t *)j->qw + (size_t)r * j->k;
        for (int t = 0; t < j->n_tok; t++) {
            const int8_t *xr = j->qx + (size_t)t * j->k;
            int64_t acc = 0;
            for (int i = 0; i < j->k; i++) acc += (int32_t)xr[i] * (int32_t)wr[i];
            j->out[(size_t)t * j->n_rows + r] = (float)acc * j->sx[t] * j->sw[r];
        }
    }
    return NULL;
}

static void w8a8_gemm(const int8_t *qx, const float *sx, int n_tok, const uint8_t *qw,
                      const float *sw, int n_rows, int k, float *out, int threads)
{
    if (threads < 1) threads = 1;
    if (threads > 256) threads = 256;
    pthread_t th[256];
    w8a8job_t jobs[256];
    int per = (n_rows + threads - 1) / threads, started = 0;
    for (int t = 0; t < threads; t++) {
        w8a8job_t *j = &jobs[t];
        j->qx = qx; j->sx = sx; j->n_tok = n_tok; j->qw = qw; j->sw = sw; j->n_rows = n_rows; j->k = k;
        j->out = out;
        j->r0 = t * per; j->r1 = (t + 1) * per > n_rows ? n_rows : (t + 1) * per;
        if (j->r0 >= j->r1) break;
        if (threads == 1) { w8a8_run(j); break; }
        pthread_create(&th[t], NULL, w8a8_run, j);
        started++;
    }
    for (int t = 0; t < started; t++) pthread_join(th[t], NULL);
}

void orc_mlp_format(int fmt, int tokens, int hidden, int inter, const uint16_t *x,
                    const uint8_t *qg, const void *sg, const uint8_t *qu, const void *su,
                    const uint8_t *qd, const void *sd, const int *rows_sel, int n_sel,
                    uint16_t *out, int threads)
{
    if (!rows_sel) n_sel = tokens;
    float *xa = (float *)malloc(sizeof(float) * (size_t)n_sel * hidden);
    float *g = (float *)malloc(sizeof(float) * (size_t)n_sel * inter);
    float *u = (float *)malloc(sizeof(float) * (size_t)n_sel * inter);
    float *mid = (float *)malloc(sizeof(float) * (size_t)n_sel * inter);
    float *o = (float *)malloc(sizeof(float) * (size_t)n_sel * hidden);
    for (int t = 0; t < n_sel; t++) {
        int src = rows_sel ? rows_sel[t] : t;
        for (int i = 0; i < hidden; i++)
            xa[(size_t)t * hidden + i] = orc_f16_to_f32(x[(size_t)src * hidden + i]);
    }
    size_t cnt = (size_t)n_sel * inter;
    if (fmt == 5) {
        int8_t *qx = (int8_t *)malloc((size_t)n_sel * (hidden > inter ? hidden : inter));
        float *sx = (float *)malloc(sizeof(float) * (size_t)n_sel);
        orc_quant_int8_per_token(xa, n_sel, hidden, qx, sx);
        w8a8_gemm(qx, sx, n_sel, qg, (const float *)sg, inter, hidden, g, threads);
        w8a8_gemm(qx, sx, n_sel, qu, (const float *)su, inter, hidden, u, threads);
        orc_swiglu_float(g, u, cnt, mid);
        orc_quant_int8_per_token(mid, n_sel, inter, qx, sx);
        w8a8_gemm(qx, sx, n_sel, qd, (const float *)sd, hidden, inter, o, threads);
        free(qx);
        free(sx);
    } else {
        rows_gemm(fmt, qg, sg, inter, hidden, xa, n_sel, g, threads);
        rows_gemm(fmt, qu, su, inter, hidden, xa, n_sel, u, threads);
        orc_swiglu_float(g, u, cnt, mid);
        rows_gemm(fmt, qd, sd, hidden, inter, mid, n_sel, o, threads);
    }
    for (size_t i = 0; i < (size_t)n_sel * hidden; i++) out[i] = orc_f32_to_f16(o[i]);
    free(xa); free(g); free(u); free(mid); free(o);
}

/* ------------------------------------------------------------------------ */
/* Reference LCG generators (MS:2785-2842):
 * state = state * 1664525 + 1013904223 + index (wrapping UInt32), applied
 * before each use. */
void orc_lcg_bytes(uint32_t seed, size_t count, uint8_t *out)
{
    uint32_t s = seed;
    for (size_t i = 0; i < count; i++) {
        s = s * 1664525u + 1013904223u + (uint32_t)i;
        out[i] = (uint8_t)(s >> 16);
    }
}

void orc_lcg_pattern(uint32_t seed, size_t count, const uint8_t *pattern, int pattern_count,
                     uint8_t *out)
{
    uint32_t s = seed;
    for (size_t i = 0; i < count; i++) {
        s = s * 1664525u + 1013904223u + (uint32_t)i;
        out[i] = pattern[s % (uint32_t)pattern_count];
    }
}

void orc_lcg_half(uint32_t seed, size_t count, float scale, uint16_t *out)
{
    uint32_t s = seed;
    for (size_t i = 0; i < count; i++) {
        s = s * 1664525u + 1013904223u + (uint32_t)i;
        int nib = (int)((s >> 28) & 15u);
        out[i] = orc_f32_to_f16((float)((nib ^ 8) - 8) * scale);
    }
}

void orc_lcg_int8(uint32_t seed, size_t count, int8_t *out)
{
    uint32_t s = seed;
    for (size_t i = 0; i < count; i++) {
        s = s * 1664525u + 1013904223u + (uint32_t)i;
        int nib = (int)((s >> 28) & 15u);
        out[i] = (int8_t)((nib ^ 8) - 8);
    }
}

/* Checksums (MS:2844-2884): sum of every (count/32)-th element. */
double orc_checksum_f32(const float *p, size_t count, int *samples)
{
    size_t step = count / 32 > 1 ? count / 32 : 1;
    double sum = 0.0;
    int n = 0;
    for (size_t i = 0; i < count; i += step) { sum += (double)p[i]; n++; }
    if (samples) *samples = n;
    return sum;
}

int64_t orc_checksum_i32(const int32_t *p, size_t count, int *samples)
{
    size_t step = count / 32 > 1 ? count / 32 : 1;
    int64_t sum = 0;
    int n = 0;
    for (size_t i = 0; i < count; i += step) { sum += p[i]; n++; }
    if (samples) *samples = n;
    return sum;
}

uint64_t orc_checksum_f16raw(const uint16_t *p, size_t count, int *samples)
{
    size_t step = count / 32 > 1 ? count / 32 : 1;
    uint64_t sum = 0;
    int n = 0;
    for (size_t i = 0; i < count; i += step) { sum += p[i]; n++; }
    if (samples) *samples = n;
    return sum;
}
