/*
 * mxfp4hip.h - C ABI of libmxfp4hip, the MI355X (gfx950) MXFP4 MLP library.
 *
 * Drop-in boundary for the reference's MXFP4 MLP hot path
 * (Anemll/MPP-4.1-FP4-FP8-block).  The reference binds its kernels through
 * Metal: positional buffers 0..6 (MXFP4Kernels.metal:108-115, 264-286),
 * encoded by main.swift helpers (encodeMXFP4MatmulDispatch main.swift:2137,
 * encodeMXFP4FusedMLP :2033, encodeMXFP4DequantMLP :2426, encodeMPPMLP
 * :2636).  Each entry point below names the reference interface it replaces.
 *
 * Conventions
 *   - Plain C types only; device pointers come from mx_alloc (or any HIP
 *     allocation on the context's device).  Host pointers are marked "host".
 *   - Every function returns an mx_status; mx_last_error(ctx) holds the
 *     message (mirrors ProbeError, main.swift:5-38).  No exceptions cross
 *     the ABI.
 *   - One context = one device + one HIP stream.  Launch functions are
 *     asynchronous in stream order; *_roundtrip, mx_download, mx_sync and
 *     the benchmark entry points are synchronous.  A context is not
 *     thread-safe; use one per host thread.
 *   - Layouts are the reference's (GUIDE:43-55): activations [T][K]
 *     row-major; weights [N][K] with K contiguous; MXFP4 data [N][K/2]
 *     (low nibble = even k), E8M0 scales [N][K/32].
 */
#ifndef MXFP4HIP_H
#define MXFP4HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes: ProbeError cases (main.swift:5-38). */
typedef enum {
  MX_OK = 0,
  MX_EINVAL = 1,    /* invalidArgument                         */
  MX_ENODEV = 2,    /* missingDevice                           */
  MX_ENOKERNEL = 3, /* missingFunction / missingShaderResource */
  MX_ENOMEM = 4,    /* missingBuffer                           */
  MX_EGPU = 5       /* gpuExecutionFailed / missingCommand*    */
} mx_status;

/* Element types. */
enum { MX_DTYPE_F32 = 0, MX_DTYPE_F16 = 1, MX_DTYPE_I8 = 2, MX_DTYPE_I32 = 3, MX_DTYPE_U8 = 4 };

/* Packed numeric formats of the roundtrip probe (PackedNumericKernels.metal:35-96). */
enum { MX_FMT_FP4_E2M1 = 0, MX_FMT_FP8_E4M3 = 1, MX_FMT_FP8_E5M2 = 2 };

/* MLP variants (rows of runMLPBenchmark, main.swift:1043-1243). */
enum {
  /* fused: FP4 weights dequantized in registers by v_cvt_scalef32_pk_f16_fp4
   * feeding fp16 MFMA, gate+up+SwiGLU in one kernel, mid f16, then down;
   * counterpart of the native scale-plane rows (MXFP4Kernels.metal:138-173). */
  MX_MLP_FUSED = 0,
  /* dequant: 3 x dequant-to-half, h_h_f gate/up, swiglu_float, down
   * (encodeMXFP4DequantMLP main.swift:2426-2538).  The down GEMM takes the
   * f32 mid as two f16 terms (hi + lo) into the fp16 MFMA, so f32 x half
   * holds to ~2^-22 of each value as in the reference's f_h_f. */
  MX_MLP_DEQUANT = 1,
  /* W4A4: x and mid quantized to MXFP4 along K, FP4 x FP4 scaled MFMA
   * (v_mfma_scale_f32_32x32x64_f8f6f4), fp16 out. */
  MX_MLP_W4A4 = 2,
  /* reference fused-row epilogue: swiglu_half (x1/16, clamp +-20, mid half),
   * f32 out (encodeMXFP4FusedMLP main.swift:2033-2135 + MPPMLPKernels.metal:204-220);
   * reproduces the reference checksum 403573 (README.md:292-294). */
  MX_MLP_REFROW = 3,
  /* scaled: the native scale-plane rows (MXFP4Kernels.metal:138-173) on the
   * CDNA4 scaled MFMA: x and mid are split into two FP8 E4M3 terms with an
   * E8M0 pair per 64 K (relative error <= 2^-8 per value), and
   * v_mfma_scale_f32_32x32x64_f8f6f4 takes the FP4 codes and their E8M0
   * bytes directly, two MFMAs per block.  One more launch (the split of x).
   * The MFMA reads E8M0 byte 255 as NaN; the outputs that turns NaN (and
   * those of non-finite activations) are recomputed in the epilogues with
   * the reference's +inf scale, so NaN and +-inf land where the reference's
   * do.  (A non-finite mid is carried as its class: NaN, +-inf, zero or the
   * sign of a finite value.) */
  MX_MLP_SCALED = 4
};

/* Weight-format rows (MPP/NAX rows main.swift:945-1042, 1247-1413;
 * BASELINE configs[3] adds the scales). */
enum {
  MX_WFMT_FP8_E4M3 = 1, /* [N][K] E4M3 + f32 row scale [N] (amax/448)   */
  MX_WFMT_FP8_E5M2 = 2, /* [N][K] E5M2 + f32 row scale [N] (amax/57344) */
  MX_WFMT_INT8 = 3,     /* [N][K] int8 + f32 row scale [N] (amax/127)   */
  MX_WFMT_INT4 = 4,     /* [N][K/2] int4 (low nibble = even k) + f16 scale [N][K/32] (amax/7) */
  MX_WFMT_W8A8 = 5,     /* int8 weights as MX_WFMT_INT8, int8 activations per token, i32 accumulate */
  /* The FP8 rows on the FP8 matrix cores: weights exactly as MX_WFMT_FP8_E4M3 /
   * MX_WFMT_FP8_E5M2; x and mid are split into two FP8 E4M3 terms with an
   * E8M0 pair per 64 K (as MX_MLP_SCALED: relative error <= 2^-8 per value)
   * and v_mfma_scale_f32_32x32x64_f8f6f4 multiplies them by the FP8 weight
   * codes with no widening; the f32 row scale is applied to the sums.  One
   * more launch (the split of x).  Hidden and intermediate % 64. */
  MX_WFMT_FP8_E4M3_F8X2 = 6,
  MX_WFMT_FP8_E5M2_F8X2 = 7
};

/* MLPConfig (main.swift:62-66, MPPMLPKernels.metal:8-12). */
typedef struct {
  uint32_t tokens;
  uint32_t hidden;
  uint32_t intermediate;
} mx_mlp_config;

/* One quantized weight matrix: data + scales (device pointers). */
typedef struct {
  const void* data;
  const void* scales;
} mx_qmatrix;

/* gate [I][H], up [I][H], down [H][I]. */
typedef struct {
  mx_qmatrix gate, up, down;
} mx_mlp_weights;

typedef struct mx_ctx mx_ctx;

/* ---- context (MTLCreateSystemDefaultDevice main.swift:91, makeQueue :193) */
int mx_create(int device, mx_ctx** out);
void mx_destroy(mx_ctx* ctx);
const char* mx_last_error(const mx_ctx* ctx);
/* Static message for a status code (usable without a context). */
const char* mx_status_string(int status);
/* Device name and compute-unit count ("Device: ..." main.swift:95). */
int mx_device_info(mx_ctx* ctx, char* name_out, size_t name_len, int* cu_count, int* clock_mhz);
/* Use the caller's HIP stream (hipStream_t as void*); NULL = context stream. */
int mx_set_stream(mx_ctx* ctx, void* stream);
void* mx_get_stream(mx_ctx* ctx);
int mx_sync(mx_ctx* ctx);
/* Device time of the work enqueued between the two calls on the context's
 * stream (HIP events; the counterpart of a command buffer's gpuStartTime /
 * gpuEndTime, main.swift:1761-1779).  mx_timer_stop waits for that work. */
int mx_timer_start(mx_ctx* ctx);
int mx_timer_stop(mx_ctx* ctx, double* seconds_out);

/* ---- device memory (device.makeBuffer, main.swift:219, 640-917) --------- */
int mx_alloc(mx_ctx* ctx, size_t bytes, void** dptr);
int mx_free(mx_ctx* ctx, void* dptr);
int mx_upload(mx_ctx* ctx, void* dst, const void* host_src, size_t bytes);
int mx_download(mx_ctx* ctx, void* host_dst, const void* src, size_t bytes);
int mx_memset(mx_ctx* ctx, void* dst, int value, size_t bytes);

/* ---- codecs --------------------------------------------------------------- */
/* Pack/unpack roundtrip of host vectors: replaces run(testCase:) +
 * fp4_e2m1_roundtrip / fp8_e4m3_roundtrip / fp8_e5m2_roundtrip
 * (main.swift:202-292, PackedNumericKernels.metal:35-96).  host_packed gets
 * n/2 (FP4) or n (FP8) bytes; host_out gets the n unpacked floats. */
int mx_roundtrip(mx_ctx* ctx, int fmt, const float* host_in, size_t n, uint8_t* host_packed,
                 float* host_out);
/* Bulk device pack / unpack with the same semantics. */
int mx_pack(mx_ctx* ctx, int fmt, const float* in, size_t n, uint8_t* packed);
int mx_unpack(mx_ctx* ctx, int fmt, const uint8_t* packed, size_t n, float* out);

/* MXFP4 block quantizer (no reference kernel: the
 * reference generates codes directly, main.swift:633-638).  src [rows][k]
 * f32 or f16; k % 32 == 0. */
int mx_mxfp4_quantize(mx_ctx* ctx, const void* src, int src_dtype, int rows, int k,
                      uint8_t* packed, uint8_t* scales);

/* Dequant to half: mxfp4_dequant_native_half / mxfp4_dequant_lut_half
 * (MXFP4Kernels.metal:509-564; ABI packed, scales, out, rows, depth). */
int mx_mxfp4_dequant_f16(mx_ctx* ctx, const uint8_t* packed, const uint8_t* scales, void* out,
                         int rows, int depth);

/* ---- matmuls -------------------------------------------------------------- */
/* C[m][n] = sum_k A[m][k] * fp4(B[n][k]) * 2^(S[n][k/32]-127):
 * mxfp4_native_sp_h_f_n64 / mxfp4_fused_h_f_n64 (MXFP4Kernels.metal:108-130,
 * 264-286; ABI a, b, c, m, n, k, scales).  a f16 or f32; c f32 or f16.
 * Any m, n >= 1 (the reference's tiles guard column < n,
 * MXFP4Kernels.metal:98); k % 32 == 0. */
int mx_mxfp4_matmul(mx_ctx* ctx, const void* a, int a_dtype, const uint8_t* b, void* c,
                    int c_dtype, int m, int n, int k, const uint8_t* scales);
/* C f32 = A * B^T with B f16 [n][k]: mpp_mlp_h_h_f_n128 (a f16) and
 * mpp_mlp_f_h_f_n128 (a f32, taken as two f16 terms hi + lo, so f32 x half
 * holds to ~2^-22 of each value) (MPPMLPKernels.metal:39-48, 164-173).
 * Any m, n >= 1; k % 32 == 0. */
int mx_gemm_f16(mx_ctx* ctx, const void* a, int a_dtype, const void* b, float* c, int m, int n,
                int k);
/* C i32 = A * B^T with A int8 [m][k], B int8 [n][k], exact i32 sums:
 * mpp_mlp_i8_i8_i32_n128 (MPPMLPKernels.metal:61-70), the W8A8 core.
 * n % 64 == 0, k % 128 == 0. */
int mx_gemm_i8(mx_ctx* ctx, const int8_t* a, const int8_t* b, int32_t* c, int m, int n, int k);
/* Typed probe GEMM: the accumulator-probe family accum_{h_h,h_fp4,fp4_fp4,
 * fp8_fp8}_{h,f} (AccumProbeKernels.metal:41-127) and the scalar benchmark
 * matmuls half_int4_matmul_half / int8_half_matmul_half /
 * int4_int8_matmul (PackedNumericKernels.metal:246-423); ABI a, b, c, m, n, k.
 * C[m][n] = sum_k A[m][k] * B[n][k], A [m][k] and B [n][k] K-contiguous in
 * format a_fmt / b_fmt (MX_PROBE_*: FP4 = E2M1 and INT4 = signed
 * ((b & 15) ^ 8) - 8, both two per byte, low nibble = even k, no scales;
 * FP8 = E4M3; I8 = int8); f32 accumulation (i32 for INT4 x INT4); C f32 or
 * f16 (c_dtype; f16 is one RNE rounding of the f32 sum, >= 65520 -> inf), i32
 * for INT4 x INT4.  Pairs: (F16, F16), (F16, FP4), (FP4, FP4), (FP8, FP8),
 * (F16, INT4), (I8, F16), (INT4, INT4).  Any k >= 1 (even with 4-bit
 * operands); n % 64 == 0; FP4 / FP8 A also needs m % 32 == 0. */
enum { MX_PROBE_F16 = 0, MX_PROBE_FP4 = 1, MX_PROBE_FP8 = 2, MX_PROBE_INT4 = 3, MX_PROBE_I8 = 4 };
int mx_accum_gemm(mx_ctx* ctx, int a_fmt, const void* a, int b_fmt, const void* b, void* c,
                  int c_dtype, int m, int n, int k);
/* SwiGLU over cfg->tokens x cfg->intermediate elements, in the Metal
 * kernels' buffer order gate, up, mid, MLPConfig (MPPMLPKernels.metal:186-257),
 * then the kernel choice: variant 0 mpp_mlp_swiglu_float (f32 -> f32),
 * 1 mpp_mlp_swiglu_half (f32 -> f16), 2 mpp_mlp_swiglu_half_from_half
 * (f16 -> f16), 3 mpp_mlp_swiglu_i8 (i32 -> i8). */
int mx_swiglu(mx_ctx* ctx, const void* gate, const void* up, void* mid, const mx_mlp_config* cfg,
              int variant);

/* ---- MLP ------------------------------------------------------------------ */
/* down(silu(gate(x)) * up(x)).  x f16 [T][H]; weights MXFP4; out f16 [T][H]
 * (f32 for MX_MLP_REFROW).  Validation as runMLPBenchmark (main.swift:592-597):
 * positive sizes, hidden and intermediate % 32 (the MXFP4 rows, :1043) for
 * FUSED, DEQUANT and REFROW; SCALED needs % 64 and W4A4 % 128.  The
 * reference's tokens % 64 rule (:946) is lifted.  Scratch memory is owned by
 * the context. */
int mx_mlp_forward(mx_ctx* ctx, int variant, const mx_mlp_config* cfg, const void* x,
                   const mx_mlp_weights* w, void* out);

/* Allocation-free forward.  No counterpart in the reference: for callers
 * that cannot allocate device memory (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc).  Same arguments, kernels
 * and results as mx_mlp_forward, but its scratch (mid activations, split-K
 * partials, re-quantized operands) lives in one static device array of
 * MX_NOALLOC_SCRATCH_BYTES per GPU, held until the process ends; it calls no
 * hipMalloc / hipFree.  Shapes needing more scratch fail with MX_EINVAL
 * (e.g. the decode and C0-C2 shapes fit, C4 W4A4 does not).  Every call on
 * one GPU shares that array: calls that overlap on one GPU (two contexts or
 * two streams at once) race; calls in one stream order are fine. */
#define MX_NOALLOC_SCRATCH_BYTES (32u << 20)
int mx_mlp_forward_noalloc(mx_ctx* ctx, int variant, const mx_mlp_config* cfg, const void* x,
                           const mx_mlp_weights* w, void* out);

/* Timed loop as runMXFP4FusedMLPBenchmarkVariant (main.swift:1953-2031):
 * `warmup` untimed iterations, then `iterations` back-to-back forwards on the
 * stream between two HIP events.  Iteration i uses weight set i % n_sets
 * (MoE-style rotation; defeats the 256 MB last-level cache).  use_graph != 0
 * captures the `iterations` forwards into one HIP graph and times one replay
 * (the reference likewise encodes all iterations into one command buffer,
 * main.swift:2062-2117); 0 launches them one by one.
 * seconds_out: total timed seconds.  kernel_us_out (optional, length
 * >= 8): average device time per launch of each kernel of the forward, in
 * launch order, each from a timed pass of that kernel alone over the same
 * rotation (max(iterations, n_sets) launches, so every set is streamed);
 * n_kernels_out: how many were written. */
int mx_mlp_benchmark(mx_ctx* ctx, int variant, const mx_mlp_config* cfg, const void* x,
                     const mx_mlp_weights* sets, int n_sets, void* out, int warmup,
                     int iterations, int use_graph, double* seconds_out, double* kernel_us_out,
                     int* n_kernels_out);
/* Name of kernel `index` of the forward that `variant` runs at shape `cfg`
 * (for the per-kernel times); NULL past the last kernel. */
const char* mx_mlp_kernel_name(int variant, const mx_mlp_config* cfg, int index);

/* ---- MoE grouped experts ------------------------------------------------------ */
/* No counterpart in the reference (a "next" item of its MXFP4 regime: MoE
 * experts whose weights are decoded inside the loop).  The MXFP4 MLP of
 * n_experts experts over one token batch in two grouped launches (gate/up +
 * SwiGLU for every expert, then down for every expert).
 *   x     f16 [tokens][hidden], rows grouped by expert: expert e owns the
 *         counts[e] rows after those of experts 0..e-1 (counts: host array
 *         of n_experts entries summing to cfg->tokens; 0 is allowed).
 *   w     experts stacked in the MXFP4 layout, pointers at expert 0: gate and
 *         up data [E][I][H/2] + scales [E][I][H/32], down data [E][H][I/2] +
 *         scales [E][H][I/32].
 *   out   f16 [tokens][hidden], rows in the same order as x.
 * 1 <= n_experts <= 256.  Experts with at most 16 tokens each take the decode
 * GEMV (hidden, intermediate % 128); otherwise % 64. */
int mx_moe_forward(mx_ctx* ctx, const mx_mlp_config* cfg, int n_experts, const int* counts,
                   const void* x, const mx_mlp_weights* w, void* out);
/* `iterations` MoE forwards between two HIP events (rotating weight sets), as
 * mx_mlp_benchmark. */
int mx_moe_benchmark(mx_ctx* ctx, const mx_mlp_config* cfg, int n_experts, const int* counts,
                     const void* x, const mx_mlp_weights* sets, int n_sets, void* out, int warmup,
                     int iterations, int use_graph, double* seconds_out);

/* ---- on-disk MXFP4 weights (safetensors) ------------------------------------- */
/* Locate tensor `name` in a safetensors file (host only: no context, no
 * device).  dtype string (e.g. "U8"), shape (first max_dims entries), number
 * of dimensions, file offset and byte size of its data. */
int mx_safetensors_find(const char* path, const char* name, char* dtype_out, size_t dtype_len,
                        long long* shape_out, int max_dims, int* ndim_out,
                        unsigned long long* offset_out, unsigned long long* nbytes_out);
/* Load MXFP4 weights onto the device with no repack: blocks U8
 * [..., n, k/32, 16] (or [..., n, k/2]) and scales U8 [..., n, k/32] are the
 * library's layout (docs/MXFP4-MPP41-GUIDE.md:43-55); leading dimensions are
 * experts, giving the stacked form mx_moe_forward takes.  out->data and
 * out->scales are new device buffers (release with mx_free).  count_out =
 * product of the leading dimensions (1 without), n_out rows, k_out = 32 x
 * the scale dimension. */
int mx_load_mxfp4(mx_ctx* ctx, const char* path, const char* blocks_name, const char* scales_name,
                  mx_qmatrix* out, int* count_out, int* n_out, int* k_out);

/* ---- weight-format rows (config 3) ------------------------------------------ */
/* Quantize f32 weights [rows][k] into format `wfmt` (scales per the enum;
 * the _F8X2 codes quantize as their FP8 format). */
int mx_fmt_quantize(mx_ctx* ctx, int wfmt, const float* w, int rows, int k, void* q,
                    void* scales);
/* MLP with format weights: mpp_mlp_h_fp8e4m3_f_n128 / _h_fp8e5m2_f_n128 /
 * h_i8_f / h_i4_f / i8_i8_i32 rows (MPPMLPKernels.metal:50-125) with scales.
 * hidden and intermediate % 32; the _F8X2 rows % 64; W8A8 % 128. */
int mx_fmt_mlp_forward(mx_ctx* ctx, int wfmt, const mx_mlp_config* cfg, const void* x,
                       const mx_mlp_weights* w, void* out);
/* Timed loop of the format rows, as mx_mlp_benchmark (kernel_us_out and
 * n_kernels_out optional, per kernel of the forward in launch order). */
int mx_fmt_mlp_benchmark(mx_ctx* ctx, int wfmt, const mx_mlp_config* cfg, const void* x,
                         const mx_mlp_weights* sets, int n_sets, void* out, int warmup,
                         int iterations, int use_graph, double* seconds_out, double* kernel_us_out,
                         int* n_kernels_out);
/* Name of kernel `index` of the format forward at shape `cfg`; NULL past the
 * last kernel. */
const char* mx_fmt_mlp_kernel_name(int wfmt, const mx_mlp_config* cfg, int index);

/* ---- synthetic data (main.swift:2785-2842) ---------------------------------- */
/* Seeded N(mean, std) on the device (f32 or f16). */
int mx_fill_normal(mx_ctx* ctx, void* dst, int dtype, size_t n, uint64_t seed, float mean,
                   float stddev);
/* Reference LCG generators, bit-exact (host memory; no context needed):
 * state = state*1664525 + 1013904223 + index, applied before each use. */
void mx_lcg_bytes(uint32_t seed, size_t count, uint8_t* host_out);          /* makePackedMatrixBytes :2785 */
void mx_lcg_pattern(uint32_t seed, size_t count, const uint8_t* pattern, int pattern_count,
                    uint8_t* host_out);                                     /* makeBytePatternValues :2812 */
void mx_lcg_half(uint32_t seed, size_t count, float scale, uint16_t* host_out); /* makeHalfMatrixValues :2822 */
void mx_lcg_int8(uint32_t seed, size_t count, int8_t* host_out);            /* makeInt8MatrixValues :2834 */
/* Checksums (sampleFloatChecksum / sampleIntChecksum / sampleHalfRawChecksum,
 * main.swift:2844-2884): sum of every max(1, count/32)-th element. */
double mx_checksum_f32(const float* host_p, size_t count, int* samples);
int64_t mx_checksum_i32(const int32_t* host_p, size_t count, int* samples);
uint64_t mx_checksum_f16raw(const uint16_t* host_p, size_t count, int* samples);

#ifdef __cplusplus
}
#endif
#endif /* MXFP4HIP_H */
