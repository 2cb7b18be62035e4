// mx_device.h - gfx950 device helpers shared by the libmxfp4hip kernels.
//
// MXFP4 layout (reference GUIDE:43-55, MXFP4Kernels.metal:3-4, 98, 345):
//   data   [N][K/2] bytes, two E2M1 codes per byte, low nibble = even k
//   scales [N][K/32] E8M0 bytes, value 2^(byte-127)
//
// MFMA operand layouts used below (each kernel's GPU parity tests against
// the oracle would fail on a wrong lane layout):
//   v_mfma_scale_f32_32x32x64_f8f6f4 (fp4): lane l holds row l%32,
//       k = 32*(l/32) + j, j = nibble j of 4 dwords (low nibble first);
//       the lane's scale byte applies to exactly that (row, 32-k block).
//   v_mfma_f32_32x32x16_f16: lane l holds row l%32, k = 8*(l/32) + j.
//   v_mfma_f32_16x16x32_f16: lane l holds row l%16, k = 8*(l/16) + j.
//   v_mfma_i32_32x32x32_i8:  lane l holds row l%32, k = 16*(l/32) + j.
//   32x32 accumulators: lane l, reg v -> row (v/4)*8 + (l/32)*4 + v%4,
//       column l%32.   16x16: row (l/16)*4 + v, column l%16.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mx {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v2i __attribute__((ext_vector_type(2)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v2f __attribute__((ext_vector_type(2)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 v4h __attribute__((ext_vector_type(4)));
typedef _Float16 v2h __attribute__((ext_vector_type(2)));
typedef short v2s __attribute__((ext_vector_type(2)));

constexpr int kBlock = 32;  // MXFP4 block along K (MXFP4Kernels.metal:24)

// E8M0 byte -> f32 with the reference's semantics: bits << 23
// (MXFP4Kernels.metal:26-29): byte 0 -> 0.0, byte 255 -> +inf.
__device__ __forceinline__ float e8m0_to_float(uint32_t b) {
  return __builtin_bit_cast(float, b << 23);
}

// Scale operand for the gfx950 cvt_scalef32 instructions: the E8M0 byte in
// the exponent field of an f32 (the hardware reads only that field).
__device__ __forceinline__ float e8m0_as_cvt_scale(uint32_t b) {
  return __builtin_bit_cast(float, (b & 255u) << 23);
}

__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
  _Float16 h = (_Float16)f;  // v_cvt_f16_f32: RNE
  return __builtin_bit_cast(uint16_t, h);
}

__device__ __forceinline__ float f16_bits_to_f32(uint16_t h) {
  return (float)__builtin_bit_cast(_Float16, h);
}

// silu(g) = g / (1 + e^-g) for the f16 and F8X2 mids of the fused rows, the
// W4A4 mid and the decode GEMV: g times the hardware reciprocal (v_rcp_f32)
// of 1 + 2^(-g log2 e) (v_exp_f32), about 1 ulp of f32 from the IEEE
// quotient, below the f16 / FP8 / FP4 rounding of the mid, and with the same
// special values (-inf -> NaN, large negative g -> -0, +inf -> +inf, NaN ->
// NaN).  Five VALU instructions against about twenty for the IEEE form,
// which cost ~1 us of a gate/up GEMM's epilogue at one wave per SIMD.  The
// f32 mid of W8A8 (re-quantized to int8, bit-exact against the oracle) and
// the reference-row SwiGLU (swiglu_half) keep the IEEE form.
__device__ __forceinline__ float silu(float g) { return g * __builtin_amdgcn_rcpf(1.0f + __expf(-g)); }

// Two FP4 codes (byte `sel` of `src`) -> two halves, each fp4 * 2^(scale-127).
template <int SEL>
__device__ __forceinline__ v2h cvt_fp4x2_f16(uint32_t src, float scale) {
  return __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(src, scale, SEL);
}

// 8 FP4 codes in a dword -> 8 halves (one 32x32x16 / 16x16x32 f16 operand).
__device__ __forceinline__ v8h fp4x8_to_f16x8(uint32_t src, float scale) {
  v2h a = cvt_fp4x2_f16<0>(src, scale);
  v2h b = cvt_fp4x2_f16<1>(src, scale);
  v2h c = cvt_fp4x2_f16<2>(src, scale);
  v2h d = cvt_fp4x2_f16<3>(src, scale);
  v8h r;
  r[0] = a[0]; r[1] = a[1]; r[2] = b[0]; r[3] = b[1];
  r[4] = c[0]; r[5] = c[1]; r[6] = d[0]; r[7] = d[1];
  return r;
}

// 8 FP4 codes times an infinite scale, as halves: +-0 codes give NaN
// (0 * inf), every other code +-inf.
__device__ __forceinline__ v8h fp4x8_times_inf_f16(uint32_t src) {
  v8h h;
#pragma unroll
  for (int e = 0; e < 8; e++) {
    const uint32_t nib = (src >> (4 * e)) & 15u;
    const uint32_t bits = (nib & 7u) ? ((nib & 8u) ? 0xfc00u : 0x7c00u) : 0x7e00u;
    h[e] = __builtin_bit_cast(_Float16, (uint16_t)bits);
  }
  return h;
}

// Dequantize 8 FP4 codes with E8M0 byte `sb` using the reference's scale
// semantics (bits << 23).  Bytes 0..254 take the single-instruction path
// (the hardware reads byte 0 as 2^-127, which gives the same halves as the
// reference's 0.0 because 6 * 2^-127 underflows f16).  Byte 255 is +inf in
// the reference but NaN to the hardware, so it is formed from the codes.
__device__ __forceinline__ v8h fp4x8_dequant_f16(uint32_t src, uint32_t sb) {
  if (__builtin_expect(sb != 255u, 1)) return fp4x8_to_f16x8(src, e8m0_as_cvt_scale(sb));
  return fp4x8_times_inf_f16(src);
}

// Block amax -> E8M0 scale byte (BASELINE quantizer:
// 2^(floor(log2(amax)) - 2)).  `amax_bits` = max of |x| bit patterns.
// Non-finite -> 255, zero -> 127, exponents below -127 clamp to byte 0.
__device__ __forceinline__ uint32_t mxfp4_scale_byte(uint32_t amax_bits) {
  if (amax_bits >= 0x7f800000u) return 255u;
  if (amax_bits == 0u) return 127u;
  int fl;
  uint32_t e = amax_bits >> 23;
  if (e == 0) fl = (31 - __builtin_clz(amax_bits)) - 149;
  else fl = (int)e - 127;
  int s = fl - 2;
  if (s < -127) s = -127;
  return (uint32_t)(s + 127);
}

// One E4M3 byte -> f32 (0x7f / 0xff NaN, no infinities).
__device__ __forceinline__ float e4m3_to_f32(uint32_t byte) {
  return __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(byte & 255u, 1.0f, false)[0];
}

// ---------------------------------------------------------------------------
// Exact (reference-semantics) recomputation of single outputs whose tiled
// result is NaN.  The scaled MFMA reads E8M0 byte 255 as NaN where the
// reference decodes it as +inf (MXFP4Kernels.metal:26-29, bits << 23), and
// its F8X2 activations cannot hold an infinity.  These scalar loops dequantize
// like the reference (w = FP4 value * 2^(s - 127), byte 255 -> +inf, byte 0
// -> 0) and accumulate in f32 in K order, so IEEE arithmetic reproduces the
// reference's non-finite results: x * inf = +-inf, 0 * inf = NaN, inf - inf =
// NaN.  Finite parts are as accurate as any f32 dot product.

// sum_k x[k] * W[k] for one f16 activation row and one MXFP4 weight row.
__device__ inline float ref_dot_f16_mxfp4(const uint16_t* x, const uint8_t* w, const uint8_t* s, int K) {
  float acc = 0.0f;
  for (int kb = 0; kb < K / 32; kb++) {
    const float sc = e8m0_to_float(s[kb]);
    for (int j = 0; j < 16; j++) {
      const v2f c = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w[kb * 16 + j], 1.0f, 0);
      acc += f16_bits_to_f32(x[kb * 32 + 2 * j]) * (c[0] * sc);
      acc += f16_bits_to_f32(x[kb * 32 + 2 * j + 1]) * (c[1] * sc);
    }
  }
  return acc;
}

// Value k of row `row` of an F8X2 matrix (layout in mx_internal.h; K % 64 ==
// 0, M rows): t1 s1 + t2 s2, or for a group with scale byte 255 the class its
// first term carries (NaN, +-inf, 0, or +-1 for a finite non-zero value).
__device__ inline float f8x2_ref_value(const uint8_t* data, const uint32_t* e8, int M, int K, int row, int k) {
  const int gi = k >> 6, kk = k & 63, q = kk >> 4;
  const int pos = (kk & 15) + 16 * (q == 1 ? 2 : q == 2 ? 1 : q);
  const uint8_t* grp = data + ((size_t)row * (K / 64) + gi) * 128;
  const uint32_t e = e8[(size_t)gi * M + row], b1 = e & 255u, b2 = (e >> 8) & 255u;
  const uint32_t t1 = grp[pos], t2 = grp[64 + pos];
  if (b1 == 255u) {
    const float sg = (t1 & 0x80u) ? -1.0f : 1.0f;
    if ((t1 & 0x7fu) == 0x7fu) return __builtin_nanf("");
    if ((t1 & 0x7fu) == 0x7eu) return sg * __builtin_inff();
    return (t1 & 0x7fu) ? sg : 0.0f;
  }
  return e4m3_to_f32(t1) * e8m0_as_cvt_scale(b1) + e4m3_to_f32(t2) * e8m0_as_cvt_scale(b2);
}

// sum_k a[row][k] * W[k] for an F8X2 activation row and one MXFP4 weight row.
__device__ inline float ref_dot_f8x2_mxfp4(const uint8_t* data, const uint32_t* e8, int M, int row,
                                           const uint8_t* w, const uint8_t* s, int K) {
  float acc = 0.0f;
  for (int kb = 0; kb < K / 32; kb++) {
    const float sc = e8m0_to_float(s[kb]);
    for (int j = 0; j < 16; j++) {
      const v2f c = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w[kb * 16 + j], 1.0f, 0);
      acc += f8x2_ref_value(data, e8, M, K, row, kb * 32 + 2 * j) * (c[0] * sc);
      acc += f8x2_ref_value(data, e8, M, K, row, kb * 32 + 2 * j + 1) * (c[1] * sc);
    }
  }
  return acc;
}

// One FP8 weight byte -> f32: E4M3 (0x7f / 0xff NaN, no infinities) or E5M2
// (IEEE-like: infinities and NaNs).
template <bool E5M2>
__device__ __forceinline__ float fp8_to_f32(uint32_t byte) {
  if constexpr (E5M2) return __builtin_amdgcn_cvt_scalef32_pk_f32_bf8(byte & 255u, 1.0f, false)[0];
  else return e4m3_to_f32(byte);
}

// sum_k x[k] * W[k] for one f16 activation row and one FP8 weight row
// (codes only: the caller applies the row scale).
template <bool E5M2>
__device__ inline float ref_dot_f16_fp8(const uint16_t* x, const uint8_t* w, int K) {
  float acc = 0.0f;
  for (int k = 0; k < K; k++) acc += f16_bits_to_f32(x[k]) * fp8_to_f32<E5M2>(w[k]);
  return acc;
}

// sum_k a[row][k] * W[k] for an F8X2 activation row and one FP8 weight row
// (codes only).
template <bool E5M2>
__device__ inline float ref_dot_f8x2_fp8(const uint8_t* data, const uint32_t* e8, int M, int row,
                                         const uint8_t* w, int K) {
  float acc = 0.0f;
  for (int k = 0; k < K; k++) acc += f8x2_ref_value(data, e8, M, K, row, k) * fp8_to_f32<E5M2>(w[k]);
  return acc;
}

// E8M0 byte of (row, 32-K block b) in a stage-major scale plane: [K/128]
// planes of `rows` dwords, each the four bytes of one row's 128-K stage.
__device__ __forceinline__ uint32_t e8m0_stage_major(const uint8_t* s, size_t rows, int row, int b) {
  return s[(((size_t)(b >> 2) * rows + row) << 2) + (b & 3)];
}

// sum_k A[row][k] * W[col][k] with both operands MXFP4 (codes [.][K/2], low
// nibble = even k; stage-major scale planes of a_rows / w_rows rows), each
// dequantized as the reference does before the product.
__device__ inline float ref_dot_mxfp4_mxfp4(const uint8_t* a, const uint8_t* as, size_t a_rows, int row,
                                           const uint8_t* w, const uint8_t* ws, size_t w_rows, int col, int K) {
  const uint8_t* ar = a + (size_t)row * (K / 2);
  const uint8_t* wr = w + (size_t)col * (K / 2);
  float acc = 0.0f;
  for (int b = 0; b < K / 32; b++) {
    const float sa = e8m0_to_float(e8m0_stage_major(as, a_rows, row, b));
    const float sw = e8m0_to_float(e8m0_stage_major(ws, w_rows, col, b));
    for (int j = 0; j < 16; j++) {
      const v2f ca = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(ar[b * 16 + j], 1.0f, 0);
      const v2f cw = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(wr[b * 16 + j], 1.0f, 0);
      acc += (ca[0] * sa) * (cw[0] * sw);
      acc += (ca[1] * sa) * (cw[1] * sw);
    }
  }
  return acc;
}

// F8X2 term scale of a group with amax bits `amax_bits` (finite, > 0): the
// smallest power of two s with amax <= 448 s (the E4M3 maximum, so no code
// saturates), as an E8M0 byte (clamped at 2^-127).
__device__ __forceinline__ uint32_t f8x2_scale_byte(uint32_t amax_bits) {
  const uint32_t e = amax_bits >> 23;
  const int fl = e ? (int)e - 127 : (31 - __builtin_clz(amax_bits)) - 149;
  int s = fl - 8 + ((e && (amax_bits & 0x7fffffu) > 0x600000u) ? 1 : 0);
  if (s < -127) s = -127;
  return (uint32_t)(s + 127);
}

// F8X2 split (layout in mx_internal.h) of one (row, 64-K group), held by L
// consecutive lanes (L = 2, 4, 8 or 16; the group starts at a lane index
// that is a multiple of L): lane j = lane % L holds the V = 64 / L values of
// k [V j, V j + V) in v.  t1 = RNE_E4M3(v / s1); the residual r = v - t1 s1
// is exact in f32; t2 = RNE_E4M3(r / s2), each s from its term's group
// maximum.  A group with a non-finite value gets scale bytes 255 (its
// products are NaN, which marks every output it feeds) and carries the class
// of each value in its first term's byte for the exact fix-up of those
// outputs (f8x2_ref_value): 0x7f NaN, 0x7e +inf, 0xfe -inf, 0x00 zero, 0x38 /
// 0xb8 a finite non-zero value of that sign (as +-1); the second term is zero.
// An all-zero group gets bytes 127 and zero codes.  All L lanes must be
// active (they exchange maxima).  Writes the lane's bytes of both terms into
// the group's 128 bytes at `grp` and, from lane j = 0, the scale dword at
// `e8`.
template <int L>
__device__ __forceinline__ void f8x2_split_store(const float* v, int j, uint8_t* grp, uint32_t* e8) {
  constexpr int V = 64 / L, D = V / 4;  // values and dwords per lane and term
  static_assert(L >= 2 && L <= 16 && (L & (L - 1)) == 0, "2..16 lanes per group");
  uint32_t am = 0;
#pragma unroll
  for (int k = 0; k < V; k++) am = max(am, __builtin_bit_cast(uint32_t, v[k]) & 0x7fffffffu);
#pragma unroll
  for (int o = 1; o < L; o <<= 1) am = max(am, (uint32_t)__shfl_xor((int)am, o));
  uint32_t t1[D], t2[D];
  uint32_t b1 = 127u, b2 = 127u;
  if (am >= 0x7f800000u) {
    b1 = b2 = 255u;
#pragma unroll
    for (int d = 0; d < D; d++) {
      uint32_t w = 0;
#pragma unroll
      for (int t = 0; t < 4; t++) {
        const uint32_t u = __builtin_bit_cast(uint32_t, v[4 * d + t]), a = u & 0x7fffffffu;
        const uint32_t sg = (u >> 24) & 0x80u;
        const uint32_t code = a > 0x7f800000u ? 0x7fu : a == 0x7f800000u ? (0x7eu | sg) : a ? (0x38u | sg) : 0u;
        w |= code << (8 * t);
      }
      t1[d] = w;
      t2[d] = 0u;
    }
  } else {
#pragma unroll
    for (int d = 0; d < D; d++) t1[d] = t2[d] = 0u;
    float r[V];
#pragma unroll
    for (int k = 0; k < V; k++) r[k] = v[k];
    if (am != 0u) {
      b1 = f8x2_scale_byte(am);
      const float sc1 = e8m0_as_cvt_scale(b1);
      uint32_t am2 = 0;
#pragma unroll
      for (int d = 0; d < D; d++) {
        v2s w = {0, 0};
        w = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(w, v[4 * d], v[4 * d + 1], sc1, false);
        w = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(w, v[4 * d + 2], v[4 * d + 3], sc1, true);
        t1[d] = __builtin_bit_cast(uint32_t, w);
        const v2f lo = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(t1[d], sc1, false);
        const v2f hi = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(t1[d], sc1, true);
        r[4 * d] = v[4 * d] - lo[0];
        r[4 * d + 1] = v[4 * d + 1] - lo[1];
        r[4 * d + 2] = v[4 * d + 2] - hi[0];
        r[4 * d + 3] = v[4 * d + 3] - hi[1];
#pragma unroll
        for (int t = 0; t < 4; t++) am2 = max(am2, __builtin_bit_cast(uint32_t, r[4 * d + t]) & 0x7fffffffu);
      }
#pragma unroll
      for (int o = 1; o < L; o <<= 1) am2 = max(am2, (uint32_t)__shfl_xor((int)am2, o));
      if (am2 != 0u) {
        b2 = f8x2_scale_byte(am2);
        const float sc2 = e8m0_as_cvt_scale(b2);
#pragma unroll
        for (int d = 0; d < D; d++) {
          v2s w = {0, 0};
          w = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(w, r[4 * d], r[4 * d + 1], sc2, false);
          w = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(w, r[4 * d + 2], r[4 * d + 3], sc2, true);
          t2[d] = __builtin_bit_cast(uint32_t, w);
        }
      }
    }
  }
  // k -> byte (k & 15) + 16 * {0, 2, 1, 3}[k / 16] within a term
#pragma unroll
  for (int d = 0; d < D; d++) {
    const int k0 = V * j + 4 * d, q = k0 >> 4;
    const int pos = (k0 & 15) + 16 * (q == 1 ? 2 : q == 2 ? 1 : q);
    *reinterpret_cast<uint32_t*>(grp + pos) = t1[d];
    *reinterpret_cast<uint32_t*>(grp + 64 + pos) = t2[d];
  }
  if (j == 0) *e8 = b1 | (b2 << 8);
}

// Quantize 8 consecutive f32 values into one dword of 8 FP4 codes with the
// block scale byte `sb` (0..254): code = RNE(x / 2^(sb-127)), saturating.
__device__ __forceinline__ uint32_t fp4x8_from_f32(const float* v, uint32_t sb) {
  float sc = e8m0_as_cvt_scale(sb);
  uint32_t r = 0;
  r = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(r, v[0], v[1], sc, 0);
  r = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(r, v[2], v[3], sc, 1);
  r = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(r, v[4], v[5], sc, 2);
  r = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(r, v[6], v[7], sc, 3);
  return r;
}

__device__ __forceinline__ uint32_t abs_bits(float f) {
  return __builtin_bit_cast(uint32_t, f) & 0x7fffffffu;
}

// Accumulator element (lane, reg v) -> (row, col) within a 32x32 tile.
__device__ __forceinline__ int acc32_row(int lane, int v) {
  return (v >> 2) * 8 + (lane >> 5) * 4 + (v & 3);
}

__device__ __forceinline__ v16f mfma_f16_32x32x16(v8h a, v8h b, v16f c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ v4f mfma_f16_16x16x32(v8h a, v8h b, v4f c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// FP4 x FP4 scaled MFMA.  OPSA/OPSB select the byte of the scale dwords.
template <int OPSA, int OPSB>
__device__ __forceinline__ v16f mfma_fp4_32x32x64(v4i a, v4i b, v16f c, int sa, int sb) {
  v8i a8, b8;
  a8[0] = a[0]; a8[1] = a[1]; a8[2] = a[2]; a8[3] = a[3];
  a8[4] = 0; a8[5] = 0; a8[6] = 0; a8[7] = 0;
  b8[0] = b[0]; b8[1] = b[1]; b8[2] = b[2]; b8[3] = b[3];
  b8[4] = 0; b8[5] = 0; b8[6] = 0; b8[7] = 0;
  return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a8, b8, c, 4, 4, OPSA, sa, OPSB, sb);
}

}  // namespace mx
