// mx_accum.hip - unscaled FP4 x FP4 and FP8 x FP8 GEMM for the accumulator
// probe: the counterpart of accum_fp4_fp4_{h,f} and accum_fp8_fp8_{h,f}
// (AccumProbeKernels.metal:87-127, all built on accum_probe_tile :16-38).
//
//   C[m][n] = sum_k A[m][k] * B[n][k]
//
// A [m][k] and B [n][k] are K-contiguous: E2M1 two per byte (low nibble =
// even k) or E4M3 one per byte, with no block scales (the scaled MFMA gets
// E8M0 127 = 1.0 for both operands).  Accumulation is f32 in the MFMA; C is
// f32, or f16 from one RNE conversion of the f32 sum (v_cvt_f16_f32, which
// overflows to inf at >= 65520 and never saturates).
//
// One wave64 per 32 x 32 block of C, v_mfma_scale_f32_32x32x64_f8f6f4 per
// 64-K step with operands read straight from global memory: lane l feeds row
// l % 32 and K values [32 (l / 32), +32) of the step, i.e. 16 bytes of FP4 or
// 32 bytes of FP8.  This is a numerics probe, not a hot path: no LDS
// staging.  K is a multiple of 64 (the host pads shorter rows with zero codes,
// see launch_pad_rows).
#include "mx_device.h"
#include "mx_internal.h"

namespace mx {

// FMT: the MFMA's operand format code (0 = FP8 E4M3, 4 = FP4 E2M1).
template <int FMT, bool OUT_F32>
__global__ __launch_bounds__(256) void k_gemm_f8f6f4_unit(const uint8_t* a, const uint8_t* b, void* c, int m,
                                                           int n, int k) {
  const int lane = threadIdx.x & 63;
  const int blk = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int nbn = n / 32;
  const int bm = blk / nbn, bn = blk % nbn;
  if (bm * 32 >= m) return;  // wave-uniform: the grid's last workgroup may be partial
  constexpr int kLaneBytes = FMT == 4 ? 16 : 32;  // per lane per 64-K step
  const size_t row_b = FMT == 4 ? (size_t)k / 2 : (size_t)k;
  const uint8_t* pa = a + (size_t)(bm * 32 + (lane & 31)) * row_b + (lane >> 5) * kLaneBytes;
  const uint8_t* pb = b + (size_t)(bn * 32 + (lane & 31)) * row_b + (lane >> 5) * kLaneBytes;
  v16f acc;
#pragma unroll
  for (int v = 0; v < 16; v++) acc[v] = 0.0f;
  for (int s = 0; s < k / 64; s++) {
    const size_t off = (size_t)s * 2 * kLaneBytes;
    v8i av, bv;
    if (FMT == 4) {
      const v4i x = *reinterpret_cast<const v4i*>(pa + off);
      const v4i y = *reinterpret_cast<const v4i*>(pb + off);
#pragma unroll
      for (int i = 0; i < 4; i++) {
        av[i] = x[i]; av[4 + i] = 0;
        bv[i] = y[i]; bv[4 + i] = 0;
      }
    } else {
      const v4i* xa = reinterpret_cast<const v4i*>(pa + off);
      const v4i* xb = reinterpret_cast<const v4i*>(pb + off);
      const v4i x0 = xa[0], x1 = xa[1], y0 = xb[0], y1 = xb[1];
#pragma unroll
      for (int i = 0; i < 4; i++) {
        av[i] = x0[i]; av[4 + i] = x1[i];
        bv[i] = y0[i]; bv[4 + i] = y1[i];
      }
    }
    acc = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(av, bv, acc, FMT, FMT, 0, 127, 0, 127);
  }
  const int col = bn * 32 + (lane & 31);
#pragma unroll
  for (int v = 0; v < 16; v++) {
    const int row = bm * 32 + acc32_row(lane, v);
    const float x = acc[v];
    if (OUT_F32) reinterpret_cast<float*>(c)[(size_t)row * n + col] = x;
    else reinterpret_cast<uint16_t*>(c)[(size_t)row * n + col] = f32_to_f16_bits(x);
  }
}

// dst rows of rbp bytes = src rows of rb bytes followed by zero bytes (a
// zero byte is a zero in every operand format here: f16 +0, E4M3 +0, two
// E2M1 +0), so a dot product over the padded K is the dot product over K.
__global__ void k_pad_rows(const uint8_t* src, size_t rows, size_t rb, uint8_t* dst, size_t rbp) {
  const size_t total = rows * rbp;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (size_t)gridDim.x * blockDim.x) {
    const size_t r = i / rbp, j = i % rbp;
    dst[i] = j < rb ? src[r * rb + j] : 0;
  }
}

hipError_t launch_pad_rows(const uint8_t* src, size_t rows, size_t rb, uint8_t* dst, size_t rbp, hipStream_t st) {
  if (rb > rbp) return hipErrorInvalidValue;
  size_t blocks = (rows * rbp + 255) / 256;
  blocks = blocks < 1 ? 1 : blocks > 4096 ? 4096 : blocks;  // grid-stride loop covers the rest
  hipLaunchKernelGGL(k_pad_rows, dim3((unsigned)blocks), dim3(256), 0, st, src, rows, rb, dst, rbp);
  return hipGetLastError();
}

// Exact widening with the same zero padding: signed INT4 (two per byte, low
// nibble first, ((b & 15) ^ 8) - 8, PackedNumericKernels.metal:25-28) or
// INT8 rows of k values -> rows of kp values, as int8 (INT4 only) or f16.
template <bool SRC_I4, bool DST_F16>
__global__ void k_widen_rows(const uint8_t* src, size_t rows, size_t k, void* dst, size_t kp) {
  const size_t total = rows * kp;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (size_t)gridDim.x * blockDim.x) {
    const size_t r = i / kp, j = i % kp;
    int v = 0;
    if (j < k) {
      if (SRC_I4) {
        const uint8_t b = src[r * (k / 2) + j / 2];
        v = ((int)((j & 1) ? b >> 4 : b & 15) ^ 8) - 8;
      } else {
        v = (int)(int8_t)src[r * k + j];
      }
    }
    if (DST_F16) reinterpret_cast<uint16_t*>(dst)[i] = f32_to_f16_bits((float)v);
    else reinterpret_cast<int8_t*>(dst)[i] = (int8_t)v;
  }
}

hipError_t launch_widen_rows(int src_int4, int dst_f16, const uint8_t* src, size_t rows, size_t k, void* dst,
                             size_t kp, hipStream_t st) {
  if (k > kp || (src_int4 && k % 2)) return hipErrorInvalidValue;
  size_t blocks = (rows * kp + 255) / 256;
  blocks = blocks < 1 ? 1 : blocks > 4096 ? 4096 : blocks;  // grid-stride loop covers the rest
  const dim3 grid((unsigned)blocks), block(256);
  if (src_int4) {
    if (dst_f16) hipLaunchKernelGGL((k_widen_rows<true, true>), grid, block, 0, st, src, rows, k, dst, kp);
    else hipLaunchKernelGGL((k_widen_rows<true, false>), grid, block, 0, st, src, rows, k, dst, kp);
  } else {
    if (dst_f16) hipLaunchKernelGGL((k_widen_rows<false, true>), grid, block, 0, st, src, rows, k, dst, kp);
    else hipLaunchKernelGGL((k_widen_rows<false, false>), grid, block, 0, st, src, rows, k, dst, kp);
  }
  return hipGetLastError();
}

// dst[0, n) = value (16-bit), same purpose as k_fill_u8.
__global__ void k_fill_u16(uint16_t* dst, size_t n, uint32_t value) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
    dst[i] = (uint16_t)value;
}

hipError_t launch_fill_u16(uint16_t* dst, size_t n, uint16_t value, hipStream_t st) {
  if (n == 0) return hipSuccess;
  size_t blocks = (n + 255) / 256;
  blocks = blocks < 1 ? 1 : blocks > 1024 ? 1024 : blocks;
  hipLaunchKernelGGL(k_fill_u16, dim3((unsigned)blocks), dim3(256), 0, st, dst, n, (uint32_t)value);
  return hipGetLastError();
}

// dst[0, n) = value, for planes a caller's graph capture may record (a fill
// kernel rather than a memset node).
__global__ void k_fill_u8(uint8_t* dst, size_t n, uint32_t value) {
  const uint32_t v4 = value * 0x01010101u;
  const size_t n4 = n / 4;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += (size_t)gridDim.x * blockDim.x)
    reinterpret_cast<uint32_t*>(dst)[i] = v4;
  if (blockIdx.x == 0 && threadIdx.x < n % 4) dst[n4 * 4 + threadIdx.x] = (uint8_t)value;
}

hipError_t launch_fill_u8(uint8_t* dst, size_t n, uint8_t value, hipStream_t st) {
  if (n == 0) return hipSuccess;
  size_t blocks = (n / 4 + 255) / 256;
  blocks = blocks < 1 ? 1 : blocks > 1024 ? 1024 : blocks;  // grid-stride loop covers the rest
  hipLaunchKernelGGL(k_fill_u8, dim3((unsigned)blocks), dim3(256), 0, st, dst, n, (uint32_t)value);
  return hipGetLastError();
}

bool gemm_f8f6f4_unit_ok(int m, int n, int k) {
  return m > 0 && n > 0 && k > 0 && m % 32 == 0 && n % 32 == 0 && k % 64 == 0;
}

hipError_t launch_gemm_f8f6f4_unit(int fp4, int out_f32, const uint8_t* a, const uint8_t* b, void* c, int m,
                                   int n, int k, hipStream_t st) {
  if (!gemm_f8f6f4_unit_ok(m, n, k)) return hipErrorInvalidValue;
  const int blocks = (m / 32) * (n / 32);
  const dim3 grid((blocks + 3) / 4), block(256);
  if (fp4) {
    if (out_f32) hipLaunchKernelGGL((k_gemm_f8f6f4_unit<4, true>), grid, block, 0, st, a, b, c, m, n, k);
    else hipLaunchKernelGGL((k_gemm_f8f6f4_unit<4, false>), grid, block, 0, st, a, b, c, m, n, k);
  } else {
    if (out_f32) hipLaunchKernelGGL((k_gemm_f8f6f4_unit<0, true>), grid, block, 0, st, a, b, c, m, n, k);
    else hipLaunchKernelGGL((k_gemm_f8f6f4_unit<0, false>), grid, block, 0, st, a, b, c, m, n, k);
  }
  return hipGetLastError();
}

}  // namespace mx
