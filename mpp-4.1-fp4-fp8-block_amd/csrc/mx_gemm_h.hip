// mx_gemm_h.hip - tiled fp16-MFMA GEMM with half (or f32) activations and
// quantized weights dequantized on the way into LDS.
//
//   C[m][n] = sum_k A[m][k] * W[n][k]
//
// Counterparts in the reference (root = Anemll/MPP-4.1-FP4-FP8-block):
//   MXFP4 weights    mxfp4_native_sp_h_f_n64 / mxfp4_fused_h_f_n64
//                    (MXFP4Kernels.metal:42-173, 264-286)
//   f16 weights      mpp_mlp_h_h_f_n128 / mpp_mlp_f_h_f_n128
//                    (MPPMLPKernels.metal:14-48, 164-173)
//   FP8/INT8/INT4    mpp_mlp_h_fp8e4m3_f / _h_fp8e5m2_f / _h_i8_f / _h_i4_f
//                    (MPPMLPKernels.metal:50-125), plus BASELINE's scales
//   SwiGLU epilogue  mpp_mlp_swiglu_float / _half (MPPMLPKernels.metal:186-220),
//                    fused: gate and up tiles are computed by the same
//                    workgroup, so silu(g)*u never leaves registers.
//
// Design (gfx950): 256 threads = 4 wave64s in a 2x2 grid; tile BM x 64
// columns per weight matrix (two matrices for the SwiGLU epilogue); K step
// 32 = one MXFP4 / INT4 scale block.  The weight tile is decoded once per
// workgroup while it is staged into LDS (FP4 via v_cvt_scalef32_pk_f16_fp4,
// which applies the E8M0 scale in the same instruction; FP8 via
// v_cvt_scalef32_pk_f16_fp8), so every MFMA operand is plain f16 and
// v_mfma_f32_32x32x16_f16 accumulates in f32.  LDS rows are padded to 80 B
// so the 16-byte fragment reads of a wave hit distinct banks.  Double-
// buffered LDS with register prefetch: one barrier per K step.
#include "mx_device.h"
#include "mx_internal.h"

namespace mx {

constexpr int kBN = 64;       // columns per weight matrix per workgroup
constexpr int kBK = 32;       // K per pipeline step
constexpr int kLdsRow = 40;   // halves per LDS row (32 + 8 pad)

template <int BKIND>
struct BChunk {  // one thread's slice of a weight tile: row r, 8 k values
  uint4 raw;
  uint32_t sc;
};

// Load this thread's 8-element slice (row r = tid/4, k offset 8*(tid%4)) of
// weight tile rows [n0, n0+64), k block kb.  Rows past the last one (n not
// a multiple of the tile) re-read row n-1: their columns are never stored.
template <int BKIND>
__device__ __forceinline__ void load_b(const void* __restrict__ b, const void* __restrict__ s,
                                       int n0, int kb, int n, int k, int tid, BChunk<BKIND>& out) {
  const int r = min(n0 + (tid >> 2), n - 1), q = tid & 3;
  if (BKIND == BK_F16) {
    const uint16_t* p = reinterpret_cast<const uint16_t*>(b) + (size_t)r * k + kb * 32 + q * 8;
    out.raw = *reinterpret_cast<const uint4*>(p);
  } else if (BKIND == BK_MXFP4) {
    const uint8_t* p = reinterpret_cast<const uint8_t*>(b) + (size_t)r * (k / 2) + kb * 16 + q * 4;
    out.raw.x = *reinterpret_cast<const uint32_t*>(p);
    out.sc = reinterpret_cast<const uint8_t*>(s)[(size_t)r * (k / 32) + kb];
  } else if (BKIND == BK_INT4G32) {
    const uint8_t* p = reinterpret_cast<const uint8_t*>(b) + (size_t)r * (k / 2) + kb * 16 + q * 4;
    out.raw.x = *reinterpret_cast<const uint32_t*>(p);
    out.sc = reinterpret_cast<const uint16_t*>(s)[(size_t)r * (k / 32) + kb];
  } else {  // 8-bit formats: 8 bytes
    const uint8_t* p = reinterpret_cast<const uint8_t*>(b) + (size_t)r * k + kb * 32 + q * 8;
    uint2 v = *reinterpret_cast<const uint2*>(p);
    out.raw.x = v.x;
    out.raw.y = v.y;
  }
}

// Decode the slice to 8 halves (exact for FP4 at in-range scales, FP8, INT8;
// INT4 rounds q*scale to half once).
template <int BKIND>
__device__ __forceinline__ uint4 decode_b(const BChunk<BKIND>& c) {
  if (BKIND == BK_F16) return c.raw;
  v8h h;
  if (BKIND == BK_MXFP4) {
    h = fp4x8_dequant_f16(c.raw.x, c.sc);
  } else if (BKIND == BK_E4M3 || BKIND == BK_E5M2) {
    uint32_t w[2] = {c.raw.x, c.raw.y};
#pragma unroll
    for (int t = 0; t < 2; t++) {
      v2h lo, hi;
      if (BKIND == BK_E4M3) {
        lo = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w[t], 1.0f, false);
        hi = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w[t], 1.0f, true);
      } else {
        lo = __builtin_amdgcn_cvt_scalef32_pk_f16_bf8(w[t], 1.0f, false);
        hi = __builtin_amdgcn_cvt_scalef32_pk_f16_bf8(w[t], 1.0f, true);
      }
      h[4 * t] = lo[0]; h[4 * t + 1] = lo[1]; h[4 * t + 2] = hi[0]; h[4 * t + 3] = hi[1];
    }
  } else if (BKIND == BK_INT8) {
    uint32_t w[2] = {c.raw.x, c.raw.y};
#pragma unroll
    for (int t = 0; t < 8; t++) h[t] = (_Float16)(int)(int8_t)(w[t >> 2] >> (8 * (t & 3)));
  } else {  // INT4 g32: ((nib ^ 8) - 8) * f16 scale (PackedNumericKernels.metal:30-33)
    float sc = f16_bits_to_f32((uint16_t)c.sc);
#pragma unroll
    for (int t = 0; t < 8; t++) {
      int v = (int)((c.raw.x >> (4 * t)) & 15u);
      h[t] = (_Float16)((float)((v ^ 8) - 8) * sc);
    }
  }
  return __builtin_bit_cast(uint4, h);
}

template <int BKIND, int EPI, int A_F32, int BM>
__global__ __launch_bounds__(256) void k_gemm_h(GemmArgs g) {
  constexpr int NB = (EPI == EPI_SWIGLU_F16 || EPI == EPI_SWIGLU_HALF) ? 2 : 1;
  constexpr int MB = BM / 64;               // 32-row blocks per wave
  constexpr int ACH = A_F32 ? BM / 32 : BM / 64;  // A chunks per thread per step
  __shared__ __attribute__((aligned(16))) _Float16 As[2][BM * kLdsRow];
  // f32 activations: the second f16 term of each value, lo = f16(x - hi)
  __shared__ __attribute__((aligned(16))) _Float16 Al[A_F32 ? 2 : 1][A_F32 ? BM * kLdsRow : 8];
  __shared__ __attribute__((aligned(16))) _Float16 Bs[2][NB * kBN * kLdsRow];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave & 1, wn = wave >> 1;
  const int n0 = blockIdx.x * kBN, m0 = blockIdx.y * BM;
  const int M = g.m, K = g.k;
  const int KT = K / kBK;

  uint4 areg[ACH];
  BChunk<BKIND> breg[NB];

#define MX_LOAD_A(kb)                                                                      \
  _Pragma("unroll") for (int c = 0; c < ACH; c++) {                                        \
    const int idx = tid + c * 256;                                                         \
    /* rows past M re-read row M-1: unconditional loads, and those tile rows */            \
    /* only feed output rows that are never stored */                                      \
    if (A_F32) {                                                                           \
      const int row = min(m0 + (idx >> 3), M - 1);                                         \
      areg[c] = *reinterpret_cast<const uint4*>(reinterpret_cast<const float*>(g.a) +      \
                                                (size_t)row * K + (kb) * 32 + (idx & 7) * 4); \
    } else {                                                                               \
      const int row = min(m0 + (idx >> 2), M - 1);                                         \
      areg[c] = *reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(g.a) +   \
                                                (size_t)row * K + (kb) * 32 + (idx & 3) * 8); \
    }                                                                                      \
  }
#define MX_STORE_A(buf)                                                                    \
  _Pragma("unroll") for (int c = 0; c < ACH; c++) {                                        \
    const int idx = tid + c * 256;                                                         \
    if (A_F32) {                                                                           \
      const float x_[4] = {__builtin_bit_cast(float, areg[c].x), __builtin_bit_cast(float, areg[c].y), \
                           __builtin_bit_cast(float, areg[c].z), __builtin_bit_cast(float, areg[c].w)}; \
      v4h h, l;                                                                            \
      _Pragma("unroll") for (int t = 0; t < 4; t++) {                                      \
        h[t] = (_Float16)x_[t];                                                            \
        l[t] = __builtin_isinf((float)h[t]) ? (_Float16)0.0f : (_Float16)(x_[t] - (float)h[t]); \
      }                                                                                    \
      *reinterpret_cast<v4h*>(&As[buf][(idx >> 3) * kLdsRow + (idx & 7) * 4]) = h;         \
      *reinterpret_cast<v4h*>(&Al[A_F32 ? buf : 0][(idx >> 3) * kLdsRow + (idx & 7) * 4]) = l; \
    } else {                                                                               \
      *reinterpret_cast<uint4*>(&As[buf][(idx >> 2) * kLdsRow + (idx & 3) * 8]) = areg[c]; \
    }                                                                                      \
  }
#define MX_LOAD_B(kb)                                                                      \
  load_b<BKIND>(g.b0, g.s0, n0, (kb), g.n, K, tid, breg[0]);                              \
  if (NB == 2) load_b<BKIND>(g.b1, g.s1, n0, (kb), g.n, K, tid, breg[NB - 1]);
#define MX_STORE_B(buf)                                                                    \
  _Pragma("unroll") for (int j = 0; j < NB; j++)                                           \
    *reinterpret_cast<uint4*>(&Bs[buf][(j * kBN + (tid >> 2)) * kLdsRow + (tid & 3) * 8]) = \
        decode_b<BKIND>(breg[j]);

  v16f acc[NB][MB];
#pragma unroll
  for (int j = 0; j < NB; j++)
#pragma unroll
    for (int i = 0; i < MB; i++)
#pragma unroll
      for (int v = 0; v < 16; v++) acc[j][i][v] = 0.0f;

  MX_LOAD_A(0)
  MX_LOAD_B(0)
  MX_STORE_A(0)
  MX_STORE_B(0)
  __syncthreads();

  const int frag_row = lane & 31, frag_k = (lane >> 5) * 8;
  for (int kt = 0; kt < KT; kt++) {
    const int buf = kt & 1;
    // Prefetch the next step unconditionally (the last step re-reads itself
    // into the idle buffer) so no load sits behind a branch.
    const int kn = kt + 1 < KT ? kt + 1 : kt;
    MX_LOAD_A(kn)
    MX_LOAD_B(kn)
#pragma unroll
    for (int ks = 0; ks < 2; ks++) {
      v8h af[MB], bf[NB];
#pragma unroll
      for (int i = 0; i < MB; i++)
        af[i] = *reinterpret_cast<const v8h*>(
            &As[buf][(wm * (BM / 2) + i * 32 + frag_row) * kLdsRow + ks * 16 + frag_k]);
#pragma unroll
      for (int j = 0; j < NB; j++)
        bf[j] = *reinterpret_cast<const v8h*>(
            &Bs[buf][(j * kBN + wn * 32 + frag_row) * kLdsRow + ks * 16 + frag_k]);
#pragma unroll
      for (int j = 0; j < NB; j++)
#pragma unroll
        for (int i = 0; i < MB; i++) acc[j][i] = mfma_f16_32x32x16(af[i], bf[j], acc[j][i]);
      if constexpr (A_F32 != 0) {  // the second term of the f32 activations
#pragma unroll
        for (int i = 0; i < MB; i++) {
          const v8h al = *reinterpret_cast<const v8h*>(
              &Al[buf][(wm * (BM / 2) + i * 32 + frag_row) * kLdsRow + ks * 16 + frag_k]);
#pragma unroll
          for (int j = 0; j < NB; j++) acc[j][i] = mfma_f16_32x32x16(al, bf[j], acc[j][i]);
        }
      }
    }
    MX_STORE_A(buf ^ 1)
    MX_STORE_B(buf ^ 1)
    __syncthreads();
  }

  // Epilogue.  Columns past n (the tail tile) are not stored.
  const int col = n0 + wn * 32 + (lane & 31);
  if (col >= g.n) return;
  float rs0 = 1.0f, rs1 = 1.0f;
  if (BKIND == BK_E4M3 || BKIND == BK_E5M2 || BKIND == BK_INT8) {
    rs0 = reinterpret_cast<const float*>(g.s0)[col];
    if (NB == 2) rs1 = reinterpret_cast<const float*>(g.s1)[col];
  }
#pragma unroll
  for (int i = 0; i < MB; i++) {
#pragma unroll
    for (int v = 0; v < 16; v++) {
      const int row = m0 + wm * (BM / 2) + i * 32 + acc32_row(lane, v);
      if (row >= M) continue;
      const size_t o = (size_t)row * g.n + col;
      float x0 = acc[0][i][v] * rs0;
      if (EPI == EPI_STORE_F32) {
        reinterpret_cast<float*>(g.c)[o] = x0;
      } else if (EPI == EPI_STORE_F16) {
        reinterpret_cast<uint16_t*>(g.c)[o] = f32_to_f16_bits(x0);
      } else {
        float u = acc[NB - 1][i][v] * rs1;
        float m;
        if (EPI == EPI_SWIGLU_F16) {
          m = silu(x0) * u;
        } else {
          float gg = fminf(fmaxf(x0 * 0.0625f, -20.0f), 20.0f);
          m = (gg / (1.0f + expf(-gg))) * (u * 0.0625f);
        }
        reinterpret_cast<uint16_t*>(g.c)[o] = f32_to_f16_bits(m);
      }
    }
  }
}

#undef MX_LOAD_A
#undef MX_STORE_A
#undef MX_LOAD_B
#undef MX_STORE_B

template <int BKIND, int EPI, int A_F32>
static hipError_t launch_bm(const GemmArgs& g, hipStream_t st) {
  // 128-row tiles when they give at least one workgroup per CU, else 64.
  const int tiles_n = (g.n + kBN - 1) / kBN;
  const int tiles128 = ((g.m + 127) / 128) * tiles_n;
  if (g.m > 64 && tiles128 >= 256) {
    dim3 grid(tiles_n, (g.m + 127) / 128);
    hipLaunchKernelGGL((k_gemm_h<BKIND, EPI, A_F32, 128>), grid, dim3(256), 0, st, g);
  } else {
    dim3 grid(tiles_n, (g.m + 63) / 64);
    hipLaunchKernelGGL((k_gemm_h<BKIND, EPI, A_F32, 64>), grid, dim3(256), 0, st, g);
  }
  return hipGetLastError();
}

template <int BKIND>
static hipError_t launch_epi(int epi, const GemmArgs& g, hipStream_t st) {
  const bool af32 = g.a_dtype == MX_DTYPE_F32;
  switch (epi) {
    case EPI_STORE_F32:
      return af32 ? launch_bm<BKIND, EPI_STORE_F32, 1>(g, st) : launch_bm<BKIND, EPI_STORE_F32, 0>(g, st);
    case EPI_STORE_F16:
      return af32 ? launch_bm<BKIND, EPI_STORE_F16, 1>(g, st) : launch_bm<BKIND, EPI_STORE_F16, 0>(g, st);
    case EPI_SWIGLU_F16:
      return launch_bm<BKIND, EPI_SWIGLU_F16, 0>(g, st);
    case EPI_SWIGLU_HALF:
      return launch_bm<BKIND, EPI_SWIGLU_HALF, 0>(g, st);
  }
  return hipErrorInvalidValue;
}

// Preconditions (checked by the caller): n >= 1, k % 32 == 0, m > 0;
// SwiGLU epilogues take f16 activations.  Any n works (the tail tile's rows
// past n re-read row n-1 and are not stored), as the reference's matmul
// tiles guard column < n (MXFP4Kernels.metal:98).
hipError_t launch_gemm_h(int bkind, int epi, const GemmArgs& g, hipStream_t st) {
  switch (bkind) {
    case BK_F16: return launch_epi<BK_F16>(epi, g, st);
    case BK_MXFP4: return launch_epi<BK_MXFP4>(epi, g, st);
    case BK_E4M3: return launch_epi<BK_E4M3>(epi, g, st);
    case BK_E5M2: return launch_epi<BK_E5M2>(epi, g, st);
    case BK_INT8: return launch_epi<BK_INT8>(epi, g, st);
    case BK_INT4G32: return launch_epi<BK_INT4G32>(epi, g, st);
  }
  return hipErrorInvalidValue;
}

}  // namespace mx
