// mx_codecs.hip - element codecs, the MXFP4 quantizer, the dequant-to-half
// unpack kernel, SwiGLU epilogues and weight-format quantizers.
//
// Reference counterparts (root = Anemll/MPP-4.1-FP4-FP8-block):
//   pack/unpack roundtrip  PackedNumericKernels.metal:35-96
//   dequant to half        MXFP4Kernels.metal:509-538 (native), 543-564 (LUT)
//   SwiGLU                 MPPMLPKernels.metal:186-257
//   MXFP4 quantizer        BASELINE.json configs[0] (not in the reference)
#include "mx_device.h"
#include "mx_internal.h"

namespace mx {

// ---------------------------------------------------------------------------
// Pack / unpack.  fmt 0 = FP4 E2M1 (2 codes per byte, low nibble = even
// index), 1 = FP8 E4M3, 2 = FP8 E5M2.  Conversions use the gfx950 scaled
// converters with scale 1.0 (E8M0 127).  FP8 inputs are clamped to the
// largest finite magnitude first (NaN passes through) so overflow saturates
// as the reference's KAT requires (main.swift:118-124: +-512 -> +-448).

__global__ void k_pack_fp4(const float* __restrict__ in, uint8_t* __restrict__ out, size_t n) {
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;  // one dword (8 codes) per thread
  size_t base = i * 8;
  if (base >= n) return;
  const float one = 1.0f;
  if (base + 8 <= n) {
    float v[8];
    const float4* p = reinterpret_cast<const float4*>(in + base);
    float4 a = p[0], b = p[1];
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    uint32_t r = 0;
    r = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(r, v[0], v[1], one, 0);
    r = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(r, v[2], v[3], one, 1);
    r = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(r, v[4], v[5], one, 2);
    r = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(r, v[6], v[7], one, 3);
    *reinterpret_cast<uint32_t*>(out + base / 2) = r;
  } else {
    for (size_t j = base; j < n; j += 2) {
      float a = in[j], b = (j + 1 < n) ? in[j + 1] : 0.0f;
      uint32_t r = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(0u, a, b, one, 0);
      uint8_t byte = (uint8_t)(r & 0xffu);
      if (j + 1 >= n) byte &= 0x0f;
      out[j / 2] = byte;
    }
  }
}

__global__ void k_unpack_fp4(const uint8_t* __restrict__ in, float* __restrict__ out, size_t n) {
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  size_t base = i * 8;
  if (base >= n) return;
  if (base + 8 <= n) {
    uint32_t w = *reinterpret_cast<const uint32_t*>(in + base / 2);
    v2f a = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 1.0f, 0);
    v2f b = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 1.0f, 1);
    v2f c = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 1.0f, 2);
    v2f d = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 1.0f, 3);
    float4* p = reinterpret_cast<float4*>(out + base);
    p[0] = make_float4(a[0], a[1], b[0], b[1]);
    p[1] = make_float4(c[0], c[1], d[0], d[1]);
  } else {
    for (size_t j = base; j < n; j += 2) {
      uint32_t w = in[j / 2];
      v2f a = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 1.0f, 0);
      out[j] = a[0];
      if (j + 1 < n) out[j + 1] = a[1];
    }
  }
}

template <bool E5M2>
__device__ __forceinline__ float fp8_clamp(float x) {
  const float lim = E5M2 ? 57344.0f : 448.0f;
  if (__builtin_isnan(x)) return x;
  return x > lim ? lim : (x < -lim ? -lim : x);
}

template <bool E5M2>
__device__ __forceinline__ uint32_t fp8x4_from_f32(float a, float b, float c, float d) {
  v2s r = {0, 0};
  a = fp8_clamp<E5M2>(a); b = fp8_clamp<E5M2>(b); c = fp8_clamp<E5M2>(c); d = fp8_clamp<E5M2>(d);
  if (E5M2) {
    r = __builtin_amdgcn_cvt_scalef32_pk_bf8_f32(r, a, b, 1.0f, false);
    r = __builtin_amdgcn_cvt_scalef32_pk_bf8_f32(r, c, d, 1.0f, true);
  } else {
    r = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(r, a, b, 1.0f, false);
    r = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(r, c, d, 1.0f, true);
  }
  return __builtin_bit_cast(uint32_t, r);
}

template <bool E5M2>
__device__ __forceinline__ void fp8x4_to_f32(uint32_t w, float* o) {
  v2f a, b;
  if (E5M2) {
    a = __builtin_amdgcn_cvt_scalef32_pk_f32_bf8(w, 1.0f, false);
    b = __builtin_amdgcn_cvt_scalef32_pk_f32_bf8(w, 1.0f, true);
  } else {
    a = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(w, 1.0f, false);
    b = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(w, 1.0f, true);
  }
  o[0] = a[0]; o[1] = a[1]; o[2] = b[0]; o[3] = b[1];
}

template <bool E5M2>
__global__ void k_pack_fp8(const float* __restrict__ in, uint8_t* __restrict__ out, size_t n) {
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;  // 4 values per thread
  size_t base = i * 4;
  if (base >= n) return;
  if (base + 4 <= n) {
    float4 v = *reinterpret_cast<const float4*>(in + base);
    *reinterpret_cast<uint32_t*>(out + base) = fp8x4_from_f32<E5M2>(v.x, v.y, v.z, v.w);
  } else {
    float v[4] = {0, 0, 0, 0};
    for (size_t j = base; j < n; j++) v[j - base] = in[j];
    uint32_t w = fp8x4_from_f32<E5M2>(v[0], v[1], v[2], v[3]);
    for (size_t j = base; j < n; j++) out[j] = (uint8_t)(w >> (8 * (j - base)));
  }
}

template <bool E5M2>
__global__ void k_unpack_fp8(const uint8_t* __restrict__ in, float* __restrict__ out, size_t n) {
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  size_t base = i * 4;
  if (base >= n) return;
  if (base + 4 <= n) {
    float o[4];
    fp8x4_to_f32<E5M2>(*reinterpret_cast<const uint32_t*>(in + base), o);
    *reinterpret_cast<float4*>(out + base) = make_float4(o[0], o[1], o[2], o[3]);
  } else {
    uint32_t w = 0;
    for (size_t j = base; j < n; j++) w |= (uint32_t)in[j] << (8 * (j - base));
    float o[4];
    fp8x4_to_f32<E5M2>(w, o);
    for (size_t j = base; j < n; j++) out[j] = o[j - base];
  }
}

// ---------------------------------------------------------------------------
// MXFP4 quantizer: one thread per 32-element block (row-major [rows][k]).
// Source f16 (SRC_F16) or f32.  Output codes [rows][k/2], scales [rows][k/32].
template <bool SRC_F16>
__global__ void k_mxfp4_quantize(const void* __restrict__ src, uint8_t* __restrict__ packed,
                                 uint8_t* __restrict__ scales, size_t nblocks) {
  size_t b = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= nblocks) return;
  float v[32];
  if (SRC_F16) {
    const uint4* p = reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(src) + b * 32);
#pragma unroll
    for (int q = 0; q < 4; q++) {
      uint4 w = p[q];
      uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
      for (int t = 0; t < 4; t++) {
        v[q * 8 + 2 * t] = f16_bits_to_f32((uint16_t)(ws[t] & 0xffffu));
        v[q * 8 + 2 * t + 1] = f16_bits_to_f32((uint16_t)(ws[t] >> 16));
      }
    }
  } else {
    const float4* p = reinterpret_cast<const float4*>(reinterpret_cast<const float*>(src) + b * 32);
#pragma unroll
    for (int q = 0; q < 8; q++) {
      float4 w = p[q];
      v[4 * q] = w.x; v[4 * q + 1] = w.y; v[4 * q + 2] = w.z; v[4 * q + 3] = w.w;
    }
  }
  uint32_t amax = 0;
#pragma unroll
  for (int j = 0; j < 32; j++) amax = max(amax, abs_bits(v[j]));
  uint32_t sb = mxfp4_scale_byte(amax);
  uint4 o = make_uint4(0, 0, 0, 0);
  if (sb != 255u) {
    o.x = fp4x8_from_f32(v + 0, sb);
    o.y = fp4x8_from_f32(v + 8, sb);
    o.z = fp4x8_from_f32(v + 16, sb);
    o.w = fp4x8_from_f32(v + 24, sb);
  }
  reinterpret_cast<uint4*>(packed)[b] = o;
  scales[b] = (uint8_t)sb;
}

// ---------------------------------------------------------------------------
// Dequant to half (MXFP4Kernels.metal:509-538): one thread per 8 elements
// (one dword of codes in, one 16-byte store out, so a wave writes 1 KB of
// contiguous output), one v_cvt_scalef32_pk_f16_fp4 per two values.  E8M0
// byte 255 decodes to +inf in the reference (bits<<23); the hardware would
// read it as NaN, so those codes take the exact path.
__global__ void k_mxfp4_dequant_f16(const uint8_t* __restrict__ packed,
                                    const uint8_t* __restrict__ scales,
                                    uint16_t* __restrict__ out, size_t nwords) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;  // dword of codes
  if (i >= nwords) return;
  const uint32_t w = reinterpret_cast<const uint32_t*>(packed)[i];
  const uint32_t sb = scales[i / 4];  // 4 dwords per 32-element block
  reinterpret_cast<uint4*>(out)[i] = __builtin_bit_cast(uint4, fp4x8_dequant_f16(w, sb));
}

// ---------------------------------------------------------------------------
// SwiGLU epilogues as separate kernels (MPPMLPKernels.metal:186-257).
// variant 0: float  -> float mid  g/(1+e^-g)*u                    (:186-202)
// variant 1: float  -> half mid   g'=clamp(g/16,+-20), u'=u/16    (:204-220)
// variant 2: half   -> half mid   as variant 1 from half inputs    (:222-238)
// variant 3: int32  -> int8 mid   g*2^-12, clamp, *32, rint        (:240-257)
__global__ void k_swiglu(int variant, const void* __restrict__ gate, const void* __restrict__ up,
                         void* __restrict__ mid, size_t count) {
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= count) return;
  if (variant == 0) {
    float g = reinterpret_cast<const float*>(gate)[i];
    float u = reinterpret_cast<const float*>(up)[i];
    reinterpret_cast<float*>(mid)[i] = (g / (1.0f + expf(-g))) * u;
  } else if (variant == 1 || variant == 2) {
    float g, u;
    if (variant == 1) {
      g = reinterpret_cast<const float*>(gate)[i];
      u = reinterpret_cast<const float*>(up)[i];
    } else {
      g = f16_bits_to_f32(reinterpret_cast<const uint16_t*>(gate)[i]);
      u = f16_bits_to_f32(reinterpret_cast<const uint16_t*>(up)[i]);
    }
    g = fminf(fmaxf(g * 0.0625f, -20.0f), 20.0f);
    u = u * 0.0625f;
    reinterpret_cast<uint16_t*>(mid)[i] = f32_to_f16_bits((g / (1.0f + expf(-g))) * u);
  } else {
    float g = (float)reinterpret_cast<const int32_t*>(gate)[i] * 0.000244140625f;
    float u = (float)reinterpret_cast<const int32_t*>(up)[i] * 0.000244140625f;
    g = fminf(fmaxf(g, -20.0f), 20.0f);
    float v = (g / (1.0f + expf(-g))) * u * 32.0f;
    v = fminf(fmaxf(v, -128.0f), 127.0f);
    reinterpret_cast<int8_t*>(mid)[i] = (int8_t)(int)rintf(v);
  }
}

// ---------------------------------------------------------------------------
// Weight-format quantizers.  One workgroup per row.
// fmt 1 = FP8 E4M3 / 2 = FP8 E5M2 (scale amax/qmax), 3 = INT8 (amax/127).
// Division in f32, matching the CPU oracle bit for bit.
// Also the per-token INT8 activation quantizer of W8A8 (SRC_F16: x in f16).

// 4 consecutive elements of row data (k % 4 == 0, so chunk c stays in the row
// and is 8- or 16-byte aligned).
template <bool SRC_F16>
__device__ __forceinline__ void ld_src4(const void* p, size_t base, int c, float v[4]) {
  if (SRC_F16) {
    const uint2 u = reinterpret_cast<const uint2*>(reinterpret_cast<const uint16_t*>(p) + base)[c];
    v[0] = f16_bits_to_f32((uint16_t)(u.x & 0xffffu));
    v[1] = f16_bits_to_f32((uint16_t)(u.x >> 16));
    v[2] = f16_bits_to_f32((uint16_t)(u.y & 0xffffu));
    v[3] = f16_bits_to_f32((uint16_t)(u.y >> 16));
  } else {
    const float4 f = reinterpret_cast<const float4*>(reinterpret_cast<const float*>(p) + base)[c];
    v[0] = f.x; v[1] = f.y; v[2] = f.z; v[3] = f.w;
  }
}

// One workgroup (512 threads) per row: amax (wave shuffles, one barrier),
// scale = amax / qmax, then every element v / scale to the format, 4
// elements per load.  Rows of at most 512 x 8 chunks (k <= 16384) keep the
// thread's chunks in registers between the two passes: all of a thread's
// loads are in flight at once and the row is read once.  Longer rows are
// read twice (the second pass from cache).
template <bool SRC_F16>
__global__ __launch_bounds__(512) void k_quant_rowwise(int fmt, const void* __restrict__ w, int k,
                                                       uint8_t* __restrict__ q, float* __restrict__ row_scale) {
  constexpr int RCH = 8;  // chunks per thread kept in registers
  __shared__ float red[8];
  const int row = blockIdx.x, tid = threadIdx.x, lane = tid & 63;
  const size_t base = (size_t)row * k;
  const int nch = k / 4;
  const bool in_regs = nch <= 512 * RCH;  // workgroup-uniform
  float v[RCH][4];
  float amax = 0.0f;
  if (in_regs) {
#pragma unroll
    for (int i = 0; i < RCH; i++) {
      if (tid + 512 * i < nch) ld_src4<SRC_F16>(w, base, tid + 512 * i, v[i]);
      else v[i][0] = v[i][1] = v[i][2] = v[i][3] = 0.0f;
    }
#pragma unroll
    for (int i = 0; i < RCH; i++)
#pragma unroll
      for (int t = 0; t < 4; t++) amax = fmaxf(amax, fabsf(v[i][t]));
  } else {
    for (int c = tid; c < nch; c += 512) {
      float u[4];
      ld_src4<SRC_F16>(w, base, c, u);
#pragma unroll
      for (int t = 0; t < 4; t++) amax = fmaxf(amax, fabsf(u[t]));
    }
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o));
  if (lane == 0) red[tid >> 6] = amax;
  __syncthreads();
  amax = red[0];
#pragma unroll
  for (int i = 1; i < 8; i++) amax = fmaxf(amax, red[i]);
  const float qmax = fmt == 1 ? 448.0f : fmt == 2 ? 57344.0f : 127.0f;
  const float sc = amax > 0.0f ? amax / qmax : 1.0f;
  if (tid == 0) row_scale[row] = sc;
  uint32_t* dst = reinterpret_cast<uint32_t*>(q + base);
  auto quant4 = [&](const float u[4]) -> uint32_t {
    const float v0 = u[0] / sc, v1 = u[1] / sc, v2 = u[2] / sc, v3 = u[3] / sc;
    if (fmt == 1) return fp8x4_from_f32<false>(v0, v1, v2, v3);
    if (fmt == 2) return fp8x4_from_f32<true>(v0, v1, v2, v3);
    const float vv[4] = {v0, v1, v2, v3};
    uint32_t r = 0;
#pragma unroll
    for (int t = 0; t < 4; t++) {
      const float rv = fminf(fmaxf(rintf(vv[t]), -127.0f), 127.0f);
      r |= ((uint32_t)(int)rv & 0xffu) << (8 * t);
    }
    return r;
  };
  if (in_regs) {
#pragma unroll
    for (int i = 0; i < RCH; i++)
      if (tid + 512 * i < nch) dst[tid + 512 * i] = quant4(v[i]);
  } else {
    for (int c = tid; c < nch; c += 512) {
      float u[4];
      ld_src4<SRC_F16>(w, base, c, u);
      dst[c] = quant4(u);
    }
  }
}

// INT4 with one f16 scale per 32 K-elements (amax/7): one thread per block.
__global__ void k_quant_int4_g32(const float* __restrict__ w, uint8_t* __restrict__ q,
                                 uint16_t* __restrict__ scales, size_t nblocks) {
  size_t b = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= nblocks) return;
  const float* src = w + b * 32;
  float amax = 0.0f;
  for (int j = 0; j < 32; j++) amax = fmaxf(amax, fabsf(src[j]));
  uint16_t sh = amax > 0.0f ? f32_to_f16_bits(amax / 7.0f) : (uint16_t)0x3c00u;
  float s = f16_bits_to_f32(sh);
  if (s == 0.0f) { sh = 0x3c00u; s = 1.0f; }
  scales[b] = sh;
  uint32_t words[4] = {0, 0, 0, 0};
  for (int j = 0; j < 32; j++) {
    float rv = fminf(fmaxf(rintf(src[j] / s), -8.0f), 7.0f);
    words[j / 8] |= ((uint32_t)(int)rv & 15u) << (4 * (j % 8));
  }
  reinterpret_cast<uint4*>(q)[b] = make_uint4(words[0], words[1], words[2], words[3]);
}

// ---------------------------------------------------------------------------
// Seeded normal generator (counter-based splitmix64 + Box-Muller).  Only
// synthetic-input plumbing; the CPU checker always consumes the exact
// tensors this produced.
__device__ __forceinline__ uint64_t splitmix64(uint64_t x) {
  x += 0x9E3779B97F4A7C15ull;
  x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
  x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
  return x ^ (x >> 31);
}

__global__ void k_fill_normal(void* __restrict__ dst, int dtype, size_t n, uint64_t seed,
                              float mean, float stddev) {
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;  // pair index
  size_t e = i * 2;
  if (e >= n) return;
  uint64_t r = splitmix64(seed * 0x2545F4914F6CDD1Dull + i);
  uint32_t a = (uint32_t)(r >> 40), c = (uint32_t)(r & 0xffffffu);
  float u1 = ((float)a + 1.0f) * (1.0f / 16777216.0f);  // (0, 1]
  float u2 = (float)c * (1.0f / 16777216.0f);           // [0, 1)
  float rad = sqrtf(-2.0f * logf(u1));
  float s, co;
  sincosf(6.283185307179586f * u2, &s, &co);
  float z0 = mean + stddev * rad * co, z1 = mean + stddev * rad * s;
  if (dtype == MX_DTYPE_F32) {
    float* o = reinterpret_cast<float*>(dst);
    o[e] = z0;
    if (e + 1 < n) o[e + 1] = z1;
  } else {
    uint16_t* o = reinterpret_cast<uint16_t*>(dst);
    o[e] = f32_to_f16_bits(z0);
    if (e + 1 < n) o[e + 1] = f32_to_f16_bits(z1);
  }
}

// ---------------------------------------------------------------------------
// Host launchers.
static inline unsigned grid_for(size_t items, unsigned block) {
  return (unsigned)((items + block - 1) / block);
}

hipError_t launch_pack(int fmt, const float* in, uint8_t* out, size_t n, hipStream_t st) {
  if (fmt == 0) {
    size_t items = (n + 7) / 8;
    hipLaunchKernelGGL(k_pack_fp4, dim3(grid_for(items, 256)), dim3(256), 0, st, in, out, n);
  } else {
    size_t items = (n + 3) / 4;
    if (fmt == 1)
      hipLaunchKernelGGL(k_pack_fp8<false>, dim3(grid_for(items, 256)), dim3(256), 0, st, in, out, n);
    else
      hipLaunchKernelGGL(k_pack_fp8<true>, dim3(grid_for(items, 256)), dim3(256), 0, st, in, out, n);
  }
  return hipGetLastError();
}

hipError_t launch_unpack(int fmt, const uint8_t* in, float* out, size_t n, hipStream_t st) {
  if (fmt == 0) {
    size_t items = (n + 7) / 8;
    hipLaunchKernelGGL(k_unpack_fp4, dim3(grid_for(items, 256)), dim3(256), 0, st, in, out, n);
  } else {
    size_t items = (n + 3) / 4;
    if (fmt == 1)
      hipLaunchKernelGGL(k_unpack_fp8<false>, dim3(grid_for(items, 256)), dim3(256), 0, st, in, out, n);
    else
      hipLaunchKernelGGL(k_unpack_fp8<true>, dim3(grid_for(items, 256)), dim3(256), 0, st, in, out, n);
  }
  return hipGetLastError();
}

hipError_t launch_mxfp4_quantize(const void* src, int src_dtype, uint8_t* packed, uint8_t* scales,
                                 size_t rows, size_t k, hipStream_t st) {
  size_t nblocks = rows * (k / 32);
  if (nblocks == 0) return hipSuccess;
  if (src_dtype == MX_DTYPE_F16)
    hipLaunchKernelGGL(k_mxfp4_quantize<true>, dim3(grid_for(nblocks, 256)), dim3(256), 0, st, src,
                       packed, scales, nblocks);
  else
    hipLaunchKernelGGL(k_mxfp4_quantize<false>, dim3(grid_for(nblocks, 256)), dim3(256), 0, st, src,
                       packed, scales, nblocks);
  return hipGetLastError();
}

hipError_t launch_mxfp4_dequant_f16(const uint8_t* packed, const uint8_t* scales, uint16_t* out,
                                    size_t rows, size_t depth, hipStream_t st) {
  const size_t nwords = rows * (depth / 32) * 4;
  if (nwords == 0) return hipSuccess;
  hipLaunchKernelGGL(k_mxfp4_dequant_f16, dim3(grid_for(nwords, 256)), dim3(256), 0, st, packed,
                     scales, out, nwords);
  return hipGetLastError();
}

hipError_t launch_swiglu(int variant, const void* gate, const void* up, void* mid, size_t count,
                         hipStream_t st) {
  if (count == 0) return hipSuccess;
  hipLaunchKernelGGL(k_swiglu, dim3(grid_for(count, 256)), dim3(256), 0, st, variant, gate, up, mid,
                     count);
  return hipGetLastError();
}

hipError_t launch_quant_rowwise(int fmt, const float* w, int rows, int k, uint8_t* q, float* scale,
                                hipStream_t st) {
  if (rows == 0) return hipSuccess;
  if (k % 4) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_quant_rowwise<false>, dim3(rows), dim3(512), 0, st, fmt, w, k, q, scale);
  return hipGetLastError();
}

// W8A8 activations: per-row INT8 with scale amax/127 (same arithmetic as
// the weight rows, so one oracle function covers both).  k % 4 == 0.
hipError_t launch_quant_act_int8(const void* x, int x_dtype, int rows, int k, int8_t* q,
                                 float* scale, hipStream_t st) {
  if (rows <= 0) return hipSuccess;
  if (k % 4) return hipErrorInvalidValue;
  if (x_dtype == MX_DTYPE_F16)
    hipLaunchKernelGGL(k_quant_rowwise<true>, dim3(rows), dim3(512), 0, st, 3, x, k,
                       reinterpret_cast<uint8_t*>(q), scale);
  else
    hipLaunchKernelGGL(k_quant_rowwise<false>, dim3(rows), dim3(512), 0, st, 3, x, k,
                       reinterpret_cast<uint8_t*>(q), scale);
  return hipGetLastError();
}

hipError_t launch_quant_int4_g32(const float* w, size_t rows, size_t k, uint8_t* q,
                                 uint16_t* scales, hipStream_t st) {
  size_t nblocks = rows * (k / 32);
  if (nblocks == 0) return hipSuccess;
  hipLaunchKernelGGL(k_quant_int4_g32, dim3(grid_for(nblocks, 256)), dim3(256), 0, st, w, q, scales,
                     nblocks);
  return hipGetLastError();
}

hipError_t launch_fill_normal(void* dst, int dtype, size_t n, uint64_t seed, float mean,
                              float stddev, hipStream_t st) {
  size_t items = (n + 1) / 2;
  if (items == 0) return hipSuccess;
  hipLaunchKernelGGL(k_fill_normal, dim3(grid_for(items, 256)), dim3(256), 0, st, dst, dtype, n,
                     seed, mean, stddev);
  return hipGetLastError();
}

// f16 [M][K] -> F8X2 (layout in mx_internal.h, split rule at
// f8x2_split_store): 4 lanes per (row, 64-K group), 16 values (two 16-byte
// loads) per lane; a group past the end exits as a whole.  Measured at
// T = 512, K = 7168 (split kernel alone, back to back): 2 lanes per group
// 7.6 us, 4 lanes 4.3 us, 8 lanes 4.8 us, 16 lanes 6.2 us.
__global__ void k_split_f8x2(const uint16_t* x, int m, int k, uint8_t* data, uint32_t* e8) {
  const size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int j = (int)(t & 3);
  const int groups = k / 64;
  const size_t gi = t >> 2;
  if (gi >= (size_t)m * groups) return;
  const int row = (int)(gi / groups), grp = (int)(gi % groups);
  const uint16_t* src = x + (size_t)row * k + (size_t)grp * 64 + 16 * j;
  float v[16];
#pragma unroll
  for (int q = 0; q < 2; q++) {
    const uint4 w = *reinterpret_cast<const uint4*>(src + 8 * q);
    const uint32_t d[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int e = 0; e < 4; e++) {
      v[8 * q + 2 * e] = f16_bits_to_f32((uint16_t)(d[e] & 0xffffu));
      v[8 * q + 2 * e + 1] = f16_bits_to_f32((uint16_t)(d[e] >> 16));
    }
  }
  f8x2_split_store<4>(v, j, data + (size_t)row * 2 * k + (size_t)grp * 128, e8 + (size_t)grp * m + row);
}

hipError_t launch_split_f8x2(const uint16_t* x, int m, int k, uint8_t* data, uint32_t* e8, hipStream_t st) {
  if (m <= 0 || k <= 0 || k % 64) return hipErrorInvalidValue;
  const size_t threads = (size_t)m * (k / 64) * 4;
  hipLaunchKernelGGL(k_split_f8x2, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, st, x, m, k, data, e8);
  return hipGetLastError();
}

}  // namespace mx
