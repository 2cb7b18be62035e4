// mx_gemv.hip - decode-shaped (tokens <= 16) MXFP4 GEMV with split-K.
//
// The reference runs every shape through the same 64 x NT matmul2d tile
// (MXFP4Kernels.metal:138-173) and only for tokens % 64 == 0
// (main.swift:946).  On MI355X a 1..16-token MLP is bound by HBM: the whole
// job is streaming 4-bit weights once.  This kernel is built for that:
//
//   unit  = one wave64 = 16 weight rows x (K / splits) of the reduction
//   lane  = (row n = lane % 16, block group g = lane / 16); per 128-K step
//           it loads 16 contiguous bytes of its row (one whole 32-element
//           E8M0 block) plus that block's scale byte, decodes them with
//           v_cvt_scalef32_pk_f16_fp4 and feeds v_mfma_f32_16x16x32_f16
//           (tokens padded to 16 rows; the MFMA is never the bottleneck).
//           The activations use the same K permutation, so each lane reads
//           64 contiguous bytes of x per step (L2-resident).
//   split = partial sums go to a workspace; the last wave of a row group
//           (atomic counter, self-resetting) adds the partials in split
//           order - deterministic - and applies the epilogue:
//             single: out = f16(sum)
//             dual:   mid = f16(silu(sum_gate) * sum_up)   (swiglu_float)
//
// Loads are issued four K steps at a time per lane (64-128 B in flight per
// lane) so that each CU keeps tens of KB of HBM requests outstanding.
#include "mx_device.h"
#include "mx_internal.h"

namespace mx {

constexpr int kGroupRows = 16;
constexpr int kStepK = 128;   // K per lane step: 4 lane groups x 32-element blocks
constexpr int kBatch = 4;     // steps whose loads are issued together

template <bool DUAL>
__global__ __launch_bounds__(256) void k_gemv_mxfp4(GemvArgs g) {
  const int lane = threadIdx.x & 63;
  const int unit = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int groups = g.n / kGroupRows;
  if (unit >= groups * g.splits) return;
  const int grp = unit % groups, split = unit / groups;
  const int n = grp * kGroupRows + (lane & 15);
  const int lg = lane >> 4;                    // block within the 128-K step
  const int tok = lane & 15;                   // activation row this lane feeds
  const int K = g.k, T = g.t;
  const int steps = K / kStepK / g.splits;
  const int step0 = split * steps;
  const size_t row_bytes = (size_t)K / 2, row_blocks = (size_t)K / 32;

  const uint8_t* w0 = g.b0 + (size_t)n * row_bytes + lg * 16;
  const uint8_t* sc0 = g.s0 + (size_t)n * row_blocks + lg;
  const uint8_t* w1 = DUAL ? g.b1 + (size_t)n * row_bytes + lg * 16 : nullptr;
  const uint8_t* sc1 = DUAL ? g.s1 + (size_t)n * row_blocks + lg : nullptr;
  const bool has_tok = tok < T;
  const uint16_t* xr = g.x + (size_t)(has_tok ? tok : 0) * K + lg * 32;

  v4f acc0 = {0, 0, 0, 0}, acc1 = {0, 0, 0, 0};
  for (int s0 = 0; s0 < steps; s0 += kBatch) {
    uint4 wv0[kBatch], wv1[kBatch];
    uint32_t sb0[kBatch], sb1[kBatch];
    uint4 xv[kBatch][4];
#pragma unroll
    for (int b = 0; b < kBatch; b++) {
      const int st = step0 + s0 + b;
      if (s0 + b < steps) {
        wv0[b] = *reinterpret_cast<const uint4*>(w0 + (size_t)st * 64);
        sb0[b] = sc0[(size_t)st * 4];
        if (DUAL) {
          wv1[b] = *reinterpret_cast<const uint4*>(w1 + (size_t)st * 64);
          sb1[b] = sc1[(size_t)st * 4];
        }
#pragma unroll
        for (int q = 0; q < 4; q++)
          xv[b][q] = has_tok ? *reinterpret_cast<const uint4*>(xr + (size_t)st * kStepK + q * 8)
                             : make_uint4(0, 0, 0, 0);
      }
    }
#pragma unroll
    for (int b = 0; b < kBatch; b++) {
      if (s0 + b < steps) {
        const uint32_t wd0[4] = {wv0[b].x, wv0[b].y, wv0[b].z, wv0[b].w};
        uint32_t wd1[4];
        if (DUAL) {
          wd1[0] = wv1[b].x; wd1[1] = wv1[b].y; wd1[2] = wv1[b].z; wd1[3] = wv1[b].w;
        }
#pragma unroll
        for (int q = 0; q < 4; q++) {
          const v8h a = __builtin_bit_cast(v8h, xv[b][q]);
          acc0 = mfma_f16_16x16x32(a, fp4x8_dequant_f16(wd0[q], sb0[b]), acc0);
          if (DUAL) acc1 = mfma_f16_16x16x32(a, fp4x8_dequant_f16(wd1[q], sb1[b]), acc1);
        }
      }
    }
  }
  // acc element v: token row (lane/16)*4 + v, weight row n.
  const int col_stride = DUAL ? 2 * g.n : g.n;
  if (g.splits == 1) {
#pragma unroll
    for (int v = 0; v < 4; v++) {
      const int t = (lane >> 4) * 4 + v;
      if (t >= T) continue;
      float r;
      if (DUAL) r = silu(acc0[v]) * acc1[v];
      else r = acc0[v];
      g.out[(size_t)t * g.n + n] = f32_to_f16_bits(r);
    }
    return;
  }
  float* part = g.partial + (size_t)split * T * col_stride;
#pragma unroll
  for (int v = 0; v < 4; v++) {
    const int t = (lane >> 4) * 4 + v;
    if (t >= T) continue;
    part[(size_t)t * col_stride + n] = acc0[v];
    if (DUAL) part[(size_t)t * col_stride + g.n + n] = acc1[v];
  }
  __threadfence();
  uint32_t prev = 0;
  if (lane == 0) prev = atomicAdd(&g.counters[grp], 1u);
  prev = __shfl(prev, 0);
  if (prev != (uint32_t)(g.splits - 1)) return;
  __threadfence();
#pragma unroll
  for (int v = 0; v < 4; v++) {
    const int t = (lane >> 4) * 4 + v;
    if (t >= T) continue;
    float s0 = 0.0f, s1 = 0.0f;
    for (int s = 0; s < g.splits; s++) {
      const float* p = g.partial + (size_t)s * T * col_stride + (size_t)t * col_stride;
      s0 += p[n];
      if (DUAL) s1 += p[g.n + n];
    }
    float r = DUAL ? silu(s0) * s1 : s0;
    g.out[(size_t)t * g.n + n] = f32_to_f16_bits(r);
  }
  if (lane == 0) atomicExch(&g.counters[grp], 0u);
}

// Splits: as many as keep ~8 waves per CU busy while dividing the K steps.
int gemv_pick_splits(int n, int k, int dual) {
  (void)dual;
  const int groups = n / kGroupRows;
  const int steps = k / kStepK;
  const int target = (2048 + groups - 1) / groups;
  int best = 1;
  for (int s = 1; s <= steps && s <= 64; s++)
    if (steps % s == 0 && s <= target) best = s;
  return best;
}

size_t gemv_partial_floats(int t, int n, int splits, int dual) {
  return (size_t)splits * t * n * (dual ? 2 : 1);
}

// Preconditions (caller): 1 <= t <= 16, n % 16 == 0, k % 128 == 0,
// (k/128) % splits == 0; counters zeroed once before first use.
hipError_t launch_gemv_mxfp4(int dual, const GemvArgs& g, hipStream_t st) {
  const int units = (g.n / kGroupRows) * g.splits;
  dim3 grid((units + 3) / 4);
  if (dual) hipLaunchKernelGGL(k_gemv_mxfp4<true>, grid, dim3(256), 0, st, g);
  else hipLaunchKernelGGL(k_gemv_mxfp4<false>, grid, dim3(256), 0, st, g);
  return hipGetLastError();
}

}  // namespace mx
