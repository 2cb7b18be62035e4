// mx_gemm_fp4.hip - W4A4 MXFP4 x MXFP4 GEMM on the gfx950 scaled MFMA.
//
//   C[m][n] = sum_kb 2^(SA[m][kb]-127) 2^(SB[n][kb]-127) sum_{k in kb} A[m][k] B[n][k]
//
// This is what the reference's native scale-plane matmul
// (MXFP4Kernels.metal:138-173: matmul2d consuming FP4 data + E8M0 plane)
// becomes when the left operand is MXFP4 too.  The
// hardware instruction v_mfma_scale_f32_32x32x64_f8f6f4 takes one E8M0 byte
// per lane and operand, and on gfx950 lane l of a 32x32x64 FP4 operand holds
// exactly row l%32, block l/32 - so the block scale is applied per 32-K block
// in hardware with no per-block accumulator juggling (the cost the
// reference's fused per-block form pays, README.md:309-312).
//
// Tiling: 256 threads (4 wave64, 2 x 2), workgroup tile 256 (M) x BN (rows
// of B, 128 or 256), K stage 128 (two MFMA K-steps of 64).  Each wave owns a
// 128 x BN/2 accumulator tile = 4 x BN/64 MFMA blocks.  Operand tiles live in
// LDS "fragment-major": the 16 bytes lane l feeds to one MFMA sit at offset
// 16*l of a 1 KB fragment, so every ds_read_b128 is contiguous across the
// wave and conflict-free, and every global load of a stage writes LDS at
// 16*thread.  Double-buffered LDS with register prefetch: the next stage's
// global loads are in flight during the current stage's MFMAs; one barrier
// per stage.  All loads are unconditional - rows past M read row M-1 and
// their results are never stored - because a predicated load makes the
// compiler wait for it at the join.  Scale dwords (4 blocks = 2 K-steps) are
// loaded per lane and shifted by 8*(lane/32) so that a uniform opsel (byte 0
// for K-step 0, byte 2 for K-step 1) picks the lane's own block.
//
// Epilogues:
//   DUAL=false  store C as f16 [M][N]                            (down proj)
//   DUAL=true   B rows [0,BN/2) are gate rows, [BN/2,BN) the same up rows;
//               mid = silu(g) * u is re-quantized to MXFP4 along N (the
//               next GEMM's K) through LDS: one lane per (row, 32-column
//               block) computes amax -> E8M0 -> 16 packed bytes + 1 scale.
//
// Workgroup order is XCD-aware: consecutive workgroup ids are dealt round-
// robin to the 8 XCDs, so the id is remapped to give each XCD a contiguous
// range of tiles, walked in groups of 8 N-tiles x all M-tiles so the 32 CUs
// of an XCD share A and B panels in their L2.
#include "mx_device.h"
#include "mx_internal.h"

namespace mx {

constexpr int kFBM = 256, kFBK = 128;  // tile M, K per stage (elements)
constexpr int kAFrag = kFBM / 32 * 2;  // A fragments per stage (8 m-blocks x 2 k-steps)
constexpr int kMidLdsStride = 33;      // floats per row in the requant tile

__device__ __forceinline__ int xcd_remap(int bid, int nblocks) {
  // Hardware deals workgroups round-robin over 8 XCDs.  Give XCD x the
  // contiguous tile range [x*per, (x+1)*per) when nblocks % 8 == 0.
  if (nblocks % 8 != 0) return bid;
  const int per = nblocks / 8;
  return (bid % 8) * per + bid / 8;
}

template <bool DUAL, int BN>
__global__ __launch_bounds__(256, 1) void k_gemm_fp4(Fp4GemmArgs g) {
  constexpr int J = BN / 64;               // n-blocks per wave
  constexpr int BCH = BN / 64;             // B chunks per thread per stage
  constexpr int kBFrag = BN / 32 * 2;
  constexpr int kStage = (kAFrag + kBFrag) * 1024;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave & 1, wn = wave >> 1;
  const int M = g.m, K = g.k;
  const int MT = (M + kFBM - 1) / kFBM;
  const int NT = DUAL ? g.n / (BN / 2) : g.n / BN;  // tiles along N

  // Tile order: XCD remap, then groups of 8 N-tiles with M fastest inside.
  const int tile = xcd_remap(blockIdx.x, MT * NT);
  const int group_sz = 8 * MT;
  const int grp = tile / group_sz, in_grp = tile % group_sz;
  const int nt_base = grp * 8;
  const int gw = min(8, NT - nt_base);
  const int mt = in_grp / gw, nt = nt_base + in_grp % gw;
  const int m0 = mt * kFBM;

  const size_t row_bytes = (size_t)K / 2, row_blocks = (size_t)K / 32;

  // Global source of each chunk this thread stages: chunk c = tid + 256u,
  // fragment f = c/64 (block f/2, k-step f%2), fragment lane fl = c%64.
  const uint8_t* a_src[4];
#pragma unroll
  for (int u = 0; u < 4; u++) {
    const int c = tid + 256 * u, f = c >> 6, fl = c & 63;
    const int row = min(m0 + (f >> 1) * 32 + (fl & 31), M - 1);
    a_src[u] = g.a + (size_t)row * row_bytes + (f & 1) * 32 + (fl >> 5) * 16;
  }
  const uint8_t* b_src[BCH];
#pragma unroll
  for (int u = 0; u < BCH; u++) {
    const int c = tid + 256 * u, f = c >> 6, fl = c & 63;
    const int j = f >> 1;  // n-block of the tile
    const uint8_t* base;
    int row;
    if (DUAL) {
      base = j < J ? g.b0 : g.b1;
      row = nt * (BN / 2) + (j % J) * 32 + (fl & 31);
    } else {
      base = g.b0;
      row = nt * BN + j * 32 + (fl & 31);
    }
    b_src[u] = base + (size_t)row * row_bytes + (f & 1) * 32 + (fl >> 5) * 16;
  }
  // Scale rows of this lane's MFMA operands.
  const int srow_sub = lane & 31, shift = 8 * (lane >> 5);
  const uint8_t* as_src[4];
#pragma unroll
  for (int i = 0; i < 4; i++)
    as_src[i] = g.as + (size_t)min(m0 + wm * 128 + i * 32 + srow_sub, M - 1) * row_blocks;
  const uint8_t* bs_src[J];
  int bfrag[J];  // which tile n-block feeds the wave's j-th accumulator column
#pragma unroll
  for (int j = 0; j < J; j++) {
    if (DUAL) {
      // j < J/2: gate blocks wn*J/2 + j ; j >= J/2: the matching up blocks
      const int gb = wn * (J / 2) + (j % (J / 2));
      bfrag[j] = j < J / 2 ? gb : J + gb;
      const uint8_t* sb = j < J / 2 ? g.s0 : g.s1;
      bs_src[j] = sb + (size_t)(nt * (BN / 2) + gb * 32 + srow_sub) * row_blocks;
    } else {
      bfrag[j] = wn * J + j;
      bs_src[j] = g.s0 + (size_t)(nt * BN + (wn * J + j) * 32 + srow_sub) * row_blocks;
    }
  }

  v16f acc[4][J];
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int j = 0; j < J; j++)
#pragma unroll
      for (int v = 0; v < 16; v++) acc[i][j][v] = 0.0f;

  const int KT = K / kFBK;
  uint4 ar[4], br[BCH];
  uint32_t asr[4], bsr[J], sa_cur[4], sb_cur[J];

  // Stage 0.
#pragma unroll
  for (int u = 0; u < 4; u++) ar[u] = *reinterpret_cast<const uint4*>(a_src[u]);
#pragma unroll
  for (int u = 0; u < BCH; u++) br[u] = *reinterpret_cast<const uint4*>(b_src[u]);
#pragma unroll
  for (int i = 0; i < 4; i++) sa_cur[i] = *reinterpret_cast<const uint32_t*>(as_src[i]) >> shift;
#pragma unroll
  for (int j = 0; j < J; j++) sb_cur[j] = *reinterpret_cast<const uint32_t*>(bs_src[j]) >> shift;
#pragma unroll
  for (int u = 0; u < 4; u++) *reinterpret_cast<uint4*>(smem + (tid + 256 * u) * 16) = ar[u];
#pragma unroll
  for (int u = 0; u < BCH; u++)
    *reinterpret_cast<uint4*>(smem + kAFrag * 1024 + (tid + 256 * u) * 16) = br[u];
  __syncthreads();

  for (int kt = 0; kt < KT; kt++) {
    const int buf = kt & 1;
    const bool more = kt + 1 < KT;
    // Prefetch the next stage (the last stage re-reads itself: unconditional).
    {
      const size_t koff = (size_t)(more ? kt + 1 : kt) * (kFBK / 2);
      const size_t soff = (size_t)(more ? kt + 1 : kt) * 4;
#pragma unroll
      for (int u = 0; u < 4; u++) ar[u] = *reinterpret_cast<const uint4*>(a_src[u] + koff);
#pragma unroll
      for (int u = 0; u < BCH; u++) br[u] = *reinterpret_cast<const uint4*>(b_src[u] + koff);
#pragma unroll
      for (int i = 0; i < 4; i++) asr[i] = *reinterpret_cast<const uint32_t*>(as_src[i] + soff);
#pragma unroll
      for (int j = 0; j < J; j++) bsr[j] = *reinterpret_cast<const uint32_t*>(bs_src[j] + soff);
    }
    const uint8_t* base = smem + buf * kStage;
#pragma unroll
    for (int ks = 0; ks < 2; ks++) {
      v4i af[4], bf[J];
#pragma unroll
      for (int i = 0; i < 4; i++)
        af[i] = *reinterpret_cast<const v4i*>(base + (((wm * 4 + i) * 2 + ks) * 64 + lane) * 16);
#pragma unroll
      for (int j = 0; j < J; j++)
        bf[j] = *reinterpret_cast<const v4i*>(base + kAFrag * 1024 + ((bfrag[j] * 2 + ks) * 64 + lane) * 16);
#pragma unroll
      for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < J; j++) {
          if (ks == 0)
            acc[i][j] = mfma_fp4_32x32x64<0, 0>(af[i], bf[j], acc[i][j], (int)sa_cur[i], (int)sb_cur[j]);
          else
            acc[i][j] = mfma_fp4_32x32x64<2, 2>(af[i], bf[j], acc[i][j], (int)sa_cur[i], (int)sb_cur[j]);
        }
    }
    uint8_t* nbase = smem + (buf ^ 1) * kStage;
#pragma unroll
    for (int u = 0; u < 4; u++) *reinterpret_cast<uint4*>(nbase + (tid + 256 * u) * 16) = ar[u];
#pragma unroll
    for (int u = 0; u < BCH; u++)
      *reinterpret_cast<uint4*>(nbase + kAFrag * 1024 + (tid + 256 * u) * 16) = br[u];
#pragma unroll
    for (int i = 0; i < 4; i++) sa_cur[i] = asr[i] >> shift;
#pragma unroll
    for (int j = 0; j < J; j++) sb_cur[j] = bsr[j] >> shift;
    __syncthreads();
  }

  if (!DUAL) {
    uint16_t* c = reinterpret_cast<uint16_t*>(g.c);
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
      for (int j = 0; j < J; j++) {
        const int col = nt * BN + (wn * J + j) * 32 + (lane & 31);
#pragma unroll
        for (int v = 0; v < 16; v++) {
          const int row = m0 + wm * 128 + i * 32 + acc32_row(lane, v);
          if (row < M) c[(size_t)row * g.n + col] = f32_to_f16_bits(acc[i][j][v]);
        }
      }
    return;
  }

  // DUAL: mid = silu(gate) * up for each of the wave's J/2 channel blocks,
  // staged per wave in LDS (64 rows x 33 floats at a time), then
  // re-quantized to MXFP4 along the channel axis.
  float* mid = reinterpret_cast<float*>(smem) + wave * (64 * kMidLdsStride);
  uint8_t* mp = reinterpret_cast<uint8_t*>(g.c);
  const size_t mid_row_bytes = (size_t)g.n / 2, mid_row_blocks = (size_t)g.n / 32;
#pragma unroll
  for (int jb = 0; jb < J / 2; jb++) {
    const int chan0 = nt * (BN / 2) + (wn * (J / 2) + jb) * 32;
#pragma unroll
    for (int h = 0; h < 2; h++) {
#pragma unroll
      for (int i2 = 0; i2 < 2; i2++)
#pragma unroll
        for (int v = 0; v < 16; v++) {
          const int r = i2 * 32 + acc32_row(lane, v);
          const float gv = acc[2 * h + i2][jb][v], uv = acc[2 * h + i2][J / 2 + jb][v];
          mid[r * kMidLdsStride + (lane & 31)] = silu(gv) * uv;
        }
      __syncthreads();
      const int row = m0 + wm * 128 + h * 64 + lane;
      float v[32];
      uint32_t amax = 0;
#pragma unroll
      for (int j = 0; j < 32; j++) {
        v[j] = mid[lane * kMidLdsStride + j];
        amax = max(amax, abs_bits(v[j]));
      }
      const uint32_t sb = mxfp4_scale_byte(amax);
      uint4 o = make_uint4(0, 0, 0, 0);
      if (sb != 255u) {
        o.x = fp4x8_from_f32(v + 0, sb);
        o.y = fp4x8_from_f32(v + 8, sb);
        o.z = fp4x8_from_f32(v + 16, sb);
        o.w = fp4x8_from_f32(v + 24, sb);
      }
      if (row < M) {
        *reinterpret_cast<uint4*>(mp + (size_t)row * mid_row_bytes + chan0 / 2) = o;
        g.cs[(size_t)row * mid_row_blocks + chan0 / 32] = (uint8_t)sb;
      }
      __syncthreads();
    }
  }
}

template <bool DUAL, int BN>
static hipError_t launch_bn(const Fp4GemmArgs& g, hipStream_t st) {
  constexpr int kStage = (kAFrag + BN / 32 * 2) * 1024;
  const int MT = (g.m + kFBM - 1) / kFBM;
  const int NT = DUAL ? g.n / (BN / 2) : g.n / BN;
  const int lds_mid = 4 * 64 * kMidLdsStride * 4;  // reuses the tile buffers
  const int lds = 2 * kStage > lds_mid ? 2 * kStage : lds_mid;
  hipLaunchKernelGGL((k_gemm_fp4<DUAL, BN>), dim3(MT * NT), dim3(256), lds, st, g);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// E8M0 byte 255 in a down-weight scale.  The reference decodes it as +inf
// (bits << 23, MXFP4Kernels.metal:26-29), so in its dequantize-then-
// accumulate a block with that scale contributes +-inf when every weight
// code of the block and every mid value it meets are non-zero and all those
// products share one sign, and NaN otherwise (0 * inf, or +inf + -inf).
// The scaled MFMA reads 255 as NaN, so the down GEMM leaves NaN in every
// output of such a row.  This pass rewrites the +-inf cases.  One workgroup
// per 16 down rows reads their scale bytes and returns when none is 255 -
// the whole cost in the common case is one read of the down scale plane.
// (Byte 255 in a gate or up scale needs no pass: the channel's mid is then
// non-finite on both sides, its block re-quantizes to byte 255 with zero
// codes, and every output of the token is NaN on both sides.)
// ms_stage_major: mid scales [I/128][tpad][4] bytes, else [T][I/32].
__global__ __launch_bounds__(256) void k_w4a4_down_inf(const uint8_t* __restrict__ wd, const uint8_t* __restrict__ sd,
                                                      const uint8_t* __restrict__ mq, const uint8_t* __restrict__ ms,
                                                      int ms_stage_major, int tpad, uint16_t* __restrict__ out,
                                                      int T, int H, int I) {
  const int KB = I / 32, r0 = blockIdx.x * 16;
  const int rows = min(16, H - r0);
  __shared__ int any;
  if (threadIdx.x == 0) any = 0;
  __syncthreads();
  bool hit = false;
  for (int i = threadIdx.x; i < rows * (KB / 4); i += blockDim.x) {
    const uint32_t d = ~*reinterpret_cast<const uint32_t*>(sd + (size_t)(r0 + i / (KB / 4)) * KB + (i % (KB / 4)) * 4);
    hit = hit || ((d - 0x01010101u) & ~d & 0x80808080u) != 0;
  }
  if (hit) any = 1;  // every writer stores the same value
  __syncthreads();
  if (!any) return;  // workgroup-uniform
  auto mid_scale = [&](int m, int b) -> uint32_t {
    return ms_stage_major ? ms[((size_t)(b >> 2) * tpad + m) * 4 + (b & 3)] : ms[(size_t)m * KB + b];
  };
  for (int rr = 0; rr < rows; rr++) {
    const int h = r0 + rr;
    const uint8_t* srow = sd + (size_t)h * KB;
    const uint8_t* wrow = wd + (size_t)h * (I / 2);
    for (int m = threadIdx.x; m < T; m += blockDim.x) {
      bool inf_row = false, finite = true;
      uint32_t sign = 0, seen = 0;  // seen: 1 = a positive, 2 = a negative infinite product
      for (int b = 0; b < KB && finite; b++) {
        if (mid_scale(m, b) == 255u) finite = false;  // mid not finite: NaN on both sides
        if (srow[b] != 255u) continue;
        inf_row = true;
        const uint8_t* mrow = mq + (size_t)m * (I / 2) + b * 16;
        for (int j = 0; j < 16 && finite; j++) {
          const uint32_t wb = wrow[b * 16 + j], mb = mrow[j];
#pragma unroll
          for (int h2 = 0; h2 < 2; h2++) {
            const uint32_t wc = (wb >> (4 * h2)) & 15u, mc = (mb >> (4 * h2)) & 15u;
            if ((wc & 7u) == 0 || (mc & 7u) == 0) finite = false;  // 0 * inf
            sign = (wc ^ mc) & 8u;
            seen |= sign ? 2u : 1u;
          }
        }
      }
      if (inf_row && finite && seen != 3u) out[(size_t)m * H + h] = seen == 2u ? 0xfc00u : 0x7c00u;
    }
  }
}

hipError_t launch_w4a4_down_inf(const uint8_t* wd, const uint8_t* sd, const uint8_t* mq, const uint8_t* ms,
                                int ms_stage_major, int t, int h, int i, uint16_t* out, hipStream_t st) {
  const int tpad = (int)stage_major_rows(t);
  hipLaunchKernelGGL(k_w4a4_down_inf, dim3((h + 15) / 16), dim3(256), 0, st, wd, sd, mq, ms, ms_stage_major, tpad,
                     out, t, h, i);
  return hipGetLastError();
}

// Preconditions (caller): k % 128 == 0; DUAL: n % 64 == 0; else n % 128 == 0.
// Stage-major scale planes go to the 256 x 256 streaming kernel
// (mx_gemm_fp4_v3.hip); reference-layout planes to the kernel above.
hipError_t launch_gemm_fp4(int dual, const Fp4GemmArgs& g, hipStream_t st) {
  if (g.stage_major == 2) return launch_gemm_fp4_v6(dual, g, st);
  if (g.stage_major) return gemm_fp4_v5_ok(g.k) ? launch_gemm_fp4_v5(dual, g, st) : launch_gemm_fp4_v3(dual, g, st);
  if (dual) return launch_bn<true, 128>(g, st);
  return launch_bn<false, 128>(g, st);
}

}  // namespace mx
