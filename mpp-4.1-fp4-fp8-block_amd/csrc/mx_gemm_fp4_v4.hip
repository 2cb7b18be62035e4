// mx_gemm_fp4_v4.hip - the W4A4 prefill GEMM with a 4-slot LDS ring (three
// K stages in flight), for K a multiple of 512.  Same tile, fragment layout,
// stage-major scales and epilogues as the 2-slot kernel in
// mx_gemm_fp4_v3.hip; what changes is the pipeline:
//
//   iteration k:  wait until this wave's DMA of stage k+1 has landed
//                 (vmcnt leaves stages k+2, k+3 in flight), s_barrier,
//                 DMA stage k+4 into the slot stage k occupied,
//                 32 MFMAs on stage k (already in VGPRs) interleaved with the
//                 ds_reads of stage k+1 into the other VGPR set.
//
// Two details make the compiler keep that overlap:
//   * the ring is four separate __shared__ arrays addressed with constant
//     slot numbers (the loop is unrolled by 4), so the backend can tell that
//     a read of one slot does not depend on DMA into another and does not
//     force vmcnt(0) before it;
//   * the stage barrier is a bare s_barrier.  __syncthreads() also fences
//     memory, which makes the backend wait for every outstanding load first.
//     Only LDS is shared through the barrier: each wave waits for its own DMA
//     (vmcnt) and for its own ds_reads (lgkmcnt) before arriving.
// Every wave issues exactly 10 DMA instructions per stage (8 x 1 KB operand
// fragments, 2 x 256 B of scales), so one vmcnt constant fits all waves.
#include "mx_device.h"
#include "mx_internal.h"

namespace mx {
namespace {

constexpr int kM = 256, kKS = 128, kNS = 4;
constexpr int kFrag = 16;
constexpr int kSlotData = 2 * kFrag * 1024;
constexpr int kSlot = kSlotData + 2048;
constexpr int kMidStride = 33;
constexpr int kDmaPerStage = 10;

__shared__ __attribute__((aligned(16))) uint8_t ring0[kSlot];
__shared__ __attribute__((aligned(16))) uint8_t ring1[kSlot];
__shared__ __attribute__((aligned(16))) uint8_t ring2[kSlot];
__shared__ __attribute__((aligned(16))) uint8_t ring3[kSlot];

template <int J>
__device__ __forceinline__ uint8_t* ring() {
  if constexpr (J == 0) return ring0;
  else if constexpr (J == 1) return ring1;
  else if constexpr (J == 2) return ring2;
  else return ring3;
}

// s_waitcnt immediate (gfx9 encoding): lgkmcnt(0), expcnt untouched, vmcnt(n).
constexpr int wait_lgkm0_vm(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4); }

__device__ __forceinline__ int xcd_tile(int bid, int nblocks) {
  if (nblocks % 8 != 0) return bid;
  const int per = nblocks / 8;
  return (bid % 8) * per + bid / 8;
}

template <bool DUAL>
__global__ __launch_bounds__(256, 1) void k_gemm_fp4_v4(Fp4GemmArgs g) {
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave & 1, wn = wave >> 1;
  const int M = g.m, K = g.k;
  const int MT = (M + kM - 1) / kM;
  const int NT = DUAL ? g.n / 128 : g.n / 256;
  const size_t Mpad = stage_major_rows(M);
  const size_t NB = (size_t)g.n;

  const int tile = xcd_tile(blockIdx.x, MT * NT);
  const int group_sz = 8 * MT;
  const int grp = tile / group_sz, in_grp = tile % group_sz;
  const int nt_base = grp * 8;
  const int gw = min(8, NT - nt_base);
  const int mt = in_grp / gw, nt = nt_base + in_grp % gw;
  const int m0 = mt * kM;
  const size_t row_bytes = (size_t)K / 2;

  const uint8_t* a_src[4];
  const uint8_t* b_src[4];
#pragma unroll
  for (int u = 0; u < 4; u++) {
    const int f = wave * 4 + u, blk = f >> 1, ks = f & 1;
    const int arow = min(m0 + blk * 32 + (lane & 31), M - 1);
    a_src[u] = g.a + (size_t)arow * row_bytes + ks * 32 + (lane >> 5) * 16;
    const uint8_t* bb;
    int brow;
    if (DUAL) {
      bb = blk < 4 ? g.b0 : g.b1;
      brow = nt * 128 + (blk & 3) * 32 + (lane & 31);
    } else {
      bb = g.b0;
      brow = nt * 256 + blk * 32 + (lane & 31);
    }
    b_src[u] = bb + (size_t)brow * row_bytes + ks * 32 + (lane >> 5) * 16;
  }
  // Scales: the stage's 512 dwords (256 A rows, then 256 B tile rows) are
  // split in 128-dword quarters, one per wave, as two 64-lane dword DMAs.
  const uint8_t* s_src;
  size_t s_stage;
  if (wave < 2) {
    s_src = g.as + (size_t)(m0 + wave * 128 + lane) * 4;
    s_stage = Mpad * 4;
  } else if (DUAL) {
    s_src = (wave == 2 ? g.s0 : g.s1) + (size_t)(nt * 128 + lane) * 4;
    s_stage = NB * 4;
  } else {
    s_src = g.s0 + (size_t)(nt * 256 + (wave - 2) * 128 + lane) * 4;
    s_stage = NB * 4;
  }

  int bfrag[4];
#pragma unroll
  for (int j = 0; j < 4; j++) {
    if (DUAL) bfrag[j] = j < 2 ? wn * 2 + (j & 1) : 4 + wn * 2 + (j & 1);
    else bfrag[j] = wn * 4 + j;
  }
  const int shift = 8 * (lane >> 5);
  // per-lane LDS byte offsets of the operand reads
  int a_off[2][4], b_off[2][4], sa_off[4], sb_off[4];
#pragma unroll
  for (int ks = 0; ks < 2; ks++)
#pragma unroll
    for (int i = 0; i < 4; i++) {
      a_off[ks][i] = (((wm * 4 + i) * 2 + ks) * 64 + lane) * 16;
      b_off[ks][i] = ((kFrag + bfrag[i] * 2 + ks) * 64 + lane) * 16;
    }
#pragma unroll
  for (int i = 0; i < 4; i++) {
    sa_off[i] = kSlotData + (wm * 128 + i * 32 + (lane & 31)) * 4;
    sb_off[i] = kSlotData + 1024 + (bfrag[i] * 32 + (lane & 31)) * 4;
  }

  v16f acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int j = 0; j < 4; j++)
#pragma unroll
      for (int v = 0; v < 16; v++) acc[i][j][v] = 0.0f;

  v4i af[2][2][4], bf[2][2][4];
  uint32_t sa[2][4], sb[2][4];
  const int KT = K / kKS;

#define MX4_ISSUE(S, SP)                                                                              \
  {                                                                                                   \
    const size_t koff_ = (size_t)(S) * (kKS / 2);                                                     \
    _Pragma("unroll") for (int u = 0; u < 4; u++)                                                     \
      __builtin_amdgcn_global_load_lds(a_src[u] + koff_, (SP) + (wave * 4 + u) * 1024, 16, 0, 0);     \
    _Pragma("unroll") for (int u = 0; u < 4; u++)                                                     \
      __builtin_amdgcn_global_load_lds(b_src[u] + koff_, (SP) + (kFrag + wave * 4 + u) * 1024, 16, 0, 0); \
    const uint8_t* ss_ = s_src + (size_t)(S) * s_stage;                                               \
    __builtin_amdgcn_global_load_lds(ss_, (SP) + kSlotData + wave * 512, 4, 0, 0);                    \
    __builtin_amdgcn_global_load_lds(ss_ + 256, (SP) + kSlotData + wave * 512 + 256, 4, 0, 0);        \
  }
#define MX4_READ(RP, B)                                                                               \
  {                                                                                                   \
    _Pragma("unroll") for (int ks = 0; ks < 2; ks++) {                                                \
      _Pragma("unroll") for (int i = 0; i < 4; i++)                                                   \
        af[B][ks][i] = *reinterpret_cast<const v4i*>((RP) + a_off[ks][i]);                            \
      _Pragma("unroll") for (int j = 0; j < 4; j++)                                                   \
        bf[B][ks][j] = *reinterpret_cast<const v4i*>((RP) + b_off[ks][j]);                            \
    }                                                                                                 \
    _Pragma("unroll") for (int i = 0; i < 4; i++) {                                                   \
      sa[B][i] = *reinterpret_cast<const uint32_t*>((RP) + sa_off[i]);                                \
      sb[B][i] = *reinterpret_cast<const uint32_t*>((RP) + sb_off[i]);                                \
    }                                                                                                 \
  }
#define MX4_MMA(B)                                                                                    \
  {                                                                                                   \
    _Pragma("unroll") for (int i = 0; i < 4; i++)                                                     \
      _Pragma("unroll") for (int j = 0; j < 4; j++)                                                   \
        acc[i][j] = mfma_fp4_32x32x64<0, 0>(af[B][0][i], bf[B][0][j], acc[i][j],                      \
                                            (int)(sa[B][i] >> shift), (int)(sb[B][j] >> shift));      \
    _Pragma("unroll") for (int i = 0; i < 4; i++)                                                     \
      _Pragma("unroll") for (int j = 0; j < 4; j++)                                                   \
        acc[i][j] = mfma_fp4_32x32x64<2, 2>(af[B][1][i], bf[B][1][j], acc[i][j],                      \
                                            (int)(sa[B][i] >> shift), (int)(sb[B][j] >> shift));      \
  }
  // One K stage; J = stage index mod 4 (a literal), kt = the stage index.
#define MX4_STAGE(J)                                                                                  \
  {                                                                                                   \
    const int kt_ = kt0 + (J);                                                                        \
    __builtin_amdgcn_s_waitcnt(wait_lgkm0_vm(2 * kDmaPerStage));                                      \
    __builtin_amdgcn_s_barrier();                                                                     \
    MX4_ISSUE(min(kt_ + kNS, KT - 1), ring<(J)>())                                                    \
    MX4_READ(ring<((J) + 1) % kNS>(), ((J) + 1) & 1)                                                  \
    MX4_MMA((J) & 1)                                                                                  \
    /* spread the 10 DMA issues and 24 ds_reads over the 32 MFMAs */                                  \
    _Pragma("unroll") for (int q_ = 0; q_ < 10; q_++) {                                               \
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                                              \
      __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);                                              \
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);                                              \
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                                              \
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);                                              \
    }                                                                                                 \
    _Pragma("unroll") for (int q_ = 0; q_ < 4; q_++) {                                                \
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                                              \
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);                                              \
    }                                                                                                 \
    __builtin_amdgcn_sched_group_barrier(0x008, 8, 0);                                                \
    __builtin_amdgcn_sched_barrier(0);                                                                \
  }

  // Prologue: stages 0..3 into the four slots, stage 0 into VGPR set 0.
  MX4_ISSUE(0, ring<0>())
  MX4_ISSUE(min(1, KT - 1), ring<1>())
  MX4_ISSUE(min(2, KT - 1), ring<2>())
  MX4_ISSUE(min(3, KT - 1), ring<3>())
  __builtin_amdgcn_s_waitcnt(wait_lgkm0_vm(3 * kDmaPerStage));
  __builtin_amdgcn_s_barrier();
  MX4_READ(ring<0>(), 0)
  // Stage k+1 of the last iteration re-reads a valid (clamped) stage; its
  // values are never used.
  for (int kt0 = 0; kt0 < KT; kt0 += kNS) {
    MX4_STAGE(0)
    MX4_STAGE(1)
    MX4_STAGE(2)
    MX4_STAGE(3)
  }
#undef MX4_STAGE
#undef MX4_MMA
#undef MX4_READ
#undef MX4_ISSUE
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();

  if (!DUAL) {
    uint16_t* c = reinterpret_cast<uint16_t*>(g.c);
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const int col = nt * 256 + (wn * 4 + j) * 32 + (lane & 31);
#pragma unroll
        for (int v = 0; v < 16; v++) {
          const int row = m0 + wm * 128 + i * 32 + acc32_row(lane, v);
          if (row < M) c[(size_t)row * g.n + col] = f32_to_f16_bits(acc[i][j][v]);
        }
      }
    return;
  }
  // mid = silu(gate) * up re-quantized along channels (stage-major scales).
  float* mid = reinterpret_cast<float*>(ring0) + wave * (64 * kMidStride);
  uint8_t* mp = reinterpret_cast<uint8_t*>(g.c);
  const size_t mid_row_bytes = (size_t)g.n / 2;
#pragma unroll
  for (int jb = 0; jb < 2; jb++) {
    const int chan0 = nt * 128 + (wn * 2 + jb) * 32;
#pragma unroll
    for (int h = 0; h < 2; h++) {
#pragma unroll
      for (int i2 = 0; i2 < 2; i2++)
#pragma unroll
        for (int v = 0; v < 16; v++) {
          const int r = i2 * 32 + acc32_row(lane, v);
          mid[r * kMidStride + (lane & 31)] = silu(acc[2 * h + i2][jb][v]) * acc[2 * h + i2][2 + jb][v];
        }
      __syncthreads();
      const int row = m0 + wm * 128 + h * 64 + lane;
      float v[32];
      uint32_t amax = 0;
#pragma unroll
      for (int j = 0; j < 32; j++) {
        v[j] = mid[lane * kMidStride + j];
        amax = max(amax, abs_bits(v[j]));
      }
      const uint32_t sbyte = mxfp4_scale_byte(amax);
      uint4 o = make_uint4(0, 0, 0, 0);
      if (sbyte != 255u) {
        o.x = fp4x8_from_f32(v + 0, sbyte);
        o.y = fp4x8_from_f32(v + 8, sbyte);
        o.z = fp4x8_from_f32(v + 16, sbyte);
        o.w = fp4x8_from_f32(v + 24, sbyte);
      }
      if (row < M) {
        *reinterpret_cast<uint4*>(mp + (size_t)row * mid_row_bytes + chan0 / 2) = o;
        const int blk = chan0 / 32;
        g.cs[((size_t)(blk >> 2) * Mpad + row) * 4 + (blk & 3)] = (uint8_t)sbyte;
      }
      __syncthreads();
    }
  }
}

}  // namespace

bool gemm_fp4_v4_ok(int k) { return k % (kKS * kNS) == 0; }

hipError_t launch_gemm_fp4_v4(int dual, const Fp4GemmArgs& g, hipStream_t st) {
  const int MT = (g.m + kM - 1) / kM;
  const int NT = dual ? g.n / 128 : g.n / 256;
  if (dual) hipLaunchKernelGGL(k_gemm_fp4_v4<true>, dim3(MT * NT), dim3(256), 0, st, g);
  else hipLaunchKernelGGL(k_gemm_fp4_v4<false>, dim3(MT * NT), dim3(256), 0, st, g);
  return hipGetLastError();
}

}  // namespace mx
