// mx_gemm_fp4_v5.hip - the W4A4 prefill GEMM, full-cache-line operand DMA.
//
// Tile 256 x 256, 4 wave64s in a 2 x 2 grid each owning 128 x 128 (4 x 4
// blocks of v_mfma_scale_f32_32x32x64 with FP4 operands, 256 AGPRs), K stage
// 256.  A K stage of one row is 128 bytes - exactly one cache line - and every
// DMA instruction (global_load_lds_dwordx4, 64 lanes x 16 B) moves 8 whole
// rows.  (With 128-element stages a row holds 64 B per stage and a fragment-
// major DMA gathers 32 rows x 32 B: 32 partly used lines per 1 KB, which made
// the L2 -> LDS path, not the MFMAs, the limit.)
//
// LDS (per slot): A [256 rows][128 B], B [256 rows][128 B], then the A and B
// scales of the stage's two 128-K planes ([2][256] dwords each).  The eight
// 16-byte chunks of a row (one E8M0 block each) are stored XOR-swizzled,
// chunk c of row r at slot c ^ swz(r), so that the MFMA operand reads
// (ds_read_b128, 32 rows x one chunk per instruction) hit distinct banks.
// The swizzle is applied by the DMA itself: lane l of an instruction writes
// LDS slot l % 8 of row l / 8, so it fetches global chunk (l % 8) ^ swz(row).
//
// Pipeline (2 slots, 2 VGPR fragment sets; k-step s = 64 K = chunks 2s, 2s+1):
//   ks0..ks2:  MFMAs of k-step s while ds_reads fetch k-step s+1
//   barrier:   this wave's ds_reads are back and its DMA of stage k+1 has
//              landed; afterwards nobody reads stage k's slot any more
//   ks3:       MFMAs of k-step 3, ds_reads of stage k+1's k-step 0 and
//              scales, DMA of stage k+2 into stage k's slot
// The ring is two separate __shared__ arrays with constant slot numbers
// (the loop is unrolled by 2) and the barrier is a bare s_barrier, so the
// backend does not turn the stage wait into vmcnt(0) for unrelated DMA.
// Every wave issues exactly 17 DMA instructions per stage.
//
// Small-M plain GEMMs (too few tiles for the CUs) split K: workgroups of
// split s run stages [s * KT/S, (s + 1) * KT/S) and store f32 partials, and a
// second launch adds the S partials in split order and stores f16.
#include "mx_device.h"
#include "mx_internal.h"

namespace mx {
namespace {

constexpr int kM = 256;            // tile rows (M) and tile columns (N)
constexpr int kKS = 256;           // K per stage
constexpr int kRowB = kKS / 2;     // bytes of one row per stage (one line)
constexpr int kOpB = 256 * kRowB;  // 32 KB of one operand per stage
constexpr int kScA = 2 * kOpB;     // A scales: [2 planes][256 rows] dwords
constexpr int kScB = kScA + 2048;  // B scales
constexpr int kSlot = kScB + 2048; // 69632 B
constexpr int kMidStride = 33;
constexpr int kDma = 17;           // DMA instructions per wave per stage

__shared__ __attribute__((aligned(16))) uint8_t ring0[kSlot];
__shared__ __attribute__((aligned(16))) uint8_t ring1[kSlot];

template <int J>
__device__ __forceinline__ uint8_t* ring() {
  if constexpr (J == 0) return ring0;
  else return ring1;
}

// Chunk swizzle of a row (depends on row % 32 only).
__device__ __forceinline__ int swz(int row) { return (row ^ ((row >> 3) & 3)) & 7; }

// s_waitcnt immediate (gfx9 encoding): lgkmcnt(0), expcnt untouched, vmcnt(n).
constexpr int wait_lgkm0_vm(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4); }

__device__ __forceinline__ int xcd_tile(int bid, int nblocks) {
  if (nblocks % 8 != 0) return bid;
  const int per = nblocks / 8;
  return (bid % 8) * per + bid / 8;
}

template <bool DUAL, bool SPLIT>
__global__ __launch_bounds__(256, 1) void k_gemm_fp4_v5(Fp4GemmArgs g) {
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave & 1, wn = wave >> 1;
  const int M = g.m, K = g.k;
  const int MT = (M + kM - 1) / kM;
  const int NT = DUAL ? g.n / 128 : g.n / 256;
  const size_t Mpad = stage_major_rows(M);
  const size_t NB = (size_t)g.n;

  // Split-K: workgroup b takes split b / tiles, stages [split * KT, +KT).
  const int tiles = MT * NT;
  const int splits = SPLIT ? g.splits : 1;
  const int split = SPLIT ? blockIdx.x / tiles : 0;
  const int KT = K / kKS / splits;
  const size_t kbeg = (size_t)split * KT;
  const int tile = xcd_tile(blockIdx.x - split * tiles, tiles);
  const int group_sz = 8 * MT;
  const int grp = tile / group_sz, in_grp = tile % group_sz;
  const int nt_base = grp * 8;
  const int gw = min(8, NT - nt_base);
  const int mt = in_grp / gw, nt = nt_base + in_grp % gw;
  const int m0 = mt * kM;
  const size_t row_bytes = (size_t)K / 2;

  // ---- DMA sources.  Wave w moves tile rows [64w, 64w + 64) of A and of B,
  // 8 rows per instruction; lane l -> row 8q + l/8, LDS chunk slot l % 8.
  const int drow = lane >> 3;
  const uint8_t* a_src[8];
#pragma unroll
  for (int q = 0; q < 8; q++) {
    const int r = wave * 64 + q * 8 + drow;
    const int c = (lane & 7) ^ swz(r);
    a_src[q] = g.a + (size_t)min(m0 + r, M - 1) * row_bytes + kbeg * kRowB + c * 16;
  }
  // B rows of one wave are consecutive rows of one matrix; the swizzle of
  // row 64w + 8q + l/8 is (l/8) ^ (q % 4), so four chunk offsets cover q.
  const uint8_t* b_src = (DUAL ? (wave < 2 ? g.b0 : g.b1) + (size_t)(nt * 128 + (wave & 1) * 64 + drow) * row_bytes
                               : g.b0 + (size_t)(nt * 256 + wave * 64 + drow) * row_bytes) + kbeg * kRowB;
  int b_co[4];
#pragma unroll
  for (int q = 0; q < 4; q++) b_co[q] = ((lane & 7) ^ swz(wave * 64 + q * 8 + drow)) * 16;
  // Scales: wave 0 / 1 move A plane 0 / 1, wave 2 / 3 B plane 0 / 1 (1 KB
  // each, lane l: 4 consecutive rows' dwords).
  const uint8_t* s_src;
  size_t s_plane;  // bytes between consecutive 128-K planes
  if (wave < 2) {
    s_src = g.as + ((size_t)wave * Mpad + m0 + 4 * lane) * 4;
    s_plane = Mpad * 4;
  } else if (DUAL) {
    s_src = (lane < 32 ? g.s0 : g.s1) + ((size_t)(wave - 2) * NB + nt * 128 + 4 * (lane & 31)) * 4;
    s_plane = NB * 4;
  } else {
    s_src = g.s0 + ((size_t)(wave - 2) * NB + nt * 256 + 4 * lane) * 4;
    s_plane = NB * 4;
  }
  s_src += kbeg * 2 * s_plane;

  // ---- operand reads.  k-step s, lane half h = lane / 32 -> chunk 2s + h.
  int bfrag[4];
#pragma unroll
  for (int j = 0; j < 4; j++) {
    if (DUAL) bfrag[j] = j < 2 ? wn * 2 + (j & 1) : 4 + wn * 2 + (j & 1);
    else bfrag[j] = wn * 4 + j;
  }
  const int r32 = lane & 31, h = lane >> 5;
  int lp[4];  // lane part of the byte offset for k-step s
#pragma unroll
  for (int s = 0; s < 4; s++) lp[s] = r32 * kRowB + (((2 * s + h) ^ swz(r32)) << 4);
  const int a_blk = wm * 128 * kRowB;  // + i * 32 rows
  int b_blk[4];
#pragma unroll
  for (int j = 0; j < 4; j++) b_blk[j] = kOpB + bfrag[j] * 32 * kRowB;
  const int shift = 8 * h;

  v16f acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int j = 0; j < 4; j++)
#pragma unroll
      for (int v = 0; v < 16; v++) acc[i][j][v] = 0.0f;

  v4i af[2][4], bf[2][4];
  uint32_t sa[2][2][4], sb[2][2][4];  // [stage parity][plane][block]

#define MX5_ISSUE(S, SP)                                                                          \
  {                                                                                               \
    const size_t koff_ = (size_t)(S) * kRowB;                                                     \
    _Pragma("unroll") for (int q = 0; q < 8; q++)                                                 \
      __builtin_amdgcn_global_load_lds(a_src[q] + koff_, (SP) + (wave * 64 + q * 8) * kRowB, 16, 0, 0); \
    _Pragma("unroll") for (int q = 0; q < 8; q++)                                                 \
      __builtin_amdgcn_global_load_lds(b_src + (size_t)q * 8 * row_bytes + koff_ + b_co[q & 3],   \
                                       (SP) + kOpB + (wave * 64 + q * 8) * kRowB, 16, 0, 0);      \
    __builtin_amdgcn_global_load_lds(s_src + (size_t)(S) * 2 * s_plane,                           \
                                     (SP) + kScA + wave * 1024, 16, 0, 0);                        \
  }
#define MX5_READ(RP, s, F)                                                                        \
  {                                                                                               \
    _Pragma("unroll") for (int i = 0; i < 4; i++)                                                 \
      af[F][i] = *reinterpret_cast<const v4i*>((RP) + a_blk + i * 32 * kRowB + lp[s]);            \
    _Pragma("unroll") for (int j = 0; j < 4; j++)                                                 \
      bf[F][j] = *reinterpret_cast<const v4i*>((RP) + b_blk[j] + lp[s]);                          \
  }
#define MX5_SCALES(RP, P)                                                                         \
  {                                                                                               \
    _Pragma("unroll") for (int p = 0; p < 2; p++)                                                 \
      _Pragma("unroll") for (int i = 0; i < 4; i++) {                                             \
        sa[P][p][i] = *reinterpret_cast<const uint32_t*>((RP) + kScA + p * 1024 +                 \
                                                         (wm * 128 + i * 32 + r32) * 4);          \
        sb[P][p][i] = *reinterpret_cast<const uint32_t*>((RP) + kScB + p * 1024 +                 \
                                                         (bfrag[i] * 32 + r32) * 4);              \
      }                                                                                           \
  }
#define MX5_MMA(F, P, s)                                                                          \
  _Pragma("unroll") for (int i = 0; i < 4; i++)                                                   \
    _Pragma("unroll") for (int j = 0; j < 4; j++) {                                               \
      const int sa_ = (int)(sa[P][(s) >> 1][i] >> shift), sb_ = (int)(sb[P][(s) >> 1][j] >> shift); \
      if (((s) & 1) == 0) acc[i][j] = mfma_fp4_32x32x64<0, 0>(af[F][i], bf[F][j], acc[i][j], sa_, sb_); \
      else acc[i][j] = mfma_fp4_32x32x64<2, 2>(af[F][i], bf[F][j], acc[i][j], sa_, sb_);         \
    }
  // k-step with the next k-step's reads interleaved (8 ds_reads, 16 MFMAs)
#define MX5_KSTEP(J, s)                                                                           \
  {                                                                                               \
    MX5_READ(ring<(J)>(), (s) + 1, ((s) + 1) & 1)                                                 \
    MX5_MMA((s) & 1, (J), (s))                                                                    \
    _Pragma("unroll") for (int q_ = 0; q_ < 8; q_++) {                                            \
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                                          \
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);                                          \
    }                                                                                             \
    __builtin_amdgcn_sched_group_barrier(0x008, 8, 0);                                            \
    __builtin_amdgcn_sched_barrier(0);                                                            \
  }
  // One stage kt = kt0 + J.  On entry fragment set 0 holds its k-step 0 and
  // scale set J its scales.
#define MX5_STAGE(J)                                                                              \
  {                                                                                               \
    const int kt_ = kt0 + (J);                                                                    \
    MX5_KSTEP(J, 0)                                                                               \
    MX5_KSTEP(J, 1)                                                                               \
    MX5_KSTEP(J, 2)                                                                               \
    __builtin_amdgcn_s_waitcnt(wait_lgkm0_vm(0));                                                 \
    __builtin_amdgcn_s_barrier();                                                                 \
    MX5_ISSUE(min(kt_ + 2, KT - 1), ring<(J)>())                                                  \
    MX5_READ(ring<(J) ^ 1>(), 0, 0)                                                               \
    MX5_SCALES(ring<(J) ^ 1>(), (J) ^ 1)                                                          \
    MX5_MMA(1, (J), 3)                                                                            \
    /* 16 MFMAs; 17 DMA, 8 + 16 (paired to 8) LDS reads between them */                          \
    _Pragma("unroll") for (int q_ = 0; q_ < 8; q_++) {                                            \
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                                          \
      __builtin_amdgcn_sched_group_barrier(0x020, 2, 0);                                          \
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);                                          \
    }                                                                                             \
    __builtin_amdgcn_sched_group_barrier(0x008, 8, 0);                                            \
    __builtin_amdgcn_sched_barrier(0);                                                            \
  }

  MX5_ISSUE(0, ring<0>())
  MX5_ISSUE(min(1, KT - 1), ring<1>())
  __builtin_amdgcn_s_waitcnt(wait_lgkm0_vm(kDma));
  __builtin_amdgcn_s_barrier();
  MX5_READ(ring<0>(), 0, 0)
  MX5_SCALES(ring<0>(), 0)
  // The last stage's look-ahead reads a clamped (valid, unused) stage.
  for (int kt0 = 0; kt0 < KT; kt0 += 2) {
    MX5_STAGE(0)
    MX5_STAGE(1)
  }
#undef MX5_STAGE
#undef MX5_KSTEP
#undef MX5_MMA
#undef MX5_SCALES
#undef MX5_READ
#undef MX5_ISSUE
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();

  if (SPLIT) {
    // f32 partials [split][M][N]
    static_assert(!(DUAL && SPLIT), "the dual epilogue needs the whole K sum");
    const size_t plane = (size_t)M * g.n;
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const int col = nt * 256 + (wn * 4 + j) * 32 + r32;
        float* dst = g.ws + (size_t)split * plane + col;
#pragma unroll
        for (int v = 0; v < 16; v++) {
          const int row = m0 + wm * 128 + i * 32 + acc32_row(lane, v);
          if (row < M) dst[(size_t)row * g.n] = acc[i][j][v];
        }
      }
    return;
  }

  if (!DUAL) {
    uint16_t* c = reinterpret_cast<uint16_t*>(g.c);
    uint64_t nanm[4] = {0u, 0u, 0u, 0u};  // bit j * 16 + v of word i: element is NaN
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const int col = nt * 256 + (wn * 4 + j) * 32 + r32;
#pragma unroll
        for (int v = 0; v < 16; v++) {
          const int row = m0 + wm * 128 + i * 32 + acc32_row(lane, v);
          const float x0 = acc[i][j][v];
          nanm[i] |= (uint64_t)(x0 != x0) << (j * 16 + v);
          if (row < M) c[(size_t)row * g.n + col] = f32_to_f16_bits(x0);
        }
      }
    // E8M0 byte 255 in a down-weight scale is NaN to the scaled MFMA and
    // +inf to the reference (MXFP4Kernels.metal:26-29), whose dequantize-
    // then-accumulate gives +-inf or NaN there: NaN outputs (rare; one
    // wave-uniform test) are recomputed with the reference's dequantization.
    if (__builtin_expect(__ballot((nanm[0] | nanm[1] | nanm[2] | nanm[3]) != 0) != 0, 0)) {
#pragma nounroll
      for (int e = 0; e < 256; e++) {
        const int i = e >> 6, j = (e >> 4) & 3, v = e & 15;
        if (!((nanm[i] >> (j * 16 + v)) & 1u)) continue;
        const int row = m0 + wm * 128 + i * 32 + acc32_row(lane, v);
        const int col = nt * 256 + (wn * 4 + j) * 32 + r32;
        if (row < M)
          c[(size_t)row * g.n + col] = f32_to_f16_bits(ref_dot_mxfp4_mxfp4(g.a, g.as, Mpad, row, g.b0, g.s0, NB, col, K));
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
    for (int hh = 0; hh < 2; hh++) {
#pragma unroll
      for (int i2 = 0; i2 < 2; i2++)
#pragma unroll
        for (int v = 0; v < 16; v++) {
          const int r = i2 * 32 + acc32_row(lane, v);
          mid[r * kMidStride + r32] = silu(acc[2 * hh + i2][jb][v]) * acc[2 * hh + i2][2 + jb][v];
        }
      __syncthreads();
      const int row = m0 + wm * 128 + hh * 64 + lane;
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

// Split-K reduce, plain epilogue: 4 consecutive outputs per thread, the
// splits summed in order 0, 1, ... in f32, stored as f16.
// A NaN sum (E8M0 byte 255 in a down-weight scale) is recomputed with the
// reference's dequantization, as in the unsplit epilogue.
__global__ __launch_bounds__(256) void k_fp4_reduce_f16(Fp4GemmArgs g) {
  const size_t plane = (size_t)g.m * g.n;
  const size_t o = ((size_t)blockIdx.x * blockDim.x + threadIdx.x) * 4;
  if (o >= plane) return;
  float s[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  for (int k = 0; k < g.splits; k++) {
    const float4 v = *reinterpret_cast<const float4*>(g.ws + (size_t)k * plane + o);
    s[0] += v.x; s[1] += v.y; s[2] += v.z; s[3] += v.w;
  }
  for (int t = 0; t < 4; t++) {
    if (s[t] != s[t]) {
      const int row = (int)((o + t) / g.n), col = (int)((o + t) % g.n);
      s[t] = ref_dot_mxfp4_mxfp4(g.a, g.as, stage_major_rows(g.m), row, g.b0, g.s0, (size_t)g.n, col, g.k);
    }
  }
  uint2 h;
  h.x = f32_to_f16_bits(s[0]) | ((uint32_t)f32_to_f16_bits(s[1]) << 16);
  h.y = f32_to_f16_bits(s[2]) | ((uint32_t)f32_to_f16_bits(s[3]) << 16);
  *reinterpret_cast<uint2*>(reinterpret_cast<uint16_t*>(g.c) + o) = h;
}

}  // namespace

bool gemm_fp4_v5_ok(int k) { return k % (2 * kKS) == 0; }

// Splits for the small-M plain GEMMs whose tiles alone leave most CUs idle
// (one workgroup per CU: the ring takes 136 KB of LDS): double while the
// grid stays within 256 workgroups and every split keeps an even number
// (>= 2) of 256-K stages.  At M=128, N=1024, K=4096 (4 tiles, 16 stages) 8
// splits take the GEMM from 29 us to about 17 us with the reduce.  The dual
// gate/up GEMM is not split: its partials are two planes and its reduce
// carries the SwiGLU + requantize epilogue, and at M=128, N=4096, K=1024 two
// splits measured 8 us slower than none.
int gemm_fp4_splits(int dual, int m, int n, int k) {
  if (dual || !gemm_fp4_v5_ok(k)) return 1;
  const int tiles = ((m + kM - 1) / kM) * (dual ? n / 128 : n / 256);
  const int kt = k / kKS;
  int s = 1;
  while (tiles * 2 * s <= 256 && kt % (4 * s) == 0) s *= 2;
  return s;
}

size_t gemm_fp4_ws_bytes(int dual, int m, int n, int k) {
  const int s = gemm_fp4_splits(dual, m, n, k);
  return s > 1 ? (size_t)s * (dual ? 2 : 1) * m * n * 4 : 0;
}

hipError_t launch_gemm_fp4_v5(int dual, const Fp4GemmArgs& g, hipStream_t st) {
  const int MT = (g.m + kM - 1) / kM;
  const int NT = dual ? g.n / 128 : g.n / 256;
  const int splits = g.splits > 1 ? g.splits : 1;
  if (splits > 1 && (dual || !g.ws || (g.k / kKS) % (2 * splits))) return hipErrorInvalidValue;
  const dim3 grid(MT * NT * splits);
  if (splits > 1) {
    hipLaunchKernelGGL((k_gemm_fp4_v5<false, true>), grid, dim3(256), 0, st, g);
    const size_t threads = (size_t)g.m * g.n / 4;
    hipLaunchKernelGGL(k_fp4_reduce_f16, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, st, g);
  } else if (dual) {
    hipLaunchKernelGGL((k_gemm_fp4_v5<true, false>), grid, dim3(256), 0, st, g);
  } else {
    hipLaunchKernelGGL((k_gemm_fp4_v5<false, false>), grid, dim3(256), 0, st, g);
  }
  return hipGetLastError();
}

}  // namespace mx
