// mx_gemm_fp4_v6.hip - the W4A4 prefill GEMM for grids of whole 256 x 256
// tiles (C4): 128-K stages in a four-slot ring, activations stage-major.
//
// Same tile and MFMA blocking as mx_gemm_fp4_v5.hip (256 x 256, 4 wave64s
// in a 2 x 2 grid each owning 128 x 128 = 4 x 4 blocks of
// v_mfma_scale_f32_32x32x64 with FP4 operands, 256 AGPRs).  What changes is
// how much operand data is in flight.  The 256-K stages of v5 take 68 KB of
// LDS each, so only two fit: the DMA of stage k+2 is issued once stage k has
// been read and must land within one stage of MFMAs, which is shorter than
// the loaded L2 / MALL latency, and the waves stall on every stage.  Here a
// stage is 128 K (34 KB) and four fit.  The DMA of stage k+4 is issued once
// stage k has been read, in two halves over the next two k-steps, so that
// the per-CU vector memory path (about 2 cycles per 128-byte line) is
// loaded evenly; it then has over two stages (one of v5's) to land.
//
// Operand layouts:
//   A (activations and the mid): stage-major, [K/128][Mpad][64 B], written
//     so by the W4A4 prologue and by this kernel's dual epilogue.  The 64 B
//     of 16 consecutive rows are 1 KB contiguous, so one DMA instruction
//     (64 lanes x 16 B) moves 8 whole cache lines.
//   B (weights): the reference layout [N][K/2]; one instruction moves the
//     64 B of a stage from 16 rows (half of each row's 128-byte line, the
//     other half being the next stage's).
//   Scales: stage-major planes [K/128][rows] dwords (one dword = the four
//     E8M0 bytes of a row's stage), as for v5.
//
// LDS per slot: A [256 rows][64 B], B [256 rows][64 B], A scales [256]
// dwords, B scales [256] dwords.  The four 16-byte chunks of a row (one E8M0
// block each) are stored XOR-swizzled, chunk c of row r at slot c ^ swz(r),
// so that the operand reads (ds_read_b128, 16 or 8 consecutive rows of one
// chunk per LDS cycle) hit distinct banks.  The DMA applies the swizzle:
// lane l of an instruction writes slot l % 4 of row l / 4 and fetches the
// global chunk (l % 4) ^ swz(row).
//
// Pipeline (k-step s = 64 K = chunks 2s, 2s+1 of a stage):
//   ks0:      MFMAs of k-step 0 while ds_reads fetch k-step 1
//   barrier:  this wave's ds_reads are back and its DMA of stage k+1 has
//             landed (stages k+2, k+3 stay in flight); afterwards nobody
//             reads stage k's slot any more
//   ks1:      MFMAs of k-step 1, ds_reads of stage k+1's k-step 0 and
//             scales, first half of the DMA of stage k+4 into stage k's
//             slot (its second half goes out during the next stage's ks0)
// The ring is four separate __shared__ arrays with constant slot numbers
// (the loop is unrolled by 4), so the backend keeps the explicit vmcnt
// waits.  Every wave issues exactly 10 DMA instructions per stage.
#include "mx_device.h"
#include "mx_internal.h"

namespace mx {
namespace {

constexpr int kM = 256;             // tile rows (M) and tile columns (N)
constexpr int kKS = 128;            // K per stage
constexpr int kRowB = kKS / 2;      // bytes of one row per stage
constexpr int kOpB = 256 * kRowB;   // 16 KB of one operand per stage
constexpr int kScA = 2 * kOpB;      // A scales: 256 dwords
constexpr int kScB = kScA + 1024;   // B scales: 256 dwords
constexpr int kSlot = kScB + 1024;  // 34816 B
constexpr int kMidStride = 33;
constexpr int kDma = 10;            // DMA instructions per wave per stage

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

// Chunk swizzle of a 64-byte row (depends on row % 32 only).  Chosen by
// measurement: with it SQ_LDS_BANK_CONFLICT is 0 for both C4 GEMMs; so it
// is with (row >> 2) & 3 or (row ^ (row >> 2)) & 3, while ((row >> 1) ^
// (row >> 3)) & 3, (row >> 1) & 3 and ((row >> 2) ^ (row >> 4)) & 3 left
// 2.5 conflict cycles per LDS instruction (and no swizzle 7.5).
__device__ __forceinline__ int swz(int row) { return (row ^ (row >> 3)) & 3; }

// s_waitcnt immediate (gfx9 encoding): lgkmcnt(0), expcnt untouched, vmcnt(n).
constexpr int wait_lgkm0_vm(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4); }

// Buffer loads into LDS (buffer_load_dwordx4 ... lds): the per-stage base
// goes into a wave-uniform buffer resource (scalar arithmetic) and each
// lane's part is one precomputed 32-bit offset, so a DMA instruction needs
// no vector address arithmetic (a 64-bit global address costs two dependent
// 64-bit adds per instruction, which the wave's in-order issue pays between
// its MFMAs).  Loads past the resource's byte count return 0.
typedef __attribute__((address_space(3))) uint32_t* lds_u32;
extern "C" __device__ void llvm_amdgcn_raw_buffer_load_lds(v4i rsrc, lds_u32 lds, int size, int voffset, int soffset,
                                                            int offset, int aux) __asm("llvm.amdgcn.raw.buffer.load.lds");

__device__ __forceinline__ v4i buf_rsrc(const uint8_t* base, uint32_t bytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  v4i r;
  r[0] = (int)(uint32_t)a;
  r[1] = (int)(uint32_t)(a >> 32);  // base[47:32]; stride 0
  r[2] = (int)bytes;
  r[3] = 0x00020000;
  return r;
}

__device__ __forceinline__ int xcd_tile(int bid, int nblocks) {
  if (nblocks % 8 != 0) return bid;
  const int per = nblocks / 8;
  return (bid % 8) * per + bid / 8;
}

// sum_k A[row][k] * W[col][k] with A stage-major ([K/128][a_rows][64 B]) and
// W in the reference layout, each dequantized as the reference does before
// the product (the byte-255 recompute of the plain epilogue).
__device__ float ref_dot_sm_a(const uint8_t* a, const uint8_t* as, size_t a_rows, int row, const uint8_t* w,
                              const uint8_t* ws, size_t w_rows, int col, int K) {
  const uint8_t* wr = w + (size_t)col * (K / 2);
  float acc = 0.0f;
  for (int b = 0; b < K / 32; b++) {
    const uint8_t* ab = a + ((size_t)(b >> 2) * a_rows + row) * kRowB + (b & 3) * 16;
    const float sa = e8m0_to_float(e8m0_stage_major(as, a_rows, row, b));
    const float sw = e8m0_to_float(e8m0_stage_major(ws, w_rows, col, b));
    for (int j = 0; j < 16; j++) {
      const v2f ca = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(ab[j], 1.0f, 0);
      const v2f cw = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(wr[b * 16 + j], 1.0f, 0);
      acc += (ca[0] * sa) * (cw[0] * sw);
      acc += (ca[1] * sa) * (cw[1] * sw);
    }
  }
  return acc;
}

template <bool DUAL>
__global__ __launch_bounds__(256, 1) void k_gemm_fp4_v6(Fp4GemmArgs g) {
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave & 1, wn = wave >> 1;
  const int M = g.m, K = g.k;
  const int MT = (M + kM - 1) / kM;
  const int NT = DUAL ? g.n / 128 : g.n / 256;
  const size_t Mpad = stage_major_rows(M);
  const size_t NB = (size_t)g.n;
  const int KT = K / kKS;

  // Each XCD takes a contiguous range of tiles, walked as groups of 8 N
  // tiles x all M tiles (32 resident tiles per XCD = 4 M x 8 N).
  const int tiles = MT * NT;
  const int tile = xcd_tile(blockIdx.x, tiles);
  const int group_sz = 8 * MT;
  const int grp = tile / group_sz, in_grp = tile % group_sz;
  const int nt_base = grp * 8;
  const int gw = min(8, NT - nt_base);
  const int mt = in_grp / gw, nt = nt_base + in_grp % gw;
  const int m0 = mt * kM;
  const size_t row_bytes = (size_t)K / 2;

  // ---- DMA sources.  Wave w moves tile rows [64w, 64w + 64) of A and of B,
  // 16 rows per instruction; lane l -> row 16q + l/4, LDS chunk slot l % 4.
  const int drow = lane >> 2, dch = lane & 3;
  const size_t a_plane = Mpad * kRowB;  // bytes of one A stage plane
  int a_off[4], b_off[4];
#pragma unroll
  for (int q = 0; q < 4; q++) {
    const int r = wave * 64 + q * 16 + drow;
    a_off[q] = (m0 + r) * kRowB + ((dch ^ swz(r)) << 4);
    // B rows of one wave are 64 consecutive rows of one matrix; the swizzle
    // of row 64w + 16q + l/4 depends on q only through q % 2.
    b_off[q] = (int)((size_t)(q * 16 + drow) * row_bytes) + ((dch ^ swz((q & 1) * 16 + drow)) << 4);
  }
  const uint8_t* b_base = DUAL ? (wave < 2 ? g.b0 : g.b1) + (size_t)(nt * 128 + (wave & 1) * 64) * row_bytes
                               : g.b0 + (size_t)(nt * 256 + wave * 64) * row_bytes;
  const uint32_t b_bytes = (uint32_t)(64 * row_bytes);  // this wave's 64 rows
  // Scales: wave 0 / 1 move A rows [0, 128) / [128, 256), wave 2 / 3 B rows
  // [0, 128) / [128, 256) (dual: the gate / up rows), 64 dwords per
  // instruction, two instructions per stage.
  const uint8_t* s_base;
  size_t s_plane;  // bytes between consecutive stage planes
  if (wave < 2) {
    s_base = g.as + ((size_t)m0 + wave * 128) * 4;
    s_plane = Mpad * 4;
  } else if (DUAL) {
    s_base = (wave == 2 ? g.s0 : g.s1) + (size_t)nt * 128 * 4;
    s_plane = NB * 4;
  } else {
    s_base = g.s0 + ((size_t)nt * 256 + (wave - 2) * 128) * 4;
    s_plane = NB * 4;
  }
  const int s_dst = (wave < 2 ? kScA : kScB) + (wave & 1) * 512;
  const int s_off[2] = {lane * 4, lane * 4 + 256};

  // ---- operand reads.  k-step s, lane half h = lane / 32 -> chunk 2s + h.
  int bfrag[4];
#pragma unroll
  for (int j = 0; j < 4; j++) {
    if (DUAL) bfrag[j] = j < 2 ? wn * 2 + (j & 1) : 4 + wn * 2 + (j & 1);
    else bfrag[j] = wn * 4 + j;
  }
  const int r32 = lane & 31, h = lane >> 5;
  int lp[2];  // lane part of the byte offset for k-step s
#pragma unroll
  for (int s = 0; s < 2; s++) lp[s] = r32 * kRowB + (((2 * s + h) ^ swz(r32)) << 4);
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
  uint32_t sa[2][4], sb[2][4];  // [stage parity][block]

// A stage's 10 DMA instructions go out in two halves of 5 (rows q = 2p,
// 2p + 1 of A and of B, scale instruction p), issued during different
// k-steps: the per-CU vector memory path takes about 2 cycles per 128-byte
// line, and a whole stage issued within one k-step's 16 MFMAs stalls the
// issuing waves.
#define MX6_ISSUE_HALF(S, SP, P)                                                                  \
  {                                                                                               \
    const int st_ = (S);                                                                          \
    const v4i ra_ = buf_rsrc(g.a + (size_t)st_ * a_plane, (uint32_t)((size_t)(KT - st_) * a_plane)); \
    const v4i rb_ = buf_rsrc(b_base + (size_t)st_ * kRowB, b_bytes - (uint32_t)st_ * kRowB);      \
    _Pragma("unroll") for (int q = 2 * (P); q < 2 * (P) + 2; q++) {                               \
      llvm_amdgcn_raw_buffer_load_lds(ra_, (lds_u32)((SP) + (wave * 64 + q * 16) * kRowB), 16, a_off[q], 0, 0, 0); \
      llvm_amdgcn_raw_buffer_load_lds(rb_, (lds_u32)((SP) + kOpB + (wave * 64 + q * 16) * kRowB), 16, b_off[q], \
                                      0, 0, 0);                                                   \
    }                                                                                             \
    const v4i rs_ = buf_rsrc(s_base + (size_t)st_ * s_plane, 512);                                \
    llvm_amdgcn_raw_buffer_load_lds(rs_, (lds_u32)((SP) + s_dst + (P) * 256), 4, s_off[P], 0, 0, 0); \
  }
#define MX6_ISSUE(S, SP) MX6_ISSUE_HALF(S, SP, 0) MX6_ISSUE_HALF(S, SP, 1)
#define MX6_READ(RP, s, F)                                                                        \
  {                                                                                               \
    _Pragma("unroll") for (int i = 0; i < 4; i++)                                                 \
      af[F][i] = *reinterpret_cast<const v4i*>((RP) + a_blk + i * 32 * kRowB + lp[s]);            \
    _Pragma("unroll") for (int j = 0; j < 4; j++)                                                 \
      bf[F][j] = *reinterpret_cast<const v4i*>((RP) + b_blk[j] + lp[s]);                          \
  }
#define MX6_SCALES(RP, P)                                                                         \
  {                                                                                               \
    _Pragma("unroll") for (int i = 0; i < 4; i++) {                                               \
      sa[P][i] = *reinterpret_cast<const uint32_t*>((RP) + kScA + (wm * 128 + i * 32 + r32) * 4); \
      sb[P][i] = *reinterpret_cast<const uint32_t*>((RP) + kScB + (bfrag[i] * 32 + r32) * 4);     \
    }                                                                                             \
  }
#define MX6_MMA(F, P, s)                                                                          \
  _Pragma("unroll") for (int i = 0; i < 4; i++)                                                   \
    _Pragma("unroll") for (int j = 0; j < 4; j++) {                                               \
      const int sa_ = (int)(sa[P][i] >> shift), sb_ = (int)(sb[P][j] >> shift);                  \
      if ((s) == 0) acc[i][j] = mfma_fp4_32x32x64<0, 0>(af[F][i], bf[F][j], acc[i][j], sa_, sb_); \
      else acc[i][j] = mfma_fp4_32x32x64<2, 2>(af[F][i], bf[F][j], acc[i][j], sa_, sb_);         \
    }
  // One stage kt = kt0 + J in slot J.  On entry fragment set 0 holds its
  // k-step 0 and scale set J % 2 its scales.  k-step 0 issues the second
  // half of stage kt + 3's DMA (slot J - 1, free since the previous stage's
  // barrier), k-step 1 the first half of stage kt + 4's (slot J).  In issue
  // order, stage kt + 1 is followed by 20 instructions at the barrier.
#define MX6_STAGE(J)                                                                              \
  {                                                                                               \
    const int kt_ = kt0 + (J);                                                                    \
    MX6_READ(ring<(J)>(), 1, 1)                                                                   \
    MX6_ISSUE_HALF(min(kt_ + 3, KT - 1), ring<((J) + 3) & 3>(), 1)                                \
    MX6_MMA(0, (J) & 1, 0)                                                                        \
    /* 16 MFMAs; 8 LDS reads and 5 DMA between them */                                            \
    _Pragma("unroll") for (int q_ = 0; q_ < 8; q_++) {                                            \
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                                          \
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);                                          \
      if (q_ % 2 == 0) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);                         \
    }                                                                                             \
    __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);                                            \
    __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);                                            \
    __builtin_amdgcn_sched_group_barrier(0x008, 6, 0);                                            \
    __builtin_amdgcn_sched_barrier(0);                                                            \
    __builtin_amdgcn_s_waitcnt(wait_lgkm0_vm(2 * kDma));                                          \
    __builtin_amdgcn_s_barrier();                                                                 \
    MX6_ISSUE_HALF(min(kt_ + 4, KT - 1), ring<(J)>(), 0)                                          \
    MX6_READ(ring<((J) + 1) & 3>(), 0, 0)                                                         \
    MX6_SCALES(ring<((J) + 1) & 3>(), ((J) + 1) & 1)                                              \
    MX6_MMA(1, (J) & 1, 1)                                                                        \
    /* 16 MFMAs; 16 LDS reads and 5 DMA between them */                                           \
    _Pragma("unroll") for (int q_ = 0; q_ < 8; q_++) {                                            \
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                                          \
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);                                          \
      if (q_ % 2 == 0) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);                         \
    }                                                                                             \
    __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);                                            \
    __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);                                            \
    __builtin_amdgcn_sched_group_barrier(0x008, 6, 0);                                            \
    __builtin_amdgcn_sched_barrier(0);                                                            \
  }

  MX6_ISSUE(0, ring<0>())
  __builtin_amdgcn_sched_barrier(0);
  MX6_ISSUE(min(1, KT - 1), ring<1>())
  __builtin_amdgcn_sched_barrier(0);
  MX6_ISSUE(min(2, KT - 1), ring<2>())
  __builtin_amdgcn_sched_barrier(0);
  MX6_ISSUE_HALF(min(3, KT - 1), ring<3>(), 0)
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_waitcnt(wait_lgkm0_vm(2 * kDma + kDma / 2));
  __builtin_amdgcn_s_barrier();
  MX6_READ(ring<0>(), 0, 0)
  MX6_SCALES(ring<0>(), 0)
  // The last stages' look-ahead DMAs re-read a clamped (valid, unused) stage.
  for (int kt0 = 0; kt0 < KT; kt0 += 4) {
    MX6_STAGE(0)
    MX6_STAGE(1)
    MX6_STAGE(2)
    MX6_STAGE(3)
  }
#undef MX6_STAGE
#undef MX6_MMA
#undef MX6_SCALES
#undef MX6_READ
#undef MX6_ISSUE
#undef MX6_ISSUE_HALF
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();

  if (!DUAL) {
    uint16_t* c = reinterpret_cast<uint16_t*>(g.c);
    uint64_t nanm[4] = {0u, 0u, 0u, 0u};  // bit j * 16 + v of word i: element is NaN
    // The wave's 128 x 128 outputs go to its own ring slot as an f16 tile
    // (row pitch 136 halves: the slot's 34816 B), then out as 16-byte
    // stores, 16 lanes per 256-byte row, where the accumulator layout gives
    // 256 two-byte stores per lane.  Same box, three alternating runs at
    // C4: down GEMM 401.5-402.8 -> 398.5-402.0 us.  The epilogue's ~10 us
    // per tile is mostly the write burst: 256 CUs store their 128 KB tiles
    // at the same time.  The W4A4 MLP entry points require 16-byte aligned
    // outputs (mx_api.cpp), and N is a whole number of 256-column tiles.
    uint16_t* tile = reinterpret_cast<uint16_t*>(wave == 0 ? ring<0>() : wave == 1 ? ring<1>() : wave == 2 ? ring<2>() : ring<3>());
    constexpr int kPitch = 136;
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
      for (int j = 0; j < 4; j++)
#pragma unroll
        for (int v = 0; v < 16; v++) {
          const float x0 = acc[i][j][v];
          nanm[i] |= (uint64_t)(x0 != x0) << (j * 16 + v);
          tile[(i * 32 + acc32_row(lane, v)) * kPitch + j * 32 + r32] = f32_to_f16_bits(x0);
        }
    // E8M0 byte 255 in a scale is NaN to the scaled MFMA and +inf to the
    // reference (MXFP4Kernels.metal:26-29), whose dequantize-then-accumulate
    // gives +-inf or NaN there: NaN outputs (rare; one wave-uniform test)
    // are recomputed with the reference's dequantization, into the tile.
    if (__builtin_expect(__ballot((nanm[0] | nanm[1] | nanm[2] | nanm[3]) != 0) != 0, 0)) {
#pragma nounroll
      for (int e = 0; e < 256; e++) {
        const int i = e >> 6, j = (e >> 4) & 3, v = e & 15;
        if (!((nanm[i] >> (j * 16 + v)) & 1u)) continue;
        const int row = m0 + wm * 128 + i * 32 + acc32_row(lane, v);
        const int col = nt * 256 + (wn * 4 + j) * 32 + r32;
        if (row < M)
          tile[(i * 32 + acc32_row(lane, v)) * kPitch + j * 32 + r32] =
              f32_to_f16_bits(ref_dot_sm_a(g.a, g.as, Mpad, row, g.b0, g.s0, NB, col, K));
      }
    }
    __syncthreads();  // the tile's elements were written by other lanes of the wave
#pragma unroll 4
    for (int q = 0; q < 32; q++) {
      const int id = q * 64 + lane, r = id >> 4, ch = id & 15;
      const int row = m0 + wm * 128 + r;
      if (row < M)
        *reinterpret_cast<uint4*>(c + (size_t)row * g.n + nt * 256 + wn * 128 + ch * 8) =
            *reinterpret_cast<const uint4*>(tile + r * kPitch + ch * 8);
    }
    return;
  }
  // mid = silu(gate) * up re-quantized along channels, written stage-major
  // for the down GEMM: channels [128 nt, 128 nt + 128) are its stage nt.
  float* mid = reinterpret_cast<float*>(ring0) + wave * (64 * kMidStride);
  uint8_t* mp = reinterpret_cast<uint8_t*>(g.c) + (size_t)nt * Mpad * kRowB;
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
        *reinterpret_cast<uint4*>(mp + (size_t)row * kRowB + (wn * 2 + jb) * 16) = o;
        const int blk = chan0 / 32;
        g.cs[((size_t)(blk >> 2) * Mpad + row) * 4 + (blk & 3)] = (uint8_t)sbyte;
      }
      __syncthreads();
    }
  }
}

}  // namespace

// Whole-tile grids only: K a multiple of 512 (the ring is unrolled by four
// 128-K stages) and N in whole tiles; the caller routes split-K shapes to v5.
bool gemm_fp4_v6_ok(int dual, int n, int k) {
  return k % (4 * kKS) == 0 && n % (dual ? 128 : 256) == 0;
}

bool w4a4_act_stage_major(int t, int hidden, int inter) {
  return t > 0 && w4a4_stage_major_ok(hidden, inter) && gemm_fp4_v6_ok(1, inter, hidden) &&
         gemm_fp4_v6_ok(0, hidden, inter) && gemm_fp4_splits(0, t, hidden, inter) <= 1;
}

hipError_t launch_gemm_fp4_v6(int dual, const Fp4GemmArgs& g, hipStream_t st) {
  if (!gemm_fp4_v6_ok(dual, g.n, g.k) || g.m <= 0 || (g.splits > 1)) return hipErrorInvalidValue;
  const int MT = (g.m + kM - 1) / kM;
  const int NT = dual ? g.n / 128 : g.n / 256;
  const dim3 grid(MT * NT);
  if (dual) hipLaunchKernelGGL((k_gemm_fp4_v6<true>), grid, dim3(256), 0, st, g);
  else hipLaunchKernelGGL((k_gemm_fp4_v6<false>), grid, dim3(256), 0, st, g);
  return hipGetLastError();
}

}  // namespace mx
