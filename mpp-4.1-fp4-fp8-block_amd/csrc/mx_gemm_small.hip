// mx_gemm_small.hip - MXFP4 GEMMs for launches with few tiles: at most 128
// token rows against a few MB of weights (the repo's
// default MLP: T=128, H=1024, I=4096).  f16 activations, MXFP4 weights
// decoded in registers, f32 accumulation (mxfp4_fused_h_f_n64 /
// mxfp4_native_sp_h_f_n64, MXFP4Kernels.metal:42-173, 264-286), with the
// SwiGLU of the fused rows (MPPMLPKernels.metal:186-220) in the gate/up
// epilogue.
//
// At such shapes the 128 x 128 tiles of mx_gemm_q.hip give 64 workgroups
// (gate/up) or need an 8-way K split plus a reduce launch (down), and each
// workgroup runs a long serial chain of stage waits.  Here every launch has
// one small tile per CU, the operands of a workgroup are requested up front
// (whole 128-byte lines by global_load_lds_dwordx4) and the waves split K
// and add their partial sums through LDS at the end:
//
//   gate/up  tile 32 tokens x 64 channels (64 gate + 64 up rows), K = 1024
//            all resident (A 64 KB + B 64 KB); 8 waves = 2 channel blocks x
//            4 K quarters; v_mfma_f32_32x32x16_f16.  A wave holds the gate
//            and the up block of its 32 channels, so a channel's two sums
//            meet in one lane.
//   down     tile 16 tokens x 32 weight rows, K % 1024 == 0; 4 waves, one
//            K quarter each, both 16-row blocks; v_mfma_f32_16x16x32_f16
//            over 128-K steps (a lane's 32 K of a step are one FP4 block).
//            Each wave streams its quarter in 256-K chunks through its own
//            3-slot ring (no data is shared between waves, so no barrier
//            until the final sum).
//
// LDS rows are 128 bytes (one 64-K stage of f16 activations, or 256 K of
// FP4 weights); the 16-byte chunk c of row r sits at c ^ ((r >> 1) & 7), so
// the fragment reads (16 rows x one chunk per 16 lanes) hit distinct banks,
// and every DMA instruction moves 8 whole lines (8 rows x 128 B).
#include "mx_device.h"
#include "mx_internal.h"

namespace mx {
namespace sgemm {

__device__ __forceinline__ void dma16(const void* src, void* lds) {
  __builtin_amdgcn_global_load_lds(src, lds, 16, 0, 0);
}
// s_waitcnt immediate (gfx9 encoding): vmcnt(n) only.
constexpr int wait_vm(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }

__device__ __forceinline__ int swz(int row) { return (row >> 1) & 7; }

// Byte `i` (0..7) of a pair of dwords.
__device__ __forceinline__ uint32_t byte_of(uint32_t lo, uint32_t hi, int i) {
  return ((i < 4 ? lo : hi) >> (8 * (i & 3))) & 255u;
}

// 8 FP4 codes -> 8 halves with E8M0 byte `sb`; EXACT takes the reference's
// byte-255 semantics (+inf) where the hardware reads NaN.
template <bool EXACT>
__device__ __forceinline__ v8h fp4_dec(uint32_t w, uint32_t sb) {
  return EXACT ? fp4x8_dequant_f16(w, sb) : fp4x8_to_f16x8(w, e8m0_as_cvt_scale(sb));
}

__device__ __forceinline__ float silu_f(float g) { return g / (1.0f + expf(-g)); }

// ---------------------------------------------------------------------------
// gate/up + SwiGLU.  Grid: tiles_m * (n / 64) workgroups, block b -> M tile
// b / tiles_n, channel tile b % tiles_n (the M tiles of one channel tile sit
// tiles_n apart, on one XCD when tiles_n % 8 == 0, so they share its L2).
template <int EPI>
__global__ __launch_bounds__(512) void k_small_gate_up(QGemmArgs g) {
  constexpr int K = 1024;
  // One __shared__ array per A stage ([kq][row][128 B]) and one for B
  // ([wave][row][128 B]): the compiler's wait insertion tells DMA targets
  // apart by array, so a stage's fragment reads wait for that stage's DMAs
  // only (one shared array made it wait for every DMA before the first read).
  __shared__ __attribute__((aligned(16))) uint8_t a_s0[4 * 32 * 128];
  __shared__ __attribute__((aligned(16))) uint8_t a_s1[4 * 32 * 128];
  __shared__ __attribute__((aligned(16))) uint8_t a_s2[4 * 32 * 128];
  __shared__ __attribute__((aligned(16))) uint8_t a_s3[4 * 32 * 128];
  __shared__ __attribute__((aligned(16))) uint8_t b_lds[8 * 64 * 128];
  __shared__ __attribute__((aligned(16))) uint8_t pf_lds[512 * 16];  // prefetch landing, never read
#define MXS_A(ST) ((ST) == 0 ? a_s0 : (ST) == 1 ? a_s1 : (ST) == 2 ? a_s2 : a_s3)
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int cb = wave & 1, kq = wave >> 1;
  const int M = g.m;
  const int tiles_n = g.n / 64;
  const int m0 = (int)(blockIdx.x / tiles_n) * 32;
  const int c0 = (int)(blockIdx.x % tiles_n) * 64 + cb * 32;  // first channel of the wave's block
  const uint8_t* wg = reinterpret_cast<const uint8_t*>(g.b0);
  const uint8_t* wu = reinterpret_cast<const uint8_t*>(g.b1);
  const uint8_t* sg = reinterpret_cast<const uint8_t*>(g.s0);
  const uint8_t* su = reinterpret_cast<const uint8_t*>(g.s1);
  const uint8_t* x = reinterpret_cast<const uint8_t*>(g.a);
  const int j = lane & 31, h = lane >> 5;

  // 1. E8M0 bytes of the lane's gate and up rows over the wave's K quarter
  //    (8 blocks: dwords kq*2, kq*2+1 of a 32-byte row)
  uint32_t sc[2][2];
  {
    const uint32_t* pg = reinterpret_cast<const uint32_t*>(sg + (size_t)(c0 + j) * (K / 32)) + kq * 2;
    const uint32_t* pu = reinterpret_cast<const uint32_t*>(su + (size_t)(c0 + j) * (K / 32)) + kq * 2;
    sc[0][0] = pg[0]; sc[0][1] = pg[1];
    sc[1][0] = pu[0]; sc[1][1] = pu[1];
  }
  // 2. B: the wave's 64 rows (32 gate, 32 up) x its K quarter, one line each
  uint8_t* bw = b_lds + wave * 8192;
#pragma unroll
  for (int q = 0; q < 8; q++) {
    const int r = 8 * q + (lane >> 3);
    const int lc = (lane & 7) ^ swz(r);
    const uint8_t* base = r < 32 ? wg : wu;
    dma16(base + (size_t)(c0 + (r & 31)) * (K / 2) + kq * 128 + lc * 16, bw + q * 1024);
  }
  // 3. A: stage st of the quarter = 32 rows x 128 B; channel block cb issues
  //    rows [16 cb, 16 cb + 16) of it
#pragma unroll
  for (int st = 0; st < 4; st++) {
#pragma unroll
    for (int q = 0; q < 2; q++) {
      const int r = 16 * cb + 8 * q + (lane >> 3);
      const int lc = (lane & 7) ^ swz(r);
      dma16(x + (size_t)min(m0 + r, M - 1) * (K * 2) + (kq * 256 + st * 64) * 2 + lc * 16,
            MXS_A(st) + (kq * 32 + 16 * cb + 8 * q) * 128);
    }
  }

  // 3b. One 16-byte DMA per thread pulls a share of the next GEMM's weights
  //    (g.pf) into this XCD's L2: the rows whose 32-row tile the plain
  //    kernel's grid places on this XCD (tile t on XCD t % 8, the workgroup
  //    order's round robin), split over this XCD's workgroups.  Issued
  //    behind this kernel's own loads, it overlaps their latency; the next
  //    kernel then starts on L2 hits (C0's down GEMM: first data 2.7 ->
  //    1.7 us).  Every thread issues it (a dummy address without g.pf), so
  //    the stage waits below count it.
  {
    const uint8_t* src = x;
    if (g.pf && g.pf_rows % 256 == 0) {
      const int xcd = (int)(blockIdx.x & 7), nwg = ((int)gridDim.x - xcd + 7) / 8, i = (int)(blockIdx.x >> 3);
      const int rb = g.pf_row_bytes;
      const long pieces = (long)(g.pf_rows / 8) * (rb / 16);  // 16-byte pieces on this XCD
      const long share = (pieces + nwg - 1) / nwg;
      long pc = (long)i * share + tid;
      if (pc >= pieces) pc = pieces - 1;
      const long off = pc * 16;
      const int rl = (int)(off / rb), n = (rl / 32) * 256 + xcd * 32 + rl % 32;
      src = reinterpret_cast<const uint8_t*>(g.pf) + (size_t)n * rb + off % rb;
    }
    dma16(src, pf_lds + wave * 1024);
  }

  v16f acc[2];
#pragma unroll
  for (int b = 0; b < 2; b++)
#pragma unroll
    for (int v = 0; v < 16; v++) acc[b][v] = 0.0f;

  // 4. stages: wait for the wave's loads up to this stage, one barrier (the
  //    partner wave's half of A), then 2 blocks x 4 k-steps of MFMAs.  Lane
  //    half h takes K [32 h, 32 h + 32) of each 64-K stage, in both operands.
#define MXS_STAGE(ST)                                                                              \
  {                                                                                                \
    __builtin_amdgcn_sched_barrier(0);                                                             \
    __builtin_amdgcn_s_waitcnt(wait_vm(2 * (3 - (ST)) + 1)); /* + the prefetch DMA */             \
    __builtin_amdgcn_s_barrier();                                                                  \
    __builtin_amdgcn_sched_barrier(0);                                                             \
    const uint8_t* as_ = MXS_A(ST) + kq * 32 * 128;                                                \
    v4i af_[4], bf_[2];                                                                            \
    _Pragma("unroll") for (int s = 0; s < 4; s++)                                                  \
      af_[s] = *reinterpret_cast<const v4i*>(as_ + j * 128 + (((4 * h + s) ^ swz(j)) << 4));       \
    _Pragma("unroll") for (int b = 0; b < 2; b++) {                                                \
      const int r_ = 32 * b + j;                                                                   \
      bf_[b] = *reinterpret_cast<const v4i*>(bw + r_ * 128 + (((2 * (ST) + h) ^ swz(r_)) << 4));   \
    }                                                                                              \
    const uint32_t s0_ = byte_of(sc[0][0], sc[0][1], 2 * (ST) + h);                                \
    const uint32_t s1_ = byte_of(sc[1][0], sc[1][1], 2 * (ST) + h);                                \
    const bool ex_ = __ballot(s0_ == 255u || s1_ == 255u) != 0;                                    \
    if (__builtin_expect(ex_, 0)) {                                                                \
      _Pragma("unroll") for (int s = 0; s < 4; s++) {                                              \
        const v8h a_ = __builtin_bit_cast(v8h, af_[s]);                                            \
        acc[0] = mfma_f16_32x32x16(a_, fp4_dec<true>(bf_[0][s], s0_), acc[0]);                     \
        acc[1] = mfma_f16_32x32x16(a_, fp4_dec<true>(bf_[1][s], s1_), acc[1]);                     \
      }                                                                                            \
    } else {                                                                                       \
      _Pragma("unroll") for (int s = 0; s < 4; s++) {                                              \
        const v8h a_ = __builtin_bit_cast(v8h, af_[s]);                                            \
        acc[0] = mfma_f16_32x32x16(a_, fp4_dec<false>(bf_[0][s], s0_), acc[0]);                    \
        acc[1] = mfma_f16_32x32x16(a_, fp4_dec<false>(bf_[1][s], s1_), acc[1]);                    \
      }                                                                                            \
    }                                                                                              \
  }
  MXS_STAGE(0) MXS_STAGE(1) MXS_STAGE(2) MXS_STAGE(3)
#undef MXS_STAGE
#undef MXS_A

  // 5. Every wave parks its sums in LDS ([kq][cb][b][v][lane], 64 KB over
  //    B); wave (cb, kq) then adds the four K quarters in order
  //    (deterministic) for its accumulator rows v = 4 kq .. 4 kq + 3, applies
  //    the SwiGLU and writes mid into an f16 tile [32 rows][64 channels] in
  //    LDS, which goes out as one 16-byte store per thread (per-element
  //    stores behind row guards are serialised by the compiler: 2.8 us).
  __syncthreads();
  v4f* red = reinterpret_cast<v4f*>(b_lds);  // [kq][cb][b][v / 4][lane] x 4 floats
#pragma unroll
  for (int b = 0; b < 2; b++)
#pragma unroll
    for (int vq = 0; vq < 4; vq++)
      red[(((kq * 2 + cb) * 2 + b) * 4 + vq) * 64 + lane] =
          (v4f){acc[b][4 * vq], acc[b][4 * vq + 1], acc[b][4 * vq + 2], acc[b][4 * vq + 3]};
  __syncthreads();
  v4f sum[2];
#pragma unroll
  for (int b = 0; b < 2; b++) {
    sum[b] = red[(((0 * 2 + cb) * 2 + b) * 4 + kq) * 64 + lane];
#pragma unroll
    for (int q = 1; q < 4; q++) sum[b] += red[(((q * 2 + cb) * 2 + b) * 4 + kq) * 64 + lane];
  }
  uint16_t* tile = reinterpret_cast<uint16_t*>(a_s0);  // [32][64] f16, row pitch 128 B
#pragma unroll
  for (int vv = 0; vv < 4; vv++) {
    const int v = 4 * kq + vv;
    const float t[2] = {sum[0][vv], sum[1][vv]};
    float mv;
    if (EPI == EPI_SWIGLU_HALF) {  // swiglu_half: silu(clamp(g/16, +-20)) * u/16
      const float gg = fminf(fmaxf(t[0] * 0.0625f, -20.0f), 20.0f);
      mv = silu_f(gg) * (t[1] * 0.0625f);
    } else {
      mv = silu(t[0]) * t[1];
    }
    tile[acc32_row(lane, v) * 64 + cb * 32 + j] = f32_to_f16_bits(mv);
  }
  __syncthreads();
  if (tid < 256) {  // row tid / 8, channels 8 (tid % 8) .. + 8
    const int r = tid >> 3, row = m0 + r;
    if (row < M) {
      const uint4 v = *reinterpret_cast<const uint4*>(tile + r * 64 + (tid & 7) * 8);
      const int ct = (int)(blockIdx.x % tiles_n) * 64;
      *reinterpret_cast<uint4*>(reinterpret_cast<uint16_t*>(g.c) + (size_t)row * g.n + ct + (tid & 7) * 8) = v;
    }
  }
}

// ---------------------------------------------------------------------------
// Plain GEMM (down).  Grid: tiles_m * (n / 32), block b -> M tile
// b / tiles_n, weight-row tile b % tiles_n.  NC = 256-K chunks per wave.
constexpr int kDnSlots = 3;
constexpr int kDnSlotBytes = 16 * 512 + 32 * 128;  // A 16 rows x 256 K f16 + B 32 rows x 256 K FP4
constexpr int kDnOps = 12;                          // vector-memory ops per chunk (8 A + 4 B DMAs)

template <int EPI, int NC>
__global__ __launch_bounds__(256) void k_small_store(QGemmArgs g) {
  // One __shared__ array per ring slot ([wave][slot bytes]), so that a
  // slot's fragment reads wait only for that slot's DMAs.
  __shared__ __attribute__((aligned(16))) uint8_t ring0[4 * kDnSlotBytes];
  __shared__ __attribute__((aligned(16))) uint8_t ring1[4 * kDnSlotBytes];
  __shared__ __attribute__((aligned(16))) uint8_t ring2[4 * kDnSlotBytes];
  static_assert(kDnSlots == 3, "three ring arrays");
  const int tid = threadIdx.x, lane = tid & 63;
  const int kq = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int M = g.m, N = g.n, K = g.k;
  const int tiles_n = N / 32;
  const int m0 = (int)(blockIdx.x / tiles_n) * 16;
  const int n0 = (int)(blockIdx.x % tiles_n) * 32;
  const int kw = K / 4;  // the wave's K range [kq kw, +kw), NC chunks of 256
  const uint8_t* w = reinterpret_cast<const uint8_t*>(g.b0);
  const uint8_t* s = reinterpret_cast<const uint8_t*>(g.s0);
  const uint8_t* x = reinterpret_cast<const uint8_t*>(g.a);
  const int j = lane & 15, q4 = lane >> 4;

  // E8M0 bytes of the lane's two rows (16 b + j) over the wave's K range:
  // 8 blocks per chunk, two dwords
  uint32_t sc[2][NC][2];
#pragma unroll
  for (int b = 0; b < 2; b++) {
    const uint32_t* p = reinterpret_cast<const uint32_t*>(s + (size_t)(n0 + 16 * b + j) * (K / 32) + kq * (kw / 32));
#pragma unroll
    for (int c = 0; c < NC; c++) { sc[b][c][0] = p[2 * c]; sc[b][c][1] = p[2 * c + 1]; }
  }
  // the wave's part of ring slot I (a constant: the slot's array must be
  // known where the DMA and the reads are compiled)
#define MXS_SLOT(I) (((I) == 0 ? ring0 : (I) == 1 ? ring1 : ring2) + kq * kDnSlotBytes)
  // chunk C -> slot C % 3: A [4 stages][16 rows][128 B], then B [32 rows][128 B]
#define MXS_ISSUE(C)                                                                               \
  {                                                                                                \
    uint8_t* sl_ = MXS_SLOT((C) % kDnSlots);                                                       \
    const int kb_ = kq * kw + (C) * 256;                                                           \
    _Pragma("unroll") for (int q = 0; q < 8; q++) {                                                \
      const int st_ = q >> 1, r_ = 8 * (q & 1) + (lane >> 3);                                      \
      const int lc_ = (lane & 7) ^ swz(r_);                                                        \
      dma16(x + (size_t)min(m0 + r_, M - 1) * ((size_t)K * 2) + (size_t)(kb_ + st_ * 64) * 2 + lc_ * 16, \
            sl_ + (st_ * 16 + 8 * (q & 1)) * 128);                                                 \
    }                                                                                              \
    _Pragma("unroll") for (int q = 0; q < 4; q++) {                                                \
      const int r_ = 8 * q + (lane >> 3);                                                          \
      const int lc_ = (lane & 7) ^ swz(r_);                                                        \
      dma16(w + (size_t)(n0 + r_) * (K / 2) + kb_ / 2 + lc_ * 16, sl_ + 16 * 512 + q * 1024);      \
    }                                                                                              \
  }
  MXS_ISSUE(0)
  if constexpr (NC > 1) MXS_ISSUE(1)
  if constexpr (NC > 2) MXS_ISSUE(2)

  v4f acc[2];
#pragma unroll
  for (int b = 0; b < 2; b++)
#pragma unroll
    for (int v = 0; v < 4; v++) acc[b][v] = 0.0f;

  // 128-K steps (two per chunk): lane group q4 takes K [32 q4, 32 q4 + 32)
  // of each step in both operands, 8 per MFMA (t = 0..3), i.e. one 16-byte
  // FP4 read per row and step (one E8M0 byte, block 4 s + q4 of the chunk)
  // and A stage-row 2 s + q4 / 2, chunks 4 (q4 & 1) + t.
#pragma unroll
  for (int c = 0; c < NC; c++) {
    // chunks in flight after this one: min(NC, c + 3) - c - 1
    constexpr int kAhead = kDnSlots - 1;
    const int ahead = (NC - 1 - c) < kAhead ? (NC - 1 - c) : kAhead;
    __builtin_amdgcn_sched_barrier(0);
    if (ahead >= 2) __builtin_amdgcn_s_waitcnt(wait_vm(2 * kDnOps));
    else if (ahead == 1) __builtin_amdgcn_s_waitcnt(wait_vm(kDnOps));
    else __builtin_amdgcn_s_waitcnt(wait_vm(0));
    __builtin_amdgcn_sched_barrier(0);
    const uint8_t* sl = MXS_SLOT(c % kDnSlots);
    v4i af[2][4], bf[2][2];
#pragma unroll
    for (int s = 0; s < 2; s++) {
      const int sr = 2 * s + (q4 >> 1);  // A stage-row
#pragma unroll
      for (int t = 0; t < 4; t++)
        af[s][t] = *reinterpret_cast<const v4i*>(sl + (sr * 16 + j) * 128 + (((4 * (q4 & 1) + t) ^ swz(j)) << 4));
#pragma unroll
      for (int b = 0; b < 2; b++) {
        const int r = 16 * b + j;
        bf[s][b] = *reinterpret_cast<const v4i*>(sl + 16 * 512 + r * 128 + (((4 * s + q4) ^ swz(r)) << 4));
      }
    }
    uint32_t sb[2][2];
    uint32_t hit = 0;
#pragma unroll
    for (int s = 0; s < 2; s++)
#pragma unroll
      for (int b = 0; b < 2; b++) {
        sb[s][b] = byte_of(sc[b][c][0], sc[b][c][1], 4 * s + q4);
        hit |= sb[s][b] == 255u;
      }
    if (__builtin_expect(__ballot(hit != 0) != 0, 0)) {
#pragma unroll
      for (int s = 0; s < 2; s++)
#pragma unroll
        for (int t = 0; t < 4; t++)
#pragma unroll
          for (int b = 0; b < 2; b++)
            acc[b] = mfma_f16_16x16x32(__builtin_bit_cast(v8h, af[s][t]), fp4_dec<true>(bf[s][b][t], sb[s][b]), acc[b]);
    } else {
#pragma unroll
      for (int s = 0; s < 2; s++)
#pragma unroll
        for (int t = 0; t < 4; t++)
#pragma unroll
          for (int b = 0; b < 2; b++)
            acc[b] = mfma_f16_16x16x32(__builtin_bit_cast(v8h, af[s][t]), fp4_dec<false>(bf[s][b][t], sb[s][b]), acc[b]);
    }
    if (c + kDnSlots < NC) {
      // every fragment read of this slot has landed before its refill
      __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
      __builtin_amdgcn_sched_barrier(0);
      MXS_ISSUE(c + kDnSlots)
    }
  }
#undef MXS_ISSUE
#undef MXS_SLOT

  // Every wave parks its sums ([kq][b][v][lane]); wave w adds the four K
  // quarters in order for accumulator row v = w of both blocks, into an
  // output tile [16 rows][32 columns] in LDS that goes out in 16-byte
  // stores (f16: 64 threads, f32: 128).
  __syncthreads();
  float* red = reinterpret_cast<float*>(ring0);
#pragma unroll
  for (int b = 0; b < 2; b++)
#pragma unroll
    for (int v = 0; v < 4; v++) red[((kq * 2 + b) * 4 + v) * 64 + lane] = acc[b][v];
  __syncthreads();
  constexpr int OB = EPI == EPI_STORE_F32 ? 4 : 2;  // output bytes
  uint8_t* tile = ring1;                            // [16][32] outputs, row pitch 32 * OB
#pragma unroll
  for (int b = 0; b < 2; b++) {
    float t = red[((0 * 2 + b) * 4 + kq) * 64 + lane];
#pragma unroll
    for (int q = 1; q < 4; q++) t += red[((q * 2 + b) * 4 + kq) * 64 + lane];
    const int r = 4 * q4 + kq, cc = 16 * b + j;  // 16x16 D: row 4 (lane / 16) + v, column lane % 16
    if (EPI == EPI_STORE_F32) reinterpret_cast<float*>(tile)[r * 32 + cc] = t;
    else reinterpret_cast<uint16_t*>(tile)[r * 32 + cc] = f32_to_f16_bits(t);
  }
  __syncthreads();
  constexpr int PER_ROW = 32 * OB / 16;  // 16-byte pieces per output row
  if (tid < 16 * PER_ROW) {
    const int r = tid / PER_ROW, pc = tid % PER_ROW, row = m0 + r;
    if (row < M) {
      const uint4 v = *reinterpret_cast<const uint4*>(tile + r * 32 * OB + pc * 16);
      *reinterpret_cast<uint4*>(reinterpret_cast<uint8_t*>(g.c) + ((size_t)row * N + n0) * OB + pc * 16) = v;
    }
  }
}

}  // namespace sgemm

using namespace sgemm;

// Shapes this family takes (f16 activations, MXFP4 weights): at most 128
// token rows, and either the dual gate/up GEMM at K = 1024 with channels % 64,
// or a plain GEMM with K a multiple of 1024 up to 4096 and N % 32 up to 2048.
bool small_gemm_ok(int epi, int m, int n, int k) {
  if (m <= 0 || m > 128) return false;
  if (epi == EPI_SWIGLU_F16 || epi == EPI_SWIGLU_HALF) return k == 1024 && n % 64 == 0 && n > 0;
  if (epi == EPI_STORE_F16 || epi == EPI_STORE_F32)
    return k % 1024 == 0 && k <= 4096 && n % 32 == 0 && n > 0 && n <= 2048;
  return false;
}

hipError_t launch_small_gemm(int epi, const QGemmArgs& g, hipStream_t st) {
  if (!small_gemm_ok(epi, g.m, g.n, g.k)) return hipErrorInvalidValue;
  if (epi == EPI_SWIGLU_F16 || epi == EPI_SWIGLU_HALF) {
    const unsigned blocks = (unsigned)((g.m + 31) / 32 * (g.n / 64));
    if (epi == EPI_SWIGLU_F16) hipLaunchKernelGGL(k_small_gate_up<EPI_SWIGLU_F16>, dim3(blocks), dim3(512), 0, st, g);
    else hipLaunchKernelGGL(k_small_gate_up<EPI_SWIGLU_HALF>, dim3(blocks), dim3(512), 0, st, g);
    return hipGetLastError();
  }
  const unsigned blocks = (unsigned)((g.m + 15) / 16 * (g.n / 32));
#define MXS_LAUNCH(E, NC) hipLaunchKernelGGL((k_small_store<E, NC>), dim3(blocks), dim3(256), 0, st, g)
  const int nc = g.k / 1024;  // chunks of 256 K per wave
  if (epi == EPI_STORE_F16) {
    switch (nc) {
      case 1: MXS_LAUNCH(EPI_STORE_F16, 1); break;
      case 2: MXS_LAUNCH(EPI_STORE_F16, 2); break;
      case 3: MXS_LAUNCH(EPI_STORE_F16, 3); break;
      default: MXS_LAUNCH(EPI_STORE_F16, 4); break;
    }
  } else {
    switch (nc) {
      case 1: MXS_LAUNCH(EPI_STORE_F32, 1); break;
      case 2: MXS_LAUNCH(EPI_STORE_F32, 2); break;
      case 3: MXS_LAUNCH(EPI_STORE_F32, 3); break;
      default: MXS_LAUNCH(EPI_STORE_F32, 4); break;
    }
  }
#undef MXS_LAUNCH
  return hipGetLastError();
}

}  // namespace mx
