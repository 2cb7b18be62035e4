// mx_gemv.hip - decode-shaped (tokens <= 16) MXFP4 GEMV.
//
// The reference runs every shape through the same 64 x NT matmul2d tile
// (MXFP4Kernels.metal:138-173) and only for tokens % 64 == 0
// (main.swift:946).  On MI355X a 1..16-token MLP is bound by HBM and by the
// fixed cost of a launch: the whole job is streaming 4-bit weights once, so
// this kernel is shaped for that.
//
//   workgroup = 16 weight rows x the whole K; its W waves split K between
//               them (wave w takes 128-K steps w, w+W, ...), so at any time
//               the workgroup sweeps one contiguous stretch of each row.
//               For the gate/up pass the 16 rows are 8 gate channels and the
//               same 8 up channels, so silu(g)*u is formed in the workgroup.
//   lane      = (row r = lane % 16, block group g = lane / 16); per step it
//               loads 16 contiguous bytes of its row (one whole 32-element
//               E8M0 block), decodes them with v_cvt_scalef32_pk_f16_fp4 and
//               feeds v_mfma_f32_16x16x32_f16 (tokens padded to 16 rows; the
//               MFMA is never the bottleneck).  The activations follow the
//               same K permutation.  In the whole-line layout the loads move
//               two steps of 8 rows (one 128-byte line each) and the lanes
//               swap halves with a DPP rotate to get the same operands.
//   order     = the activations (LDS DMA) and the rows' E8M0 scales (LDS
//               DMA of 16-byte pieces in the single launches, dwords through
//               registers in the grouped ones) are requested first, then the
//               wave's weight loads (scheduling barriers keep the order): all
//               of them, or, for whole lines with more than two line columns
//               per wave, two columns with one more issued as each lands.
//               vmcnt retires in order, so the staging can be waited for
//               while the weights are still in flight.
//   reduction = the W partial 16x16 tiles are added in LDS in wave order
//               (deterministic, one barrier), then the epilogue writes f16:
//                 single: out[t][n] = sum
//                 dual:   mid[t][c] = silu(sum_gate) * sum_up  (swiglu_float)
//
// Measured on MI355X: a one-shot launch of this size is dominated by fixed
// costs (an empty kernel costs ~2.5 us back to back, a pure 14.7 MB read
// ~4 us); cross-workgroup synchronisation is far worse (an agent-scope grid
// barrier costs ~14 us), so gate/up and down stay two plain launches.
#include "mx_device.h"
#include "mx_internal.h"

namespace mx {

constexpr int kStepK = 128;   // K per lane step: 4 lane groups x 32-element blocks
// NSTEP: steps per wave whose weight loads are issued together (2, 4 or 8).
constexpr int kW = 8;         // waves per workgroup
// scale dwords staged per thread (a quarter as many 16-byte pieces): 4 up
// to two row groups per workgroup (K <= 16384), 8 for four and 16 for eight
// (launchers check K)
constexpr int scale_regs(int ng) { return ng <= 2 ? 4 : ng <= 4 ? 8 : 16; }

// 16-byte global -> LDS DMA of one lane (LDS base wave-uniform).
__device__ __forceinline__ void dma16(const void* src, void* lds) {
  __builtin_amdgcn_global_load_lds(src, lds, 16, 0, 0);
}

// s_waitcnt immediate (gfx9 encoding): vmcnt(n), expcnt and lgkmcnt untouched.
constexpr int gemv_wait_vm(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }

// Dynamic LDS layout: [scales 16 rows x K/32 bytes][x T rows x (K+8) halves]
// [reduction W x 16 x 17 floats].
__host__ __device__ inline size_t gemv_lds_bytes(int t, int k, int ng = 1) {
  const size_t s = (size_t)16 * ng * (k / 32);
  const size_t xs = (size_t)t * (k + 8) * 2;
  return ((s + 15) / 16) * 16 + ((xs + 15) / 16) * 16 + (size_t)kW * 16 * 17 * 4;
}

// One workgroup: NG = kW / WPG row groups g0 .. g0+NG-1 (row group g =
// weight rows 16g .. 16g+15, or gate / up channels 8g .. 8g+7) over all of
// K; WPG waves share each group's K steps.  More groups per workgroup stage
// x once for more rows (the activations are T x K, as large as 16 rows of
// weights at T = 4).
// WL picks the weight load layout.  Whole lines (WL): one load moves one
// 128-byte line (two K steps) of 8 rows.  Half lines: one load moves one K
// step (64 bytes) of all 16 rows.
// TSKIP: whole-line columns past the last one are not loaded (the grouped
// launches), instead of re-reading the last one.
template <bool DUAL, int NSTEP, int WPG, bool WL, bool SC16, bool TSKIP>
__device__ __forceinline__ void gemv_body(const GemvArgs& g, int g0, uint8_t* lds) {
  constexpr int NG = kW / WPG;
  static_assert(NG * WPG == kW && NG <= 8, "row groups per workgroup");
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int gi = wave / WPG, gw = wave % WPG;  // this wave's group and its index in the group
  const int r = lane & 15, lg = lane >> 4;
  const int K = g.k, T = g.t;
  const int S = K / kStepK;
  const int KB = K / 32;
  uint8_t* s_lds = lds;
  uint16_t* x_lds = reinterpret_cast<uint16_t*>(lds + (((size_t)16 * NG * KB + 15) / 16) * 16);
  float* red = reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(x_lds) +
                                        (((size_t)T * (K + 8) * 2 + 15) / 16) * 16);

  // Weight / scale row of workgroup row `wr` (0 .. 16 NG - 1).
  auto row_ptrs = [&](int wr, const uint8_t*& w, const uint8_t*& s) {
    const int grp = g0 + wr / 16, rr = wr % 16;
    if (DUAL) {
      const int c = grp * 8 + (rr & 7);
      w = (rr < 8 ? g.b0 : g.b1) + (size_t)c * (K / 2);
      s = (rr < 8 ? g.s0 : g.s1) + (size_t)c * KB;
    } else {
      const int n = grp * 16 + rr;
      w = g.b0 + (size_t)n * (K / 2);
      s = g.s0 + (size_t)n * KB;
    }
  };
  const uint8_t* wrow;
  const uint8_t* srow;
  row_ptrs(gi * 16 + r, wrow, srow);
  wrow += lg * 16;
  // Whole-line loads.  K line column c (256 K = one 128-byte line per row)
  // holds steps 2c and 2c+1.  Load A moves rows 0-7 of the group, load B rows
  // 8-15: 8 whole lines per instruction, against 16 half lines when each load
  // is one step of all 16 rows (measured, weights alone at C1 gate/up: 3.5
  // against 4.5 us).  Lane (r, lg) takes 16 bytes of step 2c of its own row
  // from the load holding that row, and 16 bytes of step 2c+1 of row r ^ 8
  // from the other load, so that step 2c is a per-lane select of A / B and
  // step 2c+1 is the other select rotated by 8 lanes (DPP row_ror:8).
  const uint8_t* wA;
  const uint8_t* wB;
  const uint8_t* s_unused;
  row_ptrs(gi * 16 + (r & 7), wA, s_unused);
  row_ptrs(gi * 16 + 8 + (r & 7), wB, s_unused);
  wA += lg * 16;
  wB += lg * 16;
  const int hiA = r >= 8 ? 64 : 0, hiB = r < 8 ? 64 : 0;  // A / B lanes holding step 2c+1
  const int LC = (S + 1) / 2;                               // line columns (the last may be half)
  constexpr int NLC = NSTEP / 2;                            // line columns per batch
  static_assert(NSTEP % 2 == 0, "line columns load in pairs");

  // 1) Staging first: x rows go global -> LDS by DMA (no registers), the 16
  //    rows' scales into a few registers.  Issued before the weight loads,
  //    they complete first (vmcnt retires in order), so waiting for them
  //    does not wait for the weights.
  {
    const int xrow_b = K * 2, xchunks = (xrow_b + 1023) / 1024;
    for (int i = wave; i < T * xchunks; i += kW) {  // wave-uniform
      const int t = i / xchunks, c = i % xchunks;
      if (c * 1024 + lane * 16 < xrow_b)
        dma16(reinterpret_cast<const uint8_t*>(g.x) + (size_t)t * xrow_b + c * 1024 + lane * 16,
              reinterpret_cast<uint8_t*>(x_lds) + (size_t)t * (K + 8) * 2 + c * 1024);
    }
  }
  // The rows' E8M0 bytes, one piece per thread and pass.  Each 8-row block
  // (8 gate or 8 up channels, or 8 consecutive rows) is contiguous in
  // memory and in LDS.  SC16 (16-byte aligned planes): 16-byte pieces DMA'd
  // straight to LDS; waves wholly past the pieces issue nothing and lanes
  // past the end are masked.  Otherwise: dwords through registers; passes
  // wholly past the pieces are skipped and lanes past the end re-read the
  // last dword (no predicated loads).  Measured at C1: gate/up 5.95 -> 5.62
  // us with 16-byte pieces, -> 5.28 us with the idle waves skipped (the
  // staging barrier waits for every wave's loads; whole waves re-reading one
  // line had also made the grouped launches slower with pieces), down 4.05
  // -> 4.0 us by DMA instead of through registers; 64 experts x 4 tokens
  // 277.7 -> 269.8 us per MoE MLP.  Skipping the dword passes past the
  // scales took the C1 down pass from 4.27 to 3.94 us.
  constexpr int SPAS = SC16 ? scale_regs(NG) / 4 : scale_regs(NG);  // passes of 64 kW pieces
  const int QB = SC16 ? KB / 2 : 2 * KB;                             // pieces per 8-row block
  const int n_sq = 2 * NG * QB;                                      // pieces of the workgroup's rows
  uint32_t sreg[SPAS][1];  // dword pieces (the 16-byte pieces go to LDS by DMA)
#pragma unroll
  for (int q = 0; q < SPAS; q++) {
    if (q * 64 * kW + (SC16 ? wave * 64 : 0) >= n_sq) break;
    const int j = min(tid + q * 64 * kW, n_sq - 1);
    const int b = j / QB, o = j % QB;
    const uint8_t* w;
    const uint8_t* s;
    row_ptrs(8 * b, w, s);
    if constexpr (SC16) {  // straight to LDS by DMA: lane l writes piece q 64 kW + 64 wave + l
      if (tid + q * 64 * kW < n_sq) dma16(s + o * 16, s_lds + (size_t)(q * 64 * kW + wave * 64) * 16);
    } else {
      sreg[q][0] = *reinterpret_cast<const uint32_t*>(s + o * 4);
    }
  }
  __builtin_amdgcn_sched_barrier(0);

  // 2) This wave's first batch of weight loads: line columns gw + i WPG,
  //    A then B.  Tail columns re-read the last valid one; in a half column
  //    (odd S) the lanes of step 2c+1 re-read step 2c.
  uint4 wv[NSTEP];
  // Rolling issue (whole lines): RD line columns are requested up front, then
  // one more each time the oldest one has landed, so that the decode and
  // MFMAs of landed columns overlap the rest of the stream.  Measured at C1
  // T=1, gate/up (4 columns per wave): all up front 6.58 us; half up front
  // and the rest once those landed 6.16 us; rolling 1 / 2 / 3 columns 6.36 /
  // 6.06 / 6.29 us.
  constexpr int RD = 2;
  constexpr bool ROLL = WL && RD < NLC;
  auto load_cols = [&](int p0, int i0, int i1) {
#pragma unroll
    for (int i = i0; i < i1; i++) {
      // Measured: 64 experts x 4 tokens 276.8 -> 268 us per MoE MLP with the
      // tail columns skipped; C1's gate/up 5.33 -> 5.83 us (its rolling
      // issue then gets conservative waits), so the single launches re-read.
      if (TSKIP && p0 + i * WPG >= LC) break;  // wave-uniform; those steps are skipped
      const int c = min(p0 + i * WPG, LC - 1);
      const bool two = 2 * c + 1 < S;
      const v4i a4 = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(wA + (size_t)c * 128 + (two ? hiA : 0)));
      wv[2 * i] = make_uint4(a4[0], a4[1], a4[2], a4[3]);
      __builtin_amdgcn_sched_barrier(0);
      const v4i b4 = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(wB + (size_t)c * 128 + (two ? hiB : 0)));
      wv[2 * i + 1] = make_uint4(b4[0], b4[1], b4[2], b4[3]);
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  auto load_batch = [&](int p0) {
    if constexpr (WL) {
      load_cols(p0, 0, NLC);
    } else {  // steps p0 + b WPG; tail steps re-read a valid step
#pragma unroll
      for (int b = 0; b < NSTEP; b++) {
        const int st = min(p0 + b * WPG, S - 1);
        const v4i w4 = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(wrow + (size_t)st * 64));
        wv[b] = make_uint4(w4[0], w4[1], w4[2], w4[3]);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  };
  if constexpr (ROLL)
    load_cols(gw, 0, RD);
  else
    load_batch(gw);
  constexpr int INFL = ROLL ? 2 * RD : NSTEP;  // weight loads in flight at the staging wait
  static_assert(!TSKIP || WL, "skipped columns are whole-line columns");

  // 3) Staging landed (only the INFL weight loads may still be in flight):
  //    dword scales to LDS, then a bare barrier (__syncthreads would also
  //    wait for the weights).  With TSKIP a wave near the end of K issues
  //    fewer than INFL weight loads (none when its first column is past the
  //    last one), so vmcnt(INFL) would not cover its staging loads: such a
  //    wave waits for all of its loads.  The count is wave-uniform (a
  //    scalar branch around the extra wait).
  if constexpr (TSKIP) {
    const int first = ROLL ? RD : NLC;  // columns the first batch may issue
    const int cols = __builtin_amdgcn_readfirstlane(min(first, max(0, (LC - gw + WPG - 1) / WPG)));
    if (2 * cols < INFL) __builtin_amdgcn_s_waitcnt(gemv_wait_vm(0));
  }
  __builtin_amdgcn_s_waitcnt(gemv_wait_vm(INFL));
#pragma unroll
  for (int q = 0; q < SPAS; q++) {
    const int j = tid + q * 64 * kW;
    if (j < n_sq) {
      if constexpr (!SC16) *reinterpret_cast<uint32_t*>(s_lds + (size_t)j * 4) = sreg[q][0];
    }
  }
  __builtin_amdgcn_s_waitcnt(gemv_wait_vm(INFL) & ~(15 << 8));  // + lgkmcnt(0)
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_sched_barrier(0);

  // E8M0 byte 255 (+inf to the reference, NaN to the hardware) needs an
  // exact decode.  One scan of the workgroup's staged scales decides, so
  // the common loop carries no per-step check or branch.
  bool any255;
  {
    const int nbytes = 16 * NG * KB;  // a multiple of 64: K % 128 == 0
    uint32_t hit = 0;
    for (int i = lane * 16; i < nbytes; i += 64 * 16) {
      const uint4 v = *reinterpret_cast<const uint4*>(s_lds + i);
      const uint32_t d[4] = {~v.x, ~v.y, ~v.z, ~v.w};  // a 0xff byte becomes a zero byte
#pragma unroll
      for (int j = 0; j < 4; j++) hit |= (d[j] - 0x01010101u) & ~d[j] & 0x80808080u;
    }
    any255 = __ballot(hit != 0) != 0;
  }

  // Lane r feeds activation row r; rows >= T re-read row T-1 (their MFMA rows
  // are never stored), so no load or read is predicated.  Four accumulators
  // (one per 32-K slice of a step) keep four independent MFMA chains.
  const uint16_t* xr = x_lds + (size_t)(r < T ? r : T - 1) * (K + 8) + lg * 32;
  const uint8_t* sr = s_lds + (size_t)(gi * 16 + r) * KB + lg;
  v4f acc[4] = {};
  if (__builtin_expect(any255, 0)) {
    // Rare: one step at a time, weights re-read (the batch above is left in
    // flight), so this path holds few registers next to the unrolled one.
#pragma nounroll
    for (int st = gw; st < S; st += WPG) {
      const uint4 w = *reinterpret_cast<const uint4*>(wrow + (size_t)st * 64);
      const uint32_t wd[4] = {w.x, w.y, w.z, w.w};
      const uint32_t sbyte = sr[(size_t)st * 4];
#pragma unroll
      for (int q = 0; q < 4; q++) {
        const uint4 xq = *reinterpret_cast<const uint4*>(xr + (size_t)st * kStepK + q * 8);
        acc[q] = mfma_f16_16x16x32(__builtin_bit_cast(v8h, xq), fp4x8_dequant_f16(wd[q], sbyte), acc[q]);
      }
    }
  } else {
    // Batch positions p0 count line columns (whole lines) or steps.
    constexpr int PER = WL ? NLC : NSTEP;
    const int P = WL ? LC : S;
    for (int p0 = gw; p0 < P; p0 += WPG * PER) {
      if (p0 != gw) load_batch(p0);  // later batches (more than one per wave)
      // Steps of the batch in order (whole lines: 2c, 2c+1 per column).  LDS
      // operands are read one step ahead of their MFMAs so that LDS latency
      // overlaps the previous step's decode and MFMAs.
      auto step_of = [&](int k) { return WL ? 2 * (p0 + (k >> 1) * WPG) + (k & 1) : p0 + k * WPG; };
      uint4 xn[4];
      uint32_t sn;
      {
        const int st = min(step_of(0), S - 1);
#pragma unroll
        for (int q = 0; q < 4; q++) xn[q] = *reinterpret_cast<const uint4*>(xr + (size_t)st * kStepK + q * 8);
        sn = sr[(size_t)st * 4];
      }
#pragma unroll
      for (int k = 0; k < NSTEP; k++) {
        if constexpr (ROLL) {
          const int ci = k >> 1;
          if ((k & 1) == 0 && ci + RD < NLC && p0 == gw) {
            __builtin_amdgcn_s_waitcnt(gemv_wait_vm(2 * (RD - 1)));  // column ci landed
            __builtin_amdgcn_sched_barrier(0);
            load_cols(p0, ci + RD, ci + RD + 1);
          }
        }
        const int st = step_of(k);
        uint4 xq[4] = {xn[0], xn[1], xn[2], xn[3]};
        const uint32_t sbyte = sn;
        if (k + 1 < NSTEP) {
          const int stn = min(step_of(k + 1), S - 1);
#pragma unroll
          for (int q = 0; q < 4; q++) xn[q] = *reinterpret_cast<const uint4*>(xr + (size_t)stn * kStepK + q * 8);
          sn = sr[(size_t)stn * 4];
        }
        if (st < S) {  // wave-uniform; no global loads inside
          const uint4 a = wv[k & ~1], b = wv[k | 1];
          uint32_t wd[4];
          if (!WL) {
            wd[0] = wv[k].x; wd[1] = wv[k].y; wd[2] = wv[k].z; wd[3] = wv[k].w;
          } else if ((k & 1) == 0) {  // step 2c: the lane's own row, from A (rows 0-7) or B
            wd[0] = r < 8 ? a.x : b.x; wd[1] = r < 8 ? a.y : b.y;
            wd[2] = r < 8 ? a.z : b.z; wd[3] = r < 8 ? a.w : b.w;
          } else {  // step 2c+1: held 8 lanes away, in the other load
            const uint32_t o[4] = {r < 8 ? b.x : a.x, r < 8 ? b.y : a.y, r < 8 ? b.z : a.z, r < 8 ? b.w : a.w};
#pragma unroll
            for (int q = 0; q < 4; q++) wd[q] = (uint32_t)__builtin_amdgcn_mov_dpp((int)o[q], 0x128, 0xf, 0xf, false);
          }
          const float scale = e8m0_as_cvt_scale(sbyte);
#pragma unroll
          for (int q = 0; q < 4; q++)
            acc[q] = mfma_f16_16x16x32(__builtin_bit_cast(v8h, xq[q]), fp4x8_to_f16x8(wd[q], scale), acc[q]);
        }
      }
    }
  }

  // acc element v: token (lane/16)*4 + v, column (weight row) lane % 16.
#pragma unroll
  for (int v = 0; v < 4; v++) red[(wave * 16 + lg * 4 + v) * 17 + r] = (acc[0][v] + acc[1][v]) + (acc[2][v] + acc[3][v]);
  __syncthreads();
  // whole waves: thread (group g2, token tt, column cc), two groups per pass
#pragma unroll
  for (int g2 = tid >> 8; g2 < NG; g2 += 2) {
    const int tt = (tid >> 4) & 15, cc = tid & 15;
    const int grp = g0 + g2;
    float tot = 0.0f;
#pragma unroll
    for (int w = 0; w < WPG; w++) tot += red[((g2 * WPG + w) * 16 + tt) * 17 + cc];
    if (DUAL) {
      // column cc + 8 is the same channel's up sum: lanes cc and cc ^ 8 of
      // each 16-lane row swap by DPP row_ror:8 (no LDS round trip)
      const float uv = __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, tot), 0x128, 0xf, 0xf, false));
      if (cc < 8 && tt < T) g.out[(size_t)tt * g.n + grp * 8 + cc] = f32_to_f16_bits(silu(tot) * uv);
    } else if (tt < T) {
      g.out[(size_t)tt * g.n + grp * 16 + cc] = f32_to_f16_bits(tot);
    }
  }
}

// One launch per MLP half: whole lines for the dual gate/up pass, half lines
// for down (measured at C1, T = 1 / T = 8, down: 4.42 / 5.22 us with whole
// lines against 4.32 / 5.08 us; gate/up gains 0.15-0.2 us from them).
// SC16: the scale planes are 16-byte aligned (16-byte staging pieces).
template <bool DUAL, int NSTEP, int WPG, bool SC16>
__global__ __launch_bounds__(64 * kW) void k_gemv_mxfp4(GemvArgs g) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  gemv_body<DUAL, NSTEP, WPG, DUAL, SC16, false>(g, blockIdx.x * (kW / WPG), lds);
}

// Grouped (MoE) form: blockIdx.y is the group (expert).  Group e owns token
// rows [off[e], off[e+1]) of x and out, and its weights sit e * stride bytes
// after group 0's.  Groups with no tokens exit at once.  Whole-line loads
// for both passes: these launches stream far more weights than one MLP and
// are bandwidth-bound, where fewer, whole-line requests pay (measured at 64
// experts x 4 tokens of the C1 shape: 360 -> 297 us per MoE MLP, down alone
// 113 -> 105 us).
template <bool DUAL, int NSTEP, int WPG, bool SC16>
__global__ __launch_bounds__(64 * kW) void k_gemv_mxfp4_grouped(GemvArgs g, GroupTable gt) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  const int e = blockIdx.y;
  const int t0 = gt.off[e], T = gt.off[e + 1] - t0;
  if (T <= 0) return;  // workgroup-uniform
  g.t = T;
  g.x += (size_t)t0 * g.k;
  g.out += (size_t)t0 * g.n;
  g.b0 += e * gt.b_stride;
  g.s0 += e * gt.s_stride;
  if (DUAL) {
    g.b1 += e * gt.b_stride;
    g.s1 += e * gt.s_stride;
  }
  gemv_body<DUAL, NSTEP, WPG, true, SC16, true>(g, blockIdx.x * (kW / WPG), lds);
}

template <bool DUAL, int NSTEP, int WPG, bool SC16>
static hipError_t launch_ns(const GemvArgs& g, hipStream_t st) {
  constexpr int NG = kW / WPG;
  static bool attr_set = false;  // allow up to 160 KB of dynamic LDS (once per instance)
  if (!attr_set) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(k_gemv_mxfp4<DUAL, NSTEP, WPG, SC16>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    if (e != hipSuccess) return e;
    attr_set = true;
  }
  const int row_groups = DUAL ? g.n / 8 : g.n / 16;
  hipLaunchKernelGGL((k_gemv_mxfp4<DUAL, NSTEP, WPG, SC16>), dim3(row_groups / NG), dim3(64 * kW),
                     gemv_lds_bytes(g.t, g.k, NG), st, g);
  return hipGetLastError();
}

template <bool DUAL, int WPG, bool SC16>
static hipError_t launch_w(const GemvArgs& g, hipStream_t st) {
  const int per_wave = (g.k / kStepK + WPG - 1) / WPG;
  if (per_wave <= 2) return launch_ns<DUAL, 2, WPG, SC16>(g, st);
  if (per_wave <= 4) return launch_ns<DUAL, 4, WPG, SC16>(g, st);
  return launch_ns<DUAL, 8, WPG, SC16>(g, st);
}

template <bool SC16>
static hipError_t launch_single(int dual, bool pair, const GemvArgs& g, hipStream_t st) {
  if (dual) return launch_w<true, kW, SC16>(g, st);
  return pair ? launch_w<false, kW / 2, SC16>(g, st) : launch_w<false, kW, SC16>(g, st);
}

// Preconditions (caller): 1 <= t <= 16, n % 16 == 0, k % 128 == 0 and
// gemv_lds_bytes(t, k) <= 160 KB (checked here).  The batch size is the
// number of K steps each wave owns (capped at 8), so no wave issues
// redundant loads when K is short.  The single (down) GEMV takes two row
// groups per workgroup from 4 tokens on, where x (T x K) staging is large:
// x is then staged once for 32 rows (measured at C1 with HBM-cold weights:
// 5.20 -> 5.11 us at T = 8, but 4.3 -> 4.5 us at T = 1).  The dual gate/up
// GEMV keeps one group: its 256 workgroups would halve to 128, idling CUs
// (measured at C1 T = 8: gate/up 7.0 -> 9.2 us with two groups).
// Scale planes that are 16-byte aligned (the library's own allocations are)
// are staged in 16-byte pieces; the C ABI also accepts 4-byte aligned ones,
// which are staged in dwords.
hipError_t launch_gemv_mxfp4(int dual, const GemvArgs& g, hipStream_t st) {
  if (gemv_lds_bytes(g.t, g.k) > 160 * 1024 || g.k > 16384 || g.k % kStepK) return hipErrorInvalidValue;
  const bool pair = !dual && g.t >= 4 && (g.n / 16) % 2 == 0 && g.k <= 8192 &&
                    gemv_lds_bytes(g.t, g.k, 2) <= 160 * 1024;
  const uintptr_t sp = reinterpret_cast<uintptr_t>(g.s0) | (dual ? reinterpret_cast<uintptr_t>(g.s1) : 0);
  return sp % 16 == 0 ? launch_single<true>(dual, pair, g, st) : launch_single<false>(dual, pair, g, st);
}

size_t gemv_lds_need(int t, int k) { return gemv_lds_bytes(t, k); }

template <bool DUAL, int NSTEP, int WPG, bool SC16>
static hipError_t launch_grouped_ns(const GemvArgs& g, const GroupTable& gt, int groups, hipStream_t st) {
  constexpr int NG = kW / WPG;
  static bool attr_set = false;  // allow up to 160 KB of dynamic LDS (once per instance)
  if (!attr_set) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(k_gemv_mxfp4_grouped<DUAL, NSTEP, WPG, SC16>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    if (e != hipSuccess) return e;
    attr_set = true;
  }
  const int row_groups = DUAL ? g.n / 8 : g.n / 16;
  hipLaunchKernelGGL((k_gemv_mxfp4_grouped<DUAL, NSTEP, WPG, SC16>), dim3(row_groups / NG, groups), dim3(64 * kW),
                     gemv_lds_bytes(g.t, g.k, NG), st, g, gt);
  return hipGetLastError();
}

template <bool DUAL, int WPG, bool SC16>
static hipError_t launch_grouped_w(const GemvArgs& g, const GroupTable& gt, int groups, hipStream_t st) {
  const int per_wave = (g.k / kStepK + WPG - 1) / WPG;
  if (per_wave <= 2) return launch_grouped_ns<DUAL, 2, WPG, SC16>(g, gt, groups, st);
  if (per_wave <= 4) return launch_grouped_ns<DUAL, 4, WPG, SC16>(g, gt, groups, st);
  return launch_grouped_ns<DUAL, 8, WPG, SC16>(g, gt, groups, st);
}

template <bool SC16>
static hipError_t launch_grouped(int dual, int ng, const GemvArgs& g, const GroupTable& gt, int groups,
                                 hipStream_t st) {
  switch (ng) {
    case 8: return dual ? launch_grouped_w<true, kW / 8, SC16>(g, gt, groups, st)
                        : launch_grouped_w<false, kW / 8, SC16>(g, gt, groups, st);
    case 4: return dual ? launch_grouped_w<true, kW / 4, SC16>(g, gt, groups, st)
                        : launch_grouped_w<false, kW / 4, SC16>(g, gt, groups, st);
    case 2: return dual ? launch_grouped_w<true, kW / 2, SC16>(g, gt, groups, st)
                        : launch_grouped_w<false, kW / 2, SC16>(g, gt, groups, st);
    default: return dual ? launch_grouped_w<true, kW, SC16>(g, gt, groups, st)
                         : launch_grouped_w<false, kW, SC16>(g, gt, groups, st);
  }
}

// g.t = the largest group's token count (sizes the LDS); the same
// preconditions as launch_gemv_mxfp4 for it.  With many workgroups each one
// takes several row groups, so x (T x K, staged per workgroup) is staged
// once for more weight rows: two row groups (four waves each) from 1024
// one-group workgroups on, four (two waves each) from 4096 on, eight (one
// wave each) from 8192 on while two workgroups still fit a CU (measured at
// 64 experts x 4 tokens of the C1 shape: gate/up 254 -> 241 us with four,
// down 128 -> 115 us with four and 109 us with eight).
hipError_t launch_gemv_mxfp4_grouped(int dual, const GemvArgs& g, const GroupTable& gt, int groups, hipStream_t st) {
  const int row_groups = dual ? g.n / 8 : g.n / 16;
  const size_t wg1 = (size_t)groups * row_groups;  // workgroups at one row group each
  const bool pair = wg1 >= 1024 && row_groups % 2 == 0 && g.k <= 8192 && gemv_lds_bytes(g.t, g.k, 2) <= 160 * 1024;
  const bool quad = wg1 >= 4096 && row_groups % 4 == 0 && 16 * 4 * (g.k / 128) <= scale_regs(4) * 64 * kW &&
                    gemv_lds_bytes(g.t, g.k, 4) <= 160 * 1024;
  const bool octo = wg1 >= 8192 && row_groups % 8 == 0 && 16 * 8 * (g.k / 128) <= scale_regs(8) * 64 * kW &&
                    gemv_lds_bytes(g.t, g.k, 8) <= 80 * 1024;  // still two workgroups per CU
  if (groups < 1 || groups > kMaxGroups || g.t < 1 || g.t > 16 || gemv_lds_bytes(g.t, g.k) > 160 * 1024 ||
      g.k > 16384 || g.k % kStepK)
    return hipErrorInvalidValue;
  const int ng = octo ? 8 : quad ? 4 : pair ? 2 : 1;
  // 16-byte scale pieces when every group's planes are 16-byte aligned
  // (64 experts x 4 tokens of the C1 shape: 277.7 -> 269.8 us per MoE MLP)
  const uintptr_t sp = reinterpret_cast<uintptr_t>(g.s0) | (dual ? reinterpret_cast<uintptr_t>(g.s1) : 0) |
                       gt.s_stride;
  return sp % 16 == 0 ? launch_grouped<true>(dual, ng, g, gt, groups, st)
                      : launch_grouped<false>(dual, ng, g, gt, groups, st);
}

}  // namespace mx
