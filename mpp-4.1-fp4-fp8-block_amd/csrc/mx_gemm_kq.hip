// mx_gemm_kq.hip - MXFP4 gate/up + SwiGLU GEMM for launches of about one
// tile per CU with a long K: BASELINE configs[2] (the expert-shaped batch,
// T=512, H=7168, I=2048), f32 accumulation (mxfp4_fused_h_f_n64 /
// mxfp4_native_sp_h_f_n64, MXFP4Kernels.metal:42-173, 264-286), SwiGLU of the
// fused rows (MPPMLPKernels.metal:186-220).  Two forms:
//   f16 x     weights decoded in registers (v_cvt_scalef32_pk_f16_fp4) for
//             v_mfma_f32_32x32x16_f16; mid f16.
//   F8X2 x    the scaled route: x as two E4M3 terms with an E8M0 pair per
//             64 K (layout in mx_internal.h), FP4 codes and their E8M0 bytes
//             straight into v_mfma_scale_f32_32x32x64_f8f6f4, one MFMA per
//             term; mid written as F8X2 for the down GEMM.
//
// The 128 x 128 tiles of mx_gemm_q.hip give such a shape 128 tiles, so they
// split K four ways: 512 workgroups, two per CU, f32 partials of both
// matrices through HBM and a reduce launch that runs the SwiGLU.  Here the
// tile is 64 tokens x 64 channels (64 gate + 64 up weight rows), giving
// 8 x 32 = 256 workgroups, one per CU, and K is split inside the
// workgroup:
//
//   rounds   K advances in rounds of 256: A 64 rows x 4 stages of 64 K (whole
//            128-byte lines, 32 KB), B 128 rows x 128 B (16 KB), and the
//            rows' E8M0 bytes of the round (1 KB).  A 3-slot LDS ring keeps
//            two rounds in flight while one is computed.
//   roles    waves 4-7 issue the ring's DMAs and wait only on them; waves
//            0-3 compute and issue no DMA, so their LDS reads never wait on a
//            DMA (a wave that did both would have the compiler drain its DMAs
//            before each read of a runtime-indexed slot).  One barrier per
//            round passes a filled slot in and an emptied one back.
//   K split  compute wave w takes stage w of every round for the whole tile
//            (2 x 4 blocks of v_mfma_f32_32x32x16_f16, 128 accumulators), so
//            no fragment is read by two waves.  At the end the four partial
//            tiles meet in LDS, are added in wave order (deterministic), and
//            the SwiGLU'd f16 tile leaves as one 16-byte store per thread.
//   K order  within a stage, lane half h of both operands holds k [32h, 32h
//            + 32), one FP4 block: one E8M0 byte per lane and weight row.
//   byte 255 the reference reads E8M0 255 as +inf, the hardware as NaN.  The
//            loop decodes with the hardware's reading only (an exact second
//            form inside it spills the 128 accumulators); the epilogue
//            recomputes the NaN sums, in f32 with the reference's
//            dequantization, which is never finite for such a sum either.
#include "mx_device.h"
#include "mx_internal.h"

namespace mx {
namespace kqgemm {

constexpr int kThreads = 512;
constexpr int kSlots = 3;
constexpr int kSlotA = 4 * 64 * 128;          // 4 stages x 64 rows x 128 B
constexpr int kSlotB = 128 * 128;             // 128 weight rows x 128 B
constexpr int kSlotS = 128 * 8;               // 128 rows x 8 E8M0 bytes
constexpr int kSlotE = 4 * 64 * 4;            // F8X2: 4 stages x 64 rows of E8M0 pairs
constexpr int kSlot = kSlotA + kSlotB + kSlotS + kSlotE;
// DMA instructions per producer wave per round: 12 of A and B, the weight
// scales, and for F8X2 the E8M0 pairs of one stage
template <int AK> constexpr int ops() { return (kSlotA + kSlotB) / 1024 / 4 + 1 + (AK == AK_F8X2 ? 1 : 0); }
constexpr int kPull = 4;  // rounds between the L2 pull of a round and its use

__device__ __forceinline__ void dma16(const void* src, void* lds) {
  __builtin_amdgcn_global_load_lds(src, lds, 16, 0, 0);
}
__device__ __forceinline__ void dma4(const void* src, void* lds) {
  __builtin_amdgcn_global_load_lds(src, lds, 4, 0, 0);
}
// s_waitcnt immediate (gfx9 encoding): vmcnt(n) only.
constexpr int wait_vm(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }
// 16-byte chunk c of 128-byte LDS row r sits at c ^ swz(r): 32 rows x one
// chunk fall on distinct banks.
__device__ __forceinline__ int swz(int row) { return (row >> 1) & 7; }

// Grid: tiles_m * (n / 64); block b -> M tile b / tiles_n, channel tile
// b % tiles_n (the M tiles of one channel tile share an XCD's L2 when
// tiles_n % 8 == 0).
template <int AK, int EPI>
__global__ __launch_bounds__(kThreads, 1) void k_kq_gate_up(QGemmArgs g) {
  constexpr bool F8 = AK == AK_F8X2;
  constexpr int kOps = ops<AK>();
  constexpr int kAB = (kSlotA + kSlotB) / 1024 / 4;  // A and B DMAs per producer wave
  __shared__ __attribute__((aligned(16))) uint8_t ring[kSlots * kSlot];
  __shared__ __attribute__((aligned(16))) uint8_t pf_lds[4 * 1024];  // L2 pull landing, never read
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int M = g.m, K = g.k;
  const int tiles_n = g.n / 64;
  const int m0 = (int)(blockIdx.x / tiles_n) * 64;
  const int n0 = (int)(blockIdx.x % tiles_n) * 64;
  const int R = K / 256;  // rounds

  if (wave >= 4) {
    // ---- producers: round r into slot r % 3
    const int pw = wave - 4;
    const uint8_t* x = reinterpret_cast<const uint8_t*>(g.a);
    const uint8_t* src[kAB + 1];
    int dst[kAB + 1];
#pragma unroll
    for (int q = 0; q < kAB; q++) {
      const int op = pw * kAB + q;  // 0 .. 47
      const int r = (op & 7) * 8 + (lane >> 3);
      if (op < 32) {  // A: stage op / 8, rows 8 (op % 8) ..
        const int st = op >> 3;
        const int lc = (lane & 7) ^ swz(r);
        src[q] = x + (size_t)min(m0 + r, M - 1) * ((size_t)K * 2) + st * 128 + lc * 16;
        dst[q] = st * 8192 + (op & 7) * 1024;
      } else {  // B: weight rows 8 (op - 32) ..
        const int br = (op - 32) * 8 + (lane >> 3);
        const int lc = (lane & 7) ^ swz(br);
        const uint8_t* base = reinterpret_cast<const uint8_t*>(br < 64 ? g.b0 : g.b1);
        src[q] = base + (size_t)(n0 + (br & 63)) * (K / 2) + lc * 16;
        dst[q] = kSlotA + (op - 32) * 1024;
      }
    }
    {  // E8M0: dword d (0/1) of row s, 64 dwords per wave
      const int i = pw * 64 + lane, row = i >> 1;
      const uint8_t* base = reinterpret_cast<const uint8_t*>(row < 64 ? g.s0 : g.s1);
      src[kAB] = base + (size_t)(n0 + (row & 63)) * (K / 32) + (i & 1) * 4;
      dst[kAB] = kSlotA + kSlotB + pw * 256;
    }
    // F8X2: the E8M0 pairs of stage pw of the round, one dword per row
    // ([K/64][M] plane, rows clamped)
    const uint32_t* esrc = F8 ? g.a_e8 + (size_t)pw * M + min(m0 + lane, M - 1) : nullptr;
    // A rows advance 512 B per round, B rows 128 B, scale rows 8 B, the
    // pair plane 4 stages
    auto issue = [&](int rd, int sl) {
      uint8_t* s = ring + sl * kSlot;
#pragma unroll
      for (int q = 0; q < kAB; q++) {
        const int op = pw * kAB + q;
        dma16(src[q] + (size_t)rd * (op < 32 ? 512 : 128), s + dst[q]);
      }
      dma4(src[kAB] + (size_t)rd * 8, s + dst[kAB]);
      if constexpr (F8) dma4(esrc + (size_t)rd * 4 * M, s + kSlotA + kSlotB + kSlotS + pw * 256);
    };
    // L2 pull.  The ring's DMAs wait on the last-level cache (~2 us, with
    // two rounds in flight in 147 KB of LDS), so each round's lines are
    // first touched kPull rounds ahead, one line per lane, the touches split
    // over the workgroups of this XCD that share them (tile t runs on XCD
    // t % 8): producers 0 / 2 a quarter of the M tile's A rows per channel
    // tile t / 8 % 4, producers 1 / 3 an eighth of the channel tile's weight
    // rows per M tile.  Issued after the round's DMAs, a pull is never
    // waited for by an older DMA's wait; the waits count the two pulls
    // issued since.
    const uint8_t* pf_src;
    size_t pf_step;
    if ((pw & 1) == 0) {
      const int q = (int)(blockIdx.x % tiles_n) / 8 % 4;
      const int row = min(m0 + 16 * q + 8 * (pw >> 1) + (lane >> 3), M - 1);
      pf_src = x + (size_t)row * ((size_t)K * 2) + (lane & 3) * 128;
      pf_step = 512;
    } else {
      const int e = (int)(blockIdx.x / tiles_n) % 8, br = 16 * e + 8 * (pw >> 1) + (lane & 7);
      pf_src = reinterpret_cast<const uint8_t*>(br < 64 ? g.b0 : g.b1) + (size_t)(n0 + (br & 63)) * (K / 2);
      pf_step = 128;
    }
    auto pull = [&](int rd) { dma16(pf_src + (size_t)min(rd + kPull, R - 1) * pf_step, pf_lds + pw * 1024); };
    issue(0, 0);
    pull(0);
    issue(min(1, R - 1), 1);
    pull(1);
    for (int rd = 0; rd < R; rd++) {
      __builtin_amdgcn_s_waitcnt(wait_vm(kOps + 2));  // round rd has landed
      __builtin_amdgcn_s_barrier();                    // ... and slot (rd + 2) % 3 is free
      __builtin_amdgcn_sched_barrier(0);
      // past the end: the last round again, into a slot nobody reads
      issue(min(rd + 2, R - 1), (rd + 2) % kSlots);
      pull(rd + 2);
    }
    __builtin_amdgcn_s_waitcnt(wait_vm(0));
    __builtin_amdgcn_s_barrier();  // the ring is free for the epilogue
  } else {
    // ---- compute: stage w of every round, the whole 64 x 128 tile
    const int w = wave, r32 = lane & 31, h = lane >> 5;
    v16f acc[2][4];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
      for (int j = 0; j < 4; j++)
#pragma unroll
        for (int v = 0; v < 16; v++) acc[i][j][v] = 0.0f;
    for (int rd = 0; rd < R; rd++) {
      __builtin_amdgcn_sched_barrier(0);
      __builtin_amdgcn_s_barrier();  // round rd is in slot rd % 3
      __builtin_amdgcn_sched_barrier(0);
      const uint8_t* s = ring + (rd % kSlots) * kSlot;
      const uint8_t* as = s + w * 8192;
      v4i af[2][4], bf[4];
      uint32_t sb[4], ae[2];
#pragma unroll
      for (int i = 0; i < 2; i++) {
        const int row = 32 * i + r32;
        // f16: k-step t of lane half h is chunk 4h + t; F8X2: term u = t / 2
        // (chunks 0-3 / 4-7), half h reads chunks 2h, 2h + 1 of its term
#pragma unroll
        for (int t = 0; t < 4; t++) {
          const int ch = F8 ? 4 * (t >> 1) + 2 * h + (t & 1) : 4 * h + t;
          af[i][t] = *reinterpret_cast<const v4i*>(as + row * 128 + ((ch ^ swz(row)) << 4));
        }
        if constexpr (F8) ae[i] = *reinterpret_cast<const uint32_t*>(s + kSlotA + kSlotB + kSlotS + (w * 64 + row) * 4);
      }
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const int row = 32 * j + r32;  // 0..63 gate, 64..127 up
        bf[j] = *reinterpret_cast<const v4i*>(s + kSlotA + row * 128 + (((2 * w + h) ^ swz(row)) << 4));
        sb[j] = s[kSlotA + kSlotB + row * 8 + 2 * w + h];
      }
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (F8) {
        // two scaled MFMAs per block: E4M3 term 1 / 2 (its byte of the pair
        // by opsel) x FP4 (the lane's E8M0 byte)
#pragma unroll
        for (int i = 0; i < 2; i++) {
          v8i a1, a2;
#pragma unroll
          for (int t = 0; t < 4; t++) {
            a1[t] = af[i][0][t]; a1[4 + t] = af[i][1][t];
            a2[t] = af[i][2][t]; a2[4 + t] = af[i][3][t];
          }
#pragma unroll
          for (int j = 0; j < 4; j++) {
            v8i b;
#pragma unroll
            for (int t = 0; t < 4; t++) { b[t] = bf[j][t]; b[4 + t] = 0; }
            acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a1, b, acc[i][j], 0, 4, 0, (int)ae[i], 0, (int)sb[j]);
            acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a2, b, acc[i][j], 0, 4, 1, (int)ae[i], 0, (int)sb[j]);
          }
        }
      } else {
        // one weight block decoded at a time (all sixteen at once spill)
#pragma unroll
        for (int t = 0; t < 4; t++) {
#pragma unroll
          for (int j = 0; j < 4; j++) {
            const v8h b_ = fp4x8_to_f16x8((uint32_t)bf[j][t], e8m0_as_cvt_scale(sb[j]));
#pragma unroll
            for (int i = 0; i < 2; i++)
              acc[i][j] = mfma_f16_32x32x16(__builtin_bit_cast(v8h, af[i][t]), b_, acc[i][j]);
            __builtin_amdgcn_sched_barrier(0);
          }
        }
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_barrier();  // producers have drained
    __builtin_amdgcn_sched_barrier(0);
    // partial tiles into LDS: [w][i][j][v / 4][lane] x 4 floats (128 KB)
    v4f* red = reinterpret_cast<v4f*>(ring);
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
      for (int j = 0; j < 4; j++)
#pragma unroll
        for (int vq = 0; vq < 4; vq++)
          red[(((w * 2 + i) * 4 + j) * 4 + vq) * 64 + lane] =
              (v4f){acc[i][j][4 * vq], acc[i][j][4 * vq + 1], acc[i][j][4 * vq + 2], acc[i][j][4 * vq + 3]};
  }
  __syncthreads();
  // Sum of the four K quarters in wave order, SwiGLU, mid tile [64][64] in
  // LDS after the partials (f16, or f32 for the F8X2 split); thread -> (i,
  // gate block jg, v / 4, lane), two groups of four rows each.
  const uint16_t* x16 = F8 ? g.a_f16 : reinterpret_cast<const uint16_t*>(g.a);  // f16 x for the recompute
  {
    const v4f* red = reinterpret_cast<const v4f*>(ring);
    uint16_t* tile = reinterpret_cast<uint16_t*>(ring + 4 * 32768);
    float* tile32 = reinterpret_cast<float*>(ring + 4 * 32768);
#pragma unroll
    for (int half = 0; half < 2; half++) {
      const int grp = tid + half * kThreads;  // 0 .. 1023
      const int ln = grp & 63, vq = (grp >> 6) & 3, jg = (grp >> 8) & 1, i = grp >> 9;
      v4f gs = red[(((0 * 2 + i) * 4 + jg) * 4 + vq) * 64 + ln];
      v4f us = red[(((0 * 2 + i) * 4 + jg + 2) * 4 + vq) * 64 + ln];
#pragma unroll
      for (int q = 1; q < 4; q++) {
        gs += red[(((q * 2 + i) * 4 + jg) * 4 + vq) * 64 + ln];
        us += red[(((q * 2 + i) * 4 + jg + 2) * 4 + vq) * 64 + ln];
      }
      // E8M0 byte 255 reads as NaN in the decode (and in the scaled MFMA),
      // where the reference has +inf; the sums it reaches (and only those: a
      // sum over such a block is never finite in the reference) are
      // recomputed with the reference's dequantization in f32, K in order,
      // from the f16 x.  So are the sums of an F8X2 group holding a
      // non-finite x (scale bytes 255).
      bool bad = false;
#pragma unroll
      for (int e = 0; e < 4; e++) bad |= gs[e] != gs[e] || us[e] != us[e];
      if (__builtin_expect(__ballot(bad) != 0, 0)) {
#pragma unroll
        for (int e = 0; e < 4; e++) {
          const int row = m0 + 32 * i + acc32_row(ln, 4 * vq + e), ch = n0 + 32 * jg + (ln & 31);
          if ((gs[e] != gs[e] || us[e] != us[e]) && row < M && x16) {
            const uint16_t* xr = x16 + (size_t)row * K;
            gs[e] = ref_dot_f16_mxfp4(xr, reinterpret_cast<const uint8_t*>(g.b0) + (size_t)ch * (K / 2),
                                      reinterpret_cast<const uint8_t*>(g.s0) + (size_t)ch * (K / 32), K);
            us[e] = ref_dot_f16_mxfp4(xr, reinterpret_cast<const uint8_t*>(g.b1) + (size_t)ch * (K / 2),
                                      reinterpret_cast<const uint8_t*>(g.s1) + (size_t)ch * (K / 32), K);
          }
        }
      }
#pragma unroll
      for (int e = 0; e < 4; e++) {
        float mv;
        if (EPI == EPI_SWIGLU_HALF) {  // swiglu_half: silu(clamp(g/16, +-20)) * u/16
          const float gg = fminf(fmaxf(gs[e] * 0.0625f, -20.0f), 20.0f);
          mv = (gg / (1.0f + expf(-gg))) * (us[e] * 0.0625f);
        } else {
          mv = silu(gs[e]) * us[e];
        }
        const int row = 32 * i + acc32_row(ln, 4 * vq + e);
        if constexpr (F8) tile32[row * 64 + 32 * jg + (ln & 31)] = mv;
        else tile[row * 64 + 32 * jg + (ln & 31)] = f32_to_f16_bits(mv);
      }
    }
  }
  __syncthreads();
  // row tid / 8, channels 8 (tid % 8) .. + 8: one 16-byte f16 store, or the
  // row's 64 channels (one F8X2 group of the down GEMM's K) split by its
  // 8 lanes
  const int r = tid >> 3, row = m0 + r;
  if (row < M) {  // uniform over a row's 8 lanes
    if constexpr (F8) {
      float v[8];
#pragma unroll
      for (int e = 0; e < 8; e++) v[e] = reinterpret_cast<const float*>(ring + 4 * 32768)[r * 64 + (tid & 7) * 8 + e];
      f8x2_split_store<8>(v, tid & 7, reinterpret_cast<uint8_t*>(g.c) + (size_t)row * 2 * g.n + (size_t)(n0 / 64) * 128,
                          g.c_e8 + (size_t)(n0 / 64) * M + row);
    } else {
      const uint4 v = *reinterpret_cast<const uint4*>(ring + 4 * 32768 + (r * 64 + (tid & 7) * 8) * 2);
      *reinterpret_cast<uint4*>(reinterpret_cast<uint16_t*>(g.c) + (size_t)row * g.n + n0 + (tid & 7) * 8) = v;
    }
  }
}

}  // namespace kqgemm

using namespace kqgemm;

bool kq_gemm_ok(int ak, int epi, int m, int n, int k) {
  if (ak == AK_F16 ? epi != EPI_SWIGLU_F16 && epi != EPI_SWIGLU_HALF : ak != AK_F8X2 || epi != EPI_SWIGLU_F8X2)
    return false;
  if (m < 1 || n % 64 || k % 256 || k < 1024) return false;
  const long tiles = (long)((m + 63) / 64) * (n / 64);
  return tiles >= 192 && tiles <= 256;
}

hipError_t launch_kq_gemm(int ak, int epi, const QGemmArgs& g, hipStream_t st) {
  const dim3 grid((unsigned)(((g.m + 63) / 64) * (g.n / 64)));
  if (ak == AK_F8X2)
    hipLaunchKernelGGL((k_kq_gate_up<AK_F8X2, EPI_SWIGLU_F8X2>), grid, dim3(kThreads), 0, st, g);
  else if (epi == EPI_SWIGLU_HALF)
    hipLaunchKernelGGL((k_kq_gate_up<AK_F16, EPI_SWIGLU_HALF>), grid, dim3(kThreads), 0, st, g);
  else
    hipLaunchKernelGGL((k_kq_gate_up<AK_F16, EPI_SWIGLU_F16>), grid, dim3(kThreads), 0, st, g);
  return hipGetLastError();
}

}  // namespace mx
