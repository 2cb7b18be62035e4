// mx_gemm_q.hip - GEMM family for small and medium token counts (BASELINE
// configs 0, 2, 3 and the GEMM entry points): half / f32 / int8 activations
// times quantized weights.
//
//   C[m][n] = sum_k A[m][k] * W[n][k]   (epilogue: store, SwiGLU, scales)
//
// Counterparts in the reference (root = Anemll/MPP-4.1-FP4-FP8-block):
//   MXFP4 weights   mxfp4_native_sp_h_f_n64 / mxfp4_fused_h_f_n64
//                   (MXFP4Kernels.metal:42-173, 264-286)
//   f16 weights     mpp_mlp_h_h_f_n128 / mpp_mlp_f_h_f_n128 (MPPMLPKernels.metal:14-48, 164-173)
//   FP8/INT8/INT4   mpp_mlp_h_fp8e4m3_f / _h_fp8e5m2_f / _h_i8_f / _h_i4_f
//                   (MPPMLPKernels.metal:50-125), plus BASELINE's scales
//   W8A8            mpp_mlp_i8_i8_i32_n128 (MPPMLPKernels.metal:61-70), i32
//                   accumulation, per-token x scale and per-row weight scale
//   SwiGLU          mpp_mlp_swiglu_float / _half (MPPMLPKernels.metal:186-220),
//                   fused: a workgroup computes gate and up of the same channels
//
// Design (gfx950):
//   tile      128 rows of A x 128 weight rows (SwiGLU: 64 gate + the same 64
//             up channels), 4 wave64s in a 2 x 2 grid, each 64 x 64 = 2 x 2
//             blocks of v_mfma_f32_32x32x16_f16 (W8A8: v_mfma_i32_32x32x32_i8).
//             At most 80 KB of LDS and 64 accumulators, so two workgroups
//             share a CU and hide each other's waits.
//   K stage   64 (W8A8: 128).  A and B rows of a stage are moved global -> LDS
//             by global_load_lds_dwordx4, whole rows per instruction (1 KB =
//             8 rows of 128 B for f16), into a 2-slot ring of separate
//             __shared__ arrays.  The 16-byte chunks of a row are XOR-swizzled
//             (chunk c of row r at c ^ swz(r)) so the fragment reads
//             (32 rows x one chunk) hit distinct banks; each DMA lane fetches
//             the chunk that belongs in its LDS position.
//   K order   within a stage, lane half h of a fragment owns the contiguous
//             K range [32h, 32h+32) (W8A8 [64h, 64h+64)); both operands use
//             the same order, so the dot products are unchanged and every
//             lane reads whole 16-byte chunks.  A 4-bit weight lane therefore
//             holds exactly one 32-element block: one E8M0 / f16 scale.
//   decode    weights are widened in registers after the LDS read: FP4 with
//             v_cvt_scalef32_pk_f16_fp4 (E8M0 applied), FP8 with
//             v_cvt_scalef32_pk_f16_{fp8,bf8}, INT8 / INT4 with the 0x6400
//             exponent trick; f32 activations as two f16 terms, hi = f16(x)
//             and lo = f16(x - hi), two MFMAs (f32 x half kept to ~2^-22).
//   split K   shapes with few tiles split K over gridDim.y; the partial tiles
//             (f32, or i32 for W8A8) are summed in split order by a second
//             kernel that also runs the epilogue, so results are deterministic.
#include <type_traits>

#include "mx_device.h"
#include "mx_internal.h"

namespace mx {
namespace qgemm {

constexpr int kTM = 128;  // tile rows (A)

template <int AK> struct AInfo;
template <> struct AInfo<AK_F16> { static constexpr int KS = 64, RB = 128; };
template <> struct AInfo<AK_F32> { static constexpr int KS = 64, RB = 256; };
template <> struct AInfo<AK_I8> { static constexpr int KS = 128, RB = 128; };
template <> struct AInfo<AK_F8X2> { static constexpr int KS = 64, RB = 128; };  // 2 terms x 64 B

// bytes of one weight row per stage
template <int BK> constexpr int b_row_bytes(int ks) {
  return BK == BK_F16 ? ks * 2 : (BK == BK_MXFP4 || BK == BK_INT4G32) ? ks / 2 : ks;
}

// Chunk swizzle for rows of R bytes (C = R/16 chunks): rows that share a
// 256-byte bank line get different chunk rotations.
template <int R>
__device__ __forceinline__ int swz(int row) {
  constexpr int C = R / 16;
  constexpr int RPL = 16 / C > 0 ? 16 / C : 1;  // rows per 256 bytes
  return (row / RPL) % C;
}

// 16-byte global -> LDS DMA of one lane (the LDS base is wave-uniform).
// Kept behind a device function: referenced directly from this kernel
// template's body, the builtin stops the host pass from emitting the
// kernel's launch stub.
__device__ __forceinline__ void dma16(const void* src, void* lds) {
  __builtin_amdgcn_global_load_lds(src, lds, 16, 0, 0);
}
__device__ __forceinline__ void dma4(const void* src, void* lds) {
  __builtin_amdgcn_global_load_lds(src, lds, 4, 0, 0);
}

// s_waitcnt immediate (gfx9 encoding): vmcnt(n) only.
constexpr int wait_vm(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }
// s_waitcnt lgkmcnt(0) alone (vmcnt 63, expcnt 7).
constexpr int kWaitLgkm0 = 15 | (3 << 14) | (7 << 4);

// INT8 x8 -> f16 x8 (exact): byte b -> half(1024 + (b ^ 0x80)) - 1152.
__device__ __forceinline__ v8h i8x8_to_f16(uint32_t w0, uint32_t w1) {
  const uint32_t x[2] = {w0 ^ 0x80808080u, w1 ^ 0x80808080u};
  v8h out;
#pragma unroll
  for (int t = 0; t < 2; t++) {
    const uint32_t lo = __builtin_amdgcn_perm(0x64646464u, x[t], 0x04010400u);  // b0, b1
    const uint32_t hi = __builtin_amdgcn_perm(0x64646464u, x[t], 0x04030402u);  // b2, b3
    v2h l = __builtin_bit_cast(v2h, lo) - (v2h){(_Float16)1152.0f, (_Float16)1152.0f};
    v2h h = __builtin_bit_cast(v2h, hi) - (v2h){(_Float16)1152.0f, (_Float16)1152.0f};
    out[4 * t] = l[0]; out[4 * t + 1] = l[1]; out[4 * t + 2] = h[0]; out[4 * t + 3] = h[1];
  }
  return out;
}

// INT4 x8 (one dword, low nibble first) -> f16 x8: ((n ^ 8) - 8) * scale,
// rounded once to f16 (PackedNumericKernels.metal:30-33).  Per nibble pair
// (byte i): one v_perm puts byte i of w and of w >> 4 into the two halves,
// one v_bitop3 keeps their low nibbles, flips the sign bit (two's
// complement -> offset 8) and ORs in the 0x6400 exponent (1024 + u), then
// a packed subtract and the packed scale multiply: 17 VALU per dword.
__device__ __forceinline__ v8h i4x8_to_f16(uint32_t w, _Float16 sc) {
  const uint32_t y = w >> 4;
  const v2h off = {(_Float16)1032.0f, (_Float16)1032.0f};
  const v2h s2 = {sc, sc};
  v8h out;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const uint32_t t = __builtin_amdgcn_perm(y, w, 0x0c000c00u | (uint32_t)i | ((uint32_t)(4 + i) << 16));
    const uint32_t p = ((t ^ 0x00080008u) & 0x000f000fu) | 0x64006400u;
    const v2h q = (__builtin_bit_cast(v2h, p) - off) * s2;
    out[2 * i] = q[0];
    out[2 * i + 1] = q[1];
  }
  return out;
}

template <int BK>
__device__ __forceinline__ v8h fp8x8_to_f16(uint32_t w0, uint32_t w1) {
  const uint32_t w[2] = {w0, w1};
  v8h h;
#pragma unroll
  for (int t = 0; t < 2; t++) {
    v2h lo, hi;
    if (BK == BK_E4M3) {
      lo = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w[t], 1.0f, false);
      hi = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w[t], 1.0f, true);
    } else {
      lo = __builtin_amdgcn_cvt_scalef32_pk_f16_bf8(w[t], 1.0f, false);
      hi = __builtin_amdgcn_cvt_scalef32_pk_f16_bf8(w[t], 1.0f, true);
    }
    h[4 * t] = lo[0]; h[4 * t + 1] = lo[1]; h[4 * t + 2] = hi[0]; h[4 * t + 3] = hi[1];
  }
  return h;
}

// One output element's epilogue.  g (and u for SwiGLU) are the raw sums.
template <int EPI>
__device__ __forceinline__ void epi_store(void* c, size_t o, float x0, float u) {
  if (EPI == EPI_STORE_F32 || EPI == EPI_STORE_I32) {
    reinterpret_cast<float*>(c)[o] = x0;
  } else if (EPI == EPI_STORE_F16) {
    reinterpret_cast<uint16_t*>(c)[o] = f32_to_f16_bits(x0);
  } else if (EPI == EPI_SWIGLU_F32) {
    reinterpret_cast<float*>(c)[o] = (x0 / (1.0f + expf(-x0))) * u;
  } else if (EPI == EPI_SWIGLU_F16) {
    reinterpret_cast<uint16_t*>(c)[o] = f32_to_f16_bits(silu(x0) * u);
  } else {  // EPI_SWIGLU_HALF: silu(clamp(g/16, +-20)) * u/16 (MPPMLPKernels.metal:204-220)
    const float gg = fminf(fmaxf(x0 * 0.0625f, -20.0f), 20.0f);
    reinterpret_cast<uint16_t*>(c)[o] = f32_to_f16_bits((gg / (1.0f + expf(-gg))) * (u * 0.0625f));
  }
}

constexpr bool is_dual(int epi) {
  return epi == EPI_SWIGLU_F16 || epi == EPI_SWIGLU_HALF || epi == EPI_SWIGLU_F32 || epi == EPI_SWIGLU_F8X2;
}
constexpr bool row_scaled(int bk) { return bk == BK_E4M3 || bk == BK_E5M2 || bk == BK_INT8 || bk == BK_I8; }

// Scale a raw sum: weight row scale, and the per-token scale for W8A8.
template <int AK, int BK>
__device__ __forceinline__ float scaled(float acc, const QGemmArgs& g, const float* ws, int row, int col) {
  float v = acc;
  if (AK == AK_I8) v = v * g.a_scale[row];
  if (row_scaled(BK)) v = v * ws[col];
  return v;
}

// Reference-semantics raw dot products (row scales applied by the caller)
// for the exact recomputation of non-finite outputs of the F8X2 path: f16
// activation row x weight row `ch` (gate / up), and F8X2 activation row x
// weight row `col` (down).  MXFP4 weights are dequantized as the reference
// does (E8M0 byte 255 -> +inf), FP8 codes decoded as they are.
template <int BK>
__device__ inline float ref_dot_f16_w(const uint16_t* xr, const void* w, const void* s, int ch, int K) {
  const uint8_t* wb = reinterpret_cast<const uint8_t*>(w);
  if constexpr (BK == BK_MXFP4)
    return ref_dot_f16_mxfp4(xr, wb + (size_t)ch * (K / 2), reinterpret_cast<const uint8_t*>(s) + (size_t)ch * (K / 32), K);
  else
    return ref_dot_f16_fp8<BK == BK_E5M2>(xr, wb + (size_t)ch * K, K);
}
template <int BK>
__device__ inline float ref_dot_f8x2_w(const uint8_t* ad, const uint32_t* ae, int M, int row, const void* w,
                                       const void* s, int col, int K) {
  const uint8_t* wb = reinterpret_cast<const uint8_t*>(w);
  if constexpr (BK == BK_MXFP4)
    return ref_dot_f8x2_mxfp4(ad, ae, M, row, wb + (size_t)col * (K / 2),
                              reinterpret_cast<const uint8_t*>(s) + (size_t)col * (K / 32), K);
  else
    return ref_dot_f8x2_fp8<BK == BK_E5M2>(ad, ae, M, row, wb + (size_t)col * K, K);
}
// Row scale of weight row `col` (1 for formats without one).
template <int BK>
__device__ __forceinline__ float row_scale(const void* s, int col) {
  return row_scaled(BK) ? reinterpret_cast<const float*>(s)[col] : 1.0f;
}

constexpr int out_bytes(int epi) {
  return epi == EPI_STORE_F32 || epi == EPI_STORE_I32 || epi == EPI_SWIGLU_F32 ? 4 : 2;
}

// NWB: 32-column weight blocks per wave (2: 128 weight rows per tile, 1: 64).
// GROUPED (MoE): blockIdx.z is the group; group e owns rows [off[e],
// off[e+1]) of A and C and its weights / scales sit e * stride bytes after
// group 0's; g.tiles_m covers the largest group and tiles past a group's
// rows exit at once.  Grouped launches do not split K.
// BCH: K stages per B DMA chunk.  A 4-bit weight row holds 32 bytes per
// 64-K stage and an 8-bit one 64; B is staged BCH stages at a time (4 and 2)
// so that every DMA moves whole 128-byte lines (8 rows per instruction), the
// fastest LDS-DMA pattern.  BCH = 1 stages B per stage.
// NS: LDS slots of the per-stage ring.  2 (default): one stage in flight
// while one is computed, small enough for two workgroups per CU.  4: three
// stages in flight, for launches of at most one workgroup per CU, which
// otherwise sit in the DMA latency of every stage (8-bit / f16 weights,
// and MXFP4 with its scales in LDS; BCH = 1 only).
// SCL (4-bit weights): the E8M0 / f16 scales of the workgroup's weight rows
// over its whole K range are copied into LDS before the loop (at most
// kScLds bytes) and read from there per stage.  Loaded per stage from global
// memory instead, each stage waits for loads issued one stage earlier, whose
// latency the short stages do not cover.
// SCW (4-bit weights, f16 activations, chunked B, scales not in LDS): a
// lane loads its row's scales for a whole B chunk (BCH stages) with one 8-
// or 16-byte load issued beside the chunk's B DMA, instead of one element
// per stage.  A per-stage element load touches 32 rows' lines per
// instruction; the chunk load does that once per BCH stages.
constexpr int kScLds = 16384;
// F8X2 activations give 2 KB of it to the A slots' scale pairs, so that two
// workgroups still share a CU (80 KB each).  Beside the deep ring (one
// workgroup per CU, 80 KB of slots) the copy may take 48 KB.
constexpr int sc_lds_bytes(int ak, int ns = 2) {
  return ns == 4 ? 49152 : ak == AK_F8X2 ? kScLds - 2048 : kScLds;
}
// Row stride of the LDS scale copy: the row's bytes rounded up to dwords,
// plus a dword when that count is even.  A stage's scales are read at one
// offset from 32 consecutive rows, and an odd dword stride spreads them over
// distinct banks.  The unpadded 64-byte rows (16 dwords) of C2's down GEMM
// measured 5 bank-conflict cycles per LDS instruction (SQ_LDS_BANK_CONFLICT).
constexpr int sc_ld_bytes(int row_bytes) {
  return ((row_bytes + 3) / 4 + (((row_bytes + 3) / 4) % 2 == 0 ? 1 : 0)) * 4;
}
template <int AK, int BK, int EPI, int NWB, bool GROUPED, int BCH, int NS = 2, bool SCL = false, bool SCW = false>
__global__ __launch_bounds__(256, NS == 2 ? 2 : 1) void k_gemm_q(
    QGemmArgs g, typename std::conditional<GROUPED, GroupTable, int>::type grp) {
  constexpr bool DUAL = is_dual(EPI);
  if constexpr (GROUPED) {
    const int e = blockIdx.z;
    const int t0 = grp.off[e], rows = grp.off[e + 1] - t0;
    if ((int)(blockIdx.x % g.tiles_m) * kTM >= rows) return;  // workgroup-uniform, before any barrier
    g.m = rows;
    g.a = reinterpret_cast<const uint8_t*>(g.a) + (size_t)t0 * g.k * (AK == AK_F32 ? 4 : AK == AK_F16 ? 2 : 1);
    if (AK == AK_I8) g.a_scale += t0;
    g.c = reinterpret_cast<uint8_t*>(g.c) + (size_t)t0 * g.n * out_bytes(EPI);
    g.b0 = reinterpret_cast<const uint8_t*>(g.b0) + e * grp.b_stride;
    g.s0 = reinterpret_cast<const uint8_t*>(g.s0) + e * grp.s_stride;
    if (DUAL) {
      g.b1 = reinterpret_cast<const uint8_t*>(g.b1) + e * grp.b_stride;
      g.s1 = reinterpret_cast<const uint8_t*>(g.s1) + e * grp.s_stride;
    }
  }
  constexpr int KS = AInfo<AK>::KS;
  constexpr int RA = AInfo<AK>::RB;          // A bytes per row per stage
  constexpr int RB = b_row_bytes<BK>(KS);    // B bytes per row per stage
  constexpr int TBR = NWB * 64;               // weight rows per tile
  constexpr int RBC = RB * BCH;              // B bytes per row per chunk
  constexpr int NA = kTM * RA / 1024 / 4;    // A DMA instructions per wave per stage
  constexpr int NBC = TBR * RBC / 1024;      // B DMA instructions per chunk (all waves)
  constexpr int NB = NBC >= 4 ? NBC / 4 : 1; // per wave (waves >= NBC issue none)
  constexpr bool SCALES4 = BK == BK_MXFP4 || BK == BK_INT4G32;
  constexpr int KSTEPS = 4;
  static_assert(NA >= 1 && (NBC >= 4 ? NBC % 4 == 0 : true), "tile / stage mismatch");
  static_assert(BCH == 1 || RBC == 128, "B chunks are whole 128-byte lines");
  static_assert(NS == 2 || (NS == 4 && BCH == 1 && (!SCALES4 || SCL) && !GROUPED),
                "deep ring: per-stage B, 4-bit scales from LDS");
  static_assert(!SCW || (SCALES4 && !SCL && NS == 2 && BCH > 1 && AK == AK_F16), "chunk scale loads");
  using AccT = typename std::conditional<AK == AK_I8, v16i, v16f>::type;

  // One __shared__ array per slot: the compiler then knows that a DMA into
  // one slot does not write what the fragment reads of another slot read.
  // (Its wait insertion tells at most eight DMA targets apart, so the deep
  // ring keeps A and B of a slot in one array: four targets.)
  // F8X2 activations: the A slot also holds the stage's E8M0 pairs of the
  // 128 tile rows (512 B) and a spare 512 B that waves 2 and 3 fill with
  // the same dwords, so that every wave issues the same loads per stage.
  constexpr int SA = NS == 2 ? kTM * RA + (AK == AK_F8X2 ? 1024 : 0) : 16, SB = NS == 2 ? TBR * RBC : 16;
  constexpr int SD = NS > 2 ? kTM * RA + TBR * RBC + (AK == AK_F8X2 ? 1024 : 0) : 16;
  // F8X2 scale pairs of a stage: after A in the 2-slot A slot, after B in a deep slot
  constexpr int ASC = NS == 2 ? kTM * RA : kTM * RA + TBR * RBC;
  __shared__ __attribute__((aligned(16))) uint8_t a_s0[SA];
  __shared__ __attribute__((aligned(16))) uint8_t a_s1[SA];
  __shared__ __attribute__((aligned(16))) uint8_t b_s0[SB];
  __shared__ __attribute__((aligned(16))) uint8_t b_s1[SB];
  __shared__ __attribute__((aligned(16))) uint8_t d_s0[SD];
  __shared__ __attribute__((aligned(16))) uint8_t d_s1[SD];
  __shared__ __attribute__((aligned(16))) uint8_t d_s2[SD];
  __shared__ __attribute__((aligned(16))) uint8_t d_s3[SD];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave & 1, wn = wave >> 1;
  const int M = g.m, K = g.k;
  const int m0 = blockIdx.x % g.tiles_m * kTM;
  const int nt = blockIdx.x / g.tiles_m;
  const int n0 = DUAL ? nt * 64 : nt * TBR;  // first channel / weight row
  const int KT = K / KS / (int)gridDim.y;     // stages of this split
  const int kt0 = (int)blockIdx.y * KT;
  const size_t a_row = (size_t)K * (AK == AK_F32 ? 4 : (AK == AK_F16 || AK == AK_F8X2) ? 2 : 1);
  static_assert(AK != AK_F8X2 || ((BK == BK_MXFP4 || BK == BK_E4M3 || BK == BK_E5M2) && !GROUPED),
                "F8X2 activations: MXFP4 or FP8 weights on the scaled MFMA");
  const size_t b_row = (size_t)b_row_bytes<BK>(K);

  // ---- DMA sources (per lane, per instruction)
  constexpr int CA = RA / 16, CB = RBC / 16;  // 16-byte chunks per LDS row
  // F8X2: this lane's row of the stage-major E8M0 pairs (waves 0 / 1: tile
  // rows 64w + lane; waves 2 / 3 repeat them into the spare copy)
  const uint32_t* ae_src = AK == AK_F8X2 ? g.a_e8 + min(m0 + (wave & 1) * 64 + lane, M - 1) : nullptr;
  const uint8_t* a_src[NA];
#pragma unroll
  for (int q = 0; q < NA; q++) {
    const int r = (wave * NA + q) * (1024 / RA) + lane / CA;  // tile row
    const int c = (lane % CA) ^ swz<RA>(r);
    a_src[q] = reinterpret_cast<const uint8_t*>(g.a) + (size_t)min(m0 + r, M - 1) * a_row + c * 16;
  }
  const uint8_t* b_src[NB];
  const bool b_issuer = NBC >= 4 || wave < NBC;
#pragma unroll
  for (int q = 0; q < NB; q++) {
    const int r = (NBC >= 4 ? wave * NB + q : min(wave, NBC - 1)) * (1024 / RBC) + lane / CB;
    const int c = (lane % CB) ^ swz<RBC>(r);
    const uint8_t* base;
    int wrow;
    if (DUAL) {
      base = reinterpret_cast<const uint8_t*>(r < 64 ? g.b0 : g.b1);
      wrow = n0 + (r & 63);
    } else {
      base = reinterpret_cast<const uint8_t*>(g.b0);
      wrow = n0 + r;
    }
    b_src[q] = base + (size_t)wrow * b_row + c * 16;
  }

  // ---- fragment reads: lane (r32, h); A blocks i (rows 64wm + 32i), B
  // blocks j (tile rows: dual -> gate / up rows 32wn.., else 64wn + 32j or 32wn).
  const int r32 = lane & 31, h = lane >> 5;
  int b_blk[NWB];
#pragma unroll
  for (int j = 0; j < NWB; j++) b_blk[j] = DUAL ? j * 64 + wn * 32 : (NWB == 2 ? wn * 64 + j * 32 : wn * 32);
  // 4-bit scales: lane's block index within the stage is h (2 blocks / stage)
  const uint8_t* sc_src[NWB];
  if (SCALES4) {
#pragma unroll
    for (int j = 0; j < NWB; j++) {
      const int tr = b_blk[j] + r32;
      const int wrow = DUAL ? n0 + (tr & 63) : n0 + tr;
      const uint8_t* sb = reinterpret_cast<const uint8_t*>(DUAL && tr >= 64 ? g.s1 : g.s0);
      const int esz = BK == BK_INT4G32 ? 2 : 1;
      sc_src[j] = sb + ((size_t)wrow * (K / 32) + (size_t)kt0 * (KS / 32) + h) * esz;
    }
  }

  AccT acc[2][NWB];
#pragma unroll
  for (int i = 0; i < 2; i++)
#pragma unroll
    for (int j = 0; j < NWB; j++)
#pragma unroll
      for (int v = 0; v < 16; v++) acc[i][j][v] = 0;

  uint32_t scv[2][NWB];  // 4-bit scales of the stage in flight / in use

  // SCL: the scale block [TBR rows][KT * KS/32 entries] into LDS before any
  // operand DMA is issued.  Rows of a whole number of dwords go by dword DMA
  // (lane l of an instruction writes dword l of its 256 bytes) with no wait
  // here: the deep ring's first stage wait and barrier also cover these
  // older DMAs, and the 2-slot ring waits for them behind stage 0's operand
  // DMAs, before it reads stage 0's scales.  Other row lengths wait here.
  constexpr int ESZ = BK == BK_INT4G32 ? 2 : 1;
  __shared__ __attribute__((aligned(16))) uint8_t sc_lds[SCL ? sc_lds_bytes(AK, NS) : 16];
  const int sc_row = KT * (KS / 32) * ESZ;  // bytes of one row's scales
  const int sc_ld = sc_ld_bytes(sc_row);     // their LDS row stride
  const bool sc_dma =                       // workgroup-uniform
      SCL && sc_row % 4 == 0 && (K / 32 * ESZ) % 4 == 0 && (kt0 * (KS / 32) * ESZ) % 4 == 0;
  if constexpr (SCL) {
    static_assert(SCALES4, "scales in LDS are for 4-bit weights");
    auto src_of = [&](int tr, int byte) {
      const int wrow = DUAL ? n0 + (tr & 63) : n0 + tr;
      const uint8_t* sb = reinterpret_cast<const uint8_t*>(DUAL && tr >= 64 ? g.s1 : g.s0);
      return sb + ((size_t)wrow * (K / 32) + (size_t)kt0 * (KS / 32)) * ESZ + byte;
    };
    if (sc_dma) {
      // LDS dword i: row i / (sc_ld / 4), dword i % (sc_ld / 4); the pad
      // dword re-reads the row's first one
      const int dws = TBR * sc_ld / 4;
      for (int i0 = wave * 64; i0 < dws; i0 += 256) {  // wave-uniform
        const int i = i0 + lane;
        const int c = i % (sc_ld / 4);
        if (i < dws) dma4(src_of(i / (sc_ld / 4), c < sc_row / 4 ? c * 4 : 0), sc_lds + (size_t)i0 * 4);
      }
    } else {
      const int units = TBR * sc_row / 2;
      for (int i = tid; i < units; i += 256) {
        const int tr = i / (sc_row / 2), c = i % (sc_row / 2);
        *reinterpret_cast<uint16_t*>(sc_lds + tr * sc_ld + c * 2) =
            *reinterpret_cast<const uint16_t*>(src_of(tr, c * 2));
      }
      __syncthreads();
    }
  }

  // ONE_FORM: MXFP4 weights with f16 / f32 activations whose scales are all
  // in the LDS copy run the whole K loop in one byte-255 form, chosen by one
  // scan of the copy (sc_any255, once the copy has landed: a 0xff byte
  // anywhere picks the exact form for every stage).
  constexpr bool ONE_FORM = SCL && BK == BK_MXFP4 && AK != AK_F8X2;
  auto sc_any255 = [&]() -> bool {
    if constexpr (!ONE_FORM) {
      return false;
    } else {
      uint32_t hit = 0;
      for (int i = lane * 16; i < TBR * sc_ld; i += 64 * 16) {  // TBR * sc_ld: a multiple of 256
        const uint4 v = *reinterpret_cast<const uint4*>(sc_lds + i);
        const uint32_t d[4] = {~v.x, ~v.y, ~v.z, ~v.w};  // a 0xff byte becomes a zero byte
#pragma unroll
        for (int t = 0; t < 4; t++) hit |= (d[t] - 0x01010101u) & ~d[t] & 0x80808080u;
      }
      return __ballot(hit != 0) != 0;
    }
  };

  // SCW: chunk scales by chunk parity, SCWD dwords per row (chunk C's
  // element e of the lane's row is at byte e * ESZ of the chunk's bytes).
  constexpr int SCWD = SCW ? BCH * (KS / 32) * ESZ / 4 : 1;
  static_assert(!SCW || SCWD == 2 || SCWD == 4, "8- or 16-byte chunk scale loads");
  uint32_t scw[2][NWB][SCWD];

  // Deep ring, gate/up launches: loop stage S reads K stage MXQ_PS(S) =
  // (S + krot) mod KT.  All workgroups of such a launch read the same
  // activation lines of a stage, 8 KB or more apart; started in step, the
  // 28 workgroups of an XCD (workgroup ids 8 apart) request them from the
  // same few L2 channels at once.  Workgroup w starts at stage 7 (w / 8) mod
  // KT instead, which spreads an XCD's workgroups over distinct stages.  A
  // read probe of C3's gate/up pattern (224 workgroups, 128 weight rows and
  // 128 x 64 activations per stage): 38.7 -> 33.5 us per pass.  Same box,
  // three alternating runs: C3's W8A8 gate/up 35.1-35.5 -> 31.1-31.6 us,
  // its F8X2 gate/up 42.4-43.3 -> 41.7-41.8 us, FP8 / INT8 within noise.
  // Down GEMMs keep the in-step order: their activation lines are shared by
  // only the four workgroups of an XCD with the same split, and the rotated
  // order measured 2-5 us slower on C3's down GEMMs (fewer L2 hits).  Only
  // the f32 summation order of a tile changes.
  int krot = 0;
  if constexpr (NS > 2 && DUAL) krot = (int)(blockIdx.x + blockIdx.y * gridDim.x) / 8 * 7 % KT;
#define MXQ_PS(S) ((S) + krot >= KT ? (S) + krot - KT : (S) + krot)

  // A of stage S into slot AS; the 4-bit scales of stage S into register set P.
#define MXQ_DMA_A(S, AS)                                                                           \
  {                                                                                                \
    const int ps_ = MXQ_PS(S);                                                                     \
    const size_t ka_ = (size_t)(kt0 + ps_) * RA;                                                   \
    _Pragma("unroll") for (int q = 0; q < NA; q++)                                                 \
      dma16(a_src[q] + ka_, (AS) + (wave * NA + q) * 1024);                                         \
    if constexpr (AK == AK_F8X2) dma4(ae_src + (size_t)(kt0 + ps_) * M, (AS) + ASC + wave * 256);  \
  }
#define MXQ_SCALES(S, P)                                                                           \
  {                                                                                                \
    if constexpr (SCL) {                                                                           \
      _Pragma("unroll") for (int j = 0; j < NWB; j++) {                                             \
        const uint8_t* p_ = sc_lds + (b_blk[j] + r32) * sc_ld + (MXQ_PS(S) * (KS / 32) + h) * ESZ; \
        scv[P][j] = ESZ == 2 ? (uint32_t)*reinterpret_cast<const uint16_t*>(p_) : (uint32_t)*p_;  \
      }                                                                                            \
    } else if (SCALES4 && !SCW) {                                                                  \
      _Pragma("unroll") for (int j = 0; j < NWB; j++) {                                             \
        const uint8_t* p_ = sc_src[j] + (size_t)MXQ_PS(S) * (KS / 32) * (BK == BK_INT4G32 ? 2 : 1); \
        scv[P][j] = BK == BK_INT4G32 ? (uint32_t)*reinterpret_cast<const uint16_t*>(p_) : (uint32_t)*p_; \
      }                                                                                            \
    }                                                                                              \
  }
  // SCW: chunk C's scales of the lane's rows into set Q; stage POS of the
  // chunk in set Q into scv[P] (element POS * KS/32 + h).
#define MXQ_SCW_LOAD(C, Q)                                                                         \
  if constexpr (SCW) {                                                                             \
    _Pragma("unroll") for (int j = 0; j < NWB; j++) {                                               \
      const uint8_t* p_ = sc_src[j] - h * ESZ + (size_t)(C) * (SCWD * 4);                          \
      if constexpr (SCWD == 4) {                                                                   \
        const uint4 v_ = *reinterpret_cast<const uint4*>(p_);                                      \
        scw[Q][j][0] = v_.x; scw[Q][j][SCWD > 1 ? 1 : 0] = v_.y;                                   \
        scw[Q][j][SCWD > 2 ? 2 : 0] = v_.z; scw[Q][j][SCWD > 3 ? 3 : 0] = v_.w;                    \
      } else {                                                                                     \
        const uint2 v_ = *reinterpret_cast<const uint2*>(p_);                                      \
        scw[Q][j][0] = v_.x; scw[Q][j][SCWD > 1 ? 1 : 0] = v_.y;                                   \
      }                                                                                            \
    }                                                                                              \
  }
#define MXQ_SCW_PICK(Q, POS, P)                                                                    \
  if constexpr (SCW) {                                                                             \
    _Pragma("unroll") for (int j = 0; j < NWB; j++) {                                               \
      constexpr int e_ = (POS) * (KS / 32) * ESZ; /* byte of element POS * KS/32 (h = 0) */         \
      scv[P][j] = (scw[Q][j][(e_ / 4) % SCWD] >> (8 * (e_ % 4) + 8 * ESZ * h)) & (ESZ == 2 ? 0xffffu : 0xffu); \
    }                                                                                              \
  }
  // B chunk C (stages C*BCH .. C*BCH + BCH - 1) into slot BS.
#define MXQ_DMA_B(C, BS)                                                                         \
  {                                                                                                \
    const size_t kb_ = (size_t)(kt0 + MXQ_PS((C) * BCH)) * RB; /* krot is 0 for chunked B */       \
    if (b_issuer) {                                                                                \
      _Pragma("unroll") for (int q = 0; q < NB; q++) {                                             \
        const int qi_ = NBC >= 4 ? wave * NB + q : wave;                                           \
        dma16(b_src[q] + kb_, (BS) + qi_ * 1024);                                                  \
      }                                                                                            \
    }                                                                                              \
  }
  // loads one wave issues per stage (A + scales); a B chunk adds NB
  constexpr int VM_A = NA + (SCALES4 && !SCL && !SCW ? NWB : 0) + (AK == AK_F8X2 ? 1 : 0);
  constexpr int VM_W = SCW ? NWB : 0;  // chunk scale loads, with a B chunk

  // One stage's MFMAs, in two halves.  MXQ_READ issues every LDS fragment
  // read of the stage into registers (AR, BR); MXQ_MATH widens the weights
  // and runs the MFMAs from them.  Reading the whole stage first exposes one
  // LDS latency per stage instead of one per k-step (left to itself the
  // compiler reuses one register set and waits lgkmcnt(0) before each
  // k-step), and the deep ring reads stage st+1 while stage st's MFMAs run.
  //   AR[s][i][w]  A block i, k-step s: 16 bytes (f16 / int8) or 2 x 16 (f32)
  //   BR[u][j]     B block j: one 16-byte read per k-step (f16 / int8),
  //                per 2 k-steps (8-bit), per stage (4-bit)
  //   CO           the stage's first 16-byte chunk within a B row (chunked B)
  constexpr int BREADS = (BK == BK_MXFP4 || BK == BK_INT4G32) ? 1 : (AK != AK_I8 && BK != BK_F16) ? 2 : KSTEPS;
  constexpr int AW = AK == AK_F32 ? 2 : 1;
#define MXQ_READ(AS, BS, CO, AR, BR)                                                               \
  {                                                                                                \
    _Pragma("unroll") for (int s = 0; s < KSTEPS; s++) {                                           \
      _Pragma("unroll") for (int i = 0; i < 2; i++) {                                              \
        const int r_ = wm * 64 + i * 32 + r32;                                                     \
        if (AK == AK_F8X2 && s == 0) AR##_sc[i] = *reinterpret_cast<const uint32_t*>((AS) + ASC + r_ * 4); \
        _Pragma("unroll") for (int w = 0; w < AW; w++) {                                           \
          /* F8X2: s = 2 * term + u, lane half h holds chunks 2h, 2h + 1 of each term */            \
          const int ch_ = AK == AK_F32 ? 8 * h + 2 * s + w : AK == AK_F8X2 ? 4 * (s >> 1) + 2 * h + (s & 1) : 4 * h + s; \
          AR[s][i][w] = *reinterpret_cast<const v4i*>((AS) + r_ * RA + ((ch_ ^ swz<RA>(r_)) << 4)); \
        }                                                                                          \
      }                                                                                            \
    }                                                                                              \
    _Pragma("unroll") for (int u = 0; u < BREADS; u++) {                                           \
      _Pragma("unroll") for (int j = 0; j < NWB; j++) {                                            \
        const int r_ = b_blk[j] + r32;                                                             \
        /* FP8 weights under F8X2 activations: the scaled MFMA's 8-bit operand */                \
        /* layout, k [16h, +16) then [32 + 16h, +16), i.e. chunks h and h + 2 */                  \
        const int ch_ = (CO) + (BREADS == 1 ? h : BREADS == 2 ? (AK == AK_F8X2 ? h + 2 * u : 2 * h + u) : 4 * h + u); \
        BR[u][j] = *reinterpret_cast<const v4i*>((BS) + r_ * RBC + ((ch_ ^ swz<RBC>(r_)) << 4));  \
      }                                                                                            \
    }                                                                                              \
  }
  // MXFP4 weights: E8M0 byte 255 (+inf to the reference, NaN to the
  // hardware) needs the exact decode, which costs ~25 VALU instructions per
  // 8 values.  Left per lane, the compiler computes both decodes and selects
  // (~450 VALU per stage against 16 MFMAs); instead a ballot over the
  // stage's scale bytes picks one whole-stage form, the exact one only when
  // some lane's block has byte 255.
  // F8X2 activations: per A block i and weight block j, two
  // v_mfma_scale_f32_32x32x64_f8f6f4 (A E4M3 term t with its E8M0 byte t
  // of the pair, B FP4 with the lane's E8M0 byte) into one accumulator.
  // Lane half h of both operands holds 32-block h of the stage, so the
  // lane's own scale bytes are the ones each operand needs.  FP8 weights
  // (E4M3 / E5M2 codes, f32 row scale applied in the epilogue) go in as the
  // B operand at E8M0 127 (1.0): 32 bytes per lane, k [16h, +16) and
  // [32 + 16h, +16) of the stage, the same 8-bit layout as the A terms.
#define MXQ_MATH_F8X2(AR, BR, P)                                                                   \
  {                                                                                                \
    _Pragma("unroll") for (int i = 0; i < 2; i++) {                                                \
      v8i a1_, a2_;                                                                                \
      _Pragma("unroll") for (int t = 0; t < 4; t++) {                                              \
        a1_[t] = AR[0][i][0][t]; a1_[4 + t] = AR[1][i][0][t];                                      \
        a2_[t] = AR[2][i][0][t]; a2_[4 + t] = AR[3][i][0][t];                                      \
      }                                                                                            \
      _Pragma("unroll") for (int j = 0; j < NWB; j++) {                                            \
        v8i b_;                                                                                    \
        if constexpr (BK == BK_MXFP4) {                                                            \
          _Pragma("unroll") for (int t = 0; t < 4; t++) { b_[t] = BR[0][j][t]; b_[4 + t] = 0; }    \
        } else {                                                                                   \
          _Pragma("unroll") for (int t = 0; t < 4; t++) { b_[t] = BR[0][j][t]; b_[4 + t] = BR[1][j][t]; } \
        }                                                                                          \
        /* B format: FP4 (4) with the row's E8M0 byte, or E4M3 (0) / E5M2 (1) at scale 1.0 */      \
        constexpr int BF_ = BK == BK_MXFP4 ? 4 : BK == BK_E4M3 ? 0 : 1;                            \
        const int bs_ = BK == BK_MXFP4 ? (int)scv[P][j] : 127;                                     \
        acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a1_, b_, (v16f)acc[i][j], 0, BF_, 0, \
                                                                    (int)AR##_sc[i], 0, bs_);      \
        acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a2_, b_, (v16f)acc[i][j], 0, BF_, 1, \
                                                                    (int)AR##_sc[i], 0, bs_);      \
      }                                                                                            \
    }                                                                                              \
  }
  // EXF_: the byte-255 form of every stage of the loop in scope (0 fast, 1
  // exact), or 2: decided per stage.  A per-stage branch made the compiler
  // copy all accumulators between the two forms' registers at every stage
  // (64 v_accvgpr_mov per stage at C2's down GEMM); loops over a workgroup
  // whose scales are all in LDS decide once, from one scan of the copy.
#define MXQ_MATH(AR, BR, P)                                                                        \
  if constexpr (AK == AK_F8X2) {                                                                   \
    MXQ_MATH_F8X2(AR, BR, P)                                                                       \
  } else if constexpr (EXF_ == 0) {                                                                \
    MXQ_MATH_FORM(AR, BR, P, false)                                                                \
  } else if constexpr (EXF_ == 1) {                                                                \
    MXQ_MATH_FORM(AR, BR, P, true)                                                                 \
  } else {                                                                                         \
    bool exact_ = false;                                                                           \
    if constexpr (BK == BK_MXFP4) {                                                                \
      uint32_t hit_ = 0;                                                                           \
      _Pragma("unroll") for (int j = 0; j < NWB; j++) hit_ |= scv[P][j] == 255u;                    \
      exact_ = __ballot(hit_ != 0) != 0;                                                           \
    }                                                                                              \
    if (__builtin_expect(exact_, 0)) MXQ_MATH_FORM(AR, BR, P, true)                                \
    else MXQ_MATH_FORM(AR, BR, P, false)                                                           \
  }
#define MXQ_MATH_FORM(AR, BR, P, EXACT)                                                            \
  {                                                                                                \
    _Pragma("unroll") for (int s = 0; s < KSTEPS; s++) {                                           \
      if constexpr (AK == AK_I8) {                                                                 \
        _Pragma("unroll") for (int i = 0; i < 2; i++)                                              \
          _Pragma("unroll") for (int j = 0; j < NWB; j++)                                           \
            acc[i][j] = (AccT)__builtin_amdgcn_mfma_i32_32x32x32_i8(AR[s][i][0], BR[s][j], (v16i)acc[i][j], 0, 0, 0); \
      } else {                                                                                     \
        /* f32 activations: two f16 terms, x = hi + lo with lo = f16(x - hi) (0 where hi */      \
        /* is infinite), so the sums keep f32 x times the f16 weights to ~2^-22 of x */            \
        v8h af[2], afl[2], bf[NWB];                                                                \
        _Pragma("unroll") for (int i = 0; i < 2; i++) {                                            \
          if constexpr (AK == AK_F16) {                                                            \
            af[i] = __builtin_bit_cast(v8h, AR[s][i][0]);                                          \
          } else {                                                                                 \
            const v4f p0_ = __builtin_bit_cast(v4f, AR[s][i][0]);                                  \
            const v4f p1_ = __builtin_bit_cast(v4f, AR[s][i][AW - 1]);                             \
            _Pragma("unroll") for (int t = 0; t < 8; t++) {                                        \
              const float x_ = t < 4 ? p0_[t & 3] : p1_[t & 3];                                    \
              const _Float16 h_ = (_Float16)x_;                                                    \
              af[i][t] = h_;                                                                       \
              afl[i][t] = __builtin_isinf((float)h_) ? (_Float16)0.0f : (_Float16)(x_ - (float)h_); \
            }                                                                                      \
          }                                                                                        \
        }                                                                                          \
        _Pragma("unroll") for (int j = 0; j < NWB; j++) {                                           \
          if constexpr (BK == BK_F16) {                                                            \
            bf[j] = __builtin_bit_cast(v8h, BR[s][j]);                                             \
          } else if constexpr (BK == BK_MXFP4 || BK == BK_INT4G32) {                               \
            const v4i w_ = BR[0][j];                                                               \
            if (BK == BK_MXFP4) bf[j] = (EXACT) ? fp4x8_dequant_f16(w_[s], scv[P][j])               \
                                                : fp4x8_to_f16x8(w_[s], e8m0_as_cvt_scale(scv[P][j])); \
            else bf[j] = i4x8_to_f16(w_[s], __builtin_bit_cast(_Float16, (uint16_t)scv[P][j]));    \
          } else {                                                                                 \
            const v4i w_ = BR[s >> 1][j];                                                          \
            const uint32_t w0_ = (s & 1) ? w_[2] : w_[0], w1_ = (s & 1) ? w_[3] : w_[1];          \
            if (BK == BK_INT8) bf[j] = i8x8_to_f16(w0_, w1_);                                      \
            else bf[j] = fp8x8_to_f16<BK>(w0_, w1_);                                               \
          }                                                                                        \
        }                                                                                          \
        _Pragma("unroll") for (int i = 0; i < 2; i++)                                              \
          _Pragma("unroll") for (int j = 0; j < NWB; j++) {                                         \
            acc[i][j] = (AccT)mfma_f16_32x32x16(af[i], bf[j], (v16f)acc[i][j]);                    \
            if constexpr (AK == AK_F32) acc[i][j] = (AccT)mfma_f16_32x32x16(afl[i], bf[j], (v16f)acc[i][j]); \
          }                                                                                        \
      }                                                                                            \
    }                                                                                              \
  }
  // The 2-slot loops: a stage's reads, then its math, then every read of the
  // slot has landed before the barrier that frees it.  POS: the stage's
  // place within its B chunk (B rows hold BCH stages).
#define MXQ_COMPUTE(AS, BS, P, POS)                                                                \
  {                                                                                                \
    v4i ar_[KSTEPS][2][AW];                                                                        \
    uint32_t ar__sc[2] = {0u, 0u}; /* F8X2: E8M0 pairs of A blocks 0 / 1 */                       \
    v4i br_[BREADS][NWB];                                                                          \
    MXQ_READ(AS, BS, (POS) * (RB / 16), ar_, br_)                                                  \
    __builtin_amdgcn_sched_barrier(0); /* keep the reads ahead of the MFMAs */                     \
    MXQ_MATH(ar_, br_, P)                                                                          \
    __builtin_amdgcn_s_waitcnt(kWaitLgkm0);                                                        \
  }

  // Pipeline, one B stage per A stage (BCH = 1): stage k+1's DMA is in
  // flight while stage k is computed.  Scheduling barriers keep each stage's
  // DMA issue, wait and barrier in place: otherwise the compiler hoists the
  // next stage's scale arithmetic above the partial wait and has to drain
  // every load first.
#define MXQ_ISSUE(S, AS, BS, P) MXQ_DMA_A(S, AS) MXQ_DMA_B(S, BS) MXQ_SCALES(S, P)
#define MXQ_SYNC_POINT()                                                                           \
  __builtin_amdgcn_sched_barrier(0);                                                               \
  if (b_issuer) __builtin_amdgcn_s_waitcnt(wait_vm(VM_A + NB));                                    \
  else __builtin_amdgcn_s_waitcnt(wait_vm(VM_A));                                                  \
  __builtin_amdgcn_s_barrier();                                                                    \
  __builtin_amdgcn_sched_barrier(0);
  // Chunked B (BCH > 1): stage st issues stage st+1's A (and, on a chunk's
  // first stage, the next chunk's B) and scales, waits until only those are
  // in flight, computes st behind a barrier and frees its slots with a
  // second barrier.  vmcnt retires in issue order, so the wait also covers
  // the B chunk issued one chunk earlier.  The body is unrolled over 2 * BCH
  // stages so that every LDS slot is a constant.
#define MXQ_BODY(U)                                                                                \
  if constexpr ((U) < 2 * BCH) {                                                                   \
    if (kt + (U) < KT) {                                                                           \
      constexpr int AP_ = (U) & 1, BP_ = ((U) / BCH) & 1, POS_ = (U) % BCH;                        \
      const int st_ = kt + (U);                                                                    \
      MXQ_DMA_A(min(st_ + 1, KT - 1), (AP_ ? a_s0 : a_s1))                                         \
      if (POS_ == 0) MXQ_DMA_B(min(st_ / BCH + 1, KT / BCH - 1), (BP_ ? b_s0 : b_s1))              \
      if (POS_ == 0) MXQ_SCW_LOAD(min(st_ / BCH + 1, KT / BCH - 1), BP_ ^ 1)                       \
      MXQ_SCALES(min(st_ + 1, KT - 1), AP_ ^ 1)                                                    \
      __builtin_amdgcn_sched_barrier(0);                                                           \
      if (POS_ == 0 && b_issuer) __builtin_amdgcn_s_waitcnt(wait_vm(VM_A + NB + VM_W));            \
      else if (POS_ == 0) __builtin_amdgcn_s_waitcnt(wait_vm(VM_A + VM_W));                        \
      else __builtin_amdgcn_s_waitcnt(wait_vm(VM_A));                                              \
      __builtin_amdgcn_s_barrier();                                                                \
      __builtin_amdgcn_sched_barrier(0);                                                           \
      MXQ_SCW_PICK(BP_, POS_, AP_)                                                                 \
      MXQ_COMPUTE((AP_ ? a_s1 : a_s0), (BP_ ? b_s1 : b_s0), AP_, POS_)                             \
      __builtin_amdgcn_s_barrier();                                                                \
    }                                                                                              \
  }
  // Deep ring (NS = 4, KT % 4 == 0, KT >= 8): stage st sits in slot st % 4
  // and four stages are in flight from the start; the LDS fragments of stage
  // st+1 are read while stage st's MFMAs run (register sets 0 / 1 by
  // parity).  Iteration st:
  //   1. wait until stage st's fragments are in registers (lgkmcnt) and
  //      stage st+1's DMA has landed (vmcnt retires in issue order: only
  //      stages st+2, st+3 may remain), then one barrier.  Past it every
  //      wave has finished reading slot st, and stage st+1 is complete.
  //   2. refill slot st with stage st+4 (past the end: stage KT-1 again, so
  //      the wait count stays constant; those copies are never read).
  //   3. read stage st+1's fragments (after the last stage: a slot holding
  //      a repeated copy, never used), then stage st's MFMAs.
#define MXQ_AS(i) ((i) == 0 ? d_s0 : (i) == 1 ? d_s1 : (i) == 2 ? d_s2 : d_s3)
#define MXQ_BS(i) (MXQ_AS(i) + kTM * RA)
  // Stage body of the deep ring: refill slot st, read stage st+1's
  // fragments, stage st's math.  Issued as a block ahead of the MFMAs, the
  // DMAs and reads took about 320 cycles per 64-K stage at C2's down GEMM
  // (timed with s_memtime in a copy), with no MFMA running.  F8X2 stages,
  // and stages under f16 activations (MXFP4 weights in a loop of the fast
  // byte-255 form, or 8-bit weights), issue them between the MFMAs instead.
  // Same box: C2's scaled down GEMM 21.3-21.7 -> 18.8-19.0 us, C2's fused
  // down GEMM 22.1-22.2 -> 19.6-20.2 us, C3's FP8 / INT8 gate/up GEMMs
  // 46.2-46.5 -> 40.4-41.6 / 48.2-49.8 -> 43.5-44.1 us, C3's W8A8 gate/up
  // 33.2-33.4 -> 32.8 us.  Measured and not
  // kept: the interleave inside the per-stage byte-255 branch (fused down
  // 25.7 -> 30.5 us), and with four VALU instructions per MFMA in the
  // pattern for f16 activations (8-bit rows unchanged, fused down 2 us
  // slower).
#define MXQ_DEEP_ISSUE(U, NXT, PC)                                                                 \
  MXQ_DMA_A(min(st_ + NS, KT - 1), MXQ_AS(U))                                                      \
  MXQ_DMA_B(min(st_ + NS, KT - 1), MXQ_BS(U))                                                      \
  MXQ_READ(MXQ_AS(((U) + 1) % NS), MXQ_BS(((U) + 1) % NS), 0, NXT##_a, NXT##_b)                    \
  if constexpr (SCALES4) MXQ_SCALES(min(st_ + 1, KT - 1), (PC) ^ 1)
#define MXQ_DEEP(U, CUR, NXT)                                                                      \
  {                                                                                                \
    const int st_ = kt + (U);                                                                      \
    constexpr int PC_ = (U) & 1; /* scale set of stage st (4-bit weights) */                       \
    /* the previous stage's MFMAs stay ahead of this wait: moved past it, they */                  \
    /* would leave the next stage's LDS reads nothing to overlap */                                \
    __builtin_amdgcn_sched_barrier(0);                                                             \
    if (b_issuer) __builtin_amdgcn_s_waitcnt(wait_vm((NS - 2) * (VM_A + NB)) & ~(15 << 8));        \
    else __builtin_amdgcn_s_waitcnt(wait_vm((NS - 2) * VM_A) & ~(15 << 8));                        \
    __builtin_amdgcn_s_barrier();                                                                  \
    __builtin_amdgcn_sched_barrier(0);                                                             \
    MXQ_DEEP_ISSUE(U, NXT, PC_)                                                                    \
    if constexpr (DEEP_IL) {                                                                       \
      MXQ_MATH(CUR##_a, CUR##_b, PC_)                                                              \
      _Pragma("unroll") for (int q_ = 0; q_ < DEEP_VM; q_++) {                                     \
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                                         \
        __builtin_amdgcn_sched_group_barrier(0x100, DEEP_DS, 0);                                   \
        __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);                                         \
        if constexpr (DEEP_VALU > 0) __builtin_amdgcn_sched_group_barrier(0x002, DEEP_VALU, 0);    \
      }                                                                                            \
      _Pragma("unroll") for (int q_ = DEEP_VM; q_ < DEEP_MF; q_++) {                               \
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                                         \
        __builtin_amdgcn_sched_group_barrier(0x100, DEEP_DS, 0);                                   \
        if constexpr (DEEP_VALU > 0) __builtin_amdgcn_sched_group_barrier(0x002, DEEP_VALU, 0);    \
      }                                                                                            \
      __builtin_amdgcn_sched_barrier(0);                                                           \
    } else {                                                                                       \
      __builtin_amdgcn_sched_barrier(0);                                                           \
      MXQ_MATH(CUR##_a, CUR##_b, PC_)                                                              \
    }                                                                                              \
  }
  // Interleaved deep-ring stages (F8X2 activations; MXFP4 weights under f16
  // activations in the fast byte-255 form): per MFMA, DEEP_DS LDS reads, one
  // DMA while they last, and for F8X2 up to four VALU instructions (the
  // operand packing; the f16 form leaves its decode to the scheduler, which
  // measured 2 us faster at C2's down GEMM than four VALU per MFMA).
  constexpr int DEEP_MF = AK == AK_F8X2 ? 2 * NWB * 2 : 2 * NWB * KSTEPS;
  constexpr int DEEP_NDS = KSTEPS * 2 * AW + BREADS * NWB + (SCALES4 ? NWB : 0) + (AK == AK_F8X2 ? 2 : 0);
  constexpr int DEEP_VALU = AK == AK_F8X2 ? 4 : 0;
  // which loops interleave: F8X2; int8 activations (W8A8); f16 activations
  // with MXFP4 weights in the fast byte-255 loop (EXF_ 0), or with 8-bit or
  // INT4 weights (no byte-255 forms).  INT4's decode (17 VALU per 8 values)
  // is left to the scheduler too: eight VALU per MFMA in the pattern
  // measured 1-2 us slower on C3's INT4 gate/up.
#define DEEP_IL (AK == AK_F8X2 || AK == AK_I8 || (AK == AK_F16 && (EXF_ == 0 || BK != BK_MXFP4)))
  constexpr int DEEP_DS = (DEEP_NDS + DEEP_MF - 1) / DEEP_MF;
  constexpr int DEEP_VM = VM_A + NB;
  if constexpr (NS > 2) {
    static_assert(NS == 4 && (NS - 1) * (VM_A + NB) <= 63, "vmcnt range");
    v4i f0_a[KSTEPS][2][AW], f1_a[KSTEPS][2][AW];
    uint32_t f0_a_sc[2] = {0u, 0u}, f1_a_sc[2] = {0u, 0u};  // F8X2: E8M0 pairs by fragment set
    v4i f0_b[BREADS][NWB], f1_b[BREADS][NWB];
    MXQ_DMA_A(0, MXQ_AS(0)) MXQ_DMA_B(0, MXQ_BS(0))
    MXQ_DMA_A(1, MXQ_AS(1)) MXQ_DMA_B(1, MXQ_BS(1))
    MXQ_DMA_A(2, MXQ_AS(2)) MXQ_DMA_B(2, MXQ_BS(2))
    MXQ_DMA_A(3, MXQ_AS(3)) MXQ_DMA_B(3, MXQ_BS(3))
    if (b_issuer) __builtin_amdgcn_s_waitcnt(wait_vm((NS - 1) * (VM_A + NB)));
    else __builtin_amdgcn_s_waitcnt(wait_vm((NS - 1) * VM_A));
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    const bool any255 = sc_any255();
    __builtin_amdgcn_sched_barrier(0);
    MXQ_READ(MXQ_AS(0), MXQ_BS(0), 0, f0_a, f0_b)
    if constexpr (SCALES4) MXQ_SCALES(0, 0)
    __builtin_amdgcn_sched_barrier(0);
    auto deep_loop = [&](auto exf) {
      constexpr int EXF_ = decltype(exf)::value;
      for (int kt = 0; kt < KT; kt += NS) {
        MXQ_DEEP(0, f0, f1) MXQ_DEEP(1, f1, f0) MXQ_DEEP(2, f0, f1) MXQ_DEEP(3, f1, f0)
      }
    };
    if constexpr (ONE_FORM) {
      if (__builtin_expect(any255, 0)) deep_loop(std::integral_constant<int, 1>{});
      else deep_loop(std::integral_constant<int, 0>{});
    } else {
      deep_loop(std::integral_constant<int, 2>{});
    }
  } else {
  MXQ_DMA_A(0, a_s0)
  MXQ_DMA_B(0, b_s0)
  MXQ_SCW_LOAD(0, 0)
  if (sc_dma) {  // the scale DMAs (issued first) have landed; a bare barrier
    __builtin_amdgcn_sched_barrier(0);
    if (b_issuer) __builtin_amdgcn_s_waitcnt(wait_vm(VM_A + NB));
    else __builtin_amdgcn_s_waitcnt(wait_vm(VM_A));
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
  }
  const bool any255 = sc_any255();
  MXQ_SCALES(0, 0)
  auto ring2_loop = [&](auto exf) {
  constexpr int EXF_ = decltype(exf)::value;
  if constexpr (BCH == 1) {
    int kt = 0;
    for (; kt + 2 <= KT; kt += 2) {
      MXQ_ISSUE(kt + 1, a_s1, b_s1, 1)
      MXQ_SYNC_POINT()
      MXQ_COMPUTE(a_s0, b_s0, 0, 0)
      __builtin_amdgcn_s_barrier();  // slot 0 free
      MXQ_ISSUE(min(kt + 2, KT - 1), a_s0, b_s0, 0)
      MXQ_SYNC_POINT()
      MXQ_COMPUTE(a_s1, b_s1, 1, 0)
      __builtin_amdgcn_s_barrier();  // slot 1 free
    }
    if (kt < KT) {  // odd stage count: the last stage sits in slot 0
      __builtin_amdgcn_s_waitcnt(wait_vm(0));
      __builtin_amdgcn_s_barrier();
      MXQ_COMPUTE(a_s0, b_s0, 0, 0)
    }
  } else {
    for (int kt = 0; kt < KT; kt += 2 * BCH) {
      MXQ_BODY(0) MXQ_BODY(1) MXQ_BODY(2) MXQ_BODY(3)
      MXQ_BODY(4) MXQ_BODY(5) MXQ_BODY(6) MXQ_BODY(7)
    }
  }
  };
  if constexpr (ONE_FORM) {
    if (__builtin_expect(any255, 0)) ring2_loop(std::integral_constant<int, 1>{});
    else ring2_loop(std::integral_constant<int, 0>{});
  } else {
    ring2_loop(std::integral_constant<int, 2>{});
  }
  }
#undef MXQ_DEEP
#undef MXQ_DEEP_ISSUE
#undef DEEP_IL
#undef MXQ_AS
#undef MXQ_BS
#undef MXQ_BODY
#undef MXQ_SYNC_POINT
#undef MXQ_ISSUE
  __builtin_amdgcn_s_waitcnt(0);
#undef MXQ_DMA_A
#undef MXQ_DMA_B
#undef MXQ_SCALES
#undef MXQ_PS
#undef MXQ_SCW_LOAD
#undef MXQ_SCW_PICK
#undef MXQ_COMPUTE
#undef MXQ_MATH_FORM
#undef MXQ_MATH_F8X2
#undef MXQ_MATH
#undef MXQ_READ

  // ---- epilogue, or the raw partial tile when K is split (separate loops
  // behind one uniform branch).
  constexpr int PL = DUAL ? 2 : 1;
  // A tile whose rows are all below M stores without per-row guards: behind
  // the guards each store sits in its own branch and the compiler waits for
  // the previous store before reusing its address registers, one round trip
  // per element.
  const bool full_tile = m0 + kTM <= M;
  if (gridDim.y > 1) {
    const size_t plane = (size_t)M * g.n;
    uint32_t* w = reinterpret_cast<uint32_t*>(g.ws) + (size_t)blockIdx.y * PL * plane;
#pragma unroll
    for (int i = 0; i < 2; i++) {
#pragma unroll
      for (int jj = 0; jj < (DUAL ? 1 : NWB); jj++) {
        const int col = DUAL ? n0 + wn * 32 + r32 : n0 + b_blk[jj] + r32;
        uint32_t gv[16], uv[16];
#pragma unroll
        for (int v = 0; v < 16; v++) {
          // copy the vector element to a scalar first: __builtin_bit_cast of
          // a vector-element subscript yields element 0 for every v
          const auto ge = acc[i][jj][v], ue = acc[i][NWB - 1][v];
          gv[v] = __builtin_bit_cast(uint32_t, ge);
          uv[v] = DUAL ? __builtin_bit_cast(uint32_t, ue) : 0u;
        }
        auto put = [&](auto guarded) {
#pragma unroll
          for (int v = 0; v < 16; v++) {
            const int row = m0 + wm * 64 + i * 32 + acc32_row(lane, v);
            if (!decltype(guarded)::value || row < M) {
              const size_t o = (size_t)row * g.n + col;
              w[o] = gv[v];
              if (DUAL) w[plane + o] = uv[v];
            }
          }
        };
        if (full_tile) put(std::false_type{});
        else put(std::true_type{});
      }
    }
    return;
  }
  if constexpr (EPI == EPI_SWIGLU_F8X2) {
    // mid = silu(g) * u of the tile's 128 rows x 64 channels, which is one
    // 64-K group of the down GEMM's F8X2 input, goes through LDS: wave
    // (wm, wn) writes rows [64 wm, +64) x channels [32 wn, +32) into ring
    // slot wm (16 KB each: the 2-slot A slots or the first two deep slots;
    // row r, channel c at r * 64 + (c ^ (r & 31)): the column writes and the
    // row reads both spread over the banks), then lane pair p of the
    // workgroup splits row p.
    static_assert((NS == 2 ? SA : SD) >= 64 * 64 * 4, "mid tile half fits a ring slot");
    uint8_t* const ms0 = NS == 2 ? a_s0 : d_s0;
    uint8_t* const ms1 = NS == 2 ? a_s1 : d_s1;
    __syncthreads();
    float* ml = reinterpret_cast<float*>(wm ? ms1 : ms0);
    // FP8 weights: the gate / up row scales of the lane's channel
    const float csg = row_scale<BK>(g.s0, n0 + wn * 32 + r32), csu = row_scale<BK>(g.s1, n0 + wn * 32 + r32);
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
      for (int v = 0; v < 16; v++) {
        const int rl = i * 32 + acc32_row(lane, v), c = wn * 32 + r32;
        float x0 = acc[i][0][v], u = acc[i][NWB - 1][v];
        if (row_scaled(BK)) { x0 = x0 * csg; u = u * csu; }
        ml[rl * 64 + (c ^ (rl & 31))] = silu(x0) * u;
      }
    __syncthreads();
    const int pr = tid >> 1, half = tid & 1, rl = pr & 63;
    float* src = reinterpret_cast<float*>(pr < 64 ? ms0 : ms1);
    float mv[32];
    uint32_t nf = 0;  // a non-finite mid value among the lane's 32
#pragma unroll
    for (int k = 0; k < 32; k++) {
      const int c = 32 * half + k;
      mv[k] = src[rl * 64 + (c ^ (rl & 31))];
      nf |= (uint32_t)((__builtin_bit_cast(uint32_t, mv[k]) & 0x7fffffffu) >= 0x7f800000u);
    }
    const int row = m0 + pr, grp = n0 / 64;
    // E8M0 byte 255 in a gate / up scale (NaN in the scaled MFMA, +inf in the
    // reference) or a non-finite x leaves non-finite mid values: those
    // channels are recomputed from the f16 activations with the reference's
    // dequantization (rare; one wave-uniform test).  One rolled loop, results
    // back through the lane's own LDS slots.
    if (__builtin_expect(__ballot(nf != 0) != 0, 0)) {
      if (nf && row < M && g.a_f16) {
        const uint16_t* xr = g.a_f16 + (size_t)row * K;
#pragma nounroll
        for (int k = 0; k < 32; k++) {
          const int c = 32 * half + k, ch = n0 + c;
          float* p = src + rl * 64 + (c ^ (rl & 31));
          if ((__builtin_bit_cast(uint32_t, *p) & 0x7fffffffu) >= 0x7f800000u) {
            float gv = ref_dot_f16_w<BK>(xr, g.b0, g.s0, ch, K), uv = ref_dot_f16_w<BK>(xr, g.b1, g.s1, ch, K);
            if (row_scaled(BK)) { gv = gv * row_scale<BK>(g.s0, ch); uv = uv * row_scale<BK>(g.s1, ch); }
            *p = (gv / (1.0f + expf(-gv))) * uv;
          }
        }
#pragma unroll
        for (int k = 0; k < 32; k++) {
          const int c = 32 * half + k;
          mv[k] = src[rl * 64 + (c ^ (rl & 31))];
        }
      }
    }
    if (row < M)
      f8x2_split_store<2>(mv, half, reinterpret_cast<uint8_t*>(g.c) + (size_t)row * 2 * g.n + (size_t)grp * 128,
                          g.c_e8 + (size_t)grp * M + row);
    return;
  }
  // The scales are loaded up front, unconditionally (rows clamped), so the
  // per-element stores below wait on none of them: left inside the row
  // guards, each element re-loads its scales and waits for them in turn.
  float rs[2][16];  // per-token scale of each accumulator row (W8A8)
#pragma unroll
  for (int i = 0; i < 2; i++)
#pragma unroll
    for (int v = 0; v < 16; v++)
      rs[i][v] = AK == AK_I8 ? g.a_scale[min(m0 + wm * 64 + i * 32 + acc32_row(lane, v), M - 1)] : 1.0f;
  float cs0[NWB], cs1 = 1.0f;  // per weight row scales (gate / single, up)
#pragma unroll
  for (int jj = 0; jj < NWB; jj++) {
    const int col = DUAL ? n0 + wn * 32 + r32 : n0 + b_blk[jj] + r32;
    cs0[jj] = row_scaled(BK) ? reinterpret_cast<const float*>(g.s0)[col] : 1.0f;
  }
  if (DUAL && row_scaled(BK)) cs1 = reinterpret_cast<const float*>(g.s1)[n0 + wn * 32 + r32];
  auto epilogue = [&](auto guarded) {
#pragma unroll
  for (int i = 0; i < 2; i++) {
#pragma unroll
    for (int jj = 0; jj < (DUAL ? 1 : NWB); jj++) {
      const int col = DUAL ? n0 + wn * 32 + r32 : n0 + b_blk[jj] + r32;
#pragma unroll
      for (int v = 0; v < 16; v++) {
        const int row = m0 + wm * 64 + i * 32 + acc32_row(lane, v);
        if (decltype(guarded)::value && row >= M) continue;
        const size_t o = (size_t)row * g.n + col;
        if (EPI == EPI_STORE_I32) {
          reinterpret_cast<int*>(g.c)[o] = (int)acc[i][jj][v];
          continue;
        }
        // same products, in the same order, as scaled(): acc * row scale * column scale
        const float g0 = AK == AK_I8 ? (float)(int)acc[i][jj][v] : (float)acc[i][jj][v];
        float x0 = g0;
        if (AK == AK_I8) x0 = x0 * rs[i][v];
        if (row_scaled(BK)) x0 = x0 * cs0[jj];
        float u = 0.0f;
        if (DUAL) {
          const float u0 = AK == AK_I8 ? (float)(int)acc[i][NWB - 1][v] : (float)acc[i][NWB - 1][v];
          u = u0;
          if (AK == AK_I8) u = u * rs[i][v];
          if (row_scaled(BK)) u = u * cs1;
        }
        epi_store<EPI>(g.c, o, x0, u);
      }
    }
  }
  };
  if (full_tile) epilogue(std::false_type{});
  else epilogue(std::true_type{});
  if constexpr (AK == AK_F8X2 && !DUAL) {
    // A NaN output (E8M0 byte 255 in a weight scale: NaN in the scaled MFMA,
    // +inf in the reference; or a non-finite activation group) is recomputed
    // with the reference's dequantization (rare; one wave-uniform test).
    uint64_t nanm = 0;  // bit (i NWB + jj) 16 + v: element is NaN
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
      for (int jj = 0; jj < NWB; jj++)
#pragma unroll
        for (int v = 0; v < 16; v++) {
          const float x0 = acc[i][jj][v];
          nanm |= (uint64_t)(x0 != x0) << ((i * NWB + jj) * 16 + v);
        }
    if (__builtin_expect(__ballot(nanm != 0) != 0, 0)) {
      const uint8_t* ad = reinterpret_cast<const uint8_t*>(g.a);
#pragma nounroll
      for (int e = 0; e < 2 * NWB * 16; e++) {
        if (!((nanm >> e) & 1u)) continue;
        const int i = e / (NWB * 16), jj = (e / 16) % NWB, v = e % 16;
        const int row = m0 + wm * 64 + i * 32 + acc32_row(lane, v);
        const int col = n0 + b_blk[jj] + r32;
        if (row >= M) continue;
        float r = ref_dot_f8x2_w<BK>(ad, g.a_e8, M, row, g.b0, g.s0, col, K);
        if (row_scaled(BK)) r = r * row_scale<BK>(g.s0, col);
        epi_store<EPI>(g.c, (size_t)row * g.n + col, r, 0.0f);
      }
    }
  }
}

// Split-K reduction + epilogue: four consecutive output elements per thread
// (m * n % 4 == 0 since n % 64 == 0), 16-byte loads from the 256-byte
// aligned partial planes; each element still sums its splits in split order.
template <int AK, int BK, int EPI>
__global__ void k_gemm_q_reduce(QGemmArgs g, int splits) {
  constexpr bool DUAL = is_dual(EPI);
  constexpr int PL = DUAL ? 2 : 1;
  const size_t plane = (size_t)g.m * g.n;
  if constexpr (EPI == EPI_SWIGLU_F8X2) {
    // 16 lanes per (row, 64-channel group), 4 channels each; a group past
    // the end exits as a whole
    const size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int j = (int)(t & 15);
    const int groups = g.n / 64;
    const size_t gi = t >> 4;
    if (gi >= (size_t)g.m * groups) return;
    const int row = (int)(gi / groups), grp = (int)(gi % groups);
    const size_t o = (size_t)row * g.n + (size_t)grp * 64 + 4 * j;
    const float* w = reinterpret_cast<const float*>(g.ws);
    float gs[4] = {0.0f, 0.0f, 0.0f, 0.0f}, us[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int k = 0; k < splits; k++) {
      const float4 a = *reinterpret_cast<const float4*>(w + (size_t)(2 * k) * plane + o);
      const float4 b = *reinterpret_cast<const float4*>(w + (size_t)(2 * k + 1) * plane + o);
      gs[0] += a.x; gs[1] += a.y; gs[2] += a.z; gs[3] += a.w;
      us[0] += b.x; us[1] += b.y; us[2] += b.z; us[3] += b.w;
    }
    float mv[4];
#pragma unroll
    for (int c = 0; c < 4; c++) {
      const int ch = grp * 64 + 4 * j + c;
      const float gg = row_scaled(BK) ? gs[c] * row_scale<BK>(g.s0, ch) : gs[c];
      const float uu = row_scaled(BK) ? us[c] * row_scale<BK>(g.s1, ch) : us[c];
      mv[c] = silu(gg) * uu;
    }
    // non-finite mid (E8M0 byte 255 in a gate / up scale, or a non-finite x):
    // recomputed from the f16 activations with the reference's dequantization
    if (g.a_f16) {
      const int K = g.k;
#pragma unroll
      for (int c = 0; c < 4; c++) {
        if ((__builtin_bit_cast(uint32_t, mv[c]) & 0x7fffffffu) >= 0x7f800000u) {
          const int ch = grp * 64 + 4 * j + c;
          const uint16_t* xr = g.a_f16 + (size_t)row * K;
          float gv = ref_dot_f16_w<BK>(xr, g.b0, g.s0, ch, K), uv = ref_dot_f16_w<BK>(xr, g.b1, g.s1, ch, K);
          if (row_scaled(BK)) { gv = gv * row_scale<BK>(g.s0, ch); uv = uv * row_scale<BK>(g.s1, ch); }
          mv[c] = (gv / (1.0f + expf(-gv))) * uv;
        }
      }
    }
    f8x2_split_store<16>(mv, j, reinterpret_cast<uint8_t*>(g.c) + (size_t)row * 2 * g.n + (size_t)grp * 128,
                         g.c_e8 + (size_t)grp * g.m + row);
    return;
  }
  const size_t o = ((size_t)blockIdx.x * blockDim.x + threadIdx.x) * 4;
  if (o >= plane) return;
  const int row = (int)(o / g.n), col = (int)(o % g.n);
  const uint32_t* w = reinterpret_cast<const uint32_t*>(g.ws);
  auto ld4 = [&](size_t idx) { return *reinterpret_cast<const uint4*>(w + idx); };
  if (EPI == EPI_STORE_I32) {
    int s[4] = {0, 0, 0, 0};
    for (int k = 0; k < splits; k++) {
      const uint4 v = ld4((size_t)k * plane + o);
      s[0] += (int)v.x; s[1] += (int)v.y; s[2] += (int)v.z; s[3] += (int)v.w;
    }
#pragma unroll
    for (int t = 0; t < 4; t++) reinterpret_cast<int*>(g.c)[o + t] = s[t];  // caller's buffer: 4-byte aligned
    return;
  }
  float sums[2][4];
#pragma unroll
  for (int p = 0; p < PL; p++) {
    if (AK == AK_I8) {
      int s[4] = {0, 0, 0, 0};
      for (int k = 0; k < splits; k++) {
        const uint4 v = ld4(((size_t)k * PL + p) * plane + o);
        s[0] += (int)v.x; s[1] += (int)v.y; s[2] += (int)v.z; s[3] += (int)v.w;
      }
#pragma unroll
      for (int t = 0; t < 4; t++) sums[p][t] = (float)s[t];
    } else {
      float s[4] = {0.0f, 0.0f, 0.0f, 0.0f};
      for (int k = 0; k < splits; k++) {
        const uint4 v = ld4(((size_t)k * PL + p) * plane + o);
        s[0] += __builtin_bit_cast(float, v.x); s[1] += __builtin_bit_cast(float, v.y);
        s[2] += __builtin_bit_cast(float, v.z); s[3] += __builtin_bit_cast(float, v.w);
      }
#pragma unroll
      for (int t = 0; t < 4; t++) sums[p][t] = s[t];
    }
  }
#pragma unroll
  for (int t = 0; t < 4; t++) {
    float x0 = scaled<AK, BK>(sums[0][t], g, reinterpret_cast<const float*>(g.s0), row, col + t);
    const float u = DUAL ? scaled<AK, BK>(sums[PL - 1][t], g, reinterpret_cast<const float*>(g.s1), row, col + t) : 0.0f;
    if (AK == AK_F8X2 && !DUAL && x0 != x0) {
      // E8M0 byte 255 in a weight scale (NaN in the scaled MFMA, +inf in the
      // reference) or a non-finite activation group: recomputed with the
      // reference's dequantization
      x0 = ref_dot_f8x2_w<BK>(reinterpret_cast<const uint8_t*>(g.a), g.a_e8, g.m, row, g.b0, g.s0, col + t, g.k);
      if (row_scaled(BK)) x0 = x0 * row_scale<BK>(g.s0, col + t);
    }
    epi_store<EPI>(g.c, o + t, x0, u);
  }
}

// Stages per B chunk that make a chunk one 128-byte line per weight row.
// (4-bit weights only: for 8-bit rows the chunked loop measured no faster)
template <int AK, int BK> constexpr int b_chunk() {
  return (BK == BK_MXFP4 || BK == BK_INT4G32) ? 128 / b_row_bytes<BK>(AInfo<AK>::KS) : 1;
}

// True when a workgroup's scales over kt stages fit the LDS copy (SCL).
template <int AK, int BK, int NWB, int NS = 2> bool sc_lds_fits(int kt) {
  return NWB * 64 * sc_ld_bytes(kt * (AInfo<AK>::KS / 32) * (BK == BK_INT4G32 ? 2 : 1)) <= sc_lds_bytes(AK, NS);
}

// True when the chunk scale loads (SCW) are aligned: every row's scales, the
// planes and the per-group stride a multiple of a chunk's scale bytes (split
// starts are whole chunks).
template <int AK, int BK> bool scw_ok(const QGemmArgs& g, bool dual, size_t s_stride) {
  if constexpr (AK != AK_F16 || !(BK == BK_MXFP4 || BK == BK_INT4G32)) {
    return false;
  } else {
    constexpr size_t cb = b_chunk<AK, BK>() * (AInfo<AK>::KS / 32) * (BK == BK_INT4G32 ? 2 : 1);
    const size_t row = (size_t)g.k / 32 * (BK == BK_INT4G32 ? 2 : 1);
    return row % cb == 0 && s_stride % cb == 0 && (uintptr_t)g.s0 % cb == 0 && (!dual || (uintptr_t)g.s1 % cb == 0);
  }
}

// Launches of at most this many workgroups (one per CU) take the deep ring,
// for weight formats staged per stage whose four slots fit the 160 KB of LDS
// (not f32 activations x f16 weights: 4 x 48 KB).  MXFP4 weights under f16
// activations take it too, with their E8M0 scales in LDS beside the ring
// (80 KB + up to 48 KB) when those fit, for splits of at least 16 stages
// (C2's down GEMM, 224 workgroups: 27.4 -> 24.4 us).  INT4 g32 weights do
// the same with their f16 scales.  Same box, three alternating runs: C3's
// INT4 gate/up 53.1-54.0 -> 49.9-51.1 us; its down GEMM, as 32 tiles of 128
// rows x 8 splits on the deep ring against 64 tiles of 64 rows x 8 splits
// on the 2-slot ring, 30.2-30.4 -> 29.3-29.4 us (MLP 75.3-75.4 -> 73.0-73.4
// us, stream-timed).
constexpr int kDeepMaxWgs = 256;
constexpr bool deep_format(int ak, int bk) {
  const int ks = ak == AK_I8 ? 128 : 64;
  const int ra = ak == AK_F32 ? 256 : 128;
  const int rb = bk == BK_F16 ? ks * 2 : ks;
  if (bk == BK_MXFP4) return ak == AK_F16 || ak == AK_F8X2;
  if (bk == BK_INT4G32) return ak == AK_F16;
  return 4 * 128 * (ra + rb) <= 160 * 1024;
}

// Workgroups of the split-K reduction: 4 outputs per thread (16 lanes per
// (row, 64-channel group) for the F8X2 mid).
template <int EPI> unsigned reduce_blocks(int m, int n) {
  const size_t threads = (size_t)m * n / 4;
  return (unsigned)((threads + 255) / 256);
}

template <int AK, int BK, int EPI, int NWB>
hipError_t launch_q(const QGemmArgs& g0, int splits, hipStream_t st) {
  QGemmArgs g = g0;
  g.tiles_m = (g.m + kTM - 1) / kTM;
  const int tiles_n = is_dual(EPI) ? g.n / 64 : g.n / (NWB * 64);
  constexpr int BC = b_chunk<AK, BK>();
  const int kt = g.k / AInfo<AK>::KS / splits;  // stages per split
  // (the ungrouped form's second argument is an unused int: a sized type
  // keeps the host and device kernel-argument layouts identical)
  // chunked B once a split spans at least four chunks (a shorter split would
  // wait for its whole B up front)
  if constexpr (deep_format(AK, BK)) {
    // MXFP4: scales in LDS, and at least 16 stages (C0's 8-stage splits
    // measured 1 us slower per GEMM on the deep ring: its fill and drain
    // are not repaid)
    constexpr bool S4D = BK == BK_MXFP4 || BK == BK_INT4G32;
    if (g.tiles_m * tiles_n * splits <= kDeepMaxWgs && kt >= 8 && kt % 4 == 0 &&
        (!S4D || (kt >= 16 && sc_lds_fits<AK, BK, NWB, 4>(kt)))) {
      hipLaunchKernelGGL((k_gemm_q<AK, BK, EPI, NWB, false, 1, 4, S4D>), dim3(g.tiles_m * tiles_n, splits), dim3(256),
                         0, st, g, 0);
      if (splits > 1)
        hipLaunchKernelGGL((k_gemm_q_reduce<AK, BK, EPI>), dim3(reduce_blocks<EPI>(g.m, g.n)), dim3(256), 0, st, g,
                           splits);
      return hipGetLastError();
    }
  }
  const dim3 grid(g.tiles_m * tiles_n, splits);
  constexpr bool S4 = BK == BK_MXFP4 || BK == BK_INT4G32;
  const bool scl = S4 && sc_lds_fits<AK, BK, NWB>(kt);
  if (BC > 1 && kt % BC == 0 && kt >= 4 * BC) {
    constexpr bool W = AK == AK_F16 && S4 && BC > 1;
    if (scl) hipLaunchKernelGGL((k_gemm_q<AK, BK, EPI, NWB, false, BC, 2, S4>), grid, dim3(256), 0, st, g, 0);
    else if (W && scw_ok<AK, BK>(g, is_dual(EPI), 0))
      hipLaunchKernelGGL((k_gemm_q<AK, BK, EPI, NWB, false, BC, 2, false, W>), grid, dim3(256), 0, st, g, 0);
    else hipLaunchKernelGGL((k_gemm_q<AK, BK, EPI, NWB, false, BC>), grid, dim3(256), 0, st, g, 0);
  } else {
    if (scl) hipLaunchKernelGGL((k_gemm_q<AK, BK, EPI, NWB, false, 1, 2, S4>), grid, dim3(256), 0, st, g, 0);
    else hipLaunchKernelGGL((k_gemm_q<AK, BK, EPI, NWB, false, 1>), grid, dim3(256), 0, st, g, 0);
  }
  if (splits > 1)
    hipLaunchKernelGGL((k_gemm_q_reduce<AK, BK, EPI>), dim3(reduce_blocks<EPI>(g.m, g.n)), dim3(256), 0, st, g, splits);
  return hipGetLastError();
}

// Plain (non-SwiGLU) GEMMs take 128-row weight tiles when N allows, except
// MXFP4 with fewer than 16 of them: 64-row tiles then give the grid twice
// the tiles (C0's down GEMM, N = 1024: 13.5 -> 12.6 us per step with its
// reduce, 12.25 -> 11.5 us on the F8X2 path).  INT4 took 64-row tiles below
// 64 wide tiles while it ran on the 2-slot ring only (C3's down GEMM, N =
// 4096: MLP 96.8 -> 94.1 us then); on the deep ring its 128-row tiles halve
// the activation re-reads and measured faster (launch_q's note).  Other
// formats measured no gain (C3) or a loss (C2 dequant, f16 weights: +2.5
// us).  C2's MXFP4 down GEMM on 64-row tiles (448 two-slot workgroups
// instead of 224 on the deep ring): fused 23.6 -> 24.9 us; scaled 20.2 ->
// 18.7 us but the scaled MLP unchanged (66.1-67.1 against 67.0-67.3 us).
inline bool wide_tiles(int bk, int epi, int n) {
  return !is_dual(epi) && n % 128 == 0 && !(bk == BK_MXFP4 && n / 128 < 16);
}

template <int AK, int BK, int EPI>
hipError_t launch_wn(const QGemmArgs& g, int splits, hipStream_t st) {
  if (is_dual(EPI) || wide_tiles(BK, EPI, g.n)) return launch_q<AK, BK, EPI, 2>(g, splits, st);
  return launch_q<AK, BK, EPI, 1>(g, splits, st);
}

int stage_k(int ak) { return ak == AK_I8 ? 128 : 64; }

// Grouped launch: g.m = the largest group's rows.
template <int AK, int BK, int EPI, int NWB>
hipError_t launch_q_grouped(const QGemmArgs& g0, const GroupTable& gt, int groups, hipStream_t st) {
  QGemmArgs g = g0;
  g.tiles_m = (g.m + kTM - 1) / kTM;
  const int tiles_n = is_dual(EPI) ? g.n / 64 : g.n / (NWB * 64);
  constexpr int BC = b_chunk<AK, BK>();
  const int kt = g.k / AInfo<AK>::KS;
  const dim3 grid(g.tiles_m * tiles_n, 1, groups);
  const bool scl = sc_lds_fits<AK, BK, NWB>(kt);  // MXFP4 only here
  if (BC > 1 && kt % BC == 0 && kt >= 4 * BC) {
    if (scl) hipLaunchKernelGGL((k_gemm_q<AK, BK, EPI, NWB, true, BC, 2, true>), grid, dim3(256), 0, st, g, gt);
    else if (scw_ok<AK, BK>(g, is_dual(EPI), gt.s_stride))
      hipLaunchKernelGGL((k_gemm_q<AK, BK, EPI, NWB, true, BC, 2, false, true>), grid, dim3(256), 0, st, g, gt);
    else hipLaunchKernelGGL((k_gemm_q<AK, BK, EPI, NWB, true, BC>), grid, dim3(256), 0, st, g, gt);
  } else {
    if (scl) hipLaunchKernelGGL((k_gemm_q<AK, BK, EPI, NWB, true, 1, 2, true>), grid, dim3(256), 0, st, g, gt);
    else hipLaunchKernelGGL((k_gemm_q<AK, BK, EPI, NWB, true, 1>), grid, dim3(256), 0, st, g, gt);
  }
  return hipGetLastError();
}

}  // namespace qgemm

using namespace qgemm;

// Split count: enough workgroups to cover the CUs about 1.5 times when the
// tiles alone do not, keeping at least 8 stages per split (shorter splits
// lose more to the partial-sum round trip and the reduce launch than they
// gain in parallelism: the dual gate/up GEMM at M=128, N=4096, K=1024,
// 16 stages, runs 14.9 us at two splits against 17.4 us at four).  From 192
// tiles on (three quarters of the CUs busy without a split) K is not split:
// the f32 partials would move more bytes than the weights (W8A8 at M=128,
// N=2x14336, K=4096: 80 -> 72 us for the MLP without the split).
// Formats that take the deep ring split only as far as one workgroup per
// CU (at most 256 workgroups), keeping a multiple of 4 stages per split.
int gemm_q_splits(int ak, int bk, int epi, int m, int n, int k) {
  const int tiles = ((m + kTM - 1) / kTM) * (is_dual(epi) ? n / 64 : (wide_tiles(bk, epi, n) ? n / 128 : n / 64));
  const int kt = k / stage_k(ak);
  if (tiles >= 192) return 1;
  // MXFP4 gate/up with f16 activations and 16 stages: unsplit on the deep
  // ring, the SwiGLU in the GEMM's epilogue, no reduce launch (C0's gate/up
  // step 15.75 -> 15.0 us).  The F8X2 form measured slower that way (14.7
  // -> 16.0 us) and keeps two splits.
  if (bk == BK_MXFP4 && ak == AK_F16 && is_dual(epi) && kt <= 16 && tiles <= kDeepMaxWgs) return 1;
  int s = 1;
  // MXFP4 gate/up GEMMs take the deep split policy too: C2's as 2 deep
  // splits of 56 stages against 4 two-slot splits of 28 measured 72.4 ->
  // 69.7 us (fused MLP, stream) and 67.4 -> 66.3 us (scaled) once the deep
  // ring's scale staging went by DMA (2-3 us slower before).  MXFP4 store
  // GEMMs keep the 2-slot policy.
  if (deep_format(ak, bk) && (bk != BK_MXFP4 || is_dual(epi)) && kt % 4 == 0) {
    while (tiles * 2 * s <= kDeepMaxWgs && kt % (8 * s) == 0 && kt / (2 * s) >= 8) s *= 2;
    if (tiles * s >= 192) return s;  // else too few workgroups: the 2-slot policy below
    s = 1;
  }
  while (tiles * s < 384 && kt % (2 * s) == 0 && kt / (2 * s) >= 8) s *= 2;
  return s;
}

size_t gemm_q_ws_bytes(int ak, int bk, int epi, int m, int n, int k) {
  const int s = gemm_q_splits(ak, bk, epi, m, n, k);
  return s > 1 ? (size_t)s * (is_dual(epi) ? 2 : 1) * m * n * 4 : 0;
}

bool gemm_q_ok(int ak, int bk, int epi, int m, int n, int k) {
  if (m <= 0 || n <= 0 || k <= 0 || k % stage_k(ak)) return false;
  if (n % 64) return false;
  if (ak == AK_I8)
    return bk == BK_I8 && (epi == EPI_SWIGLU_F32 || epi == EPI_STORE_F16 || epi == EPI_STORE_F32 || epi == EPI_STORE_I32);
  if (ak == AK_F8X2)
    return (bk == BK_MXFP4 || bk == BK_E4M3 || bk == BK_E5M2) &&
           (epi == EPI_SWIGLU_F8X2 || epi == EPI_STORE_F16 || epi == EPI_STORE_F32);
  return bk != BK_I8 && epi != EPI_STORE_I32 && epi != EPI_SWIGLU_F32 && epi != EPI_SWIGLU_F8X2;
}

#define MXQ_EPIS(AK, BK)                                                                            \
  switch (epi) {                                                                                    \
    case EPI_STORE_F32: return launch_wn<AK, BK, EPI_STORE_F32>(g, s, st);                          \
    case EPI_STORE_F16: return launch_wn<AK, BK, EPI_STORE_F16>(g, s, st);                          \
    case EPI_SWIGLU_F16: return launch_wn<AK, BK, EPI_SWIGLU_F16>(g, s, st);                        \
    case EPI_SWIGLU_HALF: return launch_wn<AK, BK, EPI_SWIGLU_HALF>(g, s, st);                      \
    default: return hipErrorInvalidValue;                                                           \
  }

// MoE form: MXFP4 weights, f16 activations, SwiGLU (mid f16) or f16 store.
hipError_t launch_gemm_q_grouped(int epi, const QGemmArgs& g, const GroupTable& gt, int groups, hipStream_t st) {
  if (groups < 1 || groups > kMaxGroups || !gemm_q_ok(AK_F16, BK_MXFP4, epi, g.m, g.n, g.k)) return hipErrorInvalidValue;
  switch (epi) {
    case EPI_SWIGLU_F16: return launch_q_grouped<AK_F16, BK_MXFP4, EPI_SWIGLU_F16, 2>(g, gt, groups, st);
    case EPI_STORE_F16:
      return g.n % 128 == 0 ? launch_q_grouped<AK_F16, BK_MXFP4, EPI_STORE_F16, 2>(g, gt, groups, st)
                            : launch_q_grouped<AK_F16, BK_MXFP4, EPI_STORE_F16, 1>(g, gt, groups, st);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_gemm_q(int ak, int bk, int epi, const QGemmArgs& g, hipStream_t st) {
  if (!gemm_q_ok(ak, bk, epi, g.m, g.n, g.k)) return hipErrorInvalidValue;
  // few tiles (C0): one small tile per CU, operands requested up front
  // (its scale loads are dwords: planes at a 4-byte boundary)
  if (ak == AK_F16 && bk == BK_MXFP4 && small_gemm_ok(epi, g.m, g.n, g.k) &&
      ((reinterpret_cast<uintptr_t>(g.s0) | reinterpret_cast<uintptr_t>(g.s1)) & 3u) == 0)
    return launch_small_gemm(epi, g, st);
  // about one 64 x 64-channel gate/up tile per CU over a long K (C2): K
  // split between the waves of a workgroup, no split-K partials
  if (bk == BK_MXFP4 && kq_gemm_ok(ak, epi, g.m, g.n, g.k) &&
      ((reinterpret_cast<uintptr_t>(g.a) | reinterpret_cast<uintptr_t>(g.b0) | reinterpret_cast<uintptr_t>(g.b1)) & 15u) == 0 &&
      ((reinterpret_cast<uintptr_t>(g.s0) | reinterpret_cast<uintptr_t>(g.s1) |
        (ak == AK_F8X2 ? reinterpret_cast<uintptr_t>(g.a_e8) : 0)) & 3u) == 0)
    return launch_kq_gemm(ak, epi, g, st);
  const int s = gemm_q_splits(ak, bk, epi, g.m, g.n, g.k);
  if (s > 1 && !g.ws) return hipErrorInvalidValue;
  if (ak == AK_I8) {
    switch (epi) {
      case EPI_SWIGLU_F32: return launch_wn<AK_I8, BK_I8, EPI_SWIGLU_F32>(g, s, st);
      case EPI_STORE_F16: return launch_wn<AK_I8, BK_I8, EPI_STORE_F16>(g, s, st);
      case EPI_STORE_F32: return launch_wn<AK_I8, BK_I8, EPI_STORE_F32>(g, s, st);
      case EPI_STORE_I32: return launch_wn<AK_I8, BK_I8, EPI_STORE_I32>(g, s, st);
      default: return hipErrorInvalidValue;
    }
  }
  if (ak == AK_F8X2) {  // MXFP4 or FP8 weights (gemm_q_ok)
#define MXQ_F8X2(BK)                                                                                \
    switch (epi) {                                                                                  \
      case EPI_SWIGLU_F8X2: return launch_wn<AK_F8X2, BK, EPI_SWIGLU_F8X2>(g, s, st);              \
      case EPI_STORE_F16: return launch_wn<AK_F8X2, BK, EPI_STORE_F16>(g, s, st);                  \
      case EPI_STORE_F32: return launch_wn<AK_F8X2, BK, EPI_STORE_F32>(g, s, st);                  \
      default: return hipErrorInvalidValue;                                                         \
    }
    if (bk == BK_MXFP4) { MXQ_F8X2(BK_MXFP4) }
    if (bk == BK_E4M3) { MXQ_F8X2(BK_E4M3) }
    MXQ_F8X2(BK_E5M2)
#undef MXQ_F8X2
  }
  if (ak == AK_F32) {
    if (epi != EPI_STORE_F32 && epi != EPI_STORE_F16) return hipErrorInvalidValue;
    switch (bk) {
      case BK_F16:
        return epi == EPI_STORE_F32 ? launch_wn<AK_F32, BK_F16, EPI_STORE_F32>(g, s, st)
                                    : launch_wn<AK_F32, BK_F16, EPI_STORE_F16>(g, s, st);
      case BK_MXFP4:
        return epi == EPI_STORE_F32 ? launch_wn<AK_F32, BK_MXFP4, EPI_STORE_F32>(g, s, st)
                                    : launch_wn<AK_F32, BK_MXFP4, EPI_STORE_F16>(g, s, st);
      default: return hipErrorInvalidValue;
    }
  }
  switch (bk) {
    case BK_F16: MXQ_EPIS(AK_F16, BK_F16)
    case BK_MXFP4: MXQ_EPIS(AK_F16, BK_MXFP4)
    case BK_E4M3: MXQ_EPIS(AK_F16, BK_E4M3)
    case BK_E5M2: MXQ_EPIS(AK_F16, BK_E5M2)
    case BK_INT8: MXQ_EPIS(AK_F16, BK_INT8)
    case BK_INT4G32: MXQ_EPIS(AK_F16, BK_INT4G32)
  }
  return hipErrorInvalidValue;
}
#undef MXQ_EPIS

}  // namespace mx
