// mx_gemm_fp4_v3.hip - the W4A4 prefill GEMM at full tile size (BASELINE
// configs[4]), plus the one-launch prologue that prepares its operands.
//
// GEMM: 256 x 256 workgroup tile, K stage 128, 4 wave64s each owning a
// 128 x 128 accumulator tile (4 x 4 blocks of v_mfma_scale_f32_32x32x64 with
// FP4 operands, 256 AGPRs).  Operands stream straight from global memory
// into a 2-slot LDS ring with global_load_lds_dwordx4 (no register staging):
// per stage each wave moves 4 A and 4 B 1 KB fragments, laid out
// "fragment-major" (the 16 bytes lane l feeds to one MFMA at offset 16*l),
// so every ds_read_b128 is contiguous and conflict-free.  Stage loop: wait
// for this stage's loads, barrier, read all of the stage's fragments and
// scales into VGPRs, issue the next stage's loads into the other slot, then
// 32 MFMAs - the next stage's memory latency hides behind ~1000 MFMA cycles.
//
// Scales are stage-major ([K/128][rows_pad] dwords, see mx_internal.h): the
// 256 rows' scales of a stage are one contiguous 1 KB, fetched by a single
// DMA instruction.  (With the reference [rows][K/32] layout every lane
// fetched 4 bytes from its own row - 1024 tiny L2 requests per stage and
// workgroup, twice the data requests; rocprof showed the GEMM limited by
// them.)  Each lane then shifts its row's dword by 8*(lane/32) so a uniform
// opsel (byte 0 for K-step 0, byte 2 for K-step 1) selects its own block.
//
// Epilogues: DUAL=false stores f16 C; DUAL=true (B rows 0-127 gate, 128-255
// the same up channels) forms silu(g)*u and re-quantizes it to MXFP4 along
// the channel axis through LDS, writing stage-major scales for the down GEMM.
#include "mx_device.h"
#include "mx_internal.h"

namespace mx {

constexpr int kM = 256, kKS = 128;           // tile M, K per stage
constexpr int kFrag = 16;                    // A (or B) fragments per stage
constexpr int kSlotData = 2 * kFrag * 1024;  // 32 KB of operand fragments
constexpr int kSlot = kSlotData + 2048;      // + 1 KB A scales + 1 KB B scales
constexpr int kMidStride = 33;

__device__ __forceinline__ int xcd_tile(int bid, int nblocks) {
  if (nblocks % 8 != 0) return bid;  // 8 XCDs take consecutive ids round robin
  const int per = nblocks / 8;
  return (bid % 8) * per + bid / 8;
}

template <bool DUAL>
__global__ __launch_bounds__(256, 1) void k_gemm_fp4_v3(Fp4GemmArgs g) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave & 1, wn = wave >> 1;
  const int M = g.m, K = g.k;
  const int MT = (M + kM - 1) / kM;
  const int NT = DUAL ? g.n / 128 : g.n / 256;
  const size_t Mpad = stage_major_rows(M);
  const size_t NB = (size_t)g.n;  // rows of each B scale plane

  const int tile = xcd_tile(blockIdx.x, MT * NT);
  const int group_sz = 8 * MT;
  const int grp = tile / group_sz, in_grp = tile % group_sz;
  const int nt_base = grp * 8;
  const int gw = min(8, NT - nt_base);
  const int mt = in_grp / gw, nt = nt_base + in_grp % gw;
  const int m0 = mt * kM;
  const size_t row_bytes = (size_t)K / 2;

  // Operand fragments this wave streams (A f = 4*wave+u: block f/2,
  // k-step f%2; lane l: row 32*block + l%32, bytes 32*kstep + 16*(l/32)).
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
  // Scale DMA: wave 0 moves the A tile's 256 row dwords, wave 1 the B
  // tile's (lane l: rows 4l..4l+3 of the tile; DUAL: lanes 0-31 gate rows,
  // 32-63 up rows).
  const uint8_t* s_src;
  if (wave == 0) {
    s_src = g.as + (size_t)(m0 + 4 * lane) * 4;
  } else if (DUAL) {
    s_src = (lane < 32 ? g.s0 : g.s1) + (size_t)(nt * 128 + 4 * (lane & 31)) * 4;
  } else {
    s_src = g.s0 + (size_t)(nt * 256 + 4 * lane) * 4;
  }
  const size_t s_stage = wave == 0 ? Mpad * 4 : NB * 4;  // bytes per stage in the plane

  int bfrag[4];
#pragma unroll
  for (int j = 0; j < 4; j++) {
    if (DUAL) bfrag[j] = j < 2 ? wn * 2 + (j & 1) : 4 + wn * 2 + (j & 1);
    else bfrag[j] = wn * 4 + j;
  }
  const int shift = 8 * (lane >> 5);

  v16f acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int j = 0; j < 4; j++)
#pragma unroll
      for (int v = 0; v < 16; v++) acc[i][j][v] = 0.0f;

  const int KT = K / kKS;
#define MX_ISSUE(kt, slot)                                                                           \
  {                                                                                                  \
    const size_t koff_ = (size_t)(kt) * (kKS / 2);                                                   \
    uint8_t* sb_ = smem + (slot) * kSlot;                                                            \
    _Pragma("unroll") for (int u = 0; u < 4; u++)                                                    \
      __builtin_amdgcn_global_load_lds(a_src[u] + koff_, sb_ + (wave * 4 + u) * 1024, 16, 0, 0);     \
    _Pragma("unroll") for (int u = 0; u < 4; u++)                                                    \
      __builtin_amdgcn_global_load_lds(b_src[u] + koff_, sb_ + (kFrag + wave * 4 + u) * 1024, 16, 0, 0); \
    if (wave < 2)                                                                                    \
      __builtin_amdgcn_global_load_lds(s_src + (size_t)(kt) * s_stage, sb_ + kSlotData + wave * 1024, \
                                       16, 0, 0);                                                    \
  }
  MX_ISSUE(0, 0)
  for (int kt = 0; kt < KT; kt++) {
    const int slot = kt & 1;
    __builtin_amdgcn_s_waitcnt(0);  // this wave's loads for stage kt have landed
    __syncthreads();                // ... and every other wave's
    const uint8_t* base = smem + slot * kSlot;
    v4i af[2][4], bf[2][4];
    uint32_t sa[4], sbv[4];
#pragma unroll
    for (int ks = 0; ks < 2; ks++) {
#pragma unroll
      for (int i = 0; i < 4; i++)
        af[ks][i] = *reinterpret_cast<const v4i*>(base + (((wm * 4 + i) * 2 + ks) * 64 + lane) * 16);
#pragma unroll
      for (int j = 0; j < 4; j++)
        bf[ks][j] = *reinterpret_cast<const v4i*>(base + ((kFrag + bfrag[j] * 2 + ks) * 64 + lane) * 16);
    }
#pragma unroll
    for (int i = 0; i < 4; i++)
      sa[i] = *reinterpret_cast<const uint32_t*>(base + kSlotData + (wm * 128 + i * 32 + (lane & 31)) * 4) >> shift;
#pragma unroll
    for (int j = 0; j < 4; j++)
      sbv[j] = *reinterpret_cast<const uint32_t*>(base + kSlotData + 1024 + (bfrag[j] * 32 + (lane & 31)) * 4) >> shift;
    // Next stage; the last iteration re-reads its own stage into the idle
    // slot so that the issue stays unconditional.
    MX_ISSUE(kt + 1 < KT ? kt + 1 : kt, slot ^ 1)
    __builtin_amdgcn_sched_barrier(0);  // keep the loads ahead of the MFMAs
#pragma unroll
    for (int ks = 0; ks < 2; ks++)
#pragma unroll
      for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) {
          if (ks == 0)
            acc[i][j] = mfma_fp4_32x32x64<0, 0>(af[0][i], bf[0][j], acc[i][j], (int)sa[i], (int)sbv[j]);
          else
            acc[i][j] = mfma_fp4_32x32x64<2, 2>(af[1][i], bf[1][j], acc[i][j], (int)sa[i], (int)sbv[j]);
        }
  }
#undef MX_ISSUE
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();

  if (!DUAL) {
    uint16_t* c = reinterpret_cast<uint16_t*>(g.c);
    uint64_t nanm[4] = {0u, 0u, 0u, 0u};  // bit j * 16 + v of word i: element is NaN
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const int col = nt * 256 + (wn * 4 + j) * 32 + (lane & 31);
#pragma unroll
        for (int v = 0; v < 16; v++) {
          const int row = m0 + wm * 128 + i * 32 + acc32_row(lane, v);
          const float x0 = acc[i][j][v];
          nanm[i] |= (uint64_t)(x0 != x0) << (j * 16 + v);
          if (row < M) c[(size_t)row * g.n + col] = f32_to_f16_bits(x0);
        }
      }
    // NaN outputs (E8M0 byte 255 in a down-weight scale: NaN to the scaled
    // MFMA, +inf to the reference) recomputed with the reference's
    // dequantization (rare; one wave-uniform test).
    if (__builtin_expect(__ballot((nanm[0] | nanm[1] | nanm[2] | nanm[3]) != 0) != 0, 0)) {
#pragma nounroll
      for (int e = 0; e < 256; e++) {
        const int i = e >> 6, j = (e >> 4) & 3, v = e & 15;
        if (!((nanm[i] >> (j * 16 + v)) & 1u)) continue;
        const int row = m0 + wm * 128 + i * 32 + acc32_row(lane, v);
        const int col = nt * 256 + (wn * 4 + j) * 32 + (lane & 31);
        if (row < M)
          c[(size_t)row * g.n + col] = f32_to_f16_bits(
              ref_dot_mxfp4_mxfp4(g.a, g.as, stage_major_rows(M), row, g.b0, g.s0, (size_t)g.n, col, g.k));
      }
    }
    return;
  }
  // mid = silu(gate) * up, re-quantized along channels; stage-major scales
  // of the mid plane (rows = M padded, stages = n / 128).
  float* mid = reinterpret_cast<float*>(smem) + wave * (64 * kMidStride);
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
        const int blk = chan0 / 32;  // stage blk/4, byte blk%4
        g.cs[((size_t)(blk >> 2) * Mpad + row) * 4 + (blk & 3)] = (uint8_t)sb;
      }
      __syncthreads();
    }
  }
}

hipError_t launch_gemm_fp4_v3(int dual, const Fp4GemmArgs& g, hipStream_t st) {
  static bool attr_set = false;
  const int lds = 2 * kSlot;  // 68 KB
  if (!attr_set) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(k_gemm_fp4_v3<true>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, lds);
    if (e == hipSuccess)
      e = hipFuncSetAttribute(reinterpret_cast<const void*>(k_gemm_fp4_v3<false>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, lds);
    if (e != hipSuccess) return e;
    attr_set = true;
  }
  const int MT = (g.m + kM - 1) / kM;
  const int NT = dual ? g.n / 128 : g.n / 256;
  if (dual) hipLaunchKernelGGL(k_gemm_fp4_v3<true>, dim3(MT * NT), dim3(256), lds, st, g);
  else hipLaunchKernelGGL(k_gemm_fp4_v3<false>, dim3(MT * NT), dim3(256), lds, st, g);
  return hipGetLastError();
}

bool w4a4_stage_major_ok(int hidden, int inter) {
  // gate/up: N = inter in 128-column tiles; down: N = hidden in 256-column
  // tiles; K of both a multiple of 128.
  return inter % 128 == 0 && hidden % 256 == 0 && hidden % 128 == 0;
}

// ---------------------------------------------------------------------------
// Prologue: blocks [0, qb) quantize x (one thread per 32-element block, E8M0
// per BASELINE, stage-major scales); the rest convert the three weight scale
// planes from [rows][K/32] to stage-major (one 64 x 32 tile per block for
// large planes, one dword per thread for small ones).
__global__ void k_w4a4_prologue(W4A4Prologue p, unsigned qb, int tiled) {
  const size_t Tpad = stage_major_rows(p.t);
  if (blockIdx.x < qb) {
    const size_t b = (size_t)blockIdx.x * blockDim.x + threadIdx.x;  // block index
    const size_t kb = (size_t)p.h / 32;
    if (b >= (size_t)p.t * kb) return;
    const size_t row = b / kb, blk = b % kb;
    float v[32];
    const uint4* src = reinterpret_cast<const uint4*>(p.x + b * 32);
#pragma unroll
    for (int q = 0; q < 4; q++) {
      const uint4 w = src[q];
      const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
      for (int t = 0; t < 4; t++) {
        v[q * 8 + 2 * t] = f16_bits_to_f32((uint16_t)(ws[t] & 0xffffu));
        v[q * 8 + 2 * t + 1] = f16_bits_to_f32((uint16_t)(ws[t] >> 16));
      }
    }
    uint32_t amax = 0;
#pragma unroll
    for (int j = 0; j < 32; j++) amax = max(amax, abs_bits(v[j]));
    const uint32_t sb = mxfp4_scale_byte(amax);
    uint4 o = make_uint4(0, 0, 0, 0);
    if (sb != 255u) {
      o.x = fp4x8_from_f32(v + 0, sb);
      o.y = fp4x8_from_f32(v + 8, sb);
      o.z = fp4x8_from_f32(v + 16, sb);
      o.w = fp4x8_from_f32(v + 24, sb);
    }
    if (p.xq_sm)
      *reinterpret_cast<uint4*>(p.xq + (((blk >> 2) * Tpad + row) << 6) + ((blk & 3) << 4)) = o;
    else
      reinterpret_cast<uint4*>(p.xq)[b] = o;
    p.xs[((blk >> 2) * Tpad + row) * 4 + (blk & 3)] = (uint8_t)sb;
    return;
  }
  if (!tiled) {  // small planes: one thread per (matrix, stage, row) dword
    size_t it = (size_t)(blockIdx.x - qb) * blockDim.x + threadIdx.x;
    const size_t gate_items = (size_t)p.i * (p.h / 128), down_items = (size_t)p.h * (p.i / 128);
    const uint8_t* src;
    uint8_t* dst;
    size_t rows, stages;
    if (it < 2 * gate_items) {
      const bool up = it >= gate_items;
      if (up) it -= gate_items;
      src = up ? p.su : p.sg;
      dst = up ? p.su2 : p.sg2;
      rows = p.i;
      stages = p.h / 128;
    } else {
      it -= 2 * gate_items;
      if (it >= down_items) return;
      src = p.sd;
      dst = p.sd2;
      rows = p.h;
      stages = p.i / 128;
    }
    const size_t row = it % rows, stage = it / rows;  // consecutive threads: consecutive rows
    const uint32_t v = *reinterpret_cast<const uint32_t*>(src + row * (stages * 4) + stage * 4);
    *reinterpret_cast<uint32_t*>(dst + (stage * rows + row) * 4) = v;
    return;
  }
  // scale-plane conversion, one 64-row x 32-stage tile per workgroup:
  // [rows][stages] dwords (a row's four E8M0 bytes of one 128-K stage) ->
  // [stages][rows], transposed through LDS so that reads (128 bytes of a
  // row) and writes (256 bytes of a plane) are both contiguous.
  __shared__ uint32_t tile[64][33];
  unsigned t = blockIdx.x - qb;
  const int gs = p.h / 128, ds = p.i / 128;  // stages of gate/up and of down
  const unsigned gr = (p.i + 63) / 64, gc = (gs + 31) / 32, dr = (p.h + 63) / 64, dc = (ds + 31) / 32;
  const uint32_t* src;
  uint32_t* dst;
  int rows, stages;
  unsigned nr;
  if (t < 2 * gr * gc) {
    const bool up = t >= gr * gc;
    if (up) t -= gr * gc;
    src = reinterpret_cast<const uint32_t*>(up ? p.su : p.sg);
    dst = reinterpret_cast<uint32_t*>(up ? p.su2 : p.sg2);
    rows = p.i;
    stages = gs;
    nr = gr;
  } else {
    t -= 2 * gr * gc;
    if (t >= dr * dc) return;  // workgroup-uniform
    src = reinterpret_cast<const uint32_t*>(p.sd);
    dst = reinterpret_cast<uint32_t*>(p.sd2);
    rows = p.h;
    stages = ds;
    nr = dr;
  }
  const int row0 = (int)(t % nr) * 64, s0 = (int)(t / nr) * 32;
#pragma unroll
  for (int q = 0; q < 8; q++) {  // consecutive threads: consecutive stages of a row
    const int idx = q * 256 + (int)threadIdx.x, r = idx / 32, c = idx % 32;
    if (row0 + r < rows && s0 + c < stages) tile[r][c] = src[(size_t)(row0 + r) * stages + s0 + c];
  }
  __syncthreads();
#pragma unroll
  for (int q = 0; q < 8; q++) {  // consecutive threads: consecutive rows of a plane
    const int idx = q * 256 + (int)threadIdx.x, c = idx / 64, r = idx % 64;
    if (row0 + r < rows && s0 + c < stages) dst[(size_t)(s0 + c) * rows + row0 + r] = tile[r][c];
  }
}

hipError_t launch_w4a4_prologue(const W4A4Prologue& p, hipStream_t st) {
  const size_t qitems = (size_t)p.t * (p.h / 32);
  const unsigned qb = (unsigned)((qitems + 255) / 256);
  const unsigned gs = p.h / 128, ds = p.i / 128;
  const size_t sitems = 2 * (size_t)p.i * gs + (size_t)p.h * ds;
  // the tiled transpose pays off from ~1M scale dwords (C4: 5.5M); below
  // that the per-dword copy launches fewer idle lanes
  const int tiled = sitems >= ((size_t)1 << 20);
  const unsigned sbk = tiled ? 2 * ((p.i + 63) / 64) * ((gs + 31) / 32) + ((p.h + 63) / 64) * ((ds + 31) / 32)
                             : (unsigned)((sitems + 255) / 256);
  hipLaunchKernelGGL(k_w4a4_prologue, dim3(qb + sbk), dim3(256), 0, st, p, qb, tiled);
  return hipGetLastError();
}

}  // namespace mx
