// mx_api.cpp - the C ABI of libmxfp4hip (declared in include/mxfp4hip.h).
//
// Owns the device, one HIP stream, scratch memory and every launch; checks
// arguments the way runMLPBenchmark does (main.swift:592-597) and maps
// failures onto the reference's ProbeError cases (main.swift:5-38).
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <algorithm>
#include <functional>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/mxfp4hip.h"
#include "mx_internal.h"

struct mx_ctx {
  int device = 0;
  hipStream_t own_stream = nullptr;
  hipStream_t stream = nullptr;
  std::string err;
  char name[256] = {0};
  int cus = 0, clock_mhz = 0;
  // scratch owned by the context (grown on demand)
  void* ws = nullptr;
  size_t ws_bytes = 0;
  hipEvent_t t0 = nullptr, t1 = nullptr;  // mx_timer_start / mx_timer_stop
};

// Scratch of mx_mlp_forward_noalloc: one static device array, which every
// GPU the library runs on holds until the process ends.  In host code the
// array's name is a host-side stand-in, never a device address: the address
// comes from hipGetSymbolAddress, once per device at mx_create with that
// device current, and only that address is handed to kernels.
static __device__ __align__(256) uint8_t scratch[MX_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};            // device address of `scratch`, per device
hipError_t g_scratch_err[kMaxDevices] = {};       // hipGetSymbolAddress's failure, if any

int set_err(mx_ctx* c, int code, const char* fmt, ...) {
  if (c) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    c->err = buf;
  }
  return code;
}

#define MX_HIP(ctx, expr)                                                                 \
  do {                                                                                    \
    hipError_t e_ = (expr);                                                               \
    if (e_ != hipSuccess)                                                                 \
      return set_err(ctx, MX_EGPU, "%s failed: %s", #expr, hipGetErrorString(e_));        \
  } while (0)

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int ensure_ws(mx_ctx* c, size_t bytes) {
  if (bytes <= c->ws_bytes) return MX_OK;
  // Growing frees the old workspace, which a graph captured earlier may
  // still point at, and synchronises, which a capturing stream refuses.
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(c->stream, &cap) == hipSuccess && cap != hipStreamCaptureStatusNone)
    return set_err(c, MX_EINVAL,
                   "The workspace must grow to %zu bytes, which is not allowed while the stream is being "
                   "captured: run one forward of the largest shape before capturing.", bytes);
  if (c->ws) {
    MX_HIP(c, hipStreamSynchronize(c->stream));
    MX_HIP(c, hipFree(c->ws));
    c->ws = nullptr;
    c->ws_bytes = 0;
  }
  size_t want = (bytes + (1u << 20) - 1) & ~(size_t)((1u << 20) - 1);
  if (hipMalloc(&c->ws, want) != hipSuccess) {
    c->ws = nullptr;
    return set_err(c, MX_ENOMEM, "Could not create device buffer workspace (%zu bytes).", want);
  }
  c->ws_bytes = want;
  return MX_OK;
}

size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// Split-K partial bytes of a GEMM that the 64-K-stage family takes (0 when
// the shape goes to the K-step-32 kernel, which does not split K).
size_t q_ws(int ak, int bk, int epi, int m, int n, int k) {
  return mx::gemm_q_ok(ak, bk, epi, m, n, k) ? mx::gemm_q_ws_bytes(ak, bk, epi, m, n, k) : 0;
}

// One GEMM of an MLP: the 64-K-stage family when the shape fits it, else the
// K-step-32 kernel (any n, k % 32 == 0).
hipError_t launch_mlp_gemm(int ak, int bk, int epi, const mx::QGemmArgs& q, hipStream_t st) {
  if (mx::gemm_q_ok(ak, bk, epi, q.m, q.n, q.k)) return mx::launch_gemm_q(ak, bk, epi, q, st);
  mx::GemmArgs g{q.a, ak == mx::AK_F32 ? MX_DTYPE_F32 : MX_DTYPE_F16, q.b0, q.s0, q.b1, q.s1, q.c, q.m, q.n, q.k};
  return mx::launch_gemm_h(bk, epi, g, st);
}

// A forward pass as a list of launches (so the benchmark can time each).
struct Step {
  const char* name;
  std::function<hipError_t()> run;
};

int check_mlp_cfg(mx_ctx* c, int variant, const mx_mlp_config* cfg) {
  if (!cfg) return set_err(c, MX_EINVAL, "MLP config is null.");
  const long T = cfg->tokens, H = cfg->hidden, I = cfg->intermediate;
  if (T <= 0 || H <= 0 || I <= 0)
    return set_err(c, MX_EINVAL, "MLP sizes and iterations must be positive.");
  if (H % 16 || I % 16)
    return set_err(c, MX_EINVAL,
                   "MLP hidden and intermediate sizes must be multiples of 16 for packed FP4 weights.");
  if (H % 32 || I % 32)
    return set_err(c, MX_EINVAL, "MXFP4 rows need hidden and intermediate to be multiples of 32.");
  // The reference's MXFP4 rows need only % 32 (main.swift:1043); so do
  // FUSED, REFROW and DEQUANT.  The scaled-MFMA variant splits x and mid in
  // 64-K groups.
  if (variant == MX_MLP_SCALED && (H % 64 || I % 64))
    return set_err(c, MX_EINVAL, "The scaled variant needs hidden and intermediate to be multiples of 64.");
  if (variant == MX_MLP_W4A4 && (H % 128 || I % 128))
    return set_err(c, MX_EINVAL, "W4A4 needs hidden and intermediate to be multiples of 128.");
  if (variant < MX_MLP_FUSED || variant > MX_MLP_SCALED)
    return set_err(c, MX_EINVAL, "Unknown MLP variant %d.", variant);
  return MX_OK;
}

bool gemv_ok(const mx_mlp_config* cfg) {
  // decode GEMV: <= 16 tokens, K multiples of 128 up to 16384, and the
  // activations plus one row group's scales fit the workgroup's LDS
  return cfg->tokens <= 16 && cfg->hidden % 128 == 0 && cfg->intermediate % 128 == 0 &&
         cfg->hidden <= 16384 && cfg->intermediate <= 16384 &&
         mx::gemv_lds_need((int)cfg->tokens, (int)cfg->hidden) <= 160 * 1024 &&
         mx::gemv_lds_need((int)cfg->tokens, (int)cfg->intermediate) <= 160 * 1024;
}

// Which kernels a forward runs (shared by the launcher and the name query).
// PATH_GEMM_H: the fused (or reference-row) MLP at shapes the 64-K-stage
// family does not take (hidden or intermediate % 64 != 0): both GEMMs on the
// K-step-32 kernel.
// PATH_W4A4: stage-major scale planes (the 256 x 256 kernels, whose down
// epilogue recomputes byte-255 outputs itself); PATH_W4A4_REF: the
// reference-layout kernels plus a separate byte-255 pass.
enum MlpPath { PATH_GEMV, PATH_GEMM_Q, PATH_REFROW, PATH_DEQUANT, PATH_W4A4, PATH_SCALED, PATH_GEMM_H,
               PATH_REFROW_H, PATH_W4A4_REF };

bool q_shapes(const mx_mlp_config* cfg) { return cfg->hidden % 64 == 0 && cfg->intermediate % 64 == 0; }

MlpPath mlp_path(int variant, const mx_mlp_config* cfg) {
  switch (variant) {
    case MX_MLP_FUSED: return gemv_ok(cfg) ? PATH_GEMV : q_shapes(cfg) ? PATH_GEMM_Q : PATH_GEMM_H;
    case MX_MLP_REFROW: return q_shapes(cfg) ? PATH_REFROW : PATH_REFROW_H;
    case MX_MLP_DEQUANT: return PATH_DEQUANT;
    case MX_MLP_SCALED: return PATH_SCALED;
    default: return mx::w4a4_stage_major_ok((int)cfg->hidden, (int)cfg->intermediate) ? PATH_W4A4 : PATH_W4A4_REF;
  }
}

// Scratch layout for one variant; returns bytes needed.
struct MlpScratch {
  size_t mid = 0, gate = 0, up = 0, wg = 0, wu = 0, wd = 0, xq = 0, xs = 0, mq = 0, ms = 0;
  size_t sg = 0, su = 0, sd = 0;  // stage-major weight scale copies (W4A4)
  size_t qws = 0;                 // split-K partials of the small-M GEMMs
  size_t xe = 0, me = 0;          // F8X2 scale pairs of x and mid (MX_MLP_SCALED)
  size_t total = 0;
};

MlpScratch plan_scratch(int variant, const mx_mlp_config* cfg) {
  const size_t T = cfg->tokens, H = cfg->hidden, I = cfg->intermediate;
  MlpScratch s;
  size_t off = 0;
  auto take = [&](size_t bytes) { size_t o = off; off = align_up(off + bytes, 256); return o; };
  if (variant == MX_MLP_FUSED || variant == MX_MLP_REFROW) {
    s.mid = take(T * I * 2);
    const int e = variant == MX_MLP_REFROW ? mx::EPI_SWIGLU_HALF : mx::EPI_SWIGLU_F16;
    s.qws = take(std::max(q_ws(mx::AK_F16, mx::BK_MXFP4, e, (int)T, (int)I, (int)H),
                          q_ws(mx::AK_F16, mx::BK_MXFP4, mx::EPI_STORE_F32, (int)T, (int)H, (int)I)));
  } else if (variant == MX_MLP_SCALED) {
    s.xq = take(mx::f8x2_data_bytes(T, H));
    s.xe = take(mx::f8x2_e8_bytes(T, H));
    s.mq = take(mx::f8x2_data_bytes(T, I));
    s.me = take(mx::f8x2_e8_bytes(T, I));
    s.qws = take(std::max(mx::gemm_q_ws_bytes(mx::AK_F8X2, mx::BK_MXFP4, mx::EPI_SWIGLU_F8X2, (int)T, (int)I, (int)H),
                          mx::gemm_q_ws_bytes(mx::AK_F8X2, mx::BK_MXFP4, mx::EPI_STORE_F16, (int)T, (int)H, (int)I)));
  } else if (variant == MX_MLP_DEQUANT) {
    s.wg = take(I * H * 2);
    s.wu = take(I * H * 2);
    s.wd = take(H * I * 2);
    s.gate = take(T * I * 4);
    s.up = take(T * I * 4);
    s.mid = take(T * I * 4);
    s.qws = take(std::max(q_ws(mx::AK_F16, mx::BK_F16, mx::EPI_STORE_F32, (int)T, (int)I, (int)H),
                          q_ws(mx::AK_F32, mx::BK_F16, mx::EPI_STORE_F16, (int)T, (int)H, (int)I)));
  } else if (variant == MX_MLP_W4A4) {
    // stage-major codes (v6) take whole 256-row stage planes
    const size_t Tc = mx::w4a4_act_stage_major((int)T, (int)H, (int)I) ? mx::stage_major_rows(T) : T;
    s.xq = take(Tc * H / 2);
    s.mq = take(Tc * I / 2);
    if (mx::w4a4_stage_major_ok((int)H, (int)I)) {
      // stage-major planes: [K/128][rows rounded up to 256] dwords
      const size_t Tp = mx::stage_major_rows(T);
      s.xs = take(Tp * H / 32);
      s.ms = take(Tp * I / 32);
      s.sg = take(I * H / 32);
      s.su = take(I * H / 32);
      s.sd = take(H * I / 32);
      s.qws = take(std::max(mx::gemm_fp4_ws_bytes(1, (int)T, (int)I, (int)H),
                            mx::gemm_fp4_ws_bytes(0, (int)T, (int)H, (int)I)));
    } else {
      s.xs = take(T * H / 32);
      s.ms = take(T * I / 32);
    }
  }
  s.total = off;
  return s;
}

// fixed_ws: scratch memory of fixed_ws_bytes to use instead of the
// context's workspace (the allocation-free forward); nothing is allocated.
int build_mlp_steps(mx_ctx* c, int variant, const mx_mlp_config* cfg, const void* x,
                    const mx_mlp_weights* w, void* out, std::vector<Step>& steps, uint8_t* fixed_ws = nullptr,
                    size_t fixed_ws_bytes = 0) {
  int rc = check_mlp_cfg(c, variant, cfg);
  if (rc) return rc;
  if (!x || !w || !out) return set_err(c, MX_EINVAL, "MLP buffers must not be null.");
  const mx_qmatrix* mats[3] = {&w->gate, &w->up, &w->down};
  for (const mx_qmatrix* m : mats) {
    if (!m->data || !m->scales) return set_err(c, MX_EINVAL, "MLP weight buffers must not be null.");
    if (!aligned16(m->data)) return set_err(c, MX_EINVAL, "MXFP4 weight data must be 16-byte aligned.");
    if (reinterpret_cast<uintptr_t>(m->scales) & 3u)
      return set_err(c, MX_EINVAL, "MXFP4 scale planes must be 4-byte aligned.");
  }
  if (!aligned16(x) || !aligned16(out))
    return set_err(c, MX_EINVAL, "Activation and output buffers must be 16-byte aligned.");
  MlpScratch s = plan_scratch(variant, cfg);
  uint8_t* ws = fixed_ws;
  if (fixed_ws) {
    if (s.total > fixed_ws_bytes)
      return set_err(c, MX_EINVAL,
                     "This MLP needs %zu bytes of scratch; the allocation-free forward has %zu (use mx_mlp_forward).",
                     s.total, fixed_ws_bytes);
  } else {
    if ((rc = ensure_ws(c, s.total))) return rc;
    ws = static_cast<uint8_t*>(c->ws);
  }
  hipStream_t st = c->stream;
  const int T = cfg->tokens, H = cfg->hidden, I = cfg->intermediate;
  const uint8_t* wg = static_cast<const uint8_t*>(w->gate.data);
  const uint8_t* sg = static_cast<const uint8_t*>(w->gate.scales);
  const uint8_t* wu = static_cast<const uint8_t*>(w->up.data);
  const uint8_t* su = static_cast<const uint8_t*>(w->up.scales);
  const uint8_t* wd = static_cast<const uint8_t*>(w->down.data);
  const uint8_t* sd = static_cast<const uint8_t*>(w->down.scales);

  const MlpPath path = mlp_path(variant, cfg);
  if (path == PATH_GEMV) {
    uint16_t* mid = reinterpret_cast<uint16_t*>(ws + s.mid);
    mx::GemvArgs gu{static_cast<const uint16_t*>(x), wg, sg, wu, su, mid, T, I, H};
    mx::GemvArgs dn{mid, wd, sd, nullptr, nullptr, static_cast<uint16_t*>(out), T, H, I};
    steps.push_back({"gemv_mxfp4_gate_up_swiglu", [=] { return mx::launch_gemv_mxfp4(1, gu, st); }});
    steps.push_back({"gemv_mxfp4_down", [=] { return mx::launch_gemv_mxfp4(0, dn, st); }});
  } else if (path == PATH_GEMM_H || path == PATH_REFROW_H) {
    // hidden or intermediate % 64 != 0: both GEMMs on the K-step-32 kernel
    uint16_t* mid = reinterpret_cast<uint16_t*>(ws + s.mid);
    const bool ref = path == PATH_REFROW_H;
    const int e_gu = ref ? mx::EPI_SWIGLU_HALF : mx::EPI_SWIGLU_F16;
    const int e_dn = ref ? mx::EPI_STORE_F32 : mx::EPI_STORE_F16;
    mx::GemmArgs gu{x, MX_DTYPE_F16, wg, sg, wu, su, mid, T, I, H};
    mx::GemmArgs dn{mid, MX_DTYPE_F16, wd, sd, nullptr, nullptr, out, T, H, I};
    steps.push_back({ref ? "gemm_h_mxfp4_gate_up_swiglu_half" : "gemm_h_mxfp4_gate_up_swiglu",
                     [=] { return mx::launch_gemm_h(mx::BK_MXFP4, e_gu, gu, st); }});
    steps.push_back({ref ? "gemm_h_mxfp4_down_f32" : "gemm_h_mxfp4_down",
                     [=] { return mx::launch_gemm_h(mx::BK_MXFP4, e_dn, dn, st); }});
  } else if (path == PATH_GEMM_Q || path == PATH_REFROW) {
    uint16_t* mid = reinterpret_cast<uint16_t*>(ws + s.mid);
    const bool ref = path == PATH_REFROW;
    const int e_gu = ref ? mx::EPI_SWIGLU_HALF : mx::EPI_SWIGLU_F16;
    const int e_dn = ref ? mx::EPI_STORE_F32 : mx::EPI_STORE_F16;
    void* qws = ws + s.qws;
    mx::QGemmArgs gu{x, nullptr, wg, sg, wu, su, mid, qws, T, I, H, 0};
    gu.pf = wd;  // the down weights, pulled into L2 by the few-tile gate/up kernel
    gu.pf_rows = H;
    gu.pf_row_bytes = I / 2;
    mx::QGemmArgs dn{mid, nullptr, wd, sd, nullptr, nullptr, out, qws, T, H, I, 0};
    steps.push_back({ref ? "gemm_q_mxfp4_gate_up_swiglu_half" : "gemm_q_mxfp4_gate_up_swiglu",
                     [=] { return mx::launch_gemm_q(mx::AK_F16, mx::BK_MXFP4, e_gu, gu, st); }});
    steps.push_back({ref ? "gemm_q_mxfp4_down_f32" : "gemm_q_mxfp4_down",
                     [=] { return mx::launch_gemm_q(mx::AK_F16, mx::BK_MXFP4, e_dn, dn, st); }});
  } else if (path == PATH_SCALED) {
    // x and mid as two E4M3 terms with E8M0 pairs per 64 K (F8X2), both
    // GEMMs on v_mfma_scale_f32_32x32x64_f8f6f4 with the weights' FP4 codes
    // and E8M0 bytes as the B operand and its scales
    uint8_t* xq = ws + s.xq;
    uint32_t* xe = reinterpret_cast<uint32_t*>(ws + s.xe);
    uint8_t* mq = ws + s.mq;
    uint32_t* me = reinterpret_cast<uint32_t*>(ws + s.me);
    void* qws = ws + s.qws;
    mx::QGemmArgs gu{xq, nullptr, wg, sg, wu, su, mq, qws, T, I, H, 0, xe, me, static_cast<const uint16_t*>(x)};
    mx::QGemmArgs dn{mq, nullptr, wd, sd, nullptr, nullptr, out, qws, T, H, I, 0, me, nullptr};
    steps.push_back({"split_x_f8x2", [=] {
                       return mx::launch_split_f8x2(static_cast<const uint16_t*>(x), T, H, xq, xe, st);
                     }});
    steps.push_back({"gemm_q_scaled_gate_up_swiglu",
                     [=] { return mx::launch_gemm_q(mx::AK_F8X2, mx::BK_MXFP4, mx::EPI_SWIGLU_F8X2, gu, st); }});
    steps.push_back({"gemm_q_scaled_down",
                     [=] { return mx::launch_gemm_q(mx::AK_F8X2, mx::BK_MXFP4, mx::EPI_STORE_F16, dn, st); }});
  } else if (path == PATH_DEQUANT) {
    uint16_t* wg16 = reinterpret_cast<uint16_t*>(ws + s.wg);
    uint16_t* wu16 = reinterpret_cast<uint16_t*>(ws + s.wu);
    uint16_t* wd16 = reinterpret_cast<uint16_t*>(ws + s.wd);
    float* gate = reinterpret_cast<float*>(ws + s.gate);
    float* up = reinterpret_cast<float*>(ws + s.up);
    float* mid = reinterpret_cast<float*>(ws + s.mid);
    steps.push_back({"dequant_gate", [=] { return mx::launch_mxfp4_dequant_f16(wg, sg, wg16, I, H, st); }});
    steps.push_back({"dequant_up", [=] { return mx::launch_mxfp4_dequant_f16(wu, su, wu16, I, H, st); }});
    steps.push_back({"dequant_down", [=] { return mx::launch_mxfp4_dequant_f16(wd, sd, wd16, H, I, st); }});
    void* qws = ws + s.qws;
    mx::QGemmArgs gg{x, nullptr, wg16, nullptr, nullptr, nullptr, gate, qws, T, I, H, 0};
    mx::QGemmArgs gp{x, nullptr, wu16, nullptr, nullptr, nullptr, up, qws, T, I, H, 0};
    mx::QGemmArgs dn{mid, nullptr, wd16, nullptr, nullptr, nullptr, out, qws, T, H, I, 0};
    steps.push_back({"gemm_h_h_f_gate", [=] { return launch_mlp_gemm(mx::AK_F16, mx::BK_F16, mx::EPI_STORE_F32, gg, st); }});
    steps.push_back({"gemm_h_h_f_up", [=] { return launch_mlp_gemm(mx::AK_F16, mx::BK_F16, mx::EPI_STORE_F32, gp, st); }});
    steps.push_back({"swiglu_float", [=] { return mx::launch_swiglu(0, gate, up, mid, (size_t)T * I, st); }});
    steps.push_back({"gemm_f_h_down", [=] { return launch_mlp_gemm(mx::AK_F32, mx::BK_F16, mx::EPI_STORE_F16, dn, st); }});
  } else {  // W4A4
    uint8_t* xq = ws + s.xq;
    uint8_t* xs = ws + s.xs;
    uint8_t* mq = ws + s.mq;
    uint8_t* ms = ws + s.ms;
    if (mx::w4a4_stage_major_ok(H, I)) {
      // One prologue launch quantizes x and re-lays the three weight scale
      // planes stage-major; both GEMMs then fetch a stage's scales as one
      // contiguous block.
      uint8_t* sg2 = ws + s.sg;
      uint8_t* su2 = ws + s.su;
      uint8_t* sd2 = ws + s.sd;
      // Grids of whole tiles run both GEMMs on v6, which reads x and the mid
      // stage-major as well.
      const int asm_ = mx::w4a4_act_stage_major(T, H, I) ? 1 : 0;
      mx::W4A4Prologue pro{static_cast<const uint16_t*>(x), xq, xs, sg, su, sd, sg2, su2, sd2, T, H, I, asm_};
      float* part = reinterpret_cast<float*>(ws + s.qws);
      mx::Fp4GemmArgs gu{xq, xs, wg, sg2, wu, su2, mq, ms, T, I, H, 1 + asm_, part, mx::gemm_fp4_splits(1, T, I, H)};
      mx::Fp4GemmArgs dn{mq, ms, wd, sd2, nullptr, nullptr, out, nullptr, T, H, I, 1 + asm_, part,
                         mx::gemm_fp4_splits(0, T, H, I)};
      steps.push_back({"w4a4_prologue", [=] { return mx::launch_w4a4_prologue(pro, st); }});
      steps.push_back({"gemm_fp4_gate_up_swiglu_requant", [=] { return mx::launch_gemm_fp4(1, gu, st); }});
      steps.push_back({"gemm_fp4_down", [=] { return mx::launch_gemm_fp4(0, dn, st); }});
    } else {
      mx::Fp4GemmArgs gu{xq, xs, wg, sg, wu, su, mq, ms, T, I, H, 0};
      mx::Fp4GemmArgs dn{mq, ms, wd, sd, nullptr, nullptr, out, nullptr, T, H, I, 0};
      steps.push_back({"w4a4_prologue", [=] { return mx::launch_mxfp4_quantize(x, MX_DTYPE_F16, xq, xs, T, H, st); }});
      steps.push_back({"gemm_fp4_gate_up_swiglu_requant", [=] { return mx::launch_gemm_fp4(1, gu, st); }});
      steps.push_back({"gemm_fp4_down", [=] { return mx::launch_gemm_fp4(0, dn, st); }});
      steps.push_back({"w4a4_down_inf", [=] {
                         return mx::launch_w4a4_down_inf(wd, sd, mq, ms, 0, T, H, I, static_cast<uint16_t*>(out), st);
                       }});
    }
  }
  return MX_OK;
}

int run_steps(mx_ctx* c, const std::vector<Step>& steps) {
  for (const Step& s : steps) {
    hipError_t e = s.run();
    if (e != hipSuccess) return set_err(c, MX_EGPU, "launch of %s failed: %s", s.name, hipGetErrorString(e));
  }
  return MX_OK;
}

}  // namespace

// Context internals for the other translation units (mx_loader.cpp).
hipStream_t mx_ctx_stream(mx_ctx* c) { return c->stream; }
int mx_ctx_error(mx_ctx* c, int code, const char* message) { return set_err(c, code, "%s", message); }

// ===========================================================================
extern "C" {

const char* mx_status_string(int status) {
  switch (status) {
    case MX_OK: return "ok";
    case MX_EINVAL: return "invalid argument";
    case MX_ENODEV: return "No HIP device is available.";
    case MX_ENOKERNEL: return "The HIP code object does not contain the kernel for this device.";
    case MX_ENOMEM: return "Could not create device buffer.";
    case MX_EGPU: return "GPU execution failed.";
  }
  return "unknown status";
}

int mx_create(int device, mx_ctx** out) {
  if (!out) return MX_EINVAL;
  *out = nullptr;
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) return MX_ENODEV;
  if (device < 0 || device >= n) return MX_ENODEV;
  mx_ctx* c = new mx_ctx();
  c->device = device;
  if (hipSetDevice(device) != hipSuccess) { delete c; return MX_ENODEV; }
  hipDeviceProp_t p;
  if (hipGetDeviceProperties(&p, device) != hipSuccess) { delete c; return MX_ENODEV; }
  if (std::strncmp(p.gcnArchName, "gfx950", 6) != 0) { delete c; return MX_ENOKERNEL; }
  std::snprintf(c->name, sizeof c->name, "%s (%s)", p.name, p.gcnArchName);
  c->cus = p.multiProcessorCount;
  c->clock_mhz = p.clockRate / 1000;
  if (hipStreamCreateWithFlags(&c->own_stream, hipStreamNonBlocking) != hipSuccess) {
    delete c;
    return MX_EGPU;
  }
  if (device < kMaxDevices) {  // the allocation-free forward's scratch, once per device
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[device]) {
      void* p = nullptr;
      const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
      if (e == hipSuccess && p) g_scratch_ptr[device] = p;
      else {  // reported by mx_mlp_forward_noalloc; every other entry point works without it
        g_scratch_err[device] = e == hipSuccess ? hipErrorInvalidSymbol : e;
        (void)hipGetLastError();
      }
    }
  }
  c->stream = c->own_stream;
  *out = c;
  return MX_OK;
}

void mx_destroy(mx_ctx* c) {
  if (!c) return;
  (void)hipSetDevice(c->device);
  if (c->stream) (void)hipStreamSynchronize(c->stream);
  if (c->ws) (void)hipFree(c->ws);
  if (c->t0) (void)hipEventDestroy(c->t0);
  if (c->t1) (void)hipEventDestroy(c->t1);
  if (c->own_stream) (void)hipStreamDestroy(c->own_stream);
  delete c;
}

const char* mx_last_error(const mx_ctx* c) { return c ? c->err.c_str() : "null context"; }

int mx_device_info(mx_ctx* c, char* name_out, size_t name_len, int* cu_count, int* clock_mhz) {
  if (!c) return MX_EINVAL;
  if (name_out && name_len) std::snprintf(name_out, name_len, "%s", c->name);
  if (cu_count) *cu_count = c->cus;
  if (clock_mhz) *clock_mhz = c->clock_mhz;
  return MX_OK;
}

int mx_set_stream(mx_ctx* c, void* stream) {
  if (!c) return MX_EINVAL;
  c->stream = stream ? static_cast<hipStream_t>(stream) : c->own_stream;
  return MX_OK;
}

void* mx_get_stream(mx_ctx* c) { return c ? static_cast<void*>(c->stream) : nullptr; }

int mx_timer_start(mx_ctx* c) {
  if (!c) return MX_EINVAL;
  if (!c->t0) MX_HIP(c, hipEventCreate(&c->t0));
  if (!c->t1) MX_HIP(c, hipEventCreate(&c->t1));
  MX_HIP(c, hipEventRecord(c->t0, c->stream));
  return MX_OK;
}

int mx_timer_stop(mx_ctx* c, double* seconds_out) {
  if (!c || !seconds_out) return MX_EINVAL;
  if (!c->t0) return set_err(c, MX_EINVAL, "mx_timer_stop without mx_timer_start.");
  MX_HIP(c, hipEventRecord(c->t1, c->stream));
  MX_HIP(c, hipEventSynchronize(c->t1));
  float ms = 0.0f;
  MX_HIP(c, hipEventElapsedTime(&ms, c->t0, c->t1));
  *seconds_out = ms / 1000.0;
  return MX_OK;
}

int mx_sync(mx_ctx* c) {
  if (!c) return MX_EINVAL;
  MX_HIP(c, hipStreamSynchronize(c->stream));
  return MX_OK;
}

int mx_alloc(mx_ctx* c, size_t bytes, void** dptr) {
  if (!c || !dptr) return MX_EINVAL;
  *dptr = nullptr;
  if (bytes == 0) return set_err(c, MX_EINVAL, "allocation size must be positive.");
  if (hipMalloc(dptr, bytes) != hipSuccess) {
    *dptr = nullptr;
    (void)hipGetLastError();
    return set_err(c, MX_ENOMEM, "Could not create device buffer of %zu bytes.", bytes);
  }
  return MX_OK;
}

int mx_free(mx_ctx* c, void* dptr) {
  if (!c) return MX_EINVAL;
  if (dptr) MX_HIP(c, hipFree(dptr));
  return MX_OK;
}

int mx_upload(mx_ctx* c, void* dst, const void* src, size_t bytes) {
  if (!c || (!dst && bytes) || (!src && bytes)) return MX_EINVAL;
  MX_HIP(c, hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, c->stream));
  MX_HIP(c, hipStreamSynchronize(c->stream));
  return MX_OK;
}

int mx_download(mx_ctx* c, void* dst, const void* src, size_t bytes) {
  if (!c || (!dst && bytes) || (!src && bytes)) return MX_EINVAL;
  MX_HIP(c, hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, c->stream));
  MX_HIP(c, hipStreamSynchronize(c->stream));
  return MX_OK;
}

int mx_memset(mx_ctx* c, void* dst, int value, size_t bytes) {
  if (!c || (!dst && bytes)) return MX_EINVAL;
  MX_HIP(c, hipMemsetAsync(dst, value, bytes, c->stream));
  return MX_OK;
}

// ---- codecs ------------------------------------------------------------------
static int check_fmt(mx_ctx* c, int fmt) {
  if (fmt < MX_FMT_FP4_E2M1 || fmt > MX_FMT_FP8_E5M2)
    return set_err(c, MX_EINVAL, "Unknown packed numeric format %d.", fmt);
  return MX_OK;
}

int mx_pack(mx_ctx* c, int fmt, const float* in, size_t n, uint8_t* packed) {
  if (!c) return MX_EINVAL;
  if (int rc = check_fmt(c, fmt)) return rc;
  if (n == 0) return MX_OK;
  if (!in || !packed || !aligned16(in) || (reinterpret_cast<uintptr_t>(packed) & 3u))
    return set_err(c, MX_EINVAL, "pack buffers must be non-null, input 16-byte and output 4-byte aligned.");
  MX_HIP(c, mx::launch_pack(fmt, in, packed, n, c->stream));
  return MX_OK;
}

int mx_unpack(mx_ctx* c, int fmt, const uint8_t* packed, size_t n, float* out) {
  if (!c) return MX_EINVAL;
  if (int rc = check_fmt(c, fmt)) return rc;
  if (n == 0) return MX_OK;
  if (!packed || !out || !aligned16(out) || (reinterpret_cast<uintptr_t>(packed) & 3u))
    return set_err(c, MX_EINVAL, "unpack buffers must be non-null, output 16-byte and input 4-byte aligned.");
  MX_HIP(c, mx::launch_unpack(fmt, packed, out, n, c->stream));
  return MX_OK;
}

int mx_roundtrip(mx_ctx* c, int fmt, const float* host_in, size_t n, uint8_t* host_packed,
                 float* host_out) {
  if (!c) return MX_EINVAL;
  if (int rc = check_fmt(c, fmt)) return rc;
  if (n == 0) return MX_OK;
  if (!host_in || !host_packed || !host_out)
    return set_err(c, MX_EINVAL, "roundtrip buffers must not be null.");
  const size_t pbytes = fmt == MX_FMT_FP4_E2M1 ? (n + 1) / 2 : n;
  void *din = nullptr, *dp = nullptr, *dout = nullptr;
  int rc = MX_OK;
  if ((rc = mx_alloc(c, n * 4, &din)) || (rc = mx_alloc(c, align_up(pbytes, 16), &dp)) ||
      (rc = mx_alloc(c, n * 4, &dout))) {
    mx_free(c, din); mx_free(c, dp); mx_free(c, dout);
    return rc;
  }
  do {
    if ((rc = mx_upload(c, din, host_in, n * 4))) break;
    if ((rc = mx_memset(c, dp, 0, align_up(pbytes, 16)))) break;
    if ((rc = mx_pack(c, fmt, static_cast<float*>(din), n, static_cast<uint8_t*>(dp)))) break;
    if ((rc = mx_unpack(c, fmt, static_cast<uint8_t*>(dp), n, static_cast<float*>(dout)))) break;
    if ((rc = mx_download(c, host_packed, dp, pbytes))) break;
    if ((rc = mx_download(c, host_out, dout, n * 4))) break;
  } while (0);
  mx_free(c, din); mx_free(c, dp); mx_free(c, dout);
  return rc;
}

int mx_mxfp4_quantize(mx_ctx* c, const void* src, int src_dtype, int rows, int k, uint8_t* packed,
                      uint8_t* scales) {
  if (!c) return MX_EINVAL;
  if (rows <= 0 || k <= 0 || k % 32)
    return set_err(c, MX_EINVAL, "quantize needs rows > 0 and k a positive multiple of 32.");
  if (src_dtype != MX_DTYPE_F16 && src_dtype != MX_DTYPE_F32)
    return set_err(c, MX_EINVAL, "quantize source must be f16 or f32.");
  if (!src || !packed || !scales || !aligned16(src) || !aligned16(packed))
    return set_err(c, MX_EINVAL, "quantize buffers must be non-null and 16-byte aligned.");
  MX_HIP(c, mx::launch_mxfp4_quantize(src, src_dtype, packed, scales, rows, k, c->stream));
  return MX_OK;
}

int mx_mxfp4_dequant_f16(mx_ctx* c, const uint8_t* packed, const uint8_t* scales, void* out, int rows,
                         int depth) {
  if (!c) return MX_EINVAL;
  if (rows <= 0 || depth <= 0 || depth % 32)
    return set_err(c, MX_EINVAL, "dequant needs rows > 0 and depth a positive multiple of 32.");
  if (!packed || !scales || !out || !aligned16(packed) || !aligned16(out))
    return set_err(c, MX_EINVAL, "dequant buffers must be non-null and 16-byte aligned.");
  MX_HIP(c, mx::launch_mxfp4_dequant_f16(packed, scales, static_cast<uint16_t*>(out), rows, depth, c->stream));
  return MX_OK;
}

// Any n (the reference's tiles guard column < n, MXFP4Kernels.metal:98);
// k % 32 (one E8M0 block).
static int check_gemm(mx_ctx* c, int m, int n, int k, const void* a, const void* b, const void* out) {
  if (m <= 0 || n <= 0 || k <= 0) return set_err(c, MX_EINVAL, "matmul sizes must be positive.");
  if (k % 32) return set_err(c, MX_EINVAL, "matmul k must be a multiple of 32.");
  if (!a || !b || !out || !aligned16(a) || !aligned16(b) || !aligned16(out))
    return set_err(c, MX_EINVAL, "matmul buffers must be non-null and 16-byte aligned.");
  return MX_OK;
}

// One GEMM through the small-M family when the shape fits it (k % 64),
// else through the K-step-32 kernel.
// ws_off: bytes of the workspace the caller already uses (kept in front of
// the split-K partials).
static int run_gemm(mx_ctx* c, const void* a, int a_dtype, int bk, const void* b, const void* scales,
                    void* out, int epi, int m, int n, int k, size_t ws_off = 0) {
  const int ak = a_dtype == MX_DTYPE_F32 ? mx::AK_F32 : mx::AK_F16;
  if (mx::gemm_q_ok(ak, bk, epi, m, n, k)) {
    const size_t wsb = mx::gemm_q_ws_bytes(ak, bk, epi, m, n, k);
    if (int rc = ensure_ws(c, ws_off + wsb)) return rc;
    void* part = wsb ? static_cast<uint8_t*>(c->ws) + ws_off : nullptr;
    mx::QGemmArgs g{a, nullptr, b, scales, nullptr, nullptr, out, part, m, n, k, 0};
    MX_HIP(c, mx::launch_gemm_q(ak, bk, epi, g, c->stream));
    return MX_OK;
  }
  mx::GemmArgs g{a, a_dtype, b, scales, nullptr, nullptr, out, m, n, k};
  MX_HIP(c, mx::launch_gemm_h(bk, epi, g, c->stream));
  return MX_OK;
}

int mx_mxfp4_matmul(mx_ctx* c, const void* a, int a_dtype, const uint8_t* b, void* out, int c_dtype,
                    int m, int n, int k, const uint8_t* scales) {
  if (!c) return MX_EINVAL;
  if (int rc = check_gemm(c, m, n, k, a, b, out)) return rc;
  if (!scales) return set_err(c, MX_EINVAL, "matmul scales must not be null.");
  if (a_dtype != MX_DTYPE_F16 && a_dtype != MX_DTYPE_F32)
    return set_err(c, MX_EINVAL, "matmul A must be f16 or f32.");
  if (c_dtype != MX_DTYPE_F32 && c_dtype != MX_DTYPE_F16)
    return set_err(c, MX_EINVAL, "matmul C must be f32 or f16.");
  const int epi = c_dtype == MX_DTYPE_F32 ? mx::EPI_STORE_F32 : mx::EPI_STORE_F16;
  return run_gemm(c, a, a_dtype, mx::BK_MXFP4, b, scales, out, epi, m, n, k);
}

int mx_gemm_f16(mx_ctx* c, const void* a, int a_dtype, const void* b, float* out, int m, int n, int k) {
  if (!c) return MX_EINVAL;
  if (int rc = check_gemm(c, m, n, k, a, b, out)) return rc;
  if (a_dtype != MX_DTYPE_F16 && a_dtype != MX_DTYPE_F32)
    return set_err(c, MX_EINVAL, "gemm A must be f16 or f32.");
  return run_gemm(c, a, a_dtype, mx::BK_F16, b, nullptr, out, mx::EPI_STORE_F32, m, n, k);
}

int mx_gemm_i8(mx_ctx* c, const int8_t* a, const int8_t* b, int32_t* out, int m, int n, int k) {
  if (!c) return MX_EINVAL;
  if (int rc = check_gemm(c, m, n, k, a, b, out)) return rc;
  if (!mx::gemm_q_ok(mx::AK_I8, mx::BK_I8, mx::EPI_STORE_I32, m, n, k))
    return set_err(c, MX_EINVAL, "int8 matmul needs n %% 64 == 0 and k %% 128 == 0.");
  const size_t wsb = mx::gemm_q_ws_bytes(mx::AK_I8, mx::BK_I8, mx::EPI_STORE_I32, m, n, k);
  if (int rc = ensure_ws(c, wsb)) return rc;
  mx::QGemmArgs g{a, nullptr, b, nullptr, nullptr, nullptr, out, wsb ? c->ws : nullptr, m, n, k, 0};
  MX_HIP(c, mx::launch_gemm_q(mx::AK_I8, mx::BK_I8, mx::EPI_STORE_I32, g, c->stream));
  return MX_OK;
}

int mx_accum_gemm(mx_ctx* c, int a_fmt, const void* a, int b_fmt, const void* b, void* out, int c_dtype,
                  int m, int n, int k) {
  if (!c) return MX_EINVAL;
  const bool hh = a_fmt == MX_PROBE_F16 && b_fmt == MX_PROBE_F16;
  const bool hq = a_fmt == MX_PROBE_F16 && b_fmt == MX_PROBE_FP4;
  const bool qq = (a_fmt == MX_PROBE_FP4 && b_fmt == MX_PROBE_FP4) || (a_fmt == MX_PROBE_FP8 && b_fmt == MX_PROBE_FP8);
  const bool h4 = a_fmt == MX_PROBE_F16 && b_fmt == MX_PROBE_INT4;
  const bool i8h = a_fmt == MX_PROBE_I8 && b_fmt == MX_PROBE_F16;
  const bool i44 = a_fmt == MX_PROBE_INT4 && b_fmt == MX_PROBE_INT4;
  if (!hh && !hq && !qq && !h4 && !i8h && !i44)
    return set_err(c, MX_EINVAL, "Unsupported probe operand pair (%d, %d).", a_fmt, b_fmt);
  if (m <= 0 || n <= 0 || k <= 0) return set_err(c, MX_EINVAL, "matmul sizes must be positive.");
  if (n % 64) return set_err(c, MX_EINVAL, "matmul n must be a multiple of 64.");
  if (qq && m % 32) return set_err(c, MX_EINVAL, "FP4 / FP8 probe matmul needs m %% 32 == 0.");
  auto nibbles = [](int f) { return f == MX_PROBE_FP4 || f == MX_PROBE_INT4; };
  if ((nibbles(a_fmt) || nibbles(b_fmt)) && k % 2)
    return set_err(c, MX_EINVAL, "packed 4-bit rows need an even k.");
  if (!a || !b || !out || !aligned16(a) || !aligned16(b) || !aligned16(out))
    return set_err(c, MX_EINVAL, "matmul buffers must be non-null and 16-byte aligned.");
  if (i44 ? c_dtype != MX_DTYPE_I32 : (c_dtype != MX_DTYPE_F32 && c_dtype != MX_DTYPE_F16))
    return set_err(c, MX_EINVAL, i44 ? "INT4 x INT4 probe C must be i32." : "probe C must be f32 or f16.");
  const int epi = i44 ? mx::EPI_STORE_I32 : c_dtype == MX_DTYPE_F32 ? mx::EPI_STORE_F32 : mx::EPI_STORE_F16;
  // Workspace: [A'][B'][unit scale plane][split-K partials], sized once so
  // nothing moves in between.  K is padded with zeros to the GEMM's stage
  // (64; 128 for int8) since the reference takes any dot length (e.g. 1022,
  // 1818); INT8 A is widened to f16 and INT4 x INT4 to int8, both exactly.
  auto row_bytes = [](int fmt, size_t kk) {
    return fmt == MX_PROBE_F16 ? kk * 2 : (fmt == MX_PROBE_FP8 || fmt == MX_PROBE_I8) ? kk : kk / 2;
  };
  const size_t kp = align_up((size_t)k, i44 ? 128 : 64);
  const bool pad = kp != (size_t)k;
  const size_t a_sz = i8h ? align_up((size_t)m * kp * 2, 256) : i44 ? align_up((size_t)m * kp, 256)
                      : pad ? align_up((size_t)m * row_bytes(a_fmt, kp), 256) : 0;
  const size_t b_sz = i44 ? align_up((size_t)n * kp, 256) : pad ? align_up((size_t)n * row_bytes(b_fmt, kp), 256) : 0;
  const size_t plane = hq ? align_up((size_t)n * (kp / 32), 256) : h4 ? align_up((size_t)n * (kp / 32) * 2, 256) : 0;
  const int ak = i44 ? mx::AK_I8 : mx::AK_F16;
  const int bk = hq ? mx::BK_MXFP4 : h4 ? mx::BK_INT4G32 : i44 ? mx::BK_I8 : mx::BK_F16;
  const size_t part = !qq && mx::gemm_q_ok(ak, bk, epi, m, n, (int)kp) ? mx::gemm_q_ws_bytes(ak, bk, epi, m, n, (int)kp) : 0;
  if (int rc = ensure_ws(c, a_sz + b_sz + plane + part)) return rc;
  uint8_t* ws = static_cast<uint8_t*>(c->ws);
  const uint8_t* ua = static_cast<const uint8_t*>(a);
  const uint8_t* ub = static_cast<const uint8_t*>(b);
  const void* pa = a;
  const void* pb = b;
  hipStream_t st = c->stream;
  if (i8h || i44) {
    MX_HIP(c, mx::launch_widen_rows(i44, i8h, ua, m, k, ws, kp, st));
    pa = ws;
  } else if (pad) {
    MX_HIP(c, mx::launch_pad_rows(ua, m, row_bytes(a_fmt, k), ws, row_bytes(a_fmt, kp), st));
    pa = ws;
  }
  if (i44) {
    MX_HIP(c, mx::launch_widen_rows(1, 0, ub, n, k, ws + a_sz, kp, st));
    pb = ws + a_sz;
  } else if (pad) {
    MX_HIP(c, mx::launch_pad_rows(ub, n, row_bytes(b_fmt, k), ws + a_sz, row_bytes(b_fmt, kp), st));
    pb = ws + a_sz;
  }
  if (qq) {
    MX_HIP(c, mx::launch_gemm_f8f6f4_unit(a_fmt == MX_PROBE_FP4, c_dtype == MX_DTYPE_F32,
                                          static_cast<const uint8_t*>(pa), static_cast<const uint8_t*>(pb), out, m,
                                          n, (int)kp, st));
    return MX_OK;
  }
  if (i44) {  // exact i32 sums of the widened int8 operands
    mx::QGemmArgs g{pa, nullptr, pb, nullptr, nullptr, nullptr, out, part ? ws + a_sz + b_sz : nullptr, m, n, (int)kp, 0};
    MX_HIP(c, mx::launch_gemm_q(mx::AK_I8, mx::BK_I8, mx::EPI_STORE_I32, g, st));
    return MX_OK;
  }
  uint8_t* sc = nullptr;
  if (hq) {  // unscaled FP4 = MXFP4 with every E8M0 byte 127 (1.0)
    sc = ws + a_sz + b_sz;
    MX_HIP(c, mx::launch_fill_u8(sc, (size_t)n * (kp / 32), 127, st));
  } else if (h4) {  // unscaled INT4 = INT4 with every f16 group scale 1.0
    sc = ws + a_sz + b_sz;
    MX_HIP(c, mx::launch_fill_u16(reinterpret_cast<uint16_t*>(sc), (size_t)n * (kp / 32), 0x3c00, st));
  }
  return run_gemm(c, pa, MX_DTYPE_F16, bk, pb, sc, out, epi, m, n, (int)kp, a_sz + b_sz + plane);
}

int mx_swiglu(mx_ctx* c, const void* gate, const void* up, void* mid, const mx_mlp_config* cfg, int variant) {
  if (!c) return MX_EINVAL;
  if (variant < 0 || variant > 3) return set_err(c, MX_EINVAL, "Unknown SwiGLU variant %d.", variant);
  if (!cfg) return set_err(c, MX_EINVAL, "MLP config is null.");
  if (cfg->tokens == 0 || cfg->intermediate == 0) return set_err(c, MX_EINVAL, "SwiGLU sizes must be positive.");
  if (!gate || !up || !mid) return set_err(c, MX_EINVAL, "SwiGLU buffers must not be null.");
  MX_HIP(c, mx::launch_swiglu(variant, gate, up, mid, (size_t)cfg->tokens * cfg->intermediate, c->stream));
  return MX_OK;
}

// ---- MLP ------------------------------------------------------------------------
int mx_mlp_forward(mx_ctx* c, int variant, const mx_mlp_config* cfg, const void* x,
                   const mx_mlp_weights* w, void* out) {
  if (!c) return MX_EINVAL;
  std::vector<Step> steps;
  if (int rc = build_mlp_steps(c, variant, cfg, x, w, out, steps)) return rc;
  return run_steps(c, steps);
}

int mx_mlp_forward_noalloc(mx_ctx* c, int variant, const mx_mlp_config* cfg, const void* x,
                           const mx_mlp_weights* w, void* out) {
  if (!c) return MX_EINVAL;
  void* p = nullptr;
  hipError_t e = hipErrorInvalidDevice;
  if (c->device < kMaxDevices) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    p = g_scratch_ptr[c->device];
    e = g_scratch_err[c->device];
  }
  if (!p)
    return set_err(c, MX_EGPU, "The allocation-free forward has no scratch address on device %d: %s.", c->device,
                   hipGetErrorString(e));
  std::vector<Step> steps;
  if (int rc = build_mlp_steps(c, variant, cfg, x, w, out, steps, static_cast<uint8_t*>(p), MX_NOALLOC_SCRATCH_BYTES))
    return rc;
  return run_steps(c, steps);
}

const char* mx_mlp_kernel_name(int variant, const mx_mlp_config* cfg, int index) {
  static const char* gemv[] = {"gemv_mxfp4_gate_up_swiglu", "gemv_mxfp4_down"};
  static const char* fused[] = {"gemm_q_mxfp4_gate_up_swiglu", "gemm_q_mxfp4_down"};
  static const char* ref[] = {"gemm_q_mxfp4_gate_up_swiglu_half", "gemm_q_mxfp4_down_f32"};
  static const char* fused_h[] = {"gemm_h_mxfp4_gate_up_swiglu", "gemm_h_mxfp4_down"};
  static const char* ref_h[] = {"gemm_h_mxfp4_gate_up_swiglu_half", "gemm_h_mxfp4_down_f32"};
  static const char* deq[] = {"dequant_gate", "dequant_up", "dequant_down", "gemm_h_h_f_gate",
                              "gemm_h_h_f_up", "swiglu_float", "gemm_f_h_down"};
  static const char* w4[] = {"w4a4_prologue", "gemm_fp4_gate_up_swiglu_requant", "gemm_fp4_down", "w4a4_down_inf"};
  // (the stage-major path runs the first three; the reference-layout one all four)
  static const char* sc[] = {"split_x_f8x2", "gemm_q_scaled_gate_up_swiglu", "gemm_q_scaled_down"};
  if (index < 0 || !cfg || variant < MX_MLP_FUSED || variant > MX_MLP_SCALED) return nullptr;
  switch (mlp_path(variant, cfg)) {
    case PATH_GEMV: return index < 2 ? gemv[index] : nullptr;
    case PATH_GEMM_Q: return index < 2 ? fused[index] : nullptr;
    case PATH_REFROW: return index < 2 ? ref[index] : nullptr;
    case PATH_GEMM_H: return index < 2 ? fused_h[index] : nullptr;
    case PATH_REFROW_H: return index < 2 ? ref_h[index] : nullptr;
    case PATH_DEQUANT: return index < 7 ? deq[index] : nullptr;
    case PATH_W4A4: return index < 3 ? w4[index] : nullptr;
    case PATH_W4A4_REF: return index < 4 ? w4[index] : nullptr;
    case PATH_SCALED: return index < 3 ? sc[index] : nullptr;
  }
  return nullptr;
}

// Capture `iterations` forwards into one HIP graph (kernel nodes and the two
// timing events only: no memset or copy nodes) - the counterpart of the
// reference encoding all iterations into one command buffer
// (main.swift:2062-2117).  `start` / `end` are recorded as the graph's first
// and last nodes, so their interval is the graph's execution on the GPU, as
// the reference reports gpuEndTime - gpuStartTime (main.swift:2131-2133).
static int capture_graph(mx_ctx* c, const std::vector<std::vector<Step>>& sets, int iterations,
                         hipGraphExec_t* exec, hipEvent_t start, hipEvent_t end) {
  const int ns = (int)sets.size();
  hipGraph_t graph = nullptr;
  MX_HIP(c, hipStreamBeginCapture(c->stream, hipStreamCaptureModeThreadLocal));
  int rc = MX_OK;
  // hipEventRecordExternal: captured as event record nodes of the graph
  // (a plain record inside a capture only orders captured work)
  if (hipEventRecordWithFlags(start, c->stream, hipEventRecordExternal) != hipSuccess)
    rc = set_err(c, MX_EGPU, "event record failed");
  for (int i = 0; i < iterations && !rc; i++) rc = run_steps(c, sets[i % ns]);
  if (!rc && hipEventRecordWithFlags(end, c->stream, hipEventRecordExternal) != hipSuccess)
    rc = set_err(c, MX_EGPU, "event record failed");
  hipError_t e = hipStreamEndCapture(c->stream, &graph);
  if (rc) { if (graph) (void)hipGraphDestroy(graph); return rc; }
  if (e != hipSuccess) return set_err(c, MX_EGPU, "graph capture failed: %s", hipGetErrorString(e));
  e = hipGraphInstantiate(exec, graph, nullptr, nullptr, 0);
  (void)hipGraphDestroy(graph);
  if (e != hipSuccess) return set_err(c, MX_EGPU, "graph instantiate failed: %s", hipGetErrorString(e));
  return MX_OK;
}

// Time `iterations` passes over `sets` (set i % n_sets on pass i) between two
// events: replayed from one captured graph (events inside it, around its
// kernels), or launched one by one (events on the stream around the
// launches).  When there are more sets than passes, the sets the timed
// passes do not use run once (untimed) just before the timed region, so that
// what the timed passes read was evicted from the last-level cache by at
// least that many bytes.
static int time_passes(mx_ctx* c, const std::vector<std::vector<Step>>& sets, int iterations,
                       int use_graph, double* seconds) {
  const int ns = (int)sets.size();
  hipEvent_t e0 = nullptr, e1 = nullptr;
  if (hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess) {
    if (e0) (void)hipEventDestroy(e0);
    return set_err(c, MX_EGPU, "event create failed");
  }
  hipGraphExec_t gexec = nullptr;
  int rc = MX_OK;
  if (use_graph) {
    rc = capture_graph(c, sets, iterations, &gexec, e0, e1);
    // one untimed replay (first launch of an instantiated graph uploads it)
    if (!rc && hipGraphLaunch(gexec, c->stream) != hipSuccess) rc = set_err(c, MX_EGPU, "graph launch failed");
  }
  for (int i = iterations; i < ns && !rc; i++) rc = run_steps(c, sets[(size_t)i]);
  do {
    if (rc) break;
    if (hipStreamSynchronize(c->stream) != hipSuccess) { rc = set_err(c, MX_EGPU, "sync failed"); break; }
    if (gexec) {
      if (hipGraphLaunch(gexec, c->stream) != hipSuccess) rc = set_err(c, MX_EGPU, "graph launch failed");
    } else {
      if (hipEventRecord(e0, c->stream) != hipSuccess) { rc = set_err(c, MX_EGPU, "event record failed"); break; }
      for (int i = 0; i < iterations && !rc; i++) rc = run_steps(c, sets[i % ns]);
      if (!rc && hipEventRecord(e1, c->stream) != hipSuccess) rc = set_err(c, MX_EGPU, "event record failed");
    }
    if (rc) break;
    if (hipEventSynchronize(e1) != hipSuccess) { rc = set_err(c, MX_EGPU, "MXFP4 MLP timed loop failed."); break; }
    float ms = 0.0f;
    const hipError_t te = hipEventElapsedTime(&ms, e0, e1);
    if (te != hipSuccess || !(ms > 0.0f)) {
      rc = set_err(c, MX_EGPU, "timing events gave no interval: %s", hipGetErrorString(te));
      break;
    }
    *seconds = ms / 1000.0;
  } while (0);
  if (e0) (void)hipEventDestroy(e0);
  if (e1) (void)hipEventDestroy(e1);
  if (gexec) (void)hipGraphExecDestroy(gexec);
  return rc;
}

static int bench_loop(mx_ctx* c, const std::vector<std::vector<Step>>& sets, int warmup,
                      int iterations, int use_graph, double* seconds_out, double* kernel_us_out,
                      int* n_kernels_out) {
  if (iterations <= 0 || warmup < 0)
    return set_err(c, MX_EINVAL, "MLP sizes and iterations must be positive.");
  const int ns = (int)sets.size();
  for (int i = 0; i < warmup; i++)
    if (int rc = run_steps(c, sets[i % ns])) return rc;
  double secs = 0.0;
  if (int rc = time_passes(c, sets, iterations, use_graph, &secs)) return rc;
  if (seconds_out) *seconds_out = secs;
  if (kernel_us_out || n_kernels_out) {
    // Per kernel: back-to-back launches of that kernel alone (same weight-
    // set rotation, same graph / stream mode), so the average is the
    // kernel's own duration, as a kernel trace reports it.  At least one
    // launch per weight set, so that a pass streams every set once whatever
    // `iterations` is (the caller sizes the sets past the last-level cache).
    const int nk = (int)sets[0].size();
    const int kiters = std::max(iterations, ns);
    if (n_kernels_out) *n_kernels_out = nk > 8 ? 8 : nk;
    for (int k = 0; k < nk && k < 8; k++) {
      std::vector<std::vector<Step>> one((size_t)ns);
      for (int i = 0; i < ns; i++) one[(size_t)i].push_back(sets[(size_t)i][(size_t)k]);
      double ks = 0.0;
      if (int rc = time_passes(c, one, kiters, use_graph, &ks)) return rc;
      if (kernel_us_out) kernel_us_out[k] = ks * 1e6 / kiters;
    }
  }
  return MX_OK;
}

int mx_mlp_benchmark(mx_ctx* c, int variant, const mx_mlp_config* cfg, const void* x,
                     const mx_mlp_weights* sets, int n_sets, void* out, int warmup, int iterations,
                     int use_graph, double* seconds_out, double* kernel_us_out, int* n_kernels_out) {
  if (!c) return MX_EINVAL;
  if (!sets || n_sets <= 0) return set_err(c, MX_EINVAL, "benchmark needs at least one weight set.");
  std::vector<std::vector<Step>> all((size_t)n_sets);
  for (int i = 0; i < n_sets; i++)
    if (int rc = build_mlp_steps(c, variant, cfg, x, &sets[i], out, all[i])) return rc;
  return bench_loop(c, all, warmup, iterations, use_graph, seconds_out, kernel_us_out, n_kernels_out);
}

// ---- MoE: grouped experts ---------------------------------------------------------
// Two grouped launches for all experts: the decode GEMV when every expert has
// at most 16 tokens, else the small-M GEMM family (one tile grid per expert
// in blockIdx.z).  Expert e owns token rows [off[e], off[e+1]).
static int build_moe_steps(mx_ctx* c, const mx_mlp_config* cfg, int n_experts, const int* counts,
                           const void* x, const mx_mlp_weights* w, void* out, std::vector<Step>& steps) {
  if (int rc = check_mlp_cfg(c, MX_MLP_FUSED, cfg)) return rc;
  if (n_experts < 1 || n_experts > mx::kMaxGroups)
    return set_err(c, MX_EINVAL, "MoE needs 1 to %d experts.", mx::kMaxGroups);
  if (!counts || !x || !w || !out) return set_err(c, MX_EINVAL, "MoE buffers must not be null.");
  const mx_qmatrix* mats[3] = {&w->gate, &w->up, &w->down};
  for (const mx_qmatrix* m : mats) {
    if (!m->data || !m->scales) return set_err(c, MX_EINVAL, "MLP weight buffers must not be null.");
    if (!aligned16(m->data)) return set_err(c, MX_EINVAL, "MXFP4 weight data must be 16-byte aligned.");
    if (reinterpret_cast<uintptr_t>(m->scales) & 3u)
      return set_err(c, MX_EINVAL, "MXFP4 scale planes must be 4-byte aligned.");
  }
  if (!aligned16(x) || !aligned16(out))
    return set_err(c, MX_EINVAL, "Activation and output buffers must be 16-byte aligned.");
  const int T = cfg->tokens, H = cfg->hidden, I = cfg->intermediate;
  mx::GroupTable gu_t{}, dn_t{};
  long total = 0;
  int most = 0;
  for (int e = 0; e < n_experts; e++) {
    if (counts[e] < 0) return set_err(c, MX_EINVAL, "MoE token counts must not be negative.");
    gu_t.off[e] = dn_t.off[e] = (int)total;
    total += counts[e];
    most = std::max(most, counts[e]);
  }
  gu_t.off[n_experts] = dn_t.off[n_experts] = (int)total;
  if (total != T) return set_err(c, MX_EINVAL, "MoE token counts must add up to tokens (%ld != %d).", total, T);
  gu_t.b_stride = (size_t)I * H / 2;
  gu_t.s_stride = (size_t)I * H / 32;
  dn_t.b_stride = (size_t)H * I / 2;
  dn_t.s_stride = (size_t)H * I / 32;
  const size_t mid_b = align_up((size_t)T * I * 2, 256);
  if (int rc = ensure_ws(c, mid_b)) return rc;
  uint16_t* mid = static_cast<uint16_t*>(c->ws);
  hipStream_t st = c->stream;
  const uint8_t* wg = static_cast<const uint8_t*>(w->gate.data);
  const uint8_t* sg = static_cast<const uint8_t*>(w->gate.scales);
  const uint8_t* wu = static_cast<const uint8_t*>(w->up.data);
  const uint8_t* su = static_cast<const uint8_t*>(w->up.scales);
  const uint8_t* wd = static_cast<const uint8_t*>(w->down.data);
  const uint8_t* sd = static_cast<const uint8_t*>(w->down.scales);
  const int E = n_experts;
  mx_mlp_config most_cfg = *cfg;
  most_cfg.tokens = (uint32_t)std::max(most, 1);
  if (gemv_ok(&most_cfg)) {
    mx::GemvArgs gu{static_cast<const uint16_t*>(x), wg, sg, wu, su, mid, most, I, H};
    mx::GemvArgs dn{mid, wd, sd, nullptr, nullptr, static_cast<uint16_t*>(out), most, H, I};
    steps.push_back({"moe_gemv_gate_up_swiglu", [=] { return mx::launch_gemv_mxfp4_grouped(1, gu, gu_t, E, st); }});
    steps.push_back({"moe_gemv_down", [=] { return mx::launch_gemv_mxfp4_grouped(0, dn, dn_t, E, st); }});
    return MX_OK;
  }
  if (!mx::gemm_q_ok(mx::AK_F16, mx::BK_MXFP4, mx::EPI_SWIGLU_F16, most, I, H) ||
      !mx::gemm_q_ok(mx::AK_F16, mx::BK_MXFP4, mx::EPI_STORE_F16, most, H, I))
    return set_err(c, MX_EINVAL,
                   "MoE needs hidden and intermediate %% 64 == 0 (%% 128 for the decode GEMV of experts with "
                   "at most 16 tokens).");
  mx::QGemmArgs gu{x, nullptr, wg, sg, wu, su, mid, nullptr, most, I, H, 0};
  mx::QGemmArgs dn{mid, nullptr, wd, sd, nullptr, nullptr, out, nullptr, most, H, I, 0};
  steps.push_back({"moe_gemm_q_gate_up_swiglu",
                   [=] { return mx::launch_gemm_q_grouped(mx::EPI_SWIGLU_F16, gu, gu_t, E, st); }});
  steps.push_back({"moe_gemm_q_down", [=] { return mx::launch_gemm_q_grouped(mx::EPI_STORE_F16, dn, dn_t, E, st); }});
  return MX_OK;
}

int mx_moe_forward(mx_ctx* c, const mx_mlp_config* cfg, int n_experts, const int* counts, const void* x,
                   const mx_mlp_weights* w, void* out) {
  if (!c) return MX_EINVAL;
  std::vector<Step> steps;
  if (int rc = build_moe_steps(c, cfg, n_experts, counts, x, w, out, steps)) return rc;
  return run_steps(c, steps);
}

int mx_moe_benchmark(mx_ctx* c, const mx_mlp_config* cfg, int n_experts, const int* counts, const void* x,
                     const mx_mlp_weights* sets, int n_sets, void* out, int warmup, int iterations, int use_graph,
                     double* seconds_out) {
  if (!c) return MX_EINVAL;
  if (!sets || n_sets <= 0) return set_err(c, MX_EINVAL, "benchmark needs at least one weight set.");
  std::vector<std::vector<Step>> all((size_t)n_sets);
  for (int i = 0; i < n_sets; i++)
    if (int rc = build_moe_steps(c, cfg, n_experts, counts, x, &sets[i], out, all[i])) return rc;
  return bench_loop(c, all, warmup, iterations, use_graph, seconds_out, nullptr, nullptr);
}

// ---- weight formats ---------------------------------------------------------------
int mx_fmt_quantize(mx_ctx* c, int wfmt, const float* w, int rows, int k, void* q, void* scales) {
  if (!c) return MX_EINVAL;
  if (rows <= 0 || k <= 0 || k % 32) return set_err(c, MX_EINVAL, "format quantize needs k % 32 == 0.");
  if (!w || !q || !scales || !aligned16(w) || !aligned16(q))
    return set_err(c, MX_EINVAL, "format quantize buffers must be non-null and 16-byte aligned.");
  if (wfmt == MX_WFMT_FP8_E4M3_F8X2 || wfmt == MX_WFMT_FP8_E5M2_F8X2)
    wfmt = wfmt == MX_WFMT_FP8_E4M3_F8X2 ? MX_WFMT_FP8_E4M3 : MX_WFMT_FP8_E5M2;  // same weights
  switch (wfmt) {
    case MX_WFMT_FP8_E4M3:
    case MX_WFMT_FP8_E5M2:
    case MX_WFMT_INT8:
    case MX_WFMT_W8A8:
      MX_HIP(c, mx::launch_quant_rowwise(wfmt == MX_WFMT_W8A8 ? MX_WFMT_INT8 : wfmt, w, rows, k,
                                         static_cast<uint8_t*>(q), static_cast<float*>(scales), c->stream));
      return MX_OK;
    case MX_WFMT_INT4:
      MX_HIP(c, mx::launch_quant_int4_g32(w, rows, k, static_cast<uint8_t*>(q),
                                          static_cast<uint16_t*>(scales), c->stream));
      return MX_OK;
  }
  return set_err(c, MX_EINVAL, "Unknown weight format %d.", wfmt);
}

static int build_fmt_steps(mx_ctx* c, int wfmt, const mx_mlp_config* cfg, const void* x,
                           const mx_mlp_weights* w, void* out, std::vector<Step>& steps) {
  if (int rc = check_mlp_cfg(c, MX_MLP_FUSED, cfg)) return rc;
  if (!x || !w || !out) return set_err(c, MX_EINVAL, "MLP buffers must not be null.");
  int bk;
  switch (wfmt) {
    case MX_WFMT_FP8_E4M3: bk = mx::BK_E4M3; break;
    case MX_WFMT_FP8_E5M2: bk = mx::BK_E5M2; break;
    case MX_WFMT_INT8: bk = mx::BK_INT8; break;
    case MX_WFMT_INT4: bk = mx::BK_INT4G32; break;
    case MX_WFMT_W8A8: bk = mx::BK_I8; break;
    case MX_WFMT_FP8_E4M3_F8X2: bk = mx::BK_E4M3; break;
    case MX_WFMT_FP8_E5M2_F8X2: bk = mx::BK_E5M2; break;
    default: return set_err(c, MX_EINVAL, "Unknown weight format %d.", wfmt);
  }
  const mx_qmatrix* mats[3] = {&w->gate, &w->up, &w->down};
  for (const mx_qmatrix* m : mats)
    if (!m->data || !m->scales || !aligned16(m->data) || (reinterpret_cast<uintptr_t>(m->scales) & 3u))
      return set_err(c, MX_EINVAL, "format weight buffers must be non-null and 16-byte aligned.");
  const int T = cfg->tokens, H = cfg->hidden, I = cfg->intermediate;
  hipStream_t st = c->stream;
  if (bk == mx::BK_I8) {
    // W8A8 (MPPMLPKernels.metal:61-70, 240-257 with BASELINE's scales):
    // x -> int8 per token, i32 GEMMs, f32 mid re-quantized per token.
    if (H % 128 || I % 128)
      return set_err(c, MX_EINVAL, "W8A8 needs hidden and intermediate to be multiples of 128.");
    size_t off = 0;
    auto take = [&](size_t bytes) { size_t o = off; off = align_up(off + bytes, 256); return o; };
    const size_t o_xq = take((size_t)T * H), o_xs = take((size_t)T * 4), o_mid = take((size_t)T * I * 4),
                 o_mq = take((size_t)T * I), o_ms = take((size_t)T * 4),
                 o_qws = take(std::max(mx::gemm_q_ws_bytes(mx::AK_I8, mx::BK_I8, mx::EPI_SWIGLU_F32, T, I, H),
                                       mx::gemm_q_ws_bytes(mx::AK_I8, mx::BK_I8, mx::EPI_STORE_F16, T, H, I)));
    if (int rc = ensure_ws(c, off)) return rc;
    uint8_t* ws = static_cast<uint8_t*>(c->ws);
    int8_t* xq = reinterpret_cast<int8_t*>(ws + o_xq);
    float* xs = reinterpret_cast<float*>(ws + o_xs);
    float* mid = reinterpret_cast<float*>(ws + o_mid);
    int8_t* mq = reinterpret_cast<int8_t*>(ws + o_mq);
    float* ms = reinterpret_cast<float*>(ws + o_ms);
    void* qws = ws + o_qws;
    mx::QGemmArgs gu{xq, xs, w->gate.data, w->gate.scales, w->up.data, w->up.scales, mid, qws, T, I, H, 0};
    mx::QGemmArgs dn{mq, ms, w->down.data, w->down.scales, nullptr, nullptr, out, qws, T, H, I, 0};
    steps.push_back({"quant_x_int8", [=] { return mx::launch_quant_act_int8(x, MX_DTYPE_F16, T, H, xq, xs, st); }});
    steps.push_back({"gemm_q_w8a8_gate_up_swiglu", [=] { return mx::launch_gemm_q(mx::AK_I8, mx::BK_I8, mx::EPI_SWIGLU_F32, gu, st); }});
    steps.push_back({"quant_mid_int8", [=] { return mx::launch_quant_act_int8(mid, MX_DTYPE_F32, T, I, mq, ms, st); }});
    steps.push_back({"gemm_q_w8a8_down", [=] { return mx::launch_gemm_q(mx::AK_I8, mx::BK_I8, mx::EPI_STORE_F16, dn, st); }});
    return MX_OK;
  }
  if (wfmt == MX_WFMT_FP8_E4M3_F8X2 || wfmt == MX_WFMT_FP8_E5M2_F8X2) {
    // FP8 weights on the FP8 matrix cores: x and mid as F8X2 (two E4M3
    // terms + E8M0 pairs per 64 K), the weight codes as the scaled MFMA's
    // second operand at scale 1.0, the row scales applied to the sums.
    if (H % 64 || I % 64)
      return set_err(c, MX_EINVAL, "The F8X2 format rows need hidden and intermediate to be multiples of 64.");
    size_t off = 0;
    auto take = [&](size_t bytes) { size_t o = off; off = align_up(off + bytes, 256); return o; };
    const size_t o_xq = take(mx::f8x2_data_bytes(T, H)), o_xe = take(mx::f8x2_e8_bytes(T, H)),
                 o_mq = take(mx::f8x2_data_bytes(T, I)), o_me = take(mx::f8x2_e8_bytes(T, I)),
                 o_qws = take(std::max(mx::gemm_q_ws_bytes(mx::AK_F8X2, bk, mx::EPI_SWIGLU_F8X2, T, I, H),
                                       mx::gemm_q_ws_bytes(mx::AK_F8X2, bk, mx::EPI_STORE_F16, T, H, I)));
    if (int rc = ensure_ws(c, off)) return rc;
    uint8_t* ws = static_cast<uint8_t*>(c->ws);
    uint8_t* xq = ws + o_xq;
    uint32_t* xe = reinterpret_cast<uint32_t*>(ws + o_xe);
    uint8_t* mq = ws + o_mq;
    uint32_t* me = reinterpret_cast<uint32_t*>(ws + o_me);
    void* qws = ws + o_qws;
    mx::QGemmArgs gu{xq, nullptr, w->gate.data, w->gate.scales, w->up.data, w->up.scales, mq, qws, T, I, H, 0,
                     xe, me, static_cast<const uint16_t*>(x)};
    mx::QGemmArgs dn{mq, nullptr, w->down.data, w->down.scales, nullptr, nullptr, out, qws, T, H, I, 0, me,
                     nullptr};
    steps.push_back({"split_x_f8x2", [=] {
                       return mx::launch_split_f8x2(static_cast<const uint16_t*>(x), T, H, xq, xe, st);
                     }});
    steps.push_back({"gemm_q_f8x2_fmt_gate_up_swiglu",
                     [=] { return mx::launch_gemm_q(mx::AK_F8X2, bk, mx::EPI_SWIGLU_F8X2, gu, st); }});
    steps.push_back({"gemm_q_f8x2_fmt_down",
                     [=] { return mx::launch_gemm_q(mx::AK_F8X2, bk, mx::EPI_STORE_F16, dn, st); }});
    return MX_OK;
  }
  const size_t mid_b = align_up((size_t)T * I * 2, 256);
  const size_t qws_b = std::max(q_ws(mx::AK_F16, bk, mx::EPI_SWIGLU_F16, T, I, H),
                                q_ws(mx::AK_F16, bk, mx::EPI_STORE_F16, T, H, I));
  if (int rc = ensure_ws(c, mid_b + qws_b)) return rc;
  uint16_t* mid = static_cast<uint16_t*>(c->ws);
  void* qws = static_cast<uint8_t*>(c->ws) + mid_b;
  mx::QGemmArgs gu{x, nullptr, w->gate.data, w->gate.scales, w->up.data, w->up.scales, mid, qws, T, I, H, 0};
  mx::QGemmArgs dn{mid, nullptr, w->down.data, w->down.scales, nullptr, nullptr, out, qws, T, H, I, 0};
  steps.push_back({mx_fmt_mlp_kernel_name(wfmt, cfg, 0),
                   [=] { return launch_mlp_gemm(mx::AK_F16, bk, mx::EPI_SWIGLU_F16, gu, st); }});
  steps.push_back({mx_fmt_mlp_kernel_name(wfmt, cfg, 1),
                   [=] { return launch_mlp_gemm(mx::AK_F16, bk, mx::EPI_STORE_F16, dn, st); }});
  return MX_OK;
}

int mx_fmt_mlp_forward(mx_ctx* c, int wfmt, const mx_mlp_config* cfg, const void* x,
                       const mx_mlp_weights* w, void* out) {
  if (!c) return MX_EINVAL;
  std::vector<Step> steps;
  if (int rc = build_fmt_steps(c, wfmt, cfg, x, w, out, steps)) return rc;
  return run_steps(c, steps);
}

int mx_fmt_mlp_benchmark(mx_ctx* c, int wfmt, const mx_mlp_config* cfg, const void* x,
                         const mx_mlp_weights* sets, int n_sets, void* out, int warmup,
                         int iterations, int use_graph, double* seconds_out, double* kernel_us_out,
                         int* n_kernels_out) {
  if (!c) return MX_EINVAL;
  if (!sets || n_sets <= 0) return set_err(c, MX_EINVAL, "benchmark needs at least one weight set.");
  std::vector<std::vector<Step>> all((size_t)n_sets);
  for (int i = 0; i < n_sets; i++)
    if (int rc = build_fmt_steps(c, wfmt, cfg, x, &sets[i], out, all[i])) return rc;
  return bench_loop(c, all, warmup, iterations, use_graph, seconds_out, kernel_us_out, n_kernels_out);
}

const char* mx_fmt_mlp_kernel_name(int wfmt, const mx_mlp_config* cfg, int index) {
  static const char* w8a8[] = {"quant_x_int8", "gemm_q_w8a8_gate_up_swiglu", "quant_mid_int8", "gemm_q_w8a8_down"};
  static const char* q[] = {"gemm_q_fmt_gate_up_swiglu", "gemm_q_fmt_down"};
  static const char* h[] = {"gemm_h_fmt_gate_up_swiglu", "gemm_h_fmt_down"};
  static const char* f8x2[] = {"split_x_f8x2", "gemm_q_f8x2_fmt_gate_up_swiglu", "gemm_q_f8x2_fmt_down"};
  if (index < 0 || !cfg || wfmt < MX_WFMT_FP8_E4M3 || wfmt > MX_WFMT_FP8_E5M2_F8X2) return nullptr;
  if (wfmt == MX_WFMT_W8A8) return index < 4 ? w8a8[index] : nullptr;
  if (wfmt == MX_WFMT_FP8_E4M3_F8X2 || wfmt == MX_WFMT_FP8_E5M2_F8X2) return index < 3 ? f8x2[index] : nullptr;
  if (index >= 2) return nullptr;
  const int bk = wfmt == MX_WFMT_FP8_E4M3 ? mx::BK_E4M3 : wfmt == MX_WFMT_FP8_E5M2 ? mx::BK_E5M2
                 : wfmt == MX_WFMT_INT8 ? mx::BK_INT8 : mx::BK_INT4G32;
  const int T = cfg->tokens, H = cfg->hidden, I = cfg->intermediate;
  const bool on_q = index == 0 ? mx::gemm_q_ok(mx::AK_F16, bk, mx::EPI_SWIGLU_F16, T, I, H)
                               : mx::gemm_q_ok(mx::AK_F16, bk, mx::EPI_STORE_F16, T, H, I);
  return on_q ? q[index] : h[index];
}

// ---- synthetic data ------------------------------------------------------------------
int mx_fill_normal(mx_ctx* c, void* dst, int dtype, size_t n, uint64_t seed, float mean, float stddev) {
  if (!c) return MX_EINVAL;
  if (dtype != MX_DTYPE_F32 && dtype != MX_DTYPE_F16)
    return set_err(c, MX_EINVAL, "fill_normal dtype must be f32 or f16.");
  if (n && !dst) return set_err(c, MX_EINVAL, "fill_normal buffer must not be null.");
  MX_HIP(c, mx::launch_fill_normal(dst, dtype, n, seed, mean, stddev, c->stream));
  return MX_OK;
}

static inline uint16_t host_f32_to_f16(float f) {
  _Float16 h = (_Float16)f;  // host compiler: IEEE RNE
  uint16_t u;
  std::memcpy(&u, &h, 2);
  return u;
}

void mx_lcg_bytes(uint32_t seed, size_t count, uint8_t* out) {
  uint32_t s = seed;
  for (size_t i = 0; i < count; i++) {
    s = s * 1664525u + 1013904223u + (uint32_t)i;
    out[i] = (uint8_t)(s >> 16);
  }
}

void mx_lcg_pattern(uint32_t seed, size_t count, const uint8_t* pattern, int pattern_count, uint8_t* out) {
  uint32_t s = seed;
  for (size_t i = 0; i < count; i++) {
    s = s * 1664525u + 1013904223u + (uint32_t)i;
    out[i] = pattern[s % (uint32_t)pattern_count];
  }
}

void mx_lcg_half(uint32_t seed, size_t count, float scale, uint16_t* out) {
  uint32_t s = seed;
  for (size_t i = 0; i < count; i++) {
    s = s * 1664525u + 1013904223u + (uint32_t)i;
    const int nib = (int)((s >> 28) & 15u);
    out[i] = host_f32_to_f16((float)((nib ^ 8) - 8) * scale);
  }
}

void mx_lcg_int8(uint32_t seed, size_t count, int8_t* out) {
  uint32_t s = seed;
  for (size_t i = 0; i < count; i++) {
    s = s * 1664525u + 1013904223u + (uint32_t)i;
    const int nib = (int)((s >> 28) & 15u);
    out[i] = (int8_t)((nib ^ 8) - 8);
  }
}

double mx_checksum_f32(const float* p, size_t count, int* samples) {
  const size_t step = count / 32 > 1 ? count / 32 : 1;
  double sum = 0.0;
  int n = 0;
  for (size_t i = 0; i < count; i += step) { sum += (double)p[i]; n++; }
  if (samples) *samples = n;
  return sum;
}

int64_t mx_checksum_i32(const int32_t* p, size_t count, int* samples) {
  const size_t step = count / 32 > 1 ? count / 32 : 1;
  int64_t sum = 0;
  int n = 0;
  for (size_t i = 0; i < count; i += step) { sum += p[i]; n++; }
  if (samples) *samples = n;
  return sum;
}

uint64_t mx_checksum_f16raw(const uint16_t* p, size_t count, int* samples) {
  const size_t step = count / 32 > 1 ? count / 32 : 1;
  uint64_t sum = 0;
  int n = 0;
  for (size_t i = 0; i < count; i += step) { sum += p[i]; n++; }
  if (samples) *samples = n;
  return sum;
}

}  // extern "C"
