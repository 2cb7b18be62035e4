// mxfp4_probe - command-line host driver over libmxfp4hip, the counterpart of
// the reference's MetalFP41Probe executable (Sources/MetalFP41Probe/main.swift).
// Swift is not available on this platform, so the driver is C++ on the C ABI.
//
// Same surface as the reference:
//   (no flags)            packed numeric KAT probe: FP4 E2M1, FP8 E4M3, FP8 E5M2
//                         roundtrips (main.swift:98-162), printed as
//                         "[ok] <name>" / input / unpacked / expected / bytes
//   --skip-tensor         skips the tensor-object probe (no counterpart on ROCm)
//   --mlp-benchmark       gated MLP benchmark rows (runMLPBenchmark, :586-1521)
//     --mlp-tokens=T --mlp-hidden=H --mlp-intermediate=I --mlp-iterations=N
//     (defaults 128, 1024, 4*H, 3 as in :587-590)
//   --accum-probe         accumulator precision / overflow probe
//                         (runAccumulatorProbe, :1523-1713)
//   --benchmark           big matmul rows (runBigMatmulBenchmark, :380-584)
//     --matmul-size=S --m= --n= --k= --iterations= (defaults 2048, 3);
//     --fp4-group-sweep adds the g8 rows
//   success ends with "PASS"; a failure prints "error: <message>" on stderr
//   and exits 1 (:83-88).
//
// Data follows the reference generators and seeds (main.swift:611-638,
// 2785-2842): half x from the LCG with scale 1/8, packed FP4 weight bytes
// from the LCG, E8M0 scales drawn from the pattern [124..130].  The format
// rows quantize N(0, 0.02) weights as BASELINE configs[3] prescribes.
#include <cmath>
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <string>
#include <vector>

#include "mxfp4hip.h"

namespace {

struct ProbeError {
  std::string message;
};

[[noreturn]] void fail(const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  std::vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  throw ProbeError{buf};
}

std::vector<std::string> g_args;

bool has_flag(const char* name) {
  for (const std::string& a : g_args)
    if (a == name) return true;
  return false;
}

// intArgument (main.swift:2886-2892): "--name=value", default when absent or
// not an integer.
long int_argument(const char* name, long default_value) {
  const std::string prefix = std::string(name) + "=";
  for (const std::string& a : g_args) {
    if (a.compare(0, prefix.size(), prefix) == 0) {
      const char* s = a.c_str() + prefix.size();
      char* end = nullptr;
      const long v = std::strtol(s, &end, 10);
      return (end && *end == '\0' && end != s) ? v : default_value;
    }
  }
  return default_value;
}

void check(mx_ctx* ctx, int rc) {
  if (rc != MX_OK) throw ProbeError{ctx ? mx_last_error(ctx) : mx_status_string(rc)};
}

// Value formatting of the KAT printout (format / formatHex, :302-316).
std::string format_values(const std::vector<float>& v) {
  std::string out;
  char buf[64];
  for (size_t i = 0; i < v.size(); i++) {
    const float x = v[i];
    if (std::isinf(x)) std::snprintf(buf, sizeof buf, "%s", x < 0 ? "-inf" : "inf");
    else if (std::nearbyint(x) == x) std::snprintf(buf, sizeof buf, "%.0f", x);
    else std::snprintf(buf, sizeof buf, "%.6g", x);
    if (i) out += ", ";
    out += buf;
  }
  return out;
}

std::string format_hex(const std::vector<uint8_t>& b) {
  std::string out;
  char buf[8];
  for (size_t i = 0; i < b.size(); i++) {
    std::snprintf(buf, sizeof buf, "%s%02X", i ? " " : "", b[i]);
    out += buf;
  }
  return out;
}

struct KatCase {
  const char* name;
  int fmt;
  std::vector<float> inputs, expected;
  size_t packed_bytes;
};

// Packed numeric probe (runPackedNumericProbe, :91-162).  Returns true when
// every roundtrip matches.
bool run_kats(mx_ctx* ctx) {
  const KatCase cases[] = {
      {"FP4 E2M1", MX_FMT_FP4_E2M1,
       {-8, -6, -4, -3, -2, -1.5f, -1, -0.5f, 0, 0.5f, 1, 1.5f, 2, 3, 4, 8},
       {-6, -6, -4, -3, -2, -1.5f, -1, -0.5f, 0, 0.5f, 1, 1.5f, 2, 3, 4, 6}, 8},
      {"FP8 E4M3", MX_FMT_FP8_E4M3,
       {-512, -448, -16, -0.5f, 0, 0.125f, 16, 512},
       {-448, -448, -16, -0.5f, 0, 0.125f, 16, 448}, 8},
      {"FP8 E5M2", MX_FMT_FP8_E5M2,
       {-57344, -1024, -2, -0.5f, 0, 0.25f, 1024, 57344},
       {-57344, -1024, -2, -0.5f, 0, 0.25f, 1024, 57344}, 8},
  };
  bool all = true;
  for (const KatCase& c : cases) {
    std::vector<uint8_t> packed(c.packed_bytes);
    std::vector<float> out(c.inputs.size());
    check(ctx, mx_roundtrip(ctx, c.fmt, c.inputs.data(), c.inputs.size(), packed.data(), out.data()));
    bool ok = true;
    for (size_t i = 0; i < out.size(); i++) ok = ok && out[i] == c.expected[i];
    all = all && ok;
    std::printf("\n[%s] %s\n", ok ? "ok" : "FAIL", c.name);
    std::printf("  input:    %s\n", format_values(c.inputs).c_str());
    std::printf("  unpacked: %s\n", format_values(out).c_str());
    std::printf("  expected: %s\n", format_values(c.expected).c_str());
    std::printf("  bytes:    %s\n", format_hex(packed).c_str());
  }
  return all;
}

// ---- MLP benchmark --------------------------------------------------------

struct Dev {  // device buffer owned by the driver
  mx_ctx* ctx = nullptr;
  void* p = nullptr;
  Dev(mx_ctx* c, size_t bytes) : ctx(c) { check(ctx, mx_alloc(ctx, bytes, &p)); }
  ~Dev() {
    if (p) mx_free(ctx, p);
  }
  Dev(const Dev&) = delete;
  Dev& operator=(const Dev&) = delete;
};

struct RowResult {
  std::string name;
  double seconds;
  int iterations;
  std::string checksum;
};

float half_to_float(uint16_t h) {
  const uint32_t s = (h & 0x8000u) << 16, e = (h >> 10) & 31u, m = h & 0x3ffu;
  uint32_t bits;
  if (e == 0) {
    if (m == 0) bits = s;
    else {  // subnormal
      float f = std::ldexp((float)m, -24);
      std::memcpy(&bits, &f, 4);
      bits |= s;
    }
  } else if (e == 31) {
    bits = s | 0x7f800000u | (m << 13);
  } else {
    bits = s | ((e + 112) << 23) | (m << 13);
  }
  float f;
  std::memcpy(&f, &bits, 4);
  return f;
}

// sampleFloatChecksum (:2844-2856) over an f32 or f16 output.
std::string checksum(mx_ctx* ctx, const void* dev_out, size_t count, bool f16) {
  std::vector<float> host(count);
  if (f16) {
    std::vector<uint16_t> h(count);
    check(ctx, mx_download(ctx, h.data(), dev_out, count * 2));
    for (size_t i = 0; i < count; i++) host[i] = half_to_float(h[i]);
  } else {
    check(ctx, mx_download(ctx, host.data(), dev_out, count * 4));
  }
  int samples = 0;
  const double sum = mx_checksum_f32(host.data(), count, &samples);
  char buf[96];
  std::snprintf(buf, sizeof buf, "%.6g over %d samples", sum, samples);
  return buf;
}

// printMLPBenchmarkResult (:2763-2770).
void print_row(const RowResult& r, long tokens, long hidden, long inter) {
  const double macs = 3.0 * tokens * hidden * inter * r.iterations;
  const double tops = macs * 2.0 / r.seconds / 1e12;
  std::printf("  %s:\n", r.name.c_str());
  std::printf("    %.3f ms/MLP, %.3f effective TOPS\n", r.seconds * 1000.0 / r.iterations, tops);
  std::printf("    checksum: %s\n", r.checksum.c_str());
  std::fflush(stdout);
}

// printRelativeSlowdowns (:2772-2783).
void print_slowdowns(const std::vector<RowResult>& rows) {
  if (rows.empty()) return;
  const RowResult* best = &rows[0];
  for (const RowResult& r : rows)
    if (r.seconds / r.iterations < best->seconds / best->iterations) best = &r;
  const double b = best->seconds / best->iterations;
  std::printf("  relative slowdown, best = %s:\n", best->name.c_str());
  for (const RowResult& r : rows) std::printf("    %s: %.2fx\n", r.name.c_str(), (r.seconds / r.iterations) / b);
}

void run_mlp_benchmark(mx_ctx* ctx, long tokens, long hidden, long inter, long iterations) {
  std::printf("\nGated MLP benchmark:\n");
  std::printf("  op: down(silu(gate(x)) * up(x))\n");
  std::printf("  shape: tokens=%ld, hidden=%ld, intermediate=%ld\n", tokens, hidden, inter);
  std::printf("  iterations: %ld\n", iterations);
  const size_t T = tokens, H = hidden, I = inter;
  const mx_mlp_config cfg{(uint32_t)T, (uint32_t)H, (uint32_t)I};
  const int iters = (int)iterations;

  // Reference inputs (main.swift:611-638).
  std::vector<uint16_t> x_host(T * H);
  mx_lcg_half(0x11112222u, x_host.size(), 0.125f, x_host.data());
  Dev x(ctx, T * H * 2), out(ctx, T * H * 4);
  check(ctx, mx_upload(ctx, x.p, x_host.data(), x_host.size() * 2));

  std::vector<RowResult> rows;
  auto record = [&](RowResult r) {
    print_row(r, tokens, hidden, inter);
    rows.push_back(std::move(r));
  };

  // MXFP4 rows run whenever hidden and intermediate are multiples of 32, as
  // the reference's (main.swift:1043).
  if (H % 32 == 0 && I % 32 == 0) {
    const uint8_t pattern[] = {124, 125, 126, 127, 127, 128, 128, 129, 130};
    const uint32_t data_seeds[3] = {0xabcd1357u, 0x2468bdf0u, 0x0badcafeu};
    const uint32_t scale_seeds[3] = {0x7777ddddu, 0x8888eeeeu, 0x9999ffffu};
    const size_t elems = I * H;
    Dev q0(ctx, elems / 2), q1(ctx, elems / 2), q2(ctx, elems / 2);
    Dev s0(ctx, elems / 32), s1(ctx, elems / 32), s2(ctx, elems / 32);
    Dev* qs[3] = {&q0, &q1, &q2};
    Dev* ss[3] = {&s0, &s1, &s2};
    std::vector<uint8_t> host(elems / 2);
    for (int m = 0; m < 3; m++) {
      mx_lcg_bytes(data_seeds[m], elems / 2, host.data());
      check(ctx, mx_upload(ctx, qs[m]->p, host.data(), elems / 2));
      mx_lcg_pattern(scale_seeds[m], elems / 32, pattern, 9, host.data());
      check(ctx, mx_upload(ctx, ss[m]->p, host.data(), elems / 32));
    }
    const mx_mlp_weights w{{q0.p, s0.p}, {q1.p, s1.p}, {q2.p, s2.p}};
    struct Variant {
      int id;
      const char* name;
      bool f16_out;
    };
    const Variant variants[] = {
        {MX_MLP_REFROW,
         "MXFP4 fused (FP4 + E8M0 decoded in registers, fp16 MFMA, reference epilogue): h_mxfp4_f", false},
        {MX_MLP_FUSED, "MXFP4 fused (plain SwiGLU, fp16 out): h_mxfp4_h", true},
        {MX_MLP_DEQUANT, "MXFP4 dequant (v_cvt_scalef32_pk_f16_fp4 -> half) + h_h_f", true},
        {MX_MLP_W4A4, "MXFP4 W4A4 (x, mid -> MXFP4; FP4 x FP4 scaled MFMA): fp4_fp4_h", true},
        {MX_MLP_SCALED, "MXFP4 scaled MFMA (x, mid -> two E4M3 terms; FP8 x FP4 scaled MFMA): h_mxfp4_h", true},
    };
    for (const Variant& v : variants) {
      if (v.id == MX_MLP_W4A4 && (H % 128 || I % 128)) {
        std::printf("  W4A4 row: skipped; hidden and intermediate must be multiples of 128.\n");
        continue;
      }
      if (v.id == MX_MLP_SCALED && (H % 64 || I % 64)) {
        std::printf("  scaled-MFMA row: skipped; hidden and intermediate must be multiples of 64.\n");
        continue;
      }
      double secs = 0.0;
      // warm-up 1, then `iterations` back to back from one graph (the
      // reference encodes them into one command buffer, :2062-2117)
      check(ctx, mx_mlp_benchmark(ctx, v.id, &cfg, x.p, &w, 1, out.p, 1, iters, 1, &secs, nullptr, nullptr));
      record({v.name, secs, iters, checksum(ctx, out.p, T * H, v.f16_out)});
    }
  } else {
    std::printf("  MXFP4 rows: skipped; hidden and intermediate must be multiples of 32.\n");
  }

  if (H % 32 == 0 && I % 32 == 0) {
    struct Fmt {
      int id;
      const char* name;
    };
    const Fmt fmts[] = {
        {MX_WFMT_FP8_E4M3, "FP8 E4M3 weights (row scale): h_fp8_h"},
        {MX_WFMT_FP8_E5M2, "FP8 E5M2 weights (row scale): h_fp8e5m2_h"},
        {MX_WFMT_INT8, "INT8 weights (row scale): h_i8_h"},
        {MX_WFMT_INT4, "INT4 weights (f16 scale per 32): h_i4_h"},
        {MX_WFMT_W8A8, "W8A8 MLP: i8 x int8_t -> i32"},
    };
    Dev wf(ctx, I * H * 4);
    for (const Fmt& f : fmts) {
      if (f.id == MX_WFMT_W8A8 && (H % 128 || I % 128)) {
        std::printf("  W8A8 row: skipped; hidden and intermediate must be multiples of 128.\n");
        continue;
      }
      const bool i4 = f.id == MX_WFMT_INT4;
      const size_t qb = i4 ? I * H / 2 : I * H;
      Dev q0(ctx, qb), q1(ctx, qb), q2(ctx, qb);
      const size_t sb_gu = i4 ? I * (H / 32) * 2 : I * 4, sb_dn = i4 ? H * (I / 32) * 2 : H * 4;
      Dev s0(ctx, sb_gu), s1(ctx, sb_gu), s2(ctx, sb_dn);
      Dev* qs[3] = {&q0, &q1, &q2};
      Dev* ss[3] = {&s0, &s1, &s2};
      for (int m = 0; m < 3; m++) {
        const int rows_n = m < 2 ? (int)I : (int)H, k = m < 2 ? (int)H : (int)I;
        check(ctx, mx_fill_normal(ctx, wf.p, MX_DTYPE_F32, (size_t)rows_n * k, 0x5eed0000ull + 16 * f.id + m, 0.0f,
                                  0.02f));
        check(ctx, mx_fmt_quantize(ctx, f.id, static_cast<const float*>(wf.p), rows_n, k, qs[m]->p, ss[m]->p));
      }
      const mx_mlp_weights w{{q0.p, s0.p}, {q1.p, s1.p}, {q2.p, s2.p}};
      double secs = 0.0;
      check(ctx, mx_fmt_mlp_benchmark(ctx, f.id, &cfg, x.p, &w, 1, out.p, 1, iters, 1, &secs, nullptr, nullptr));
      record({f.name, secs, iters, checksum(ctx, out.p, T * H, true)});
    }
  }
  print_slowdowns(rows);
}

// ---- big matmul benchmark ---------------------------------------------------
// runBigMatmulBenchmark (main.swift:380-584): the reference's scalar
// one-thread-per-output matmul rows, here on the matrix cores through
// mx_accum_gemm, with the reference's data generators, timing span (device
// time of `iterations` back-to-back matmuls, :1761-1779) and checksums.
// --fp4-group-sweep asks for the g8 rows as well; the unpack group width is a
// property of Metal's packed_numeric decode, and on MI355X FP4 feeds the
// matrix cores directly, so g8 and g16 are one kernel: the sweep prints each
// kernel once, named for both widths.

std::string format_mib(size_t bytes) {  // formatBytes (:2894-2897)
  char buf[64];
  std::snprintf(buf, sizeof buf, "%.2f MiB", bytes / (1024.0 * 1024.0));
  return buf;
}

void run_matmul_benchmark(mx_ctx* ctx, long rows, long columns, long depth, long iterations, bool sweep) {
  const size_t R = rows, C = columns, D = depth;
  std::printf("\nBig packed matmul benchmark:\n");
  std::printf("  shape: A %ldx%ld, B %ldx%ld, C %ldx%ld\n", rows, depth, depth, columns, rows, columns);
  std::printf("  packed A bytes: %s, packed B^T bytes: %s\n", format_mib(R * D / 2).c_str(), format_mib(C * D / 2).c_str());
  std::printf("  half A bytes: %s\n", format_mib(R * D * 2).c_str());
  std::printf("  iterations: %ld\n", iterations);
  if (sweep)
    std::printf("  FP4 unpack group sweep: 8 and 16 elements (one kernel here: FP4 goes to the matrix cores "
                "without a grouped unpack)\n");

  // Reference inputs (:408-412).
  std::vector<uint8_t> a_bytes(R * D / 2), b_bytes(C * D / 2);
  std::vector<uint16_t> a_half(R * D), b_half(C * D);
  std::vector<int8_t> a_i8(R * D);
  mx_lcg_bytes(0x12345678u, a_bytes.size(), a_bytes.data());
  mx_lcg_bytes(0x87654321u, b_bytes.size(), b_bytes.data());
  mx_lcg_half(0x2468ace0u, a_half.size(), 0.25f, a_half.data());
  mx_lcg_int8(0x13579bdfu, a_i8.size(), a_i8.data());
  mx_lcg_half(0xfdb97531u, b_half.size(), 0.03125f, b_half.data());
  Dev a(ctx, a_bytes.size()), b(ctx, b_bytes.size()), ah(ctx, a_half.size() * 2), bh(ctx, b_half.size() * 2),
      a8(ctx, a_i8.size()), out(ctx, R * C * 4);
  check(ctx, mx_upload(ctx, a.p, a_bytes.data(), a_bytes.size()));
  check(ctx, mx_upload(ctx, b.p, b_bytes.data(), b_bytes.size()));
  check(ctx, mx_upload(ctx, ah.p, a_half.data(), a_half.size() * 2));
  check(ctx, mx_upload(ctx, bh.p, b_half.data(), b_half.size() * 2));
  check(ctx, mx_upload(ctx, a8.p, a_i8.data(), a_i8.size()));

  enum Sum { SUM_F32, SUM_F16RAW, SUM_I32 };
  std::vector<RowResult> rows_out;
  auto run_row = [&](const char* name, int a_fmt, const Dev& pa, int b_fmt, const Dev& pb, int c_dtype, Sum sum) {
    const int m = (int)rows, n = (int)columns, k = (int)depth;
    check(ctx, mx_accum_gemm(ctx, a_fmt, pa.p, b_fmt, pb.p, out.p, c_dtype, m, n, k));  // warm-up
    check(ctx, mx_memset(ctx, out.p, 0, R * C * 4));
    double secs = 0.0;
    check(ctx, mx_timer_start(ctx));
    for (long i = 0; i < iterations; i++) check(ctx, mx_accum_gemm(ctx, a_fmt, pa.p, b_fmt, pb.p, out.p, c_dtype, m, n, k));
    check(ctx, mx_timer_stop(ctx, &secs));
    std::string cs;
    char buf[96];
    int samples = 0;
    if (sum == SUM_F32) {
      cs = checksum(ctx, out.p, R * C, false);
    } else if (sum == SUM_F16RAW) {
      std::vector<uint16_t> h(R * C);
      check(ctx, mx_download(ctx, h.data(), out.p, h.size() * 2));
      const unsigned long long v = mx_checksum_f16raw(h.data(), h.size(), &samples);
      std::snprintf(buf, sizeof buf, "raw16 sum %llu over %d samples", v, samples);
      cs = buf;
    } else {
      std::vector<int32_t> h(R * C);
      check(ctx, mx_download(ctx, h.data(), out.p, h.size() * 4));
      const long long v = mx_checksum_i32(h.data(), h.size(), &samples);
      std::snprintf(buf, sizeof buf, "%lld over %d samples", v, samples);
      cs = buf;
    }
    rows_out.push_back({name, secs, (int)iterations, cs});
  };
  run_row(sweep ? "FP4 E2M1 g8/g16 -> FP32 accumulate" : "FP4 E2M1 g16 -> FP32 accumulate", MX_PROBE_FP4, a,
          MX_PROBE_FP4, b, MX_DTYPE_F32, SUM_F32);
  run_row(sweep ? "half x FP4 E2M1 g8/g16 -> half accumulate" : "half x FP4 E2M1 g16 -> half accumulate",
          MX_PROBE_F16, ah, MX_PROBE_FP4, b, MX_DTYPE_F16, SUM_F16RAW);
  run_row("half x INT4 -> half accumulate", MX_PROBE_F16, ah, MX_PROBE_INT4, b, MX_DTYPE_F16, SUM_F16RAW);
  run_row("INT8 x half -> half accumulate", MX_PROBE_I8, a8, MX_PROBE_F16, bh, MX_DTYPE_F16, SUM_F16RAW);
  run_row("INT4 x INT4 -> INT32 accumulate", MX_PROBE_INT4, a, MX_PROBE_INT4, b, MX_DTYPE_I32, SUM_I32);
  for (const RowResult& r : rows_out) {  // printMatmulBenchmarkResult (:2754-2761)
    const double tops = 2.0 * R * C * D * r.iterations / r.seconds / 1e12;
    std::printf("  %s:\n", r.name.c_str());
    std::printf("    %.3f ms/matmul, %.3f effective TOPS\n", r.seconds * 1000.0 / r.iterations, tops);
    std::printf("    checksum: %s\n", r.checksum.c_str());
  }
  print_slowdowns(rows_out);
  std::fflush(stdout);
}

// ---- accumulator precision / overflow probe -------------------------------
// runAccumulatorProbe (main.swift:1523-1713): constant-fill 64 x 128 GEMMs of
// dot length K with a half and a float destination, for half x half,
// half x FP4, FP4 x FP4 and FP8 E4M3 x FP8 E4M3 (mx_accum_gemm).  Every C
// element has the same exact value, so C[0] against K * product isolates the
// accumulator and destination rounding.

std::string format_value(double v) {  // formatValue (:1647-1658)
  char buf[64];
  if (std::isinf(v)) return v < 0 ? "-inf" : "inf";
  if (std::isnan(v)) return "nan";
  if (v == std::nearbyint(v) && std::fabs(v) < 1e15) std::snprintf(buf, sizeof buf, "%.0f", v);
  else std::snprintf(buf, sizeof buf, "%.6g", v);
  return buf;
}

void run_accum_probe(mx_ctx* ctx) {
  const int m = 64, n = 128, max_k = 131072;
  auto half_fill = [&](size_t count, uint16_t bits) {
    std::vector<uint16_t> h(count, bits);
    auto d = std::make_unique<Dev>(ctx, count * 2);
    check(ctx, mx_upload(ctx, d->p, h.data(), count * 2));
    return d;
  };
  auto byte_fill = [&](size_t count, int value) {
    auto d = std::make_unique<Dev>(ctx, count);
    check(ctx, mx_memset(ctx, d->p, value, count));
    return d;
  };
  // 0x3c00 = half 1.0, 0x4800 = half 8.0; bytes 0x22 = two FP4 1.0,
  // 0x77 = two FP4 6.0, 0x38 = E4M3 1.0, 0x58 = E4M3 16.0 (:1545-1547)
  const auto a_h1 = half_fill((size_t)m * max_k, 0x3c00), b_h1 = half_fill((size_t)n * max_k, 0x3c00);
  const auto a_h8 = half_fill((size_t)m * max_k, 0x4800), b_h8 = half_fill((size_t)n * max_k, 0x4800);
  const auto a_q1 = byte_fill((size_t)m * max_k / 2, 0x22), b_q1 = byte_fill((size_t)n * max_k / 2, 0x22);
  const auto a_q6 = byte_fill((size_t)m * max_k / 2, 0x77), b_q6 = byte_fill((size_t)n * max_k / 2, 0x77);
  const auto a_e1 = byte_fill((size_t)m * max_k, 0x38), b_e1 = byte_fill((size_t)n * max_k, 0x38);
  const auto a_e16 = byte_fill((size_t)m * max_k, 0x58), b_e16 = byte_fill((size_t)n * max_k, 0x58);
  Dev c_half(ctx, (size_t)m * n * 2), c_float(ctx, (size_t)m * n * 4);

  struct Path {
    const char* name;
    int a_fmt, b_fmt;
    const Dev* a;
    const Dev* b;
    double product;
  };
  // (first, last) of C for one case
  auto run_case = [&](const Path& p, int k, bool half) {
    const Dev& c = half ? c_half : c_float;
    const size_t bytes = (size_t)m * n * (half ? 2 : 4);
    check(ctx, mx_memset(ctx, c.p, 0, bytes));
    check(ctx, mx_accum_gemm(ctx, p.a_fmt, p.a->p, p.b_fmt, p.b->p, c.p, half ? MX_DTYPE_F16 : MX_DTYPE_F32, m,
                             n, k));
    if (half) {
      std::vector<uint16_t> h((size_t)m * n);
      check(ctx, mx_download(ctx, h.data(), c.p, bytes));
      return std::make_pair((double)half_to_float(h.front()), (double)half_to_float(h.back()));
    }
    std::vector<float> f((size_t)m * n);
    check(ctx, mx_download(ctx, f.data(), c.p, bytes));
    return std::make_pair((double)f.front(), (double)f.back());
  };
  auto sweep = [&](const Path& p, const std::vector<int>& ks) {
    std::printf("\n  %s, product per element = %s:\n", p.name, format_value(p.product).c_str());
    std::printf("    K | exact | half dest C[0] | float dest C[0]\n");
    for (int k : ks) {
      const auto hv = run_case(p, k, true);
      const auto fv = run_case(p, k, false);
      std::string note;
      if (!(hv.first == hv.second && fv.first == fv.second))
        note = "  [non-uniform: half last " + format_value(hv.second) + ", float last " +
               format_value(fv.second) + "]";
      std::printf("    %d | %s | %s | %s%s\n", k, format_value(p.product * k).c_str(),
                  format_value(hv.first).c_str(), format_value(fv.first).c_str(), note.c_str());
      std::fflush(stdout);
    }
  };

  std::printf("\nAccumulator precision/overflow probe (64x128 tile, dot length K):\n");
  std::printf("  All inputs are constant fills, so every C element has the same exact value.\n");
  std::printf("  A deviation in 'half dest' but not 'float dest' isolates destination/accumulator precision.\n");
  const std::vector<int> ones_ks = {1024, 2048, 2080, 4096, 4160, 8192, 16384, 32768, 65504, 65536, 131072};
  sweep({"half x half -> C, ones", MX_PROBE_F16, MX_PROBE_F16, a_h1.get(), b_h1.get(), 1.0}, ones_ks);
  sweep({"half x FP4 E2M1 -> C, ones", MX_PROBE_F16, MX_PROBE_FP4, a_h1.get(), b_q1.get(), 1.0}, ones_ks);
  sweep({"FP4 E2M1 x FP4 E2M1 -> C, ones", MX_PROBE_FP4, MX_PROBE_FP4, a_q1.get(), b_q1.get(), 1.0}, ones_ks);
  sweep({"FP8 E4M3 x FP8 E4M3 -> C, ones", MX_PROBE_FP8, MX_PROBE_FP8, a_e1.get(), b_e1.get(), 1.0}, ones_ks);
  std::printf("\n  Overflow cases (products sized to cross half max 65504):\n");
  sweep({"half x half -> C, 8.0 x 8.0 (product 64)", MX_PROBE_F16, MX_PROBE_F16, a_h8.get(), b_h8.get(), 64.0},
        {512, 1022, 1024, 2048});
  sweep({"FP4 E2M1 x FP4 E2M1 -> C, 6.0 x 6.0 (product 36)", MX_PROBE_FP4, MX_PROBE_FP4, a_q6.get(), b_q6.get(),
         36.0},
        {1024, 1818, 1820, 2048, 4096});
  sweep({"FP8 E4M3 x FP8 E4M3 -> C, 16.0 x 16.0 (product 256)", MX_PROBE_FP8, MX_PROBE_FP8, a_e16.get(),
         b_e16.get(), 256.0},
        {128, 254, 256, 1024});
}

}  // namespace

int main(int argc, char** argv) {
  for (int i = 1; i < argc; i++) g_args.emplace_back(argv[i]);
  mx_ctx* ctx = nullptr;
  try {
    // Argument checks of runMLPBenchmark (:592-597), done before the device
    // is opened so that a bad command line fails the same way everywhere.
    const bool mlp = has_flag("--mlp-benchmark");
    const bool bench = has_flag("--benchmark");
    const long msize = int_argument("--matmul-size", 2048);
    const long mm = int_argument("--m", msize), mn = int_argument("--n", msize), mk = int_argument("--k", msize);
    const long miters = int_argument("--iterations", 3);
    if (bench) {  // runBigMatmulBenchmark's checks (:387-392)
      if (mm <= 0 || mn <= 0 || mk <= 0 || miters <= 0) fail("Matmul sizes and iterations must be positive.");
      if (mk % 16) fail("Matmul K/depth must be a multiple of 16 for packed FP4 groups.");
    }
    const long tokens = int_argument("--mlp-tokens", 128);
    const long hidden = int_argument("--mlp-hidden", 1024);
    const long inter = int_argument("--mlp-intermediate", hidden * 4);
    const long iterations = int_argument("--mlp-iterations", 3);
    if (mlp) {
      if (tokens <= 0 || hidden <= 0 || inter <= 0 || iterations <= 0)
        fail("MLP sizes and iterations must be positive.");
      if (hidden % 16 || inter % 16)
        fail("MLP hidden and intermediate sizes must be multiples of 16 for packed FP4 weights.");
    }

    const int rc = mx_create(0, &ctx);
    if (rc != MX_OK) fail("%s", mx_status_string(rc));
    char name[256];
    int cus = 0, mhz = 0;
    check(ctx, mx_device_info(ctx, name, sizeof name, &cus, &mhz));
    std::printf("Device: %s\n", name);
    std::printf("Compute units: %d, max clock: %d MHz\n", cus, mhz);
    std::fflush(stdout);

    const bool kats_ok = run_kats(ctx);
    if (has_flag("--skip-tensor")) std::printf("Tensor creation probe: skipped by --skip-tensor.\n");
    else std::printf("Tensor creation probe: not applicable (no tensor objects on ROCm).\n");
    if (bench) run_matmul_benchmark(ctx, mm, mn, mk, miters, has_flag("--fp4-group-sweep"));
    if (mlp) run_mlp_benchmark(ctx, tokens, hidden, inter, iterations);
    if (has_flag("--accum-probe")) run_accum_probe(ctx);
    if (!kats_ok) fail("One or more packed numeric checks failed.");
    std::printf("PASS\n");
  } catch (const ProbeError& e) {
    std::fflush(stdout);
    std::fprintf(stderr, "error: %s\n", e.message.c_str());
    if (ctx) mx_destroy(ctx);
    return 1;
  }
  mx_destroy(ctx);
  return 0;
}
