// A C/C++ caller of libggemm_vark.so (TEST PROGRAM): the way a C++ training framework or the
// reference's own launcher (reference launcher.cpp:47-192, which allocates with hipMalloc and
// launches on the null stream) would use the library -- headers from include/, -lggemm_vark, device
// buffers from hipMalloc, no Python. It checks the ABI version, runs the reference-signature wgrad
// (the 192-row kernel for a small shape, a wide-tile kernel for OUT_M >= 1024), the fp32 main-grad
// accumulation and the persistent fwd GEMM on contiguous K = 2880 rows, and checks every output
// against the oracle's C restatement (oracle/vark_oracle.c, linked in as the checker only) with the
// bar of the parity tests: cosine >= 0.99999, max relative error <= 2e-2 over |ref| > 1e-3 max|ref|,
// empty groups exactly zero; the accumulation bit for bit against C0 + the fp32 result. Inputs are
// seeded normal values rounded to the nearest fp8 code (the configurations' value recipe).
// Exit status 0 when every check passes; one line per check on stdout.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <random>
#include <utility>
#include <vector>

#include "../../include/ggemm_persistent.h"
#include "../../include/ggemm_vark.h"

extern "C" {
float vo_e4m3_to_f32(uint8_t b);
float vo_e5m2_to_f32(uint8_t b);
int vo_vark_tensorwise(const uint8_t* lhs, const uint8_t* rhs, float sl, float sr, const int64_t* offs, int G,
                       int64_t M, int OUT_M, int OUT_N, int64_t slm, int64_t srm, uint16_t* out_bits);
int vo_persistent_fp8(const uint8_t* a, const uint8_t* b, float sa, float sb, const int64_t* offs, int G, int64_t M,
                      int N, int K, int64_t sam, int64_t sbg, int64_t sbn, int a_e5m2, uint16_t* out_bits,
                      int64_t som);
}

namespace {

int failures = 0;

#define HIP_OK(x)                                                                        \
  do {                                                                                   \
    hipError_t e_ = (x);                                                                 \
    if (e_ != hipSuccess) {                                                              \
      std::printf("FAIL hip %s: %s\n", #x, hipGetErrorString(e_));                       \
      std::exit(2);                                                                      \
    }                                                                                    \
  } while (0)

void check(bool ok, const char* what, const char* detail) {
  std::printf("%s %s: %s\n", ok ? "ok" : "FAIL", what, detail);
  if (!ok) ++failures;
}

// Nearest fp8 code of x (finite codes only), by search over the decoded values.
struct Fp8Encoder {
  std::vector<std::pair<float, uint8_t>> table;
  explicit Fp8Encoder(bool e5m2) {
    for (int c = 0; c < 256; ++c) {
      const float v = e5m2 ? vo_e5m2_to_f32((uint8_t)c) : vo_e4m3_to_f32((uint8_t)c);
      if (std::isfinite(v)) table.emplace_back(v, (uint8_t)c);
    }
    std::sort(table.begin(), table.end());
  }
  uint8_t operator()(float x) const {
    auto it = std::lower_bound(table.begin(), table.end(), std::make_pair(x, (uint8_t)0));
    if (it == table.end()) return table.back().second;
    if (it == table.begin()) return it->second;
    auto prev = it - 1;
    return (x - prev->first <= it->first - x) ? prev->second : it->second;
  }
};

// x ~ N(0, std) quantized per tensor (scale = amax / fmax) as the configurations quantize.
std::vector<uint8_t> make_fp8(std::mt19937& rng, size_t n, float std_, bool e5m2, float* scale) {
  std::normal_distribution<float> nd(0.0f, std_);
  std::vector<float> x(n);
  float amax = 0.0f;
  for (auto& v : x) {
    v = nd(rng);
    amax = std::max(amax, std::fabs(v));
  }
  const float fmax = e5m2 ? 57344.0f : 448.0f;
  *scale = amax > 0 ? amax / fmax : 1.0f;
  Fp8Encoder enc(e5m2);
  std::vector<uint8_t> q(n);
  for (size_t i = 0; i < n; ++i) q[i] = enc(std::min(std::max(x[i] / *scale, -fmax), fmax));
  return q;
}

float bf16_to_f32(uint16_t b) {
  const uint32_t u = (uint32_t)b << 16;
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}

// The parity bar over the whole output (got / ref: bf16 bits, same layout); empty-group rows given
// as [lo, hi) element ranges of got that must be exactly zero.
void bar(const char* what, const std::vector<uint16_t>& got, const std::vector<uint16_t>& ref,
         const std::vector<std::pair<size_t, size_t>>& zero_ranges) {
  double dot = 0, na = 0, nb = 0, amax = 0, rel = 0;
  size_t nonfinite = 0;
  for (size_t i = 0; i < ref.size(); ++i) amax = std::max(amax, (double)std::fabs(bf16_to_f32(ref[i])));
  for (size_t i = 0; i < ref.size(); ++i) {
    const double a = bf16_to_f32(got[i]), b = bf16_to_f32(ref[i]);
    if (!std::isfinite(a)) ++nonfinite;
    dot += a * b;
    na += a * a;
    nb += b * b;
    if (std::fabs(b) > 1e-3 * amax) rel = std::max(rel, std::fabs(a - b) / std::fabs(b));
  }
  bool empty_zero = true;
  for (auto [lo, hi] : zero_ranges)
    for (size_t i = lo; i < hi; ++i) empty_zero &= (got[i] & 0x7fff) == 0;
  const double cos = dot / (std::sqrt(na) * std::sqrt(nb));
  char buf[200];
  std::snprintf(buf, sizeof buf, "cos %.8f max_rel %.5f nonfinite %zu empty groups zero %d", cos, rel, nonfinite,
                (int)empty_zero);
  check(cos >= 0.99999 && rel <= 2e-2 && nonfinite == 0 && empty_zero, what, buf);
}

void wgrad_case(const char* what, int OUT_M, int OUT_N, std::mt19937& rng) {
  const std::vector<int64_t> lens = {96, 160, 0, 256};
  const int G = (int)lens.size();
  std::vector<int64_t> offs(G + 1, 0);
  for (int g = 0; g < G; ++g) offs[g + 1] = offs[g] + lens[g];
  const int64_t M = offs[G];
  float sl, sr;
  const auto lhs = make_fp8(rng, (size_t)M * OUT_M, 1.0f, false, &sl);
  const auto rhs = make_fp8(rng, (size_t)M * OUT_N, 1e-3f, true, &sr);
  const size_t nc = (size_t)G * OUT_M * OUT_N;
  uint8_t *dl, *dr;
  uint16_t* dc;
  float *dsl, *dsr, *dc32;
  int64_t* doffs;
  HIP_OK(hipMalloc(&dl, lhs.size()));
  HIP_OK(hipMalloc(&dr, rhs.size()));
  HIP_OK(hipMalloc(&dc, nc * 2));
  HIP_OK(hipMalloc(&dc32, nc * 4));
  HIP_OK(hipMalloc(&dsl, 4));
  HIP_OK(hipMalloc(&dsr, 4));
  HIP_OK(hipMalloc(&doffs, offs.size() * 8));
  HIP_OK(hipMemcpy(dl, lhs.data(), lhs.size(), hipMemcpyHostToDevice));
  HIP_OK(hipMemcpy(dr, rhs.data(), rhs.size(), hipMemcpyHostToDevice));
  HIP_OK(hipMemcpy(dsl, &sl, 4, hipMemcpyHostToDevice));
  HIP_OK(hipMemcpy(dsr, &sr, 4, hipMemcpyHostToDevice));
  HIP_OK(hipMemcpy(doffs, offs.data(), offs.size() * 8, hipMemcpyHostToDevice));
  HIP_OK(hipMemset(dc, 0xff, nc * 2));   // NaN everywhere: every element must be written

  const int kernel = ggemm_vark_bf16_kernel(OUT_M, OUT_N, OUT_N, dc);
  // the reference's argument list (launcher.cpp:123-171), the null stream
  int rc = ggemm_vark_wgrad_fp8(dl, dr, dc, dsl, dsr, doffs, G, OUT_M, OUT_N, OUT_M, OUT_N, OUT_M * OUT_N, OUT_N, 1,
                                nullptr);
  HIP_OK(hipDeviceSynchronize());
  std::vector<uint16_t> got(nc), ref(nc);
  HIP_OK(hipMemcpy(got.data(), dc, nc * 2, hipMemcpyDeviceToHost));
  char name[160];
  std::snprintf(name, sizeof name, "%s wgrad %dx%d on the %s kernel (rc %d)", what, OUT_M, OUT_N,
                kernel == 320 ? "320x320" : kernel == 256 ? "256x384" : "192-row", rc);
  if (vo_vark_tensorwise(lhs.data(), rhs.data(), sl, sr, offs.data(), G, M, OUT_M, OUT_N, OUT_M, OUT_N, ref.data()))
    check(false, name, "oracle failed");
  else if (rc != 0)
    check(false, name, ggemm_vark_strerror(rc));
  else
    bar(name, got, ref, {{(size_t)2 * OUT_M * OUT_N, (size_t)3 * OUT_M * OUT_N}});

  // fp32 main-grad accumulation: C = C0 + the fp32 result, bit for bit
  std::vector<float> c0(nc), r32(nc), acc(nc);
  std::normal_distribution<float> nd(0.0f, 1.0f);
  for (auto& v : c0) v = nd(rng);
  rc = ggemm_vark_wgrad_fp8_out(dl, dr, dc32, dsl, dsr, doffs, G, OUT_M, OUT_N, OUT_M, OUT_N, OUT_M * OUT_N, OUT_N,
                                1, GGEMM_OUT_F32, M, nullptr);
  HIP_OK(hipDeviceSynchronize());
  HIP_OK(hipMemcpy(r32.data(), dc32, nc * 4, hipMemcpyDeviceToHost));
  HIP_OK(hipMemcpy(dc32, c0.data(), nc * 4, hipMemcpyHostToDevice));
  const int rc2 = ggemm_vark_wgrad_fp8_out(dl, dr, dc32, dsl, dsr, doffs, G, OUT_M, OUT_N, OUT_M, OUT_N,
                                           OUT_M * OUT_N, OUT_N, 1, GGEMM_OUT_F32_ACCUM, M, nullptr);
  HIP_OK(hipDeviceSynchronize());
  HIP_OK(hipMemcpy(acc.data(), dc32, nc * 4, hipMemcpyDeviceToHost));
  size_t diff = 0;
  for (size_t i = 0; i < nc; ++i) {
    const float want = c0[i] + r32[i];
    diff += std::memcmp(&want, &acc[i], 4) != 0;
  }
  std::snprintf(name, sizeof name, "%s fp32 accumulate %dx%d (rc %d, %d)", what, OUT_M, OUT_N, rc, rc2);
  char detail[96];
  std::snprintf(detail, sizeof detail, "%zu of %zu elements differ from C0 + result", diff, nc);
  check(rc == 0 && rc2 == 0 && diff == 0, name, detail);
  for (void* p : {(void*)dl, (void*)dr, (void*)dc, (void*)dc32, (void*)dsl, (void*)dsr, (void*)doffs})
    HIP_OK(hipFree(p));
}

void persistent_case(std::mt19937& rng) {
  const std::vector<int64_t> lens = {100, 0, 300};
  const int G = (int)lens.size(), K = 2880, N = 384;
  std::vector<int64_t> offs(G + 1, 0);
  for (int g = 0; g < G; ++g) offs[g + 1] = offs[g] + lens[g];
  const int64_t M = offs[G];
  float sa, sb;
  const auto a = make_fp8(rng, (size_t)M * K, 1.0f, false, &sa);
  const auto b = make_fp8(rng, (size_t)G * N * K, 0.02f, false, &sb);
  uint8_t *da, *db;
  uint16_t* dout;
  float *dsa, *dsb;
  int64_t* doffs;
  HIP_OK(hipMalloc(&da, a.size()));
  HIP_OK(hipMalloc(&db, b.size()));
  HIP_OK(hipMalloc(&dout, (size_t)M * N * 2));
  HIP_OK(hipMalloc(&dsa, 4));
  HIP_OK(hipMalloc(&dsb, 4));
  HIP_OK(hipMalloc(&doffs, offs.size() * 8));
  HIP_OK(hipMemcpy(da, a.data(), a.size(), hipMemcpyHostToDevice));
  HIP_OK(hipMemcpy(db, b.data(), b.size(), hipMemcpyHostToDevice));
  HIP_OK(hipMemcpy(dsa, &sa, 4, hipMemcpyHostToDevice));
  HIP_OK(hipMemcpy(dsb, &sb, 4, hipMemcpyHostToDevice));
  HIP_OK(hipMemcpy(doffs, offs.data(), offs.size() * 8, hipMemcpyHostToDevice));
  HIP_OK(hipMemset(dout, 0xff, (size_t)M * N * 2));
  const int rc = ggemm_persistent_fp8(da, db, dout, dsa, dsb, doffs, G, N, K, K, N * K, K, N, 1, GGEMM_FP8_E4M3, M,
                                      nullptr);
  HIP_OK(hipDeviceSynchronize());
  std::vector<uint16_t> got((size_t)M * N), ref((size_t)M * N, 0);
  HIP_OK(hipMemcpy(got.data(), dout, got.size() * 2, hipMemcpyDeviceToHost));
  char name[120];
  std::snprintf(name, sizeof name, "persistent fwd GEMM K=%d N=%d, contiguous rows (rc %d)", K, N, rc);
  if (vo_persistent_fp8(a.data(), b.data(), sa, sb, offs.data(), G, M, N, K, K, (int64_t)N * K, K, 0, ref.data(), N))
    check(false, name, "oracle failed");
  else if (rc != 0)
    check(false, name, ggemm_vark_strerror(rc));
  else
    bar(name, got, ref, {});
  for (void* p : {(void*)da, (void*)db, (void*)dout, (void*)dsa, (void*)dsb, (void*)doffs}) HIP_OK(hipFree(p));
}

}  // namespace

int main() {
  const int ver = ggemm_vark_abi_version();
  char detail[64];
  std::snprintf(detail, sizeof detail, "library %d, headers %d", ver, GGEMM_VARK_ABI_VERSION);
  check(ver == GGEMM_VARK_ABI_VERSION, "ABI version", detail);
  int cus = 0;
  const int rc = ggemm_vark_num_cus(0, &cus);
  std::snprintf(detail, sizeof detail, "rc %d, %d CUs", rc, cus);
  check(rc == 0 && cus > 0, "device", detail);
  std::mt19937 rng(20261202);
  wgrad_case("small", 64, 128, rng);
  wgrad_case("wide", 1280, 640, rng);
  persistent_case(rng);
  std::printf("%s: %d failed check(s)\n", failures ? "FAILED" : "PASSED", failures);
  return failures ? 1 : 0;
}
