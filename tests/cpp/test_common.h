// test_common.h -- shared helpers of the C++ mirror tests: the oracle's C
// entry points (the checker), a seeded generator, random GGUF blocks,
// device buffers and the row-norm tolerance check.
#ifndef IFX_TEST_COMMON_H
#define IFX_TEST_COMMON_H

#include <hip/hip_runtime.h>

#include <array>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <string>
#include <vector>

#include "../../include/ifx_fused_quant_gemm.h"
#include "../../include/ifx_qgemm.h"

extern "C" {
int orc_block_bytes(int qtype);
int orc_block_elems(int qtype);
uint16_t orc_f32_to_f16(float f);
float orc_f16_to_f32(uint16_t h);
int orc_quantize_q8_1_f32(const float *x, void *out, int64_t M, int64_t K);
int orc_rmsnorm_quantize_q8_1(const float *x, const uint16_t *w, void *out, int64_t M, int64_t K,
                              float eps);
int orc_silu_mul_quantize_q8_1(const float *g, const float *u, void *out, int64_t M, int64_t K);
int orc_gemv_exact(int qtype, const void *W, const void *A, double *y, int M, int N, int K,
                   int threads);
int orc_quantize_rows_symmetric(const float *x, int8_t *codes, float *scales, int64_t M, int64_t K);
int orc_gemv_packed_exact(int qtype, const void *W, const int8_t *codes, const float *scales,
                          double *y, int M, int N, int K, int threads);
}

using inferflux::rocm::FusedDispatchGeometry;
using inferflux::rocm::FusedQuantGemm;
using inferflux::rocm::KernelFamily;
using inferflux::rocm::NativeExecutionPolicy;
using inferflux::rocm::PackedActivationInfo;
using inferflux::rocm::PackedProjectionSpec;
using inferflux::rocm::QuantizedWeightInfo;

namespace {

int g_failures = 0;

#define EXPECT(cond)                                                            \
  do {                                                                          \
    if (!(cond)) {                                                              \
      std::printf("  FAILED %s:%d: %s\n", __FILE__, __LINE__, #cond);           \
      ++g_failures;                                                             \
    }                                                                           \
  } while (0)

#define HIP_OK(x)                                                               \
  do {                                                                          \
    hipError_t e_ = (x);                                                        \
    if (e_ != hipSuccess) {                                                     \
      std::printf("  HIP error %s at %s:%d\n", hipGetErrorString(e_), __FILE__, \
                  __LINE__);                                                    \
      std::exit(2);                                                             \
    }                                                                           \
  } while (0)

constexpr int Q8_0 = 8, Q8_1 = 9, Q4_K = 12, Q6_K = 14;

// xorshift64*: the test's own seeded generator.
struct Rng {
  uint64_t s;
  explicit Rng(uint64_t seed) : s(seed * 0x9E3779B97F4A7C15ull + 1) {}
  uint64_t next() {
    s ^= s >> 12;
    s ^= s << 25;
    s ^= s >> 27;
    return s * 0x2545F4914F6CDD1Dull;
  }
  float uniform() { return (next() >> 40) * (1.0f / 16777216.0f); }
  float normal() {
    const float u1 = uniform() + 1e-7f, u2 = uniform();
    return std::sqrt(-2.0f * std::log(u1)) * std::cos(6.2831853f * u2);
  }
};

// Random blocks with finite fp16 scales: d, dmin = |N(0,1)| * 0.01.
std::vector<uint8_t> MakeBlocks(int qtype, int N, int K, uint64_t seed) {
  Rng r(seed);
  const int bb = orc_block_bytes(qtype), be = orc_block_elems(qtype);
  const int64_t nb = static_cast<int64_t>(N) * (K / be);
  std::vector<uint8_t> w(nb * bb);
  for (auto &b : w) b = static_cast<uint8_t>(r.next() >> 56);
  for (int64_t i = 0; i < nb; ++i) {
    uint8_t *blk = w.data() + i * bb;
    auto put = [&](int off) {
      const uint16_t h = orc_f32_to_f16(std::fabs(r.normal()) * 0.01f);
      std::memcpy(blk + off, &h, 2);
    };
    if (qtype == Q4_K || qtype == 13) { put(0); put(2); }  // Q4_K, Q5_K
    else if (qtype == 15) {                                   // Q8_K: fp32 d
      const float d = std::fabs(r.normal()) * 0.01f;
      std::memcpy(blk, &d, 4);
    } else if (qtype == Q6_K) {
      for (int j = 0; j < 16; ++j) blk[192 + j] = static_cast<uint8_t>(static_cast<int8_t>(r.next() % 128) - 64);
      put(208);
    } else {
      put(0);
      for (int j = 0; j < 32; ++j) blk[2 + j] = static_cast<uint8_t>(static_cast<int8_t>(r.next() % 255) - 127);
    }
  }
  return w;
}

struct Dev {
  void *p = nullptr;
  explicit Dev(size_t n) { HIP_OK(hipMalloc(&p, n ? n : 1)); }
  ~Dev() { (void)hipFree(p); }
  template <typename T> T *as() { return static_cast<T *>(p); }
};

// max_row |y - ye| <= rel * ||ye_row|| (+ fp16 output rounding when half).
bool RowsClose(const std::vector<float> &y, const std::vector<double> &ye, int M, int N,
               double rel, bool half_out) {
  for (int m = 0; m < M; ++m) {
    double nrm = 0, err = 0, mag = 0;
    for (int n = 0; n < N; ++n) {
      const double e = ye[static_cast<size_t>(m) * N + n];
      nrm += e * e;
      mag = std::fmax(mag, std::fabs(e));
      err = std::fmax(err, std::fabs(y[static_cast<size_t>(m) * N + n] - e));
    }
    const double lim = rel * std::sqrt(nrm) + (half_out ? mag * (1.0 / 1024) : 0.0);
    if (!(err <= lim)) {
      std::printf("  row %d: max err %.3e > %.3e\n", m, err, lim);
      return false;
    }
  }
  return true;
}

std::vector<float> HalfToFloat(const std::vector<uint16_t> &h) {
  std::vector<float> f(h.size());
  for (size_t i = 0; i < h.size(); ++i) f[i] = orc_f16_to_f32(h[i]);
  return f;
}

struct Problem {
  int qtype, M, N, K;
  std::vector<uint8_t> w;
  std::vector<float> x;
  std::vector<uint8_t> a;  // oracle Q8_1
  std::vector<double> ye;  // oracle fp64 product
};

Problem MakeProblem(int qtype, int M, int N, int K, uint64_t seed) {
  Problem p{qtype, M, N, K, MakeBlocks(qtype, N, K, seed), {}, {}, {}};
  Rng r(seed + 1000);
  p.x.resize(static_cast<size_t>(M) * K);
  for (auto &v : p.x) v = r.normal();
  p.a.resize(static_cast<size_t>(M) * (K / 32) * 36);
  orc_quantize_q8_1_f32(p.x.data(), p.a.data(), M, K);
  p.ye.resize(static_cast<size_t>(M) * N);
  orc_gemv_exact(qtype, p.w.data(), p.a.data(), p.ye.data(), M, N, K, 8);
  return p;
}

}  // namespace

#endif  // IFX_TEST_COMMON_H
