// Row-wise softmax for Dense layers whose activation is "softmax"
// (Enilnets/nn/activations.py:38-40): e = exp(x - max(x)); e / sum(e); and
// the standalone activation fake-quantization pass (forward.py:798-805) for
// outputs no GEMM epilogue produces.
#include <algorithm>

#include "common.hpp"
#include "epilogue.hpp"

namespace enq {
namespace {

__global__ __launch_bounds__(256) void softmax_rows_kernel(float* __restrict__ y, int64_t n) {
  __shared__ float s_red[4];
  float* row = y + int64_t(blockIdx.x) * n;
  float mx = -__builtin_inff();
  int nan = 0;
  for (int64_t j = threadIdx.x; j < n; j += 256) {
    float v = row[j];
    if (v != v) nan = 1;
    mx = v > mx ? v : mx;
  }
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) {
    float o = __shfl_xor(mx, m, 64);
    mx = o > mx ? o : mx;
    nan |= __shfl_xor(nan, m, 64);
  }
  if ((threadIdx.x & 63) == 0) s_red[threadIdx.x / 64] = nan ? __builtin_nanf("") : mx;
  __syncthreads();
  mx = s_red[0];
  for (int i = 1; i < 4; ++i) mx = (s_red[i] > mx || s_red[i] != s_red[i]) ? s_red[i] : mx;
  __syncthreads();
  float sum = 0.f;
  for (int64_t j = threadIdx.x; j < n; j += 256) {
    float e = expf(row[j] - mx);
    row[j] = e;
    sum += e;
  }
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) sum += __shfl_xor(sum, m, 64);
  if ((threadIdx.x & 63) == 0) s_red[threadIdx.x / 64] = sum;
  __syncthreads();
  sum = s_red[0] + s_red[1] + s_red[2] + s_red[3];
  for (int64_t j = threadIdx.x; j < n; j += 256) row[j] = row[j] / sum;
}

__global__ __launch_bounds__(256) void act_quant_kernel(const float* x, int64_t n, Epilogue ep,
                                                        float* y) {
  for (int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x; i < n;
       i += int64_t(gridDim.x) * 256)
    y[i] = fake_quant(x[i], ep);
}

// 16-byte aligned x and y: workgroup b owns vectors [b * 256 * U, (b + 1) *
// 256 * U) of 4 floats, thread t the vectors b * 256 * U + u * 256 + t.  All U
// loads of a thread issue before its arithmetic and stores (indices clamped
// into the array, stores masked), so a thread's requests are in flight
// together; the last n % 4 values are done by the first threads.  x == y is
// allowed: a thread reads its own elements before writing them.
// fake_quant in float64 (a calibrated spec's float64 scale) with the
// division replaced by a multiply by the reciprocal wherever that cannot
// change the result: x * inv + zp differs from x / scale + zp by a few ulps
// (under 1e-6 for |t| < 1e9, and larger quotients clip either way), so it
// rounds to the same integer unless it lies within 1e-6 of a half-integer;
// those values take the true division.  NaN and infinities fall through to
// the same results as fake_quant.
__device__ __forceinline__ float fake_quant_f64_recip(float v, const Epilogue& e, double inv) {
  const double t = double(v) * inv + e.aq_zp;
  const double fr = t - floor(t);
  // rint keeps the sign of a zero quotient (-0.0 for small negatives)
  const double q = fabs(fr - 0.5) < 1e-6 ? rint(double(v) / e.aq_scale + e.aq_zp) : rint(t);
  const double c = q < double(e.aq_qmin) ? double(e.aq_qmin)
                                          : (q > double(e.aq_qmax) ? double(e.aq_qmax) : q);
  return float((c - e.aq_zp) * e.aq_scale);
}

template <int U, int MODE>
__global__ __launch_bounds__(256) void act_quant_vec_kernel(const float* x, int64_t n,
                                                            Epilogue ep, float* y) {
  ep.aq = MODE;
  const double inv = 1.0 / ep.aq_scale;
  auto fq = [&](float v) {
    if constexpr (MODE == ENQ_AQ_F64) return fake_quant_f64_recip(v, ep, inv);
    return fake_quant(v, ep);
  };
  const int64_t n4 = n / 4;
  const int64_t base = int64_t(blockIdx.x) * 256 * U + threadIdx.x;
  const float4* x4 = reinterpret_cast<const float4*>(x);
  float4 v[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int64_t i = base + int64_t(u) * 256;
    v[u] = x4[i < n4 ? i : n4 - 1];
  }
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int64_t i = base + int64_t(u) * 256;
    if (i < n4) {
      float4 r;
      r.x = fq(v[u].x);
      r.y = fq(v[u].y);
      r.z = fq(v[u].z);
      r.w = fq(v[u].w);
      reinterpret_cast<float4*>(y)[i] = r;
    }
  }
  if (blockIdx.x == 0 && threadIdx.x < n - 4 * n4) {
    const int64_t i = 4 * n4 + threadIdx.x;
    y[i] = fq(x[i]);
  }
}

}  // namespace

void act_quant(const float* x, int64_t n, const Epilogue& ep, float* y) {
  if (n == 0 || ep.aq == ENQ_AQ_NONE) return;
  if (n >= 4 && aligned(x, 16) && aligned(y, 16)) {
    constexpr int kUnits = 4;
    const int64_t blocks = ceil_div(n / 4, int64_t(256) * kUnits);
    ENQ_REQUIRE(blocks <= 0x7fffffff, "tensor too large");
    if (ep.aq == ENQ_AQ_F64)
      act_quant_vec_kernel<kUnits, ENQ_AQ_F64><<<unsigned(blocks), 256, 0, stream()>>>(x, n, ep, y);
    else
      act_quant_vec_kernel<kUnits, ENQ_AQ_F32><<<unsigned(blocks), 256, 0, stream()>>>(x, n, ep, y);
    check_launch("act_quant_vec_kernel");
    return;
  }
  const int64_t blocks = std::min<int64_t>(ceil_div(n, 256), int64_t(device_cu_count()) * 32);
  act_quant_kernel<<<unsigned(blocks), 256, 0, stream()>>>(x, n, ep, y);
  check_launch("act_quant_kernel");
}

void finish_rows(float* y, int64_t m, int64_t n, const Epilogue& ep, bool fused_aq) {
  const bool softmax = ep.activation == ENQ_ACT_SOFTMAX;
  if (softmax) softmax_rows(y, m, n);
  if (softmax || !fused_aq) act_quant(y, m * n, ep, y);
}

bool valid_act_quant(int mode, double scale, float qmin, float qmax) {
  if (mode == ENQ_AQ_NONE) return true;
  return (mode == ENQ_AQ_F32 || mode == ENQ_AQ_F64) && scale == scale && qmin <= qmax;
}

void softmax_rows(float* y, int64_t m, int64_t n) {
  ENQ_REQUIRE(m <= 0x7fffffff, "too many rows for softmax");
  softmax_rows_kernel<<<unsigned(m), 256, 0, stream()>>>(y, n);
  check_launch("softmax_rows_kernel");
}

bool valid_activation(int act) { return act >= ENQ_ACT_LINEAR && act <= ENQ_ACT_SOFTMAX; }

}  // namespace enq

using namespace enq;

extern "C" int enq_act_quant(const float* x, int64_t n, int mode, double scale, double zero_point,
                             float qmin, float qmax, float* y) {
  return guarded([&] {
    require_init();
    ENQ_REQUIRE(n >= 0, "n must be non-negative");
    ENQ_REQUIRE(mode == ENQ_AQ_F32 || mode == ENQ_AQ_F64, "unknown act-quant mode %d", mode);
    ENQ_REQUIRE(valid_act_quant(mode, scale, qmin, qmax), "invalid act-quant parameters");
    if (n == 0) return;
    ENQ_REQUIRE(x && y, "NULL pointer argument");
    Epilogue ep{ENQ_ACT_LINEAR, 0.0f, 0.0f};
    ep.aq = mode;
    ep.aq_scale = scale;
    ep.aq_zp = zero_point;
    ep.aq_qmin = qmin;
    ep.aq_qmax = qmax;
    act_quant(x, n, ep, y);
  });
}
