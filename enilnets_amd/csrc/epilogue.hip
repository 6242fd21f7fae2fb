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

__global__ __launch_bounds__(256) void act_quant_kernel(const float* __restrict__ x, int64_t n,
                                                        Epilogue ep, float* __restrict__ y) {
  for (int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x; i < n;
       i += int64_t(gridDim.x) * 256)
    y[i] = fake_quant(x[i], ep);
}

}  // namespace

void act_quant(const float* x, int64_t n, const Epilogue& ep, float* y) {
  if (n == 0 || ep.aq == ENQ_AQ_NONE) return;
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
