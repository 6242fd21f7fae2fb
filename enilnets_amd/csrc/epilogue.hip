// Row-wise softmax for Dense layers whose activation is "softmax"
// (Enilnets/nn/activations.py:38-40): e = exp(x - max(x)); e / sum(e).
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

}  // namespace

void softmax_rows(float* y, int64_t m, int64_t n) {
  ENQ_REQUIRE(m <= 0x7fffffff, "too many rows for softmax");
  softmax_rows_kernel<<<unsigned(m), 256, 0, stream()>>>(y, n);
  check_launch("softmax_rows_kernel");
}

bool valid_activation(int act) { return act >= ENQ_ACT_LINEAR && act <= ENQ_ACT_SOFTMAX; }

}  // namespace enq
