// Dense epilogue: per-output-channel scale, bias and the elementwise
// activations of Enilnets/nn/activations.py:21-41, in fp32.
#pragma once

#include <hip/hip_runtime.h>

#include "enilnets_amd.h"

namespace enq {

struct Epilogue {
  int activation;
  float alpha;  // leakyrelu / elu slope (activations.py:22-27)
  float clip;   // sigmoid / softplus clip (activations.py:36-37)
};

// activations.py:21-41, one element.  relu keeps -0.0 and NaN as np.maximum
// does; softmax is a row operation and is applied by a separate kernel.
__device__ __forceinline__ float activate(float x, const Epilogue& e) {
  switch (e.activation) {
    case ENQ_ACT_RELU:
      return x < 0.0f ? 0.0f : x;
    case ENQ_ACT_LEAKYRELU:
      return x > 0.0f ? x : e.alpha * x;
    case ENQ_ACT_ELU:
      return x > 0.0f ? x : e.alpha * (expf(x) - 1.0f);
    case ENQ_ACT_SELU: {
      const float lam = 1.0507009873554804934193349852946f;
      const float alp = 1.6732632423543772848170429916717f;
      return lam * (x > 0.0f ? x : alp * (expf(x) - 1.0f));
    }
    case ENQ_ACT_GELU: {
      const float c = 0.7978845608028654f;  // sqrt(2 / pi)
      float inner = c * (x + 0.044715f * (x * x * x));
      return 0.5f * x * (1.0f + tanhf(inner));
    }
    case ENQ_ACT_SWISH:
      return x * 1.0f / (1.0f + expf(-x));
    case ENQ_ACT_MISH:
      return x * tanhf(logf(1.0f + expf(x)));
    case ENQ_ACT_SIGMOID: {
      float c = x < -e.clip ? -e.clip : (x > e.clip ? e.clip : x);
      return 1.0f / (1.0f + expf(-c));
    }
    case ENQ_ACT_TANH:
      return tanhf(x);
    case ENQ_ACT_SOFTPLUS: {
      float c = x < -e.clip ? -e.clip : (x > e.clip ? e.clip : x);
      return logf(1.0f + expf(c));
    }
    default:  // linear, and softmax's pre-activation
      return x;
  }
}

// Calls body(f) with f the activation as a callable, so the common
// activations compile into straight-line epilogues instead of a switch per
// element.
template <class Body>
__device__ __forceinline__ void with_activation(const Epilogue& ep, Body&& body) {
  switch (ep.activation) {
    case ENQ_ACT_LINEAR:
    case ENQ_ACT_SOFTMAX:
      body([](float x) { return x; });
      break;
    case ENQ_ACT_RELU:
      body([](float x) { return x < 0.0f ? 0.0f : x; });
      break;
    default:
      body([ep](float x) { return activate(x, ep); });
      break;
  }
}

// Row-wise softmax in place over an (m, n) fp32 matrix (activations.py:38-40).
void softmax_rows(float* y, int64_t m, int64_t n);

bool valid_activation(int act);

}  // namespace enq
