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
  // activation fake-quantization after the activation (forward.py:798-805):
  // ENQ_AQ_NONE, ENQ_AQ_F32 or ENQ_AQ_F64 (the arithmetic of the spec's dtype)
  int aq = ENQ_AQ_NONE;
  double aq_scale = 1.0, aq_zp = 0.0;
  float aq_qmin = 0.0f, aq_qmax = 0.0f;
};

// fake_quantize (compression/quantization.py:53-69) of one value with a
// per-tensor scale and zero point: clip(rint(x / scale + zp), qmin, qmax),
// then (q - zp) * scale; true division, NaN passes the clip.
__device__ __forceinline__ float fake_quant(float v, const Epilogue& e) {
  if (e.aq == ENQ_AQ_F64) {
    const double q = rint(double(v) / e.aq_scale + e.aq_zp);
    const double c = q < double(e.aq_qmin) ? double(e.aq_qmin)
                                            : (q > double(e.aq_qmax) ? double(e.aq_qmax) : q);
    return float((c - e.aq_zp) * e.aq_scale);
  }
  const float s = float(e.aq_scale), zp = float(e.aq_zp);
  const float q = rintf(__fdiv_rn(v, s) + zp);
  const float c = q < e.aq_qmin ? e.aq_qmin : (q > e.aq_qmax ? e.aq_qmax : q);
  return __fmul_rn(c - zp, s);
}

// activations.py GELU (tanh form), one element:
//   0.5 x (1 + tanh(u)) = x / (1 + exp(-2u)),  u = sqrt(2/pi) (x + 0.044715 x^3),
// the same function with one exponential and one reciprocal in place of tanh
// (a third of the instructions in the GEMM epilogues).  exp2 of a rounded
// argument is within |2u| 2^-24 relative; where that exceeds 2e-6 (|2u| > 33)
// the output is below 1e-13.  The reciprocal form has no cancellation in
// 1 + tanh(u) for negative x.
__device__ __forceinline__ float gelu(float x) {
  const float c2 = -2.0f * 0.7978845608028654f * 1.4426950408889634f;  // -2 sqrt(2/pi) log2(e)
  const float t = c2 * (x + 0.044715f * (x * x * x));
  return x * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(t));
}

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
    case ENQ_ACT_GELU:
      return gelu(x);
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

// activate, then the fake-quantization when the epilogue has one.
__device__ __forceinline__ float epilogue_out(float x, const Epilogue& e) {
  const float a = activate(x, e);
  return e.aq != ENQ_AQ_NONE ? fake_quant(a, e) : a;
}

// Calls body(f) with f the activation as a callable, so the common
// activations compile into straight-line epilogues instead of a switch per
// element.  FUSE_AQ instantiates the fake-quantizing variant too.  Kernels without
// register headroom (the 256 x 256 tiles) leave it out: its float64
// arithmetic next to live accumulators spills them, so their callers run the
// fake-quantization as a separate pass (gemm_epilogue / finish_rows).
template <bool FUSE_AQ, class Body>
__device__ __forceinline__ void with_activation(const Epilogue& ep, Body&& body) {
  if constexpr (FUSE_AQ) {
    if (ep.aq != ENQ_AQ_NONE) {
      // the common activations straight-line here too, not a switch per element
      switch (ep.activation) {
        case ENQ_ACT_LINEAR:
          body([ep](float x) { return fake_quant(x, ep); });
          break;
        case ENQ_ACT_RELU:
          body([ep](float x) { return fake_quant(x < 0.0f ? 0.0f : x, ep); });
          break;
        default:
          body([ep](float x) { return epilogue_out(x, ep); });
          break;
      }
      return;
    }
  }
  switch (ep.activation) {
    case ENQ_ACT_LINEAR:
    case ENQ_ACT_SOFTMAX:
      body([](float x) { return x; });
      break;
    case ENQ_ACT_RELU:
      body([](float x) { return x < 0.0f ? 0.0f : x; });
      break;
    case ENQ_ACT_GELU:
      body([](float x) { return gelu(x); });
      break;
    default:
      body([ep](float x) { return activate(x, ep); });
      break;
  }
}

// Row-wise softmax in place over an (m, n) fp32 matrix (activations.py:38-40).
void softmax_rows(float* y, int64_t m, int64_t n);

// The epilogue a GEMM applies itself: a softmax activation runs afterwards
// as a row kernel, so its fake-quantization must wait for it; a kernel that
// does not fuse the fake-quantization leaves it to finish_rows as well.
inline Epilogue gemm_epilogue(const Epilogue& ep, bool fuse_aq) {
  Epilogue e = ep;
  if (e.activation == ENQ_ACT_SOFTMAX || !fuse_aq) e.aq = ENQ_AQ_NONE;
  return e;
}

// Row softmax (if the activation is softmax) and the fake-quantization the
// GEMM did not apply, after a GEMM that ran gemm_epilogue(ep, fused_aq).
void finish_rows(float* y, int64_t m, int64_t n, const Epilogue& ep, bool fused_aq);

// y = fake_quant(x) over n values (in place allowed).
void act_quant(const float* x, int64_t n, const Epilogue& ep, float* y);

bool valid_activation(int act);
bool valid_act_quant(int mode, double scale, float qmin, float qmax);

}  // namespace enq
