// Internal entry points shared between translation units: the W8 Dense
// pieces that the layer-level operations (attention, mixture of experts)
// compose.
#pragma once

#include <cstdint>

#include "epilogue.hpp"
#include "tiling.hpp"

namespace enq {

// act(x @ (codes * w_scale).T + bias), fp32 x of shape (m, k); z receives the
// pre-activation when non-null.  Uses the kernel workspace slot, or with
// `no_alloc` the fixed scratch (noalloc_scratch), checked before any launch.
void dense_w8(const float* x, int64_t m, int64_t k, const int8_t* codes, const float* w_scale,
              int64_t n, const float* bias, const Epilogue& ep, int variant, float* y, float* z,
              bool no_alloc = false);

// x rows (gathered through `gather` when non-null) -> `planes` bf16 planes of
// shape (mp, kp), zero padded; plane p starts at xa + p * mp * kp.
void split_planes(const float* x, const int* gather, int64_t m, int64_t k, uint16_t* xa,
                  int64_t mp, int64_t kp, int planes);

// K padding of the planes the LDS-tiled GEMM reads.
int64_t gemm_k_pad(int64_t k);

// fp32-accurate split of the large-tile W8 GEMM (gemm_w8_f8.hip): x (m, k)
// -> fp16 high parts (m, kp), e4m3 low parts (m, kp) and a power-of-two row
// exponent (m int32), packed in that order into f16f8_bytes(m, k) bytes;
// kp = f16f8_k_pad(k).
int64_t f16f8_k_pad(int64_t k);
size_t f16f8_bytes(int64_t m, int64_t k);
bool f16f8_supported(int64_t k, const int8_t* codes);
// Row r of the split comes from row gather[r] of x (nullptr: row r).  With
// `bound` (f16f8_bound_params' two floats on the device), exps2[r] receives
// the exponent of a split of a Dense output computed from row r, bounded by
// ||x_r||_2 * bound[0] + bound[1].
void split_f16f8(const float* x, int64_t m, int64_t k, void* buf, const int* gather = nullptr,
                 const float* bound = nullptr, int* exps2 = nullptr);
// The two constants of that bound for the Dense with codes (rows, k), scales
// w_scale and bias (rows values or nullptr) under the epilogue's activation,
// written to out[0..1]; out[2 .. 2 + kBoundParts) is scratch.
constexpr int kBoundParts = 1024;
void f16f8_bound_params(const int8_t* codes, int64_t rows, int64_t k, const float* w_scale,
                        const float* bias, const Epilogue& ep, float* out);
// The same with the kBoundParts scratch floats at `part` instead of out + 2.
void f16f8_bound_params(const int8_t* codes, int64_t rows, int64_t k, const float* w_scale,
                        const float* bias, const Epilogue& ep, float* out, float* part);
// Row-grouped GEMM on split activations (256 x 256 tiles); with `out_split`
// the activated (m, n) output is written as the next GEMM's split (n a
// multiple of 64) with the exponents already in out_split's exponent array.
// ksplit > 1 (linear epilogue, y output): K in that many parts, part p's
// sums (bias in part 0 only) at y + p * m * n, for the caller to add.
void gemm_w8_f16f8_grouped(const void* buf, int64_t m, int64_t k, const int8_t* codes,
                           const float* w_scale, int64_t n, const float* bias,
                           const RowGroups& grp, const Epilogue& ep, float* y, void* out_split,
                           int ksplit = 1);
// act(x @ (codes * w_scale).T + bias) from split_f16f8's buffer; the
// epilogue's fake-quantization is not applied (gemm_epilogue(ep, false)).
void gemm_w8_f16f8(const void* buf, int64_t m, int64_t k, const int8_t* codes,
                   const float* w_scale, int64_t n, const float* bias, const Epilogue& ep,
                   float* y, float* z);

// Whether the grouped GEMM takes weights of this K and alignment.
bool grouped_gemm_supported(int64_t k, const int8_t* codes);

// GEMM over pre-split planes with rows in groups (`grp`), group g using
// codes + g * grp.w_stride and w_scale / bias + g * grp.v_stride.  With `yp`
// the (m, n) output is written as bf16 planes of the same split and layout
// (plane p at yp + p * yp_plane_stride, rows of n; n a multiple of 32),
// ready for the next grouped GEMM, instead of as fp32 into y.
void dense_w8_grouped(const uint16_t* xa, int64_t plane_stride, int64_t kp, int planes,
                      int64_t m, int64_t k, const int8_t* codes, const float* w_scale, int64_t n,
                      const float* bias, const RowGroups& grp, const Epilogue& ep, float* y,
                      uint16_t* yp = nullptr, int64_t yp_plane_stride = 0);

}  // namespace enq
