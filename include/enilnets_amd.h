/*
 * enilnets_amd.h -- C ABI of libenilnets_amd.so, the MI355X (gfx950)
 * implementation of Enilnets' quantized-inference hot path.
 *
 * The reference (Enilnets v4.11.0) is pure NumPy and has no FFI; the path sits
 * behind the module functions of Enilnets/compression/quantization.py and the
 * Dense branch of Enilnets/nn/forward.py.  Each entry point below names the
 * reference expression it replaces (path:line under the reference tree).
 *
 * Conventions
 *   - Every function returns an int status: ENQ_OK (0) or one of the
 *     ENQ_ERR_* codes.  enq_last_error() gives the message of the last failure
 *     on the calling thread.
 *   - Array arguments are DEVICE pointers (from enq_malloc or any other HIP
 *     allocation on the current device) unless the name says "host".
 *   - Kernels are enqueued on the library stream (enq_get_stream /
 *     enq_set_stream) and return before they finish; enq_synchronize() waits.
 *     The copy functions are synchronous.
 *   - Tensors are dense and row-major.  A per-channel tensor is described as
 *     (outer, channels, inner): element (o, c, i) sits at (o*channels + c)*inner
 *     + i and belongs to channel c.  A per-tensor operation is channels == 1.
 *   - Weights are (n_out, n_in) as in Enilnets/nn/weight_init.py:13-14, so the
 *     Dense GEMM is y = x . W^T + b (Enilnets/nn/forward.py:318-319).
 */
#ifndef ENILNETS_AMD_H
#define ENILNETS_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ENQ_ABI_VERSION 1

/* status codes */
#define ENQ_OK 0
#define ENQ_ERR_INVALID 1     /* bad argument: maps to ValueError          */
#define ENQ_ERR_RUNTIME 2     /* HIP runtime failure: maps to RuntimeError */
#define ENQ_ERR_NO_DEVICE 3   /* no usable gfx950 device: RuntimeError     */
#define ENQ_ERR_UNSUPPORTED 4 /* valid but not implemented: NotImplementedError */

/* element types of float tensors */
#define ENQ_F32 0
#define ENQ_F64 1

/* quantization schemes, Enilnets/compression/quantization.py:25-28 */
#define ENQ_SYMMETRIC 0
#define ENQ_ASYMMETRIC 1

/* activations, Enilnets/nn/activations.py:21-41 */
#define ENQ_ACT_LINEAR 0
#define ENQ_ACT_RELU 1
#define ENQ_ACT_LEAKYRELU 2
#define ENQ_ACT_ELU 3
#define ENQ_ACT_SELU 4
#define ENQ_ACT_GELU 5
#define ENQ_ACT_SWISH 6
#define ENQ_ACT_MISH 7
#define ENQ_ACT_SIGMOID 8
#define ENQ_ACT_TANH 9
#define ENQ_ACT_SOFTPLUS 10
#define ENQ_ACT_SOFTMAX 11

/* W8 Dense arithmetic variants */
/* activation fake-quantization arithmetic (the dtype of the spec's scale
 * and zero point as NumPy promotes them with float32 outputs) */
#define ENQ_AQ_NONE 0
#define ENQ_AQ_F32 1
#define ENQ_AQ_F64 2

#define ENQ_W8_FP32 0 /* fp32-accurate: activations split into bf16 hi+lo   */
#define ENQ_W8_BF16 1 /* activations rounded to bf16 once                    */

typedef struct enq_device_info {
  char name[128];
  char arch[64];         /* e.g. "gfx950:sramecc+:xnack-" */
  int device;
  int compute_units;
  int clock_khz;
  int memory_clock_khz;
  int memory_bus_width;
  int l2_bytes;
  int lds_bytes_per_block;
  int wavefront_size;
  long long global_memory_bytes;
} enq_device_info;

/* ---- lifecycle ------------------------------------------------------- */
int enq_abi_version(void);
/* Select `device`, check it is gfx950, create the library stream. */
int enq_init(int device);
int enq_get_device_info(enq_device_info* out);
int enq_synchronize(void);
const char* enq_last_error(void);
/* The stream kernels are launched on (a hipStream_t). */
int enq_get_stream(void** stream);
/* Launch on a caller-owned stream instead (NULL restores the library's). */
int enq_set_stream(void* stream);

/* HIP graph of a fixed sequence of calls, for callers that repeat it (a
 * serving loop's layer): enq_graph_begin starts capturing the library
 * stream; the calls that follow are recorded, not run; enq_graph_end stops
 * and instantiates the graph (an error if a recorded call failed or
 * synchronised); enq_graph_launch replays it on the library stream;
 * enq_graph_destroy waits for the stream and frees it.  Run every call once
 * before capturing it: while a graph is alive the library's workspace does
 * not grow (a call needing more fails with ENQ_ERR_INVALID), and the
 * buffers the recorded calls use must stay allocated.  No counterpart in
 * the reference. */
int enq_graph_begin(void);
int enq_graph_end(void** graph);
int enq_graph_launch(void* graph);
int enq_graph_destroy(void* graph);

/* ---- device memory -------------------------------------------------- */
/* Device buffers from a caching allocator: enq_free keeps the block for the
 * next enq_malloc of its size class instead of returning it to HIP (work
 * already enqueued on the library stream may still use it; later work on
 * the same stream is ordered after it).  No counterpart in the reference,
 * which holds NumPy arrays on the host. */
int enq_malloc(void** dptr, size_t bytes);
int enq_free(void* dptr);
/* Synchronises the stream and returns every cached idle block to HIP. */
int enq_release_cached_memory(void);
int enq_copy_to_device(void* dst, const void* host_src, size_t bytes);
int enq_copy_to_host(void* host_dst, const void* src, size_t bytes);
int enq_copy_on_device(void* dst, const void* src, size_t bytes);

/* ---- timing (HIP events recorded on the library stream) ----------- */
int enq_event_create(void** event);
int enq_event_destroy(void* event);
int enq_event_record(void* event);
int enq_event_elapsed_ms(void* start, void* end, float* ms);

/* ---- quantization primitives ---------------------------------------
 * dtype is ENQ_F32 or ENQ_F64 for x, scale, zero_point, low, high and the
 * float outputs.  qmin/qmax come from quant_range
 * (Enilnets/compression/quantization.py:21-30).
 */

/* Per-channel min and max (NaN-propagating like np.min/np.max).
 * Replaces np.min/np.max(w, axis=all-but-axis, keepdims=True) and the global
 * np.min(w)/np.max(w) of quantize_tensor, quantization.py:86-91.
 * low/high hold `channels` values. */
int enq_minmax(int dtype, const void* x, int64_t outer, int64_t channels,
               int64_t inner, void* low, void* high);

/* Elementwise scale and zero point from ranges.
 * Replaces compute_scale, quantization.py:33-50. */
int enq_compute_scale(int dtype, const void* low, const void* high, int64_t n,
                      int bits, int scheme, void* scale, void* zero_point);

/* codes = clip(round_half_even(x / scale + zero_point), qmin, qmax), as floats
 * of `dtype`.  Replaces quantize, quantization.py:53-56.  scale/zero_point hold
 * `channels` values. */
int enq_quantize(int dtype, const void* x, int64_t outer, int64_t channels,
                 int64_t inner, const void* scale, const void* zero_point,
                 int qmin, int qmax, void* codes);

/* The codes of enq_quantize stored as int8 (NaN -> 0): quantize,
 * quantization.py:53-56, with a given scale.  Requires -128 <= qmin <= qmax
 * <= 127.  Used to rebuild int8 weight codes from fake-quantized floats and
 * their stored scale. */
int enq_quantize_codes_i8(int dtype, const void* x, int64_t outer,
                          int64_t channels, int64_t inner, const void* scale,
                          const void* zero_point, int qmin, int qmax,
                          int8_t* codes);

/* out = (q - zero_point) * scale.  Replaces dequantize, quantization.py:59-61. */
int enq_dequantize(int dtype, const void* q, int64_t outer, int64_t channels,
                   int64_t inner, const void* scale, const void* zero_point,
                   void* out);

/* dequantize(quantize(x)).  Replaces fake_quantize, quantization.py:64-69. */
int enq_fake_quantize(int dtype, const void* x, int64_t outer, int64_t channels,
                      int64_t inner, const void* scale, const void* zero_point,
                      int qmin, int qmax, void* out);

/* Fused quantize_tensor: statistics, scale, zero point and the fake-quantized
 * tensor in one call.  Replaces quantize_tensor, quantization.py:76-93
 * (channels == 1 is the per-tensor branch :90-91).
 *   out_fake   (nullable) fake-quantized tensor of `dtype`
 *   out_codes  (nullable) the same codes as int8; requires qmin >= -128 and
 *              qmax <= 127; a NaN element gets code 0
 *   scale, zero_point  `channels` values of `dtype`
 *   abs_err    (nullable) one double: sum |fake - w| over the tensor, the
 *              numerator of quantize_weights' mean_abs_error (:137) */
int enq_quantize_tensor(int dtype, const void* w, int64_t outer,
                        int64_t channels, int64_t inner, int bits, int scheme,
                        void* out_fake, int8_t* out_codes, void* scale,
                        void* zero_point, double* abs_err);

/* Symmetric 8-bit per-row quantization of fp32 rows to int8 codes plus one
 * fp32 scale per row: quantize_tensor(x, 8, "symmetric", per_channel=True)
 * (quantization.py:76-93) with the codes kept as int8.  Used for the
 * per-output-channel weight codes and for per-token activation codes. */
int enq_quantize_rows_i8(const float* x, int64_t rows, int64_t cols,
                         int8_t* codes, float* scale);

/* Int8 codes back to floats: out = code * scale, scale per channel.
 * Replaces dequantize (quantization.py:59-61) for symmetric int8 storage. */
int enq_dequantize_i8(int dtype, const int8_t* codes, int64_t outer,
                      int64_t channels, int64_t inner, const void* scale,
                      void* out);

/* Sums for quantization_error (quantization.py:218-229) over n elements:
 * out[0] = sum|b-a|, out[1] = max|b-a|, out[2] = sum a*a, out[3] = sum (b-a)^2,
 * accumulated in double. */
int enq_error_stats(int dtype, const void* reference, const void* candidate,
                    int64_t n, double* host_out4);

/* Order statistics for ActivationCalibrator(percentile=p)
 * (quantization.py:183-188, np.percentile(out, 100 - p) and
 * np.percentile(out, p)): out[i] = the element at position host_ranks[i]
 * (0 <= rank < n) of x (n elements of dtype) sorted ascending, NaN after
 * every number, as np.partition places it.  out is device memory of count
 * elements.  The host forms NumPy's 'linear' virtual index and interpolates
 * between the two order statistics around it. */
int enq_order_stats(int dtype, const void* x, int64_t n, const int64_t* host_ranks,
                    int count, void* out);

/* ---- Dense on int8 weights -----------------------------------------
 * y = act(x . (codes * w_scale)^T + bias) with x (m, k) fp32, codes (n, k)
 * int8, w_scale (n) fp32, bias (n) fp32 or NULL, y (m, n) fp32.
 * Replaces the Dense branch z = np.dot(x, W.T) + b; activate(z),
 * Enilnets/nn/forward.py:318-321 with W the fake-quantized weights (which
 * equal codes * scale to within one fp32 rounding).  z (nullable) receives the
 * pre-activation.  act_alpha is the leakyrelu/elu alpha, act_clip the
 * sigmoid/softplus clip (activations.py:20-37).  Small m runs the split-K
 * GEMV kernel, larger m the LDS-tiled MFMA GEMM. */
int enq_dense_w8(const float* x, int64_t m, int64_t k, const int8_t* codes,
                 const float* w_scale, int64_t n, const float* bias,
                 int activation, float act_alpha, float act_clip, int variant,
                 float* y, float* z);

/* The two halves of enq_dense_w8 for large m, for callers that multiply
 * one batch of activations by several weights (the Q, K and V projections
 * of one input): enq_split_planes writes x (m, k) fp32 as bf16 planes,
 * hi = bf16(x) and, for ENQ_W8_FP32, lo = bf16(x - hi), each (m, kp) with kp
 * = k rounded up to a multiple of 32 and zero padding, plane p at
 * planes + p * m * kp (2 * planes * m * kp bytes, 16-byte aligned).
 * enq_gemm_w8_planes then computes enq_dense_w8's y and z from them (same
 * tile kernels as enq_dense_w8 for m > 64, no activation fake-quantization).
 * No counterpart in the reference: they split the Dense of forward.py:318-321
 * in two. */
int enq_split_planes(const float* x, int64_t m, int64_t k, int variant, uint16_t* planes);
int enq_gemm_w8_planes(const uint16_t* planes, int64_t m, int64_t k, const int8_t* codes,
                       const float* w_scale, int64_t n, const float* bias, int activation,
                       float act_alpha, float act_clip, int variant, float* y, float* z);

/* The two halves of enq_dense_w8's fp32-accurate path for large tiles (k a
 * multiple of 16, 16-byte aligned codes), for callers that multiply one batch
 * of activations by several weights.  enq_split_f16f8 writes, per row of x
 * (m, k) fp32, the power of two e with max |x| * 2^e in [2^14, 2^15), the
 * fp16 high parts hi = fp16(x * 2^e) and the e4m3 low parts
 * lo = e4m3(x * 2^e - hi), rows padded with zeros to kp = k rounded up to a
 * multiple of 64: hi (m, kp) uint16 at buf, lo (m, kp) bytes at
 * buf + 2 * m * kp, e (m) int32 at buf + 3 * m * kp; buf holds
 * m * (3 * kp + 4) bytes, 16-byte aligned.  enq_gemm_w8_f16f8 computes
 * enq_dense_w8's y and z from that buffer, within 1e-4 * max |z| per row of
 * the float64 product (no activation fake-quantization).  No counterpart in
 * the reference: they split the Dense of forward.py:318-321 in two. */
int enq_split_f16f8(const float* x, int64_t m, int64_t k, void* buf);
int enq_gemm_w8_f16f8(const void* buf, int64_t m, int64_t k, const int8_t* codes,
                      const float* w_scale, int64_t n, const float* bias, int activation,
                      float act_alpha, float act_clip, float* y, float* z);

/* Two Dense layers in a row (a transformer block's feed-forward pair):
 * y = act2(act1(x . W1^T + b1) . W2^T + b2), W1 = codes1 (n1, k) * scale1,
 * W2 = codes2 (n2, n1) * scale2, biases nullable, each layer as
 * enq_dense_w8 with its activation (act1 not softmax on the fused path).
 * Replaces two consecutive Dense branches of forward.py:318-321 when only
 * the second output is wanted.  For the fp32-accurate variant at sizes where
 * enq_dense_w8 takes the fp16/e4m3 split for both layers (k and n1 multiples
 * of 16, n1 of 64, aligned codes), the first GEMM writes its activated
 * output straight as the second's split, with row exponents from a bound on
 * the first layer's outputs (||x_r||_2 times the largest weight row norm,
 * plus the bias): no fp32 hidden rows in HBM and no split pass over them;
 * y within 1e-4 * max |z2| per row of the float64 result.  bound1
 * (nullable) is that bound's two floats from enq_f16f8_bound for (codes1,
 * scale1, bias1, act1), computed once per weight; NULL computes it in the
 * call (two more launches).  Otherwise two enq_dense_w8 calls through an
 * fp32 hidden buffer.  No counterpart in the reference as one call. */
int enq_dense_w8_ffn(const float* x, int64_t m, int64_t k, const int8_t* codes1,
                     const float* scale1, int64_t n1, const float* bias1, int act1,
                     float alpha1, float clip1, const float* bound1, const int8_t* codes2,
                     const float* scale2, int64_t n2, const float* bias2, int act2,
                     float alpha2, float clip2, int variant, float* y);

/* The output bound of a Dense layer that enq_dense_w8_ffn uses for the
 * exponents of its hidden rows: out[0..1] (device) = (c * max_n scale_n *
 * ||codes_n||_2, c * max |bias| + d), each widened by 1%, with
 * |act(z)| <= c |z| + d for the activation (not softmax); a row x then has
 * every output within ||x||_2 * out[0] + out[1].  k a multiple of 16 and
 * codes 16-byte aligned, as the split GEMM needs.  A property of the
 * weights only, so a caller computes it once per weight.  No counterpart in
 * the reference. */
int enq_f16f8_bound(const int8_t* codes, int64_t rows, int64_t k, const float* scale,
                    const float* bias, int activation, float alpha, float clip, float* out);

/* enq_dense_w8 without any allocation.  No counterpart in the reference: it
 * is for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  Same
 * arguments, kernels and results as enq_dense_w8; the GEMV partial sums and
 * split activations some shapes need come from a fixed 64 MiB device array
 * per device instead of the growable workspace.  A call that needs more
 * (GEMV partials: 4 * K-slices * n * rows rounded up to 16, 32 or 64 for
 * m <= 64, to a multiple of 16 above; the fp32-accurate variant's fp16 / e4m3
 * split of large GEMMs: m * (3 * kp + 4) with kp = k rounded up to 64;
 * bf16 activation planes, taken by the bf16 variant at 256 x 256 tiles and
 * by unaligned activations: 2 * planes * m * k rounded up to a multiple of
 * 32) fails with ENQ_ERR_INVALID before launching anything.  Calls that overlap on one
 * device share that array and race: issue them on one stream, in order. */
int enq_dense_w8_noalloc(const float* x, int64_t m, int64_t k, const int8_t* codes,
                         const float* w_scale, int64_t n, const float* bias,
                         int activation, float act_alpha, float act_clip, int variant,
                         float* y, float* z);

/* enq_dense_w8 followed, in the same epilogue, by the activation
 * fake-quantization of forward.py:798-805 (act_quant spec of a calibrated
 * layer, compression/quantization.py:156-209):
 *   y = (clip(rint(act(z) / aq_scale + aq_zero_point), qmin, qmax)
 *        - aq_zero_point) * aq_scale
 * in float64 (aq_mode ENQ_AQ_F64: the calibrator's float64 scale promotes the
 * expression) or float32 (ENQ_AQ_F32), stored as float32.  z is unaffected. */
int enq_dense_w8_aq(const float* x, int64_t m, int64_t k, const int8_t* codes,
                    const float* w_scale, int64_t n, const float* bias,
                    int activation, float act_alpha, float act_clip, int variant,
                    int aq_mode, double aq_scale, double aq_zero_point,
                    float aq_qmin, float aq_qmax, float* y, float* z);

/* The same fake-quantization as a standalone pass over n values (for layer
 * outputs no Dense epilogue produces); y may equal x. */
int enq_act_quant(const float* x, int64_t n, int mode, double scale, double zero_point,
                  float qmin, float qmax, float* y);

/* W8A8: int8 activation codes (m, k) with one fp32 scale per row, int8
 * weight codes (n, k) with one fp32 scale per row of W.
 * acc = x_codes . w_codes^T (int32, exact); y = act(acc * x_scale * w_scale + b).
 * acc (nullable) receives the int32 accumulators.  The reference has no
 * integer GEMM (quantization.py:1-14); this is the composition of its
 * quantize_tensor (:76-93) with the Dense branch (forward.py:318-321). */
int enq_gemm_w8a8(const int8_t* x_codes, const float* x_scale,
                  const int8_t* w_codes, const float* w_scale,
                  const float* bias, int64_t m, int64_t n, int64_t k,
                  int activation, float act_alpha, float act_clip, float* y,
                  int32_t* acc);

/* W8A8 Dense from fp32 activations: per-token quantization
 * (enq_quantize_rows_i8) followed by enq_gemm_w8a8, using the library
 * workspace for the activation codes. */
int enq_dense_w8a8(const float* x, int64_t m, int64_t k, const int8_t* codes,
                   const float* w_scale, int64_t n, const float* bias,
                   int activation, float act_alpha, float act_clip, float* y,
                   int32_t* acc);

/* Static W8A8 Dense: the activations are quantized with a calibrated
 * per-tensor spec (ActivationCalibrator, quantization.py:156-209: the
 * act_quant spec of the layer that produced x, applied as forward.py:798-805
 * does) instead of per token.  Codes q = clip(rint(x / x_scale +
 * x_zero_point), qmin, qmax) in the spec's arithmetic (aq_mode ENQ_AQ_F32 or
 * ENQ_AQ_F64), so for an x the spec already fake-quantized they are that
 * grid's integers exactly.  acc[m,n] = sum_k (q - zp) * codes[n,k] (exact
 * int32), y = act((float(acc) * float(x_scale)) * w_scale[n] + bias[n]).
 * Grids wider than int8 (asymmetric [0, 255]) are stored shifted by 128, and
 * (128 - zp) * w_code_sums[n] is added back to the accumulators:
 * w_code_sums (from enq_code_row_sums) may be NULL only when that term is 0.
 * No counterpart in the reference (it has no integer GEMM); the composed
 * oracle is its quantize (:53-56) and Dense (forward.py:318-321). */
int enq_dense_w8a8_static(const float* x, int64_t m, int64_t k, int aq_mode,
                          double x_scale, double x_zero_point, float qmin, float qmax,
                          const int8_t* codes, const float* w_scale,
                          const int32_t* w_code_sums, int64_t n, const float* bias,
                          int activation, float act_alpha, float act_clip, float* y,
                          int32_t* acc);

/* sums[r] = sum over k of codes[r, k] (int32), for enq_dense_w8a8_static. */
int enq_code_row_sums(const int8_t* codes, int64_t rows, int64_t k, int32_t* sums);

/* ---- Transformer-block pieces around the quantized projections -------
 * LayerNorm over the last axis of an fp32 (rows, cols) matrix:
 * y = gamma * (x - mean) / sqrt(var + eps) + beta, mean and biased variance
 * per row.  Replaces layernorm_forward's 2-D / 3-D branches,
 * Enilnets/nn/forward.py:216-221,240-253 (3-D inputs are (B*S, E) rows). */
int enq_layernorm(const float* x, int64_t rows, int64_t cols, const float* gamma,
                  const float* beta, float eps, float* y);

/* y = a + b over n fp32 values (16-byte aligned buffers).  Replaces the
 * residual_add branch x = x + outputs[save_index], forward.py:762-766. */
int enq_add(const float* a, const float* b, int64_t n, float* y);

/* Softmax attention core of the multi-head attention layer,
 * forward.py:431-436,525-549 (absolute positions, softmax kernel):
 * for batch b, query head h and its K/V head h / (heads / kv_heads)
 * (_repeat_kv, forward.py:165-171),
 *   out[b, s, h*D:(h+1)*D] = softmax(q_h k_h^T / sqrt(D) + mask) v_h
 * with the mask of _window_mask (forward.py:102-117): causal forbids key
 * j > query i, window >= 0 forbids |i - j| > window (window < 0: none).
 * q, k, v, out are row-major (batch*seq, ld*) fp32 matrices whose head h
 * occupies columns [h*D, (h+1)*D); a fused QKV projection output is passed
 * as three pointers into one buffer with the same row stride.  head_dim is
 * 16, 32, 64 or 128 (other values: ENQ_ERR_UNSUPPORTED); rows 16-byte
 * aligned.  Products are fp32-accurate: with at most 8 queries per sequence
 * they are fp32 FMAs; otherwise at head_dim 32-128 each is six bf16
 * matrix-core products of the operands' three-part bf16 splits (within about
 * 2^-25 of the fp32 product), at 16 an fp32 matrix-core product; sums and
 * exponentials are fp32. */
int enq_attention(const float* q, int64_t ldq, const float* k, int64_t ldk,
                  const float* v, int64_t ldv, int64_t batch, int64_t seq,
                  int heads, int kv_heads, int head_dim, int causal,
                  int64_t window, float* out, int64_t ldo);

/* Attention of seq_q new queries over seq_k keys and values (a KV-cache
 * decode step, Enilnets/nn/kvcache.py:124-213): queries of batch b are rows
 * b*q_bstride + [0, seq_q) of q and out, keys/values rows b*kv_bstride +
 * [0, seq_k) of k and v; query i is at absolute position q_pos0 + i, key j
 * at k_pos0 + j, and the masks of _window_mask apply to those positions.
 * Otherwise as enq_attention. */
int enq_attention_kv(const float* q, int64_t ldq, int64_t q_bstride, int64_t seq_q,
                     int64_t q_pos0, const float* k, int64_t ldk, const float* v,
                     int64_t ldv, int64_t kv_bstride, int64_t seq_k, int64_t k_pos0,
                     int64_t batch, int heads, int kv_heads, int head_dim, int causal,
                     int64_t window, float* out, int64_t ldo);

/* y[o, i] = a[o, i] + b[i] for o < outer, i < inner: the positional-table
 * add x + table[pos:pos+S][None] of forward.py:597-603 / kvcache.py:88-91. */
int enq_add_bcast(const float* a, const float* b, int64_t outer, int64_t inner, float* y);

/* Strided row copy over `batch` row blocks: dst[(b*dst_bstride + r)*ld_dst + c]
 * = src[(b*src_bstride + s)*ld_src + c] for r < nrows, c < width, with s = r,
 * or s = rows[b*nrows + r] when rows is not NULL (an embedding lookup,
 * forward.py:414-422, with batch 1).  Appends keys and values to a cache. */
int enq_copy_rows(const float* src, int64_t ld_src, int64_t src_bstride,
                  const int32_t* rows, float* dst, int64_t ld_dst, int64_t dst_bstride,
                  int64_t nrows, int64_t width, int64_t batch);

/* ---- Mixture of experts on int8 expert weights ------------------------
 * Replaces moe_forward, Enilnets/nn/moe.py:52-87, for x (tokens, d) fp32:
 * router logits = x . (wr * sr)^T + br (experts, d) unless router_logits
 * (tokens, experts) is given; probs = softmax(logits); the top_k experts of
 * each token by probability (ties: lower expert index first); gates = the
 * raw probabilities; for each expert e, over its tokens in token order,
 *   y = act(x . (w1[e] * s1[e])^T + b1[e]) . (w2[e] * s2[e])^T + b2[e]
 * and out[t] = sum over t's experts in ascending expert index of gate * y.
 * w1 (experts, hidden, d) and w2 (experts, d, hidden) int8 codes with one
 * fp32 scale per output row (s1: experts*hidden, s2: experts*d); biases may
 * be NULL.  Optional outputs: probs (tokens, experts), top_idx (tokens,
 * top_k) int32 in slot order, aux_loss (one double on the device: the
 * load-balancing loss of moe.py:38-49).  experts <= 256; softmax is not an
 * accepted expert activation.  variant as in enq_dense_w8.  bound1
 * (nullable): enq_f16f8_bound of the stacked first layer (w1 as experts *
 * hidden rows of d, s1, b1, the activation), computed once per weight; NULL
 * computes it in the call. */
int enq_moe_w8(const float* x, int64_t tokens, int64_t d, const float* router_logits,
               const int8_t* wr, const float* sr, const float* br,
               const int8_t* w1, const float* s1, const float* b1,
               const int8_t* w2, const float* s2, const float* b2,
               int64_t experts, int64_t hidden, int top_k,
               int activation, float act_alpha, float act_clip,
               const float* bound1, int variant,
               float* out, float* probs, int32_t* top_idx, double* aux_loss);

#ifdef __cplusplus
}
#endif

#endif /* ENILNETS_AMD_H */
