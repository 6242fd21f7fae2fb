// Quantization kernels: range statistics, scales, quantize / dequantize /
// fake-quantize, the fused quantize_tensor, int8 rows and error sums.
//
// Arithmetic follows Enilnets/compression/quantization.py exactly:
//   scale  = amax > 0 ? amax / qmax : 1        (:43-44, true division)
//   zp     = round(qmin - low / scale)         (:49, asymmetric only)
//   code   = clip(round(x / scale + zp), qmin, qmax)   (:56)
//   fake   = (code - zp) * scale               (:61)
// round is half-to-even (rint), division is IEEE (no reciprocal multiply) and
// no multiply-add is contracted into an FMA, so results are bit-identical to
// NumPy on the same inputs.
#pragma clang fp contract(off)

#include <algorithm>
#include <cfloat>
#include <cmath>

#include <type_traits>

#include "common.hpp"

namespace enq {
namespace {

constexpr int kBlock = 256;

template <class T>
__device__ __forceinline__ T nan_value();
template <>
__device__ __forceinline__ float nan_value<float>() { return __builtin_nanf(""); }
template <>
__device__ __forceinline__ double nan_value<double>() { return __builtin_nan(""); }

template <class T>
__device__ __forceinline__ T pos_inf();
template <>
__device__ __forceinline__ float pos_inf<float>() { return __builtin_inff(); }
template <>
__device__ __forceinline__ double pos_inf<double>() { return __builtin_inf(); }

// Running min / max with a separate NaN flag (np.min/np.max propagate NaN).
template <class T>
struct Range {
  T lo, hi;
  int nan;
  __device__ __forceinline__ void init() {
    lo = pos_inf<T>();
    hi = -pos_inf<T>();
    nan = 0;
  }
  __device__ __forceinline__ void add(T v) {
    if (v != v) {
      nan = 1;
    } else {
      lo = v < lo ? v : lo;
      hi = v > hi ? v : hi;
    }
  }
  __device__ __forceinline__ void merge(T olo, T ohi, int onan) {
    lo = olo < lo ? olo : lo;
    hi = ohi > hi ? ohi : hi;
    nan |= onan;
  }
  __device__ __forceinline__ T low() const { return nan ? nan_value<T>() : lo; }
  __device__ __forceinline__ T high() const { return nan ? nan_value<T>() : hi; }
};

template <class T>
__device__ __forceinline__ void wave_reduce(Range<T>& r) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) {
    T olo = __shfl_xor(r.lo, m, 64);
    T ohi = __shfl_xor(r.hi, m, 64);
    int on = __shfl_xor(r.nan, m, 64);
    r.merge(olo, ohi, on);
  }
}

__device__ __forceinline__ double wave_sum(double v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
  return v;
}

struct QParams {
  int scheme;
  int qmin, qmax;
};

// compute_scale (quantization.py:33-50) on one channel's range.
template <class T>
__device__ __forceinline__ void scale_from_range(T lo, T hi, const QParams& p,
                                                 T& scale, T& zp) {
  if (p.scheme == ENQ_SYMMETRIC) {
    T alo = lo < 0 ? -lo : lo;  // fabs without touching NaN handling below
    T ahi = hi < 0 ? -hi : hi;
    bool nan = (lo != lo) || (hi != hi);
    T amax = nan ? nan_value<T>() : (alo > ahi ? alo : ahi);
    scale = amax > T(0) ? amax / T(p.qmax) : T(1);
    zp = T(0);
  } else {
    T span = hi - lo;
    scale = span > T(0) ? span / T(p.qmax - p.qmin) : T(1);
    zp = round_even(T(p.qmin) - lo / scale);
  }
}

template <class T>
__device__ __forceinline__ T quantize_one(T x, T scale, T zp, T qmin, T qmax) {
  T shifted = x / scale + zp;
  return clip(round_even(shifted), qmin, qmax);
}

template <class T>
__device__ __forceinline__ T dequantize_one(T q, T scale, T zp) {
  return (q - zp) * scale;
}

// A NaN code has no int8 form; it is stored as 0.
template <class T>
__device__ __forceinline__ int8_t code_to_i8(T q) {
  return q != q ? int8_t(0) : static_cast<int8_t>(static_cast<int>(q));
}

// 16-byte vector of T (4 floats or 2 doubles), or a single element.
template <class T, int V>
struct alignas(sizeof(T) * V) Vec {
  T v[V];
};

// Streaming (non-temporal) vector accesses: every tensor here is touched
// once, so the loads and stores bypass cache allocation.
template <class T, int V>
struct NativeVec {
  typedef T type __attribute__((ext_vector_type(V)));
};
template <class T>
struct NativeVec<T, 1> {
  typedef T type;
};

template <class T, int V>
__device__ __forceinline__ Vec<T, V> load_vec(const T* p) {
  typedef typename NativeVec<T, V>::type N;
  N n = __builtin_nontemporal_load(reinterpret_cast<const N*>(p));
  return __builtin_bit_cast(Vec<T, V>, n);
}
template <class T, int V>
__device__ __forceinline__ void store_vec(T* p, const Vec<T, V>& v) {
  typedef typename NativeVec<T, V>::type N;
  __builtin_nontemporal_store(__builtin_bit_cast(N, v), reinterpret_cast<N*>(p));
}

template <int V>
__device__ __forceinline__ void store_codes(int8_t* p, const int8_t (&c)[V]) {
  if constexpr (V == 4) {
    uint32_t packed = uint32_t(uint8_t(c[0])) | (uint32_t(uint8_t(c[1])) << 8) |
                      (uint32_t(uint8_t(c[2])) << 16) | (uint32_t(uint8_t(c[3])) << 24);
    __builtin_nontemporal_store(packed, reinterpret_cast<uint32_t*>(p));
  } else if constexpr (V == 2) {
    uint16_t packed = uint16_t(uint8_t(c[0])) | uint16_t(uint16_t(uint8_t(c[1])) << 8);
    __builtin_nontemporal_store(packed, reinterpret_cast<uint16_t*>(p));
  } else {
    p[0] = c[0];
  }
}

// Unsigned 32-bit division by a run-time constant: q = (umulhi(n, m) + n) >> s.
struct FastDiv {
  uint32_t d, magic, shift;
};

FastDiv make_fastdiv(uint32_t d) {
  FastDiv f;
  f.d = d;
  uint32_t s = 0;
  while ((uint64_t(1) << s) < d) ++s;
  f.shift = s;
  f.magic = uint32_t(((uint64_t(1) << 32) * ((uint64_t(1) << s) - d)) / d + 1);
  if (d == 1) f.magic = 0;
  return f;
}

__device__ __forceinline__ uint32_t fast_div(uint32_t n, const FastDiv& f) {
  uint64_t t = uint64_t(__umulhi(n, f.magic)) + n;
  return uint32_t(t >> f.shift);
}

// ---------------------------------------------------------------------------
// Per-row fused quantize_tensor: one row group (TPR threads) per row, the row
// held in registers, so HBM is read once.  Used for per-channel quantization
// along axis 0 (outer == 1) and for int8 per-row (per-token) codes.
//
// SYM: the symmetric scheme only needs max |x| (one fmax per element plus a
// NaN flag); asymmetric tracks min and max.  OUT is a bitmask of the outputs
// (kOutFake, kOutCodes, kOutErr) so unused ones cost neither instructions
// nor registers.  All blocks walk their rows in the same chunk order, which
// keeps HBM traffic in lockstep (measured: rotating the order per row halves
// the bandwidth).
// ---------------------------------------------------------------------------
constexpr int kOutFake = 1, kOutCodes = 2, kOutErr = 4;

template <class T>
__device__ __forceinline__ T fmax_t(T a, T b);
template <>
__device__ __forceinline__ float fmax_t<float>(float a, float b) { return __builtin_fmaxf(a, b); }
template <>
__device__ __forceinline__ double fmax_t<double>(double a, double b) { return __builtin_fmax(a, b); }
template <class T>
__device__ __forceinline__ T fmin_t(T a, T b);
template <>
__device__ __forceinline__ float fmin_t<float>(float a, float b) { return __builtin_fminf(a, b); }
template <>
__device__ __forceinline__ double fmin_t<double>(double a, double b) { return __builtin_fmin(a, b); }

// GIVEN: one scale and zero point for every row, read from scale_out[0] and
// zp_out[0] (the codes pass of a per-tensor quantize), no row statistics.
template <class T, int TPR, int CHUNKS, int V, bool SYM, int OUT, bool GIVEN = false>
__global__ __launch_bounds__(TPR < kBlock ? kBlock : TPR) void rows_quant_kernel(
    const T* __restrict__ w, int64_t rows, int64_t cols, QParams p,
    T* __restrict__ out_fake, int8_t* __restrict__ out_codes,
    T* __restrict__ scale_out, T* __restrict__ zp_out, double* __restrict__ err_rows) {
  constexpr int kThreads = TPR < kBlock ? kBlock : TPR;
  constexpr int kRowsPerBlock = kThreads / TPR;
  constexpr int kWavesPerRow = TPR / 64;
  __shared__ T s_a[kThreads / 64];
  __shared__ T s_b[kThreads / 64];
  __shared__ int s_nan[kThreads / 64];
  __shared__ double s_err[kThreads / 64];

  const int t = threadIdx.x % TPR;
  const int64_t row = int64_t(blockIdx.x) * kRowsPerBlock + threadIdx.x / TPR;
  const bool active = row < rows;
  const T* src = w + (active ? row : 0) * cols;

  // every chunk is loaded from an in-bounds address and zeroed afterwards if
  // it lies outside the row: a load behind a guard branch whose other arm
  // writes zeros makes the compiler wait for it before the next chunk's load
  T vals[CHUNKS][V];
  {
    Vec<T, V> raw[CHUNKS];
#pragma unroll
    for (int c = 0; c < CHUNKS; ++c) {
      const int64_t idx = (int64_t(c) * TPR + t) * V;
      raw[c] = load_vec<T, V>(src + (idx < cols ? idx : 0));
    }
#pragma unroll
    for (int c = 0; c < CHUNKS; ++c) {
      const bool live = active && (int64_t(c) * TPR + t) * V < cols;
#pragma unroll
      for (int e = 0; e < V; ++e) vals[c][e] = live ? raw[c].v[e] : T(0);
    }
  }
  // a: max |x| (SYM) or min x; b: max x (asymmetric only).  Padding zeros do
  // not change max |x|; for min / max they are excluded below.
  T a = SYM ? T(0) : pos_inf<T>(), b = -pos_inf<T>();
  int nan = 0;
  if constexpr (!GIVEN) {
#pragma unroll
    for (int c = 0; c < CHUNKS; ++c) {
      const int64_t idx = (int64_t(c) * TPR + t) * V;
      const bool live = SYM || (active && idx < cols);
#pragma unroll
      for (int e = 0; e < V; ++e) {
        const T x = vals[c][e];
        nan |= (x != x);
        if (SYM) {
          a = fmax_t(a, x < T(0) ? -x : x);
        } else if (live) {
          a = fmin_t(a, x);
          b = fmax_t(b, x);
        }
      }
    }
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) {
      a = SYM ? fmax_t(a, __shfl_xor(a, m, 64)) : fmin_t(a, __shfl_xor(a, m, 64));
      if (!SYM) b = fmax_t(b, __shfl_xor(b, m, 64));
      nan |= __shfl_xor(nan, m, 64);
    }
    if constexpr (kWavesPerRow > 1) {
      const int wave = threadIdx.x / 64;
      if ((threadIdx.x & 63) == 0) {
        s_a[wave] = a;
        if (!SYM) s_b[wave] = b;
        s_nan[wave] = nan;
      }
      __syncthreads();
      const int first = (threadIdx.x / TPR) * kWavesPerRow;
      a = s_a[first];
      if (!SYM) b = s_b[first];
      nan = s_nan[first];
#pragma unroll
      for (int i = 1; i < kWavesPerRow; ++i) {
        a = SYM ? fmax_t(a, s_a[first + i]) : fmin_t(a, s_a[first + i]);
        if (!SYM) b = fmax_t(b, s_b[first + i]);
        nan |= s_nan[first + i];
      }
    }
  }
  T scale, zp;
  if constexpr (GIVEN) {
    scale = scale_out[0];
    zp = zp_out[0];
  } else if (SYM) {
    // compute_scale with low = -a, high = a gives max(|low|, |high|) = a
    scale_from_range(nan ? nan_value<T>() : -a, nan ? nan_value<T>() : a, p, scale, zp);
  } else {
    scale_from_range(nan ? nan_value<T>() : a, nan ? nan_value<T>() : b, p, scale, zp);
  }
  if (!GIVEN && active && t == 0) {
    scale_out[row] = scale;
    zp_out[row] = zp;
  }
  const T qmin = T(p.qmin), qmax = T(p.qmax);
  double err = 0.0;
#pragma unroll
  for (int c = 0; c < CHUNKS; ++c) {
    const int64_t idx = (int64_t(c) * TPR + t) * V;
    if (active && idx < cols) {
      Vec<T, V> f;
      int8_t codes[V];
#pragma unroll
      for (int e = 0; e < V; ++e) {
        T q = quantize_one(vals[c][e], scale, zp, qmin, qmax);
        if (OUT & (kOutFake | kOutErr)) f.v[e] = dequantize_one(q, scale, zp);
        if (OUT & kOutCodes) codes[e] = code_to_i8(q);
        if (OUT & kOutErr) {
          T d = f.v[e] - vals[c][e];
          err += double(d < 0 ? -d : d);
        }
      }
      if (OUT & kOutFake) store_vec<T, V>(out_fake + row * cols + idx, f);
      if (OUT & kOutCodes) store_codes<V>(out_codes + row * cols + idx, codes);
    }
  }
  if (OUT & kOutErr) {
    err = wave_sum(err);
    if constexpr (kWavesPerRow > 1) {
      const int wave = threadIdx.x / 64;
      if ((threadIdx.x & 63) == 0) s_err[wave] = err;
      __syncthreads();
      const int first = (threadIdx.x / TPR) * kWavesPerRow;
      err = 0.0;
#pragma unroll
      for (int i = 0; i < kWavesPerRow; ++i) err += s_err[first + i];
    }
    if (active && t == 0) err_rows[row] = err;
  }
}

// Rows too long for registers: two passes over the row (the second mostly
// served from cache), one block of 1024 threads per row.
template <class T, int V>
__global__ __launch_bounds__(1024) void rows_quant_stream_kernel(
    const T* __restrict__ w, int64_t rows, int64_t cols, QParams p,
    T* __restrict__ out_fake, int8_t* __restrict__ out_codes,
    T* __restrict__ scale_out, T* __restrict__ zp_out, double* __restrict__ err_rows) {
  __shared__ T s_lo[16];
  __shared__ T s_hi[16];
  __shared__ int s_nan[16];
  __shared__ double s_err[16];
  const int64_t row = blockIdx.x;
  const T* src = w + row * cols;
  Range<T> r;
  r.init();
  for (int64_t idx = int64_t(threadIdx.x) * V; idx < cols; idx += int64_t(blockDim.x) * V) {
    Vec<T, V> v = load_vec<T, V>(src + idx);
#pragma unroll
    for (int e = 0; e < V; ++e) r.add(v.v[e]);
  }
  wave_reduce(r);
  const int wave = threadIdx.x / 64, nwaves = blockDim.x / 64;
  if ((threadIdx.x & 63) == 0) {
    s_lo[wave] = r.lo;
    s_hi[wave] = r.hi;
    s_nan[wave] = r.nan;
  }
  __syncthreads();
  r.init();
  for (int i = 0; i < nwaves; ++i) r.merge(s_lo[i], s_hi[i], s_nan[i]);
  T scale, zp;
  scale_from_range(r.low(), r.high(), p, scale, zp);
  if (threadIdx.x == 0) {
    scale_out[row] = scale;
    zp_out[row] = zp;
  }
  const T qmin = T(p.qmin), qmax = T(p.qmax);
  double err = 0.0;
  for (int64_t idx = int64_t(threadIdx.x) * V; idx < cols; idx += int64_t(blockDim.x) * V) {
    Vec<T, V> v = load_vec<T, V>(src + idx);
    Vec<T, V> f;
    int8_t codes[V];
#pragma unroll
    for (int e = 0; e < V; ++e) {
      T q = quantize_one(v.v[e], scale, zp, qmin, qmax);
      f.v[e] = dequantize_one(q, scale, zp);
      codes[e] = code_to_i8(q);
      T d = f.v[e] - v.v[e];
      err += double(d < 0 ? -d : d);
    }
    if (out_fake) store_vec<T, V>(out_fake + row * cols + idx, f);
    if (out_codes) store_codes<V>(out_codes + row * cols + idx, codes);
  }
  if (err_rows) {
    err = wave_sum(err);
    if ((threadIdx.x & 63) == 0) s_err[wave] = err;
    __syncthreads();
    if (threadIdx.x == 0) {
      double total = 0.0;
      for (int i = 0; i < nwaves; ++i) total += s_err[i];
      err_rows[row] = total;
    }
  }
}

// ---------------------------------------------------------------------------
// Two-stage range statistics for per-tensor and general-axis layouts.
// Stage 1 writes partial ranges; stage 2 reduces them per channel and
// computes scale / zero point.
// ---------------------------------------------------------------------------
template <class T>
struct PartialRange {
  T lo, hi;
  int nan;
};

template <class T, int V>
__global__ __launch_bounds__(kBlock) void minmax_flat_kernel(
    const T* __restrict__ x, int64_t n, PartialRange<T>* __restrict__ part) {
  __shared__ T s_lo[kBlock / 64];
  __shared__ T s_hi[kBlock / 64];
  __shared__ int s_nan[kBlock / 64];
  Range<T> r;
  r.init();
  const int64_t nvec = n / V;
  const int64_t stride = int64_t(gridDim.x) * kBlock;
  for (int64_t i = int64_t(blockIdx.x) * kBlock + threadIdx.x; i < nvec; i += stride) {
    Vec<T, V> v = load_vec<T, V>(x + i * V);
#pragma unroll
    for (int e = 0; e < V; ++e) r.add(v.v[e]);
  }
  // tail elements (n % V) go to block 0
  if (blockIdx.x == 0) {
    for (int64_t i = nvec * V + threadIdx.x; i < n; i += kBlock) r.add(x[i]);
  }
  wave_reduce(r);
  const int wave = threadIdx.x / 64;
  if ((threadIdx.x & 63) == 0) {
    s_lo[wave] = r.lo;
    s_hi[wave] = r.hi;
    s_nan[wave] = r.nan;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    Range<T> b;
    b.init();
    for (int i = 0; i < kBlock / 64; ++i) b.merge(s_lo[i], s_hi[i], s_nan[i]);
    part[blockIdx.x] = PartialRange<T>{b.lo, b.hi, b.nan};
  }
}

// Column statistics of an (outer, L) matrix over slices of `rows_per_slice`
// rows: part[s * L + j] covers column j of slice s.
template <class T>
__global__ __launch_bounds__(kBlock) void minmax_cols_kernel(
    const T* __restrict__ x, int64_t outer, int64_t L, int64_t rows_per_slice,
    PartialRange<T>* __restrict__ part) {
  const int64_t j = int64_t(blockIdx.x) * kBlock + threadIdx.x;
  const int64_t s = blockIdx.y;
  if (j >= L) return;
  Range<T> r;
  r.init();
  const int64_t o0 = s * rows_per_slice;
  const int64_t o1 = o0 + rows_per_slice < outer ? o0 + rows_per_slice : outer;
  for (int64_t o = o0; o < o1; ++o) r.add(x[o * L + j]);
  part[s * L + j] = PartialRange<T>{r.lo, r.hi, r.nan};
}

// One block per channel: reduce part[c * stride_c + s * stride_s + i] over
// s < slices, i < inner; then scale / zero point (and optionally the range).
template <class T>
__global__ __launch_bounds__(kBlock) void finish_range_kernel(
    const PartialRange<T>* __restrict__ part, int64_t slices, int64_t stride_c,
    int64_t stride_s, int64_t inner, QParams p, int want_scale, T* __restrict__ low,
    T* __restrict__ high, T* __restrict__ scale_out, T* __restrict__ zp_out) {
  __shared__ T s_lo[kBlock / 64];
  __shared__ T s_hi[kBlock / 64];
  __shared__ int s_nan[kBlock / 64];
  const int64_t c = blockIdx.x;
  Range<T> r;
  r.init();
  // min, max and the NaN flag merge exactly in any order
  if (inner == 1) {
    // no index division, and eight loads in flight per thread
#pragma unroll 8
    for (int64_t s = threadIdx.x; s < slices; s += kBlock) {
      const PartialRange<T> e = part[c * stride_c + s * stride_s];
      r.merge(e.lo, e.hi, e.nan);
    }
  } else {
    const int64_t total = slices * inner;
    for (int64_t k = threadIdx.x; k < total; k += kBlock) {
      const int64_t s = k / inner, i = k - s * inner;
      const PartialRange<T> e = part[c * stride_c + s * stride_s + i];
      r.merge(e.lo, e.hi, e.nan);
    }
  }
  wave_reduce(r);
  const int wave = threadIdx.x / 64;
  if ((threadIdx.x & 63) == 0) {
    s_lo[wave] = r.lo;
    s_hi[wave] = r.hi;
    s_nan[wave] = r.nan;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    Range<T> b;
    b.init();
    for (int i = 0; i < kBlock / 64; ++i) b.merge(s_lo[i], s_hi[i], s_nan[i]);
    if (low) low[c] = b.low();
    if (high) high[c] = b.high();
    if (want_scale) {
      T scale, zp;
      scale_from_range(b.low(), b.high(), p, scale, zp);
      scale_out[c] = scale;
      zp_out[c] = zp;
    }
  }
}

// Per-tensor quantize of float32 after minmax_flat_kernel, in one launch
// with the statistics' last step.  Every workgroup first merges the `parts`
// partial ranges itself and derives the scale and zero point from them (as
// finish_range_kernel does; workgroup 0 also writes them out), then walks
// its share of 4096-value chunks: each thread takes 16 consecutive values,
// four 16-byte loads issued together, and writes its 16 codes as one 16-byte
// store (the elementwise pass stores 4 codes per instruction).  The grid is
// small (a few workgroups per CU), so the partials are read few times.
// Needs 16-byte aligned x, fake and codes.
template <bool FAKE, bool CODES, bool ERR>
__global__ __launch_bounds__(kBlock) void quantize_flat_kernel(
    const float* __restrict__ x, int64_t n, const PartialRange<float>* __restrict__ part,
    int parts, QParams p, float* __restrict__ scale_out, float* __restrict__ zp_out,
    float* __restrict__ fake, int8_t* __restrict__ codes, double* __restrict__ err_part) {
  __shared__ float s_lo[kBlock / 64];
  __shared__ float s_hi[kBlock / 64];
  __shared__ int s_nan[kBlock / 64];
  __shared__ double s_err[kBlock / 64];
  Range<float> r;
  r.init();
#pragma unroll 8
  for (int i = threadIdx.x; i < parts; i += kBlock) {
    const PartialRange<float> e = part[i];
    r.merge(e.lo, e.hi, e.nan);
  }
  wave_reduce(r);
  if ((threadIdx.x & 63) == 0) {
    s_lo[threadIdx.x / 64] = r.lo;
    s_hi[threadIdx.x / 64] = r.hi;
    s_nan[threadIdx.x / 64] = r.nan;
  }
  __syncthreads();
  Range<float> b;
  b.init();
  for (int i = 0; i < kBlock / 64; ++i) b.merge(s_lo[i], s_hi[i], s_nan[i]);
  float scale, zp;
  scale_from_range(b.low(), b.high(), p, scale, zp);
  if (blockIdx.x == 0 && threadIdx.x == 0) {
    scale_out[0] = scale;
    zp_out[0] = zp;
  }
  const float qmin = float(p.qmin), qmax = float(p.qmax);
  double err = 0.0;
  constexpr int64_t kChunk = int64_t(kBlock) * 16;
  const int64_t chunks = ceil_div(n, kChunk);
  for (int64_t c = blockIdx.x; c < chunks; c += gridDim.x) {
    const int64_t base = c * kChunk + int64_t(threadIdx.x) * 16;
    if (base + 16 <= n) {
      float4 v[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) v[u] = reinterpret_cast<const float4*>(x + base)[u];
      uint32_t word[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const float xs[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
        float f[4];
        uint32_t wd = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float q = quantize_one(xs[e], scale, zp, qmin, qmax);
          if (CODES) wd |= uint32_t(uint8_t(code_to_i8(q))) << (8 * e);
          if (FAKE || ERR) f[e] = dequantize_one(q, scale, zp);
          if (ERR) {
            const float d = f[e] - xs[e];
            err += double(d < 0 ? -d : d);
          }
        }
        word[u] = wd;
        if (FAKE)
          reinterpret_cast<float4*>(fake + base)[u] = make_float4(f[0], f[1], f[2], f[3]);
      }
      if (CODES)
        *reinterpret_cast<uint4*>(codes + base) = make_uint4(word[0], word[1], word[2], word[3]);
    } else {
      for (int64_t i = base; i < n; ++i) {
        const float q = quantize_one(x[i], scale, zp, qmin, qmax);
        if (CODES) codes[i] = code_to_i8(q);
        const float f = dequantize_one(q, scale, zp);
        if (FAKE) fake[i] = f;
        if (ERR) {
          const float d = f - x[i];
          err += double(d < 0 ? -d : d);
        }
      }
    }
  }
  if (ERR) {
    err = wave_sum(err);
    if ((threadIdx.x & 63) == 0) s_err[threadIdx.x / 64] = err;
    __syncthreads();
    if (threadIdx.x == 0) {
      double total = 0.0;
      for (int i = 0; i < kBlock / 64; ++i) total += s_err[i];
      err_part[blockIdx.x] = total;
    }
  }
}

// Segment statistics: channel c is the contiguous run x[c * len, (c+1) * len);
// block (b, c) reduces the b-th of `blocks` pieces of it into part[c * blocks + b].
template <class T, int V>
__global__ __launch_bounds__(kBlock) void minmax_segments_kernel(
    const T* __restrict__ x, int64_t len, PartialRange<T>* __restrict__ part) {
  __shared__ T s_lo[kBlock / 64];
  __shared__ T s_hi[kBlock / 64];
  __shared__ int s_nan[kBlock / 64];
  const int64_t c = blockIdx.y;
  const T* seg = x + c * len;
  Range<T> r;
  r.init();
  const int64_t nvec = len / V;
  const int64_t stride = int64_t(gridDim.x) * kBlock;
  for (int64_t i = int64_t(blockIdx.x) * kBlock + threadIdx.x; i < nvec; i += stride) {
    Vec<T, V> v = load_vec<T, V>(seg + i * V);
#pragma unroll
    for (int e = 0; e < V; ++e) r.add(v.v[e]);
  }
  if (blockIdx.x == 0) {
    for (int64_t i = nvec * V + threadIdx.x; i < len; i += kBlock) r.add(seg[i]);
  }
  wave_reduce(r);
  const int wave = threadIdx.x / 64;
  if ((threadIdx.x & 63) == 0) {
    s_lo[wave] = r.lo;
    s_hi[wave] = r.hi;
    s_nan[wave] = r.nan;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    Range<T> b;
    b.init();
    for (int i = 0; i < kBlock / 64; ++i) b.merge(s_lo[i], s_hi[i], s_nan[i]);
    part[c * gridDim.x + blockIdx.x] = PartialRange<T>{b.lo, b.hi, b.nan};
  }
}

// ---------------------------------------------------------------------------
// Elementwise quantize / dequantize / fake-quantize with a per-channel scale.
// ---------------------------------------------------------------------------
enum class Op { kQuantize, kDequantize, kFake, kFakeTensor, kDequantI8 };

struct ChannelMap {
  // channel(i) = (i / inner) % channels; channels == 1 means scalar.
  int64_t channels, inner;
  FastDiv div_inner, div_channels;  // valid when `small`
  int small;                        // every index fits in 32 bits
};

__device__ __forceinline__ int64_t channel_of(int64_t i, const ChannelMap& m) {
  if (m.channels == 1) return 0;
  if (m.small) {
    uint32_t a = fast_div(uint32_t(i), m.div_inner);
    uint32_t q = fast_div(a, m.div_channels);
    return int64_t(a - q * m.div_channels.d);
  }
  return (i / m.inner) % m.channels;
}

template <class T, Op OP, int V>
__global__ __launch_bounds__(kBlock) void elementwise_kernel(
    const void* __restrict__ in_ptr, int64_t n, ChannelMap map,
    const T* __restrict__ scale, const T* __restrict__ zero_point, QParams p,
    T* __restrict__ out, int8_t* __restrict__ out_codes, double* __restrict__ err_part) {
  const T qmin = T(p.qmin), qmax = T(p.qmax);
  const bool same_channel = (map.inner % V) == 0;  // a vector never spans channels
  double err = 0.0;
  const int64_t nvec = n / V;
  const int64_t stride = int64_t(gridDim.x) * kBlock;
  for (int64_t vi = int64_t(blockIdx.x) * kBlock + threadIdx.x; vi < nvec + (n % V ? 1 : 0);
       vi += stride) {
    const int64_t base = vi * V;
    const bool full = base + V <= n;
    T xs[V];
    if constexpr (OP == Op::kDequantI8) {
      const int8_t* in = static_cast<const int8_t*>(in_ptr);
#pragma unroll
      for (int e = 0; e < V; ++e) xs[e] = (full || base + e < n) ? T(in[base + e]) : T(0);
    } else {
      const T* in = static_cast<const T*>(in_ptr);
      if (full) {
        Vec<T, V> v = load_vec<T, V>(in + base);
#pragma unroll
        for (int e = 0; e < V; ++e) xs[e] = v.v[e];
      } else {
#pragma unroll
        for (int e = 0; e < V; ++e) xs[e] = base + e < n ? in[base + e] : T(0);
      }
    }
    Vec<T, V> res;
    int8_t codes[V];
    int64_t ch = channel_of(base, map);
    T s = scale[ch];
    T z = OP == Op::kDequantI8 ? T(0) : zero_point[ch];
#pragma unroll
    for (int e = 0; e < V; ++e) {
      if (!same_channel && e > 0) {
        ch = channel_of(base + e, map);
        s = scale[ch];
        z = OP == Op::kDequantI8 ? T(0) : zero_point[ch];
      }
      T x = xs[e];
      if constexpr (OP == Op::kQuantize) {
        res.v[e] = quantize_one(x, s, z, qmin, qmax);
      } else if constexpr (OP == Op::kDequantize) {
        res.v[e] = dequantize_one(x, s, z);
      } else if constexpr (OP == Op::kDequantI8) {
        res.v[e] = x * s;
      } else {
        T q = quantize_one(x, s, z, qmin, qmax);
        res.v[e] = dequantize_one(q, s, z);
        codes[e] = code_to_i8(q);
        if (OP == Op::kFakeTensor && err_part && (full || base + e < n)) {
          T d = res.v[e] - x;
          err += double(d < 0 ? -d : d);
        }
      }
    }
    if (full) {
      if (out) store_vec<T, V>(out + base, res);
      if (OP == Op::kFakeTensor && out_codes) store_codes<V>(out_codes + base, codes);
    } else {
#pragma unroll
      for (int e = 0; e < V; ++e) {
        if (base + e < n) {
          if (out) out[base + e] = res.v[e];
          if (OP == Op::kFakeTensor && out_codes) out_codes[base + e] = codes[e];
        }
      }
    }
  }
  if (OP == Op::kFakeTensor && err_part) {
    __shared__ double s_err[kBlock / 64];
    err = wave_sum(err);
    if ((threadIdx.x & 63) == 0) s_err[threadIdx.x / 64] = err;
    __syncthreads();
    if (threadIdx.x == 0) {
      double total = 0.0;
      for (int i = 0; i < kBlock / 64; ++i) total += s_err[i];
      err_part[blockIdx.x] = total;
    }
  }
}

// The same operations on 16-byte vectors, for aligned T inputs.  Workgroup g
// owns the contiguous vectors [g * kBlock * U, (g + 1) * kBlock * U) and
// thread t takes vectors t + kBlock * r, r < U, so every wave load and store
// is one contiguous run and the waves pass through memory in order.  All U
// loads of a thread issue before any arithmetic, each from an index clamped
// to the last full vector and masked where it is used: a guard branch around
// a load whose other arm zeroes the same registers makes the compiler wait
// for the load before the arms rejoin, one round trip per vector.  Measured
// on the per-tensor int8 quantize pass of 8192 x 8192: 74 us (4.5 TB/s)
// against 85 us for the grid-stride loop; eight vectors per thread, or the
// blocks taken in reverse order (to find the statistics pass's last reads in
// the MALL), were no faster.  A partial last vector is done by the thread
// that owns its index, element by element.
template <class T, Op OP, int V, int U>
__global__ __launch_bounds__(kBlock) void elementwise_vec_kernel(
    const T* __restrict__ in, int64_t n, ChannelMap map, const T* __restrict__ scale,
    const T* __restrict__ zero_point, QParams p, T* __restrict__ out,
    int8_t* __restrict__ out_codes, double* __restrict__ err_part) {
  static_assert(OP != Op::kDequantI8, "int8 input takes elementwise_kernel");
  const T qmin = T(p.qmin), qmax = T(p.qmax);
  const bool same_channel = (map.inner % V) == 0;  // a vector never spans channels
  const int64_t nfull = n / V;
  const int64_t v0 = int64_t(blockIdx.x) * kBlock * U + threadIdx.x;
  // one channel (per-tensor parameters): its scale and zero point are loaded
  // once per thread instead of once per vector, which halves the memory
  // instructions of the pass (int8 codes of 8192 x 8192 with a given scale:
  // 77-82 us -> 69-74 us on one box)
  const bool one_channel = map.channels == 1;
  const T sc1 = one_channel ? scale[0] : T(0);
  const T z1 = one_channel ? zero_point[0] : T(0);
  double err = 0.0;
  // one vector's results: outputs, codes and absolute errors
  auto apply = [&](const T (&xs)[V], int64_t base, int valid, Vec<T, V>& res,
                   int8_t (&codes)[V]) {
    int64_t ch = 0;
    T sc = sc1, z = z1;
    if (!one_channel) {
      ch = channel_of(base, map);
      sc = scale[ch];
      z = zero_point[ch];
    }
#pragma unroll
    for (int e = 0; e < V; ++e) {
      if (!one_channel && !same_channel && e > 0) {
        ch = channel_of(base + (e < valid ? e : 0), map);
        sc = scale[ch];
        z = zero_point[ch];
      }
      const T x = xs[e];
      if constexpr (OP == Op::kQuantize) {
        res.v[e] = quantize_one(x, sc, z, qmin, qmax);
      } else if constexpr (OP == Op::kDequantize) {
        res.v[e] = dequantize_one(x, sc, z);
      } else {
        const T q = quantize_one(x, sc, z, qmin, qmax);
        res.v[e] = dequantize_one(q, sc, z);
        codes[e] = code_to_i8(q);
        if (OP == Op::kFakeTensor && err_part && e < valid) {
          const T d = res.v[e] - x;
          err += double(d < 0 ? -d : d);
        }
      }
    }
  };
  if (nfull > 0) {
    Vec<T, V> raw[U];
#pragma unroll
    for (int r = 0; r < U; ++r) {
      const int64_t vi = v0 + int64_t(r) * kBlock;
      raw[r] = load_vec<T, V>(in + (vi < nfull ? vi : nfull - 1) * V);
    }
    Vec<T, V> res[U];
    int8_t codes[U][V];
#pragma unroll
    for (int r = 0; r < U; ++r) {
      const int64_t vi = v0 + int64_t(r) * kBlock;
      T xs[V];
#pragma unroll
      for (int e = 0; e < V; ++e) xs[e] = raw[r].v[e];
      apply(xs, vi < nfull ? vi * V : 0, vi < nfull ? V : 0, res[r], codes[r]);
    }
    // every store after every load of the thread, so a wave's reads and
    // writes reach HBM in separate bursts (storing each vector as its load
    // arrived: 69.1 us against 65.3 for the per-tensor int8 codes pass)
    asm volatile("" ::: "memory");
#pragma unroll
    for (int r = 0; r < U; ++r) {
      const int64_t vi = v0 + int64_t(r) * kBlock;
      if (vi < nfull) {
        if (out) store_vec<T, V>(out + vi * V, res[r]);
        if (OP == Op::kFakeTensor && out_codes) store_codes<V>(out_codes + vi * V, codes[r]);
      }
    }
  }
  if (n % V != 0) {
#pragma unroll
    for (int r = 0; r < U; ++r) {
      if (v0 + int64_t(r) * kBlock == nfull) {
        const int64_t base = nfull * V;
        const int valid = int(n - base);
        T xs[V];
#pragma unroll
        for (int e = 0; e < V; ++e) xs[e] = e < valid ? in[base + e] : T(0);
        Vec<T, V> res;
        int8_t codes[V];
        apply(xs, base, valid, res, codes);
        for (int e = 0; e < valid; ++e) {
          if (out) out[base + e] = res.v[e];
          if (OP == Op::kFakeTensor && out_codes) out_codes[base + e] = codes[e];
        }
      }
    }
  }
  if (OP == Op::kFakeTensor && err_part) {
    __shared__ double s_err[kBlock / 64];
    err = wave_sum(err);
    if ((threadIdx.x & 63) == 0) s_err[threadIdx.x / 64] = err;
    __syncthreads();
    if (threadIdx.x == 0) {
      double total = 0.0;
      for (int i = 0; i < kBlock / 64; ++i) total += s_err[i];
      err_part[blockIdx.x] = total;
    }
  }
}

// int8 codes -> T with a per-channel scale.  A unit is 4 consecutive codes
// (one 32-bit load, one 4-wide store); workgroup g owns units
// [g * 256 * U, (g + 1) * 256 * U), thread t units t + 256 r.  So every wave
// load is one contiguous 256 B run, every wave store one contiguous 1 KiB
// run (fp32), and the waves write the output in order: measured on the box,
// this write-heavy stream runs at 74% of HBM with U = 2, against 60% for a
// grid-stride loop.  Requires n % 4 == 0, inner % 4 == 0 (a unit never
// spans channels), 4-byte aligned codes and 16-byte aligned output.
template <class T, int U>
__global__ __launch_bounds__(kBlock) void dequant_i8_kernel(const int8_t* __restrict__ codes,
                                                            int64_t n, ChannelMap map,
                                                            const T* __restrict__ scale,
                                                            T* __restrict__ out) {
  const uint32_t* c32 = reinterpret_cast<const uint32_t*>(codes);
  const int64_t units = n / 4;
  const int64_t base = int64_t(blockIdx.x) * kBlock * U + threadIdx.x;
  uint32_t raw[U];
  T s[U];
#pragma unroll
  for (int r = 0; r < U; ++r) {
    const int64_t u = base + int64_t(r) * kBlock;
    raw[r] = u < units ? __builtin_nontemporal_load(c32 + u) : 0u;
    s[r] = u < units ? scale[channel_of(u * 4, map)] : T(0);
  }
#pragma unroll
  for (int r = 0; r < U; ++r) {
    const int64_t u = base + int64_t(r) * kBlock;
    if (u >= units) break;
    Vec<T, 4> v;
#pragma unroll
    for (int e = 0; e < 4; ++e) v.v[e] = T(int8_t((raw[r] >> (8 * e)) & 0xff)) * s[r];
    store_vec<T, 4>(out + u * 4, v);
  }
}

// Deterministic sum of `n` doubles into out[0] (one block).
__global__ __launch_bounds__(kBlock) void sum_doubles_kernel(const double* __restrict__ in,
                                                             int64_t n, double* __restrict__ out) {
  __shared__ double s[kBlock / 64];
  double acc = 0.0;
  for (int64_t i = threadIdx.x; i < n; i += kBlock) acc += in[i];
  acc = wave_sum(acc);
  if ((threadIdx.x & 63) == 0) s[threadIdx.x / 64] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    double total = 0.0;
    for (int i = 0; i < kBlock / 64; ++i) total += s[i];
    out[0] = total;
  }
}

template <class T>
__global__ __launch_bounds__(kBlock) void compute_scale_kernel(
    const T* __restrict__ low, const T* __restrict__ high, int64_t n, QParams p,
    T* __restrict__ scale, T* __restrict__ zp) {
  const int64_t i = int64_t(blockIdx.x) * kBlock + threadIdx.x;
  if (i >= n) return;
  T s, z;
  scale_from_range(low[i], high[i], p, s, z);
  scale[i] = s;
  zp[i] = z;
}

// Error sums for quantization_error: |d| sum, |d| max, a^2 sum, d^2 sum.
template <class T>
__global__ __launch_bounds__(kBlock) void error_stats_kernel(
    const T* __restrict__ a, const T* __restrict__ b, int64_t n, double* __restrict__ part) {
  __shared__ double s[4][kBlock / 64];
  double sum_abs = 0.0, max_abs = 0.0, sum_aa = 0.0, sum_dd = 0.0;
  int nan = 0;
  const int64_t stride = int64_t(gridDim.x) * kBlock;
  for (int64_t i = int64_t(blockIdx.x) * kBlock + threadIdx.x; i < n; i += stride) {
    T av = a[i];
    T d = b[i] - av;
    double ad = double(d < 0 ? -d : d);
    if (d != d) nan = 1;
    sum_abs += ad;
    max_abs = ad > max_abs ? ad : max_abs;
    sum_aa += double(av) * double(av);
    sum_dd += double(d) * double(d);
  }
  if (nan) max_abs = __builtin_nan("");
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) {
    sum_abs += __shfl_xor(sum_abs, m, 64);
    double o = __shfl_xor(max_abs, m, 64);
    max_abs = (o > max_abs || o != o) ? o : max_abs;
    sum_aa += __shfl_xor(sum_aa, m, 64);
    sum_dd += __shfl_xor(sum_dd, m, 64);
  }
  const int wave = threadIdx.x / 64;
  if ((threadIdx.x & 63) == 0) {
    s[0][wave] = sum_abs;
    s[1][wave] = max_abs;
    s[2][wave] = sum_aa;
    s[3][wave] = sum_dd;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    double r0 = 0, r1 = 0, r2 = 0, r3 = 0;
    for (int i = 0; i < kBlock / 64; ++i) {
      r0 += s[0][i];
      r1 = (s[1][i] > r1 || s[1][i] != s[1][i]) ? s[1][i] : r1;
      r2 += s[2][i];
      r3 += s[3][i];
    }
    part[blockIdx.x * 4 + 0] = r0;
    part[blockIdx.x * 4 + 1] = r1;
    part[blockIdx.x * 4 + 2] = r2;
    part[blockIdx.x * 4 + 3] = r3;
  }
}

__global__ void error_finish_kernel(const double* __restrict__ part, int64_t blocks,
                                    double* __restrict__ out) {
  if (threadIdx.x != 0) return;
  double r0 = 0, r1 = 0, r2 = 0, r3 = 0;
  for (int64_t i = 0; i < blocks; ++i) {
    r0 += part[i * 4 + 0];
    double m = part[i * 4 + 1];
    r1 = (m > r1 || m != m) ? m : r1;
    r2 += part[i * 4 + 2];
    r3 += part[i * 4 + 3];
  }
  out[0] = r0;
  out[1] = r1;
  out[2] = r2;
  out[3] = r3;
}

// ---------------------------------------------------------------------------
// Host-side dispatch
// ---------------------------------------------------------------------------
QParams make_params(int bits, int scheme) {
  ENQ_REQUIRE(bits >= 2 && bits <= 16, "bits must be between 2 and 16, got %d", bits);
  ENQ_REQUIRE(scheme == ENQ_SYMMETRIC || scheme == ENQ_ASYMMETRIC, "unknown scheme %d", scheme);
  QParams p;
  p.scheme = scheme;
  if (scheme == ENQ_SYMMETRIC) {
    p.qmax = (1 << (bits - 1)) - 1;
    p.qmin = -p.qmax;
  } else {
    p.qmin = 0;
    p.qmax = (1 << bits) - 1;
  }
  return p;
}

void check_dtype(int dtype) {
  ENQ_REQUIRE(dtype == ENQ_F32 || dtype == ENQ_F64, "dtype must be ENQ_F32 or ENQ_F64, got %d",
              dtype);
}

void check_shape(int64_t outer, int64_t channels, int64_t inner) {
  ENQ_REQUIRE(outer >= 1 && channels >= 1 && inner >= 1,
              "shape (outer=%lld, channels=%lld, inner=%lld) must be positive",
              (long long)outer, (long long)channels, (long long)inner);
}

ChannelMap make_map(int64_t n, int64_t channels, int64_t inner) {
  ChannelMap m;
  m.channels = channels;
  m.inner = inner;
  m.small = n < (int64_t(1) << 31) ? 1 : 0;
  m.div_inner = make_fastdiv(uint32_t(m.small ? inner : 1));
  m.div_channels = make_fastdiv(uint32_t(m.small ? channels : 1));
  return m;
}

int grid_for(int64_t work_items, int per_cu = 8) {
  int64_t blocks = ceil_div(work_items, kBlock);
  int64_t cap = int64_t(device_cu_count() > 0 ? device_cu_count() : 256) * per_cu;
  if (blocks > cap) blocks = cap;
  return int(blocks < 1 ? 1 : blocks);
}

constexpr int kElemUnroll = 4;  // vectors per thread of elementwise_vec_kernel (2: 4% slower, 8: 18%)

template <class T, Op OP>
void launch_elementwise(const void* in, int64_t n, int64_t channels, int64_t inner,
                        const T* scale, const T* zp, QParams p, T* out, int8_t* codes,
                        double* err_part, int grid) {
  constexpr int V = 16 / sizeof(T);
  ChannelMap map = make_map(n, channels, inner);
  // the vector kernels store V codes as one V-byte word
  bool vec_ok = (out == nullptr || aligned(out, 16)) && (codes == nullptr || aligned(codes, V));
  if constexpr (OP != Op::kDequantI8) vec_ok = vec_ok && aligned(in, 16);
  if constexpr (OP != Op::kDequantI8) {
    if (vec_ok) {
      // `grid` (elementwise_grid) covers every vector, kElemUnroll per thread
      elementwise_vec_kernel<T, OP, V, kElemUnroll><<<grid, kBlock, 0, stream()>>>(
          static_cast<const T*>(in), n, map, scale, zp, p, out, codes, err_part);
      check_launch("elementwise_vec_kernel");
      return;
    }
  }
  if (vec_ok) {
    elementwise_kernel<T, OP, V><<<grid, kBlock, 0, stream()>>>(in, n, map, scale, zp, p, out,
                                                               codes, err_part);
  } else {
    elementwise_kernel<T, OP, 1><<<grid, kBlock, 0, stream()>>>(in, n, map, scale, zp, p, out,
                                                               codes, err_part);
  }
  check_launch("elementwise_kernel");
}

// Workgroups of an elementwise launch: enough for elementwise_vec_kernel to
// cover every vector (the grid-stride elementwise_kernel takes any grid).
template <class T>
int elementwise_grid(int64_t n) {
  const int64_t g = ceil_div(ceil_div(n, int64_t(16 / sizeof(T))), int64_t(kBlock) * kElemUnroll);
  ENQ_REQUIRE(g <= 0x7fffffff, "tensor too large");
  return int(g < 1 ? 1 : g);
}

// Range statistics to per-channel (low, high) and/or (scale, zp).
template <class T>
void range_stats(const T* x, int64_t outer, int64_t channels, int64_t inner, QParams p,
                 bool want_scale, T* low, T* high, T* scale, T* zp) {
  constexpr int V = 16 / sizeof(T);
  const int64_t n = outer * channels * inner;
  const int64_t cus = device_cu_count() > 0 ? device_cu_count() : 256;
  if (channels == 1) {
    // global statistics
    const int grid = grid_for(ceil_div(n, V * 4));
    auto* part = static_cast<PartialRange<T>*>(workspace(sizeof(PartialRange<T>) * grid));
    if (aligned(x, 16))
      minmax_flat_kernel<T, V><<<grid, kBlock, 0, stream()>>>(x, n, part);
    else
      minmax_flat_kernel<T, 1><<<grid, kBlock, 0, stream()>>>(x, n, part);
    check_launch("minmax_flat_kernel");
    finish_range_kernel<T><<<1, kBlock, 0, stream()>>>(part, grid, 0, 1, 1, p, want_scale, low,
                                                       high, scale, zp);
    check_launch("finish_range_kernel");
    return;
  }
  ENQ_REQUIRE(channels <= 0x7fffffff, "too many channels");
  if (outer == 1) {
    // each channel is one contiguous segment of `inner` elements
    ENQ_REQUIRE(channels <= 65535, "too many channels for the segment reduction");
    int64_t blocks = ceil_div(cus * 8, channels);
    blocks = std::max<int64_t>(1, std::min<int64_t>(blocks, ceil_div(inner, kBlock * V * 4)));
    auto* part =
        static_cast<PartialRange<T>*>(workspace(sizeof(PartialRange<T>) * blocks * channels));
    const bool vec = aligned(x, 16) && (inner % V) == 0;
    if (vec)
      minmax_segments_kernel<T, V><<<dim3(unsigned(blocks), unsigned(channels)), kBlock, 0,
                                     stream()>>>(x, inner, part);
    else
      minmax_segments_kernel<T, 1><<<dim3(unsigned(blocks), unsigned(channels)), kBlock, 0,
                                     stream()>>>(x, inner, part);
    check_launch("minmax_segments_kernel");
    finish_range_kernel<T><<<unsigned(channels), kBlock, 0, stream()>>>(
        part, blocks, blocks, 1, 1, p, want_scale, low, high, scale, zp);
    check_launch("finish_range_kernel");
    return;
  }
  // (outer, L) column statistics, then per-channel reduction.
  const int64_t L = channels * inner;
  int64_t rows_per_slice = outer;
  const int64_t col_blocks = ceil_div(L, kBlock);
  const int64_t want_blocks = cus * 4;
  if (col_blocks < want_blocks) {
    int64_t slices = ceil_div(want_blocks, col_blocks);
    if (slices > outer) slices = outer;
    if (slices > 65535) slices = 65535;
    rows_per_slice = ceil_div(outer, slices);
  }
  const int64_t slices = ceil_div(outer, rows_per_slice);
  ENQ_REQUIRE(col_blocks <= 0x7fffffff, "tensor row too long");
  auto* part = static_cast<PartialRange<T>*>(workspace(sizeof(PartialRange<T>) * slices * L));
  minmax_cols_kernel<T><<<dim3(unsigned(col_blocks), unsigned(slices)), kBlock, 0, stream()>>>(
      x, outer, L, rows_per_slice, part);
  check_launch("minmax_cols_kernel");
  finish_range_kernel<T><<<unsigned(channels), kBlock, 0, stream()>>>(
      part, slices, inner, L, inner, p, want_scale, low, high, scale, zp);
  check_launch("finish_range_kernel");
}

// Row-kernel configurations: (threads per row, 16-byte chunks per thread)
// that hold the row in registers.
template <class T, int V, bool SYM, int OUT>
void launch_rows(const T* w, int64_t rows, int64_t cols, QParams p, T* fake, int8_t* codes,
                 T* scale, T* zp, double* err_rows) {
  auto go = [&](auto kernel, int tpr) {
    const int threads = tpr < kBlock ? kBlock : tpr;
    const int rows_per_block = threads / tpr;
    const int64_t grid = ceil_div(rows, rows_per_block);
    ENQ_REQUIRE(grid <= 0x7fffffff, "too many rows");
    kernel<<<unsigned(grid), threads, 0, stream()>>>(w, rows, cols, p, fake, codes, scale, zp,
                                                     err_rows);
    check_launch("rows_quant_kernel");
  };
  if (cols <= 64 * 4 * V) return go(rows_quant_kernel<T, 64, 4, V, SYM, OUT>, 64);
  if (cols <= 256 * 4 * V) return go(rows_quant_kernel<T, 256, 4, V, SYM, OUT>, 256);
  // rows up to 2048 vectors: 256 threads x 8 chunks.  At 8192 x 8192 fp32
  // -> int8 codes this ran 64.7 us against 71.4 for 512 threads x 4 chunks
  // (half the registers, but only four rows in flight per CU instead of
  // seven) and 69 for 128 x 16 (occupancy four).
  if (cols <= 256 * 8 * V) return go(rows_quant_kernel<T, 256, 8, V, SYM, OUT>, 256);
  if (cols <= 1024 * 4 * V) return go(rows_quant_kernel<T, 1024, 4, V, SYM, OUT>, 1024);
  if (cols <= 1024 * 8 * V) return go(rows_quant_kernel<T, 1024, 8, V, SYM, OUT>, 1024);
  ENQ_REQUIRE(rows <= 0x7fffffff, "too many rows");
  rows_quant_stream_kernel<T, V><<<unsigned(rows), 1024, 0, stream()>>>(w, rows, cols, p, fake,
                                                                         codes, scale, zp,
                                                                         err_rows);
  check_launch("rows_quant_stream_kernel");
}

template <class T, int V>
void launch_rows_any(const T* w, int64_t rows, int64_t cols, QParams p, T* fake, int8_t* codes,
                     T* scale, T* zp, double* err_rows) {
  const int out = (fake ? kOutFake : 0) | (codes ? kOutCodes : 0) | (err_rows ? kOutErr : 0);
  const bool sym = p.scheme == ENQ_SYMMETRIC;
#define ENQ_ROWS_CASE(SYMV, OUTV)                                                            \
  if (sym == (SYMV) && out == (OUTV))                                                        \
    return launch_rows<T, V, (SYMV), (OUTV)>(w, rows, cols, p, fake, codes, scale, zp, err_rows);
  ENQ_ROWS_CASE(true, kOutCodes)
  ENQ_ROWS_CASE(true, kOutFake)
  ENQ_ROWS_CASE(true, kOutFake | kOutErr)
  ENQ_ROWS_CASE(true, kOutFake | kOutCodes | kOutErr)
  ENQ_ROWS_CASE(true, kOutFake | kOutCodes)
  ENQ_ROWS_CASE(false, kOutFake)
  ENQ_ROWS_CASE(false, kOutFake | kOutErr)
#undef ENQ_ROWS_CASE
  // any other combination: the general kernel computes every output it is given
  return launch_rows<T, V, false, kOutFake | kOutCodes | kOutErr>(w, rows, cols, p, fake, codes,
                                                                 scale, zp, err_rows);
}

template <class T>
void rows_quantize(const T* w, int64_t rows, int64_t cols, QParams p, T* fake, int8_t* codes,
                   T* scale, T* zp, double* err_rows) {
  constexpr int V = 16 / sizeof(T);
  const bool vec_ok = (cols % V) == 0 && aligned(w, 16) && (fake == nullptr || aligned(fake, 16)) &&
                      (codes == nullptr || aligned(codes, V));
  if (vec_ok)
    launch_rows_any<T, V>(w, rows, cols, p, fake, codes, scale, zp, err_rows);
  else
    launch_rows_any<T, 1>(w, rows, cols, p, fake, codes, scale, zp, err_rows);
}

// Whether the one-pass row kernel (row held in registers) suits the shape:
// rows fit in registers, or there are enough rows to fill the device.
bool rows_kernel_fits(int64_t rows, int64_t cols) {
  const int64_t cus = device_cu_count() > 0 ? device_cu_count() : 256;
  if (cols <= 1024 * 8 * 4) return rows >= cus || cols <= 8192;
  return rows >= 2 * cus;
}

template <class T>
void quantize_tensor_impl(const T* w, int64_t outer, int64_t channels, int64_t inner, QParams p,
                          T* fake, int8_t* codes, T* scale, T* zp, double* abs_err) {
  const int64_t n = outer * channels * inner;
  if (outer == 1 && channels > 1 && rows_kernel_fits(channels, inner)) {
    // per-channel along axis 0: one row per channel, fused single pass
    double* err_rows = nullptr;
    if (abs_err) err_rows = static_cast<double*>(workspace(sizeof(double) * channels));
    rows_quantize<T>(w, channels, inner, p, fake, codes, scale, zp, err_rows);
    if (abs_err) {
      sum_doubles_kernel<<<1, kBlock, 0, stream()>>>(err_rows, channels, abs_err);
      check_launch("sum_doubles_kernel");
    }
    return;
  }
  if constexpr (std::is_same_v<T, float>) {
    if (channels == 1 && aligned(w, 16) && (fake == nullptr || aligned(fake, 16)) &&
        (codes == nullptr || aligned(codes, 16))) {
      // per-tensor: the statistics pass, then either the row kernel with the
      // one finished scale (whole rows of 8192 values, no error sum) or one
      // launch that finishes the statistics in every workgroup and
      // quantizes.  8192 x 8192 to int8 codes took 120-128 us as statistics,
      // finish_range_kernel and the elementwise pass
      const int sgrid = grid_for(ceil_div(n, 16));
      const int qgrid = int(std::min<int64_t>(ceil_div(n, int64_t(kBlock) * 16),
                                              int64_t(device_cu_count()) * 8));
      const size_t part_bytes = ceil_div(sizeof(PartialRange<float>) * sgrid, 256) * 256;
      char* ws = static_cast<char*>(workspace(part_bytes + sizeof(double) * qgrid));
      auto* part = reinterpret_cast<PartialRange<float>*>(ws);
      double* err_part = abs_err ? reinterpret_cast<double*>(ws + part_bytes) : nullptr;
      minmax_flat_kernel<float, 4><<<sgrid, kBlock, 0, stream()>>>(w, n, part);
      check_launch("minmax_flat_kernel");
      if (!abs_err && n % 8192 == 0 && n / 8192 <= 0x7fffffff) {
        // the range in one workgroup, then the row kernel over rows of 8192
        // values with that one scale: 8192 x 8192 to codes 109.4 -> 104.9 us
        // against the pass below, whose every workgroup merges the partials
        finish_range_kernel<float><<<1, kBlock, 0, stream()>>>(part, sgrid, 0, 1, 1, p, 1, nullptr,
                                                               nullptr, scale, zp);
        check_launch("finish_range_kernel");
        const unsigned rows = unsigned(n / 8192);
        if (fake && codes)
          rows_quant_kernel<float, 256, 8, 4, true, kOutFake | kOutCodes, true>
              <<<rows, 256, 0, stream()>>>(w, rows, 8192, p, fake, codes, scale, zp, nullptr);
        else if (codes)
          rows_quant_kernel<float, 256, 8, 4, true, kOutCodes, true>
              <<<rows, 256, 0, stream()>>>(w, rows, 8192, p, nullptr, codes, scale, zp, nullptr);
        else
          rows_quant_kernel<float, 256, 8, 4, true, kOutFake, true>
              <<<rows, 256, 0, stream()>>>(w, rows, 8192, p, fake, nullptr, scale, zp, nullptr);
        check_launch("rows_quant_kernel");
        return;
      }
      auto launch = [&](auto fake_c, auto codes_c, auto err_c) {
        quantize_flat_kernel<decltype(fake_c)::value, decltype(codes_c)::value,
                             decltype(err_c)::value><<<qgrid, kBlock, 0, stream()>>>(
            w, n, part, sgrid, p, scale, zp, fake, codes, err_part);
      };
      using Y = std::true_type;
      using N = std::false_type;
      if (fake && codes && abs_err) launch(Y{}, Y{}, Y{});
      else if (fake && codes) launch(Y{}, Y{}, N{});
      else if (fake && abs_err) launch(Y{}, N{}, Y{});
      else if (codes && abs_err) launch(N{}, Y{}, Y{});
      else if (fake) launch(Y{}, N{}, N{});
      else if (codes) launch(N{}, Y{}, N{});
      else launch(N{}, N{}, Y{});
      check_launch("quantize_flat_kernel");
      if (abs_err) {
        sum_doubles_kernel<<<1, kBlock, 0, stream()>>>(err_part, qgrid, abs_err);
        check_launch("sum_doubles_kernel");
      }
      return;
    }
  }
  range_stats<T>(w, outer, channels, inner, p, true, nullptr, nullptr, scale, zp);
  const int grid = elementwise_grid<T>(n);
  double* err_part = nullptr;
  if (abs_err) {
    // The range partials in the workspace are consumed by the stage-2 kernel,
    // which is ordered before this reuse on the same stream.
    err_part = static_cast<double*>(workspace(sizeof(double) * grid));
  }
  launch_elementwise<T, Op::kFakeTensor>(w, n, channels, inner, scale, zp, p, fake, codes,
                                         err_part, grid);
  if (abs_err) {
    sum_doubles_kernel<<<1, kBlock, 0, stream()>>>(err_part, grid, abs_err);
    check_launch("sum_doubles_kernel");
  }
}

}  // namespace

// Per-row symmetric int8 codes for callers inside the library that manage
// their own scratch (zp_scratch receives the all-zero zero points).
void quantize_rows_i8_internal(const float* x, int64_t rows, int64_t cols, int8_t* codes,
                               float* scale, float* zp_scratch) {
  QParams p = make_params(8, ENQ_SYMMETRIC);
  rows_quantize<float>(x, rows, cols, p, nullptr, codes, scale, zp_scratch, nullptr);
}

}  // namespace enq

using namespace enq;

extern "C" {

int enq_minmax(int dtype, const void* x, int64_t outer, int64_t channels, int64_t inner,
               void* low, void* high) {
  return guarded([&] {
    require_init();
    check_dtype(dtype);
    check_shape(outer, channels, inner);
    ENQ_REQUIRE(x && low && high, "NULL pointer argument");
    QParams p = make_params(8, ENQ_SYMMETRIC);
    if (dtype == ENQ_F32)
      range_stats<float>(static_cast<const float*>(x), outer, channels, inner, p, false,
                         static_cast<float*>(low), static_cast<float*>(high), nullptr, nullptr);
    else
      range_stats<double>(static_cast<const double*>(x), outer, channels, inner, p, false,
                          static_cast<double*>(low), static_cast<double*>(high), nullptr,
                          nullptr);
  });
}

int enq_compute_scale(int dtype, const void* low, const void* high, int64_t n, int bits,
                      int scheme, void* scale, void* zero_point) {
  return guarded([&] {
    require_init();
    check_dtype(dtype);
    QParams p = make_params(bits, scheme);
    ENQ_REQUIRE(n >= 0, "n must be >= 0");
    if (n == 0) return;
    ENQ_REQUIRE(low && high && scale && zero_point, "NULL pointer argument");
    const int64_t grid = ceil_div(n, kBlock);
    ENQ_REQUIRE(grid <= 0x7fffffff, "n too large");
    if (dtype == ENQ_F32)
      compute_scale_kernel<float><<<unsigned(grid), kBlock, 0, stream()>>>(
          static_cast<const float*>(low), static_cast<const float*>(high), n, p,
          static_cast<float*>(scale), static_cast<float*>(zero_point));
    else
      compute_scale_kernel<double><<<unsigned(grid), kBlock, 0, stream()>>>(
          static_cast<const double*>(low), static_cast<const double*>(high), n, p,
          static_cast<double*>(scale), static_cast<double*>(zero_point));
    check_launch("compute_scale_kernel");
  });
}

static int elementwise_entry(Op op, int dtype, const void* x, int64_t outer, int64_t channels,
                             int64_t inner, const void* scale, const void* zp, int qmin, int qmax,
                             void* out) {
  return guarded([&] {
    require_init();
    check_dtype(dtype);
    check_shape(outer, channels, inner);
    ENQ_REQUIRE(x && scale && out, "NULL pointer argument");
    ENQ_REQUIRE(zp || op == Op::kDequantI8, "zero_point is NULL");
    ENQ_REQUIRE(qmin <= qmax, "qmin > qmax");
    QParams p;
    p.scheme = ENQ_SYMMETRIC;
    p.qmin = qmin;
    p.qmax = qmax;
    const int64_t n = outer * channels * inner;
    auto run = [&](auto tag) {
      using T = decltype(tag);
      const T* s = static_cast<const T*>(scale);
      const T* z = static_cast<const T*>(zp);
      T* o = static_cast<T*>(out);
      const int grid = elementwise_grid<T>(n);
      switch (op) {
        case Op::kQuantize:
          launch_elementwise<T, Op::kQuantize>(x, n, channels, inner, s, z, p, o, nullptr,
                                               nullptr, grid);
          break;
        case Op::kDequantize:
          launch_elementwise<T, Op::kDequantize>(x, n, channels, inner, s, z, p, o, nullptr,
                                                 nullptr, grid);
          break;
        case Op::kFake:
          launch_elementwise<T, Op::kFake>(x, n, channels, inner, s, z, p, o, nullptr, nullptr,
                                           grid);
          break;
        case Op::kDequantI8:
          if (n % 4 == 0 && inner % 4 == 0 && aligned(x, 4) && aligned(o, 16)) {
            constexpr int kUnits = 2;
            const int64_t g = ceil_div(n / 4, int64_t(kBlock) * kUnits);
            ENQ_REQUIRE(g <= 0x7fffffff, "tensor too large");
            dequant_i8_kernel<T, kUnits><<<unsigned(g), kBlock, 0, stream()>>>(
                static_cast<const int8_t*>(x), n, make_map(n, channels, inner), s, o);
            check_launch("dequant_i8_kernel");
          } else {
            launch_elementwise<T, Op::kDequantI8>(x, n, channels, inner, s, nullptr, p, o,
                                                  nullptr, nullptr, grid);
          }
          break;
        default:
          fail(ENQ_ERR_INVALID, "bad op");
      }
    };
    if (dtype == ENQ_F32)
      run(float{});
    else
      run(double{});
  });
}

int enq_quantize(int dtype, const void* x, int64_t outer, int64_t channels, int64_t inner,
                 const void* scale, const void* zero_point, int qmin, int qmax, void* codes) {
  return elementwise_entry(Op::kQuantize, dtype, x, outer, channels, inner, scale, zero_point,
                           qmin, qmax, codes);
}

int enq_quantize_codes_i8(int dtype, const void* x, int64_t outer, int64_t channels,
                          int64_t inner, const void* scale, const void* zero_point, int qmin,
                          int qmax, int8_t* codes) {
  return guarded([&] {
    require_init();
    check_dtype(dtype);
    check_shape(outer, channels, inner);
    ENQ_REQUIRE(x && scale && zero_point && codes, "NULL pointer argument");
    ENQ_REQUIRE(qmin <= qmax && qmin >= -128 && qmax <= 127,
                "int8 codes need qmin <= qmax inside [-128, 127]");
    QParams p;
    p.scheme = ENQ_SYMMETRIC;
    p.qmin = qmin;
    p.qmax = qmax;
    const int64_t n = outer * channels * inner;
    auto run = [&](auto tag) {
      using T = decltype(tag);
      launch_elementwise<T, Op::kFakeTensor>(x, n, channels, inner, static_cast<const T*>(scale),
                                             static_cast<const T*>(zero_point), p, nullptr,
                                             codes, nullptr, elementwise_grid<T>(n));
    };
    if (dtype == ENQ_F32)
      run(float{});
    else
      run(double{});
  });
}

int enq_dequantize(int dtype, const void* q, int64_t outer, int64_t channels, int64_t inner,
                   const void* scale, const void* zero_point, void* out) {
  return elementwise_entry(Op::kDequantize, dtype, q, outer, channels, inner, scale, zero_point,
                           0, 0, out);
}

int enq_fake_quantize(int dtype, const void* x, int64_t outer, int64_t channels, int64_t inner,
                      const void* scale, const void* zero_point, int qmin, int qmax, void* out) {
  return elementwise_entry(Op::kFake, dtype, x, outer, channels, inner, scale, zero_point, qmin,
                           qmax, out);
}

int enq_dequantize_i8(int dtype, const int8_t* codes, int64_t outer, int64_t channels,
                      int64_t inner, const void* scale, void* out) {
  return elementwise_entry(Op::kDequantI8, dtype, codes, outer, channels, inner, scale, nullptr,
                           0, 0, out);
}

int enq_quantize_tensor(int dtype, const void* w, int64_t outer, int64_t channels, int64_t inner,
                        int bits, int scheme, void* out_fake, int8_t* out_codes, void* scale,
                        void* zero_point, double* abs_err) {
  return guarded([&] {
    require_init();
    check_dtype(dtype);
    check_shape(outer, channels, inner);
    QParams p = make_params(bits, scheme);
    ENQ_REQUIRE(w && scale && zero_point, "NULL pointer argument");
    ENQ_REQUIRE(out_fake || out_codes || abs_err, "no output requested");
    ENQ_REQUIRE(out_codes == nullptr || (p.qmin >= -128 && p.qmax <= 127),
                "int8 codes need a grid inside [-128, 127] (bits <= 8, symmetric)");
    if (dtype == ENQ_F32)
      quantize_tensor_impl<float>(static_cast<const float*>(w), outer, channels, inner, p,
                                  static_cast<float*>(out_fake), out_codes,
                                  static_cast<float*>(scale), static_cast<float*>(zero_point),
                                  abs_err);
    else
      quantize_tensor_impl<double>(static_cast<const double*>(w), outer, channels, inner, p,
                                   static_cast<double*>(out_fake), out_codes,
                                   static_cast<double*>(scale),
                                   static_cast<double*>(zero_point), abs_err);
  });
}

int enq_quantize_rows_i8(const float* x, int64_t rows, int64_t cols, int8_t* codes,
                         float* scale) {
  return guarded([&] {
    require_init();
    ENQ_REQUIRE(rows >= 1 && cols >= 1, "rows and cols must be positive");
    ENQ_REQUIRE(x && codes && scale, "NULL pointer argument");
    QParams p = make_params(8, ENQ_SYMMETRIC);
    float* zp = static_cast<float*>(workspace(sizeof(float) * rows));
    rows_quantize<float>(x, rows, cols, p, nullptr, codes, scale, zp, nullptr);
  });
}

int enq_error_stats(int dtype, const void* reference, const void* candidate, int64_t n,
                    double* host_out4) {
  return guarded([&] {
    require_init();
    check_dtype(dtype);
    ENQ_REQUIRE(n >= 1, "n must be >= 1");
    ENQ_REQUIRE(reference && candidate && host_out4, "NULL pointer argument");
    const int grid = grid_for(n);
    auto* part = static_cast<double*>(workspace(sizeof(double) * (4 * grid + 4)));
    double* result = part + 4 * grid;
    if (dtype == ENQ_F32)
      error_stats_kernel<float><<<grid, kBlock, 0, stream()>>>(
          static_cast<const float*>(reference), static_cast<const float*>(candidate), n, part);
    else
      error_stats_kernel<double><<<grid, kBlock, 0, stream()>>>(
          static_cast<const double*>(reference), static_cast<const double*>(candidate), n, part);
    check_launch("error_stats_kernel");
    error_finish_kernel<<<1, 64, 0, stream()>>>(part, grid, result);
    check_launch("error_finish_kernel");
    ENQ_HIP(hipMemcpyAsync(host_out4, result, 4 * sizeof(double), hipMemcpyDeviceToHost,
                           stream()));
    ENQ_HIP(hipStreamSynchronize(stream()));
  });
}

}  // extern "C"
