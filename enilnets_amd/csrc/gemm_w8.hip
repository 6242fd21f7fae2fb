// Dense on int8 weights with fp32 activations (the W8 path).
//
//   y = act(scale[n] * sum_k x[m,k] * codes[n,k] + bias[n])
//
// The codes are integers in [-127, 127], exact in bf16, so the weight side of
// every MFMA product is exact.  The activations are split into bf16 planes:
// hi = bf16(x), lo = bf16(x - hi) (ENQ_W8_FP32; residual |x - hi - lo| is
// about 2^-17 |x|, far inside the 1e-4 * ||row||_inf tolerance), or hi only
// (ENQ_W8_BF16).  Both planes accumulate into one fp32 MFMA accumulator.
//
// Kernels
//   split_planes_kernel  x (m, k) fp32 -> P bf16 planes (mp, kp), zero padded
//   gemv_w8_kernel       m <= 64, or n <= 32 (grid z over 16-row blocks):
//                        split-K, W streamed with 128-bit loads, 16x16x32
//                        bf16 MFMA, partial sums per K-split
//   gemv_finish_kernel   sums the K-split partials, scale, bias, activation
//   w8_ring_kernel       m > 64: direct-to-LDS multi-stage ring, int8 tiles
//                        expanded to bf16 in registers, fused epilogue
//   w8_gemm_kernel       the same GEMM with register staging, for K not a
//                        multiple of 16 or unaligned codes
#include <algorithm>
#include "common.hpp"
#include "epilogue.hpp"
#include "mfma.hpp"
#include "ops.hpp"
#include "tiling.hpp"

namespace enq {
namespace {

// ---------------------------------------------------------------------------
// Activation split into bf16 planes
// ---------------------------------------------------------------------------
// Row r of the planes comes from row gather[r] of x (gather == nullptr: row r).
template <int PLANES>
__global__ __launch_bounds__(256) void split_planes_kernel(const float* __restrict__ x,
                                                           const int* __restrict__ gather,
                                                           int64_t m, int64_t k,
                                                           uint16_t* __restrict__ out,
                                                           int64_t mp, int64_t kp, int vec) {
  // one thread per 8 consecutive elements of a padded row
  const int64_t groups_per_row = kp / 8;
  const int64_t gid = int64_t(blockIdx.x) * 256 + threadIdx.x;
  if (gid >= mp * groups_per_row) return;
  const int64_t row = gid / groups_per_row;
  const int64_t k0 = (gid - row * groups_per_row) * 8;
  const int64_t src = row < m ? (gather ? int64_t(gather[row]) : row) : 0;
  const float* xr = x + src * k;
  float v[8];
  if (row < m && vec && k0 + 8 <= k) {
    const float4 a = *reinterpret_cast<const float4*>(xr + k0);
    const float4 b = *reinterpret_cast<const float4*>(xr + k0 + 4);
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = (row < m && k0 + e < k) ? xr[k0 + e] : 0.0f;
  }
  Pack8 hi, lo;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    uint16_t h = bf16_bits_rne(v[e]);
    hi.h[e] = h;
    if (PLANES == 2) lo.h[e] = bf16_bits_rne(v[e] - bf16_to_float(h));
  }
  *reinterpret_cast<Pack8*>(out + row * kp + k0) = hi;
  if (PLANES == 2) *reinterpret_cast<Pack8*>(out + mp * kp + row * kp + k0) = lo;
}

// ---------------------------------------------------------------------------
// Weight loads: 16 int8 codes of row `row` starting at column k0.
// KMODE 0: k % 32 == 0, aligned rows, no guard.  1: k % 16 == 0, a 16-byte
// chunk is entirely inside or outside.  2: byte-wise guard.
// ---------------------------------------------------------------------------
template <int KMODE>
__device__ __forceinline__ int4 load_codes16(const int8_t* __restrict__ w, int64_t ldw, int64_t row,
                                             int64_t k0, int64_t k) {
  const int8_t* p = w + row * ldw + k0;
  if constexpr (KMODE == 0) {
    return *reinterpret_cast<const int4*>(p);
  } else if constexpr (KMODE == 1) {
    if (k0 < k) return *reinterpret_cast<const int4*>(p);
    return make_int4(0, 0, 0, 0);
  } else {
    uint32_t wd[4] = {0, 0, 0, 0};
#pragma unroll
    for (int e = 0; e < 16; ++e)
      if (k0 + e < k) wd[e / 4] |= uint32_t(uint8_t(p[e])) << (8 * (e % 4));
    return make_int4(int(wd[0]), int(wd[1]), int(wd[2]), int(wd[3]));
  }
}

// ---------------------------------------------------------------------------
// Activation fragments straight from fp32: 8 consecutive values of a row
// (zero outside the matrix), split into bf16 hi (and lo) parts.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void load_row8(const float* __restrict__ x, int64_t row, int64_t m,
                                          int64_t k, int64_t k0, bool vec, float (&v)[8]) {
  const float* p = x + row * k + k0;
  if (row < m && vec && k0 + 8 <= k) {
    const float4 a = *reinterpret_cast<const float4*>(p);
    const float4 b = *reinterpret_cast<const float4*>(p + 4);
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = (row < m && k0 + e < k) ? p[e] : 0.0f;
  }
}

template <int PLANES>
__device__ __forceinline__ void split8(const float (&v)[8], Pack8& hi, Pack8& lo) {
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const uint16_t h = bf16_bits_rne(v[e]);
    hi.h[e] = h;
    if (PLANES == 2) lo.h[e] = bf16_bits_rne(v[e] - bf16_to_float(h));
  }
}

// ---------------------------------------------------------------------------
// GEMV kernels.  Lane layout per 128-wide K chunk: lane l covers column
// n = l % 16 and, in lane group g = l / 16, the 16-byte pieces
// k = 16 g + [0, 16) and 64 + 16 g + [0, 16), so each of the two 128-bit
// weight loads of a chunk reads 64 contiguous bytes of 16 rows.  MFMA i of
// the chunk (16x16x32 bf16, x as the A operand) takes k offsets
// gemv_koff(g, i) + [0, 8).  Both kernels write fp32 partial sums per K
// slice, part[slice][row][n], which gemv_finish_kernel adds up with the
// scale, bias and activation (the skinny kernel applies them itself when
// there is one slice).
//
// Every load of these kernels is issued unconditionally from an address
// clamped into its array, and out-of-range values are zeroed where they are
// used.  A branch around a load whose other arm writes zeros into the same
// registers makes the compiler wait for the load before the arms rejoin,
// which serialises a wave's loads one round trip at a time.
// ---------------------------------------------------------------------------
__device__ __forceinline__ int gemv_koff(int g, int i) { return 64 * (i >> 1) + 16 * g + 8 * (i & 1); }

constexpr int kGemvWaves = 8;
constexpr int kGemvChunk = 128;
// 16-column blocks per wave of the decode GEMV: two halve the activation
// re-reads but measured slower at M = 16, N = K = 8192 (23.4 against 21.0 us
// for the kernel), one workgroup per CU instead of two
constexpr int kDecodeCB = 1;
// outputs this narrow go through the GEMV even for many rows: a GEMM tile
// grid over them has too few workgroups to stream the activations
constexpr int64_t kSkinnyN = 32;

// 16 codes of row `row` from column k0, loaded without a guard branch: for
// KMODE 1 a piece past k reads the row's last piece instead (zeroed later by
// mask_codes16); KMODE 2 keeps the byte-wise guarded load.
template <int KMODE>
__device__ __forceinline__ int4 load_codes16_raw(const int8_t* __restrict__ w, int64_t ldw,
                                                 int64_t row, int64_t k0, int64_t k) {
  if constexpr (KMODE == 2) {
    return load_codes16<2>(w, ldw, row, k0, k);
  } else {
    const int64_t kk = (KMODE == 0 || k0 < k) ? k0 : k - 16;
    return *reinterpret_cast<const int4*>(w + row * ldw + kk);
  }
}

template <int KMODE>
__device__ __forceinline__ int4 mask_codes16(int4 v, int64_t k0, int64_t k) {
  if constexpr (KMODE == 1) return k0 < k ? v : make_int4(0, 0, 0, 0);
  return v;
}

// Eight consecutive activations x[row, k0:k0+8] as two float4 loads from
// clamped addresses (k % 4 == 0 and 16-byte aligned rows), and their
// zero-masked values once loaded.
__device__ __forceinline__ void load_row8_raw(const float* __restrict__ x, int64_t row, int64_t m,
                                              int64_t k, int64_t k0, float4 (&r)[2]) {
  const float* p = x + (row < m ? row : m - 1) * k;
  r[0] = *reinterpret_cast<const float4*>(p + (k0 < k ? k0 : 0));
  r[1] = *reinterpret_cast<const float4*>(p + (k0 + 4 < k ? k0 + 4 : 0));
}

__device__ __forceinline__ void row8_values(const float4 (&r)[2], int64_t row, int64_t m,
                                            int64_t k, int64_t k0, float (&v)[8]) {
  const bool a = row < m && k0 < k, b = row < m && k0 + 4 < k;
  v[0] = a ? r[0].x : 0.f; v[1] = a ? r[0].y : 0.f; v[2] = a ? r[0].z : 0.f; v[3] = a ? r[0].w : 0.f;
  v[4] = b ? r[1].x : 0.f; v[5] = b ? r[1].y : 0.f; v[6] = b ? r[1].z : 0.f; v[7] = b ? r[1].w : 0.f;
}

// scale, bias and activation of one GEMV output (the finish of one sum)
__device__ __forceinline__ void gemv_output(float s, int64_t row, int64_t c, int64_t n,
                                            const float* __restrict__ scale,
                                            const float* __restrict__ bias, const Epilogue& ep,
                                            float* __restrict__ y, float* __restrict__ z) {
  float v = s * scale[c];
  if (bias) v = v + bias[c];
  if (z) z[row * n + c] = v;
  y[row * n + c] = epilogue_out(v, ep);
}

// Decode GEMV (m <= 64): grid (groups of 8 waves x CB x 16 columns, K slices
// of kr).  The workgroup splits its activation slice x[0:16 MB, k0:k0+kr]
// into bf16 planes in LDS once (rows padded by 16 bytes: a row pitch of 16
// modulo 128 bytes puts the 16-byte fragment reads of 8 consecutive rows on
// 8 distinct bank groups); each wave then owns CB blocks of 16 columns over
// the whole slice, so one activation fragment read feeds CB MFMAs.  A wave
// issues its activation loads, then all its weight loads, and stages the
// activations while the weights are in flight.
//
// With one slice the workgroup writes the outputs; otherwise it writes
// partial sums, part[slice][row][n], for gemv_finish_kernel.  (Adding the
// slices up inside the kernel, by the last slice of a column group to finish,
// needs an agent-scope release and acquire per workgroup; on gfx950 those
// write back and invalidate the whole L2 of the XCD, which measured 3.6x
// slower than the separate finish pass.)
template <int MB, int PLANES, int KMODE, int CHUNKS, int CB>
__global__ __launch_bounds__(512) void gemv_decode_kernel(
    const float* __restrict__ x, int64_t m, int64_t k, int vec, const int8_t* __restrict__ w,
    int64_t n, int kr, int splits, float* __restrict__ part,
    const float* __restrict__ scale, const float* __restrict__ bias, Epilogue ep,
    float* __restrict__ y, float* __restrict__ z) {
  extern __shared__ __align__(16) uint16_t xs[];
  constexpr int ROWS = 16 * MB;
  constexpr int COLS = kGemvWaves * CB * 16;  // columns of a workgroup
  // ROWS x kr / 8 staging items <= 16 x 1024 / 8 = ITEMS per thread x 512
  constexpr int ITEMS = 4;
  const int pitch = kr + 8;  // bf16 elements per LDS row
  const int64_t k0 = int64_t(blockIdx.y) * kr;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int col = lane & 15, grp = lane >> 4;
  const int64_t c0 = int64_t(blockIdx.x) * COLS;
  const int64_t n0 = c0 + int64_t(wave) * CB * 16;  // first column of this wave
  const bool active = n0 < n;
  const int64_t k_end = k0 + kr < k ? k0 + kr : k;
  const int nchunks = int((k_end - k0 + kGemvChunk - 1) / kGemvChunk);  // >= 1
  const int groups8 = kr / 8, items = ROWS * groups8;

  float4 xr[ITEMS][2];
  if (vec) {
#pragma unroll
    for (int it = 0; it < ITEMS; ++it) {
      const int idx = threadIdx.x + it * 512;
      const int r = idx < items ? idx / groups8 : 0;
      const int c8 = idx < items ? (idx - r * groups8) * 8 : 0;
      load_row8_raw(x, r, m, k, k0 + c8, xr[it]);
    }
  }
  int4 wc[CB][CHUNKS][2];
#pragma unroll
  for (int b = 0; b < CB; ++b) {
    int64_t wrow = n0 + b * 16 + col;
    wrow = wrow < n ? wrow : n - 1;
#pragma unroll
    for (int c = 0; c < CHUNKS; ++c) {
      // chunks past the slice re-read its last chunk; their MFMAs are skipped
      const int cc = c < nchunks ? c : nchunks - 1;
      const int64_t kc = k0 + int64_t(cc) * kGemvChunk + 16 * grp;
      wc[b][c][0] = load_codes16_raw<KMODE>(w, k, wrow, kc, k);
      wc[b][c][1] = load_codes16_raw<KMODE>(w, k, wrow, kc + 64, k);
    }
  }
  if (vec) {
#pragma unroll
    for (int it = 0; it < ITEMS; ++it) {
      const int idx = threadIdx.x + it * 512;
      if (idx < items) {
        const int r = idx / groups8, c8 = (idx - r * groups8) * 8;
        float v[8];
        row8_values(xr[it], r, m, k, k0 + c8, v);
        Pack8 hi, lo;
        split8<PLANES>(v, hi, lo);
        *reinterpret_cast<Pack8*>(xs + r * pitch + c8) = hi;
        if (PLANES == 2) *reinterpret_cast<Pack8*>(xs + (ROWS + r) * pitch + c8) = lo;
      }
    }
  } else {
    for (int idx = threadIdx.x; idx < items; idx += 512) {
      const int r = idx / groups8, c8 = (idx - r * groups8) * 8;
      float v[8];
      load_row8(x, r, m, k, k0 + c8, false, v);
      Pack8 hi, lo;
      split8<PLANES>(v, hi, lo);
      *reinterpret_cast<Pack8*>(xs + r * pitch + c8) = hi;
      if (PLANES == 2) *reinterpret_cast<Pack8*>(xs + (ROWS + r) * pitch + c8) = lo;
    }
  }
  __syncthreads();
  if (!active) return;  // no barrier follows
  floatx4 acc[CB][MB];
#pragma unroll
  for (int b = 0; b < CB; ++b)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) acc[b][mb] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int c = 0; c < CHUNKS; ++c) {
    if (c >= nchunks) break;
    const int64_t kc = k0 + int64_t(c) * kGemvChunk + 16 * grp;
    bf16x8 wb[CB][4];
#pragma unroll
    for (int b = 0; b < CB; ++b) {
      codes16_to_bf16(mask_codes16<KMODE>(wc[b][c][0], kc, k), wb[b][0], wb[b][1]);
      codes16_to_bf16(mask_codes16<KMODE>(wc[b][c][1], kc + 64, k), wb[b][2], wb[b][3]);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int p = 0; p < PLANES; ++p) {
          const bf16x8 xf = *reinterpret_cast<const bf16x8*>(
              xs + (p * ROWS + mb * 16 + col) * pitch + c * kGemvChunk + gemv_koff(grp, i));
#pragma unroll
          for (int b = 0; b < CB; ++b) acc[b][mb] = mfma_16x16x32_bf16(xf, wb[b][i], acc[b][mb]);
        }
  }
  // 16x16 output layout: lane holds column l % 16, rows 4 * (l / 16) + r
#pragma unroll
  for (int b = 0; b < CB; ++b) {
    const int64_t cn = n0 + b * 16 + col;
    if (cn >= n) continue;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int64_t row = mb * 16 + 4 * grp + r;
        if (splits == 1) {
          if (row < m) gemv_output(0.f + acc[b][mb][r], row, cn, n, scale, bias, ep, y, z);
        } else {
          part[(int64_t(blockIdx.y) * ROWS + row) * n + cn] = acc[b][mb][r];
        }
      }
  }
}

// Tall-skinny GEMV (n <= 32, any m): grid (column groups, K splits, 16-row
// blocks).  Each wave owns a K range of `chunks_per_wave` (<= CHUNKS) x 128
// and keeps the activation fragments of its rows in registers, read from
// fp32 and split there; it then streams 16-column blocks of W (the next
// block's loads in flight while one is multiplied), and the 8 waves' partial
// tiles are summed through LDS.  With one K split (part == nullptr) the
// kernel finishes the outputs itself.  CHUNKS is the host's bound on
// chunks_per_wave: loading two chunks for waves that own one (K = 1024)
// doubled the activation requests and the registers, and the kernel streamed
// at 2.1 TB/s.
template <int PLANES, int KMODE, int CHUNKS>
__global__ __launch_bounds__(512) void gemv_skinny_kernel(
    const float* __restrict__ x, int64_t m, int64_t k, int vec, const int8_t* __restrict__ w,
    int64_t n, int chunks_per_wave, int col_blocks_per_group, int64_t mp,
    float* __restrict__ part, const float* __restrict__ scale, const float* __restrict__ bias,
    Epilogue ep, float* __restrict__ y, float* __restrict__ z) {
  __shared__ float red[kGemvWaves][16][17];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int col = lane & 15;
  const int grp = lane >> 4;
  const int64_t k_wave0 = (int64_t(blockIdx.y) * kGemvWaves + wave) * chunks_per_wave * kGemvChunk;
  const int64_t row0 = int64_t(blockIdx.z) * 16;
  const int64_t xrow = row0 + col;

  // activation loads first, then the first block's weights
  float4 xr[CHUNKS][4][2];
  if (vec) {
#pragma unroll
    for (int c = 0; c < CHUNKS; ++c)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        load_row8_raw(x, xrow, m, k, k_wave0 + int64_t(c) * kGemvChunk + gemv_koff(grp, i),
                      xr[c][i]);
  }
  auto load_block = [&](int cb, int4 (&wc)[CHUNKS][2]) {
    int64_t nb = (int64_t(blockIdx.x) * col_blocks_per_group + cb) * 16 + col;
    nb = nb < n ? nb : n - 1;
#pragma unroll
    for (int c = 0; c < CHUNKS; ++c) {
      // a chunk past k re-reads valid codes (KMODE 0, k % 128 == 0: the
      // last chunk; otherwise the loader clamps each piece); they are zeroed
      // below
      int64_t kb = k_wave0 + int64_t(c) * kGemvChunk;
      if (KMODE == 0) kb = kb < k ? kb : k - kGemvChunk;
      const int64_t kc = kb + 16 * grp;
      wc[c][0] = load_codes16_raw<KMODE>(w, k, nb, kc, k);
      wc[c][1] = load_codes16_raw<KMODE>(w, k, nb, kc + 64, k);
    }
  };
  int4 wc[CHUNKS][2], wn[CHUNKS][2];
  load_block(0, wc);

  bf16x8 xf[CHUNKS][PLANES][4];
#pragma unroll
  for (int c = 0; c < CHUNKS; ++c) {
    const int64_t kc = k_wave0 + int64_t(c) * kGemvChunk;
    const bool live = c < chunks_per_wave;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float v[8];
      if (vec)
        row8_values(xr[c][i], live ? xrow : m, m, k, kc + gemv_koff(grp, i), v);
      else
        load_row8(x, live ? xrow : m, m, k, kc + gemv_koff(grp, i), false, v);
      Pack8 hi, lo;
      split8<PLANES>(v, hi, lo);
      xf[c][0][i] = __builtin_bit_cast(bf16x8, hi);
      if (PLANES == 2) xf[c][PLANES - 1][i] = __builtin_bit_cast(bf16x8, lo);
    }
  }

  for (int cb = 0; cb < col_blocks_per_group; ++cb) {
    const int64_t n0 = (int64_t(blockIdx.x) * col_blocks_per_group + cb) * 16;
    if (n0 >= n) break;
    const bool next = cb + 1 < col_blocks_per_group && n0 + 16 < n;
    if (next) load_block(cb + 1, wn);
    floatx4 acc = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < CHUNKS; ++c) {
      const int64_t kbase = k_wave0 + int64_t(c) * kGemvChunk;
      const bool live = c < chunks_per_wave && kbase < k;
      const int64_t kc = kbase + 16 * grp;
      const int4 z4 = make_int4(0, 0, 0, 0);
      bf16x8 wb[4];
      codes16_to_bf16(live ? mask_codes16<KMODE>(wc[c][0], kc, k) : z4, wb[0], wb[1]);
      codes16_to_bf16(live ? mask_codes16<KMODE>(wc[c][1], kc + 64, k) : z4, wb[2], wb[3]);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int p = 0; p < PLANES; ++p) acc = mfma_16x16x32_bf16(xf[c][p][i], wb[i], acc);
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) red[wave][4 * grp + r][col] = acc[r];
    __syncthreads();
    if (threadIdx.x < 256) {
      const int mm = threadIdx.x >> 4, nn = threadIdx.x & 15;
      float s = 0.f;
#pragma unroll
      for (int v = 0; v < kGemvWaves; ++v) s += red[v][mm][nn];
      if (n0 + nn < n) {
        if (part)
          part[(int64_t(blockIdx.y) * mp + row0 + mm) * n + n0 + nn] = s;
        else if (row0 + mm < m)
          gemv_output(0.f + s, row0 + mm, n0 + nn, n, scale, bias, ep, y, z);
      }
    }
    __syncthreads();
    if (next) {
#pragma unroll
      for (int c = 0; c < CHUNKS; ++c) {
        wc[c][0] = wn[c][0];
        wc[c][1] = wn[c][1];
      }
    }
  }
}

__global__ __launch_bounds__(256) void gemv_finish_kernel(const float* __restrict__ part,
                                                          int splits, int64_t mp, int64_t m,
                                                          int64_t n, const float* __restrict__ scale,
                                                          const float* __restrict__ bias,
                                                          Epilogue ep, float* __restrict__ y,
                                                          float* __restrict__ z) {
  const int64_t idx = int64_t(blockIdx.x) * 256 + threadIdx.x;
  if (idx >= m * n) return;
  const int64_t row = idx / n, c = idx - row * n;
  const float* p = part + row * n + c;
  const int64_t stride = mp * n;
  // eight slices' loads in flight at a time; the sum keeps slice order
  float s = 0.f;
  int sp = 0;
  for (; sp + 8 <= splits; sp += 8) {
    float v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = p[int64_t(sp + j) * stride];
#pragma unroll
    for (int j = 0; j < 8; ++j) s += v[j];
  }
  for (; sp < splits; ++sp) s += p[int64_t(sp) * stride];
  gemv_output(s, row, c, n, scale, bias, ep, y, z);
}

// ---------------------------------------------------------------------------
// GEMM (m > 64): BM x BN block tile, BK = 32, WM x WN waves.
// LDS rows are 32 bf16 + 8 pad (80 bytes): 16 consecutive rows then fall in
// 16 distinct 16-byte bank groups for the MFMA operand reads.
// ---------------------------------------------------------------------------
constexpr int kBK = 32;
constexpr int kPitch = 40;  // bf16 elements per LDS row

template <int BM, int BN, int WM, int WN, int PLANES, int KMODE>
__global__ __launch_bounds__(WM * WN * 64) void w8_gemm_kernel(
    const uint16_t* __restrict__ xa, int64_t plane_stride, int64_t kp,
    const int8_t* __restrict__ w, int64_t ldw, const float* __restrict__ scale,
    const float* __restrict__ bias, int64_t m, int64_t n, int64_t k, int tiles_m, int tiles_n,
    Epilogue ep, float* __restrict__ y, float* __restrict__ z) {
  constexpr int NT = WM * WN * 64;
  constexpr int TM = BM / WM, TN = BN / WN;
  constexpr int FM = TM / 32, FN = TN / 32;
  constexpr int A_CHUNKS = PLANES * BM * (kBK / 8);  // 16-byte chunks per stage
  constexpr int B_CHUNKS = BN * (kBK / 16);          // 16 codes per chunk
  static_assert(A_CHUNKS % NT == 0, "A tile must split evenly over threads");
  static_assert(B_CHUNKS <= NT && NT % B_CHUNKS == 0, "B tile must split over threads");
  constexpr int A_PER_T = A_CHUNKS / NT;

  extern __shared__ __align__(16) uint16_t lds[];
  uint16_t* lds_a = lds;                                  // [2][PLANES][BM][kPitch]
  uint16_t* lds_b = lds + 2 * PLANES * BM * kPitch;       // [2][BN][kPitch]

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;

  int tm, tn;
  xcd_tile(blockIdx.x, tiles_m, tiles_n, 4, tm, tn);
  const int64_t m0 = int64_t(tm) * BM;
  const int64_t n0 = int64_t(tn) * BN;

  // global -> register staging
  int4 a_reg[A_PER_T];
  int4 b_reg;
  const bool b_loader = tid < B_CHUNKS;

  auto load_stage = [&](int64_t k0) {
#pragma unroll
    for (int i = 0; i < A_PER_T; ++i) {
      const int q = tid + i * NT;
      const int p = q / (BM * 4);
      const int r = (q / 4) % BM;
      const int c = q % 4;
      int64_t row = m0 + r;
      row = row < m ? row : m - 1;
      a_reg[i] = *reinterpret_cast<const int4*>(xa + p * plane_stride + row * kp + k0 + c * 8);
    }
    if (b_loader) {
      const int r = tid / 2, h = tid % 2;
      int64_t row = n0 + r;
      row = row < n ? row : n - 1;
      b_reg = load_codes16<KMODE>(w, ldw, row, k0 + h * 16, k);
    }
  };
  auto store_stage = [&](int buf) {
    uint16_t* la = lds_a + buf * PLANES * BM * kPitch;
#pragma unroll
    for (int i = 0; i < A_PER_T; ++i) {
      const int q = tid + i * NT;
      const int p = q / (BM * 4);
      const int r = (q / 4) % BM;
      const int c = q % 4;
      *reinterpret_cast<int4*>(la + (p * BM + r) * kPitch + c * 8) = a_reg[i];
    }
    if (b_loader) {
      const int r = tid / 2, h = tid % 2;
      bf16x8 lo8, hi8;
      codes16_to_bf16(b_reg, lo8, hi8);
      uint16_t* lb = lds_b + buf * BN * kPitch + r * kPitch + h * 16;
      *reinterpret_cast<bf16x8*>(lb) = lo8;
      *reinterpret_cast<bf16x8*>(lb + 8) = hi8;
    }
  };

  floatx16 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

  const int ktiles = int(kp / kBK);
  load_stage(0);
  store_stage(0);
  __syncthreads();
  if (ktiles > 1) load_stage(kBK);

  const int lrow = lane & 31;
  const int lk = (lane >> 5) * 8;
  for (int kt = 0; kt < ktiles; ++kt) {
    const int buf = kt & 1;
    const uint16_t* la = lds_a + buf * PLANES * BM * kPitch;
    const uint16_t* lb = lds_b + buf * BN * kPitch;
#pragma unroll
    for (int ks = 0; ks < kBK / 16; ++ks) {
      bf16x8 af[FM][PLANES], bfr[FN];
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int p = 0; p < PLANES; ++p)
          af[i][p] = *reinterpret_cast<const bf16x8*>(
              la + (p * BM + wm * TM + i * 32 + lrow) * kPitch + ks * 16 + lk);
#pragma unroll
      for (int j = 0; j < FN; ++j)
        bfr[j] = *reinterpret_cast<const bf16x8*>(lb + (wn * TN + j * 32 + lrow) * kPitch +
                                                  ks * 16 + lk);
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
          for (int p = 0; p < PLANES; ++p)
            acc[i][j] = mfma_32x32x16_bf16(af[i][p], bfr[j], acc[i][j]);
    }
    if (kt + 1 < ktiles) {
      store_stage(buf ^ 1);
      if (kt + 2 < ktiles) load_stage(int64_t(kt + 2) * kBK);
    }
    __syncthreads();
  }

  // epilogue: lane holds column l % 32, rows 8 * (e / 4) + 4 * (l / 32) + e % 4
#pragma unroll
  for (int j = 0; j < FN; ++j) {
    const int64_t col = n0 + wn * TN + j * 32 + (lane & 31);
    if (col >= n) continue;
    const float s = scale[col];
    const float b = bias ? bias[col] : 0.f;
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int64_t row = m0 + wm * TM + i * 32 + 8 * (e / 4) + 4 * (lane >> 5) + (e % 4);
        if (row < m) {
          float v = acc[i][j][e] * s;
          if (bias) v = v + b;
          if (z) z[row * n + col] = v;
          y[row * n + col] = activate(v, ep);
        }
      }
  }
}

// ---------------------------------------------------------------------------
// Ring W8 GEMM: activations as bf16 planes and int8 weight codes both stream
// into an LDS ring through direct-to-LDS loads (global_load_lds_dwordx4),
// STAGES - 1 stages in flight.  Per stage (32 columns of K):
//   A: PLANES x BM rows of 64 bytes (32 bf16), chunks XOR-swizzled (swz64);
//   B: BN rows of 32 bytes (32 codes), 16-byte halves swapped on bit 3 of the
//      row, so 16 consecutive rows read at one half hit distinct banks.
// Each stage's codes are expanded to bf16 once per workgroup (one 16-code
// item per thread) into one of two bf16 copies of the B tile (64-byte rows,
// swz64, the A layout), one stage ahead of the MFMAs that read them.
// Within a stage lane group g = l / 32 owns k in [16 g, 16 g + 16): the two
// 32x32x16 MFMA steps take k 16 g + [0, 8) and 16 g + [8, 16), i.e. chunks
// 2 g and 2 g + 1 of an A or bf16 B row.
// ---------------------------------------------------------------------------
// FUSED_A: A arrives as the fp32 activations themselves (128-byte rows per
// stage, 16-byte chunks XOR-swizzled by swz_a32) and each wave reads its
// 8-float runs straight from the ring and splits them into bf16 hi / lo
// fragments in registers; no separate pass.  Splitting once per workgroup
// into a double-buffered LDS copy instead moves a quarter more LDS bytes per
// stage and needs 32 KiB more LDS; it measured 1.5% slower on the MLP layer
// (4096 x 1024 x 1024).
template <int BM_, int BN_, int WM_, int WN_, int PLANES_, int STAGES_, bool FUSED_A_ = false>
struct RingCfg {
  static constexpr int BM = BM_, BN = BN_, WM = WM_, WN = WN_, PLANES = PLANES_;
  static constexpr int STAGES = STAGES_, BK = 32;
  static constexpr bool FUSED_A = FUSED_A_;
  static constexpr int NT = WM * WN * 64;
  static constexpr int TM = BM / WM, TN = BN / WN, FM = TM / 32, FN = TN / 32;
  // bf16 plane rows of 64 bytes, or fp32 rows of 128 bytes
  static constexpr int A_BYTES = FUSED_A ? BM * 128 : PLANES * BM * 64;
  static constexpr int B_BYTES = BN * 32;            // code rows of 32 bytes
  static constexpr int STAGE_BYTES = A_BYTES + B_BYTES;
  static constexpr int BCONV_BYTES = BN * 64;         // one bf16 copy of a B tile
  static constexpr int A_BLOCKS = A_BYTES / 1024, B_BLOCKS = B_BYTES / 1024;
  static constexpr int BLOCKS = A_BLOCKS + B_BLOCKS;
  // every wave issues the same number of 1 KiB blocks (vmcnt accounting);
  // waves past the last block repeat it, rewriting identical bytes
  static constexpr int DMA_PER_WAVE = (BLOCKS + NT / 64 - 1) / (NT / 64);
  static_assert(A_BYTES % 1024 == 0 && B_BYTES % 1024 == 0, "whole 1 KiB blocks");
  static constexpr int LDS_BYTES = STAGES * STAGE_BYTES + 2 * BCONV_BYTES;
  static_assert(LDS_BYTES <= 160 * 1024, "LDS budget");
  // workgroups the LDS lets a CU hold, and so the waves per SIMD
  static constexpr int WG_PER_CU = (160 * 1024) / LDS_BYTES;
  static constexpr int WAVES_PER_EU = (NT / 256) * WG_PER_CU < 8 ? (NT / 256) * WG_PER_CU : 8;
  static_assert((4 * BN) % NT == 0, "whole 8-code expansion items per thread");
};

// fp32 A rows of 128 bytes (8 chunks of 16): chunk XOR bits 1-3 of the row.
// A fragment read takes the same logical chunk of 32 consecutive rows; any
// 16 consecutive rows then cover the 16 chunk slots of two rows' 256 bytes
// (row parity x swizzled chunk) once each, so every 16 lanes are
// conflict-free.
__device__ __forceinline__ int swz_a32(int row, int chunk) { return chunk ^ ((row >> 1) & 7); }

// The ring's LDS bounds the workgroups per CU, and so the waves per SIMD:
// said to the compiler, which otherwise assumes eight and trades the
// registers that would hold a whole stage's fragments for occupancy it never
// gets.
// YP: the output goes to bf16 planes (yp) instead of fp32 (y); a separate
// instantiation, so the fp32-output kernels carry none of its registers.
template <class C, bool KTAIL, bool YP = false>
__global__ __launch_bounds__(C::NT) __attribute__((amdgpu_waves_per_eu(C::WAVES_PER_EU, C::WAVES_PER_EU)))
void w8_ring_kernel(
    const uint16_t* __restrict__ xa, int64_t plane_stride, int64_t kp,
    const float* __restrict__ x, const int8_t* __restrict__ w, const float* __restrict__ scale,
    const float* __restrict__ bias, int64_t m, int64_t n, int64_t k, int tiles_m, int tiles_n,
    RowGroups grp, Epilogue ep, float* __restrict__ y, float* __restrict__ z,
    uint16_t* __restrict__ yp, int64_t yp_plane_stride, int64_t yp_ld) {
  constexpr int BM = C::BM, BN = C::BN, WN = C::WN, PLANES = C::PLANES, STAGES = C::STAGES;
  constexpr int TM = C::TM, TN = C::TN, FM = C::FM, FN = C::FN, BK = C::BK;
  constexpr int DPW = C::DMA_PER_WAVE;
  extern __shared__ __align__(16) uint16_t lds_raw[];
  char* lds = reinterpret_cast<char*>(lds_raw);
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WN, wn = wave % WN;
  int tm, tn;
  xcd_tile(blockIdx.x, tiles_m, tiles_n, 4, tm, tn);
  int64_t m0 = int64_t(tm) * BM, m_end = m;
  const int64_t n0 = int64_t(tn) * BN;
  if (grp.offsets) {
    // grouped rows: tile row tm lives in the group whose tile range holds
    // it; workgroups past the last group's tiles have nothing to do
    const int e = group_tile(grp, BM, tm, m0, m_end);
    if (e < 0) return;
    w += int64_t(e) * grp.w_stride;
    scale += int64_t(e) * grp.v_stride;
    if (bias) bias += int64_t(e) * grp.v_stride;
  }

  // DMA sources.  Block b (of A_BLOCKS + B_BLOCKS per stage) is handled by
  // wave b / DPW.  A block: 16 rows x 64 B of one plane (fused: 8 rows x
  // 128 B of fp32); B block: 32 rows x 32 B.
  const char* src[DPW];
  int src_koff[DPW];   // byte offset of this lane's chunk inside a stage's K range
  bool is_b[DPW];
#pragma unroll
  for (int j = 0; j < DPW; ++j) {
    const int blk = min(wave * DPW + j, C::BLOCKS - 1);
    if (C::FUSED_A && blk < C::A_BLOCKS) {
      const int r = blk * 8 + (lane >> 3);
      const int chunk = swz_a32(r, lane & 7);               // logical chunk: 4 floats
      int64_t g = m0 + r;
      g = g < m ? g : m - 1;
      src[j] = reinterpret_cast<const char*>(x + g * k);
      src_koff[j] = chunk * 16;
      is_b[j] = false;
    } else if (blk < C::A_BLOCKS) {
      const int r_all = blk * 16 + (lane >> 2);          // row within the PLANES x BM rows
      const int p = r_all / BM, r = r_all % BM;
      const int chunk = swz64(r, lane & 3);                 // logical 16-byte chunk
      int64_t g = m0 + r;
      g = g < m ? g : m - 1;
      src[j] = reinterpret_cast<const char*>(xa + p * plane_stride + g * kp);
      src_koff[j] = chunk * 16;                              // bytes (8 bf16 per chunk)
      is_b[j] = false;
    } else {
      const int r = (blk - C::A_BLOCKS) * 32 + (lane >> 1);
      const int half = swz32(r, lane & 1);
      int64_t g = n0 + r;
      g = g < n ? g : n - 1;
      src[j] = reinterpret_cast<const char*>(w + g * k);
      src_koff[j] = half * 16;
      is_b[j] = true;
    }
  }
  const int ktiles = int(kp / BK);
  const void* zero = g_zero16;
  // Stages issued ahead of the one being multiplied: the A fragments of
  // stage t are read from the ring in iteration t, so stage t's slot is
  // refilled in iteration t + 1.
  constexpr int AHEAD = STAGES - 1;
  // blocks [J0, J1) of this wave's share of stage t
  auto issue_blocks = [&](int t, auto j0, auto j1) {
    const uint32_t dst = lds_addr(lds) + (t % STAGES) * C::STAGE_BYTES;
#pragma unroll
    for (int j = decltype(j0)::value; j < decltype(j1)::value; ++j) {
      const int blk = min(wave * DPW + j, C::BLOCKS - 1);
      // A planes hold 2 bytes per K column, B codes 1 byte
      const void* sp;
      if (is_b[j]) {
        const int64_t kb = int64_t(t) * BK + src_koff[j];
        sp = (KTAIL && kb >= k) ? zero : static_cast<const void*>(src[j] + kb);
      } else if (C::FUSED_A) {
        const int64_t ke = int64_t(t) * BK + src_koff[j] / 4;  // first column of the chunk
        sp = (KTAIL && ke >= k) ? zero
                                : static_cast<const void*>(src[j] + int64_t(t) * BK * 4 +
                                                           src_koff[j]);
      } else {
        sp = src[j] + int64_t(t) * BK * 2 + src_koff[j];
      }
      dma16(sp, dst + blk * 1024);
    }
  };
  // The steady loop issues a stage's DMA in two groups, the second after the
  // first half of the MFMAs, so the eight waves' blocks do not all reach the
  // memory pipeline at once after the barrier (as in the W8A8 ring).
  constexpr int DMA_HALF = DPW / 2;
  using JA = std::integral_constant<int, 0>;
  using JB = std::integral_constant<int, DMA_HALF>;
  using JC = std::integral_constant<int, DPW>;
  auto issue = [&](int t) { issue_blocks(t, JA{}, JC{}); };
  auto wait_stage = [&](int t, int issued) {
    const int later = (issued < ktiles - 1 ? issued : ktiles - 1) - t;
    wait_stages_after<DPW, AHEAD - 1>(later);
  };

  floatx16 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

  const int lrow = lane & 31, g = lane >> 5;
  // the epilogue's column scales and biases, loaded before the first DMA so
  // that they arrive during the main loop (a launch with one tile per CU
  // would otherwise wait a memory round trip after its last MFMA); being
  // older than every DMA they only make the stage waits conservative
  float col_scale[FN], col_bias[FN];
#pragma unroll
  for (int j = 0; j < FN; ++j) {
    int64_t col = n0 + wn * TN + j * 32 + lrow;
    col = col < n ? col : n - 1;
    col_scale[j] = scale[col];
    col_bias[j] = bias ? bias[col] : 0.f;
  }

  // bf16 copies of the B tiles, double-buffered after the ring: each tile
  // is expanded once per workgroup instead of once per wave that reads it
  char* bconv = lds + STAGES * C::STAGE_BYTES;
  int a_off[PLANES][FM][2], b_off[FN][2];
  // fused A: half h of the 8-float run of MFMA step ks, row of fragment i
  // (k = 16 g + 8 ks + [0, 8): logical chunks 4 g + 2 ks + h)
  int ar_off[FM][2][2];
#pragma unroll
  for (int i = 0; i < FM; ++i) {
    const int r = wm * TM + i * 32 + lrow;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
      for (int h = 0; h < 2; ++h) ar_off[i][ks][h] = r * 128 + 16 * swz_a32(r, 4 * g + 2 * ks + h);
  }
#pragma unroll
  for (int p = 0; p < PLANES; ++p)
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      const int r = wm * TM + i * 32 + lrow;
#pragma unroll
      for (int ks = 0; ks < 2; ++ks)
        a_off[p][i][ks] = (p * BM + r) * 64 + 16 * swz64(r, 2 * g + ks);
    }
#pragma unroll
  for (int j = 0; j < FN; ++j) {
    const int r = wn * TN + j * 32 + lrow;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) b_off[j][ks] = r * 64 + 16 * swz64(r, 2 * g + ks);
  }
  // Expansion items, every thread the same number so that no branch splits
  // the loop body: piece q of 8 codes of B row cr (logical bytes 8 q ..
  // 8 q + 7 of the 32-code row) becomes logical 16-byte chunk q of the bf16
  // row.
  constexpr int B_ITEMS = 4 * BN / C::NT;
  int conv_src[B_ITEMS], conv_dst[B_ITEMS];
#pragma unroll
  for (int it = 0; it < B_ITEMS; ++it) {
    const int item = tid + it * C::NT, cr = item >> 2, q = item & 3;
    conv_src[it] = C::A_BYTES + cr * 32 + 16 * swz32(cr, q >> 1) + 8 * (q & 1);
    conv_dst[it] = cr * 64 + 16 * swz64(cr, q);
  }
  // expansion of stage t in two halves: the LDS reads, issued beside the
  // fragment reads, and the conversion and LDS writes, scheduled among the
  // MFMAs so that they issue while the MFMAs execute
  uint2 craw[B_ITEMS];
  auto convert_load = [&](int t) {
    const char* st = lds + (t % STAGES) * C::STAGE_BYTES;
#pragma unroll
    for (int it = 0; it < B_ITEMS; ++it) craw[it] = *reinterpret_cast<const uint2*>(st + conv_src[it]);
  };
  auto convert_store = [&](int t) {
    char* bdst = bconv + (t & 1) * C::BCONV_BYTES;
#pragma unroll
    for (int it = 0; it < B_ITEMS; ++it)
      *reinterpret_cast<bf16x8*>(bdst + conv_dst[it]) = codes8_to_bf16(craw[it].x, craw[it].y);
  };
  bf16x8 fa[PLANES][FM][2], fb[FN][2];
  float4 araw[FM][2][2];  // fused A: the raw fp32 runs, split by split_frags
  auto read_frags = [&](int t) {
    const char* st = lds + (t % STAGES) * C::STAGE_BYTES;
    const char* bt = bconv + (t & 1) * C::BCONV_BYTES;
    // in the order the MFMAs consume them
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        if constexpr (C::FUSED_A) {
#pragma unroll
          for (int h = 0; h < 2; ++h)
            araw[i][ks][h] = *reinterpret_cast<const float4*>(st + ar_off[i][ks][h]);
        } else {
#pragma unroll
          for (int p = 0; p < PLANES; ++p)
            fa[p][i][ks] = *reinterpret_cast<const bf16x8*>(st + a_off[p][i][ks]);
        }
      }
#pragma unroll
      for (int j = 0; j < FN; ++j)
        fb[j][ks] = *reinterpret_cast<const bf16x8*>(bt + b_off[j][ks]);
    }
  };
  auto split_frags = [&]() {
    if constexpr (C::FUSED_A) {
#pragma unroll
      for (int ks = 0; ks < 2; ++ks)
#pragma unroll
        for (int i = 0; i < FM; ++i) {
          const float4 u = araw[i][ks][0], w4 = araw[i][ks][1];
          const float v[8] = {u.x, u.y, u.z, u.w, w4.x, w4.y, w4.z, w4.w};
          Pack8 hi, lo;
          split8<PLANES>(v, hi, lo);
          fa[0][i][ks] = __builtin_bit_cast(bf16x8, hi);
          if constexpr (PLANES == 2) fa[PLANES - 1][i][ks] = __builtin_bit_cast(bf16x8, lo);
        }
    }
  };

#pragma unroll
  for (int s0 = 0; s0 < AHEAD; ++s0)
    if (s0 < ktiles) issue(s0);
  wait_stage(0, AHEAD - 1);
  block_barrier();
  convert_load(0);
  convert_store(0);

  // Iteration t: once every wave's copy of stage t + 1 has landed and the
  // expansion of stage t is written, a barrier; then issue stage t + AHEAD,
  // read stage t's fragments and stage t + 1's raw tile, run stage t's
  // MFMAs, and expand stage t + 1 into the other bf16 buffer while they
  // execute.
  // The steady part (stage t + AHEAD exists) has a fixed wait count and no
  // branch; the last AHEAD stages drain the ring.
  auto stage = [&](int t, auto steady) {
    if constexpr (decltype(steady)::value)
      wait_vmcnt<(AHEAD - 2) * DPW>();  // stages t+2 .. t+AHEAD-1 may fly
    else if (t + 1 < ktiles)
      wait_stage(t + 1, t + AHEAD - 1);
    wait_lgkmcnt0();  // this wave's expansion writes of stage t are done
    block_barrier();
    // the first group of the stage's DMA (the second follows k-step 0)
    const bool refill = decltype(steady)::value || t + AHEAD < ktiles;
    if (refill) issue_blocks(t + AHEAD, JA{}, JB{});
    // every LDS read of the iteration issues before the first MFMA (stage
    // t's fragments, then stage t + 1's raw tile, whose conversion then
    // issues among the MFMAs); the last iteration expands a stage past the
    // end into the buffer no one reads again (no branch in the body)
    read_frags(t);
    convert_load(t + 1);
    issue_fence();
    split_frags();
    auto mfma_step = [&](int ks) {
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
          for (int p = 0; p < PLANES; ++p)
            acc[i][j] = mfma_32x32x16_bf16(fa[p][i][ks], fb[j][ks], acc[i][j]);
    };
    mfma_step(0);
    sched_fence();
    if (refill) issue_blocks(t + AHEAD, JB{}, JC{});
    sched_fence();
    mfma_step(1);
    convert_store(t + 1);
    sched_fence();
  };
  // With two stages ahead the wait count is the same in every iteration, and
  // one loop (half the code) measured 2% faster on the 256 x 256 fp32 GEMM.
  int t = 0;
  if constexpr (AHEAD > 2)
    for (; t + AHEAD < ktiles; ++t) stage(t, std::true_type{});
  for (; t < ktiles; ++t) stage(t, std::false_type{});

  const int lhalf = lane >> 5;
  with_activation<(C::BM <= 128)>(ep, [&](auto act) {
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const int64_t col = n0 + wn * TN + j * 32 + lrow;
      if (col >= n) continue;
      const float s = col_scale[j];
      const float b = col_bias[j];
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        if constexpr (!YP && C::BM <= 128) {
          // the wave's 32 rows all inside the tile's rows: no per-element
          // row test, wave-uniform row offsets (8 q + r) * n (the 256 x 256
          // tiles spill 37 VGPRs with this path)
          if (m0 + wm * TM + i * 32 + 32 <= m_end) {
            const int64_t at = (m0 + wm * TM + i * 32 + 4 * lhalf) * n + col;
#pragma unroll
            for (int e = 0; e < 16; ++e) {
              const int64_t off = at + int64_t(8 * (e / 4) + (e % 4)) * n;
              float v = acc[i][j][e] * s;
              if (bias) v = v + b;
              if (z) __builtin_nontemporal_store(v, &z[off]);
              __builtin_nontemporal_store(act(v), &y[off]);
            }
            continue;
          }
        }
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int64_t row = m0 + wm * TM + i * 32 + 8 * (e / 4) + 4 * lhalf + (e % 4);
          if (row < m_end) {
            float v = acc[i][j][e] * s;
            if (bias) v = v + b;
            if (z) __builtin_nontemporal_store(v, &z[row * n + col]);
            if constexpr (YP) {
              // the output as the next GEMM's bf16 planes (split_planes_kernel's split)
              const float h = act(v);
              const uint16_t hi = bf16_bits_rne(h);
              yp[row * yp_ld + col] = hi;
              if constexpr (PLANES == 2)
                yp[yp_plane_stride + row * yp_ld + col] = bf16_bits_rne(h - bf16_to_float(hi));
            } else {
              __builtin_nontemporal_store(act(v), &y[row * n + col]);
            }
          }
        }
      }
    }
  });
}

template <class C>
void launch_w8_ring(const uint16_t* xa, int64_t plane_stride, int64_t kp, const int8_t* w,
                    const float* scale, const float* bias, int64_t m, int64_t n, int64_t k,
                    const Epilogue& ep, float* y, float* z, const RowGroups& grp,
                    const float* x = nullptr, uint16_t* yp = nullptr, int64_t yp_plane_stride = 0,
                    int64_t yp_ld = 0) {
  // grouped rows: every group may end in a partial tile
  const int64_t tiles_m = ceil_div(m, C::BM) + (grp.offsets ? grp.groups : 0);
  const int64_t tiles_n = ceil_div(n, C::BN);
  ENQ_REQUIRE(tiles_m * tiles_n <= 0x7fffffff, "problem too large");
  const size_t lds_bytes = size_t(C::LDS_BYTES);
  static bool attr_set = false;
  if (!attr_set) {
    ENQ_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(w8_ring_kernel<C, false>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, int(lds_bytes)));
    ENQ_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(w8_ring_kernel<C, true>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, int(lds_bytes)));
    if constexpr (!C::FUSED_A) {
      ENQ_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(w8_ring_kernel<C, false, true>),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, int(lds_bytes)));
      ENQ_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(w8_ring_kernel<C, true, true>),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, int(lds_bytes)));
    }
    attr_set = true;
  }
  auto kernel = (k % C::BK == 0) ? w8_ring_kernel<C, false> : w8_ring_kernel<C, true>;
  if constexpr (!C::FUSED_A) {
    if (yp) kernel = (k % C::BK == 0) ? w8_ring_kernel<C, false, true> : w8_ring_kernel<C, true, true>;
  } else {
    ENQ_REQUIRE(yp == nullptr, "plane outputs take pre-split activations");
  }
  kernel<<<unsigned(tiles_m * tiles_n), C::NT, lds_bytes, stream()>>>(
      xa, plane_stride, kp, x, w, scale, bias, m, n, k, int(tiles_m), int(tiles_n), grp, ep, y, z,
      yp, yp_plane_stride, yp_ld);
  check_launch("w8_ring_kernel");
}

template <int BM, int BN, int WM, int WN, int PLANES, int KMODE>
void launch_gemm(const uint16_t* xa, int64_t plane_stride, int64_t kp, const int8_t* w,
                 int64_t ldw, const float* scale, const float* bias, int64_t m, int64_t n,
                 int64_t k, const Epilogue& ep, float* y, float* z) {
  const int64_t tiles_m = ceil_div(m, BM), tiles_n = ceil_div(n, BN);
  ENQ_REQUIRE(tiles_m * tiles_n <= 0x7fffffff, "problem too large");
  const size_t lds_bytes = size_t(2) * (PLANES * BM + BN) * kPitch * sizeof(uint16_t);
  auto kernel = w8_gemm_kernel<BM, BN, WM, WN, PLANES, KMODE>;
  static bool attr_set = false;
  if (!attr_set) {
    ENQ_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                hipFuncAttributeMaxDynamicSharedMemorySize, int(lds_bytes)));
    attr_set = true;
  }
  kernel<<<unsigned(tiles_m * tiles_n), WM * WN * 64, lds_bytes, stream()>>>(
      xa, plane_stride, kp, w, ldw, scale, bias, m, n, k, int(tiles_m), int(tiles_n), ep, y, z);
  check_launch("w8_gemm_kernel");
}

// Tile choice: 256 x 256 tiles when they alone fill the device, otherwise
// 128 x 128 tiles with 8 waves.  Measured on the MLP step (0.108 ms vs
// 0.118 for 64 x 64 tiles), the transformer block (0.671 vs 0.756 ms) and
// the 4096 x 8192 x 8192 GEMM (1.24 ms for 256 x 256 vs 1.84 ms).
template <int PLANES, int KMODE>
void gemm_dispatch(const uint16_t* xa, int64_t plane_stride, int64_t kp, const int8_t* w,
                   int64_t ldw, const float* scale, const float* bias, int64_t m, int64_t n,
                   int64_t k, const Epilogue& ep, float* y, float* z,
                   const RowGroups& grp = RowGroups{}, uint16_t* yp = nullptr,
                   int64_t yp_plane_stride = 0, int64_t yp_ld = 0) {
  const int64_t big_tiles = ceil_div(m, 256) * ceil_div(n, 256);
  const bool big = big_tiles >= device_cu_count();
  if (KMODE != 2) {
    if (big)
      launch_w8_ring<RingCfg<256, 256, 4, 2, PLANES, PLANES == 2 ? 3 : 4>>(
          xa, plane_stride, kp, w, scale, bias, m, n, k, ep, y, z, grp, nullptr, yp,
          yp_plane_stride, yp_ld);
    else
      launch_w8_ring<RingCfg<128, 128, 4, 2, PLANES, 4>>(
          xa, plane_stride, kp, w, scale, bias, m, n, k, ep, y, z, grp, nullptr, yp,
          yp_plane_stride, yp_ld);
    return;
  }
  // register-staged kernel: any K, any code alignment; no row groups
  ENQ_REQUIRE(grp.offsets == nullptr, "grouped rows need K a multiple of 16");
  ENQ_REQUIRE(yp == nullptr, "plane outputs need K a multiple of 16");
  if (big)
    launch_gemm<256, 256, 4, 2, PLANES, KMODE>(xa, plane_stride, kp, w, ldw, scale, bias, m, n, k,
                                               ep, y, z);
  else
    launch_gemm<128, 128, 2, 2, PLANES, KMODE>(xa, plane_stride, kp, w, ldw, scale, bias, m, n, k,
                                               ep, y, z);
}

// Launch geometry of a GEMV: grid (groups, splits, m_blocks), the K slice of
// a split, and the partial-sum buffer it needs.
struct GemvPlan {
  bool decode;       // gemv_decode_kernel (m <= 64), else gemv_skinny_kernel
  int mb;            // decode: 16-row activation blocks (1, 2 or 4)
  int kr;            // decode: K slice per workgroup (multiple of 128)
  int chunks_per_wave, cb_per_group;  // skinny
  int64_t groups, splits, m_blocks, mp;
  size_t part_bytes(int64_t n) const {
    return splits > 1 ? sizeof(float) * size_t(splits * mp * n) : 0;
  }
};

GemvPlan plan_gemv(int64_t m, int64_t n, int64_t k) {
  GemvPlan g{};
  const int64_t cus = device_cu_count();
  if (m <= 64) {
    g.decode = true;
    g.mb = m <= 16 ? 1 : (m <= 32 ? 2 : 4);
    g.m_blocks = 1;
    g.mp = 16 * g.mb;
    g.groups = ceil_div(n, 16 * kGemvWaves * kDecodeCB);
    // the longest slice the LDS copy allows (16 MB rows x kr <= 16 x 1024),
    // shortened until groups x splits fill the device twice over
    const int64_t kr_max = 1024 / g.mb;
    const int64_t want_splits = ceil_div(2 * cus, g.groups);
    int64_t kr = ceil_div(ceil_div(k, want_splits), kGemvChunk) * kGemvChunk;
    kr = std::max<int64_t>(kGemvChunk, std::min(kr, kr_max));
    g.kr = int(kr);
    g.splits = ceil_div(k, kr);
  } else {
    g.decode = false;
    g.mb = 1;
    g.m_blocks = ceil_div(m, 16);
    g.mp = 16 * g.m_blocks;
    const int64_t chunks_total = ceil_div(k, kGemvChunk);
    g.splits = ceil_div(chunks_total, int64_t(kGemvWaves) * 2);
    g.chunks_per_wave = int(ceil_div(chunks_total, g.splits * kGemvWaves));
    const int64_t col_blocks = ceil_div(n, 16);
    const int64_t want_groups = std::max<int64_t>(1, (2 * cus) / (g.splits * g.m_blocks));
    g.cb_per_group = int(std::min<int64_t>(8, std::max<int64_t>(1, col_blocks / want_groups)));
    g.groups = ceil_div(col_blocks, g.cb_per_group);
  }
  ENQ_REQUIRE(g.groups <= 0x7fffffff && g.splits <= 65535 && g.m_blocks <= 65535,
              "problem too large");
  return g;
}

template <int MB, int PLANES, int KMODE>
void launch_decode(const GemvPlan& g, const float* x, int64_t m, int64_t k, int vec,
                   const int8_t* w, int64_t n, float* part, const float* scale,
                   const float* bias, const Epilogue& ep, float* y, float* z) {
  constexpr int CHUNKS = 8 / MB;  // kr <= 1024 / MB
  const size_t lds = size_t(PLANES) * 16 * MB * (g.kr + 8) * sizeof(uint16_t);
  auto kernel = gemv_decode_kernel<MB, PLANES, KMODE, CHUNKS, kDecodeCB>;
  static bool attr_set = false;
  if (!attr_set) {
    ENQ_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                hipFuncAttributeMaxDynamicSharedMemorySize, 80 * 1024));
    attr_set = true;
  }
  kernel<<<dim3(unsigned(g.groups), unsigned(g.splits)), 512, lds, stream()>>>(
      x, m, k, vec, w, n, g.kr, int(g.splits), part, scale, bias, ep, y, z);
  check_launch("gemv_decode_kernel");
}

template <int PLANES, int KMODE>
void gemv_dispatch(const GemvPlan& g, const float* x, const int8_t* w, const float* scale,
                   const float* bias, int64_t m, int64_t n, int64_t k, const Epilogue& ep,
                   float* y, float* z, float* part) {
  const int vec = (k % 4 == 0) && aligned(x, 16);
  if (g.decode) {
    if (g.mb == 1)
      launch_decode<1, PLANES, KMODE>(g, x, m, k, vec, w, n, part, scale, bias, ep, y, z);
    else if (g.mb == 2)
      launch_decode<2, PLANES, KMODE>(g, x, m, k, vec, w, n, part, scale, bias, ep, y, z);
    else
      launch_decode<4, PLANES, KMODE>(g, x, m, k, vec, w, n, part, scale, bias, ep, y, z);
    if (g.splits == 1) return;
  } else {
    // one K split: the kernel finishes the outputs itself
    const bool direct = g.splits == 1;
    ENQ_REQUIRE(g.chunks_per_wave >= 1 && g.chunks_per_wave <= 2, "skinny GEMV plan");
    auto kernel = g.chunks_per_wave == 1 ? gemv_skinny_kernel<PLANES, KMODE, 1>
                                         : gemv_skinny_kernel<PLANES, KMODE, 2>;
    kernel<<<dim3(unsigned(g.groups), unsigned(g.splits), unsigned(g.m_blocks)), 512, 0,
             stream()>>>(x, m, k, vec, w, n, g.chunks_per_wave, g.cb_per_group, g.mp,
                         direct ? nullptr : part, scale, bias, ep, y, z);
    check_launch("gemv_skinny_kernel");
    if (direct) return;
  }
  gemv_finish_kernel<<<unsigned(ceil_div(m * n, 256)), 256, 0, stream()>>>(
      part, int(g.splits), g.mp, m, n, scale, bias, ep, y, z);
  check_launch("gemv_finish_kernel");
}

}  // namespace

void split_planes(const float* x, const int* gather, int64_t m, int64_t k, uint16_t* xa,
                  int64_t mp, int64_t kp, int planes) {
  const int64_t groups = mp * (kp / 8);
  const int vec = (k % 4 == 0) && aligned(x, 16);
  ENQ_REQUIRE(ceil_div(groups, 256) <= 0x7fffffff, "problem too large");
  if (planes == 2)
    split_planes_kernel<2><<<unsigned(ceil_div(groups, 256)), 256, 0, stream()>>>(
        x, gather, m, k, xa, mp, kp, vec);
  else
    split_planes_kernel<1><<<unsigned(ceil_div(groups, 256)), 256, 0, stream()>>>(
        x, gather, m, k, xa, mp, kp, vec);
  check_launch("split_planes_kernel");
}

int64_t gemm_k_pad(int64_t k) { return ceil_div(k, kBK) * kBK; }

bool grouped_gemm_supported(int64_t k, const int8_t* codes) {
  return k % 16 == 0 && aligned(codes, 16);
}

void dense_w8_grouped(const uint16_t* xa, int64_t plane_stride, int64_t kp, int planes,
                      int64_t m, int64_t k, const int8_t* codes, const float* w_scale, int64_t n,
                      const float* bias, const RowGroups& grp, const Epilogue& ep, float* y,
                      uint16_t* yp, int64_t yp_plane_stride) {
  ENQ_REQUIRE(grouped_gemm_supported(k, codes), "grouped rows need K a multiple of 16");
  ENQ_REQUIRE(ep.activation != ENQ_ACT_SOFTMAX, "softmax epilogue is not fused");
  // plane outputs have no padding columns to clear: rows of n = gemm_k_pad(n)
  ENQ_REQUIRE(yp == nullptr || gemm_k_pad(n) == n, "plane outputs need N a multiple of 32");
  const int kmode = k % 32 == 0 ? 0 : 1;
  auto run = [&](auto planes_tag, auto kmode_tag) {
    constexpr int P = decltype(planes_tag)::value;
    constexpr int KM = decltype(kmode_tag)::value;
    gemm_dispatch<P, KM>(xa, plane_stride, kp, codes, k, w_scale, bias, m, n, k, ep, y, nullptr,
                         grp, yp, yp_plane_stride, n);
  };
  using P1 = std::integral_constant<int, 1>;
  using P2 = std::integral_constant<int, 2>;
  using K0 = std::integral_constant<int, 0>;
  using K1 = std::integral_constant<int, 1>;
  if (planes == 2) {
    if (kmode == 0) run(P2{}, K0{});
    else run(P2{}, K1{});
  } else {
    if (kmode == 0) run(P1{}, K0{});
    else run(P1{}, K1{});
  }
}

void dense_w8(const float* x, int64_t m, int64_t k, const int8_t* codes, const float* w_scale,
              int64_t n, const float* bias, const Epilogue& ep_all, int variant, float* y,
              float* z, bool no_alloc) {
  auto scratch_of = [&](size_t bytes) { return no_alloc ? noalloc_scratch(bytes) : workspace(bytes); };
  const int planes = variant == ENQ_W8_FP32 ? 2 : 1;
  // split-K GEMV for few activation rows, and for tall-skinny outputs (one
  // 16-row block per grid z index, so at most 65535 * 16 rows); both read
  // the fp32 activations directly
  const bool gemv = m <= 64 || (n <= kSkinnyN && m <= int64_t(65535) * 16);
  const int kmode = (k % 32 == 0 && aligned(codes, 16)) ? 0 : ((k % 16 == 0 && aligned(codes, 16)) ? 1 : 2);
  using P1 = std::integral_constant<int, 1>;
  using P2 = std::integral_constant<int, 2>;
  using K0 = std::integral_constant<int, 0>;
  using K1 = std::integral_constant<int, 1>;
  using K2 = std::integral_constant<int, 2>;
  auto with_modes = [&](int km, auto&& run) {
    if (planes == 2) {
      if (km == 0) run(P2{}, K0{});
      else if (km == 1) run(P2{}, K1{});
      else run(P2{}, K2{});
    } else {
      if (km == 0) run(P1{}, K0{});
      else if (km == 1) run(P1{}, K1{});
      else run(P1{}, K2{});
    }
  };
  // the GEMV finish kernel and the 128 x 128 kernel fuse the activation
  // fake-quantization; the other GEMM kernels leave it to finish_rows
  const bool big = ceil_div(m, 256) * ceil_div(n, 256) >= device_cu_count();
  // fp32-accurate GEMMs of more than 2^33 multiply-adds take the fp16 / e4m3
  // split even below the 256 x 256 tile count: its pass over x costs less
  // than the in-register split saves there (4096 x 3072 x 1024: 86.9 against
  // 94.8 us; 4096 x 1024 x 4096: 98.0 against 108.9), while the MLP layers
  // (4096 x 1024 x 1024: 38.5 against 33.2 us) keep the fused kernel
  const bool split_f8 = !gemv && planes == 2 && f16f8_supported(k, codes) &&
                        (big || double(m) * double(n) * double(k) > 8589934592.0);
  const bool fused_mid = !gemv && !big && !split_f8 && kmode != 2 && k % 4 == 0 && aligned(x, 16);
  const bool fuse_aq = gemv || fused_mid;
  const Epilogue ep = gemm_epilogue(ep_all, fuse_aq);
  if (gemv) {
    const GemvPlan plan = plan_gemv(m, n, k);
    auto* part = static_cast<float*>(scratch_of(plan.part_bytes(n)));
    // 128-wide K chunks need per-chunk guards unless k is a multiple of 128
    const int km = kmode == 0 ? (k % 128 == 0 ? 0 : 1) : kmode;
    with_modes(km, [&](auto planes_tag, auto kmode_tag) {
      gemv_dispatch<decltype(planes_tag)::value, decltype(kmode_tag)::value>(
          plan, x, codes, w_scale, bias, m, n, k, ep, y, z, part);
    });
  } else {
    const int64_t kp = ceil_div(k, kBK) * kBK;
    if (fused_mid) {
      // mid-size GEMM: the 128 x 128 kernel splits the activations itself.
      // MLP step with this kernel: 0.080 ms at 4 stages against
      // 0.083 at 5, 0.095 at 3, 0.089 for 64 x 128 tiles (two workgroups per
      // CU) and 0.119 for 64 x 64.  With the A split in registers, 64 x 128
      // tiles of four waves (two workgroups per CU) again lost: 38.9 against
      // 34.1 us for the 4096 x 1024 x 1024 layer.
      with_modes(kmode, [&](auto planes_tag, auto) {
        constexpr int P = decltype(planes_tag)::value;
        launch_w8_ring<RingCfg<128, 128, 4, 2, P, 4, true>>(nullptr, 0, kp, codes, w_scale, bias,
                                                            m, n, k, ep, y, z, RowGroups{}, x);
      });
    } else if (split_f8) {
      // fp32-accurate: fp16 high parts and e4m3 low parts, split in a pass of
      // their own (a quarter fewer matrix-core cycles than the bf16 hi/lo
      // planes)
      void* buf = scratch_of(f16f8_bytes(m, k));
      split_f16f8(x, m, k, buf);
      gemm_w8_f16f8(buf, m, k, codes, w_scale, n, bias, ep, y, z);
    } else {
      // Large GEMMs split the activations in a pass of their own.  Splitting
      // them inside the 256 x 256 kernel instead (as the 128 x 128 kernel
      // does) issues 64 more VALU instructions per wave per 16-deep k-step,
      // which the SIMD does not overlap with its MFMAs: 4096 x 8192 x 8192
      // took 1.167 against 1.048-1.068 ms (split pass included) on one box,
      // 1.041 against 1.056 on another.
      const int64_t plane_stride = m * kp;
      auto* xa =
          static_cast<uint16_t*>(scratch_of(size_t(planes) * plane_stride * sizeof(uint16_t)));
      split_planes(x, nullptr, m, k, xa, m, kp, planes);
      with_modes(kmode, [&](auto planes_tag, auto kmode_tag) {
        gemm_dispatch<decltype(planes_tag)::value, decltype(kmode_tag)::value>(
            xa, plane_stride, kp, codes, k, w_scale, bias, m, n, k, ep, y, z);
      });
    }
  }
  finish_rows(y, m, n, ep_all, fuse_aq);
}

}  // namespace enq

using namespace enq;

extern "C" int enq_dense_w8(const float* x, int64_t m, int64_t k, const int8_t* codes,
                            const float* w_scale, int64_t n, const float* bias, int activation,
                            float act_alpha, float act_clip, int variant, float* y, float* z) {
  return guarded([&] {
    require_init();
    ENQ_REQUIRE(m >= 1 && n >= 1 && k >= 1, "m, n, k must be positive (m=%lld n=%lld k=%lld)",
                (long long)m, (long long)n, (long long)k);
    ENQ_REQUIRE(x && codes && w_scale && y, "NULL pointer argument");
    ENQ_REQUIRE(valid_activation(activation), "unknown activation code %d", activation);
    ENQ_REQUIRE(variant == ENQ_W8_FP32 || variant == ENQ_W8_BF16, "unknown variant %d", variant);
    Epilogue ep{activation, act_alpha, act_clip};
    dense_w8(x, m, k, codes, w_scale, n, bias, ep, variant, y, z);
  });
}

extern "C" int enq_split_planes(const float* x, int64_t m, int64_t k, int variant,
                                uint16_t* planes) {
  return guarded([&] {
    require_init();
    ENQ_REQUIRE(m >= 1 && k >= 1, "m and k must be positive (m=%lld k=%lld)", (long long)m,
                (long long)k);
    ENQ_REQUIRE(x && planes, "NULL pointer argument");
    ENQ_REQUIRE(variant == ENQ_W8_FP32 || variant == ENQ_W8_BF16, "unknown variant %d", variant);
    const int64_t kp = gemm_k_pad(k);
    split_planes(x, nullptr, m, k, planes, m, kp, variant == ENQ_W8_FP32 ? 2 : 1);
  });
}

extern "C" int enq_gemm_w8_planes(const uint16_t* planes, int64_t m, int64_t k,
                                  const int8_t* codes, const float* w_scale, int64_t n,
                                  const float* bias, int activation, float act_alpha,
                                  float act_clip, int variant, float* y, float* z) {
  return guarded([&] {
    require_init();
    ENQ_REQUIRE(m >= 1 && n >= 1 && k >= 1, "m, n, k must be positive (m=%lld n=%lld k=%lld)",
                (long long)m, (long long)n, (long long)k);
    ENQ_REQUIRE(planes && codes && w_scale && y, "NULL pointer argument");
    ENQ_REQUIRE(valid_activation(activation), "unknown activation code %d", activation);
    ENQ_REQUIRE(variant == ENQ_W8_FP32 || variant == ENQ_W8_BF16, "unknown variant %d", variant);
    ENQ_REQUIRE(aligned(planes, 16), "planes must be 16-byte aligned");
    const Epilogue ep{activation, act_alpha, act_clip};
    const int64_t kp = gemm_k_pad(k);
    const int kmode = (k % 32 == 0 && aligned(codes, 16))
                          ? 0
                          : ((k % 16 == 0 && aligned(codes, 16)) ? 1 : 2);
    auto run = [&](auto planes_tag, auto kmode_tag) {
      gemm_dispatch<decltype(planes_tag)::value, decltype(kmode_tag)::value>(
          planes, m * kp, kp, codes, k, w_scale, bias, m, n, k, gemm_epilogue(ep, false), y, z);
    };
    using P1 = std::integral_constant<int, 1>;
    using P2 = std::integral_constant<int, 2>;
    using K0 = std::integral_constant<int, 0>;
    using K1 = std::integral_constant<int, 1>;
    using K2 = std::integral_constant<int, 2>;
    if (variant == ENQ_W8_FP32) {
      if (kmode == 0) run(P2{}, K0{});
      else if (kmode == 1) run(P2{}, K1{});
      else run(P2{}, K2{});
    } else {
      if (kmode == 0) run(P1{}, K0{});
      else if (kmode == 1) run(P1{}, K1{});
      else run(P1{}, K2{});
    }
    finish_rows(y, m, n, ep, false);
  });
}

extern "C" int enq_dense_w8_noalloc(const float* x, int64_t m, int64_t k, const int8_t* codes,
                                    const float* w_scale, int64_t n, const float* bias,
                                    int activation, float act_alpha, float act_clip, int variant,
                                    float* y, float* z) {
  return guarded([&] {
    require_init();
    ENQ_REQUIRE(m >= 1 && n >= 1 && k >= 1, "m, n, k must be positive (m=%lld n=%lld k=%lld)",
                (long long)m, (long long)n, (long long)k);
    ENQ_REQUIRE(x && codes && w_scale && y, "NULL pointer argument");
    ENQ_REQUIRE(valid_activation(activation), "unknown activation code %d", activation);
    ENQ_REQUIRE(variant == ENQ_W8_FP32 || variant == ENQ_W8_BF16, "unknown variant %d", variant);
    Epilogue ep{activation, act_alpha, act_clip};
    dense_w8(x, m, k, codes, w_scale, n, bias, ep, variant, y, z, /*no_alloc=*/true);
  });
}

extern "C" int enq_dense_w8_aq(const float* x, int64_t m, int64_t k, const int8_t* codes,
                               const float* w_scale, int64_t n, const float* bias, int activation,
                               float act_alpha, float act_clip, int variant, int aq_mode,
                               double aq_scale, double aq_zero_point, float aq_qmin,
                               float aq_qmax, float* y, float* z) {
  return guarded([&] {
    require_init();
    ENQ_REQUIRE(m >= 1 && n >= 1 && k >= 1, "m, n, k must be positive (m=%lld n=%lld k=%lld)",
                (long long)m, (long long)n, (long long)k);
    ENQ_REQUIRE(x && codes && w_scale && y, "NULL pointer argument");
    ENQ_REQUIRE(valid_activation(activation), "unknown activation code %d", activation);
    ENQ_REQUIRE(variant == ENQ_W8_FP32 || variant == ENQ_W8_BF16, "unknown variant %d", variant);
    ENQ_REQUIRE(aq_mode == ENQ_AQ_F32 || aq_mode == ENQ_AQ_F64, "unknown act-quant mode %d",
                aq_mode);
    ENQ_REQUIRE(valid_act_quant(aq_mode, aq_scale, aq_qmin, aq_qmax),
                "invalid act-quant parameters");
    Epilogue ep{activation, act_alpha, act_clip};
    ep.aq = aq_mode;
    ep.aq_scale = aq_scale;
    ep.aq_zp = aq_zero_point;
    ep.aq_qmin = aq_qmin;
    ep.aq_qmax = aq_qmax;
    dense_w8(x, m, k, codes, w_scale, n, bias, ep, variant, y, z);
  });
}
