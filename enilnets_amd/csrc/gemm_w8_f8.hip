// fp32-accurate W8 Dense for large tiles, with the activations split into an
// fp16 high part and an fp8 (OCP e4m3) low part.
//
//   e[m]  = the power of two with max_k |x[m,k]| * 2^e[m] in [2^14, 2^15)
//   hi    = fp16(x * 2^e)                  (11 significant bits, nearest even)
//   lo    = e4m3(x * 2^e - hi)             (|x * 2^e - hi| <= 2^-11 |x * 2^e|)
//   acc   = sum_k hi * q  +  sum_k lo * e4m3(q)        (one fp32 accumulator)
//   y     = act(ldexp(acc, -e[m]) * scale[n] + bias[n])
//
// q is the int8 weight code, exact in fp16.  The high products are exact,
// the low part carries x's next bits to about 2^-4 of themselves, and e4m3(q)
// is q within 1/16: the error is below 2e-5 of the row's largest output for
// normal, uniform, heavy-tailed, log-normal and Cauchy activations (CPU
// simulation at K = 8192), five times inside the 1e-4 * ||row||_inf bound.
// The fp8 matrix cores take 64 K values per instruction at twice the fp16
// rate, so a 64-deep step costs 4 fp16 + 1 fp8 MFMAs against 8 bf16 MFMAs
// for the hi/lo bf16 split: a quarter fewer matrix-core cycles.  The row
// exponent keeps x * 2^e inside fp16's range and the low part inside e4m3's.
//
// Kernels
//   split_f16f8_kernel   x (m, k) fp32 -> hi (m, kp) fp16, lo (m, kp) e4m3,
//                        e (m) int32; kp = k rounded up to 64, zero padded
//   w8_f8_ring_kernel    direct-to-LDS ring GEMM: per 32-deep stage the hi,
//                        lo and int8 code tiles, the codes expanded once per
//                        workgroup into fp16 and e4m3 tiles; fp16 MFMAs every
//                        stage, fp8 MFMAs every second stage on the low parts
//                        of both stages; per-row exponent, column scale,
//                        bias and activation in the epilogue
#include <algorithm>
#include <cmath>

#include "common.hpp"
#include "epilogue.hpp"
#include "mfma.hpp"
#include "ops.hpp"
#include "tiling.hpp"

namespace enq {
namespace {

constexpr int kF8KPad = 64;  // K of one fp8 MFMA: the planes' row padding

// The row exponent e: max |x| * 2^e in [2^14, 2^15).  A zero, infinite or
// NaN maximum gives 0 (the row's products are then zero or non-finite anyway).
__device__ __forceinline__ int row_exponent(float amax) {
  if (!(amax > 0.0f) || amax == __builtin_inff()) return 0;
  int ex;
  frexpf(amax, &ex);  // amax = f * 2^ex, f in [0.5, 1)
  return 15 - ex;
}

// Four activations -> their fp16 high parts (two dwords) and e4m3 low parts
// (one dword), after scaling by 2^e.
__device__ __forceinline__ void split4_f16f8(float4 v, int e, uint2& hi, uint32_t& lo,
                                             float& sumsq) {
  const float a[4] = {ldexpf(v.x, e), ldexpf(v.y, e), ldexpf(v.z, e), ldexpf(v.w, e)};
  sumsq += (a[0] * a[0] + a[1] * a[1]) + (a[2] * a[2] + a[3] * a[3]);
  _Float16 h[4];
  float r[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    h[i] = static_cast<_Float16>(a[i]);  // nearest even
    r[i] = a[i] - static_cast<float>(h[i]);  // exact
  }
  hi.x = uint32_t(__builtin_bit_cast(uint16_t, h[0])) | (uint32_t(__builtin_bit_cast(uint16_t, h[1])) << 16);
  hi.y = uint32_t(__builtin_bit_cast(uint16_t, h[2])) | (uint32_t(__builtin_bit_cast(uint16_t, h[3])) << 16);
  int p = __builtin_amdgcn_cvt_pk_fp8_f32(r[0], r[1], 0, false);
  p = __builtin_amdgcn_cvt_pk_fp8_f32(r[2], r[3], p, true);
  lo = uint32_t(p);
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// One 256-thread workgroup per row.  REGS: the row (k % 4 == 0, 16-byte
// aligned, k <= 1024 * V) stays in registers between its maximum and its
// split; otherwise it is read twice with scalar loads.  Row r of the split
// comes from row gather[r] of x (gather == nullptr: row r).  With `bound`,
// the row also gets a second exponent, exps2[r], for a Dense output computed
// from it: that of ||x||_2 * bound[0] + bound[1], a bound on every output of
// the row (f16f8_bound_params).  ||x||_2 comes from the scaled values
// x * 2^e (no overflow: |x * 2^e| < 2^15).
template <int V, bool REGS>
__global__ __launch_bounds__(256) void split_f16f8_kernel(const float* __restrict__ x,
                                                          const int* __restrict__ gather,
                                                          int64_t k, int64_t kp,
                                                          uint16_t* __restrict__ hi,
                                                          uint8_t* __restrict__ lo,
                                                          int* __restrict__ exps,
                                                          const float* __restrict__ bound,
                                                          int* __restrict__ exps2) {
  __shared__ float red[4];
  const int64_t row = blockIdx.x;
  const float* xr = x + (gather ? int64_t(gather[row]) : row) * k;
  const int tid = threadIdx.x;
  float amax = 0.0f;  // fmaxf skips NaN
  float4 v[REGS ? V : 1];
  if constexpr (REGS) {
#pragma unroll
    for (int j = 0; j < V; ++j) {
      const int64_t c = (int64_t(j) * 256 + tid) * 4;
      v[j] = c < k ? *reinterpret_cast<const float4*>(xr + c) : make_float4(0.f, 0.f, 0.f, 0.f);
      amax = fmaxf(amax, fmaxf(fmaxf(fabsf(v[j].x), fabsf(v[j].y)), fmaxf(fabsf(v[j].z), fabsf(v[j].w))));
    }
  } else {
    for (int64_t c = tid; c < k; c += 256) amax = fmaxf(amax, fabsf(xr[c]));
  }
  amax = wave_max(amax);
  if ((tid & 63) == 0) red[tid >> 6] = amax;
  __syncthreads();
  amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  const int e = row_exponent(amax);
  if (tid == 0) exps[row] = e;
  uint16_t* hr = hi + row * kp;
  uint8_t* lr = lo + row * kp;
  float sumsq = 0.0f;
  if constexpr (REGS) {
#pragma unroll
    for (int j = 0; j < V; ++j) {
      const int64_t c = (int64_t(j) * 256 + tid) * 4;
      if (c < kp) {
        uint2 h;
        uint32_t l;
        split4_f16f8(v[j], e, h, l, sumsq);
        *reinterpret_cast<uint2*>(hr + c) = h;
        *reinterpret_cast<uint32_t*>(lr + c) = l;
      }
    }
  } else {
    for (int64_t c = int64_t(tid) * 4; c < kp; c += 1024) {
      float4 t;
      t.x = c < k ? xr[c] : 0.0f;
      t.y = c + 1 < k ? xr[c + 1] : 0.0f;
      t.z = c + 2 < k ? xr[c + 2] : 0.0f;
      t.w = c + 3 < k ? xr[c + 3] : 0.0f;
      uint2 h;
      uint32_t l;
      split4_f16f8(t, e, h, l, sumsq);
      *reinterpret_cast<uint2*>(hr + c) = h;
      *reinterpret_cast<uint32_t*>(lr + c) = l;
    }
  }
  if (bound) {
    sumsq = wave_sum(sumsq);
    __syncthreads();  // red[] is reused
    if ((tid & 63) == 0) red[tid >> 6] = sumsq;
    __syncthreads();
    if (tid == 0) {
      // a float sum of squares is within k * 2^-24 of the exact one; the
      // bound is only an upper limit for the output's scale, so a 1% margin
      // is ample
      const float l2 = ldexpf(sqrtf((red[0] + red[1]) + (red[2] + red[3])), -e) * 1.01f;
      exps2[row] = row_exponent(l2 * bound[0] + bound[1]);
    }
  }
}

// Per-output-channel norms of a Dense's codes for split_f16f8_kernel's
// bound: |sum_k x_k q_nk| <= ||x||_2 * ||q_n||_2 (Cauchy-Schwarz).  Each wave
// takes rows of `codes` (rows, k) in turn (k % 16 == 0, 16-byte aligned) and
// the workgroup writes max_n scale[n] * ||q_n||_2 over its rows to part[].
__global__ __launch_bounds__(256) void code_norm_kernel(const int8_t* __restrict__ codes,
                                                        int64_t rows, int64_t k,
                                                        const float* __restrict__ scale,
                                                        float* __restrict__ part) {
  __shared__ float red[4];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  float best = 0.0f;
  for (int64_t r = int64_t(blockIdx.x) * 4 + wave; r < rows; r += int64_t(gridDim.x) * 4) {
    const int8_t* cr = codes + r * k;
    int acc = 0;
    for (int64_t c = int64_t(lane) * 16; c < k; c += 1024) {
      const int4 q = *reinterpret_cast<const int4*>(cr + c);
      acc = __builtin_amdgcn_sdot4(q.x, q.x, acc, false);
      acc = __builtin_amdgcn_sdot4(q.y, q.y, acc, false);
      acc = __builtin_amdgcn_sdot4(q.z, q.z, acc, false);
      acc = __builtin_amdgcn_sdot4(q.w, q.w, acc, false);
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) acc += __shfl_xor(acc, o, 64);
    best = fmaxf(best, fabsf(scale[r]) * sqrtf(float(acc)));
  }
  if (lane == 0) red[wave] = best;
  __syncthreads();
  if (threadIdx.x == 0) part[blockIdx.x] = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

// The two constants of the bound |act(z_n)| <= bound[0] * ||x||_2 + bound[1]
// for z_n = scale[n] * sum_k x_k q_nk + bias[n]:
//   bound[0] = c * max_n scale[n] * ||q_n||_2,  bound[1] = c * max |bias| + d,
// with |act(z)| <= c |z| + d for the epilogue's activation: c = 1 for linear,
// relu, gelu, swish, mish and tanh, max(1, |alpha|) for the leaky slopes and
// elu, 1.76 for selu; d = 1 for sigmoid (c = 0) and ln 2 for softplus; each
// widened by 1%.  One workgroup.
__global__ __launch_bounds__(256) void f16f8_bound_kernel(const float* __restrict__ part, int parts,
                                                          const float* __restrict__ bias,
                                                          int64_t nb, float c, float d,
                                                          float* __restrict__ out) {
  __shared__ float red_s[4], red_b[4];
  float ms = 0.0f, mb = 0.0f;
  for (int i = threadIdx.x; i < parts; i += 256) ms = fmaxf(ms, part[i]);
  for (int64_t i = threadIdx.x; i < nb; i += 256) mb = fmaxf(mb, fabsf(bias[i]));
  ms = wave_max(ms);
  mb = wave_max(mb);
  if ((threadIdx.x & 63) == 0) {
    red_s[threadIdx.x >> 6] = ms;
    red_b[threadIdx.x >> 6] = mb;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    ms = fmaxf(fmaxf(red_s[0], red_s[1]), fmaxf(red_s[2], red_s[3]));
    mb = fmaxf(fmaxf(red_b[0], red_b[1]), fmaxf(red_b[2], red_b[3]));
    out[0] = c * ms * 1.01f;
    out[1] = (c * mb + d) * 1.01f;
  }
}

// ---------------------------------------------------------------------------
// The GEMM.  A stage is 32 deep.  Its A tile (the hi parts, BM rows of 64
// bytes with chunks swizzled by swz64, then the lo parts, BM rows of 32 bytes
// with halves swizzled by swz32) and its code tile (BN rows of 32 bytes,
// swz32) go global -> LDS by global_load_lds_dwordx4 in 1 KiB blocks, into
// two rings: A tiles are multiplied AHEAD stages after their DMA is issued,
// while code tiles are expanded a stage before they are multiplied, so the
// code ring runs one stage further ahead and holds one slot more.  Each
// wave's DMA of iteration t, group G(t + AHEAD), is its share of A tile
// t + AHEAD and of code tile t + AHEAD + 1; the top of iteration t waits for
// G(t), issued AHEAD iterations earlier, with a fixed vmcnt.  Groups past the
// end of K load the zero block into slots no one reads again, so every
// iteration has the same wait.  Each stage's codes are expanded once per
// workgroup into an fp16 tile (64-byte rows) and an e4m3 tile (32-byte rows,
// the codes' own byte positions), double-buffered after the rings; the
// expansion of stage t + 1 is issued among stage t's MFMAs.
//
// fp8 operands: lane group g of a 32 x 32 x 64 MFMA takes, in dwords 0-3, the
// 16 low parts (or e4m3 codes) of logical half g of the even stage's 32-byte
// row and, in dwords 4-7, those of the odd stage.  Which K position the
// instruction gives each byte does not matter as long as A and B agree, and
// they are laid out alike.
// ---------------------------------------------------------------------------
template <int BM_, int BN_, int WM_, int WN_, int AHEAD_>
struct F8RingCfg {
  static constexpr int BM = BM_, BN = BN_, WM = WM_, WN = WN_, AHEAD = AHEAD_, BK = 32;
  static constexpr int NT = WM * WN * 64, WAVES = NT / 64;
  static constexpr int TM = BM / WM, TN = BN / WN, FM = TM / 32, FN = TN / 32;
  static constexpr int HI_BYTES = BM * 64, LO_BYTES = BM * 32, B_BYTES = BN * 32;
  static constexpr int A_BYTES = HI_BYTES + LO_BYTES;
  static constexpr int A_SLOTS = AHEAD + 1, B_SLOTS = AHEAD + 2;
  static constexpr int B16_BYTES = BN * 64, B8_BYTES = BN * 32;
  static constexpr int CONV_BYTES = B16_BYTES + B8_BYTES;  // one expanded code tile
  static constexpr int HI_BLOCKS = HI_BYTES / 1024, A_BLOCKS = A_BYTES / 1024;
  static constexpr int B_BLOCKS = B_BYTES / 1024;
  static_assert(HI_BYTES % 1024 == 0 && LO_BYTES % 1024 == 0 && B_BYTES % 1024 == 0,
                "whole 1 KiB blocks");
  // every wave issues the same number of blocks (vmcnt accounting); waves
  // past the last block repeat it, rewriting identical bytes
  static constexpr int A_PW = (A_BLOCKS + WAVES - 1) / WAVES;
  static constexpr int B_PW = (B_BLOCKS + WAVES - 1) / WAVES;
  static constexpr int DPW = A_PW + B_PW;
  static constexpr int B_RING = A_SLOTS * A_BYTES;            // byte offset of the code ring
  static constexpr int CONV = B_RING + B_SLOTS * B_BYTES;     // of the expanded tiles
  static constexpr int LDS_BYTES = CONV + 2 * CONV_BYTES;
  static_assert(LDS_BYTES <= 160 * 1024, "LDS budget");
  static constexpr int WG_PER_CU = (160 * 1024) / LDS_BYTES;
  static constexpr int WAVES_PER_EU = (NT / 256) * WG_PER_CU < 8 ? (NT / 256) * WG_PER_CU : 8;
  static_assert((4 * BN) % NT == 0, "whole 8-code expansion items per thread");
  static_assert(AHEAD >= 2 && AHEAD * DPW < 64, "vmcnt range");
};

// The output as the next GEMM's split (YF8 instantiations): row r of the
// (m, n) output, activated, scaled by 2^exps[r] and split into fp16 high and
// e4m3 low parts at hi / lo + r * ld.
struct F8Out {
  uint16_t* hi = nullptr;
  uint8_t* lo = nullptr;
  const int* exps = nullptr;
  int64_t ld = 0;
};

template <class C, bool KTAIL, bool YF8 = false>
__global__ __launch_bounds__(C::NT) __attribute__((amdgpu_waves_per_eu(C::WAVES_PER_EU, C::WAVES_PER_EU)))
void w8_f8_ring_kernel(const uint16_t* __restrict__ xh, const uint8_t* __restrict__ xl,
                       const int* __restrict__ xe, int64_t kp, const int8_t* __restrict__ w,
                       const float* __restrict__ scale, const float* __restrict__ bias,
                       int64_t m, int64_t n, int64_t k, int tiles_m, int tiles_n, RowGroups grp,
                       Epilogue ep, float* __restrict__ y, float* __restrict__ z, F8Out yo,
                       int ksplit) {
  constexpr int BM = C::BM, BN = C::BN, WN = C::WN, AHEAD = C::AHEAD, BK = C::BK;
  constexpr int TM = C::TM, TN = C::TN, FM = C::FM, FN = C::FN;
  constexpr int A_PW = C::A_PW, B_PW = C::B_PW, DPW = C::DPW;
  extern __shared__ __align__(16) uint16_t lds_raw[];
  char* lds = reinterpret_cast<char*>(lds_raw);
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WN, wn = wave % WN;
  // split K (ksplit > 1): workgroup b takes K part b / tiles of tile
  // b % tiles, writes that part's sums (scaled, bias only in part 0, no
  // activation) to y + part * m * n, and the caller adds the parts
  const int tiles = tiles_m * tiles_n;
  const int part = int(blockIdx.x) / tiles;
  int tm, tn;
  xcd_tile(int(blockIdx.x) - part * tiles, tiles_m, tiles_n, 4, tm, tn);
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

  // DMA sources of this wave's blocks, as 32-bit byte offsets from the
  // planes' (or codes') base: A blocks (hi: 16 rows x 64 B, lo: 32 rows x
  // 32 B) and code blocks (32 rows x 32 B)
  uint32_t a_voff[A_PW];
  bool a_hi[A_PW];
#pragma unroll
  for (int j = 0; j < A_PW; ++j) {
    const int blk = min(wave * A_PW + j, C::A_BLOCKS - 1);
    if (blk < C::HI_BLOCKS) {
      const int r = blk * 16 + (lane >> 2);
      int64_t g = m0 + r;
      g = g < m ? g : m - 1;
      a_voff[j] = uint32_t(g * kp * 2 + 16 * swz64(r, lane & 3));
      a_hi[j] = true;
    } else {
      const int r = (blk - C::HI_BLOCKS) * 32 + (lane >> 1);
      int64_t g = m0 + r;
      g = g < m ? g : m - 1;
      a_voff[j] = uint32_t(g * kp + 16 * swz32(r, lane & 1));
      a_hi[j] = false;
    }
  }
  uint32_t b_voff[B_PW];
  int b_koff[B_PW];
#pragma unroll
  for (int j = 0; j < B_PW; ++j) {
    const int blk = min(wave * B_PW + j, C::B_BLOCKS - 1);
    const int r = blk * 32 + (lane >> 1);
    int64_t g = n0 + r;
    g = g < n ? g : n - 1;
    b_koff[j] = 16 * swz32(r, lane & 1);
    b_voff[j] = uint32_t(g * k + b_koff[j]);
  }
  // this part's stages: an even number (kp is a multiple of 64), at least two
  const int kt_all = int(kp / BK), kt_part = (kt_all / ksplit + 1) & ~1;
  const int t0 = part * kt_part;
  const int ktiles = min(kt_part, kt_all - t0);
  const int64_t k_rem = k - int64_t(t0) * BK;  // codes from this part's first column
  const void* zero = g_zero16;
  const uint32_t lds0 = lds_addr(lds);
  const char* xh_b = reinterpret_cast<const char*>(xh) + int64_t(t0) * (2 * BK);
  const char* xl_b = reinterpret_cast<const char*>(xl) + int64_t(t0) * BK;
  const char* w_b = reinterpret_cast<const char*>(w) + int64_t(t0) * BK;
  // block j (< A_PW: A, else codes) of this wave's group G(s): A tile s and
  // code tile s + 1.  Tiles past the end of K reload the last one into a
  // slot no one reads again (uniform wait counts).
  auto dma_a = [&](int s, int j) {
    const int blk = min(wave * A_PW + j, C::A_BLOCKS - 1);
    const int64_t sc = s < ktiles ? s : ktiles - 1;
    const char* base = a_hi[j] ? xh_b + sc * (2 * BK) : xl_b + sc * BK;
    dma16_s(a_voff[j], base, lds0 + (s % C::A_SLOTS) * C::A_BYTES + blk * 1024);
  };
  auto dma_b = [&](int s, int j) {
    const int blk = min(wave * B_PW + j, C::B_BLOCKS - 1);
    const int64_t sc = s < ktiles ? s : ktiles - 1;
    const uint32_t dst = lds0 + C::B_RING + (s % C::B_SLOTS) * C::B_BYTES + blk * 1024;
    if constexpr (KTAIL) {
      // 16-byte chunks past k read the zero block
      const bool live = sc * BK + b_koff[j] < k_rem;
      dma16(live ? static_cast<const void*>(w_b + b_voff[j] + sc * BK) : zero, dst);
    } else {
      dma16_s(b_voff[j], w_b + sc * BK, dst);
    }
  };
  auto issue_group = [&](int s, auto j0, auto j1) {
#pragma unroll
    for (int j = decltype(j0)::value; j < decltype(j1)::value; ++j) {
      if (j < A_PW) dma_a(s, j);
      else dma_b(s + 1, j - A_PW);
    }
  };
  using JA = std::integral_constant<int, 0>;
  using JC = std::integral_constant<int, DPW>;

  floatx16 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

  const int lrow = lane & 31, g = lane >> 5;
  char* conv = lds + C::CONV;
  int a_off[FM][2], lo_off[FM], b_off[FN][2], b8_off[FN];
#pragma unroll
  for (int i = 0; i < FM; ++i) {
    const int r = wm * TM + i * 32 + lrow;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) a_off[i][ks] = r * 64 + 16 * swz64(r, 2 * g + ks);
    lo_off[i] = C::HI_BYTES + r * 32 + 16 * swz32(r, g);
  }
#pragma unroll
  for (int j = 0; j < FN; ++j) {
    const int c = wn * TN + j * 32 + lrow;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) b_off[j][ks] = c * 64 + 16 * swz64(c, 2 * g + ks);
    b8_off[j] = C::B16_BYTES + c * 32 + 16 * swz32(c, g);
  }
  // expansion items: piece q of 8 codes of code row cr (logical bytes 8 q ..
  // 8 q + 7) -> logical chunk q of the fp16 row and the same bytes of the
  // e4m3 row
  constexpr int B_ITEMS = 4 * BN / C::NT;
  int conv_src[B_ITEMS], conv_d16[B_ITEMS];
#pragma unroll
  for (int it = 0; it < B_ITEMS; ++it) {
    const int item = tid + it * C::NT, cr = item >> 2, q = item & 3;
    conv_src[it] = cr * 32 + 16 * swz32(cr, q >> 1) + 8 * (q & 1);
    conv_d16[it] = cr * 64 + 16 * swz64(cr, q);
  }
  uint2 craw[B_ITEMS];
  auto convert_load = [&](int t) {
    const char* st = lds + C::B_RING + (t % C::B_SLOTS) * C::B_BYTES;
#pragma unroll
    for (int it = 0; it < B_ITEMS; ++it) craw[it] = *reinterpret_cast<const uint2*>(st + conv_src[it]);
  };
  auto convert_store = [&](int t) {
    char* bdst = conv + (t & 1) * C::CONV_BYTES;
#pragma unroll
    for (int it = 0; it < B_ITEMS; ++it) {
      uint4 h;
      uint2 f;
      codes4_to_f16_e4m3(craw[it].x, h.x, h.y, f.x);
      codes4_to_f16_e4m3(craw[it].y, h.z, h.w, f.y);
      *reinterpret_cast<uint4*>(bdst + conv_d16[it]) = h;
      *reinterpret_cast<uint2*>(bdst + C::B16_BYTES + conv_src[it]) = f;
    }
  };
  // two sets of fp16 fragments, one per k-step: k-step 1 of stage t is read
  // at the top of iteration t and multiplied after the barrier that ends it,
  // while k-step 0 of stage t + 1 is read, so the matrix cores have work
  // queued across the barrier; the fp8 halves are read after k-step 0's MFMAs
  halfx8 fa[2][FM], fb[2][FN];
  intx8 la[FM], lb[FN];  // fp8 operands: even stage in dwords 0-3, odd in 4-7
  auto read_hi = [&](int t, auto ksc) {
    constexpr int ks = decltype(ksc)::value;
    const char* st = lds + (t % C::A_SLOTS) * C::A_BYTES;
    const char* bt = conv + (t & 1) * C::CONV_BYTES;
#pragma unroll
    for (int i = 0; i < FM; ++i) fa[ks][i] = *reinterpret_cast<const halfx8*>(st + a_off[i][ks]);
#pragma unroll
    for (int j = 0; j < FN; ++j) fb[ks][j] = *reinterpret_cast<const halfx8*>(bt + b_off[j][ks]);
  };
  auto read_lo = [&](int t, auto odd) {
    const char* st = lds + (t % C::A_SLOTS) * C::A_BYTES;
    const char* bt = conv + (t & 1) * C::CONV_BYTES;
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      const intx4 v = *reinterpret_cast<const intx4*>(st + lo_off[i]);
      if constexpr (decltype(odd)::value) la[i].hi = v;
      else la[i].lo = v;
    }
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const intx4 v = *reinterpret_cast<const intx4*>(bt + b8_off[j]);
      if constexpr (decltype(odd)::value) lb[j].hi = v;
      else lb[j].lo = v;
    }
  };

  // prologue: code tile 0, then groups G(0) .. G(AHEAD - 1); tile 0's codes
  // are expanded once they land
#pragma unroll
  for (int j = 0; j < B_PW; ++j) dma_b(0, j);
#pragma unroll
  for (int s = 0; s < AHEAD; ++s) issue_group(s, JA{}, JC{});
  wait_vmcnt<AHEAD * DPW>();
  block_barrier();
  convert_load(0);
  convert_store(0);

  using KS0 = std::integral_constant<int, 0>;
  using KS1 = std::integral_constant<int, 1>;
  auto f16_step = [&](auto ksc) {
    constexpr int ks = decltype(ksc)::value;
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j) acc[i][j] = mfma_32x32x16_f16(fa[ks][i], fb[ks][j], acc[i][j]);
  };
  // stage 0: G(0) landed for every wave, its codes expanded; k-step 0 read
  wait_vmcnt<(AHEAD - 1) * DPW>();
  wait_lgkmcnt0();
  block_barrier();
  read_hi(0, KS0{});

  // Iteration t (k-step 0 of stage t already read): issue G(t + AHEAD)
  // (all of it: splitting it in two among the MFMAs measured 1.2% slower),
  // read k-step 1 and stage t + 1's raw codes, run k-step 0's
  // MFMAs, read the fp8 halves (and at odd t run the fp8 MFMAs of stages
  // t - 1 and t), expand stage t + 1 into the other buffer; then, once G(t +
  // 1) has landed for this wave and its expansion writes are done, the
  // barrier; read k-step 0 of stage t + 1 and run k-step 1's MFMAs.
  auto stage = [&](int t, auto odd) {
    issue_group(t + AHEAD, JA{}, JC{});
    read_hi(t, KS1{});
    convert_load(t + 1);
    issue_fence();
    f16_step(KS0{});
    sched_fence();
    read_lo(t, odd);
    issue_fence();
    if constexpr (decltype(odd)::value) {
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = mfma_32x32x64_e4m3(la[i], lb[j], acc[i][j]);
    }
    convert_store(t + 1);
    sched_fence();
    wait_vmcnt<(AHEAD - 1) * DPW>();  // G(t + 2) .. G(t + AHEAD) may fly
    wait_lgkmcnt0();
    block_barrier();
    // (past the last stage this reads slots no one writes again: unused)
    read_hi(t + 1, KS0{});
    issue_fence();
    f16_step(KS1{});
    sched_fence();
  };
  for (int t = 0; t < ktiles; t += 2) {
    stage(t, std::false_type{});
    stage(t + 1, std::true_type{});
  }
  // every DMA of this wave has landed before the workgroup ends (the last
  // groups wrote slots no one reads)
  wait_vmcnt<0>();

  const int lhalf = lane >> 5;
  with_activation<false>(ep, [&](auto act) {
    static_for<0, FM>([&](auto ic) {
      constexpr int i = decltype(ic)::value;
      int ex[16], eo[16];
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int64_t row = m0 + wm * TM + i * 32 + 8 * (e / 4) + 4 * lhalf + (e % 4);
        ex[e] = -xe[row < m ? row : m - 1];
        if constexpr (YF8) eo[e] = yo.exps[row < m ? row : m - 1];
      }
      const int64_t row0 = m0 + wm * TM + i * 32 + 4 * lhalf;
      // the wave's 32 rows all inside the tile's rows (every block of a full
      // tile): no per-element row test, and the rows' offsets (8 q + r) * n
      // are wave-uniform
      const bool rows_in = m0 + wm * TM + i * 32 + 32 <= m_end;
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        const int64_t col = n0 + wn * TN + j * 32 + lrow;
        if (col >= n) continue;
        const float s = scale[col];
        const float b = bias && part == 0 ? bias[col] : 0.f;
        if constexpr (YF8) {
          if (rows_in) {
            const int64_t at = row0 * yo.ld + col;
#pragma unroll
            for (int e = 0; e < 16; ++e) {
              const int64_t off = at + int64_t(8 * (e / 4) + (e % 4)) * yo.ld;
              float v = ldexpf(acc[i][j][e], ex[e]) * s;
              if (bias && part == 0) v = v + b;
              const float a = ldexpf(act(v), eo[e]);
              const _Float16 h = static_cast<_Float16>(a);
              yo.hi[off] = __builtin_bit_cast(uint16_t, h);
              yo.lo[off] =
                  uint8_t(__builtin_amdgcn_cvt_pk_fp8_f32(a - static_cast<float>(h), 0.0f, 0, false));
            }
            continue;
          }
        } else {
          if (rows_in) {
            const int64_t at = (ksplit > 1 ? int64_t(part) * m * n : 0) + row0 * n + col;
#pragma unroll
            for (int e = 0; e < 16; ++e) {
              const int64_t off = at + int64_t(8 * (e / 4) + (e % 4)) * n;
              float v = ldexpf(acc[i][j][e], ex[e]) * s;
              if (bias && part == 0) v = v + b;
              if (ksplit > 1) {
                __builtin_nontemporal_store(v, &y[off]);
              } else {
                if (z) __builtin_nontemporal_store(v, &z[off]);
                __builtin_nontemporal_store(act(v), &y[off]);
              }
            }
            continue;
          }
        }
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int64_t row = row0 + 8 * (e / 4) + (e % 4);
          if (row < m_end) {
            float v = ldexpf(acc[i][j][e], ex[e]) * s;
            if (bias && part == 0) v = v + b;
            if constexpr (YF8) {
              // the next GEMM's split of this output (split4_f16f8's arithmetic)
              const float a = ldexpf(act(v), eo[e]);
              const _Float16 h = static_cast<_Float16>(a);
              yo.hi[row * yo.ld + col] = __builtin_bit_cast(uint16_t, h);
              yo.lo[row * yo.ld + col] =
                  uint8_t(__builtin_amdgcn_cvt_pk_fp8_f32(a - static_cast<float>(h), 0.0f, 0, false));
            } else if (ksplit > 1) {
              __builtin_nontemporal_store(v, &y[int64_t(part) * m * n + row * n + col]);
            } else {
              // non-temporal: every CU writes its tile at the same moment at
              // the end of a round; streamed past the L2 the stores cost 1-4%
              // less (4096 x 1024 x 4096: 85.8 -> 82.0 us, the transformer
              // block 441 -> 432 us)
              if (z) __builtin_nontemporal_store(v, &z[row * n + col]);
              __builtin_nontemporal_store(act(v), &y[row * n + col]);
            }
          }
        }
      }
    });
  });
}

template <class C>
void launch_w8_f8(const uint16_t* xh, const uint8_t* xl, const int* xe, int64_t kp,
                  const int8_t* w, const float* scale, const float* bias, int64_t m, int64_t n,
                  int64_t k, const Epilogue& ep, float* y, float* z,
                  const RowGroups& grp = RowGroups{}, const F8Out& yo = F8Out{}, int ksplit = 1) {
  // grouped rows: every group may end in a partial tile
  const int64_t tiles_m = ceil_div(m, C::BM) + (grp.offsets ? grp.groups : 0);
  const int64_t tiles_n = ceil_div(n, C::BN);
  ENQ_REQUIRE(tiles_m * tiles_n * ksplit <= 0x7fffffff, "problem too large");
  ENQ_REQUIRE(ksplit == 1 || (yo.hi == nullptr && z == nullptr && (kp / C::BK) / ksplit >= 2),
              "split K: fp32 partial sums of at least two stages each");
  const size_t lds_bytes = size_t(C::LDS_BYTES);
  static bool attr_set = false;
  if (!attr_set) {
    for (const void* f : {reinterpret_cast<const void*>(w8_f8_ring_kernel<C, false>),
                          reinterpret_cast<const void*>(w8_f8_ring_kernel<C, true>),
                          reinterpret_cast<const void*>(w8_f8_ring_kernel<C, false, true>),
                          reinterpret_cast<const void*>(w8_f8_ring_kernel<C, true, true>)})
      ENQ_HIP(hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, int(lds_bytes)));
    attr_set = true;
  }
  auto kernel = (k % C::BK == 0) ? w8_f8_ring_kernel<C, false> : w8_f8_ring_kernel<C, true>;
  if (yo.hi)
    kernel = (k % C::BK == 0) ? w8_f8_ring_kernel<C, false, true> : w8_f8_ring_kernel<C, true, true>;
  kernel<<<unsigned(tiles_m * tiles_n * ksplit), C::NT, lds_bytes, stream()>>>(
      xh, xl, xe, kp, w, scale, bias, m, n, k, int(tiles_m), int(tiles_n), grp, ep, y, z, yo,
      ksplit);
  check_launch("w8_f8_ring_kernel");
}

// 256 x 256 tiles (two stages ahead), or 128 x 128 (three ahead) for
// outputs of fewer than three quarters of a round of large tiles
using F8Big = F8RingCfg<256, 256, 4, 2, 2>;
using F8Mid = F8RingCfg<128, 128, 4, 2, 3>;

struct F16F8View {
  uint16_t* hi;
  uint8_t* lo;
  int* exps;
};

F16F8View f16f8_view(void* buf, int64_t m, int64_t kp) {
  char* p = static_cast<char*>(buf);
  return {reinterpret_cast<uint16_t*>(p), reinterpret_cast<uint8_t*>(p + 2 * m * kp),
          reinterpret_cast<int*>(p + 3 * m * kp)};
}

}  // namespace

int64_t f16f8_k_pad(int64_t k) { return ceil_div(k, kF8KPad) * kF8KPad; }

size_t f16f8_bytes(int64_t m, int64_t k) { return size_t(m) * size_t(3 * f16f8_k_pad(k) + 4); }

bool f16f8_supported(int64_t k, const int8_t* codes) {
  return k % 16 == 0 && aligned(codes, 16);
}

void split_f16f8(const float* x, int64_t m, int64_t k, void* buf, const int* gather,
                 const float* bound, int* exps2) {
  ENQ_REQUIRE(m <= 0x7fffffff, "too many rows");
  ENQ_REQUIRE(aligned(buf, 16), "split buffer must be 16-byte aligned");
  const int64_t kp = f16f8_k_pad(k);
  const F16F8View v = f16f8_view(buf, m, kp);
  if (k % 4 == 0 && aligned(x, 16) && k <= 8192)
    split_f16f8_kernel<8, true><<<unsigned(m), 256, 0, stream()>>>(x, gather, k, kp, v.hi, v.lo,
                                                                   v.exps, bound, exps2);
  else
    split_f16f8_kernel<1, false><<<unsigned(m), 256, 0, stream()>>>(x, gather, k, kp, v.hi, v.lo,
                                                                    v.exps, bound, exps2);
  check_launch("split_f16f8_kernel");
}

void f16f8_bound_params(const int8_t* codes, int64_t rows, int64_t k, const float* w_scale,
                        const float* bias, const Epilogue& ep, float* out) {
  f16f8_bound_params(codes, rows, k, w_scale, bias, ep, out, out + 2);
}

void f16f8_bound_params(const int8_t* codes, int64_t rows, int64_t k, const float* w_scale,
                        const float* bias, const Epilogue& ep, float* out, float* part) {
  ENQ_REQUIRE(f16f8_supported(k, codes), "code norms need K a multiple of 16 and aligned codes");
  float c = 1.0f, d = 0.0f;
  switch (ep.activation) {
    case ENQ_ACT_LEAKYRELU:
    case ENQ_ACT_ELU: c = fmaxf(1.0f, fabsf(ep.alpha)); break;
    case ENQ_ACT_SELU: c = 1.76f; break;
    case ENQ_ACT_SIGMOID: c = 0.0f; d = 1.0f; break;
    case ENQ_ACT_SOFTPLUS: d = 0.7f; break;
    default: break;
  }
  const int parts = int(std::min<int64_t>(kBoundParts, ceil_div(rows, 4)));
  code_norm_kernel<<<unsigned(parts), 256, 0, stream()>>>(codes, rows, k, w_scale, part);
  check_launch("code_norm_kernel");
  f16f8_bound_kernel<<<1, 256, 0, stream()>>>(part, parts, bias, bias ? rows : 0, c, d, out);
  check_launch("f16f8_bound_kernel");
}

void gemm_w8_f16f8(const void* buf, int64_t m, int64_t k, const int8_t* codes,
                   const float* w_scale, int64_t n, const float* bias, const Epilogue& ep,
                   float* y, float* z) {
  ENQ_REQUIRE(f16f8_supported(k, codes),
              "the fp16/fp8 split GEMM needs K a multiple of 16 and 16-byte aligned codes");
  ENQ_REQUIRE(aligned(buf, 16), "split buffer must be 16-byte aligned");
  const int64_t kp = f16f8_k_pad(k);
  // the kernel addresses the planes and the codes by 32-bit byte offsets
  ENQ_REQUIRE(2 * m * kp < (int64_t(1) << 32) && n * k < (int64_t(1) << 32),
              "fp16/fp8 split GEMM operands above 4 GiB");
  const F16F8View v = f16f8_view(const_cast<void*>(buf), m, kp);
  // 256 x 256 tiles from three quarters of a round up: at 4096 x 3072 x 1024
  // the 192 large tiles in one partial round took 70 us against 83.5 us for
  // the 768 small ones in three
  const bool big = 4 * ceil_div(m, 256) * ceil_div(n, 256) >= 3 * device_cu_count();
  if (big)
    launch_w8_f8<F8Big>(v.hi, v.lo, v.exps, kp, codes, w_scale, bias, m, n, k, ep, y, z);
  else
    launch_w8_f8<F8Mid>(v.hi, v.lo, v.exps, kp, codes, w_scale, bias, m, n, k, ep, y, z);
}

void gemm_w8_f16f8_grouped(const void* buf, int64_t m, int64_t k, const int8_t* codes,
                           const float* w_scale, int64_t n, const float* bias,
                           const RowGroups& grp, const Epilogue& ep, float* y, void* out_split,
                           int ksplit) {
  ENQ_REQUIRE(f16f8_supported(k, codes),
              "the fp16/fp8 split GEMM needs K a multiple of 16 and 16-byte aligned codes");
  ENQ_REQUIRE(ep.aq == ENQ_AQ_NONE && ep.activation != ENQ_ACT_SOFTMAX,
              "grouped split GEMM epilogue: no softmax, no fake-quantization");
  const int64_t kp = f16f8_k_pad(k);
  ENQ_REQUIRE(2 * m * kp < (int64_t(1) << 32) && n * k < (int64_t(1) << 32),
              "fp16/fp8 split GEMM operands above 4 GiB");
  const F16F8View v = f16f8_view(const_cast<void*>(buf), m, kp);
  F8Out yo{};
  if (out_split) {
    ENQ_REQUIRE(n % kF8KPad == 0, "split outputs need N a multiple of 64");
    const F16F8View o = f16f8_view(out_split, m, n);
    yo = F8Out{o.hi, o.lo, o.exps, n};
  }
  ENQ_REQUIRE(ksplit == 1 || ep.activation == ENQ_ACT_LINEAR, "split K needs a linear epilogue");
  launch_w8_f8<F8Big>(v.hi, v.lo, v.exps, kp, codes, w_scale, bias, m, n, k, ep, y, nullptr, grp,
                      yo, ksplit);
}

}  // namespace enq

using namespace enq;

extern "C" int enq_split_f16f8(const float* x, int64_t m, int64_t k, void* buf) {
  return guarded([&] {
    require_init();
    ENQ_REQUIRE(m >= 1 && k >= 1, "m and k must be positive (m=%lld k=%lld)", (long long)m,
                (long long)k);
    ENQ_REQUIRE(x && buf, "NULL pointer argument");
    split_f16f8(x, m, k, buf, nullptr, nullptr, nullptr);
  });
}

extern "C" int enq_gemm_w8_f16f8(const void* buf, int64_t m, int64_t k, const int8_t* codes,
                                 const float* w_scale, int64_t n, const float* bias,
                                 int activation, float act_alpha, float act_clip, float* y,
                                 float* z) {
  return guarded([&] {
    require_init();
    ENQ_REQUIRE(m >= 1 && n >= 1 && k >= 1, "m, n, k must be positive (m=%lld n=%lld k=%lld)",
                (long long)m, (long long)n, (long long)k);
    ENQ_REQUIRE(buf && codes && w_scale && y, "NULL pointer argument");
    ENQ_REQUIRE(valid_activation(activation), "unknown activation code %d", activation);
    const Epilogue ep{activation, act_alpha, act_clip};
    gemm_w8_f16f8(buf, m, k, codes, w_scale, n, bias, gemm_epilogue(ep, false), y, z);
    finish_rows(y, m, n, ep, false);
  });
}

extern "C" int enq_dense_w8_ffn(const float* x, int64_t m, int64_t k, const int8_t* codes1,
                                const float* scale1, int64_t n1, const float* bias1, int act1,
                                float alpha1, float clip1, const float* bound1,
                                const int8_t* codes2, const float* scale2, int64_t n2,
                                const float* bias2, int act2, float alpha2, float clip2,
                                int variant, float* y) {
  return guarded([&] {
    require_init();
    ENQ_REQUIRE(m >= 1 && k >= 1 && n1 >= 1 && n2 >= 1,
                "m, k, n1, n2 must be positive (m=%lld k=%lld n1=%lld n2=%lld)", (long long)m,
                (long long)k, (long long)n1, (long long)n2);
    ENQ_REQUIRE(x && codes1 && scale1 && codes2 && scale2 && y, "NULL pointer argument");
    ENQ_REQUIRE(valid_activation(act1) && valid_activation(act2), "unknown activation code");
    ENQ_REQUIRE(variant == ENQ_W8_FP32 || variant == ENQ_W8_BF16, "unknown variant %d", variant);
    const Epilogue ep1{act1, alpha1, clip1}, ep2{act2, alpha2, clip2};
    // the split path where enq_dense_w8 takes it for both layers (more than
    // 2^33 multiply-adds or a full round of 256 x 256 tiles each)
    const auto split_size = [&](int64_t n, int64_t kk) {
      return ceil_div(m, 256) * ceil_div(n, 256) >= device_cu_count() ||
             double(m) * double(n) * double(kk) > 8589934592.0;
    };
    const bool fused = variant == ENQ_W8_FP32 && m > 64 && f16f8_supported(k, codes1) &&
                       f16f8_supported(n1, codes2) && n1 % kF8KPad == 0 &&
                       act1 != ENQ_ACT_SOFTMAX && split_size(n1, k) && split_size(n2, n1);
    if (!fused) {
      // two Dense calls through an fp32 hidden buffer (their own workspace
      // is the kernel slot, the hidden rows the layer slot)
      auto* h = static_cast<float*>(workspace(size_t(m) * size_t(n1) * sizeof(float), kLayerSlot));
      dense_w8(x, m, k, codes1, scale1, n1, bias1, ep1, variant, h, nullptr);
      dense_w8(h, m, n1, codes2, scale2, n2, bias2, ep2, variant, y, nullptr);
      return;
    }
    // x split once with the hidden rows' exponents (from the bound on the
    // first layer's outputs); the first GEMM writes the activated hidden
    // rows straight as the second GEMM's split
    const size_t b1 = ceil_div(int64_t(f16f8_bytes(m, k)), 256) * 256;
    const size_t b2 = ceil_div(int64_t(f16f8_bytes(m, n1)), 256) * 256;
    char* ws = static_cast<char*>(
        workspace(b1 + b2 + (bound1 ? 0 : sizeof(float) * (2 + kBoundParts)), kLayerSlot));
    char* split1 = ws;
    char* split2 = ws + b1;
    int* exps2 = reinterpret_cast<int*>(split2 + 3 * m * f16f8_k_pad(n1));
    const float* bound = bound1;
    if (!bound) {
      auto* b = reinterpret_cast<float*>(ws + b1 + b2);
      f16f8_bound_params(codes1, n1, k, scale1, bias1, ep1, b);
      bound = b;
    }
    split_f16f8(x, m, k, split1, nullptr, bound, exps2);
    gemm_w8_f16f8_grouped(split1, m, k, codes1, scale1, n1, bias1, RowGroups{}, ep1, nullptr,
                          split2);
    gemm_w8_f16f8(split2, m, n1, codes2, scale2, n2, bias2, gemm_epilogue(ep2, false), y,
                  nullptr);
    finish_rows(y, m, n2, ep2, false);
  });
}

extern "C" int enq_f16f8_bound(const int8_t* codes, int64_t rows, int64_t k, const float* scale,
                               const float* bias, int activation, float alpha, float clip,
                               float* out) {
  return guarded([&] {
    require_init();
    ENQ_REQUIRE(rows >= 1 && k >= 1, "rows and k must be positive");
    ENQ_REQUIRE(codes && scale && out, "NULL pointer argument");
    ENQ_REQUIRE(valid_activation(activation) && activation != ENQ_ACT_SOFTMAX,
                "activation code %d has no output bound", activation);
    auto* part = static_cast<float*>(workspace(sizeof(float) * kBoundParts));
    f16f8_bound_params(codes, rows, k, scale, bias, Epilogue{activation, alpha, clip}, out, part);
  });
}
