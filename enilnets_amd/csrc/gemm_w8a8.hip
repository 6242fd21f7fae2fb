// W8A8 Dense: int8 activation codes x int8 weight codes on the int8 matrix
// cores, int32 accumulation, fp32 epilogue.
//
//   acc[m,n] = sum_k xq[m,k] * wq[n,k]                       (exact int32)
//   y[m,n]   = act(((float)acc * x_scale[m]) * w_scale[n] + bias[n])
//
// The epilogue is evaluated in exactly that order with no fused multiply-add,
// so for the linear activation y is bit-identical to the NumPy composition
//   (acc.astype(float32) * x_scale) * w_scale.T + b.
#pragma clang fp contract(off)

#include <algorithm>
#include <cmath>
#include <cstdlib>

#include "common.hpp"
#include "epilogue.hpp"
#include "mfma.hpp"
#include "tiling.hpp"

namespace enq {

void quantize_rows_i8_internal(const float* x, int64_t rows, int64_t cols, int8_t* codes,
                               float* scale, float* zp_scratch);

namespace {

constexpr int kBK8 = 64;     // int8 codes per row per stage
constexpr int kPitch8 = 80;  // bytes per LDS row (64 + 16 pad)

// 16 codes of row `row` at column k0 of an (rows, k) int8 matrix.
template <int KMODE>
__device__ __forceinline__ int4 load_i8x16(const int8_t* __restrict__ base, int64_t ld,
                                           int64_t row, int64_t k0, int64_t k) {
  const int8_t* p = base + row * ld + k0;
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

template <int BM, int BN, int WM, int WN, int KMODE>
__global__ __launch_bounds__(WM * WN * 64) void w8a8_gemm_kernel(
    const int8_t* __restrict__ xq, const float* __restrict__ x_scale,
    const int8_t* __restrict__ wq, const float* __restrict__ w_scale,
    const float* __restrict__ bias, int64_t m, int64_t n, int64_t k, int tiles_n, Epilogue ep,
    float* __restrict__ y, int32_t* __restrict__ acc_out, const int32_t* __restrict__ w_sums,
    int corr) {
  constexpr int NT = WM * WN * 64;
  constexpr int TM = BM / WM, TN = BN / WN;
  constexpr int FM = TM / 32, FN = TN / 32;
  constexpr int A_CHUNKS = BM * (kBK8 / 16);
  constexpr int B_CHUNKS = BN * (kBK8 / 16);
  static_assert(A_CHUNKS % NT == 0 && B_CHUNKS % NT == 0, "tiles must split over threads");
  constexpr int A_PER_T = A_CHUNKS / NT, B_PER_T = B_CHUNKS / NT;

  extern __shared__ __align__(16) int8_t lds8[];
  int8_t* lds_a = lds8;                         // [2][BM][kPitch8]
  int8_t* lds_b = lds8 + 2 * BM * kPitch8;      // [2][BN][kPitch8]

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int tile = blockIdx.x;
  const int64_t m0 = int64_t(tile / tiles_n) * BM;
  const int64_t n0 = int64_t(tile % tiles_n) * BN;

  int4 a_reg[A_PER_T], b_reg[B_PER_T];
  auto load_stage = [&](int64_t k0) {
#pragma unroll
    for (int i = 0; i < A_PER_T; ++i) {
      const int q = tid + i * NT;
      const int r = q / 4, c = q % 4;
      int64_t row = m0 + r;
      row = row < m ? row : m - 1;
      a_reg[i] = load_i8x16<KMODE>(xq, k, row, k0 + c * 16, k);
    }
#pragma unroll
    for (int i = 0; i < B_PER_T; ++i) {
      const int q = tid + i * NT;
      const int r = q / 4, c = q % 4;
      int64_t row = n0 + r;
      row = row < n ? row : n - 1;
      b_reg[i] = load_i8x16<KMODE>(wq, k, row, k0 + c * 16, k);
    }
  };
  auto store_stage = [&](int buf) {
    int8_t* la = lds_a + buf * BM * kPitch8;
    int8_t* lb = lds_b + buf * BN * kPitch8;
#pragma unroll
    for (int i = 0; i < A_PER_T; ++i) {
      const int q = tid + i * NT;
      *reinterpret_cast<int4*>(la + (q / 4) * kPitch8 + (q % 4) * 16) = a_reg[i];
    }
#pragma unroll
    for (int i = 0; i < B_PER_T; ++i) {
      const int q = tid + i * NT;
      *reinterpret_cast<int4*>(lb + (q / 4) * kPitch8 + (q % 4) * 16) = b_reg[i];
    }
  };

  intx16 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0;

  const int ktiles = int(ceil_div(k, kBK8));
  load_stage(0);
  store_stage(0);
  __syncthreads();
  if (ktiles > 1) load_stage(kBK8);

  const int lrow = lane & 31;
  const int lk = (lane >> 5) * 16;
  for (int kt = 0; kt < ktiles; ++kt) {
    const int buf = kt & 1;
    const int8_t* la = lds_a + buf * BM * kPitch8;
    const int8_t* lb = lds_b + buf * BN * kPitch8;
#pragma unroll
    for (int ks = 0; ks < kBK8 / 32; ++ks) {
      intx4 af[FM], bfr[FN];
#pragma unroll
      for (int i = 0; i < FM; ++i)
        af[i] = *reinterpret_cast<const intx4*>(la + (wm * TM + i * 32 + lrow) * kPitch8 +
                                                ks * 32 + lk);
#pragma unroll
      for (int j = 0; j < FN; ++j)
        bfr[j] = *reinterpret_cast<const intx4*>(lb + (wn * TN + j * 32 + lrow) * kPitch8 +
                                                 ks * 32 + lk);
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = mfma_32x32x32_i8(af[i], bfr[j], acc[i][j]);
    }
    if (kt + 1 < ktiles) {
      store_stage(buf ^ 1);
      if (kt + 2 < ktiles) load_stage(int64_t(kt + 2) * kBK8);
    }
    __syncthreads();
  }

#pragma unroll
  for (int j = 0; j < FN; ++j) {
    const int64_t col = n0 + wn * TN + j * 32 + (lane & 31);
    if (col >= n) continue;
    const float sw = w_scale[col];
    const float b = bias ? bias[col] : 0.f;
    const int32_t add = w_sums ? corr * w_sums[col] : 0;
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int64_t row = m0 + wm * TM + i * 32 + 8 * (e / 4) + 4 * (lane >> 5) + (e % 4);
        if (row < m) {
          const int32_t a = acc[i][j][e] + add;
          if (acc_out) acc_out[row * n + col] = a;
          float v = float(a) * x_scale[row];
          v = v * sw;
          if (bias) v = v + b;
          y[row * n + col] = activate(v, ep);
        }
      }
  }
}

// ---------------------------------------------------------------------------
// Main W8A8 kernel: 256 x 256 tile, 8 waves (4 x 2, 64 x 128 each), K in
// steps of 64 codes through a 4-stage LDS ring filled by direct-to-LDS loads
// (global_load_lds_dwordx4), three stages in flight.  LDS rows are 64 bytes
// with the 16-byte chunks XOR-swizzled by row, so both the DMA writes (one
// 1 KiB block of 16 rows per instruction) and the MFMA operand reads are
// bank-conflict free.  Requires k % 16 == 0 and 16-byte aligned operands;
// 16-byte chunks past k are read from a zero block.
// ---------------------------------------------------------------------------
template <int WM_, int WN_, int STAGES_ = 4>
struct RingShape {
  static constexpr int BM = 256, BN = 256, BK = 64, STAGES = STAGES_;
  static constexpr int WM = WM_, WN = WN_, NT = WM * WN * 64;
  static constexpr int TM = BM / WM, TN = BN / WN, FM = TM / 32, FN = TN / 32;
  static constexpr int ROWS = BM + BN;                      // rows per stage (A then B)
  static constexpr int STAGE_BYTES = ROWS * BK;             // 32 KiB
  static constexpr int DMA_PER_WAVE = ROWS / 16 / (NT / 64);  // 1 KiB blocks per wave per stage
};
// 4 x 2 waves of 64 x 128: two waves per SIMD.  2 x 2 waves of 128 x 128 read
// a third less LDS per MFMA but measured 13% slower at 8192^3: with one wave
// per SIMD nothing covers the per-stage barrier and wait.
using W8a8Ring = RingShape<4, 2>;

template <class R, bool KTAIL>
__global__ __launch_bounds__(R::NT, 1) void w8a8_ring_kernel(
    const int8_t* __restrict__ xq, const float* __restrict__ x_scale,
    const int8_t* __restrict__ wq, const float* __restrict__ w_scale,
    const float* __restrict__ bias, int64_t m, int64_t n, int64_t k, int tiles_m, int tiles_n,
    Epilogue ep, float* __restrict__ y, int32_t* __restrict__ acc_out,
    const int32_t* __restrict__ w_sums, int corr) {
  constexpr int BM = R::BM, BN = R::BN, BK = R::BK, STAGES = R::STAGES;
  constexpr int WN = R::WN, TM = R::TM, TN = R::TN, FM = R::FM, FN = R::FN;
  constexpr int STAGE_BYTES = R::STAGE_BYTES, DMA_PER_WAVE = R::DMA_PER_WAVE;
  extern __shared__ __align__(16) int8_t lds8[];
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WN, wn = wave % WN;
  int tm, tn;
  xcd_tile(blockIdx.x, tiles_m, tiles_n, 4, tm, tn);
  const int64_t m0 = int64_t(tm) * BM, n0 = int64_t(tn) * BN;

  // DMA sources: block j of wave w covers stage rows w * 64 + 16 j + lane / 4,
  // physical chunk lane % 4 (logical chunk swz64(row, lane % 4)).
  const int8_t* src[DMA_PER_WAVE];
  int chunk_off[DMA_PER_WAVE];
#pragma unroll
  for (int j = 0; j < DMA_PER_WAVE; ++j) {
    const int r = wave * (DMA_PER_WAVE * 16) + 16 * j + (lane >> 2);
    chunk_off[j] = 16 * swz64(r, lane & 3);
    if (r < BM) {
      int64_t g = m0 + r;
      g = g < m ? g : m - 1;
      src[j] = xq + g * k + chunk_off[j];
    } else {
      int64_t g = n0 + (r - BM);
      g = g < n ? g : n - 1;
      src[j] = wq + g * k + chunk_off[j];
    }
  }
  const int ktiles = int(ceil_div(k, BK));
  const void* zero = g_zero16;
  // blocks [J0, J1) of this wave's share of stage t
  auto issue_blocks = [&](int t, auto j0, auto j1) {
    const uint32_t dst = lds_addr(lds8) + (t % STAGES) * STAGE_BYTES + wave * DMA_PER_WAVE * 1024;
    const int64_t k0 = int64_t(t) * BK;
#pragma unroll
    for (int j = decltype(j0)::value; j < decltype(j1)::value; ++j) {
      const void* s_ptr = src[j] + k0;
      if (KTAIL && k0 + chunk_off[j] >= k) s_ptr = zero;
      dma16(s_ptr, dst + j * 1024);
    }
  };
  auto issue = [&](int t) {
    issue_blocks(t, std::integral_constant<int, 0>{}, std::integral_constant<int, DMA_PER_WAVE>{});
  };

  intx16 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0;

  const int lrow = lane & 31, lhalf = lane >> 5;
  // per-lane LDS byte offsets of the fragments, for k-step 0 and 1
  int a_off[2][FM], b_off[2][FN];
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      const int r = wm * TM + i * 32 + lrow;
      a_off[ks][i] = r * BK + 16 * swz64(r, 2 * ks + lhalf);
    }
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const int r = BM + wn * TN + j * 32 + lrow;
      b_off[ks][j] = r * BK + 16 * swz64(r, 2 * ks + lhalf);
    }
  }
  intx4 fa[2][FM], fb[2][FN];
  auto read_frags = [&](int t, int ks) {
    const int8_t* st = lds8 + (t % STAGES) * STAGE_BYTES;
#pragma unroll
    for (int i = 0; i < FM; ++i) fa[ks][i] = *reinterpret_cast<const intx4*>(st + a_off[ks][i]);
#pragma unroll
    for (int j = 0; j < FN; ++j) fb[ks][j] = *reinterpret_cast<const intx4*>(st + b_off[ks][j]);
  };
  auto mfmas = [&](int ks) {
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j) acc[i][j] = mfma_32x32x32_i8(fa[ks][i], fb[ks][j], acc[i][j]);
  };
  // The steady loop issues a stage's DMA in DMA_GROUPS groups of blocks,
  // each followed by its share of the k-step 0 MFMAs: the eight waves'
  // blocks then reach the memory pipeline spread over the MFMAs instead of
  // all at once after the barrier (a wave stalled on a full queue cannot
  // issue the MFMAs behind it).  Same-box sweeps on 8192^3: all blocks at
  // once after the barrier 0.636-0.651 ms; two groups among the k-step 1
  // MFMAs 0.606-0.616 (four groups 0.615-0.626); two groups among the
  // k-step 0 MFMAs, one stage less ahead, 0.600-0.610.
  constexpr int DMA_GROUPS = 2;
  static_assert(DMA_PER_WAVE % DMA_GROUPS == 0 && FM * FN % DMA_GROUPS == 0, "whole shares");
  // MFMAs [Q * FM * FN / DMA_GROUPS, (Q + 1) * FM * FN / DMA_GROUPS) of
  // k-step ks, in (i, j) order: the share that follows DMA group Q
  auto mfmas_part = [&](int ks, auto qc) {
    constexpr int Q = decltype(qc)::value, PER = FM * FN / DMA_GROUPS;
#pragma unroll
    for (int f = Q * PER; f < (Q + 1) * PER; ++f)
      acc[f / FN][f % FN] = mfma_32x32x32_i8(fa[ks][f / FN], fb[ks][f % FN], acc[f / FN][f % FN]);
  };
  // the epilogue's column scales and biases, loaded before the first DMA so
  // that they arrive during the main loop; being older than every DMA they
  // only make the stage waits conservative
  float sw[FN], bj[FN];
  int32_t add[FN];
#pragma unroll
  for (int j = 0; j < FN; ++j) {
    int64_t col = n0 + wn * TN + j * 32 + lrow;
    col = col < n ? col : n - 1;
    sw[j] = w_scale[col];
    bj[j] = bias ? bias[col] : 0.f;
    add[j] = w_sums ? corr * w_sums[col] : 0;
  }
  // Stage t is complete for every wave once this wave's own DMA for it has
  // landed (vmcnt counts the later stages still in flight) and all waves
  // passed the barrier.  `issued` is the last stage issued so far.
  auto wait_stage = [&](int t, int issued) {
    const int later = (issued < ktiles - 1 ? issued : ktiles - 1) - t;
    wait_stages_after<DMA_PER_WAVE, STAGES - 2>(later);
  };

#pragma unroll
  for (int s = 0; s < STAGES - 1; ++s)
    if (s < ktiles) issue(s);
  wait_stage(0, STAGES - 2);
  wait_lgkmcnt0();  // no scalar loads pending: the loop's partial LDS waits stay exact
  block_barrier();
  read_frags(0, 0);

  // Software pipeline per stage t:
  //   read k-step 1 of t | DMA stage t+STAGES-1 into the slot of t-1, in
  //   groups among the MFMAs of k-step 0 of t | wait stage t+1, barrier |
  //   read k-step 0 of t+1 | MFMA k-step 1 of t
  // Every wave read stage t-1 before the previous barrier, so its slot is
  // free.  MFMAs stay in flight across the barrier and every LDS read
  // overlaps MFMAs.  The steady part (stage t + STAGES - 1 exists) has a
  // fixed wait count and no branch; the last stages drain the ring.
  auto stage = [&](int t, auto steady) {
    read_frags(t, 1);
    wait_lgkmcnt<FM + FN>();  // k-step 0 fragments landed, k-step 1 in flight
    sched_fence();
    if constexpr (decltype(steady)::value) {
      static_for<0, DMA_GROUPS>([&](auto qc) {
        constexpr int Q = decltype(qc)::value, B = DMA_PER_WAVE / DMA_GROUPS;
        issue_blocks(t + STAGES - 1, std::integral_constant<int, Q * B>{},
                     std::integral_constant<int, (Q + 1) * B>{});
        sched_fence();
        mfmas_part(0, qc);
        sched_fence();
      });
    } else {
      mfmas(0);
    }
    sched_fence();
    wait_lgkmcnt0();
    if constexpr (decltype(steady)::value) {
      wait_vmcnt<(STAGES - 2) * DMA_PER_WAVE>();  // stages t+2 .. t+STAGES-1 may fly
      block_barrier();
      read_frags(t + 1, 0);
    } else if (t + 1 < ktiles) {
      wait_stage(t + 1, t + STAGES - 1);
      block_barrier();
      read_frags(t + 1, 0);
    }
    sched_fence();
    mfmas(1);
    sched_fence();
  };
  int t = 0;
  for (; t + STAGES - 1 < ktiles; ++t) stage(t, std::true_type{});
  for (; t < ktiles; ++t) stage(t, std::false_type{});

  // epilogue: lane holds column l % 32; register e holds row
  // 8 * (e / 4) + 4 * (l / 32) + e % 4 of each 32 x 32 block.  One block row
  // at a time, so only its 16 row scales are live beside the accumulators.
  with_activation<false>(ep, [&](auto act) {
    static_for<0, FM>([&](auto ic) {
      constexpr int i = decltype(ic)::value;
      float xs[16];
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int64_t row = m0 + wm * TM + i * 32 + 8 * (e / 4) + 4 * lhalf + (e % 4);
        xs[e] = x_scale[row < m ? row : m - 1];
      }
      const int64_t row0 = m0 + wm * TM + i * 32 + 4 * lhalf;
      static_for<0, FN>([&](auto jc) {
        constexpr int j = decltype(jc)::value;
        const int64_t col = n0 + wn * TN + j * 32 + lrow;
        if (col >= n) return;
        if (m0 + wm * TM + i * 32 + 32 <= m) {
          // the wave's 32 rows all inside the output: no per-element row
          // test, wave-uniform row offsets (8 q + r) * n
          const int64_t at = row0 * n + col;
#pragma unroll
          for (int e = 0; e < 16; ++e) {
            const int64_t off = at + int64_t(8 * (e / 4) + (e % 4)) * n;
            const int32_t a = acc[i][j][e] + add[j];
            if (acc_out) __builtin_nontemporal_store(a, &acc_out[off]);
            float v = float(a) * xs[e];
            v = v * sw[j];
            if (bias) v = v + bj[j];
            __builtin_nontemporal_store(act(v), &y[off]);
          }
          return;
        }
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int64_t row = row0 + 8 * (e / 4) + (e % 4);
          if (row < m) {
            const int32_t a = acc[i][j][e] + add[j];
            if (acc_out) __builtin_nontemporal_store(a, &acc_out[row * n + col]);
            float v = float(a) * xs[e];
            v = v * sw[j];
            if (bias) v = v + bj[j];
            __builtin_nontemporal_store(act(v), &y[row * n + col]);
          }
        }
      });
    });
  });
}

template <class R>
void launch_w8a8_ring(const int8_t* xq, const float* xs, const int8_t* wq, const float* ws,
                      const float* bias, int64_t m, int64_t n, int64_t k, const Epilogue& ep,
                      float* y, int32_t* acc, const int32_t* w_sums, int corr) {
  const int64_t tiles_m = ceil_div(m, R::BM), tiles_n = ceil_div(n, R::BN);
  ENQ_REQUIRE(tiles_m * tiles_n <= 0x7fffffff, "problem too large");
  const size_t lds_bytes = size_t(R::STAGES) * R::STAGE_BYTES;
  static bool attr_set = false;
  if (!attr_set) {
    ENQ_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(w8a8_ring_kernel<R, false>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, int(lds_bytes)));
    ENQ_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(w8a8_ring_kernel<R, true>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, int(lds_bytes)));
    attr_set = true;
  }
  auto kernel = (k % R::BK == 0) ? w8a8_ring_kernel<R, false> : w8a8_ring_kernel<R, true>;
  kernel<<<unsigned(tiles_m * tiles_n), R::NT, lds_bytes, stream()>>>(
      xq, xs, wq, ws, bias, m, n, k, int(tiles_m), int(tiles_n), ep, y, acc, w_sums, corr);
  check_launch("w8a8_ring_kernel");
}

template <int BM, int BN, int WM, int WN, int KMODE>
void launch_w8a8(const int8_t* xq, const float* xs, const int8_t* wq, const float* ws,
                 const float* bias, int64_t m, int64_t n, int64_t k, const Epilogue& ep, float* y,
                 int32_t* acc, const int32_t* w_sums, int corr) {
  const int64_t tiles_m = ceil_div(m, BM), tiles_n = ceil_div(n, BN);
  ENQ_REQUIRE(tiles_m * tiles_n <= 0x7fffffff, "problem too large");
  const size_t lds_bytes = size_t(2) * (BM + BN) * kPitch8;
  auto kernel = w8a8_gemm_kernel<BM, BN, WM, WN, KMODE>;
  static bool attr_set = false;
  if (!attr_set) {
    ENQ_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                hipFuncAttributeMaxDynamicSharedMemorySize, int(lds_bytes)));
    attr_set = true;
  }
  kernel<<<unsigned(tiles_m * tiles_n), WM * WN * 64, lds_bytes, stream()>>>(
      xq, xs, wq, ws, bias, m, n, k, int(tiles_n), ep, y, acc, w_sums, corr);
  check_launch("w8a8_gemm_kernel");
}

template <int KMODE>
void w8a8_dispatch(const int8_t* xq, const float* xs, const int8_t* wq, const float* ws,
                   const float* bias, int64_t m, int64_t n, int64_t k, const Epilogue& ep,
                   float* y, int32_t* acc, const int32_t* w_sums, int corr) {
  const int64_t big_tiles = ceil_div(m, 256) * ceil_div(n, 256);
  if (big_tiles >= device_cu_count())
    launch_w8a8<256, 256, 4, 2, KMODE>(xq, xs, wq, ws, bias, m, n, k, ep, y, acc, w_sums, corr);
  else
    launch_w8a8<128, 128, 2, 2, KMODE>(xq, xs, wq, ws, bias, m, n, k, ep, y, acc, w_sums, corr);
}

}  // namespace

// w_sums (nullable): per output row of wq, the sum of its codes; corr * w_sums[n]
// is added to every accumulator of column n (exact int32), which turns codes
// stored shifted by `shift` with a zero point zp (corr = shift - zp) back into
// sum_k (q - zp) w.
void gemm_w8a8(const int8_t* xq, const float* xs, const int8_t* wq, const float* ws,
               const float* bias, int64_t m, int64_t n, int64_t k, const Epilogue& ep, float* y,
               int32_t* acc, const int32_t* w_sums = nullptr, int corr = 0) {
  const bool al = aligned(xq, 16) && aligned(wq, 16);
  const int64_t big_tiles = ceil_div(m, 256) * ceil_div(n, 256);
  if (k % 16 == 0 && al && big_tiles >= device_cu_count() / 2) {
    launch_w8a8_ring<W8a8Ring>(xq, xs, wq, ws, bias, m, n, k, ep, y, acc, w_sums, corr);
  }
  else if (k % kBK8 == 0 && al)
    w8a8_dispatch<0>(xq, xs, wq, ws, bias, m, n, k, ep, y, acc, w_sums, corr);
  else if (k % 16 == 0 && al)
    w8a8_dispatch<1>(xq, xs, wq, ws, bias, m, n, k, ep, y, acc, w_sums, corr);
  else
    w8a8_dispatch<2>(xq, xs, wq, ws, bias, m, n, k, ep, y, acc, w_sums, corr);
  finish_rows(y, m, n, ep, false);
}

namespace {

// Codes of x under a calibrated per-tensor spec (forward.py:798-805 with
// quantize, quantization.py:53-56): q = clip(rint(x / scale + zp), qmin,
// qmax) in the spec's arithmetic (float64 or float32), stored as int8 q -
// shift; every row's x_scale is float(scale).
__global__ __launch_bounds__(256) void quantize_static_kernel(
    const float* __restrict__ x, int64_t n, int64_t rows, Epilogue ep, int shift,
    int8_t* __restrict__ codes, float* __restrict__ x_scale) {
  const double inv = 1.0 / ep.aq_scale;
  for (int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x; i < n;
       i += int64_t(gridDim.x) * 256) {
    const float v = x[i];
    double q;
    if (ep.aq == ENQ_AQ_F64) {
      // multiply by the reciprocal except within 1e-6 of a rounding tie,
      // where the two can differ: then the true division
      const double t = double(v) * inv + ep.aq_zp;
      const double fr = t - floor(t);
      q = fabs(fr - 0.5) < 1e-6 ? rint(double(v) / ep.aq_scale + ep.aq_zp) : rint(t);
    } else {
      q = double(rintf(__fdiv_rn(v, float(ep.aq_scale)) + float(ep.aq_zp)));
    }
    // NaN stays NaN through the reference's clip; its code is 0 (q = shift)
    q = q != q ? double(shift) : (q < double(ep.aq_qmin) ? double(ep.aq_qmin)
                                  : (q > double(ep.aq_qmax) ? double(ep.aq_qmax) : q));
    codes[i] = int8_t(int(q) - shift);
  }
  for (int64_t r = int64_t(blockIdx.x) * 256 + threadIdx.x; r < rows;
       r += int64_t(gridDim.x) * 256)
    x_scale[r] = float(ep.aq_scale);
}

// sums[r] = sum of the k int8 codes of row r (one wave per row).
__global__ __launch_bounds__(256) void code_row_sums_kernel(const int8_t* __restrict__ codes,
                                                            int64_t rows, int64_t k,
                                                            int32_t* __restrict__ sums) {
  const int64_t r = int64_t(blockIdx.x) * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (r >= rows) return;
  const int8_t* row = codes + r * k;
  int32_t s = 0;
  for (int64_t i = lane; i < k; i += 64) s += row[i];
  for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off);
  if (lane == 0) sums[r] = s;
}

}  // namespace

}  // namespace enq

using namespace enq;

extern "C" {

int enq_gemm_w8a8(const int8_t* x_codes, const float* x_scale, const int8_t* w_codes,
                  const float* w_scale, const float* bias, int64_t m, int64_t n, int64_t k,
                  int activation, float act_alpha, float act_clip, float* y, int32_t* acc) {
  return guarded([&] {
    require_init();
    ENQ_REQUIRE(m >= 1 && n >= 1 && k >= 1, "m, n, k must be positive");
    ENQ_REQUIRE(k <= 133143, "k=%lld can overflow the int32 accumulator (max 133143)",
                (long long)k);
    ENQ_REQUIRE(x_codes && x_scale && w_codes && w_scale && y, "NULL pointer argument");
    ENQ_REQUIRE(valid_activation(activation), "unknown activation code %d", activation);
    Epilogue ep{activation, act_alpha, act_clip};
    gemm_w8a8(x_codes, x_scale, w_codes, w_scale, bias, m, n, k, ep, y, acc);
  });
}

int enq_code_row_sums(const int8_t* codes, int64_t rows, int64_t k, int32_t* sums) {
  return guarded([&] {
    require_init();
    ENQ_REQUIRE(rows >= 1 && k >= 1, "rows and k must be positive");
    ENQ_REQUIRE(k <= 16909320, "k=%lld can overflow an int32 code sum", (long long)k);
    ENQ_REQUIRE(codes && sums, "NULL pointer argument");
    const int64_t blocks = ceil_div(rows, 4);
    ENQ_REQUIRE(blocks <= 0x7fffffff, "too many rows");
    code_row_sums_kernel<<<unsigned(blocks), 256, 0, stream()>>>(codes, rows, k, sums);
    check_launch("code_row_sums_kernel");
  });
}

int enq_dense_w8a8_static(const float* x, int64_t m, int64_t k, int aq_mode, double x_scale,
                          double x_zero_point, float qmin, float qmax, const int8_t* codes,
                          const float* w_scale, const int32_t* w_code_sums, int64_t n,
                          const float* bias, int activation, float act_alpha, float act_clip,
                          float* y, int32_t* acc) {
  return guarded([&] {
    require_init();
    ENQ_REQUIRE(m >= 1 && n >= 1 && k >= 1, "m, n, k must be positive");
    ENQ_REQUIRE(x && codes && w_scale && y, "NULL pointer argument");
    ENQ_REQUIRE(valid_activation(activation), "unknown activation code %d", activation);
    ENQ_REQUIRE(aq_mode == ENQ_AQ_F32 || aq_mode == ENQ_AQ_F64, "unknown act-quant mode %d",
                aq_mode);
    ENQ_REQUIRE(valid_act_quant(aq_mode, x_scale, qmin, qmax), "invalid act-quant parameters");
    ENQ_REQUIRE(qmin == float(int(qmin)) && qmax == float(int(qmax)) && qmax - qmin <= 255.0f,
                "the activation grid [%g, %g] does not fit 8 bits", double(qmin), double(qmax));
    ENQ_REQUIRE(x_zero_point == double(int64_t(x_zero_point)) && x_zero_point >= -1024 &&
                    x_zero_point <= 1024,
                "the zero point must be a small integer (got %g)", x_zero_point);
    // codes are stored as int8 q - shift
    const int shift = qmax > 127.0f ? 128 : 0;
    ENQ_REQUIRE(qmin - shift >= -128.0f && qmax - shift <= 127.0f,
                "the activation grid [%g, %g] does not fit int8", double(qmin), double(qmax));
    const int corr = shift - int(x_zero_point);
    ENQ_REQUIRE(corr == 0 || w_code_sums, "w_code_sums is needed for a zero point of %g",
                x_zero_point);
    // |sum (q - shift) w| + |corr sum w| <= (128 + |corr|) * 127 * k < 2^31
    ENQ_REQUIRE(double(128 + std::abs(corr)) * 127.0 * double(k) < 2147483648.0,
                "k=%lld can overflow the int32 accumulator", (long long)k);
    const size_t code_bytes = (size_t(m) * size_t(k) + 255) / 256 * 256;
    char* ws = static_cast<char*>(workspace(code_bytes + sizeof(float) * size_t(m)));
    auto* xq = reinterpret_cast<int8_t*>(ws);
    auto* xs = reinterpret_cast<float*>(ws + code_bytes);
    Epilogue aq{ENQ_ACT_LINEAR, 0.f, 0.f};
    aq.aq = aq_mode;
    aq.aq_scale = x_scale;
    aq.aq_zp = x_zero_point;
    aq.aq_qmin = qmin;
    aq.aq_qmax = qmax;
    const int64_t total = m * k;
    const int64_t blocks = std::min<int64_t>(ceil_div(total, 256), int64_t(device_cu_count()) * 32);
    quantize_static_kernel<<<unsigned(blocks), 256, 0, stream()>>>(x, total, m, aq, shift, xq, xs);
    check_launch("quantize_static_kernel");
    Epilogue ep{activation, act_alpha, act_clip};
    gemm_w8a8(xq, xs, codes, w_scale, bias, m, n, k, ep, y, acc, corr ? w_code_sums : nullptr,
              corr);
  });
}

int enq_dense_w8a8(const float* x, int64_t m, int64_t k, const int8_t* codes,
                   const float* w_scale, int64_t n, const float* bias, int activation,
                   float act_alpha, float act_clip, float* y, int32_t* acc) {
  return guarded([&] {
    require_init();
    ENQ_REQUIRE(m >= 1 && n >= 1 && k >= 1, "m, n, k must be positive");
    ENQ_REQUIRE(k <= 133143, "k=%lld can overflow the int32 accumulator (max 133143)",
                (long long)k);
    ENQ_REQUIRE(x && codes && w_scale && y, "NULL pointer argument");
    ENQ_REQUIRE(valid_activation(activation), "unknown activation code %d", activation);
    const size_t code_bytes = (size_t(m) * size_t(k) + 255) / 256 * 256;
    char* ws = static_cast<char*>(workspace(code_bytes + 2 * sizeof(float) * size_t(m)));
    auto* xq = reinterpret_cast<int8_t*>(ws);
    auto* xs = reinterpret_cast<float*>(ws + code_bytes);
    float* zp = xs + m;
    quantize_rows_i8_internal(x, m, k, xq, xs, zp);
    Epilogue ep{activation, act_alpha, act_clip};
    gemm_w8a8(xq, xs, codes, w_scale, bias, m, n, k, ep, y, acc);
  });
}

}  // extern "C"
