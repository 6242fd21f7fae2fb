// Mixture-of-experts layer on int8 expert weights
// (Enilnets/nn/moe.py:23-87).
//
//   router      logits = x . Wr^T + br (the W8 Dense), or caller-given logits
//   route       softmax over experts, top-k per token, gates = raw probabilities
//   sort        tokens grouped by expert, each group in token order: the
//               order of np.nonzero(top_idx == e) (moe.py:72-75)
//   expert FFN  one grouped GEMM per weight: rows of group e use expert e's
//               codes; act(x_e . W1[e]^T + b1[e]) . W2[e]^T + b2[e]
//   combine     out[t] = sum over t's experts in ascending expert index of
//               gate * y, the accumulation order of np.add.at (moe.py:82)
//
// Nothing is copied to the host: group sizes stay on the device and the
// grouped GEMM finds each tile's expert from the group offsets.
#include <algorithm>
#include <climits>

#include "common.hpp"
#include "epilogue.hpp"
#include "ops.hpp"

#pragma clang fp contract(off)

namespace enq {
namespace {

constexpr int kMaxExperts = 256;
constexpr int kSortBlock = 256;

// moe.py:23-28 (softmax of the logits) and :31-35 (top-k).  One thread per
// token.  Slots are filled largest probability first; among equal
// probabilities the lower expert index comes first.
__global__ __launch_bounds__(256) void moe_route_kernel(const float* __restrict__ logits,
                                                        int64_t tokens, int experts, int top_k,
                                                        float* __restrict__ probs,
                                                        int* __restrict__ chosen,
                                                        float* __restrict__ gates) {
  const int64_t t = int64_t(blockIdx.x) * 256 + threadIdx.x;
  if (t >= tokens) return;
  const float* l = logits + t * experts;
  float* p = probs + t * experts;
  float mx = l[0];
  for (int e = 1; e < experts; ++e) {
    const float v = l[e];
    mx = (v > mx || v != v) ? v : mx;  // np.max propagates NaN
  }
  float sum = 0.0f;
  for (int e = 0; e < experts; ++e) {
    const float v = expf(l[e] - mx);
    p[e] = v;
    sum = sum + v;
  }
  for (int e = 0; e < experts; ++e) p[e] = p[e] / sum;
  uint64_t taken[kMaxExperts / 64] = {};
  for (int s = 0; s < top_k; ++s) {
    int best = -1;
    float bv = 0.0f;
    for (int e = 0; e < experts; ++e) {
      if ((taken[e >> 6] >> (e & 63)) & 1) continue;
      const float v = p[e];
      if (best < 0 || v > bv) {
        best = e;
        bv = v;
      }
    }
    taken[best >> 6] |= uint64_t(1) << (best & 63);
    chosen[t * top_k + s] = best;
    gates[t * top_k + s] = bv;
  }
}

// The same routing with the token's logits and probabilities held in
// registers, for experts <= EMAX: the kernel above reads each probability
// back from global memory after storing it, and its dynamically indexed
// mask lives in private memory.  Same operations in the same order, so the
// same bits.
template <int EMAX>
__global__ __launch_bounds__(256) void moe_route_regs_kernel(const float* __restrict__ logits,
                                                             int64_t tokens, int experts,
                                                             int top_k,
                                                             float* __restrict__ probs,
                                                             int* __restrict__ chosen,
                                                             float* __restrict__ gates) {
  static_assert(EMAX <= 32, "the mask is one 32-bit word");
  const int64_t t = int64_t(blockIdx.x) * 256 + threadIdx.x;
  if (t >= tokens) return;
  const float* l = logits + t * experts;
  float v[EMAX];
#pragma unroll
  for (int e = 0; e < EMAX; ++e) v[e] = l[e < experts ? e : 0];  // in-bounds, masked below
  float mx = v[0];
#pragma unroll
  for (int e = 1; e < EMAX; ++e)
    if (e < experts) mx = (v[e] > mx || v[e] != v[e]) ? v[e] : mx;  // np.max propagates NaN
  float sum = 0.0f;
#pragma unroll
  for (int e = 0; e < EMAX; ++e) {
    if (e < experts) {
      v[e] = expf(v[e] - mx);
      sum = sum + v[e];
    }
  }
  float* p = probs + t * experts;
#pragma unroll
  for (int e = 0; e < EMAX; ++e) {
    if (e < experts) {
      v[e] = v[e] / sum;
      p[e] = v[e];
    }
  }
  uint32_t taken = 0;
  for (int s = 0; s < top_k; ++s) {
    int best = -1;  // top_k <= experts: an expert is always left
    float bv = 0.0f;
#pragma unroll
    for (int e = 0; e < EMAX; ++e) {
      if (e >= experts || ((taken >> e) & 1u)) continue;
      if (best < 0 || v[e] > bv) {
        best = e;
        bv = v[e];
      }
    }
    taken |= 1u << best;
    chosen[t * top_k + s] = best;
    gates[t * top_k + s] = bv;
  }
}

// Per-block count of the (token, slot) entries routed to each expert.
__global__ __launch_bounds__(kSortBlock) void moe_count_kernel(const int* __restrict__ chosen,
                                                               int64_t entries, int experts,
                                                               int* __restrict__ hist) {
  __shared__ int cnt[kMaxExperts];
  for (int e = threadIdx.x; e < experts; e += kSortBlock) cnt[e] = 0;
  __syncthreads();
  const int64_t i = int64_t(blockIdx.x) * kSortBlock + threadIdx.x;
  if (i < entries) atomicAdd(&cnt[chosen[i]], 1);
  __syncthreads();
  for (int e = threadIdx.x; e < experts; e += kSortBlock)
    hist[int64_t(blockIdx.x) * experts + e] = cnt[e];
}

// One workgroup: turns the block counts into each block's first position per
// expert, and writes the group offsets (experts + 1 values).
__global__ __launch_bounds__(256) void moe_scan_kernel(int* __restrict__ hist, int blocks,
                                                       int experts, int* __restrict__ offsets) {
  // one wave per expert column of hist, 64 blocks at a time
  __shared__ int total[kMaxExperts];
  __shared__ int first[kMaxExperts];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  for (int e = wave; e < experts; e += 4) {
    int sum = 0;
    for (int b0 = 0; b0 < blocks; b0 += 64) {
      const int b = b0 + lane;
      sum += b < blocks ? hist[int64_t(b) * experts + e] : 0;
    }
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) sum += __shfl_xor(sum, m, 64);
    if (lane == 0) total[e] = sum;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    int run = 0;
    for (int e = 0; e < experts; ++e) {
      first[e] = run;
      offsets[e] = run;
      run += total[e];
    }
    offsets[experts] = run;
  }
  __syncthreads();
  // exclusive prefix over the blocks, from the expert's first position
  for (int e = wave; e < experts; e += 4) {
    int run = first[e];
    for (int b0 = 0; b0 < blocks; b0 += 64) {
      const int b = b0 + lane;
      const int c = b < blocks ? hist[int64_t(b) * experts + e] : 0;
      int x = c;
#pragma unroll
      for (int d = 1; d < 64; d <<= 1) {
        const int y = __shfl_up(x, d, 64);
        if (lane >= d) x += y;
      }
      if (b < blocks) hist[int64_t(b) * experts + e] = run + x - c;
      run += __shfl(x, 63, 64);
    }
  }
}

// Position of every entry in the expert-sorted order: its block's first
// position for the expert plus the number of earlier entries of the block
// with the same expert.
__global__ __launch_bounds__(kSortBlock) void moe_place_kernel(const int* __restrict__ chosen,
                                                               int64_t entries, int top_k,
                                                               int experts,
                                                               const int* __restrict__ base,
                                                               int* __restrict__ row_token,
                                                               int* __restrict__ entry_pos) {
  __shared__ int ex[kSortBlock];
  const int64_t i = int64_t(blockIdx.x) * kSortBlock + threadIdx.x;
  const int e = i < entries ? chosen[i] : -1;
  ex[threadIdx.x] = e;
  __syncthreads();
  if (i >= entries) return;
  int rank = 0;
  for (int j = 0; j < int(threadIdx.x); ++j) rank += ex[j] == e;
  const int pos = base[int64_t(blockIdx.x) * experts + e] + rank;
  row_token[pos] = int(i / top_k);
  entry_pos[i] = pos;
}

// out[t, c] = sum over t's slots in ascending expert order of gate * y.
template <int V>
__global__ __launch_bounds__(256) void moe_combine_kernel(const float* __restrict__ yg,
                                                          const float* __restrict__ yg2,
                                                          const int* __restrict__ chosen,
                                                          const float* __restrict__ gates,
                                                          const int* __restrict__ entry_pos,
                                                          int64_t tokens, int64_t d, int top_k,
                                                          float* __restrict__ out) {
  const int64_t per_row = d / V;
  const int64_t gid = int64_t(blockIdx.x) * 256 + threadIdx.x;
  if (gid >= tokens * per_row) return;
  const int64_t t = gid / per_row;
  const int64_t c0 = (gid - t * per_row) * V;
  float acc[V];
#pragma unroll
  for (int v = 0; v < V; ++v) acc[v] = 0.0f;
  const int* ch = chosen + t * top_k;
  int last = -1;
  for (int s = 0; s < top_k; ++s) {
    int slot = 0, best = INT_MAX;
    for (int q = 0; q < top_k; ++q) {
      const int e = ch[q];
      if (e > last && e < best) {
        best = e;
        slot = q;
      }
    }
    last = best;
    const float g = gates[t * top_k + slot];
    const int64_t at = int64_t(entry_pos[t * top_k + slot]) * d + c0;
    const float* y = yg + at;
    float q[V];
    if constexpr (V == 4) {
      const float4 w = *reinterpret_cast<const float4*>(y);
      q[0] = w.x;
      q[1] = w.y;
      q[2] = w.z;
      q[3] = w.w;
      if (yg2) {
        // the second K part of the expert GEMM
        const float4 w2 = *reinterpret_cast<const float4*>(yg2 + at);
        q[0] = q[0] + w2.x;
        q[1] = q[1] + w2.y;
        q[2] = q[2] + w2.z;
        q[3] = q[3] + w2.w;
      }
    } else {
#pragma unroll
      for (int v = 0; v < V; ++v) q[v] = yg2 ? y[v] + yg2[at + v] : y[v];
    }
#pragma unroll
    for (int v = 0; v < V; ++v) acc[v] = acc[v] + g * q[v];
  }
  float* o = out + t * d + c0;
  if constexpr (V == 4) {
    *reinterpret_cast<float4*>(o) = make_float4(acc[0], acc[1], acc[2], acc[3]);
  } else {
#pragma unroll
    for (int v = 0; v < V; ++v) o[v] = acc[v];
  }
}

// Load-balancing loss terms (moe.py:38-49): for expert e (one workgroup
// each), f_e = share of tokens whose first choice is e and P_e = mean router
// probability; term[e] = f_e * P_e.
__global__ __launch_bounds__(256) void moe_aux_terms_kernel(const float* __restrict__ probs,
                                                            const int* __restrict__ chosen,
                                                            int64_t tokens, int experts,
                                                            int top_k, double* __restrict__ term) {
  __shared__ double ps[256];
  __shared__ int64_t cs[256];
  const int e = blockIdx.x;
  double p = 0.0;
  int64_t c = 0;
  for (int64_t t = threadIdx.x; t < tokens; t += 256) {
    p += double(probs[t * experts + e]);
    c += chosen[t * top_k] == e;
  }
  ps[threadIdx.x] = p;
  cs[threadIdx.x] = c;
  __syncthreads();
  for (int w = 128; w > 0; w >>= 1) {
    if (int(threadIdx.x) < w) {
      ps[threadIdx.x] += ps[threadIdx.x + w];
      cs[threadIdx.x] += cs[threadIdx.x + w];
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    const double n = double(tokens > 0 ? tokens : 1);
    term[e] = (double(cs[0]) / n) * (ps[0] / double(tokens));
  }
}

__global__ void moe_aux_sum_kernel(const double* __restrict__ term, int experts,
                                   double* __restrict__ loss) {
  if (threadIdx.x != 0 || blockIdx.x != 0) return;
  double s = 0.0;
  for (int e = 0; e < experts; ++e) s += term[e];
  loss[0] = double(experts) * s;
}

// Copies rows: out[r] = x[rows[r]].
__global__ __launch_bounds__(256) void gather_rows_kernel(const float* __restrict__ x,
                                                          const int* __restrict__ rows,
                                                          int64_t m, int64_t k,
                                                          float* __restrict__ out) {
  const int64_t gid = int64_t(blockIdx.x) * 256 + threadIdx.x;
  if (gid >= m * k) return;
  const int64_t r = gid / k, c = gid - r * k;
  out[gid] = x[int64_t(rows[r]) * k + c];
}

// Bump allocator over one workspace block, 256-byte aligned pieces.
class Carve {
 public:
  explicit Carve(char* base) : base_(base) {}
  template <class T>
  T* take(int64_t count) {
    T* p = reinterpret_cast<T*>(base_ ? base_ + used_ : nullptr);
    used_ += (size_t(count) * sizeof(T) + 255) / 256 * 256;
    return p;
  }
  size_t used() const { return used_; }

 private:
  char* base_;
  size_t used_ = 0;
};

unsigned blocks_for(int64_t work, int per_block = 256) {
  const int64_t b = ceil_div(work, per_block);
  ENQ_REQUIRE(b <= 0x7fffffff, "problem too large");
  return unsigned(b > 0 ? b : 1);
}

struct MoeArgs {
  const float* x;
  int64_t tokens, d;
  const float* logits;
  const int8_t* wr;
  const float* sr;
  const float* br;
  const int8_t* w1;
  const float* s1;
  const float* b1;
  const int8_t* w2;
  const float* s2;
  const float* b2;
  int64_t experts, hidden;
  int top_k;
  Epilogue ep;
  int variant;
  float* out;
  float* probs;
  int32_t* top_idx;
  double* aux_loss;
  const float* bound1;  // the first layer's output bound (enq_f16f8_bound), or null
};

void moe_w8(const MoeArgs& a) {
  const int64_t entries = a.tokens * a.top_k;
  const int64_t sort_blocks = ceil_div(entries, kSortBlock);
  const int planes = a.variant == ENQ_W8_FP32 ? 2 : 1;
  const int E = int(a.experts);
  const bool grouped = grouped_gemm_supported(a.d, a.w1) && grouped_gemm_supported(a.hidden, a.w2);
  const int64_t kp1 = gemm_k_pad(a.d), kp2 = gemm_k_pad(a.hidden);
  // fp32-accurate expert GEMMs on the fp16 / e4m3 split: the gathered token
  // rows are split once, the first GEMM writes the hidden activations as the
  // second's split, and neither GEMM reads bf16 planes.  The hidden rows'
  // exponents come from a bound computed in the first split,
  // ||x||_2 * max_n scale_n ||q_n||_2 (+ bias, widened for the activation),
  // which stays within a few powers of two of the rows' true maxima, so the
  // high parts stay inside fp16's range and the low parts of the outputs
  // that matter inside e4m3's normal range
  const bool split8 = grouped && planes == 2 && f16f8_supported(a.d, a.w1) &&
                      f16f8_supported(a.hidden, a.w2) && a.hidden % 64 == 0 &&
                      a.ep.aq == ENQ_AQ_NONE && a.ep.activation != ENQ_ACT_SOFTMAX;

  // sizes first (null base), then the real carve of one workspace block
  auto layout = [&](char* base, auto&& use) {
    Carve c(base);
    float* logits = a.logits ? nullptr : c.take<float>(a.tokens * E);
    float* probs = a.probs ? nullptr : c.take<float>(a.tokens * E);
    int* chosen = c.take<int>(entries);
    float* gates = c.take<float>(entries);
    int* hist = c.take<int>(sort_blocks * E);
    int* offsets = c.take<int>(E + 1);
    int* row_token = c.take<int>(entries);
    int* entry_pos = c.take<int>(entries);
    double* terms = c.take<double>(E);
    const bool pl = grouped && !split8;
    uint16_t* planes1 = pl ? c.take<uint16_t>(int64_t(planes) * entries * kp1) : nullptr;
    float* xg = grouped ? nullptr : c.take<float>(entries * a.d);
    float* h = split8 ? nullptr : c.take<float>(entries * a.hidden);
    uint16_t* planes2 = pl ? c.take<uint16_t>(int64_t(planes) * entries * kp2) : nullptr;
    float* yg = c.take<float>(entries * a.d * (split8 ? 2 : 1));
    char* split1 = split8 ? c.take<char>(int64_t(f16f8_bytes(entries, a.d))) : nullptr;
    char* split2 = split8 ? c.take<char>(int64_t(f16f8_bytes(entries, a.hidden))) : nullptr;
    float* bound = split8 ? c.take<float>(2 + kBoundParts) : nullptr;
    use(c.used(), logits, probs, chosen, gates, hist, offsets, row_token, entry_pos, terms,
        planes1, xg, h, planes2, yg, split1, split2, bound);
  };
  size_t bytes = 0;
  layout(nullptr, [&](size_t used, auto...) { bytes = used; });
  char* ws = static_cast<char*>(workspace(bytes, kLayerSlot));
  layout(ws, [&](size_t, float* logits, float* probs, int* chosen, float* gates, int* hist,
                 int* offsets, int* row_token, int* entry_pos, double* terms, uint16_t* planes1,
                 float* xg, float* h, uint16_t* planes2, float* yg, char* split1, char* split2,
                 float* bound) {
    if (a.logits) logits = const_cast<float*>(a.logits);
    if (a.probs) probs = a.probs;
    hipStream_t s = stream();
    if (!a.logits) {
      const Epilogue lin{ENQ_ACT_LINEAR, 0.0f, 0.0f};
      dense_w8(a.x, a.tokens, a.d, a.wr, a.sr, E, a.br, lin, a.variant, logits, nullptr);
    }
    if (E <= 8)
      moe_route_regs_kernel<8><<<blocks_for(a.tokens), 256, 0, s>>>(logits, a.tokens, E, a.top_k,
                                                                    probs, chosen, gates);
    else if (E <= 32)
      moe_route_regs_kernel<32><<<blocks_for(a.tokens), 256, 0, s>>>(logits, a.tokens, E,
                                                                     a.top_k, probs, chosen, gates);
    else
      moe_route_kernel<<<blocks_for(a.tokens), 256, 0, s>>>(logits, a.tokens, E, a.top_k, probs,
                                                             chosen, gates);
    check_launch("moe_route_kernel");
    moe_count_kernel<<<unsigned(sort_blocks), kSortBlock, 0, s>>>(chosen, entries, E, hist);
    check_launch("moe_count_kernel");
    moe_scan_kernel<<<1, 256, 0, s>>>(hist, int(sort_blocks), E, offsets);
    check_launch("moe_scan_kernel");
    moe_place_kernel<<<unsigned(sort_blocks), kSortBlock, 0, s>>>(chosen, entries, a.top_k, E,
                                                                  hist, row_token, entry_pos);
    check_launch("moe_place_kernel");

    const Epilogue lin{ENQ_ACT_LINEAR, 0.0f, 0.0f};
    const float* yg2 = nullptr;  // the second K part of the expert outputs, if split
    if (split8) {
      RowGroups g1{offsets, E, a.hidden * a.d, a.hidden};
      RowGroups g2{offsets, E, a.d * a.hidden, a.d};
      // the second split's exponents sit after its two planes
      int* exps2 = reinterpret_cast<int*>(split2 + 3 * entries * f16f8_k_pad(a.hidden));
      const float* bnd = a.bound1;
      if (!bnd) {
        f16f8_bound_params(a.w1, E * a.hidden, a.d, a.s1, a.b1, a.ep, bound);
        bnd = bound;
      }
      split_f16f8(a.x, entries, a.d, split1, row_token, bnd, exps2);
      gemm_w8_f16f8_grouped(split1, entries, a.d, a.w1, a.s1, a.hidden, a.b1, g1, a.ep, nullptr,
                            split2);
      // K of the second GEMM in two parts, added in the combine: its tiles
      // (ceil(entries / 256) + E tile rows x d / 256) slightly exceed one
      // round of the device at configs[4], where a second round held 8 tiles
      const int64_t t2 = (ceil_div(entries, 256) + E) * ceil_div(a.d, 256);
      const int64_t cus = device_cu_count();
      const bool halves = a.hidden >= 256 && ceil_div(2 * t2, cus) < 2 * ceil_div(t2, cus);
      gemm_w8_f16f8_grouped(split2, entries, a.hidden, a.w2, a.s2, a.d, a.b2, g2, lin, yg,
                            nullptr, halves ? 2 : 1);
      if (halves) yg2 = yg + entries * a.d;
    } else if (grouped) {
      RowGroups g1{offsets, E, a.hidden * a.d, a.hidden};
      RowGroups g2{offsets, E, a.d * a.hidden, a.d};
      split_planes(a.x, row_token, entries, a.d, planes1, entries, kp1, planes);
      if (kp2 == a.hidden) {
        // the first GEMM writes the hidden activations straight into the
        // second's planes (no fp32 round trip through HBM)
        dense_w8_grouped(planes1, entries * kp1, kp1, planes, entries, a.d, a.w1, a.s1,
                         a.hidden, a.b1, g1, a.ep, nullptr, planes2, entries * kp2);
      } else {
        dense_w8_grouped(planes1, entries * kp1, kp1, planes, entries, a.d, a.w1, a.s1,
                         a.hidden, a.b1, g1, a.ep, h);
        split_planes(h, nullptr, entries, a.hidden, planes2, entries, kp2, planes);
      }
      dense_w8_grouped(planes2, entries * kp2, kp2, planes, entries, a.hidden, a.w2, a.s2, a.d,
                       a.b2, g2, lin, yg);
    } else {
      // K not a multiple of 16 (or unaligned codes): one Dense call per
      // expert, which needs the group sizes on the host
      gather_rows_kernel<<<blocks_for(entries * a.d), 256, 0, s>>>(a.x, row_token, entries, a.d,
                                                                   xg);
      check_launch("gather_rows_kernel");
      int host_off[kMaxExperts + 1];
      ENQ_HIP(hipMemcpyAsync(host_off, offsets, sizeof(int) * (E + 1), hipMemcpyDeviceToHost, s));
      ENQ_HIP(hipStreamSynchronize(s));
      for (int e = 0; e < E; ++e) {
        const int64_t r0 = host_off[e], me = host_off[e + 1] - host_off[e];
        if (me == 0) continue;
        dense_w8(xg + r0 * a.d, me, a.d, a.w1 + int64_t(e) * a.hidden * a.d,
                 a.s1 + int64_t(e) * a.hidden, a.hidden,
                 a.b1 ? a.b1 + int64_t(e) * a.hidden : nullptr, a.ep, a.variant,
                 h + r0 * a.hidden, nullptr);
        dense_w8(h + r0 * a.hidden, me, a.hidden, a.w2 + int64_t(e) * a.d * a.hidden,
                 a.s2 + int64_t(e) * a.d, a.d, a.b2 ? a.b2 + int64_t(e) * a.d : nullptr, lin,
                 a.variant, yg + r0 * a.d, nullptr);
      }
    }
    if (a.d % 4 == 0 && aligned(a.out, 16))
      moe_combine_kernel<4><<<blocks_for(a.tokens * (a.d / 4)), 256, 0, s>>>(
          yg, yg2, chosen, gates, entry_pos, a.tokens, a.d, a.top_k, a.out);
    else
      moe_combine_kernel<1><<<blocks_for(a.tokens * a.d), 256, 0, s>>>(
          yg, yg2, chosen, gates, entry_pos, a.tokens, a.d, a.top_k, a.out);
    check_launch("moe_combine_kernel");
    if (a.top_idx)
      ENQ_HIP(hipMemcpyAsync(a.top_idx, chosen, sizeof(int) * entries, hipMemcpyDeviceToDevice,
                             s));
    if (a.aux_loss) {
      moe_aux_terms_kernel<<<unsigned(E), 256, 0, s>>>(probs, chosen, a.tokens, E, a.top_k,
                                                       terms);
      check_launch("moe_aux_terms_kernel");
      moe_aux_sum_kernel<<<1, 64, 0, s>>>(terms, E, a.aux_loss);
      check_launch("moe_aux_sum_kernel");
    }
  });
}

}  // namespace
}  // namespace enq

using namespace enq;

extern "C" int enq_moe_w8(const float* x, int64_t tokens, int64_t d, const float* router_logits,
                          const int8_t* wr, const float* sr, const float* br, const int8_t* w1,
                          const float* s1, const float* b1, const int8_t* w2, const float* s2,
                          const float* b2, int64_t experts, int64_t hidden, int top_k,
                          int activation, float act_alpha, float act_clip,
                          const float* bound1, int variant, float* out, float* probs,
                          int32_t* top_idx, double* aux_loss) {
  return guarded([&] {
    require_init();
    ENQ_REQUIRE(tokens >= 1 && d >= 1 && hidden >= 1,
                "tokens, d, hidden must be positive (tokens=%lld d=%lld hidden=%lld)",
                (long long)tokens, (long long)d, (long long)hidden);
    ENQ_REQUIRE(experts >= 1 && experts <= kMaxExperts, "experts must be in [1, %d], got %lld",
                kMaxExperts, (long long)experts);
    ENQ_REQUIRE(top_k >= 1 && top_k <= experts,
                "top_k must be between 1 and num_experts (%lld), got %d", (long long)experts,
                top_k);
    ENQ_REQUIRE(x && w1 && s1 && w2 && s2 && out, "NULL pointer argument");
    ENQ_REQUIRE(router_logits || (wr && sr), "router weights or logits required");
    ENQ_REQUIRE(tokens * top_k <= INT_MAX && tokens * top_k * std::max(d, hidden) <= (int64_t(1) << 40),
                "problem too large");
    ENQ_REQUIRE(valid_activation(activation) && activation != ENQ_ACT_SOFTMAX,
                "unsupported expert activation code %d", activation);
    ENQ_REQUIRE(variant == ENQ_W8_FP32 || variant == ENQ_W8_BF16, "unknown variant %d", variant);
    MoeArgs a{x,  tokens, d,  router_logits, wr, sr, br, w1, s1, b1, w2, s2, b2, experts, hidden,
              top_k, Epilogue{activation, act_alpha, act_clip}, variant, out, probs, top_idx,
              aux_loss, bound1};
    moe_w8(a);
  });
}
