// The non-GEMM pieces of a transformer block on the quantized path:
// LayerNorm over the last axis (Enilnets/nn/forward.py:207-254), the residual
// add (forward.py:762-766) and the softmax attention core between the
// projections of the multi-head attention layer (forward.py:423-436,525-549).
//
// attention_kernel: one workgroup per (64 queries, head, batch), four waves
// of 16 queries.  Each 64-key block of K and V is staged in LDS; a wave forms
// S^T = K . Q^T (keys x queries) with fp32 MFMA 16x16x4, so every lane owns
// one query's column and the softmax statistics are per lane; masks,
// running max and the rescale follow; then O^T += V^T . P^T reuses the score
// registers directly as the B operand.  Everything is fp32: products are
// exact fp32 products, sums fp32.  attention_bf16_kernel (head_dim 32, 64,
// 128) keeps that layout on the bf16 matrix cores: every operand split into
// three bf16 parts, six part products per product.
#include <algorithm>
#include <cmath>

#include "common.hpp"
#include "mfma.hpp"

namespace enq {
namespace {

// ---------------------------------------------------------------------------
// LayerNorm: y = gamma * (x - mean) / sqrt(var + eps) + beta per row, with the
// mean and the (biased) variance of the row, two passes over values held in
// registers.  One 256-thread workgroup per row; PER values per thread.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float block_sum256(float v, float* red) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  __syncthreads();  // red may still be read from the previous reduction
  if (lane == 0) red[wave] = v;
  __syncthreads();
  return (red[0] + red[1]) + (red[2] + red[3]);
}

template <int PER>
__global__ __launch_bounds__(256) void layernorm_kernel(const float* __restrict__ x, int64_t cols,
                                                        const float* __restrict__ gamma,
                                                        const float* __restrict__ beta, float eps,
                                                        float* __restrict__ y) {
  __shared__ float red[4];
  const float* xr = x + int64_t(blockIdx.x) * cols;
  float* yr = y + int64_t(blockIdx.x) * cols;
  // the row, gamma and beta are all loaded up front from in-bounds
  // addresses and masked afterwards, so the loads are in flight together
  // (loads inside the guarded store blocks were each waited on in turn)
  float v[PER], gm[PER], bt[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int64_t c = int64_t(i) * 256 + threadIdx.x;
    const int64_t cc = c < cols ? c : 0;
    v[i] = xr[cc];
    gm[i] = gamma[cc];
    bt[i] = beta[cc];
  }
  float s = 0.0f;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int64_t c = int64_t(i) * 256 + threadIdx.x;
    v[i] = c < cols ? v[i] : 0.0f;
    s += v[i];
  }
  const float mean = block_sum256(s, red) / float(cols);
  float q = 0.0f;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int64_t c = int64_t(i) * 256 + threadIdx.x;
    const float dlt = c < cols ? v[i] - mean : 0.0f;
    q += dlt * dlt;
  }
  const float var = block_sum256(q, red) / float(cols);
  const float den = sqrtf(var + eps);
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int64_t c = int64_t(i) * 256 + threadIdx.x;
    if (c < cols) yr[c] = gm[i] * ((v[i] - mean) / den) + bt[i];
  }
}

// One wave per row, four rows per workgroup, for 16-byte aligned rows of at
// most 64 * 4 * PER4 floats: float4 loads and reductions by wave shuffles
// alone, with no workgroup barrier between the loads and the stores.
template <int PER4>
__global__ __launch_bounds__(256) void layernorm_wave_kernel(
    const float* __restrict__ x, int64_t rows, int64_t cols, const float* __restrict__ gamma,
    const float* __restrict__ beta, float eps, float* __restrict__ y) {
  const int lane = threadIdx.x & 63;
  const int64_t row = int64_t(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;  // a whole wave
  const int64_t nvec = cols / 4;
  const float4* xr = reinterpret_cast<const float4*>(x + row * cols);
  const float4* g4 = reinterpret_cast<const float4*>(gamma);
  const float4* b4 = reinterpret_cast<const float4*>(beta);
  float4* yr = reinterpret_cast<float4*>(y + row * cols);
  // every load from an in-bounds address, masked where it is used
  float4 v[PER4], gm[PER4], bt[PER4];
#pragma unroll
  for (int i = 0; i < PER4; ++i) {
    const int64_t c = int64_t(i) * 64 + lane;
    const int64_t cc = c < nvec ? c : 0;
    v[i] = xr[cc];
    gm[i] = g4[cc];
    bt[i] = b4[cc];
  }
  float s = 0.0f;
#pragma unroll
  for (int i = 0; i < PER4; ++i) {
    const bool live = int64_t(i) * 64 + lane < nvec;
    s += live ? (v[i].x + v[i].y) + (v[i].z + v[i].w) : 0.0f;
  }
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) s += __shfl_xor(s, m, 64);
  const float mean = s / float(cols);
  float q = 0.0f;
#pragma unroll
  for (int i = 0; i < PER4; ++i) {
    const bool live = int64_t(i) * 64 + lane < nvec;
    const float a = v[i].x - mean, b = v[i].y - mean, c = v[i].z - mean, d = v[i].w - mean;
    q += live ? (a * a + b * b) + (c * c + d * d) : 0.0f;
  }
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) q += __shfl_xor(q, m, 64);
  const float den = sqrtf(q / float(cols) + eps);
#pragma unroll
  for (int i = 0; i < PER4; ++i) {
    const int64_t c = int64_t(i) * 64 + lane;
    if (c < nvec) {
      float4 o;
      o.x = gm[i].x * ((v[i].x - mean) / den) + bt[i].x;
      o.y = gm[i].y * ((v[i].y - mean) / den) + bt[i].y;
      o.z = gm[i].z * ((v[i].z - mean) / den) + bt[i].z;
      o.w = gm[i].w * ((v[i].w - mean) / den) + bt[i].w;
      yr[c] = o;
    }
  }
}

// Rows longer than 256 * 16: the same arithmetic, re-reading the row.
__global__ __launch_bounds__(256) void layernorm_long_kernel(const float* __restrict__ x,
                                                             int64_t cols,
                                                             const float* __restrict__ gamma,
                                                             const float* __restrict__ beta,
                                                             float eps, float* __restrict__ y) {
  __shared__ float red[4];
  const float* xr = x + int64_t(blockIdx.x) * cols;
  float* yr = y + int64_t(blockIdx.x) * cols;
  float s = 0.0f;
  for (int64_t c = threadIdx.x; c < cols; c += 256) s += xr[c];
  const float mean = block_sum256(s, red) / float(cols);
  float q = 0.0f;
  for (int64_t c = threadIdx.x; c < cols; c += 256) {
    const float dlt = xr[c] - mean;
    q += dlt * dlt;
  }
  const float den = sqrtf(block_sum256(q, red) / float(cols) + eps);
  for (int64_t c = threadIdx.x; c < cols; c += 256)
    yr[c] = gamma[c] * ((xr[c] - mean) / den) + beta[c];
}

__global__ __launch_bounds__(256) void add_kernel(const float* __restrict__ a,
                                                  const float* __restrict__ b, int64_t n,
                                                  float* __restrict__ y) {
  const int64_t i4 = (int64_t(blockIdx.x) * 256 + threadIdx.x) * 4;
  if (i4 + 4 <= n) {
    const float4 p = *reinterpret_cast<const float4*>(a + i4);
    const float4 q = *reinterpret_cast<const float4*>(b + i4);
    *reinterpret_cast<float4*>(y + i4) = make_float4(p.x + q.x, p.y + q.y, p.z + q.z, p.w + q.w);
  } else {
    for (int64_t i = i4; i < n; ++i) y[i] = a[i] + b[i];
  }
}

// y[o, i] = a[o, i] + b[i]: a positional table slice added to every batch row
// block (forward.py:597-603).
__global__ __launch_bounds__(256) void add_bcast_kernel(const float* __restrict__ a,
                                                        const float* __restrict__ b,
                                                        int64_t outer, int64_t inner,
                                                        float* __restrict__ y) {
  for (int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x; i < outer * inner;
       i += int64_t(gridDim.x) * 256)
    y[i] = a[i] + b[i % inner];
}

// Strided row copy, batch by batch: dst row b * dst_bstride + r (pitch
// ld_dst) <- src row b * src_bstride + r (pitch ld_src), `width` values.
// Appends new keys / values to a KV cache and gathers embedding rows
// (rows == nullptr: identity; else src row rows[r]).
__global__ __launch_bounds__(256) void copy_rows_kernel(const float* __restrict__ src,
                                                        int64_t ld_src, int64_t src_bstride,
                                                        const int* __restrict__ rows,
                                                        float* __restrict__ dst, int64_t ld_dst,
                                                        int64_t dst_bstride, int64_t nrows,
                                                        int64_t width, int64_t batch) {
  const int64_t total = batch * nrows * width;
  for (int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x; i < total;
       i += int64_t(gridDim.x) * 256) {
    const int64_t c = i % width, br = i / width;
    const int64_t r = br % nrows, b = br / nrows;
    const int64_t sr = rows ? int64_t(rows[b * nrows + r]) : r;
    dst[(b * dst_bstride + r) * ld_dst + c] = src[(b * src_bstride + sr) * ld_src + c];
  }
}

unsigned stride_grid(int64_t work) {
  return unsigned(std::min<int64_t>(ceil_div(work, 256), int64_t(device_cu_count()) * 32));
}

// ---------------------------------------------------------------------------
// Attention core
// ---------------------------------------------------------------------------
__device__ __forceinline__ floatx4 mfma_16x16x4_f32(float a, float b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// Queries of batch b are rows b * q_bstride + [0, seq_q) of q and out, keys
// and values rows b * kv_bstride + [0, seq_k) of k and v; query i sits at
// absolute position q_pos0 + i and key j at k_pos0 + j (a KV cache's keys
// precede the step's queries).
struct AttnShape {
  int64_t batch, seq_q, seq_k;
  int heads, kv_heads;
  int64_t ldq, ldk, ldv, ldo;  // row strides (elements)
  int64_t q_bstride, kv_bstride;
  int64_t q_pos0, k_pos0;
  float scale;                 // 1 / sqrt(head_dim)
  int causal;
  int64_t window;              // < 0: unbounded
};

constexpr int kAttnQ = 64;   // queries per workgroup (4 waves x 16)
constexpr int kAttnKB = 64;  // keys per LDS block

template <int DH>
__global__ __launch_bounds__(256) void attention_kernel(const float* __restrict__ q,
                                                        const float* __restrict__ k,
                                                        const float* __restrict__ v,
                                                        AttnShape sh, float* __restrict__ out) {
  constexpr int PITCH = DH + 4;     // LDS row pitch (floats): conflict-free reads
  constexpr int DG = DH / 4;        // dims per lane group in the S^T steps
  constexpr int DT = DH / 16;       // 16-dim output tiles
  __shared__ __align__(16) float kt[kAttnKB * PITCH];
  __shared__ __align__(16) float vt[kAttnKB * PITCH];
  __shared__ __align__(16) float ot[4][16 * PITCH];

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int col = lane & 15, grp = lane >> 4;
  const int64_t b = blockIdx.z;
  const int h = blockIdx.y;
  const int kvh = h / (sh.heads / sh.kv_heads);
  const int64_t qblk0 = int64_t(blockIdx.x) * kAttnQ;
  const int64_t qi = qblk0 + wave * 16 + col;  // this lane's query
  const int64_t S = sh.seq_q, SK = sh.seq_k;
  const int64_t qpos = sh.q_pos0 + qi;         // absolute positions
  const float* qb = q + (b * sh.q_bstride) * sh.ldq + int64_t(h) * DH;
  const float* kb = k + (b * sh.kv_bstride) * sh.ldk + int64_t(kvh) * DH;
  const float* vb = v + (b * sh.kv_bstride) * sh.ldv + int64_t(kvh) * DH;

  // Q^T operand: step st of lane group g uses dim g * DG + st.
  float qreg[DG];
  {
    const float* src = qb + (qi < S ? qi : 0) * sh.ldq + grp * DG;
#pragma unroll
    for (int c = 0; c < DG / 4; ++c) {
      const float4 t = qi < S ? *reinterpret_cast<const float4*>(src + 4 * c)
                              : make_float4(0.f, 0.f, 0.f, 0.f);
      qreg[4 * c] = t.x;
      qreg[4 * c + 1] = t.y;
      qreg[4 * c + 2] = t.z;
      qreg[4 * c + 3] = t.w;
    }
  }

  floatx4 o[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t) o[t] = floatx4{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY;  // running max of this lane's query
  float l_part = 0.0f;      // this lane's share of the running sum

  // key blocks that can hold an allowed key for any query of the workgroup
  // (key indices j, positions k_pos0 + j)
  const int64_t q_last = (qblk0 + kAttnQ - 1 < S - 1) ? qblk0 + kAttnQ - 1 : S - 1;
  const int64_t rel_last = sh.q_pos0 + q_last - sh.k_pos0;  // newest query, in key index
  const int64_t rel_first = sh.q_pos0 + qblk0 - sh.k_pos0;  // oldest query, in key index
  int64_t key_end = SK;
  if (sh.causal && rel_last + 1 < key_end) key_end = rel_last + 1;
  if (sh.window >= 0 && rel_last + sh.window + 1 < key_end) key_end = rel_last + sh.window + 1;
  int64_t key_begin = 0;
  if (sh.window >= 0 && rel_first - sh.window > 0) key_begin = rel_first - sh.window;
  if (key_end < 0) key_end = 0;
  const int64_t kb_begin = key_begin / kAttnKB;
  const int64_t kb_end = (key_end + kAttnKB - 1) / kAttnKB;

  for (int64_t blk = kb_begin; blk < kb_end; ++blk) {
    const int64_t key0 = blk * kAttnKB;
    __syncthreads();  // previous block's K/V reads are done
    // stage 64 keys x DH of K and V (float4 per thread per step); rows past
    // the sequence are zero so masked products stay finite
    for (int idx = threadIdx.x; idx < kAttnKB * DH / 4; idx += 256) {
      const int r = idx / (DH / 4), c4 = (idx % (DH / 4)) * 4;
      const int64_t key = key0 + r;
      float4 kv = make_float4(0.f, 0.f, 0.f, 0.f), vv = kv;
      if (key < SK) {
        kv = *reinterpret_cast<const float4*>(kb + key * sh.ldk + c4);
        vv = *reinterpret_cast<const float4*>(vb + key * sh.ldv + c4);
      }
      *reinterpret_cast<float4*>(&kt[r * PITCH + c4]) = kv;
      *reinterpret_cast<float4*>(&vt[r * PITCH + c4]) = vv;
    }
    __syncthreads();

    // S^T: 4 subtiles of 16 keys; lane holds keys 16 ks + 4 grp + i of query qi
    floatx4 s[4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      s[ks] = floatx4{0.f, 0.f, 0.f, 0.f};
      const float* krow = &kt[(ks * 16 + col) * PITCH + grp * DG];
#pragma unroll
      for (int c = 0; c < DG / 4; ++c) {
        const float4 a4 = *reinterpret_cast<const float4*>(krow + 4 * c);
        s[ks] = mfma_16x16x4_f32(a4.x, qreg[4 * c], s[ks]);
        s[ks] = mfma_16x16x4_f32(a4.y, qreg[4 * c + 1], s[ks]);
        s[ks] = mfma_16x16x4_f32(a4.z, qreg[4 * c + 2], s[ks]);
        s[ks] = mfma_16x16x4_f32(a4.w, qreg[4 * c + 3], s[ks]);
      }
    }
    // scale, mask, block max
    float mx = -INFINITY;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int64_t key = key0 + ks * 16 + 4 * grp + i;
        const int64_t kpos = sh.k_pos0 + key;
        bool blocked = key >= SK;
        if (sh.causal) blocked = blocked || kpos > qpos;
        if (sh.window >= 0) {
          const int64_t dlt = qpos - kpos;
          blocked = blocked || (dlt > sh.window || -dlt > sh.window);
        }
        const float val = blocked ? -INFINITY : s[ks][i] * sh.scale;
        s[ks][i] = val;
        mx = fmaxf(mx, val);
      }
    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float m_new = fmaxf(m_run, mx);
    const float m_use = m_new == -INFINITY ? 0.0f : m_new;
    const float alpha = expf(m_run - m_use);
    m_run = m_new;
    float psum = 0.0f;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float p = expf(s[ks][i] - m_use);
        s[ks][i] = p;
        psum += p;
      }
    l_part = l_part * alpha + psum;
#pragma unroll
    for (int t = 0; t < DT; ++t) o[t] *= alpha;

    // O^T += V^T . P^T: step (ks, i) of lane group g is key 16 ks + 4 g + i
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float* vrow = &vt[(ks * 16 + 4 * grp + i) * PITCH + col];
#pragma unroll
        for (int t = 0; t < DT; ++t) o[t] = mfma_16x16x4_f32(vrow[16 * t], s[ks][i], o[t]);
      }
  }

  // total sum over the four lanes of this query; normalise; write through
  // LDS so each query row leaves as contiguous float4 stores
  float l_tot = l_part + __shfl_xor(l_part, 16, 64);
  l_tot = l_tot + __shfl_xor(l_tot, 32, 64);
  float* my = ot[wave];
#pragma unroll
  for (int t = 0; t < DT; ++t)
#pragma unroll
    for (int r = 0; r < 4; ++r) my[col * PITCH + t * 16 + 4 * grp + r] = o[t][r] / l_tot;
  __syncthreads();
  for (int idx = lane; idx < 16 * (DH / 4); idx += 64) {
    const int r = idx / (DH / 4), c4 = (idx % (DH / 4)) * 4;
    const int64_t qq = qblk0 + wave * 16 + r;
    if (qq < S)
      *reinterpret_cast<float4*>(out + (b * sh.q_bstride + qq) * sh.ldo + int64_t(h) * DH + c4) =
          *reinterpret_cast<const float4*>(&my[r * PITCH + c4]);
  }
}

// fp32 x -> bf16 h + m + l with x - h - m - l within about 2^-27 |x| (each
// difference is exact in fp32, each part nearest even).
__device__ __forceinline__ void split3_bf16(float x, uint16_t& h, uint16_t& m, uint16_t& l) {
  h = bf16_bits_rne(x);
  const float r = x - bf16_to_float(h);
  m = bf16_bits_rne(r);
  l = bf16_bits_rne(r - bf16_to_float(m));
}

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// The same for two values at once (one v_cvt_pk_bf16_f32 per part), each
// part returned as a packed pair, a in the low half.
__device__ __forceinline__ void split3_bf16x2(float a, float b, uint32_t& h, uint32_t& m,
                                              uint32_t& l) {
  h = __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{a, b}, bf16x2));
  const float ra = a - __uint_as_float(h << 16), rb = b - __uint_as_float(h & 0xffff0000u);
  m = __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{ra, rb}, bf16x2));
  const float sa = ra - __uint_as_float(m << 16), sb = rb - __uint_as_float(m & 0xffff0000u);
  l = __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{sa, sb}, bf16x2));
}

// Eight values -> their three bf16 parts as MFMA operands.
__device__ __forceinline__ void split3_bf16x8(const float (&x)[8], bf16x8& h, bf16x8& m,
                                              bf16x8& l) {
  uint32_t ph[4], pm[4], pl[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) split3_bf16x2(x[2 * i], x[2 * i + 1], ph[i], pm[i], pl[i]);
  h = __builtin_bit_cast(bf16x8, make_uint4(ph[0], ph[1], ph[2], ph[3]));
  m = __builtin_bit_cast(bf16x8, make_uint4(pm[0], pm[1], pm[2], pm[3]));
  l = __builtin_bit_cast(bf16x8, make_uint4(pl[0], pl[1], pl[2], pl[3]));
}

// a . b to fp32 accuracy from three-part operands: the six products whose
// parts are above 2^-18 of the whole, smallest first into the accumulator.
__device__ __forceinline__ floatx4 mfma6_bf16(bf16x8 ah, bf16x8 am, bf16x8 al, bf16x8 bh,
                                              bf16x8 bm, bf16x8 bl, floatx4 c) {
  c = mfma_16x16x32_bf16(al, bh, c);
  c = mfma_16x16x32_bf16(ah, bl, c);
  c = mfma_16x16x32_bf16(am, bm, c);
  c = mfma_16x16x32_bf16(am, bh, c);
  c = mfma_16x16x32_bf16(ah, bm, c);
  return mfma_16x16x32_bf16(ah, bh, c);
}

// The attention core on the bf16 matrix cores (head_dim 32, 64 or 128).
// Same workgroup, lane and softmax layout as attention_kernel; every fp32
// operand is split into three bf16 parts (x = h + m + l to about 2^-27 |x|)
// and each product takes the six part products above 2^-18 of it, 16x16x32
// bf16 MFMAs: within about 2^-25 of the fp32 product, against 16x16x4 fp32
// MFMAs at a sixteenth of the rate.  K is staged as three bf16 planes
// [key][dim]; V transposed, [dim][key], so that O^T = V^T . P^T takes P^T
// straight from the score registers: a lane of group g holds keys
// 16 ks + 4 g + i of subtiles ks and ks + 1, and reads the same eight keys of
// V^T as two 8-byte runs.  Up to head_dim 64 the registers are held to 128
// so that two 8-wave workgroups share a CU (B8 S512 H16 D64: 75.0 -> 69.8 us;
// holding the next key block's K and V in registers during the products
// does not fit in that budget).
template <int DH, int WAVES>
__global__ __launch_bounds__(64 * WAVES)
__attribute__((amdgpu_waves_per_eu(DH <= 64 ? WAVES / 2 : 1, DH <= 64 ? WAVES / 2 : 2)))
void attention_bf16_kernel(const float* __restrict__ q,
                                                             const float* __restrict__ k,
                                                             const float* __restrict__ v,
                                                             AttnShape sh,
                                                             float* __restrict__ out) {
  constexpr int KP = DH + 8;             // K plane pitch (bf16): conflict-free 16-byte reads
  constexpr int VP = kAttnKB + 4;        // V^T plane pitch (bf16): conflict-free 8-byte reads
  constexpr int K_PLANE = kAttnKB * KP;  // elements per plane
  constexpr int V_PLANE = DH * VP;
  constexpr int ST = DH / 32;            // 32-dim steps of S^T
  constexpr int DT = DH / 16;            // 16-dim output tiles
  constexpr int NT = 64 * WAVES, QB = 16 * WAVES;         // threads, queries per workgroup
  constexpr int KITEMS = kAttnKB * DH / 4 / NT;           // K float4s per thread
  constexpr int VITEMS = (4 * DH + NT - 1) / NT;          // 4 keys x 4 dims V items per thread
  constexpr int OPITCH = DH + 4;                          // output staging pitch (floats)
  static_assert(DH % 32 == 0 && KITEMS >= 1, "head_dim 32, 64 or 128");
  static_assert(WAVES * 16 * OPITCH * 4 <= 3 * (K_PLANE + V_PLANE) * 2,
                "output staging fits the planes");
  extern __shared__ __align__(16) uint16_t attn_lds[];
  uint16_t* kl = attn_lds;                 // 3 planes [key][dim]
  uint16_t* vl = attn_lds + 3 * K_PLANE;   // 3 planes [dim][key]

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int col = lane & 15, grp = lane >> 4;
  const int64_t b = blockIdx.z;
  const int h = blockIdx.y;
  const int kvh = h / (sh.heads / sh.kv_heads);
  const int64_t qblk0 = int64_t(blockIdx.x) * QB;
  const int64_t qi = qblk0 + wave * 16 + col;  // this lane's query
  const int64_t S = sh.seq_q, SK = sh.seq_k;
  const int64_t qpos = sh.q_pos0 + qi;
  const float* qb = q + (b * sh.q_bstride) * sh.ldq + int64_t(h) * DH;
  const float* kb = k + (b * sh.kv_bstride) * sh.ldk + int64_t(kvh) * DH;
  const float* vb = v + (b * sh.kv_bstride) * sh.ldv + int64_t(kvh) * DH;

  // Q^T operand of step st: dims 32 st + 8 grp + [0, 8) of query qi
  bf16x8 qh[ST], qm[ST], ql[ST];
#pragma unroll
  for (int st = 0; st < ST; ++st) {
    float x[8];
    const float* src = qb + (qi < S ? qi : 0) * sh.ldq + st * 32 + 8 * grp;
    const float4 a = *reinterpret_cast<const float4*>(src);
    const float4 c = *reinterpret_cast<const float4*>(src + 4);
    const bool live = qi < S;
    x[0] = live ? a.x : 0.f; x[1] = live ? a.y : 0.f; x[2] = live ? a.z : 0.f; x[3] = live ? a.w : 0.f;
    x[4] = live ? c.x : 0.f; x[5] = live ? c.y : 0.f; x[6] = live ? c.z : 0.f; x[7] = live ? c.w : 0.f;
    split3_bf16x8(x, qh[st], qm[st], ql[st]);
  }

  floatx4 o[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t) o[t] = floatx4{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY;
  float l_part = 0.0f;

  const int64_t q_last = (qblk0 + QB - 1 < S - 1) ? qblk0 + QB - 1 : S - 1;
  const int64_t rel_last = sh.q_pos0 + q_last - sh.k_pos0;
  const int64_t rel_first = sh.q_pos0 + qblk0 - sh.k_pos0;
  int64_t key_end = SK;
  if (sh.causal && rel_last + 1 < key_end) key_end = rel_last + 1;
  if (sh.window >= 0 && rel_last + sh.window + 1 < key_end) key_end = rel_last + sh.window + 1;
  int64_t key_begin = 0;
  if (sh.window >= 0 && rel_first - sh.window > 0) key_begin = rel_first - sh.window;
  if (key_end < 0) key_end = 0;
  const int64_t kb_begin = key_begin / kAttnKB;
  const int64_t kb_end = (key_end + kAttnKB - 1) / kAttnKB;

  // a key block's K (float4 of one key) and V (4 keys x 4 dims) in
  // registers; keys past the sequence read key 0 and are zeroed when staged
  float4 kreg[KITEMS], vreg[VITEMS][4];
  auto load_block = [&](int64_t key0) {
#pragma unroll
    for (int it = 0; it < KITEMS; ++it) {
      const int idx = tid + it * NT, r = idx / (DH / 4), c4 = (idx % (DH / 4)) * 4;
      const int64_t key = key0 + r;
      kreg[it] = *reinterpret_cast<const float4*>(kb + (key < SK ? key : 0) * sh.ldk + c4);
    }
#pragma unroll
    for (int it = 0; it < VITEMS; ++it) {
      const int idx = tid + it * NT;
      const int item = idx < 4 * DH ? idx : 0;
      const int kg = item / (DH / 4), d4 = (item % (DH / 4)) * 4;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int64_t key = key0 + 4 * kg + j;
        vreg[it][j] = *reinterpret_cast<const float4*>(vb + (key < SK ? key : 0) * sh.ldv + d4);
      }
    }
  };
  auto store_block = [&](int64_t key0) {
#pragma unroll
    for (int it = 0; it < KITEMS; ++it) {
      const int idx = tid + it * NT, r = idx / (DH / 4), c4 = (idx % (DH / 4)) * 4;
      const bool live = key0 + r < SK;
      const float4 t = live ? kreg[it] : make_float4(0.f, 0.f, 0.f, 0.f);
      uint32_t h0, m0, l0, h1, m1, l1;
      split3_bf16x2(t.x, t.y, h0, m0, l0);
      split3_bf16x2(t.z, t.w, h1, m1, l1);
      uint16_t* dst = kl + r * KP + c4;
      *reinterpret_cast<uint2*>(dst) = make_uint2(h0, h1);
      *reinterpret_cast<uint2*>(dst + K_PLANE) = make_uint2(m0, m1);
      *reinterpret_cast<uint2*>(dst + 2 * K_PLANE) = make_uint2(l0, l1);
    }
#pragma unroll
    for (int it = 0; it < VITEMS; ++it) {
      const int idx = tid + it * NT;
      if (idx < 4 * DH) {
        const int kg = idx / (DH / 4), d4 = (idx % (DH / 4)) * 4;
        float4 t[4];
#pragma unroll
        for (int j = 0; j < 4; ++j)
          t[j] = key0 + 4 * kg + j < SK ? vreg[it][j] : make_float4(0.f, 0.f, 0.f, 0.f);
        const float x[4][4] = {{t[0].x, t[1].x, t[2].x, t[3].x}, {t[0].y, t[1].y, t[2].y, t[3].y},
                               {t[0].z, t[1].z, t[2].z, t[3].z}, {t[0].w, t[1].w, t[2].w, t[3].w}};
#pragma unroll
        for (int dd = 0; dd < 4; ++dd) {
          uint32_t h0, m0, l0, h1, m1, l1;
          split3_bf16x2(x[dd][0], x[dd][1], h0, m0, l0);
          split3_bf16x2(x[dd][2], x[dd][3], h1, m1, l1);
          uint16_t* dst = vl + (d4 + dd) * VP + 4 * kg;
          *reinterpret_cast<uint2*>(dst) = make_uint2(h0, h1);
          *reinterpret_cast<uint2*>(dst + V_PLANE) = make_uint2(m0, m1);
          *reinterpret_cast<uint2*>(dst + 2 * V_PLANE) = make_uint2(l0, l1);
        }
      }
    }
  };

  for (int64_t blk = kb_begin; blk < kb_end; ++blk) {
    const int64_t key0 = blk * kAttnKB;
    load_block(key0);
    __syncthreads();  // the previous block's planes are no longer read
    store_block(key0);
    __syncthreads();

    // S^T: 4 subtiles of 16 keys; lane holds keys 16 ks + 4 grp + i of query qi
    floatx4 s[4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      s[ks] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int st = 0; st < ST; ++st) {
        const uint16_t* kr = kl + (ks * 16 + col) * KP + st * 32 + 8 * grp;
        const bf16x8 ah = *reinterpret_cast<const bf16x8*>(kr);
        const bf16x8 am = *reinterpret_cast<const bf16x8*>(kr + K_PLANE);
        const bf16x8 al = *reinterpret_cast<const bf16x8*>(kr + 2 * K_PLANE);
        s[ks] = mfma6_bf16(ah, am, al, qh[st], qm[st], ql[st], s[ks]);
      }
    }
    // scale (into log2 units), mask, block max.  Key 16 ks + 4 grp + i of
    // the block is allowed for this lane's query iff it lies in [jlo, jhi)
    // (the sequence end, causality and the window as bounds on the key
    // index); a wave whose queries all see the whole block skips the masks.
    const int64_t rel = qpos - sh.k_pos0 - key0;  // the query's position as a key index
    int64_t jhi = SK - key0, jlo = 0;
    if (sh.causal && rel + 1 < jhi) jhi = rel + 1;
    if (sh.window >= 0) {
      if (rel + sh.window + 1 < jhi) jhi = rel + sh.window + 1;
      if (rel - sh.window > jlo) jlo = rel - sh.window;
    }
    const int lo32 = int(jlo < kAttnKB ? jlo : kAttnKB) - 4 * grp;
    const int hi32 = int(jhi > 0 ? (jhi < kAttnKB ? jhi : kAttnKB) : 0) - 4 * grp;
    const float sc = sh.scale * 1.44269504088896341f;  // log2(e)
    float mx = -INFINITY;
    if (__all(lo32 <= -4 * grp && hi32 >= kAttnKB - 4 * grp)) {
#pragma unroll
      for (int ks = 0; ks < 4; ++ks)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          s[ks][i] *= sc;
          mx = fmaxf(mx, s[ks][i]);
        }
    } else {
#pragma unroll
      for (int ks = 0; ks < 4; ++ks)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int c = ks * 16 + i;
          const float val = (c >= lo32 && c < hi32) ? s[ks][i] * sc : -INFINITY;
          s[ks][i] = val;
          mx = fmaxf(mx, val);
        }
    }
    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float m_new = fmaxf(m_run, mx);
    const float m_use = m_new == -INFINITY ? 0.0f : m_new;
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_use);
    m_run = m_new;
    float psum = 0.0f;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float p = __builtin_amdgcn_exp2f(s[ks][i] - m_use);
        s[ks][i] = p;
        psum += p;
      }
    l_part = l_part * alpha + psum;
#pragma unroll
    for (int t = 0; t < DT; ++t) o[t] *= alpha;

    // O^T += V^T . P^T over two 32-key steps
#pragma unroll
    for (int kp = 0; kp < 2; ++kp) {
      const float pv[8] = {s[2 * kp][0], s[2 * kp][1], s[2 * kp][2], s[2 * kp][3],
                           s[2 * kp + 1][0], s[2 * kp + 1][1], s[2 * kp + 1][2], s[2 * kp + 1][3]};
      bf16x8 ph, pm, pl;
      split3_bf16x8(pv, ph, pm, pl);
#pragma unroll
      for (int t = 0; t < DT; ++t) {
        const uint16_t* vr = vl + (16 * t + col) * VP + 32 * kp + 4 * grp;
        bf16x8 a[3];
#pragma unroll
        for (int pl3 = 0; pl3 < 3; ++pl3) {
          const uint2 lo = *reinterpret_cast<const uint2*>(vr + pl3 * V_PLANE);
          const uint2 hi = *reinterpret_cast<const uint2*>(vr + pl3 * V_PLANE + 16);
          a[pl3] = __builtin_bit_cast(bf16x8, make_uint4(lo.x, lo.y, hi.x, hi.y));
        }
        o[t] = mfma6_bf16(a[0], a[1], a[2], ph, pm, pl, o[t]);
      }
    }
  }

  // total sum over the four lanes of this query; normalise; write through
  // LDS (the K planes, no longer read) so each query row leaves as float4s
  float l_tot = l_part + __shfl_xor(l_part, 16, 64);
  l_tot = l_tot + __shfl_xor(l_tot, 32, 64);
  __syncthreads();
  float* my = reinterpret_cast<float*>(attn_lds) + wave * 16 * OPITCH;
#pragma unroll
  for (int t = 0; t < DT; ++t)
#pragma unroll
    for (int r = 0; r < 4; ++r) my[col * OPITCH + t * 16 + 4 * grp + r] = o[t][r] / l_tot;
  __syncthreads();
  for (int idx = lane; idx < 16 * (DH / 4); idx += 64) {
    const int r = idx / (DH / 4), c4 = (idx % (DH / 4)) * 4;
    const int64_t qq = qblk0 + wave * 16 + r;
    if (qq < S)
      *reinterpret_cast<float4*>(out + (b * sh.q_bstride + qq) * sh.ldo + int64_t(h) * DH + c4) =
          *reinterpret_cast<const float4*>(&my[r * OPITCH + c4]);
  }
}

// 8 waves (128 queries) per workgroup: each staged K / V block serves twice
// the queries of the fp32 kernel's 64 (B8 S512 H16 D64: 88.6 -> 77 us); 4
// waves when there are at most 64 queries (decode steps)
template <int DH, int WAVES>
void launch_attention_bf16_waves(const float* q, const float* k, const float* v,
                                 const AttnShape& sh, float* out) {
  constexpr size_t lds = size_t(3) * (kAttnKB * (DH + 8) + DH * (kAttnKB + 4)) * sizeof(uint16_t);
  auto kernel = attention_bf16_kernel<DH, WAVES>;
  static bool attr_set = false;
  if (!attr_set) {
    ENQ_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                hipFuncAttributeMaxDynamicSharedMemorySize, int(lds)));
    attr_set = true;
  }
  const dim3 grid(unsigned(ceil_div(sh.seq_q, int64_t(16 * WAVES))), unsigned(sh.heads),
                  unsigned(sh.batch));
  kernel<<<grid, 64 * WAVES, lds, stream()>>>(q, k, v, sh, out);
}

template <int DH>
void launch_attention_bf16(const float* q, const float* k, const float* v, const AttnShape& sh,
                           float* out) {
  if (sh.seq_q <= 64)
    launch_attention_bf16_waves<DH, 4>(q, k, v, sh, out);
  else
    launch_attention_bf16_waves<DH, 8>(q, k, v, sh, out);
}

// Decode steps (a few queries over a KV cache): one workgroup per query and
// head.  For one query the allowed keys are one range [jlo, jhi) (sequence
// end, causality, window); each wave takes a contiguous part of it.  A lane
// holds four dims of the query; LPK = DH / 4 lanes hold one key row, so one
// 16-byte load per lane reads KPI = 64 / LPK key rows.  Each batch issues
// all its K and V loads before any arithmetic, then the fp32 scores (dot
// product over the key's LPK lanes), an online softmax in log2 units and
// the weighted V rows.  The (max, sum, output) triples then merge across
// the wave's key slots and across the waves.  No LDS staging, no barrier
// per key block: the K and V rows are read once, straight into registers.
template <int DH, int WAVES, int ITB>
__global__ __launch_bounds__(64 * WAVES) void attention_decode_kernel(
    const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
    AttnShape sh, float* __restrict__ out) {
  constexpr int LPK = DH / 4, KPI = 64 / LPK;
  __shared__ float s_m[WAVES], s_l[WAVES];
  __shared__ __align__(16) float s_o[WAVES][DH];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int slot = lane / LPK, d4 = (lane % LPK) * 4;
  const int64_t qi = blockIdx.x, b = blockIdx.z;
  const int h = blockIdx.y;
  const int kvh = h / (sh.heads / sh.kv_heads);
  const int64_t SK = sh.seq_k;
  const float* kb = k + (b * sh.kv_bstride) * sh.ldk + int64_t(kvh) * DH + d4;
  const float* vb = v + (b * sh.kv_bstride) * sh.ldv + int64_t(kvh) * DH + d4;
  const float4 qv =
      *reinterpret_cast<const float4*>(q + (b * sh.q_bstride + qi) * sh.ldq + int64_t(h) * DH + d4);

  const int64_t rel = sh.q_pos0 + qi - sh.k_pos0;  // the query's position as a key index
  int64_t jhi = SK, jlo = 0;
  if (sh.causal && rel + 1 < jhi) jhi = rel + 1;
  if (sh.window >= 0) {
    if (rel + sh.window + 1 < jhi) jhi = rel + sh.window + 1;
    if (rel - sh.window > jlo) jlo = rel - sh.window;
  }
  const int64_t nk = jhi > jlo ? jhi - jlo : 0;
  const int64_t chunk = (nk + WAVES * KPI - 1) / (WAVES * KPI) * KPI;
  const int64_t wb = jlo + wave * chunk;
  const int64_t we = wb + chunk < jhi ? wb + chunk : jhi;
  const int64_t nit = we > wb ? (we - wb + KPI - 1) / KPI : 0;  // wave-uniform

  const float sc = sh.scale * 1.44269504088896341f;  // log2(e)
  float m_run = -INFINITY, l = 0.0f;
  float o[4] = {0.f, 0.f, 0.f, 0.f};
  for (int64_t it0 = 0; it0 < nit; it0 += ITB) {
    float4 kr[ITB], vr[ITB];
#pragma unroll
    for (int it = 0; it < ITB; ++it) {
      const int64_t j = wb + (it0 + it) * KPI + slot;
      const int64_t jc = j < we ? j : we - 1;  // in [wb, we): we > wb here
      kr[it] = *reinterpret_cast<const float4*>(kb + jc * sh.ldk);
    }
#pragma unroll
    for (int it = 0; it < ITB; ++it) {
      const int64_t j = wb + (it0 + it) * KPI + slot;
      const int64_t jc = j < we ? j : we - 1;
      vr[it] = *reinterpret_cast<const float4*>(vb + jc * sh.ldv);
    }
    float s[ITB];
    float mx = -INFINITY;
#pragma unroll
    for (int it = 0; it < ITB; ++it) {
      float d = qv.x * kr[it].x;
      d = fmaf(qv.y, kr[it].y, d);
      d = fmaf(qv.z, kr[it].z, d);
      d = fmaf(qv.w, kr[it].w, d);
#pragma unroll
      for (int m = 1; m < LPK; m <<= 1) d += __shfl_xor(d, m, 64);
      const int64_t j = wb + (it0 + it) * KPI + slot;
      s[it] = j < we ? d * sc : -INFINITY;
      mx = fmaxf(mx, s[it]);
    }
    const float m_new = fmaxf(m_run, mx);
    const float m_use = m_new == -INFINITY ? 0.0f : m_new;
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_use);
    m_run = m_new;
    l *= alpha;
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] *= alpha;
#pragma unroll
    for (int it = 0; it < ITB; ++it) {
      const float p = __builtin_amdgcn_exp2f(s[it] - m_use);
      l += p;
      o[0] = fmaf(p, vr[it].x, o[0]);
      o[1] = fmaf(p, vr[it].y, o[1]);
      o[2] = fmaf(p, vr[it].z, o[2]);
      o[3] = fmaf(p, vr[it].w, o[3]);
    }
  }
  // merge (m, l, o) of (m2, l2, o2) into this lane's triple
  auto merge = [&](float m2, float l2, const float* o2) {
    const float m_new = fmaxf(m_run, m2);
    const float m_use = m_new == -INFINITY ? 0.0f : m_new;
    const float a1 = __builtin_amdgcn_exp2f(m_run - m_use);
    const float a2 = __builtin_amdgcn_exp2f(m2 - m_use);
    m_run = m_new;
    l = l * a1 + l2 * a2;
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] = o[e] * a1 + o2[e] * a2;
  };
#pragma unroll
  for (int off = LPK; off < 64; off <<= 1) {
    const float m2 = __shfl_xor(m_run, off, 64), l2 = __shfl_xor(l, off, 64);
    float o2[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) o2[e] = __shfl_xor(o[e], off, 64);
    merge(m2, l2, o2);
  }
  if (lane < LPK) {
    *reinterpret_cast<float4*>(&s_o[wave][d4]) = make_float4(o[0], o[1], o[2], o[3]);
    if (lane == 0) {
      s_m[wave] = m_run;
      s_l[wave] = l;
    }
  }
  __syncthreads();
  if (wave == 0 && lane < LPK) {
#pragma unroll
    for (int w = 1; w < WAVES; ++w) {
      const float4 t = *reinterpret_cast<const float4*>(&s_o[w][d4]);
      const float o2[4] = {t.x, t.y, t.z, t.w};
      merge(s_m[w], s_l[w], o2);
    }
    // no allowed key: 0 / 0, as the blocked kernels give
    *reinterpret_cast<float4*>(out + (b * sh.q_bstride + qi) * sh.ldo + int64_t(h) * DH + d4) =
        make_float4(o[0] / l, o[1] / l, o[2] / l, o[3] / l);
  }
}

constexpr int kDecodeMaxQ = 8;  // queries per step taken by the decode kernel

template <int DH>
void launch_attention_decode(const float* q, const float* k, const float* v, const AttnShape& sh,
                             float* out) {
  const dim3 grid(unsigned(sh.seq_q), unsigned(sh.heads), unsigned(sh.batch));
  attention_decode_kernel<DH, 16, 12><<<grid, 1024, 0, stream()>>>(q, k, v, sh, out);
}

void attention(const float* q, const float* k, const float* v, const AttnShape& sh, int head_dim,
               float* out) {
  if (sh.seq_q <= kDecodeMaxQ) {
    switch (head_dim) {
      case 16: launch_attention_decode<16>(q, k, v, sh, out); break;
      case 32: launch_attention_decode<32>(q, k, v, sh, out); break;
      case 64: launch_attention_decode<64>(q, k, v, sh, out); break;
      case 128: launch_attention_decode<128>(q, k, v, sh, out); break;
      default:
        fail(ENQ_ERR_UNSUPPORTED, "attention head_dim %d is not one of 16, 32, 64, 128",
             head_dim);
    }
    check_launch("attention_decode_kernel");
    return;
  }
  const dim3 grid(unsigned(ceil_div(sh.seq_q, kAttnQ)), unsigned(sh.heads), unsigned(sh.batch));
  switch (head_dim) {
    case 16:
      attention_kernel<16><<<grid, 256, 0, stream()>>>(q, k, v, sh, out);
      break;
    case 32:
      launch_attention_bf16<32>(q, k, v, sh, out);
      break;
    case 64:
      launch_attention_bf16<64>(q, k, v, sh, out);
      break;
    case 128:
      launch_attention_bf16<128>(q, k, v, sh, out);
      break;
    default:
      fail(ENQ_ERR_UNSUPPORTED, "attention head_dim %d is not one of 16, 32, 64, 128", head_dim);
  }
  check_launch("attention_kernel");
}

}  // namespace
}  // namespace enq

using namespace enq;

extern "C" int enq_layernorm(const float* x, int64_t rows, int64_t cols, const float* gamma,
                             const float* beta, float eps, float* y) {
  return guarded([&] {
    require_init();
    ENQ_REQUIRE(rows >= 1 && cols >= 1, "rows and cols must be positive");
    ENQ_REQUIRE(x && gamma && beta && y, "NULL pointer argument");
    ENQ_REQUIRE(rows <= 0x7fffffff, "too many rows");
    const unsigned grid = unsigned(rows);
    hipStream_t s = stream();
    const bool vec = cols % 4 == 0 && aligned(x, 16) && aligned(gamma, 16) &&
                     aligned(beta, 16) && aligned(y, 16);
    if (vec && cols <= 64 * 4 * 8) {
      const unsigned g4 = unsigned(ceil_div(rows, int64_t(4)));
      if (cols <= 64 * 4 * 1)
        layernorm_wave_kernel<1><<<g4, 256, 0, s>>>(x, rows, cols, gamma, beta, eps, y);
      else if (cols <= 64 * 4 * 2)
        layernorm_wave_kernel<2><<<g4, 256, 0, s>>>(x, rows, cols, gamma, beta, eps, y);
      else if (cols <= 64 * 4 * 4)
        layernorm_wave_kernel<4><<<g4, 256, 0, s>>>(x, rows, cols, gamma, beta, eps, y);
      else
        layernorm_wave_kernel<8><<<g4, 256, 0, s>>>(x, rows, cols, gamma, beta, eps, y);
    } else if (cols <= 256 * 1)
      layernorm_kernel<1><<<grid, 256, 0, s>>>(x, cols, gamma, beta, eps, y);
    else if (cols <= 256 * 2)
      layernorm_kernel<2><<<grid, 256, 0, s>>>(x, cols, gamma, beta, eps, y);
    else if (cols <= 256 * 4)
      layernorm_kernel<4><<<grid, 256, 0, s>>>(x, cols, gamma, beta, eps, y);
    else if (cols <= 256 * 8)
      layernorm_kernel<8><<<grid, 256, 0, s>>>(x, cols, gamma, beta, eps, y);
    else if (cols <= 256 * 16)
      layernorm_kernel<16><<<grid, 256, 0, s>>>(x, cols, gamma, beta, eps, y);
    else
      layernorm_long_kernel<<<grid, 256, 0, s>>>(x, cols, gamma, beta, eps, y);
    check_launch("layernorm_kernel");
  });
}

extern "C" int enq_add(const float* a, const float* b, int64_t n, float* y) {
  return guarded([&] {
    require_init();
    ENQ_REQUIRE(n >= 0, "n must be non-negative");
    if (n == 0) return;
    ENQ_REQUIRE(a && b && y, "NULL pointer argument");
    ENQ_REQUIRE(aligned(a, 16) && aligned(b, 16) && aligned(y, 16),
                "enq_add needs 16-byte aligned buffers");
    const int64_t blocks = ceil_div(ceil_div(n, 4), 256);
    ENQ_REQUIRE(blocks <= 0x7fffffff, "problem too large");
    add_kernel<<<unsigned(blocks), 256, 0, stream()>>>(a, b, n, y);
    check_launch("add_kernel");
  });
}

namespace {

void check_attention(const float* q, int64_t ldq, const float* k, int64_t ldk, const float* v,
                     int64_t ldv, int64_t batch, int heads, int kv_heads, int head_dim,
                     const float* out, int64_t ldo) {
  ENQ_REQUIRE(batch >= 1 && heads >= 1 && kv_heads >= 1,
              "batch, heads and kv_heads must be positive");
  ENQ_REQUIRE(heads % kv_heads == 0, "heads (%d) must be a multiple of kv_heads (%d)", heads,
              kv_heads);
  ENQ_REQUIRE(q && k && v && out, "NULL pointer argument");
  ENQ_REQUIRE(batch <= 65535 && heads <= 65535, "problem too large");
  ENQ_REQUIRE(ldq >= int64_t(heads) * head_dim && ldo >= int64_t(heads) * head_dim &&
                  ldk >= int64_t(kv_heads) * head_dim && ldv >= int64_t(kv_heads) * head_dim,
              "row strides smaller than the heads they hold");
  ENQ_REQUIRE(ldq % 4 == 0 && ldk % 4 == 0 && ldv % 4 == 0 && ldo % 4 == 0 && aligned(q, 16) &&
                  aligned(k, 16) && aligned(v, 16) && aligned(out, 16),
              "attention needs 16-byte aligned rows");
}

}  // namespace

extern "C" int enq_attention(const float* q, int64_t ldq, const float* k, int64_t ldk,
                             const float* v, int64_t ldv, int64_t batch, int64_t seq, int heads,
                             int kv_heads, int head_dim, int causal, int64_t window, float* out,
                             int64_t ldo) {
  return guarded([&] {
    require_init();
    ENQ_REQUIRE(seq >= 1, "seq must be positive");
    check_attention(q, ldq, k, ldk, v, ldv, batch, heads, kv_heads, head_dim, out, ldo);
    ENQ_REQUIRE(ceil_div(seq, kAttnQ) <= 0x7fffffff, "problem too large");
    AttnShape sh{batch, seq, seq, heads, kv_heads, ldq, ldk, ldv, ldo, seq, seq, 0, 0,
                 float(1.0 / std::sqrt(double(head_dim))), causal ? 1 : 0, window};
    attention(q, k, v, sh, head_dim, out);
  });
}

extern "C" int enq_attention_kv(const float* q, int64_t ldq, int64_t q_bstride, int64_t seq_q,
                                int64_t q_pos0, const float* k, int64_t ldk, const float* v,
                                int64_t ldv, int64_t kv_bstride, int64_t seq_k, int64_t k_pos0,
                                int64_t batch, int heads, int kv_heads, int head_dim, int causal,
                                int64_t window, float* out, int64_t ldo) {
  return guarded([&] {
    require_init();
    ENQ_REQUIRE(seq_q >= 1 && seq_k >= 1, "seq_q and seq_k must be positive");
    ENQ_REQUIRE(q_bstride >= seq_q && kv_bstride >= seq_k, "batch strides below the lengths");
    check_attention(q, ldq, k, ldk, v, ldv, batch, heads, kv_heads, head_dim, out, ldo);
    ENQ_REQUIRE(ceil_div(seq_q, kAttnQ) <= 0x7fffffff, "problem too large");
    AttnShape sh{batch, seq_q, seq_k, heads, kv_heads, ldq, ldk, ldv, ldo, q_bstride, kv_bstride,
                 q_pos0, k_pos0, float(1.0 / std::sqrt(double(head_dim))), causal ? 1 : 0,
                 window};
    attention(q, k, v, sh, head_dim, out);
  });
}

extern "C" int enq_add_bcast(const float* a, const float* b, int64_t outer, int64_t inner,
                             float* y) {
  return guarded([&] {
    require_init();
    ENQ_REQUIRE(outer >= 0 && inner >= 1, "bad shape");
    if (outer == 0) return;
    ENQ_REQUIRE(a && b && y, "NULL pointer argument");
    add_bcast_kernel<<<stride_grid(outer * inner), 256, 0, stream()>>>(a, b, outer, inner, y);
    check_launch("add_bcast_kernel");
  });
}

extern "C" int enq_copy_rows(const float* src, int64_t ld_src, int64_t src_bstride,
                             const int32_t* rows, float* dst, int64_t ld_dst,
                             int64_t dst_bstride, int64_t nrows, int64_t width, int64_t batch) {
  return guarded([&] {
    require_init();
    ENQ_REQUIRE(nrows >= 0 && width >= 0 && batch >= 0, "bad shape");
    if (nrows == 0 || width == 0 || batch == 0) return;
    ENQ_REQUIRE(src && dst, "NULL pointer argument");
    ENQ_REQUIRE(ld_src >= width && ld_dst >= width, "row pitch below the width");
    copy_rows_kernel<<<stride_grid(batch * nrows * width), 256, 0, stream()>>>(
        src, ld_src, src_bstride, rows, dst, ld_dst, dst_bstride, nrows, width, batch);
    check_launch("copy_rows_kernel");
  });
}
