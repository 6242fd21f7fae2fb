// Order statistics of a flat array: the value at position `rank` of the
// array sorted ascending, NaN after every number (NumPy's sort order), found
// by a most-significant-digit radix select.
//
// Each value maps to an unsigned key whose integer order is the sort order:
// positive floats get the sign bit set, negative floats are inverted
// bitwise, NaN takes the largest key.  (-0.0 then precedes +0.0; NumPy
// orders the two as equal, so either may sit at a given rank, and they are
// equal under ==.)  One pass per 8-bit digit, from the top: every workgroup
// histograms the digit of the keys that match the prefix found so far into
// LDS and writes its 256 counts to its own row of a global table (no global
// atomics, so the result does not depend on timing); one workgroup then adds
// the rows up, finds the digit whose cumulative count passes the remaining
// rank, and extends the prefix.  The prefix, its mask and the remaining rank
// live in device memory, so the passes queue on the stream without a host
// round trip.  After the last pass the prefix is the key of the wanted value.
#include <algorithm>

#include "common.hpp"

namespace enq {
namespace {

constexpr int kSelBlock = 256;
constexpr int kSelBins = 256;
constexpr int kSelMaxBlocks = 512;

template <class T> struct KeyOf;
template <> struct KeyOf<float> { using U = uint32_t; };
template <> struct KeyOf<double> { using U = uint64_t; };

template <class T>
__device__ __forceinline__ typename KeyOf<T>::U order_key(T v) {
  using U = typename KeyOf<T>::U;
  constexpr U kSign = U(1) << (sizeof(U) * 8 - 1);
  if (v != v) return ~U(0);
  U b;
  __builtin_memcpy(&b, &v, sizeof(U));
  return (b & kSign) ? ~b : (b | kSign);
}

template <class T>
__device__ __forceinline__ T key_value(typename KeyOf<T>::U k) {
  using U = typename KeyOf<T>::U;
  constexpr U kSign = U(1) << (sizeof(U) * 8 - 1);
  const U b = (k & kSign) ? (k & ~kSign) : ~k;
  T v;
  __builtin_memcpy(&v, &b, sizeof(U));
  return v;
}

// Select state: the key prefix found so far, its mask, and the rank still to
// find among the keys that match the prefix.
template <class U>
struct SelState {
  U prefix;
  U mask;
  int64_t rank;
};

template <class T>
__global__ __launch_bounds__(kSelBlock) void select_init_kernel(
    SelState<typename KeyOf<T>::U>* st, int64_t rank) {
  if (threadIdx.x == 0) {
    st->prefix = 0;
    st->mask = 0;
    st->rank = rank;
  }
}

template <class T>
__global__ __launch_bounds__(kSelBlock) void select_hist_kernel(
    const T* __restrict__ x, int64_t n, const SelState<typename KeyOf<T>::U>* __restrict__ st,
    int shift, uint32_t* __restrict__ table) {
  using U = typename KeyOf<T>::U;
  __shared__ uint32_t hist[kSelBins];
  hist[threadIdx.x] = 0;
  __syncthreads();
  const U prefix = st->prefix, mask = st->mask;
  const int64_t stride = int64_t(gridDim.x) * kSelBlock;
  for (int64_t i = int64_t(blockIdx.x) * kSelBlock + threadIdx.x; i < n; i += stride) {
    const U key = order_key<T>(x[i]);
    if ((key & mask) == prefix) atomicAdd(&hist[unsigned(key >> shift) & 255u], 1u);
  }
  __syncthreads();
  table[int64_t(blockIdx.x) * kSelBins + threadIdx.x] = hist[threadIdx.x];
}

// One workgroup: bin b's total over the table rows, an inclusive scan over
// the bins, and the digit whose range holds the remaining rank.
template <class T>
__global__ __launch_bounds__(kSelBlock) void select_pick_kernel(
    const uint32_t* __restrict__ table, int rows, SelState<typename KeyOf<T>::U>* st,
    int shift) {
  using U = typename KeyOf<T>::U;
  __shared__ int64_t cum[kSelBins];
  const int b = threadIdx.x;
  int64_t total = 0;
  for (int r = 0; r < rows; ++r) total += table[int64_t(r) * kSelBins + b];
  cum[b] = total;
  __syncthreads();
  // Hillis-Steele inclusive scan over the 256 bins
  for (int off = 1; off < kSelBins; off <<= 1) {
    const int64_t add = b >= off ? cum[b - off] : 0;
    __syncthreads();
    cum[b] += add;
    __syncthreads();
  }
  const int64_t rank = st->rank;
  const int64_t before = b > 0 ? cum[b - 1] : 0;
  // exactly one bin has before <= rank < cum[b] (the rank is below the count
  // of matching keys, which is cum[255])
  const bool mine = before <= rank && rank < cum[b];
  __syncthreads();
  if (mine) {
    st->prefix |= U(b) << shift;
    st->mask |= U(255) << shift;
    st->rank = rank - before;
  }
}

template <class T>
__global__ __launch_bounds__(kSelBlock) void select_store_kernel(
    const SelState<typename KeyOf<T>::U>* st, T* out, int i) {
  if (threadIdx.x == 0) out[i] = key_value<T>(st->prefix);
}

template <class T>
void order_stats(const T* x, int64_t n, const int64_t* ranks, int count, T* out) {
  using U = typename KeyOf<T>::U;
  constexpr int kBits = int(sizeof(U)) * 8;
  const int blocks = int(std::min<int64_t>(kSelMaxBlocks, ceil_div(n, int64_t(kSelBlock) * 8)));
  const size_t table_bytes = size_t(blocks) * kSelBins * sizeof(uint32_t);
  const size_t state_off = ceil_div(table_bytes, 256) * 256;
  char* ws = static_cast<char*>(workspace(state_off + sizeof(SelState<U>)));
  auto* table = reinterpret_cast<uint32_t*>(ws);
  auto* st = reinterpret_cast<SelState<U>*>(ws + state_off);
  for (int i = 0; i < count; ++i) {
    select_init_kernel<T><<<1, kSelBlock, 0, stream()>>>(st, ranks[i]);
    check_launch("select_init_kernel");
    for (int shift = kBits - 8; shift >= 0; shift -= 8) {
      select_hist_kernel<T><<<blocks, kSelBlock, 0, stream()>>>(x, n, st, shift, table);
      check_launch("select_hist_kernel");
      select_pick_kernel<T><<<1, kSelBlock, 0, stream()>>>(table, blocks, st, shift);
      check_launch("select_pick_kernel");
    }
    select_store_kernel<T><<<1, kSelBlock, 0, stream()>>>(st, out, i);
    check_launch("select_store_kernel");
  }
}

}  // namespace
}  // namespace enq

using namespace enq;

extern "C" int enq_order_stats(int dtype, const void* x, int64_t n, const int64_t* ranks,
                               int count, void* out) {
  return guarded([&] {
    require_init();
    ENQ_REQUIRE(dtype == ENQ_F32 || dtype == ENQ_F64, "unsupported dtype %d", dtype);
    ENQ_REQUIRE(n >= 1, "n must be positive (n=%lld)", (long long)n);
    ENQ_REQUIRE(count >= 0, "count must not be negative (count=%d)", count);
    ENQ_REQUIRE(x && out && (ranks || count == 0), "NULL pointer argument");
    for (int i = 0; i < count; ++i)
      ENQ_REQUIRE(ranks[i] >= 0 && ranks[i] < n, "rank %lld outside [0, %lld)",
                  (long long)ranks[i], (long long)n);
    if (dtype == ENQ_F32)
      order_stats<float>(static_cast<const float*>(x), n, ranks, count, static_cast<float*>(out));
    else
      order_stats<double>(static_cast<const double*>(x), n, ranks, count,
                          static_cast<double*>(out));
  });
}
