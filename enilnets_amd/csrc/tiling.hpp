// Tile scheduling and LDS staging helpers shared by the GEMM kernels.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace enq {

// Workgroups are dispatched round-robin over the 8 XCDs, each with its own
// L2.  Logical tiles are assigned so that each XCD owns one contiguous run
// of tiles, ordered in groups of `group_m` tile rows: the tiles that run at
// the same time on one XCD then share A row panels and B column panels in
// that XCD's L2.  The mapping is a bijection for any grid size.
__device__ __forceinline__ void xcd_tile(int bid, int tiles_m, int tiles_n, int group_m,
                                         int& tm, int& tn) {
  constexpr int kXcds = 8;
  const int total = tiles_m * tiles_n;
  const int per = total / kXcds, rem = total % kXcds;
  const int xcd = bid % kXcds, local = bid / kXcds;
  const int t = xcd * per + (xcd < rem ? xcd : rem) + local;
  const int group = group_m * tiles_n;
  const int first_m = (t / group) * group_m;
  const int rows = tiles_m - first_m < group_m ? tiles_m - first_m : group_m;
  const int in_group = t % group;
  tm = first_m + in_group % rows;
  tn = in_group / rows;
}

// Rows split into consecutive groups (the tokens routed to each expert),
// each multiplied by its own weight matrix.  Every group is tiled on its own,
// so a tile never straddles two groups.
struct RowGroups {
  const int* offsets = nullptr;  // groups + 1 ascending row offsets (device)
  int groups = 0;
  int64_t w_stride = 0;          // weight elements from one group to the next
  int64_t v_stride = 0;          // scale and bias elements from one group to the next
};

// Group of virtual tile row `tm` and the rows [m0, m_end) of that tile's
// group; -1 past the last group's tiles.  Uniform across a workgroup.
__device__ inline int group_tile(const RowGroups& g, int bm, int tm, int64_t& m0,
                                 int64_t& m_end) {
  int base = 0;
  for (int e = 0; e < g.groups; ++e) {
    const int r0 = g.offsets[e], r1 = g.offsets[e + 1];
    const int t = (r1 - r0 + bm - 1) / bm;
    if (tm < base + t) {
      m0 = r0 + int64_t(tm - base) * bm;
      m_end = r1;
      return e;
    }
    base += t;
  }
  return -1;
}

// s_waitcnt with only the vector-memory counter constrained (gfx9 encoding:
// vmcnt in bits 3:0 and 15:14, expcnt 6:4 and lgkmcnt 11:8 left at "no wait").
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// Waits until at most `later` * per_stage vector-memory operations are in
// flight, for a wave that issues `per_stage` loads per pipeline stage and has
// issued `later` (0 .. MAX) stages after the one it needs.
template <int PER_STAGE, int MAX>
__device__ __forceinline__ void wait_stages_after(int later) {
  if constexpr (MAX == 0) {
    wait_vmcnt<0>();
  } else {
    if (later >= MAX)
      wait_vmcnt<MAX * PER_STAGE>();
    else
      wait_stages_after<PER_STAGE, MAX - 1>(later);
  }
}

__device__ __forceinline__ void wait_lgkmcnt0() {
  __builtin_amdgcn_s_waitcnt(15 | (7 << 4) | (0 << 8) | (3 << 14));
}

// s_waitcnt with only the LDS/scalar counter constrained to <= N.
template <int N>
__device__ __forceinline__ void wait_lgkmcnt() {
  static_assert(N >= 0 && N < 16, "lgkmcnt range");
  __builtin_amdgcn_s_waitcnt(15 | (7 << 4) | (N << 8) | (3 << 14));
}

// Keeps the machine scheduler from moving any instruction across this point.
__device__ __forceinline__ void sched_fence() { __builtin_amdgcn_sched_barrier(0); }

// Keeps every memory access on its side of this point, in the IR passes and
// the machine scheduler alike (sched_fence alone does not stop IR passes from
// sinking loads towards their first use).  Placed after a block of LDS reads,
// it makes all of them issue before the arithmetic that consumes them.
__device__ __forceinline__ void issue_fence() { asm volatile("" ::: "memory"); }

// Workgroup barrier that neither waits for outstanding loads nor lets the
// compiler move memory operations across it.
__device__ __forceinline__ void block_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// LDS byte address of a pointer into shared memory.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return uint32_t(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const void*)(p)));
}

// 16 bytes from global memory straight into LDS (gfx950 global_load_lds_dwordx4).
// LDS destination of lane l is lds_base + 16 * l: one instruction fills 1 KiB;
// lds_base must be uniform across the wave (it goes through M0).
//
// Written as inline assembly on purpose: the compiler's wait-count pass
// treats the intrinsic as an LDS access that may complete out of order, and
// then turns every later partial LDS wait (s_waitcnt lgkmcnt(N)) into a full
// drain, which serialises each MFMA step behind its own fragment reads.  The
// instruction only counts on vmcnt; callers order it with explicit vmcnt
// waits and workgroup barriers before reading the stage it fills.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void dma16(const void* src, uint32_t lds_base) {
  // one wait state between the M0 write and the LDS DMA that reads it
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off"
               :
               : "v"(src), "s"(lds_base)
               : "memory", "m0");
}
// The same with a wave-uniform 64-bit base in SGPRs and a 32-bit per-lane
// byte offset (the instruction's saddr form): one VGPR per source instead of
// two, and no per-lane address arithmetic when the base advances.
__device__ __forceinline__ void dma16_s(uint32_t voff, const void* sbase, uint32_t lds_base) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
               :
               : "v"(voff), "s"(sbase), "s"(lds_base)
               : "memory", "m0");
}
#pragma clang diagnostic pop

// XOR swizzle of the four 16-byte chunks of a 64-byte LDS row: conflict-free
// ds_read_b128 when lanes 0..31 read 32 consecutive rows at one chunk.
__device__ __forceinline__ int swz64(int row, int chunk) { return chunk ^ ((row >> 2) & 3); }

// The same for the two 16-byte halves of a 32-byte LDS row: 16 consecutive
// rows read at one logical half touch every bank once.
__device__ __forceinline__ int swz32(int row, int half) { return half ^ ((row >> 3) & 1); }

// Zero bytes (static storage is zero-initialised): the DMA source for chunks
// past the end of K.  One copy per translation unit.
static __device__ __align__(16) int4 g_zero16[4];

}  // namespace enq
