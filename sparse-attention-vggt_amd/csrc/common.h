// Shared definitions of the gfx950 kernels: geometry of the packed layout, vector types,
// the sortable fp32 key and the thread-local error channel of the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>

#include "saf3r_hip.h"

namespace saf3r {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Work-item and work-group ids read as the hardware registers they are: threadIdx / blockIdx compile
// to out-of-line library calls here (a call with register saves per use).
__device__ __forceinline__ int tid_x() { return (int)__builtin_amdgcn_workitem_id_x(); }
__device__ __forceinline__ int bid_x() { return (int)__builtin_amdgcn_workgroup_id_x(); }
__device__ __forceinline__ int bid_y() { return (int)__builtin_amdgcn_workgroup_id_y(); }
__device__ __forceinline__ int bid_z() { return (int)__builtin_amdgcn_workgroup_id_z(); }

// LDS pointer type of the LDS-DMA loads (__builtin_amdgcn_global_load_lds)
typedef __attribute__((address_space(3))) void lds_void;

// 32-bit LDS address of a __shared__ object
__device__ inline uint32_t lds_addr(const void* p) { return (uint32_t)(uintptr_t)(const lds_void*)p; }

// LDS-DMA load of 16 bytes per lane: lane i's bytes at global src land at LDS lds_base + 16 i
// (lds_base wave-uniform). Written as inline assembly so that the compiler does not see an LDS
// write: after __builtin_amdgcn_global_load_lds it treats every later LDS read of the kernel as
// possibly aliasing the DMA destination and waits for vmcnt(0) before it, which drains a load
// ring every step. The caller orders reads of the destination itself (wait_vm, then a barrier).
// A scalar write of M0 needs a wait state before a global load with LDS destination reads it; the
// compiler writes M0 (the LDS base) just ahead of the statement but its hazard checks do not see
// into it, so the statement starts with the wait states itself.
__device__ inline void dma16(const void* src, uint32_t lds_base) {
  asm volatile("s_nop 1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "{m0}"(lds_base) : "memory");
}
// The same in the scalar-base form: wave-uniform base, per-lane 32-bit byte offset, and an
// immediate IMM that moves the global and the LDS address alike.
template <int IMM = 0>
__device__ inline void dma16s(const void* base, uint32_t off, uint32_t lds_base) {
  asm volatile("s_nop 1\n\tglobal_load_lds_dwordx4 %0, %1 offset:%2" ::"v"(off), "s"(base), "i"(IMM),
               "{m0}"(lds_base)
               : "memory");
}

// s_waitcnt on vmcnt only (gfx9 encoding: vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] | vmcnt_hi[15:14]),
// followed by a compiler barrier so no LDS read is hoisted above it.
template <int N>
__device__ inline void wait_vm() {
  __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
  asm volatile("" ::: "memory");
}

// s_barrier without the workgroup fences of __syncthreads(): those make the compiler wait for
// every outstanding LDS-DMA load (vmcnt(0)) before the barrier, which serialises a load ring. The
// caller waits for what it needs (wait_vm) first; the clobber keeps LDS accesses on their side.
__device__ inline void barrier_only() {
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// XOR swizzles of the 16-byte chunk index. 128-byte rows (8 chunks): rows r and r ^ 8 get
// different masks, so 16 lanes reading 16 consecutive rows at one logical chunk hit 16 distinct
// 16-byte bank groups whether the LDS serves 8 lanes over 32 banks or 16 lanes over 64 banks.
// 64-byte rows (4 chunks) use the analogous mask.
__device__ inline int swz8(int r) { return (r & 7) ^ ((r >> 3) & 1); }
__device__ inline int swz4(int r) { return ((r >> 1) & 3) ^ ((r >> 3) & 1); }

constexpr int kHeadDim = 64;
constexpr int kBlock = 64;
constexpr int kMaxHeads = 64;
// Block means (the pooled rows of the dynamic pattern) sum each feature in groups of kPoolGroup
// consecutive rows, each group in row order from +0.0, then the group sums in group order from +0.0,
// and divide once by the block's population.
constexpr int kPoolGroup = 16;

// ---------------------------------------------------------------------------------------
// Error channel
// ---------------------------------------------------------------------------------------
void set_error(const char* fmt, ...);
int fail(int code, const char* fmt, ...);
// Returns SAF3R_ERR_INJECTED when the environment variable SAF3R_FAULT_INJECT names `entry`
// (or is "all"); used by the error-path tests to force a failure before any launch.
int injected(const char* entry);
int check_launch(const char* what);

// ---------------------------------------------------------------------------------------
// Geometry of one layer in the packed layout
// ---------------------------------------------------------------------------------------
struct Geom {
  int F;      // frames
  int T;      // tokens per frame
  int ns;     // special tokens per frame
  int P;      // patch tokens per frame
  int NBf;    // patch blocks per frame
  int Pp;     // padded patch slots per frame (NBf * 64)
  int S;      // special slots (F * ns)
  int Sp;     // padded special slots
  int nst;    // special tiles (Sp / 64)
  int NT;     // tiles per head (L / 64)
  int64_t L;  // slots per head
  int NBT;    // framed layout: tiles per frame (ceil(T / 64)), frame f at tiles f*NBT .. f*NBT + NBT - 1
};

inline bool make_geom(int F, int T, int ns, Geom* g) {
  if (F <= 0 || T <= 0 || ns < 0 || ns >= T) return false;
  // sizes in 64 bits first: every count kept in 32 bits below must fit
  const int64_t P = (int64_t)T - ns, NBf = (P + kBlock - 1) / kBlock, Pp = NBf * kBlock;
  const int64_t S = (int64_t)F * ns, Sp = (S + kBlock - 1) / kBlock * kBlock;
  const int64_t L = Sp + (int64_t)F * Pp;
  if (Pp > 0x7fffffff || Sp > 0x7fffffff || L / kBlock > 0x7fffffff) return false;
  g->F = F;
  g->T = T;
  g->ns = ns;
  g->P = (int)P;
  g->NBf = (int)NBf;
  g->Pp = (int)Pp;
  g->S = (int)S;
  g->Sp = (int)Sp;
  g->nst = (int)(Sp / kBlock);
  g->L = L;
  g->NT = (int)(L / kBlock);
  g->NBT = (int)(((int64_t)T + kBlock - 1) / kBlock);
  return true;
}

// Framed layout (heads of the frame-relative patterns): frame f's T tokens in token order at slots
// f*NBT*64 .. f*NBT*64 + T - 1, the rest of its NBT tiles zero. It fits the L slots of a head when the
// special tokens fit the padding of the last patch tile (NBT == NBf) or there are no special tokens.
inline bool framed_fits(const Geom& g) { return (int64_t)g.F * g.NBT * kBlock <= g.L; }
__host__ __device__ inline int64_t framed_token(const Geom& g, int64_t slot) {
  const int64_t tp = (int64_t)g.NBT * kBlock, f = slot / tp, t = slot - f * tp;
  return (f < g.F && t < g.T) ? f * g.T + t : -1;
}

// Token index of a packed slot, or -1 for padding.
__host__ __device__ inline int64_t slot_token(const Geom& g, int64_t slot) {
  if (slot < g.Sp) {
    if (slot >= g.S) return -1;
    return (slot / g.ns) * g.T + slot % g.ns;
  }
  int64_t o = slot - g.Sp;
  int64_t f = o / g.Pp, p = o % g.Pp;
  if (p >= g.P) return -1;
  return f * g.T + g.ns + p;
}

// ---------------------------------------------------------------------------------------
// Sortable key: integer order == float order; -0.0 < +0.0; +NaN above +inf, -NaN below -inf.
// ref: saf3r/triton/topk_utils.py:26-29
// ---------------------------------------------------------------------------------------
__host__ __device__ inline uint32_t fkey(float x) {
  // negative: all bits flipped; otherwise the sign bit set (an arithmetic shift spreads the sign)
  const uint32_t b = __builtin_bit_cast(uint32_t, x);
  return b ^ ((uint32_t)((int32_t)b >> 31) | 0x80000000u);
}

// Composite 64-bit key: higher score first, then lower index. Any real candidate is > 0.
__host__ __device__ inline uint64_t ckey(float x, uint32_t idx) {
  return ((uint64_t)fkey(x) << 32) | (uint64_t)(0xFFFFFFFEu - idx);
}
__host__ __device__ inline uint32_t ckey_index(uint64_t c) { return 0xFFFFFFFEu - (uint32_t)(c & 0xFFFFFFFFu); }

// Insert composite key x into a descending list a[0..K), dropping the last entry. Entries equal to
// 0 are empty; real composites are > 0 and pairwise distinct, and x = 0 changes nothing. With a
// sorted, the K comparisons are independent (x > a[t] implies x > a[t+1]) and each slot takes one
// select: the slot above it (x goes higher), x (x goes here) or itself.
template <int K>
__device__ inline void topk_insert(uint64_t (&a)[K], uint64_t x) {
  bool c[K];
#pragma unroll
  for (int t = 0; t < K; ++t) c[t] = x > a[t];
#pragma unroll
  for (int t = K - 1; t > 0; --t) a[t] = c[t - 1] ? a[t - 1] : (c[t] ? x : a[t]);
  a[0] = c[0] ? x : a[0];
}

// Reductions over a whole wave without LDS: DPP within each row of 16 lanes (quad swaps, row
// rotations by 4 and 8), then the row pairs and the halves through v_permlane16_swap /
// v_permlane32_swap. Every lane receives the result.
template <int CTL>
__device__ inline float dpp_mov(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTL, 0xF, 0xF, false));
}

template <typename Op>
__device__ inline float wave_reduce(float x, Op op) {
  x = op(x, dpp_mov<0xB1>(x));   // quad_perm [1, 0, 3, 2]
  x = op(x, dpp_mov<0x4E>(x));   // quad_perm [2, 3, 0, 1]
  x = op(x, dpp_mov<0x124>(x));  // row_ror:4
  x = op(x, dpp_mov<0x128>(x));  // row_ror:8
  const uint32_t u = __builtin_bit_cast(uint32_t, x);
  const auto r16 = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  x = op(__builtin_bit_cast(float, (uint32_t)r16[0]), __builtin_bit_cast(float, (uint32_t)r16[1]));
  const uint32_t v = __builtin_bit_cast(uint32_t, x);
  const auto r32 = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  return op(__builtin_bit_cast(float, (uint32_t)r32[0]), __builtin_bit_cast(float, (uint32_t)r32[1]));
}

// ---------------------------------------------------------------------------------------
// Split record of a pooled row for the matrix-core block scores. A wave holds the row's 64 fp32
// values, one per lane. The row is scaled by 2^s (s chosen so that its largest magnitude lies in
// [2^14, 2^15)) and written as two fp16 parts, x * 2^s = h1 + h2 + r with h1 = fp16(x * 2^s),
// h2 = fp16(x * 2^s - h1) (the difference is exact in fp32) and |r| <= 2^-22 |x * 2^s| in fp16's normal
// range. meta[0] is an upper bound of the row's L2 norm (+inf for a row outside the range the score
// error bound covers: a non-finite value, or a largest magnitude outside [2^-50, 2^50] for a row
// that is not all zero), meta[1] = 2^-s.
// ---------------------------------------------------------------------------------------
__device__ inline void pooled_split_row(float x, int lane, uint16_t* __restrict__ split, float* __restrict__ meta) {
  const float mx = wave_reduce(fabsf(x), [](float a, float b) { return fmaxf(a, b); });
  const float ss = wave_reduce(x * x, [](float a, float b) { return a + b; });
  int e = 0;
  (void)frexpf(mx, &e);  // mx = m * 2^e, m in [0.5, 1)
  const bool zero = mx == 0.f;
  // maxNum drops a NaN, the sum of squares does not: a row with an inf or a NaN has a non-finite ss
  // and is not safe (tested on the bits, so that no NaN assumption of the compiler can drop it)
  const bool safe = ((__builtin_bit_cast(uint32_t, ss) & 0x7F800000u) != 0x7F800000u) &&
                    (zero || (mx >= 0x1p-50f && mx <= 0x1p50f));
  const int sc = zero ? 0 : 15 - e;                            // mx * 2^sc in [2^14, 2^15)
  const float xs = ldexpf(x, sc);
  const _Float16 h1 = (_Float16)xs;
  const _Float16 h2 = (_Float16)(xs - (float)h1);
  split[lane] = __builtin_bit_cast(uint16_t, h1);
  split[64 + lane] = __builtin_bit_cast(uint16_t, h2);
  if (lane == 0) {
    // the fp32 sum of squares and the root are within 2^-17 of the exact norm: 2^-10 covers them
    meta[0] = safe ? sqrtf(ss) * (1.0f + 0x1p-10f) : __builtin_inff();
    meta[1] = ldexpf(1.0f, -sc);
  }
}

__device__ inline float bf16_lo(uint32_t w) { return __builtin_bit_cast(float, w << 16); }
__device__ inline float bf16_hi(uint32_t w) { return __builtin_bit_cast(float, w & 0xFFFF0000u); }

}  // namespace saf3r
