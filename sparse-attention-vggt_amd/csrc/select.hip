// Block selection of the dynamic pattern: pooled patch-block means, block scores and the
// per-frame (or global) top-k with the sortable-key / lowest-index tie rule.
//
// ref: saf3r/triton/fused_qk_topk.py:73-100 (composite key = sortable fp32 bits << 32 | reversed
//      index, running top-k per frame, frame-major flush in descending order),
//      saf3r/triton/topk_utils.py:26-29 (sortable key), saf3r/patch/wrapper.py:48 (top-k per frame),
//      saf3r/patch/adaptive_block_value.py:16-24 (block mean over the real population).
// Every fp32 result is produced in a fixed operation order (block sums in groups of 16 rows, one
// division, sequential fma), so it is bit-identical to that definition.
#include <algorithm>

#include "common.h"

namespace saf3r {

// ---------------------------------------------------------------------------------------
// Pooling: eight lanes per (head, patch block), each lane owning 8 features (16-byte loads), so a
// wave streams eight blocks at once. Every feature is summed in the block-mean order: groups of
// kPoolGroup rows, each in row order from +0.0, the group sums added in order from +0.0.
// ---------------------------------------------------------------------------------------
struct PoolParams {
  const __bf16* q;
  const __bf16* k;
  float* pq;
  float* pk;
  Geom g;
  int nb;  // F * NBf
  int heads[kMaxHeads];
};

__device__ inline void add_row8(float (&acc)[8], const u32x4& x) {
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    acc[2 * e] = acc[2 * e] + bf16_lo(x[e]);
    acc[2 * e + 1] = acc[2 * e + 1] + bf16_hi(x[e]);
  }
}

__global__ __launch_bounds__(256) void block_pool_kernel(PoolParams p) {
  const Geom& g = p.g;
  const int lane = tid_x() & 63, sub = lane & 7;
  const int bi = (bid_x() * 4 + (tid_x() >> 6)) * 8 + (lane >> 3);
  if (bi >= p.nb) return;
  const int hs = bid_y();
  const int h = p.heads[hs];
  const int f = bi / g.NBf, b = bi % g.NBf;
  const int cnt = min(64, g.P - 64 * b);
  const int64_t row0 = (int64_t)h * g.L + g.Sp + (int64_t)f * g.Pp + 64 * b;
  const u32x4* qs = reinterpret_cast<const u32x4*>(p.q + row0 * 64) + sub;
  const u32x4* ks = p.k ? reinterpret_cast<const u32x4*>(p.k + row0 * 64) + sub : nullptr;
  float aq[8], ak[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) aq[e] = ak[e] = 0.f;
  for (int g0 = 0; g0 < cnt; g0 += kPoolGroup) {
    const int g1 = min(cnt, g0 + kPoolGroup);
    float gq[8], gk[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) gq[e] = gk[e] = 0.f;
    int r = g0;
    for (; r + 4 <= g1; r += 4) {
      u32x4 xq[4], xk[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) xq[j] = qs[(r + j) * 8];
      if (ks) {
#pragma unroll
        for (int j = 0; j < 4; ++j) xk[j] = ks[(r + j) * 8];
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) add_row8(gq, xq[j]);
      if (ks) {
#pragma unroll
        for (int j = 0; j < 4; ++j) add_row8(gk, xk[j]);
      }
    }
    for (; r < g1; ++r) {
      add_row8(gq, qs[r * 8]);
      if (ks) add_row8(gk, ks[r * 8]);
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      aq[e] = aq[e] + gq[e];
      ak[e] = ak[e] + gk[e];
    }
  }
  const float fc = (float)cnt;
  const int64_t o = ((int64_t)hs * p.nb + bi) * 64 + 8 * sub;
  f32x4* dq = reinterpret_cast<f32x4*>(p.pq + o);
  dq[0] = f32x4{aq[0] / fc, aq[1] / fc, aq[2] / fc, aq[3] / fc};
  dq[1] = f32x4{aq[4] / fc, aq[5] / fc, aq[6] / fc, aq[7] / fc};
  if (ks) {
    f32x4* dk = reinterpret_cast<f32x4*>(p.pk + o);
    dk[0] = f32x4{ak[0] / fc, ak[1] / fc, ak[2] / fc, ak[3] / fc};
    dk[1] = f32x4{ak[4] / fc, ak[5] / fc, ak[6] / fc, ak[7] / fc};
  }
}

// ---------------------------------------------------------------------------------------
// Top-k from a score matrix. Rows of up to kRowLds floats are staged in LDS with coalesced
// 16-byte LDS-DMA loads (as many rows per workgroup as keep its threads busy) and each thread then selects
// one (row, frame); longer rows are read directly, one thread per (row, frame).
// ---------------------------------------------------------------------------------------
constexpr int kRowLds = 12288;

template <int K>
__device__ inline void select_frame(const float* sp, int C, int f, int ke, int32_t* o) {
  uint64_t a[K];
#pragma unroll
  for (int t = 0; t < K; ++t) a[t] = 0;
  for (int c = 0; c < C; ++c) {
    uint64_t x = ckey(sp[c], (uint32_t)c);
    if (x > a[K - 1]) topk_insert<K>(a, x);
  }
  int32_t v[K];
#pragma unroll
  for (int t = 0; t < K; ++t) v[t] = a[t] ? (int32_t)(f * C + ckey_index(a[t])) : -1;
  if (K >= 4 && ke == K && ((uintptr_t)o & 15) == 0) {
    // whole 16-byte groups: one vector store each (consecutive frames are consecutive groups)
#pragma unroll
    for (int t = 0; t + 3 < K; t += 4) reinterpret_cast<u32x4*>(o)[t >> 2] = u32x4{(uint32_t)v[t], (uint32_t)v[t + 1],
                                                                                     (uint32_t)v[t + 2], (uint32_t)v[t + 3]};
  } else {
#pragma unroll
    for (int t = 0; t < K; ++t)
      if (t < ke) o[t] = v[t];
  }
}

// A workgroup stages `rpw` consecutive rows (contiguous in memory) with coalesced 16-byte loads
// and then every thread selects one (row, frame): with F = 128 frames two rows keep all 256
// threads busy.
template <int K>
__global__ __launch_bounds__(256) void topk_scores_row_kernel(const float* __restrict__ s, int64_t nrows, int F,
                                                              int C, int ke, int rpw, int32_t* __restrict__ idx) {
  extern __shared__ __align__(16) float buf[];  // rpw * F * C floats (dynamic: sized per launch)
  const int64_t r0 = (int64_t)bid_x() * rpw;
  const int nr = (int)min((int64_t)rpw, nrows - r0);
  const int n = F * C;
  const int tot = nr * n;
  const float* src = s + r0 * n;
  if ((tot & 3) == 0 && ((uintptr_t)src & 15) == 0) {
    // LDS-DMA copy: every 16-byte chunk goes straight to LDS and a thread's loads are all in flight
    // at once (wave w of pass i0 fills chunks i0 + 64w .. i0 + 64w + 63, lane by lane)
    const int n4 = tot >> 2, w = tid_x() >> 6;
    for (int i0 = 0; i0 < n4; i0 += 256) {
      const int i = i0 + tid_x();
      if (i < n4)
        __builtin_amdgcn_global_load_lds((const void*)(src + 4 * (int64_t)i), (lds_void*)(buf + 4 * (i0 + 64 * w)), 16, 0,
                                         0);
    }
    wait_vm<0>();
  } else {
    for (int i = tid_x(); i < tot; i += 256) buf[i] = src[i];
  }
  __syncthreads();
  for (int t = tid_x(); t < nr * F; t += 256) {
    const int rr = t / F, f = t % F;
    select_frame<K>(buf + rr * n + f * C, C, f, ke, idx + (r0 + rr) * ((int64_t)F * ke) + (int64_t)f * ke);
  }
}

template <int K>
__global__ __launch_bounds__(256) void topk_scores_kernel(const float* __restrict__ s, int64_t nrows, int F, int C,
                                                          int ke, int32_t* __restrict__ idx) {
  const int64_t gid = (int64_t)bid_x() * 256 + tid_x();
  if (gid >= nrows * F) return;
  const int64_t row = gid / F;
  const int f = (int)(gid % F);
  select_frame<K>(s + row * ((int64_t)F * C) + (int64_t)f * C, C, f, ke, idx + row * ((int64_t)F * ke) + (int64_t)f * ke);
}

// ---------------------------------------------------------------------------------------
// Fused block select from pooled Q/K. A workgroup owns 256 query blocks of one head (one per
// thread, its pooled vector in registers) and a range of key frames; each frame's pooled key
// blocks are staged once in LDS (double-buffered) and read as broadcasts, every score is the
// sequential fmaf chain over d = 0..63, and each thread keeps its top-k per frame.
// ---------------------------------------------------------------------------------------
constexpr int kSelFramesPerGroup = 8;

template <int K>
__global__ __launch_bounds__(256) void block_select_frame_kernel(const float* __restrict__ pq,
                                                                 const float* __restrict__ pk, int nbq, int F,
                                                                 int NBf, int ke, int32_t* __restrict__ idx) {
  __shared__ __align__(16) float kt[2][32 * 64];
  const int hs = bid_y();
  const int i = bid_x() * 256 + tid_x();
  const int f0 = bid_z() * kSelFramesPerGroup;
  const int f1 = min(F, f0 + kSelFramesPerGroup);
  const bool active = i < nbq;
  float qv[64];
  {
    const f32x4* qr = reinterpret_cast<const f32x4*>(pq + ((int64_t)hs * nbq + (active ? i : 0)) * 64);
#pragma unroll
    for (int d4 = 0; d4 < 16; ++d4) {
      const f32x4 x = qr[d4];
      qv[4 * d4] = x[0];
      qv[4 * d4 + 1] = x[1];
      qv[4 * d4 + 2] = x[2];
      qv[4 * d4 + 3] = x[3];
    }
  }
  const int64_t nbk = (int64_t)F * NBf;
  const float* kbase = pk + (int64_t)hs * nbk * 64;
  const int nvec = NBf * 16;  // f32x4 per frame
  auto stage = [&](int f, int b) {
    const f32x4* src = reinterpret_cast<const f32x4*>(kbase + (int64_t)f * NBf * 64);
    for (int v = tid_x(); v < nvec; v += 256) reinterpret_cast<f32x4*>(kt[b])[v] = src[v];
  };
  stage(f0, 0);
  __syncthreads();
  int32_t* orow = idx + ((int64_t)hs * nbq + (active ? i : 0)) * ((int64_t)F * ke);
  for (int f = f0; f < f1; ++f) {
    const int b = (f - f0) & 1;
    if (f + 1 < f1) stage(f + 1, b ^ 1);
    uint64_t a[K];
#pragma unroll
    for (int t = 0; t < K; ++t) a[t] = 0;
    for (int c = 0; c < NBf; ++c) {
      const f32x4* kr = reinterpret_cast<const f32x4*>(kt[b] + c * 64);
      float acc = 0.f;
#pragma unroll
      for (int d4 = 0; d4 < 16; ++d4) {
        const f32x4 kv = kr[d4];
        acc = __builtin_fmaf(qv[4 * d4 + 0], kv[0], acc);
        acc = __builtin_fmaf(qv[4 * d4 + 1], kv[1], acc);
        acc = __builtin_fmaf(qv[4 * d4 + 2], kv[2], acc);
        acc = __builtin_fmaf(qv[4 * d4 + 3], kv[3], acc);
      }
      const uint64_t x = ckey(acc, (uint32_t)c);
      if (x > a[K - 1]) topk_insert<K>(a, x);
    }
    if (active) {
      int32_t* o = orow + (int64_t)f * ke;
#pragma unroll
      for (int t = 0; t < K; ++t)
        if (t < ke) o[t] = a[t] ? (int32_t)(f * NBf + ckey_index(a[t])) : -1;
    }
    __syncthreads();
  }
}

// Global scope: each thread keeps the top-k of a strided candidate subset, lists are merged in LDS.
template <int K>
__global__ __launch_bounds__(256) void block_select_global_kernel(const float* __restrict__ pq,
                                                                  const float* __restrict__ pk, int nbq, int nbk,
                                                                  int ke, int32_t* __restrict__ idx) {
  __shared__ float qv[64];
  __shared__ uint64_t lists[256 * K];
  const int i = bid_x(), hs = bid_y();
  if (tid_x() < 64) qv[tid_x()] = pq[((int64_t)hs * nbq + i) * 64 + tid_x()];
  __syncthreads();
  const float* kbase = pk + (int64_t)hs * nbk * 64;
  uint64_t a[K];
#pragma unroll
  for (int t = 0; t < K; ++t) a[t] = 0;
  for (int c = tid_x(); c < nbk; c += 256) {
    const f32x4* kr = reinterpret_cast<const f32x4*>(kbase + (int64_t)c * 64);
    float acc = 0.f;
#pragma unroll
    for (int d4 = 0; d4 < 16; ++d4) {
      f32x4 kv = kr[d4];
      acc = __builtin_fmaf(qv[4 * d4 + 0], kv[0], acc);
      acc = __builtin_fmaf(qv[4 * d4 + 1], kv[1], acc);
      acc = __builtin_fmaf(qv[4 * d4 + 2], kv[2], acc);
      acc = __builtin_fmaf(qv[4 * d4 + 3], kv[3], acc);
    }
    uint64_t x = ckey(acc, (uint32_t)c);
    if (x > a[K - 1]) topk_insert<K>(a, x);
  }
#pragma unroll
  for (int t = 0; t < K; ++t) lists[tid_x() * K + t] = a[t];
  __syncthreads();
  // tree merge: at each step thread t < s merges list t + s into list t
  for (int s = 128; s > 0; s >>= 1) {
    if (tid_x() < s) {
#pragma unroll
      for (int t = 0; t < K; ++t) {
        uint64_t x = lists[(tid_x() + s) * K + t];
        if (x > a[K - 1]) topk_insert<K>(a, x);
      }
#pragma unroll
      for (int t = 0; t < K; ++t) lists[tid_x() * K + t] = a[t];
    }
    __syncthreads();
  }
  if (tid_x() == 0) {
    int32_t* o = idx + ((int64_t)hs * nbq + i) * ke;
#pragma unroll
    for (int t = 0; t < K; ++t)
      if (t < ke) o[t] = a[t] ? (int32_t)ckey_index(a[t]) : -1;
  }
}


template <template <int> class Launcher, typename... Args>
int dispatch_k(int k, Args... args) {
  if (k <= 1) return Launcher<1>::run(args...);
  if (k <= 2) return Launcher<2>::run(args...);
  if (k <= 4) return Launcher<4>::run(args...);
  if (k <= 8) return Launcher<8>::run(args...);
  if (k <= 16) return Launcher<16>::run(args...);
  return Launcher<32>::run(args...);
}

template <int K>
struct TopkScoresLaunch {
  static int run(const float* s, int64_t nrows, int F, int C, int ke, int32_t* idx, hipStream_t st) {
    const int64_t n = (int64_t)F * C;
    if (n <= kRowLds && nrows <= 0x7fffffff) {
      const int rpw = (int)std::max<int64_t>(1, std::min<int64_t>(256 / std::max(F, 1), kRowLds / n));
      const int64_t groups = (nrows + rpw - 1) / rpw;
      const size_t lds = (size_t)rpw * n * sizeof(float);
      hipLaunchKernelGGL(topk_scores_row_kernel<K>, dim3((unsigned)groups), dim3(256), lds, st, s, nrows, F, C, ke,
                         rpw, idx);
    } else {
      const int64_t nt = nrows * F;
      hipLaunchKernelGGL(topk_scores_kernel<K>, dim3((unsigned)((nt + 255) / 256)), dim3(256), 0, st, s, nrows, F, C,
                         ke, idx);
    }
    return check_launch("saf3r_topk_from_scores");
  }
};

template <int K>
struct SelectFrameLaunch {
  static int run(const float* pq, const float* pk, int n, int nbq, int F, int NBf, int ke, int32_t* idx,
                 hipStream_t st) {
    dim3 grid((nbq + 255) / 256, n, (F + kSelFramesPerGroup - 1) / kSelFramesPerGroup);
    hipLaunchKernelGGL(block_select_frame_kernel<K>, grid, dim3(256), 0, st, pq, pk, nbq, F, NBf, ke, idx);
    return check_launch("saf3r_block_select");
  }
};

template <int K>
struct SelectGlobalLaunch {
  static int run(const float* pq, const float* pk, int n, int nbq, int nbk, int ke, int32_t* idx, hipStream_t st) {
    hipLaunchKernelGGL(block_select_global_kernel<K>, dim3(nbq, n), dim3(256), 0, st, pq, pk, nbq, nbk, ke, idx);
    return check_launch("saf3r_block_select");
  }
};

}  // namespace saf3r

using namespace saf3r;

extern "C" int saf3r_block_pool(const void* q_packed, const void* k_packed, int frames, int tokens_per_frame,
                                int num_special, int num_heads, const int32_t* head_ids, int n_heads_sel,
                                float* pooled_q, float* pooled_k, void* stream) {
  if (int e = injected("saf3r_block_pool")) return e;
  PoolParams p;
  if (!make_geom(frames, tokens_per_frame, num_special, &p.g))
    return fail(SAF3R_ERR_INVALID, "saf3r_block_pool: invalid geometry");
  if (n_heads_sel <= 0 || n_heads_sel > kMaxHeads || !head_ids)
    return fail(SAF3R_ERR_INVALID, "saf3r_block_pool: need 1..%d head ids", kMaxHeads);
  if (!q_packed || !pooled_q || ((k_packed == nullptr) != (pooled_k == nullptr)))
    return fail(SAF3R_ERR_INVALID, "saf3r_block_pool: null / mismatched pointers");
  for (int i = 0; i < n_heads_sel; ++i) {
    if (head_ids[i] < 0 || head_ids[i] >= num_heads)
      return fail(SAF3R_ERR_INVALID, "saf3r_block_pool: head id %d out of range", head_ids[i]);
    p.heads[i] = head_ids[i];
  }
  p.q = (const __bf16*)q_packed;
  p.k = (const __bf16*)k_packed;
  p.pq = pooled_q;
  p.pk = pooled_k;
  p.nb = frames * p.g.NBf;
  hipLaunchKernelGGL(block_pool_kernel, dim3((p.nb + 31) / 32, n_heads_sel), dim3(256), 0, (hipStream_t)stream, p);
  return check_launch("saf3r_block_pool");
}

extern "C" int saf3r_topk_from_scores(const float* scores, int n, int rows, int frames, int cands_per_frame, int k,
                                      int32_t* idx, void* stream) {
  if (int e = injected("saf3r_topk_from_scores")) return e;
  if (!scores || !idx) return fail(SAF3R_ERR_INVALID, "saf3r_topk_from_scores: null pointer");
  if (n <= 0 || rows <= 0 || frames <= 0 || cands_per_frame <= 0)
    return fail(SAF3R_ERR_INVALID, "saf3r_topk_from_scores: bad shape");
  if (k < 1 || k > 32) return fail(SAF3R_ERR_UNSUPPORTED, "saf3r_topk_from_scores: k must be in [1, 32] (got %d)", k);
  int ke = k < cands_per_frame ? k : cands_per_frame;
  return dispatch_k<TopkScoresLaunch>(ke, scores, (int64_t)n * rows, frames, cands_per_frame, ke, idx,
                                      (hipStream_t)stream);
}

extern "C" int saf3r_block_select(const float* pooled_q, const float* pooled_k, int n, int nbq, int frames,
                                  int blocks_per_frame, int k, int scope, int32_t* idx, void* stream) {
  if (int e = injected("saf3r_block_select")) return e;
  if (!pooled_q || !pooled_k || !idx) return fail(SAF3R_ERR_INVALID, "saf3r_block_select: null pointer");
  if (n <= 0 || n > 65535 || nbq <= 0 || frames <= 0 || blocks_per_frame <= 0)
    return fail(SAF3R_ERR_INVALID, "saf3r_block_select: bad shape");
  if (k < 1 || k > 32) return fail(SAF3R_ERR_UNSUPPORTED, "saf3r_block_select: k must be in [1, 32] (got %d)", k);
  if (scope == 0) {
    if (blocks_per_frame > 32)
      return fail(SAF3R_ERR_UNSUPPORTED, "saf3r_block_select: per-frame scope supports at most 32 blocks per frame");
    int ke = k < blocks_per_frame ? k : blocks_per_frame;
    return dispatch_k<SelectFrameLaunch>(ke, pooled_q, pooled_k, n, nbq, frames, blocks_per_frame, ke, idx,
                                         (hipStream_t)stream);
  }
  if (scope == 1) {
    int nbk = frames * blocks_per_frame;
    int ke = k < nbk ? k : nbk;
    if (ke > 16) return fail(SAF3R_ERR_UNSUPPORTED, "saf3r_block_select: global scope supports k <= 16");
    return dispatch_k<SelectGlobalLaunch>(ke, pooled_q, pooled_k, n, nbq, nbk, ke, idx, (hipStream_t)stream);
  }
  return fail(SAF3R_ERR_INVALID, "saf3r_block_select: scope must be 0 (frame) or 1 (global)");
}
