// Block selection of the dynamic pattern: pooled patch-block means, block scores and the
// per-frame (or global) top-k with the sortable-key / lowest-index tie rule.
//
// ref: saf3r/triton/fused_qk_topk.py:73-100 (composite key = sortable fp32 bits << 32 | reversed
//      index, running top-k per frame, frame-major flush in descending order),
//      saf3r/triton/topk_utils.py:26-29 (sortable key), saf3r/patch/wrapper.py:48 (top-k per frame),
//      saf3r/patch/adaptive_block_value.py:16-24 (block mean over the real population).
// Every fp32 result is produced in a fixed operation order (sequential sums, one division,
// sequential fma), so it is bit-identical to that definition.
#include "common.h"

namespace saf3r {

// Insert composite key x into a descending list a[0..K) (strict '>' bubble). Entries equal to
// 0 are empty; real composites are > 0 and pairwise distinct.
template <int K>
__device__ inline void topk_insert(uint64_t (&a)[K], uint64_t x) {
#pragma unroll
  for (int t = 0; t < K; ++t) {
    uint64_t hi = x > a[t] ? x : a[t];
    uint64_t lo = x > a[t] ? a[t] : x;
    a[t] = hi;
    x = lo;
  }
}

// ---------------------------------------------------------------------------------------
// Pooling: one wave per (head, patch block), lane = feature.
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

__global__ __launch_bounds__(256) void block_pool_kernel(PoolParams p) {
  const Geom& g = p.g;
  const int lane = threadIdx.x & 63;
  const int bi = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (bi >= p.nb) return;
  const int hs = blockIdx.y;
  const int h = p.heads[hs];
  const int f = bi / g.NBf, b = bi % g.NBf;
  const int cnt = min(64, g.P - 64 * b);
  const int64_t row0 = (int64_t)h * g.L + g.Sp + (int64_t)f * g.Pp + 64 * b;
  const __bf16* qs = p.q + row0 * 64 + lane;
  const __bf16* ks = p.k ? p.k + row0 * 64 + lane : nullptr;
  float aq = 0.f, ak = 0.f;
  int r = 0;
  for (; r + 8 <= cnt; r += 8) {
    float vq[8], vk[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) vq[j] = (float)qs[(r + j) * 64];
    if (ks) {
#pragma unroll
      for (int j = 0; j < 8; ++j) vk[j] = (float)ks[(r + j) * 64];
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) aq = aq + vq[j];
    if (ks) {
#pragma unroll
      for (int j = 0; j < 8; ++j) ak = ak + vk[j];
    }
  }
  for (; r < cnt; ++r) {
    aq = aq + (float)qs[r * 64];
    if (ks) ak = ak + (float)ks[r * 64];
  }
  const int64_t o = ((int64_t)hs * p.nb + bi) * 64 + lane;
  p.pq[o] = aq / (float)cnt;
  if (ks) p.pk[o] = ak / (float)cnt;
}

// ---------------------------------------------------------------------------------------
// Top-k from a score matrix: one thread per (row, frame).
// ---------------------------------------------------------------------------------------
template <int K>
__global__ __launch_bounds__(256) void topk_scores_kernel(const float* __restrict__ s, int64_t nrows, int F, int C,
                                                          int ke, int32_t* __restrict__ idx) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= nrows * F) return;
  const int64_t row = gid / F;
  const int f = (int)(gid % F);
  const float* sp = s + row * ((int64_t)F * C) + (int64_t)f * C;
  uint64_t a[K];
#pragma unroll
  for (int t = 0; t < K; ++t) a[t] = 0;
  for (int c = 0; c < C; ++c) {
    uint64_t x = ckey(sp[c], (uint32_t)c);
    if (x > a[K - 1]) topk_insert<K>(a, x);
  }
  int32_t* o = idx + row * ((int64_t)F * ke) + (int64_t)f * ke;
#pragma unroll
  for (int t = 0; t < K; ++t)
    if (t < ke) o[t] = a[t] ? (int32_t)(f * C + ckey_index(a[t])) : -1;
}

// ---------------------------------------------------------------------------------------
// Fused block select from pooled Q/K: one workgroup per (head, query block); the pooled query
// vector is broadcast from LDS, each thread scores one frame's candidates and keeps its top-k.
// ---------------------------------------------------------------------------------------
template <int K>
__global__ __launch_bounds__(128) void block_select_frame_kernel(const float* __restrict__ pq,
                                                                 const float* __restrict__ pk, int nbq, int F,
                                                                 int NBf, int ke, int32_t* __restrict__ idx) {
  __shared__ float qv[64];
  const int i = blockIdx.x, hs = blockIdx.y;
  if (threadIdx.x < 64) qv[threadIdx.x] = pq[((int64_t)hs * nbq + i) * 64 + threadIdx.x];
  __syncthreads();
  const int64_t nbk = (int64_t)F * NBf;
  const float* kbase = pk + (int64_t)hs * nbk * 64;
  int32_t* orow = idx + ((int64_t)hs * nbq + i) * ((int64_t)F * ke);
  for (int f = threadIdx.x; f < F; f += blockDim.x) {
    uint64_t a[K];
#pragma unroll
    for (int t = 0; t < K; ++t) a[t] = 0;
    for (int c = 0; c < NBf; ++c) {
      const f32x4* kr = reinterpret_cast<const f32x4*>(kbase + ((int64_t)f * NBf + c) * 64);
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
    int32_t* o = orow + (int64_t)f * ke;
#pragma unroll
    for (int t = 0; t < K; ++t)
      if (t < ke) o[t] = a[t] ? (int32_t)(f * NBf + ckey_index(a[t])) : -1;
  }
}

// Global scope: each thread keeps the top-k of a strided candidate subset, lists are merged in LDS.
template <int K>
__global__ __launch_bounds__(256) void block_select_global_kernel(const float* __restrict__ pq,
                                                                  const float* __restrict__ pk, int nbq, int nbk,
                                                                  int ke, int32_t* __restrict__ idx) {
  __shared__ float qv[64];
  __shared__ uint64_t lists[256 * K];
  const int i = blockIdx.x, hs = blockIdx.y;
  if (threadIdx.x < 64) qv[threadIdx.x] = pq[((int64_t)hs * nbq + i) * 64 + threadIdx.x];
  __syncthreads();
  const float* kbase = pk + (int64_t)hs * nbk * 64;
  uint64_t a[K];
#pragma unroll
  for (int t = 0; t < K; ++t) a[t] = 0;
  for (int c = threadIdx.x; c < nbk; c += 256) {
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
  for (int t = 0; t < K; ++t) lists[threadIdx.x * K + t] = a[t];
  __syncthreads();
  // tree merge: at each step thread t < s merges list t + s into list t
  for (int s = 128; s > 0; s >>= 1) {
    if (threadIdx.x < s) {
#pragma unroll
      for (int t = 0; t < K; ++t) {
        uint64_t x = lists[(threadIdx.x + s) * K + t];
        if (x > a[K - 1]) topk_insert<K>(a, x);
      }
#pragma unroll
      for (int t = 0; t < K; ++t) lists[threadIdx.x * K + t] = a[t];
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) {
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
    int64_t n = nrows * F;
    hipLaunchKernelGGL(topk_scores_kernel<K>, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, s, nrows, F, C, ke,
                       idx);
    return check_launch("saf3r_topk_from_scores");
  }
};

template <int K>
struct SelectFrameLaunch {
  static int run(const float* pq, const float* pk, int n, int nbq, int F, int NBf, int ke, int32_t* idx,
                 hipStream_t st) {
    hipLaunchKernelGGL(block_select_frame_kernel<K>, dim3(nbq, n), dim3(128), 0, st, pq, pk, nbq, F, NBf, ke, idx);
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
  hipLaunchKernelGGL(block_pool_kernel, dim3((p.nb + 3) / 4, n_heads_sel), dim3(256), 0, (hipStream_t)stream, p);
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
