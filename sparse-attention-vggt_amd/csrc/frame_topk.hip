// Token top-k from blocks of bf16 scores: the selection half of the non-lazy DINO-feature path.
//
// ref: saf3r/patch/utils.py:54-184 (compute_qk_topk_indices_batched: per-frame torch.topk of bf16
//      q.k scores, optional exclusion of frame 0 with strided first-frame samples prepended, and a
//      cap on the number of kept keys), saf3r/patch/patch_vggt.py:313-357 (its caller).
//
// Scores are bf16 bit patterns; a key is ranked by the score, ties go to the lower key index. The
// 16-bit order key of a score is its sortable transform (larger score -> larger key, -0 < +0).
//   frame stage: one wave per (row, frame) takes the frame's top-k by a two-pass byte radix select
//                in registers and LDS, then writes the k keys in increasing key order;
//   cap stage:   one work-group per row takes the best `cap` of a candidate list (the frame stage's
//                output, or every key of the row when selection is not per frame) the same way,
//                in list order, which is increasing key order.
#include "common.h"

namespace saf3r {

constexpr int kMaxSegRegs = 64;  // frame stage: per_frame <= 64 * 64

struct FrameTopkParams {
  const uint16_t* scores;
  int64_t srs;        // score row stride (elements)
  int rows, F, P, f0;  // f0: first frame selected from (1 excludes frame 0)
  int k;              // keys per frame
  int32_t* out;       // frame stage output (idx or candidate list)
  int64_t ors;        // its row stride
  int ocol;           // first column written
  uint16_t* okey;     // candidate order keys (cap stage input), row stride ors, or null
};

struct CapParams {
  const uint16_t* scores;  // dense mode: the score rows
  int64_t srs;
  int64_t dense_base;      // dense mode: first key, dense_n: key count
  int64_t dense_n;
  const int32_t* cidx;     // list mode: candidate keys and their order keys
  const uint16_t* ckey;
  int64_t crs;
  int64_t n;               // list mode: candidates per row
  int rows, cap;
  int32_t* out;
  int64_t ors;
  int ocol;
};

__device__ inline uint32_t sortable16(uint16_t b) { return (uint32_t)(b ^ ((b & 0x8000u) ? 0xFFFFu : 0x8000u)); }

// Byte-histogram step of a radix select over keys held by the caller: counts[256] in LDS; returns
// the bin holding the rank-`need` largest key and, through above, the number of keys above it.
template <int NT>
__device__ inline int radix_bin(uint32_t* counts, int need, int* above, int lane, uint32_t* scan) {
  // NT threads cooperate; thread t owns bins 256 - (t + 1) * (256 / NT) .. (from the top)
  constexpr int per = 256 / NT;
  uint32_t s = 0;
#pragma unroll
  for (int i = 0; i < per; ++i) s += counts[255 - (lane * per + i)];
  scan[lane] = s;
  __syncthreads();
  // exclusive prefix over threads from the top (small: NT <= 256)
  uint32_t pre = 0;
  for (int t = 0; t < lane; ++t) pre += scan[t];
  int bin = -1, ab = 0;
  if ((int)pre < need && (int)(pre + s) >= need) {
    uint32_t acc = pre;
#pragma unroll
    for (int i = 0; i < per; ++i) {
      const uint32_t c = counts[255 - (lane * per + i)];
      if ((int)(acc + c) >= need) {
        bin = 255 - (lane * per + i);
        ab = (int)acc;
        break;
      }
      acc += c;
    }
  }
  __syncthreads();
  if (bin >= 0) {
    scan[0] = (uint32_t)bin;
    scan[1] = (uint32_t)ab;
  }
  __syncthreads();
  *above = (int)scan[1];
  const int b = (int)scan[0];
  __syncthreads();
  return b;
}

// ---- frame stage: four waves, one (row, frame) each ----
template <int RM>  // key registers per lane: per_frame <= 64 * RM
__global__ __launch_bounds__(256) void frame_select_kernel(FrameTopkParams p) {
  __shared__ uint32_t hist[4][256];
  __shared__ uint32_t scan[4][64];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int row = blockIdx.y;
  const int nfr = p.F - p.f0;
  const int fs = blockIdx.x * 4 + w;  // selected-frame index
  const bool active = fs < nfr;
  const int f = p.f0 + (active ? fs : 0);
  const int R = (p.P + 63) >> 6;
  const uint16_t* src = p.scores + (int64_t)row * p.srs + (int64_t)f * p.P;
  uint32_t key[RM];
#pragma unroll
  for (int r = 0; r < RM; ++r) {
    const int j = r * 64 + lane;
    key[r] = (r < R && j < p.P && active) ? sortable16(src[j]) : 0xFFFFFFFFu;  // 0xFFFFFFFF: no key
  }
  uint32_t* h = hist[w];
  uint32_t* sc = scan[w];
  // wave-local passes (waves share nothing; the barriers keep the work-group in step)
  auto clear = [&]() {
#pragma unroll
    for (int i = 0; i < 4; ++i) h[lane * 4 + i] = 0;
  };
  auto wave_bin = [&](int need, int* above) {
    // lane owns bins 255 - 4*lane - i; inclusive counts from the top via a wave scan
    uint32_t c[4], s = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      c[i] = h[255 - (lane * 4 + i)];
      s += c[i];
    }
    sc[lane] = s;
    __builtin_amdgcn_wave_barrier();
    uint32_t pre = 0;
    for (int t = 0; t < lane; ++t) pre += sc[t];
    int bin = -1, ab = 0;
    if ((int)pre < need && (int)(pre + s) >= need) {
      uint32_t acc = pre;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if (bin < 0 && (int)(acc + c[i]) >= need) {
          bin = 255 - (lane * 4 + i);
          ab = (int)acc;
        }
        acc += c[i];
      }
    }
    const uint64_t m = __ballot(bin >= 0);
    const int src_lane = m ? __builtin_ctzll(m) : 0;
    *above = __shfl(ab, src_lane, 64);
    return __shfl(bin, src_lane, 64);
  };
  const int k = p.k;
  clear();
  __syncthreads();
#pragma unroll
  for (int r = 0; r < RM; ++r)
    if (r < R && key[r] != 0xFFFFFFFFu) atomicAdd(&h[key[r] >> 8], 1u);
  __syncthreads();
  int above1 = 0;
  const int b1 = wave_bin(k, &above1);
  __syncthreads();
  clear();
  __syncthreads();
#pragma unroll
  for (int r = 0; r < RM; ++r)
    if (r < R && key[r] != 0xFFFFFFFFu && (int)(key[r] >> 8) == b1) atomicAdd(&h[key[r] & 255], 1u);
  __syncthreads();
  int above2 = 0;
  const int b2 = wave_bin(k - above1, &above2);
  const uint32_t t = ((uint32_t)b1 << 8) | (uint32_t)b2;
  const int need_eq = k - above1 - above2;  // keys equal to t to keep, lowest index first
  // ordered compaction: element order r-major, lane-minor = increasing key index
  int base = 0, eq_seen = 0;
  int32_t* o = p.out + (int64_t)row * p.ors + p.ocol + (int64_t)fs * k;
  uint16_t* ok = p.okey ? p.okey + (int64_t)row * p.ors + (int64_t)fs * k : nullptr;
#pragma unroll
  for (int r = 0; r < RM; ++r) {
    if (r < R) {
      const bool valid = key[r] != 0xFFFFFFFFu;
      const bool eq = valid && key[r] == t;
      const uint64_t me = __ballot(eq);
      const int eq_rank = eq_seen + (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(me >> 32),
                                                                 __builtin_amdgcn_mbcnt_lo((uint32_t)me, 0));
      const bool sel = valid && (key[r] > t || (eq && eq_rank < need_eq));
      const uint64_t ms = __ballot(sel);
      const int pos = base + (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(ms >> 32),
                                                          __builtin_amdgcn_mbcnt_lo((uint32_t)ms, 0));
      if (sel && active) {
        o[pos] = f * p.P + r * 64 + lane;
        if (ok) ok[pos] = (uint16_t)key[r];
      }
      base += __popcll(ms);
      eq_seen += __popcll(me);
    }
  }
}

// ---- cap stage: one work-group per row ----
__device__ inline void cap_item(const CapParams& p, int row, int64_t i, uint32_t* key, int32_t* idx) {
  if (p.cidx) {
    *idx = p.cidx[(int64_t)row * p.crs + i];
    *key = p.ckey[(int64_t)row * p.crs + i];
  } else {
    *idx = (int32_t)(p.dense_base + i);
    *key = sortable16(p.scores[(int64_t)row * p.srs + p.dense_base + i]);
  }
}

__global__ __launch_bounds__(256) void cap_select_kernel(CapParams p) {
  __shared__ uint32_t hist[256];
  __shared__ uint32_t scan[256];
  __shared__ uint32_t wsum[4];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int row = blockIdx.x;
  const int64_t n = p.cidx ? p.n : p.dense_n;
  const int m = p.cap;
  hist[tid] = 0;
  __syncthreads();
  for (int64_t i = tid; i < n; i += 256) {
    uint32_t k;
    int32_t x;
    cap_item(p, row, i, &k, &x);
    atomicAdd(&hist[k >> 8], 1u);
  }
  __syncthreads();
  int above1 = 0;
  const int b1 = radix_bin<256>(hist, m, &above1, tid, scan);
  hist[tid] = 0;
  __syncthreads();
  for (int64_t i = tid; i < n; i += 256) {
    uint32_t k;
    int32_t x;
    cap_item(p, row, i, &k, &x);
    if ((int)(k >> 8) == b1) atomicAdd(&hist[k & 255], 1u);
  }
  __syncthreads();
  int above2 = 0;
  const int b2 = radix_bin<256>(hist, m - above1, &above2, tid, scan);
  const uint32_t t = ((uint32_t)b1 << 8) | (uint32_t)b2;
  const int need_eq = m - above1 - above2;
  // ordered compaction over the list in chunks of 256 (block prefix of ballots)
  int base = 0, eq_seen = 0;
  int32_t* o = p.out + (int64_t)row * p.ors + p.ocol;
  for (int64_t c0 = 0; c0 < n; c0 += 256) {
    const int64_t i = c0 + tid;
    uint32_t k = 0;
    int32_t x = 0;
    const bool valid = i < n;
    if (valid) cap_item(p, row, i, &k, &x);
    const bool eq = valid && k == t;
    // rank of eq among the list's eq items before i
    const uint64_t me = __ballot(eq);
    const int in_wave_eq = (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(me >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)me, 0));
    if (lane == 0) wsum[w] = __popcll(me);
    __syncthreads();
    int eq_before = eq_seen;
    for (int v = 0; v < w; ++v) eq_before += wsum[v];
    const int eq_tot = wsum[0] + wsum[1] + wsum[2] + wsum[3];
    __syncthreads();
    const bool sel = valid && (k > t || (eq && eq_before + in_wave_eq < need_eq));
    const uint64_t ms = __ballot(sel);
    const int in_wave = (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(ms >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)ms, 0));
    if (lane == 0) wsum[w] = __popcll(ms);
    __syncthreads();
    int before = base;
    for (int v = 0; v < w; ++v) before += wsum[v];
    const int tot = wsum[0] + wsum[1] + wsum[2] + wsum[3];
    __syncthreads();
    if (sel) o[before + in_wave] = x;
    base += tot;
    eq_seen += eq_tot;
  }
}

__global__ __launch_bounds__(256) void first_samples_kernel(int32_t* idx, int64_t idx_stride, int n, int stride) {
  int32_t* o = idx + (int64_t)blockIdx.x * idx_stride;
  for (int i = threadIdx.x; i < n; i += 256) o[i] = i * stride;
}

}  // namespace saf3r

using namespace saf3r;

extern "C" int saf3r_frame_topk_scores(const void* scores, int64_t score_stride, int rows, int frames, int per_frame,
                                       int exclude_first, int first_stride, int per_frame_mode, int topk, int cap,
                                       int32_t* idx, int64_t idx_stride, int32_t* cand_idx, uint16_t* cand_key,
                                       void* stream) {
  if (int e = injected("saf3r_frame_topk_scores")) return e;
  if (!scores || !idx) return fail(SAF3R_ERR_INVALID, "saf3r_frame_topk_scores: null pointer");
  if (rows < 0 || frames <= 0 || per_frame <= 0 || topk <= 0 || first_stride < 0 || rows > 65535)
    return fail(SAF3R_ERR_INVALID, "saf3r_frame_topk_scores: bad shape");
  const int64_t nk = (int64_t)frames * per_frame;
  if (nk > 0x7fffffff || score_stride < nk) return fail(SAF3R_ERR_INVALID, "saf3r_frame_topk_scores: bad score stride");
  const int f0 = exclude_first ? 1 : 0;
  const int nfr = frames - f0;
  const int fsel = exclude_first && first_stride > 0 ? (per_frame + first_stride - 1) / first_stride : 0;
  if (exclude_first && first_stride <= 0)
    return fail(SAF3R_ERR_INVALID, "saf3r_frame_topk_scores: first_stride must be positive with exclude_first");
  // keys drawn from the frames after the optional frame 0, before the cap
  int64_t rest;
  if (per_frame_mode) rest = (int64_t)min(topk, per_frame) * nfr;
  else rest = min((int64_t)topk, nk - (int64_t)f0 * per_frame);
  const int64_t kept = cap > 0 ? min(rest, (int64_t)cap) : rest;
  if (idx_stride < fsel + kept) return fail(SAF3R_ERR_INVALID, "saf3r_frame_topk_scores: idx_stride too small");
  if (per_frame_mode && per_frame > 64 * kMaxSegRegs)
    return fail(SAF3R_ERR_UNSUPPORTED, "saf3r_frame_topk_scores: per_frame must be <= %d", 64 * kMaxSegRegs);
  if (rows == 0) return SAF3R_OK;
  hipStream_t st = (hipStream_t)stream;
  if (fsel > 0) {
    // the guaranteed first-frame samples 0, s, 2s, ... in the first columns of every row
    hipLaunchKernelGGL(first_samples_kernel, dim3(rows), dim3(256), 0, st, idx, idx_stride, fsel, first_stride);
    if (int e = check_launch("saf3r_frame_topk_scores")) return e;
  }
  const bool capped = kept < rest;
  if (per_frame_mode && nfr > 0) {
    const int k = min(topk, per_frame);
    if (capped && (!cand_idx || !cand_key))
      return fail(SAF3R_ERR_INVALID, "saf3r_frame_topk_scores: the cap needs the candidate buffers");
    FrameTopkParams p;
    p.scores = (const uint16_t*)scores;
    p.srs = score_stride;
    p.rows = rows;
    p.F = frames;
    p.P = per_frame;
    p.f0 = f0;
    p.k = k;
    p.out = capped ? cand_idx : idx;
    p.ors = capped ? rest : idx_stride;
    p.ocol = capped ? 0 : fsel;
    p.okey = capped ? cand_key : nullptr;
    const dim3 grid((nfr + 3) / 4, rows);
    const int R = (per_frame + 63) / 64;
    if (R <= 8) hipLaunchKernelGGL(frame_select_kernel<8>, grid, dim3(256), 0, st, p);
    else if (R <= 16) hipLaunchKernelGGL(frame_select_kernel<16>, grid, dim3(256), 0, st, p);
    else if (R <= 24) hipLaunchKernelGGL(frame_select_kernel<24>, grid, dim3(256), 0, st, p);
    else if (R <= 32) hipLaunchKernelGGL(frame_select_kernel<32>, grid, dim3(256), 0, st, p);
    else hipLaunchKernelGGL(frame_select_kernel<kMaxSegRegs>, grid, dim3(256), 0, st, p);
    if (int e = check_launch("saf3r_frame_topk_scores")) return e;
    if (!capped) return SAF3R_OK;
  }
  if (kept <= 0) return SAF3R_OK;
  CapParams c;
  c.scores = (const uint16_t*)scores;
  c.srs = score_stride;
  c.dense_base = (int64_t)f0 * per_frame;
  c.dense_n = nk - c.dense_base;
  c.cidx = per_frame_mode ? cand_idx : nullptr;
  c.ckey = per_frame_mode ? cand_key : nullptr;
  c.crs = rest;
  c.n = rest;
  c.rows = rows;
  c.cap = (int)kept;
  c.out = idx;
  c.ors = idx_stride;
  c.ocol = fsel;
  hipLaunchKernelGGL(cap_select_kernel, dim3(rows), dim3(256), 0, st, c);
  return check_launch("saf3r_frame_topk_scores");
}
