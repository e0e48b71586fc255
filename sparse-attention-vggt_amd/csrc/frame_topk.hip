// Token top-k from blocks of bf16 scores: the selection half of the non-lazy DINO-feature path.
//
// ref: saf3r/patch/utils.py:54-184 (compute_qk_topk_indices_batched: per-frame torch.topk of bf16
//      q.k scores, optional exclusion of frame 0 with strided first-frame samples prepended, and a
//      cap on the number of kept keys), saf3r/patch/patch_vggt.py:313-357 (its caller).
//
// Scores are bf16 bit patterns; a key is ranked by the score, ties go to the lower key index. The
// 16-bit order key of a score is its sortable transform (larger score -> larger key, -0 < +0).
//   frame stage: one wave per (row, frame) holds the frame's scores in registers, finds the k-th
//                largest order key by bisection with wave-wide counts, and writes the k keys in
//                increasing key order;
//   cap stage:   one work-group per row takes the best `cap` of a candidate list (the frame stage's
//                output, or every key of the row when selection is not per frame) the same way,
//                in list order, which is increasing key order.
#include "common.h"

namespace saf3r {

constexpr int kMaxPerFrame = 4096;  // frame stage: at most 9 chunks of 8 keys per lane

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

// Wave-wide exclusive prefix of a small per-lane count (0..15) and the wave total, from four
// ballots of its bits.
__device__ inline int wave_prefix4(int cnt, int* total) {
  int pre = 0, tot = 0;
#pragma unroll
  for (int bit = 0; bit < 4; ++bit) {
    const uint64_t m = __ballot((cnt >> bit) & 1);
    pre += (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0)) << bit;
    tot += __popcll(m) << bit;
  }
  *total = tot;
  return pre;
}

// ---- frame stage: four waves, one (row, frame) each ----
// A lane holds RC 16-byte chunks (8 scores each) of its frame: chunk c = lane + 64 r of the frame's
// aligned span, so element order (r, lane, e) is increasing key order. The threshold t (the k-th
// largest order key) is found by bisection over the 16-bit key range with wave-wide counts.
template <int RC>
__global__ __launch_bounds__(256) void frame_select_kernel(FrameTopkParams p) {
  const int lane = tid_x() & 63, w = tid_x() >> 6;
  const int row = bid_y();
  const int nfr = p.F - p.f0;
  const int fs = bid_x() * 4 + w;  // selected-frame index
  if (fs >= nfr) return;              // whole wave: no barrier below
  const int f = p.f0 + fs;
  const int64_t s0 = (int64_t)f * p.P;        // first key of the frame in the row
  const int64_t a0 = s0 & ~(int64_t)7;        // aligned span start
  const uint16_t* rowp = p.scores + (int64_t)row * p.srs;
  // order keys of the frame's scores; slots outside the frame hold 0, which no threshold of the
  // search counts (its thresholds are >= 1; a real key 0, the lowest, only matters at t = 0)
  uint32_t key[RC][8];
  const int lo_e = (int)(s0 - a0);  // valid slot positions: lo_e <= 8 (lane + 64 r) + e < lo_e + P
  auto valid = [&](int r, int e) {
    const uint32_t pos = (uint32_t)(8 * (lane + 64 * r) + e - lo_e);
    return pos < (uint32_t)p.P;
  };
  int nv = 0;
#pragma unroll
  for (int r = 0; r < RC; ++r) {
    const int64_t e0 = a0 + 8 * (int64_t)(lane + 64 * r);
    u32x4 v = {0, 0, 0, 0};
    if (e0 < s0 + p.P) v = *reinterpret_cast<const u32x4*>(rowp + e0);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const uint16_t b = (uint16_t)(v[e >> 1] >> (16 * (e & 1)));
      const bool in = valid(r, e);
      key[r][e] = in ? sortable16(b) : 0u;
      nv += in ? 1 : 0;
    }
  }
  auto count_ge = [&](uint32_t t) {  // keys >= t (t >= 1), wave-wide
    int c = 0;
#pragma unroll
    for (int r = 0; r < RC; ++r)
#pragma unroll
      for (int e = 0; e < 8; ++e) c += key[r][e] >= t ? 1 : 0;
    // per-lane counts summed by ballots of their bits (c <= 8 * RC <= 72)
    int sum = 0;
#pragma unroll
    for (int bit = 0; bit < 7; ++bit) sum += __popcll(__ballot((c >> bit) & 1)) << bit;
    return sum;
  };
  const int k = p.k;
  // Bracket for the bisection: t is at most the largest key, and for k <= 64 at least the k-th
  // largest of the lanes' largest keys (k distinct keys reach it), found by a bisection over one
  // value per lane (a compare and a ballot per step).
  uint32_t lmax = 0;
#pragma unroll
  for (int r = 0; r < RC; ++r)
#pragma unroll
    for (int e = 0; e < 8; ++e) lmax = max(lmax, key[r][e]);
  uint32_t hi = lmax;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) hi = max(hi, (uint32_t)__shfl_xor((int)hi, o));
  uint32_t lo = 0;  // count(key >= lo) >= k holds for lo = 0
  const bool any = nv > 0;
  if (k <= 64 && __popcll(__ballot(any)) >= k) {
    uint32_t a = 0, b = hi;  // count(lane maxima >= a) >= k
    while (a < b) {
      const uint32_t mid = (a + b + 1) >> 1;
      if (__popcll(__ballot(any && lmax >= mid)) >= k) a = mid;
      else b = mid - 1;
    }
    lo = a;
  }
  int c_above = 0;  // count(key >= hi + 1): 0 for the largest key, then the count of the last miss
  while (lo < hi) {
    const uint32_t mid = (lo + hi + 1) >> 1;
    const int c = count_ge(mid);
    if (c >= k) {
      lo = mid;
    } else {
      hi = mid - 1;
      c_above = c;
    }
  }
  const uint32_t t = lo;
  const int need_eq = k - c_above;  // keys equal to t to keep, lowest first
  int32_t* o = p.out + (int64_t)row * p.ors + p.ocol + (int64_t)fs * k;
  uint16_t* ok = p.okey ? p.okey + (int64_t)row * p.ors + (int64_t)fs * k : nullptr;
  int base = 0, eq_seen = 0;
#pragma unroll
  for (int r = 0; r < RC; ++r) {
    int neq = 0;
#pragma unroll
    for (int e = 0; e < 8; ++e) neq += (valid(r, e) && key[r][e] == t) ? 1 : 0;
    int eq_tot;
    const int eq_pre = eq_seen + wave_prefix4(neq, &eq_tot);
    int nsel = 0, eq_run = 0;
    bool sel[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const bool in = valid(r, e);
      const bool eq = in && key[r][e] == t;
      sel[e] = in && (key[r][e] > t || (eq && eq_pre + eq_run < need_eq));
      eq_run += eq ? 1 : 0;
      nsel += sel[e] ? 1 : 0;
    }
    int sel_tot;
    int pos = base + wave_prefix4(nsel, &sel_tot);
    const int64_t e0 = a0 + 8 * (int64_t)(lane + 64 * r);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      if (sel[e]) {
        o[pos] = (int32_t)(e0 + e);
        if (ok) ok[pos] = (uint16_t)key[r][e];
        ++pos;
      }
    }
    base += sel_tot;
    eq_seen += eq_tot;
  }
}

// ---- frame stage for k <= 8: running per-lane top-K lists merged across the wave ----
// (larger k take the bisection above: at k = 16 over 128 frames of 1369 keys, 4096 rows, 1.23 ms
// with lists of 16 against about 1 ms)
constexpr int kSmallMaxK = 8;
// Composite key (order key << 16 | 0xFFFF - j) of key j of the frame: larger is better, equal
// scores order by the lower j. Each lane keeps the K best of its keys, a butterfly over the wave
// merges the lists (bitonic merge of two descending lists), and the K winners are written in
// increasing key order.
template <int K>
__device__ inline void cas_desc(uint32_t (&c)[K], int i, int j) {
  const uint32_t hi = max(c[i], c[j]), lo = min(c[i], c[j]);
  c[i] = hi;
  c[j] = lo;
}

template <int K>
__device__ inline void sort_bitonic_desc(uint32_t (&c)[K]) {
  // c is bitonic: half-cleaners of sizes K, K/2, ..., 2 sort it descending
#pragma unroll
  for (int len = K; len >= 2; len >>= 1)
#pragma unroll
    for (int i = 0; i < K; ++i)
      if ((i % len) < len / 2) cas_desc<K>(c, i, i + len / 2);
}

template <int RC, int K>
__global__ __launch_bounds__(256) void frame_select_small_kernel(FrameTopkParams p) {
  const int lane = tid_x() & 63, w = tid_x() >> 6;
  const int row = bid_y();
  const int nfr = p.F - p.f0;
  const int fs = bid_x() * 4 + w;
  if (fs >= nfr) return;
  const int f = p.f0 + fs;
  const int64_t s0 = (int64_t)f * p.P;
  const int64_t a0 = s0 & ~(int64_t)7;
  const uint16_t* rowp = p.scores + (int64_t)row * p.srs;
  uint32_t c[K];
#pragma unroll
  for (int i = 0; i < K; ++i) c[i] = 0;  // 0 ranks below every key (j < 0xFFFF keeps the low half > 0)
  const int lo_e = (int)(s0 - a0);  // slot 8 (lane + 64 r) + e holds key (that - lo_e) of the frame
#pragma unroll
  for (int r = 0; r < RC; ++r) {
    const int64_t e0 = a0 + 8 * (int64_t)(lane + 64 * r);
    u32x4 v = {0, 0, 0, 0};
    if (e0 < s0 + p.P) v = *reinterpret_cast<const u32x4*>(rowp + e0);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const uint32_t j = (uint32_t)(8 * (lane + 64 * r) + e - lo_e);  // key of the frame (or out of it)
      const uint16_t b = (uint16_t)(v[e >> 1] >> (16 * (e & 1)));
      // keys outside the frame: 0, which ranks below every key (its low half is never 0xFFFF - j)
      const uint32_t y = j < (uint32_t)p.P ? (sortable16(b) << 16) | (0xFFFFu - j) : 0u;
      // insertion into the descending list: every new slot from the old list (independent steps)
#pragma unroll
      for (int i = K - 1; i > 0; --i) c[i] = max(c[i], min(c[i - 1], y));
      c[0] = max(c[0], y);
    }
  }
  // butterfly merge: after step d every lane holds the best K of its 2^d-lane group
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    uint32_t o[K];
#pragma unroll
    for (int i = 0; i < K; ++i) o[i] = (uint32_t)__shfl_xor((int)c[i], d, 64);
#pragma unroll
    for (int i = 0; i < K; ++i) c[i] = max(c[i], o[K - 1 - i]);
    sort_bitonic_desc<K>(c);
  }
  // the k winners (k <= K), in increasing key order: reversed order of the low halves
  const int k = p.k;
  int32_t* out = p.out + (int64_t)row * p.ors + p.ocol + (int64_t)fs * k;
  uint16_t* ok = p.okey ? p.okey + (int64_t)row * p.ors + (int64_t)fs * k : nullptr;
  if (lane < k) {
    // rank of winner `lane` by key index among the k winners
    uint32_t mine = 0;
    int jm = 0;
#pragma unroll
    for (int i = 0; i < K; ++i)
      if (i == lane) mine = c[i];
    jm = 0xFFFF - (int)(mine & 0xFFFFu);
    int rank = 0;
#pragma unroll
    for (int i = 0; i < K; ++i)
      if (i < k) rank += (0xFFFF - (int)(c[i] & 0xFFFFu)) < jm ? 1 : 0;
    out[rank] = (int32_t)(s0 + jm);
    if (ok) ok[rank] = (uint16_t)(mine >> 16);
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
  const int tid = tid_x(), lane = tid & 63, w = tid >> 6;
  const int row = bid_x();
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
  int32_t* o = idx + (int64_t)bid_x() * idx_stride;
  for (int i = tid_x(); i < n; i += 256) o[i] = i * stride;
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
  if (per_frame_mode && per_frame > kMaxPerFrame)
    return fail(SAF3R_ERR_UNSUPPORTED, "saf3r_frame_topk_scores: per_frame must be <= %d", kMaxPerFrame);
  if (score_stride % 8 || (uintptr_t)scores % 16)
    return fail(SAF3R_ERR_INVALID, "saf3r_frame_topk_scores: score rows must be 16-byte aligned (stride %% 8)");
  const bool capped = kept < rest;
  if (per_frame_mode && nfr > 0 && capped && (!cand_idx || !cand_key))
    return fail(SAF3R_ERR_INVALID, "saf3r_frame_topk_scores: the cap needs the candidate buffers");
  if (rows == 0) return SAF3R_OK;
  hipStream_t st = (hipStream_t)stream;
  if (fsel > 0) {
    // the guaranteed first-frame samples 0, s, 2s, ... in the first columns of every row
    hipLaunchKernelGGL(first_samples_kernel, dim3(rows), dim3(256), 0, st, idx, idx_stride, fsel, first_stride);
    if (int e = check_launch("saf3r_frame_topk_scores")) return e;
  }
  if (per_frame_mode && nfr > 0) {
    const int k = min(topk, per_frame);
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
    const int RC = (per_frame / 8 + 2 + 63) / 64;  // 16-byte chunks per lane
#define SAF3R_SMALL(RCV)                                                                                  \
  if (k <= 4) hipLaunchKernelGGL((frame_select_small_kernel<RCV, 4>), grid, dim3(256), 0, st, p);           \
  else hipLaunchKernelGGL((frame_select_small_kernel<RCV, 8>), grid, dim3(256), 0, st, p);
    if (k <= kSmallMaxK) {
      if (RC <= 1) { SAF3R_SMALL(1) }
      else if (RC <= 2) { SAF3R_SMALL(2) }
      else if (RC <= 3) { SAF3R_SMALL(3) }
      else if (RC <= 4) { SAF3R_SMALL(4) }
      else { SAF3R_SMALL(9) }
    } else if (RC <= 1) hipLaunchKernelGGL(frame_select_kernel<1>, grid, dim3(256), 0, st, p);
    else if (RC <= 2) hipLaunchKernelGGL(frame_select_kernel<2>, grid, dim3(256), 0, st, p);
    else if (RC <= 3) hipLaunchKernelGGL(frame_select_kernel<3>, grid, dim3(256), 0, st, p);
    else if (RC <= 4) hipLaunchKernelGGL(frame_select_kernel<4>, grid, dim3(256), 0, st, p);
    else hipLaunchKernelGGL(frame_select_kernel<9>, grid, dim3(256), 0, st, p);
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
