// Shared key sets of the `stride` and `q_probe_topk` modes: one key set per head, attended by
// every query of the head.
//
// ref: saf3r/patch/sparse_attention.py:56-85 (dispatch: q_probe topk = N // stride when the group
//      has a stride, else min(topk, N); include_as defaults False for q_probe, True for stride;
//      start = head % stride with `shift`), :143-186 (q_probe_topk_attention: mean query over
//      every token, fp32 scores qbar . k / sqrt(D), top-k keys, union with the anchor frame and
//      the special tokens, sorted unique set), :256-273 (stride_attention: keys start,
//      start + stride, ..., same union).
//
// Kernels:
//   probe_partial_kernel / probe_finish_kernel: the mean query in a fixed order (chunks of
//     R = ceil(N / 256) tokens summed sequentially, chunk sums added in order, one division).
//   probe_scores_kernel: score[t] = sequential fmaf over d of qbar[d] k[t][d], times 1/sqrt(D).
//   keyset_build_kernel: one work-group per head. Top-k by a 4-pass radix select on the
//     sortable key (ties to the lower index), then the members (top-k or strided, plus the anchor
//     frame and specials) in increasing token order: each wave marks a contiguous run of tokens
//     in LDS masks, one prefix over the waves places the runs, and each wave writes its own.
//   keyset_gather_kernel: compact K rows and transposed, permuted V tiles of the members, in
//     the packed layout the attention kernel reads.
#include <mutex>

#include "common.h"

namespace saf3r {

constexpr int kProbeChunks = 256;
constexpr int kBuildThreads = 1024;

// Packed slot of token t (the inverse of slot_token).
__device__ inline int64_t token_slot(const Geom& g, int64_t t) {
  const int64_t f = t / g.T, r = t % g.T;
  if (r < g.ns) return f * g.ns + r;
  return (int64_t)g.Sp + f * g.Pp + (r - g.ns);
}

struct ProbeParams {
  const float* q;  // fp32 q rows of slot s at q + s * slot_stride, token t at + 64 t
  const float* k;  // fp32 k rows, same layout
  int64_t slot_stride;
  int n;       // tokens
  int n_samp;  // rows of the mean: every token (sample == nullptr) or the listed ones
  const int32_t* sample;
  int chunk;
  int nchunks;
  const int32_t* slots;  // [n_sel] slots of the selected heads
  float* partial;        // [n_sel][kProbeChunks][64]
  float* qbar;           // [n_sel][64]
  float* scores;         // [n_sel][scores_stride]
  int64_t scores_stride;
  float scale;
};

// grid (nchunks, n_sel), 64 threads: feature d of chunk c, summed over the chunk's rows in order.
// Rows are read 64 at a time (independent loads in flight: the chain of adds is cheap, the load
// latency is not) and added in order, so the sum is the sequential one.
constexpr int kProbeBatch = 64;
__global__ __launch_bounds__(64) void probe_partial_kernel(ProbeParams p) {
  const int c = bid_x(), hs = bid_y(), d = tid_x();
  const float* base = p.q + (int64_t)p.slots[hs] * p.slot_stride + d;
  const int i0 = c * p.chunk, i1 = min(p.n_samp, i0 + p.chunk);
  float acc = 0.f;
  int i = i0;
  for (; i + kProbeBatch <= i1; i += kProbeBatch) {
    float x[kProbeBatch];
#pragma unroll
    for (int j = 0; j < kProbeBatch; ++j) {
      const int t = p.sample ? min(max(p.sample[i + j], 0), p.n - 1) : i + j;
      x[j] = base[(int64_t)t * 64];
    }
#pragma unroll
    for (int j = 0; j < kProbeBatch; ++j) acc = acc + x[j];
  }
  for (; i < i1; ++i) {
    const int t = p.sample ? min(max(p.sample[i], 0), p.n - 1) : i;
    acc = acc + base[(int64_t)t * 64];
  }
  p.partial[((int64_t)hs * kProbeChunks + c) * 64 + d] = acc;
}

// grid (n_sel), 64 threads: chunk sums in chunk order (read 64 at a time), then one correctly
// rounded division
__global__ __launch_bounds__(64) void probe_finish_kernel(ProbeParams p) {
  const int hs = bid_x(), d = tid_x();
  const float* part = p.partial + (int64_t)hs * kProbeChunks * 64 + d;
  float total = 0.f;
  int c = 0;
  for (; c + kProbeBatch <= p.nchunks; c += kProbeBatch) {
    float x[kProbeBatch];
#pragma unroll
    for (int j = 0; j < kProbeBatch; ++j) x[j] = part[(int64_t)(c + j) * 64];
#pragma unroll
    for (int j = 0; j < kProbeBatch; ++j) total = total + x[j];
  }
  for (; c < p.nchunks; ++c) total = total + part[(int64_t)c * 64];
  p.qbar[hs * 64 + d] = __fdiv_rn(total, (float)p.n_samp);
}

// grid (ceil(N / 256), n_sel), 256 threads: one token per thread
__global__ __launch_bounds__(256) void probe_scores_kernel(ProbeParams p) {
  __shared__ float qb[64];
  const int hs = bid_y();
  if (tid_x() < 64) qb[tid_x()] = p.qbar[hs * 64 + tid_x()];
  __syncthreads();
  const int t = bid_x() * 256 + tid_x();
  if (t >= p.n) return;
  const f32x4* row = reinterpret_cast<const f32x4*>(p.k + (int64_t)p.slots[hs] * p.slot_stride + (int64_t)t * 64);
  float acc = 0.f;
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    const f32x4 w = row[j];
    acc = __builtin_fmaf(qb[4 * j], w[0], acc);
    acc = __builtin_fmaf(qb[4 * j + 1], w[1], acc);
    acc = __builtin_fmaf(qb[4 * j + 2], w[2], acc);
    acc = __builtin_fmaf(qb[4 * j + 3], w[3], acc);
  }
  p.scores[hs * p.scores_stride + t] = acc * p.scale;
}

struct BuildParams {
  const float* scores;  // [n_heads][scores_stride] (top-k heads)
  int64_t scores_stride;
  const int32_t* mode;   // per head: 0 stride, 1 top-k
  const int32_t* param;  // stride, or k
  const int32_t* start;  // first strided token
  const int32_t* include;
  int n, T, ns;
  int32_t* idx;  // [n_heads][idx_stride]
  int64_t idx_stride;
  int32_t* count;
};

// grid (n_heads), kBuildThreads threads
__global__ __launch_bounds__(kBuildThreads) void keyset_build_kernel(BuildParams p) {
  constexpr int kWaves = kBuildThreads / 64;
  constexpr int kSegChunks = 4096;  // chunks of 64 tokens whose member masks a segment holds
  constexpr int kInFlight = 16;  // score reads per thread in flight in the radix passes
  __shared__ int hist[256];
  __shared__ int wscan[4];
  __shared__ uint64_t fmask[kSegChunks];
  __shared__ int wcnt[kWaves], weq[kWaves];
  __shared__ uint32_t sh_prefix;
  __shared__ int sh_remaining;
  const int hh = bid_x(), tid = tid_x();
  const int mode = p.mode[hh], param = p.param[hh], start = p.start[hh];
  const bool include = p.include[hh] != 0;
  const float* sc = p.scores + (int64_t)hh * p.scores_stride;

  // ---- top-k: threshold key by radix select (most significant digit first) ----
  // (a non-positive k or stride selects no token)
  uint32_t thr = 0xFFFFFFFFu;
  int need_eq = 0;
  if (mode == 1 && param > 0) {
    const int k = min(param, p.n);
    uint32_t prefix = 0, mask = 0;
    int remaining = k;
    for (int shift = 24; shift >= 0; shift -= 8) {
      if (tid < 256) hist[tid] = 0;
      __syncthreads();
      // kInFlight scores per thread read at once, then their counts
      for (int t0 = tid; t0 < p.n; t0 += kInFlight * kBuildThreads) {
        float v[kInFlight];
#pragma unroll
        for (int u = 0; u < kInFlight; ++u) {
          const int t = t0 + u * kBuildThreads;
          v[u] = t < p.n ? sc[t] : 0.f;
        }
#pragma unroll
        for (int u = 0; u < kInFlight; ++u) {
          const uint32_t key = fkey(v[u]);
          if (t0 + u * kBuildThreads < p.n && (key & mask) == prefix) atomicAdd(&hist[(key >> shift) & 255], 1);
        }
      }
      __syncthreads();
      // the bin of the remaining-th largest key: thread i < 256 holds bin 255 - i; inclusive sums
      // from the top over the four waves of those threads, and the one thread whose bin reaches
      // `remaining` first records it
      int cnt = 0, inc = 0;
      if (tid < 256) {
        cnt = hist[255 - tid];
        inc = cnt;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
          const int y = __shfl_up(inc, o);
          if ((tid & 63) >= o) inc += y;
        }
        if ((tid & 63) == 63) wscan[tid >> 6] = inc;
      }
      __syncthreads();
      if (tid < 256) {
        for (int i = 0; i < (tid >> 6); ++i) inc += wscan[i];
        const int excl = inc - cnt;
        if (excl < remaining && inc >= remaining) {
          sh_prefix = prefix | ((uint32_t)(255 - tid) << shift);
          sh_remaining = remaining - excl;
        }
      }
      __syncthreads();
      prefix = sh_prefix;
      remaining = sh_remaining;
      mask |= 255u << shift;
      __syncthreads();
    }
    thr = prefix;        // key of the k-th best token
    need_eq = remaining; // how many tokens with exactly that key are taken (lowest indices)
  }

  // ---- members in token order: select, union, compact ----
  // Segments of up to kSegChunks chunks of 64 tokens; wave w takes a contiguous run of a segment's
  // chunks. Top-k heads first count their keys equal to the threshold per wave (their ranks among
  // those keys decide which are taken); then every wave computes its chunks' member masks into
  // LDS and counts them, one prefix over the waves places each wave's members, and the wave writes
  // them from its masks: three barriers per segment instead of two prefix steps per 1024 tokens.
  int32_t* out = p.idx + (int64_t)hh * p.idx_stride;
  const int lane = tid & 63, w = tid >> 6;
  int run_eq = 0, run_out = 0;  // equal keys and members before the segment
  for (int seg0 = 0; seg0 < p.n; seg0 += kSegChunks * 64) {
    const int nch = (min(p.n - seg0, kSegChunks * 64) + 63) / 64;
    const int per = (nch + kWaves - 1) / kWaves;
    const int c0 = min(nch, w * per), c1 = min(nch, c0 + per);
    // the score of chunk c's token for this lane (0 outside the head's tokens)
    auto key_at = [&](int c) {
      const int t = seg0 + 64 * c + lane;
      return t < p.n ? fkey(sc[t]) : 0u;
    };
    int eq_before = run_eq, seg_eq = 0;
    if (mode == 1) {
      int e = 0;
      for (int c = c0; c < c1; c += 8) {  // eight chunks' scores in flight at once
        uint32_t kk[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) kk[u] = c + u < c1 ? key_at(c + u) : 0u;
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const int t = seg0 + 64 * (c + u) + lane;
          e += __popcll(__ballot(c + u < c1 && t < p.n && kk[u] == thr));
        }
      }
      if (lane == 0) weq[w] = e;
      __syncthreads();
      for (int i = 0; i < kWaves; ++i) {
        const int v = weq[i];
        eq_before += i < w ? v : 0;
        seg_eq += v;
      }
    }
    int cnt = 0, eqr = eq_before;  // rank of the wave's next key equal to the threshold
    // t mod T and (t - start) mod stride of the lane's token, stepped by 64 tokens per chunk (no
    // division in the loop)
    const int t_first = seg0 + 64 * c0 + lane;
    int rT = t_first % p.T;
    const int stepT = 64 % p.T;
    const int stride = (mode == 0 && param > 0) ? param : 1;
    int rS = t_first >= start ? (t_first - start) % stride : 0;
    const int stepS = 64 % stride;
    for (int c = c0; c < c1; c += 8) {
      uint32_t kk[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) kk[u] = (mode == 1 && c + u < c1) ? key_at(c + u) : 0u;
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        if (c + u >= c1) break;  // uniform
        const int t = seg0 + 64 * (c + u) + lane;
        const bool valid = t < p.n;
        bool sel;
        if (mode == 1) {
          const bool eq = valid && kk[u] == thr;
          const uint64_t meq = __ballot(eq);
          const int rank = eqr + (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(meq >> 32),
                                                                __builtin_amdgcn_mbcnt_lo((uint32_t)meq, 0));
          eqr += __popcll(meq);
          sel = valid && param > 0 && (kk[u] > thr || (eq && rank < need_eq));
        } else {
          sel = valid && param > 0 && t >= start && rS == 0;
        }
        const bool flag = sel || (include && valid && (t < p.T || rT < p.ns));
        const uint64_t m = __ballot(flag);
        if (lane == 0) fmask[c + u] = m;
        cnt += __popcll(m);
        // the next chunk's token, t + 64 (below start the residue is not used)
        rT += stepT;
        if (rT >= p.T) rT -= p.T;
        if (t + 64 >= start) {
          rS = t >= start ? rS + stepS : (t + 64 - start) % stride;
          if (rS >= stride) rS -= stride;
        }
      }
    }
    if (lane == 0) wcnt[w] = cnt;
    __syncthreads();
    int pos = run_out, seg_out = 0;
    for (int i = 0; i < kWaves; ++i) {
      const int v = wcnt[i];
      pos += i < w ? v : 0;
      seg_out += v;
    }
    for (int c = c0; c < c1; ++c) {
      const uint64_t m = fmask[c];
      if ((m >> lane) & 1)
        out[pos + (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0))] =
            seg0 + 64 * c + lane;
      pos += __popcll(m);
    }
    run_out += seg_out;
    run_eq += seg_eq;
    __syncthreads();  // the next segment rewrites the masks and the wave counts
  }
  if (tid == 0) p.count[hh] = run_out;
}

struct GatherKParams {
  const __bf16* k;  // packed K
  Geom g;
  const int32_t* head_ids;
  const __bf16* v;  // natural V rows
  int64_t v_tok_stride, v_head_stride;
  const int32_t* idx;
  int64_t idx_stride;
  const int32_t* count;
  __bf16* kc;  // [n_sel][capacity][64]
  __bf16* vc;  // [n_sel][capacity / 64][64][64] transposed, permuted tiles
  int64_t capacity;
};

// grid (tiles, n_sel), 256 threads; four threads per key row, 16 features each (as the packing
// kernel). Tiles at or beyond the member count are skipped; rows beyond it are zero.
__global__ __launch_bounds__(256) void keyset_gather_kernel(GatherKParams p) {
  __shared__ __align__(16) __bf16 vs[64 * 72];
  const int tile = bid_x(), hs = bid_y();
  const int cnt = p.count[hs];
  if (tile * 64 >= cnt) return;
  const int h = p.head_ids[hs];
  const int t = tid_x(), row = t >> 2, c = t & 3;
  const int j = tile * 64 + row;
  const int64_t tok = j < cnt ? p.idx[hs * p.idx_stride + j] : -1;
  u32x4 a = {0, 0, 0, 0}, b = {0, 0, 0, 0};
  if (tok >= 0) {
    const u32x4* s4 =
        reinterpret_cast<const u32x4*>(p.k + ((int64_t)h * p.g.L + token_slot(p.g, tok)) * 64 + 16 * c);
    a = s4[0];
    b = s4[1];
  }
  u32x4* d4 = reinterpret_cast<u32x4*>(p.kc + ((int64_t)hs * p.capacity + j) * 64 + 16 * c);
  d4[0] = a;
  d4[1] = b;

  u32x4 va = {0, 0, 0, 0}, vb = {0, 0, 0, 0};
  if (tok >= 0) {
    const u32x4* s4 = reinterpret_cast<const u32x4*>(p.v + tok * p.v_tok_stride + h * p.v_head_stride + 16 * c);
    va = s4[0];
    vb = s4[1];
  }
  u32x4* l4 = reinterpret_cast<u32x4*>(vs + row * 72 + 16 * c);
  l4[0] = va;
  l4[1] = vb;
  __syncthreads();
  // transposed tile: row i = feature phi(i), column position kappa(key); see the packing kernel
  const int i = t >> 2, ii = i & 31;
  const int dd = 32 * (i >> 5) + 16 * ((ii >> 2) & 1) + 4 * (ii >> 3) + (ii & 3);
  uint32_t wv[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int c0 = 16 * c + 2 * e, c1 = c0 + 1;
    const int k0 = (c0 & ~12) | ((c0 & 4) << 1) | ((c0 & 8) >> 1);
    const int k1 = (c1 & ~12) | ((c1 & 4) << 1) | ((c1 & 8) >> 1);
    const uint16_t lo = __builtin_bit_cast(uint16_t, vs[k0 * 72 + dd]);
    const uint16_t hi = __builtin_bit_cast(uint16_t, vs[k1 * 72 + dd]);
    wv[e] = (uint32_t)lo | ((uint32_t)hi << 16);
  }
  u32x4* o4 = reinterpret_cast<u32x4*>(p.vc + ((int64_t)hs * p.capacity + (int64_t)tile * 64) * 64 + i * 64 + 16 * c);
  o4[0] = u32x4{wv[0], wv[1], wv[2], wv[3]};
  o4[1] = u32x4{wv[4], wv[5], wv[6], wv[7]};
}

}  // namespace saf3r

using namespace saf3r;

// Checks the arguments of both probe entries and fills everything but the workspace pointer.
// Checks the arguments of both probe entries and fills everything but the workspace pointer.
static int probe_setup(const char* who, const float* q32, const float* k32, int64_t slot_stride, int n_tokens,
                       const int32_t* slots, int n_sel, const int32_t* sample_idx, int n_samples, float scale,
                       float* qbar, float* scores, int64_t scores_stride, ProbeParams* pp) {
  ProbeParams& p = *pp;
  if (!q32 || !k32 || !slots || !qbar || !scores) return fail(SAF3R_ERR_INVALID, "%s: null pointer", who);
  if (n_tokens <= 0) return fail(SAF3R_ERR_INVALID, "%s: n_tokens must be positive", who);
  if (n_sel <= 0 || n_sel > 65535 || scores_stride < n_tokens || slot_stride < (int64_t)n_tokens * 64)
    return fail(SAF3R_ERR_INVALID, "%s: bad n_sel %d, slot_stride or scores_stride", who, n_sel);
  if (sample_idx && (n_samples <= 0 || n_samples > n_tokens))
    return fail(SAF3R_ERR_INVALID, "%s: n_samples must be in [1, %d]", who, n_tokens);
  if (((uintptr_t)q32 | (uintptr_t)k32) % 16 || slot_stride % 4)
    return fail(SAF3R_ERR_INVALID, "%s: fp32 rows must be 16-byte aligned (slot_stride %% 4)", who);
  p.q = q32;
  p.k = k32;
  p.slot_stride = slot_stride;
  p.n = n_tokens;
  p.sample = sample_idx;
  p.n_samp = sample_idx ? n_samples : n_tokens;
  p.chunk = (p.n_samp + kProbeChunks - 1) / kProbeChunks;
  p.nchunks = (p.n_samp + p.chunk - 1) / p.chunk;
  p.slots = slots;
  p.partial = nullptr;
  p.qbar = qbar;
  p.scores = scores;
  p.scores_stride = scores_stride;
  p.scale = scale;
  return SAF3R_OK;
}

static int probe_launch(const ProbeParams& p, int n_sel, void* stream) {
  hipStream_t s = (hipStream_t)stream;
  hipLaunchKernelGGL(probe_partial_kernel, dim3(p.nchunks, n_sel), dim3(64), 0, s, p);
  hipLaunchKernelGGL(probe_finish_kernel, dim3(n_sel), dim3(64), 0, s, p);
  hipLaunchKernelGGL(probe_scores_kernel, dim3((unsigned)((p.n + 255) / 256), n_sel), dim3(256), 0, s, p);
  return check_launch("saf3r_probe_scores");
}

extern "C" int saf3r_probe_scores(const float* q32, const float* k32, int64_t slot_stride, int n_tokens,
                                  const int32_t* slots, int n_sel, const int32_t* sample_idx, int n_samples,
                                  float scale, float* partial, float* qbar, float* scores, int64_t scores_stride,
                                  void* stream) {
  if (int e = injected("saf3r_probe_scores")) return e;
  ProbeParams p;
  if (int e = probe_setup("saf3r_probe_scores", q32, k32, slot_stride, n_tokens, slots, n_sel, sample_idx, n_samples,
                          scale, qbar, scores, scores_stride, &p))
    return e;
  if (!partial) return fail(SAF3R_ERR_INVALID, "saf3r_probe_scores: null workspace");
  p.partial = partial;
  return probe_launch(p, n_sel, stream);
}

// ---- allocation-free probe entry ------------------------------------------------------------
// The partial sums of saf3r_probe_scores_noalloc live in this file-scope device array (one copy per
// GPU, held until the process ends) instead of a caller workspace. Host code never passes the array's
// name to a kernel: its device address on the GPU of the call's stream comes from
// hipGetSymbolAddress, resolved once per device and kept in scratch_addr. Every chunk sum the finish kernel reads is written by the
// partial kernel of the same call first, so nothing needs clearing; calls that overlap on one GPU
// (different streams, or several host threads) share the array and race.
constexpr int kScratchHeads = 64;
constexpr int kMaxDevices = 64;
static __device__ __align__(256) float scratch[kScratchHeads * kProbeChunks * 64];  // 4 MiB

static std::mutex scratch_mu;
static float* scratch_addr[kMaxDevices];  // per device, set once

// The array of the device `stream` belongs to (the current device for the NULL stream): each GPU
// holds its own copy at its own address, which hipGetSymbolAddress reports for the current device,
// so the lookup runs with that device current and restores the caller's device afterwards.
static int scratch_ptr(const char* who, hipStream_t stream, float** out) {
  int cur = -1, dev = -1;
  if (hipGetDevice(&cur) != hipSuccess || cur < 0)
    return fail(SAF3R_ERR_LAUNCH, "%s: no current device", who);
  dev = cur;
  if (stream) {
    hipDevice_t sd = -1;
    if (hipStreamGetDevice(stream, &sd) != hipSuccess || sd < 0)
      return fail(SAF3R_ERR_INVALID, "%s: the stream's device could not be determined", who);
    dev = (int)sd;
  }
  if (dev >= kMaxDevices) return fail(SAF3R_ERR_UNSUPPORTED, "%s: device id %d >= %d", who, dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(scratch_mu);
  if (!scratch_addr[dev]) {
    if (dev != cur && hipSetDevice(dev) != hipSuccess)
      return fail(SAF3R_ERR_LAUNCH, "%s: cannot make device %d current", who, dev);
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (dev != cur) (void)hipSetDevice(cur);
    if (e != hipSuccess || !ptr)
      return fail(SAF3R_ERR_LAUNCH, "%s: hipGetSymbolAddress of the static workspace failed on device %d: %s", who,
                  dev, hipGetErrorString(e));
    scratch_addr[dev] = static_cast<float*>(ptr);
  }
  *out = scratch_addr[dev];
  return SAF3R_OK;
}

extern "C" int saf3r_probe_scores_noalloc(const float* q32, const float* k32, int64_t slot_stride, int n_tokens,
                                          const int32_t* slots, int n_sel, const int32_t* sample_idx, int n_samples,
                                          float scale, float* qbar, float* scores, int64_t scores_stride,
                                          void* stream) {
  const char* who = "saf3r_probe_scores_noalloc";
  if (int e = injected(who)) return e;
  ProbeParams p;
  if (int e = probe_setup(who, q32, k32, slot_stride, n_tokens, slots, n_sel, sample_idx, n_samples, scale, qbar,
                          scores, scores_stride, &p))
    return e;
  if (n_sel > kScratchHeads)
    return fail(SAF3R_ERR_UNSUPPORTED, "%s: n_sel %d exceeds the %d heads of the static workspace", who, n_sel,
                kScratchHeads);
  float* ws = nullptr;
  if (int e = scratch_ptr(who, (hipStream_t)stream, &ws)) return e;
  p.partial = ws;
  return probe_launch(p, n_sel, stream);
}

extern "C" int saf3r_keyset_build(const float* scores, int64_t scores_stride, int n_heads, const int32_t* mode,
                                  const int32_t* param, const int32_t* start, const int32_t* include, int frames,
                                  int tokens_per_frame, int num_special, int32_t* idx, int64_t idx_stride,
                                  int32_t* count, void* stream) {
  if (int e = injected("saf3r_keyset_build")) return e;
  Geom g;
  if (!make_geom(frames, tokens_per_frame, num_special, &g))
    return fail(SAF3R_ERR_INVALID, "saf3r_keyset_build: invalid geometry");
  const int64_t n = (int64_t)frames * tokens_per_frame;
  if (n > 0x7fffffff) return fail(SAF3R_ERR_UNSUPPORTED, "saf3r_keyset_build: too many tokens");
  if (n_heads <= 0 || n_heads > 65535) return fail(SAF3R_ERR_INVALID, "saf3r_keyset_build: bad n_heads %d", n_heads);
  if (!mode || !param || !start || !include || !idx || !count)
    return fail(SAF3R_ERR_INVALID, "saf3r_keyset_build: null pointer");
  if (idx_stride < n) return fail(SAF3R_ERR_INVALID, "saf3r_keyset_build: idx_stride below the token count");
  BuildParams p;
  p.scores = scores;
  p.scores_stride = scores_stride;
  p.mode = mode;
  p.param = param;
  p.start = start;
  p.include = include;
  p.n = (int)n;
  p.T = tokens_per_frame;
  p.ns = num_special;
  p.idx = idx;
  p.idx_stride = idx_stride;
  p.count = count;
  hipLaunchKernelGGL(keyset_build_kernel, dim3(n_heads), dim3(kBuildThreads), 0, (hipStream_t)stream, p);
  return check_launch("saf3r_keyset_build");
}

extern "C" int saf3r_keyset_gather(const void* k_packed, int frames, int tokens_per_frame, int num_special,
                                   const int32_t* head_ids, int n_sel, const void* v, int64_t v_tok_stride,
                                   int64_t v_head_stride, const int32_t* idx, int64_t idx_stride,
                                   const int32_t* count, int max_tiles, void* keyset_k, void* keyset_v,
                                   int64_t capacity, void* stream) {
  if (int e = injected("saf3r_keyset_gather")) return e;
  GatherKParams p;
  if (!make_geom(frames, tokens_per_frame, num_special, &p.g))
    return fail(SAF3R_ERR_INVALID, "saf3r_keyset_gather: invalid geometry");
  if (!k_packed || !head_ids || !v || !idx || !count || !keyset_k || !keyset_v)
    return fail(SAF3R_ERR_INVALID, "saf3r_keyset_gather: null pointer");
  if (n_sel <= 0 || n_sel > 65535 || max_tiles <= 0 || capacity % 64 || (int64_t)max_tiles * 64 > capacity)
    return fail(SAF3R_ERR_INVALID, "saf3r_keyset_gather: bad n_sel %d, max_tiles %d or capacity %lld", n_sel,
                max_tiles, (long long)capacity);
  if (v_tok_stride % 8 || v_head_stride % 8 || ((uintptr_t)v | (uintptr_t)k_packed) % 16 ||
      ((uintptr_t)keyset_k | (uintptr_t)keyset_v) % 16)
    return fail(SAF3R_ERR_INVALID, "saf3r_keyset_gather: 16-byte alignment required");
  p.k = (const __bf16*)k_packed;
  p.head_ids = head_ids;
  p.v = (const __bf16*)v;
  p.v_tok_stride = v_tok_stride;
  p.v_head_stride = v_head_stride;
  p.idx = idx;
  p.idx_stride = idx_stride;
  p.count = count;
  p.kc = (__bf16*)keyset_k;
  p.vc = (__bf16*)keyset_v;
  p.capacity = capacity;
  hipLaunchKernelGGL(keyset_gather_kernel, dim3(max_tiles, n_sel), dim3(256), 0, (hipStream_t)stream, p);
  return check_launch("saf3r_keyset_gather");
}
