// Gather attention over per-row key lists (the image rows of the reference dino_topk heads).
//
// ref: saf3r/triton/sparse_topk_attention.py:36-112 (one program per query: gathered K rows,
//      fp32 scores, exact max-subtracted softmax, fp32 P.V, output in v.dtype), :115-166 (API:
//      q [N, D], k/v [Nk, D], kv_indices [N, TopK], scale default 1/sqrt(D); a stride-0 index view
//      shares one list across rows), :173-258 (online-softmax variant for TopK > 2048).
// The work is one gathered K row and one V row per (query, listed key): bound by the cache
// bandwidth of those row reads, not by arithmetic (a list is one query's own, so there is no
// matrix product to share between queries). A wave owns two query rows (32 lanes each) and walks
// their lists in steps of ENT entries with an fp32 online softmax, so any list length is handled by
// the same kernel. Lane l of a row's 32 serves key slot ks = l / 8 of every group of 4 keys and dims
// 8 dg .. 8 dg + 7 (dg = l % 8): 8 lanes read a K or V row together (32 bytes each of an fp32 K row,
// 16 of a bf16 row), so one load instruction moves 8 whole rows (4 of each query), and the 8 partial
// dot products of a row are summed by three DPP steps inside the 8 lanes. Entries < 0 or >= num_keys are skipped. q and k
// are bf16 or fp32 rows (the reference's kernel upcasts either); v and out are bf16 or fp32 rows
// (the reference writes out in v.dtype from its fp32 accumulator).
//
// Walk order: the rows are shared by many queries (at the dino-head shape each key row is in about
// 512 lists), but a list spans every frame, far more than an L2 holds. So the waves resident at one
// moment walk the same window of list positions: row r starts its walk at step
// s0 = max(0, r - C) * nsteps / C (mod nsteps), C = the rows the GPU holds at once (resident waves,
// from the kernel's occupancy, times rows per wave). Waves are dispatched in row order and take
// about the same time, so when row r starts, the rows still running started one step time apart per
// C / nsteps rows and stand at the step r does: every resident wave reads the rows of the same few
// steps. The order depends on r alone, so results are run-to-run identical.
#include "common.h"

namespace saf3r {

// Row addressing (saf3r_rows) with the frame index r / rows_per_frame taken by a multiply-high:
// for 0 <= r < 2^31 and a divisor 1 <= d < 2^31, with s = ceil(log2 d) and
// m = floor(2^32 (2^s - d) / d) + 1 (< 2^32), r / d = (mulhi(m, r) + r) >> s (Granlund and
// Montgomery, "Division by invariant integers using multiplication", 1994). Row numbers here are
// below 2^31 (the entry rejects larger key counts). rows_per_frame >= 2^31 (all rows one frame)
// takes frame 0 (shift -1).
struct RowsDev {
  const void* ptr;
  int64_t row_stride, base_row, rows_per_frame, frame_row_stride;
  uint32_t magic;
  int shift;
  template <typename T = __bf16>
  __device__ inline const T* row(int64_t r) const {
    const uint32_t u = (uint32_t)r;
    const int64_t f = shift < 0 ? 0 : (int64_t)((__umulhi(magic, u) + u) >> shift);
    return static_cast<const T*>(ptr) + (base_row + f * frame_row_stride + (r - f * rows_per_frame)) * row_stride;
  }
};

static void set_divisor(RowsDev* d) {
  if (d->rows_per_frame >= ((int64_t)1 << 31)) {
    d->shift = -1;
    d->magic = 0;
    return;
  }
  const uint64_t dv = (uint64_t)d->rows_per_frame;
  int sh = 0;
  while (((uint64_t)1 << sh) < dv) ++sh;
  d->shift = sh;
  d->magic = (uint32_t)((((uint64_t)1 << 32) * (((uint64_t)1 << sh) - dv)) / dv + 1);
}

struct GatherParams {
  RowsDev q, k, v, out;
  const int32_t* idx;
  int64_t idx_stride;
  int n, topk;
  int64_t nk;
  float c;          // scale * log2(e)
  int64_t resident; // C: waves resident on the GPU at once (walk order only)
  float* part;      // sliced mode: partial results [n][kGatherSlices][66] of the rows of this launch
  int64_t r0;       // sliced mode: the first row of this launch (rows r0 .. r0 + n - 1)
};

constexpr int kGatherSlices = 8;  // sliced mode: list slices, a multiple of the 8 XCDs

// sum of x over the 8 lanes of this lane's group (quad swaps, then the mirrored quad of the group)
__device__ inline float sum8(float x) {
  x += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), 0xB1, 0xF, 0xF, true));
  x += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), 0x4E, 0xF, 0xF, true));
  x += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), 0x141, 0xF, 0xF, true));
  return x;
}
// reductions over the key slots of a query's LANES lanes (lanes dg, dg + 8, ... of its group)
template <int LANES = 64>
__device__ inline float slots_max(float x) {
#pragma unroll
  for (int o = 8; o < LANES; o <<= 1) x = fmaxf(x, __shfl_xor(x, o));
  return x;
}
template <int LANES = 64>
__device__ inline float slots_sum(float x) {
#pragma unroll
  for (int o = 8; o < LANES; o <<= 1) x += __shfl_xor(x, o);
  return x;
}

// 4 waves per workgroup, QPW query rows per wave (each on 64 / QPW lanes: its key slots are 8 / QPW
// groups of 8 lanes). Two rows per wave put twice the rows of a walk step in flight at once, so the
// L2 serves more reads of the step's key rows between two fetches of them. QK32: q and k rows are
// fp32 (the reference's gather reads the fp32 q / k of the autocast forward and multiplies in fp32);
// otherwise bf16. V32 / O32: v / out rows are fp32; otherwise bf16.
template <bool QK32, bool V32, bool O32, int ENT, bool SLICED, int QPW>
__global__ __launch_bounds__(256) void gather_attn_kernel(GatherParams p) {
  static_assert(QPW == 1 || QPW == 2, "one or two rows per wave");
  constexpr int LANES = 64 / QPW;       // lanes of one row
  constexpr int SLOTS = LANES / 8;      // key slots of one row
  constexpr int NIT = ENT / SLOTS;      // groups of SLOTS keys per step
  static_assert(ENT <= LANES && ENT % SLOTS == 0, "a step's entries sit in the row's lanes");
  const int lane = tid_x() & 63, w = tid_x() >> 6, dg = lane & 7;
  const int qh = lane / LANES, qbase = qh * LANES, ks = (lane - qbase) >> 3;
  constexpr int RPW = 4 * QPW;  // rows per workgroup
  // sliced: workgroup b takes rows RPW g .. RPW g + RPW - 1, g = (b / 8) % G (G = ceil(n / RPW)),
  // of slice (b % 8) + 8 (b / 8G): slice s runs on XCD s % 8, the XCD's slices one after the other
  const int64_t ng = (p.n + RPW - 1) / RPW;
  const int slice = SLICED ? (int)(bid_x() % 8 + 8 * (bid_x() / (8 * ng))) : 0;
  const int64_t rw = (SLICED ? (int64_t)(bid_x() / 8) % ng : (int64_t)bid_x()) * RPW + w * QPW;  // the wave's first row
  if (rw >= p.n) return;  // a whole wave leaves; the kernel has no barrier
  const int64_t rl_raw = rw + qh;  // row of this launch (this lane's half)
  const bool rvalid = rl_raw < p.n;  // a second row past the end computes on the first's and stores nothing
  const int64_t rl = rvalid ? rl_raw : rw;
  const int64_t r = SLICED ? p.r0 + rl : rl;

  // this lane's 8 dims of q: fp32 values (QK32) or bf16 pairs
  float qv[8];
  uint32_t qw[4];
  if constexpr (QK32) {
    const f32x4* q4 = reinterpret_cast<const f32x4*>(p.q.row<float>(r) + 8 * dg);
    const f32x4 a = q4[0], b = q4[1];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      qv[e] = a[e];
      qv[4 + e] = b[e];
    }
  } else {
    const u32x4 x = *reinterpret_cast<const u32x4*>(p.q.row(r) + 8 * dg);
    qw[0] = x.x;
    qw[1] = x.y;
    qw[2] = x.z;
    qw[3] = x.w;
  }
  float acc[8];
#pragma unroll
  for (int d = 0; d < 8; ++d) acc[d] = 0.f;
  float m_run = -__builtin_inff(), l_run = 0.f;
  // this wave's part of the list: entries [e_begin, e_end)
  const int per = SLICED ? (p.topk + kGatherSlices - 1) / kGatherSlices : p.topk;
  const int e_begin = SLICED ? min(p.topk, slice * per) : 0, e_end = SLICED ? min(p.topk, e_begin + per) : p.topk;
  const int32_t* il = p.idx + r * p.idx_stride + e_begin;
  const int len = e_end - e_begin;

  const int nsteps = max(1, (len + ENT - 1) / ENT);
  // rows resident at once (waves x rows per wave)
  const int64_t res = (SLICED ? max((int64_t)1, p.resident / kGatherSlices) : p.resident) * QPW;
  const int s0 = rl < res ? 0 : (int)(((rl - res) * nsteps / res) % nsteps);
  // entry st * ENT + l of the part, in the row's lane qbase + l, l < ENT (-1 past it or out of range)
  auto entry = [&](int st) {  // (range-checked where it is used)
    const int li = lane - qbase;
    const int e = st * ENT + (li & (ENT - 1));
    return (li < ENT && e < len) ? il[e] : -1;
  };
  int next_id = entry(s0);  // each step's entries are read one step ahead
  for (int sc = 0, st = s0; sc < nsteps; ++sc) {
    const int myid = next_id < p.nk ? next_id : -1;
    st = st + 1 == nsteps ? 0 : st + 1;
    if (sc + 1 < nsteps) next_id = entry(st);
    // key SLOTS it + ks of the step: its score and its V dims
    float s[NIT];
    float vf[NIT][8];     // V32: the V dims of key slot it
    uint32_t vw[NIT][4];  // otherwise the same dims as bf16 pairs
#pragma unroll
    for (int it = 0; it < NIT; ++it) {
      const int id = __shfl(myid, qbase + SLOTS * it + ks);
      const int64_t rid = id >= 0 ? id : 0;  // a masked entry reads row 0; its score is dropped
      float part = 0.f;
      if constexpr (QK32) {
        const f32x4* k4 = reinterpret_cast<const f32x4*>(p.k.row<float>(rid) + 8 * dg);
        const f32x4 a = k4[0], b = k4[1];
#pragma unroll
        for (int e = 0; e < 4; ++e) part = __builtin_fmaf(qv[e], a[e], part);
#pragma unroll
        for (int e = 0; e < 4; ++e) part = __builtin_fmaf(qv[4 + e], b[e], part);
      } else {
        const u32x4 kx = *reinterpret_cast<const u32x4*>(p.k.row(rid) + 8 * dg);
        // elements are copied to scalars before the bf16x2 bit_cast: a bit_cast applied directly to
        // a vector element (kx[e]) was lowered to element 0 for every e by this compiler
        const uint32_t kw[4] = {kx.x, kx.y, kx.z, kx.w};
#pragma unroll
        for (int e = 0; e < 4; ++e)
          part = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, kw[e]), __builtin_bit_cast(bf16x2, qw[e]),
                                                 part, false);
      }
      if constexpr (V32) {
        const f32x4* v4 = reinterpret_cast<const f32x4*>(p.v.row<float>(rid) + 8 * dg);
        const f32x4 a = v4[0], b = v4[1];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          vf[it][e] = a[e];
          vf[it][4 + e] = b[e];
        }
      } else {
        const u32x4 vx = *reinterpret_cast<const u32x4*>(p.v.row(rid) + 8 * dg);
        vw[it][0] = vx.x;
        vw[it][1] = vx.y;
        vw[it][2] = vx.z;
        vw[it][3] = vx.w;
      }
      part = sum8(part);
      s[it] = id >= 0 ? part : -__builtin_inff();
    }
    float mx = s[0];
#pragma unroll
    for (int it = 1; it < NIT; ++it) mx = fmaxf(mx, s[it]);
    mx = slots_max<LANES>(mx);
    const float m_new = fmaxf(m_run, mx);
    const float m_use = m_new == -__builtin_inff() ? 0.f : m_new;
    const float alpha = __builtin_amdgcn_exp2f((m_run - m_use) * p.c);
#pragma unroll
    for (int d = 0; d < 8; ++d) acc[d] *= alpha;
    float lsum = 0.f;
#pragma unroll
    for (int it = 0; it < NIT; ++it) {
      const float pj = __builtin_amdgcn_exp2f(__builtin_fmaf(s[it], p.c, -m_use * p.c));
      lsum += pj;
      if constexpr (V32) {
#pragma unroll
        for (int d = 0; d < 8; ++d) acc[d] = __builtin_fmaf(pj, vf[it][d], acc[d]);
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          acc[2 * e] = __builtin_fmaf(pj, bf16_lo(vw[it][e]), acc[2 * e]);
          acc[2 * e + 1] = __builtin_fmaf(pj, bf16_hi(vw[it][e]), acc[2 * e + 1]);
        }
      }
    }
    l_run = l_run * alpha + slots_sum<LANES>(lsum);
    m_run = m_new;
  }

  // sum the key slots' partial outputs; lanes of slot 0 store dims 8 dg .. 8 dg + 7
#pragma unroll
  for (int d = 0; d < 8; ++d) acc[d] = slots_sum<LANES>(acc[d]);
  if (!rvalid) return;
  if constexpr (SLICED) {  // the slice's unnormalised sum, its maximum and its sum of weights
    float* pr = p.part + (rl * kGatherSlices + slice) * 66;
    if (ks == 0) {
      *reinterpret_cast<f32x4*>(pr + 8 * dg) = f32x4{acc[0], acc[1], acc[2], acc[3]};
      *reinterpret_cast<f32x4*>(pr + 8 * dg + 4) = f32x4{acc[4], acc[5], acc[6], acc[7]};
    }
    if (lane == qbase) {
      pr[64] = m_run;
      pr[65] = l_run;
    }
    return;
  }
  if (ks == 0) {
    const float inv = l_run > 0.f ? 1.0f / l_run : 0.f;
    if constexpr (O32) {
      float* orow = const_cast<float*>(p.out.row<float>(r)) + 8 * dg;
      *reinterpret_cast<f32x4*>(orow) = f32x4{acc[0] * inv, acc[1] * inv, acc[2] * inv, acc[3] * inv};
      *reinterpret_cast<f32x4*>(orow + 4) = f32x4{acc[4] * inv, acc[5] * inv, acc[6] * inv, acc[7] * inv};
    } else {
      uint32_t o[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const bf16x2 pr = {(__bf16)(acc[2 * e] * inv), (__bf16)(acc[2 * e + 1] * inv)};
        o[e] = __builtin_bit_cast(uint32_t, pr);
      }
      __bf16* orow = const_cast<__bf16*>(p.out.row<__bf16>(r));
      *reinterpret_cast<u32x4*>(orow + 8 * dg) = u32x4{o[0], o[1], o[2], o[3]};
    }
  }
}

// Sliced mode, second pass: one wave per row; lane (slice = l / 8, dg = l % 8) reads the slice's dims
// 8 dg .. 8 dg + 7, rescales them to the row's maximum and the 8 slices are summed.
template <bool O32>
__global__ __launch_bounds__(256) void gather_merge_kernel(GatherParams p) {
  const int lane = tid_x() & 63, w = tid_x() >> 6, sl = lane >> 3, dg = lane & 7;
  const int64_t rl = (int64_t)bid_x() * 4 + w, r = p.r0 + rl;
  if (rl >= p.n) return;
  constexpr int H = kGatherSlices / 8;  // slices per lane: sl, sl + 8, ...
  f32x4 a[H], b[H];
  float m[H], l[H], mx = -__builtin_inff();
#pragma unroll
  for (int j = 0; j < H; ++j) {
    const float* pr = p.part + (rl * kGatherSlices + sl + 8 * j) * 66;
    a[j] = *reinterpret_cast<const f32x4*>(pr + 8 * dg);
    b[j] = *reinterpret_cast<const f32x4*>(pr + 8 * dg + 4);
    m[j] = pr[64];
    l[j] = pr[65];
    mx = fmaxf(mx, m[j]);
  }
  mx = slots_max(mx);
  float acc[8] = {}, lt = 0.f;
#pragma unroll
  for (int j = 0; j < H; ++j) {
    const float sc = mx == -__builtin_inff() ? 0.f : __builtin_amdgcn_exp2f((m[j] - mx) * p.c);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      acc[e] = __builtin_fmaf(a[j][e], sc, acc[e]);
      acc[4 + e] = __builtin_fmaf(b[j][e], sc, acc[4 + e]);
    }
    lt = __builtin_fmaf(l[j], sc, lt);
  }
#pragma unroll
  for (int d = 0; d < 8; ++d) acc[d] = slots_sum(acc[d]);
  lt = slots_sum(lt);
  if (sl == 0) {
    const float inv = lt > 0.f ? 1.0f / lt : 0.f;
    if constexpr (O32) {
      float* orow = const_cast<float*>(p.out.row<float>(r)) + 8 * dg;
      *reinterpret_cast<f32x4*>(orow) = f32x4{acc[0] * inv, acc[1] * inv, acc[2] * inv, acc[3] * inv};
      *reinterpret_cast<f32x4*>(orow + 4) = f32x4{acc[4] * inv, acc[5] * inv, acc[6] * inv, acc[7] * inv};
    } else {
      uint32_t o[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const bf16x2 pv = {(__bf16)(acc[2 * e] * inv), (__bf16)(acc[2 * e + 1] * inv)};
        o[e] = __builtin_bit_cast(uint32_t, pv);
      }
      __bf16* orow = const_cast<__bf16*>(p.out.row<__bf16>(r));
      *reinterpret_cast<u32x4*>(orow + 8 * dg) = u32x4{o[0], o[1], o[2], o[3]};
    }
  }
}

static bool to_dev(const saf3r_rows* s, RowsDev* d, const char* name, bool fp32 = false) {
  if (!s || !s->ptr) return fail(SAF3R_ERR_INVALID, "saf3r_gather_attn_fwd: null %s", name), false;
  if (s->row_stride % (fp32 ? 4 : 8) || ((uintptr_t)s->ptr % 16) || s->rows_per_frame <= 0 || s->base_row < 0)
    return fail(SAF3R_ERR_INVALID, "saf3r_gather_attn_fwd: %s must be 16-byte aligned, row stride %% %d, rows_per_frame > 0",
                name, fp32 ? 4 : 8), false;
  d->ptr = s->ptr;
  d->row_stride = s->row_stride;
  d->base_row = s->base_row;
  d->rows_per_frame = s->rows_per_frame;
  d->frame_row_stride = s->frame_row_stride;
  set_divisor(d);
  return true;
}

constexpr int kGatherStep = 32;        // list entries per walk step
constexpr int kGatherStepSliced = 16;  // the same in sliced mode (a slice's 64 entries in 4 steps)
constexpr int kGatherRows = 2;  // rows per wave (both modes)
constexpr int64_t kGatherChunkRows = 65536;  // sliced mode: rows per pair of launches

// waves of this kernel the device holds at once (for the walk order; 1 if unknown)
template <typename K>
static int64_t resident_waves(K kernel) {
  int dev = 0, cus = 0, blocks = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, kernel, 256, 0) != hipSuccess || cus <= 0 || blocks <= 0)
    return 1;
  return (int64_t)cus * blocks * 4;
}

template <bool QK32, bool V32, bool O32>
static void launch_gather_o(GatherParams p, bool sliced, hipStream_t st) {
  if (sliced) {
    auto kernel = gather_attn_kernel<QK32, V32, O32, kGatherStepSliced, true, kGatherRows>;
    p.resident = resident_waves(kernel);
    // rows in chunks: one chunk's partial results (138 MB) stay in the memory-side cache between
    // its two kernels, and the workspace holds one chunk
    const int64_t n = p.n;
    for (int64_t r0 = 0; r0 < n; r0 += kGatherChunkRows) {
      p.r0 = r0;
      p.n = (int)(n - r0 < kGatherChunkRows ? n - r0 : kGatherChunkRows);
      const unsigned gs = (unsigned)((p.n + 4 * kGatherRows - 1) / (4 * kGatherRows));
      const unsigned g4 = (unsigned)((p.n + 3) / 4);
      hipLaunchKernelGGL(kernel, dim3(gs * kGatherSlices), dim3(256), 0, st, p);
      hipLaunchKernelGGL(gather_merge_kernel<O32>, dim3(g4), dim3(256), 0, st, p);
    }
  } else {
    auto kernel = gather_attn_kernel<QK32, V32, O32, kGatherStep, false, kGatherRows>;
    p.resident = resident_waves(kernel);
    hipLaunchKernelGGL(kernel, dim3((unsigned)((p.n + 4 * kGatherRows - 1) / (4 * kGatherRows))), dim3(256), 0, st, p);
  }
}

template <bool QK32, bool V32>
static void launch_gather(const GatherParams& p, bool o32, bool sliced, hipStream_t st) {
  if (o32) launch_gather_o<QK32, V32, true>(p, sliced, st);
  else launch_gather_o<QK32, V32, false>(p, sliced, st);
}

// shared by both entries: argument checks and the launch
static int gather_run(const char* who, const saf3r_rows* q, const saf3r_rows* k, const saf3r_rows* v,
                      const int32_t* idx, int64_t idx_row_stride, int n, int topk, int64_t num_keys, float scale,
                      int dtype_flags, const saf3r_rows* out, float* part, void* stream) {
  GatherParams p;
  if (dtype_flags & ~(SAF3R_GATHER_QK_FP32 | SAF3R_GATHER_V_FP32 | SAF3R_GATHER_OUT_FP32))
    return fail(SAF3R_ERR_INVALID, "%s: unknown dtype flags 0x%x", who, dtype_flags);
  const bool qk32 = dtype_flags & SAF3R_GATHER_QK_FP32, v32 = dtype_flags & SAF3R_GATHER_V_FP32,
             o32 = dtype_flags & SAF3R_GATHER_OUT_FP32;
  if (!to_dev(q, &p.q, "q", qk32) || !to_dev(k, &p.k, "k", qk32) || !to_dev(v, &p.v, "v", v32) ||
      !to_dev(out, &p.out, "out", o32))
    return SAF3R_ERR_INVALID;
  if (!idx || n < 0 || topk <= 0 || idx_row_stride < 0 || num_keys <= 0 || num_keys > 0x7fffffff)
    return fail(SAF3R_ERR_INVALID, "%s: bad index list", who);
  if (n == 0) return SAF3R_OK;
  p.idx = idx;
  p.idx_stride = idx_row_stride;
  p.n = n;
  p.topk = topk;
  p.nk = num_keys;
  p.c = scale * 1.4426950408889634f;
  p.part = part;
  p.r0 = 0;
  const bool sliced = part != nullptr;
  hipStream_t st = (hipStream_t)stream;
  if (qk32) {
    if (v32) launch_gather<true, true>(p, o32, sliced, st);
    else launch_gather<true, false>(p, o32, sliced, st);
  } else {
    if (v32) launch_gather<false, true>(p, o32, sliced, st);
    else launch_gather<false, false>(p, o32, sliced, st);
  }
  return check_launch(who);
}

}  // namespace saf3r

using namespace saf3r;

extern "C" int saf3r_gather_attn_fwd(const saf3r_rows* q, const saf3r_rows* k, const saf3r_rows* v,
                                     const int32_t* idx, int64_t idx_row_stride, int n, int topk,
                                     int64_t num_keys, float scale, int dtype_flags, const saf3r_rows* out,
                                     void* stream) {
  if (int e = injected("saf3r_gather_attn_fwd")) return e;
  return gather_run("saf3r_gather_attn_fwd", q, k, v, idx, idx_row_stride, n, topk, num_keys, scale, dtype_flags,
                    out, nullptr, stream);
}

extern "C" int64_t saf3r_gather_attn_workspace_bytes(int n, int topk) {
  if (n < 0 || topk <= 0) return -1;
  return (n < kGatherChunkRows ? (int64_t)n : kGatherChunkRows) * kGatherSlices * 66 * (int64_t)sizeof(float);
}

extern "C" int saf3r_gather_attn_fwd_sliced(const saf3r_rows* q, const saf3r_rows* k, const saf3r_rows* v,
                                            const int32_t* idx, int64_t idx_row_stride, int n, int topk,
                                            int64_t num_keys, float scale, int dtype_flags, const saf3r_rows* out,
                                            void* workspace, int64_t workspace_bytes, void* stream) {
  if (int e = injected("saf3r_gather_attn_fwd_sliced")) return e;
  const int64_t need = saf3r_gather_attn_workspace_bytes(n, topk);
  if (need < 0) return fail(SAF3R_ERR_INVALID, "saf3r_gather_attn_fwd_sliced: bad index list");
  if (n > 0 && (!workspace || workspace_bytes < need || (uintptr_t)workspace % 16))
    return fail(SAF3R_ERR_INVALID,
                "saf3r_gather_attn_fwd_sliced: needs a 16-byte aligned workspace of %lld bytes, got %lld",
                (long long)need, (long long)(workspace ? workspace_bytes : 0));
  return gather_run("saf3r_gather_attn_fwd_sliced", q, k, v, idx, idx_row_stride, n, topk, num_keys, scale,
                    dtype_flags, out, static_cast<float*>(workspace), stream);
}
