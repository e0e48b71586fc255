// Gather attention over per-row key lists (the image rows of the reference dino_topk heads).
//
// ref: saf3r/triton/sparse_topk_attention.py:36-112 (one program per query: gathered K rows,
//      fp32 scores, exact max-subtracted softmax, fp32 P.V, output in v.dtype), :115-166 (API:
//      q [N, D], k/v [Nk, D], kv_indices [N, TopK], scale default 1/sqrt(D); a stride-0 index view
//      shares one list across rows), :173-258 (online-softmax variant for TopK > 2048).
// Here one wave owns one query row and walks its list in chunks of 64 keys (one key per lane)
// with an fp32 online softmax, so any list length is handled by the same kernel. Entries < 0 or
// >= num_keys are skipped. q and k are bf16 or fp32 rows (the reference's kernel upcasts either).
#include "common.h"

namespace saf3r {

struct RowsDev {
  const void* ptr;
  int64_t row_stride, base_row, rows_per_frame, frame_row_stride;
  template <typename T = __bf16>
  __device__ inline const T* row(int64_t r) const {
    int64_t f = r / rows_per_frame;
    return static_cast<const T*>(ptr) + (base_row + f * frame_row_stride + (r - f * rows_per_frame)) * row_stride;
  }
};

struct GatherParams {
  RowsDev q, k, v, out;
  const int32_t* idx;
  int64_t idx_stride;
  int n, topk;
  int64_t nk;
  float c;  // scale * log2(e)
};

__device__ inline float wave_max(float x) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) x = fmaxf(x, __shfl_xor(x, o));
  return x;
}
__device__ inline float wave_sum(float x) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) x += __shfl_xor(x, o);
  return x;
}

// 2 waves per workgroup, one query row per wave. QK32: q and k rows are fp32 (the reference's gather
// reads the fp32 q / k of the autocast forward and multiplies in fp32); otherwise bf16.
template <bool QK32>
__global__ __launch_bounds__(128) void gather_attn_kernel(GatherParams p) {
  __shared__ float red[2][64][65];
  __shared__ __align__(16) float qs[2][64];
  const int lane = tid_x() & 63, w = tid_x() >> 6;
  const int64_t r = (int64_t)bid_x() * 2 + w;
  const bool active = r < p.n;
  const int64_t rr = active ? r : 0;

  // q row: bf16 pairs in registers, identical in every lane; fp32 in LDS (read as broadcasts)
  uint32_t qw[32];
  if constexpr (QK32) {
    qs[w][lane] = p.q.row<float>(rr)[lane];
    __syncthreads();
  } else {
    const u32x4* q4 = reinterpret_cast<const u32x4*>(p.q.row(rr));
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      u32x4 x = q4[j];
      qw[4 * j] = x[0];
      qw[4 * j + 1] = x[1];
      qw[4 * j + 2] = x[2];
      qw[4 * j + 3] = x[3];
    }
  }
  float acc[64];
#pragma unroll
  for (int d = 0; d < 64; ++d) acc[d] = 0.f;
  float m_run = -__builtin_inff(), l_run = 0.f;
  const int32_t* il = p.idx + rr * p.idx_stride;

  for (int c0 = 0; c0 < p.topk; c0 += 64) {
    const int j = c0 + lane;
    int id = (active && j < p.topk) ? il[j] : -1;
    if (id >= p.nk) id = -1;
    float s = -__builtin_inff();
    uint32_t vw[32];
    if (id >= 0) {
      const u32x4* v4 = reinterpret_cast<const u32x4*>(p.v.row(id));
      float dot = 0.f;
      if constexpr (QK32) {
        const f32x4* k4 = reinterpret_cast<const f32x4*>(p.k.row<float>(id));
        const f32x4* q4 = reinterpret_cast<const f32x4*>(qs[w]);
#pragma unroll
        for (int t = 0; t < 16; ++t) {
          const f32x4 kx = k4[t], qx = q4[t];
          dot = __builtin_fmaf(qx[0], kx[0], dot);
          dot = __builtin_fmaf(qx[1], kx[1], dot);
          dot = __builtin_fmaf(qx[2], kx[2], dot);
          dot = __builtin_fmaf(qx[3], kx[3], dot);
        }
      }
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        const u32x4 vx = v4[t];
        if constexpr (!QK32) {
          const u32x4 kx = reinterpret_cast<const u32x4*>(p.k.row(id))[t];
          // elements are copied to scalars before the bf16x2 bit_cast: a bit_cast applied directly to
          // a vector element (kx[e]) was lowered to element 0 for every e by this compiler
          const uint32_t kw[4] = {kx.x, kx.y, kx.z, kx.w};
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const uint32_t kk = kw[e], qq = qw[4 * t + e];
            dot = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, kk), __builtin_bit_cast(bf16x2, qq),
                                                  dot, false);
          }
        }
        vw[4 * t + 0] = vx.x;
        vw[4 * t + 1] = vx.y;
        vw[4 * t + 2] = vx.z;
        vw[4 * t + 3] = vx.w;
      }
      s = dot;
    } else {
#pragma unroll
      for (int t = 0; t < 32; ++t) vw[t] = 0;
    }
    const float mx = wave_max(s);
    const float m_new = fmaxf(m_run, mx);
    const float m_use = m_new == -__builtin_inff() ? 0.f : m_new;
    const float alpha = __builtin_amdgcn_exp2f((m_run - m_use) * p.c);
    const float pj = __builtin_amdgcn_exp2f(__builtin_fmaf(s, p.c, -m_use * p.c));
    l_run = l_run * alpha + wave_sum(pj);
    m_run = m_new;
#pragma unroll
    for (int t = 0; t < 32; ++t) {
      acc[2 * t] = __builtin_fmaf(pj, bf16_lo(vw[t]), acc[2 * t] * alpha);
      acc[2 * t + 1] = __builtin_fmaf(pj, bf16_hi(vw[t]), acc[2 * t + 1] * alpha);
    }
  }

  // column sums of acc over the 64 lanes through LDS
#pragma unroll
  for (int d = 0; d < 64; ++d) red[w][lane][d] = acc[d];
  __syncthreads();
  float o = 0.f;
  for (int j = 0; j < 64; ++j) o += red[w][j][lane];
  if (active) {
    const float inv = l_run > 0.f ? 1.0f / l_run : 0.f;
    __bf16* orow = const_cast<__bf16*>(p.out.row<__bf16>(r));
    orow[lane] = (__bf16)(o * inv);
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
  return true;
}

}  // namespace saf3r

using namespace saf3r;

extern "C" int saf3r_gather_attn_fwd(const saf3r_rows* q, const saf3r_rows* k, const saf3r_rows* v,
                                     const int32_t* idx, int64_t idx_row_stride, int n, int topk,
                                     int64_t num_keys, float scale, int qk_fp32, const saf3r_rows* out,
                                     void* stream) {
  if (int e = injected("saf3r_gather_attn_fwd")) return e;
  GatherParams p;
  if (qk_fp32 != 0 && qk_fp32 != 1) return fail(SAF3R_ERR_INVALID, "saf3r_gather_attn_fwd: qk_fp32 must be 0 or 1");
  if (!to_dev(q, &p.q, "q", qk_fp32) || !to_dev(k, &p.k, "k", qk_fp32) || !to_dev(v, &p.v, "v") ||
      !to_dev(out, &p.out, "out"))
    return SAF3R_ERR_INVALID;
  if (!idx || n < 0 || topk <= 0 || idx_row_stride < 0 || num_keys <= 0 || num_keys > 0x7fffffff)
    return fail(SAF3R_ERR_INVALID, "saf3r_gather_attn_fwd: bad index list");
  if (n == 0) return SAF3R_OK;
  p.idx = idx;
  p.idx_stride = idx_row_stride;
  p.n = n;
  p.topk = topk;
  p.nk = num_keys;
  p.c = scale * 1.4426950408889634f;
  if (qk_fp32)
    hipLaunchKernelGGL(gather_attn_kernel<true>, dim3((unsigned)((n + 1) / 2)), dim3(128), 0, (hipStream_t)stream, p);
  else
    hipLaunchKernelGGL(gather_attn_kernel<false>, dim3((unsigned)((n + 1) / 2)), dim3(128), 0, (hipStream_t)stream, p);
  return check_launch("saf3r_gather_attn_fwd");
}
