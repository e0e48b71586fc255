// Per-frame token top-k of q.k: the lazy selector of the reference dino_topk heads.
//
// ref: saf3r/triton/fused_qk_topk.py:26-102 (bf16 q.k with fp32 accumulation per 64-key tile;
//      composite key = sortable fp32 bits << 32 | reversed index so ties go to the lower index;
//      running per-frame top-k; frame-major flush in descending order, -1 for empty slots),
//      :120-217 (API: q [B, Nq, D], k [B, Nk, D], Nk = frames * num_toks_per_img, output
//      int32 [B, Nq, frames * min(topk, num_toks_per_img)] of key indices).
// A 256-thread workgroup owns 128 queries (32 per wave). Key tiles of 64 keys are staged in LDS,
// scored with v_mfma_f32_32x32x16_bf16 (S^T = K . Q^T), and every lane keeps a running top-k of
// the 32 keys of the tile it holds; the two lane halves of a query merge their lists when the
// frame ends.
#include <type_traits>

#include "common.h"

namespace saf3r {

struct TopkParams {
  const __bf16* qptr;
  int64_t q_rs, q_base, q_rpf, q_frs;
  const __bf16* kptr;
  int64_t k_rs, k_base, k_rpf, k_frs;
  int nq, F, P, ke;
  int kmode;  // key row of (frame f, token j): 1 = frame f row j (rows_per_frame == P), 0 = flat row f*P + j, 2 = general
  int32_t* idx;
};

__device__ inline const __bf16* rows_at(const __bf16* ptr, int64_t rs, int64_t base, int64_t rpf, int64_t frs,
                                        int64_t r) {
  int64_t f = r / rpf;
  return ptr + (base + f * frs + (r - f * rpf)) * rs;
}


__device__ inline uint64_t partner_u64(uint64_t x) {
  uint32_t lo = (uint32_t)x, hi = (uint32_t)(x >> 32);
  auto rl = __builtin_amdgcn_permlane32_swap(lo, lo, false, false);
  auto rh = __builtin_amdgcn_permlane32_swap(hi, hi, false, false);
  const bool upper = (tid_x() & 63) >= 32;
  uint32_t plo = upper ? (uint32_t)rl[0] : (uint32_t)rl[1];
  uint32_t phi = upper ? (uint32_t)rh[0] : (uint32_t)rh[1];
  return ((uint64_t)phi << 32) | plo;
}

template <int K>
__global__ __launch_bounds__(256) void token_topk_kernel(TopkParams p) {
  __shared__ __align__(16) char kbuf[2][8192];
  const int tid = tid_x(), lane = tid & 63, w = tid >> 6, half = lane >> 5, col = lane & 31;
  const int64_t q0 = (int64_t)bid_x() * 128;
  const int64_t qi = q0 + 32 * w + col;
  const bool qvalid = qi < p.nq;

  bf16x8 qfrag[4];
  {
    const u32x4* qs = reinterpret_cast<const u32x4*>(
        rows_at(p.qptr, p.q_rs, p.q_base, p.q_rpf, p.q_frs, qvalid ? qi : 0) + 32 * half);
#pragma unroll
    for (int s = 0; s < 4; ++s) qfrag[s] = __builtin_bit_cast(bf16x8, qvalid ? qs[s] : u32x4{0, 0, 0, 0});
  }

  const int tiles_pf = (p.P + 63) / 64;
  const int total = p.F * tiles_pf;
  u32x4 kreg[2];
  auto load_tile = [&](int f, int u) {
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const int id = tid + 256 * e, r = id >> 3, ch = id & 7;
      const int pp = 64 * u + r;
      if (pp < p.P) {
        // the frame / row split of the key row without a 64-bit division where the layout allows
        const __bf16* row = p.kmode == 1   ? p.kptr + (p.k_base + (int64_t)f * p.k_frs + pp) * p.k_rs
                            : p.kmode == 0 ? p.kptr + (p.k_base + (int64_t)f * p.P + pp) * p.k_rs
                                           : rows_at(p.kptr, p.k_rs, p.k_base, p.k_rpf, p.k_frs, (int64_t)f * p.P + pp);
        const u32x4* src = reinterpret_cast<const u32x4*>(row);
        kreg[e] = src[ch];
      } else {
        kreg[e] = u32x4{0, 0, 0, 0};
      }
    }
  };
  auto store_tile = [&](int buf) {
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const int id = tid + 256 * e, r = id >> 3, ch = id & 7;
      *reinterpret_cast<u32x4*>(&kbuf[buf][r * 128 + ((ch ^ (r & 7)) << 4)]) = kreg[e];
    }
  };

  // running top-k of the lane's even and of its odd candidates of the frame: two independent
  // branch-free insertion chains whose instructions interleave (one chain alone waits on the
  // compare-to-select hazards); keys are distinct, so merging the two lists loses nothing
  uint64_t a[K], b2[K];
#pragma unroll
  for (int t = 0; t < K; ++t) a[t] = b2[t] = 0;

  load_tile(0, 0);
  store_tile(0);
  __syncthreads();
  int f = 0, u = 0;  // frame and tile of step t
  for (int t = 0; t < total; ++t) {
    const int cur = t & 1;
    const int un = u + 1 == tiles_pf ? 0 : u + 1, fn = u + 1 == tiles_pf ? f + 1 : f;
    if (t + 1 < total) load_tile(fn, un);
    f32x16 s0 = {}, s1 = {};
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const int chn = 4 * half + s;
      const int r0 = col, r1 = 32 + col;
      bf16x8 ka = *reinterpret_cast<const bf16x8*>(&kbuf[cur][r0 * 128 + ((chn ^ (r0 & 7)) << 4)]);
      bf16x8 kb = *reinterpret_cast<const bf16x8*>(&kbuf[cur][r1 * 128 + ((chn ^ (r1 & 7)) << 4)]);
      s0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ka, qfrag[s], s0, 0, 0, 0);
      s1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kb, qfrag[s], s1, 0, 0, 0);
    }
    // candidates of this lane (key 0 stands for a padding position: it never enters a list); only
    // a frame's last tile can hold padding, so the other tiles skip the test
    auto scan = [&](auto padded) {
#pragma unroll
      for (int e = 0; e < 32; e += 2) {
        uint64_t x[2];
#pragma unroll
        for (int o = 0; o < 2; ++o) {
          const float sv = e + o < 16 ? s0[e + o] : s1[e + o - 16];
          const int r = (e + o) & 15;
          const int key = 32 * ((e + o) >> 4) + 8 * (r >> 2) + 4 * half + (r & 3);
          const int pp = 64 * u + key;
          x[o] = ckey(sv, (uint32_t)pp);
          if constexpr (decltype(padded)::value) x[o] = pp < p.P ? x[o] : 0ull;
        }
        topk_insert<K>(a, x[0]);
        topk_insert<K>(b2, x[1]);
      }
    };
    if (64 * u + 64 <= p.P) scan(std::false_type{});
    else scan(std::true_type{});
    if (u == tiles_pf - 1) {
      // merge the odd list and the partner half's list, then flush this frame
#pragma unroll
      for (int e = 0; e < K; ++e) {
        topk_insert<K>(a, b2[e]);
        b2[e] = 0;
      }
      uint64_t b[K];
#pragma unroll
      for (int e = 0; e < K; ++e) b[e] = partner_u64(a[e]);
#pragma unroll
      for (int e = 0; e < K; ++e)
        if (b[e] > a[K - 1]) topk_insert<K>(a, b[e]);
      if (qvalid && half == 0) {
        int32_t* o = p.idx + qi * ((int64_t)p.F * p.ke) + (int64_t)f * p.ke;
#pragma unroll
        for (int e = 0; e < K; ++e)
          if (e < p.ke) o[e] = a[e] ? (int32_t)(f * p.P + ckey_index(a[e])) : -1;
      }
#pragma unroll
      for (int e = 0; e < K; ++e) a[e] = 0;
    }
    if (t + 1 < total) store_tile(cur ^ 1);
    __syncthreads();
    f = fn;
    u = un;
  }
}

template <int K>
static int launch_topk(const TopkParams& p, hipStream_t st) {
  hipLaunchKernelGGL(token_topk_kernel<K>, dim3((unsigned)((p.nq + 127) / 128)), dim3(256), 0, st, p);
  return check_launch("saf3r_token_topk");
}

}  // namespace saf3r

using namespace saf3r;

extern "C" int saf3r_token_topk(const saf3r_rows* q, const saf3r_rows* k, int n_q, int frames, int per_frame,
                                int topk, int32_t* idx, void* stream) {
  if (int e = injected("saf3r_token_topk")) return e;
  if (!q || !k || !q->ptr || !k->ptr || !idx) return fail(SAF3R_ERR_INVALID, "saf3r_token_topk: null pointer");
  if (n_q < 0 || frames <= 0 || per_frame <= 0) return fail(SAF3R_ERR_INVALID, "saf3r_token_topk: bad shape");
  if (topk < 1 || topk > 16) return fail(SAF3R_ERR_UNSUPPORTED, "saf3r_token_topk: topk must be in [1, 16]");
  if (q->row_stride % 8 || k->row_stride % 8 || ((uintptr_t)q->ptr | (uintptr_t)k->ptr) % 16 ||
      q->rows_per_frame <= 0 || k->rows_per_frame <= 0)
    return fail(SAF3R_ERR_INVALID, "saf3r_token_topk: rows must be 16-byte aligned, row stride %% 8");
  if (n_q == 0) return SAF3R_OK;
  TopkParams p;
  p.qptr = (const __bf16*)q->ptr;
  p.q_rs = q->row_stride;
  p.q_base = q->base_row;
  p.q_rpf = q->rows_per_frame;
  p.q_frs = q->frame_row_stride;
  p.kptr = (const __bf16*)k->ptr;
  p.k_rs = k->row_stride;
  p.k_base = k->base_row;
  p.k_rpf = k->rows_per_frame;
  p.k_frs = k->frame_row_stride;
  p.kmode = k->rows_per_frame == per_frame ? 1 : k->rows_per_frame >= (int64_t)frames * per_frame ? 0 : 2;
  p.nq = n_q;
  p.F = frames;
  p.P = per_frame;
  p.ke = topk < per_frame ? topk : per_frame;
  p.idx = idx;
  hipStream_t st = (hipStream_t)stream;
  if (p.ke <= 1) return launch_topk<1>(p, st);
  if (p.ke <= 2) return launch_topk<2>(p, st);
  if (p.ke <= 4) return launch_topk<4>(p, st);
  if (p.ke <= 8) return launch_topk<8>(p, st);
  return launch_topk<16>(p, st);
}
