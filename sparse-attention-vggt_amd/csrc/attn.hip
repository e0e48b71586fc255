// Block-sparse flash-attention forward (head_dim 64, bf16, fp32 online softmax) over the packed
// layout. One launch covers every head; each head's pattern (dense, frame-local, anchor+local,
// block-dynamic, special rows of token-dynamic, anchor, skip) decides which 64-slot key tiles a
// query tile visits and how partial tiles are masked.
//
// ref: saf3r/patch/wrapper.py:94-106 (per-head loop, "full" -> SDPA),
//      saf3r/patch/sparse_attention.py:12-90 (mode dispatch), :134-140 (all_to_first),
//      :189-231 (dino_topk: special rows dense, image rows over selected keys only),
//      :234-253 (global_to_frame).
//
// Work decomposition: a workgroup of two waves owns one (head, 64-slot query tile); wave w owns
// query rows 32w..32w+31. Key tiles (64 slots x 64 features, 8 KB for K and 8 KB for V) are
// staged in LDS, double-buffered, and consumed with v_mfma_f32_32x32x16_bf16:
//   S^T (64 keys x 32 queries) = K . Q^T   (A = K rows from LDS, B = Q kept in registers)
//   O^T (64 d x 32 queries)   += V^T . P^T (A = transposed V tile from LDS, B = P in registers)
// In the S^T accumulator a lane holds one query and 32 keys, so row max / row sum need a single
// cross-half exchange (v_permlane32_swap). Work items are ordered by decreasing per-item cost.
#include "common.h"

namespace saf3r {

constexpr int kMaxSel = 2048;

struct AttnParams {
  const __bf16* q;
  const __bf16* k;
  const __bf16* v;
  const int32_t* sel;
  __bf16* out;
  int64_t out_stride;
  Geom g;
  int sel_width;
  float c;  // softmax scale * log2(e)
  int n_order;
  int order[kMaxHeads];
  int item_start[kMaxHeads + 1];
  int8_t pattern[kMaxHeads];
  int8_t slot[kMaxHeads];
};

__device__ inline float permlane_partner_max(float x) {
  uint32_t u = __builtin_bit_cast(uint32_t, x);
  auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return fmaxf(__builtin_bit_cast(float, (uint32_t)r[0]), __builtin_bit_cast(float, (uint32_t)r[1]));
}
__device__ inline float permlane_partner_sum(float x) {
  uint32_t u = __builtin_bit_cast(uint32_t, x);
  auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return __builtin_bit_cast(float, (uint32_t)r[0]) + __builtin_bit_cast(float, (uint32_t)r[1]);
}

// Key-tile sequence of one work item: up to four contiguous ranges, or a compacted list in LDS.
// Fields are scalars (no indexed arrays) so the sequence stays in registers.
struct TileSeq {
  int s0, l0, s1, l1, s2, l2, s3, l3;
  int nr;
  int count;
  const int* list;  // LDS, when non-null
  __device__ inline int at(int n) const {
    if (list) return list[n];
    if (n < l0) return s0 + n;
    n -= l0;
    if (n < l1) return s1 + n;
    n -= l1;
    if (n < l2) return s2 + n;
    return s3 + (n - l2);
  }
  __device__ inline void add(int s, int l) {
    if (l <= 0) return;
    if (nr == 0) { s0 = s; l0 = l; }
    else if (nr == 1) { s1 = s; l1 = l; }
    else if (nr == 2) { s2 = s; l2 = l; }
    else { s3 = s; l3 = l; }
    ++nr;
    count += l;
  }
};

__global__ __launch_bounds__(128) void sparse_attn_kernel(AttnParams p) {
  __shared__ __align__(16) char kbuf[2][8192];
  __shared__ __align__(16) char vbuf[2][8192];
  __shared__ int tiles[kMaxSel];
  __shared__ int wave_cnt[2];

  const Geom& g = p.g;
  const int tid = threadIdx.x;
  const int lane = tid & 63, w = tid >> 6, half = lane >> 5, col = lane & 31;
  const int bid = blockIdx.x;

  // ---- decode the work item (uniform) ----
  int oh = 0;
  while (oh + 1 < p.n_order && bid >= p.item_start[oh + 1]) ++oh;
  const int h = p.order[oh];
  const int pat = p.pattern[h];
  const int qt = bid - p.item_start[oh];
  const bool qspecial = qt < g.nst;
  const int qf = qspecial ? 0 : (qt - g.nst) / g.NBf;  // frame of a patch query tile
  const int qb = qspecial ? 0 : (qt - g.nst) % g.NBf;

  // query row owned by this lane and its frame / validity
  const int qrow = 32 * w + col;
  const int64_t qslot = (int64_t)qt * 64 + qrow;
  int64_t qtok;
  int frow;
  if (qspecial) {
    qtok = qslot < g.S ? (qslot / g.ns) * g.T + qslot % g.ns : -1;
    frow = g.ns > 0 ? (int)(qslot / g.ns) : 0;
  } else {
    int pp = qb * 64 + qrow;
    qtok = pp < g.P ? (int64_t)qf * g.T + g.ns + pp : -1;
    frow = qf;
  }

  const int64_t head_base = (int64_t)h * g.L;  // slot offset of this head
  __bf16* orow = p.out + (qtok >= 0 ? qtok : 0) * p.out_stride + (int64_t)h * 64;

  if (pat == SAF3R_SKIP) {
    if (qtok >= 0) {
      u32x4 z = {0, 0, 0, 0};
      u32x4* o4 = reinterpret_cast<u32x4*>(orow + 16 * half);
      o4[0] = z;
      o4[1] = z;
      o4[4] = z;
      o4[5] = z;
    }
    return;
  }

  // ---- key-tile sequence (uniform) ----
  TileSeq seq;
  seq.s0 = seq.s1 = seq.s2 = seq.s3 = 0;
  seq.l0 = seq.l1 = seq.l2 = seq.l3 = 0;
  seq.nr = 0;
  seq.count = 0;
  seq.list = nullptr;
  const int eff = (pat == SAF3R_TOKEN_DYNAMIC || (pat == SAF3R_BLOCK_DYNAMIC && qspecial)) ? SAF3R_DENSE : pat;
  bool frame_rel = false;
  if (eff == SAF3R_DENSE) {
    seq.add(0, g.NT);
  } else if (eff == SAF3R_BLOCK_DYNAMIC) {
    // compact the selection row into LDS (drop -1 entries, keep order)
    const int32_t* srow = p.sel + ((int64_t)p.slot[h] * ((int64_t)g.F * g.NBf) + (qt - g.nst)) * p.sel_width;
    int base = 0;
    for (int c0 = 0; c0 < p.sel_width; c0 += 128) {
      int j = c0 + tid;
      int v = j < p.sel_width ? srow[j] : -1;
      bool ok = v >= 0 && v < g.F * g.NBf;
      uint64_t m = __ballot(ok);
      int pre = __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0));
      if (lane == 0) wave_cnt[w] = __popcll(m);
      __syncthreads();
      int off = base + (w ? wave_cnt[0] : 0) + pre;
      if (ok) tiles[off] = g.nst + v;
      base += wave_cnt[0] + wave_cnt[1];
      __syncthreads();
    }
    seq.count = base;
    seq.list = tiles;
  } else {
    frame_rel = true;
    // frames covered by the query tile
    int f0 = qf, f1 = qf;
    if (qspecial) {
      int last = min(g.S, (qt + 1) * 64) - 1;
      f0 = (qt * 64) / g.ns;
      f1 = last / g.ns;
    }
    const bool need_anchor = (eff == SAF3R_ANCHOR_LOCAL || eff == SAF3R_ANCHOR);
    const bool need_local = (eff != SAF3R_ANCHOR);
    // special key tiles
    int ls0 = 1, ls1 = 0;  // local special tile range [ls0, ls1]
    if (g.ns > 0 && need_local) {
      ls0 = (f0 * g.ns) / 64;
      ls1 = ((f1 + 1) * g.ns - 1) / 64;
    }
    if (g.ns > 0 && need_anchor && !(need_local && ls0 == 0)) seq.add(0, (g.ns - 1) / 64 + 1);
    if (g.ns > 0 && need_local) seq.add(ls0, ls1 - ls0 + 1);
    // patch key tiles
    if (need_anchor && !(need_local && f0 == 0)) seq.add(g.nst, g.NBf);
    if (need_local) seq.add(g.nst + f0 * g.NBf, (f1 - f0 + 1) * g.NBf);
  }

  // ---- Q fragments: lane holds features 32*half .. 32*half+31 of its query row ----
  bf16x8 qfrag[4];
  {
    const u32x4* qsrc = reinterpret_cast<const u32x4*>(p.q + (head_base + qslot) * 64 + 32 * half);
#pragma unroll
    for (int s = 0; s < 4; ++s) qfrag[s] = __builtin_bit_cast(bf16x8, qsrc[s]);
  }

  f32x16 o0 = {}, o1 = {};
  float m_run = -__builtin_inff();
  float l_run = 0.f;
  const float c = p.c;

  // staging: thread handles 16-byte chunks tid + 128*u of the 8 KB K and V tiles
  u32x4 kreg[4], vreg[4];
  auto load_tile = [&](int kt) {
    const u32x4* ks = reinterpret_cast<const u32x4*>(p.k + (head_base + (int64_t)kt * 64) * 64);
    const u32x4* vs = reinterpret_cast<const u32x4*>(p.v + (head_base + (int64_t)kt * 64) * 64);
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      kreg[u] = ks[tid + 128 * u];
      vreg[u] = vs[tid + 128 * u];
    }
  };
  auto store_tile = [&](int buf) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      int id = tid + 128 * u, r = id >> 3, ch = id & 7;
      int off = r * 128 + ((ch ^ (r & 7)) << 4);
      *reinterpret_cast<u32x4*>(&kbuf[buf][off]) = kreg[u];
      *reinterpret_cast<u32x4*>(&vbuf[buf][off]) = vreg[u];
    }
  };

  const int count = seq.count;
  if (count > 0) {
    load_tile(seq.at(0));
    store_tile(0);
  }
  __syncthreads();

  for (int n = 0; n < count; ++n) {
    const int cur = n & 1;
    const int kt = seq.at(n);
    if (n + 1 < count) load_tile(seq.at(n + 1));

    // ---- S^T = K . Q^T ----
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

    // ---- masking of partial / multi-frame tiles ----
    const bool kspecial = kt < g.nst;
    bool partial;
    if (kspecial) partial = (kt + 1) * 64 > g.S;
    else partial = (g.P & 63) != 0 && ((kt - g.nst) % g.NBf) == g.NBf - 1;
    const bool need_mask = partial || (frame_rel && (kspecial || qspecial));
    if (need_mask) {
      const int kfrm_patch = kspecial ? 0 : (kt - g.nst) / g.NBf;
      const int kp0 = kspecial ? 0 : ((kt - g.nst) % g.NBf) * 64;
#pragma unroll
      for (int a = 0; a < 32; ++a) {
        const int key = 32 * (a >> 4) + 8 * ((a & 15) >> 2) + 4 * half + (a & 3);
        bool ok;
        int fc;
        if (kspecial) {
          const int sl = kt * 64 + key;
          ok = sl < g.S;
          fc = sl / g.ns;
        } else {
          ok = kp0 + key < g.P;
          fc = kfrm_patch;
        }
        if (eff == SAF3R_FRAME_LOCAL) ok = ok && fc == frow;
        else if (eff == SAF3R_ANCHOR_LOCAL) ok = ok && (fc == 0 || fc == frow);
        else if (eff == SAF3R_ANCHOR) ok = ok && fc == 0;
        if (!ok) {
          if (a < 16) s0[a] = -__builtin_inff();
          else s1[a - 16] = -__builtin_inff();
        }
      }
    }

    // ---- online softmax (base 2) ----
    float mx = -__builtin_inff();
#pragma unroll
    for (int a = 0; a < 16; ++a) mx = fmaxf(mx, fmaxf(s0[a], s1[a]));
    mx = permlane_partner_max(mx);
    const float m_new = fmaxf(m_run, mx);
    const float m_use = m_new == -__builtin_inff() ? 0.f : m_new;
    const float alpha = __builtin_amdgcn_exp2f((m_run - m_use) * c);
    const float mc = m_use * c;
    float ls = 0.f;
#pragma unroll
    for (int a = 0; a < 16; ++a) {
      s0[a] = __builtin_amdgcn_exp2f(__builtin_fmaf(s0[a], c, -mc));
      s1[a] = __builtin_amdgcn_exp2f(__builtin_fmaf(s1[a], c, -mc));
      ls += s0[a] + s1[a];
    }
    l_run = l_run * alpha + ls;
    m_run = m_new;
#pragma unroll
    for (int a = 0; a < 16; ++a) {
      o0[a] *= alpha;
      o1[a] *= alpha;
    }

    // ---- O^T += V^T . P^T ----
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const f32x16& sj = (j < 2) ? s0 : s1;
      const int a0 = 8 * (j & 1);
      bf16x8 pf;
#pragma unroll
      for (int t = 0; t < 8; ++t) pf[t] = (__bf16)sj[a0 + t];
      const int chn = 2 * j + half;
      const int r0 = col, r1 = 32 + col;
      bf16x8 va = *reinterpret_cast<const bf16x8*>(&vbuf[cur][r0 * 128 + ((chn ^ (r0 & 7)) << 4)]);
      bf16x8 vb = *reinterpret_cast<const bf16x8*>(&vbuf[cur][r1 * 128 + ((chn ^ (r1 & 7)) << 4)]);
      o0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(va, pf, o0, 0, 0, 0);
      o1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vb, pf, o1, 0, 0, 0);
    }

    if (n + 1 < count) store_tile(cur ^ 1);
    __syncthreads();
  }

  // ---- epilogue: normalise and store 2 x 32 bytes per lane ----
  const float lt = permlane_partner_sum(l_run);
  const float inv = lt > 0.f ? 1.0f / lt : 0.f;
  if (qtok >= 0) {
    uint32_t wv[16];
#pragma unroll
    for (int a = 0; a < 8; ++a) {
      bf16x2 x0 = {(__bf16)(o0[2 * a] * inv), (__bf16)(o0[2 * a + 1] * inv)};
      bf16x2 x1 = {(__bf16)(o1[2 * a] * inv), (__bf16)(o1[2 * a + 1] * inv)};
      wv[a] = __builtin_bit_cast(uint32_t, x0);
      wv[8 + a] = __builtin_bit_cast(uint32_t, x1);
    }
    u32x4* o4 = reinterpret_cast<u32x4*>(orow + 16 * half);
    o4[0] = u32x4{wv[0], wv[1], wv[2], wv[3]};
    o4[1] = u32x4{wv[4], wv[5], wv[6], wv[7]};
    o4[4] = u32x4{wv[8], wv[9], wv[10], wv[11]};
    o4[5] = u32x4{wv[12], wv[13], wv[14], wv[15]};
  }
}

// Relative cost of one work item (key tiles visited), used to order heads longest-first.
static int64_t item_cost(int pat, const Geom& g, int sel_width) {
  switch (pat) {
    case SAF3R_DENSE: return g.NT;
    case SAF3R_TOKEN_DYNAMIC: return g.NT;
    case SAF3R_BLOCK_DYNAMIC: return sel_width;
    case SAF3R_ANCHOR_LOCAL: return 2 * (g.NBf + 1);
    case SAF3R_FRAME_LOCAL: return g.NBf + 1;
    case SAF3R_ANCHOR: return g.NBf + 1;
    default: return 0;
  }
}

}  // namespace saf3r

using namespace saf3r;

extern "C" int saf3r_sparse_attn_fwd(const void* q_packed, const void* k_packed, const void* v_packed, int frames,
                                     int tokens_per_frame, int num_special, int num_heads,
                                     const int32_t* head_pattern, const int32_t* sel, int sel_width, float scale,
                                     void* out, int64_t out_row_stride, void* stream) {
  if (int e = injected("saf3r_sparse_attn_fwd")) return e;
  AttnParams p;
  if (!make_geom(frames, tokens_per_frame, num_special, &p.g))
    return fail(SAF3R_ERR_INVALID, "saf3r_sparse_attn_fwd: invalid geometry");
  if (num_heads <= 0 || num_heads > kMaxHeads)
    return fail(SAF3R_ERR_UNSUPPORTED, "saf3r_sparse_attn_fwd: num_heads must be in [1, %d]", kMaxHeads);
  if (!q_packed || !k_packed || !v_packed || !out || !head_pattern)
    return fail(SAF3R_ERR_INVALID, "saf3r_sparse_attn_fwd: null pointer");
  if (((uintptr_t)out % 16) || (out_row_stride % 8) || out_row_stride < (int64_t)num_heads * 64)
    return fail(SAF3R_ERR_INVALID, "saf3r_sparse_attn_fwd: out must be 16-byte aligned with row stride >= H*64, %% 8");
  int n_dyn = 0;
  for (int h = 0; h < num_heads; ++h) {
    int pt = head_pattern[h];
    if (pt < SAF3R_DENSE || pt > SAF3R_SKIP)
      return fail(SAF3R_ERR_INVALID, "saf3r_sparse_attn_fwd: head %d has unknown pattern %d", h, pt);
    p.pattern[h] = (int8_t)pt;
    p.slot[h] = (int8_t)(pt == SAF3R_BLOCK_DYNAMIC ? n_dyn++ : -1);
  }
  if (n_dyn > 0) {
    if (!sel) return fail(SAF3R_ERR_INVALID, "saf3r_sparse_attn_fwd: block-dynamic heads need a selection list");
    if (sel_width <= 0 || sel_width > kMaxSel)
      return fail(SAF3R_ERR_UNSUPPORTED, "saf3r_sparse_attn_fwd: sel_width must be in [1, %d] (got %d)", kMaxSel,
                  sel_width);
  }
  p.q = (const __bf16*)q_packed;
  p.k = (const __bf16*)k_packed;
  p.v = (const __bf16*)v_packed;
  p.sel = sel;
  p.sel_width = sel_width;
  p.out = (__bf16*)out;
  p.out_stride = out_row_stride;
  p.c = scale * 1.4426950408889634f;
  // heads ordered by decreasing item cost (stable by head id), each with its item range
  int idx[kMaxHeads];
  for (int h = 0; h < num_heads; ++h) idx[h] = h;
  for (int i = 1; i < num_heads; ++i) {
    int x = idx[i], j = i;
    int64_t cx = item_cost(p.pattern[x], p.g, sel_width);
    while (j > 0 && item_cost(p.pattern[idx[j - 1]], p.g, sel_width) < cx) {
      idx[j] = idx[j - 1];
      --j;
    }
    idx[j] = x;
  }
  int64_t total = 0;
  p.n_order = 0;
  for (int i = 0; i < num_heads; ++i) {
    int h = idx[i];
    int items = p.pattern[h] == SAF3R_TOKEN_DYNAMIC ? p.g.nst : p.g.NT;
    if (items == 0) continue;
    p.order[p.n_order] = h;
    p.item_start[p.n_order] = (int)total;
    ++p.n_order;
    total += items;
  }
  p.item_start[p.n_order] = (int)total;
  if (total == 0) return SAF3R_OK;
  if (total > 0x7fffffff) return fail(SAF3R_ERR_UNSUPPORTED, "saf3r_sparse_attn_fwd: too many work items");
  hipLaunchKernelGGL(sparse_attn_kernel, dim3((unsigned)total), dim3(128), 0, (hipStream_t)stream, p);
  return check_launch("saf3r_sparse_attn_fwd");
}
