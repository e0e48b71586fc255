// Prologue of the patched global attention: QK-LayerNorm(64) + 2-D RoPE in fp32, bf16 packing
// of Q, K (row-major slots) and V (transposed, permuted 64x64 tiles).
//
// ref: saf3r/patch/patch_vggt.py:577-583 (qkv reshape, q_norm / k_norm, rope on q and k),
//      saf3r/models/official_vggt/layers/rope.py:86-188 (RoPE-2D: first 32 features rotated by
//      the y position, last 32 by x; within each 32: rotate(t) = cat(-t[16:], t[:16])).
// Under autocast(bf16) the reference runs LayerNorm and RoPE in fp32 and hands bf16 q/k/v to
// attention; this kernel does the same and rounds once, to nearest-even bf16. The cos/sin tables
// come from the caller, computed as the reference does (fp32 angles = position * inv_freq).
// Heads flagged for fp32 rows also get their fp32 q and k (after LayerNorm and RoPE, before the
// rounding) in token order: the reference reads those fp32 values in the q_probe_topk mean and scores
// (saf3r/patch/sparse_attention.py:160-166) and in the dino_topk gather (sparse_topk_attention.py:74-80).
#include "common.h"

namespace saf3r {

struct PackParams {
  const __bf16* q;
  const __bf16* k;
  const __bf16* v;
  int64_t tok_stride, head_stride;
  const float* qw;
  const float* qb;
  const float* kw;
  const float* kb;
  float eps;
  int apply_ln;
  int apply_rope;
  const int32_t* pos;
  const float* rcos;
  const float* rsin;
  int rpos;
  __bf16* qp;
  __bf16* kp;
  __bf16* vp;
  Geom g;
  uint64_t tok_order;  // heads (bit h) packed in token order: slot = token, no special/frame padding
  uint64_t framed;     // heads (bit h) packed in the framed layout: frame f's tokens in order at tile f*NBT
  float* qk32;         // fp32 q and k rows of the flagged heads: [slot][q, k][F*T tokens][64]
  uint64_t f32_heads;  // heads (bit h) whose fp32 q / k rows are also written
  int8_t f32slot[64];  // slot of a flagged head in qk32
  uint64_t q_scaled;   // heads (bit h) whose packed Q is q * q_scale
  float q_scale;
  uint64_t pool_heads;  // heads (bit h) whose patch-block means of bf16(q) and bf16(k) are written
  int8_t pool_slot[64]; // slot of a pooled head in the pooled arrays
  float* pool_mean;     // [slot][q, k][F*NBf][64]
  uint16_t* pool_split; // [slot][q, k][F*NBf][2][64] fp16 bits (pooled_split_row)
  float* pool_meta;     // [slot][q, k][F*NBf][2]
};

// One 512-thread workgroup per (64-slot tile, head). Eight threads own one slot row, 8 features
// each (thread c8 of a row: features 8 c8 .. 8 c8 + 7); LayerNorm reduces across the eight, RoPE
// pairs feature d with d +- 16 (partner thread c8 ^ 2). Every load of a row is issued before any
// processing, so the q, k and v loads are in flight together.
// Pooled heads: a patch tile of the packed layout is one selection block; its bf16(q) (without the
// Q scale) and bf16(k) rows are staged in LDS, every thread sums one (tensor, group of kPoolGroup
// rows, feature) in row order, and one thread per (tensor, feature) adds the group sums in order
// and divides once by the block population: the block means of the block-dynamic pattern,
// bit-identical to that definition. Rows past the population hold +0.0, which changes no sum
// started at +0.0. Each of those two waves then writes its row's split record.
__global__ __launch_bounds__(512) void pack_qkv_kernel(PackParams p) {
  __shared__ __align__(16) __bf16 vs[64 * 72];  // V rows of the tile, 144-byte row pitch
  __shared__ __align__(16) __bf16 ps[2][64 * 64];  // pooled heads: bf16 q / k rows of the tile
  __shared__ float pp[2][64 / kPoolGroup][64];     // pooled heads: group sums
  const Geom& g = p.g;
  const int tile = bid_x(), h = bid_y();
  const int t = tid_x(), row = t >> 3, c8 = t & 7;
  const int64_t slot = (int64_t)tile * 64 + row;
  const int64_t ntok = (int64_t)g.F * g.T;
  const int64_t tok = (h < 64 && ((p.tok_order >> h) & 1)) ? (slot < ntok ? slot : -1)
                      : (h < 64 && ((p.framed >> h) & 1)) ? framed_token(g, slot)
                                                           : slot_token(g, slot);
  const int64_t src = tok * p.tok_stride + (int64_t)h * p.head_stride + 8 * c8;
  const int64_t dst = ((int64_t)h * g.L + slot) * 64 + 8 * c8;
  // a patch tile of a pooled head (pooled heads are packed in the padded layout: tile = block)
  const bool pool = h < 64 && ((p.pool_heads >> h) & 1) && tile >= g.nst;

  u32x4 raw[3];
#pragma unroll
  for (int m = 0; m < 3; ++m) {
    raw[m] = u32x4{0, 0, 0, 0};
    if (tok >= 0) raw[m] = *reinterpret_cast<const u32x4*>((m == 0 ? p.q : m == 1 ? p.k : p.v) + src);
  }

  // RoPE: features 0..31 turn with the y position, 32..63 with x; feature e of a 32-half takes
  // angle index e % 16 and, for e < 16, -t[e + 16] (else +t[e - 16]) as its partner term
  float cs[8], sn[8];
  if (p.apply_rope && tok >= 0) {
    const int pv = min(max(p.pos[tok * 2 + (c8 >> 2)], 0), p.rpos - 1);
    const f32x4* c4 = reinterpret_cast<const f32x4*>(p.rcos + pv * 16 + 8 * (c8 & 1));
    const f32x4* s4 = reinterpret_cast<const f32x4*>(p.rsin + pv * 16 + 8 * (c8 & 1));
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const f32x4 cv = c4[j], sv = s4[j];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        cs[4 * j + e] = cv[e];
        sn[4 * j + e] = sv[e];
      }
    }
  }

#pragma unroll
  for (int which = 0; which < 2; ++which) {
    __bf16* outp = which == 0 ? p.qp : p.kp;
    float x[8];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      x[2 * j] = bf16_lo(raw[which][j]);
      x[2 * j + 1] = bf16_hi(raw[which][j]);
    }
    if (p.apply_ln) {
      float s = 0.f;
#pragma unroll
      for (int j = 0; j < 8; ++j) s += x[j];
      s += __shfl_xor(s, 1);
      s += __shfl_xor(s, 2);
      s += __shfl_xor(s, 4);
      const float mean = s * (1.0f / 64.0f);
      float v2 = 0.f;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        float dlt = x[j] - mean;
        v2 += dlt * dlt;
      }
      v2 += __shfl_xor(v2, 1);
      v2 += __shfl_xor(v2, 2);
      v2 += __shfl_xor(v2, 4);
      const float rstd = 1.0f / sqrtf(v2 * (1.0f / 64.0f) + p.eps);
      const float* w = which == 0 ? p.qw : p.kw;
      const float* b = which == 0 ? p.qb : p.kb;
#pragma unroll
      for (int j = 0; j < 8; ++j) x[j] = (x[j] - mean) * rstd * w[8 * c8 + j] + b[8 * c8 + j];
    }
    if (p.apply_rope) {
      float y[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) y[j] = __shfl_xor(x[j], 2);
      const float sg = (c8 & 2) ? 1.0f : -1.0f;
#pragma unroll
      for (int j = 0; j < 8; ++j) x[j] = x[j] * cs[j] + sg * y[j] * sn[j];
    }
    if (tok < 0) {
#pragma unroll
      for (int j = 0; j < 8; ++j) x[j] = 0.f;
    } else if (h < 64 && ((p.f32_heads >> h) & 1)) {
      // the fp32 values before the bf16 rounding, in token order (the probe and gather inputs)
      f32x4* d32 = reinterpret_cast<f32x4*>(p.qk32 + (((int64_t)p.f32slot[h] * 2 + which) * ntok + tok) * 64 + 8 * c8);
      d32[0] = f32x4{x[0], x[1], x[2], x[3]};
      d32[1] = f32x4{x[4], x[5], x[6], x[7]};
    }
    if (pool) {  // the unscaled bf16 row (zeros past the block's population)
      u32x4 o;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const bf16x2 a = {(__bf16)x[2 * j], (__bf16)x[2 * j + 1]};
        o[j] = __builtin_bit_cast(uint32_t, a);
      }
      *reinterpret_cast<u32x4*>(&ps[which][row * 64 + 8 * c8]) = o;
    }
    if (which == 0 && h < 64 && ((p.q_scaled >> h) & 1)) {
#pragma unroll
      for (int j = 0; j < 8; ++j) x[j] *= p.q_scale;
    }
    u32x4 o;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const bf16x2 a = {(__bf16)x[2 * j], (__bf16)x[2 * j + 1]};
      o[j] = __builtin_bit_cast(uint32_t, a);
    }
    *reinterpret_cast<u32x4*>(outp + dst) = o;
  }

  // V: stage the tile's 64 rows, then write the transposed, permuted tile.
  *reinterpret_cast<u32x4*>(vs + row * 72 + 8 * c8) = raw[2];
  __syncthreads();
  {
    const int i = t >> 3;                               // tile row (d after permutation)
    const int ii = i & 31;
    const int d = 32 * (i >> 5) + 16 * ((ii >> 2) & 1) + 4 * (ii >> 3) + (ii & 3);  // phi
    uint32_t w[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      int c0 = 8 * c8 + 2 * j, c1 = c0 + 1;
      int k0 = (c0 & ~12) | ((c0 & 4) << 1) | ((c0 & 8) >> 1);  // kappa
      int k1 = (c1 & ~12) | ((c1 & 4) << 1) | ((c1 & 8) >> 1);
      uint16_t lo = __builtin_bit_cast(uint16_t, vs[k0 * 72 + d]);
      uint16_t hi = __builtin_bit_cast(uint16_t, vs[k1 * 72 + d]);
      w[j] = (uint32_t)lo | ((uint32_t)hi << 16);
    }
    *reinterpret_cast<u32x4*>(p.vp + ((int64_t)h * g.L + (int64_t)tile * 64) * 64 + i * 64 + 8 * c8) =
        u32x4{w[0], w[1], w[2], w[3]};
  }
  if (pool) {  // uniform over the workgroup
    static_assert(2 * (64 / kPoolGroup) * 64 == 512, "one thread per (tensor, group, feature)");
    {
      const int which = t >> 8, grp = (t >> 6) & 3, d = t & 63;
      const __bf16* col = &ps[which][grp * kPoolGroup * 64 + d];
      float x[kPoolGroup];  // every read in flight, then the additions in row order
#pragma unroll
      for (int i = 0; i < kPoolGroup; ++i) x[i] = (float)col[i * 64];
      float part = 0.f;
#pragma unroll
      for (int i = 0; i < kPoolGroup; ++i) part = part + x[i];
      pp[which][grp][d] = part;
    }
    __syncthreads();
  }
  if (pool && t < 128) {  // waves 0 (q) and 1 (k): lane = feature
    const int which = t >> 6, d = t & 63;
    const int pt = tile - g.nst, b = pt % g.NBf;
    const int cnt = min(64, g.P - 64 * b);
    float sum = 0.f;
#pragma unroll
    for (int grp = 0; grp < 64 / kPoolGroup; ++grp) sum = sum + pp[which][grp][d];
    const float mean = sum / (float)cnt;
    const int64_t nb = (int64_t)g.F * g.NBf;
    const int64_t rec = ((int64_t)p.pool_slot[h] * 2 + which) * nb + pt;  // pt = f * NBf + b
    p.pool_mean[rec * 64 + d] = mean;
    pooled_split_row(mean, d, p.pool_split + rec * 128, p.pool_meta + rec * 2);
  }
}

}  // namespace saf3r

using namespace saf3r;

extern "C" int saf3r_pack_qkv(const void* q, const void* k, const void* v, int64_t tok_stride, int64_t head_stride,
                              int frames, int tokens_per_frame, int num_special, int num_heads,
                              const float* q_ln_weight, const float* q_ln_bias, const float* k_ln_weight,
                              const float* k_ln_bias, float ln_eps, int apply_ln, const int32_t* pos,
                              const float* rope_cos, const float* rope_sin, int rope_positions, void* q_packed,
                              void* k_packed, void* v_packed, const uint8_t* token_order, const uint8_t* fp32_heads,
                              float* qk32, const uint8_t* q_scaled, float q_scale, const uint8_t* pool_heads,
                              float* pool_mean, uint16_t* pool_split, float* pool_meta, void* stream) {
  if (int e = injected("saf3r_pack_qkv")) return e;
  PackParams p;
  if (!make_geom(frames, tokens_per_frame, num_special, &p.g))
    return fail(SAF3R_ERR_INVALID, "saf3r_pack_qkv: invalid geometry F=%d T=%d ns=%d", frames, tokens_per_frame,
                num_special);
  if (num_heads <= 0 || num_heads > 65535) return fail(SAF3R_ERR_INVALID, "saf3r_pack_qkv: bad num_heads %d", num_heads);
  if (!q || !k || !v || !q_packed || !k_packed || !v_packed)
    return fail(SAF3R_ERR_INVALID, "saf3r_pack_qkv: null tensor pointer");
  if (tok_stride % 8 || head_stride % 8 || ((uintptr_t)q | (uintptr_t)k | (uintptr_t)v) % 16)
    return fail(SAF3R_ERR_INVALID, "saf3r_pack_qkv: inputs must be 16-byte aligned with strides a multiple of 8");
  if (((uintptr_t)q_packed | (uintptr_t)k_packed | (uintptr_t)v_packed) % 16)
    return fail(SAF3R_ERR_INVALID, "saf3r_pack_qkv: packed outputs must be 16-byte aligned");
  if (apply_ln && (!q_ln_weight || !q_ln_bias || !k_ln_weight || !k_ln_bias))
    return fail(SAF3R_ERR_INVALID, "saf3r_pack_qkv: LayerNorm requested without parameters");
  if (rope_cos && (!pos || !rope_sin || rope_positions <= 0 || ((uintptr_t)rope_cos | (uintptr_t)rope_sin) % 16))
    return fail(SAF3R_ERR_INVALID, "saf3r_pack_qkv: RoPE needs positions and 16-byte aligned cos/sin tables");
  p.q = (const __bf16*)q;
  p.k = (const __bf16*)k;
  p.v = (const __bf16*)v;
  p.tok_stride = tok_stride;
  p.head_stride = head_stride;
  p.qw = q_ln_weight;
  p.qb = q_ln_bias;
  p.kw = k_ln_weight;
  p.kb = k_ln_bias;
  p.eps = ln_eps;
  p.apply_ln = apply_ln != 0;
  p.apply_rope = rope_cos != nullptr;
  p.pos = pos;
  p.rcos = rope_cos;
  p.rsin = rope_sin;
  p.rpos = rope_positions;
  p.qp = (__bf16*)q_packed;
  p.kp = (__bf16*)k_packed;
  p.vp = (__bf16*)v_packed;
  p.tok_order = p.framed = 0;
  if (token_order) {
    for (int h = 0; h < num_heads; ++h) {
      const int lay = token_order[h];
      if (!lay) continue;
      if (h >= 64) return fail(SAF3R_ERR_UNSUPPORTED, "saf3r_pack_qkv: token order is supported for heads 0..63");
      if (lay == SAF3R_LAYOUT_TOKEN) {
        p.tok_order |= 1ull << h;
      } else if (lay == SAF3R_LAYOUT_FRAMED) {
        if (!framed_fits(p.g))
          return fail(SAF3R_ERR_UNSUPPORTED, "saf3r_pack_qkv: the framed layout needs ceil(T/64) = ceil(P/64) here");
        p.framed |= 1ull << h;
      } else {
        return fail(SAF3R_ERR_INVALID, "saf3r_pack_qkv: head %d: unknown layout %d", h, lay);
      }
    }
  }
  p.qk32 = qk32;
  p.f32_heads = 0;
  if (fp32_heads) {
    int n32 = 0;
    for (int h = 0; h < num_heads; ++h) {
      if (!fp32_heads[h]) continue;
      if (h >= 64) return fail(SAF3R_ERR_UNSUPPORTED, "saf3r_pack_qkv: fp32 rows are supported for heads 0..63");
      p.f32_heads |= 1ull << h;
      p.f32slot[h] = (int8_t)n32++;
    }
    if (n32 > 0 && (!qk32 || (uintptr_t)qk32 % 16))
      return fail(SAF3R_ERR_INVALID, "saf3r_pack_qkv: fp32 heads need a 16-byte aligned qk32 buffer");
  }
  p.q_scaled = 0;
  p.q_scale = q_scale;
  if (q_scaled) {
    for (int h = 0; h < num_heads; ++h) {
      if (!q_scaled[h]) continue;
      if (h >= 64) return fail(SAF3R_ERR_UNSUPPORTED, "saf3r_pack_qkv: scaled Q is supported for heads 0..63");
      p.q_scaled |= 1ull << h;
    }
    if (p.q_scaled && !(q_scale > 0.f && q_scale < 3.0e38f))
      return fail(SAF3R_ERR_INVALID, "saf3r_pack_qkv: q_scale must be positive and finite");
  }
  p.pool_heads = 0;
  p.pool_mean = pool_mean;
  p.pool_split = pool_split;
  p.pool_meta = pool_meta;
  if (pool_heads) {
    int np = 0;
    for (int h = 0; h < num_heads; ++h) {
      if (!pool_heads[h]) continue;
      if (h >= 64) return fail(SAF3R_ERR_UNSUPPORTED, "saf3r_pack_qkv: pooling is supported for heads 0..63");
      if (((p.tok_order | p.framed) >> h) & 1)
        return fail(SAF3R_ERR_INVALID, "saf3r_pack_qkv: pooled head %d must use the packed layout", h);
      p.pool_heads |= 1ull << h;
      p.pool_slot[h] = (int8_t)np++;
    }
    if (np > 0 && (!pool_mean || !pool_split || !pool_meta || ((uintptr_t)pool_mean | (uintptr_t)pool_split |
                                                                (uintptr_t)pool_meta) % 16))
      return fail(SAF3R_ERR_INVALID, "saf3r_pack_qkv: pooled heads need 16-byte aligned pool_mean / split / meta");
  }
  dim3 grid(p.g.NT, num_heads);
  hipLaunchKernelGGL(pack_qkv_kernel, grid, dim3(512), 0, (hipStream_t)stream, p);
  return check_launch("saf3r_pack_qkv");
}
